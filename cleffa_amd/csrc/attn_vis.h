// Vision tower attention for head dim 72 on CDNA4: bidirectional attention within each image
// (metal/clef.metal:1720-1964, vis_attention_mma / _mpp), Q and K already biased and rotated
// by the vision prologue. Same data flow as the text kernel (S^T = K . Q^T and
// O^T += V^T . P^T with v_mfma_f32_16x16x32_bf16, K and V^T tiles of 64 keys streamed
// global -> LDS with global_load_lds, double buffered, XOR-swizzled), but 4 waves of 32 query
// rows: each LDS operand read feeds the products of both 16-row halves, and the two halves'
// softmax chains interleave. The small head dim leaves room for both halves' registers at two
// workgroups per CU.
// The 72-dim contraction runs as three 32-dim chunks: Q holds zeros in dims 72..95, and the
// K slots of those dims hold copies of real K chunks of the same row (finite), so they add 0.
// O^T covers 80 rows in five 16-row tiles: tiles 0-3 hold dims 0-63 in the permuted row order
// below, tile 4 rows 64-79 in natural order. V^T rows 73..79 of both LDS buffers are zeroed once
// per workgroup and row 72 is set to 1, so O^T row 72 accumulates the row sum of the rounded P
// (the softmax denominator, rescaled with O) in the padding products the MFMAs run anyway.
// Q is pre-scaled by scale * log2 e and the S accumulators start at minus the row's running max,
// so the products deliver the exponent of P directly; only when a tile moves the max (by more
// than 8, rarely) is the difference subtracted and O rescaled.
#pragma once
#include "attn_text.h"

namespace clef_hip {
namespace vis {
constexpr int HD = 72;                 // head dim
constexpr int ROWB = HD * 2;           // bytes per Q / K plane row (9 chunks of 16 bytes)
constexpr int RCH = ROWB / 16;         // 16-byte chunks per plane row
constexpr int NC = 3;                  // 32-dim chunks of the contraction (96 with padding)
constexpr int NM = 5;                  // 16-row O^T tiles (80 rows)
constexpr int HDV = 80;                // V^T rows in LDS
constexpr int BQ = 128, BK = 64, WAVES = 4, ROWS = 32;
constexpr int KSLOTS = 16;             // 16-byte slots per K row in LDS (12 carry data)
constexpr int KTILE = BK * KSLOTS * 8; // elements per K tile (16 KB)
constexpr int VTILE = HDV * BK;        // elements per V^T tile (10 KB)
constexpr int LDS_ELEMS = 2 * KTILE + 2 * VTILE;
}  // namespace vis

__global__ __launch_bounds__(256, 2) void attn_vis_kernel(AttnParams p) {
    using namespace vis;
    using text::k_swz;
    using text::s_row_key;
    using text::lds_read16;
    using text::lds_wait;
    using text::lds_wait2;
    using text::lds_addr;
    using text::static_for;
    using text::xrow_max;
    using text::xrow_sum;
    typedef __attribute__((ext_vector_type(4))) float f32x4;
    __shared__ __attribute__((aligned(16))) uint16_t smem[LDS_ELEMS];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int q16 = lane & 15, g = lane >> 4;
    const int bi = blockIdx.x / p.nh, h = blockIdx.x - bi * p.nh;
    const int32_t *blk = p.blocks + 8 * bi;
    const int q_row0 = blk[0], nq = blk[1], k_row0 = blk[3], k_len = blk[4];
    const int flag_row = blk[5];
    const bool wave_live = wave * ROWS < nq;

    const uint16_t *kbase = p.k_plane + ((size_t)h * p.kvT + k_row0) * HD;
    const uint16_t *vbase = p.vt_plane + (size_t)h * HD * p.kvT + k_row0;
    uint16_t *const k0s = smem, *const k1s = smem + KTILE, *const v0s = smem + 2 * KTILE,
                   *const v1s = smem + 2 * KTILE + VTILE;
    const int wave_s = __builtin_amdgcn_readfirstlane(wave);

    // K fills: slot s of a tile = key s/16, LDS slot s%16 holding logical chunk
    // (s%16) ^ k_swz(key); logical chunks 9..15 are padding and take chunk (logical - 9).
    // Wave w fills K slot groups 4w .. 4w+3. V^T fills: slot s = dim s/8, chunk
    // (s%8) ^ v_swz(dim), 72 dims = 9 groups of 64 slots: wave w fills groups 2w, 2w+1, and wave
    // 0 also group 8.
    unsigned kfo[4], vfo[3];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int s = (wave_s * 4 + j) * 64 + lane;
        const int key = s >> 4;
        const int lc = (s & 15) ^ k_swz(key);
        kfo[j] = (unsigned)(key * ROWB + (lc < RCH ? lc : lc - RCH) * 16);
    }
#pragma unroll
    for (int j = 0; j < 3; j++) {
        const int grp = j < 2 ? wave_s * 2 + j : 8;
        const int vs = grp * 64 + lane;
        const int d = vs >> 3, c = (vs & 7) ^ text::v_swz(d);
        vfo[j] = (unsigned)d * (unsigned)p.kvT * 2u + (unsigned)c * 16u;
    }
    // a uniform base plus a 32-bit lane offset widened at the use (the empty asm keeps it 32-bit
    // there): the scalar-base form of the load, no 64-bit address math
    auto lds_fill = [&](const char *base, unsigned off, uint16_t *dst) {
        asm volatile("" : "+v"(off));
        __builtin_amdgcn_global_load_lds((const void *)(base + off), (lds_void *)dst, 16, 0, 0);
    };
    auto load_tiles = [&](int kb, uint16_t *Ks, uint16_t *Vs) {
        const char *kt_base = (const char *)(kbase + (size_t)kb * HD);
        const char *vt_base = (const char *)(vbase + kb);
#pragma unroll
        for (int j = 0; j < 4; j++) lds_fill(kt_base, kfo[j], Ks + (wave_s * 4 + j) * 512);
#pragma unroll
        for (int j = 0; j < 2; j++) lds_fill(vt_base, vfo[j], Vs + (wave_s * 2 + j) * 512);
        if (wave_s == 0) lds_fill(vt_base, vfo[2], Vs + 8 * 512);
    };
    auto zero_tail = [&](int kb, uint16_t *Vs) {   // V^T entries of keys >= k_len -> 0
        const int valid = k_len - kb;
#pragma unroll
        for (int j = 0; j < 3; j++) {
            const int s = tid + 256 * j;
            if (s < HD * 8) {
                const int d = s >> 3, c = (s & 7) ^ text::v_swz(d);
                const int k0 = c * 8;
                u32x4 w = *(u32x4 *)(Vs + s * 8);
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const unsigned keep = (k0 + 2 * e + 1 < valid) ? 0xffffffffu : (k0 + 2 * e < valid ? 0xffffu : 0u);
                    w[e] &= keep;
                }
                *(u32x4 *)(Vs + s * 8) = w;
            }
        }
    };

    // per-lane LDS byte addresses of the A operands
    const unsigned kl = lds_addr(smem), vl = kl + 2 * 2 * KTILE;
    unsigned ka[4][NC];
#pragma unroll
    for (int kt = 0; kt < 4; kt++) {
        const int key = s_row_key(kt, q16);
        const int x = k_swz(key);
#pragma unroll
        for (int c = 0; c < NC; c++) ka[kt][c] = kl + 16 * (key * KSLOTS + ((4 * c + g) ^ x));
    }
    const int vrow = 8 * (q16 >> 2) + (q16 & 3);   // + 32*(mt>>1) + 4*(mt&1)
    const int vx = text::v_swz(vrow);
    const unsigned va0 = vl + 2 * (vrow * BK + ((g ^ vx) * 8));
    const unsigned va1 = vl + 2 * (vrow * BK + (((4 + g) ^ vx) * 8));
    // tile 4: row 64 + q16 (the swizzle of 64 + d is that of d)
    const int nx = text::v_swz(q16);
    const unsigned vn0 = vl + 2 * ((64 + q16) * BK + ((g ^ nx) * 8));
    const unsigned vn1 = vl + 2 * ((64 + q16) * BK + (((4 + g) ^ nx) * 8));

    const int n_tiles = (k_len + BK - 1) / BK;
    // V^T rows 72..79 of both buffers: row 72 all ones (bf16 1.0), the rest zero. A row is 64
    // keys in 8 chunks whose order the swizzle permutes; the values are the same in every chunk.
    for (int i = tid; i < 2 * (HDV - HD) * BK / 8; i += 256) {
        const int b = i / ((HDV - HD) * BK / 8), r = i % ((HDV - HD) * BK / 8);
        const unsigned one = r < BK / 8 ? 0x3f803f80u : 0u;
        *(u32x4 *)((b ? v1s : v0s) + HD * BK + r * 8) = u32x4{one, one, one, one};
    }
    if (n_tiles > 0) load_tiles(0, k0s, v0s);

    // ---- Q: half hh of the wave holds rows 32w + 16hh + q16; lane holds Q[row][32c + 8g + j]
    // (zero past dim 72), the B operand of chunk c.
    bf16x8 qf[2][NC];
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
        const int my_q = wave * ROWS + 16 * hh + q16;
        const bool q_valid = my_q < nq;
        const uint16_t *src = p.q_plane + ((size_t)h * p.T + (size_t)q_row0 + (q_valid ? my_q : 0)) * HD;
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const int ch = 4 * c + g;
            const u32x4 w = (q_valid && ch < RCH) ? *(const u32x4 *)(src + ch * 8) : u32x4{0, 0, 0, 0};
            u32x4 ws;
#pragma unroll
            for (int j = 0; j < 4; j++) ws[j] = pack_bf16(bf_lo(w[j]) * p.scale_log2, bf_hi(w[j]) * p.scale_log2);
            qf[hh][c] = __builtin_bit_cast(bf16x8, ws);
        }
    }
    f32x4 o[2][NM];
#pragma unroll
    for (int hh = 0; hh < 2; hh++)
#pragma unroll
        for (int mt = 0; mt < NM; mt++) o[hh][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    // running max per half in the scaled (log2) domain; msub: what the S accumulators start from
    float m_run[2] = {-INFINITY, -INFINITY};
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    auto tile = [&](const int t, auto BUF) {
        constexpr int buf = decltype(BUF)::value;
        // The two workgroups of a CU (b and b + grid/2 under the round-robin dispatch) take turns
        // at issue priority, tile by tile. Left to the hardware, the older one wins every tie:
        // it finished its key loop at 21.6 us and the younger at 27.5 us, alone on the CU for the
        // last 6 us.
        if ((t + (blockIdx.x >= (gridDim.x >> 1) ? 1 : 0)) & 1) __builtin_amdgcn_s_setprio(1);
        else __builtin_amdgcn_s_setprio(0);
        uint16_t *const Vs = buf ? v1s : v0s, *const Kn = buf ? k0s : k1s, *const Vn = buf ? v0s : v1s;
        const int kb = t * BK;
        if (kb + BK > k_len) {   // WG-uniform: the block's last tile
            zero_tail(kb, Vs);
            __syncthreads();
        }
        if (t + 1 < n_tiles) load_tiles(kb + BK, Kn, Vn);
        if (wave_live) {
            constexpr int DEPTH = 6, QK = 4 * NC;
            f32x4 s[2][4];
            bf16x8 ring[DEPTH];
            static_for<DEPTH>([&](auto I) {
                constexpr int st = decltype(I)::value, kt = st & 3, c = st >> 2;
                ring[st] = lds_read16<buf * 2 * KTILE>(ka[kt][c]);
            });
            const float ms0 = m_run[0] == -INFINITY ? 0.f : m_run[0];
            const float ms1 = m_run[1] == -INFINITY ? 0.f : m_run[1];
            // one K operand, both halves' products; operands waited for two at a time (one
            // s_waitcnt per four products)
            static_for<QK / 2>([&](auto P) {
                constexpr int st = 2 * decltype(P)::value;
                constexpr int last = (st + DEPTH - 1) < (QK - 1) ? (st + DEPTH - 1) : (QK - 1);
                bf16x8 a2[2] = {ring[st % DEPTH], ring[(st + 1) % DEPTH]};
                lds_wait2<last - (st + 1)>(a2[0], a2[1]);
                static_for<2>([&](auto H) {
                    constexpr int sp = st + decltype(H)::value, kt = sp & 3, c = sp >> 2;
                    bf16x8 a = a2[decltype(H)::value];
                    if constexpr (c == 0) {
                        s[0][kt] = f32x4{-ms0, -ms0, -ms0, -ms0};
                        s[1][kt] = f32x4{-ms1, -ms1, -ms1, -ms1};
                    }
                    s[0][kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[0][c], s[0][kt], 0, 0, 0);
                    s[1][kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[1][c], s[1][kt], 0, 0, 0);
                });
                static_for<2>([&](auto H) {
                    constexpr int n = st + decltype(H)::value + DEPTH, nkt = n & 3, nc = n >> 2;
                    if constexpr (n < QK) ring[(st + decltype(H)::value) % DEPTH] = lds_read16<buf * 2 * KTILE>(ka[nkt][nc]);
                });
            });
            constexpr int PV = NM * 2;
            auto vread = [&](auto I) {   // step st = NM * kc + mt
                constexpr int st = decltype(I)::value, mt = st % NM, kc = st / NM;
                if constexpr (mt < 4) {
                    constexpr int off = buf * 2 * VTILE + (32 * (mt >> 1) + 4 * (mt & 1)) * BK * 2;
                    return lds_read16<off>(kc ? va1 : va0);
                } else {
                    return lds_read16<buf * 2 * VTILE>(kc ? vn1 : vn0);
                }
            };
            bf16x8 vring[DEPTH];
            static_for<DEPTH>([&](auto I) { vring[decltype(I)::value] = vread(I); });
            bf16x8 pk[2][2];
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                if (kb + BK > k_len) {
                    // element (kt, i) is key kb + 32(kt>>1) + 8g + 4(kt&1) + i
                    const int lim = k_len - 1 - kb - 8 * g;
#pragma unroll
                    for (int kt = 0; kt < 4; kt++)
#pragma unroll
                        for (int i = 0; i < 4; i++)
                            s[hh][kt][i] = (32 * (kt >> 1) + 4 * (kt & 1) + i > lim) ? -INFINITY : s[hh][kt][i];
                }
                float mx = -INFINITY;
#pragma unroll
                for (int kt = 0; kt < 4; kt++)
                    mx = __builtin_elementwise_maximum(__builtin_elementwise_maximum(mx, __builtin_elementwise_maximum(s[hh][kt][0], s[hh][kt][1])),
                                                       __builtin_elementwise_maximum(s[hh][kt][2], s[hh][kt][3]));
                // s holds score - running max. The max moves only when a tile's max passes it by
                // more than 8 (log2 units), or on the first tile: P stays below 2^8, and the
                // shift and the O rescale below run on few tiles. The lane's own max decides
                // whether any row may move; only then is the row max reduced over its four lanes.
                const float mr = m_run[hh];
                if (__any(mx > 8.f || mr == -INFINITY)) {
                    const float rmx = xrow_max(mx);
                    const float d = (mr == -INFINITY || rmx > 8.f) ? (rmx == -INFINITY ? 0.f : rmx) : 0.f;
                    const float alpha = (mr == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(-d);
                    m_run[hh] = (mr == -INFINITY) ? (rmx == -INFINITY ? -INFINITY : d) : mr + d;
#pragma unroll
                    for (int kt = 0; kt < 4; kt++) s[hh][kt] -= d;
#pragma unroll
                    for (int mt = 0; mt < NM; mt++) o[hh][mt] *= alpha;
                }
#pragma unroll
                for (int kc = 0; kc < 2; kc++) {
                    unsigned w[4];
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int kt = 2 * kc + (j >> 1), i = 2 * (j & 1);
                        w[j] = pack_bf16(__builtin_amdgcn_exp2f(s[hh][kt][i]), __builtin_amdgcn_exp2f(s[hh][kt][i + 1]));
                    }
                    u32x4 wv = {w[0], w[1], w[2], w[3]};
                    pk[hh][kc] = __builtin_bit_cast(bf16x8, wv);
                }
            }
            static_for<PV / 2>([&](auto P) {   // one V^T operand, both halves' products, waited in pairs
                constexpr int st = 2 * decltype(P)::value;
                constexpr int last = (st + DEPTH - 1) < (PV - 1) ? (st + DEPTH - 1) : (PV - 1);
                bf16x8 a2[2] = {vring[st % DEPTH], vring[(st + 1) % DEPTH]};
                lds_wait2<last - (st + 1)>(a2[0], a2[1]);
                static_for<2>([&](auto H) {
                    constexpr int sp = st + decltype(H)::value, mt = sp % NM, kc = sp / NM;
                    bf16x8 a = a2[decltype(H)::value];
                    o[0][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pk[0][kc], o[0][mt], 0, 0, 0);
                    o[1][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pk[1][kc], o[1][mt], 0, 0, 0);
                });
                static_for<2>([&](auto H) {
                    constexpr int n = st + decltype(H)::value + DEPTH;
                    if constexpr (n < PV) vring[(st + decltype(H)::value) % DEPTH] = vread(std::integral_constant<int, n>{});
                });
            });
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    };
    for (int t = 0; t < n_tiles; t += 2) {
        tile(t, std::integral_constant<int, 0>{});
        if (t + 1 < n_tiles) tile(t + 1, std::integral_constant<int, 1>{});
    }

    // ---- Epilogue: O / l; lane (q16, g) holds dims 32u + 8g + [0, 8) of tiles 2u, 2u + 1 (u < 2)
    // and dims 64 + 4g + [0, 4) of tile 4 (stored for g < 2)
    int32_t *flag = p.ovf ? p.ovf + flag_row : nullptr;
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
        const int my_q = wave * ROWS + 16 * hh + q16;
        // the row sum sits in O^T row 72: tile 4, lane 32 + q16, element 0
        const float l_row = __shfl(o[hh][4][0], 32 + q16);   // before the row-divergent exit
        if (my_q >= nq) continue;
        const float il = l_row > 0.f ? 1.f / l_row : 0.f;
        const size_t t = (size_t)q_row0 + my_q;
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int d0 = 32 * u + 8 * g;
            float v[8];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                v[i] = o[hh][2 * u][i] * il;
                v[4 + i] = o[hh][2 * u + 1][i] * il;
            }
            store_out8(p.out, t * p.out_ld + (size_t)h * HD + d0, v, p.out_type, p.f16_lim, flag);
        }
        if (g < 2) store_out4(p.out, t * p.out_ld + (size_t)h * HD + 64 + 4 * g, o[hh][4] * il, p.out_type, p.f16_lim, flag);
    }
}

}  // namespace clef_hip
