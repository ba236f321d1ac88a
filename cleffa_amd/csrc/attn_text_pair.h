// Text prefill attention for head dim 256, wave-pair form. Same semantics, block list, prologue and
// epilogue as attn_text.h (metal/clef.metal:930-1093, 245-300, 709-849); the work split differs.
//
// Workgroup: 8 wavefronts as 4 pairs, one block of 128 query rows of one q head. Pair p owns rows
// 32p .. 32p+31 and both of its waves hold all 32 rows (Q as two 16-row B operands):
//   S^T = K . Q^T   wave h of the pair takes keys 32h .. 32h+31 of each 64-key tile, all 256 dims;
//                   every K operand read from LDS feeds two products (one per 16-row half).
//   O^T += V^T.P^T  wave h takes dims 128h .. 128h+127 over all 64 keys; every V^T operand read
//                   feeds two products. The keys of the other wave come as its bf16 P (2 KB per
//                   wave and tile) through LDS.
// Per wave and tile that is the same 64 MFMAs as the one-wave-per-16-rows form with half of the
// LDS operand traffic (32 KB instead of 64 KB), the bound of that form. The row max is exchanged
// through LDS before the exponentials, so both waves of a pair scale P by the same running max.
//
// Each tile runs in two phases between workgroup barriers A and B:
//   phase 1: partner's P(t-1) read; S(t) = K(t) Q^T; masked row max written for the partner; [A]
//   phase 2: partner's max read; P(t) = exp2(S - m) interleaved with O += V(t-1) P(t-1);
//            O rescaled if the running max moved; P(t) written for the partner;             [B]
// so the softmax of one tile overlaps the P.V products of the previous one inside each wave.
// Fills (global_load_lds, double-buffered K and V^T): K(t+2) after A(t) into the buffer K(t) left,
// V(t+1) after B(t) into the buffer V(t-1) left. The gate rows load into both K buffers after the
// last A; the next item's Q rows into the V buffers once the last P.V is done, its first two K
// tiles once every wave has read its gate values.
#pragma once
#include "attn_text.h"

namespace clef_hip {

namespace tpair {
using namespace text;
constexpr int P_OFF = 4 * KTILE * 2;            // bytes: P exchange slots follow the four tiles
constexpr int M_OFF = P_OFF + 8 * 2048;         // row max / row sum exchange slots
constexpr int SMEM_BYTES = M_OFF + 8 * 32 * 4;  // 148,480 bytes

__device__ __forceinline__ void ds_write16(unsigned addr, bf16x8 v) {
    asm volatile("ds_write_b128 %0, %1" : : "v"(addr), "v"(v) : "memory");
}
template <int OFF>
__device__ __forceinline__ void ds_write4(unsigned addr, float v) {
    asm volatile("ds_write_b32 %0, %1 offset:%2" : : "v"(addr), "v"(v), "i"(OFF) : "memory");
}
template <int OFF>
__device__ __forceinline__ float ds_read4(unsigned addr) {
    float r;
    asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF) : "memory");
    return r;
}
template <int N, typename T>
__device__ __forceinline__ void lgkm_wait(T &r) {
    asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(r) : "i"(N));
}
// wait until at most n (0, 4 or 8; wave-uniform) of this wave's vector memory operations are in flight
__device__ __forceinline__ void vm_wait(int n) {
    if (n >= 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else if (n >= 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}
// workgroup barrier after this wave's LDS accesses have completed (fills are waited for separately)
__device__ __forceinline__ void bar() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
}  // namespace tpair

template <int NROT>
__device__ __forceinline__ void text_pair_items(const AttnParams &p, uint16_t *smem, float *qn_lds) {
    using namespace text;
    using namespace tpair;
    static_assert(NROT % 64 == 0 && NROT <= HD, "rotary pairs must sit in one lane");
    const int tid = threadIdx.x, lane = tid & 63;
    const int q16 = lane & 15, g = lane >> 4;
    const int wave_s = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hh = wave_s & 1, pr = wave_s >> 1;
    ItemList items;
    items.setup(p);
    int item = items.get(0);
    if (item < 0) return;

    uint16_t *const k0s = smem, *const k1s = smem + KTILE, *const v0s = smem + 2 * KTILE,
                   *const v1s = smem + 3 * KTILE;
    const unsigned kl = lds_addr(smem), vl = kl + 2 * 2 * KTILE;
    // K operand of this wave's key tile ktl (keys 32hh + 8(r/4) + 4 ktl + r%4), chunk c, in K0:
    // chunk 4c' + g of key row `key` sits at slot (4c' + g) ^ k_swz(key), i.e. at byte
    // kb0 + ((64 c') ^ kx) + 2048 ktl with the two per-lane terms below (k_swz's low bits depend on
    // the row only through r%4, its high bits flip with ktl).
    unsigned kb0, kx;
    {
        const int key = s_row_key(2 * hh, q16);
        const int x = k_swz(key);
        kb0 = kl + 2 * key * HD + 16 * (g ^ (x & 3));
        kx = 64 * (x >> 2);
    }
    // V^T operands of this wave's dims (128hh + ...), for its own key half and the partner's
    const int vrow = 8 * (q16 >> 2) + (q16 & 3);
    const int vx = v_swz(vrow);
    const unsigned vh = (unsigned)(hh * 128 * BK * 2);
    const unsigned va_lo = vl + vh + 2 * (vrow * BK + ((g ^ vx) * 8));
    const unsigned va_hi = vl + vh + 2 * (vrow * BK + (((4 + g) ^ vx) * 8));
    const unsigned va_own = hh ? va_hi : va_lo, va_par = hh ? va_lo : va_hi;
    const unsigned pl_own = kl + P_OFF + wave_s * 2048 + lane * 16;
    const unsigned pl_par = kl + P_OFF + (wave_s ^ 1) * 2048 + lane * 16;
    const unsigned ml_own = kl + M_OFF + wave_s * 128 + q16 * 4;
    const unsigned ml_par = kl + M_OFF + (wave_s ^ 1) * 128 + q16 * 4;
    const unsigned qn_addr = lds_addr((const uint16_t *)qn_lds);
    constexpr int R = NROT / 64;

    struct Item {
        int q_row0, nq, q_pos0, k_row0, k_len, flag_row, h, kh, n_tiles;
        const uint16_t *kbase, *vbase;
    };
    auto decode = [&](int it) {
        Item s;
        const int bi = it / p.nh;
        s.h = it - bi * p.nh;
        const int32_t *blk = p.blocks + 8 * bi;
        i32x8 e;
        asm volatile("s_load_dwordx8 %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(e) : "s"(blk) : "memory");
        s.q_row0 = e[0]; s.nq = e[1]; s.q_pos0 = e[2]; s.k_row0 = e[3]; s.k_len = e[4];
        s.flag_row = e[5];
        s.kh = s.h / (p.nh / p.nkv);
        s.n_tiles = (s.k_len + BK - 1) / BK;
        s.kbase = p.k_plane + ((size_t)s.kh * p.kvT + s.k_row0) * HD;
        s.vbase = p.vt_plane + (size_t)s.kh * HD * p.kvT + s.k_row0;
        return s;
    };
    // Tile fills, 4 loads per wave. Wave w fills slots [(4w + j) * 64, +64): K slot s = key s/32,
    // chunk (s%32) ^ k_swz(key); V^T slot s = dim s/8, chunk (s%8) ^ v_swz(dim) (the layout of
    // attn_text.h). Offsets come from an opaque lane id so that they are recomputed at each use.
    auto load_k = [&](const Item &s, int kb, uint16_t *Ks) {
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const char *base = (const char *)(s.kbase + (size_t)kb * HD);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int key = (wave_s * 4 + j) * 2 + (ln >> 5);
            const unsigned off = (unsigned)(key * HD + (((ln & 31) ^ k_swz(key)) * 8)) * 2u;
            __builtin_amdgcn_global_load_lds((const void *)(base + off), (lds_void *)(Ks + (wave_s * 4 + j) * 512), 16, 0, 0);
        }
    };
    auto load_v = [&](const Item &s, int kb, uint16_t *Vs) {
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const char *base = (const char *)(s.vbase + kb);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int d = (wave_s * 4 + j) * 8 + (ln >> 3);
            const unsigned off = ((unsigned)d * (unsigned)p.kvT + (unsigned)(((ln & 7) ^ v_swz(d)) * 8)) * 2u;
            __builtin_amdgcn_global_load_lds((const void *)(base + off), (lds_void *)(Vs + (wave_s * 4 + j) * 512), 16, 0, 0);
        }
    };
    // Q or gate rows of the block (128 x 256 bf16, `off` 0 or HD): rows 0-63 into G0, 64-127 into
    // G1, row r at (r & 63) * 256, 16-byte chunk c at slot c ^ (r & 15). 8 loads per wave.
    auto load_rows = [&](const Item &s, uint16_t *G0, uint16_t *G1, const int off) {
        int ln = lane;
        asm volatile("" : "+v"(ln));
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int grp = wave_s * 8 + j;
            const int row = grp * 2 + (ln >> 5);
            const int c = (ln & 31) ^ (row & 15);
            int rc = min(row, s.nq - 1);
            uint16_t *dst = (grp < 32 ? G0 : G1) + (grp & 31) * 512;
            __builtin_amdgcn_global_load_lds((const void *)(p.qkv + ((size_t)s.q_row0 + rc) * p.row + (size_t)s.h * 2 * HD + off + c * 8),
                                             (lds_void *)dst, 16, 0, 0);
        }
    };
    float4 csv[R > 0 ? R : 1][4];
    auto load_cs = [&](const Item &s) {
        if (NROT > 0 && p.rope_cs) {
            const int my_q = wave_s * 16 + q16;
            const size_t qrow = (size_t)s.q_row0 + (my_q < s.nq ? my_q : 0);
            const float *cs = p.rope_cs + qrow * (NROT / 2) * 2;
#pragma unroll
            for (int c = 0; c < R; c++)
#pragma unroll
                for (int q4 = 0; q4 < 4; q4++) csv[c][q4] = *(const float4 *)(cs + 2 * (c * 32 + 8 * g) + 4 * q4);
        }
    };

    Item cur = decode(item);
    {
        const float qn_v = (p.q_norm && tid < HD) ? p.q_norm[tid] : 0.f;
        load_cs(cur);
        load_rows(cur, v0s, v1s, 0);
        if (cur.n_tiles > 0) load_k(cur, 0, k0s);
        if (cur.n_tiles > 1) load_k(cur, BK, k1s);
        if (tid < HD) asm volatile("ds_write_b32 %0, %1" : : "v"(qn_addr + 4u * tid), "v"(qn_v) : "memory");
    }

    for (int k = 0;; k++) {
        uint64_t *const tr = (p.trace && tid == 0) ? p.trace + 8 * (size_t)item : nullptr;
        if (tr) {
            tr[0] = wall_clock64();
            tr[2] = __builtin_amdgcn_s_getreg((31 << 11) | 4);
            tr[3] = __builtin_amdgcn_s_getreg((15 << 11) | 20);
            tr[6] = blockIdx.x;
            tr[7] = k;
        }
        const int T = cur.n_tiles, k_len = cur.k_len;
        const int row0 = 32 * pr;
        const bool pair_live = row0 < cur.nq;
        const int pair_last_pos = cur.q_pos0 + row0 + 31;
        const int qpos0 = cur.q_pos0 + row0 + q16, qpos1 = qpos0 + 16;

        // ---- Q prologue: this wave normalises and rotates rows 16 wave .. +15 (half hh of its
        // pair) and writes them back as f16 in place; then each wave reads both halves of its pair.
        f16x8 qf[2][NC];
        {
            if (k > 0) load_cs(cur);
            __builtin_amdgcn_s_waitcnt(0);
            __builtin_amdgcn_s_barrier();   // Q rows, q_norm and the first K tiles are in LDS
            int ln = lane;
            asm volatile("" : "+v"(ln));
            const int mq = wave_s * 16 + (ln & 15), gg = ln >> 4;
            uint16_t *const qr = (mq < 64 ? v0s : v1s) + (mq & 63) * 256;
            u32x4 qw[NC];
#pragma unroll
            for (int c = 0; c < NC; c++) qw[c] = *(const u32x4 *)(qr + (((4 * c + gg) ^ (mq & 15)) * 8));
            float x[NC][8];
            float ss = 0.f;
#pragma unroll
            for (int c = 0; c < NC; c++) {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    x[c][2 * j] = bf_lo(qw[c][j]);
                    x[c][2 * j + 1] = bf_hi(qw[c][j]);
                }
#pragma unroll
                for (int j = 0; j < 8; j++) ss += x[c][j] * x[c][j];
            }
            ss = xrow_sum(ss);
            if (p.q_norm) {
                const float inv = rsqrtf(ss / (float)HD + p.eps);
#pragma unroll
                for (int c = 0; c < NC; c++) {
                    const float4 w0 = *(const float4 *)(qn_lds + c * 32 + 8 * gg);
                    const float4 w1 = *(const float4 *)(qn_lds + c * 32 + 8 * gg + 4);
                    const float wn[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
                    for (int j = 0; j < 8; j++) x[c][j] = x[c][j] * inv * wn[j];
                }
            }
            if (NROT > 0) {
                if (p.rope_cs) {
#pragma unroll
                    for (int c = 0; c < R; c++) {
                        const float t[16] = {csv[c][0].x, csv[c][0].y, csv[c][0].z, csv[c][0].w,
                                             csv[c][1].x, csv[c][1].y, csv[c][1].z, csv[c][1].w,
                                             csv[c][2].x, csv[c][2].y, csv[c][2].z, csv[c][2].w,
                                             csv[c][3].x, csv[c][3].y, csv[c][3].z, csv[c][3].w};
#pragma unroll
                        for (int j = 0; j < 8; j++) {
                            const float cs_ = t[2 * j], sn = t[2 * j + 1];
                            const float x0 = x[c][j], x1 = x[c + R][j];
                            x[c][j] = x0 * cs_ - x1 * sn;
                            x[c + R][j] = x1 * cs_ + x0 * sn;
                        }
                    }
                } else {
                    const int my_q = wave_s * 16 + q16;
                    const size_t qrow = (size_t)cur.q_row0 + (my_q < cur.nq ? my_q : 0);
                    const int32_t *pp = p.pos3 + 3 * qrow;
                    const float pt = (float)pp[0], ph = (float)pp[1], pw = (float)pp[2];
#pragma unroll
                    for (int c = 0; c < R; c++) {
                        const float4 f0 = *(const float4 *)(p.inv_freq + c * 32 + 8 * g);
                        const float4 f1 = *(const float4 *)(p.inv_freq + c * 32 + 8 * g + 4);
                        const float fr[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
#pragma unroll
                        for (int j = 0; j < 8; j++) {
                            const int i = c * 32 + 8 * g + j;
                            const int ax = i % 3;
                            const float pos = ax == 0 ? pt : (ax == 1 ? ph : pw);
                            float sn, cs;
                            rope_sincos(pos * fr[j], &sn, &cs);
                            const float x0 = x[c][j], x1 = x[c + R][j];
                            x[c][j] = x0 * cs - x1 * sn;
                            x[c + R][j] = x1 * cs + x0 * sn;
                        }
                    }
                }
            }
#pragma unroll
            for (int c = 0; c < NC; c++) {
                u32x4 w = {pack_f16(x[c][0], x[c][1]), pack_f16(x[c][2], x[c][3]),
                           pack_f16(x[c][4], x[c][5]), pack_f16(x[c][6], x[c][7])};
                *(u32x4 *)(qr + (((4 * c + gg) ^ (mq & 15)) * 8)) = w;
            }
            bar();   // both halves of every pair are in LDS as f16
#pragma unroll
            for (int rb = 0; rb < 2; rb++) {
                const int mr = 32 * pr + 16 * rb + (ln & 15);
                const uint16_t *qq = (mr < 64 ? v0s : v1s) + (mr & 63) * 256;
#pragma unroll
                for (int c = 0; c < NC; c++) qf[rb][c] = *(const f16x8 *)(qq + (((4 * c + gg) ^ (mr & 15)) * 8));
            }
            bar();   // every wave holds its Q: the V buffers may take V(0)
        }
        if (T > 0) load_v(cur, 0, v0s);
        if (tr) tr[4] = wall_clock64();

        f32x4 o[2][8];
#pragma unroll
        for (int rb = 0; rb < 2; rb++)
#pragma unroll
            for (int mt = 0; mt < 8; mt++) o[rb][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
        float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};
        float mx[2] = {-INFINITY, -INFINITY};
        bf16x8 pown[2], ppar[2];
        f32x4 s[2][2];
        bool prev_live = false;
        const float sl2 = p.scale_log2;
        constexpr int DEPTH = 4;

        // O += V^T(buffer VB) . P for the previous tile: 16 V^T operands (own key half first), each
        // feeding both 16-row halves; `mid(f)` runs after operand f's two products.
        auto pv = [&](auto VB, auto &&mid) {
            constexpr int vb = decltype(VB)::value;
            auto vread = [&](auto F) {
                constexpr int f = decltype(F)::value, mt = f & 7, kc = f >> 3;
                constexpr int off = vb * 2 * VTILE + (32 * (mt >> 1) + 4 * (mt & 1)) * BK * 2;
                return lds_read16<off>(kc ? va_par : va_own);
            };
            bf16x8 vring[DEPTH];
            static_for<DEPTH>([&](auto I) { vring[decltype(I)::value] = vread(I); });
            mid(std::integral_constant<int, -1>{});
            static_for<16>([&](auto F) {
                constexpr int f = decltype(F)::value, mt = f & 7, kc = f >> 3;
                constexpr int ahead = (15 - f) < (DEPTH - 1) ? (15 - f) : (DEPTH - 1);
                bf16x8 a = vring[f % DEPTH];
                lds_wait<ahead>(a);
                o[0][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, kc ? ppar[0] : pown[0], o[0][mt], 0, 0, 0);
                o[1][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, kc ? ppar[1] : pown[1], o[1][mt], 0, 0, 0);
                if constexpr (f + DEPTH < 16) vring[f % DEPTH] = vread(std::integral_constant<int, f + DEPTH>{});
                mid(F);
            });
        };

        auto tile = [&](const int t, auto BUF) {
            constexpr int buf = decltype(BUF)::value;
            uint16_t *const Kb = buf ? k1s : k0s;
            const int kb = t * BK;
            const bool live = pair_live && (!p.causal || kb <= pair_last_pos);
            // ---- phase 1
            if (prev_live) {
                ppar[0] = lds_read16<0>(pl_par);
                ppar[1] = lds_read16<1024>(pl_par);
            }
            if (live) {
                bf16x8 ring[DEPTH];
                auto kread = [&](auto I) {   // operand st: key tile st & 1, chunk st >> 1
                    constexpr int st = decltype(I)::value, ktl = st & 1, c = st >> 1;
                    return lds_read16<buf * 2 * KTILE + (c >> 2) * 256 + 2048 * ktl>(kb0 + ((64u * ((c & 3) ^ ktl)) ^ kx));
                };
                static_for<DEPTH>([&](auto I) { ring[decltype(I)::value] = kread(I); });
                static_for<16>([&](auto I) {
                    constexpr int st = decltype(I)::value, ktl = st & 1, c = st >> 1;
                    constexpr int ahead = (15 - st) < (DEPTH - 1) ? (15 - st) : (DEPTH - 1);
                    bf16x8 a = ring[st % DEPTH];
                    lds_wait<ahead>(a);
                    if constexpr (c == 0) {
                        s[0][ktl] = f32x4{0.f, 0.f, 0.f, 0.f};
                        s[1][ktl] = f32x4{0.f, 0.f, 0.f, 0.f};
                    }
                    const f16x8 af = __builtin_bit_cast(f16x8, a);
                    s[0][ktl] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, qf[0][c], s[0][ktl], 0, 0, 0);
                    s[1][ktl] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, qf[1][c], s[1][ktl], 0, 0, 0);
                    if constexpr (st + DEPTH < 16) ring[st % DEPTH] = kread(std::integral_constant<int, st + DEPTH>{});
                });
                // element (ktl, i) of half rb is key kb + 32hh + 8g + 4ktl + i
                if ((kb + BK > k_len) || (p.causal && kb + BK - 1 > cur.q_pos0 + row0)) {
                    const int base = kb + 32 * hh + 8 * g;
                    const int lim0 = min(k_len - 1, p.causal ? qpos0 : k_len - 1) - base;
                    const int lim1 = min(k_len - 1, p.causal ? qpos1 : k_len - 1) - base;
#pragma unroll
                    for (int ktl = 0; ktl < 2; ktl++)
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            s[0][ktl][i] = (4 * ktl + i > lim0) ? -INFINITY : s[0][ktl][i];
                            s[1][ktl][i] = (4 * ktl + i > lim1) ? -INFINITY : s[1][ktl][i];
                        }
                }
#pragma unroll
                for (int rb = 0; rb < 2; rb++) {
                    float m = fmaxf(fmaxf(fmaxf(s[rb][0][0], s[rb][0][1]), fmaxf(s[rb][0][2], s[rb][0][3])),
                                    fmaxf(fmaxf(s[rb][1][0], s[rb][1][1]), fmaxf(s[rb][1][2], s[rb][1][3])));
                    mx[rb] = xrow_max(m);
                }
                if (g == 0) {
                    ds_write4<0>(ml_own, mx[0]);
                    ds_write4<64>(ml_own, mx[1]);
                }
            }
            // PV(t-1) reads V(t-1): issued after it are K(t+1) (if any) and V(t)
            if (prev_live) vm_wait(4 + (t + 1 < T ? 4 : 0));
            const bool tail = kb + BK > k_len;
            if (tail) vm_wait(0);   // V(t) is patched below, after A
            bar();   // ---- A(t)
            if (tail) {   // V^T entries of keys >= k_len -> 0 (garbage there would turn P = 0 into NaN)
                uint16_t *const Vs = buf ? v1s : v0s;
                const int valid = k_len - kb;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int sl = tid + 512 * j;
                    const int d = sl >> 3, c = (sl & 7) ^ v_swz(d);
                    const int k0 = c * 8;
                    u32x4 w = *(u32x4 *)(Vs + sl * 8);
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const unsigned keep = (k0 + 2 * e + 1 < valid) ? 0xffffffffu : (k0 + 2 * e < valid ? 0xffffu : 0u);
                        w[e] &= keep;
                    }
                    *(u32x4 *)(Vs + sl * 8) = w;
                }
            }
            if (t + 2 < T) load_k(cur, kb + 2 * BK, Kb);
            else if (t == T - 1 && p.gate) load_rows(cur, k0s, k1s, HD);
            // ---- phase 2
            float pm0 = 0.f, pm1 = 0.f;
            if (live) {
                pm0 = ds_read4<0>(ml_par);
                pm1 = ds_read4<64>(ml_par);
            }
            float mn[2], msub[2], alpha[2], rs[2] = {0.f, 0.f};
            unsigned w[2][4];
            auto head = [&]() {
                const float pm[2] = {pm0, pm1};
#pragma unroll
                for (int rb = 0; rb < 2; rb++) {
                    const float tmx = fmaxf(mx[rb], pm[rb]) * sl2;
                    mn[rb] = (tmx > m_run[rb] + 8.f) ? tmx : m_run[rb];
                    msub[rb] = (mn[rb] == -INFINITY) ? 0.f : mn[rb];
                    alpha[rb] = (mn[rb] == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(m_run[rb] - mn[rb]);
                }
            };
            auto piece = [&](int j) {   // j = 4 rb + jj: keys 8g + 2jj, +1 of half rb
                const int rb = j >> 2, jj = j & 3, ktl = jj >> 1, i = 2 * (jj & 1);
                const float p0 = __builtin_amdgcn_exp2f(fmaf(s[rb][ktl][i], sl2, -msub[rb]));
                const float p1 = __builtin_amdgcn_exp2f(fmaf(s[rb][ktl][i + 1], sl2, -msub[rb]));
                w[rb][jj] = pack_bf16(p0, p1);
                // the row sum takes the rounded P that the P.V product multiplies
                rs[rb] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w[rb][jj]),
                                                         bf16x2{(__bf16)1.0f, (__bf16)1.0f}, rs[rb], false);
            };
            if (prev_live) {
                // the partner's max was read before the V operands: DEPTH reads are younger
                auto mid = [&](auto F) {
                    constexpr int f = decltype(F)::value;
                    if constexpr (f == -1) {
                        lgkm_wait<DEPTH>(pm0);
                        lgkm_wait<DEPTH>(pm1);
                        head();
                    } else if constexpr (f < 8) {
                        piece(f);
                    }
                };
                if (buf) pv(std::integral_constant<int, 0>{}, mid);
                else pv(std::integral_constant<int, 1>{}, mid);
            } else if (live) {
                lgkm_wait<0>(pm0);
                lgkm_wait<0>(pm1);
                head();
#pragma unroll
                for (int j = 0; j < 8; j++) piece(j);
            }
            if (live) {
#pragma unroll
                for (int rb = 0; rb < 2; rb++) {
                    l_run[rb] = l_run[rb] * alpha[rb] + rs[rb];   // the lane's share of the row
                    m_run[rb] = mn[rb];
                }
                if (__any(alpha[0] != 1.f || alpha[1] != 1.f)) {
#pragma unroll
                    for (int mt = 0; mt < 8; mt++) {
                        o[0][mt] *= alpha[0];
                        o[1][mt] *= alpha[1];
                    }
                }
#pragma unroll
                for (int rb = 0; rb < 2; rb++) {
                    u32x4 wv = {w[rb][0], w[rb][1], w[rb][2], w[rb][3]};
                    pown[rb] = __builtin_bit_cast(bf16x8, wv);
                }
                ds_write16(pl_own, pown[0]);
                ds_write16(pl_own + 1024, pown[1]);
            }
            // K(t+1) must have landed before B (issued after it: V(t), K(t+2)); in the last tile
            // V(t) (issued after it: the gate rows)
            if (t + 1 < T) vm_wait(4 + (t + 2 < T ? 4 : 0));
            else if (!tail) vm_wait(p.gate ? 8 : 0);
            bar();   // ---- B(t)
            if (t + 1 < T) load_v(cur, kb + BK, buf ? v0s : v1s);
            prev_live = live;
        };
        for (int t = 0; t < T; t += 2) {
            tile(t, std::integral_constant<int, 0>{});
            if (t + 1 < T) tile(t + 1, std::integral_constant<int, 1>{});
        }
        if (prev_live) {   // the last tile's P.V
            ppar[0] = lds_read16<0>(pl_par);
            ppar[1] = lds_read16<1024>(pl_par);
            lgkm_wait<0>(ppar[1]);
            auto none = [](auto) {};
            if (T & 1) pv(std::integral_constant<int, 0>{}, none);
            else pv(std::integral_constant<int, 1>{}, none);
        }
        if (tr) tr[5] = wall_clock64();

        // ---- Epilogue: O / l times sigmoid(gate). Lane (q16, g) of half rb holds row 32 pr + 16 rb
        // + q16, dims 128 hh + 32 u + 8 g + [0, 8) for u < 4. l adds the partner's key half.
        float lrow[2];
        lrow[0] = xrow_sum(l_run[0]);
        lrow[1] = xrow_sum(l_run[1]);
        if (g == 0) {
            ds_write4<0>(ml_own, lrow[0]);
            ds_write4<64>(ml_own, lrow[1]);
        }
        vm_wait(0);
        bar();   // gate rows in LDS, every P.V done (V buffers free), row sums exchanged
        float lp0 = ds_read4<0>(ml_par), lp1 = ds_read4<64>(ml_par);
        lgkm_wait<0>(lp0);
        lgkm_wait<0>(lp1);
        const float lt[2] = {lrow[0] + lp0, lrow[1] + lp1};
        const int q_row0 = cur.q_row0, flag_row = cur.flag_row, h = cur.h, nq = cur.nq;
        item = items.get(k + 1);
        if (item >= 0) {
            cur = decode(item);
            load_rows(cur, v0s, v1s, 0);
        }
        int32_t *flag = p.ovf ? p.ovf + flag_row : nullptr;
#pragma unroll
        for (int rb = 0; rb < 2; rb++) {
            const int my_q = row0 + 16 * rb + q16;
            if (my_q < nq) {
                const float il = lt[rb] > 0.f ? 1.f / lt[rb] : 0.f;
                const size_t tt = (size_t)q_row0 + my_q;
                const unsigned gbase = lds_addr(my_q < 64 ? k0s : k1s) + (unsigned)(my_q & 63) * 512u;
                bf16x8 gv[4];
                if (p.gate) {
#pragma unroll
                    for (int u = 0; u < 4; u++)
                        gv[u] = lds_read16<0>(gbase + (unsigned)(((16 * hh + 4 * u + g) ^ (my_q & 15)) * 16));
                    lgkm_wait<0>(gv[3]);
                }
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    float v[8];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        v[i] = o[rb][2 * u][i] * il;
                        v[4 + i] = o[rb][2 * u + 1][i] * il;
                    }
                    if (p.gate) {
                        const u32x4 gw = __builtin_bit_cast(u32x4, gv[u]);
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            v[2 * j] *= sigmoidf(bf_lo(gw[j]));
                            v[2 * j + 1] *= sigmoidf(bf_hi(gw[j]));
                        }
                    }
                    store_out8(p.out, tt * p.out_ld + (size_t)h * HD + 128 * hh + 32 * u + 8 * g, v, p.out_type, p.f16_lim, flag);
                }
            }
        }
        if (item >= 0) {
            bar();   // every wave has read its gate values: the K buffers are free
            if (cur.n_tiles > 0) load_k(cur, 0, k0s);
            if (cur.n_tiles > 1) load_k(cur, BK, k1s);
        }
        if (tr) tr[1] = wall_clock64();
        if (item < 0) break;
    }
}

template <int NROT>
__global__ __launch_bounds__(512, 1) void attn_text_pair_kernel(AttnParams p) {
    __shared__ __attribute__((aligned(16))) uint16_t smem[tpair::SMEM_BYTES / 2];
    __shared__ __attribute__((aligned(16))) float qn_lds[text::HD];
    text_pair_items<NROT>(p, smem, qn_lds);
}

}  // namespace clef_hip
