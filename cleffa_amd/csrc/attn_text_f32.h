// FP32 text attention for head dim 256 on CDNA4 (gfx950): the precision the reference's FP32
// kernels give (metal/clef.metal:250-302 attn_prep, 316-654 attention / attention_fa /
// attention_reuse / attention_prefetch_64), used for the per-record rerun after an f16 overflow
// (clef.c:526-550) and with CLEF_ATTN_TU=0.
//
// Semantics (the reference's, per query row t of head h, kv head h / (nh / nkv)):
//   q, k = RMSNorm(x) * w (w as given, already 1 + w), then partial rotary over dims [0, 64):
//   pair (i, i + 32) turns by pos3[t][i % 3] * inv_freq[i]; V copied. S = (q . k) * scale over
//   the record's keys up to the query's position, softmax with exp, O = P.V / l, times
//   sigmoid(gate) (the second half of the head's row), written through act16 (bf16, or f16
//   that saturates and flags the record) or as f32.
//
// Everything is FP32: the products run on v_mfma_f32_16x16x4f32 (FP32 operands, FP32
// accumulation), the softmax in FP32 VALU (exp2 domain). Key tiles start at the record's first key, so a
// record's arithmetic does not depend on what is packed with it.
//
// Workgroup: a chunk of W <= 8 q heads of the GQA group (a group of more than 8 heads runs as
// several chunks), X = 1 or 2 waves per head, all on the same 16 query rows, so one 32-key K / V
// tile in LDS (64 KB, double buffered: 128 KB) serves the chunk. With two waves per head each
// takes half of the head dims (see attn_text_f32_kernel).
//   S^T = K . Q^T      A = 16 keys x 4 dims of K (LDS), B = the wave's Q (registers).
//   O^T += V^T . P^T   A = 16 dims x 4 keys of V (LDS), B = P (registers).
// Lane l = 16 g + r. S^T's A row r takes key 4(r % 4) + r / 4 of the 16-key subtile, so the four
// scores a lane holds (accumulator rows 4g + v) are keys 4v + g: the B operand of the four 4-key
// steps of the P.V product, with no shuffle. In S^T, lane (g, r) reads chunks 16g + j of its
// key's K row (dims 64g + 4j + e); the K rows are padded to 1,040 bytes so those 16 rows fall in
// distinct banks. In the P.V product, read j of lane r takes chunk 16j + r of its key's V row: a
// read's 16 lanes cover 256 contiguous bytes. The A row r of dim tile 4j + e is then dim
// 64j + 4r + e, and accumulator v of lane (g, r) in tile 4j + e holds dim 64j + 16g + 4v + e of
// query row r. Every LDS read is a per-lane base register plus an immediate offset.
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <utility>

#include "attn_kernels.h"
#include "clef_hip_attn.h"

namespace clef_hip {
namespace text32 {

constexpr int HD = 256;
constexpr int BQ = 16;                  // query rows per workgroup
constexpr int SUB = 128 / BQ;           // workgroups per 128-row plan block
constexpr int BK = 32;                  // keys per LDS tile
constexpr int ROW = HD + 4;             // LDS floats per key row: 1,040 bytes, so the 16 rows
                                        // one K read touches start 16 bytes apart in the banks
constexpr int TILE = BK * ROW;          // floats per K or V tile (32.5 KB)
constexpr int TB = TILE * 4;            // bytes per tile
constexpr int RUN = 4;                  // K chunks read ahead of their products
constexpr int NRUN = 16 / RUN;

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((address_space(3))) void lds_void;

struct PrepParams {
    const float *qkv;           // [T][row]
    const float *k_norm;        // [256] or NULL
    const int32_t *pos3;
    const float *inv_freq;      // [32]
    const int32_t *kv_tok;      // pass row of each plane row, -1: not written
    float *k_plane, *v_plane;   // [nkv][kvT][256]
    float *rope_cs;             // [T][32][2] or NULL
    int kv_rows, row, nh, nkv, n_rot, kvT;
    float eps;
};

struct Params {
    const float *qkv;
    const float *q_norm;        // [256] or NULL
    const int32_t *pos3;
    const float *inv_freq;
    const float *rope_cs;       // [T][32][2] written by the prep, or NULL
    const float *k_plane, *v_plane;
    const int32_t *blocks;      // the plan's 128-row blocks {q_row0, nq, q_pos0, k_row0, k_len, flag_row, ..}
    void *out;
    int32_t *ovf;
    int row, kvT, nh, nkv, n_rot, causal, gate, out_type;
    int n_blk, n_chunks;        // plan blocks; head chunks per kv group (ceil(group / 8))
    float eps, scale, f16_lim;
};

// The rotary angle's cos / sin in full FP32 precision (the reference: precise::cos / sin).
__device__ __forceinline__ void rope_cs_f32(const int32_t *pos3, const float *inv_freq, int t, int i, float *c, float *s) {
    const float ang = (float)pos3[3 * (size_t)t + i % 3] * inv_freq[i];
    sincosf(ang, s, c);
}

// K / V prologue, FP32 planes: 32 lanes per (plane row, kv head); lane holds dims lane + 32 j,
// so the rotary pair (i, i + 32), i < 32, sits in one lane. Plane rows with kv_tok -1 are left
// as they are. Head 0's groups also store the rotary cos / sin of their pass row.
__global__ __launch_bounds__(256) void text_prep_kv_f32_kernel(PrepParams p) {
    const long item = (long)blockIdx.x * 8 + (threadIdx.x >> 5);
    const int lane = threadIdx.x & 31;
    if (item >= (long)p.kv_rows * p.nkv) return;
    const int r = (int)(item / p.nkv), kh = (int)(item % p.nkv);
    const int t = p.kv_tok[r];
    if (t < 0) return;
    const float *src = p.qkv + (size_t)t * p.row + (size_t)p.nh * 2 * HD + (size_t)kh * HD;
    float x[8], v[8], ss = 0.f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        x[j] = src[lane + 32 * j];
        v[j] = src[(size_t)p.nkv * HD + lane + 32 * j];
        ss += x[j] * x[j];
    }
    if (p.k_norm) {
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 32);
        const float inv = 1.0f / sqrtf(ss / (float)HD + p.eps);
#pragma unroll
        for (int j = 0; j < 8; j++) x[j] = x[j] * inv * p.k_norm[lane + 32 * j];
    }
    if (p.n_rot) {
        float c, s;
        rope_cs_f32(p.pos3, p.inv_freq, t, lane, &c, &s);
        const float x0 = x[0], x1 = x[1];
        x[0] = x0 * c - x1 * s;
        x[1] = x1 * c + x0 * s;
        if (p.rope_cs && kh == 0) *(float2 *)(p.rope_cs + ((size_t)t * 32 + lane) * 2) = make_float2(c, s);
    }
    float *kd = p.k_plane + ((size_t)kh * p.kvT + r) * HD, *vd = p.v_plane + ((size_t)kh * p.kvT + r) * HD;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        kd[lane + 32 * j] = x[j];
        vd[lane + 32 * j] = v[j];
    }
}

// max over the four 16-lane rows of a wave (permlane swaps, VALU only); every lane gets it
__device__ __forceinline__ float xrow_max(float x) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float m = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    return fmaxf(__uint_as_float(q[0]), __uint_as_float(q[1]));
}

template <int OFF>
__device__ __forceinline__ f32x4 lds_read_f4(unsigned addr) {
    f32x4 r;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF) : "memory");
    return r;
}
template <int N>
__device__ __forceinline__ void lds_wait_f4(f32x4 &r) {
    asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(r) : "i"(N));
}

template <typename F, int... I>
__device__ __forceinline__ void sfor_impl(F &&f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void sfor(F &&f) {
    sfor_impl(f, std::make_integer_sequence<int, N>{});
}

// Work items are (16-row sub-block, kv head, head chunk): the kv group's G = nh / nkv q heads
// split into n_chunks chunks of at most W <= 8 heads, X waves per head (a chunk's spare waves
// fill tiles and take barriers but compute nothing). With X = 2 the two waves of a head split
// its 256 dims: wave (slot s, half x), wave id s + W x, holds Q steps c = 4j + e of the chunks
// j in {4x .. 4x + 3, 8 + 4x .. 8 + 4x + 3} (so a rotary pair (i, i + 32) stays in one wave)
// and O for dims 128x .. 128x + 127; the halves' partial scores meet through LDS and each wave
// adds its partner's to its own (the same sum in both, bitwise), then both run the softmax. Six
// q heads then fill twelve waves, three per SIMD, where six waves left two SIMDs with one. Items run in the plan's longest-first
// block order, each block's last 16 rows (its longest causal rows) first. With G workgroups,
// workgroup b takes items b, then 2G - 1 - b, ... (snake order, so long and short items mix;
// one item each when G is the item count); while an item's epilogue runs, the next item's
// first K / V tile loads into the idle LDS buffers.
template <int W, int X>
__global__ __launch_bounds__(64 * W * X) void attn_text_f32_kernel(Params p) {
    static_assert(X == 1 || X == 2, "one or two waves per head");
    constexpr int NW = W * X;           // waves
    constexpr int QN = 64 / X;          // Q steps (and B registers) per wave
    __shared__ __attribute__((aligned(16))) float smem[4 * TILE];   // K0 | K1 | V0 | V1
    // partial scores of the two halves: slot (wave, lane) holds its two 16-key subtiles
    __shared__ __attribute__((aligned(16))) f32x4 xch[X > 1 ? NW * 64 * 2 : 1];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int slot = X == 1 ? wave : wave % W, half = X == 1 ? 0 : wave / W;   // head slot in the chunk, dim half
    const int r16 = lane & 15, g = lane >> 4;
    const int group = p.nh / p.nkv;
    const int n_items = p.n_blk * SUB * p.nkv * p.n_chunks;
    const int G = gridDim.x;
    struct Item {
        int nq, q_row0, q_pos0, k_row0, k_len, n_tiles, kh, h;
        bool live;   // this wave has a head in the item's chunk
        int32_t *flag;
    };
    // the k-th item of this workgroup, or nq = 0 past the end
    auto item_at = [&](int k, Item &it) {
        const int j = k * G + ((k & 1) ? G - 1 - (int)blockIdx.x : (int)blockIdx.x);
        it.nq = 0;
        if (j >= n_items) return false;
        const int chunk = j % p.n_chunks, rest = j / p.n_chunks;
        it.kh = rest % p.nkv;
        const int sb = rest / p.nkv, bi = sb / SUB, sub = SUB - 1 - sb % SUB;
        const int32_t *blk = p.blocks + 8 * bi;
        it.nq = min(BQ, blk[1] - BQ * sub);
        if (it.nq <= 0) { it.nq = 0; return true; }      // a sub-block past the block's rows
        it.q_row0 = blk[0] + BQ * sub;
        it.q_pos0 = blk[2] + BQ * sub;
        it.k_row0 = blk[3];
        it.k_len = p.causal ? min(blk[4], it.q_pos0 + it.nq) : blk[4];
        it.n_tiles = (it.k_len + BK - 1) / BK;
        it.flag = p.ovf ? p.ovf + blk[5] : nullptr;
        const int hw = chunk * W + slot;
        it.live = hw < group;
        it.h = it.kh * group + (it.live ? hw : 0);
        return true;
    };
    // next item with rows, from ordinal k on; false past the end
    auto advance = [&](int &k, Item &it) {
        while (item_at(k, it)) {
            if (it.nq > 0) return true;
            k++;
        }
        return false;
    };

    // ---- tile fills: one 1 KB DMA group per key row; wave w fills rows w, w + NW, ...
    auto fill = [&](const Item &it, int kb, float *Ks, float *Vs) {
        const float *kbase = p.k_plane + ((size_t)it.kh * p.kvT + it.k_row0) * HD;
        const float *vbase = p.v_plane + ((size_t)it.kh * p.kvT + it.k_row0) * HD;
        for (int r = wave; r < BK; r += NW) {
            const size_t off = (size_t)(kb + r) * HD + 4 * lane;
            __builtin_amdgcn_global_load_lds((const void *)(kbase + off), (lds_void *)(Ks + r * ROW), 16, 0, 0);
            __builtin_amdgcn_global_load_lds((const void *)(vbase + off), (lds_void *)(Vs + r * ROW), 16, 0, 0);
        }
    };
    // Rows past the keys (not written by this pass, possibly not finite) -> 0 in V, so that the
    // zero probabilities of masked keys give exact zero products.
    auto clear_tail = [&](const Item &it, int kb, float *Vs) {
        if (kb + BK <= it.k_len) return;                  // workgroup-uniform
        for (int r = wave; r < BK; r += NW)
            if (kb + r >= it.k_len) *(f32x4 *)(Vs + r * ROW + 4 * lane) = f32x4{0.f, 0.f, 0.f, 0.f};
    };

    const unsigned lds0 = (unsigned)(uintptr_t)(const __attribute__((address_space(3))) float *)smem;
    // K: row 4(r16 % 4) + r16 / 4 of subtile 0, chunk 16g (+ 4 half); V: row g, chunk r16
    // (+ 32 half) (buffer 0)
    const unsigned ka = lds0 + (unsigned)(4 * (r16 & 3) + (r16 >> 2)) * ROW * 4u + 256u * g + 64u * half;
    const unsigned va = lds0 + 2u * TB + (unsigned)g * ROW * 4u + 16u * r16 + 512u * half;
    // the K chunk (of 16 per 64 dims) of this wave's chunk step q4
    auto kchunk = [](int q4) { return X == 1 ? q4 : (q4 < 4 ? q4 : q4 + 4); };

    int k = 0;
    Item cur;
    if (!advance(k, cur)) return;
    if (cur.n_tiles > 0) fill(cur, 0, smem, smem + 2 * TILE);
    for (;;) {
        const bool q_valid = r16 < cur.nq;
        const int qpos = cur.q_pos0 + r16;
        const int t = cur.q_row0 + (q_valid ? r16 : 0);
        const int h = cur.h;
        const int k_len = cur.k_len, n_tiles = cur.n_tiles;

        // ---- Q prologue: lane holds Q[row r16][64 g + c(q)] for the wave's QN steps q, with
        // c(q) = 4 kchunk(q / 4) + q % 4 + 16 half: normalised (the sum of squares over the
        // whole row) and rotated, FP32. Rotary pair i < 32 / X of the wave is (qv[i], qv[i + NP]),
        // dims 16 half + i and 32 + 16 half + i (lanes g = 0).
        constexpr int NP = 32 / X;
        constexpr int RX = X == 1 ? RUN : 2;   // K chunks per run (two per run in the split layout, for registers)
        float qv[QN];
        {
            float ss = 0.f;
            {
                // the wave's own QN elements of the lane's 64 (the chunks kchunk(q4) + 4 half)
                const float *qs = p.qkv + (size_t)t * p.row + (size_t)h * 2 * HD + 64 * g + 16 * half;
#pragma unroll
                for (int q4 = 0; q4 < QN / 4; q4++) {
                    const f32x4 v = *(const f32x4 *)(qs + 4 * kchunk(q4));
                    qv[4 * q4] = v.x; qv[4 * q4 + 1] = v.y; qv[4 * q4 + 2] = v.z; qv[4 * q4 + 3] = v.w;
                }
                if (p.q_norm) {
#pragma unroll
                    for (int q = 0; q < QN; q++) ss += qv[q] * qv[q];
                }
            }
            if (p.q_norm) {
                ss += __shfl_xor(ss, 16);
                ss += __shfl_xor(ss, 32);
                if constexpr (X > 1) {
                    // the two halves' sums of squares meet through LDS: the row's sum is the same
                    // in both (own + partner's); the nop covers a VALU result read by the LDS write
                    float *xs = (float *)xch;
                    asm volatile("s_nop 1\n\tds_write_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier"
                                 : : "v"((unsigned)(uintptr_t)(const __attribute__((address_space(3))) float *)(xs + wave * 64 + lane)), "v"(ss) : "memory");
                    float o;
                    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)"
                                 : "=v"(o) : "v"((unsigned)(uintptr_t)(const __attribute__((address_space(3))) float *)(xs + (half ? wave - W : wave + W) * 64 + lane)) : "memory");
                    ss = half ? o + ss : ss + o;
                }
                const float inv = 1.0f / sqrtf(ss / (float)HD + p.eps);
                const float *w = p.q_norm + 64 * g + 16 * half;
#pragma unroll
                for (int q4 = 0; q4 < QN / 4; q4++) {
                    const f32x4 wv = *(const f32x4 *)(w + 4 * kchunk(q4));
#pragma unroll
                    for (int e = 0; e < 4; e++) qv[4 * q4 + e] = qv[4 * q4 + e] * inv * wv[e];
                }
            }
            if (p.n_rot && g == 0) {
#pragma unroll
                for (int i = 0; i < NP; i++) {
                    const int i0 = NP * half + i;
                    float c, s;
                    if (p.rope_cs) {
                        const float2 cs = *(const float2 *)(p.rope_cs + ((size_t)t * 32 + i0) * 2);
                        c = cs.x; s = cs.y;
                    } else {
                        rope_cs_f32(p.pos3, p.inv_freq, t, i0, &c, &s);
                    }
                    const float x0 = qv[i], x1 = qv[i + NP];
                    qv[i] = x0 * c - x1 * s;
                    qv[i + NP] = x1 * c + x0 * s;
                }
            }
            // the scores in the exp2 domain: scale * log2 e folded into Q
            const float sl2 = p.scale * 1.4426950408889634f;
#pragma unroll
            for (int q = 0; q < QN; q++) qv[q] *= sl2;
        }
        __builtin_amdgcn_s_waitcnt(0);
        if (n_tiles > 0) clear_tail(cur, 0, smem + 2 * TILE);
        __syncthreads();

        constexpr int NO = 16 / X;   // dim tiles 4j + e of this wave (j < 4 / X)
        f32x4 o[NO];
#pragma unroll
        for (int n = 0; n < NO; n++) o[n] = f32x4{0.f, 0.f, 0.f, 0.f};
        float m_run = -INFINITY, l_run = 0.f;

        auto tile = [&](const int ti, auto BUF) {
            constexpr int buf = decltype(BUF)::value;
            const int kb = ti * BK;
            if (ti + 1 < n_tiles) fill(cur, kb + BK, smem + (buf ^ 1) * TILE, smem + 2 * TILE + (buf ^ 1) * TILE);
            // S^T: two 16-key subtiles, QN four-dim steps each, their products interleaved (two
            // independent accumulator chains); K read in runs of RX chunks per subtile
            f32x4 s[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
            if (cur.live) {   // wave-uniform: a spare wave of the last head chunk only fills
                sfor<16 / X / RX>([&](auto H) {
                    constexpr int hh = decltype(H)::value;
                    f32x4 a[2][RX];
                    sfor<RX>([&](auto J) {
                        constexpr int j = decltype(J)::value;
                        constexpr int ch = X == 1 ? RX * hh + j : (RX * hh + j < 4 ? RX * hh + j : RX * hh + j + 4);
                        a[0][j] = lds_read_f4<buf * TB + ch * 16>(ka);
                        a[1][j] = lds_read_f4<buf * TB + 16 * ROW * 4 + ch * 16>(ka);
                    });
                    sfor<RX>([&](auto J) {
                        constexpr int j = decltype(J)::value;
                        lds_wait_f4<2 * (RX - 1 - j) + 1>(a[0][j]);
                        lds_wait_f4<2 * (RX - 1 - j)>(a[1][j]);
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            s[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[0][j][e], qv[4 * (RX * hh + j) + e], s[0], 0, 0, 0);
                            s[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[1][j][e], qv[4 * (RX * hh + j) + e], s[1], 0, 0, 0);
                        }
                    });
                });
            }
            if constexpr (X > 1) {
                // the halves' partial scores meet: write this wave's, barrier, add the partner's
                const unsigned xa = (unsigned)(uintptr_t)(const __attribute__((address_space(3))) f32x4 *)(xch + 2 * (wave * 64 + lane));
                // (the wait states cover an MFMA result read by the LDS write: the compiler does
                // not see inside the statement)
                asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 4\n\tds_write_b128 %0, %1\n\tds_write_b128 %0, %2 offset:16" : : "v"(xa), "v"(s[0]), "v"(s[1]) : "memory");
                asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
                const unsigned pa = xa + (half ? -1 : 1) * (unsigned)(W * 64 * 32);
                f32x4 t0, t1;
                asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %2 offset:16\n\ts_waitcnt lgkmcnt(0)" : "=&v"(t0), "=&v"(t1) : "v"(pa) : "memory");
                s[0] += t0;
                s[1] += t1;
            }
            if (cur.live) {
                // V chunk j of step st = (u, v): key 16u + 4v + g, chunk 16j + r16 of its row
                auto vread = [&](auto ST, auto J) {
                    constexpr int st = decltype(ST)::value, u = st >> 2, v = st & 3, j = decltype(J)::value;
                    return lds_read_f4<buf * TB + (16 * u + 4 * v) * ROW * 4 + 256 * j>(va);
                };
                constexpr int NJ = 4 / X;   // V chunks per step of this wave
                f32x4 vb[NJ];   // step 0's chunks load while the softmax runs
                sfor<NJ>([&](auto J) { vb[decltype(J)::value] = vread(std::integral_constant<int, 0>{}, J); });
                // Online softmax. s[u][v] is the score of key kb + 16u + 4v + g for query row r16.
                float x[2][4], mx = -INFINITY;
#pragma unroll
                for (int u = 0; u < 2; u++)
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        const int key = kb + 16 * u + 4 * v + g;
                        const bool ok = q_valid && key < k_len && (!p.causal || key <= qpos);
                        x[u][v] = ok ? s[u][v] : -INFINITY;
                        mx = fmaxf(mx, x[u][v]);
                    }
                const float mn = fmaxf(m_run, xrow_max(mx));
                float pv[2][4];
                float alpha = 1.f, rs = 0.f;
                if (mn != -INFINITY) {
                    alpha = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run - mn);
#pragma unroll
                    for (int u = 0; u < 2; u++)
#pragma unroll
                        for (int v = 0; v < 4; v++) {
                            pv[u][v] = x[u][v] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(x[u][v] - mn);
                            rs += pv[u][v];
                        }
                } else {
#pragma unroll
                    for (int u = 0; u < 2; u++)
#pragma unroll
                        for (int v = 0; v < 4; v++) pv[u][v] = 0.f;
                }
                m_run = mn;
                l_run = l_run * alpha + rs;
                const float alpha_o = alpha;
                // O^T += V^T . P^T: 8 four-key steps (u, v), each 16 dim tiles. The V chunks roll
                // through four registers: chunk j of the next step is read as soon as the current
                // step's chunk j has fed its four products, so three reads are always in flight.
#pragma unroll
                for (int n = 0; n < NO; n++) o[n] *= alpha_o;
                sfor<8>([&](auto S) {
                    constexpr int st = decltype(S)::value, u = st >> 2, v = st & 3;
                    const float b = pv[u][v];
                    sfor<NJ>([&](auto J) {
                        constexpr int j = decltype(J)::value;
                        if constexpr (st + 1 < 8) lds_wait_f4<NJ - 1>(vb[j]);
                        else lds_wait_f4<NJ - 1 - j>(vb[j]);
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            o[4 * j + e] = __builtin_amdgcn_mfma_f32_16x16x4f32(vb[j][e], b, o[4 * j + e], 0, 0, 0);
                        if constexpr (st + 1 < 8) vb[j] = vread(std::integral_constant<int, st + 1>{}, J);
                    });
                });
            }
            __builtin_amdgcn_s_waitcnt(0);
            if (ti + 1 < n_tiles) clear_tail(cur, kb + BK, smem + 2 * TILE + (buf ^ 1) * TILE);
            __syncthreads();
        };
        for (int ti = 0; ti < n_tiles; ti += 2) {
            tile(ti, std::integral_constant<int, 0>{});
            if (ti + 1 < n_tiles) tile(ti + 1, std::integral_constant<int, 1>{});
        }

        // ---- the next item's first tile loads into the buffers the key loop has left (every
        // wave passed its closing barrier) while this item's epilogue runs
        const Item done = cur;
        k++;
        const bool more = advance(k, cur);
        if (more && cur.n_tiles > 0) fill(cur, 0, smem, smem + 2 * TILE);

        // ---- epilogue: O = O^T / l, times sigmoid(gate). Accumulator n = 4j + e, entry v of lane
        // (g, r16) is dim 64j + 16g + 4v + e of row r16.
        float l_row = l_run;
        l_row += __shfl_xor(l_row, 16);
        l_row += __shfl_xor(l_row, 32);
        if (q_valid && done.live) {
            const float il = l_row > 0.f ? 1.0f / l_row : 0.f;
            const float *grow = p.qkv + (size_t)t * p.row + (size_t)h * 2 * HD + HD;
            const size_t obase = (size_t)t * p.nh * HD + (size_t)h * HD;
#pragma unroll
            for (int v = 0; v < 4; v++)
#pragma unroll
                for (int j = 0; j < 4 / X; j++) {
                    const int d = 64 * (j + (4 / X) * half) + 16 * g + 4 * v;
                    f32x4 w;
#pragma unroll
                    for (int e = 0; e < 4; e++) w[e] = o[4 * j + e][v] * il;
                    if (p.gate) {
                        const f32x4 gv = *(const f32x4 *)(grow + d);
#pragma unroll
                        for (int e = 0; e < 4; e++) w[e] = w[e] * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-gv[e] * 1.4426950408889634f));
                    }
                    store_out4(p.out, obase + d, w, p.out_type, p.f16_lim, done.flag);
                }
        }
        if (!more) break;
    }
}

}  // namespace text32
}  // namespace clef_hip
