// The text path's K/V prologue on a tile of pass rows held in LDS (bf16, row stride cs bytes):
// K rows are RMS-normalised, rotated (partial NeoX rotary, interleaved M-RoPE angles) and split
// to the f16 K plane; V rows go to the V^T plane. Semantics: metal/clef.metal:245-300 (attn_prep
// K and V) and 857-928 (split16 and attn_prep_split: the f16 planes, |x| > f16_lim or NaN
// saturating and flagging the record).
//
// Two producers: the QKV GEMM (gemm_kernel.h) leaves its bf16 output tile in LDS and runs k_rows /
// v_rows on it; text_prep_direct_kernel reads the qkv rows straight into registers. Both go through
// k_row_out, rope_sincos and v_word, so the planes they write are bitwise the same.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_kernels.h"

namespace clef_hip {

struct KvRows {
    int T, nh, nkv, n_rot, kvT;
    float eps, f16_lim;
    const float *k_norm;      // [256] or NULL
    const int32_t *pos3;      // [T][3]
    const float *inv_freq;    // [n_rot / 2]
    const int32_t *tok_kv;    // [T]: plane row of each pass row's key
    const int32_t *seq_start; // [T] or NULL
    int32_t *ovf;             // [T] or NULL
    uint16_t *k_plane;        // [nkv][kvT][256] f16
    uint16_t *vt_plane;       // [nkv][256][kvT] bf16
    float *rope_cs;           // [T][n_rot / 2][2] or NULL
};

// The rotary cos/sin of row `row` (pass row m0 + row), pairs 2k and 2k + 1, into the table (and,
// for kv head 0, into rope_cs for the Q prologue).
__device__ __forceinline__ void k_table(const KvRows &p, int m0, int row, int k, int kh, float2 *table) {
    const int t = m0 + row, half_rot = p.n_rot / 2;
    if (t >= p.T) return;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int i = 2 * k + h;
        const float ang = (float)p.pos3[3 * (size_t)t + i % 3] * p.inv_freq[i];
        float sn, cn;
        rope_sincos(ang, &sn, &cn);
        table[32 * row + i] = make_float2(cn, sn);
        if (p.rope_cs && kh == 0) *(float2 *)(p.rope_cs + (size_t)t * 2 * half_rot + 2 * i) = make_float2(cn, sn);
    }
}

// K rows m0 .. m0 + BM - 1 of kv head kh (those below T): 16 lanes per row, 16 dims per lane,
// NTHREADS / 16 rows per pass. Lane k of a row holds dims d(k, e), e < 16: for k < 4 the rotary
// pairs in place, dims 8k + e and 32 + 8k + e for e < 8 (pair i = 8k + e is x[e], x[e + 8]), and
// for k >= 4 dims 64 + 16(k - 4) + e; so the rotation needs no lane exchange. Each pass first
// computes the rotary cos/sin of its rows, two pairs per lane, into `table` (LDS,
// [NTHREADS / 16][32] float2), and kv head 0 stores them in rope_cs for the Q prologue. Every
// thread runs every pass (the table needs two barriers). TABLED: one pass (NTHREADS / 16 == BM)
// whose table the caller has already filled with k_table and made visible.
__device__ __forceinline__ int k_lane_dim(int k, int h) {   // first dim of the lane's half h (8 dims)
    return k < 4 ? 8 * k + 32 * h : 64 + 16 * (k - 4) + 8 * h;
}
// One K row's arithmetic, lane k of its 16 (dims d(k, 0..15) as above, the row's bf16 values in
// kw0 / kw1): RMSNorm with the lane's weights wn, the rotary turn of the lane's pairs with their
// (cos, sin) in c4 (lanes k < 4; c4[q] holds pairs 8k + 2q and 8k + 2q + 1), split16's
// saturation and flag, and the f16 stores to plane row tok_kv[t]. All 16 lanes of the row call it
// together (the sum of squares is a row-wide DPP sum). Every producer of the K plane goes through
// here, so the planes come out bitwise the same whichever wrote them.
__device__ __forceinline__ void k_row_out(const KvRows &p, const u32x4 &kw0, const u32x4 &kw1, const float (&wn)[16],
                                          const float4 (&c4)[4], int k, int t, int kh) {
    constexpr int HD = 256;
    const int d0 = k_lane_dim(k, 0), d1 = k_lane_dim(k, 1);
    float x[16];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        x[2 * j] = bf_lo(kw0[j]);
        x[2 * j + 1] = bf_hi(kw0[j]);
        x[8 + 2 * j] = bf_lo(kw1[j]);
        x[8 + 2 * j + 1] = bf_hi(kw1[j]);
    }
    if (p.k_norm) {
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 16; e++) ss += x[e] * x[e];
        ss = row16_sum(ss);
        const float inv = rsqrtf(ss / (float)HD + p.eps);
#pragma unroll
        for (int e = 0; e < 16; e++) x[e] *= inv * wn[e];
    }
    if (p.n_rot && k < 4) {   // pair 8k + e: x[e] turns with x[e + 8]
#pragma unroll
        for (int q = 0; q < 4; q++) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int e = 2 * q + h;
                const float cn = h ? c4[q].z : c4[q].x, sn = h ? c4[q].w : c4[q].y;
                const float x0 = x[e], x1 = x[e + 8];
                x[e] = x0 * cn - x1 * sn;
                x[e + 8] = x1 * cn + x0 * sn;
            }
        }
    }
    // split16's saturation: the largest magnitude decides (NaN propagates through the maximum,
    // and fails the compare); only a row holding one takes the elementwise pass
    float amax = 0.f;
#pragma unroll
    for (int e = 0; e < 16; e += 2)
        amax = __builtin_elementwise_maximum(amax, __builtin_elementwise_maximum(fabsf(x[e]), fabsf(x[e + 1])));
    if (!(amax <= p.f16_lim)) {
#pragma unroll
        for (int e = 0; e < 16; e++)
            if (!(fabsf(x[e]) <= p.f16_lim)) x[e] = copysignf(65504.f, x[e]);
        if (p.ovf && p.seq_start) __hip_atomic_store(p.ovf + p.seq_start[t], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    uint16_t *dst = p.k_plane + ((size_t)kh * p.kvT + p.tok_kv[t]) * HD;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const float *xs = x + 8 * h;
        u32x4 ko = {pack_f16(xs[0], xs[1]), pack_f16(xs[2], xs[3]), pack_f16(xs[4], xs[5]), pack_f16(xs[6], xs[7])};
        *(u32x4 *)(dst + (h ? d1 : d0)) = ko;
    }
}

// the lane's k_norm weights, in its dim order
__device__ __forceinline__ void k_lane_weights(const KvRows &p, int k, float (&wn)[16]) {
    const int d0 = k_lane_dim(k, 0), d1 = k_lane_dim(k, 1);
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const float4 w4 = *(const float4 *)(p.k_norm + ((q < 2) ? d0 : d1) + 4 * (q & 1));
        wn[4 * q] = w4.x; wn[4 * q + 1] = w4.y; wn[4 * q + 2] = w4.z; wn[4 * q + 3] = w4.w;
    }
}

// A V word (two bf16 of one row) through split16's check: |v| > f16_lim or NaN saturates to
// +-65536 (bf16's rounding of 65504); returns whether any did.
__device__ __forceinline__ bool v_word(unsigned &w, float lim) {
    const bool lo_bad = !(__uint_as_float((w & 0x7fffu) << 16) <= lim), hi_bad = !(__uint_as_float(w & 0x7fff0000u) <= lim);
    if (lo_bad) w = (w & 0xffff8000u) | 0x4780u;
    if (hi_bad) w = (w & 0x8000ffffu) | 0x47800000u;
    return lo_bad | hi_bad;
}

template <int NTHREADS, int BM, bool TABLED = false>
__device__ __forceinline__ void k_rows(const KvRows &p, const uint8_t *ct, int cs, int m0, int kh, float2 *table) {
    static_assert(!TABLED || NTHREADS / 16 == BM, "a caller-filled table covers one pass");
    constexpr int HD = 256, RPP = NTHREADS / 16;
    const int tid = threadIdx.x, rr = tid >> 4, k = tid & 15;
    const int half_rot = p.n_rot / 2;   // 0 or 32: dims [0, 32) pair with [32, 64)
    const int d0 = k_lane_dim(k, 0), d1 = k_lane_dim(k, 1);
    float wn[16];
    if (p.k_norm) k_lane_weights(p, k, wn);
    for (int pass = 0; pass < BM / RPP; pass++) {
        const int row = RPP * pass + rr, t = m0 + row;
        const bool valid = t < p.T;
        if (half_rot && !TABLED) {
            k_table(p, m0 + RPP * pass, rr, k, kh, table);
            __syncthreads();
        }
        if (valid) {
            const u32x4 kw0 = *(const u32x4 *)(ct + row * cs + 2 * d0), kw1 = *(const u32x4 *)(ct + row * cs + 2 * d1);
            float4 c4[4] = {};
            if (half_rot && k < 4) {
                const float4 *c = (const float4 *)(table + 32 * rr + 8 * k);
#pragma unroll
                for (int q = 0; q < 4; q++) c4[q] = c[q];
            }
            k_row_out(p, kw0, kw1, wn, c4, k, t, kh);
        }
        if (half_rot && !TABLED) __syncthreads();   // the table is read before the next pass rewrites it
    }
}

// V^T entries of rows m0 .. m0 + BM - 1 of kv head kh: lane = pass row, so each store of one
// dim covers 64 consecutive plane rows of a record (2 bytes a lane, one 128-byte line); only the
// pass's own plane rows are written. The NWAVES waves split the tile into (row block of 64,
// dim range) tasks. Values with |v| > f16_lim or NaN saturate to +-65536 (bf16's rounding of
// 65504) and flag the record.
template <int NWAVES, int BM>
__device__ __forceinline__ void v_rows(const KvRows &p, const uint8_t *ct, int cs, int m0, int kh) {
    constexpr int HD = 256, RB = BM / 64;
    constexpr int TASKS = NWAVES > RB ? NWAVES : RB, DPT = HD * RB / TASKS;   // dims per task
    static_assert(DPT % 2 == 0 && HD * RB % TASKS == 0, "tasks split the dims evenly");
    const int tid = threadIdx.x, lane = tid & 63;
    for (int task = tid >> 6; task < TASKS; task += NWAVES) {
        const int row = 64 * (task % RB) + lane, t = m0 + row, d0 = DPT * (task / RB);
        if (t >= p.T) continue;
        uint16_t *col = p.vt_plane + ((size_t)kh * HD + d0) * p.kvT + (size_t)p.tok_kv[t];
        bool bad = false;
#pragma unroll 8
        for (int d = 0; d < DPT; d += 2) {
            unsigned w = *(const unsigned *)(ct + row * cs + 2 * (d0 + d));
            bad |= v_word(w, p.f16_lim);
            col[(size_t)d * p.kvT] = (uint16_t)w;
            col[(size_t)(d + 1) * p.kvT] = (uint16_t)(w >> 16);
        }
        if (bad && p.ovf && p.seq_start) __hip_atomic_store(p.ovf + p.seq_start[t], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// The K/V prologue as its own kernel with no LDS tile and no barrier: every wave works alone,
// so the loads of some waves overlap the stores of others, as in a copy kernel.
//  - K waves (the first n_kwaves): 4 pass rows, 16 lanes each, every kv head. A lane's loads for
//    all its kv heads go out first; meanwhile it computes the rotary cos/sin of pairs 2k and
//    2k + 1 of its row (k_table's arithmetic; rope_cs gets them once per row), and the lanes
//    k < 4 fetch the four pairs-of-pairs they turn from lanes 4k .. 4k + 3 with ds_bpermute.
//    Then k_row_out per kv head.
//  - V waves: 64 pass rows (lane = row) x 16 dims of one kv head: two 16-byte loads, then 16
//    two-byte stores, each one 128-byte V^T line, through split16's check.
// Planes, flags and rope_cs are bitwise those of the QKV GEMM's epilogue (the same k_row_out,
// rope_sincos and v_word).
constexpr int kPrepDirectThreads = 256, kPrepDirectKvChunk = 4;
__device__ __forceinline__ int prep_direct_kwaves(int T) { return (T + 3) / 4; }
__device__ __forceinline__ float bperm(int src_lane, float v) {
    return __int_as_float(__builtin_amdgcn_ds_bpermute(4 * src_lane, __float_as_int(v)));
}
__global__ __launch_bounds__(kPrepDirectThreads) void text_prep_direct_kernel(const uint16_t *qkv, int row_len, KvRows p) {
    constexpr int HD = 256, KC = kPrepDirectKvChunk;
    const int lane = threadIdx.x & 63;
    const int gw = (int)blockIdx.x * (kPrepDirectThreads / 64) + (int)(threadIdx.x >> 6);
    const int n_kwaves = prep_direct_kwaves(p.T);
    if (gw < n_kwaves) {
        const int rr = lane >> 4, k = lane & 15, t = gw * 4 + rr;
        const bool valid = t < p.T;
        const int tt = valid ? t : p.T - 1;   // rows past the pass load the last row, then stop
        const int d0 = k_lane_dim(k, 0), d1 = k_lane_dim(k, 1);
        const uint16_t *src = qkv + (size_t)tt * row_len + (size_t)p.nh * 2 * HD;
        u32x4 kw[KC][2];
#pragma unroll
        for (int j = 0; j < KC; j++) {
            const int kh = min(j, p.nkv - 1);
            kw[j][0] = *(const u32x4 *)(src + (size_t)kh * HD + d0);
            kw[j][1] = *(const u32x4 *)(src + (size_t)kh * HD + d1);
        }
        float wn[16];
        if (p.k_norm) k_lane_weights(p, k, wn);
        float4 c4[4] = {};
        if (p.n_rot) {
            float cs[4];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int i = 2 * k + h;
                const float ang = (float)p.pos3[3 * (size_t)tt + i % 3] * p.inv_freq[i];
                rope_sincos(ang, &cs[2 * h + 1], &cs[2 * h]);
            }
            if (valid && p.rope_cs) *(float4 *)(p.rope_cs + (size_t)t * 64 + 4 * k) = make_float4(cs[0], cs[1], cs[2], cs[3]);
            const int base = 16 * rr + 4 * (k & 3);
#pragma unroll
            for (int q = 0; q < 4; q++)
                c4[q] = make_float4(bperm(base + q, cs[0]), bperm(base + q, cs[1]), bperm(base + q, cs[2]), bperm(base + q, cs[3]));
        }
        if (!valid) return;
        for (int kh0 = 0; kh0 < p.nkv; kh0 += KC) {
            if (kh0 > 0) {
#pragma unroll
                for (int j = 0; j < KC; j++) {
                    const int kh = min(kh0 + j, p.nkv - 1);
                    kw[j][0] = *(const u32x4 *)(src + (size_t)kh * HD + d0);
                    kw[j][1] = *(const u32x4 *)(src + (size_t)kh * HD + d1);
                }
            }
#pragma unroll
            for (int j = 0; j < KC; j++)
                if (kh0 + j < p.nkv) k_row_out(p, kw[j][0], kw[j][1], wn, c4, k, t, kh0 + j);
        }
        return;
    }
    // V: task (kv head, 64-row block, 16-dim group)
    const int gv = gw - n_kwaves, n_rb = (p.T + 63) / 64;
    if (gv >= p.nkv * n_rb * 16) return;
    const int dg = gv & 15, rb = (gv >> 4) % n_rb, kh = (gv >> 4) / n_rb;
    const int t = rb * 64 + lane;
    if (t >= p.T) return;
    const uint16_t *src = qkv + (size_t)t * row_len + (size_t)p.nh * 2 * HD + (size_t)p.nkv * HD + (size_t)kh * HD + 16 * dg;
    const u32x4 v0 = *(const u32x4 *)src, v1 = *(const u32x4 *)(src + 8);
    uint16_t *col = p.vt_plane + ((size_t)kh * HD + 16 * dg) * p.kvT + (size_t)p.tok_kv[t];
    bool bad = false;
#pragma unroll
    for (int d = 0; d < 16; d += 2) {
        unsigned w = d < 8 ? v0[d / 2] : v1[(d - 8) / 2];
        bad |= v_word(w, p.f16_lim);
        col[(size_t)d * p.kvT] = (uint16_t)w;
        col[(size_t)(d + 1) * p.kvT] = (uint16_t)(w >> 16);
    }
    if (bad && p.ovf && p.seq_start) __hip_atomic_store(p.ovf + p.seq_start[t], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace clef_hip
