// The text path's K/V prologue on a tile of pass rows held in LDS (bf16, row stride cs bytes):
// K rows are RMS-normalised, rotated (partial NeoX rotary, interleaved M-RoPE angles) and split
// to the f16 K plane; V rows go to the V^T plane. Semantics: metal/clef.metal:245-300 (attn_prep
// K and V) and 857-928 (split16 and attn_prep_split: the f16 planes, |x| > f16_lim or NaN
// saturating and flagging the record).
//
// Two producers fill the tile: text_prep_rows_kernel (attn_kernels.h) loads it from the qkv
// rows, and the QKV GEMM (gemm_kernel.h) leaves its bf16 output tile there; both then call these
// functions, so the planes they write are bitwise the same.
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
template <int NTHREADS, int BM, bool TABLED = false>
__device__ __forceinline__ void k_rows(const KvRows &p, const uint8_t *ct, int cs, int m0, int kh, float2 *table) {
    static_assert(!TABLED || NTHREADS / 16 == BM, "a caller-filled table covers one pass");
    constexpr int HD = 256, RPP = NTHREADS / 16;
    const int tid = threadIdx.x, rr = tid >> 4, k = tid & 15;
    const int half_rot = p.n_rot / 2;   // 0 or 32: dims [0, 32) pair with [32, 64)
    const int d0 = k_lane_dim(k, 0), d1 = k_lane_dim(k, 1);
    float wn[16];
    if (p.k_norm) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 w4 = *(const float4 *)(p.k_norm + ((q < 2) ? d0 : d1) + 4 * (q & 1));
            wn[4 * q] = w4.x; wn[4 * q + 1] = w4.y; wn[4 * q + 2] = w4.z; wn[4 * q + 3] = w4.w;
        }
    }
    for (int pass = 0; pass < BM / RPP; pass++) {
        const int row = RPP * pass + rr, t = m0 + row;
        const bool valid = t < p.T;
        if (half_rot && !TABLED) {
            k_table(p, m0 + RPP * pass, rr, k, kh, table);
            __syncthreads();
        }
        if (valid) {
            const u32x4 kw0 = *(const u32x4 *)(ct + row * cs + 2 * d0), kw1 = *(const u32x4 *)(ct + row * cs + 2 * d1);
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
            if (half_rot && k < 4) {   // pair 8k + e: x[e] turns with x[e + 8]
                const float4 *c = (const float4 *)(table + 32 * rr + 8 * k);
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float4 cs2 = c[q];   // (cos, sin) of pairs 8k + 2q, 8k + 2q + 1
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        const int e = 2 * q + h;
                        const float cn = h ? cs2.z : cs2.x, sn = h ? cs2.w : cs2.y;
                        const float x0 = x[e], x1 = x[e + 8];
                        x[e] = x0 * cn - x1 * sn;
                        x[e + 8] = x1 * cn + x0 * sn;
                    }
                }
            }
            // split16's saturation: the largest magnitude decides (NaN propagates through the
            // maximum, and fails the compare); only a row holding one takes the elementwise pass
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
            const bool lo_bad = !(__uint_as_float((w & 0x7fffu) << 16) <= p.f16_lim),
                       hi_bad = !(__uint_as_float(w & 0x7fff0000u) <= p.f16_lim);
            if (lo_bad) w = (w & 0xffff8000u) | 0x4780u;
            if (hi_bad) w = (w & 0x8000ffffu) | 0x47800000u;
            bad |= lo_bad | hi_bad;
            col[(size_t)d * p.kvT] = (uint16_t)w;
            col[(size_t)(d + 1) * p.kvT] = (uint16_t)(w >> 16);
        }
        if (bad && p.ovf && p.seq_start) __hip_atomic_store(p.ovf + p.seq_start[t], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// The K/V prologue as its own kernel, over pass rows: workgroup (b, j) loads rows 64b .. 64b + 63
// of K head j (j < nkv) or V head j - nkv into LDS and runs k_rows / v_rows on them. All loads
// are issued at once (no load depends on another), a K workgroup fills its rotary table while
// they land, and the plane rows come from tok_kv.
constexpr int kPrepRowsBM = 64, kPrepRowsThreads = 1024, kPrepRowsCS = 512 + 16;
__global__ __launch_bounds__(kPrepRowsThreads) void text_prep_rows_kernel(const uint16_t *qkv, int row_len, KvRows p) {
    constexpr int BM = kPrepRowsBM, NT = kPrepRowsThreads, CSB = kPrepRowsCS;
    __shared__ __attribute__((aligned(16))) uint8_t tile[BM * CSB];
    __shared__ __attribute__((aligned(16))) float2 table[NT / 16 * 32];
    const int tid = threadIdx.x, m0 = blockIdx.x * BM, j = blockIdx.y;
    const bool is_k = j < p.nkv;
    const int head = is_k ? j : j - p.nkv;
    const uint16_t *src = qkv + (size_t)p.nh * 2 * 256 + (size_t)(is_k ? 0 : p.nkv * 256) + (size_t)head * 256;
    constexpr int PER = BM * 32 / NT;
    u32x4 w[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int id = tid + NT * i, r = id >> 5, c16 = id & 31;
        const int t = min(m0 + r, p.T - 1);
        w[i] = *(const u32x4 *)(src + (size_t)t * row_len + 8 * c16);
    }
    if (is_k && p.n_rot) k_table(p, m0, tid >> 4, tid & 15, head, table);
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int id = tid + NT * i, r = id >> 5, c16 = id & 31;
        *(u32x4 *)(tile + r * CSB + 16 * c16) = w[i];
    }
    __syncthreads();
    if (is_k) k_rows<NT, BM, true>(p, tile, CSB, m0, head, table);
    else v_rows<NT / 64, BM>(p, tile, CSB, m0, head);
}

}  // namespace clef_hip
