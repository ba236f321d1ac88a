// Shared pieces of the prefill attention path for CDNA4 (gfx950): bf16 helpers, the rotary
// sin/cos, the output conversion (act16), and the two prologue kernels that write the K / V^T
// planes the attention kernels stream (text: attn_text.h, vision: attn_vis.h).
//
// Semantics follow cleffa's attention family (metal/clef.metal:245-300 attn_prep,
// metal/clef.metal:930-1093 attention_tu, metal/clef.metal:657-849 prefix variant,
// metal/clef.metal:1616-1964 vision), restated for 64-wide wavefronts and bf16 MFMA.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_params.h"

namespace clef_hip {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;
typedef __attribute__((ext_vector_type(4))) unsigned u32x4;
typedef __attribute__((ext_vector_type(2))) unsigned u32x2;

__device__ __forceinline__ float bf_lo(unsigned w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(unsigned w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float((unsigned)b << 16); }

// Round-to-nearest-even pair conversion (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ unsigned pack_bf16(float a, float b) {
    bf16x2 v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(unsigned, v);
}
// Round-to-nearest-even pair conversion to f16 (the text path's Q and K operands).
__device__ __forceinline__ unsigned pack_f16(float a, float b) {
    f16x2 v = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(unsigned, v);
}
__device__ __forceinline__ uint16_t f2bf(float a) {
    __bf16 v = (__bf16)a;
    return __builtin_bit_cast(uint16_t, v);
}

// sigmoid(x) = 1 / (1 + 2^(-x log2 e)) with the hardware exp2 and reciprocal (~1 ulp each).
__device__ __forceinline__ float sigmoidf(float x) {
    return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-x * 1.4426950408889634f));
}

// sin and cos of a rotary angle (|x| < 2^20), without the memory tables of a general-range
// routine. Cody-Waite reduction by pi/2 in three parts with fma (the parts come from the double
// pi/2 split into floats), then Taylor polynomials on |r| <= pi/4: sin to r^9 (truncation
// < 2e-9), cos to r^10 (< 1e-10); about 1-2 ulp overall for the float angle the caller formed.
__device__ __forceinline__ void rope_sincos(float x, float *s, float *c) {
    constexpr double kHalfPi = 1.5707963267948966;
    constexpr float C1 = (float)kHalfPi;
    constexpr float C2 = (float)(kHalfPi - (double)C1);
    constexpr float C3 = (float)(kHalfPi - (double)C1 - (double)C2);
    const float j = __builtin_rintf(x * 0.63661977236758134f);
    float r = fmaf(-j, C1, x);
    r = fmaf(-j, C2, r);
    r = fmaf(-j, C3, r);
    const float r2 = r * r;
    float ps = fmaf(r2, 1.f / 362880.f, -1.f / 5040.f);
    ps = fmaf(ps, r2, 1.f / 120.f);
    ps = fmaf(ps, r2, -1.f / 6.f);
    const float sr = fmaf(ps * r2, r, r);
    float pc = fmaf(r2, -1.f / 3628800.f, 1.f / 40320.f);
    pc = fmaf(pc, r2, -1.f / 720.f);
    pc = fmaf(pc, r2, 1.f / 24.f);
    pc = fmaf(pc, r2, -0.5f);
    const float cr = fmaf(pc, r2, 1.f);
    const int q = (int)j & 3;   // x = j pi/2 + r
    const float sv = (q & 1) ? cr : sr, cv = (q & 1) ? sr : cr;
    *s = (q & 2) ? -sv : sv;
    *c = ((q + 1) & 2) ? -cv : cv;
}

// Output conversion of the o_proj operand (metal/clef.metal:98-106, act16): bf16, or f16
// that saturates to +-65504 and flags the record when |v| > lim or v is NaN, or plain f32.
__device__ __forceinline__ void store_out8(void *out, size_t idx, const float *v, int out_type,
                                           float lim, int32_t *flag) {
    if (out_type == CLEF_HIP_OUT_BF16) {
        u32x4 w = {pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]), pack_bf16(v[4], v[5]),
                   pack_bf16(v[6], v[7])};
        *(u32x4 *)((uint16_t *)out + idx) = w;
    } else if (out_type == CLEF_HIP_OUT_F16) {
        _Float16 h[8];
        bool bad = false;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            float x = v[j];
            if (!(fabsf(x) <= lim)) {
                bad = true;
                x = copysignf(65504.0f, x);
            }
            h[j] = (_Float16)x;
        }
        if (bad && flag) __hip_atomic_store(flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *(u32x4 *)((uint16_t *)out + idx) = __builtin_bit_cast(u32x4, h);
    } else {
        float *o = (float *)out + idx;
        *(float4 *)o = make_float4(v[0], v[1], v[2], v[3]);
        *(float4 *)(o + 4) = make_float4(v[4], v[5], v[6], v[7]);
    }
}

// act16 of four consecutive output elements of one row (metal/clef.metal:98-106), as store_out8:
// bf16, f16 saturating at +-65504 with the record flag when |v| > lim or NaN, or f32.
typedef float f32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void store_out4(void *out, size_t idx, f32x4_t v, int out_type, float lim, int32_t *flag) {
    if (out_type == CLEF_HIP_OUT_F32) {
        *(f32x4_t *)((float *)out + idx) = v;
        return;
    }
    uint16_t h[4];
    if (out_type == CLEF_HIP_OUT_BF16) {
#pragma unroll
        for (int e = 0; e < 4; e++) h[e] = __builtin_bit_cast(uint16_t, (__bf16)v[e]);
    } else {
        bool bad = false;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float x = v[e];
            if (!(fabsf(x) <= lim)) {
                bad = true;
                x = copysignf(65504.0f, x);
            }
            h[e] = __builtin_bit_cast(uint16_t, (_Float16)x);
        }
        if (bad && flag) __hip_atomic_store(flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    *(uint2 *)((uint16_t *)out + idx) = make_uint2(h[0] | ((unsigned)h[1] << 16), h[2] | ((unsigned)h[3] << 16));
}

typedef __attribute__((address_space(3))) void lds_void;

// ------------------------------------------------------------------------------------------
// Text K/V prologue (metal/clef.metal:245-300 and 873-928 for K and V): K = RMSNorm(k) * (1+w)
// then partial rotary into the f16 K plane [nkv][kvT][HD]; V unnormalised into the V^T plane
// [nkv][HD][kvT]; the rotary cos/sin of each pass row into rope_cs for the Q prologue.
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ float row16_sum(float v) {   // sum over the lane's 16-lane row
    v += __builtin_amdgcn_update_dpp(0.f, v, 0x128, 0xf, 0xf, false);   // row_ror:8
    v += __builtin_amdgcn_update_dpp(0.f, v, 0x124, 0xf, 0xf, false);   // row_ror:4
    v += __builtin_amdgcn_update_dpp(0.f, v, 0x4e, 0xf, 0xf, false);    // quad_perm [2,3,0,1]
    v += __builtin_amdgcn_update_dpp(0.f, v, 0xb1, 0xf, 0xf, false);    // quad_perm [1,0,3,2]
    return v;
}

// K/V prologue over plane rows: workgroup (b, kh) owns plane rows 16b .. 16b+15 of kv head kh
// and takes each row's key from pass row kv_tok[row] (-1: the row is left as it is). 16 lanes
// per row, 16 dims per lane. K rows are normalised, rotated and stored whole (512 B per row).
// V rows are staged row-major in LDS and read back transposed with ds_read_b64_tr_b16 (lane i
// of a 16-lane group receives element i % 4 of the 8 bytes lane 4j + i / 4 addressed, for
// j = 0..3), which hands each lane one head dim of 4 consecutive rows; two such reads make a
// 16-byte V^T run of 8 plane rows. A run with rows the pass does not own (a prefix record's
// cached rows, rows past a record) is merged with the plane's contents.
constexpr int kPrepRows = 16;
typedef short short4_t __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(16 * kPrepRows) void text_prep_kv_kernel(PrepParams p) {
    constexpr int HD = 256, ROWS = kPrepRows, NT = 16 * ROWS;
    constexpr int VS = HD + 64;   // LDS row stride: 4 rows' 128-byte reads fall in distinct banks
    __shared__ __attribute__((aligned(16))) uint16_t vl[ROWS * VS];
    __shared__ __attribute__((aligned(16))) float2 csl[ROWS][32];
    __shared__ int trow[ROWS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int rr = tid >> 4, k = tid & 15;       // row of the tile, 16-dim group of the row
    const int r0 = blockIdx.x * ROWS, kh = blockIdx.y;
    const int half_rot = p.n_rot / 2;            // 0 or 32: dims [0, 32) pair with [32, 64)
    const int t = (r0 + rr < p.kv_rows) ? p.kv_tok[r0 + rr] : -1;
    if (k == 0) trow[rr] = t;
    if (!__syncthreads_or(t >= 0)) return;       // no row of this tile belongs to the pass
    // Global loads first, all in flight together: the row's K and V chunks, the positions and
    // frequencies of this thread's rotary-table entries, the k_norm weights. The loads are
    // unconditional (a row the pass does not own reads pass row 0) and the values selected after:
    // a load under a condition becomes a branch, and the compiler waits for it at the join.
    const uint16_t *src = p.qkv + (size_t)(t >= 0 ? t : 0) * p.row + (size_t)p.nh * 2 * HD + (size_t)kh * HD + 16 * k;
    u32x4 kw[2], vw[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        kw[h] = *(const u32x4 *)(src + 8 * h);
        vw[h] = *(const u32x4 *)(src + (size_t)p.nkv * HD + 8 * h);
    }
    // rotary table of the tile: ROWS x 32 pairs, pair i turns by axis i % 3; entry idx = tid + NT j
    constexpr int TJ = ROWS * 32 / NT;
    int rtt[TJ], rpos[TJ];
    float rfreq[TJ];
    if (half_rot) {
#pragma unroll
        for (int j = 0; j < TJ; j++) {
            const int idx = tid + NT * j, row = idx >> 5, i = idx & 31;
            rtt[j] = trow[row];
            rpos[j] = p.pos3[3 * (size_t)(rtt[j] >= 0 ? rtt[j] : 0) + i % 3];
            rfreq[j] = p.inv_freq[i];
        }
    }
    float wn[16];
    if (p.k_norm) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 w4 = *(const float4 *)(p.k_norm + 16 * k + 4 * q);
            wn[4 * q] = w4.x; wn[4 * q + 1] = w4.y; wn[4 * q + 2] = w4.z; wn[4 * q + 3] = w4.w;
        }
    }
    // A V element with |v| > f16_lim, or NaN, saturates to +-65536 (bf16's rounding of 65504)
    // and flags the record, as split16 does for the reference's f16 V plane
    // (metal/clef.metal:857-867): the same records are flagged for the FP32 rerun, and nothing
    // past a record's own keys can read inf or NaN.
    bool bad = false;
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            kw[h][j] = t >= 0 ? kw[h][j] : 0u;
            unsigned w = t >= 0 ? vw[h][j] : 0u;
            const bool lo_bad = !(__uint_as_float((w & 0x7fffu) << 16) <= p.f16_lim),
                       hi_bad = !(__uint_as_float(w & 0x7fff0000u) <= p.f16_lim);
            if (lo_bad) w = (w & 0xffff8000u) | 0x4780u;
            if (hi_bad) w = (w & 0x8000ffffu) | 0x47800000u;
            bad |= lo_bad | hi_bad;
            vw[h][j] = w;
        }
    if (half_rot) {
#pragma unroll
        for (int j = 0; j < TJ; j++) {
            const int idx = tid + NT * j, row = idx >> 5, i = idx & 31;
            if (rtt[j] >= 0) {
                const float ang = (float)rpos[j] * rfreq[j];
                float sn, cn;
                rope_sincos(ang, &sn, &cn);
                csl[row][i] = make_float2(cn, sn);
                if (p.rope_cs && kh == 0) *(float2 *)(p.rope_cs + (size_t)rtt[j] * 2 * half_rot + 2 * i) = make_float2(cn, sn);
            }
        }
    }
    // V rows into LDS, row-major
    *(u32x4 *)(vl + rr * VS + 16 * k) = vw[0];
    *(u32x4 *)(vl + rr * VS + 16 * k + 8) = vw[1];
    __syncthreads();
    float x[16];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        x[2 * j] = bf_lo(kw[0][j]);
        x[2 * j + 1] = bf_hi(kw[0][j]);
        x[8 + 2 * j] = bf_lo(kw[1][j]);
        x[8 + 2 * j + 1] = bf_hi(kw[1][j]);
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
    if (half_rot) {
        // lanes 0, 1 hold dims 0-31, lanes 2, 3 their partners 32-63 (two lanes apart)
        float y[16];
#pragma unroll
        for (int e = 0; e < 16; e++) {
            // row_ror:n hands lane i the value of lane (i - n) mod 16
            const float up = __builtin_amdgcn_update_dpp(0.f, x[e], 0x12e, 0xf, 0xf, false);   // lane + 2
            const float dn = __builtin_amdgcn_update_dpp(0.f, x[e], 0x122, 0xf, 0xf, false);   // lane - 2
            y[e] = (k & 2) ? dn : up;
        }
        if (k < 4) {
            const bool first = k < 2;
            const float2 *cs = csl[rr] + 16 * (k & 1);
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const float2 v = cs[e];
                x[e] = first ? x[e] * v.x - y[e] * v.y : x[e] * v.x + y[e] * v.y;
            }
        }
    }
    // The f16 K plane follows split16: |k| > f16_lim or NaN saturates to +-65504 and flags the
    // record (at its first pass row, seq_start).
    {
        const unsigned lim = __float_as_uint(p.f16_lim);
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const bool over = (__float_as_uint(x[e]) & 0x7fffffffu) > lim;
            x[e] = over ? copysignf(65504.f, x[e]) : x[e];
            bad |= over;
        }
    }
    if (bad && t >= 0 && p.ovf && p.seq_start)
        __hip_atomic_store(p.ovf + p.seq_start[t], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (t >= 0) {
        uint16_t *dst = p.k_plane + ((size_t)kh * p.kvT + r0 + rr) * HD + 16 * k;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const float *xs = x + 8 * h;
            u32x4 ko = {pack_f16(xs[0], xs[1]), pack_f16(xs[2], xs[3]), pack_f16(xs[4], xs[5]), pack_f16(xs[6], xs[7])};
            *(u32x4 *)(dst + 8 * h) = ko;
        }
    }
    // V^T: wave w covers dims 64(w%4) .. +63 of rows 16(w/4) .. +15. In read q (rows
    // 16(w/4) + 4q .. +3), lane s of 16-lane group g addresses row 16(w/4) + 4q + s/4, dims
    // 64(w%4) + 16g + 4(s%4) .. +3, and receives dim 64(w%4) + 16g + s of the 4 rows.
    const int g = lane >> 4, s16 = lane & 15, db = wave & 3, rg = wave >> 2;
    const int d = 64 * db + 16 * g + s16;
    const unsigned base = (unsigned)(uintptr_t)(const __attribute__((address_space(3))) uint16_t *)vl;
    short4_t rd[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const unsigned a = base + 2u * (unsigned)((16 * rg + 4 * q + (s16 >> 2)) * VS + 64 * db + 16 * g + 4 * (s16 & 3));
        rd[q] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4_t *)(uintptr_t)a);
    }
#pragma unroll
    for (int run = 0; run < 2; run++) {
        const int rb = 16 * rg + 8 * run;
        unsigned own = 0;
#pragma unroll
        for (int e = 0; e < 8; e++) own |= (trow[rb + e] >= 0 ? 1u : 0u) << e;
        if (!own) continue;
        const short4_t lo = rd[2 * run], hi = rd[2 * run + 1];
        u32x4 w = {(unsigned)(uint16_t)lo[0] | ((unsigned)(uint16_t)lo[1] << 16), (unsigned)(uint16_t)lo[2] | ((unsigned)(uint16_t)lo[3] << 16),
                   (unsigned)(uint16_t)hi[0] | ((unsigned)(uint16_t)hi[1] << 16), (unsigned)(uint16_t)hi[2] | ((unsigned)(uint16_t)hi[3] << 16)};
        uint16_t *dst = p.vt_plane + ((size_t)kh * HD + d) * p.kvT + r0 + rb;
        if (own != 0xffu) {   // keep the rows this pass does not own
            const u32x4 old = *(const u32x4 *)dst;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const unsigned m = ((own >> (2 * j)) & 1u ? 0xffffu : 0u) | ((own >> (2 * j + 1)) & 1u ? 0xffff0000u : 0u);
                w[j] = (w[j] & m) | (old[j] & ~m);
            }
        }
        *(u32x4 *)dst = w;
    }
}

// ------------------------------------------------------------------------------------------
// Vision prologue (metal/clef.metal:1616-1656, vis_qkv_rope) over plane rows: workgroup
// (b, h) owns kv rows 16b .. 16b+15 of head h and takes each row's patch from kv_tok (-1: the
// row is left as it is). qkv [P][3E] (+ bias): Q and K take the 2-D rotary, pair (i, i + 36),
// the first 18 pairs turning by the patch's grid row and the rest by its column (pos2 [P][2]);
// Q goes to its patch's row of the Q plane [heads][P][72], K to the kv row of the K plane
// [heads][kvT][72], V (biased) to the V^T plane [heads][72][kvT] in 16-byte runs of 8 rows.
// 256 threads: 16 lanes per row for the loads and stores, one lane per (row, pair) for the
// rotary, the rows staged in LDS.
// ------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void vis_prep_kernel(VisPrepParams p) {
    constexpr int HD = 72, ROWS = 16, HALF = HD / 2, QUART = HD / 4, CH = HD / 8;   // 9 chunks
    constexpr int VS = ROWS + 8;   // LDS stride of a V^T row
    __shared__ __attribute__((aligned(16))) float xs[ROWS][3][HD];   // biased q, k, v
    __shared__ __attribute__((aligned(16))) uint16_t qo[ROWS][HD], ko[ROWS][HD];
    __shared__ __attribute__((aligned(16))) uint16_t vt[HD * VS];
    __shared__ int trow[ROWS];
    __shared__ float ang_pos[ROWS][2];
    const int tid = threadIdx.x, rr = tid >> 4, k = tid & 15;
    // Work unit u = h * n_tiles + tile. Workgroup L runs on XCD L % 8 (round-robin dispatch);
    // the four consecutive tiles whose 32-byte V^T runs share a 128-byte line go to four
    // consecutive workgroups of one XCD, so the partial lines merge in that XCD's L2.
    const int n_tiles = (p.kv_rows + ROWS - 1) / ROWS;
    const int L = blockIdx.x, j = L >> 3;
    const int u = 4 * (((j >> 2) << 3) + (L & 7)) + (j & 3);
    if (u >= n_tiles * p.heads) return;
    const int h = u / n_tiles, r0 = (u - h * n_tiles) * ROWS;
    const int E = p.heads * HD;
    // loads that do not depend on the row's patch go first: the lane's bias chunks and the
    // rotary frequencies of the pairs it turns
    float bv[2][8];
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int id = k + 16 * r;
        if (id < 3 * CH && p.bias) {
            const int part = id / CH, ch = id % CH;
            const float *bb = p.bias + (size_t)part * E + (size_t)h * HD + ch * 8;
            const float4 b0 = *(const float4 *)bb, b1 = *(const float4 *)(bb + 4);
            bv[r][0] = b0.x; bv[r][1] = b0.y; bv[r][2] = b0.z; bv[r][3] = b0.w;
            bv[r][4] = b1.x; bv[r][5] = b1.y; bv[r][6] = b1.z; bv[r][7] = b1.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) bv[r][j] = 0.f;
        }
    }
    float fr[3];
#pragma unroll
    for (int r = 0; r < 3; r++) {
        const int i = (tid + 256 * r) % HALF;
        fr[r] = p.inv_freq[i < QUART ? i : i - QUART];
    }
    const int t = (r0 + rr < p.kv_rows) ? p.kv_tok[r0 + rr] : -1;
    if (k == 0) trow[rr] = t;
    if (!__syncthreads_or(t >= 0)) return;
    // the row's 27 chunks (q, k, v) over 16 lanes, bias added in float; its grid position
    if (t >= 0) {
        const uint16_t *row = p.qkv + (size_t)t * 3 * E + (size_t)h * HD;
        u32x4 w[2];
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int id = k + 16 * r;
            if (id < 3 * CH) w[r] = *(const u32x4 *)(row + (size_t)(id / CH) * E + (id % CH) * 8);
        }
        if (k < 2) ang_pos[rr][k] = (float)p.pos2[2 * (size_t)t + k];
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int id = k + 16 * r;
            if (id < 3 * CH) {
                const int part = id / CH, ch = id % CH;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    xs[rr][part][ch * 8 + 2 * j] = bf_lo(w[r][j]) + bv[r][2 * j];
                    xs[rr][part][ch * 8 + 2 * j + 1] = bf_hi(w[r][j]) + bv[r][2 * j + 1];
                }
            }
        }
    }
    __syncthreads();
    // rotary: one lane per (row, pair); V goes to the transposed LDS tile
#pragma unroll
    for (int r = 0; r < 3; r++) {
        const int id = tid + 256 * r;
        if (id >= ROWS * HALF) break;
        const int row = id / HALF, i = id % HALF;
        if (trow[row] < 0) continue;
        float sn, cs;
        rope_sincos(ang_pos[row][i < QUART ? 0 : 1] * fr[r], &sn, &cs);
        const float q0 = xs[row][0][i], q1 = xs[row][0][i + HALF];
        const float k0 = xs[row][1][i], k1 = xs[row][1][i + HALF];
        qo[row][i] = f2bf(q0 * cs - q1 * sn);
        qo[row][i + HALF] = f2bf(q1 * cs + q0 * sn);
        ko[row][i] = f2bf(k0 * cs - k1 * sn);
        ko[row][i + HALF] = f2bf(k1 * cs + k0 * sn);
    }
    for (int id = tid; id < ROWS * HD; id += 256) {
        const int row = id / HD, d = id % HD;
        vt[d * VS + row] = f2bf(xs[row][2][d]);
    }
    __syncthreads();
    // Q and K rows: 9 chunks each
    if (t >= 0 && k < CH) {
        *(u32x4 *)(p.q_plane + ((size_t)h * p.P + t) * HD + k * 8) = *(const u32x4 *)(&qo[rr][k * 8]);
        *(u32x4 *)(p.k_plane + ((size_t)h * p.kvT + r0 + rr) * HD + k * 8) = *(const u32x4 *)(&ko[rr][k * 8]);
    }
    // V^T runs: dim d, rows 8q .. 8q+7
    for (int id = tid; id < HD * (ROWS / 8); id += 256) {
        const int d = id / (ROWS / 8), q = id % (ROWS / 8);
        unsigned own = 0;
#pragma unroll
        for (int e = 0; e < 8; e++) own |= (trow[8 * q + e] >= 0 ? 1u : 0u) << e;
        if (!own) continue;
        uint16_t *dst = p.vt_plane + ((size_t)h * HD + d) * p.kvT + r0 + 8 * q;
        u32x4 w = *(const u32x4 *)(vt + d * VS + 8 * q);
        if (own != 0xffu) {   // keep the rows this pass does not own
            const u32x4 old = *(const u32x4 *)dst;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const unsigned m = ((own >> (2 * j)) & 1u ? 0xffffu : 0u) | ((own >> (2 * j + 1)) & 1u ? 0xffff0000u : 0u);
                w[j] = (w[j] & m) | (old[j] & ~m);
            }
        }
        *(u32x4 *)dst = w;
    }
}

}  // namespace clef_hip
