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
// Text K/V prologue helpers (the kernel and its epilogue form live in kv_rows.h).
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ float row16_sum(float v) {   // sum over the lane's 16-lane row
    v += __builtin_amdgcn_update_dpp(0.f, v, 0x128, 0xf, 0xf, false);   // row_ror:8
    v += __builtin_amdgcn_update_dpp(0.f, v, 0x124, 0xf, 0xf, false);   // row_ror:4
    v += __builtin_amdgcn_update_dpp(0.f, v, 0x4e, 0xf, 0xf, false);    // quad_perm [2,3,0,1]
    v += __builtin_amdgcn_update_dpp(0.f, v, 0xb1, 0xf, 0xf, false);    // quad_perm [1,0,3,2]
    return v;
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
// The vision prologue over pass rows (the form used when the caller passes tok_kv): workgroup
// (b, g) takes patches 64b .. 64b + 63: for g < G (the groups of 8 heads) the q and k of heads
// 8g .. 8g + 7, for g >= G the v of head g - G (workgroups of their own, so the two run side by
// side). Everything goes through registers, with no LDS tile and no plane-row lookup ahead of the
// loads. The rows' rotary cos/sin go to an LDS table while the q/k loads land (the angles do not
// depend on the head: eight heads share it).
//  - q and k: thread (dims 4j .. 4j + 3, head) holds both halves of four rotary pairs (dims
//    4j + e and 4j + 36 + e) for 8 rows, loaded as 8-byte pieces, biased and turned in
//    registers, stored to the Q plane (row = patch) and the K plane (row = tok_kv);
//  - v (workgroups of one head, one wave per 16-byte chunk of 8 dims): lane = row, biased, then
//    stored dim by dim: each store covers 64 consecutive plane rows of an image, one 128-byte
//    V^T line.
// Same arithmetic as vis_prep_kernel (metal/clef.metal:1616-1656: bias in f32, pair (i, i + 36)
// turned by the grid row's angle for i < 18 and the column's otherwise, each result rounded once
// to bf16).
constexpr int kVisRowsBM = 64, kVisRowsHeads = 8, kVisRowsThreads = 576;
__global__ __launch_bounds__(kVisRowsThreads) void vis_prep_rows_kernel(VisPrepParams p) {
    constexpr int HD = 72, HALF = HD / 2, QUART = HD / 4, CH = HD / 8, BM = kVisRowsBM, HG = kVisRowsHeads;
    constexpr int NT = kVisRowsThreads, RPT = 8;   // q/k: (HALF / 4) x HG x (BM / RPT) threads, RPT rows each
    static_assert((HALF / 4) * HG * (BM / RPT) == NT, "q/k threads");
    __shared__ float2 table[BM * HALF];   // [row][pair] (cos, sin)
    const int tid = threadIdx.x, m0 = blockIdx.x * BM;
    const int n_groups = (p.heads + HG - 1) / HG;
    const bool is_v = (int)blockIdx.y >= n_groups;
    const int E = p.heads * HD;
    if (is_v) {
        // v: head blockIdx.y - G, wave c takes dims 8c .. 8c + 7 of the 64 rows; lane = row
        static_assert(NT / 64 == CH, "one wave per 16-byte chunk of a v row");
        const int lane = tid & 63, c = tid >> 6, t = min(m0 + lane, p.P - 1), h = blockIdx.y - n_groups;
        const u32x4 v = *(const u32x4 *)(p.qkv + (size_t)t * 3 * E + 2 * (size_t)E + (size_t)h * HD + 8 * c);
        float bb[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (p.bias) {
            const float *bp = p.bias + 2 * (size_t)E + (size_t)h * HD + 8 * c;
            const float4 b0 = *(const float4 *)bp, b1 = *(const float4 *)(bp + 4);
            bb[0] = b0.x; bb[1] = b0.y; bb[2] = b0.z; bb[3] = b0.w; bb[4] = b1.x; bb[5] = b1.y; bb[6] = b1.z; bb[7] = b1.w;
        }
        if (m0 + lane >= p.P) return;
        uint16_t *col = p.vt_plane + ((size_t)h * HD + 8 * c) * p.kvT + (size_t)p.tok_kv[t];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            col[(size_t)(2 * e) * p.kvT] = f2bf(bf_lo(v[e]) + bb[2 * e]);
            col[(size_t)(2 * e + 1) * p.kvT] = f2bf(bf_hi(v[e]) + bb[2 * e + 1]);
        }
        return;
    }
    const int h0 = blockIdx.y * HG, hg = min(HG, p.heads - h0);
    // q and k: the loads go out first, the cos/sin table is computed while they land
    const int j = tid % (HALF / 4), hh = (tid / (HALF / 4)) % HG, rg = tid / (HALF / 4 * HG);
    const int h = h0 + min(hh, hg - 1);
    uint2 x[RPT][2][2];
#pragma unroll
    for (int k = 0; k < RPT; k++) {
        const int t = min(m0 + rg * RPT + k, p.P - 1);
        const uint16_t *row = p.qkv + (size_t)t * 3 * E + (size_t)h * HD + 4 * j;
#pragma unroll
        for (int part = 0; part < 2; part++)
#pragma unroll
            for (int s = 0; s < 2; s++) x[k][part][s] = *(const uint2 *)(row + (size_t)part * E + s * HALF);
    }
    float b[2][2][4];   // [q, k][dims 4j.., 4j + 36..][e]
#pragma unroll
    for (int part = 0; part < 2; part++)
#pragma unroll
        for (int s = 0; s < 2; s++) {
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (p.bias) v = *(const float4 *)(p.bias + (size_t)part * E + (size_t)h * HD + 4 * j + s * HALF);
            b[part][s][0] = v.x; b[part][s][1] = v.y; b[part][s][2] = v.z; b[part][s][3] = v.w;
        }
    for (int id = tid; id < BM * HALF; id += NT) {
        const int r = id / HALF, i = id % HALF, t = min(m0 + r, p.P - 1);
        const float pos = (float)p.pos2[2 * (size_t)t + (i < QUART ? 0 : 1)];
        float sn, cs;
        rope_sincos(pos * p.inv_freq[i < QUART ? i : i - QUART], &sn, &cs);
        table[id] = make_float2(cs, sn);
    }
    __syncthreads();
    if (hh >= hg) return;
#pragma unroll
    for (int k = 0; k < RPT; k++) {
        const int r = rg * RPT + k, t = m0 + r;
        if (t >= p.P) break;
        const float2 *c = table + r * HALF + 4 * j;
        const float2 c4[4] = {c[0], c[1], c[2], c[3]};
        const size_t kv = (size_t)p.tok_kv[t];
#pragma unroll
        for (int part = 0; part < 2; part++) {
            const uint2 lo = x[k][part][0], hi = x[k][part][1];
            const float a[4] = {bf_lo(lo.x) + b[part][0][0], bf_hi(lo.x) + b[part][0][1], bf_lo(lo.y) + b[part][0][2], bf_hi(lo.y) + b[part][0][3]};
            const float z[4] = {bf_lo(hi.x) + b[part][1][0], bf_hi(hi.x) + b[part][1][1], bf_lo(hi.y) + b[part][1][2], bf_hi(hi.y) + b[part][1][3]};
            uint16_t ro[4], rh[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                ro[e] = f2bf(fmaf(a[e], c4[e].x, -z[e] * c4[e].y));
                rh[e] = f2bf(fmaf(z[e], c4[e].x, a[e] * c4[e].y));
            }
            const uint2 wo = make_uint2(ro[0] | ((unsigned)ro[1] << 16), ro[2] | ((unsigned)ro[3] << 16));
            const uint2 wh = make_uint2(rh[0] | ((unsigned)rh[1] << 16), rh[2] | ((unsigned)rh[3] << 16));
            uint16_t *dst = part == 0 ? p.q_plane + ((size_t)h * p.P + t) * HD : p.k_plane + ((size_t)h * p.kvT + kv) * HD;
            *(uint2 *)(dst + 4 * j) = wo;
            *(uint2 *)(dst + 4 * j + HALF) = wh;
        }
    }
}

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
        // explicit fmas: the rounding is the same in every form of the prologue
        qo[row][i] = f2bf(fmaf(q0, cs, -q1 * sn));
        qo[row][i + HALF] = f2bf(fmaf(q1, cs, q0 * sn));
        ko[row][i] = f2bf(fmaf(k0, cs, -k1 * sn));
        ko[row][i + HALF] = f2bf(fmaf(k1, cs, k0 * sn));
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
