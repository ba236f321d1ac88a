// Omni decoder attention for head dim 128 on CDNA4: FP32 operands, causal within each packed
// record, ungated, with the output accumulated in FP64 (metal/clef.metal:2055-2319:
// omni_attn_prep, omni_attention).
//
// The reference keeps the P.V accumulator as an FP32 hi/lo pair so that thousands of updates
// do not round into one component. Here the P.V product runs on the FP64 matrix cores
// (v_mfma_f64_16x16x4f64): P and V widened to FP64 give exact products and FP64 sums, which
// covers the same need with no VALU compensation steps. The scores stay FP32 like the
// reference's (v_mfma_f32_16x16x4f32).
//
// Workgroup: one wave per q head of a GQA group (nh / nkv waves), all on the same 16 query
// rows of one record, so one 32-key K/V tile in LDS serves the whole group.
//   S^T = K . Q^T      f32 MFMA: A = 16 keys x 4 dims of K (LDS), B = the wave's Q (registers).
//   O^T += V^T . P^T   f64 MFMA: A = 16 dims x 4 keys of V (LDS, widened), B = P (registers).
// S^T's A rows take key 4(r%4) + r/4 for row r, so the four scores a lane holds are the keys of
// four consecutive 4-key steps of the P.V product: P is the next product's B operand with no
// shuffle. The f64 product's A rows take dim 32(r%4) + 8(r/4) + n in dim tile n, so a lane's
// accumulators cover 32 consecutive dims of its query row and the epilogue stores whole runs.
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <utility>


namespace clef_hip {
namespace omni {

constexpr int HD = 128;
constexpr int BQ = 16;                  // query rows per block (every wave of the group)
constexpr int BK = 32;                  // keys per LDS tile
constexpr int TILE = BK * HD;           // floats per K or V tile (16 KB)
constexpr int SLACK = 32;               // zero rows after each kv head's T rows

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) double f64x4;

struct PrepParams {
    const float *qkv;           // [T][(nh + 2 nkv) * 128]
    const float *q_norm, *k_norm;
    const int32_t *pos3;        // [T][3]
    const float *freq;          // [192]: f32 inverse frequencies, then FP64 hi, lo parts
    float *q_plane;             // [nh][T][128]
    float *k_plane, *v_plane;   // [nkv][kvT][128]
    uint32_t *status;
    int nh, nkv, T, kvT, rope_exact;
    float eps;
};

struct AttnParams {
    const float *q_plane, *k_plane, *v_plane;
    const int32_t *blocks;      // [n_blk][8] {q_row0, nq, q_pos0, k_row0, k_len, 0, record, 0}
    float *out;                 // [T][nh * 128]
    int nh, nkv, T, kvT, n_blk;
    float scale;
};

// Rotary angle pos * f reduced to [-pi, pi] in FP64 (f = hi + lo, the FP64 frequency): the
// product of an integer below 2^24 and f is exact to FP64 rounding, and the reduction by a
// two-part 2*pi leaves an error far below FP32's resolution of the reduced angle.
__device__ __forceinline__ float omni_angle_exact(int position, float hi, float lo) {
    const double a = (double)position * ((double)hi + (double)lo);
    const double k = rint(a * 0.15915494309189535);   // 1 / (2 pi)
    double r = fma(-k, 6.283185307179586, a);          // 2 pi, FP64 nearest
    r = fma(-k, 2.4492935982947064e-16, r);           // 2 pi - its FP64 nearest
    return (float)r;
}

// One (pass row, head) item per 32 lanes; lane holds dims lane + 32 j, so the rotary pairs
// (d, d + 64) of d = lane and lane + 32 sit in the lane. Items past the pass rows zero the
// kv planes' slack rows.
__global__ __launch_bounds__(256) void omni_prep_kernel(PrepParams p) {
    const int heads = p.nh + p.nkv;
    const long item = (long)blockIdx.x * 8 + (threadIdx.x >> 5);
    const int lane = threadIdx.x & 31;
    const long n_items = (long)(p.T + SLACK) * heads;
    if (item >= n_items) return;
    const int t = (int)(item / heads), h = (int)(item % heads);
    const bool query = h < p.nh;
    const int kh = h - p.nh;
    if (t >= p.T) {
        if (!query) {
            float *kd = p.k_plane + ((size_t)kh * p.kvT + t) * HD, *vd = p.v_plane + ((size_t)kh * p.kvT + t) * HD;
#pragma unroll
            for (int j = 0; j < 4; j++) { kd[lane + 32 * j] = 0.f; vd[lane + 32 * j] = 0.f; }
        }
        return;
    }
    const size_t row = (size_t)(p.nh + 2 * p.nkv) * HD;
    const float *src = p.qkv + (size_t)t * row + (size_t)h * HD;
    const float *w = query ? p.q_norm : p.k_norm;
    float x[4], ss = 0.f;
    bool bad = false;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        x[j] = src[lane + 32 * j];
        bad |= !isfinite(x[j]);
        ss += x[j] * x[j];
    }
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 32);
    const float inv = 1.0f / sqrtf(ss / (float)HD + p.eps);
#pragma unroll
    for (int j = 0; j < 4; j++) x[j] = x[j] * inv * w[lane + 32 * j];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        // interleaved M-RoPE over 64 pairs: pair i turns by axis i % 3, the last 4 by axis 0
        const int pair = lane + 32 * j, axis = pair < 60 ? pair % 3 : 0;
        const int position = p.pos3[3 * (size_t)t + axis];
        const float ang = p.rope_exact ? omni_angle_exact(position, p.freq[64 + pair], p.freq[128 + pair])
                                       : (float)position * p.freq[pair];
        float s, c;
        sincosf(ang, &s, &c);
        const float lo = x[j], hi = x[j + 2];
        x[j] = lo * c - hi * s;
        x[j + 2] = hi * c + lo * s;
    }
    if (query) {
        float *dst = p.q_plane + ((size_t)h * p.T + t) * HD;
#pragma unroll
        for (int j = 0; j < 4; j++) { bad |= !isfinite(x[j]); dst[lane + 32 * j] = x[j]; }
    } else {
        const float *vs = p.qkv + (size_t)t * row + (size_t)(p.nh + p.nkv + kh) * HD;
        float *kd = p.k_plane + ((size_t)kh * p.kvT + t) * HD, *vd = p.v_plane + ((size_t)kh * p.kvT + t) * HD;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float v = vs[lane + 32 * j];
            bad |= !isfinite(x[j]) || !isfinite(v);
            kd[lane + 32 * j] = x[j];
            vd[lane + 32 * j] = v;
        }
    }
    // A softmax max can hide a non-finite input; it is reported on its own.
    if (bad) atomicOr(p.status, 2u);
}

typedef __attribute__((address_space(3))) void lds_void;

// max over the four 16-lane rows of a wave (permlane swaps, VALU only); every lane gets it
__device__ __forceinline__ float xrow_max(float x) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float m = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    return fmaxf(__uint_as_float(q[0]), __uint_as_float(q[1]));
}

// 16-byte chunk swizzle of a 512-byte K / V row: distinct over the 16 keys one read touches
__device__ __forceinline__ int swz(int key) { return (key & 15) ^ ((key >> 4) << 2); }

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

// Grid: one workgroup per (block, kv head); wave w is q head kh * W + w.
template <int W>
__global__ __launch_bounds__(64 * W) void omni_attn_kernel(AttnParams p) {
    __shared__ __attribute__((aligned(16))) float smem[4 * TILE];   // K0 | K1 | V0 | V1
    const int bi = blockIdx.x / p.nkv, kh = blockIdx.x % p.nkv;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r16 = lane & 15, g = lane >> 4;
    const int h = kh * W + wave;
    const int32_t *blk = p.blocks + 8 * bi;
    const int q_row0 = blk[0], nq = blk[1], q_pos0 = blk[2], k_row0 = blk[3], k_len = blk[4];
    const int n_tiles = (k_len + BK - 1) / BK;
    const bool q_valid = r16 < nq;
    const int qpos = q_pos0 + r16;

    // ---- tile fills: a tile is 16 DMA groups of 1 KB (2 keys); wave w fills groups w*16/W ...
    const float *kbase = p.k_plane + ((size_t)kh * p.kvT + k_row0) * HD;
    const float *vbase = p.v_plane + ((size_t)kh * p.kvT + k_row0) * HD;
    constexpr int PER = 16 / W;
    unsigned fo[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int grp = wave * PER + j, key = 2 * grp + (lane >> 5);
        fo[j] = (unsigned)(key * HD + ((lane & 31) ^ swz(key)) * 4) * 4u;
    }
    auto fill = [&](int kb, float *Ks, float *Vs) {
        const char *kt = (const char *)(kbase + (size_t)kb * HD), *vt = (const char *)(vbase + (size_t)kb * HD);
#pragma unroll
        for (int j = 0; j < PER; j++)
            __builtin_amdgcn_global_load_lds((const void *)(kt + fo[j]), (lds_void *)(Ks + (wave * PER + j) * 256), 16, 0, 0);
#pragma unroll
        for (int j = 0; j < PER; j++)
            __builtin_amdgcn_global_load_lds((const void *)(vt + fo[j]), (lds_void *)(Vs + (wave * PER + j) * 256), 16, 0, 0);
    };

    // ---- per-lane LDS byte addresses of the operand reads (buffer 0; buffer 1 at +TILE floats)
    const unsigned base = (unsigned)(uintptr_t)(const __attribute__((address_space(3))) float *)smem;
    unsigned ka[2];   // K row of S^T A row r16 in 16-key subtile u, chunk 8g (+ j via XOR below)
    int kx[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int key = 16 * u + 4 * (r16 & 3) + (r16 >> 2);
        ka[u] = base + (unsigned)key * HD * 4u;
        kx[u] = swz(key);
    }
    const int vd0 = 32 * (r16 & 3) + 8 * (r16 >> 2);   // first of the 8 dims this lane's V A rows take

    // ---- Q: lane holds Q[row r16][32 g + c], c = 0..31 (the B operand of step c)
    float qf[32];
    {
        const int qr = q_valid ? r16 : 0;
        const f32x4 *qs = (const f32x4 *)(p.q_plane + ((size_t)h * p.T + q_row0 + qr) * HD + 32 * g);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const f32x4 v = qs[j];
            qf[4 * j] = v.x; qf[4 * j + 1] = v.y; qf[4 * j + 2] = v.z; qf[4 * j + 3] = v.w;
        }
    }
    if (n_tiles > 0) fill(0, smem, smem + 2 * TILE);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    f64x4 o[8];
#pragma unroll
    for (int n = 0; n < 8; n++) o[n] = f64x4{0.0, 0.0, 0.0, 0.0};
    float m_run = -INFINITY;
    double l_run = 0.0;

    auto tile = [&](const int t, auto BUF) {
        constexpr int buf = decltype(BUF)::value;
        const int kb = t * BK;
        if (t + 1 < n_tiles) fill(kb + BK, smem + (buf ^ 1) * TILE, smem + 2 * TILE + (buf ^ 1) * TILE);
        // S^T: two 16-key subtiles, 32 four-dim steps each
        f32x4 s[2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            f32x4 a[8];
            sfor<8>([&](auto J) {
                constexpr int j = decltype(J)::value;
                a[j] = lds_read_f4<buf * TILE * 4>(ka[u] + (unsigned)(((8 * g + j) ^ kx[u]) * 16));
            });
            s[u] = f32x4{0.f, 0.f, 0.f, 0.f};
            sfor<8>([&](auto J) {
                constexpr int j = decltype(J)::value;
                lds_wait_f4<7 - j>(a[j]);
#pragma unroll
                for (int e = 0; e < 4; e++)
                    s[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j][e], qf[4 * j + e], s[u], 0, 0, 0);
            });
        }
        // Online softmax. s[u][v] is the score of key kb + 16u + 4v + g for query row r16.
        float x[2][4], mx = -INFINITY;
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int key = kb + 16 * u + 4 * v + g;
                const bool ok = q_valid && key < k_len && key <= qpos;
                x[u][v] = ok ? s[u][v] * p.scale : -INFINITY;
                mx = fmaxf(mx, x[u][v]);
            }
        const float mn = fmaxf(m_run, xrow_max(mx));
        double pd[2][4];
        float alpha = 1.f, rs = 0.f;
        if (mn != -INFINITY) {
            alpha = (m_run == -INFINITY) ? 0.f : expf(m_run - mn);
#pragma unroll
            for (int u = 0; u < 2; u++)
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const float pv = x[u][v] == -INFINITY ? 0.f : expf(x[u][v] - mn);
                    pd[u][v] = (double)pv;
                    rs += pv;
                }
        } else {
#pragma unroll
            for (int u = 0; u < 2; u++)
#pragma unroll
                for (int v = 0; v < 4; v++) pd[u][v] = 0.0;
        }
        m_run = mn;
        l_run = l_run * (double)alpha + (double)rs;
        if (__any(alpha != 1.f)) {
            const double ad = (double)alpha;
#pragma unroll
            for (int n = 0; n < 8; n++) o[n] *= ad;
        }
        // O^T += V^T . P^T: 8 four-key steps (u, v), each 8 dim tiles
        f32x4 vb[2][2];
        auto vread = [&](auto U, auto V, f32x4 *dst) {
            constexpr int u = decltype(U)::value, v = decltype(V)::value;
            const int key = 16 * u + 4 * v + g;
            const unsigned row = base + (unsigned)(2 * TILE + key * HD) * 4u;
            const int x = swz(key);
            dst[0] = lds_read_f4<buf * TILE * 4>(row + (unsigned)((((vd0 >> 2)) ^ x) * 16));
            dst[1] = lds_read_f4<buf * TILE * 4>(row + (unsigned)((((vd0 >> 2) + 1) ^ x) * 16));
        };
        vread(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, vb[0]);
        sfor<8>([&](auto S) {
            constexpr int st = decltype(S)::value, u = st >> 2, v = st & 3, cur = st & 1;
            if constexpr (st + 1 < 8)
                vread(std::integral_constant<int, ((st + 1) >> 2)>{}, std::integral_constant<int, (st + 1) & 3>{}, vb[cur ^ 1]);
            if constexpr (st + 1 < 8) {
                lds_wait_f4<2>(vb[cur][0]);
                lds_wait_f4<2>(vb[cur][1]);
            } else {
                lds_wait_f4<0>(vb[cur][0]);
                lds_wait_f4<0>(vb[cur][1]);
            }
            const double b = pd[u][v];
#pragma unroll
            for (int n = 0; n < 8; n++) {
                const float a = n < 4 ? vb[cur][0][n] : vb[cur][1][n - 4];
                o[n] = __builtin_amdgcn_mfma_f64_16x16x4f64((double)a, b, o[n], 0, 0, 0);
            }
        });
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    };
    for (int t = 0; t < n_tiles; t += 2) {
        tile(t, std::integral_constant<int, 0>{});
        if (t + 1 < n_tiles) tile(t + 1, std::integral_constant<int, 1>{});
    }

    // ---- epilogue: O = O^T / l; lane holds dims 32 g + 8 v + n of row r16 (accumulator n, entry v)
    double l_row = l_run;
    l_row += __shfl_xor(l_row, 16);
    l_row += __shfl_xor(l_row, 32);
    if (q_valid) {
        const double il = l_row > 0.0 ? 1.0 / l_row : 0.0;
        float *dst = p.out + (size_t)(q_row0 + r16) * p.nh * HD + (size_t)h * HD + 32 * g;
#pragma unroll
        for (int v = 0; v < 4; v++) {
            f32x4 w0, w1;
#pragma unroll
            for (int n = 0; n < 4; n++) {
                w0[n] = (float)(o[n][v] * il);
                w1[n] = (float)(o[n + 4][v] * il);
            }
            *(f32x4 *)(dst + 8 * v) = w0;
            *(f32x4 *)(dst + 8 * v + 4) = w1;
        }
    }
}

}  // namespace omni
}  // namespace clef_hip
