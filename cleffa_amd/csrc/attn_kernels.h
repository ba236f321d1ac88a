// Prefill attention kernels for CDNA4 (gfx950): packed varlen causal GQA attention over
// record-aligned query blocks, with the Q prologue (per-head RMSNorm + partial rotary) fused
// into the attention kernel and the sigmoid output gate fused into its epilogue, a K/V
// prologue kernel that writes the K and V^T planes, and the vision tower's prologue
// (bias + 2-D rotary) feeding the same attention kernel at head dim 72.
//
// Semantics follow cleffa's attention family (metal/clef.metal:245-300 attn_prep,
// metal/clef.metal:930-1093 attention_tu, metal/clef.metal:657-849 prefix variant,
// metal/clef.metal:1616-1964 vision), restated for 64-wide wavefronts and bf16 MFMA.
//
// Compute layout (per workgroup = 4 wavefronts, one query block of 128 rows of one q head):
//   S^T = K . Q^T      v_mfma_f32_32x32x16_bf16, A = K rows from LDS, B = Q held in VGPRs.
//                      Each lane ends up owning one query column and 32 keys of a 64-key tile,
//                      so the row max / row sum need one cross-half exchange only.
//   O^T += V^T . P^T   A = V^T rows from LDS (V is stored transposed in HBM by the prologue),
//                      B = bf16 P straight from the softmax registers (no LDS round trip).
// The A-operand rows of both products are read in a bit-permuted order (bits 2 and 3 of the
// row index swapped) so that the MFMA output rows a lane owns are 8 consecutive keys / dims:
// P feeds the next product without shuffles and the epilogue stores 16-byte runs.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_params.h"

namespace clef_hip {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(16))) float f32x16;
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
__device__ __forceinline__ uint16_t f2bf(float a) {
    __bf16 v = (__bf16)a;
    return __builtin_bit_cast(uint16_t, v);
}

// Row permutation of the MFMA A operand: swap bits 2 and 3.
__device__ __forceinline__ int perm_row(int r) {
    return (r & 0x13) | ((r & 4) << 1) | ((r & 8) >> 1);
}
// Key (or head dim) offset within a 32-row MFMA tile of output element i of a lane in half hf.
__device__ __forceinline__ constexpr int out_off(int i, int hf) {
    return (i & 7) + 8 * hf + 16 * (i >> 3);
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

__device__ __forceinline__ float wave_max_pair(float v) {
    return fmaxf(v, __shfl_xor(v, 32, 64));
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

// ------------------------------------------------------------------------------------------
// Attention core.
//   HD     logical head dim (256 text, 72 vision)
//   HDK    QK^T contraction length, HD rounded up to 16 (also the K / Q plane row stride)
//   HDM    PV output rows, HD rounded up to 32
//   BK     keys per LDS tile (64)
//   TEXT   true: Q comes from the fused qkv rows with RMSNorm + rotary applied here and the
//          sigmoid gate from the same rows; false: Q from a prepared plane, no gate.
//   NROT   rotary dims of the text Q prologue (0 or a multiple of 32)
//   PIPE   true: S(t+1) = K(t+1).Q^T is issued before the softmax of tile t so the MFMA and
//          VALU work of neighbouring tiles can overlap (two score register sets).
//   DIRECT true: K / V^T tiles go global -> LDS with global_load_lds (no VGPR staging) into
//          unpadded, XOR-swizzled LDS rows; needs 512-byte K rows (HD 256). false: tiles are
//          staged through VGPRs into padded LDS rows.
// ------------------------------------------------------------------------------------------
template <int HD, int BK, bool DIRECT>
struct AttnCfg {
    static constexpr int HDK = (HD + 15) / 16 * 16;
    static constexpr int HDM = (HD + 31) / 32 * 32;
    static constexpr int NC = HDK / 16;          // Q chunks (MFMA k steps of S)
    static constexpr int NM = HDM / 32;          // O^T row tiles
    static constexpr int NKT = BK / 32;          // S^T row tiles per key tile
    static constexpr int KROW = DIRECT ? HDK : HDK + 8;   // LDS row stride of the K tile (elements)
    static constexpr int VROW = DIRECT ? BK : BK + 8;     // LDS row stride of the V^T tile (elements)
    static constexpr int KTILE = BK * KROW;
    static constexpr int VTILE = HDM * VROW;
    static constexpr int STAGE = KTILE + VTILE;   // one K + one V^T buffer
    static constexpr int KCHUNKS = BK * HDK / 8;  // 16-byte chunks per K tile
    static constexpr int VCHUNKS = HD * BK / 8;   // 16-byte chunks per V^T tile (HD rows)
    static constexpr int KCH = (KCHUNKS + 255) / 256;
    static constexpr int VCH = (VCHUNKS + 255) / 256;
    static_assert(!DIRECT || (HDK == 256 && BK == 64 && HD == HDM), "direct tiles assume hd 256, 64 keys");
};

typedef __attribute__((address_space(3))) void lds_void;

template <int HD, int BK, bool TEXT, int NROT, bool DIRECT, bool PIPE>
__global__ __launch_bounds__(256, 1) void attn_fwd_kernel(AttnParams p) {
    using C = AttnCfg<HD, BK, DIRECT>;
    constexpr int HDK = C::HDK, NC = C::NC, NM = C::NM, NKT = C::NKT;
    constexpr int KROW = C::KROW, VROW = C::VROW;
    static_assert(NROT % 32 == 0 && NROT <= HDK, "rotary dims");
    __shared__ __attribute__((aligned(16))) uint16_t smem[2 * C::STAGE];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lq = lane & 31, hf = lane >> 5;

    const int bi = blockIdx.x / p.nh;
    const int h = blockIdx.x - bi * p.nh;
    const int32_t *blk = p.blocks + 8 * bi;
    const int q_row0 = blk[0], nq = blk[1], q_pos0 = blk[2], k_row0 = blk[3], k_len = blk[4];
    const int flag_row = blk[5];
    const int kh = h / (p.nh / p.nkv);

    const int my_q = wave * 32 + lq;
    const bool q_valid = my_q < nq;
    const int qpos = q_pos0 + my_q;
    const bool wave_live = wave * 32 < nq;
    const int wave_last_pos = q_pos0 + wave * 32 + 31;

    // ---- Q prologue: lane holds Q[my_q][c*16 + hf*8 + j] for chunks c, as the S^T B operand.
    bf16x8 qf[NC];
    {
        float x[NC][8];
        const size_t qrow = (size_t)q_row0 + (q_valid ? my_q : 0);
        if (TEXT) {
            const uint16_t *src = p.qkv + qrow * p.row + (size_t)h * 2 * HD;
            float ss = 0.f;
#pragma unroll
            for (int c = 0; c < NC; c++) {
                u32x4 w = q_valid ? *(const u32x4 *)(src + c * 16 + hf * 8) : u32x4{0, 0, 0, 0};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    x[c][2 * j] = bf_lo(w[j]);
                    x[c][2 * j + 1] = bf_hi(w[j]);
                }
#pragma unroll
                for (int j = 0; j < 8; j++) ss += x[c][j] * x[c][j];
            }
            ss += __shfl_xor(ss, 32, 64);
            if (p.q_norm) {   // NULL: no q/k norm (plain SDPA inputs)
                const float inv = rsqrtf(ss / (float)HD + p.eps);
#pragma unroll
                for (int c = 0; c < NC; c++) {
                    const float4 w0 = *(const float4 *)(p.q_norm + c * 16 + hf * 8);
                    const float4 w1 = *(const float4 *)(p.q_norm + c * 16 + hf * 8 + 4);
                    const float wn[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
                    for (int j = 0; j < 8; j++) x[c][j] = x[c][j] * inv * wn[j];
                }
            }
            if (NROT > 0) {
                // NeoX partial rotary: pair (i, i + NROT/2), both dims in this lane at chunks
                // c and c + R. Interleaved M-RoPE: pair i turns by axis i % 3 of pos3.
                constexpr int R = NROT / 32;
                const int32_t *pp = p.pos3 + 3 * qrow;
                const float pt = (float)pp[0], ph = (float)pp[1], pw = (float)pp[2];
#pragma unroll
                for (int c = 0; c < R; c++) {
                    const float4 f0 = *(const float4 *)(p.inv_freq + c * 16 + hf * 8);
                    const float4 f1 = *(const float4 *)(p.inv_freq + c * 16 + hf * 8 + 4);
                    const float fr[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        const int i = c * 16 + hf * 8 + j;
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
        } else {
            const uint16_t *src = p.q_plane + ((size_t)h * p.T + qrow) * HDK;
#pragma unroll
            for (int c = 0; c < NC; c++) {
                u32x4 w = q_valid ? *(const u32x4 *)(src + c * 16 + hf * 8) : u32x4{0, 0, 0, 0};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    x[c][2 * j] = bf_lo(w[j]);
                    x[c][2 * j + 1] = bf_hi(w[j]);
                }
            }
        }
#pragma unroll
        for (int c = 0; c < NC; c++) {
            u32x4 w = {pack_bf16(x[c][0], x[c][1]), pack_bf16(x[c][2], x[c][3]),
                       pack_bf16(x[c][4], x[c][5]), pack_bf16(x[c][6], x[c][7])};
            qf[c] = __builtin_bit_cast(bf16x8, w);
        }
    }

    // ---- K / V^T tiles in LDS: two K buffers, then two V^T buffers.
    // Iteration t computes S(t+1) = K(t+1).Q^T on the MFMA pipe while the VALU runs the softmax
    // of S(t), then O += V(t)^T.P(t); meanwhile K(t+2) and V(t+1) stream into the free buffers.
    const uint16_t *kbase = p.k_plane + ((size_t)kh * p.kvT + k_row0) * HDK;
    const uint16_t *vbase = p.vt_plane + (size_t)kh * HD * p.kvT + k_row0;
    const int last_chunk = ((k_len > 0 ? k_len - 1 : 0) / 8) * 8;   // start of the last valid 8-key chunk
    u32x4 stK[DIRECT ? 1 : C::KCH], stV[DIRECT ? 1 : C::VCH];
    auto Kbuf = [&](int b) { return smem + b * C::KTILE; };
    auto Vbuf = [&](int b) { return smem + 2 * C::KTILE + b * C::VTILE; };

    // DIRECT: wave w fills LDS slots [(w*8 + j)*64, +64) of each 2048-slot tile with one
    // global_load_lds per j. K slot s holds key s/32, chunk (s%32) ^ (key & 15); V^T slot s
    // holds dim s/8, key chunk (s%8) ^ ((dim >> 1) & 7). Rows past the record are clamped to
    // valid addresses (their scores are masked; their values are zeroed in LDS before use).
    // Staged (not DIRECT): global -> VGPRs now, VGPRs -> padded LDS rows in store_k / store_v.
    auto load_k = [&](int kb, int b) {
        if (DIRECT) {
            uint16_t *Ks = Kbuf(b);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int grp = wave * 8 + j;
                const int key = grp * 2 + (lane >> 5);
                const int c = (lane & 31) ^ (key & 15);
                const int krow = min(kb + key, k_len - 1);
                __builtin_amdgcn_global_load_lds((const void *)(kbase + (size_t)krow * HDK + c * 8),
                                                 (lds_void *)(Ks + grp * 512), 16, 0, 0);
            }
        } else {
#pragma unroll
            for (int j = 0; j < C::KCH; j++) {
                const int id = tid + 256 * j;
                const int key = id / (HDK / 8), c8 = id % (HDK / 8);
                u32x4 w = {0, 0, 0, 0};
                if ((C::KCHUNKS % 256 == 0 || id < C::KCHUNKS) && kb + key < k_len)
                    w = *(const u32x4 *)(kbase + (size_t)(kb + key) * HDK + c8 * 8);
                stK[j] = w;
            }
        }
    };
    auto load_v = [&](int kb, int b) {
        if (DIRECT) {
            uint16_t *Vs = Vbuf(b);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int grp = wave * 8 + j;
                const int d = grp * 8 + (lane >> 3);
                const int c = (lane & 7) ^ ((d >> 1) & 7);
                const int kk = min(kb + c * 8, last_chunk);
                __builtin_amdgcn_global_load_lds((const void *)(vbase + (size_t)d * p.kvT + kk),
                                                 (lds_void *)(Vs + grp * 512), 16, 0, 0);
            }
        } else {
#pragma unroll
            for (int j = 0; j < C::VCH; j++) {
                const int id = tid + 256 * j;
                const int d = id / (BK / 8), c8 = id % (BK / 8);
                const int kk = kb + c8 * 8;
                u32x4 w = {0, 0, 0, 0};
                if ((C::VCHUNKS % 256 == 0 || id < C::VCHUNKS) && kk < k_len)
                    w = *(const u32x4 *)(vbase + (size_t)d * p.kvT + kk);
                stV[j] = w;
            }
        }
    };
    auto store_k = [&](int b) {
        uint16_t *Ks = Kbuf(b);
#pragma unroll
        for (int j = 0; j < C::KCH; j++) {
            const int id = tid + 256 * j;
            if (C::KCHUNKS % 256 == 0 || id < C::KCHUNKS) {
                const int key = id / (HDK / 8), c8 = id % (HDK / 8);
                *(u32x4 *)(Ks + key * KROW + c8 * 8) = stK[j];
            }
        }
    };
    auto store_v = [&](int kb, int b) {   // keys past the record are written as zeros
        uint16_t *Vs = Vbuf(b);
#pragma unroll
        for (int j = 0; j < C::VCH; j++) {
            const int id = tid + 256 * j;
            if (C::VCHUNKS % 256 == 0 || id < C::VCHUNKS) {
                const int d = id / (BK / 8), c8 = id % (BK / 8);
                const int kk = kb + c8 * 8;
                u32x4 w = stV[j];
                if (kk + 8 > k_len) {
                    const int keep = k_len - kk;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        if (2 * e >= keep) w[e] = 0;
                        else if (2 * e + 1 >= keep) w[e] &= 0xffffu;
                    }
                }
                *(u32x4 *)(Vs + d * VROW + c8 * 8) = w;
            }
        }
    };
    // DIRECT tail tile: zero the V^T entries of keys >= k_len (the loads left clamped copies).
    auto zero_tail = [&](int kb, int b) {
        uint16_t *Vs = Vbuf(b);
        const int valid = k_len - kb;   // 1..BK-1
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int s = tid + 256 * j;
            const int d = s >> 3, c = (s & 7) ^ ((d >> 1) & 7);
            const int k0 = c * 8;
            u32x4 w = *(u32x4 *)(Vs + s * 8);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const unsigned keep = (k0 + 2 * e + 1 < valid) ? 0xffffffffu : (k0 + 2 * e < valid ? 0xffffu : 0u);
                w[e] &= keep;
            }
            *(u32x4 *)(Vs + s * 8) = w;
        }
    };

    f32x16 o[NM];
#pragma unroll
    for (int mt = 0; mt < NM; mt++)
#pragma unroll
        for (int i = 0; i < 16; i++) o[mt][i] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;
    const float sl2 = p.scale_log2;
    const int n_tiles = (k_len + BK - 1) / BK;
    const int prow = perm_row(lq);
    // per-lane LDS element offsets of the A operands
    //   K: row (kt*32 + prow), 16-byte chunk 2c + hf, c = 8*ch + cl (DIRECT: chunk ^ (prow & 15))
    //   V: row (mt*32 + prow), chunk 4kt + 2cc + hf (DIRECT: chunk ^ ((prow >> 1) & 7))
    int koff[C::NC < 8 ? C::NC : 8], voff[NKT][2];
#pragma unroll
    for (int cl = 0; cl < (NC < 8 ? NC : 8); cl++)
        koff[cl] = DIRECT ? prow * KROW + (((2 * cl + hf) ^ (prow & 15)) * 8) : prow * KROW + (2 * cl + hf) * 8;
#pragma unroll
    for (int kt = 0; kt < NKT; kt++)
#pragma unroll
        for (int cc = 0; cc < 2; cc++)
            voff[kt][cc] = DIRECT ? prow * VROW + (((4 * kt + 2 * cc + hf) ^ ((prow >> 1) & 7)) * 8)
                                  : prow * VROW + kt * 32 + cc * 16 + hf * 8;

    auto act = [&](int t) { return wave_live && (!p.causal || t * BK <= wave_last_pos); };
    auto qk = [&](int b, f32x16 *s) {
        const uint16_t *Ks = Kbuf(b);
#pragma unroll
        for (int kt = 0; kt < NKT; kt++) {
#pragma unroll
            for (int i = 0; i < 16; i++) s[kt][i] = 0.f;
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const bf16x8 a = *(const bf16x8 *)(Ks + kt * 32 * KROW + (c >> 3) * 128 + koff[c & 7]);
                s[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[c], s[kt], 0, 0, 0);
            }
        }
    };

    auto tile = [&](int t, f32x16 *s_cur, f32x16 *s_nxt) {
        const int kb = t * BK;
        const int vb = t & 1;
        if (DIRECT && kb + BK > k_len) {   // WG-uniform: only the block's last tile
            zero_tail(kb, vb);
            __syncthreads();
        }
        if (PIPE) {
            if (t + 2 < n_tiles) load_k(kb + 2 * BK, vb);
            if (t + 1 < n_tiles) load_v(kb + BK, vb ^ 1);
            if (t + 1 < n_tiles && act(t + 1)) qk(vb ^ 1, s_nxt);
        } else if (t + 1 < n_tiles) {
            load_k(kb + BK, vb ^ 1);
            load_v(kb + BK, vb ^ 1);
        }
        if (act(t)) {
            if (!PIPE) qk(vb, s_cur);
            const uint16_t *Vs = Vbuf(vb);
            // Online softmax in the exp2 domain. Masked scores are -inf, so their P is an
            // exact zero and a tile past a row's diagonal rescales the row by exactly 1.
            const bool need_mask = (kb + BK > k_len) || (p.causal && kb + BK - 1 > q_pos0 + wave * 32);
            if (need_mask) {
                // key kb + kt*32 + out_off(i, hf) is visible iff <= lim
                const int lim = min(k_len - 1, p.causal ? qpos : k_len - 1) - kb - 8 * hf;
#pragma unroll
                for (int kt = 0; kt < NKT; kt++)
#pragma unroll
                    for (int i = 0; i < 16; i++)
                        s_cur[kt][i] = (kt * 32 + (i & 7) + 16 * (i >> 3) > lim) ? -INFINITY : s_cur[kt][i];
            }
            float mx = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < NKT; kt++)
#pragma unroll
                for (int i = 0; i < 16; i++) mx = fmaxf(mx, s_cur[kt][i]);
            mx = wave_max_pair(mx) * sl2;
            const float mn = fmaxf(m_run, mx);
            const float msub = (mn == -INFINITY) ? 0.f : mn;
            const float alpha = (mn == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(m_run - mn);
            float rs = 0.f;
            bf16x8 pk[NKT][2];
#pragma unroll
            for (int kt = 0; kt < NKT; kt++)
#pragma unroll
                for (int cc = 0; cc < 2; cc++) {
                    unsigned w[4];
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const float p0 = __builtin_amdgcn_exp2f(fmaf(s_cur[kt][cc * 8 + 2 * j], sl2, -msub));
                        const float p1 = __builtin_amdgcn_exp2f(fmaf(s_cur[kt][cc * 8 + 2 * j + 1], sl2, -msub));
                        w[j] = pack_bf16(p0, p1);
                        // The row sum takes the rounded P that the PV product multiplies.
                        rs = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w[j]),
                                                             bf16x2{(__bf16)1.0f, (__bf16)1.0f}, rs, false);
                    }
                    u32x4 wv = {w[0], w[1], w[2], w[3]};
                    pk[kt][cc] = __builtin_bit_cast(bf16x8, wv);
                }
            rs += __shfl_xor(rs, 32, 64);
            l_run = l_run * alpha + rs;
            m_run = mn;
            if (__any(alpha != 1.f)) {
#pragma unroll
                for (int mt = 0; mt < NM; mt++)
#pragma unroll
                    for (int i = 0; i < 16; i++) o[mt][i] *= alpha;
            }
#pragma unroll
            for (int mt = 0; mt < NM; mt++) {
#pragma unroll
                for (int kt = 0; kt < NKT; kt++)
#pragma unroll
                    for (int cc = 0; cc < 2; cc++) {
                        const bf16x8 a = *(const bf16x8 *)(Vs + mt * 32 * VROW + voff[kt][cc]);
                        o[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pk[kt][cc], o[mt], 0, 0, 0);
                    }
            }
        }
        if (!DIRECT) {
            if (PIPE ? t + 2 < n_tiles : t + 1 < n_tiles) store_k(PIPE ? vb : vb ^ 1);
            if (t + 1 < n_tiles) store_v(kb + BK, vb ^ 1);
        } else {
            __builtin_amdgcn_s_waitcnt(0);
        }
        __syncthreads();
    };

    f32x16 s0[NKT], s1[NKT];
    if (n_tiles > 0) {
        load_k(0, 0);
        if (!DIRECT) store_k(0);
        load_v(0, 0);
        if (!DIRECT) store_v(0, 0);
        if (PIPE && n_tiles > 1) {
            load_k(BK, 1);
            if (!DIRECT) store_k(1);
        }
        if (DIRECT) __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (PIPE && act(0)) qk(0, s0);
    }
    if (PIPE) {
        // two tiles per trip so the score registers swap roles without copies
        for (int t = 0; t < n_tiles; t += 2) {
            tile(t, s0, s1);
            if (t + 1 < n_tiles) tile(t + 1, s1, s0);
        }
    } else {
        for (int t = 0; t < n_tiles; t++) tile(t, s0, s0);
    }

    // ---- Epilogue: O / l, times sigmoid(gate) for text, converted and stored.
    if (q_valid) {
        const float il = l_run > 0.f ? 1.f / l_run : 0.f;
        const size_t t = (size_t)q_row0 + my_q;
        int32_t *flag = p.ovf ? p.ovf + flag_row : nullptr;
#pragma unroll
        for (int mt = 0; mt < NM; mt++)
#pragma unroll
            for (int run = 0; run < 2; run++) {
                const int d0 = mt * 32 + 16 * run + 8 * hf;
                if (d0 >= HD) continue;
                float v[8];
#pragma unroll
                for (int j = 0; j < 8; j++) v[j] = o[mt][run * 8 + j] * il;
                if (TEXT && p.gate) {
                    const u32x4 g = *(const u32x4 *)(p.qkv + t * p.row + (size_t)h * 2 * HD + HD + d0);
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        v[2 * j] *= sigmoidf(bf_lo(g[j]));
                        v[2 * j + 1] *= sigmoidf(bf_hi(g[j]));
                    }
                }
                store_out8(p.out, t * p.out_ld + (size_t)h * HD + d0, v, p.out_type, p.f16_lim, flag);
            }
    }
}
// ------------------------------------------------------------------------------------------
// Text K/V prologue (metal/clef.metal:245-300 and 873-928 for K and V): for every pass row t,
// K = RMSNorm(k) * (1+w) then partial rotary, written to row tok_kv[t] of the K plane
// [nkv][kvT][HD]; V copied unnormalised and written transposed into the V^T plane
// [nkv][HD][kvT]. Rows of the planes that no pass row maps to (cached prefix rows, alignment
// padding) are left untouched. When rope_cs is set, the cos/sin of every pass row's rotary
// angles are also written there ([T][n_rot/2] float2) for the attention kernel's Q prologue.
// Grid (T / 16, nkv), 256 threads. The workgroup's rows are consecutive pass rows, so the
// qkv loads need no lookup. A row is handled by 32 lanes with 8 dims each; the RMS sum
// reduces over DPP rows, a rotary pair (i, i + 32) sits in lanes 4 apart.
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
    // global loads first
    const uint16_t *src = p.qkv + (size_t)(t >= 0 ? t : 0) * p.row + (size_t)p.nh * 2 * HD + (size_t)kh * HD + 16 * k;
    u32x4 kw[2], vw[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        kw[h] = t >= 0 ? *(const u32x4 *)(src + 8 * h) : u32x4{0, 0, 0, 0};
        vw[h] = t >= 0 ? *(const u32x4 *)(src + (size_t)p.nkv * HD + 8 * h) : u32x4{0, 0, 0, 0};
    }
    float wn[16];
    if (p.k_norm) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 w4 = *(const float4 *)(p.k_norm + 16 * k + 4 * q);
            wn[4 * q] = w4.x; wn[4 * q + 1] = w4.y; wn[4 * q + 2] = w4.z; wn[4 * q + 3] = w4.w;
        }
    }
    if (half_rot) {
        // rotary table of the tile: ROWS x 32 pairs, pair i turns by axis i % 3
#pragma unroll
        for (int j = 0; j < ROWS * 32 / NT; j++) {
            const int idx = tid + NT * j, row = idx >> 5, i = idx & 31;
            const int tt = trow[row];
            if (tt >= 0) {
                const float ang = (float)p.pos3[3 * (size_t)tt + i % 3] * p.inv_freq[i];
                float sn, cn;
                rope_sincos(ang, &sn, &cn);
                csl[row][i] = make_float2(cn, sn);
                if (p.rope_cs && kh == 0) *(float2 *)(p.rope_cs + (size_t)tt * 2 * half_rot + 2 * i) = make_float2(cn, sn);
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
    if (t >= 0) {
        uint16_t *dst = p.k_plane + ((size_t)kh * p.kvT + r0 + rr) * HD + 16 * k;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const float *xs = x + 8 * h;
            u32x4 ko = {pack_bf16(xs[0], xs[1]), pack_bf16(xs[2], xs[3]), pack_bf16(xs[4], xs[5]), pack_bf16(xs[6], xs[7])};
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
// Vision prologue (metal/clef.metal:1616-1656, vis_qkv_rope): qkv [P][3E] (+ bias) ->
// Q plane [heads][P][VHDK] (row = patch), K plane [heads][kvT][VHDK] (row tok_kv[patch]),
// V^T [heads][VHD][kvT]. Q and K take the 2-D rotary: pair (i, i + hd/2); the first hd/4
// pairs turn by the patch's grid row, the rest by its column; pos2 [P][2] holds each patch's
// (row, column). Grid (P / 16, heads), 256 threads: 16 lanes per patch, lane j owns the rotary
// pairs j, j + 16 and (j < 4) j + 32.
// ------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void vis_prep_kernel(VisPrepParams p) {
    constexpr int HD = 72, HDK = 80, ROWS = 16, HALF = HD / 2, QUART = HD / 4, VS = HD + 8;
    __shared__ __attribute__((aligned(16))) uint16_t vr[ROWS * VS];
    __shared__ int krows[ROWS];
    const int tid = threadIdx.x, rr = tid >> 4, j = tid & 15;
    const int t0 = blockIdx.x * ROWS, h = blockIdx.y;
    const int E = p.heads * HD;
    const int tok = t0 + rr;
    if (tid < ROWS) krows[tid] = t0 + tid < p.P ? p.tok_kv[t0 + tid] : -1;
    __syncthreads();
    const int krow = krows[rr];
    if (tok < p.P) {
        const uint16_t *row = p.qkv + (size_t)tok * 3 * E;
        uint16_t *qd = p.q_plane + ((size_t)h * p.P + tok) * HDK;
        uint16_t *kd = krow >= 0 ? p.k_plane + ((size_t)h * p.kvT + krow) * HDK : nullptr;
#pragma unroll
        for (int k = 0; k < 3; k++) {
            const int i = j + 16 * k;
            if (i >= HALF) break;
            const float ang = (float)p.pos2[2 * tok + (i < QUART ? 0 : 1)] * p.inv_freq[i < QUART ? i : i - QUART];
            float sn, cs;
            rope_sincos(ang, &sn, &cs);
#pragma unroll
            for (int part = 0; part < 2; part++) {
                const int base = part * E + h * HD;
                float x0 = bf2f(row[base + i]), x1 = bf2f(row[base + i + HALF]);
                if (p.bias) { x0 += p.bias[base + i]; x1 += p.bias[base + i + HALF]; }
                const float y0 = x0 * cs - x1 * sn, y1 = x1 * cs + x0 * sn;
                uint16_t *dst = part == 0 ? qd : kd;
                if (dst) {
                    dst[i] = f2bf(y0);
                    dst[i + HALF] = f2bf(y1);
                }
            }
            const int vb = 2 * E + h * HD;
            float v0 = bf2f(row[vb + i]), v1 = bf2f(row[vb + i + HALF]);
            if (p.bias) { v0 += p.bias[vb + i]; v1 += p.bias[vb + i + HALF]; }
            vr[rr * VS + i] = f2bf(v0);
            vr[rr * VS + i + HALF] = f2bf(v1);
        }
        if (j < HDK - HD) {   // zero the contraction padding dims of Q and K
            qd[HD + j] = 0;
            if (kd) kd[HD + j] = 0;
        }
    }
    __syncthreads();
    const int e = tid & 15, ke = krows[e];
    for (int d = tid >> 4; d < HD; d += 16)
        if (ke >= 0) p.vt_plane[((size_t)h * HD + d) * p.kvT + ke] = vr[e * VS + d];
}

}  // namespace clef_hip
