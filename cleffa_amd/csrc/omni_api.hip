// C ABI of the Omni decoder attention (hd 128, FP32): argument checks, the block list and the
// two launches. Declarations and layouts are documented in include/clef_hip_attn.h.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <array>
#include <vector>

#include "clef_hip_attn.h"
#include "omni_attn.h"

using namespace clef_hip;

namespace {

bool fail(char *err, size_t errlen, const char *fmt, ...) {
    if (err && errlen) {
        int n = snprintf(err, errlen, "hip: ");
        if (n < 0) n = 0;
        if ((size_t)n < errlen) {
            va_list ap;
            va_start(ap, fmt);
            vsnprintf(err + n, errlen - (size_t)n, fmt, ap);
            va_end(ap);
        }
    }
    return false;
}

bool aligned16(const void *p) { return p && ((uintptr_t)p & 15u) == 0; }

bool heads_ok(int nh, int nkv) {
    if (nh <= 0 || nkv <= 0 || nh % nkv) return false;
    const int w = nh / nkv;
    return w == 1 || w == 2 || w == 4 || w == 8;   // one wave per q head of the group
}

}  // namespace

extern "C" {

void clef_hip_omni_rope_table(float theta, float *freq) {
    for (int j = 0; j < 192; j++) freq[j] = 0.f;
    for (int j = 0; j < 64; j++) {
        freq[j] = 1.0f / powf(theta, (float)(2 * j) / 128.0f);
        const double f = pow((double)theta, -(double)(2 * j) / 128.0);
        freq[64 + j] = (float)f;
        freq[128 + j] = (float)(f - (double)freq[64 + j]);
    }
}

bool clef_hip_omni_prep(const clef_hip_omni_prep_args *a, void *stream, char *err, size_t errlen) {
    if (!a) return fail(err, errlen, "null Omni prep arguments");
    if (!heads_ok(a->nh, a->nkv)) return fail(err, errlen, "bad Omni head counts nh=%d nkv=%d", a->nh, a->nkv);
    if (a->T < 0) return fail(err, errlen, "negative T");
    if (a->kvT < a->T + CLEF_HIP_OMNI_SLACK) return fail(err, errlen, "kvT %d must be >= T + %d", a->kvT, CLEF_HIP_OMNI_SLACK);
    if ((long)a->kvT * a->nkv * 128 >= (1L << 40)) return fail(err, errlen, "planes too large");
    if (!aligned16(a->qkv) || !aligned16(a->q_norm) || !aligned16(a->k_norm) || !a->pos3 || !a->freq)
        return fail(err, errlen, "qkv, norm weights, pos3 and freq must be device pointers (16-byte aligned)");
    if (!aligned16(a->q_plane) || !aligned16(a->k_plane) || !aligned16(a->v_plane) || !a->status)
        return fail(err, errlen, "Q / K / V planes (16-byte aligned) and status are required");
    omni::PrepParams p;
    p.qkv = a->qkv; p.q_norm = a->q_norm; p.k_norm = a->k_norm; p.pos3 = a->pos3; p.freq = a->freq;
    p.q_plane = a->q_plane; p.k_plane = a->k_plane; p.v_plane = a->v_plane; p.status = a->status;
    p.nh = a->nh; p.nkv = a->nkv; p.T = a->T; p.kvT = a->kvT; p.rope_exact = a->rope_exact ? 1 : 0;
    p.eps = a->eps;
    const long items = (long)(a->T + CLEF_HIP_OMNI_SLACK) * (a->nh + a->nkv);
    const long blocks = (items + 7) / 8;
    if (blocks > 0x7fffffffL) return fail(err, errlen, "grid too large");
    hipLaunchKernelGGL(omni::omni_prep_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(err, errlen, "omni_prep launch failed: %s", hipGetErrorString(e));
    return true;
}

int clef_hip_omni_plan_max_blocks(int n_seq, int T) {
    if (n_seq < 0 || T < 0) return 0;
    return T / CLEF_HIP_OMNI_BLOCK_Q + n_seq + 1;
}

bool clef_hip_omni_plan(const int32_t *cu, int n_seq, int32_t *blocks, int max_blocks, int *n_blk,
                        char *err, size_t errlen) {
    if (!cu || n_seq < 0 || !n_blk) return fail(err, errlen, "bad Omni plan arguments");
    if (cu[0] != 0) return fail(err, errlen, "cu_seqlens must start at 0");
    std::vector<std::array<int32_t, 8>> ents;
    for (int r = 0; r < n_seq; r++) {
        const int n = cu[r + 1] - cu[r];
        if (n < 0) return fail(err, errlen, "cu_seqlens decreases at record %d", r);
        for (int i0 = 0; i0 < n; i0 += CLEF_HIP_OMNI_BLOCK_Q) {
            const int nq = std::min(CLEF_HIP_OMNI_BLOCK_Q, n - i0);
            ents.push_back({cu[r] + i0, nq, i0, cu[r], i0 + nq, 0, r, 0});
        }
    }
    if ((int)ents.size() > max_blocks) return fail(err, errlen, "plan needs %zu blocks, room for %d", ents.size(), max_blocks);
    if (!blocks && !ents.empty()) return fail(err, errlen, "missing block array");
    std::stable_sort(ents.begin(), ents.end(), [](const std::array<int32_t, 8> &x, const std::array<int32_t, 8> &y) { return x[4] > y[4]; });
    for (size_t i = 0; i < ents.size(); i++) memcpy(blocks + 8 * i, ents[i].data(), 8 * sizeof(int32_t));
    *n_blk = (int)ents.size();
    return true;
}

bool clef_hip_omni_attention(const clef_hip_omni_attn_args *a, void *stream, char *err, size_t errlen) {
    if (!a) return fail(err, errlen, "null Omni attention arguments");
    if (!heads_ok(a->nh, a->nkv)) return fail(err, errlen, "bad Omni head counts nh=%d nkv=%d", a->nh, a->nkv);
    if (a->T < 0 || a->n_blk < 0) return fail(err, errlen, "negative sizes");
    if (a->kvT < a->T + CLEF_HIP_OMNI_SLACK) return fail(err, errlen, "kvT %d must be >= T + %d", a->kvT, CLEF_HIP_OMNI_SLACK);
    if (!(a->scale > 0.f)) return fail(err, errlen, "bad scale");
    if (a->n_blk == 0) return true;
    if (!a->blocks) return fail(err, errlen, "missing block list");
    if (!aligned16(a->q_plane) || !aligned16(a->k_plane) || !aligned16(a->v_plane) || !aligned16(a->out))
        return fail(err, errlen, "planes and out must be 16-byte aligned device pointers");
    omni::AttnParams p;
    p.q_plane = a->q_plane; p.k_plane = a->k_plane; p.v_plane = a->v_plane; p.blocks = a->blocks;
    p.out = a->out; p.nh = a->nh; p.nkv = a->nkv; p.T = a->T; p.kvT = a->kvT; p.n_blk = a->n_blk;
    p.scale = a->scale;
    const long grid = (long)a->n_blk * a->nkv;
    if (grid > 0x7fffffffL) return fail(err, errlen, "grid too large");
    const int w = a->nh / a->nkv;
    const dim3 g((unsigned)grid), b(64 * w);
    hipStream_t s = (hipStream_t)stream;
    switch (w) {
        case 1: hipLaunchKernelGGL(omni::omni_attn_kernel<1>, g, b, 0, s, p); break;
        case 2: hipLaunchKernelGGL(omni::omni_attn_kernel<2>, g, b, 0, s, p); break;
        case 4: hipLaunchKernelGGL(omni::omni_attn_kernel<4>, g, b, 0, s, p); break;
        default: hipLaunchKernelGGL(omni::omni_attn_kernel<8>, g, b, 0, s, p); break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(err, errlen, "omni_attention launch failed: %s", hipGetErrorString(e));
    return true;
}

}  // extern "C"
