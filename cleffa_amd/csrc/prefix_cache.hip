// Prefix-cache entry planes: the capacity policy and the growth copy of one layer's K and V^T
// planes (clef_metal.m:762-805, prefix_reserve). The copy is HBM-bound: it reads the kept rows
// once and writes every row of the new planes once, in 16-byte chunks.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "clef_hip_attn.h"

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

struct CopyParams {
    const u32x4 *k_src, *vt_src;
    u32x4 *k_dst, *vt_dst;
    long k_chunks;        // 16-byte chunks of the K plane, nkv * dst_cap * hd / 8
    long total;           // k_chunks + the V^T plane's chunks
    int row8;             // chunks per K row, hd / 8
    int src_cap, dst_cap, keep;
};

constexpr int kThreads = 256, kPerThread = 4;

// Thread t of block b handles chunks (b * kPerThread + j) * kThreads + t: each of the four
// groups is a coalesced 4 KB run, and all four loads are issued before the stores.
__global__ __launch_bounds__(kThreads) void prefix_copy_kernel(CopyParams p) {
    u32x4 v[kPerThread];
    long idx[kPerThread];
#pragma unroll
    for (int j = 0; j < kPerThread; j++) {
        const long i = ((long)blockIdx.x * kPerThread + j) * kThreads + threadIdx.x;
        idx[j] = i;
        v[j] = u32x4{0u, 0u, 0u, 0u};
        if (i >= p.total) continue;
        if (i < p.k_chunks) {   // K: [nkv][dst_cap][hd]
            const long per_head = (long)p.dst_cap * p.row8;
            const long h = i / per_head, rem = i - h * per_head;
            const long row = rem / p.row8;
            if (row < p.keep) v[j] = p.k_src[(h * p.src_cap + row) * p.row8 + (rem - row * p.row8)];
        } else {                // V^T: [nkv * hd][dst_cap], keep columns of each row
            const long e = i - p.k_chunks, per_row = p.dst_cap / 8;
            const long r = e / per_row;
            const int col = (int)(e - r * per_row) * 8;
            if (col < p.keep) {
                v[j] = p.vt_src[(r * p.src_cap + col) / 8];
                const int valid = p.keep - col;   // the chunk holding column keep - 1 keeps part
                if (valid < 8) {
#pragma unroll
                    for (int w = 0; w < 4; w++) {
                        const unsigned keepm = (2 * w + 1 < valid) ? 0xffffffffu : (2 * w < valid ? 0xffffu : 0u);
                        v[j][w] &= keepm;
                    }
                }
            }
        }
    }
#pragma unroll
    for (int j = 0; j < kPerThread; j++) {
        const long i = idx[j];
        if (i >= p.total) continue;
        u32x4 *dst = i < p.k_chunks ? p.k_dst + i : p.vt_dst + (i - p.k_chunks);
        __builtin_nontemporal_store(v[j], dst);
    }
}

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

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

extern "C" {

int clef_hip_prefix_capacity(int rows, int cur_cap, int hd) {
    if (rows < 0 || cur_cap < 0 || hd <= 0) return -1;
    if (rows <= cur_cap) return cur_cap;
    long want = rows;
    const long grow = (long)cur_cap + cur_cap / 4;
    if (want < grow) want = grow;
    const long cap = (want + 1023) / 1024 * 1024;
    if (cap * hd * 2 >= (1L << 32)) return -1;
    return (int)cap;
}

size_t clef_hip_prefix_plane_bytes(int nkv, int hd, int cap) {
    if (nkv <= 0 || hd <= 0 || cap < 0) return 0;
    return (size_t)nkv * (size_t)cap * (size_t)hd * 2;
}

bool clef_hip_prefix_copy(const uint16_t *k_src, const uint16_t *vt_src, int src_cap,
                          uint16_t *k_dst, uint16_t *vt_dst, int dst_cap, int nkv, int hd, int keep,
                          void *stream, char *err, size_t errlen) {
    if (nkv <= 0 || hd <= 0 || hd % 8) return fail(err, errlen, "bad plane shape nkv=%d hd=%d", nkv, hd);
    if (src_cap < 0 || dst_cap <= 0 || src_cap % 8 || dst_cap % 8)
        return fail(err, errlen, "capacities %d -> %d must be multiples of 8", src_cap, dst_cap);
    if (keep < 0 || keep > src_cap || keep > dst_cap)
        return fail(err, errlen, "keep %d exceeds a capacity (%d -> %d)", keep, src_cap, dst_cap);
    if ((long)dst_cap * hd * 2 >= (1L << 32)) return fail(err, errlen, "capacity %d too large", dst_cap);
    if (!k_dst || !vt_dst || !aligned16(k_dst) || !aligned16(vt_dst))
        return fail(err, errlen, "destination planes must be 16-byte aligned device pointers");
    if (keep > 0 && (!k_src || !vt_src || !aligned16(k_src) || !aligned16(vt_src)))
        return fail(err, errlen, "source planes must be 16-byte aligned device pointers");
    CopyParams p;
    p.k_src = (const u32x4 *)k_src; p.vt_src = (const u32x4 *)vt_src;
    p.k_dst = (u32x4 *)k_dst; p.vt_dst = (u32x4 *)vt_dst;
    p.row8 = hd / 8;
    p.k_chunks = (long)nkv * dst_cap * p.row8;
    p.total = 2 * p.k_chunks;   // the V^T plane has as many chunks as the K plane
    p.src_cap = src_cap; p.dst_cap = dst_cap; p.keep = keep;
    const long per_block = (long)kThreads * kPerThread;
    const long blocks = (p.total + per_block - 1) / per_block;
    if (blocks > 0x7fffffffL) return fail(err, errlen, "planes too large for one launch");
    hipLaunchKernelGGL(prefix_copy_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, (hipStream_t)stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(err, errlen, "prefix_copy launch failed: %s", hipGetErrorString(e));
    return true;
}

}  // extern "C"
