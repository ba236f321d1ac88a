// MFMA ceiling of the attention kernels' operand stream on this device: v_mfma_f32_16x16x32_bf16
// fed by one ds_read_b128 A operand per product (as the text kernel's S and P.V loops are), 8
// waves per CU, 4 accumulators per wave, LDS reads 6 ahead. With random bf16 operands the part
// draws more power than with a constant bit pattern and holds a lower shader clock, so the
// random-operand rate is what the matrix cores sustain on attention data. A measurement utility
// with no reference counterpart, built into its own library (libclef_hip_bench.so, used by
// bench.py), apart from the engine-facing one.
//
// bool clef_hip_mfma_ceiling(int random, int iters, void *scratch, size_t scratch_bytes,
//                            double *tflops, double *ghz, char *err, size_t errlen);
// Runs on the default stream and waits for it; scratch: device memory of at least
// CUs * (2048 + 16) bytes; writes the sustained TF/s and the shader clock it held (cycle counter
// against the 100 MHz wall clock). Returns false with "hip: ..." in err on failure.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <utility>


namespace {
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;

template <int OFF>
__device__ __forceinline__ bf16x8 rd(unsigned a) {
    bf16x8 r;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(a), "i"(OFF) : "memory");
    return r;
}
template <int N>
__device__ __forceinline__ void wt(bf16x8 &r) {
    asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(r) : "i"(N));
}
template <typename F, int... I>
__device__ __forceinline__ void sfor_(F &&f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void sfor(F &&f) {
    sfor_(f, std::make_integer_sequence<int, N>{});
}
__device__ __forceinline__ unsigned mix(unsigned x) {
    x ^= x >> 16; x *= 0x7feb352du; x ^= x >> 15; x *= 0x846ca68bu; x ^= x >> 16;
    return x;
}
// bf16 in [-2, 2): random, or a constant pattern
__device__ __forceinline__ __bf16 operand(unsigned i, int random) {
    return random ? (__bf16)(((int)(mix(i) & 0xffffu) - 32768) / 16384.f) : (__bf16)(1.0f + (float)(i & 7) / 8.f);
}

constexpr int kDepth = 6, kAcc = 4, kSteps = 16;
__global__ __launch_bounds__(512) void mfma_ceiling_kernel(float *sink, unsigned long long *clk, int iters, int random) {
    __shared__ __attribute__((aligned(16))) __bf16 lds[32768];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int i = threadIdx.x; i < 32768; i += blockDim.x) lds[i] = operand(i + 77u * blockIdx.x, random);
    bf16x8 b;
    for (int j = 0; j < 8; j++) b[j] = operand(1000003u + lane * 8 + j, random);
    __syncthreads();
    const unsigned long long c0 = __builtin_readcyclecounter(), w0 = __builtin_amdgcn_s_memrealtime();
    const unsigned base = (unsigned)(uintptr_t)(const __attribute__((address_space(3))) __bf16 *)lds + lane * 16 + (wave & 3) * 1024;
    f32x4 acc[kAcc];
    for (int a = 0; a < kAcc; a++) acc[a] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int it = 0; it < iters; it++) {
        bf16x8 ring[kDepth];
        sfor<kDepth>([&](auto I) { constexpr int i = decltype(I)::value; ring[i] = rd<i * 4096>(base); });
        sfor<kSteps>([&](auto I) {
            constexpr int i = decltype(I)::value;
            constexpr int ahead = (kSteps - 1 - i) < (kDepth - 1) ? (kSteps - 1 - i) : (kDepth - 1);
            bf16x8 a = ring[i % kDepth];
            wt<ahead>(a);
            acc[i % kAcc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[i % kAcc], 0, 0, 0);
            if constexpr (i + kDepth < kSteps) ring[i % kDepth] = rd<((i + kDepth) % 16) * 4096>(base);
        });
    }
    float s = 0.f;
    for (int a = 0; a < kAcc; a++) s += acc[a][0] + acc[a][1] + acc[a][2] + acc[a][3];
    sink[blockIdx.x * blockDim.x + threadIdx.x] = s;
    if (threadIdx.x == 0) {
        clk[2 * blockIdx.x] = __builtin_readcyclecounter() - c0;
        clk[2 * blockIdx.x + 1] = __builtin_amdgcn_s_memrealtime() - w0;
    }
}
}  // namespace

extern "C" bool clef_hip_mfma_ceiling(int random, int iters, void *scratch, size_t scratch_bytes,
                                      double *tflops, double *ghz, char *err, size_t errlen) {
    int dev = 0, cus = 0;
    auto fail = [&](const char *m) {
        if (err && errlen) snprintf(err, errlen, "hip: %s", m);
        return false;
    };
    if (!tflops || !ghz || iters <= 0) return fail("bad mfma ceiling arguments");
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        return fail("no device");
    const size_t need = (size_t)cus * 512 * sizeof(float) + (size_t)cus * 2 * sizeof(unsigned long long);
    if (!scratch || scratch_bytes < need) {
        if (err && errlen) snprintf(err, errlen, "hip: mfma ceiling needs %zu bytes of scratch", need);
        return false;
    }
    float *sink = (float *)scratch;
    unsigned long long *clk = (unsigned long long *)((char *)scratch + (size_t)cus * 512 * sizeof(float));
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return fail("event create failed");
    hipLaunchKernelGGL(mfma_ceiling_kernel, dim3(cus), dim3(512), 0, 0, sink, clk, 20, random);   // warm-up
    hipEventRecord(e0, 0);
    hipLaunchKernelGGL(mfma_ceiling_kernel, dim3(cus), dim3(512), 0, 0, sink, clk, iters, random);
    hipEventRecord(e1, 0);
    bool ok = hipEventSynchronize(e1) == hipSuccess && hipGetLastError() == hipSuccess;
    float ms = 0.f;
    ok = ok && hipEventElapsedTime(&ms, e0, e1) == hipSuccess && ms > 0.f;
    unsigned long long c[2] = {0, 0};
    ok = ok && hipMemcpy(c, clk, sizeof(c), hipMemcpyDeviceToHost) == hipSuccess;
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (!ok) return fail("mfma ceiling launch failed");
    const double flops = 16.0 * 16 * 32 * 2 * kSteps * (double)iters * 8 * cus;
    *tflops = flops / (ms * 1e-3) / 1e12;
    *ghz = c[1] ? (double)c[0] / ((double)c[1] * 10.0) : 0.0;   // s_memrealtime runs at 100 MHz
    return true;
}
