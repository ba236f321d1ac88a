// The GEMMs either side of the attention path (clef_metal.m:463-499, clef_metal_gemm): the fused
// QKV projection that produces the path's qkv rows and the o_proj that accumulates its output
// into the f32 residual stream. Both are plain Y (+)= X . W^T products with bf16 weights and
// f32 accumulation, so they run on hipBLASLt; the algorithm for each shape is chosen once and
// cached. Device memory is the caller's: the optional workspace is passed in.
// Choosing the algorithm: for a product that overwrites Y, the first call times hipBLASLt's
// first kTune candidates on the caller's own operands and stream (each result is overwritten by
// the next, and the call ends with the chosen one), and keeps the fastest. hipBLASLt's first
// candidate was 30% slower than the best for the QKV shape. An accumulating product cannot be
// run more than once, and a stream under graph capture cannot be timed: those take the first
// candidate. A choice made under capture is replaced by a timed one at the next uncaptured call.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <tuple>

#include "clef_hip_attn.h"

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

struct Plan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    hipblasLtMatmulAlgo_t algo;
    size_t ws = 0;
    bool final = false;   // timed, or nothing to time (an accumulating product)
};

void destroy(Plan *p) {
    if (p->a) hipblasLtMatrixLayoutDestroy(p->a);
    if (p->b) hipblasLtMatrixLayoutDestroy(p->b);
    if (p->c) hipblasLtMatrixLayoutDestroy(p->c);
    if (p->desc) hipblasLtMatmulDescDestroy(p->desc);
    *p = Plan();
}

using Key = std::tuple<int, int, int, int, int, int, size_t>;   // device, T, N, K, y_type, acc, ws

std::mutex mu;
std::map<int, hipblasLtHandle_t> handles;
std::map<Key, Plan> plans;

// Candidates timed on a shape's first call, and runs per candidate (after one warm-up): the one
// with the shortest median run is kept.
constexpr int kTune = 16;
constexpr int kTuneRuns = 5;
bool tune(hipblasLtHandle_t h, Plan *p, const hipblasLtMatmulHeuristicResult_t *res, int found, const uint16_t *X,
          const uint16_t *W, void *Y, void *workspace, size_t ws_bytes, hipStream_t stream, char *err, size_t errlen) {
    hipEvent_t ev[kTuneRuns + 1];
    for (int i = 0; i <= kTuneRuns; i++)
        if (hipEventCreate(&ev[i]) != hipSuccess) {
            while (i-- > 0) (void)hipEventDestroy(ev[i]);
            return fail(err, errlen, "hipEventCreate failed");
        }
    const float alpha = 1.f, beta = 0.f;
    float best = 0.f;
    int best_i = -1;
    for (int i = 0; i < found; i++) {
        if (res[i].workspaceSize > ws_bytes) continue;
        auto run = [&]() {
            return hipblasLtMatmul(h, p->desc, &alpha, W, p->a, X, p->b, &beta, Y, p->c, Y, p->c, &res[i].algo, workspace,
                                   res[i].workspaceSize, stream) == HIPBLAS_STATUS_SUCCESS;
        };
        if (!run()) continue;
        bool ok = hipEventRecord(ev[0], stream) == hipSuccess;
        for (int r = 0; r < kTuneRuns && ok; r++) ok = run() && hipEventRecord(ev[r + 1], stream) == hipSuccess;
        if (!ok || hipEventSynchronize(ev[kTuneRuns]) != hipSuccess) {
            (void)hipGetLastError();
            continue;
        }
        float t[kTuneRuns];
        for (int r = 0; r < kTuneRuns && ok; r++) ok = hipEventElapsedTime(&t[r], ev[r], ev[r + 1]) == hipSuccess;
        if (!ok) continue;
        for (int a = 1; a < kTuneRuns; a++)   // insertion sort, for the median
            for (int b = a; b > 0 && t[b] < t[b - 1]; b--) std::swap(t[b], t[b - 1]);
        const float med = t[kTuneRuns / 2];
        if (best_i < 0 || med < best) {
            best = med;
            best_i = i;
        }
    }
    for (int i = 0; i <= kTuneRuns; i++) (void)hipEventDestroy(ev[i]);
    if (best_i < 0) return fail(err, errlen, "no hipBLASLt candidate ran");
    p->algo = res[best_i].algo;
    p->ws = res[best_i].workspaceSize;
    return true;
}

// Row-major Y[T][N] = X[T][K] . W[N][K]^T is, column-major, Y^T (N x T) = W^T' (N x K) . X^T (K x T)
// with W read as a K x N column-major matrix, transposed (A), and X as K x T, not transposed (B).
// `timed`: the operands may be used to time the candidates (see the header of this file).
bool make_plan(hipblasLtHandle_t h, int T, int N, int K, int y_type, size_t ws, bool timed, const uint16_t *X,
               const uint16_t *W, void *Y, void *workspace, hipStream_t stream, Plan *p, char *err, size_t errlen) {
    const hipDataType yt = y_type == CLEF_HIP_GEMM_Y_BF16 ? HIP_R_16BF : HIP_R_32F;
    if (hipblasLtMatmulDescCreate(&p->desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS)
        return fail(err, errlen, "hipblasLtMatmulDescCreate failed");
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta));
    hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb));
    if (hipblasLtMatrixLayoutCreate(&p->a, HIP_R_16BF, K, N, K) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&p->b, HIP_R_16BF, K, T, K) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&p->c, yt, N, T, N) != HIPBLAS_STATUS_SUCCESS)
        return fail(err, errlen, "hipblasLtMatrixLayoutCreate failed");
    hipblasLtMatmulPreference_t pref;
    if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return fail(err, errlen, "preference create failed");
    const uint64_t wsb = ws;
    hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb, sizeof(wsb));
    hipblasLtMatmulHeuristicResult_t res[kTune];
    int found = 0;
    const hipblasStatus_t st = hipblasLtMatmulAlgoGetHeuristic(h, p->desc, p->a, p->b, p->c, p->c, pref, timed ? kTune : 1, res, &found);
    hipblasLtMatmulPreferenceDestroy(pref);
    if (st != HIPBLAS_STATUS_SUCCESS || found < 1)
        return fail(err, errlen, "no hipBLASLt algorithm for T=%d N=%d K=%d", T, N, K);
    if (timed && found > 1) return tune(h, p, res, found, X, W, Y, workspace, ws, stream, err, errlen);
    p->algo = res[0].algo;
    p->ws = res[0].workspaceSize;
    return true;
}

}  // namespace

extern "C" {

bool clef_hip_gemm(int T, int N, int K, const uint16_t *X, const uint16_t *W, void *Y, int y_type, int acc,
                   void *workspace, size_t ws_bytes, void *stream, char *err, size_t errlen) {
    if (T < 0 || N <= 0 || K <= 0) return fail(err, errlen, "bad GEMM shape T=%d N=%d K=%d", T, N, K);
    if (y_type != CLEF_HIP_GEMM_Y_F32 && y_type != CLEF_HIP_GEMM_Y_BF16) return fail(err, errlen, "bad y_type %d", y_type);
    if (acc && y_type != CLEF_HIP_GEMM_Y_F32) return fail(err, errlen, "accumulation needs an f32 Y");
    if (!X || !W || !Y) return fail(err, errlen, "null GEMM operand");
    if (ws_bytes && !workspace) return fail(err, errlen, "workspace size without a workspace");
    if (T == 0) return true;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(err, errlen, "hipGetDevice failed");
    Plan p;
    {
        std::lock_guard<std::mutex> lock(mu);
        auto hi = handles.find(dev);
        if (hi == handles.end()) {
            hipblasLtHandle_t h;
            if (hipblasLtCreate(&h) != HIPBLAS_STATUS_SUCCESS) return fail(err, errlen, "hipblasLtCreate failed");
            hi = handles.emplace(dev, h).first;
        }
        const Key key{dev, T, N, K, y_type, acc ? 1 : 0, ws_bytes};
        auto pi = plans.find(key);
        if (pi == plans.end() || !pi->second.final) {
            hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
            if (hipStreamIsCapturing((hipStream_t)stream, &cap) != hipSuccess)
                return fail(err, errlen, "hipStreamIsCapturing failed");
            const bool captured = cap != hipStreamCaptureStatusNone;
            if (pi == plans.end() || !captured) {   // a new plan, or the untimed one replaced
                Plan np;
                if (!make_plan(hi->second, T, N, K, y_type, ws_bytes, !acc && !captured, X, W, Y, workspace,
                               (hipStream_t)stream, &np, err, errlen)) {
                    destroy(&np);
                    return false;
                }
                np.final = acc || !captured;
                if (pi != plans.end()) {
                    destroy(&pi->second);
                    pi->second = np;
                } else {
                    pi = plans.emplace(key, np).first;
                }
            }
        }
        p = pi->second;
        const float alpha = 1.f, beta = acc ? 1.f : 0.f;
        const hipblasStatus_t st = hipblasLtMatmul(hi->second, p.desc, &alpha, W, p.a, X, p.b, &beta, Y, p.c, Y, p.c,
                                                   &p.algo, workspace, p.ws, (hipStream_t)stream);
        if (st != HIPBLAS_STATUS_SUCCESS) return fail(err, errlen, "hipblasLtMatmul failed (%d)", (int)st);
    }
    return true;
}

}  // extern "C"
