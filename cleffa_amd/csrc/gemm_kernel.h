// The QKV projection on CDNA4 with the text path's K/V prologue in its epilogue: Y = X . W^T
// (X [T][K] bf16 activations, W [N][K] bf16 weights, both K-contiguous as the model file stores
// them; f32 accumulation), the role of clef_metal_gemm (clef_metal.m:463-499) at its QKV call
// (clef_metal.m:1326).
//
// Tiles of BM (256) rows x 256 columns, one per workgroup of 8 waves (2 per SIMD). A 256-column
// tile of the QKV output is exactly one head's slice (a query or gate half of a q head, one K
// head or one V head), so the epilogue of a K tile holds whole key rows: it runs the RMSNorm,
// rotary and f16 split of the K/V prologue on them and writes the K plane rows; a V tile writes
// its V^T plane entries. Every output tile also leaves its bf16 rows in the qkv buffer.
//   k loop:   BK-deep K slices of X and W stream global -> LDS with global_load_lds (16 bytes a
//             lane), STAGES deep, into unpadded rows whose 16-byte chunks are XOR-swizzled, so
//             the ds_read_b128 operand reads of 16 consecutive rows hit distinct banks. The
//             L2 -> LDS stream is the bound at this size: a 256 x 256 tile moves 1 KB per
//             128 KFLOP of products (a 128-row tile moved 1.5 times that and ran fill-bound).
//   products: v_mfma_f32_16x16x32_bf16, each wave a WM x WN block of the tile: A = 16 columns
//             of W (16 output columns), B = 16 rows of X (16 output rows), so a lane's four
//             accumulators are four consecutive columns of one output row.
//   epilogue: accumulators rounded to bf16 into an LDS copy of the tile, then coalesced row
//             stores; K and V tiles take the prologue from that copy, so their planes hold
//             bitwise what text_prep_direct_kernel makes of the same bf16 rows (both run kv_rows.h).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

#include "attn_kernels.h"
#include "kv_rows.h"

namespace clef_hip {
namespace gemm {

typedef __attribute__((ext_vector_type(4))) float f32x4;

constexpr int BN = 256, HD = 256;
constexpr int CS = 2 * BN + 16;                      // C-tile row stride in LDS (bytes)
constexpr int KALIGN = 64;                           // K must be a multiple of this

struct Params {
    const uint16_t *X, *W;
    uint16_t *Y;              // [T][ldy] bf16
    int T, N, K, ldy;
    int m_tiles, n_tiles, n_per_xcd;   // n_per_xcd: the most N tiles any XCD owns
    int kv;                   // the fused K/V prologue: the QKV layout of the text path
    KvRows r;
};

__device__ __forceinline__ unsigned lds_u32(const void *p) {
    return (unsigned)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
template <int OFF>
__device__ __forceinline__ bf16x8 rd16(unsigned addr) {
    bf16x8 r;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF) : "memory");
    return r;
}
template <typename F, int... I>
__device__ __forceinline__ void static_for_g_impl(F &&f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for_g(F &&f) {
    static_for_g_impl(f, std::make_integer_sequence<int, N>{});
}

// Output tile of workgroup b: XCD x (workgroup b runs on XCD b % 8, each with its own L2) owns
// the N tiles x, x + 8, x + 16, ... and walks them row of tiles by row of tiles, so the tiles
// running together on an XCD share X rows and W columns in its L2. The stride spreads the K and
// V head tiles (the last 2 nkv N tiles), whose epilogues carry the K/V prologue, over the XCDs.
__device__ __forceinline__ bool tile_of(const Params &p, int b, int *tm, int *tn) {
    const int x = b & 7, j = b >> 3;
    const int cnt = (p.n_tiles - x + 7) >> 3;
    if (cnt <= 0 || j >= cnt * p.m_tiles) return false;
    *tm = j / cnt;
    *tn = x + 8 * (j % cnt);
    return true;
}

// Kernel configuration: WM x WN output block per wave ((BM / WM) x (BN / WN) waves), K slices
// of BK (32 or 64) staged STAGES deep in LDS.
template <int BM_, int WM_, int WN_, int BK_, int STAGES_>
struct Cfg {
    static constexpr int BM = BM_, WM = WM_, WN = WN_, BK = BK_, STAGES = STAGES_;
    static constexpr int WAVES = (BM / WM) * (BN / WN), THREADS = 64 * WAVES;
    static constexpr int MT = WM / 16, NT = WN / 16, FR = MT + NT;   // 16-row / 16-column fragments
    static constexpr int KS = BK / 32;                               // 32-deep product steps per slice
    static constexpr int A_BYTES = BM * BK * 2, B_BYTES = BN * BK * 2, STAGE_BYTES = A_BYTES + B_BYTES;
    // the stages, or the C tile and the rotary table of the K rows' epilogue (kv_rows.h)
    static constexpr int EPI_BYTES = BM * CS + THREADS / 16 * 32 * 8;
    static constexpr int LDS_BYTES = STAGES * STAGE_BYTES > EPI_BYTES ? STAGES * STAGE_BYTES : EPI_BYTES;
    static constexpr int CH = BK / 8;                  // 16-byte chunks per LDS row
    static constexpr int RPI = 1024 / (2 * BK);        // rows per 1 KB fill instruction
    static constexpr int R256 = 256 / (2 * BK);        // rows per 256 bytes (one pass over the banks)
    static constexpr int A_FILLS = A_BYTES / 1024 / WAVES, B_FILLS = B_BYTES / 1024 / WAVES, FILLS = A_FILLS + B_FILLS;
    static_assert(A_BYTES / 1024 % WAVES == 0 && B_BYTES / 1024 % WAVES == 0, "fills divide over the waves");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
    static_assert(STAGES >= 2 && KALIGN % BK == 0, "pipeline depth and K alignment");
    // chunk position of k-chunk c in row r: 16 consecutive rows reading one chunk hit 16
    // distinct 16-byte bank groups
    __device__ static constexpr int swz(int r) { return (r / R256) % CH; }
};

// The operand fragments of one 32-deep k step: NT column fragments of W, then MT row fragments
// of X, read by ds_read_b128 in inline asm (the wait for them is separate, at their use).
template <int NT, int MT, int RS>
__device__ __forceinline__ void read_frags(bf16x8 (&r)[NT + MT], unsigned wk, unsigned xk) {
    static_for_g<NT>([&](auto I) { r[decltype(I)::value] = rd16<decltype(I)::value * 16 * RS>(wk); });
    static_for_g<MT>([&](auto I) { r[NT + decltype(I)::value] = rd16<decltype(I)::value * 16 * RS>(xk); });
}
// Waits until at most N LDS operations are outstanding, in one asm statement that names the
// fragments, so that no copy or use of them can be placed between their reads and the wait.
template <int N, int F>
__device__ __forceinline__ void wait_frags(bf16x8 (&r)[F]) {
    static_assert(F == 8 || F == 12, "fragment counts of the wave layouts");
    if constexpr (F == 8)
        asm volatile("s_waitcnt lgkmcnt(%8)" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5]), "+v"(r[6]), "+v"(r[7]) : "i"(N) : "memory");
    else
        asm volatile("s_waitcnt lgkmcnt(%12)" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5]), "+v"(r[6]), "+v"(r[7]), "+v"(r[8]), "+v"(r[9]), "+v"(r[10]), "+v"(r[11]) : "i"(N) : "memory");
}
// s_waitcnt vmcnt(b * FILLS) for a run-time b in [0, 4], then the workgroup barrier
template <int FILLS>
__device__ __forceinline__ void wait_fills_barrier(int b) {
    switch (b) {
        case 0: asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory"); break;
        case 1: asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"i"(FILLS) : "memory"); break;
        case 2: asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"i"(2 * FILLS) : "memory"); break;
        case 3: asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"i"(3 * FILLS) : "memory"); break;
        default: asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"i"(4 * FILLS) : "memory"); break;
    }
}

template <typename C>
__global__ __launch_bounds__(C::THREADS, 1) void qkv_gemm_kernel(Params p) {
    constexpr int MT = C::MT, NT = C::NT, FR = C::FR, FILLS = C::FILLS, A_FILLS = C::A_FILLS, B_FILLS = C::B_FILLS;
    constexpr int BM = C::BM, BK = C::BK, STAGES = C::STAGES, KS = C::KS, RS = 2 * BK;   // RS: LDS row bytes
    static_assert(FILLS * (STAGES - 2) <= 63, "vmcnt range");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[C::LDS_BYTES];
    int tm, tn;
    if (!tile_of(p, blockIdx.x, &tm, &tn)) return;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int m0 = tm * BM, n0 = tn * BN;

    // Fill offsets (bytes from the slice's first element): instruction j of a tile covers LDS
    // rows RPI j .. RPI j + RPI - 1; lane l lands in row RPI j + l / CH at chunk position l % CH,
    // which holds the row's k-chunk (l % CH) ^ swz(row).
    unsigned fo[FILLS];
#pragma unroll
    for (int f = 0; f < FILLS; f++) {
        const bool a = f < A_FILLS;
        const int j = a ? wave * A_FILLS + f : wave * B_FILLS + (f - A_FILLS);
        const int row = C::RPI * j + lane / C::CH;
        const int c = (lane % C::CH) ^ C::swz(row);
        const int grow = a ? min(m0 + row, p.T - 1) : n0 + row;
        fo[f] = ((unsigned)grow * (unsigned)p.K + (unsigned)(8 * c)) * 2u;
    }
    auto fill = [&](int slice, int stage) {
        const char *xa = (const char *)(p.X + (size_t)slice * BK), *wa = (const char *)(p.W + (size_t)slice * BK);
        uint8_t *sa = lds + stage * C::STAGE_BYTES;
#pragma unroll
        for (int f = 0; f < FILLS; f++) {
            const bool a = f < A_FILLS;
            const int j = a ? wave * A_FILLS + f : wave * B_FILLS + (f - A_FILLS);
            unsigned off = fo[f];
            asm volatile("" : "+v"(off));
            uint8_t *dst = a ? sa + 1024 * j : sa + C::A_BYTES + 1024 * j;
            __builtin_amdgcn_global_load_lds((const void *)((a ? xa : wa) + off), (lds_void *)dst, 16, 0, 0);
        }
    };
    // operand read addresses: rows (lane & 15) of the wave's blocks, k-chunk 4 ks + lane / 16 (the
    // swizzle of a fragment's rows does not depend on which 16-row fragment it is)
    constexpr int WAVES_N = BN / C::WN;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N, r16 = lane & 15, g = lane >> 4, sw = C::swz(r16);
    const unsigned base = lds_u32(lds);
    unsigned xa[KS], wa[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
        const unsigned ch = (unsigned)(((4 * ks + g) ^ sw) * 16);
        xa[ks] = base + (unsigned)((C::WM * wm + r16) * RS) + ch;
        wa[ks] = base + C::A_BYTES + (unsigned)((C::WN * wn + r16) * RS) + ch;
    }

    f32x4 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int j = 0; j < NT; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto products = [&](bf16x8 (&r)[FR]) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
                acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(r[nt], r[NT + mt], acc[mt][nt], 0, 0, 0);
    };

    // Pipeline over 32-deep steps (KS per slice). While the products of step s issue, the reads
    // of step s + 1 are in flight; they are waited for after those products have issued, so
    // every fragment set crosses the loop's back edge complete (the compiler's register moves
    // there never copy a read still in flight). Before the first step of slice q is read, a
    // barrier behind the wave's wait for slice q's fills makes the slice visible, and tells
    // every wave that the others have finished reading slice q - 1: its buffer then takes the
    // fills of slice q + STAGES - 1. Slices q + 1 .. q + STAGES - 2 stay in flight meanwhile.
    const int nk = p.K / BK, nsteps = nk * KS;
    for (int q = 0; q < STAGES - 1 && q < nk; q++) fill(q, q);
    auto enter_slice = [&](int q) {   // slice q may be read once this returns
        if constexpr (STAGES == 2) asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
        else wait_fills_barrier<FILLS>(min(STAGES - 2, nk - 1 - q));
        if (q + STAGES - 1 < nk) fill(q + STAGES - 1, (q + STAGES - 1) % STAGES);
    };
    auto step_addr = [&](int s, const unsigned *a) {
        return a[s % KS] + (unsigned)(((s / KS) % STAGES) * C::STAGE_BYTES);
    };
    bf16x8 r0[FR], r1[FR];
    enter_slice(0);
    read_frags<NT, MT, RS>(r0, step_addr(0, wa), step_addr(0, xa));
    wait_frags<0>(r0);
    // Two steps per slice (K is a multiple of 64, so nsteps is even and at least 2). The loop
    // body is branch-free apart from the slice's fill: with conditional steps inside it the
    // compiler split the accumulators' live ranges and copied them on every pass.
    static_assert(KS == 2, "two 32-deep steps per slice");
    for (int s = 0; s < nsteps - 2; s += 2) {
        read_frags<NT, MT, RS>(r1, step_addr(s + 1, wa), step_addr(s + 1, xa));
        products(r0);
        wait_frags<0>(r1);
        enter_slice(s / 2 + 1);
        read_frags<NT, MT, RS>(r0, step_addr(s + 2, wa), step_addr(s + 2, xa));
        products(r1);
        wait_frags<0>(r0);
    }
    read_frags<NT, MT, RS>(r1, step_addr(nsteps - 1, wa), step_addr(nsteps - 1, xa));
    products(r0);
    wait_frags<0>(r1);
    products(r1);

    // ---- epilogue: bf16 C tile into LDS (every wave has left the stage buffers)
    __syncthreads();
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int row = C::WM * wm + 16 * mt + r16, c = C::WN * wn + 16 * nt + 4 * g;
            const f32x4 v = acc[mt][nt];
            *(u32x2 *)(lds + row * CS + 2 * c) = u32x2{pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3])};
        }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < BM * BN * 2 / 16 / C::THREADS; i++) {
        const int id = tid + C::THREADS * i, row = id >> 5, c16 = id & 31;
        if (m0 + row < p.T)
            *(u32x4 *)(p.Y + (size_t)(m0 + row) * p.ldy + n0 + 8 * c16) = *(const u32x4 *)(lds + row * CS + 16 * c16);
    }
    if (p.kv) {
        const int kcol = 2 * p.r.nh * HD;
        float2 *table = (float2 *)(lds + BM * CS);
        if (n0 >= kcol && n0 < kcol + p.r.nkv * HD) k_rows<C::THREADS, BM>(p.r, lds, CS, m0, (n0 - kcol) / HD, table);
        else if (n0 >= kcol + p.r.nkv * HD) v_rows<C::WAVES, BM>(p.r, lds, CS, m0, (n0 - kcol - p.r.nkv * HD) / HD);
    }
}

}  // namespace gemm
}  // namespace clef_hip
