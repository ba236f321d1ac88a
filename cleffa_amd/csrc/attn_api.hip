// C ABI of the prefill attention path: argument checks, the host-side plan builder and the
// kernel launches. Declarations and layouts are documented in include/clef_hip_attn.h.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "attn_kernels.h"
#include "attn_text.h"
#include "attn_text_f32.h"
#include "attn_vis.h"
#include "gemm_kernel.h"
#include "kv_rows.h"
#include "attn_params.h"
#include "clef_hip_attn.h"

using namespace clef_hip;

// Device scratch of clef_hip_vis_attention_noalloc: the three vision planes, one copy per GPU.
static __device__ __align__(256) unsigned char scratch[CLEF_HIP_VIS_SCRATCH_BYTES];

namespace {

constexpr int kVersion = 4;
constexpr int32_t kSchedMagic = 0x53434844;   // header word of a schedule ('SCHD')
constexpr int kSchedHeader = 8;                 // {magic, n_blk, nh, n_wg, nkv, fingerprint, 0, 0}
// A 32-bit fingerprint of a block list: FNV-1a over words 0-6 of every entry (word 7 holds the
// fingerprint itself), never 0. The plan stores it in word 7 of every entry and the schedule in
// its header, so the kernel can tell whether a schedule was built for the plan it runs.
int32_t blocks_fingerprint(const int32_t *blocks, int n_blk) {
    uint32_t h = 2166136261u;
    for (int b = 0; b < n_blk; b++)
        for (int i = 0; i < CLEF_HIP_BLOCK_INTS - 1; i++) {
            const uint32_t w = (uint32_t)blocks[CLEF_HIP_BLOCK_INTS * b + i];
            for (int k = 0; k < 4; k++) h = (h ^ ((w >> (8 * k)) & 0xffu)) * 16777619u;
        }
    return (int32_t)(h | 1u);
}
constexpr int kVisHD = 72;

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

bool launch_ok(const char *what, char *err, size_t errlen) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(err, errlen, "%s launch failed: %s", what, hipGetErrorString(e));
    return true;
}

// The f16 overflow limit as the reference clamps it (clef_metal.m:237-238): (0, 65504], else 65504.
float f16_limit(float lim) { return (lim > 0.f && lim <= 65504.f) ? lim : 65504.f; }

bool rot_ok(int n_rot, int hd) {
    // the fused Q prologue is compiled for these rotary widths (Clef pins 64, clef.c:116-120)
    return (n_rot == 0 || n_rot == 64) && n_rot <= hd;
}

bool check_text(const clef_hip_attn_args *a, bool need_core, char *err, size_t errlen) {
    if (!a) return fail(err, errlen, "null attention arguments");
    if (a->hd != 256) return fail(err, errlen, "text attention supports hd 256 only (got %d)", a->hd);
    if (a->qkv_type != CLEF_HIP_QKV_BF16 && a->qkv_type != CLEF_HIP_QKV_F32)
        return fail(err, errlen, "qkv_type %d not supported: the qkv rows must be bf16 or f32", a->qkv_type);
    const bool f32 = a->qkv_type == CLEF_HIP_QKV_F32;
    if (a->nh <= 0 || a->nkv <= 0 || a->nh % a->nkv) return fail(err, errlen, "bad head counts nh=%d nkv=%d", a->nh, a->nkv);
    if (!rot_ok(a->n_rot, a->hd)) return fail(err, errlen, "unsupported n_rot %d", a->n_rot);
    if (a->T < 0 || a->n_blk < 0 || a->kv_rows < 0) return fail(err, errlen, "negative sizes");
    const long need_row = 2L * a->nh * a->hd + 2L * a->nkv * a->hd;
    if (a->row < need_row || a->row % 8) return fail(err, errlen, "qkv row %d must be >= %ld and a multiple of 8", a->row, need_row);
    if (a->kvT % 8 || a->kvT < a->kv_rows) return fail(err, errlen, "kvT %d must be a multiple of 8 and >= kv_rows %d", a->kvT, a->kv_rows);
    if (!f32 && (long)a->kvT * a->hd * 2 >= (1L << 32)) return fail(err, errlen, "kvT %d too large for 32-bit plane offsets", a->kvT);
    if (!a->qkv || !aligned16(a->qkv)) return fail(err, errlen, "qkv must be a 16-byte aligned device pointer");
    if (!aligned16(a->k_norm) || !aligned16(a->q_norm)) return fail(err, errlen, "norm weights must be 16-byte aligned");
    if (!a->k_norm != !a->q_norm) return fail(err, errlen, "q_norm and k_norm must both be set or both be NULL");
    if (a->n_rot && (!a->pos3 || !a->inv_freq)) return fail(err, errlen, "rotary needs pos3 and inv_freq");
    if (!aligned16(a->rope_cs)) return fail(err, errlen, "rope_cs must be 16-byte aligned");
    if (!a->k_plane || !aligned16(a->k_plane) || !a->vt_plane || !aligned16(a->vt_plane)) return fail(err, errlen, "K / V^T planes must be 16-byte aligned");
    if (need_core) {
        if (a->n_blk && !a->blocks) return fail(err, errlen, "missing block list");
        if (!a->out || !aligned16(a->out)) return fail(err, errlen, "out must be a 16-byte aligned device pointer");
        if (a->out_type < CLEF_HIP_OUT_BF16 || a->out_type > CLEF_HIP_OUT_F32) return fail(err, errlen, "bad out_type %d", a->out_type);
        if (!(a->scale > 0.f)) return fail(err, errlen, "bad scale");
    } else if (a->kv_rows && !a->kv_tok) {
        return fail(err, errlen, "missing kv_tok");
    }
    return true;
}

// Grid of the text kernel: one workgroup per CU looping over its items, so that the next item's
// loads overlap the current one's epilogue (measured 2-3% faster at C1, 1% at C2), or one
// workgroup per item with CLEF_HIP_TEXT_PERSISTENT=0.
bool text_persistent() {
    const char *e = getenv("CLEF_HIP_TEXT_PERSISTENT");
    return !(e && e[0] == '0');
}

long device_cus() {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    return n;
}


// ---- Library-owned vision scratch (clef_hip_vis_attention_noalloc). The array's name is a
// host-side stand-in: its device address on each GPU comes from hipGetSymbolAddress, taken once
// per device with that device current, and only that address is handed to kernels.
constexpr size_t kVisScratchBytes = CLEF_HIP_VIS_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
char *g_scratch_ptr[kMaxDevices];

// Bytes of one [heads][rows][72] bf16 plane, rounded up to 256 so the next plane stays aligned.
size_t vis_plane_bytes(int heads, int rows) {
    return ((size_t)heads * (size_t)rows * kVisHD * sizeof(uint16_t) + 255) & ~(size_t)255;
}

bool scratch_base(char **out, char *err, size_t errlen) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(err, errlen, "no device: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return fail(err, errlen, "device %d beyond the scratch table", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) return fail(err, errlen, "scratch address on device %d: %s", dev, hipGetErrorString(e));
        g_scratch_ptr[dev] = (char *)ptr;
    }
    *out = g_scratch_ptr[dev];
    return true;
}

// The vision step on the given planes (the caller's, or the library's scratch).
bool vis_run(const clef_hip_vis_args *a, uint16_t *q_plane, uint16_t *k_plane, uint16_t *vt_plane, void *stream,
             char *err, size_t errlen) {
    if (a->hd != kVisHD) return fail(err, errlen, "vision attention supports hd 72 only (got %d)", a->hd);
    if (a->P < 0 || a->heads <= 0 || a->n_blk < 0 || a->kv_rows < 0) return fail(err, errlen, "bad vision sizes");
    if (a->kvT % 8 || a->kvT < a->kv_rows) return fail(err, errlen, "kvT %d must be a multiple of 8 and >= kv_rows %d", a->kvT, a->kv_rows);
    if (!a->qkv || !a->pos2 || !a->inv_freq || !q_plane || !k_plane || !vt_plane || !a->out)
        return fail(err, errlen, "missing vision buffer");
    if (!aligned16(q_plane) || !aligned16(k_plane) || !aligned16(vt_plane) || !aligned16(a->out))
        return fail(err, errlen, "vision planes and output must be 16-byte aligned");
    if (a->out_type < CLEF_HIP_OUT_BF16 || a->out_type > CLEF_HIP_OUT_F32) return fail(err, errlen, "bad out_type %d", a->out_type);
    if ((a->n_blk && !a->blocks) || (a->kv_rows && !a->kv_tok)) return fail(err, errlen, "missing plan");
    if (a->P && a->kv_rows) {
        VisPrepParams q;
        q.qkv = a->qkv; q.bias = a->bias; q.pos2 = a->pos2; q.inv_freq = a->inv_freq; q.kv_tok = a->kv_tok;
        q.q_plane = q_plane; q.k_plane = k_plane; q.vt_plane = vt_plane;
        q.P = a->P; q.heads = a->heads; q.kvT = a->kvT; q.kv_rows = a->kv_rows; q.tok_kv = a->tok_kv;
        if (a->tok_kv)
            hipLaunchKernelGGL(vis_prep_rows_kernel, dim3((a->P + kVisRowsBM - 1) / kVisRowsBM, (a->heads + kVisRowsHeads - 1) / kVisRowsHeads + a->heads),
                               dim3(kVisRowsThreads), 0, (hipStream_t)stream, q);
        else
            hipLaunchKernelGGL(vis_prep_kernel, dim3(((a->kv_rows + 15) / 16 * a->heads + 31) / 32 * 32), dim3(256), 0, (hipStream_t)stream, q);
        if (!launch_ok("vis_prep", err, errlen)) return false;
    }
    if (a->n_blk == 0) return true;
    AttnParams p;
    memset(&p, 0, sizeof(p));
    p.q_plane = q_plane; p.k_plane = k_plane; p.vt_plane = vt_plane; p.blocks = a->blocks;
    p.out = a->out; p.ovf = a->ovf;
    p.T = a->P; p.kvT = a->kvT; p.nh = a->heads; p.nkv = a->heads;
    p.scale_log2 = a->scale * 1.4426950408889634f; p.f16_lim = f16_limit(a->f16_lim);
    p.causal = 0; p.gate = 0; p.out_type = a->out_type; p.out_ld = a->heads * kVisHD;
    hipLaunchKernelGGL(attn_vis_kernel, dim3((unsigned)(a->n_blk * a->heads)), dim3(64 * vis::WAVES), 0, (hipStream_t)stream, p);
    return launch_ok("attn_vis", err, errlen);
}

// The FP32 core over the (16-row sub-block, kv head, head chunk) items (the kernel's LDS allows
// one workgroup per CU): a chunk of W <= 6 heads runs two waves per head, each on half of the
// head dims, so that the waves spread evenly over the four SIMDs (12 for the 6 q heads of a
// 24 / 4 model); 7 and 8 heads run one wave per head.
template <int W>
void launch_f32(const text32::Params &p, long grid, hipStream_t s) {
    constexpr int X = W <= 6 ? 2 : 1;
    hipLaunchKernelGGL((text32::attn_text_f32_kernel<W, X>), dim3((unsigned)grid), dim3(64 * W * X), 0, s, p);
}

bool core_f32(const clef_hip_attn_args *a, void *stream, char *err, size_t errlen) {
    text32::Params p;
    p.qkv = (const float *)a->qkv; p.q_norm = a->q_norm; p.pos3 = a->pos3; p.inv_freq = a->inv_freq;
    p.rope_cs = a->n_rot ? a->rope_cs : nullptr;
    p.k_plane = (const float *)a->k_plane; p.v_plane = (const float *)a->vt_plane; p.blocks = a->blocks;
    p.out = a->out; p.ovf = a->ovf;
    p.row = a->row; p.kvT = a->kvT; p.nh = a->nh; p.nkv = a->nkv; p.n_rot = a->n_rot;
    p.causal = a->causal ? 1 : 0; p.gate = a->gate ? 1 : 0; p.out_type = a->out_type;
    p.eps = a->eps; p.scale = a->scale; p.f16_lim = f16_limit(a->f16_lim);
    // a kv group of G q heads runs as ceil(G / 8) chunks of W = ceil(G / chunks) heads
    const int group = a->nh / a->nkv;
    p.n_chunks = (group + 7) / 8;
    const int W = (group + p.n_chunks - 1) / p.n_chunks;
    p.n_blk = a->n_blk;
    const long n_items = (long)a->n_blk * text32::SUB * a->nkv * p.n_chunks;
    if (n_items > 0x7fffffffL) return fail(err, errlen, "grid too large");
    // One workgroup per item, dispatched in the items' longest-first order: the hardware hands
    // each free CU the next item, which balanced C1 better (594 us) than a persistent grid of
    // one workgroup per CU over a static snake order (660 us; C2 within 1%).
    // CLEF_HIP_F32_PERSISTENT=1 selects the persistent grid.
    long grid = n_items;
    const char *ge = getenv("CLEF_HIP_F32_PERSISTENT");
    const long cus = device_cus();
    if (ge && ge[0] == '1' && cus > 0 && cus < n_items) grid = cus;
    hipStream_t s = (hipStream_t)stream;
    switch (W) {
        case 1: launch_f32<1>(p, grid, s); break;
        case 2: launch_f32<2>(p, grid, s); break;
        case 3: launch_f32<3>(p, grid, s); break;
        case 4: launch_f32<4>(p, grid, s); break;
        case 5: launch_f32<5>(p, grid, s); break;
        case 6: launch_f32<6>(p, grid, s); break;
        case 7: launch_f32<7>(p, grid, s); break;
        default: launch_f32<8>(p, grid, s); break;
    }
    return launch_ok("attn_text_f32", err, errlen);
}

// a pass with fewer (block, head) items than workgroups splits its blocks of more than 64 rows
bool sched_splits(int n_blk, int nh, int n_wg) { return (long)n_blk * nh < n_wg; }

// The K/V prologue's arguments (kv_rows.h) from the call's: the shared fields of the separate
// prologue kernel and of the QKV GEMM's epilogue.
KvRows kv_rows_params(const clef_hip_attn_args *a, const int32_t *tok_kv) {
    KvRows r;
    r.T = a->T; r.nh = a->nh; r.nkv = a->nkv; r.n_rot = a->n_rot; r.kvT = a->kvT;
    r.eps = a->eps; r.f16_lim = f16_limit(a->f16_lim);
    r.k_norm = a->k_norm; r.pos3 = a->pos3; r.inv_freq = a->inv_freq; r.tok_kv = tok_kv;
    r.seq_start = a->seq_start; r.ovf = a->ovf;
    r.k_plane = (uint16_t *)a->k_plane; r.vt_plane = (uint16_t *)a->vt_plane;
    r.rope_cs = a->n_rot ? a->rope_cs : nullptr;
    return r;
}

}  // namespace

extern "C" {

int clef_hip_attn_version(void) { return kVersion; }
int clef_hip_attn_wave_size(void) { return 64; }

bool clef_hip_attn_init(char *err, size_t errlen) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(err, errlen, "no device: %s", hipGetErrorString(e));
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) return fail(err, errlen, "device query failed: %s", hipGetErrorString(e));
    if (!strstr(prop.gcnArchName, "gfx950")) return fail(err, errlen, "kernels are built for gfx950, device is %s", prop.gcnArchName);
    if (prop.warpSize != 64) return fail(err, errlen, "attention kernels need 64-wide wavefronts (device reports %d)", prop.warpSize);
    const size_t need = sizeof(uint16_t) * text::LDS_ELEMS;
    if (prop.sharedMemPerBlock < need) return fail(err, errlen, "device LDS %zu < %zu bytes", (size_t)prop.sharedMemPerBlock, need);
    // Resolve this device's scratch address now, not on a first call. A failure disables only
    // clef_hip_vis_attention_noalloc, which tries again and reports it on each call.
    char *scratch_ptr = nullptr;
    char ignored[8];
    (void)scratch_base(&scratch_ptr, ignored, sizeof(ignored));
    return true;
}

int clef_hip_attn_sched_size(int n_blk, int nh, int n_wg) {
    if (n_blk < 0 || nh <= 0 || n_wg <= 0) return 0;
    const long items = (long)n_blk * nh * (sched_splits(n_blk, nh, n_wg) ? 2 : 1);
    return items + kSchedHeader + 1 + n_wg > 0x7fffffffL ? 0 : (int)(kSchedHeader + n_wg + 1 + items);
}

bool clef_hip_attn_schedule(const int32_t *blocks, int n_blk, int nh, int nkv, int n_wg,
                            int32_t *sched, int max_sched, char *err, size_t errlen) {
    if ((n_blk && !blocks) || !sched || n_blk < 0 || nh <= 0 || nkv <= 0 || nh % nkv || n_wg <= 0)
        return fail(err, errlen, "bad schedule arguments");
    if ((long)n_blk * nh >= (1L << 28)) return fail(err, errlen, "too many items for a schedule");
    const bool split = sched_splits(n_blk, nh, n_wg);
    const long need = (long)kSchedHeader + n_wg + 1 + (long)n_blk * nh * (split ? 2 : 1);
    if (need > max_sched) return fail(err, errlen, "schedule needs %ld entries, room for %d", need, max_sched);
    // cost of an item in 64-key tiles: its tiles plus the prologue / epilogue (Q rows, gate,
    // output stores). Measured at about three tiles' time per item, but a weight of 6 balances
    // C1 best (core 74-76.5 us against 76-78 us at 3, in two calls; 8 and 10 lose again): it
    // spreads the item counts, and the items' real durations vary more than their tiles do. A
    // first half's keys end at its last row when the pass is causal (the estimate assumes it is).
    constexpr int kFixed = 6;
    const int xh = (nh % 8 == 0 && ((nh / nkv) % (nh / 8) == 0 || (nh / 8) % (nh / nkv) == 0)) ? nh / 8 : 0;
    const int groups = (xh && n_wg % 8 == 0) ? 8 : 1;
    auto cost_of = [&](int item) {
        const int32_t *e = blocks + 8 * ((item & ((1 << 28) - 1)) / nh);
        const int k_len = ((item >> 28) & 3) == 1 ? std::min(e[4], e[2] + 64) : e[4];
        return (k_len + 63) / 64 + kFixed;
    };
    // Every item with its cost; then each to an XCD group: its head's, or for a packed item whose
    // heads span several groups (all of them hold the kv head's planes), the least loaded of
    // them, taking the items longest first. Without that, a pass of short records, all packed,
    // would leave the groups of the heads that never start a packed item idle.
    std::vector<std::pair<int, int>> all;   // (cost, item)
    for (int bi = 0; bi < n_blk; bi++) {
        // a block of at most 64 rows runs k heads of a kv group at once (unless the pass splits
        // blocks, which wants more items, not fewer)
        const int pk = split ? 1 : clef_hip::pack_heads(blocks[8 * bi + 1], nh / nkv);
        // a block of more than 64 rows runs as its two halves for two heads each (bit 30) when
        // the kv group has an even size
        const bool pair = !split && blocks[8 * bi + 1] > 64 && (nh / nkv) % 2 == 0;
        for (int h = 0; h < nh; h++) {
            const int it = bi * nh + h;
            if (split && blocks[8 * bi + 1] > 64) {   // the block's rows 0-63 and 64-127
                all.push_back({cost_of(it | (1 << 28)), it | (1 << 28)});
                all.push_back({cost_of(it | (2 << 28)), it | (2 << 28)});
            } else if (pair) {                        // heads h, h + 1: rows 0-63, then 64-127
                if (h % 2 == 0) {
                    all.push_back({cost_of(it | (1 << 28) | (1 << 30)), it | (1 << 28) | (1 << 30)});
                    all.push_back({cost_of(it | (2 << 28) | (1 << 30)), it | (2 << 28) | (1 << 30)});
                }
            } else if (pk > 1) {                      // heads h .. h + pk - 1 (group-aligned)
                if (h % pk == 0) all.push_back({cost_of(it | (3 << 28)), it | (3 << 28)});
            } else {
                all.push_back({cost_of(it), it});
            }
        }
    }
    std::stable_sort(all.begin(), all.end(), [](const std::pair<int, int> &u, const std::pair<int, int> &v) { return u.first > v.first; });
    std::vector<std::vector<std::pair<int, int>>> per_x(groups);
    std::vector<long> xload(groups, 0);
    for (const auto &c : all) {
        int x = 0;
        if (groups != 1) {
            const int base = c.second & ((1 << 28) - 1), h0 = base % nh;
            const int hk = ((c.second >> 28) & 3) == 3 ? clef_hip::pack_heads(blocks[8 * (base / nh) + 1], nh / nkv)
                                                      : ((c.second >> 30) & 1) ? 2 : 1;
            x = h0 / xh;
            for (int y = h0 / xh + 1; y <= (h0 + hk - 1) / xh; y++)
                if (xload[y] < xload[x]) x = y;
        }
        per_x[x].push_back(c);
        xload[x] += c.first;
    }
    std::vector<std::vector<int>> lists(n_wg);
    std::vector<long> load(n_wg, 0);
    for (int x = 0; x < groups; x++) {
        const std::vector<std::pair<int, int>> &its = per_x[x];   // longest first
        for (const auto &it : its) {
            int best = -1;
            for (int b = x; b < n_wg; b += groups)
                if (best < 0 || load[b] < load[best]) best = b;
            load[best] += it.first;
            lists[best].push_back(it.second);
        }
        // Local search on the greedy result: while an item of the most loaded workgroup can
        // move to another workgroup, or be swapped for a shorter one there, so that the other
        // workgroup stays below the current maximum, do it. Each step lowers the sum of squared
        // loads, so the search ends; on C1 it takes the makespan from 37 to 35 tiles.
        std::vector<int> wgs;
        for (int b = x; b < n_wg; b += groups) wgs.push_back(b);
        for (int step = 0; step < 100000; step++) {   // a cap on host time for adversarial plans
            int mx = wgs[0];
            for (int b : wgs)
                if (load[b] > load[mx]) mx = b;
            bool moved = false;
            for (int j : wgs) {
                if (j == mx) continue;
                auto &src = lists[mx], &dst = lists[j];
                for (size_t u = 0; u < src.size() && !moved; u++) {
                    const int cu = cost_of(src[u]);
                    if (load[j] + cu < load[mx]) {
                        dst.push_back(src[u]);
                        src.erase(src.begin() + u);
                        load[mx] -= cu; load[j] += cu; moved = true;
                        break;
                    }
                    for (size_t v = 0; v < dst.size(); v++) {
                        const int d = cu - cost_of(dst[v]);
                        if (d > 0 && load[j] + d < load[mx]) {
                            std::swap(src[u], dst[v]);
                            load[mx] -= d; load[j] += d; moved = true;
                            break;
                        }
                    }
                }
                if (moved) break;
            }
            if (!moved) break;
        }
    }
    for (auto &l : lists)   // each workgroup takes its items longest first
        std::stable_sort(l.begin(), l.end(), [&](int u, int v) { return cost_of(u) > cost_of(v); });
    sched[0] = kSchedMagic;
    sched[1] = n_blk;
    sched[2] = nh;
    sched[3] = n_wg;
    sched[4] = nkv;
    sched[5] = blocks_fingerprint(blocks, n_blk);
    sched[6] = sched[7] = 0;
    int32_t *const offs = sched + kSchedHeader;
    int off = 0;
    for (int b = 0; b < n_wg; b++) {
        offs[b] = off;
        for (int it : lists[b]) offs[n_wg + 1 + off++] = it;
    }
    offs[n_wg] = off;
    return true;
}

int clef_hip_attn_plan_max_blocks(int n_seq, int Tq) {
    if (n_seq < 0 || Tq < 0) return 0;
    return Tq / CLEF_HIP_BLOCK_Q + n_seq + 1;
}


bool clef_hip_attn_plan(const int32_t *cu_q, const int32_t *cu_k, int n_seq, int causal,
                        int32_t *blocks, int max_blocks, int32_t *tok_kv, int max_tok,
                        int32_t *kv_tok, int max_kv, int *n_blk, int *kv_rows, char *err, size_t errlen) {
    if (!cu_q || n_seq < 0 || !n_blk || !kv_rows) return fail(err, errlen, "bad plan arguments");
    if (cu_q[0] != 0) return fail(err, errlen, "cu_seqlens_q must start at 0");
    if (cu_k && cu_k[0] != 0) return fail(err, errlen, "cu_seqlens_k must start at 0");
    struct Ent { int32_t v[CLEF_HIP_BLOCK_INTS]; };
    std::vector<Ent> ents;
    int kv_off = 0;
    for (int r = 0; r < n_seq; r++) {
        const int nq = cu_q[r + 1] - cu_q[r];
        if (nq < 0) return fail(err, errlen, "cu_seqlens_q decreases at record %d", r);
        int nk = nq, k0 = kv_off;
        if (cu_k) {
            nk = cu_k[r + 1] - cu_k[r];
            k0 = cu_k[r];
            if (nk < nq) return fail(err, errlen, "record %d has %d keys for %d queries", r, nk, nq);
            if (k0 % 8) return fail(err, errlen, "cu_seqlens_k[%d] = %d is not a multiple of 8", r, k0);
        } else {
            kv_off += (nq + CLEF_HIP_KV_ALIGN - 1) / CLEF_HIP_KV_ALIGN * CLEF_HIP_KV_ALIGN;
        }
        const int L = nk - nq;
        for (int i0 = 0; i0 < nq; i0 += CLEF_HIP_BLOCK_Q) {
            Ent e;
            const int n = std::min(CLEF_HIP_BLOCK_Q, nq - i0);
            e.v[0] = cu_q[r] + i0;
            e.v[1] = n;
            e.v[2] = L + i0;
            e.v[3] = k0;
            e.v[4] = causal ? std::min(nk, L + i0 + n) : nk;
            e.v[5] = cu_q[r];
            e.v[6] = r;
            e.v[7] = 0;
            ents.push_back(e);
        }
    }
    // rows per head the planes need: the fills read whole 64-key tiles from each record's first
    // key (past a record's last key they read the next record's rows, masked in the scores and
    // zeroed in the V tile, or the slack at the end)
    constexpr int kTileKeys = 64;
    int total_kv = 0;
    kv_off = 0;
    for (int r = 0; r < n_seq; r++) {
        const int nq = cu_q[r + 1] - cu_q[r];
        const int nk = cu_k ? cu_k[r + 1] - cu_k[r] : nq;
        const int k0 = cu_k ? cu_k[r] : kv_off;
        total_kv = std::max(total_kv, k0 + (nk + kTileKeys - 1) / kTileKeys * kTileKeys);
        if (!cu_k) kv_off += (nq + CLEF_HIP_KV_ALIGN - 1) / CLEF_HIP_KV_ALIGN * CLEF_HIP_KV_ALIGN;
    }
    if ((int)ents.size() > max_blocks) return fail(err, errlen, "plan needs %zu blocks, room for %d", ents.size(), max_blocks);
    if (cu_q[n_seq] > max_tok) return fail(err, errlen, "plan needs %d tok_kv entries, room for %d", cu_q[n_seq], max_tok);
    if ((!blocks && !ents.empty()) || (!tok_kv && cu_q[n_seq])) return fail(err, errlen, "missing plan output arrays");
    if (kv_tok && total_kv > max_kv) return fail(err, errlen, "plan needs %d kv_tok entries, room for %d", total_kv, max_kv);
    // Longest key range first, so the long causal blocks start early (clef_metal.m:1243-1257
    // orders each record's blocks longest first; here the order is global across records).
    std::stable_sort(ents.begin(), ents.end(), [](const Ent &x, const Ent &y) { return x.v[4] > y.v[4]; });
    for (size_t i = 0; i < ents.size(); i++) memcpy(blocks + CLEF_HIP_BLOCK_INTS * i, ents[i].v, sizeof(ents[i].v));
    const int32_t fp = blocks_fingerprint(blocks, (int)ents.size());
    for (size_t i = 0; i < ents.size(); i++) blocks[CLEF_HIP_BLOCK_INTS * i + 7] = fp;
    kv_off = 0;
    for (int r = 0; r < n_seq; r++) {
        const int nq = cu_q[r + 1] - cu_q[r];
        const int nk = cu_k ? cu_k[r + 1] - cu_k[r] : nq;
        const int k0 = cu_k ? cu_k[r] : kv_off;
        for (int j = 0; j < nq; j++) tok_kv[cu_q[r] + j] = k0 + (nk - nq) + j;
        if (!cu_k) kv_off += (nq + CLEF_HIP_KV_ALIGN - 1) / CLEF_HIP_KV_ALIGN * CLEF_HIP_KV_ALIGN;
    }
    if (kv_tok) {
        for (int k = 0; k < total_kv; k++) kv_tok[k] = -1;
        for (int t = 0; t < cu_q[n_seq]; t++) kv_tok[tok_kv[t]] = t;
    }
    *n_blk = (int)ents.size();
    *kv_rows = total_kv;
    return true;
}

void clef_hip_rope_inv_freq(float theta, int n_rot, float *inv_freq) {
    for (int j = 0; j < n_rot / 2; j++) inv_freq[j] = 1.0f / powf(theta, (float)(2 * j) / (float)n_rot);
}

bool clef_hip_vis_positions(const int32_t *cu, int n_img, const int32_t *grid_w, int merge,
                            int32_t *pos2, char *err, size_t errlen) {
    if (!cu || !grid_w || !pos2 || n_img < 0 || merge <= 0) return fail(err, errlen, "bad vision position arguments");
    for (int g = 0; g < n_img; g++) {
        const int P = cu[g + 1] - cu[g];
        if (P < 0 || grid_w[g] <= 0 || grid_w[g] % merge) return fail(err, errlen, "bad image %d geometry", g);
        const int window = merge * merge, w2 = grid_w[g] / merge;
        for (int p = 0; p < P; p++) {
            const int blk = p / window, within = p % window;
            pos2[2 * (cu[g] + p)] = (blk / w2) * merge + within / merge;
            pos2[2 * (cu[g] + p) + 1] = (blk % w2) * merge + within % merge;
        }
    }
    return true;
}

bool clef_hip_attn_prep_kv(const clef_hip_attn_args *a, void *stream, char *err, size_t errlen) {
    if (!check_text(a, false, err, errlen)) return false;
    if (a->T == 0 || a->kv_rows == 0) return true;
    if (a->qkv_type == CLEF_HIP_QKV_F32) {
        text32::PrepParams p;
        p.qkv = (const float *)a->qkv; p.k_norm = a->k_norm; p.pos3 = a->pos3; p.inv_freq = a->inv_freq;
        p.kv_tok = a->kv_tok; p.k_plane = (float *)a->k_plane; p.v_plane = (float *)a->vt_plane;
        p.rope_cs = a->n_rot ? a->rope_cs : nullptr;
        p.kv_rows = a->kv_rows; p.row = a->row; p.nh = a->nh; p.nkv = a->nkv; p.n_rot = a->n_rot; p.kvT = a->kvT;
        p.eps = a->eps;
        const long groups = (long)a->kv_rows * a->nkv;
        hipLaunchKernelGGL(text32::text_prep_kv_f32_kernel, dim3((unsigned)((groups + 7) / 8)), dim3(256), 0, (hipStream_t)stream, p);
        return launch_ok("text_prep_kv_f32", err, errlen);
    }
    if (!a->tok_kv) return fail(err, errlen, "the K/V prologue needs tok_kv (the plan's pass row -> plane row map)");
    // K waves of 4 pass rows, then V waves of (kv head, 64 rows, 16 dims); 4 waves per workgroup
    const long waves = (long)(a->T + 3) / 4 + (long)a->nkv * ((a->T + 63) / 64) * 16;
    hipLaunchKernelGGL(text_prep_direct_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(kPrepDirectThreads), 0, (hipStream_t)stream,
                       (const uint16_t *)a->qkv, a->row, kv_rows_params(a, a->tok_kv));
    return launch_ok("text_prep_direct", err, errlen);
}

bool clef_hip_attn_core(const clef_hip_attn_args *a, void *stream, char *err, size_t errlen) {
    if (!check_text(a, true, err, errlen)) return false;
    if (a->n_blk == 0) return true;
    if (a->qkv_type == CLEF_HIP_QKV_F32) return core_f32(a, stream, err, errlen);
    AttnParams p;
    memset(&p, 0, sizeof(p));
    p.qkv = (const uint16_t *)a->qkv; p.q_norm = a->q_norm; p.pos3 = a->pos3; p.inv_freq = a->inv_freq;
    p.rope_cs = a->n_rot ? a->rope_cs : nullptr;
    p.k_plane = (const uint16_t *)a->k_plane; p.vt_plane = (const uint16_t *)a->vt_plane; p.blocks = a->blocks;
    p.out = a->out; p.ovf = a->ovf;
    p.row = a->row; p.T = a->T; p.kvT = a->kvT; p.nh = a->nh; p.nkv = a->nkv; p.n_rot = a->n_rot;
    p.eps = a->eps; p.scale_log2 = a->scale * 1.4426950408889634f;
    p.f16_lim = f16_limit(a->f16_lim);
    p.causal = a->causal ? 1 : 0; p.gate = a->gate ? 1 : 0; p.out_type = a->out_type;
    p.out_ld = a->nh * a->hd;
    p.trace = a->trace;
    p.n_blk = a->n_blk;
    p.xcd_heads = (a->nh % 8 == 0 && (a->nh / 8) > 0 && ((a->nh / a->nkv) % (a->nh / 8) == 0 || (a->nh / 8) % (a->nh / a->nkv) == 0)) ? a->nh / 8 : 0;
    const long n_items = (long)a->n_blk * a->nh;
    if (n_items > 0x7fffffffL) return fail(err, errlen, "grid too large");
    long grid = n_items;
    if (a->sched) {
        if (a->n_wg <= 0) return fail(err, errlen, "bad n_wg %d for the schedule", a->n_wg);
        p.sched = a->sched;
        grid = a->n_wg;
    } else if (text_persistent()) {
        // one workgroup per CU, each looping over its items (a multiple of 8 for the XCD mapping)
        const long cus = device_cus();
        if (cus > 0 && cus < n_items) grid = p.xcd_heads ? std::max(8L, cus / 8 * 8) : cus;
    }
    if (a->n_rot == 64)
        hipLaunchKernelGGL(attn_text_kernel<64>, dim3((unsigned)grid), dim3(512), 0, (hipStream_t)stream, p);
    else
        hipLaunchKernelGGL(attn_text_kernel<0>, dim3((unsigned)grid), dim3(512), 0, (hipStream_t)stream, p);
    return launch_ok("attn_fwd<256>", err, errlen);
}

bool clef_hip_qkv_gemm(int H, const uint16_t *X, const uint16_t *W, const clef_hip_attn_args *a, const int32_t *tok_kv,
                       void *stream, char *err, size_t errlen) {
    if (!a) return fail(err, errlen, "null attention arguments");
    if (a->qkv_type != CLEF_HIP_QKV_BF16) return fail(err, errlen, "the QKV GEMM writes bf16 qkv rows (qkv_type 0)");
    if (tok_kv ? !check_text(a, false, err, errlen)
               : (a->hd != 256 || a->nh <= 0 || a->nkv <= 0 || a->nh % a->nkv || a->T < 0 || !a->qkv || !aligned16(a->qkv)))
        return tok_kv ? false : fail(err, errlen, "bad QKV GEMM geometry or qkv pointer");
    const long N = 2L * a->nh * a->hd + 2L * a->nkv * a->hd;
    if (a->row < N || a->row % 8) return fail(err, errlen, "qkv row %d must be >= %ld and a multiple of 8", a->row, N);
    if (H <= 0 || H % gemm::KALIGN) return fail(err, errlen, "hidden size %d must be a positive multiple of %d", H, gemm::KALIGN);
    if (!X || !W || !aligned16(X) || !aligned16(W)) return fail(err, errlen, "X and W must be 16-byte aligned device pointers");
    if ((long)a->T * H * 2 >= (1L << 32) || N * H * 2 >= (1L << 32))
        return fail(err, errlen, "X or W above 4 GiB (32-bit fill offsets)");
    if (tok_kv && a->n_rot && a->n_rot != 64) return fail(err, errlen, "the fused prologue takes n_rot 0 or 64 (got %d)", a->n_rot);
    if (a->T == 0) return true;
    gemm::Params p;
    memset(&p, 0, sizeof(p));
    p.X = X; p.W = W; p.Y = (uint16_t *)a->qkv;
    p.T = a->T; p.N = (int)N; p.K = H; p.ldy = a->row;
    p.n_tiles = (int)(N / gemm::BN);
    p.n_per_xcd = (p.n_tiles + 7) / 8;
    p.r.T = a->T; p.r.nh = a->nh; p.r.nkv = a->nkv;
    if (tok_kv) {
        p.kv = 1;
        p.r = kv_rows_params(a, tok_kv);
    }
    // 256 x 256 tiles, 8 waves of 128 x 64, 64-deep K slices double-buffered (128 KB of LDS):
    // 128-row tiles moved 1.5x the operand bytes per product and ran fill-bound (0.59 against
    // 0.53 ms at 4096 x 14336 x 5120); 32-deep slices four deep and 64 x 128 wave blocks measured
    // no better
    using C = gemm::Cfg<256, 128, 64, 64, 2>;
    p.m_tiles = (a->T + C::BM - 1) / C::BM;
    const long grid = 8L * p.n_per_xcd * p.m_tiles;
    hipLaunchKernelGGL(gemm::qkv_gemm_kernel<C>, dim3((unsigned)grid), dim3(C::THREADS), 0, (hipStream_t)stream, p);
    return launch_ok("qkv_gemm", err, errlen);
}

bool clef_hip_attn_prefill(const clef_hip_attn_args *a, void *stream, char *err, size_t errlen) {
    if (!check_text(a, true, err, errlen)) return false;
    if (!clef_hip_attn_prep_kv(a, stream, err, errlen)) return false;
    return clef_hip_attn_core(a, stream, err, errlen);
}

bool clef_hip_vis_attention(const clef_hip_vis_args *a, void *stream, char *err, size_t errlen) {
    if (!a) return fail(err, errlen, "null vision arguments");
    return vis_run(a, a->q_plane, a->k_plane, a->vt_plane, stream, err, errlen);
}

bool clef_hip_vis_attention_noalloc(const clef_hip_vis_args *a, void *stream, char *err, size_t errlen) {
    if (!a) return fail(err, errlen, "null vision arguments");
    if (a->hd != kVisHD) return fail(err, errlen, "vision attention supports hd 72 only (got %d)", a->hd);
    if (a->P < 0 || a->heads <= 0 || a->kvT < 0) return fail(err, errlen, "bad vision sizes");
    const size_t qb = vis_plane_bytes(a->heads, a->P > 0 ? a->P : 1), kb = vis_plane_bytes(a->heads, a->kvT);
    const size_t need = qb + 2 * kb;
    if (need > kVisScratchBytes)
        return fail(err, errlen, "vision planes need %zu bytes (heads %d, P %d, kvT %d): above the %zu-byte scratch",
                    need, a->heads, a->P, a->kvT, kVisScratchBytes);
    char *base = nullptr;
    if (!scratch_base(&base, err, errlen)) return false;
    return vis_run(a, (uint16_t *)base, (uint16_t *)(base + qb), (uint16_t *)(base + qb + kb), stream, err, errlen);
}

}  // extern "C"
