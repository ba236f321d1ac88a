// Text prefill attention for head dim 256 on CDNA4: packed varlen causal GQA attention over a
// record-aligned block list, with the Q prologue (per-head RMSNorm + partial interleaved
// M-RoPE) fused into the block's start and the sigmoid output gate fused into the epilogue.
// Semantics: metal/clef.metal:930-1093 (attention_tu: block list, record-aligned key tiles,
// sum of the rounded P, O / l * sigmoid(G)), metal/clef.metal:245-300 (prologue),
// metal/clef.metal:709-849 (prefix: queries offset into the record's keys).
//
// Workgroup: 8 wavefronts (2 per SIMD), one block of 128 query rows of one q head per work item;
// wave w owns rows 16w .. 16w+15. The state per wave (O^T 64, Q 32, S 16 VGPRs, operand rings,
// addresses) fits 215 VGPRs, so two waves share a SIMD.
//   S^T = K . Q^T      v_mfma_f32_16x16x32_f16: A = 16 keys x 32 dims of K from LDS,
//                      B = the wave's Q (registers). A lane owns one query column. Q and K are
//                      f16: their 11-bit significands keep the scores of sharp rows within the
//                      output tolerance, where bf16-rounded K alone misses it (the normalised
//                      values are bounded by 16 max|w|, far inside f16's range; without the
//                      norms, Q and K must lie within it).
//   O^T += V^T . P^T   v_mfma_f32_16x16x32_bf16: A = 16 dims x 32 keys of V^T (bf16) from LDS,
//                      B = P (bf16) straight from registers.
// The A rows are read in a permuted order (key / dim 8*(r/4) + 4*(tile&1) + r%4 for row r) so
// that the 8 keys a lane's P covers and the 8 dims its O covers are consecutive: P is the next
// product's B operand with no shuffle, and the epilogue stores 16-byte runs.
// K and V^T tiles (64 keys) stream global -> LDS with global_load_lds, double buffered, into
// unpadded rows whose 16-byte chunks are XOR-swizzled so the A reads are bank-conflict free.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

#include "attn_kernels.h"
#include "attn_params.h"

namespace clef_hip {

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(8))) int i32x8;

namespace text {
constexpr int HD = 256;                 // head dim
constexpr int BQ = 128;                 // query rows per block
constexpr int BK = 64;                  // keys per LDS tile
constexpr int WAVES = 8;
constexpr int ROWS = 16;                // query rows per wave
constexpr int NC = HD / 32;             // 32-dim contraction chunks of S
constexpr int KTILE = BK * HD;          // elements per K tile  (32 KB)
constexpr int VTILE = HD * BK;          // elements per V^T tile (32 KB)
constexpr int LDS_ELEMS = 2 * KTILE + 2 * VTILE;   // 128 KB

// key of A-operand row r in S tile kt (four 16-key tiles per 64-key LDS tile)
__device__ __forceinline__ int s_row_key(int kt, int r) {
    return 32 * (kt >> 1) + 8 * (r >> 2) + 4 * (kt & 1) + (r & 3);
}
// XOR swizzle of a K row's 16-byte chunks (rows of 32 chunks); distinct over the 16 keys
// that one A read touches
__device__ __forceinline__ int k_swz(int key) { return (key & 15) ^ ((key >> 4) << 2); }
// XOR swizzle of a V^T row's chunks (rows of 8 chunks, two rows per 256-byte bank line)
__device__ __forceinline__ int v_swz(int d) { return ((d >> 1) & 1) | (((d >> 3) & 3) << 1); }
// Sum / max over the four 16-lane rows of a wave (v_permlane16_swap / v_permlane32_swap, VALU
// only, so no LDS traffic). Every lane gets the same bits.
__device__ __forceinline__ float xrow_max(float x) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float m = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    return fmaxf(__uint_as_float(q[0]), __uint_as_float(q[1]));
}
__device__ __forceinline__ float xrow_sum(float x) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float m = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// LDS operand reads issued as ds_read_b128 with an explicit lgkmcnt wait per use. The compiler
// would otherwise wait for every outstanding LDS access (lgkmcnt(0)) before each use while the
// global_load_lds fills of the other buffer are in flight. lds_wait ties the wait to the value
// it guards, so the product that consumes it cannot be scheduled above the wait.
template <int OFF>
__device__ __forceinline__ bf16x8 lds_read16(unsigned addr) {
    bf16x8 r;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF) : "memory");
    return r;
}
template <int N>
__device__ __forceinline__ void lds_wait(bf16x8 &r) {
    asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(r) : "i"(N));
}
// One wait for two reads (the two operands of a pair of products): half the waits, and the
// compiler's wait state after the asm falls before the first product only.
template <int N>
__device__ __forceinline__ void lds_wait2(bf16x8 &r0, bf16x8 &r1) {
    asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(r0), "+v"(r1) : "i"(N));
}
template <int N>
__device__ __forceinline__ void lds_wait4(bf16x8 &r0, bf16x8 &r1, bf16x8 &r2, bf16x8 &r3) {
    asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(r0), "+v"(r1), "+v"(r2), "+v"(r3) : "i"(N));
}
__device__ __forceinline__ unsigned lds_addr(const uint16_t *p) {
    return (unsigned)(uintptr_t)(const __attribute__((address_space(3))) uint16_t *)p;
}
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}
}  // namespace text

// Work items are (query block, q head) pairs. Workgroup b takes items get(0), get(1), ... With a
// host schedule (p.sched, clef_hip_attn_schedule) they are the workgroup's own list; an item
// index outside the plan ends the list, so no list can make the kernel touch memory outside it. Otherwise
// they come from a static order: with xcd_heads, the items of XCD x (workgroup ids go round-robin
// over the 8 XCDs, each with its own L2) are the heads x*xcd_heads .. +xcd_heads-1 of every block,
// so an XCD streams the K/V of as few kv heads as possible; items keep the plan's longest-first
// block order and are dealt to the XCD's workgroups in snake order (round r left to right when r
// is even, right to left when odd), so long and short blocks mix. A grid of one workgroup per
// item gives every workgroup exactly one.
// Schedule entries are read with scalar loads, which leave the vector memory counter (the tile
// fills' waits count on it) alone.
__device__ __forceinline__ int sload(const int32_t *ptr) {
    int v;
    asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(ptr) : "memory");
    return v;
}
// A schedule item: block * nh + head in bits 0-27, and in bits 28-29 the rows of the block it
// covers: 0 all, 1 rows 0-63, 2 rows 64-127 (a pass with fewer items than workgroups splits its
// blocks so that every workgroup has work), or 3: the block's rows (at most 64) for heads
// h .. h + k - 1 of one kv group, ceil(rows / 16) waves per head (pack_heads), which share its
// key tiles. Bit 30 with code 1 or 2: that half of the block for heads h and h + 1 of one kv
// group (four waves per head), so that a causal block's last 64 keys, which only its rows 64-127
// see, run on a full workgroup. A row's arithmetic does not depend on any of this: each 16-row
// wave runs the key tiles up to its own last row, from the record's first key.
constexpr int kItemBits = 28;
__device__ __forceinline__ int item_base(int it) { return it & ((1 << kItemBits) - 1); }
// Heads per packed item of a block of nq <= 64 rows: the largest divisor of the kv group size
// that fits 8 waves at ceil(nq / 16) waves per head (the host schedule uses the same rule).
__host__ __device__ inline int pack_heads(int nq, int group) {
    const int wph = (nq + 15) / 16;
    if (nq <= 0 || nq > 64) return 1;
    for (int k = 8 / wph; k > 1; k--)
        if (group % k == 0) return k;
    return 1;
}
struct ItemList {
    int n_items, per_x, gx, xh, nh, s0, s1;
    const int32_t *list;
    __device__ __forceinline__ void setup(const AttnParams &p) {
        nh = p.nh;
        xh = p.xcd_heads;
        gx = (int)gridDim.x >> 3;
        n_items = p.n_blk * p.nh;
        per_x = xh ? p.n_blk * xh : 0;
        list = nullptr;
        s0 = s1 = 0;
        // A schedule: header {magic, n_blk, nh, n_wg, nkv, fingerprint, 0, 0}, then offsets and
        // items. It is used only when the header names this pass: its sizes, this grid, and the
        // fingerprint the plan wrote into word 7 of every block entry. Otherwise every
        // workgroup (all read the same words) takes the static order, which covers every item.
        if (p.sched) {
            // the header and the plan's fingerprint in one round trip, then the workgroup's two
            // offsets in one
            i32x8 h;
            int fp;
            asm volatile("s_load_dwordx8 %0, %2, 0x0\n\ts_load_dword %1, %3, 0x1c\n\ts_waitcnt lgkmcnt(0)"
                         : "=&s"(h), "=&s"(fp) : "s"(p.sched), "s"(p.blocks) : "memory");
            if (h[0] == 0x53434844 && h[1] == p.n_blk && h[2] == p.nh && h[3] == (int)gridDim.x && h[4] == p.nkv && h[5] == fp) {
                const int32_t *offs = p.sched + 8;
                typedef __attribute__((ext_vector_type(2))) int i32x2;
                i32x2 o;
                asm volatile("s_load_dwordx2 %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(o) : "s"(offs + blockIdx.x) : "memory");
                s0 = o[0];
                s1 = o[1];
                list = offs + gridDim.x + 1;
            }
        }
    }
    // the k-th item of this workgroup (block * nh + head, with the rows code above), or -1
    __device__ __forceinline__ int get(int k) const {
        if (list) {
            if (s0 + k >= s1) return -1;
            const int it = sload(list + s0 + k);
            return (it >= 0 && item_base(it) < n_items) ? it : -1;   // never an item outside the plan
        }
        if (xh && gx && ((int)gridDim.x & 7) == 0) {
            const int x = blockIdx.x & 7, wl = blockIdx.x >> 3;
            const int j = k * gx + ((k & 1) ? gx - 1 - wl : wl);
            if (j >= per_x) return -1;
            const int bi = j / xh;
            return bi * nh + x * xh + (j - bi * xh);
        }
        const int G = gridDim.x;
        const int j = k * G + ((k & 1) ? G - 1 - (int)blockIdx.x : (int)blockIdx.x);
        return j < n_items ? j : -1;
    }
};

// A workgroup's loop over its items. While one item's epilogue runs (sigmoid gate, stores), the
// next item's Q rows and first K / V^T tile load by DMA into the LDS buffers the finished key loop
// left free, and its rotary cos/sin into registers.
template <int NROT>
__device__ __forceinline__ void text_items(const AttnParams &p, uint16_t *smem, float *qn_lds) {
    using namespace text;
    static_assert(NROT % 64 == 0 && NROT <= HD, "rotary pairs must sit in one lane");
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int q16 = lane & 15, g = lane >> 4;
    ItemList items;
    items.setup(p);
    int item = items.get(0);
    if (item < 0) return;

    // LDS: K0 | K1 | V0 | V1 (32 KB each). Operand reads address K buffers from the LDS base and
    // V buffers from base + 64 KB, so the buffer choice is an immediate offset.
    uint16_t *const k0s = smem, *const k1s = smem + KTILE, *const v0s = smem + 2 * KTILE,
                   *const v1s = smem + 2 * KTILE + VTILE;
    // Wave w fills slots [(4w + j) * 64, +64) of each 2048-slot tile, one global_load_lds per j.
    // K slot s: key s/32, chunk (s%32) ^ k_swz(key). V^T slot s: dim s/8, chunk (s%8) ^ v_swz(dim).
    // Tiles may reach past the record's last key (up to the 64-key boundary): the plan sizes the
    // planes so that those reads stay inside them, their scores are masked and their V^T entries
    // zeroed in LDS before use.
    const int wave_s = __builtin_amdgcn_readfirstlane(wave);
    unsigned kfo[4], vfo[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int grp = wave_s * 4 + j;
        const int key = grp * 2 + (lane >> 5);
        kfo[j] = (unsigned)(key * HD + (((lane & 31) ^ k_swz(key)) * 8)) * 2u;
        const int d = grp * 8 + (lane >> 3);
        vfo[j] = ((unsigned)d * (unsigned)p.kvT + (unsigned)(((lane & 7) ^ v_swz(d)) * 8)) * 2u;
    }
    // per-lane LDS byte addresses of the A operands
    const unsigned kl = lds_addr(smem), vl = kl + 2 * 2 * KTILE;
    unsigned ka[4][4];   // byte address of (S tile kt, chunk c & 3) in K0; c >> 2 and K1 are offsets
#pragma unroll
    for (int kt = 0; kt < 4; kt++) {
        const int key = s_row_key(kt, q16);
        const int x = k_swz(key);
#pragma unroll
        for (int cl = 0; cl < 4; cl++) ka[kt][cl] = kl + 2 * (key * HD + (((4 * cl + g) ^ x) * 8));
    }
    const int vrow = 8 * (q16 >> 2) + (q16 & 3);   // + 32*(mt>>1) + 4*(mt&1)
    const int vx = v_swz(vrow);                      // the mt part does not change the swizzle
    const unsigned va0 = vl + 2 * (vrow * BK + ((g ^ vx) * 8));
    const unsigned va1 = vl + 2 * (vrow * BK + (((4 + g) ^ vx) * 8));
    const unsigned qn_addr = lds_addr((const uint16_t *)qn_lds);
    constexpr int R = NROT / 64;

    // Item state: the block entry and the lane's query row.
    struct Item {
        int q_row0, nq, q_pos0, k_row0, k_len, flag_row, h, kh, n_tiles;
        int wph, hk;   // waves per head (8: one head on all waves), heads in the item
        const uint16_t *kbase, *vbase;
    };
    // The block entry is read with a scalar load: the compiler would read it with vector loads
    // once the kernel has stored anything, and those would wait behind the in-flight tile fills.
    auto decode_from = [&](const i32x8 &e, int it) {
        Item s;
        const int base = item_base(it), half = (it >> kItemBits) & 3, pair = (it >> 30) & 1;
        const int bi = base / p.nh;
        s.h = base - bi * p.nh;
        s.q_row0 = e[0]; s.nq = e[1]; s.q_pos0 = e[2]; s.k_row0 = e[3]; s.k_len = e[4];
        if (half == 1) {          // rows 0-63: a causal half sees keys up to its own last row
            s.nq = min(s.nq, 64);
            if (p.causal) s.k_len = min(s.k_len, s.q_pos0 + s.nq);
        } else if (half == 2 && s.nq > 64) {   // rows 64-127 (of a smaller block: all of it, so
            s.q_row0 += 64; s.q_pos0 += 64; s.nq -= 64;   // that no list reaches rows outside it)
        }
        const int group = p.nh / p.nkv;
        s.wph = 8; s.hk = 1;
        if (half == 3 || pair) {   // heads h .. h + k - 1, all in h's kv group (else the item runs head h)
            const int k = pair ? ((group % 2 == 0 && s.nq <= 64) ? 2 : 1) : pack_heads(s.nq, group);
            if (k > 1 && s.h % group + k <= group) { s.wph = (s.nq + 15) / 16; s.hk = k; }
        }
        s.flag_row = e[5];
        s.kh = s.h / group;
        s.n_tiles = (s.k_len + BK - 1) / BK;
        s.kbase = p.k_plane + ((size_t)s.kh * p.kvT + s.k_row0) * HD;
        s.vbase = p.vt_plane + (size_t)s.kh * HD * p.kvT + s.k_row0;
        return s;
    };
    auto decode = [&](int it) {
        i32x8 e;
        asm volatile("s_load_dwordx8 %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(e) : "s"(p.blocks + 8 * (item_base(it) / p.nh)) : "memory");
        return decode_from(e, it);
    };
    // Each fill is a uniform base plus a 32-bit per-lane offset, widened at the use (the empty asm
    // keeps it 32-bit there), so the load takes the scalar-base form with no 64-bit address math.
    auto lds_fill = [&](const char *base, unsigned off, uint16_t *dst) {
        asm volatile("" : "+v"(off));
        __builtin_amdgcn_global_load_lds((const void *)(base + off), (lds_void *)dst, 16, 0, 0);
    };
    // The key tiles' fills with sc0 set (they miss the CU's vector L1 on the way to LDS: each
    // tile is read once per CU, and the fills only pushed other lines out of it). Measured,
    // eight interleaved runs in one call, medians: C1 kernel alone 68.25 -> 67.57 us, step
    // 76.88 -> 76.52 us; C2 unchanged. The same bit on the Q and gate row loads: +1.1 us.
    auto lds_fill_g = [&](const char *base, unsigned off, uint16_t *dst) {
        asm volatile("" : "+v"(off));
        __builtin_amdgcn_global_load_lds((const void *)(base + off), (lds_void *)dst, 16, 0, 1);
    };
    auto load_tiles = [&](const Item &s, int kb, uint16_t *Ks, uint16_t *Vs) {
        const char *kt_base = (const char *)(s.kbase + (size_t)kb * HD);
        const char *vt_base = (const char *)(s.vbase + kb);
#pragma unroll
        for (int j = 0; j < 4; j++) lds_fill_g(kt_base, kfo[j], Ks + (wave_s * 4 + j) * 512);
#pragma unroll
        for (int j = 0; j < 4; j++) lds_fill_g(vt_base, vfo[j], Vs + (wave_s * 4 + j) * 512);
    };
    // Q or gate rows of the block (128 x 256 bf16 = 64 KB, `off` 0 or HD within the head's
    // 2*HD columns): rows 0-63 into G0, 64-127 into G1, slot s of a half = row s/32, 16-byte
    // chunk (s%32) ^ (row & 15).
    auto load_rows = [&](const Item &s, uint16_t *G0, uint16_t *G1, const int off) {
        // An opaque copy of the lane id keeps this address math at each use: hoisted out of the
        // item and tile loops, its 16 per-lane offsets would stay live and spill.
        int ln = lane;
        asm volatile("" : "+v"(ln));
        // wave w loads LDS rows 16w .. 16w + 15, the rows it runs: head slot w / wph, block rows
        // 16 (w mod wph) + [0, 16)
        const int jw = wave_s / s.wph, hw = s.h + min(jw, s.hk - 1), r0w = (wave_s - jw * s.wph) * ROWS;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int grp = wave_s * 8 + j;   // 64-slot group, 0..63
            const int row = grp * 2 + (ln >> 5);
            const int c = (ln & 31) ^ (row & 15);
            int rc = min(r0w + (row & 15), s.nq - 1);
            uint16_t *dst = (grp < 32 ? G0 : G1) + (grp & 31) * 512;
            // the block's rows lie within 128 rows of the head's first: a 32-bit offset
            const char *base = (const char *)(p.qkv + (size_t)s.q_row0 * p.row + (size_t)hw * 2 * HD + off);
            lds_fill(base, (unsigned)(rc * p.row + c * 8) * 2u, dst);
        }
    };
    // the row's rotary cos/sin, written by the K/V prologue for this pass row
    float4 csv[R > 0 ? R : 1][4];
    // Loaded unconditionally (without a table, from the pass's own qkv rows, and not used): a load
    // under a branch made the compiler reshuffle the registers inside it, right after the loads,
    // waiting for them there.
    auto load_cs = [&](const Item &s) {
        if (NROT > 0) {
            const int jw = wave_s / s.wph;
            const int my_q = (wave_s - jw * s.wph) * ROWS + q16;
            const size_t qrow = (size_t)s.q_row0 + (my_q < s.nq ? my_q : 0);
            const float *cs = p.rope_cs ? p.rope_cs + qrow * (NROT / 2) * 2 : (const float *)p.qkv;
#pragma unroll
            for (int c = 0; c < R; c++)
#pragma unroll
                for (int q4 = 0; q4 < 4; q4++) csv[c][q4] = *(const float4 *)(cs + 2 * (c * 32 + 8 * g) + 4 * q4);
        }
    };

    // ---- first item's loads; q_norm (one element per thread) staged in LDS once
    Item cur = decode(item);
    // Buffers of an item: its first key tile arrives in buffer pair `par` (K and V^T buffers of
    // that parity), its Q rows in the other pair, and the tiles alternate from there. The Q rows are issued first, then the rotary
    // cos/sin, then the first tile (8 loads per wave), so the prologue waits for the Q rows alone
    // and rotates them while the tile lands.
    int par = 0;
    {
        // q_norm weights staged with the score scale (scale * log2 e) folded in
        const float qn_w = (p.q_norm && tid < HD) ? p.q_norm[tid] : 0.f;
        const float qn_v = qn_w * p.scale_log2;
        // A normalised, rotated element is at most 16 max|w| (|x_i| / rms <= sqrt(HD) = 16, and
        // the rotation keeps a pair's norm): only weights past f16_lim / 16 (or NaN) can take an
        // element past f16_lim. Each wave stores whether it holds one, after q_norm.
        const int wide = __any(!(fabsf(qn_w) * 16.f <= p.f16_lim)) ? 1 : 0;
        load_rows(cur, k1s, v1s, 0);
        if (cur.n_tiles > 0) load_tiles(cur, 0, k0s, v0s);
        // The LDS stores are issued as asm: the compiler would otherwise wait for the tile's
        // global_load_lds fills (vmcnt(0)) before touching LDS.
        if (tid < HD) asm volatile("ds_write_b32 %0, %1" : : "v"(qn_addr + 4u * tid), "v"(qn_v) : "memory");
        if (lane == 0) asm volatile("ds_write_b32 %0, %1" : : "v"(qn_addr + 4u * (HD + wave)), "v"(wide) : "memory");
    }
    int wide_w = 0;   // some q_norm weight can leave f16's range: check the Q operands elementwise

    for (int k = 0;; k++) {
        // trace row of this item (100 MHz wall clock): start, end, HW_ID, XCC_ID, prologue end,
        // key loop end, workgroup, ordinal within the workgroup
        uint64_t *const tr = (p.trace && tid == 0 && ((item >> kItemBits) & 3) != 2) ? p.trace + 8 * (size_t)item_base(item) : nullptr;
        if (tr) {
            tr[0] = wall_clock64();
            tr[2] = __builtin_amdgcn_s_getreg((31 << 11) | 4);
            tr[3] = __builtin_amdgcn_s_getreg((15 << 11) | 20);
            tr[6] = blockIdx.x;
            tr[7] = k;
        }
        // this wave's head and rows in the item (one head on all waves but in a packed item)
        const int jw = wave_s / cur.wph, row0w = (wave_s - jw * cur.wph) * ROWS, my_h = cur.h + jw;
        const int my_q = row0w + q16;
        const bool q_valid = jw < cur.hk && my_q < cur.nq;
        const int qpos = cur.q_pos0 + my_q;
        const bool wave_live = jw < cur.hk && row0w < cur.nq;
        const int wave_last_pos = cur.q_pos0 + row0w + ROWS - 1;
        const int k_len = cur.k_len, n_tiles = cur.n_tiles;

        // The rotary cos/sin load here, at the item's start: they are first needed after the
        // normalisation, and loaded in the previous item's epilogue, the compiler's moves of
        // their registers at the loop's back edge waited there for the Q-row fills just issued.
        load_cs(cur);
        // ---- Q prologue: lane holds Q[my_q][c*32 + 8g + j], the B operand of chunk c.
        f16x8 qf[NC];
        const int nxt = items.get(k + 1);
        i32x8 ne;
        {
            // the Q rows and q_norm are in LDS once the first tile's 8 loads are all that remain
            if (cur.n_tiles > 0) asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory");
            else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
            // addresses from an opaque lane id, so that they are not hoisted out of the item loop
            int ln = lane;
            asm volatile("" : "+v"(ln));
            const int mq = wave_s * ROWS + (ln & 15), gg = ln >> 4;
            u32x4 qw[NC];
            {
                const uint16_t *qr = (mq < 64 ? (par ? k0s : k1s) : (par ? v0s : v1s)) + (mq & 63) * 256;
#pragma unroll
                for (int c = 0; c < NC; c++) qw[c] = *(const u32x4 *)(qr + (((4 * c + gg) ^ (mq & 15)) * 8));
            }
            float x[NC][8];
            float ss = 0.f;
#pragma unroll
            for (int c = 0; c < NC; c++) {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    x[c][2 * j] = bf_lo(qw[c][j]);
                    x[c][2 * j + 1] = bf_hi(qw[c][j]);
                }
#pragma unroll
                for (int j = 0; j < 8; j++) ss += x[c][j] * x[c][j];
            }
            ss = xrow_sum(ss);
            if (p.q_norm && k == 0) {   // the waves' wide-weight words, once per workgroup
                u32x4 f0, f1;
                asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %2 offset:16\n\ts_waitcnt lgkmcnt(0)"
                             : "=&v"(f0), "=&v"(f1) : "v"(qn_addr + 4u * HD) : "memory");
                wide_w = __builtin_amdgcn_readfirstlane((int)(f0[0] | f0[1] | f0[2] | f0[3] | f1[0] | f1[1] | f1[2] | f1[3]));
            }
            if (p.q_norm) {   // NULL: no q/k norm (plain SDPA operands)
                const float inv = rsqrtf(ss / (float)HD + p.eps);
#pragma unroll
                for (int c = 0; c < NC; c++) {
                    // both reads and their wait in one statement: nothing can touch the
                    // registers while the reads are in flight
                    bf16x8 r0, r1;
                    asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %2 offset:16\n\ts_waitcnt lgkmcnt(0)"
                                 : "=&v"(r0), "=&v"(r1) : "v"(qn_addr + 4u * (c * 32 + 8 * gg)) : "memory");
                    const float4 w0 = __builtin_bit_cast(float4, r0), w1 = __builtin_bit_cast(float4, r1);
                    const float wn[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
                    for (int j = 0; j < 8; j++) x[c][j] = x[c][j] * inv * wn[j];
                }
            }
            if (NROT > 0) {
                // NeoX partial rotary: pair (i, i + NROT/2) sits in this lane at chunks c and c + R.
                // Interleaved M-RoPE: pair i turns by axis i % 3 of pos3.
                if (p.rope_cs) {
#pragma unroll
                    for (int c = 0; c < R; c++) {
                        const float t[16] = {csv[c][0].x, csv[c][0].y, csv[c][0].z, csv[c][0].w,
                                             csv[c][1].x, csv[c][1].y, csv[c][1].z, csv[c][1].w,
                                             csv[c][2].x, csv[c][2].y, csv[c][2].z, csv[c][2].w,
                                             csv[c][3].x, csv[c][3].y, csv[c][3].z, csv[c][3].w};
#pragma unroll
                        for (int j = 0; j < 8; j++) {
                            const float cs_ = t[2 * j], sn = t[2 * j + 1];
                            const float x0 = x[c][j], x1 = x[c + R][j];
                            x[c][j] = x0 * cs_ - x1 * sn;
                            x[c + R][j] = x1 * cs_ + x0 * sn;
                        }
                    }
                } else {
                    const size_t qrow = (size_t)cur.q_row0 + (q_valid ? my_q : 0);
                    const int32_t *pp = p.pos3 + 3 * qrow;
                    const float pt = (float)pp[0], ph = (float)pp[1], pw = (float)pp[2];
#pragma unroll
                    for (int c = 0; c < R; c++) {
                        const float4 f0 = *(const float4 *)(p.inv_freq + c * 32 + 8 * g);
                        const float4 f1 = *(const float4 *)(p.inv_freq + c * 32 + 8 * g + 4);
                        const float fr[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
#pragma unroll
                        for (int j = 0; j < 8; j++) {
                            const int i = c * 32 + 8 * g + j;
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
            }
            // Scaled by scale * log2 e before the one rounding to f16: the products give scores in
            // the exp2 domain. The f16 operand follows split16 (metal/clef.metal:857-867): an
            // element with |q| > f16_lim or NaN flags the record, and the operand saturates.
            // Normalised rows are bounded by 16 max|w|: unless a weight is that large, only a row
            // that is not finite (its sum of squares) can flag, and only then do the wave's rows
            // take the elementwise check. Plain rows are always checked element by element (the
            // largest magnitude's bits, which order NaN above every number) and clamped.
            const float sc = p.scale_log2;
            bool q_bad;
            auto pack_checked = [&](const float mul, const float lim) {
                unsigned amax = 0;
#pragma unroll
                for (int c = 0; c < NC; c++) {
                    float y[8];
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        amax = max(amax, __float_as_uint(x[c][j]) & 0x7fffffffu);
                        y[j] = __builtin_amdgcn_fmed3f(x[c][j] * mul, -65504.f, 65504.f);
                    }
                    u32x4 w = {pack_f16(y[0], y[1]), pack_f16(y[2], y[3]), pack_f16(y[4], y[5]), pack_f16(y[6], y[7])};
                    qf[c] = __builtin_bit_cast(f16x8, w);
                }
                return amax > __float_as_uint(lim);
            };
            if (p.q_norm) {   // the scale came in with the staged weights
                q_bad = !(ss <= 3.0e38f);
                if (wide_w || __any(q_bad)) {
                    q_bad = pack_checked(1.f, p.f16_lim * sc) || q_bad;
                } else {
#pragma unroll
                    for (int c = 0; c < NC; c++) {
                        u32x4 w = {pack_f16(x[c][0], x[c][1]), pack_f16(x[c][2], x[c][3]),
                                   pack_f16(x[c][4], x[c][5]), pack_f16(x[c][6], x[c][7])};
                        qf[c] = __builtin_bit_cast(f16x8, w);
                    }
                }
            } else {
                q_bad = pack_checked(sc, p.f16_lim);
            }
            if (q_bad && q_valid && p.ovf)
                __hip_atomic_store(p.ovf + cur.flag_row, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }

        f32x4 o[16];
#pragma unroll
        for (int mt = 0; mt < 16; mt++) o[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
        float m_run = -INFINITY, l_run = 0.f, msub = 0.f;   // msub: where the S accumulators start (-msub)
        // Every wave has read its Q rows (the second tile may take their buffers) and the first
        // tile has landed. The next item's block entry loads during this wait.
        if (nxt >= 0)
            asm volatile("s_load_dwordx8 %0, %1, 0x0\n\ts_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier"
                         : "=s"(ne) : "s"(p.blocks + 8 * (item_base(nxt) / p.nh)) : "memory");
        else
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (tr) tr[4] = wall_clock64();
        auto zero_tail = [&](int kb, uint16_t *Vs) {   // V^T entries of keys >= k_len -> 0
            const int valid = k_len - kb;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int s = tid + 512 * j;
                const int d = s >> 3, c = (s & 7) ^ v_swz(d);
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
        // Two tiles per trip: each call names its read and fill buffers statically.
        auto tile = [&](const int t, auto BUF) {
            constexpr int buf = decltype(BUF)::value;
            uint16_t *const Vs = buf ? v1s : v0s, *const Kn = buf ? k0s : k1s, *const Vn = buf ? v0s : v1s;
            const int kb = t * BK;
            if (kb + BK > k_len) {   // WG-uniform: the block's last tile
                zero_tail(kb, Vs);
                __syncthreads();
            }
            if (t + 1 < n_tiles) load_tiles(cur, kb + BK, Kn, Vn);
            else if (p.gate) load_rows(cur, Kn, Vn, HD);   // the idle buffers take the epilogue's gate rows
            if (wave_live && (!p.causal || kb <= wave_last_pos)) {
                // S^T: 32 MFMAs (4 key tiles x 8 dim chunks), chunk-major so consecutive products
                // go to different accumulators. K operands are read DEPTH steps ahead of their
                // product so the LDS latency overlaps the matrix work.
                constexpr int DEPTH = 8, QK = 4 * NC;
                f32x4 s[4];
                bf16x8 ring[DEPTH];
                static_for<DEPTH>([&](auto I) {
                    constexpr int st = decltype(I)::value, kt = st & 3, c = st >> 2;
                    ring[st] = lds_read16<buf * 2 * KTILE + (c >> 2) * 256>(ka[kt][c & 3]);
                });
                // steps in pairs: one wait covers both operands (reads are issued up to step
                // 2p + DEPTH - 1 when pair p's wait runs)
                static_for<QK / 4>([&](auto P) {
                    constexpr int st = 4 * decltype(P)::value;
                    constexpr int last = (st + DEPTH - 1) < (QK - 1) ? (st + DEPTH - 1) : (QK - 1);
                    bf16x8 a[4] = {ring[st % DEPTH], ring[(st + 1) % DEPTH], ring[(st + 2) % DEPTH], ring[(st + 3) % DEPTH]};
                    lds_wait4<last - (st + 3)>(a[0], a[1], a[2], a[3]);
                    static_for<4>([&](auto H) {
                        constexpr int sp = st + decltype(H)::value, kt = sp & 3, c = sp >> 2;
                        if constexpr (c == 0) s[kt] = f32x4{-msub, -msub, -msub, -msub};
                        s[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a[decltype(H)::value]), qf[c], s[kt], 0, 0, 0);
                    });
                    static_for<4>([&](auto H) {
                        constexpr int n = st + decltype(H)::value + DEPTH, nkt = n & 3, nc = n >> 2;
                        if constexpr (n < QK)
                            ring[(st + decltype(H)::value) % DEPTH] = lds_read16<buf * 2 * KTILE + (nc >> 2) * 256>(ka[nkt][nc & 3]);
                    });
                });
                // first V operands, in flight during the softmax
                auto vread = [&](auto I) {   // step st = 16 * kc + mt
                    constexpr int st = decltype(I)::value, mt = st & 15, kc = st >> 4;
                    constexpr int off = buf * 2 * VTILE + (32 * (mt >> 1) + 4 * (mt & 1)) * BK * 2;
                    return lds_read16<off>(kc ? va1 : va0);
                };
                bf16x8 vring[DEPTH];
                static_for<DEPTH>([&](auto I) { vring[decltype(I)::value] = vread(I); });
                // Online softmax in the exp2 domain. Masked scores are -inf, so their P is an exact
                // zero and a tile past a row's diagonal rescales the row by exactly 1.
                if ((kb + BK > k_len) || (p.causal && kb + BK - 1 > cur.q_pos0 + row0w)) {
                    // element (kt, i) is key kb + 32(kt>>1) + 8g + 4(kt&1) + i
                    const int lim = min(k_len - 1, p.causal ? qpos : k_len - 1) - kb - 8 * g;
#pragma unroll
                    for (int kt = 0; kt < 4; kt++)
#pragma unroll
                        for (int i = 0; i < 4; i++)
                            s[kt][i] = (32 * (kt >> 1) + 4 * (kt & 1) + i > lim) ? -INFINITY : s[kt][i];
                }
                // s holds the score minus the running max (exp2 domain). The max moves only when a
                // tile's max passes it by more than 8, or on the row's first tile: P stays below
                // 2^8, and the shift and the O rescale below run on few tiles. The lane's own max
                // decides whether any row of the wave may move; only then is the row max reduced
                // over the row's four lanes.
                float mx = -INFINITY;
#pragma unroll
                for (int kt = 0; kt < 4; kt++)
                    mx = __builtin_elementwise_maximum(__builtin_elementwise_maximum(mx, __builtin_elementwise_maximum(s[kt][0], s[kt][1])),
                                                       __builtin_elementwise_maximum(s[kt][2], s[kt][3]));
                float alpha = 1.f;
                if (__any(mx > 8.f || m_run == -INFINITY)) {
                    const float rmx = xrow_max(mx);
                    const float d = (m_run == -INFINITY || rmx > 8.f) ? (rmx == -INFINITY ? 0.f : rmx) : 0.f;
                    alpha = (m_run == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(-d);
                    m_run = (m_run == -INFINITY) ? (rmx == -INFINITY ? -INFINITY : d) : m_run + d;
                    msub = m_run == -INFINITY ? 0.f : m_run;
#pragma unroll
                    for (int kt = 0; kt < 4; kt++) s[kt] -= d;
                }
                float rs = 0.f;
                bf16x8 pk[2];
#pragma unroll
                for (int kc = 0; kc < 2; kc++) {
                    unsigned w[4];
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int kt = 2 * kc + (j >> 1), i = 2 * (j & 1);
                        w[j] = pack_bf16(__builtin_amdgcn_exp2f(s[kt][i]), __builtin_amdgcn_exp2f(s[kt][i + 1]));
                        // the row sum takes the rounded P that the PV product multiplies
                        rs = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w[j]),
                                                             bf16x2{(__bf16)1.0f, (__bf16)1.0f}, rs, false);
                    }
                    u32x4 wv = {w[0], w[1], w[2], w[3]};
                    pk[kc] = __builtin_bit_cast(bf16x8, wv);
                }
                l_run = l_run * alpha + rs;   // the lane's share; the row's four lanes add up at the end
                if (__any(alpha != 1.f)) {
#pragma unroll
                    for (int mt = 0; mt < 16; mt++) o[mt] *= alpha;
                }
                static_for<8>([&](auto P) {   // O^T: 32 MFMAs over 16 rotating accumulators, same read-ahead, in fours
                    constexpr int st = 4 * decltype(P)::value;
                    constexpr int last = (st + DEPTH - 1) < 31 ? (st + DEPTH - 1) : 31;
                    bf16x8 a[4] = {vring[st % DEPTH], vring[(st + 1) % DEPTH], vring[(st + 2) % DEPTH], vring[(st + 3) % DEPTH]};
                    lds_wait4<last - (st + 3)>(a[0], a[1], a[2], a[3]);
                    static_for<4>([&](auto H) {
                        constexpr int sp = st + decltype(H)::value, mt = sp & 15, kc = sp >> 4;
                        o[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[decltype(H)::value], pk[kc], o[mt], 0, 0, 0);
                    });
                    static_for<4>([&](auto H) {
                        constexpr int n = st + decltype(H)::value + DEPTH;
                        if constexpr (n < 32) vring[(st + decltype(H)::value) % DEPTH] = vread(std::integral_constant<int, n>{});
                    });
                });
            }
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
        };
        if (par == 0) {
            for (int t = 0; t < n_tiles; t += 2) {
                tile(t, std::integral_constant<int, 0>{});
                if (t + 1 < n_tiles) tile(t + 1, std::integral_constant<int, 1>{});
            }
        } else {
            for (int t = 0; t < n_tiles; t += 2) {
                tile(t, std::integral_constant<int, 1>{});
                if (t + 1 < n_tiles) tile(t + 1, std::integral_constant<int, 0>{});
            }
        }
        if (tr) tr[5] = wall_clock64();

        // ---- Epilogue: O / l times sigmoid(gate); lane (q16, g) holds dims 32u + 8g + [0, 8).
        // The gate rows sit in the buffers the last tile left idle. The next item's Q rows and
        // rotary cos/sin load before the gate work, its Q rows into the buffers the last tile used
        // (every wave left that tile at its closing barrier); its first tile goes into the gate's
        // buffers once every wave has read its gate values.
        const float l_row = xrow_sum(l_run);   // outside the row-divergent branch: lanes exchange values
        const int last_buf = (par + n_tiles + 1) & 1;
        const int gate_buf = last_buf ^ 1;
        const int q_row0 = cur.q_row0, flag_row = cur.flag_row, h = my_h, hk_done = cur.hk;
        item = nxt;
        if (item >= 0) {
            cur = decode_from(ne, item);
            if (last_buf) load_rows(cur, k1s, v1s, 0);
            else load_rows(cur, k0s, v0s, 0);
        }
        if (q_valid) {
            const float il = l_row > 0.f ? 1.f / l_row : 0.f;
            const size_t t = (size_t)q_row0 + my_q;
            int32_t *flag = p.ovf ? p.ovf + flag_row : nullptr;
            // Gate chunks come two at a time, both reads and their wait in one statement, so
            // nothing can copy their registers while the reads are in flight (split into a read
            // and a later wait, the compiler moved ring registers between the two), and the wait
            // is for LDS alone, not for the next item's loads in flight.
            int ln = lane;
            asm volatile("" : "+v"(ln));
            const int mq = wave_s * ROWS + (ln & 15), gg = ln >> 4;
            const unsigned gbase = lds_addr(gate_buf ? k1s : k0s) + (mq < 64 ? 0u : 2u * 2 * KTILE) + (unsigned)(mq & 63) * 512u;
            auto gaddr = [&](int u) { return gbase + (unsigned)(((4 * u + gg) ^ (mq & 15)) * 16); };
            u32x4 gq[2];
            static_for<8>([&](auto U) {
                constexpr int u = decltype(U)::value;
                const int d0 = 32 * u + 8 * g;
                float v[8];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    v[i] = o[2 * u][i];
                    v[4 + i] = o[2 * u + 1][i];
                }
                if (p.gate) {
                    if constexpr ((u & 1) == 0)
                        asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %3\n\ts_waitcnt lgkmcnt(0)"
                                     : "=&v"(gq[0]), "=&v"(gq[1]) : "v"(gaddr(u)), "v"(gaddr(u + 1)) : "memory");
                    const u32x4 gw = gq[u & 1];
                    // O / l * sigmoid(g) = O / (l + l * 2^(-g log2 e)): one reciprocal per element
                    // (a row's l is at least 1: its own key's P is 2^0 at the running max)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        v[2 * j] *= __builtin_amdgcn_rcpf(fmaf(l_row, __builtin_amdgcn_exp2f(-bf_lo(gw[j]) * 1.4426950408889634f), l_row));
                        v[2 * j + 1] *= __builtin_amdgcn_rcpf(fmaf(l_row, __builtin_amdgcn_exp2f(-bf_hi(gw[j]) * 1.4426950408889634f), l_row));
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 8; i++) v[i] *= il;
                }
                store_out8(p.out, t * p.out_ld + (size_t)h * HD + d0, v, p.out_type, p.f16_lim, flag);
            });
        }
        if (item >= 0) {
            // every wave has read its gate values (each read waited for): their buffers are free.
            // A bare barrier: a fence would also wait for the stores and the fills in flight.
            __builtin_amdgcn_s_barrier();
            if (cur.n_tiles > 0) {
                if (gate_buf) load_tiles(cur, 0, k1s, v1s);
                else load_tiles(cur, 0, k0s, v0s);
            }
            par = gate_buf;
        }
        if (tr) {
            tr[1] = wall_clock64();
            // the other heads of a packed item get the same row
            for (int j = 1; j < hk_done; j++)
                for (int i = 0; i < 8; i++) tr[8 * j + i] = tr[i];
        }
        if (item < 0) break;
    }
}

// Grid: G workgroups; workgroup b runs the items ItemList assigns it (one each when G is the
// item count, several when G is the CU count).
template <int NROT>
__global__ __launch_bounds__(512, 1) void attn_text_kernel(AttnParams p) {
    __shared__ __attribute__((aligned(16))) uint16_t smem[text::LDS_ELEMS];
    __shared__ __attribute__((aligned(16))) float qn_lds[text::HD + 8];   // q_norm, then a word per wave
    text_items<NROT>(p, smem, qn_lds);
}

}  // namespace clef_hip
