/* Host-side harness for an AddressSanitizer build of libclef_hip_attn.so (tests/test_host_asan.py):
 * drives every host-only entry point (plans, schedules, positions, packing, prefix capacity, the
 * GGUF reader) over seeded random and edge-case inputs, with every output buffer allocated at
 * exactly the size the API documents, so a write or read past it is reported. No GPU call is made.
 * argv[1..]: GGUF files to open, the first well-formed (its tensors must all resolve by name),
 * the rest truncated or corrupted; each must open or fail cleanly. Prints "ok <checks>" on success; any failed expectation exits 1. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "clef_hip_attn.h"

static unsigned long long rng = 0x9e3779b97f4a7c15ULL;
static unsigned rnd(void) {
    rng ^= rng << 13;
    rng ^= rng >> 7;
    rng ^= rng << 17;
    return (unsigned)(rng >> 11);
}
static long checks = 0;
#define EXPECT(c, ...)                                  \
    do {                                                \
        checks++;                                       \
        if (!(c)) {                                     \
            fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
            fprintf(stderr, __VA_ARGS__);               \
            fputc('\n', stderr);                        \
            exit(1);                                    \
        }                                               \
    } while (0)

static int32_t *imalloc(size_t n) { return (int32_t *)malloc((n ? n : 1) * sizeof(int32_t)); }

/* plan + schedule of one pass; cu_k NULL for a fresh pass */
static void plan_case(const int32_t *cu_q, const int32_t *cu_k, int n_seq, int causal, int nh, int nkv) {
    char err[256];
    const int Tq = cu_q[n_seq];
    const int maxb = clef_hip_attn_plan_max_blocks(n_seq, Tq);
    EXPECT(maxb >= 0, "max_blocks %d", maxb);
    int32_t *blocks = imalloc((size_t)maxb * 8), *tok_kv = imalloc((size_t)Tq);
    int n_blk = -1, kv_rows = -1;
    /* kv_rows first (kv_tok NULL), then the inverse map at exactly that size */
    bool ok = clef_hip_attn_plan(cu_q, cu_k, n_seq, causal, blocks, maxb, tok_kv, Tq, NULL, 0, &n_blk, &kv_rows, err, sizeof err);
    EXPECT(ok, "plan: %s", err);
    EXPECT(n_blk >= 0 && n_blk <= maxb && kv_rows >= 0, "n_blk %d kv_rows %d", n_blk, kv_rows);
    int32_t *kv_tok = imalloc((size_t)kv_rows);
    ok = clef_hip_attn_plan(cu_q, cu_k, n_seq, causal, blocks, maxb, tok_kv, Tq, kv_tok, kv_rows, &n_blk, &kv_rows, err, sizeof err);
    EXPECT(ok, "plan with kv_tok: %s", err);
    for (int t = 0; t < Tq; t++) EXPECT(tok_kv[t] >= 0 && tok_kv[t] < kv_rows && kv_tok[tok_kv[t]] == t, "kv map at %d", t);
    /* a block list one entry short must be refused, not overrun */
    if (n_blk > 0) {
        int32_t *small = imalloc((size_t)(n_blk - 1) * 8);
        int nb2 = 0, kr2 = 0;
        EXPECT(!clef_hip_attn_plan(cu_q, cu_k, n_seq, causal, small, n_blk - 1, tok_kv, Tq, NULL, 0, &nb2, &kr2, err, sizeof err),
               "undersized block list accepted");
        free(small);
    }
    const int wgs[3] = {1, 8, 256};
    for (int i = 0; i < 3 && n_blk > 0; i++) {
        const int n_wg = wgs[i];
        const int sz = clef_hip_attn_sched_size(n_blk, nh, n_wg);
        EXPECT(sz > 0, "sched_size %d", sz);
        int32_t *sched = imalloc((size_t)sz);
        ok = clef_hip_attn_schedule(blocks, n_blk, nh, nkv, n_wg, sched, sz, err, sizeof err);
        EXPECT(ok, "schedule: %s", err);
        /* every (block, head) covered once by the items' rows (codes 0-3) */
        /* header {magic, n_blk, nh, n_wg, nkv, fingerprint of the block list (word 7 of every
           block entry), 0, 0}, then the offsets */
        EXPECT(sched[0] == 0x53434844 && sched[1] == n_blk && sched[2] == nh && sched[3] == n_wg && sched[4] == nkv &&
               sched[5] == blocks[7] && sched[5] != 0, "sched header");
        const int32_t *offs = sched + 8;
        EXPECT(offs[0] == 0 && offs[n_wg] <= sz - 8 - n_wg - 1, "sched offsets");
        free(sched);
        int32_t *tiny = imalloc(4);
        EXPECT(!clef_hip_attn_schedule(blocks, n_blk, nh, nkv, n_wg, tiny, 4, err, sizeof err), "tiny schedule accepted");
        free(tiny);
    }
    free(blocks);
    free(tok_kv);
    free(kv_tok);
}

static void plans(void) {
    char err[256];
    for (int it = 0; it < 400; it++) {
        const int n_seq = (int)(rnd() % 40);
        int32_t *cu_q = imalloc((size_t)n_seq + 1), *cu_k = imalloc((size_t)n_seq + 1);
        cu_q[0] = cu_k[0] = 0;
        for (int r = 0; r < n_seq; r++) {
            const int len = (rnd() % 5 == 0) ? 1 + (int)(rnd() % 3) : (int)(rnd() % 400) + 1;
            cu_q[r + 1] = cu_q[r] + len;
            const int cached = (rnd() % 2) ? (int)(rnd() % 700) : 0;
            cu_k[r + 1] = cu_k[r] + ((len + cached + 7) / 8) * 8;   /* room for the keys, multiple of 8 */
            (void)cached;
        }
        const int causal = (int)(rnd() % 2);
        const int nkv = 1 + (int)(rnd() % 4), nh = nkv * (1 + (int)(rnd() % 6));
        plan_case(cu_q, NULL, n_seq, causal, nh, nkv);
        /* prefix passes: queries are the last tokens of each record's keys */
        int32_t *cu_kp = imalloc((size_t)n_seq + 1);
        cu_kp[0] = 0;
        for (int r = 0; r < n_seq; r++) {
            const int nq = cu_q[r + 1] - cu_q[r];
            const int nk = nq + 8 * (int)(rnd() % 64);
            cu_kp[r + 1] = cu_kp[r] + ((nk + 7) / 8) * 8;
        }
        plan_case(cu_q, cu_kp, n_seq, 1, nh, nkv);
        free(cu_kp);
        free(cu_q);
        free(cu_k);
    }
    /* refused inputs: decreasing bounds, a negative record count, keys fewer than queries */
    int32_t bad[3] = {0, 10, 5}, blocks[64 * 8], tok[16], nb, kr;
    EXPECT(!clef_hip_attn_plan(bad, NULL, 2, 1, blocks, 64, tok, 16, NULL, 0, &nb, &kr, err, sizeof err), "decreasing cu_q accepted");
    EXPECT(!clef_hip_attn_plan(bad, NULL, -1, 1, blocks, 64, tok, 16, NULL, 0, &nb, &kr, err, sizeof err), "negative n_seq accepted");
    int32_t q[2] = {0, 16}, k[2] = {0, 8};
    EXPECT(!clef_hip_attn_plan(q, k, 1, 1, blocks, 64, tok, 16, NULL, 0, &nb, &kr, err, sizeof err), "fewer keys than queries accepted");
}

static void omni_plans(void) {
    char err[256];
    for (int it = 0; it < 200; it++) {
        const int n_seq = 1 + (int)(rnd() % 20);
        int32_t *cu = imalloc((size_t)n_seq + 1);
        cu[0] = 0;
        for (int r = 0; r < n_seq; r++) cu[r + 1] = cu[r] + 1 + (int)(rnd() % 300);
        const int maxb = clef_hip_omni_plan_max_blocks(n_seq, cu[n_seq]);
        int32_t *blocks = imalloc((size_t)maxb * 8);
        int n_blk = -1;
        EXPECT(clef_hip_omni_plan(cu, n_seq, blocks, maxb, &n_blk, err, sizeof err), "omni plan: %s", err);
        EXPECT(n_blk > 0 && n_blk <= maxb, "omni n_blk %d", n_blk);
        free(blocks);
        free(cu);
    }
}

static void positions_and_packing(void) {
    char err[256];
    for (int it = 0; it < 300; it++) {
        /* text + image spans of one record */
        const int merge = 2, n_spans = (int)(rnd() % 4);
        int32_t st[4], gh[4], gw[4];
        int T = (int)(rnd() % 20);
        for (int i = 0; i < n_spans; i++) {
            st[i] = T;
            gh[i] = 2 * (1 + (int)(rnd() % 8));
            gw[i] = 2 * (1 + (int)(rnd() % 8));
            T += (gh[i] / merge) * (gw[i] / merge) + (int)(rnd() % 10);
        }
        int32_t *pos3 = imalloc((size_t)T * 3);
        EXPECT(clef_hip_record_positions(T, NULL, st, gh, gw, n_spans, merge, pos3, err, sizeof err), "positions: %s", err);
        free(pos3);
        /* vision patch positions of a few images */
        const int n_img = 1 + (int)(rnd() % 4);
        int32_t cu[5], gws[4];
        cu[0] = 0;
        for (int i = 0; i < n_img; i++) {
            const int h = 2 * (1 + (int)(rnd() % 6)), w = 2 * (1 + (int)(rnd() % 6));
            gws[i] = w;
            cu[i + 1] = cu[i] + h * w;
        }
        int32_t *pos2 = imalloc((size_t)cu[n_img] * 2);
        EXPECT(clef_hip_vis_positions(cu, n_img, gws, 2, pos2, err, sizeof err), "vis positions: %s", err);
        free(pos2);
        /* packing of a queue */
        const int n_queue = (int)(rnd() % 30);
        int32_t *len = imalloc((size_t)n_queue);
        uint8_t *keyed = (uint8_t *)malloc((size_t)n_queue + 1);
        for (int i = 0; i < n_queue; i++) {
            len[i] = 1 + (int)(rnd() % 2000);
            keyed[i] = rnd() % 7 == 0;
        }
        const int max_batch = 1 + (int)(rnd() % 8);
        int32_t *cus = imalloc((size_t)max_batch + 1);
        const int n = clef_hip_pack_batch(len, keyed, n_queue, max_batch, 4096, cus);
        EXPECT(n >= 0 && n <= max_batch && n <= n_queue && (n_queue == 0 || n >= 1), "pack_batch %d", n);
        free(len);
        free(keyed);
        free(cus);
    }
    EXPECT(clef_hip_prefix_capacity(-1, 0, 256) == -1, "negative rows");
    EXPECT(clef_hip_prefix_capacity(100, 0, 256) == 1024, "first capacity");
    EXPECT(clef_hip_prefix_capacity(0x7fffffff, 0, 256) == -1, "capacity past 32-bit offsets");
    float inv[64];
    clef_hip_rope_inv_freq(1e7f, 64, inv);
    EXPECT(inv[0] == 1.0f, "inv_freq[0]");
}

static void gguf_file(const char *path, int strict) {
    char err[256];
    clef_hip_gguf *g = NULL;
    if (!clef_hip_gguf_open(path, &g, err, sizeof err)) {
        EXPECT(err[0] != 0, "failed open without a message (%s)", path);
        return;
    }
    const int n = clef_hip_gguf_tensor_count(g);
    char name[64];
    for (int i = 0; i < n; i++) {
        clef_hip_gguf_tensor_info info;
        if (clef_hip_gguf_tensor_at(g, i, &info, name, sizeof name)) {
            EXPECT(strlen(name) < sizeof name, "name not terminated");
            /* touch the first and last data byte through the mapping */
            if (info.nbytes) {
                volatile const uint8_t *d = (const uint8_t *)info.data;
                (void)d[0];
                (void)d[info.nbytes - 1];
            }
            clef_hip_gguf_tensor_info again;
            const bool found = clef_hip_gguf_find_tensor(g, name, &again);
            /* a corrupted file may hold a NUL inside a name; the well-formed one must resolve */
            EXPECT(found || !strict || strlen(name) == sizeof name - 1, "find %s", name);
        }
    }
    uint32_t u;
    float f;
    (void)clef_hip_gguf_get_u32(g, "clef.block_count", &u);
    (void)clef_hip_gguf_get_f32(g, "clef.rope.freq_base", &f);
    clef_hip_attn_config c;
    (void)clef_hip_gguf_attn_config(g, &c, err, sizeof err);
    clef_hip_gguf_close(g);
}

int main(int argc, char **argv) {
    plans();
    omni_plans();
    positions_and_packing();
    for (int i = 1; i < argc; i++) gguf_file(argv[i], i == 1);
    printf("ok %ld\n", checks);
    return 0;
}
