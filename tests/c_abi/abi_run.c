/* A C caller of the prefill path, built against include/clef_hip_attn.h and linked with
 * libclef_hip_attn.so the way the engine would link it: plan -> prefill on a small packed pass,
 * twice (without and with a host schedule), results written for tests/test_c_abi.py to check
 * against the oracle.
 *
 * usage: abi_run <dir>   reads <dir>/qkv.bin (bf16 [T][row]), qn.bin, kn.bin (f32 [256]),
 *                        pos3.bin (int32 [T][3]); writes <dir>/out.bin and out_sched.bin (bf16
 *                        [T][nh*256]). Shapes are fixed below. Exit status 0 on success. */
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "clef_hip_attn.h"

enum { NH = 8, NKV = 2, HD = 256, NROT = 64, NSEQ = 4 };
static const int32_t CU[NSEQ + 1] = {0, 37, 101, 102, 232};

static int die(const char *what, const char *err) {
    fprintf(stderr, "abi_run: %s: %s\n", what, err ? err : "");
    return 1;
}

static void *load(const char *dir, const char *name, size_t bytes) {
    char path[512];
    snprintf(path, sizeof path, "%s/%s", dir, name);
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    void *p = malloc(bytes);
    const size_t got = fread(p, 1, bytes, f);
    fclose(f);
    if (got != bytes) {
        free(p);
        return NULL;
    }
    return p;
}

static int save(const char *dir, const char *name, const void *p, size_t bytes) {
    char path[512];
    snprintf(path, sizeof path, "%s/%s", dir, name);
    FILE *f = fopen(path, "wb");
    if (!f) return 0;
    const size_t put = fwrite(p, 1, bytes, f);
    fclose(f);
    return put == bytes;
}

#define CK(x)                                                     \
    do {                                                          \
        hipError_t e_ = (x);                                      \
        if (e_ != hipSuccess) return die(#x, hipGetErrorString(e_)); \
    } while (0)

int main(int argc, char **argv) {
    if (argc != 2) return die("usage", "abi_run <dir>");
    const char *dir = argv[1];
    const int T = CU[NSEQ], row = 2 * NH * HD + 2 * NKV * HD;
    char err[256] = {0};
    uint16_t *qkv = load(dir, "qkv.bin", (size_t)T * row * 2);
    float *qn = load(dir, "qn.bin", HD * 4), *kn = load(dir, "kn.bin", HD * 4);
    int32_t *pos3 = load(dir, "pos3.bin", (size_t)T * 3 * 4);
    if (!qkv || !qn || !kn || !pos3) return die("inputs", dir);
    if (!clef_hip_attn_init(err, sizeof err)) return die("init", err);

    /* the plan, on the host */
    const int max_blk = clef_hip_attn_plan_max_blocks(NSEQ, T);
    int32_t *blocks = calloc((size_t)max_blk * CLEF_HIP_BLOCK_INTS, 4), *tok_kv = calloc(T, 4);
    const int max_kv = T + 64 * NSEQ + 64;
    int32_t *kv_tok = calloc(max_kv, 4), *seq_start = calloc(T, 4);
    int n_blk = 0, kv_rows = 0;
    if (!clef_hip_attn_plan(CU, NULL, NSEQ, 1, blocks, max_blk, tok_kv, T, kv_tok, max_kv, &n_blk, &kv_rows,
                            err, sizeof err))
        return die("plan", err);
    for (int r = 0; r < NSEQ; r++)
        for (int t = CU[r]; t < CU[r + 1]; t++) seq_start[t] = CU[r];
    const int kvT = (kv_rows + 7) / 8 * 8;
    float inv_freq[NROT / 2];
    clef_hip_rope_inv_freq(1e7f, NROT, inv_freq);

    /* device buffers */
    void *d_qkv, *d_qn, *d_kn, *d_pos, *d_inv, *d_cs, *d_k, *d_vt, *d_blk, *d_kvtok, *d_tokkv, *d_ss, *d_out, *d_ovf;
    CK(hipMalloc(&d_qkv, (size_t)T * row * 2));
    CK(hipMalloc(&d_qn, HD * 4));
    CK(hipMalloc(&d_kn, HD * 4));
    CK(hipMalloc(&d_pos, (size_t)T * 12));
    CK(hipMalloc(&d_inv, sizeof inv_freq));
    CK(hipMalloc(&d_cs, (size_t)T * NROT * 4));
    CK(hipMalloc(&d_k, (size_t)NKV * kvT * HD * 2));
    CK(hipMalloc(&d_vt, (size_t)NKV * kvT * HD * 2));
    CK(hipMalloc(&d_blk, (size_t)n_blk * CLEF_HIP_BLOCK_INTS * 4));
    CK(hipMalloc(&d_kvtok, (size_t)kv_rows * 4));
    CK(hipMalloc(&d_tokkv, (size_t)T * 4));
    CK(hipMalloc(&d_ss, (size_t)T * 4));
    CK(hipMalloc(&d_out, (size_t)T * NH * HD * 2));
    CK(hipMalloc(&d_ovf, (size_t)T * 4));
    CK(hipMemcpy(d_qkv, qkv, (size_t)T * row * 2, hipMemcpyHostToDevice));
    CK(hipMemcpy(d_qn, qn, HD * 4, hipMemcpyHostToDevice));
    CK(hipMemcpy(d_kn, kn, HD * 4, hipMemcpyHostToDevice));
    CK(hipMemcpy(d_pos, pos3, (size_t)T * 12, hipMemcpyHostToDevice));
    CK(hipMemcpy(d_inv, inv_freq, sizeof inv_freq, hipMemcpyHostToDevice));
    CK(hipMemcpy(d_blk, blocks, (size_t)n_blk * CLEF_HIP_BLOCK_INTS * 4, hipMemcpyHostToDevice));
    CK(hipMemcpy(d_kvtok, kv_tok, (size_t)kv_rows * 4, hipMemcpyHostToDevice));
    CK(hipMemcpy(d_tokkv, tok_kv, (size_t)T * 4, hipMemcpyHostToDevice));
    CK(hipMemcpy(d_ss, seq_start, (size_t)T * 4, hipMemcpyHostToDevice));
    CK(hipMemset(d_ovf, 0, (size_t)T * 4));

    clef_hip_attn_args a;
    memset(&a, 0, sizeof a);
    a.nh = NH; a.nkv = NKV; a.hd = HD; a.n_rot = NROT; a.eps = 1e-6f; a.scale = 1.0f / 16.0f;
    a.T = T; a.row = row; a.qkv = d_qkv; a.q_norm = d_qn; a.k_norm = d_kn; a.pos3 = d_pos;
    a.inv_freq = d_inv; a.rope_cs = d_cs; a.k_plane = d_k; a.vt_plane = d_vt; a.kvT = kvT;
    a.blocks = d_blk; a.n_blk = n_blk; a.kv_tok = d_kvtok; a.tok_kv = d_tokkv; a.kv_rows = kv_rows; a.causal = 1;
    a.gate = 1; a.out = d_out; a.out_type = CLEF_HIP_OUT_BF16; a.f16_lim = 65504.0f; a.ovf = d_ovf;
    a.seq_start = d_ss; a.qkv_type = CLEF_HIP_QKV_BF16;
    uint16_t *out = malloc((size_t)T * NH * HD * 2);

    if (!clef_hip_attn_prefill(&a, NULL, err, sizeof err)) return die("prefill", err);
    CK(hipDeviceSynchronize());
    CK(hipMemcpy(out, d_out, (size_t)T * NH * HD * 2, hipMemcpyDeviceToHost));
    if (!save(dir, "out.bin", out, (size_t)T * NH * HD * 2)) return die("write", "out.bin");

    /* again over a host schedule for 16 workgroups */
    const int n_wg = 16, n_sched = clef_hip_attn_sched_size(n_blk, NH, n_wg);
    int32_t *sched = calloc(n_sched, 4);
    if (!clef_hip_attn_schedule(blocks, n_blk, NH, NKV, n_wg, sched, n_sched, err, sizeof err))
        return die("schedule", err);
    void *d_sched;
    CK(hipMalloc(&d_sched, (size_t)n_sched * 4));
    CK(hipMemcpy(d_sched, sched, (size_t)n_sched * 4, hipMemcpyHostToDevice));
    CK(hipMemset(d_out, 0, (size_t)T * NH * HD * 2));
    a.sched = d_sched; a.n_wg = n_wg;
    if (!clef_hip_attn_prefill(&a, NULL, err, sizeof err)) return die("prefill (schedule)", err);
    CK(hipDeviceSynchronize());
    CK(hipMemcpy(out, d_out, (size_t)T * NH * HD * 2, hipMemcpyDeviceToHost));
    if (!save(dir, "out_sched.bin", out, (size_t)T * NH * HD * 2)) return die("write", "out_sched.bin");

    /* f32 rows are refused before anything runs */
    a.qkv_type = 2;
    if (clef_hip_attn_prefill(&a, NULL, err, sizeof err) || strncmp(err, "hip: ", 5))
        return die("qkv_type", "an unknown qkv_type was not refused");
    printf("abi_run ok: T %d, %d blocks, kvT %d\n", T, n_blk, kvT);
    return 0;
}
