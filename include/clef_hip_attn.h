/* clef_hip_attn.h - C ABI of the MI355X (gfx950) prefill attention path for cleffa.
 *
 * This library replaces the attention dispatch inside cleffa's GPU backend. The engine's public
 * entry points clef_gpu_forward and clef_gpu_forward_prefix (clef_engine.h:178-205) keep their
 * signatures; inside them the full-attention layer calls clef_hip_attn_prefill where the Metal
 * backend calls encode_attention_tu (clef_metal.m:829-882) or its FP32 branch
 * (clef_metal.m:1330-1413), and the vision tower calls clef_hip_vis_attention where it runs
 * vis_qkv_rope + vis_attention_mma/_mpp (clef_metal.m:1022-1049).
 *
 * Conventions (clef_metal.m:83-86, 39-49): every entry point returns true on success; on failure
 * it returns false and writes a message starting with "hip: " into err (errlen bytes, may be
 * NULL/0) and launches nothing further. Device pointers are plain pointers into device memory;
 * `stream` is a hipStream_t passed as void * (NULL = the default stream). Calls are asynchronous
 * with respect to the host and not reentrant for buffers they share. Nothing here allocates
 * device memory: the caller owns every buffer (clef_metal.m:337-412 ownership model).
 *
 * Layouts (bf16 / f16 = raw uint16 bits):
 *   qkv     [T][row] bf16, the fused projection row: [nh x (query hd | gate hd)] [nkv x hd K]
 *           [nkv x hd V] (tools/convert.py:23-25, metal/clef.metal:245-248).
 *   pos3    [T][3] int32 rotary positions per pass row (temporal, grid row, grid column).
 *   K plane [nkv][kvT][hd] f16, normalised and rotated keys, one row per key (f16: the scores
 *           of sharp rows need its 11-bit significand to stay within tolerance).
 *   V^T     [nkv][hd][kvT] bf16, values transposed (keys contiguous per head dim).
 *   out     [T][nh*hd] (text) or [P][heads*hd] (vision): the o_proj operand, bf16 / f16 / f32.
 *   The plan (clef_hip_attn_plan) maps records to query blocks and kv rows; it is built once per
 *   pass on the host and copied to the device, then reused by every attention layer of the pass,
 *   as the Metal backend builds attn_blk once per forward (clef_metal.m:1243-1257).
 */
#ifndef CLEF_HIP_ATTN_H
#define CLEF_HIP_ATTN_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CLEF_HIP_OUT_BF16 0 /* bf16 (act16 with f16 off, metal/clef.metal:101) */
#define CLEF_HIP_OUT_F16 1  /* f16; |v| > f16_lim or NaN saturates and flags (metal/clef.metal:98-106) */
#define CLEF_HIP_OUT_F32 2  /* f32, unrounded: a store width only; FP32 arithmetic is qkv_type CLEF_HIP_QKV_F32 */

#define CLEF_HIP_BLOCK_Q 128  /* query rows per block */
#define CLEF_HIP_KV_ALIGN 8   /* kv row alignment of each record in a fresh pass (V^T runs of 8 keys) */
#define CLEF_HIP_BLOCK_INTS 8 /* int32 per block entry */

/* Library version and the wave size the kernels were compiled for (64). The Metal backend
 * refuses attention pipelines that are not 32 lanes wide (clef_metal.m:95-108); this is the
 * CDNA equivalent: clef_hip_attn_init fails unless the device runs 64-wide wavefronts. */
int clef_hip_attn_version(void);
int clef_hip_attn_wave_size(void);

/* Checks the current device (gfx950, wave64, LDS for the kernels) and sets kernel attributes.
 * Call once per device before the first launch. Replaces the pipeline checks of clef_gpu_open
 * (clef_metal.m:95-108, 133-140). */
bool clef_hip_attn_init(char *err, size_t errlen);

/* Upper bound for the plan's block count of a pass with n_seq records and Tq query rows. */
int clef_hip_attn_plan_max_blocks(int n_seq, int Tq);

/* Host-only: builds the query-block list and the kv-row map of a pass (clef_metal.m:1243-1257
 * block list; clef.c:470-497 packing). cu_q[n_seq+1] are the records' pass-row bounds
 * (seq_bounds). cu_k = NULL is a fresh pass: every record's keys are its own queries and the
 * plan lays them out at kv rows aligned to CLEF_HIP_KV_ALIGN (8), with *kv_rows covering a whole
 * 64-key tile from each record's first key. cu_k != NULL is a prefix-cache pass
 * (clef_gpu_forward_prefix, clef_metal.m:1640-1666): record r's keys occupy kv rows
 * cu_k[r] .. cu_k[r+1] (multiples of 8), its first cu_k[r+1]-cu_k[r]-(cu_q[r+1]-cu_q[r]) keys are
 * cached, and its queries are the last tokens. causal = 0 gives bidirectional attention within
 * each record (vision). Outputs: blocks [max_blocks][8] (sorted longest first; an entry is
 * {q_row0, nq, q_pos0, k_row0, k_len, record's first pass row, record, fingerprint}, the last a
 * 32-bit hash of words 0-6 of all entries, the same in each, that ties a schedule to the plan), tok_kv
 * [max_tok >= cu_q[n_seq]] (the K/V plane row each pass row's key lands in), kv_tok
 * [max_kv >= *kv_rows] (the inverse: the pass row whose key each plane row takes, -1 for rows
 * the pass does not write; NULL skips it), *n_blk, *kv_rows (rows per head the K and V^T
 * planes need: every record's first kv row plus its key count rounded up to 64, since the
 * attention kernel reads whole 64-key tiles). */
bool clef_hip_attn_plan(const int32_t *cu_q, const int32_t *cu_k, int n_seq, int causal,
                        int32_t *blocks, int max_blocks, int32_t *tok_kv, int max_tok,
                        int32_t *kv_tok, int max_kv, int *n_blk, int *kv_rows, char *err, size_t errlen);

/* RoPE frequency table: inv_freq[j] = 1 / theta^(2j/n_rot) in f32, j < n_rot/2
 * (clef_metal.m:176-184 text, 186-192 vision with n_rot = hd/2 and theta = 10000). */
void clef_hip_rope_inv_freq(float theta, int n_rot, float *inv_freq);

/* Host-only: per-patch (grid row, grid column) of the vision rotary, patches stored in
 * merge x merge window order (metal/clef.metal:1639-1641). pos2 [cu[n_img]][2]. */
bool clef_hip_vis_positions(const int32_t *cu, int n_img, const int32_t *grid_w, int merge,
                            int32_t *pos2, char *err, size_t errlen);

/* One full-attention layer of the dense text models (hd 256, GQA). */
typedef struct {
    int nh, nkv, hd, n_rot;   /* hd must be 256; n_rot 64 (Clef) or 0 */
    float eps, scale;         /* RMSNorm eps (1e-6), softmax scale (1/sqrt(hd)) */
    int T, row;               /* pass rows; qkv row stride in elements (multiple of 8) */
    const void *qkv;          /* [T][row]: bf16 (qkv_type CLEF_HIP_QKV_BF16) or f32 (CLEF_HIP_QKV_F32) */
    const float *q_norm;      /* [hd] f32, already 1 + w (tools/convert.py:7-8); NULL with k_norm: no norm */
    const float *k_norm;      /* [hd] f32, already 1 + w */
    const int32_t *pos3;      /* [T][3] */
    const float *inv_freq;    /* [n_rot/2] */
    float *rope_cs;           /* [T][n_rot/2][2] f32 scratch or NULL: prep_kv writes each pass row's
                                 rotary cos/sin there and core reads them (core alone with a table
                                 that prep_kv did not fill for this pass is undefined); NULL: core
                                 evaluates the angles itself */
    void *k_plane;            /* [nkv][kvT][hd]: f16 (bf16 mode) or f32 (FP32 mode) */
    void *vt_plane;           /* bf16 mode: V^T [nkv][hd][kvT] bf16; FP32 mode: V [nkv][kvT][hd] f32 */
    int kvT;                  /* rows per head of the planes: >= plan kv_rows, multiple of 8 */
    const int32_t *blocks;    /* device copy of the plan's blocks */
    int n_blk;
    const int32_t *kv_tok;    /* device copy of the plan's kv_tok [kv_rows] (the FP32 prologue runs
                                 over plane rows with it) */
    int kv_rows;              /* the plan's kv_rows */
    int causal;               /* 1 for the text models */
    int gate;                 /* 1: multiply by sigmoid(gate) (Qwen3.5 gated attention) */
    void *out;                /* [T][nh*hd] */
    int out_type;             /* CLEF_HIP_OUT_* */
    float f16_lim;            /* f16 overflow limit (65504): the K plane and Q operand are f16, so
                                 a key or query element with |x| > f16_lim or NaN is saturated to
                                 +-65504 and flags its record, as split16 does
                                 (metal/clef.metal:857-867); so does an f16 output (act16) with
                                 CLEF_HIP_OUT_F16. V elements (bf16 here) with |v| > f16_lim
                                 or NaN are saturated to +-65536 and flag too */
    int32_t *ovf;             /* [T] int32 flags, set at the record's first pass row; may be NULL */
    uint64_t *trace;          /* NULL, or [n_blk * nh][8] u64 per work item (query block, q head;
                                 of a block split in halves by the schedule, the first half):
                                 start, end (100 MHz device wall clock), HW_ID and XCC_ID
                                 registers, end of the prologue, end of the key loop, workgroup,
                                 ordinal in the workgroup; the CLEF_PROFILE analogue
                                 (clef_metal.m:52-68) at work-item grain. The heads of an item
                                 that runs several heads of a short block get the same row */
    const int32_t *sched;     /* NULL, or device copy of clef_hip_attn_schedule's output for this
                                 plan, nh, nkv and n_wg: the core then runs n_wg workgroups, each
                                 over its own item list. The kernel checks the list's header
                                 against the call (n_blk, nh, nkv, n_wg) and against the plan
                                 fingerprint in word 7 of the block entries; a list built for
                                 another plan or shape is not used, and the n_wg workgroups run
                                 the static order instead (the same output, unbalanced) */
    int n_wg;
    const int32_t *seq_start; /* [T] device int32: each pass row's record start (the reference's
                                 seq_start, clef_engine.h:179), where prep_kv flags a key that
                                 leaves f16's range (see f16_lim); NULL: such keys are still
                                 saturated, but not flagged */
    int qkv_type;             /* CLEF_HIP_QKV_BF16 (0): the tensor-unit path (encode_attention_tu):
                                 bf16 rows, f16 Q/K and bf16 P/V operands, f32 accumulation.
                                 CLEF_HIP_QKV_F32 (1): the FP32 path (clef_metal.m:1330-1413,
                                 attn_prep + attention_prefetch_64 and kin): f32 rows, f32 K and V
                                 planes, FP32 products and softmax, for the per-record rerun after
                                 an overflow (clef.c:526-550) and CLEF_ATTN_TU=0. In FP32 mode any
                                 nh / nkv works (groups above 8 heads run as several head
                                 chunks), sched and trace are ignored, and only the output (f16
                                 out_type) can flag. Other values are rejected */
    const int32_t *tok_kv;    /* [T] device int32: the plan's pass row -> plane row map (the inverse
                                 of kv_tok); the bf16 K/V prologue runs over pass rows with it */
} clef_hip_attn_args;

#define CLEF_HIP_QKV_BF16 0
#define CLEF_HIP_QKV_F32 1

/* Static split of a text pass's work items (query block, q head) over n_wg workgroups of the
 * attention core, for clef_hip_attn_args.sched. No reference counterpart: the Metal backend
 * dispatches one threadgroup per block and head (clef_metal.m:829-882); a persistent grid needs
 * the split made on the host. Items are dealt longest first to the least loaded workgroup
 * (cost: the block's 64-key tiles plus a fixed per-item cost), within the workgroups of the XCD
 * that owns the item's q head when the heads divide evenly over the 8 XCDs (workgroup b runs on
 * XCD b % 8). blocks: the plan's host block list. Output: a header {0x53434844, n_blk, nh,
 * n_wg, nkv, fingerprint of the block list (the value clef_hip_attn_plan writes into word 7 of
 * every block entry), 0, 0}, then n_wg + 1 item offsets per workgroup, then the items, each workgroup's longest
 * first. An item is block * nh + head in bits 0-27 and, in bits 28-29, what it runs: 0 the whole
 * block for that head; when the pass has fewer items than workgroups, a block of more than 64
 * rows becomes two items, 1 (rows 0-63) and 2 (rows 64-127), so that more workgroups have work;
 * otherwise a block of at most 64 rows runs k heads h .. h + k - 1 of one kv group in one item,
 * 3 (k the largest divisor of nh / nkv with k * ceil(rows / 16) <= 8), so that they share its key
 * tiles, and when nh / nkv is even a block of more than 64 rows runs as two items for heads h and
 * h + 1, codes 1 and 2 with bit 30 set (a causal block's last 64 keys, which only its rows 64-127
 * see, then run on a full workgroup). Outputs are bitwise the same in every case (a code 2 of a block of 64 rows or fewer runs
 * the whole block, a code 3 that does not fit its kv group runs head h only, so no list reaches
 * rows or heads outside its item). clef_hip_attn_sched_size gives the room to allocate (an upper
 * bound: the last offset is the item count). */
int clef_hip_attn_sched_size(int n_blk, int nh, int n_wg);

bool clef_hip_attn_schedule(const int32_t *blocks, int n_blk, int nh, int nkv, int n_wg,
                            int32_t *sched, int max_sched, char *err, size_t errlen);

/* The QKV projection with the K/V prologue fused into its epilogue: qkv[T][row] (bf16, a->qkv)
 * = X . W^T with X [T][H] bf16 activations and W [N][H] the attn_qkv weight as stored
 * (N = 2 nh hd + 2 nkv hd columns: [q | gate] per q head, then K heads, then V heads), f32
 * accumulation; replaces clef_metal_gemm at the QKV call (clef_metal.m:463-499, 1326) and the
 * attn_prep K/V kernels (metal/clef.metal:245-300, 873-928). tok_kv (the plan's pass row ->
 * plane row map, [T]) != NULL: every K head's rows are normalised, rotated and written to the K
 * plane and every V head's to the V^T plane, bitwise what clef_hip_attn_prep_kv writes from the
 * same qkv rows (with the same flags and rope_cs), so clef_hip_attn_core may follow directly;
 * NULL: the product only. H must be a multiple of 64; X and W at most 4 GiB each. */
bool clef_hip_qkv_gemm(int H, const uint16_t *X, const uint16_t *W, const clef_hip_attn_args *a, const int32_t *tok_kv,
                       void *stream, char *err, size_t errlen);

/* K/V prologue only: RMSNorm + rotary of each pass row's K into its plane row (tok_kv; kv_tok in
 * FP32 mode), V into
 * the V^T plane (attn_prep / attn_prep_split / attn_prep_prefix K and V parts,
 * metal/clef.metal:245-300, 657-707, 873-928). Plane rows no pass row maps to are not written. */
bool clef_hip_attn_prep_kv(const clef_hip_attn_args *a, void *stream, char *err, size_t errlen);
/* Attention core with the Q prologue and gate epilogue fused (attention_tu and the FP32
 * kernels, metal/clef.metal:316-654, 709-849, 930-1093). Reads the planes prep_kv wrote. */
bool clef_hip_attn_core(const clef_hip_attn_args *a, void *stream, char *err, size_t errlen);
/* prep_kv then core: the whole attention step of one layer (encode_attention_tu). */
bool clef_hip_attn_prefill(const clef_hip_attn_args *a, void *stream, char *err, size_t errlen);

/* Vision tower attention (hd 72, MHA, bidirectional within each image). */
typedef struct {
    int P, heads, hd;         /* hd must be 72 */
    float scale;              /* 1/sqrt(hd) */
    const uint16_t *qkv;      /* [P][3*heads*hd] bf16 */
    const float *bias;        /* [3*heads*hd] f32 or NULL */
    const int32_t *pos2;      /* [P][2] grid (row, column) per patch */
    const float *inv_freq;    /* [hd/4] */
    uint16_t *q_plane;        /* [heads][P][72] scratch: biased, rotated Q */
    uint16_t *k_plane;        /* [heads][kvT][72] scratch: biased, rotated K */
    uint16_t *vt_plane;       /* [heads][72][kvT] scratch: biased V, transposed */
    int kvT;                  /* >= the plan's kv_rows, multiple of 8 */
    const int32_t *blocks;    /* device copy of a bidirectional plan's blocks */
    int n_blk;
    const int32_t *kv_tok;    /* device copy of the plan's kv_tok [kv_rows] */
    int kv_rows;
    void *out;                /* [P][heads*hd] */
    int out_type;
    float f16_lim;
    int32_t *ovf;             /* [P] or NULL; flag at the image's first patch */
    const int32_t *tok_kv;    /* [P] device int32 or NULL: the plan's patch -> plane row map (the
                                 inverse of kv_tok); given, the prologue runs over patches with all
                                 its loads at once, else over plane rows through kv_tok */
} clef_hip_vis_args;

bool clef_hip_vis_attention(const clef_hip_vis_args *a, void *stream, char *err, size_t errlen);

/* clef_hip_vis_attention with the three planes in the library's own device scratch: it has no
 * counterpart in the reference (whose vision planes are Metal buffers the backend owns), and is
 * for callers that cannot allocate device memory (code under graph capture, serving loops,
 * harnesses that forbid hipMalloc). q_plane, k_plane and vt_plane are ignored; the other fields
 * mean what they mean above. The planes need heads * (max(P, 1) + 2 kvT) * 144 bytes (each plane
 * rounded up to 256), at most CLEF_HIP_VIS_SCRATCH_BYTES; larger calls fail with an error. The
 * scratch is one static array per GPU, held until the process ends and shared by every call on
 * that GPU: calls that overlap on one GPU (other streams, other threads) race and must be
 * serialised by the caller. Nothing in it needs clearing between calls. Allocates nothing. */
#define CLEF_HIP_VIS_SCRATCH_BYTES ((size_t)64 << 20)
bool clef_hip_vis_attention_noalloc(const clef_hip_vis_args *a, void *stream, char *err, size_t errlen);

/* ---- The GEMMs either side of the path (clef_metal.m:463-499 clef_metal_gemm; callers
 * clef_metal.m:1326 QKV projection, 1415 o_proj into the residual).
 * Y[T][N] (+)= X[T][K] . W[N][K]^T with X and W bf16 row-major, f32 accumulation. y_type
 * CLEF_HIP_GEMM_Y_BF16 writes bf16 (the qkv rows clef_hip_attn_prefill reads), CLEF_HIP_GEMM_Y_F32
 * f32; acc != 0 adds into an f32 Y (the residual stream). workspace (may be NULL with ws_bytes 0)
 * is device scratch the algorithm may use. Runs on hipBLASLt; the algorithm of each shape is
 * chosen on its first call. For acc == 0 that call times up to 16 of hipBLASLt's candidates on
 * the caller's operands and stream (Y is overwritten by each and finally by the chosen one), so
 * it waits for the stream once. An accumulating call, or one under graph capture, takes
 * hipBLASLt's first candidate; a choice made under capture is timed at the next uncaptured call. */
#define CLEF_HIP_GEMM_Y_F32 0
#define CLEF_HIP_GEMM_Y_BF16 1
bool clef_hip_gemm(int T, int N, int K, const uint16_t *X, const uint16_t *W, void *Y, int y_type, int acc,
                   void *workspace, size_t ws_bytes, void *stream, char *err, size_t errlen);

/* ---- The GEMMs' weights from the model file (replaces clef_gguf.h:52-63 gguf_open / find /
 * get and clef.c:27-59 load_config, 180-256 bind_weights). Host-only except the copies: a
 * read-only index over an mmap'd GGUF v3 file, every read bounds-checked (the file is untrusted),
 * the attention geometry, and one layer's attention tensors copied into device buffers the
 * caller owns. */
#define CLEF_HIP_GGML_F32 0
#define CLEF_HIP_GGML_F16 1
#define CLEF_HIP_GGML_BF16 30
#define CLEF_HIP_MAX_LAYERS 128   /* clef_engine.h:14 */
typedef struct clef_hip_gguf clef_hip_gguf;
typedef struct {
    uint32_t n_dims, type;    /* 1..4; CLEF_HIP_GGML_* */
    uint64_t ne[4];           /* ne[0] is the row length (fastest varying); unused dims are 1 */
    uint64_t offset, nbytes;  /* absolute file offset and size of the data */
    const void *data;         /* into the mapping, valid until clef_hip_gguf_close */
} clef_hip_gguf_tensor_info;
typedef struct {
    int n_layer, H, nh, nkv, hd, n_rot;   /* clef.block_count, embedding_length, attention.head_count,
                                             head_count_kv, key_length, rope.dimension_count */
    float eps, rope_theta;                /* attention.layer_norm_rms_epsilon, rope.freq_base */
    int32_t layer_full[CLEF_HIP_MAX_LAYERS];   /* clef.layer_types: 1 full attention, 0 DeltaNet */
} clef_hip_attn_config;

/* Fails on a missing file, a bad magic or version (3 only), counts the file cannot hold, nested
 * arrays deeper than two, an alignment that is not a power of two, tensor types other than
 * F32 / F16 / BF16, ranks outside 1..4 and tensor data outside the file. */
bool clef_hip_gguf_open(const char *path, clef_hip_gguf **out, char *err, size_t errlen);
void clef_hip_gguf_close(clef_hip_gguf *g);
int clef_hip_gguf_tensor_count(const clef_hip_gguf *g);
/* Tensor i of the table (file order) and its name, NUL-terminated into name[name_len]. */
bool clef_hip_gguf_tensor_at(const clef_hip_gguf *g, int i, clef_hip_gguf_tensor_info *info, char *name, size_t name_len);
bool clef_hip_gguf_find_tensor(const clef_hip_gguf *g, const char *name, clef_hip_gguf_tensor_info *info);
bool clef_hip_gguf_get_u32(const clef_hip_gguf *g, const char *key, uint32_t *out);
bool clef_hip_gguf_get_f32(const clef_hip_gguf *g, const char *key, float *out);
/* general.architecture "clef", the keys above (u32 values in 1 .. 2^24), layer_types of
 * n_layer entries each 0 or 1, nh a multiple of nkv. */
bool clef_hip_gguf_attn_config(const clef_hip_gguf *g, clef_hip_attn_config *c, char *err, size_t errlen);
/* Full-attention layer `layer`: blk.L.attn_qkv.weight BF16 [n_attn][H] (n_attn = 2 nh hd + 2 nkv hd,
 * rows [q | gate] per head, then K, then V: the QKV GEMM's W), blk.L.attn_output.weight BF16
 * [H][nh hd] (the o_proj's W), blk.L.attn_q_norm / attn_k_norm.weight F32 [hd] (already 1 + w).
 * Each is checked for type and shape, then copied on `stream` into the given device buffer
 * (NULL skips that tensor); the call waits for the stream before it returns, so the handle may
 * be closed right after. */
bool clef_hip_gguf_attn_layer(const clef_hip_gguf *g, const clef_hip_attn_config *c, int layer, uint16_t *w_qkv,
                              uint16_t *w_o, float *q_norm, float *k_norm, void *stream, char *err, size_t errlen);
/* Vision tower layer `layer` (clef.c:291-294): v.blk.L.attn_qkv.weight BF16 [3E][E] and .bias F32 [3E],
 * v.blk.L.attn_out.weight BF16 [E][E] and .bias F32 [E], E = 72 heads. */
bool clef_hip_gguf_vis_layer(const clef_hip_gguf *g, int layer, int heads, uint16_t *w_qkv, float *b_qkv,
                             uint16_t *w_o, float *b_o, void *stream, char *err, size_t errlen);

/* ---- Omni decoder attention (metal/clef.metal:2055-2319 omni_attn_prep / omni_attention, host
 * clef_metal_omni.m:200-245 clef_omni_encode_attention). FP32 operands, hd 128, causal within
 * each record, no gate; the output is accumulated in FP64 (the reference: FP32 hi/lo pairs).
 *
 * clef_hip_omni_rope_table: the 192-float rotary table of the reference (clef_metal.m:172-180):
 * [0, 64) 1 / theta^(2j/128) in FP32, [64, 128) and [128, 192) the FP64 theta^(-2j/128) as an
 * FP32 hi / lo pair. */
#define CLEF_HIP_OMNI_BLOCK_Q 16   /* query rows per block */
#define CLEF_HIP_OMNI_SLACK 32     /* zero rows after each kv head's T rows (kvT >= T + 32) */
void clef_hip_omni_rope_table(float theta, float *freq192);

/* omni_attn_prep: per pass row t and head h, RMSNorm (weights as given) and rotary over all 128
 * dims (pairs (i, i + 64), pair i turning by pos3 axis i % 3 for i < 60 and axis 0 above),
 * with the angle from the FP64 frequency reduced in FP64 (rope_exact) or the FP32 product
 * pos * freq[i] (rope_exact 0, CLEF_OMNI_ROPE=f32). Writes Q [nh][T][128], K and V [nkv][kvT][128]
 * (V copied), zeroes K / V rows T .. T+31, and ORs 2 into *status when any input or output value
 * is not finite. */
typedef struct {
    int nh, nkv, T, kvT;
    float eps;
    int rope_exact;
    const float *qkv;         /* [T][(nh + 2 nkv) * 128]: Q heads, K heads, V heads */
    const float *q_norm, *k_norm;   /* [128] */
    const int32_t *pos3;      /* [T][3] */
    const float *freq;        /* [192], clef_hip_omni_rope_table */
    float *q_plane, *k_plane, *v_plane;
    uint32_t *status;
} clef_hip_omni_prep_args;
bool clef_hip_omni_prep(const clef_hip_omni_prep_args *a, void *stream, char *err, size_t errlen);

/* Block list of an Omni pass: 16-row query blocks per record, each with its record's keys from
 * the record's first row (seq_start of the reference), longest first. Entries as for
 * clef_hip_attn_plan: {q_row0, nq, q_pos0, k_row0, k_len, 0, record, 0}. */
int clef_hip_omni_plan_max_blocks(int n_seq, int T);
bool clef_hip_omni_plan(const int32_t *cu_seqlens, int n_seq, int32_t *blocks, int max_blocks, int *n_blk,
                        char *err, size_t errlen);

/* omni_attention: out[t][h*128 + d] = sum_s softmax(scale * Q_h[t] . K_kh[s]) V_kh[s][d] over the
 * keys s <= t of t's record, FP32 output. Key tiles start at each record's first row, so a
 * record's output bytes do not depend on what else is packed with it. */
typedef struct {
    int nh, nkv, T, kvT;
    float scale;
    const float *q_plane, *k_plane, *v_plane;
    const int32_t *blocks;
    int n_blk;
    float *out;               /* [T][nh * 128] */
} clef_hip_omni_attn_args;
bool clef_hip_omni_attention(const clef_hip_omni_attn_args *a, void *stream, char *err, size_t errlen);

/* Prefix-cache entry planes (clef_metal.m:15-29 struct clef_gpu_prefix, 762-805 prefix_reserve).
 * An entry holds, per attention layer, a K plane [nkv][cap][hd] and a V^T plane [nkv][hd][cap],
 * K f16 and V^T bf16, rows (columns of V^T) indexed by the record's own token index; a prefix pass uses them as
 * k_plane / vt_plane with kvT = cap and cu_seqlens_k = {0, L + n}. The caller allocates them.
 *
 * clef_hip_prefix_capacity: the capacity an entry of cur_cap rows needs to hold `rows` tokens:
 * cur_cap when it already fits, else max(rows, cur_cap + cur_cap / 4) rounded up to a multiple of
 * 1024 (an entry that keeps growing is copied a handful of times, not every 1,024 tokens).
 * Returns -1 when the planes would pass the 32-bit plane offsets of the kernels (cap * hd * 2 >=
 * 2^32) or `rows` is negative. */
int clef_hip_prefix_capacity(int rows, int cur_cap, int hd);
/* Bytes of one plane (K or V^T) of one layer: nkv * cap * hd * 2. */
size_t clef_hip_prefix_plane_bytes(int nkv, int hd, int cap);
/* Growth copy of one layer's planes (the memcpy loop of prefix_reserve): dst rows [0, keep) take
 * the src rows, dst rows [keep, dst_cap) are zeroed (Metal's zero-filled new buffers). K planes
 * copy whole rows; V^T planes copy the first `keep` columns of each of the nkv * hd rows. One
 * kernel on `stream` covers both planes. src_cap and dst_cap multiples of 8, keep <= both,
 * pointers 16-byte aligned, src and dst not overlapping. */
bool clef_hip_prefix_copy(const uint16_t *k_src, const uint16_t *vt_src, int src_cap,
                          uint16_t *k_dst, uint16_t *vt_dst, int dst_cap, int nkv, int hd, int keep,
                          void *stream, char *err, size_t errlen);

/* Host-only producers of the path's inputs. */

/* M-RoPE positions pos3 [T][3] of one record (clef_record.c:938-962, clef_record_positions).
 * A record that carries its own positions (the reference's r->pos3, Omni records) passes them as
 * pos3_given [T][3]: they are copied and the span arguments are not read. Otherwise (pos3_given
 * NULL) text tokens take (p, p, p) with p counting up from 0; vision span i (an image, or one
 * frame of a video) starts at token span_start[i] and covers its merged grid,
 * (span_grid_h[i] / merge) x (span_grid_w[i] / merge) tokens row-major, token (y, x) taking
 * (p, p + y, p + x), after which p advances by the larger merged side. Spans in token order, not
 * overlapping. */
bool clef_hip_record_positions(int T, const int32_t *pos3_given, const int32_t *span_start,
                               const int32_t *span_grid_h, const int32_t *span_grid_w, int n_spans, int merge,
                               int32_t *pos3, char *err, size_t errlen);

/* Micro-batch packing of the server's queue (clef_server.c:311-327): first in, first out; the
 * head is always taken, then requests while fewer than max_batch are taken and the tokens stay
 * within max_tokens; a request with a prefix-cache key (keyed[i] != 0, keyed may be NULL) runs
 * alone. Writes cu_seqlens[0 .. n] of the n records taken and returns n (0 for an empty queue). */
int clef_hip_pack_batch(const int32_t *lengths, const uint8_t *keyed, int n_queue, int max_batch,
                        long max_tokens, int32_t *cu_seqlens);

#ifdef __cplusplus
}
#endif
#endif
