// Kernel argument blocks shared by the HIP kernels and the host layer (internal).
#pragma once
#include <stdint.h>

#include "clef_hip_attn.h"

namespace clef_hip {

struct AttnParams {
    const uint16_t *qkv;      // text: fused qkv rows [T][row]
    const float *q_norm;
    const int32_t *pos3;
    const float *inv_freq;
    const float *rope_cs;     // text: cos/sin per pass row [T][n_rot/2][2], or NULL
    const uint16_t *q_plane;  // vision: prepared Q [heads][T][72]
    const uint16_t *k_plane;
    const uint16_t *vt_plane;
    const int32_t *blocks;
    void *out;
    int32_t *ovf;
    int row, T, kvT, nh, nkv, n_rot;
    float eps, scale_log2, f16_lim;
    int causal, gate, out_type, out_ld;
    int n_blk;                // blocks in the plan (work items = n_blk * nh)
    int xcd_heads;            // nh / 8 when heads split evenly over the 8 XCDs, else 0
    uint64_t *trace;          // NULL, or [n_blk * nh][8] per work item: start, end, HW_ID, XCC_ID, prologue end, loop end, workgroup, ordinal
    const int32_t *sched;     // NULL, or a schedule: header {magic, n_blk, nh, n_wg, nkv, fingerprint, 0, 0}, [n_wg + 1] offsets, items
};

struct VisPrepParams {
    const uint16_t *qkv;
    const float *bias;
    const int32_t *pos2;
    const float *inv_freq;
    const int32_t *kv_tok;    // patch of each plane row, -1: not written
    const int32_t *tok_kv;    // plane row of each patch (the rows kernel)
    uint16_t *q_plane;
    uint16_t *k_plane;
    uint16_t *vt_plane;
    int P, heads, kvT, kv_rows;
};

}  // namespace clef_hip
