/* attn_oracle.c - CPU restatement of cleffa's prefill attention semantics.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker for the HIP path: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. The product path
 * (cleffa_amd/) never calls it.
 *
 * Every function is compiled twice from attn_oracle_impl.h: a float64 flavour (suffix _f64,
 * the parity oracle) and a float32 flavour (suffix _f32, OpenMP-parallel, the timed CPU
 * baseline). Inputs are the bf16-rounded operands as f32; all arithmetic after that is in the
 * flavour's precision.
 *
 * What each function restates (reference citations, /root/reference):
 *   orc_text_prep_*   attn_prep: per-head RMSNorm with (1+w) folded into w, NeoX partial rotary
 *                     on the first n_rot dims with interleaved M-RoPE axis i % 3, gate split;
 *                     metal/clef.metal:245-300 (the same math as attn_prep_split 873-928 without
 *                     the hi/lo split), QKV row layout tools/convert.py:23-25.
 *   orc_attention_*   causal / bidirectional GQA SDPA over packed records with cu_seqlens,
 *                     prefix keys (query j of a record with L cached keys sees keys 0..L+j),
 *                     fully masked rows = 0, optional sigmoid(gate) epilogue;
 *                     ref/safe_attn.py:25-52 and 55-68 (semantics), metal/clef.metal:316-352
 *                     (reference kernel, gate epilogue), 709-849 (prefix mask key <= q + qoff),
 *                     930-1093 (block list qbase/kbase addressing).
 *   orc_omni_prep_*   omni_attn_prep: hd-128 RMSNorm (weights as given) and full rotary over 64
 *                     pairs, axis i % 3 below pair 60 and axis 0 above, angle from the FP64
 *                     frequency (exact) or the f32 product; metal/clef.metal:2055-2131, checked
 *                     the way tests/test_omni_attention.m:104-122 checks it. Omni attention
 *                     itself is orc_attention_* with no gate (metal/clef.metal:2165-2319).
 *   orc_vis_prep_*    vis_qkv_rope: bias add, 2-D rotary on pairs (i, i + hd/2), first hd/4 pairs
 *                     by grid row, the rest by grid column; metal/clef.metal:1616-1656.
 */
#include <tgmath.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define REAL double
#define SFX(name) name##_f64
#include "attn_oracle_impl.h"
#undef REAL
#undef SFX

#define REAL float
#define SFX(name) name##_f32
#include "attn_oracle_impl.h"
#undef REAL
#undef SFX

int orc_num_threads(void) {
#ifdef _OPENMP
    extern int omp_get_max_threads(void);
    return omp_get_max_threads();
#else
    return 1;
#endif
}
