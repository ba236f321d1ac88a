/* Prints the layout of every argument struct of include/clef_hip_attn.h as the C compiler sees
 * it: one line "<struct> <field> <offset> <size>" per field, then "<struct> sizeof <size>".
 * tests/test_c_abi.py compares it with the ctypes mirror in cleffa_amd/_lib.py. */
#include <stddef.h>
#include <stdio.h>

#include "clef_hip_attn.h"

#define F(S, f) printf("%s %s %zu %zu\n", #S, #f, offsetof(S, f), sizeof(((S *)0)->f))
#define Z(S) printf("%s sizeof %zu\n", #S, sizeof(S))

int main(void) {
    F(clef_hip_attn_args, nh); F(clef_hip_attn_args, nkv); F(clef_hip_attn_args, hd);
    F(clef_hip_attn_args, n_rot); F(clef_hip_attn_args, eps); F(clef_hip_attn_args, scale);
    F(clef_hip_attn_args, T); F(clef_hip_attn_args, row); F(clef_hip_attn_args, qkv);
    F(clef_hip_attn_args, q_norm); F(clef_hip_attn_args, k_norm); F(clef_hip_attn_args, pos3);
    F(clef_hip_attn_args, inv_freq); F(clef_hip_attn_args, rope_cs); F(clef_hip_attn_args, k_plane);
    F(clef_hip_attn_args, vt_plane); F(clef_hip_attn_args, kvT); F(clef_hip_attn_args, blocks);
    F(clef_hip_attn_args, n_blk); F(clef_hip_attn_args, kv_tok); F(clef_hip_attn_args, kv_rows);
    F(clef_hip_attn_args, causal); F(clef_hip_attn_args, gate); F(clef_hip_attn_args, out);
    F(clef_hip_attn_args, out_type); F(clef_hip_attn_args, f16_lim); F(clef_hip_attn_args, ovf);
    F(clef_hip_attn_args, trace); F(clef_hip_attn_args, sched); F(clef_hip_attn_args, n_wg);
    F(clef_hip_attn_args, seq_start); F(clef_hip_attn_args, qkv_type); F(clef_hip_attn_args, tok_kv);
    Z(clef_hip_attn_args);

    F(clef_hip_vis_args, P); F(clef_hip_vis_args, heads); F(clef_hip_vis_args, hd);
    F(clef_hip_vis_args, scale); F(clef_hip_vis_args, qkv); F(clef_hip_vis_args, bias);
    F(clef_hip_vis_args, pos2); F(clef_hip_vis_args, inv_freq); F(clef_hip_vis_args, q_plane);
    F(clef_hip_vis_args, k_plane); F(clef_hip_vis_args, vt_plane); F(clef_hip_vis_args, kvT);
    F(clef_hip_vis_args, blocks); F(clef_hip_vis_args, n_blk); F(clef_hip_vis_args, kv_tok);
    F(clef_hip_vis_args, kv_rows); F(clef_hip_vis_args, out); F(clef_hip_vis_args, out_type);
    F(clef_hip_vis_args, f16_lim); F(clef_hip_vis_args, ovf); F(clef_hip_vis_args, tok_kv);
    Z(clef_hip_vis_args);

    F(clef_hip_omni_prep_args, nh); F(clef_hip_omni_prep_args, nkv); F(clef_hip_omni_prep_args, T);
    F(clef_hip_omni_prep_args, kvT); F(clef_hip_omni_prep_args, eps); F(clef_hip_omni_prep_args, rope_exact);
    F(clef_hip_omni_prep_args, qkv); F(clef_hip_omni_prep_args, q_norm); F(clef_hip_omni_prep_args, k_norm);
    F(clef_hip_omni_prep_args, pos3); F(clef_hip_omni_prep_args, freq); F(clef_hip_omni_prep_args, q_plane);
    F(clef_hip_omni_prep_args, k_plane); F(clef_hip_omni_prep_args, v_plane); F(clef_hip_omni_prep_args, status);
    Z(clef_hip_omni_prep_args);

    F(clef_hip_omni_attn_args, nh); F(clef_hip_omni_attn_args, nkv); F(clef_hip_omni_attn_args, T);
    F(clef_hip_omni_attn_args, kvT); F(clef_hip_omni_attn_args, scale); F(clef_hip_omni_attn_args, q_plane);
    F(clef_hip_omni_attn_args, k_plane); F(clef_hip_omni_attn_args, v_plane); F(clef_hip_omni_attn_args, blocks);
    F(clef_hip_omni_attn_args, n_blk); F(clef_hip_omni_attn_args, out);
    Z(clef_hip_omni_attn_args);
    return 0;
}
