"""Benchmark of the prefill attention hot path on one MI355X.

One step = one full-attention layer's attention over the C1 micro-batch (8 packed causal
records, 4,096 tokens, 24/4 heads, hd 256): the K/V prologue kernel plus the attention kernel
with the fused Q prologue and gate epilogue, on qkv rows already resident in HBM. Steps are
replayed from a HIP graph (captured once) so host launch cost is not part of the GPU time; the
timed region is bracketed by torch.cuda.synchronize() and HIP events on the launch stream.
Untimed passes of the step run for WARM_S seconds before it, so that the device's clocks are up.

Prints one JSON line. `value` is algorithmic TFLOP/s of the whole step (QK^T + PV flops,
4*hd*nh*pairs); `roofline` covers the attention kernel alone, priced at its time inside the
step (the step minus the prologue kernel timed alone, `launch_ms_in_step`), with its time in
back-to-back replays beside it (`launch_ms`); `layer` times the engine's layer instead: the
QKV GEMM whose epilogue writes the K / V^T planes (no prologue kernel), then the attention
kernel; `cpu_baseline` is the fp32 CPU oracle (OpenMP) on the same C1 inputs.
"""
import argparse
import json
import os
import statistics
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA (published)
PEAK_HBM_GBS = 8000.0
CALIB_BYTES = 256 << 20     # bf16 copy used to scale the FETCH_SIZE / WRITE_SIZE counters
WARM_S = 0.3                # untimed passes of the step before the timed one (device clocks)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic.txt")


def measured_traffic(cfg):
    """HBM bytes per launch of the attention kernel from the committed rocprofv3 --pmc summary
    (lines 'traffic <config> <bytes>'), or None when it has not been measured."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                p = line.split()
                if len(p) == 3 and p[0] == "traffic" and p[1] == cfg:
                    return int(p[2])
    except OSError:
        pass
    return None


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="C1", choices=["C0", "C1", "C2", "C3", "C4", "S", "P", "O", "G", "M"],
                    help="C0-C4: attention configurations; S: 256 records x 16 tokens (short prompts); "
                         "P: prefix-cache growth copy (HBM-bound); "
                         "O: Omni attention (hd 128, FP32, 16,344 tokens); G: the QKV and o_proj GEMMs around C1")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--fp32", action="store_true",
                    help="C0-C3 and S in the FP32 mode (f32 qkv rows, FP32 planes and products: the reference's "
                         "FP32 kernels); the roofline is then priced against the fp32 MFMA peak")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-graph", action="store_true", help="launch eagerly instead of graph replay")
    ap.add_argument("--no-layer", action="store_true",
                    help="skip the layer diagnostics (QKV GEMM with the fused K/V prologue, then the attention kernel)")
    ap.add_argument("--profile-pass", action="store_true",
                    help="for rocprofv3 --pmc: a 256 MiB device copy and a 256 MiB elementwise pass "
                         "(counter calibration), then 3 eager "
                         "steps; prints no JSON line")
    return ap.parse_args()


def build_step(cfg, seed, fp32=False):
    """Returns (step_fn, core_fn, info) for one configuration, inputs resident on cuda:0."""
    from cleffa_amd import AttnPlan, TextAttention, VisionAttention, workloads
    dev = torch.device("cuda", 0)
    w = workloads.config(cfg, seed=seed, device=dev)
    if fp32:
        if cfg == "C4":
            raise SystemExit("--fp32 applies to the text configurations C0-C3 and S")
        w["qkv"] = w["qkv"].float()
    if cfg == "C4":
        vis = VisionAttention(w["heads"], w["hd"], device=dev)
        plan = AttnPlan(w["cu_seqlens"], causal=False, device=dev)
        out = torch.empty((plan.T, vis.E), dtype=torch.bfloat16, device=dev)
        scratch = vis.scratch(plan.T, plan.kvT)
        step = lambda: vis.forward(w["qkv"], w["bias"], w["pos2"], plan, out=out, scratch=scratch)
        info = dict(workload="C4 vision: 4 images x 1,024 patches (32x32), bidirectional, 16 heads MHA, "
                    "hd 72, 2-D rotary", tokens=plan.T, pairs=plan.pairs(), hd=w["hd"], nh=w["heads"],
                    bytes=plan.T * 3 * vis.E * 2 + plan.T * vis.E * 2, core=None)
        return step, None, None, info, w
    att = TextAttention(w["nh"], w["nkv"], w["hd"], w["n_rot"], rope_theta=w["theta"], device=dev)
    if cfg == "C3":
        plan = AttnPlan(w["cu_seqlens"], w["cu_seqlens_k"], causal=True, device=dev)
        if fp32:
            kp, vt = w["k_cache"].float().contiguous(), w["v_cache"].float().contiguous()
        else:
            kp = w["k_cache"].half().contiguous()   # f16 K plane
            vt = w["v_cache"].transpose(1, 2).contiguous()
        kvT = kp.shape[1]
    else:
        plan = AttnPlan(w["cu_seqlens"], causal=True, device=dev)
        kvT = plan.kvT
        kp, vt = att.planes(kvT, fp32=fp32)
    out = torch.empty((plan.T, w["nh"] * w["hd"]), dtype=torch.bfloat16, device=dev)
    kwargs = dict(out=out, gate=w["gate"], k_plane=kp, vt_plane=vt, kvT=kvT,
                  rope_cs=att.rope_table(plan.T) if w["n_rot"] else None)
    args = (w["qkv"], w["q_norm"], w["k_norm"], w["pos3"], plan)
    step = lambda: att.forward(*args, stage="prefill", **kwargs)
    core = lambda: att.forward(*args, stage="core", **kwargs)
    prep = lambda: att.forward(*args, stage="prep", **kwargs)
    layer = None
    if not fp32:
        # The engine's path: the QKV GEMM (hidden 5,120, the 27B width) writes the qkv rows and,
        # in its epilogue, the K / V^T planes and rope_cs; the attention kernel follows.
        X, Wq = workloads.qkv_projection(plan.T, w["nh"], w["nkv"], w["hd"], H=5120, seed=seed, device=dev,
                                         outlier_frac=0.0 if cfg in ("C0", "C2", "C3") else 0.02)
        qkv_out = torch.empty_like(w["qkv"])
        fused = lambda: att.project(X, Wq, plan, w["q_norm"], w["k_norm"], w["pos3"], qkv=qkv_out, k_plane=kp,
                                    vt_plane=vt, kvT=kvT, rope_cs=kwargs["rope_cs"])
        plain = lambda: att.project(X, Wq, plan, qkv=qkv_out, prologue=False)
        core_l = lambda: att.forward(qkv_out, w["q_norm"], w["k_norm"], w["pos3"], plan, stage="core", **kwargs)
        layer = dict(fused=fused, plain=plain, layer=lambda: (fused(), core_l()), H=5120)
    T, nh, nkv, hd = plan.T, w["nh"], w["nkv"], w["hd"]
    # algorithmic bytes: qkv rows read once, O written once, cached K/V read (C3)
    esz = 4 if fp32 else 2
    nbytes = T * (2 * nh + 2 * nkv) * hd * esz + T * nh * hd * 2
    if cfg == "C3":
        nbytes += 2 * nkv * (int(w["cu_seqlens_k"][-1]) - T) * hd * esz
    names = {"C0": "C0 one causal 1,024-token record, 16/4 heads, hd 256, plain SDPA operands (no norm, "
                   "rotary or gate)",
             "C1": "C1 packed varlen causal micro-batch: 8 records, 4,096 tokens, 24/4 heads, hd 256, "
                   "fused q/k RMSNorm + rotary(64, theta 1e7) + sigmoid gate",
             "C2": "C2 single causal request: 16,384 tokens, 24/4 heads, hd 256, fused prologue/gate",
             "C3": "C3 prefix-cache continuation: 4 x (2,048 cached + 512 new), 16/4 heads, hd 256",
             "S": "S batch of short records: 256 x 16 tokens (4,096 tokens), 24/4 heads, hd 256, fused "
                  "q/k RMSNorm + rotary(64, theta 1e7) + sigmoid gate"}
    # the attention kernel alone: Q and gate rows read once, each K / V plane row read once, O
    # written once (the scope of roofline.traffic)
    kv_rows = int(w["cu_seqlens_k"][-1]) if cfg == "C3" else T
    core_bytes = T * 2 * nh * hd * esz + 2 * nkv * kv_rows * hd * (4 if fp32 else 2) + T * nh * hd * 2
    info = dict(workload=names[cfg], tokens=T, pairs=plan.pairs(), hd=hd, nh=nh, bytes=nbytes, core_bytes=core_bytes,
                lengths=[int(x) for x in np.diff(plan.cu_q)], layer=layer)
    return step, core, prep, info, w


def time_fn(fn, steps, warmup, graph):
    """Mean ms per call over `steps` calls (HIP events on the launch stream)."""
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    per = 1
    g = None
    if graph:
        per = next(d for d in (10, 5, 4, 2, 1) if steps % d == 0)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(per):
                fn()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    if g is not None:
        for _ in range(steps // per):
            g.replay()
    else:
        for _ in range(steps):
            fn()
    end.record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3
    return start.elapsed_time(end) / steps, wall / steps


def warm(fn, steps, warmup, graph):
    """Untimed passes of fn, as time_fn runs them, for at least WARM_S seconds (device clocks)."""
    t0 = time.perf_counter()
    while True:
        time_fn(fn, steps, warmup, graph)
        if time.perf_counter() - t0 >= WARM_S:
            return


def cpu_baseline(w, cfg):
    """fp32 CPU oracle (OpenMP) on the same inputs: prologue + attention, median of 5 runs."""
    from cleffa_amd import rope_inv_freq
    from oracle import oracle
    qkv = w["qkv"].float().cpu().numpy()
    nh, nkv, hd, n_rot = w["nh"], w["nkv"], w["hd"], w["n_rot"]
    inv = rope_inv_freq(w["theta"], n_rot) if n_rot else None
    qn = None if w["q_norm"] is None else w["q_norm"].cpu().numpy()
    kn = None if w["k_norm"] is None else w["k_norm"].cpu().numpy()
    pos = w["pos3"].cpu().numpy()

    def run():
        Q, K, V, G = oracle.text_prep(qkv, nh, nkv, hd, n_rot, qn, kn, pos, inv, precision="f32")
        oracle.attention(Q, K, V, w["cu_seqlens"], None, True, hd ** -0.5, G if w["gate"] else None,
                         precision="f32")

    run()
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), oracle.num_threads()


def bench_prefix_growth(a):
    """Growth copy of one layer's prefix-cache planes (nkv 4, hd 256): an entry of 65,536 rows
    grows to 81,920, keeping all 65,536 (600 MB moved, more than the 256 MB last-level cache).
    Algorithmic bytes: the kept rows read once, every row of the new planes written once."""
    import ctypes
    from cleffa_amd import _lib
    nkv, hd, src_cap, dst_cap, keep = 4, 256, 65536, 81920, 65536
    lib = _lib.load()
    ks = torch.randn(nkv, src_cap, hd, device="cuda").bfloat16()
    vs = torch.randn(nkv, hd, src_cap, device="cuda").bfloat16()
    kd = torch.empty(nkv, dst_cap, hd, device="cuda", dtype=torch.bfloat16)
    vd = torch.empty(nkv, hd, dst_cap, device="cuda", dtype=torch.bfloat16)
    err = ctypes.create_string_buffer(256)

    def step():
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _lib.check(lib.clef_hip_prefix_copy(ks.data_ptr(), vs.data_ptr(), src_cap, kd.data_ptr(), vd.data_ptr(),
                                            dst_cap, nkv, hd, keep, s, err, 256), err)

    warm(step, a.steps, a.warmup, not a.no_graph)
    ms, wall_ms = time_fn(step, a.steps, a.warmup, not a.no_graph)
    nbytes = 2 * nkv * hd * 2 * (keep + dst_cap)
    gbs = nbytes / (ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "prefix-cache growth copy GB/s (one layer, 4 x 256 planes, 65,536 -> 81,920 rows)",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms, 5), "host_ms_per_step": round(wall_ms, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "u16", "data": "synthetic",
        "config": {"workload": "P prefix growth copy", "bytes": nbytes},
        "roofline": {"bound": "hbm", "kernel": "prefix_copy_kernel", "achieved": round(gbs, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                     "traffic": None, "launch_ms": round(ms, 5)},
    }), flush=True)


PEAK_F32_MFMA = 157.3       # MI355X dense fp32 MFMA TFLOP/s (published)
PEAK_F64_MFMA = 78.6        # MI355X dense fp64 MFMA TFLOP/s (published)


def bench_omni(a):
    """Omni decoder attention, one causal record of 16,344 tokens (the largest default length of
    bench/omni_attention_bench.m), 32/4 heads, hd 128, FP32 operands. Step = prep + attention.
    Half the flops (S = Q.K^T) run on fp32 MFMA and half (P.V) on fp64 MFMA, so the matrix-core
    ceiling for the attention kernel is 2 / (1/157.3 + 1/78.6) = 104.8 TFLOP/s."""
    from cleffa_amd.omni import OmniAttention, OmniPlan
    T, nh, nkv = 16344, 32, 4
    g = torch.Generator(device="cuda")
    g.manual_seed(a.seed)
    qkv = torch.randn(T, (nh + 2 * nkv) * 128, generator=g, device="cuda")
    qn = 1 + 0.1 * torch.randn(128, generator=g, device="cuda")
    kn = 1 + 0.1 * torch.randn(128, generator=g, device="cuda")
    pos3 = torch.arange(T, device="cuda", dtype=torch.int32)[:, None].repeat(1, 3).contiguous()
    att = OmniAttention(nh, nkv)
    plan = OmniPlan([0, T])
    planes = att.planes(T)
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    out = torch.empty(T, nh * 128, device="cuda")
    step = lambda: (att.prep(qkv, qn, kn, pos3, planes=planes, status=status), att.attention(*planes, plan, out=out))
    core = lambda: att.attention(*planes, plan, out=out)
    step()
    warm(step, a.steps, a.warmup, not a.no_graph)
    ms, wall_ms = time_fn(step, a.steps, a.warmup, not a.no_graph)
    core_ms, _ = time_fn(core, a.steps, a.warmup, not a.no_graph)
    flops = 4.0 * 128 * nh * plan.pairs()
    peak = 2.0 / (1.0 / PEAK_F32_MFMA + 1.0 / PEAK_F64_MFMA)
    achieved = flops / (core_ms * 1e-3) / 1e12
    print(json.dumps({
        "metric": "Omni attention TFLOP/s (16,344-token causal record, 32/4 heads, hd 128, FP32 in, FP64 accumulate)",
        "value": round(flops / (ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s",
        "tokens_per_s": round(T / (ms * 1e-3), 1), "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms, 5), "host_ms_per_step": round(wall_ms, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded N(0,1))",
        "config": {"workload": "O Omni attention: 1 x 16,344 tokens, 32/4 heads, hd 128", "gflop": round(flops / 1e9, 2)},
        "roofline": {"bound": "mfma", "kernel": "omni_attn_kernel<8>", "achieved": round(achieved, 2),
                     "peak": round(peak, 1), "unit": "TFLOP/s", "frac": round(achieved / peak, 4),
                     "traffic": None, "launch_ms": round(core_ms, 5)},
        "prep_ms": round(ms - core_ms, 5),
    }), flush=True)


def bench_gemms(a):
    """The projections either side of the C1 layer at the 27B model's widths (H 5120, 24 x 256
    query + gate, 4 x 256 K and V): QKV [4096 x 5120] . [14336 x 5120]^T -> bf16 qkv rows, and
    o_proj [4096 x 6144] . [5120 x 6144]^T accumulated into the f32 residual. Step = both."""
    from cleffa_amd.gemm import gemm
    T, H, nq = 4096, 5120, 6144
    nqkv = 2 * nq + 2 * 4 * 256
    g = torch.Generator(device="cuda")
    g.manual_seed(a.seed)
    xn = torch.randn(T, H, generator=g, device="cuda").bfloat16()
    wqkv = (0.02 * torch.randn(nqkv, H, generator=g, device="cuda")).bfloat16()
    attn = torch.randn(T, nq, generator=g, device="cuda").bfloat16()
    wo = (0.02 * torch.randn(H, nq, generator=g, device="cuda")).bfloat16()
    qkv = torch.empty(T, nqkv, dtype=torch.bfloat16, device="cuda")
    resid = torch.zeros(T, H, device="cuda")
    ws = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")
    f_qkv, f_o = 2.0 * T * nqkv * H, 2.0 * T * H * nq
    qkv_fn = lambda: gemm(xn, wqkv, Y=qkv, out="bf16", workspace=ws)
    o_fn = lambda: gemm(attn, wo, Y=resid, out="f32", acc=True, workspace=ws)
    qkv_fn(); o_fn()
    warm(qkv_fn, a.steps, a.warmup, not a.no_graph)
    ms_q, _ = time_fn(qkv_fn, a.steps, a.warmup, not a.no_graph)
    ms_o, _ = time_fn(o_fn, a.steps, a.warmup, not a.no_graph)
    # this build's own QKV kernel (clef_hip_qkv_gemm) on the same operands, with C1's plan: the
    # product alone, and with the K/V prologue fused into its epilogue
    from cleffa_amd import AttnPlan, TextAttention, workloads
    wl = workloads.config("C1", seed=a.seed)
    att = TextAttention(24, 4, 256, 64, rope_theta=1e7)
    plan = AttnPlan(wl["cu_seqlens"], causal=True)
    qn, kn, p3 = wl["q_norm"].cuda(), wl["k_norm"].cuda(), wl["pos3"].cuda()
    kp, vt = att.planes(plan.kvT)
    cs = att.rope_table(T)
    own_fn = lambda: att.project(xn, wqkv, plan, qkv=qkv, prologue=False)
    fused_fn = lambda: att.project(xn, wqkv, plan, qn, kn, p3, qkv=qkv, k_plane=kp, vt_plane=vt, rope_cs=cs)
    own_fn(); fused_fn()
    ms_own, _ = time_fn(own_fn, a.steps, a.warmup, not a.no_graph)
    ms_fused, _ = time_fn(fused_fn, a.steps, a.warmup, not a.no_graph)
    t_own, t_fused = f_qkv / (ms_own * 1e-3) / 1e12, f_qkv / (ms_fused * 1e-3) / 1e12
    tq, to = f_qkv / (ms_q * 1e-3) / 1e12, f_o / (ms_o * 1e-3) / 1e12
    ms = ms_q + ms_o
    print(json.dumps({
        "metric": "QKV + o_proj GEMM TFLOP/s (C1 layer, 4,096 tokens, 27B widths)",
        "value": round((f_qkv + f_o) / (ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded N(0,1))",
        "config": {"workload": "G: QKV 4096x14336x5120 -> bf16, o_proj 4096x5120x6144 += f32"},
        "qkv": {"ms": round(ms_q, 5), "tflops": round(tq, 1), "frac": round(tq / PEAK_BF16_TFLOPS, 4)},
        "o_proj": {"ms": round(ms_o, 5), "tflops": round(to, 1), "frac": round(to / PEAK_BF16_TFLOPS, 4)},
        "qkv_own_kernel": {"ms": round(ms_own, 5), "tflops": round(t_own, 1), "frac": round(t_own / PEAK_BF16_TFLOPS, 4)},
        "qkv_own_fused_prologue": {"ms": round(ms_fused, 5), "tflops": round(t_fused, 1),
                                   "frac": round(t_fused / PEAK_BF16_TFLOPS, 4)},
        "roofline": {"bound": "mfma", "kernel": "hipBLASLt (QKV)", "achieved": round(tq, 1), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tq / PEAK_BF16_TFLOPS, 4), "traffic": None,
                     "launch_ms": round(ms_q, 5)},
    }), flush=True)


def mfma_ceiling(random, iters=4000):
    """(TF/s, GHz) of clef_hip_mfma_ceiling: the attention kernels' MFMA operand stream with
    random or constant-pattern bf16 operands, and the shader clock it held."""
    import ctypes
    from cleffa_amd import _lib
    lib = _lib.load_bench()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    scratch = torch.empty(cus * (2048 + 16), dtype=torch.uint8, device="cuda")
    tf, ghz = ctypes.c_double(0.0), ctypes.c_double(0.0)
    err = ctypes.create_string_buffer(256)
    torch.cuda.synchronize()
    _lib.check(lib.clef_hip_mfma_ceiling(int(random), iters, scratch.data_ptr(), scratch.numel(),
                                         ctypes.byref(tf), ctypes.byref(ghz), err, len(err)), err)
    return tf.value, ghz.value


def bench_mfma_ceiling(a):
    c_tf, c_ghz = mfma_ceiling(False)   # constant operands first, on the cooler part
    r_tf, r_ghz = mfma_ceiling(True)
    print(json.dumps({
        "metric": "MFMA ceiling of the attention operand stream (v_mfma_f32_16x16x32_bf16, one "
                  "ds_read_b128 A operand per product, 8 waves per CU)",
        "value": round(r_tf, 1), "unit": "TFLOP/s", "n_gpus": 1, "higher_is_better": True,
        "dtype": "f32" if a.fp32 else "bf16", "data": "synthetic: random bf16 operands (the value) and a constant bit pattern",
        "config": {"workload": "MFMA ceiling, random and constant operands"},
        "random": {"tflops": round(r_tf, 1), "clock_ghz": round(r_ghz, 3), "frac": round(r_tf / PEAK_BF16_TFLOPS, 4)},
        "constant": {"tflops": round(c_tf, 1), "clock_ghz": round(c_ghz, 3), "frac": round(c_tf / PEAK_BF16_TFLOPS, 4)},
        "vs_baseline": None,
    }), flush=True)


def main():
    a = parse()
    if a.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                          "(the path would shard by records or kv heads; no multi-GPU run is launched)"}))
        sys.exit(2)
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(2)
    torch.cuda.set_device(0)
    if a.config == "P":
        return bench_prefix_growth(a)
    if a.config == "O":
        return bench_omni(a)
    if a.config == "G":
        return bench_gemms(a)
    if a.config == "M":
        return bench_mfma_ceiling(a)
    step, core, prep, info, w = build_step(a.config, a.seed, a.fp32)
    if a.profile_pass:
        src = torch.randn(CALIB_BYTES // 2, device="cuda").to(torch.bfloat16)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)                     # the runtime's copy kernel
        torch.mul(src, 1.0, out=dst)       # and an elementwise kernel with plain vector loads
        for _ in range(3):
            step()
        torch.cuda.synchronize()
        print(f"profile pass done: copy of {CALIB_BYTES} bytes, 3 steps of {a.config}", flush=True)
        return
    graph = not a.no_graph
    # Untimed passes of the same shape first, for at least WARM_S seconds: in a fresh process the
    # first passes of a HIP graph ran 8-12% slower than later ones (C1 at --steps 20: 86.5 us for
    # the first timed pass after one untimed pass, 76.3 us in the passes a second later), while
    # the device's clocks come up. The timed pass is then K steps after W warmup steps, as ever.
    warm(step, a.steps, a.warmup, graph)
    ms, wall_ms = time_fn(step, a.steps, a.warmup, graph)
    layer = info.get("layer")
    layer_info = None
    if layer is not None and not a.no_layer:
        # The engine's layer: the QKV GEMM with the K/V prologue in its epilogue, then the
        # attention kernel. Medians of interleaved runs; the attention's share of the layer is
        # (GEMM with prologue + kernel) - plain GEMM.
        t = {"layer": [], "plain": [], "fused": []}
        for _ in range(3):
            for k in t:
                t[k].append(time_fn(layer[k], a.steps, a.warmup, graph)[0])
        med = {k: statistics.median(v) for k, v in t.items()}
        layer_info = {"hidden": layer["H"], "layer_ms": round(med["layer"], 5), "qkv_gemm_ms": round(med["plain"], 5),
                      "qkv_gemm_fused_prologue_ms": round(med["fused"], 5),
                      "prologue_in_gemm_ms": round(med["fused"] - med["plain"], 5),
                      "attention_share_of_layer_ms": round(med["layer"] - med["plain"], 5),
                      "core_in_layer_ms": round(med["layer"] - med["fused"], 5)}
    flops = 4.0 * info["hd"] * info["nh"] * info["pairs"]
    tflops = flops / (ms * 1e-3) / 1e12
    res = {
        "metric": "prefill attention TFLOP/s (4096-tok packed causal GQA micro-batch, hd 256)"
        if a.config == "C1" and not a.fp32 else f"prefill attention TFLOP/s ({a.config}{', FP32 mode' if a.fp32 else ''})",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "tokens_per_s": round(info["tokens"] / (ms * 1e-3), 1),
        "mfma_peak_frac": round(tflops / PEAK_BF16_TFLOPS, 4),
        "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms, 5), "host_ms_per_step": round(wall_ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32" if a.fp32 else "bf16", "data": "synthetic (seeded N(0,1) inputs, random-init norm weights)",
        "config": {"workload": info["workload"], "seed": a.seed, "tokens": info["tokens"],
                   "pairs": info["pairs"], "gflop": round(flops / 1e9, 3),
                   **({"lengths": info["lengths"]} if "lengths" in info else {})},
    }
    if core is not None:
        # The kernel alone and inside the step: five interleaved rounds of the step, the kernel
        # alone and the K/V prologue alone (each round K steps), medians, so that all three see
        # the same clock; in-step = step - prologue.
        rounds = {"step": [], "core": [], "prep": []}
        for _ in range(5):
            for k, f in (("step", step), ("core", core), ("prep", prep)):
                rounds[k].append(time_fn(f, a.steps, a.warmup, graph)[0])
        core_ms = statistics.median(rounds["core"])
        achieved = flops / (core_ms * 1e-3) / 1e12
        peak = PEAK_F32_MFMA if a.fp32 else PEAK_BF16_TFLOPS
        kname = f"attn_text_f32_kernel<{info['nh'] // w['nkv']}>" if a.fp32 else "attn_text_kernel<64>"
        res["roofline"] = {"bound": "mfma", "kernel": kname,
                           "achieved": round(achieved, 2), "peak": peak, "unit": "TFLOP/s",
                           "frac": round(achieved / peak, 4),
                           "traffic": None if a.fp32 else measured_traffic(a.config),
                           "launch_ms": round(core_ms, 5),
                           "algorithmic_bytes": info["core_bytes"],
                           "step_algorithmic_bytes": info["bytes"],
                           "hbm_frac_at_this_time": round(info["core_bytes"] / (core_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
        # the same MFMA operand stream with random operands, measured now on this device: the
        # rate the part's power and clock allow (the nominal peak assumes 2.4 GHz)
        if not a.fp32:
            ceil_tf, ceil_ghz = mfma_ceiling(True)
            res["roofline"].update({"mfma_stream_ceiling": round(ceil_tf, 1), "mfma_stream_clock_ghz": round(ceil_ghz, 3),
                                    "frac_of_stream_ceiling": round(achieved / ceil_tf, 4)})
        # the kernel as it runs inside the step: the step minus the K/V prologue kernel alone
        prep_ms = statistics.median(rounds["prep"])
        in_step = statistics.median(rounds["step"]) - prep_ms
        ach = flops / (in_step * 1e-3) / 1e12
        res["roofline"].update({"launch_ms_in_step": round(in_step, 5), "step_ms_rounds": round(statistics.median(rounds["step"]), 5), "achieved_replay": res["roofline"]["achieved"],
                                "frac_replay": res["roofline"]["frac"], "achieved": round(ach, 2),
                                "frac": round(ach / peak, 4)})
        if "frac_of_stream_ceiling" in res["roofline"]:
            res["roofline"]["frac_of_stream_ceiling"] = round(ach / res["roofline"]["mfma_stream_ceiling"], 4)
        res["prep_ms"] = round(prep_ms, 5)
        if layer_info is not None:
            res["layer"] = layer_info
    if not a.no_cpu and a.config == "C1" and not a.fp32:
        sec, threads = cpu_baseline(w, a.config)
        res["cpu_baseline"] = {"value": round(flops / sec / 1e12, 5), "unit": "TFLOP/s",
                               "tokens_per_s": round(info["tokens"] / sec, 1), "ms": round(sec * 1e3, 2),
                               "cores": threads, "kind": "port",
                               "sample": "the full C1 step (prologue + attention, 4,096 tokens) in fp32, "
                                         "median of 5 runs"}
        # the reference's CPU configuration (C0: one causal 1,024-token record, 16/4 heads, plain
        # SDPA operands), timed the same way
        from cleffa_amd import workloads
        w0 = workloads.config("C0", seed=a.seed)
        sec0, _ = cpu_baseline(w0, "C0")
        f0 = 4.0 * 256 * 16 * (1024 * 1025 // 2)
        res["cpu_baseline"]["c0"] = {"ms": round(sec0 * 1e3, 2), "tflops": round(f0 / sec0 / 1e12, 5),
                                     "gflop": round(f0 / 1e9, 3)}
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
