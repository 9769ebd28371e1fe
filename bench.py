#!/usr/bin/env python3
"""DiT denoise-step benchmark on one MI355X.

Workload: one 1024x1024 denoise step of the
32-layer DiT with classifier-free guidance as ONE batch-2 forward
(cond + uncond stacked, 4096 image + 256 text tokens each, M = 8704 rows in
every linear), hidden 3072, 24 x 128 heads, GELU-tanh MLP 12288,
shift/scale/gate adaLN, biases, int8 weight-only block linears with fp32
per-output-channel scales, bf16 activations, fp32 softmax. Weights and
inputs are seeded synthetic data generated on the device (no checkpoint).

Timed region: K forward steps (embed, conditioning, 32 blocks, final head)
with every input already resident in HBM, bracketed by a device sync and
hipEvents on the library's stream. Right after it, the same forwards run
with a HIP event pair around every stage of every block on that stream
(`in_step`, no synchronisation inside a forward); the dominant kernel's
average there (the down-projection GEMM, M=8704 K=12288 N=3072,
residual-gate epilogue, with the int8 weight's widening pass ahead of it
in the same span) is the roofline entry's launch time. Every linear shape and the attention
kernel are also timed alone, back to back, for the breakdown.

cpu_baseline: the CPU oracle (oracle/, OpenMP) on BASELINE configs[0]-[2]
(block, linear sweep, SDPA; 1 warm-up + median of 5), composed to a step.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
       python bench.py --profile-kernel   (launches for rocprofv3 --pmc)
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0

CFG = dict(hidden=3072, heads=24, mlp_width=12288, text_dim=4096, z_dim=64, layers=32,
           mlp_act=1, adaln_shift=1, has_bias=1, text_causal=0, int8_weights=1)
TEXT, GH, GW, BATCH, SIGMA, SEED = 256, 64, 64, 2, 0.5, 2026
W8_MIN_K = 8192  # int8 linears with K >= this may widen in LDS inside the GEMM ("_w8")


def int8_in_lds(M, K, N, cus=256):
    """The library's automatic int8 route for an M-row linear (linear_impl
    in h3_gpu_hip.cpp): True where the "_w8" kernels widen the weight in LDS
    inside the GEMM, False where a widening pass runs ahead of the bf16
    kernels (or, for at most 8 rows, the GEMV kernels widen in registers).
    A launch of at most cus / 2 tiles widens by a pass; a larger one of
    fewer than 512 rows stays on "_w8"; from 512 rows "_w8" needs K >= 8192
    and a shape on which the bf16 kernels would not take 224-row tiles."""
    tn = (N + 255) // 256
    tiles = (M + 255) // 256 * tn
    if M <= 8 or 2 * tiles <= cus:
        return False
    if M < 512:
        return True
    if K < W8_MIN_K:
        return False
    r = tiles % cus
    w256 = tiles // cus + ((0.5 if 2 * r <= cus else 1.0) if r else 0.0)
    w224 = 0.875 * (((M + 223) // 224 * tn + cus - 1) // cus)
    return not w224 < 0.97 * w256


def load_qdit():
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "qdit", os.path.join(ROOT, "qwen-metal_amd", "qdit.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def flops(cfg, rows, text_rows, batch):
    H, F, heads = cfg["hidden"], cfg["mlp_width"], cfg["heads"]
    f1 = 2 * F if cfg["mlp_act"] == 0 else F
    per_row = 3 * H * H + H * H + f1 * H + F * H
    lin = 2.0 * rows * per_row * cfg["layers"] * batch
    image = rows - text_rows
    text_keys = text_rows * (text_rows + 1) // 2 if cfg["text_causal"] else text_rows * text_rows
    visible = text_keys + image * rows
    sdpa = 4.0 * 128 * heads * visible * cfg["layers"] * batch
    extra = 2.0 * batch * (text_rows * (cfg["text_dim"] * H + H * H) + image * cfg["z_dim"] * H +
                           rows * H * cfg["z_dim"])
    return lin, sdpa, extra


def time_ms(gpu, fn, reps):
    gpu.submit()
    gpu.timer_begin()
    for _ in range(reps):
        fn()
    return gpu.timer_end() / reps


def kernel_breakdown(qd, gpu, reps=10):
    """Each linear shape of the step and the attention kernel, alone, on the
    library's stream. `ms` is the int8 linear as the step runs it: at this
    workload all four are two launches, the weight widening pass
    (qw_widen_i8_bf16) and the bf16 GEMM with the scale in its epilogue (the
    out and down projections on 224-row tiles), both also timed on their own
    (`widen_ms`, `gemm_ms`); a shape the library runs on a "_w8" kernel (the
    int8 weight widened in LDS inside the GEMM) is one launch, `gemm_ms`
    being that launch."""
    H, F, M = CFG["hidden"], CFG["mlp_width"], BATCH * (TEXT + GH * GW)
    L = qd.lib()
    a = gpu.new(M * F, qd.BF16)
    out = gpu.new(M * 3 * H, qd.BF16)
    gpu.check(L.qw_gpu_fill_normal_bf16(gpu.h, a.h, 0, M * F, 1, 1, 1.0, 0.0), "fill")
    # the step's epilogues: q/k norm + RoPE, residual gate, GELU, residual gate
    shapes = {"qkv": (H, 3 * H, qd.LINEAR_QKNORM), "out": (H, H, qd.LINEAR_GATE),
              "up": (H, F, qd.LINEAR_GELU), "down": (F, H, qd.LINEAR_GATE)}
    R = TEXT + GH * GW
    ep = epilogue_operands(qd, gpu, M, R)
    res = {}
    for name, (k, n, epi) in shapes.items():
        wb = gpu.new(n * k, qd.BF16)
        q = gpu.new(n * k, qd.I8)
        s = gpu.new(n, qd.F32)
        gpu.check(L.qw_gpu_fill_normal_bf16(gpu.h, wb.h, 0, n * k, 1, 2, 0.02, 0.0), "fill")
        gpu.check(L.h3_gpu_quantize_weight_int8(gpu.h, q.h, s.h, wb.h, n, k), "quant")
        big = gpu.new(M * n, qd.BF16) if n > 3 * H else out
        kw = ep.get(epi, {})
        full = lambda: gpu.linear(big, a, q, M, k, n, wscale=s, epilogue=epi, **kw)  # noqa
        widen = lambda: gpu.check(L.qw_gpu_widen_int8_bf16(gpu.h, wb.h, q.h, n * k),  # noqa
                                  "widen")
        gemm = lambda: gpu.linear(big, a, wb, M, k, n, wscale=s, epilogue=epi, **kw)  # noqa
        full()
        ms = time_ms(gpu, full, reps)
        in_gemm = int8_in_lds(M, k, n)  # the library's int8 route at these rows
        if in_gemm:
            gemm_ms, widen_ms = ms, 0.0
        else:
            widen()
            widen_ms = time_ms(gpu, widen, reps)
            gemm()
            gemm_ms = time_ms(gpu, gemm, reps)
        fl = 2.0 * M * n * k
        res[name] = {"M": M, "K": k, "N": n, "ms": ms, "tflops": fl / ms / 1e9,
                     "frac_peak": fl / ms / 1e9 / PEAK_BF16_TFLOPS,
                     "int8_route": "w8 (widened in LDS)" if in_gemm else "widening pass + bf16",
                     "gemm_ms": gemm_ms, "gemm_tflops": fl / gemm_ms / 1e9,
                     "widen_ms": widen_ms,
                     "widen_gbs": 3.0 * n * k / widen_ms / 1e6 if widen_ms else None}
        wb.free()
    qkv = gpu.new(M * 3 * H, qd.BF16)
    gpu.check(L.qw_gpu_fill_normal_bf16(gpu.h, qkv.h, 0, M * 3 * H, 1, 3, 1.0, 0.0), "fill")
    att = gpu.new(M * H, qd.BF16)
    run = lambda: gpu.attention(att, qkv, qkv, qkv, BATCH, R, R, CFG["heads"], 3 * H, 3 * H,  # noqa
                                3 * H, H, 0, H, 2 * H, text_rows=TEXT, text_causal=0)
    run()
    ms = time_ms(gpu, run, reps)
    _, sd, _ = flops(dict(CFG, layers=1), R, TEXT, BATCH)
    res["attention"] = {"batch": BATCH, "q_rows": R, "heads": CFG["heads"], "ms": ms,
                        "tflops": sd / ms / 1e9, "frac_peak": sd / ms / 1e9 / PEAK_BF16_TFLOPS}
    return res


SPAN_NAMES = ["ln1", "qkv", "attention", "out", "ln2", "up", "down"]  # QW_SPAN_* order


def stage_spans(qd, gpu, dit, step, steps):
    """Each stage of every block as the step runs it: `steps` forwards of
    the workload right after the timed region, with a HIP event pair per
    stage recorded on the library's stream (qw_dit_set_spans; no
    synchronisation inside a forward). Average device ms per launch, and
    for the linears and attention their FLOP rate."""
    import ctypes as C
    L = qd.lib()
    H, F, M = CFG["hidden"], CFG["mlp_width"], BATCH * (TEXT + GH * GW)
    gpu.check(L.qw_dit_set_spans(dit.h, 1), "spans on")
    acc = {n: [] for n in SPAN_NAMES}
    tags = (C.c_int * 4096)()
    ms = (C.c_double * 4096)()
    try:
        gpu.submit()
        L.qw_gpu_span_collect(gpu.h, tags, ms, 4096)  # nothing pending
        for _ in range(steps):
            step()
            n = L.qw_gpu_span_collect(gpu.h, tags, ms, 4096)
            if n < 0:
                raise RuntimeError(gpu.error())
            for i in range(n):
                acc[SPAN_NAMES[tags[i]]].append(ms[i])
    finally:
        gpu.check(L.qw_dit_set_spans(dit.h, 0), "spans off")
    _, sd, _ = flops(dict(CFG, layers=1), TEXT + GH * GW, TEXT, BATCH)
    fl = {"qkv": 2.0 * M * H * 3 * H, "out": 2.0 * M * H * H, "up": 2.0 * M * H * F,
          "down": 2.0 * M * F * H, "attention": sd}
    res = {"steps": steps, "launches_per_stage": len(acc["down"])}
    for n, v in acc.items():
        avg = sum(v) / len(v)
        res[n] = {"ms": avg}
        if n in fl:
            res[n]["tflops"] = fl[n] / avg / 1e9
            res[n]["frac_peak"] = fl[n] / avg / 1e9 / PEAK_BF16_TFLOPS
        else:
            res[n]["gbs"] = 4.0 * M * H / avg / 1e6  # read + write of [M, H] bf16
    return res


def sweep_4352(qd, gpu, reps=10):
    """BASELINE configs[1] on the GPU: the four bf16 linears at M = 4352
    with bias (plain store), W N(0, 0.02), X N(0, 1), HIP events on the
    library's stream."""
    H, F, M = CFG["hidden"], CFG["mlp_width"], TEXT + GH * GW
    L = qd.lib()
    x = gpu.new(M * F, qd.BF16)
    gpu.check(L.qw_gpu_fill_normal_bf16(gpu.h, x.h, 0, x.n, 1, 11, 1.0, 0.0), "fill")
    out = gpu.new(M * F, qd.BF16)
    res = {}
    for name, k, n in (("qkv", H, 3 * H), ("out", H, H), ("up", H, F), ("down", F, H)):
        w, b = gpu.new(n * k, qd.BF16), gpu.new(n, qd.BF16)
        gpu.check(L.qw_gpu_fill_normal_bf16(gpu.h, w.h, 0, w.n, 1, 12, 0.02, 0.0), "fill")
        gpu.check(L.qw_gpu_fill_normal_bf16(gpu.h, b.h, 0, b.n, 1, 13, 0.02, 0.0), "fill")
        run = lambda: gpu.linear(out, x, w, M, k, n, bias=b)  # noqa: E731
        run()
        ms = time_ms(gpu, run, reps)
        fl = 2.0 * M * n * k
        res[name] = {"M": M, "K": k, "N": n, "ms": ms, "tflops": fl / ms / 1e9,
                     "frac_peak": fl / ms / 1e9 / PEAK_BF16_TFLOPS}
        w.free()
        b.free()
    x.free()
    out.free()
    return res


def vendor_gemm(qd, gpu, reps=20):
    """The step's attention (against torch's SDPA) and the four step linears (bf16 W N(0, 0.02), X N(0, 1), plain store, no
    bias) through this library's GEMM and through the vendor library's
    (torch.matmul -> hipBLASLt), alternating, same inputs' distribution:
    a frame for the roofline fraction, not part of the product path."""
    import torch
    H, F, M = CFG["hidden"], CFG["mlp_width"], 2 * (TEXT + GH * GW)
    L = qd.lib()
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(7)
    res = {}
    for name, k, n in (("qkv", H, 3 * H), ("out", H, H), ("up", H, F), ("down", F, H)):
        x = gpu.new(M * k, qd.BF16)
        w = gpu.new(n * k, qd.BF16)
        out = gpu.new(M * n, qd.BF16)
        gpu.check(L.qw_gpu_fill_normal_bf16(gpu.h, x.h, 0, x.n, 1, 21, 1.0, 0.0), "fill")
        gpu.check(L.qw_gpu_fill_normal_bf16(gpu.h, w.h, 0, w.n, 1, 22, 0.02, 0.0), "fill")
        run = lambda: gpu.linear(out, x, w, M, k, n)  # noqa: E731
        run()
        tx = torch.randn(M, k, device=dev, dtype=torch.bfloat16, generator=gen)
        tw = (torch.randn(n, k, device=dev, dtype=torch.bfloat16, generator=gen) * 0.02)
        to = torch.empty(M, n, device=dev, dtype=torch.bfloat16)
        torch.matmul(tx, tw.t(), out=to)
        torch.cuda.synchronize()
        fl = 2.0 * M * n * k
        ours, vend = [], []
        for _ in range(3):
            ours.append(time_ms(gpu, run, reps))
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                torch.matmul(tx, tw.t(), out=to)
            e1.record()
            torch.cuda.synchronize()
            vend.append(e0.elapsed_time(e1) / reps)
        o, v = min(ours), min(vend)
        res[name] = {"M": M, "K": k, "N": n, "ours_ms": o, "vendor_ms": v,
                     "ours_tflops": fl / o / 1e9, "vendor_tflops": fl / v / 1e9,
                     "ours_over_vendor": v / o}
        for b in (x, w, out):
            b.free()
        del tx, tw, to
    # the step's attention (joint, full, B 2 x 24 heads x 4352 rows, d 128)
    # against torch's scaled_dot_product_attention on the same shape
    R = TEXT + GH * GW
    qkv = gpu.new(M * 3 * H, qd.BF16)
    att = gpu.new(M * H, qd.BF16)
    gpu.check(L.qw_gpu_fill_normal_bf16(gpu.h, qkv.h, 0, M * 3 * H, 1, 3, 1.0, 0.0), "fill")
    run = lambda: gpu.attention(att, qkv, qkv, qkv, BATCH, R, R, CFG["heads"], 3 * H,  # noqa
                                3 * H, 3 * H, H, 0, H, 2 * H, text_rows=TEXT, text_causal=0)
    run()
    tq, tk, tv = (torch.randn(BATCH, CFG["heads"], R, H // CFG["heads"], device=dev,
                              dtype=torch.bfloat16, generator=gen) for _ in range(3))
    sdpa = torch.nn.functional.scaled_dot_product_attention
    sdpa(tq, tk, tv)
    torch.cuda.synchronize()
    ours, vend = [], []
    for _ in range(3):
        ours.append(time_ms(gpu, run, 10))
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(10):
            sdpa(tq, tk, tv)
        e1.record()
        torch.cuda.synchronize()
        vend.append(e0.elapsed_time(e1) / 10)
    _, sd, _ = flops(dict(CFG, layers=1), R, TEXT, BATCH)
    o, v = min(ours), min(vend)
    res["attention"] = {"batch": BATCH, "rows": R, "heads": CFG["heads"], "ours_ms": o,
                        "vendor_ms": v, "ours_tflops": sd / o / 1e9,
                        "vendor_tflops": sd / v / 1e9, "ours_over_vendor": v / o}
    qkv.free()
    att.free()
    return res


def epilogue_operands(qd, gpu, M, R):
    """Operands of the step's fused epilogues: the modulation (6 slots, gate
    slots 2 / 3 through the row map of the batch-2 stack) and the q/k norm
    weights with the joint RoPE tables."""
    H = CFG["hidden"]
    L = qd.lib()
    if R != TEXT + GH * GW:  # the RoPE tables below are written for the module's geometry
        raise ValueError(f"epilogue_operands: R = {R} is not {TEXT} + {GH} x {GW}")
    mod = gpu.new(2 * 6 * H, qd.BF16)
    gpu.check(L.qw_gpu_fill_normal_bf16(gpu.h, mod.h, 0, mod.n, 1, 5, 0.3, 0.0), "fill")
    rm = np.tile((np.arange(R) < TEXT).astype(np.uint32), M // R)
    nw = gpu.new(2 * 128, qd.BF16)
    gpu.check(L.qw_gpu_fill_normal_bf16(gpu.h, nw.h, 0, nw.n, 1, 6, 0.02, 1.0), "fill")
    cos = np.empty((R, 64), np.float32)
    sin = np.empty((R, 64), np.float32)
    L.qw_pipe_rope_tables_host(TEXT, GH, GW, cos.ctypes.data, sin.ctypes.data)
    keep = [mod, nw, gpu.put(rm), gpu.put(cos), gpu.put(sin)]
    nq, nk = nw.view(0, 128), nw.view(128, 128)
    keep += [nq, nk]
    return {qd.LINEAR_GATE: dict(modulation=mod, row_map=keep[2], slots=6, gate_slot=3),
            qd.LINEAR_QKNORM: dict(qknorm=(nq, nk, keep[3], keep[4], R, 1e-6)),
            "keep": keep}


def measured_traffic():
    """HBM bytes per launch of the dominant kernel from the committed
    rocprofv3 --pmc summary (FETCH_SIZE and WRITE_SIZE, calibrated against
    a copy kernel of known size), or None when it has not been measured."""
    p = os.path.join(ROOT, "profiles", "gemm_down_int8_step_route_traffic.md")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_launch"):
                return float(line.split("=")[1])
    return None


def _median_ms(fn, runs=5):
    fn()  # warm-up
    ts = []
    for _ in range(runs):
        t = time.perf_counter()
        fn()
        ts.append((time.perf_counter() - t) * 1e3)
    return float(np.median(ts)), ts


def cpu_baseline(runs=5):
    """The CPU oracle (oracle/, C11 + OpenMP, fp32 accumulation) on the
    host cores, per BASELINE configs[0]-[2]: one warm-up then the median of
    `runs` timed runs (perf_counter, i.e. CLOCK_MONOTONIC) of
      configs[0]  one block at 64 text + 256 image rows (int8 weights off),
      configs[1]  the four linears at M = 4352 (bf16 weights, bias),
      configs[2]  the B2 x 24-head SDPA over 256 + 4096 rows.
    value: a step of the workload composed from those medians: 32 layers x
    (2 CFG branches x the four M = 4352 linears + the batch-2 SDPA), i.e.
    everything but the bandwidth-bound elementwise work (under 5% of the
    step's time on the CPU; it is in configs[0]'s block time)."""
    from oracle import oracle as o
    L = o.lib()
    H, F, hd = CFG["hidden"], CFG["mlp_width"], CFG["heads"] * 128
    res = {}
    # one block, 64 + 256 rows
    T1, R1 = 64, 64 + 256
    m = o.Model(dict(CFG, layers=1, int8_weights=0), SEED, 1)
    hid0 = o.fill_normal_bf16(R1 * H, SEED, 990)
    mod = o.fill_normal_bf16(2 * 6 * H, SEED, 991, 0.2)
    rm = (np.arange(R1) < T1).astype(np.uint32)
    c1, s1 = o.rope_tables(T1, 16, 16)
    med, ts = _median_ms(lambda: m.block(0, hid0.copy(), mod, c1, s1, rm, R1, T1), runs)
    m.close()
    res["block_320"] = {"median_ms": med, "runs_ms": ts}
    # the sweep at M = 4352
    M = TEXT + GH * GW
    x = o.fill_normal_bf16(M * F, SEED, 992)
    sweep = {}
    for name, k, n in (("qkv", H, 3 * H), ("out", H, H), ("up", H, F), ("down", F, H)):
        w = o.fill_normal_bf16(n * k, SEED, 993, 0.02)
        b = o.fill_normal_bf16(n, SEED, 994, 0.02)
        xs = x[:M * k]
        med, ts = _median_ms(lambda: o.linear(xs, w, b, M, k, n), runs)
        sweep[name] = {"median_ms": med, "gflops": 2e-6 * M * n * k / med}
    res["sweep_4352"] = sweep
    # SDPA B2 x 24 heads x 4352
    q, k_, v = (o.fill_normal_bf16(M * hd, SEED, 995 + i) for i in range(3))
    lim = o.t2i_limits(M, TEXT, 0)
    one = lambda: o.attention(q, k_, v, lim, M, M, CFG["heads"], prescale_rows=TEXT)  # noqa
    med, ts = _median_ms(lambda: (one(), one()), runs)  # batch 2
    res["sdpa_b2_4352"] = {"median_ms": med}
    lin_ms = sum(v_["median_ms"] for v_ in sweep.values())
    step = CFG["layers"] * (BATCH * lin_ms + med)
    return {"value": step, "unit": "ms/step", "cores": L.qo_num_threads(), "kind": "port",
            "sample": f"BASELINE configs[0]-[2] on the CPU oracle, 1 warm-up + median of {runs}: "
                      f"the block at 320 rows, the 4 linears at M={M}, the B2x24h SDPA at "
                      f"{M} rows; value = {CFG['layers']} x ({BATCH} x linears + SDPA)",
            "configs": res}


def calibration_copy(qd, gpu):
    """The counter calibration of the profile modes: a plain copy
    (qw_copy2d) of 256 MiB, launched three times."""
    copy_elems = 128 << 20  # bf16: 256 MiB
    src, dst = gpu.new(copy_elems, qd.BF16), gpu.new(copy_elems, qd.BF16)
    for _ in range(3):
        gpu.check(qd.lib().qw_gpu_copy_rows(gpu.h, dst.h, 0, 4096, src.h, 0, 4096,
                                            copy_elems // 4096, 4096), "copy")
    gpu.submit()
    src.free()
    dst.free()


def profile_kernel(qd, gpu, reps=5):
    """Launch-only mode for rocprofv3 --pmc passes: a plain copy of a known
    size (the counter calibration: 256 MiB read + 256 MiB written), then
    the dominant GEMM -- the down projection, M=8704 K=12288 N=3072, on the
    int8 weight with the residual-gate epilogue, as the step runs it (the
    widening pass qw_widen_i8_bf16, then qw_gemm_bf16_gate_t224) -- `reps`
    times. Nothing is timed or printed as a result."""
    H, F, M = CFG["hidden"], CFG["mlp_width"], BATCH * (TEXT + GH * GW)
    L = qd.lib()
    calibration_copy(qd, gpu)
    a = gpu.new(M * F, qd.BF16)
    gpu.check(L.qw_gpu_fill_normal_bf16(gpu.h, a.h, 0, M * F, 1, 1, 1.0, 0.0), "fill")
    wb, q, s = gpu.new(F * H, qd.BF16), gpu.new(F * H, qd.I8), gpu.new(H, qd.F32)
    gpu.check(L.qw_gpu_fill_normal_bf16(gpu.h, wb.h, 0, F * H, 1, 2, 0.02, 0.0), "fill")
    gpu.check(L.h3_gpu_quantize_weight_int8(gpu.h, q.h, s.h, wb.h, H, F), "quant")
    ep = epilogue_operands(qd, gpu, M, TEXT + GH * GW)
    out = gpu.new(M * H, qd.BF16)
    for _ in range(reps):
        gpu.linear(out, a, q, M, F, H, wscale=s, epilogue=qd.LINEAR_GATE,
                   **ep[qd.LINEAR_GATE])
    gpu.submit()


def profile_attention(qd, gpu, reps=5):
    """Launch-only mode for rocprofv3 --pmc: the calibration copy, then the
    step's attention call (batch 2 x 24 heads x 4352 rows over the fused
    q|k|v buffer, text rows attending the text prefix) `reps` times."""
    H, M, R = CFG["hidden"], BATCH * (TEXT + GH * GW), TEXT + GH * GW
    L = qd.lib()
    calibration_copy(qd, gpu)
    qkv = gpu.new(M * 3 * H, qd.BF16)
    gpu.check(L.qw_gpu_fill_normal_bf16(gpu.h, qkv.h, 0, M * 3 * H, 1, 3, 1.0, 0.0), "fill")
    att = gpu.new(M * H, qd.BF16)
    for _ in range(reps):
        gpu.attention(att, qkv, qkv, qkv, BATCH, R, R, CFG["heads"], 3 * H, 3 * H, 3 * H, H, 0,
                      H, 2 * H, text_rows=TEXT, text_causal=0)
    gpu.submit()


def block_320(qd, gpu, reps=10):
    """BASELINE configs[0] on the GPU: one DiT block (bf16 weights) at 64
    text + 256 image rows, batch 1, through qw_dit_block, HIP events on the
    library's stream."""
    L = qd.lib()
    H, T, gh, gw = CFG["hidden"], 64, 16, 16
    R = T + gh * gw
    cfg = dict(CFG, layers=1, int8_weights=0)
    dit = qd.Dit(gpu, cfg, SEED)
    hid = gpu.new(R * H, qd.BF16)
    gpu.check(L.qw_gpu_fill_normal_bf16(gpu.h, hid.h, 0, hid.n, SEED, 990, 1.0, 0.0), "fill")
    mod = gpu.new(2 * 6 * H, qd.BF16)
    gpu.check(L.qw_gpu_fill_normal_bf16(gpu.h, mod.h, 0, mod.n, SEED, 991, 0.2, 0.0), "fill")
    rm = gpu.put((np.arange(R) < T).astype(np.uint32))
    cos = np.empty((R, 64), np.float32)
    sin = np.empty((R, 64), np.float32)
    L.qw_pipe_rope_tables_host(T, gh, gw, cos.ctypes.data, sin.ctypes.data)
    ct, st = gpu.put(cos), gpu.put(sin)
    run = lambda: dit.block(0, hid, mod, ct, st, rm, R, T)  # noqa: E731
    run()
    ms = time_ms(gpu, run, reps)
    F = CFG["mlp_width"]
    fl = 2.0 * R * (3 * H * H + H * H + 2 * F * H) + 4.0 * 128 * CFG["heads"] * (T * T + (R - T) * R)
    dit.close()
    return {"rows": R, "text_rows": T, "ms": ms, "tflops": fl / ms / 1e9,
            "frac_peak": fl / ms / 1e9 / PEAK_BF16_TFLOPS}


def denoise_512(qd, gpu):
    """the 32-layer DiT (bf16 weights) in the 8-step
    FlowMatch Euler loop at 512x512 (1024 image + 128 text rows, batch 1,
    dynamic shift mu = 1), through qw_pipe_denoise. Timed twice: the loop
    with the latents resident on the device (the default) and the
    reference's host round trip per step (QW_PIPE_HOST_LOOP=1)."""
    import ctypes as C
    L = qd.lib()
    cfg = dict(CFG, int8_weights=0)
    text_rows, gh, gw, steps = 128, 32, 32, 8
    dit = qd.Dit(gpu, cfg, SEED)
    text = gpu.new(text_rows * cfg["text_dim"], qd.BF16)
    gpu.check(L.qw_gpu_fill_normal_bf16(gpu.h, text.h, 0, text.n, SEED, 820, 1.0, 0.0), "fill")
    rng = np.random.default_rng(SEED)
    x0 = rng.standard_normal(gh * gw * cfg["z_dim"]).astype(np.float32)
    # mu = 1: base_shift = max_shift = 1 over an empty sequence range

    class Sched(C.Structure):
        _fields_ = [("dynamic_shifting", C.c_int), ("base_seq", C.c_double),
                    ("max_seq", C.c_double), ("base_shift", C.c_double),
                    ("max_shift", C.c_double), ("has_terminal", C.c_int),
                    ("shift_terminal", C.c_double)]
    sc = Sched(1, 256.0, 256.0, 1.0, 1.0, 0, 0.0)
    res = {}
    for name, flag in (("device_loop_ms", "0"), ("host_loop_ms", "1")):
        os.environ["QW_PIPE_HOST_LOOP"] = flag
        best = None
        for _ in range(2):
            x = x0.copy()
            err = C.create_string_buffer(1024)
            t = time.time()
            ok = L.qw_pipe_denoise(dit.h, gpu.h, text.h, text_rows, None, 0, x.ctypes.data, gh,
                                   gw, steps, 1.0, None, 0, C.byref(sc), err, 1024)
            ms = (time.time() - t) * 1e3
            if not ok:
                raise RuntimeError(err.value.decode())
            best = ms if best is None else min(best, ms)
        res[name] = best
    os.environ.pop("QW_PIPE_HOST_LOOP", None)
    dit.close()
    res.update({"steps": steps, "image_rows": gh * gw, "text_rows": text_rows,
                "weights": "bf16", "latents_finite": bool(np.isfinite(x).all())})
    return res


def ti2i_1024(qd, gpu, dit):
    """ti2i at the workload's geometry (the step's int8 model): 256 text
    rows, a 1024x1024 condition image (4096 rows), 64 text rows and the
    1024x1024 target (4096 rows); one forward through qw_dit_forward_ti2i
    as a full pass (cache cleared) against one with the conditioning K/V
    cached (target rows only), the reference's cross-step cache
    (qwen_dit.m:1694-1699)."""
    import ctypes as C
    L = qd.lib()

    class Seg(C.Structure):
        _fields_ = [("rows", C.c_uint32), ("is_image", C.c_int), ("src_offset", C.c_uint32)]
    segs = (Seg * 4)(Seg(256, 0, 0), Seg(4096, 1, 0), Seg(64, 0, 256), Seg(4096, 1, 4096))
    rows = 256 + 4096 + 64 + 4096
    err = C.create_string_buffer(1024)
    text = gpu.new(320 * CFG["text_dim"], qd.BF16)
    lat = gpu.new(8192 * CFG["z_dim"], qd.BF16)
    gpu.check(L.qw_gpu_fill_normal_bf16(gpu.h, text.h, 0, text.n, SEED, 840, 1.0, 0.0), "fill")
    gpu.check(L.qw_gpu_fill_normal_bf16(gpu.h, lat.h, 0, lat.n, SEED, 841, 1.0, 0.0), "fill")
    # the reference's ti2i tables (qwen_pipeline.m:611-680): each block's
    # text rows, then its 64 x 64 grid with the frame frozen where it starts
    bh, bw, tb = (np.array(v, np.uint32) for v in ([64, 64], [64, 64], [256, 64]))
    cp, sp = C.c_void_p(), C.c_void_p()
    if not L.qw_pipe_rope_tables_blocks(gpu.h, bh.ctypes.data, bw.ctypes.data, tb.ctypes.data,
                                        2, C.byref(cp), C.byref(sp), err, 1024):
        raise RuntimeError(err.value.decode())
    ct, st = qd.Tensor(gpu, cp.value, rows * 64, qd.F32), qd.Tensor(gpu, sp.value, rows * 64,
                                                                   qd.F32)
    out = gpu.new(rows * CFG["z_dim"], qd.BF16)

    def run(sigma):
        if not L.qw_dit_forward_ti2i(dit.h, text.h, lat.h, segs, 4, 0, ct.h, st.h, sigma, out.h,
                                     err, 1024):
            raise RuntimeError(err.value.decode())
    full, cached = [], []
    for _ in range(2):
        L.qw_dit_ti2i_cache_clear(dit.h)
        gpu.submit()
        t = time.time()
        run(0.9)
        gpu.submit()
        full.append((time.time() - t) * 1e3)
        t = time.time()
        run(0.8)
        gpu.submit()
        cached.append((time.time() - t) * 1e3)
    L.qw_dit_ti2i_cache_clear(dit.h)
    for x in (text, lat, ct, st, out):
        x.free()
    return {"rows": rows, "target_rows": 4096, "full_pass_ms": min(full),
            "cached_step_ms": min(cached), "speedup": min(full) / min(cached)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-breakdown", action="store_true")
    ap.add_argument("--no-denoise", action="store_true",
                    help="skip the 8-step 512x512 denoise-loop measurement")
    ap.add_argument("--profile-kernel", nargs="?", const="down", default=None,
                    choices=["down", "attention"],
                    help="only launch a calibration copy and the dominant GEMM (default) or "
                         "the attention kernel, for rocprofv3 --pmc")
    ap.add_argument("--denoise-only", action="store_true",
                    help="only run the 8-step 512x512 denoise loop (BASELINE configs[3]) and "
                         "print its line, for a kernel trace of that configuration")
    ap.add_argument("--vendor", action="store_true",
                    help="only time the four step linears (bf16 W) here and through "
                         "torch.matmul (hipBLASLt), alternating, and print that line")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    if args.vendor:
        import torch  # its HIP runtime takes the device before this library's
        torch.zeros(1, device="cuda:0")
    qd = load_qdit()
    gpu = qd.Gpu()
    if args.vendor:
        print(json.dumps({"vendor_gemm": vendor_gemm(qd, gpu)}))
        gpu.close()
        return
    if args.denoise_only:
        print(json.dumps({"denoise_512_8step": denoise_512(qd, gpu)}))
        gpu.close()
        return
    if args.profile_kernel:
        (profile_attention if args.profile_kernel == "attention" else profile_kernel)(qd, gpu)
        gpu.close()
        return
    R, I = TEXT + GH * GW, GH * GW
    L = qd.lib()
    t0 = time.time()
    dit = qd.Dit(gpu, CFG, SEED)
    text = gpu.new(BATCH * TEXT * CFG["text_dim"], qd.BF16)
    lat = gpu.new(BATCH * I * CFG["z_dim"], qd.BF16)
    gpu.check(L.qw_gpu_fill_normal_bf16(gpu.h, text.h, 0, text.n, SEED, 800, 1.0, 0.0), "fill")
    gpu.check(L.qw_gpu_fill_normal_bf16(gpu.h, lat.h, 0, lat.n, SEED, 801, 1.0, 0.0), "fill")
    cos = np.empty((R, 64), np.float32)
    sin = np.empty((R, 64), np.float32)
    L.qw_pipe_rope_tables_host(TEXT, GH, GW, cos.ctypes.data, sin.ctypes.data)
    cos_t, sin_t = gpu.put(cos), gpu.put(sin)
    out = gpu.new(BATCH * R * CFG["z_dim"], qd.BF16)
    gpu.submit()
    setup_s = time.time() - t0
    # the CPU baseline first (host cores only, the device idle), so that the
    # device work -- warm-up, the timed steps, the breakdown -- runs as one
    # uninterrupted stretch at the end
    cpu = None if args.no_cpu else cpu_baseline()

    step = lambda: dit.forward_batch(text, TEXT, lat, I, BATCH, SIGMA, cos_t, sin_t, out)  # noqa
    for _ in range(args.warmup):
        step()
    gpu.submit()
    gpu.timer_begin()
    w0 = time.time()
    for _ in range(args.steps):
        step()
    dev_ms = gpu.timer_end()
    gpu.submit()
    wall_ms = (time.time() - w0) * 1e3
    ms_step = dev_ms / args.steps
    v = out.read().view(np.uint16)
    finite = bool(np.all((v & 0x7F80) != 0x7F80))

    in_step = stage_spans(qd, gpu, dit, step, min(args.steps, 10))
    lin, sdpa, extra = flops(CFG, R, TEXT, BATCH)
    total_tflops = (lin + sdpa + extra) / ms_step / 1e9
    brk = {} if args.no_breakdown else kernel_breakdown(qd, gpu)
    down = dict(M=BATCH * R, K=CFG["mlp_width"], N=CFG["hidden"], ms=in_step["down"]["ms"])
    roofline = None
    if down:
        # the dominant kernel of the step (largest total time in the kernel
        # trace): the down projection's GEMM, one launch per block (with its
        # widening pass where the route has one: the span covers both), its
        # average over the blocks of the forwards right after the timed
        # region (HIP events on the library's stream)
        fl = 2.0 * down["M"] * down["N"] * down["K"]
        achieved = fl / down["ms"] / 1e9
        roofline = {"bound": "mfma", "achieved": achieved, "peak": PEAK_BF16_TFLOPS,
                    "unit": "TFLOP/s", "frac": achieved / PEAK_BF16_TFLOPS,
                    "traffic": measured_traffic(),
                    "kernel": ("qw_gemm_w8_gate_q (down projection, M=8704 K=12288 N=3072, "
                               "int8 weight widened to bf16 in LDS once per workgroup, scale "
                               "and residual gate in the epilogue)"
                               if int8_in_lds(down["M"], down["K"], down["N"]) else
                               "qw_widen_i8_bf16 + qw_gemm_bf16_gate_t224 (down projection, "
                               "M=8704 K=12288 N=3072: the int8 weight widened to bf16 by a "
                               "pass, then 224 x 256 tiles in 2 waves, scale and residual "
                               "gate in the epilogue; the span covers both launches)"),
                    "flop_per_launch": fl, "ms_per_launch": down["ms"],
                    "ms_per_launch_alone": brk["down"]["ms"] if brk else None,
                    # A bf16 + W int8 + row scales + residual and output bf16
                    "algorithmic_bytes_per_launch": (2.0 * down["M"] * down["K"] +
                                                     down["N"] * down["K"] + 4.0 * down["N"] +
                                                     4.0 * down["M"] * down["N"])}
    sweep = None if args.no_breakdown else sweep_4352(qd, gpu)
    blk = None if args.no_breakdown else block_320(qd, gpu)
    den = None if args.no_breakdown or args.no_denoise else denoise_512(qd, gpu)
    ti2i = None if args.no_breakdown or args.no_denoise else ti2i_1024(qd, gpu, dit)
    line = {
        "metric": "DiT ms/step @1024^2 (4352 tok, CFG b=2); linear+SDPA TFLOP/s & % MFMA peak",
        "value": ms_step, "unit": "ms/step", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms_step, "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16 (int8 weight-only linears)",
        "data": "synthetic (seeded device generator; random-init weights)",
        "config": {"workload": "BASELINE configs[4]: 32-layer DiT, 1024^2, 4096 image + 256 "
                               "text tokens, CFG batch 2, int8 weight-only linears",
                   "hidden": CFG["hidden"], "heads": CFG["heads"], "mlp": CFG["mlp_width"],
                   "rows_per_linear": BATCH * R, "layers": CFG["layers"]},
        "step_tflops": total_tflops,
        "step_frac_peak": total_tflops / PEAK_BF16_TFLOPS,
        "flop_per_step": {"linear": lin, "sdpa": sdpa, "other": extra},
        "in_step": in_step,
        "breakdown": brk,
        "sweep_4352_bf16": sweep,
        "block_320_bf16": blk,
        "denoise_512_8step": den,
        "ti2i_1024_one_condition": ti2i,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "wall_ms_per_step": wall_ms / args.steps,
        "setup_s": setup_s,
        "output_finite": finite,
    }
    print(json.dumps(line))
    dit.close()
    gpu.close()


if __name__ == "__main__":
    main()
