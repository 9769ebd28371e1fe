"""CPU checks of the drop-in boundary: the C-ABI library loads, exports
every function declared in include/*.h, the ctypes table covers them, and
the code object carries every kernel the runtime looks up. No GPU calls."""
import os
import re

import ctypes as C

import numpy as np

from conftest import ROOT

INCLUDE = os.path.join(ROOT, "include")


def declared_functions():
    names = set()
    for h in os.listdir(INCLUDE):
        if not h.endswith(".h"):
            continue
        text = open(os.path.join(INCLUDE, h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"typedef[^;]*;", "", text, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b((?:h3|qw)_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol(qd):
    L = qd.lib()
    names = declared_functions()
    assert len(names) > 60
    missing = [n for n in sorted(names) if not hasattr(L, n)]
    assert not missing, missing
    untyped = [n for n in sorted(names) if n not in qd.SIGNATURES]
    assert not untyped, untyped


def test_code_object_has_every_kernel(qd):
    src = open(os.path.join(ROOT, "qwen-metal_amd", "csrc", "h3_gpu_hip.cpp")).read()
    block = src[src.index("k_names[K_COUNT]"):]
    block = block[: block.index("};")]
    kernels = re.findall(r'"(qw_\w+)"', block)
    blob = open(qd.HSACO_PATH, "rb").read()
    assert len(kernels) >= 19
    for k in kernels:
        assert k.encode() in blob, k


def test_create_without_gpu_fails_cleanly(qd):
    import ctypes as C
    if os.path.exists("/dev/kfd"):
        return  # a GPU box: covered by the gpu tests
    err = C.create_string_buffer(256)
    assert not qd.lib().h3_gpu_create(None, err, 256)
    assert err.value  # an error string, no abort


def test_host_math_matches_oracle(qd, oracle):
    """The product's own host math (qwen_host.c, qwen_pipeline.c) against
    the pinned oracle: schedule, rng, rope tables."""
    import ctypes as C
    import numpy as np
    L = qd.lib()

    class Sched(C.Structure):
        _fields_ = [("steps", C.c_int), ("sigma", C.c_float * 1001)]
    for steps, seq in [(8, 1024), (20, 4096), (50, 4096), (4, 1024)]:
        s = Sched()
        assert L.qw_schedule_build(steps, seq, C.byref(s))
        ref = np.empty(steps + 1, np.float32)
        oracle.lib().qo_schedule_build(steps, seq, ref)
        assert np.array_equal(np.array(s.sigma[: steps + 1], np.float32), ref)
    rng = (C.c_uint64 * 3)()
    orng = oracle.QoRng()
    L.qw_rng_seed(rng, 42)
    oracle.lib().qo_rng_seed(C.byref(orng), 42)
    for _ in range(50):
        assert L.qw_rng_normal(rng) == oracle.lib().qo_rng_normal(C.byref(orng))
    c = np.empty((23 + 64, 64), np.float32)
    s_ = np.empty_like(c)
    L.qw_pipe_rope_tables_host(23, 8, 8, c.ctypes.data, s_.ctypes.data)
    oc, os_ = oracle.rope_tables(23, 8, 8)
    assert np.array_equal(c, oc) and np.array_equal(s_, os_)
    # ti2i multi-block tables: two condition images and the target
    bh, bw, tb = (np.array(v, np.uint32) for v in ([12, 7, 16], [9, 7, 16], [30, 5, 11]))
    rows = L.qw_pipe_rope_tables_blocks_host(bh.ctypes.data, bw.ctypes.data, tb.ctypes.data, 3,
                                             None, None)
    assert rows == int(tb.sum() + (bh * bw).sum())
    cb = np.empty((rows, 64), np.float32)
    sb = np.empty_like(cb)
    assert L.qw_pipe_rope_tables_blocks_host(bh.ctypes.data, bw.ctypes.data, tb.ctypes.data, 3,
                                             cb.ctypes.data, sb.ctypes.data) == rows
    oc, os_ = oracle.rope_tables_blocks(bh, bw, tb)
    assert np.array_equal(cb, oc) and np.array_equal(sb, os_)
    # pipeline schedule with mu = 1 (config 4: exp(mu) = e, no terminal)
    cfg = (C.c_byte * 64)()
    L.qw_sched_cfg_default(cfg)
    sig = np.empty(9, np.float64)
    err = C.create_string_buffer(128)
    assert L.qw_pipe_schedule(8, 1024, None, 0, cfg, sig.ctypes.data, err, 128)
    ref = np.empty(9, np.float32)
    import math
    oracle.lib().qo_schedule_exp_mu(8, math.exp(oracle.lib().qo_calculate_shift(1024)), 0.02, ref)
    assert np.array_equal(sig.astype(np.float32), ref)


class SchedCfg(C.Structure):
    """qw_sched_cfg (include/qwen_pipeline.h)"""
    _fields_ = [("dynamic_shifting", C.c_int), ("base_seq", C.c_double),
                ("max_seq", C.c_double), ("base_shift", C.c_double),
                ("max_shift", C.c_double), ("has_terminal", C.c_int),
                ("shift_terminal", C.c_double)]


def _schedule(L, steps, seq, cfg, turbo=None):
    sig = np.empty(steps + 1, np.float64)
    err = C.create_string_buffer(256)
    tb = None if turbo is None else np.ascontiguousarray(turbo, np.float64)
    ok = L.qw_pipe_schedule(steps, seq, None if tb is None else tb.ctypes.data,
                            0 if tb is None else len(tb), C.byref(cfg), sig.ctypes.data, err, 256)
    return ok, sig, err.value.decode()


def test_pipe_schedule_reference_fixtures(qd):
    """qw_pipe_schedule against the reference's own pipeline fixtures, with
    the cases and 1e-6 bar of tests/test_pipeline.c:125-181: the released
    base config at 40 steps (seq 64 and 4096) and the turbo config fed the
    released 8 sample sigmas."""
    from conftest import ROOT as R
    L = qd.lib()
    fx = os.path.join(R, "tests", "golden", "pipeline_fixture")
    base = SchedCfg(1, 256.0, 8192.0, 0.5, 0.9, 1, 0.02)
    for steps, seq, name in ((40, 64, "schedule_s40"), (40, 4096, "schedule_s40_1024")):
        ok, sig, err = _schedule(L, steps, seq, base)
        assert ok, err
        ref = np.fromfile(os.path.join(fx, name + ".f32"), np.float32)
        assert ref.size == steps + 1
        assert np.max(np.abs(sig.astype(np.float32) - ref)) <= 1e-6
        # every value is a float32 (the schedule's rounding points)
        assert np.array_equal(sig.astype(np.float32).astype(np.float64), sig)
    turbo = [1.0, 0.978453, 0.95418, 0.926626, 0.89508, 0.845148, 0.704534, 0.414568]
    tcfg = SchedCfg(0, 256.0, 8192.0, 0.5, 0.9, 0, 0.0)
    ok, sig, err = _schedule(L, 8, 64, tcfg, turbo)
    assert ok, err
    ref = np.fromfile(os.path.join(fx, "schedule_t8.f32"), np.float32)
    assert np.max(np.abs(sig.astype(np.float32) - ref)) <= 1e-6


def test_pipe_schedule_matches_oracle_grid(qd, oracle):
    """Bit-exact against the oracle's restatement over step counts (1 and
    above 1000 included: the reference accepts any positive count) and
    sequence lengths; closed-form checks of the shift-free, stretch-free
    case; argument errors."""
    import math
    L = qd.lib()
    base = SchedCfg(1, 256.0, 8192.0, 0.5, 0.9, 1, 0.02)
    for steps in (1, 2, 3, 8, 28, 50, 1200):
        for seq in (64, 1024, 4096, 16384):
            ok, sig, err = _schedule(L, steps, seq, base)
            assert ok, err
            ref = np.empty(steps + 1, np.float32)
            assert oracle.lib().qo_schedule_exp_mu(
                steps, math.exp(oracle.lib().qo_calculate_shift(seq)), 0.02, ref)
            assert np.array_equal(sig.astype(np.float32), ref), (steps, seq)
            # the stretch lands the last sigma on the terminal (one step: t = 1
            # maps to sigma 1, and a zero tail leaves it unstretched)
            assert sig[-1] == 0.0
            assert abs(sig[steps - 1] - (0.02 if steps > 1 else 1.0)) < 1e-6
            assert np.all(np.diff(sig) <= 0)
    # no shift, no stretch: sigma_i is the float32 of 1 + i (1/n - 1)/(n - 1)
    plain = SchedCfg(0, 256.0, 8192.0, 0.5, 0.9, 0, 0.0)
    ok, sig, _ = _schedule(L, 5, 64, plain)
    want = np.float32([1.0 + i * (1.0 / 5 - 1.0) / 4 for i in range(5)] + [0.0])
    assert ok and np.array_equal(sig.astype(np.float32), want)
    ok, _, err = _schedule(L, 0, 64, base)
    assert not ok and "steps" in err
    ok, _, err = _schedule(L, 4, 64, plain, [1.0, 0.5])
    assert not ok and "turbo" in err
