"""CPU checks of the drop-in boundary: the C-ABI library loads, exports
every function declared in include/*.h, the ctypes table covers them, and
the code object carries every kernel the runtime looks up. No GPU calls."""
import os
import re

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
