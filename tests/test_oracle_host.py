"""Pin the oracle's host math against the reference's own known answers:
tests/host_ref.h (schedules, RoPE samples), tests/pipeline_fixture
(joint RoPE tables, schedules), tests/dit_fixture rope tables, and the
reference qwen_host.c compiled in place (oracle/_ref)."""
import ctypes as C
import math
import os

import numpy as np
import pytest

from conftest import ROOT, golden_json, read_f32

REF_SO = os.path.join(ROOT, "oracle", "_ref", "libqwen_host_ref.so")


def test_schedule_host_ref(oracle):
    # tests/test_host.c:22-52 — 2e-6 relative to max(1, sigma)
    for case in golden_json("host_ref.json")["schedule_cases"]:
        out = np.empty(case["steps"] + 1, np.float32)
        assert oracle.lib().qo_schedule_build(case["steps"], case["seq_len"], out)
        ref = np.array(case["sigmas"], np.float32)
        assert np.all(np.abs(out - ref) <= 2e-6 * np.maximum(ref, 1.0)), case["steps"]
        assert out[-1] == 0.0 and np.all(np.diff(out) <= 0)


def test_schedule_rejects_bad_steps(oracle):
    out = np.empty(1002, np.float32)
    assert oracle.lib().qo_schedule_build(0, 1024, out) == 0
    assert oracle.lib().qo_schedule_build(1001, 1024, out) == 0


def test_calculate_shift_endpoints(oracle):
    assert abs(oracle.lib().qo_calculate_shift(256) - 0.5) < 1e-12
    assert abs(oracle.lib().qo_calculate_shift(8192) - 0.9) < 1e-12


@pytest.mark.parametrize("name,steps,seq", [("schedule_s40", 40, 64),
                                            ("schedule_s40_1024", 40, 4096)])
def test_schedule_pipeline_fixture(oracle, name, steps, seq):
    # tests/test_pipeline.c:125-160: the pipeline schedule (exp(mu) in double)
    ref = read_f32(name + ".f32", "pipeline_fixture")
    out = np.empty(steps + 1, np.float32)
    exp_mu = math.exp(oracle.lib().qo_calculate_shift(seq))
    assert oracle.lib().qo_schedule_exp_mu(steps, exp_mu, 0.02, out)
    assert np.max(np.abs(out - ref)) <= 1e-6


def test_rope_samples_host_ref(oracle):
    # tests/test_host.c:54-108 — 5e-3 (libm vs torch argument reduction)
    dims = [16, 56, 56]
    c = C.c_float()
    s = C.c_float()
    for smp in golden_json("host_ref.json")["rope_samples"]:
        oracle.lib().qo_rope_table_entry(dims[smp["axis"]], smp["table_row"],
                                         smp["pair"], C.byref(c), C.byref(s))
        assert abs(c.value - smp["cos"]) < 5e-3
        assert abs(s.value - smp["sin"]) < 5e-3


@pytest.mark.parametrize("grid", [4, 8])
def test_rope_tables_pipeline_fixture(oracle, grid):
    # tests/test_pipeline.c:73-120 (23 text rows + grid x grid image)
    cos, sin = oracle.rope_tables(23, grid, grid)
    ref_c = read_f32(f"rope_cos_{grid}.f32", "pipeline_fixture").reshape(-1, 64)
    ref_s = read_f32(f"rope_sin_{grid}.f32", "pipeline_fixture").reshape(-1, 64)
    assert cos.shape == ref_c.shape
    assert np.max(np.abs(cos - ref_c)) < 1e-5
    assert np.max(np.abs(sin - ref_s)) < 1e-5


@pytest.mark.parametrize("case,text,gh,gw", [("a", 0, 4, 4), ("b", 8, 3, 4)])
def test_rope_tables_dit_fixture(oracle, case, text, gh, gw):
    ref_c = read_f32(f"{case}_rope_cos.f32").reshape(-1, 64)
    ref_s = read_f32(f"{case}_rope_sin.f32").reshape(-1, 64)
    if text == 0:
        # case a has no text rows: the image frame coordinate is 0
        cos, sin = oracle.rope_tables(0, gh, gw)
    else:
        cos, sin = oracle.rope_tables(text, gh, gw)
    assert cos.shape == ref_c.shape
    assert np.max(np.abs(cos - ref_c)) < 1e-5
    assert np.max(np.abs(sin - ref_s)) < 1e-5


def _blocks_angle_rows(positions):
    """the 64 (cos, sin) of each (frame, h, w) position, axes (16, 56, 56)"""
    c = np.empty((len(positions), 64), np.float32)
    s = np.empty_like(c)
    for r, pos in enumerate(positions):
        col = 0
        for a, dim in enumerate((16, 56, 56)):
            for p in range(dim // 2):
                ang = pos[a] * 10000.0 ** (-2.0 * p / dim)
                c[r, col], s[r, col] = math.cos(ang), math.sin(ang)
                col += 1
    return c, s


def test_rope_tables_blocks_hand_positions(oracle):
    """ti2i multi-block tables (qwen_pipeline.m:611-680) on a 3-block layout
    whose positions are written out by hand: text rows advance one
    position each, an image block's frame is the position it starts at,
    its grid is centred at (ceil(h/2), ceil(w/2)), then the position jumps
    by max(h, w)."""
    text_before, bh, bw = [3, 2, 4], [2, 1, 4], [3, 1, 2]
    pos = [(0, 0, 0), (1, 1, 1), (2, 2, 2),                       # text 0..2
           (3, -1, -2), (3, -1, -1), (3, -1, 0),                   # 2 x 3 at frame 3
           (3, 0, -2), (3, 0, -1), (3, 0, 0),
           (6, 6, 6), (7, 7, 7),                                   # 3 + max(2, 3)
           (8, -1, -1),                                            # 1 x 1 at frame 8
           (9, 9, 9), (10, 10, 10), (11, 11, 11), (12, 12, 12),    # 8 + 1
           (13, -2, -1), (13, -2, 0), (13, -1, -1), (13, -1, 0),   # 4 x 2 at frame 13
           (13, 0, -1), (13, 0, 0), (13, 1, -1), (13, 1, 0)]
    c, s = oracle.rope_tables_blocks(bh, bw, text_before)
    wc, ws = _blocks_angle_rows(pos)
    assert c.shape == (len(pos), 64)
    assert np.array_equal(c, wc) and np.array_equal(s, ws)


@pytest.mark.parametrize("text,gh,gw", [(0, 4, 4), (23, 8, 8), (64, 16, 12), (7, 5, 9)])
def test_rope_tables_blocks_single_block_is_t2i_table(oracle, text, gh, gw):
    """One block of `text` rows and a gh x gw grid is the t2i table
    (qwen_pipeline.m:212-273), whose image frame is the text length."""
    c, s = oracle.rope_tables_blocks([gh], [gw], [text])
    rc, rs = oracle.rope_tables(text, gh, gw)
    assert np.array_equal(c, rc) and np.array_equal(s, rs)


def test_timestep_features_closed_form(oracle):
    feats = oracle.timestep_features([0.37, 0.0])
    # sigma = 0 -> cos 1, sin 0 everywhere; i = 0 -> frequency 1
    assert np.all(feats[1, :128] == 1.0) and np.all(feats[1, 128:] == 0.0)
    raw = float(np.float32(0.37)) * 1000.0
    assert feats[0, 0] == np.float32(math.cos(raw))
    assert feats[0, 128] == np.float32(math.sin(raw))
    i = 64  # frequency 10000^-0.5 = 0.01
    assert abs(feats[0, i] - math.cos(raw * 0.01)) < 1e-6
    assert abs(feats[0, 128 + i] - math.sin(raw * 0.01)) < 1e-6


def test_euler_step_exact(oracle):
    # tests/test_host.c:110-123: x + (s - s_next) v, exact in float
    rng = oracle.QoRng()
    oracle.lib().qo_rng_seed(C.byref(rng), 7)
    x = np.empty(257, np.float32)
    v = np.empty(257, np.float32)
    oracle.lib().qo_rng_fill_normal(C.byref(rng), x, 257)
    oracle.lib().qo_rng_fill_normal(C.byref(rng), v, 257)
    ref = x.copy()
    oracle.lib().qo_euler_step(x, v, 257, 0.37, 0.11)
    dt = np.float32(np.float32(0.37) - np.float32(0.11))
    assert np.array_equal(x, (ref.astype(np.float64) + dt * v).astype(np.float32))


def test_rng_statistics(oracle):
    # tests/test_host.c:125-140
    a, b = oracle.QoRng(), oracle.QoRng()
    L = oracle.lib()
    L.qo_rng_seed(C.byref(a), 42)
    L.qo_rng_seed(C.byref(b), 42)
    assert all(L.qo_rng_u32(C.byref(a)) == L.qo_rng_u32(C.byref(b)) for _ in range(64))
    L.qo_rng_seed(C.byref(a), 1)
    vals = np.array([L.qo_rng_normal(C.byref(a)) for _ in range(4096)])
    assert abs(vals.mean()) < 0.08 and abs(vals.std() - 1) < 0.05


@pytest.mark.skipif(not os.path.exists(REF_SO), reason="oracle/_ref not built")
def test_against_reference_qwen_host(oracle):
    """The reference's own qwen_host.c, compiled in place, vs the oracle."""
    ref = C.CDLL(REF_SO)

    class Rng(C.Structure):
        _fields_ = oracle.QoRng._fields_

    ref.qw_rng_seed.argtypes = [C.POINTER(Rng), C.c_uint64]
    ref.qw_rng_u32.restype = C.c_uint32
    ref.qw_rng_u32.argtypes = [C.POINTER(Rng)]
    ref.qw_rng_normal.restype = C.c_float
    ref.qw_rng_normal.argtypes = [C.POINTER(Rng)]
    L = oracle.lib()
    for seed in [0, 1, 7, 42, 2**40 + 3]:
        r1, r2 = Rng(), oracle.QoRng()
        ref.qw_rng_seed(C.byref(r1), seed)
        L.qo_rng_seed(C.byref(r2), seed)
        for _ in range(100):
            assert ref.qw_rng_u32(C.byref(r1)) == L.qo_rng_u32(C.byref(r2))
        for _ in range(1001):
            assert ref.qw_rng_normal(C.byref(r1)) == L.qo_rng_normal(C.byref(r2))

    class Sched(C.Structure):
        _fields_ = [("steps", C.c_int), ("sigma", C.c_float * 1001)]

    ref.qw_schedule_build.argtypes = [C.c_int, C.c_int, C.POINTER(Sched)]
    for steps, seq in [(1, 64), (8, 1024), (20, 4096), (40, 64), (50, 8192), (1000, 300)]:
        sch = Sched()
        assert ref.qw_schedule_build(steps, seq, C.byref(sch))
        out = np.empty(steps + 1, np.float32)
        assert L.qo_schedule_build(steps, seq, out)
        assert np.array_equal(out, np.array(sch.sigma[: steps + 1], np.float32), equal_nan=True)

    class Rope(C.Structure):
        _fields_ = [("axes", C.c_int), ("axis_dim", C.c_int * 3),
                    ("cos", C.POINTER(C.c_float)), ("sin", C.POINTER(C.c_float))]

    ref.qw_rope_build.argtypes = [C.POINTER(C.c_int), C.c_int, C.POINTER(Rope)]
    ref.qw_rope_free.argtypes = [C.POINTER(Rope)]
    dims = (C.c_int * 3)(16, 56, 56)
    t = Rope()
    assert ref.qw_rope_build(dims, 3, C.byref(t))
    rows = 9216
    c, s = C.c_float(), C.c_float()
    off = 0
    for axis, d in enumerate([16, 56, 56]):
        pairs = d // 2
        for row in [0, 1, 5, 100, 4095, 8191, 8192, 9000, 9215]:
            for p in range(pairs):
                L.qo_rope_table_entry(d, row, p, C.byref(c), C.byref(s))
                assert c.value == t.cos[off + row * pairs + p]
                assert s.value == t.sin[off + row * pairs + p]
        off += rows * pairs
    ref.qw_rope_free(C.byref(t))

    ref.qw_euler_velocity_step.argtypes = [C.POINTER(C.c_float), C.POINTER(C.c_float),
                                           C.c_size_t, C.c_float, C.c_float]
    x = np.linspace(-3, 3, 101).astype(np.float32)
    v = np.cos(np.arange(101)).astype(np.float32)
    x2 = x.copy()
    ref.qw_euler_velocity_step(x.ctypes.data_as(C.POINTER(C.c_float)),
                               v.ctypes.data_as(C.POINTER(C.c_float)), 101, 0.7, 0.3)
    L.qo_euler_step(x2, v, 101, 0.7, 0.3)
    assert np.array_equal(x, x2)
