"""GPU parity of every hot-path kernel, through the C-ABI, against the
pinned CPU oracle on the same seeded inputs. Integer/byte work (generator,
int8 quantizer, dequantised weights, copies) is bit-exact; floating point
is held to bf16-ulp or relL2 bounds written next to each check."""
import math

import numpy as np
import pytest

from conftest import bf16_neighbours, cosine, read_bf16, rel_l2, ulp_diff

pytestmark = pytest.mark.gpu
SEED = 1234


def bf(o, x):
    return o.f32_to_bf16(np.asarray(x, np.float32))


def synth(o, n, stream, std=1.0):
    return o.fill_normal_bf16(n, SEED, stream, std)


def test_fill_normal_bit_exact(gpu, qd, oracle):
    n = 100003
    t = gpu.new(n + 16, qd.BF16)
    gpu.check(qd.lib().qw_gpu_fill_normal_bf16(gpu.h, t.h, 16, n, 77, 5, 0.02, 1.0), "fill")
    gpu.submit()
    got = t.read()[16:]
    ref = oracle.fill_normal_bf16(n, 77, 5, 0.02, 1.0)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("rows,cols", [(3, 64), (257, 3072), (64, 12288)])
def test_quantize_and_dequant_bit_exact(gpu, qd, oracle, rows, cols):
    w = synth(oracle, rows * cols, 11, 0.02)
    w[:cols] = 0  # an all-zero row -> scale 1/127
    q_ref, s_ref = oracle.quantize_int8_rows(w, rows, cols)
    wt = gpu.put(w)
    qt = gpu.new(rows * cols, qd.I8)
    st = gpu.new(rows, qd.F32)
    gpu.check(qd.lib().h3_gpu_quantize_weight_int8(gpu.h, qt.h, st.h, wt.h, rows, cols), "quant")
    dq = gpu.new(rows * cols, qd.F32)
    gpu.check(qd.lib().qw_gpu_dequant_int8_f32(gpu.h, dq.h, qt.h, st.h, rows, cols), "dequant")
    gpu.submit()
    assert np.array_equal(qt.read(), q_ref.ravel())
    assert np.array_equal(st.read(), s_ref)
    deq_ref = np.empty(rows * cols, np.float32)
    oracle.lib().qo_dequant_int8_rows(deq_ref, q_ref.ravel(), s_ref, rows, cols)
    assert np.array_equal(dq.read(), deq_ref)


def assert_linear_close(oracle, got, ref, mag):
    """Two fp32 sums of the same bf16 products in different orders round
    to bf16 at most one ulp apart, except where cancellation leaves a
    result small against sum |x w| (mag): there the fp32 accumulation
    error (worst case k * 2^-24 * mag, typically sqrt(k) * 2^-24 * mag)
    bounds the difference; 2^-14 * mag is a quarter of the worst case at
    k = 3072."""
    d = ulp_diff(got, ref)
    diff = np.abs(oracle.bf16_to_f32(got).astype(np.float64) - oracle.bf16_to_f32(ref))
    ok = (d <= 1) | (diff <= 2.0 ** -14 * mag)
    assert ok.all(), (d.max(), np.flatnonzero(~ok)[:5])
    assert np.mean(d == 0) > 0.98


def assert_gelu_close(oracle, got, lin, mag):
    """bf16(gelu(y)), y = bf16(sum): where the sum sits at a rounding
    boundary of y, another summation order rounds y the other way (one bf16
    ulp of y), and gelu moves by up to 1.13 ulp(y) -- 3 output ulps where
    gelu(y) falls into the binade below y (y = 2.016 / 2.031 -> 1.969 /
    1.992). Accept gelu of y or of either bf16 neighbour of y within 2
    output ulps, or the accumulation bound."""
    lin = np.ascontiguousarray(lin.ravel())
    best, plain = None, None
    for yv in (lin,) + bf16_neighbours(lin):
        want = np.empty_like(lin)
        oracle.lib().qo_gelu_tanh(want, np.ascontiguousarray(yv), lin.size)
        d = ulp_diff(got, want)
        if plain is None:
            plain = want
        best = d if best is None else np.minimum(best, d)
    diff = np.abs(oracle.bf16_to_f32(got).astype(np.float64) - oracle.bf16_to_f32(plain))
    ok = (best <= 2) | (diff <= 2.0 ** -13 * mag)
    assert ok.all() and np.mean(ulp_diff(got, plain) == 0) > 0.97, (best.max(), np.flatnonzero(~ok)[:5])


LINEAR_CASES = [
    # rows, k, n, bias, int8
    (1, 64, 64, False, False),
    (37, 256, 136, True, False),
    (300, 3072, 520, True, False),
    (256, 64, 3072, False, False),
    (513, 1024, 256, True, True),   # int8 widened to bf16 before the GEMM
    (37, 256, 136, True, True),     # int8 widened in LDS inside the GEMM
    (40, 64, 256, False, True),     # ... one K-slice: the prologue only
    (100, 128, 520, True, True),    # ... two K-slices, ragged N
    (700, 512, 264, False, True),
    (2, 3072, 12288, True, False),
    # at most 8 rows: the streaming GEMV kernels (bf16 and int8 weights)
    (3, 3072, 3072, True, False),
    (8, 512, 1032, True, True),
    (1, 3072, 18432, False, True),
]


@pytest.mark.parametrize("rows,k,n,bias,int8", LINEAR_CASES)
def test_linear_store(gpu, qd, oracle, rows, k, n, bias, int8):
    x = synth(oracle, rows * k, 1)
    w = synth(oracle, n * k, 2, 0.02)
    b = synth(oracle, n, 3, 0.02) if bias else None
    xt, bt = gpu.put(x), (gpu.put(b) if bias else None)
    out = gpu.new(rows * n, qd.BF16)
    if int8:
        q, s = oracle.quantize_int8_rows(w, n, k)
        wt, st = gpu.put(q), gpu.put(s)
        gpu.linear(out, xt, wt, rows, k, n, bias=bt, wscale=st)
        ref = oracle.linear_i8(x, q, s, b, rows, k, n)
    else:
        wt = gpu.put(w)
        gpu.linear(out, xt, wt, rows, k, n, bias=bt)
        ref = oracle.linear(x, w, b, rows, k, n)
    gpu.submit()
    got = out.read()
    absx, absw = x & np.uint16(0x7FFF), w & np.uint16(0x7FFF)
    # sum |x| |w| (|w| within half a quantisation step of |q s| for int8)
    mag = oracle.bf16_to_f32(oracle.linear(absx, absw, None, rows, k, n)).ravel()
    assert_linear_close(oracle, got, ref.ravel(), mag)


@pytest.mark.parametrize("rows,k,n,bias", [c[:4] for c in LINEAR_CASES if c[4] and c[0] > 8])
def test_linear_int8_in_lds_route(qd, oracle, monkeypatch, rows, k, n, bias):
    """The "_w8" kernels (int8 W widened in LDS inside the GEMM) on the int8
    cases, forced by QW_INT8_ROUTE=w8: by default these small launches widen
    by a pass and run the bf16 half tiles instead."""
    monkeypatch.setenv("QW_INT8_ROUTE", "w8")
    gpu = qd.Gpu()
    try:
        x = synth(oracle, rows * k, 1)
        w = synth(oracle, n * k, 2, 0.02)
        b = synth(oracle, n, 3, 0.02) if bias else None
        q, s = oracle.quantize_int8_rows(w, n, k)
        out = gpu.new(rows * n, qd.BF16)
        gpu.linear(out, gpu.put(x), gpu.put(q), rows, k, n, bias=gpu.put(b) if bias else None,
                   wscale=gpu.put(s))
        gpu.submit()
        ref = oracle.linear_i8(x, q, s, b, rows, k, n)
        absx, absw = x & np.uint16(0x7FFF), w & np.uint16(0x7FFF)
        mag = oracle.bf16_to_f32(oracle.linear(absx, absw, None, rows, k, n)).ravel()
        assert_linear_close(oracle, out.read(), ref.ravel(), mag)
    finally:
        gpu.close()


@pytest.mark.parametrize("int8,rows,rm_blocks", [(False, 300, 0), (True, 300, 0), (True, 600, 0),
                                                 (False, 4, 0), (True, 7, 0), (False, 300, 1),
                                                 (True, 600, 1)])
def test_linear_gelu_and_gate_epilogues(gpu, qd, oracle, int8, rows, rm_blocks):
    """rm_blocks: gate rows constant over whole 128-row blocks but one (the
    text/image boundary at row 200), as in the DiT's row map."""
    k, n = 512, 768
    x = synth(oracle, rows * k, 4)
    w = synth(oracle, n * k, 5, 0.02)
    b = synth(oracle, n, 6, 0.02)
    xt, bt = gpu.put(x), gpu.put(b)
    if int8:
        q, s = oracle.quantize_int8_rows(w, n, k)
        wt, st = gpu.put(q), gpu.put(s)
        lin = oracle.linear_i8(x, q, s, b, rows, k, n)
    else:
        wt, st = gpu.put(w), None
        lin = oracle.linear(x, w, b, rows, k, n)
    # GELU: bf16(gelu(bf16(y)))
    out = gpu.new(rows * n, qd.BF16)
    gpu.linear(out, xt, wt, rows, k, n, bias=bt, wscale=st, epilogue=qd.LINEAR_GELU)
    ref = np.empty_like(lin)
    oracle.lib().qo_gelu_tanh(ref.ravel(), lin.ravel(), lin.size)
    # GATE: h = bf16(h + bf16(y) * gate[row_map[r], slot 2])
    slots = 6
    mod = synth(oracle, 2 * slots * n, 7, 0.5)
    rm = ((np.arange(rows) >= 200) if rm_blocks else (np.arange(rows) % 3 == 0)).astype(np.uint32)
    h0 = synth(oracle, rows * n, 8)
    ht, mt, rmt = gpu.put(h0), gpu.put(mod), gpu.put(rm)
    gpu.linear(ht, xt, wt, rows, k, n, bias=bt, wscale=st, epilogue=qd.LINEAR_GATE,
               modulation=mt, row_map=rmt, slots=slots, gate_slot=2)
    gate_ref = np.empty(rows * n, np.uint16)
    oracle.lib().qo_gate(gate_ref, h0, lin.ravel(), mod, rm, rows, n, slots, 2)
    gpu.submit()
    absx, absw = x & np.uint16(0x7FFF), w & np.uint16(0x7FFF)
    mag = oracle.bf16_to_f32(oracle.linear(absx, absw, None, rows, k, n)).ravel()
    for got, want in ((out.read(), ref.ravel()), (ht.read(), gate_ref)):
        d = ulp_diff(got, want)
        diff = np.abs(oracle.bf16_to_f32(got).astype(np.float64) - oracle.bf16_to_f32(want))
        # one flip of the linear's rounding propagates through gelu (slope
        # <= 1.13) or the gate (|g| <= 1) plus one output rounding
        ok = (d <= 2) | (diff <= 2.0 ** -13 * mag)
        assert ok.all() and np.mean(d == 0) > 0.97, (d.max(), np.mean(d == 0))


# (rows, k, n, int8, epilogue). On the 256-CU part a grid of 256 x 256
# tiles that leaves the last wave of workgroups partly filled has those tiles
# cut into k-ranges of at least 2048, one workgroup each; the last piece of a
# tile to finish adds the fp32 partials in piece order. 16 tiles with
# k = 4096 are cut in 2; 10 ragged tiles (300 rows, 1032 columns) with
# k = 8192 in 4; 12 tiles with k = 12288 (the MLP down projection's depth)
# in 6; 64 tiles with k = 8192 in 4 (256 pieces, one per CU).
SPLIT_CASES = [
    (512, 4096, 2048, False, "store"),
    (300, 8192, 1032, True, "gelu"),
    (512, 4096, 2048, False, "gate"),
    (256, 12288, 3072, False, "store"),
    # bf16 GELU and K >= 4096 stores run the 4-wave (one wave per SIMD)
    # kernels: their split-tile path
    (512, 8192, 2048, False, "gelu"),
    # int8 weights with K >= 8192: widened in LDS inside the GEMM, split
    (512, 8192, 2048, True, "gate"),
    # 64 tiles, 4 pieces each: every CU runs one piece; ragged, int8 in LDS
    (2048, 8192, 2048, False, "gate"),
    (2000, 8192, 2000, True, "gelu"),
    # gate rows constant over whole 128-row blocks but one (the text/image
    # boundary at row 200), as in the DiT's row map
    (512, 8192, 2048, True, "gate_blocks"),
    (300, 4096, 1024, False, "gate_blocks"),
]


@pytest.mark.parametrize("rows,k,n,int8,epi", SPLIT_CASES)
def test_linear_split_tiles(gpu, qd, oracle, rows, k, n, int8, epi):
    x = synth(oracle, rows * k, 11)
    w = synth(oracle, n * k, 12, 0.02)
    b = synth(oracle, n, 13, 0.02)
    xt, bt = gpu.put(x), gpu.put(b)
    if int8:
        q, s = oracle.quantize_int8_rows(w, n, k)
        wt, st = gpu.put(q), gpu.put(s)
        lin = oracle.linear_i8(x, q, s, b, rows, k, n)
    else:
        wt, st = gpu.put(w), None
        lin = oracle.linear(x, w, b, rows, k, n)
    absx, absw = x & np.uint16(0x7FFF), w & np.uint16(0x7FFF)
    mag = oracle.bf16_to_f32(oracle.linear(absx, absw, None, rows, k, n)).ravel()
    outs = []
    for rep in range(2):  # piece counters must be back at 0 for the second call
        if epi in ("gate", "gate_blocks"):
            slots = 6
            mod = synth(oracle, 2 * slots * n, 14, 0.5)
            rm = ((np.arange(rows) % 3 == 1) if epi == "gate" else
                  (np.arange(rows) >= 200)).astype(np.uint32)
            h0 = synth(oracle, rows * n, 15)
            out = gpu.put(h0)
            gpu.linear(out, xt, wt, rows, k, n, bias=bt, wscale=st, epilogue=qd.LINEAR_GATE,
                       modulation=gpu.put(mod), row_map=gpu.put(rm), slots=slots, gate_slot=2)
        else:
            out = gpu.new(rows * n, qd.BF16)
            gpu.linear(out, xt, wt, rows, k, n, bias=bt, wscale=st,
                       epilogue=qd.LINEAR_GELU if epi == "gelu" else qd.LINEAR_STORE)
        gpu.submit()
        outs.append(out.read())
    assert np.array_equal(outs[0], outs[1]), "split-tile result differs between two calls"
    got = outs[0]
    if epi == "store":
        assert_linear_close(oracle, got, lin.ravel(), mag)
        return
    if epi in ("gate", "gate_blocks"):
        # out = bf16(h + bf16(y) g): where h and y g nearly cancel, the one
        # flip of bf16(y) that a different summation order may cause moves
        # the output by many of its ulps, so accept the gate of y or of
        # either bf16 neighbour of y (each within one output ulp)
        best = None
        for yv in (lin.ravel(),) + bf16_neighbours(lin.ravel()):
            want = np.empty(rows * n, np.uint16)
            oracle.lib().qo_gate(want, h0, np.ascontiguousarray(yv), mod, rm, rows, n, slots, 2)
            d = ulp_diff(got, want)
            best = d if best is None else np.minimum(best, d)
        assert best.max() <= 1, best.max()
        return
    assert_gelu_close(oracle, got, lin, mag)


@pytest.mark.parametrize("rows,k,n,epi", [(300, 3072, 1024, "gelu"), (1100, 12288, 768, "gate"),
                                          (2000, 8192, 2000, "store")])
def test_int8_in_gemm_widening_bit_identical(qd, oracle, monkeypatch, rows, k, n, epi):
    """The int8 kernels that widen each W tile once per workgroup in LDS
    (taken below 512 rows and for K >= 8192) give the same bits as widening
    the weight to a bf16 copy (qw_gpu_widen_int8_bf16) and running the bf16
    kernel with the same row scales: the widening is exact and the scale
    multiplies the finished fp32 sums in both. Split tiles included
    (K = 8192 and 12288). Same k-ranges on both sides: the bf16 kernels'
    half tiles for small launches (which may split K differently) are
    turned off for this context."""
    monkeypatch.setenv("QW_GEMM_HALF_SMALL", "0")
    gpu = qd.Gpu()
    try:
        _widening_bit_identical(gpu, qd, oracle, rows, k, n, epi)
    finally:
        gpu.close()


def _widening_bit_identical(gpu, qd, oracle, rows, k, n, epi):
    L = qd.lib()
    x = synth(oracle, rows * k, 61)
    w = synth(oracle, n * k, 62, 0.02)
    b = synth(oracle, n, 63, 0.02)
    q, sc = oracle.quantize_int8_rows(w, n, k)
    xt, bt, qt, st = gpu.put(x), gpu.put(b), gpu.put(q), gpu.put(sc)
    wide = gpu.new(n * k, qd.BF16)
    gpu.check(L.qw_gpu_widen_int8_bf16(gpu.h, wide.h, qt.h, n * k), "widen")
    E = {"store": qd.LINEAR_STORE, "gelu": qd.LINEAR_GELU, "gate": qd.LINEAR_GATE}[epi]
    kw = {}
    if epi == "gate":
        mod = synth(oracle, 2 * 4 * n, 64, 0.3)
        rm = (np.arange(rows) % 5 == 0).astype(np.uint32)
        kw = dict(modulation=gpu.put(mod), row_map=gpu.put(rm), slots=4, gate_slot=3)
    h0 = synth(oracle, rows * n, 65)
    outs = []
    for weight in (qt, wide):
        out = gpu.put(h0)
        gpu.linear(out, xt, weight, rows, k, n, bias=bt, wscale=st, epilogue=E, **kw)
        gpu.submit()
        outs.append(out.read())
    assert np.array_equal(outs[0], outs[1])


def test_linear_full_waves_never_split(qd, oracle):
    """Every wave of tiles full (1024 tiles of 256 x 256: a whole number of
    waves on any CU count dividing 1024, 256 on MI355X) with a long K
    (4096): no tile is left for a split, so the runtime allocates no
    split-tile workspace (a fresh context's allocated bytes do not move) and
    the tile walk computes every tile whole; sampled rows against the
    oracle to the linear bar."""
    rows, k, n = 32768, 4096, 2048
    gpu = qd.Gpu()
    try:
        x = synth(oracle, rows * k, 51)
        w = synth(oracle, n * k, 52, 0.02)
        xt, wt = gpu.put(x), gpu.put(w)
        out = gpu.new(rows * n, qd.BF16)
        gpu.submit()
        before = gpu.stats().allocated_bytes
        gpu.linear(out, xt, wt, rows, k, n)
        gpu.submit()
        assert gpu.stats().allocated_bytes == before
        got = out.read().reshape(rows, n)
    finally:
        gpu.close()
    pick = np.unique(np.linspace(0, rows - 1, 96).round().astype(np.int64))
    xs = x.reshape(rows, k)[pick].copy()
    ref = oracle.linear(xs, w, None, len(pick), k, n).ravel()
    mag = oracle.bf16_to_f32(oracle.linear(xs & np.uint16(0x7FFF), w & np.uint16(0x7FFF), None,
                                           len(pick), k, n)).ravel()
    assert_linear_close(oracle, got[pick].ravel(), ref, mag)


@pytest.mark.parametrize("rows,k,epi", [(4315, 512, "store"), (4315, 512, "gelu"),
                                        (8604, 256, "gate"), (4315, 512, "qkn")])
def test_linear_224_row_tiles(gpu, qd, oracle, rows, k, epi):
    """Shapes whose 256 x 256 tiling leaves a partly filled last wave that
    224 x 256 tiles avoid (on 256 CUs: 204 tiles of 256 rows, 1 wave, become
    240 of 224 rows; 408 tiles, 2 waves, become 468 in 2 waves of 0.875 the
    work): ragged rows through all four epilogues, against the oracle, and
    the fused q/k norm + RoPE bit for bit against the plain linear followed
    by the standalone kernel."""
    n = 3072
    x = synth(oracle, rows * k, 71)
    w = synth(oracle, n * k, 72, 0.02)
    b = synth(oracle, n, 73, 0.02)
    xt, wt, bt = gpu.put(x), gpu.put(w), gpu.put(b)
    lin = oracle.linear(x, w, b, rows, k, n)
    absx, absw = x & np.uint16(0x7FFF), w & np.uint16(0x7FFF)
    mag = oracle.bf16_to_f32(oracle.linear(absx, absw, None, rows, k, n)).ravel()
    if epi == "qkn":
        heads = n // 384
        nq, nk = synth(oracle, 128, 74, 0.1), synth(oracle, 128, 75, 0.1)
        ang = np.random.default_rng(76).uniform(-3, 3, (rows, 64)).astype(np.float32)
        cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
        nqt, nkt, ct, st_ = (gpu.put(v) for v in (nq, nk, cos, sin))
        fused, ref = gpu.new(rows * n, qd.BF16), gpu.new(rows * n, qd.BF16)
        gpu.linear(fused, xt, wt, rows, k, n, bias=bt, epilogue=qd.LINEAR_QKNORM,
                   qknorm=(nqt, nkt, ct, st_, rows, 1e-6))
        gpu.linear(ref, xt, wt, rows, k, n, bias=bt)
        gpu.check(qd.lib().qw_gpu_qk_norm_rope_bf16(gpu.h, ref.h, rows, heads, n, n // 3, nqt.h,
                                                     nkt.h, ct.h, st_.h, rows, 1e-6), "qk")
        gpu.submit()
        plain = gpu.new(rows * n, qd.BF16)
        gpu.linear(plain, xt, wt, rows, k, n, bias=bt)
        gpu.submit()
        assert_linear_close(oracle, plain.read(), lin.ravel(), mag)
        assert np.array_equal(fused.read(), ref.read())
        return
    if epi == "gate":
        slots = 6
        mod = synth(oracle, 2 * slots * n, 77, 0.5)
        rm = (np.arange(rows) >= 200).astype(np.uint32)
        h0 = synth(oracle, rows * n, 78)
        out = gpu.put(h0)
        gpu.linear(out, xt, wt, rows, k, n, bias=bt, epilogue=qd.LINEAR_GATE,
                   modulation=gpu.put(mod), row_map=gpu.put(rm), slots=slots, gate_slot=2)
    else:
        out = gpu.new(rows * n, qd.BF16)
        gpu.linear(out, xt, wt, rows, k, n, bias=bt,
                   epilogue=qd.LINEAR_GELU if epi == "gelu" else qd.LINEAR_STORE)
    gpu.submit()
    got = out.read()
    if epi == "store":
        assert_linear_close(oracle, got, lin.ravel(), mag)
        return
    if epi == "gelu":
        assert_gelu_close(oracle, got, lin, mag)
        return
    if epi == "gate":
        # where h and y g nearly cancel, one flip of bf16(y) moves the output
        # by many of its ulps: accept the gate of y or of either bf16
        # neighbour of y, each within one output ulp (as the split tiles)
        best = None
        for yv in (lin.ravel(),) + bf16_neighbours(lin.ravel()):
            want = np.empty(rows * n, np.uint16)
            oracle.lib().qo_gate(want, h0, np.ascontiguousarray(yv), mod, rm, rows, n, slots, 2)
            d = ulp_diff(got, want)
            best = d if best is None else np.minimum(best, d)
        assert best.max() <= 1, best.max()


@pytest.mark.parametrize("n,int8", [(1800, False), (1784, True)])
def test_linear_224_row_tiles_ragged_cols(gpu, qd, oracle, n, int8):
    """224-row tiles with a partial last tile column (N not a multiple of
    256): 17 x 8 = 136 tiles of 256 rows (one wave, more than half full)
    become 20 x 8 = 160 of 224 rows; int8 weights take the widening pass
    (K < 8192, 512+ rows) into the same kernel."""
    rows, k = 4315, 512
    x = synth(oracle, rows * k, 81)
    w = synth(oracle, n * k, 82, 0.02)
    b = synth(oracle, n, 83, 0.02)
    xt, bt = gpu.put(x), gpu.put(b)
    out = gpu.new(rows * n, qd.BF16)
    if int8:
        q, s = oracle.quantize_int8_rows(w, n, k)
        gpu.linear(out, xt, gpu.put(q), rows, k, n, bias=bt, wscale=gpu.put(s))
        ref = oracle.linear_i8(x, q, s, b, rows, k, n)
    else:
        gpu.linear(out, xt, gpu.put(w), rows, k, n, bias=bt)
        ref = oracle.linear(x, w, b, rows, k, n)
    gpu.submit()
    absx, absw = x & np.uint16(0x7FFF), w & np.uint16(0x7FFF)
    mag = oracle.bf16_to_f32(oracle.linear(absx, absw, None, rows, k, n)).ravel()
    assert_linear_close(oracle, out.read(), ref.ravel(), mag)


@pytest.mark.parametrize("epi", ["store", "gelu", "gate"])
def test_linear_tile_walk(gpu, qd, oracle, epi):
    """More tiles than compute units: the 16x16x32 GEMM launches one
    workgroup per CU and each walks its tiles in strides of the grid. 17 x
    17 tiles of 256 x 256 (289 > 256), ragged in both the last tile row
    (4100 rows) and the last tile column (4104 columns), called twice in a
    row (the workgroups keep no state between tiles or calls). The 33 tiles
    of the last, partly filled wave run as 66 half tiles of 128 x 256; the
    last tile row's second halves hold no rows at all."""
    rows, k, n = 4100, 256, 4104
    x = synth(oracle, rows * k, 41)
    w = synth(oracle, n * k, 42, 0.02)
    b = synth(oracle, n, 43, 0.02)
    xt, wt, bt = gpu.put(x), gpu.put(w), gpu.put(b)
    slots = 6
    mod = synth(oracle, 2 * slots * n, 44, 0.5)
    rm = (np.arange(rows) % 3 == 0).astype(np.uint32)
    h0 = synth(oracle, rows * n, 45)
    mt, rmt = gpu.put(mod), gpu.put(rm)
    outs = []
    for _ in range(2):
        if epi == "gate":
            out = gpu.put(h0)
            gpu.linear(out, xt, wt, rows, k, n, bias=bt, epilogue=qd.LINEAR_GATE,
                       modulation=mt, row_map=rmt, slots=slots, gate_slot=2)
        else:
            out = gpu.new(rows * n, qd.BF16)
            gpu.linear(out, xt, wt, rows, k, n, bias=bt,
                       epilogue=qd.LINEAR_GELU if epi == "gelu" else qd.LINEAR_STORE)
        gpu.submit()
        outs.append(out.read())
    assert np.array_equal(outs[0], outs[1])
    lin = oracle.linear(x, w, b, rows, k, n).ravel()
    absx, absw = x & np.uint16(0x7FFF), w & np.uint16(0x7FFF)
    mag = oracle.bf16_to_f32(oracle.linear(absx, absw, None, rows, k, n)).ravel()
    if epi == "store":
        assert_linear_close(oracle, outs[0], lin, mag)
        return
    want = np.empty_like(lin)
    f = oracle.bf16_to_f32
    if epi == "gate":
        want = np.empty(rows * n, np.uint16)
        oracle.lib().qo_gate(want, h0, lin, mod, rm, rows, n, slots, 2)
    else:
        oracle.lib().qo_gelu_tanh(want, lin, lin.size)
    d = ulp_diff(outs[0], want)
    diff = np.abs(f(outs[0]).astype(np.float64) - f(want))
    ok = (d <= 2) | (diff <= 2.0 ** -13 * mag)
    if epi == "gate":
        # where the sum sits at a rounding boundary of y = bf16(sum), y can
        # round the other way (one bf16 ulp of y); the output then moves by
        # |g| ulp(y) plus its own rounding, many output ulps where h + y g
        # cancels
        g = f(mod).reshape(2, slots, n)[rm, 2, :].ravel().astype(np.float64)
        down, up = bf16_neighbours(lin)
        ulp_y = np.maximum(np.abs(f(up) - f(lin)), np.abs(f(lin) - f(down)))
        wd, wu = bf16_neighbours(want)
        ulp_o = np.maximum(np.abs(f(wu) - f(want)), np.abs(f(want) - f(wd)))
        ok |= diff <= np.abs(g) * ulp_y + ulp_o
    assert ok.all() and np.mean(d == 0) > 0.97, (d.max(), np.mean(d == 0))


@pytest.mark.parametrize("rows,int8,rope_rows,k", [(300, False, 300, 512), (300, True, 150, 512),
                                                   (1000, True, 500, 512),
                                                   (4357, False, 4357, 512),
                                                   # tables under 128 rows: the plain
                                                   # linear, then the standalone kernel
                                                   (300, False, 100, 512), (300, True, 64, 512),
                                                   # 270 tiles: a tile walk whose last 14
                                                   # tiles run as half tiles
                                                   (11400, False, 11400, 512),
                                                   # a small launch's half tiles in 3
                                                   # k-range pieces
                                                   (300, False, 300, 3072),
                                                   (600, True, 600, 3072)])
def test_linear_qknorm_epilogue_bit_identical(gpu, qd, oracle, rows, int8, rope_rows, k):
    """The fused q|k|v linear with the per-head RMS norm and RoPE of q and k
    in its epilogue equals the linear followed by qw_gpu_qk_norm_rope_bf16,
    bit for bit (same sums, same reduction order, same roundings): fused
    int8 kernel, widen route, ragged rows, a RoPE table shorter than the
    rows (batched sequences), tables shorter than a wave's 128 rows."""
    heads = 4
    n = 3 * heads * 128
    x = synth(oracle, rows * k, 31)
    w = synth(oracle, n * k, 32, 0.02)
    b = synth(oracle, n, 33, 0.02)
    nq, nk = synth(oracle, 128, 34, 0.1), synth(oracle, 128, 35, 0.1)
    rng = np.random.default_rng(9)
    ang = rng.uniform(-3, 3, (rope_rows, 64)).astype(np.float32)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    xt, bt, nqt, nkt, ct, st_ = (gpu.put(v) for v in (x, b, nq, nk, cos, sin))
    if int8:
        q, s = oracle.quantize_int8_rows(w, n, k)
        wt, sc = gpu.put(q), gpu.put(s)
    else:
        wt, sc = gpu.put(w), None
    fused, ref = gpu.new(rows * n, qd.BF16), gpu.new(rows * n, qd.BF16)
    gpu.linear(fused, xt, wt, rows, k, n, bias=bt, wscale=sc, epilogue=qd.LINEAR_QKNORM,
               qknorm=(nqt, nkt, ct, st_, rope_rows, 1e-6))
    gpu.linear(ref, xt, wt, rows, k, n, bias=bt, wscale=sc)
    gpu.check(qd.lib().qw_gpu_qk_norm_rope_bf16(gpu.h, ref.h, rows, heads, n, n // 3, nqt.h,
                                                 nkt.h, ct.h, st_.h, rope_rows, 1e-6), "qk")
    gpu.submit()
    assert np.array_equal(fused.read(), ref.read())
    bad = gpu.new(rows * 1024, qd.BF16)
    with pytest.raises(RuntimeError, match="heads of 128"):
        gpu.linear(bad, xt, gpu.new(1024 * k, qd.BF16), rows, k, 1024,
                   epilogue=qd.LINEAR_QKNORM, qknorm=(nqt, nkt, ct, st_, rope_rows, 1e-6))


def test_linear_strided_views(gpu, qd, oracle):
    """Offsets/strides as the DiT uses them (rows written into a joint
    buffer at a row offset, input read from a wider buffer)."""
    rows, k, n, ld_in, ld_out = 70, 128, 256, 384, 512
    x_full = synth(oracle, rows * ld_in, 9)
    w = synth(oracle, n * k, 10, 0.02)
    x = x_full.reshape(rows, ld_in)[:, 128:256].copy()
    out = gpu.new(rows * ld_out + 4096, qd.BF16)
    gpu.linear(out, gpu.put(x_full), gpu.put(w), rows, k, n, lda=ld_in, in_offset=128,
               ldc=ld_out, out_offset=4096 + 64)
    gpu.submit()
    got = out.read()
    ref = oracle.linear(x, w, None, rows, k, n)
    region = got[4096 + 64:].reshape(-1)[: (rows - 1) * ld_out + n]
    tiles = np.stack([region[r * ld_out: r * ld_out + n] for r in range(rows)])
    assert ulp_diff(tiles, ref).max() <= 1
    # untouched elements stay zero (no stray writes)
    assert np.all(got[:4096 + 64] == 0)


def test_linear_rejects_bad_shapes(gpu, qd):
    x = gpu.new(64 * 100, qd.BF16)
    w = gpu.new(64 * 100, qd.BF16)
    out = gpu.new(64 * 64, qd.BF16)
    with pytest.raises(RuntimeError, match="multiple of 64"):
        gpu.linear(out, x, w, 64, 100, 64)
    with pytest.raises(RuntimeError, match="too small"):
        gpu.linear(out, x, w, 64, 64, 128)


@pytest.mark.parametrize("width,shift", [(3072, True), (4096, False), (256, True), (6144, True)])
def test_layer_norm_mod(gpu, qd, oracle, width, shift):
    rows, slots = 129, 6 if shift else 4
    x = synth(oracle, rows * width, 12, 2.0)
    mod = synth(oracle, 2 * slots * width, 13, 0.3)
    rm = (np.arange(rows) < 17).astype(np.uint32)
    out = gpu.new(rows * width, qd.BF16)
    gpu.check(qd.lib().qw_gpu_layer_norm_mod_shift_bf16(
        gpu.h, out.h, gpu.put(x).h, gpu.put(mod).h, gpu.put(rm).h, rows, width, slots, 1,
        5 if shift else -1, 1e-6), "ln")
    gpu.submit()
    ref = np.empty(rows * width, np.uint16)
    oracle.lib().qo_layer_norm_mod(ref, x, mod, rm, rows, width, slots, 1, 5 if shift else -1, 1e-6)
    got = out.read()
    d = ulp_diff(got, ref)
    # outputs are O(1); with a shift, x_hat (1 + s) + shift can cancel to
    # near zero, where one fp32 ulp of the O(1) terms is many bf16 ulps of
    # the result: bound those by an absolute 2^-9 instead
    diff = np.abs(oracle.bf16_to_f32(got) - oracle.bf16_to_f32(ref))
    assert np.all((d <= 1) | (diff <= 2.0 ** -9)) and np.mean(d == 0) > 0.99


@pytest.mark.parametrize("case,text,rows", [("a", 0, 16), ("b", 8, 20)])
def test_layer_norm_mod_dit_fixture(gpu, qd, oracle, case, text, rows):
    """Reference stage pair joint_in -> attn_in (tests/test_dit_block.c:204-214)."""
    H = 4096
    j, mod = read_bf16(f"{case}_joint_in.bin"), read_bf16(f"{case}_modulation.bin")
    rm = (np.arange(rows) < text).astype(np.uint32)
    out = gpu.new(rows * H, qd.BF16)
    gpu.check(qd.lib().qw_gpu_layer_norm_mod_bf16(gpu.h, out.h, gpu.put(j).h, gpu.put(mod).h,
                                                  gpu.put(rm).h, rows, H, 4, 0, 1e-6), "ln")
    gpu.submit()
    got = out.read()
    ref = read_bf16(f"{case}_attn_in.bin")
    assert rel_l2(oracle.bf16_to_f32(got), oracle.bf16_to_f32(ref)) < 2e-2
    o = np.empty_like(got)
    oracle.lib().qo_layer_norm_mod(o, j, mod, rm, rows, H, 4, 0, -1, 1e-6)
    assert ulp_diff(got, o).max() <= 1


def test_qk_norm_rope(gpu, qd, oracle):
    rows, heads, H = 75, 4, 512
    ld = 3 * H
    qkv = synth(oracle, rows * ld, 14, 3.0)
    nq = oracle.fill_normal_bf16(128, SEED, 15, 0.02, 1.0)
    nk = oracle.fill_normal_bf16(128, SEED, 16, 0.02, 1.0)
    cos, sin = oracle.rope_tables(11, 8, 8)
    t = gpu.put(qkv)
    gpu.check(qd.lib().qw_gpu_qk_norm_rope_bf16(gpu.h, t.h, rows, heads, ld, H, gpu.put(nq).h,
                                                gpu.put(nk).h, gpu.put(cos).h, gpu.put(sin).h,
                                                rows, 1e-6), "qk")
    gpu.submit()
    ref = qkv.copy()
    L = oracle.lib()
    L.qo_head_rms_norm(ref, ld, nq, rows, heads, 128, 1e-6)
    L.qo_head_rms_norm(ref[H:], ld, nk, rows, heads, 128, 1e-6)
    L.qo_qk_rope(ref, ld, cos, sin, rows, heads, 128)
    L.qo_qk_rope(ref[H:], ld, cos, sin, rows, heads, 128)
    got = t.read()
    d = ulp_diff(got, ref)
    assert d.max() <= 2 and np.mean(d == 0) > 0.99
    assert np.array_equal(got.reshape(rows, ld)[:, 2 * H:], qkv.reshape(rows, ld)[:, 2 * H:])


def _attn_case(gpu, qd, oracle, rows, heads, limits_mode, batch=1, text=0, causal=1):
    hd = heads * 128
    rng = np.random.default_rng(rows + heads)
    q = bf(oracle, rng.uniform(-1, 1, (batch * rows, hd)))
    k = bf(oracle, rng.uniform(-1, 1, (batch * rows, hd)))
    v = bf(oracle, rng.uniform(-1, 1, (batch * rows, hd)))
    if limits_mode == "prefix":
        # tests/test_prefix_kernel.c:65-70: text causal / image block end
        lim = np.empty(rows, np.uint32)
        lim[:20] = np.arange(1, 21)
        lim[20:68] = 68
        lim[68:85] = 68 + np.arange(1, 18)
        lim[85:] = rows
    else:
        lim = oracle.t2i_limits(rows, text, causal)
    out = gpu.new(batch * rows * hd, qd.BF16)
    gpu.attention(out, gpu.put(q), gpu.put(k), gpu.put(v), batch, rows, rows, heads, hd, hd, hd,
                  hd, kv_limit=gpu.put(lim) if limits_mode == "prefix" else None,
                  text_rows=text, text_causal=causal)
    gpu.submit()
    got = out.read().reshape(batch * rows, hd)
    ref = np.concatenate([oracle.attention(q[b * rows:(b + 1) * rows].copy(),
                                           k[b * rows:(b + 1) * rows].copy(),
                                           v[b * rows:(b + 1) * rows].copy(), lim, rows, rows,
                                           heads, prescale_rows=text if limits_mode == "t2i"
                                           else 0) for b in range(batch)])
    f = oracle.bf16_to_f32
    return rel_l2(f(got), f(ref)), cosine(f(got), f(ref))


def test_attention_prefix_table(gpu, qd, oracle):
    """tests/test_prefix_kernel.c: 149 rows, 32 heads, ti2i-like limits,
    relL2 < 5e-3 against the O(n^2) CPU softmax."""
    rel, cos = _attn_case(gpu, qd, oracle, 149, 32, "prefix")
    assert rel < 5e-3 and cos > 0.9999


@pytest.mark.parametrize("rows,heads,text,causal,batch", [
    (20, 2, 8, 1, 1), (320, 4, 64, 0, 1), (300, 2, 44, 1, 2), (4352 // 8, 2, 32, 0, 2),
    (64, 1, 0, 1, 1), (1, 1, 0, 0, 1)])
def test_attention_t2i(gpu, qd, oracle, rows, heads, text, causal, batch):
    rel, cos = _attn_case(gpu, qd, oracle, rows, heads, "t2i", batch, text, causal)
    assert rel < 5e-3 and cos > 0.9999


@pytest.mark.parametrize("causal", [1, 0])
def test_attention_text_rows_prescale_q(gpu, qd, oracle, causal):
    """t2i text rows contract bf16(q * scale) with K (h3_shaders.metal:
    4397-4401). Sharp scores (|q|, |k| up to 8) make the re-rounding visible:
    the kernel must sit much closer to the oracle with the rule than to the
    oracle without it. The oracle rounds P to bf16 here, as the kernel's P
    operand is, so the comparison isolates the q rule."""
    rows, heads, text = 160, 2, 96
    hd = heads * 128
    rng = np.random.default_rng(41)
    q, k, v = (bf(oracle, a * rng.uniform(-1, 1, (rows, hd))) for a in (8.0, 8.0, 1.0))
    out = gpu.new(rows * hd, qd.BF16)
    gpu.attention(out, gpu.put(q), gpu.put(k), gpu.put(v), 1, rows, rows, heads, hd, hd, hd, hd,
                  text_rows=text, text_causal=causal)
    gpu.submit()
    f = oracle.bf16_to_f32
    got = f(out.read().reshape(rows, hd))
    lim = oracle.t2i_limits(rows, text, causal)
    oracle.set_attention_p_mode(1)
    try:
        with_rule = f(oracle.attention(q, k, v, lim, rows, rows, heads, prescale_rows=text))
        without = f(oracle.attention(q, k, v, lim, rows, rows, heads))
    finally:
        oracle.set_attention_p_mode(0)
    e_rule = rel_l2(got[:text], with_rule[:text])
    e_plain = rel_l2(got[:text], without[:text])
    assert e_rule < 2.5e-3 and e_plain > 2 * e_rule, (e_rule, e_plain)
    # image rows keep the scale in the softmax: identical in both oracles
    assert rel_l2(got[text:], with_rule[text:]) < 5e-3
    assert np.array_equal(with_rule[text:], without[text:])


def test_attention_strided_qkv(gpu, qd, oracle):
    """q|k|v read from one fused [rows, 3H] buffer, as the block does."""
    rows, heads = 130, 2
    H = heads * 128
    qkv = synth(oracle, 2 * rows * 3 * H, 17)
    out = gpu.new(2 * rows * H, qd.BF16)
    t = gpu.put(qkv)
    gpu.attention(out, t, t, t, 2, rows, rows, heads, 3 * H, 3 * H, 3 * H, H, q_offset=0,
                  k_offset=H, v_offset=2 * H, text_rows=10, text_causal=1)
    gpu.submit()
    got = out.read().reshape(2 * rows, H)
    m = qkv.reshape(2 * rows, 3 * H)
    lim = oracle.t2i_limits(rows, 10, 1)
    for b in range(2):
        blk = m[b * rows:(b + 1) * rows]
        ref = oracle.attention(blk[:, :H].copy(), blk[:, H:2 * H].copy(),
                               blk[:, 2 * H:].copy(), lim, rows, rows, heads, prescale_rows=10)
        assert rel_l2(oracle.bf16_to_f32(got[b * rows:(b + 1) * rows]),
                      oracle.bf16_to_f32(ref)) < 5e-3


@pytest.mark.parametrize("rows,heads,text,causal,batch,limits", [
    (1152, 3, 128, 0, 1, False), (320, 4, 64, 1, 1, False), (300, 2, 44, 1, 2, False),
    (200, 2, 0, 0, 1, True), (1, 1, 0, 0, 1, False)])
def test_attention_small_launch_kernel_bit_identical(qd, oracle, monkeypatch, rows, heads, text,
                                                     causal, batch, limits):
    """Launches of fewer 256-query blocks than CUs run the 128-query (4-wave)
    kernel; every query row's arithmetic is the 256-query kernel's, so both
    give the same bits (t2i masks, ragged rows, batch 2, a per-row limit
    table)."""
    H = heads * 128
    qkv = synth(oracle, batch * rows * 3 * H, 91)
    lim = None
    if limits:
        lim = np.random.default_rng(92).integers(1, rows + 1, rows).astype(np.uint32)
    outs = []
    for w4 in ("1", "0"):
        monkeypatch.setenv("QW_ATTN_W4", w4)
        g = qd.Gpu()
        try:
            t = g.put(qkv)
            out = g.new(batch * rows * H, qd.BF16)
            g.attention(out, t, t, t, batch, rows, rows, heads, 3 * H, 3 * H, 3 * H, H,
                        q_offset=0, k_offset=H, v_offset=2 * H,
                        kv_limit=g.put(lim) if limits else None, text_rows=text,
                        text_causal=causal)
            g.submit()
            outs.append(out.read())
        finally:
            g.close()
    assert np.array_equal(outs[0], outs[1])


def test_elementwise_family(gpu, qd, oracle):
    L, OL = qd.lib(), oracle.lib()
    n = 70001
    x = synth(oracle, n, 18, 3.0)
    xt = gpu.put(x)
    outs = {k: gpu.new(n, qd.BF16) for k in ("gelu", "silu", "tanh")}
    gpu.check(L.h3_gpu_gelu_bf16(gpu.h, outs["gelu"].h, xt.h, n, 1), "gelu")
    gpu.check(L.h3_gpu_silu_bf16(gpu.h, outs["silu"].h, xt.h, n), "silu")
    gpu.check(L.qw_gpu_tanh_bf16(gpu.h, outs["tanh"].h, xt.h, n), "tanh")
    rows, width = 37, 96
    fc1 = synth(oracle, rows * 2 * width, 19, 2.0)
    sw = gpu.new(rows * width, qd.BF16)
    gpu.check(L.qw_gpu_swiglu_bf16(gpu.h, sw.h, gpu.put(fc1).h, rows, width), "swiglu")
    # rounding cases: normals, random finite bit patterns, subnormals and
    # exact ties (low 16 bits 0x8000, both parities)
    rg = np.random.default_rng(0)
    bits = rg.integers(0, 2**32, 4000, dtype=np.uint64).astype(np.uint32)
    bits = bits[(bits & 0x7F800000) != 0x7F800000][:1500]
    sub = (rg.integers(0, 2**23, 500, dtype=np.uint64) | (rg.integers(0, 2, 500, dtype=np.uint64) << 31)).astype(np.uint32)
    ties = ((rg.integers(0x00800000, 0x7F000000, 500, dtype=np.uint64) & ~np.uint64(0xFFFF)) | 0x8000).astype(np.uint32)
    f = np.concatenate([rg.standard_normal(999).astype(np.float32), bits.view(np.float32),
                        sub.view(np.float32), ties.view(np.float32)])
    ct = gpu.new(f.size, qd.BF16)
    gpu.check(L.h3_gpu_cast_f32_to_bf16(gpu.h, ct.h, gpu.put(f).h, f.size), "cast")
    gpu.submit()
    ref = np.empty(n, np.uint16)
    OL.qo_gelu_tanh(ref, x, n)
    g = outs["gelu"].read()
    # the device evaluates 0.5 v (1 + tanh u) as v / (1 + e^-2u); for
    # u < -8.7 the fp32 tanh form rounds 1 + tanh u to exactly 0 while the
    # device keeps the true |gelu| < 1e-7: equal within 1e-6 absolute
    absdiff = np.abs(oracle.bf16_to_f32(g) - oracle.bf16_to_f32(ref))
    assert np.all((ulp_diff(g, ref) <= 1) | (absdiff < 1e-6))
    OL.qo_silu(ref, x, n)
    assert ulp_diff(outs["silu"].read(), ref).max() <= 1
    tanh_ref = oracle.f32_to_bf16(np.tanh(oracle.bf16_to_f32(x).astype(np.float64)).astype(np.float32))
    assert ulp_diff(outs["tanh"].read(), tanh_ref).max() <= 1
    swr = np.empty(rows * width, np.uint16)
    OL.qo_swiglu(swr, fc1, rows, width)
    assert ulp_diff(sw.read(), swr).max() <= 1
    assert np.array_equal(ct.read(), oracle.f32_to_bf16(f))


def test_gate_kernel(gpu, qd, oracle):
    rows, width, slots = 33, 512, 4
    r, b = synth(oracle, rows * width, 20), synth(oracle, rows * width, 21)
    mod = synth(oracle, 2 * slots * width, 22, 0.5)
    rm = (np.arange(rows) % 2).astype(np.uint32)
    out = gpu.new(rows * width, qd.BF16)
    gpu.check(qd.lib().h3_gpu_gate_bf16(gpu.h, out.h, gpu.put(r).h, gpu.put(b).h,
                                        gpu.put(mod).h, gpu.put(rm).h, rows, width, slots, 3),
              "gate")
    gpu.submit()
    ref = np.empty(rows * width, np.uint16)
    oracle.lib().qo_gate(ref, r, b, mod, rm, rows, width, slots, 3)
    assert ulp_diff(out.read(), ref).max() <= 1


@pytest.mark.parametrize("shift", [0, 1])
def test_modulation_reorder(gpu, qd, oracle, shift):
    H, S = 512, 6 if shift else 4
    raw = synth(oracle, 2 * S * H, 23, 2.0)
    out = gpu.new(2 * S * H, qd.BF16)
    gpu.check(qd.lib().qw_gpu_modulation_reorder_bf16(gpu.h, out.h, gpu.put(raw).h, 2, H,
                                                      shift), "reorder")
    gpu.submit()
    ref = np.empty(2 * S * H, np.uint16)
    oracle.lib().qo_modulation_reorder(ref, raw, 2, H, shift)
    # tanh: device vs libm may differ in the last fp32 bit before truncation
    assert ulp_diff(out.read(), ref).max() <= 1


def test_copy_rows_bit_exact(gpu, qd, oracle):
    src = synth(oracle, 50 * 96, 24)
    dst = gpu.new(50 * 40, qd.BF16)
    gpu.check(qd.lib().qw_gpu_copy_rows(gpu.h, dst.h, 0, 40, gpu.put(src).h, 32, 96, 50, 40),
              "copy")
    gpu.submit()
    assert np.array_equal(dst.read().reshape(50, 40), src.reshape(50, 96)[:, 32:72])


@pytest.fixture(autouse=True)
def _release_uploads(gpu):
    yield
    gpu.release()
