"""qw_gpu_linear_static (the entry point that allocates nothing) against
qw_gpu_linear on the same inputs, through the C-ABI: two calls in a row,
the second on a smaller input, each within one bf16 ulp of the allocating
entry point (or within 2^-14 sum |x||w| where the sum cancels; with the
residual gate, both within one ulp of the oracle's gate of y or of a bf16
neighbour of y), and no
device allocation by the runtime across the static calls."""
import numpy as np
import pytest

from conftest import bf16_neighbours, ulp_diff

pytestmark = pytest.mark.gpu
SEED = 77


def _close(oracle, got, ref, mag, epi):
    """the linear bar of the parity tests: one ulp (or 2^-14 sum |x||w|);
    after GELU or the residual gate one flip of the linear's rounding plus
    one output rounding: two ulps (or 2^-13 sum |x||w|)"""
    ulps, frac = (1, 2.0 ** -14) if epi == "store" else (2, 2.0 ** -13)
    d = ulp_diff(got, ref)
    diff = np.abs(oracle.bf16_to_f32(got).astype(np.float64) - oracle.bf16_to_f32(ref))
    ok = (d <= ulps) | (diff <= frac * mag)
    assert ok.all(), (int(d.max()), np.flatnonzero(~ok)[:5])


# (k, n, int8, epilogue, rows of the first call, rows of the second)
CASES = [
    # K = 12288: split tiles in both entry points (static: fewer pieces)
    (12288, 3072, False, "store", 1152, 600),
    # int8: qw_gpu_linear widens to bf16 first (>= 512 rows), the static
    # form widens in LDS inside the GEMM
    (3072, 1536, True, "gelu", 1100, 520),
    (3072, 3072, True, "gate", 700, 64),
]


@pytest.mark.parametrize("k,n,int8,epi,m1,m2", CASES)
def test_linear_static_matches_linear(qd, oracle, k, n, int8, epi, m1, m2):
    gpu = qd.Gpu()  # a fresh context: its runtime owns no workspace yet
    try:
        E = {"store": qd.LINEAR_STORE, "gelu": qd.LINEAR_GELU, "gate": qd.LINEAR_GATE}[epi]
        x = oracle.fill_normal_bf16(m1 * k, SEED, 1)
        w = oracle.fill_normal_bf16(n * k, SEED, 2, 0.02)
        b = oracle.fill_normal_bf16(n, SEED, 3, 0.02)
        if int8:
            q, s = oracle.quantize_int8_rows(w, n, k)
            wt, st = gpu.put(q), gpu.put(s)
        else:
            wt, st = gpu.put(w), None
        xt, bt = gpu.put(x), gpu.put(b)
        res = oracle.fill_normal_bf16(m1 * n, SEED, 4)
        gmod = oracle.fill_normal_bf16(2 * 4 * n, SEED, 5, 0.3)
        rm = (np.arange(m1) % 3 == 0).astype(np.uint32)
        gate = dict(modulation=gpu.put(gmod), row_map=gpu.put(rm), slots=4, gate_slot=2) \
            if epi == "gate" else {}
        absx, absw = x & np.uint16(0x7FFF), w & np.uint16(0x7FFF)
        outs = {}
        for no_alloc in (False, True):
            outs[no_alloc] = []
            for rows in (m1, m2):
                out = gpu.put(res[:rows * n].copy())  # the GATE epilogue adds into it
                gpu.submit()
                before = gpu.stats().allocated_bytes
                gpu.linear(out, xt, wt, rows, k, n, bias=bt, wscale=st, epilogue=E,
                           no_alloc=no_alloc, **gate)
                gpu.submit()
                grew = gpu.stats().allocated_bytes > before
                if no_alloc:
                    assert not grew
                elif rows == m1:
                    # the allocating entry point's first call does allocate
                    # its workspace (split partials or the int8 widening
                    # buffer): the check above would see an allocation
                    assert grew
                outs[no_alloc].append(out.read())
        for i, rows in enumerate((m1, m2)):
            if epi == "gate":
                # the entry points may split K differently (the allocating
                # one runs a small launch as half tiles in k-ranges), so
                # bf16(y) can round the other way at a rounding boundary;
                # where h + y g cancels, that moves the output by many of its
                # ulps. Both hold the gate of the oracle's y or of either bf16
                # neighbour of y within one output ulp.
                xs = x[:rows * k].copy()
                lin = (oracle.linear_i8(xs, q, s, b, rows, k, n) if int8 else
                       oracle.linear(xs, w, b, rows, k, n)).ravel()
                h0 = res[:rows * n].copy()
                for got in (outs[True][i], outs[False][i]):
                    best = None
                    for yv in (lin,) + bf16_neighbours(lin):
                        want = np.empty(rows * n, np.uint16)
                        oracle.lib().qo_gate(want, h0, np.ascontiguousarray(yv), gmod,
                                             np.ascontiguousarray(rm[:rows]), rows, n, 4, 2)
                        d = ulp_diff(got, want)
                        best = d if best is None else np.minimum(best, d)
                    assert best.max() <= 1, best.max()
                continue
            mag = oracle.bf16_to_f32(oracle.linear(absx[:rows * k].copy(), absw, None, rows, k,
                                                   n)).ravel()
            _close(oracle, outs[True][i], outs[False][i], mag, epi)
    finally:
        gpu.close()


def test_linear_static_two_contexts_in_flight(qd, oracle):
    """Two contexts (two streams) on one GPU share the static workspace: the
    second context's call is issued while the first one's split-tile linear
    (K = 12288, its pieces' fp32 partials and counters in the workspace) is
    still in flight, with no synchronisation between them. The per-device
    ordering makes the second call wait for the first, so both outputs equal
    those of the same calls run one at a time on the allocating entry
    point (bit for bit where both split alike, else to the linear bar), and the workspace's counters are left
    at zero (a third call matches too)."""
    k, n, rows = 12288, 3072, 1152
    gpus = [qd.Gpu(), qd.Gpu()]
    try:
        ins = []
        for i, g in enumerate(gpus):
            x = oracle.fill_normal_bf16(rows * k, SEED, 10 + i)
            w = oracle.fill_normal_bf16(n * k, SEED, 20 + i, 0.02)
            ins.append((g.put(x), g.put(w), g.new(rows * n, qd.BF16), g.new(rows * n, qd.BF16)))
        for g in gpus:
            g.submit()
        # one at a time, allocating path, as the reference result
        for g, (xt, wt, ref, _) in zip(gpus, ins):
            g.linear(ref, xt, wt, rows, k, n)
            g.submit()
        # both static calls in flight together, then a third on the first context
        for g, (xt, wt, _, out) in zip(gpus, ins):
            g.linear(out, xt, wt, rows, k, n, no_alloc=True)
        for g in gpus:
            g.submit()
        got = [out.read() for (_, _, _, out) in ins]
        want = [ref.read() for (_, _, ref, _) in ins]
        xt, wt, _, out = ins[0]
        gpus[0].linear(out, xt, wt, rows, k, n, no_alloc=True)
        gpus[0].submit()
        again = out.read()
    finally:
        for g in gpus:
            g.close()
    mag = None
    for i in range(2):
        if not np.array_equal(got[i], want[i]):
            # the static form may split differently from the allocating one
            # (its workspace holds 128 pieces; it runs whole tiles where the
            # allocating one runs a small launch as half tiles): then the
            # linear bar applies
            x = oracle.fill_normal_bf16(rows * k, SEED, 10 + i)
            w = oracle.fill_normal_bf16(n * k, SEED, 20 + i, 0.02)
            mag = oracle.bf16_to_f32(oracle.linear(x & np.uint16(0x7FFF), w & np.uint16(0x7FFF),
                                                   None, rows, k, n)).ravel()
            _close(oracle, got[i], want[i], mag, "store")
    assert np.array_equal(again, got[0])
