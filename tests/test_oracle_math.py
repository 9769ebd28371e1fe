"""Pin the oracle's dense/elementwise kernels with closed forms and brute
force in float64 (tests/test_prefix_kernel.c:72-97 style), chosen so a
dropped term, transposed operand, wrong sign or index fails."""
import math

import numpy as np
import pytest

from conftest import rel_l2


def bfv(o, x):
    return o.f32_to_bf16(np.asarray(x, np.float32))


def test_bf16_rounding_ties(oracle):
    L = oracle.lib()
    # exact ties: 1 + 2^-8 rounds to even (1.0), 1 + 3*2^-8 rounds up
    assert L.qo_f32_to_bf16(1.0 + 2**-8) == 0x3F80
    assert L.qo_f32_to_bf16(1.0 + 3 * 2**-8) == 0x3F82
    assert L.qo_f32_to_bf16(-2.5) == 0xC020
    assert L.qo_f32_to_bf16_trunc(1.0 + 255 * 2**-16) == 0x3F80
    rng = np.random.default_rng(0)
    x = rng.standard_normal(4096).astype(np.float32)
    v = np.array([L.qo_f32_to_bf16(float(t)) for t in x], np.uint16)
    assert np.array_equal(v, oracle.f32_to_bf16(x))
    # round trip error bounded by half an ulp (2^-9 relative)
    back = oracle.bf16_to_f32(v)
    assert np.all(np.abs(back - x) <= np.abs(x) * 2**-8)


def test_synth_normal_moments(oracle):
    v = oracle.bf16_to_f32(oracle.fill_normal_bf16(1 << 18, 5, 9)).astype(np.float64)
    assert abs(v.mean()) < 0.01 and abs(v.std() - 1.0) < 0.01
    assert abs(np.mean(v ** 4) - 3.0) < 0.1  # Irwin-Hall(12) kurtosis 2.9
    w = oracle.fill_normal_bf16(1000, 5, 10, 0.02, 1.0)
    assert abs(oracle.bf16_to_f32(w).mean() - 1.0) < 0.01
    # distinct streams / seeds give distinct values; same args reproduce
    assert not np.array_equal(oracle.fill_normal_bf16(64, 5, 9), oracle.fill_normal_bf16(64, 5, 10))
    assert np.array_equal(oracle.fill_normal_bf16(64, 5, 9), oracle.fill_normal_bf16(64, 5, 9))


@pytest.mark.parametrize("rows,k,n,bias", [(5, 64, 7, True), (33, 256, 130, False),
                                           (1, 3072, 3, True)])
def test_linear_brute_force(oracle, rows, k, n, bias):
    rng = np.random.default_rng(rows * 31 + n)
    x = bfv(oracle, rng.standard_normal((rows, k)))
    w = bfv(oracle, 0.02 * rng.standard_normal((n, k)))
    b = bfv(oracle, 0.02 * rng.standard_normal(n)) if bias else None
    y = oracle.linear(x, w, b, rows, k, n)
    ref = oracle.bf16_to_f32(x).astype(np.float64) @ oracle.bf16_to_f32(w).astype(np.float64).T
    if bias:
        ref += oracle.bf16_to_f32(b)
    # one rounding: within one bf16 ulp of the exact value
    got = oracle.bf16_to_f32(y)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2**-7 + 1e-6)


def test_linear_identity_and_one_hot(oracle):
    k = 64
    x = bfv(oracle, np.arange(3 * k).reshape(3, k) / 7.0)
    eye = bfv(oracle, np.eye(k))
    assert np.array_equal(oracle.linear(x, eye, None, 3, k, k), x)
    # one-hot row j picks column perm[j]: transposition would fail this
    perm = np.random.default_rng(1).permutation(k)
    w = np.zeros((k, k), np.float32)
    w[np.arange(k), perm] = 1.0
    y = oracle.linear(x, bfv(oracle, w), None, 3, k, k)
    assert np.array_equal(y, x[:, perm])


def test_int8_quantizer_closed_form(oracle):
    rows, cols = 4, 64
    w = np.zeros((rows, cols), np.float32)
    w[0] = np.linspace(-1, 1, cols)
    w[1, 5] = -0.5          # single element -> -127, rest 0
    w[2] = 0.0              # all-zero row: scale 1/127
    w[3] = np.full(cols, 0.25)
    w[3, 0] = 1.0
    wb = bfv(oracle, w)
    q, s = oracle.quantize_int8_rows(wb, rows, cols)
    wf = oracle.bf16_to_f32(wb)
    assert q[0, 0] == -127 and q[0, -1] == 127
    assert q[1, 5] == -127 and np.count_nonzero(q[1]) == 1
    assert np.all(q[2] == 0) and s[2] == np.float32(1.0 / 127.0)
    assert q[3, 0] == 127 and np.all(q[3, 1:] == 32)  # 0.25*127 = 31.75 -> 32
    inv = np.float32(127.0) / np.max(np.abs(wf), axis=1)
    for r in (0, 1, 3):
        exp = np.clip(np.rint((wf[r] * inv[r]).astype(np.float32)), -127, 127)
        assert np.array_equal(q[r], exp.astype(np.int8))
        assert s[r] == np.float32(np.max(np.abs(wf[r])) / np.float32(127.0))
    # ties go to even: value exactly 0.5 * max/127 * (2k+1)
    t = np.zeros((1, 4), np.float32)
    t[0] = [127.0, 0.5, 1.5, 2.5]
    qt, _ = oracle.quantize_int8_rows(bfv(oracle, t), 1, 4)
    assert list(qt[0]) == [127, 0, 2, 2]


def test_linear_i8_matches_dequantised(oracle):
    rng = np.random.default_rng(3)
    rows, k, n = 17, 128, 40
    x = bfv(oracle, rng.standard_normal((rows, k)))
    w = bfv(oracle, 0.02 * rng.standard_normal((n, k)))
    q, s = oracle.quantize_int8_rows(w, n, k)
    y = oracle.linear_i8(x, q, s, None, rows, k, n)
    deq = q.astype(np.float64) * s[:, None].astype(np.float64)
    ref = oracle.bf16_to_f32(x).astype(np.float64) @ deq.T
    assert np.all(np.abs(oracle.bf16_to_f32(y) - ref) <= np.abs(ref) * 2**-7 + 1e-5)
    # dequantised weights close to the originals (per-row step = scale)
    assert np.all(np.abs(deq - oracle.bf16_to_f32(w)) <= s[:, None] * 0.5 + 1e-9)


def _attn_ref(q, k, v, limits, heads, D, scale):
    qf, kf, vf = (np.asarray(t, np.float64).reshape(t.shape[0], heads, D) for t in (q, k, v))
    out = np.zeros_like(qf)
    for r in range(qf.shape[0]):
        lim = limits[r]
        for h in range(heads):
            s = kf[:lim, h] @ qf[r, h] * scale
            p = np.exp(s - s.max())
            out[r, h] = (p / p.sum()) @ vf[:lim, h]
    return out.reshape(qf.shape[0], heads * D)


@pytest.mark.parametrize("text,rows,causal", [(0, 16, 1), (8, 20, 1), (5, 37, 0)])
def test_attention_brute_force(oracle, text, rows, causal):
    heads, D = 2, 128
    rng = np.random.default_rng(rows)
    q, k, v = (bfv(oracle, rng.uniform(-1, 1, (rows, heads * D))) for _ in range(3))
    lim = oracle.t2i_limits(rows, text, causal)
    out = oracle.attention(q, k, v, lim, rows, rows, heads)
    f = oracle.bf16_to_f32
    ref = _attn_ref(f(q), f(k), f(v), lim, heads, D, 1 / math.sqrt(D))
    assert rel_l2(f(out), ref) < 4e-3  # bf16 output rounding only
    if text and causal:
        assert np.array_equal(out[0], v[0])  # first text row sees one key
    # text rows never see image keys: perturbing image keys leaves them fixed
    k2 = k.copy()
    k2[text:] = bfv(oracle, rng.uniform(-1, 1, (rows - text, heads * D)))
    out2 = oracle.attention(q, k2, v, lim, rows, rows, heads)
    assert np.array_equal(out2[:text], out[:text])


def test_attention_uniform_scores_mean_v(oracle):
    heads, D, rows = 1, 128, 9
    q = np.zeros((rows, D), np.uint16)  # zero query -> uniform softmax
    rng = np.random.default_rng(0)
    k = bfv(oracle, rng.standard_normal((rows, D)))
    v = bfv(oracle, rng.standard_normal((rows, D)))
    lim = np.arange(1, rows + 1, dtype=np.uint32)
    out = oracle.bf16_to_f32(oracle.attention(q, k, v, lim, rows, rows, heads))
    vf = oracle.bf16_to_f32(v).astype(np.float64)
    for r in range(rows):
        exp = vf[: r + 1].mean(axis=0)
        assert np.all(np.abs(out[r] - exp) <= np.abs(exp) * 2**-8 + 1e-6)


def test_t2i_limits(oracle):
    assert list(oracle.t2i_limits(6, 3, 1)) == [1, 2, 3, 6, 6, 6]
    assert list(oracle.t2i_limits(6, 3, 0)) == [3, 3, 3, 6, 6, 6]
    assert list(oracle.t2i_limits(4, 0, 1)) == [4, 4, 4, 4]


def test_head_rms_norm_and_rope(oracle):
    rows, heads, D = 3, 2, 128
    rng = np.random.default_rng(2)
    x = bfv(oracle, 3.0 * rng.standard_normal((rows, heads * D)))
    ones = bfv(oracle, np.ones(D))
    t = x.copy()
    oracle.lib().qo_head_rms_norm(t, heads * D, ones, rows, heads, D, 1e-6)
    tf = oracle.bf16_to_f32(t).reshape(rows, heads, D).astype(np.float64)
    assert np.allclose(np.sqrt((tf ** 2).mean(-1)), 1.0, atol=4e-3)
    # weight multiplies elementwise: w = 2 doubles the output exactly
    t2 = x.copy()
    oracle.lib().qo_head_rms_norm(t2, heads * D, bfv(oracle, 2 * np.ones(D)), rows, heads, D, 1e-6)
    assert np.array_equal(oracle.bf16_to_f32(t2), 2 * oracle.bf16_to_f32(t))
    # RoPE: zero angle is identity; quarter turn maps (a, b) -> (-b, a)
    c = np.ones((rows, 64), np.float32)
    s = np.zeros((rows, 64), np.float32)
    r = t.copy()
    oracle.lib().qo_qk_rope(r, heads * D, c, s, rows, heads, D)
    assert np.array_equal(r, t)
    c[:] = 0.0
    s[:] = 1.0
    oracle.lib().qo_qk_rope(r, heads * D, c, s, rows, heads, D)
    tv = oracle.bf16_to_f32(t).reshape(rows, heads, 64, 2)
    rv = oracle.bf16_to_f32(r).reshape(rows, heads, 64, 2)
    assert np.array_equal(rv[..., 0], -tv[..., 1]) and np.array_equal(rv[..., 1], tv[..., 0])
    # generic angle preserves each pair's norm
    ang = rng.uniform(-3, 3, (rows, 64))
    r = t.copy()
    oracle.lib().qo_qk_rope(r, heads * D, np.cos(ang).astype(np.float32),
                            np.sin(ang).astype(np.float32), rows, heads, D)
    n0 = np.hypot(tv[..., 0], tv[..., 1])
    n1 = np.hypot(*np.moveaxis(oracle.bf16_to_f32(r).reshape(rows, heads, 64, 2), -1, 0))
    assert np.allclose(n0, n1, rtol=1e-2)


def test_activations_textbook(oracle):
    xs = np.array([0.0, 1.0, -1.0, 2.0, -3.0, 20.0, -20.0], np.float32)
    xb = bfv(oracle, xs)
    out = np.empty_like(xb)
    oracle.lib().qo_gelu_tanh(out, xb, len(xs))
    g = oracle.bf16_to_f32(out)
    exact = 0.5 * xs * (1 + np.tanh(math.sqrt(2 / math.pi) * (xs + 0.044715 * xs ** 3)))
    assert np.allclose(g, exact, rtol=8e-3, atol=1e-6)
    assert g[5] == 20.0 and g[6] == 0.0  # saturation branches
    oracle.lib().qo_silu(out, xb, len(xs))
    assert np.allclose(oracle.bf16_to_f32(out), xs / (1 + np.exp(-xs.astype(np.float64))),
                       rtol=8e-3, atol=1e-6)
    fc1 = np.concatenate([xb, bfv(oracle, np.full(len(xs), 2.0))])[None, :]
    sw = np.empty((1, len(xs)), np.uint16)
    oracle.lib().qo_swiglu(sw, np.ascontiguousarray(fc1), 1, len(xs))
    assert np.array_equal(oracle.bf16_to_f32(sw[0]), 2 * oracle.bf16_to_f32(out))


def test_rms_norm_one(oracle):
    x = bfv(oracle, np.array([[3.0, 4.0, 0.0, 0.0]]))
    w = bfv(oracle, np.array([0.0, 0.0, 0.0, 1.0]))  # effective weight w + 1
    out = np.empty_like(x)
    oracle.lib().qo_rms_norm_one(out, x, w, 1, 4, 0.0)
    # rms = sqrt(25/4) = 2.5
    assert list(oracle.bf16_to_f32(out)[0]) == [1.203125, 1.6015625, 0.0, 0.0]


def test_prefix_limits_layouts(oracle, qd):
    """qwen_dit.m:1651-1665 by hand on a mixed layout, and the library's own
    host copy (qw_dit_prefix_limits) agrees."""
    import ctypes as C
    segs = [(3, 0, 0), (2, 1, 0), (2, 0, 3), (3, 1, 2)]
    want = [1, 2, 3, 5, 5, 6, 7, 10, 10, 10]
    assert oracle.prefix_limits(segs).tolist() == want
    out = np.zeros(10, np.uint32)
    qd.lib().qw_dit_prefix_limits(C.cast(oracle.segment_array(segs), C.c_void_p), 4,
                                  out.ctypes.data)
    assert out.tolist() == want
    # [text T, image I] is the t2i table with causal text
    assert oracle.prefix_limits([(4, 0, 0), (6, 1, 0)]).tolist() == \
        oracle.t2i_limits(10, 4, True).tolist()


def test_ti2i_reduces_to_causal_t2i(oracle):
    """The ti2i full pass over [text T; target image I] is the t2i forward
    with causal text rows: same rows, row map (text at t = 0) and limits. The
    one difference is the t2i text-row rule (q pre-scaled and re-rounded to
    bf16, h3_shaders.metal:4397-4401), which the ti2i prefix kernel does not
    apply: the two agree to the bf16 band (bit for bit with q = k = 0, see
    test_oracle_composition.py)."""
    cfg = dict(hidden=256, heads=2, mlp_width=512, text_dim=256, z_dim=64, layers=2,
               mlp_act=0, adaln_shift=0, has_bias=0, text_causal=1, int8_weights=0)
    T, gh, gw = 6, 4, 4
    I = gh * gw
    text = oracle.fill_normal_bf16(T * 256, 3, 50)
    lat = oracle.fill_normal_bf16(I * 64, 3, 51)
    cos, sin = oracle.rope_tables(T, gh, gw)
    m = oracle.Model(cfg, 9, 2)
    a = m.forward(text, T, lat, I, 0.7, cos, sin, 2)
    b = m.forward_ti2i(text, T, lat, I, [(T, 0, 0), (I, 1, 0)], 0.7, cos, sin, 2)
    m.close()
    f = oracle.bf16_to_f32
    assert not np.array_equal(a, b)
    assert rel_l2(f(a), f(b)) < 1e-2
