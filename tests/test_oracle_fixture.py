"""Pin the oracle's block-level elementwise ops against the reference's
weights-free dit_fixture stage pairs (tests/gen_dit_fixture.py:342-373,
tests/test_dit_block.c:204-244).

Two modes are checked. The fixture was written by diffusers on CPU bf16,
which rounds LN output, (1 + scale) and branch * gate to bf16 separately;
the oracle's torch_rounding mode reproduces those points and must be
BIT-EXACT, which pins the LayerNorm core (mean, variance, eps, row_map,
slot indexing) with no tolerance. The default mode is the Metal kernels'
single rounding and is held to the reference's own stage bound (2e-2)."""
import numpy as np
import pytest

from conftest import read_bf16, rel_l2

H = 4096
CASES = [("a", 0, 16), ("b", 8, 20)]


def _load(case, text, rows):
    rm = np.array([1 if i < text else 0 for i in range(rows)], np.uint32)
    return (read_bf16(f"{case}_joint_in.bin"), read_bf16(f"{case}_modulation.bin"), rm)


@pytest.mark.parametrize("case,text,rows", CASES)
def test_layer_norm_mod_attn_in(oracle, case, text, rows):
    joint, mod, rm = _load(case, text, rows)
    ref = read_bf16(f"{case}_attn_in.bin")
    out = np.empty_like(joint)
    oracle.lib().qo_layer_norm_mod_r(out, joint, mod, rm, rows, H, 4, 0, -1, 1e-6, 1)
    assert np.mean(out == ref) > 0.9999
    oracle.lib().qo_layer_norm_mod(out, joint, mod, rm, rows, H, 4, 0, -1, 1e-6)
    f = oracle.bf16_to_f32
    assert rel_l2(f(out), f(ref)) < 2e-2
    assert np.max(np.abs(out.astype(np.int32) - ref.astype(np.int32))) <= 2


@pytest.mark.parametrize("case,text,rows", CASES)
def test_gate_ln_gate_block_out(oracle, case, text, rows):
    joint, mod, rm = _load(case, text, rows)
    attn_out = read_bf16(f"{case}_attn_out.bin")
    mlp_out = read_bf16(f"{case}_mlp_out.bin")
    L = oracle.lib()
    for torch_rounding in (1, 0):
        h1 = np.empty_like(joint)
        L.qo_gate_r(h1, joint, attn_out, mod, rm, rows, H, 4, 2, torch_rounding)
        mlp_in = np.empty_like(joint)
        L.qo_layer_norm_mod_r(mlp_in, h1, mod, rm, rows, H, 4, 1, -1, 1e-6,
                              torch_rounding)
        out = np.empty_like(joint)
        L.qo_gate_r(out, h1, mlp_out, mod, rm, rows, H, 4, 3, torch_rounding)
        ref_in = read_bf16(f"{case}_mlp_in.bin")
        ref_out = read_bf16(f"{case}_block_out.bin")
        if torch_rounding:
            assert np.array_equal(mlp_in, ref_in)
            assert np.array_equal(out, ref_out)
        else:
            f = oracle.bf16_to_f32
            assert rel_l2(f(mlp_in), f(ref_in)) < 2e-2
            assert rel_l2(f(out), f(ref_out)) < 1e-2


@pytest.mark.parametrize("case,text,rows", CASES)
def test_norm_out_per_column_scale(oracle, case, text, rows):
    """norm_out = LN(block_out) * (1 + s_c) per column c for the image rows
    (the weight-dependent s_c is unknown). With torch rounding, each column
    must admit ONE bf16 factor reproducing every image row exactly."""
    block = read_bf16(f"{case}_block_out.bin")
    ref = oracle.bf16_to_f32(read_bf16(f"{case}_norm_out.bin")).reshape(rows, H)
    zero_mod = np.zeros(H, np.uint16)
    ln = np.empty_like(block)
    oracle.lib().qo_layer_norm_mod_r(ln, block, zero_mod, np.zeros(rows, np.uint32),
                                     rows, H, 1, 0, -1, 1e-6, 1)
    ln = oracle.bf16_to_f32(ln).reshape(rows, H)[text:]
    tgt = ref[text:]
    good = 0
    for c in range(H):
        big = np.abs(ln[:, c]) > 1e-3
        if not np.any(big):
            good += 1
            continue
        guess = np.median(tgt[big, c] / ln[big, c])
        base = int(oracle.f32_to_bf16(np.array([guess], np.float32))[0])
        ok = False
        for d in range(-3, 4):
            if not 0 <= base + d < 65536:
                continue
            f = oracle.bf16_to_f32(np.array([base + d], np.uint16))[0]
            pred = oracle.bf16_to_f32(oracle.f32_to_bf16((ln[:, c] * f).astype(np.float32)))
            if np.array_equal(pred, tgt[:, c]):
                ok = True
                break
        good += ok
    assert good / H > 0.999


@pytest.mark.parametrize("case", ["a", "b"])
def test_modulation_slot_layout(oracle, case):
    """The fixture modulation is in slot layout [s1, s2, tanh g1, tanh g2]:
    gates lie in [-1, 1] (tanh saturates to 1 in bf16). A raw vector built
    from it must reorder back."""
    mod = read_bf16(f"{case}_modulation.bin").reshape(2, 4, H)
    g = oracle.bf16_to_f32(mod[:, 2:])
    assert np.all(np.abs(g) <= 1.0)
    g = np.clip(g, -0.9999, 0.9999)
    # raw layout [s1 | g1_raw | s2 | g2_raw] with g_raw = atanh(g): tanh(g_raw)
    # truncated to bf16 must land within 1 ulp of g
    raw = np.empty((2, 4, H), np.uint16)
    raw[:, 0] = mod[:, 0]
    raw[:, 2] = mod[:, 1]
    raw[:, 1] = oracle.f32_to_bf16(np.arctanh(g[:, 0]).astype(np.float32))
    raw[:, 3] = oracle.f32_to_bf16(np.arctanh(g[:, 1]).astype(np.float32))
    out = np.empty_like(raw)
    oracle.lib().qo_modulation_reorder(out.reshape(-1), raw.reshape(-1), 2, H, 0)
    assert np.array_equal(out[:, :2], mod[:, :2])
    diff = np.abs(out[:, 2:].astype(np.int32) - mod[:, 2:].astype(np.int32))
    assert np.mean(diff <= 2) > 0.99
