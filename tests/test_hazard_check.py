"""The code-object hazard scanner (qwen-metal_amd/hazard_check.py): each
rule flags a short distance and passes the same sequence once the gfx9
minimum of wait states separates the two instructions, over straight-line
code and over a loop's back edge; and the built kernels pass it. (CPU only:
the scanner reads disassembly.)"""
import importlib.util
import os
import shutil

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
_spec = importlib.util.spec_from_file_location(
    "hazard_check", os.path.join(ROOT, "qwen-metal_amd", "hazard_check.py"))
hc = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(hc)

BASE = 0x1000


def objdump(body, name="k"):
    """llvm-objdump-style text for one function: `body` lists instructions
    (4 bytes each); '@N' in a branch names the target instruction index."""
    out = ["%016x <%s>:" % (BASE, name)]
    for i, ins in enumerate(body):
        addr = BASE + 4 * i
        tgt = ""
        if "@" in ins:
            ins, t = ins.split("@")
            tgt = " <%s+0x%x>" % (name, 4 * int(t))
        out.append("\t%-58s// %012X: 00000000%s" % (ins.strip(), addr, tgt))
    return "\n".join(out) + "\n"


def kinds(body):
    return sorted({(b[1], b[2], b[3]) for b in hc.check(hc.functions(objdump(body)))})


MFMA = "v_mfma_f32_16x16x32_bf16 a[0:3], v[4:7], v[8:11], a[0:3]"


def test_valu_write_then_mfma():
    assert kinds(["v_accvgpr_write_b32 a1, v20", MFMA]) == [("valu->mfma", 0, 2)]
    assert kinds(["v_mov_b32 v9, 0", "s_nop 0", MFMA]) == [("valu->mfma", 1, 2)]
    assert kinds(["v_mov_b32 v9, 0", "s_nop 1", MFMA]) == []
    assert kinds(["v_mov_b32 v12, 0", MFMA]) == []            # not an operand
    assert kinds(["v_cmp_eq_u32_e32 vcc, v4, v5", MFMA]) == []  # writes no VGPR


def test_mfma_result_then_read():
    # 8 passes + 3 = 11 wait states before anything else reads the result
    assert kinds([MFMA, "s_nop 7", "ds_write_b128 v30, a[0:3]"]) == [("mfma->read", 8, 11)]
    assert kinds([MFMA, "s_nop 7", "s_nop 2", "ds_write_b128 v30, a[0:3]"]) == []
    assert kinds([MFMA, "v_accvgpr_read_b32 v1, a2"]) == [("mfma->read", 0, 11)]
    assert kinds([MFMA, "v_add_f32_e32 v1, v2, v3"]) == []
    # as srcA of the next MFMA; as srcC of another shape of range
    assert kinds([MFMA, "v_mfma_f32_16x16x32_bf16 a[4:7], a[0:3], v[8:11], a[4:7]"]) == \
        [("mfma->read", 0, 11)]
    assert kinds([MFMA, "v_mfma_f32_16x16x32_bf16 a[2:5], v[4:7], v[8:11], a[2:5]"]) == \
        [("mfma->read", 0, 11)]
    # the same accumulator chained: no wait
    assert kinds([MFMA, MFMA]) == []


def test_mfma_then_valu_write():
    big = "v_mfma_f32_32x32x16_bf16 a[0:15], v[4:7], v[8:11], a[0:15]"
    got = kinds([big, "s_nop 7", "v_accvgpr_write_b32 a3, 0"])
    assert ("mfma->write", 8, 19) in got and ("srcc->write", 8, 16) in got
    assert kinds([big] + ["s_nop 7"] * 3 + ["v_accvgpr_write_b32 a3, 0"]) == []


def test_m0_then_lds_dma():
    dma = "buffer_load_dwordx4 v1, s[8:11], s12 offen lds"
    assert kinds(["s_mov_b32 m0, s4", dma]) == [("m0->lds", 0, 1)]
    assert kinds(["s_mov_b32 m0, s4", "s_nop 0", dma]) == []
    assert kinds(["s_mov_b32 m0, s4", "buffer_load_dwordx4 v1, s[8:11], s12 offen"]) == []


def test_across_back_edge_and_branches():
    # the loop's last instruction writes what its first MFMA reads
    loop = [MFMA, "s_add_u32 s0, s0, 1", "v_mov_b32 v5, v6", "s_cbranch_scc1 @0"]
    assert kinds(loop) == [("valu->mfma", 1, 2)]  # the branch is one wait state
    # a forward branch over the padding: the short path is the one flagged
    fwd = ["v_mov_b32 v5, v6", "s_cbranch_scc1 @4", "s_nop 7", "s_nop 7", MFMA]
    assert kinds(fwd) == [("valu->mfma", 1, 2)]
    # s_branch does not fall through
    jmp = ["v_mov_b32 v5, v6", "s_branch @4", "s_nop 7", "s_endpgm", "s_nop 1", MFMA]
    assert kinds(jmp) == []


def test_built_code_object_is_clean():
    hsaco = os.path.join(ROOT, "qwen-metal_amd", "lib", "qwen_kernels.hsaco")
    if not os.path.exists(hsaco):
        pytest.skip("code object not built")
    if not shutil.which(os.path.join(hc.LLVM, "llvm-objdump")):
        pytest.skip("llvm-objdump absent")
    funcs = hc.functions(hc.disassemble(hsaco))
    assert any(any(x.mfma for x in v) for v in funcs.values())
    assert any(any(x.lds_dma for x in v) for v in funcs.values())
    bad = hc.check(funcs)
    assert not bad, [(b[0], b[1], b[2], b[3], b[4].text, b[5].text) for b in bad[:5]]


PROBE = r"""
#include <hip/hip_runtime.h>
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
extern "C" __global__ void k16(const bf16x8 *a, float *o) {
    floatx4 acc = {0, 0, 0, 0};
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[threadIdx.x], a[threadIdx.x + 64], acc, 0, 0, 0);
    o[threadIdx.x] = acc[0] * 3.0f;
}
extern "C" __global__ void k32(const bf16x8 *a, float *o) {
    floatx16 acc = {};
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[threadIdx.x], a[threadIdx.x + 64], acc, 0, 0, 0);
    o[threadIdx.x] = acc[0] * 3.0f;
}
extern "C" __global__ void kw(const bf16x8 *a, float *o) {
    bf16x8 x = a[threadIdx.x];
    x[0] = (__bf16)(o[threadIdx.x] * 2.0f);
    floatx4 acc = {0, 0, 0, 0};
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x, a[threadIdx.x + 64], acc, 0, 0, 0);
    o[threadIdx.x + 64] = acc[1];
}
"""


def test_distances_not_below_the_compilers(tmp_path):
    """The compiler pads its own (builtin) MFMAs with the wait states it
    deems necessary; the scanner must demand at least as many. Probe: a
    VALU read right after a 16x16x32 and a 32x32x16 result, and an MFMA
    right after a VALU write of its srcA; the padding the compiler chose is
    measured with the scanner's own distance walk."""
    hipcc = os.path.join(os.path.dirname(hc.LLVM), "..", "bin", "hipcc")
    hipcc = os.path.normpath(hipcc)
    if not os.path.exists(hipcc):
        pytest.skip("hipcc absent")
    import subprocess
    src, s = tmp_path / "probe.hip", tmp_path / "probe.s"
    src.write_text(PROBE)
    subprocess.run([hipcc, "--offload-arch=gfx950", "-O3", "--cuda-device-only", "-S",
                    "-o", str(s), str(src)], check=True, capture_output=True)
    # the assembly listing in llvm-objdump's layout: one function per kernel
    text, addr, name = [], 0, None
    for line in s.read_text().split("\n"):
        body = line.split(";")[0].strip()
        if body.endswith(":") and body[:-1] in ("k16", "k32", "kw"):
            name = body[:-1]
            text.append("%016x <%s>:" % (addr, name))
            continue
        if name is None or not body or body.startswith(".") or body.endswith(":"):
            continue
        text.append("\t%-58s// %012X: 00000000" % (body, addr))
        addr += 4
        if body.startswith("s_endpgm"):
            name = None
    funcs = hc.functions("\n".join(text) + "\n")
    seen = {}
    for fn, ins in funcs.items():
        for x in ins:
            if not x.mfma and x.srcs[0]:
                for ws, y in hc._back(x, 40, lambda y: y.mfma and y.dst & x.srcs[0]):
                    seen[(fn, "mfma->read")] = min(ws, seen.get((fn, "mfma->read"), 99))
                    need = hc._passes(y.op) + hc.MFMA_EXTRA
                    assert need >= ws, (fn, ws, need)
            if x.mfma:
                reads = set().union(*x.srcs)
                for ws, y in hc._back(x, 12, lambda y: y.valu_write & reads):
                    seen[(fn, "valu->mfma")] = min(ws, seen.get((fn, "valu->mfma"), 99))
                    assert hc.VALU_WRITE_TO_MFMA >= ws, (fn, ws)
    # the probe exercised every case (the compiler's padding: 8, 12 and 1)
    assert {("k16", "mfma->read"), ("k32", "mfma->read"), ("kw", "valu->mfma")} <= set(seen)
