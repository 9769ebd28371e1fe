"""Static check of the built gfx950 code object for the instruction-distance
hazards that inline assembly hides from the compiler.

The GEMM kernels issue their MFMAs, the int8 GEMMs their raw weight loads
and widening conversions, and all kernels their LDS-direct loads, from
inline assembly. The compiler's hazard recognizer does not look inside
an asm statement, so the wait states that gfx9 requires between these
instructions and the compiler's own are not guaranteed by construction; a
schedule change can place, say, an accumulator write right before the MFMA
that reads it, and the MFMA then reads the old value with no error. This
script disassembles the code object (``llvm-objdump``, after unbundling the
gfx950 image) and measures, along every control-flow path (fall-through and
branches), the wait states between:

  valu->mfma   a VALU write of a VGPR/AGPR and an MFMA reading it
               (srcA, srcB or srcC): 2
  mfma->read   an MFMA result and any other instruction reading it
               (VALU, accvgpr read, LDS/global store data or address), or
               another MFMA reading it as srcA/srcB: passes + 3
  mfma->write  an MFMA result and a VALU write of the same register: passes + 3
  srcc->write  an MFMA reading a register as srcC and a VALU write of it: passes
  m0->lds      an SALU write of M0 and an LDS-direct load (``... lds``): 1

(``s_nop N`` counts N + 1 wait states, every other instruction 1; passes
as counted here: 4x4 2, 16x16 8, 32x32 16. These are upper bounds: for its
own builtin MFMAs the compiler pads a VALU read of a 16x16x32 result with 8
wait states, of a 32x32x16 result with 12, and an MFMA after a VALU write
of its srcA with 1, so every limit here is at least the compiler's; the
tests compile such a probe and check that.) An MFMA reading its own
destination as srcC with the same register range chains in hardware and
needs none. Exit status 1 and
a listing when any distance is short.

Usage: python hazard_check.py <code object .hsaco> [--max N]
"""
import os
import re
import subprocess
import sys
import tempfile

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
LLVM = os.path.join(ROCM, "llvm", "bin")

VALU_WRITE_TO_MFMA = 2
MFMA_EXTRA = 3
M0_TO_LDS_DMA = 1


def _regs(tok):
    m = re.fullmatch(r"([va])\[(\d+):(\d+)\]", tok)
    if m:
        return {(m.group(1), i) for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.fullmatch(r"([va])(\d+)", tok)
    if m:
        return {(m.group(1), int(m.group(2)))}
    return set()


def _passes(op):
    if "_32x32x" in op:
        return 16
    if "_16x16x" in op:
        return 8
    if "_4x4x" in op:
        return 2
    return 16


class Insn:
    __slots__ = ("addr", "text", "op", "ops", "nws", "dst", "srcs", "mfma", "m0w",
                 "lds_dma", "succ", "pred", "valu_write")

    def __init__(self, addr, text):
        self.addr, self.text = addr, text
        self.op = text.split()[0]
        rest = text[len(self.op):]
        rest = re.split(r"\s(?:offen|idxen|offset:|lds|glc|slc|nt|sc0|sc1|neg_lo|neg_hi|"
                        r"cbsz|abid|blgp|op_sel)", rest)[0]
        self.ops = [t.strip() for t in rest.split(",") if t.strip()]
        self.nws = int(self.ops[0], 0) + 1 if self.op == "s_nop" else 1
        self.mfma = self.op.startswith("v_mfma") or self.op.startswith("v_smfmac")
        op = self.op
        writes_vreg = (op.startswith("v_") and not self.mfma and not op.startswith("v_cmp")
                       and not op.startswith("v_readfirstlane") and not op.startswith("v_readlane")
                       and bool(self.ops))
        self.valu_write = _regs(self.ops[0]) if writes_vreg else set()
        if self.mfma:
            self.dst = _regs(self.ops[0])
            self.srcs = [_regs(t) for t in self.ops[1:4]]
        else:
            self.dst = set()
            # every register this instruction reads (for a VALU write the
            # first operand is the destination)
            toks = self.ops[1:] if writes_vreg or op.startswith(("ds_read", "buffer_load",
                                                                 "global_load", "flat_load",
                                                                 "scratch_load")) else self.ops
            self.srcs = [set().union(*[_regs(t) for t in toks])] if toks else [set()]
        self.m0w = op.startswith("s_") and bool(self.ops) and self.ops[0] == "m0"
        self.lds_dma = (op.startswith(("buffer_load", "global_load")) and
                        re.search(r"\slds(\s|$)", text) is not None)
        self.succ, self.pred = [], []


def disassemble(hsaco):
    with tempfile.TemporaryDirectory() as td:
        co = os.path.join(td, "k.co")
        subprocess.run([os.path.join(LLVM, "clang-offload-bundler"), "--type=o",
                        "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", "--input=" + hsaco,
                        "--output=" + co, "--unbundle"], check=True)
        return subprocess.run([os.path.join(LLVM, "llvm-objdump"), "-d", "--mcpu=gfx950", co],
                              check=True, capture_output=True, text=True).stdout


def functions(dis):
    """{name: [Insn]} with successor/predecessor links inside each function."""
    funcs, cur, name, base = {}, None, None, 0
    for line in dis.split("\n"):
        m = re.match(r"^([0-9a-f]+) <([^>]+)>:$", line)
        if m:
            base, name = int(m.group(1), 16), m.group(2)
            cur = funcs.setdefault(name, [])
            continue
        if cur is None or not line.startswith("\t"):
            continue
        body, _, cmt = line.strip().partition("//")
        body = body.strip()
        am = re.match(r"\s*([0-9A-Fa-f]+):", cmt)
        if not body or not am:
            continue
        ins = Insn(int(am.group(1), 16), body)
        tm = re.search(r"<([^>+]+)\+0x([0-9a-f]+)>", cmt)
        ins.succ = [("target", tm.group(1), base + int(tm.group(2), 16))] if tm else []
        cur.append(ins)
    for name, ins in funcs.items():
        at = {x.addr: x for x in ins}
        for i, x in enumerate(ins):
            tgt = [at.get(a) for _, f, a in x.succ if f == name]
            x.succ = [t for t in tgt if t is not None]
            if i + 1 < len(ins) and x.op not in ("s_branch", "s_endpgm", "s_setpc_b64"):
                x.succ.append(ins[i + 1])
            for s in x.succ:
                s.pred.append(x)
    return funcs


def _back(x, budget, want):
    """Instructions before x (over all paths) within `budget` wait states:
    yields (wait states between, instruction) for those matching want()."""
    seen = {}
    stack = [(p, 0) for p in x.pred]
    while stack:
        y, ws = stack.pop()
        if ws >= budget or seen.get(id(y), budget + 1) <= ws:
            continue
        seen[id(y)] = ws
        if want(y):
            yield ws, y
        stack.extend((p, ws + y.nws) for p in y.pred)


def check(funcs):
    bad = []
    for name, ins in funcs.items():
        for x in ins:
            if x.mfma:
                reads = set().union(*x.srcs)
                for ws, y in _back(x, VALU_WRITE_TO_MFMA, lambda y: y.valu_write & reads):
                    bad.append((name, "valu->mfma", ws, VALU_WRITE_TO_MFMA, y, x))
                ab = set().union(*x.srcs[:2])
                for ws, y in _back(x, 16 + MFMA_EXTRA,
                                   lambda y: y.mfma and y.dst & ab):
                    need = _passes(y.op) + MFMA_EXTRA
                    if ws < need:
                        bad.append((name, "mfma->read", ws, need, y, x))
                srcc = x.srcs[2] if len(x.srcs) > 2 else set()
                for ws, y in _back(x, 16 + MFMA_EXTRA,
                                   lambda y: y.mfma and y.dst & srcc and y.dst != srcc):
                    need = _passes(y.op) + MFMA_EXTRA
                    if ws < need:
                        bad.append((name, "mfma->read", ws, need, y, x))
            else:
                reads = x.srcs[0]
                if reads:
                    for ws, y in _back(x, 16 + MFMA_EXTRA, lambda y: y.mfma and y.dst & reads):
                        need = _passes(y.op) + MFMA_EXTRA
                        if ws < need:
                            bad.append((name, "mfma->read", ws, need, y, x))
                if x.valu_write:
                    w = x.valu_write
                    for ws, y in _back(x, 16 + MFMA_EXTRA, lambda y: y.mfma and y.dst & w):
                        need = _passes(y.op) + MFMA_EXTRA
                        if ws < need:
                            bad.append((name, "mfma->write", ws, need, y, x))
                    for ws, y in _back(x, 16, lambda y: y.mfma and len(y.srcs) > 2
                                       and y.srcs[2] & w):
                        need = _passes(y.op)
                        if ws < need:
                            bad.append((name, "srcc->write", ws, need, y, x))
                if x.lds_dma:
                    for ws, y in _back(x, M0_TO_LDS_DMA, lambda y: y.m0w):
                        bad.append((name, "m0->lds", ws, M0_TO_LDS_DMA, y, x))
    return bad


def main(argv):
    if len(argv) < 2:
        print(__doc__)
        return 2
    show = int(argv[argv.index("--max") + 1]) if "--max" in argv else 20
    funcs = functions(disassemble(argv[1]))
    bad = check(funcs)
    n = sum(len(v) for v in funcs.values())
    if not bad:
        print("hazard_check: %d instructions in %d kernels, no short distances" % (n, len(funcs)))
        return 0
    kinds = {}
    for b in bad:
        kinds.setdefault((b[0], b[1]), 0)
        kinds[(b[0], b[1])] += 1
    print("hazard_check: %d short distances" % len(bad))
    for (f, k), c in sorted(kinds.items()):
        print("  %-48s %-12s %d" % (f, k, c))
    for f, k, ws, need, y, x in bad[:show]:
        print("  %s %s: %d < %d wait states\n      %06x %s\n      %06x %s"
              % (f, k, ws, need, y.addr, y.text, x.addr, x.text))
    return 1


if __name__ == "__main__":
    sys.exit(main(sys.argv))
