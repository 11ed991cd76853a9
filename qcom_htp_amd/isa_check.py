"""Static check of the GEMM's hand-counted memory waits in its compiled gfx950 assembly.

The GEMM k loop issues every vector-memory request (the activation DMA and the weight-fragment
loads) from inline assembly and waits for them with explicit ``s_waitcnt vmcnt(N)`` counts; the
compiler does not see those loads, so nothing stops it from reading, copying or reusing a
destination register before its data has arrived.  This check walks the assembly of each kernel
from its entry through the first loop (three times, for the requests carried from one iteration
into the next) to the first ``vmcnt(0)`` after it, keeping the in-order queue of outstanding
vector-memory requests, and reports every instruction that names a register a pending load
will still write.  ``qcom_htp_amd.build`` runs it on every build and fails on a violation.

    python -m qcom_htp_amd.isa_check path/to/qmm_gemm-hip-amdgcn-amd-amdhsa-gfx950.s
"""

from __future__ import annotations

import re
import sys

_VMEM = re.compile(r"^(global_|buffer_|flat_|scratch_)(\w+)")
_REG = re.compile(r"\bv\[(\d+):(\d+)\]|\bv(\d+)\b")
_VMCNT = re.compile(r"s_waitcnt\b.*?vmcnt\((\d+)\)")


def _regs(text: str) -> set:
    out = set()
    for a, b, c in _REG.findall(text):
        if c:
            out.add(int(c))
        else:
            out.update(range(int(a), int(b) + 1))
    return out


def _body(lines: list, name: str) -> list:
    start = next(i for i, l in enumerate(lines) if l.startswith(name + ":"))
    end = next(i for i in range(start, len(lines)) if "s_endpgm" in lines[i])
    return [l.split(";")[0].strip() for l in lines[start:end + 1]]


def _target(ins: str):
    return ins.split()[-1] if ins.startswith(("s_cbranch", "s_branch")) else None


def check_kernel(lines: list, name: str) -> list:
    """Violations in kernel ``name`` (empty list: none)."""
    ins = _body(lines, name)
    head = next((i for i, l in enumerate(ins) if l.startswith(".LBB") and l.endswith(":")
                 and any(_target(x) == l[:-1] for x in ins[i + 1:])), None)
    if head is None:
        return [f"{name}: no loop found"]
    label = ins[head][:-1]
    back = next(i for i in range(head + 1, len(ins)) if _target(ins[i]) == label)
    after = next((i for i in range(back, len(ins)) if re.search(r"vmcnt\(0\)", ins[i])), None)
    if after is None:
        return [f"{name}: no vmcnt(0) after the loop"]
    seq = ins[:head] + ins[head:back + 1] * 3 + ins[back + 1:after + 1]
    queue: list = []  # (destination registers, instruction), oldest first
    errs = []
    for t in seq:
        if not t or t.startswith(".") or t.endswith(":"):
            continue
        m = _VMCNT.search(t)
        if m:
            del queue[:max(0, len(queue) - int(m.group(1)))]
            continue
        if t.startswith("s_waitcnt"):
            continue
        touched = _regs(t)
        for dst, src in queue:
            if dst & touched:
                errs.append(f"{name}: '{t}' names v{sorted(dst & touched)} while '{src}' is pending")
        mv = _VMEM.match(t)
        if mv:
            op = mv.group(2)
            dst = _regs(t.split(None, 1)[1].split(",")[0]) if op.startswith("load") and "_lds" not in op else set()
            queue.append((dst, t))
    return errs


def check_file(path: str, pattern: str = r"qmm_gemm_kernel") -> tuple:
    """(kernels checked, violations) for the kernels whose symbol matches ``pattern``."""
    lines = open(path).read().splitlines()
    names = [l.split(":")[0] for l in lines if re.match(r"^_Z\w*" + pattern + r"\w*:", l)]
    errs = []
    for n in names:
        errs += check_kernel(lines, n)
    return names, errs


if __name__ == "__main__":
    names, errs = check_file(sys.argv[1])
    print(f"{len(names)} kernels checked, {len(errs)} violations")
    for e in errs[:20]:
        print(" ", e)
    sys.exit(1 if errs or not names else 0)
