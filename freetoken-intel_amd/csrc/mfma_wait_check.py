#!/usr/bin/env python3
"""Build check over the gfx950 assembly of this library's own kernels.

The gfx950 compiler in ROCm 7.2 inserts the wait states between an MFMA and a
VALU instruction that reads its result when both sit in one basic block, but
on a path that leaves the block through a taken branch it has emitted the read
one instruction after the MFMA.  The read then returns the accumulator from
before the MFMA (seen on hardware as whole rows of a GEMM tile missing the last
K slice).  The kernels are written to keep such reads in the MFMA's own block;
this script makes the build fail if any kernel breaks that rule.

For every MFMA it walks all control-flow paths forward and reports a non-MFMA
instruction that reads the MFMA's destination registers fewer than ``--need``
wait states later, counting one state per instruction and N+1 per
``s_nop N``.  The default of 8 is what the compiler itself places in-block for
the 16x16x32 bf16 MFMA used here.  It also reports a VALU write that an MFMA
reads across a block boundary within 3 states.

Usage: mfma_wait_check.py [--need N] file.s [file.s ...]   (exit 1 on findings)
"""
from __future__ import annotations

import re
import sys

_FUNC = re.compile(r"\n(_Z\w+):[^\n]*\n(.*?)\.Lfunc_end", re.S)
_RANGE = re.compile(r"([av])\[(\d+):(\d+)\]")
_SINGLE = re.compile(r"([av])(\d+)$")
_CBRANCH = ("s_cbranch_scc0", "s_cbranch_scc1", "s_cbranch_vccz", "s_cbranch_vccnz",
            "s_cbranch_execz", "s_cbranch_execnz")


def _regs(tok: str) -> set:
    m = _RANGE.match(tok)
    if m:
        return {f"{m.group(1)}{i}" for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    return {tok} if _SINGLE.match(tok) else set()


def _parse(body: str):
    insts, labels = [], {}
    for raw in body.split("\n"):
        ln = raw.split(";")[0].strip()
        if not ln:
            continue
        if ln.endswith(":"):
            labels[ln[:-1]] = len(insts)
            insts.append(("LABEL", ln[:-1], []))
            continue
        if ln.startswith("."):
            continue
        parts = ln.replace(",", " ").split()
        insts.append((parts[0], ln, parts[1:]))
    return insts, labels


def _states(op: str, args) -> int:
    return int(args[0]) + 1 if op == "s_nop" else 1


def _src_regs(op: str, args) -> set:
    out = set()
    srcs = args if op.startswith(("buffer_store", "global_store", "ds_write", "ds_store")) else args[1:]
    for a in srcs:
        out |= _regs(a)
    return out


def _late_reads(insts, labels, pc, dst, left, seen, path):
    """Non-MFMA readers of ``dst`` reached with ``left`` > 0 states remaining."""
    hits = []
    while pc < len(insts) and left > 0:
        op, txt, args = insts[pc]
        if op == "LABEL":
            pc += 1
            continue
        if op.startswith("v_mfma"):
            left -= 1
            pc += 1
            continue
        if not op.startswith("s_") and _src_regs(op, args) & dst:
            hits.append((path, txt, left))
            return hits
        if op in _CBRANCH:
            key = (args[0], left)
            if key not in seen:
                seen.add(key)
                hits += _late_reads(insts, labels, labels[args[0]], dst, left - 1, seen, path + [args[0]])
        elif op == "s_branch":
            key = (args[0], left)
            if key in seen:
                return hits
            seen.add(key)
            pc, left, path = labels[args[0]], left - 1, path + [args[0]]
            continue
        elif op == "s_endpgm":
            return hits
        left -= _states(op, args)
        pc += 1
    return hits


def _early_mfma_reads(insts, labels, i, dst):
    """MFMAs reading ``dst`` within 3 states of its VALU write, across a block boundary."""
    hits, stack, seen = [], [(i + 1, 3, False)], set()
    while stack:
        pc, left, crossed = stack.pop()
        while pc < len(insts) and left > 0:
            op, txt, args = insts[pc]
            if op == "LABEL":
                crossed = True
                pc += 1
                continue
            if op.startswith("v_mfma"):
                if crossed and _src_regs(op, args) & dst:
                    hits.append(txt)
                left -= 1
                pc += 1
                continue
            if op in _CBRANCH and args[0] not in seen:
                seen.add(args[0])
                stack.append((labels[args[0]], left - 1, True))
            if op == "s_branch":
                pc, left, crossed = labels[args[0]], left - 1, True
                continue
            if op == "s_endpgm":
                break
            left -= _states(op, args)
            pc += 1
    return hits


def check(path: str, need: int) -> list:
    findings = []
    src = open(path).read()
    for name, body in _FUNC.findall(src):
        insts, labels = _parse(body)
        for i, (op, txt, args) in enumerate(insts):
            if not args:
                continue
            if op.startswith("v_mfma"):
                for p, reader, left in _late_reads(insts, labels, i + 1, _regs(args[0]), need, set(), []):
                    findings.append(f"{path}: {name}: '{txt}' read {need - left} states later "
                                    f"via {p or 'fallthrough'} by '{reader}'")
            elif op.startswith("v_"):
                dst = _regs(args[0])
                if dst:
                    for reader in _early_mfma_reads(insts, labels, i, dst):
                        findings.append(f"{path}: {name}: '{txt}' read across a branch by '{reader}'")
    return findings


def main(argv) -> int:
    need = 8
    files = []
    it = iter(argv)
    for a in it:
        if a == "--need":
            need = int(next(it))
        else:
            files.append(a)
    findings = [f for p in files for f in check(p, need)]
    for f in findings:
        print(f)
    if findings:
        print(f"mfma_wait_check: {len(findings)} MFMA result(s) read too early; "
              "keep MFMA consumers in the MFMA's basic block", file=sys.stderr)
        return 1
    print(f"mfma_wait_check: {len(files)} file(s) clean")
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
