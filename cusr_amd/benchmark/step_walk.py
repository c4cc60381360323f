"""Instruction counts of one interpreter step, walked through a kernel's assembly.

The fit kernels interpret a decoded program one instruction word per step; every
branch of a step depends on fields of that word (a scalar load), so the path a
word takes through the code object is fixed by the word. This walks it
symbolically: starting at the interpreter loop's header with the word in the
scalar registers the `s_load_dwordx2` writes, it executes the scalar ALU
instructions and branches on known values and counts every instruction up to
the loop's back edge. Vector compares (the data-dependent selects of the
elementary functions) take a value from a policy (default: no lane set, the
ordinary-argument path).

    hipcc -O3 -std=c++17 --offload-arch=gfx950 -ffp-contract=off -fno-fast-math \\
        -Xclang -target-feature -Xclang -packed-fp32-ops \\
        -mllvm -structurizecfg-skip-uniform-regions=1 -Iinclude -x hip \\
        -DCUSR_FIT_R=double -DCUSR_FIT_AD=0 -DCUSR_FIT_LAUNCH=launch_fit_f64_fwd \\
        -DCUSR_PASS_LAUNCH=launch_pass_f64_fwd --cuda-device-only -S \\
        cusr_amd/csrc/fit_kernels.hip -o /tmp/fwd.s
    python -m cusr_amd.benchmark.step_walk /tmp/fwd.s \\
        --kernel '_ZN4cusr13lm_fit_kernelILi7EdLi0ELi0EEEvNS_7FitArgsE' \\
        --head .LBB15_1231 --regs '{"s62": 0, "s63": 0, "s85": 100, "s70": 0}'

--head is the loop header block of the interpreter (the block holding the
`s_load_dwordx2` of the instruction word: the first `This Loop Header` of the
LM loop's pass); --regs gives the scalar registers the loop keeps (the program
counter and its high word, the instruction count, a zero register) so the walk
takes the back edge. Each operator is walked with the word of program.h's fast
format that the default cases build (operand kinds, ranks and scale flags).
The walk stops at the next `s_load` of the header; a branch on an unknown
value is reported and falls through.
"""
from __future__ import annotations

import argparse
import json
import re
import struct
from collections import Counter

M32 = 0xFFFFFFFF
M64 = (1 << 64) - 1

ACC, VAR, CONST, SLOT = 0, 1, 2, 3


def word(fid, binary=0, ak=ACC, ai=0, bk=ACC, bi=0, toslot=0, didx=0, lo=0, mid=0, hi=0,
         sel=0, sa=0, sb=0, tape=0, ta=0, tb=0):
    """A fast-format instruction word (cusr_amd/csrc/program.h bit layout)."""
    return (fid | binary << 6 | ak << 7 | ai << 9 | bk << 13 | bi << 15 | toslot << 19 |
            didx << 20 | lo << 24 | mid << 29 | hi << 34 | tape << 39 | sel << 47 | sa << 48 |
            sb << 49 | ta << 50 | tb << 51)


# operator steps of the C2 mix: (name, word)
CASES = [
    ("ADD acc,const", word(1, 1, ACC, 0, CONST, 3, lo=0, mid=2, hi=3)),
    ("SUB acc,var", word(2, 1, ACC, 0, VAR, 0, lo=0, mid=3, hi=3)),
    ("MUL acc,const, both scaled", word(3, 1, ACC, 0, CONST, 4, lo=0, mid=4, hi=5, sa=1, sb=1)),
    ("MUL slot,acc, both scaled", word(3, 1, SLOT, 0, ACC, 0, lo=0, mid=3, hi=7, sa=1, sb=1)),
    ("PDIV acc,var, left scaled", word(32, 1, ACC, 0, VAR, 0, lo=0, mid=4, hi=4, sa=1, sel=1)),
    ("SIN acc, scaled", word(14, 0, ACC, 0, lo=0, mid=5, hi=5, sa=1)),
    ("COS acc, scaled", word(15, 0, ACC, 0, lo=0, mid=5, hi=5, sa=1)),
    ("CEXP acc, scaled", word(33, 0, ACC, 0, lo=0, mid=5, hi=5, sa=1, sel=1)),
    ("PLOG acc, scaled", word(35, 0, ACC, 0, lo=0, mid=5, hi=5, sa=1)),
    ("LOOSE_SQRT acc, scaled", word(28, 0, ACC, 0, lo=0, mid=5, hi=5, sa=1)),
    ("SQUARE acc, scaled", word(34, 0, ACC, 0, lo=0, mid=5, hi=5, sa=1)),
]


def parse(path, kernel):
    """{block label: [instructions]}, labels in order, for one kernel's body."""
    lines = open(path).read().splitlines()
    start = next(i for i, ln in enumerate(lines) if ln.startswith(kernel + ":"))
    end = next((i for i in range(start + 1, len(lines)) if re.match(r"^_Z\w+:", lines[i])),
               len(lines))
    blocks, order, cur = {}, [], None
    for ln in lines[start:end]:
        m = re.match(r"^\s*(\.L[\w.]+):", ln) or re.match(r"^; (%bb\.\d+):", ln)
        if m:
            cur = m.group(1)
            blocks[cur] = []
            order.append(cur)
            continue
        t = ln.strip()
        if cur is not None and re.match(r"^(?:[sv]_|ds_|global_|buffer_|scratch_|flat_)", t):
            blocks[cur].append(t.split(";")[0].strip())
    return blocks, order


def _sx(v, bits):
    v &= (1 << bits) - 1
    return v - (1 << bits) if v >> (bits - 1) else v


class _Machine:
    def __init__(self, regs):
        self.r = dict(regs)
        self.scc = None
        self.exec_ = M64

    def get(self, op):
        op = op.strip().rstrip(",")
        if op == "exec":
            return self.exec_
        if op == "vcc":
            return self.r.get("vcc")
        m = re.match(r"^s\[(\d+):(\d+)\]$", op)
        if m:
            lo, hi = self.r.get(f"s{m.group(1)}"), self.r.get(f"s{m.group(2)}")
            return None if lo is None or hi is None else lo | hi << 32
        if re.match(r"^s\d+$", op):
            return self.r.get(op)
        try:
            return int(op, 0) & M64
        except ValueError:
            pass
        try:
            return struct.unpack("<Q", struct.pack("<d", float(op)))[0]
        except ValueError:
            return None

    def set(self, op, v, wide):
        op = op.strip().rstrip(",")
        if op == "exec":
            self.exec_ = M64 if v is None else v
            return
        if op == "vcc":
            self.r["vcc"] = v
            return
        m = re.match(r"^s\[(\d+):(\d+)\]$", op)
        if m:
            a = int(m.group(1))
            for k, part in ((a, None if v is None else v & M32),
                            (a + 1, None if v is None else (v >> 32) & M32)):
                if part is None:
                    self.r.pop(f"s{k}", None)
                else:
                    self.r[f"s{k}"] = part
            return
        if v is None:
            self.r.pop(op, None)
        else:
            self.r[op] = v & (M64 if wide else M32)


def _kind(op):
    if op.startswith("v_"):
        return "valu"
    if op.startswith("ds_"):
        return "lds"
    if op.split("_")[0] in ("global", "buffer", "scratch", "flat"):
        return "vmem"
    if op.startswith("s_load") or op.startswith("s_buffer_load"):
        return "smem"
    if op.startswith("s_cbranch") or op in ("s_branch", "s_setpc_b64"):
        return "branch"
    if op == "s_nop" or op.startswith("s_waitcnt"):
        return "wait/nop"
    return "salu"


def _salu(m, op, a):
    """Execute one scalar instruction (unknown results clear the target)."""
    wide = op.endswith("64")
    bits = 64 if wide else 32
    mask = M64 if wide else M32
    if op in ("s_mov_b32", "s_movk_i32", "s_mov_b64"):
        m.set(a[0], m.get(a[1]), wide)
    elif op in ("s_cselect_b32", "s_cselect_b64"):
        m.set(a[0], None if m.scc is None else m.get(a[1] if m.scc else a[2]), wide)
    elif op in ("s_bfe_u32", "s_bfe_i32", "s_bfe_u64"):
        v, c = m.get(a[1]), m.get(a[2])
        if v is None or c is None:
            m.set(a[0], None, wide)
            m.scc = None
            return
        off, w = c & 63, (c >> 16) & 127
        r = (v >> off) & ((1 << w) - 1)
        if op == "s_bfe_i32" and w:
            r = _sx(r, w) & M32
        m.set(a[0], r, wide)
        m.scc = int(r != 0)
    elif op.split("_")[1] in ("and", "or", "xor", "andn2", "orn2", "nand", "nor") and \
            not op.endswith("saveexec_b64"):
        x, y = m.get(a[1]), m.get(a[2])
        if x is None or y is None:
            m.set(a[0], None, wide)
            m.scc = None
            return
        f = op.split("_")[1]
        r = {"and": x & y, "or": x | y, "xor": x ^ y, "andn2": x & ~y, "orn2": x | ~y,
             "nand": ~(x & y), "nor": ~(x | y)}[f] & mask
        m.set(a[0], r, wide)
        m.scc = int(r != 0)
    elif op in ("s_lshl_b32", "s_lshr_b32", "s_ashr_i32", "s_lshl_b64", "s_lshr_b64",
                "s_ashr_i64"):
        x, y = m.get(a[1]), m.get(a[2])
        if x is None or y is None:
            m.set(a[0], None, wide)
            m.scc = None
            return
        y &= bits - 1
        r = (x << y) & mask if "lshl" in op else x >> y if "lshr" in op else \
            (_sx(x, bits) >> y) & mask
        m.set(a[0], r, wide)
        m.scc = int(r != 0)
    elif op in ("s_add_u32", "s_add_i32", "s_sub_u32", "s_sub_i32", "s_addc_u32",
                "s_mul_i32"):
        x, y = m.get(a[1]), m.get(a[2])
        if x is None or y is None:
            m.set(a[0], None, False)
            m.scc = None
            return
        if op == "s_addc_u32":
            r = x + y + (m.scc or 0)
        elif op.startswith("s_add"):
            r = x + y
        elif op.startswith("s_sub"):
            r = x - y
        else:
            r = _sx(x, 32) * _sx(y, 32)
        m.scc = int(r > M32 or r < 0) if op in ("s_add_u32", "s_addc_u32", "s_sub_u32") \
            else None
        m.set(a[0], r & M32, False)
    elif op.startswith("s_cmp_") or op.startswith("s_cmpk_"):
        x, y = m.get(a[0]), m.get(a[1])
        if x is None or y is None:
            m.scc = None
            return
        cond, ty = op.split("_")[2], op.split("_")[3]
        if ty.startswith("i"):
            x, y = _sx(x, 32), _sx(y, 32)
        m.scc = int({"eq": x == y, "lg": x != y, "lt": x < y, "le": x <= y, "gt": x > y,
                     "ge": x >= y}[cond])
    elif op.startswith("s_bitcmp"):
        x, y = m.get(a[0]), m.get(a[1])
        if x is None or y is None:
            m.scc = None
            return
        m.scc = int(((x >> (y & 63)) & 1) == int(op[8]))
    elif op.endswith("saveexec_b64"):
        x = m.get(a[1])
        old = m.exec_
        m.set(a[0], old, True)
        if x is None:
            m.exec_ = M64
            m.scc = None
            return
        m.exec_ = {"s_and_saveexec_b64": old & x, "s_or_saveexec_b64": old | x,
                   "s_andn2_saveexec_b64": x & ~old}.get(op, M64) & M64
        m.scc = int(m.exec_ != 0)
    elif a:
        m.set(a[0], None, wide)
        m.scc = None


def walk(blocks, order, head, w, regs, vcmp=0, max_instr=20000):
    """Counts per instruction kind of one step of word w from block head."""
    m = _Machine(regs)
    cnt, unknown = Counter(), []
    b, i, loaded = head, 0, False
    for _ in range(max_instr):
        ins = blocks[b]
        if i >= len(ins):
            b, i = order[order.index(b) + 1], 0
            continue
        t = ins[i]
        i += 1
        op = t.split()[0]
        a = [x.strip() for x in t[len(op):].split(",")] if len(t) > len(op) else []
        if op.startswith("s_load_dwordx2") and not loaded:
            m.set(a[0], w, True)
            loaded = True
            cnt["smem"] += 1
            continue
        if op.startswith("s_load") and loaded and b == head:
            break
        k = _kind(op)
        cnt[k] += 1
        if op.startswith("v_cmp"):
            if a and (a[0] == "vcc" or a[0].startswith("s")):
                m.set(a[0], M64 if vcmp else 0, True)
            continue
        if op in ("v_readfirstlane_b32", "v_readlane_b32"):
            m.set(a[0], None, False)
            continue
        if k == "salu":
            _salu(m, op, a)
            continue
        if k != "branch":
            continue
        target = None
        if op in ("s_cbranch_scc0", "s_cbranch_scc1"):
            if m.scc is None:
                unknown.append(t)
            elif m.scc == int(op[-1]):
                target = a[0]
        elif op in ("s_cbranch_vccz", "s_cbranch_vccnz"):
            v = m.r.get("vcc")
            if v is None:
                unknown.append(t)
            elif ((v & m.exec_) == 0) == (op == "s_cbranch_vccz"):
                target = a[0]
        elif op in ("s_cbranch_execz", "s_cbranch_execnz"):
            if (m.exec_ == 0) == (op == "s_cbranch_execz"):
                target = a[0]
        elif op == "s_branch":
            target = a[0]
        if target is not None:
            b, i = target, 0
    return cnt, unknown


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("asm")
    ap.add_argument("--kernel", required=True, help="the kernel's mangled symbol")
    ap.add_argument("--head", required=True, help="the interpreter loop's header block")
    ap.add_argument("--regs", default="{}", help="JSON: known scalar registers")
    ap.add_argument("--vcmp", type=int, default=0, help="value of every vector compare")
    a = ap.parse_args()
    blocks, order = parse(a.asm, a.kernel)
    print("| step | VALU | SALU | branch | LDS | SMEM | unknown branches |")
    print("|---|---|---|---|---|---|---|")
    for name, w in CASES:
        c, u = walk(blocks, order, a.head, w, json.loads(a.regs), a.vcmp)
        print(f"| {name} | {c['valu']} | {c['salu']} | {c['branch']} | {c['lds']} | "
              f"{c['smem']} | {len(u)} |")


if __name__ == "__main__":
    main()
