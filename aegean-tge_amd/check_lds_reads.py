"""Check of the attention kernels' untracked LDS reads in the gfx950 assembly.

The page-pair paths read V operands with inline-asm ``ds_read_b64``
(attn_common.h ``lds_read_b64``) and wait for them with an inline-asm
``s_waitcnt lgkmcnt(0)`` (``lds_wait_operands``). The compiler does not know
that such a read's destination registers are written only when the read
returns, so it may copy or reuse them before the wait; a copy made there
reads stale values. This scans the device assembly of every
paged_{decode,prefill,mixed}_kernel and reports any instruction that reads
or writes a register of an inline-asm ``ds_read_b64`` before the next
``lgkmcnt(0)`` wait in layout order (a linear scan: it follows fall-through
order, not every branch, which is where the compiler places such copies).

Usage (about five minutes: one device-only compile of the attention TU):
    make asm-check
or, with an assembly file made by hipcc --cuda-device-only -S:
    python3 check_lds_reads.py _build/paged_attention.s
Exit status 1 when a violation is found.
"""
import re
import sys

KERNEL = re.compile(r"^(_Z\S*paged_(?:prefill|mixed|decode)_kernel\S*):")


def vregs(token):
    """VGPR numbers named by an operand (v7, v[4:7]); empty for others."""
    m = re.match(r"v\[(\d+):(\d+)\]", token)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", token)
    return {int(m.group(1))} if m else set()


def scan(lines):
    """Violations in one kernel's lines: (line index, text, registers)."""
    pending = {}  # VGPR -> index of the untracked read that writes it
    in_asm = False
    found = []
    for i, line in enumerate(lines):
        s = line.strip()
        if s.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if s.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if not s or s.startswith((";", ".")) or s.endswith(":"):
            continue
        op, _, rest = s.partition(" ")
        args = [a.strip() for a in rest.split(",")] if rest else []
        if op == "s_waitcnt" and "lgkmcnt(0)" in s:
            pending.clear()
            continue
        if in_asm and op == "ds_read_b64" and args:
            for r in vregs(args[0]):
                pending[r] = i
            continue
        if not pending or not args:
            continue
        # the first operand of a vector instruction is its destination
        writes = set() if op.startswith(("s_", "ds_write", "buffer_store", "global_store")) \
            else vregs(args[0])
        reads = set()
        for a in (args[1:] if writes else args):
            reads |= vregs(a.split()[0])
        hit = (reads | writes) & set(pending)
        if hit:
            found.append((i, s, sorted(hit)))
    return found


def main(path):
    text = open(path).read().split("\n")
    kernels = 0
    bad = 0
    i = 0
    while i < len(text):
        m = KERNEL.match(text[i])
        if not m:
            i += 1
            continue
        end = i
        while end < len(text) and not text[end].startswith("\t.size"):
            end += 1
        kernels += 1
        for j, s, regs in scan(text[i:end]):
            bad += 1
            if bad <= 10:
                print(f"{m.group(1)[:80]}: +{j}: {s}  (registers {regs[:4]} of a pending read)")
        i = end
    print(f"{kernels} kernels, {bad} violations")
    return 1 if bad or kernels == 0 else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1] if len(sys.argv) > 1 else "_build/paged_attention.s"))
