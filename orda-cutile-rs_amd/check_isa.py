"""Build-time check of the GEMM's gfx950 assembly.

The bf16 GEMM kernels issue their MFMAs as inline asm (accumulators tied to
AGPRs), so the compiler's hazard recognizer does not see them and the kernel
inserts the required wait states itself. This script verifies, on every
control-flow path of every bf16 GEMM variant, that
  * no non-MFMA instruction reads or writes an MFMA result register within
    MFMA_RESULT_WAIT wait states of the MFMA that wrote it, and no MFMA reads
    it as an operand that soon either;
  * no MFMA reads (as A, B or C) a register that a VALU instruction wrote
    within VALU_TO_MFMA_WAIT wait states.
Every instruction counts as one wait state and `s_nop N` as N + 1. The
analysis is a forward dataflow over the kernel's basic blocks keeping, per
register, the fewest wait states since the last such write on any path.
It also reports (as warnings) variants that spill to scratch.

Usage: python check_isa.py <gemm.s>   (exit status 1 on a violation)
"""
import re
import sys

MFMA_RESULT_WAIT = 19     # a 16-pass XDL result is readable 18 wait states later
VALU_TO_MFMA_WAIT = 4     # VALU write -> MFMA operand read needs 2; keep margin
CAP = 64                  # distances at or above every threshold


def reg_set(tok):
    """Registers named by one operand token, e.g. v[10:11] -> {v10, v11}."""
    m = re.fullmatch(r"([va])\[(\d+):(\d+)\]", tok)
    if m:
        return {f"{m.group(1)}{i}" for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.fullmatch(r"([va])(\d+)", tok)
    return {tok} if m else set()


def parse(line):
    body = line.split(";")[0].strip()
    parts = body.split(None, 1)
    if not parts:
        return "", []
    args = [t.strip() for t in parts[1].split(",")] if len(parts) > 1 else []
    return parts[0], args


def blocks_of(fn_lines):
    """[(label, [instr lines])] in text order; the entry block is labelled ''."""
    blocks = [["", []]]
    for raw in fn_lines:
        line = raw.strip()
        if not line or line.startswith(";") or line.startswith("."):
            m = re.match(r"^(\.LBB\d+_\d+):", line)
            if m:
                blocks.append([m.group(1), []])
            continue
        if line.endswith(":"):
            continue
        blocks[-1][1].append(line)
    return blocks


def successors(blocks, i):
    instrs = blocks[i][1]
    last = parse(instrs[-1])[0] if instrs else ""
    nxt = [blocks[i + 1][0]] if i + 1 < len(blocks) else []
    targets = []
    for ins in instrs:
        op, args = parse(ins)
        if op.startswith("s_cbranch") or op == "s_branch":
            targets.append(args[0])
    if last in ("s_branch", "s_endpgm", "s_setpc_b64"):
        return targets          # no fall-through
    return targets + nxt


def advance(state, n):
    return {r: d + n for r, d in state.items() if d + n < CAP}


def transfer(instrs, entry, name, errors):
    """entry: (mfma_dist, valu_dist) dicts register -> wait states since write."""
    mf, va = dict(entry[0]), dict(entry[1])
    for line in instrs:
        op, args = parse(line)
        if op == "s_nop":
            n = int(args[0], 0) + 1
            mf, va = advance(mf, n), advance(va, n)
            continue
        regs = [reg_set(a) for a in args]
        if op.startswith("v_mfma"):
            srcs = set().union(*regs[1:4]) if len(regs) >= 4 else set()
            for r in srcs:
                if r in mf and mf[r] < MFMA_RESULT_WAIT:
                    errors.add(f"{name}: '{line}' reads {r} {mf[r]} wait states after an MFMA wrote it")
                if r in va and va[r] < VALU_TO_MFMA_WAIT:
                    errors.add(f"{name}: '{line}' reads {r} {va[r]} wait states after a VALU wrote it")
            mf, va = advance(mf, 1), advance(va, 1)
            for r in regs[0]:
                mf[r] = 0
                va.pop(r, None)
            continue
        touched = set().union(*regs) if regs else set()
        for r in touched:
            if r in mf and mf[r] < MFMA_RESULT_WAIT:
                errors.add(f"{name}: '{line}' touches {r} {mf[r]} wait states after an MFMA wrote it")
        mf, va = advance(mf, 1), advance(va, 1)
        if op.startswith("v_") and regs:
            for r in regs[0]:
                va[r] = 0
                mf.pop(r, None)
        elif regs and (op.startswith("ds_read") or op.startswith("global_load")
                       or op.startswith("buffer_load") or op.startswith("scratch_load")):
            for r in regs[0]:
                mf.pop(r, None)
                va.pop(r, None)
    return mf, va


def merge(a, b):
    out = dict(a)
    for r, d in b.items():
        out[r] = min(d, out.get(r, CAP))
    return out


warnings = set()


def check(path):
    text = open(path).read()
    errors = set()
    checked = 0
    for fn in re.split(r"\n(?=_Z\w+:)", text):
        name = fn.split(":")[0]
        if not re.search(r"gemm_(kk|km|kmt)_(logits|logits_pre|logits_pre16|store|accum)_bf16", name):
            continue
        checked += 1
        end = fn.find("s_endpgm")
        body = fn[: fn.find("\n", end) if end >= 0 else len(fn)]
        if re.search(r"scratch_(load|store)", body):
            warnings.add(f"{name}: spills to scratch")
        blocks = blocks_of(body.split("\n")[1:])
        index = {b[0]: k for k, b in enumerate(blocks)}
        entry = {k: ({}, {}) for k in range(len(blocks))}
        seen_out = {}
        work = list(range(len(blocks)))
        while work:
            k = work.pop(0)
            out = transfer(blocks[k][1], entry[k], name, errors)
            if seen_out.get(k) == out:
                continue
            seen_out[k] = out
            for s in successors(blocks, k):
                j = index.get(s)
                if j is None:
                    continue
                merged = (merge(entry[j][0], out[0]), merge(entry[j][1], out[1]))
                if merged != entry[j] or j not in seen_out:
                    entry[j] = merged
                    if j not in work:
                        work.append(j)
    if checked < 8:
        errors.add(f"expected the 8 bf16 GEMM variants, found {checked}")
    return sorted(errors)


if __name__ == "__main__":
    errs = check(sys.argv[1])
    for w in sorted(warnings):
        print("warning:", w)
    for e in errs[:20]:
        print(e)
    print(f"check_isa: {len(errs)} violation(s)")
    sys.exit(1 if errs else 0)
