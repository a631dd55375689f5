"""Build-time check of the GEMM's gfx950 assembly.

The MN-major operand fragments are read with inline-asm ds_read_b64_tr_b16,
which the compiler does not track as pending LDS loads. This script verifies,
for every GEMM variant, that on every control-flow path no instruction reads
or writes a destination register of such a read before an s_waitcnt that
drains LDS operations (lgkmcnt(0)). It runs a forward dataflow over the
kernel's basic blocks (union of pending registers at joins).

Usage: python check_isa.py <gemm.s>   (exit status 1 on a violation)
"""
import re
import sys


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


def transfer(instrs, pending, name, errors):
    pending = set(pending)
    for line in instrs:
        op, args = parse(line)
        if op == "s_waitcnt" and "lgkmcnt(0)" in line:
            pending.clear()
            continue
        if op.startswith("s_"):
            continue
        regs = set()
        for a in args:
            regs |= reg_set(a)
        if op == "ds_read_b64_tr_b16":
            dst = reg_set(args[0])
            if dst & pending:
                errors.add(f"{name}: tr read overwrites a pending destination: {line}")
            if reg_set(args[1]) & pending:
                errors.add(f"{name}: tr read address is a pending register: {line}")
            pending |= dst
            continue
        if regs & pending:
            errors.add(f"{name}: '{line}' touches {sorted(regs & pending)} before lgkmcnt(0)")
    return pending


warnings = set()


def check(path):
    text = open(path).read()
    errors = set()
    for fn in re.split(r"\n(?=_Z\w+:)", text):
        name = fn.split(":")[0]
        if "gemm_kernel" not in name:
            continue
        end = fn.find("s_endpgm")
        body = fn[: fn.find("\n", end) if end >= 0 else len(fn)]
        if re.search(r"scratch_(load|store)", body):
            warnings.add(f"{name}: spills to scratch (outside the hazard rule; check the loop)")
        blocks = blocks_of(body.split("\n")[1:])
        index = {b[0]: k for k, b in enumerate(blocks)}
        entry = {k: set() for k in range(len(blocks))}
        work = list(range(len(blocks)))
        seen_out = {}
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
                merged = entry[j] | out
                if merged != entry[j] or j not in seen_out:
                    entry[j] = merged
                    if j not in work:
                        work.append(j)
    return sorted(errors)


if __name__ == "__main__":
    errs = check(sys.argv[1])
    for w in sorted(warnings):
        print("warning:", w)
    for e in errs[:20]:
        print(e)
    print(f"check_isa: {len(errs)} violation(s)")
    sys.exit(1 if errs else 0)
