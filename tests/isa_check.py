"""Static checks of a gfx950 kernel's main loop, from the compiler's assembly output.

Used by test_gemm_schedule.py on the fused GEMM, whose main loop is a hand-ordered inline-asm
schedule.  The compiler cannot see the latency of asm LDS loads, so two rules are checked
over three passes of the loop body (the state carries across the back edge):
  - no instruction reads or overwrites a register that an LDS load still in flight will
    write (LDS loads complete in issue order: s_waitcnt lgkmcnt(n) retires all but the n
    most recent).  A d16 load that preserves half of its destination reads that register
    at issue, so a d16 merge into a register with a load still in flight is flagged too;
  - an MFMA does not read a register written by a VALU instruction fewer than 3 wait states
    earlier (s_nop n counts n+1).
"""
import re


def regs(tok):
    tok = tok.strip().rstrip(',')
    m = re.fullmatch(r'([va])\[(\d+):(\d+)\]', tok)
    if m:
        return {f"{m.group(1)}{i}" for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    if re.fullmatch(r'[va]\d+', tok):
        return {tok}
    return set()


def parse(lines):
    out = []
    for ln in lines:
        s = ln.split(';')[0].strip()
        if not s or s.endswith(':') or s.startswith('.'):
            continue
        parts = s.split(None, 1)
        ops = [o.strip() for o in parts[1].split(',')] if len(parts) > 1 else []
        out.append((parts[0], ops, s))
    return out


def classify(op, ops):
    """(kind, destination registers, source registers)"""
    def srcs(items):
        out = set()
        for o in items:
            out |= regs(o.split()[0])
        return out
    if op.startswith('ds_read') or op.startswith('ds_load'):
        d = regs(ops[0])
        s = regs(ops[1].split()[0]) if len(ops) > 1 else set()
        if 'd16' in op:
            s |= d
        return 'lds_load', d, s
    if op.startswith('ds_write') or op.startswith('ds_store'):
        return 'lds_store', set(), srcs(ops)
    if op.startswith('buffer_load') or op.startswith('global_load'):
        if ops and (ops[-1].endswith('lds') or ' lds' in ' '.join(ops)):
            return 'lds_dma', set(), regs(ops[0])
        return 'vmem_load', regs(ops[0]), srcs(ops[1:])
    if op.startswith('v_mfma'):
        return 'mfma', regs(ops[0]), regs(ops[1]) | regs(ops[2]) | regs(ops[3].split()[0])
    if op.startswith('v_'):
        return 'valu', (regs(ops[0]) if ops else set()), srcs(ops[1:])
    if op == 's_waitcnt':
        return 'wait', set(), set()
    if op == 's_nop':
        return 'nop', set(), set()
    return 'salu', set(), set()


def check_body(body, passes=3):
    lds_q, vm_q = [], []
    last_valu = {}
    clock = 0
    errors = []
    for p in range(passes):
        for idx, (op, ops, text) in enumerate(body):
            kind, dst, src = classify(op, ops)
            if kind == 'wait':
                m = re.search(r'lgkmcnt\((\d+)\)', text)
                if m:
                    del lds_q[:max(0, len(lds_q) - int(m.group(1)))]
                m = re.search(r'vmcnt\((\d+)\)', text)
                if m:
                    del vm_q[:max(0, len(vm_q) - int(m.group(1)))]
                clock += 1
                continue
            if kind == 'nop':
                clock += (int(ops[0], 0) + 1) if ops else 1
                continue
            pend = set().union(*lds_q) if lds_q else set()
            vpend = set().union(*vm_q) if vm_q else set()
            if kind == 'lds_load':
                # a plain load may be issued over a register an older LDS load still writes
                # (in-order completion); a d16 merge reads its destination at issue
                bad = (src & pend) | (dst & vpend)
            else:
                bad = (src | dst) & (pend | vpend)
            if bad and p > 0:
                errors.append(f"pass {p} #{idx}: {text}: register in flight {sorted(bad)[:4]}")
            if kind == 'mfma' and p > 0:
                for r in src:
                    if r in last_valu and clock - last_valu[r] < 3:
                        errors.append(f"pass {p} #{idx}: {text}: reads {r} {clock - last_valu[r]} states after a VALU write")
            if kind == 'valu':
                for r in dst:
                    last_valu[r] = clock
            if kind == 'lds_load':
                lds_q.append(dst)
            if kind == 'vmem_load':
                vm_q.append(dst)
            clock += 1
    return errors


def mfma_loops(asm_text):
    """Bodies of every loop that contains MFMAs (one per kernel instantiation), parsed."""
    lines = asm_text.splitlines()
    out = []
    for s, line in enumerate(lines):
        if 'Loop Header' not in line:
            continue
        e = next(i for i in range(s + 1, len(lines)) if re.search(r's_cbranch_scc|s_cbranch_vcc', lines[i]))
        if any('v_mfma' in x for x in lines[s:e]):
            out.append(parse(lines[s + 1:e]))
    return out


def mfma_loop(asm_text):
    """Body of the first loop that contains MFMAs, as parsed instructions."""
    loops = mfma_loops(asm_text)
    return loops[0] if loops else []


def census(body):
    kinds = {}
    for op, ops, _ in body:
        k = classify(op, ops)[0]
        kinds[k] = kinds.get(k, 0) + 1
    return kinds
