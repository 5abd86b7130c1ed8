"""Generate hif8_gemm_schedule.inc and hif8_gemm_schedule_w16.inc: the phase bodies of the
main loops of the fused GEMM (hif8_gemm_dtl.hip) and of its decode-free twin
(hif8_gemm_w16.hip).

A k-step (64 k) is two phases of 32 k.  A phase issues the wave's 64 MFMAs
(v_mfma_f32_16x16x32_bf16, 16 cycles each) and, in the gaps between them, what the NEXT phase
needs.  Gap g holds the ops issued right after MFMA g; ("pre", n) holds ops issued right before
MFMA n.  Between two 16-cycle MFMAs a wave has three more issue slots.  LDS operations complete
in order, so lgkmcnt(n) means "all but the n most recent LDS operations are done".

    python3 gen_gemm_schedule.py [out.inc [out_w16.inc]]
        (defaults: hif8_gemm_schedule.inc, hif8_gemm_schedule_w16.inc)
"""
import os
import sys

# ---------------------------------------------------------------------------------------------
# The fused GEMM (hif8_gemm_dtl.hip).  Wave w owns output features 64w .. +63 for all 256 rows:
# MFMA m of a phase is n-tile i = m / 16 (16 features) times m-tile j = m % 16 (16 rows).  For
# the next phase a phase reads its 16 X fragments (ds_read_b128) and the wave's W codes (one
# ds_read_b64 of 8 codes per n-tile and lane), looks the 32 codes of each lane up in the
# per-lane decode table (a v_perm address and a ds_read_u16 each) and packs n-tiles 0 and 1's
# looked-up values into their MFMA operands; n-tiles 2 and 3 are packed in the phase that uses
# them, before MFMA 32.  (The MFMAs go in 2 x 2 blocks of n-tiles x m-tiles, n-tiles 0 and 1 in
# the first half of the phase, 2 and 3 in the second: see mm in hif8_gemm_dtl.hip.)  Phase 1 opens with the k-step's barrier and issues the 12
# global->LDS loads of the k-step after next (into the stage the barrier freed); the next phase 0
# advances the source offsets.  Issued four gaps apart from gap 1, the last load has the rest of
# phase 1 and all of phase 0 to land (with 5 of them in phase 0, as before, the kernel ran
# 1-1.5 % slower).
#
# The ops are placed greedily, in the order below, each at the first gap from its pacing
# position on that has a free slot: fragment reads are never in adjacent gaps and loads sit
# four gaps apart (the spacing the decode-free twin measured best), so the LDS and load traffic
# is spread over the phase instead of bunched.  Waits are derived from the placement: before an
# op that consumes an LDS load, lgkmcnt(number of LDS ops issued after that load), unless an
# earlier wait already covered it (at most 15, the counter's width).

NGAPS = 64
# Non-MFMA issue slots used per gap (a load with its m0 write takes two).  A gap has room for
# three, but lab copies timed with s_memtime ran the loop at 2611 cycles per k-step with three
# and 2474 with two (MFMAs alone: 2089).
CAP = 2
DTL_GAPS = {1: tuple(range(1, 48, 4)), 0: ()}
# pacing (first gap each op may take): X fragment j at X_START + X_STEP * j; lookup LL at
# LK_START + LK_NUM * LL // LK_DEN, at least CODE_GAPS after the last code read; the packs of
# the current set's n-tile i (2, 3) from PK_CUR[i] (two gaps apart), the next set's n-tile t (0, 1)
# from PK_NEXT[t].  With the 2 x 2 MFMA order, X reads from gap 4 (was 2) and lookups 1.5 gaps
# apart (was 1.25) ran 1.2-1.9 % faster on the 14B shapes, and n-tile 3's packs from gap 0 (was
# 8) another 2-2.9 % (from gap 4 0.5-1.0 %, then from 0 1.5-1.9 %), lookups at least 8 gaps
# after the code reads (was 6) 0.5-0.9 %, and the next set's packs from gaps 48 and 40 (was 52 and
# 44) 0.2-0.9 % (A/B of builds on one box, each step at least twice).
X_START, X_STEP = 4, 3
LK_START, LK_NUM, LK_DEN = 10, 3, 2
CODE_GAPS = 8
PK_CUR = (0, 0, 0, 0)
PK_NEXT = (48, 40)


class _Op:
    def __init__(self, text, kind, cost=1, lds=False, deps=(), after=(), earliest=0, latest=NGAPS - 1, ties=()):
        self.text, self.kind, self.cost, self.lds = text, kind, cost, lds
        self.deps, self.after, self.earliest, self.latest, self.ties = list(deps), list(after), earliest, latest, ties
        self.gap = None


def schedule(phase):
    cur, nxt = phase, 1 - phase
    ns = "S" if phase == 0 else "1 - S"     # stage the next phase reads
    npar = 1 if phase == 0 else 0           # k-half (p) of the next phase
    slots = [[] for _ in range(NGAPS)]
    used = [0] * NGAPS
    b128 = [False] * NGAPS
    placed = {}

    def put(op, g):
        slots[g].append(op)
        used[g] += op.cost
        b128[g] = b128[g] or op.kind == "b128"
        op.gap = g
        placed[op.text] = op

    def place(op):
        lo = op.earliest
        for a, dist in op.after:
            lo = max(lo, placed[a].gap + dist)
        for g in range(lo, NGAPS):
            if used[g] + op.cost > CAP:
                continue
            if op.kind == "b128" and any(b128[h] for h in (g - 1, g, g + 1) if 0 <= h < NGAPS):
                continue
            if g > op.latest:
                raise RuntimeError(f"{op.text} misses gap {op.latest}")
            put(op, g)
            return
        raise RuntimeError(f"no room for {op.text}")

    for n, g in enumerate(DTL_GAPS[phase]):
        # a load that opens a group of four also writes m0 (two issue slots)
        if phase == 1:
            put(_Op(f"issue_dtl<S, {n}>(c);", "dtl", cost=2 if n % 4 == 0 else 1), g)
        else:
            n1 = len(DTL_GAPS[1]) + n
            put(_Op(f"issue_dtl<1 - S, {n1}>(c);", "dtl", cost=2 if n1 % 4 == 0 else 1), g)
    for i in (2, 3):
        for d in range(4):
            place(_Op(f"pk<{cur}, {i}, {d}>(c);", "valu", earliest=PK_CUR[i] + 2 * d, latest=30))
    codes = [f"rd_code<{ns}, {npar}, {i}>(c);" for i in range(4)]
    for t in codes:
        place(_Op(t, "b64", lds=True))
    for j in range(16):
        place(_Op(f"rd_x<{ns}, {npar}, {nxt}, {j}>(c);", "b128", lds=True, earliest=X_START + X_STEP * j))
    for ll in range(32):
        r = ll % 4
        after = [(codes[-1], CODE_GAPS)]
        if ll >= 4:   # the address slot is free once the lookup 4 before has read it
            after.append((f"lkr<{nxt}, {r}, {ll - 4}>(c);", 0))
        place(_Op(f"lka<{r}, {ll}>(c);", "valu", deps=codes, after=after, earliest=LK_START + (LK_NUM * ll) // LK_DEN,
                  ties=("tie_cd(c);",)))
        place(_Op(f"lkr<{nxt}, {r}, {ll}>(c);", "u16", lds=True, after=[(f"lka<{r}, {ll}>(c);", 1)]))
    for tt in (1, 0):
        tl = [f"lkr<{nxt}, {ll % 4}, {ll}>(c);" for ll in range(8 * tt, 8 * tt + 8)]
        for d in range(4):
            place(_Op(f"pk<{nxt}, {tt}, {d}>(c);", "valu", deps=tl, after=[(t, 4) for t in tl], earliest=PK_NEXT[tt] + d,
                      latest=NGAPS - 3, ties=(f"tie8(c.T[{nxt}][{tt}]);",)))
    if phase == 0:
        for a in range(12):
            place(_Op(f"adv<{a}>(c);", "valu", earliest=(DTL_GAPS[0][-1] + 1 if DTL_GAPS[0] else 0) + 2 * a))

    ops = {}
    pre = ["wait_lgkm<0>();"] if phase == 0 else ["wait_lgkm<0>();", "wait_vm<0>();", "barrier();"]
    ops[("pre", 0)] = pre + [f"tie_set<{cur}>(c);"]
    issued, done, index = 0, 0, {}
    for g in range(NGAPS):
        lines = []
        for op in slots[g]:
            if op.deps:
                need = max(index[d] for d in op.deps) + 1
                if need > done:
                    # lgkmcnt is a 4-bit field: waiting for at most 15 outstanding covers more
                    n = min(issued - need, 15)
                    lines.append(f"wait_lgkm<{n}>();")
                    lines += list(op.ties)
                    done = issued - n
            lines.append(op.text)
            if op.lds:
                index[op.text] = issued
                issued += 1
        ops[g] = lines
    return ops


def emit(phase):
    ops = schedule(phase)
    cur = 0 if phase == 0 else 1
    lines = [f"template <int S> __device__ __forceinline__ void phase{phase}(Ctx &c)", "{"]
    for m in range(NGAPS):
        lines += ["    " + op for op in ops.get(("pre", m), [])]
        lines.append(f"    mm<{cur}, {m}>(c);")
        lines += ["    " + op for op in ops.get(m, [])]
    lines.append("}")
    return "\n".join(lines)


def generate():
    return ("// Generated by gen_gemm_schedule.py -- do not edit.\n"
            "// Main-loop phase bodies of k_linear_dtl (hif8_gemm_dtl.hip).\n\n"
            "// global->LDS loads of a k-step issued by phase 1 (the following phase 0 issues the rest)\n"
            f"constexpr int kLoadsPhase1 = {len(DTL_GAPS[1])};\n\n"
            + emit(0) + "\n\n" + emit(1) + "\n")


# ---------------------------------------------------------------------------------------------
# The decode-free twin (hif8_gemm_w16.hip): W arrives already dequantised, as bf16 rows laid out
# in LDS exactly like X, so both operands are plain fragment reads.  Each wave owns a 128 x 128
# quadrant of the tile as 8 x 8 tiles of v_mfma_f32_16x16x32_bf16 (64 MFMAs of 16 cycles per
# 32-k phase).  LDS is a ring of five operand stages (X and W of k-step j in stages 2j and
# 2j + 1).  The even phase of k-step j (its first 32 k) reads the odd phase's 16 fragments (W 0,
# X 0..7, W 1..7 in the order the MFMAs consume them) and loads X of k-step j + 2; the odd phase
# opens with the k-step's barrier, reads the fragments of k-step j + 1's even phase and loads W
# of k-step j + 2.  Between 16-cycle MFMAs a fragment read right after another delays the MFMA
# stream by about 12 cycles and two loads two gaps apart by about 30 (lab copies timed with
# s_memtime: reads in gaps 0..15 and loads every 2-4 gaps, 2606 cycles per k-step; reads every
# other gap and loads every fourth, 2238): reads go in even gaps 4..34, loads in gaps 1, 5, .. 29.  Every phase first waits for all of its fragments (lgkmcnt(0):
# they were read at least 29 MFMAs earlier).  At the barrier every wave's reads of k-step j are
# complete and so are its loads of k-step j + 1 (vmcnt(8): only the X loads of the even phase
# before may still be in flight); X and W of k-step j + 2 then go into the stages of X of k-step
# j and W of k-step j - 1, with three and two phases to land.  The source offsets of an operand
# advance by a k-step after its loads.

W16_MFMAS = 64
W16_READ_ORDER = [("w", 0)] + [("x", j) for j in range(8)] + [("w", i) for i in range(1, 8)]
W16_READ_GAPS = tuple(range(4, 36, 2))   # from gap 4 (was 0), with the 2 x 2 MFMA order: 0.4-1.3 % faster, wgrad 2.5 %
W16_DTL_GAPS = {0: tuple(range(1, 32, 4)), 1: tuple(range(1, 32, 4))}
W16_ADV_GAPS = tuple(range(40, 48))


def schedule_w16(phase, tr=False):
    """tr: token-major operands, each fragment two transposing reads (its k-rows 0..3 and 4..7 of
    the lane group); the first goes in the even gap of the plain schedule, the second in the odd
    gap after it, so that no two reads issue back to back."""
    ops = {}

    def at(pos, *items):
        ops.setdefault(pos, []).extend(items)

    cur, nxt = phase, 1 - phase
    if phase == 1:
        at(("pre", 0), "wait_lgkm<0>();", "wait_vm<8>();", "barrier();")
    else:
        at(("pre", 0), "wait_lgkm<0>();")
    at(("pre", 0), f"tie_set<{cur}>(c);")
    for gap, (op, n) in zip(W16_READ_GAPS, W16_READ_ORDER):
        if tr:
            at(gap, f"rd_{op}_half<{nxt}, {n}, 0>(c);")
            at(gap + 1, f"rd_{op}_half<{nxt}, {n}, 1>(c);")
        else:
            at(gap, f"rd_{op}<{nxt}, {n}>(c);")
    for n, g in enumerate(W16_DTL_GAPS[phase]):
        at(g, f"issue_dtl<{phase}>(c, {n});")
    for n, g in enumerate(W16_ADV_GAPS):
        at(g, f"adv<{8 * phase + n}>(c);")
    at(("post",), "rotate(c);", f"read_bases<{nxt}>(c);")
    return ops


def emit_w16(phase, tr=False):
    ops = schedule_w16(phase, tr)
    name = f"phase{phase}_tr" if tr else f"phase{phase}"
    lines = ["template <bool TR>", f"__device__ __forceinline__ void {name}(Ctx<TR> &c)", "{"]
    for m in range(W16_MFMAS):
        lines += ["    " + op for op in ops.get(("pre", m), [])]
        lines.append(f"    mm<{phase}, {m}>(c);")
        lines += ["    " + op for op in ops.get(m, [])]
    lines += ["    " + op for op in ops.get(("post",), [])]
    lines.append("}")
    return "\n".join(lines)


def generate_w16():
    return ("// Generated by gen_gemm_schedule.py -- do not edit.\n"
            "// Main-loop phase bodies of k_linear_w16 (hif8_gemm_w16.hip): row-major operands\n"
            "// (phase0, phase1) and token-major ones (phase0_tr, phase1_tr).\n\n"
            + emit_w16(0) + "\n\n" + emit_w16(1) + "\n\n" + emit_w16(0, True) + "\n\n" + emit_w16(1, True) + "\n")


if __name__ == "__main__":
    here = os.path.dirname(os.path.abspath(__file__))
    out = sys.argv[1] if len(sys.argv) > 1 else os.path.join(here, "hif8_gemm_schedule.inc")
    with open(out, "w") as f:
        f.write(generate())
    out16 = sys.argv[2] if len(sys.argv) > 2 else os.path.join(here, "hif8_gemm_schedule_w16.inc")
    with open(out16, "w") as f:
        f.write(generate_w16())
