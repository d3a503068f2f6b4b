#!/usr/bin/env python3
"""Generate ``attn_q64_loop.inc``: the tile loop of ``attn_q64_kernel``.

The loop is one inline-asm block.  Its registers are fixed, which the
compiler will not hold on its own for this shape: each wave owns 64 queries,
so a 64-key tile is 64 MFMAs per wave and every K / Vᵀ fragment read from LDS
feeds two of them (half the LDS bytes per MFMA of a 32-query wave), at one
wave per SIMD with 512 registers:

    a0   .. a127   O accumulators   O(qb, db) = a[16 (4 qb + db) ...], Oᵀ blocks
    a128 .. a191   Q fragments      Q(qb, j)  = a[128 + 32 qb + 4 j ...]
    a192 .. a255   K fragments      K(kh, j)  = a[192 + 32 kh + 4 j ...]
    v0   .. v63    scores           S(qb, kh) = v[16 (2 qb + kh) ...], Sᵀ blocks
    v64  .. v95    P (bf16 pairs)   P(qb, kh, u) = v[64 + 16 qb + 8 kh + 4 u ...]
    v96  .. v159   Vᵀ fragments     VF(kh, db, u) = v[96 + 32 kh + 8 db + 4 u ...]
    v160 .. v195   softmax state and temporaries

(qb: 32-query block of the wave; kh: 32-key half of the tile; j: 16-wide
slice of the head dim; db: 32-wide block of the value dim; u: 16-key step.)
The products and their operand layouts are those of ``attn_fwd_kernel``
(transposed scores Sᵀ = K Qᵀ, Oᵀ += Vᵀ Pᵀ, P fed from the accumulator
layout), with the same lazy online softmax in the exp2 domain.

Schedule.  A wave running alone on its SIMD has no second wave to cover the
softmax, and between two MFMAs (32 cycles) it can issue only about four
VALU instructions without delaying the next one.  So each key half's
softmax is spread over the MFMA windows of the neighbouring products, across
tiles:

    W1  QK0(t)    ||  exponentials of half 1 of tile t-1, second part;
                      K half 1 and Vᵀ half 0 fragment reads
        [O *= alpha1(t-1) if half 1 of tile t-1 moved the reference max]
    W2  PV1(t-1)  ||  max of half 0 of tile t (a move is applied to m, l at
                      once and to O after W2), exponentials, first part
        [O *= alpha0(t) if it moved]
    W3  QK1(t)    ||  exponentials of half 0, second part; Vᵀ half 1 reads
    W4  PV0(t)    ||  max of half 1 (its O factor deferred to the next W1),
                      exponentials of half 1, first part; the next tile's
                      K half 0 reads

O is scaled by a move's factor after every product of probabilities
relative to the old reference max has been added and before any relative to
the new one, and l at the same point of the sum, so a / l is exactly the
unpipelined online softmax's.  A virtual tile before the first (scores -inf,
P = 0, Vᵀ = 0) makes the first iteration's W1 and W2 work on zeros; after
the loop the pending half 1 of the last tile is drained.

Tiles: a ring of three 32 KB LDS stages (K then V, laid out and swizzled as
in ``attn_fwd_kernel``), loaded by direct global->LDS loads through buffer
resources over the whole head (the tile's byte offset in soffset).  The
loads of tile t+2 are issued at the start of tile t and waited for at its
end, so that tile t+1 is visible during tile t (its first K half is read in
W4).  One barrier per tile publishes the stage and retires the one the next
loads overwrite.

The emitter inserts ``s_waitcnt lgkmcnt`` before the first use of an LDS
read's registers and ``s_nop`` for the MFMA / VALU / transcendental hazards,
with wait-state counts above the hardware's (MFMA result read by VALU or an
MFMA source: 19; VALU result read by an MFMA: 4; v_exp result read by VALU:
2; VALU result read by v_permlane32_swap: 2); conditional blocks (the causal
mask, lazy moves, rescales) count as skipped for hazards that reach past
them.

Run ``python gen_attn_q64.py > attn_q64_loop.inc``; tests/test_host_cpu.py
checks that the committed file is this script's output.
"""
from __future__ import annotations

import sys

NEG_INF = "0xff800000"
LAZY = "0x41000000"  # 8.0: the reference max moves when a tile raises it by more than 8 (log2 units)
NSTAGE = 3
SPLIT = 6            # elements of a key half in the first part of its exponentials

# ---------------------------------------------------------------- registers
def S(qb, kh):
    return 16 * (2 * qb + kh)


def P(qb, kh, u):
    return 64 + 16 * qb + 8 * kh + 4 * u


def VF(kh, db, u):
    return 96 + 32 * kh + 8 * db + 4 * u


def O(qb, db):
    return 16 * (4 * qb + db)


def Q(qb, j):
    return 128 + 32 * qb + 4 * j


def K(kh, j):
    return 192 + 32 * kh + 4 * j


MRUN = (160, 161)    # reference max per query block (raw score units)
MTRUE = (162, 163)   # true max
LRUN = (164, 165)    # denominator (this lane's half of the keys)
ALPHA1 = (166, 167)  # deferred O factor of half 1
MT = (168, 169)
TMP = (170, 171)
MR = (172, 173)
MC = (174, 175)      # m_run * c of the half being exponentiated
ALPHA0 = (176, 177)  # deferred O factor of half 0
LIM = 178            # causal limit of the tile
AL = (179, 180)
NINF = 181           # -inf (a literal beside vcc would exceed the constant bus)
LSA = {0: (182, 183), 1: (184, 185)}  # first-part row sums per key half
TREE = {0: [186, 187, 188, 189, 190], 1: [191, 192, 193, 194, 195]}
RTMP = [186 + i for i in range(8)]    # rescale temporaries (the max trees are idle then)
NVGPR = 196


def vrng(b, n):
    return f"v[{b}:{b + n - 1}]" if n > 1 else f"v{b}"


def arng(b, n):
    return f"a[{b}:{b + n - 1}]" if n > 1 else f"a{b}"


def vset(b, n=1):
    return [f"v{b + i}" for i in range(n)]


def aset(b, n=1):
    return [f"a{b + i}" for i in range(n)]


# hazard wait states (conservative)
W_MFMA_TO_READ = 19
W_VALU_TO_MFMA = 4
W_TRANS_TO_VALU = 2
W_VALU_TO_PERM = 2


class Emitter:
    """Straight-line emission with register-level wait and hazard tracking."""

    def __init__(self):
        self.out: list[str] = []
        self.time = 0                                   # wait states issued so far
        self.w: dict[str, tuple[int, str, str]] = {}    # reg -> (time, kind, MFMA range)
        self.lgkm: list[set[str]] = []                  # outstanding LDS ops, oldest first
        self.in_block = False
        self.block_writes: set[str] = set()
        self.block_t0 = 0

    def raw(self, text):
        self.out.append(text)

    def label(self, name):
        self.out.append(f"{name}%=:")

    def _wait_lgkm(self, regs):
        idx = -1
        for i, s in enumerate(self.lgkm):
            if s & regs:
                idx = i
        if idx >= 0:
            n = min(len(self.lgkm) - 1 - idx, 15)
            self.out.append(f"s_waitcnt lgkmcnt({n})")
            self.lgkm = self.lgkm[len(self.lgkm) - n:] if n > 0 else []

    @staticmethod
    def _required(wkind, wkey, rkind, role, rkey):
        if wkind == "mfma":
            # an MFMA accumulating onto the previous MFMA's exact range needs none
            if rkind == "mfma" and role in ("srcc", "dst") and rkey == wkey:
                return 0
            return W_MFMA_TO_READ
        if wkind in ("valu", "trans", "perm", "accw"):
            if rkind == "mfma":
                return W_VALU_TO_MFMA
            if wkind == "trans" and rkind in ("valu", "trans", "perm", "accr", "accw"):
                return W_TRANS_TO_VALU
            if rkind == "perm":
                return W_VALU_TO_PERM
        return 0

    def ins(self, text, kind, reads=(), writes=(), srcc=(), key=""):
        """kind: mfma valu trans perm accr accw ds dsw salu vmem dma."""
        reads, writes, srcc = set(reads), set(writes), set(srcc)
        self._wait_lgkm(reads | writes | srcc)
        need = 0
        for r in reads | srcc | writes:
            if r in self.w:
                wt, wk, wkey = self.w[r]
                role = "srcc" if r in srcc else ("dst" if r in writes and r not in reads else "src")
                need = max(need, self._required(wk, wkey, kind, role, key) - (self.time - wt - 1))
        while need > 0:
            n = min(need, 16)
            self.out.append(f"s_nop {n - 1}")
            self.time += n
            need -= n
        self.out.append(text)
        for r in writes:
            self.w[r] = (self.time, kind, key)
            if self.in_block:
                self.block_writes.add(r)
        self.time += 1
        if kind == "ds":
            assert not self.in_block
            self.lgkm.append(set(writes))
        elif kind == "dsw":
            self.lgkm.append(set())

    def block(self, branch, items, label):
        """A conditional block of VALU / SALU items, skipped when `branch` is taken."""
        self.raw(branch)
        t0 = self.time
        self.in_block, self.block_writes = True, set()
        for it in items:
            self.item(it)
        self.label(label)
        self.in_block = False
        # hazards reaching past the block: the skipping path's distances, and
        # the block's writes taken as made just before it ends on that path
        self.time = t0
        for r in self.block_writes:
            _, k, key = self.w[r]
            self.w[r] = (t0 - 1, k, key)

    def item(self, it):
        if it[0] == "block":
            self.block(it[1], it[2], it[3])
        else:
            kind, text, reads, writes = it
            self.ins(text, kind, reads=reads, writes=writes)

    def fence(self):
        self.out += ["s_nop 15", "s_nop 15"]
        self.time += 32


# ------------------------------------------------------------------ pieces
def mfma(e, dst_kind, dst, a, b, first=False):
    rng = vrng if dst_kind == "v" else arng
    dset = (vset if dst_kind == "v" else aset)(dst, 16)

    def src(k, base):
        return (vrng(base, 4), vset(base, 4)) if k == "v" else (arng(base, 4), aset(base, 4))

    at, ar_ = src(*a)
    bt, br = src(*b)
    c = "0" if first else rng(dst, 16)
    e.ins(f"v_mfma_f32_32x32x16_bf16 {rng(dst, 16)}, {at}, {bt}, {c}", "mfma",
          reads=set(ar_) | set(br), writes=dset, srcc=() if first else dset, key=rng(dst, 16))


def sbase(st):
    """Address register set and immediate of stage st (ds offsets are 16-bit:
    stage 2 is read through the second set, 64 KB further)."""
    return ("", st * 32768) if st < 2 else ("h", 0)


def k_reads(st, kh):
    sfx, b0 = sbase(st)
    return [("ds", f"ds_read_b128 {arng(K(kh, j), 4)}, %[ka{sfx}{j}] offset:{b0 + kh * 8192}", (),
             aset(K(kh, j), 4)) for j in range(8)]


def v_reads(st, kh):
    sfx, b0 = sbase(st)
    out = []
    for db in range(4):
        for u in range(2):
            base = VF(kh, db, u)
            off = b0 + kh * 8192 + u * 4096
            out.append(("ds", f"ds_read_b64_tr_b16 {vrng(base, 2)}, %[va{sfx}{db}] offset:{off}", (),
                        vset(base, 2)))
            out.append(("ds", f"ds_read_b64_tr_b16 {vrng(base + 2, 2)}, %[va{sfx}{db}] offset:{off + 2048}", (),
                        vset(base + 2, 2)))
    return out


def rescale(qb, alpha):
    items = []
    for db in range(4):
        for r in range(16):
            a = O(qb, db) + r
            t = RTMP[r & 7]
            items.append(("accr", f"v_accvgpr_read_b32 v{t}, a{a}", [f"a{a}"], [f"v{t}"]))
            items.append(("valu", f"v_mul_f32_e32 v{t}, v{alpha}, v{t}", [f"v{t}", f"v{alpha}"], [f"v{t}"]))
            items.append(("accw", f"v_accvgpr_write_b32 a{a}, v{t}", [f"v{t}"], [f"a{a}"]))
    return items


def resc_block(kh, tag):
    alpha = ALPHA0 if kh == 0 else ALPHA1
    fl = "%[fl0]" if kh == 0 else "%[fl1]"
    return ("block", f"s_cmp_eq_u32 {fl}, 0\n\ts_cbranch_scc1 L_rs{tag}%=", rescale(0, alpha[0]) + rescale(1, alpha[1]),
            f"L_rs{tag}")


def pre_items(kh):
    alpha = ALPHA0 if kh == 0 else ALPHA1
    fl = "%[fl0]" if kh == 0 else "%[fl1]"
    return [("salu", f"s_mov_b32 {fl}, 0", (), []),
            ("valu", f"v_mov_b32_e32 v{alpha[0]}, 1.0", (), [f"v{alpha[0]}"]),
            ("valu", f"v_mov_b32_e32 v{alpha[1]}, 1.0", (), [f"v{alpha[1]}"])]


def mask_block(kh, tag):
    """Causal mask of key half kh (tiles at or past mask_from): key kv0 + 32 kh +
    row(r, g) is kept for query qw0 + 32 qb + l32 iff it is at most the query
    plus the offset, i.e. iff 32 (kh - qb) + 8 (r / 4) + r % 4 <= lim0 - kv0
    with lim0 = qw0 + offset + l32 - 4 g."""
    body = [("valu", f"v_subrev_u32_e32 v{LIM}, %[kv0], %[lim0]", (), [f"v{LIM}"])]
    for qb in range(2):
        for r in range(16):
            cst = 32 * (kh - qb) + 8 * (r >> 2) + (r & 3)
            sr = S(qb, kh) + r
            body.append(("valu", f"v_cmp_le_i32_e32 vcc, {cst}, v{LIM}", [f"v{LIM}"], []))
            body.append(("valu", f"v_cndmask_b32_e32 v{sr}, v{NINF}, v{sr}, vcc", [f"v{sr}", f"v{NINF}"],
                         [f"v{sr}"]))
    return ("block", f"s_cmp_ge_u32 %[t], %[mfrom]\n\ts_cbranch_scc0 L_nm{tag}%=", body, f"L_nm{tag}")


def max_items(kh, tag):
    """Row maxima of both query blocks (trees; the lane halves combined by a
    permlane32 swap), the true max, and the lazy check.  A move updates m_run
    and l_run at once and leaves O's factor in ALPHA{kh} with its flag set."""
    items = []
    for i in range(5):
        for qb in range(2):
            s0 = S(qb, kh) + 3 * i
            items.append(("valu", f"v_max3_f32 v{TREE[qb][i]}, v{s0}, v{s0 + 1}, v{s0 + 2}", vset(s0, 3),
                          [f"v{TREE[qb][i]}"]))
    for qb in range(2):
        t = TREE[qb]
        items.append(("valu", f"v_max3_f32 v{t[0]}, v{t[0]}, v{t[1]}, v{t[2]}", [f"v{t[0]}", f"v{t[1]}", f"v{t[2]}"],
                      [f"v{t[0]}"]))
    for qb in range(2):
        t = TREE[qb]
        s15 = S(qb, kh) + 15
        items.append(("valu", f"v_max3_f32 v{t[3]}, v{t[3]}, v{t[4]}, v{s15}", [f"v{t[3]}", f"v{t[4]}", f"v{s15}"],
                      [f"v{t[3]}"]))
    for qb in range(2):
        t = TREE[qb]
        items.append(("valu", f"v_max_f32_e32 v{MT[qb]}, v{t[0]}, v{t[3]}", [f"v{t[0]}", f"v{t[3]}"], [f"v{MT[qb]}"]))
    for qb in range(2):
        items.append(("valu", f"v_mov_b32_e32 v{TMP[qb]}, v{MT[qb]}", [f"v{MT[qb]}"], [f"v{TMP[qb]}"]))
    for qb in range(2):
        mt, tmp = MT[qb], TMP[qb]
        items.append(("perm", f"v_permlane32_swap_b32 v{mt}, v{tmp}", [f"v{mt}", f"v{tmp}"], [f"v{mt}", f"v{tmp}"]))
    for qb in range(2):
        mt, tmp = MT[qb], TMP[qb]
        items.append(("valu", f"v_max_f32_e32 v{mt}, v{mt}, v{tmp}", [f"v{mt}", f"v{tmp}"], [f"v{mt}"]))
    alpha = ALPHA0 if kh == 0 else ALPHA1
    fl = "%[fl0]" if kh == 0 else "%[fl1]"
    for qb in range(2):
        mt, tmp, al = MT[qb], TMP[qb], AL[qb]
        items.append(("valu", f"v_max_f32_e32 v{MTRUE[qb]}, v{MTRUE[qb]}, v{mt}", [f"v{MTRUE[qb]}", f"v{mt}"],
                      [f"v{MTRUE[qb]}"]))
        items.append(("valu", f"v_sub_f32_e32 v{tmp}, v{mt}, v{MRUN[qb]}", [f"v{mt}", f"v{MRUN[qb]}"], [f"v{tmp}"]))
        items.append(("valu", f"v_mul_f32_e32 v{tmp}, %[c], v{tmp}", [f"v{tmp}"], [f"v{tmp}"]))
        items.append(("valu", f"v_cmp_lt_f32_e32 vcc, {LAZY}, v{tmp}", [f"v{tmp}"], []))
        mv = [
            ("valu", f"v_max_f32_e32 v{tmp}, v{MRUN[qb]}, v{mt}", [f"v{MRUN[qb]}", f"v{mt}"], [f"v{tmp}"]),
            ("valu", f"v_sub_f32_e32 v{al}, v{MRUN[qb]}, v{tmp}", [f"v{MRUN[qb]}", f"v{tmp}"], [f"v{al}"]),
            ("valu", f"v_mul_f32_e32 v{al}, %[c], v{al}", [f"v{al}"], [f"v{al}"]),
            ("trans", f"v_exp_f32_e32 v{al}, v{al}", [f"v{al}"], [f"v{al}"]),
            ("valu", f"v_cmp_neq_f32_e32 vcc, {NEG_INF}, v{MRUN[qb]}", [f"v{MRUN[qb]}"], []),
            ("valu", f"v_cndmask_b32_e32 v{al}, 0, v{al}, vcc", [f"v{al}"], [f"v{al}"]),
            ("valu", f"v_mul_f32_e32 v{LRUN[qb]}, v{LRUN[qb]}, v{al}", [f"v{LRUN[qb]}", f"v{al}"], [f"v{LRUN[qb]}"]),
            ("valu", f"v_mov_b32_e32 v{MRUN[qb]}, v{tmp}", [f"v{tmp}"], [f"v{MRUN[qb]}"]),
            ("valu", f"v_mov_b32_e32 v{alpha[qb]}, v{al}", [f"v{al}"], [f"v{alpha[qb]}"]),
            ("salu", f"s_mov_b32 {fl}, 1", (), []),
        ]
        items.append(("block", f"s_cbranch_vccz L_mv{qb}{tag}%=", mv, f"L_mv{qb}{tag}"))
    return items


def exp_part(kh, h):
    """p = exp2(s c - m c) for part h of key half kh (elements [0, SPLIT) or
    [SPLIT, 16), both query blocks), packed to bf16 into P, and their row sum
    (a tree in place; the first part's sum waits in LSA, the second adds both
    to l_run)."""
    items = []
    if h == 0:
        for qb in range(2):
            mr, mc = MR[qb], MC[qb]
            items += [
                ("valu", f"v_cmp_neq_f32_e32 vcc, {NEG_INF}, v{MRUN[qb]}", [f"v{MRUN[qb]}"], []),
                ("valu", f"v_cndmask_b32_e32 v{mr}, 0, v{MRUN[qb]}, vcc", [f"v{MRUN[qb]}"], [f"v{mr}"]),
                ("valu", f"v_mul_f32_e32 v{mc}, %[c], v{mr}", [f"v{mr}"], [f"v{mc}"]),
            ]
    lo, hi = (0, SPLIT) if h == 0 else (SPLIT, 16)
    for r in range(lo, hi):
        for qb in range(2):
            a = S(qb, kh) + r
            items.append(("valu", f"v_fma_f32 v{a}, v{a}, %[c], -v{MC[qb]}", [f"v{a}", f"v{MC[qb]}"], [f"v{a}"]))
    for r in range(lo, hi):
        for qb in range(2):
            a = S(qb, kh) + r
            items.append(("trans", f"v_exp_f32_e32 v{a}, v{a}", [f"v{a}"], [f"v{a}"]))
    for r in range(lo, hi, 2):
        for qb in range(2):
            a = S(qb, kh) + r
            p = P(qb, kh, r >> 3) + ((r & 7) >> 1)
            items.append(("valu", f"v_cvt_pk_bf16_f32 v{p}, v{a}, v{a + 1}", [f"v{a}", f"v{a + 1}"], [f"v{p}"]))
    n, step = hi - lo, 1
    while step < n:
        for i in range(0, n - step, 2 * step):
            for qb in range(2):
                a = S(qb, kh) + lo + i
                items.append(("valu", f"v_add_f32_e32 v{a}, v{a}, v{a + step}", [f"v{a}", f"v{a + step}"], [f"v{a}"]))
        step *= 2
    for qb in range(2):
        a = S(qb, kh) + lo
        if h == 0:
            items.append(("valu", f"v_mov_b32_e32 v{LSA[kh][qb]}, v{a}", [f"v{a}"], [f"v{LSA[kh][qb]}"]))
        else:
            items.append(("valu", f"v_add_f32_e32 v{a}, v{a}, v{LSA[kh][qb]}", [f"v{a}", f"v{LSA[kh][qb]}"], [f"v{a}"]))
            items.append(("valu", f"v_add_f32_e32 v{LRUN[qb]}, v{LRUN[qb]}, v{a}", [f"v{LRUN[qb]}", f"v{a}"],
                          [f"v{LRUN[qb]}"]))
    return items


def qk(e, kh):
    return [(lambda j=j, qb=qb: mfma(e, "v", S(qb, kh), ("a", K(kh, j)), ("a", Q(qb, j)), first=(j == 0)))
            for j in range(8) for qb in range(2)]


def pv(e, kh):
    return [(lambda qb=qb, db=db, u=u: mfma(e, "a", O(qb, db), ("v", VF(kh, db, u)), ("v", P(qb, kh, u))))
            for u in range(2) for qb in range(2) for db in range(4)]


def interleave(e, mfmas, others):
    """MFMAs with the other items spread evenly between them."""
    cost = [4 if it[0] == "block" else 1 for it in others]
    per = -(-sum(cost) // len(mfmas))
    oi = 0
    for m in mfmas:
        m()
        budget = per
        while oi < len(others) and budget > 0:
            e.item(others[oi])
            budget -= cost[oi]
            oi += 1
    while oi < len(others):
        e.item(others[oi])
        oi += 1


def dma(e, stage):
    """Global->LDS loads of one tile (K then V) into `stage`."""
    for i in range(4):
        e.ins(f"s_add_u32 m0, %[dmab], {stage * 32768 + i * 4096}", "salu")
        e.ins("s_nop 0", "salu")  # SALU write of M0 -> LDS-DMA read of it
        e.ins(f"buffer_load_dwordx4 %[ko{i}], %[krs], %[kso] offen lds", "dma")
        e.ins(f"s_add_u32 m0, %[dmab], {stage * 32768 + 16384 + i * 4096}", "salu")
        e.ins("s_nop 0", "salu")
        e.ins(f"buffer_load_dwordx4 %[vo{i}], %[vrs], %[vso] offen lds", "dma")


def compute(e, st):
    interleave(e, qk(e, 0), exp_part(1, 1) + k_reads(st, 1) + v_reads(st, 0))
    e.item(resc_block(1, f"a{st}"))
    interleave(e, pv(e, 1), pre_items(0) + [mask_block(0, f"0_{st}")] + max_items(0, f"0_{st}") + exp_part(0, 0))
    e.item(resc_block(0, f"b{st}"))
    interleave(e, qk(e, 1), exp_part(0, 1) + v_reads(st, 1))
    interleave(e, pv(e, 0), pre_items(1) + [mask_block(1, f"1_{st}")] + max_items(1, f"1_{st}") + exp_part(1, 0)
               + k_reads((st + 1) % NSTAGE, 0))


def body(e, st):
    e.raw("s_add_u32 %[tmp], %[t], 2")
    e.raw("s_cmp_lt_u32 %[tmp], %[nkv]")
    e.raw(f"s_cbranch_scc0 L_nd{st}%=")
    dma(e, (st + 2) % NSTAGE)
    e.label(f"L_nd{st}")
    e.raw("s_cmp_lt_u32 %[t], %[wnt]")
    e.raw(f"s_cbranch_scc0 L_nc{st}%=")
    compute(e, st)
    e.label(f"L_nc{st}")
    e.raw("s_waitcnt vmcnt(0) lgkmcnt(0)")
    e.lgkm = []
    e.raw("s_barrier")
    e.raw("s_add_u32 %[t], %[t], 1")
    e.raw("s_add_u32 %[kv0], %[kv0], 64")
    e.raw("s_add_u32 %[kso], %[kso], %[kstep]")
    e.raw("s_add_u32 %[vso], %[vso], %[vstep]")


def generate() -> str:
    e = Emitter()
    e.raw("s_waitcnt vmcnt(0) lgkmcnt(0)")
    # Q into AGPRs, O = 0, softmax state, the virtual tile before the first
    for qb in range(2):
        for j in range(8):
            e.ins(f"global_load_dwordx4 {arng(Q(qb, j), 4)}, %[qa{qb}], off offset:{32 * j}", "vmem",
                  writes=aset(Q(qb, j), 4))
    for i in range(128):
        e.ins(f"v_accvgpr_write_b32 a{i}, 0", "accw", writes=[f"a{i}"])
    e.ins(f"v_mov_b32_e32 v{NINF}, {NEG_INF}", "valu", writes=[f"v{NINF}"])
    for qb in range(2):
        e.ins(f"v_mov_b32_e32 v{MRUN[qb]}, {NEG_INF}", "valu", writes=[f"v{MRUN[qb]}"])
        e.ins(f"v_mov_b32_e32 v{MTRUE[qb]}, {NEG_INF}", "valu", writes=[f"v{MTRUE[qb]}"])
        e.ins(f"v_mov_b32_e32 v{LRUN[qb]}, 0", "valu", writes=[f"v{LRUN[qb]}"])
        e.ins(f"v_mov_b32_e32 v{MC[qb]}, 0", "valu", writes=[f"v{MC[qb]}"])
        e.ins(f"v_mov_b32_e32 v{LSA[1][qb]}, 0", "valu", writes=[f"v{LSA[1][qb]}"])
        e.ins(f"v_mov_b32_e32 v{ALPHA1[qb]}, 1.0", "valu", writes=[f"v{ALPHA1[qb]}"])
        for r in range(16):
            e.ins(f"v_mov_b32_e32 v{S(qb, 1) + r}, v{NINF}", "valu", reads=[f"v{NINF}"], writes=[f"v{S(qb, 1) + r}"])
        for i in range(8):
            e.ins(f"v_mov_b32_e32 v{P(qb, 1, 0) + i}, 0", "valu", writes=[f"v{P(qb, 1, 0) + i}"])
    for i in range(32):
        e.ins(f"v_mov_b32_e32 v{VF(1, 0, 0) + i}, 0", "valu", writes=[f"v{VF(1, 0, 0) + i}"])
    e.raw("s_mov_b32 %[fl1], 0")
    e.raw("s_mov_b32 %[t], 0")
    e.raw("s_mov_b32 %[kv0], 0")
    e.raw("s_mov_b32 %[kso], 0")
    e.raw("s_mov_b32 %[vso], 0")
    e.raw("s_cmp_eq_u32 %[nkv], 0")
    e.raw("s_cbranch_scc1 L_end%=")
    # tiles 0 and 1, and tile 0's first K half
    dma(e, 0)
    e.raw("s_add_u32 %[kso], %[kso], %[kstep]")
    e.raw("s_add_u32 %[vso], %[vso], %[vstep]")
    e.raw("s_cmp_lt_u32 1, %[nkv]")
    e.raw("s_cbranch_scc0 L_p1%=")
    dma(e, 1)
    e.label("L_p1")
    e.raw("s_waitcnt vmcnt(0)")
    e.raw("s_add_u32 %[kso], %[kso], %[kstep]")
    e.raw("s_add_u32 %[vso], %[vso], %[vstep]")
    e.raw("s_barrier")
    for it in k_reads(0, 0):
        e.item(it)
    e.raw("s_waitcnt lgkmcnt(0)")
    e.lgkm = []
    e.fence()
    # the loop, unrolled over the three stages; a first pass gives the state
    # at the back edge, from which the emitted pass starts
    head = len(e.out)
    for st in range(NSTAGE):
        body(e, st)
    time_end, w_end = e.time, dict(e.w)
    del e.out[head:]
    e.time, e.w, e.lgkm = time_end, w_end, []
    e.label("L_loop")
    for st in range(NSTAGE):
        body(e, st)
        if st < NSTAGE - 1:
            e.raw("s_cmp_ge_u32 %[t], %[nkv]")
            e.raw("s_cbranch_scc1 L_end%=")
    e.raw("s_cmp_lt_u32 %[t], %[nkv]")
    e.raw("s_cbranch_scc1 L_loop%=")
    e.label("L_end")
    # drain: the pending half 1 of the last tile this wave computed
    e.fence()
    for it in exp_part(1, 1):
        e.item(it)
    e.item(resc_block(1, "d"))
    for m in pv(e, 1):
        m()
    # O to LDS (16-byte pieces, lane-major), softmax state out
    e.fence()
    for qb in range(2):
        for db in range(4):
            for r4 in range(4):
                a = O(qb, db) + 4 * r4
                e.ins(f"ds_write_b128 %[ob], {arng(a, 4)} offset:{((qb * 4 + db) * 4 + r4) * 1024}", "dsw",
                      reads=aset(a, 4))
    for qb in range(2):
        e.raw(f"v_mov_b32_e32 %[mr{qb}], v{MRUN[qb]}")
        e.raw(f"v_mov_b32_e32 %[mt{qb}], v{MTRUE[qb]}")
        e.raw(f"v_mov_b32_e32 %[lr{qb}], v{LRUN[qb]}")
    e.raw("s_waitcnt lgkmcnt(0)")
    return "\n".join(e.out)


def render() -> str:
    lines = ["// Generated by gen_attn_q64.py (the tile loop of attn_q64_kernel); do not edit.",
             "#define ATTN_Q64_ASM \\"]
    for ln in generate().split("\n"):
        lines.append(f'  "{ln}\\n\\t" \\')
    lines.append('  ""')
    regs = [f'"v{i}"' for i in range(NVGPR)] + [f'"a{i}"' for i in range(256)]
    lines.append("#define ATTN_Q64_CLOBBERS " + ", ".join(regs))
    return "\n".join(lines) + "\n"


if __name__ == "__main__":
    sys.stdout.write(render())
