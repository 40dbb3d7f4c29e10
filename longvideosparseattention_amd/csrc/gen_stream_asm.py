"""Generate the key loop of the single-stream attention kernel (every 16-bit head size).

    python gen_stream_asm.py [out.inc]   (default: lvsa_attn_stream_body.inc beside this file)
    python gen_stream_asm.py --census    (instruction counts per 32-key sub-block of each loop)

The loop is hand-scheduled gfx950 assembly, emitted as the body of one inline
asm statement of ``attn_fwd_stream_kernel`` (lvsa_attn_stream.h), whose
operands pin every register this text names; the operand lists are emitted
here too (``LVSA_STREAM<D>_OUTPUTS`` / ``_INPUTS`` / ``_CLOBBERS``), so the
register map lives in one place.  Each of the 8 waves of a work-group owns
32 query rows of a 256-row tile and walks the tile's 64-key blocks as two
32-key sub-blocks; sub-iteration i issues, as one stream,

    QK(i)   S = K Q^T of sub-block i          D/16 MFMAs  (K from LDS)
    SM(i-1) softmax of sub-block i - 1        ~50 VALU    (P = 2^(S*cs - m))
    PV(i-2) O += V^T P^T of sub-block i - 2   D/16 MFMAs  (V^T from LDS)

so every wave keeps the matrix core and the VALU busy at once, and the two
waves that share a SIMD fill each other's gaps.  Per 64-key block: one
work-group barrier, D/64 1 KiB global->LDS copies of K and as many of V per
wave (block j + 2 into a 4-stage ring) and one scalar load of a plan entry.
Options (PRODUCT below has the ones in use per head size): `lead` PV MFMAs
open each block with V operands read before the barrier (V of block j - 1
has been in LDS since the previous barrier), so the matrix core has work
while the first K operands of the block are read; `early_load` issues the
scalar load of entry j + 3 in the middle of block j, not just before the
barrier that waits for it; `dot_init` starts the two row-sum chains of a
sub-block with a non-accumulating v_dot2 (C = 0) instead of zeroing them;
`rs_mfma` replaces those chains by two v_mfma_f32_16x16x32 per sub-block with
A = a constant ones pattern and B = the packed P, which leave the full row sum
of query l in lane l (l < 32) and zero in lanes 32-63.

Softmax without a row max: P is formed against the running max m of the
earlier blocks; m has to move only if some P exceeds 2^8, and then the
lane's share of the sub-block's row sum exceeds 2^8 too.  That rare case
(and the first block, whose m is -1e30) calls RARE: true row max, rescale of
O and of the row sum, P recomputed.  Blocks with a two-part mask descriptor
call MASK first (-inf on the masked keys).  Generic descriptors are not
handled here: the host runs the compiler-built kernel for geometries that
can produce them.

Hazards (gfx950, software-managed; the wait states are the ones hipcc inserts
for the same pairs): an MFMA result is read by VALU at least two MFMAs after
the MFMA that wrote it (12 states for the 8-pass 32x32x16 MFMA); RARE waits
24 states before it touches O; a v_dot2 result is read by another VALU 3
states later; a v_exp result 1 state later; VALU results feed MFMAs a
sub-iteration later; M0 writes are followed by one state before an LDS copy;
v_permlane32_swap is fenced by two states on each side.

Register map (VGPRs; the kernel's operands pin them), D = 128 (D = 64):
  O (D/32 d-tiles x 16) v[0:63] (v[0:31]); Q (D/16 k-steps x 4) v[64:95]
  (v[32:47]); then two S tiles (16 each), two P tiles (8 each), eight LDS
  operand slots (4 each), the K read offsets (one per k-step), the V^T read
  offsets (two per d-tile), then m, l, two partial row sums, the copy row and
  chunk, the two copy offsets, the tile row, 4*h, -inf, a mask temp, four
  RARE temps and sixteen softmax temps: 224 (168) VGPRs in all.  With
  rs_mfma the two partial row sums give way to a ones pattern and a row-sum
  tile (4 each).  The 12-wave D = 64 map (Layout nw = 12) has four operand
  slots, eight softmax temps and the RARE temps inside them: 148 VGPRs.
  The dual map (D = 64, Layout nw = 4) gives each wave 64 query rows as two
  32-row halves: every operand item (an LDS read) feeds two MFMAs, one per
  half (S + 16 r with Q + 16 r; O + 32 r with P + 8 r), and the softmax, the
  rare path (either half's row sum over 2^8 takes both) and the mask run per
  half (m and l of half r in VM + r and VL + r, its row sum in RS + 4 r, its
  tile row in ROW + 32 r = ROW1); four operand slots, eight softmax temps:
  249 VGPRs, two waves per SIMD (4 waves per work-group, two work-groups per
  CU, 2 copies of K and 2 of V per wave and block).
  D = 96 (6 k-steps, 3 d-tiles) follows the D = 128 map with fewer O, Q and
  offset registers (202 VGPRs) and uses the D = 128 LDS layout: 256-byte rows
  whose chunks 12-15 the copies fill with zeros and no read touches.
  D = 192 and 256 use the wide map (Layout nw = 4): 4 waves of 32 rows, one per
  SIMD, O in AGPRs a[0 : 16 NDT], Q from v0, two lane copy offsets per tensor
  (the swizzle of copy ii depends on its parity) and four soffsets; 512-byte
  rows, K and V in two-stage rings of their own: block j copies K(j+1) and V(j)
  and waits for all copies at the next barrier, K and V tracking their key
  sources separately (SWITCHK / SWITCHV).  218 (194) VGPRs.
  D = 192 by default runs the dual-wide map (Layout nw = 4, dual = True): the
  wide map's copies, rings and AGPR-held O with the dual map's two 32-row
  halves per wave (256-row tiles): O of half r in a[96 r : 96 r + 95], Q of
  half 0 in v[0:47] and of half 1 in the AGPRs after O, a[192:239] (MFMAs
  take B from AGPRs), the S, P, m, l and row-sum registers per half as in the
  dual map, sixteen softmax temps: 241 VGPRs and 240 AGPRs.
SGPRs: s[20:21] entry pointer, s22 blocks, s23 scale*log2(e), s[24:31] K/V
bases (video, extra), s32-35 row strides, s36-37 source lengths, s38 wave,
s39 LDS copy base of the wave; s40-s95 scratch.
"""

from __future__ import annotations

import sys
from pathlib import Path

# ── SGPR map ──
S_EPTR, S_N, S_CS = 20, 22, 23
S_KB0, S_VB0, S_KB1, S_VB1 = 24, 26, 28, 30
S_KRS0, S_VRS0, S_KRS1, S_VRS1, S_NK, S_NX, S_WAVE, S_LDSK = 32, 33, 34, 35, 36, 37, 38, 39
S_J, S_NM1, S_CUR, S_ENT, S_RK, S_RV = 40, 41, 42, 44, 52, 56
S_SOK, S_SOV, S_KRSC = 60, 62, 64  # copy soffsets (K: 60, 61; V: 62, 63); strides, 32-row strides
S_RET = 76
S_SOVW, S_CURV = 68, 72            # wide map: V soffsets (68-71) and V's key source
S_ONE = 43                         # a pair of 1.0 in the element type (row-sum dots)
CLOBBER_S = list(range(40, 96))
NSLOT = 8                         # LDS operand slots
LA = 3                            # MFMAs of LDS operand lookahead (< NSLOT); 3 measured best:
                                  # 2.5% (D = 128) and 4.3% (D = 64) fewer cycles than 6


class Layout:
    """Head-size dependent shapes and the VGPR map.  `nw` = 12 is the compact
    map of the 12-wave kernel (three waves per SIMD, at most 168 VGPRs in all):
    four operand slots read two MFMAs ahead, eight softmax temporaries, and the
    rare path's temporaries shared with them.  `nw` = 4 is the wide map of
    D = 192 and 256: one wave per SIMD, O in AGPRs, K and V in two-stage LDS
    rings of their own (rows on the 512-byte pitch); at D = 64 it is the dual
    map: 64 rows per wave in two 32-row halves (NR = 2), the compact map's
    slots and temporaries, at most 256 VGPRs (two waves per SIMD).  `dual`
    with D = 192 is the dual-wide map: the wide map with two 32-row halves
    per wave, half 1's Q in the AGPRs after O (QA)."""

    def __init__(self, D: int, nw: int = 8, rs: bool = False, dual: bool | None = None):
        dual = (nw == 4 and D == 64) if dual is None else dual
        assert (D, nw, dual) in ((64, 8, False), (96, 8, False), (128, 8, False), (64, 12, False), (192, 4, False),
                                 (256, 4, False), (64, 4, True), (192, 4, True))
        self.D = D
        self.nw = nw
        self.wide = nw == 4 and D >= 192
        self.dual = dual                  # two 32-row halves per wave (64 rows)
        self.NR = 2 if self.dual else 1   # 32-row halves per wave
        assert rs or not self.dual
        self.rs = rs                      # row sums by MFMA: ONES (A pattern) and RS (result) tiles
        compact = nw == 12 or (self.dual and not self.wide)
        self.nslot = 4 if compact else NSLOT
        self.NT = 8 if compact or self.dual else 16   # softmax temporaries
        self.NQK = D // 16                # MFMA k-steps of a score tile
        self.NDT = D // 32                # 32-wide d-tiles of O
        # D = 96 rows sit on the D = 128 LDS pitch and D = 192 rows on the
        # D = 256 pitch: the chunks past a row's data are filled by copy lanes
        # reading out of range (zeros) and never read
        self.RB = 2 * {96: 128, 192: 256}.get(D, D)   # bytes per K/V row in LDS
        self.TILE = 64 * self.RB          # one K or V block
        self.NST = 2 if self.wide else 4  # LDS stages per tensor
        self.VBASE = self.NST * self.TILE  # V stages follow the K stages
        self.NCP = self.TILE // 1024 // (4 if nw == 4 else 8)   # 1 KiB copies per tensor, wave and block
        # rows between a wave's consecutive copies of one tensor (8 or 4 waves x 1 KiB)
        self.CPROWS = (4 if nw == 4 else 8) * 1024 // self.RB
        r = 0

        def take(n: int) -> int:
            nonlocal r
            r += n
            return r - n
        NR = self.NR
        self.O = 0 if self.wide else take(16 * self.NDT * NR)   # wide: a[0 : 16 NDT]; dual: half 0, half 1
        if self.wide and self.dual:
            # the dual-wide map: Q of half 0 in VGPRs, of half 1 in the AGPRs after O
            self.Q = take(4 * self.NQK)
            self.QA = 16 * self.NDT * NR
        else:
            self.Q = take(4 * self.NQK * NR)
            self.QA = None
        self.SA, self.SB = take(16 * NR), take(16 * NR)      # dual: the S tile of half r at + 16 r
        self.PA, self.PB = take(8 * NR), take(8 * NR)        # and its P at + 8 r
        self.OPS = take(4 * self.nslot)
        self.KOFF = take(self.NQK)
        self.VOFFA = take(self.NDT)
        self.VOFFB = take(self.NDT)
        if rs:
            self.VM, self.VL = take(NR), take(NR)            # m and l of each half
            self.ONES, self.RS = take(4), take(4 * NR)
            self.LS0 = self.LS1 = self.RS        # the row sum of the sub-block: RS register 0
        else:
            self.VM, self.VL, self.LS0, self.LS1 = take(1), take(1), take(1), take(1)
        # copy geometry: the row and chunk offset of a lane's copies (wide: one
        # pair per parity of the copy index), and the lane offsets of K and V
        npar = 2 if self.wide else 1
        self.DMAROW = take(2 * npar)
        self.C16 = self.DMAROW + 1
        self.DK, self.DV = take(npar), take(npar)
        self.ROW, self.H4, self.NEGINF, self.VT = take(1), take(1), take(1), take(1)
        self.ROW1 = take(1) if self.dual else None           # tile row of half 1 (ROW + 32)
        if compact:
            self.T = take(self.NT)
            self.RT = self.T                 # the rare path runs between softmaxes
        else:
            self.RT = take(4)                # (the wide maps scale O through T in the rare path)
            self.T = take(self.NT)
        self.NVGPR = r
        self.NAGPR = (16 * self.NDT * NR + (4 * self.NQK if self.QA is not None else 0)) if self.wide else 0
        sums = list(range(self.RS, self.RS + 4 * NR)) if rs else [self.LS0, self.LS1]
        self.CLOBBER_V = (list(range(self.SA, self.KOFF)) + sums + list(range(self.DK, self.DV + npar)) +
                          ([self.ROW1] if self.dual else []) + list(range(min(self.RT, self.T), self.NVGPR)))


def vr(a: int, n: int = 1) -> str:
    return f"v{a}" if n == 1 else f"v[{a}:{a + n - 1}]"


def ar(a: int, n: int = 1) -> str:
    return f"a{a}" if n == 1 else f"a[{a}:{a + n - 1}]"


def sr(a: int, n: int = 1) -> str:
    return f"s{a}" if n == 1 else f"s[{a}:{a + n - 1}]"


def lbl(name: str) -> str:
    return f"{name}_%="


class Gen:
    def __init__(self, dt: str, D: int = 128, nw: int = 8, always_rare: bool = False,
                 la: int | None = None, order: str = "group",
                 lead: int = 0, early_load: bool = False, dot_init: bool = False,
                 and_scc: bool = False, copy_split: bool = False, sm_start: int = 2, rs_mfma: bool = False,
                 wait_pair: bool = False, rs_mix: bool = False, tail_nop: int = 12, tail_split: bool = False,
                 mask_fast: bool = False, mfma_order: str = "alt", copy_every: int = 2, prio: int = 0,
                 dual_copy: tuple = (4, 8), sm_mfma: int | None = None, sm_late: bool = False,
                 dual: bool | None = None):
        assert dt in ("bf16", "f16")
        self.dt = dt
        self.L = Layout(D, nw, rs=rs_mfma, dual=dual)
        self.rs_mfma = rs_mfma          # row sums by two 16x16x32 MFMAs against a ones pattern, no v_dot2
        self.wait_pair = wait_pair      # one LDS wait per two MFMAs (before the even one, for both)
        self.rs_mix = rs_mix            # rs_mfma softmax with the exponentials interleaved one by one
        self.tail_nop = tail_nop        # wait states between the last row-sum MFMA and its VALU read
        self.tail_split = tail_split    # rare test issued one MFMA before its branch
        self.mask_fast = mask_fast      # MASK: one lane mask for all 16 keys when the key split lies outside
        self.mfma_order = mfma_order    # QK / PV order in a sub-iteration: alternate, in pairs, or grouped
        self.copy_every = copy_every    # wide map: MFMAs between a block's copies
        self.prio = prio                # s_setprio prio before each P.V / S MFMA, s_setprio 0 after it
        self.dual_copy = tuple(dual_copy)  # dual map: MFMA of a block's first copy, MFMAs between copies
        self.sm_mfma = sm_mfma          # first MFMA (not item) of a sub-iteration's softmax, when set
        self.sm_late = sm_late          # the softmax spread also after the last item's first MFMAs
        self.always_rare = always_rare  # diagnostics: exact row max on every sub-block
        self.la = (2 if nw == 12 else LA) if la is None else la   # MFMAs of LDS operand lookahead
        assert self.la < self.L.nslot
        self.order = order              # softmax op order: "group" (4 fma, 4 exp) or "mix"
        self.lead = lead                # PV MFMAs that open a block, their V operands read before the barrier
        self.early_load = early_load    # plan entry j+3 loaded in the middle of block j, not after it
        self.dot_init = dot_init        # row-sum chains start with v_dot2 (C = 0) instead of two v_mov
        self.and_scc = and_scc          # mask test branches on the SCC of s_and (no s_cmp)
        self.copy_split = copy_split    # M0 of a copy set one MFMA slot ahead (no s_nop)
        self.sm_start = sm_start        # first MFMA slot of a sub-iteration's softmax (mask test one before)
        self.lines: list[str] = []
        self.stubs: list[str] = []
        self.phase = 0                  # operand slot of the next stream's first MFMA

    def e(self, *ins: str) -> None:
        self.lines.extend(ins)

    def ov(self, a: int, n: int = 1) -> str:
        """O registers: AGPRs in the wide map, VGPRs otherwise."""
        return ar(a, n) if self.L.wide else vr(a, n)

    def qreg(self, h: int, c: int) -> str:
        """Q operand of k-step c for 32-row half h (the dual-wide map keeps half
        1's Q in AGPRs)."""
        L = self.L
        if h == 1 and L.QA is not None:
            return ar(L.QA + 4 * c, 4)
        return vr(L.Q + 4 * L.NQK * h + 4 * c, 4)

    @property
    def mfma(self) -> str:
        return "v_mfma_f32_32x32x16_bf16" if self.dt == "bf16" else "v_mfma_f32_32x32x16_f16"

    def u(self, p: int) -> int:
        """Index of the first MFMA of operand item p (NR MFMAs per item)."""
        return self.L.NR * p

    def ue(self, p: int) -> int:
        """Index of the last MFMA of operand item p."""
        return self.L.NR * p + self.L.NR - 1

    # ── softmax ──
    def softmax_all(self, S: int, P: int) -> list[str]:
        """The softmax of every 32-row half of the (S, P) tiles."""
        return [x for r in range(self.L.NR) for x in self.softmax_ops(S + 16 * r, P + 8 * r, r)]

    def softmax_ops(self, S: int, P: int, r: int = 0) -> list[str]:
        """P = 2^(S*cs - m) as bf16/f16 pairs; this sub-block's row sum in LS0 + LS1
        (half r of the dual map: m in VM + r, the row sum in RS + 4 r)."""
        L = self.L
        cvt = "v_cvt_pk_bf16_f32" if self.dt == "bf16" else "v_cvt_pk_f16_f32"
        one = "0x3f803f80" if self.dt == "bf16" else "0x3c003c00"
        dot = "v_dot2c_f32_bf16" if self.dt == "bf16" else "v_dot2c_f32_f16"
        t = lambda k: L.T + k % L.NT  # noqa: E731   (eight temporaries: groups g and g + 2 share)
        fma = lambda k: f"v_fma_f32 {vr(t(k))}, {vr(S + k)}, {sr(S_CS)}, -{vr(L.VM + r)}"  # noqa: E731
        exp = lambda k: f"v_exp_f32 {vr(t(k))}, {vr(t(k))}"  # noqa: E731
        pk = lambda q: f"{cvt} {vr(P + q)}, {vr(t(2 * q))}, {vr(t(2 * q + 1))}"  # noqa: E731
        dot3 = "v_dot2_f32_bf16" if self.dt == "bf16" else "v_dot2_f32_f16"

        def d2(q: int) -> str:
            if self.dot_init and q < 2:   # first term of each chain: C = 0, the ones pair in S_ONE
                return f"{dot3} {vr(L.LS0 + q)}, {sr(S_ONE)}, {vr(P + q)}, 0"
            return f"{dot} {vr(L.LS0 + (q & 1))}, {one}, {vr(P + q)}"
        if self.rs_mfma:
            # Row sums on the matrix core: P of 16 keys (the B operand layout of the
            # 32x32x16 PV MFMA: lane l = query l%32, keys 8(l/32)..) read as the B
            # operand of v_mfma_f32_16x16x32 is B[k][n] with n = l%16 and k-group
            # l/16 = (key half, query >= 16); the ONES pattern (lanes 0, 32: row 0,
            # k-groups 0, 2; lanes 20, 52: row 4, k-groups 1, 3) puts the full row
            # sum of query l in register 0 of lanes 0-31 (lanes 32-63: zero).
            mf16 = "v_mfma_f32_16x16x32_bf16" if self.dt == "bf16" else "v_mfma_f32_16x16x32_f16"
            RS = L.RS + 4 * r
            rs = lambda h: (f"{mf16} {vr(RS, 4)}, {vr(L.ONES, 4)}, {vr(P + 4 * h, 4)}, "  # noqa: E731
                            f"{'0' if h == 0 else vr(RS, 4)}")
            ops = []
            if self.rs_mix:
                # fma k+2, exp k; the pack of pair q two instructions after exp 2q+1
                ops = [fma(0), fma(1)]
                for k in range(16):
                    if k + 2 < 16:
                        ops.append(fma(k + 2))
                    ops.append(exp(k))
                    if k % 2 == 0 and k >= 2:
                        ops.append(pk(k // 2 - 1))
                    if k == 11:
                        ops.append(rs(0))        # P + 0..3: packed by k = 8
                ops += [pk(7), "s_nop 4", rs(1)]
                return ops
            for g in range(4):
                ops += [fma(4 * g + i) for i in range(4)]
                if g:
                    ops += [pk(2 * g - 2), pk(2 * g - 1)]
                ops += [exp(4 * g + i) for i in range(4)]
                if g == 3:
                    ops.append(rs(0))            # P + 0..3 packed in groups 1 and 2
            ops += [pk(6), pk(7), "s_nop 4", rs(1)]   # VALU write -> MFMA read of the packs
            return ops
        ops = [] if self.dot_init else [f"v_mov_b32 {vr(L.LS0)}, 0", f"v_mov_b32 {vr(L.LS1)}, 0"]
        if self.order == "mix":
            # one exponential between two other ops: fma k+2, exp k; packs and dots
            # trail their exponentials by two
            seq = [fma(0), fma(1)]
            for k in range(16):
                if k + 2 < 16:
                    seq.append(fma(k + 2))
                seq.append(exp(k))
                if k % 2 == 1 and k >= 3:
                    seq.append(pk((k - 3) // 2))
                    seq.append(d2((k - 3) // 2))
            seq += [pk(7), d2(7)]
            return ops + seq
        for g in range(4):
            ops += [fma(4 * g + i) for i in range(4)]
            if g:
                ops += [pk(2 * g - 2), pk(2 * g - 1)]
            ops += [exp(4 * g + i) for i in range(4)]
            if g:
                ops += [d2(2 * g - 2), d2(2 * g - 1)]
        ops += [pk(6), pk(7), d2(6), d2(7)]
        return ops

    def softmax_tail(self, site: str, sset: str) -> list[str]:
        """Rare-case test on this sub-block's row sum, then l += sum.  Runs after
        the last PV MFMA of the sub-iteration, so RARE rescales every
        contribution made with the old m."""
        L = self.L
        self.stubs += [f"{lbl('RSTUB_' + site)}:", f"s_call_b64 {sr(S_RET, 2)}, {lbl('RARE_' + sset)}",
                       f"s_branch {lbl('RRET_' + site)}"]
        if L.NR == 2:
            # either half's row sum over 2^8 (or NaN) takes the rare path for both
            return ["s_nop 7"] + ([f"s_nop {self.tail_nop - 9}"] if self.tail_nop > 8 else []) + [
                f"v_cmp_nge_f32 vcc, 0x43800000, {vr(L.RS + 4)}",
                "s_mov_b64 s[78:79], vcc",
                f"v_cmp_nge_f32 vcc, 0x43800000, {vr(L.RS)}",
                "s_or_b64 vcc, vcc, s[78:79]",
                (f"s_branch {lbl('RSTUB_' + site)}" if self.always_rare else
                 f"s_cbranch_vccnz {lbl('RSTUB_' + site)}"),
                f"{lbl('RRET_' + site)}:",
                f"v_add_f32 {vr(L.VL)}, {vr(L.VL)}, {vr(L.RS)}",
                f"v_add_f32 {vr(L.VL + 1)}, {vr(L.VL + 1)}, {vr(L.RS + 4)}"]
        if self.rs_mfma:                                       # 16x16x32 MFMA result -> VALU
            head = ["s_nop 7"] + ([f"s_nop {self.tail_nop - 9}"] if self.tail_nop > 8 else [])
        else:
            head = ["s_nop 2",                                 # dot2 result -> VALU: 3 states
                    f"v_add_f32 {vr(L.LS0)}, {vr(L.LS0)}, {vr(L.LS1)}"]
        return head + [
                f"v_cmp_nge_f32 vcc, 0x43800000, {vr(L.LS0)}",    # !(256 >= ls): ls > 256 or NaN
                (f"s_branch {lbl('RSTUB_' + site)}" if self.always_rare else
                 f"s_cbranch_vccnz {lbl('RSTUB_' + site)}"),
                f"{lbl('RRET_' + site)}:",
                f"v_add_f32 {vr(L.VL)}, {vr(L.VL)}, {vr(L.LS0)}"]

    def place_softmax(self, fill: dict[int, list[str]], S: int, P: int, slots: list[int], at: int,
                      site: str, sset: str) -> None:
        """The softmax of (S, P) spread over `slots`, its rare test and branch after
        MFMA `at`.  With tail_split the compare ends the spread ops (one MFMA and its
        operand reads before the branch, so the branch does not wait on it)."""
        tail = self.softmax_tail(site, sset)
        if self.tail_split:
            # the compares (up to the last instruction that sets vcc) end the spread ops
            k = 1 + max(i for i, x in enumerate(tail) if x.startswith(("v_cmp_nge_f32", "s_or_b64 vcc")))
            self.spread(self.softmax_all(S, P) + tail[:k], slots, fill)
            fill.setdefault(at, []).extend(tail[k:])
        else:
            self.spread(self.softmax_all(S, P), slots, fill)
            fill.setdefault(at, []).extend(tail)

    def mask_check(self, site: str, sset: str, desc: int, half: int) -> list[str]:
        self.stubs += [f"{lbl('MSTUB_' + site)}:", f"s_mov_b32 s91, {sr(desc)}", f"s_mov_b32 s75, {32 * half}",
                       f"s_call_b64 {sr(S_RET, 2)}, {lbl('MASK_' + sset)}", f"s_branch {lbl('MRET_' + site)}"]
        test = [f"s_and_b32 s74, {sr(desc)}, 3"] + ([] if self.and_scc else ["s_cmp_lg_u32 s74, 0"])
        return test + [f"s_cbranch_scc1 {lbl('MSTUB_' + site)}", f"{lbl('MRET_' + site)}:"]

    def rare_routine(self, S: int, P: int, name: str) -> list[str]:
        """True row max of the sub-block, m -> max(m, max*cs), O and l rescaled, P
        recomputed (the dual map: each 32-row half in turn, then both softmaxes)."""
        r = [f"{lbl(name)}:", "s_nop 15", "s_nop 7"]
        for h in range(self.L.NR):
            r += self.rare_half(S + 16 * h, h)
        r += self.softmax_all(S, P)
        if self.rs_mfma:
            r += ["s_nop 7", "s_nop 3", f"s_setpc_b64 {sr(S_RET, 2)}"]
        else:
            r += ["s_nop 2", f"v_add_f32 {vr(self.L.LS0)}, {vr(self.L.LS0)}, {vr(self.L.LS1)}",
                  f"s_setpc_b64 {sr(S_RET, 2)}"]
        return r

    def rare_half(self, S: int, h: int) -> list[str]:
        """Row max of the S tile of 32-row half h, its m (VM + h) moved, its l
        (VL + h) and O tiles scaled by alpha = 2^(m - m_new)."""
        L = self.L
        RT = L.RT
        VM, VL = L.VM + h, L.VL + h
        r = [f"v_max3_f32 {vr(RT)}, {vr(S)}, {vr(S + 1)}, {vr(S + 2)}",
             f"v_max3_f32 {vr(RT + 1)}, {vr(S + 3)}, {vr(S + 4)}, {vr(S + 5)}",
             f"v_max3_f32 {vr(RT + 2)}, {vr(S + 6)}, {vr(S + 7)}, {vr(S + 8)}",
             f"v_max3_f32 {vr(RT + 3)}, {vr(S + 9)}, {vr(S + 10)}, {vr(S + 11)}",
             f"v_max3_f32 {vr(RT)}, {vr(RT)}, {vr(S + 12)}, {vr(S + 13)}",
             f"v_max3_f32 {vr(RT + 1)}, {vr(RT + 1)}, {vr(S + 14)}, {vr(S + 15)}",
             f"v_max3_f32 {vr(RT)}, {vr(RT)}, {vr(RT + 1)}, {vr(RT + 2)}",
             f"v_max_f32 {vr(RT)}, {vr(RT)}, {vr(RT + 3)}",
             f"v_mov_b32 {vr(RT + 1)}, {vr(RT)}",
             "s_nop 1",
             f"v_permlane32_swap_b32 {vr(RT)}, {vr(RT + 1)}",
             "s_nop 1",
             f"v_max_f32 {vr(RT)}, {vr(RT)}, {vr(RT + 1)}",       # row max over both lane halves
             f"v_mul_f32 {vr(RT)}, {sr(S_CS)}, {vr(RT)}",
             f"v_max_f32 {vr(RT)}, {vr(VM)}, {vr(RT)}",           # m_new
             f"v_sub_f32 {vr(RT + 1)}, {vr(VM)}, {vr(RT)}",
             f"v_exp_f32 {vr(RT + 1)}, {vr(RT + 1)}",             # alpha = 2^(m - m_new)
             f"v_mov_b32 {vr(VM)}, {vr(RT)}",
             "s_nop 0",
             f"v_mul_f32 {vr(VL)}, {vr(RT + 1)}, {vr(VL)}"]
        O = L.O + 16 * L.NDT * h
        if L.wide:
            # O in AGPRs: read, scale and write back through the softmax
            # temporaries, eight at a time (free until P is recomputed)
            for k0 in range(0, 16 * L.NDT, 8):
                r += [f"v_accvgpr_read_b32 {vr(L.T + i)}, {ar(O + k0 + i)}" for i in range(8)]
                r += [f"v_mul_f32 {vr(L.T + i)}, {vr(RT + 1)}, {vr(L.T + i)}" for i in range(8)]
                r += [f"v_accvgpr_write_b32 {ar(O + k0 + i)}, {vr(L.T + i)}" for i in range(8)]
        else:
            r += [f"v_mul_f32 {vr(O + k)}, {vr(RT + 1)}, {vr(O + k)}" for k in range(16 * L.NDT)]
        return r

    def mask_routine(self, S: int, name: str) -> list[str]:
        """-inf on the keys a two-part descriptor (s91) excludes, for sub-block half s75/32.

        Row part b = tile rows >= qs; keys below kb take the part's lo bit, the rest
        its hi bit (bits a.lo, a.hi, b.lo, b.hi).  Element k of the sub-block holds key
        32*half + 8*(k/4) + 4*h + k%4."""
        L = self.L
        if L.NR == 2:
            return self.mask_routine_dual(S, name)
        r = [f"{lbl(name)}:",
             "s_bfe_u32 s88, s91, 0x80008",       # kb
             "s_bfe_u32 s89, s91, 0x90010",       # qs (9 bits: tiles of up to 384 rows)
             "s_bfe_u32 s90, s91, 0x40002",       # allow bits
             "s_sub_u32 s88, s88, s75",
             f"v_cmp_ge_u32_e64 s[78:79], {vr(L.ROW)}, s89",   # lanes of part b
             "s_bitcmp1_b32 s90, 0", "s_cselect_b64 s[92:93], -1, 0", "s_andn2_b64 s[92:93], s[92:93], s[78:79]",
             "s_bitcmp1_b32 s90, 2", "s_cselect_b64 s[94:95], -1, 0", "s_and_b64 s[94:95], s[94:95], s[78:79]",
             "s_or_b64 s[80:81], s[92:93], s[94:95]",      # lanes whose lo keys are allowed
             "s_bitcmp1_b32 s90, 1", "s_cselect_b64 s[92:93], -1, 0", "s_andn2_b64 s[92:93], s[92:93], s[78:79]",
             "s_bitcmp1_b32 s90, 3", "s_cselect_b64 s[94:95], -1, 0", "s_and_b64 s[94:95], s[94:95], s[78:79]",
             "s_or_b64 s[82:83], s[92:93], s[94:95]",      # lanes whose hi keys are allowed
             f"v_sub_u32 {vr(L.VT)}, s88, {vr(L.H4)}"]      # kb - 32*half - 4h
        if self.mask_fast:
            # key split outside this sub-block: all its keys are lo (kb - 32*half >= 32)
            # or all hi (<= 0), so one lane mask (the allowed part) covers every key,
            # and a mask of all lanes needs nothing at all
            lo, hi, one, ret = (lbl(name + x) for x in ("_LO", "_HI", "_ONE", "_RET"))
            r += ["s_cmp_ge_i32 s88, 32", f"s_cbranch_scc1 {lo}", "s_cmp_le_i32 s88, 0", f"s_cbranch_scc1 {hi}"]
            tail = [f"{lo}:", "s_mov_b64 s[84:85], s[80:81]", f"s_branch {one}",
                    f"{hi}:", "s_mov_b64 s[84:85], s[82:83]",
                    f"{one}:", "s_cmp_eq_u64 s[84:85], -1", f"s_cbranch_scc1 {ret}", "s_nop 0"]
            tail += [f"v_cndmask_b32_e64 {vr(S + k)}, {vr(L.NEGINF)}, {vr(S + k)}, s[84:85]" for k in range(16)]
            tail += [f"{ret}:", f"s_setpc_b64 {sr(S_RET, 2)}"]
        else:
            tail = []
        for k in range(16):
            ck = 8 * (k // 4) + (k % 4)
            r += [f"v_cmp_lt_i32 vcc, {ck}, {vr(L.VT)}",    # key below kb
                  "s_and_b64 s[84:85], vcc, s[80:81]",
                  "s_andn2_b64 s[86:87], s[82:83], vcc",
                  "s_or_b64 s[84:85], s[84:85], s[86:87]",
                  "s_nop 0",
                  f"v_cndmask_b32_e64 {vr(S + k)}, {vr(L.NEGINF)}, {vr(S + k)}, s[84:85]"]
        r += [f"s_setpc_b64 {sr(S_RET, 2)}"]
        return r + tail

    def mask_routine_dual(self, S: int, name: str) -> list[str]:
        """MASK of the dual map: the key split is shared, the row split applies to
        each 32-row half (tile rows in ROW and ROW1) in turn."""
        L = self.L

        def keys(Sh: int) -> list[str]:
            r = []
            for k in range(16):
                ck = 8 * (k // 4) + (k % 4)
                r += [f"v_cmp_lt_i32 vcc, {ck}, {vr(L.VT)}",    # key below kb
                      "s_and_b64 s[84:85], vcc, s[80:81]",
                      "s_andn2_b64 s[86:87], s[82:83], vcc",
                      "s_or_b64 s[84:85], s[84:85], s[86:87]",
                      "s_nop 0",
                      f"v_cndmask_b32_e64 {vr(Sh + k)}, {vr(L.NEGINF)}, {vr(Sh + k)}, s[84:85]"]
            return r
        r = [f"{lbl(name)}:",
             "s_bfe_u32 s88, s91, 0x80008",       # kb
             "s_bfe_u32 s89, s91, 0x90010",       # qs
             "s_bfe_u32 s90, s91, 0x40002",       # allow bits
             "s_sub_u32 s88, s88, s75",
             f"v_sub_u32 {vr(L.VT)}, s88, {vr(L.H4)}"]      # kb - 32*half - 4h
        for h, row in enumerate((L.ROW, L.ROW1)):
            Sh = S + 16 * h
            r += [f"v_cmp_ge_u32_e64 s[78:79], {vr(row)}, s89",   # lanes of part b
                  "s_bitcmp1_b32 s90, 0", "s_cselect_b64 s[92:93], -1, 0", "s_andn2_b64 s[92:93], s[92:93], s[78:79]",
                  "s_bitcmp1_b32 s90, 2", "s_cselect_b64 s[94:95], -1, 0", "s_and_b64 s[94:95], s[94:95], s[78:79]",
                  "s_or_b64 s[80:81], s[92:93], s[94:95]",      # lanes whose lo keys are allowed
                  "s_bitcmp1_b32 s90, 1", "s_cselect_b64 s[92:93], -1, 0", "s_andn2_b64 s[92:93], s[92:93], s[78:79]",
                  "s_bitcmp1_b32 s90, 3", "s_cselect_b64 s[94:95], -1, 0", "s_and_b64 s[94:95], s[94:95], s[78:79]",
                  "s_or_b64 s[82:83], s[92:93], s[94:95]"]      # lanes whose hi keys are allowed
            if not self.mask_fast:
                r += keys(Sh)
                continue
            # key split outside this sub-block: one lane mask covers every key
            lo, hi, one, nxt = (lbl(f"{name}_{x}{h}") for x in ("LO", "HI", "ONE", "NEXT"))
            r += ["s_cmp_ge_i32 s88, 32", f"s_cbranch_scc1 {lo}", "s_cmp_le_i32 s88, 0", f"s_cbranch_scc1 {hi}"]
            r += keys(Sh)
            r += [f"s_branch {nxt}",
                  f"{lo}:", "s_mov_b64 s[84:85], s[80:81]", f"s_branch {one}",
                  f"{hi}:", "s_mov_b64 s[84:85], s[82:83]",
                  f"{one}:", "s_cmp_eq_u64 s[84:85], -1", f"s_cbranch_scc1 {nxt}", "s_nop 0"]
            r += [f"v_cndmask_b32_e64 {vr(Sh + k)}, {vr(L.NEGINF)}, {vr(Sh + k)}, s[84:85]" for k in range(16)]
            r += [f"{nxt}:"]
        return r + [f"s_setpc_b64 {sr(S_RET, 2)}"]

    # ── copies ──
    def decode(self, x: int, site: str) -> list[str]:
        """Copy offsets of the block named by entry word x.  The buffer resources
        span a whole key source (rows past its end read zeros), so a block only
        moves the soffsets; a change of source (video <-> extra rows) calls SWITCH."""
        self.stubs += [f"{lbl('SWSTUB_' + site)}:", f"s_call_b64 {sr(S_RET, 2)}, {lbl('SWITCH')}",
                       f"s_branch {lbl('SWRET_' + site)}"]
        chk = [f"s_lshr_b32 s74, {sr(x)}, 31", f"s_cmp_lg_u32 s74, {sr(S_CUR)}",
               f"s_cbranch_scc1 {lbl('SWSTUB_' + site)}"]
        r = chk + [
            f"{lbl('SWRET_' + site)}:",
            f"s_and_b32 s73, {sr(x)}, 0x7fffffff",
            "s_lshl_b32 s73, s73, 6",                                  # first row of the block
            f"s_mul_i32 {sr(S_SOK)}, s73, {sr(S_KRSC)}",
        ]
        if self.L.NCP == 2:
            r.append(f"s_add_u32 {sr(S_SOK + 1)}, {sr(S_SOK)}, {sr(S_KRSC + 2)}")  # + 32 rows
        r.append(f"s_mul_i32 {sr(S_SOV)}, s73, {sr(S_KRSC + 1)}")
        if self.L.NCP == 2:
            r.append(f"s_add_u32 {sr(S_SOV + 1)}, {sr(S_SOV)}, {sr(S_KRSC + 3)}")
        return r

    def decode_wide(self, x: int, site: str, v: bool) -> list[str]:
        """Wide map: soffsets of the K (or V) copies of the block named by entry
        word x, copy ii taking rows 16*(ii >> 1) on (four soffsets).  K and V of
        one iteration belong to different blocks, so each tensor tracks its own
        key source (SWITCHK / SWITCHV)."""
        t = "V" if v else "K"
        cur, so, stride, st16 = (S_CURV, S_SOVW, S_KRSC + 1, S_KRSC + 3) if v else (S_CUR, S_SOK, S_KRSC, S_KRSC + 2)
        self.stubs += [f"{lbl(f'SWSTUB{t}_' + site)}:", f"s_call_b64 {sr(S_RET, 2)}, {lbl('SWITCH' + t)}",
                       f"s_branch {lbl(f'SWRET{t}_' + site)}"]
        r = [f"s_lshr_b32 s74, {sr(x)}, 31", f"s_cmp_lg_u32 s74, {sr(cur)}",
             f"s_cbranch_scc1 {lbl(f'SWSTUB{t}_' + site)}",
             f"{lbl(f'SWRET{t}_' + site)}:",
             f"s_and_b32 s73, {sr(x)}, 0x7fffffff",
             "s_lshl_b32 s73, s73, 6",                                  # first row of the block
             f"s_mul_i32 {sr(so)}, s73, {sr(stride)}"]
        r += [f"s_add_u32 {sr(so + i)}, {sr(so + i - 1)}, {sr(st16)}" for i in range(1, 4)]   # + 16 rows
        return r

    def switch_wide(self, v: bool) -> list[str]:
        """Wide map: buffer resource, row stride, 16-row stride and the lane copy
        offsets (both parities) of K (or V) for key source s74."""
        L = self.L
        t = "V" if v else "K"
        cur, rs, st, st16, kb, off = ((S_CURV, S_RV, S_KRSC + 1, S_KRSC + 3, (S_VB0, S_VB1), L.DV) if v else
                                      (S_CUR, S_RK, S_KRSC, S_KRSC + 2, (S_KB0, S_KB1), L.DK))
        srs = (S_VRS0, S_VRS1) if v else (S_KRS0, S_KRS1)
        return [
            f"{lbl('SWITCH' + t)}:",
            f"s_mov_b32 {sr(cur)}, s74",
            "s_cmp_eq_u32 s74, 0",
            f"s_cselect_b32 s75, {sr(S_NK)}, {sr(S_NX)}",
            f"s_cselect_b32 {sr(st)}, {sr(srs[0])}, {sr(srs[1])}",
            f"s_cselect_b64 {sr(rs, 2)}, {sr(kb[0], 2)}, {sr(kb[1], 2)}",
            f"s_and_b32 {sr(rs + 1)}, {sr(rs + 1)}, 0xffff",
            f"s_mul_i32 {sr(rs + 2)}, s75, {sr(st)}",
            f"s_mov_b32 {sr(rs + 3)}, 0x20000",
            f"s_lshl_b32 {sr(st16)}, {sr(st)}, 4",
            f"v_mad_u32_u24 {vr(off)}, {vr(L.DMAROW)}, {sr(st)}, {vr(L.C16)}",
            f"v_mad_u32_u24 {vr(off + 1)}, {vr(L.DMAROW + 2)}, {sr(st)}, {vr(L.C16 + 2)}",
            "s_nop 1",
            f"s_setpc_b64 {sr(S_RET, 2)}",
        ]

    def switch_routine(self) -> list[str]:
        """Buffer resources, row strides and lane copy offsets of key source s74."""
        L = self.L
        return [
            f"{lbl('SWITCH')}:",
            f"s_mov_b32 {sr(S_CUR)}, s74",
            "s_cmp_eq_u32 s74, 0",
            f"s_cselect_b32 s68, {sr(S_NK)}, {sr(S_NX)}",
            f"s_cselect_b32 {sr(S_KRSC)}, {sr(S_KRS0)}, {sr(S_KRS1)}",
            f"s_cselect_b32 {sr(S_KRSC + 1)}, {sr(S_VRS0)}, {sr(S_VRS1)}",
            f"s_cselect_b64 {sr(S_RK, 2)}, {sr(S_KB0, 2)}, {sr(S_KB1, 2)}",
            f"s_cselect_b64 {sr(S_RV, 2)}, {sr(S_VB0, 2)}, {sr(S_VB1, 2)}",
            f"s_and_b32 {sr(S_RK + 1)}, {sr(S_RK + 1)}, 0xffff",
            f"s_and_b32 {sr(S_RV + 1)}, {sr(S_RV + 1)}, 0xffff",
            f"s_mul_i32 {sr(S_RK + 2)}, s68, {sr(S_KRSC)}",
            f"s_mov_b32 {sr(S_RK + 3)}, 0x20000",
            f"s_mul_i32 {sr(S_RV + 2)}, s68, {sr(S_KRSC + 1)}",
            f"s_mov_b32 {sr(S_RV + 3)}, 0x20000",
            f"s_lshl_b32 {sr(S_KRSC + 2)}, {sr(S_KRSC)}, 5",
            f"s_lshl_b32 {sr(S_KRSC + 3)}, {sr(S_KRSC + 1)}, 5",
            f"v_mad_u32_u24 {vr(L.DK)}, {vr(L.DMAROW)}, {sr(S_KRSC)}, {vr(L.C16)}",
            f"v_mad_u32_u24 {vr(L.DV)}, {vr(L.DMAROW)}, {sr(S_KRSC + 1)}, {vr(L.C16)}",
            "s_nop 1",
            f"s_setpc_b64 {sr(S_RET, 2)}",
        ]

    def copy(self, stage: int, k: int) -> list[str]:
        """Copy instruction k of a block into `stage`: the first NCP copy K, the
        rest V; copy ii of a tensor fills LDS KiB 8*ii + wave of the block, i.e.
        rows 32*ii + 4*wave + lane/16 (D = 128) or 8*wave + lane/8 (D = 64)."""
        L = self.L
        v, ii = k // L.NCP, k % L.NCP
        rs = S_RV if v else S_RK
        if L.wide:
            # copy ii of wave w fills LDS KiB 4*ii + w of the block: rows
            # 8*ii + 2*w + lane/32; rows 16*(ii >> 1) in the soffset, the rest
            # (and the swizzle, which depends on ii's parity) in the lane offset
            lds = (L.VBASE if v else 0) + stage * L.TILE + ii * 4096
            so = sr((S_SOVW if v else S_SOK) + (ii >> 1))
            lane = (L.DV if v else L.DK) + (ii & 1)
        else:
            lds = (L.VBASE if v else 0) + stage * L.TILE + ii * L.CPROWS * L.RB
            so = sr((S_SOV if v else S_SOK) + ii)
            lane = L.DV if v else L.DK
        return [f"s_add_u32 m0, {sr(S_LDSK)}, {lds}", "s_nop 0",
                f"buffer_load_dwordx4 {vr(lane)}, {sr(rs, 4)}, {so} offen lds"]

    def place_copy(self, fill: dict[int, list[str]], at: int, stage: int, k: int) -> None:
        """Copy k of a block after MFMA `at`; with copy_split, its M0 is set after
        MFMA at - 1 (an MFMA and its operand reads in between cover the M0 ->
        LDS-copy wait state)."""
        c = self.copy(stage, k)
        if self.copy_split and at > 0:
            fill.setdefault(at - 1, []).append(c[0])
            fill.setdefault(at, []).append(c[2])
        else:
            fill.setdefault(at, []).extend(c)

    # ── an MFMA stream with its operand reads and the interleaved work ──
    def stream(self, mfmas: list[tuple], fill: dict[int, list[str]], pre: int = 0,
               nxt: list[tuple] = ()) -> None:
        """mfmas: ("qk", stage, half, c, S) or ("pv", stage, st16, dt, P), one
        operand item each, issued as NR MFMAs (one per 32-row half of the wave: S +
        16 r with the half's Q, or the half's O with P + 8 r) sharing the operand.
        fill[m]: instructions emitted right after MFMA m (item m // NR).  The LDS
        operands of item i go to slot i % nslot and are read `la` items ahead.  The
        operands of the first `pre` items were read by the previous stream; `nxt`
        are the first items of the next stream, whose operands this one reads as if
        they followed it."""
        L = self.L
        seq = list(mfmas) + list(nxt)
        n, nn = len(mfmas), len(seq)
        LA = self.la
        nreads = [1 if m[0] == "qk" else 2 for m in seq]

        def reads(i: int) -> list[str]:
            m = seq[i]
            slot = slot_of(i)
            if m[0] == "qk":
                _, st, half, c, _ = m
                return [f"ds_read_b128 {vr(slot, 4)}, {vr(L.KOFF + c)} offset:{st * L.TILE + half * 32 * L.RB}"]
            _, st, st16, dt, _ = m
            off = st * L.TILE + st16 * 16 * L.RB    # the V^T read offsets include VBASE
            return [f"ds_read_b64_tr_b16 {vr(slot, 2)}, {vr(L.VOFFA + dt)} offset:{off}",
                    f"ds_read_b64_tr_b16 {vr(slot + 2, 2)}, {vr(L.VOFFB + dt)} offset:{off}"]

        ph = self.phase

        def slot_of(i: int) -> int:
            return L.OPS + 4 * ((ph + i) % L.nslot)

        issued = min(LA + pre, n)
        for i in range(pre, issued):
            self.e(*reads(i))
        for i in range(n):
            if not self.wait_pair:
                pending = sum(nreads[j] for j in range(max(i + 1, pre), issued))
                self.e(f"s_waitcnt lgkmcnt({min(15, pending)})")
            elif i >= pre and (i - pre) % 2 == 0:
                # one wait for the operands of MFMAs i and i + 1 (the pre-read ones need none)
                last = i + 1 if i + 1 < n else i
                pending = sum(nreads[j] for j in range(last + 1, issued))
                self.e(f"s_waitcnt lgkmcnt({min(15, pending)})")
            m = mfmas[i]
            slot = slot_of(i)
            for h in range(L.NR):
                if self.prio:
                    self.e(f"s_setprio {self.prio}")
                if m[0] == "qk":
                    _, _, _, c, S = m
                    S += 16 * h
                    q = self.qreg(h, c)
                    self.e(f"{self.mfma} {vr(S, 16)}, {vr(slot, 4)}, {q}, {'0' if c == 0 else vr(S, 16)}")
                else:
                    _, _, st16, dt, P = m
                    acc = self.ov(L.O + 16 * L.NDT * h + 16 * dt, 16)
                    self.e(f"{self.mfma} {acc}, {vr(slot, 4)}, {vr(P + 8 * h + 4 * (st16 & 1), 4)}, {acc}")
                if self.prio:
                    self.e("s_setprio 0")
                if h == 0:
                    while issued < min(nn, i + 1 + LA):
                        self.e(*reads(issued))
                        issued += 1
                self.e(*fill.get(L.NR * i + h, []))
        while issued < nn:                # the next stream's operands not yet read
            self.e(*reads(issued))
            issued += 1
        # the next stream's MFMA k takes the slot this one gave item n + k
        self.phase = (ph + n) % L.nslot

    @staticmethod
    def spread(ops: list[str], slots: list[int], fill: dict[int, list[str]]) -> None:
        per = -(-len(ops) // len(slots))
        for i, s in enumerate(slots):
            fill.setdefault(s, []).extend(ops[i * per:(i + 1) * per])

    def entry_load(self, stage: int) -> list[str]:
        """Scalar load of entry j+3 (clamped to the last) into the ring slot of entry j-1."""
        return [f"s_add_u32 s74, {sr(S_J)}, 3", f"s_min_u32 s74, s74, {sr(S_NM1)}", "s_lshl_b32 s74, s74, 3",
                f"s_load_dwordx2 {sr(S_ENT + 2 * ((stage + 3) & 3), 2)}, {sr(S_EPTR, 2)}, s74"]

    def iteration_tail(self, stage: int, load: bool = True) -> None:
        """Scalar load of entry j+3 (unless issued earlier), j += 1, leave for the
        drain after the last block."""
        if load:
            self.e(*self.entry_load(stage))
        self.e(f"s_add_u32 {sr(S_J)}, {sr(S_J)}, 1", f"s_cmp_ge_u32 {sr(S_J)}, {sr(S_N)}",
               f"s_cbranch_scc1 {lbl(f'DRAIN{stage}')}")

    def lead_pv(self, stage: int) -> list[tuple]:
        """The PV MFMAs that open the block after the one in `stage` (V of that block,
        first 16 keys): their operands are read before the barrier."""
        return [("pv", stage, 0, dt, self.L.PA) for dt in range(min(self.lead, self.L.NDT))]

    def iteration(self, stage: int) -> None:
        """Block j: QK of its two sub-blocks (K in `stage`), softmax of sub-blocks
        2j-1 and 2j, PV of block j-1 (V in stage-1), copies of block j+2."""
        L = self.L
        vst, cst = (stage + 3) & 3, (stage + 2) & 3       # entry slots of blocks j-1 and j+2
        # LDS stages of K(j) and V(j-1) (wide: two-stage rings of their own)
        kld, vld = (stage & 1, (stage + 1) & 1) if L.wide else (stage, vst)
        site = f"I{stage}"
        M = 2 * L.NQK                     # MFMAs per sub-iteration (QK and PV interleaved)
        self.e(f"; ── block j, K stage {stage}", f"s_waitcnt vmcnt({0 if L.wide else 2 * L.NCP})",
               "s_barrier", "s_waitcnt lgkmcnt(0)")
        mf = []
        half_q = L.NQK // 2               # QK k-steps per 16-key PV step
        for half, S, P in ((0, L.SA, L.PA), (1, L.SB, L.PB)):
            qks = [("qk", kld, half, c, S) for c in range(L.NQK)]
            pvs = [("pv", vld, 2 * half + c // half_q, c % L.NDT, P) for c in range(L.NQK)]
            lead = len(self.lead_pv(vst)) if half == 0 else 0
            mf += pvs[:lead]
            rest = pvs[lead:]
            if self.mfma_order == "group":
                mf += qks + rest
                continue
            step = 2 if self.mfma_order == "pair" else 1
            for c in range(0, L.NQK, step):
                mf += qks[c:c + step] + rest[c:c + step]
            mf += rest[L.NQK:]
        assert mf[:len(self.lead_pv(vst))] == self.lead_pv(vst)
        if L.wide:
            # K(j+1) into the K stage K(j-1) left, V(j) into the V stage V(j-2) left
            fill = {0: self.decode_wide(S_ENT + 2 * ((stage + 1) & 3), site, False) +
                    self.decode_wide(S_ENT + 2 * stage, site, True)}
            for k in range(2 * L.NCP):
                self.place_copy(fill, self.u(1 + self.copy_every * k), (stage + 1) & 1 if k < L.NCP else stage & 1, k)
        else:
            fill = {0: self.decode(S_ENT + 2 * cst, site)}
            # copies after MFMAs spread over the block's 4*NQK*NR MFMAs
            if L.dual:
                at_copy = tuple(self.dual_copy[0] + self.dual_copy[1] * k for k in range(2 * L.NCP))
            else:
                at_copy = {8: (6, 10, 22, 26), 6: (4, 8, 16, 20), 4: (5, 13)}[L.NQK]
            for k, at in enumerate(at_copy):
                self.place_copy(fill, at, cst, k)
        u, ue = self.u, self.ue
        # MFMA slots of a sub-iteration's softmax (from its start to the last
        # item's first MFMA) and of its mask test (the slot before)
        s0 = u(self.sm_start) if self.sm_mfma is None else self.sm_mfma
        s1 = ue(M - 1) if self.sm_late else u(M - 1)
        # sub-iteration a: softmax of sub-block 2j-1 (S_B, block j-1 half 1)
        fill.setdefault(s0 - 1, []).extend(self.mask_check(site + "a", "B", S_ENT + 2 * vst + 1, 1))
        self.place_softmax(fill, L.SB, L.PB, list(range(s0, s1)), ue(M - 1), site + "a", "B")
        # sub-iteration b: softmax of sub-block 2j (S_A, block j half 0)
        if self.early_load:
            fill.setdefault(u(M), []).extend(self.entry_load(stage))
        fill.setdefault(u(M) + s0 - 1, []).extend(self.mask_check(site + "b", "A", S_ENT + 2 * stage + 1, 0))
        self.place_softmax(fill, L.SA, L.PA, list(range(u(M) + s0, u(M) + s1)), ue(2 * M - 1), site + "b", "A")
        lead = self.lead_pv(vst)
        self.stream(mf, fill, pre=len(lead), nxt=self.lead_pv(stage))
        self.iteration_tail(stage, load=not self.early_load)

    def first_iteration(self) -> None:
        """Block 0: QK of its two sub-blocks, softmax of sub-block 0, copies of block 2."""
        L = self.L
        self.e("; ── block 0", f"s_waitcnt vmcnt({0 if L.wide else 2 * L.NCP})", "s_barrier", "s_waitcnt lgkmcnt(0)")
        mf = [("qk", 0, 0, c, L.SA) for c in range(L.NQK)] + [("qk", 0, 1, c, L.SB) for c in range(L.NQK)]
        if L.wide:
            # K(1) into K stage 1, V(0) into V stage 0, spread over the block's QK MFMAs
            fill = {0: self.decode_wide(S_ENT + 2, "F", False) + self.decode_wide(S_ENT, "F", True)}
            n = len(mf)
            for k in range(2 * L.NCP):
                self.place_copy(fill, self.u(1 + (k * (n - 2)) // (2 * L.NCP - 1)), 1 if k < L.NCP else 0, k)
        else:
            fill = {0: self.decode(S_ENT + 4, "F")}
            for k in range(2 * L.NCP):
                self.place_copy(fill, 1 + k, 2, k)
        u, ue = self.u, self.ue
        fill.setdefault(ue(L.NQK + 1), []).extend(self.mask_check("F", "A", S_ENT + 1, 0))
        self.place_softmax(fill, L.SA, L.PA, list(range(u(L.NQK + 2), u(2 * L.NQK - 1))), ue(2 * L.NQK - 1),
                           "F", "A")
        self.stream(mf, fill, nxt=self.lead_pv(0))
        self.iteration_tail(0)

    def drain(self, stage: int) -> None:
        """After block n-1 (in `stage`): softmax of sub-block 2n-1, PV of block n-1."""
        L = self.L
        self.e(f"{lbl(f'DRAIN{stage}')}:")
        vld = stage & 1 if L.wide else stage
        if L.wide:
            # V(n-1) was copied during block n-1: wait for every wave's copies
            self.e("s_waitcnt vmcnt(0)", "s_barrier")
        nh = L.NQK                        # PV MFMAs per half: 2 16-key steps x NDT d-tiles
        mf = [("pv", vld, k // L.NDT, k % L.NDT, L.PA) for k in range(nh)] + \
             [("pv", vld, 2 + k // L.NDT, k % L.NDT, L.PB) for k in range(nh)]
        fill: dict[int, list[str]] = {0: self.mask_check(f"D{stage}", "B", S_ENT + 2 * stage + 1, 1)}
        self.place_softmax(fill, L.SB, L.PB, list(range(self.u(1), self.u(nh - 1))), self.ue(nh - 1),
                           f"D{stage}", "B")
        self.stream(mf, fill)
        # the code after the asm reads O with VALU: 12 states after the last MFMA
        self.e("s_waitcnt vmcnt(0) lgkmcnt(0)", "s_nop 15", f"s_branch {lbl('END')}")

    def build(self) -> list[str]:
        L = self.L
        e = self.e
        # setup: entries 0..2 (clamped to the last block), copies of blocks 0 and 1
        if L.dual:
            e(f"v_add_u32 {vr(L.ROW1)}, 32, {vr(L.ROW)}")
        if self.dot_init:
            e(f"s_mov_b32 {sr(S_ONE)}, {'0x3f803f80' if self.dt == 'bf16' else '0x3c003c00'}")
        e(f"s_sub_u32 {sr(S_NM1)}, {sr(S_N)}, 1",
          f"s_load_dwordx2 {sr(S_ENT, 2)}, {sr(S_EPTR, 2)}, 0x0",
          f"s_min_u32 s74, {sr(S_NM1)}, 1", "s_lshl_b32 s74, s74, 3",
          f"s_load_dwordx2 {sr(S_ENT + 2, 2)}, {sr(S_EPTR, 2)}, s74",
          f"s_min_u32 s74, {sr(S_NM1)}, 2", "s_lshl_b32 s74, s74, 3",
          f"s_load_dwordx2 {sr(S_ENT + 4, 2)}, {sr(S_EPTR, 2)}, s74",
          f"s_mov_b32 {sr(S_J)}, 0",
          f"s_mov_b32 {sr(S_CUR)}, 2",
          "s_waitcnt lgkmcnt(0)")
        if L.wide:
            # K(0) into K stage 0; V(0) and K(1) follow in block 0
            e(f"s_mov_b32 {sr(S_CURV)}, 2")
            e(*self.decode_wide(S_ENT, "S0", False))
            for k in range(L.NCP):
                e(*self.copy(0, k))
        else:
            for blk in (0, 1):
                e(*self.decode(S_ENT + 2 * blk, f"S{blk}"))
                for k in range(2 * L.NCP):
                    e(*self.copy(blk, k))
        self.first_iteration()
        e(f"{lbl('LOOP')}:")
        for stage in (1, 2, 3, 0):
            self.iteration(stage)
        e(f"s_branch {lbl('LOOP')}")
        loop_phase = self.phase           # every iteration ends at the same slot phase
        for stage in range(4):
            self.phase = loop_phase
            self.drain(stage)
        e(*self.stubs)
        e(*self.rare_routine(L.SA, L.PA, "RARE_A"), *self.rare_routine(L.SB, L.PB, "RARE_B"))
        e(*(self.switch_wide(False) + self.switch_wide(True) if L.wide else self.switch_routine()))
        e(*self.mask_routine(L.SA, "MASK_A"), *self.mask_routine(L.SB, "MASK_B"))
        e(f"{lbl('END')}:")
        return self.lines


# (head size, waves, two 32-row halves per wave): the dual map of D = 64 and
# the dual-wide map of D = 192 run 64 rows per wave
MAPS = ((128, 8, False), (96, 8, False), (64, 8, False), (64, 12, False), (64, 4, True), (256, 4, False),
        (192, 4, False), (192, 4, True))


def map_key(D: int, nw: int, dual: bool) -> tuple:
    """PRODUCT_MAP / per-map option key: (D, nw), or (D, nw, "dual") for the
    dual-wide map (the one (D, nw) pair with two maps)."""
    return (D, nw, "dual") if dual and D >= 192 else (D, nw)


def map_opts(D: int, nw: int, dual: bool) -> dict:
    """The product's generator options for a map."""
    return {**PRODUCT[D], **PRODUCT_MAP.get(map_key(D, nw, dual), {}), "dual": dual}


def prefix(D: int, nw: int, dual: bool = False) -> str:
    return f"LVSA_STREAM{D}" + ("" if nw == 8 else f"W{nw}") + ("D" if dual and D >= 192 else "")


def operands(D: int, nw: int = 8, rs: bool = False, dual: bool | None = None) -> list[str]:
    """Macros with the asm operand lists of the D kernel (outputs, inputs, clobbers)."""
    L = Layout(D, nw, rs, dual)
    pf = prefix(D, nw, L.dual)
    no = L.NDT * L.NR                   # O tiles (dual: half 0's, then half 1's)
    os_ = ", ".join(f"o{t}" for t in range(no))
    orr = ar if L.wide else vr          # the wide map keeps O in AGPRs
    outs = ", ".join(f'"+{{{orr(L.O + 16 * t, 16)}}}"(o{t})' for t in range(no))
    outs += f', "+{{{vr(L.VM, 2 * L.NR)}}}"(ml), "+{{{vr(L.ROW, 4)}}}"(misc)'
    if L.QA is not None:                # dual-wide: Q of half 0 in VGPRs, of half 1 in AGPRs, each 32 + 16
        n = 4 * L.NQK
        q = (f'"{{{vr(L.Q, 32)}}}"(qv.lo), "{{{vr(L.Q + 32, n - 32)}}}"(qv.hi), '
             f'"{{{ar(L.QA, 32)}}}"(qv.alo), "{{{ar(L.QA + 32, n - 32)}}}"(qv.ahi)')
    elif L.dual:                        # Q of both halves: one 32-register operand
        q = f'"{{{vr(L.Q, 4 * L.NQK * L.NR)}}}"(qv)'
    elif 4 * L.NQK in (24, 48, 64):   # no such operand class (or too wide): Q as two operands (qv.lo, qv.hi)
        lo = 16 if 4 * L.NQK == 24 else 32
        q = f'"{{{vr(L.Q, lo)}}}"(qv.lo), "{{{vr(L.Q + lo, 4 * L.NQK - lo)}}}"(qv.hi)'
    else:
        q = f'"{{{vr(L.Q, 4 * L.NQK)}}}"(qv)'
    ins = (f'{q}, "{{{vr(L.KOFF, L.NQK)}}}"(koff), '
           f'"{{{vr(L.VOFFA, 2 * L.NDT)}}}"(voff), "{{{vr(L.DMAROW, 4 if L.wide else 2)}}}"(dma), '
           f'"{{s[20:23]}}"(sa), "{{s[24:31]}}"(sb), "{{s[32:39]}}"(sc)')
    if L.rs:
        ins += f', "{{{vr(L.ONES, 4)}}}"(ones)'
    clob = [f'"v{r}"' for r in L.CLOBBER_V] + [f'"s{r}"' for r in CLOBBER_S]
    out = [f"#define {pf}_OUTPUTS({os_}, ml, misc) {outs}",
           f"#define {pf}_INPUTS(qv, koff, voff, dma, sa, sb, sc, ones) {ins}",
           f"#define {pf}_CLOBBERS \\"]
    for i in range(0, len(clob), 12):
        out.append("  " + ", ".join(clob[i:i + 12]) + ", \\")
    out.append('  "vcc", "m0", "scc", "memory"')
    return out


# The product's options per head size (paired runs on one box, against the
# same loop without them): D = 128 opens each block with two PV MFMAs whose
# operands were read before the barrier and loads plan entries mid-block
# (0.4% faster on Wan 4x); both head sizes start the row-sum chains with a
# non-accumulating v_dot2 (Wan 4x 0.8%, HunyuanVideo 1.1%, CogVideoX neutral),
# branch on the SCC of the mask test's s_and and set a copy's M0 one MFMA
# slot early (together 0.6% on Wan 4x, CogVideoX neutral); both take the row
# sums from two 16x16x32 MFMAs against a ones pattern instead of eight v_dot2
# and an add per sub-block (Wan 4x 2.7%, CogVideoX 1.9%), issue the rare
# test one MFMA before its branch (Wan 4x 1.2%, CogVideoX 0.6%), and mask a
# sub-block that lies on one side of the key split with one lane mask
# (CogVideoX 1.0%, Wan 4x 0.25%).  The wide map (D = 192, 256) reads operands
# four MFMAs ahead and starts each softmax four MFMA slots into its
# sub-iteration (1.2% / 1.4% faster than 3 and 2; lookahead 2 and 5, start 3
# and no mid-block entry load measured slower); at D = 256 its copies go out
# every third MFMA (1.0% faster than every second; at D = 192, whose blocks
# have 48 MFMAs, 8% slower; every MFMA 3-5% slower), and waits for LDS
# operands once per two MFMAs (its one wave per SIMD issues every
# instruction of the loop itself: D = 192 0.9% fewer cycles and 0.4% less
# time over three pairs, D = 256 0.3% fewer cycles; D = 96 2% more cycles).
# Measured neutral and not used: the D = 64 softmax spread over one more MFMA slot
# (sm_start 1), one LDS wait per two MFMAs (wait_pair), 8 wait states before
# the row sum is read (tail_nop 8), QK / PV MFMAs in pairs or grouped
# (mfma_order).  Measured in cycles (GRBM_GUI_ACTIVE) and time, paired on one
# box: D = 96 with the softmax one slot earlier and 10 wait states before the
# row sum is read, 3.5% fewer cycles and 1.0% less time; the 12-wave D = 64
# loop with the same start and 8 wait states, 2.8% / 1.2%; D = 128 with 8 or
# 10 wait states, 1% more cycles (it keeps 12), D = 256 with 8, 0.6% more;
# D = 192 with 8 wait states and its softmax one slot later (five MFMA slots
# into the sub-iteration), 1.25% fewer cycles and 0.75% less time.
PRODUCT = {128: dict(lead=2, early_load=True, dot_init=True, and_scc=True, copy_split=True, rs_mfma=True,
                     tail_split=True, mask_fast=True),
           96: dict(lead=2, early_load=True, dot_init=True, and_scc=True, copy_split=True, rs_mfma=True,
                    tail_split=True, mask_fast=True, sm_start=1, tail_nop=10),
           64: dict(dot_init=True, and_scc=True, copy_split=True, rs_mfma=True, tail_split=True, mask_fast=True),
           256: dict(early_load=True, dot_init=True, and_scc=True, copy_split=True, rs_mfma=True, tail_split=True,
                     mask_fast=True, la=4, sm_start=4, copy_every=3, wait_pair=True),
           192: dict(early_load=True, dot_init=True, and_scc=True, copy_split=True, rs_mfma=True, tail_split=True,
                     mask_fast=True, la=4, sm_start=5, wait_pair=True, tail_nop=8)}
# Measured and not used (paired runs on one box): s_setprio 1 or 3 around each
# MFMA (`prio`; 12-wave CogVideoX 0.5-0.9% slower, Wan 4x 0.4%); lead PV
# MFMAs and mid-block entry loads in the 12-wave loop (neutral); for the dual
# map, the softmax from the first MFMA slot (`sm_mfma` 1) or also beside the
# last item's first MFMA (`sm_late`), within 0.5% of the product's start.
# Options of one map only, over PRODUCT[D]: the 12-wave D = 64 loop starts
# its softmax one MFMA slot earlier and reads the row sum 8 wait states after
# its MFMA (the compiler's own count for a 16x16x32 result read by VALU).  The
# dual map (D = 64, 4 waves of 64 rows) likewise, with its copies after MFMAs
# 6, 14, 22 and 30 of a block (CogVideoX, against the defaults: start 1 5.6%
# fewer cycles, 8 wait states 0.75%, copies 0.8%; together 6.0% fewer cycles
# and 2.5% less time, the clock falling with the busier matrix core).  The
# dual-wide map of D = 192 (key (192, 4, "dual")) runs PRODUCT[192] as it is:
# against it at the Wan 4x geometry (three runs each, one box), lookahead 3, 5
# or 6, the softmax from slot 3 or 8, no paired LDS waits, copies every MFMA
# pair and 12 tail wait states all landed between -0.3% and +0.75%, and
# copies every third MFMA pair +4.4%.
PRODUCT_MAP = {(64, 12): dict(sm_start=1, tail_nop=8),
               (64, 4): dict(sm_start=1, tail_nop=8, dual_copy=(6, 8))}


def render(per_d: dict | None = None, **opts) -> str:
    out = ["// Generated by gen_stream_asm.py: the hand-scheduled key loops of",
           "// attn_fwd_stream_kernel (lvsa_attn_stream.h) and their asm operand lists.",
           "// Do not edit; regenerate.",
           "#pragma once", ""]
    for D, nw, dual in MAPS:
        pf = prefix(D, nw, dual)
        for dt, name in (("bf16", f"{pf}_LOOP_BF16"), ("f16", f"{pf}_LOOP_F16")):
            o = {**map_opts(D, nw, dual), **opts, **(per_d or {}).get(D, {}),
                 **(per_d or {}).get(map_key(D, nw, dual), {})}
            lines = Gen(dt, D=D, nw=nw, **o).build()
            out.append(f"#define {name} \\")
            for ln in lines:
                if not ln:
                    continue
                if ln.startswith(";"):
                    continue
                out.append(f'  "{ln}\\n" \\')
            out.append('  ""')
            out.append("")
        out += operands(D, nw, o.get("rs_mfma", False), dual)
        out.append("")
    return "\n".join(out)


CENSUS_KINDS = ("mfma 32x32x16", "mfma 16x16x32", "valu", "of which v_exp", "lds", "vmem copy", "salu",
                "smem", "branch", "barrier", "s_waitcnt", "s_nop states")


def census(D: int, nw: int, dual: bool = False, dt: str = "bf16") -> dict:
    """Instruction counts per 32-key sub-block of the steady-state loop (the
    four unrolled blocks between LOOP and its back branch) of the product's
    loop for (D, nw): the common path, without the subroutines a masked
    block or the rare case calls."""
    lines = Gen(dt, D=D, nw=nw, **map_opts(D, nw, dual)).build()
    a = next(i for i, x in enumerate(lines) if x.startswith("LOOP_"))
    b = next(i for i, x in enumerate(lines) if x.startswith("s_branch LOOP_"))
    c = dict.fromkeys(CENSUS_KINDS, 0)
    for ln in lines[a + 1:b]:
        op = ln.split()[0] if ln and not ln.startswith(";") and not ln.endswith(":") else ""
        if not op:
            continue
        if op.startswith("v_mfma_f32_32x32"):
            c["mfma 32x32x16"] += 1
        elif op.startswith("v_mfma_f32_16x16"):
            c["mfma 16x16x32"] += 1
        elif op.startswith("v_"):
            c["valu"] += 1
            c["of which v_exp"] += op.startswith("v_exp")
        elif op.startswith("ds_"):
            c["lds"] += 1
        elif op.startswith("buffer_"):
            c["vmem copy"] += 1
        elif op == "s_barrier":
            c["barrier"] += 1
        elif op == "s_waitcnt":
            c["s_waitcnt"] += 1
        elif op == "s_nop":
            c["s_nop states"] += int(ln.split()[1]) + 1
        elif op.startswith(("s_cbranch", "s_branch", "s_call", "s_setpc")):
            c["branch"] += 1
        elif op.startswith(("s_load", "s_buffer_load")):
            c["smem"] += 1
        elif op.startswith("s_"):
            c["salu"] += 1
        else:
            raise ValueError(f"census: unclassified instruction {ln!r}")
    return {k: v / 8 for k, v in c.items()}          # 4 blocks x 2 sub-blocks


def print_census() -> None:
    cols = [(128, 8, False), (96, 8, False), (64, 12, False), (64, 8, False), (64, 4, True), (192, 4, False),
            (192, 4, True), (256, 4, False)]
    res = {col: census(*col) for col in cols}
    print("| per 32-key sub-block, per wave | " +
          " | ".join(f"D={d}, {n} waves" + (" (64 rows)" if dual else "") for d, n, dual in cols) + " |")
    print("|---|" + "---|" * len(cols))
    for k in CENSUS_KINDS:
        print(f"| {k} | " + " | ".join(f"{res[col][k]:g}" for col in cols) + " |")


def main(argv=None) -> int:
    argv = sys.argv[1:] if argv is None else argv
    if argv and argv[0] == "--census":
        print_census()
        return 0
    dst = Path(argv[0]) if argv else Path(__file__).with_name("lvsa_attn_stream_body.inc")
    text = render()
    if not dst.exists() or dst.read_text() != text:
        dst.write_text(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
