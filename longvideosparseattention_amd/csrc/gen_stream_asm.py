"""Generate the key loop of the single-stream D = 128 attention kernel.

    python gen_stream_asm.py [out.inc]   (default: lvsa_attn_stream_body.inc beside this file)

The loop is hand-scheduled gfx950 assembly, emitted as the body of one inline
asm statement of ``attn_fwd_stream_kernel`` (lvsa_attn_stream.h), whose
operands pin every register this text names.  Each of the 8 waves of a
work-group owns 32 query rows of a 256-row tile and walks the tile's 64-key
blocks as two 32-key sub-blocks; sub-iteration i issues, as one stream,

    QK(i)   S = K Q^T of sub-block i          8 MFMAs   (K from LDS)
    SM(i-1) softmax of sub-block i - 1        ~50 VALU  (P = 2^(S*cs - m))
    PV(i-2) O += V^T P^T of sub-block i - 2   8 MFMAs   (V^T from LDS)

so every wave keeps the matrix core and the VALU busy at once, and the two
waves that share a SIMD fill each other's gaps.  Per 64-key block: one
work-group barrier, four 1 KiB global->LDS copies per wave (block j + 2 into
a 4-stage ring) and one scalar load of a plan entry.

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

Register map (VGPRs; the kernel's operands pin them):
  v[0:63] O (4 d-tiles x 16)      v[64:95] Q (8 k-steps x 4)
  v[96:111] S_A, v[112:127] S_B   v[128:135] P_A, v[136:143] P_B
  v[144:175] LDS operand slots    v[176:183] K read offsets, v[184:191] V^T
  v192 m, v193 l, v194-195 partial row sums, v196 copy row, v197 copy chunk
  v198-199 copy offsets (K, V), v200 tile row, v201 4*h, v202 -inf, v203
  mask temp, v[204:207] RARE temps, v[208:223] softmax temps
SGPRs: s[20:21] entry pointer, s22 blocks, s23 scale*log2(e), s[24:31] K/V
bases (video, extra), s32-35 row strides, s36-37 source lengths, s39 LDS
copy base of the wave; s40-s95 scratch.
"""

from __future__ import annotations

import sys
from pathlib import Path

# ── register map ──
O, Q, SA, SB, PA, PB, OPS, NSLOT = 0, 64, 96, 112, 128, 136, 144, 8
KOFF, VOFFA, VOFFB = 176, 184, 188
VM, VL, LS0, LS1, DMAROW, C16, DK, DV = 192, 193, 194, 195, 196, 197, 198, 199
ROW, H4, NEGINF, VT, RT, T = 200, 201, 202, 203, 204, 208
S_EPTR, S_N, S_CS = 20, 22, 23
S_KB0, S_VB0, S_KB1, S_VB1 = 24, 26, 28, 30
S_KRS0, S_VRS0, S_KRS1, S_VRS1, S_NK, S_NX, S_WAVE, S_LDSK = 32, 33, 34, 35, 36, 37, 38, 39
S_J, S_NM1, S_CUR, S_ENT, S_RK, S_RV = 40, 41, 42, 44, 52, 56
S_SOK, S_SOV, S_KRSC = 60, 62, 64  # copy soffsets (K: 60, 61; V: 62, 63); strides, 32-row strides
S_RET = 76
TILE, VBASE = 16384, 65536        # bytes of a K (V) block of 64 rows x 256 B; V tiles start at 64 KiB
LA = 6                            # MFMAs of LDS operand lookahead (< NSLOT)

CLOBBER_V = list(range(96, 176)) + [LS0, LS1, DK, DV] + list(range(204, 224))
CLOBBER_S = list(range(40, 96))


def vr(a: int, n: int = 1) -> str:
    return f"v{a}" if n == 1 else f"v[{a}:{a + n - 1}]"


def sr(a: int, n: int = 1) -> str:
    return f"s{a}" if n == 1 else f"s[{a}:{a + n - 1}]"


def lbl(name: str) -> str:
    return f"{name}_%="


class Gen:
    def __init__(self, dt: str, pad: bool = False, always_rare: bool = False, la: int = LA,
                 pv_b128: bool = False, no_softmax: bool = False, order: str = "group",
                 no_barrier: bool = False, no_decode: bool = False, no_exp: bool = False):
        assert dt in ("bf16", "f16")
        self.dt = dt
        self.pad = pad                  # diagnostics: 16 wait states after every MFMA
        self.always_rare = always_rare  # diagnostics: exact row max on every sub-block
        self.la = la                    # MFMAs of LDS operand lookahead
        self.pv_b128 = pv_b128          # timing only (wrong results): one b128 read per PV operand
        self.no_softmax = no_softmax    # timing only (wrong results): no softmax VALU
        self.order = order              # softmax op order: "group" (4 fma, 4 exp) or "mix"
        self.no_barrier = no_barrier    # timing only (wrong results): no work-group barrier
        self.no_decode = no_decode      # timing only (wrong results): copy sources not updated
        self.no_exp = no_exp            # timing only (wrong results): no exponentials
        self.lines: list[str] = []
        self.stubs: list[str] = []

    def e(self, *ins: str) -> None:
        self.lines.extend(ins)

    @property
    def mfma(self) -> str:
        return "v_mfma_f32_32x32x16_bf16" if self.dt == "bf16" else "v_mfma_f32_32x32x16_f16"

    # ── softmax ──
    def softmax_ops(self, S: int, P: int) -> list[str]:
        """P = 2^(S*cs - m) as bf16/f16 pairs; this sub-block's row sum in LS0 + LS1."""
        if self.no_softmax:
            return [f"v_mov_b32 {vr(LS0)}, 0", f"v_mov_b32 {vr(LS1)}, 0"]
        cvt = "v_cvt_pk_bf16_f32" if self.dt == "bf16" else "v_cvt_pk_f16_f32"
        one = "0x3f803f80" if self.dt == "bf16" else "0x3c003c00"
        dot = "v_dot2c_f32_bf16" if self.dt == "bf16" else "v_dot2c_f32_f16"
        fma = lambda k: f"v_fma_f32 {vr(T + k)}, {vr(S + k)}, {sr(S_CS)}, -{vr(VM)}"  # noqa: E731
        exp = lambda k: ("s_nop 0" if self.no_exp else f"v_exp_f32 {vr(T + k)}, {vr(T + k)}")  # noqa: E731
        pk = lambda q: f"{cvt} {vr(P + q)}, {vr(T + 2 * q)}, {vr(T + 2 * q + 1)}"  # noqa: E731
        d2 = lambda q: f"{dot} {vr(LS0 + (q & 1))}, {one}, {vr(P + q)}"  # noqa: E731
        ops = [f"v_mov_b32 {vr(LS0)}, 0", f"v_mov_b32 {vr(LS1)}, 0"]
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
        self.stubs += [f"{lbl('RSTUB_' + site)}:", f"s_call_b64 {sr(S_RET, 2)}, {lbl('RARE_' + sset)}",
                       f"s_branch {lbl('RRET_' + site)}"]
        return ["s_nop 2",                                         # dot2 result -> VALU: 3 states
                f"v_add_f32 {vr(LS0)}, {vr(LS0)}, {vr(LS1)}",
                f"v_cmp_nge_f32 vcc, 0x43800000, {vr(LS0)}",      # !(256 >= ls): ls > 256 or NaN
                f"s_branch {lbl('RSTUB_' + site)}" if self.always_rare else f"s_cbranch_vccnz {lbl('RSTUB_' + site)}",
                f"{lbl('RRET_' + site)}:",
                f"v_add_f32 {vr(VL)}, {vr(VL)}, {vr(LS0)}"]

    def mask_check(self, site: str, sset: str, desc: int, half: int) -> list[str]:
        self.stubs += [f"{lbl('MSTUB_' + site)}:", f"s_mov_b32 s91, {sr(desc)}", f"s_mov_b32 s75, {32 * half}",
                       f"s_call_b64 {sr(S_RET, 2)}, {lbl('MASK_' + sset)}", f"s_branch {lbl('MRET_' + site)}"]
        return [f"s_and_b32 s74, {sr(desc)}, 3", "s_cmp_lg_u32 s74, 0", f"s_cbranch_scc1 {lbl('MSTUB_' + site)}",
                f"{lbl('MRET_' + site)}:"]

    def rare_routine(self, S: int, P: int, name: str) -> list[str]:
        """True row max of the sub-block, m -> max(m, max*cs), O and l rescaled, P recomputed."""
        r = [f"{lbl(name)}:", "s_nop 15", "s_nop 7",
             f"v_max3_f32 {vr(RT)}, {vr(S)}, {vr(S + 1)}, {vr(S + 2)}",
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
        r += [f"v_mul_f32 {vr(O + k)}, {vr(RT + 1)}, {vr(O + k)}" for k in range(64)]
        r += self.softmax_ops(S, P)
        r += ["s_nop 2", f"v_add_f32 {vr(LS0)}, {vr(LS0)}, {vr(LS1)}", f"s_setpc_b64 {sr(S_RET, 2)}"]
        return r

    def mask_routine(self, S: int, name: str) -> list[str]:
        """-inf on the keys a two-part descriptor (s91) excludes, for sub-block half s75/32.

        Row part b = tile rows >= qs; keys below kb take the part's lo bit, the rest
        its hi bit (bits a.lo, a.hi, b.lo, b.hi).  Element k of the sub-block holds key
        32*half + 8*(k/4) + 4*h + k%4."""
        r = [f"{lbl(name)}:",
             "s_bfe_u32 s88, s91, 0x80008",       # kb
             "s_bfe_u32 s89, s91, 0x80010",       # qs
             "s_bfe_u32 s90, s91, 0x40002",       # allow bits
             "s_sub_u32 s88, s88, s75",
             f"v_cmp_ge_u32_e64 s[78:79], {vr(ROW)}, s89",   # lanes of part b
             "s_bitcmp1_b32 s90, 0", "s_cselect_b64 s[92:93], -1, 0", "s_andn2_b64 s[92:93], s[92:93], s[78:79]",
             "s_bitcmp1_b32 s90, 2", "s_cselect_b64 s[94:95], -1, 0", "s_and_b64 s[94:95], s[94:95], s[78:79]",
             "s_or_b64 s[80:81], s[92:93], s[94:95]",      # lanes whose lo keys are allowed
             "s_bitcmp1_b32 s90, 1", "s_cselect_b64 s[92:93], -1, 0", "s_andn2_b64 s[92:93], s[92:93], s[78:79]",
             "s_bitcmp1_b32 s90, 3", "s_cselect_b64 s[94:95], -1, 0", "s_and_b64 s[94:95], s[94:95], s[78:79]",
             "s_or_b64 s[82:83], s[92:93], s[94:95]",      # lanes whose hi keys are allowed
             f"v_sub_u32 {vr(VT)}, s88, {vr(H4)}"]          # kb - 32*half - 4h
        for k in range(16):
            ck = 8 * (k // 4) + (k % 4)
            r += [f"v_cmp_lt_i32 vcc, {ck}, {vr(VT)}",      # key below kb
                  "s_and_b64 s[84:85], vcc, s[80:81]",
                  "s_andn2_b64 s[86:87], s[82:83], vcc",
                  "s_or_b64 s[84:85], s[84:85], s[86:87]",
                  "s_nop 0",
                  f"v_cndmask_b32_e64 {vr(S + k)}, {vr(NEGINF)}, {vr(S + k)}, s[84:85]"]
        r += [f"s_setpc_b64 {sr(S_RET, 2)}"]
        return r

    # ── copies ──
    def decode(self, x: int, site: str) -> list[str]:
        """Copy offsets of the block named by entry word x.  The buffer resources
        span a whole key source (rows past its end read zeros), so a block only
        moves the soffsets; a change of source (video <-> extra rows) calls SWITCH."""
        self.stubs += [f"{lbl('SWSTUB_' + site)}:", f"s_call_b64 {sr(S_RET, 2)}, {lbl('SWITCH')}",
                       f"s_branch {lbl('SWRET_' + site)}"]
        return [
            f"s_lshr_b32 s74, {sr(x)}, 31",
            f"s_cmp_lg_u32 s74, {sr(S_CUR)}",
            f"s_cbranch_scc1 {lbl('SWSTUB_' + site)}",
            f"{lbl('SWRET_' + site)}:",
            f"s_and_b32 s73, {sr(x)}, 0x7fffffff",
            "s_lshl_b32 s73, s73, 6",                                  # first row of the block
            f"s_mul_i32 {sr(S_SOK)}, s73, {sr(S_KRSC)}",
            f"s_add_u32 {sr(S_SOK + 1)}, {sr(S_SOK)}, {sr(S_KRSC + 2)}",  # + 32 rows
            f"s_mul_i32 {sr(S_SOV)}, s73, {sr(S_KRSC + 1)}",
            f"s_add_u32 {sr(S_SOV + 1)}, {sr(S_SOV)}, {sr(S_KRSC + 3)}",
        ]

    def switch_routine(self) -> list[str]:
        """Buffer resources, row strides and lane copy offsets of key source s74."""
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
            f"v_mad_u32_u24 {vr(DK)}, {vr(DMAROW)}, {sr(S_KRSC)}, {vr(C16)}",
            f"v_mad_u32_u24 {vr(DV)}, {vr(DMAROW)}, {sr(S_KRSC + 1)}, {vr(C16)}",
            "s_nop 1",
            f"s_setpc_b64 {sr(S_RET, 2)}",
        ]

    @staticmethod
    def copy(stage: int, k: int) -> list[str]:
        """Copy instruction k of a block into `stage`: k = 0, 1 K rows 32k + 4*wave + lane/16,
        k = 2, 3 the same V rows."""
        v, ii = k >> 1, k & 1
        lds = (VBASE if v else 0) + stage * TILE + ii * 8192
        rs = S_RV if v else S_RK
        so = sr((S_SOV if v else S_SOK) + ii)
        return [f"s_add_u32 m0, {sr(S_LDSK)}, {lds}", "s_nop 0",
                f"buffer_load_dwordx4 {vr(DV if v else DK)}, {sr(rs, 4)}, {so} offen lds"]

    # ── an MFMA stream with its operand reads and the interleaved work ──
    def stream(self, mfmas: list[tuple], fill: dict[int, list[str]]) -> None:
        """mfmas: ("qk", stage, half, c, S) or ("pv", stage, st16, dt, P).
        fill[i]: instructions emitted right after MFMA i.  The LDS operands of MFMA i
        go to slot i % NSLOT and are read LA MFMAs ahead."""
        n = len(mfmas)
        LA = self.la
        nreads = [1 if (m[0] == "qk" or self.pv_b128) else 2 for m in mfmas]

        def reads(i: int) -> list[str]:
            m = mfmas[i]
            slot = OPS + 4 * (i % NSLOT)
            if m[0] == "qk":
                _, st, half, c, _ = m
                return [f"ds_read_b128 {vr(slot, 4)}, {vr(KOFF + c)} offset:{st * TILE + half * 8192}"]
            _, st, st16, dt, _ = m
            off = st * TILE + st16 * 4096    # the V^T read offsets include VBASE
            if self.pv_b128:
                return [f"ds_read_b128 {vr(slot, 4)}, {vr(KOFF + dt)} offset:{off}"]
            return [f"ds_read_b64_tr_b16 {vr(slot, 2)}, {vr(VOFFA + dt)} offset:{off}",
                    f"ds_read_b64_tr_b16 {vr(slot + 2, 2)}, {vr(VOFFB + dt)} offset:{off}"]

        issued = min(LA, n)
        for i in range(issued):
            self.e(*reads(i))
        for i in range(n):
            pending = sum(nreads[j] for j in range(i + 1, issued))
            self.e(f"s_waitcnt lgkmcnt({min(15, pending)})")
            m = mfmas[i]
            slot = OPS + 4 * (i % NSLOT)
            if m[0] == "qk":
                _, _, _, c, S = m
                self.e(f"{self.mfma} {vr(S, 16)}, {vr(slot, 4)}, {vr(Q + 4 * c, 4)}, {'0' if c == 0 else vr(S, 16)}")
            else:
                _, _, st16, dt, P = m
                acc = vr(O + 16 * dt, 16)
                self.e(f"{self.mfma} {acc}, {vr(slot, 4)}, {vr(P + 4 * (st16 & 1), 4)}, {acc}")
            if self.pad:
                self.e("s_nop 15")
            if issued < n:
                self.e(*reads(issued))
                issued += 1
            self.e(*fill.get(i, []))

    @staticmethod
    def spread(ops: list[str], slots: list[int], fill: dict[int, list[str]]) -> None:
        per = -(-len(ops) // len(slots))
        for i, s in enumerate(slots):
            fill.setdefault(s, []).extend(ops[i * per:(i + 1) * per])

    def iteration_tail(self, stage: int) -> None:
        """Scalar load of entry j+3, j += 1, leave for the drain after the last block."""
        self.e(f"s_add_u32 s74, {sr(S_J)}, 3", f"s_min_u32 s74, s74, {sr(S_NM1)}", "s_lshl_b32 s74, s74, 3",
               f"s_load_dwordx2 {sr(S_ENT + 2 * ((stage + 3) & 3), 2)}, {sr(S_EPTR, 2)}, s74",
               f"s_add_u32 {sr(S_J)}, {sr(S_J)}, 1", f"s_cmp_ge_u32 {sr(S_J)}, {sr(S_N)}",
               f"s_cbranch_scc1 {lbl(f'DRAIN{stage}')}")

    def iteration(self, stage: int) -> None:
        """Block j: QK of its two sub-blocks (K in `stage`), softmax of sub-blocks
        2j-1 and 2j, PV of block j-1 (V in stage-1), copies of block j+2."""
        vst, cst = (stage + 3) & 3, (stage + 2) & 3
        site = f"I{stage}"
        self.e(f"; ── block j, K stage {stage}", "s_waitcnt vmcnt(4)", "s_nop 0" if self.no_barrier else "s_barrier",
               "s_waitcnt lgkmcnt(0)")
        mf = []
        for half, S, P in ((0, SA, PA), (1, SB, PB)):
            for c in range(8):
                mf.append(("qk", stage, half, c, S))
                mf.append(("pv", vst, 2 * half + c // 4, c % 4, P))
        fill: dict[int, list[str]] = {0: [] if self.no_decode else self.decode(S_ENT + 2 * cst, site)}
        for k, at in enumerate((6, 10, 22, 26)):
            fill.setdefault(at, []).extend(self.copy(cst, k))
        # sub-iteration a: softmax of sub-block 2j-1 (S_B, block j-1 half 1)
        fill.setdefault(1, []).extend(self.mask_check(site + "a", "B", S_ENT + 2 * vst + 1, 1))
        self.spread(self.softmax_ops(SB, PB), list(range(2, 15)), fill)
        fill.setdefault(15, []).extend(self.softmax_tail(site + "a", "B"))
        # sub-iteration b: softmax of sub-block 2j (S_A, block j half 0)
        fill.setdefault(17, []).extend(self.mask_check(site + "b", "A", S_ENT + 2 * stage + 1, 0))
        self.spread(self.softmax_ops(SA, PA), list(range(18, 31)), fill)
        fill.setdefault(31, []).extend(self.softmax_tail(site + "b", "A"))
        self.stream(mf, fill)
        self.iteration_tail(stage)

    def first_iteration(self) -> None:
        """Block 0: QK of its two sub-blocks, softmax of sub-block 0, copies of block 2."""
        self.e("; ── block 0", "s_waitcnt vmcnt(4)", "s_barrier", "s_waitcnt lgkmcnt(0)")
        mf = [("qk", 0, 0, c, SA) for c in range(8)] + [("qk", 0, 1, c, SB) for c in range(8)]
        fill: dict[int, list[str]] = {0: self.decode(S_ENT + 4, "F")}
        for k in range(4):
            fill.setdefault(1 + k, []).extend(self.copy(2, k))
        fill.setdefault(9, []).extend(self.mask_check("F", "A", S_ENT + 1, 0))
        self.spread(self.softmax_ops(SA, PA), list(range(10, 15)), fill)
        fill.setdefault(15, []).extend(self.softmax_tail("F", "A"))
        self.stream(mf, fill)
        self.iteration_tail(0)

    def drain(self, stage: int) -> None:
        """After block n-1 (in `stage`): softmax of sub-block 2n-1, PV of block n-1."""
        self.e(f"{lbl(f'DRAIN{stage}')}:")
        mf = [("pv", stage, k // 4, k % 4, PA) for k in range(8)] + \
             [("pv", stage, 2 + k // 4, k % 4, PB) for k in range(8)]
        fill: dict[int, list[str]] = {0: self.mask_check(f"D{stage}", "B", S_ENT + 2 * stage + 1, 1)}
        self.spread(self.softmax_ops(SB, PB), list(range(1, 7)), fill)
        fill.setdefault(7, []).extend(self.softmax_tail(f"D{stage}", "B"))
        self.stream(mf, fill)
        # the code after the asm reads O with VALU: 12 states after the last MFMA
        self.e("s_waitcnt vmcnt(0) lgkmcnt(0)", "s_nop 15", f"s_branch {lbl('END')}")

    def build(self) -> list[str]:
        e = self.e
        # setup: entries 0..2 (clamped to the last block), copies of blocks 0 and 1
        e(f"s_sub_u32 {sr(S_NM1)}, {sr(S_N)}, 1",
          f"s_load_dwordx2 {sr(S_ENT, 2)}, {sr(S_EPTR, 2)}, 0x0",
          f"s_min_u32 s74, {sr(S_NM1)}, 1", "s_lshl_b32 s74, s74, 3",
          f"s_load_dwordx2 {sr(S_ENT + 2, 2)}, {sr(S_EPTR, 2)}, s74",
          f"s_min_u32 s74, {sr(S_NM1)}, 2", "s_lshl_b32 s74, s74, 3",
          f"s_load_dwordx2 {sr(S_ENT + 4, 2)}, {sr(S_EPTR, 2)}, s74",
          f"s_mov_b32 {sr(S_J)}, 0",
          f"s_mov_b32 {sr(S_CUR)}, 2",
          "s_waitcnt lgkmcnt(0)")
        for blk in (0, 1):
            e(*self.decode(S_ENT + 2 * blk, f"S{blk}"))
            for k in range(4):
                e(*self.copy(blk, k))
        self.first_iteration()
        e(f"{lbl('LOOP')}:")
        for stage in (1, 2, 3, 0):
            self.iteration(stage)
        e(f"s_branch {lbl('LOOP')}")
        for stage in range(4):
            self.drain(stage)
        e(*self.stubs)
        e(*self.rare_routine(SA, PA, "RARE_A"), *self.rare_routine(SB, PB, "RARE_B"), *self.switch_routine())
        e(*self.mask_routine(SA, "MASK_A"), *self.mask_routine(SB, "MASK_B"))
        e(f"{lbl('END')}:")
        return self.lines


def render(**opts) -> str:
    out = ["// Generated by gen_stream_asm.py: the hand-scheduled key loop of",
           "// attn_fwd_stream_kernel (lvsa_attn_stream.h).  Do not edit; regenerate.",
           "#pragma once", ""]
    for dt, name in (("bf16", "LVSA_STREAM_LOOP_BF16"), ("f16", "LVSA_STREAM_LOOP_F16")):
        lines = Gen(dt, **opts).build()
        out.append(f"#define {name} \\")
        for ln in lines:
            if not ln:
                continue
            if ln.startswith(";"):
                continue
            out.append(f'  "{ln}\\n" \\')
        out.append('  ""')
        out.append("")
    clob = [f'"v{r}"' for r in CLOBBER_V] + [f'"s{r}"' for r in CLOBBER_S]
    out.append("#define LVSA_STREAM_CLOBBERS \\")
    for i in range(0, len(clob), 12):
        out.append("  " + ", ".join(clob[i:i + 12]) + ", \\")
    out.append('  "vcc", "m0", "scc", "memory"')
    out.append("")
    return "\n".join(out)


def main(argv=None) -> int:
    argv = sys.argv[1:] if argv is None else argv
    dst = Path(argv[0]) if argv else Path(__file__).with_name("lvsa_attn_stream_body.inc")
    text = render()
    if not dst.exists() or dst.read_text() != text:
        dst.write_text(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
