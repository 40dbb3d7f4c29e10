"""The hand-scheduled key loops of the single-stream kernel (D = 64, 128), on the CPU.

* The committed lvsa_attn_stream_body.inc is what gen_stream_asm.py generates.
* tests/asm_sim.py runs the generated loop for the 8 waves of one 256-row
  work-group over small K/V/Q and plans (full blocks, a key tail, text rows
  as the extra source, two-part descriptors with a row split, the rare path
  forced on every sub-block) and the result is compared with float64
  attention over the keys the plan allows.  Tolerance: bf16 inputs and P,
  fp32 accumulation: max |err| <= 4e-3, LSE within 2e-3.
"""
import math
import struct
from pathlib import Path

import numpy as np
import pytest

import asm_sim as A

CSRC = Path(__file__).resolve().parents[1] / "longvideosparseattention_amd" / "csrc"


def test_committed_loop_is_generated():
    assert (CSRC / "lvsa_attn_stream_body.inc").read_text() == A.G.render()


def _swz(r, D=128):
    """16-byte chunk swizzle of LDS row r (lvsa_attn_kernels.h swz<D>; D = 96
    rows use the D = 128 layout, D = 192 and 256 the D = 128 swizzle on the
    low four chunk bits)."""
    if D in (96, 128, 192, 256):
        return ((r & 3) << 2) | ((r >> 2) & 3)
    return (((r >> 1) & 1) << 2) | (((r >> 2) & 1) << 1) | ((r >> 3) & 1)


def _desc_two_part(bits, kb, qs):
    return 1 | (bits << 2) | (kb << 8) | (qs << 16)


def _allowed(y, row, key_in_block):
    """Reference meaning of a plan descriptor (lvsa_amd.h)."""
    if y & 3 == 0:
        return True
    bits, kb, qs = (y >> 2) & 0xF, (y >> 8) & 0xFF, (y >> 16) & 0x1FF
    part_b = row >= qs
    lo = key_in_block < kb
    bit = (2 if part_b else 0) + (0 if lo else 1)
    return bool((bits >> bit) & 1)


def run_loop(entries, nk, n_x, seed=0, dt="bf16", D=128, nw=8, **opts):
    """Run the generated loop for the `nw` waves of one work-group with the
    registers the C++ prologue of attn_fwd_stream_kernel sets up (the 12-wave
    kernel: 384 query rows, waves 8-11 repeat the copies of waves 0-3; the
    dual map, D = 64 with 4 waves, and the dual-wide map, D = 192 with 4 waves
    and dual=True: 64 rows per wave as two 32-row halves)."""
    rng = np.random.default_rng(seed)
    L = A.G.Layout(D, nw, rs=opts.get("rs_mfma", A.G.PRODUCT[D].get("rs_mfma", False)), dual=opts.get("dual"))
    NR = L.NR
    R = 32 * NR * nw
    RB, NCH = L.RB, L.RB // 16            # LDS row pitch (D = 96: the D = 128 pitch), chunks per row
    GRB = 2 * D                           # global row stride of K and V
    rnd = (lambda x: A.bf16_to_f32(A.bf16_round(x))) if dt == "bf16" else (lambda x: x.astype(np.float16).astype(np.float32))
    enc = (lambda x: A.bf16_round(x).astype(np.uint16).tobytes()) if dt == "bf16" else (lambda x: x.astype(np.float16).tobytes())
    q = rnd(rng.standard_normal((R, D)).astype(np.float32))
    k, v = (rnd(rng.standard_normal((nk, D)).astype(np.float32)) for _ in range(2))
    kx, vx = (rnd(rng.standard_normal((max(n_x, 1), D)).astype(np.float32)) for _ in range(2))
    sim = A.Sim(dt, D=D, nw=nw, **opts)
    kb0, vb0, kb1, vb1 = (sim.mem.alloc(enc(x)) for x in (k, v, kx, vx))
    ep = sim.mem.alloc(b"".join(struct.pack("<II", x, y) for x, y in entries))
    scale = 1 / math.sqrt(D)
    lane = np.arange(64)
    h, i32 = lane >> 5, lane & 31
    qbits = (A.bf16_round(q) if dt == "bf16" else q.astype(np.float16).view(np.uint16).astype(np.uint32))
    waves = []
    for w in range(nw):
        W = A.Wave(w, sim)
        V = W.v
        for r in range(NR):
            rows = 32 * NR * w + 32 * r + i32
            for c in range(L.NQK):
                for j in range(4):
                    d0 = 16 * c + 8 * h + 2 * j
                    # the dual-wide map holds half 1's Q in AGPRs (register file index 256 +)
                    dst = (256 + L.QA + 4 * c + j if r == 1 and L.QA is not None
                           else L.Q + 4 * L.NQK * r + 4 * c + j)
                    V[dst] = qbits[rows, d0] | (qbits[rows, d0 + 1] << 16)
        sw = np.array([_swz(x & 15, D) for x in i32])
        for c in range(L.NQK):
            V[L.KOFF + c] = i32 * RB + (((2 * c + h) ^ sw) << 4)
        rowA = 4 * h + ((lane & 15) >> 2)
        dgrp = (lane >> 4) & 1
        for dt_ in range(L.NDT):
            chunk = 4 * dt_ + 2 * dgrp + ((lane & 3) >> 1)
            inb = (lane & 1) * 8
            V[L.VOFFA + dt_] = L.VBASE + rowA * RB + ((chunk ^ np.array([_swz(x, D) for x in rowA])) << 4) + inb
            V[L.VOFFB + dt_] = (L.VBASE + (rowA + 8) * RB +
                                ((chunk ^ np.array([_swz(x, D) for x in rowA + 8])) << 4) + inb)
        ndata = 2 * D // 16                   # chunks of a row that hold data
        if L.wide:
            # copy ii fills LDS KiB 4*ii + w: rows 8*ii + 2*w + lane/32, one
            # (row, chunk offset) pair per parity of ii
            for par in (0, 1):
                crow = 8 * par + 2 * w + lane // 32
                c16 = ((lane % NCH) ^ np.array([_swz(x & 15, D) for x in crow])) * 16
                V[L.DMAROW + 2 * par] = crow
                V[L.C16 + 2 * par] = np.where(c16 >= 16 * ndata, 0x7FFF0000, c16)
        else:
            crow = (w % 8) * (1024 // RB) + lane // NCH
            V[L.DMAROW] = crow
            V[L.C16] = ((lane % NCH) ^ np.array([_swz(x & 15, D) for x in crow])) * 16
            if ndata < NCH:   # chunks past the row's data: an offset beyond every source (zeros, no access)
                V[L.C16] = np.where(V[L.C16] >= 16 * ndata, 0x7FFF0000, V[L.C16])
        V[L.ROW], V[L.H4], V[L.NEGINF], V[L.VT] = 32 * NR * w + i32, 4 * h, 0xFF800000, 0
        for r in range(NR):
            V[L.VM + r] = A.f2u(np.full(64, -1e30, np.float32))
        if L.rs:
            one = 0x3F803F80 if dt == "bf16" else 0x3C003C00
            for j in range(4):
                V[L.ONES + j] = np.where(np.isin(lane, [0, 20, 32, 52]), one, 0)
        S = W.s
        S[20], S[21], S[22] = ep & 0xFFFFFFFF, ep >> 32, len(entries)
        S[23] = int(A.f2u(np.float32(scale * 1.4426950408889634)))
        for i, b in enumerate((kb0, vb0, kb1, vb1)):
            S[24 + 2 * i], S[25 + 2 * i] = b & 0xFFFFFFFF, b >> 32
        S[32:36] = [GRB, GRB, GRB, GRB]
        S[36], S[37], S[38], S[39] = nk, n_x, w, 1024 * (w % 8)
        waves.append(W)
    sim.run(waves)
    O = np.zeros((R, D))
    lsum, mrun = np.zeros(R), np.zeros(R)
    obase = 256 if L.wide else 0          # the wide map keeps O in AGPRs
    for w, W in enumerate(waves):
        for ln in range(64):
            for hr in range(NR):
                r, hh = 32 * NR * w + 32 * hr + (ln & 31), ln >> 5
                for dt_ in range(L.NDT):
                    for rr in range(16):
                        O[r, 32 * dt_ + 8 * (rr // 4) + 4 * hh + rr % 4] = \
                            A.u2f(W.v[obase + L.O + 16 * L.NDT * hr + 16 * dt_ + rr, ln])
                lsum[r] += A.u2f(W.v[L.VL + hr, ln])
                mrun[r] = A.u2f(W.v[L.VM + hr, ln])
    # reference: float64 softmax attention over the allowed keys
    ref = np.zeros((R, D))
    lse_ref = np.zeros(R)
    for r in range(R):
        ks, vs = [], []
        for x, y in entries:
            src_k, src_v, nn = (kx, vx, n_x) if x >> 31 else (k, v, nk)
            j = x & 0x7FFFFFFF
            for t in range(64 * j, min(64 * j + 64, nn)):
                if _allowed(y, r, t - 64 * j):
                    ks.append(src_k[t])
                    vs.append(src_v[t])
        s = np.asarray(ks, np.float64) @ q[r].astype(np.float64) * scale
        p = np.exp(s - s.max())
        ref[r] = p @ np.asarray(vs, np.float64) / p.sum()
        lse_ref[r] = math.log(p.sum()) + s.max()
    out = O / lsum[:, None]
    lse = (mrun + np.log2(lsum)) * math.log(2)
    return np.abs(out - ref).max(), np.abs(lse - lse_ref).max(), sim.copies


def _tail(nn, j):
    kn = min(64, nn - 64 * j)
    return 0 if kn == 64 else _desc_two_part(0x5, kn, 255)


CASES = {
    "full_blocks": (lambda: [(j, 0) for j in range(3)], 192, 0),
    "tail_and_text": (lambda: [(j, _tail(150, j)) for j in range(3)] + [(0x80000000, _tail(5, 0))], 150, 5),
    "row_split": (lambda: [(0, 0), (1, _desc_two_part(0b1011, 40, 100)), (2, _desc_two_part(0b0110, 64, 37)),
                           (3, _desc_two_part(0b1101, 17, 255))], 256, 0),
    "one_block": (lambda: [(1, _tail(100, 1))], 100, 0),
}


@pytest.mark.parametrize("D", [128, 64, 96])
@pytest.mark.parametrize("case", sorted(CASES))
def test_loop_matches_attention(case, D):
    make, nk, n_x = CASES[case]
    entries = make()
    err, lse_err, copies = run_loop(entries, nk, n_x, D=D)
    assert err <= 4e-3 and lse_err <= 2e-3, (case, err, lse_err)
    # 2 * NCP copies (K and V) per wave per block for blocks 0..n+1 (the last
    # two repeat block n-1); D = 96 copies whole D = 128 rows
    assert copies == 8 * 2 * A.G.Layout(D).NCP * (len(entries) + 2)


@pytest.mark.parametrize("case", sorted(CASES))
def test_loop_12_waves(case):
    """The 12-wave D = 64 loop (384 query rows, compact register map, waves
    8-11 repeating the copies of waves 0-3)."""
    make, nk, n_x = CASES[case]
    err, lse_err, copies = run_loop(make(), nk, n_x, D=64, nw=12)
    assert err <= 4e-3 and lse_err <= 2e-3, (case, err, lse_err)
    assert copies == 12 * 2 * (len(make()) + 2)


@pytest.mark.parametrize("case", sorted(CASES))
def test_loop_dual(case):
    """The dual map: D = 64, 4 waves of 64 rows (two 32-row halves sharing
    each LDS operand), 256-row tiles."""
    make, nk, n_x = CASES[case]
    err, lse_err, copies = run_loop(make(), nk, n_x, D=64, nw=4)
    assert err <= 4e-3 and lse_err <= 2e-3, (case, err, lse_err)
    # two copies of K and two of V per wave and block, blocks 0..n+1
    assert copies == 4 * 4 * (len(make()) + 2)


def test_loop_dual_rare_path_and_fp16():
    """The dual map with the exact-max path on every sub-block (both halves),
    and with fp16 inputs."""
    err, lse_err, _ = run_loop([(j, 0) for j in range(3)], 192, 0, seed=6, D=64, nw=4, always_rare=True)
    assert err <= 4e-3 and lse_err <= 2e-3, (err, lse_err)
    err, lse_err, _ = run_loop([(j, _tail(150, j)) for j in range(3)], 150, 0, seed=7, dt="f16", D=64, nw=4)
    assert err <= 2e-3 and lse_err <= 2e-3, (err, lse_err)


def test_loop_12_waves_row_split_past_255_and_rare_path():
    """Row splits above row 255 (the 9-bit split of 384-row tiles) and the
    exact-max path on every sub-block, 12 waves."""
    entries = [(0, 0), (1, _desc_two_part(0b1011, 40, 300)), (2, _desc_two_part(0b0110, 64, 257)),
               (3, _desc_two_part(0b1101, 17, 383))]
    err, lse_err, _ = run_loop(entries, 256, 0, seed=5, D=64, nw=12)
    assert err <= 4e-3 and lse_err <= 2e-3, (err, lse_err)
    err, lse_err, _ = run_loop([(j, 0) for j in range(3)], 192, 0, seed=6, D=64, nw=12, always_rare=True)
    assert err <= 4e-3 and lse_err <= 2e-3, (err, lse_err)
    err, lse_err, _ = run_loop([(j, _tail(150, j)) for j in range(3)], 150, 0, seed=7, dt="f16", D=64, nw=12)
    assert err <= 2e-3 and lse_err <= 2e-3, (err, lse_err)


@pytest.mark.parametrize("D", [128, 64, 96])
def test_loop_rare_path_every_sub_block(D):
    """The exact-max path (rescale of O and l) on every sub-block gives the
    same attention."""
    err, lse_err, _ = run_loop([(j, 0) for j in range(3)], 192, 0, seed=3, D=D, always_rare=True)
    assert err <= 4e-3 and lse_err <= 2e-3


@pytest.mark.parametrize("D", [128, 64, 96])
def test_loop_fp16(D):
    err, lse_err, _ = run_loop([(j, _tail(150, j)) for j in range(3)], 150, 0, seed=4, dt="f16", D=D)
    assert err <= 2e-3 and lse_err <= 2e-3


@pytest.mark.parametrize("D", [256, 192])
@pytest.mark.parametrize("case", sorted(CASES))
def test_wide_loop(case, D):
    """The wide map of D = 192 and 256: 4 waves (one per SIMD) on 128 query
    rows, O in AGPRs, K and V in two-stage rings of their own (K of block
    j + 1 and V of block j copied during block j); rows on the 512-byte
    pitch (D = 192: chunks 24-31 zero-filled and never read)."""
    make, nk, n_x = CASES[case]
    entries = make()
    err, lse_err, copies = run_loop(entries, nk, n_x, D=D, nw=4)
    assert err <= 4e-3 and lse_err <= 2e-3, (case, err, lse_err)
    # K(0) in the setup, then K(j + 1) and V(j) in every block: 8 copies per tensor
    assert copies == 4 * 8 * (1 + 2 * len(entries))


@pytest.mark.parametrize("D", [256, 192])
def test_wide_loop_source_switches_rare_path_and_fp16(D):
    """K and V of one block come from different plan entries: sources switch
    (video -> extra rows -> video) for each tensor on its own; the exact-max
    path on every sub-block; fp16."""
    ent = [(0, 0), (0x80000000, _tail(5, 0)), (1, 0), (2, _tail(150, 2))]
    err, lse_err, _ = run_loop(ent, 150, 5, seed=8, D=D, nw=4)
    assert err <= 4e-3 and lse_err <= 2e-3, (err, lse_err)
    err, lse_err, _ = run_loop([(j, 0) for j in range(3)], 192, 0, seed=3, D=D, nw=4, always_rare=True)
    assert err <= 4e-3 and lse_err <= 2e-3, (err, lse_err)
    err, lse_err, _ = run_loop([(j, _tail(150, j)) for j in range(3)], 150, 0, seed=4, dt="f16", D=D, nw=4)
    assert err <= 2e-3 and lse_err <= 2e-3, (err, lse_err)


@pytest.mark.parametrize("case", sorted(CASES))
def test_wide_loop_dual(case):
    """The dual-wide map of D = 192: 4 waves of 64 rows (two 32-row halves
    sharing each K and V operand read from LDS), 256-row tiles, O of both
    halves and half 1's Q in AGPRs; the wide map's copies and rings."""
    make, nk, n_x = CASES[case]
    err, lse_err, copies = run_loop(make(), nk, n_x, D=192, nw=4, dual=True)
    assert err <= 4e-3 and lse_err <= 2e-3, (case, err, lse_err)
    assert copies == 4 * 8 * (1 + 2 * len(make()))


def test_wide_loop_dual_rare_path_and_fp16():
    err, lse_err, _ = run_loop([(j, 0) for j in range(3)], 192, 0, seed=6, D=192, nw=4, dual=True, always_rare=True)
    assert err <= 4e-3 and lse_err <= 2e-3, (err, lse_err)
    err, lse_err, _ = run_loop([(j, _tail(150, j)) for j in range(3)], 150, 0, seed=7, dt="f16", D=192, nw=4,
                               dual=True)
    assert err <= 2e-3 and lse_err <= 2e-3, (err, lse_err)
