"""CPU model of the gfx950 instructions the single-stream kernel's key loop uses.

Test infrastructure: runs the generated loop text (gen_stream_asm.py) for the
8 waves of one work-group, wave by wave between barriers, over numpy K/V/Q and
a plan in a byte-addressed memory model, so that the loop's logic (pipeline
bookkeeping, LDS ring and swizzle, copies, entry decode, masks, the rare path)
is checked on the CPU.  It models results, not timing: hazards and wait
states are out of its reach (those are pinned by the GPU parity tests).

Semantics modelled (the ones the attention kernels rely on):
  v_mfma_f32_32x32x16_{bf16,f16}: lane l holds A[l%32][8(l/32)..+7],
      B[8(l/32)..+7][l%32]; C/D register r of lane l is element
      (8(r/4) + 4(l/32) + r%4, l%32).
  ds_read_b64_tr_b16: lane i of a 16-lane group gets, as element j, the
      16-bit element i%4 of the 8 bytes addressed by lane 4j + i/4.
  buffer_load_dwordx4 ... lds: lane l's 16 bytes land at M0 + 16 l; dwords
      past num_records (voffset + soffset counted) read as zero.
  v_permlane32_swap_b32 a, b: lanes 32-63 of a trade places with lanes 0-31 of b.
"""
import re
import struct
import sys
from pathlib import Path

import numpy as np

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "longvideosparseattention_amd" / "csrc"))
import gen_stream_asm as G  # noqa: E402

M32 = 0xFFFFFFFF


def i32(x):
    return x - (1 << 32) if x & 0x80000000 else x


def f2u(x):
    return np.asarray(x, dtype=np.float32).view(np.uint32)


def u2f(x):
    return np.asarray(x, dtype=np.uint32).view(np.float32)


def bf16_round(x):
    u = f2u(x).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    # NaN handling not needed
    return r.astype(np.uint32)


def bf16_to_f32(h):
    return u2f((np.asarray(h, dtype=np.uint32) & 0xFFFF) << 16)


class Mem:
    def __init__(self):
        self.bufs = []  # (base, bytearray)
        self.next = 0x100000000

    def alloc(self, data: bytes):
        base = self.next
        self.bufs.append((base, bytearray(data)))
        self.next += (len(data) + 0xFFFF) & ~0xFFFF
        self.next += 0x10000
        return base

    def read(self, addr, n):
        for b, d in self.bufs:
            if b <= addr and addr + n <= b + len(d):
                return bytes(d[addr - b:addr - b + n])
        raise IndexError(f"bad global read {addr:#x}+{n}")


def parse_program(lines):
    prog, labels = [], {}
    for ln in lines:
        ln = ln.strip()
        if not ln or ln.startswith(';'):
            continue
        ln = ln.replace('%=', '0')
        if ln.endswith(':'):
            labels[ln[:-1]] = len(prog)
            continue
        parts = ln.split(None, 1)
        op = parts[0]
        args = [a.strip() for a in re.split(r',(?![^\[]*\])', parts[1])] if len(parts) > 1 else []
        mods = {}
        if args:
            toks = args[-1].split()
            args[-1] = toks[0]
            for t in toks[1:]:
                if ':' in t:
                    k_, v_ = t.split(':')
                    mods[k_] = int(v_, 0)
                else:
                    mods[t] = True
        if 'offset' in mods:
            args.append(f"offset:{mods['offset']}")
        prog.append((op, args, ln))
    return prog, labels


class Wave:
    def __init__(self, wid, sim):
        self.w = wid
        self.sim = sim
        self.v = np.zeros((512, 64), dtype=np.uint32)   # VGPRs, then AGPRs a0.. at 256..
        self.s = [0] * 112
        self.vcc = 0
        self.scc = 0
        self.m0 = 0
        self.pc = 0
        self.done = False

    # operand helpers
    def vreg(self, tok):
        base = 256 if tok[0] == 'a' else 0          # AGPRs follow the VGPRs
        m = re.fullmatch(r'[va](\d+)', tok)
        if m:
            return base + int(m.group(1)), 1
        m = re.fullmatch(r'[va]\[(\d+):(\d+)\]', tok)
        return base + int(m.group(1)), int(m.group(2)) - int(m.group(1)) + 1

    def sreg(self, tok):
        m = re.fullmatch(r's(\d+)', tok)
        if m:
            return int(m.group(1)), 1
        m = re.fullmatch(r's\[(\d+):(\d+)\]', tok)
        return int(m.group(1)), int(m.group(2)) - int(m.group(1)) + 1

    def sval(self, tok):
        """scalar operand value (32-bit)"""
        if tok == 'vcc':
            return self.vcc
        if tok == 'm0':
            return self.m0
        if tok.startswith('s'):
            return self.s[self.sreg(tok)[0]]
        if tok.startswith('0x'):
            return int(tok, 16)
        if tok == '-1':
            return M32
        return int(tok) & M32

    def sval64(self, tok):
        if tok == 'vcc':
            return self.vcc
        if tok == '-1':
            return (1 << 64) - 1
        if tok == '0':
            return 0
        r, n = self.sreg(tok)
        return self.s[r] | (self.s[r + 1] << 32)

    def sset64(self, tok, val):
        val &= (1 << 64) - 1
        if tok == 'vcc':
            self.vcc = val
            return
        r, n = self.sreg(tok)
        self.s[r] = val & M32
        self.s[r + 1] = val >> 32

    def vsrc_u(self, tok):
        """vector source (uint32 per lane)"""
        neg = tok.startswith('-')
        if neg:
            tok = tok[1:]
        if tok.startswith(('v', 'a')):
            x = self.v[self.vreg(tok)[0]].copy()
        elif tok.startswith('s'):
            x = np.full(64, self.s[self.sreg(tok)[0]], dtype=np.uint32)
        elif tok.startswith('0x'):
            x = np.full(64, int(tok, 16), dtype=np.uint32)
        elif tok in ('1.0', '-1.0', '2.0', '0.5'):
            x = f2u(np.full(64, float(tok), dtype=np.float32))
        else:
            x = np.full(64, int(tok) & M32, dtype=np.uint32)
        if neg:
            x = f2u(-u2f(x))
        return x

    def vsrc_f(self, tok):
        return u2f(self.vsrc_u(tok))

    def vdst(self, tok, val):
        self.v[self.vreg(tok)[0]] = np.asarray(val).astype(np.float32).view(np.uint32) \
            if np.asarray(val).dtype == np.float32 else np.asarray(val, dtype=np.uint32)

    def step(self):
        op, a, raw = self.sim.prog[self.pc]
        self.pc += 1
        S = self.s
        if op in ('s_waitcnt', 's_nop', 's_setprio'):
            return
        if op == 's_barrier':
            return 'barrier'
        if op == 's_add_u32':
            r = self.sval(a[1]) + self.sval(a[2])
            self.scc = int(r > M32)
            self._sd(a[0], r & M32)
        elif op == 's_addc_u32':
            r = self.sval(a[1]) + self.sval(a[2]) + self.scc
            self.scc = int(r > M32)
            self._sd(a[0], r & M32)
        elif op == 's_sub_u32':
            x, y = self.sval(a[1]), self.sval(a[2])
            self.scc = int(y > x)
            self._sd(a[0], (x - y) & M32)
        elif op == 's_min_u32':
            self._sd(a[0], min(self.sval(a[1]), self.sval(a[2])))
        elif op == 's_lshl_b32':
            r = (self.sval(a[1]) << (self.sval(a[2]) & 31)) & M32
            self.scc = int(r != 0)
            self._sd(a[0], r)
        elif op == 's_lshr_b32':
            r = self.sval(a[1]) >> (self.sval(a[2]) & 31)
            self.scc = int(r != 0)
            self._sd(a[0], r)
        elif op == 's_and_b32':
            r = self.sval(a[1]) & self.sval(a[2])
            self.scc = int(r != 0)
            self._sd(a[0], r)
        elif op == 's_mul_i32':
            self._sd(a[0], (self.sval(a[1]) * self.sval(a[2])) & M32)
        elif op == 's_mul_hi_u32':
            self._sd(a[0], (self.sval(a[1]) * self.sval(a[2])) >> 32)
        elif op == 's_mov_b32':
            if a[0] == 'm0':
                self.m0 = self.sval(a[1])
            else:
                self._sd(a[0], self.sval(a[1]))
        elif op == 's_cselect_b32':
            self._sd(a[0], self.sval(a[1]) if self.scc else self.sval(a[2]))
        elif op == 's_cselect_b64':
            self.sset64(a[0], self.sval64(a[1]) if self.scc else self.sval64(a[2]))
        elif op == 's_cmp_eq_u32':
            self.scc = int(self.sval(a[0]) == self.sval(a[1]))
        elif op == 's_cmp_lg_u32':
            self.scc = int(self.sval(a[0]) != self.sval(a[1]))
        elif op == 's_cmp_lt_u32':
            self.scc = int(self.sval(a[0]) < self.sval(a[1]))
        elif op == 's_cmp_ge_u32':
            self.scc = int(self.sval(a[0]) >= self.sval(a[1]))
        elif op in ('s_cmp_ge_i32', 's_cmp_le_i32'):
            x, y = (i32(self.sval(t)) for t in a[:2])
            self.scc = int(x >= y if op == 's_cmp_ge_i32' else x <= y)
        elif op == 's_cmp_eq_u64':
            self.scc = int(self.sval64(a[0]) == self.sval64(a[1]))
        elif op == 's_mov_b64':
            self.sset64(a[0], self.sval64(a[1]))
        elif op == 's_bfe_u32':
            x, c = self.sval(a[1]), self.sval(a[2])
            off, wd = c & 31, (c >> 16) & 0x7F
            r = (x >> off) & ((1 << wd) - 1)
            self.scc = int(r != 0)
            self._sd(a[0], r)
        elif op == 's_bitcmp1_b32':
            self.scc = (self.sval(a[0]) >> (self.sval(a[1]) & 31)) & 1
        elif op == 's_and_b64':
            r = self.sval64(a[1]) & self.sval64(a[2])
            self.scc = int(r != 0)
            self.sset64(a[0], r)
        elif op == 's_andn2_b64':
            r = self.sval64(a[1]) & ~self.sval64(a[2])
            self.scc = int(r != 0)
            self.sset64(a[0], r)
        elif op == 's_or_b64':
            r = self.sval64(a[1]) | self.sval64(a[2])
            self.scc = int(r != 0)
            self.sset64(a[0], r)
        elif op == 's_cbranch_scc1':
            if self.scc:
                self.pc = self.sim.labels[a[0].replace('%=', '0')]
        elif op == 's_cbranch_scc0':
            if not self.scc:
                self.pc = self.sim.labels[a[0].replace('%=', '0')]
        elif op == 's_cbranch_vccnz':
            if self.vcc:
                self.pc = self.sim.labels[a[0].replace('%=', '0')]
        elif op == 's_branch':
            self.pc = self.sim.labels[a[0].replace('%=', '0')]
        elif op == 's_call_b64':
            self.sset64(a[0], self.pc)
            self.pc = self.sim.labels[a[1].replace('%=', '0')]
        elif op == 's_setpc_b64':
            self.pc = self.sval64(a[0])
        elif op == 's_load_dwordx2':
            base = self.sval64(a[1])
            off = self.sval(a[2]) if a[2].startswith('s') else int(a[2], 0)
            d = self.sim.mem.read(base + off, 8)
            r, _ = self.sreg(a[0])
            S[r], S[r + 1] = struct.unpack('<II', d)
        elif op == 'buffer_load_dwordx4':
            vo = self.v[self.vreg(a[0])[0]]
            r, _ = self.sreg(a[1])
            base = S[r] | ((S[r + 1] & 0xFFFF) << 32)
            nrec = S[r + 2]
            so = self.sval(a[2])
            lds = self.sim.lds
            for ln in range(64):
                off = (int(vo[ln]) + so) & M32       # 32-bit offset arithmetic
                dst = self.m0 + 16 * ln
                for dw in range(4):
                    o = off + 4 * dw
                    val = self.sim.mem.read(base + o, 4) if o + 4 <= nrec else b'\0\0\0\0'
                    assert 0 <= dst and dst + 4 * dw + 4 <= len(lds), f"LDS copy out of range: {dst:#x}"
                    lds[dst + 4 * dw:dst + 4 * dw + 4] = val
            self.sim.copies += 1
        elif op == 'ds_read_b128' or op == 'ds_read_b64_tr_b16':
            dreg, n = self.vreg(a[0])
            addr = self.v[self.vreg(a[1])[0]].astype(np.int64)
            off = int(a[2].split(':')[1]) if len(a) > 2 else 0
            addr = addr + off
            lds = np.frombuffer(bytes(self.sim.lds), dtype=np.uint8)
            if op == 'ds_read_b128':
                for ln in range(64):
                    x = int(addr[ln])
                    assert 0 <= x and x + 16 <= len(lds), x
                    self.v[dreg:dreg + 4, ln] = np.frombuffer(lds[x:x + 16].tobytes(), dtype=np.uint32)
            else:
                res = np.zeros((64, 4), dtype=np.uint32)
                for ln in range(64):
                    g, i = ln // 16, ln % 16
                    for j in range(4):
                        src = 16 * g + 4 * j + i // 4
                        x = int(addr[src]) + 2 * (i % 4)
                        assert 0 <= x and x + 2 <= len(lds), x
                        res[ln, j] = int(lds[x]) | (int(lds[x + 1]) << 8)
                self.v[dreg, :] = res[:, 0] | (res[:, 1] << 16)
                self.v[dreg + 1, :] = res[:, 2] | (res[:, 3] << 16)
        elif op.startswith('v_mfma_f32_16x16x32'):
            # lane l: A[l%16][8(l/16)..+7], B[8(l/16)..+7][l%16]; D register r of
            # lane l is element (4(l/16) + r, l%16)
            bf = op.endswith('bf16')
            d, _ = self.vreg(a[0])
            ra, _ = self.vreg(a[1])
            rb, _ = self.vreg(a[2])
            cv = None if a[3] == '0' else self.vreg(a[3])[0]
            conv = (lambda h: bf16_to_f32(h)) if bf else (lambda h: (h & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float32))

            def elems16(r0):
                x = self.v[r0:r0 + 4].T
                return np.stack([conv(x & 0xFFFF), conv(x >> 16)], axis=2).reshape(64, 8)
            Ae, Be = elems16(ra), elems16(rb)
            A = np.zeros((16, 32), dtype=np.float64)
            B = np.zeros((32, 16), dtype=np.float64)
            for ln in range(64):
                A[ln % 16, 8 * (ln // 16):8 * (ln // 16) + 8] = Ae[ln]
                B[8 * (ln // 16):8 * (ln // 16) + 8, ln % 16] = Be[ln]
            Cm = np.zeros((16, 16), dtype=np.float64)
            if cv is not None:
                for ln in range(64):
                    for r in range(4):
                        Cm[4 * (ln // 16) + r, ln % 16] = u2f(self.v[cv + r, ln])
            with np.errstate(invalid="ignore", over="ignore"):   # inf * 0 of the first block -> NaN
                Dm = (A @ B + Cm).astype(np.float32)
            out = np.zeros((4, 64), dtype=np.float32)
            for ln in range(64):
                for r in range(4):
                    out[r, ln] = Dm[4 * (ln // 16) + r, ln % 16]
            self.v[d:d + 4] = out.view(np.uint32)
        elif op.startswith('v_mfma_f32_32x32x16'):
            bf = op.endswith('bf16')
            d, _ = self.vreg(a[0])
            ra, _ = self.vreg(a[1])
            rb, _ = self.vreg(a[2])
            cv = None if a[3] == '0' else self.vreg(a[3])[0]
            conv = (lambda h: bf16_to_f32(h)) if bf else (lambda h: (h & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float32))

            def elems(r0):  # [64 lanes, 8 elements]
                x = self.v[r0:r0 + 4].T  # [64, 4] uint32
                lo = conv(x & 0xFFFF)
                hi = conv(x >> 16)
                return np.stack([lo, hi], axis=2).reshape(64, 8)
            Ae = elems(ra)
            Be = elems(rb)
            A = np.zeros((32, 16), dtype=np.float64)
            B = np.zeros((16, 32), dtype=np.float64)
            for ln in range(64):
                A[ln % 32, 8 * (ln // 32):8 * (ln // 32) + 8] = Ae[ln]
                B[8 * (ln // 32):8 * (ln // 32) + 8, ln % 32] = Be[ln]
            Cm = np.zeros((32, 32), dtype=np.float64)
            if cv is not None:
                for ln in range(64):
                    for r in range(16):
                        Cm[8 * (r // 4) + 4 * (ln // 32) + r % 4, ln % 32] = u2f(self.v[cv + r, ln])
            Dm = (A @ B + Cm).astype(np.float32)
            out = np.zeros((16, 64), dtype=np.float32)
            for ln in range(64):
                for r in range(16):
                    out[r, ln] = Dm[8 * (r // 4) + 4 * (ln // 32) + r % 4, ln % 32]
            self.v[d:d + 16] = out.view(np.uint32)
        elif op == 'v_fma_f32':
            x, y, z = (self.vsrc_f(t) for t in a[1:4])
            self.vdst(a[0], (x.astype(np.float64) * y + z).astype(np.float32))
        elif op == 'v_exp_f32':
            with np.errstate(over='ignore'):
                self.vdst(a[0], np.exp2(self.vsrc_f(a[1]).astype(np.float64)).astype(np.float32))
        elif op == 'v_cvt_pk_bf16_f32':
            lo, hi = bf16_round(self.vsrc_f(a[1])), bf16_round(self.vsrc_f(a[2]))
            self.vdst(a[0], (lo | (hi << 16)).astype(np.uint32))
        elif op == 'v_cvt_pk_f16_f32':
            lo = self.vsrc_f(a[1]).astype(np.float16).view(np.uint16).astype(np.uint32)
            hi = self.vsrc_f(a[2]).astype(np.float16).view(np.uint16).astype(np.uint32)
            self.vdst(a[0], lo | (hi << 16))
        elif op in ('v_dot2c_f32_bf16', 'v_dot2c_f32_f16'):
            p = self.vsrc_u(a[2])
            if op.endswith('bf16'):
                lo, hi = bf16_to_f32(p & 0xFFFF), bf16_to_f32(p >> 16)
            else:
                lo = (p & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float32)
                hi = (p >> 16).astype(np.uint16).view(np.float16).astype(np.float32)
            acc = self.vsrc_f(a[0])
            self.vdst(a[0], (acc + lo + hi).astype(np.float32))
        elif op in ('v_dot2_f32_bf16', 'v_dot2_f32_f16'):
            def pairs(x):
                if op.endswith('bf16'):
                    return bf16_to_f32(x & 0xFFFF), bf16_to_f32(x >> 16)
                return ((x & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float32),
                        (x >> 16).astype(np.uint16).view(np.float16).astype(np.float32))
            a0, a1 = pairs(self.vsrc_u(a[1]))
            b0, b1 = pairs(self.vsrc_u(a[2]))
            self.vdst(a[0], (a0 * b0 + a1 * b1 + self.vsrc_f(a[3])).astype(np.float32))
        elif op in ('v_mov_b32', 'v_accvgpr_read_b32', 'v_accvgpr_write_b32'):
            self.vdst(a[0], self.vsrc_u(a[1]))
        elif op == 'v_add_f32':
            self.vdst(a[0], (self.vsrc_f(a[1]) + self.vsrc_f(a[2])).astype(np.float32))
        elif op == 'v_sub_f32':
            self.vdst(a[0], (self.vsrc_f(a[1]) - self.vsrc_f(a[2])).astype(np.float32))
        elif op == 'v_mul_f32':
            self.vdst(a[0], (self.vsrc_f(a[1]) * self.vsrc_f(a[2])).astype(np.float32))
        elif op == 'v_max_f32':
            self.vdst(a[0], np.maximum(self.vsrc_f(a[1]), self.vsrc_f(a[2])).astype(np.float32))
        elif op == 'v_max3_f32':
            self.vdst(a[0], np.maximum(np.maximum(self.vsrc_f(a[1]), self.vsrc_f(a[2])), self.vsrc_f(a[3])).astype(np.float32))
        elif op == 'v_cmp_nge_f32':
            x, y = self.vsrc_f(a[1]), self.vsrc_f(a[2])
            bits = ~(x >= y)
            self.vcc = int(sum(int(b) << i for i, b in enumerate(bits)))
        elif op == 'v_cmp_lt_i32':
            x, y = self.vsrc_u(a[1]).view(np.int32), self.vsrc_u(a[2]).view(np.int32)
            bits = x < y
            self.vcc = int(sum(int(b) << i for i, b in enumerate(bits)))
        elif op == 'v_cmp_ge_u32_e64':
            x, y = self.vsrc_u(a[1]), self.vsrc_u(a[2])
            bits = x >= y
            self.sset64(a[0], int(sum(int(b) << i for i, b in enumerate(bits))))
        elif op == 'v_cndmask_b32_e64':
            m = self.sval64(a[3])
            bits = np.array([(m >> i) & 1 for i in range(64)], dtype=bool)
            self.vdst(a[0], np.where(bits, self.vsrc_u(a[2]), self.vsrc_u(a[1])))
        elif op == 'v_add_u32':
            self.vdst(a[0], (self.vsrc_u(a[1]).astype(np.int64) + self.vsrc_u(a[2])) & M32)
        elif op == 'v_sub_u32':
            self.vdst(a[0], (self.vsrc_u(a[1]).astype(np.int64) - self.vsrc_u(a[2])) & M32)
        elif op == 'v_mad_u32_u24':
            x, y, z = (self.vsrc_u(t).astype(np.uint64) for t in a[1:4])
            self.vdst(a[0], (((x & 0xFFFFFF) * (y & 0xFFFFFF) + z) & M32).astype(np.uint32))
        elif op == 'v_permlane32_swap_b32':
            r0, r1 = self.vreg(a[0])[0], self.vreg(a[1])[0]
            x, y = self.v[r0].copy(), self.v[r1].copy()
            self.v[r0, 32:], self.v[r1, :32] = y[:32], x[32:]
        else:
            raise NotImplementedError(raw)

    def _sd(self, tok, val):
        if tok == 'm0':
            self.m0 = val & M32
        else:
            self.s[self.sreg(tok)[0]] = val & M32


class Sim:
    def __init__(self, dt='bf16', **opts):
        # the product's loop for the head size, with any options of the test on top
        D, nw = opts.get("D", 128), opts.get("nw", 8)
        dual = opts.get("dual")
        dual = (nw == 4 and D == 64) if dual is None else dual
        lines = G.Gen(dt, **{**G.map_opts(D, nw, dual), **opts}).build()
        self.nw = opts.get("nw", 8)
        self.prog, self.labels = parse_program(lines)
        self.mem = Mem()
        self.lds = bytearray(131072)
        self.copies = 0

    def run(self, waves, max_steps=10_000_000):
        active = list(waves)
        steps = 0
        while True:
            at_barrier = 0
            for w in waves:
                if w.done:
                    continue
                while True:
                    if w.pc >= len(self.prog) or w.pc == self.labels['END_0']:
                        w.done = True
                        break
                    r = w.step()
                    steps += 1
                    assert steps < max_steps
                    if r == 'barrier':
                        at_barrier += 1
                        break
            if all(w.done for w in waves):
                return
            alive = [w for w in waves if not w.done]
            assert at_barrier == len(alive), "barrier mismatch"
