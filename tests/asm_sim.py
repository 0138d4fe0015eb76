"""A CPU interpreter for the gfx950 instructions of the prefill step's
generated assembly (crane_amd/csrc/prefill_step.inc), one wave of 64 lanes.

Test infrastructure: it runs the generated text on numpy registers and LDS so
the assembly's data flow (register map, in-place P pairs, LDS addresses,
branches) can be checked on the CPU against the model of the kernel's
arithmetic.  Floating point follows IEEE f32 (products and sums formed in f64
and rounded once, where the hardware may round differently in the last bit;
MFMA sums are taken in f64), so results are compared within a bound, not bit
for bit.

Operand layouts (CDNA3/CDNA4 ISA):
  v_mfma_f32_32x32x16_bf16 D, A, B, C: lane l holds A[l % 32][8 (l // 32) + e]
    and B[8 (l // 32) + e][l % 32] for e = 0..7 (bf16 pairs, low half first);
    register r of D holds D[8 (r // 4) + 4 (l // 32) + r % 4][l % 32].
  ds_read_b64_tr_b16: within each group of 16 lanes, lane i supplies the 4
    bf16 x[i][0..3] at its address and receives x[4 k + i // 4][i % 4] for
    k = 0..3.
"""
from __future__ import annotations

import re

import numpy as np

LANES = 64


def f32(u):
    return np.asarray(u, dtype=np.uint32).view(np.float32)


def u32(f):
    return np.asarray(f, dtype=np.float32).view(np.uint32)


def bf16_rne_bits(f):
    """f32 -> bf16 bits, round to nearest even (NaN kept quiet)."""
    u = u32(np.asarray(f, np.float32)).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    nan = np.isnan(np.asarray(f, np.float32))
    return np.where(nan, 0x7FC0, r).astype(np.uint32)


def bf16_to_f32(bits):
    return f32((np.asarray(bits, np.uint32) & 0xFFFF) << 16)


class Wave:
    def __init__(self, lds: np.ndarray):
        self.v = np.zeros((256, LANES), np.uint32)
        self.sgpr = {}
        self.vcc = np.zeros(LANES, bool)
        self.scc = False
        self.lds = lds  # uint8 array shared by the workgroup

    # ---- operands -------------------------------------------------------
    def vreg(self, tok):
        m = re.fullmatch(r"v(\d+)", tok)
        return int(m.group(1))

    def vrange(self, tok):
        m = re.fullmatch(r"v\[(\d+):(\d+)\]", tok)
        if m:
            return int(m.group(1)), int(m.group(2)) - int(m.group(1)) + 1
        return self.vreg(tok), 1

    def read(self, tok):
        """A 32-bit source operand as uint32[64] (negation prefix allowed for floats)."""
        neg = tok.startswith("-")
        t = tok[1:] if neg else tok
        if re.fullmatch(r"v\d+", t):
            x = self.v[self.vreg(t)].copy()
        elif re.fullmatch(r"s\d+", t):
            x = np.full(LANES, self.sgpr[t], np.uint32)
        elif t.startswith("0x"):
            x = np.full(LANES, int(t, 16), np.uint32)
        elif t in ("1.0", "-1.0", "0.5", "2.0", "4.0"):
            x = np.full(LANES, u32(np.float32(float(t))), np.uint32)
        else:
            x = np.full(LANES, np.uint32(int(t) & 0xFFFFFFFF), np.uint32)
        if neg:
            x = x ^ np.uint32(0x80000000)
        return x

    def write(self, tok, val):
        self.v[self.vreg(tok)] = np.asarray(val).astype(np.uint32, copy=False) if np.asarray(val).dtype == np.uint32 \
            else u32(np.asarray(val, np.float32))

    # ---- LDS ------------------------------------------------------------
    def lds_read(self, addr, nbytes):
        out = np.zeros((LANES, nbytes), np.uint8)
        for l in range(LANES):
            a = int(addr[l])
            if 0 <= a and a + nbytes <= self.lds.size:
                out[l] = self.lds[a:a + nbytes]
        return out

    # ---- execution ------------------------------------------------------
    def run(self, lines):
        labels = {ln[:-1]: i for i, ln in enumerate(lines) if ln.endswith(":")}
        pc = 0
        steps = 0
        while pc < len(lines):
            steps += 1
            assert steps < 100000, "runaway"
            ln = lines[pc]
            pc += 1
            if ln.endswith(":"):
                continue
            op, *rest = ln.split(None, 1)
            args = [a.strip() for a in rest[0].split(",")] if rest else []
            jump = self.exec(op, args)
            if jump is not None:
                pc = labels[jump]

    def exec(self, op, a):
        v = self.v
        if op in ("s_nop", "s_waitcnt"):
            return None
        if op == "s_mov_b32":
            self.sgpr[a[0]] = int(a[1], 0) & 0xFFFFFFFF
        elif op == "s_bitcmp1_b32":
            self.scc = bool((self.sgpr[a[0]] >> int(a[1])) & 1)
        elif op == "s_cbranch_scc0":
            return a[0] if not self.scc else None
        elif op == "s_cbranch_scc1":
            return a[0] if self.scc else None
        elif op == "s_branch":
            return a[0]
        elif op == "s_cmp_eq_u32":
            self.scc = self.sgpr[a[0]] == int(a[1], 0)
        elif op == "s_cmp_lg_u64":
            assert a[0] == "vcc" and a[1] == "0"
            self.scc = bool(self.vcc.any())
        elif op == "s_cselect_b32":
            self.sgpr[a[0]] = int(a[1], 0) if self.scc else int(a[2], 0)
        elif op == "s_or_b64":
            assert a[0] == "vcc" and a[1] == "vcc"
            self.vcc = self.vcc | self.sgpr[a[2]]
        elif op in ("v_mov_b32", "v_mov_b32_e32"):
            v[self.vreg(a[0])] = self.read(a[1])
        elif op == "v_xor_b32_e32":
            v[self.vreg(a[0])] = self.read(a[1]) ^ self.read(a[2])
        elif op == "v_cvt_pk_bf16_f32":
            lo = bf16_rne_bits(f32(self.read(a[1])))
            hi = bf16_rne_bits(f32(self.read(a[2])))
            v[self.vreg(a[0])] = lo | (hi << 16)
        elif op in ("v_mul_f32_e32", "v_add_f32_e32", "v_sub_f32_e32"):
            x, y = f32(self.read(a[1])), f32(self.read(a[2]))
            r = {"v_mul_f32_e32": x * y, "v_add_f32_e32": x + y, "v_sub_f32_e32": x - y}[op]
            v[self.vreg(a[0])] = u32(r.astype(np.float32))
        elif op == "v_fma_f32":
            x, y, z = (f32(self.read(t)).astype(np.float64) for t in a[1:])
            with np.errstate(invalid="ignore", over="ignore"):
                v[self.vreg(a[0])] = u32((x * y + z).astype(np.float32))
        elif op == "v_exp_f32_e32":
            with np.errstate(over="ignore", invalid="ignore"):
                v[self.vreg(a[0])] = u32(np.exp2(f32(self.read(a[1])).astype(np.float64)).astype(np.float32))
        elif op == "v_dot2c_f32_bf16_e32":
            s0, s1 = self.read(a[1]), self.read(a[2])
            acc = f32(v[self.vreg(a[0])]).astype(np.float64)
            r = acc + bf16_to_f32(s0).astype(np.float64) * bf16_to_f32(s1) + \
                bf16_to_f32(s0 >> 16).astype(np.float64) * bf16_to_f32(s1 >> 16)
            v[self.vreg(a[0])] = u32(r.astype(np.float32))
        elif op in ("v_max3_f32", "v_max_f32_e32"):
            xs = [f32(self.read(t)) for t in a[1:]]
            r = xs[0]
            for x in xs[1:]:
                r = np.maximum(r, x)
            v[self.vreg(a[0])] = u32(r)
        elif op == "v_cmp_le_i32_e32":
            assert a[0] == "vcc"
            self.vcc = self.read(a[1]).view(np.int32) <= self.read(a[2]).view(np.int32)
        elif op == "v_cmp_lt_f32_e32":
            assert a[0] == "vcc"
            self.vcc = f32(self.read(a[1])) < f32(self.read(a[2]))
        elif op == "v_cmp_nge_f32_e32":  # not (a >= b): true when unordered
            assert a[0] == "vcc"
            with np.errstate(invalid="ignore"):
                self.vcc = ~(f32(self.read(a[1])) >= f32(self.read(a[2])))
        elif op == "v_cmp_class_f32_e64":
            assert a[2] == "4"
            r = f32(self.read(a[1])) == -np.inf
            if a[0] == "vcc":
                self.vcc = r
            else:
                self.sgpr[a[0]] = r
        elif op == "v_cndmask_b32_e32":
            assert a[3] == "vcc"
            v[self.vreg(a[0])] = np.where(self.vcc, self.read(a[2]), self.read(a[1]))
        elif op == "v_cndmask_b32_e64":
            assert a[3] == "vcc"
            v[self.vreg(a[0])] = np.where(self.vcc, self.read(a[2]), self.read(a[1]))
        elif op == "ds_read_b128":
            base, n = self.vrange(a[0])
            addr = self._address(a[1])
            data = self.lds_read(addr, 16).view(np.uint32).reshape(LANES, 4)
            v[base:base + 4] = data.T
        elif op == "ds_read_b64_tr_b16":
            base, n = self.vrange(a[0])
            addr = self._address(a[1])
            x = self.lds_read(addr, 8).view(np.uint16).reshape(LANES, 4)
            out = np.zeros((LANES, 4), np.uint16)
            for g in range(4):
                for i in range(16):
                    for k in range(4):
                        out[16 * g + i, k] = x[16 * g + 4 * k + i // 4, i % 4]
            v[base:base + 2] = out.view(np.uint32).reshape(LANES, 2).T
        elif op == "ds_bpermute_b32":
            addr = v[self.vreg(a[1])] // 4
            v[self.vreg(a[0])] = self.read(a[2])[addr % LANES]
        elif op == "v_mfma_f32_32x32x16_bf16":
            self._mfma(a)
        else:
            raise NotImplementedError(op)
        return None

    def _address(self, tok):
        """`vN offset:K` -> per-lane byte address."""
        parts = tok.split()
        off = int(parts[1].split(":")[1]) if len(parts) > 1 else 0
        return self.v[self.vreg(parts[0])].astype(np.int64) + off

    # lane l, element e (0..7) of an A/B operand -> (row or column, k)
    _L = np.arange(LANES)
    _AB_K = 8 * (_L[:, None] // 32) + np.arange(8)[None, :]           # [64, 8]
    _AB_MN = np.repeat((_L % 32)[:, None], 8, axis=1)                  # [64, 8]
    # lane l, register r of C/D -> (row, column)
    _CD_ROW = 8 * (np.arange(16)[None, :] // 4) + 4 * (_L[:, None] // 32) + np.arange(16)[None, :] % 4
    _CD_COL = np.repeat((_L % 32)[:, None], 16, axis=1)

    def _operand_bf16(self, base):
        w = self.v[base:base + 4].T.astype(np.uint32)                  # [64, 4]
        halves = np.stack([w & 0xFFFF, w >> 16], axis=2).reshape(LANES, 8)
        return bf16_to_f32(halves).astype(np.float64)                  # [64, 8]

    def _mfma(self, a):
        d0, dn = self.vrange(a[0])
        a0, _ = self.vrange(a[1])
        b0, _ = self.vrange(a[2])
        assert dn == 16
        A = np.zeros((32, 16))
        Bm = np.zeros((16, 32))
        A[self._AB_MN, self._AB_K] = self._operand_bf16(a0)
        Bm[self._AB_K, self._AB_MN] = self._operand_bf16(b0)
        D = A @ Bm
        if a[3] != "0":
            c0, _ = self.vrange(a[3])
            C = np.zeros((32, 32))
            C[self._CD_ROW, self._CD_COL] = f32(self.v[c0:c0 + 16].T)
            D = D + C
        D = D.astype(np.float32)
        self.v[d0:d0 + 16] = u32(D[self._CD_ROW, self._CD_COL]).T


def expand(text: str, operands: dict) -> list:
    """The lines of one generated asm string (the C macro's body) with the
    %N operands replaced by register names."""
    lines = []
    for ln in text:
        for k in sorted(operands, key=lambda s: -len(s)):
            ln = ln.replace(k, operands[k])
        lines.append(ln.strip())
    return [ln for ln in lines if ln]


def load_macros(path: str) -> dict:
    """{macro name: [asm lines]} from prefill_step.inc."""
    out, cur, name = {}, None, None
    for raw in open(path):
        m = re.match(r"#define (\w+) \\", raw)
        if m:
            name, cur = m.group(1), []
            out[name] = cur
            continue
        if cur is not None:
            m = re.match(r'\s*"(.*)\\n" \\$', raw.rstrip("\n"))
            if m:
                cur.append(m.group(1))
            else:
                cur = None
    return out
