"""The bf16 prefill kernel (crane_amd/csrc/prefill.hip) run on the CPU: the
C++ around the key loop restated in numpy (workgroup map, Q fragments, LDS
tile layout and copy schedule, the first QK^T, the exact few-key waves, the
key-group merge and the output), and every loop step executed from the
generated assembly (prefill_step.inc) by the asm_sim interpreter.

Test infrastructure for the CPU: it checks the assembly's data flow against
the model of the kernel's arithmetic without a GPU.  Copies land in LDS at
the barrier after they are issued, as the kernel waits for them there."""
from __future__ import annotations

import os

import numpy as np

import asm_sim
from asm_sim import LANES, bf16_rne_bits, bf16_to_f32, f32, u32

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "crane_amd", "csrc", "prefill_step.inc")
D, KBM, KBN, TILE = 128, 128, 64, 16384
LONG_ROW_KEYS = 1024
LOG2E = np.float32(1.4426950408889634)
MASK_RAW = np.float32(-1.0e30)

# registers of the generated step's operands (any free ones)
OPS = {"%10": "v230", "%11": "v231", "%16": "s16", "%17": "v232", "%18": "v233", "%19": "s19", "%20": "s20",
       "%=": "0"}


def swz(row):
    return ((row & 3) << 2) | ((row >> 2) & 3)


def tile_bytes(rows):
    """A [64, 128] bf16 tile (uint16 bits) in the LDS layout of the copy:
    16-byte chunk c of row r holds global chunk c ^ swz(r)."""
    out = np.zeros((KBN, 16, 8), np.uint16)
    g = rows.reshape(KBN, 16, 8)
    for r in range(KBN):
        for c in range(16):
            out[r, c] = g[r, c ^ swz(r)]
    return out.reshape(-1).view(np.uint8)


def bf16_bits(x):
    return bf16_rne_bits(np.asarray(x, np.float32)).astype(np.uint16)


def simulate(q, k, v, st, causal, one_rounding=False, cus=256, only=None):
    """q [B, Hq, S, D], k/v [B, Hkv, L, D] float32 holding bf16 values, st [B]
    start positions.  Returns out [B, S, Hq*D] as float32 (bf16 values).
    only: a set of (qt, b, hq) workgroups to run (others stay zero)."""
    B, Hq, S, _ = q.shape
    Hkv = k.shape[1]
    n_rep = Hq // Hkv
    n_qt = (S + KBM - 1) // KBM
    units = n_qt * B * Hkv
    blocks = ((units + 7) // 8) * 8 * n_rep
    split = 2 if blocks <= cus else 1
    macros = asm_sim.load_macros(INC)
    scale = 1.0 / np.sqrt(D)
    scale_f = bf16_to_f32(bf16_rne_bits(np.float32(scale)))
    scale_log2 = np.float32(scale_f * LOG2E)
    out = np.zeros((B, S, Hq, D), np.float32)
    qb, kb, vb = bf16_bits(q), bf16_bits(k), bf16_bits(v)
    lane = np.arange(LANES)
    n, hh = lane % 32, lane // 32
    for qt in range(n_qt):
        for b in range(B):
            for hq in range(Hq):
                if only is not None and (qt, b, hq) not in only:
                    continue
                _workgroup(out, qb, kb, vb, qt, b, hq, int(st[b]), S, n_rep, causal, one_rounding, split, macros,
                           scale_f, scale_log2, n, hh)
    return out.reshape(B, S, Hq * D)


def _workgroup(out, qb, kb, vb, qt, b, hq, start, S, n_rep, causal, one_rounding, split, macros, scale_f,
               scale_log2, n, hh):
    kvh = hq // n_rep
    m0 = qt * KBM
    L = start + S
    kend = min(start + m0 + KBM, L) if causal else L
    n_all = (kend + KBN - 1) // KBN
    half = (n_all + split - 1) // split
    long_rows = (start + m0 + 1 >= LONG_ROW_KEYS) if causal else (L >= LONG_ROW_KEYS)
    R = 1 if (one_rounding and long_rows) else 2
    fac = LOG2E if R == 2 else scale_log2
    K = kb[b, kvh, :L]
    V = vb[b, kvh, :L]

    def tile(src, x):
        rows = np.zeros((KBN, D), np.uint16)
        lo = x * KBN
        cnt = max(0, min(KBN, L - lo))
        if cnt:
            rows[:cnt] = src[lo:lo + cnt]
        return tile_bytes(rows)

    # LDS per group: kbuf[2] at 0 and 16 KiB, vbuf[2] at 32 and 48 KiB
    groups = []
    for grp in range(split):
        t0 = grp * half
        n_tiles = max(0, min(half, n_all - t0))
        lds = np.zeros(4 * TILE, np.uint8)
        pending_copies = []
        if n_tiles > 0:
            pending_copies += [(0, tile(K, t0)), (2 * TILE, tile(V, t0))]
        if n_tiles > 1:
            pending_copies += [(TILE, tile(K, t0 + 1))]
        groups.append(dict(t0=t0, n_tiles=n_tiles, lds=lds, copies=pending_copies, waves=[]))

    def land(g):
        for off, data in g["copies"]:
            g["lds"][off:off + TILE] = data
        g["copies"] = []

    results = {}
    for gi, g in enumerate(groups):
        land(g)
        for w in range(4):
            wv = asm_sim.Wave(g["lds"])
            qrow = m0 + 32 * w + n
            rows_q = np.minimum(qrow, S - 1)
            qf = qb[b, hq, rows_q]                                  # [64, 128] uint16
            qf = np.where((qrow < S)[:, None], qf, 0).astype(np.uint16)
            for ks in range(8):
                words = qf[:, 16 * ks:16 * ks + 16].reshape(LANES, 2, 8)[np.arange(LANES), hh]  # [64, 8]
                wv.v[64 + 4 * ks:68 + 4 * ks] = words.view(np.uint32).reshape(LANES, 4).T
            for ks in range(8):
                wv.v[160 + ks] = (n * 256 + 16 * ((2 * ks + hh) ^ swz(n))).astype(np.uint32)
            vg, vi = lane_split = (np.arange(LANES) >> 4, np.arange(LANES) & 15)
            v_h = vg >> 1
            v_col = 16 * (vg & 1) + 4 * (vi & 3)
            for db in range(4):
                for h in range(2):
                    r = 4 * v_h + (vi >> 2) + 8 * h
                    col = 32 * db + v_col
                    wv.v[168 + 2 * db + h] = (2 * TILE + r * 256 + 16 * ((col >> 3) ^ swz(r)) + 2 * (col & 7)).astype(
                        np.uint32)
            wv.sgpr.update({"s19": int(u32(np.float32(fac))), "s20": int(u32(np.float32(scale_f)))})
            wv.v[232 - 0] = 0
            wv.v[233] = ((np.arange(LANES) ^ 32) << 2).astype(np.uint32)
            wv.v[230] = u32(np.full(LANES, -np.inf, np.float32))
            wv.v[231] = 0
            # S(0) = K(0) Q^T into set 0 (the C++ prologue's MFMAs)
            for nb in range(2):
                for ks in range(8):
                    wv.v[176:180] = _kfrag(g["lds"], wv.v[160 + ks] + nb * 8192)
                    c = "0" if ks == 0 else f"v[{96 + 16 * nb}:{111 + 16 * nb}]"
                    wv.exec("v_mfma_f32_32x32x16_bf16", [f"v[{96 + 16 * nb}:{111 + 16 * nb}]", "v[176:179]",
                                                          f"v[{64 + 4 * ks}:{67 + 4 * ks}]", c])
            wave_first = start + m0 + 32 * w
            exact = gi == 0 and ((wave_first + 31 < KBN) if causal else (L <= KBN))
            if exact:
                _exact_rows(wv, qrow, start, causal, L, kend, scale_f, hh)
            g["waves"].append(dict(w=w, wave=wv, wave_first=wave_first, exact=exact, qrow=qrow, pending=False))

    n_steps = half if split > 1 else groups[0]["n_tiles"]
    for t in range(0, n_steps + 1, 2):
        for t_ in (t, t + 1):
            par = t_ & 1
            for g in groups:
                land(g)                               # copies issued last step land at this barrier
                if t_ + 2 < g["n_tiles"]:
                    g["copies"].append((par * TILE, tile(K, g["t0"] + t_ + 2)))
                if 1 <= t_ < g["n_tiles"]:
                    g["copies"].append((2 * TILE + par * TILE, tile(V, g["t0"] + t_)))
                kt = (g["t0"] + t_) * KBN
                for wd in g["waves"]:
                    wv = wd["wave"]
                    live = t_ < g["n_tiles"] and not wd["exact"] and not (causal and kt > wd["wave_first"] + 31)
                    full = kt + KBN <= kend and not (causal and kt + KBN - 1 > wd["wave_first"])
                    flags = (1 if live else 0) | (2 if full else 0) | (4 if wd["pending"] else 0)
                    qpos = start + wd["qrow"]
                    thr = (np.minimum(qpos, kend - 1) if causal else np.full(LANES, kend - 1)) - kt - 4 * hh
                    wv.sgpr["s16"] = flags
                    wv.v[232] = thr.astype(np.int32).view(np.uint32)
                    wv.run(asm_sim.expand(macros[f"CRANE_PF_STEP_P{par}_R{R}"], OPS))
                    wd["pending"] = live
    # merge the key groups, normalise, store
    for w in range(4):
        wv = groups[0]["waves"][w]["wave"]
        O = f32(wv.v[0:64]).astype(np.float32).copy()           # [64 regs, 64 lanes]
        m = f32(wv.v[230]).copy()
        l = f32(wv.v[231]).copy()
        if split == 2:
            w1 = groups[1]["waves"][w]["wave"]
            O1, m1, l1 = f32(w1.v[0:64]), f32(w1.v[230]), f32(w1.v[231])
            mm = np.maximum(m, m1)
            with np.errstate(invalid="ignore"):
                a0 = np.where(m == -np.inf, 0, np.exp2(m - mm)).astype(np.float32)
                a1 = np.where(m1 == -np.inf, 0, np.exp2(m1 - mm)).astype(np.float32)
            l = (l * a0 + l1 * a1).astype(np.float32)
            O = (O * a0[None, :] + O1 * a1[None, :]).astype(np.float32)
        l = (l + l[np.arange(LANES) ^ 32]).astype(np.float32)
        inv = (np.float32(1.0) / l).astype(np.float32)
        qrow = groups[0]["waves"][w]["qrow"]
        for db in range(4):
            for r in range(16):
                dim = db * 32 + 8 * (r // 4) + 4 * hh + r % 4
                val = bf16_to_f32(bf16_rne_bits((O[16 * db + r] * inv).astype(np.float32)))
                ok = qrow < S
                out[b, qrow[ok], hq, dim[ok]] = val[ok]


def _kfrag(lds, addr):
    data = np.stack([lds[int(a):int(a) + 16] for a in addr]).view(np.uint32).reshape(LANES, 4)
    return data.T


def _exact_rows(wv, qrow, start, causal, L, kend, scale_f, hh):
    """Rows that see tile 0 only: candle's softmax chain in bf16 exactly, then
    O = P V over V(0) (the C++ before the loop)."""
    s = f32(wv.v[96:128]).astype(np.float32).copy()       # [32 regs, 64 lanes], raw scores
    qpos = start + qrow
    for reg in range(32):
        nb, r = reg // 16, reg % 16
        key = nb * 32 + 8 * (r >> 2) + 4 * hh + (r & 3)
        masked = (key >= L) | ((key > qpos) if causal else False)
        s[reg] = np.where(masked, MASK_RAW, s[reg])
    r16 = lambda x: bf16_to_f32(bf16_rne_bits(np.asarray(x, np.float32)))
    sc = r16(r16(s) * scale_f)
    mx = sc.max(0)
    mx = np.maximum(mx, mx[np.arange(LANES) ^ 32])
    e = r16(np.exp2((r16(sc - mx[None, :]) * LOG2E).astype(np.float64)).astype(np.float32))
    ssum = e.sum(0, dtype=np.float32)
    ssum = r16(ssum + ssum[np.arange(LANES) ^ 32])
    p = r16(e / ssum[None, :])
    pk = bf16_rne_bits(p[0::2]) | (bf16_rne_bits(p[1::2]) << 16)
    wv.v[96:112] = pk
    for st in range(4):
        for db in range(4):
            base = 176
            wv.exec("ds_read_b64_tr_b16", ["v[176:177]", f"v{168 + 2 * db} offset:{st * 4096}"])
            wv.exec("ds_read_b64_tr_b16", ["v[178:179]", f"v{169 + 2 * db} offset:{st * 4096}"])
            wv.exec("v_mfma_f32_32x32x16_bf16", [f"v[{16 * db}:{16 * db + 15}]", f"v[{base}:{base + 3}]",
                                                  f"v[{96 + 4 * st}:{99 + 4 * st}]", f"v[{16 * db}:{16 * db + 15}]"])
    wv.v[230] = 0
    wv.v[231] = u32(np.full(LANES, 0.5, np.float32))
