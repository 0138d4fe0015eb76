#!/usr/bin/env python3
"""Write prefill_step.inc: one step of the bf16 flash prefill's key loop
(prefill.hip) as inline gfx950 assembly over a fixed register map.

A wave (32 query rows) walks the 64-key tiles of its rows.  Tile t's raw
scores S(t) = K(t) Q^T sit in the score set of parity t & 1; the P V product
of a tile runs one step later.  A step over tile t has two halves:

  PRE   O^T += V(t-1)^T P(t-1)^T (16 v_mfma_f32_32x32x16_bf16: 4 dim blocks x
        4 key steps of 16; the A operand by transposed reads ds_read_b64_tr_b16
        of the row-major V tile, the B operand the P pairs of the last step),
        beside candle's rounding of S(t)'s scores (bf16(q.k), and for R = 2
        bf16(bf16(q.k) * scale)), written over the raw scores in place;
  POST  S(t+1) = K(t+1) Q^T (16 MFMAs: 2 blocks of 32 keys x 8 steps of 16
        dims, K fragments by ds_read_b128) into the other score set, beside
        p = bf16(exp2(s * fac - m)) for the 32 scores a lane holds, written as
        packed bf16 pairs into the P registers, and their sum (v_dot2c against
        (1, 1)), added to the row sum l.

The reference max m moves (every row of the wave to its max of s * fac, O and
l scaled by exp2(m - m_new)) when a row has no reference yet (its first tile),
and otherwise after the fact: when some lane's sum of p passes 256 or is not
finite, the max is taken and the p computed again from the intact scores.

The step is one asm statement (the compiler's register allocator copies the
pinned state around asm statements on alternative paths of a branch), so its
cases branch inside it on a flags operand (bit 0: the tile has keys for this
wave; bit 1: no key of the tile is masked; bit 2: a P V is pending).  A tile
without keys for the wave runs only the pending P V; a tile with masked keys
(diagonal, last) first sets them to a huge negative raw score.

Register map (every other value the loop carries is an ordinary operand):

  v[0:63]     O^T accumulators, 4 dim blocks of 16
  v[64:95]    Q fragments, 8 steps of 4
  v[96:127]   score set 0, v[128:159] score set 1
  v[160:167]  K fragment LDS addresses (one per 16-dim step)
  v[168:175]  V^T fragment LDS addresses (dim block db, half h: 168 + 2 db + h)
  v[176:207]  scratch: a ring of 6 fragment buffers, 4 softmax temporaries,
              the lane's max, a temporary, -m and the tile's sum of p
  v[208:223]  the P pairs of the last softmax, read by the next step's P V

Wait states (gfx950, as the compiler places them for the same patterns): an
MFMA result read by VALU or memory needs 12 (s_nop 11 after each MFMA run), a
VALU write read by an MFMA as A/B/C needs 2 (s_nop 1 before each MFMA run), a
v_exp_f32 result read by VALU needs 1, a v_dot2c result read by VALU needs 3
(both checked below; v_dot2c chains and a VALU write read by v_dot2c need
none), a v_cmp result read as a lane mask gets 2 (s_nop 1), LDS reads are
waited for with s_waitcnt lgkmcnt before the MFMA that consumes them.

Usage: python gen_prefill_step.py  (rewrites prefill_step.inc beside it)."""
from __future__ import annotations

import os

OACC = [0, 16, 32, 48]
QF = 64
SET = [96, 128]
KOFF = 160
VOFF = 168
RING = 176          # 6 fragment buffers of 4 registers
N_RING = 6
TMP = 200           # 4 softmax temporaries
TMAX, TVAL, NEGM, PSUM = 204, 205, 206, 207
PB = 208            # 16 registers: the P pairs of the last softmax, read by the next P V
LOOKAHEAD = 4       # fragment reads issued this many MFMAs ahead
SUM_ADD = False     # row sum by v_dot2c of the bf16 p (False) or v_add_f32 of the f32 p
UNITS = 2           # score pairs interleaved stage by stage in the exp2 list
PRE_VALU = 8        # VALU instructions before a run's first MFMA
TILE = 16384        # bytes of one K or V tile in LDS
ONES = "0x3f803f80"      # the bf16 pair (1, 1)
MASK_RAW = "0xf149f2ca"  # -1e30f, the raw score of a masked key
NO_KEY = "0xee013f39"     # -1e28f: a row max of s * fac at or below it saw no key (a masked key: -1.3e29)
PSUM_MAX = "0x43800000"  # 256.0: a lane's sum of p above it (or not finite) redoes the tile
NEG_INF = "0xff800000"
RESCALE_LOG2 = "0x41000000"  # 8.0: m moves before any p passes 2^8
FLAG_LIVE, FLAG_FULL, FLAG_PENDING = 0, 1, 2

# operand numbers of the step's asm statement (pf_step in prefill.hip)
OP_M, OP_L = "%10", "%11"
OP_FLAGS, OP_THR, OP_XADDR, OP_FAC, OP_SCALE = "%16", "%17", "%18", "%19", "%20"


def v(i, n=1):
    return f"v{i}" if n == 1 else f"v[{i}:{i + n - 1}]"


def mfma_order(with_pv, with_qk):
    """MFMAs of a run in issue order."""
    pv = [("pv", st, db) for st in range(4) for db in range(4)] if with_pv else []
    qk1 = [("qk", ks, 1) for ks in range(8)] if with_qk else []
    qk0 = [("qk", ks, 0) for ks in range(8)] if with_qk else []
    if with_pv and with_qk:
        order = []
        for g in range(8):      # every P V MFMA before the S(t+1) block over P(t-1)
            order += [pv[2 * g], pv[2 * g + 1], qk1[g]]
        return order + qk0
    if with_qk:
        return [m for pair in zip(qk0, qk1) for m in pair]
    return pv


def reads_for(m, pset, buf):
    """LDS reads that fill fragment buffer `buf` for MFMA m; pset: parity of
    the K tile (QK^T) or of the V tile and P pairs (P V)."""
    b = RING + 4 * buf
    if m[0] == "qk":
        _, ks, nb = m
        return [f"ds_read_b128 {v(b, 4)}, {v(KOFF + ks)} offset:{pset * TILE + nb * 8192}"]
    _, st, db = m
    off = pset * TILE + st * 4096
    return [f"ds_read_b64_tr_b16 {v(b, 2)}, {v(VOFF + 2 * db)} offset:{off}",
            f"ds_read_b64_tr_b16 {v(b + 2, 2)}, {v(VOFF + 2 * db + 1)} offset:{off}"]


def mfma_text(m, pset, buf, first_in_chain):
    a = v(RING + 4 * buf, 4)
    if m[0] == "qk":
        _, ks, nb = m
        d = v(SET[pset] + 16 * nb, 16)
        c = "0" if first_in_chain else d
        return f"v_mfma_f32_32x32x16_bf16 {d}, {a}, {v(QF + 4 * ks, 4)}, {c}"
    _, st, db = m
    d = v(OACC[db], 16)
    return f"v_mfma_f32_32x32x16_bf16 {d}, {a}, {v(PB + 4 * st, 4)}, {d}"


def round_list(par, R):
    """The m-independent part of the softmax of the set of parity `par`:
    candle's rounded score (bf16(q.k), and for R = 2 bf16(bf16(q.k) * scale))
    written over each raw score in place, eight scores a stage so every
    result is read two or more instructions after it is written."""
    cur = SET[par]
    out = []
    for g in range(4):
        regs = [v(cur + 8 * g + i) for i in range(8)]
        out += [f"v_cvt_pk_bf16_f32 {r}, 0, {r}" for r in regs]
        if R == 2:  # candle's second rounding: bf16(bf16(q.k) * scale)
            out += [f"v_mul_f32_e32 {r}, {OP_SCALE}, {r}" for r in regs]
            out += [f"v_cvt_pk_bf16_f32 {r}, 0, {r}" for r in regs]
    return out


def exp_list(par):
    """The rest of the softmax of the set of parity `par` (rounded scores in
    place, -m in NEGM): p = bf16(exp2(s * fac - m)) as packed pairs into PB,
    and the lane's sum of the bf16 p into PSUM.  Two score pairs at a time,
    interleaved stage by stage."""
    cur = SET[par]
    out = [f"v_mov_b32 {v(PSUM)}, 0"]
    tmps = [TMP, TMP + 1, TMP + 2, TMP + 3] + [RING + 4 * N_RING + i for i in range(4)]
    assert UNITS <= 2 or N_RING <= 5, "four exp2 units need the last fragment buffer as temporaries"
    for k0 in range(0, 16, UNITS):
        units = []
        for j, k in enumerate(range(k0, k0 + UNITS)):
            ta, tb = tmps[2 * j], tmps[2 * j + 1]
            s0, s1 = cur + 2 * k, cur + 2 * k + 1
            u = [f"v_fma_f32 {v(ta)}, {v(s0)}, {OP_FAC}, {v(NEGM)}",
                 f"v_fma_f32 {v(tb)}, {v(s1)}, {OP_FAC}, {v(NEGM)}",
                 f"v_exp_f32_e32 {v(ta)}, {v(ta)}",
                 f"v_exp_f32_e32 {v(tb)}, {v(tb)}",
                 f"v_cvt_pk_bf16_f32 {v(PB + k)}, {v(ta)}, {v(tb)}"]    # P pair k
            if SUM_ADD:
                u += [f"v_add_f32_e32 {v(PSUM)}, {v(PSUM)}, {v(ta)}",
                      f"v_add_f32_e32 {v(PSUM)}, {v(PSUM)}, {v(tb)}"]
            else:
                u += [f"v_dot2c_f32_bf16_e32 {v(PSUM)}, {ONES}, {v(PB + k)}"]
            units.append(u)
        for stage in zip(*units):
            out += list(stage)
    if not SUM_ADD:
        out.append("s_nop 2")          # a v_dot2c result read by VALU needs 3 wait states
    return out


def max_list(par):
    """The lane's max of the (rounded) scores of a set into TMAX: four
    independent chains over eight scores each (into the softmax temporaries),
    then one combining step."""
    cur = SET[par]
    chains = []
    for c in range(4):
        r = [v(cur + 8 * c + i) for i in range(8)]
        t = v(TMP + c)
        chains.append([f"v_max3_f32 {t}, {r[0]}, {r[1]}, {r[2]}",
                       f"v_max3_f32 {t}, {t}, {r[3]}, {r[4]}",
                       f"v_max3_f32 {t}, {t}, {r[5]}, {r[6]}",
                       f"v_max_f32_e32 {t}, {t}, {r[7]}"])
    out = [ins for stage in zip(*chains) for ins in stage]
    out += [f"v_max3_f32 {v(TMAX)}, {v(TMP)}, {v(TMP + 1)}, {v(TMP + 2)}",
            f"v_max_f32_e32 {v(TMAX)}, {v(TMAX)}, {v(TMP + 3)}"]
    return out


def check_dot2_distance(lines):
    """A v_dot2c result is read by another VALU instruction (other than the
    next v_dot2c of its chain) no earlier than four instructions later (three
    wait states: v_dot2 runs in the matrix pipe on gfx950)."""
    last = {}
    for i, ins in enumerate(lines):
        op, *regs = ins.replace(",", " ").split()
        if op.startswith("s_nop"):
            for r in last:
                last[r] -= int(regs[0])     # s_nop n adds n wait states beyond its own
        if op.startswith("v_") and op != "v_dot2c_f32_bf16_e32":
            for r in regs[1:]:
                if r in last:
                    assert i - last[r] >= 4, f"v_dot2c result {r} read too early: {ins}"
        if op == "v_dot2c_f32_bf16_e32":
            last[regs[0]] = i
        elif op.startswith("v_") and regs and regs[0] in last:
            del last[regs[0]]


def check_exp_distance(lines):
    """A v_exp_f32 result is read no earlier than two instructions later."""
    last_exp = {}
    for i, ins in enumerate(lines):
        op, *regs = ins.replace(",", " ").split()
        if op.startswith("v_"):
            for r in regs[1:]:
                if r in last_exp:
                    assert i - last_exp[r] >= 2, f"exp result {r} read too early: {ins}"
        if op == "v_exp_f32_e32":
            last_exp[regs[0]] = i
        elif op.startswith("v_") and regs and regs[0] in last_exp:
            del last_exp[regs[0]]


def mfma_run(ms, pset, vals):
    """MFMAs `ms` (P V of the parity `pset` tile, or QK^T into the parity
    `pset` set) with the VALU list `vals` spread between them."""
    lines = ["s_nop 1", "s_waitcnt lgkmcnt(0)"]
    if not ms:
        return lines + vals
    nreads = [len(reads_for(m, pset, 0)) for m in ms]
    issued = 0
    for j in range(min(LOOKAHEAD, len(ms))):
        lines += reads_for(ms[j], pset, j % N_RING)
        issued += 1
    pre = min(PRE_VALU, len(vals))     # VALU before the first MFMA (covers the first reads)
    lines += vals[:pre]
    vi = pre
    per = -(-(len(vals) - pre) // len(ms))
    seen_chain = set()
    for i, m in enumerate(ms):
        lines.append(f"s_waitcnt lgkmcnt({sum(nreads[i + 1:issued])})")
        first = m[0] == "qk" and (m[2] not in seen_chain)
        if m[0] == "qk":
            seen_chain.add(m[2])
        lines.append(mfma_text(m, pset, i % N_RING, first))
        if issued < len(ms):
            lines += reads_for(ms[issued], pset, issued % N_RING)
            issued += 1
        lines += vals[vi:vi + per]
        vi += per
    lines += vals[vi:]
    lines.append("s_nop 11")           # MFMA results read after the run
    check_exp_distance(lines)
    check_dot2_distance(lines)
    return lines


def mask_lines(par):
    """Raw score of key e (lane-constant offset of score register (nb, r)) to
    MASK_RAW when e > thr."""
    lines = [f"v_mov_b32_e32 {v(TVAL)}, {MASK_RAW}"]   # a literal and VCC would break the constant bus limit
    for nb in range(2):
        for r in range(16):
            e = nb * 32 + 8 * (r >> 2) + (r & 3)
            reg = v(SET[par] + 16 * nb + r)
            lines += [f"v_cmp_le_i32_e32 vcc, {e}, {OP_THR}", "s_nop 1",
                      f"v_cndmask_b32_e32 {reg}, {v(TVAL)}, {reg}, vcc"]
    return lines


def rescale_lines():
    """Every row's reference max to its running max: m_new = max(m, row max of
    s * fac) (-inf while the row has seen no key), alpha = exp2(m - m_new)
    (1 when m_new is -inf), l and O scaled by alpha."""
    lines = [f"ds_bpermute_b32 {v(TVAL)}, {OP_XADDR}, {v(TMAX)}",   # the other lane half's max
             "s_waitcnt lgkmcnt(0)",
             f"v_max_f32_e32 {v(TMAX)}, {v(TMAX)}, {v(TVAL)}",
             f"v_mul_f32_e32 {v(TVAL)}, {OP_FAC}, {v(TMAX)}",
             f"v_cmp_lt_f32_e32 vcc, {NO_KEY}, {v(TVAL)}",
             f"v_mov_b32_e32 {v(NEGM)}, {NEG_INF}",
             "s_nop 1",
             f"v_cndmask_b32_e32 {v(TVAL)}, {v(NEGM)}, {v(TVAL)}, vcc",
             f"v_max_f32_e32 {v(TVAL)}, {OP_M}, {v(TVAL)}",            # m_new
             f"v_sub_f32_e32 {v(NEGM)}, {OP_M}, {v(TVAL)}",
             f"v_exp_f32_e32 {v(NEGM)}, {v(NEGM)}",
             f"v_cmp_class_f32_e64 vcc, {v(TVAL)}, 4",
             "s_nop 1",
             f"v_cndmask_b32_e64 {v(NEGM)}, {v(NEGM)}, 1.0, vcc",      # alpha
             f"v_mul_f32_e32 {OP_L}, {OP_L}, {v(NEGM)}",
             f"v_mov_b32_e32 {OP_M}, {v(TVAL)}"]
    lines += [f"v_mul_f32_e32 {v(i)}, {v(NEGM)}, {v(i)}" for i in range(64)]
    lines += [f"v_cmp_class_f32_e64 vcc, {OP_M}, 4",
              "s_nop 1",
              f"v_cndmask_b32_e64 {v(NEGM)}, -{OP_M}, 0, vcc"]          # -m, or 0 for a row with no key
    return lines


def step_lines(par, R):
    """The whole step for the tile of parity `par` (see the docstring): PRE
    runs the pending P V MFMAs beside candle's score roundings (in place);
    POST runs the QK^T MFMAs of the next tile beside p = exp2(s * fac - m),
    the P pairs and their sum.  m moves (every row of the wave to its max of
    s * fac, O and l rescaled, the p taken again) when a row has no reference
    yet, or when a lane's sum of p passes 256 or is not finite."""
    L = lambda name: f".Lpf_{name}_%="
    pv = mfma_order(True, False)
    qk = mfma_order(False, True)
    out = [f"s_bitcmp1_b32 {OP_FLAGS}, {FLAG_LIVE}",
           f"s_cbranch_scc1 {L('live')}",
           # no keys in this tile: only the pending P V
           f"s_bitcmp1_b32 {OP_FLAGS}, {FLAG_PENDING}",
           f"s_cbranch_scc0 {L('end')}"]
    out += mfma_run(pv, par ^ 1, [])
    out += [f"s_branch {L('end')}",
            f"{L('live')}:",
            f"s_bitcmp1_b32 {OP_FLAGS}, {FLAG_FULL}",
            f"s_cbranch_scc1 {L('pre')}"]
    out += mask_lines(par)
    out += [f"{L('pre')}:",
            f"s_bitcmp1_b32 {OP_FLAGS}, {FLAG_PENDING}",
            f"s_cbranch_scc0 {L('prenopv')}"]
    out += mfma_run(pv, par ^ 1, round_list(par, R))
    out += [f"s_branch {L('decide')}",
            f"{L('prenopv')}:"]
    out += round_list(par, R)
    out += [f"{L('decide')}:",
            f"v_cmp_class_f32_e64 vcc, {OP_M}, 4",                 # a row with no reference max yet
            "s_cmp_lg_u64 vcc, 0",
            f"s_cbranch_scc1 {L('first')}",
            f"v_xor_b32_e32 {v(NEGM)}, 0x80000000, {OP_M}"]
    out += mfma_run(qk, par ^ 1, exp_list(par))
    out += [f"v_cmp_nge_f32_e32 vcc, {PSUM_MAX}, {v(PSUM)}",     # not (psum <= 256): redo
            "s_cmp_lg_u64 vcc, 0",
            f"s_cbranch_scc0 {L('acc')}"]
    out += max_list(par)
    out += rescale_lines()
    out += exp_list(par)
    out += [f"s_branch {L('acc')}",
            f"{L('first')}:"]
    out += max_list(par)
    out += rescale_lines()
    out += mfma_run(qk, par ^ 1, exp_list(par))
    out += [f"{L('acc')}:",
            f"v_add_f32_e32 {OP_L}, {OP_L}, {v(PSUM)}",
            f"{L('end')}:"]
    check_exp_distance(out)
    check_dot2_distance(out)
    return out


def main():
    import argparse
    global LOOKAHEAD, SUM_ADD, UNITS, PRE_VALU, N_RING
    ap = argparse.ArgumentParser()
    ap.add_argument("--out", default=None, help="output file (default: prefill_step.inc beside this script)")
    ap.add_argument("--lookahead", type=int, default=LOOKAHEAD, help="fragment reads in flight, in MFMAs")
    ap.add_argument("--sum-add", action="store_true", help="row sum of the f32 p by v_add_f32 instead of v_dot2c")
    ap.add_argument("--units", type=int, default=UNITS, help="score pairs interleaved stage by stage in the exp2 list")
    ap.add_argument("--pre-valu", type=int, default=PRE_VALU, help="VALU instructions before a run's first MFMA")
    ap.add_argument("--ring", type=int, default=N_RING, help="fragment buffers (at most 6)")
    args = ap.parse_args()
    LOOKAHEAD, SUM_ADD, UNITS, PRE_VALU, N_RING = args.lookahead, args.sum_add, args.units, args.pre_valu, args.ring
    assert 1 <= N_RING <= 6 and LOOKAHEAD <= N_RING - 1
    here = os.path.dirname(os.path.abspath(__file__))
    out = ["// Generated by gen_prefill_step.py: one step of the bf16 prefill's key loop",
           "// as gfx950 assembly over a fixed register map (see the generator's",
           "// docstring).  P: parity of the tile whose softmax runs; R: candle's score",
           "// roundings reproduced.  Do not edit.", ""]
    n = 0
    for par in (0, 1):
        for R in (1, 2):
            lines = step_lines(par, R)
            n += len(lines)
            out.append(f"#define CRANE_PF_STEP_P{par}_R{R} \\")
            out += [f'    "{ins}\\n" \\' for ins in lines]
            out.append('    ""')
            out.append("")
    with open(args.out or os.path.join(here, "prefill_step.inc"), "w") as f:
        f.write("\n".join(out))
    print(f"wrote prefill_step.inc ({n} lines)")


if __name__ == "__main__":
    main()
