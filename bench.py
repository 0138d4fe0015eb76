#!/usr/bin/env python3
"""Benchmark of the MI355X attention hot path on BASELINE.json's configurations.

Headline (`value`): config 3, Qwen3-8B-shape batched decode attention (B=32,
32 q / 8 kv heads, D=128, bf16 cache, per-sequence lengths L_i ~ U{512..4096}
seeded, one new token per sequence, so each sequence attends L_i+1 rows),
reported as algorithmic KV-read GB/s: sum_b (L_b+1) * Hkv * D * 2 (K and V) *
2 bytes (+ q and out) per step, over the measured step time.  One step = one
decode-attention launch over the whole batch, inputs resident in HBM.  Three
copies of the cache are rotated so the 256 MB Infinity Cache cannot serve a
step from the previous step's reads.

Also reported in the same line: config 4 (Qwen2.5-7B-shape causal prefill,
B=8, S=4096, 28/4 heads) in TFLOP/s, algorithmic flops 4*D*Hq*B*S(S+1)/2; the
fused QK-norm/RoPE/KV-append kernel at config 2 and config 3; and the CPU
baseline (the C restatement of Crane's candle-CPU op chain, tests' oracle)
timed on the host on a bounded sample of the same workloads.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only decode|prefill|append]
       [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, TFLOP/s
F32_PEAK_TFLOPS = 157.3        # MI355X dense f32 MFMA, TFLOP/s
METRIC = "decode attn KV GB/s (% of HBM peak) + prefill attn TFLOP/s, Qwen3-8B shape"
SEED0 = 0xC3A7E000
D = 128


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def c3_lengths() -> np.ndarray:
    return np.random.Generator(np.random.PCG64(SEED0 + 3)).integers(512, 4096, size=32, endpoint=True).astype(np.int32)


def randn(shape, gen, dtype, device, std=1.0):
    import torch
    t = torch.randn(shape, generator=gen, dtype=torch.float32, device=device)
    if std != 1.0:
        t.mul_(std)
    return t.to(dtype)


WARM_SECONDS = 0.5  # minimum untimed run before a timed region: lets the GPU clocks settle


def timed(launch, steps: int, warmup: int, stream):
    """Run `launch(i)` warmup + steps times; returns ms per step over the timed
    steps, bracketed by synchronize and measured with events on `stream`.
    The untimed warmup runs at least `warmup` launches and at least
    WARM_SECONDS of wall time: a cold GPU runs its first ~0.2 s at lower clocks."""
    import torch
    i = 0
    t0 = time.perf_counter()
    while i < warmup or time.perf_counter() - t0 < WARM_SECONDS:
        launch(i)
        i += 1
        if i % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for j in range(steps):
        launch(i + j)
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "hbm_traffic_pmc.md")


def pmc_traffic():
    """HBM bytes per launch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE
    (scaled by a calibration kernel of known traffic) for each workload, from
    the TRAFFIC lines of the committed counter summary; {} if absent."""
    out = {}
    try:
        for line in open(TRAFFIC_FILE):
            f = line.split()
            if len(f) == 3 and f[0] == "TRAFFIC":
                out[f[1]] = int(f[2])
    except OSError:
        pass
    return out


def launch_percentiles(launch, n: int, stream, first: int = 0):
    """Per-launch times (events around each launch, on `stream`) over n
    launches after the timed region: [p10, p50, p90] in ms."""
    import torch
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for j, (a, b) in enumerate(evs):
        a.record(stream)
        launch(first + j)
        b.record(stream)
    torch.cuda.synchronize()
    t = np.array([a.elapsed_time(b) for a, b in evs])
    return [round(float(x), 5) for x in np.percentile(t, [10, 50, 90])]


def cpu_info():
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or len(os.sched_getaffinity(0))
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return threads, model


# ---------------------------------------------------------------- decode

def bench_decode(args, dev, stream, lib):
    import torch
    lens = c3_lengths()
    B, Hq, Hkv = 32, 32, 8
    kv_len = lens + 1                      # the new token is already appended
    cap = int(kv_len.max())
    R = 3
    gen = torch.Generator(device=dev).manual_seed(SEED0 + 3)
    ks = [randn((B, Hkv, cap, D), gen, torch.bfloat16, dev) for _ in range(R)]
    vs = [randn((B, Hkv, cap, D), gen, torch.bfloat16, dev) for _ in range(R)]
    q = randn((B, Hq, D), gen, torch.bfloat16, dev)
    out = torch.empty((B, 1, Hq * D), dtype=torch.bfloat16, device=dev)
    kv_len_d = torch.as_tensor(kv_len, device=dev)
    need = lib.crane_hip_attn_decode_workspace(B, Hq, Hkv, D, cap, 1)
    ws = torch.zeros(need, dtype=torch.uint8, device=dev)
    scale = 1.0 / math.sqrt(D)
    st = stream.cuda_stream
    qp, op, lp, wp = q.data_ptr(), out.data_ptr(), kv_len_d.data_ptr(), ws.data_ptr()
    kps = [k.data_ptr() for k in ks]
    vps = [v.data_ptr() for v in vs]
    fn = lib.crane_hip_attn_decode

    def launch(i):
        # Qwen3-8B (n_rep 4): Crane's GQA-grouped decode form
        rc = fn(qp, kps[i % R], vps[i % R], cap, lp, cap, B, Hq, Hkv, D, scale, 0, wp, need, op, 1, st)
        if rc:
            raise RuntimeError(f"crane_hip_attn_decode failed: {rc}")

    ms = timed(launch, args.steps, args.warmup, stream)
    pct = launch_percentiles(launch, 100, stream)
    kv_bytes = int(kv_len.sum()) * Hkv * D * 2 * 2
    algo_bytes = kv_bytes + 2 * B * Hq * D * 2
    gbs = algo_bytes / (ms * 1e-3) / 1e9
    log(f"[decode c3] {ms * 1e3:.2f} us/step, {gbs:.1f} GB/s algorithmic ({gbs / HBM_PEAK_GBS * 100:.1f}% of HBM)")
    data = dict(ms=ms, gbs=gbs, algo_bytes=algo_bytes, kv_bytes=kv_bytes, lens=lens, kv_len=kv_len,
                B=B, Hq=Hq, Hkv=Hkv, cap=cap, pct=pct)
    data["_tensors"] = (q, ks[0], vs[0], kv_len)
    return data


def bench_decode_c5(args, dev, stream, lib):
    """Config 5 (Qwen2.5-72B shape, one layer, B=8, 64/8 heads, 32768-token cache,
    K/V ~ N(0, 0.5)): reported beside the headline."""
    import torch
    B, Hq, Hkv, L = 8, 64, 8, 32768
    kv_len = np.full(B, L + 1, np.int32)
    cap = L + 1
    gen = torch.Generator(device=dev).manual_seed(SEED0 + 5)
    R = 2                                   # 2 x 1.07 GB: far beyond the 256 MB MALL
    ks = [randn((B, Hkv, cap, D), gen, torch.bfloat16, dev, math.sqrt(0.5)) for _ in range(R)]
    vs = [randn((B, Hkv, cap, D), gen, torch.bfloat16, dev, math.sqrt(0.5)) for _ in range(R)]
    q = randn((B, Hq, D), gen, torch.bfloat16, dev)
    out = torch.empty((B, 1, Hq * D), dtype=torch.bfloat16, device=dev)
    kv_len_d = torch.as_tensor(kv_len, device=dev)
    need = lib.crane_hip_attn_decode_workspace(B, Hq, Hkv, D, cap, 1)
    ws = torch.zeros(need, dtype=torch.uint8, device=dev)
    st = stream.cuda_stream
    fn = lib.crane_hip_attn_decode

    def launch(i):
        # Qwen2.5-72B (candle-transformers qwen2): the standard SDPA form
        rc = fn(q.data_ptr(), ks[i % R].data_ptr(), vs[i % R].data_ptr(), cap, kv_len_d.data_ptr(), cap, B, Hq, Hkv,
                D, 1.0 / math.sqrt(D), 1, ws.data_ptr(), need, out.data_ptr(), 1, st)
        if rc:
            raise RuntimeError(f"crane_hip_attn_decode failed: {rc}")

    ms = timed(launch, max(3, args.steps // 2), args.warmup, stream)
    algo = int(kv_len.sum()) * Hkv * D * 2 * 2 + 2 * B * Hq * D * 2
    gbs = algo / (ms * 1e-3) / 1e9
    log(f"[decode c5] {ms * 1e3:.2f} us/step, {gbs:.1f} GB/s ({gbs / HBM_PEAK_GBS * 100:.1f}% of HBM)")
    del ks, vs
    torch.cuda.empty_cache()
    return dict(ms=ms, gbs=gbs, algo_bytes=algo)


def bench_decode_paged(args, dev, stream, lib):
    """Config 3 over the paged layout: the same lengths, K/V in pools of
    256-row pages whose ids are shuffled over the pool, read in place through
    the block table (crane_hip_attn_decode_paged)."""
    import torch
    lens = c3_lengths()
    B, Hq, Hkv, P = 32, 32, 8, 256
    kv_len = lens + 1
    need = [(int(n) + P - 1) // P for n in kv_len]
    stride, n_pages = max(need), sum(need)
    R = 3
    gen = torch.Generator(device=dev).manual_seed(SEED0 + 3)
    pools = [(randn((n_pages, Hkv, P, D), gen, torch.bfloat16, dev), randn((n_pages, Hkv, P, D), gen, torch.bfloat16,
                                                                          dev)) for _ in range(R)]
    perm = np.random.Generator(np.random.PCG64(SEED0 + 3)).permutation(n_pages).astype(np.int32)
    table = np.full((B, stride), -1, np.int32)
    nxt = 0
    for b in range(B):
        table[b, :need[b]] = perm[nxt:nxt + need[b]]
        nxt += need[b]
    table_d = torch.as_tensor(table, device=dev)
    q = randn((B, Hq, D), gen, torch.bfloat16, dev)
    out = torch.empty((B, 1, Hq * D), dtype=torch.bfloat16, device=dev)
    kv_len_d = torch.as_tensor(kv_len, device=dev)
    mx = int(kv_len.max())
    ws_need = lib.crane_hip_attn_decode_workspace(B, Hq, Hkv, D, mx, 1)
    ws = torch.zeros(ws_need, dtype=torch.uint8, device=dev)
    st = stream.cuda_stream
    fn = lib.crane_hip_attn_decode_paged

    def launch(i):
        kp, vp = pools[i % R]
        rc = fn(q.data_ptr(), kp.data_ptr(), vp.data_ptr(), n_pages, P, table_d.data_ptr(), stride,
                kv_len_d.data_ptr(), mx, B, Hq, Hkv, D, 1.0 / math.sqrt(D), 0, ws.data_ptr(), ws_need, out.data_ptr(),
                1, st)
        if rc:
            raise RuntimeError(f"crane_hip_attn_decode_paged failed: {rc}")

    ms = timed(launch, args.steps, args.warmup, stream)
    algo = int(kv_len.sum()) * Hkv * D * 2 * 2 + 2 * B * Hq * D * 2
    gbs = algo / (ms * 1e-3) / 1e9
    log(f"[decode c3 paged] {ms * 1e3:.2f} us/step, {gbs:.1f} GB/s ({gbs / HBM_PEAK_GBS * 100:.1f}% of HBM), "
        f"{n_pages} pages of {P} rows")
    del pools
    torch.cuda.empty_cache()
    return dict(ms=ms, gbs=gbs, page_rows=P, n_pages=n_pages)


def bench_layer(args, dev, stream, lib):
    """The decoder-layer row kernels (include/crane_layer.h) at config 4's
    prefill rows (Qwen2.5-7B: 8 x 4096 rows, hidden 3584, intermediate 18944)
    and config 3's decode rows (Qwen3-8B: 32 rows, hidden 4096, intermediate
    12288).  Algorithmic bytes: every tensor read or written once (the norm
    weight counted once).  At config 4 the hidden-size tensors (235 MB each)
    rotate through 3 copies, so a call's reads cannot come from the 256 MB
    Infinity Cache left warm by the call before; silu_mul moves 3.7 GB a call."""
    import torch
    res = {}
    st = stream.cuda_stream
    for tag, rows, hidden, inter in (("c4_prefill_rows", 8 * 4096, 3584, 18944), ("c3_decode_rows", 32, 4096, 12288)):
        gen = torch.Generator(device=dev).manual_seed(SEED0 + 7)
        R = 3 if rows >= 4096 else 1
        xs = [randn((rows, hidden), gen, torch.bfloat16, dev) for _ in range(R)]
        hs = [randn((rows, hidden), gen, torch.bfloat16, dev) for _ in range(R)]
        w = randn((hidden,), gen, torch.bfloat16, dev)
        outs = [torch.empty_like(xs[0]) for _ in range(R)]
        gu = randn((rows, 2 * inter), gen, torch.bfloat16, dev)
        act = torch.empty((rows, inter), dtype=torch.bfloat16, device=dev)
        row_bytes = hidden * 2
        ops_ = {
            "rms_norm": (lambda i: lib.crane_hip_rms_norm(xs[i % R].data_ptr(), w.data_ptr(), outs[i % R].data_ptr(),
                                                           rows, hidden, 1e-6, 1, st), 2 * rows * row_bytes + row_bytes),
            "add_rms_norm": (lambda i: lib.crane_hip_add_rms_norm(xs[i % R].data_ptr(), hs[i % R].data_ptr(),
                                                                   w.data_ptr(), outs[i % R].data_ptr(), rows, hidden,
                                                                   1e-6, 1, st),
                             4 * rows * row_bytes + row_bytes),
            "silu_mul": (lambda i: lib.crane_hip_silu_mul(gu.data_ptr(), act.data_ptr(), rows, inter, 1, st),
                         3 * rows * inter * 2),
            "residual_add": (lambda i: lib.crane_hip_residual_add(xs[i % R].data_ptr(), hs[i % R].data_ptr(),
                                                                   rows * hidden, 1, st),
                             3 * rows * row_bytes),
        }
        res[tag] = {}
        for name, (fn, nbytes) in ops_.items():
            def launch(i, fn=fn, name=name):
                rc = fn(i)
                if rc:
                    raise RuntimeError(f"{name} failed: {rc}")
            ms = timed(launch, args.steps, args.warmup, stream)
            gbs = nbytes / (ms * 1e-3) / 1e9
            res[tag][name] = dict(us=ms * 1e3, gbs=gbs, frac=gbs / HBM_PEAK_GBS, bytes=nbytes)
            log(f"[layer {tag}] {name}: {ms * 1e3:.1f} us, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS * 100:.1f}% of HBM)")
        del xs, hs, outs, gu, act
        torch.cuda.empty_cache()
    return res


def bench_gemm(args, dev, stream, lib):
    """The projections (include/crane_gemm.h): Qwen2.5-7B qkv_proj (with bias)
    and o_proj at config 4's 8 x 4096 rows (hipBLASLt), and at config 3's 32
    decode rows the Qwen3-8B qkv_proj, o_proj, gate_up (alone, and with the
    SiLU*mul in the same launch) and lm_head (the per-wave ring kernel) and
    down_proj (hipBLASLt).  The decode shapes rotate
    over enough weight copies (> 600 MB) that every launch streams its weight
    from HBM, not from the 256 MB Infinity Cache."""
    import ctypes
    import torch
    h = ctypes.c_void_p()
    if lib.crane_gemm_create(0, ctypes.byref(h)):
        raise RuntimeError("crane_gemm_create failed")
    st = stream.cuda_stream
    res = {}
    for tag, M, N, K, bias in (("c4_qkv_proj", 8 * 4096, 4608, 3584, True), ("c4_o_proj", 8 * 4096, 3584, 3584, False),
                               ("c3_qkv_proj", 32, 6144, 4096, False), ("c3_o_proj", 32, 4096, 4096, False),
                               ("c3_gate_up", 32, 24576, 4096, False), ("c3_gate_up_silu_mul", 32, 24576, 4096, False),
                               ("c3_down_proj", 32, 4096, 12288, False), ("c3_lm_head", 32, 151936, 4096, False)):
        gen = torch.Generator(device=dev).manual_seed(SEED0 + 9)
        x = randn((M, K), gen, torch.bfloat16, dev)
        copies = max(1, -(-600_000_000 // (N * K * 2))) if M <= 64 else 1
        ws_ = [randn((N, K), gen, torch.bfloat16, dev, 1.0 / math.sqrt(K)) for _ in range(copies)]
        b = randn((N,), gen, torch.bfloat16, dev) if bias else None
        gated = tag.endswith("silu_mul")  # one launch: gate_up, then silu(gate) * up [M, N / 2]
        y = torch.empty((M, N // 2 if gated else N), dtype=torch.bfloat16, device=dev)

        def launch(i):
            if gated:
                rc = lib.crane_gemm_linear_silu_mul(h, x.data_ptr(), ws_[i % copies].data_ptr(), y.data_ptr(), M,
                                                    N // 2, K, 1, st)
            else:
                rc = lib.crane_gemm_linear(h, x.data_ptr(), ws_[i % copies].data_ptr(),
                                           b.data_ptr() if b is not None else None, y.data_ptr(), M, N, K, 1, st)
            if rc:
                raise RuntimeError(f"crane_gemm_linear failed: {rc}")
        ms = timed(launch, args.steps, args.warmup, stream)
        flops = 2.0 * M * N * K
        tf = flops / (ms * 1e-3) / 1e12
        nbytes = (M * K + N * K + M * (N // 2 if gated else N)) * 2
        res[tag] = dict(us=ms * 1e3, tflops=tf, frac=tf / BF16_PEAK_TFLOPS, gbs=nbytes / (ms * 1e-3) / 1e9)
        log(f"[gemm {tag}] M={M} N={N} K={K}: {ms * 1e3:.1f} us, {tf:.1f} TFLOP/s ({tf / BF16_PEAK_TFLOPS * 100:.1f}% "
            f"of bf16 peak), {res[tag]['gbs']:.0f} GB/s ({res[tag]['gbs'] / HBM_PEAK_GBS * 100:.1f}% of HBM)")
        if M > 64 and not args.no_const_inputs:
            # the same product on constant inputs (every x and w element
            # 2^-6): the MFMA pipes toggle few bits and the chip holds higher
            # clocks, so the gap to the N(0, 1) figure is the data-dependent
            # power limit, not the kernel
            x.fill_(2.0 ** -6)
            for t in ws_:
                t.fill_(2.0 ** -6)
            msc = timed(launch, args.steps, args.warmup, stream)
            tfc = flops / (msc * 1e-3) / 1e12
            res[tag].update(us_const_inputs=msc * 1e3, frac_const_inputs=tfc / BF16_PEAK_TFLOPS)
            log(f"[gemm {tag}] same product on constant inputs: {msc * 1e3:.1f} us, {tfc:.1f} TFLOP/s "
                f"({tfc / BF16_PEAK_TFLOPS * 100:.1f}% of bf16 peak)")
        del x, ws_, b, y
    # the decode step's qkv_proj, o_proj and down_proj as the model driver runs
    # them: f32 partial products over 2 or 4 splits of K (summed by the append
    # or the add + norm that follows)
    for tag, M, N, K, sp in (("c3_qkv_proj_split2", 32, 6144, 4096, 2), ("c3_o_proj_split4", 32, 4096, 4096, 4),
                             ("c3_down_proj_split4", 32, 4096, 12288, 4)):
        gen = torch.Generator(device=dev).manual_seed(SEED0 + 9)
        x = randn((M, K), gen, torch.bfloat16, dev)
        copies = max(1, -(-600_000_000 // (N * K * 2)))
        ws_ = [randn((N, K), gen, torch.bfloat16, dev, 1.0 / math.sqrt(K)) for _ in range(copies)]
        part = torch.empty((sp, M, N), dtype=torch.float32, device=dev)

        def launch_split(i):
            rc = lib.crane_gemm_linear_split(h, x.data_ptr(), ws_[i % copies].data_ptr(), part.data_ptr(), M, N, K,
                                             sp, 1, st)
            if rc:
                raise RuntimeError(f"crane_gemm_linear_split failed: {rc}")
        ms = timed(launch_split, args.steps, args.warmup, stream)
        nbytes = (M * K + N * K) * 2 + sp * M * N * 4
        res[tag] = dict(us=ms * 1e3, gbs=nbytes / (ms * 1e-3) / 1e9)
        log(f"[gemm {tag}] M={M} N={N} K={K}, {sp} f32 partial products: {ms * 1e3:.1f} us, "
            f"{res[tag]['gbs']:.0f} GB/s ({res[tag]['gbs'] / HBM_PEAK_GBS * 100:.1f}% of HBM)")
        del x, ws_, part
    lib.crane_gemm_destroy(h)
    torch.cuda.empty_cache()
    return res


def bench_sampling(args, dev, stream, lib):
    """Token selection over Qwen vocabulary logits (151936): argmax on bf16
    (greedy) and top-64 on f32, one row and a c3 batch of 32 rows; the
    split-row (_ws) entry points, which the ops wrappers call, and the
    single-pass kernels (one workgroup per row) beside them."""
    import torch
    res = {}
    st = stream.cuda_stream
    n = 151936
    for rows in (1, 32):
        gen = torch.Generator(device=dev).manual_seed(SEED0 + 11)
        xb = randn((rows, n), gen, torch.bfloat16, dev, 4.0)
        xf = randn((rows, n), gen, torch.float32, dev, 4.0)
        out = torch.empty((rows, 64), dtype=torch.int32, device=dev)
        wsb = int(lib.crane_hip_select_workspace_bytes(rows, n))
        ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=dev)
        for name, fn in (("argmax_bf16", lambda i: lib.crane_hip_argmax_ws(xb.data_ptr(), rows, n, 1, ws.data_ptr(),
                                                                            wsb, out.data_ptr(), st)),
                         ("topk64_f32", lambda i: lib.crane_hip_topk_ws(xf.data_ptr(), rows, n, 64, ws.data_ptr(),
                                                                         wsb, out.data_ptr(), st)),
                         ("argmax_bf16_single_pass",
                          lambda i: lib.crane_hip_argmax(xb.data_ptr(), rows, n, 1, out.data_ptr(), st)),
                         ("topk64_f32_single_pass",
                          lambda i: lib.crane_hip_topk(xf.data_ptr(), rows, n, 64, out.data_ptr(), st))):
            def launch(i, fn=fn, name=name):
                rc = fn(i)
                if rc:
                    raise RuntimeError(f"{name} failed: {rc}")
            ms = timed(launch, args.steps, args.warmup, stream)
            res[f"{name}_rows{rows}"] = dict(us=ms * 1e3)
            log(f"[sampling] {name} {rows} x {n}: {ms * 1e3:.1f} us")
            if not name.endswith("single_pass"):
                # as a serving step runs it: captured with the step's other
                # kernels in a HIP graph, so back-to-back launches cost no
                # host round trip (graph of 10 selections, time per selection)
                cs = torch.cuda.Stream(device=dev)
                cs.wait_stream(stream)
                g = torch.cuda.CUDAGraph()
                st_c = cs.cuda_stream
                fn_c = {"argmax_bf16": lambda: lib.crane_hip_argmax_ws(xb.data_ptr(), rows, n, 1, ws.data_ptr(), wsb,
                                                                       out.data_ptr(), st_c),
                        "topk64_f32": lambda: lib.crane_hip_topk_ws(xf.data_ptr(), rows, n, 64, ws.data_ptr(), wsb,
                                                                    out.data_ptr(), st_c)}[name]
                with torch.cuda.graph(g, stream=cs):
                    for _ in range(10):
                        if fn_c():
                            raise RuntimeError(f"{name} failed under capture")
                stream.wait_stream(cs)
                torch.cuda.synchronize(dev)
                msg = timed(lambda i: g.replay(), max(3, args.steps // 10), args.warmup, stream) / 10
                res[f"{name}_rows{rows}"]["us_graph"] = msg * 1e3
                log(f"[sampling] {name} {rows} x {n}, graph replay: {msg * 1e3:.1f} us")
    return res


def bench_read_ceiling(args, dev, stream):
    """The HBM read rate this GPU reaches with the decode kernel's access
    pattern: crane_amd's libcrane_probe.so (a measurement helper beside the
    library, not part of it) reads 3 rotated buffers of the config 3 decode's
    bytes per call (320 MB, past the 256 MB Infinity Cache), one workgroup per
    contiguous span with all of the span's loads in flight, at 8, 16 and 32
    loads per thread (32-128 KiB spans); the fastest is the ceiling the decode
    call is compared with.  None when the probe library is not built."""
    import ctypes
    import torch
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "crane_amd", "libcrane_probe.so")
    if not os.path.exists(path):
        log("[read ceiling] libcrane_probe.so not built: skipped")
        return None
    probe = ctypes.CDLL(path)
    probe.crane_probe_read.restype = ctypes.c_int
    probe.crane_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    probe.crane_probe_workgroups.restype = ctypes.c_int64
    probe.crane_probe_workgroups.argtypes = [ctypes.c_int64, ctypes.c_int]
    nbytes, R = 320 * 1000 * 1000, 3
    bufs = [torch.ones(nbytes // 4, dtype=torch.int32, device=dev) for _ in range(R)]
    sink = torch.empty(int(probe.crane_probe_workgroups(nbytes, 8)), dtype=torch.int32, device=dev)
    st = stream.cuda_stream
    best = None
    for loads in (8, 16, 32):
        def launch(i, loads=loads):
            rc = probe.crane_probe_read(bufs[i % R].data_ptr(), nbytes, sink.data_ptr(), loads, st)
            if rc:
                raise RuntimeError(f"crane_probe_read failed: {rc}")
        ms = timed(launch, args.steps, args.warmup, stream)
        gbs = nbytes / (ms * 1e-3) / 1e9
        log(f"[read ceiling] {16 * 256 * loads // 1024} KiB per workgroup: {ms * 1e3:.2f} us per 320 MB, "
            f"{gbs:.1f} GB/s ({gbs / HBM_PEAK_GBS * 100:.1f}% of HBM)")
        if best is None or gbs > best["gbs"]:
            best = dict(gbs=gbs, ms=ms, span_kib=16 * 256 * loads // 1024)
    # One launch reading the bytes of one decode-step weight (Qwen3-8B shape,
    # bf16), back to back over rotated slices of the buffers (> 600 MB in all,
    # so every read comes from HBM): the rate a kernel of that size reaches
    # with nothing but reads, its launch, ramp and drain included.  The
    # fastest span of the three per size.
    best["single_reads"] = {}
    for name, n in (("o_proj", 4096 * 4096 * 2), ("qkv_proj", 6144 * 4096 * 2), ("down_proj", 12288 * 4096 * 2),
                    ("gate_up", 24576 * 4096 * 2)):
        n = n // 4096 * 4096
        slots = [(b, off) for b in range(R) for off in range(0, nbytes - n + 1, n)]
        top = None
        for loads in (8, 16, 32):
            def launch(i, loads=loads, n=n, slots=slots):
                b, off = slots[i % len(slots)]
                rc = probe.crane_probe_read(bufs[b].data_ptr() + off, n, sink.data_ptr(), loads, st)
                if rc:
                    raise RuntimeError(f"crane_probe_read failed: {rc}")
            ms = timed(launch, args.steps, args.warmup, stream)
            if top is None or ms < top[0]:
                top = (ms, loads)
        gbs = n / (top[0] * 1e-3) / 1e9
        best["single_reads"][name] = dict(bytes=n, us=round(top[0] * 1e3, 2), gbs=round(gbs, 1),
                                          span_kib=16 * 256 * top[1] // 1024)
        log(f"[read ceiling] one read of {name}'s {n / 1e6:.1f} MB: {top[0] * 1e3:.2f} us, {gbs:.1f} GB/s "
            f"({gbs / HBM_PEAK_GBS * 100:.1f}% of HBM)")
    del bufs
    torch.cuda.empty_cache()
    return best


# ---------------------------------------------------------------- prefill

def bench_prefill(args, dev, stream, lib):
    """Config 4 causal prefill, once per flags value of --prefill-modes (the
    first is the headline): 1 = both of candle's score roundings (the
    library's default), 3 = + CRANE_HIP_PREFILL_LONG_ROWS_ONE_ROUNDING."""
    import torch
    B, S, Hq, Hkv = 8, 4096, 28, 4
    gen = torch.Generator(device=dev).manual_seed(SEED0 + 4)
    q = randn((B, Hq, S, D), gen, torch.bfloat16, dev)
    k = randn((B, Hkv, S, D), gen, torch.bfloat16, dev)
    v = randn((B, Hkv, S, D), gen, torch.bfloat16, dev)
    out = torch.empty((B, S, Hq * D), dtype=torch.bfloat16, device=dev)
    start = torch.zeros(B, dtype=torch.int32, device=dev)
    st = stream.cuda_stream
    fn = lib.crane_hip_attn_prefill
    flops = 4.0 * D * Hq * B * S * (S + 1) / 2
    modes = [int(x) for x in args.prefill_modes.split(",")]
    res = {}
    for flags in modes:
        def launch(i, flags=flags):
            rc = fn(q.data_ptr(), k.data_ptr(), v.data_ptr(), S, start.data_ptr(), 0, B, S, Hq, Hkv, D,
                    1.0 / math.sqrt(D), flags, out.data_ptr(), 1, st)
            if rc:
                raise RuntimeError(f"crane_hip_attn_prefill failed: {rc}")

        ms = timed(launch, max(3, args.steps // 2), max(2, args.warmup // 2), stream)
        pct = launch_percentiles(launch, 100, stream)
        tflops = flops / (ms * 1e-3) / 1e12
        log(f"[prefill c4, flags {flags}] {ms:.3f} ms/step, {tflops:.1f} TFLOP/s "
            f"({tflops / BF16_PEAK_TFLOPS * 100:.1f}% of bf16 peak), median launch {pct[1]:.3f} ms")
        res[flags] = dict(ms=ms, tflops=tflops, pct=pct)
    head = res[modes[0]]
    if args.no_const_inputs:
        return dict(ms=head["ms"], tflops=head["tflops"], flops=flops, B=B, S=S, Hq=Hq, Hkv=Hkv, pct=head["pct"],
                    flags=modes[0], modes=res, ms_const=None, _tensors=(q, k, v))
    # the headline mode on constant inputs (every q, K, V element 2^-6): the
    # same instructions (no tile of the constant rows redoes its softmax
    # either way at this size) with few toggling bits; the gap to the N(0, 1)
    # figure is the data-dependent power limit
    qc, kc_, vc_ = (torch.full_like(t, 2.0 ** -6) for t in (q, k, v))
    flags0 = modes[0]

    def launch_const(i):
        rc = fn(qc.data_ptr(), kc_.data_ptr(), vc_.data_ptr(), S, start.data_ptr(), 0, B, S, Hq, Hkv, D,
                1.0 / math.sqrt(D), flags0, out.data_ptr(), 1, st)
        if rc:
            raise RuntimeError(f"crane_hip_attn_prefill failed: {rc}")

    msc = timed(launch_const, max(3, args.steps // 2), max(2, args.warmup // 2), stream)
    tfc = flops / (msc * 1e-3) / 1e12
    log(f"[prefill c4, flags {flags0}] the same call on constant inputs: {msc:.3f} ms/step, {tfc:.1f} TFLOP/s "
        f"({tfc / BF16_PEAK_TFLOPS * 100:.1f}% of bf16 peak)")
    del qc, kc_, vc_
    return dict(ms=head["ms"], tflops=head["tflops"], flops=flops, B=B, S=S, Hq=Hq, Hkv=Hkv, pct=head["pct"],
                flags=modes[0], modes=res, ms_const=msc, _tensors=(q, k, v))


def bench_prefill_c2(args, dev, stream, lib):
    """Config 2 (Qwen3-0.6B-shape prefill, B=1, S=2048, 16/8 heads): fused
    QK-norm + RoPE append into an empty cap-4096 cache, then causal prefill."""
    import torch
    B, S, Hq, Hkv, cap = 1, 2048, 16, 8, 4096
    gen = torch.Generator(device=dev).manual_seed(SEED0 + 2)
    qkv = randn((B, S, (Hq + 2 * Hkv) * D), gen, torch.bfloat16, dev)
    from crane_amd import ops
    cos, sin = ops.rope_tables(D, 1e6, 40960, device=dev, dtype=torch.bfloat16)
    kc = torch.zeros((B, Hkv, cap, D), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    q_out = torch.empty((B, Hq, S, D), dtype=torch.bfloat16, device=dev)
    out = torch.empty((B, S, Hq * D), dtype=torch.bfloat16, device=dev)
    zeros = torch.zeros(B, dtype=torch.int32, device=dev)
    st = stream.cuda_stream
    L = lib

    def launch(i):
        rc = L.crane_hip_qknorm_rope_append(qkv.data_ptr(), qkv.stride(1), None, None, 1e-6, 0, cos.data_ptr(),
                                           sin.data_ptr(), cos.stride(0), cos.shape[0], zeros.data_ptr(),
                                           q_out.data_ptr(), kc.data_ptr(), vc.data_ptr(), cap, zeros.data_ptr(),
                                           S, B, S, Hq, Hkv, D, 1, st)
        rc = rc or L.crane_hip_attn_prefill(q_out.data_ptr(), kc.data_ptr(), vc.data_ptr(), cap, zeros.data_ptr(), 0,
                                            B, S, Hq, Hkv, D, 1.0 / math.sqrt(D), 1, out.data_ptr(), 1, st)
        if rc:
            raise RuntimeError(f"c2 step failed: {rc}")

    ms = timed(launch, args.steps, args.warmup, stream)
    flops = 4.0 * D * Hq * B * S * (S + 1) / 2
    log(f"[prefill c2] append+prefill {ms * 1e3:.1f} us/step, {flops / (ms * 1e-3) / 1e12:.1f} TFLOP/s (launch-bound)")
    return dict(ms=ms, tflops=flops / (ms * 1e-3) / 1e12)


def bench_prefill_f32(args, dev, stream, lib):
    """Config 2's prefill shape (B=1, S=2048, 16 / 8 heads, causal) in f32:
    the f32 MFMA kernel (v_mfma_f32_32x32x2_f32), against the f32 MFMA peak."""
    import torch
    B, S, Hq, Hkv = 1, 2048, 16, 8
    gen = torch.Generator(device=dev).manual_seed(SEED0 + 21)
    q = randn((B, Hq, S, D), gen, torch.float32, dev)
    k = randn((B, Hkv, S, D), gen, torch.float32, dev)
    v = randn((B, Hkv, S, D), gen, torch.float32, dev)
    out = torch.empty((B, S, Hq * D), dtype=torch.float32, device=dev)
    start = torch.zeros(B, dtype=torch.int32, device=dev)
    st = stream.cuda_stream

    def launch(i):
        rc = lib.crane_hip_attn_prefill(q.data_ptr(), k.data_ptr(), v.data_ptr(), S, start.data_ptr(), 0, B, S, Hq,
                                        Hkv, D, 1.0 / math.sqrt(D), 1, out.data_ptr(), 0, st)
        if rc:
            raise RuntimeError(f"crane_hip_attn_prefill (f32) failed: {rc}")

    ms = timed(launch, args.steps, args.warmup, stream)
    flops = 4.0 * D * Hq * B * S * (S + 1) / 2
    tf = flops / (ms * 1e-3) / 1e12
    log(f"[prefill c2 f32] {ms * 1e3:.1f} us/step, {tf:.1f} TFLOP/s ({tf / F32_PEAK_TFLOPS * 100:.1f}% of the f32 "
        f"MFMA peak)")
    return dict(ms=ms, tflops=tf)


def bench_append(args, dev, stream, lib):
    """Fused QK-norm + RoPE + KV append at config 4's prefill size (8 x 4096
    tokens, 28/4 heads, rope only) and config 3's decode step (32 tokens).  At
    config 4 the inputs and outputs (670 MB a call) rotate through 2 copies, so
    a call cannot read what the one before left in the 256 MB Infinity Cache."""
    import torch
    from crane_amd import ops
    res = {}
    cos, sin = ops.rope_tables(D, 1e6, 40960, device=dev, dtype=torch.bfloat16)
    st = stream.cuda_stream
    for name, (B, S, Hq, Hkv, order, start) in {
            "c4_prefill_append": (8, 4096, 28, 4, 2, 0),
            "c3_decode_append": (32, 1, 32, 8, 0, 4096)}.items():
        gen = torch.Generator(device=dev).manual_seed(SEED0 + 40)
        R = 2 if S > 1 else 1
        qkvs = [randn((B, S, (Hq + 2 * Hkv) * D), gen, torch.bfloat16, dev) for _ in range(R)]
        cap = start + S
        kcs = [torch.zeros((B, Hkv, cap, D), dtype=torch.bfloat16, device=dev) for _ in range(R)]
        vcs = [torch.zeros_like(kcs[0]) for _ in range(R)]
        q_outs = [torch.empty((B, Hq, S, D), dtype=torch.bfloat16, device=dev) for _ in range(R)]
        pos = torch.full((B,), start, dtype=torch.int32, device=dev)
        w = torch.ones(D, dtype=torch.bfloat16, device=dev)

        def launch(i):
            qkv, q_out, kc, vc = qkvs[i % R], q_outs[i % R], kcs[i % R], vcs[i % R]
            rc = lib.crane_hip_qknorm_rope_append(
                qkv.data_ptr(), qkv.stride(1), w.data_ptr(), w.data_ptr(), 1e-6, order, cos.data_ptr(),
                sin.data_ptr(), cos.stride(0), cos.shape[0], pos.data_ptr(), q_out.data_ptr(), kc.data_ptr(),
                vc.data_ptr(), cap, pos.data_ptr(), cap, B, S, Hq, Hkv, D, 1, st)
            if rc:
                raise RuntimeError(f"append failed: {rc}")

        ms = timed(launch, args.steps, args.warmup, stream)
        nbytes = B * S * (Hq + 2 * Hkv) * D * 2 * 2   # read qkv once, write q and the cache rows once
        res[name] = dict(us=ms * 1e3, gbs=nbytes / (ms * 1e-3) / 1e9, bytes=nbytes)
        log(f"[append {name}] {ms * 1e3:.1f} us, {nbytes / (ms * 1e-3) / 1e9:.0f} GB/s")
    return res


# ------------------------------------------------------- whole decode step

def bench_model_step(args, dev, stream, lib):
    """One decode step of a whole Qwen3-8B-shape model at config 3's batch: 36
    layers (hidden 4096, 32 q / 8 kv heads, intermediate 12288, QK-norm), the
    final norm and the lm_head (vocab 151936), B=32 sequences at the config 3
    lengths (each attends its L_i+1 rows in every layer).  The step is the
    model driver's decode step (crane_amd/model.py) captured once in a HIP
    graph and replayed; the lengths are put back before every replay so each
    step is the same workload.  Random weights of the model's shapes; the
    roofline is HBM: every weight and every layer's K/V rows are read once a
    step."""
    import torch
    from crane_amd import decoder, model
    L, H, Hq, Hkv, I, V = 36, 4096, 32, 8, 12288, 151936
    lens = c3_lengths()
    B = len(lens)
    cap = int(lens.max()) + 8
    gen = torch.Generator(device=dev).manual_seed(SEED0 + 36)
    bf = torch.bfloat16

    def w(*shape, std):
        return randn(shape, gen, bf, dev, std)

    layers = [decoder.LayerWeights(input_norm=torch.ones(H, dtype=bf, device=dev),
                                   qkv=w((Hq + 2 * Hkv) * D, H, std=H ** -0.5), o=w(H, Hq * D, std=(Hq * D) ** -0.5),
                                   post_norm=torch.ones(H, dtype=bf, device=dev), gate_up=w(2 * I, H, std=H ** -0.5),
                                   down=w(H, I, std=I ** -0.5), q_norm=torch.ones(D, dtype=bf, device=dev),
                                   k_norm=torch.ones(D, dtype=bf, device=dev)) for _ in range(L)]
    cfg = model.ModelConfig(hidden=H, num_heads=Hq, num_kv_heads=Hkv, intermediate=I, num_layers=L, family="qwen3")
    m = model.DecoderModel(cfg, layers, torch.ones(H, dtype=bf, device=dev), w(V, H, std=H ** -0.5), B, cap)
    for i in range(L):
        m.k[i].copy_(randn(m.k[i].shape, gen, bf, dev))
        m.v[i].copy_(randn(m.v[i].shape, gen, bf, dev))
    base = torch.as_tensor(lens, device=dev)
    m.lengths.copy_(base)
    m.host_lengths[:] = lens
    g = model.DecodeGraph(m)
    g.x.copy_(randn((B, 1, H), gen, bf, dev))
    g.positions.copy_(base)

    def launch(i):
        m.lengths.copy_(base)
        m.host_lengths[:] = lens
        g.replay()

    steps = max(3, args.steps // 2)
    ms = timed(launch, steps, args.warmup, stream)
    weight_bytes = sum(t.numel() * 2 for lw in layers for t in (lw.input_norm, lw.qkv, lw.o, lw.post_norm,
                                                                 lw.gate_up, lw.down, lw.q_norm, lw.k_norm))
    weight_bytes += (V * H + H) * 2
    kv_bytes = L * int((lens + 1).sum()) * Hkv * D * 2 * 2
    gbs = (weight_bytes + kv_bytes) / (ms * 1e-3) / 1e9
    log(f"[model step] Qwen3-8B shape, {L} layers, B={B}: {ms:.3f} ms/step, {B / (ms * 1e-3):.0f} tokens/s, "
        f"{gbs:.0f} GB/s of weights + K/V ({gbs / HBM_PEAK_GBS * 100:.1f}% of HBM)")
    res = dict(ms=ms, tokens_per_s=B / (ms * 1e-3), gbs=gbs, weight_bytes=weight_bytes, kv_bytes=kv_bytes, layers=L)
    del g, m, layers
    torch.cuda.empty_cache()
    return res


def bench_model_prefill(args, dev, stream, lib):
    """One prefill step of a whole Qwen2.5-7B-shape model at config 4's size:
    28 layers (hidden 3584, 28 q / 4 kv heads with the QKV bias, intermediate
    18944, rope only), B=8 sequences of 4096 new tokens into empty caches,
    then the final norm and the lm_head (vocab 152064) on the last position.
    The step is the model driver's forward (crane_amd/model.py) with the
    caches reset before every step.  Random weights of the model's shapes; the
    roofline is MFMA: the flops of every projection (2 M N K) and of the causal
    attention (4 D Hq per query-key pair) per step."""
    import torch
    from crane_amd import decoder, model
    L, H, Hq, Hkv, I, V = 28, 3584, 28, 4, 18944, 152064
    B, S = 8, 4096
    gen = torch.Generator(device=dev).manual_seed(SEED0 + 28)
    bf = torch.bfloat16

    def w(*shape, std):
        return randn(shape, gen, bf, dev, std)

    nqkv = (Hq + 2 * Hkv) * D
    layers = [decoder.LayerWeights(input_norm=torch.ones(H, dtype=bf, device=dev), qkv=w(nqkv, H, std=H ** -0.5),
                                   o=w(H, Hq * D, std=(Hq * D) ** -0.5),
                                   post_norm=torch.ones(H, dtype=bf, device=dev), gate_up=w(2 * I, H, std=H ** -0.5),
                                   down=w(H, I, std=I ** -0.5), qkv_bias=w(nqkv, std=0.1)) for _ in range(L)]
    cfg = model.ModelConfig(hidden=H, num_heads=Hq, num_kv_heads=Hkv, intermediate=I, num_layers=L, family="qwen2",
                            max_position=32768)
    m = model.DecoderModel(cfg, layers, torch.ones(H, dtype=bf, device=dev), w(V, H, std=H ** -0.5), B, S)
    x = randn((B, S, H), gen, bf, dev)
    positions = torch.zeros(B, dtype=torch.int32, device=dev)

    def launch(i):
        m.reset()
        m.forward(x, positions)

    ms = timed(launch, 3, 1, stream)
    M = B * S
    proj = 2.0 * M * H * (nqkv + Hq * D + 2 * I + I) * L  # qkv, o, gate_up, down
    attn = 4.0 * D * Hq * B * S * (S + 1) / 2 * L
    head = 2.0 * B * H * V
    flops = proj + attn + head
    tflops = flops / (ms * 1e-3) / 1e12
    log(f"[model prefill] Qwen2.5-7B shape, {L} layers, B={B} x S={S}: {ms:.1f} ms/step, "
        f"{M / (ms * 1e-3):.0f} tokens/s, {tflops:.1f} TFLOP/s ({tflops / BF16_PEAK_TFLOPS * 100:.1f}% of bf16 peak; "
        f"projections {proj / flops * 100:.0f}% of the flops, attention {attn / flops * 100:.0f}%)")
    res = dict(ms=ms, tokens_per_s=M / (ms * 1e-3), tflops=tflops, flops=flops, proj_flops=proj, attn_flops=attn,
               layers=L)
    del m, layers, x
    torch.cuda.empty_cache()
    return res


# ----------------------------------------------------------- CPU baseline

def _timed_runs(fn, min_seconds: float, min_runs: int):
    """Run fn() until both min_runs runs and min_seconds of wall time are done;
    returns the list of per-run seconds."""
    times = []
    t_end = time.perf_counter() + min_seconds
    while len(times) < min_runs or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return times


def cpu_baseline(dec, pre):
    """The oracle (C restatement of Crane's candle-CPU path, bf16 rounding
    points) on the host cores, on bounded samples of configs 3 and 4: the full
    config-3 step repeated for >= 10 s (median run), config 4 sequence by
    sequence for >= 10 s, and 1-thread samples of each."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import oracle
    threads, model = cpu_info()
    res = {}
    scale = 1.0 / math.sqrt(D)
    if dec is not None:
        q, k, v, kv_len = dec["_tensors"]
        qn = q.float().cpu().numpy()
        kn = np.ascontiguousarray(k.float().cpu().numpy())
        vn = np.ascontiguousarray(v.float().cpu().numpy())
        lens = np.ascontiguousarray(kv_len)
        B = qn.shape[0]

        def step(nb, nt):
            return lambda: oracle.attn_decode(qn[:nb], kn[:nb], vn[:nb], lens[:nb], scale, "bf16",
                                              oracle.DECODE_GROUPED, nt)

        def nbytes(nb):
            return int(lens[:nb].sum()) * dec["Hkv"] * D * 2 * 2 + 2 * nb * dec["Hq"] * D * 2

        times = _timed_runs(step(B, threads), 10.0, 5)
        t = float(np.median(times))
        t1 = float(np.median(_timed_runs(step(4, 1), 3.0, 3)))
        res["decode"] = dict(value=nbytes(B) / t / 1e9, unit="GB/s", cores=threads, kind="port",
                             one_thread=round(nbytes(4) / t1 / 1e9, 3),
                             sample=f"the full config-3 step (32 sequences, sum L={int(lens.sum())}), bf16 op chain, "
                                    f"median of {len(times)} runs ({sum(times):.1f} s, {t * 1e3:.1f} ms each); "
                                    f"one_thread: sequences 0-3 on 1 thread; host {model}")
        log(f"[cpu decode] {res['decode']['value']:.2f} GB/s on {threads} threads "
            f"({res['decode']['one_thread']:.2f} GB/s on 1)")
    if pre is not None:
        q, k, v = pre["_tensors"]
        B, S, Hq = pre["B"], pre["S"], pre["Hq"]
        start = np.zeros(1, np.int32)

        def seq_flops(r0, r1):
            return 4.0 * D * Hq * (r1 * (r1 + 1) - r0 * (r0 + 1)) / 2

        flops, t, done = 0.0, 0.0, 0
        for b in range(B):
            qn = np.ascontiguousarray(q[b:b + 1].float().cpu().numpy())
            kn = np.ascontiguousarray(k[b:b + 1].float().cpu().numpy())
            vn = np.ascontiguousarray(v[b:b + 1].float().cpu().numpy())
            t0 = time.perf_counter()
            oracle.attn_prefill(qn, kn, vn, start, scale, True, "bf16", nthreads=threads)
            t += time.perf_counter() - t0
            flops += seq_flops(0, S)
            done += 1
            if t >= 10.0:
                break
        r0 = S - 64                                           # 1 thread: the 64 heaviest rows of sequence 0
        t0 = time.perf_counter()
        oracle.attn_prefill(qn, kn, vn, start, scale, True, "bf16", rows=(r0, S), nthreads=1)
        t1 = time.perf_counter() - t0
        res["prefill"] = dict(value=flops / t / 1e12, unit="TFLOP/s", cores=threads, kind="port",
                              one_thread=round(seq_flops(r0, S) / t1 / 1e12, 5),
                              sample=f"config 4, {done} of {B} sequences (all {S} rows x {Hq} heads, causal flops "
                                     f"counted), bf16 op chain, {t:.1f} s; one_thread: rows {r0}-{S - 1} of the last "
                                     f"sequence run, {t1:.1f} s; host {model}")
        log(f"[cpu prefill] {res['prefill']['value'] * 1e3:.3f} GFLOP/s on {threads} threads "
            f"({res['prefill']['one_thread'] * 1e3:.3f} on 1)")
    return res


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--only", choices=["decode", "prefill", "append", "layer", "gemm", "sampling", "model",
                                       "model_prefill", "all"],
                    default="all")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--prefill-modes", default="1,3",
                    help="flags values of the timed c4 prefill, the first one the headline: 1 = causal (both of "
                         "candle's score roundings, the default), 3 = causal + "
                         "CRANE_HIP_PREFILL_LONG_ROWS_ONE_ROUNDING")
    ap.add_argument("--no-const-inputs", action="store_true",
                    help="skip the constant-input legs of the prefill and GEMM benches (for counter runs, so every "
                         "dispatch of a kernel is the N(0, 1) workload)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain elementwise kernel over 1 GiB (scales FETCH_SIZE/WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the attention path runs on a single MI355X and this build "
              "launches nothing on a second GPU (the kernels would shard by kv head across GPUs). Use --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from crane_amd import _lib
    lib = _lib.lib()
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    log(f"device: {torch.cuda.get_device_name(dev)}; lib: {_lib.version()}")

    if args.copy_calibration:
        # A plain elementwise kernel of known traffic: reads 1 GiB, writes 1 GiB.
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        log("[calibration] 3 x neg over 2^28 f32 (1073741824 B read + 1073741824 B written each)")
        del src, dst
        torch.cuda.empty_cache()
    dec = pre = c5 = c2 = app = pg = pf32 = None
    ceil = None
    if args.only in ("decode", "all"):
        dec = bench_decode(args, dev, stream, lib)
        ceil = bench_read_ceiling(args, dev, stream)
        if args.only == "all":
            c5 = bench_decode_c5(args, dev, stream, lib)
            pg = bench_decode_paged(args, dev, stream, lib)
    if args.only in ("prefill", "all"):
        pre = bench_prefill(args, dev, stream, lib)
        if args.only == "all":
            c2 = bench_prefill_c2(args, dev, stream, lib)
            pf32 = bench_prefill_f32(args, dev, stream, lib)
    if args.only in ("append", "all"):
        app = bench_append(args, dev, stream, lib)
    lay = bench_layer(args, dev, stream, lib) if args.only in ("layer", "all") else None
    gem = bench_gemm(args, dev, stream, lib) if args.only in ("gemm", "all") else None
    smp = bench_sampling(args, dev, stream, lib) if args.only in ("sampling", "all") else None
    mod = bench_model_step(args, dev, stream, lib) if args.only in ("model", "all") else None
    mpf = bench_model_prefill(args, dev, stream, lib) if args.only in ("model_prefill", "all") else None
    cpu = {} if args.no_cpu_baseline else cpu_baseline(dec, pre)

    traffic = pmc_traffic()
    src = os.path.relpath(TRAFFIC_FILE, os.path.dirname(os.path.abspath(__file__)))
    line = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded N(0,1) q/K/V; lengths U{512..4096} seeded)"}
    if dec is not None:
        line.update({
            "value": round(dec["gbs"], 2), "unit": "GB/s", "ms_per_step": round(dec["ms"], 5),
            "config": {"workload": "c3: Qwen3-8B-shape batched decode attention, B=32, 32 q / 8 kv heads, "
                                   "D=128, bf16 KV cache, L_i~U{512..4096} seeded (+1 new token each)",
                       "batch": 32, "q_heads": 32, "kv_heads": 8, "head_dim": 128,
                       "sum_kv_rows": int(dec["kv_len"].sum()), "kv_bytes_per_step": dec["kv_bytes"]},
            "roofline": {"bound": "hbm", "achieved": round(dec["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(dec["gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic.get("decode_c3"),
                         "traffic_source": src,
                         "kernel": "decode_chunk_kernel + decode_merge_kernel (one crane_hip_attn_decode call)",
                         "algo_bytes_per_launch": dec["algo_bytes"]},
            "ms_p10_p50_p90": dec["pct"],
            "statistic": "value and ms_per_step: mean over the K timed back-to-back launches (one event pair "
                         "around all K, caches rotated over 3 copies); ms_p10_p50_p90: 100 individually "
                         "event-timed launches after the timed region; value_p50: GB/s at that median",
            "value_p50": round(dec["algo_bytes"] / (dec["pct"][1] * 1e-3) / 1e9, 2),
        })
        if ceil is not None:
            line["hbm_read_ceiling"] = {
                "gbs": round(ceil["gbs"], 1), "frac_of_peak": round(ceil["gbs"] / HBM_PEAK_GBS, 4),
                "span_kib_per_workgroup": ceil["span_kib"], "bytes_per_launch": 320 * 1000 * 1000,
                "decode_frac_of_ceiling": round(dec["gbs"] / ceil["gbs"], 4),
                "decode_p50_frac_of_ceiling": round(line["value_p50"] / ceil["gbs"], 4),
                "single_reads": ceil["single_reads"],
                "note": "a read-only stream with the decode kernel's access pattern and load form "
                        "(crane_amd/csrc/probe/hbm_probe.hip, a measurement helper outside the library: one "
                        "workgroup per contiguous span, all its loads in flight), 3 rotated 320 MB buffers; the "
                        "decode roofline's peak stays the 8 TB/s datasheet figure; single_reads: one launch reading "
                        "one decode-step weight's bytes (Qwen3-8B shape), back to back from HBM"}
    if pre is not None:
        pre_obj = {"metric": "prefill attn TFLOP/s (c4: Qwen2.5-7B shape, B=8, S=4096, 28/4 heads, causal, bf16)",
                   "value": round(pre["tflops"], 2), "unit": "TFLOP/s", "ms_per_step": round(pre["ms"], 4),
                   "roofline": {"bound": "mfma", "achieved": round(pre["tflops"], 2), "peak": BF16_PEAK_TFLOPS,
                                "unit": "TFLOP/s", "frac": round(pre["tflops"] / BF16_PEAK_TFLOPS, 4),
                                "traffic": traffic.get("prefill_c4"), "traffic_source": src,
                                "kernel": "prefill_bf16_kernel<true>",
                                "algo_flops_per_launch": pre["flops"]},
                   "ms_p10_p50_p90": pre["pct"], "flags": pre["flags"],
                   "modes": {str(f): {"ms": round(r["ms"], 4), "tflops": round(r["tflops"], 2),
                                      "frac": round(r["tflops"] / BF16_PEAK_TFLOPS, 4),
                                      "ms_p10_p50_p90": r["pct"]} for f, r in pre["modes"].items()},
                   "modes_note": "flags 1: causal, both of candle's score roundings (the library default); "
                                 "flags 3: + CRANE_HIP_PREFILL_LONG_ROWS_ONE_ROUNDING (opt-in)",
                   "ms_const_inputs": round(pre["ms_const"], 4) if pre["ms_const"] else None,
                   "frac_const_inputs": (round(pre["flops"] / (pre["ms_const"] * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4)
                                         if pre["ms_const"] else None)}
        if "prefill" in cpu:
            pre_obj["cpu_baseline"] = cpu["prefill"]
        if dec is None:
            line.update({"value": pre_obj["value"], "unit": "TFLOP/s", "ms_per_step": pre_obj["ms_per_step"],
                         "config": {"workload": "c4: Qwen2.5-7B-shape causal prefill"},
                         "roofline": pre_obj["roofline"]})
        line["prefill"] = pre_obj
    if c5 is not None:
        line["decode_c5"] = {"workload": "c5: Qwen2.5-72B-shape decode, B=8, 64/8 heads, L=32768+1",
                             "value": round(c5["gbs"], 2), "unit": "GB/s", "us_per_step": round(c5["ms"] * 1e3, 2),
                             "frac": round(c5["gbs"] / HBM_PEAK_GBS, 4)}
    if pg is not None:
        line["decode_c3_paged"] = {"workload": "c3 over a paged cache (shuffled 256-row pages, block table)",
                                   "value": round(pg["gbs"], 2), "unit": "GB/s",
                                   "us_per_step": round(pg["ms"] * 1e3, 2), "frac": round(pg["gbs"] / HBM_PEAK_GBS, 4),
                                   "kernel": "decode_chunk_kernel<PagedRows> + decode_merge_kernel"}
    if pf32 is not None:
        line["prefill_c2_f32"] = {"workload": "c2 shape in f32: causal prefill, S=2048, 16/8 heads (f32 MFMA kernel)",
                                  "us_per_step": round(pf32["ms"] * 1e3, 1), "value": round(pf32["tflops"], 2),
                                  "unit": "TFLOP/s", "frac": round(pf32["tflops"] / F32_PEAK_TFLOPS, 4),
                                  "peak": F32_PEAK_TFLOPS}
    if c2 is not None:
        line["prefill_c2"] = {"workload": "c2: Qwen3-0.6B-shape append+causal prefill, S=2048, 16/8 heads",
                              "us_per_step": round(c2["ms"] * 1e3, 2), "tflops": round(c2["tflops"], 2)}
    if app is not None:
        line["append"] = {k: {kk: (round(vv, 2) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                          for k, v in app.items()}
        if dec is None and pre is None:
            a = app["c4_prefill_append"]
            line.update({"value": round(a["gbs"], 2), "unit": "GB/s", "ms_per_step": round(a["us"] / 1e3, 5),
                         "config": {"workload": "fused QK-norm+RoPE+KV append, c4 prefill size"}})
    if lay is not None:
        line["layer_ops"] = {t: {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                                 for k, v in d.items()} for t, d in lay.items()}
    if gem is not None:
        line["gemm"] = {t: {k: round(v, 4) for k, v in d.items()} for t, d in gem.items()}
    if smp is not None:
        line["sampling"] = {t: {k: round(v, 2) for k, v in d.items()} for t, d in smp.items()}
    if mod is not None:
        line["model_decode_step"] = {
            "workload": "Qwen3-8B-shape model decode step (36 layers, final norm, lm_head 151936) at c3: B=32, "
                        "L_i~U{512..4096}; HIP-graph replay of crane_amd.model.DecodeGraph",
            "ms_per_step": round(mod["ms"], 4), "tokens_per_s": round(mod["tokens_per_s"], 1),
            "roofline": {"bound": "hbm", "achieved": round(mod["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(mod["gbs"] / HBM_PEAK_GBS, 4),
                         "bytes_per_step": mod["weight_bytes"] + mod["kv_bytes"],
                         "weight_bytes": mod["weight_bytes"], "kv_bytes": mod["kv_bytes"]}}
    if mpf is not None:
        line["model_prefill_step"] = {
            "workload": "Qwen2.5-7B-shape model prefill step (28 layers, QKV bias, final norm, lm_head 152064 on "
                        "the last position) at c4: B=8 x S=4096 new tokens into empty caches; "
                        "crane_amd.model.DecoderModel.forward",
            "ms_per_step": round(mpf["ms"], 3), "tokens_per_s": round(mpf["tokens_per_s"], 1),
            "roofline": {"bound": "mfma", "achieved": round(mpf["tflops"], 1), "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(mpf["tflops"] / BF16_PEAK_TFLOPS, 4),
                         "flops_per_step": mpf["flops"], "projection_flops": mpf["proj_flops"],
                         "attention_flops": mpf["attn_flops"]}}
    if "decode" in cpu:
        line["cpu_baseline"] = cpu["decode"]
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
