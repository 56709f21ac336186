"""Benchmark of the MI355X decode path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload decode|prefill|gemv|gemv_i8|gemv_rows|copy|floor|gemm|attn|moe] [--no-cpu]

Prints one JSON line.

decode (the default, BASELINE's headline): the 28-layer synthetic Qwen3 (hidden 2048, 16/8 heads,
head_dim 128, SwiGLU 6144, vocab 151936, tied fp16 embeddings, MXFP4 linears of std-0.02 weights,
seed 0) on one GPU. A 1024-token prompt (ids uniform over the vocabulary) is prefilled, then 256
tokens are greedy-decoded, each step one replay of a step graph; both step graphs are captured
before any timing. The first 256 - K steps (at least W) run untimed and the last K are timed
(decode_tokens grows past 256 only when K + W exceed it). value = K / the timed region's seconds
(HIP events on the replay stream): decode tokens per second at batch 1. The prefill rate is
reported beside it.

roofline: the batch-1 MXFP4 GEMV of the GEMV configuration (W 8192 x 2048 MXFP4, x fp16, y fp16),
the decode step's dominant kernel kind: 64 back-to-back GEMVs over 64 distinct weight copies (572
MB, past the 256 MB MALL) in one HIP graph, timed with HIP events on the replay stream; achieved =
8,933,376 algorithmic bytes a launch (codes 8,388,608 + scales 524,288 + x 4,096 + y 16,384) over
the average launch time. traffic: HBM bytes a launch moves, measured each run by four child
processes under `rocprofv3 --pmc` (FETCH_SIZE, WRITE_SIZE of the GEMV dispatches, each scaled by the
counter's reading of a plain device copy of the same bytes) before this process touches the GPU;
null, with the reason, when rocprofv3 is unavailable.

gemv: only that GEMV measurement. copy: a plain device copy of the same 8,933,376 bytes timed the
same way (the calibration run for the FETCH_SIZE / WRITE_SIZE counters). floor: hwk_read_floor, one
launch that only reads the same bytes, over a sweep of waves a CU and loads a lane in flight: the
shortest time a single launch needs for them (roofline.read_floor carries its best of three shapes).

The other configurations (each a graph of back-to-back launches over distinct input copies, timed
with HIP events; the decode line carries them under "configs" without CPU baselines, and the
workloads below print them with theirs):
- prefill: the C5 prefill alone, the 1024-token prompt through the 28-layer model (median of K runs),
  tokens/s and TFLOP/s against the fp16 MFMA peak (linears 2.886 TFLOP + causal attention 0.120).
- gemv_i8: K2, the int8 GEMV 8192 x 2048 with fp16 row scales (16,814,080 B), 64 copies; gemv_rows:
  K1r, C1's MXFP4 matrix times T = 1, 2, 4, 8 fp16 vectors (the verify form), the matrix read once.
- gemm: the int8 weight-only prefill GEMM, M=512 K=2048 N=6144 (fp16 X, int8 W, fp16 per-row
  scale, fp16 Y): 12.88 GFLOP a launch, TFLOP/s against the 2.5 PFLOP/s dense fp16 MFMA peak; CPU:
  the oracle's shiftScale dequant (cached, as milcpu caches constants) + blocked fp32 sgemm on 64
  rows of X, scaled.
- attn: GQA decode attention, 32 query / 8 KV heads, head_dim 128, L in {512, 2048, 8192, 32768},
  fp16 KV (4,096 L + 16,384 B) and int8 KV with per-(head, token) scales (2,080 L + 16,384 B):
  GB/s against 8 TB/s; CPU: the oracle's chunk attention + Merge (runner.attentionCPU's form).
- moe: the MoE decode layer, hidden 2048, 32 experts, top-4 softmax routing, SwiGLU 768, MXFP4:
  route + experts at T = 1 and 5; bytes = unique experts x 2,506,752 + activations; GB/s; CPU: the
  oracle's Routing.Choose + Host.Run with int8-quantized activations (the reference's production
  numerics).

cpu_baseline (decode): the oracle's restatement of the reference's CPU decode step, timed on the
host's cores on a bounded sample and scaled to one token: one layer's MXFP4 linears through
mxfp4.Run with the int8-quantized activation (internal/mxfp4/matvec.go:33-160), one layer's chunked
attention + Merge at 1152 keys (internal/llm/paged/paged.go:70-310), each times 28, plus the tied
head as dequantized fp32 sgemm (internal/sgemm/sgemm.go:127-163).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
C5 = dict(layers=28, hidden=2048, heads=16, kv_heads=8, head_dim=128, inter=6144, vocab=151936)
PROMPT = 1024
# algorithmic bytes of one decode token at cache position p: MXFP4 linears 28 x 50,331,648 params
# x 17/32 B, the tied fp16 head, K/V read 114,688 B a position and written once, the embedding row
LIN_BYTES = 28 * 50331648 * 17 // 32
HEAD_BYTES = 151936 * 2048 * 2
KV_POS_BYTES = 28 * 2 * 8 * 128 * 2
GEMV_N, GEMV_K = 8192, 2048
GEMV_BYTES = GEMV_N * GEMV_K // 2 + GEMV_N * GEMV_K // 32 + GEMV_K * 2 + GEMV_N * 2  # 8,933,376
COPIES = 64
# the K1 kernel's name as rocprofv3 reports it (the dispatches whose counters measure_traffic reads)
GEMV_KERNEL = "k_mxfp4_gemv_lds"


def _graph_time(launch_all, steps: int, warmup: int, eager: bool = False):
    """Per-launch microseconds of COPIES launches captured in one graph, replayed until at least
    `steps` launches ran, timed with events on the replay stream. eager: the same launches issued
    one by one without a graph (for counter collection, which profiles dispatches one at a time)."""
    import torch

    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        launch_all()  # eager once: loads the code objects before capture
    torch.cuda.synchronize()
    if eager:
        run = launch_all
    else:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            launch_all()
        run = g.replay
    replays = max(1, -(-steps // COPIES))
    with torch.cuda.stream(s):
        for _ in range(-(-warmup // COPIES)):
            run()
        s.synchronize()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        a.record(s)
        for _ in range(replays):
            run()
        b.record(s)
        b.synchronize()
        wall = time.perf_counter() - t0
    launches = replays * COPIES
    return a.elapsed_time(b) * 1e3 / launches, launches, wall


def gemv_roofline(steps: int, warmup: int, eager: bool = False):
    import torch

    from hwnpu_amd import ops, synth

    ws = [synth.mxfp4_uniform(GEMV_N, GEMV_K, f"bench.c1.{i}") for i in range(COPIES)]
    x = synth.normal(GEMV_K, "bench.c1.x", dtype=torch.float16)
    y = torch.empty(GEMV_N, dtype=torch.float16, device="cuda")

    def launch_all():
        for w, e in ws:
            ops.mxfp4_gemv(w, e, x, "f16", y=y)

    us, launches, wall = _graph_time(launch_all, steps, warmup, eager)
    return {"us": us, "launches": launches, "wall_s": wall, "gbs": GEMV_BYTES / (us * 1e-6) / 1e9}


# K2, the int8 GEMV on C1's shape (SURVEY's "C1 int8 GEMV"): codes + fp16 row scales + x + fp16 y
GEMV_I8_BYTES = GEMV_N * GEMV_K + GEMV_N * 2 + GEMV_K * 2 + GEMV_N * 2


def gemv_i8_rate(steps: int = 1280, warmup: int = 128):
    """K2 (hwk_i8_gemv) on 8192 x 2048 int8 rows with fp16 scales, 64 distinct copies in a graph."""
    import torch

    from hwnpu_amd import ops, synth

    ws = [(synth.uniform_int(GEMV_N * GEMV_K, -127, 255, f"bench.k2.q{i}", dtype=torch.int8).view(GEMV_N, GEMV_K),
           synth.uniform_real(GEMV_N, 0.002, 0.02, f"bench.k2.s{i}")) for i in range(COPIES)]
    x = synth.normal(GEMV_K, "bench.k2.x", dtype=torch.float16)
    y = torch.empty(GEMV_N, dtype=torch.float16, device="cuda")

    def launch_all():
        for q, s in ws:
            ops.i8_gemv(q, s, x, "f16", y=y)

    us, launches, _ = _graph_time(launch_all, steps, warmup)
    gbs = GEMV_I8_BYTES / (us * 1e-6) / 1e9
    return {"config": "int8 GEMV 8192x2048, fp16 scales, fp16 x and y", "us": round(us, 3),
            "bytes": GEMV_I8_BYTES, "gbs": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}


def gemv_rows_rate(T: int, steps: int = 640, warmup: int = 64):
    """K1r (hwk_mxfp4_gemv_rows): C1's MXFP4 matrix times T fp16 vectors (the verify step's form),
    each weight row read once for all T; 64 distinct matrices in a graph."""
    import torch

    from hwnpu_amd import ops, synth

    ws = [synth.mxfp4_uniform(GEMV_N, GEMV_K, f"bench.c1.{i}") for i in range(COPIES)]
    x = synth.normal(T * GEMV_K, f"bench.k1r.x{T}", dtype=torch.float16).view(T, GEMV_K)
    y = torch.empty((T, GEMV_N), dtype=torch.float16, device="cuda")

    def launch_all():
        for w, e in ws:
            ops.mxfp4_gemv_rows(w, e, x, "f16", y=y)

    us, _, _ = _graph_time(launch_all, steps, warmup)
    nbytes = GEMV_N * GEMV_K // 2 + GEMV_N * GEMV_K // 32 + T * (GEMV_K * 2 + GEMV_N * 2)
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"T": T, "us": round(us, 3), "bytes": nbytes, "gbs": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}


FLOOR_SHAPES = [(wpc, lpl) for wpc in (8, 16, 32) for lpl in (1, 2, 4)]


def read_floor(steps: int = 1280, warmup: int = 128, shapes=FLOOR_SHAPES):
    """The read floor of the GEMV configuration's bytes: hwk_read_floor over 64 distinct buffers of
    GEMV_BYTES each (one launch each, in a graph, as the GEMV is timed), for each (waves a CU, loads a
    lane in flight); the fastest is the shortest time in which one launch reads those bytes here."""
    import torch

    from hwnpu_amd import hwk

    lib = hwk.load()
    src = [torch.empty(GEMV_BYTES, dtype=torch.uint8, device="cuda") for _ in range(COPIES)]
    for t in src:
        t.random_(0, 255)
    out = torch.zeros(16, dtype=torch.int32, device="cuda")
    rows = []
    for wpc, lpl in shapes:
        def launch_all():
            s = torch.cuda.current_stream().cuda_stream
            for t in src:
                lib.hwk_read_floor(s, t.data_ptr(), GEMV_BYTES, out.data_ptr(), wpc, lpl)

        us, _, _ = _graph_time(launch_all, steps, warmup)
        rows.append({"waves_per_cu": wpc, "loads_per_lane": lpl, "us": round(us, 3),
                     "gbs": round(GEMV_BYTES / (us * 1e-6) / 1e9, 1)})
    best = min(rows, key=lambda r: r["us"])
    return best, rows


def copy_roofline(steps: int, warmup: int, eager: bool = False):
    import torch

    src = [torch.empty(GEMV_BYTES, dtype=torch.uint8, device="cuda") for _ in range(COPIES)]
    dst = torch.empty(GEMV_BYTES, dtype=torch.uint8, device="cuda")

    def launch_all():
        for t in src:
            dst.copy_(t)

    us, launches, wall = _graph_time(launch_all, steps, warmup, eager)
    return {"us": us, "launches": launches, "wall_s": wall, "gbs": 2 * GEMV_BYTES / (us * 1e-6) / 1e9}


def _graph_us(launch_all, copies: int, replays: int = 20):
    """Microseconds a launch of `copies` launches captured in one graph, replayed `replays` times."""
    import torch

    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        launch_all()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        launch_all()
    with torch.cuda.stream(st):
        g.replay()
        st.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(st)
        for _ in range(replays):
            g.replay()
        b.record(st)
        b.synchronize()
    return a.elapsed_time(b) * 1e3 / (replays * copies)


GEMM_M, GEMM_N, GEMM_K = 512, 6144, 2048
GEMM_FLOP = 2 * GEMM_M * GEMM_N * GEMM_K
GEMM_BYTES = GEMM_N * GEMM_K + GEMM_N * 2 + GEMM_M * GEMM_K * 2 + GEMM_M * GEMM_N * 2
MFMA_PEAK_TFLOPS = 2500.0


def gemm_rate(copies: int = 8):
    import torch

    from hwnpu_amd import ops, synth

    x = synth.normal(GEMM_M * GEMM_K, "bench.c2.x").view(GEMM_M, GEMM_K)
    ws = [(synth.uniform_int(GEMM_N * GEMM_K, -127, 255, f"bench.c2.q.{i}", dtype=torch.int8).view(GEMM_N, GEMM_K),
           synth.uniform_real(GEMM_N, 0.002, 0.02, f"bench.c2.s.{i}")) for i in range(copies)]
    y = torch.empty((GEMM_M, GEMM_N), dtype=torch.float16, device="cuda")

    def launch_all():
        for q, sc in ws:
            ops.i8_gemm(x, q, sc, "f16", y=y)

    us = _graph_us(launch_all, copies)
    tf = GEMM_FLOP / (us * 1e-6) / 1e12
    return {"config": "int8 GEMM M=512 K=2048 N=6144, fp16 out", "us": round(us, 2), "tflops": round(tf, 1),
            "frac_mfma": round(tf / MFMA_PEAK_TFLOPS, 4), "gbs": round(GEMM_BYTES / (us * 1e-6) / 1e9, 1)}


def gemm_cpu(rows: int = 64):
    import numpy as np

    from oracle import oracle

    rng = np.random.default_rng(0)
    q = rng.integers(-127, 128, (GEMM_N, GEMM_K), dtype=np.int8)
    sc = (rng.uniform(0.002, 0.02, GEMM_N).astype(np.float16)).view(np.uint16)
    wd = oracle.i8_dequant(q, sc)  # once: milcpu caches the dequantized constant
    x = rng.standard_normal((rows, GEMM_K)).astype(np.float16).astype(np.float32)
    oracle.sgemm(x[:8], wd, transb=True)
    ts = []
    for _ in range(3):
        t = time.perf_counter()
        oracle.sgemm(x, wd, transb=True)
        ts.append(time.perf_counter() - t)
    t = sorted(ts)[1] * GEMM_M / rows
    return {"value": round(GEMM_FLOP / t / 1e12, 4), "unit": "TFLOP/s", "cores": oracle.max_threads(), "kind": "port",
            "sample": f"sgemm of {rows} of the 512 rows against the dequantized weights, median of 3, scaled"}


ATTN_LENS = (512, 2048, 8192, 32768)


def attn_rate(L: int, int8: bool):
    import math

    import torch

    from hwnpu_amd import ops, synth

    kv_bytes = (2080 if int8 else 4096) * L + 16384
    copies = max(2, min(160, -(-(320 << 20) // kv_bytes)))
    q = synth.normal(32 * 128, f"bench.c3.q.{L}").view(32, 128)
    caches = []
    for i in range(copies):
        k = synth.normal(8 * L * 128, f"bench.c3.k.{L}.{i}").view(8, L, 128)
        v = synth.normal(8 * L * 128, f"bench.c3.v.{L}.{i}").view(8, L, 128)
        if int8:
            kq, ks = ops.kv_quantize_i8(k)
            vq, vs = ops.kv_quantize_i8(v)
            caches.append((kq, vq, ks, vs))
        else:
            caches.append((k, v, None, None))
    torch.cuda.synchronize()
    out = torch.empty((32, 128), dtype=torch.float16, device="cuda")
    p = ops.attn_params(32, 8, L, L, int8, 1 / math.sqrt(128), "f16")
    ws = ops.attn_workspace(p)

    def launch_all():
        for k, v, ks, vs in caches:
            ops.attn_decode(q, k, v, L, ks, vs, out_mode="f16", out=out, workspace=ws)

    us = _graph_us(launch_all, copies, 10)
    gbs = kv_bytes / (us * 1e-6) / 1e9
    return {"L": L, "kv": "int8" if int8 else "fp16", "us": round(us, 2), "gbs": round(gbs, 1),
            "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "copies": copies}


def attn_cpu(L: int):
    import numpy as np

    from oracle import oracle

    rng = np.random.default_rng(0)
    q = rng.standard_normal((32, 128)).astype(np.float32)
    k = rng.standard_normal((8, L, 128)).astype(np.float32)
    v = rng.standard_normal((8, L, 128)).astype(np.float32)
    oracle.attn_decode(q, k[:, :64], v[:, :64], 128 ** -0.5)
    ts = []
    for _ in range(3):
        t = time.perf_counter()
        oracle.attn_decode(q, k, v, 128 ** -0.5)
        ts.append(time.perf_counter() - t)
    t = sorted(ts)[1]
    return {"value": round((4096 * L + 16384) / t / 1e9, 3), "unit": "GB/s (fp16-KV bytes)",
            "cores": oracle.max_threads(), "kind": "port", "sample": f"L={L}, median of 3"}


MOE_E, MOE_H, MOE_I, MOE_K = 32, 2048, 768, 4
MOE_EXPERT_BYTES = 2 * MOE_I * MOE_H // 2 + 2 * MOE_I * MOE_H // 32 + MOE_H * MOE_I // 2 + MOE_H * MOE_I // 32


def moe_rate(T: int, copies: int = 4):
    import torch

    from hwnpu_amd import ops, synth

    layers = []
    uniq = []
    for i in range(copies):
        gw, ge = synth.mxfp4_uniform(MOE_E * 2 * MOE_I, MOE_H, f"bench.c4.gu.{i}")
        dw, de = synth.mxfp4_uniform(MOE_E * MOE_H, MOE_I, f"bench.c4.dn.{i}")
        gw = gw.view(MOE_E, 2 * MOE_I, MOE_H // 32, 16)
        ge = ge.view(MOE_E, 2 * MOE_I, MOE_H // 32)
        dw = dw.view(MOE_E, MOE_H, MOE_I // 32, 16)
        de = de.view(MOE_E, MOE_H, MOE_I // 32)
        logits = synth.normal(T * MOE_E, f"bench.c4.logits.{T}.{i}", dtype=torch.float32).view(T, MOE_E)
        x = synth.normal(T * MOE_H, f"bench.c4.x.{T}.{i}").view(T, MOE_H)
        idx, _ = ops.moe_route(logits, MOE_K)
        uniq.append(len(set(idx.cpu().numpy().ravel().tolist())))
        layers.append((gw, ge, dw, de, logits, x))
    out = torch.empty((T, MOE_H), dtype=torch.float32, device="cuda")
    ws = torch.empty(T * MOE_K * MOE_I * 4, dtype=torch.uint8, device="cuda")

    def launch_all():
        # hwk_moe_layer: the route folded into the gate_up launch, down with the ordered combine
        for gw, ge, dw, de, logits, x in layers:
            ops.moe_layer(x, logits, MOE_K, gw, ge, dw, de, out=out, workspace=ws)

    us = _graph_us(launch_all, copies, 20)
    u = sum(uniq) / len(uniq)
    nbytes = u * MOE_EXPERT_BYTES + T * MOE_H * 2 + T * MOE_H * 4 + T * MOE_E * 4
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"T": T, "unique_experts": u, "us": round(us, 2), "gbs": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}


def moe_cpu(T: int):
    import numpy as np

    from oracle import oracle

    rng = np.random.default_rng(0)
    gw = rng.integers(0, 256, (MOE_E, 2 * MOE_I, MOE_H // 32, 16), dtype=np.uint8)
    ge = rng.integers(123, 130, (MOE_E, 2 * MOE_I, MOE_H // 32), dtype=np.uint8)
    dw = rng.integers(0, 256, (MOE_E, MOE_H, MOE_I // 32, 16), dtype=np.uint8)
    de = rng.integers(123, 130, (MOE_E, MOE_H, MOE_I // 32), dtype=np.uint8)
    logits = rng.standard_normal((T, MOE_E)).astype(np.float32)
    x = rng.standard_normal((T, MOE_H)).astype(np.float16).astype(np.float32)

    def run():
        idx = np.empty((T, MOE_K), np.int32)
        w = np.empty((T, MOE_K), np.float32)
        for t in range(T):
            idx[t], w[t] = oracle.choose(logits[t], MOE_K)
        oracle.experts(x, idx, w, gw, ge, dw, de, quantized=True)
        return len(set(idx.ravel().tolist()))

    u = run()
    ts = []
    for _ in range(5):
        t = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t)
    t = sorted(ts)[2]
    nbytes = u * MOE_EXPERT_BYTES + T * MOE_H * 6 + T * MOE_E * 4
    return {"value": round(nbytes / t / 1e9, 3), "unit": "GB/s", "cores": oracle.max_threads(), "kind": "port",
            "sample": f"T={T}: Choose + Host.Run (int8 activations, mxfp4.Run), median of 5, {u} unique experts"}


DECODE_TOKENS = 256  # C5: greedy-decode 256 tokens after the 1024-token prompt


def decode_rate(steps: int, warmup: int):
    """The C5 run: prefill the 1024-token prompt, then greedy-decode DECODE_TOKENS tokens (more only
    when steps + warmup exceed it), each step a replay of a step graph captured before any timing.
    The first decode_tokens - steps steps (at least `warmup`) run untimed; the last `steps` are timed
    with HIP events on the replay stream."""
    import numpy as np
    import torch

    from hwnpu_amd import synth
    from hwnpu_amd.qwen3 import Qwen3

    untimed = max(warmup, DECODE_TOKENS - steps)
    total = untimed + steps
    m = Qwen3(**C5, max_ctx=PROMPT + total + 8, max_prompt=PROMPT)
    m.synth(seed=0, std=0.02)
    prompt = synth.uniform_int(PROMPT, 0, C5["vocab"], "c5.prompt").cpu().numpy().astype(np.int32)
    s = torch.cuda.current_stream()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    m.prefill(prompt[:16], 0)  # first use: code objects load outside the timed prefill
    torch.cuda.synchronize()
    a.record(s)
    m.prefill(prompt, 0)
    b.record(s)
    b.synchronize()
    prefill_s = a.elapsed_time(b) / 1e3
    m.capture()  # both step graphs, captured and instantiated before any timed region
    m.decode(untimed)
    torch.cuda.synchronize()
    a.record(s)
    m.decode(steps)
    b.record(s)
    b.synchronize()
    dec_s = a.elapsed_time(b) / 1e3
    first = PROMPT + untimed  # position of the first timed step
    toks = m.history(PROMPT, 8)
    m.close()
    p_mean = first + (steps - 1) / 2
    step_bytes = LIN_BYTES + HEAD_BYTES + KV_POS_BYTES * (p_mean + 1) + KV_POS_BYTES + C5["hidden"] * 2
    return {"tok_s": steps / dec_s, "ms_per_tok": dec_s / steps * 1e3, "prefill_tok_s": PROMPT / prefill_s,
            "prefill_ms": prefill_s * 1e3, "step_bytes": step_bytes, "first_tokens": [int(t) for t in toks],
            "decode_tokens": total, "untimed": untimed, "timed_positions": [first, first + steps - 1]}


# C5 prefill work (algorithmic): the linears 2 * 1024 * 1,409,286,144 FLOP and the causal attention
# (QK^T and PV over the lower triangle: 4 * 128 * 16 heads * 1024 * 1025 / 2 FLOP a layer)
PREFILL_LIN_FLOP = 2 * PROMPT * 1_409_286_144
PREFILL_ATT_FLOP = C5["layers"] * 4 * 128 * C5["heads"] * PROMPT * (PROMPT + 1) // 2


def prefill_rate(reps: int):
    """The C5 prefill alone: the 1024-token prompt run `reps` times through the 28-layer model (each
    run overwrites the cache positions 0..1023), each timed with HIP events."""
    import numpy as np
    import torch

    from hwnpu_amd import synth
    from hwnpu_amd.qwen3 import Qwen3

    m = Qwen3(**C5, max_ctx=PROMPT + 8, max_prompt=PROMPT)
    m.synth(seed=0, std=0.02)
    prompt = synth.uniform_int(PROMPT, 0, C5["vocab"], "c5.prompt").cpu().numpy().astype(np.int32)
    s = torch.cuda.current_stream()
    m.prefill(prompt, 0)  # first use: code objects load outside the timed runs
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(s)
        m.prefill(prompt, 0)
        b.record(s)
        b.synchronize()
        times.append(a.elapsed_time(b))
    m.close()
    ms = sorted(times)[len(times) // 2]
    flop = PREFILL_LIN_FLOP + PREFILL_ATT_FLOP
    return {"workload": "prefill", "tokens": PROMPT, "reps": reps, "ms_median": round(ms, 3),
            "ms_all": [round(t, 3) for t in times], "tok_s": round(PROMPT / ms * 1e3, 1),
            "tflops": round(flop / ms / 1e9, 1), "frac_mfma": round(flop / ms / 1e9 / MFMA_PEAK_TFLOPS, 4),
            "flop": flop}


def host_cpu():
    """The host's CPU model (/proc/cpuinfo) and the cores this process may use."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return model, n


def _counter_mean_kib(counter: str, workload: str, match: str):
    """Mean per-dispatch value (KiB) of one rocprofv3 counter over the dispatches whose kernel name
    contains `match`, from a child `bench.py --workload <workload> --eager` run under
    `rocprofv3 --pmc <counter>` (a process of its own, started before this one touches the GPU)."""
    import csv
    import shutil
    import subprocess
    import tempfile

    prof = shutil.which("rocprofv3")
    if not prof:
        return None, "rocprofv3 not found"
    d = tempfile.mkdtemp(prefix="hwk_pmc_")
    cmd = ["timeout", "-s", "KILL", "120", prof, "--pmc", counter, "--output-format", "csv", "-d", d, "-o", "run",
           "--", sys.executable, os.path.abspath(__file__), "--workload", workload, "--eager", "--steps", "128",
           "--warmup", "0"]
    try:
        subprocess.run(cmd, stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL, timeout=150)
        vals = []
        for root, _, files in os.walk(d):
            for fn in files:
                if fn.endswith("counter_collection.csv"):
                    with open(os.path.join(root, fn)) as f:
                        for row in csv.DictReader(f):
                            if match in row["Kernel_Name"] and row["Counter_Name"] == counter:
                                vals.append(float(row["Counter_Value"]))
        if not vals:
            return None, f"no {counter} rows for {match}"
        return sum(vals) / len(vals), f"{len(vals)} dispatches"
    except Exception as e:  # the traffic figure is evidence, not the headline: report why it is missing
        return None, f"{type(e).__name__}: {e}"
    finally:
        shutil.rmtree(d, ignore_errors=True)


def measure_traffic():
    """HBM bytes a K1 launch moves: FETCH_SIZE and WRITE_SIZE of the GEMV's dispatches, each scaled by
    the ratio of a plain device copy's known byte count to what the same counter reads for it. Runs
    four child processes under rocprofv3 before this process uses the GPU; None when unavailable."""
    copy_kib = GEMV_BYTES / 1024.0
    fc, nfc = _counter_mean_kib("FETCH_SIZE", "copy", "copyBuffer")
    wc, nwc = _counter_mean_kib("WRITE_SIZE", "copy", "copyBuffer")
    fg, nfg = _counter_mean_kib("FETCH_SIZE", "gemv", GEMV_KERNEL)
    wg, nwg = _counter_mean_kib("WRITE_SIZE", "gemv", GEMV_KERNEL)
    if None in (fc, wc, fg, wg) or fc <= 0 or wc <= 0:
        return None, {"error": [nfc, nwc, nfg, nwg]}
    rf, rw = copy_kib / fc, copy_kib / wc
    read_b, write_b = fg * rf * 1024, wg * rw * 1024
    return int(read_b + write_b), {"fetch_kib": round(fg, 2), "write_kib": round(wg, 2),
                                   "fetch_scale": round(rf, 4), "write_scale": round(rw, 4),
                                   "read_bytes": int(read_b), "write_bytes": int(write_b),
                                   "dispatches": [nfg, nwg], "over_algorithmic": round((read_b + write_b) / GEMV_BYTES, 4)}


def cpu_decode_baseline():
    """The reference's CPU decode step restated (oracle, test infrastructure), on a bounded sample
    scaled to one token: one layer's linears through mxfp4.Run and its attention at 1152 keys, each
    times 28, plus the head in fp32 sgemm; every host core."""
    import numpy as np

    from oracle import oracle

    rng = np.random.default_rng(0)
    H, I, V = C5["hidden"], C5["inter"], C5["vocab"]
    mats = [(4096, H), (H, 2048), (2 * I, H), (H, I)]  # qkv, o, gate_up, down
    ws = [(rng.integers(0, 256, (n, k // 2), dtype=np.uint8), rng.integers(120, 125, (n, k // 32), dtype=np.uint8))
          for n, k in mats]
    xs = {k: oracle.vec_quantize(rng.standard_normal(k).astype(np.float32)) for _, k in mats}
    L = 1152
    q = rng.standard_normal((16, 128)).astype(np.float32)
    kv = rng.standard_normal((8, L, 128)).astype(np.float32)
    head = (rng.standard_normal((V, H)) * 0.02).astype(np.float32)
    xh = rng.standard_normal((1, H)).astype(np.float32)
    threads = oracle.max_threads()

    def med(fn, n):
        ts = []
        for _ in range(n):
            t = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t)
        return sorted(ts)[len(ts) // 2]

    def lin():
        for (w, e), (n, k) in zip(ws, mats):
            qv, sv = xs[k]
            oracle.mxfp4_run(w, e, qv[None, :], sv[None, :], threads=threads)

    t_lin = med(lin, 7)
    t_att = med(lambda: oracle.attn_decode(q, kv, kv, 128 ** -0.5, threads=threads), 5)
    t_head = med(lambda: oracle.sgemm(xh, head, transb=True, threads=threads), 5)
    per_tok = 28 * (t_lin + t_att) + t_head
    return {"value": round(1.0 / per_tok, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": (f"one layer's 4 MXFP4 linears via mxfp4.Run (median of 7: {t_lin * 1e3:.2f} ms) and attention "
                       f"at 1152 keys (median of 5: {t_att * 1e3:.2f} ms), each x28, plus the fp32 head "
                       f"({t_head * 1e3:.2f} ms): {per_tok * 1e3:.1f} ms a token")}


def cpu_gemv_baseline(budget_s: float = 12.0):
    """The reference's CPU MXFP4 GEMV restated (oracle, test infrastructure): the int8-quantized
    activation and mxfp4.Run's 32-row spans over every host core, on one 8192 x 2048 GEMV."""
    import numpy as np

    from oracle import oracle

    rng = np.random.default_rng(0)
    w = rng.integers(0, 256, (GEMV_N, GEMV_K // 2), dtype=np.uint8)
    e = rng.integers(123, 130, (GEMV_N, GEMV_K // 32), dtype=np.uint8)
    x = rng.standard_normal(GEMV_K).astype(np.float16).astype(np.float32)
    threads = oracle.max_threads()
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t = time.perf_counter()
        q, s = oracle.vec_quantize(x)
        oracle.mxfp4_run(w, e, q[None, :], s[None, :], threads=threads)
        times.append(time.perf_counter() - t)
        if len(times) >= 200:
            break
    times.sort()
    med = times[len(times) // 2]
    return {"value": round(GEMV_BYTES / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{len(times)} MXFP4 GEMVs 8192x2048 (int8 activation, mxfp4.Run), median"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default="decode",
                    choices=["decode", "prefill", "gemv", "gemv_i8", "gemv_rows", "copy", "floor", "gemm", "attn",
                             "moe"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--eager", action="store_true", help="gemv/copy: launch one by one, no graph (counter runs)")
    ap.add_argument("--no-counters", action="store_true", help="decode: skip the rocprofv3 traffic runs")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(sharding is a design note, not a measured path)", file=sys.stderr)
        sys.exit(2)
    traffic, traffic_detail = None, {"skipped": True}
    if args.workload == "decode" and not args.no_counters:
        # the counter runs are child processes started before this process touches the GPU
        traffic, traffic_detail = measure_traffic()
    import torch

    torch.cuda.synchronize()
    if args.workload == "copy":
        r = copy_roofline(args.steps or 3200, 320 if args.warmup is None else args.warmup, args.eager)
        print(json.dumps({"workload": "copy", "bytes": GEMV_BYTES, "launches": r["launches"],
                          "us_per_launch": round(r["us"], 3), "gbs_read_plus_write": round(r["gbs"], 1)}))
        return
    if args.workload == "gemm":
        r = gemm_rate()
        r["roofline"] = {"bound": "mfma", "achieved": r["tflops"], "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": r["frac_mfma"]}
        r["cpu_baseline"] = None if args.no_cpu else gemm_cpu()
        print(json.dumps(r))
        return
    if args.workload == "attn":
        rows = [attn_rate(L, i8) for L in ATTN_LENS for i8 in (False, True)]
        cpu = None if args.no_cpu else [attn_cpu(L) for L in ATTN_LENS]
        print(json.dumps({"workload": "attn", "results": rows, "cpu_baseline": cpu}))
        return
    if args.workload == "moe":
        rows = [moe_rate(T) for T in (1, 5)]
        cpu = None if args.no_cpu else [moe_cpu(T) for T in (1, 5)]
        print(json.dumps({"workload": "moe", "results": rows, "cpu_baseline": cpu}))
        return
    if args.workload == "prefill":
        print(json.dumps(prefill_rate(args.steps or 5)))
        return
    if args.workload == "gemv_i8":
        print(json.dumps(dict(gemv_i8_rate(), workload="gemv_i8")))
        return
    if args.workload == "gemv_rows":
        print(json.dumps({"workload": "gemv_rows", "results": [gemv_rows_rate(T) for T in (1, 2, 4, 8)]}))
        return
    if args.workload == "floor":
        best, rows = read_floor()
        print(json.dumps({"workload": "floor", "bytes": GEMV_BYTES, "best": best, "sweep": rows}))
        return
    if args.workload == "gemv":
        r = gemv_roofline(args.steps or 3200, 320 if args.warmup is None else args.warmup, args.eager)
        print(json.dumps({"workload": "gemv", "launches": r["launches"], "us_per_launch": round(r["us"], 3),
                          "gbs": round(r["gbs"], 1), "frac": round(r["gbs"] / HBM_PEAK_GBS, 4)}))
        return
    steps = args.steps if args.steps is not None else 240
    warmup = args.warmup if args.warmup is not None else 16
    d = decode_rate(steps, warmup)
    g = gemv_roofline(3200, 320)
    floor, _ = read_floor(shapes=[(16, 1), (32, 1), (32, 2)])
    configs = {"c2_int8_gemm": gemm_rate(4),
               "c3_attention": [attn_rate(L, i8) for L in (2048, 32768) for i8 in (False, True)],
               "c4_moe": [moe_rate(T) for T in (1, 5)],
               "k2_i8_gemv": gemv_i8_rate(),
               "k1r_gemv_rows": [gemv_rows_rate(T) for T in (2, 8)]}
    cpu = None
    if not args.no_cpu:
        cpu = cpu_decode_baseline()
        cpu["cpu_model"], cpu["host_cores"] = host_cpu()
    out = {
        "metric": "decode tok/s at batch 1 (1 GPU); MXFP4 GEMV achieved HBM GB/s vs peak",
        "value": round(d["tok_s"], 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(d["ms_per_tok"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "mxfp4*fp16->f32",
        "data": "synthetic (seed-0 random-init weights and prompt ids drawn on the GPU)",
        "config": {"workload": "qwen3-shape 28-layer decoder, prompt 1024 then greedy decode at batch 1",
                   "layers": 28, "hidden": 2048, "heads": 16, "kv_heads": 8, "head_dim": 128, "ffn": 6144,
                   "vocab": 151936, "prompt": PROMPT, "decode_tokens": d["decode_tokens"],
                   "untimed_decode_steps": d["untimed"], "timed_positions": d["timed_positions"],
                   "weights": "MXFP4", "kv_cache": "fp16",
                   "step": "one HIP graph replay (graphs captured before timing)"},
        "prefill_tok_s": round(d["prefill_tok_s"], 1),
        "prefill_ms": round(d["prefill_ms"], 3),
        "decode_step_hbm": {"bytes_per_token": int(d["step_bytes"]),
                            "achieved_gbs": round(d["step_bytes"] / (d["ms_per_tok"] * 1e-3) / 1e9, 1),
                            "frac": round(d["step_bytes"] / (d["ms_per_tok"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
        "first_tokens": d["first_tokens"],
        "roofline": {"bound": "hbm", "achieved": round(g["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(g["gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_detail": traffic_detail,
                     "kernel": f"{GEMV_KERNEL} (MXFP4 GEMV 8192x2048, 64 distinct copies, graph)",
                     "us_per_launch": round(g["us"], 3), "bytes_per_launch": GEMV_BYTES,
                     "read_floor": dict(floor, frac=round(GEMV_BYTES / (floor["us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                                        gemv_over_floor=round(floor["us"] / g["us"], 4),
                                        kernel="hwk_read_floor: one launch reading the same bytes, no compute")},
        "cpu_baseline": cpu,
        "configs": configs,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
