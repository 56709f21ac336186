"""GPU parity of the decode attention (K4), the int8 KV rule and the merge, through libhwk's C
ABI, against the CPU oracle (the reference's chunk program + Merge, runner.attentionCPU's form).

Bar: max|o - o_oracle| <= 2e-3 * RMS(o_oracle) in fp32; fp16 output == RNE(fp32 output); int8
codes and scales bit-exact against the oracle's KV rule.
"""
import math

import numpy as np
import pytest
import torch

from hwnpu_amd import ops, synth

pytestmark = pytest.mark.gpu

TOL = 2e-3


def rms(a):
    return float(np.sqrt(np.mean(np.asarray(a, np.float64) ** 2)))


def check_close(got, want, tol=TOL):
    err = float(np.max(np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))))
    assert err <= tol * rms(want), f"max|d|={err:.4g} rms={rms(want):.4g} ratio={err / rms(want):.3g}"


def case(heads, kvh, L, cap, name):
    q = synth.normal(heads * 128, name + ".q").view(heads, 128)
    k = synth.normal(kvh * cap * 128, name + ".k").view(kvh, cap, 128)
    v = synth.normal(kvh * cap * 128, name + ".v").view(kvh, cap, 128)
    return q, k, v


@pytest.mark.parametrize("heads,kvh,L,cap", [
    (32, 8, 512, 512), (32, 8, 2048, 2048), (32, 8, 8192, 8192), (32, 8, 32768, 32768),  # the attention config
    (16, 8, 1152, 1280),  # the model's heads, a cache with room left
    (32, 8, 1, 16), (32, 8, 17, 40), (16, 8, 1000, 1000), (8, 8, 300, 333), (32, 8, 9000, 9000)])
def test_attn_decode_fp16(dev, orc, heads, kvh, L, cap):
    print(f"attn fp16 heads={heads} kv={kvh} L={L} cap={cap}", flush=True)
    q, k, v = case(heads, kvh, L, cap, f"c3.{heads}.{L}.{cap}")
    scale = 1 / math.sqrt(128)
    want = orc.attn_decode(q.cpu().numpy().astype(np.float32), k[:, :L].cpu().numpy().astype(np.float32),
                           v[:, :L].cpu().numpy().astype(np.float32), scale, chunk=8192)
    got = ops.attn_decode(q, k, v, L, out_mode="f32").cpu().numpy()
    check_close(got, want)
    g16 = ops.attn_decode(q, k, v, L, out_mode="f16").cpu().numpy()
    assert np.array_equal(g16.view(np.uint16), orc.f32_to_f16(got))


@pytest.mark.parametrize("split", [64, 192, 1024, 4096])
def test_attn_decode_splits_agree(dev, orc, split):
    q, k, v = case(32, 8, 3000, 3000, "c3.split")
    want = orc.attn_decode(q.cpu().numpy().astype(np.float32), k.cpu().numpy().astype(np.float32),
                           v.cpu().numpy().astype(np.float32), 1 / math.sqrt(128))
    got = ops.attn_decode(q, k, v, 3000, split=split).cpu().numpy()
    check_close(got, want)


def test_attn_workspace_reuse_and_graph(dev, orc):
    """One workspace across calls of several lengths (the chunk counters go back to zero after
    each call), then the same calls captured in a graph and replayed, each checked."""
    q, k, v = case(16, 8, 4000, 4000, "c3.reuse")
    p = ops.attn_params(16, 8, 4000, 4000)
    ws = ops.attn_workspace(p)
    lens = [4000, 37, 1153, 4000, 700]
    want = {L: orc.attn_decode(q.cpu().numpy().astype(np.float32), k[:, :L].cpu().numpy().astype(np.float32),
                               v[:, :L].cpu().numpy().astype(np.float32), 1 / math.sqrt(128)) for L in set(lens)}
    for L in lens:
        check_close(ops.attn_decode(q, k, v, L, workspace=ws).cpu().numpy(), want[L])
    outs = [torch.empty((16, 128), dtype=torch.float32, device="cuda") for _ in lens]
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for L, o in zip(lens, outs):
                ops.attn_decode(q, k, v, L, workspace=ws, out=o)
    torch.cuda.synchronize()
    for rep in range(3):
        for o in outs:
            o.zero_()
        g.replay()
        torch.cuda.synchronize()
        for L, o in zip(lens, outs):
            check_close(o.cpu().numpy(), want[L])


def test_kv_quantize_rule(dev, orc):
    x = synth.normal(777 * 128, "kvq.x").view(777, 128)
    x[5] = 0
    x[6, :7] = 0.0
    qd, sd = ops.kv_quantize_i8(x)
    qo, so = orc.i8_quantize_rows(x.cpu().numpy().astype(np.float32))
    assert np.array_equal(sd.cpu().numpy().view(np.uint16), so)
    assert np.array_equal(qd.cpu().numpy(), qo)


# 777, 5, 516 and 20: capacities whose last tile passes the last row (its loads clamped to it)
@pytest.mark.parametrize("heads,kvh,L", [(32, 8, 512), (32, 8, 2048), (32, 8, 8192), (32, 8, 32768), (16, 8, 777),
                                         (32, 8, 5), (32, 8, 516), (16, 8, 20)])
def test_attn_decode_int8(dev, orc, heads, kvh, L):
    print(f"attn int8 heads={heads} kv={kvh} L={L}", flush=True)
    q, k, v = case(heads, kvh, L, L, f"c3i8.{heads}.{L}")
    kq, ksc = ops.kv_quantize_i8(k)
    vq, vsc = ops.kv_quantize_i8(v)
    # the oracle attends over the dequantized cache, code * scale (exact in fp32)
    kd = kq.cpu().numpy().astype(np.float32) * ksc.cpu().numpy().astype(np.float32)[..., None]
    vd = vq.cpu().numpy().astype(np.float32) * vsc.cpu().numpy().astype(np.float32)[..., None]
    want = orc.attn_decode(q.cpu().numpy().astype(np.float32), kd, vd, 1 / math.sqrt(128))
    got = ops.attn_decode(q, kq, vq, L, k_scale=ksc, v_scale=vsc).cpu().numpy()
    check_close(got, want)


def test_attn_decode_empty_is_zero(dev):
    q, k, v = case(32, 8, 0, 16, "c3.empty")
    got = ops.attn_decode(q, k, v, 0).cpu().numpy()
    assert not np.any(got)


def test_attn_merge_kats(dev):
    """TestMergeOrder and TestMergeSink (internal/llm/paged/paged_test.go:133-186) on the GPU merge."""
    o = torch.tensor([[[1, 2]], [[3, 4]], [[5, 6]]], dtype=torch.float32, device="cuda")
    m = torch.tensor([[-1], [4], [2]], dtype=torch.float32, device="cuda")
    l = torch.tensor([[2], [1], [3]], dtype=torch.float32, device="cuda")
    w = [l[j, 0].item() * math.exp(m[j, 0].item() - 4) for j in range(3)]
    want = [sum(w[j] * o[j, 0, i].item() for j in range(3)) / sum(w) for i in range(2)]
    for order in ([0, 1, 2], [2, 1, 0], [1, 0, 2]):
        got = ops.attn_merge(o[order].contiguous(), m[order].contiguous(), l[order].contiguous()).cpu().numpy()[0]
        assert abs(got[0] - want[0]) <= 1e-5 and abs(got[1] - want[1]) <= 1e-5
    scores, vals, sink = [0.5, -1, 2], [[1, 2], [3, -1], [0.5, 4]], 1.5
    tot = sum(math.exp(s) for s in scores) + math.exp(sink)
    want = [sum(math.exp(s) / tot * v[j] for s, v in zip(scores, vals)) for j in range(2)]
    # the sink as a chunk of score `sink`, sum of exps 1 and output zero (Merge.AddSink)
    o = torch.tensor([[x] for x in vals] + [[[0, 0]]], dtype=torch.float32, device="cuda")
    m = torch.tensor([[s] for s in scores] + [[sink]], dtype=torch.float32, device="cuda")
    l = torch.ones((4, 1), dtype=torch.float32, device="cuda")
    got = ops.attn_merge(o, m, l).cpu().numpy()[0]
    assert abs(got[0] - want[0]) <= 1e-5 and abs(got[1] - want[1]) <= 1e-5


def test_attn_merge_vs_oracle(dev, orc):
    rng = np.random.default_rng(31)
    chunks, rows, dim = 7, 48, 128
    o = rng.standard_normal((chunks, rows, dim)).astype(np.float32)
    m = (rng.standard_normal((chunks, rows)) * 5).astype(np.float32)
    l = rng.uniform(0.5, 40, (chunks, rows)).astype(np.float32)
    l[2, :10] = 0  # rows whose keys were all masked in chunk 2: skipped
    mg = orc.Merge(rows, dim)
    for c in range(chunks):
        mg.add(o[c], m[c], l[c])
    want = mg.result()
    got = ops.attn_merge(*(torch.from_numpy(a).cuda() for a in (o, m, l))).cpu().numpy()
    assert np.max(np.abs(got - want)) <= 1e-5 * max(1.0, float(np.max(np.abs(want))))


def test_attn_merge_skipped_chunk_never_read(dev, orc):
    """A chunk whose l is not positive is skipped without reading its o (Merge.Add's `continue`,
    internal/llm/paged/paged.go:254-256): NaN and Inf there leave the result finite and equal to
    the merge of the other chunks."""
    rng = np.random.default_rng(5)
    chunks, rows, dim = 5, 16, 128
    o = rng.standard_normal((chunks, rows, dim)).astype(np.float32)
    m = (rng.standard_normal((chunks, rows)) * 3).astype(np.float32)
    l = rng.uniform(0.5, 20, (chunks, rows)).astype(np.float32)
    l[1, :] = 0.0
    l[3, ::2] = -1.0
    o[1] = np.nan
    o[3, ::2] = np.inf
    m[1] = 50.0  # a skipped chunk's m does not set the top either
    mg = orc.Merge(rows, dim)
    for c in range(chunks):
        mg.add(np.where(l[c][:, None] > 0, o[c], 0.0).astype(np.float32), m[c], l[c])
    want = mg.result()
    got = ops.attn_merge(*(torch.from_numpy(a).cuda() for a in (o, m, l))).cpu().numpy()
    assert np.all(np.isfinite(got))
    assert np.max(np.abs(got - want)) <= 1e-5 * max(1.0, float(np.max(np.abs(want))))


def oracle_prefill(orc, q, k, v, start, scale):
    """The reference's chunk program over the whole cache with the causal mask (0 / -1e4), as the
    session runs a prompt (one chunk: every case here is under DefaultChunk = 8192 keys)."""
    T, H, d = q.shape
    kvh = k.shape[0]
    L = start + T
    mask = np.where(np.arange(L)[None, :] <= start + np.arange(T)[:, None], 0.0, -1e4).astype(np.float32)
    qh = np.ascontiguousarray(q.transpose(1, 0, 2))  # (heads, tokens, d)
    o, m, l = orc.paged_chunk(qh, k[:, :L], v[:, :L], mask, scale)
    return o.transpose(1, 0, 2)


# three key groups past 256 keys (the first and the last two), two past 128, one below
@pytest.mark.parametrize("heads,kvh,T,start,cap", [
    (16, 8, 1024, 0, 1280),  # the model's prompt
    (32, 8, 200, 0, 256), (16, 8, 37, 100, 160), (8, 8, 70, 5, 80), (16, 16, 1, 0, 8), (16, 8, 33, 31, 64),
    (32, 8, 300, 0, 320), (8, 8, 250, 10, 288)])
def test_attn_prefill_causal(dev, orc, heads, kvh, T, start, cap):
    print(f"attn prefill heads={heads} kv={kvh} T={T} start={start} cap={cap}", flush=True)
    name = f"c3p.{heads}.{T}.{start}"
    q = synth.normal(T * heads * 128, name + ".q").view(T, heads, 128)
    k = synth.normal(kvh * cap * 128, name + ".k").view(kvh, cap, 128)
    v = synth.normal(kvh * cap * 128, name + ".v").view(kvh, cap, 128)
    scale = 1 / math.sqrt(128)
    want = oracle_prefill(orc, q.cpu().numpy().astype(np.float32), k.cpu().numpy().astype(np.float32),
                          v.cpu().numpy().astype(np.float32), start, scale)
    got = ops.attn_prefill(q, k, v, start, out_mode="f32").cpu().numpy()
    for t in range(T):  # every row against its own scale
        check_close(got[t], want[t])
    g16 = ops.attn_prefill(q, k, v, start, out_mode="f16").cpu().numpy()
    assert np.array_equal(g16.view(np.uint16), orc.f32_to_f16(got))
    # the last row equals decode attention at that position
    dec = ops.attn_decode(q[T - 1].contiguous(), k, v, start + T).cpu().numpy()
    check_close(got[T - 1], dec)
