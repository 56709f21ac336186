"""GPU parity of the decoder's small ops (K6) through libhwk's C ABI against the CPU oracle, on the
same seeded inputs.

The bar: copies, gathers and the argmax bit-exact; the float ops equal to the oracle bit for bit
except where the two sides' float64 library calls (sqrt of a float64 sum taken in another order,
exp) may land on either side of a float32 rounding boundary: there at most 1 ulp, in a small
fraction of the values.
"""
import numpy as np
import pytest
import torch

from hwnpu_amd import ops, synth

pytestmark = pytest.mark.gpu

EPS = float(np.float32(1e-6))  # a float32 value, so the oracle's float eps is the same number


def ulps(a, b):
    a = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.ascontiguousarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(a - b)


def near_exact(got, want, frac=1e-3):
    d = ulps(got, want)
    assert d.max() <= 1, f"max ulp difference {d.max()}"
    assert (d > 0).mean() <= frac, f"{(d > 0).mean():.4g} of values differ"


@pytest.mark.parametrize("rows,n", [(1, 2048), (7, 2048), (3, 6144), (5, 1), (2, 300), (64, 128)])
def test_rmsnorm(dev, orc, rows, n):
    print(f"rmsnorm rows={rows} n={n}", flush=True)
    x = synth.normal(rows * n, f"k6.rms.{rows}.{n}", dtype=torch.float32).view(rows, n)
    x *= torch.arange(1, rows + 1, device="cuda", dtype=torch.float32)[:, None] ** 3
    w = synth.normal(n, f"k6.rms.w.{n}", dtype=torch.float32) + 1.0
    want = orc.rmsnorm(x.cpu().numpy(), w.cpu().numpy(), EPS)
    got32 = ops.rmsnorm(x, w, EPS, "f32").cpu().numpy()
    near_exact(got32, want)
    got16 = ops.rmsnorm(x, w, EPS, "f16").cpu().numpy()
    assert np.array_equal(got16.view(np.uint16), orc.f32_to_f16(got32))
    # invariant: with unit weights each output row has RMS sqrt(ms / (ms + eps)) ~ 1
    ones = torch.ones(n, device="cuda")
    r = ops.rmsnorm(x, ones, EPS, "f32").cpu().numpy().astype(np.float64)
    assert np.allclose(np.sqrt((r ** 2).mean(axis=1)), 1.0, atol=1e-4)


def test_rmsnorm_zero_row(dev):
    x = torch.zeros((2, 256), device="cuda")
    w = torch.ones(256, device="cuda")
    assert torch.count_nonzero(ops.rmsnorm(x, w, EPS, "f32")) == 0


@pytest.mark.parametrize("T,heads,pos0,norm", [(1, 16, 0, True), (1, 8, 1000, True), (5, 16, 37, False),
                                               (3, 24, 4090, True)])
def test_rope(dev, orc, T, heads, pos0, norm):
    print(f"rope T={T} heads={heads} pos0={pos0} norm={norm}", flush=True)
    P = 4096 + 8
    c, s = ops.rope_tables(1e6, 0, P)
    x = synth.normal(T * heads * 128, f"k6.rope.{T}.{heads}", dtype=torch.float32).view(T, heads, 128) * 3
    w = synth.normal(128, "k6.rope.w", dtype=torch.float32) + 1.0
    got = ops.rope(x, c, s, pos0, w if norm else None, EPS, "f32").cpu().numpy()
    oc, os_ = orc.rope_tables(1e6, 0, P, 128)
    xs = x.cpu().numpy()
    for t in range(T):
        v = orc.rmsnorm(xs[t], w.cpu().numpy(), EPS) if norm else xs[t]
        want = orc.apply_rope(v, oc[pos0 + t], os_[pos0 + t])
        if norm:
            near_exact(got[t], want, frac=0.02)
        else:
            assert np.array_equal(got[t], want)  # no float64 step: bit-exact
    g16 = ops.rope(x, c, s, pos0, w if norm else None, EPS, "f16").cpu().numpy()
    assert np.array_equal(g16.view(np.uint16), orc.f32_to_f16(got))
    # a rotation keeps each (j, j+64) pair's length
    src = orc.rmsnorm(xs, w.cpu().numpy(), EPS) if norm else xs
    a = np.hypot(got[..., :64].astype(np.float64), got[..., 64:])
    b = np.hypot(src[..., :64].astype(np.float64), src[..., 64:])
    assert np.allclose(a, b, rtol=1e-5, atol=1e-6)


def test_rope_position_zero_is_identity(dev):
    c, s = ops.rope_tables(1e6, 0, 4)
    x = synth.normal(2 * 128, "k6.rope0", dtype=torch.float32).view(1, 2, 128)
    assert torch.equal(ops.rope(x, c, s, 0, None, EPS, "f32"), x)


def test_kv_append(dev):
    kvh, cap, T, pos0 = 8, 64, 5, 17
    kc = synth.normal(kvh * cap * 128, "k6.kc").view(kvh, cap, 128)
    vc = synth.normal(kvh * cap * 128, "k6.vc").view(kvh, cap, 128)
    k = synth.normal(T * kvh * 128, "k6.k").view(T, kvh, 128)
    v = synth.normal(T * kvh * 128, "k6.v").view(T, kvh, 128)
    wk, wv = kc.clone(), vc.clone()
    wk[:, pos0:pos0 + T] = k.transpose(0, 1)
    wv[:, pos0:pos0 + T] = v.transpose(0, 1)
    ops.kv_append(k, v, kc, vc, pos0)
    assert torch.equal(kc, wk) and torch.equal(vc, wv)
    ops.kv_append(k[:0], v[:0], kc, vc, cap)  # nothing to write at the end of the cache
    assert torch.equal(kc, wk)


@pytest.mark.parametrize("n", [1, 1000, 6144, 5 * 6144])
def test_silu_mul(dev, orc, n):
    g = synth.normal(n, f"k6.g.{n}", dtype=torch.float32) * 4
    u = synth.normal(n, f"k6.u.{n}", dtype=torch.float32)
    want = orc.silu_mul(g.cpu().numpy(), u.cpu().numpy())
    got = ops.silu_mul(g, u, "f32").cpu().numpy()
    near_exact(got, want, frac=0.01)
    got16 = ops.silu_mul(g, u, "f16").cpu().numpy()
    assert np.array_equal(got16.view(np.uint16), orc.f32_to_f16(got))
    # interleaved gate/up (gate at even, up at odd), as the fused gate_up rows are stored
    gu = torch.stack([g, u], dim=1).reshape(-1).contiguous()
    inter = ops.silu_mul(gu, gu[1:], "f32", stride=2, n=n).cpu().numpy()
    assert np.array_equal(inter, got)


def test_silu_mul_special_values(dev, orc):
    g = torch.tensor([0.0, -0.0, 1e-30, -100.0, 100.0, 88.0, -88.0, float("inf")], device="cuda")
    u = torch.ones_like(g)
    got = ops.silu_mul(g, u, "f32").cpu().numpy()
    want = orc.silu_mul(g.cpu().numpy(), u.cpu().numpy())
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    assert np.array_equal(got[fin], want[fin])


def test_add(dev):
    y = synth.normal(100003, "k6.y", dtype=torch.float32)
    x = synth.normal(100003, "k6.x", dtype=torch.float32)
    want = y.cpu().numpy() + x.cpu().numpy()
    ops.add_(y, x)
    assert np.array_equal(y.cpu().numpy(), want)


def test_embed(dev):
    vocab, hidden = 1000, 2048
    table = synth.normal(vocab * hidden, "k6.emb").view(vocab, hidden)
    ids = torch.tensor([0, 999, 5, 5, 123], dtype=torch.int32, device="cuda")
    got = ops.embed(table, ids).cpu().numpy()
    want = table.cpu().numpy()[ids.cpu().numpy()].astype(np.float32)
    assert np.array_equal(got, want)
    bad = ops.embed(table, torch.tensor([3, -1, 1000], dtype=torch.int32, device="cuda")).cpu().numpy()
    assert np.array_equal(bad[0], table.cpu().numpy()[3].astype(np.float32))
    assert np.isnan(bad[1]).all() and np.isnan(bad[2]).all()


@pytest.mark.parametrize("rows,n", [(1, 151936), (5, 151936), (3, 1), (2, 7), (4, 300), (1, 65)])
def test_argmax(dev, orc, rows, n):
    x = synth.normal(rows * n, f"k6.arg.{rows}.{n}", dtype=torch.float32).view(rows, n)
    got = ops.argmax(x).cpu().numpy()
    xs = x.cpu().numpy()
    assert [orc.argmax(xs[r]) for r in range(rows)] == got.tolist()


def test_argmax_ties_and_specials(dev, orc):
    n = 151936
    rows = []
    r = np.zeros(n, np.float32)
    r[[70000, 5, 150000]] = 3.0  # ties: the lowest index
    rows.append(r)
    rows.append(np.full(n, -np.inf, np.float32))  # all -inf: index 0
    r = np.random.default_rng(1).standard_normal(n).astype(np.float32)
    r[0] = np.nan  # NaN at index 0 is kept, as strict > never replaces it
    rows.append(r)
    r = np.random.default_rng(2).standard_normal(n).astype(np.float32)
    r[[3, 90000]] = np.nan  # NaNs elsewhere never win
    r[100] = 9.0
    rows.append(r)
    r = np.zeros(n, np.float32)
    r[n - 1] = 1e-45  # the largest is the last, a subnormal
    rows.append(r)
    x = np.stack(rows)
    got = ops.argmax(torch.from_numpy(x).cuda()).cpu().numpy().tolist()
    assert got == [orc.argmax(row) for row in rows] == [5, 0, 0, 100, n - 1]
