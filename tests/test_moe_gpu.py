"""GPU parity of the MoE path (K5) through libhwk's C ABI against the CPU oracle.

Routing: expert indices bit-exact against the oracle's restatement of Routing.Choose, weights
equal to within one float32 ulp (the device's float64 exp may differ from glibc's in the last
place). Experts: fp32 output within max|d| <= 2e-3 * RMS against the dequantized fp32 experts
(the reference Host.Run's structure with fp32 activations), on the MoE configuration: hidden 2048,
32 experts, top-4, intermediate 768, T in {1, 5}.
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


def ulp_diff(a, b):
    return np.abs(a.view(np.int32).astype(np.int64) - b.view(np.int32).astype(np.int64))


@pytest.mark.parametrize("E,k", [(32, 4), (64, 8), (8, 2), (32, 1)])
def test_route_softmax_bit_exact(dev, orc, E, k):
    rows = 4096
    logits = synth.normal(rows * E, f"route.{E}.{k}", dtype=torch.float32).view(rows, E)
    lg = logits.cpu().numpy()
    # planted exact ties: equal logits must go to the lower index
    lg[:64, 3] = lg[:64, 7]
    lg[64:128, :] = 0.5
    logits.copy_(torch.from_numpy(lg))
    idx, w = ops.moe_route(logits, k)
    idx, w = idx.cpu().numpy(), w.cpu().numpy()
    for r in range(rows):
        oi, ow = orc.choose(lg[r], k)
        assert np.array_equal(idx[r], oi), (r, idx[r], oi)
        assert np.all(ulp_diff(w[r], ow) <= 1), (r, w[r], ow)
    assert np.array_equal(idx[64], np.arange(k))


def test_route_sigmoid_bias_kat(dev):
    """TestChooseSigmoidBias (internal/llm/experts/weights_test.go:11-26)."""
    logits = torch.tensor([[2, 1, 0, -1]], dtype=torch.float32, device="cuda")
    bias = torch.tensor([0, 0, 3, 0], dtype=torch.float32, device="cuda")
    idx, w = ops.moe_route(logits, 2, score="sigmoid", norm=True, bias=bias)
    assert idx.cpu().tolist() == [[2, 0]]
    sig = lambda x: 1 / (1 + math.exp(-x))
    s2, s0 = sig(0), sig(2)
    got = w.cpu().numpy()[0]
    assert abs(got[0] - s2 / (s2 + s0)) <= 1e-5 and abs(got[1] - s0 / (s2 + s0)) <= 1e-5


def test_route_scale_and_no_norm(dev, orc):
    logits = synth.normal(64 * 16, "route.scale", dtype=torch.float32).view(64, 16)
    idx, w = ops.moe_route(logits, 3, norm=False, scale=2.5)
    lg = logits.cpu().numpy()
    for r in range(64):
        oi, ow = orc.choose(lg[r], 3, norm=False, scale=2.5)
        assert np.array_equal(idx.cpu().numpy()[r], oi)
        assert np.all(ulp_diff(w.cpu().numpy()[r], ow) <= 1)


def experts_case(T, E=32, H=2048, I=768, name="c4"):
    gw, ge = synth.mxfp4_uniform(E * 2 * I, H, name + ".gate_up")
    dw, de = synth.mxfp4_uniform(E * H, I, name + ".down")
    gw, ge = gw.view(E, 2 * I, H // 32, 16), ge.view(E, 2 * I, H // 32)
    dw, de = dw.view(E, H, I // 32, 16), de.view(E, H, I // 32)
    x = synth.normal(T * H, name + f".x{T}").view(T, H)
    logits = synth.normal(T * E, name + f".logits{T}", dtype=torch.float32).view(T, E)
    return x, logits, gw, ge, dw, de


@pytest.mark.parametrize("T", [1, 5, 2, 8])
def test_experts_parity(dev, orc, T):
    print(f"moe experts T={T}", flush=True)
    x, logits, gw, ge, dw, de = experts_case(T)
    idx, w = ops.moe_route(logits, 4)
    out = ops.moe_experts(x, idx, w, gw, ge, dw, de)
    want = orc.experts(x.cpu().numpy().astype(np.float32), idx.cpu().numpy(), w.cpu().numpy(), gw.cpu().numpy(),
                       ge.cpu().numpy(), dw.cpu().numpy(), de.cpu().numpy())
    check_close(out.cpu().numpy(), want)
    # add mode adds the same sums into out
    base = synth.normal(T * 2048, "c4.base", std=1000.0, dtype=torch.float32).view(T, 2048)
    b0 = base.cpu().numpy()
    ops.moe_experts(x, idx, w, gw, ge, dw, de, out=base, out_mode="add")
    check_close(base.cpu().numpy(), want + b0)


def test_experts_small_shapes(dev, orc):
    """Other widths: H=256 (8 of 64 lanes' blocks), I=96 (3 blocks a row), E=6, k=2, tokens sharing
    experts."""
    T, E, H, I = 3, 6, 256, 96
    x, logits, gw, ge, dw, de = experts_case(T, E, H, I, name="c4s")
    idx = torch.tensor([[4, 1], [1, 2], [0, 4]], dtype=torch.int32, device="cuda")
    w = torch.tensor([[0.7, 0.3], [0.5, 0.5], [0.2, 0.8]], dtype=torch.float32, device="cuda")
    out = ops.moe_experts(x, idx, w, gw, ge, dw, de)
    want = orc.experts(x.cpu().numpy().astype(np.float32), idx.cpu().numpy(), w.cpu().numpy(), gw.cpu().numpy(),
                       ge.cpu().numpy(), dw.cpu().numpy(), de.cpu().numpy())
    check_close(out.cpu().numpy(), want)


def _np(*ts):
    return [t.cpu().numpy() for t in ts]


@pytest.mark.parametrize("T", [1, 2, 5, 8])
def test_moe_layer_route_folded(dev, orc, T):
    """hwk_moe_layer (route folded into the gate_up launch up to 2 tokens, a route launch past that):
    idx bit-exact to the oracle's Choose, w within one ulp, the output as hwk_moe_experts' on the
    same choice (and the oracle's)."""
    print(f"moe layer T={T}", flush=True)
    x, logits, gw, ge, dw, de = experts_case(T)
    out, idx, w = ops.moe_layer(x, logits, 4, gw, ge, dw, de)
    lg = logits.cpu().numpy()
    ii, ww = idx.cpu().numpy(), w.cpu().numpy()
    for t in range(T):
        oi, ow = orc.choose(lg[t], 4)
        assert np.array_equal(ii[t], oi), (t, ii[t], oi)
        assert np.all(ulp_diff(ww[t], ow) <= 1)
    want = orc.experts(x.cpu().numpy().astype(np.float32), ii, ww, *_np(gw, ge, dw, de))
    check_close(out.cpu().numpy(), want)
    same = ops.moe_experts(x, idx, w, gw, ge, dw, de)
    check_close(out.cpu().numpy(), same.cpu().numpy(), tol=1e-6)


@pytest.mark.parametrize("T,row", [(1, 0), (5, 3)])
def test_moe_layer_score_collision(dev, orc, T, row):
    """A float32 score collision at the top-k boundary: token `row` has three clear leaders and, for
    the fourth place, expert 5 (logit 0.5) against expert 7 (the next float32 above 0.5): relative to
    the maximum 9 both differences round to -8.5, their scores are equal, and Choose's stable order
    takes the lower index 5 where an order by logit would take 7. The layer (the route folded into
    gate_up at T = 1, a route launch at T = 5) must use expert 5: idx bit-exact, output as the
    oracle's."""
    x, logits, gw, ge, dw, de = experts_case(T)
    lg = logits.cpu().numpy()
    lg[row, :] = -5.0
    lg[row, :3] = [9.0, 8.5, 8.0]
    lg[row, 5] = 0.5
    lg[row, 7] = np.nextafter(np.float32(0.5), np.float32(1.0))
    assert lg[row, 7] > lg[row, 5] and np.float32(lg[row, 7] - 9.0) == np.float32(lg[row, 5] - 9.0)
    logits.copy_(torch.from_numpy(lg))
    oi, _ = orc.choose(lg[row], 4)
    assert list(oi) == [0, 1, 2, 5]
    out, idx, w = ops.moe_layer(x, logits, 4, gw, ge, dw, de)
    ii, ww = idx.cpu().numpy(), w.cpu().numpy()
    for t in range(T):
        oi, ow = orc.choose(lg[t], 4)
        assert np.array_equal(ii[t], oi), (t, ii[t], oi)
        assert np.all(ulp_diff(ww[t], ow) <= 1)
    want = orc.experts(x.cpu().numpy().astype(np.float32), ii, ww, *_np(gw, ge, dw, de))
    check_close(out.cpu().numpy(), want)


@pytest.mark.parametrize("T,case", [(1, "gap"), (2, "gap"), (1, "far"), (2, "clear")])
def test_moe_layer_route_near_ties(dev, orc, T, case):
    """The folded route reads the choice off the logits when the differences logit - max of the
    first k+1 ranks are at least 2^-20 apart (and the k-th at least -80), else runs Choose first.
    "gap": the 4th and 5th differ by 2^-21 (float32 spacing near -4; Choose's scores still differ),
    "far": the 4th chosen at -95 (a denormal score), "clear": 2^-20 apart (near -8.5), taken from
    the logits. Each must give Choose's idx bit for bit and the oracle's output."""
    x, logits, gw, ge, dw, de = experts_case(T)
    lg = logits.cpu().numpy()
    lg[0, :] = -5.0 if case != "far" else -300.0
    if case == "gap":
        lg[0, :3] = [9.0, 8.5, 8.0]
        lg[0, 5] = 5.0
        lg[0, 7] = np.nextafter(np.float32(5.0), np.float32(6.0))
        assert np.float32(lg[0, 7] - 9.0) - np.float32(lg[0, 5] - 9.0) == np.float32(2.0 ** -21)
    elif case == "far":
        lg[0, :4] = [0.0, -85.0, -90.0, -95.0]
    else:
        lg[0, :3] = [9.0, 8.5, 8.0]
        lg[0, 5] = 0.5
        lg[0, 7] = np.float32(0.5) + np.float32(2.0 ** -20)
        assert np.float32(lg[0, 7] - 9.0) - np.float32(lg[0, 5] - 9.0) == np.float32(2.0 ** -20)
    logits.copy_(torch.from_numpy(lg))
    out, idx, w = ops.moe_layer(x, logits, 4, gw, ge, dw, de)
    ii, ww = idx.cpu().numpy(), w.cpu().numpy()
    for t in range(T):
        oi, ow = orc.choose(lg[t], 4)
        assert np.array_equal(ii[t], oi), (t, ii[t], oi)
        assert np.all(ulp_diff(ww[t], ow) <= 1)
    want = orc.experts(x.cpu().numpy().astype(np.float32), ii, ww, *_np(gw, ge, dw, de))
    check_close(out.cpu().numpy(), want)


@pytest.mark.parametrize("T,exp_hi", [(1, False), (5, False), (3, True)])
def test_experts_gptoss_biases(dev, orc, T, exp_hi):
    """The gpt-oss gated unit (alpha 1.702, limit 7) with gate/up and down biases (host.go:44-57,
    505-527, 566-578), as gpt-oss's checkpoints run it; exp_hi: gate/up scales past the limit, so
    that the clamps are taken."""
    E, H, I = 32, 2048, 768
    x, logits, gw, ge, dw, de = experts_case(T, E, H, I, name="c4g")
    if exp_hi:
        ge = (ge % 4 + 126).to(torch.uint8)
    gb = synth.normal(E * 2 * I, "c4g.gu_bias", std=0.1, dtype=torch.float32).view(E, 2 * I)
    db = synth.normal(E * H, "c4g.dn_bias", std=0.1, dtype=torch.float32).view(E, H)
    kw = dict(gu_b=gb, dn_b=db, act="gptoss", alpha=1.702, limit=7.0)
    out, idx, w = ops.moe_layer(x, logits, 4, gw, ge, dw, de, **kw)
    want = orc.experts(x.cpu().numpy().astype(np.float32), *_np(idx, w, gw, ge, dw, de), gu_b=gb.cpu().numpy(),
                       dn_b=db.cpu().numpy(), act="gptoss", alpha=1.702, limit=7.0)
    check_close(out.cpu().numpy(), want)
    # SiLU with the biases through hwk_moe_experts, add mode
    base = synth.normal(T * H, "c4g.base", std=10.0, dtype=torch.float32).view(T, H)
    b0 = base.cpu().numpy()
    ops.moe_experts(x, idx, w, gw, ge, dw, de, out=base, out_mode="add", gu_b=gb, dn_b=db)
    want2 = orc.experts(x.cpu().numpy().astype(np.float32), *_np(idx, w, gw, ge, dw, de), gu_b=gb.cpu().numpy(),
                        dn_b=db.cpu().numpy())
    check_close(base.cpu().numpy(), want2 + b0)


def test_moe_layer_small_shapes_sigmoid(dev, orc):
    """E=6, k=2, H=256, I=96, sigmoid routing with a router bias and a weight scale."""
    T, E, H, I = 3, 6, 256, 96
    x, logits, gw, ge, dw, de = experts_case(T, E, H, I, name="c4t")
    rb = torch.tensor([0, 0.5, 0, 0, 1.0, 0], dtype=torch.float32, device="cuda")
    out, idx, w = ops.moe_layer(x, logits, 2, gw, ge, dw, de, score="sigmoid", norm=True, scale=2.5,
                                router_bias=rb)
    lg = logits.cpu().numpy()
    for t in range(T):
        oi, ow = orc.choose(lg[t], 2, score="sigmoid", norm=True, scale=2.5, bias=rb.cpu().numpy())
        assert np.array_equal(idx.cpu().numpy()[t], oi)
        assert np.all(ulp_diff(w.cpu().numpy()[t], ow) <= 1)
    want = orc.experts(x.cpu().numpy().astype(np.float32), *_np(idx, w, gw, ge, dw, de))
    check_close(out.cpu().numpy(), want)
