"""GPU parity of the prefill/verify GEMM (K3) through libhwk's C ABI against the oracle's
dequantize + blocked fp32 GEMM (the reference's shiftScale/Dequantize + sgemm.MulAdd).

Bar: max|Y - Y_oracle| <= 2e-3 * RMS(Y_oracle) in fp32; the fp16 output equal to RNE of the fp32
accumulator, bit for bit.
"""
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


# (512, 6144, 2048) and (500, 6000, 2080) take the 128 x 96 tile of two k groups (the latter with a
# ragged last step and partial edge tiles); the others the one-group tiles
@pytest.mark.parametrize("m,n,k", [(512, 6144, 2048), (5, 6144, 2048), (1, 128, 32), (130, 200, 96), (7, 1000, 4096),
                                   (256, 256, 6144), (300, 130, 2880), (500, 6000, 2080)])
def test_i8_gemm_parity(dev, orc, m, n, k):
    print(f"i8_gemm m={m} n={n} k={k}", flush=True)
    name = f"k3i8.{m}.{n}.{k}"
    x = synth.normal(m * k, name + ".x").view(m, k)
    q = synth.uniform_int(n * k, -127, 255, name + ".q", dtype=torch.int8).view(n, k)
    s = synth.uniform_real(n, 0.002, 0.02, name + ".s")
    wd = orc.i8_dequant(q.cpu().numpy(), s.cpu().numpy().view(np.uint16))
    want = orc.sgemm(x.cpu().numpy().astype(np.float32), wd, transb=True)
    y32 = ops.i8_gemm(x, q, s, "f32").cpu().numpy()
    check_close(y32, want)
    y16 = ops.i8_gemm(x, q, s, "f16").cpu().numpy()
    assert np.array_equal(y16.view(np.uint16), orc.f32_to_f16(y32))


# (1024, 2048, 6144) and (1024, 2048, 2048) are the prompt's down and o_proj shapes, (260, 1000, 4096)
# their tile with ragged rows and columns
@pytest.mark.parametrize("m,n,k", [(1024, 4096, 2048), (5, 2048, 6144), (1, 96, 64), (200, 12288, 2048), (33, 130, 32),
                                   (1024, 2048, 6144), (260, 1000, 4096), (1024, 2048, 2048)])
def test_mxfp4_gemm_parity(dev, orc, m, n, k):
    print(f"mxfp4_gemm m={m} n={n} k={k}", flush=True)
    name = f"k3mx.{m}.{n}.{k}"
    x = synth.normal(m * k, name + ".x").view(m, k)
    w, e = synth.mxfp4_normal(n, k, name + ".w", std=0.02)
    wd = orc.mxfp4_dequantize(w.cpu().numpy(), e.cpu().numpy())
    want = orc.sgemm(x.cpu().numpy().astype(np.float32), wd, transb=True)
    y32 = ops.mxfp4_gemm(x, w, e, "f32").cpu().numpy()
    check_close(y32, want)
    y16 = ops.mxfp4_gemm(x, w, e, "f16").cpu().numpy()
    assert np.array_equal(y16.view(np.uint16), orc.f32_to_f16(y32))
    # add mode
    y0 = synth.normal(m * n, name + ".y0", dtype=torch.float32).view(m, n)
    b0 = y0.cpu().numpy()
    ops.mxfp4_gemm(x, w, e, "add", y=y0)
    assert np.array_equal(y0.cpu().numpy(), (b0 + y32).astype(np.float32))


def test_mxfp4_gemm_uniform_codes(dev, orc):
    """The GEMV configuration's weights (every code, exponents -4..2) through the GEMM at m = 5."""
    m, n, k = 5, 8192, 2048
    x = synth.normal(m * k, "k3u.x").view(m, k)
    w, e = synth.mxfp4_uniform(n, k, "k3u.w")
    wd = orc.mxfp4_dequantize(w.cpu().numpy(), e.cpu().numpy())
    want = orc.sgemm(x.cpu().numpy().astype(np.float32), wd, transb=True)
    check_close(ops.mxfp4_gemm(x, w, e, "f32").cpu().numpy(), want)


def test_mxfp4_gemm_edge_exponents(dev, orc):
    """Block exponents outside [-23, 13], where a code times its scale is no fp16 value: rows whose
    scales reach 2^20 (6 * 2^20 overflows fp16) or fall to 2^-40, rows spanning 36 and 50 exponents,
    zero scales (e = 0) among normal ones. Each output column (one weight row) is checked against the
    oracle's fp32 Dequantize + sgemm relative to its own size."""
    m, n, k = 33, 96, 256
    rng = np.random.default_rng(11)
    x = synth.normal(m * k, "k3edge.x").view(m, k)
    w = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    e = np.empty((n, k // 32), np.int64)
    nb = k // 32
    e[0:16] = rng.integers(127 + 10, 127 + 21, (16, nb))   # scales up to 2^20
    e[16:32] = rng.integers(127 - 40, 127 - 29, (16, nb))  # down to 2^-40
    e[32:48] = rng.integers(127 - 21, 127 + 16, (16, nb))  # a span of 36
    e[48:64] = rng.integers(127 - 4, 127 + 3, (16, nb))    # the usual range
    e[64:80] = rng.integers(127 - 4, 127 + 3, (16, nb))
    e[64:80, ::3] = 0                                       # zero scales among them
    e[80:96] = rng.integers(127 - 4, 127 + 3, (16, nb))
    e[80:96, 0] = 127 + 20                                  # a span of 50: the 2^-30 blocks lose
    e[80:96, 1] = 127 - 30                                  # bits below 2^-24 of the shifted scale
    e = e.astype(np.uint8)
    wd = orc.mxfp4_dequantize(w, e)
    want = orc.sgemm(x.cpu().numpy().astype(np.float32), wd, transb=True)
    got = ops.mxfp4_gemm(x, torch.from_numpy(w).cuda(), torch.from_numpy(e).cuda(), "f32").cpu().numpy()
    assert np.all(np.isfinite(got))
    for j in range(n):
        col_rms = rms(want[:, j])
        err = float(np.max(np.abs(got[:, j].astype(np.float64) - want[:, j])))
        assert err <= TOL * col_rms, f"column {j}: max|d|={err:.4g} rms={col_rms:.4g}"


@pytest.mark.parametrize("kind,m,n,k", [("mx", 1024, 3072, 2048), ("mx", 33, 96, 256), ("mx", 5, 512, 6144),
                                        ("i8", 200, 1536, 2048), ("i8", 7, 32, 96), ("i8", 512, 6144, 2048)])
def test_gemm_swiglu_output(dev, kind, m, n, k):
    """out_mode "swiglu" (the prompt's gate/up projection with its SwiGLU in the epilogue) equals the
    fp32 output followed by hwk_silu_mul over the column pairs (g, u) = (2c, 2c+1), bit for bit; both
    of those are pinned to the oracle on their own (the parity tests above, test_glue_gpu)."""
    print(f"gemm swiglu {kind} m={m} n={n} k={k}", flush=True)
    name = f"k3sw.{kind}.{m}.{n}.{k}"
    x = synth.normal(m * k, name + ".x").view(m, k)
    if kind == "mx":
        w, e = synth.mxfp4_normal(n, k, name + ".w", std=0.02)
        run = lambda mode: ops.mxfp4_gemm(x, w, e, mode)  # noqa: E731
    else:
        q = synth.uniform_int(n * k, -127, 255, name + ".q", dtype=torch.int8).view(n, k)
        s = synth.uniform_real(n, 0.002, 0.02, name + ".s")
        run = lambda mode: ops.i8_gemm(x, q, s, mode)  # noqa: E731
    y32 = run("f32")
    flat = y32.view(-1)
    want = ops.silu_mul(flat, flat[1:], "f16", stride=2, n=m * n // 2).view(m, n // 2)
    got = run("swiglu")
    assert got.shape == (m, n // 2) and got.dtype == torch.float16
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_gemm_swiglu_rejects_ragged_n(dev):
    x = synth.normal(4 * 64, "k3swr.x").view(4, 64)
    w, e = synth.mxfp4_normal(24, 64, "k3swr.w", std=0.02)
    with pytest.raises(Exception, match="SwiGLU"):
        ops.mxfp4_gemm(x, w, e, "swiglu")
