"""GPU parity of the weight GEMVs and the synthetic inputs, through libhwk's C ABI, against the CPU
oracle on the same seeded inputs.

The bar: dequantized weights bit-exact; GEMV outputs within
max|y - y_oracle| <= 2e-3 * RMS(y_oracle) in fp32; the fp16 output equal to RNE of the fp32
accumulator, bit for bit; the synthetic draws equal to their host restatement.
"""
import numpy as np
import pytest
import torch

import synth_np
from hwnpu_amd import ops, synth

pytestmark = pytest.mark.gpu

TOL = 2e-3  # max-abs error relative to the oracle output's RMS


def rms(a):
    return float(np.sqrt(np.mean(np.asarray(a, np.float64) ** 2)))


def check_close(got, want, tol=TOL):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = float(np.max(np.abs(got - want))) if want.size else 0.0
    assert err <= tol * rms(want), f"max|d|={err:.4g} rms={rms(want):.4g}"


# ---------------- synthetic inputs: device draws == host restatement ----------------

def test_synth_bytes_and_uniform(dev):
    torch.manual_seed(0)
    b = synth.bytes_(100003, "t.bytes").cpu().numpy()
    assert np.array_equal(b, synth_np.bytes_(100003, "t.bytes"))
    u = synth.uniform_int(50001, 123, 7, "t.scales", dtype=torch.uint8).cpu().numpy()
    assert np.array_equal(u, synth_np.uniform_int(50001, 123, 7, "t.scales").astype(np.uint8))
    ids = synth.uniform_int(4099, 0, 151936, "t.ids").cpu().numpy()
    assert np.array_equal(ids, synth_np.uniform_int(4099, 0, 151936, "t.ids"))
    assert ids.min() >= 0 and ids.max() < 151936


def test_synth_normal_matches_host(dev):
    n = 200001
    g32 = synth.normal(n, "t.n", std=0.02, dtype=torch.float32).cpu().numpy()
    h32 = synth_np.normal32(n, "t.n", std=0.02)
    # float64 log/cos/sin of the device library and of glibc may differ in the last place; after
    # rounding to float32 that shows in about 2^-29 of values: allow a handful, 1 ulp apart
    diff = g32 != h32
    assert diff.sum() <= 2
    assert np.all(np.abs(g32[diff].view(np.int32) - h32[diff].view(np.int32)) <= 1)
    g16 = synth.normal(n, "t.n16", dtype=torch.float16).cpu().numpy()
    h16 = synth_np.normal16(n, "t.n16")
    assert (g16 != h16).sum() <= 2
    assert abs(float(h32.astype(np.float64).std()) - 0.02) < 0.0005


def test_synth_mxfp4_equals_oracle_encode(dev, orc):
    rows, k = 64, 2048
    w, e = synth.mxfp4_normal(rows, k, "t.w", std=0.02)
    x = synth.normal(rows * k, "t.w", std=0.02, dtype=torch.float32).view(rows, k)
    ow, oe = orc.mxfp4_encode(x.cpu().numpy())
    assert np.array_equal(w.cpu().numpy(), ow) and np.array_equal(e.cpu().numpy(), oe)


def test_mxfp4_encode_equals_oracle(dev, orc):
    rng = np.random.default_rng(21)
    x = (rng.standard_normal((50, 256)) * np.exp(rng.standard_normal((50, 1)) * 3)).astype(np.float32)
    x[3, :32] = 0
    x[4, 5] = 0
    x[7, :] = np.float32(1e-40)  # subnormal: out of e8m0's range, zeros at e=0
    w, e = ops.mxfp4_encode(torch.from_numpy(x).cuda())
    ow, oe = orc.mxfp4_encode(x)
    assert np.array_equal(w.cpu().numpy(), ow) and np.array_equal(e.cpu().numpy(), oe)


# ---------------- MXFP4 dequantization and K1 ----------------

def test_mxfp4_dequant_f16_bit_exact(dev, orc):
    # every byte with every exponent but 255 (Inf: its NaNs are checked apart)
    w = np.tile(np.arange(256, dtype=np.uint8), (255, 1))
    e = np.tile(np.arange(255, dtype=np.uint8)[:, None], (1, 16))
    got = ops.mxfp4_dequant_f16(torch.from_numpy(w).cuda(), torch.from_numpy(e).cuda()).cpu().numpy()
    want = orc.f32_to_f16(orc.mxfp4_dequantize(w, e)).view(np.float16)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    e255 = np.full((1, 16), 255, np.uint8)
    got = ops.mxfp4_dequant_f16(torch.from_numpy(w[:1]).cuda(), torch.from_numpy(e255).cuda()).cpu().numpy()
    want = orc.mxfp4_dequantize(w[:1], e255)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    assert np.array_equal(got[fin].astype(np.float32), want[fin])


def mxfp4_case(n, k, name, emin=-4, emax=2):
    w, e = synth.mxfp4_uniform(n, k, name, emin=emin, emax=emax)
    x = synth.normal(k, name + ".x", dtype=torch.float16)
    return w, e, x


def oracle_gemv(orc, w, e, x):
    """The reference's dequant + sgemm (milcpu linear: x times W transposed)."""
    wd = orc.mxfp4_dequantize(w.cpu().numpy(), e.cpu().numpy())
    xf = x.cpu().numpy().astype(np.float32)[None, :]
    return orc.sgemm(xf, wd, transb=True)[0]


@pytest.mark.parametrize("n,k", [(8192, 2048), (1, 32), (7, 64), (33, 96), (100, 768), (300, 6144),
                                 (5, 4128), (129, 1024), (6144, 2048), (2048, 6144), (3072, 768)])
def test_mxfp4_gemv_parity(dev, orc, n, k):
    print(f"mxfp4_gemv n={n} k={k}", flush=True)
    w, e, x = mxfp4_case(n, k, f"c1.{n}.{k}")
    want = oracle_gemv(orc, w, e, x)
    y32 = ops.mxfp4_gemv(w, e, x, "f32")
    y16 = ops.mxfp4_gemv(w, e, x, "f16")
    torch.cuda.synchronize()
    y32 = y32.cpu().numpy()
    check_close(y32, want)
    # fp16 mode is RNE of the same fp32 accumulator, bit for bit
    assert np.array_equal(y16.cpu().numpy().view(np.uint16), orc.f32_to_f16(y32))
    # add mode adds the same fp32 value into y
    y0 = synth.normal(n, "c1.y0", dtype=torch.float32)
    base = y0.cpu().numpy()
    ops.mxfp4_gemv(w, e, x, "add", y=y0)
    assert np.array_equal(y0.cpu().numpy(), (base + y32).astype(np.float32))


def test_mxfp4_gemv_edge_values(dev, orc):
    """Codes 0 and 8 (+0 and -0), all-zero rows, e=0 (scale +0) and the widest exponents."""
    n, k = 64, 2048
    w, e, x = mxfp4_case(n, k, "c1.edge", emin=-20, emax=20)
    w[0] = 0
    w[1] = 0x88
    e[2] = 0
    e[3, :5] = 1
    e[4, :7] = 160
    want = oracle_gemv(orc, w, e, x)
    y32 = ops.mxfp4_gemv(w, e, x, "f32").cpu().numpy()
    assert y32[0] == 0 and y32[1] == 0 and y32[2] == 0
    check_close(y32, want)
    rest = np.arange(n) >= 5
    check_close(y32[rest], want[rest])


# ---------------- K2 (int8 per-channel) and K7 (fp16) ----------------

def i8_case(n, k, name):
    q = synth.uniform_int(n * k, -127, 255, name + ".q", dtype=torch.int8).view(n, k)
    s = synth.uniform_real(n, 0.002, 0.02, name + ".s", dtype=torch.float16)
    x = synth.normal(k, name + ".x", dtype=torch.float16)
    return q, s, x


@pytest.mark.parametrize("n,k", [(8192, 2048), (6144, 2048), (1, 16), (9, 48), (70, 800), (257, 6144), (33, 4096)])
def test_i8_gemv_parity(dev, orc, n, k):
    print(f"i8_gemv n={n} k={k}", flush=True)
    q, s, x = i8_case(n, k, f"k2.{n}.{k}")
    wd = orc.i8_dequant(q.cpu().numpy(), s.cpu().numpy().view(np.uint16))
    want = orc.sgemm(x.cpu().numpy().astype(np.float32)[None, :], wd, transb=True)[0]
    y32 = ops.i8_gemv(q, s, x, "f32").cpu().numpy()
    check_close(y32, want)
    y16 = ops.i8_gemv(q, s, x, "f16").cpu().numpy()
    assert np.array_equal(y16.view(np.uint16), orc.f32_to_f16(y32))


@pytest.mark.parametrize("n,k", [(151936, 2048), (1, 8), (13, 40), (100, 2048), (64, 6144)])
def test_f16_gemv_parity(dev, orc, n, k):
    print(f"f16_gemv n={n} k={k}", flush=True)
    w = synth.normal(n * k, f"k7.{n}.{k}", std=0.02).view(n, k)
    x = synth.normal(k, f"k7.{n}.{k}.x")
    wf = w.cpu().numpy().astype(np.float32)
    want = orc.sgemm(x.cpu().numpy().astype(np.float32)[None, :], wf, transb=True)[0]
    y32 = ops.f16_gemv(w, x, "f32").cpu().numpy()
    check_close(y32, want)
    y16 = ops.f16_gemv(w, x, "f16").cpu().numpy()
    assert np.array_equal(y16.view(np.uint16), orc.f32_to_f16(y32))


# K7r: the tied head over the T <= 8 rows of a speculative verify, each weight row read once
@pytest.mark.parametrize("T,n,k", [(5, 151936, 2048), (8, 4099, 2048), (1, 77, 2056), (3, 1000, 4096), (2, 5, 8)])
def test_f16_gemv_rows_parity(dev, orc, T, n, k):
    print(f"f16_gemv_rows T={T} n={n} k={k}", flush=True)
    w = synth.normal(n * k, f"k7r.{n}.{k}", std=0.02).view(n, k)
    x = synth.normal(T * k, f"k7r.{T}.{n}.{k}.x").view(T, k)
    want = orc.sgemm(x.cpu().numpy().astype(np.float32), w.cpu().numpy().astype(np.float32), transb=True)
    y32 = ops.f16_gemv_rows(w, x, "f32").cpu().numpy()
    for t in range(T):
        check_close(y32[t], want[t])
    y16 = ops.f16_gemv_rows(w, x, "f16").cpu().numpy()
    assert np.array_equal(y16.view(np.uint16), orc.f32_to_f16(y32))
    one = ops.f16_gemv(w, x[T - 1].contiguous(), "f32").cpu().numpy()
    check_close(one, y32[T - 1], tol=1e-5)


# ---------------- K1r: several vectors, weights read once ----------------

# (T >= 6 with k a multiple of 512: the matrix-core form; the rest: the VALU form)
@pytest.mark.parametrize("T,n,k", [(5, 8192, 2048), (1, 300, 6144), (2, 33, 96), (8, 2048, 2048), (3, 7, 4128),
                                   (5, 6144, 2048), (4, 2048, 6144), (6, 1000, 4096), (7, 33, 512), (8, 5, 2048)])
def test_mxfp4_gemv_rows_parity(dev, orc, T, n, k):
    print(f"mxfp4_gemv_rows T={T} n={n} k={k}", flush=True)
    w, e = synth.mxfp4_uniform(n, k, f"k1r.{n}.{k}")
    x = synth.normal(T * k, f"k1r.{T}.{n}.{k}.x").view(T, k)
    wd = orc.mxfp4_dequantize(w.cpu().numpy(), e.cpu().numpy())
    want = orc.sgemm(x.cpu().numpy().astype(np.float32), wd, transb=True)
    y32 = ops.mxfp4_gemv_rows(w, e, x, "f32").cpu().numpy()
    for t in range(T):
        check_close(y32[t], want[t])
    # each vector's fp16 output is RNE of its fp32 accumulator; one vector alone equals K1's
    y16 = ops.mxfp4_gemv_rows(w, e, x, "f16").cpu().numpy()
    assert np.array_equal(y16.view(np.uint16), orc.f32_to_f16(y32))
    one = ops.mxfp4_gemv(w, e, x[0].contiguous(), "f32").cpu().numpy()
    check_close(one, y32[0], tol=1e-5)


def test_mxfp4_gemv_rows_rejects_too_many(dev):
    from hwnpu_amd import HwkError

    w, e = synth.mxfp4_uniform(64, 256, "k1r.bad")
    x = synth.normal(9 * 256, "k1r.bad.x").view(9, 256)
    with pytest.raises(HwkError, match="1..8"):
        ops.mxfp4_gemv_rows(w, e, x)
