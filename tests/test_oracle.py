"""The CPU oracle pinned against the reference's own known-answer tests and invariants, and
against what the mathematics fixes (closed forms, brute force, textbook routines). CPU only."""
import math
import struct

import numpy as np
import pytest

VALUES = [0, 0.5, 1, 1.5, 2, 3, 4, 6, -0.0, -0.5, -1, -1.5, -2, -3, -4, -6]


def f32_of_bits(b):
    return struct.unpack("<f", struct.pack("<I", b))[0]


# ---------------- fp16 (internal/vecops/vecops.go:297-352) ----------------

def half_cases():
    """halfCases of internal/vecops/vecops_test.go:404-420."""
    bits = [0, 0x80000000, 1, 0x00800000,
            0x33000000, 0x33000001, 0x337FFFFF, 0x33800000, 0x33C00000, 0x33A00000,
            0x387FC000, 0x387FE000, 0x38800000,
            0x477FE000, 0x477FEFFF, 0x477FF000, 0x47800000,
            0x7F7FFFFF, 0x7F800000, 0xFF800000,
            0x3F801000, 0x3F803000, 0x3F800FFF, 0x3F801001]
    out = []
    for b in bits:
        out += [b, b | 0x80000000]
    return np.array(out, dtype=np.uint32).view(np.float32)


def test_f16_half_cases_match_ieee_rne(orc):
    # numpy's float32 -> float16 cast is IEEE round-to-nearest-even with overflow to infinity
    x = half_cases()
    got = orc.f32_to_f16(x)
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_f16_random_match_ieee_rne(orc):
    rng = np.random.default_rng(5)
    x = np.concatenate([
        rng.integers(0, 2**32, 20000, dtype=np.uint64).astype(np.uint32).view(np.float32),
        (rng.standard_normal(20000) * 2.0 ** rng.integers(-25, 15, 20000)).astype(np.float32),
    ])
    nan = np.isnan(x)
    got = orc.f32_to_f16(x)
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got[~nan], want[~nan])
    # a NaN becomes the quiet NaN sign|0x7e00, its payload dropped (vecops.go:303-306)
    sign = (x[nan].view(np.uint32) >> 16).astype(np.uint16) & 0x8000
    assert np.array_equal(got[nan], sign | 0x7E00)


def test_f16_all_halves_round_trip(orc):
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    f = orc.f16_to_f32(h)
    ok = ~((h & 0x7C00) == 0x7C00) | ((h & 0x3FF) == 0)  # not NaN
    assert np.array_equal(f[ok].view(np.uint32), h[ok].view(np.float16).astype(np.float32).view(np.uint32))
    assert np.array_equal(orc.f32_to_f16(f[ok]), h[ok])


# ---------------- MXFP4 (internal/mxfp4) ----------------

def test_mxfp4_scale_closed_form(orc):
    assert orc.mxfp4_scale(0) == 0.0 and math.copysign(1, orc.mxfp4_scale(0)) == 1  # e=0: +0
    assert orc.mxfp4_scale(255) == math.inf
    for e in range(1, 255):
        assert orc.mxfp4_scale(e) == math.ldexp(1.0, e - 127)


def test_mxfp4_dequantize_every_code_and_exponent(orc):
    # one row per exponent, every byte value once per 256 bytes = 16 blocks
    w = np.tile(np.arange(256, dtype=np.uint8), (256, 1))
    e = np.tile(np.arange(256, dtype=np.uint8)[:, None], (1, 16))
    got = orc.mxfp4_dequantize(w, e)
    for ex in range(256):
        s = 0.0 if ex == 0 else math.inf if ex == 255 else math.ldexp(1.0, ex - 127)
        for b in range(256):
            lo, hi = VALUES[b & 15], VALUES[b >> 4]
            with np.errstate(invalid="ignore"):
                want = np.array([lo * s, hi * s], dtype=np.float64).astype(np.float32)
            g = got[ex, 2 * b: 2 * b + 2]
            # even element from the low nibble, -0 kept as -0 (bits compared), NaN for 0 x Inf
            for gv, wv in zip(g, want):
                if np.isnan(wv):
                    assert np.isnan(gv)
                else:
                    assert gv.view(np.uint32) == wv.view(np.uint32), (ex, b)


def test_nearest_kat(orc):
    """internal/mxfp4/mxfp4_test.go:168-175."""
    cases = [(0.25, 0), (0.26, 1), (0.75, 2), (1.25, 2), (1.75, 4), (2.5, 4), (3.5, 6), (5, 6), (5.1, 7),
             (100, 7), (-0.6, 9), (-0.1, 0)]
    for x, want in cases:
        assert orc.mxfp4_nearest(x) == want, x


def brute_nearest(x):
    """argmin over the 16 codes of |x - value|; ties to the even code; 0 as +0 (code 0)."""
    best = None
    for c in range(16):
        d = abs(x - VALUES[c])
        if best is None or d < best[0] or (d == best[0] and (c & 1) == 0 and (best[1] & 1) == 1):
            best = (d, c)
    c = best[1]
    return 0 if VALUES[c] == 0 else c


def test_nearest_brute_force(orc):
    rng = np.random.default_rng(1)
    xs = list(rng.uniform(-8, 8, 4000)) + [v / 2 for v in range(-16, 17)] + [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0]
    xs += [-x for x in xs]
    for x in xs:
        assert orc.mxfp4_nearest(float(x)) == brute_nearest(float(x)), x


def block_sse(blk, eb):
    s = math.ldexp(1.0, eb - 127)
    return sum((float(v) - VALUES[brute_nearest(float(v) / s)] * s) ** 2 for v in blk)


def test_encode_invariants(orc):
    """TestEncode (internal/mxfp4/mxfp4_test.go:131-176), plus: the chosen scale has the least
    squared error among all e8m0 exponents, and every code is the nearest at that scale."""
    rng = np.random.default_rng(3)
    nb = 64
    row = (rng.standard_normal(nb * 32) * 0.02).astype(np.float32)
    row[5] = 0
    row[32:64] = 0
    w, e = orc.mxfp4_encode(row[None, :])
    got = orc.mxfp4_dequantize(w, e)[0]
    assert got[5] == 0 and got[32] == 0 and e[0, 1] == 0
    rel = np.sqrt(np.sum((row - got).astype(np.float64) ** 2) / np.sum(row.astype(np.float64) ** 2))
    assert rel <= 0.12
    for b in range(nb):
        blk = row[b * 32:(b + 1) * 32]
        if not np.any(blk):
            continue
        eb = int(e[0, b])
        s = math.ldexp(1.0, eb - 127)
        for j in range(32):
            code = (w[0, b * 16 + j // 2] >> (4 * (j & 1))) & 15
            assert code == brute_nearest(float(blk[j]) / s)
        best = min(block_sse(blk, x) for x in range(1, 255))
        assert block_sse(blk, eb) == best


def test_vec_quantize_and_dot(orc):
    """TestDot (internal/mxfp4/mxfp4_test.go:21-55)."""
    rng = np.random.default_rng(2)
    for nb in (1, 2, 3, 90):
        w = rng.integers(0, 256, nb * 16, dtype=np.uint8)
        e = rng.integers(118, 126, nb, dtype=np.uint8)
        x = rng.standard_normal(nb * 32).astype(np.float32)
        q, s = orc.vec_quantize(x)
        row = orc.mxfp4_dequantize(w[None, :], e[None, :])[0].astype(np.float64)
        # q holds a block's 16 even values then its 16 odd ones
        xq = np.empty(nb * 32)
        for b in range(nb):
            xq[b * 32:(b + 1) * 32:2] = q[b * 32:b * 32 + 16] * np.float64(s[b])
            xq[b * 32 + 1:(b + 1) * 32:2] = q[b * 32 + 16:(b + 1) * 32] * np.float64(s[b])
        want = float(row @ xq)
        got = orc.mxfp4_dot(w, e, q, s)
        assert abs(got - want) <= 1e-4 * max(1, abs(want))
        exact = float(row @ x.astype(np.float64))
        assert abs(want - exact) <= 0.01 * math.sqrt(float(row @ row) * float(x.astype(np.float64) @ x))
        # the quantized values are within half a step of x
        assert np.all(np.abs(xq - x) <= np.repeat(s, 32) / 2 + 1e-7)


def test_run_matches_dot(orc):
    """TestRunVectors (mxfp4_test.go:76-104): Run gives Dot's values for every vector and row."""
    rng = np.random.default_rng(4)
    rows, nb = 71, 90
    w = rng.integers(0, 256, (rows, nb * 16), dtype=np.uint8)
    e = rng.integers(118, 126, (rows, nb), dtype=np.uint8)
    xs = rng.standard_normal((5, nb * 32)).astype(np.float32)
    qs, ss = zip(*(orc.vec_quantize(x) for x in xs))
    out = orc.mxfp4_run(w, e, np.stack(qs), np.stack(ss), threads=4)
    for v in range(5):
        for r in range(rows):
            assert out[v, r] == orc.mxfp4_dot(w[r], e[r], qs[v], ss[v])


# ---------------- fp32 GEMM (internal/sgemm) ----------------

@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (6, 16, 8), (7, 17, 3), (13, 50, 300), (100, 33, 513),
                                   (5, 4000, 70), (200, 9, 64)])
@pytest.mark.parametrize("transb", [False, True])
@pytest.mark.parametrize("threads", [1, 4])
def test_sgemm_vs_f64(orc, m, n, k, transb, threads):
    """TestMulAdd (internal/sgemm/sgemm_test.go:31-62): adds to C, tolerance 1e-4*sqrt(k)+1e-5."""
    rng = np.random.default_rng(m * 1000 + n + k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((n, k) if transb else (k, n)).astype(np.float32)
    c0 = rng.standard_normal((m, n)).astype(np.float32)
    bb = b.T if transb else b
    want = c0.astype(np.float64) + a.astype(np.float64) @ bb.astype(np.float64)
    got = orc.sgemm(a, b, c0.copy(), transb=transb, threads=threads)
    assert np.max(np.abs(got - want)) <= 1e-4 * math.sqrt(k) + 1e-5


# ---------------- int8 weights and the int8 KV rule ----------------

def test_i8_dequant_exact(orc):
    rng = np.random.default_rng(6)
    q = rng.integers(-128, 128, (37, 64), dtype=np.int8)
    s16 = rng.uniform(0.002, 0.02, 37).astype(np.float16)
    got = orc.i8_dequant(q, s16.view(np.uint16))
    want = q.astype(np.float64) * s16.astype(np.float64)[:, None]  # exact in float32
    assert np.array_equal(got.astype(np.float64), want)


def test_i8_quantize_rows(orc):
    """The int8 KV rule: scale fp16(absmax/127) (1 for a zero row, experts weights_test.go:28-41),
    codes within half a scale of the value, the largest magnitude at +-127 or +-126."""
    rng = np.random.default_rng(7)
    x = rng.standard_normal((20, 128)).astype(np.float32)
    x[3] = 0
    q, s16 = orc.i8_quantize_rows(x)
    s = s16.view(np.float16).astype(np.float32)
    assert s[3] == 1 and not np.any(q[3])
    back = q.astype(np.float32) * s[:, None]
    assert np.all(np.abs(back - x) <= s[:, None] / 2 * (1 + 1e-6))
    assert np.all(np.abs(q).max(axis=1)[np.arange(20) != 3] >= 126)
    assert np.array_equal(s16, (np.abs(x).max(axis=1) / np.float32(127)).astype(np.float16).view(np.uint16)
                          * (np.arange(20) != 3) + (np.arange(20) == 3) * np.float16(1).view(np.uint16))


# ---------------- chunk attention and merge (internal/llm/paged) ----------------

def test_merge_order_kat(orc):
    """TestMergeOrder (internal/llm/paged/paged_test.go:133-157)."""
    o = [[1, 2], [3, 4], [5, 6]]
    m = [-1, 4, 2]
    l = [2, 1, 3]
    wsum = x0 = x1 = 0.0
    for j in range(3):
        wj = l[j] * math.exp(m[j] - 4)
        wsum += wj
        x0 += wj * o[j][0]
        x1 += wj * o[j][1]
    for order in ([0, 1, 2], [2, 1, 0], [1, 0, 2]):
        mg = orc.Merge(1, 2)
        for j in order:
            mg.add(np.array(o[j], np.float32), np.array([m[j]], np.float32), np.array([l[j]], np.float32))
        out = mg.result()[0]
        assert abs(out[0] - x0 / wsum) <= 1e-5 and abs(out[1] - x1 / wsum) <= 1e-5


def test_merge_sink_kat(orc):
    """TestMergeSink (paged_test.go:159-186)."""
    scores = [0.5, -1, 2]
    vals = [[1, 2], [3, -1], [0.5, 4]]
    sink = 1.5
    tot = sum(math.exp(s) for s in scores) + math.exp(sink)
    want = [sum(math.exp(s) / tot * v[j] for s, v in zip(scores, vals)) for j in range(2)]
    mg = orc.Merge(1, 2)
    for s, v in zip(scores, vals):
        mg.add(np.array(v, np.float32), np.array([s], np.float32), np.array([1], np.float32))
    mg.add_sink(np.array([sink], np.float32), 1)
    got = mg.result()[0]
    assert abs(got[0] - want[0]) <= 1e-5 and abs(got[1] - want[1]) <= 1e-5


def full_softmax_attention(q, k, v, visible, scale):
    """One float64 softmax over every visible key (paged_test.go:36-75)."""
    heads, tokens, d = q.shape
    kvh, cache, _ = k.shape
    rep = heads // kvh
    out = np.zeros((heads, tokens, d))
    for h in range(heads):
        for r in range(tokens):
            sc = np.array([q[h, r].astype(np.float64) @ k[h // rep, p].astype(np.float64) * scale
                           if visible(r, p) else -np.inf for p in range(cache)])
            e = np.exp(sc - sc.max())
            out[h, r] = (e[:, None] * v[h // rep].astype(np.float64)).sum(0) / e.sum()
    return out


@pytest.mark.parametrize("heads,kvh,d,scale", [(16, 4, 32, None), (16, 8, 8, None), (4, 4, 8, None), (8, 1, 16, 1.0)])
def test_chunks_merged_match_full_softmax(orc, heads, kvh, d, scale):
    """TestMergeMatchesFull (paged_test.go:17-131): chunks wholly visible, one partly visible under
    a causal mask over several query rows, one wholly masked; relative error <= 5e-3."""
    chunk, chunks, tokens, first = 16, 4, 3, 37
    cache = chunk * chunks
    rng = np.random.default_rng(3)
    q = rng.standard_normal((heads, tokens, d)).astype(np.float32)
    k = rng.standard_normal((kvh, cache, d)).astype(np.float32)
    v = rng.standard_normal((kvh, cache, d)).astype(np.float32)
    sc = 1 / math.sqrt(d) if scale is None else scale
    visible = lambda r, p: p < first + r + 1
    want = full_softmax_attention(q, k, v, visible, sc)
    mg = orc.Merge(heads * tokens, d)
    for j in range(chunks):
        mask = np.array([[0 if visible(r, j * chunk + c) else -1e4 for c in range(chunk)] for r in range(tokens)],
                        np.float32)
        o, m, l = orc.paged_chunk(q, k[:, j * chunk:(j + 1) * chunk], v[:, j * chunk:(j + 1) * chunk], mask, sc)
        mg.add(o.reshape(heads * tokens, d), m.reshape(-1), l.reshape(-1))
    got = mg.result().reshape(heads, tokens, d)
    err = np.sqrt(np.sum((got - want) ** 2) / np.sum(want ** 2))
    assert err <= 5e-3


def test_attn_decode_matches_full_softmax(orc):
    rng = np.random.default_rng(9)
    heads, kvh, d, L = 8, 2, 64, 300
    q = rng.standard_normal((heads, d)).astype(np.float32)
    k = rng.standard_normal((kvh, L, d)).astype(np.float32)
    v = rng.standard_normal((kvh, L, d)).astype(np.float32)
    want = full_softmax_attention(q[:, None], k, v, lambda r, p: True, 1 / 8)[:, 0]
    for chunk in (64, 100, 8192):
        got = orc.attn_decode(q, k, v, 1 / 8, chunk=chunk)
        assert np.max(np.abs(got - want)) <= 1e-5 * max(1, np.max(np.abs(want)))


# ---------------- routing (internal/llm/experts/weights.go:33-81) ----------------

def test_choose_sigmoid_bias_kat(orc):
    """TestChooseSigmoidBias (internal/llm/experts/weights_test.go:11-26)."""
    idx, w = orc.choose(np.array([2, 1, 0, -1], np.float32), 2, score="sigmoid", norm=True,
                        bias=np.array([0, 0, 3, 0], np.float32))
    assert list(idx) == [2, 0]
    sig = lambda x: 1 / (1 + math.exp(-x))
    s2, s0 = sig(0), sig(2)
    assert abs(w[0] - s2 / (s2 + s0)) <= 1e-5 and abs(w[1] - s0 / (s2 + s0)) <= 1e-5


def test_choose_softmax_is_stable_topk(orc):
    """top-k equals a full stable sort's first k, ties to the lower index
    (internal/llm/iron/moe_test.go:9-29); weights are the chosen softmax scores renormalized."""
    rng = np.random.default_rng(11)
    for trial in range(300):
        logits = rng.standard_normal(32).astype(np.float32)
        if trial % 3 == 0:  # exact ties
            logits[rng.integers(0, 32, 6)] = logits[0]
        idx, w = orc.choose(logits, 4)
        order = np.argsort(-logits.astype(np.float64), kind="stable")
        assert list(idx) == list(order[:4])
        p = np.exp(logits.astype(np.float64) - logits.max())
        p /= p.sum()
        want = p[order[:4]] / (p[order[:4]].sum() + 1e-6)
        assert np.allclose(w, want, rtol=1e-5, atol=0)


# ---------------- experts (internal/llm/experts/host.go) ----------------

def experts_f64(orc, x, idx, w, gu_w, gu_e, dn_w, dn_e):
    T, H = x.shape
    E, I2 = gu_e.shape[:2]
    I = I2 // 2
    out = np.zeros((T, H))
    for t in range(T):
        for j in np.argsort(idx[t]):
            e = idx[t, j]
            gu = orc.mxfp4_dequantize(gu_w[e].reshape(I2, -1), gu_e[e]).astype(np.float64) @ x[t].astype(np.float64)
            g, u = gu[0::2], gu[1::2]
            a = g / (1 + np.exp(-g)) * u
            y = orc.mxfp4_dequantize(dn_w[e].reshape(H, -1), dn_e[e]).astype(np.float64) @ a
            out[t] += w[t, j] * y
    return out


def test_experts_f32_vs_f64_and_host(orc):
    """The fp32 experts against a float64 brute force, and the int8-activation (production) form
    against them: cosine >= 0.999, norm ratio within 2 % (experts/host_test.go:211-285)."""
    rng = np.random.default_rng(12)
    E, H, I, T, k = 6, 128, 64, 3, 2
    gu_w = rng.integers(0, 256, (E, 2 * I, H // 32, 16), dtype=np.uint8)
    gu_e = rng.integers(122, 127, (E, 2 * I, H // 32), dtype=np.uint8)
    dn_w = rng.integers(0, 256, (E, H, I // 32, 16), dtype=np.uint8)
    dn_e = rng.integers(118, 123, (E, H, I // 32), dtype=np.uint8)
    x = rng.standard_normal((T, H)).astype(np.float32)
    idx = np.array([[4, 1], [1, 2], [0, 4]], np.int32)
    w = rng.uniform(0.2, 0.8, (T, k)).astype(np.float32)
    want = experts_f64(orc, x, idx, w, gu_w, gu_e, dn_w, dn_e)
    got = orc.experts(x, idx, w, gu_w, gu_e, dn_w, dn_e)
    assert np.max(np.abs(got - want)) <= 1e-5 * np.sqrt(np.mean(want ** 2))
    host = orc.experts(x, idx, w, gu_w, gu_e, dn_w, dn_e, quantized=True)
    for t in range(T):
        cos = host[t] @ want[t] / np.linalg.norm(host[t]) / np.linalg.norm(want[t])
        assert cos >= 0.999
        assert abs(np.linalg.norm(host[t]) / np.linalg.norm(want[t]) - 1) <= 0.02


def experts_gptoss_f64(orc, x, idx, w, gu_w, gu_e, gu_b, dn_w, dn_e, dn_b, alpha=1.702, limit=7.0, clamp=True,
                       plus_one=True, bias=True):
    """TestHostRunSmall's float64 reference (internal/llm/experts/host_test.go:208-284): gate/up in
    float64 plus their bias, g = min(g, 7), u = clamp(u, -7, 7), act = float32(g/(1+e^(-1.702 g))*(u+1)),
    out += w * (down(act) + down bias). The switches drop a step, for the mutation checks."""
    T, H = x.shape
    E, I2 = gu_e.shape[:2]
    I = I2 // 2
    out = np.zeros((T, H))
    for t in range(T):
        for j in range(idx.shape[1]):
            e = idx[t, j]
            gu = orc.mxfp4_dequantize(gu_w[e].reshape(I2, -1), gu_e[e]).astype(np.float64) @ x[t].astype(np.float64)
            if bias:
                gu += gu_b[e]
            g, u = gu[0::2], gu[1::2]
            if clamp:
                g, u = np.minimum(g, limit), np.clip(u, -limit, limit)
            a = (g / (1 + np.exp(-alpha * g)) * ((u + 1) if plus_one else u)).astype(np.float32).astype(np.float64)
            y = orc.mxfp4_dequantize(dn_w[e].reshape(H, -1), dn_e[e]).astype(np.float64) @ a
            out[t] += w[t, j] * (y + (dn_b[e] if bias else 0))
    return out


@pytest.mark.parametrize("exp_lo", [118, 126])
def test_experts_gptoss_unit_and_biases(orc, exp_lo):
    """The gpt-oss gated unit and the expert biases against TestHostRunSmall's float64 form: the fp32
    path within 1e-4 * RMS, the int8-activation path at cosine >= 0.999 and norms within 2 %, as that
    test asks at its scales (exponents 118..123). Exponents from 126 put many gate/up sums past the limit (the clamp taken). Each
    mutation (no clamp, no +1, no biases) of the float64 form moves it away from the oracle."""
    rng = np.random.default_rng(21)
    E, K, H, I = 4, 2, 128, 64
    gu_w = rng.integers(0, 256, (E, 2 * I, H // 32, 16), dtype=np.uint8)
    dn_w = rng.integers(0, 256, (E, H, I // 32, 16), dtype=np.uint8)
    gu_e = rng.integers(exp_lo, exp_lo + 6, (E, 2 * I, H // 32), dtype=np.uint8)
    dn_e = rng.integers(118, 124, (E, H, I // 32), dtype=np.uint8)
    gu_b = (rng.standard_normal((E, 2 * I)) * 0.1).astype(np.float32)
    dn_b = (rng.standard_normal((E, H)) * 0.1).astype(np.float32)
    for n in (1, 3):
        x = rng.standard_normal((n, H)).astype(np.float32)
        idx = np.stack([rng.permutation(E)[:K] for _ in range(n)]).astype(np.int32)
        w = np.tile(np.array([0.7, 0.3], np.float32), (n, 1))
        kw = dict(gu_b=gu_b, dn_b=dn_b, act="gptoss", alpha=1.702, limit=7.0)
        want = experts_gptoss_f64(orc, x, idx, w, gu_w, gu_e, gu_b, dn_w, dn_e, dn_b)
        got = orc.experts(x, idx, w, gu_w, gu_e, dn_w, dn_e, **kw)
        rms = np.sqrt(np.mean(want ** 2))
        assert np.max(np.abs(got - want)) <= 1e-4 * rms
        if exp_lo == 118:  # the reference test's scales (the int8 activations lose more past them)
            host = orc.experts(x, idx, w, gu_w, gu_e, dn_w, dn_e, quantized=True, **kw)
            for t in range(n):
                cos = host[t] @ want[t] / np.linalg.norm(host[t]) / np.linalg.norm(want[t])
                assert cos >= 0.999 and abs(np.linalg.norm(host[t]) / np.linalg.norm(want[t]) - 1) <= 0.02
        muts = [dict(plus_one=False), dict(bias=False)] + ([dict(clamp=False)] if exp_lo >= 126 else [])
        for mut in muts:
            bad = experts_gptoss_f64(orc, x, idx, w, gu_w, gu_e, gu_b, dn_w, dn_e, dn_b, **mut)
            assert np.max(np.abs(got - bad)) > 1e-2 * rms, mut
    # the clamp is taken at the large exponents
    if exp_lo >= 126:
        gu = orc.mxfp4_dequantize(gu_w[0].reshape(2 * I, -1), gu_e[0]).astype(np.float64) @ x[0].astype(np.float64)
        assert np.any(np.abs(gu) > 7)


def test_experts_silu_with_biases(orc):
    """The SiLU unit with biases: the fp32 path against a float64 brute force of silu(g+bg)*(u+bu)
    and w * (y + bd)."""
    rng = np.random.default_rng(22)
    E, H, I = 5, 96, 64
    gu_w = rng.integers(0, 256, (E, 2 * I, H // 32, 16), dtype=np.uint8)
    gu_e = rng.integers(122, 126, (E, 2 * I, H // 32), dtype=np.uint8)
    dn_w = rng.integers(0, 256, (E, H, I // 32, 16), dtype=np.uint8)
    dn_e = rng.integers(118, 122, (E, H, I // 32), dtype=np.uint8)
    gu_b = rng.standard_normal((E, 2 * I)).astype(np.float32)
    dn_b = rng.standard_normal((E, H)).astype(np.float32)
    x = rng.standard_normal((2, H)).astype(np.float32)
    idx = np.array([[3, 0, 4], [1, 3, 2]], np.int32)
    w = rng.uniform(0.1, 0.5, (2, 3)).astype(np.float32)
    got = orc.experts(x, idx, w, gu_w, gu_e, dn_w, dn_e, gu_b=gu_b, dn_b=dn_b)
    want = np.zeros((2, H))
    for t in range(2):
        for j in range(3):
            e = idx[t, j]
            gu = orc.mxfp4_dequantize(gu_w[e].reshape(2 * I, -1), gu_e[e]).astype(np.float64) @ x[t] + gu_b[e]
            g, u = gu[0::2], gu[1::2]
            y = orc.mxfp4_dequantize(dn_w[e].reshape(H, -1), dn_e[e]).astype(np.float64) @ (g / (1 + np.exp(-g)) * u)
            want[t] += w[t, j] * (y + dn_b[e])
    assert np.max(np.abs(got - want)) <= 1e-4 * np.sqrt(np.mean(want ** 2))


# ---------------- decoder ops ----------------

def test_rmsnorm_closed_form(orc):
    rng = np.random.default_rng(13)
    x = (rng.standard_normal((4, 2048)) * 7).astype(np.float32)
    y = orc.rmsnorm(x, np.ones(2048, np.float32), 1e-6)
    assert np.allclose(np.sqrt(np.mean(y.astype(np.float64) ** 2, axis=1)), 1, atol=1e-6)
    w = rng.standard_normal(2048).astype(np.float32)
    y2 = orc.rmsnorm(x, w, 1e-6)
    assert np.allclose(y2, y * w, rtol=1e-6, atol=0)


def test_rope_tables_and_rotation(orc):
    c, s = orc.rope_tables(1e6, 0, 1200, 128)
    assert np.all(c[0] == 1) and np.all(s[0] == 0)
    j = np.arange(64)
    inv = 1 / 1e6 ** (2 * j / 128)
    for pos in (1, 77, 1199):
        a = pos * inv
        assert np.array_equal(c[pos, :64], np.cos(a).astype(np.float32)) and np.array_equal(c[pos, 64:], c[pos, :64])
        assert np.array_equal(s[pos, :64], np.sin(a).astype(np.float32))
    rng = np.random.default_rng(14)
    x = rng.standard_normal((8, 128)).astype(np.float32)
    assert np.array_equal(orc.apply_rope(x, c[0], s[0]), x)
    y = orc.apply_rope(x, c[500], s[500])
    # a rotation of each (j, j+64) pair: norms kept per pair
    n0 = x[:, :64] ** 2 + x[:, 64:] ** 2
    n1 = y[:, :64].astype(np.float64) ** 2 + y[:, 64:].astype(np.float64) ** 2
    assert np.allclose(n0, n1, rtol=1e-5)


def test_silu_and_argmax(orc):
    g = np.array([-20, -1, 0, 1, 20], np.float32)
    u = np.array([1, 2, 3, 4, 5], np.float32)
    want = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.allclose(orc.silu_mul(g, u), want, rtol=1e-6)
    x = np.array([0, 3, 1, 3, 2], np.float32)
    assert orc.argmax(x) == 1  # ties to the lowest index (internal/chat/sample.go:80-87)


# ---------------- the reference's synthetic checkpoint (internal/llm/synth.go:17-35) ----------------

def test_fnv64a_published_vectors(orc):
    """FNV-1a 64-bit test vectors from the algorithm's authors (the seed of Synthetic.Get)."""
    assert orc.fnv64a("") == 0xCBF29CE484222325
    assert orc.fnv64a("a") == 0xAF63DC4C8601EC8C
    assert orc.fnv64a("foobar") == 0x85944171F73967E8


def test_synth_reference_sequence_and_distribution(orc):
    """The first values against the recurrence evaluated with Python integers mod 2^64 (another
    implementation of Knuth's MMIX LCG), and the distribution of 2^20 values: inside [-0.2, 0.2),
    mean near 0, 64 equal bins within a chi-square bound."""
    name = "model.layers.3.mlp.down_proj.weight"
    got = orc.synth_reference(name, 1 << 20)
    seed = orc.fnv64a(name)
    for i in range(64):
        seed = (seed * 6364136223846793005 + 1442695040888963407) % (1 << 64)
        want = np.float32(np.float32((seed >> 40) - (1 << 23)) / np.float32(1 << 23)) * np.float32(0.2)
        assert got[i] == want, i
    assert got.min() >= -0.2 and got.max() < 0.2
    assert abs(float(got.astype(np.float64).mean())) < 5 * 0.2 / np.sqrt(3) / np.sqrt(got.size)
    hist, _ = np.histogram(got, bins=64, range=(-0.2, 0.2))
    e = got.size / 64
    chi2 = float(((hist - e) ** 2 / e).sum())
    assert chi2 < 120, chi2  # 63 degrees of freedom: p < 1e-5 past 120
    # names give independent streams
    other = orc.synth_reference(name + "x", 1024)
    assert not np.array_equal(other, got[:1024])
