"""Pins the oracle's Qwen3 decoder (oracle/qwen3.c) the way the reference pins its program:
against a float64 forward written out from modeling_qwen3.py's semantics on the same weights
(reference internal/llm/qwen3/qwen3_test.go:77-207, relative RMS error of the logits :225-234),
and cached stepping against the full prompt (cache_test.go:187-213, <= 5e-3). Also the synthetic
checkpoint: the normal stream against its numpy restatement and the checksums against a recount.
"""
import numpy as np
import pytest

import synth_np
from hwnpu_amd.synth import key_of

TINY = dict(layers=2, hidden=64, heads=4, kv_heads=2, head_dim=16, inter=96, vocab=50, max_ctx=32)


def weights(orc, cfg, seed=0, std=0.02):
    """The synthetic checkpoint rebuilt in numpy: normal32 per name, the oracle's MXFP4 encoder,
    dequantized (the encoder itself is pinned by the nearest() KAT and brute force elsewhere)."""
    def lin(name, rows, cols):
        x = synth_np.normal32(rows * cols, name, std, seed).reshape(rows, cols)
        w, e = orc.mxfp4_encode(x)
        return orc.mxfp4_dequantize(w, e).astype(np.float64), int(w.astype(np.uint64).sum()), int(e.astype(np.uint64).sum())

    hd, nh, nkv = cfg["head_dim"], cfg["heads"], cfg["kv_heads"]
    W, sb, ss = [], 0, 0
    for i in range(cfg["layers"]):
        p = f"model.layers.{i}."
        d = {}
        for nm, rows, cols in (("self_attn.q_proj.weight", nh * hd, cfg["hidden"]),
                               ("self_attn.k_proj.weight", nkv * hd, cfg["hidden"]),
                               ("self_attn.v_proj.weight", nkv * hd, cfg["hidden"]),
                               ("self_attn.o_proj.weight", cfg["hidden"], nh * hd),
                               ("mlp.gate_proj.weight", cfg["inter"], cfg["hidden"]),
                               ("mlp.up_proj.weight", cfg["inter"], cfg["hidden"]),
                               ("mlp.down_proj.weight", cfg["hidden"], cfg["inter"])):
            d[nm], b, s = lin(p + nm, rows, cols)
            sb, ss = sb + b, ss + s
        W.append(d)
    e16 = synth_np.normal32(cfg["vocab"] * cfg["hidden"], "model.embed_tokens.weight", std, seed).astype(np.float16)
    se = int(e16.view(np.uint16).astype(np.uint64).sum())
    return W, e16.astype(np.float64).reshape(cfg["vocab"], cfg["hidden"]), [sb, ss, se]


NORMS = ("input_layernorm.weight", "post_attention_layernorm.weight", "self_attn.q_norm.weight",
         "self_attn.k_norm.weight")


def forward64(cfg, W, E, ids, theta=1e6, eps=1e-6, final_norm=None):
    """Qwen3ForCausalLM in float64 (qwen3_test.go:77-207), logits of every row. A layer's dict may
    hold its RMSNorm weights under their Hugging Face names (NORMS; qwen3_test.go:155-163,196,205),
    final_norm is model.norm's; absent ones are 1."""
    s, d, nh, nkv, hd = len(ids), cfg["hidden"], cfg["heads"], cfg["kv_heads"], cfg["head_dim"]

    def rms(x, w=None):
        y = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
        return y if w is None else y * np.asarray(w, np.float64)

    half = hd // 2
    inv = 1.0 / theta ** (np.arange(half) * 2.0 / hd)
    ang = np.arange(s)[:, None] * inv[None, :]
    cos = np.concatenate([np.cos(ang), np.cos(ang)], 1)[:, None, :]
    sin = np.concatenate([np.sin(ang), np.sin(ang)], 1)[:, None, :]

    def rope(x):
        rot = np.concatenate([-x[..., half:], x[..., :half]], -1)
        return x * cos + rot * sin

    h = E[np.asarray(ids)]
    for w in W:
        x = rms(h, w.get("input_layernorm.weight"))
        q = rms((x @ w["self_attn.q_proj.weight"].T).reshape(s, nh, hd), w.get("self_attn.q_norm.weight"))
        k = rms((x @ w["self_attn.k_proj.weight"].T).reshape(s, nkv, hd), w.get("self_attn.k_norm.weight"))
        v = (x @ w["self_attn.v_proj.weight"].T).reshape(s, nkv, hd)
        q, k = rope(q), rope(k)
        o = np.zeros((s, nh, hd))
        for hh in range(nh):
            kh = hh // (nh // nkv)
            sc = q[:, hh] @ k[:, kh].T / np.sqrt(hd)
            sc = np.where(np.tril(np.ones((s, s), bool)), sc, -np.inf)
            p = np.exp(sc - sc.max(1, keepdims=True))
            o[:, hh] = (p / p.sum(1, keepdims=True)) @ v[:, kh]
        h = h + o.reshape(s, nh * hd) @ w["self_attn.o_proj.weight"].T
        x = rms(h, w.get("post_attention_layernorm.weight"))
        g, u = x @ w["mlp.gate_proj.weight"].T, x @ w["mlp.up_proj.weight"].T
        h = h + (g / (1 + np.exp(-g)) * u) @ w["mlp.down_proj.weight"].T
    return rms(h, final_norm) @ E.T


def norm_weights(cfg, seed=11, sd=0.2):
    """Non-unit RMSNorm weights N(1, sd) for every norm of the model, by Hugging Face name."""
    rng = np.random.default_rng(seed)
    out = {}
    for i in range(cfg["layers"]):
        for n in NORMS:
            size = cfg["head_dim"] if "_norm." in n and "self_attn" in n else cfg["hidden"]
            out[f"model.layers.{i}.{n}"] = (1 + sd * rng.standard_normal(size)).astype(np.float32)
    out["model.norm.weight"] = (1 + sd * rng.standard_normal(cfg["hidden"])).astype(np.float32)
    return out


def with_norms(W, norms, drop=()):
    """W's layer dicts with the norm weights added, except the names in drop (mutations)."""
    out = []
    for i, w in enumerate(W):
        d = dict(w)
        for n in NORMS:
            if n not in drop:
                d[n] = norms[f"model.layers.{i}.{n}"]
        out.append(d)
    return out


def rel_rms(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.sqrt(np.mean((a - b) ** 2)) / np.sqrt(np.mean(b ** 2)))


def test_normal_stream_matches_numpy(orc):
    key = key_of("t.normal")
    got = np.array([orc.normal_at(key, i) for i in range(1001)])
    want = synth_np.normal64(1001, "t.normal")
    # glibc's and numpy's float64 log/cos/sin may differ in the last place
    assert np.allclose(got, want, rtol=4e-16, atol=0)
    assert np.sum(got.astype(np.float32) != want.astype(np.float32)) <= 1
    assert orc.fnv64a("model.embed_tokens.weight") == key_of("model.embed_tokens.weight")


def test_qwen3_oracle_matches_float64_forward(orc):
    W, E, sums = weights(orc, TINY)
    m = orc.Qwen3(**TINY, seed=0, std=0.02)
    assert m.checksums() == sums
    ids = [3, 17, 42, 8, 8, 0, 49, 21, 5, 33, 12]
    want = forward64(TINY, W, E, ids)
    # the prompt's last row, then each following position stepped with the KV cache
    tok, got = m.run(ids[:6], 0)
    assert rel_rms(got, want[5]) < 5e-3
    assert tok == int(np.argmax(got))
    for p in range(6, len(ids)):
        _, got = m.run([ids[p]], p)
        assert rel_rms(got, want[p]) < 5e-3, p


def test_qwen3_oracle_cached_matches_full(orc):
    ids = [7, 1, 30, 30, 2, 44, 19, 9]
    a = orc.Qwen3(**TINY)
    _, full = a.run(ids, 0)
    b = orc.Qwen3(**TINY)
    b.run(ids[:3], 0)
    for p in range(3, len(ids)):
        _, got = b.run([ids[p]], p)
    assert rel_rms(got, full) < 5e-3


def test_qwen3_float64_forward_catches_plausible_mistakes(orc):
    """The comparison above has teeth: the oracle's logits are far (> 5e-3) from a float64 forward
    without RoPE, and from one with the gate and up projections swapped."""
    W, E, _ = weights(orc, TINY)
    ids = [3, 17, 42, 8, 8, 0]
    m = orc.Qwen3(**TINY)
    _, got = m.run(ids, 0)
    assert rel_rms(got, forward64(TINY, W, E, ids)[-1]) < 5e-3
    assert rel_rms(got, forward64(TINY, W, E, ids, theta=1e300)[-1]) > 5e-3
    swapped = [dict(w, **{"mlp.gate_proj.weight": w["mlp.up_proj.weight"], "mlp.up_proj.weight": w["mlp.gate_proj.weight"]})
               for w in W]
    assert rel_rms(got, forward64(TINY, swapped, E, ids)[-1]) > 5e-3


def test_qwen3_oracle_set_reproduces_synthetic(orc):
    """or_qwen3_set: an oracle built with no weights (std 0) and given the synthetic checkpoint's
    dequantized linears and embedding by name computes the same logits, bit for bit, as the one
    that drew them."""
    W, E, _ = weights(orc, TINY)
    a = orc.Qwen3(**TINY)
    b = orc.Qwen3(**TINY, std=0.0)
    for i, w in enumerate(W):
        for n, v in w.items():
            b.set(f"model.layers.{i}.{n}", v.astype(np.float32))
    b.set("model.embed_tokens.weight", E.astype(np.float32))
    ids = [3, 17, 42, 8]
    ta, la = a.run(ids, 0)
    tb, lb = b.run(ids, 0)
    assert ta == tb and np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    with pytest.raises(ValueError):
        b.set("model.layers.9.input_layernorm.weight", np.ones(TINY["hidden"], np.float32))
    with pytest.raises(ValueError):
        b.set("model.norm.weight", np.ones(TINY["hidden"] + 1, np.float32))


def test_qwen3_oracle_norm_weights_match_float64_forward(orc):
    """Non-unit RMSNorm weights (input, post-attention, per-head q/k before RoPE, final), as a real
    checkpoint carries them (qwen3_test.go:155-163,196,205): the oracle against the float64 forward
    with the same weights, at the prompt's last row and at cached steps (< 5e-3). The comparison
    fails, by at least twice its bound, when the forward drops any one of the five weights or swaps
    q_norm and k_norm, so the oracle applies each where the model does."""
    W, E, _ = weights(orc, TINY)
    norms = norm_weights(TINY)
    m = orc.Qwen3(**TINY)
    for n, v in norms.items():
        m.set(n, v)
    ids = [3, 17, 42, 8, 8, 0, 49, 21]
    fn = norms["model.norm.weight"]
    want = forward64(TINY, with_norms(W, norms), E, ids, final_norm=fn)
    _, got = m.run(ids[:6], 0)
    assert rel_rms(got, want[5]) < 5e-3
    for p in range(6, len(ids)):
        _, step = m.run([ids[p]], p)
        assert rel_rms(step, want[p]) < 5e-3, p
    ref = want[-1]
    for drop in NORMS:
        assert rel_rms(step, forward64(TINY, with_norms(W, norms, drop=(drop,)), E, ids, final_norm=fn)[-1]) > 1e-2, drop
    assert rel_rms(step, forward64(TINY, with_norms(W, norms), E, ids)[-1]) > 1e-2, "model.norm.weight"
    swapped = [dict(w, **{"self_attn.q_norm.weight": w["self_attn.k_norm.weight"],
                          "self_attn.k_norm.weight": w["self_attn.q_norm.weight"]}) for w in with_norms(W, norms)]
    assert rel_rms(step, forward64(TINY, swapped, E, ids, final_norm=fn)[-1]) > 1e-2, "q/k norms swapped"
    assert rel_rms(step, ref) < 5e-3
