"""GPU tests of the checkpoint loaders (hwnpu_amd.checkpoint): safetensors files written here, loaded
into libhwk's device layouts, checked against the CPU oracle or against the model they came from.

- An MXFP4 checkpoint of a synthetic decoder (blocks/scales per linear, the gpt-oss convention)
  loads into a fresh model with the same weight checksums and the same greedy tokens.
- A float checkpoint (F32 and BF16 linears, Hugging Face names) is encoded on the device to MXFP4
  bit-exactly as the oracle's Encode (internal/mxfp4/encode.go:11-78) encodes it, into the stacked
  q/k/v and interleaved gate/up layout; norms and the fp16 embedding land as they are. The loaded
  model, whose RMSNorm weights are N(1, 0.1), then runs against the oracle given the same tensors.
- gpt-oss-named experts with BF16 biases (internal/llm/gptoss/config.go:193-194) run through
  hwk_moe_layer with the gpt-oss unit and match the oracle on the same arrays.
"""
import numpy as np
import pytest
import torch

import synth_np
from hwnpu_amd import checkpoint, ops, synth
from hwnpu_amd.qwen3 import Qwen3, d2h
from test_moe_gpu import check_close, experts_case

pytestmark = pytest.mark.gpu

SMALL = dict(layers=2, hidden=2048, heads=16, kv_heads=8, head_dim=128, inter=6144, vocab=4096)


def dev_bytes(m, name, dtype=np.uint8):
    ptr, n = m.tensor(name)
    return d2h(ptr, n, dtype)


def test_qwen3_mxfp4_checkpoint_round_trip(dev, tmp_path):
    cfg = SMALL
    hd = cfg["head_dim"]
    qn, kn, nb = cfg["heads"] * hd, cfg["kv_heads"] * hd, cfg["hidden"] // 32
    a = Qwen3(**cfg, max_ctx=96, max_prompt=64)
    b = Qwen3(**cfg, max_ctx=96, max_prompt=64)
    try:
        a.synth(seed=5, std=0.02)
        t = {}
        for i in range(cfg["layers"]):
            p = f"model.layers.{i}."
            qkv_w = dev_bytes(a, f"layers.{i}.qkv.blocks").reshape(-1, nb, 16)
            qkv_e = dev_bytes(a, f"layers.{i}.qkv.scales").reshape(-1, nb)
            for name, lo, hi in (("q", 0, qn), ("k", qn, qn + kn), ("v", qn + kn, qn + 2 * kn)):
                t[p + f"self_attn.{name}_proj_blocks"] = ("U8", qkv_w[lo:hi])
                t[p + f"self_attn.{name}_proj_scales"] = ("U8", qkv_e[lo:hi])
            t[p + "self_attn.o_proj_blocks"] = ("U8", dev_bytes(a, f"layers.{i}.o.blocks").reshape(-1, qn // 32, 16))
            t[p + "self_attn.o_proj_scales"] = ("U8", dev_bytes(a, f"layers.{i}.o.scales").reshape(-1, qn // 32))
            gw = dev_bytes(a, f"layers.{i}.gate_up.blocks").reshape(-1, nb, 16)
            ge = dev_bytes(a, f"layers.{i}.gate_up.scales").reshape(-1, nb)
            t[p + "mlp.gate_proj_blocks"], t[p + "mlp.gate_proj_scales"] = ("U8", gw[0::2]), ("U8", ge[0::2])
            t[p + "mlp.up_proj_blocks"], t[p + "mlp.up_proj_scales"] = ("U8", gw[1::2]), ("U8", ge[1::2])
            ni = cfg["inter"] // 32
            t[p + "mlp.down_proj_blocks"] = ("U8", dev_bytes(a, f"layers.{i}.down.blocks").reshape(-1, ni, 16))
            t[p + "mlp.down_proj_scales"] = ("U8", dev_bytes(a, f"layers.{i}.down.scales").reshape(-1, ni))
            for hf, mine in (("input_layernorm.weight", "input_norm"), ("post_attention_layernorm.weight", "post_norm"),
                             ("self_attn.q_norm.weight", "q_norm"), ("self_attn.k_norm.weight", "k_norm")):
                t[p + hf] = ("F32", dev_bytes(a, f"layers.{i}.{mine}", np.float32))
        t["model.norm.weight"] = ("F32", dev_bytes(a, "norm", np.float32))
        t["model.embed_tokens.weight"] = ("F16", dev_bytes(a, "embed", np.float16).reshape(cfg["vocab"], -1))
        path = str(tmp_path / "model.safetensors")
        checkpoint.write_safetensors(path, t, {"format": "hwnpu-mxfp4"})
        with checkpoint.Checkpoint(path) as ck:
            checkpoint.load_qwen3(b, ck)
        assert b.checksums() == a.checksums()
        prompt = synth_np.uniform_int(30, 0, cfg["vocab"], "t.ckpt.prompt").astype(np.int32)
        for m in (a, b):
            m.prefill(prompt, 0)
            m.decode(6)
        assert list(a.history(30, 7)) == list(b.history(30, 7))
        assert np.array_equal(a.logits(), b.logits())
    finally:
        a.close()
        b.close()


LINEARS = ("self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight", "self_attn.o_proj.weight",
           "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight")


def float_checkpoint(cfg, path, seed=9, norm_sd=0.1):
    """A float Qwen3 checkpoint under Hugging Face names: linears N(0, 0.02) (F32, or BF16 for every
    other one), every RMSNorm weight N(1, norm_sd) (input, post-attention, q/k per head, final), an
    F32 embedding. Returns the values the loader sees: {name: float32 array}."""
    hd = cfg["head_dim"]
    qn, kn, H, I = cfg["heads"] * hd, cfg["kv_heads"] * hd, cfg["hidden"], cfg["inter"]
    shapes = dict(zip(LINEARS, ((qn, H), (kn, H), (kn, H), (H, qn), (I, H), (I, H), (H, I))))
    rng = np.random.default_rng(seed)
    t, vals = {}, {}
    for i in range(cfg["layers"]):
        p = f"model.layers.{i}."
        for j, name in enumerate(LINEARS):
            x = (rng.standard_normal(shapes[name]) * 0.02).astype(np.float32)
            if j % 2:  # BF16 for half of them: the values the loader sees are the bf16 ones
                bits = (x.view(np.uint32) >> 16).astype(np.uint16)
                t[p + name] = ("BF16", bits)
                x = (bits.astype(np.uint32) << 16).view(np.float32)
            else:
                t[p + name] = ("F32", x)
            vals[p + name] = x
        for n, size in (("input_layernorm.weight", H), ("post_attention_layernorm.weight", H),
                        ("self_attn.q_norm.weight", hd), ("self_attn.k_norm.weight", hd)):
            v = (rng.standard_normal(size) * norm_sd + 1).astype(np.float32)
            t[p + n], vals[p + n] = ("F32", v), v
    v = (rng.standard_normal(H) * norm_sd + 1).astype(np.float32)
    t["model.norm.weight"], vals["model.norm.weight"] = ("F32", v), v
    emb = (rng.standard_normal((cfg["vocab"], H)) * 0.02).astype(np.float32)
    t["model.embed_tokens.weight"], vals["model.embed_tokens.weight"] = ("F32", emb), emb
    checkpoint.write_safetensors(path, t)
    return vals


def test_qwen3_float_checkpoint_encodes_like_oracle(dev, orc, tmp_path):
    cfg = dict(SMALL, layers=1, vocab=512)
    path = str(tmp_path / "float.safetensors")
    vals = float_checkpoint(cfg, path)
    m = Qwen3(**cfg, max_ctx=64, max_prompt=32)
    try:
        with checkpoint.Checkpoint(path) as ck:
            checkpoint.load_qwen3(m, ck)
        p = "model.layers.0."
        enc = {n: orc.mxfp4_encode(vals[p + n]) for n in LINEARS}
        qkv_w = np.concatenate([enc[f"self_attn.{x}_proj.weight"][0] for x in "qkv"])
        qkv_e = np.concatenate([enc[f"self_attn.{x}_proj.weight"][1] for x in "qkv"])
        assert np.array_equal(dev_bytes(m, "layers.0.qkv.blocks"), qkv_w.reshape(-1))
        assert np.array_equal(dev_bytes(m, "layers.0.qkv.scales"), qkv_e.reshape(-1))
        gw = np.stack([enc["mlp.gate_proj.weight"][0], enc["mlp.up_proj.weight"][0]], 1)
        ge = np.stack([enc["mlp.gate_proj.weight"][1], enc["mlp.up_proj.weight"][1]], 1)
        assert np.array_equal(dev_bytes(m, "layers.0.gate_up.blocks"), gw.reshape(-1))
        assert np.array_equal(dev_bytes(m, "layers.0.gate_up.scales"), ge.reshape(-1))
        for name, mine in (("self_attn.o_proj.weight", "o"), ("mlp.down_proj.weight", "down")):
            assert np.array_equal(dev_bytes(m, f"layers.0.{mine}.blocks"), enc[name][0].reshape(-1))
            assert np.array_equal(dev_bytes(m, f"layers.0.{mine}.scales"), enc[name][1].reshape(-1))
        for hf, mine in (("input_layernorm.weight", "input_norm"), ("post_attention_layernorm.weight", "post_norm"),
                         ("self_attn.q_norm.weight", "q_norm"), ("self_attn.k_norm.weight", "k_norm")):
            assert np.array_equal(dev_bytes(m, f"layers.0.{mine}", np.float32), vals[p + hf])
        assert np.array_equal(dev_bytes(m, "norm", np.float32), vals["model.norm.weight"])
        assert np.array_equal(dev_bytes(m, "embed", np.uint16), orc.f32_to_f16(vals["model.embed_tokens.weight"]).reshape(-1))
    finally:
        m.close()


# max_ctx past 16384 takes the decode step's split attention with a separate merge
@pytest.mark.parametrize("max_ctx", [160, 16500])
def test_qwen3_float_checkpoint_runs_like_oracle(dev, orc, tmp_path, max_ctx):
    """A checkpoint-loaded model with real (non-unit) RMSNorm weights, run end to end against the
    oracle given the same tensors (the linears as the oracle's Encode then Dequantize of the file's
    values, which the device encoding matches bit for bit above): the prompt (RMSNorm kernel, the
    prompt's per-head q/k norm + RoPE), eager steps and graph replays (the norm folded into the qkv
    and gate_up GEMVs, q/k norms in the decode attention's prologue, the final norm), and a verify
    of three rows. Greedy tokens identical, logits within the model bar (test_qwen3_gpu)."""
    from test_qwen3_gpu import check_close

    cfg = dict(SMALL)
    path = str(tmp_path / "float.safetensors")
    vals = float_checkpoint(cfg, path, seed=21)
    print(f"float checkpoint {cfg} max_ctx={max_ctx}", flush=True)
    m = Qwen3(**cfg, max_ctx=max_ctx, max_prompt=64)
    try:
        with checkpoint.Checkpoint(path) as ck:
            checkpoint.load_qwen3(m, ck)
        ref = orc.Qwen3(**cfg, max_ctx=max_ctx, std=0.0)
        for name, v in vals.items():
            if name.endswith("_proj.weight"):
                v = orc.mxfp4_dequantize(*orc.mxfp4_encode(v)).astype(np.float32)
            ref.set(name, v)
        prompt = synth_np.uniform_int(60, 0, cfg["vocab"], "t.ckpt.float.prompt").astype(np.int32)
        m.prefill(prompt, 0)
        tok, want = ref.run(prompt, 0)
        check_close(m.logits(), want, "prefill logits")
        assert m.history(60, 1)[0] == tok
        pos = 60
        for i in range(3):
            m.step()
            tok, want = ref.run([tok], pos)
            check_close(m.logits(), want, f"step {i} logits")
            pos += 1
            assert m.history(pos, 1)[0] == tok, f"step {i}"
        m.decode(8)
        want_toks = []
        for i in range(8):
            tok, want = ref.run([tok], pos + i)
            want_toks.append(tok)
        check_close(m.logits(), want, "graph step logits")
        assert [int(t) for t in m.history(pos + 1, 8)] == want_toks
        pos += 8
        rows = [tok, 5, 77]
        lg, am = m.verify(rows)
        for j, t in enumerate(rows):
            wt, want = ref.run([t], pos + j)
            check_close(lg[j], want, f"verify row {j}")
            assert int(am[j]) == wt, f"verify row {j}"
    finally:
        m.close()


def test_gptoss_experts_checkpoint(dev, orc, tmp_path):
    T, E, H, I = 3, 32, 2048, 768
    x, logits, gw, ge, dw, de = experts_case(T, E, H, I, name="ck.e")
    rng = np.random.default_rng(4)
    gb = (rng.standard_normal((E, 2 * I)) * 0.1).astype(np.float32)
    db = (rng.standard_normal((E, H)) * 0.1).astype(np.float32)
    gbb = (gb.view(np.uint32) >> 16).astype(np.uint16)  # BF16 biases, as gpt-oss ships them
    dbb = (db.view(np.uint32) >> 16).astype(np.uint16)
    pre = "model.layers.7.mlp.experts."
    names = checkpoint.expert_names(pre)
    path = str(tmp_path / "experts.safetensors")
    checkpoint.write_safetensors(path, {names["gate_up_blocks"]: ("U8", gw.cpu().numpy()),
                                        names["gate_up_scales"]: ("U8", ge.cpu().numpy()),
                                        names["gate_up_bias"]: ("BF16", gbb),
                                        names["down_blocks"]: ("U8", dw.cpu().numpy()),
                                        names["down_scales"]: ("U8", de.cpu().numpy()),
                                        names["down_bias"]: ("BF16", dbb)})
    with checkpoint.Checkpoint(path) as ck:
        ex = checkpoint.load_experts(ck, names)
    for k, v in (("gu_w", gw), ("gu_e", ge), ("dn_w", dw), ("dn_e", de)):
        assert torch.equal(ex[k], v)
    out, idx, w = ops.moe_layer(x, logits, 4, ex["gu_w"], ex["gu_e"], ex["dn_w"], ex["dn_e"], gu_b=ex["gu_b"],
                                dn_b=ex["dn_b"], act="gptoss", alpha=1.702, limit=7.0)
    gbf = (gbb.astype(np.uint32) << 16).view(np.float32)
    dbf = (dbb.astype(np.uint32) << 16).view(np.float32)
    want = orc.experts(x.cpu().numpy().astype(np.float32), idx.cpu().numpy(), w.cpu().numpy(), gw.cpu().numpy(),
                       ge.cpu().numpy(), dw.cpu().numpy(), de.cpu().numpy(), gu_b=gbf, dn_b=dbf, act="gptoss")
    check_close(out.cpu().numpy(), want)
    # a record naming no biases runs without them
    nob = dict(names, gate_up_bias="", down_bias="")
    with checkpoint.Checkpoint(path) as ck:
        assert checkpoint.load_experts(ck, nob)["gu_b"] is None
    bad = dict(names, down_blocks=pre + "missing")
    with checkpoint.Checkpoint(path) as ck, pytest.raises(checkpoint.CheckpointError):
        checkpoint.load_experts(ck, bad)


def test_synth_reference_matches_oracle(dev, orc):
    """hwk_synth_reference (the reference's llm.Synthetic values) against the oracle's sequential
    generator, bit for bit, across lengths that cross the device's 64-element runs."""
    for name, n in (("model.embed_tokens.weight", 1_000_003), ("x", 1), ("model.layers.0.self_attn.q_proj.weight", 130)):
        want = orc.synth_reference(name, n)
        got = synth.reference(name, n).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), name
        g16 = synth.reference(name, n, torch.float16).cpu().numpy()
        assert np.array_equal(g16.view(np.uint16), orc.f32_to_f16(want)), name
