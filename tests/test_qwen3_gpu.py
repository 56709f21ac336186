"""GPU parity of the device-resident Qwen3 decoder (hwk_qwen3_*) against the CPU oracle's forward
(oracle/qwen3.c) on the same synthetic checkpoint, through libhwk's C ABI.

Bar (model level): greedy tokens identical at every checked position, and the
full 28-layer model's first 64 greedy tokens after a 1024-token prompt equal to the oracle's
(committed fixture tests/golden/qwen3_c5_greedy.json, written by tests/golden/make_qwen3_golden.py).

The logits are compared with the reference's model-level metric, the relative RMS error
(internal/llm/qwen3/qwen3_test.go:225-234), at the bound of its cached-vs-full check (5e-3,
cache_test.go:187-213), plus max|d| <= 1e-2 * RMS. The kernel-level bar (max|d| <= 2e-3 * RMS) holds
for every kernel on its own (test_gemv_gpu, test_gemm_gpu, test_attn_gpu) but not for a whole
model that stores activations in fp16: the oracle itself moves by max|d| = 2.3e-3 * RMS (relative
RMS 6e-4) on the 2-layer model when every linear's fp32 output is perturbed by one ulp, since a
one-ulp change flips some fp16 roundings downstream.
"""
import json
import os

import numpy as np
import pytest
import torch

import synth_np
from hwnpu_amd.qwen3 import Qwen3

pytestmark = pytest.mark.gpu

REL_RMS, MAX_REL = 5e-3, 1e-2
HERE = os.path.dirname(os.path.abspath(__file__))


def check_close(got, want, what):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    rms = float(np.sqrt(np.mean(want ** 2)))
    rel = float(np.sqrt(np.mean((got - want) ** 2))) / rms
    err = float(np.max(np.abs(got - want)))
    print(f"{what}: rel rms {rel:.3g}, max|d|/rms {err / rms:.3g}", flush=True)
    assert rel <= REL_RMS and err <= MAX_REL * rms, f"{what}: rel rms {rel:.4g}, max|d|={err:.4g} rms={rms:.4g}"


SMALL = dict(layers=2, hidden=2048, heads=16, kv_heads=8, head_dim=128, inter=6144, vocab=4096)


# max_ctx past 16384 takes the split attention with a separate merge instead of attn_head
@pytest.mark.parametrize("heads,kv_heads,max_prompt,max_ctx", [(16, 8, 64, 192), (8, 8, 128, 192), (16, 4, 48, 192),
                                                               (16, 8, 64, 16500)])
def test_qwen3_small_matches_oracle(dev, orc, heads, kv_heads, max_prompt, max_ctx):
    cfg = dict(SMALL, heads=heads, kv_heads=kv_heads)
    print(f"qwen3 small {cfg} max_prompt={max_prompt} max_ctx={max_ctx}", flush=True)
    m = Qwen3(**cfg, max_ctx=max_ctx, max_prompt=max_prompt)
    m.synth(seed=0, std=0.02)
    ref = orc.Qwen3(**cfg, max_ctx=max_ctx, seed=0, std=0.02)
    assert m.checksums() == ref.checksums()
    prompt = synth_np.uniform_int(100, 0, cfg["vocab"], "t.qwen3.prompt").astype(np.int32)
    m.prefill(prompt, 0)
    want_tok, want = ref.run(prompt, 0)
    check_close(m.logits(), want, "prefill logits")
    assert m.pos() == 100
    assert m.history(100, 1)[0] == want_tok
    pos, tok = 100, want_tok
    for i in range(6):  # eager steps, each checked against the oracle's step at that position
        m.step()
        want_tok, want = ref.run([tok], pos)
        check_close(m.logits(), want, f"step {i} logits")
        pos += 1
        assert m.pos() == pos
        assert m.history(pos, 1)[0] == want_tok, f"step {i}"
        tok = want_tok
    m.decode(10)  # graph replays
    got = m.history(pos + 1, 10)
    want_toks = []
    for i in range(10):
        tok, want = ref.run([tok], pos + i)
        want_toks.append(tok)
    check_close(m.logits(), want, "graph step logits")
    assert list(got) == want_toks
    assert m.pos() == pos + 10
    m.close()


def test_qwen3_rejects_bad_input(dev):
    m = Qwen3(**SMALL, max_ctx=64, max_prompt=32)
    m.synth()
    from hwnpu_amd import HwkError

    with pytest.raises(HwkError):
        m.step()  # no prompt yet
    with pytest.raises(HwkError):
        m.prefill([SMALL["vocab"]], 0)  # token past the vocabulary
    with pytest.raises(HwkError):
        m.prefill(np.zeros(64, np.int32), 0)  # no room left in the cache
    m.prefill(np.arange(10, dtype=np.int32), 0)
    with pytest.raises(HwkError):
        m.decode(60)  # past max_ctx
    with pytest.raises(HwkError):
        m.prefill([1, 2], 20)  # past the cached positions
    m.close()


def test_qwen3_c5_greedy_64(dev):
    """The headline model configuration: 28 layers, prompt 1024, 64 greedy tokens == the oracle's. The
    fixture's prompt was chosen (before any GPU run) so that every step's oracle top-2 logit gap is at
    least 0.008, above the largest margin change measured between two fp32 summation orders of the
    GPU's decode (5.5e-3); a step closer than that would test the summation order, not the model."""
    with open(os.path.join(HERE, "golden", "qwen3_c5_greedy.json")) as f:
        gold = json.load(f)
    assert min(gold["top2_gaps"]) >= 0.008
    c = gold["config"]
    print(f"qwen3 c5 {c}", flush=True)
    m = Qwen3(**{k: c[k] for k in ("layers", "hidden", "heads", "kv_heads", "head_dim", "inter", "vocab")},
              max_ctx=c["max_ctx"], max_prompt=1024, theta=gold["theta"], eps=gold["eps"])
    m.synth(seed=gold["seed"], std=gold["std"])
    assert m.checksums() == [gold["checksums"][k] for k in ("blocks", "scales", "embed")]
    prompt = synth_np.uniform_int(gold["prompt"]["n"], 0, c["vocab"], gold["prompt"]["name"]).astype(np.int32)
    m.prefill(prompt, 0)
    n = len(gold["tokens"])
    m.decode(n - 1)
    got = [int(t) for t in m.history(gold["prompt"]["n"], n)]
    if got != gold["tokens"]:
        first = next(i for i, (a, b) in enumerate(zip(got, gold["tokens"])) if a != b)
        pytest.fail(f"first diverging step {first}: got {got[first]} want {gold['tokens'][first]}, "
                    f"oracle top-2 gap there {gold['top2_gaps'][first]}")
    m.close()


def test_decode_argmax_ties_and_nan(dev):
    """The decode step's greedy pick (the step graph's own argmax kernel) through the model: strict >
    from index 0 (internal/chat/sample.go:80-87), so a tie goes to the lowest index and a NaN never
    wins except at index 0, where the reference keeps it. Rows of the tied embedding are edited on the
    device to make the logits tie or hold NaN; the inputs never use an edited row (the table is also
    the input embedding), and the same position is stepped again after a rewind."""
    from hwnpu_amd.qwen3 import d2d, d2h

    cfg = dict(SMALL, layers=1, vocab=1024)
    H, V = cfg["hidden"], cfg["vocab"]
    m = Qwen3(**cfg, max_ctx=96, max_prompt=64)
    try:
        m.synth(seed=1, std=0.02)
        ptr, nbytes = m.tensor("embed")
        table = d2h(ptr, nbytes, np.uint16).reshape(V, H)

        def put_row(r, row):
            t = torch.from_numpy(np.ascontiguousarray(row, dtype=np.uint16)).cuda()
            d2d(ptr + r * H * 2, t.data_ptr(), H * 2)

        prompt = np.arange(200, 240, dtype=np.int32)
        m.prefill(prompt, 0)
        P = m.position()
        t0 = int(m.history(P, 1)[0])
        used = set(prompt.tolist()) | {t0}

        def pick():
            m.rewind(P)
            m.step()
            return int(m.history(P + 1, 1)[0]), m.logits()

        a, logits = pick()
        assert a == int(np.argmax(logits)), "the step's token is the first index of the largest logit"
        free = [r for r in range(V) if r not in used and r != a]
        # a tie with a later row: the lower index (a) stays
        b = next(r for r in free if r > a)
        put_row(b, table[a])
        tok, lg = pick()
        assert lg[a] == lg[b] and tok == a, (a, b, tok)
        put_row(b, table[b])
        # a tie with an earlier row: the earlier one wins
        below = [r for r in free if 0 < r < a]
        if below:
            c = below[0]
            put_row(c, table[a])
            tok, lg = pick()
            assert lg[a] == lg[c] and tok == c, (a, c, tok)
            put_row(c, table[c])
        # a NaN logit away from index 0 never wins
        d = next(r for r in free if r > 0)
        put_row(d, np.full(H, 0x7E00, np.uint16))
        tok, lg = pick()
        assert np.isnan(lg[d]) and tok == a, (d, tok)
        put_row(d, table[d])
        # a NaN at index 0 is kept
        if 0 not in used:
            put_row(0, np.full(H, 0x7E00, np.uint16))
            tok, lg = pick()
            assert np.isnan(lg[0]) and tok == 0, tok
            put_row(0, table[0])
        tok, _ = pick()
        assert tok == a
    finally:
        m.close()
