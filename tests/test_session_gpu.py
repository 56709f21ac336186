"""GPU tests of the decoder session's cache and position (hwk_qwen3_export_rows / import_rows /
position / rewind / verify / keep), through libhwk's C ABI.

What each pins:
- export_rows lays the rows out as the reference's ExportRows does (internal/llm/decode/
  decode.go:1857-1881): per position, the caches kv_k_N_new / kv_v_N_new in the order of their names
  sorted as strings (decode.go:484; with 12 layers kv_k_1 comes after kv_k_10 and kv_k_11), each
  kv_heads rows of head_dim fp16. The expected bytes are gathered here in numpy from the caches
  themselves, read through hwk_qwen3_tensor.
- import_rows then rewind (Resume, decode.go:1930-1968) in a second session of the same model
  continues with the same greedy tokens and bit-identical logits as the first.
- rewind to a mark (Rewind, decode.go:1190-1203) and decoding again repeats the same tokens.
- verify (Speculate, decode.go:1235-1261) gives, for each row, the logits of the decode step at that
  position (model bar of test_qwen3_gpu) and the CPU oracle's (oracle/qwen3.c); keep moves past the
  kept rows and the decode after it continues the greedy sequence, for full and partial acceptance.
"""
import numpy as np
import pytest
import torch

import synth_np
from hwnpu_amd.qwen3 import Qwen3, d2h
from test_qwen3_gpu import check_close

pytestmark = pytest.mark.gpu

SMALL = dict(layers=2, hidden=2048, heads=16, kv_heads=8, head_dim=128, inter=6144, vocab=4096)


def expected_rows(m, cfg, start, end, max_ctx):
    """ExportRows restated on the host from the caches' bytes."""
    names = []
    for i in range(cfg["layers"]):
        names.append((f"kv_k_{i}_new", f"layers.{i}.k_cache"))
        names.append((f"kv_v_{i}_new", f"layers.{i}.v_cache"))
    names.sort(key=lambda t: t[0])
    caches = []
    for _, tname in names:
        ptr, n = m.tensor(tname)
        caches.append(d2h(ptr, n, np.uint16).reshape(cfg["kv_heads"], max_ctx, cfg["head_dim"]))
    out = []
    for p in range(start, end):
        for c in caches:
            for h in range(cfg["kv_heads"]):
                out.append(c[h, p])
    return np.concatenate(out).view(np.uint8) if out else np.zeros(0, np.uint8)


def test_export_rows_layout(dev):
    cfg = dict(SMALL, layers=12, vocab=1024)
    max_ctx = 96
    print(f"export rows {cfg}", flush=True)
    m = Qwen3(**cfg, max_ctx=max_ctx, max_prompt=64)
    try:
        m.synth(seed=3, std=0.02)
        prompt = synth_np.uniform_int(40, 0, cfg["vocab"], "t.session.export").astype(np.int32)
        m.prefill(prompt, 0)
        m.decode(5)
        assert m.row_bytes() == 2 * 12 * 8 * 128 * 2
        got = m.export_rows(5, 44).cpu().numpy()
        want = expected_rows(m, cfg, 5, 44, max_ctx)
        assert got.size == 39 * m.row_bytes()
        assert np.array_equal(got, want)
        assert m.export_rows(7, 7).numel() == 0
        from hwnpu_amd import HwkError

        with pytest.raises(HwkError):
            m.export_rows(10, max_ctx + 1)
        with pytest.raises(HwkError):
            m.import_rows(max_ctx - 1, torch.zeros(2 * m.row_bytes(), dtype=torch.uint8, device="cuda"))
        with pytest.raises(HwkError):
            m.import_rows(0, torch.zeros(m.row_bytes() + 16, dtype=torch.uint8, device="cuda"))
    finally:
        m.close()


def test_import_rows_resume_and_rewind(dev):
    max_ctx = 128
    print(f"resume {SMALL}", flush=True)
    a = Qwen3(**SMALL, max_ctx=max_ctx, max_prompt=64)
    b = Qwen3(**SMALL, max_ctx=max_ctx, max_prompt=64)
    try:
        a.synth(seed=0, std=0.02)
        b.synth(seed=0, std=0.02)
        prompt = synth_np.uniform_int(50, 0, SMALL["vocab"], "t.session.resume").astype(np.int32)
        a.prefill(prompt, 0)
        a.decode(6)
        first = [int(t) for t in a.history(51, 6)]
        saved = a.save()
        assert saved[0] == 56 and a.mark() == 56
        a.decode(8)
        toks_a = [int(t) for t in a.history(57, 8)]
        logits_a = a.logits()
        # a second session brought to the saved point continues identically
        b.resume(saved)
        assert b.position() == 56
        assert np.array_equal(b.export_rows(0, 56).cpu().numpy(), saved[1].cpu().numpy())
        b.decode(8)
        assert [int(t) for t in b.history(57, 8)] == toks_a
        assert np.array_equal(b.logits(), logits_a)
        # back to the mark in the first session: the same continuation again
        a.rewind(saved[0])
        assert a.position() == 56
        a.decode(8)
        assert [int(t) for t in a.history(57, 8)] == toks_a
        assert np.array_equal(a.logits(), logits_a)
        # rewind further back, past rows the steps since overwrote nothing before: decode from 50
        a.rewind(50)
        a.decode(4)
        assert [int(t) for t in a.history(51, 4)] == first[:4]
    finally:
        a.close()
        b.close()


@pytest.mark.parametrize("n_draft", [4, 7])
def test_verify_matches_steps_and_oracle(dev, orc, n_draft):
    max_ctx = 128
    print(f"verify {SMALL} drafts={n_draft}", flush=True)
    m = Qwen3(**SMALL, max_ctx=max_ctx, max_prompt=64)
    try:
        m.synth(seed=0, std=0.02)
        ref = orc.Qwen3(**SMALL, max_ctx=max_ctx, seed=0, std=0.02)
        prompt = synth_np.uniform_int(60, 0, SMALL["vocab"], "t.session.verify").astype(np.int32)
        m.prefill(prompt, 0)
        P = m.position()
        g = [int(m.history(P, 1)[0])]
        step_logits = []
        for _ in range(n_draft + 3):  # the sequential greedy steps
            m.step()
            step_logits.append(m.logits())
            g.append(int(m.history(m.position(), 1)[0]))
        # all drafts right: every row kept
        m.rewind(P)
        logits, am = m.verify(g[:n_draft + 1])
        ref.run(prompt, 0)
        for i in range(n_draft + 1):
            check_close(logits[i], step_logits[i], f"verify row {i} vs decode step")
            tok, want = ref.run([g[i]], P + i)
            check_close(logits[i], want, f"verify row {i} vs oracle")
            assert int(am[i]) == g[i + 1] == tok
        m.keep(n_draft + 1)
        assert m.position() == P + n_draft + 1
        assert int(m.history(P + n_draft + 1, 1)[0]) == g[n_draft + 1]
        check_close(m.logits(), step_logits[n_draft], "logits after keep")
        m.decode(2)
        assert [int(t) for t in m.history(P + n_draft + 2, 2)] == g[n_draft + 2:n_draft + 4]
        # the second draft wrong: two rows kept, the greedy sequence goes on from there
        m.rewind(P)
        wrong = (g[2] + 1) % SMALL["vocab"]
        kept, toks = m.speculate([g[1], wrong] + g[3:n_draft + 1])
        assert kept == 2 and toks == g[1:3]
        assert m.position() == P + 2 and int(m.history(P + 2, 1)[0]) == g[2]
        m.decode(3)
        assert [int(t) for t in m.history(P + 3, 3)] == g[3:6]
        # the first draft wrong: one row kept (the step's own token)
        m.rewind(P)
        kept, toks = m.speculate([(g[1] + 1) % SMALL["vocab"]])
        assert kept == 1 and toks == [g[1]]
        from hwnpu_amd import HwkError

        with pytest.raises(HwkError):
            m.keep(1)  # the verify was kept already
        with pytest.raises(HwkError):
            m.verify(list(range(9)))  # more than 8 rows
    finally:
        m.close()


def test_rewind_and_step_refuse_positions_past_the_cache(dev):
    """A rewind to 2**32 - 1 (what ctypes makes of -1 for the uint32 argument) is refused by the
    library before any launch, as is every position without room for a step; the session stays
    usable afterwards."""
    from hwnpu_amd import HwkError, hwk
    from hwnpu_amd.ops import _stream

    m = Qwen3(**dict(SMALL, layers=1, vocab=512), max_ctx=32, max_prompt=16)
    try:
        m.synth(seed=0, std=0.02)
        m.prefill(np.arange(8, dtype=np.int32), 0)
        for bad in (0xFFFFFFFF, 0xFFFFFFFE, 31, 32):
            with pytest.raises(HwkError):
                hwk.load().hwk_qwen3_rewind(m._h, _stream(), bad, -1)
        with pytest.raises(ValueError):
            m.rewind(-1)
        assert m.position() == 8
        m.rewind(30)
        m.step()  # position 30 -> 31, the last
        with pytest.raises(HwkError):
            m.step()
        m.rewind(4)
        m.step()
        assert m.position() == 5
    finally:
        m.close()
