"""Writes the greedy-decode fixture of the synthetic 28-layer model (qwen3_c5_greedy.json) with the
CPU oracle (oracle/qwen3.c): the checkpoint of seed 0 and weight std 0.02, a 1024-token prompt of
ids uniform over the vocabulary, then 64 greedy steps. Also the weights' checksums, so that a GPU
test can tell a mismatch of the weights from one of the forward pass.

    python tests/golden/make_qwen3_golden.py [--steps 64] [--out tests/golden/qwen3_c5_greedy.json]

Takes a few minutes on 8 cores and about 8 GB of memory.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

import numpy as np  # noqa: E402

import synth_np  # noqa: E402
from oracle import oracle  # noqa: E402

C5 = dict(layers=28, hidden=2048, heads=16, kv_heads=8, head_dim=128, inter=6144, vocab=151936, max_ctx=1280)
PROMPT = 1024
PROMPT_NAME = "c5.prompt"


def prompt_tokens():
    return synth_np.uniform_int(PROMPT, 0, C5["vocab"], PROMPT_NAME).astype(np.int32)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--out", default=os.path.join(HERE, "qwen3_c5_greedy.json"))
    args = ap.parse_args()
    t0 = time.time()
    m = oracle.Qwen3(**C5, theta=1e6, eps=1e-6, seed=0, std=0.02)
    print(f"weights {time.time() - t0:.1f}s", flush=True)
    toks = prompt_tokens()
    tok, logits = m.run(toks, 0)
    print(f"prefill {time.time() - t0:.1f}s -> {tok}", flush=True)
    out, gaps = [tok], []
    for i in range(args.steps - 1):
        srt = np.sort(logits)
        gaps.append(float(srt[-1] - srt[-2]))
        tok, logits = m.run([tok], PROMPT + i)
        out.append(tok)
        if i % 8 == 0:
            print(f"step {i + 1} {time.time() - t0:.1f}s -> {tok}", flush=True)
    srt = np.sort(logits)
    gaps.append(float(srt[-1] - srt[-2]))
    doc = {
        "what": "greedy tokens of the synthetic Qwen3 (28 layers) after a 1024-token prompt, CPU oracle",
        "config": C5, "theta": 1e6, "eps": 1e-6, "seed": 0, "std": 0.02,
        "prompt": {"n": PROMPT, "name": PROMPT_NAME, "rule": "uniform ints [0, vocab), synth key c5.prompt"},
        "checksums": dict(zip(["blocks", "scales", "embed"], m.checksums())),
        "tokens": out,
        "top2_gaps": [round(g, 6) for g in gaps],
    }
    with open(args.out, "w") as f:
        json.dump(doc, f, indent=1)
    print(f"wrote {args.out} in {time.time() - t0:.1f}s", flush=True)


if __name__ == "__main__":
    main()
