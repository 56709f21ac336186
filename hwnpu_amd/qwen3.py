"""The device-resident Qwen3 decoder of libhwk (hwk_qwen3_*), as a Python session.

The shape of the reference's device session (internal/llm/iron/model.go:578, Step(token, pos) ->
logits; internal/chat/session.go:9-31, StepTokens): weights, KV cache, token history and
position live on the GPU. ``prefill`` runs a prompt; ``step`` runs one greedy decode step
eagerly; ``decode`` replays the captured step graph. Device state is read back with
``hipMemcpy`` through libamdhip64, the way a purego binding reads it.
"""
from __future__ import annotations

import ctypes as C
import struct

import numpy as np
import torch

from . import hwk
from .ops import _stream, f32_bits

_hip = None


def _hiprt():
    global _hip
    if _hip is None:
        lib = C.CDLL("libamdhip64.so")
        lib.hipMemcpy.restype = C.c_int
        lib.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        _hip = lib
    return _hip


def d2h(ptr: int, nbytes: int, dtype) -> np.ndarray:
    """A synchronous copy of device memory at ptr into a new host array."""
    out = np.empty(nbytes // np.dtype(dtype).itemsize, dtype)
    torch.cuda.current_stream().synchronize()
    rc = _hiprt().hipMemcpy(out.ctypes.data_as(C.c_void_p), C.c_void_p(ptr), nbytes, 2)  # device to host
    if rc != 0:
        raise hwk.HwkError(f"hipMemcpy device to host: error {rc}")
    return out


def d2d(dst: int, src: int, nbytes: int) -> None:
    torch.cuda.current_stream().synchronize()
    rc = _hiprt().hipMemcpy(C.c_void_p(dst), C.c_void_p(src), nbytes, 3)  # device to device
    if rc != 0:
        raise hwk.HwkError(f"hipMemcpy device to device: error {rc}")


def _f64_bits(v: float) -> int:
    return struct.unpack("<Q", struct.pack("<d", float(v)))[0]


C5 = dict(layers=28, hidden=2048, heads=16, kv_heads=8, head_dim=128, inter=6144, vocab=151936)


class Qwen3:
    def __init__(self, layers=28, hidden=2048, heads=16, kv_heads=8, head_dim=128, inter=6144, vocab=151936,
                 max_ctx=1280, max_prompt=1024, theta=1e6, eps=1e-6):
        c = hwk.Qwen3Config()
        c.layers, c.hidden, c.heads, c.kv_heads, c.head_dim = layers, hidden, heads, kv_heads, head_dim
        c.inter, c.vocab, c.max_ctx, c.max_prompt = inter, vocab, max_ctx, max_prompt
        c.theta_bits, c.eps_bits = _f64_bits(theta), _f64_bits(eps)
        self.cfg = c
        self.vocab, self.max_ctx = vocab, max_ctx
        h = C.c_void_p()
        hwk.load().hwk_qwen3_new(C.byref(c), C.byref(h))
        self._h = h
        lg, hist, pos = C.c_void_p(), C.c_void_p(), C.c_void_p()
        hwk.load().hwk_qwen3_state(h, C.byref(lg), C.byref(hist), C.byref(pos))
        self._logits, self._hist, self._pos = lg.value, hist.value, pos.value

    def close(self):
        if getattr(self, "_h", None):
            torch.cuda.synchronize()
            hwk.load().hwk_qwen3_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def synth(self, seed=0, std=0.02):
        hwk.load().hwk_qwen3_synth(self._h, _stream(), seed, f32_bits(std))

    def tensor(self, name: str):
        """(device pointer, bytes) of a weight in libhwk's layout."""
        ptr, n = C.c_void_p(), C.c_size_t()
        hwk.load().hwk_qwen3_tensor(self._h, name.encode(), C.byref(ptr), C.byref(n))
        return ptr.value, n.value

    def prefill(self, tokens, start=0):
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        hwk.load().hwk_qwen3_prefill(self._h, _stream(), toks.ctypes.data_as(C.POINTER(C.c_int32)), toks.size, start)

    def step(self):
        hwk.load().hwk_qwen3_step(self._h, _stream())

    def decode(self, steps: int):
        hwk.load().hwk_qwen3_decode(self._h, _stream(), steps)

    def capture(self):
        """Captures both step graphs now (no replay), so that decode() afterwards only replays."""
        hwk.load().hwk_qwen3_capture(self._h)

    def logits(self) -> np.ndarray:
        return d2h(self._logits, 4 * self.vocab, np.float32)

    def pos(self) -> int:
        return int(d2h(self._pos, 4, np.int32)[0])

    def history(self, start: int, n: int) -> np.ndarray:
        """Tokens at positions start .. start+n-1."""
        return d2h(self._hist + 4 * start, 4 * n, np.int32)

    def checksums(self):
        """Sums of every linear's code bytes, of their scale bytes, and of the embedding's fp16 bits
        (the oracle's or_qwen3_checksums)."""
        sb = ss = 0
        for i in range(self.cfg.layers):
            for lin in ("qkv", "o", "gate_up", "down"):
                for part in ("blocks", "scales"):
                    ptr, n = self.tensor(f"layers.{i}.{lin}.{part}")
                    t = torch.empty(n, dtype=torch.uint8, device="cuda")
                    d2d(t.data_ptr(), ptr, n)
                    v = int(t.to(torch.int64).sum().item())
                    if part == "blocks":
                        sb += v
                    else:
                        ss += v
        ptr, n = self.tensor("embed")
        t = torch.empty(n // 2, dtype=torch.int16, device="cuda")
        d2d(t.data_ptr(), ptr, n)
        se = int((t.to(torch.int64) & 0xFFFF).sum().item())
        return [sb, ss, se]
