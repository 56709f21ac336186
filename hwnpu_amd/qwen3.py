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
        lib.hipMemcpy2D.restype = C.c_int
        lib.hipMemcpy2D.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t, C.c_size_t, C.c_size_t, C.c_int]
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


def h2d(dst: int, a: np.ndarray) -> None:
    """A synchronous copy of a C-contiguous host array (a read-only view of a mapped file is fine) into
    device memory at dst."""
    if not a.flags.c_contiguous:
        raise ValueError("h2d: a C-contiguous array")
    torch.cuda.current_stream().synchronize()
    rc = _hiprt().hipMemcpy(C.c_void_p(dst), C.c_void_p(a.ctypes.data), a.nbytes, 1)  # host to device
    if rc != 0:
        raise hwk.HwkError(f"hipMemcpy host to device: error {rc}")


def copy_rows(dst: int, dst_pitch: int, src: int, src_pitch: int, width: int, rows: int, kind: int) -> None:
    """rows rows of width bytes, src_pitch apart at src, into rows dst_pitch apart at dst
    (hipMemcpy2D; kind 1 host to device, 3 device to device), synchronously."""
    torch.cuda.current_stream().synchronize()
    rc = _hiprt().hipMemcpy2D(C.c_void_p(dst), dst_pitch, C.c_void_p(src), src_pitch, width, rows, kind)
    if rc != 0:
        raise hwk.HwkError(f"hipMemcpy2D: error {rc}")


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

    # ---- the session's cache and position (reference decode.Session, internal/llm/decode/decode.go) ----

    def row_bytes(self) -> int:
        """Bytes of one position's rows in export_rows (RowBytes, decode.go:1849-1855)."""
        n = C.c_size_t()
        hwk.load().hwk_qwen3_row_bytes(self._h, C.byref(n))
        return n.value

    def export_rows(self, start: int, end: int) -> torch.Tensor:
        """The cache rows of positions [start, end) packed as ExportRows packs them (decode.go:1857-1881),
        a uint8 tensor on the GPU of (end - start) * row_bytes() bytes."""
        out = torch.empty(max(end - start, 0) * self.row_bytes(), dtype=torch.uint8, device="cuda")
        hwk.load().hwk_qwen3_export_rows(self._h, _stream(), start, end, out.data_ptr())
        return out

    def import_rows(self, start: int, rows: torch.Tensor) -> None:
        """Writes rows from export_rows at positions start on (ImportRows, decode.go:1883-1914)."""
        if rows.dtype != torch.uint8 or not rows.is_cuda or not rows.is_contiguous():
            raise ValueError("rows: a contiguous uint8 tensor on the GPU")
        hwk.load().hwk_qwen3_import_rows(self._h, _stream(), start, rows.data_ptr(), rows.numel())

    def position(self) -> int:
        """The position the next step takes (a Mark of the sequence, decode.go:1120-1137)."""
        p = C.c_uint32()
        hwk.load().hwk_qwen3_position(self._h, C.byref(p))
        return p.value

    def mark(self) -> int:
        return self.position()

    def rewind(self, pos: int, next_token: int = -1) -> None:
        """Back to a mark (Rewind, decode.go:1190-1203); next_token >= 0 is written as the token the
        next step takes."""
        if not 0 <= pos < 2 ** 32:
            raise ValueError(f"rewind: position {pos} is not a cache position")
        hwk.load().hwk_qwen3_rewind(self._h, _stream(), pos, next_token)

    def save(self):
        """A mark with the rows before it and the token the next step takes (Save, decode.go:1180-1188)."""
        pos = self.position()
        return pos, self.export_rows(0, pos), int(self.history(pos, 1)[0])

    def resume(self, saved) -> None:
        """Brings the sequence to a saved point, in this session or another of the same model (Resume,
        decode.go:1930-1968)."""
        pos, rows, tok = saved
        if rows.numel() != pos * self.row_bytes():
            raise ValueError(f"{rows.numel()} bytes of rows for a mark at {pos}, want {pos * self.row_bytes()}")
        self.import_rows(0, rows)
        self.rewind(pos, tok)

    def verify(self, tokens):
        """Runs tokens (the next step's token, then drafts; at most 8) at the next positions and
        returns the logits after each (fp32 (n, vocab)) and each row's greedy token; the position
        moves only with keep()."""
        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        lg, am = C.c_void_p(), C.c_void_p()
        hwk.load().hwk_qwen3_verify(self._h, _stream(), toks.ctypes.data_as(C.POINTER(C.c_int32)), toks.size,
                                    C.byref(lg), C.byref(am))
        n = toks.size
        return d2h(lg.value, 4 * n * self.vocab, np.float32).reshape(n, self.vocab), d2h(am.value, 4 * n, np.int32)

    def keep(self, kept: int) -> None:
        hwk.load().hwk_qwen3_keep(self._h, _stream(), kept)

    def speculate(self, drafts):
        """Greedy speculative decoding (Speculate, decode.go:1235-1261): verifies the next step's token
        followed by the drafts, keeps the rows whose draft is the greedy token of the row before, and
        returns (kept, the greedy tokens of the rows up to the last kept)."""
        pos = self.position()
        first = int(self.history(pos, 1)[0])
        toks = [first] + [int(t) for t in drafts]
        _, am = self.verify(toks)
        kept = 1
        while kept < len(toks) and int(am[kept - 1]) == toks[kept]:
            kept += 1
        self.keep(kept)
        return kept, [int(t) for t in am[:kept]]

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
