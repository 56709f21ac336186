"""The hot-path ops on torch tensors, each a call through libhwk's C ABI.

torch supplies device memory and the stream (its current stream); every computation is one of
libhwk's HIP kernels. Shapes, dtypes and devices are checked here before any launch, so that a
kernel never sees operands that disagree with its grid. Nothing falls back to the CPU: without
libhwk or a GPU, every op raises.
"""
from __future__ import annotations

import struct

import torch

from . import hwk

OUT_MODES = {"f32": hwk.OUT_F32, "f16": hwk.OUT_F16, "add": hwk.OUT_ADD_F32}


def f32_bits(v: float) -> int:
    """A float32 scalar as the uint32 bit pattern the ABI takes."""
    return struct.unpack("<I", struct.pack("<f", float(v)))[0]


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _need(t: torch.Tensor, name: str, dtype, shape=None):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a tensor")
    if not t.is_cuda:
        raise ValueError(f"{name}: must be on the GPU (no CPU path)")
    if t.dtype != dtype:
        raise TypeError(f"{name}: dtype {t.dtype}, want {dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: shape {tuple(t.shape)}, want {tuple(shape)}")


def _out(y, n, mode, device):
    dt = torch.float16 if mode == "f16" else torch.float32
    if y is None:
        if mode == "add":
            raise ValueError("out_mode 'add' needs y")
        return torch.empty(n, dtype=dt, device=device)
    _need(y, "y", dt, (n,))
    return y


def mxfp4_dequant_f16(w: torch.Tensor, e: torch.Tensor) -> torch.Tensor:
    """fp16 (rows, k) of MXFP4 codes w (rows, k/2) and scales e (rows, k/32)."""
    rows, half = w.shape
    k = half * 2
    _need(w, "w", torch.uint8, (rows, half))
    _need(e, "e", torch.uint8, (rows, k // 32))
    out = torch.empty((rows, k), dtype=torch.float16, device=w.device)
    hwk.load().hwk_mxfp4_dequant_f16(_stream(), w.data_ptr(), e.data_ptr(), out.data_ptr(), rows, k)
    return out


def mxfp4_gemv(w, e, x, out_mode="f32", y=None):
    """y = W x for MXFP4 W (n, k): codes w (n, k/2), scales e (n, k/32); x fp16 (k)."""
    n, half = w.shape
    k = half * 2
    _need(w, "w", torch.uint8, (n, half))
    _need(e, "e", torch.uint8, (n, k // 32))
    _need(x, "x", torch.float16, (k,))
    y = _out(y, n, out_mode, w.device)
    hwk.load().hwk_mxfp4_gemv(_stream(), w.data_ptr(), e.data_ptr(), x.data_ptr(), y.data_ptr(), n, k,
                              OUT_MODES[out_mode])
    return y


def i8_gemv(q, scale16, x, out_mode="f32", y=None):
    """y = scale * (Q x) for int8 Q (n, k) and fp16 per-row scales; x fp16 (k)."""
    n, k = q.shape
    _need(q, "q", torch.int8, (n, k))
    _need(scale16, "scale", torch.float16, (n,))
    _need(x, "x", torch.float16, (k,))
    y = _out(y, n, out_mode, q.device)
    hwk.load().hwk_i8_gemv(_stream(), q.data_ptr(), scale16.data_ptr(), x.data_ptr(), y.data_ptr(), n, k,
                           OUT_MODES[out_mode])
    return y


def f16_gemv(w, x, out_mode="f32", y=None):
    """y = W x for fp16 W (n, k) and x (k)."""
    n, k = w.shape
    _need(w, "w", torch.float16, (n, k))
    _need(x, "x", torch.float16, (k,))
    y = _out(y, n, out_mode, w.device)
    hwk.load().hwk_f16_gemv(_stream(), w.data_ptr(), x.data_ptr(), y.data_ptr(), n, k, OUT_MODES[out_mode])
    return y


def mxfp4_encode(x: torch.Tensor):
    """MXFP4 codes (rows, k/2) and scales (rows, k/32) of fp32 x (rows, k)."""
    rows, k = x.shape
    _need(x, "x", torch.float32, (rows, k))
    w = torch.empty((rows, k // 2), dtype=torch.uint8, device=x.device)
    e = torch.empty((rows, k // 32), dtype=torch.uint8, device=x.device)
    hwk.load().hwk_mxfp4_encode(_stream(), x.data_ptr(), w.data_ptr(), e.data_ptr(), rows, k)
    return w, e
