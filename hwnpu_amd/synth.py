"""Synthetic inputs of the benchmark configurations, drawn on the GPU by libhwk.

A tensor's stream key is ``seed ^ fnv64a(name)``, so a tensor's values depend on the seed and its
name alone, not on the order tensors are made in (the role of the reference's deterministic
synthetic checkpoints, internal/llm/synth.go:12-56). Element i of a stream reads splitmix64 at
state ``key + (i+1)*gamma``; see csrc/synth.h for the draws.
"""
from __future__ import annotations

import torch

from . import hwk
from .ops import _stream, f32_bits

MASK64 = (1 << 64) - 1


def fnv64a(name: str) -> int:
    h = 0xCBF29CE484222325
    for b in name.encode():
        h ^= b
        h = (h * 0x100000001B3) & MASK64
    return h


def key_of(name: str, seed: int = 0) -> int:
    return (seed ^ fnv64a(name)) & MASK64


def bytes_(n: int, name: str, seed: int = 0, device="cuda") -> torch.Tensor:
    out = torch.empty(n, dtype=torch.uint8, device=device)
    hwk.load().hwk_synth_bytes(_stream(), out.data_ptr(), n, key_of(name, seed))
    return out


def uniform_int(n: int, lo: int, span: int, name: str, seed: int = 0, dtype=torch.int32, device="cuda"):
    """n ints uniform in [lo, lo+span), as int8/uint8 (bytes) or int32."""
    limits = {torch.int8: (-128, 127), torch.uint8: (0, 255), torch.int32: (-(2**31), 2**31 - 1)}
    if dtype not in limits:
        raise TypeError(f"uniform_int: dtype {dtype}")
    if span < 1 or lo < limits[dtype][0] or lo + span - 1 > limits[dtype][1]:
        raise ValueError(f"uniform_int: [{lo}, {lo + span}) does not fit {dtype}")
    out = torch.empty(n, dtype=torch.int32, device=device)
    hwk.load().hwk_synth_uniform(_stream(), out.data_ptr(), n, key_of(name, seed), lo, span, 4)
    return out if dtype == torch.int32 else out.to(dtype)


def normal(n: int, name: str, std: float = 1.0, seed: int = 0, dtype=torch.float16, device="cuda"):
    if dtype not in (torch.float16, torch.float32):
        raise TypeError(f"normal: dtype {dtype}")
    out = torch.empty(n, dtype=dtype, device=device)
    hwk.load().hwk_synth_normal(_stream(), out.data_ptr(), n, key_of(name, seed), f32_bits(std),
                                1 if dtype == torch.float16 else 0)
    return out


def mxfp4_normal(rows: int, k: int, name: str, std: float, seed: int = 0, device="cuda"):
    """MXFP4 codes (rows, k/2) and scales (rows, k/32) of N(0, std) weights, encoded on the GPU."""
    w = torch.empty((rows, k // 2), dtype=torch.uint8, device=device)
    e = torch.empty((rows, k // 32), dtype=torch.uint8, device=device)
    hwk.load().hwk_synth_mxfp4(_stream(), w.data_ptr(), e.data_ptr(), rows, k, key_of(name, seed), f32_bits(std))
    return w, e


def mxfp4_uniform(rows: int, k: int, name: str, seed: int = 0, emin: int = -4, emax: int = 2, device="cuda"):
    """The GEMV configuration's MXFP4 weights: every nibble uniform over the 16 codes (uniform
    bytes), e8m0 exponents uniform in [emin, emax] (scale bytes 127+emin .. 127+emax)."""
    w = bytes_(rows * (k // 2), name + ".blocks", seed, device).view(rows, k // 2)
    e = uniform_int(rows * (k // 32), 127 + emin, emax - emin + 1, name + ".scales", seed, torch.uint8,
                    device).view(rows, k // 32)
    return w, e


def uniform_real(n: int, lo: float, hi: float, name: str, seed: int = 0, dtype=torch.float16, device="cuda"):
    """n values lo + (hi - lo) * u / 2^24 for u uniform in [0, 2^24), computed in float64 and
    rounded to dtype (RNE): the per-channel scales of the int8 configuration."""
    u = uniform_int(n, 0, 1 << 24, name, seed, torch.int32, device).to(torch.float64)
    return (lo + (hi - lo) * u / float(1 << 24)).to(torch.float32).to(dtype)


def reference(name: str, n: int, dtype=torch.float32) -> torch.Tensor:
    """The reference's synthetic values of tensor `name` (llm.Synthetic.Get, internal/llm/synth.go:17-35):
    n values uniform in [-0.2, 0.2) (the code's range; its comment says +-0.1) from FNV-64a(name) and
    the MMIX LCG, fp32 or fp16, made on the GPU."""
    out = torch.empty(n, dtype=dtype, device="cuda")
    hwk.load().hwk_synth_reference(_stream(), out.data_ptr(), n, name.encode(), 1 if dtype == torch.float16 else 0)
    return out
