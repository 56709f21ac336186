"""hwnpu_amd: an MI355X (gfx950) execution backend for hwnpu's quantized LLM decode path.

libhwk (csrc/, C ABI in include/hwk.h) holds the HIP kernels; this package binds it (hwk), wraps
its ops over torch's device memory and stream (ops), and draws the benchmark inputs on the GPU
(synth). There is no CPU path: without libhwk or a GPU every op raises.
"""
from . import hwk
from .hwk import HwkError, HwkLibraryError

__all__ = ["hwk", "HwkError", "HwkLibraryError"]
