"""ctypes binding of libhwk (include/hwk.h), the way a purego binding in hwnpu would bind it.

The library is loaded from the package's own lib/ directory (built in-tree by
``__graft_entry__.build()``). There is no fallback: when libhwk is missing or of another ABI,
every call raises :class:`HwkLibraryError` (the reference's ``types.ErrLibrary``,
internal/types/errors.go:9-30, raised by ``dl.Open`` with every path it tried,
internal/dl/dl.go:23-36).
"""
from __future__ import annotations

import ctypes as C
import os
import threading

ABI = 4

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib")
LIB_PATH = os.path.join(LIB_DIR, "libhwk.so")
# the library's gfx950 code object (hwk_module_load): the batch-1 MXFP4 GEMV and a streaming read
CODE_OBJECT_PATH = os.path.join(LIB_DIR, "hwk_gfx950.hsaco")

# include/hwk.h enums
BUF_MIRRORED, BUF_DEVICE = 0, 1
SYNC_TO_DEVICE, SYNC_FROM_DEVICE = 0, 1
INFO_NAME, INFO_ARCH, INFO_PCI_BUS, INFO_CUS, INFO_MEM_BYTES = 0, 1, 2, 3, 4
STATE_DONE, STATE_PENDING = 0, 1
OUT_F32, OUT_F16, OUT_ADD_F32, OUT_SWIGLU_F16 = 0, 1, 2, 3
ATTN_SCRATCH_BYTES = 4 << 20  # HWK_ATTN_SCRATCH_BYTES


class HwkError(RuntimeError):
    """An error string returned by a libhwk call (a HIP error or a rejected argument)."""


class HwkLibraryError(HwkError):
    """libhwk could not be loaded (missing, or built for another ABI)."""


P = C.c_void_p
U32, U64, I32, SZ = C.c_uint32, C.c_uint64, C.c_int32, C.c_size_t


class AttnParams(C.Structure):
    """hwk_attn_params (include/hwk.h)."""
    _fields_ = [("heads", U32), ("kv_heads", U32), ("head_dim", U32), ("len", U32), ("capacity", U32),
                ("kv_int8", U32), ("scale_bits", U32), ("out_mode", U32), ("split", U32)]


class MoeParams(C.Structure):
    """hwk_moe_params (include/hwk.h)."""
    _fields_ = [("tokens", U32), ("hidden", U32), ("inter", U32), ("experts", U32), ("k", U32),
                ("out_mode", U32), ("act", U32), ("alpha_bits", U32), ("limit_bits", U32), ("score", U32),
                ("norm", U32), ("scale_bits", U32)]


SCORE_SOFTMAX, SCORE_SIGMOID = 0, 1
ACT_SILU, ACT_GPTOSS = 0, 1


class KernelInfo(C.Structure):
    """hwk_kernel_info (include/hwk.h)."""
    _fields_ = [("name", C.c_char * 64), ("args", U32), ("kernarg_bytes", U32), ("block", U32), ("max_block", U32),
                ("lds_bytes", U32), ("cus", U32), ("runnable", U32), ("reserved", U32)]


class KernelArg(C.Structure):
    """hwk_kernel_arg (include/hwk.h)."""
    _fields_ = [("index", U32), ("offset", U32), ("size", U32), ("buffer", U32), ("nullable", U32),
                ("name", C.c_char * 64), ("type", C.c_char * 32)]


class Qwen3Config(C.Structure):
    """hwk_qwen3_config (include/hwk.h)."""
    _fields_ = [("layers", U32), ("hidden", U32), ("heads", U32), ("kv_heads", U32), ("head_dim", U32),
                ("inter", U32), ("vocab", U32), ("max_ctx", U32), ("max_prompt", U32), ("pad", U32),
                ("theta_bits", U64), ("eps_bits", U64)]

# name -> (restype, argtypes). ERR marks calls returning an error string (NULL on success).
ERR = "err"
SIGNATURES = {
    "hwk_abi": (C.c_int, []),
    "hwk_free_error": (None, [P]),
    "hwk_device_count": (ERR, [C.POINTER(U32)]),
    "hwk_device_open": (ERR, [U32, C.POINTER(P)]),
    "hwk_device_free": (None, [P]),
    "hwk_device_info": (ERR, [P, C.c_int, C.c_char_p, SZ, C.POINTER(SZ)]),
    "hwk_device_synchronize": (ERR, [P]),
    "hwk_buf_alloc": (ERR, [P, SZ, C.c_int, C.POINTER(P)]),
    "hwk_buf_free": (None, [P]),
    "hwk_buf_host_ptr": (P, [P]),
    "hwk_buf_dev_ptr": (P, [P]),
    "hwk_buf_size": (SZ, [P]),
    "hwk_buf_sync": (ERR, [P, C.c_int, SZ, SZ]),
    "hwk_stream_new": (ERR, [P, C.POINTER(P)]),
    "hwk_stream_free": (None, [P]),
    "hwk_stream_sync": (ERR, [P]),
    "hwk_event_new": (ERR, [P, C.POINTER(P)]),
    "hwk_event_free": (None, [P]),
    "hwk_event_record": (ERR, [P, P]),
    "hwk_event_wait": (ERR, [P, U32, C.POINTER(C.c_int)]),
    "hwk_event_elapsed_ns": (ERR, [P, P, C.POINTER(U64)]),
    "hwk_module_load": (ERR, [P, P, SZ, C.POINTER(P)]),
    "hwk_module_free": (None, [P]),
    "hwk_module_kernel_count": (ERR, [P, C.POINTER(U32)]),
    "hwk_module_kernel_info": (ERR, [P, U32, C.POINTER(KernelInfo)]),
    "hwk_module_kernel_arg": (ERR, [P, U32, U32, C.POINTER(KernelArg)]),
    "hwk_run_new": (ERR, [P, C.c_char_p, C.POINTER(P)]),
    "hwk_run_set_arg": (ERR, [P, U32, P, SZ]),
    "hwk_run_set_buffer": (ERR, [P, U32, P]),
    "hwk_run_set_buffer_at": (ERR, [P, U32, P, SZ, SZ]),
    "hwk_run_set_null": (ERR, [P, U32]),
    "hwk_run_err": (ERR, [P]),
    "hwk_run_submit": (ERR, [P, P]),
    "hwk_run_wait": (ERR, [P, U32, C.POINTER(C.c_int)]),
    "hwk_run_free": (ERR, [P]),
    "hwk_mxfp4_dequant_f16": (ERR, [P, P, P, P, U32, U32]),
    "hwk_mxfp4_gemv": (ERR, [P, P, P, P, P, U32, U32, C.c_int]),
    "hwk_mxfp4_gemv_rows": (ERR, [P, P, P, P, P, U32, U32, U32, C.c_int]),
    "hwk_i8_gemv": (ERR, [P, P, P, P, P, U32, U32, C.c_int]),
    "hwk_f16_gemv": (ERR, [P, P, P, P, U32, U32, C.c_int]),
    "hwk_f16_gemv_rows": (ERR, [P, P, P, P, U32, U32, U32, C.c_int]),
    "hwk_rope_tables": (ERR, [U64, U32, U32, U32, P, P]),
    "hwk_rmsnorm": (ERR, [P, P, P, P, U32, U32, U64, C.c_int]),
    "hwk_rope": (ERR, [P, P, P, P, P, P, U32, U32, U32, U32, U32, U64, C.c_int]),
    "hwk_kv_append": (ERR, [P, P, P, P, P, U32, U32, U32, U32, U32]),
    "hwk_silu_mul": (ERR, [P, P, P, P, U64, U32, C.c_int]),
    "hwk_add": (ERR, [P, P, P, U64]),
    "hwk_embed": (ERR, [P, P, P, P, U32, U32, U32]),
    "hwk_argmax_workspace_bytes": (SZ, [U32]),
    "hwk_argmax": (ERR, [P, P, P, U32, U64, P, SZ]),
    "hwk_i8_gemm": (ERR, [P, P, P, P, P, U32, U32, U32, C.c_int]),
    "hwk_mxfp4_gemm": (ERR, [P, P, P, P, P, U32, U32, U32, C.c_int]),
    "hwk_attn_workspace_bytes": (SZ, [C.POINTER(AttnParams)]),
    "hwk_attn_decode": (ERR, [P, P, P, P, P, P, P, P, SZ, C.POINTER(AttnParams)]),
    "hwk_attn_decode_noalloc": (ERR, [P, P, P, P, P, P, P, C.POINTER(AttnParams)]),
    "hwk_kv_quantize_i8": (ERR, [P, P, P, P, U32, U32]),
    "hwk_attn_merge": (ERR, [P, P, P, P, P, U32, U32, U32, C.c_int]),
    "hwk_attn_prefill": (ERR, [P, P, P, P, P, U32, U32, C.POINTER(AttnParams)]),
    "hwk_qwen3_new": (ERR, [C.POINTER(Qwen3Config), C.POINTER(P)]),
    "hwk_qwen3_free": (None, [P]),
    "hwk_qwen3_synth": (ERR, [P, P, U64, U32]),
    "hwk_qwen3_tensor": (ERR, [P, C.c_char_p, C.POINTER(P), C.POINTER(SZ)]),
    "hwk_qwen3_state": (ERR, [P, C.POINTER(P), C.POINTER(P), C.POINTER(P)]),
    "hwk_qwen3_prefill": (ERR, [P, P, C.POINTER(I32), U32, U32]),
    "hwk_qwen3_step": (ERR, [P, P]),
    "hwk_qwen3_decode": (ERR, [P, P, U32]),
    "hwk_qwen3_capture": (ERR, [P]),
    "hwk_qwen3_row_bytes": (ERR, [P, C.POINTER(SZ)]),
    "hwk_qwen3_export_rows": (ERR, [P, P, U32, U32, P]),
    "hwk_qwen3_import_rows": (ERR, [P, P, U32, P, SZ]),
    "hwk_qwen3_position": (ERR, [P, C.POINTER(U32)]),
    "hwk_qwen3_rewind": (ERR, [P, P, U32, I32]),
    "hwk_qwen3_verify": (ERR, [P, P, C.POINTER(I32), U32, C.POINTER(P), C.POINTER(P)]),
    "hwk_qwen3_keep": (ERR, [P, P, U32]),
    "hwk_moe_route": (ERR, [P, P, P, P, P, U32, U32, U32, C.c_int, C.c_int, U32]),
    "hwk_moe_workspace_bytes": (SZ, [C.POINTER(MoeParams)]),
    "hwk_moe_experts": (ERR, [P, P, P, P, P, P, P, P, P, P, P, P, SZ, C.POINTER(MoeParams)]),
    "hwk_moe_layer": (ERR, [P, P, P, P, P, P, P, P, P, P, P, P, P, P, SZ, C.POINTER(MoeParams)]),
    "hwk_synth_bytes": (ERR, [P, P, U64, U64]),
    "hwk_synth_uniform": (ERR, [P, P, U64, U64, I32, U32, C.c_int]),
    "hwk_synth_normal": (ERR, [P, P, U64, U64, U32, C.c_int]),
    "hwk_synth_mxfp4": (ERR, [P, P, P, U32, U32, U64, U32]),
    "hwk_mxfp4_encode": (ERR, [P, P, P, P, U32, U32]),
    "hwk_read_floor": (ERR, [P, P, SZ, P, U32, U32]),
    "hwk_synth_reference": (ERR, [P, P, U64, C.c_char_p, C.c_int]),
}

_lock = threading.Lock()
_lib = None


class _Lib:
    """The loaded library: attribute access gives a checked Python callable per entry point."""

    def __init__(self, path: str):
        self.path = path
        self._cdll = C.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(self._cdll, name)
            fn.restype = P if res == ERR else res
            fn.argtypes = args
        abi = self._cdll.hwk_abi()
        if abi != ABI:
            raise HwkLibraryError(f"{path}: ABI {abi}, this binding speaks {ABI}")

    def raw(self, name: str):
        return getattr(self._cdll, name)

    def __getattr__(self, name: str):
        if name not in SIGNATURES:
            raise AttributeError(name)
        fn = getattr(self._cdll, name)
        if SIGNATURES[name][0] != ERR:
            return fn
        free = self._cdll.hwk_free_error

        def call(*args):
            err = fn(*args)
            if err:
                msg = C.string_at(err).decode(errors="replace")
                free(err)
                raise HwkError(msg)

        call.__name__ = name
        return call


def load(path: str | None = None) -> _Lib:
    """The process's libhwk; raises HwkLibraryError when it is missing or of another ABI."""
    global _lib
    with _lock:
        if _lib is not None and (path is None or path == _lib.path):
            return _lib
        p = path or os.environ.get("HWNPU_HWK_LIB", LIB_PATH)
        if not os.path.exists(p):
            raise HwkLibraryError(f"libhwk not found (tried {p}); build it with __graft_entry__.build()")
        try:
            lib = _Lib(p)
        except OSError as e:
            raise HwkLibraryError(f"libhwk at {p} failed to load: {e}") from e
        _lib = lib
        return lib
