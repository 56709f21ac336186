"""libhwk's C ABI on the CPU: it loads, speaks ABI 1, exports every entry point include/hwk.h
declares, and rejects bad arguments with an error string before any launch. No GPU needed."""
import ctypes as C
import os
import re

import pytest

from hwnpu_amd import hwk

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    names = []
    for fn in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if fn.endswith(".h"):
            text = open(os.path.join(ROOT, "include", fn)).read()
            names += re.findall(r"HWK_API\s+[\w\s\*]+?\b(hwk_\w+)\s*\(", text)
    return names


def test_header_declares_entry_points():
    names = declared()
    assert "hwk_abi" in names and "hwk_mxfp4_gemv" in names
    assert len(names) == len(set(names))


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(hwk.LIB_PATH)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_header():
    assert sorted(declared()) == sorted(hwk.SIGNATURES)


def test_abi_version():
    assert hwk.load().hwk_abi() == hwk.ABI == 4


def test_wrong_abi_refused(tmp_path, monkeypatch):
    monkeypatch.setattr(hwk, "ABI", hwk.ABI + 1)
    monkeypatch.setattr(hwk, "_lib", None)
    with pytest.raises(hwk.HwkLibraryError):
        hwk.load()
    monkeypatch.undo()
    hwk._lib = None
    hwk.load()


def test_missing_library_is_loud(tmp_path, monkeypatch):
    monkeypatch.setattr(hwk, "_lib", None)
    monkeypatch.setenv("HWNPU_HWK_LIB", str(tmp_path / "nope.so"))
    with pytest.raises(hwk.HwkLibraryError, match="not found"):
        hwk.load()
    monkeypatch.undo()
    hwk._lib = None


def test_device_count_without_gpu_is_zero_or_error():
    lib = hwk.load()
    n = C.c_uint32(99)
    try:
        lib.hwk_device_count(C.byref(n))
    except hwk.HwkError:
        return
    assert n.value >= 0


FAKE = 0x10000  # never dereferenced: every case below is refused before a launch


@pytest.mark.parametrize("call,match", [
    (lambda L: L.hwk_mxfp4_gemv(None, None, FAKE, FAKE, FAKE, 8, 64, 0), "null pointer"),
    (lambda L: L.hwk_mxfp4_gemv(None, FAKE, FAKE, FAKE, FAKE, 8, 31, 0), "multiple of 32"),
    (lambda L: L.hwk_mxfp4_gemv(None, FAKE + 4, FAKE, FAKE, FAKE, 8, 64, 0), "16-byte aligned"),
    (lambda L: L.hwk_mxfp4_gemv(None, FAKE, FAKE, FAKE, FAKE, 8, 64, 7), "out_mode"),
    (lambda L: L.hwk_i8_gemv(None, FAKE, FAKE, FAKE, FAKE, 8, 24, 0), "multiple of 16"),
    (lambda L: L.hwk_f16_gemv(None, FAKE, FAKE + 8, FAKE, 8, 64, 0), "16-byte aligned"),
    (lambda L: L.hwk_mxfp4_dequant_f16(None, FAKE, FAKE, FAKE, 4, 0), "multiple of 32"),
    (lambda L: L.hwk_synth_uniform(None, FAKE, 10, 1, 120, 20, 1), "range past int8"),
    (lambda L: L.hwk_synth_uniform(None, FAKE, 10, 1, 0, 20, 2), "elem_size"),
    (lambda L: L.hwk_mxfp4_gemv_rows(None, FAKE, FAKE, FAKE, FAKE, 8, 64, 9, 0), "1..8"),
    (lambda L: L.hwk_mxfp4_gemv_rows(None, FAKE, FAKE, FAKE, FAKE, 8, 8192, 5, 0), "exceed 64 KB"),
    (lambda L: L.hwk_rmsnorm(None, FAKE, FAKE, FAKE, 4, 64, 0, 2), "out_mode"),
    (lambda L: L.hwk_rmsnorm(None, FAKE, FAKE, FAKE, 4, 64, 0xFFF0000000000000, 0), "eps"),
    (lambda L: L.hwk_rope(None, FAKE, 0, FAKE, FAKE, FAKE, 2, 4, 64, 0, 8, 0, 0), "head_dim"),
    (lambda L: L.hwk_rope(None, FAKE, 0, FAKE, FAKE, FAKE, 2, 4, 128, 7, 8, 0, 0), "table rows"),
    (lambda L: L.hwk_kv_append(None, FAKE, FAKE, FAKE, FAKE, 4, 8, 128, 64, 61), "past capacity"),
    (lambda L: L.hwk_kv_append(None, FAKE + 8, FAKE, FAKE, FAKE, 4, 8, 128, 64, 0), "16-byte aligned"),
    (lambda L: L.hwk_silu_mul(None, FAKE, FAKE, FAKE, 10, 0, 0), "stride 0"),
    (lambda L: L.hwk_embed(None, FAKE, FAKE, FAKE, 70000, 64, 10), "65535"),
    (lambda L: L.hwk_argmax(None, FAKE, FAKE, 4, 100, FAKE, 64), "workspace"),
    (lambda L: L.hwk_argmax(None, FAKE, FAKE, 1, 0, FAKE, 4096), "values a row"),
])
def test_bad_arguments_rejected(call, match):
    with pytest.raises(hwk.HwkError, match=match):
        call(hwk.load())


def test_attn_noalloc_refuses_past_scratch():
    """hwk_attn_decode_noalloc checks its parameters against the library's scratch before any HIP
    call: split 64 over 1M keys needs 16,384 chunks of 130 floats per query head, past 4 MiB."""
    import math

    from hwnpu_amd import ops

    p = ops.attn_params(32, 8, 1 << 20, 1 << 20, False, 1 / math.sqrt(128), "f32", 64)
    need = hwk.load().hwk_attn_workspace_bytes(p)
    assert need > hwk.ATTN_SCRATCH_BYTES
    with pytest.raises(hwk.HwkError, match="scratch"):
        hwk.load().hwk_attn_decode_noalloc(None, FAKE, FAKE, FAKE, None, None, FAKE, p)


def test_attn_prefill_rejects_bad_params():
    L = hwk.load()
    p = hwk.AttnParams()
    p.heads, p.kv_heads, p.head_dim, p.len, p.capacity, p.out_mode = 16, 8, 128, 10, 64, 0
    with pytest.raises(hwk.HwkError, match="start \\+ tokens"):
        L.hwk_attn_prefill(None, FAKE, FAKE, FAKE, FAKE, 8, 0, C.byref(p))  # len 10 != 0 + 8
    p.len = 70
    with pytest.raises(hwk.HwkError, match="past capacity"):
        L.hwk_attn_prefill(None, FAKE, FAKE, FAKE, FAKE, 70, 0, C.byref(p))
    p.len, p.kv_heads = 8, 3
    with pytest.raises(hwk.HwkError, match="kv heads"):
        L.hwk_attn_prefill(None, FAKE, FAKE, FAKE, FAKE, 8, 0, C.byref(p))


@pytest.mark.parametrize("field,value,match", [
    ("head_dim", 64, "head_dim"), ("kv_heads", 3, "kv heads"), ("hidden", 100, "hidden"),
    ("inter", 0, "inter"), ("max_prompt", 5000, "max_prompt"), ("layers", 0, "layers")])
def test_qwen3_new_rejects_bad_config(field, value, match):
    c = hwk.Qwen3Config()
    c.layers, c.hidden, c.heads, c.kv_heads, c.head_dim = 2, 2048, 16, 8, 128
    c.inter, c.vocab, c.max_ctx, c.max_prompt = 6144, 1000, 4096, 64
    setattr(c, field, value)
    out = C.c_void_p()
    with pytest.raises(hwk.HwkError, match=match):
        hwk.load().hwk_qwen3_new(C.byref(c), C.byref(out))


def test_rope_tables_on_host_match_oracle():
    """hwk_rope_tables runs on the host (no device): float32 of float64 cos/sin, as the oracle's."""
    import numpy as np

    from hwnpu_amd import ops
    from oracle import oracle

    n, start, d = 40, 1000, 128
    c = np.empty((n, d // 2), np.float32)
    s = np.empty((n, d // 2), np.float32)
    hwk.load().hwk_rope_tables(ops.f64_bits(1e6), start, n, d, c.ctypes.data, s.ctypes.data)
    oc, os_ = oracle.rope_tables(1e6, start, n, d)
    assert np.array_equal(c, oc[:, : d // 2]) and np.array_equal(s, os_[:, : d // 2])
    # position 0 is the identity rotation; cos^2 + sin^2 = 1
    hwk.load().hwk_rope_tables(ops.f64_bits(1e6), 0, 1, d, c.ctypes.data, s.ctypes.data)
    assert np.all(c[0] == 1) and np.all(s[0] == 0)
    with pytest.raises(hwk.HwkError, match="theta"):
        hwk.load().hwk_rope_tables(ops.f64_bits(0.5), 0, 1, d, c.ctypes.data, s.ctypes.data)


def test_gemm_rejects_bad_out_modes():
    L = hwk.load()
    with pytest.raises(hwk.HwkError, match="SwiGLU output needs n % 16"):
        L.hwk_mxfp4_gemm(None, FAKE, FAKE, FAKE, FAKE, 4, 24, 64, hwk.OUT_SWIGLU_F16)
    with pytest.raises(hwk.HwkError, match="SwiGLU output needs n % 16"):
        L.hwk_i8_gemm(None, FAKE, FAKE, FAKE, FAKE, 4, 40, 64, hwk.OUT_SWIGLU_F16)
    with pytest.raises(hwk.HwkError, match="out_mode 4"):
        L.hwk_mxfp4_gemm(None, FAKE, FAKE, FAKE, FAKE, 4, 32, 64, 4)
    with pytest.raises(hwk.HwkError, match="out_mode"):  # the GEMVs have no SwiGLU output
        L.hwk_mxfp4_gemv(None, FAKE, FAKE, FAKE, FAKE, 32, 64, hwk.OUT_SWIGLU_F16)
