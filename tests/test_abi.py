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
    assert hwk.load().hwk_abi() == hwk.ABI == 1


def test_wrong_abi_refused(tmp_path, monkeypatch):
    monkeypatch.setattr(hwk, "ABI", 2)
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
])
def test_bad_arguments_rejected(call, match):
    with pytest.raises(hwk.HwkError, match=match):
        call(hwk.load())


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
