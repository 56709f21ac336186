"""numpy binding of the C oracle (oracle/lib/liboracle.so).

TEST INFRASTRUCTURE ONLY: the checker and the timed CPU baseline. Only tests/, the package smoke
check (__graft_entry__.smoke) and bench.py's cpu_baseline leg may import this module; the product
path never does. See oracle.h for what each function restates and how it is pinned.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "liboracle.so")

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle not built: {LIB_PATH} (run make -C oracle)")
        L = C.CDLL(LIB_PATH)
        P = C.c_void_p
        sz = C.c_size_t
        sig = {
            "or_f16_bits": (C.c_uint16, [C.c_float]),
            "or_f16_value": (C.c_float, [C.c_uint16]),
            "or_f32_to_f16": (None, [P, P, sz]),
            "or_f16_to_f32": (None, [P, P, sz]),
            "or_mxfp4_value": (C.c_float, [C.c_int]),
            "or_mxfp4_scale": (C.c_float, [C.c_uint8]),
            "or_mxfp4_dequantize": (None, [P, P, P, sz]),
            "or_mxfp4_dequantize_rows": (None, [P, P, P, sz, sz, C.c_int]),
            "or_mxfp4_nearest": (C.c_uint8, [C.c_double]),
            "or_mxfp4_encode": (None, [P, P, P, sz]),
            "or_mxfp4_encode_rows": (None, [P, P, P, sz, sz, C.c_int]),
            "or_vec_quantize": (None, [P, P, P, sz]),
            "or_mxfp4_dot": (C.c_float, [P, P, sz, P, P]),
            "or_mxfp4_run": (None, [P, P, P, sz, sz, P, P, sz, C.c_int]),
            "or_sgemm": (None, [C.c_int, C.c_int, C.c_int, P, C.c_int, C.c_int, P, C.c_int, C.c_int, P,
                                C.c_int, C.c_int]),
            "or_i8_dequant": (None, [P, P, P, sz, sz, C.c_int]),
            "or_i8_quantize_rows": (None, [P, P, P, sz, sz]),
            "or_merge_new": (P, [C.c_int, C.c_int]),
            "or_merge_free": (None, [P]),
            "or_merge_reset": (None, [P]),
            "or_merge_add": (None, [P, P, P, P]),
            "or_merge_add_sink": (None, [P, P, C.c_int]),
            "or_merge_result": (None, [P, P]),
            "or_paged_chunk": (None, [P, P, P, sz, P, P, P, P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                      C.c_float]),
            "or_attn_decode": (None, [P, P, P, P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, C.c_int,
                                      C.c_int]),
            "or_choose": (None, [P, P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_double, P, P]),
            "or_experts_f32": (None, [P, C.c_int, P, P, C.c_int, P, P, P, P, P, P, C.c_int, C.c_int, C.c_int,
                                      C.c_int, C.c_float, C.c_float, P, C.c_int]),
            "or_experts_host": (None, [P, C.c_int, P, P, C.c_int, P, P, P, P, P, P, C.c_int, C.c_int, C.c_int,
                                       C.c_int, C.c_float, C.c_float, P, C.c_int]),
            "or_rmsnorm": (None, [P, P, P, C.c_int, C.c_int, C.c_float]),
            "or_rope_tables": (None, [P, P, C.c_double, C.c_int, C.c_int, C.c_int]),
            "or_apply_rope": (None, [P, C.c_int, C.c_int, P, P]),
            "or_silu_mul": (None, [P, P, P, sz]),
            "or_fnv64a": (C.c_uint64, [C.c_char_p]),
            "or_synth_reference": (None, [C.c_char_p, sz, P]),
            "or_argmax": (C.c_int32, [P, sz]),
            "or_max_threads": (C.c_int, []),
            "or_normal_at": (C.c_double, [C.c_uint64, C.c_uint64]),
            "or_fnv64a": (C.c_uint64, [C.c_char_p]),
            "or_qwen3_new": (P, [P, C.c_uint64, C.c_float, C.c_int]),
            "or_qwen3_free": (None, [P]),
            "or_qwen3_checksums": (None, [P, P]),
            "or_qwen3_run": (C.c_int32, [P, P, C.c_int, C.c_int, P]),
            "or_qwen3_set": (C.c_int, [P, C.c_char_p, P, C.c_size_t]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(C.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def max_threads() -> int:
    return lib().or_max_threads()


# ---- fp16 ----
def f16_bits(f: float) -> int:
    return lib().or_f16_bits(float(f))


def f16_value(h: int) -> float:
    return lib().or_f16_value(int(h))


def f32_to_f16(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().or_f32_to_f16(_p(out), _p(x), x.size)
    return out


def f16_to_f32(h) -> np.ndarray:
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().or_f16_to_f32(_p(out), _p(h), h.size)
    return out


# ---- MXFP4 ----
def mxfp4_scale(e: int) -> float:
    return lib().or_mxfp4_scale(int(e))


def mxfp4_nearest(x: float) -> int:
    return lib().or_mxfp4_nearest(float(x))


def mxfp4_dequantize(w, e, threads=0) -> np.ndarray:
    """fp32 (rows, k) of codes w (rows, k/2) and scales e (rows, k/32)."""
    w = _c(w, np.uint8)
    e = _c(e, np.uint8)
    rows, nb = e.shape
    out = np.empty((rows, nb * 32), np.float32)
    lib().or_mxfp4_dequantize_rows(_p(out), _p(w), _p(e), rows, nb, threads)
    return out


def mxfp4_encode(m, threads=0):
    m = _c(m, np.float32)
    rows, n = m.shape
    w = np.empty((rows, n // 2), np.uint8)
    e = np.empty((rows, n // 32), np.uint8)
    lib().or_mxfp4_encode_rows(_p(w), _p(e), _p(m), rows, n, threads)
    return w, e


def vec_quantize(x):
    x = _c(x, np.float32)
    q = np.empty(x.shape, np.int8)
    s = np.empty(x.size // 32, np.float32)
    lib().or_vec_quantize(_p(q), _p(s), _p(x), x.size)
    return q, s


def mxfp4_dot(w_row, e_row, q, s) -> float:
    w_row, e_row = _c(w_row, np.uint8), _c(e_row, np.uint8)
    q, s = _c(q, np.int8), _c(s, np.float32)
    return lib().or_mxfp4_dot(_p(w_row), _p(e_row), e_row.size, _p(q), _p(s))


def mxfp4_run(w, e, qs, ss, threads=0) -> np.ndarray:
    """mxfp4.Run: out (nvec, rows) for quantized vectors qs (nvec, k) int8, ss (nvec, k/32)."""
    w, e = _c(w, np.uint8), _c(e, np.uint8)
    qs, ss = _c(qs, np.int8), _c(ss, np.float32)
    rows, nb = e.shape
    nvec = qs.shape[0] if qs.ndim == 2 else 1
    out = np.empty((nvec, rows), np.float32)
    lib().or_mxfp4_run(_p(out), _p(w), _p(e), rows, nb, _p(qs), _p(ss), nvec, threads)
    return out


# ---- GEMM ----
def sgemm(a, b, c=None, transb=False, threads=0) -> np.ndarray:
    """C += A B (A m x k, B k x n; with transb B given as n x k)."""
    a = _c(a, np.float32)
    b = _c(b, np.float32)
    m, k = a.shape
    n = b.shape[0] if transb else b.shape[1]
    c = np.zeros((m, n), np.float32) if c is None else _c(c, np.float32)
    lib().or_sgemm(m, n, k, _p(a), k, 0, _p(b), k if transb else n, 1 if transb else 0, _p(c), n, threads)
    return c


def i8_dequant(q, scale16, threads=0) -> np.ndarray:
    q = _c(q, np.int8)
    scale16 = _c(scale16, np.uint16)
    rows, cols = q.shape
    out = np.empty((rows, cols), np.float32)
    lib().or_i8_dequant(_p(out), _p(q), _p(scale16), rows, cols, threads)
    return out


def i8_quantize_rows(x):
    x = _c(x, np.float32)
    rows, cols = x.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty(rows, np.uint16)
    lib().or_i8_quantize_rows(_p(q), _p(s), _p(x), rows, cols)
    return q, s


# ---- attention ----
class Merge:
    def __init__(self, rows: int, dim: int):
        self.rows, self.dim = rows, dim
        self._h = lib().or_merge_new(rows, dim)

    def __del__(self):
        if getattr(self, "_h", None):
            lib().or_merge_free(self._h)
            self._h = None

    def reset(self):
        lib().or_merge_reset(self._h)

    def add(self, o, m, l):
        o, m, l = _c(o, np.float32), _c(m, np.float32), _c(l, np.float32)
        lib().or_merge_add(self._h, _p(o), _p(m), _p(l))

    def add_sink(self, sinks, tokens):
        sinks = _c(sinks, np.float32)
        lib().or_merge_add_sink(self._h, _p(sinks), tokens)

    def result(self) -> np.ndarray:
        out = np.empty((self.rows, self.dim), np.float32)
        lib().or_merge_result(self._h, _p(out))
        return out


def paged_chunk(q, k, v, mask, scale):
    """q (heads, tokens, d), k/v (kv_heads, chunk, d), mask (tokens, chunk) or None."""
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    heads, tokens, d = q.shape
    kvh, chunk, _ = k.shape
    o = np.empty((heads, tokens, d), np.float32)
    m = np.empty((heads, tokens), np.float32)
    l = np.empty((heads, tokens), np.float32)
    mk = None if mask is None else _c(mask, np.float32)
    lib().or_paged_chunk(_p(q), _p(k), _p(v), chunk, None if mk is None else _p(mk), _p(o), _p(m), _p(l), heads,
                         kvh, tokens, chunk, d, float(scale))
    return o, m, l


def attn_decode(q, k, v, scale, chunk=8192, threads=0) -> np.ndarray:
    """q (heads, d); k/v (kv_heads, L, d) floats; out (heads, d)."""
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    heads, d = q.shape
    kvh, L, _ = k.shape
    out = np.empty((heads, d), np.float32)
    lib().or_attn_decode(_p(q), _p(k), _p(v), _p(out), heads, kvh, L, d, float(scale), chunk, threads)
    return out


# ---- MoE ----
def choose(logits, k, score="softmax", norm=True, scale=0.0, bias=None):
    logits = _c(logits, np.float32)
    n = logits.size
    idx = np.empty(k, np.int32)
    w = np.empty(k, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    lib().or_choose(_p(logits), None if b is None else _p(b), n, k, 0 if score == "softmax" else 1, 1 if norm else 0,
                    float(scale), _p(idx), _p(w))
    return idx, w


def experts(x, idx, w, gu_w, gu_e, dn_w, dn_e, quantized=False, threads=0, gu_b=None, dn_b=None, act="silu",
            alpha=1.702, limit=7.0) -> np.ndarray:
    """x (T, H); idx/w (T, k); gu_w (E, 2I, H/32, 16) ...; optional biases gu_b (E, 2I), dn_b (E, H);
    act 'silu' or 'gptoss' -> out (T, H) fp32."""
    x = _c(x, np.float32)
    idx, w = _c(idx, np.int32), _c(w, np.float32)
    gu_w, gu_e, dn_w, dn_e = (_c(a, np.uint8) for a in (gu_w, gu_e, dn_w, dn_e))
    gb = None if gu_b is None else _c(gu_b, np.float32)
    db = None if dn_b is None else _c(dn_b, np.float32)
    T, H = x.shape
    k = idx.shape[1]
    E = gu_e.shape[0]
    I = gu_e.shape[1] // 2
    out = np.zeros((T, H), np.float32)
    fn = lib().or_experts_host if quantized else lib().or_experts_f32
    fn(_p(x), T, _p(idx), _p(w), k, _p(gu_w), _p(gu_e), None if gb is None else _p(gb), _p(dn_w), _p(dn_e),
       None if db is None else _p(db), E, H, I, 0 if act == "silu" else 1, float(alpha), float(limit), _p(out),
       threads)
    return out


# ---- model ops ----
def rmsnorm(x, w, eps):
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    n = x.shape[-1]
    rows = x.size // n
    out = np.empty(x.shape, np.float32)
    lib().or_rmsnorm(_p(out), _p(x), _p(w), rows, n, float(eps))
    return out


def rope_tables(theta, start, n, head_dim):
    c = np.empty((n, head_dim), np.float32)
    s = np.empty((n, head_dim), np.float32)
    lib().or_rope_tables(_p(c), _p(s), float(theta), start, n, head_dim)
    return c, s


def apply_rope(x, cos_row, sin_row):
    x = np.array(x, dtype=np.float32, order="C")
    heads, hd = x.shape
    cos_row, sin_row = _c(cos_row, np.float32), _c(sin_row, np.float32)
    lib().or_apply_rope(_p(x), heads, hd, _p(cos_row), _p(sin_row))
    return x


def silu_mul(g, u):
    g, u = _c(g, np.float32), _c(u, np.float32)
    out = np.empty(g.shape, np.float32)
    lib().or_silu_mul(_p(out), _p(g), _p(u), g.size)
    return out


def argmax(x) -> int:
    x = _c(x, np.float32)
    return int(lib().or_argmax(_p(x), x.size))


# ---- the Qwen3 decoder ----
class Qwen3Cfg(C.Structure):
    _fields_ = [("layers", C.c_int), ("hidden", C.c_int), ("heads", C.c_int), ("kv_heads", C.c_int),
                ("head_dim", C.c_int), ("inter", C.c_int), ("vocab", C.c_int), ("max_ctx", C.c_int),
                ("theta", C.c_double), ("eps", C.c_double)]


class Qwen3:
    """The oracle's synthetic Qwen3 (qwen3.c): run(tokens, start) -> (greedy token, logits)."""

    def __init__(self, layers, hidden, heads, kv_heads, head_dim, inter, vocab, max_ctx, theta=1e6, eps=1e-6,
                 seed=0, std=0.02, threads=0):
        self.cfg = Qwen3Cfg(layers, hidden, heads, kv_heads, head_dim, inter, vocab, max_ctx, theta, eps)
        self.vocab = vocab
        self._h = lib().or_qwen3_new(C.byref(self.cfg), seed, std, threads)

    def __del__(self):
        if getattr(self, "_h", None):
            lib().or_qwen3_free(self._h)
            self._h = None

    def checksums(self):
        out = np.zeros(3, np.uint64)
        lib().or_qwen3_checksums(self._h, _p(out))
        return [int(v) for v in out]

    def set(self, name: str, values) -> None:
        """Replaces a tensor by its Hugging Face name (norm weights, linears as the float values they
        compute with, the embedding); std=0 at construction starts from zero weights."""
        v = _c(values, np.float32)
        rc = lib().or_qwen3_set(self._h, name.encode(), _p(v), v.size)
        if rc:
            raise ValueError(f"or_qwen3_set({name!r}, {v.size} values): " +
                             ("unknown name" if rc == -1 else "wrong number of values"))

    def run(self, tokens, start):
        toks = _c(tokens, np.int32)
        logits = np.empty(self.vocab, np.float32)
        tok = lib().or_qwen3_run(self._h, _p(toks), toks.size, int(start), _p(logits))
        return int(tok), logits


def normal_at(key: int, i: int) -> float:
    return lib().or_normal_at(key, i)


# ---- the reference's synthetic checkpoint (internal/llm/synth.go:17-35) ----
def fnv64a(name: str) -> int:
    return int(lib().or_fnv64a(name.encode()))


def synth_reference(name: str, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().or_synth_reference(name.encode(), n, _p(out))
    return out
