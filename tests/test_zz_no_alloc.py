"""hwk_attn_decode_noalloc (the allocation-free decode attention) against hwk_attn_decode, through
libhwk's C ABI: bit-identical outputs on two calls in a row, the second with a smaller input, in fp16
and int8 KV forms. (Parameters past the library's scratch are refused on the host before any HIP
call: tests/test_abi.py.)"""
import numpy as np
import pytest
import torch

from hwnpu_amd import hwk, ops, synth

pytestmark = pytest.mark.gpu


def _case(heads, kvh, cap, name):
    q = synth.normal(heads * 128, name + ".q").view(heads, 128)
    k = synth.normal(kvh * cap * 128, name + ".k").view(kvh, cap, 128)
    v = synth.normal(kvh * cap * 128, name + ".v").view(kvh, cap, 128)
    return q, k, v


@pytest.mark.parametrize("int8", [False, True])
def test_noalloc_matches_workspace_entry(dev, int8):
    print(f"noalloc int8={int8}", flush=True)
    calls = [(32, 8, 32768, 32768), (16, 8, 1153, 2048)]  # the second call smaller than the first
    for i, (heads, kvh, L, cap) in enumerate(calls):
        q, k, v = _case(heads, kvh, cap, f"noalloc.{int8}.{i}")
        ks = vs = None
        if int8:
            k, ks = ops.kv_quantize_i8(k)
            v, vs = ops.kv_quantize_i8(v)
        for mode in ("f32", "f16"):
            want = ops.attn_decode(q, k, v, L, ks, vs, out_mode=mode)
            out = torch.full_like(want, float("nan"))
            got = ops.attn_decode_noalloc(q, k, v, L, ks, vs, out_mode=mode, out=out)
            torch.cuda.synchronize()
            a, b = got.cpu().numpy(), want.cpu().numpy()
            assert np.array_equal(a.view(np.uint16 if mode == "f16" else np.uint32),
                                  b.view(np.uint16 if mode == "f16" else np.uint32)), (heads, L, mode)
