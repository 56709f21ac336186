"""The code-object half of the boundary on the CPU: libhwk lists the kernels of its gfx950 code object
from the object's own AMDGPU metadata and launch manifest (no device needed), the way the reference's
Program.Kernels reports KernelInfo (internal/types/kernel.go:22-36), and refuses images that are not
gfx950 code objects. The GPU half (runs, fences, argument checks on a device) is in
test_runtime_gpu.py."""
import struct

import pytest

from hwnpu_amd import hwk
from hwnpu_amd.runtime import Program


def image():
    with open(hwk.CODE_OBJECT_PATH, "rb") as f:
        return f.read()


def by_name(kernels):
    return {k.name: k for k in kernels}


CO_KERNELS = {"hwk_co_mxfp4_gemv", "hwk_co_stream_read", "hwk_co_attn_decode_f16_g1", "hwk_co_attn_decode_f16_g2",
              "hwk_co_attn_decode_f16_g4", "hwk_co_attn_decode_i8_g4", "hwk_co_attn_merge", "hwk_co_i8_gemm",
              "hwk_co_mxfp4_gemm", "hwk_co_moe_route", "hwk_co_moe_gate_up", "hwk_co_moe_down"}


def test_kernels_from_metadata():
    ks = by_name(Program.load(None, image()).kernels())
    assert set(ks) == CO_KERNELS
    assert all(k.runnable and k.block > 0 for k in ks.values())
    g = ks["hwk_co_mxfp4_gemv"]
    assert [(a.index, a.name, a.offset, a.size, a.buffer) for a in g.args] == [
        (0, "w", 0, 8, True), (1, "e", 8, 8, True), (2, "x", 16, 8, True), (3, "y", 24, 8, True),
        (4, "n", 32, 4, False), (5, "nb", 36, 4, False)]
    assert [a.type for a in g.args] == ["void *"] * 4 + ["uint32_t"] * 2
    assert g.kernarg_bytes == 40 and g.block == 512 and g.runnable and g.cus == 0
    r = ks["hwk_co_stream_read"]
    assert [(a.name, a.size, a.buffer) for a in r.args] == [("p", 8, True), ("n16", 4, False), ("sink", 8, True)]
    assert r.block == 256 and r.runnable
    a = ks["hwk_co_attn_decode_f16_g4"]
    assert [x.name for x in a.args] == ["q", "k", "v", "ws_o", "ws_m", "ws_l", "out", "groups", "kv_heads", "mode",
                                        "len", "cap", "chunk", "nchunk", "kpw", "scale_bits"]
    assert [x.buffer for x in a.args] == [True] * 7 + [False] * 9 and a.block == 256
    g = ks["hwk_co_i8_gemm"]
    assert [(x.name, x.size) for x in g.args][-1] == ("tiles", 4) and g.block == 256


def test_optional_buffers_from_manifest():
    """The manifest marks the buffers a kernel accepts as null (the MoE biases, the router bias); no
    other argument is optional."""
    ks = by_name(Program.load(None, image()).kernels())
    opt = {k: [a.name for a in v.args if a.nullable] for k, v in ks.items()}
    assert opt["hwk_co_moe_route"] == ["bias"]
    assert opt["hwk_co_moe_gate_up"] == ["gb"] and opt["hwk_co_moe_down"] == ["db"]
    assert all(not v for k, v in opt.items() if "moe" not in k)


def test_inspection_module_cannot_run():
    p = Program.load(None, image())
    with pytest.raises(hwk.HwkError, match="without a device"):
        p.new_run("hwk_co_mxfp4_gemv")


def test_offload_bundle_is_unpacked():
    """A clang offload bundle holding the ELF under a gfx950 triple lists the same kernels."""
    elf = image()
    triples = [b"host-x86_64-unknown-linux-gnu-", b"hipv4-amdgcn-amd-amdhsa--gfx950"]
    head = b"__CLANG_OFFLOAD_BUNDLE__" + struct.pack("<Q", 2)
    entries_len = sum(24 + len(t) for t in triples)
    off = (len(head) + entries_len + 4095) // 4096 * 4096
    ent = struct.pack("<QQQ", off, 0, len(triples[0])) + triples[0]
    ent += struct.pack("<QQQ", off, len(elf), len(triples[1])) + triples[1]
    blob = head + ent
    blob += b"\0" * (off - len(blob)) + elf
    assert set(by_name(Program.load(None, blob).kernels())) == CO_KERNELS
    no950 = blob.replace(b"gfx950", b"gfx942", 1)
    with pytest.raises(hwk.HwkError, match="gfx950"):
        Program.load(None, no950)


@pytest.mark.parametrize("mutate,match", [
    (lambda b: b[:40], "ELF"),
    (lambda b: b"\0" * 64 + b[64:], "ELF"),
    (lambda b: b.replace(b"amdgcn-amd-amdhsa--gfx950", b"amdgcn-amd-amdhsa--gfx942"), "not gfx950"),
    (lambda b: b.replace(b"AMDGPU\0", b"XMDGPU\0"), "metadata"),
])
def test_bad_images_refused(mutate, match):
    with pytest.raises(hwk.HwkError, match=match):
        Program.load(None, mutate(image()))


def test_image_without_manifest_lists_kernels_but_none_runnable():
    b = image().replace(b"hwk_co_manifest_count", b"hwk_co_manifest_xxxxx")
    ks = Program.load(None, b).kernels()
    assert ks and not any(k.runnable for k in ks) and all(k.block == 0 for k in ks)
