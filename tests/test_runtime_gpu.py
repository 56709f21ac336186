"""The runtime half of the boundary on the GPU, through libhwk's C ABI only: device enumeration and
info, mirrored buffers synced explicitly, the library's gfx950 code object loaded as a program, a run
of its MXFP4 GEMV with arguments set by index (size-checked) and the launch geometry taken from the
code object's manifest, its fence, and the refusals the reference's AMD backend makes (a wrong
argument size, a buffer where a value goes and the reverse, a submit while the previous submission
still runs; internal/backend/amd/device.go:349-401). The GEMV's output is checked against the CPU
oracle (dequantize + fp32 GEMM) and equals hwk_mxfp4_gemv's bit for bit."""
import ctypes as C
import struct

import numpy as np
import pytest
import torch

from hwnpu_amd import hwk, ops
from hwnpu_amd.runtime import Device, Program

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def device(dev):
    d = Device.open(0)
    yield d
    d.close()


@pytest.fixture(scope="module")
def program(device):
    p = device.load_program(path=hwk.CODE_OBJECT_PATH)
    yield p
    p.close()


def test_device_enumerate_and_info(device):
    assert Device.count() >= 1
    assert device.info(hwk.INFO_ARCH).startswith("gfx950")
    assert int(device.info(hwk.INFO_CUS)) > 0
    assert int(device.info(hwk.INFO_MEM_BYTES)) > (1 << 30)
    assert device.info(hwk.INFO_NAME)
    assert device.info(hwk.INFO_PCI_BUS).count(":") == 2
    with pytest.raises(hwk.HwkError, match="device 99"):
        Device.open(99)


def test_buffer_round_trip(device):
    b = device.alloc(1 << 20)
    try:
        v = np.frombuffer(b.bytes(), np.uint8)
        v[:] = np.arange(1 << 20, dtype=np.uint64).astype(np.uint8)
        b.sync_to_device()
        v[:] = 0
        b.sync_from_device(4096, 8192)
        assert np.array_equal(v[4096:4096 + 8192], (np.arange(4096, 4096 + 8192) % 256).astype(np.uint8))
        assert not v[:4096].any()
        assert b.device_address() != 0
        with pytest.raises(hwk.HwkError, match="past"):
            b.sync_from_device(1 << 20, 1)
    finally:
        b.close()
    d = device.alloc(4096, hwk.BUF_DEVICE)
    try:
        with pytest.raises(hwk.HwkError, match="no host"):
            d.bytes()
    finally:
        d.close()


def test_program_kernels_on_device(program, device):
    ks = {k.name: k for k in program.kernels()}
    assert ks["hwk_co_mxfp4_gemv"].cus == int(device.info(hwk.INFO_CUS))
    assert all(k.runnable for k in ks.values())
    with pytest.raises(hwk.HwkError, match="no kernel"):
        program.new_run("nope")


def _gemv_inputs(device, n, k, seed):
    rng = np.random.default_rng(seed)
    w = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    e = rng.integers(123, 130, (n, k // 32), dtype=np.uint8)
    x = rng.standard_normal(k).astype(np.float16)
    bufs = []
    for arr in (w, e, x):
        b = device.alloc(arr.nbytes)
        np.frombuffer(b.bytes(), np.uint8)[:] = arr.view(np.uint8).ravel()
        b.sync_to_device()
        bufs.append(b)
    y = device.alloc(n * 2)
    return (w, e, x), bufs + [y]


@pytest.mark.parametrize("n,k", [(8192, 2048), (100, 2048), (37, 1056)])
def test_gemv_run_vs_oracle(device, program, orc, n, k):
    print(f"code-object gemv n={n} k={k}", flush=True)
    (w, e, x), (bw, be, bx, by) = _gemv_inputs(device, n, k, n + k)
    run = program.new_run("hwk_co_mxfp4_gemv")
    try:
        run.set_buffer(0, bw).set_buffer(1, be).set_buffer(2, bx).set_buffer(3, by).set_uint32(4, n).set_uint32(5, k // 32)
        assert run.err() is None
        fence = run.submit()
        assert fence.wait(60000)
        by.sync_from_device()
        got = np.frombuffer(by.bytes(), np.float16).copy()
        wd = orc.mxfp4_dequantize(w, e)
        want = orc.sgemm(x.astype(np.float32)[None, :], wd, transb=True)[0]
        rms = float(np.sqrt(np.mean(want.astype(np.float64) ** 2)))
        # fp16 output: RNE of a float32 within the bar, so the bar plus half an fp16 ulp of each value
        tol = 2e-3 * rms + np.abs(want) * 2.0 ** -11
        assert np.all(np.abs(got.astype(np.float64) - want) <= tol)
        if k == 2048:  # 64 blocks a row: the library's entry point runs the same kernel, bit-identical
            t = [torch.from_numpy(a).cuda() for a in (w, e, x)]
            lib = ops.mxfp4_gemv(t[0], t[1], t[2], "f16").cpu().numpy()
            assert np.array_equal(lib.view(np.uint16), got.view(np.uint16))
    finally:
        run.close()
        for b in (bw, be, bx, by):
            b.close()


def test_gemv_rows_past_build_are_nan(device, program):
    (w, e, x), (bw, be, bx, by) = _gemv_inputs(device, 16, 4096, 3)
    run = program.new_run("hwk_co_mxfp4_gemv")
    try:
        run.set_buffer(0, bw).set_buffer(1, be).set_buffer(2, bx).set_buffer(3, by).set_uint32(4, 16).set_uint32(5, 128)
        assert run.submit().wait(60000)
        by.sync_from_device()
        assert np.all(np.isnan(np.frombuffer(by.bytes(), np.float16)))
    finally:
        run.close()
        for b in (bw, be, bx, by):
            b.close()


def test_argument_checks_and_first_error(device, program):
    b = device.alloc(4096)
    run = program.new_run("hwk_co_mxfp4_gemv")
    try:
        L = hwk.load()
        with pytest.raises(hwk.HwkError, match="takes 4 bytes, got 8"):
            L.hwk_run_set_arg(run._h, 4, C.create_string_buffer(8), 8)
        with pytest.raises(hwk.HwkError, match="is a buffer"):
            L.hwk_run_set_arg(run._h, 0, C.create_string_buffer(8), 8)
        with pytest.raises(hwk.HwkError, match="not a buffer"):
            L.hwk_run_set_buffer(run._h, 4, b._h)
        with pytest.raises(hwk.HwkError, match="no argument 9"):
            L.hwk_run_set_arg(run._h, 9, C.create_string_buffer(4), 4)
        with pytest.raises(hwk.HwkError, match="byte buffer"):
            L.hwk_run_set_buffer_at(run._h, 0, b._h, 4000, 200)
        # the first error is kept and refuses the submit
        assert "takes 4 bytes, got 8" in run.err()
        with pytest.raises(hwk.HwkError, match="takes 4 bytes, got 8"):
            run.submit()
    finally:
        run.close()
        b.close()


def test_unset_buffer_refused_and_empty_grid_launches_nothing(device, program):
    """A submit with a buffer argument never set is refused before any launch (the kernel would
    read a null address); a grid argument of 0 launches nothing and its fence still completes."""
    (w, e, x), (bw, be, bx, by) = _gemv_inputs(device, 16, 2048, 5)
    np.frombuffer(by.bytes(), np.uint16)[:] = 0x7bff
    by.sync_to_device()
    run = program.new_run("hwk_co_mxfp4_gemv")
    try:
        run.set_buffer(0, bw).set_buffer(1, be).set_buffer(2, bx).set_uint32(4, 16).set_uint32(5, 64)
        with pytest.raises(hwk.HwkError, match="never set"):
            run.submit()
        run.set_buffer(3, by).set_uint32(4, 0)
        assert run.submit().wait(60000)
        by.sync_from_device()
        assert np.all(np.frombuffer(by.bytes(), np.uint16) == 0x7bff)
        run.set_uint32(4, 16)
        assert run.submit().wait(60000)
        by.sync_from_device()
        assert not np.any(np.frombuffer(by.bytes(), np.uint16) == 0x7bff)
    finally:
        run.close()
        for b in (bw, be, bx, by):
            b.close()


def test_submit_while_running_refused(device, program):
    """A GEMV run queued behind 2 GB of streaming reads on one stream is still running when it is
    submitted again: the second submit is refused; after its fence it runs again."""
    L = hwk.load()
    st = C.c_void_p()
    L.hwk_stream_new(device._h, C.byref(st))
    big = device.alloc(2 << 30, hwk.BUF_DEVICE)
    sink = device.alloc((2 << 30) // 16 // 256 * 4 + 4096, hwk.BUF_DEVICE)
    (w, e, x), (bw, be, bx, by) = _gemv_inputs(device, 8192, 2048, 9)
    reads = [program.new_run("hwk_co_stream_read") for _ in range(4)]
    gemv = program.new_run("hwk_co_mxfp4_gemv")
    try:
        for r in reads:
            r.set_buffer(0, big).set_uint32(1, (2 << 30) // 16).set_buffer(2, sink)
        gemv.set_buffer(0, bw).set_buffer(1, be).set_buffer(2, bx).set_buffer(3, by).set_uint32(4, 8192).set_uint32(5, 64)
        for r in reads:
            r.submit(st.value)
        fence = gemv.submit(st.value)
        with pytest.raises(hwk.HwkError, match="still running"):
            gemv.submit(st.value)
        assert fence.wait(60000)
        gemv.submit(st.value).wait(60000)
        # events around a run on the same stream
        a, b2 = C.c_void_p(), C.c_void_p()
        L.hwk_event_new(device._h, C.byref(a))
        L.hwk_event_new(device._h, C.byref(b2))
        L.hwk_event_record(a, st.value)
        reads[0].submit(st.value)
        L.hwk_event_record(b2, st.value)
        state = C.c_int()
        L.hwk_event_wait(b2, 60000, C.byref(state))
        assert state.value == hwk.STATE_DONE
        ns = C.c_uint64()
        L.hwk_event_elapsed_ns(a, b2, C.byref(ns))
        assert ns.value > 0
        print(f"2 GB streaming read: {ns.value / 1e3:.1f} us, {(2 << 30) / ns.value:.0f} GB/s", flush=True)
        L.hwk_event_free(a)
        L.hwk_event_free(b2)
    finally:
        for r in reads + [gemv]:
            r.close()
        for b in (big, sink, bw, be, bx, by):
            b.close()
        L.hwk_stream_free(st)


# ---- the code object's attention, GEMM and MoE kernels: runs through the runtime (arguments by
# index, geometry from the manifest) against the library's entry points on the same inputs (the
# same device code, so the same bits) and against the oracle ----

def _buf(device, arr):
    a = np.ascontiguousarray(arr)
    b = device.alloc(max(a.nbytes, 16))
    np.frombuffer(b.bytes(), np.uint8)[:a.nbytes] = a.reshape(-1).view(np.uint8)
    b.sync_to_device()
    return b


def _read(b, dtype, n):
    b.sync_from_device()
    return np.frombuffer(b.bytes(), dtype)[:n].copy()


def _f32_bits(v):
    return struct.unpack("<I", struct.pack("<f", v))[0]


def _close_all(*objs):
    for o in objs:
        if o is not None:
            o.close()


@pytest.mark.parametrize("L,int8", [(2048, False), (1000, False), (96, False), (2048, True)])
def test_co_attention_matches_library(device, program, orc, L, int8):
    """hwk_co_attn_decode_* (+ hwk_co_attn_merge past one chunk) at the GQA decode configuration (32
    query heads, 8 kv heads, head_dim 128): equal to hwk_attn_decode's output on the same caches,
    and within the kernel bar of the oracle's chunk attention + Merge."""
    import math

    from hwnpu_amd import synth

    print(f"code-object attention L={L} int8={int8}", flush=True)
    heads, kvh, cap, kpw = 32, 8, L, 32
    q = synth.normal(heads * 128, f"co.attn.q.{L}").view(heads, 128)
    k = synth.normal(kvh * cap * 128, f"co.attn.k.{L}").view(kvh, cap, 128)
    v = synth.normal(kvh * cap * 128, f"co.attn.v.{L}").view(kvh, cap, 128)
    ks = vs = None
    if int8:
        k, ks = ops.kv_quantize_i8(k)
        v, vs = ops.kv_quantize_i8(v)
    # the library's split set to the code object's (4 waves of kpw keys a workgroup)
    want = ops.attn_decode(q, k, v, L, ks, vs, out_mode="f16", split=4 * kpw).cpu().numpy()
    chunk, nchunk = 4 * kpw, -(-L // (4 * kpw))
    slots = heads * nchunk
    arrs = [q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy()] + ([ks.cpu().numpy(), vs.cpu().numpy()] if int8 else [])
    bufs = [_buf(device, a) for a in arrs]
    wo, wm, wl = (device.alloc(slots * 128 * 4), device.alloc(slots * 4), device.alloc(slots * 4))
    out = device.alloc(heads * 128 * 2)
    name = "hwk_co_attn_decode_i8_g4" if int8 else "hwk_co_attn_decode_f16_g4"
    run = program.new_run(name)
    merge = program.new_run("hwk_co_attn_merge")
    try:
        for i, b in enumerate(bufs):
            run.set_buffer(i, b)
        base = len(bufs)
        run.set_buffer(base, wo).set_buffer(base + 1, wm).set_buffer(base + 2, wl).set_buffer(base + 3, out)
        for j, val in enumerate((kvh * nchunk, kvh, 1, L, cap, chunk, nchunk, kpw, _f32_bits(1 / math.sqrt(128)))):
            run.set_uint32(base + 4 + j, val)
        assert run.err() is None
        assert run.submit().wait(60000)
        if nchunk > 1:
            merge.set_buffer(0, wo).set_buffer(1, wm).set_buffer(2, wl).set_buffer(3, out)
            merge.set_uint32(4, heads * 8).set_uint32(5, nchunk).set_uint32(6, heads // kvh).set_uint32(7, 1)
            assert merge.err() is None
            assert merge.submit().wait(60000)
        got = _read(out, np.float16, heads * 128).reshape(heads, 128)
        assert np.array_equal(got, want)  # fp16 values: the same device code on the same inputs
        kf, vf = k.cpu().numpy().astype(np.float32), v.cpu().numpy().astype(np.float32)
        if int8:
            kf = kf * ks.cpu().numpy().astype(np.float32)[..., None]
            vf = vf * vs.cpu().numpy().astype(np.float32)[..., None]
        ref = orc.attn_decode(q.cpu().numpy().astype(np.float32), kf, vf, 1 / math.sqrt(128))
        rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
        tol = 2e-3 * rms + np.abs(ref) * 2.0 ** -11
        assert np.all(np.abs(got.astype(np.float64) - ref) <= tol)
    finally:
        _close_all(run, merge, *bufs, wo, wm, wl, out)


def test_co_attention_bad_shape_is_nan(device, program):
    """A chunking that does not cover the keys (chunk * nchunk < len) writes NaN, reads nothing."""
    heads, kvh, L = 32, 8, 256
    bufs = [device.alloc(heads * 128 * 2), device.alloc(kvh * L * 256), device.alloc(kvh * L * 256)]
    ws = [device.alloc(heads * 128 * 4), device.alloc(heads * 4), device.alloc(heads * 4)]
    out = device.alloc(heads * 128 * 2)
    run = program.new_run("hwk_co_attn_decode_f16_g4")
    try:
        for i, b in enumerate(bufs + ws + [out]):
            run.set_buffer(i, b)
        for j, val in enumerate((kvh, kvh, 1, L, L, 128, 1, 32, _f32_bits(0.088))):
            run.set_uint32(7 + j, val)
        assert run.submit().wait(60000)
        assert np.all(np.isnan(_read(out, np.float16, heads * 128)))
    finally:
        _close_all(run, *bufs, *ws, out)


@pytest.mark.parametrize("mx,m,n,k", [(False, 512, 768, 2048), (False, 200, 320, 256), (True, 256, 512, 2048),
                                      (True, 70, 160, 1056)])
def test_co_gemm_matches_library(device, program, orc, mx, m, n, k):
    """hwk_co_i8_gemm / hwk_co_mxfp4_gemm against hwk_i8_gemm / hwk_mxfp4_gemm (fp16 out) on the same
    operands, and against the oracle's dequant + fp32 GEMM."""
    from hwnpu_amd import synth

    print(f"code-object gemm mx={mx} {m}x{n}x{k}", flush=True)
    x = synth.normal(m * k, f"co.gemm.x.{m}.{k}").view(m, k)
    if mx:
        w, e = synth.mxfp4_uniform(n, k, f"co.gemm.w.{n}.{k}")
        want = ops.mxfp4_gemm(x, w, e, "f16").cpu().numpy()
        wd = orc.mxfp4_dequantize(w.cpu().numpy(), e.cpu().numpy())
        arrs = [x.cpu().numpy(), w.cpu().numpy(), e.cpu().numpy()]
    else:
        w = synth.uniform_int(n * k, -127, 255, f"co.gemm.q.{n}.{k}", dtype=torch.int8).view(n, k)
        s = synth.uniform_real(n, 0.002, 0.02, f"co.gemm.s.{n}")
        want = ops.i8_gemm(x, w, s, "f16").cpu().numpy()
        wd = orc.i8_dequant(w.cpu().numpy(), s.cpu().numpy().view(np.uint16))
        arrs = [x.cpu().numpy(), w.cpu().numpy(), s.cpu().numpy()]
    bufs = [_buf(device, a) for a in arrs]
    y = device.alloc(m * n * 2)
    run = program.new_run("hwk_co_mxfp4_gemm" if mx else "hwk_co_i8_gemm")
    try:
        for i, b in enumerate(bufs):
            run.set_buffer(i, b)
        run.set_buffer(3, y)
        tiles = -(-m // 128) * -(-n // 128)
        for j, val in enumerate((m, n, k, 1, tiles)):
            run.set_uint32(4 + j, val)
        assert run.err() is None
        assert run.submit().wait(60000)
        got = _read(y, np.float16, m * n).reshape(m, n)
        assert np.array_equal(got, want)
        ref = orc.sgemm(x.cpu().numpy().astype(np.float32), wd, transb=True)
        rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
        assert float(np.max(np.abs(got.astype(np.float64) - ref) - np.abs(ref) * 2.0 ** -11)) <= 2e-3 * rms
    finally:
        _close_all(run, *bufs, y)


@pytest.mark.parametrize("T,biases", [(5, False), (1, False), (3, True)])
def test_co_moe_matches_library(device, program, orc, T, biases):
    """hwk_co_moe_route, hwk_co_moe_gate_up and hwk_co_moe_down (the MoE configuration: hidden 2048, 32
    experts, top-4, intermediate 768) against hwk_moe_route + hwk_moe_experts on the same operands:
    idx and w bit-exact, the output equal; with gpt-oss's unit and biases, and without biases through
    the null address of the optional bias arguments."""
    from test_moe_gpu import experts_case

    from hwnpu_amd import synth

    print(f"code-object moe T={T} biases={biases}", flush=True)
    E, H, I, k = 32, 2048, 768, 4
    x, logits, gw, ge, dw, de = experts_case(T, name="co.moe")
    idx_l, w_l = ops.moe_route(logits, k)
    kw = {}
    if biases:
        gb = synth.normal(E * 2 * I, "co.moe.gb", std=0.1, dtype=torch.float32).view(E, 2 * I)
        db = synth.normal(E * H, "co.moe.db", std=0.1, dtype=torch.float32).view(E, H)
        kw = dict(gu_b=gb, dn_b=db, act="gptoss", alpha=1.702, limit=7.0)
    want = ops.moe_experts(x, idx_l, w_l, gw, ge, dw, de, **kw).cpu().numpy()
    bl = {n: _buf(device, t.cpu().numpy()) for n, t in (("x", x), ("logits", logits), ("gw", gw), ("ge", ge),
                                                          ("dw", dw), ("de", de))}
    if biases:
        bl["gb"], bl["db"] = _buf(device, kw["gu_b"].cpu().numpy()), _buf(device, kw["dn_b"].cpu().numpy())
    idx, w = device.alloc(T * k * 4), device.alloc(T * k * 4)
    act, out = device.alloc(T * k * I * 4), device.alloc(T * H * 4)
    route, gu, dn = (program.new_run(n) for n in ("hwk_co_moe_route", "hwk_co_moe_gate_up", "hwk_co_moe_down"))
    try:
        route.set_buffer(0, bl["logits"]).set_null(1).set_buffer(2, idx).set_buffer(3, w)
        for j, val in enumerate((T, E, k, 0, 1, 0)):
            route.set_uint32(4 + j, val)
        gu.set_buffer(0, bl["x"]).set_buffer(1, idx).set_buffer(2, bl["gw"]).set_buffer(3, bl["ge"])
        gu.set_buffer(4, bl["gb"]) if biases else gu.set_null(4)
        gu.set_buffer(5, act)
        act_kind, alpha, limit = (1, _f32_bits(1.702), _f32_bits(7.0)) if biases else (0, 0, 0)
        for j, val in enumerate((T, H, I, E, k, act_kind, alpha, limit, -(-I // 8) * min(T * k, E))):
            gu.set_uint32(6 + j, val)
        dn.set_buffer(0, act).set_buffer(1, idx).set_buffer(2, w).set_buffer(3, bl["dw"]).set_buffer(4, bl["de"])
        dn.set_buffer(5, bl["db"]) if biases else dn.set_null(5)
        dn.set_buffer(6, out)
        for j, val in enumerate((T, H, I, E, k, 0)):
            dn.set_uint32(7 + j, val)
        for r in (route, gu, dn):
            assert r.err() is None
            assert r.submit().wait(60000)
        assert np.array_equal(_read(idx, np.int32, T * k), idx_l.cpu().numpy().reshape(-1))
        assert np.array_equal(_read(w, np.uint32, T * k), w_l.cpu().numpy().reshape(-1).view(np.uint32))
        got = _read(out, np.float32, T * H).reshape(T, H)
        assert np.array_equal(got, want)
    finally:
        _close_all(route, gu, dn, *bl.values(), idx, w, act, out)


def test_co_set_null_refuses_required_buffers(device, program):
    run = program.new_run("hwk_co_moe_down")
    try:
        with pytest.raises(hwk.HwkError, match="not an optional buffer"):
            hwk.load().hwk_run_set_null(run._h, 0)  # act is required
        with pytest.raises(hwk.HwkError, match="not an optional buffer"):
            hwk.load().hwk_run_set_null(run._h, 7)  # a value argument
    finally:
        run.close()
