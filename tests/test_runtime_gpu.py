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
