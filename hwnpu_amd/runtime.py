"""hwnpu's backend objects over libhwk's runtime calls: the shape of the reference's Go API for a
kernel device (internal/backend/backend.go:12-118, the root package's Program/Kernel/Run,
kernel.go:109-254), as a Go binding over purego would present them.

    dev = Device.open(0)                       # Provider.Open
    buf = dev.alloc(nbytes)                    # Device.AllocBuffer; buf.bytes() is the host view
    buf.sync_to_device()                       # Buffer.SyncToDevice
    prog = dev.load_program(path=...)          # KernelDevice.LoadProgram (a gfx950 code object)
    prog.kernels()                             # Program.Kernels -> [KernelInfo]
    run = prog.new_run("hwk_co_mxfp4_gemv")    # Kernel.NewRun
    run.set_buffer(0, buf).set_uint32(4, n)    # setters keep the first error (Run.Err)
    fence = run.submit()                       # launch geometry from the code object's manifest
    fence.wait(timeout_ms)                     # cancelable: the submission keeps running

There is no CPU path: every call is libhwk's, and a missing library raises HwkLibraryError.
"""
from __future__ import annotations

import ctypes as C
import struct
from dataclasses import dataclass, field

from . import hwk


@dataclass
class KernelArg:
    index: int
    name: str
    type: str
    offset: int
    size: int
    buffer: bool
    nullable: bool = False  # an optional buffer: Run.set_null passes the null address


@dataclass
class KernelInfo:
    name: str
    args: list = field(default_factory=list)
    cus: int = 0
    block: int = 0
    kernarg_bytes: int = 0
    runnable: bool = False


class Device:
    def __init__(self, handle, index):
        self._h = handle
        self.index = index

    @staticmethod
    def count() -> int:
        n = C.c_uint32()
        hwk.load().hwk_device_count(C.byref(n))
        return n.value

    @classmethod
    def open(cls, index: int = 0) -> "Device":
        h = C.c_void_p()
        hwk.load().hwk_device_open(index, C.byref(h))
        return cls(h, index)

    def info(self, key: int) -> str:
        need = C.c_size_t()
        buf = C.create_string_buffer(256)
        hwk.load().hwk_device_info(self._h, key, buf, 256, C.byref(need))
        return buf.value.decode()

    def alloc(self, size: int, kind: int = hwk.BUF_MIRRORED) -> "Buffer":
        h = C.c_void_p()
        hwk.load().hwk_buf_alloc(self._h, size, kind, C.byref(h))
        return Buffer(h, size)

    def load_program(self, path: str | None = None, image: bytes | None = None) -> "Program":
        if image is None:
            with open(path, "rb") as f:
                image = f.read()
        return Program.load(self, image)

    def synchronize(self):
        hwk.load().hwk_device_synchronize(self._h)

    def close(self):
        if self._h:
            hwk.load().hwk_device_free(self._h)
            self._h = None


class Buffer:
    def __init__(self, handle, size):
        self._h = handle
        self.size = size

    def bytes(self) -> memoryview:
        """The pinned host mirror (zero-copy view, valid until close)."""
        p = hwk.load().hwk_buf_host_ptr(self._h)
        if not p:
            raise hwk.HwkError("device-only buffer has no host view")
        return memoryview((C.c_char * self.size).from_address(p)).cast("B")

    def device_address(self) -> int:
        return hwk.load().hwk_buf_dev_ptr(self._h)

    def sync_to_device(self, off: int = 0, n: int | None = None):
        hwk.load().hwk_buf_sync(self._h, hwk.SYNC_TO_DEVICE, off, self.size - off if n is None else n)

    def sync_from_device(self, off: int = 0, n: int | None = None):
        hwk.load().hwk_buf_sync(self._h, hwk.SYNC_FROM_DEVICE, off, self.size - off if n is None else n)

    def close(self):
        if self._h:
            hwk.load().hwk_buf_free(self._h)
            self._h = None


class Program:
    def __init__(self, handle, device):
        self._h = handle
        self.device = device

    @classmethod
    def load(cls, device: Device | None, image: bytes) -> "Program":
        """device None: the code object's kernels are listed, nothing runs (no HIP call)."""
        h = C.c_void_p()
        buf = C.create_string_buffer(image, len(image))
        hwk.load().hwk_module_load(device._h if device else None, buf, len(image), C.byref(h))
        return cls(h, device)

    def kernels(self) -> list:
        L = hwk.load()
        n = C.c_uint32()
        L.hwk_module_kernel_count(self._h, C.byref(n))
        out = []
        for i in range(n.value):
            ki = hwk.KernelInfo()
            L.hwk_module_kernel_info(self._h, i, C.byref(ki))
            args = []
            for a in range(ki.args):
                ka = hwk.KernelArg()
                L.hwk_module_kernel_arg(self._h, i, a, C.byref(ka))
                args.append(KernelArg(ka.index, ka.name.decode(), ka.type.decode(), ka.offset, ka.size, bool(ka.buffer),
                                      bool(ka.nullable)))
            out.append(KernelInfo(ki.name.decode(), args, ki.cus, ki.block, ki.kernarg_bytes, bool(ki.runnable)))
        return out

    def new_run(self, kernel: str) -> "Run":
        h = C.c_void_p()
        hwk.load().hwk_run_new(self._h, kernel.encode(), C.byref(h))
        return Run(h)

    def close(self):
        if self._h:
            hwk.load().hwk_module_free(self._h)
            self._h = None


class Fence:
    def __init__(self, run):
        self._run = run

    def wait(self, timeout_ms: int = 60000) -> bool:
        """True when the submission finished within timeout_ms; False when it is still running."""
        st = C.c_int()
        hwk.load().hwk_run_wait(self._run._h, timeout_ms, C.byref(st))
        return st.value == hwk.STATE_DONE

    def done(self) -> bool:
        return self.wait(0)


class Run:
    """Setters record the first error and return self; err() gives it and submit() raises it."""

    def __init__(self, handle):
        self._h = handle

    def _set(self, fn, *args):
        try:
            fn(self._h, *args)
        except hwk.HwkError:
            pass  # kept by the library as the run's first error
        return self

    def set_bytes(self, index: int, value: bytes) -> "Run":
        b = C.create_string_buffer(value, len(value))
        return self._set(hwk.load().hwk_run_set_arg, index, b, len(value))

    def set_uint32(self, index: int, v: int) -> "Run":
        return self.set_bytes(index, struct.pack("<I", v))

    def set_uint64(self, index: int, v: int) -> "Run":
        return self.set_bytes(index, struct.pack("<Q", v))

    def set_buffer(self, index: int, b: Buffer) -> "Run":
        return self._set(hwk.load().hwk_run_set_buffer, index, b._h if b else None)

    def set_buffer_at(self, index: int, b: Buffer, off: int, n: int) -> "Run":
        return self._set(hwk.load().hwk_run_set_buffer_at, index, b._h if b else None, off, n)

    def set_null(self, index: int) -> "Run":
        """An optional buffer argument (KernelArg.nullable) set to the null address."""
        return self._set(hwk.load().hwk_run_set_null, index)

    def err(self) -> str | None:
        try:
            hwk.load().hwk_run_err(self._h)
        except hwk.HwkError as e:
            return str(e)
        return None

    def submit(self, stream: int | None = None) -> Fence:
        hwk.load().hwk_run_submit(self._h, stream)
        return Fence(self)

    def close(self):
        if self._h:
            h, self._h = self._h, None
            hwk.load().hwk_run_free(h)
