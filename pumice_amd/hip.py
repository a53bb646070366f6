"""Minimal ctypes view of the HIP runtime: device / pinned memory, copies,
streams and events.  Plumbing for tests and benchmarks; the sampler itself is
the C ABI in libpumice_sampler.so.

The HIP runtime is resolved after the sampler library is loaded, so both use
the one libamdhip64.so.7 already mapped into the process.
"""
import ctypes

import numpy as np

_hip = None

hipMemcpyHostToDevice = 1
hipMemcpyDeviceToHost = 2
hipMemcpyDeviceToDevice = 3
hipHostMallocMapped = 0x2


class HipError(RuntimeError):
    pass


def rt():
    global _hip
    if _hip is None:
        from . import sampler  # loads libpumice_sampler.so (and its HIP runtime) first

        sampler.lib()
        try:
            h = ctypes.CDLL("libamdhip64.so.7")
        except OSError:
            h = ctypes.CDLL("/opt/rocm/lib/libamdhip64.so.7")
        P, S, I = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
        sig = {
            "hipMalloc": [ctypes.POINTER(P), S],
            "hipFree": [P],
            "hipHostMalloc": [ctypes.POINTER(P), S, ctypes.c_uint],
            "hipHostFree": [P],
            "hipHostGetDevicePointer": [ctypes.POINTER(P), P, ctypes.c_uint],
            "hipMemcpy": [P, P, S, I],
            "hipMemcpyAsync": [P, P, S, I, P],
            "hipMemsetD32": [P, ctypes.c_int, S],
            "hipDeviceSynchronize": [],
            "hipStreamSynchronize": [P],
            "hipStreamCreate": [ctypes.POINTER(P)],
            "hipStreamDestroy": [P],
            "hipEventCreate": [ctypes.POINTER(P)],
            "hipEventDestroy": [P],
            "hipEventRecord": [P, P],
            "hipEventSynchronize": [P],
            "hipEventElapsedTime": [ctypes.POINTER(ctypes.c_float), P, P],
            "hipGetDeviceCount": [ctypes.POINTER(I)],
            "hipGetLastError": [],
        }
        for name, args in sig.items():
            f = getattr(h, name)
            f.argtypes = args
            f.restype = I
        h.hipGetErrorString.argtypes = [I]
        h.hipGetErrorString.restype = ctypes.c_char_p
        _hip = h
    return _hip


def check(err, what=""):
    if err != 0:
        raise HipError(f"{what}: HIP error {err} ({rt().hipGetErrorString(err).decode()})")


def device_count():
    n = ctypes.c_int(0)
    err = rt().hipGetDeviceCount(ctypes.byref(n))
    return n.value if err == 0 else 0


def synchronize():
    check(rt().hipDeviceSynchronize(), "hipDeviceSynchronize")


class DeviceBuffer:
    """Device allocation of `nbytes`; upload / download numpy arrays."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(rt().hipMalloc(ctypes.byref(p), max(self.nbytes, 4)), "hipMalloc")
        self.ptr = p.value

    @classmethod
    def from_array(cls, a):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a, offset=0):
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        check(rt().hipMemcpy(self.ptr + offset, a.ctypes.data, a.nbytes, hipMemcpyHostToDevice), "upload")

    def download(self, dtype, shape, offset=0):
        out = np.empty(shape, dtype)
        assert offset + out.nbytes <= self.nbytes
        check(rt().hipMemcpy(out.ctypes.data, self.ptr + offset, out.nbytes, hipMemcpyDeviceToHost), "download")
        return out

    def fill_u32(self, value):
        check(rt().hipMemsetD32(self.ptr, ctypes.c_int(np.uint32(value).view(np.int32)), self.nbytes // 4), "memset")

    def free(self):
        if self.ptr:
            rt().hipFree(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class PinnedBuffer:
    """Pinned, device-mapped host memory (hipHostMalloc + Mapped)."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(rt().hipHostMalloc(ctypes.byref(p), max(self.nbytes, 4), hipHostMallocMapped), "hipHostMalloc")
        self.ptr = p.value
        d = ctypes.c_void_p()
        check(rt().hipHostGetDevicePointer(ctypes.byref(d), self.ptr, 0), "hipHostGetDevicePointer")
        self.dev_ptr = d.value

    def view(self, dtype, count):
        buf = (ctypes.c_char * self.nbytes).from_address(self.ptr)
        return np.frombuffer(buf, dtype=dtype, count=count)

    def free(self):
        if self.ptr:
            rt().hipHostFree(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Event:
    def __init__(self):
        e = ctypes.c_void_p()
        check(rt().hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        self.ptr = e.value

    def record(self, stream):
        check(rt().hipEventRecord(self.ptr, stream), "hipEventRecord")

    def synchronize(self):
        check(rt().hipEventSynchronize(self.ptr), "hipEventSynchronize")

    def elapsed_ms(self, end):
        ms = ctypes.c_float(0)
        check(rt().hipEventElapsedTime(ctypes.byref(ms), self.ptr, end.ptr), "hipEventElapsedTime")
        return ms.value

    def __del__(self):
        try:
            rt().hipEventDestroy(self.ptr)
        except Exception:
            pass


def stream_sync(stream):
    check(rt().hipStreamSynchronize(stream), "hipStreamSynchronize")
