"""Device buffers for GPU tests through the HIP runtime the library already
loaded (ctypes on libamdhip64.so.7), without torch: torch bundles its own
ROCm runtime under the same soname, and whichever of the two a process
loads first is the one both get, so a test that brings torch in after the
library has started cannot use the device through torch."""
import ctypes as C

import numpy as np

_hip = None


def hip():
    global _hip
    if _hip is None:
        import pywelvet
        pywelvet.lib()  # the library's runtime is the one to share
        h = C.CDLL("libamdhip64.so.7")
        h.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        h.hipFree.argtypes = [C.c_void_p]
        h.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        h.hipMemset.argtypes = [C.c_void_p, C.c_int, C.c_size_t]
        h.hipDeviceSynchronize.argtypes = []
        h.hipStreamCreate.argtypes = [C.POINTER(C.c_void_p)]
        h.hipStreamDestroy.argtypes = [C.c_void_p]
        h.hipStreamSynchronize.argtypes = [C.c_void_p]
        for f in (h.hipMalloc, h.hipFree, h.hipMemcpy, h.hipMemset, h.hipDeviceSynchronize,
                  h.hipStreamCreate, h.hipStreamDestroy, h.hipStreamSynchronize):
            f.restype = C.c_int
        _hip = h
    return _hip


def _ok(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what}: hip error {rc}")


class DeviceArray:
    """An f32 buffer in HBM (hipMalloc), filled from / read into numpy."""

    def __init__(self, shape, fill=None):
        self.shape = tuple(shape)
        self.nbytes = int(np.prod(self.shape)) * 4
        p = C.c_void_p()
        _ok(hip().hipMalloc(C.byref(p), max(self.nbytes, 4)), "hipMalloc")
        self.ptr = p.value
        if fill is not None:
            self.upload(np.full(self.shape, fill, np.float32))

    def upload(self, a):
        a = np.ascontiguousarray(a, np.float32)
        assert a.nbytes == self.nbytes
        _ok(hip().hipMemcpy(self.ptr, a.ctypes.data, self.nbytes, 1), "hipMemcpy H2D")

    def download(self):
        out = np.empty(self.shape, np.float32)
        _ok(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")
        _ok(hip().hipMemcpy(out.ctypes.data, self.ptr, self.nbytes, 2), "hipMemcpy D2H")
        return out

    def free(self):
        if self.ptr:
            hip().hipFree(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        s = C.c_void_p()
        _ok(hip().hipStreamCreate(C.byref(s)), "hipStreamCreate")
        self.h = s.value

    def sync(self):
        _ok(hip().hipStreamSynchronize(self.h), "hipStreamSynchronize")

    def close(self):
        if self.h:
            hip().hipStreamDestroy(self.h)
            self.h = None
