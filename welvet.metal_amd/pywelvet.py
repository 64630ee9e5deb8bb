"""ctypes binding of libwelvet_hip.so (include/welvet_c.h).

The argument lists follow the reference's own ctypes use of the same ABI
(scripts/release_smoke.py:38-44).  This module is the host-side mirror used by
the tests and bench.py; it loads only the HIP library and raises when the
library is missing, so nothing here can fall back to a CPU path.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libwelvet_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "welvet_c.h")

# include/welvet/dtype.hpp:9-44
DTYPE_NAMES = [
    "float64", "float32", "float16", "bfloat16", "fp8e4m3", "fp8e5m2", "int64", "int32",
    "int16", "int8", "uint64", "uint32", "uint16", "uint8", "int4", "uint4", "fp4", "int2",
    "uint2", "ternary", "binary", "int", "uint", "uintptr", "complex64", "complex128", "nf4",
    "fp6", "int6", "uint6", "int5", "uint5", "int3", "uint3",
]
DTYPE = {n: i for i, n in enumerate(DTYPE_NAMES)}
# bits per element of each dtype's native code (include/welvet/dtype.hpp order)
DTYPE_BITS = [64, 32, 16, 16, 8, 8, 64, 32, 16, 8, 64, 32, 16, 8, 4, 4, 4, 2, 2, 2, 1, 64, 64, 64,
              64, 128, 4, 6, 6, 6, 5, 5, 3, 3]


def dtype_bits(dtype: int) -> int:
    return DTYPE_BITS[dtype]
ACT = {"linear": -1, "relu": 0, "silu": 1, "gelu": 2, "tanh": 3, "sigmoid": 4, "leakyrelu": 5,
       "relu2": 6}


class Status(C.Structure):
    _fields_ = [("code", C.c_int32), ("message", C.c_char * 256)]


class WelvetError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"welvet code={code}: {message}")
        self.code = code


_f = C.POINTER(C.c_float)
_d = C.POINTER(C.c_double)
_u8 = C.POINTER(C.c_uint8)


class Blob(C.Structure):
    """welvet_metal_blob: a library-owned byte buffer."""
    _fields_ = [("data", C.POINTER(C.c_uint8)), ("size", C.c_size_t)]
_vp = C.c_void_p
_i32 = C.c_int32


def _fp(a):
    return None if a is None else a.ctypes.data_as(_f)


def _dp(a):
    return None if a is None else a.ctypes.data_as(_d)


_LIB = None


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} is not built: run python welvet.metal_amd/build.py")
        L = C.CDLL(LIB_PATH)
        L.welvet_version.restype = C.c_char_p
        L.welvet_runtime_identity.restype = C.c_char_p
        L.welvet_metal_init.restype = Status
        L.welvet_metal_available.restype = _i32
        geometry = [_i32] * 6
        prefix = geometry + [_f, _d, C.c_size_t, _f]
        L.welvet_dense_forward_f32.argtypes = prefix + [_f, _f]
        L.welvet_dense_forward_f32.restype = Status
        L.welvet_dense_normalbp_f32.argtypes = prefix + [_f, _i32, C.c_double] + [_f] * 5 + [_d]
        L.welvet_dense_normalbp_f32.restype = Status
        sw = [_i32] * 6 + [_f] * 4
        L.welvet_swiglu_forward_f32.argtypes = sw + [_f, _f]
        L.welvet_swiglu_forward_f32.restype = Status
        L.welvet_swiglu_normalbp_f32.argtypes = sw + [_f, _i32, C.c_double] + [_f] * 5 + [_d]
        L.welvet_swiglu_normalbp_f32.restype = Status
        ch = [_i32] * 7 + [_f, _f]
        for nm in ("sequential", "residual"):
            getattr(L, f"welvet_{nm}_forward_f32").argtypes = ch + [_f, _f]
            getattr(L, f"welvet_{nm}_forward_f32").restype = Status
            getattr(L, f"welvet_{nm}_normalbp_f32").argtypes = ch + [_f, _i32, C.c_double] + \
                [_f] * 5 + [_d]
            getattr(L, f"welvet_{nm}_normalbp_f32").restype = Status
        _bp = C.POINTER(Blob)
        L.welvet_model_abi_version.argtypes = []
        L.welvet_model_abi_version.restype = _i32
        L.welvet_model_mount.argtypes = [_u8, C.c_size_t, C.POINTER(_vp)]
        L.welvet_model_mount.restype = Status
        for nm in ("forward", "forward_pair", "backward"):
            getattr(L, f"welvet_model_{nm}").argtypes = [_vp, _u8, C.c_size_t, _bp]
            getattr(L, f"welvet_model_{nm}").restype = Status
        L.welvet_model_apply_sgd.argtypes = [_vp, C.c_double, _u8, C.c_size_t]
        L.welvet_model_apply_sgd.restype = Status
        L.welvet_model_train_mse.argtypes = [_vp, _i32, C.c_double, _i32, _u8, C.c_size_t, _d]
        L.welvet_model_train_mse.restype = Status
        L.welvet_model_export_weights.argtypes = [_vp, _bp]
        L.welvet_model_export_weights.restype = Status
        L.welvet_model_sync.argtypes = [_vp, _i32]
        L.welvet_model_sync.restype = Status
        L.welvet_model_release.argtypes = [_vp]
        L.welvet_model_release.restype = None
        L.welvet_metal_blob_free.argtypes = [_bp]
        L.welvet_metal_blob_free.restype = None
        L.welvet_hip_swiglu_mount.argtypes = [_i32] * 4 + [_f] * 3 + [C.POINTER(_vp)]
        L.welvet_hip_swiglu_mount.restype = Status
        L.welvet_hip_swiglu_forward_device.argtypes = [_vp] * 5
        L.welvet_hip_swiglu_forward_device.restype = Status
        L.welvet_hip_swiglu_release.argtypes = [_vp]
        L.welvet_hip_swiglu_release.restype = None
        L.welvet_hip_volume_train_step_grad.argtypes = [_vp, _f, _i32, _f, _i32, C.c_double, _d,
                                                        _f, _f]
        L.welvet_hip_volume_train_step_grad.restype = Status
        L.welvet_dense_mount.argtypes = [_i32] * 5 + [_f, _d, C.c_size_t, C.POINTER(_vp)]
        L.welvet_dense_mount.restype = Status
        L.welvet_dense_execute.argtypes = [_vp, _f, _f, _f]
        L.welvet_dense_execute.restype = Status
        L.welvet_dense_release.argtypes = [_vp]
        L.welvet_dense_release.restype = None
        L.welvet_hip_dense_mount_device.argtypes = [_i32] * 5 + [_vp, _d, C.c_size_t,
                                                             C.POINTER(_vp)]
        L.welvet_hip_dense_mount_device.restype = Status
        L.welvet_hip_dense_mount_native.argtypes = [_i32] * 5 + [_u8, C.c_size_t, C.c_float, _d,
                                                             C.c_size_t, C.POINTER(_vp)]
        L.welvet_hip_dense_mount_native.restype = Status
        L.welvet_hip_dense_forward_device.argtypes = [_vp, _vp, _vp, _vp, _vp]
        L.welvet_hip_dense_forward_device.restype = Status
        L.welvet_hip_dense_forward_noalloc.argtypes = [_vp, _i32, _vp, _vp, _vp, _vp]
        L.welvet_hip_dense_forward_noalloc.restype = Status
        L.welvet_hip_dense_native.argtypes = [_vp, _u8, C.c_size_t, C.POINTER(C.c_size_t), _f]
        L.welvet_hip_dense_native.restype = Status
        L.welvet_hip_dense_repack.argtypes = [_vp, _f, C.c_size_t]
        L.welvet_hip_dense_repack.restype = Status
        L.welvet_hip_grid_repack.argtypes = [_vp] + [_i32] * 4 + [_f, C.c_size_t]
        L.welvet_hip_grid_repack.restype = Status
        L.welvet_hip_dense_export_f32.argtypes = [_vp, _f]
        L.welvet_hip_dense_export_f32.restype = Status
        L.welvet_hip_dense_backward.argtypes = [_vp, _f, _f, _f, _f, _f]
        L.welvet_hip_dense_backward.restype = Status
        L.welvet_hip_dense_sgd.argtypes = [_vp, _f, C.c_double]
        L.welvet_hip_dense_sgd.restype = Status
        L.welvet_hip_mse_f32.argtypes = [_f, _f, C.c_size_t, _d, _f]
        L.welvet_hip_mse_f32.restype = Status
        L.welvet_hip_set_forward_path.argtypes = [_i32]
        L.welvet_hip_set_forward_path.restype = None
        L.welvet_hip_set_tuning.argtypes = [_i32, _i32]
        L.welvet_hip_set_tuning.restype = _i32
        L.welvet_hip_probe_read.argtypes = [_vp, C.c_uint64, _vp, _vp]
        L.welvet_hip_probe_read.restype = Status
        coord = [_vp] + [_i32] * 4
        L.welvet_hip_grid_new.argtypes = [_i32] * 5 + [C.POINTER(_vp)]
        L.welvet_hip_grid_new.restype = Status
        L.welvet_hip_grid_release.argtypes = [_vp]
        L.welvet_hip_grid_release.restype = None
        L.welvet_hip_grid_bind_dense.argtypes = coord + [_i32] * 4 + [_f, _d, C.c_size_t]
        L.welvet_hip_grid_bind_dense.restype = Status
        L.welvet_hip_grid_set_remote_link.argtypes = coord + [_i32] * 4
        L.welvet_hip_grid_set_remote_link.restype = Status
        L.welvet_hip_grid_set_disabled.argtypes = coord + [_i32]
        L.welvet_hip_grid_set_disabled.restype = Status
        L.welvet_hip_volume_forward.argtypes = [_vp, _f, _i32, _f, _i32]
        L.welvet_hip_volume_forward.restype = Status
        L.welvet_hip_volume_forward_device.argtypes = [_vp, _vp, _i32, _vp, _i32, _vp]
        L.welvet_hip_volume_forward_device.restype = Status
        L.welvet_hip_volume_train_step.argtypes = [_vp, _f, _i32, _f, _i32, C.c_double, _d, _f]
        L.welvet_hip_volume_train_step.restype = Status
        L.welvet_hip_volume_train_step_device.argtypes = [_vp, _vp, _i32, _vp, _i32, C.c_double,
                                                          _d, _vp]
        L.welvet_hip_volume_train_step_device.restype = Status
        L.welvet_hip_grid_export_f32.argtypes = coord + [_f]
        L.welvet_hip_grid_export_f32.restype = Status
        L.welvet_hip_grid_native.argtypes = coord + [_u8, C.c_size_t, C.POINTER(C.c_size_t), _f]
        L.welvet_hip_grid_native.restype = Status
        _LIB = L
    return _LIB


def check(st: Status) -> None:
    if st.code:
        raise WelvetError(st.code, st.message.decode(errors="replace"))


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def version() -> str:
    return lib().welvet_version().decode()


def identity() -> str:
    return lib().welvet_runtime_identity().decode()


def available() -> bool:
    return bool(lib().welvet_metal_available())


def init() -> None:
    check(lib().welvet_metal_init())


def set_forward_path(path: int) -> None:
    lib().welvet_hip_set_forward_path(path)


# Route switches of welvet_hip_set_tuning (include/welvet_c.h).
TUNE = {"bf3": 10, "bf3_rows": 16, "fold_deriv": 17, "sgd_batch": 18, "dw_batch": 19,
        "gemv_batch": 20, "regx": 21}


def set_tuning(key: str, value: int) -> int:
    return lib().welvet_hip_set_tuning(TUNE[key], int(value))


def probe_read(d_bytes: int, nbytes: int, d_sink: int, stream: int = 0) -> None:
    """welvet_hip_probe_read: stream nbytes of device memory once (a floor
    measurement); raises on a non-zero status."""
    check(lib().welvet_hip_probe_read(C.c_void_p(d_bytes), C.c_uint64(nbytes), C.c_void_p(d_sink),
                                      C.c_void_p(stream)))


def forward(W, x, act=-1, dtype=1, bias=None, status=False):
    """welvet_dense_forward_f32: W [out][in] f32, x [batch][in] -> (pre, post)."""
    W = _f32(W)
    x = _f32(x)
    out, inn = W.shape
    batch = x.shape[0]
    b = None if bias is None else np.ascontiguousarray(bias, np.float64)
    pre = np.zeros((batch, out), np.float32)
    post = np.zeros((batch, out), np.float32)
    st = lib().welvet_dense_forward_f32(batch, inn, out, act, dtype, 0, _fp(W), _dp(b),
                                        0 if b is None else b.size, _fp(x), _fp(pre), _fp(post))
    if status:
        return st, pre, post
    check(st)
    return pre, post


def normalbp(W, x, grad_or_target, use_target, lr, act=-1, dtype=1, bias=None, status=False):
    """welvet_dense_normalbp_f32 -> dict(pre, post, dX, dW, W_after, loss)."""
    W = _f32(W)
    x = _f32(x)
    g = _f32(grad_or_target)
    out, inn = W.shape
    batch = x.shape[0]
    b = None if bias is None else np.ascontiguousarray(bias, np.float64)
    r = dict(pre=np.zeros((batch, out), np.float32), post=np.zeros((batch, out), np.float32),
             dX=np.zeros((batch, inn), np.float32), dW=np.zeros((out, inn), np.float32),
             W_after=np.zeros((out, inn), np.float32))
    loss = C.c_double()
    st = lib().welvet_dense_normalbp_f32(batch, inn, out, act, dtype, 0, _fp(W), _dp(b),
                                         0 if b is None else b.size, _fp(x), _fp(g),
                                         int(use_target), lr, _fp(r["pre"]), _fp(r["post"]),
                                         _fp(r["dX"]), _fp(r["dW"]), _fp(r["W_after"]),
                                         C.byref(loss))
    r["loss"] = loss.value
    if status:
        r["status"] = st
        return r
    check(st)
    return r


def swiglu_forward(Gate, Up, Down, x, dtype=1, seq=1, status=False):
    """welvet_swiglu_forward_f32; x [batch*seq][in] -> (pre = h, post)."""
    Gate, Up, Down, x = _f32(Gate), _f32(Up), _f32(Down), _f32(x)
    inter, inn = Gate.shape
    rows = x.shape[0]
    pre = np.zeros((rows, inter), np.float32)
    post = np.zeros((rows, inn), np.float32)
    st = lib().welvet_swiglu_forward_f32(rows // seq, seq, inn, inter, dtype, 0, _fp(Gate), _fp(Up),
                                         _fp(Down), _fp(x), _fp(pre), _fp(post))
    if status:
        return st, pre, post
    check(st)
    return pre, post


def swiglu_normalbp(Gate, Up, Down, x, grad_or_target, use_target, lr, dtype=1, seq=1,
                    status=False):
    """welvet_swiglu_normalbp_f32 -> dict(pre, post, dX, dW, W_after, loss)."""
    Gate, Up, Down, x, g = _f32(Gate), _f32(Up), _f32(Down), _f32(x), _f32(grad_or_target)
    inter, inn = Gate.shape
    rows = x.shape[0]
    nw = 3 * inter * inn
    r = dict(pre=np.zeros((rows, inter), np.float32), post=np.zeros((rows, inn), np.float32),
             dX=np.zeros((rows, inn), np.float32), dW=np.zeros(nw, np.float32),
             W_after=np.zeros(nw, np.float32))
    loss = C.c_double()
    st = lib().welvet_swiglu_normalbp_f32(rows // seq, seq, inn, inter, dtype, 0, _fp(Gate), _fp(Up),
                                          _fp(Down), _fp(x), _fp(g), int(use_target), lr,
                                          _fp(r["pre"]), _fp(r["post"]), _fp(r["dX"]), _fp(r["dW"]),
                                          _fp(r["W_after"]), C.byref(loss))
    r["loss"] = loss.value
    if status:
        r["status"] = st
        return r
    check(st)
    return r


def chain_forward(kind, packed, x, child_act=-1, dtype=1, seq=1, status=False):
    """welvet_{kind}_forward_f32, kind "sequential" or "residual"; packed
    [depth][dim][dim], x [batch*seq][dim] -> (pre, post)."""
    packed, x = _f32(packed), _f32(x)
    depth, dim = packed.shape[0], packed.shape[1]
    pre = np.zeros(x.shape, np.float32)
    post = np.zeros(x.shape, np.float32)
    st = getattr(lib(), f"welvet_{kind}_forward_f32")(x.shape[0] // seq, seq, dim, depth, child_act,
                                                       dtype, 0, _fp(packed), _fp(x), _fp(pre),
                                                       _fp(post))
    if status:
        return st, pre, post
    check(st)
    return pre, post


def chain_normalbp(kind, packed, x, grad_or_target, use_target, lr, child_act=-1, dtype=1, seq=1,
                   status=False):
    """welvet_{kind}_normalbp_f32 -> dict(pre, post, dX, dW, W_after, loss)."""
    packed, x, g = _f32(packed), _f32(x), _f32(grad_or_target)
    depth, dim = packed.shape[0], packed.shape[1]
    r = dict(pre=np.zeros(x.shape, np.float32), post=np.zeros(x.shape, np.float32),
             dX=np.zeros(x.shape, np.float32), dW=np.zeros(packed.size, np.float32),
             W_after=np.zeros(packed.size, np.float32))
    loss = C.c_double()
    st = getattr(lib(), f"welvet_{kind}_normalbp_f32")(
        x.shape[0] // seq, seq, dim, depth, child_act, dtype, 0, _fp(packed), _fp(x), _fp(g),
        int(use_target), lr, _fp(r["pre"]), _fp(r["post"]), _fp(r["dX"]), _fp(r["dW"]),
        _fp(r["W_after"]), C.byref(loss))
    r["loss"] = loss.value
    if status:
        r["status"] = st
        return r
    check(st)
    return r


class SwigluSession:
    """welvet_hip_swiglu_mount / _forward_device / _release."""

    def __init__(self, Gate, Up, Down, rows, dtype=1):
        Gate, Up, Down = _f32(Gate), _f32(Up), _f32(Down)
        self.inter, self.inn = Gate.shape
        self.rows = rows
        self.h = C.c_void_p()
        check(lib().welvet_hip_swiglu_mount(rows, self.inn, self.inter, dtype, _fp(Gate), _fp(Up),
                                            _fp(Down), C.byref(self.h)))

    def forward_device(self, d_x, d_pre, d_post, stream=None):
        """Device pointers (ints); enqueued on `stream` (a hipStream_t int)."""
        return lib().welvet_hip_swiglu_forward_device(self.h, d_x, d_pre, d_post, stream)

    def close(self):
        if self.h:
            lib().welvet_hip_swiglu_release(self.h)
            self.h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class Model:
    """welvet_model_* session (ABI 1): mount a WMN1 descriptor; calls take and
    return the ABI's byte messages."""

    def __init__(self, descriptor: bytes, status=False):
        self.h = C.c_void_p()
        buf = (C.c_uint8 * max(1, len(descriptor))).from_buffer_copy(descriptor or b"\0")
        self.status = lib().welvet_model_mount(buf, len(descriptor), C.byref(self.h))
        if not status:
            check(self.status)

    @staticmethod
    def _buf(b: bytes):
        return (C.c_uint8 * max(1, len(b))).from_buffer_copy(b or b"\0")

    def _blob_call(self, fn, *args):
        blob = Blob()
        st = fn(self.h, *args, C.byref(blob))
        data = bytes(C.string_at(blob.data, blob.size)) if st.code == 0 and blob.size else b""
        lib().welvet_metal_blob_free(C.byref(blob))
        return st, data

    def call(self, name: str, payload: bytes):
        """forward / forward_pair / backward -> (status, reply bytes)."""
        return self._blob_call(getattr(lib(), f"welvet_model_{name}"), self._buf(payload),
                               len(payload))

    def train_mse(self, mode: int, lr: float, payload: bytes, ticks: int = 1):
        loss = C.c_double()
        st = lib().welvet_model_train_mse(self.h, mode, lr, ticks, self._buf(payload), len(payload),
                                          C.byref(loss))
        return st, loss.value

    def apply_sgd(self, lr: float, payload: bytes):
        return lib().welvet_model_apply_sgd(self.h, lr, self._buf(payload), len(payload))

    def export(self):
        return self._blob_call(lib().welvet_model_export_weights)

    def sync(self, event: int):
        return lib().welvet_model_sync(self.h, event)

    def close(self):
        if self.h:
            lib().welvet_model_release(self.h)
            self.h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class Session:
    """welvet_dense_mount / execute / release plus the welvet_hip_ extensions."""

    def __init__(self, W, batch, act=-1, dtype=1, bias=None, native=None):
        """W: f32 [out][in] encoded into dtype, or, with native=(bytes, scale),
        the shape (out, in) of a store taken byte for byte from a snapshot in
        the reference layout (welvet_hip_dense_mount_native)."""
        self.h = None
        if native is None:
            W = _f32(W)
            self.out, self.inn = W.shape
        else:
            self.out, self.inn = W
        self.batch = batch
        self.dtype = dtype
        b = None if bias is None else np.ascontiguousarray(bias, np.float64)
        h = _vp()
        if native is None:
            check(lib().welvet_dense_mount(batch, self.inn, self.out, act, dtype, _fp(W), _dp(b),
                                           0 if b is None else b.size, C.byref(h)))
        else:
            raw = np.ascontiguousarray(native[0], np.uint8)
            check(lib().welvet_hip_dense_mount_native(
                batch, self.inn, self.out, act, dtype, raw.ctypes.data_as(_u8), raw.size,
                float(native[1]), _dp(b), 0 if b is None else b.size, C.byref(h)))
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            lib().welvet_dense_release(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def execute(self, x):
        x = _f32(x)
        pre = np.zeros((self.batch, self.out), np.float32)
        post = np.zeros((self.batch, self.out), np.float32)
        check(lib().welvet_dense_execute(self.h, _fp(x), _fp(pre), _fp(post)))
        return pre, post

    def forward_device(self, d_x: int, d_pre: int, d_post: int, stream: int | None = None):
        check(lib().welvet_hip_dense_forward_device(self.h, d_x, d_pre, d_post, stream))

    def forward_noalloc(self, batch: int, d_x: int, d_pre: int, d_post: int,
                        stream: int | None = None, status: bool = False):
        st = lib().welvet_hip_dense_forward_noalloc(self.h, batch, d_x, d_pre, d_post, stream)
        if status:
            return st
        check(st)

    def native(self):
        n = C.c_size_t()
        s = C.c_float()
        lib().welvet_hip_dense_native(self.h, None, 0, C.byref(n), C.byref(s))
        out = np.zeros(n.value, np.uint8)
        check(lib().welvet_hip_dense_native(self.h, out.ctypes.data_as(_u8), out.size, C.byref(n),
                                            C.byref(s)))
        return out, s.value

    def export_f32(self):
        out = np.zeros((self.out, self.inn), np.float32)
        check(lib().welvet_hip_dense_export_f32(self.h, _fp(out)))
        return out

    def repack(self, values, status=False):
        """WeightStore::set_from_f32_gpu: re-encode with fresh statistics."""
        v = _f32(values).ravel()
        st = lib().welvet_hip_dense_repack(self.h, _fp(v), v.size)
        if status:
            return st
        check(st)

    def backward(self, x, pre, gy):
        x, pre, gy = _f32(x), _f32(pre), _f32(gy)
        dX = np.zeros((self.batch, self.inn), np.float32)
        dW = np.zeros((self.out, self.inn), np.float32)
        check(lib().welvet_hip_dense_backward(self.h, _fp(x), _fp(pre), _fp(gy), _fp(dX), _fp(dW)))
        return dX, dW

    def sgd(self, dW, lr, status=False):
        st = lib().welvet_hip_dense_sgd(self.h, _fp(_f32(dW)), lr)
        if status:
            return st
        check(st)


def mse(pred, target):
    p, t = _f32(pred).ravel(), _f32(target).ravel()
    loss = C.c_double()
    g = np.zeros(p.size, np.float32)
    check(lib().welvet_hip_mse_f32(_fp(p), _fp(t), p.size, C.byref(loss), _fp(g)))
    return loss.value, g


class Grid:
    """The volume runtime: architecture::Grid with Dense cells, volume forward
    and training::step_dense (welvet_hip_grid_* / welvet_hip_volume_*)."""

    def __init__(self, depth, rows, cols, layers, batch):
        h = _vp()
        check(lib().welvet_hip_grid_new(depth, rows, cols, layers, batch, C.byref(h)))
        self.h = h
        self.batch = batch
        self.widths = {}

    def close(self):
        if self.h:
            lib().welvet_hip_grid_release(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def bind_dense(self, coord, W, act=-1, dtype=1, bias=None, status=False):
        W = _f32(W)
        out, inn = W.shape
        b = None if bias is None else np.ascontiguousarray(bias, np.float64)
        st = lib().welvet_hip_grid_bind_dense(self.h, *coord, inn, out, act, dtype, _fp(W), _dp(b),
                                              0 if b is None else b.size)
        if status:
            return st
        check(st)
        self.widths[tuple(coord)] = (inn, out)

    def set_remote_link(self, coord, target, status=False):
        st = lib().welvet_hip_grid_set_remote_link(self.h, *coord, *target)
        if status:
            return st
        check(st)

    def set_disabled(self, coord, disabled=True):
        check(lib().welvet_hip_grid_set_disabled(self.h, *coord, int(disabled)))

    def forward(self, x, out, status=False):
        x = _f32(x)
        y = np.zeros((self.batch, out), np.float32)
        st = lib().welvet_hip_volume_forward(self.h, _fp(x), x.shape[-1], _fp(y), out)
        if status:
            return st, y
        check(st)
        return y

    def train_step(self, x, target, lr, status=False):
        x, t = _f32(x), _f32(target)
        y = np.zeros(t.shape, np.float32)
        loss = C.c_double()
        st = lib().welvet_hip_volume_train_step(self.h, _fp(x), x.shape[-1], _fp(t), t.shape[-1],
                                                lr, C.byref(loss), _fp(y))
        if status:
            return st, loss.value, y
        check(st)
        return loss.value, y

    def export_f32(self, coord):
        inn, out = self.widths[tuple(coord)]
        W = np.zeros((out, inn), np.float32)
        check(lib().welvet_hip_grid_export_f32(self.h, *coord, _fp(W)))
        return W

    def repack(self, coord, values, status=False):
        v = _f32(values).ravel()
        st = lib().welvet_hip_grid_repack(self.h, *coord, _fp(v), v.size)
        if status:
            return st
        check(st)

    def native(self, coord):
        n = C.c_size_t()
        s = C.c_float()
        lib().welvet_hip_grid_native(self.h, *coord, None, 0, C.byref(n), C.byref(s))
        out = np.zeros(n.value, np.uint8)
        check(lib().welvet_hip_grid_native(self.h, *coord, out.ctypes.data_as(_u8), out.size,
                                           C.byref(n), C.byref(s)))
        return out, s.value
