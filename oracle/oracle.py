"""ctypes view of the oracle (oracle/liboracle.so) and of the reference build
(oracle/_ref/libwelvet_ref.so).

TEST INFRASTRUCTURE ONLY.  Imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, always as the checker; the product library never
loads this module or the libraries behind it.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# WELVET_ORACLE_SO: another build of the same sources (the sanitizer build)
ORACLE_SO = os.environ.get("WELVET_ORACLE_SO") or os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libwelvet_ref.so")

# include/welvet/dtype.hpp:9-44 and src/core/dtype.cpp:5-43
DTYPE_NAMES = [
    "float64", "float32", "float16", "bfloat16", "fp8e4m3", "fp8e5m2", "int64", "int32",
    "int16", "int8", "uint64", "uint32", "uint16", "uint8", "int4", "uint4", "fp4", "int2",
    "uint2", "ternary", "binary", "int", "uint", "uintptr", "complex64", "complex128", "nf4",
    "fp6", "int6", "uint6", "int5", "uint5", "int3", "uint3",
]
DTYPE = {name: i for i, name in enumerate(DTYPE_NAMES)}
ACT = {"linear": -1, "relu": 0, "silu": 1, "gelu": 2, "tanh": 3, "sigmoid": 4, "leakyrelu": 5,
       "relu2": 6}

_f = C.c_float
_d = C.c_double
_vp = C.c_void_p
_i = C.c_int
_i64 = C.c_int64


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


class Oracle:
    """The CPU restatement (plain C, -O2 -ffp-contract=off)."""

    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = self.lib = C.CDLL(path)
        for nm, enc, dec, ct in (("f16", "or_f32_to_f16", "or_f16_to_f32", C.c_uint16),
                                 ("bf16", "or_f32_to_bf16", "or_bf16_to_f32", C.c_uint16),
                                 ("e4m3", "or_f32_to_e4m3", "or_e4m3_to_f32", C.c_uint8),
                                 ("e5m2", "or_f32_to_e5m2", "or_e5m2_to_f32", C.c_uint8),
                                 ("fp4", "or_f32_to_fp4", "or_fp4_to_f32", C.c_uint8)):
            getattr(L, enc).argtypes = [_f]
            getattr(L, enc).restype = ct
            getattr(L, dec).argtypes = [ct]
            getattr(L, dec).restype = _f
        L.or_native_bytes.argtypes = [_i, _i64]
        L.or_native_bytes.restype = _i64
        L.or_pack.argtypes = [_i, _vp, _i64, _vp, C.POINTER(_f)]
        L.or_pack.restype = _i
        L.or_decode.argtypes = [_i, _vp, _i64, _f, _i64, _vp]
        L.or_decode.restype = _i
        L.or_decode_f64.argtypes = [_i, _vp, _i64, _f, _i64, _vp]
        L.or_decode_f64.restype = _i
        L.or_set.argtypes = [_i, _vp, _i64, _f, _i64, _i64, _f]
        L.or_set.restype = _i
        L.or_native_sgd.argtypes = [_i, _vp, _i64, _f, _i64, _vp, _d]
        L.or_native_sgd.restype = _i
        L.or_sgd_f32.argtypes = [_vp, _vp, _i64, _d]
        L.or_sgd_f32.restype = None
        L.or_mse.argtypes = [_vp, _vp, _i64]
        L.or_mse.restype = _d
        L.or_mse_grad.argtypes = [_vp, _vp, _i64, _vp]
        L.or_mse_grad.restype = None
        L.or_act.argtypes = [_f, _i]
        L.or_act.restype = _f
        L.or_act_prime.argtypes = [_f, _i]
        L.or_act_prime.restype = _f
        L.or_dense_forward.argtypes = [_i, _i, _i, _i, _vp, _vp, _i64, _vp, _vp, _vp]
        L.or_dense_forward.restype = None
        L.or_dense_backward.argtypes = [_i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp]
        L.or_dense_backward.restype = None
        L.or_normalbp.argtypes = [_i, _i, _i, _i, _i, _vp, _vp, _i64, _vp, _vp, _i, _d,
                                  _vp, _vp, _vp, _vp, _vp, _vp]
        L.or_normalbp.restype = _i
        L.or_dense_forward_native.argtypes = [_i, _i, _i, _i, _i, _vp, _i64, _f, _vp, _i64, _vp,
                                              _vp, _vp, _i]
        L.or_dense_forward_native.restype = None
        L.or_encode_many.argtypes = [_i, _vp, _i64, _vp]
        L.or_encode_many.restype = None
        L.or_decode_many.argtypes = [_i, _vp, _i64, _vp]
        L.or_decode_many.restype = None
        L.or_repack.argtypes = [_i, _vp, _i64, _vp, _i64, C.POINTER(_f)]
        L.or_repack.restype = _i
        L.or_swiglu_h.argtypes = [_vp, _vp, _i64, _vp]
        L.or_swiglu_h.restype = None
        L.or_swiglu_split.argtypes = [_vp, _vp, _vp, _i64, _vp, _vp]
        L.or_swiglu_split.restype = None

    # -- codecs ---------------------------------------------------------------
    def native_bytes(self, dtype: int, n: int) -> int:
        return int(self.lib.or_native_bytes(dtype, n))

    def pack(self, dtype: int, w: np.ndarray) -> tuple[np.ndarray, float]:
        w = np.ascontiguousarray(w, dtype=np.float32).ravel()
        out = np.zeros(self.native_bytes(dtype, w.size), np.uint8)
        s = _f()
        st = self.lib.or_pack(dtype, _ptr(w), w.size, _ptr(out), C.byref(s))
        if st:
            raise ValueError(f"or_pack status {st}")
        return out, s.value

    def decode(self, dtype: int, raw: np.ndarray, scale: float, n: int) -> np.ndarray:
        raw = np.ascontiguousarray(raw, dtype=np.uint8)
        out = np.zeros(n, np.float32)
        st = self.lib.or_decode(dtype, _ptr(raw), raw.size, scale, n, _ptr(out))
        if st:
            raise ValueError(f"or_decode status {st}")
        return out

    def decode_f64(self, dtype: int, raw: np.ndarray, scale: float, n: int) -> np.ndarray:
        raw = np.ascontiguousarray(raw, dtype=np.uint8)
        out = np.zeros(n, np.float64)
        st = self.lib.or_decode_f64(dtype, _ptr(raw), raw.size, scale, n, _ptr(out))
        if st:
            raise ValueError(f"or_decode_f64 status {st}")
        return out

    def set(self, dtype: int, raw: np.ndarray, scale: float, i: int, n: int, v: float) -> int:
        return int(self.lib.or_set(dtype, _ptr(raw), raw.size, scale, i, n, v))

    def native_sgd(self, dtype: int, raw: np.ndarray, scale: float, n: int, dW: np.ndarray,
                   lr: float) -> int:
        dW = np.ascontiguousarray(dW, dtype=np.float32).ravel()
        return int(self.lib.or_native_sgd(dtype, _ptr(raw), raw.size, scale, n, _ptr(dW), lr))

    def sgd_f32(self, w: np.ndarray, dW: np.ndarray, lr: float) -> None:
        dW = np.ascontiguousarray(dW, dtype=np.float32)
        self.lib.or_sgd_f32(_ptr(w), _ptr(dW), w.size, lr)

    def encode_many(self, kind: int, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros(x.size, np.uint16 if kind in (0, 1) else np.uint8)
        self.lib.or_encode_many(kind, _ptr(x), x.size, _ptr(out))
        return out

    def repack(self, dtype: int, w: np.ndarray) -> tuple[np.ndarray, float]:
        """op_native_repack: fresh statistics and scale, every element re-encoded."""
        w = np.ascontiguousarray(w, dtype=np.float32).ravel()
        out = np.zeros(self.native_bytes(dtype, w.size), np.uint8)
        s = _f()
        st = self.lib.or_repack(dtype, _ptr(w), w.size, _ptr(out), out.size, C.byref(s))
        if st:
            raise ValueError(f"or_repack status {st}")
        return out, s.value

    def decode_many(self, kind: int, codes) -> np.ndarray:
        """Scalar-codec decode of every code (kind 0 f16, 1 bf16, 2 e4m3,
        3 e5m2, 4 fp4), written to memory: signaling-NaN payloads survive."""
        c = np.ascontiguousarray(codes, np.uint32)
        out = np.zeros(c.size, np.float32)
        self.lib.or_decode_many(kind, _ptr(c), c.size, _ptr(out))
        return out

    # -- dense ----------------------------------------------------------------
    def act(self, v: float, act: int) -> float:
        return self.lib.or_act(v, act)

    def act_prime(self, v: float, act: int) -> float:
        return self.lib.or_act_prime(v, act)

    def mse(self, p: np.ndarray, t: np.ndarray) -> float:
        p = np.ascontiguousarray(p, np.float32)
        t = np.ascontiguousarray(t, np.float32)
        return float(self.lib.or_mse(_ptr(p), _ptr(t), p.size))

    def mse_grad(self, p: np.ndarray, t: np.ndarray) -> np.ndarray:
        p = np.ascontiguousarray(p, np.float32)
        t = np.ascontiguousarray(t, np.float32)
        g = np.zeros(p.size, np.float32)
        self.lib.or_mse_grad(_ptr(p), _ptr(t), p.size, _ptr(g))
        return g.reshape(p.shape)

    def forward(self, Wd: np.ndarray, x: np.ndarray, act: int, bias: np.ndarray | None = None):
        out, inn = Wd.shape
        batch = x.shape[0]
        Wd = np.ascontiguousarray(Wd, np.float64)
        x = np.ascontiguousarray(x, np.float32)
        pre = np.zeros((batch, out), np.float32)
        post = np.zeros((batch, out), np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float64)
        self.lib.or_dense_forward(batch, inn, out, act, _ptr(Wd), _ptr(b),
                                  0 if b is None else b.size, _ptr(x), _ptr(pre), _ptr(post))
        return pre, post

    def backward(self, Wd: np.ndarray, x: np.ndarray, pre: np.ndarray, gy: np.ndarray, act: int):
        out, inn = Wd.shape
        batch = x.shape[0]
        Wd = np.ascontiguousarray(Wd, np.float64)
        x = np.ascontiguousarray(x, np.float32)
        pre = np.ascontiguousarray(pre, np.float32)
        gy = np.ascontiguousarray(gy, np.float32)
        dpre = np.zeros((batch, out), np.float32)
        dX = np.zeros((batch, inn), np.float32)
        dW = np.zeros((out, inn), np.float32)
        self.lib.or_dense_backward(batch, inn, out, act, _ptr(Wd), _ptr(x), _ptr(pre), _ptr(gy),
                                   _ptr(dpre), _ptr(dX), _ptr(dW))
        return dpre, dX, dW

    def normalbp(self, batch, inn, out, act, dtype, W_init, x, grad_or_target, use_target, lr,
                 bias=None):
        W_init = np.ascontiguousarray(W_init, np.float32)
        x = np.ascontiguousarray(x, np.float32)
        g = np.ascontiguousarray(grad_or_target, np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float64)
        r = dict(pre=np.zeros((batch, out), np.float32), post=np.zeros((batch, out), np.float32),
                 dX=np.zeros((batch, inn), np.float32), dW=np.zeros((out, inn), np.float32),
                 W_after=np.zeros((out, inn), np.float32))
        loss = _d()
        st = self.lib.or_normalbp(batch, inn, out, act, dtype, _ptr(W_init), _ptr(b),
                                  0 if b is None else b.size, _ptr(x), _ptr(g), int(use_target),
                                  lr, _ptr(r["pre"]), _ptr(r["post"]), _ptr(r["dX"]),
                                  _ptr(r["dW"]), _ptr(r["W_after"]), C.byref(loss))
        r["loss"] = loss.value
        r["status"] = st
        return r

    # -- SwiGLU over Dense (src/layers/swiglu/swiglu.cpp) -------------------
    def swiglu_h(self, gate, up):
        gate = np.ascontiguousarray(gate, np.float32)
        up = np.ascontiguousarray(up, np.float32)
        h = np.zeros_like(gate)
        self.lib.or_swiglu_h(_ptr(gate), _ptr(up), gate.size, _ptr(h))
        return h

    def swiglu_split(self, gate, up, gh):
        gate, up, gh = (np.ascontiguousarray(a, np.float32) for a in (gate, up, gh))
        d_up, d_gate = np.zeros_like(gate), np.zeros_like(gate)
        self.lib.or_swiglu_split(_ptr(gate), _ptr(up), _ptr(gh), gate.size, _ptr(d_up),
                                 _ptr(d_gate))
        return d_up, d_gate

    def swiglu_normalbp(self, dtype, Gate, Up, Down, x, grad_or_target=None, use_target=0,
                        lr=0.0):
        """welvet_swiglu_forward_f32 / welvet_swiglu_normalbp_f32
        (c_abi.cpp:326-432) over swiglu.cpp:70-275: Gate/Up/Down Dense
        layers (Linear, no bias) packed into `dtype`, forward h = silu(gate) *
        up, post = Down h; backward through Down, op_swiglu, Gate and Up;
        SGD Gate, Up, Down (the first error stops).  x is [rows][in] with
        rows = batch * seq.  grad_or_target None = forward only.
        -> dict(status, pre, post[, dX, dW, W_after, loss])."""
        inter, inn = Gate.shape
        x = np.ascontiguousarray(x, np.float32)
        parts = []
        for W in (Gate, Up, Down):
            W = np.ascontiguousarray(W, np.float32)
            raw, scale = self.pack(dtype, W)
            parts.append([raw, scale, W.shape])
        Wd = [self.decode_f64(dtype, r, sc, sh[0] * sh[1]).reshape(sh) for r, sc, sh in parts]
        g_pre, _ = self.forward(Wd[0], x, -1)
        u_pre, u_post = self.forward(Wd[1], x, -1)
        h = self.swiglu_h(g_pre, u_post)
        d_pre, post = self.forward(Wd[2], h, -1)
        res = dict(status=0, pre=h, post=post)
        if grad_or_target is None:
            return res
        t = np.ascontiguousarray(grad_or_target, np.float32).reshape(post.shape)
        loss, gy = 0.0, t
        if use_target:
            loss, gy = self.mse(post, t), self.mse_grad(post, t)
        _, grad_h, dW_d = self.backward(Wd[2], h, d_pre, gy, -1)
        d_up, d_gate = self.swiglu_split(g_pre, u_post, grad_h)
        _, gx_g, dW_g = self.backward(Wd[0], x, g_pre, d_gate, -1)
        _, gx_u, dW_u = self.backward(Wd[1], x, u_pre, d_up, -1)
        res.update(dX=gx_g + gx_u, dW=np.concatenate([dW_g.ravel(), dW_u.ravel(), dW_d.ravel()]),
                   loss=loss)
        if lr != 0.0:
            for (raw, scale, sh), dW in zip(parts, (dW_g, dW_u, dW_d)):
                n = sh[0] * sh[1]
                if dtype == 1:
                    if not np.all(np.isfinite(dW)):
                        res["status"] = 2
                        return res
                    if abs(lr) > np.finfo(np.float32).max or abs(lr) < np.finfo(np.float32).tiny:
                        res["status"] = 2
                        return res
                    self.sgd_f32(raw.view(np.float32), dW.ravel(), lr)
                elif self.native_sgd(dtype, raw, scale, n, dW, lr):
                    res["status"] = 1
                    return res
        res["W_after"] = np.concatenate([self.decode(dtype, r, sc, sh[0] * sh[1])
                                         for r, sc, sh in parts])
        return res

    # -- Sequential / Residual chains of Dense (src/layers/{sequential,residual}) --
    def chain_normalbp(self, residual, dtype, packed, x, child_act, grad_or_target=None,
                       use_target=0, lr=0.0):
        """welvet_{sequential,residual}_{forward,normalbp}_f32 (c_abi.cpp:918-1090)
        over sequential.cpp:117-245 / residual.cpp:117-275: packed
        [depth][dim][dim] Dense children (child_act, no bias) chained on x
        [rows][dim]; Residual adds fl32(F(x) + x) on the way out and the
        skip gradient on the way back; SGD children in order (the first error
        stops).  -> dict(status, pre, post[, dX, dW, W_after, loss])."""
        packed = np.ascontiguousarray(packed, np.float32)
        depth, dim = packed.shape[0], packed.shape[1]
        x = np.ascontiguousarray(x, np.float32)
        parts, Wd = [], []
        for i in range(depth):
            raw, scale = self.pack(dtype, packed[i])
            parts.append((raw, scale))
            Wd.append(self.decode_f64(dtype, raw, scale, dim * dim).reshape(dim, dim))
        ins, pres, cur = [], [], x
        for i in range(depth):
            ins.append(cur)
            p, cur = self.forward(Wd[i], cur, child_act)
            pres.append(p)
        post = (cur + x).astype(np.float32) if residual else cur
        res = dict(status=0, pre=pres[-1], post=post)
        if grad_or_target is None:
            return res
        t = np.ascontiguousarray(grad_or_target, np.float32).reshape(post.shape)
        loss, gy = 0.0, t
        if use_target:
            loss, gy = self.mse(post, t), self.mse_grad(post, t)
        g, dWs = gy, [None] * depth
        for i in range(depth - 1, -1, -1):
            _, g, dWs[i] = self.backward(Wd[i], ins[i], pres[i], g, child_act)
        res.update(dX=(g + gy).astype(np.float32) if residual else g,
                   dW=np.concatenate([d.ravel() for d in dWs]), loss=loss)
        if lr != 0.0:
            for (raw, scale), dW in zip(parts, dWs):
                if dtype == 1:
                    if not np.all(np.isfinite(dW)) or abs(lr) > np.finfo(np.float32).max or \
                            abs(lr) < np.finfo(np.float32).tiny:
                        res["status"] = 2
                        return res
                    self.sgd_f32(raw.view(np.float32), dW.ravel(), lr)
                elif self.native_sgd(dtype, raw, scale, dim * dim, dW, lr):
                    res["status"] = 1
                    return res
        res["W_after"] = np.concatenate([self.decode(dtype, r, sc, dim * dim) for r, sc in parts])
        return res

    def forward_native(self, dtype, raw, scale, x, out, inn, act, bias=None, threads=1):
        raw = np.ascontiguousarray(raw, np.uint8)
        x = np.ascontiguousarray(x, np.float32)
        batch = x.shape[0]
        pre = np.zeros((batch, out), np.float32)
        post = np.zeros((batch, out), np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float64)
        self.lib.or_dense_forward_native(batch, inn, out, act, dtype, _ptr(raw), raw.size, scale,
                                         _ptr(b), 0 if b is None else b.size, _ptr(x), _ptr(pre),
                                         _ptr(post), threads)
        return pre, post


class Reference:
    """The reference's own host codec compiled from its sources (oracle/_ref)."""

    def __init__(self, path: str = REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        L = self.lib = C.CDLL(path)
        L.ref_pack.argtypes = [_i, _vp, _i, _vp, C.c_long, C.POINTER(_f)]
        L.ref_pack.restype = C.c_long
        L.ref_decode.argtypes = [_i, _vp, C.c_long, _f, _i, _vp]
        L.ref_decode.restype = _i
        L.ref_decode_f64.argtypes = [_i, _vp, C.c_long, _f, _i, _vp]
        L.ref_decode_f64.restype = _i
        L.ref_encode_many.argtypes = [_i, _vp, C.c_long, _vp]
        L.ref_encode_many.restype = None
        L.ref_decode_many.argtypes = [_i, _vp, C.c_long, _vp]
        L.ref_decode_many.restype = None
        for nm, ct in (("f16", C.c_uint16), ("bf16", C.c_uint16), ("e4m3", C.c_uint8),
                       ("e5m2", C.c_uint8), ("fp4", C.c_uint8)):
            dec = getattr(L, f"ref_{nm}_to_f32")
            dec.argtypes = [ct]
            dec.restype = _f

    def pack(self, dtype: int, w: np.ndarray) -> tuple[np.ndarray, float]:
        w = np.ascontiguousarray(w, dtype=np.float32).ravel()
        cap = 16 * w.size + 16
        out = np.zeros(cap, np.uint8)
        s = _f()
        n = self.lib.ref_pack(dtype, _ptr(w), w.size, _ptr(out), cap, C.byref(s))
        if n < 0:
            raise ValueError(f"ref_pack status {-n}")
        return out[:n].copy(), s.value

    def decode(self, dtype: int, raw: np.ndarray, scale: float, n: int) -> np.ndarray:
        raw = np.ascontiguousarray(raw, np.uint8)
        out = np.zeros(n, np.float32)
        st = self.lib.ref_decode(dtype, _ptr(raw), raw.size, scale, n, _ptr(out))
        if st:
            raise ValueError(f"ref_decode status {st}")
        return out

    def decode_f64(self, dtype: int, raw: np.ndarray, scale: float, n: int) -> np.ndarray:
        raw = np.ascontiguousarray(raw, np.uint8)
        out = np.zeros(n, np.float64)
        st = self.lib.ref_decode_f64(dtype, _ptr(raw), raw.size, scale, n, _ptr(out))
        if st:
            raise ValueError(f"ref_decode_f64 status {st}")
        return out

    def encode_many(self, kind: int, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        out = np.zeros(x.size, np.uint16 if kind in (0, 1) else np.uint8)
        self.lib.ref_encode_many(kind, _ptr(x), x.size, _ptr(out))
        return out

    def decode_many(self, kind: int, codes) -> np.ndarray:
        c = np.ascontiguousarray(codes, np.uint32)
        out = np.zeros(c.size, np.float32)
        self.lib.ref_decode_many(kind, _ptr(c), c.size, _ptr(out))
        return out


def have_reference() -> bool:
    return os.path.exists(REF_SO)


class Stack:
    """CPU restatement of a Stack of Dense children (the model ABI's root 0).

    TEST INFRASTRUCTURE ONLY.  stack::forward / backward_f32 / apply_grad_sgd
    (src/layers/stack/stack.cpp:446-556) over Dense children in order, and
    cameral_train::train_stack_mse for the back-propagation family
    (src/runtime/cameral_train.cpp:348-403: forward, MSE, backward, SGD of
    every child in order even at lr 0).  Each child holds its packed store
    (raw, scale) like Volume's cells."""

    def __init__(self, oracle: Oracle):
        self.O = oracle
        self.children = []

    def add_dense(self, W, act=-1, dtype=1, bias=None):
        W = np.ascontiguousarray(W, np.float32)
        raw, scale = self.O.pack(dtype, W)
        self.children.append(dict(dtype=dtype, act=act, raw=raw, scale=scale, out=W.shape[0],
                                  inn=W.shape[1],
                                  bias=None if bias is None else np.asarray(bias, np.float64)))

    def _wd(self, c):
        return self.O.decode_f64(c["dtype"], c["raw"], c["scale"],
                                 c["out"] * c["inn"]).reshape(c["out"], c["inn"])

    def export_f32(self, i):
        c = self.children[i]
        return self.O.decode(c["dtype"], c["raw"], c["scale"], c["out"] * c["inn"]).reshape(
            c["out"], c["inn"])

    def forward(self, x):
        """-> (ins, pres, posts)."""
        cur = np.ascontiguousarray(x, np.float32)
        ins, pres, posts = [], [], []
        for c in self.children:
            ins.append(cur)
            p, cur = self.O.forward(self._wd(c), cur, c["act"], c["bias"])
            pres.append(p)
            posts.append(cur)
        return ins, pres, posts

    def backward(self, x, gy):
        """-> (gx, dW concatenated in child order)."""
        ins, pres, _ = self.forward(x)
        g = np.ascontiguousarray(gy, np.float32)
        dws = [None] * len(self.children)
        for i in range(len(self.children) - 1, -1, -1):
            c = self.children[i]
            _, g, dws[i] = self.O.backward(self._wd(c), ins[i], pres[i], g, c["act"])
        return g, np.concatenate([d.ravel() for d in dws])

    def apply_sgd(self, dw, lr):
        """-> status code (0, or the first failing child's)."""
        off = 0
        for c in self.children:
            n = c["out"] * c["inn"]
            g = np.ascontiguousarray(dw[off:off + n], np.float32)
            off += n
            if c["dtype"] == 1:
                if not np.all(np.isfinite(g)) or abs(lr) > np.finfo(np.float32).max or \
                        (lr != 0 and abs(lr) < np.finfo(np.float32).tiny):
                    return 2
                self.O.sgd_f32(c["raw"].view(np.float32), g, lr)
            elif self.O.native_sgd(c["dtype"], c["raw"], c["scale"], n, g, lr):
                return 1
        return 0

    def train_mse(self, x, t, lr, frozen=False):
        """-> (status, loss)."""
        _, _, posts = self.forward(x)
        loss = self.O.mse(posts[-1], t)
        if frozen:
            return 0, loss
        gx, dw = self.backward(x, self.O.mse_grad(posts[-1], t))
        return self.apply_sgd(dw, lr), loss


class Volume:
    """CPU restatement of the volume runtime over Dense cells.

    TEST INFRASTRUCTURE ONLY.  Sequencing follows the reference:
      hop order z, y, x, l                      src/architecture/grid.cpp:82-95
      runtime::forward::volume_dense            src/runtime/forward.cpp:74-132
        (disabled cells skipped, an enabled cell without an op, a remote hop
        without a recorded post, or a width mismatch is an error)
      runtime::backward::volume_dense           src/runtime/backward.cpp:88-127
        (tape in reverse; each step's input gradient feeds the step before it)
      runtime::training::sgd_dense, step_dense  src/runtime/training.cpp:61-184
        (LR 0 is an error; SGD per cell in forward order, the first failing
        cell stops the rest)
    and every arithmetic step is one of this oracle's pinned Dense functions.
    Results are (code, message, ...) like the C ABI's status.
    """

    def __init__(self, oracle: Oracle, depth: int, rows: int, cols: int, layers: int, batch: int):
        self.O = oracle
        self.dims = (max(1, depth), max(1, rows), max(1, cols), max(1, layers))
        self.batch = batch
        self.cells = {}
        self.remote = {}
        self.disabled = set()

    def bind_dense(self, coord, W, act=-1, dtype=1, bias=None):
        W = np.ascontiguousarray(W, np.float32)
        raw, scale = self.O.pack(dtype, W)
        self.cells[tuple(coord)] = dict(dtype=dtype, act=act, raw=raw, scale=scale,
                                        out=W.shape[0], inn=W.shape[1],
                                        bias=None if bias is None else np.asarray(bias, np.float64))

    def set_remote_link(self, coord, target):
        self.remote[tuple(coord)] = tuple(target)

    def set_disabled(self, coord, disabled=True):
        (self.disabled.add if disabled else self.disabled.discard)(tuple(coord))

    def weights(self, coord) -> np.ndarray:
        c = self.cells[tuple(coord)]
        return self.O.decode_f64(c["dtype"], c["raw"], c["scale"],
                                 c["out"] * c["inn"]).reshape(c["out"], c["inn"])

    def export_f32(self, coord) -> np.ndarray:
        c = self.cells[tuple(coord)]
        return self.O.decode(c["dtype"], c["raw"], c["scale"],
                             c["out"] * c["inn"]).reshape(c["out"], c["inn"])

    def hop_order(self):
        D, R, Cc, L = self.dims
        for z in range(D):
            for y in range(R):
                for x in range(Cc):
                    for l in range(L):
                        yield (z, y, x, l)

    def forward(self, x):
        """-> (code, message, y, tape); tape = [(coord, input, pre, post)]."""
        cur = np.ascontiguousarray(x, np.float32)
        posts, tape = {}, []
        for co in self.hop_order():
            if co in self.disabled:
                continue
            if co not in self.cells:
                return 1, "runtime.forward: no op at z=%d y=%d x=%d l=%d" % co, None, tape
            inp = cur
            if co in self.remote:
                t = self.remote[co]
                if t not in posts:
                    return 1, "runtime.forward: remote hop has no recorded activation", None, tape
                inp = posts[t]
            c = self.cells[co]
            if inp.shape[1] != c["inn"]:
                return 1, "dense: input width mismatch", None, tape
            pre, post = self.O.forward(self.weights(co), inp, c["act"], c["bias"])
            tape.append((co, inp, pre, post))
            posts[co] = post
            cur = post
        if not tape:
            return 1, "runtime.forward: grid has no enabled cells with ops", None, tape
        return 0, "", cur, tape

    def train_step(self, x, target, lr):
        """-> (code, message, loss, y).  After the backward, self.grad_in holds
        backward::Result::grad_in (backward.cpp:125): the input gradient of
        the first tape entry."""
        self.grad_in = None
        code, msg, y, tape = self.forward(x)
        if code:
            return code, msg, 0.0, None
        t = np.ascontiguousarray(target, np.float32)
        if t.shape != y.shape:
            return 1, "training: MSE shape", 0.0, y
        loss = self.O.mse(y, t)
        gy = self.O.mse_grad(y, t)
        grads = {}
        for co, inp, pre, _ in reversed(tape):
            c = self.cells[co]
            if gy.shape[1] != c["out"]:  # dense::backward_f32 shape check, dense.cpp:171-178
                return 1, "dense: bwd shape mismatch", loss, y
            _, dX, dW = self.O.backward(self.weights(co), inp, pre, gy, c["act"])
            grads[co] = dW
            gy = dX
        self.grad_in = gy
        if lr == 0.0:
            return 1, "training: LR is 0", loss, y
        if not np.isfinite(lr):
            return 1, "weights: bad SGD arguments", loss, y
        for co, _, _, _ in tape:
            c = self.cells[co]
            dW = grads[co]
            if c["dtype"] == 1:  # Float32 launcher checks, training.mm:71-128
                if not np.all(np.isfinite(dW)):
                    return 2, "SGD: gradient is not a finite f32", loss, y
                if abs(lr) > np.finfo(np.float32).max or abs(lr) < np.finfo(np.float32).tiny:
                    return 2, "SGD: learning rate outside the f32 range", loss, y
                w = c["raw"].view(np.float32)
                self.O.sgd_f32(w, dW.ravel(), lr)
            else:
                st = self.O.native_sgd(c["dtype"], c["raw"], c["scale"], c["out"] * c["inn"],
                                       dW, lr)
                if st:
                    return 1, "weights: nonfinite gradient", loss, y
        return 0, "", loss, y
