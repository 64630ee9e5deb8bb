"""Writers and readers of the Dense wire formats of the reference's
`welvet_dense_fwd` tool (little-endian, no padding), and a runner for this
build's tool of the same name.

  WVD1/2/3  batch, in, out, act [, dtype [, backend]] i32; W [out*in] f32;
            bias_len u32, bias f64; x [batch*in] f32
            -> WVO1 pre, post [batch*out] f32 (no counts)
            tools/dense_fwd/main.cpp:43-151
  WDB1      batch, in, out, act, dtype, backend i32; W; bias_len, bias; x;
            use_target i32; grad_or_target [batch*out] f32; lr f64
            -> WDBO (n i32, values) for pre, post, dX, dW, W_after; loss f64
            tools/dense_fwd/volume_fwd.cpp:1614-1757
  WVF1      depth, rows, cols, lpc, batch, backend, n_links i32; links
            n_links x 8 i32; per hop (z, y, x, l order) enabled i32 and, when
            enabled, in, out, act, dtype i32, W, bias_len, bias; x
            -> WVFO n i32, y            tools/dense_fwd/volume_fwd.cpp:100-207
  WVN1      WVF1's body, then target [batch*out_last] f32 and lr f64
            -> WVNO loss f64; n, grad_in; n_cells; per enabled cell out, in,
            W_after; n, y               tools/dense_fwd/volume_fwd.cpp:1759-1929
  WVS1      batch, seq, in, inter, dtype, backend i32; Gate, Up [inter*in],
            Down [in*inter] f32; x [batch*seq*in]
            -> WVSO (n, values) for pre (h), post   tools/dense_fwd/main.cpp:650-720
  WSB1      WVS1's fields, then use_target i32; grad_or_target [batch*seq*in];
            lr f64 -> WSBO as WDBO (dW, W_after = concat(Gate, Up, Down))
            tools/dense_fwd/volume_fwd.cpp:2539-2690
  WSQ1/WRE1 batch, seq, dim, depth, child_act, dtype, backend i32; packed
            [depth][dim][dim] f32; x [batch*seq*dim]
            -> WSQO / WREO (n, values) for pre, post   tools/dense_fwd/main.cpp:302-430
  SQB1/REB1 WSQ1's fields, then use_target i32; grad_or_target; lr f64
            -> SQBO / REBO as WDBO    tools/dense_fwd/volume_fwd.cpp:6187-6587
  --bench=N puts WVB2 (mount_ns i64, exec_ns i64, iters i32) before WVO1 and
  WVFO, WVB1 (ns i64, iters i32) before WDBO and WVNO.
"""
import os
import struct
import subprocess

import numpy as np

TOOL = os.path.join(os.path.dirname(os.path.abspath(__file__)), "welvet_dense_fwd")


def run(payload: bytes, *args, timeout=120):
    """-> (returncode, stdout bytes, stderr text)."""
    if not os.path.exists(TOOL):
        raise FileNotFoundError(f"{TOOL} is not built (python welvet.metal_amd/build.py)")
    r = subprocess.run([TOOL, *args], input=payload, capture_output=True, timeout=timeout)
    return r.returncode, r.stdout, r.stderr.decode(errors="replace")


def _i32(*v):
    return struct.pack("<%di" % len(v), *v)


def _f32(a):
    return np.ascontiguousarray(a, np.float32).tobytes()


def _bias(bias):
    if bias is None:
        return struct.pack("<I", 0)
    b = np.ascontiguousarray(bias, np.float64)
    return struct.pack("<I", b.size) + b.tobytes()


def wvd(W, x, act=-1, dtype=1, backend=0, bias=None, version=3):
    out, inn = W.shape
    head = {1: _i32(x.shape[0], inn, out, act),
            2: _i32(x.shape[0], inn, out, act, dtype),
            3: _i32(x.shape[0], inn, out, act, dtype, backend)}[version]
    return b"WVD%d" % version + head + _f32(W) + _bias(bias) + _f32(x)


def wdb(W, x, grad_or_target, use_target, lr, act=-1, dtype=1, bias=None, backend=0):
    out, inn = W.shape
    return (b"WDB1" + _i32(x.shape[0], inn, out, act, dtype, backend) + _f32(W) + _bias(bias) +
            _f32(x) + _i32(int(use_target)) + _f32(grad_or_target) + struct.pack("<d", lr))


def wvs(Gate, Up, Down, x, dtype=1, seq=1, backend=0):
    inter, inn = Gate.shape
    return (b"WVS1" + _i32(x.shape[0] // seq, seq, inn, inter, dtype, backend) + _f32(Gate) +
            _f32(Up) + _f32(Down) + _f32(x))


def wsb(Gate, Up, Down, x, grad_or_target, use_target, lr, dtype=1, seq=1, backend=0):
    inter, inn = Gate.shape
    return (b"WSB1" + _i32(x.shape[0] // seq, seq, inn, inter, dtype, backend) + _f32(Gate) +
            _f32(Up) + _f32(Down) + _f32(x) + _i32(int(use_target)) + _f32(grad_or_target) +
            struct.pack("<d", lr))


def chain(magic, packed, x, child_act=-1, dtype=1, seq=1, backend=0):
    """WSQ1 / WRE1 forward wires."""
    depth, dim = packed.shape[0], packed.shape[1]
    return (magic + _i32(x.shape[0] // seq, seq, dim, depth, child_act, dtype, backend) +
            _f32(packed) + _f32(x))


def chain_nbp(magic, packed, x, grad_or_target, use_target, lr, child_act=-1, dtype=1, seq=1,
              backend=0):
    """SQB1 / REB1 NormalBP wires."""
    return (chain(magic, packed, x, child_act, dtype, seq, backend) + _i32(int(use_target)) +
            _f32(grad_or_target) + struct.pack("<d", lr))


def hops(dims):
    D, R, C, L = (max(1, d) for d in dims)
    return [(z, y, x, l) for z in range(D) for y in range(R) for x in range(C) for l in range(L)]


def volume_body(dims, batch, cells, links=(), backend=0):
    """cells: {coord: (W, act, dtype, bias)}; hops without an entry go out
    with enabled = 0."""
    b = _i32(*dims, batch, backend, len(links))
    for (src, dst) in links:
        b += _i32(*src, *dst)
    for co in hops(dims):
        if co not in cells:
            b += _i32(0)
            continue
        W, act, dtype, bias = cells[co]
        out, inn = W.shape
        b += _i32(1, inn, out, act, dtype) + _f32(W) + _bias(bias)
    return b


def wvf(dims, batch, cells, x, links=()):
    return b"WVF1" + volume_body(dims, batch, cells, links) + _f32(x)


def wvn(dims, batch, cells, x, target, lr, links=()):
    return (b"WVN1" + volume_body(dims, batch, cells, links) + _f32(x) + _f32(target) +
            struct.pack("<d", lr))


class Reader:
    def __init__(self, data: bytes):
        self.d, self.p = data, 0

    def take(self, n):
        assert self.p + n <= len(self.d), ("short reply", self.p, n, len(self.d))
        v = self.d[self.p:self.p + n]
        self.p += n
        return v

    def magic(self):
        return self.take(4)

    def i32(self):
        return struct.unpack("<i", self.take(4))[0]

    def i64(self):
        return struct.unpack("<q", self.take(8))[0]

    def f64(self):
        return struct.unpack("<d", self.take(8))[0]

    def f32s(self, n):
        return np.frombuffer(self.take(4 * n), np.float32).copy()

    def counted(self):
        return self.f32s(self.i32())

    def done(self):
        return self.p == len(self.d)


def read_bench(r: Reader):
    """WVB2 -> dict(mount_ns, exec_ns, iters); WVB1 -> dict(ns, iters)."""
    m = r.magic()
    if m == b"WVB2":
        return dict(mount_ns=r.i64(), exec_ns=r.i64(), iters=r.i32())
    assert m == b"WVB1", m
    return dict(ns=r.i64(), iters=r.i32())


def read_wvo(r: Reader, batch, out):
    assert r.magic() == b"WVO1"
    pre = r.f32s(batch * out).reshape(batch, out)
    post = r.f32s(batch * out).reshape(batch, out)
    return pre, post


def read_wdbo(r: Reader):
    assert r.magic() == b"WDBO"
    res = {k: r.counted() for k in ("pre", "post", "dX", "dW", "W_after")}
    res["loss"] = r.f64()
    return res


def read_wvso(r: Reader):
    assert r.magic() == b"WVSO"
    return r.counted(), r.counted()


def read_pair(r: Reader, magic: bytes):
    """WVSO / WSQO / WREO: counted pre, counted post."""
    assert r.magic() == magic
    return r.counted(), r.counted()


def read_leaf(r: Reader, magic: bytes):
    """WDBO-framed NormalBP replies (WSBO, SQBO, REBO)."""
    assert r.magic() == magic
    res = {k: r.counted() for k in ("pre", "post", "dX", "dW", "W_after")}
    res["loss"] = r.f64()
    return res


def read_wsbo(r: Reader):
    assert r.magic() == b"WSBO"
    res = {k: r.counted() for k in ("pre", "post", "dX", "dW", "W_after")}
    res["loss"] = r.f64()
    return res


def read_wvfo(r: Reader):
    assert r.magic() == b"WVFO"
    return r.counted()


def read_wvno(r: Reader):
    assert r.magic() == b"WVNO"
    res = dict(loss=r.f64(), grad_in=r.counted())
    cells = []
    for _ in range(r.i32()):
        out, inn = r.i32(), r.i32()
        cells.append(r.f32s(out * inn).reshape(out, inn))
    res["W_after"] = cells
    res["y"] = r.counted()
    return res


# ---- model sessions: WMN1 descriptors, tensors, NWS1 snapshots ---------------
# src/interop/model_session.cpp:99-160, :319-404, :521-550;
# include/welvet/interop/child_wire.hpp:21-55 (Dense child);
# include/welvet/interop/model_wire.hpp:195-263 (Cameral controls).

def plain_controls():
    """Controls with no modes, no branch rates, zero coefficients, no CamSync."""
    return _i32(0) + _i32(0) + struct.pack("<3d", 0.0, 0.0, 0.0) + _i32(0)


def dense_child(W, act=-1, dtype=1, bias=None):
    out, inn = W.shape
    return _i32(1, inn, out, act, dtype) + _f32(W) + _bias(bias)


def store_snapshot(dtype, rows, cols, scale, f32=None, raw=None, bias=None):
    """One WeightStore record: dtype, rows, cols, scale, counted f32, counted
    native bytes, counted f64 bias."""
    f = np.zeros(0, np.float32) if f32 is None else np.ascontiguousarray(f32, np.float32).ravel()
    r = np.zeros(0, np.uint8) if raw is None else np.ascontiguousarray(raw, np.uint8).ravel()
    b = np.zeros(0, np.float64) if bias is None else np.ascontiguousarray(bias, np.float64)
    return (_i32(dtype, rows, cols) + struct.pack("<f", scale) + _i32(f.size) + f.tobytes() +
            _i32(r.size) + r.tobytes() + _i32(b.size) + b.tobytes())


def wmn1(root, children, snapshots, dims=(1, 1, 1, 1), cells=None):
    """children: list of child records (bytes; b"" + _i32(0) for an empty
    one), snapshots: the store records in child order, cells (Grid root):
    per cell (enabled, remote, tz, ty, tx, tl)."""
    b = struct.pack("<I", 0x314E4D57) + _i32(root, len(children), *dims)
    for c in children:
        b += c
    b += plain_controls()
    for _ in children:
        b += plain_controls()
    b += _i32(len(snapshots))
    for sn in snapshots:
        b += sn
    for meta in cells or ():
        b += _i32(*meta)
    return b


def empty_child():
    return _i32(0)


def tensor(a):
    a = np.ascontiguousarray(a, np.float32)
    return _i32(a.ndim, *a.shape) + a.tobytes()


def read_tensor(r: Reader):
    shape = tuple(r.i32() for _ in range(r.i32()))
    return r.counted().reshape(shape)


def read_nws1(data: bytes):
    """-> list of dict(dtype, rows, cols, scale, f32, raw, bias) and the
    count of extra (Mamba/GDN) records."""
    r = Reader(data)
    assert r.take(4) == struct.pack("<I", 0x3153574E)
    stores = []
    for _ in range(r.i32()):
        dt, rows, cols = r.i32(), r.i32(), r.i32()
        scale = struct.unpack("<f", r.take(4))[0]
        f = r.counted()
        raw = np.frombuffer(r.take(r.i32()), np.uint8).copy()
        bias = np.frombuffer(r.take(8 * r.i32()), np.float64).copy()
        stores.append(dict(dtype=dt, rows=rows, cols=cols, scale=scale, f32=f, raw=raw, bias=bias))
    extras = r.i32()
    assert r.done()
    return stores, extras

