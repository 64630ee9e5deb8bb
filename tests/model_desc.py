"""WMN1 descriptors for the model-session tests, with store snapshots made
by the oracle's pinned codec (the bytes a reference store holds)."""
import numpy as np

import wire


def snapshot(oracle, W, dtype, bias=None):
    W = np.ascontiguousarray(W, np.float32)
    out, inn = W.shape
    if dtype == 1:  # WeightStore::f32, no native bytes, scale 1
        return wire.store_snapshot(1, out, inn, 1.0, f32=W, bias=bias)
    raw, scale = oracle.pack(dtype, W)
    return wire.store_snapshot(dtype, out, inn, scale, raw=raw, bias=bias)


def stack(oracle, layers):
    """layers: [(W, act, dtype, bias)] -> WMN1 bytes of a Stack root."""
    children = [wire.dense_child(W, act, dt, b) for W, act, dt, b in layers]
    snaps = [snapshot(oracle, W, dt, b) for W, act, dt, b in layers]
    return wire.wmn1(0, children, snaps)


def grid(oracle, dims, cells):
    """cells: {coord: dict(W=, act=, dtype=, bias=, enabled=, remote=None|coord)}
    in any order; hops without an entry are empty and disabled."""
    children, snaps, meta = [], [], []
    for co in wire.hops(dims):
        c = cells.get(co)
        if c is None:
            children.append(wire.empty_child())
            meta.append((0, 0, 0, 0, 0, 0))
            continue
        children.append(wire.dense_child(c["W"], c.get("act", -1), c.get("dtype", 1), c.get("bias")))
        snaps.append(snapshot(oracle, c["W"], c.get("dtype", 1), c.get("bias")))
        rem = c.get("remote")
        meta.append((int(c.get("enabled", True)), 0 if rem is None else 1, *(rem or (0, 0, 0, 0))))
    return wire.wmn1(2, children, snaps, dims=dims, cells=meta)
