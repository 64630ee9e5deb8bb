"""GPU parity of the fresh-scale repack (welvet_hip_dense_repack /
welvet_hip_grid_repack: WeightStore::set_from_f32_gpu native_codec.cpp:872-907,
op_native_repack ops_storage.metal:971-1144) against the oracle's or_repack,
bit for bit, for all 34 dtypes: the native bytes, the scale, the decode, and a
forward after the repack (decode tables and the FP8 decode-ready copy follow
the new codes)."""
import numpy as np
import pytest

import pywelvet
from oracle import DTYPE_NAMES, Volume
from parity import assert_bit_equal, assert_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    pywelvet.init()


def inputs(rng, out, inn):
    yield "normal", rng.normal(0, 0.5, (out, inn)).astype(np.float32)
    yield "uniform6", rng.uniform(-6, 6, (out, inn)).astype(np.float32)
    w = rng.normal(0, 1, (out, inn)).astype(np.float32)
    w[0, 0] = np.nan                 # element 0 is NaN: skipped by the statistics
    w[3, 7], w[5, 1] = np.nan, -0.0
    yield "nan", w
    yield "constant", np.full((out, inn), 0.375, np.float32)   # span 0 -> 1
    yield "zeros", np.zeros((out, inn), np.float32)            # absmax 0 -> 1
    w = rng.uniform(0, 1, (out, inn)).astype(np.float32)
    w[0, :3] = [0.0, 1.0, np.float32(13981013 * 2.0 ** -24)]   # the Uint2 f32-product case
    yield "ratios", w


@pytest.mark.parametrize("dtype", range(34), ids=DTYPE_NAMES)
def test_repack_matches_oracle(oracle, dtype):
    rng = np.random.default_rng(900 + dtype)
    out, inn = 48, 256
    W0 = rng.normal(0, 0.1, (out, inn)).astype(np.float32)
    with pywelvet.Session(W0, batch=3, act=-1, dtype=dtype) as s:
        for name, W in inputs(rng, out, inn):
            s.repack(W)
            raw, scale = s.native()
            want, wscale = oracle.repack(dtype, W)
            assert_bit_equal(raw, want, f"{DTYPE_NAMES[dtype]} {name} native")
            assert np.float32(scale) == np.float32(wscale), (name, scale, wscale)
            dec = s.export_f32()
            assert_bit_equal(dec.ravel(), oracle.decode(dtype, want, wscale, W.size), f"{name} decode")
            if not np.all(np.isfinite(dec)):
                continue
            x = rng.normal(0, 1, (3, inn)).astype(np.float32)
            pre, _ = s.execute(x)
            Wd = oracle.decode_f64(dtype, want, wscale, W.size).reshape(out, inn)
            rpre, _ = oracle.forward(Wd, x, -1)
            assert_close(pre, rpre, inn, f"{DTYPE_NAMES[dtype]} {name} forward after repack")


@pytest.mark.parametrize("dtype", [4, 5, 26, 16, 9])
@pytest.mark.parametrize("batch", [1, 8, 64])
def test_forward_routes_after_repack(oracle, dtype, batch):
    """The GEMV and both GEMM routes read the repacked store: FP8 through its
    decode-ready copy, NF4 through its rebuilt table and split parts, E5M2
    after a repack that brings Inf codes in (the split-x GEMM stays off)."""
    rng = np.random.default_rng(950 + dtype + batch)
    out, inn = 300, 1024
    W0 = rng.normal(0, 0.02, (out, inn)).astype(np.float32)
    W1 = rng.normal(0, 2.0, (out, inn)).astype(np.float32)
    if dtype == 5:
        W1[7, 9] = 1e6  # past E5M2's range: an Inf code
    with pywelvet.Session(W0, batch=batch, act=1, dtype=dtype) as s:
        s.repack(W1)
        want, wscale = oracle.repack(dtype, W1)
        Wd = oracle.decode_f64(dtype, want, wscale, W1.size).reshape(out, inn)
        x = rng.normal(0, 1, (batch, inn)).astype(np.float32)
        pre, post = s.execute(x)
        rpre, rpost = oracle.forward(Wd, x, 1)
        if dtype == 5:
            fin = np.isfinite(rpre)
            np.testing.assert_array_equal(np.isfinite(pre), fin)
            assert_close(np.where(fin, pre, 0), np.where(fin, rpre, 0), inn, "e5m2 finite outputs")
        else:
            assert_close(pre, rpre, inn, "pre")
            assert_close(post, rpost, inn, "post")


def test_repack_errors_and_grid_cell(oracle):
    rng = np.random.default_rng(77)
    W = rng.normal(0, 0.1, (16, 32)).astype(np.float32)
    with pywelvet.Session(W, batch=1, dtype=9) as s:
        st = s.repack(np.zeros(15 * 32, np.float32), status=True)
        assert (st.code, st.message.decode()) == (1, "blend: invalid native store replacement")
        before, _ = s.native()
        st = s.repack(np.zeros(0, np.float32), status=True)
        assert st.code == 1
        after, _ = s.native()
        np.testing.assert_array_equal(before, after)  # a refused repack leaves the store alone
    # a grid cell, then the volume forward reads the repacked cell
    G = pywelvet.Grid(1, 1, 2, 1, 2)
    V = Volume(oracle, 1, 1, 2, 1, 2)
    W0, W1 = rng.normal(0, 0.2, (24, 32)), rng.normal(0, 0.2, (8, 24))
    for co, Wc, dt in (((0, 0, 0, 0), W0, 26), ((0, 0, 1, 0), W1, 13)):
        G.bind_dense(co, Wc, act=0, dtype=dt)
        V.bind_dense(co, Wc, act=0, dtype=dt)
    Wn = rng.normal(0, 0.5, (24, 32)).astype(np.float32)
    with G:
        G.repack((0, 0, 0, 0), Wn)
        raw, scale = oracle.repack(26, Wn)
        V.cells[(0, 0, 0, 0)]["raw"], V.cells[(0, 0, 0, 0)]["scale"] = raw, scale
        got, gscale = G.native((0, 0, 0, 0))
        assert_bit_equal(got, raw, "grid cell native")
        assert np.float32(gscale) == np.float32(scale)
        st = G.repack((0, 0, 1, 0), np.zeros(3, np.float32), status=True)
        assert st.code == 1
        x = rng.normal(0, 1, (2, 32)).astype(np.float32)
        y = G.forward(x, 8)
        code, _, ry, _ = V.forward(x)
        assert code == 0
        assert_close(y, ry, 24, "volume forward after a cell repack")
