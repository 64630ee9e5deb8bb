"""SwiGLU over Dense on the GPU (welvet_swiglu_forward_f32 /
welvet_swiglu_normalbp_f32, reference c_abi.cpp:326-432 and
src/layers/swiglu/swiglu.cpp) against the oracle's composition of pinned
Dense functions: pre (h), post, dX within 1e-5 relative per layer stage (two
chained Dense products: 2e-5), dW within the backward bar, W_after up to one
code step at <= 1% of elements; the WVS1 / WSB1 wires through the tool."""
import numpy as np
import pytest

import pywelvet
import wire
from parity import rel_err

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    pywelvet.init()


def _weights(rng, inter, inn, dtype):
    if dtype == 16:  # unscaled FP4: a range the format resolves
        mk = lambda *s: rng.uniform(-6, 6, s).astype(np.float32)
    else:
        mk = lambda *s: rng.normal(0, 1.0 / np.sqrt(s[1]), s).astype(np.float32)
    return mk(inter, inn), mk(inter, inn), mk(inn, inter)


def _check_w_after(got, want, dtype, lr, dW):
    """Float stores: within the error lr * dW carries (dW of Gate and Up is
    fp32-rounded from a different summation order) plus a few ulp; coded
    stores: identical but for <= 1% of elements one code step apart (values
    of fl32(old - lr g) within that error of a rounding boundary)."""
    if dtype in (0, 1):
        atol = 4 * float(np.spacing(np.float32(np.abs(want).max()))) + abs(lr) * 3e-5 * np.abs(dW).max()
        np.testing.assert_allclose(got, want, rtol=0, atol=atol)
        return
    diff = got != want
    assert diff.mean() <= 1e-2, diff.mean()
    if diff.any():
        vals = np.unique(want)
        step = np.max(np.abs(np.diff(vals))) if vals.size > 1 else 0
        assert np.abs(got[diff] - want[diff]).max() <= step + 1e-6


@pytest.mark.parametrize("dtype,rows,seq", [(1, 1, 1), (4, 1, 1), (26, 1, 1), (9, 6, 2), (16, 8, 1),
                                            (5, 3, 3), (14, 40, 1), (0, 2, 1)])
def test_forward_matches_oracle(oracle, dtype, rows, seq):
    rng = np.random.default_rng(300 + dtype)
    inn, inter = 128, 344
    G, U, D = _weights(rng, inter, inn, dtype)
    x = rng.normal(0, 1, (rows, inn)).astype(np.float32)
    print(f"swiglu fwd dtype={dtype} rows={rows} seq={seq}", flush=True)
    pre, post = pywelvet.swiglu_forward(G, U, D, x, dtype=dtype, seq=seq)
    o = oracle.swiglu_normalbp(dtype, G, U, D, x)
    assert rel_err(pre, o["pre"]) <= 1e-5, rel_err(pre, o["pre"])
    assert rel_err(post, o["post"]) <= 2e-5, rel_err(post, o["post"])


@pytest.mark.parametrize("dtype", [1, 4, 9, 26, 16, 3])
def test_normalbp_matches_oracle(oracle, dtype):
    rng = np.random.default_rng(400 + dtype)
    for rows, inn, inter, use_target, lr in ((1, 64, 96, 1, 1e-2), (6, 48, 128, 0, 0.1),
                                             (12, 40, 72, 1, 0.0)):
        G, U, D = _weights(rng, inter, inn, dtype)
        x = rng.normal(0, 1, (rows, inn)).astype(np.float32)
        t = rng.normal(0, 1, (rows, inn)).astype(np.float32)
        print(f"swiglu nbp dtype={dtype} rows={rows} {inn}/{inter}", flush=True)
        r = pywelvet.swiglu_normalbp(G, U, D, x, t, use_target, lr, dtype=dtype)
        o = oracle.swiglu_normalbp(dtype, G, U, D, x, t, use_target, lr)
        assert o["status"] == 0
        assert rel_err(r["pre"], o["pre"]) <= 1e-5
        assert rel_err(r["post"], o["post"]) <= 2e-5
        # dX passes back through two Dense products and op_swiglu: 3e-5
        assert rel_err(r["dX"], o["dX"]) <= 3e-5, rel_err(r["dX"], o["dX"])
        n = inter * inn
        for k in range(3):  # Gate, Up, Down thirds, each against its own scale
            e = rel_err(r["dW"][k * n:(k + 1) * n], o["dW"][k * n:(k + 1) * n])
            assert e <= 3e-5, (k, e)
        assert abs(r["loss"] - o["loss"]) <= 2e-5 * max(1.0, abs(o["loss"]))
        _check_w_after(r["W_after"], o["W_after"], dtype, lr, o["dW"])


def test_argument_errors():
    G = np.ones((4, 2), np.float32)
    D = np.ones((2, 4), np.float32)
    x = np.ones((1, 2), np.float32)
    st, _, _ = pywelvet.swiglu_forward(G, G, D, x, dtype=34, status=True)
    assert st.code == 2 and st.message.decode().startswith("swiglu Gate: ")
    r = pywelvet.swiglu_normalbp(G, G, D, x, np.zeros((1, 2)), 1, 0.1, dtype=34, status=True)
    assert (r["status"].code, r["status"].message.decode()) == (1, "swiglu nbp: bad dtype 34")
    # a non-finite gradient stops the SGD at the first part (Gate)
    r = pywelvet.swiglu_normalbp(G, G, D, x, np.array([[np.inf, 0]], np.float32), 0, 0.1, dtype=9,
                                 status=True)
    assert (r["status"].code, r["status"].message.decode()) == (1, "weights: nonfinite gradient")


def test_wires_match_the_abi(oracle):
    rng = np.random.default_rng(500)
    inn, inter, rows = 96, 160, 4
    G, U, D = _weights(rng, inter, inn, 26)
    x = rng.normal(0, 1, (rows, inn)).astype(np.float32)
    t = rng.normal(0, 1, (rows, inn)).astype(np.float32)
    rc, out, err = wire.run(wire.wvs(G, U, D, x, dtype=26, seq=2))
    assert rc == 0, err
    r = wire.Reader(out)
    pre, post = wire.read_wvso(r)
    assert r.done()
    a_pre, a_post = pywelvet.swiglu_forward(G, U, D, x, dtype=26, seq=2)
    np.testing.assert_array_equal(pre, a_pre.ravel())
    np.testing.assert_array_equal(post, a_post.ravel())
    rc, out, err = wire.run(wire.wsb(G, U, D, x, t, 1, 1e-2, dtype=26), "--bench=3")
    assert rc == 0, err
    r = wire.Reader(out)
    b = wire.read_bench(r)
    assert b["iters"] == 3 and b["ns"] > 0
    got = wire.read_wsbo(r)
    assert r.done()
    ab = pywelvet.swiglu_normalbp(G, U, D, x, t, 1, 1e-2, dtype=26)
    for k in ("pre", "post", "dX", "dW", "W_after"):
        np.testing.assert_array_equal(got[k], ab[k].ravel(), err_msg=k)
    assert got["loss"] == ab["loss"]
    o = oracle.swiglu_normalbp(26, G, U, D, x, t, 1, 1e-2)
    assert rel_err(got["post"], o["post"].ravel()) <= 2e-5


@pytest.mark.parametrize("inn", [512, 2560])
@pytest.mark.parametrize("rows", [1, 3, 8, 40])
@pytest.mark.parametrize("dtype", [4, 26, 1, 9])
def test_gated_epilogue_on_every_up_route(oracle, dtype, rows, inn):
    """op_swiglu's product runs in the Up projection's epilogue (Gate leaves
    g in h, Up turns each element into fl32(silu(g)) * u): batch 1 (GEMV),
    3 (batched GEMV), 8 (no-split GEMM at K = 512, the k-split GEMM and its
    reduction at K = 2560) and 40 (32/64-row GEMM + reduction), split-x and
    fp32-MFMA formats; h and the output against the oracle."""
    rng = np.random.default_rng(700 + dtype + rows + inn)
    inter = 392
    G, U, D = _weights(rng, inter, inn, dtype)
    x = rng.normal(0, 1, (rows, inn)).astype(np.float32)
    print(f"swiglu gated dtype={dtype} rows={rows} in={inn}", flush=True)
    pre, post = pywelvet.swiglu_forward(G, U, D, x, dtype=dtype)
    o = oracle.swiglu_normalbp(dtype, G, U, D, x)
    assert rel_err(pre, o["pre"]) <= 1e-5, rel_err(pre, o["pre"])
    assert rel_err(post, o["post"]) <= 2e-5, rel_err(post, o["post"])


@pytest.mark.parametrize("inn,inter", [(128, 389), (1056, 389), (4096, 1024), (8192, 264)])
@pytest.mark.parametrize("dtype", [4, 5, 26, 16, 9, 14, 15])
def test_batch1_gate_up_one_launch(oracle, dtype, inn, inter):
    """Batch 1: Gate and Up in one launch (x read once per block, the
    product in the epilogue) for every format the pair kernel takes, with
    one wave per row (the in-wave epilogue), 2-8 waves (the slice sum), a
    ragged last wave and a partial last row group; h and the output against
    the oracle."""
    rng = np.random.default_rng(900 + dtype + inn + inter)
    G, U, D = _weights(rng, inter, inn, dtype)
    x = rng.normal(0, 1, (1, inn)).astype(np.float32)
    print(f"swiglu pair dtype={dtype} {inn}/{inter}", flush=True)
    pre, post = pywelvet.swiglu_forward(G, U, D, x, dtype=dtype)
    o = oracle.swiglu_normalbp(dtype, G, U, D, x)
    assert rel_err(pre, o["pre"]) <= 1e-5, rel_err(pre, o["pre"])
    assert rel_err(post, o["post"]) <= 2e-5, rel_err(post, o["post"])


def test_c3_shape_forward(oracle):
    """The config-3 shape 4096 -> 11008 -> 4096 as one SwiGLU (NF4 and FP4
    Gate/Up/Down) at batch 1 and 8, against the oracle."""
    rng = np.random.default_rng(0x5EED0003)
    inn, inter = 4096, 11008
    for dtype in (26, 16):
        G, U, D = _weights(rng, inter, inn, dtype)
        for rows in (1, 8):
            x = rng.normal(0, 1, (rows, inn)).astype(np.float32)
            print(f"swiglu C3 dtype={dtype} rows={rows}", flush=True)
            pre, post = pywelvet.swiglu_forward(G, U, D, x, dtype=dtype)
            o = oracle.swiglu_normalbp(dtype, G, U, D, x)
            assert rel_err(pre, o["pre"]) <= 1e-5
            assert rel_err(post, o["post"]) <= 1e-4  # K = 11008 in Down: the 1e-4 bar


def test_resident_session_matches_one_shot():
    """welvet_hip_swiglu_forward_device gives the one-shot forward's bytes
    (device buffers from the HIP runtime the library itself uses)."""
    import ctypes as C
    hip = C.CDLL("libamdhip64.so")
    hip.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    hip.hipFree.argtypes = [C.c_void_p]
    rng = np.random.default_rng(501)
    inn, inter, rows = 256, 688, 8
    G, U, D = _weights(rng, inter, inn, 26)
    x = rng.normal(0, 1, (rows, inn)).astype(np.float32)
    pre, post = pywelvet.swiglu_forward(G, U, D, x, dtype=26)
    bufs = []
    for n in (x.nbytes, pre.nbytes, post.nbytes):
        p = C.c_void_p()
        assert hip.hipMalloc(C.byref(p), n) == 0
        bufs.append(p)
    try:
        assert hip.hipMemcpy(bufs[0], x.ctypes.data, x.nbytes, 1) == 0  # host to device
        with pywelvet.SwigluSession(G, U, D, rows, dtype=26) as L:
            for _ in range(2):
                pywelvet.check(L.forward_device(bufs[0].value, bufs[1].value, bufs[2].value))
            assert hip.hipDeviceSynchronize() == 0
        h, y = np.empty_like(pre), np.empty_like(post)
        assert hip.hipMemcpy(h.ctypes.data, bufs[1], h.nbytes, 2) == 0  # device to host
        assert hip.hipMemcpy(y.ctypes.data, bufs[2], y.nbytes, 2) == 0
    finally:
        for p in bufs:
            hip.hipFree(p)
    np.testing.assert_array_equal(h, pre)
    np.testing.assert_array_equal(y, post)
