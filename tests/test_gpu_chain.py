"""Sequential and Residual Dense chains on the GPU
(welvet_{sequential,residual}_{forward,normalbp}_f32, reference
c_abi.cpp:918-1090, src/layers/sequential/sequential.cpp,
src/layers/residual/residual.cpp) against the oracle's composition of pinned
Dense functions, and the WSQ1 / WRE1 / SQB1 / REB1 wires through the tool.
Each chained Dense stage carries the 1e-5 relative forward/backward bar, so
a depth-d chain is held to d * 1e-5."""
import numpy as np
import pytest

import pywelvet
import wire
from parity import rel_err

pytestmark = pytest.mark.gpu

KINDS = ["sequential", "residual"]


@pytest.fixture(scope="module", autouse=True)
def device():
    pywelvet.init()


def _packed(rng, depth, dim, dtype):
    if dtype == 16:
        return rng.uniform(-6, 6, (depth, dim, dim)).astype(np.float32) / np.float32(4)
    return rng.normal(0, 1.0 / np.sqrt(dim), (depth, dim, dim)).astype(np.float32)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("dtype,rows,seq,act", [(1, 1, 1, 3), (4, 1, 1, 0), (26, 5, 1, 1),
                                                (9, 8, 2, 2), (16, 3, 3, 4), (0, 64, 1, 6)])
def test_forward_matches_oracle(oracle, kind, dtype, rows, seq, act):
    rng = np.random.default_rng(600 + dtype + 7 * act)
    depth, dim = 3, 192
    P = _packed(rng, depth, dim, dtype)
    x = rng.normal(0, 1, (rows, dim)).astype(np.float32)
    print(f"{kind} fwd dtype={dtype} rows={rows} act={act}", flush=True)
    pre, post = pywelvet.chain_forward(kind, P, x, child_act=act, dtype=dtype, seq=seq)
    o = oracle.chain_normalbp(kind == "residual", dtype, P, x, act)
    assert rel_err(pre, o["pre"]) <= depth * 1e-5, rel_err(pre, o["pre"])
    assert rel_err(post, o["post"]) <= depth * 1e-5, rel_err(post, o["post"])


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("dtype", [1, 4, 9, 26, 3])
def test_normalbp_matches_oracle(oracle, kind, dtype):
    rng = np.random.default_rng(700 + dtype)
    for rows, dim, depth, act, use_target, lr in ((1, 64, 2, 3, 1, 1e-2), (6, 48, 3, 0, 0, 0.1),
                                                  (12, 40, 4, 2, 1, 0.0)):
        P = _packed(rng, depth, dim, dtype)
        x = rng.normal(0, 1, (rows, dim)).astype(np.float32)
        t = rng.normal(0, 1, (rows, dim)).astype(np.float32)
        print(f"{kind} nbp dtype={dtype} rows={rows} dim={dim} depth={depth}", flush=True)
        r = pywelvet.chain_normalbp(kind, P, x, t, use_target, lr, child_act=act, dtype=dtype)
        o = oracle.chain_normalbp(kind == "residual", dtype, P, x, act, t, use_target, lr)
        assert o["status"] == 0
        bar = depth * 1e-5
        for key in ("pre", "post", "dX"):
            assert rel_err(r[key], o[key]) <= 2 * bar, (key, rel_err(r[key], o[key]))
        cn = dim * dim
        for i in range(depth):
            e = rel_err(r["dW"][i * cn:(i + 1) * cn], o["dW"][i * cn:(i + 1) * cn])
            assert e <= 2 * bar, (i, e)
        assert abs(r["loss"] - o["loss"]) <= 2 * bar * max(1.0, abs(o["loss"]))
        if dtype in (0, 1):
            atol = 4 * float(np.spacing(np.float32(np.abs(o["W_after"]).max()))) + \
                abs(lr) * 2 * bar * np.abs(o["dW"]).max()
            np.testing.assert_allclose(r["W_after"], o["W_after"], rtol=0, atol=atol)
        else:
            diff = r["W_after"] != o["W_after"]
            assert diff.mean() <= 1e-2, diff.mean()


def test_errors():
    P = np.ones((2, 3, 3), np.float32)
    x = np.ones((1, 3), np.float32)
    st, _, _ = pywelvet.chain_forward("sequential", P, x, dtype=34, status=True)
    assert st.code == 2 and st.message.decode().startswith("sequential child 0: ")
    st, _, _ = pywelvet.chain_forward("residual", P, x, dtype=34, status=True)
    assert st.code == 2 and st.message.decode().startswith("residual F child 0: ")
    r = pywelvet.chain_normalbp("residual", P, x, np.array([[np.nan, 0, 0]], np.float32), 0, 0.1,
                                dtype=9, status=True)
    assert (r["status"].code, r["status"].message.decode()) == (1, "weights: nonfinite gradient")


@pytest.mark.parametrize("kind,fmagic,bmagic", [("sequential", b"WSQ1", b"SQB1"),
                                                ("residual", b"WRE1", b"REB1")])
def test_wires_match_the_abi(kind, fmagic, bmagic):
    rng = np.random.default_rng(800)
    P = _packed(rng, 3, 64, 4)
    x = rng.normal(0, 1, (4, 64)).astype(np.float32)
    t = rng.normal(0, 1, (4, 64)).astype(np.float32)
    rc, out, err = wire.run(wire.chain(fmagic, P, x, child_act=0, dtype=4, seq=2))
    assert rc == 0, err
    r = wire.Reader(out)
    pre, post = wire.read_pair(r, fmagic[:3] + b"O" if fmagic == b"WSQ1" else b"WREO")
    assert r.done()
    a_pre, a_post = pywelvet.chain_forward(kind, P, x, child_act=0, dtype=4, seq=2)
    np.testing.assert_array_equal(pre, a_pre.ravel())
    np.testing.assert_array_equal(post, a_post.ravel())
    rc, out, err = wire.run(wire.chain_nbp(bmagic, P, x, t, 1, 1e-2, child_act=0, dtype=4),
                            "--bench=2")
    assert rc == 0, err
    r = wire.Reader(out)
    assert wire.read_bench(r)["iters"] == 2
    got = wire.read_leaf(r, bmagic[:3] + b"O")
    assert r.done()
    ab = pywelvet.chain_normalbp(kind, P, x, t, 1, 1e-2, child_act=0, dtype=4)
    for k in ("pre", "post", "dX", "dW", "W_after"):
        np.testing.assert_array_equal(got[k], ab[k].ravel(), err_msg=k)
    assert got["loss"] == ab["loss"]
