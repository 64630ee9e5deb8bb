"""The wire tool on the GPU: each Dense wire's reply against the oracle, to
the same bars as the C-ABI tests (pre/post/dX within 1e-5 relative of the f64
restatement, dW and losses as there, W_after up to one code step at <= 1% of
elements), and the bench framing.  The tool is its own process, so each case
starts one short-lived process on the GPU, one after the other."""
import numpy as np
import pytest

import wire
from oracle import Volume
from parity import assert_close, rel_err

pytestmark = pytest.mark.gpu


def _oracle_forward(oracle, W, x, act, dtype, bias):
    raw, scale = oracle.pack(dtype, W)
    return oracle.forward_native(dtype, raw, scale, x, W.shape[0], W.shape[1], act, bias)


@pytest.mark.parametrize("dtype,batch,act", [(1, 1, 3), (4, 1, -1), (26, 1, 0), (9, 5, 1),
                                             (16, 8, 2), (5, 3, 4), (14, 64, 6), (0, 2, 5)])
def test_wvd3_matches_oracle(oracle, dtype, batch, act):
    rng = np.random.default_rng(100 + dtype)
    out, inn = 96, 256
    W = rng.normal(0, 0.3, (out, inn)).astype(np.float32)
    if dtype == 16:
        W = rng.uniform(-6, 6, (out, inn)).astype(np.float32)  # unscaled FP4
    x = rng.normal(0, 1, (batch, inn)).astype(np.float32)
    bias = rng.normal(0, 0.1, out - 7)  # partial bias: o < bias_len only
    print(f"WVD3 dtype={dtype} batch={batch} act={act}", flush=True)
    rc, outb, err = wire.run(wire.wvd(W, x, act=act, dtype=dtype, bias=bias))
    assert rc == 0, err
    r = wire.Reader(outb)
    pre, post = wire.read_wvo(r, batch, out)
    assert r.done()
    rpre, rpost = _oracle_forward(oracle, W, x, act, dtype, bias)
    assert_close(pre, rpre, inn, "pre")
    assert_close(post, rpost, inn, "post")


def test_wvd1_wvd2_defaults(oracle):
    """WVD1 carries no dtype (Float32); WVD2 no backend (main.cpp:44-56)."""
    rng = np.random.default_rng(3)
    W = rng.normal(0, 0.3, (40, 64)).astype(np.float32)
    x = rng.normal(0, 1, (2, 64)).astype(np.float32)
    rpre, rpost = _oracle_forward(oracle, W, x, 0, 1, None)
    rc, outb, err = wire.run(wire.wvd(W, x, act=0, version=1))
    assert rc == 0, err
    pre, post = wire.read_wvo(wire.Reader(outb), 2, 40)
    assert_close(post, rpost, 64, "WVD1")
    rc, outb, err = wire.run(wire.wvd(W, x, act=0, dtype=9, version=2))
    assert rc == 0, err
    pre, post = wire.read_wvo(wire.Reader(outb), 2, 40)
    assert_close(post, _oracle_forward(oracle, W, x, 0, 9, None)[1], 64, "WVD2")


def test_wvd_bench_framing_and_errors(oracle):
    rng = np.random.default_rng(4)
    W = rng.normal(0, 0.02, (11008, 4096)).astype(np.float32)
    x = rng.normal(0, 1, (1, 4096)).astype(np.float32)
    payload = wire.wvd(W, x, dtype=4)
    rc, plain, err = wire.run(payload)
    assert rc == 0, err
    rc, outb, err = wire.run(payload, "--bench=20")
    assert rc == 0, err
    r = wire.Reader(outb)
    b = wire.read_bench(r)
    assert b["iters"] == 20 and b["mount_ns"] > 0 and b["exec_ns"] > 0
    pre, post = wire.read_wvo(r, 1, 11008)
    assert r.done()
    # the bench's last execute and the one-shot forward give the same bytes
    assert outb[-len(plain):] == plain
    print(f"WVD3 fp8 4096x11008 b1 through the wire: mount {b['mount_ns'] / 1e6:.2f} ms, "
          f"execute {b['exec_ns'] / 20 / 1e3:.1f} us (host buffers)", flush=True)
    rpre, _ = _oracle_forward(oracle, W, x, -1, 4, None)
    assert_close(pre, rpre, 4096, "bench pre")
    # a library error is exit 1 with its message (main.cpp:138-141)
    rc, outb, err = wire.run(wire.wvd(W[:4, :8], x[:, :8], dtype=34))
    assert rc == 1 and outb == b"" and err.startswith("welvet_dense_fwd: ")


@pytest.mark.parametrize("dtype", [1, 4, 9, 26, 16, 3])
def test_wdb1_matches_oracle(oracle, dtype):
    rng = np.random.default_rng(200 + dtype)
    for batch, out, inn, act, use_target, lr in ((1, 64, 128, 3, 1, 1e-2), (6, 40, 96, 0, 0, 0.1),
                                                 (3, 24, 97, 2, 1, 0.0)):
        W = rng.normal(0, 0.3, (out, inn)).astype(np.float32)
        if dtype == 16:
            W = rng.uniform(-6, 6, (out, inn)).astype(np.float32)
        x = rng.normal(0, 1, (batch, inn)).astype(np.float32)
        t = rng.normal(0, 1, (batch, out)).astype(np.float32)
        bias = rng.normal(0, 0.1, out)
        print(f"WDB1 dtype={dtype} batch={batch} {out}x{inn}", flush=True)
        rc, outb, err = wire.run(wire.wdb(W, x, t, use_target, lr, act=act, dtype=dtype, bias=bias))
        assert rc == 0, err
        r = wire.Reader(outb)
        got = wire.read_wdbo(r)
        assert r.done()
        o = oracle.normalbp(batch, inn, out, act, dtype, W, x, t, use_target, lr, bias=bias)
        assert o["status"] == 0
        for key in ("pre", "post", "dX", "dW"):
            assert got[key].size == o[key].size, key
            assert rel_err(got[key], o[key].ravel()) <= 1e-5, (key, rel_err(got[key], o[key].ravel()))
        assert abs(got["loss"] - o["loss"]) <= 1e-5 * max(1.0, abs(o["loss"]))
        if use_target == 0:
            assert got["loss"] == 0.0
        diff = np.abs(got["W_after"].astype(np.float64) - o["W_after"].ravel())
        vals = np.unique(o["W_after"])
        step = np.max(np.abs(np.diff(vals))) if vals.size > 1 else 0
        assert np.mean(diff > 0) <= 0.01 and (diff.max() <= step + 1e-6 or diff.max() <= 1e-5)


def test_wdb1_bench_framing():
    rng = np.random.default_rng(5)
    W = rng.normal(0, 0.3, (32, 48)).astype(np.float32)
    x = rng.normal(0, 1, (4, 48)).astype(np.float32)
    t = rng.normal(0, 1, (4, 32)).astype(np.float32)
    payload = wire.wdb(W, x, t, 1, 1e-2, act=0, dtype=9)
    rc, plain, err = wire.run(payload)
    assert rc == 0, err
    rc, outb, err = wire.run(payload, "--bench=5")
    assert rc == 0, err
    r = wire.Reader(outb)
    b = wire.read_bench(r)
    assert b["iters"] == 5 and b["ns"] > 0
    # every step starts from the wire's weights, so the exported step equals
    # the one-shot reply byte for byte
    assert outb[r.p:] == plain


def _volume_cells(rng, dims, width, dtypes):
    cells = {}
    co_list = wire.hops(dims)
    for i, co in enumerate(co_list):
        W = rng.normal(0, 1.0 / np.sqrt(width), (width, width)).astype(np.float32)
        act = 0 if i < len(co_list) - 1 else -1
        bias = rng.normal(0, 0.1, width) if i % 3 == 0 else None
        cells[co] = (W, act, dtypes[i % len(dtypes)], bias)
    return cells


def _oracle_volume(oracle, dims, batch, cells, links=()):
    V = Volume(oracle, *dims, batch)
    for co, (W, act, dt, bias) in cells.items():
        V.bind_dense(co, W, act=act, dtype=dt, bias=bias)
    for src, dst in links:
        V.set_remote_link(src, dst)
    return V


def test_wvf1_matches_oracle(oracle):
    rng = np.random.default_rng(6)
    dims = (2, 1, 2, 2)
    cells = _volume_cells(rng, dims, 64, [1, 4, 26, 9, 16, 2])
    x = rng.normal(0, 1, (4, 64)).astype(np.float32)
    rc, outb, err = wire.run(wire.wvf(dims, 4, cells, x))
    assert rc == 0, err
    r = wire.Reader(outb)
    y = wire.read_wvfo(r)
    assert r.done()
    code, _, ry, _ = _oracle_volume(oracle, dims, 4, cells).forward(x)
    assert code == 0
    assert rel_err(y, ry.ravel()) <= 8 * 1e-5  # 8 chained layers, 1e-5 each

    # remote link: hop 2 reads hop 0's post; bench framing
    cells = {(0, 0, 0, 0): (rng.normal(0, 0.3, (24, 16)).astype(np.float32), 0, 4, None),
             (0, 0, 1, 0): (rng.normal(0, 0.3, (12, 24)).astype(np.float32), 1, 26, rng.normal(0, 1, 12)),
             (0, 0, 2, 0): (rng.normal(0, 0.3, (8, 24)).astype(np.float32), 3, 9, None)}
    links = [((0, 0, 2, 0), (0, 0, 0, 0))]
    x = rng.normal(0, 1, (3, 16)).astype(np.float32)
    rc, outb, err = wire.run(wire.wvf((1, 1, 3, 1), 3, cells, x, links), "--bench=4")
    assert rc == 0, err
    r = wire.Reader(outb)
    b = wire.read_bench(r)
    assert b["iters"] == 4 and b["mount_ns"] > 0
    y = wire.read_wvfo(r)
    code, _, ry, _ = _oracle_volume(oracle, (1, 1, 3, 1), 3, cells, links).forward(x)
    assert code == 0
    assert_close(y, ry.ravel(), 24, "remote")


def test_wvf1_errors():
    rng = np.random.default_rng(7)
    W = rng.normal(0, 0.3, (4, 4)).astype(np.float32)
    x = np.ones((1, 4), np.float32)
    # a hop sent without a record has no op: the forward names it
    rc, outb, err = wire.run(wire.wvf((1, 1, 2, 1), 1, {(0, 0, 0, 0): (W, -1, 1, None)}, x))
    assert (rc, outb) == (1, b"")
    assert err.strip() == "welvet_dense_fwd: runtime.forward: no op at z=0 y=0 x=1 l=0"
    # a link outside the grid
    rc, outb, err = wire.run(wire.wvf((1, 1, 1, 1), 1, {(0, 0, 0, 0): (W, -1, 1, None)}, x,
                                      links=[((0, 0, 0, 0), (0, 0, 5, 0))]))
    assert rc == 1 and "bad target coord" in err


@pytest.mark.parametrize("dtypes", [[1], [4, 9], [26, 1, 16]], ids=["f32", "fp8-int8", "nf4-f32-fp4"])
def test_wvn1_matches_oracle(oracle, dtypes):
    rng = np.random.default_rng(8 + len(dtypes))
    dims = (1, 2, 1, 2)
    cells = _volume_cells(rng, dims, 48, dtypes)
    x = rng.normal(0, 1, (6, 48)).astype(np.float32)
    t = rng.normal(0, 1, (6, 48)).astype(np.float32)
    print(f"WVN1 dtypes={dtypes}", flush=True)
    rc, outb, err = wire.run(wire.wvn(dims, 6, cells, x, t, 1e-2))
    assert rc == 0, err
    r = wire.Reader(outb)
    got = wire.read_wvno(r)
    assert r.done()
    V = _oracle_volume(oracle, dims, 6, cells)
    code, _, loss, ry = V.train_step(x, t, 1e-2)
    assert code == 0
    assert abs(got["loss"] - loss) <= 4 * 1e-5 * abs(loss)
    assert rel_err(got["y"], ry.ravel()) <= 4 * 1e-5
    # the input gradient passes back through all 4 cells
    assert got["grad_in"].size == x.size
    assert rel_err(got["grad_in"], V.grad_in.ravel()) <= 8 * 1e-5
    assert len(got["W_after"]) == len(cells)
    for Wa, co in zip(got["W_after"], wire.hops(dims)):
        want = V.export_f32(co)
        if cells[co][2] in (0, 1):
            atol = 4 * float(np.spacing(np.float32(np.abs(want).max())))
            np.testing.assert_allclose(Wa, want, rtol=4e-7, atol=atol)
        else:
            diff = Wa != want
            assert diff.mean() <= 1e-2, (co, diff.mean())


def test_wvn1_bench_and_errors():
    rng = np.random.default_rng(9)
    cells = {(0, 0, 0, 0): (rng.normal(0, 0.3, (8, 8)).astype(np.float32), 0, 9, None),
             (0, 0, 1, 0): (rng.normal(0, 0.3, (8, 8)).astype(np.float32), -1, 4, None)}
    x = rng.normal(0, 1, (2, 8)).astype(np.float32)
    t = rng.normal(0, 1, (2, 8)).astype(np.float32)
    payload = wire.wvn((1, 1, 2, 1), 2, cells, x, t, 1e-2)
    rc, plain, err = wire.run(payload)
    assert rc == 0, err
    rc, outb, err = wire.run(payload, "--bench=3")
    assert rc == 0, err
    r = wire.Reader(outb)
    b = wire.read_bench(r)
    assert b["iters"] == 3 and b["ns"] > 0
    assert outb[r.p:] == plain  # every step rebuilds the grid from the wire
    # LR 0 is a training error (training.cpp:61-70)
    rc, outb, err = wire.run(wire.wvn((1, 1, 2, 1), 2, cells, x, t, 0.0))
    assert (rc, outb, err.strip()) == (1, b"", "welvet_dense_fwd: training: LR is 0")
    # a bad link: the library's message, then the wire's own
    rc, outb, err = wire.run(wire.wvn((1, 1, 2, 1), 2, cells, x, t, 1e-2,
                                      links=[((0, 0, 9, 0), (0, 0, 0, 0))]))
    lines = err.strip().splitlines()
    assert rc == 1 and "bad source coord" in lines[0]
    assert lines[1] == "welvet_dense_fwd: WVN1: bad links"
