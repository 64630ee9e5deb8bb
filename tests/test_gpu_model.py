"""welvet_model_* sessions on the GPU for Dense-only Stack and Grid roots
against the oracle's Stack and Volume restatements: forward, forward_pair,
backward, apply_sgd and train_mse to the Dense bars (1e-5 relative per
chained stage), and the NWS1 snapshot — byte for byte the descriptor's stores
before any training, the oracle's re-encoded stores after it (a few elements
one code step apart at most, where fl32(old - lr g) sat on a rounding
boundary within the dW error)."""
import numpy as np
import pytest

import model_desc
import pywelvet
import wire
from oracle import Stack, Volume
from parity import rel_err

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    pywelvet.init()


def _layers(rng):
    return [(rng.normal(0, 0.2, (48, 64)).astype(np.float32), 0, 4, rng.normal(0, 0.1, 48)),
            (rng.normal(0, 0.2, (40, 48)).astype(np.float32), 3, 26, None),
            (rng.normal(0, 0.2, (32, 40)).astype(np.float32), -1, 1, rng.normal(0, 0.1, 32))]


def _oracle_stack(oracle, layers):
    S = Stack(oracle)
    for W, act, dt, b in layers:
        S.add_dense(W, act, dt, b)
    return S


def _snap_bytes(oracle, layers):
    return [model_desc.snapshot(oracle, W, dt, b) for W, act, dt, b in layers]


def _check_store(got, want_raw, want_scale, dtype, label):
    if dtype == 1:
        w = want_raw.view(np.float32)
        atol = 4 * float(np.spacing(np.float32(np.abs(w).max())))
        np.testing.assert_allclose(got["f32"], w, rtol=0, atol=atol, err_msg=label)
        return
    assert got["scale"] == np.float32(want_scale), label
    diff = got["raw"] != want_raw
    assert diff.mean() <= 1e-2, (label, diff.mean())


def test_stack_session(oracle):
    rng = np.random.default_rng(900)
    layers = _layers(rng)
    desc = model_desc.stack(oracle, layers)
    x = rng.normal(0, 1, (5, 64)).astype(np.float32)
    t = rng.normal(0, 1, (5, 32)).astype(np.float32)
    gy = rng.normal(0, 1, (5, 32)).astype(np.float32)
    S = _oracle_stack(oracle, layers)
    with pywelvet.Model(desc) as m:
        # untouched: the snapshot comes back byte for byte
        st, blob = m.export()
        assert st.code == 0
        want = b"".join(_snap_bytes(oracle, layers))
        assert blob[:4] == b"NWS1" and blob[8:8 + len(want)] == want
        stores, extras = wire.read_nws1(blob)
        assert len(stores) == 3 and extras == 0
        # forward, forward_pair
        st, out = m.call("forward", wire.tensor(x))
        assert st.code == 0, st.message
        y = wire.read_tensor(wire.Reader(out))
        _, pres, posts = S.forward(x)
        assert y.shape == (5, 32) and rel_err(y, posts[-1]) <= 3e-5
        st, out = m.call("forward_pair", wire.tensor(x))
        r = wire.Reader(out)
        pre, post = wire.read_tensor(r), wire.read_tensor(r)
        assert rel_err(pre, pres[-1]) <= 3e-5 and rel_err(post, posts[-1]) <= 3e-5
        # backward: input gradient and dW, no update
        st, out = m.call("backward", wire.tensor(x) + wire.tensor(gy))
        assert st.code == 0, st.message
        r = wire.Reader(out)
        gx, dw = wire.read_tensor(r), wire.read_tensor(r)
        ogx, odw = S.backward(x, gy)
        assert gx.shape == x.shape and dw.shape == (1, odw.size)
        assert rel_err(gx, ogx) <= 3e-5 and rel_err(dw.ravel(), odw) <= 3e-5
        assert m.export()[1] == blob  # backward left the stores alone
        # train_mse (NormalBP): loss and the updated stores
        st, loss = m.train_mse(1, 1e-2, wire.tensor(x) + wire.tensor(t))
        assert st.code == 0, st.message
        code, oloss = S.train_mse(x, t, 1e-2)
        assert code == 0 and abs(loss - oloss) <= 3e-5 * oloss
        stores, _ = wire.read_nws1(m.export()[1])
        for i, (got, c) in enumerate(zip(stores, S.children)):
            _check_store(got, c["raw"], c["scale"], c["dtype"], f"child {i}")
        # Freeze: the loss only
        before = m.export()[1]
        st, loss = m.train_mse(30, 1e-2, wire.tensor(x) + wire.tensor(t))
        assert st.code == 0 and loss > 0 and m.export()[1] == before
        # apply_sgd with a given dW
        dwt = rng.normal(0, 1e-2, odw.size).astype(np.float32)
        assert m.apply_sgd(0.5, wire.tensor(dwt.reshape(1, -1))).code == 0
        # the oracle from the same stores as the session now holds
        for c, got in zip(S.children, wire.read_nws1(before)[0]):
            c["raw"] = (got["f32"].view(np.uint8) if c["dtype"] == 1 else got["raw"]).copy()
        assert S.apply_sgd(dwt, 0.5) == 0
        for i, (got, c) in enumerate(zip(wire.read_nws1(m.export()[1])[0], S.children)):
            _check_store(got, c["raw"], c["scale"], c["dtype"], f"sgd child {i}")
        # errors of the segment calls
        st, _ = m.call("backward", wire.tensor(x) + wire.tensor(gy[:, :5]))
        assert (st.code, st.message.decode()) == (1, "segment output gradient shape mismatch")
        st, _ = m.call("forward", wire.tensor(x[:, :7]))
        assert (st.code, st.message.decode()) == (1, "stack fwd: dense: input width mismatch")
        assert m.sync(0).code == 0


def test_grid_session(oracle):
    rng = np.random.default_rng(901)
    dims = (1, 1, 2, 2)
    cells = {(0, 0, 0, 0): dict(W=rng.normal(0, 0.3, (24, 16)).astype(np.float32), act=0, dtype=4),
             (0, 0, 0, 1): dict(W=rng.normal(0, 0.3, (24, 24)).astype(np.float32), act=1, dtype=26,
                                bias=rng.normal(0, 0.1, 24)),
             (0, 0, 1, 0): dict(W=rng.normal(0, 0.3, (9, 24)).astype(np.float32), act=3, dtype=9,
                                enabled=False),
             (0, 0, 1, 1): dict(W=rng.normal(0, 0.3, (8, 24)).astype(np.float32), act=-1, dtype=1,
                                remote=(0, 0, 0, 0))}
    # widths chain through the tape (the backward passes each step's input
    # gradient to the step before it, remote link or not: backward.cpp:100-120)
    desc = model_desc.grid(oracle, dims, cells)
    V = Volume(oracle, *dims, 6)
    for co, c in cells.items():
        V.bind_dense(co, c["W"], act=c.get("act", -1), dtype=c.get("dtype", 1), bias=c.get("bias"))
        if not c.get("enabled", True):
            V.set_disabled(co)
        if c.get("remote"):
            V.set_remote_link(co, c["remote"])
    x = rng.normal(0, 1, (6, 16)).astype(np.float32)
    t = rng.normal(0, 1, (6, 8)).astype(np.float32)
    with pywelvet.Model(desc) as m:
        snap = m.export()[1]
        st, out = m.call("forward", wire.tensor(x))
        assert st.code == 0, st.message
        y = wire.read_tensor(wire.Reader(out))
        code, _, ry, _ = V.forward(x)
        assert code == 0 and y.shape == (6, 8) and rel_err(y, ry) <= 3e-5
        # a batch of another size in the same session
        st, out = m.call("forward", wire.tensor(x[:2]))
        assert st.code == 0 and rel_err(wire.read_tensor(wire.Reader(out)), V.forward(x[:2])[2]) <= 3e-5
        # lr 0 and Freeze: the loss only (cameral_train.cpp:416-419)
        for mode, lr in ((1, 0.0), (30, 1e-2)):
            st, loss = m.train_mse(mode, lr, wire.tensor(x) + wire.tensor(t))
            assert st.code == 0 and abs(loss - oracle.mse(ry, t)) <= 3e-5 * loss
            assert m.export()[1] == snap
        # NormalBP (Inherit resolves to it)
        st, loss = m.train_mse(0, 1e-2, wire.tensor(x) + wire.tensor(t))
        assert st.code == 0, st.message
        code, _, oloss, _ = V.train_step(x, t, 1e-2)
        assert code == 0 and abs(loss - oloss) <= 3e-5 * oloss
        stores, _ = wire.read_nws1(m.export()[1])
        order = [co for co in wire.hops(dims) if co in cells]
        for got, co in zip(stores, order):
            c = V.cells[co]
            _check_store(got, c["raw"], c["scale"], c["dtype"], str(co))
        # outside the BP family, and the grid's sync
        st, _ = m.train_mse(3, 1e-2, wire.tensor(x) + wire.tensor(t))
        assert st.code == 2
        st = m.sync(0)
        assert (st.code, st.message.decode()) == (1, "grid synchronization is configured per cell at mount")
        st, _ = m.call("backward", wire.tensor(x) + wire.tensor(t))
        assert (st.code, st.message.decode()) == (1, "segment backward expects Stack or Parallel")


def test_grid_session_trains_at_two_batches(oracle):
    """A grid session trained at batch 2 and then at batch 6: the second step
    needs every cell's [batch][out] gradient buffer at the larger batch (the
    step's dX writes the cell below's buffer, the derivative is applied in
    place).  Each step's loss and stores agree with the oracle's volume at
    that batch started from the session's own stores."""
    rng = np.random.default_rng(902)
    dims = (1, 1, 1, 3)
    cells = {(0, 0, 0, 0): dict(W=rng.normal(0, 0.1, (128, 64)).astype(np.float32), act=0, dtype=9),
             (0, 0, 0, 1): dict(W=rng.normal(0, 0.1, (256, 128)).astype(np.float32), act=6, dtype=1),
             (0, 0, 0, 2): dict(W=rng.normal(0, 0.1, (128, 256)).astype(np.float32), act=-1, dtype=4)}
    desc = model_desc.grid(oracle, dims, cells)
    order = [co for co in wire.hops(dims) if co in cells]
    with pywelvet.Model(desc) as m:
        for batch in (2, 6, 3):
            before = wire.read_nws1(m.export()[1])[0]
            V = Volume(oracle, *dims, batch)
            for co, c in cells.items():
                V.bind_dense(co, c["W"], act=c["act"], dtype=c["dtype"])
            for got, co in zip(before, order):
                c = V.cells[co]
                c["raw"] = (got["f32"].view(np.uint8) if c["dtype"] == 1 else got["raw"]).copy()
            x = rng.normal(0, 1, (batch, 64)).astype(np.float32)
            t = rng.normal(0, 1, (batch, 128)).astype(np.float32)
            st, loss = m.train_mse(1, 1e-2, wire.tensor(x) + wire.tensor(t))
            assert st.code == 0, st.message
            code, _, oloss, _ = V.train_step(x, t, 1e-2)
            assert code == 0 and abs(loss - oloss) <= 3e-5 * oloss, (batch, loss, oloss)
            for got, co in zip(wire.read_nws1(m.export()[1])[0], order):
                c = V.cells[co]
                _check_store(got, c["raw"], c["scale"], c["dtype"], f"batch {batch} {co}")


@pytest.mark.parametrize("dtype", [1, 2, 4, 5, 7, 9, 14, 26, 33],
                         ids=["f32", "f16", "e4m3", "e5m2", "int32", "int8", "int4", "nf4", "uint3"])
def test_stack_apply_sgd_unaligned_slices(oracle, dtype):
    """apply_sgd on a Stack whose children's dW slices of the one gradient
    tensor start off 16-byte boundaries (15 and 50 floats in): each child's
    SGD takes the one-element-per-thread kernel and its stored bytes equal the
    oracle's re-encode exactly."""
    from parity import assert_bit_equal

    rng = np.random.default_rng(3100 + dtype)
    layers = [(rng.normal(0, 0.3, (5, 3)).astype(np.float32), -1, dtype, None),
              (rng.normal(0, 0.3, (7, 5)).astype(np.float32), -1, dtype, None),
              (rng.normal(0, 0.3, (6, 7)).astype(np.float32), -1, dtype, None)]
    S = _oracle_stack(oracle, layers)
    dwt = rng.normal(0, 0.5, 15 + 35 + 42).astype(np.float32)
    with pywelvet.Model(model_desc.stack(oracle, layers)) as m:
        assert m.apply_sgd(0.25, wire.tensor(dwt.reshape(1, -1))).code == 0
        stores, _ = wire.read_nws1(m.export()[1])
    assert S.apply_sgd(dwt, 0.25) == 0
    moved = 0
    for i, (got, c) in enumerate(zip(stores, S.children)):
        if dtype == 1:
            assert_bit_equal(got["f32"], c["raw"].view(np.float32), f"child {i}")
            moved += int(np.count_nonzero(got["f32"] != layers[i][0].ravel()))
            continue
        assert got["scale"] == np.float32(c["scale"]), i
        assert_bit_equal(got["raw"], c["raw"], f"child {i}")
        moved += int(np.count_nonzero(got["raw"] != oracle.pack(dtype, layers[i][0])[0]))
    assert moved > 0
