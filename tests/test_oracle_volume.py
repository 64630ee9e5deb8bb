"""Pins for the oracle's volume restatement (oracle.Volume): hop order,
remote links, disabled cells, the backward chain and step_dense, checked
against hand-computable cases and against the single-layer NormalBP flow
(itself pinned by the reference's known-answer test)."""
import numpy as np

from oracle import Volume


def test_one_cell_step_is_normalbp(oracle):
    """A 1x1x1x1 volume step equals the NormalBP leaf on the same inputs:
    same loss bits and same stored weights after SGD, for several dtypes."""
    rng = np.random.default_rng(0)
    for dtype in (1, 4, 9, 26, 0):
        W = rng.normal(0, 0.3, (6, 10)).astype(np.float32)
        x = rng.normal(0, 1, (3, 10)).astype(np.float32)
        t = rng.normal(0, 1, (3, 6)).astype(np.float32)
        V = Volume(oracle, 1, 1, 1, 1, 3)
        V.bind_dense((0, 0, 0, 0), W, act=0, dtype=dtype)
        code, _, loss, y = V.train_step(x, t, 0.05)
        r = oracle.normalbp(3, 10, 6, 0, dtype, W, x, t, 1, 0.05)
        assert code == 0 and r["status"] == 0
        assert loss == r["loss"]
        np.testing.assert_array_equal(y, r["post"])
        np.testing.assert_array_equal(V.export_f32((0, 0, 0, 0)), r["W_after"])


def test_hop_order_is_z_y_x_l(oracle):
    """Cells that scale by distinct powers of two and add one only through
    their bias: the output records the order of application."""
    V = Volume(oracle, 2, 2, 1, 2, 1)
    order = []
    for k, co in enumerate(V.hop_order()):
        order.append(co)
        # y = 2*x + k (k distinct per cell): the composition is order-dependent
        V.bind_dense(co, np.array([[2.0]], np.float32), act=-1, dtype=1, bias=[float(k)])
    assert order == [(0, 0, 0, 0), (0, 0, 0, 1), (0, 1, 0, 0), (0, 1, 0, 1),
                     (1, 0, 0, 0), (1, 0, 0, 1), (1, 1, 0, 0), (1, 1, 0, 1)]
    code, _, y, tape = V.forward(np.array([[1.0]], np.float32))
    v = 1.0
    for k in range(8):
        v = 2 * v + k
    assert code == 0 and y[0, 0] == v and [c for c, *_ in tape] == order


def test_remote_link_and_disabled_cell(oracle):
    V = Volume(oracle, 1, 1, 4, 1, 2)
    V.bind_dense((0, 0, 0, 0), np.eye(3, dtype=np.float32) * 3, dtype=1)   # 3x
    V.bind_dense((0, 0, 1, 0), np.ones((2, 3), np.float32), dtype=1)        # sums
    V.bind_dense((0, 0, 2, 0), np.eye(3, dtype=np.float32) * 5, dtype=1)    # reads cell 0
    V.set_remote_link((0, 0, 2, 0), (0, 0, 0, 0))
    V.bind_dense((0, 0, 3, 0), np.eye(3, dtype=np.float32) * 7, dtype=1)
    V.set_disabled((0, 0, 3, 0))
    x = np.array([[1, 2, 3], [-1, 0, 4]], np.float32)
    code, _, y, tape = V.forward(x)
    assert code == 0 and len(tape) == 3
    np.testing.assert_array_equal(y, 15 * x)
    V.set_disabled((0, 0, 3, 0), False)
    assert V.forward(x)[2].tolist() == (105 * x).tolist()


def test_forward_errors(oracle):
    V = Volume(oracle, 1, 1, 2, 1, 1)
    V.bind_dense((0, 0, 0, 0), np.ones((2, 2), np.float32))
    code, msg, _, _ = V.forward(np.ones((1, 2), np.float32))
    assert code == 1 and msg.startswith("runtime.forward: no op")
    V.set_disabled((0, 0, 1, 0))
    assert V.forward(np.ones((1, 2), np.float32))[0] == 0
    assert V.forward(np.ones((1, 3), np.float32))[1] == "dense: input width mismatch"
    V2 = Volume(oracle, 1, 1, 2, 1, 1)
    V2.bind_dense((0, 0, 0, 0), np.ones((2, 2), np.float32))
    V2.bind_dense((0, 0, 1, 0), np.ones((2, 2), np.float32))
    V2.set_remote_link((0, 0, 0, 0), (0, 0, 1, 0))
    assert V2.forward(np.ones((1, 2), np.float32))[1].startswith("runtime.forward: remote hop")


def test_backward_chain_feeds_the_previous_step(oracle):
    """Two linear Float32 cells y = B(Ax): after one step with lr, the weight
    updates are the textbook chain-rule gradients of the MSE."""
    rng = np.random.default_rng(3)
    A = (rng.integers(-4, 5, (3, 4)) / 4).astype(np.float32)
    B = (rng.integers(-4, 5, (2, 3)) / 4).astype(np.float32)
    x = (rng.integers(-4, 5, (2, 4)) / 2).astype(np.float32)
    t = (rng.integers(-4, 5, (2, 2)) / 2).astype(np.float32)
    V = Volume(oracle, 1, 1, 2, 1, 2)
    V.bind_dense((0, 0, 0, 0), A)
    V.bind_dense((0, 0, 1, 0), B)
    code, _, loss, y = V.train_step(x, t, 0.125)
    h = x.astype(np.float64) @ A.T
    out = h @ B.T
    g = 2 * (out - t) / out.size
    assert loss == np.mean((out - t) ** 2)
    np.testing.assert_allclose(V.export_f32((0, 0, 1, 0)), B - 0.125 * (g.T @ h), rtol=1e-6)
    np.testing.assert_allclose(V.export_f32((0, 0, 0, 0)), A - 0.125 * ((g @ B).T @ x), rtol=1e-6)


def test_step_errors(oracle):
    V = Volume(oracle, 1, 1, 1, 1, 1)
    V.bind_dense((0, 0, 0, 0), np.ones((2, 2), np.float32), dtype=9)
    before = V.export_f32((0, 0, 0, 0)).copy()
    x = np.ones((1, 2), np.float32)
    assert V.train_step(x, np.zeros((1, 2), np.float32), 0.0)[:2] == (1, "training: LR is 0")
    assert V.train_step(x, np.zeros((1, 3), np.float32), 0.1)[:2] == (1, "training: MSE shape")
    code, msg, _, _ = V.train_step(x, np.array([[np.nan, 0]], np.float32), 0.1)
    assert (code, msg) == (1, "weights: nonfinite gradient")
    np.testing.assert_array_equal(V.export_f32((0, 0, 0, 0)), before)
    # a remote hop whose gradient does not fit the step before it
    V2 = Volume(oracle, 1, 1, 3, 1, 1)
    V2.bind_dense((0, 0, 0, 0), np.ones((3, 4), np.float32))
    V2.bind_dense((0, 0, 1, 0), np.ones((5, 3), np.float32))
    V2.bind_dense((0, 0, 2, 0), np.ones((2, 3), np.float32))
    V2.set_remote_link((0, 0, 2, 0), (0, 0, 0, 0))
    assert V2.train_step(np.ones((1, 4), np.float32), np.zeros((1, 2), np.float32),
                         0.1)[:2] == (1, "dense: bwd shape mismatch")
