"""GPU volume runtime against the oracle's volume restatement: hop order,
remote links, disabled cells, error messages, and training steps
(MSE, reverse backward, SGD with re-encode) on multi-cell grids."""
import numpy as np
import pytest

import pywelvet
from oracle import Volume
from parity import assert_close, rel_err, tol_for_k

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    pywelvet.init()


def build(oracle, dims, batch, spec, remote=(), disabled=()):
    """spec: {coord: (W, act, dtype, bias)} -> (GPU grid, oracle volume)."""
    G = pywelvet.Grid(*dims, batch)
    V = Volume(oracle, *dims, batch)
    for co, (W, act, dt, bias) in spec.items():
        G.bind_dense(co, W, act=act, dtype=dt, bias=bias)
        V.bind_dense(co, W, act=act, dtype=dt, bias=bias)
    for co, t in remote:
        G.set_remote_link(co, t)
        V.set_remote_link(co, t)
    for co in disabled:
        G.set_disabled(co)
        V.set_disabled(co)
    return G, V


def test_c1_single_cell_tanh(oracle):
    """Config 1: 1x1x1 volume, Dense 512->512 Float32, batch 1, tanh,
    W ~ U(-0.05, 0.05), x ~ N(0, 1)."""
    rng = np.random.default_rng(0x5EED0000)
    W = rng.uniform(-0.05, 0.05, (512, 512)).astype(np.float32)
    x = rng.normal(0, 1, (1, 512)).astype(np.float32)
    G, V = build(oracle, (1, 1, 1, 1), 1, {(0, 0, 0, 0): (W, 3, 1, None)})
    with G:
        y = G.forward(x, 512)
    code, _, ry, _ = V.forward(x)
    assert code == 0
    assert_close(y, ry, 512, "c1")


def _stack_spec(rng, dims, width, dtypes, acts=None):
    spec = {}
    coords = [(z, yy, xx, l) for z in range(dims[0]) for yy in range(dims[1])
              for xx in range(dims[2]) for l in range(dims[3])]
    for i, co in enumerate(coords):
        W = rng.normal(0, 1.0 / np.sqrt(width), (width, width)).astype(np.float32)
        act = (acts[i] if acts else (0 if i < len(coords) - 1 else -1))
        bias = rng.normal(0, 0.1, width) if i % 3 == 0 else None
        spec[co] = (W, act, dtypes[i % len(dtypes)], bias)
    return spec


def test_forward_2x2x2x4_mixed_dtypes(oracle):
    rng = np.random.default_rng(5)
    dtypes = [1, 4, 26, 9, 16, 2, 3, 5, 14, 0, 27, 13]
    spec = _stack_spec(rng, (2, 2, 2, 4), 128, dtypes)
    G, V = build(oracle, (2, 2, 2, 4), 16, spec)
    x = rng.normal(0, 1, (16, 128)).astype(np.float32)
    with G:
        y = G.forward(x, 128)
    code, _, ry, _ = V.forward(x)
    assert code == 0
    # 32 chained layers, each within the 1e-5 per-layer bound: 1e-5 per layer
    e = rel_err(y, ry)
    assert e <= 32 * 1e-5, e


def test_remote_link_disabled_and_widths(oracle):
    rng = np.random.default_rng(6)
    spec = {(0, 0, 0, 0): (rng.normal(0, 0.3, (24, 16)), 0, 4, None),
            (0, 0, 1, 0): (rng.normal(0, 0.3, (12, 24)), 1, 26, rng.normal(0, 1, 12)),
            (0, 0, 2, 0): (rng.normal(0, 0.3, (8, 24)), 3, 9, None),
            (0, 0, 3, 0): (rng.normal(0, 0.3, (8, 8)), -1, 1, None)}
    G, V = build(oracle, (1, 1, 5, 1), 3, spec, remote=[((0, 0, 2, 0), (0, 0, 0, 0))],
                 disabled=[(0, 0, 4, 0)])
    x = rng.normal(0, 1, (3, 16)).astype(np.float32)
    with G:
        y = G.forward(x, 8)
        code, _, ry, _ = V.forward(x)
        assert code == 0
        assert_close(y, ry, 24, "remote")


def test_forward_errors_match_oracle(oracle):
    rng = np.random.default_rng(7)
    W = rng.normal(0, 0.3, (4, 4)).astype(np.float32)
    x = np.ones((1, 4), np.float32)
    with pywelvet.Grid(1, 1, 2, 1, 1) as G:
        G.bind_dense((0, 0, 0, 0), W)
        st, _ = G.forward(x, 4, status=True)
        assert st.code == 1 and st.message.decode().startswith("runtime.forward: no op at z=0 y=0 x=1")
        G.set_disabled((0, 0, 1, 0))
        assert G.forward(x, 4).shape == (1, 4)
        st, _ = G.forward(np.ones((1, 5), np.float32), 4, status=True)
        assert (st.code, st.message.decode()) == (1, "dense: input width mismatch")
        st = G.bind_dense((0, 0, 2, 0), W, status=True)
        assert st.code == 1 and st.message.decode() == "architecture: bad bind coord z=0 y=0 x=2 l=0"
        st = G.set_remote_link((0, 0, 0, 0), (0, 0, 9, 0), status=True)
        assert st.code == 1 and "bad target coord" in st.message.decode()
        st = G.bind_dense((0, 0, 1, 0), W, dtype=34, status=True)
        assert st.code == 2
    with pywelvet.Grid(1, 1, 2, 1, 1) as G:
        G.bind_dense((0, 0, 0, 0), W)
        G.bind_dense((0, 0, 1, 0), W)
        G.set_remote_link((0, 0, 0, 0), (0, 0, 1, 0))
        st, _ = G.forward(x, 4, status=True)
        assert st.code == 1 and "remote hop has no recorded activation" in st.message.decode()


def _check_weights(G, V, spec, label):
    """After SGD the stored weights agree with the oracle's up to what the
    forward/backward tolerance allows in dW: Float32/Float64 stores within a
    few ulp (lr*dW is far below one ulp of the weight's error budget); coded
    stores identical except where fl32(old - lr*g) sat within that error of a
    rounding boundary — at most 1% of elements, each by about one code step."""
    for co, (_, _, dtype, _) in spec.items():
        a, b = G.export_f32(co), V.export_f32(co)
        if dtype in (0, 1):
            # a few ulp of the matrix's largest weight: the error of lr*dW is
            # absolute, not relative to each weight
            atol = 4 * float(np.spacing(np.float32(np.abs(b).max())))
            np.testing.assert_allclose(a, b, rtol=4e-7, atol=atol, err_msg=f"{label} {co}")
            continue
        diff = a != b
        assert diff.mean() <= 1e-2, (label, co, diff.mean())
        if diff.any():
            step = np.abs(a[diff] - b[diff])
            span = np.abs(b).max() + 1e-30
            assert np.all(step <= max(span * 0.3, 1e-6)), (label, co, step.max())


@pytest.mark.parametrize("dtypes", [[1], [4, 9], [26, 1, 16], [2, 3, 5, 14]],
                         ids=["f32", "fp8-int8", "nf4-f32-fp4", "mixed"])
def test_train_steps_match_oracle(oracle, dtypes):
    rng = np.random.default_rng(11 + len(dtypes))
    dims = (1, 2, 2, 2)
    spec = _stack_spec(rng, dims, 64, dtypes)
    G, V = build(oracle, dims, 8, spec)
    x = rng.normal(0, 1, (8, 64)).astype(np.float32)
    t = rng.normal(0, 1, (8, 64)).astype(np.float32)
    with G:
        for step in range(3):
            loss, y = G.train_step(x, t, 1e-2)
            code, _, rloss, ry = V.train_step(x, t, 1e-2)
            assert code == 0
            # 8 chained layers: 1e-5 relative per layer
            assert rel_err(y, ry) <= 8 * 1e-5, (step, rel_err(y, ry))
            assert abs(loss - rloss) <= 8 * 1e-5 * abs(rloss), (step, loss, rloss)
            _check_weights(G, V, spec, f"step {step}")
            # re-sync the oracle to the GPU's stored bytes so later steps
            # compare one step each, not an accumulated drift
            for co in spec:
                raw, _ = G.native(co)
                V.cells[co]["raw"] = raw.copy()


def test_step_errors_match_oracle(oracle):
    rng = np.random.default_rng(13)
    W = rng.normal(0, 0.3, (4, 4)).astype(np.float32)
    x = rng.normal(0, 1, (2, 4)).astype(np.float32)
    for dtype, nan_code, nan_msg in ((9, 1, "weights: nonfinite gradient"),
                                     (1, 2, "SGD: gradient is not a finite f32")):
        with pywelvet.Grid(1, 1, 2, 1, 2) as G:
            G.bind_dense((0, 0, 0, 0), W, act=0, dtype=dtype)
            G.bind_dense((0, 0, 1, 0), W, dtype=dtype)
            before = [G.export_f32((0, 0, i, 0)) for i in range(2)]
            st, _, _ = G.train_step(x, np.zeros((2, 4)), 0.0, status=True)
            assert (st.code, st.message.decode()) == (1, "training: LR is 0")
            st, _, _ = G.train_step(x, np.zeros((2, 3)), 0.1, status=True)
            assert (st.code, st.message.decode()) == (1, "training: MSE shape")
            t = np.zeros((2, 4), np.float32)
            t[1, 2] = np.nan
            st, _, _ = G.train_step(x, t, 0.1, status=True)
            assert (st.code, st.message.decode()) == (nan_code, nan_msg)
            for i in range(2):
                np.testing.assert_array_equal(G.export_f32((0, 0, i, 0)), before[i])
    with pywelvet.Grid(1, 1, 2, 1, 1) as G:
        G.bind_dense((0, 0, 0, 0), W, dtype=1)
        G.bind_dense((0, 0, 1, 0), W, dtype=1)
        st, _, _ = G.train_step(x[:1], np.zeros((1, 4)), 1e300, status=True)
        assert (st.code, st.message.decode()) == (2, "SGD: learning rate outside the f32 range")
    with pywelvet.Grid(1, 1, 3, 1, 1) as G:
        G.bind_dense((0, 0, 0, 0), rng.normal(0, 1, (3, 4)))
        G.bind_dense((0, 0, 1, 0), rng.normal(0, 1, (5, 3)))
        G.bind_dense((0, 0, 2, 0), rng.normal(0, 1, (2, 3)))
        G.set_remote_link((0, 0, 2, 0), (0, 0, 0, 0))
        st, _, _ = G.train_step(np.ones((1, 4)), np.zeros((1, 2)), 0.1, status=True)
        assert (st.code, st.message.decode()) == (1, "dense: bwd shape mismatch")


def test_device_forward_writes_the_callers_buffer(oracle):
    """welvet_hip_volume_forward_device: the last layer writes the caller's
    d_y itself; the bytes equal the host-pointer forward's, on repeated calls,
    in place (d_y == d_x, where the output is copied after the layers run),
    and a host forward afterwards is unchanged."""
    from devmem import DeviceArray, Stream
    from parity import assert_bit_equal

    rng = np.random.default_rng(77)
    st = Stream()
    try:
        for widths, dt in (([256, 256], 4), ([256, 384, 256], 26), ([128, 320, 192], 1)):
            L, batch = len(widths) - 1, 3
            spec = {(0, 0, l, 0): (rng.normal(0, 0.1, (widths[l + 1], widths[l])).astype(np.float32),
                                   0 if l < L - 1 else 2, dt, rng.normal(0, 0.1, widths[l + 1]))
                    for l in range(L)}
            G, V = build(oracle, (1, 1, L, 1), batch, spec)
            with G:
                x = rng.normal(0, 1, (batch, widths[0])).astype(np.float32)
                want = G.forward(x, widths[-1])
                code, _, ry, _ = V.forward(x)
                assert code == 0
                assert_close(want, ry, max(widths), "host forward")
                dx = DeviceArray(x.shape)
                dx.upload(x)
                dy = DeviceArray((batch, widths[-1]), fill=np.nan)
                for _ in range(2):
                    pywelvet.check(pywelvet.lib().welvet_hip_volume_forward_device(
                        G.h, dx.ptr, widths[0], dy.ptr, widths[-1], st.h))
                    st.sync()
                    assert_bit_equal(dy.download(), want, f"device forward {widths}")
                if widths[0] == widths[-1]:
                    pywelvet.check(pywelvet.lib().welvet_hip_volume_forward_device(
                        G.h, dx.ptr, widths[0], dx.ptr, widths[-1], st.h))
                    st.sync()
                    assert_bit_equal(dx.download(), want, f"in-place device forward {widths}")
                assert_bit_equal(G.forward(x, widths[-1]), want, "host forward after")
                dx.free()
                dy.free()
    finally:
        st.close()


@pytest.mark.parametrize("dtype", [1, 4, 26])
@pytest.mark.parametrize("batch", [5, 16, 40])
def test_train_derivative_in_dx_epilogue(oracle, dtype, batch):
    """The piecewise activation derivatives (ReLU, ReLU2, LeakyReLU hidden
    layers) applied in the layer above's dX epilogue give the same losses and
    stored bytes, bit for bit, as the separate derivative launch, and the
    steps agree with the oracle.  Batch 40 folds it into the reduction of the
    stream-K dX GEMMs, the smaller batches into the no-split dX kernel."""
    from parity import assert_bit_equal

    rng = np.random.default_rng(2300 + 3 * dtype + batch)
    widths = [96, 128, 128, 64, 48]
    acts = [0, 6, 5, -1]
    spec = {(0, 0, l, 0): (rng.normal(0, 0.15, (widths[l + 1], widths[l])).astype(np.float32),
                           acts[l], dtype, None) for l in range(4)}
    x = rng.normal(0, 1, (batch, widths[0])).astype(np.float32)
    t = rng.normal(0, 1, (batch, widths[-1])).astype(np.float32)
    runs = {}
    for fold in (1, 0):
        old = pywelvet.set_tuning("fold_deriv", fold)
        try:
            G, V = build(oracle, (1, 1, 4, 1), batch, spec)
            with G:
                losses = []
                for step in range(2):
                    loss, y = G.train_step(x, t, 1e-2)
                    losses.append(loss)
                    if fold:
                        code, _, rloss, ry = V.train_step(x, t, 1e-2)
                        assert code == 0
                        assert rel_err(y, ry) <= 4 * 1e-5, (step, rel_err(y, ry))
                        _check_weights(G, V, spec, f"fold step {step}")
                        for co in spec:
                            V.cells[co]["raw"] = G.native(co)[0].copy()
                runs[fold] = (losses, {co: G.native(co)[0].copy() for co in spec})
        finally:
            pywelvet.set_tuning("fold_deriv", old)
    assert runs[1][0] == runs[0][0], (runs[1][0], runs[0][0])
    for co in spec:
        assert_bit_equal(runs[1][1][co], runs[0][1][co], f"store {co}")


@pytest.mark.parametrize("dtype", [4, 5, 9])
def test_train_transposed_codes_whole_tiles(oracle, dtype):
    """A training step whose second layer (512 inputs, a multiple of 256)
    refreshes its transposed codes through whole 64 x 256-byte tiles and
    takes dX through them at batch 32: outputs, losses and stored bytes
    follow the oracle over three steps."""
    rng = np.random.default_rng(2500 + dtype)
    widths = [256, 512, 256]
    acts = [0, -1]
    spec = {(0, 0, l, 0): (rng.normal(0, 0.05, (widths[l + 1], widths[l])).astype(np.float32),
                           acts[l], dtype, None) for l in range(2)}
    x = rng.normal(0, 1, (32, widths[0])).astype(np.float32)
    t = rng.normal(0, 1, (32, widths[-1])).astype(np.float32)
    G, V = build(oracle, (1, 1, 2, 1), 32, spec)
    with G:
        for step in range(3):
            loss, y = G.train_step(x, t, 1e-2)
            code, _, rloss, ry = V.train_step(x, t, 1e-2)
            assert code == 0
            assert rel_err(y, ry) <= 4 * 1e-5, (step, rel_err(y, ry))
            assert abs(loss - rloss) <= 1e-4 * max(1.0, abs(rloss)), (step, loss, rloss)
            _check_weights(G, V, spec, f"whole-tile step {step}")
            for co in spec:
                V.cells[co]["raw"] = G.native(co)[0].copy()


@pytest.mark.parametrize("dtypes,widths,xs,lr", [
    ([1, 1, 4, 4, 26, 9], [128, 256, 128, 256, 128, 128, 128], 1.0, 1e-2),
    ([5, 5, 5, 0, 16, 16], [64, 128, 128, 256, 128, 96, 48], 0.05, 1e-3)],
    ids=["f32-fp8-nf4-int8-all128", "e5m2-f64-fp4-mixed"])
def test_train_batched_sgd_and_dw_match_per_cell(oracle, dtypes, widths, xs, lr):
    """The SGD of consecutive cells of one dtype in one launch, and every
    layer's dW deferred to the end of the backward and launched several
    layers at a time (layers of 128-multiple sizes; the others keep their
    own dW launch), give the same losses and stored bytes, bit for bit, as a
    launch per cell, and agree with the oracle.  The unscaled FP4 cells of
    the mixed chain amplify: its input is scaled down and its rate lowered
    so the steps stay finite (they diverge at x ~ N(0, 1), lr 1e-2)."""
    from parity import assert_bit_equal

    rng = np.random.default_rng(2500 + sum(dtypes))
    L = len(dtypes)
    spec = {(0, 0, l, 0): (rng.normal(0, 0.15, (widths[l + 1], widths[l])).astype(np.float32),
                           0 if l < L - 1 else -1, dtypes[l], None) for l in range(L)}
    for co, (W, act, dt, b) in spec.items():
        if dt == 16:
            spec[co] = (rng.uniform(-1.5, 1.5, W.shape).astype(np.float32), act, dt, b)
    x = (rng.normal(0, 1, (6, widths[0])) * xs).astype(np.float32)
    t = rng.normal(0, 1, (6, widths[-1])).astype(np.float32)
    runs = {}
    for knobs in ((1, 1), (0, 0), (1, 0), (0, 1)):
        old = [pywelvet.set_tuning(k, v) for k, v in zip(("sgd_batch", "dw_batch"), knobs)]
        try:
            G, V = build(oracle, (1, 1, L, 1), 6, spec)
            with G:
                losses = []
                for step in range(2):
                    loss, y = G.train_step(x, t, lr)
                    losses.append(loss)
                    if knobs == (1, 1):
                        code, _, rloss, ry = V.train_step(x, t, lr)
                        assert code == 0
                        assert rel_err(y, ry) <= L * 1e-5, (step, rel_err(y, ry))
                        _check_weights(G, V, spec, f"batched step {step}")
                        for co in spec:
                            V.cells[co]["raw"] = G.native(co)[0].copy()
                runs[knobs] = (losses, {co: G.native(co)[0].copy() for co in spec})
        finally:
            for k, v in zip(("sgd_batch", "dw_batch"), old):
                pywelvet.set_tuning(k, v)
    for knobs in ((0, 0), (1, 0), (0, 1)):
        assert runs[knobs][0] == runs[(1, 1)][0], (knobs, runs[knobs][0], runs[(1, 1)][0])
        for co in spec:
            assert_bit_equal(runs[knobs][1][co], runs[(1, 1)][1][co], f"store {co} knobs {knobs}")


GROUPED_SGD = [2, 3, 7, 8, 11, 12, 14, 15, 16, 17, 18, 19, 20, 26, 27, 28, 29, 30, 31, 32, 33]


@pytest.mark.parametrize("dtype", GROUPED_SGD, ids=[pywelvet.DTYPE_NAMES[d] for d in GROUPED_SGD])
def test_batched_grouped_sgd_matches_per_cell(oracle, dtype):
    """The formats whose SGD runs several whole code words per thread: one
    batched SGD launch over three cells of ragged sizes (tails of 1-31
    elements past the last whole group, several blocks for the largest)
    stores the same bytes as a launch per cell, whose kernel the codec
    tests pin to the oracle for every dtype."""
    from parity import assert_bit_equal

    rng = np.random.default_rng(2800 + dtype)
    widths = [257, 97, 131, 40]
    spec = {(0, 0, l, 0): (rng.normal(0, 0.15, (widths[l + 1], widths[l])).astype(np.float32),
                           0 if l < 2 else -1, dtype, None) for l in range(3)}
    x = (rng.normal(0, 1, (4, widths[0])) * 0.2).astype(np.float32)
    t = rng.normal(0, 1, (4, widths[-1])).astype(np.float32)
    runs = {}
    for knob in (1, 0):
        old = pywelvet.set_tuning("sgd_batch", knob)
        try:
            G, _ = build(oracle, (1, 1, 3, 1), 4, spec)
            with G:
                before = [G.native(co)[0].copy() for co in spec]
                # a rate large enough that the coarse formats' codes move
                lr = 5e-2 if pywelvet.dtype_bits(dtype) >= 16 else 50.0
                st, loss, _ = G.train_step(x, t, lr, status=True)
                runs[knob] = (st.code, loss, before, [G.native(co)[0].copy() for co in spec])
        finally:
            pywelvet.set_tuning("sgd_batch", old)
    assert runs[1][:2] == runs[0][:2]
    for i, co in enumerate(spec):
        assert_bit_equal(runs[1][3][i], runs[0][3][i], f"{pywelvet.DTYPE_NAMES[dtype]} store {co}")
    if runs[1][0] == 0:
        assert any((runs[1][3][i] != runs[1][2][i]).any() for i in range(3))


@pytest.mark.parametrize("sgd_batch", [1, 0])
def test_train_e5m2_overflow_then_forward(oracle, sgd_batch):
    """E5M2 cells after training steps, batch 8 (where a finite E5M2 store
    takes the split-x GEMM): a step that stays finite, then one whose update
    pushes weights past the format's range (Inf codes).  After each, the
    stores are read back into the oracle and the next forward keeps the IEEE
    results: NaN and Inf where the oracle has them, finite outputs within
    tolerance."""
    rng = np.random.default_rng(2700 + sgd_batch)
    spec = {(0, 0, 0, 0): (rng.normal(0, 0.1, (128, 128)).astype(np.float32), 0, 5, None),
            (0, 0, 0, 1): (rng.normal(0, 0.1, (64, 128)).astype(np.float32), -1, 5, None)}
    x = rng.normal(0, 1, (8, 128)).astype(np.float32)
    t = rng.normal(0, 1, (8, 64)).astype(np.float32)
    old = pywelvet.set_tuning("sgd_batch", sgd_batch)
    try:
        G, V = build(oracle, (1, 1, 1, 2), 8, spec)
        with G:
            # lr 1e6: about 0.1% of the top layer's codes go to Inf (oracle)
            for step, lr in enumerate((1e-2, 1e6)):
                G.train_step(x, t, lr)
                for co in spec:
                    V.cells[co]["raw"] = G.native(co)[0].copy()
                finite = all(np.isfinite(G.export_f32(co)).all() for co in spec)
                assert finite == (step == 0), step
                x2 = rng.normal(0, 1, (8, 128)).astype(np.float32)
                y = G.forward(x2, 64)
                code, _, ry, _ = V.forward(x2)
                assert code == 0
                np.testing.assert_array_equal(np.isnan(y), np.isnan(ry))
                inf = np.isinf(ry)
                np.testing.assert_array_equal(np.where(inf, y, 0), np.where(inf, ry, 0))
                fin = np.isfinite(ry)
                assert_close(np.where(fin, y, 0), np.where(fin, ry, 0), 2 * 128, f"step {step}")
    finally:
        pywelvet.set_tuning("sgd_batch", old)


@pytest.mark.parametrize("dtype", [9, 13, 14], ids=["int8", "uint8", "int4"])
def test_batched_sgd_bad_last_store_updates_the_earlier_ones(oracle, dtype):
    """One SGD launch for two stores of one dtype where only the second
    store's dW is non-finite: the first store (1 M weights, many blocks) is
    updated in full, bit for bit as with a launch per store, and the step
    reports the reference's code.  Layer 0 has weights near 1e25, so the
    top layer's dW = dpre ⊗ h overflows f32 while layer 0's dW stays finite."""
    from parity import assert_bit_equal

    rng = np.random.default_rng(2600 + dtype)
    W0 = (rng.normal(0, 1, (1024, 1024)) * 1e25).astype(np.float32)
    W1 = rng.normal(0, 0.05, (64, 1024)).astype(np.float32)
    x = rng.normal(0, 1, (4, 1024)).astype(np.float32)
    t = rng.normal(0, 1, (4, 64)).astype(np.float32)
    spec = {(0, 0, 0, 0): (W0, -1, dtype, None), (0, 0, 0, 1): (W1, -1, dtype, None)}
    runs = {}
    for knob in (1, 0):
        old = pywelvet.set_tuning("sgd_batch", knob)
        try:
            G, V = build(oracle, (1, 1, 1, 2), 4, spec)
            with G:
                before = [G.native(co)[0].copy() for co in spec]
                st, loss, _ = G.train_step(x, t, 1.0, status=True)
                after = [G.native(co)[0].copy() for co in spec]
            runs[knob] = (st.code, st.message.decode(), before, after)
        finally:
            pywelvet.set_tuning("sgd_batch", old)
    code, msg, before, after = runs[1]
    assert (code, msg) == (1, "weights: nonfinite gradient")
    assert runs[0][:2] == (code, msg)
    # the bad store is untouched, the good one moved, both as per-store launches
    assert_bit_equal(after[1], before[1], "bad store")
    assert (after[0] != before[0]).any()
    for i in range(2):
        assert_bit_equal(after[i], runs[0][3][i], f"store {i}")
    ocode, _, _, _ = V.train_step(x, t, 1.0)
    assert ocode == 1
