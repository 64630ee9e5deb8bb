"""GPU codec parity: the device encoder, decoder and SGD re-encode against the
reference's golden vectors and the oracle, bit for bit, all 34 dtypes."""
import os

import numpy as np
import pytest

import pywelvet
from oracle import DTYPE_NAMES
from parity import assert_bit_equal, bits

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    pywelvet.init()
    assert pywelvet.identity().startswith("hip:gfx950")


def gpu_pack(dtype, w2d):
    with pywelvet.Session(w2d, batch=1, dtype=dtype) as s:
        native, scale = s.native()
        dec = s.export_f32()
    return native, scale, dec


@pytest.mark.parametrize("dtype", range(34), ids=DTYPE_NAMES)
def test_pack_and_decode_match_reference_vectors(dtype, golden_dir):
    """Golden vectors written by the compiled reference codec (tests/golden)."""
    z = np.load(os.path.join(golden_dir, "codec_vectors.npz"))
    name = DTYPE_NAMES[dtype]
    for s in sorted({k.split("/")[0] for k in z.files}):
        w = z[f"{s}/input"]
        native, scale, dec = gpu_pack(dtype, w.reshape(1, -1))
        key = f"{s}/{name}"
        assert_bit_equal(native, z[key + "/native"], key + " native")
        assert bits(np.float32(scale)) == bits(z[key + "/scale"][0]), key
        assert_bit_equal(dec.ravel(), z[key + "/decode"], key + " decode")


@pytest.mark.parametrize("dtype", range(34), ids=DTYPE_NAMES)
def test_pack_matches_oracle_on_matrices(dtype, oracle):
    rng = np.random.default_rng(1000 + dtype)
    for shape, dist in (((64, 1000), "n002"), ((33, 257), "u6"), ((128, 4096), "n1")):
        if dist == "n002":
            w = rng.normal(0, 0.02, shape)
        elif dist == "u6":
            w = rng.uniform(-6, 6, shape)
        else:
            w = rng.normal(0, 1, shape)
        w = w.astype(np.float32)
        native, scale, dec = gpu_pack(dtype, w)
        want, wscale = oracle.pack(dtype, w)
        assert_bit_equal(native, want, f"{DTYPE_NAMES[dtype]} {shape} native")
        assert np.float32(scale) == np.float32(wscale)
        assert_bit_equal(dec.ravel(), oracle.decode(dtype, want, wscale, w.size), "decode")


@pytest.mark.parametrize("dtype", range(34), ids=DTYPE_NAMES)
def test_sgd_reencode_matches_oracle(dtype, oracle):
    """WeightStore::apply_sgd with a host gradient: every native byte equal."""
    rng = np.random.default_rng(2000 + dtype)
    # (129, 257): many blocks of the grouped kernels and a one-element tail
    for shape, lr, gscale in (((16, 96), 1e-3, 1.0), ((7, 33), 0.5, 3.0), ((64, 512), 1e-2, 0.1),
                              ((129, 257), 1e-2, 1.0)):
        w = rng.normal(0, 0.5, shape).astype(np.float32)
        g = (rng.normal(0, gscale, shape)).astype(np.float32)
        with pywelvet.Session(w, batch=1, dtype=dtype) as s:
            s.sgd(g, lr)
            native, _ = s.native()
            after = s.export_f32()
        if dtype == 1:  # Float32 store: welvet_sgd_f32_f64_grad
            ref = w.copy()
            oracle.sgd_f32(ref, g, lr)
            assert_bit_equal(after, ref, "float32 sgd")
            continue
        raw, scale = oracle.pack(dtype, w)
        assert oracle.native_sgd(dtype, raw, scale, w.size, g, lr) == 0
        assert_bit_equal(native, raw, f"{DTYPE_NAMES[dtype]} {shape} sgd native")
        assert_bit_equal(after.ravel(), oracle.decode(dtype, raw, scale, w.size), "sgd decode")


@pytest.mark.parametrize("dtype", [d for d in range(34) if d != 1], ids=[n for i, n in enumerate(DTYPE_NAMES) if i != 1])
def test_sgd_zero_rate_matches_oracle(dtype, oracle):
    """lr = 0 still re-encodes every element (ops_storage.metal:946-957): the
    bytes must follow the reference, including codes the re-encode rewrites."""
    rng = np.random.default_rng(3000 + dtype)
    w = rng.normal(0, 0.02, (32, 96)).astype(np.float32)
    g = rng.normal(0, 1, w.shape).astype(np.float32)
    with pywelvet.Session(w, batch=1, dtype=dtype) as s:
        s.sgd(g, 0.0)
        native, _ = s.native()
    raw, scale = oracle.pack(dtype, w)
    oracle.native_sgd(dtype, raw, scale, w.size, g, 0.0)
    assert_bit_equal(native, raw, DTYPE_NAMES[dtype])


def test_sgd_rewrites_e4m3_subnormal_codes(oracle):
    """E4M3 subnormal codes decode to signed zero (float_codecs.cpp:106-111) and
    zero encodes to 0x00 (:58-60), so any SGD step rewrites them to 0x00."""
    w = np.array([[2.0**-8, -(2.0**-8), 3 * 2.0**-9, 1.0]], np.float32)
    with pywelvet.Session(w, batch=1, dtype=4) as s:
        before, _ = s.native()
        s.sgd(np.zeros_like(w), 0.0)
        after, _ = s.native()
    assert list(before[:3]) != [0, 0, 0] and list(after[:3]) == [0, 0, 0]
    raw, scale = oracle.pack(4, w)
    oracle.native_sgd(4, raw, scale, w.size, np.zeros(w.size, np.float32), 0.0)
    assert_bit_equal(after, raw, "e4m3 subnormal rewrite")


def test_sgd_rejects_nonfinite(oracle):
    w = np.ones((2, 2), np.float32)
    g = np.array([[0, np.inf], [0, 0]], np.float32)
    with pywelvet.Session(w, batch=1, dtype=9) as s:
        before, _ = s.native()
        st = s.sgd(g, 0.1, status=True)
        assert st.code == 1  # native_codec.cpp:926-927
        assert_bit_equal(s.native()[0], before, "unchanged")
        st = s.sgd(np.zeros_like(w), float("nan"), status=True)
        assert st.code == 1
    with pywelvet.Session(w, batch=1, dtype=1) as s:
        assert s.sgd(g, 0.1, status=True).code == 2  # training.mm:122-124
        assert s.sgd(np.zeros_like(w), 1e300, status=True).code == 2  # training.mm:75-78


@pytest.mark.parametrize("dtype", [9, 4], ids=["int8", "e4m3"])
def test_sgd_reencode_at_config4_size(dtype, oracle):
    """WeightStore::apply_sgd on config 4's 8192 x 2048 store (16.8 M codes:
    the 16-codes-per-thread kernel) with a host gradient: every native byte
    equal to the oracle's re-encode, and a fair share of the codes moved."""
    rng = np.random.default_rng(2100 + dtype)
    shape = (8192, 2048)
    w = (rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02 if dtype == 9 else 1.0))
    g = rng.standard_normal(shape, dtype=np.float32)
    lr = 2e-3 if dtype == 9 else 2e-2
    with pywelvet.Session(w, batch=1, dtype=dtype) as s:
        before, _ = s.native()
        s.sgd(g, lr)
        native, _ = s.native()
    raw, scale = oracle.pack(dtype, w)
    assert_bit_equal(before, raw, "packed")
    assert oracle.native_sgd(dtype, raw, scale, w.size, g, lr) == 0
    assert_bit_equal(native, raw, f"{DTYPE_NAMES[dtype]} 8192x2048 sgd native")
    assert np.count_nonzero(native != before) > w.size // 20
