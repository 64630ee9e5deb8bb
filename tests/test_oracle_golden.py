"""The oracle against the reference's own outputs: the golden vectors written
from the compiled reference codec (tests/golden/make_golden.py), the
release_smoke known-answer test, and — when oracle/_ref is built — direct
comparison with the reference build on fresh random inputs."""
import json
import os

import numpy as np
import pytest

from oracle import DTYPE_NAMES, Reference, have_reference


def _bits(a):
    a = np.asarray(a)
    return a.view(np.uint64 if a.dtype == np.float64 else np.uint32)


def test_codec_vectors_bit_exact(oracle, golden_dir):
    z = np.load(os.path.join(golden_dir, "codec_vectors.npz"))
    sets = sorted({k.split("/")[0] for k in z.files})
    checked = 0
    for s in sets:
        w = z[f"{s}/input"]
        for dt, name in enumerate(DTYPE_NAMES):
            key = f"{s}/{name}"
            native, scale = oracle.pack(dt, w)
            np.testing.assert_array_equal(native, z[key + "/native"], err_msg=key)
            assert _bits(np.float32(scale)) == _bits(z[key + "/scale"][0]), key
            np.testing.assert_array_equal(_bits(oracle.decode(dt, native, scale, w.size)),
                                          _bits(z[key + "/decode"]), err_msg=key)
            np.testing.assert_array_equal(_bits(oracle.decode_f64(dt, native, scale, w.size)),
                                          _bits(z[key + "/decode_f64"]), err_msg=key)
            checked += 1
    assert checked == len(sets) * 34


def test_platform_patches_are_the_documented_ones(golden_dir):
    """The x86/arm64 divergences in the fixtures are only the undefined
    conversions: Int32 +absmax (reference native_codec.cpp:256-258) and a NaN
    quotient in the 64-bit unsigned formats (:333-336)."""
    z = np.load(os.path.join(golden_dir, "codec_vectors.npz"))
    for k in z.files:
        if not k.endswith("/native_x86"):
            continue
        name = k.split("/")[1]
        if name == "int32":
            a = z[k].view("<i4")
            b = z[k.replace("native_x86", "native")].view("<i4")
            d = np.nonzero(a != b)[0]
            assert len(d) >= 1 and np.all(a[d] == -2**31) and np.all(b[d] == 2**31 - 1)
        else:
            assert name in ("uint64", "uint", "uintptr"), k
            a = z[k][4:].view("<u8")
            b = z[k.replace("native_x86", "native")][4:].view("<u8")
            d = np.nonzero(a != b)[0]
            assert len(d) == 1 and a[d[0]] == 1 << 63 and b[d[0]] == 0


def test_scalar_tables(oracle, golden_dir):
    t = np.load(os.path.join(golden_dir, "scalar_tables.npz"))
    for kind, (nm, n) in enumerate((("f16", 65536), ("bf16", 65536), ("e4m3", 256), ("e5m2", 256),
                                    ("fp4", 16))):
        got = oracle.decode_many(kind, np.arange(n))
        np.testing.assert_array_equal(_bits(got), _bits(t[f"{nm}_decode"]), err_msg=nm)
    # signaling-NaN codes keep their payload bits (f16: sign | 0x7f800000 |
    # mant << 13, float_codecs.cpp:41-46; bf16: the code << 16)
    f16 = _bits(t["f16_decode"])
    for h in (0x7C01, 0x7D55, 0xFC01, 0x7E00):
        assert f16[h] == ((h & 0x8000) << 16) | 0x7F800000 | ((h & 0x3FF) << 13), hex(h)
    assert _bits(t["bf16_decode"])[0x7F81] == 0x7F810000
    for kind, nm in enumerate(("f16", "bf16", "e4m3", "e5m2", "fp4")):
        np.testing.assert_array_equal(oracle.encode_many(kind, t["encode_input"]),
                                      t[f"{nm}_encode"], err_msg=nm)


def test_release_smoke_kat(oracle, golden_dir):
    k = json.load(open(os.path.join(golden_dir, "release_kat.json")))
    g = k["geometry"]
    r = oracle.normalbp(g["batch"], g["in"], g["out"], g["act"], g["dtype"],
                        np.array(k["W_init"], np.float32), np.array(k["x"], np.float32),
                        np.array(k["target"], np.float32), k["use_target"], k["lr"])
    assert r["status"] == 0
    assert list(r["post"].ravel()) == k["expect_post"]
    assert abs(r["loss"] - k["expect_loss"]) < k["tolerance"]
    assert np.all(np.abs(r["W_after"].ravel() - np.array(k["expect_W_after"])) < k["tolerance"])


@pytest.mark.skipif(not have_reference(), reason="oracle/_ref not built (no reference checkout)")
@pytest.mark.parametrize("seed", range(3))
def test_oracle_matches_reference_build(oracle, seed):
    R = Reference()
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 3000))
    for w in (rng.normal(0, 0.02, n), rng.uniform(-6, 6, n), rng.normal(0, 10, n)):
        w = w.astype(np.float32)
        for dt, name in enumerate(DTYPE_NAMES):
            a, sa = oracle.pack(dt, w)
            b, sb = R.pack(dt, w)
            if name == "int32":  # +absmax element: arm64 saturates, x86 wraps
                d = np.nonzero(a.view("<i4") != b.view("<i4"))[0]
                assert np.all(a.view("<i4")[d] == 2**31 - 1)
                b = a.copy()
            np.testing.assert_array_equal(a, b, err_msg=name)
            assert np.float32(sa) == np.float32(sb)
            np.testing.assert_array_equal(_bits(oracle.decode(dt, a, sa, n)),
                                          _bits(R.decode(dt, a, sa, n)), err_msg=name)


@pytest.mark.skipif(not have_reference(), reason="oracle/_ref not built (no reference checkout)")
def test_scalar_encoders_strided_sweep(oracle):
    """Every 4099th f32 bit pattern (about 1M inputs incl. NaN/Inf/subnormals).
    WELVET_FULL_SWEEP=1 runs all 2^32 (about 10 minutes)."""
    R = Reference()
    full = os.environ.get("WELVET_FULL_SWEEP") == "1"
    step = 1 if full else 4099
    chunk = 1 << 24
    for start in range(0, 1 << 32, chunk * step):
        x = (np.arange(start, min(start + chunk * step, 1 << 32), step, dtype=np.uint64)
             .astype(np.uint32).view(np.float32))
        for kind in range(5):
            np.testing.assert_array_equal(oracle.encode_many(kind, x), R.encode_many(kind, x))
