"""Pins for the oracle's op_native_repack restatement (or_repack,
shaders/ops_storage.metal:971-1144; WeightStore::set_from_f32_gpu
native_codec.cpp:872-907).  The kernel is Metal-only, so the reference build
cannot run it: its codes are pinned against or_pack (itself pinned to the
reference build's golden vectors) where the two are the same arithmetic, and
by closed forms where they differ (the Uint2 f32 product, the NaN rule of the
statistics) and for every scale rule.
"""
import math

import numpy as np
import pytest

from oracle import DTYPE_NAMES

UNSIGNED = {10: 1e15, 22: 1e15, 23: 1e15, 11: 4294967295.0, 12: 65535.0, 13: 255.0, 15: 15.0,
            18: 3.0, 29: 63.0, 31: 31.0, 33: 7.0}


def f32(v):
    return np.float32(v)


@pytest.mark.parametrize("dtype", range(34), ids=DTYPE_NAMES)
def test_repack_equals_pack_where_the_arithmetic_is_the_same(oracle, dtype):
    """On inputs with no NaN, every dtype's bytes and scale equal pack_native's
    (cam_div / cam_mul are the correctly rounded f32 '/' and '*'); Uint2 is
    checked element by element against its own rule in the next test."""
    rng = np.random.default_rng(dtype)
    for w in (rng.normal(0, 1, 777), rng.normal(0, 0.02, 1024), rng.uniform(-6, 6, 333),
              np.zeros(64), np.full(40, -2.5), np.array([0.0, -0.0, 1e-30, -1e30, 3.0])):
        w = w.astype(np.float32)
        a, sa = oracle.pack(dtype, w)
        b, sb = oracle.repack(dtype, w)
        assert f32(sa) == f32(sb), (DTYPE_NAMES[dtype], sa, sb)
        if dtype == 18:
            continue
        np.testing.assert_array_equal(b, a, err_msg=DTYPE_NAMES[dtype])


def _round_half_away(x):
    return np.sign(x) * np.floor(np.abs(x) + 0.5)


def test_uint2_product_is_an_f32_multiply(oracle):
    """Uint2 repack code = round(fl32(fl32((v - min) / span) * 3)), where pack
    rounds the double product.  With min 0 and span 1, r = 13981013 * 2^-24
    gives 3r = 2.5 - 2^-24 exactly: pack rounds it to 2, the f32 product is
    2.5, which rounds (half away from zero) to 3."""
    r = f32(13981013 * 2.0 ** -24)
    w = np.array([0.0, 1.0, r, 0.5, 1.0 / 6.0], np.float32)
    raw, scale = oracle.repack(18, w)
    codes = [(raw[4 + i // 4] >> (2 * (i % 4))) & 3 for i in range(w.size)]
    praw, _ = oracle.pack(18, w)
    pcodes = [(praw[4 + i // 4] >> (2 * (i % 4))) & 3 for i in range(w.size)]
    assert codes[2] == 3 and pcodes[2] == 2
    assert f32(scale) == f32(1.0) / f32(3.0)
    # every element by the closed form, on a dense sweep of ratios
    w = np.concatenate([[0.0, 1.0], np.linspace(0, 1, 20001)]).astype(np.float32)
    w = np.concatenate([w, (np.arange(13981000, 13981030) * 2.0 ** -24).astype(np.float32)])
    raw, _ = oracle.repack(18, w)
    got = np.array([(raw[4 + i // 4] >> (2 * (i % 4))) & 3 for i in range(w.size)])
    want = _round_half_away((w / np.float32(1.0)).astype(np.float32) * np.float32(3.0)).astype(int)
    np.testing.assert_array_equal(got, np.clip(want, 0, 3))


def test_statistics_skip_nan_elements(oracle):
    """Metal's min/max return the number when the other operand is NaN: a NaN
    element 0 does not become the min (pack_native's sequential compare
    keeps it: its header is NaN); with no number at all min = max = NaN."""
    w = np.array([np.nan, 1.0, 3.0, 2.0, np.nan], np.float32)
    raw, scale = oracle.repack(13, w)
    assert raw[:4].view("<f4")[0] == 1.0
    assert f32(scale) == f32(2.0) / f32(255.0)
    assert list(raw[5:8]) == [0, 255, 128]  # 1 -> 0, 3 -> 255, 2 -> round(127.5) = 128
    assert raw[4] == 0 and raw[8] == 0      # NaN elements: max(0, NaN) = 0
    praw, _ = oracle.pack(13, w)
    assert np.isnan(praw[:4].view("<f4")[0])
    raw, _ = oracle.repack(13, np.full(6, np.nan, np.float32))
    assert np.isnan(raw[:4].view("<f4")[0])
    # absmax skips NaN too: Int8 scale = fl32(max|w| / 127)
    _, scale = oracle.repack(9, np.array([np.nan, -4.0, 2.0], np.float32))
    assert f32(scale) == f32(4.0) / f32(127.0)


@pytest.mark.parametrize("dtype", range(34), ids=DTYPE_NAMES)
def test_scale_rules(oracle, dtype):
    """The scale each dtype keeps (ops_storage.metal:993-1039), computed here
    from the closed form: absmax hi (base = hi, 0 -> 1), span = max - min."""
    w = np.array([-1.5, 0.25, 3.0, -0.75, 2.0], np.float32)
    hi, mn, mx = f32(3.0), f32(-1.5), f32(3.0)
    span = mx - mn
    want = {6: hi / f32(1e6), 21: hi / f32(1e6), 7: hi / f32(2147483647.0), 8: hi / f32(32767.0),
            9: hi / f32(127.0), 14: hi / f32(7.0), 17: hi, 19: hi, 20: hi, 26: hi,
            27: hi / f32(31.0), 28: hi / f32(31.0), 30: hi / f32(15.0), 32: hi / f32(3.0)}
    want.update({d: span / f32(m) for d, m in UNSIGNED.items()})
    raw, scale = oracle.repack(dtype, w)
    assert f32(scale) == f32(want.get(dtype, 1.0)), (DTYPE_NAMES[dtype], scale)
    if dtype in UNSIGNED:
        assert raw[:4].view("<f4")[0] == mn
    # all zeros: absmax 0 -> base 1 (Int8 / Int4 / n-bit: scale 0 -> 1), span 0 -> 1
    _, scale0 = oracle.repack(dtype, np.zeros(8, np.float32))
    z = {6: f32(1) / f32(1e6), 21: f32(1) / f32(1e6), 7: f32(1) / f32(2147483647.0),
         8: f32(1) / f32(32767.0)}
    z.update({d: f32(1) / f32(m) for d, m in UNSIGNED.items()})
    assert f32(scale0) == f32(z.get(dtype, 1.0)), (DTYPE_NAMES[dtype], scale0)


def test_integer_codes_closed_form(oracle):
    """Int8: q = clamp(round-half-away(v / fl32(hi / 127)), -128, 127); Int32:
    clamp(round(fl32(v / hi) * 2^31)) saturates the +absmax element at
    2^31 - 1; NF4: the nearest table entry of v / hi, first index on ties."""
    w = np.array([127.0, -63.5, 0.5, -0.5, 1.5, 2.5], np.float32)
    raw, scale = oracle.repack(9, w)
    assert f32(scale) == f32(1.0)
    assert list(raw.view(np.int8)) == [127, -64, 1, -1, 2, 3]
    raw, _ = oracle.repack(7, np.array([2.0, -2.0, 1.0], np.float32))
    assert list(raw.view("<i4")) == [2**31 - 1, -2**31, 2**30]
    raw, scale = oracle.repack(26, np.array([-2.0, 2.0, 0.0, 1.0], np.float32))
    assert f32(scale) == f32(2.0)
    codes = [raw[0] & 15, raw[0] >> 4, raw[1] & 15, raw[1] >> 4]
    assert codes[:3] == [0, 15, 7]  # -1, +1, 0 of the NF4 table
    assert codes[3] == 12           # 0.5: nearest entry 0.4407 (code 12) vs 0.5626 (13)
