"""Exhaustive GPU codec checks against the reference's scalar codecs.

* Every code of FP8 E4M3 / E5M2 (256), FP4 / NF4 (16) and F16 / BF16 (65536)
  decoded by the export path and by each forward route's own decode (GEMV
  kernels, the batch 2-4 kernel, the split-x bf16 GEMM, the fp32 MFMA GEMMs,
  the element-wise kernel and the FP8 dX through the transposed codes), with
  one-hot inputs so every output is one decoded weight.  Stores are mounted
  from native bytes (welvet_hip_dense_mount_native), so each code is present
  exactly as written.  Expected values: tests/golden/scalar_tables.npz (the
  reference build's decode of every code) and, for NF4, kNf4[c] * scale in
  fp32 (native_codec.cpp:93-110, :562-813).
* The device encoders (pack) over every 4099th f32 bit pattern against the
  oracle's scalar encoders (float_codecs.cpp:23-200), which the CPU suite pins
  to the reference build; WELVET_FULL_SWEEP=1 sweeps all 2^32 patterns.
* The element-0 probe of the native SGD (ops_storage.metal:941-945): an F16
  subnormal at element 0 is flushed by the probe before its update.
"""
import os
import sys

import numpy as np
import pytest

import pywelvet
from oracle import DTYPE_NAMES
from parity import assert_bit_equal, bits

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
TABLES = np.load(os.path.join(HERE, "golden", "scalar_tables.npz"))
NF4_SCALE = np.float32(0.3712)


@pytest.fixture(scope="module", autouse=True)
def device():
    pywelvet.init()


def say(*a):
    print(*a, file=sys.stderr, flush=True)


# dtype -> (bits, number of codes, reference decode of every code)
def code_table(dtype):
    if dtype == 4:
        return 8, TABLES["e4m3_decode"]
    if dtype == 5:
        return 8, TABLES["e5m2_decode"]
    if dtype == 16:
        return 4, TABLES["fp4_decode"]
    if dtype == 26:
        kNf4 = np.array([-1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
                         -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
                         0.07958029955625534, 0.16093020141124725, 0.24611230194568634,
                         0.33791524171829224, 0.44070982933044434, 0.5626170039176941,
                         0.7229568362236023, 1.0], np.float32)
        return 4, (kNf4 * NF4_SCALE).astype(np.float32)
    if dtype == 2:
        return 16, TABLES["f16_decode"]
    if dtype == 3:
        return 16, TABLES["bf16_decode"]
    raise ValueError(dtype)


def native_bytes(dtype, codes):
    """The reference byte layout of a flat code array (LSB-first nibbles)."""
    b, _ = code_table(dtype)
    codes = np.asarray(codes)
    if b == 8:
        return codes.astype(np.uint8)
    if b == 16:
        return codes.astype("<u2").view(np.uint8)
    assert codes.size % 2 == 0
    c = codes.astype(np.uint8)
    return (c[0::2] | (c[1::2] << 4)).astype(np.uint8)


def scale_of(dtype):
    return float(NF4_SCALE) if dtype == 26 else 1.0


def test_nf4_table_matches_the_oracle(oracle):
    """The NF4 values above are the oracle's decode (pinned to the reference
    build's vectors) of every code at this scale."""
    _, want = code_table(26)
    got = oracle.decode(26, native_bytes(26, np.arange(16)), float(NF4_SCALE), 16)
    assert_bit_equal(got, want, "nf4 table")


@pytest.mark.parametrize("dtype", [4, 5, 16, 26, 2, 3], ids=lambda d: DTYPE_NAMES[d])
def test_export_decodes_every_code(oracle, dtype):
    b, table = code_table(dtype)
    codes = np.arange(table.size)
    cols = 256 if table.size >= 256 else 16
    raw = native_bytes(dtype, codes)
    with pywelvet.Session((table.size // cols, cols), batch=1, dtype=dtype,
                          native=(raw, scale_of(dtype))) as s:
        dec = s.export_f32().ravel()
        back, _ = s.native()
    assert_bit_equal(back, raw, "native bytes round trip")
    assert_bit_equal(dec, table, f"{DTYPE_NAMES[dtype]} export decode")
    assert_bit_equal(oracle.decode(dtype, raw, scale_of(dtype), table.size), table, "oracle")


# Knob sets that route the forward through each decode: the default kernels
# (hardware FP8 / FP4 converts, the byte-pair NF4 table, the split-x GEMM),
# the k-split GEMMs that default to the no-split ones at these shapes, the
# fp32 MFMA GEMMs and the element-wise kernel.
ROUTES = {
    "default": {},
    "k_split": dict(bf3_rows=0),
    "no_split_x": dict(bf3=0),
    "no_split_x_k_split": dict(bf3=0, bf3_rows=0),
    "elementwise": "path3",
}


def finite_codes(table):
    return np.nonzero(np.isfinite(table))[0]


def run_forward(dtype, raw, shape, x, route):
    knobs = ROUTES[route]
    old = {}
    if knobs == "path3":
        pywelvet.set_forward_path(3)
    else:
        old = {k: pywelvet.set_tuning(k, v) for k, v in knobs.items()}
    try:
        with pywelvet.Session(shape, batch=x.shape[0], dtype=dtype,
                              native=(raw, scale_of(dtype))) as s:
            pre, _ = s.execute(x)
    finally:
        pywelvet.set_forward_path(0)
        for k, v in old.items():
            pywelvet.set_tuning(k, v)
    return pre


@pytest.mark.parametrize("route", list(ROUTES))
@pytest.mark.parametrize("batch", [1, 3, 8, 40])
@pytest.mark.parametrize("dtype", [4, 5, 16, 26, 2, 3], ids=lambda d: DTYPE_NAMES[d])
def test_forward_decodes_every_code(dtype, batch, route):
    """Row o holds F[(o + k) mod |F|] over the finite codes F; x row b is
    one-hot at column j_b, so pre[b][o] = decode(F[(o + j_b) mod |F|]) exactly
    (one product of 1.0, every other term an exact zero), which puts every
    finite code through the route's decode at several lane and chunk
    positions."""
    _, table = code_table(dtype)
    F = finite_codes(table)
    cols = 256
    rows = F.size
    k = np.arange(cols)
    codes = F[(np.arange(rows)[:, None] + k[None, :]) % F.size]
    raw = native_bytes(dtype, codes.ravel())
    js = [(0, 1, 2, 3, 5, 17, 100, 255)[b % 8] + 8 * (b // 8) for b in range(batch)]
    js = [j % cols for j in js]
    x = np.zeros((batch, cols), np.float32)
    x[np.arange(batch), js] = 1.0
    say(f"forward every code: {DTYPE_NAMES[dtype]} b{batch} {route} ({rows}x{cols})")
    pre = run_forward(dtype, raw, (rows, cols), x, route)
    want = np.stack([table[F[(np.arange(rows) + j) % F.size]] for j in js])
    want = np.where(want == 0, np.float32(0.0), want)  # +0 + (-0 * 1) sums to +0
    assert_bit_equal(pre, want.astype(np.float32), f"{DTYPE_NAMES[dtype]} b{batch} {route}")


@pytest.mark.parametrize("route", ["default", "no_split_x", "elementwise"])
@pytest.mark.parametrize("batch", [1, 8])
@pytest.mark.parametrize("dtype", [5, 2, 3], ids=lambda d: DTYPE_NAMES[d])
def test_forward_decodes_nonfinite_codes(dtype, batch, route):
    """Inf and NaN codes, each alone in its row at column j0 (every other
    weight code 0, every other x 0), so pre = decode(code) * 1: +-Inf exactly,
    NaN as NaN."""
    _, table = code_table(dtype)
    NF = np.nonzero(~np.isfinite(table))[0]
    cols, j0 = 64, 37
    codes = np.zeros((NF.size, cols), np.int64)
    codes[:, j0] = NF
    raw = native_bytes(dtype, codes.ravel())
    x = np.zeros((batch, cols), np.float32)
    x[:, j0] = 1.0
    pre = run_forward(dtype, raw, (NF.size, cols), x, route)
    want = np.broadcast_to(table[NF], pre.shape)
    np.testing.assert_array_equal(np.isnan(pre), np.isnan(want))
    inf = np.isinf(want)
    np.testing.assert_array_equal(pre[inf], want[inf])


@pytest.mark.parametrize("batch", [1, 2, 3, 8, 40])
@pytest.mark.parametrize("dtype", [4, 5], ids=lambda d: DTYPE_NAMES[d])
def test_dx_decodes_every_code(dtype, batch):
    """dX = dpre W with one-hot dpre (Linear): dX[b] = decoded row o_b, whose
    256 columns hold every finite code; batches > 2 read the store's
    transposed codes on the split-x GEMM."""
    _, table = code_table(dtype)
    F = finite_codes(table)
    rows, cols = 272, 256
    codes = F[(np.arange(rows)[:, None] + np.arange(cols)[None, :]) % F.size]
    raw = native_bytes(dtype, codes.ravel())
    o = [(7 * b + 3) % rows for b in range(batch)]
    gy = np.zeros((batch, rows), np.float32)
    gy[np.arange(batch), o] = 1.0
    x = np.zeros((batch, cols), np.float32)
    pre = np.zeros((batch, rows), np.float32)
    with pywelvet.Session((rows, cols), batch=batch, act=-1, dtype=dtype, native=(raw, 1.0)) as s:
        dX, _ = s.backward(x, pre, gy)
    want = np.stack([table[codes[ob]] for ob in o])
    want = np.where(want == 0, np.float32(0.0), want)
    assert_bit_equal(dX, want.astype(np.float32), f"{DTYPE_NAMES[dtype]} dX b{batch}")


# ---------------------------------------------------------- encoder sweep
SWEEP_KINDS = {2: 0, 3: 1, 4: 2, 5: 3, 16: 4}  # dtype -> or_encode_many kind


def sweep_inputs(start, stop, step):
    return np.arange(start, stop, step, dtype=np.uint64).astype(np.uint32).view(np.float32)


def device_codes(dtype, values):
    """Native codes the device pack writes for `values` (no scale for these formats)."""
    n = values.size
    pad = (-n) % 2
    w = np.concatenate([values, np.zeros(pad, np.float32)]).reshape(1, -1)
    with pywelvet.Session(w, batch=1, dtype=dtype) as s:
        raw, scale = s.native()
    assert scale == 1.0
    if dtype in (2, 3):
        return raw.view("<u2")[:n]
    if dtype == 16:
        return np.stack([raw & 15, raw >> 4], axis=1).ravel()[:n]
    return raw[:n]


@pytest.mark.parametrize("dtype", list(SWEEP_KINDS), ids=lambda d: DTYPE_NAMES[d])
def test_device_encoder_bit_pattern_sweep(oracle, dtype):
    """Every 4099th f32 bit pattern (NaN, Inf, subnormals and both signs
    included): the device pack equals the scalar encoder bit for bit."""
    full = os.environ.get("WELVET_FULL_SWEEP") == "1"
    step, chunk = (1, 1 << 26) if full else (4099, 1 << 32)
    for start in range(0, 1 << 32, chunk):
        v = sweep_inputs(start, min(start + chunk, 1 << 32), step)
        got = device_codes(dtype, v)
        want = oracle.encode_many(SWEEP_KINDS[dtype], v)
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, (DTYPE_NAMES[dtype], bad[:5], bits(v[bad[:5]]), got[bad[:5]], want[bad[:5]])
    say(f"encoder sweep {DTYPE_NAMES[dtype]}: {'all 2^32' if full else 'every 4099th'} patterns")


@pytest.mark.parametrize("dtype", list(SWEEP_KINDS), ids=lambda d: DTYPE_NAMES[d])
def test_device_encoder_reference_edge_set(dtype):
    """The reference build's own encodes of the 8295-input edge set."""
    name = {2: "f16", 3: "bf16", 4: "e4m3", 5: "e5m2", 16: "fp4"}[dtype]
    v = TABLES["encode_input"]
    got = device_codes(dtype, v)
    assert_bit_equal(got.astype(TABLES[f"{name}_encode"].dtype), TABLES[f"{name}_encode"], name)


# ------------------------------------------------------- SGD element-0 probe
def test_sgd_probe_flushes_f16_subnormal_element0(oracle):
    """op_native_sgd decodes and re-encodes element 0 once before the update
    (ops_storage.metal:941-945).  F16 encode flushes subnormals, so a
    subnormal element 0 (0x0200 = 2^-15) enters its update as 0: with
    lr * g = -2^-14 it becomes 2^-14 (code 0x0400), where an update of the
    stored value would give 1.5 * 2^-14 (code 0x0600).  Element 1 holds the
    same subnormal and takes the update from its stored value, whose result
    also re-encodes exactly (0x0600)."""
    n = 8
    codes = np.array([0x0200, 0x0200, 0x3C00, 0xBC00, 0x0001, 0x4000, 0x0000, 0x8000], np.uint16)
    raw = codes.astype("<u2").view(np.uint8).copy()
    g = np.zeros(n, np.float32)
    g[0] = g[1] = -np.float32(2.0 ** -13)
    lr = 0.5
    with pywelvet.Session((1, n), batch=1, dtype=2, native=(raw, 1.0)) as s:
        s.sgd(g.reshape(1, n), lr)
        got, _ = s.native()
    want = raw.copy()
    assert oracle.native_sgd(2, want, 1.0, n, g, lr) == 0
    assert_bit_equal(got, want, "f16 sgd bytes")
    got16 = got.view("<u2")
    assert got16[0] == 0x0400 and got16[1] == 0x0600, [hex(c) for c in got16[:2]]
    # element 4 (the smallest subnormal, g = 0) flushes to +0 on re-encode
    assert got16[4] == 0x0000
