"""GPU Dense parity against the oracle: forward (GEMV, MFMA GEMM and the
element-wise route), activations with bias, backward dX/dW, MSE, and the
NormalBP leaf including the reference's packaged known-answer test."""
import json
import os

import numpy as np
import pytest

import pywelvet
from oracle import ACT, DTYPE_NAMES
from parity import assert_bit_equal, assert_close, rel_err, tol_for_k

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    pywelvet.init()


def oracle_weights(oracle, dtype, W):
    raw, scale = oracle.pack(dtype, W)
    return oracle.decode_f64(dtype, raw, scale, W.size).reshape(W.shape)


def elementwise_bound(Wd, x, rtol):
    """|dpre| <= rtol * sum_k |w x| per output: the condition-number bound."""
    return rtol * (np.abs(x.astype(np.float64)) @ np.abs(Wd).T) + 1e-30


def check_forward(oracle, dtype, W, x, act=-1, bias=None, path=0):
    pywelvet.set_forward_path(path)
    try:
        pre, post = pywelvet.forward(W, x, act=act, dtype=dtype, bias=bias)
    finally:
        pywelvet.set_forward_path(0)
    Wd = oracle_weights(oracle, dtype, W)
    rpre, rpost = oracle.forward(Wd, x, act, bias)
    k = W.shape[1]
    assert_close(pre, rpre, k, f"{DTYPE_NAMES[dtype]} pre")
    assert_close(post, rpost, k, f"{DTYPE_NAMES[dtype]} post")
    if bias is None:
        d = np.abs(pre.astype(np.float64) - rpre)
        assert np.all(d <= elementwise_bound(Wd, x, tol_for_k(k)))
    return pre, rpre


@pytest.mark.parametrize("dtype", range(34), ids=DTYPE_NAMES)
@pytest.mark.parametrize("batch", [1, 3, 8, 64])
def test_forward_all_dtypes(oracle, dtype, batch):
    rng = np.random.default_rng(dtype * 100 + batch)
    W = rng.normal(0, 0.5, (96, 256)).astype(np.float32)
    x = rng.normal(0, 1, (batch, 256)).astype(np.float32)
    check_forward(oracle, dtype, W, x)


@pytest.mark.parametrize("dtype", [1, 4, 9, 14, 26, 28, 0, 25])
@pytest.mark.parametrize("path", [1, 2, 3])
def test_forward_each_route(oracle, dtype, path):
    rng = np.random.default_rng(7 + dtype)
    W = rng.normal(0, 0.1, (70, 320)).astype(np.float32)
    x = rng.normal(0, 1, (2 if path == 1 else 5, 320)).astype(np.float32)
    check_forward(oracle, dtype, W, x, path=path)


KNOBS = [dict(), dict(bf3=0), dict(bf3_rows=0), dict(bf3_rows=2), dict(regx=0),
         dict(regx=0, bf3_rows=2), dict(bf3=0, bf3_rows=0), dict(gemv_batch=0)]


@pytest.mark.parametrize("knobs", KNOBS, ids=[",".join(f"{k}={v}" for k, v in d.items()) for d in KNOBS])
def test_forward_kernel_variants(oracle, knobs):
    """Every route the tuning knobs select gives the same parity."""
    old = {k: pywelvet.set_tuning(k, v) for k, v in knobs.items()}
    try:
        rng = np.random.default_rng(21)
        for dtype in (4, 5, 9, 16, 26, 2, 1, 0, 30):
            for out, inn, batch in ((200, 1024, 1), (96, 4096, 1), (130, 768, 40), (64, 2048, 9)):
                W = rng.normal(0, 0.1, (out, inn)).astype(np.float32)
                x = rng.normal(0, 1, (batch, inn)).astype(np.float32)
                check_forward(oracle, dtype, W, x)
            W = rng.normal(0, 1.0, (96, 512)).astype(np.float32)  # exercises every E4M3 exponent
            for batch in (1, 6):
                x = rng.normal(0, 1, (batch, 512)).astype(np.float32)
                check_forward(oracle, dtype, W, x)
                gy = rng.normal(0, 1, (batch, 96)).astype(np.float32)
                pre = rng.normal(0, 1, (batch, 96)).astype(np.float32)
                with pywelvet.Session(W, batch=batch, act=0, dtype=dtype) as s:
                    dX, dW = s.backward(x, pre, gy)
                _, rdX, rdW = oracle.backward(oracle_weights(oracle, dtype, W), x, pre, gy, 0)
                assert_close(dX, rdX, 96, "dX")
                assert_bit_equal(dW, rdW, "dW")
    finally:
        for k, v in old.items():
            pywelvet.set_tuning(k, v)


@pytest.mark.parametrize("dtype", [4, 5, 9, 16, 26])
def test_split_x_two_group_workgroups(oracle, dtype):
    """The split-x GEMM on 8-wave workgroups whose two wave groups take
    alternate k stages and add their sums through LDS at each tile's end:
    64-row tiles (batch 33-64, ragged batch included) and the 32-row tiles of
    the 4-bit kinds, K whose last stage runs past it, shares crossing tile
    boundaries, and the dX of a forward through the transposed codes (K =
    rows)."""
    rng = np.random.default_rng(1500 + dtype)
    cases = ((300, 2016, 64), (257, 1024, 48), (128, 4096, 33), (1000, 512, 64), (300, 2016, 20))
    for out, inn, batch in cases:
        W = rng.normal(0, 0.1, (out, inn)).astype(np.float32)
        if dtype == 16:
            W = rng.uniform(-6, 6, (out, inn)).astype(np.float32)
        x = rng.normal(0, 1, (batch, inn)).astype(np.float32)
        check_forward(oracle, dtype, W, x, act=2, bias=rng.normal(0, 0.1, out))
    W = rng.normal(0, 0.1, (384, 640)).astype(np.float32)
    x = rng.normal(0, 1, (40, 640)).astype(np.float32)
    gy = rng.normal(0, 1, (40, 384)).astype(np.float32)
    pre = rng.normal(0, 1, (40, 384)).astype(np.float32)
    with pywelvet.Session(W, batch=40, act=-1, dtype=dtype) as s:
        dX, dW = s.backward(x, pre, gy)
    _, rdX, rdW = oracle.backward(oracle_weights(oracle, dtype, W), x, pre, gy, -1)
    assert_close(dX, rdX, 384, "dX")
    assert_bit_equal(dW, rdW, "dW")


@pytest.mark.parametrize("dtype", [16, 26, 14, 15, 4, 5])
@pytest.mark.parametrize("cols", [8448, 11008, 8232])
def test_long_row_gemv(oracle, dtype, cols):
    """Batch-1 GEMV on long rows: three or more waves of two chunks per lane
    (the 8-rows-per-block default for 4-bit formats), NF4 at one chunk per
    lane over 5-6 waves in the loop, FP8 at two chunks per lane over 5-6
    waves; ragged row count, K just past the switch-over and not a multiple
    of the chunk."""
    rng = np.random.default_rng(1400 + dtype + cols)
    W = rng.normal(0, 0.1, (203, cols)).astype(np.float32)
    if dtype == 16:
        W = rng.uniform(-6, 6, (203, cols)).astype(np.float32)
    x = rng.normal(0, 1, (1, cols)).astype(np.float32)
    check_forward(oracle, dtype, W, x, act=1, bias=rng.normal(0, 0.1, 203))


@pytest.mark.parametrize("dtype", [4, 5, 9, 16, 26])
@pytest.mark.parametrize("batch", [5, 8, 13, 16, 17])
def test_split_x_small_batch_tile(oracle, dtype, batch):
    """The split-x GEMM's 16-row tile (16x16x32 MFMA, batch <= 16) and the
    no-split 16-row kernel that replaces it by default: ragged N (304 rows), K
    not a multiple of the 64-deep stage, forward and the dX that runs through
    the store's transposed codes."""
    rng = np.random.default_rng(1300 + 17 * dtype + batch)
    W = rng.normal(0, 0.1, (304, 1040)).astype(np.float32)
    if dtype == 16:
        W = rng.uniform(-6, 6, (304, 1040)).astype(np.float32)
    x = rng.normal(0, 1, (batch, 1040)).astype(np.float32)
    gy = rng.normal(0, 1, (batch, 304)).astype(np.float32)
    pre = rng.normal(0, 1, (batch, 304)).astype(np.float32)
    Wd = oracle_weights(oracle, dtype, W)
    _, rdX, rdW = oracle.backward(Wd, x, pre, gy, -1)
    for knobs in (dict(), dict(bf3_rows=0), dict(bf3_rows=2)):
        old = {k: pywelvet.set_tuning(k, v) for k, v in knobs.items()}
        try:
            check_forward(oracle, dtype, W, x)
            with pywelvet.Session(W, batch=batch, act=-1, dtype=dtype) as s:
                dX, dW = s.backward(x, pre, gy)
            assert_close(dX, rdX, 304, f"dX {knobs}")
            assert_bit_equal(dW, rdW, f"dW {knobs}")
        finally:
            for k, v in old.items():
                pywelvet.set_tuning(k, v)


@pytest.mark.parametrize("dtype", range(34), ids=DTYPE_NAMES)
def test_small_batch_no_split_gemm(oracle, dtype):
    """Batch <= 16 forwards on the no-split GEMM (fp32 MFMA 16x16x4 for the
    fp32-MFMA formats, the 16-row split-x GEMM for the others): ragged N (70,
    300 and 1000 rows), K of 2.5 stages (320), at the K <= 2048 bound, past
    it (4160: the fp32-MFMA formats' rule for at most 8192 outputs), a
    1024^2 layer at batch 16, a dX over 3000 rows (past 2048: the rule for
    formats without a transposed copy), bias + activation, and the same
    cases with the no-split route off and forced.  W ~ N(0, 1/K) keeps pre of order 1,
    where a saturating activation's output is compared at the scale its
    input has."""
    rng = np.random.default_rng(1700 + dtype)
    cases = [(70, 320, 5, -1), (1000, 2048, 16, 1), (1024, 1024, 16, 3), (70, 320, 13, 0),
             (300, 4160, 12, -1), (3000, 512, 12, -1)]
    for knob in (1, 0, 2):
        old = pywelvet.set_tuning("bf3_rows", knob)
        try:
            for out, inn, batch, act in cases:
                W = rng.normal(0, inn ** -0.5, (out, inn)).astype(np.float32)
                x = rng.normal(0, 1, (batch, inn)).astype(np.float32)
                if dtype == 16:  # FP4 has no scale: weights on its grid, x scaled instead
                    W = rng.uniform(-6, 6, (out, inn)).astype(np.float32)
                    x = (x / (3.5 * inn ** 0.5)).astype(np.float32)
                bias = rng.normal(0, 0.1, out) if act >= 0 else None
                check_forward(oracle, dtype, W, x, act=act, bias=bias)
                # dX through W^T on the same route family (rows = the
                # reduction length), dW bit for bit
                gy = rng.normal(0, 1, (batch, out)).astype(np.float32)
                pre = rng.normal(0, 1, (batch, out)).astype(np.float32)
                with pywelvet.Session(W, batch=batch, act=act, dtype=dtype) as s:
                    dX, dW = s.backward(x, pre, gy)
                _, rdX, rdW = oracle.backward(oracle_weights(oracle, dtype, W), x, pre, gy, act)
                assert_close(dX, rdX, out, f"{DTYPE_NAMES[dtype]} dX {out}x{inn} b{batch} rows={knob}")
                assert_bit_equal(dW, rdW, f"{DTYPE_NAMES[dtype]} dW")
        finally:
            pywelvet.set_tuning("bf3_rows", old)


@pytest.mark.parametrize("dtype", [7, 11, 17, 19, 20, 32, 6, 25])
def test_no_split_gemm_wide_outputs(oracle, dtype):
    """Batch 9-16 forwards of the formats that take the no-split fp32-MFMA
    GEMM past K = 2048 also at more than 8192 outputs (32- and 64-bit
    integers, 1- to 3-bit tables, Complex128): 8448 outputs, K = 2112
    (ragged last stage), batch 12 and 16."""
    rng = np.random.default_rng(1800 + dtype)
    W = rng.normal(0, 2112 ** -0.5, (8448, 2112)).astype(np.float32)
    for batch in (12, 16):
        x = rng.normal(0, 1, (batch, 2112)).astype(np.float32)
        check_forward(oracle, dtype, W, x)


# (dtype, rows, cols) whose batch-1 GEMV takes the fixed-grid loop with a
# partial last row group: FP8 at one chunk per lane and 4 rows per group
# (4096 inputs, 2752 groups over 1024 blocks) and at two chunks per lane
# (8192 inputs, 1025 groups over 1024 blocks), FP4 at 8 rows per group (4096
# inputs, 2501 groups over 2048 blocks), NF4 at one chunk per lane over 2
# waves (4096 inputs) and over 6 waves at 12 waves per CU (11008 inputs, 1025
# groups over 512 blocks)
LOOP_CASES = [(4, 11007, 4096), (4, 4099, 8192), (5, 11007, 4096), (16, 20003, 4096),
              (26, 11007, 4096), (26, 4097, 11008)]


@pytest.mark.parametrize("dtype,rows,cols", LOOP_CASES,
                         ids=[f"{DTYPE_NAMES[d]}-{r}x{c}" for d, r, c in LOOP_CASES])
def test_loop_gemv_ragged_rows(oracle, dtype, rows, cols):
    """The fixed-grid batch-1 GEMV (blocks walking several row groups) on
    the shapes that select it, with a partial last group."""
    rng = np.random.default_rng(29 + dtype + rows)
    if dtype == 16:
        W = rng.uniform(-6, 6, (rows, cols)).astype(np.float32)
    else:
        W = rng.normal(0, 0.05, (rows, cols)).astype(np.float32)
    x = rng.normal(0, 1, (1, cols)).astype(np.float32)
    check_forward(oracle, dtype, W, x, act=1, bias=rng.normal(0, 0.1, rows))


@pytest.mark.parametrize("dtype", [4, 26, 2, 7])
def test_batched_gemv_bias_act(oracle, dtype):
    """The batch 2-8 GEMV's epilogue: one bias per output row for every batch
    row (shorter than the outputs: rows past it take none), each activation,
    on one-wave and multi-wave rows with a partial last group."""
    rng = np.random.default_rng(53 + dtype)
    for out, inn in ((203, 4096), (37, 1024)):
        W = rng.normal(0, inn ** -0.5, (out, inn)).astype(np.float32)
        bias = rng.normal(0, 0.5, out - 5)
        for act in (0, 1, 2, 3):
            for batch in (2, 3, 6):
                x = rng.normal(0, 1, (batch, inn)).astype(np.float32)
                check_forward(oracle, dtype, W, x, act=act, bias=bias)


@pytest.mark.parametrize("dtype", [4, 5, 9, 16, 26, 1, 2, 3, 13, 8, 12, 7, 6, 17, 20, 32, 30, 27])
def test_batched_gemv(oracle, dtype):
    """Batch 2-8 through the GEMV that holds x of every batch row in
    registers: batches that fill and that pad its 2 / 4 / 8 register rows,
    rows of one wave (1024 inputs), of a partial last wave (2080), of one and
    two chunks per lane (4096, 11008), row counts that leave a partial last
    group, and three grids (8, 4 and 16 waves per CU)."""
    rng = np.random.default_rng(31 + dtype)
    old = pywelvet.set_tuning("gemv_batch", 1)
    try:
        for knob in (1, 4, 16):
            pywelvet.set_tuning("gemv_batch", knob)
            for out, inn in ((203, 4096), (37, 1024), (11, 2080), (40, 11008)):
                if dtype == 16:
                    W = rng.uniform(-6, 6, (out, inn)).astype(np.float32)
                else:
                    W = rng.normal(0, 0.1, (out, inn)).astype(np.float32)
                for batch in (2, 3, 4, 5, 8):
                    x = rng.normal(0, 1, (batch, inn)).astype(np.float32)
                    check_forward(oracle, dtype, W, x)
    finally:
        pywelvet.set_tuning("gemv_batch", old)


@pytest.mark.parametrize("dtype", [1, 2, 4, 9, 16, 26, 27, 33])
def test_forward_ragged_shapes(oracle, dtype):
    """Columns that are not a whole number of chunks take the element-wise route."""
    rng = np.random.default_rng(11)
    for out, inn, batch in ((5, 97, 1), (1, 1, 1), (3, 33, 7), (17, 250, 2)):
        W = rng.normal(0, 0.3, (out, inn)).astype(np.float32)
        x = rng.normal(0, 1, (batch, inn)).astype(np.float32)
        check_forward(oracle, dtype, W, x)


@pytest.mark.parametrize("act", list(ACT.values()) + [42], ids=list(ACT) + ["unknown"])
def test_activations_with_bias(oracle, act):
    rng = np.random.default_rng(5)
    W = rng.normal(0, 0.2, (64, 128)).astype(np.float32)
    x = rng.normal(0, 2, (4, 128)).astype(np.float32)
    bias = rng.normal(0, 1, 40)  # shorter than out: bias only for o < 40
    for batch in (1, 4, 9):
        xb = np.resize(x, (batch, 128)).astype(np.float32)
        check_forward(oracle, 1, W, xb, act=act, bias=bias)
        check_forward(oracle, 26, W, xb, act=act, bias=bias)


@pytest.mark.parametrize("dtype,batch", [(4, 1), (26, 1), (4, 64), (26, 64), (16, 1), (16, 8),
                                         (16, 64), (5, 32)])
def test_forward_headline_shapes(oracle, dtype, batch):
    """4096 -> 11008 and 11008 -> 4096 (the LLM-MLP pair) with N(0, 0.02)
    weights; FP4 (no scale: N(0, 0.02) would encode every weight to code 0)
    with U(-6, 6), which spans its whole grid."""
    rng = np.random.default_rng(0x5EED0003 + batch)
    for out, inn in ((11008, 4096), (4096, 11008)):
        if dtype == 16:
            W = rng.uniform(-6, 6, (out, inn)).astype(np.float32)
        else:
            W = rng.normal(0, 0.02, (out, inn)).astype(np.float32)
        x = rng.normal(0, 1, (batch, inn)).astype(np.float32)
        check_forward(oracle, dtype, W, x)


@pytest.mark.parametrize("batch", [1, 8, 40])
def test_e5m2_nonfinite_weights(oracle, batch):
    """E5M2 stores Inf for values past its range and a NaN code for NaN
    (float_codecs.cpp:119-158): the products keep IEEE results (the split-x
    GEMM, which cannot carry Inf * x exactly, is not used for such a store);
    finite outputs within tolerance, non-finite ones identical in class."""
    rng = np.random.default_rng(77 + batch)
    W = rng.normal(0, 0.1, (70, 256)).astype(np.float32)
    W[3, 5], W[10, 200], W[40, 7] = 1e6, -1e6, np.nan
    x = rng.normal(0, 1, (batch, 256)).astype(np.float32)
    pre, _ = pywelvet.forward(W, x, act=-1, dtype=5)
    rpre, _ = oracle.forward(oracle_weights(oracle, 5, W), x, -1, None)
    fin = np.isfinite(rpre)
    assert not fin.all()
    np.testing.assert_array_equal(np.isnan(pre), np.isnan(rpre))
    np.testing.assert_array_equal(np.where(np.isinf(rpre), pre, 0), np.where(np.isinf(rpre), rpre, 0))
    assert_close(np.where(fin, pre, 0), np.where(fin, rpre, 0), 256, "finite outputs")


@pytest.mark.parametrize("shape", [(96, 512), (96, 2560)])
@pytest.mark.parametrize("batch", [1, 3, 8, 40, 64])
@pytest.mark.parametrize("dtype", [4, 26, 16, 9], ids=lambda d: DTYPE_NAMES[d])
def test_nonfinite_inputs(oracle, dtype, batch, shape):
    """Inf and NaN inputs through every forward route (GEMV, the split-x
    GEMMs with and without a k split): NaN and Inf outputs where the f64
    reference has them, with the same signs, including a NaN whose payload
    sits only in the low 16 bits (its leading bf16 part reads as an
    infinity); finite outputs within tolerance."""
    rng = np.random.default_rng(1700 + dtype + batch + shape[1])
    out, inn = shape
    W = rng.normal(0, 0.1, (out, inn)).astype(np.float32)
    if dtype == 16:
        W = rng.uniform(-6, 6, (out, inn)).astype(np.float32)
    x = rng.normal(0, 1, (batch, inn)).astype(np.float32)
    low_nan = np.array([0x7F800001], np.uint32).view(np.float32)[0]
    planted = [np.inf, -np.inf, np.nan, low_nan]
    for i, v in enumerate(planted):
        if i < batch:
            x[i, (37 * i + 5) % inn] = v
    Wd = oracle_weights(oracle, dtype, W)
    pre, _ = pywelvet.forward(W, x, act=-1, dtype=dtype)
    rpre, _ = oracle.forward(Wd, x, -1, None)
    assert not np.all(np.isfinite(rpre))
    np.testing.assert_array_equal(np.isnan(pre), np.isnan(rpre))
    inf = np.isinf(rpre)
    np.testing.assert_array_equal(np.where(inf, pre, 0), np.where(inf, rpre, 0))
    fin = np.isfinite(rpre)
    assert_close(np.where(fin, pre, 0), np.where(fin, rpre, 0), inn, "finite outputs")


@pytest.mark.parametrize("batch", [5, 40])
def test_backward_e5m2_nonfinite_weights(oracle, batch):
    """dX through an E5M2 store holding Inf and NaN codes keeps the IEEE
    products (the transposed split-x route is not used for it); dW does not
    depend on the weights and stays bit-identical."""
    rng = np.random.default_rng(91 + batch)
    out, inn = 96, 160
    W = rng.normal(0, 0.2, (out, inn)).astype(np.float32)
    W[4, 9], W[50, 100], W[70, 3] = 1e6, -1e6, np.nan
    x = rng.normal(0, 1, (batch, inn)).astype(np.float32)
    gy = rng.normal(0, 1, (batch, out)).astype(np.float32)
    pre = rng.normal(0, 1, (batch, out)).astype(np.float32)
    with pywelvet.Session(W, batch=batch, act=-1, dtype=5) as s:
        dX, dW = s.backward(x, pre, gy)
    _, rdX, rdW = oracle.backward(oracle_weights(oracle, 5, W), x, pre, gy, -1)
    fin = np.isfinite(rdX)
    assert not fin.all()
    np.testing.assert_array_equal(np.isnan(dX), np.isnan(rdX))
    np.testing.assert_array_equal(np.where(np.isinf(rdX), dX, 0), np.where(np.isinf(rdX), rdX, 0))
    assert_close(np.where(fin, dX, 0), np.where(fin, rdX, 0), out, "finite dX")
    assert_bit_equal(dW, rdW, "dW")


def test_session_reuse(oracle):
    rng = np.random.default_rng(3)
    W = rng.normal(0, 0.02, (300, 512)).astype(np.float32)
    Wd = oracle_weights(oracle, 4, W)
    with pywelvet.Session(W, batch=2, act=3, dtype=4) as s:
        for i in range(3):
            x = rng.normal(0, 1, (2, 512)).astype(np.float32)
            pre, post = s.execute(x)
            rpre, rpost = oracle.forward(Wd, x, 3)
            assert_close(post, rpost, 512, f"iter {i}")


@pytest.mark.parametrize("dtype", [4, 5])
@pytest.mark.parametrize("batch", [1, 8, 64])
def test_forward_after_sgd_reads_updated_store(oracle, dtype, batch):
    """FP8 kernels decode the store's decode-ready copy: after an SGD step
    (which rewrites both) the forward must match the oracle on the exported
    weights, including codes the update moved into or out of the subnormal
    range (decoded as signed zero)."""
    rng = np.random.default_rng(40 + dtype + batch)
    out, inn = 260, 1024
    W = rng.normal(0, 0.02, (out, inn)).astype(np.float32)
    with pywelvet.Session(W, batch=batch, act=-1, dtype=dtype) as s:
        for step in range(2):
            g = rng.normal(0, 1, (out, inn)).astype(np.float32)
            s.sgd(g, 5e-3)
            Wd = s.export_f32().astype(np.float64)
            x = rng.normal(0, 1, (batch, inn)).astype(np.float32)
            pre, _ = s.execute(x)
            rpre, _ = oracle.forward(Wd, x, -1)
            assert_close(pre, rpre, inn, f"{DTYPE_NAMES[dtype]} step {step}")


def assert_same_nonfinite(got, want, k, label):
    """NaN where want has NaN, the same infinities, finite values within the
    tolerance for a length-k reduction."""
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want), err_msg=f"{label} NaN")
    inf = np.isinf(want)
    np.testing.assert_array_equal(np.where(inf, got, 0), np.where(inf, want, 0), err_msg=f"{label} Inf")
    fin = np.isfinite(want)
    assert_close(np.where(fin, got, 0), np.where(fin, want, 0), k, f"{label} finite")


@pytest.mark.parametrize("batch", [8, 40])
def test_e5m2_finiteness_follows_sgd(oracle, batch):
    """An E5M2 store's Inf / NaN status is re-read from the codes each SGD
    writes: an update that stays finite keeps the store on the split-x GEMM,
    one that pushes weights past the format's range (Inf codes) moves the
    forward and dX off it.  Each matches the oracle on the exported weights,
    non-finite outputs identical in class; dW bit for bit."""
    rng = np.random.default_rng(4100 + batch)
    out, inn = 96, 512
    W = rng.normal(0, 0.05, (out, inn)).astype(np.float32)
    with pywelvet.Session(W, batch=batch, act=-1, dtype=5) as s:
        for step in range(2):
            g = rng.normal(0, 1, (out, inn)).astype(np.float32)
            if step == 1:
                g[5, 17], g[60, 300] = -1e9, 1e9  # lr * g = -+1e6, past E5M2's range
            s.sgd(g, 1e-3)
            Wd = s.export_f32().astype(np.float64)
            assert bool(np.isfinite(Wd).all()) == (step == 0)
            x = rng.normal(0, 1, (batch, inn)).astype(np.float32)
            pre, _ = s.execute(x)
            rpre, _ = oracle.forward(Wd, x, -1)
            assert_same_nonfinite(pre, rpre, inn, f"forward step {step}")
            gy = rng.normal(0, 1, (batch, out)).astype(np.float32)
            bpre = rng.normal(0, 1, (batch, out)).astype(np.float32)
            dX, dW = s.backward(x, bpre, gy)
            _, rdX, rdW = oracle.backward(Wd, x, bpre, gy, -1)
            assert_same_nonfinite(dX, rdX, out, f"dX step {step}")
            assert_bit_equal(dW, rdW, f"dW step {step}")


@pytest.mark.parametrize("dtype", [4, 26, 1])
def test_gemm_session_repeat(oracle, dtype):
    """Repeated MFMA launches on one session reuse its stream-K workspace:
    every later forward and dX must come out right."""
    rng = np.random.default_rng(17 + dtype)
    out, inn, batch = 1500, 2048, 48
    W = rng.normal(0, 0.05, (out, inn)).astype(np.float32)
    Wd = oracle_weights(oracle, dtype, W)
    bias = rng.normal(0, 1, out)
    with pywelvet.Session(W, batch=batch, act=1, dtype=dtype, bias=bias) as s:
        for i in range(4):
            x = rng.normal(0, 1, (batch, inn)).astype(np.float32)
            pre, post = s.execute(x)
            rpre, rpost = oracle.forward(Wd, x, 1, bias)
            assert_close(pre, rpre, inn, f"pre iter {i}")
            assert_close(post, rpost, inn, f"post iter {i}")
            gy = rng.normal(0, 1, (batch, out)).astype(np.float32)
            dX, dW = s.backward(x, pre, gy)
            _, rdX, rdW = oracle.backward(Wd, x, pre, gy, 1)
            assert_close(dX, rdX, out, f"dX iter {i}")
            assert_bit_equal(dW, rdW, f"dW iter {i}")


@pytest.mark.parametrize("dtype", [1, 0, 4, 5, 9, 26, 14, 12, 27, 20, 16])
@pytest.mark.parametrize("batch", [1, 2, 5, 40])
def test_backward(oracle, dtype, batch):
    """dX within tolerance of the f64 contract; dW bit-identical (sequential
    fmaf over the batch, welvet_dense.metal:155-178)."""
    rng = np.random.default_rng(dtype + 31 * batch)
    out, inn = 160, 256
    W = rng.normal(0, 0.3, (out, inn)).astype(np.float32)
    x = rng.normal(0, 1, (batch, inn)).astype(np.float32)
    gy = rng.normal(0, 1, (batch, out)).astype(np.float32)
    pre = rng.normal(0, 1, (batch, out)).astype(np.float32)
    for act in (-1, 0, 3):
        with pywelvet.Session(W, batch=batch, act=act, dtype=dtype) as s:
            dX, dW = s.backward(x, pre, gy)
        Wd = oracle_weights(oracle, dtype, W)
        dpre, rdX, rdW = oracle.backward(Wd, x, pre, gy, act)
        assert_close(dX, rdX, out, f"dX act={act}")
        assert_bit_equal(dW, rdW, f"dW act={act}")


@pytest.mark.parametrize("shape", [(70, 130), (256, 384)], ids=["ragged", "tiled"])
@pytest.mark.parametrize("batch", [1, 2, 3, 7, 64, 65])
def test_dw_bit_exact_special_values(oracle, batch, shape):
    """dW stays the reference's sequential fmaf over the batch, bit for bit,
    on both dW kernels (LDS-staged MFMA for whole 128-tiles, direct MFMA for
    ragged shapes), with signed zeros
    (ReLU passes -0 gradients), denormal inputs and products across the
    exponent range, odd and even batches, ragged and whole 128-tiles."""
    rng = np.random.default_rng(131 + batch)
    out, inn = shape
    W = rng.normal(0, 0.3, (out, inn)).astype(np.float32)
    x = rng.normal(0, 1, (batch, inn)).astype(np.float32)
    x[:, ::7] = -0.0
    x[:, 3::11] = np.float32(1e-40) * np.sign(x[:, 3::11] + 0.5)
    x[:, 5::13] *= np.float32(1e25)
    gy = rng.normal(0, 1, (batch, out)).astype(np.float32)
    gy[:, ::5] = -0.0
    gy[:, 2::9] *= np.float32(1e-25)
    pre = rng.normal(0, 1, (batch, out)).astype(np.float32)
    Wd = oracle_weights(oracle, 1, W)
    for act in (-1, 0):
        with pywelvet.Session(W, batch=batch, act=act, dtype=1) as s:
            _, dW = s.backward(x, pre, gy)
        _, _, rdW = oracle.backward(Wd, x, pre, gy, act)
        assert_bit_equal(dW, rdW, f"dW act={act}")


def test_backward_ragged(oracle):
    rng = np.random.default_rng(9)
    W = rng.normal(0, 0.3, (13, 45)).astype(np.float32)
    x = rng.normal(0, 1, (3, 45)).astype(np.float32)
    gy = rng.normal(0, 1, (3, 13)).astype(np.float32)
    pre = rng.normal(0, 1, (3, 13)).astype(np.float32)
    for dtype in (1, 9, 26, 32):
        with pywelvet.Session(W, batch=3, act=1, dtype=dtype) as s:
            dX, dW = s.backward(x, pre, gy)
        _, rdX, rdW = oracle.backward(oracle_weights(oracle, dtype, W), x, pre, gy, 1)
        assert_close(dX, rdX, 13)
        assert_bit_equal(dW, rdW, "dW")


def test_mse(oracle):
    rng = np.random.default_rng(4)
    for n in (1, 2, 1000, 262144 + 7):
        p = rng.normal(0, 1, n).astype(np.float32)
        t = rng.normal(0, 1, n).astype(np.float32)
        loss, g = pywelvet.mse(p, t)
        rl = oracle.mse(p, t)
        assert abs(loss - rl) <= 1e-12 * max(1.0, abs(rl))
        assert_bit_equal(g, oracle.mse_grad(p, t), "mse grad")


def test_release_smoke_kat(golden_dir):
    """scripts/release_smoke.py:45-55 through the C ABI."""
    k = json.load(open(os.path.join(golden_dir, "release_kat.json")))
    W = np.array(k["W_init"], np.float32).reshape(2, 2)
    x = np.array(k["x"], np.float32).reshape(1, 2)
    pre, post = pywelvet.forward(W, x, act=-1, dtype=1)
    assert list(post.ravel()) == k["expect_post"]
    r = pywelvet.normalbp(W, x, np.array(k["target"], np.float32).reshape(1, 2), 1, k["lr"])
    assert abs(r["loss"] - k["expect_loss"]) < k["tolerance"]
    assert np.all(np.abs(r["W_after"].ravel() - np.array(k["expect_W_after"])) < k["tolerance"])


@pytest.mark.parametrize("dtype", [1, 0, 2, 3, 4, 5, 9, 13, 14, 16, 26, 19, 28, 7])
def test_normalbp_matches_oracle(oracle, dtype):
    rng = np.random.default_rng(77 + dtype)
    for batch, out, inn, act, use_target, lr in ((1, 64, 128, 3, 1, 1e-2), (6, 40, 96, 0, 0, 0.1),
                                                 (3, 24, 97, 2, 1, 0.0)):
        W = rng.normal(0, 0.3, (out, inn)).astype(np.float32)
        x = rng.normal(0, 1, (batch, inn)).astype(np.float32)
        t = rng.normal(0, 1, (batch, out)).astype(np.float32)
        bias = rng.normal(0, 0.1, out)
        r = pywelvet.normalbp(W, x, t, use_target, lr, act=act, dtype=dtype, bias=bias)
        o = oracle.normalbp(batch, inn, out, act, dtype, W, x, t, use_target, lr, bias=bias)
        assert o["status"] == 0
        for key in ("pre", "post", "dX", "dW"):
            assert rel_err(r[key], o[key]) <= 1e-5, (key, rel_err(r[key], o[key]))
        assert abs(r["loss"] - o["loss"]) <= 1e-5 * max(1.0, abs(o["loss"]))
        # W_after: decode of the re-encoded store; tiny dW differences may move
        # a value across one quantisation boundary, never further
        diff = np.abs(r["W_after"].astype(np.float64) - o["W_after"])
        step = np.max(np.abs(np.diff(np.unique(o["W_after"])))) if np.unique(o["W_after"]).size > 1 else 0
        assert np.mean(diff > 0) <= 0.01 and (diff.max() <= step + 1e-6 or diff.max() <= 1e-5)


def test_normalbp_error_codes():
    W = np.ones((2, 2), np.float32)
    x = np.ones((1, 2), np.float32)
    g = np.array([[np.inf, 0]], np.float32)
    r = pywelvet.normalbp(W, x, g, 0, 0.1, dtype=9, status=True)
    assert r["status"].code == 1  # nonfinite gradient on the native path
    r = pywelvet.normalbp(W, x, g, 0, 0.1, dtype=1, status=True)
    assert r["status"].code == 2  # Float32 path: training.mm:122-124
    r = pywelvet.normalbp(W, x, np.zeros((1, 2), np.float32), 0, float("inf"), dtype=9, status=True)
    assert r["status"].code == 1
    r = pywelvet.normalbp(W, x, np.zeros((1, 2), np.float32), 1, 0.0, dtype=9)
    assert r["loss"] >= 0


def test_read_probe():
    """welvet_hip_probe_read (the bench's single-launch read floor) streams a
    buffer without writing the sink in practice, and refuses misaligned or
    ragged arguments with code 1."""
    from devmem import DeviceArray, Stream

    buf = DeviceArray((1 << 20,), fill=1.0)   # 4 MiB
    sink = DeviceArray((1024,), fill=0.0)
    st = Stream()
    try:
        pywelvet.probe_read(buf.ptr, buf.nbytes, sink.ptr, st.h)
        pywelvet.probe_read(buf.ptr, 48, sink.ptr, st.h)   # less than one block
        st.sync()
        assert np.all(sink.download() == 0.0)
        for args in ((buf.ptr + 4, 1024), (buf.ptr, 1000), (buf.ptr, 0)):
            s = pywelvet.lib().welvet_hip_probe_read(pywelvet.C.c_void_p(args[0]), pywelvet.C.c_uint64(args[1]),
                                                     pywelvet.C.c_void_p(sink.ptr), pywelvet.C.c_void_p(st.h))
            assert s.code == 1, args
    finally:
        st.close()
        buf.free()
        sink.free()
