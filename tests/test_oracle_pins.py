"""Pins for the oracle functions the reference's golden vectors do not reach:
the Dense forward/backward contract, activations, fixed-scale re-encode,
SGD and MSE.  Each expectation is computed a different way than the oracle
computes it: exact rational arithmetic with an explicit round-to-nearest-even
to f32, integer arithmetic on dyadic inputs (where every summation order is
exact), textbook formulas, finite differences and structural invariants.
"""
import math
from fractions import Fraction

import numpy as np
import pytest

from oracle import ACT, DTYPE_NAMES


def rnd32(q: Fraction) -> np.float32:
    """Round an exact rational to the nearest f32, ties to even (normal range)."""
    if q == 0:
        return np.float32(0.0)
    sign = -1 if q < 0 else 1
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    assert -126 <= e <= 127, "outside the f32 normal range"
    ulp = Fraction(2) ** (e - 23)
    n = a / ulp
    fl = n.numerator // n.denominator
    rem = n - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return np.float32(sign * float(fl * ulp))


def F(v) -> Fraction:
    return Fraction(float(v))


def test_rnd32_helper():
    assert rnd32(Fraction(1) + Fraction(1, 2**24)) == np.float32(1.0)  # tie -> even
    assert rnd32(Fraction(1) + Fraction(3, 2**24)) == np.float32(1.0 + 2**-22)
    for v in np.random.default_rng(0).normal(0, 100, 200).astype(np.float32):
        assert rnd32(F(v)) == v


# ---------------------------------------------------------------- forward
def test_forward_dyadic_brute_force(oracle):
    """Dyadic W, x, bias: every partial sum is exact, so pre must equal the
    integer product exactly; a transposed operand, a dropped bias or a wrong
    index changes the result."""
    rng = np.random.default_rng(1)
    for out, inn, batch in ((3, 5, 2), (7, 16, 3), (1, 1, 1), (12, 33, 4)):
        Wi = rng.integers(-16, 17, (out, inn))
        xi = rng.integers(-16, 17, (batch, inn))
        bi = rng.integers(-64, 65, out)
        W = Wi / 8.0
        x = (xi / 4.0).astype(np.float32)
        bias = bi / 32.0
        blen = max(1, out - 1)  # the last output gets no bias
        exact = (xi @ Wi.T).astype(np.int64)  # in units of 1/32
        for act in (-1, 0, 5, 6):
            pre, post = oracle.forward(W, x, act, bias[:blen])
            want = exact.astype(np.float64) / 32.0
            want[:, :blen] += bias[:blen]
            np.testing.assert_array_equal(pre, want.astype(np.float32))
            v = pre.astype(np.float64)
            ref = {-1: v, 0: np.where(v > 0, v, 0.0), 5: np.where(v < 0, v * 0.01, v),
                   6: np.where(v < 0, 0.0, v * v)}[act]
            np.testing.assert_array_equal(post, ref.astype(np.float32))


def test_forward_rounds_an_f64_sum_once(oracle):
    """pre = fl32(sum w*x) with the sum carried far beyond f32 precision: equal
    to the correctly rounded exact sum (within one f32 ulp on near-ties), and
    different from an f32 running sum on these inputs."""
    rng = np.random.default_rng(2)
    W = rng.normal(0, 1, (40, 24))
    x = rng.normal(0, 1, (2, 24)).astype(np.float32)
    pre, _ = oracle.forward(W, x, -1)
    f32_differs = 0
    for b in range(2):
        for o in range(40):
            exact = sum(F(W[o, k]) * F(x[b, k]) for k in range(24))
            want = rnd32(exact)
            assert abs(float(pre[b, o]) - float(want)) <= abs(np.spacing(np.float32(want))), (b, o)
            acc = np.float32(0)
            for k in range(24):
                acc = np.float32(acc + np.float32(np.float32(W[o, k]) * x[b, k]))
            f32_differs += acc != want
    assert f32_differs > 0


# --------------------------------------------------------------- backward
def test_backward_dyadic_brute_force(oracle):
    rng = np.random.default_rng(3)
    out, inn, batch = 6, 9, 4
    Wi = rng.integers(-16, 17, (out, inn))
    xi = rng.integers(-16, 17, (batch, inn))
    gi = rng.integers(-16, 17, (batch, out))
    pi = rng.integers(-4, 5, (batch, out))
    W, x, gy, pre = Wi / 8.0, (xi / 4.0).astype(np.float32), (gi / 4.0).astype(np.float32), \
        (pi / 2.0).astype(np.float32)
    for act, mask in ((-1, np.ones_like(pi)), (0, (pi > 0).astype(np.int64))):
        dpre, dX, dW = oracle.backward(W, x, pre, gy, act)
        dpi = gi * mask  # units of 1/4
        np.testing.assert_array_equal(dpre, (dpi / 4.0).astype(np.float32))
        np.testing.assert_array_equal(dX, ((dpi @ Wi) / 32.0).astype(np.float32))  # not Wi.T
        np.testing.assert_array_equal(dW, ((dpi.T @ xi) / 16.0).astype(np.float32))


def test_backward_dw_is_a_sequential_fused_multiply_add(oracle):
    """dW[o,i] = fl32(acc + g*x) over the batch with the product exact: the
    exact-rational model of that recurrence, which differs from a rounded
    product followed by a rounded add on some of these entries."""
    rng = np.random.default_rng(4)
    out, inn, batch = 5, 7, 6
    W = np.zeros((out, inn))
    x = rng.normal(0, 1, (batch, inn)).astype(np.float32)
    gy = rng.normal(0, 1, (batch, out)).astype(np.float32)
    pre = np.ones((batch, out), np.float32)
    _, _, dW = oracle.backward(W, x, pre, gy, -1)
    unfused_differs = 0
    for o in range(out):
        for i in range(inn):
            acc = np.float32(0)
            acc_u = np.float32(0)
            for b in range(batch):
                acc = rnd32(F(acc) + F(gy[b, o]) * F(x[b, i]))
                acc_u = np.float32(acc_u + np.float32(gy[b, o] * x[b, i]))
            assert dW[o, i] == acc, (o, i)
            unfused_differs += acc_u != acc
    assert unfused_differs > 0


# ------------------------------------------------------------ activations
def _gelu_tanh(x):  # Hendrycks & Gimpel's tanh approximation
    return 0.5 * x * (1 + math.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))


TEXTBOOK = {
    "silu": lambda x: x / (1 + math.exp(-x)),
    "gelu": _gelu_tanh,
    "tanh": math.tanh,
    "sigmoid": lambda x: 1 / (1 + math.exp(-x)),
}


@pytest.mark.parametrize("name", list(TEXTBOOK))
def test_smooth_activations_match_textbook(oracle, name):
    act = ACT[name]
    f = TEXTBOOK[name]
    for v in np.linspace(-12, 12, 481).astype(np.float32):
        got = oracle.act(float(v), act)
        want = f(float(v))
        # 1 + tanh(u) cancels for GELU at large negative x: absolute slack there
        assert abs(got - want) <= 2 * abs(np.spacing(np.float32(want))) + 1e-14, (name, v)


@pytest.mark.parametrize("name", list(TEXTBOOK) + ["relu", "leakyrelu", "relu2", "linear"])
def test_derivatives_match_finite_differences(oracle, name):
    act = ACT[name]
    exact = {"relu": lambda x: max(x, 0.0), "leakyrelu": lambda x: x if x >= 0 else 0.01 * x,
             "relu2": lambda x: 0.0 if x < 0 else x * x, "linear": lambda x: x}
    f = TEXTBOOK.get(name) or exact[name]
    h = 1e-5
    for v in np.linspace(-6, 6, 97).astype(np.float32):
        x = float(v)
        if abs(x) < 2 * h:
            continue  # the kinks at 0
        fd = (f(x + h) - f(x - h)) / (2 * h)
        got = oracle.act_prime(x, act)
        assert abs(got - fd) <= 2e-4 * max(1.0, abs(fd)), (name, x, got, fd)


def test_activation_special_points(oracle):
    assert oracle.act(0.0, ACT["sigmoid"]) == 0.5
    for name in ("silu", "gelu", "tanh", "relu", "relu2", "leakyrelu"):
        assert oracle.act(0.0, ACT[name]) == 0.0
    assert oracle.act(18.5, ACT["tanh"]) == 1.0 and oracle.act(-18.5, ACT["tanh"]) == -1.0
    assert oracle.act(30.0, ACT["gelu"]) == 30.0
    assert oracle.act_prime(0.0, ACT["relu"]) == 0.0      # v > 0 ? 1 : 0
    assert oracle.act_prime(0.0, ACT["relu2"]) == 0.0
    assert oracle.act_prime(-1.0, ACT["leakyrelu"]) == np.float32(0.01)
    # v > 0 ? 1 : 0.01f (ops_common.metal:135-136): the slope at exactly 0 is
    # the negative side's, the f32 constant
    assert oracle.act_prime(0.0, ACT["leakyrelu"]) == np.float32(0.01)
    assert oracle.act_prime(-0.0, ACT["leakyrelu"]) == np.float32(0.01)
    assert oracle.act_prime(2.0 ** -140, ACT["leakyrelu"]) == 1.0
    assert oracle.act_prime(0.0, ACT["tanh"]) == 1.0
    assert oracle.act_prime(0.0, ACT["sigmoid"]) == 0.25
    for unknown in (7, 42, -2):  # unknown ids act as Linear
        assert oracle.act(-3.5, unknown) == -3.5 and oracle.act_prime(-3.5, unknown) == 1.0


# ---------------------------------------------------- fixed-scale re-encode
NATIVE = [d for d in range(34) if d not in (0, 1)]


# Codes that decode to a value which re-encodes to another code of the same
# value: E4M3 -0 and subnormals (all decode to zero, re-encode to 0x00) and the
# 64-bit unsigned formats (the f32 value cannot hold a 64-bit code).
LOSSY_CODES = ("uint64", "uint", "uintptr")


def _byte_fixed_point_expected(dtype, raw, dec, i):
    name = DTYPE_NAMES[dtype]
    if name in LOSSY_CODES:
        return False
    if name == "fp8e4m3" and dec[i] == 0 and raw[i] != 0:
        return False
    return True


@pytest.mark.parametrize("dtype", NATIVE, ids=[DTYPE_NAMES[d] for d in NATIVE])
def test_set_decoded_value_is_a_fixed_point(oracle, dtype):
    """Re-encoding an element's own decoded value keeps that value
    (decode(encode(decode(c))) == decode(c)) and, for every code that is the
    only one of its value, keeps every byte."""
    rng = np.random.default_rng(dtype)
    n = 37
    for w in (rng.normal(0, 0.05, n), rng.uniform(-3, 3, n)):
        raw, scale = oracle.pack(dtype, w.astype(np.float32))
        dec = oracle.decode(dtype, raw, scale, n)
        for i in range(n):
            r2 = raw.copy()
            assert oracle.set(dtype, r2, scale, i, n, float(dec[i])) == 0
            assert oracle.decode(dtype, r2, scale, n)[i] == dec[i], (DTYPE_NAMES[dtype], i)
            if _byte_fixed_point_expected(dtype, raw, dec, i):
                np.testing.assert_array_equal(r2, raw, err_msg=f"{DTYPE_NAMES[dtype]} i={i}")


@pytest.mark.parametrize("dtype", NATIVE, ids=[DTYPE_NAMES[d] for d in NATIVE])
def test_set_touches_only_its_element(oracle, dtype):
    rng = np.random.default_rng(100 + dtype)
    n = 29
    raw, scale = oracle.pack(dtype, rng.uniform(-2, 2, n).astype(np.float32))
    before = oracle.decode(dtype, raw, scale, n)
    for i in (0, 1, 7, 13, n - 1):
        r2 = raw.copy()
        oracle.set(dtype, r2, scale, i, n, float(rng.uniform(-2, 2)))
        after = oracle.decode(dtype, r2, scale, n)
        others = np.arange(n) != i
        np.testing.assert_array_equal(after[others], before[others],
                                      err_msg=f"{DTYPE_NAMES[dtype]} i={i}")


def test_set_signed_integer_quantizer(oracle):
    """Int8/Int4/Int16 with a power-of-two scale: code = clamp(round-half-away(v/s))."""
    for dtype, lo, hi in ((9, -128, 127), (14, -8, 7), (8, -32768, 32767)):
        n = 8
        raw, scale = oracle.pack(dtype, np.full(n, 0.0, np.float32))
        s = float(np.float32(scale))
        for v in (0.3, -0.3, 2.5, -2.5, 1e9, -1e9, 7.49, 126.5):
            r = raw.copy()
            oracle.set(dtype, r, scale, 3, n, v * s)
            q = math.floor(abs(v) + 0.5) * (1 if v >= 0 else -1)
            want = min(max(q, lo), hi) * s
            assert oracle.decode(dtype, r, scale, n)[3] == np.float32(want), (dtype, v)


# (dtype, largest code, signed): the fixed-scale re-encode of
# ops_storage.metal:636-654 (n-bit), :692-762 (integers), :748-755 (quant_u64)
UNSIGNED_SET = [(13, 255), (12, 65535), (15, 15), (18, 3), (29, 63), (31, 31), (33, 7)]
SIGNED_SET = [(28, 31), (27, 31), (30, 15), (32, 3), (17, 1)]


def _q_of(oracle, dtype, raw, s, mn, n, i):
    """The integer code of element i from its decode q*s + min (s a power of two)."""
    return (float(oracle.decode(dtype, raw, s, n)[i]) - mn) / s


@pytest.mark.parametrize("dtype,qmax", UNSIGNED_SET, ids=[DTYPE_NAMES[d] for d, _ in UNSIGNED_SET])
def test_set_unsigned_closed_form(oracle, dtype, qmax):
    """Unsigned re-encode with the stored min m and a power-of-two scale s:
    code = clamp(round-half-away((v - m) / s), 0, qmax).  Values exactly half
    way between two codes (even and odd lower code alike) go up, values just
    below half way go down, and both clamp bounds hold; ties-to-even, a
    truncation, a dropped min or an off-by-one bound fails."""
    n, i = 16, 5
    s, mn = 2.0 ** -4, -1.25
    raw = np.zeros(oracle.native_bytes(dtype, n), np.uint8)
    raw[:4] = np.frombuffer(np.float32(mn).tobytes(), np.uint8)
    cases = [(q + 0.5, q + 1) for q in range(0, min(qmax, 6))]
    cases += [(q + 0.5 - 2.0 ** -8, q) for q in range(0, min(qmax, 6))]
    cases += [(qmax + 0.5, qmax), (qmax + 40.0, qmax), (-0.5 + 2.0 ** -8, 0), (-0.5, 0), (-30.0, 0), (0.0, 0)]
    for t, want in cases:
        r = raw.copy()
        v = np.float32(mn + t * s)
        assert float(v) == mn + t * s  # the input is exact, so only the rounding rule decides
        assert oracle.set(dtype, r, s, i, n, float(v)) == 0
        assert _q_of(oracle, dtype, r, s, mn, n, i) == want, (DTYPE_NAMES[dtype], t, want)
        assert np.count_nonzero(r[:4] != raw[:4]) == 0  # the min header is kept


# Uint32 (clamp to 4294967295.0 as f32 = 2^32, saturating conversion) and the
# 64-bit unsigned formats (quant_u64 ops_storage.metal:106-113: 0 at or below
# zero, 1e15 at or above 1e15f): (dtype, code bytes, largest code)
UNSIGNED_WIDE = [(11, 4, 4294967295), (10, 8, 10**15), (22, 8, 10**15), (23, 8, 10**15)]


@pytest.mark.parametrize("dtype,width,qtop", UNSIGNED_WIDE, ids=[DTYPE_NAMES[d] for d, _, _ in UNSIGNED_WIDE])
def test_set_unsigned_wide_closed_form(oracle, dtype, width, qtop):
    """The wide unsigned re-encode (ops_storage.metal:739-755, :826-858) read
    back as the stored integer: with the stored min m and a power-of-two scale
    s, small codes are round-half-away((v - m) / s) (an exact quotient, so only
    the rounding rule decides: a truncation or ties-to-even fails), negative
    quotients store 0, and huge values store the saturated top code."""
    n, i = 16, 5
    s, mn = 2.0 ** -4, -1.25
    raw = np.zeros(oracle.native_bytes(dtype, n), np.uint8)
    raw[:4] = np.frombuffer(np.float32(mn).tobytes(), np.uint8)
    cases = [(q + 0.5, q + 1) for q in range(0, 8)]
    cases += [(q + 0.5 - 2.0 ** -8, q) for q in range(0, 8)]
    cases += [(q + 2.0 ** -8, q) for q in range(1, 8)]
    cases += [(-0.5 + 2.0 ** -8, 0), (-0.5, 0), (-30.0, 0), (0.0, 0), (1000.5, 1001)]
    dt = "<u4" if width == 4 else "<u8"
    for t, want in cases + [(None, qtop)]:
        r = raw.copy()
        v = np.float32(1e30) if t is None else np.float32(mn + t * s)
        if t is not None:
            assert float(v) == mn + t * s
        assert oracle.set(dtype, r, s, i, n, float(v)) == 0
        got = int(r[4 + i * width:4 + (i + 1) * width].view(dt)[0])
        assert got == want, (DTYPE_NAMES[dtype], t, got, want)
        assert np.count_nonzero(r[:4] != raw[:4]) == 0
        others = np.ones(r.size, bool)
        others[4 + i * width:4 + (i + 1) * width] = False
        assert not np.any(r[others] != raw[others])


def _nf4_table(oracle):
    codes = np.arange(16, dtype=np.uint8)
    raw = (codes[0::2] | (codes[1::2] << 4)).astype(np.uint8)
    return oracle.decode(26, raw, 1.0, 16)


def _nf4_ties(table):
    """f32 values r with |r - t[c]| == |r - t[c+1]| (both f32 differences) for
    adjacent entries, found around each midpoint."""
    ties = []
    for c in range(15):
        a, b = np.float32(table[c]), np.float32(table[c + 1])
        mid = np.float32((np.float64(a) + np.float64(b)) / 2)
        r = mid
        for _ in range(64):
            ea, eb = np.float32(abs(r - a)), np.float32(abs(r - b))
            if ea == eb:
                ties.append((c, float(r)))
                break
            r = np.nextafter(r, b if ea < eb else a, dtype=np.float32)
    return ties


def test_nf4_ties_go_to_the_first_index(oracle):
    """NF4's nearest-entry search takes the first index on an exact tie of the
    f32 distances, in the re-encode (ops_storage.metal:863-878) and in pack
    (native_codec.cpp:93-110, scale 1 when the absmax is 1): values that sit
    exactly between two adjacent table entries get the lower code, and the
    values one f32 step to either side get the nearer one.  A `<=` search
    (the last index wins) fails."""
    table = _nf4_table(oracle)
    ties = _nf4_ties(table)
    assert len(ties) >= 5, ties
    n, i = 8, 3
    for c, r in ties:
        for v, want in ((r, c), (float(np.nextafter(np.float32(r), np.float32(9), dtype=np.float32)), c + 1),
                        (float(np.nextafter(np.float32(r), np.float32(-9), dtype=np.float32)), c)):
            raw = np.zeros(n // 2, np.uint8)
            assert oracle.set(26, raw, 1.0, i, n, v) == 0
            assert (raw[i // 2] >> 4 * (i % 2)) & 0xF == want, (c, v, want)
        # pack: absmax 1 fixes the scale at 1
        w = np.zeros(n, np.float32)
        w[0], w[i] = 1.0, r
        raw, scale = oracle.pack(26, w)
        assert scale == 1.0 and (raw[i // 2] >> 4 * (i % 2)) & 0xF == c, (c, r)


@pytest.mark.parametrize("dtype,qmax", SIGNED_SET, ids=[DTYPE_NAMES[d] for d, _ in SIGNED_SET])
def test_set_signed_nbit_closed_form(oracle, dtype, qmax):
    """Signed n-bit re-encode (Int6 / FP6 / Int5 / Int3, two's complement; Int2
    stored as q + 2): code = clamp(round-half-away(v / s), -qmax - 1, qmax)."""
    n, i = 16, 9
    s = 2.0 ** -3
    raw = np.zeros(oracle.native_bytes(dtype, n), np.uint8)
    cases = []
    for q in range(0, min(qmax, 5)):
        cases += [(q + 0.5, q + 1), (-(q + 0.5), -(q + 1)), (q + 0.5 - 2.0 ** -8, q),
                  (-(q + 0.5 - 2.0 ** -8), -q)]
    cases += [(qmax + 0.5, qmax), (qmax + 100.0, qmax), (-(qmax + 1.5), -qmax - 1),
              (-(qmax + 100.0), -qmax - 1)]
    for t, want in cases:
        r = raw.copy()
        assert oracle.set(dtype, r, s, i, n, t * s) == 0
        got = float(oracle.decode(dtype, r, s, n)[i]) / s
        assert got == want, (DTYPE_NAMES[dtype], t, got, want)
        others = np.arange(n) != i
        assert np.all(oracle.decode(dtype, r, s, n)[others] == oracle.decode(dtype, raw, s, n)[others])


def test_set_ternary_and_binary_thresholds(oracle):
    """Ternary: v/s > 0.5 -> +s, < -0.5 -> -s, else 0 (0.5 itself is 0);
    Binary: v >= 0 -> +s, else -s (ops_storage.metal set_weight_at)."""
    n, s = 8, 0.25
    raw = np.zeros(oracle.native_bytes(19, n), np.uint8)
    for t, want in ((0.5, 0.0), (0.5 + 2.0 ** -10, s), (-0.5, 0.0), (-0.5 - 2.0 ** -10, -s),
                    (3.0, s), (-3.0, -s), (0.0, 0.0)):
        r = raw.copy()
        oracle.set(19, r, s, 2, n, t * s)
        assert oracle.decode(19, r, s, n)[2] == np.float32(want), t
    raw = np.zeros(oracle.native_bytes(20, n), np.uint8)
    for v, want in ((0.0, s), (-0.0, s), (1e-30, s), (-1e-30, -s), (-5.0, -s)):
        r = raw.copy()
        oracle.set(20, r, s, 3, n, v)
        assert oracle.decode(20, r, s, n)[3] == np.float32(want), v


def test_set_saturating_clamp_bounds(oracle):
    """The float clamp bounds 2147483647.0f and 4294967295.0f are 2^31 and 2^32:
    the following conversion saturates (arm64)."""
    raw, scale = oracle.pack(7, np.array([1.0, -1.0], np.float32))  # Int32, scale 1/(2^31-1)
    oracle.set(7, raw, scale, 0, 2, 10.0)
    assert raw[:4].view("<i4")[0] == 2**31 - 1
    oracle.set(7, raw, scale, 0, 2, -10.0)
    assert raw[:4].view("<i4")[0] == -2**31


# ------------------------------------------------------------------- SGD
def test_native_sgd_zero_rate_is_identity(oracle):
    """lr = 0 re-encodes every element's own value: values are unchanged, and
    bytes too wherever the code is the only one of its value."""
    rng = np.random.default_rng(7)
    n = 50
    for dtype in NATIVE:
        raw, scale = oracle.pack(dtype, rng.normal(0, 0.3, n).astype(np.float32))
        dec = oracle.decode(dtype, raw, scale, n)
        r2 = raw.copy()
        assert oracle.native_sgd(dtype, r2, scale, n, rng.normal(0, 1, n), 0.0) == 0
        np.testing.assert_array_equal(oracle.decode(dtype, r2, scale, n), dec)
        if DTYPE_NAMES[dtype] not in LOSSY_CODES + ("fp8e4m3",):
            np.testing.assert_array_equal(r2, raw, err_msg=DTYPE_NAMES[dtype])


def test_native_sgd_exact_grid_steps(oracle):
    """Int8 with scale 2^-6 (absmax 127/64) and steps that land on the grid:
    the new codes are exactly old - lr*g / scale."""
    n = 16
    rng = np.random.default_rng(8)
    codes = rng.integers(-100, 100, n)
    codes[0] = 127
    w = (codes / 64.0).astype(np.float32)
    raw, scale = oracle.pack(9, w)
    assert np.float32(scale) == np.float32(2**-6)
    steps = rng.integers(-20, 21, n)
    steps[0] = 0
    g = (steps / 64.0 / 0.5).astype(np.float32)  # lr 0.5
    assert oracle.native_sgd(9, raw, scale, n, g, 0.5) == 0
    np.testing.assert_array_equal(raw.view(np.int8).astype(np.int64),
                                  np.clip(codes - steps, -128, 127))


def test_native_sgd_is_rounded_difference_then_reencode(oracle):
    """E4M3: each new code is the encoder applied to fl32(old - lr*g), with the
    encoder pinned by the reference's own tables."""
    rng = np.random.default_rng(9)
    n = 64
    raw, scale = oracle.pack(4, rng.normal(0, 1, n).astype(np.float32))
    old = oracle.decode(4, raw, scale, n)
    g = rng.normal(0, 1, n).astype(np.float32)
    lr = 0.37
    r2 = raw.copy()
    oracle.native_sgd(4, r2, scale, n, g, lr)
    want = [int(oracle.encode_many(2, np.array([rnd32(F(old[i]) - Fraction(lr) * F(g[i]))],
                                              np.float32))[0]) for i in range(n)]
    assert list(r2) == want


def test_sgd_f32_rounds_the_step_first(oracle):
    rng = np.random.default_rng(10)
    w = rng.normal(0, 1, 300).astype(np.float32)
    g = rng.normal(0, 1, 300).astype(np.float32)
    lr = 0.1
    got = w.copy()
    oracle.sgd_f32(got, g, lr)
    one_rounding_differs = 0
    for i in range(300):
        step = rnd32(Fraction(lr) * F(g[i]))
        assert got[i] == rnd32(F(w[i]) - F(step)), i
        one_rounding_differs += rnd32(F(w[i]) - Fraction(lr) * F(g[i])) != got[i]
    assert one_rounding_differs > 0


def test_float64_native_sgd_closed_form(oracle):
    rng = np.random.default_rng(11)
    w = rng.normal(0, 1, 20)
    raw = np.frombuffer(w.tobytes(), np.uint8).copy()
    g = rng.normal(0, 1, 20).astype(np.float32)
    assert oracle.native_sgd(0, raw, 1.0, 20, g, 0.25) == 0
    np.testing.assert_array_equal(raw.view("<f8"), w - 0.25 * g.astype(np.float64))


# ------------------------------------------------------------------- MSE
def test_mse_exact_rationals(oracle):
    rng = np.random.default_rng(12)
    p = rng.normal(0, 1, 9).astype(np.float32)
    t = rng.normal(0, 1, 9).astype(np.float32)
    exact = sum((F(a) - F(b)) ** 2 for a, b in zip(p, t)) / 9
    assert abs(oracle.mse(p, t) - float(exact)) <= 4 * abs(np.spacing(float(exact)))
    g = oracle.mse_grad(p, t)
    for i in range(9):
        assert g[i] == rnd32(2 * (F(p[i]) - F(t[i])) / 9)
    assert oracle.mse(p, p) == 0.0 and not np.any(oracle.mse_grad(p, p))


def test_mse_grad_rounds_once(oracle):
    """grad = fl32(2 (p - t) / n) with the difference and quotient exact
    before the one rounding (welvet_dense.metal:207-215: two_sum, then the
    soft-double quotient): over inputs chosen so the difference p - t is not
    an f32 (opposite signs, far-apart magnitudes), a gradient formed in f32
    (rounded difference, rounded quotient) differs from the single rounding
    in many places, and the oracle must match the single rounding in all."""
    rng = np.random.default_rng(14)
    n = 1536
    p = (rng.normal(0, 1, n) * np.exp2(rng.integers(-6, 7, n))).astype(np.float32)
    t = (-np.sign(p) * np.abs(rng.normal(0, 1, n)) * np.exp2(rng.integers(-14, -2, n))).astype(np.float32)
    g = oracle.mse_grad(p, t)
    want = np.array([rnd32(2 * (F(a) - F(b)) / n) for a, b in zip(p, t)], np.float32)
    np.testing.assert_array_equal(g, want)
    in_f32 = (np.float32(2) * (p - t)) / np.float32(n)
    assert np.count_nonzero(in_f32 != want) >= 50


# ------------------------------------------------------- CPU baseline path
@pytest.mark.parametrize("dtype", [1, 0, 4, 9, 26, 16, 27, 33, 10])
def test_forward_native_is_decode_then_forward(oracle, dtype):
    """The timed CPU baseline (per-element decode inside the dot) gives the
    same bits as decode_f64 followed by the forward contract, single- and
    multi-threaded."""
    rng = np.random.default_rng(dtype)
    W = rng.normal(0, 0.2, (33, 70)).astype(np.float32)
    x = rng.normal(0, 1, (3, 70)).astype(np.float32)
    bias = rng.normal(0, 1, 20)
    raw, scale = oracle.pack(dtype, W)
    Wd = oracle.decode_f64(dtype, raw, scale, W.size).reshape(W.shape)
    rpre, rpost = oracle.forward(Wd, x, 3, bias)
    for threads in (1, 4):
        pre, post = oracle.forward_native(dtype, raw, scale, x, 33, 70, 3, bias, threads=threads)
        np.testing.assert_array_equal(pre, rpre)
        np.testing.assert_array_equal(post, rpost)


# ------------------------------------------------------------ SwiGLU layer
def _silu64(x):
    x = np.asarray(x, np.float64)
    return x / (1.0 + np.exp(-x))


def test_swiglu_identity_weights_closed_form(oracle):
    """Gate = I, Up = c I, Down = I (Float64 stores hold them exactly): the
    layer is post = h = fl32(silu(x)) * fl32(c x).  A swap of the roles of
    gate and up (silu(c x) * x) or a missing silu would not match."""
    rng = np.random.default_rng(21)
    n, c = 24, np.float32(2.0)
    x = rng.normal(0, 1.5, (3, n)).astype(np.float32)
    I = np.eye(n, dtype=np.float32)
    r = oracle.swiglu_normalbp(0, I, c * I, I, x)
    want = _silu64(x).astype(np.float32) * (c * x)
    np.testing.assert_array_equal(r["pre"], want)
    np.testing.assert_array_equal(r["post"], want)
    assert not np.allclose(want, _silu64(c * x).astype(np.float32) * x)


def test_swiglu_backward_matches_finite_differences(oracle):
    """dX and each third of dW (Gate, Up, Down in that order) against
    central differences of L = sum(post * g) through the oracle's own forward,
    Float64 weights; an O(1) mistake (sign, operand, order) fails by far."""
    rng = np.random.default_rng(22)
    inn, inter, rows = 6, 10, 2
    G = rng.normal(0, 0.5, (inter, inn)).astype(np.float32)
    U = rng.normal(0, 0.5, (inter, inn)).astype(np.float32)
    D = rng.normal(0, 0.5, (inn, inter)).astype(np.float32)
    x = rng.normal(0, 1, (rows, inn)).astype(np.float32)
    g = rng.normal(0, 1, (rows, inn)).astype(np.float32)
    r = oracle.swiglu_normalbp(0, G, U, D, x, g, 0, 0.0)

    def L(G_, U_, D_, x_):
        post = oracle.swiglu_normalbp(0, G_, U_, D_, x_)["post"].astype(np.float64)
        return float(np.sum(post * g))

    eps = 1e-2
    def fd(arrs, k, idx):
        a = [np.array(v, np.float32) for v in arrs]
        hi, lo = [v.copy() for v in a], [v.copy() for v in a]
        hi[k][idx] += eps
        lo[k][idx] -= eps
        return (L(*hi) - L(*lo)) / (2 * eps)

    args = (G, U, D, x)
    dW = r["dW"]
    n_gu = inter * inn
    for k, (arr, base) in enumerate(zip(args[:3], (0, n_gu, 2 * n_gu))):
        for idx in [(0, 0), (arr.shape[0] - 1, arr.shape[1] - 1), (1, 2)]:
            got = dW[base + idx[0] * arr.shape[1] + idx[1]]
            want = fd(args, k, idx)
            assert abs(got - want) <= 2e-3 * max(1.0, abs(want)), (k, idx, got, want)
    for idx in [(0, 0), (1, inn - 1), (0, 3)]:
        want = fd(args, 3, idx)
        assert abs(r["dX"][idx] - want) <= 2e-3 * max(1.0, abs(want)), (idx, r["dX"][idx], want)


def test_swiglu_split_elementwise_closed_form(oracle):
    """op_swiglu's backward split at points where silu and silu' are known:
    gate 0 gives silu 0 and silu' 1/2."""
    gate = np.zeros(4, np.float32)
    up = np.array([1.0, -2.0, 0.5, 3.0], np.float32)
    gh = np.array([2.0, 1.0, -4.0, 0.25], np.float32)
    d_up, d_gate = oracle.swiglu_split(gate, up, gh)
    np.testing.assert_array_equal(d_up, np.zeros(4, np.float32))
    np.testing.assert_array_equal(d_gate, gh * up * np.float32(0.5))
    np.testing.assert_array_equal(oracle.swiglu_h(gate, up), np.zeros(4, np.float32))


# ------------------------------------------------ Sequential / Residual chains
def test_chain_closed_forms(oracle):
    """Identity children, Linear: Sequential post = x, Residual post = 2x;
    zero children: Residual post = x, Sequential post = 0; ReLU identity
    children: Sequential post = relu(x) (Float64 stores hold I exactly)."""
    rng = np.random.default_rng(31)
    dim, depth = 8, 3
    x = rng.normal(0, 1, (4, dim)).astype(np.float32)
    eye = np.stack([np.eye(dim, dtype=np.float32)] * depth)
    zero = np.zeros_like(eye)
    np.testing.assert_array_equal(oracle.chain_normalbp(False, 0, eye, x, -1)["post"], x)
    np.testing.assert_array_equal(oracle.chain_normalbp(True, 0, eye, x, -1)["post"], 2 * x)
    np.testing.assert_array_equal(oracle.chain_normalbp(True, 0, zero, x, -1)["post"], x)
    np.testing.assert_array_equal(oracle.chain_normalbp(False, 0, zero, x, -1)["post"], 0 * x)
    np.testing.assert_array_equal(oracle.chain_normalbp(False, 0, eye, x, ACT["relu"])["post"],
                                  np.maximum(x, 0))


@pytest.mark.parametrize("residual", [False, True])
def test_chain_backward_matches_finite_differences(oracle, residual):
    """dX and dW (children concatenated in order) against central differences
    of L = sum(post * g), Float64 weights, tanh children."""
    rng = np.random.default_rng(32 + residual)
    dim, depth, rows = 5, 3, 2
    P = rng.normal(0, 0.6, (depth, dim, dim)).astype(np.float32)
    x = rng.normal(0, 1, (rows, dim)).astype(np.float32)
    g = rng.normal(0, 1, (rows, dim)).astype(np.float32)
    act = ACT["tanh"]
    r = oracle.chain_normalbp(residual, 0, P, x, act, g, 0, 0.0)

    def L(P_, x_):
        post = oracle.chain_normalbp(residual, 0, P_, x_, act)["post"].astype(np.float64)
        return float(np.sum(post * g))

    eps = 1e-2
    for idx in [(0, 0, 0), (1, 2, 3), (2, dim - 1, 0)]:
        hi, lo = P.copy(), P.copy()
        hi[idx] += eps
        lo[idx] -= eps
        want = (L(hi, x) - L(lo, x)) / (2 * eps)
        got = r["dW"][idx[0] * dim * dim + idx[1] * dim + idx[2]]
        assert abs(got - want) <= 2e-3 * max(1.0, abs(want)), (idx, got, want)
    for idx in [(0, 0), (1, dim - 1)]:
        hi, lo = x.copy(), x.copy()
        hi[idx] += eps
        lo[idx] -= eps
        want = (L(P, hi) - L(P, lo)) / (2 * eps)
        assert abs(r["dX"][idx] - want) <= 2e-3 * max(1.0, abs(want)), (idx, r["dX"][idx], want)
