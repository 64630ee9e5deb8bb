"""welvet_hip_dense_forward_noalloc (no reference counterpart: the forward for
callers that cannot allocate) against welvet_hip_dense_forward_device, the
entry point it varies, on the same session and inputs: bit-identical pre and
post, on two calls in a row with the second on a smaller input, across the
kernel routes whose partial tiles live in the scratch array (split-x bf16,
register-B and LDS-staged fp32 MFMA GEMMs) and the batch-1 GEMV, plus its
size limit and argument errors.  The larger call is also checked against the
oracle's f64 forward at the stated tolerance."""
import sys

import numpy as np
import pytest

import pywelvet
from devmem import DeviceArray, Stream
from oracle import DTYPE_NAMES
from parity import assert_bit_equal, assert_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    pywelvet.init()


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def run(s, batch, x, noalloc):
    """One forward on device buffers; pre and post are prefilled with NaN so
    an output the call does not write shows up."""
    dx = DeviceArray(x.shape)
    dx.upload(x)
    pre = DeviceArray((batch, s.out), fill=np.nan)
    post = DeviceArray((batch, s.out), fill=np.nan)
    st = Stream()
    try:
        if noalloc:
            s.forward_noalloc(batch, dx.ptr, pre.ptr, post.ptr, st.h)
        else:
            s.forward_device(dx.ptr, pre.ptr, post.ptr, st.h)
        st.sync()
        return pre.download(), post.download()
    finally:
        st.close()
        for a in (dx, pre, post):
            a.free()


# (dtype, knobs): FP8 and NF4 on the split-x GEMM, F16 on the register-B GEMM,
# Float32 on the LDS-staged GEMM, FP8 with the split-x GEMM off
CASES = [(4, {}), (26, {}), (2, {}), (1, {}), (4, {"bf3": 0})]


@pytest.mark.parametrize("dtype,knobs", CASES,
                         ids=[f"{DTYPE_NAMES[d]}{'-' + str(k) if k else ''}" for d, k in CASES])
def test_noalloc_matches_forward_device(oracle, dtype, knobs):
    old = {k: pywelvet.set_tuning(k, v) for k, v in knobs.items()}
    try:
        rng = np.random.default_rng(0x5EED00AA + dtype)
        out, inn = 11008, 4096
        W = (rng.standard_normal((out, inn), dtype=np.float32) * np.float32(0.02))
        bias = rng.normal(0, 0.1, out)
        # calls in a row on one session: batch 64 (the 60 MB plan), then a
        # smaller input, batch 8, then batch 1 (the GEMV, no scratch); each
        # against welvet_hip_dense_forward_device on a session mounted at that
        # batch from the same weights
        s = pywelvet.Session(W, batch=1, act=1, dtype=dtype, bias=bias)
        for batch in (64, 8, 1):
            say(f"noalloc {DTYPE_NAMES[dtype]} {knobs} batch {batch}")
            x = rng.standard_normal((batch, inn), dtype=np.float32)
            got_pre, got_post = run(s, batch, x, noalloc=True)
            with pywelvet.Session(W, batch=batch, act=1, dtype=dtype, bias=bias) as ref:
                want_pre, want_post = run(ref, batch, x, noalloc=False)
            assert_bit_equal(got_pre, want_pre, f"pre b{batch}")
            assert_bit_equal(got_post, want_post, f"post b{batch}")
            if batch == 64 and not knobs:
                raw, scale = oracle.pack(dtype, W)
                Wd = oracle.decode_f64(dtype, raw, scale, W.size).reshape(out, inn)
                rpre, rpost = oracle.forward(Wd, x, 1, bias)
                assert_close(got_pre, rpre, inn, "pre vs oracle")
                assert_close(got_post, rpost, inn, "post vs oracle")
        s.close()
    finally:
        for k, v in old.items():
            pywelvet.set_tuning(k, v)


def test_noalloc_limits_and_errors():
    """Rejected before any launch: a plan past the 64 MiB scratch (batch 2048
    at 4096 -> 11008), batch 0, a misaligned or null pointer."""
    rng = np.random.default_rng(5)
    W = rng.normal(0, 0.02, (11008, 4096)).astype(np.float32)
    dx, dy = DeviceArray((2048, 4096)), DeviceArray((2048, 11008))
    try:
        with pywelvet.Session(W, batch=1, dtype=4) as s:
            st = s.forward_noalloc(2048, dx.ptr, dy.ptr, dy.ptr, None, status=True)
            assert st.code == 1 and b"no-allocation forward" in st.message, st.message
            st = s.forward_noalloc(0, dx.ptr, dy.ptr, dy.ptr, None, status=True)
            assert st.code == 1
            st = s.forward_noalloc(4, dx.ptr + 4, dy.ptr, dy.ptr, None, status=True)
            assert st.code == 1 and b"aligned" in st.message
            st = s.forward_noalloc(4, None, dy.ptr, dy.ptr, None, status=True)
            assert st.code == 1
    finally:
        dx.free()
        dy.free()
