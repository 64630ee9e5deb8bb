"""The wire tool's command line and wire parsing, on the CPU: flags, messages
and exit codes follow the reference's tools/dense_fwd/main.cpp:1253-1711 (2 for
a short or malformed wire, before any device work).  Replies on the GPU are
checked in test_gpu_wire.py."""
import struct
import subprocess

import numpy as np
import pytest

import wire


def test_version_and_help():
    r = subprocess.run([wire.TOOL, "--version"], capture_output=True, text=True)
    assert (r.returncode, r.stdout) == (0, "0.71\n")  # reference c_abi.cpp:79-82
    r = subprocess.run([wire.TOOL, "-h"], capture_output=True, text=True)
    assert r.returncode == 0 and "WVD3" in r.stderr and "WVN1" in r.stderr
    r = subprocess.run([wire.TOOL, "--gaps"], capture_output=True, text=True)
    assert r.returncode == 0 and "Dense" in r.stdout


def test_unknown_arg_and_empty_stdin():
    rc, out, err = wire.run(b"", "--frobnicate")
    assert rc == 2 and err.startswith("unknown arg --frobnicate")
    rc, out, err = wire.run(b"")
    assert rc == 2 and out == b"" and "WVD3" in err  # usage


def test_bad_magic_and_other_layer_wires():
    rc, out, err = wire.run(b"ZZZZ")
    assert (rc, err.strip()) == (2, "welvet_dense_fwd: bad magic ZZZZ")
    for m in (b"WVM1", b"WRB1", b"C2V1", b"MCG1"):
        rc, out, err = wire.run(m + b"\0" * 64)
        assert rc == 2 and out == b"" and "is not a Dense wire" in err, m


# WVD3 of W [2][3], bias [2], x [4][3]: magic 4 + header 24 -> 28; W 24 -> 52;
# bias_len 4 -> 56; bias 16 -> 72; x 48 -> 120
@pytest.mark.parametrize("cut,msg", [(10, "short header"), (24, "short backend"),
                                     (40, "short weights"), (54, "short bias_len"),
                                     (64, "short bias"), (100, "short input")])
def test_wvd_short_wires(cut, msg):
    full = wire.wvd(np.ones((2, 3)), np.ones((4, 3)), bias=np.ones(2))
    assert len(full) == 120
    rc, out, err = wire.run(full[:cut])
    assert (rc, out, err.strip()) == (2, b"", "welvet_dense_fwd: " + msg)


def test_wvd2_short_dtype():
    rc, out, err = wire.run(b"WVD2" + struct.pack("<4i", 1, 3, 2, -1))
    assert (rc, out, err.strip()) == (2, b"", "welvet_dense_fwd: short dtype")


def test_wvd_bad_dims():
    for dims in ((0, 3, 2), (1, -1, 2), (1, 3, 0)):
        payload = b"WVD3" + struct.pack("<6i", dims[0], dims[1], dims[2], -1, 1, 0)
        rc, out, err = wire.run(payload)
        assert (rc, err.strip()) == (2, "welvet_dense_fwd: bad dims"), dims


def test_wdb1_short_wires():
    rc, out, err = wire.run(b"WDB1" + struct.pack("<3i", 1, 2, 2))
    assert (rc, err.strip()) == (2, "welvet_dense_fwd: short WDB1 header")
    W = np.ones((2, 2), np.float32)
    x = np.ones((1, 2), np.float32)
    full = wire.wdb(W, x, np.zeros((1, 2)), 1, 0.1)
    for cut in (30, len(full) - 9, len(full) - 1):  # in W, in the target, in lr
        rc, out, err = wire.run(full[:cut])
        assert (rc, out) == (2, b""), cut


def test_volume_wire_headers():
    for m in (b"WVF1", b"WVN1"):
        rc, out, err = wire.run(m + struct.pack("<4i", 1, 1, 1, 1))
        assert (rc, err.strip()) == (2, "welvet_dense_fwd: short %s header" % m.decode()), m
        rc, out, err = wire.run(m + struct.pack("<7i", 1, 1, 1, 1, 0, 0, 0))
        assert (rc, err.strip()) == (2, "welvet_dense_fwd: bad batch"), m
    # every hop disabled: WVF1 exits 1 without a message, WVN1 names it
    # (volume_fwd.cpp:171, :1808-1811)
    body = wire.volume_body((1, 1, 2, 1), 1, {})
    rc, out, err = wire.run(b"WVF1" + body)
    assert (rc, out, err) == (1, b"", "")
    rc, out, err = wire.run(b"WVN1" + body)
    assert (rc, err.strip()) == (1, "welvet_dense_fwd: no enabled cells")
    # a cell record cut short
    W = np.ones((3, 2), np.float32)
    body = wire.volume_body((1, 1, 1, 1), 1, {(0, 0, 0, 0): (W, -1, 1, None)})
    rc, out, err = wire.run(b"WVF1" + body[:-10])
    assert (rc, out) == (2, b"")


def test_wire_writers_round_trip():
    """The test-side writers lay fields out as the readers expect (a
    mistake here would hide behind every GPU wire test)."""
    W = np.arange(6, dtype=np.float32).reshape(2, 3)
    x = np.arange(3, dtype=np.float32).reshape(1, 3)
    b = wire.wvd(W, x, act=3, dtype=4, bias=np.array([0.5, -1.0]))
    r = wire.Reader(b)
    assert r.magic() == b"WVD3"
    assert [r.i32() for _ in range(6)] == [1, 3, 2, 3, 4, 0]
    np.testing.assert_array_equal(r.f32s(6), W.ravel())
    assert r.i32() == 2 and (r.f64(), r.f64()) == (0.5, -1.0)
    np.testing.assert_array_equal(r.f32s(3), x.ravel())
    assert r.done()
    body = wire.volume_body((1, 1, 2, 1), 4, {(0, 0, 1, 0): (W, 0, 9, None)},
                            links=[((0, 0, 1, 0), (0, 0, 0, 0))])
    r = wire.Reader(body)
    assert [r.i32() for _ in range(7)] == [1, 1, 2, 1, 4, 0, 1]
    assert [r.i32() for _ in range(8)] == [0, 0, 1, 0, 0, 0, 0, 0]
    assert r.i32() == 0  # hop (0,0,0,0) disabled
    assert [r.i32() for _ in range(5)] == [1, 3, 2, 0, 9]
    np.testing.assert_array_equal(r.f32s(6), W.ravel())
    assert r.i32() == 0 and r.done()


def test_swiglu_wire_parsing():
    rc, out, err = wire.run(b"WVS1" + struct.pack("<3i", 1, 1, 4))
    assert (rc, err.strip()) == (2, "welvet_dense_fwd: short WVS1 header")
    rc, out, err = wire.run(b"WVS1" + struct.pack("<6i", 1, 0, 4, 8, 1, 0))
    assert (rc, err.strip()) == (2, "welvet_dense_fwd: bad swiglu dims")
    G = np.ones((8, 4), np.float32)
    D = np.ones((4, 8), np.float32)
    x = np.ones((2, 4), np.float32)
    full = wire.wvs(G, G, D, x)
    rc, out, err = wire.run(full[:60])
    assert (rc, err.strip()) == (2, "welvet_dense_fwd: short WVS1 weights")
    rc, out, err = wire.run(full[:-4])
    assert (rc, err.strip()) == (2, "welvet_dense_fwd: short WVS1 input")
    rc, out, err = wire.run(b"WSB1" + struct.pack("<2i", 1, 1))
    assert (rc, err.strip()) == (2, "welvet_dense_fwd: short WSB1 header")
    full = wire.wsb(G, G, D, x, np.zeros((2, 4)), 1, 0.1)
    rc, out, err = wire.run(full[:-3])  # inside lr: silent exit 2 as the reference
    assert (rc, out, err) == (2, b"", "")


def test_chain_wire_parsing():
    for magic, kind in ((b"WSQ1", "sequential"), (b"WRE1", "residual")):
        rc, out, err = wire.run(magic + struct.pack("<4i", 1, 1, 4, 2))
        assert (rc, err.strip()) == (2, "welvet_dense_fwd: short %s header" % magic.decode())
        rc, out, err = wire.run(magic + struct.pack("<7i", 1, 1, 4, 0, -1, 1, 0))
        assert (rc, err.strip()) == (2, "welvet_dense_fwd: bad %s dims" % kind)
        P = np.ones((2, 4, 4), np.float32)
        rc, out, err = wire.run(wire.chain(magic, P, np.ones((1, 4)))[:-2])
        assert (rc, out, err) == (2, b"", "")
    for magic in (b"SQB1", b"REB1"):
        rc, out, err = wire.run(magic + struct.pack("<2i", 1, 1))
        assert (rc, err.strip()) == (2, "welvet_dense_fwd: short %s header" % magic.decode())
