"""welvet_model_mount's descriptor checks on the CPU: every malformed WMN1
descriptor is refused with the reference's message (model_session.cpp:
319-404) before any device work; what this Dense-only build does not hold is
refused with code 2."""
import struct

import numpy as np
import pytest

import model_desc
import pywelvet
import wire


def _stack_desc(oracle, dtype=4):
    rng = np.random.default_rng(1)
    return model_desc.stack(oracle, [(rng.normal(0, 0.3, (6, 4)).astype(np.float32), 0, dtype, None),
                                     (rng.normal(0, 0.3, (3, 6)).astype(np.float32), -1, 1, np.ones(3))])


def _mount(desc):
    m = pywelvet.Model(desc, status=True)
    st = m.status
    m.close()
    return st.code, st.message.decode()


def test_abi_version():
    assert pywelvet.lib().welvet_model_abi_version() == 1


def test_header_checks(oracle):
    good = _stack_desc(oracle)
    assert _mount(good[:20]) == (1, "invalid mount arguments")
    assert _mount(b"XMN1" + good[4:]) == (1, "unsupported model descriptor version")
    bad_root = good[:4] + struct.pack("<i", 7) + good[8:]
    assert _mount(bad_root) == (1, "invalid model root/count")
    assert _mount(good + b"\0") == (1, "trailing descriptor bytes")
    assert _mount(good[:-1])[0] == 1


def test_store_checks(oracle):
    rng = np.random.default_rng(2)
    W = rng.normal(0, 0.3, (6, 4)).astype(np.float32)
    child = wire.dense_child(W, 0, 9)
    raw, scale = oracle.pack(9, W)
    # one Dense child but no store
    assert _mount(wire.wmn1(0, [child], [])) == (1, "store count mismatch")
    # rows that do not match the child's out
    bad = wire.store_snapshot(9, 5, 4, scale, raw=raw)
    assert _mount(wire.wmn1(0, [child], [bad])) == (1, "native store metadata mismatch")
    # a native payload one byte short, and an f32 payload on an Int8 store
    bad = wire.store_snapshot(9, 6, 4, scale, raw=raw[:-1])
    assert _mount(wire.wmn1(0, [child], [bad])) == (1, "native store payload length mismatch")
    bad = wire.store_snapshot(9, 6, 4, scale, f32=W, raw=raw)
    assert _mount(wire.wmn1(0, [child], [bad])) == (1, "native store payload length mismatch")
    bad = wire.store_snapshot(9, 6, 4, float("inf"), raw=raw)
    assert _mount(wire.wmn1(0, [child], [bad])) == (1, "native store metadata mismatch")


def test_grid_checks(oracle):
    rng = np.random.default_rng(3)
    W = rng.normal(0, 0.3, (4, 4)).astype(np.float32)
    cells = {(0, 0, 0, 0): dict(W=W), (0, 0, 1, 0): dict(W=W, remote=(0, 0, 0, 0))}
    desc = model_desc.grid(oracle, (1, 1, 2, 1), cells)
    # cell count against the dimensions
    bad = desc[:12] + struct.pack("<4i", 1, 1, 3, 1) + desc[28:]
    assert _mount(bad) == (1, "grid cell count mismatch")
    # a remote link outside the grid
    cells[(0, 0, 1, 0)]["remote"] = (0, 0, 5, 0)
    assert _mount(model_desc.grid(oracle, (1, 1, 2, 1), cells)) == (1, "invalid remote link")
    # an enabled cell without an operation
    children = [wire.dense_child(W), wire.empty_child()]
    snaps = [model_desc.snapshot(oracle, W, 1)]
    desc = wire.wmn1(2, children, snaps, dims=(1, 1, 2, 1),
                     cells=[(1, 0, 0, 0, 0, 0), (1, 0, 0, 0, 0, 0)])
    assert _mount(desc) == (1, "enabled grid cell has no operation")


def test_outside_this_build_is_code_2(oracle):
    desc = _stack_desc(oracle)
    parallel = desc[:4] + struct.pack("<i", 1) + desc[8:]
    assert _mount(parallel)[0] == 2
    rms = struct.pack("<I", 0x314E4D57) + struct.pack("<6i", 0, 1, 1, 1, 1, 1) + struct.pack("<i", 2) + b"\0" * 64
    code, msg = _mount(rms)
    assert code == 2 and "non-Dense" in msg


def test_valid_descriptor_without_device(oracle):
    if pywelvet.available():
        pytest.skip("a GPU is present")
    assert _mount(_stack_desc(oracle))[0] == 2  # parsed, then no HIP device
