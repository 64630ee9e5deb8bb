"""CPU-side checks of the C-ABI library: it loads, exports every entry point
include/welvet_c.h declares, and the no-device path answers Unsupported
(reference device.mm:66-69) without touching a GPU."""
import ctypes
import os
import re

import pytest

import pywelvet

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    src = open(os.path.join(ROOT, "include", "welvet_c.h")).read()
    return sorted(set(re.findall(r"WELVET_API\s+[\w\s\*]+?\b(welvet_\w+)\s*\(", src)))


def test_header_declares_the_reference_dense_subset():
    syms = declared_symbols()
    for s in ("welvet_version", "welvet_runtime_identity", "welvet_metal_init",
              "welvet_metal_available", "welvet_dense_forward_f32", "welvet_dense_normalbp_f32",
              "welvet_dense_mount", "welvet_dense_execute", "welvet_dense_release"):
        assert s in syms


def test_library_exports_every_declared_symbol():
    L = pywelvet.lib()
    for s in declared_symbols():
        assert hasattr(L, s), s


def test_version_matches_reference():
    assert pywelvet.version() == "0.71"  # reference c_abi.cpp:79-82


def test_status_struct_layout():
    assert ctypes.sizeof(pywelvet.Status) == 4 + 256


def test_no_device_is_unsupported():
    if pywelvet.available():
        pytest.skip("a GPU is present")
    import numpy as np
    st, _, _ = pywelvet.forward(np.eye(2, dtype=np.float32), np.ones((1, 2), np.float32),
                                status=True)
    assert st.code == 2
    with pytest.raises(pywelvet.WelvetError) as e:
        pywelvet.init()
    assert e.value.code == 2
    with pytest.raises(pywelvet.WelvetError) as e:
        pywelvet.Grid(1, 1, 1, 1, 1)
    assert e.value.code == 2


def test_argument_errors_before_device():
    """Null/invalid arguments are rejected before any device work
    (reference c_abi.cpp:105-110, :148-160)."""
    import numpy as np
    L = pywelvet.lib()
    x = np.ones(2, np.float32)
    st = L.welvet_dense_mount(1, 2, 2, -1, 1, None, None, 0, ctypes.byref(ctypes.c_void_p()))
    assert st.code == 1
    st = L.welvet_dense_mount(1, 2, 2, -1, 1, pywelvet._fp(x), None, 0, None)
    assert st.code == 1
    st = L.welvet_dense_mount(1, 2, 2, -1, 99, pywelvet._fp(np.ones(4, np.float32)), None, 0,
                              ctypes.byref(ctypes.c_void_p()))
    assert st.code == 2  # session.cpp:40-43: unsupported dtype
    r = pywelvet.normalbp(np.eye(2), np.ones((1, 2)), np.zeros((1, 2)), 1, 0.1, dtype=99,
                          status=True)
    assert r["status"].code == 1  # c_abi.cpp:155-160
    r = pywelvet.normalbp(np.eye(2), np.ones((0, 2)), np.zeros((0, 2)), 1, 0.1, status=True)
    assert r["status"].code == 1
    h = ctypes.c_void_p()
    assert L.welvet_hip_grid_new(1, 1, 1, 1, 0, ctypes.byref(h)).code == 1  # batch <= 0
    assert L.welvet_hip_grid_new(1, 1, 1, 1, 1, None).code == 1
    assert L.welvet_hip_volume_forward(None, None, 0, None, 0).code == 1


def test_swiglu_argument_errors_before_device():
    """c_abi.cpp:330-336, :369-381: dims and null checks come first."""
    import numpy as np
    G = np.ones((4, 2), np.float32)
    D = np.ones((2, 4), np.float32)
    st, _, _ = pywelvet.swiglu_forward(G, G, D, np.ones((0, 2), np.float32), status=True)
    assert (st.code, st.message.decode()) == (1, "swiglu: invalid argument")
    r = pywelvet.swiglu_normalbp(G, G, D, np.ones((1, 2), np.float32), np.zeros((1, 2)), 1, 0.1,
                                 dtype=-1, status=True)
    assert (r["status"].code, r["status"].message.decode()) == (1, "swiglu nbp: bad dtype -1")


@pytest.mark.parametrize("kind", ["sequential", "residual"])
def test_chain_argument_errors_before_device(kind):
    """c_abi.cpp:922-928, :956-962, :1017-1023, :1051-1057."""
    import numpy as np
    P = np.ones((2, 3, 3), np.float32)
    st, _, _ = pywelvet.chain_forward(kind, P, np.ones((0, 3), np.float32), status=True)
    assert (st.code, st.message.decode()) == (1, f"{kind}: invalid argument")
    r = pywelvet.chain_normalbp(kind, np.ones((0, 3, 3), np.float32), np.ones((1, 3), np.float32),
                                np.zeros((1, 3)), 1, 0.1, status=True)
    assert (r["status"].code, r["status"].message.decode()) == (1, f"{kind} nbp: invalid argument")
