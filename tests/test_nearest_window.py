"""The SGD's windowed FP4 / NF4 table search (common.hpp nearest_window)
against nearest16, the reference's full search (float_codecs.cpp:187-198,
native_codec.cpp:525-534), on every f32 bit pattern of r for both tables:
tests/native/nearest_check.cpp, built host-only (no device code runs)."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "welvet.metal_amd", "csrc")
OUT = os.path.join(ROOT, "welvet.metal_amd", "_build", "nearest")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def _run(cmd, **kw):
    r = subprocess.run(cmd, capture_output=True, text=True, **kw)
    assert r.returncode == 0, f"{' '.join(cmd)}\n{r.stdout[-4000:]}\n{r.stderr[-4000:]}"
    return r


def test_window_search_equals_full_search_on_every_f32():
    src = os.path.join(ROOT, "tests", "native", "nearest_check.cpp")
    exe = os.path.join(OUT, "nearest_check")
    deps = [src, os.path.join(CSRC, "common.hpp")]
    if not (os.path.exists(exe) and os.path.getmtime(exe) > max(os.path.getmtime(d) for d in deps)):
        os.makedirs(OUT, exist_ok=True)
        obj = exe + ".o"
        _run([HIPCC, "-x", "hip", "--offload-host-only", "-fgpu-rdc", "-std=c++17", "-O2", "-ffp-contract=off",
              "-I", CSRC, "-c", src, "-o", obj])
        _run([HIPCC, "-fgpu-rdc", "--offload-arch=gfx950", obj, "-o", exe, "-lpthread"])
    r = _run([exe, str(min(8, os.cpu_count() or 1))], timeout=600)
    assert "nearest_check: ok 8589934592" in r.stdout, r.stdout[-2000:]
