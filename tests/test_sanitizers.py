"""Host code under AddressSanitizer + UndefinedBehaviorSanitizer, on the CPU.

* The oracle: oracle/sanitize_driver.c calls every entry point over every
  dtype with exactly sized heap buffers, ragged and empty stores, special
  values and bad arguments (`make -C oracle sanitize`).  The whole CPU suite
  can also run on the UBSan build of the oracle library:
  WELVET_ORACLE_SO=oracle/_san/liboracle_ubsan.so.
* The parsers: tests/native/fuzz_parsers.cpp mutates valid WMN1 model
  descriptors (welvet_model_mount) and wire-tool messages (every Dense wire
  this build serves) and runs each through the library's host code, compiled
  host-only with the sanitizers (no device code: every parse ends before the
  first device call, which then fails for want of a GPU).
"""
import concurrent.futures as cf
import glob
import os
import subprocess

import numpy as np
import pytest

import model_desc
import wire

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "welvet.metal_amd", "csrc")
OUT = os.path.join(ROOT, "welvet.metal_amd", "_build", "san")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
LIB_SOURCES = ["codec.hip", "dense.hip", "runtime.cpp", "volume.cpp", "swiglu.cpp", "chain.cpp",
               "model.cpp"]
# host code only: -Xarch_host keeps the sanitizers off any device pass
SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
       "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]
SAN_ENV = {"ASAN_OPTIONS": "detect_leaks=0:max_allocation_size_mb=4096:abort_on_error=1",
           "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1"}


def _run(cmd, **kw):
    r = subprocess.run(cmd, capture_output=True, text=True, **kw)
    assert r.returncode == 0, f"{' '.join(cmd)}\n{r.stdout[-4000:]}\n{r.stderr[-4000:]}"
    return r


def test_oracle_under_asan_ubsan():
    _run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "_san/sanitize_driver"])
    r = subprocess.run([os.path.join(ROOT, "oracle", "_san", "sanitize_driver")], capture_output=True,
                       text=True, timeout=300, env={**os.environ, **SAN_ENV})
    assert r.returncode == 0 and "sanitize_driver: ok" in r.stdout, r.stderr[-4000:]


def _fuzzer() -> str:
    """Builds (when a source is newer than it) the sanitized parser fuzzer."""
    exe = os.path.join(OUT, "fuzz_parsers")
    sources = [os.path.join(CSRC, s) for s in LIB_SOURCES + ["wire_tool.cpp"]]
    sources += glob.glob(os.path.join(CSRC, "*.hpp")) + [os.path.join(ROOT, "include", "welvet_c.h"),
                                                        os.path.join(ROOT, "tests", "native",
                                                                     "fuzz_parsers.cpp")]
    if os.path.exists(exe) and os.path.getmtime(exe) > max(os.path.getmtime(s) for s in sources):
        return exe
    os.makedirs(OUT, exist_ok=True)
    inc = ["-I", os.path.join(ROOT, "include")]

    def lib_obj(src):
        obj = os.path.join(OUT, src + ".o")
        _run([HIPCC, "-x", "hip", "-std=c++17", "-fPIC", "--offload-arch=gfx950", "--offload-host-only",
              "-fgpu-rdc", "-ffp-contract=off", *SAN, "-c", os.path.join(CSRC, src), "-o", obj])
        return obj

    def host_obj(src, *extra):
        obj = os.path.join(OUT, os.path.basename(src) + ".o")
        _run([HIPCC, "-std=c++17", *SAN, *inc, *extra, "-c", src, "-o", obj])
        return obj

    with cf.ThreadPoolExecutor(max_workers=6) as ex:
        jobs = [ex.submit(lib_obj, s) for s in LIB_SOURCES]
        jobs.append(ex.submit(host_obj, os.path.join(CSRC, "wire_tool.cpp"), "-Dmain=wire_tool_main"))
        jobs.append(ex.submit(host_obj, os.path.join(ROOT, "tests", "native", "fuzz_parsers.cpp")))
        objs = [j.result() for j in jobs]
    tmp = exe + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-fgpu-rdc", *SAN, *objs, "-o", tmp])
    os.replace(tmp, exe)
    return exe


def _seeds(oracle, d):
    """Valid messages of every kind the parsers read, small enough that
    every prefix and every field overwrite of each is tried."""
    rng = np.random.default_rng(0)

    def m(*shape):
        return rng.normal(0, 0.3, shape).astype(np.float32)

    W, x = m(3, 4), m(2, 4)
    G, U, D, xs = m(6, 4), m(6, 4), m(4, 6), m(2, 4)
    packed = np.stack([m(4, 4), m(4, 4)])  # [depth][dim][dim]
    files = {
        "wvd3.wire": wire.wvd(W, x, act=0, dtype=9, bias=np.ones(3)),
        "wvd2.wire": wire.wvd(W, x, act=1, dtype=4, version=2),
        "wvd1.wire": wire.wvd(W, x, version=1),
        "wdb_target.wire": wire.wdb(W, x, m(2, 3), True, 0.1, act=0, dtype=26, bias=np.ones(2)),
        "wdb_grad.wire": wire.wdb(W, x, m(2, 3), False, 0.0),
        "wvs.wire": wire.wvs(G, U, D, xs, dtype=4),
        "wsb.wire": wire.wsb(G, U, D, xs, m(2, 4), True, 0.1),
        "wsq.wire": wire.chain(b"WSQ1", packed, m(2, 4), child_act=0),
        "wre.wire": wire.chain(b"WRE1", packed, m(2, 4), dtype=9),
        "sqb.wire": wire.chain_nbp(b"SQB1", packed, m(2, 4), m(2, 4), True, 0.1),
        "reb.wire": wire.chain_nbp(b"REB1", packed, m(2, 4), m(2, 4), False, 0.5),
        "stack.wmn": model_desc.stack(oracle, [(m(6, 4), 0, 4, None), (m(3, 6), -1, 1, np.ones(3))]),
        "stack_int4.wmn": model_desc.stack(oracle, [(m(5, 8), 3, 14, np.ones(5))]),
        "grid.wmn": model_desc.grid(oracle, (1, 1, 2, 2), {
            (0, 0, 0, 0): dict(W=m(4, 4), act=0, dtype=9),
            (0, 0, 0, 1): dict(W=m(4, 4), dtype=1, remote=(0, 0, 0, 0)),
            (0, 0, 1, 0): dict(W=m(2, 4), dtype=26, bias=np.ones(2), enabled=False)}),
    }
    files.update(_volume_seeds(m))
    paths = []
    for name, data in files.items():
        p = os.path.join(d, name)
        with open(p, "wb") as f:
            f.write(data)
        paths.append(p)
    return paths


def _volume_seeds(m):
    """WVF1 / WVN1 over a 1x1x2x1 volume with a remote link."""
    cells = {(0, 0, 0, 0): (m(4, 4), 0, 1, None), (0, 0, 1, 0): (m(2, 4), -1, 9, np.ones(2))}
    links = [((0, 0, 1, 0), (0, 0, 0, 0))]
    return {"wvf.wire": wire.wvf((1, 1, 2, 1), 2, cells, m(2, 4), links=links),
            "wvn.wire": wire.wvn((1, 1, 2, 1), 2, cells, m(2, 4), m(2, 2), 0.1)}


def test_parsers_fuzzed_under_asan_ubsan(oracle, tmp_path):
    exe = _fuzzer()
    seeds = _seeds(oracle, str(tmp_path))
    report = str(tmp_path / "report")
    r = subprocess.run([exe, report, "30000", "7", *seeds], capture_output=True, text=True, timeout=600,
                       env={**os.environ, **SAN_ENV})
    reports = [p for p in glob.glob(report + ".*") if not p.endswith((".summary", ".stdin"))]
    text = "".join(open(p).read() for p in reports)
    assert r.returncode == 0 and not reports, text[-6000:] or r.stderr[-4000:]
    summary = open(report + ".summary").read().split()
    model_runs, wire_runs = int(summary[2]), int(summary[summary.index("wire") + 2])
    assert model_runs > 10000 and wire_runs > 10000, summary
    # exits 0 / 1 / 2 of the wire runs: messages that parsed reach the library
    # (code 1 without a GPU) and malformed ones stop at the parser (2)
    exits = [int(v) for v in summary[-3:]]
    assert exits[1] > 0 and exits[2] > 0, summary
