"""Writes the golden vectors under tests/golden/ from the reference's own host
codec, compiled from the reference sources by `make -C oracle ref` into
oracle/_ref/libwelvet_ref.so.  Run in the build container (the only place the
reference checkout exists):

    make -C oracle ref && python tests/golden/make_golden.py

Outputs (data only: inputs and the reference's outputs):
  codec_vectors.npz   per dtype x input set: f32 inputs, native bytes, scale,
                      export_f32 decode, decode_row_f64 decode
  scalar_tables.npz   decode of every code: f16/bf16 (65536), e4m3/e5m2 (256),
                      fp4 (16); encode of a fixed set of edge floats
  release_kat.json    the known-answer test of scripts/release_smoke.py:45-55

Platform note: two float->integer conversions in the reference pack are
undefined behaviour in C++ and differ between the reference platform (arm64:
fcvtzs/fcvtzu saturate, NaN -> 0) and this x86 build (the "integer
indefinite" 0x80...0):
  * Int32 (native_codec.cpp:256-258): the +absmax element converts 2^31;
    arm64 gives 0x7fffffff.
  * Uint64/Uint/Uintptr (native_codec.cpp:333-336, :467-470, :495-498): an
    element whose f32 quotient is NaN (span overflowed to Inf); arm64 gives 0.
The fixture stores the arm64 value in `native` and keeps the x86 bytes in
`native_x86`, so each patched element stays visible.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
from oracle import DTYPE_NAMES, Reference  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))
N = 97  # odd, not a multiple of 8: exercises partial bytes of every bitstream

EDGE = np.array([
    0.0, -0.0, 448.0, -448.0, 240.0, 247.9, 248.0, 256.0, 1e3, -1e3, 2.0**-6, 2.0**-7, 2.0**-9,
    2.0**-10, -(2.0**-8), 3e-5, 6.1e-5, 6.0e-8, 65504.0, 65520.0, 1e5, -1e5, 0.25, 0.75, 1.25,
    1.75, 2.5, 3.5, 5.0, 7.0, -5.0, -6.0, 6.0, 0.5, -0.5, 1.0, -1.0, 0.1, -0.1, 1e-20, 1e-40,
    57344.0, 61440.0, 3.4e38, -3.4e38, 0.3, -0.7, 12.0, 0.03125, 0.046875,
], dtype=np.float32)


def input_sets(rng: np.random.Generator) -> dict[str, np.ndarray]:
    sets = {
        "normal002": rng.normal(0, 0.02, N).astype(np.float32),
        "uniform6": rng.uniform(-6, 6, N).astype(np.float32),
        "normal1": rng.normal(0, 1, N).astype(np.float32),
        "edge": EDGE.copy(),
        "constant": np.full(N, 0.375, np.float32),  # span 0 -> 1, absmax path
        "zeros": np.zeros(N, np.float32),           # absmax 0 -> scale 1
    }
    ties = rng.normal(0, 0.5, N).astype(np.float32)
    ties[5] = 3.0
    ties[17] = -3.0  # two elements share the absmax
    sets["absmax_tie"] = ties
    return sets


def patch_platform_ub(name: str, w: np.ndarray, native: np.ndarray) -> None:
    """Rewrites, in place, the elements whose reference value depends on the
    undefined conversions listed in the module docstring."""
    with np.errstate(all="ignore"):
        if name == "int32":
            s = np.float32(np.abs(w).max()) or np.float32(1)
            q = native.view("<i4")
            hit = (q == np.iinfo(np.int32).min) & (w / s * np.float32(2147483647.0)
                                                   == np.float32(2.0**31))
            q[hit] = np.iinfo(np.int32).max
        elif name in ("uint64", "uint", "uintptr"):
            mn, mx = np.float32(w.min()), np.float32(w.max())
            span = np.float32(mx - mn)
            if span == 0:
                span = np.float32(1)
            qf = (w - mn) / span * np.float32(1e15)
            q = native[4:].view("<u8")
            q[np.isnan(qf)] = 0


def main() -> None:
    R = Reference()
    rng = np.random.default_rng(0x5EED0000)
    arrays: dict[str, np.ndarray] = {}
    for set_name, w in input_sets(rng).items():
        arrays[f"{set_name}/input"] = w
        for dt, name in enumerate(DTYPE_NAMES):
            native, scale = R.pack(dt, w)
            x86 = native.copy()
            patch_platform_ub(name, w, native)
            key = f"{set_name}/{name}"
            arrays[key + "/native"] = native
            if not np.array_equal(native, x86):
                arrays[key + "/native_x86"] = x86
            arrays[key + "/scale"] = np.array([scale], np.float32)
            arrays[key + "/decode"] = R.decode(dt, native, scale, w.size)
            arrays[key + "/decode_f64"] = R.decode_f64(dt, native, scale, w.size)
    np.savez_compressed(os.path.join(OUT, "codec_vectors.npz"), **arrays)

    # decoded into arrays by the reference build: every bit kept, including
    # the payloads of signaling NaNs (a scalar float return read back as a
    # Python float would have been widened to double and quieted)
    tables = {
        "f16_decode": R.decode_many(0, np.arange(65536)),
        "bf16_decode": R.decode_many(1, np.arange(65536)),
        "e4m3_decode": R.decode_many(2, np.arange(256)),
        "e5m2_decode": R.decode_many(3, np.arange(256)),
        "fp4_decode": R.decode_many(4, np.arange(16)),
    }
    probe = np.concatenate([EDGE, -EDGE, np.array([np.inf, -np.inf, np.nan], np.float32),
                            rng.normal(0, 100, 4096).astype(np.float32),
                            rng.normal(0, 1e-3, 4096).astype(np.float32)])
    tables["encode_input"] = probe
    for kind, nm in enumerate(("f16", "bf16", "e4m3", "e5m2", "fp4")):
        tables[f"{nm}_encode"] = R.encode_many(kind, probe)
    np.savez_compressed(os.path.join(OUT, "scalar_tables.npz"), **tables)

    kat = {
        "source": "scripts/release_smoke.py:45-55",
        "geometry": {"batch": 1, "in": 2, "out": 2, "act": -1, "dtype": 1, "backend": 0},
        "W_init": [1, 0, 0, 1], "x": [0.5, -0.25], "target": [0, 0], "use_target": 1, "lr": 0.1,
        "expect_post": [0.5, -0.25], "expect_loss": 0.15625,
        "expect_W_after": [0.975, 0.0125, 0.0125, 0.99375], "tolerance": 1e-6,
    }
    with open(os.path.join(OUT, "release_kat.json"), "w") as f:
        json.dump(kat, f, indent=1)
    print("wrote", sorted(os.listdir(OUT)))


if __name__ == "__main__":
    main()
