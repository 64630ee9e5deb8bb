"""Headline benchmark: Dense forward over packed native weights, 4096 -> 11008.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only fp8b1,...]

A step is one Dense forward (welvet_hip_dense_forward_device) over one batch
of synthetic input already resident in HBM.  The primary line is FP8 E4M3,
batch 1: value = packed-weight bytes per step / step time (GB/s), the BASELINE
metric; a batch-1 step is exactly one GEMV kernel launch.  The same run
measures NF4 batch 1 and FP8 / NF4 batch 64 (TFLOP/s = 2*B*K*N / step time)
and reports them under "results"; `--only fp8b2,fp8b4,nf4b2,nf4b4` times the
batch 2-4 GEMV instead (one launch per step, reported against HBM).

Weights are N(0, 0.02) (generated on the device, seeded), x ~ N(0, 1).  Steps
rotate over enough distinct weight copies that the working set exceeds
512 MB, so the 256 MB MALL cannot serve repeated launches.  Timing: HIP events
on the stream the kernels are launched on (an explicit torch stream handed to
the library), K back-to-back steps between them after W warm-up steps.

roofline.traffic comes from the committed rocprofv3 --pmc passes
(profiles/hbm_traffic.json); it is not measured live.  roofline.read_floor
(batch-1 primary) is measured live: the library's streaming-read probe over
the same bytes, rotated and timed like the steps.

cpu_baseline: the oracle's scalar port of the reference host path (per-element
decode switch + f64 dot, oracle/oracle.c or_dense_forward_native) on full
FP8 and NF4 batch-1 steps, the median of 15 after a warm-up, one thread; an
all-core OpenMP run of the same port and the host CPU model are reported
beside it.

Batched cases: roofline_frac is the executed MFMA rate against that
instruction's dense peak (the split-x GEMM runs 3 bf16 products per fp32
product, 6 for NF4, against the 2.5 PFLOP/s bf16 peak); the fp32-equivalent
rate is reported beside it.  Configs 2-3 are timed as the median of 5
repeats of at least 20 ms of back-to-back steps each.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "welvet.metal_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

METRIC = "Dense fwd HBM GB/s (batch 1) & TFLOP/s (batch 64), FP8/NF4 4096x11008"
HBM_PEAK = 8000.0        # GB/s, MI355X
FP32_MFMA_PEAK = 157.3   # TFLOP/s, MI355X dense fp32 matrix
BF16_MFMA_PEAK = 2500.0  # TFLOP/s, MI355X dense bf16 matrix
SPLIT_X_DTYPES = ("fp8e4m3", "fp8e5m2", "int8", "fp4", "nf4")  # weights the split-x bf16 GEMM takes
IN, OUT = 4096, 11008
MALL_BYTES = 512 << 20   # rotate past 2x the 256 MB Infinity Cache


def packed_bytes(dtype: int) -> int:
    bits = {4: 8, 26: 4, 5: 8, 16: 4, 9: 8}[dtype]
    scale = 4 if dtype == 26 else 0  # NF4 keeps one f32 per-tensor scale
    return IN * OUT * bits // 8 + scale


def run_case(torch, pywelvet, dtype: int, batch: int, steps: int, warmup: int, seed: int):
    dev = torch.device("cuda:0")
    wbytes = packed_bytes(dtype)
    copies = max(2, -(-MALL_BYTES // wbytes))
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    sessions = []
    Wf = torch.empty((OUT, IN), dtype=torch.float32, device=dev)
    for _ in range(copies):
        Wf.normal_(0.0, 0.02, generator=g)
        torch.cuda.synchronize()
        s = pywelvet.Session.__new__(pywelvet.Session)
        s.out, s.inn, s.batch, s.dtype = OUT, IN, batch, dtype
        h = pywelvet.C.c_void_p()
        pywelvet.check(pywelvet.lib().welvet_hip_dense_mount_device(
            batch, IN, OUT, -1, dtype, pywelvet.C.c_void_p(Wf.data_ptr()), None, 0,
            pywelvet.C.byref(h)))
        s.h = h
        sessions.append(s)
    del Wf
    x = torch.empty((batch, IN), dtype=torch.float32, device=dev).normal_(0.0, 1.0, generator=g)
    pre = torch.empty((batch, OUT), dtype=torch.float32, device=dev)
    post = torch.empty_like(pre)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream(device=dev)  # default priority; all launches and events on it
    sh = stream.cuda_stream

    def step(i):
        sessions[i % copies].forward_device(x.data_ptr(), pre.data_ptr(), post.data_ptr(), sh)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for i in range(steps):
        step(i)
    t1.record(stream)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    flops = 2.0 * batch * IN * OUT
    r = {
        "case": f"{pywelvet.DTYPE_NAMES[dtype]}_4096x11008_b{batch}",
        "weight_dtype": pywelvet.DTYPE_NAMES[dtype], "batch": batch, "in": IN, "out": OUT,
        "packed_bytes": wbytes, "weight_copies": copies, "ms_per_step": ms,
        "hbm_gbs": wbytes / (ms * 1e-3) / 1e9, "tflops": flops / (ms * 1e-3) / 1e12,
    }
    for s in sessions:
        s.close()
    return r


def read_floor(torch, pywelvet, nbytes: int, steps: int, warmup: int):
    """The single-launch read floor for a case's packed bytes: the library's
    streaming-read probe (welvet_hip_probe_read) over the same number of
    bytes, rotating through copies larger than the MALL and timed like the
    case's steps, so value / floor says how much of what one launch can read
    the kernel reaches."""
    dev = torch.device("cuda:0")
    n = (nbytes + 15) // 16 * 16
    copies = max(2, -(-MALL_BYTES // n))
    bufs = [torch.full((n,), i, dtype=torch.uint8, device=dev) for i in range(copies)]
    sink = torch.zeros(1024, dtype=torch.int32, device=dev)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream(device=dev)  # default priority
    sh = stream.cuda_stream
    for i in range(warmup):
        pywelvet.probe_read(bufs[i % copies].data_ptr(), n, sink.data_ptr(), sh)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for i in range(steps):
        pywelvet.probe_read(bufs[i % copies].data_ptr(), n, sink.data_ptr(), sh)
    t1.record(stream)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    return {"kernel": "read_probe_kernel (16-byte non-temporal loads, four in flight per thread)",
            "bytes": n, "copies": copies, "us": ms * 1e3, "gbs": n / (ms * 1e-3) / 1e9}


def cpu_model() -> str:
    """The host CPU's model string (/proc/cpuinfo, as lscpu reports it)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(dtypes=(4, 26), batch: int = 1, runs: int = 15):
    """Oracle scalar port of the reference host path (per-element decode
    switch + f64 dot) on full 4096x11008 batch-1 steps: one warm-up, then the
    median of `runs` timed steps on one thread (the baseline) and on every
    host core the run may use (reported beside).  The first dtype is the
    headline's."""
    import numpy as np
    from oracle import Oracle

    O = Oracle()
    rng = np.random.default_rng(0x5EED0002)
    W = rng.standard_normal((OUT, IN), dtype=np.float32) * np.float32(0.02)
    x = rng.standard_normal((batch, IN), dtype=np.float32)
    ncores = min(16, len(os.sched_getaffinity(0)))  # the GPU box grants 16 host threads

    def median_ms(dtype, raw, scale, threads):
        O.forward_native(dtype, raw, scale, x, OUT, IN, -1, threads=threads)  # warm-up
        t = []
        for _ in range(runs):
            t0 = time.perf_counter()
            O.forward_native(dtype, raw, scale, x, OUT, IN, -1, threads=threads)
            t.append(time.perf_counter() - t0)
        t.sort()
        return t[len(t) // 2] * 1e3, t

    per = {}
    total = 0.0
    for dtype in dtypes:
        raw, scale = O.pack(dtype, W)
        ms1, t1 = median_ms(dtype, raw, scale, 1)
        msn, tn = median_ms(dtype, raw, scale, ncores)
        total += sum(t1) + sum(tn)
        per[pywelvet_name(dtype)] = {
            "gbs": packed_bytes(dtype) / (ms1 * 1e-3) / 1e9, "ms_per_step": ms1,
            "all_cores": {"gbs": packed_bytes(dtype) / (msn * 1e-3) / 1e9, "ms_per_step": msn,
                          "cores": ncores}}
    head = per[pywelvet_name(dtypes[0])]
    return {"value": head["gbs"], "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"median of {runs} full {pywelvet_name(dtypes[0])} 4096x11008 b{batch} "
                      f"forward steps after one warm-up ({total:.1f} s of CPU work over all "
                      f"legs): per-element decode switch + f64 dot, 1 thread",
            "ms_per_step": head["ms_per_step"], "cpu_model": cpu_model(), "per_dtype": per,
            "all_cores": {**head["all_cores"], "unit": "GB/s", "value": head["all_cores"]["gbs"],
                          "sample": "same steps, OpenMP over output rows"}}


def cpu_config_baselines(runs: int = 5):
    """BASELINE configs 2-5 on the host with the oracle's scalar port of the
    reference host path (per-element decode switch, f64 dots, sequential fmaf
    dW, fixed-scale re-encode SGD), the same shapes, seeds and weight
    distributions as the GPU legs (inputs from numpy).  C2 / C3 forwards:
    median of `runs` after one warm-up, on one thread at batch 1 (and C2's
    batch 32) and on every host core the run may use at every batch.  C4: one
    timed training step per dtype; C5: one timed step per dtype for all 34
    (the GPU legs time 10 and 2; the oracle keeps no state between steps that
    a warm-up would fill): the oracle's training kernels are OpenMP over the
    host cores, so these report all cores."""
    import numpy as np
    from oracle import Oracle, Volume

    O = Oracle()
    ncores = min(16, len(os.sched_getaffinity(0)))
    seed = 0x5EED0000
    out = {"cores": ncores, "cpu_model": cpu_model(), "kind": "port"}

    def med(fn, n):
        fn()
        t = []
        for _ in range(n):
            t0 = time.perf_counter()
            fn()
            t.append(time.perf_counter() - t0)
        t.sort()
        return round(t[len(t) // 2] * 1e3, 3)

    def chain(widths, dtype, init, rng):
        return [O.pack(dtype, _weights(rng, widths[l + 1], widths[l], init)) for l in range(len(widths) - 1)]

    def forward(widths, dtype, layers, x, threads):
        for l, (raw, scale) in enumerate(layers):
            _, x = O.forward_native(dtype, raw, scale, x, widths[l + 1], widths[l], -1, threads=threads)
        return x

    legs = [("c2", name, dt, [4096, 4096], "normal", b, seed + 1)
            for name, dt in (("e4m3", 4), ("e5m2", 5)) for b in (1, 32)]
    legs += [("c3", name, dt, [4096, 11008, 4096], init, b, seed + 2)
             for name, dt, init in (("nf4", 26, "normal"), ("fp4_u6", 16, "uniform6")) for b in (1, 8, 64)]
    cache = {}
    for cfg, name, dt, widths, init, b, sd in legs:
        key = (cfg, name)
        if key not in cache:
            cache[key] = chain(widths, dt, init, np.random.default_rng(sd))
        layers = cache[key]
        x = np.random.default_rng(sd + 100).standard_normal((b, widths[0]), dtype=np.float32)
        leg = {"all_cores_ms": med(lambda: forward(widths, dt, layers, x, ncores), runs)}
        if b == 1 or cfg == "c2":
            leg["one_thread_ms"] = med(lambda: forward(widths, dt, layers, x, 1), runs)
        tag = "x".join(map(str, widths)) if cfg == "c2" else "-".join(map(str, widths))
        out[f"{cfg}_{name}_{tag}_b{b}"] = leg
        print(f"# cpu {cfg} {name} b{b}: {leg}", file=sys.stderr, flush=True)

    def train(dims, widths, dt, batch, sd):
        rng = np.random.default_rng(sd)
        D, R, Cc, L = dims
        v = Volume(O, D, R, Cc, L, batch)
        k = 0
        for z in range(D):
            for yy in range(R):
                for xx in range(Cc):
                    for l in range(L):
                        W = _weights(rng, widths[k + 1], widths[k], "normal")
                        v.bind_dense((z, yy, xx, l), W, act=-1 if k == len(widths) - 2 else 0, dtype=dt)
                        k += 1
        x = rng.standard_normal((batch, widths[0]), dtype=np.float32)
        t = rng.standard_normal((batch, widths[-1]), dtype=np.float32)
        return v, x, t

    for name, dt in (("int8", 9), ("e4m3", 4)):
        v, x, t = train((1, 1, 2, 1), [2048, 8192, 2048], dt, 256, seed + 3)
        t0 = time.perf_counter()
        v.train_step(x, t, 1e-3)
        ms = (time.perf_counter() - t0) * 1e3
        out[f"c4_{name}_2048-8192-2048_b256"] = {"all_cores_ms": round(ms, 3), "steps": 1}
        print(f"# cpu c4 {name}: {ms:.1f} ms/step", file=sys.stderr, flush=True)
    c5 = {}
    for dt in range(34):
        v, x, t = train((2, 2, 2, 4), [1024] * 33, dt, 16, seed + 4)
        t0 = time.perf_counter()
        v.train_step(x, t, 1e-3)
        c5[pywelvet_name(dt)] = round((time.perf_counter() - t0) * 1e3, 3)
    out["c5_2x2x2x4_1024_b16_all_cores_ms"] = c5
    print(f"# cpu c5: {min(c5.values()):.1f}-{max(c5.values()):.1f} ms/step over 34 dtypes",
          file=sys.stderr, flush=True)
    return out


# ---------------------------------------------------------------- configs
# The other BASELINE configurations, reported under "config_results" (they
# are not the headline metric).  Weights are seeded per config and layer.


def _weights(rng, out, inn, init):
    import numpy as np
    if init == "uniform05":
        return rng.uniform(-0.05, 0.05, (out, inn)).astype(np.float32)
    if init == "uniform6":
        return rng.uniform(-6, 6, (out, inn)).astype(np.float32)
    return (rng.standard_normal((out, inn), dtype=np.float32) * np.float32(0.02))


def _grid(P, widths, dtype, batch, rng, init, act_hidden=-1, act_out=-1, shared=None):
    """A 1 x 1 x L x 1 grid of Dense cells widths[0] -> ... -> widths[-1]."""
    L = len(widths) - 1
    g = P.Grid(1, 1, L, 1, batch)
    for l in range(L):
        key = (widths[l], widths[l + 1])
        if shared is not None and key in shared:
            W = shared[key]
        else:
            W = _weights(rng, widths[l + 1], widths[l], init)
            if shared is not None:
                shared[key] = W
        g.bind_dense((0, 0, l, 0), W, act=act_hidden if l < L - 1 else act_out, dtype=dtype)
    return g


def timed_repeats(torch, stream, step, est_ms, min_ms=20.0, repeats=5, min_steps=50):
    """Median-of-repeats timing: each repeat runs enough back-to-back steps to
    cover at least `min_ms` of GPU work (HIP events on the launch stream)."""
    n = max(min_steps, int(min_ms / max(est_ms, 1e-4)) + 1)
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    per = []
    i = 0
    for _ in range(repeats):
        torch.cuda.synchronize()
        t0.record(stream)
        for _ in range(n):
            step(i)
            i += 1
        t1.record(stream)
        torch.cuda.synchronize()
        per.append(t0.elapsed_time(t1) / n)
    per.sort()
    return {"ms_per_step": per[len(per) // 2], "ms_min": per[0], "ms_repeats": per,
            "steps_per_repeat": n, "repeats": repeats}


def time_volume_forward(torch, P, widths, dtype, batch, steps, warmup, seed, init="normal", act_out=-1):
    """Forward of a Dense chain on device buffers; rotates grid copies so the
    working set exceeds the MALL.  Median of 5 repeats of >= 20 ms each."""
    import numpy as np
    rng = np.random.default_rng(seed)
    bits = P.dtype_bits(dtype)
    wbytes = sum(widths[i] * widths[i + 1] * bits // 8 for i in range(len(widths) - 1))
    copies = max(2, -(-MALL_BYTES // wbytes))
    shared = {}
    grids = [_grid(P, widths, dtype, batch, rng, init, act_out=act_out, shared=shared) for _ in range(copies)]
    dev = torch.device("cuda:0")
    x = torch.randn((batch, widths[0]), device=dev)
    y = torch.empty((batch, widths[-1]), device=dev)
    stream = torch.cuda.Stream(device=dev)
    sh = stream.cuda_stream

    def step(i):
        P.check(P.lib().welvet_hip_volume_forward_device(
            grids[i % copies].h, x.data_ptr(), widths[0], y.data_ptr(), widths[-1], sh))

    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for i in range(warmup):
        step(i)
    t1.record(stream)
    torch.cuda.synchronize()
    est = t0.elapsed_time(t1) / max(1, warmup)
    r = timed_repeats(torch, stream, step, est, min_steps=steps)
    ms = r["ms_per_step"]
    for g in grids:
        g.close()
    flops = 2.0 * batch * sum(widths[i] * widths[i + 1] for i in range(len(widths) - 1))
    return {"widths": widths, "weight_dtype": P.DTYPE_NAMES[dtype], "batch": batch, "init": init,
            "packed_bytes": wbytes, "weight_copies": copies, **r,
            "hbm_gbs": wbytes / (ms * 1e-3) / 1e9, "tflops": flops / (ms * 1e-3) / 1e12}


def time_swiglu_forward(torch, P, inn, inter, dtype, batch, steps, warmup, seed):
    """Resident SwiGLU forward (Gate and Up GEMVs/GEMMs, op_swiglu, Down) on
    device buffers; rotates mounted copies so the working set exceeds the
    MALL."""
    import numpy as np
    rng = np.random.default_rng(seed)
    wbytes = 3 * inn * inter * P.dtype_bits(dtype) // 8
    copies = max(2, -(-MALL_BYTES // wbytes))
    G, U, D = (_weights(rng, *shape, "normal") for shape in ((inter, inn), (inter, inn), (inn, inter)))
    layers = [P.SwigluSession(G, U, D, batch, dtype) for _ in range(copies)]
    del G, U, D
    dev = torch.device("cuda:0")
    x = torch.randn((batch, inn), device=dev)
    h = torch.empty((batch, inter), device=dev)
    y = torch.empty((batch, inn), device=dev)
    stream = torch.cuda.Stream(device=dev)
    sh = stream.cuda_stream

    def step(i):
        P.check(layers[i % copies].forward_device(x.data_ptr(), h.data_ptr(), y.data_ptr(), sh))

    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for i in range(warmup):
        step(i)
    t1.record(stream)
    torch.cuda.synchronize()
    r = timed_repeats(torch, stream, step, t0.elapsed_time(t1) / max(1, warmup), min_steps=steps)
    ms = r["ms_per_step"]
    for L in layers:
        L.close()
    flops = 2.0 * batch * 3 * inn * inter
    return {"shape": [inn, inter], "weight_dtype": P.DTYPE_NAMES[dtype], "batch": batch,
            "packed_bytes": wbytes, "weight_copies": copies, **r,
            "hbm_gbs": wbytes / (ms * 1e-3) / 1e9, "tflops": flops / (ms * 1e-3) / 1e12}


def time_volume_train(torch, P, dims, widths, dtype, batch, steps, seed, lr=1e-3):
    """training::step_dense on device buffers (forward, MSE vs N(0,1) targets,
    backward, SGD with re-encode); one synchronisation per step."""
    import numpy as np
    rng = np.random.default_rng(seed)
    D, R, Cc, L = dims
    g = P.Grid(D, R, Cc, L, batch)
    n_layers = 0
    for z in range(D):
        for yy in range(R):
            for xx in range(Cc):
                for l in range(L):
                    k = n_layers
                    W = _weights(rng, widths[k + 1], widths[k], "normal")
                    last = k == len(widths) - 2
                    g.bind_dense((z, yy, xx, l), W, act=-1 if last else 0, dtype=dtype)
                    n_layers += 1
    dev = torch.device("cuda:0")
    x = torch.from_numpy(rng.standard_normal((batch, widths[0]), dtype=np.float32)).to(dev)
    t = torch.from_numpy(rng.standard_normal((batch, widths[-1]), dtype=np.float32)).to(dev)
    stream = torch.cuda.Stream(device=dev)
    loss = P.C.c_double()
    codes = []

    def step():
        st = P.lib().welvet_hip_volume_train_step_device(
            g.h, x.data_ptr(), widths[0], t.data_ptr(), widths[-1], lr, P.C.byref(loss),
            stream.cuda_stream)
        # a non-finite gradient (a diverging deep quantized stack) is the
        # reference's own error: the step ran, SGD was skipped; report it
        if st.code not in (0, 1, 2) or (st.code and b"nonfinite" not in st.message
                                          and b"finite f32" not in st.message):
            P.check(st)
        codes.append(st.code)

    torch.cuda.synchronize()
    step()  # first step allocates dW and gradient buffers
    first_loss = loss.value
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    g.close()
    mac = sum(widths[i] * widths[i + 1] for i in range(len(widths) - 1))
    # executed: forward, dX and dW of every layer (2 flops per MAC each),
    # except the first layer's dX, which the step never computes (its input
    # gradient is not returned)
    flops = 6.0 * batch * mac - 2.0 * batch * widths[0] * widths[1]
    return {"widths": widths if len(widths) < 8 else f"{len(widths) - 1} x {widths[1]}",
            "weight_dtype": P.DTYPE_NAMES[dtype], "batch": batch, "steps": steps, "lr": lr,
            "ms_per_step": ms, "gflop_per_step": flops / 1e9,
            "tflops": flops / (ms * 1e-3) / 1e12,
            "loss_first": first_loss, "loss_last": loss.value,
            "sgd_skipped_nonfinite": sum(1 for c in codes if c)}


# untimed forwards before each config-2/3 leg's timed ones (the GPU clocks
# settle: batch-1 steps drift down by ~3% over the first few hundred)
FWD_WARMUP = 500


def c1_cpu_baseline(runs: int = 200):
    """Config 1 as the reference runs it, on the host: the oracle's scalar port
    of the CPU path (per-element decode switch + f64 dot, tanh) for the 1x1x1
    volume's Dense 512 -> 512 Float32 at batch 1, one thread; median of `runs`
    forwards after one warm-up."""
    import numpy as np
    from oracle import Oracle

    O = Oracle()
    rng = np.random.default_rng(0x5EED0000)
    W = _weights(rng, 512, 512, "uniform05")
    x = rng.standard_normal((1, 512), dtype=np.float32)
    raw, scale = O.pack(1, W)
    O.forward_native(1, raw, scale, x, 512, 512, 3, threads=1)
    t = []
    for _ in range(runs):
        t0 = time.perf_counter()
        O.forward_native(1, raw, scale, x, 512, 512, 3, threads=1)
        t.append(time.perf_counter() - t0)
    t.sort()
    return {"ms_per_step": round(t[len(t) // 2] * 1e3, 4), "cores": 1, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"median of {runs} forwards after one warm-up (per-element decode switch, "
                      "f64 dot, tanh; 1 thread)"}


def run_configs(torch, P, only=("c1", "c2", "c3", "c4", "c5"), cpu=True, c5_dtypes=range(34)):
    """BASELINE configs 1-5; `only` selects configs by name prefix.  Config 1
    is the reference's own CPU case: the GPU volume forward is timed, and with
    `cpu` the CPU path on the host beside it."""
    out = {}
    seed = 0x5EED0000
    if "c1" in only:
        # 1x1x1 volume, Dense 512 -> 512 Float32, batch 1, tanh, W ~ U(-0.05, 0.05)
        leg = time_volume_forward(torch, P, [512, 512], 1, 1, 100, FWD_WARMUP, seed, init="uniform05",
                                  act_out=3)
        if cpu:
            leg["cpu_baseline"] = c1_cpu_baseline()
            leg["gpu_speedup_vs_cpu_path"] = round(leg["cpu_baseline"]["ms_per_step"] / leg["ms_per_step"], 1)
        out["c1_f32_512x512_b1_tanh"] = leg
    for name, dt in (("e4m3", 4), ("e5m2", 5)) if "c2" in only else ():
        for b in (1, 32):
            out[f"c2_{name}_4096x4096_b{b}"] = time_volume_forward(
                torch, P, [4096, 4096], dt, b, 100, FWD_WARMUP, seed + 1)
    if "c2" in only:
        # the batch-1 legs against one launch's read of the same 16.8 MB
        fl = read_floor(torch, P, 4096 * 4096, 200, FWD_WARMUP)
        out["c2_read_floor_4096x4096"] = {"us": round(fl["us"], 3), "gbs": round(fl["gbs"], 1),
                                          "kernel": fl["kernel"]}
        for name in ("e4m3", "e5m2"):
            leg = out[f"c2_{name}_4096x4096_b1"]
            leg["frac_of_read_floor"] = round(fl["us"] / (leg["ms_per_step"] * 1e3), 4)
        print(f"# c2 read floor (16.8 MB): {fl['us']:.2f} us/launch  {fl['gbs']:.0f} GB/s",
              file=sys.stderr, flush=True)
    for name, dt, init in (("nf4", 26, "normal"), ("fp4", 16, "normal"), ("fp4_u6", 16, "uniform6")) \
            if "c3" in only else ():
        for b in (1, 8, 64):
            out[f"c3_{name}_4096-11008-4096_b{b}"] = time_volume_forward(
                torch, P, [4096, 11008, 4096], dt, b, 50, FWD_WARMUP, seed + 2, init=init)
    for name, dt in (("nf4", 26), ("fp4", 16)) if "c3" in only else ():
        for b in (1, 8, 64):  # the config-3 shape as one SwiGLU (Gate, Up, Down)
            out[f"c3_swiglu_{name}_4096x11008_b{b}"] = time_swiglu_forward(
                torch, P, 4096, 11008, dt, b, 50, FWD_WARMUP, seed + 5)
    for name, dt in (("int8", 9), ("e4m3", 4)) if "c4" in only else ():
        out[f"c4_{name}_2048-8192-2048_b256"] = time_volume_train(
            torch, P, (1, 1, 2, 1), [2048, 8192, 2048], dt, 256, 10, seed + 3)
    c5, skipped = {}, []
    for dt in c5_dtypes if "c5" in only else ():
        # 10 timed steps per dtype (about 5 ms; mounting the 32 stores dominates the leg)
        r = time_volume_train(torch, P, (2, 2, 2, 4), [1024] * 33, dt, 16, 10, seed + 4)
        c5[P.DTYPE_NAMES[dt]] = round(r["ms_per_step"], 4)
        if r["sgd_skipped_nonfinite"]:
            skipped.append(P.DTYPE_NAMES[dt])
    if "c5" in only:
        out["c5_2x2x2x4_1024_b16_ms_per_step"] = c5
        out["c5_nonfinite_gradient_dtypes"] = skipped
    for k, v in out.items():
        if isinstance(v, dict) and "ms_per_step" in v:
            print(f"# {k}: {v['ms_per_step'] * 1e3:.1f} us/step  {v.get('tflops', 0):.2f} TFLOP/s",
                  file=sys.stderr, flush=True)
    return out


def calibrate_copy(torch, mib: int = 256, launches: int = 5):
    """Element-wise copy out = in * 1 of `mib` MiB, `launches` times: each launch
    reads and writes exactly mib MiB, the yardstick for FETCH_SIZE/WRITE_SIZE."""
    dev = torch.device("cuda:0")
    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(launches):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    print(json.dumps({"calibrate_copy": {"bytes_read": n * 4, "bytes_written": n * 4,
                                         "launches": launches}}), flush=True)


def run_wire():
    """The wire tool's own --bench framing, one tool process per wire: host
    buffers in and out through the C ABI (PCIe-inclusive), the reference's
    warm-ups.  WVD3 at the headline shape (mount = encode; execute = copy x
    in, forward, copy pre/post out) and WVN1 at config 4 (each step rebuilds
    the grid from the wire's f32 weights, as the reference's tool does)."""
    import numpy as np
    import wire

    rng = np.random.default_rng(0x5EED00F0)
    res = {}
    W = rng.normal(0, 0.02, (OUT, IN)).astype(np.float32)
    for name, dtype, batch in (("wvd3_fp8e4m3_b1", 4, 1), ("wvd3_nf4_b1", 26, 1),
                               ("wvd3_fp8e4m3_b64", 4, 64)):
        x = rng.normal(0, 1, (batch, IN)).astype(np.float32)
        iters = 200
        rc, out, err = wire.run(wire.wvd(W, x, dtype=dtype), f"--bench={iters}", timeout=300)
        if rc:
            raise RuntimeError(f"wire {name}: {err}")
        b = wire.read_bench(wire.Reader(out))
        res[name] = {"mount_ms": round(b["mount_ns"] / 1e6, 3),
                     "exec_us": round(b["exec_ns"] / iters / 1e3, 2), "iters": iters}
        print(f"# wire {name}: mount {res[name]['mount_ms']} ms, execute {res[name]['exec_us']} us",
              file=sys.stderr, flush=True)
    cells = {(0, 0, 0, 0): (_weights(rng, 8192, 2048, "normal"), 0, 9, None),
             (0, 0, 1, 0): (_weights(rng, 2048, 8192, "normal"), -1, 9, None)}
    x = rng.normal(0, 1, (256, 2048)).astype(np.float32)
    t = rng.normal(0, 1, (256, 2048)).astype(np.float32)
    iters = 10
    rc, out, err = wire.run(wire.wvn((1, 1, 2, 1), 256, cells, x, t, 1e-3), f"--bench={iters}",
                            timeout=300)
    if rc:
        raise RuntimeError(f"wire wvn1: {err}")
    b = wire.read_bench(wire.Reader(out))
    res["wvn1_c4_int8_b256"] = {"step_ms": round(b["ns"] / iters / 1e6, 3), "iters": iters}
    print(f"# wire wvn1_c4_int8_b256: {res['wvn1_c4_int8_b256']['step_ms']} ms per rebuild + step",
          file=sys.stderr, flush=True)
    return res


def pywelvet_name(dtype):
    import pywelvet
    return pywelvet.DTYPE_NAMES[dtype]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=2000,
                    help="untimed steps per case before the timed ones (the GPU clocks settle)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default="", help="comma list of cases: fp8b1,nf4b1,fp8b64,nf4b64 (the "
                    "default set), fp8b2,fp8b4,nf4b2,nf4b4 (the batch 2-4 GEMV, only when named)")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip BASELINE configs 1-5 (reported under config_results)")
    ap.add_argument("--configs", default="c1,c2,c3,c4,c5",
                    help="comma list of the BASELINE configs to run: c1,c2,c3,c4,c5")
    ap.add_argument("--c5-dtypes", default="",
                    help="comma list of dtype names for config 5 (default: all 34)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only a plain copy kernel of known size (for scaling HBM counters)")
    ap.add_argument("--cpu-configs", action="store_true",
                    help="also time BASELINE configs 2-5 on the host with the oracle (a few "
                         "minutes of CPU work; not in the default run)")
    ap.add_argument("--wire", action="store_true",
                    help="run only the wire tool's --bench framing (host buffers; not the headline)")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs on one GPU only (no multi-GPU path); use --gpus 1",
              file=sys.stderr)
        sys.exit(2)
    import torch
    if a.calibrate_copy:
        calibrate_copy(torch)
        return
    if a.wire:
        print(json.dumps({"wire": run_wire()}), flush=True)
        return
    import pywelvet

    pywelvet.init()
    cases = [("fp8b1", 4, 1), ("nf4b1", 26, 1), ("fp8b64", 4, 64), ("nf4b64", 26, 64)]
    if a.only:
        keep = set(a.only.split(","))
        extra = [("fp8b2", 4, 2), ("fp8b4", 4, 4), ("nf4b2", 26, 2), ("nf4b4", 26, 4)]
        cases = [c for c in cases + extra if c[0] in keep]
    results = {}
    for i, (name, dtype, batch) in enumerate(cases):
        results[name] = run_case(torch, pywelvet, dtype, batch, a.steps, a.warmup, 0x5EED0000 + i)
        print(f"# {name}: {results[name]['hbm_gbs']:.1f} GB/s  {results[name]['tflops']:.2f} TFLOP/s"
              f"  {results[name]['ms_per_step'] * 1e3:.2f} us/step", file=sys.stderr, flush=True)
    prim = results.get("fp8b1") or next(iter(results.values()))
    for r in results.values():
        annotate_roofline(r)
    # One step of a batch 1-4 case is exactly one GEMV launch, so the timed
    # region's mean step time is that kernel's mean launch duration.
    if prim["bound"] == "hbm":
        ach = prim["hbm_gbs"]
        roof = {"bound": "hbm", "achieved": ach, "peak": HBM_PEAK, "unit": "GB/s",
                "frac": ach / HBM_PEAK, "traffic": measured_traffic(prim_name(results, prim))}
        fl = read_floor(torch, pywelvet, prim["packed_bytes"], a.steps, min(a.warmup, 500))
        fl["frac_of_floor"] = ach / fl["gbs"]
        roof["read_floor"] = fl
        print(f"# read floor ({fl['bytes']} B): {fl['gbs']:.1f} GB/s  {fl['us']:.2f} us/launch",
              file=sys.stderr, flush=True)
    else:
        roof = {"bound": "mfma", "achieved": prim["executed_tflops"], "peak": prim["peak_tflops"],
                "unit": "TFLOP/s", "frac": prim["roofline_frac"],
                "traffic": measured_traffic(prim_name(results, prim)),
                "fp32_equivalent": {"achieved": prim["tflops"], "peak": FP32_MFMA_PEAK,
                                    "frac": prim["tflops"] / FP32_MFMA_PEAK}}
    line = {
        "metric": METRIC, "value": prim["hbm_gbs"] if prim["bound"] == "hbm" else prim["tflops"],
        "unit": "GB/s" if prim["bound"] == "hbm" else "TFLOP/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": prim["ms_per_step"], "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: W ~ N(0,0.02) encoded to the native dtype, x ~ N(0,1)",
        "config": {"workload": f"dense_fwd_{prim['case']}", "in": IN, "out": OUT,
                   "batch": prim["batch"], "weight_dtype": prim["weight_dtype"],
                   "weight_copies": prim["weight_copies"], "act": "linear"},
        "roofline": roof,
        "results": {k: {kk: (round(vv, 6) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                    for k, v in results.items()},
    }
    if not a.no_configs:
        c5 = [pywelvet.DTYPE_NAMES.index(n) for n in a.c5_dtypes.split(",")] if a.c5_dtypes else range(34)
        line["config_results"] = run_configs(torch, pywelvet, tuple(a.configs.split(",")), cpu=not a.no_cpu,
                                             c5_dtypes=c5)
    if not a.no_cpu:
        first = 26 if prim["weight_dtype"] == "nf4" else 4
        line["cpu_baseline"] = cpu_baseline((first, 30 - first), prim["batch"])
    if a.cpu_configs:
        line["cpu_config_baselines"] = cpu_config_baselines()
    print(json.dumps(line), flush=True)


def annotate_roofline(r):
    """Roofline fraction of one case.  Batch 1: packed-weight bytes against the
    HBM peak.  Batched: the flops the MFMA pipe executes against that
    instruction's dense peak.  The split-x GEMM (FP8, Int8, FP4, NF4 weights)
    forms each fp32 product from exact bf16 products, 3 per product (x split
    into three parts), 6 for NF4 (its table values are split too), on the
    bf16 MFMA; other formats run the fp32 MFMA.  The fp32-equivalent rate
    (2*B*K*N / time) is kept beside it."""
    r["hbm_frac"] = r["hbm_gbs"] / HBM_PEAK
    if r["batch"] <= 4:
        r["roofline_frac"] = r["hbm_frac"]
        r["bound"] = "hbm"
        return
    r["bound"] = "mfma"
    if r["weight_dtype"] in SPLIT_X_DTYPES:
        mult = 6 if r["weight_dtype"] == "nf4" else 3
        r["gemm"] = (f"split-x bf16 MFMA: x = hi + mid + lo exactly, {mult} exact bf16 products "
                     f"per fp32 product, fp32 accumulate")
        r["executed_tflops"] = mult * r["tflops"]
        r["peak_tflops"] = BF16_MFMA_PEAK
    else:
        r["gemm"] = "fp32 MFMA (v_mfma_f32_32x32x2f32)"
        r["executed_tflops"] = r["tflops"]
        r["peak_tflops"] = FP32_MFMA_PEAK
    r["roofline_frac"] = r["executed_tflops"] / r["peak_tflops"]
    r["fp32_equivalent_frac"] = r["tflops"] / FP32_MFMA_PEAK


def prim_name(results, prim):
    return next(k for k, v in results.items() if v is prim)


def measured_traffic(case: str):
    """HBM bytes per launch of the case's kernel from the committed rocprofv3
    --pmc FETCH_SIZE / WRITE_SIZE passes, each scaled by what the counter reads
    for a copy kernel of known size (profiles/hbm_traffic.json); None when that
    case was not profiled."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)["cases"][case]
    except (OSError, KeyError, ValueError):
        return None
    return rec["bytes_per_launch"]


if __name__ == "__main__":
    main()
