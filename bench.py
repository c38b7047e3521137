"""Throughput of the gradtrack training step (forward + backward + Adam::step)
on one MI355X, on BASELINE config 5: batch 8192, six Linear(4096, 4096) layers
with bias, ReLU after layers 1-5, MSE loss, fp32, Adam(lr 1e-3).

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--config c5|c4|c1|c2|c3]
                    [--no-cpu-baseline] [--cpu-sample-rows R] [--graph]

Prints one JSON line.  `value` is steps/s of config 5 measured over exactly K
steps with all inputs resident in HBM; without --config the same line carries
every other BASELINE config under "configs" (each with its own steps, roofline
and CPU baseline), measured in the same run.  The timed region runs
uninstrumented.  `roofline` is the roofline of the dominant kernel class,
measured over a second pass of the same K steps in which every launch of that
class carries kernel-attached events (ts_hip_timing_begin/end: the events ride
in the kernels' own dispatches, so a launch's time is its kernels' time, as
rocprofv3 reports it): for the MLP configs (c1, c4, c5) the fp32-MFMA roofline
of the GEMMs (algorithmic FLOPs of every GEMM launch over their summed kernel
time); for the elementwise chain (c2) and Adam alone (c3) the HBM roofline of
the bandwidth-bound kernels (algorithmic bytes over kernel time).  `cpu_baseline` times the CPU
restatement of the reference (oracle/, one core) on a bounded sample of the
same step and extrapolates to steps/s.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import pathlib
import sys
import time

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_FP32_MFMA_TFLOPS = 157.3   # MI355X dense fp32 matrix peak (published)
PEAK_HBM_GBS = 8000.0           # MI355X HBM3E (published)

CONFIGS = {
    # name: (batch, layer widths, init)
    "c5": (8192, [4096] * 7, "normal"),
    "c4": (1024, [784, 1024, 10], "kaiming"),
    "c1": (32, [784, 128], "readme"),
}
CHAIN_N = 1 << 26        # config 2: elementwise autograd chain length
ADAM_P = 1 << 28         # config 3: Adam alone, parameter count
# config 2's algorithmic bytes per element and step: the fused floor, each of a, b, c read once and
# ga, gb, gc written once (the roofline's `achieved` is taken against it); the reference's op-by-op
# sequence moves 148 (forward 60 + backward 88)
CHAIN_BYTES_PER_ELEM = 24
# the configs measured after the headline in a default run: (name, timed steps, warm-up steps)
OTHER_CONFIGS = (("c1", 200, 10), ("c4", 100, 5), ("c2", 20, 3), ("c3", 100, 3))
ADAM_BYTES_PER_PARAM = 28    # read p, g, m, v; write p, m, v


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_params(TS, widths, init, rng):
    ps = []
    for i in range(len(widths) - 1):
        fan_in, fan_out = widths[i], widths[i + 1]
        if init == "normal":        # N(0, 1/fan_in)
            w = rng.standard_normal((fan_in, fan_out), dtype=np.float32) * np.float32(1.0 / np.sqrt(fan_in))
        elif init == "kaiming":     # Kaiming-uniform U(+-sqrt(6/fan_in))
            bound = np.float32(np.sqrt(6.0 / fan_in))
            w = rng.uniform(-bound, bound, (fan_in, fan_out)).astype(np.float32)
        else:                       # README: W ~ N(0, 1)
            w = rng.standard_normal((fan_in, fan_out), dtype=np.float32)
        ps.append(TS.Tensor.from_slice(w, w.shape).with_requires_grad())
        ps.append(TS.Tensor.zeros([fan_out]).with_requires_grad())
    return ps


def forward_loss(x, t, ps, readme: bool):
    h = x
    n = len(ps) // 2
    for i in range(n):
        h = h.matmul(ps[2 * i]).add_tensor(ps[2 * i + 1])
        if i < n - 1 or readme:
            h = h.relu()
    if readme:                                   # README.md:71-79: loss = sum(relu(xW + b))
        return h.sum()
    return h.sub_tensor(t).pow_scalar(2.0).mean()   # feedforward_network.rs:478-479


def step_flops(batch, widths, readme):
    """Algorithmic GEMM FLOPs of one step: forward, dW for every layer, dX for
    every layer but the first (x does not require grad)."""
    f = 0
    for i in range(len(widths) - 1):
        mnk = 2.0 * batch * widths[i] * widths[i + 1]
        f += mnk * (3 if i > 0 else 2)
    return f


def pmc_traffic(cfg_name: str):
    """HBM bytes per launch of the roofline's kernel (the GEMMs; Adam for config
    3) from the committed rocprofv3 --pmc summary of this workload (FETCH_SIZE and
    WRITE_SIZE runs, each scaled by the copy-kernel calibration recorded in the
    same file), or None."""
    import re

    kernel = {"c3": "adam", "c2": "map"}.get(cfg_name, "gemm")
    path = ROOT / "profiles" / f"{cfg_name}_{kernel}_pmc.md"
    if not path.exists():
        return None, None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+-]+)", path.read_text())
    return (float(m.group(1)), str(path.relative_to(ROOT))) if m else (None, None)


def host_info():
    """The host the CPU baseline ran on: CPU model, logical cores present and
    cores this process may use (the baseline itself uses one)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "host_cores": os.cpu_count(), "usable_cores": len(os.sched_getaffinity(0))}


def cpu_baseline(cfg_name: str, sample_rows: int):
    """Single-core CPU restatement (oracle/) of one MLP step of `cfg_name`,
    timed on a bounded sample and scaled, layer by layer: the forward product
    and the dX product on `sample_rows` of the batch rows, the dW product on
    `sample_rows` of its output rows; the elementwise and reduction passes on
    1/64 of each activation's rows; Adam on 1/16 of the parameters."""
    import oracle as O

    batch, widths, init = CONFIGS[cfg_name]
    readme = init == "readme"
    rng = np.random.default_rng(7)
    layers = len(widths) - 1
    R = min(sample_rows, batch)
    rows = max(1, batch // 64)  # activation rows of the elementwise sample
    timings = {"gemm_s": 0.0, "elementwise_s": 0.0}

    product_s = {}  # each product timed once per shape: (kind, fan_in, fan_out) -> seconds per step

    def product(kind, fi, fo):
        key = (kind, fi, fo)
        if key not in product_s:
            W = rng.standard_normal((fi, fo), dtype=np.float32)
            if kind == "dW":                                   # X^T.dY on up to sample_rows output rows
                Rw = min(sample_rows, fi)
                Xt = rng.standard_normal((batch, Rw), dtype=np.float32)
                dY = rng.standard_normal((batch, fo), dtype=np.float32)
                t0 = time.perf_counter(); O.gemm_f32(Xt, dY, ta=True)
                product_s[key] = (time.perf_counter() - t0) * fi / Rw
            elif kind == "dX":                                 # dY.W^T on R batch rows
                dY = rng.standard_normal((R, fo), dtype=np.float32)
                t0 = time.perf_counter(); O.gemm_f32(dY, W, tb=True)
                product_s[key] = (time.perf_counter() - t0) * batch / R
            else:                                              # X.W on R batch rows
                X = rng.standard_normal((R, fi), dtype=np.float32)
                t0 = time.perf_counter(); O.gemm_f32(X, W)
                product_s[key] = (time.perf_counter() - t0) * batch / R
        return product_s[key]

    for i in range(layers):
        fi, fo = widths[i], widths[i + 1]
        timings["gemm_s"] += product("fwd", fi, fo) + product("dW", fi, fo) + (product("dX", fi, fo) if i > 0 else 0.0)

        n = rows * fo
        a = rng.standard_normal(n, dtype=np.float32)
        b = rng.standard_normal(n, dtype=np.float32)
        bias = rng.standard_normal(fo, dtype=np.float32)
        t0 = time.perf_counter()
        z = O.bias_add(a.reshape(-1, fo), bias)            # forward bias add
        if i < layers - 1 or readme:
            r = O.relu(z)                                  # forward relu
            O.relu_bwd(r, b)                               # relu mask gradient
        O.sum_dim0(b.reshape(-1, fo))                      # bias gradient
        if i > 0:
            O.add(a, b)                                    # gradient accumulation
        if i == layers - 1:
            if readme:
                O.mean(a); O.fill(n, 1.0)                  # sum forward, its backward fill
            else:
                d = O.sub(a, b); p2 = O.pow2(d); O.mean(p2)    # MSE forward
                O.pow_bwd(d, b, 2.0); O.fill(n, 1.0)           # MSE backward
        timings["elementwise_s"] += (time.perf_counter() - t0) * batch / rows

    P = sum(widths[i] * widths[i + 1] + widths[i + 1] for i in range(layers))
    ns = max(1, P // 16)
    p = rng.standard_normal(ns, dtype=np.float32)
    g = rng.standard_normal(ns, dtype=np.float32) * np.float32(0.1)
    m = np.zeros(ns, np.float32)
    v = np.zeros(ns, np.float32)
    t0 = time.perf_counter()
    O.adam_step(p, g, m, v, 1)
    timings["adam_s"] = (time.perf_counter() - t0) * P / ns
    total = sum(timings.values())
    sample = (f"per layer: forward and dX products on {R} of {batch} rows, dW on up to {sample_rows} of its "
              f"output rows, elementwise/reduction passes on {rows} of {batch} rows, Adam on 1/16 of "
              f"{P} params; scaled to one full step ({total:.2f} s)")
    return {"value": 1.0 / total, "unit": "steps/s", "cores": 1, "kind": "port",
            "sample": sample, "breakdown_s": {k: round(v, 4) for k, v in timings.items()}, "host": host_info()}


def cpu_baseline_chain(sample: int):
    """Config 2 on the CPU restatement of the engine (oracle/gradtrack.py): the
    forward chain and its backward on `sample` elements, scaled to 2^26."""
    from oracle import gradtrack as G

    rng = np.random.default_rng(7)
    a = rng.standard_normal(sample, dtype=np.float32)
    b = rng.standard_normal(sample, dtype=np.float32)
    c = rng.uniform(0.5, 2.0, sample).astype(np.float32)
    A, Bt, C = (G.OTensor(v.copy(), True) for v in (a, b, c))
    t0 = time.perf_counter()
    loss = A.add_tensor(Bt).mul_tensor(C).sub_tensor(A.div_tensor(C)).relu().sum()
    loss.backward()
    dt = (time.perf_counter() - t0) * (CHAIN_N / sample)
    G.clear_gradients()
    return {"value": 1.0 / dt, "unit": "steps/s", "cores": 1, "kind": "port",
            "sample": f"forward chain + backward through the restated engine on {sample} of {CHAIN_N} "
                      f"elements, scaled to one full step ({dt:.2f} s)", "host": host_info()}


def cpu_baseline_adam(sample: int):
    """Config 3 on the CPU restatement of Adam::step (oracle/): one step on
    `sample` parameters, scaled to 2^28."""
    import oracle as O

    rng = np.random.default_rng(7)
    p = rng.standard_normal(sample, dtype=np.float32)
    g = rng.standard_normal(sample, dtype=np.float32) * np.float32(0.1)
    m = np.zeros(sample, np.float32)
    v = np.zeros(sample, np.float32)
    t0 = time.perf_counter()
    O.adam_step(p, g, m, v, 1)
    dt = (time.perf_counter() - t0) * (ADAM_P / sample)
    return {"value": 1.0 / dt, "unit": "steps/s", "cores": 1, "kind": "port",
            "sample": f"one Adam step on {sample} of {ADAM_P} parameters, scaled ({dt:.2f} s)", "host": host_info()}


def run_bandwidth(TS, cfg: str, steps: int, warmup: int, cpu: bool) -> dict:
    """Configs 2 and 3: the HBM-bound paths, each step timed like the MLP step."""
    rng = np.random.default_rng(0)
    if cfg == "c2":
        n = CHAIN_N
        log(f"config c2: chain over {n} elements; uploading inputs")
        a = TS.Tensor.from_slice(rng.standard_normal(n, dtype=np.float32), [n]).with_requires_grad()
        b = TS.Tensor.from_slice(rng.standard_normal(n, dtype=np.float32), [n]).with_requires_grad()
        c = TS.Tensor.from_slice(rng.uniform(0.5, 2.0, n).astype(np.float32), [n]).with_requires_grad()

        def step():
            loss = a.add_tensor(b).mul_tensor(c).sub_tensor(a.div_tensor(c)).relu().sum()
            loss.backward()
            TS.clear_gradients()      # leaves start every step without a gradient
            return loss
        work = float(CHAIN_BYTES_PER_ELEM) * n
        classes = ("elementwise", "reduction")
        workload = ("BASELINE config 2: elementwise autograd chain over 2^26 fp32, a,b ~N(0,1), c ~U(0.5,2), "
                    "y=relu((a+b)*c - a/c), loss=sum(y), backward to a,b,c")
        data = "synthetic (numpy default_rng(0))"
    else:
        n = ADAM_P
        log(f"config c3: Adam on {n} parameters; p ~N(0,1), g ~N(0,1e-2) (sigma 0.1) from numpy, uploaded")
        rng = np.random.default_rng(0)
        pv = rng.standard_normal(n, dtype=np.float32)
        p = TS.Tensor.from_slice(pv, [n]).with_requires_grad()
        del pv
        gv = rng.standard_normal(n, dtype=np.float32)
        gv *= np.float32(0.1)
        g = TS.Tensor.from_slice(gv, [n])
        del gv
        p.set_grad(g)
        opt = TS.Adam.with_learning_rate(1e-3)
        opt.add_parameter(p)

        def step():
            opt.step([p])
            return None
        work = float(ADAM_BYTES_PER_PARAM) * n
        classes = ("adam",)
        workload = ("BASELINE config 3: Adam::step alone on 2^28 fp32 params, grads ~N(0, 1e-2) set once, "
                    "m=v=0 initially, lr=1e-3, betas (0.9, 0.999), eps 1e-8")
        data = "synthetic (numpy default_rng(0): p ~N(0,1), g = 0.1 * N(0,1), float32)"

    for i in range(warmup):
        step()
    TS.synchronize()
    t0 = time.perf_counter()      # the timed region: uninstrumented
    for _ in range(steps):
        step()
    TS.synchronize()
    t1 = time.perf_counter()
    wall_ms = (t1 - t0) * 1000.0 / steps
    # Roofline pass: the same K steps again with kernel-attached events on
    # every launch (each launch's own kernel time, as rocprofv3 reports it).
    TS.Profile.reset()
    TS.Profile.enable(True)
    for _ in range(steps):
        step()
    TS.synchronize()
    TS.Profile.enable(False)
    names = {"elementwise": TS.Profile.ELEMENTWISE, "reduction": TS.Profile.REDUCTION, "adam": TS.Profile.ADAM}
    prof = {k: TS.Profile.read(names[k]) for k in classes}
    kern_ms = sum(v["ms"] for v in prof.values())
    kern_work = sum(v["work"] for v in prof.values())
    # achieved: the algorithmic bytes (config 2: the fused floor) over the kernels' time
    achieved = work * steps / (kern_ms * 1e-3) / 1e9 if kern_ms > 0 else 0.0
    kernels = {k: {"ms_per_step": round(v["ms"] / steps, 3), "launches_per_step": v["launches"] // steps,
                   "GB/s": round(v["work"] / (v["ms"] * 1e-3) / 1e9, 1) if v["ms"] > 0 else 0.0}
               for k, v in prof.items()}
    # HBM bytes per launch of the step's pass from the committed counters
    traffic, traffic_src = pmc_traffic(cfg)
    result = {
        "metric": {"c2": "fwd+bwd steps/sec of the elementwise chain (1 GPU); % HBM GB/s roofline",
                   "c3": "Adam::step steps/sec (1 GPU); % HBM GB/s roofline"}[cfg],
        "value": round(1000.0 / wall_ms, 4),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(wall_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": data,
        "config": {"workload": workload, "elements": n, "algorithmic_bytes_per_step": work,
                   "bytes_moved_per_step": round(kern_work / steps, 1)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": traffic, "traffic_source": traffic_src,
                     "kernel": " + ".join(classes) + " kernels of the step (every launch of the roofline pass: "
                               f"the same {steps} steps again with kernel-attached events)"},
        "kernels": kernels,
    }
    if cpu:
        log("timing the CPU baseline (oracle port, one core, bounded sample)")
        result["cpu_baseline"] = (cpu_baseline_chain(CHAIN_N) if cfg == "c2"
                                  else cpu_baseline_adam(1 << 26))
    else:
        result["cpu_baseline"] = None
    return result


def run_mlp(TS, hip, hip_check, cfg: str, steps: int, warmup: int, cpu: bool, cpu_rows: int, graph: bool) -> dict:
    """An MLP config (c1, c4, c5): W untimed warm-up steps, then exactly K
    steps between two device synchronisations, the GEMMs timed with events."""
    batch, widths, init = CONFIGS[cfg]
    readme = init == "readme"
    rng = np.random.default_rng(0)
    log(f"config {cfg}: batch {batch}, widths {widths}; uploading inputs")
    ps = make_params(TS, widths, init, rng)
    x = TS.Tensor.from_slice(rng.standard_normal((batch, widths[0]), dtype=np.float32), [batch, widths[0]])
    t = TS.Tensor.from_slice(rng.standard_normal((batch, widths[-1]), dtype=np.float32), [batch, widths[-1]])
    opt = TS.Adam.with_learning_rate(1e-3)
    opt.add_parameters(ps)

    def step():
        loss = forward_loss(x, t, ps, readme)
        loss.backward()
        opt.step(ps)
        opt.zero_grad(ps)
        return loss

    for i in range(warmup):
        loss = step()
        log(f"warmup step {i}: loss {loss.value():.6f}")
    TS.synchronize()

    stream = TS.stream()
    ev0, ev1 = ctypes.c_void_p(), ctypes.c_void_p()
    hip_check(hip.ts_hip_event_create(ctypes.byref(ev0)))
    hip_check(hip.ts_hip_event_create(ctypes.byref(ev1)))
    # The timed region runs uninstrumented: only two events on the library
    # stream bracket it.
    TS.synchronize()
    t0 = time.perf_counter()
    hip_check(hip.ts_hip_event_record(ev0, stream))
    for _ in range(steps):
        loss = step()
    hip_check(hip.ts_hip_event_record(ev1, stream))
    TS.synchronize()
    t1 = time.perf_counter()
    ev_ms = ctypes.c_float()
    hip_check(hip.ts_hip_event_elapsed_ms(ctypes.byref(ev_ms), ev0, ev1))
    final_loss = loss.value()

    # Roofline pass: the same K steps again, every GEMM launch carrying
    # kernel-attached events (the first kernel's start, the last kernel's end:
    # the kernels' own duration, as rocprofv3 reports it); the other classes
    # run untimed.
    TS.Profile.reset()
    TS.Profile.enable(True, classes=[TS.Profile.GEMM])
    r0 = time.perf_counter()
    for _ in range(steps):
        step()
    TS.synchronize()
    roof_ms = (time.perf_counter() - r0) * 1000.0 / steps
    TS.Profile.enable(False)
    g = TS.Profile.read(TS.Profile.GEMM)

    # Per-class breakdown: a separate pass after the timed one, every class timed.
    breakdown_steps = max(1, min(steps, 5))
    TS.Profile.reset()
    TS.Profile.enable(True)
    for _ in range(breakdown_steps):
        step()
    TS.synchronize()
    TS.Profile.enable(False)
    classes = {"gemm": TS.Profile.GEMM, "elementwise": TS.Profile.ELEMENTWISE,
               "reduction": TS.Profile.REDUCTION, "adam": TS.Profile.ADAM}
    prof = {k: TS.Profile.read(v) for k, v in classes.items()}

    wall_ms = (t1 - t0) * 1000.0 / steps
    gemm_tflops = g["work"] / (g["ms"] * 1e-3) / 1e12 if g["ms"] > 0 else 0.0
    kernels = {"pass": f"a separate pass of {breakdown_steps} steps after the timed region, every class timed"}
    for k, s in prof.items():
        if s["launches"] == 0:
            continue
        rate = s["work"] / (s["ms"] * 1e-3) if s["ms"] > 0 else 0.0
        per_step = {"ms_per_step": round(s["ms"] / breakdown_steps, 3),
                    "launches_per_step": s["launches"] // breakdown_steps}
        if k == "gemm":
            kernels[k] = {**per_step, "TFLOP/s": round(rate / 1e12, 2),
                          "frac_mfma_peak": round(rate / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4)}
        else:
            kernels[k] = {**per_step, "GB/s": round(rate / 1e9, 1), "frac_hbm_peak": round(rate / 1e9 / PEAK_HBM_GBS, 4)}
    per_launch_flops = g["work"] / g["launches"] if g["launches"] else 0.0
    traffic, traffic_src = pmc_traffic(cfg)

    result = {
        "metric": "fwd+bwd+Adam steps/sec (1 GPU); % fp32 MFMA peak and % HBM GB/s roofline",
        "value": round(1000.0 / wall_ms, 4),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(wall_ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": {"c5": "synthetic (numpy default_rng(0); N(0,1/fan_in) weights, N(0,1) inputs and targets)",
                 "c4": "synthetic (numpy default_rng(0); Kaiming-uniform weights, N(0,1) inputs and targets)",
                 "c1": "synthetic (numpy default_rng(0); N(0,1) weights and inputs, zero bias)"}[cfg],
        "config": {"workload": {"c5": "BASELINE config 5: deep wide MLP, batch 8192, 6 x Linear(4096,4096)+bias, "
                                      "ReLU on layers 1-5, MSE, fwd+bwd+Adam(lr 1e-3)",
                                "c4": "BASELINE config 4: MLP batch 1024, 784->1024->10, MSE, fwd+bwd+Adam",
                                "c1": "BASELINE config 1: README step x[32,784] W[784,128], relu, sum, Adam"}[cfg],
                   "batch": batch, "widths": widths, "gemm_flop_per_step": step_flops(batch, widths, readme)},
        "roofline": {"bound": "mfma", "achieved": round(gemm_tflops, 2), "peak": PEAK_FP32_MFMA_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(gemm_tflops / PEAK_FP32_MFMA_TFLOPS, 4), "traffic": traffic,
                     "traffic_source": traffic_src,
                     "kernel": ("gemm_f32_w16 (all 3 layouts, every launch of the roofline pass)" if cfg == "c5"
                                else "every GEMM launch of the roofline pass (gemm_f32_mfma tiles, the skinny "
                                     "kernel for N <= 16, split-K where the output has few tiles)"),
                     "flop_per_launch": per_launch_flops,
                     "avg_launch_ms": round(g["ms"] / g["launches"], 4) if g["launches"] else None,
                     "timing": (f"kernel-attached events on every GEMM launch of a second pass of the same "
                                f"{steps} steps ({round(roof_ms, 3)} ms/step wall with the events); the timed "
                                f"region itself is uninstrumented")},
        "kernels": kernels,
        "event_ms_per_step": round(ev_ms.value / steps, 3),
        "final_loss": final_loss,
    }
    if graph:
        # the same loop, one step recorded and then replayed: every replay
        # runs the whole step; untimed replays warm the graph up
        with TS.StepGraph.record() as g:
            gloss = step()
        g.replay(max(1, warmup))
        TS.synchronize()
        t0 = time.perf_counter()
        g.replay(steps)
        t_issued = time.perf_counter()
        TS.synchronize()
        g_ms = (time.perf_counter() - t0) * 1000.0 / steps
        result["graph"] = {"value": round(1000.0 / g_ms, 4), "unit": "steps/s", "ms_per_step": round(g_ms, 4),
                           # host time until every replay was issued: close to ms_per_step when the
                           # graph launches themselves, not the kernels, set the pace
                           "host_ms_per_replay": round((t_issued - t0) * 1000.0 / steps, 4),
                           "final_loss": gloss.value(), "note": "the same step replayed from a HIP graph"}
        g.free()
    if cpu:
        log("timing the CPU baseline (oracle port, one core, bounded sample)")
        result["cpu_baseline"] = cpu_baseline(cfg, cpu_rows)
    else:
        result["cpu_baseline"] = None
    return result


# (name, trans_a, trans_b, M, N, K): the products of configs 5 and 4
GEMM_SHAPES = (
    ("c5_fwd_NN", 0, 0, 8192, 4096, 4096),
    ("c5_dX_NT", 0, 1, 8192, 4096, 4096),
    ("c5_dW_TN", 1, 0, 4096, 4096, 8192),
    ("c4_fwd1_NN", 0, 0, 1024, 1024, 784),
    ("c4_dW1_TN", 1, 0, 784, 1024, 1024),
    ("c4_fwd2_NN", 0, 0, 1024, 10, 1024),
    ("c4_dX2_NT", 0, 1, 1024, 1024, 10),
    ("c4_dW2_TN", 1, 0, 1024, 10, 1024),
    ("c1_fwd_NN", 0, 0, 32, 128, 784),
    ("c1_dW_TN", 1, 0, 784, 128, 32),
)


def gemm_compare(hip, hip_check, reps: int) -> dict:
    """Each product of configs 5, 4 and 1 through this library's GEMM
    (ts_hip_gemm_noalloc: ts_hip_gemm's kernels, the split-K temporary from its
    fixed array, so no allocation is timed) and through torch's fp32 matmul
    (rocBLAS / hipBLASLt, transposes passed as operand flags on views, no
    copies), on the same stream, each timed over `reps` launches with events on
    that stream in two alternating rounds (the faster kept per side); max
    relative difference of the two results."""
    import torch

    torch.backends.cuda.matmul.allow_tf32 = False
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream
    out = {}
    for name, ta, tb, M, N, K in GEMM_SHAPES:
        g = torch.Generator(device=dev).manual_seed(1)
        a = torch.randn((K, M) if ta else (M, K), device=dev, generator=g)
        b = torch.randn((N, K) if tb else (K, N), device=dev, generator=g)
        c = torch.empty((M, N), device=dev)
        lda, ldb = a.shape[1], b.shape[1]
        av, bv = (a.t() if ta else a), (b.t() if tb else b)

        def ours():
            hip_check(hip.ts_hip_gemm_noalloc(ta, tb, M, N, K, a.data_ptr(), lda, b.data_ptr(), ldb, c.data_ptr(), N,
                                              sp))

        def theirs():
            torch.matmul(av, bv, out=c_ref)

        c_ref = torch.empty((M, N), device=dev)
        rec = {}
        # two alternating rounds (ours, theirs, ours, theirs), each side's
        # faster round kept: neither side always runs first on fresh buffers
        # or a cold clock
        for _round in range(2):
            for label, fn in (("ours", ours), ("torch_matmul", theirs)):
                for _ in range(3):
                    fn()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for _ in range(reps):
                    fn()
                e1.record(stream)
                e1.synchronize()
                ms = e0.elapsed_time(e1) / reps
                if label not in rec or ms * 1e3 < rec[label]["us"]:
                    rec[label] = {"us": round(ms * 1e3, 2),
                                  "TFLOP/s": round(2.0 * M * N * K / (ms * 1e-3) / 1e12, 2)}
        diff = (c - c_ref).abs().max().item() / max(c_ref.abs().max().item(), 1e-30)
        rec["max_rel_diff"] = diff
        rec["ours_over_theirs"] = round(rec["torch_matmul"]["us"] / rec["ours"]["us"], 3)
        out[name] = rec
        log(f"{name}: {rec}")
        del a, b, c, c_ref
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default=None, choices=sorted(list(CONFIGS) + ["c2", "c3"]),
                    help="measure this config alone (default: config 5 as the headline, then every other "
                         "config under \"configs\")")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-rows", type=int, default=2048)
    ap.add_argument("--graph", action="store_true",
                    help="also time the same step recorded once as a HIP graph and replayed (StepGraph); "
                         "reported beside the eager figure, which stays `value`")
    ap.add_argument("--gemm-compare", type=int, default=0, metavar="REPS",
                    help="instead of a training step: time every product of configs 5 and 4 through "
                         "ts_hip_gemm and through torch's fp32 matmul (rocBLAS / hipBLASLt), REPS launches each")
    ap.add_argument("--copy-probe", type=int, default=0,
                    help="first launch a plain copy kernel (x * 1.0 -> out, 8 bytes per float) over "
                         "this many floats three times, as the calibration point of HBM byte counters")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build measures one GPU: the path is built and measured on "
                          "a single MI355X (multi-GPU sharding is a design, not built); "
                          "run with --gpus 1"}))
        return 2

    import train_station_amd as TS
    from train_station_amd._ffi import hip, hip_check

    if args.copy_probe:
        n = args.copy_probe
        src, dst = TS.Tensor.zeros([n]), TS.Tensor.zeros([n])
        TS.synchronize()
        for _ in range(3):
            hip_check(hip.ts_hip_mul_scalar(src.device_ptr(), 1.0, dst.device_ptr(), n, TS.stream()))
        TS.synchronize()
        log(f"copy probe: 3 launches over {n} floats ({8 * n} bytes each)")
        del src, dst

    if args.gemm_compare:
        print(json.dumps({"gemm_compare": gemm_compare(hip, hip_check, args.gemm_compare),
                          "peak_TFLOPs": PEAK_FP32_MFMA_TFLOPS}), flush=True)
        return 0

    if args.config:
        result = (run_bandwidth(TS, args.config, args.steps, args.warmup, not args.no_cpu_baseline)
                  if args.config in ("c2", "c3") else
                  run_mlp(TS, hip, hip_check, args.config, args.steps, args.warmup, not args.no_cpu_baseline,
                          args.cpu_sample_rows, args.graph))
        print(json.dumps(result), flush=True)
        return 0

    # Default: config 5 is the headline (value, steps, warmup and roofline of
    # the line); every other BASELINE config is measured in the same run, with
    # its own steps, roofline and CPU baseline, under "configs".
    result = run_mlp(TS, hip, hip_check, "c5", args.steps, args.warmup, not args.no_cpu_baseline,
                     args.cpu_sample_rows, args.graph)
    others = {}
    for cfg, steps, warmup in OTHER_CONFIGS:
        TS.clear_gradients()
        TS.empty_cache()
        log(f"config {cfg}: {steps} timed steps after {warmup} warm-up steps")
        if cfg in ("c2", "c3"):
            r = run_bandwidth(TS, cfg, steps, warmup, not args.no_cpu_baseline)
        else:
            r = run_mlp(TS, hip, hip_check, cfg, steps, warmup, not args.no_cpu_baseline, args.cpu_sample_rows,
                        graph=True)
        others[cfg] = {k: r[k] for k in ("metric", "value", "unit", "steps", "warmup", "ms_per_step", "config",
                                         "roofline", "kernels", "cpu_baseline", "graph") if k in r}
    result["configs"] = others
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
