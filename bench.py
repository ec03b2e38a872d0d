#!/usr/bin/env python3
"""Weight-read bandwidth of Kapel's product by quantized weights on one MI355X.

A step is one decode layer of Llama-3.2-3B in Q4_K_M at M = 1 (BASELINE.json
config 2): the four stacked products [q; k; v], o, [gate; up] and down, with
f32 activations resident in HBM.  28 distinct copies of the layer's weights
(1.77 GB, one per layer of the model) are walked in turn, so more than 512 MB
is read between two reuses of any weight and the 256 MB Infinity Cache cannot
serve them.  The 28 layers are one HIP graph; a run replays it.

    python bench.py [--gpus 1] [--steps 280] [--warmup 56]

One JSON line: `value` is the whole job's weight bytes / time (GB/s);
`roofline` is the [gate; up] product kernel's own duration from HIP events
around each launch on its stream (activations prepared beforehand); `m64_bytes`
is config 3 (the same layer, M = 64, byte activations: int8 MFMA TOPS);
`cpu_baseline` is the oracle's f32 product (the restated kapel-cpu algorithm)
on this host's cores.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0          # MI355X HBM3E
INT8_PEAK_TOPS = 5000.0         # MI355X dense int8 MFMA
METRIC = "Q4_K GEMV weight-read GB/s (% of HBM peak) at M=1; int8 MFMA TOPS at M=64"

# (name, n, k, format) of the layer; products in call order.
LAYER = [("q", 3072, 3072, "q4k"), ("k", 1024, 3072, "q4k"), ("v", 1024, 3072, "q4k"),
         ("o", 3072, 3072, "q4k"), ("gate", 8192, 3072, "q4k"), ("up", 8192, 3072, "q4k"),
         ("down", 3072, 8192, "q6k")]
CALLS = [("q", "k", "v"), ("o",), ("gate", "up"), ("down",)]


def physical_cores():
    """One thread per physical core, as kapel-cpu/src/isa.rs:92-125, at most
    the CPUs this process may use and 16 (the share of one GPU's box)."""
    cores = set()
    phys = None
    try:
        for line in open("/proc/cpuinfo"):
            key, _, value = line.partition(":")
            key, value = key.strip(), value.strip()
            if key == "physical id":
                phys = value
            elif key == "core id":
                cores.add((phys, value))
    except OSError:
        pass
    allowed = len(os.sched_getaffinity(0))
    n = len(cores) if cores else allowed
    return max(1, min(n, allowed, 16))


def build_layer(ka, synth, torch):
    """One layer's weights: f32 ~ N(0, 0.02), seeded per matrix, quantized."""
    fmts = {"q4k": ka.Q4K, "q6k": ka.Q6K}
    host, nbytes = {}, 0
    for i, (name, n, k, fmt) in enumerate(LAYER):
        values = synth.normal(100 + i, n * k, 0.02)
        data = ka.quantize(fmts[fmt], 0, values)
        host[name] = (fmts[fmt], data, n, k)
        nbytes += data.size
    return host, nbytes


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=280)
    ap.add_argument("--warmup", type=int, default=56)
    ap.add_argument("--layers", type=int, default=28)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-m64", action="store_true")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(the product shards by output rows; see the design notes). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import kapel_amd as ka
    from kapel_amd import synth

    hip = ka.Hip(0)
    dev = hip.device
    host, layer_bytes = build_layer(ka, synth, torch)
    L = args.layers
    # 28 distinct copies of the layer on the device.
    layers = []
    for l in range(L):
        layers.append({name: ka.QuantizedTensor(torch.from_numpy(data).to(dev), fmt, 0, n, k)
                       for name, (fmt, data, n, k) in host.items()})
    torch.cuda.synchronize()

    def make_inputs(rows):
        xs, outs = [], []
        for ci, call in enumerate(CALLS):
            k = host[call[0]][3]
            width = sum(host[c][2] for c in call)
            x = torch.from_numpy(synth.normal(7 + ci, rows * k, 1.0).reshape(rows, k)).to(dev)
            xs.append(x)
            outs.append(torch.empty((rows, width), dtype=torch.float32, device=dev))
        return xs, outs

    op = ka.QuantizedMatmul()

    def step(layer, xs, outs):
        for ci, call in enumerate(CALLS):
            hip.forward(op, [xs[ci]] + [layer[c] for c in call], out=outs[ci])

    def reserve_workspace(rows, byte):
        size = 0
        for call in CALLS:
            ws = [layers[0][c] for c in call]
            arr = (ka._Weight * len(ws))(*[w.weight() for w in ws])
            size = max(size, ka.lib().kh_qmatmul_workspace(
                arr, len(ws), ws[0].k, rows, ka.BYTE_ACTIVATIONS if byte else 0))
        hip.workspace(size)

    def capture(count, xs, outs):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for l in range(count):
                step(layers[l % L], xs, outs)
        return g

    def run_mode(rows, byte, steps, warmup):
        hip.with_byte_activations(byte)
        reserve_workspace(rows, byte)
        xs, outs = make_inputs(rows)
        # Eager reference of the last layer's outputs.
        step(layers[(steps - 1) % L], xs, outs)
        torch.cuda.synchronize()
        eager = [o.clone() for o in outs]
        full = capture(L, xs, outs)
        rest = steps % L
        part = capture(rest, xs, outs) if rest else None

        def replay(nsteps):
            for _ in range(nsteps // L):
                full.replay()
            if nsteps % L:
                assert part is not None and nsteps % L == rest
                part.replay()

        # Graph replays agree with the eager run, bit for bit, replay after replay.
        for _ in range(2):
            replay(steps)
            torch.cuda.synchronize()
            for a, b in zip(outs, eager):
                assert torch.equal(a, b), "graph replay differs from the eager product"
        for _ in range(max(1, warmup // L)):
            full.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        replay(steps)
        torch.cuda.synchronize()
        seconds = time.perf_counter() - t0
        hip.with_byte_activations(False)
        return seconds, xs, outs

    steps = args.steps
    seconds, xs, outs = run_mode(1, False, steps, args.warmup)
    ms_per_step = seconds * 1e3 / steps
    value = layer_bytes * steps / seconds / 1e9

    # The dominant kernel: the [gate; up] product (28.3 MB of Q4_K), timed
    # with events around each launch; its activations prepared by a first call.
    gate_bytes = host["gate"][1].size + host["up"][1].size
    hip.with_byte_activations(False)
    reserve_workspace(1, False)
    x3, o3 = xs[2], outs[2]
    hip.forward(op, [x3, layers[0]["gate"], layers[0]["up"]], out=o3)
    torch.cuda.synchronize()
    durations = []
    for rep in range(4):
        pairs = []
        torch.cuda._sleep(int(2.0e7))  # keeps the GPU behind the host's launches
        for l in range(L):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            hip.forward(op, [x3, layers[l]["gate"], layers[l]["up"]], out=o3,
                        reuse_activations=True)
            b.record()
            pairs.append((a, b))
        torch.cuda.synchronize()
        if rep:
            durations += [a.elapsed_time(b) for a, b in pairs]
    kernel_ms = float(np.mean(durations))
    achieved = gate_bytes / (kernel_ms * 1e-3) / 1e9
    roofline = {"kernel": "qmv_kernel<Q4K, 3, 1> ([gate; up], 16384 x 3072 Q4_K, M = 1)",
                "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                "traffic": None, "algorithmic_bytes": gate_bytes,
                "avg_launch_us": round(kernel_ms * 1e3, 2), "launches": len(durations)}

    m64 = None
    if not args.no_m64:
        s64, _, _ = run_mode(64, True, L * 2, L)
        ops = 2 * 64 * sum(n * k for _, n, k, _ in LAYER)
        t = s64 / (L * 2)
        m64 = {"workload": "config 3: the same layer, M = 64, byte activations",
               "ms_per_step": round(t * 1e3, 4),
               "tops": round(ops / t / 1e12, 2),
               "mfma_frac": round(ops / t / 1e12 / INT8_PEAK_TOPS, 4),
               "weight_gbps": round(layer_bytes / t / 1e9, 1)}

    cpu = None
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as ko
        threads = physical_cores()
        parts = [[(host[c][0], 0, host[c][1], host[c][2]) for c in call] for call in CALLS]
        cx = [synth.normal(7 + ci, host[call[0]][3], 1.0).reshape(1, -1)
              for ci, call in enumerate(CALLS)]
        for ci in range(len(CALLS)):
            ko.product_f32(parts[ci], host[CALLS[ci][0]][3], cx[ci], threads)
        passes, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_seconds:
            for ci in range(len(CALLS)):
                ko.product_f32(parts[ci], host[CALLS[ci][0]][3], cx[ci], threads)
            passes += 1
        el = time.perf_counter() - t0
        cpu = {"value": round(layer_bytes * passes / el / 1e9, 2), "unit": "GB/s",
               "cores": threads, "kind": "port",
               "sample": f"{passes} passes of the config-2 layer (63.1 MB) at M = 1, "
                         f"f32 activations, {el:.1f} s, the oracle's threaded restatement of "
                         "kapel-cpu's portable quantized product"}

    line = {"metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
            "steps": steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "int8 (i8 x i8 -> i32 MFMA dots, f32 scales)", "data": "synthetic",
            "config": {"workload": "config 2: Llama-3.2-3B decode layer, Q4_K (q, k, v, o, "
                                   "gate, up) + Q6_K (down), M = 1, f32 activations",
                       "weight_bytes_per_step": layer_bytes, "layers_rotated": L,
                       "frac_of_hbm_peak": round(value / HBM_PEAK_GBPS, 4)},
            "roofline": roofline, "m64_bytes": m64, "cpu_baseline": cpu}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
