#!/usr/bin/env python3
"""Throughput of Kapel's product by quantized weights on one MI355X.

A step is one decode layer of Llama-3.2-3B in Q4_K_M at M = 1 (BASELINE.json
config 2): the four stacked products [q; k; v], o, [gate; up] and down, with f32
activations resident in HBM.  28 distinct copies of the layer's weights (1.77
GB, one per layer of the model) are walked in turn, so more than 512 MB is read
between two reuses of any weight and the 256 MB Infinity Cache cannot serve
them.  The 28 layers are one HIP graph; a run replays it.

    python bench.py [--gpus 1] [--steps 280] [--warmup 56]

One JSON line.  `value` is the whole job's weight bytes / time (GB/s).
`roofline` is the dominant kernel, the Q4_K M = 1 product on the [gate; up]
call (28,311,552 weight bytes a launch), timed with HIP events around graph
replays of that call alone on its stream; `traffic` comes from rocprofv3
FETCH_SIZE / WRITE_SIZE runs recorded in profiles/traffic.json.  `configs`
holds the other BASELINE.json configurations (1, 3, 4, 5).  `cpu_baseline` is
kapel-cpu's AVX-512 product (restated in the oracle) on this host's cores, with
a one-thread figure and its VNNI byte product at config 3.  Every GPU figure is
the median of 3 timed graph replays.
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
# Config 4: Qwen3-8B layer in Q8_0.
QWEN_LAYER = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
              ("gate", 12288, 4096), ("up", 12288, 4096), ("down", 4096, 12288)]
QWEN_CALLS = [("q", "k", "v"), ("o",), ("gate", "up"), ("down",)]


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


def cpu_baseline(args, host, layer_bytes, synth, with_bytes):
    """kapel-cpu's products on this host's cores: its AVX-512 kernels
    (quantized.rs:699-1021) restated in the oracle, on the config-2 layer at
    M = 1, all cores and one thread; with `with_bytes`, its VNNI byte kernels
    (bytes.rs:395-652) on the config-3 layer at M = 64.  Weight copies rotate
    over more than 1 GB so that no pass is served from the host's caches.
    Best of the timed passes, as kapel-cpu/examples/quantized.rs:14-27."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as ko

    wide, vnni = ko.wide_available()
    copies = max(2, -(-(1 << 30) // layer_bytes))
    sets = [[[(host[c][0], 0, np.copy(host[c][1]), host[c][2]) for c in call] for call in CALLS]
            for _ in range(copies)]
    cx = [synth.normal(7 + ci, host[call[0]][3], 1.0).reshape(1, -1) for ci, call in enumerate(CALLS)]
    product = ko.product_wide if wide else ko.product_f32

    def passes(fn, seconds, most=1000):
        best, times, i = float("inf"), [], 0
        fn(0)
        t_end = time.perf_counter() + seconds
        while time.perf_counter() < t_end and i < most:
            t0 = time.perf_counter()
            fn(i)
            times.append(time.perf_counter() - t0)
            i += 1
        return min(times), len(times), sum(times)

    def layer(threads):
        def run(i):
            for ci, call in enumerate(CALLS):
                product(sets[i % copies][ci], host[call[0]][3], cx[ci], threads)
        return run

    threads = physical_cores()
    best, n_all, el_all = passes(layer(threads), args.cpu_seconds * 0.5)
    best1, n_one, el_one = passes(layer(1), args.cpu_seconds * 0.5)
    kind = "restated AVX-512 wide::fused" if wide else "portable loop (no AVX-512 on this host)"
    cpu = {"value": round(layer_bytes / best / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": "port",
           "variant": "restated-avx512" if wide else "portable",
           "value_1thread": round(layer_bytes / best1 / 1e9, 2),
           "sample": f"config-2 layer (63.1 MB, M = 1, f32 x), {kind}: best of {n_all} passes on "
                     f"{threads} threads ({el_all:.1f} s) and of {n_one} on 1 thread ({el_one:.1f} s), "
                     f"{copies} weight copies rotated"}
    if with_bytes and vnni:
        xs = [synth.normal(7 + ci, 64 * host[call[0]][3], 1.0).reshape(64, -1) for ci, call in enumerate(CALLS)]
        prepared = [ko.quantize_x(x) for x in xs]

        def layer64(i):
            for ci, call in enumerate(CALLS):
                ko.product_vnni(sets[i % copies][ci], host[call[0]][3], threads=threads, prepared=prepared[ci])
        b64, n64, el64 = passes(layer64, args.cpu_seconds * 0.5)
        ops = 2 * 64 * sum(n * k for _, n, k, _ in LAYER)
        cpu["config3"] = {"ms_per_layer": round(b64 * 1e3, 3), "tops": round(ops / b64 / 1e12, 4),
                          "sample": f"config-3 layer at M = 64 in bytes, restated AVX-512 VNNI kernels, "
                                    f"best of {n64} passes on {threads} threads ({el64:.1f} s)"}
    return cpu


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=280)
    ap.add_argument("--warmup", type=int, default=56)
    ap.add_argument("--layers", type=int, default=28)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-configs", action="store_true")
    ap.add_argument("--configs", default="1,3,4,5,moe",
                    help="which of the other configs to run (comma-separated), after config 2")
    ap.add_argument("--profile", choices=["gateup", "copy", "mmf4", "table"],
                    help="only launch the [gate; up] call (or a 256 MiB device copy, or "
                         "(table) config 5's Q6_K output table at M = 1) 20 times, or "
                         "(mmf4) the four calls of config 4 with bf16 activations 10 "
                         "times each, for rocprofv3 counter runs")
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
    op = ka.QuantizedMatmul()
    fmts = {"q4k": ka.Q4K, "q6k": ka.Q6K}

    if args.profile == "copy":
        # A plain copy of known size: the reference point of FETCH_SIZE and
        # WRITE_SIZE (268,435,456 bytes read and written per launch).
        src = torch.empty(1 << 28, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(20):
            dst.copy_(src)
        torch.cuda.synchronize()
        return

    def values(seed, count):
        """count weights ~ N(0, 0.02): 4 Mi seeded values, repeated (the
        timing does not depend on the values; the parity tests use full
        seeded matrices)."""
        base = synth.normal(seed, min(count, 1 << 22), 0.02)
        return np.resize(base, count) if count > base.size else base

    def quantized_layer(spec, seed0, fmt_of):
        host, nbytes = {}, 0
        for i, (name, n, k, *rest) in enumerate(spec):
            fmt = fmt_of(rest)
            data = ka.quantize(fmt, 0, values(seed0 + i, n * k))
            host[name] = (fmt, data, n, k)
            nbytes += data.size
        return host, nbytes

    if args.profile == "mmf4":
        # The four calls of the Q8_0 layer of config 4 at M = 512 with bf16
        # activations (the float many-row kernel), 10 times each.
        qhost, _ = quantized_layer(QWEN_LAYER, 300, lambda r: ka.Q8_0)
        qlayer = {name: ka.QuantizedTensor(torch.from_numpy(data).to(dev), fmt, 0, n, k)
                  for name, (fmt, data, n, k) in qhost.items()}
        for ci, call in enumerate(QWEN_CALLS):
            k = qhost[call[0]][3]
            x = torch.from_numpy(synth.normal(7 + ci, 512 * k, 1.0).reshape(512, k)).to(dev, torch.bfloat16)
            for _ in range(10):
                hip.forward(op, [x] + [qlayer[c] for c in call])
        torch.cuda.synchronize()
        return
    if args.profile == "table":
        # Config 5's 151936 x 4096 Q6_K output table at M = 1 (the streamed
        # decode kernel, walking), as the bench times it.
        table = ka.quantize(ka.Q6K, 0, values(77, 151936 * 4096))
        wt = ka.QuantizedTensor(torch.from_numpy(table).to(dev), ka.Q6K, 0, 151936, 4096)
        xt = torch.from_numpy(synth.normal(6, 4096, 1.0).reshape(1, 4096)).to(dev)
        ot = torch.empty((1, 151936), device=dev)
        for _ in range(20):
            hip.forward(op, [xt, wt], out=ot)
        torch.cuda.synchronize()
        return
    host, layer_bytes = quantized_layer(LAYER, 100, lambda r: fmts[r[0]])
    L = args.layers
    if args.profile == "gateup":
        ws = [[ka.QuantizedTensor(torch.from_numpy(host[c][1]).to(dev), host[c][0], 0, host[c][2], host[c][3])
               for c in ("gate", "up")] for _ in range(L)]
        x = torch.from_numpy(synth.normal(9, 3072, 1.0).reshape(1, 3072)).to(dev)
        o = torch.empty((1, 16384), device=dev)
        for i in range(20):
            hip.forward(op, [x] + ws[i % L], out=o)
        torch.cuda.synchronize()
        return
    layers = [{name: ka.QuantizedTensor(torch.from_numpy(data).to(dev), fmt, 0, n, k)
               for name, (fmt, data, n, k) in host.items()} for _ in range(L)]
    torch.cuda.synchronize()

    def inputs_for(calls, host_w, rows, dtype=torch.float32, seed=7):
        xs, outs = [], []
        for ci, call in enumerate(calls):
            k = host_w[call[0]][3]
            width = sum(host_w[c][2] for c in call)
            x = torch.from_numpy(synth.normal(seed + ci, rows * k, 1.0).reshape(rows, k)).to(dev, dtype)
            xs.append(x)
            outs.append(torch.empty((rows, width), dtype=dtype, device=dev))
        return xs, outs

    def reserve(calls, layer, rows, byte):
        """The workspace of the largest call (byte activations at every row
        count with `byte`)."""
        size = 0
        for call in calls:
            ws = [layer[c] for c in call]
            arr = (ka._Weight * len(ws))(*[w.weight() for w in ws])
            size = max(size, ka.lib().kh_qmatmul_workspace(
                arr, len(ws), ws[0].k, rows, ka.BYTE_ACTIVATIONS_ALL_ROWS if byte else 0))
        hip.workspace(size)

    def timed(step_fns, steps, warmup, replays=3):
        """One HIP graph of `steps` steps (step i runs step_fns[i % len]),
        checked against an eager run; `warmup` steps' worth of untimed
        replays, then `replays` replays, each bracketed by synchronizations
        and timed with events on the capture stream.  Seconds per step (the
        median replay) and the per-replay figures."""
        steps = max(1, steps)
        step_fns[(steps - 1) % len(step_fns)]()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(steps):
                step_fns[i % len(step_fns)]()
        for _ in range(max(1, -(-warmup // steps))):
            g.replay()
        torch.cuda.synchronize()
        per = []
        for _ in range(max(3, replays)):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            a.record()
            g.replay()
            b.record()
            torch.cuda.synchronize()
            per.append(a.elapsed_time(b) * 1e-3 / steps)
        return sorted(per)[len(per) // 2], per

    # ---- config 2: the layer at M = 1 (value) ----------------------------------
    hip.with_byte_activations(False)
    reserve(CALLS, layers[0], 1, False)
    xs, outs = inputs_for(CALLS, host, 1)

    def layer_step(l):
        def run():
            for ci, call in enumerate(CALLS):
                hip.forward(op, [xs[ci]] + [layers[l][c] for c in call], out=outs[ci])
        return run

    # Graph replays agree with the eager product, bit for bit.
    layer_step((args.steps - 1) % L)()
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs]
    sec, per_replay = timed([layer_step(l) for l in range(L)], args.steps, args.warmup)
    for a_, b_ in zip(outs, eager):
        assert torch.equal(a_, b_), "graph replay differs from the eager product"
    value = layer_bytes / sec / 1e9

    # ---- roofline: the [gate; up] call alone ------------------------------------
    gate_bytes = host["gate"][1].size + host["up"][1].size
    x3, o3 = xs[2], outs[2]

    def gate_step(l):
        return lambda: hip.forward(op, [x3, layers[l]["gate"], layers[l]["up"]], out=o3)

    gsec, _ = timed([gate_step(l) for l in range(L)], 10 * L, L)
    achieved = gate_bytes / gsec / 1e9
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        traffic = json.load(open(tpath)).get("gemv_q4k_gateup_m1_bytes_per_launch")
    roofline = {"kernel": "gemv2_kernel<Q4K, 3 planes, 1 row, f32 x>: weights staged in LDS by direct "
                          "loads ([gate; up], 16384 x 3072 Q4_K, M = 1)",
                "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                "algorithmic_bytes_per_launch": gate_bytes,
                "avg_launch_us": round(gsec * 1e6, 2),
                "timing": "HIP events around graph replays of 280 launches over 28 rotated weight "
                          "copies, median of 3 replays"}

    configs = {}
    only = set() if args.no_configs else set(args.configs.split(","))
    if only:
        if "3" in only:
            # ---- config 3: the same layer, M = 64, byte activations at every
            # row count (the reference's CPU takes bytes up to 16 rows only)
            hip.with_byte_activations(True, all_rows=True)
            reserve(CALLS, layers[0], 64, True)
            xs, outs = inputs_for(CALLS, host, 64)
            s3, _ = timed([layer_step(l) for l in range(L)], 2 * L, L)
            ops3 = 2 * 64 * sum(n * k for _, n, k, _ in LAYER)
            configs["3"] = {"workload": "Llama-3.2-3B layer (Q4_K + Q6_K down), M = 64, byte activations",
                            "ms_per_step": round(s3 * 1e3, 4), "tops": round(ops3 / s3 / 1e12, 2),
                            "mfma_frac": round(ops3 / s3 / 1e12 / INT8_PEAK_TOPS, 4),
                            "weight_gbps": round(layer_bytes / s3 / 1e9, 1)}
            hip.with_byte_activations(False)

        if "1" in only:
            # ---- config 1: Q4_0 8192 x 2048, M = 1 ---------------------------------
            d1 = ka.quantize(ka.Q4_0, 0, synth.normal(0, 8192 * 2048, 0.02))  # seed 0, as config 1 says
            copies = max(2, int(1.2e9 // d1.size))
            w1 = [ka.QuantizedTensor(torch.from_numpy(d1).to(dev), ka.Q4_0, 0, 8192, 2048)
                  for _ in range(copies)]
            x1 = torch.from_numpy(synth.normal(1, 2048, 1.0).reshape(1, 2048)).to(dev)
            o1 = torch.empty((1, 8192), device=dev)
            s1, _ = timed([(lambda w=w: hip.forward(op, [x1, w], out=o1)) for w in w1], 4 * copies, copies)
            configs["1"] = {"workload": "Q4_0 8192 x 2048, M = 1, f32 activations",
                            "us_per_call": round(s1 * 1e6, 2), "weight_gbps": round(d1.size / s1 / 1e9, 1)}
            del w1

        if "5" in only:
            # ---- config 5: low-bit FFN, int4 attention, Q6_K output table, M in {1, 8}
            c5 = {}
            parts = [("up_q2k", ka.Q2K, 0, 12288, 4096), ("down_q2k", ka.Q2K, 0, 4096, 12288),
                     ("up_q3k", ka.Q3K, 0, 12288, 4096), ("down_q3k", ka.Q3K, 0, 4096, 12288),
                     ("up_q5k", ka.Q5K, 0, 12288, 4096), ("down_q5k", ka.Q5K, 0, 4096, 12288),
                     ("q_int4", ka.INT4, 32, 4096, 4096)]
            for name, fmt, group, n, k in parts:
                d = ka.quantize(fmt, group, values(500 + len(c5), n * k))
                copies = max(2, int(1.2e9 // d.size))
                ws5 = [ka.QuantizedTensor(torch.from_numpy(d).to(dev), fmt, group, n, k) for _ in range(copies)]
                for rows in (1, 8):
                    x5 = torch.from_numpy(synth.normal(5, rows * k, 1.0).reshape(rows, k)).to(dev)
                    o5 = torch.empty((rows, n), device=dev)
                    reserve([("w",)], {"w": ws5[0]}, rows, False)
                    s5, _ = timed([(lambda w=w: hip.forward(op, [x5, w], out=o5)) for w in ws5], 4 * copies, copies)
                    c5[f"{name}_m{rows}"] = {"us": round(s5 * 1e6, 2), "gbps": round(d.size / s5 / 1e9, 1)}
                del ws5
            table = ka.quantize(ka.Q6K, 0, values(77, 151936 * 4096))
            wt = ka.QuantizedTensor(torch.from_numpy(table).to(dev), ka.Q6K, 0, 151936, 4096)
            for rows in (1, 8):
                xt = torch.from_numpy(synth.normal(6, rows * 4096, 1.0).reshape(rows, 4096)).to(dev)
                ot = torch.empty((rows, 151936), device=dev)
                reserve([("w",)], {"w": wt}, rows, False)
                st, _ = timed([lambda: hip.forward(op, [xt, wt], out=ot)], 20, 60)  # three warm-up replays: the first launches after the allocation run slow
                c5[f"table_q6k_m{rows}"] = {"us": round(st * 1e6, 2), "gbps": round(table.size / st / 1e9, 1)}
            configs["5"] = {"workload": "Q2_K/Q3_K/Q5_K FFN (12288x4096, 4096x12288), int4/32 4096x4096, "
                                        "Q6_K output table 151936x4096; f32 x; weights from 4 Mi N(0, 0.02) values repeated",
                            "calls": c5}
            del wt

        if "4" in only:
            # ---- config 4: Qwen3-8B layer, Q8_0, M = 512, bf16 activations in bytes
            qhost, qbytes = quantized_layer(QWEN_LAYER, 300, lambda r: ka.Q8_0)
            qlayers = [{name: ka.QuantizedTensor(torch.from_numpy(data).to(dev), fmt, 0, n, k)
                        for name, (fmt, data, n, k) in qhost.items()} for _ in range(2)]
            hip.with_byte_activations(True, all_rows=True)
            reserve(QWEN_CALLS, qlayers[0], 512, True)
            xq, oq = inputs_for(QWEN_CALLS, qhost, 512, dtype=torch.bfloat16)

            def qwen_step(l):
                def run():
                    for ci, call in enumerate(QWEN_CALLS):
                        hip.forward(op, [xq[ci]] + [qlayers[l][c] for c in call], out=oq[ci])
                return run

            s4, _ = timed([qwen_step(0), qwen_step(1)], 4, 2)
            hip.with_byte_activations(False)
            ops4 = 2 * 512 * sum(n * k for _, n, k in QWEN_LAYER)
            # The reference's own arithmetic at 512 rows: activations as they
            # are (the float many-row kernel: bf16 activations and the Q8_0
            # codes on the bf16 matrix cores, f32 sums scaled by block).
            reserve(QWEN_CALLS, qlayers[0], 512, False)
            s4f, _ = timed([qwen_step(0), qwen_step(1)], 4, 2)
            configs["4"] = {"workload": "Qwen3-8B layer in Q8_0, M = 512, bf16 activations quantized to bytes",
                            "ms_per_step": round(s4 * 1e3, 3), "tops": round(ops4 / s4 / 1e12, 2),
                            "mfma_frac": round(ops4 / s4 / 1e12 / INT8_PEAK_TOPS, 4),
                            "weight_gbps": round(qbytes / s4 / 1e9, 1),
                            "bf16_activations": {"ms_per_step": round(s4f * 1e3, 3),
                                                 "tops": round(ops4 / s4f / 1e12, 2),
                                                 "note": "activations not rounded to bytes (the drop-in "
                                                         "default above 16 rows): bf16 matrix cores, the Q8_0 "
                                                         "codes as bf16 and one scale fma per block of 32"}}
            del qlayers

        if "moe" in only:
            # ---- the experts' product at decode: the shapes of the reference's
            # kapel-cuda/examples/experts.rs (one token, bf16 x; bytes = the
            # codes of the experts read).  Weight copies and expert choices
            # rotate so that no call finds its experts in a cache.
            cm = {}
            shapes = [("qwen3.6-35b-a3b", 256, 8, 2048, 512), ("qwen3.8-flash-next", 512, 10, 2560, 640)]
            for model, experts, topk, hidden, width in shapes:
                for fmt, what, n, kk in ((ka.IQ3_S, "gate_iq3s", width, hidden),
                                         (ka.IQ4_XS, "down_iq4xs", hidden, width),
                                         (ka.Q8_0, "gate_q8_0", width, hidden)):
                    if kk % ka.block_len(fmt):
                        continue
                    rng = np.random.default_rng(experts + n)
                    size = experts * n * ka.row_bytes(fmt, 0, kk)
                    raw = rng.integers(0, 256, size=size, dtype=np.uint8)
                    blocks = raw.reshape(-1, ka.block_bytes(fmt))
                    blocks[:, 0:2] = np.frombuffer(np.float16(0.01).tobytes(), np.uint8)
                    copies = max(2, int(1.2e9 // size))
                    wm = [ka.QuantizedTensor(torch.from_numpy(raw).to(dev), fmt, 0, experts * n, kk)
                          for _ in range(copies)]
                    xm = torch.from_numpy(synth.normal(8, kk, 1.0).reshape(1, kk)).to(dev, torch.bfloat16)
                    om = torch.empty((1, topk, n), device=dev, dtype=torch.bfloat16)
                    idxs = [torch.tensor([[(c * 101 + i * 37) % experts for i in range(topk)]],
                                         dtype=torch.int32, device=dev) for c in range(copies)]
                    mop = ka.ExpertMatmul(experts)
                    sm, _ = timed([(lambda w=w, ix=ix: hip.forward(mop, [xm, w, ix], out=om, check_indices=False))
                                   for w, ix in zip(wm, idxs)], 8 * copies, copies)
                    read = topk * n * ka.row_bytes(fmt, 0, kk)
                    cm[f"{model}_{what}"] = {"shape": f"1 x {kk} -> {n} x {topk} of {experts}",
                                             "us": round(sm * 1e6, 2), "gbps": round(read / sm / 1e9, 1)}
                    del wm
            configs["moe"] = {"workload": "ExpertMatmul decode (1 token, bf16 x) at the shapes of "
                                          "kapel-cuda/examples/experts.rs; random codes, f16 scales 0.01",
                              "calls": cm}

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(args, host, layer_bytes, synth, "3" in only)

    line = {"metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
            "steps": max(1, args.steps), "warmup": args.warmup, "ms_per_step": round(sec * 1e3, 4),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "int8 (i8 x i8 -> i32 MFMA dots, f32 scales)", "data": "synthetic",
            "config": {"workload": "config 2: Llama-3.2-3B decode layer, Q4_K (q, k, v, o, "
                                   "gate, up) + Q6_K (down), M = 1, f32 activations",
                       "weight_bytes_per_step": layer_bytes, "layers_rotated": L,
                       "ms_per_step_replays": [round(t * 1e3, 4) for t in per_replay],
                       "frac_of_hbm_peak": round(value / HBM_PEAK_GBPS, 4)},
            "roofline": roofline, "configs": configs, "cpu_baseline": cpu}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
