"""Benchmark of the hot path on one MI355X.

A step is the pair stack's two triangle multiplications (outgoing, then
incoming) at N_res = 384, c_z = c_hidden = 128: z f16
~N(0,1), projection weights ~N(0, 1/128), f16 operands with f32
accumulation, f32 output. Inputs are generated once on the host (splitmix64 +
Box-Muller, seed 0xAF2000 + 2), rounded to f16 and resident in HBM before
the timed region.

Prints one JSON line. `value` is the step's algorithmic TFLOP/s (2*M*K*N
per GEMM, LayerNorm and sigmoid not counted, as src/runtime/kernel-cost.ts:71
counts). `roofline` is the dominant kernel (the channel-batched contraction)
measured with hipEvents on its own stream inside this run. `cpu_baseline`
is the CPU oracle (oracle/afref.c, one thread) on a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "alphafold2-webgpu_amd"))
sys.path.insert(0, ROOT)

METRIC = "Evoformer GEMM TFLOP/s (% MFMA peak); triangle-mult ms @N_res=384"
PEAK_F16_TFLOPS = 2500.0   # MI355X dense f16 MFMA, published
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E, published
L, CZ, CH = 384, 128, 128


def triangle_flops(length: int, cz: int, ch: int) -> dict:
    pairs = length * length
    return {
        "project": 2 * pairs * cz * (4 * ch),
        "contract": 2 * length * length * length * ch,
        "output": 2 * pairs * ch * cz,
        "gate": 2 * pairs * cz * cz,
    }


def cpu_baseline() -> dict:
    """The oracle (a restatement of src/triangle/cpu-reference.ts) on one
    thread, timed on an L=128 outgoing triangle multiplication and reported
    as its algorithmic TFLOP/s (the unit of `value`)."""
    from oracle import ref

    length = 128
    inp = ref.deterministic_triangle_input(length, CZ, CH, seed=11)
    start = time.perf_counter()
    ref.triangle("outgoing", inp["z"], inp["mask"], inp["weights"])
    seconds = time.perf_counter() - start
    flops = sum(triangle_flops(length, CZ, CH).values())
    full = 2 * sum(triangle_flops(L, CZ, CH).values())
    return {"value": flops / seconds / 1e12, "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"one outgoing triangle multiplication at L={length}, c_z=c_h={CH} "
                      f"({seconds:.2f} s); a full step would take {full / (flops / seconds):.0f} s",
            "ms_per_step_extrapolated": full / (flops / seconds) * 1e3}


def copy_probe(mib: int) -> None:
    import torch

    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_each_way": n * 4, "launches": 10}))


def main() -> None:
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=3)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                        help="only run a plain device-to-device copy of MIB MiB 10 times (the known-size kernel "
                             "rocprof's FETCH_SIZE / WRITE_SIZE readings are scaled by) and exit")
    args = parser.parse_args()
    if args.copy_probe:
        copy_probe(args.copy_probe)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: the path runs on one device and bench.py "
                                   "--gpus N>1 is not supported (see DESIGN.md for how it would shard)"}))
        sys.exit(2)

    import numpy as np
    import torch

    from afhip import device, triangle
    from oracle import ref  # input generation only (splitmix64 + Box-Muller)

    device.open_device(0)
    dev = device.device()
    seed = 0xAF2000 + 2
    z = ref.round_f16(ref.normal(seed, (L, L, CZ)))
    mask = np.ones((L, L), np.float32)
    weights = {}
    shapes = ref.triangle_weight_shapes(CZ, CH)
    for i, name in enumerate(ref.TRIANGLE_ORDER):
        shape = shapes[name]
        if name.startswith("layerNorm"):
            center = 1.0 if name.endswith("Weight") else 0.0
            weights[name] = ref.normal(seed + 100 + i, shape, 0.01, center)
        elif name.endswith("Bias"):
            weights[name] = ref.normal(seed + 100 + i, shape, 0.02)
        else:
            weights[name] = ref.normal(seed + 100 + i, shape, 1.0 / shape[1])
    zd = torch.from_numpy(z).half().to(dev)
    md = torch.from_numpy(mask).to(dev)
    ops = []
    for direction in ("outgoing", "incoming"):
        op = triangle.TriangleMultiplication(L, CZ, CH, direction=direction, precision="f16", pair_dtype="f16",
                                             out_dtype="f32")
        op.prepare(weights)
        ops.append((op, torch.empty((L, L, CZ), dtype=torch.float32, device=dev)))

    def step():
        for op, out in ops:
            op(zd, md, out=out)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    start = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - start) * 1e3 / args.steps

    # Per-kernel durations: hipEvents bracket every launch on its own stream.
    device.timing_reset()
    device.timing_enable(True)
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    timings = device.timing_report()
    device.timing_enable(False)
    per_kernel = {k: v["total_ms"] / v["count"] for k, v in timings.items()}

    flops = triangle_flops(L, CZ, CH)
    step_flops = 2 * sum(flops.values())
    value = step_flops / (ms_per_step * 1e-3) / 1e12
    contract_ms = per_kernel.get("triangle.contract", float("nan"))
    achieved = flops["contract"] / (contract_ms * 1e-3) / 1e12
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "triangle multiplication outgoing + incoming, N_res=384, c_z=c_hidden=128, "
                               "f16 in, f32 accumulate, f32 out (BASELINE config 3)",
                   "n_res": L, "c_z": CZ, "c_hidden": CH, "parallelism": "none (1 GPU)"},
        "roofline": {"kernel": "triangle.contract", "bound": "mfma", "achieved": round(achieved, 2),
                     "peak": PEAK_F16_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / PEAK_F16_TFLOPS, 4),
                     "traffic": None, "avg_ms": round(contract_ms, 5)},
        "kernel_ms": {k: round(v, 5) for k, v in per_kernel.items()},
        "triangle_ms": round(ms_per_step / 2, 4),
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result))


if __name__ == "__main__":
    main()
