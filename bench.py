"""Benchmark of the hot path on one MI355X.

Headline: a step is the pair stack's two triangle
multiplications (outgoing, then incoming) at N_res = 384,
c_z = c_hidden = 128: z f16 ~N(0,1), projection weights ~N(0, 1/128), f16
operands with f32 accumulation, f32 output. Inputs are generated once on the
host (splitmix64 + Box-Muller, seed 0xAF2000 + config index, N(mu, v) read
as variance v), rounded to f16 and resident in HBM before the timed region.

Prints one JSON line. `value` is the step's algorithmic TFLOP/s (2*M*K*N per
GEMM; LayerNorm and sigmoid not counted, as src/runtime/kernel-cost.ts:71
counts); `triangle_ms` is the per-operation time the metric quotes.
`kernels` holds each triangle kernel's roofline, measured with hipEvents on
the stream it is launched on (afhip_timing_*) during the same run;
`roofline` is the dominant one (largest average duration). `traffic` is the
HBM bytes per launch from rocprofv3's FETCH_SIZE and WRITE_SIZE counters,
scaled against a plain copy, as recorded in
profiles/hbm_traffic_by_kernel.md. `configs` measures BASELINE's other
configurations the same way. `cpu_baseline` is the reference's CPU path
(cpu-reference.ts restated in plain JS, oracle/cpu_reference.js) under node
on one thread, on a bounded sample, with the C oracle on one thread and on
every core beside it.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "alphafold2-webgpu_amd"))
sys.path.insert(0, ROOT)

METRIC = "Evoformer GEMM TFLOP/s (% MFMA peak); triangle-mult ms @N_res=384"
PEAK_F16_TFLOPS = 2500.0   # MI355X dense f16 MFMA, published
PEAK_F32_TFLOPS = 157.3    # MI355X fp32, published
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E, published
L, CZ, CH = 384, 128, 128
SEED = 0xAF2000
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_by_kernel.md")


def triangle_flops(length: int, cz: int, ch: int) -> dict:
    pairs = length * length
    return {
        "project": 2 * pairs * cz * (4 * ch),
        "contract": 2 * length * length * length * ch,
        "output": 2 * pairs * ch * cz,
        "gate": 2 * pairs * cz * cz,
    }


def triangle_bytes(length: int, cz: int, ch: int, pair_bytes: int = 2, out_bytes: int = 4) -> dict:
    """Algorithmic HBM bytes per launch of each f16-path kernel."""
    pairs = length * length
    return {
        "triangle.project": pairs * cz * pair_bytes + pairs * 4 + 2 * ch * pairs * 2,
        "triangle.contract": 2 * ch * pairs * 2 + ch * pairs * 2,
        "triangle.output": ch * pairs * 2 + pairs * cz * pair_bytes + pairs * cz * out_bytes,
    }


def recorded_traffic() -> dict:
    """traffic_bytes lines of the committed rocprof summary, if present."""
    try:
        text = open(TRAFFIC_FILE, encoding="utf-8").read()
    except OSError:
        return {}
    return {m.group(1): int(m.group(2)) for m in re.finditer(r"traffic_bytes (\S+) (\d+)", text)}


def triangle_weights(seed: int, cz: int, ch: int) -> dict:
    from oracle import ref

    weights = {}
    shapes = ref.triangle_weight_shapes(cz, ch)
    for i, name in enumerate(ref.TRIANGLE_ORDER):
        shape = shapes[name]
        if name.startswith("layerNorm"):
            weights[name] = ref.normal(seed + 100 + i, shape, 0.01, 1.0 if name.endswith("Weight") else 0.0)
        elif name.endswith("Bias"):
            weights[name] = ref.normal(seed + 100 + i, shape, 0.02)
        else:
            weights[name] = ref.normal(seed + 100 + i, shape, 1.0 / shape[1])
    return weights


def cpu_baseline() -> dict:
    """The reference's CPU path timed on this host, a reported baseline.

    Primary: oracle/cpu_reference.js, the reference's
    triangleMultiplicationOutgoingReference (src/triangle/cpu-reference.ts:56-100)
    in plain JavaScript, under this machine's node, one JS thread, on the
    reference's deterministic input at L = 160 (a bounded sample, ~10-20 s).
    Secondary: the C oracle (oracle/afref.c, -O2, no fast-math) on one thread
    and on every core (OpenMP). Each is reported as the outgoing operator's
    algorithmic TFLOP/s (the unit of `value`) and as the L = 384 step it
    extrapolates to by FLOPs."""
    import shutil
    import subprocess

    from oracle import ref

    full = 2 * sum(triangle_flops(L, CZ, CH).values())

    def rate(length, seconds):
        flops = sum(triangle_flops(length, CZ, CH).values())
        return flops / seconds / 1e12, full / (flops / seconds) * 1e3

    secondary = {}
    for threads, length in ((1, 128), (ref.max_threads(), 256)):
        inp = ref.deterministic_triangle_input(length, CZ, CH, seed=11)
        ref.set_threads(threads)
        start = time.perf_counter()
        ref.triangle("outgoing", inp["z"], inp["mask"], inp["weights"])
        seconds = time.perf_counter() - start
        tflops, step_ms = rate(length, seconds)
        secondary[f"c_oracle_{threads}_threads"] = {
            "value": tflops, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"oracle/afref.c, one outgoing triangle multiplication at L={length}, c_z=c_h={CH} "
                      f"({seconds:.2f} s)", "ms_per_step_extrapolated": step_ms}
    ref.set_threads(ref.max_threads())

    node = shutil.which("node")
    length = 160
    if node is not None:
        proc = subprocess.run([node, os.path.join(ROOT, "oracle", "cpu_reference.js"), str(length), str(CZ), str(CH),
                               "11"], capture_output=True, text=True, timeout=600)
        if proc.returncode == 0:
            js = json.loads(proc.stdout.strip().splitlines()[-1])
            tflops, step_ms = rate(length, js["seconds"])
            return {"value": tflops, "unit": "TFLOP/s", "cores": 1, "kind": "port",
                    "sample": f"the reference's cpu-reference.ts loops in plain JS (oracle/cpu_reference.js) under "
                              f"node {js['node']}, one JS thread, on {js['cpus']} host CPUs ({js['cpuModel']}): one "
                              f"outgoing triangle multiplication at L={length}, c_z=c_h={CH} ({js['seconds']:.1f} s); "
                              f"a full L={L} step would take {step_ms / 1e3:.0f} s",
                    "node": js["node"], "host_cpus": js["cpus"], "cpu_model": js["cpuModel"],
                    "ms_per_step_extrapolated": step_ms, "secondary": secondary}
    one = secondary["c_oracle_1_threads"]
    return dict(one, secondary=secondary, note="node unavailable: the C oracle is the primary figure")


def copy_probe(mib: int) -> None:
    import torch

    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_each_way": n * 4, "launches": 10}))


# tools/gemm-candidates.ts:637-669 (SHAPES): the model's projection and
# contraction shapes, their 32-aligned twins and the calibration probe shapes.
GEMM_SHAPES = [
    ("opm-contract", 128, 508, 32000), ("opm-out", 4096, 1024, 128), ("opm-out2", 3000, 1024, 128),
    ("project", 29972, 256, 1024), ("output", 29972, 256, 256), ("trans1", 29972, 256, 1024),
    ("trans2", 29972, 1024, 256), ("extra1", 60416, 64, 256), ("project32", 29984, 256, 1024),
    ("output32", 29984, 256, 256), ("trans2-32", 29984, 1024, 256), ("opmcon32", 128, 512, 32000),
    ("probeA", 1024, 512, 512), ("probeB", 8192, 128, 512), ("probeC", 16384, 256, 256), ("probeD", 4096, 256, 512),
    # trans2 with the bundle's mixed-q8 weight: int8 [N][K], per-column f32 scales
    # (tools/quantize-web-model.ts:98-119 quantises every weight of the bundle).
    ("trans2-q8", 29972, 1024, 256, "i8"),
    # f32 activations into the f16 units (the reference's f32 storage,
    # src/runtime/gemm.ts:308-321 sourceFormat) and the outer-product mean's
    # sequence-major operand as a row-contiguous source [K][M]
    # (src/evoformer/outer-product-mean.ts:376-389).
    ("project-f32a", 29972, 256, 1024, "f16", "f32"), ("trans2-f32a", 29972, 1024, 256, "f16", "f32"),
    ("opmcon32-rowA", 128, 512, 32000, "f16", "f16", "row"),
]
GEMM_CANDIDATES = [("register", 64, 64), ("register", 64, 128), ("register", 128, 64), ("register", 128, 128),
                   ("lds_dma", 128, 128), ("lds_dma", 192, 192), ("lds_dma", 128, 256), ("lds_dma", 256, 256),
                   ("stream", 64, 512)]


def gemm_shapes(launches: int = 20) -> dict:
    """The gemm-candidates benchmark (tools/gemm-candidates.ts:571-669,
    tools/benchmark-gemm.ts:46-104) on MI355X: every candidate tile of the
    f16 GEMM (f16 operands, f32 accumulation, f16 output, weight [N][K]) on
    every shape of SHAPES, beside the variant the heuristic picks; a shape
    marked i8 has an int8 weight with per-column scales (the plan widens it
    to f16 for LDS_DMA, inside the timed run); one marked with an f32 source
    or a row-contiguous ([K][M]) source says so. A candidate is timed only
    where its family takes the operands (LDS_DMA: K even, a multiple of 8 for
    an f32 or row-contiguous source; STREAM: an f16 k-contiguous source, K of
    64, 128 or 256 and N a multiple of 64), as the library would otherwise
    run it on another family. ms is the average of `launches` back-to-back
    launches between two events after three warm-up launches."""
    import torch

    from afhip import device, gemm

    device.open_device(0)
    dev = device.device()
    out = {"unit": "ms", "launches": launches, "shapes": []}
    for name, M, K, N, *kind in GEMM_SHAPES:
        wdt, adt, a_layout = (list(kind) + ["f16", "f16", "k"][len(kind):])[:3]
        a = torch.randn(*((K, M) if a_layout == "row" else (M, K)), device=dev)
        a = a if adt == "f32" else a.half()
        if wdt == "i8":
            w = torch.randint(-127, 128, (N, K), device=dev, dtype=torch.int8)
            scale = torch.rand(N, device=dev) * 9e-3 + 1e-3
        else:
            w = (torch.randn(N, K, device=dev) / K ** 0.5).half()
            scale = None
        c = torch.empty(M, N, device=dev, dtype=torch.float16)

        def run(pin):
            gemm.force_variant(pin)
            try:
                plan = gemm.TiledGemm(M, K, N, precision="f16", a_dtype=adt, w_dtype=wdt, w_layout="k",
                                      out_dtype="f16", epilogue=("scale",) if scale is not None else (),
                                      a_layout=a_layout)
                chosen = plan.variant()
                for _ in range(3):
                    plan.run(a, w, scale=scale, out=c)
                start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                start.record()
                for _ in range(launches):
                    plan.run(a, w, scale=scale, out=c)
                stop.record()
                stop.synchronize()
                return chosen, start.elapsed_time(stop) / launches
            finally:
                gemm.force_variant(None)

        flops = 2.0 * M * K * N
        chosen, heuristic_ms = run(None)
        entry = {"shape": name, "M": M, "K": K, "N": N, "weight": wdt, "source": adt, "source_layout": a_layout,
                 "heuristic": {"variant": chosen.name, "ms": round(heuristic_ms, 5),
                               "tflops": round(flops / heuristic_ms / 1e9, 1)},
                 "candidates": {}}
        for kernel, tr, tc in GEMM_CANDIDATES:
            if kernel == "lds_dma" and K % (2 if adt == "f16" and a_layout == "k" else 8):
                continue
            if kernel == "stream" and (K not in (64, 128, 256) or N % 64 or adt != "f16" or a_layout != "k"):
                continue
            v = gemm.GemmVariant("f16", tr, tc, source="pinned", kernel=kernel)
            _, ms = run(v)
            entry["candidates"][v.name] = {"ms": round(ms, 5), "tflops": round(flops / ms / 1e9, 1)}
        best = min(entry["candidates"].items(), key=lambda kv: kv[1]["ms"])
        entry["best"] = {"variant": best[0], "ms": best[1]["ms"]}
        entry["heuristic_over_best"] = round(heuristic_ms / best[1]["ms"], 3)
        out["shapes"].append(entry)
        print(f"gemm-shapes: {name} heuristic {chosen.name} {heuristic_ms:.4f} ms, best {best[0]} "
              f"{best[1]['ms']:.4f} ms", file=sys.stderr, flush=True)
        del a, w, c
    return out


# Untimed clock settle before each measurement's warm-up steps. From a cold
# start the headline step runs ~20% slow for its first ~20 ms of continuous
# work while the GPU's clocks ramp (0.118 ms an operation, then 0.0955 from
# ~20 ms on, measured on one MI355X), so a short timed region would measure
# the ramp. `--settle-ms 0` turns it off.
SETTLE_MS = 60.0


def timed(fn, steps: int, warmup: int):
    """(ms per call by wall clock around synchronised loops, per-kernel
    average ms from the library's hipEvents). The calls run for SETTLE_MS of
    wall time first (untimed), then `warmup` untimed calls, then the timed
    ones."""
    import torch

    from afhip import device

    if SETTLE_MS > 0:
        start = time.perf_counter()
        while (time.perf_counter() - start) * 1e3 < SETTLE_MS:
            for _ in range(4):
                fn()
            torch.cuda.synchronize()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - start) * 1e3 / steps
    device.timing_reset()
    device.timing_enable(True)
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    report = device.timing_report()
    device.timing_enable(False)
    return ms, {k: v["total_ms"] / v["count"] for k, v in report.items()}


def rate(kernel: str, ms: float, *, flops: float | None = None, nbytes: float | None = None,
         peak_tflops: float = PEAK_F16_TFLOPS, traffic=None) -> dict:
    if flops is not None:
        achieved = flops / (ms * 1e-3) / 1e12
        out = {"kernel": kernel, "bound": "mfma", "achieved": round(achieved, 2), "peak": peak_tflops,
               "unit": "TFLOP/s", "frac": round(achieved / peak_tflops, 4)}
    else:
        achieved = nbytes / (ms * 1e-3) / 1e9
        out = {"kernel": kernel, "bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
               "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4)}
    out["traffic"] = traffic
    out["avg_ms"] = round(ms, 5)
    return out


def measure_configs(steps: int, warmup: int, which=(1, 2, 4, 5)) -> dict:
    """BASELINE configs 1, 2, 4 and 5, each with synthetic inputs of the
    stated shape and distribution."""
    import numpy as np
    import torch

    from afhip import device, gemm, opm, transition, triangle
    from oracle import ref

    dev = device.device()
    out = {}
    if 1 in which:
        # Config 1: pair-transition first linear, f32, 4096x128x512, bias, ReLU.
        s = SEED
        x = torch.from_numpy(ref.normal(s, (4096, 128))).to(dev)
        w = torch.from_numpy(np.ascontiguousarray(ref.normal(s + 1, (128, 512), 1 / 128).T)).to(dev)  # [N][K]
        b = torch.from_numpy(ref.normal(s + 2, (512,), 0.02)).to(dev)
        plan = gemm.TiledGemm(4096, 128, 512, precision="f32", w_layout="k", epilogue=("bias", "relu"))
        y = plan.run(x, w, bias=b)
        ms, k = timed(lambda: plan.run(x, w, bias=b, out=y), steps * 5, warmup)
        kms = k.get("gemm", ms)
        out["1_pair_transition_linear_f32"] = {
            "ms": round(kms, 5), "wall_ms": round(ms, 5), "variant": plan.variant().name,
            "roofline": rate("gemm", kms, flops=2 * 4096 * 128 * 512, peak_tflops=PEAK_F32_TFLOPS)}
        del x, w, b, y, plan
    if 2 in which:
        # Config 2: fused QKV+gate projection, mixed-q8: X f16 [131072x256],
        # W int8 [256x1024] (per-column f32 scales), f32 accumulate, f16 out.
        s = SEED + 1
        rows = 512 * 256
        x = torch.from_numpy(ref.round_f16(ref.normal(s, (rows, 256)))).half().to(dev)
        q = torch.from_numpy(np.ascontiguousarray(ref.uniform_i8(s + 1, (256, 1024)).T)).to(dev)  # [N][K] int8
        scale = torch.from_numpy(ref.uniform(s + 2, (1024,), 1e-3, 1e-2)).to(dev)
        plan = gemm.TiledGemm(rows, 256, 1024, precision="f16", a_dtype="f16", w_dtype="i8", w_layout="k",
                              out_dtype="f16", epilogue=("scale", "attention"), heads=8, head_dim=32)
        y = plan.run(x, q, scale=scale)
        ms, k = timed(lambda: plan.run(x, q, scale=scale, out=y), steps, warmup)
        kms = k.get("gemm", ms)
        nbytes = 2 * rows * 256 + 256 * 1024 + 4 * 1024 + 2 * rows * 1024
        out["2_qkv_gate_projection_q8"] = {
            "ms": round(kms, 5), "wall_ms": round(ms, 5), "variant": plan.variant().name,
            "tflops": round(2 * rows * 256 * 1024 / (kms * 1e-3) / 1e12, 2),
            "roofline": rate("gemm", kms, nbytes=nbytes, traffic=recorded_traffic().get("config2.gemm"))}
        del x, q, scale, y, plan
    if 4 in which:
        # Config 4: outer-product mean, N_seq=512, N_res=256, c_m=256 -> 32+32 -> 128, f16.
        s = SEED + 3
        S4, L4, CM, CO, CZ4 = 512, 256, 256, 32, 128
        act = torch.from_numpy(ref.round_f16(ref.normal(s, (S4, L4, CM)))).half().to(dev)
        mask = torch.ones((S4, L4), dtype=torch.float32, device=dev)
        wts = {"layerNormScale": ref.normal(s + 1, (CM,), 0.01, 1.0), "layerNormOffset": ref.normal(s + 2, (CM,), 0.01),
               "leftWeight": ref.normal(s + 3, (CM, CO), 1 / CM), "leftBias": ref.normal(s + 4, (CO,), 0.02),
               "rightWeight": ref.normal(s + 5, (CM, CO), 1 / CM), "rightBias": ref.normal(s + 6, (CO,), 0.02),
               "outputWeight": ref.normal(s + 7, (CO * CO, CZ4), 1 / (CO * CO)), "outputBias": ref.normal(s + 8, (CZ4,), 0.02)}
        op = opm.OuterProductMean(S4, L4, CM, CO, CZ4, precision="f16", msa_dtype="f16", out_dtype="f32")
        op.prepare(wts)
        y = op(act, mask)
        ms, k = timed(lambda: op(act, mask, out=y), steps, warmup)
        # opm.fused is the contraction and the output projection in one launch
        # (opm.contract + opm.output where the shape does not fuse).
        flops4 = {"opm.project": 2 * S4 * L4 * CM * 2 * CO, "opm.contract": 2 * (L4 * CO) ** 2 * S4,
                  "opm.output": 2 * L4 * L4 * CO * CO * CZ4}
        flops4["opm.fused"] = flops4["opm.contract"] + flops4["opm.output"]
        total4 = flops4["opm.project"] + flops4["opm.fused"]
        out["4_outer_product_mean"] = {
            "ms": round(ms, 5), "tflops": round(total4 / (ms * 1e-3) / 1e12, 2),
            "kernel_ms": {kk: round(v, 5) for kk, v in k.items()},
            "kernels": {kk: rate(kk, k[kk], flops=f) for kk, f in flops4.items() if kk in k and kk != "opm.project"}}
        # The projection is bandwidth-bound: it reads m f16 and the mask and
        # writes left and right f16 ([L*c_o][S] each).
        if "opm.project" in k:
            out["4_outer_product_mean"]["kernels"]["opm.project"] = rate(
                "opm.project", k["opm.project"], nbytes=2 * S4 * L4 * CM + 4 * S4 * L4 + 2 * 2 * L4 * CO * S4)
        del act, mask, op, y
    if 5 in which:
        # Config 5: long-complex pair stack at N_res=1024: triangle incoming
        # (128 batched 1024^3 contractions) + pair transition 128->512->128 over
        # 1,048,576 rows, f16 activations, f32 accumulation.
        s = SEED + 4
        L5 = 1024
        z = torch.from_numpy(ref.round_f16(ref.normal(s, (L5, L5, CZ)))).half().to(dev)
        mask = torch.ones((L5, L5), dtype=torch.float32, device=dev)
        tri = triangle.TriangleMultiplication(L5, CZ, CH, direction="incoming", precision="f16", pair_dtype="f16",
                                              out_dtype="f16")
        tri.prepare(triangle_weights(s, CZ, CH))
        zo = tri(z, mask)
        ms, k = timed(lambda: tri(z, mask, out=zo), max(3, steps // 4), 1)
        f5 = triangle_flops(L5, CZ, CH)
        entry = {"triangle_incoming_ms": round(ms, 4),
                 "triangle_tflops": round((f5["project"] + f5["contract"] + f5["output"] + f5["gate"]) / (ms * 1e-3) / 1e12, 2),
                 "triangle_kernel_ms": {kk: round(v, 5) for kk, v in k.items()}}
        if "triangle.contract" in k:
            entry["contract"] = rate("triangle.contract", k["triangle.contract"], flops=f5["contract"],
                                     traffic=recorded_traffic().get("config5.contract"))
        rows5 = L5 * L5
        tw = {"layerNormScale": ref.normal(s + 20, (CZ,), 0.01, 1.0), "layerNormOffset": ref.normal(s + 21, (CZ,), 0.01),
              "firstWeight": ref.normal(s + 22, (CZ, 4 * CZ), 1 / CZ), "firstBias": ref.normal(s + 23, (4 * CZ,), 0.02),
              "secondWeight": ref.normal(s + 24, (4 * CZ, CZ), 1 / (4 * CZ)), "secondBias": ref.normal(s + 25, (CZ,), 0.02)}
        trans = transition.Transition(rows5, CZ, 4 * CZ, precision="f16", in_dtype="f16", out_dtype="f16")
        trans.prepare(tw)
        zf = z.reshape(rows5, CZ)
        to = trans(zf)
        ms_t, k_t = timed(lambda: trans(zf, out=to), max(3, steps // 4), 1)
        ft = 2 * 2 * rows5 * CZ * 4 * CZ
        entry.update({"transition_ms": round(ms_t, 4), "transition_tflops": round(ft / (ms_t * 1e-3) / 1e12, 2),
                      "transition_kernel_ms": {kk: round(v, 5) for kk, v in k_t.items()}})
        # The fused transition keeps the hidden activation on chip: MFMA-bound
        # (274.9 GFLOP against 537 MB of f16 rows in and out).
        if "transition.fused" in k_t:
            entry["transition"] = rate("transition.fused", k_t["transition.fused"], flops=ft,
                                       traffic=recorded_traffic().get("config5.transition"))
        out["5_long_complex_pair_stack_l1024"] = entry
        del z, mask, tri, zo, trans, zf, to
        torch.cuda.empty_cache()
    if "attention" in which:
        out["attention"] = measure_attention(steps, warmup)
    if "block" in which:
        out["evoformer_block"] = measure_block(steps, warmup)
    return out


def measure_block(steps: int, warmup: int) -> dict:
    """One whole Evoformer block on the device (afhip_execution_evoformer_block:
    MSA row and column attention, MSA transition, outer-product mean, the two
    triangle multiplications and attentions, pair transition) at config 4's
    shape: N_seq = 512, N_res = 256, c_m = 256, c_z = 128, f16, synthetic
    weights ~N(0, 1/fan_in) and activations ~N(0, 1), all-ones masks."""
    import torch

    from afhip import device
    from afhip.execution import EvoformerBlock, Execution
    from oracle import ref

    dev = device.device()
    S, L, cm, cz, co, ch = 512, 256, 256, 128, 32, 128
    s = SEED + 7
    counter = iter(range(1000))

    def n(shape, fan_in=None, mean=0.0):
        return ref.normal(s + next(counter), shape, 1.0 / fan_in if fan_in else 0.01, mean)

    def att(c):
        return {"queryNormScale": n((c,), mean=1.0), "queryNormOffset": n((c,)), "queryWeight": n((c, c), c),
                "keyWeight": n((c, c), c), "valueWeight": n((c, c), c), "gatingWeight": n((c, c), c),
                "gatingBias": n((c,), mean=1.0), "outputWeight": n((c, c), c), "outputBias": n((c,))}

    def trans(c):
        return {"layerNormScale": n((c,), mean=1.0), "layerNormOffset": n((c,)), "firstWeight": n((c, 4 * c), c),
                "firstBias": n((4 * c,)), "secondWeight": n((4 * c, c), 4 * c), "secondBias": n((c,))}

    w = {"msaRowAttention": {"attention": att(cm), "pairLayerNormScale": n((cz,), mean=1.0),
                             "pairLayerNormOffset": n((cz,)), "pairProjectionWeight": n((cz, 8), cz)},
         "msaColumnAttention": {"attention": att(cm)}, "msaTransition": trans(cm),
         "outerProductMean": {"layerNormScale": n((cm,), mean=1.0), "layerNormOffset": n((cm,)),
                              "leftWeight": n((cm, co), cm), "leftBias": n((co,)), "rightWeight": n((cm, co), cm),
                              "rightBias": n((co,)), "outputWeight": n((co * co, cz), co * co), "outputBias": n((cz,))},
         "triangleMultiplicationOutgoing": triangle_weights(s + 500, cz, ch),
         "triangleMultiplicationIncoming": triangle_weights(s + 600, cz, ch),
         "triangleAttentionStarting": {"attention": att(cz), "pairProjectionWeight": n((cz, 4), cz)},
         "triangleAttentionEnding": {"attention": att(cz), "pairProjectionWeight": n((cz, 4), cz)},
         "pairTransition": trans(cz)}
    ex = Execution()
    blk = EvoformerBlock(ex, L, sequences=S, c_m=cm, c_z=cz, c_outer=co, c_hidden=ch)
    blk.prepare(w)
    msa = torch.from_numpy(ref.round_f16(ref.normal(s + 900, (S, L, cm)))).half().to(dev)
    pair = torch.from_numpy(ref.round_f16(ref.normal(s + 901, (L, L, cz)))).half().to(dev)
    msa_mask = torch.ones((S, L), dtype=torch.float32, device=dev)
    pair_mask = torch.ones((L, L), dtype=torch.float32, device=dev)
    m0, z0 = msa.clone(), pair.clone()

    def step():
        msa.copy_(m0)
        pair.copy_(z0)
        blk(msa, msa_mask, pair, pair_mask)

    def resets():
        msa.copy_(m0)
        pair.copy_(z0)

    ms, k = timed(step, max(5, steps // 10), warmup)
    copies_ms, _ = timed(resets, max(5, steps // 10), warmup)
    entry = {"ms": round(ms, 4), "workload": f"Evoformer block, N_seq={S}, N_res={L}, c_m={cm}, c_z={cz}, f16",
             "copies_ms": round(copies_ms, 4), "ms_without_copies": round(ms - copies_ms, 4),
             "kernel_avg_ms": {kk: round(v, 5) for kk, v in sorted(k.items(), key=lambda kv: -kv[1])}}
    entry["note"] = ("ms includes two device copies that reset the MSA and the pair before each block; "
                     "copies_ms times those copies alone and ms_without_copies is the difference; "
                     "kernel_avg_ms averages every launch under a label, whichever step made it")
    ex.release()
    return entry


def measure_attention(steps: int, warmup: int) -> dict:
    """The Evoformer's attentions at f16 (head dimension 32, the MFMA flash
    kernel), synthetic inputs: triangle attention around the starting node at
    N_res=384 (c_z 128, 4 heads, normalized-input pair bias) and MSA row
    attention at N_seq=512, N_res=256 (c_m 256, 8 heads, pair bias from a
    [256, 256, 128] pair), and MSA column attention at the same shape
    (transposed: 256 batch entries of 512 queries, no pair bias). Flash FLOPs:
    4 d per (batch, head, query, key)."""
    import numpy as np
    import torch

    from afhip import attention, device
    from oracle import ref

    dev = device.device()
    out = {}
    for name, B, Q, C, H, pair, Cp, s in (("triangle_start_l384", 384, 384, 128, 4, "normalized-input", 0, SEED + 5),
                                          ("msa_row_s512_l256", 512, 256, 256, 8, "separate", 128, SEED + 6),
                                          ("msa_column_s512_l256", 256, 512, 256, 8, None, 0, SEED + 7)):
        w = {"queryNormScale": ref.normal(s, (C,), 0.01, 1.0), "queryNormOffset": ref.normal(s + 1, (C,), 0.01),
             "queryWeight": ref.normal(s + 2, (C, C), 1 / C), "keyWeight": ref.normal(s + 3, (C, C), 1 / C),
             "valueWeight": ref.normal(s + 4, (C, C), 1 / C), "gatingWeight": ref.normal(s + 5, (C, C), 1 / C),
             "gatingBias": ref.normal(s + 6, (C,), 0.1, 1.0), "outputWeight": ref.normal(s + 7, (C, C), 1 / C),
             "outputBias": ref.normal(s + 8, (C,), 0.01)}
        pc = Cp or C
        pb = None if pair is None else {"source": pair, "projectionWeight": ref.normal(s + 9, (pc, H), 1 / pc)}
        if pair == "separate":
            pb.update(channels=Cp, layerNormScale=ref.normal(s + 10, (Cp,), 0.01, 1.0),
                      layerNormOffset=ref.normal(s + 11, (Cp,), 0.01))
        op = attention.Attention(B, Q, C, H, transpose=pair is None, pair_bias=pair, pair_channels=Cp,
                                 precision="f16", in_dtype="f16", out_dtype="f16", residual=True)
        op.prepare(attention.pack_weights(w, pb))
        x = torch.from_numpy(ref.round_f16(ref.normal(s + 12, (B * Q, C)))).half().to(dev)
        mask = torch.ones(B * Q, dtype=torch.float32, device=dev)
        p = None
        if pair == "separate":
            p = torch.from_numpy(ref.round_f16(ref.normal(s + 13, (Q * Q * Cp,)))).half().to(dev)
        y = x.clone()
        ms, k = timed(lambda: op(x, mask, p, out=y), max(5, steps // 5), warmup)
        d = C // H
        flash = 4 * B * H * Q * Q * d
        total = flash + 2 * B * Q * C * 4 * C + 2 * B * Q * C * C + (2 * Q * Q * pc * H if pair else 0)
        entry = {"ms": round(ms, 4), "tflops": round(total / (ms * 1e-3) / 1e12, 2),
                 "kernel_ms": {kk: round(v, 5) for kk, v in k.items()}}
        if "attention.flash" in k:
            entry["flash"] = rate("attention.flash", k["attention.flash"], flops=flash)
        out[name] = entry
        del op, x, mask, p, y
        torch.cuda.empty_cache()
    return out


def main() -> None:
    global SETTLE_MS
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    # A headline step is ~0.2 ms: 100 steps keep the timed region short while
    # averaging past the first steps' clock ramp.
    parser.add_argument("--steps", type=int, default=100)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--settle-ms", type=float, default=SETTLE_MS,
                        help="untimed run time before each measurement's warm-up steps, so the timed steps run at "
                             "settled clocks (0: none)")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--headline-only", action="store_true", help="skip BASELINE configs 1, 2, 4 and 5")
    parser.add_argument("--configs", default="1,2,4,5,attention,block",
                        help="comma-separated BASELINE configs to measure besides the headline (config 3), "
                             "'attention' for the Evoformer attentions and 'block' for a whole Evoformer block")
    parser.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                        help="only run a plain device-to-device copy of MIB MiB 10 times (the known-size kernel "
                             "rocprof's FETCH_SIZE / WRITE_SIZE readings are scaled by) and exit")
    parser.add_argument("--gemm-shapes", action="store_true",
                        help="only run the gemm-candidates benchmark (every candidate tile and the heuristic's "
                             "choice on the reference's SHAPES) and print it as one JSON line")
    args = parser.parse_args()
    SETTLE_MS = args.settle_ms
    if args.gemm_shapes:
        print(json.dumps(gemm_shapes()))
        return
    if args.copy_probe:
        copy_probe(args.copy_probe)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: the path runs on one device and bench.py "
                                   "--gpus N>1 is not supported: every GPU box here has one GPU; the path would shard on "
                                   "output rows i, one process per GPU, with one all-gather of b"}))
        sys.exit(2)

    import numpy as np
    import torch

    from afhip import device, triangle
    from oracle import ref  # input generation only (splitmix64 + Box-Muller)

    device.open_device(0)
    dev = device.device()
    seed = SEED + 2
    z = ref.round_f16(ref.normal(seed, (L, L, CZ)))
    mask = np.ones((L, L), np.float32)
    weights = triangle_weights(seed, CZ, CH)
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

    ms_per_step, per_kernel = timed(step, args.steps, args.warmup)

    flops = triangle_flops(L, CZ, CH)
    step_flops = 2 * sum(flops.values())
    value = step_flops / (ms_per_step * 1e-3) / 1e12
    traffic = recorded_traffic()
    nbytes = triangle_bytes(L, CZ, CH)
    kernels = {}
    for name in ("triangle.project", "triangle.contract", "triangle.output"):
        if name not in per_kernel:
            continue
        if name == "triangle.contract":
            kernels[name] = rate(name, per_kernel[name], flops=flops["contract"], traffic=traffic.get(name))
        else:
            kernels[name] = rate(name, per_kernel[name], nbytes=nbytes[name], traffic=traffic.get(name))
        kernels[name]["algorithmic"] = flops["contract"] if name == "triangle.contract" else nbytes[name]
    dominant = max(kernels, key=lambda n: kernels[n]["avg_ms"])
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_ms": args.settle_ms,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "triangle multiplication outgoing + incoming, N_res=384, c_z=c_hidden=128, "
                               "f16 in, f32 accumulate, f32 out (BASELINE config 3)",
                   "n_res": L, "c_z": CZ, "c_hidden": CH, "parallelism": "none (1 GPU)"},
        "triangle_ms": round(ms_per_step / 2, 4),
        "roofline": kernels[dominant],
        "kernels": kernels,
        "kernel_ms": {k: round(v, 5) for k, v in per_kernel.items()},
    }
    # The same step with a mask that is 0 for ~15% of the pairs: the projection then multiplies by the
    # mask (all-ones tiles skip that), and the timing shows what a real MSA-derived mask costs.
    md.copy_(torch.from_numpy((ref.uniform(seed + 1, (L, L), 0, 1) > 0.15).astype(np.float32)))
    ms_masked, per_kernel_masked = timed(step, args.steps, args.warmup)
    result["masked_15pct"] = {"ms_per_step": round(ms_masked, 4), "triangle_ms": round(ms_masked / 2, 4),
                              "kernel_ms": {k: round(v, 5) for k, v in per_kernel_masked.items()},
                              "note": "secondary: same workload, mask 0 on ~15% of pairs (seeded); not the headline value"}
    which = tuple(c.strip() if c.strip() in ("attention", "block") else int(c) for c in args.configs.split(",")
                  if c.strip()) if not args.headline_only else ()
    if which:
        del ops, zd, md
        torch.cuda.empty_cache()
        result["configs"] = measure_configs(args.steps, args.warmup, which)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result))


if __name__ == "__main__":
    main()
