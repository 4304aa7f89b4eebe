"""Benchmark of the quantized-linear hot path on one MI355X.

Metric: int4 dequant-GEMV GB/s (% HBM peak) at Qwen2.5-7B
shapes; prefill GEMM TFLOP/s.

A "step" is one dequant-matmul call over one batch of synthetic inputs that
are resident in HBM.  The headline ``value`` is the decode GEMV at the
Qwen2.5-7B down-proj shape (M=1, K=18944, N=3584, int4
g128): algorithmic bytes (weights + scales + zeros + x + y, each once) per
step divided by the time per step.  The other BASELINE configs are measured
the same way and reported under ``extra``.

Method:
* weights, scales and zeros rotate through enough independent copies that the
  working set exceeds the 256 MB Infinity Cache, so HBM is really read;
* the launches are captured in a HIP graph (host launch overhead excluded),
  the graph is replayed, and HIP events on the replay stream bracket the
  timed region, with a device synchronisation on both sides;
* the CPU baseline is the reference's path restated on this host: torch-CPU
  exact fp16 dequantize, then fp32 torch.matmul (warm-up 5, median of 20),
  on the same workload, with the core count and CPU model stated.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only NAME]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "metal-native_amd"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "int4 dequant-GEMV GB/s (% HBM peak) at Qwen2.5-7B shapes; prefill GEMM TFLOP/s"
HBM_PEAK_GBS = 8000.0
FP16_MFMA_PEAK_TFLOPS = 2500.0
CACHE_BYTES = 256 * 2**20
ROTATE_TARGET = int(1.3 * CACHE_BYTES)


KERNEL_DESC = {
    "rows": "persistent row-block dequant GEMV, v_mfma_f32_16x16x32_f16, fp32 accumulation",
    "decode": "split-K dequant GEMV, v_mfma_f32_16x16x32_f16, fp32 accumulation",
    "tiled": "dequant GEMM, v_mfma_f32_32x32x16_f16, fp32 accumulation",
}
TRAFFIC_JSON = os.path.join(ROOT, "profiles", "traffic_rows_kernel_cfg2_m1.json")


def traffic_bytes():
    """HBM bytes per launch of the headline kernel, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (each counter scaled by what it
    reads for a plain copy of known size).  None when no summary exists."""
    try:
        with open(TRAFFIC_JSON) as f:
            return json.load(f).get("traffic_bytes_per_launch")
    except (OSError, ValueError):
        return None


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# --------------------------------------------------------------------------
# workloads
# --------------------------------------------------------------------------

CONFIGS = {
    # name: (qtype, M, K, N(weight rows), g, epilogue, bound)
    "cfg1_qwen05b_gate_m1": ("int4", 1, 896, 4864, 64, None, "hbm"),
    "cfg2_qwen7b_down_m1": ("int4", 1, 18944, 3584, 128, None, "hbm"),
    "cfg2_qwen7b_down_m4": ("int4", 4, 18944, 3584, 128, None, "hbm"),
    "cfg2_qwen7b_down_m8": ("int4", 8, 18944, 3584, 128, None, "hbm"),
    "cfg3_llama3b_qkv_m512": ("int4", 512, 3072, 5120, 128, None, "mfma"),
    "cfg3_llama3b_qkv_m512_g64": ("int4", 512, 3072, 5120, 64, None, "mfma"),
    "cfg3_llama3b_qkv_m512_g32": ("int4", 512, 3072, 5120, 32, None, "mfma"),
    "cfg4_qwen7b_gateup_int8_swiglu_m1": ("int8", 1, 3584, 2 * 18944, 3584, "swiglu", "hbm"),
    "cfg4_qwen7b_gateup_int8_swiglu_m16": ("int8", 16, 3584, 2 * 18944, 3584, "swiglu", "hbm"),
    "cfg4_qwen7b_gateup_int8_swiglu_m64": ("int8", 64, 3584, 2 * 18944, 3584, "swiglu", "hbm"),
    # the band between decode and prefill at the config-2 shape (not a baseline config)
    "midband_qwen7b_down_m16": ("int4", 16, 18944, 3584, 128, None, "hbm"),
    "midband_qwen7b_down_m32": ("int4", 32, 18944, 3584, 128, None, "hbm"),
}
HEADLINE = "cfg2_qwen7b_down_m1"


def algo_bytes(qtype, M, K, N, g, epi):
    """Weights + scales + zeros + x + y, each counted once (int8 per-channel:
    one fp16 scale per row and no zeros read as bytes of the metric)."""
    G = (K + g - 1) // g
    w = N * K // 2 if qtype == "int4" else N * K
    sz = 2 * N * G * 2 if qtype == "int4" else N * G * 2
    n_out = N // 2 if epi == "swiglu" else N
    return w + sz + M * K * 2 + M * n_out * 2


def flops(M, K, N):
    return 2.0 * M * N * K


def make_weights(qtype, K, N, g, gen, device):
    import torch

    G = (K + g - 1) // g
    if qtype == "int4":
        wp = torch.randint(0, 256, (N, K // 2), dtype=torch.uint8, device=device, generator=gen)
        s = (torch.rand((N, G), device=device, generator=gen) * 0.015 + 0.005).half()
        zp = torch.randint(0, 16, (N, G), device=device, generator=gen).float()
        z = ((zp - 8.0) * s.float()).half()
    else:
        wp = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=device, generator=gen)
        s = (torch.rand((N, G), device=device, generator=gen) * 0.009 + 0.001).half()
        z = torch.zeros_like(s)
    return wp, s, z


def measure(name, steps, warmup, device):
    import torch

    import metal_native as mn

    qtype, M, K, N, g, epi, bound = CONFIGS[name]
    gen = torch.Generator(device=device)
    gen.manual_seed(0)
    per_copy = algo_bytes(qtype, M, K, N, g, epi)
    copies = max(2, min(256, -(-ROTATE_TARGET // per_copy)))
    weights = [make_weights(qtype, K, N, g, gen, device) for _ in range(copies)]
    x = torch.randn((M, K), device=device, generator=gen).half()
    fn = lambda i: mn.dequant_matmul(x, *weights[i % copies], g, qtype, epilogue=epi)

    # two graphs cycling through the copies: `warmup` untimed launches, then
    # exactly `steps` timed ones
    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(stream):
        for i in range(copies):
            fn(i)  # eager: workspace for this stream, code objects loaded
    torch.cuda.synchronize(device)
    path = mn.last_path()
    gwarm = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gwarm, stream=stream):
        for i in range(max(1, warmup)):
            fn(i)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(steps):
            fn(i)
    cur = torch.cuda.current_stream(device)
    gwarm.replay()
    torch.cuda.synchronize(device)
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    t0.record(cur)
    graph.replay()
    t1.record(cur)
    torch.cuda.synchronize(device)
    wall = time.perf_counter() - wall0
    ms = t0.elapsed_time(t1)
    n_steps = steps
    us_per_step = ms * 1000.0 / n_steps
    gbs = per_copy / (us_per_step * 1e-6) / 1e9
    res = {
        "us_per_step": round(us_per_step, 3),
        "GB/s": round(gbs, 1),
        "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
        "algo_bytes_per_step": per_copy,
        "steps": n_steps,
        "copies_rotated": copies,
        "working_set_MB": round(copies * per_copy / 2**20, 1),
        "kernel_path": path,
        "wall_s": round(wall, 3),
        "M": M, "K": K, "N": N, "group_size": g, "quant_type": qtype, "epilogue": epi or "none",
    }
    n_out = N // 2 if epi == "swiglu" else N
    tf = flops(M, K, N) / (us_per_step * 1e-6) / 1e12
    res["TFLOP/s"] = round(tf, 2)
    res["pct_fp16_mfma_peak"] = round(100 * tf / FP16_MFMA_PEAK_TFLOPS, 2)
    res["output_shape"] = [M, n_out]
    del graph, gwarm
    del weights
    torch.cuda.empty_cache()
    return res


def read_ceiling(name, steps, warmup, device):
    """The one-launch read ceiling of the headline's bytes: mq_read_probe over
    as many rotated copies of the config's algorithmic bytes as the headline
    rotates, timed exactly like the headline (graph replay, HIP events)."""
    import ctypes

    import torch

    from metal_native import _lib

    qtype, M, K, N, g, epi, bound = CONFIGS[name]
    per_copy = algo_bytes(qtype, M, K, N, g, epi)
    copies = max(2, min(256, -(-ROTATE_TARGET // per_copy)))
    bufs = [torch.randint(0, 256, (per_copy,), dtype=torch.uint8, device=device) for _ in range(copies)]
    sink = torch.zeros(int(_lib.lib.mq_read_probe_sink_size()) // 4 + 1, dtype=torch.int32, device=device)
    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))

    def fn(i):
        rc = _lib.lib.mq_read_probe(ctypes.c_void_p(bufs[i % copies].data_ptr()), per_copy,
                                    ctypes.c_void_p(sink.data_ptr()), ctypes.c_void_p(stream.cuda_stream))
        if rc != 0:
            raise RuntimeError(_lib.lib.mq_last_error().decode())

    with torch.cuda.stream(stream):
        for i in range(copies):
            fn(i)
    torch.cuda.synchronize(device)
    gwarm = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gwarm, stream=stream):
        for i in range(max(1, warmup)):
            fn(i)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(steps):
            fn(i)
    cur = torch.cuda.current_stream(device)
    gwarm.replay()
    torch.cuda.synchronize(device)
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(cur)
    graph.replay()
    t1.record(cur)
    torch.cuda.synchronize(device)
    us = t0.elapsed_time(t1) * 1000.0 / steps
    gbs = per_copy / (us * 1e-6) / 1e9
    del graph, gwarm, bufs
    torch.cuda.empty_cache()
    return {"us_per_launch": round(us, 3), "GB/s": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
            "bytes_per_launch": per_copy, "copies_rotated": copies,
            "what": "mq_read_probe: one read of the headline's algorithmic bytes per launch, no compute"}


def decode_bench(device):
    """28-layer Qwen2.5-7B-shaped decoder, int4 g128
    everywhere (lm_head included), batch 1, 512-token random KV cache, greedy
    decode of 64 tokens, one HIP graph replay per token."""
    import torch

    from metal_native.decoder import SyntheticDecoder, decode_tokens_per_second, qwen25_7b

    cfg = qwen25_7b()
    model = SyntheticDecoder(cfg, device, seed=0, prefilled=512)
    r = decode_tokens_per_second(model, n_tokens=64)
    per_layer = sum(ql.wp.numel() + 2 * ql.scales.numel() * 2
                    for L in model.layers for ql in (L["qkv"], L["o"], L["gate_up"], L["down"])) / cfg.layers
    head = model.lm_head.wp.numel() + 4 * model.lm_head.scales.numel()
    weight_bytes = per_layer * cfg.layers + head
    r["weight_bytes_per_token"] = int(weight_bytes)
    r["weight_stream_GB/s"] = round(weight_bytes / (r["ms_per_token"] * 1e-3) / 1e9, 1)
    r["floor_ms_per_token_at_8TBps"] = round(weight_bytes / 8e12 * 1e3, 3)
    r["ms_per_token"] = round(r["ms_per_token"], 4)
    r["tokens_per_s"] = round(r["tokens_per_s"], 1)
    del model
    torch.cuda.empty_cache()
    return r


def prep_bench(device, reps: int = 50):
    """Weight-preparation kernels at the config-2 shape (K=18944, N=3584,
    g=128), timed in a HIP graph: ``quantize`` (fp16 W -> int4 + scales +
    zeros; reads 2 B and writes 0.5 B per weight plus 4 B per group) and the
    flat ``dequantize`` behind QuantWeightCache.get_dequantized (reads 0.5 B +
    2 B per group, writes 2 B per weight)."""
    import torch

    import metal_native as mn

    N, K, g = 3584, 18944, 128
    G = K // g
    gen = torch.Generator(device=device)
    gen.manual_seed(0)
    copies = 3   # 3 x 136 MB of fp16 weights exceed the 256 MB MALL
    ws = [(torch.randn((N, K), device=device, generator=gen) * 0.05).half() for _ in range(copies)]
    out = {}

    def timed(fn):
        stream = torch.cuda.Stream(device)
        stream.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(stream):
            for i in range(copies):
                fn(i)
        torch.cuda.synchronize(device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(reps):
                fn(i % copies)
        graph.replay()
        torch.cuda.synchronize(device)
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        cur = torch.cuda.current_stream(device)
        t0.record(cur)
        graph.replay()
        t1.record(cur)
        torch.cuda.synchronize(device)
        return t0.elapsed_time(t1) * 1e3 / reps

    us = timed(lambda i: mn.quantize(ws[i], g, "int4"))
    nbytes = N * K * 2 + N * K // 2 + 4 * N * G
    out["quantize_int4_cfg2"] = {"us_per_call": round(us, 2), "algo_bytes": nbytes,
                                 "GB/s": round(nbytes / us / 1e3, 1), "pct_hbm_peak": round(nbytes / us / 1e3 / 80, 1)}
    qs = [mn.quantize(w, g, "int4") for w in ws]
    flat = [(bp.reshape(1, -1), s.reshape(-1)) for bp, s, _ in qs]
    del ws
    us = timed(lambda i: mn.dequantize(flat[i][0], flat[i][1], None, g, "int4", K=N * K, flat_groups=True))
    nbytes = N * K // 2 + 2 * N * G + 2 * N * K
    out["dequantize_flat_int4_cfg2"] = {"us_per_call": round(us, 2), "algo_bytes": nbytes,
                                        "GB/s": round(nbytes / us / 1e3, 1),
                                        "pct_hbm_peak": round(nbytes / us / 1e3 / 80, 1)}
    torch.cuda.empty_cache()
    return out


# --------------------------------------------------------------------------
# CPU baseline: the oracle on this host
# --------------------------------------------------------------------------

def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(warmup: int = 5, reps: int = 20):
    """The reference's path restated on this host (it has no CPU dequant):
    torch-CPU dequantize with the exact two-rounding fp16 formula, then
    ``torch.matmul(x.float(), W.float().T).half()``, timed with warm-up 5 and
    median of 20 (README.md:86-90 method), at the full headline problem.
    Threads: os.cpu_count() capped by OMP_NUM_THREADS (the GPU box grants one
    GPU's share of its cores).  The oracle checks the dequantized weights."""
    import numpy as np
    import torch

    from oracle import mq_oracle as O

    ncpu = os.cpu_count() or 1
    threads = min(ncpu, int(os.environ.get("OMP_NUM_THREADS", ncpu) or ncpu))
    torch.set_num_threads(threads)
    qtype, M, K, N, g, epi, _ = CONFIGS[HEADLINE]
    x, wp, s, z = O.make_int4_problem(M, K, N, g, seed=0)
    xt = torch.from_numpy(x)
    wpt = torch.from_numpy(wp)
    st = torch.from_numpy(s)
    zt = torch.from_numpy(z)

    def dequant():
        q = torch.stack([(wpt & 15), (wpt >> 4)], dim=-1).reshape(N, K).to(torch.int16)
        sx = st.repeat_interleave(g, dim=1)[:, :K]
        zx = zt.repeat_interleave(g, dim=1)[:, :K]
        return (q - 8).half() * sx - zx   # two fp16 roundings, as the reference kernel

    w = dequant()
    if not np.array_equal(w.numpy().view(np.uint16), O.dequant_int4(wp, s, z, K, g).view(np.uint16)):
        raise AssertionError("cpu baseline: torch-CPU dequant differs from the oracle")
    td, tm = [], []
    for r in range(warmup + reps):
        t0 = time.perf_counter()
        w = dequant()
        t1 = time.perf_counter()
        y = torch.matmul(xt.float(), w.float().t()).half()
        t2 = time.perf_counter()
        if r >= warmup:
            td.append(t1 - t0)
            tm.append(t2 - t1)
    dq, mm = float(np.median(td)), float(np.median(tm))
    total = dq + mm
    by = algo_bytes(qtype, M, K, N, g, epi)
    fl = flops(M, K, N)
    del y
    return {
        "value": round(by / total / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{HEADLINE} full problem (M={M},K={K},N={N},g={g}) on the host ({_cpu_model()}, "
                   f"os.cpu_count()={ncpu}, torch threads={threads}): torch-CPU exact fp16 dequantize, then "
                   f"fp32 torch.matmul and fp16 round; median of {reps} after {warmup} warm-up; dequant "
                   f"{dq*1e3:.1f} ms + matmul {mm*1e3:.1f} ms"),
        "ms_per_step": round(total * 1e3, 2),
        "dequant_ms": round(dq * 1e3, 2),
        "matmul_ms": round(mm * 1e3, 2),
        "GFLOP/s": round(fl / total / 1e9, 2),
        "cpu_model": _cpu_model(),
        "os_cpu_count": ncpu,
    }


def copy_calibration(device, nbytes: int = 2**30, reps: int = 20):
    """A plain copy of known size (nbytes read + nbytes written per launch):
    the FETCH_SIZE / WRITE_SIZE counters of this kernel give the scale factor
    from counter units to bytes."""
    import torch

    src = torch.empty(nbytes, dtype=torch.uint8, device=device).fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize(device)
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(reps):
        dst.copy_(src)
    t1.record()
    torch.cuda.synchronize(device)
    us = t0.elapsed_time(t1) * 1000.0 / reps
    print(json.dumps({"copy_bytes_read": nbytes, "copy_bytes_written": nbytes, "us_per_copy": round(us, 2),
                      "GB/s_read+write": round(2 * nbytes / (us * 1e-6) / 1e9, 1)}), flush=True)


# --------------------------------------------------------------------------

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-reps", type=int, default=20)
    ap.add_argument("--only", default=None, help="comma-separated config names (headline always runs)")
    ap.add_argument("--only-headline", action="store_true", help="measure the headline config only")
    ap.add_argument("--decode-only", action="store_true",
                    help="run only the config-5 decode step and print its JSON (for profiling)")
    ap.add_argument("--copy-calib", action="store_true",
                    help="only run a plain 1 GiB device-to-device copy (rocprof counter calibration)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the kernels would shard by weight rows, one shard per GPU). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    import metal_native  # noqa: F401  (fails loudly if the library is not built)

    device = torch.device("cuda:0")
    if args.copy_calib:
        copy_calibration(device)
        return
    if args.decode_only:
        print(json.dumps(decode_bench(device)))
        return
    names = list(CONFIGS)
    if args.only_headline:
        names = [HEADLINE]
    elif args.only:
        want = set(args.only.split(",")) | {HEADLINE}
        names = [n for n in names if n in want]
    results = {}
    for n in names:
        log(f"[bench] {n} ...")
        steps = args.steps if n == HEADLINE else max(200, args.steps // 4)
        results[n] = measure(n, steps, args.warmup, device)
        log(f"[bench] {n}: {json.dumps(results[n])}")
    head = results[HEADLINE]
    try:
        ceil = read_ceiling(HEADLINE, max(200, args.steps // 4), args.warmup, device)
        results["read_ceiling_cfg2"] = ceil
        log(f"[bench] read ceiling: {json.dumps(ceil)}")
    except Exception as e:  # noqa: BLE001  (the headline line must still print)
        ceil = None
        results["read_ceiling_cfg2"] = {"error": repr(e)}

    if not args.only_headline and not args.only:
        try:
            log("[bench] cfg5 synthetic Qwen2.5-7B decode step ...")
            results["cfg5_qwen7b_decode_64tok"] = decode_bench(device)
            log(f"[bench] cfg5: {json.dumps(results['cfg5_qwen7b_decode_64tok'])}")
        except Exception as e:  # noqa: BLE001  (the headline line must still print)
            results["cfg5_qwen7b_decode_64tok"] = {"error": repr(e)}
        try:
            log("[bench] weight preparation (quantize, flat dequantize) ...")
            results.update(prep_bench(device))
        except Exception as e:  # noqa: BLE001
            results["prep"] = {"error": repr(e)}

    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baseline ...")
        cpu = cpu_baseline(5, args.cpu_reps)
        log(f"[bench] cpu: {json.dumps(cpu)}")

    achieved = head["GB/s"]
    line = {
        "metric": METRIC,
        "value": achieved,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": head["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(head["us_per_step"] / 1000.0, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded torch RNG on device; int4 nibbles U{0..15}, scales U(0.005,0.02), "
                "zero-points U{0..15}, x ~ N(0,1))",
        "config": {
            "workload": "BASELINE config 2: Qwen2.5-7B down-proj int4 g128 dequant-GEMV, M=1, K=18944, N=3584",
            "kernel": head["kernel_path"] + " (" + KERNEL_DESC.get(head["kernel_path"], "?") + ")",
            "weights_rotated": head["copies_rotated"],
            "working_set_MB": head["working_set_MB"],
        },
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_bytes(),
        },
        "cpu_baseline": cpu,
        "extra": results,
    }
    if ceil:
        line["headline_frac_of_read_ceiling"] = round(head["GB/s"] / ceil["GB/s"], 4)
    prefill = results.get("cfg3_llama3b_qkv_m512")
    if prefill:
        line["prefill_TFLOP/s"] = prefill["TFLOP/s"]
        line["prefill_frac_fp16_mfma_peak"] = round(prefill["TFLOP/s"] / FP16_MFMA_PEAK_TFLOPS, 4)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
