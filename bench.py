"""Benchmark of the verification hot path on one MI355X.

The headline line (the one JSON line printed) is the bf16 Llama-MLP-shaped linear layer checked with both block
checksums:  x 4096 tokens x 4096, W 14336 x 4096, y = x W^T in bf16 with fp32 accumulation.  A step is one
sdc_linear_check call (column-block check against the layer's precomputed block sums, row-block check of
y^T = W x^T, one pass over y for both).  Inputs are resident in HBM; the timed loop rotates over enough copies of
(x, y) that a step's reads of them miss the 256 MB Infinity Cache (W, 117 MB, is one tensor, as served).

  value         algorithmic bytes of one step / time per step, GB/s: x + y + W + the layer's block-sum parts
                (33.55 + 117.44 + 117.44 + 5.51 = 273.94 MB), what the two checks must read at least
  roofline      the kernel with the largest share of the step, against its bound: algorithmic bytes (or MFMA
                flops) per launch / its average launch time from HIP events recorded on its launch stream;
                traffic = HBM bytes per launch from the committed rocprofv3 counter summary of the same workload
  overhead      the check after its GEMM (warm: x and y still in the caches, as served) and alone (cold), against
                the guarded GEMM's time on the same GPU and stream
  cpu_baseline  the torch restatement of the check (both block checks, fp32 on every host core) on the same
                workload at full size, median of >= 5 runs

"more" holds one line per other workload, each with its own value, roofline and cpu_baseline:
  serve_bf16_4096x4096x14336  the serving check alone (column-block, ServeGuard.check) of the headline's layer
  fused_bf16_4096x4096x14336  the layer's GEMM with both checksums scored in its epilogue, against hipBLASLt's GEMM
  fp8_mlp_4096x4096x14336   fp8 e4m3 linear layer with per-token / per-channel scales, bf16 output, column check
  int8_2048x7168x4096       int8 W8A8 GEMM, exact int32 check
  fp8_2048x7168x4096        fp8 e4m3 GEMM with scales 10^U(-3,-1), bf16 output
  moe_4096x8of64_2048x1408  MoE grouped GEMM: 4096 tokens, top-8 of 64 experts (Zipf 1.1), bf16
  moe_recompute_4096x8of64_2048x1408  the sampled fused-MoE recompute (two rows, their experts' weights)
  fp8_quant_check_4096x4096  the FP8 input-quantization check of a serving layer (per-tensor and per-token scales)
  route_check_8192x256_grouped  the MoE router check of a DeepSeek-V3 router (microseconds per call)
  kv_fingerprint_28x4096    fingerprints of every block of a 28-layer x 4096-block paged KV cache (7.52 GB)
  attn_recompute_28x64      sampled attention recompute: one decode step of 64 sequences over 28 layers, 16
                            sampled (row, head) pairs a layer

    python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--only NAME] [--no-cpu]
    python bench.py --summarize DIR [DIR ...]     # rocprofv3 csv output -> the text summary kept in profiles/
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import platform
import re
import statistics
import sys
import time

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = {"bf16": 2500.0, "fp8": 5000.0, "int8": 5000.0}
HERE = os.path.dirname(os.path.abspath(__file__))
METRIC = "checksum-verify GB/s (% of HBM peak) + overhead % vs guarded GEMM, 1 GPU"


def _args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--settle", type=float, default=0.4,
                   help="seconds of further untimed calls after the warmup steps, so the clocks reach steady state")
    p.add_argument("--copies", type=int, default=4)
    p.add_argument("--only", default=None, help="run one workload and print its line alone")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="time budget of each CPU baseline")
    p.add_argument("--summarize", nargs="+", default=None, help="rocprofv3 output directories to summarize")
    return p.parse_args()


# ---------------------------------------------------------------------------------------------------------------
# rocprofv3 summaries (profiles/*.txt are written by --summarize and read back for the traffic figure)

def _csv_rows(d: str, suffix: str):
    rows = []
    for f in sorted(glob.glob(os.path.join(d, "**", f"*{suffix}"), recursive=True)):
        with open(f, newline="") as fh:
            rows.extend(csv.DictReader(fh))
    return rows


def summarize(dirs) -> str:
    """Kernel-trace statistics and per-dispatch HBM bytes of each kernel from rocprofv3 csv output.  Read bytes are
    32 TCC_EA0_RDREQ_32B + 64 TCC_EA0_RDREQ_64B + 128 TCC_EA0_RDREQ_128B (each request counted at its size), write
    bytes 32 (TCC_EA0_WRREQ - TCC_EA0_WRREQ_64B) + 64 TCC_EA0_WRREQ_64B; counters are summed over the L2 channels."""
    out = []
    keep = lambda name: "at::native" not in name and "at::cuda" not in name     # noqa: E731  (torch's own kernels)
    for d in dirs:
        stats = [r for r in _csv_rows(d, "kernel_stats.csv") if keep(r["Name"])]
        if stats:
            out.append(f"# kernel trace ({os.path.basename(os.path.normpath(d))})")
            out.append("stats\tname\tcalls\tavg_us\tmin_us\tmax_us\tpct")
            for r in sorted(stats, key=lambda r: -float(r["TotalDurationNs"])):
                out.append("stats\t{}\t{}\t{:.2f}\t{:.2f}\t{:.2f}\t{:.1f}".format(
                    r["Name"], r["Calls"], float(r["AverageNs"]) / 1e3, float(r["MinNs"]) / 1e3,
                    float(r["MaxNs"]) / 1e3, float(r["Percentage"])))
    per = {}
    for d in dirs:
        for r in _csv_rows(d, "counter_collection.csv"):
            key = r["Kernel_Name"]
            if not keep(key):
                continue
            per.setdefault(key, {}).setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    if per:
        out.append("# HBM bytes per dispatch (averages over the dispatches of each kernel)")
        out.append("traffic\tname\tdispatches\tread_bytes\twrite_bytes")
        for name, c in per.items():
            def avg(n):
                v = c.get(n)
                return sum(v) / len(v) if v else None
            r32, r64, r128 = avg("TCC_EA0_RDREQ_32B_sum"), avg("TCC_EA0_RDREQ_64B_sum"), avg("TCC_EA0_RDREQ_128B_sum")
            w, w64 = avg("TCC_EA0_WRREQ_sum"), avg("TCC_EA0_WRREQ_64B_sum")
            rd = None if r32 is None else 32 * r32 + 64 * (r64 or 0) + 128 * (r128 or 0)
            wr = None if w is None else 32 * (w - (w64 or 0)) + 64 * (w64 or 0)
            n = max(len(v) for v in c.values())
            out.append(f"traffic\t{name}\t{n}\t{'' if rd is None else int(rd)}\t{'' if wr is None else int(wr)}")
    return "\n".join(out)


def _profile_table(workload: str):
    """{kernel name: (read bytes, write bytes)} from profiles/<workload>.txt, or {} without one."""
    path = os.path.join(HERE, "profiles", f"{workload}.txt")
    t = {}
    try:
        with open(path) as f:
            for line in f:
                p = line.rstrip("\n").split("\t")
                if len(p) == 5 and p[0] == "traffic" and p[2] != "dispatches":
                    t[p[1]] = (float(p[3]) if p[3] else None, float(p[4]) if p[4] else None)
    except OSError:
        pass
    return t


def _traffic(workload: str, pattern: str):
    """HBM bytes (read + write) per launch of the kernels matching `pattern`, from the committed summary."""
    hits = [v for k, v in _profile_table(workload).items() if re.search(pattern, k)]
    if not hits or any(r is None or w is None for r, w in hits):
        return None
    return int(sum(r + w for r, w in hits) / len(hits))


# ---------------------------------------------------------------------------------------------------------------
# measurement helpers

class Ctx:
    def __init__(self, a):
        import torch
        from sdcguard_amd import _lib
        self.a, self.torch, self._lib = a, torch, _lib
        self.L = _lib.lib()
        self.dev = torch.device("cuda", 0)
        torch.cuda.set_device(self.dev)

    def settle(self, fn) -> int:
        """Untimed calls of fn(i), in batches of 20, until --settle seconds have passed (at most 20,000 calls).
        Measured on MI355X, a loop of calls right after a few warmup steps runs up to 15% slower than the same loop
        a few hundred calls later; the timed steps follow this."""
        t0, n = time.perf_counter(), 0
        while n < 20000 and time.perf_counter() - t0 < self.a.settle:
            for i in range(20):
                fn(n + i)
            n += 20
            self.torch.cuda.synchronize()
        return n

    def loop_ms(self, fn, steps: int) -> float:
        """Milliseconds per call of fn(i) over `steps` calls, HIP events on the current stream, synchronized on
        both sides."""
        torch = self.torch
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        for i in range(steps):
            fn(i)
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / steps

    def kernel_ms(self, fn, steps: int, names) -> dict:
        """Average launch duration (ms) of each named library kernel over `steps` calls of fn(i): the library
        brackets every launch with HIP events on the stream it launches on."""
        self.L.sdc_profile_reset()
        self.L.sdc_profile_enable(1)
        for i in range(steps):
            fn(i)
        self.torch.cuda.synchronize()
        self.L.sdc_profile_enable(0)
        out = {}
        for nm in names:
            tot, cnt = self._lib.profile_read(nm)
            out[nm] = (tot / cnt if cnt else 0.0, cnt)
        self.L.sdc_profile_reset()
        return out


def _roof(kernels: dict, amounts: dict, workload: str, patterns: dict, steps: int):
    """Per-kernel roofline entries and the dominant kernel's `roofline` object.  amounts: name -> (bound, amount
    per launch, dtype for an MFMA bound); kernels: name -> (avg ms, launches)."""
    ent = {}
    for nm, (bound, amount, dt) in amounts.items():
        ms, cnt = kernels[nm]
        if cnt == 0 or ms <= 0:
            raise RuntimeError(f"no timing recorded for kernel {nm}")
        if bound == "mfma":
            ach = amount / (ms * 1e-3) / 1e12
            peak, unit = MFMA_PEAK_TFLOPS[dt], "TFLOP/s"
        else:
            ach = amount / (ms * 1e-3) / 1e9
            peak, unit = HBM_PEAK_GBS, "GB/s"
        ent[nm] = {"avg_us": round(ms * 1e3, 2), "launches_per_step": round(cnt / steps, 3), "bound": bound,
                   "algorithmic": amount, "achieved": round(ach, 1), "peak": peak, "unit": unit,
                   "frac": round(ach / peak, 4), "traffic": _traffic(workload, patterns[nm]) if nm in patterns else None}
    dom = max(ent, key=lambda nm: kernels[nm][0] * kernels[nm][1])
    d = ent[dom]
    roof = {"kernel": dom, "bound": d["bound"], "achieved": d["achieved"], "peak": d["peak"], "unit": d["unit"],
            "frac": d["frac"], "traffic": d["traffic"], "algorithmic": d["algorithmic"], "avg_us": d["avg_us"],
            "profile": f"profiles/{workload}.txt"}
    return ent, roof


def _cpu_info() -> dict:
    import torch
    model = platform.processor() or "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "torch": torch.__version__}


def _cpu_median(fn, seconds: float, min_runs: int = 5, max_runs: int = 50):
    """Median seconds of fn() over at least `min_runs` runs, more while `seconds` last."""
    times = []
    t0 = time.perf_counter()
    while len(times) < min_runs or (time.perf_counter() - t0 < seconds and len(times) < max_runs):
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    return statistics.median(times), len(times)


def _cpu_threads() -> int:
    import torch
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    torch.set_num_threads(n)
    return n


# ---------------------------------------------------------------------------------------------------------------
# workloads

def bench_bf16_mlp(ctx: Ctx) -> dict:
    torch, a = ctx.torch, ctx.a
    from sdcguard_amd.linear import check_linear_both, resolve_both
    from sdcguard_amd.serve import LayerChecksums
    M, K, N = 4096, 4096, 14336
    name = "bf16_mlp_4096x4096x14336"
    g = torch.Generator(device=ctx.dev).manual_seed(0)
    W = (torch.randn(N, K, device=ctx.dev, generator=g) * 0.02).bfloat16()
    xs = [torch.randn(M, K, device=ctx.dev, generator=g).bfloat16() for _ in range(a.copies)]
    ys = [torch.nn.functional.linear(x, W) for x in xs]
    cs = LayerChecksums(W, None, 128)
    nb, mb = cs.nb, M // 128
    state = torch.zeros(4, dtype=torch.int64, device=ctx.dev)
    rows = torch.zeros(3, dtype=torch.int64, device=ctx.dev)

    def check(i):
        # the library's default: every kernel on the caller's stream (the per-kernel times are taken on this one)
        check_linear_both(xs[i % a.copies], W, None, ys[i % a.copies], cs, state=state, row_result=rows)

    def check_two_streams(i):
        # the variant with the column check's GEMM on a side stream, beside the x pass and the row GEMM
        check_linear_both(xs[i % a.copies], W, None, ys[i % a.copies], cs, state=state, row_result=rows,
                          concurrent=True)

    for i in range(a.warmup):
        check(i)
    torch.cuda.synchronize()
    if int(state[2].item()) != a.warmup:
        raise RuntimeError(f"the check did not run: {int(state[2].item())} calls counted of {a.warmup}")
    col, row = resolve_both(state, rows, M, N)
    settled = ctx.settle(check)
    ms = ctx.loop_ms(check, a.steps)
    for i in range(a.warmup):
        check_two_streams(i)                                  # (its side stream is made on the first call)
    two_ms = ctx.loop_ms(check_two_streams, a.steps)
    names = ("xstage", "xfinish", "col_gemm", "row_gemm", "ypass")
    km = ctx.kernel_ms(check, a.steps, names)

    def gemm(i):
        torch.mm(xs[i % a.copies], W.t(), out=ys[i % a.copies])

    for i in range(3):
        gemm(i)
    gemm_ms = ctx.loop_ms(gemm, a.steps)

    def both(i):
        gemm(i)
        check(i)
    both_ms = ctx.loop_ms(both, a.steps)
    buf = torch.empty_like(ys[0])
    copy_ms = ctx.loop_ms(lambda i: buf.copy_(ys[i % a.copies]), a.steps)
    del buf
    xb, yb, wb, pb = M * K * 2, M * N * 2, N * K * 2, K * 6 * nb * 2
    alg = xb + yb + wb + pb
    amounts = {"xstage": ("hbm", xb, None), "row_gemm": ("hbm", wb, None),
               "col_gemm": ("mfma", 2.0 * M * K * 6 * nb, "bf16"), "ypass": ("hbm", yb, None)}
    # (rs_gemm_kernel<dtype, ring, role> or rs_gemm_tall_kernel<dtype, role, ...>)
    patterns = {"xstage": r"xstage_kernel", "ypass": r"ypass_kernel",
                "row_gemm": r"rs_gemm_kernel<0, 4, 1>|rs_gemm_tall_kernel<0, 1,",
                "col_gemm": r"rs_gemm_kernel<0, 4, 0>|rs_gemm_tall_kernel<0, 0,"}
    ent, roof = _roof(km, amounts, name, patterns, a.steps)
    if km["xfinish"][1]:
        ent["xfinish"] = {"avg_us": round(km["xfinish"][0] * 1e3, 2), "launches_per_step": km["xfinish"][1] / a.steps,
                          "bound": "latency"}
    else:
        ent["xfinish"] = {"launches_per_step": 0, "note": "run by the row GEMM's spare workgroups"}
    value = alg / (ms * 1e-3) / 1e9
    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "settle_calls": settled, "ms_per_step": round(ms, 5),
        "ms_per_step_two_streams": round(two_ms, 5),
        "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "both block checksums (column-block against the layer's block sums, row-block of "
                               "y^T = W x^T) of a bf16 Llama-MLP linear layer, x 4096x4096 N(0,1), W 14336x4096 "
                               "N(0,0.02), y = x W^T bf16 (fp32 accumulation), block 128",
                   "name": name, "m": M, "k": K, "n": N, "block": 128, "copies_rotated": a.copies,
                   "algorithmic_bytes": alg},
        "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "roofline": roof, "kernels": ent,
        "device_copy_gbs": round(2 * yb / (copy_ms * 1e-3) / 1e9, 1),
        "guarded_gemm_ms": round(gemm_ms, 5),
        "overhead_pct_warm": round(100.0 * (both_ms - gemm_ms) / gemm_ms, 2),
        "overhead_pct_cold": round(100.0 * ms / gemm_ms, 2),
        "clean_max_z": {"column": round(col.max_z, 4), "row": round(row.max_z, 4)},
    }
    if not a.no_cpu:
        out["cpu_baseline"] = cpu_linear(xs[0], W, ys[0], alg, a.cpu_seconds)
    return out


def cpu_linear(x, W, y, alg: int, seconds: float) -> dict:
    """The torch restatement of both block checks (oracle.torch_check) on the full layer, every host core."""
    from oracle import torch_check
    cores = _cpu_threads()
    xc, Wc, yc = x.cpu(), W.cpu(), y.cpu()
    med, runs = _cpu_median(lambda: torch_check.linear_both(xc, Wc, None, yc), seconds)
    return {"value": round(alg / med / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
            "median_s": round(med, 4), "runs": runs, **_cpu_info(),
            "sample": "oracle.torch_check.linear_both (the reference's checksum._zscores in torch, fp32, on the CPU) "
                      "over the whole 4096x4096x14336 layer: column-block and row-block checks, block sums of W "
                      "made in the call as the reference's CPU path makes them; GB/s over the same 273.94 MB"}


def bench_serve_bf16(ctx: Ctx) -> dict:
    """The column-block check alone, as serving runs it (ServeGuard.check -> sdc_check_static: what register()
    queues after every checked linear layer), on the same layer as the headline."""
    torch, a = ctx.torch, ctx.a
    from sdcguard_amd.serve import ServeGuard, decode_counts, decode_state
    M, K, N = 4096, 4096, 14336
    name = "serve_bf16_4096x4096x14336"
    g = torch.Generator(device=ctx.dev).manual_seed(0)
    W = (torch.randn(N, K, device=ctx.dev, generator=g) * 0.02).bfloat16()
    xs = [torch.randn(M, K, device=ctx.dev, generator=g).bfloat16() for _ in range(a.copies)]
    ys = [torch.nn.functional.linear(x, W) for x in xs]
    guard = ServeGuard()
    layer = torch.nn.Module()
    slot = guard.add_layer(layer, "mlp.gate_up_proj", weight=W)
    nb = guard.layers[slot]["cs"].nb

    def check(i):
        guard.check(slot, xs[i % a.copies], ys[i % a.copies], with_bias=False)

    for i in range(a.warmup):
        check(i)
    torch.cuda.synchronize()
    st = guard.state(ctx.dev)[slot:slot + 1].cpu()
    z = decode_state(st)[0][0]
    checks = decode_counts(st)[0][0]
    if checks != a.warmup or not z < guard.z:
        raise RuntimeError(f"{name}: {checks} checks counted of {a.warmup}, clean max z {z}")
    ctx.settle(check)
    ms = ctx.loop_ms(check, a.steps)
    km = ctx.kernel_ms(check, a.steps, ("expected_gemm", "serve_fused"))
    xb, yb, pb = M * K * 2, M * N * 2, K * 6 * nb * 2
    alg = xb + yb + pb
    amounts = {"expected_gemm": ("mfma", 2.0 * M * K * 6 * nb, "bf16"), "serve_fused": ("hbm", yb, None)}
    patterns = {"expected_gemm": r"expected_gemm_kernel<0|rs_gemm_tall_kernel<0, 2,", "serve_fused": r"serve_fused_kernel"}
    ent, roof = _roof(km, amounts, name, patterns, a.steps)

    def gemm(i):
        torch.mm(xs[i % a.copies], W.t(), out=ys[i % a.copies])

    for i in range(3):
        gemm(i)
    gemm_ms = ctx.loop_ms(gemm, a.steps)
    both_ms = ctx.loop_ms(lambda i: (gemm(i), check(i)), a.steps)
    value = alg / (ms * 1e-3) / 1e9
    line = {"metric": METRIC, "value": round(value, 2), "unit": "GB/s", "ms_per_step": round(ms, 5), "dtype": "bf16",
            "hbm_frac": round(value / HBM_PEAK_GBS, 4),
            "config": {"workload": "the serving check alone (column-block checksums against the layer's block sums, "
                                   "ServeGuard.check as the vLLM plugin queues it) of the bf16 Llama-MLP linear "
                                   "layer, x 4096x4096 N(0,1), W 14336x4096 N(0,0.02), y = x W^T bf16, block 128",
                       "name": name, "m": M, "k": K, "n": N, "algorithmic_bytes": alg},
            "roofline": roof, "kernels": ent, "clean_max_z": round(z, 4),
            "guarded_gemm_ms": round(gemm_ms, 5),
            "overhead_pct_warm": round(100.0 * (both_ms - gemm_ms) / gemm_ms, 2),
            "overhead_pct_cold": round(100.0 * ms / gemm_ms, 2)}
    if not a.no_cpu:
        line["cpu_baseline"] = cpu_serve(xs[0], W, ys[0], alg, a.cpu_seconds)
    return line


def cpu_serve(x, W, y, alg: int, seconds: float) -> dict:
    """The torch restatement of the column-block check (oracle.torch_check.zscores) on the whole layer."""
    from oracle import torch_check
    cores = _cpu_threads()
    xc, Wt, yc = x.cpu(), W.cpu().t(), y.cpu()
    med, runs = _cpu_median(lambda: torch_check.zscores(xc, Wt, yc), seconds)
    return {"value": round(alg / med / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
            "median_s": round(med, 4), "runs": runs, **_cpu_info(),
            "sample": "oracle.torch_check.zscores (the reference's checksum._zscores in torch, fp32, on the CPU) over "
                      "the whole 4096x4096x14336 layer, block sums of W made in the call; GB/s over the same bytes"}


def bench_fused(ctx: Ctx) -> dict:
    """The GEMM with the check in its epilogue (fused_mm_checked: the product and both checksums' scores from one
    fp32 accumulator, nothing read back) against hipBLASLt's GEMM alone, on the headline's layer."""
    torch, a = ctx.torch, ctx.a
    from sdcguard_amd import checksum as csm
    from sdcguard_amd.fused import fused_mm_checked
    M, K, N = 4096, 4096, 14336
    name = "fused_bf16_4096x4096x14336"
    g = torch.Generator(device=ctx.dev).manual_seed(0)
    W = (torch.randn(N, K, device=ctx.dev, generator=g) * 0.02).bfloat16()
    Wt = W.t()
    xs = [torch.randn(M, K, device=ctx.dev, generator=g).bfloat16() for _ in range(a.copies)]
    ys = [torch.empty(M, N, dtype=torch.bfloat16, device=ctx.dev) for _ in range(a.copies)]
    res = torch.zeros(3, dtype=torch.int64, device=ctx.dev)

    def fused(i):
        fused_mm_checked(xs[i % a.copies], Wt, out=res)

    for i in range(a.warmup):
        fused(i)
    torch.cuda.synchronize()
    st = csm.resolve([csm.CheckStat(result=res, m=M, nb=N // 128, batched=False, z=6.0)], 6.0)[0]
    if not st.ok:
        raise RuntimeError(f"{name}: the clean product raised (max z {st.max_z})")
    ctx.settle(fused)
    ms = ctx.loop_ms(fused, a.steps)
    km = ctx.kernel_ms(fused, a.steps, ("fused_mm_checked", "fused_pack"))

    def gemm(i):
        torch.mm(xs[i % a.copies], Wt, out=ys[i % a.copies])

    for i in range(3):
        gemm(i)
    gemm_ms = ctx.loop_ms(gemm, a.steps)
    nb = N // 128
    flops = 2.0 * M * K * N + 2.0 * M * K * 12 * nb       # the product and the expected side (2 sums x 3 parts x 2)
    amounts = {"fused_mm_checked": ("mfma", flops, "bf16")}
    ent, roof = _roof({"fused_mm_checked": km["fused_mm_checked"]}, amounts, name,
                      {"fused_mm_checked": r"fused_(mm|gemm).*kernel"}, a.steps)
    alg = M * K * 2 + N * K * 2 + M * N * 2
    value = alg / (ms * 1e-3) / 1e9
    return {"metric": METRIC, "value": round(value, 2), "unit": "GB/s", "ms_per_step": round(ms, 5), "dtype": "bf16",
            "hbm_frac": round(value / HBM_PEAK_GBS, 4),
            "config": {"workload": "the product y = x W^T of the bf16 Llama-MLP linear layer (x 4096x4096, W "
                                   "14336x4096) from the library's MFMA GEMM with both checksums scored in its "
                                   "epilogue (fused_mm_checked), against the same product from hipBLASLt (torch.mm)",
                       "name": name, "m": M, "k": K, "n": N, "algorithmic_bytes": alg},
            "roofline": roof, "kernels": ent, "clean_max_z": round(st.max_z, 4),
            "fused_pack_us": round(km["fused_pack"][0] * 1e3, 2) if km["fused_pack"][1] else 0.0,
            "guarded_gemm_ms": round(gemm_ms, 5),
            "overhead_pct_vs_hipblaslt": round(100.0 * (ms - gemm_ms) / gemm_ms, 2),
            "cpu_baseline": {"value": None, "unit": "GB/s", "cores": 0, "kind": "port",
                             "sample": "none: the fused line is the GEMM itself; the CPU check of this layer is the "
                                       "headline's and the serving line's baseline"}}


def _fp8_problem(ctx, seed, m, k, n, copies):
    torch = ctx.torch
    g = torch.Generator(device=ctx.dev).manual_seed(seed)
    Bq = (torch.randn(k, n, device=ctx.dev, generator=g) * 4).clamp(-448, 448).to(torch.float8_e4m3fn)
    sb = (10.0 ** (torch.rand(n, device=ctx.dev, generator=g) * 2 - 3)).float()
    As, sas, Cs = [], [], []
    for _ in range(copies):
        Aq = (torch.randn(m, k, device=ctx.dev, generator=g) * 4).clamp(-448, 448).to(torch.float8_e4m3fn)
        sa = (10.0 ** (torch.rand(m, device=ctx.dev, generator=g) * 2 - 3)).float()
        C = ((Aq.float() @ Bq.float()) * sa[:, None] * sb[None, :]).bfloat16()
        As.append(Aq)
        sas.append(sa)
        Cs.append(C)
    return Bq, sb, As, sas, Cs


def bench_quant(ctx: Ctx, kind: str, m: int, k: int, n: int, name: str, seed: int) -> dict:
    torch, a = ctx.torch, ctx.a
    from sdcguard_amd import modes
    copies = a.copies
    if kind == "int8":
        g = torch.Generator(device=ctx.dev).manual_seed(seed)
        B = torch.randint(-127, 128, (k, n), device=ctx.dev, generator=g, dtype=torch.int32).to(torch.int8)
        As = [torch.randint(-127, 128, (m, k), device=ctx.dev, generator=g, dtype=torch.int32).to(torch.int8)
              for _ in range(copies)]
        Cs = [(A.double() @ B.double()).to(torch.int32) for A in As]
        sas, sb = [None] * copies, None
        consts = modes.QuantChecksums.make(B)
    else:
        B, sb, As, sas, Cs = _fp8_problem(ctx, seed, m, k, n, copies)
        consts = modes.QuantChecksums.make(B, sb)
    nb = -(-n // 128)
    res = torch.zeros(4, dtype=torch.int64, device=ctx.dev)

    def check(i):
        modes.quant_zscores(As[i % copies], consts, Cs[i % copies], sa=sas[i % copies], out=res)

    for i in range(a.warmup):
        check(i)
    torch.cuda.synchronize()
    st = modes.resolve(modes.QuantStat(res, m, nb, consts.kind, 6.0))
    if st["wrong_blocks"] != 0:
        raise RuntimeError(f"{name}: the clean workload raised {st['wrong_blocks']} blocks")
    ctx.settle(check)
    ms = ctx.loop_ms(check, a.steps)
    gname, sname = ("quant_gemm_i8", "quant_score_i8") if kind == "int8" else ("quant_gemm_fp8", "quant_score_fp8")
    km = ctx.kernel_ms(check, a.steps, (gname, sname))
    ab = m * k
    cb = Cs[0].numel() * Cs[0].element_size()
    pb = consts.parts.numel() * consts.parts.element_size()
    sc = 0 if kind == "int8" else 4 * m
    alg = ab + cb + pb + sc
    amounts = {gname: ("mfma", 2.0 * m * k * consts.parts.shape[0] * consts.parts.shape[1], kind),
               sname: ("hbm", cb, None)}
    # (the tall-tile GEMM: rs_gemm_tall_kernel<0, 5, ..> for int8, <0, 3, ..> for fp8)
    patterns = {gname: r"rs_gemm_tall_kernel<0, 5," if kind == "int8" else r"rs_gemm_tall_kernel<0, 3,",
                sname: r"quant_(tile|score)_kernel<" + ("0" if kind == "int8" else "1")}
    ent, roof = _roof(km, amounts, name, patterns, a.steps)
    value = alg / (ms * 1e-3) / 1e9
    gemm_ms = None
    try:
        if kind == "int8":
            def gemm(i):
                torch._int_mm(As[i % copies], B)
        else:
            Bt = B.t().contiguous().t()

            def gemm(i):
                torch._scaled_mm(As[i % copies], Bt, scale_a=sas[i % copies].view(-1, 1),
                                 scale_b=sb.view(1, -1), out_dtype=torch.bfloat16)
        for i in range(3):
            gemm(i)
        gemm_ms = ctx.loop_ms(gemm, a.steps)
        both_ms = ctx.loop_ms(lambda i: (gemm(i), check(i)), a.steps)
    except (RuntimeError, TypeError) as e:                          # no library GEMM for this layout here
        gemm_err = str(e).splitlines()[0][:160]
    out = {"metric": METRIC, "value": round(value, 2), "unit": "GB/s", "ms_per_step": round(ms, 5),
           "dtype": kind, "hbm_frac": round(value / HBM_PEAK_GBS, 4),
           "config": {"workload": f"{kind} GEMM {m}x{k}x{n} column-block check" +
                      (" (exact int32)" if kind == "int8" else ", per-token / per-channel scales 10^U(-3,-1), "
                                                                 "bf16 output"),
                      "name": name, "m": m, "k": k, "n": n, "algorithmic_bytes": alg},
           "roofline": roof, "kernels": ent,
           "guarded_gemm_ms": None if gemm_ms is None else round(gemm_ms, 5),
           "overhead_pct_warm": None if gemm_ms is None else round(100.0 * (both_ms - gemm_ms) / gemm_ms, 2),
           "overhead_pct_cold": None if gemm_ms is None else round(100.0 * ms / gemm_ms, 2)}
    if gemm_ms is None:
        out["guarded_gemm_note"] = gemm_err
    if not a.no_cpu:
        out["cpu_baseline"] = cpu_quant(kind, As[0], B, sas[0], sb, Cs[0], alg, a.cpu_seconds)
    return out


def cpu_quant(kind, A, B, sa, sb, C, alg: int, seconds: float) -> dict:
    """The oracle's quantized check (numpy, float64 / int64 BLAS on every host core) on a sample of rows."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import quant
    cores = _cpu_threads()
    m = A.shape[0]
    rows = min(m, 512)
    W = quant.patterns(1)
    if kind == "int8":
        Ac, Bc, Cc = A[:rows].cpu().numpy(), B.cpu().numpy(), C[:rows].cpu().numpy()
        fn = lambda: quant.int8_judge(Ac, Bc, Cc, W)                         # noqa: E731
    else:
        vals = quant.fp8_e4m3_values()
        Ac = vals[A[:rows].view(__import__("torch").uint8).cpu().numpy()]
        Bc = vals[B.view(__import__("torch").uint8).cpu().numpy()]
        sac, sbc = sa[:rows].double().cpu().numpy(), sb.double().cpu().numpy()
        Cc = C[:rows].double().cpu().numpy()
        fn = lambda: quant.fp8_judge(Ac, Bc, sac, sbc, Cc, W, c_bf16=True)  # noqa: E731
    with threadpool_limits(limits=cores):
        med, runs = _cpu_median(fn, seconds)
    k, n = B.shape
    sample_bytes = rows * k * A.element_size() + rows * n * C.element_size() + (alg - m * k * A.element_size() -
                                                                               m * n * C.element_size())
    del np
    return {"value": round(sample_bytes / med / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
            "median_s": round(med, 4), "runs": runs, **_cpu_info(),
            "sample": f"oracle.quant.{kind}_judge (numpy) on the first {rows} of {m} rows (block sums of B made in "
                      f"the call); GB/s over the sample's algorithmic bytes"}


def bench_moe(ctx: Ctx) -> dict:
    torch, a = ctx.torch, ctx.a
    from sdcguard_amd.checksum import GroupedChecksums, grouped_zscores, resolve_grouped
    name = "moe_4096x8of64_2048x1408"
    T0, E, TOPK, K, N = 4096, 64, 8, 2048, 1408
    gen = torch.Generator().manual_seed(7)
    p = torch.tensor([1.0 / (r + 1) ** 1.1 for r in range(E)], dtype=torch.float64)
    picks = torch.multinomial(p.expand(T0, E), TOPK, replacement=False, generator=gen)
    sizes = torch.bincount(picks.reshape(-1), minlength=E)
    T = int(sizes.sum())
    g = torch.Generator(device=ctx.dev).manual_seed(8)
    A = torch.randn(T, K, device=ctx.dev, generator=g).bfloat16()
    Bw = (torch.randn(E, K, N, device=ctx.dev, generator=g) * 0.02).bfloat16()
    offs = torch.cumsum(sizes, 0).to(torch.int32).to(ctx.dev)
    out = torch.empty(T, N, dtype=torch.bfloat16, device=ctx.dev)
    s = 0
    for e, c in enumerate(sizes.tolist()):
        if c:
            out[s:s + c] = (A[s:s + c].float() @ Bw[e].float()).bfloat16()
        s += c

    # the serving form: the experts' constants made once (as at load), each step the GEMM and the pass over out
    cs = GroupedChecksums(Bw)

    def check(i):
        grouped_zscores(A, None, out, offs, checksums=cs)

    def check_per_call(i):
        grouped_zscores(A, Bw, out, offs)

    for i in range(a.warmup):
        check(i)
    res = resolve_grouped(grouped_zscores(A, None, out, offs, checksums=cs))
    if not all(r.ok for r in res) or not all(r.ok for r in resolve_grouped(grouped_zscores(A, Bw, out, offs))):
        raise RuntimeError(f"{name}: the clean workload raised")
    ctx.settle(check)
    ms = ctx.loop_ms(check, a.steps)
    per_call_ms = ctx.loop_ms(check_per_call, a.steps)
    names = ("train_gemm", "train_score")
    km = ctx.kernel_ms(check, a.steps, names)
    nb = -(-N // 128)
    ab, cb, b2 = T * K * 2, T * N * 2, E * K * 2 * nb * 4
    alg = ab + cb + b2
    amounts = {"train_gemm": ("mfma", 2.0 * T * K * 6 * nb, "bf16"), "train_score": ("hbm", cb, None)}
    patterns = {"train_gemm": r"rs_gemm_tall_kernel<0, 4,", "train_score": r"grouped_score_kernel"}
    ent, roof = _roof(km, amounts, name, patterns, a.steps)
    value = alg / (ms * 1e-3) / 1e9
    gemm_ms = None
    try:
        def gemm(i):
            torch._grouped_mm(A, Bw, offs=offs, out_dtype=torch.bfloat16)
        for i in range(3):
            gemm(i)
        gemm_ms = ctx.loop_ms(gemm, a.steps)
        both_ms = ctx.loop_ms(lambda i: (gemm(i), check(i)), a.steps)
    except (RuntimeError, TypeError, AttributeError) as e:
        gemm_err = str(e).splitlines()[0][:160]
    line = {"metric": METRIC, "value": round(value, 2), "unit": "GB/s", "ms_per_step": round(ms, 5), "dtype": "bf16",
            "hbm_frac": round(value / HBM_PEAK_GBS, 4),
            "config": {"workload": "MoE grouped-GEMM column-block check, 4096 tokens x top-8 of 64 experts (Zipf "
                                   "1.1 loads), expert weights 2048x1408 bf16, the experts' block sums made once "
                                   "(GroupedChecksums, as when served)",
                       "name": name, "rows": T, "k": K, "n": N, "experts": E, "algorithmic_bytes": alg},
            "roofline": roof, "kernels": ent,
            "ms_per_step_sums_made_in_the_call": round(per_call_ms, 5),
            "guarded_gemm_ms": None if gemm_ms is None else round(gemm_ms, 5),
            "overhead_pct_warm": None if gemm_ms is None else round(100.0 * (both_ms - gemm_ms) / gemm_ms, 2),
            "overhead_pct_cold": None if gemm_ms is None else round(100.0 * ms / gemm_ms, 2)}
    if gemm_ms is None:
        line["guarded_gemm_note"] = gemm_err
    if not a.no_cpu:
        line["cpu_baseline"] = cpu_moe(A, Bw, out, sizes.tolist(), alg, a.cpu_seconds)
    return line


def cpu_moe(A, Bw, out, sizes, alg, seconds) -> dict:
    """The torch restatement of the column-block check, expert by expert, every host core."""
    from oracle import torch_check
    cores = _cpu_threads()
    Ac, Bc, Oc = A.cpu(), Bw.cpu(), out.cpu()

    def run():
        s = 0
        for e, c in enumerate(sizes):
            if c:
                torch_check.zscores(Ac[s:s + c], Bc[e], Oc[s:s + c])
            s += c
    med, runs = _cpu_median(run, seconds)
    return {"value": round(alg / med / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
            "median_s": round(med, 4), "runs": runs, **_cpu_info(),
            "sample": "oracle.torch_check.zscores per expert over the whole grouped product (64 experts)"}


def bench_fp8_quant(ctx: Ctx) -> dict:
    """The FP8 input-quantization check of a serving layer (sdc_fp8_quant_check) on the headline layer's input:
    per-tensor dynamic scales (the scale against max |x| over the step's 4096 real rows: one read of x, the
    line's value), and per-token scales (two sampled rows: a latency figure)."""
    torch, a = ctx.torch, ctx.a
    from sdcguard_amd import serve_fp8 as sf
    M, K = 4096, 4096
    name = "fp8_quant_check_4096x4096"
    g = torch.Generator(device=ctx.dev).manual_seed(31)
    xs = [torch.randn(M, K, device=ctx.dev, generator=g).bfloat16() for _ in range(a.copies)]
    qt, st_, qk, sk = [], [], [], []
    for x in xs:
        s_t = (x.float().abs().amax() / 448.0).reshape(1)
        qt.append((x.float() * (1.0 / s_t)).clamp(-448, 448).to(torch.float8_e4m3fn))
        st_.append(s_t)
        s_k = (x.float().abs().amax(1) / 448.0).clamp(min=1.0 / (448 * 512))
        qk.append((x.float() / s_k[:, None]).clamp(-448, 448).to(torch.float8_e4m3fn))
        sk.append(s_k.reshape(-1, 1))
    rows = torch.tensor([M], dtype=torch.int64, device=ctx.dev)
    step = torch.zeros(1, dtype=torch.int64, device=ctx.dev)
    state = torch.zeros(2, sf.COLS, dtype=torch.int64, device=ctx.dev)

    def tensor_check(i):
        sf.quant_check(xs[i % a.copies], qt[i % a.copies], st_[i % a.copies], sf.RECIPES["dynamic_tensor"], None,
                       None, rows, step, state, 0)

    def token_check(i):
        sf.quant_check(xs[i % a.copies], qk[i % a.copies], sk[i % a.copies], sf.RECIPES["dynamic_token"], None,
                       None, rows, step, state, 1)

    for i in range(a.warmup):
        tensor_check(i)
        token_check(i)
    torch.cuda.synchronize()
    k = state.cpu().tolist()
    if k[0][sf.C_CALLS] != a.warmup or k[1][sf.C_CALLS] != a.warmup or any(
            r[c] for r in k for c in (sf.C_SCALE, sf.C_OUTSIDE, sf.C_VALUES, sf.C_STATIC)):
        raise RuntimeError(f"{name}: the clean quantization raised or was not judged: {k}")
    ctx.settle(tensor_check)
    ms = ctx.loop_ms(tensor_check, a.steps)
    km = ctx.kernel_ms(tensor_check, a.steps, ("fp8q_amax", "fp8q_judge"))
    ms_tok = ctx.loop_ms(token_check, a.steps)
    km_tok = ctx.kernel_ms(token_check, a.steps, ("fp8q_judge",))
    xb = M * K * 2
    alg = xb + 2 * K * 3 + 4
    ent, roof = _roof(km, {"fp8q_amax": ("hbm", xb, None)}, name, {"fp8q_amax": r"amax"}, a.steps)
    ent["fp8q_judge"] = {"avg_us": round(km["fp8q_judge"][0] * 1e3, 2), "bound": "latency"}
    value = alg / (ms * 1e-3) / 1e9
    return {"metric": METRIC, "value": round(value, 2), "unit": "GB/s", "ms_per_step": round(ms, 5), "dtype": "bf16",
            "hbm_frac": round(value / HBM_PEAK_GBS, 4),
            "config": {"workload": "the FP8 input-quantization check of one serving layer: x 4096x4096 bf16 N(0,1) "
                                   "quantized to e4m3 with a per-tensor dynamic scale (max |x| over the 4096 real "
                                   "rows / 448, against the scale the GEMM got; two sampled rows' codes); also the "
                                   "per-token recipe (two sampled rows' scales and codes)",
                       "name": name, "m": M, "k": K, "algorithmic_bytes": alg},
            "roofline": roof, "kernels": ent,
            "per_token_us_per_call": round(ms_tok * 1e3, 2),
            "per_token_judge_us": round(km_tok["fp8q_judge"][0] * 1e3, 2),
            "cpu_baseline": cpu_fp8_quant(xs[0], qt[0], st_[0], alg, a.cpu_seconds) if not a.no_cpu else None}


def cpu_fp8_quant(x, xq, s, alg, seconds) -> dict:
    """The oracle's quantization check (numpy) of the per-tensor call."""
    import numpy as np
    import torch

    from oracle import serve_fp8 as of8
    cores = _cpu_threads()
    xf = x.float().cpu().numpy()
    q = xq.view(torch.uint8).cpu().numpy()
    sc = s.float().cpu().numpy()
    fn = lambda: of8.quant_check(xf, q, sc, 1, None, None, x.shape[0], 0)    # noqa: E731
    med, runs = _cpu_median(fn, seconds)
    del np
    return {"value": round(alg / med / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "median_s": round(med, 4), "runs": runs, **_cpu_info(),
            "sample": "oracle.serve_fp8.quant_check (numpy, one thread: the amax is one pass) of the whole "
                      "per-tensor call, 4096 rows"}


def _moe_outputs(torch, x, w13, w2, ids, gw):
    """The fused MoE kernel's output with its roundings: per expert, x W13^T in fp32 rounded, SiLU(gate) rounded,
    times up rounded, (.) W2^T in fp32 times the routing weight rounded, the experts' terms added in fp32."""
    T, H = x.shape
    I = w2.shape[2]
    acc = torch.zeros(T, H, dtype=torch.float32, device=x.device)
    for e in range(w13.shape[0]):
        r, slot = (ids == e).nonzero(as_tuple=True)
        if r.numel() == 0:
            continue
        h = (x[r].float() @ w13[e].float().t()).bfloat16()
        act = torch.nn.functional.silu(h[:, :I].float()).bfloat16()
        p = (act.float() * h[:, I:].float()).bfloat16()
        o = ((p.float() @ w2[e].float().t()) * gw[r, slot].float()[:, None]).bfloat16()
        acc.index_add_(0, r, o.float())
    return acc.bfloat16()


def bench_moe_recompute(ctx: Ctx) -> dict:
    """The sampled recompute of a fused MoE layer (sdc_moe_check) at the grouped workload's shape: 4096 tokens, top-8
    of 64 experts, H 2048, I 1408; every call is the active one (one layer), two rows recomputed."""
    torch, a = ctx.torch, ctx.a
    from sdcguard_amd import serve_moe as sm
    name = "moe_recompute_4096x8of64_2048x1408"
    T, E, TOPK, H, I = 4096, 64, 8, 2048, 1408
    g = torch.Generator(device=ctx.dev).manual_seed(41)
    x = torch.randn(T, H, device=ctx.dev, generator=g).bfloat16()
    w13 = (torch.randn(E, 2 * I, H, device=ctx.dev, generator=g) * 0.02).bfloat16()
    w2 = (torch.randn(E, H, I, device=ctx.dev, generator=g) * 0.02).bfloat16()
    gw, ids = torch.topk(torch.softmax(torch.randn(T, E, device=ctx.dev, generator=g), -1), TOPK, -1)
    gw = (gw / gw.sum(-1, keepdim=True)).float()
    ids = ids.to(torch.int32)
    out = _moe_outputs(torch, x, w13, w2, ids, gw)
    state = torch.zeros(1, sm.COLS, dtype=torch.int64, device=ctx.dev)
    cap = (torch.zeros(1, sm.CAP_COLS, dtype=torch.int32, device=ctx.dev), torch.zeros(1, H, device=ctx.dev),
           torch.zeros(1, H, device=ctx.dev), torch.zeros(1, 64, dtype=torch.int64, device=ctx.dev),
           torch.zeros(1, 64, device=ctx.dev))
    words = torch.tensor([(T << 32) | (1000 + i) for i in range(64)], dtype=torch.int64, device=ctx.dev)

    def check(i):
        sm.moe_check(x, out, gw, ids, w13, w2, None, 0, False, state, 0, words[i % 64:i % 64 + 1], 1, 0, *cap,
                     sm.MOE_Z)

    for i in range(a.warmup):
        check(i)
    torch.cuda.synchronize()
    k = state[0].cpu().tolist()
    z = struct_f32(k[sm.C_ROW] >> 32)
    if k[sm.C_CALLS] != a.warmup or not z < sm.MOE_Z:
        raise RuntimeError(f"{name}: clean calls counted {k[sm.C_CALLS]} of {a.warmup}, max z {z}")
    ctx.settle(check)
    ms = ctx.loop_ms(check, a.steps)
    names = ("moe_up", "moe_act", "moe_down", "moe_compare")
    km = ctx.kernel_ms(check, a.steps, names)
    # bytes: the distinct experts of the two sampled rows (their W13 and W2), the rows' x and outputs
    idc = ids.cpu()
    per_expert = (2 * I * H + H * I) * 2
    tot = 0
    for i in range(a.steps):
        rows = sm.sample_rows(torch.tensor(1000 + i % 64), T, "cpu").tolist()
        tot += len({int(e) for r in rows for e in idc[r].tolist()}) * per_expert + 2 * 2 * H * 2
    alg = tot / a.steps
    up_bytes = alg * (2 * I * H) / (3 * I * H)
    amounts = {"moe_up": ("hbm", up_bytes, None), "moe_down": ("hbm", alg - up_bytes, None)}
    ent, roof = _roof(km, amounts, name, {"moe_up": r"moe_up", "moe_down": r"moe_down"}, a.steps)
    for nm in ("moe_act", "moe_compare"):
        ent[nm] = {"avg_us": round(km[nm][0] * 1e3, 2), "bound": "latency"}
    value = alg / (ms * 1e-3) / 1e9
    return {"metric": "sampled MoE recompute GB/s of the sampled rows' expert weights, 1 GPU",
            "value": round(value, 2), "unit": "GB/s", "ms_per_step": round(ms, 5), "us_per_call": round(ms * 1e3, 2),
            "dtype": "bf16", "hbm_frac": round(value / HBM_PEAK_GBS, 4),
            "config": {"workload": "one active call of the sampled fused-MoE recompute: 4096 tokens, top-8 of 64 "
                                   "experts (softmax routing), H 2048, I 1408 (gate-up 2816x2048, down 2048x1408 "
                                   "bf16), SiLU; two rows recomputed with the fused kernel's roundings",
                       "name": name, "tokens": T, "experts": E, "top_k": TOPK, "hidden": H, "inter": I,
                       "algorithmic_bytes_per_call": int(alg)},
            "roofline": roof, "kernels": ent, "clean_max_z": round(z, 4),
            "cpu_baseline": cpu_moe_recompute(x, out, gw, ids, w13, w2, alg, a.cpu_seconds) if not a.no_cpu else None}


def struct_f32(bits: int) -> float:
    import struct
    return struct.unpack("<f", struct.pack("<I", int(bits) & 0xFFFFFFFF))[0]


def cpu_moe_recompute(x, out, gw, ids, w13, w2, alg, seconds) -> dict:
    """The oracle's recompute (numpy) of one call's two sampled rows, on the experts they use."""
    import numpy as np

    from oracle import serve_moe as om
    cores = _cpu_threads()
    rows = om.sample_rows(1000, x.shape[0], 1)
    used = sorted({int(e) for r in rows for e in ids[r].tolist()})
    remap = {e: i for i, e in enumerate(used)}
    xs = x[rows].float().cpu().numpy()
    ids_c = np.array([[remap[int(e)] for e in ids[r].tolist()] for r in rows], np.int32)
    g_c = gw[rows].cpu().numpy()
    w13_c = w13[used].float().cpu().numpy()
    w2_c = w2[used].float().cpu().numpy()
    fn = lambda: om.recompute(xs, ids_c, g_c, w13_c, w2_c, None, 0, False, "bf16")   # noqa: E731
    med, runs = _cpu_median(fn, seconds)
    nbytes = len(used) * (w13_c[0].size + w2_c[0].size) * 2 + 2 * 2 * x.shape[1] * 2
    return {"value": round(nbytes / med / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
            "median_s": round(med, 4), "runs": runs, **_cpu_info(),
            "sample": f"oracle.serve_moe.recompute (numpy BLAS) of one call's two sampled rows over their "
                      f"{len(used)} experts"}


def bench_route(ctx: Ctx) -> dict:
    """The MoE router check (sdc_route_check) of a DeepSeek-V3 router: 8192 tokens, sigmoid scores with a correction
    bias, top-8 of 256 experts within the best 4 of 8 groups, scaled by 2.5; every call is the active one."""
    torch, a = ctx.torch, ctx.a
    from sdcguard_amd import serve_route as sr
    name = "route_check_8192x256_grouped"
    T, E, TOPK, G, TG = 8192, 256, 8, 8, 4
    g = torch.Generator(device=ctx.dev).manual_seed(43)
    lg = (torch.randn(T, E, device=ctx.dev, generator=g) * 2).bfloat16()
    bias = torch.randn(E, device=ctx.dev, generator=g) * 0.03
    s = torch.sigmoid(lg.float())
    ch = (s + bias).view(T, G, E // G)
    keep = torch.zeros(T, G, dtype=torch.bool, device=ctx.dev)
    keep.scatter_(1, ch.topk(2, -1).values.sum(-1).topk(TG, -1).indices, True)
    ids = (s + bias).masked_fill(~keep.repeat_interleave(E // G, 1), float("-inf")).topk(TOPK, -1).indices
    w = s.gather(1, ids)
    w = (w / w.sum(-1, keepdim=True) * 2.5).float()
    ids = ids.to(torch.int32)
    st = torch.zeros(1, sr.COLS, dtype=torch.int64, device=ctx.dev)
    cap = (torch.zeros(1, sr.CAP_COLS, dtype=torch.int64, device=ctx.dev), torch.zeros(1, E, device=ctx.dev),
           torch.zeros(1, TOPK, dtype=torch.int64, device=ctx.dev), torch.zeros(1, TOPK, device=ctx.dev))
    real = torch.tensor([T], dtype=torch.int64, device=ctx.dev)
    steps_t = torch.arange(64, dtype=torch.int64, device=ctx.dev) + 1000

    def check(i):
        sr.route_check(lg, w, ids, TOPK, 1, True, bias, G, TG, 2.5, real, steps_t[i % 64:i % 64 + 1], st, 0, 1, 0,
                       *cap)

    for i in range(a.warmup):
        check(i)
    torch.cuda.synchronize()
    k = st[0].cpu().tolist()
    if k[sr.C_CALLS] != a.warmup or k[sr.C_SET] or k[sr.C_WEIGHT]:
        raise RuntimeError(f"{name}: the clean routing raised or was not judged: {k}")
    ctx.settle(check)
    ms = ctx.loop_ms(check, a.steps)
    km = ctx.kernel_ms(check, a.steps, ("route_check",))
    alg = 2 * (E * 2 + TOPK * 4 + TOPK * 4)
    ent, roof = _roof(km, {"route_check": ("hbm", alg, None)}, name, {"route_check": r"route_kernel"}, a.steps)
    return {"metric": "MoE router check microseconds per router call, 1 GPU", "value": round(ms * 1e3, 2),
            "unit": "us", "higher_is_better": False, "ms_per_step": round(ms, 5), "dtype": "f32",
            "config": {"workload": "one active call of the MoE router check: DeepSeek-V3 routing (8192 tokens, bf16 "
                                   "logits, sigmoid + correction bias, top-8 of 256 experts in the best 4 of 8 groups, "
                                   "renormalized, x2.5); two rows' policy recomputed and judged",
                       "name": name, "tokens": T, "experts": E, "top_k": TOPK, "algorithmic_bytes": alg},
            "roofline": roof, "kernels": ent,
            "note": "latency-bound: a call reads two rows (about 1.1 KB); the figure is the launch's duration"}


def _kv_cache(ctx, layers=28, nblk=4096):
    torch = ctx.torch
    g = torch.Generator(device=ctx.dev).manual_seed(55)
    kv = torch.empty(layers, nblk, 8, 16, 256, dtype=torch.bfloat16, device=ctx.dev)
    for lay in range(layers):
        kv[lay].normal_(generator=g)
    return kv


def bench_kv(ctx: Ctx, kv) -> dict:
    torch, a = ctx.torch, ctx.a
    from sdcguard_amd.kv import block_fingerprints
    name = "kv_fingerprint_28x4096"
    cache = kv.view(-1, 8, 16, 256)
    fp = torch.zeros(cache.shape[0], 3, dtype=torch.int64, device=ctx.dev)
    steps = max(5, a.steps // 5)

    def run(i):
        block_fingerprints(cache, out=fp)

    for i in range(2):
        run(i)
    ctx.settle(run)
    ms = ctx.loop_ms(run, steps)
    km = ctx.kernel_ms(run, steps, ("kv_fingerprint",))
    alg = cache.numel() * 2
    ent, roof = _roof(km, {"kv_fingerprint": ("hbm", alg, None)}, name, {"kv_fingerprint": r"kv_mfma_kernel"}, steps)
    value = alg / (ms * 1e-3) / 1e9
    line = {"metric": "KV block fingerprint GB/s (% of HBM peak), 1 GPU", "value": round(value, 2), "unit": "GB/s",
            "ms_per_step": round(ms, 5), "dtype": "u16", "hbm_frac": round(value / HBM_PEAK_GBS, 4),
            "config": {"workload": "fingerprints (sums of the 16-bit words, weighted twice, mod 2^64) of every "
                                   "block of a 28-layer x 4096-block paged KV cache, blocks [8 heads, 16 tokens, "
                                   "2 x 128] bf16", "name": name, "blocks": cache.shape[0],
                       "block_bytes": cache[0].numel() * 2, "algorithmic_bytes": alg},
            "roofline": roof, "kernels": ent}
    if not a.no_cpu:
        line["cpu_baseline"] = cpu_kv(cache, a.cpu_seconds)
    return line


def cpu_kv(cache, seconds) -> dict:
    """The oracle's C fingerprint (oracle/fingerprint.c, one thread per core) on a sample of blocks."""
    import numpy as np

    from oracle import fingerprint as F
    cores = _cpu_threads()
    nb = 2048
    sub = cache[:nb].view(__import__("torch").int16).cpu().numpy()
    if F.c_lib() is None:
        return {"value": None, "unit": "GB/s", "cores": 0, "kind": "port", "sample": "oracle C library not built"}
    med, runs = _cpu_median(lambda: F.kv_block_fp3_c(sub, threads=cores), seconds)
    del np
    return {"value": round(sub.nbytes / med / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
            "median_s": round(med, 4), "runs": runs, **_cpu_info(),
            "sample": f"oracle.fingerprint.kv_block_fp3_c (C, {cores} threads) on {nb} of the "
                      f"{cache.shape[0]} blocks ({sub.nbytes / 1e6:.0f} MB)"}


def bench_attn(ctx: Ctx, kv) -> dict:
    torch, a = ctx.torch, ctx.a
    from sdcguard_amd import serve_attn as SA
    name = "attn_recompute_28x64"
    L_, NBLK, HKV, NTOK, D, HQ, NSEQ = kv.shape[0], kv.shape[1], 8, 16, 128, 16, 64
    samples = 16
    gc = torch.Generator().manual_seed(56)
    lens = torch.randint(512, 2049, (NSEQ,), generator=gc)
    Wt = 2048 // NTOK
    bt = torch.zeros(NSEQ, Wt, dtype=torch.int32)
    for r in range(NSEQ):
        nbk = -(-int(lens[r]) // NTOK)
        bt[r, :nbk] = torch.randperm(NBLK, generator=gc)[:nbk].to(torch.int32)
    q = (torch.randn(L_, NSEQ, HQ, D, generator=gc) * 0.5).bfloat16().to(ctx.dev)
    qsl = torch.arange(NSEQ + 1, dtype=torch.int32, device=ctx.dev)
    pos = lens - 1
    blk_of = bt[torch.arange(NSEQ), (pos // NTOK).long()]
    slots = (blk_of.long() * NTOK + pos % NTOK).to(ctx.dev)
    lens_d, bt_d = lens.to(torch.int32).to(ctx.dev), bt.to(ctx.dev)
    live = torch.arange(Wt * NTOK, device=ctx.dev)[None, :] < lens_d[:, None]
    outs, keys, vals = [], [], []
    for layer in range(L_):
        kv_l = kv[layer]
        rows = kv_l[bt_d.long()].permute(0, 1, 3, 2, 4).reshape(NSEQ, Wt * NTOK, HKV, 2 * D).float()
        Kt, Vt = rows[..., :D].permute(0, 2, 1, 3).contiguous(), rows[..., D:].permute(0, 2, 1, 3).contiguous()
        qf = q[layer].float().view(NSEQ, HKV, HQ // HKV, D)
        s = torch.matmul(qf, Kt.transpose(-1, -2).contiguous()) * D ** -0.5           # [seq, hkv, g, keys]
        s = s.masked_fill(~live[:, None, None, :], float("-inf"))
        o = torch.matmul(torch.softmax(s, -1), Vt).reshape(NSEQ, HQ, D).bfloat16()
        outs.append(o)
        keys.append(kv_l[blk_of.long().to(ctx.dev), :, (pos % NTOK).long().to(ctx.dev), :D].contiguous())
        vals.append(kv_l[blk_of.long().to(ctx.dev), :, (pos % NTOK).long().to(ctx.dev), D:].contiguous())
        del rows, Kt, Vt, s
    bufs = SA.buffers(ctx.dev, L_, D, 64, torch.bfloat16, samples=samples)
    scale = D ** -0.5

    def step(i):
        bufs["ctrl"][0] = 1000 + i
        for layer in range(L_):
            SA.attn_check(q[layer], outs[layer], kv[layer], keys[layer], vals[layer], qsl, lens_d, bt_d, slots,
                          bufs["state"], layer, bufs["ctrl"], 1, 0, scale, -1, SA.ATTN_Z, bufs["capm"],
                          bufs["capq"], bufs["capo"], None, None, bufs["ws"], True, False, samples=samples)

    bufs["ctrl"][1] = 1
    steps = max(5, a.steps // 5)
    for i in range(2):
        step(i)
    torch.cuda.synchronize()
    rep = [SA.decode_state(bufs["state"][l_].cpu()) for l_ in range(L_)]
    worst = max(r["max_z"] for r in rep)
    if not worst < SA.ATTN_Z or any(r["writes_wrong"] or r["bad_blocks"] for r in rep):
        raise RuntimeError(f"{name}: the clean decode step raised (z {worst})")
    ctx.settle(step)
    ms = ctx.loop_ms(step, steps)
    km = ctx.kernel_ms(step, steps, ("attn_check",))
    # every layer call is live (one check per layer per step) and samples the same (row, head) pairs at a step.
    # bytes: the K and V rows of every distinct sampled (request, kv head), per layer, averaged over the timed steps
    ql, ll = qsl.cpu().tolist(), lens.tolist()
    tot = 0
    for i in range(steps):
        for layer in range(L_):
            seen = set()
            for j in range(samples):
                p_ = SA.sample_python(1000 + i, 0, 1, j, ql, ll, NSEQ, HQ)
                if p_:
                    seen.add((p_["request"], p_["head"] // (HQ // HKV)))
            tot += sum(ll[r] * D * 2 * 2 for r, _ in seen)
    alg_step = tot / steps
    ent, roof = _roof(km, {"attn_check": ("hbm", alg_step / L_, None)}, name,
                      {"attn_check": r"attn_check_kernel"}, steps)
    line = {"metric": "sampled attention recompute GB/s of sampled K/V rows, 1 GPU",
            "value": round(alg_step / (ms * 1e-3) / 1e9, 2), "unit": "GB/s", "ms_per_step": round(ms, 5),
            "us_per_layer_call": round(ms * 1e3 / L_, 2), "dtype": "bf16",
            "config": {"workload": "one decode step of 64 sequences (512-2048 tokens) over 28 layers of a paged "
                                   "bf16 KV cache (4096 blocks a layer, [8 heads, 16 tokens, 2 x 128]): each layer's "
                                   "check recomputes 16 sampled (row, head) attentions and checks the step's KV write",
                       "name": name, "layers": L_, "samples_per_layer": samples,
                       "algorithmic_bytes_per_step": int(alg_step)},
            "roofline": roof, "kernels": ent, "clean_max_z": round(worst, 4)}
    if not a.no_cpu:
        line["cpu_baseline"] = cpu_attn(kv, q, outs, keys, vals, qsl, lens, bt, slots, L_, samples, alg_step,
                                        a.cpu_seconds)
    return line


def cpu_attn(kv, q, outs, keys, vals, qsl, lens, bt, slots, L_, samples, alg_step, seconds) -> dict:
    """The oracle's attention check (numpy) of one layer call at a time, on the blocks its samples can read."""
    import numpy as np
    import torch

    from oracle import attn as OA
    cores = _cpu_threads()
    layer = 3
    kv_l = kv[layer]
    ids = sorted({int(v) for r in range(bt.shape[0]) for v in bt[r].tolist()})
    remap = torch.zeros(kv.shape[1], dtype=torch.int32)
    remap[torch.tensor(ids)] = torch.arange(len(ids), dtype=torch.int32)
    bt_c = remap[bt.long()].numpy()
    sl = slots.cpu()
    sl_c = (remap[(sl // 16)].long() * 16 + sl % 16).numpy()
    w = kv_l[torch.tensor(ids, device=kv.device)].view(torch.int16).cpu().numpy().view(np.uint16)
    kv_c = (w.astype(np.uint32) << 16).view(np.float32)
    f = lambda t: t.float().cpu().numpy()                                   # noqa: E731
    args = (f(q[layer]), f(outs[layer]), kv_c, f(keys[layer]), f(vals[layer]), qsl.cpu().numpy(), lens.numpy(),
            bt_c, sl_c)
    from concurrent.futures import ThreadPoolExecutor

    from threadpoolctl import threadpool_limits

    def one(_):
        OA.check(*args, step=1000, scale=128 ** -0.5, samples=samples)

    # one layer call per host thread at a time (numpy's kernels release the GIL; BLAS kept to one thread each)
    with threadpool_limits(limits=1), ThreadPoolExecutor(cores) as ex:
        med, runs = _cpu_median(lambda: list(ex.map(one, range(cores))), seconds)
    return {"value": round(cores * alg_step / L_ / med / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
            "median_s": round(med, 4), "runs": runs, **_cpu_info(),
            "sample": f"oracle.attn.check (numpy) of a layer's call (16 samples) over the blocks the step's sequences "
                      f"hold, {cores} calls at once on {cores} threads; GB/s over a layer's average sampled K/V bytes "
                      f"times the calls"}


WORKLOADS = ("bf16_mlp_4096x4096x14336", "serve_bf16_4096x4096x14336", "fused_bf16_4096x4096x14336",
             "fp8_mlp_4096x4096x14336", "int8_2048x7168x4096", "fp8_2048x7168x4096", "moe_4096x8of64_2048x1408",
             "moe_recompute_4096x8of64_2048x1408", "fp8_quant_check_4096x4096", "route_check_8192x256_grouped",
             "kv_fingerprint_28x4096", "attn_recompute_28x64")


def run(ctx: Ctx, name: str, kv_holder: dict) -> dict:
    if name == "bf16_mlp_4096x4096x14336":
        return bench_bf16_mlp(ctx)
    if name == "serve_bf16_4096x4096x14336":
        return bench_serve_bf16(ctx)
    if name == "fused_bf16_4096x4096x14336":
        return bench_fused(ctx)
    if name == "moe_recompute_4096x8of64_2048x1408":
        return bench_moe_recompute(ctx)
    if name == "fp8_quant_check_4096x4096":
        return bench_fp8_quant(ctx)
    if name == "route_check_8192x256_grouped":
        return bench_route(ctx)
    if name == "fp8_mlp_4096x4096x14336":
        return bench_quant(ctx, "fp8", 4096, 4096, 14336, name, seed=21)
    if name == "int8_2048x7168x4096":
        return bench_quant(ctx, "int8", 2048, 7168, 4096, name, seed=22)
    if name == "fp8_2048x7168x4096":
        return bench_quant(ctx, "fp8", 2048, 7168, 4096, name, seed=23)
    if name == "moe_4096x8of64_2048x1408":
        return bench_moe(ctx)
    if "kv" not in kv_holder:
        kv_holder["kv"] = _kv_cache(ctx)
    if name == "kv_fingerprint_28x4096":
        return bench_kv(ctx, kv_holder["kv"])
    if name == "attn_recompute_28x64":
        return bench_attn(ctx, kv_holder["kv"])
    raise SystemExit(f"unknown workload {name}; one of {', '.join(WORKLOADS)}")


def main():
    a = _args()
    if a.summarize:
        print(summarize(a.summarize))
        return
    if a.gpus != 1:
        print(f"bench.py measures one GPU (asked for {a.gpus}): the checks are independent per GPU shard, and "
              "their multi-GPU sharding is a design note, not a measured path", file=sys.stderr)
        sys.exit(2)
    ctx = Ctx(a)
    ctx.torch.backends.cuda.matmul.allow_bf16_reduced_precision_reduction = False
    kv_holder: dict = {}
    if a.only:
        line = run(ctx, a.only, kv_holder)
        line.setdefault("n_gpus", 1)
        print(json.dumps(line))
        return
    main_line = run(ctx, WORKLOADS[0], kv_holder)
    more = []
    for nm in WORKLOADS[1:]:
        print(f"# {nm}", file=sys.stderr, flush=True)
        more.append(run(ctx, nm, kv_holder))
        ctx.torch.cuda.empty_cache()
    main_line["more"] = more
    print(json.dumps(main_line))


if __name__ == "__main__":
    main()
