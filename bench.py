"""Benchmark of the MI355X FP8 paged-attention hot path (one GPU).

Headline: FP8 paged decode at Qwen3-0.6B attention shapes (16 query / 8 kv
heads, head_dim 128, block 256, B = 256 sequences, context U[100, 2048]),
reported as achieved HBM GB/s over the algorithmic bytes (each FP8 K/V byte
once + bf16 Q/O + block-table row + context length).  Secondary fields:
varlen chunked prefill at Qwen3-8B shapes (16 x 512-token chunks over
cached context U[0, 4096]) in TFLOP/s of unmasked causal pairs, and the
long-context split-KV decode at Qwen3-32B shapes.

Inputs are resident in HBM before timing; two KV pools with different
contents are alternated so the working set stays far above the 256 MB
last-level cache.  Each timed region is bracketed by synchronisation and
measured with HIP events on the stream the kernels are launched on.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only decode|prefill|long|all]
                    [--no-cpu-baseline]
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "my-nano-vllm_amd"))

import torch  # noqa: E402

from nanovllm_amd import workloads as W  # noqa: E402
from nanovllm_amd.kernels.fp8_attention import fp8_decode_attention, fp8_prefill_attention  # noqa: E402
from nanovllm_amd.layers.attention import store_kvcache  # noqa: E402

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
SCALE = 128 ** -0.5


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--only", default="all", choices=["decode", "prefill", "long", "all"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    return ap.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def timed(fn, steps, warmup):
    """Median-free average: HIP events around `steps` back-to-back calls."""
    for _ in range(warmup):
        fn(0)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        fn(i)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps  # ms


def gpu_pools(wl, n_pools):
    pools = []
    for i in range(n_pools):
        kc, vc = wl.empty_caches("cuda")
        wl.seed += 1000 * i
        wl.fill_cache(kc, vc, store_kvcache, gen_device="cuda")
        wl.seed -= 1000 * i
        pools.append((kc, vc))
    torch.cuda.synchronize()
    return pools


def bench_decode(wl, steps, warmup, n_pools=2):
    pools = gpu_pools(wl, n_pools)
    q = wl.make_q("cuda")
    bt = torch.from_numpy(wl.block_tables).cuda()
    ctx = torch.from_numpy(wl.context_lens()).cuda()

    def step(i):
        kc, vc = pools[i % n_pools]
        fp8_decode_attention(q, kc, vc, bt, ctx, SCALE)

    ms = timed(step, steps, warmup)
    nbytes = wl.decode_bytes()
    return dict(ms=ms, bytes=nbytes, gbs=nbytes / (ms * 1e-3) / 1e9), pools, q


def bench_prefill(wl, steps, warmup, n_pools=2):
    pools = gpu_pools(wl, n_pools)
    q = wl.make_q("cuda")
    bt = torch.from_numpy(wl.block_tables).cuda()
    cu_q, cu_k = (torch.from_numpy(x).cuda() for x in wl.cu_seqlens())
    max_q, max_k = int(wl.lq().max()), int(wl.lk().max())

    def step(i):
        kc, vc = pools[i % n_pools]
        fp8_prefill_attention(q, kc, vc, block_tables=bt, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k,
                              max_seqlen_q=max_q, max_seqlen_k=max_k, softmax_scale=SCALE)

    ms = timed(step, steps, warmup)
    flops = wl.attention_flops()
    return dict(ms=ms, flops=flops, tflops=flops / (ms * 1e-3) / 1e12), pools, q


def cpu_baseline_decode(wl, pool, q, n_seqs=64, repeats=3):
    """The oracle (torch-CPU dequant + fp32 attention) on a bounded sample of
    the same workload: the first `n_seqs` sequences, same cache bytes."""
    from oracle import attention as oa
    sub = W.sub_workload(wl, range(min(n_seqs, wl.num_seqs)))
    kc = pool[0].view(torch.uint8).cpu()
    vc = pool[1].view(torch.uint8).cpu()
    qc = q[:sub.num_seqs].cpu()
    bt = torch.from_numpy(sub.block_tables)
    ctx = torch.from_numpy(sub.context_lens())
    torch.set_num_threads(os.cpu_count() or 1)
    oa.decode_attention(qc, kc, vc, bt, ctx, SCALE)  # warm-up
    times = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        oa.decode_attention(qc, kc, vc, bt, ctx, SCALE)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    return dict(value=round(sub.decode_bytes() / t / 1e9, 4), unit="GB/s",
                cores=torch.get_num_threads(), kind="port",
                sample=f"first {sub.num_seqs} of {wl.num_seqs} sequences of {wl.name} "
                       f"({sub.decode_bytes() / 1e6:.1f} MB algorithmic), median of {repeats} "
                       f"runs of {t:.3f}s; cpu={_cpu_model()}")


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no "
              "multi-GPU path -- run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)
    torch.cuda.set_device(0)
    line = {}
    extra = {}

    if args.only in ("decode", "all"):
        wl = W.qwen3_0p6b_decode()
        log(f"decode workload {wl.name}: B={wl.num_seqs} bytes={wl.decode_bytes()}")
        res, pools, q = bench_decode(wl, args.steps, args.warmup)
        log(f"decode: {res['ms'] * 1e3:.1f} us/step, {res['gbs']:.1f} GB/s")
        line.update(metric="decode attn HBM GB/s (%peak) + prefill attn TFLOP/s, Qwen3-8B shapes, FP8 KV",
                    value=round(res["gbs"], 2), unit="GB/s", ms_per_step=round(res["ms"], 5),
                    roofline=dict(bound="hbm", achieved=round(res["gbs"], 2), peak=HBM_PEAK_GBS,
                                  unit="GB/s", frac=round(res["gbs"] / HBM_PEAK_GBS, 4),
                                  traffic=None, kernel="paged_mq_attn_kernel<1> + mq_reduce_kernel",
                                  algorithmic_bytes_per_step=res["bytes"]),
                    config=dict(workload=wl.name, batch=wl.num_seqs, num_heads=wl.num_heads,
                                num_kv_heads=wl.num_kv_heads, head_dim=128, block_size=wl.block_size,
                                context="uniform[100,2048]", kv_dtype="float8_e4m3fn", kv_pools=2))
        if not args.no_cpu_baseline:
            log("cpu baseline (oracle) on a sample of the decode workload")
            line["cpu_baseline"] = cpu_baseline_decode(wl, pools[0], q)
        del pools
        torch.cuda.empty_cache()

    if args.only in ("prefill", "all"):
        wl = W.qwen3_8b_prefill()
        log(f"prefill workload {wl.name}: flops={wl.attention_flops()}")
        res, pools, _ = bench_prefill(wl, max(args.steps // 2, 5), max(args.warmup // 2, 2))
        log(f"prefill: {res['ms'] * 1e3:.1f} us/step, {res['tflops']:.1f} TFLOP/s")
        extra["prefill"] = dict(workload=wl.name, ms_per_step=round(res["ms"], 5),
                                tflops=round(res["tflops"], 2),
                                frac_bf16_peak=round(res["tflops"] / BF16_PEAK_TFLOPS, 4),
                                algorithmic_flops_per_step=res["flops"], kernel="varlen_prefill_kernel")
        del pools
        torch.cuda.empty_cache()

    if args.only in ("long", "all"):
        wl = W.qwen3_32b_long_decode()
        log(f"long decode workload {wl.name}: bytes={wl.decode_bytes()}")
        res, pools, _ = bench_decode(wl, max(args.steps // 5, 5), max(args.warmup // 5, 2), n_pools=1)
        log(f"long decode: {res['ms'] * 1e3:.1f} us/step, {res['gbs']:.1f} GB/s")
        extra["long_decode"] = dict(workload=wl.name, ms_per_step=round(res["ms"], 5),
                                    gbs=round(res["gbs"], 2), frac_hbm_peak=round(res["gbs"] / HBM_PEAK_GBS, 4),
                                    algorithmic_bytes_per_step=res["bytes"])
        del pools
        torch.cuda.empty_cache()

    if "value" not in line:   # partial runs (profiling) still print one line
        first = next(iter(extra.values()))
        line.update(metric="partial run", value=first.get("tflops", first.get("gbs")),
                    unit="TFLOP/s" if "tflops" in first else "GB/s", ms_per_step=first["ms_per_step"],
                    config=dict(workload=first["workload"]))
    line.update(n_gpus=1, steps=args.steps, warmup=args.warmup, higher_is_better=True, scaling="weak",
                vs_baseline=None, dtype="fp8_e4m3 kv -> bf16 mfma, fp32 accumulate, bf16 out",
                data="synthetic (seeded N(0,1) bf16 quantised to E4M3)")
    line.update(extra)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
