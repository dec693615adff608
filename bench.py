"""Benchmark of the MI355X FP8 paged-attention hot path (one GPU).

Headline (``value``): FP8 paged decode at Qwen3-8B attention shapes -- the
mixed batch's 192 plain-decode sequences on their own (32 query / 8 kv heads,
head_dim 128, block 256, one query token each, context U[256, 4096], seeded,
over the mixed batch's paged pool) -- as achieved HBM GB/s over the
algorithmic bytes of a step: each FP8 K/V byte once + bf16 Q in and O out +
the block-table row and context length of every sequence.  One decode call
is two launches: the balanced stream-K pass (``decode_sk_kernel<1,8,QL>``,
one persistent workgroup per CU streaming an equal share of the KV stages)
and the merge pass for sequences cut between workgroups
(``decode_sk_merge_heads_kernel``: one wave per sequence and kv head).  The
HIP-event time of a call covers both, so
``roofline.achieved`` is the algorithmic bytes over the two launches
together (a lower bound on the stream-K kernel's own rate).

Secondary fields in the same JSON line:
  decode_qwen3_0p6b  decode at Qwen3-0.6B shapes (16/8 heads, B = 256,
               context U[100, 2048]), GB/s;
  prefill      varlen chunked prefill at Qwen3-8B shapes (32/8 heads, 16 x
               512-token chunks over cached context U[0, 4096]) in TFLOP/s of
               unmasked causal pairs, vs the bf16 dense MFMA peak, with its
               own CPU baseline;
  long_decode  long-context decode at Qwen3-32B shapes (64/8 heads, B = 32,
               context U[32K, 128K], 1% of K/V x20);
  store        the KV store/quantise of the prefill workload's 8192 new
               tokens (strided K/V views of a fused qkv tensor), GB/s;
  qk_norm_rope_store  the fused q/k RMSNorm + RoPE + FP8 KV store of the
               same tokens (QKV projection output in, q and cache rows out), GB/s;
  mixed        the mixed batch's varlen call (32 speculative x 5 rows + 3 x
               512-token chunks, Qwen3-8B shapes), TFLOP/s, and its
               speculative rows alone, GB/s over their decode bytes;
  contiguous_prefill  the mixed batch's 1024-token contiguous-layout prompt
               (block_tables=None), TFLOP/s;
  contiguous_prefill_batch  the prefill workload in the contiguous layout
               (its K/V rows gathered per sequence), TFLOP/s;
  fp8_linear   the FP8 block-scaled linear layer at Qwen3-8B shapes: the qkv
               projection of the 16 x 512-token prefill step (M = 8192, N =
               6144, K = 4096) in TFLOP/s vs the dense FP8 MFMA peak, and the
               gate/up projection of the 192 decode rows (M = 192, N = 24576)
               in GB/s of weights vs HBM; the activation quantisation and the
               whole fp8_block_linear call beside each, and an oracle CPU
               baseline;
  metadata     one engine step's attention metadata (positions, slots,
               cu_seqlens, context lengths, block tables) for the mixed batch
               and for the 16 x 512 prefill step: host time per call and time
               to completion of the on-device build and of the vectorised host
               build, the on-device build's GPU time, and, as CPU baseline,
               the reference's own per-token loops and per-tensor copies;
  lm_head      the sampler over the mixed step's 355 LM-head rows (Qwen3
               vocabulary, bf16 logits) in GB/s of logits vs HBM, beside the
               reference's arithmetic as eager torch ops, and the LM-head row
               selection;
  host_overhead  host time per call of the Python entry points (checks,
               workspace lookup, ctypes, launches) and of the bare C-ABI
               decode call, with nothing synchronised in the loop.
These are timed after 0.15 s of sustained warm-up calls (the shader clock
settles lower under continuous MFMA load within the first tens of
milliseconds); the headline decode field runs exactly --warmup warm-up calls.

Inputs are resident in HBM before timing; two KV pools with different
contents are alternated so the working set stays far above the 256 MB
last-level cache.  The timed region is bracketed by synchronisation and
measured with HIP events recorded on the stream the kernels are launched on
(torch's current stream).

``roofline.traffic`` comes from the committed rocprofv3 counter summary
(profiles/decode_qwen3_8b_b192_pmc.json: FETCH_SIZE / WRITE_SIZE of the
decode kernels, each scaled by the same counter's reading for a plain copy
of known size, which ``--copy-probe`` runs); it is null if that file is
absent.

``cpu_baseline`` times the oracle (torch-CPU dequant + fp32 attention, the
parity tests' checker) on the host cores for a bounded sample of the same
workload; the prefill field carries one of its own.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
                    [--only FIELD[,FIELD...]]   (decode decode06 prefill long store mixed linear metadata lm_head host, or all)
                    [--no-cpu-baseline]
                    [--copy-probe]
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "my-nano-vllm_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))  # seeded workloads (shared with the parity tests)

import numpy as np  # noqa: E402
import torch  # noqa: E402

import workloads as W  # noqa: E402
from nanovllm_amd.kernels.fp8_attention import fp8_decode_attention, fp8_prefill_attention  # noqa: E402
from nanovllm_amd.layers.attention import store_kvcache  # noqa: E402

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
SCALE = 128 ** -0.5
METRIC = "decode attn HBM GB/s (%peak) + prefill attn TFLOP/s, Qwen3-8B shapes, FP8 KV"
PMC_SUMMARY = os.path.join(ROOT, "profiles", "decode_qwen3_8b_b192_pmc.json")
COPY_PROBE_BYTES = 1 << 30
# The secondary fields (prefill, store, mixed, long decode) are timed after this much
# sustained warm-up: under continuous MFMA load the shader clock drops over
# the first tens of milliseconds, and the steady state is what a serving
# loop sees.  The headline decode field keeps exactly --warmup warm-up calls.
SECONDARY_WARM_S = 0.15
FIELDS = ("decode", "decode06", "prefill", "long", "store", "mixed", "linear", "metadata", "lm_head", "host")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--only", default="all",
                    help="comma-separated fields: " + ",".join(FIELDS) + " or all")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run a plain 1 GiB device copy (counter scale for rocprofv3 --pmc)")
    return ap.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def timed(fn, steps, warmup, warm_s=0.0):
    """Average ms per call over `steps` back-to-back calls, HIP events on the
    current stream (the stream the kernels are launched on).  `warmup` calls
    run first; with warm_s > 0, warm-up calls continue until that many seconds
    of them have run (the shader clock settles under sustained load)."""
    for i in range(warmup):
        fn(i)
    if warm_s > 0:
        torch.cuda.synchronize()
        t_end = time.perf_counter() + warm_s
        i = warmup
        while time.perf_counter() < t_end:
            for _ in range(8):
                fn(i)
                i += 1
            torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(steps):
        fn(i)
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


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


def bench_decode(wl, steps, warmup, n_pools=2, warm_s=0.0):
    pools = gpu_pools(wl, n_pools)
    q = wl.make_q("cuda")
    bt = torch.from_numpy(wl.block_tables).cuda()
    ctx = torch.from_numpy(wl.context_lens()).cuda()

    def step(i):
        kc, vc = pools[i % n_pools]
        fp8_decode_attention(q, kc, vc, bt, ctx, SCALE)

    ms = timed(step, steps, warmup, warm_s)
    nbytes = wl.decode_bytes()
    return dict(ms=ms, bytes=nbytes, gbs=nbytes / (ms * 1e-3) / 1e9), pools, q


def bench_prefill(wl, steps, warmup, n_pools=2, warm_s=0.0):
    pools = gpu_pools(wl, n_pools)
    q = wl.make_q("cuda")
    bt = torch.from_numpy(wl.block_tables).cuda()
    cu_q, cu_k = (torch.from_numpy(x).cuda() for x in wl.cu_seqlens())
    max_q, max_k = int(wl.lq().max()), int(wl.lk().max())

    def step(i):
        kc, vc = pools[i % n_pools]
        fp8_prefill_attention(q, kc, vc, block_tables=bt, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k,
                              max_seqlen_q=max_q, max_seqlen_k=max_k, softmax_scale=SCALE)

    ms = timed(step, steps, warmup, warm_s)
    flops = wl.attention_flops()
    return dict(ms=ms, flops=flops, tflops=flops / (ms * 1e-3) / 1e12), pools, q


def bench_store(wl, steps, warmup, n_src=6):
    """KV store/quantise of the workload's new tokens (the prefill step's own
    K/V): key/value are strided views of a fused qkv tensor, as in the model
    (q, k, v = qkv.split(...)); n_src source tensors rotate so the reads come
    from HBM.  Algorithmic bytes: bf16 K/V read + FP8 K/V written + slot ids."""
    n = wl.num_q_tokens()
    hq, hkv = wl.num_heads, wl.num_kv_heads
    slots = torch.from_numpy(wl.new_token_slots()).cuda()
    kc, vc = wl.empty_caches("cuda")
    srcs = []
    g = torch.Generator(device="cuda").manual_seed(wl.seed)
    for _ in range(n_src):
        qkv = torch.randn(n, (hq + 2 * hkv) * 128, generator=g, device="cuda").to(torch.bfloat16)
        k = qkv[:, hq * 128:(hq + hkv) * 128].view(n, hkv, 128)
        v = qkv[:, (hq + hkv) * 128:].view(n, hkv, 128)
        srcs.append((k, v))

    def step(i):
        k, v = srcs[i % n_src]
        store_kvcache(k, v, kc, vc, slots)

    ms = timed(step, steps, warmup, SECONDARY_WARM_S)
    nbytes = n * hkv * 128 * (2 * 2 + 2) + 4 * n
    # Ceilings for the same traffic: torch's own bf16 -> float8_e4m3fn
    # conversion of as many contiguous elements (2 B read, 1 B written per
    # element), and a device-to-device copy moving the same total bytes
    # (nbytes / 2 read, nbytes / 2 written); n_src sources rotate as above.
    elems = 2 * n * hkv * 128
    conv_src = [torch.randn(elems, generator=g, device="cuda").to(torch.bfloat16) for _ in range(n_src)]
    conv_dst = torch.empty(elems, dtype=torch.float8_e4m3fn, device="cuda")
    ms_conv = timed(lambda i: conv_dst.copy_(conv_src[i % n_src]), steps, warmup, SECONDARY_WARM_S)
    half = nbytes // 2 // 16 * 16
    cp_src = [t.view(torch.uint8)[:half] for t in conv_src]
    cp_dst = torch.empty(half, dtype=torch.uint8, device="cuda")
    ms_copy = timed(lambda i: cp_dst.copy_(cp_src[i % n_src]), steps, warmup, SECONDARY_WARM_S)
    del conv_src, conv_dst, cp_src, cp_dst
    return dict(ms=ms, bytes=nbytes, gbs=nbytes / (ms * 1e-3) / 1e9, conversion_copy_ms=ms_conv,
                device_copy_ms=ms_copy, device_copy_bytes=2 * half)


def bench_qk_norm_rope(wl, steps, warmup, n_src=6):
    """Fused q/k RMSNorm + RoPE + FP8 KV store of the workload's new tokens:
    the projection output [N, (Hq + 2 Hkv) * 128] bf16 in, q bf16 and the
    FP8 K/V cache rows out; n_src projection outputs rotate so the reads
    come from HBM.  Algorithmic bytes: qkv read, positions, slot ids, one
    fp32 cos/sin row per token, q written, FP8 K and V written."""
    from nanovllm_amd.layers.qk_norm_rope import qk_norm_rope_store
    n = wl.num_q_tokens()
    hq, hkv = wl.num_heads, wl.num_kv_heads
    slots = torch.from_numpy(wl.new_token_slots()).cuda()
    positions = torch.from_numpy(np.concatenate([np.arange(s.cached, s.lk) for s in wl.seqs])).cuda()
    kc, vc = wl.empty_caches("cuda")
    g = torch.Generator(device="cuda").manual_seed(wl.seed)
    srcs = [torch.randn(n, (hq + 2 * hkv) * 128, generator=g, device="cuda").to(torch.bfloat16) for _ in range(n_src)]
    wq = (1.0 + 0.1 * torch.randn(128, generator=g, device="cuda")).to(torch.bfloat16)
    wk = (1.0 + 0.1 * torch.randn(128, generator=g, device="cuda")).to(torch.bfloat16)
    inv_freq = 1.0 / (1e6 ** (torch.arange(0, 128, 2, dtype=torch.float32, device="cuda") / 128))
    ang = torch.outer(torch.arange(40960, dtype=torch.float32, device="cuda"), inv_freq)
    cos_sin = torch.cat((ang.cos(), ang.sin()), dim=-1)

    def step(i):
        qk_norm_rope_store(positions, srcs[i % n_src], wq, wk, 1e-6, cos_sin, kc, vc, slots, hq, hkv)

    ms = timed(step, steps, warmup, SECONDARY_WARM_S)
    nbytes = n * ((hq + 2 * hkv) * 128 * 2 + 8 + 4 + 128 * 4 + hq * 128 * 2 + 2 * hkv * 128)
    return dict(ms=ms, bytes=nbytes, gbs=nbytes / (ms * 1e-3) / 1e9)


def bench_contiguous(n_tok, hq, hkv, steps, warmup):
    """One contiguous-layout prompt (block_tables=None): FP8 K/V [n, Hkv, 128]."""
    g = torch.Generator(device="cuda").manual_seed(17)
    q = torch.randn(n_tok, hq, 128, generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn(n_tok, hkv, 128, generator=g, device="cuda").to(torch.bfloat16).to(torch.float8_e4m3fn)
    v = torch.randn(n_tok, hkv, 128, generator=g, device="cuda").to(torch.bfloat16).to(torch.float8_e4m3fn)
    cu = torch.tensor([0, n_tok], dtype=torch.int32, device="cuda")

    def step(i):
        fp8_prefill_attention(q, k, v, block_tables=None, cu_seqlens_q=cu, cu_seqlens_k=cu,
                              max_seqlen_q=n_tok, max_seqlen_k=n_tok, softmax_scale=SCALE)

    ms = timed(step, steps, warmup, SECONDARY_WARM_S)
    flops = 4 * 128 * hq * (n_tok * (n_tok + 1) // 2)
    return dict(ms=ms, flops=flops, tflops=flops / (ms * 1e-3) / 1e12)


def bench_contiguous_batch(wl, pools, q, steps, warmup):
    """The workload's own sequences in the contiguous layout (block_tables=None):
    each pool's K/V rows of every sequence gathered into [sum Lk, Hkv, 128]
    tensors (one copy per pool, alternated), same queries, same flops."""
    rows = np.concatenate([wl.slots_for(i, 0, s.lk) for i, s in enumerate(wl.seqs)]).astype(np.int64)
    idx = torch.from_numpy(rows).cuda()
    hkv = wl.num_kv_heads
    conts = []
    for kc, vc in pools:
        conts.append(tuple(c.view(torch.uint8).reshape(-1, hkv, 128)[idx].view(torch.float8_e4m3fn)
                           for c in (kc, vc)))
    cu_q_np, _ = wl.cu_seqlens()
    cu_q = torch.from_numpy(cu_q_np).cuda()
    cu_k = torch.from_numpy(np.concatenate([[0], np.cumsum(wl.lk())]).astype(np.int32)).cuda()
    max_q, max_k = int(wl.lq().max()), int(wl.lk().max())

    def step(i):
        k, v = conts[i % len(conts)]
        fp8_prefill_attention(q, k, v, block_tables=None, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k,
                              max_seqlen_q=max_q, max_seqlen_k=max_k, softmax_scale=SCALE)

    ms = timed(step, steps, warmup, SECONDARY_WARM_S)
    flops = wl.attention_flops()
    return dict(ms=ms, flops=flops, tflops=flops / (ms * 1e-3) / 1e12)


FP8_PEAK_TFLOPS = 5000.0       # MI355X dense FP8 MFMA


def bench_fp8_linear(M, N, K, steps, warmup):
    """The FP8 block-scaled linear layer at one shape: the GEMM alone (on
    already-quantised activations, the reference's second kernel), the
    activation quantisation alone, and fp8_block_linear end to end.  Random
    finite E4M3FN weights; copies totalling more than 600 MiB are cycled, so
    the weights stream from HBM as in a model step (which reads every layer's
    weights once) and not from the 256 MB last-level cache."""
    from nanovllm_amd import _native
    from nanovllm_amd.kernels.fp8_linear import fp8_block_linear
    lib = _native.load()
    g = torch.Generator(device="cuda").manual_seed(M + N + K)
    x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    n_weights = max(2, -(-(600 << 20) // (N * K)))
    ws = []
    for _ in range(n_weights):
        c = torch.randint(0, 256, (N, K), device="cuda", generator=g, dtype=torch.int32).to(torch.uint8)
        ws.append(torch.where((c & 0x7F) == 0x7F, c ^ 1, c).view(torch.float8_e4m3fn))
    w_scale = (torch.rand(N // 128, K // 128, device="cuda", generator=g) * 1e-3).to(torch.bfloat16)
    xq = torch.empty(M, K, dtype=torch.uint8, device="cuda")
    xs = torch.empty(M, K // 128, dtype=torch.bfloat16, device="cuda")
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    _native.check(lib.nvamd_fp8_act_quant(x.data_ptr(), K, 0, xq.data_ptr(), xs.data_ptr(), M, K, stream), "quant")
    gws_n = lib.nvamd_fp8_block_gemm_workspace_bytes(M, N, K)
    gws = torch.empty(max(gws_n, 16), dtype=torch.uint8, device="cuda")

    def gemm(i):
        w = ws[i % n_weights]
        _native.check(lib.nvamd_fp8_block_gemm(xq.data_ptr(), xs.data_ptr(), w.data_ptr(), K, w_scale.data_ptr(),
                                               out.data_ptr(), N, 0, M, N, K, gws.data_ptr(), gws_n, stream),
                      "gemm")

    def quant(i):
        _native.check(lib.nvamd_fp8_act_quant(x.data_ptr(), K, 0, xq.data_ptr(), xs.data_ptr(), M, K, stream), "quant")

    ms_gemm = timed(gemm, steps, warmup, warm_s=SECONDARY_WARM_S)
    ms_quant = timed(quant, steps, warmup)
    ms_linear = timed(lambda i: fp8_block_linear(x, ws[i % n_weights], w_scale), steps, warmup)
    flops = 2.0 * M * N * K
    weight_bytes = N * K + (N // 128) * (K // 128) * 2
    res = dict(ms=ms_gemm, tflops=flops / (ms_gemm * 1e-3) / 1e12,
               weight_gbs=weight_bytes / (ms_gemm * 1e-3) / 1e9,
               quant_us=ms_quant * 1e3, quant_gbs=3.0 * M * K / (ms_quant * 1e-3) / 1e9,
               linear_us=ms_linear * 1e3, flops=flops, weight_bytes=weight_bytes)
    res["hipblaslt_per_tensor_us"] = scaled_mm_us(xq.view(torch.float8_e4m3fn), ws, steps, warmup)
    return res


def scaled_mm_us(xq, ws, steps, warmup):
    """The same product through torch._scaled_mm (hipBLASLt's FP8 GEMM) with
    ONE scale per tensor instead of 128 x 128 block scales: a comparison
    figure for the block-scaled kernel (less work: no per-block promotion).
    None where torch has no FP8 GEMM for this device."""
    one = torch.ones((), device="cuda", dtype=torch.float32)
    try:
        ms = timed(lambda i: torch._scaled_mm(xq, ws[i % len(ws)].t(), scale_a=one, scale_b=one,
                                              out_dtype=torch.bfloat16), steps, warmup, warm_s=SECONDARY_WARM_S)
    except (RuntimeError, TypeError) as e:
        log(f"torch._scaled_mm unavailable: {e}")
        return None
    return round(ms * 1e3, 2)


def bench_host_overhead(calls=300):
    """Host time per call of the drop-in Python entry points at the bench's
    Qwen3-8B head shapes: wall-clock time of `calls` back-to-back calls with
    nothing synchronised inside the loop (argument checks, workspace lookup,
    ctypes, kernel launches), beside the decode launch through the C ABI with
    its arguments prepared once (ctypes and launches only).  The inputs have
    the shapes of the bench's workloads but short contexts, so that the GPU
    keeps up and no launch waits for queue space: the host work does not
    depend on the KV bytes."""
    from nanovllm_amd import _native
    from nanovllm_amd.kernels.fp8_linear import fp8_block_linear
    lib = _native.load()
    g = torch.Generator(device="cuda").manual_seed(7)
    B, hq, hkv, bs, nb_pool, max_nb = 192, 32, 8, 256, 64, 16

    def fp8(shape):
        c = torch.randint(0, 120, shape, device="cuda", generator=g, dtype=torch.int32).to(torch.uint8)
        return c.view(torch.float8_e4m3fn)

    kc, vc = fp8((nb_pool, bs, hkv, 128)), fp8((nb_pool, bs, hkv, 128))
    q = torch.randn(B, hq, 128, device="cuda", generator=g).to(torch.bfloat16)
    bt = torch.randint(0, nb_pool, (B, max_nb), device="cuda", generator=g, dtype=torch.int32)
    ctx = torch.randint(1, 64, (B,), device="cuda", generator=g, dtype=torch.int32)

    def host_us(fn):
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(calls):
            fn()
        t1 = time.perf_counter()
        torch.cuda.synchronize()
        return round((t1 - t0) / calls * 1e6, 2)

    res = dict(unit="us per call (host)", calls=calls)
    res["fp8_decode_attention"] = host_us(lambda: fp8_decode_attention(q, kc, vc, bt, ctx, SCALE))
    ws_n = lib.nvamd_decode_workspace_bytes(B, hq, hkv, max_nb, bs, 0)
    ws = torch.empty(max(ws_n, 1), dtype=torch.uint8, device="cuda")
    out = torch.empty_like(q)
    args = (out.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(), bt.data_ptr(), ctx.data_ptr(), B, hq, hkv, 128,
            nb_pool, bs, max_nb, SCALE, 0, ws.data_ptr(), ws_n, 0, torch.cuda.current_stream().cuda_stream)
    dec = lib.nvamd_fp8_decode_attention
    res["c_abi_decode"] = host_us(lambda: dec(*args))
    # the mixed batch's varlen call: 32 speculative sequences of 5 rows + 3 chunks (64 rows here)
    lq = [5] * 32 + [64] * 3
    lk = [l + 40 for l in lq]
    cu_q = torch.tensor([0] + list(np.cumsum(lq)), dtype=torch.int32, device="cuda")
    cu_k = torch.tensor([0] + list(np.cumsum(lk)), dtype=torch.int32, device="cuda")
    qv = torch.randn(int(sum(lq)), hq, 128, device="cuda", generator=g).to(torch.bfloat16)
    btv = bt[:len(lq)].contiguous()
    res["fp8_prefill_attention"] = host_us(lambda: fp8_prefill_attention(
        qv, kc, vc, block_tables=btv, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, max_seqlen_q=max(lq),
        max_seqlen_k=max(lk), softmax_scale=SCALE))
    # the prefill step's 8192 new tokens, strided K/V views of a fused qkv tensor
    qkv = torch.randn(8192, (hq + 2 * hkv) * 128, device="cuda", generator=g).to(torch.bfloat16)
    key = qkv[:, hq * 128:(hq + hkv) * 128].view(8192, hkv, 128)
    value = qkv[:, (hq + hkv) * 128:].view(8192, hkv, 128)
    slots = torch.randperm(nb_pool * bs, device="cuda", generator=g)[:8192].to(torch.int32)
    res["store_kvcache"] = host_us(lambda: store_kvcache(key, value, kc, vc, slots))
    # the gate/up projection of 192 decode rows
    x = torch.randn(B, 4096, device="cuda", generator=g).to(torch.bfloat16)
    w = fp8((24576, 4096))
    w_scale = (torch.rand(24576 // 128, 4096 // 128, device="cuda", generator=g) * 1e-3).to(torch.bfloat16)
    res["fp8_block_linear"] = host_us(lambda: fp8_block_linear(x, w, w_scale))
    return res


def cpu_baseline_fp8_linear(N, K, rows=16, target_s=8.0):
    """The oracle's quantisation + block GEMM (numpy, float64 partials) on a
    bounded sample: `rows` tokens of the shape, repeated for ~target_s."""
    from oracle import fp8_linear as ol
    g = torch.Generator().manual_seed(1)
    x = torch.randn(rows, K, generator=g).to(torch.bfloat16)
    w = torch.randint(0, 120, (N, K), generator=g, dtype=torch.int32).to(torch.uint8).numpy()
    w_scale = (torch.rand(N // 128, K // 128, generator=g) * 1e-3).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < target_s or n == 0:
        ol.block_linear(x, w, w_scale)
        n += 1
    dt = (time.perf_counter() - t0) / n
    return dict(value=round(2.0 * rows * N * K / dt / 1e9, 3), unit="GFLOP/s", cores=_blas_threads(), kind="port",
                sample=f"oracle act_quant + block_gemm on {rows} tokens of the {N}x{K} weight, {n} runs")


def _blas_threads():
    """Threads of the BLAS numpy's matmul runs on (the oracle's GEMM)."""
    try:
        from threadpoolctl import threadpool_info
        n = [p["num_threads"] for p in threadpool_info() if p.get("user_api") == "blas"]
        if n:
            return max(n)
    except Exception:  # noqa: BLE001
        pass
    return os.cpu_count() or 1


def bench_sampler(rows, vocab, steps, warmup):
    """Temperature sampling of `rows` bf16 logit rows: the HIP sampler (in-kernel
    Philox noise) and the reference's arithmetic as eager torch ops on the same
    GPU (float copy, divide, softmax, exponential_, divide, argmax)."""
    from nanovllm_amd.layers.sampler import sample_tokens
    g = torch.Generator(device="cuda").manual_seed(rows)
    logits = [(torch.randn(rows, vocab, device="cuda", generator=g) * 3).to(torch.bfloat16) for _ in range(2)]
    temps = torch.rand(rows, device="cuda", generator=g) + 0.5

    def ours(i):
        sample_tokens(logits[i & 1], temps, seed=i)

    def torch_ref(i):
        y = logits[i & 1].float().div_(temps.unsqueeze(1))
        p = torch.softmax(y, dim=-1)
        p.div_(torch.empty_like(p).exponential_(1).clamp_min_(1e-10)).argmax(dim=-1)

    ms = timed(ours, steps, warmup)
    ms_ref = timed(torch_ref, max(steps // 2, 5), max(warmup // 2, 2))
    nbytes = rows * vocab * 2
    return dict(ms=ms, gbs=nbytes / (ms * 1e-3) / 1e9, ms_torch=ms_ref, bytes=nbytes)


def bench_select_rows(steps, warmup):
    """LM-head row selection of the mixed step: 192 decode + 32 x 5 speculative
    rows + 3 prefill chunks of 512 (their last rows), hidden 4096, bf16."""
    from nanovllm_amd.layers.embed_head import select_lm_head_rows
    from nanovllm_amd.utils.context import get_context, set_context, reset_context
    lq = [5] * 32 + [512] * 3
    cu = [0] + list(np.cumsum(lq))
    x = torch.randn(192 + cu[-1], 4096, device="cuda").to(torch.bfloat16)
    set_context(split_pt=192, num_spec_seqs=32, num_spec_rows=160,
                cu_seqlens_q=torch.tensor(cu, dtype=torch.int32, device="cuda"))
    try:
        ms = timed(lambda i: select_lm_head_rows(x, get_context()), steps, warmup)
    finally:
        reset_context()
    return dict(ms=ms, rows=192 + 160 + 3)


def cpu_baseline_sampler(vocab, rows=8, target_s=6.0):
    from oracle import lm_head as olh
    rng = np.random.default_rng(0)
    logits = rng.normal(size=(rows, vocab)).astype(np.float32)
    temps = np.ones(rows, np.float32)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < target_s or n == 0:
        olh.sample(logits, temps, olh.exponential_noise(n, 0, rows, vocab))
        n += 1
    dt = (time.perf_counter() - t0) / n
    return dict(value=round(rows * vocab * 2 / dt / 1e9, 3), unit="GB/s of bf16 logits", cores=1, kind="port",
                sample=f"oracle Philox noise + sample on {rows} rows x {vocab}, {n} runs")


class _StepSeq:
    """The fields of nano-vLLM's Sequence that the attention metadata reads."""
    __slots__ = ("num_tokens", "num_cached_tokens", "num_scheduled_tokens", "block_table", "block_size")

    def __init__(self, num_tokens, num_cached_tokens, num_scheduled_tokens, block_table, block_size):
        self.num_tokens, self.num_cached_tokens = num_tokens, num_cached_tokens
        self.num_scheduled_tokens, self.block_table, self.block_size = num_scheduled_tokens, block_table, block_size

    @property
    def num_blocks(self):  # nanovllm/engine/sequence.py:58-60
        return (self.num_tokens + self.block_size - 1) // self.block_size

    @property
    def last_block_num_tokens(self):  # nanovllm/engine/sequence.py:62-64
        return self.num_tokens - (self.num_blocks - 1) * self.block_size


def step_sequences(wl):
    """A workload as one engine step: sequence i has its cached keys plus lq
    scheduled tokens (plain decode: lq = 1, num_tokens = cached + 1;
    speculative: 1 + drafts scheduled on num_tokens = cached + 1; prefill
    chunk: num_tokens = cached + lq), and the block-table prefix covering them."""
    dseqs, pseqs = [], []
    bs = wl.block_size
    for i, sp in enumerate(wl.seqs):
        table = [int(b) for b in wl.block_tables[i, :-(-sp.lk // bs)]]
        is_decode = sp.lq == 1 or i < wl.extra.get("split_pt", 0) + wl.extra.get("num_spec_seqs", 0)
        n_tok = sp.cached + 1 if is_decode else sp.cached + sp.lq
        (dseqs if is_decode else pseqs).append(_StepSeq(n_tok, sp.cached, sp.lq, table, bs))
    return dseqs, pseqs


def bench_metadata(wl, steps=200, warmup=20):
    """Per-step metadata build for a workload step: host time of the call and
    time to completion (call + synchronize), for the on-device build and the
    vectorised host build, and the GPU time of the on-device build's upload +
    kernel (HIP events on the current stream)."""
    from nanovllm_amd.engine import metadata as nm
    from nanovllm_amd.utils.context import set_context
    dseqs, pseqs = step_sequences(wl)
    bs = wl.block_size
    res = {}
    for name, fn in (("device", lambda: nm.prepare_sequence_device(dseqs, pseqs, bs, set_context)),
                     ("host_numpy", lambda: nm.prepare_sequence(dseqs, pseqs, bs, set_context))):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        host = (time.perf_counter() - t0) / steps
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
            torch.cuda.synchronize()
        e2e = (time.perf_counter() - t0) / steps
        res[name] = dict(host_us=round(host * 1e6, 2), to_completion_us=round(e2e * 1e6, 2))
    step = nm.pack_step(dseqs, pseqs, bs)
    ms = timed(lambda i: nm.build_device_metadata(step, bs), steps, warmup)
    res["device"]["gpu_us"] = round(ms * 1e3, 2)
    res["tokens"], res["sequences"] = step.num_tokens, step.num_seqs
    return res, dseqs, pseqs


def cpu_baseline_metadata(dseqs, pseqs, bs, steps=50):
    """The reference's own per-step work, restated by the oracle's Python loops
    (model_runner.py:133-220), plus its per-tensor pinned copies."""
    from oracle import metadata as om
    dev = torch.device("cuda")

    def ref_step():
        m = om.prepare_sequence(dseqs, pseqs, bs)
        out = [torch.tensor(m["positions"], dtype=torch.int64, pin_memory=True).to(dev, non_blocking=True),
               torch.tensor(m["slot_mapping"], dtype=torch.int32, pin_memory=True).to(dev, non_blocking=True)]
        for key in ("context_lens", "cu_seqlens_q", "cu_seqlens_k"):
            if m[key] is not None:
                out.append(torch.tensor(m[key], dtype=torch.int32, pin_memory=True).to(dev, non_blocking=True))
        if m["block_tables"] is not None:
            out.append(torch.tensor(m["block_tables"], dtype=torch.int32, pin_memory=True).to(dev, non_blocking=True))
        return out

    for _ in range(5):
        ref_step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        ref_step()
    host = (time.perf_counter() - t0) / steps
    torch.cuda.synchronize()
    return dict(value=round(host * 1e6, 2), unit="us per step (host)", cores=1, kind="port",
                sample=f"{steps} steps of the same workload step")


def copy_probe(reps=4):
    """A plain device copy of known size: its FETCH_SIZE / WRITE_SIZE readings
    under rocprofv3 --pmc give the counters' scale."""
    src = torch.full((COPY_PROBE_BYTES,), 7, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copy probe: {reps} x {COPY_PROBE_BYTES} bytes")


def cpu_baseline_decode(wl, pool, q, target_s=12.0):
    """The oracle (torch-CPU dequant + fp32 attention) on a bounded sample of
    the same workload: whole passes over all sequences, same cache bytes,
    repeated until about `target_s` seconds of CPU work."""
    from oracle import attention as oa
    kc = pool[0].view(torch.uint8).cpu()
    vc = pool[1].view(torch.uint8).cpu()
    qc = q[:wl.num_seqs].cpu()
    bt = torch.from_numpy(wl.block_tables)
    ctx = torch.from_numpy(wl.context_lens())
    torch.set_num_threads(os.cpu_count() or 1)
    oa.decode_attention(qc, kc, vc, bt, ctx, SCALE)  # warm-up
    times = []
    t_start = time.perf_counter()
    while time.perf_counter() - t_start < target_s or len(times) < 3:
        t0 = time.perf_counter()
        oa.decode_attention(qc, kc, vc, bt, ctx, SCALE)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    return dict(value=round(wl.decode_bytes() / t / 1e9, 4), unit="GB/s",
                cores=torch.get_num_threads(), kind="port",
                sample=f"all {wl.num_seqs} sequences of {wl.name} ({wl.decode_bytes() / 1e6:.1f} MB "
                       f"algorithmic) per pass, median of {len(times)} passes of {t:.3f}s "
                       f"({sum(times):.1f}s total); cpu={_cpu_model()}")


def cpu_baseline_prefill(wl, pool, q, seqs=(0, 1), target_s=12.0):
    """The oracle's varlen prefill on a bounded sample of the prefill workload:
    the sequences ``seqs`` (their query rows and paged keys), repeated until
    about `target_s` seconds of CPU work; the rate is the sample's unmasked
    causal flops over the median pass."""
    from oracle import attention as oa
    sub = W.sub_workload(wl, list(seqs))
    kc = pool[0].view(torch.uint8).cpu()
    vc = pool[1].view(torch.uint8).cpu()
    cu_q_full, _ = wl.cu_seqlens()
    rows = np.concatenate([np.arange(cu_q_full[i], cu_q_full[i + 1]) for i in seqs])
    qc = q[torch.from_numpy(rows).cuda()].cpu()
    cu_q, cu_k = (torch.from_numpy(x) for x in sub.cu_seqlens())
    bt = torch.from_numpy(sub.block_tables)
    torch.set_num_threads(os.cpu_count() or 1)
    oa.prefill_attention(qc, kc, vc, bt, cu_q, cu_k, SCALE)  # warm-up
    times = []
    t_start = time.perf_counter()
    while time.perf_counter() - t_start < target_s or len(times) < 3:
        t0 = time.perf_counter()
        oa.prefill_attention(qc, kc, vc, bt, cu_q, cu_k, SCALE)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    flops = sub.attention_flops()
    desc = ", ".join(f"seq {i}: {wl.seqs[i].lq} rows over {wl.seqs[i].lk} keys" for i in seqs)
    return dict(value=round(flops / t / 1e12, 5), unit="TFLOP/s", cores=torch.get_num_threads(), kind="port",
                sample=f"{len(seqs)} of {wl.num_seqs} sequences of {wl.name} ({desc}; {flops / 1e9:.2f} GFLOP "
                       f"of the call's {wl.attention_flops() / 1e9:.1f}) per pass, median of {len(times)} passes "
                       f"of {t:.3f}s ({sum(times):.1f}s total); cpu={_cpu_model()}")


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _traffic_from_profile():
    """HBM bytes per decode launch from the committed counter summary."""
    try:
        with open(PMC_SUMMARY) as f:
            d = json.load(f)
        return int(d["hbm_bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None


def main():
    args = parse()
    only = set(args.only.split(","))
    unknown = only - set(FIELDS) - {"all"}
    if unknown:
        print(f"bench.py: unknown --only field(s) {sorted(unknown)}; choose from {FIELDS} or all", file=sys.stderr)
        sys.exit(2)

    def want(field):
        return "all" in only or field in only

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}): this build has no "
              "multi-GPU path; run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)
    torch.cuda.set_device(0)
    line = {}
    extra = {}
    if args.copy_probe:
        copy_probe()

    if want("decode"):
        wl = W.qwen3_8b_decode()
        log(f"decode workload {wl.name}: B={wl.num_seqs} bytes={wl.decode_bytes()}")
        res, pools, q = bench_decode(wl, args.steps, args.warmup)
        log(f"decode: {res['ms'] * 1e3:.1f} us/step, {res['gbs']:.1f} GB/s")
        line.update(metric=METRIC, value=round(res["gbs"], 2), unit="GB/s",
                    ms_per_step=round(res["ms"], 5),
                    roofline=dict(bound="hbm", achieved=round(res["gbs"], 2), peak=HBM_PEAK_GBS,
                                  unit="GB/s", frac=round(res["gbs"] / HBM_PEAK_GBS, 4),
                                  traffic=_traffic_from_profile(),
                                  kernel="decode_sk_kernel<1,8,QL> + decode_sk_merge_heads_kernel (one decode call)",
                                  algorithmic_bytes_per_launch=res["bytes"]),
                    config=dict(workload=wl.name, batch=wl.num_seqs, num_heads=wl.num_heads,
                                num_kv_heads=wl.num_kv_heads, head_dim=128, block_size=wl.block_size,
                                context="uniform[256,4096] (the mixed batch's plain-decode rows)",
                                kv_dtype="float8_e4m3fn", kv_pools=2))
        if not args.no_cpu_baseline:
            log("cpu baseline (oracle) on the decode workload")
            line["cpu_baseline"] = cpu_baseline_decode(wl, pools[0], q)
        del pools
        torch.cuda.empty_cache()

    if want("decode06"):
        wl = W.qwen3_0p6b_decode()
        log(f"decode workload {wl.name}: B={wl.num_seqs} bytes={wl.decode_bytes()}")
        res, pools, q = bench_decode(wl, args.steps, args.warmup)
        log(f"decode (0.6B shapes): {res['ms'] * 1e3:.1f} us/step, {res['gbs']:.1f} GB/s")
        extra["decode_qwen3_0p6b"] = dict(workload=wl.name + " (16/8 heads, B=256, ctx U[100, 2048])",
                                          ms_per_step=round(res["ms"], 5), gbs=round(res["gbs"], 2),
                                          frac_hbm_peak=round(res["gbs"] / HBM_PEAK_GBS, 4),
                                          algorithmic_bytes_per_step=res["bytes"],
                                          kernels="decode_sk_kernel<1,8,QL> + decode_sk_merge_heads_kernel")
        del pools
        torch.cuda.empty_cache()

    if want("prefill"):
        wl = W.qwen3_8b_prefill()
        log(f"prefill workload {wl.name}: flops={wl.attention_flops()}")
        res, pools, q = bench_prefill(wl, max(args.steps // 2, 5), max(args.warmup // 2, 2), warm_s=SECONDARY_WARM_S)
        log(f"prefill: {res['ms'] * 1e3:.1f} us/step, {res['tflops']:.1f} TFLOP/s")
        extra["prefill"] = dict(workload=wl.name, ms_per_step=round(res["ms"], 5),
                                tflops=round(res["tflops"], 2),
                                frac_bf16_peak=round(res["tflops"] / BF16_PEAK_TFLOPS, 4),
                                algorithmic_flops_per_step=res["flops"],
                                kernels="decode_sk_kernel<2,4> (short-query rows, none here; one workgroup "
                                        "writes the work list) + varlen_prefill_kernel<true>")
        if not args.no_cpu_baseline:
            log("cpu baseline (oracle) on a sample of the prefill workload")
            extra["prefill"]["cpu_baseline"] = cpu_baseline_prefill(wl, pools[0], q)
        res_b = bench_contiguous_batch(wl, pools, q, max(args.steps // 2, 5), max(args.warmup // 2, 2))
        log(f"prefill, contiguous layout: {res_b['ms'] * 1e3:.1f} us/step, {res_b['tflops']:.1f} TFLOP/s")
        extra["contiguous_prefill_batch"] = dict(
            workload=wl.name + " in the contiguous layout (block_tables=None, K/V gathered per sequence)",
            ms_per_step=round(res_b["ms"], 5), tflops=round(res_b["tflops"], 2),
            frac_bf16_peak=round(res_b["tflops"] / BF16_PEAK_TFLOPS, 4), algorithmic_flops_per_step=res_b["flops"],
            kernels="prefill_short_kernel (the work list) + varlen_prefill_kernel<false>")
        del pools, q
        torch.cuda.empty_cache()

    if want("store"):
        wl = W.qwen3_8b_prefill()
        res = bench_store(wl, max(args.steps, 20), max(args.warmup, 5))
        log(f"store: {res['ms'] * 1e3:.1f} us/step, {res['gbs']:.1f} GB/s")
        log(f"store ceilings: torch bf16->fp8 conversion of as many elements {res['conversion_copy_ms'] * 1e3:.1f} us; "
            f"device copy of the same total bytes {res['device_copy_ms'] * 1e3:.1f} us")
        extra["store"] = dict(workload=wl.name + " new tokens (8192 x 8 kv heads, strided K/V views of qkv)",
                              ms_per_step=round(res["ms"], 5), gbs=round(res["gbs"], 2),
                              frac_hbm_peak=round(res["gbs"] / HBM_PEAK_GBS, 4), algorithmic_bytes_per_step=res["bytes"],
                              kernels="kv_store_fp8_pair_kernel",
                              ceilings=dict(
                                  conversion_copy_ms=round(res["conversion_copy_ms"], 5),
                                  conversion_copy="torch bf16 -> float8_e4m3fn copy_ of the same 2 x 8192 x 8 x 128 "
                                                  "contiguous elements (same read and write bytes, no slot ids)",
                                  device_copy_ms=round(res["device_copy_ms"], 5),
                                  device_copy_gbs=round(res["device_copy_bytes"] / (res["device_copy_ms"] * 1e-3) / 1e9, 2),
                                  device_copy="torch uint8 copy_ moving the same total bytes (half read, half written)"))
        torch.cuda.empty_cache()

    if want("store"):
        wl = W.qwen3_8b_prefill()
        res = bench_qk_norm_rope(wl, max(args.steps, 20), max(args.warmup, 5))
        log(f"fused q/k norm + rope + store: {res['ms'] * 1e3:.1f} us/step, {res['gbs']:.1f} GB/s")
        extra["qk_norm_rope_store"] = dict(
            workload=wl.name + " new tokens (8192 x (32 + 2 x 8) head rows of the QKV projection output)",
            ms_per_step=round(res["ms"], 5), gbs=round(res["gbs"], 2), frac_hbm_peak=round(res["gbs"] / HBM_PEAK_GBS, 4),
            algorithmic_bytes_per_step=res["bytes"], kernels="qk_norm_rope_store_kernel")
        torch.cuda.empty_cache()

    if want("mixed"):
        full = W.qwen3_8b_mixed()
        varlen = W.sub_workload(full, range(full.extra["split_pt"], full.num_seqs), name="qwen3_8b_mixed_varlen")
        spec = W.sub_workload(full, range(full.extra["split_pt"], full.extra["split_pt"] + full.extra["num_spec_seqs"]),
                              name="qwen3_8b_mixed_spec")
        res, pools, _ = bench_prefill(varlen, max(args.steps // 2, 5), max(args.warmup // 2, 2), warm_s=SECONDARY_WARM_S)
        del pools
        res_s, pools, _ = bench_prefill(spec, max(args.steps // 2, 5), max(args.warmup // 2, 2), warm_s=SECONDARY_WARM_S)
        del pools
        spec_bytes = spec.decode_bytes()
        res_c = bench_contiguous(full.extra["contiguous_prompt_len"], full.num_heads, full.num_kv_heads,
                                 max(args.steps // 2, 5), max(args.warmup // 2, 2))
        log(f"mixed varlen: {res['ms'] * 1e3:.1f} us/step; spec rows: {res_s['ms'] * 1e3:.1f} us/step; "
            f"contiguous prompt: {res_c['ms'] * 1e3:.1f} us/step")
        extra["mixed"] = dict(
            workload="qwen3_8b_mixed varlen call: 32 speculative x 5 rows + 3 x 512-token chunks (32/8 heads)",
            ms_per_step=round(res["ms"], 5), tflops=round(res["tflops"], 2),
            frac_bf16_peak=round(res["tflops"] / BF16_PEAK_TFLOPS, 4), algorithmic_flops_per_step=res["flops"],
            spec_rows_only=dict(ms_per_step=round(res_s["ms"], 5), algorithmic_bytes_per_step=spec_bytes,
                                gbs=round(spec_bytes / (res_s["ms"] * 1e-3) / 1e9, 2),
                                frac_hbm_peak=round(spec_bytes / (res_s["ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)),
            kernels="decode_sk_kernel<2,4> (speculative rows, stream-K; one workgroup writes the work list) + "
                    "varlen_prefill_kernel<true> (chunks, and the merge); speculative rows alone: decode_sk_kernel "
                    "+ decode_sk_merge_kernel")
        extra["contiguous_prefill"] = dict(
            workload="qwen3_8b_mixed contiguous prompt: 1024 tokens, block_tables=None (32/8 heads)",
            ms_per_step=round(res_c["ms"], 5), tflops=round(res_c["tflops"], 2),
            frac_bf16_peak=round(res_c["tflops"] / BF16_PEAK_TFLOPS, 4), algorithmic_flops_per_step=res_c["flops"],
            kernels="varlen_prefill_kernel<false>")
        torch.cuda.empty_cache()

    if want("long"):
        wl = W.qwen3_32b_long_decode()
        log(f"long decode workload {wl.name}: bytes={wl.decode_bytes()}")
        res, pools, _ = bench_decode(wl, max(args.steps // 5, 5), max(args.warmup // 5, 2), n_pools=1,
                                     warm_s=SECONDARY_WARM_S)
        log(f"long decode: {res['ms'] * 1e3:.1f} us/step, {res['gbs']:.1f} GB/s")
        extra["long_decode"] = dict(workload=wl.name, ms_per_step=round(res["ms"], 5),
                                    gbs=round(res["gbs"], 2), frac_hbm_peak=round(res["gbs"] / HBM_PEAK_GBS, 4),
                                    algorithmic_bytes_per_step=res["bytes"],
                                    kernels="decode_sk_kernel<1,8,QL> + decode_sk_merge_kernel")
        del pools
        torch.cuda.empty_cache()

    if want("linear"):
        # Qwen3-8B FP8 checkpoints: the qkv projection of a 16 x 512-token
        # prefill step (MFMA-bound) and the gate/up projection of the mixed
        # batch's 192 decode rows (weight-streaming, HBM-bound)
        # Qwen3-8B FP8 checkpoints at the 16 x 512-token prefill step (qkv,
        # gate/up and down projections, MFMA-bound) and at the mixed batch's
        # 192 decode rows (weight-streaming, HBM-bound)
        lin = {}
        for name, (M, N, K) in (("prefill_qkv", (8192, 6144, 4096)), ("prefill_gate_up", (8192, 24576, 4096)),
                                ("prefill_down", (8192, 4096, 12288)), ("decode_qkv", (192, 6144, 4096)),
                                ("decode_gate_up", (192, 24576, 4096)), ("decode_down", (192, 4096, 12288))):
            big = M >= 1024
            r = bench_fp8_linear(M, N, K, max(args.steps // 2, 10) if big else max(args.steps, 20),
                                 max(args.warmup // 2, 3) if big else max(args.warmup, 5))
            e = dict(shape=f"M={M} tokens, N={N}, K={K}", ms_per_step=round(r["ms"], 5),
                     tflops=round(r["tflops"], 1), frac_fp8_peak=round(r["tflops"] / FP8_PEAK_TFLOPS, 4),
                     algorithmic_flops=r["flops"], quant_us=round(r["quant_us"], 2),
                     quant_gbs=round(r["quant_gbs"], 1), fp8_block_linear_us=round(r["linear_us"], 2),
                     hipblaslt_per_tensor_us=r["hipblaslt_per_tensor_us"])
            if not big:
                e.update(weight_gbs=round(r["weight_gbs"], 1), frac_hbm_peak=round(r["weight_gbs"] / HBM_PEAK_GBS, 4),
                         algorithmic_bytes=r["weight_bytes"])
            lin[name] = e
            log(f"fp8 linear {name} M={M} N={N} K={K}: {r['ms'] * 1e3:.1f} us ({r['tflops']:.0f} TFLOP/s"
                + ("" if big else f", {r['weight_gbs']:.0f} GB/s of weights")
                + f"); hipBLASLt per-tensor {r['hipblaslt_per_tensor_us']} us")
        extra["fp8_linear"] = dict(
            workload="FP8 block-scaled linear (128x128 weight blocks), Qwen3-8B shapes",
            kernels="block_gemm_kernel; skinny_gemm_kernel (+ skinny_reduce_kernel when K is split) for at most "
                    "256 tokens where the tile grid would leave CUs idle; act_quant_kernel timed separately; "
                    "hipblaslt_per_tensor_us: torch._scaled_mm with one scale per tensor, same operands; weights "
                    "cycled over > 600 MiB (streamed from HBM)", **lin)
        if not args.no_cpu_baseline:
            log("cpu baseline (oracle) for the FP8 linear")
            extra["fp8_linear"]["cpu_baseline"] = cpu_baseline_fp8_linear(6144, 4096)
        torch.cuda.empty_cache()

    if want("metadata"):
        out = {}
        for wl in (W.qwen3_8b_mixed(), W.qwen3_8b_prefill()):
            res, dseqs, pseqs = bench_metadata(wl)
            if not args.no_cpu_baseline:
                res["cpu_baseline"] = cpu_baseline_metadata(dseqs, pseqs, wl.block_size)
            out[wl.name] = res
            log(f"metadata {wl.name}: device {res['device']['host_us']:.1f} us host / "
                f"{res['device']['to_completion_us']:.1f} us to completion; host numpy "
                f"{res['host_numpy']['host_us']:.1f} / {res['host_numpy']['to_completion_us']:.1f} us")
        extra["metadata"] = dict(workload="one engine step's attention metadata (mixed batch; 16 x 512 prefill)",
                                 kernels="build_metadata_kernel", **out)

    if want("lm_head"):
        res = bench_sampler(355, 151936, max(args.steps, 20), max(args.warmup, 5))
        sel = bench_select_rows(max(args.steps, 20), max(args.warmup, 5))
        log(f"sampler: {res['ms'] * 1e3:.1f} us ({res['gbs']:.0f} GB/s), reference arithmetic in torch "
            f"{res['ms_torch'] * 1e3:.1f} us; row selection {sel['ms'] * 1e3:.1f} us")
        extra["lm_head"] = dict(
            workload="the mixed step's LM-head rows (192 decode + 32 x 5 speculative + 3 prefill = 355), "
                     "Qwen3 vocabulary 151936, bf16 logits",
            kernels="sample_group_kernel + sample_group_pick_kernel, select_rows_kernel",
            sampler=dict(ms_per_step=round(res["ms"], 5), gbs=round(res["gbs"], 1),
                         frac_hbm_peak=round(res["gbs"] / HBM_PEAK_GBS, 4), algorithmic_bytes=res["bytes"],
                         reference_arithmetic_torch_ms=round(res["ms_torch"], 5)),
            select_rows=dict(ms_per_step=round(sel["ms"], 5), rows=sel["rows"]))
        if not args.no_cpu_baseline:
            extra["lm_head"]["cpu_baseline"] = cpu_baseline_sampler(151936)
        torch.cuda.empty_cache()

    if want("host"):
        res = bench_host_overhead()
        log("host time per call: " + ", ".join(f"{k} {v} us" for k, v in res.items() if isinstance(v, float)))
        extra["host_overhead"] = dict(
            workload="host time per call of the Python entry points (Qwen3-8B head shapes: 192-row decode, the "
                     "mixed batch's 35-sequence varlen call, 8192-token store, 192 x 4096 -> 24576 FP8 linear)",
            **res)
        torch.cuda.empty_cache()

    if "value" not in line:   # partial runs (profiling) still print one line
        first = next(iter(extra.values()))
        line.update(metric=METRIC + " (partial run: " + first["workload"] + ")",
                    value=first.get("tflops", first.get("gbs")),
                    unit="TFLOP/s" if "tflops" in first else "GB/s", ms_per_step=first.get("ms_per_step"),
                    config=dict(workload=first["workload"]))
    line.update(n_gpus=1, steps=args.steps, warmup=args.warmup, higher_is_better=True, scaling="weak",
                vs_baseline=None, dtype="bf16",
                data="synthetic (seeded N(0,1) bf16, K/V quantised to FP8 E4M3 by the store kernel)")
    line.update(extra)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
