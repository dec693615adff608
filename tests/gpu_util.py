"""Shared helpers for the GPU parity tests (imported only by tests)."""
import sys

import numpy as np
import torch

from oracle import attention as oa
from oracle import fp8 as ofp8
import workloads as W
from nanovllm_amd.layers.attention import store_kvcache

TOL = dict(atol=1e-2, rtol=1e-2)


def announce(msg):
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def cpu_store(k, v, kc, vc, slots):
    ofp8.store_kvcache(k, v, kc.view(torch.uint8), vc.view(torch.uint8), slots)


def build_pair(wl, include_new=True, gen_device="cpu", dtype=torch.bfloat16):
    """Fills a CPU cache (oracle store) and a GPU cache (HIP store) with the same
    seeded K/V of ``dtype`` (bf16 or fp16; generated on ``gen_device``: "cuda"
    is faster for large workloads); asserts the two caches are byte-identical."""
    kc_cpu, vc_cpu = wl.empty_caches("cpu")
    wl.fill_cache(kc_cpu, vc_cpu, cpu_store, gen_device=gen_device, include_new=include_new, dtype=dtype)
    kc_gpu, vc_gpu = wl.empty_caches("cuda")
    wl.fill_cache(kc_gpu, vc_gpu, store_kvcache, gen_device=gen_device, include_new=include_new, dtype=dtype)
    torch.cuda.synchronize()
    assert torch.equal(kc_gpu.view(torch.uint8).cpu(), kc_cpu.view(torch.uint8)), "K cache bytes differ"
    assert torch.equal(vc_gpu.view(torch.uint8).cpu(), vc_cpu.view(torch.uint8)), "V cache bytes differ"
    return (kc_cpu, vc_cpu), (kc_gpu, vc_gpu)


def assert_close(got, want, what, mask_rows=None, **tol):
    tol = tol or TOL
    g = got.float().cpu()
    w = want.float().cpu()
    if mask_rows is not None:
        g, w = g[mask_rows], w[mask_rows]
    ok = torch.isclose(g, w, **tol)
    if not bool(ok.all()):
        bad = (~ok).nonzero()
        i = tuple(bad[0].tolist())
        raise AssertionError(f"{what}: {int((~ok).sum())} / {ok.numel()} elements outside tolerance; "
                             f"first at {i}: got {g[i].item()} want {w[i].item()}; "
                             f"max abs err {float((g - w).abs().max())}")
