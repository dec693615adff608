"""The decode entry point that allocates nothing (nvamd_fp8_decode_attention_noalloc),
through the C ABI, against nvamd_fp8_decode_attention with a caller workspace.

Both run the same kernels on the same inputs, so the outputs must be
bit-identical.  The calls come in a row with shrinking inputs (the library's
scratch array keeps the previous call's contents), through the balanced
(stream-K) kernel and the split-KV kernel (which keeps its partials in the
scratch too), and a shape whose workspace exceeds the array is rejected
before anything is launched.
"""
import numpy as np
import pytest
import torch

import workloads as W
from gpu_util import announce
from nanovllm_amd import _native

pytestmark = pytest.mark.gpu
SCALE = 128 ** -0.5


def _inputs(wl):
    kc, vc = wl.empty_caches("cuda")
    from nanovllm_amd.layers.attention import store_kvcache
    wl.fill_cache(kc, vc, store_kvcache, gen_device="cuda")
    q = wl.make_q("cuda")
    bt = torch.from_numpy(wl.block_tables).cuda()
    ctx = torch.from_numpy(wl.context_lens()).cuda()
    return q, kc, vc, bt, ctx


def _args(wl, q, kc, vc, bt, ctx):
    return (q.data_ptr(), kc.data_ptr(), vc.data_ptr(), bt.data_ptr(), ctx.data_ptr(), wl.num_seqs,
            wl.num_heads, wl.num_kv_heads, 128, wl.num_blocks, wl.block_size, bt.shape[1], SCALE)


def _with_workspace(lib, wl, inputs):
    q, kc, vc, bt, ctx = inputs
    n = lib.nvamd_decode_workspace_bytes(wl.num_seqs, wl.num_heads, wl.num_kv_heads, bt.shape[1],
                                         wl.block_size, 0)
    ws = torch.empty(max(n, 1), dtype=torch.uint8, device="cuda")
    out = torch.empty_like(q)
    st = lib.nvamd_fp8_decode_attention(out.data_ptr(), *_args(wl, *inputs), 0, ws.data_ptr(), n, 0,
                                        torch.cuda.current_stream().cuda_stream)
    _native.check(st, "nvamd_fp8_decode_attention")
    return out, n


def _no_alloc(lib, wl, inputs):
    out = torch.empty_like(inputs[0])
    st = lib.nvamd_fp8_decode_attention_noalloc(out.data_ptr(), *_args(wl, *inputs), 0,
                                                torch.cuda.current_stream().cuda_stream)
    _native.check(st, "nvamd_fp8_decode_attention_noalloc")
    return out


def test_no_alloc_decode_matches_workspace_decode():
    lib = _native.load()
    rng = np.random.default_rng(41)
    cases = [
        # (name, num_heads, num_kv_heads, contexts): stream-K with G = 4 and
        # G = 8, then the split-KV kernel (Hkv = 2) with partitions
        ("stream-K 32/8, B=160", 32, 8, rng.integers(1, 6000, size=160)),
        ("stream-K 64/8, B=24", 64, 8, rng.integers(1, 9000, size=24)),
        ("split-KV 32/2, B=6", 32, 2, rng.integers(20000, 60000, size=6)),
    ]
    for name, hq, hkv, ctx in cases:
        seqs = [W.SeqSpec(lq=1, cached=int(c) - 1) for c in ctx]
        wl = W.make_workload(f"noalloc_{hq}_{hkv}_{len(seqs)}", hq, hkv, seqs, seed=int(rng.integers(1 << 30)))
        announce(f"no-alloc decode: {name}")
        inputs = _inputs(wl)
        want, need = _with_workspace(lib, wl, inputs)
        assert 0 < need <= lib_scratch_bytes()
        got = _no_alloc(lib, wl, inputs)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"{name}: no-alloc output differs from the workspace call"


def lib_scratch_bytes():
    return 32 << 20  # NVAMD_NOALLOC_SCRATCH_BYTES


def test_no_alloc_decode_rejects_shapes_beyond_the_scratch():
    lib = _native.load()
    # split-KV partials of 4096 rows x 64 heads x 2 partitions: 272 MB
    need = lib.nvamd_decode_workspace_bytes(4096, 64, 2, 64, 256, 0)
    assert need > lib_scratch_bytes()
    fake = 0x1000  # rejected before any pointer is used
    st = lib.nvamd_fp8_decode_attention_noalloc(fake, fake, fake, fake, fake, fake, 4096, 64, 2, 128, 20000, 256,
                                                64, SCALE, 0, None)
    assert st == 3 and b"scratch" in lib.nvamd_last_error()
