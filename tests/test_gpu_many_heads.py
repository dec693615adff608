"""More than 32 query heads per kv head (G > 32) through the drop-in calls.

The reference's kernels take any G (fp8_attention.py:92-94,104,213-215
take the head counts as arguments).  The kernels here take at most 32 query
heads per kv head, so the operators run such a call as G / gs calls on
gs-head slices of every kv head's query heads (gs the largest divisor of G up
to 32) and copy each slice's output back.  These tests check that
layout against the oracle: G = 64 (two slices of 32), G = 48 (two slices of
24) and G = 40 (two slices of 20), for decode and for ragged paged and
contiguous prefill.
"""
import numpy as np
import pytest
import torch

from gpu_util import announce, assert_close, build_pair
from oracle import attention as oa
import workloads as W
from nanovllm_amd.kernels.fp8_attention import fp8_decode_attention, fp8_prefill_attention

pytestmark = pytest.mark.gpu

SCALE = 128 ** -0.5
FP8 = torch.float8_e4m3fn
SHAPES = [(64, 1), (96, 2), (40, 1)]


@pytest.mark.parametrize("hq,hkv", SHAPES)
def test_decode_many_heads_per_kv_head(hq, hkv):
    wl = W.decode_workload(f"decode_g{hq // hkv}_{hq}_{hkv}", 12, hq, hkv, 1, 1500, seed=hq + hkv)
    announce(f"many heads: decode {hq}/{hkv} heads (G = {hq // hkv}), 12 sequences")
    cpu_c, gpu_c = build_pair(wl)
    q = wl.make_q("cpu")
    bt = torch.from_numpy(wl.block_tables)
    ctx = torch.from_numpy(wl.context_lens())
    out = fp8_decode_attention(q.cuda(), gpu_c[0], gpu_c[1], bt.cuda(), ctx.cuda(), SCALE)
    torch.cuda.synchronize()
    assert out.shape == q.shape and out.dtype == q.dtype
    want = oa.decode_attention(q, cpu_c[0], cpu_c[1], bt, ctx, SCALE)
    assert_close(out, want, wl.name)


@pytest.mark.parametrize("hq,hkv", SHAPES)
def test_prefill_many_heads_per_kv_head(hq, hkv):
    """Ragged query lengths (single-token rows included), paged, then the same
    rows in the contiguous layout."""
    rng = np.random.default_rng(7 * hq + hkv)
    lqs = [1, 3, 17, 64, 130, 257]
    seqs = [W.SeqSpec(lq=int(l), cached=int(rng.integers(0, 600))) for l in lqs]
    wl = W.make_workload(f"prefill_g{hq // hkv}_{hq}_{hkv}", hq, hkv, seqs, seed=int(rng.integers(1 << 30)))
    announce(f"many heads: prefill {hq}/{hkv} heads (G = {hq // hkv}), ragged, paged and contiguous")
    cpu_c, gpu_c = build_pair(wl)
    q = wl.make_q("cpu")
    cu_q, cu_k = wl.cu_seqlens()
    kw = dict(cu_seqlens_q=torch.from_numpy(cu_q).cuda(), cu_seqlens_k=torch.from_numpy(cu_k).cuda(),
              max_seqlen_q=int(wl.lq().max()), max_seqlen_k=int(wl.lk().max()), softmax_scale=SCALE)
    out = fp8_prefill_attention(q.cuda(), gpu_c[0], gpu_c[1], block_tables=torch.from_numpy(wl.block_tables).cuda(),
                                **kw)
    torch.cuda.synchronize()
    want = oa.prefill_attention(q, cpu_c[0], cpu_c[1], torch.from_numpy(wl.block_tables), torch.from_numpy(cu_q),
                                torch.from_numpy(cu_k), SCALE)
    assert_close(out, want, wl.name)
    rows = np.concatenate([wl.slots_for(i, 0, s.lk) for i, s in enumerate(wl.seqs)]).astype(np.int64)
    idx = torch.from_numpy(rows).cuda()
    kcont = gpu_c[0].view(torch.uint8).reshape(-1, hkv, 128)[idx].view(FP8)
    vcont = gpu_c[1].view(torch.uint8).reshape(-1, hkv, 128)[idx].view(FP8)
    out_c = fp8_prefill_attention(q.cuda(), kcont, vcont, block_tables=None, **kw)
    torch.cuda.synchronize()
    want_c = oa.prefill_attention(q, kcont.cpu(), vcont.cpu(), None, torch.from_numpy(cu_q), torch.from_numpy(cu_k),
                                  SCALE)
    assert_close(out_c, want_c, wl.name + " contiguous")
