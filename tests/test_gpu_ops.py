"""torch.ops.nvamd.* on the GPU give the same bytes as the Python functions
they register (same C-ABI calls), which the other GPU tests check against
the oracle."""
import pytest
import torch

import workloads as W
from gpu_util import announce
import nanovllm_amd  # noqa: F401
from nanovllm_amd.kernels.fp8_attention import fp8_decode_attention, fp8_prefill_attention
from nanovllm_amd.layers.attention import store_kvcache

pytestmark = pytest.mark.gpu
SCALE = 128 ** -0.5


def _caches(wl, fn):
    kc, vc = wl.empty_caches("cuda")
    wl.fill_cache(kc, vc, fn)
    return kc, vc


def test_ops_store_decode_prefill_equal_the_functions():
    announce("ops: store / decode / prefill through torch.ops.nvamd")
    wl = W.tiny_decode()
    kc_f, vc_f = _caches(wl, store_kvcache)
    kc_o, vc_o = _caches(wl, torch.ops.nvamd.store_kvcache)
    torch.cuda.synchronize()
    assert torch.equal(kc_o.view(torch.uint8), kc_f.view(torch.uint8))
    assert torch.equal(vc_o.view(torch.uint8), vc_f.view(torch.uint8))
    q = wl.make_q("cuda")
    bt = torch.from_numpy(wl.block_tables).cuda()
    ctx = torch.from_numpy(wl.context_lens()).cuda()
    assert torch.equal(torch.ops.nvamd.decode(q, kc_o, vc_o, bt, ctx, SCALE),
                       fp8_decode_attention(q, kc_f, vc_f, bt, ctx, SCALE))

    seqs = [W.SeqSpec(lq=l, cached=c) for l, c in ((5, 300), (70, 0), (129, 40))]
    wl = W.make_workload("ops_prefill", 8, 2, seqs, seed=5)
    kc, vc = _caches(wl, store_kvcache)
    q = wl.make_q("cuda")
    cu_q, cu_k = (torch.from_numpy(x).cuda() for x in wl.cu_seqlens())
    bt = torch.from_numpy(wl.block_tables).cuda()
    mq, mk = int(wl.lq().max()), int(wl.lk().max())
    want = fp8_prefill_attention(q, kc, vc, block_tables=bt, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k,
                                 max_seqlen_q=mq, max_seqlen_k=mk, softmax_scale=SCALE)
    assert torch.equal(torch.ops.nvamd.prefill(q, kc, vc, bt, cu_q, cu_k, mq, mk, SCALE), want)
