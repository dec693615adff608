"""Varlen causal (chunked) FP8 prefill on the GPU vs the oracle, paged and contiguous."""
import numpy as np
import pytest
import torch

from gpu_util import announce, assert_close, build_pair
from oracle import attention as oa
import workloads as W
from nanovllm_amd.kernels.fp8_attention import fp8_decode_attention, fp8_prefill_attention

pytestmark = pytest.mark.gpu
SCALE = 128 ** -0.5


def _prefill_gpu(wl, gpu_c, q, paged=True, kv=None, cu_k=None):
    cu_q, cu_k_p = wl.cu_seqlens()
    kw = dict(cu_seqlens_q=torch.from_numpy(cu_q).cuda(),
              cu_seqlens_k=torch.from_numpy(cu_k_p if cu_k is None else cu_k).cuda(),
              max_seqlen_q=int(wl.lq().max()), max_seqlen_k=int(wl.lk().max()), softmax_scale=SCALE)
    if paged:
        out = fp8_prefill_attention(q, gpu_c[0], gpu_c[1], block_tables=torch.from_numpy(wl.block_tables).cuda(), **kw)
    else:
        out = fp8_prefill_attention(q, kv[0], kv[1], block_tables=None, **kw)
    torch.cuda.synchronize()
    return out


def _prefill_oracle(wl, cpu_c, q):
    cu_q, cu_k = wl.cu_seqlens()
    return oa.prefill_attention(q, cpu_c[0], cpu_c[1], torch.from_numpy(wl.block_tables),
                                torch.from_numpy(cu_q), torch.from_numpy(cu_k), SCALE)


def _check(wl):
    cpu_c, gpu_c = build_pair(wl)
    q = wl.make_q("cpu")
    out = _prefill_gpu(wl, gpu_c, q.cuda())
    assert_close(out, _prefill_oracle(wl, cpu_c, q), wl.name)
    return cpu_c, gpu_c, q, out


def test_prefill_qwen3_8b_chunks():
    wl = W.qwen3_8b_prefill()
    announce(f"prefill: {wl.name}")
    _check(wl)


def test_mixed_batch_through_the_attention_layer():
    """The whole mixed batch at Qwen3-8B shapes, as the reference's Attention
    layer runs it (nanovllm/layers/attention.py:58-96): 192 plain-decode rows
    before split_pt go to fp8_decode_attention, the 32 speculative sequences
    (5 rows each) and 3 chunks of 512 tokens to fp8_prefill_attention, and the
    outputs are concatenated.  Every row against the oracle."""
    from attention_layer import Attention
    from nanovllm_amd.utils.context import reset_context, set_context
    wl = W.qwen3_8b_mixed()
    sp = wl.extra["split_pt"]
    announce(f"mixed batch through the attention layer: {sp} decode + {wl.num_seqs - sp} varlen sequences")
    cpu_c, gpu_c = build_pair(wl, gen_device="cuda")
    q = wl.make_q("cpu")
    vl = W.sub_workload(wl, range(sp, wl.num_seqs))
    cu_q, cu_k = vl.cu_seqlens()
    bt = torch.from_numpy(wl.block_tables).cuda()
    n = q.shape[0]
    attn = Attention(wl.num_heads, 128, SCALE)
    attn.k_cache, attn.v_cache = gpu_c
    # K/V of this step are already in the cache: every slot is -1, nothing is stored
    set_context(split_pt=sp, num_spec_seqs=wl.extra["num_spec_seqs"],
                cu_seqlens_q=torch.from_numpy(cu_q).cuda(), cu_seqlens_k=torch.from_numpy(cu_k).cuda(),
                max_seqlen_q=int(vl.lq().max()), max_seqlen_k=int(vl.lk().max()),
                slot_mapping=torch.full((n,), -1, dtype=torch.int32, device="cuda"),
                context_lens=torch.from_numpy(wl.context_lens()[:sp]).cuda(), block_tables=bt)
    try:
        kv = torch.zeros(n, wl.num_kv_heads, 128, dtype=torch.bfloat16, device="cuda")
        out = attn(q.cuda(), kv, kv)
        torch.cuda.synchronize()
    finally:
        reset_context()
    want_d = oa.decode_attention(q[:sp], cpu_c[0], cpu_c[1], torch.from_numpy(wl.block_tables[:sp]),
                                 torch.from_numpy(wl.context_lens()[:sp]), SCALE)
    want_p = oa.prefill_attention(q[sp:], cpu_c[0], cpu_c[1], torch.from_numpy(vl.block_tables),
                                  torch.from_numpy(cu_q), torch.from_numpy(cu_k), SCALE)
    assert out.shape == q.shape
    assert_close(out[:sp], want_d, "mixed batch: plain-decode rows")
    assert_close(out[sp:], want_p, "mixed batch: speculative rows and chunks")


def test_prefill_mixed_spec_and_chunks():
    full = W.qwen3_8b_mixed()
    wl = W.sub_workload(full, range(192, full.num_seqs), name="mixed_varlen")  # spec + chunks
    announce(f"prefill: {wl.name} (32 spec x 5 + 3 x 512)")
    _check(wl)


@pytest.mark.parametrize("hq,hkv", [(32, 8), (16, 8), (64, 8), (8, 8), (24, 8), (12, 4), (16, 2)])
def test_prefill_ragged(hq, hkv):
    rng = np.random.default_rng(hq + 7 * hkv)
    lqs = [1, 2, 3, 5, 8, 9, 17, 31, 32, 33, 64, 100, 129, 300]
    seqs = [W.SeqSpec(lq=int(l), cached=int(rng.integers(0, 700))) for l in lqs]
    seqs.append(W.SeqSpec(lq=77, cached=0))
    wl = W.make_workload(f"ragged_{hq}_{hkv}", hq, hkv, seqs, seed=int(rng.integers(1 << 30)))
    announce(f"prefill: ragged GQA {hq}/{hkv}")
    _check(wl)


def test_prefill_contiguous_equals_paged():
    rng = np.random.default_rng(3)
    seqs = [W.SeqSpec(lq=l, cached=0) for l in (1024, 300, 65, 4)]
    wl = W.make_workload("contiguous_prompts", 32, 8, seqs, seed=99)
    announce("prefill: contiguous layout (block_tables=None)")
    cpu_c, gpu_c, q, paged_out = _check(wl)
    # gather each sequence's K/V rows out of the paged cache into [Nk, Hkv, D]
    bt = wl.block_tables
    rows = np.concatenate([wl.slots_for(i, 0, s.lk) for i, s in enumerate(wl.seqs)]).astype(np.int64)
    idx = torch.from_numpy(rows).cuda()
    kcont = gpu_c[0].view(torch.uint8).reshape(-1, 8, 128)[idx].view(torch.float8_e4m3fn)
    vcont = gpu_c[1].view(torch.uint8).reshape(-1, 8, 128)[idx].view(torch.float8_e4m3fn)
    out = _prefill_gpu(wl, gpu_c, q.cuda(), paged=False, kv=(kcont, vcont))
    cu_q, cu_k = wl.cu_seqlens()
    want = oa.prefill_attention(q, kcont.cpu(), vcont.cpu(), None, torch.from_numpy(cu_q),
                                torch.from_numpy(cu_k), SCALE)
    assert_close(out, want, "contiguous")
    assert_close(out, paged_out, "contiguous vs paged", atol=1e-3, rtol=1e-3)


def test_prefill_lq1_equals_decode():
    """Lq = 1 prefill rows against decode: at this shape (Hkv % 4 == 0, paged)
    both run the balanced stream-K kernel over the same stages.  Decode gives
    the even-numbered workgroups a slightly larger share than a varlen call
    does, so the two cut pairs at different stages and differ by the rounding
    of the merge: one bf16 ulp, or 2^-10 absolute where a cut pair's fp16
    partial (2^-11 of the V values) meets cancellation; each stays within the
    tolerance of the oracle."""
    announce("prefill: Lq=1 rows equal decode")
    wl = W.qwen3_0p6b_decode(B=24)
    cpu_c, gpu_c = build_pair(wl)
    q = wl.make_q("cpu")
    dec = fp8_decode_attention(q.cuda(), gpu_c[0], gpu_c[1], torch.from_numpy(wl.block_tables).cuda(),
                               torch.from_numpy(wl.context_lens()).cuda(), SCALE)
    pre = _prefill_gpu(wl, gpu_c, q.cuda())
    want = oa.decode_attention(q, cpu_c[0], cpu_c[1], torch.from_numpy(wl.block_tables),
                               torch.from_numpy(wl.context_lens()), SCALE)
    assert_close(dec, want, "decode")
    assert_close(pre, want, "Lq=1 prefill")
    torch.testing.assert_close(pre.float(), dec.float(), rtol=2.0 ** -7, atol=2.0 ** -10,
                               msg="Lq=1 prefill vs decode: more than one bf16 ulp apart")


@pytest.mark.parametrize("bs", [16, 32, 48, 64, 192, 512])
def test_prefill_block_sizes(bs):
    """Block sizes other than 256, down to 16 (the reference accepts any
    kvcache_block_size % 16 == 0): each wave's 8- or 16-row load group gets
    the block of its first row from a multiply with the reciprocal of the
    block size; 48 and 192 are not powers of two; with 16 and 32 a 64-token
    tile spans several blocks.  Chunks cross many block borders."""
    rng = np.random.default_rng(bs)
    seqs = [W.SeqSpec(lq=int(l), cached=int(rng.integers(0, 900))) for l in (300, 129, 64, 7, 512)]
    wl = W.make_workload(f"prefill_bs{bs}", 32, 8, seqs, seed=int(rng.integers(1 << 30)), block_size=bs)
    announce(f"prefill: block_size {bs}")
    _check(wl)


@pytest.mark.parametrize("bs,cached,lq", [(16, 2500, 300), (64, 4500, 300), (256, 16900, 200)])
def test_prefill_multi_window_block_tables(bs, cached, lq):
    """Sequences with more than 64 blocks: the kernel holds a 64-entry window
    of the block table in one register and reloads it at the window edge
    (4096 tokens at block size 64, 16384 at 256); the chunk straddles it."""
    seqs = [W.SeqSpec(lq=lq, cached=cached), W.SeqSpec(lq=65, cached=4000), W.SeqSpec(lq=33, cached=100)]
    wl = W.make_workload(f"prefill_windows_bs{bs}", 32, 8, seqs, seed=bs + 11, block_size=bs)
    announce(f"prefill: block-table windows, block_size {bs}, Lk {cached + lq}")
    _check(wl)


@pytest.mark.parametrize("bs", [16, 32])
def test_prefill_small_blocks_split_kv_short_rows(bs):
    """Block sizes 16 and 32 with 2 kv heads: the short-query rows take the
    split-KV kernel (its stages span several blocks) and the long ones the
    prefill kernel, in one call."""
    rng = np.random.default_rng(bs + 5)
    seqs = [W.SeqSpec(lq=int(l), cached=int(rng.integers(0, 1500))) for l in (1, 3, 5, 16, 17, 200, 64)]
    wl = W.make_workload(f"prefill_small_blocks_{bs}", 32, 2, seqs, seed=int(rng.integers(1 << 30)), block_size=bs)
    announce(f"prefill: block_size {bs}, 32/2 heads (split-KV short rows)")
    _check(wl)


@pytest.mark.parametrize("hq,hkv", [(32, 8), (8, 8), (16, 2)])
def test_prefill_split_pieces_both_layouts(hq, hkv):
    """Calls with fewer work items than a round of workgroups split their long
    items' key ranges into pieces merged by the item's last piece: a
    2048-token prompt (pieces cross the causal diagonal of every m-block
    near the end), a 700-token chunk over 1000 cached keys and a short chunk,
    in the paged layout and in the contiguous one (the same K/V rows
    gathered), against the oracle."""
    seqs = [W.SeqSpec(lq=2048, cached=0), W.SeqSpec(lq=700, cached=1000), W.SeqSpec(lq=40, cached=90)]
    wl = W.make_workload(f"prefill_split_{hq}_{hkv}", hq, hkv, seqs, seed=hq * 7 + hkv)
    announce(f"prefill: split key ranges, {hq}/{hkv} heads, paged and contiguous")
    cpu_c, gpu_c, q, paged_out = _check(wl)
    rows = np.concatenate([wl.slots_for(i, 0, s.lk) for i, s in enumerate(wl.seqs)]).astype(np.int64)
    idx = torch.from_numpy(rows).cuda()
    kcont = gpu_c[0].view(torch.uint8).reshape(-1, hkv, 128)[idx].view(torch.float8_e4m3fn)
    vcont = gpu_c[1].view(torch.uint8).reshape(-1, hkv, 128)[idx].view(torch.float8_e4m3fn)
    out = _prefill_gpu(wl, gpu_c, q.cuda(), paged=False, kv=(kcont, vcont))
    cu_q, cu_k = wl.cu_seqlens()
    want = oa.prefill_attention(q, kcont.cpu(), vcont.cpu(), None, torch.from_numpy(cu_q),
                                torch.from_numpy(cu_k), SCALE)
    assert_close(out, want, "contiguous, split pieces")
    again = _prefill_gpu(wl, gpu_c, q.cuda(), paged=False, kv=(kcont, vcont))
    assert torch.equal(out, again), "split pieces: the merge order is fixed, so repeated calls are bit-identical"


def test_prefill_outlier_kv():
    """1 % of the K/V entries scaled by 20 before quantisation (peaked scores,
    values near the E4M3 range): the lazy rescale and the bf16 weights stay
    within tolerance."""
    seqs = [W.SeqSpec(lq=l, cached=c) for l, c in ((512, 1500), (129, 3000), (64, 0), (300, 700), (5, 2000))]
    wl = W.make_workload("prefill_outliers", 32, 8, seqs, seed=21, outlier_frac=0.01, outlier_scale=20.0)
    announce("prefill: outlier K/V (1% x20)")
    _check(wl)


def test_prefill_zero_length_sequences():
    """Sequences that contribute no query rows (repeated cu_seqlens_q entries),
    with and without cached keys, between ordinary ones."""
    seqs = [W.SeqSpec(lq=0, cached=300), W.SeqSpec(lq=100, cached=50), W.SeqSpec(lq=0, cached=0),
            W.SeqSpec(lq=70, cached=900), W.SeqSpec(lq=3, cached=40), W.SeqSpec(lq=0, cached=1000)]
    wl = W.make_workload("prefill_zero_lq", 32, 8, seqs, seed=23)
    announce("prefill: zero-length sequences in the batch")
    _check(wl)


@pytest.mark.parametrize("q_scale", [4096.0, 1.0e6])
def test_prefill_large_queries(q_scale):
    """The first sequence's queries scaled up.  At 4096 every q * scale * log2(e)
    still fits fp16 (the scaled form, QK^T on fp16 operands) and the scores are
    sharply peaked; at 10^6 some do not, and those workgroups keep q in bf16
    and scale each score instead.  Both must match the oracle."""
    seqs = [W.SeqSpec(lq=l, cached=c) for l, c in ((200, 300), (64, 0), (129, 1000))]
    wl = W.make_workload("prefill_large_q", 32, 8, seqs, seed=25)
    announce(f"prefill: queries of sequence 0 scaled by {q_scale:g}")
    cpu_c, gpu_c = build_pair(wl)
    q = wl.make_q("cpu")
    q[:200] = (q[:200].float() * q_scale).to(torch.bfloat16)
    out = _prefill_gpu(wl, gpu_c, q.cuda())
    assert_close(out, _prefill_oracle(wl, cpu_c, q), f"{wl.name} x{q_scale:g}")
