"""fp16 queries, keys and values (the reference's kernels take whatever 16-bit
float type they are given; out = empty_like(q)): the store's E4M3FN bytes for
every fp16 pattern, and decode / prefill outputs (fp16, rounded fp32 -> fp16
only) against the oracle on the same inputs, atol/rtol 1e-2."""
import numpy as np
import pytest
import torch

from gpu_util import announce, assert_close, build_pair
from oracle import attention as oa
from oracle import fp8 as ofp8
import workloads as W
from nanovllm_amd.kernels.fp8_attention import fp8_decode_attention, fp8_prefill_attention
from nanovllm_amd.layers.attention import store_kvcache

pytestmark = pytest.mark.gpu
SCALE = 128 ** -0.5
F16 = torch.float16
FP8 = torch.float8_e4m3fn


def test_store_all_fp16_patterns_byte_exact():
    """All 65,536 fp16 bit patterns (K, and reversed as V) against the oracle's
    E4M3FN encoding of their values; NaN inputs must give NaN codes."""
    announce("fp16: store of all 65536 fp16 patterns")
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    key = torch.from_numpy(bits.view(np.int16).copy()).view(F16).reshape(512, 1, 128).cuda()
    value = key.flip(0).contiguous()
    kc = torch.zeros(2, 256, 1, 128, dtype=torch.uint8, device="cuda").view(FP8)
    vc = torch.zeros_like(kc)
    store_kvcache(key, value, kc, vc, torch.arange(512, dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    f = bits.view(np.float16).astype(np.float32)
    want = ofp8.e4m3_encode(f)
    nan = np.isnan(f)
    got_k = kc.view(torch.uint8).cpu().numpy().reshape(-1)
    got_v = vc.view(torch.uint8).cpu().numpy().reshape(-1)[::-1].reshape(512, 128)[:, ::-1].reshape(-1)
    for got in (got_k, got_v):
        mism = np.nonzero((got != want) & ~nan)[0]
        assert mism.size == 0, (f"{mism.size} mismatches, first fp16 0x{int(bits[mism[0]]):04x}: "
                                f"got 0x{got[mism[0]]:02x} want 0x{want[mism[0]]:02x}")
        assert np.all((got[nan] & 0x7F) == 0x7F), "NaN inputs must give NaN codes"


def test_store_fp16_strided_rows_and_padding():
    announce("fp16: store of strided fused-qkv rows with -1 slots")
    torch.manual_seed(1)
    N, Hq, Hkv, D, P, bs = 45, 16, 8, 128, 6, 256
    qkv = (torch.randn(N, (Hq + 2 * Hkv) * D, device="cuda") * 30).to(F16)
    k = qkv[:, Hq * D:(Hq + Hkv) * D].view(N, Hkv, D)
    v = qkv[:, (Hq + Hkv) * D:].view(N, Hkv, D)
    kc = torch.full((P, bs, Hkv, D), 0xAB, dtype=torch.uint8, device="cuda").view(FP8)
    vc = torch.full((P, bs, Hkv, D), 0xCD, dtype=torch.uint8, device="cuda").view(FP8)
    slots = torch.randperm(P * bs)[:N].to(torch.int32)
    slots[::4] = -1
    store_kvcache(k, v, kc, vc, slots.cuda())
    kc_ref = torch.full((P, bs, Hkv, D), 0xAB, dtype=torch.uint8)
    vc_ref = torch.full((P, bs, Hkv, D), 0xCD, dtype=torch.uint8)
    ofp8.store_kvcache(k.cpu(), v.cpu(), kc_ref, vc_ref, slots)
    assert torch.equal(kc.view(torch.uint8).cpu(), kc_ref)
    assert torch.equal(vc.view(torch.uint8).cpu(), vc_ref)


def test_store_rejects_mixed_dtypes():
    k = torch.zeros(2, 1, 128, dtype=F16, device="cuda")
    kc = torch.zeros(1, 16, 1, 128, dtype=torch.uint8, device="cuda").view(FP8)
    with pytest.raises(ValueError):
        store_kvcache(k, k.to(torch.bfloat16), kc, kc.clone(), torch.zeros(2, dtype=torch.int32, device="cuda"))


@pytest.mark.parametrize("make", [W.qwen3_0p6b_decode, W.tiny_decode])
def test_decode_fp16_matches_oracle(make):
    """The Qwen3-0.6B decode batch (B = 256, 16/8 heads: the balanced
    kernel) and the small case (4/2 heads: the split-KV kernel), K/V stored
    from fp16 values and fp16 queries; the output is fp16."""
    wl = make()
    announce(f"fp16: decode {wl.name}")
    cpu_c, gpu_c = build_pair(wl, gen_device="cuda", dtype=F16)
    q = wl.make_q("cpu", dtype=F16)
    bt = torch.from_numpy(wl.block_tables)
    ctx = torch.from_numpy(wl.context_lens())
    out = fp8_decode_attention(q.cuda(), gpu_c[0], gpu_c[1], bt.cuda(), ctx.cuda(), SCALE)
    torch.cuda.synchronize()
    assert out.dtype == F16
    want = oa.decode_attention(q, cpu_c[0], cpu_c[1], bt, ctx, SCALE)
    assert want.dtype == F16
    assert_close(out, want, wl.name)


def test_decode_fp16_agrees_with_bf16_on_exact_inputs():
    """Queries whose values are exact in both types (integers times 2^-4)
    and the same cache: the fp16 and bf16 calls compute the same products
    (the MFMAs' fp32 sums may round differently), so the bf16 rounding of the
    fp16 output is within a bf16 ulp of the bf16 output."""
    wl = W.qwen3_0p6b_decode(B=32)
    announce("fp16: decode fp16 vs bf16 on exactly representable queries")
    _, gpu_c = build_pair(wl, gen_device="cuda")
    g = torch.Generator().manual_seed(5)
    q = (torch.randint(-48, 49, (wl.num_q_tokens(), wl.num_heads, 128), generator=g).float() / 16)
    bt = torch.from_numpy(wl.block_tables).cuda()
    ctx = torch.from_numpy(wl.context_lens()).cuda()
    o16 = fp8_decode_attention(q.to(F16).cuda(), gpu_c[0], gpu_c[1], bt, ctx, SCALE)
    ob = fp8_decode_attention(q.to(torch.bfloat16).cuda(), gpu_c[0], gpu_c[1], bt, ctx, SCALE)
    torch.cuda.synchronize()
    assert_close(o16.to(torch.bfloat16), ob, "fp16 vs bf16 queries", atol=1e-3, rtol=8e-3)


def _prefill(wl, gpu_c, q, paged=True, kv=None):
    cu_q, cu_k = wl.cu_seqlens()
    kw = dict(cu_seqlens_q=torch.from_numpy(cu_q).cuda(), cu_seqlens_k=torch.from_numpy(cu_k).cuda(),
              max_seqlen_q=int(wl.lq().max()), max_seqlen_k=int(wl.lk().max()), softmax_scale=SCALE)
    if paged:
        out = fp8_prefill_attention(q, gpu_c[0], gpu_c[1], block_tables=torch.from_numpy(wl.block_tables).cuda(), **kw)
    else:
        out = fp8_prefill_attention(q, kv[0], kv[1], block_tables=None, **kw)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("hq,hkv", [(32, 8), (16, 2)])
def test_prefill_fp16_ragged(hq, hkv):
    """Ragged query lengths (short-query rows on the balanced kernel at 32/8
    and on the split-KV kernel at 16/2, the rest on the MFMA prefill
    kernel), paged, against the oracle; then the same rows in the contiguous
    layout."""
    rng = np.random.default_rng(hq + 11 * hkv)
    lqs = [1, 2, 3, 5, 9, 17, 33, 64, 129, 300, 700]
    seqs = [W.SeqSpec(lq=int(l), cached=int(rng.integers(0, 900))) for l in lqs]
    wl = W.make_workload(f"ragged_fp16_{hq}_{hkv}", hq, hkv, seqs, seed=int(rng.integers(1 << 30)))
    announce(f"fp16: prefill ragged {hq}/{hkv}, paged and contiguous")
    cpu_c, gpu_c = build_pair(wl, dtype=F16)
    q = wl.make_q("cpu", dtype=F16)
    cu_q, cu_k = wl.cu_seqlens()
    out = _prefill(wl, gpu_c, q.cuda())
    assert out.dtype == F16
    want = oa.prefill_attention(q, cpu_c[0], cpu_c[1], torch.from_numpy(wl.block_tables), torch.from_numpy(cu_q),
                                torch.from_numpy(cu_k), SCALE)
    assert want.dtype == F16
    assert_close(out, want, wl.name)
    rows = np.concatenate([wl.slots_for(i, 0, s.lk) for i, s in enumerate(wl.seqs)]).astype(np.int64)
    idx = torch.from_numpy(rows).cuda()
    kcont = gpu_c[0].view(torch.uint8).reshape(-1, hkv, 128)[idx].view(FP8)
    vcont = gpu_c[1].view(torch.uint8).reshape(-1, hkv, 128)[idx].view(FP8)
    out_c = _prefill(wl, gpu_c, q.cuda(), paged=False, kv=(kcont, vcont))
    want_c = oa.prefill_attention(q, kcont.cpu(), vcont.cpu(), None, torch.from_numpy(cu_q), torch.from_numpy(cu_k),
                                  SCALE)
    assert_close(out_c, want_c, wl.name + " contiguous")


def test_prefill_fp16_split_pieces_and_small_blocks():
    """A call with few items (a 2048-token prompt split into key-range pieces
    merged by the last piece) at block size 16 (the small-block kernel), and
    the mixed batch's speculative rows + chunks at block size 256."""
    seqs = [W.SeqSpec(lq=2048, cached=0), W.SeqSpec(lq=700, cached=1000), W.SeqSpec(lq=3, cached=90)]
    for wl in (W.make_workload("split_fp16_bs16", 32, 8, seqs, seed=21, block_size=16),
               W.sub_workload(W.qwen3_8b_mixed(), range(192, 227), name="mixed_varlen_fp16")):
        announce(f"fp16: prefill {wl.name}")
        cpu_c, gpu_c = build_pair(wl, dtype=F16)
        q = wl.make_q("cpu", dtype=F16)
        cu_q, cu_k = wl.cu_seqlens()
        out = _prefill(wl, gpu_c, q.cuda())
        want = oa.prefill_attention(q, cpu_c[0], cpu_c[1], torch.from_numpy(wl.block_tables),
                                    torch.from_numpy(cu_q), torch.from_numpy(cu_k), SCALE)
        assert_close(out, want, wl.name)
