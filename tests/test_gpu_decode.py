"""Paged FP8 decode on the GPU vs the oracle (atol/rtol 1e-2, bf16 output)."""
import numpy as np
import pytest
import torch

from gpu_util import announce, assert_close, build_pair
from oracle import attention as oa
from oracle import fp8 as ofp8
from nanovllm_amd import _native
import workloads as W
from nanovllm_amd.kernels.fp8_attention import fp8_decode_attention
from nanovllm_amd.layers.attention import store_kvcache

pytestmark = pytest.mark.gpu
SCALE = 128 ** -0.5


def _run_decode(wl, gpu_caches, q_gpu):
    bt = torch.from_numpy(wl.block_tables).cuda()
    ctx = torch.from_numpy(wl.context_lens()).cuda()
    out = fp8_decode_attention(q_gpu, gpu_caches[0], gpu_caches[1], bt, ctx, SCALE)
    torch.cuda.synchronize()
    return out


def _oracle_decode(wl, cpu_caches, q_cpu):
    return oa.decode_attention(q_cpu, cpu_caches[0], cpu_caches[1], torch.from_numpy(wl.block_tables),
                               torch.from_numpy(wl.context_lens()), SCALE)


@pytest.mark.parametrize("make", [W.tiny_decode, W.qwen3_0p6b_decode, W.qwen3_8b_decode])
def test_decode_matches_oracle(make):
    """The small CPU case, the Qwen3-0.6B decode batch (B = 256, 16/8 heads) and
    the mixed batch's 192 plain-decode rows at Qwen3-8B shapes (32/8 heads, ctx
    U[256, 4096]), all rows and heads against the oracle."""
    wl = make()
    announce(f"decode: {wl.name}")
    cpu_c, gpu_c = build_pair(wl, gen_device="cuda")
    q = wl.make_q("cpu")
    out = _run_decode(wl, gpu_c, q.cuda())
    assert_close(out, _oracle_decode(wl, cpu_c, q), wl.name)


@pytest.mark.parametrize("hq,hkv", [(4, 4), (16, 8), (32, 8), (64, 8), (32, 2), (64, 2), (24, 8)])
def test_decode_gqa_ratios(hq, hkv):
    rng = np.random.default_rng(hq * 100 + hkv)
    ctx = [1, 31, 32, 33, 255, 256, 257, 700, 1500]
    seqs = [W.SeqSpec(lq=1, cached=c - 1) for c in ctx]
    wl = W.make_workload(f"gqa_{hq}_{hkv}", hq, hkv, seqs, seed=int(rng.integers(1 << 30)))
    announce(f"decode: GQA {hq}/{hkv}")
    cpu_c, gpu_c = build_pair(wl)
    q = wl.make_q("cpu")
    out = _run_decode(wl, gpu_c, q.cuda())
    assert_close(out, _oracle_decode(wl, cpu_c, q), wl.name)


def test_decode_single_key_returns_v0_for_every_code():
    """ctx = 1: out = bf16(fp16(V_0)) = V_0 exactly, for all finite E4M3 codes."""
    announce("decode: ctx=1 exhaustive dequant")
    Hkv, Hq, bs = 2, 4, 256
    codes = np.arange(256, dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0
    vc = torch.zeros(1, bs, Hkv, 128, dtype=torch.uint8)
    vc[0, 0] = torch.from_numpy(codes.reshape(Hkv, 128))
    kc = torch.randint(0, 0x70, (1, bs, Hkv, 128), dtype=torch.uint8)
    q = torch.randn(1, Hq, 128).to(torch.bfloat16)
    out = fp8_decode_attention(q.cuda(), kc.cuda().view(torch.float8_e4m3fn), vc.cuda().view(torch.float8_e4m3fn),
                               torch.zeros(1, 1, dtype=torch.int32, device="cuda"),
                               torch.ones(1, dtype=torch.int32, device="cuda"), SCALE).cpu()
    want = ofp8.dequant_codes_tensor(vc[0, 0])          # [Hkv, 128] exact values
    for h in range(Hq):
        assert torch.equal(out[0, h].float(), want[h // 2]), f"head {h}"


def test_decode_zero_context_rows_are_zero():
    announce("decode: ctx=0 rows")
    wl = W.tiny_decode()
    cpu_c, gpu_c = build_pair(wl)
    q = wl.make_q("cpu").cuda()
    bt = torch.from_numpy(wl.block_tables).cuda()
    ctx = torch.from_numpy(wl.context_lens()).cuda()
    ctx[1] = 0
    out = fp8_decode_attention(q, gpu_c[0], gpu_c[1], bt, ctx, SCALE).cpu()
    assert bool((out[1] == 0).all())
    want = oa.decode_attention(q.cpu(), cpu_c[0], cpu_c[1], bt.cpu(), ctx.cpu(), SCALE)
    keep = torch.tensor([True, False, True, True])
    assert_close(out, want, "ctx0", mask_rows=keep)


@pytest.mark.parametrize("part_tokens", [256, 512, 1024])
def test_decode_forced_split_kv(part_tokens):
    """Explicit partition sizes through the C ABI: split + reduce == oracle."""
    wl = W.qwen3_0p6b_decode(B=48)
    announce(f"decode: forced split part_tokens={part_tokens}")
    cpu_c, gpu_c = build_pair(wl)
    q = wl.make_q("cpu")
    qg = q.cuda()
    bt = torch.from_numpy(wl.block_tables).cuda()
    ctx = torch.from_numpy(wl.context_lens()).cuda()
    lib = _native.load()
    B, Hq = q.shape[0], wl.num_heads
    nb = bt.shape[1]
    ws_bytes = lib.nvamd_decode_workspace_bytes(B, Hq, wl.num_kv_heads, nb, 256, part_tokens)
    assert ws_bytes > 0
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    out = torch.empty_like(qg)
    st = lib.nvamd_fp8_decode_attention(out.data_ptr(), qg.data_ptr(), gpu_c[0].data_ptr(), gpu_c[1].data_ptr(),
                                        bt.data_ptr(), ctx.data_ptr(), B, Hq, wl.num_kv_heads, 128,
                                        wl.num_blocks, 256, nb, SCALE, part_tokens, ws.data_ptr(), ws_bytes, 0,
                                        torch.cuda.current_stream().cuda_stream)
    _native.check(st, "decode")
    torch.cuda.synchronize()
    assert_close(out, _oracle_decode(wl, cpu_c, q), f"split{part_tokens}")


def test_decode_long_context_big_pool():
    """Long contexts (split-KV) with block ids beyond the reference's int32 limit."""
    full = W.qwen3_32b_long_decode(B=4, ctx_lo=40000, ctx_hi=70000)
    announce("decode: long context, pool > 8192 blocks")
    # GPU pool: the workload's own (> 8192 blocks, ids spread over it)
    assert full.num_blocks > 8192 or full.block_tables.max() > 0
    big = W.make_workload("long_big_pool", 64, 8, full.seqs, seed=11, num_blocks=13000)
    assert int(big.block_tables.max()) >= 8192
    small = W.sub_workload(big, range(big.num_seqs), compact=True)
    # same K/V values: fill both through the same token order
    kc_cpu, vc_cpu = small.empty_caches("cpu")
    from gpu_util import cpu_store
    small.fill_cache(kc_cpu, vc_cpu, cpu_store)
    kc_gpu, vc_gpu = big.empty_caches("cuda")
    big.fill_cache(kc_gpu, vc_gpu, store_kvcache)
    q = big.make_q("cpu")
    out = _run_decode(big, (kc_gpu, vc_gpu), q.cuda())
    want = oa.decode_attention(q, kc_cpu, vc_cpu, torch.from_numpy(small.block_tables),
                               torch.from_numpy(small.context_lens()), SCALE)
    assert_close(out, want, "long_big_pool")


def test_decode_block_permutation_invariance():
    announce("decode: block permutation invariance")
    wl = W.qwen3_0p6b_decode(B=32)
    _, gpu_c = build_pair(wl)
    q = wl.make_q("cuda")
    out1 = _run_decode(wl, gpu_c, q)
    perm = torch.randperm(wl.num_blocks, device="cuda")
    inv = torch.argsort(perm)
    kc2, vc2 = gpu_c[0][perm].contiguous(), gpu_c[1][perm].contiguous()
    bt = torch.from_numpy(wl.block_tables).cuda().long()
    bt2 = torch.where(bt >= 0, inv[bt.clamp(min=0)], bt).to(torch.int32)
    ctx = torch.from_numpy(wl.context_lens()).cuda()
    out2 = fp8_decode_attention(q, kc2, vc2, bt2, ctx, SCALE)
    assert torch.equal(out1, out2)


def _forced_split_decode(wl, gpu_c, qg, part_tokens):
    bt = torch.from_numpy(wl.block_tables).cuda()
    ctx = torch.from_numpy(wl.context_lens()).cuda()
    lib = _native.load()
    B, Hq = qg.shape[0], wl.num_heads
    nb = bt.shape[1]
    ws_bytes = lib.nvamd_decode_workspace_bytes(B, Hq, wl.num_kv_heads, nb, wl.block_size, part_tokens)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    out = torch.empty_like(qg)
    st = lib.nvamd_fp8_decode_attention(out.data_ptr(), qg.data_ptr(), gpu_c[0].data_ptr(), gpu_c[1].data_ptr(),
                                        bt.data_ptr(), ctx.data_ptr(), B, Hq, wl.num_kv_heads, 128,
                                        wl.num_blocks, wl.block_size, nb, SCALE, part_tokens, ws.data_ptr(), ws_bytes, 0,
                                        torch.cuda.current_stream().cuda_stream)
    _native.check(st, "decode")
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("ctx_lo,ctx_hi", [(30, 500), (2000, 8000)])
def test_decode_outlier_kv(ctx_lo, ctx_hi):
    """Qwen3-32B head shapes with 1 % of the K/V entries scaled by 20 before
    quantisation (the long-decode configuration's outliers): peaked scores
    and large V values, through the balanced kernel and the split-KV kernel."""
    wl = W.decode_workload(f"decode_outliers_{ctx_lo}", 24, 64, 8, ctx_lo, ctx_hi, seed=31,
                           outlier_frac=0.01, outlier_scale=20.0)
    announce(f"decode: outlier K/V (1% x20), ctx U[{ctx_lo}, {ctx_hi}]")
    cpu_c, gpu_c = build_pair(wl)
    q = wl.make_q("cpu")
    want = _oracle_decode(wl, cpu_c, q)
    assert_close(_run_decode(wl, gpu_c, q.cuda()), want, "balanced decode, outliers")
    assert_close(_forced_split_decode(wl, gpu_c, q.cuda(), 256), want, "split-KV decode, outliers")


def test_decode_long_context_outliers_full_size():
    """The long-decode workload at full size: B = 32, 64/8 heads, ctx U[32K, 128K]
    (up to 130,832 keys), 1 % of the K/V entries x20 before quantisation, a
    pool of 13,673 blocks (past the reference's int32 offsets).  Every row of
    the balanced (stream-K) kernel is compared with the split-KV kernel
    (15,872-token partitions) on the same cache, and the shortest sequence,
    the longest and two more (all 64 heads) with the oracle on the same cache
    bytes (the blocks they use copied to the host)."""
    wl = W.qwen3_32b_long_decode()
    announce(f"decode: {wl.name} full size, B={wl.num_seqs}, max ctx {int(wl.context_lens().max())}")
    kc, vc = wl.empty_caches("cuda")
    wl.fill_cache(kc, vc, store_kvcache, gen_device="cuda")
    q = wl.make_q("cuda")
    bal = _run_decode(wl, (kc, vc), q)
    split = _forced_split_decode(wl, (kc, vc), q, 15872)
    assert_close(bal, split, "long decode: balanced vs split-KV")
    ctx = wl.context_lens()
    pick = sorted({int(ctx.argmin()), int(ctx.argmax()), 7, 19})
    sub = W.sub_workload(wl, pick, compact=True)
    bt = wl.block_tables[pick]
    used = torch.from_numpy(np.unique(bt[bt >= 0]).astype(np.int64)).cuda()
    kc_s, vc_s = kc[used].cpu(), vc[used].cpu()
    want = oa.decode_attention(q[pick].cpu(), kc_s, vc_s, torch.from_numpy(sub.block_tables),
                               torch.from_numpy(sub.context_lens()), SCALE)
    assert_close(bal[pick], want, f"long decode: sequences {pick} vs oracle")


@pytest.mark.parametrize("bs", [16, 32])
@pytest.mark.parametrize("hq,hkv,part", [(32, 8, 0), (32, 2, 0), (32, 8, 512)])
def test_decode_small_blocks(bs, hq, hkv, part):
    """Block sizes 16 and 32 (the reference accepts any kvcache_block_size
    % 16 == 0): the balanced kernel (32/8), the split-KV kernel chosen by the
    library (32/2) and forced 512-token partitions, whose 32- or 64-token
    stages then span several blocks."""
    rng = np.random.default_rng(bs * 10 + hkv + part)
    ctx = [1, 15, 16, 17, 31, 32, 33, 63, 64, 65, 300, 1000, 2500] + [int(c) for c in rng.integers(1, 3000, 10)]
    seqs = [W.SeqSpec(lq=1, cached=c - 1) for c in ctx]
    wl = W.make_workload(f"small_blocks_{bs}_{hq}_{hkv}", hq, hkv, seqs, seed=int(rng.integers(1 << 30)),
                         block_size=bs)
    announce(f"decode: block_size {bs}, {hq}/{hkv} heads, part_tokens {part}")
    cpu_c, gpu_c = build_pair(wl)
    q = wl.make_q("cpu")
    want = _oracle_decode(wl, cpu_c, q)
    out = _run_decode(wl, gpu_c, q.cuda()) if part == 0 else _forced_split_decode(wl, gpu_c, q.cuda(), part)
    assert_close(out, want, wl.name)
