"""Balanced (stream-K) decode on the GPU: the default decode path when the kv
heads split into groups of 4.  Checked against the oracle on ragged batches
(empty, 1-token and stage-boundary contexts, batches past one 256-sequence
prefix chunk, one and two query-column blocks) and, at sizes the oracle is
too slow for, against the split-KV kernel (explicit partitions), which the
oracle pins at smaller sizes."""
import numpy as np
import pytest
import torch

from gpu_util import announce, assert_close, build_pair
from oracle import attention as oa
from nanovllm_amd import _native
import workloads as W
from nanovllm_amd.kernels.fp8_attention import fp8_decode_attention

pytestmark = pytest.mark.gpu
SCALE = 128 ** -0.5


def _decode_capi(q, kc, vc, bt, ctx, hkv, block_size, part_tokens):
    lib = _native.load()
    B, Hq = q.shape[0], q.shape[1]
    nb = bt.shape[1]
    ws_bytes = lib.nvamd_decode_workspace_bytes(B, Hq, hkv, nb, block_size, part_tokens)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    out = torch.empty_like(q)
    st = lib.nvamd_fp8_decode_attention(out.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(), bt.data_ptr(),
                                        ctx.data_ptr(), B, Hq, hkv, 128, kc.shape[0], block_size, nb, SCALE,
                                        part_tokens, ws.data_ptr(), ws_bytes, 0,
                                        torch.cuda.current_stream().cuda_stream)
    _native.check(st, "decode")
    torch.cuda.synchronize()
    return out


def _oracle(wl, cpu_c, q, ctx=None):
    ctx = torch.from_numpy(wl.context_lens()) if ctx is None else ctx
    return oa.decode_attention(q, cpu_c[0], cpu_c[1], torch.from_numpy(wl.block_tables), ctx, SCALE)


@pytest.mark.parametrize("hq,hkv,bs", [(4, 4, 256), (16, 8, 256), (32, 8, 64), (24, 8, 128), (256, 8, 256),
                                       (32, 8, 16), (64, 8, 32), (16, 4, 16), (32, 8, 48)])
def test_balanced_decode_ragged_batch(hq, hkv, bs):
    """Contexts 1..2000 around stage (16) and block boundaries, in random order."""
    rng = np.random.default_rng(hq * 7 + hkv + bs)
    edge = [1, 2, 15, 16, 17, 31, 32, 33, bs - 1, bs, bs + 1, 2 * bs + 16, 1000, 2000]
    ctx = list(rng.permutation(edge + [int(c) for c in rng.integers(1, 2000, size=26)]))
    seqs = [W.SeqSpec(lq=1, cached=int(c) - 1) for c in ctx]
    wl = W.make_workload(f"bal_{hq}_{hkv}_{bs}", hq, hkv, seqs, seed=int(rng.integers(1 << 30)), block_size=bs)
    announce(f"balanced decode: ragged {hq}/{hkv} bs={bs} B={len(seqs)}")
    cpu_c, gpu_c = build_pair(wl)
    q = wl.make_q("cpu")
    bt = torch.from_numpy(wl.block_tables).cuda()
    ctx_t = torch.from_numpy(wl.context_lens()).cuda()
    out = fp8_decode_attention(q.cuda(), gpu_c[0], gpu_c[1], bt, ctx_t, SCALE)
    torch.cuda.synchronize()
    assert_close(out, _oracle(wl, cpu_c, q), wl.name)


def test_balanced_decode_big_batch_with_empty_rows():
    """B = 600 (three prefix chunks); every 7th row has an empty context."""
    wl = W.decode_workload("bal_b600", 600, 16, 8, 1, 300, seed=5)
    announce("balanced decode: B=600 with empty rows")
    cpu_c, gpu_c = build_pair(wl)
    q = wl.make_q("cpu")
    bt = torch.from_numpy(wl.block_tables).cuda()
    ctx = torch.from_numpy(wl.context_lens()).clone()
    ctx[::7] = 0
    out = fp8_decode_attention(q.cuda(), gpu_c[0], gpu_c[1], bt, ctx.cuda(), SCALE).cpu()
    assert bool((out[::7] == 0).all()), "empty-context rows must be 0"
    keep = torch.ones(600, dtype=torch.bool)
    keep[::7] = False
    assert_close(out, _oracle(wl, cpu_c, q, ctx), "bal_b600", mask_rows=keep)


def test_balanced_decode_all_empty():
    wl = W.decode_workload("bal_empty", 8, 16, 8, 1, 50, seed=6)
    announce("balanced decode: all contexts empty")
    _, gpu_c = build_pair(wl)
    q = wl.make_q("cuda")
    bt = torch.from_numpy(wl.block_tables).cuda()
    out = fp8_decode_attention(q, gpu_c[0], gpu_c[1], bt, torch.zeros(8, dtype=torch.int32, device="cuda"), SCALE)
    torch.cuda.synchronize()
    assert bool((out == 0).all())


def test_balanced_decode_matches_split_kv_on_long_segments():
    """8 sequences of ~800K tokens with 64-token blocks: each workgroup's
    range spans more than the 64-entry block-table window, so the window is
    reloaded inside a pair.  Compared with the split-KV kernel (explicit
    3840-token partitions) on the same cache."""
    B, hkv, hq, bs = 8, 4, 4, 64
    rng = np.random.default_rng(9)
    ctx = rng.integers(780_000, 800_000, size=B).astype(np.int32)
    nblk = (ctx + bs - 1) // bs
    pool = int(nblk.sum())
    perm = rng.permutation(pool).astype(np.int32)
    bt = np.full((B, int(nblk.max())), -1, dtype=np.int32)
    o = 0
    for b in range(B):
        bt[b, :nblk[b]] = perm[o:o + nblk[b]]
        o += nblk[b]
    announce(f"balanced decode: long segments, KV pool {2 * pool * bs * hkv * 128 / 2**30:.1f} GiB")
    g = torch.Generator(device="cuda").manual_seed(3)
    # random E4M3 bytes without the NaN codes (0x7F, 0xFF)
    kc = torch.randint(0, 0x7F, (pool, bs, hkv, 128), dtype=torch.uint8, device="cuda", generator=g)
    vc = torch.randint(0, 0x7F, (pool, bs, hkv, 128), dtype=torch.uint8, device="cuda", generator=g)
    kc |= (torch.randint(0, 2, kc.shape, dtype=torch.uint8, device="cuda", generator=g) << 7)
    vc |= (torch.randint(0, 2, vc.shape, dtype=torch.uint8, device="cuda", generator=g) << 7)
    q = torch.randn(B, hq, 128, device="cuda", generator=g).to(torch.bfloat16)
    bt_g = torch.from_numpy(bt).cuda()
    ctx_g = torch.from_numpy(ctx).cuda()
    kc8, vc8 = kc.view(torch.float8_e4m3fn), vc.view(torch.float8_e4m3fn)
    bal = _decode_capi(q, kc8, vc8, bt_g, ctx_g, hkv, bs, 0)
    ref = _decode_capi(q, kc8, vc8, bt_g, ctx_g, hkv, bs, 3840)
    assert_close(bal, ref, "long_segments")


def test_balanced_decode_workspace_is_required():
    lib = _native.load()
    need = lib.nvamd_decode_workspace_bytes(4, 16, 8, 8, 256, 0)
    assert need > 0
    wl = W.decode_workload("bal_ws", 4, 16, 8, 10, 2000, seed=8)
    _, gpu_c = build_pair(wl)
    q = wl.make_q("cuda")
    bt = torch.from_numpy(wl.block_tables).cuda()
    ctx = torch.from_numpy(wl.context_lens()).cuda()
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    out = torch.empty_like(q)
    st = lib.nvamd_fp8_decode_attention(out.data_ptr(), q.data_ptr(), gpu_c[0].data_ptr(), gpu_c[1].data_ptr(),
                                        bt.data_ptr(), ctx.data_ptr(), 4, 16, 8, 128, wl.num_blocks, 256,
                                        bt.shape[1], SCALE, 0, ws.data_ptr(), need - 1, 0,
                                        torch.cuda.current_stream().cuda_stream)
    assert st != 0 and b"workspace" in lib.nvamd_last_error()


def test_balanced_decode_garbage_and_reused_workspace():
    """The workspace needs no initialisation: random bytes in it (including
    the arrival words of cut pairs) and reuse across calls give the same
    result as the oracle."""
    wl = W.decode_workload("bal_ws_garbage", 96, 16, 8, 1, 3000, seed=12)
    announce("balanced decode: garbage / reused workspace")
    cpu_c, gpu_c = build_pair(wl)
    q = wl.make_q("cpu")
    qg = q.cuda()
    bt = torch.from_numpy(wl.block_tables).cuda()
    ctx = torch.from_numpy(wl.context_lens()).cuda()
    lib = _native.load()
    nb = bt.shape[1]
    need = lib.nvamd_decode_workspace_bytes(96, 16, 8, nb, 256, 0)
    ws = torch.randint(0, 256, (need,), dtype=torch.uint8, device="cuda")
    want = _oracle(wl, cpu_c, q)
    for call in range(3):
        out = torch.empty_like(qg)
        st = lib.nvamd_fp8_decode_attention(out.data_ptr(), qg.data_ptr(), gpu_c[0].data_ptr(), gpu_c[1].data_ptr(),
                                            bt.data_ptr(), ctx.data_ptr(), 96, 16, 8, 128, wl.num_blocks, 256, nb,
                                            SCALE, 0, ws.data_ptr(), need, 0, torch.cuda.current_stream().cuda_stream)
        _native.check(st, "decode")
        torch.cuda.synchronize()
        assert_close(out, want, f"garbage_ws call {call}")
