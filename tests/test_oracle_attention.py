"""Pins the oracle's paged decode / varlen prefill (nanovllm/kernels/fp8_attention.py).

Known answers (one key -> V_0, constant V -> V, q = 0 -> mean of V), an
fp64 brute-force softmax written per (row, key) with Python loops on tiny
inputs, invariances (block-id permutation, chunking, paged == contiguous,
Lq = 1 prefill == decode), the bottom-right causal alignment, the
fp32 -> fp16 -> bf16 output rounding, and the log-sum-exp merge used by the
split-KV reduction.
"""
import math

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import fp8

D = 128


def _cache_from_codes(rng, P, bs, Hkv):
    """Random finite E4M3 codes (no NaN codes)."""
    codes = rng.integers(0, 256, size=(P, bs, Hkv, D), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x00
    return torch.from_numpy(codes)


def _q(rng, n, H):
    return torch.from_numpy(rng.standard_normal((n, H, D)).astype(np.float32)).to(torch.bfloat16)


def _bt(rng, B, nb, P):
    ids = rng.permutation(P)[:B * nb].reshape(B, nb)
    return torch.from_numpy(ids.astype(np.int32))


def test_single_key_returns_v0():
    rng = np.random.default_rng(0)
    kc, vc = _cache_from_codes(rng, 4, 64, 2), _cache_from_codes(rng, 4, 64, 2)
    q = _q(rng, 1, 4)
    bt = torch.tensor([[2, 0]], dtype=torch.int32)
    out = oa.decode_attention(q, kc, vc, bt, torch.tensor([1], dtype=torch.int32), 0.088,
                              return_fp32=True)
    v0 = fp8.dequant_codes_tensor(vc[2, 0])  # [Hkv, D]
    assert torch.equal(out[0, :2], v0[0].expand(2, D).to(out.dtype))
    assert torch.equal(out[0, 2:], v0[1].expand(2, D).to(out.dtype))


def test_constant_v_and_zero_q():
    rng = np.random.default_rng(1)
    P, bs, Hkv = 6, 64, 1
    kc = _cache_from_codes(rng, P, bs, Hkv)
    vc = torch.full((P, bs, Hkv, D), 0x3C, dtype=torch.uint8)  # 1.5
    q = _q(rng, 2, 2)
    bt = _bt(rng, 2, 3, P)
    ctx = torch.tensor([150, 17], dtype=torch.int32)
    out = oa.decode_attention(q, kc, vc, bt, ctx, 0.1)
    assert bool((out.float() == 1.5).all())
    # q = 0: uniform softmax -> mean of V over the context
    vc = _cache_from_codes(rng, P, bs, Hkv)
    q0 = torch.zeros(2, 2, D, dtype=torch.bfloat16)
    out = oa.decode_attention(q0, kc, vc, bt, ctx, 0.1, compute_dtype=torch.float64, return_fp32=True)
    for b in range(2):
        n = int(ctx[b])
        rows = torch.cat([fp8.dequant_codes_tensor(vc[int(bt[b, i])]) for i in range(3)])[:n, 0]
        assert torch.allclose(out[b, 0], rows.double().mean(0), atol=1e-12)


def _brute_force(q, K, V, scale, limits):
    """Per-row, per-key fp64 softmax with explicit loops (tiny inputs only)."""
    R, L = q.shape[0], K.shape[0]
    out = np.zeros((R, V.shape[1]))
    for r in range(R):
        s = [sum(float(q[r, d]) * float(K[j, d]) for d in range(q.shape[1])) * scale
             for j in range(limits[r])]
        m = max(s)
        w = [math.exp(x - m) for x in s]
        tot = sum(w)
        for j in range(limits[r]):
            out[r] += w[j] / tot * V[j].numpy().astype(np.float64)
    return out


def test_decode_matches_brute_force():
    rng = np.random.default_rng(2)
    P, bs, Hkv, Hq = 5, 64, 2, 4
    kc, vc = _cache_from_codes(rng, P, bs, Hkv), _cache_from_codes(rng, P, bs, Hkv)
    q = _q(rng, 2, Hq)
    bt = torch.tensor([[4, 1, 0], [2, 3, 0]], dtype=torch.int32)
    ctx = torch.tensor([130, 7], dtype=torch.int32)
    out = oa.decode_attention(q, kc, vc, bt, ctx, 0.0883, compute_dtype=torch.float64, return_fp32=True)
    for b in range(2):
        n = int(ctx[b])
        for g in range(Hkv):
            K = torch.cat([fp8.dequant_codes_tensor(kc[int(bt[b, i]), :, g]) for i in range(3)])[:n]
            V = torch.cat([fp8.dequant_codes_tensor(vc[int(bt[b, i]), :, g]) for i in range(3)])[:n]
            ref = _brute_force(q[b, 2 * g:2 * g + 2].float(), K, V, 0.0883, [n, n])
            assert np.allclose(out[b, 2 * g:2 * g + 2].numpy(), ref, atol=1e-9)


def test_fp32_oracle_close_to_fp64():
    rng = np.random.default_rng(3)
    P, bs, Hkv, Hq = 12, 64, 2, 8
    kc, vc = _cache_from_codes(rng, P, bs, Hkv), _cache_from_codes(rng, P, bs, Hkv)
    q = _q(rng, 3, Hq)
    bt = _bt(rng, 3, 4, P)
    ctx = torch.tensor([256, 1, 199], dtype=torch.int32)
    a = oa.decode_attention(q, kc, vc, bt, ctx, 0.0883, return_fp32=True)
    b = oa.decode_attention(q, kc, vc, bt, ctx, 0.0883, compute_dtype=torch.float64, return_fp32=True)
    assert torch.allclose(a.double(), b, atol=1e-4, rtol=1e-4)


def test_block_permutation_invariance():
    rng = np.random.default_rng(4)
    P, bs, Hkv, Hq = 8, 64, 1, 2
    kc, vc = _cache_from_codes(rng, P, bs, Hkv), _cache_from_codes(rng, P, bs, Hkv)
    q = _q(rng, 1, Hq)
    bt = torch.tensor([[5, 2, 7]], dtype=torch.int32)
    ctx = torch.tensor([170], dtype=torch.int32)
    base = oa.decode_attention(q, kc, vc, bt, ctx, 0.1, compute_dtype=torch.float64, return_fp32=True)
    perm = torch.from_numpy(rng.permutation(P))
    inv = torch.argsort(perm)
    kc2, vc2 = kc[perm], vc[perm]                  # block b now lives at inv[b]
    bt2 = inv[bt.long()].to(torch.int32)
    got = oa.decode_attention(q, kc2, vc2, bt2, ctx, 0.1, compute_dtype=torch.float64, return_fp32=True)
    assert torch.allclose(base, got, atol=1e-12)


def _paged_case(rng, lens_q, lens_k, Hq, Hkv, bs=64):
    nbs = [-(-lk // bs) for lk in lens_k]
    P = sum(nbs) + 3
    kc, vc = _cache_from_codes(rng, P, bs, Hkv), _cache_from_codes(rng, P, bs, Hkv)
    ids = rng.permutation(P)
    bt = torch.full((len(lens_k), max(nbs)), -1, dtype=torch.int32)
    o = 0
    for i, n in enumerate(nbs):
        bt[i, :n] = torch.from_numpy(ids[o:o + n].astype(np.int32))
        o += n
    q = _q(rng, sum(lens_q), Hq)
    cu_q = torch.tensor(np.concatenate([[0], np.cumsum(lens_q)]), dtype=torch.int32)
    cu_k = torch.tensor(np.concatenate([[0], np.cumsum(lens_k)]), dtype=torch.int32)
    return q, kc, vc, bt, cu_q, cu_k


def _gather_contig(kc, bt, lens_k):
    bs = kc.shape[1]
    rows = []
    for i, lk in enumerate(lens_k):
        nb = -(-lk // bs)
        rows.append(kc[bt[i, :nb].long()].reshape(nb * bs, kc.shape[2], D)[:lk])
    return torch.cat(rows)


def test_prefill_causal_alignment_brute_force():
    rng = np.random.default_rng(5)
    lens_q, lens_k = [3, 1], [7, 4]
    q, kc, vc, bt, cu_q, cu_k = _paged_case(rng, lens_q, lens_k, 2, 1)
    out = oa.prefill_attention(q, kc, vc, bt, cu_q, cu_k, 0.09, compute_dtype=torch.float64,
                               return_fp32=True)
    K = _gather_contig(kc, bt, lens_k)
    V = _gather_contig(vc, bt, lens_k)
    for s in range(2):
        q0, k0 = int(cu_q[s]), int(cu_k[s])
        Lq, Lk = lens_q[s], lens_k[s]
        limits = [i + (Lk - Lq) + 1 for i in range(Lq)]   # row i sees j <= i + Lk - Lq
        for h in range(2):
            ref = _brute_force(q[q0:q0 + Lq, h].float(), fp8.dequant_codes_tensor(K[k0:k0 + Lk, 0]),
                               fp8.dequant_codes_tensor(V[k0:k0 + Lk, 0]), 0.09, limits)
            assert np.allclose(out[q0:q0 + Lq, h].numpy(), ref, atol=1e-9)


def test_paged_equals_contiguous_and_lq1_equals_decode():
    rng = np.random.default_rng(6)
    lens_q, lens_k = [5, 1, 40, 1], [70, 129, 40, 1]
    q, kc, vc, bt, cu_q, cu_k = _paged_case(rng, lens_q, lens_k, 4, 2)
    paged = oa.prefill_attention(q, kc, vc, bt, cu_q, cu_k, 0.0883, return_fp32=True)
    kcont, vcont = _gather_contig(kc, bt, lens_k), _gather_contig(vc, bt, lens_k)
    contig = oa.prefill_attention(q, kcont, vcont, None, cu_q, cu_k, 0.0883, return_fp32=True)
    assert torch.allclose(paged, contig, atol=1e-6)
    # the Lq == 1 sequences equal single-query decode at context Lk
    for s in (1, 3):
        row = int(cu_q[s])
        dec = oa.decode_attention(q[row:row + 1], kc, vc, bt[s:s + 1], torch.tensor([lens_k[s]]),
                                  0.0883, return_fp32=True)
        assert torch.allclose(paged[row], dec[0], atol=1e-6)


def test_chunked_prefill_matches_full_prefill():
    rng = np.random.default_rng(7)
    L, split = 90, 57
    q, kc, vc, bt, cu_q, cu_k = _paged_case(rng, [L], [L], 4, 1)
    full = oa.prefill_attention(q, kc, vc, bt, cu_q, cu_k, 0.0883, return_fp32=True)
    # second chunk alone: rows [split, L) with split tokens already cached
    chunk = oa.prefill_attention(q[split:], kc, vc, bt, torch.tensor([0, L - split]),
                                 torch.tensor([0, L]), 0.0883, return_fp32=True)
    assert torch.allclose(full[split:], chunk, atol=1e-6)


def test_output_double_rounding():
    # x just below a bf16 midpoint: fp16 rounds it onto the midpoint, which then
    # ties to the even bf16 neighbour above, while a direct cast rounds down.
    x = torch.tensor([1.0 + 3 * 2 ** -8 - 2 ** -12], dtype=torch.float32)
    direct = x.to(torch.bfloat16)
    double = oa.round_output(x)
    assert float(direct) != float(double)
    assert float(double) == float(x.to(torch.float16).to(torch.bfloat16))
    # and the decode oracle applies it: 3 keys, q = 0 -> mean of V
    rng = np.random.default_rng(8)
    kc = _cache_from_codes(rng, 1, 64, 1)
    vc = torch.zeros(1, 64, 1, D, dtype=torch.uint8)
    vc[0, :3, 0, :] = torch.tensor([0x38, 0x39, 0x3B], dtype=torch.uint8).view(3, 1)  # 1, 1.125, 1.375
    out = oa.decode_attention(torch.zeros(1, 1, D, dtype=torch.bfloat16), kc, vc,
                              torch.tensor([[0]], dtype=torch.int32), torch.tensor([3]), 0.1)
    mean = torch.tensor([(1 + 1.125 + 1.375) / 3], dtype=torch.float32)
    assert float(out[0, 0, 0]) == float(oa.round_output(mean))


def test_log_sum_exp_merge_identity():
    """Splitting the keys into partitions and merging (m, l, acc) with
    exp(m_p - M) weights reproduces the unsplit softmax (split-KV reduce)."""
    rng = np.random.default_rng(9)
    s = rng.standard_normal(300) * 4
    V = rng.standard_normal((300, 8))
    full = np.exp(s - s.max()) @ V / np.exp(s - s.max()).sum()
    parts = [(0, 64), (64, 256), (256, 300)]
    ms, ls, accs = [], [], []
    for a, b in parts:
        m = s[a:b].max()
        w = np.exp(s[a:b] - m)
        ms.append(m); ls.append(w.sum()); accs.append(w @ V[a:b])
    M = max(ms)
    L = sum(l * np.exp(m - M) for m, l in zip(ms, ls))
    merged = sum(acc * np.exp(m - M) for m, acc in zip(ms, accs)) / L
    assert np.allclose(merged, full, atol=1e-12)


def test_zero_context_decode_is_nan_like_reference():
    rng = np.random.default_rng(10)
    kc, vc = _cache_from_codes(rng, 2, 64, 1), _cache_from_codes(rng, 2, 64, 1)
    out = oa.decode_attention(_q(rng, 1, 1), kc, vc, torch.tensor([[0]], dtype=torch.int32),
                              torch.tensor([0]), 0.1)
    assert bool(torch.isnan(out.float()).all())
