"""Oracle: torch-CPU restatement of the FP8 paged attention (TEST INFRASTRUCTURE ONLY).

Follows the reference kernels' semantics, not their tiling:

* decode -- nanovllm/kernels/fp8_attention.py:88-207.  For sequence b and
  query head h (kv head h // (Hq // Hkv), :104-105) attend over the first
  ``context_lens[b]`` cached tokens, gathered through ``block_tables[b]``
  (token t lives at slot ``bt[b, t // bs] * bs + t % bs``, :127-142).
  Scores are ``(q . k) * softmax_scale`` (:153), softmax over the context,
  ``out = acc / max(s, 1e-10)`` cast to fp16 (:169) and stored into
  ``empty_like(q)`` (:193) -- i.e. fp32 -> fp16 -> bf16 for bf16 queries,
  fp32 -> fp16 for fp16 queries.
  ``context_lens[b] == 0`` yields NaN in the reference (exp(-inf - -inf));
  the oracle returns NaN there too and callers treat such rows as
  don't-care.
* prefill -- nanovllm/kernels/fp8_attention.py:209-353.  Sequence s owns q
  rows ``[cu_q[s], cu_q[s+1])`` and ``Lk = cu_k[s+1] - cu_k[s]`` keys; row i
  (0-based inside the sequence) sees key j iff ``j <= i + (Lk - Lq)``
  (bottom-right aligned causal mask, :237, :267, :297).  Keys come from the
  paged cache through ``block_tables[s]`` (:280-308) or, when
  ``block_tables is None``, from the contiguous ``k[cu_k[s] + j]`` (:254-278).
  Rows whose softmax denominator is 0 output 0 (:311); output is
  fp32 -> fp16 -> q's dtype (:311, :337).
* The FP8 cache is dequantised exactly (``.to(tl.float32)``; scale 1).

``compute_dtype`` selects float32 (the reference's accumulation type) or
float64 (used by the tests that pin the oracle itself).
"""
import torch

from . import fp8 as _fp8


def _as_codes(t):
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8)
    assert t.dtype == torch.uint8, t.dtype
    return t


def round_output(x, dtype=torch.bfloat16):
    """fp32 attention output -> fp16 -> the output dtype (q's: bf16 or fp16),
    as the reference stores it."""
    return x.to(torch.float32).to(torch.float16).to(dtype)


def _gather_paged(cache_codes, table_row, n_tokens, kv_head):
    """[n_tokens, D] float32 of one kv head, gathered via one block-table row."""
    bs = cache_codes.shape[1]
    n_blocks = (n_tokens + bs - 1) // bs
    blocks = table_row[:n_blocks].to(torch.int64)
    rows = cache_codes[blocks, :, kv_head, :].reshape(n_blocks * bs, -1)[:n_tokens]
    return _fp8.dequant_codes_tensor(rows)


def _attend(qg, k, v, scale, limits, compute_dtype):
    """qg: [R, D]; k, v: [L, D]; limits: [R] number of visible keys per row."""
    qg = qg.to(compute_dtype)
    k = k.to(compute_dtype)
    v = v.to(compute_dtype)
    s = (qg @ k.T) * scale
    L = k.shape[0]
    col = torch.arange(L).unsqueeze(0)
    visible = col < limits.unsqueeze(1)
    s = s.masked_fill(~visible, float("-inf"))
    m = s.max(dim=1, keepdim=True).values
    p = torch.exp(s - m)
    p = torch.where(visible, p, torch.zeros_like(p))
    l = p.sum(dim=1, keepdim=True)
    o = (p @ v) / l
    return o, l.squeeze(1)


def decode_attention(q, k_cache, v_cache, block_tables, context_lens, softmax_scale,
                     compute_dtype=torch.float32, return_fp32=False):
    """Reference-semantics paged decode on the CPU.

    q: bf16 or fp16 [B, Hq, D]; k_cache/v_cache: uint8 or float8_e4m3fn
    [P, bs, Hkv, D]; block_tables: int [B, max_nb]; context_lens: int [B].
    Returns [B, Hq, D] of q's dtype (or the unrounded result if
    ``return_fp32``).
    """
    kc, vc = _as_codes(k_cache), _as_codes(v_cache)
    B, Hq, D = q.shape
    Hkv = kc.shape[2]
    G = Hq // Hkv
    out = torch.empty(B, Hq, D, dtype=compute_dtype)
    for b in range(B):
        ctx = int(context_lens[b])
        if ctx <= 0:
            out[b] = float("nan")
            continue
        for g in range(Hkv):
            k = _gather_paged(kc, block_tables[b], ctx, g)
            v = _gather_paged(vc, block_tables[b], ctx, g)
            qg = q[b, g * G:(g + 1) * G].float()
            limits = torch.full((G,), ctx, dtype=torch.int64)
            o, _ = _attend(qg, k, v, softmax_scale, limits, compute_dtype)
            out[b, g * G:(g + 1) * G] = o
    return out if return_fp32 else round_output(out, q.dtype)


def prefill_attention(q, k, v, block_tables, cu_seqlens_q, cu_seqlens_k, softmax_scale,
                      compute_dtype=torch.float32, return_fp32=False):
    """Reference-semantics varlen causal prefill on the CPU.

    q: bf16 or fp16 [Nq, Hq, D] (the output's dtype).  Paged: k/v are caches [P, bs, Hkv, D] and
    block_tables int [S, max_nb].  Contiguous (block_tables is None): k/v are
    [Nk, Hkv, D] FP8 codes indexed by cu_seqlens_k.
    """
    kc, vc = _as_codes(k), _as_codes(v)
    Nq, Hq, D = q.shape
    paged = block_tables is not None
    Hkv = kc.shape[2] if paged else kc.shape[1]
    G = Hq // Hkv
    cq = [int(x) for x in cu_seqlens_q]
    ck = [int(x) for x in cu_seqlens_k]
    out = torch.zeros(Nq, Hq, D, dtype=compute_dtype)
    for s in range(len(cq) - 1):
        q0, q1 = cq[s], cq[s + 1]
        Lq, Lk = q1 - q0, ck[s + 1] - ck[s]
        if Lq <= 0:
            continue
        c = Lk - Lq
        limits = torch.clamp(torch.arange(Lq) + c + 1, min=0, max=max(Lk, 0))
        for g in range(Hkv):
            if paged:
                kk = _gather_paged(kc, block_tables[s], Lk, g)
                vv = _gather_paged(vc, block_tables[s], Lk, g)
            else:
                kk = _fp8.dequant_codes_tensor(kc[ck[s]:ck[s + 1], g])
                vv = _fp8.dequant_codes_tensor(vc[ck[s]:ck[s + 1], g])
            # the G query heads of this kv head share K/V: stack them as rows
            qg = q[q0:q1, g * G:(g + 1) * G].float().permute(1, 0, 2).reshape(G * Lq, D)
            o, l = _attend(qg, kk, vv, softmax_scale, limits.repeat(G), compute_dtype)
            o = torch.where((l > 0).unsqueeze(1), o, torch.zeros_like(o))
            out[q0:q1, g * G:(g + 1) * G] = o.reshape(G, Lq, D).permute(1, 0, 2)
    return out if return_fp32 else round_output(out, q.dtype)

