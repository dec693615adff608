"""Oracle: LM-head row selection and the sampler (TEST INFRASTRUCTURE ONLY).

* ``select_rows`` restates the row selection of ParallelLMHead.forward
  (nanovllm/layers/embed_head.py:56-72): with varlen rows present, keep the
  plain-decode rows ``x[:split_pt]``, every row of the speculative sequences
  (``x[split_pt : split_pt + cu_seqlens_q[nspec]]``) and the last row of each
  remaining varlen (prefill) sequence (``cu_seqlens_q[nspec + 1:] - 1``).
* ``sample`` restates Sampler.forward (nanovllm/layers/sampler.py:7-12) for a
  given noise matrix E: ``y = logits.float() / T`` (fp32 division), ``p =
  softmax(y)`` (``exp(y - max) / sum``), ``argmax(p / max(E, 1e-10))``, the
  first index on ties.  The reference draws E with torch's exponential_(1);
  the noise here is a parameter.  It also returns the scores p / E, so that
  a test can tell a near tie from a wrong pick.
* ``philox4x32_10`` is the counter-based generator of Salmon, Moraes, Dror and
  Shaw, "Parallel random numbers: as easy as 1, 2, 3" (SC'11): ten rounds of
  two 32 x 32 -> 64-bit multiplies (0xD2511F53, 0xCD9E8D57) with the key
  bumped by the Weyl constants (0x9E3779B9, 0xBB67AE85).  ``exponential_noise``
  maps its output to E = -log(u), u = ((x >> 8) + 1) 2^-24 in (0, 1], with
  counter (v / 4, row, offset_lo, offset_hi) and key (seed_lo, seed_hi) for
  elements v .. v + 3 of a row -- the token stream.
* ``sample_grouped`` restates the GPU sampler's in-kernel draw, top down by
  groups of 16 tokens (the Gumbel-max property: max_v (c z_v - log2 E_v) over
  a group is itself -log2 E located at log2 sum_v 2^(c z_v), c = log2(e) / T,
  independent of the token attaining it): group g's maximum M_g = log2 sum_v
  2^(c z_v) - log2(max(E_g, 1e-10)) with E_g from the group stream (counter
  (2^31 + 64 (g // 256) + g % 64, row, offset_lo, offset_hi), word
  (g // 64) % 4), the winning group is the first argmax of M_g, and the token
  the first argmax inside it of c z_v - log2(max(E_v, 1e-10)) on the token
  stream.  The token distribution is softmax(z / T), as with one E per token.

Pinned by tests/test_oracle_lm_head.py: Random123's published known-answer
vectors for Philox4x32-10; torch's own CPU softmax + argmax on the same noise;
the Gumbel-max identity argmax(p / E) = argmax(y - log E); the empirical
distribution of samples against softmax (per-token and grouped draws, the
latter with many groups and with partial groups); the group maximum's law
against the per-token maxima of the same groups; and the selection against
torch's index_select of the reference's index construction.
"""
import numpy as np

M0, M1 = 0xD2511F53, 0xCD9E8D57
W0, W1 = 0x9E3779B9, 0xBB67AE85
MASK32 = 0xFFFFFFFF


def select_rows(x, split_pt, num_spec_seqs, cu_seqlens_q):
    """x: [T, H] (numpy or torch); cu_seqlens_q: sequence of ints for the varlen
    sequences, or None (no varlen rows: x unchanged)."""
    if cu_seqlens_q is None:
        return x
    cu = [int(c) for c in cu_seqlens_q]
    keep = list(range(split_pt)) + [split_pt + i for i in range(cu[num_spec_seqs])] + \
        [split_pt + c - 1 for c in cu[num_spec_seqs + 1:]]
    return x[keep]


def philox4x32_10(ctr, key):
    """ctr: uint64 array [..., 4] (32-bit words), key: uint64 array [..., 2] -> uint64 [..., 4]."""
    c = [np.asarray(ctr[..., i], dtype=np.uint64) for i in range(4)]
    k0 = np.asarray(key[..., 0], dtype=np.uint64)
    k1 = np.asarray(key[..., 1], dtype=np.uint64)
    m0, m1 = np.uint64(M0), np.uint64(M1)
    for _ in range(10):
        p0 = c[0] * m0
        p1 = c[2] * m1
        hi0, lo0 = p0 >> np.uint64(32), p0 & np.uint64(MASK32)
        hi1, lo1 = p1 >> np.uint64(32), p1 & np.uint64(MASK32)
        c = [hi1 ^ c[1] ^ k0, lo1, hi0 ^ c[3] ^ k1, lo0]
        k0 = (k0 + np.uint64(W0)) & np.uint64(MASK32)
        k1 = (k1 + np.uint64(W1)) & np.uint64(MASK32)
    return np.stack(c, axis=-1)


def exponential_noise(seed, offset, rows, vocab):
    """float32 [rows, vocab] Exp(1) samples from the Philox stream (module docstring)."""
    nb = (vocab + 3) // 4
    j = np.arange(nb, dtype=np.uint64)[None, :].repeat(rows, 0)
    r = np.arange(rows, dtype=np.uint64)[:, None].repeat(nb, 1)
    ctr = np.stack([j, r, np.full_like(j, offset & MASK32), np.full_like(j, (offset >> 32) & MASK32)], -1)
    key = np.stack([np.full_like(j, seed & MASK32), np.full_like(j, (seed >> 32) & MASK32)], -1)
    bits = philox4x32_10(ctr, key).reshape(rows, nb * 4)[:, :vocab]
    u = (((bits >> np.uint64(8)) + np.uint64(1)).astype(np.float32) * np.float32(2.0 ** -24)).astype(np.float32)
    return (-np.log(u)).astype(np.float32)


def sample(logits, temperatures, noise):
    """logits: float array [R, V] (the values of the bf16 / fp16 / fp32
    logits); temperatures: [R]; noise: float32 [R, V] -> int64 [R]."""
    y = np.asarray(logits, dtype=np.float32) / np.asarray(temperatures, dtype=np.float32)[:, None]
    m = y.max(axis=-1, keepdims=True)
    e = np.exp(y - m).astype(np.float32)
    p = (e / e.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)
    q = (p / np.maximum(noise, np.float32(1e-10))).astype(np.float32)
    return q.argmax(axis=-1).astype(np.int64), q


GROUP_TOK = 16
GROUP_COUNTER = 1 << 31


def _uniform_exp(bits):
    """E = -log(u), u = ((x >> 8) + 1) 2^-24, float32."""
    u = (((bits >> np.uint64(8)) + np.uint64(1)).astype(np.float32) * np.float32(2.0 ** -24)).astype(np.float32)
    return (-np.log(u)).astype(np.float32)


def group_noise(seed, offset, rows, n_groups):
    """float32 [rows, n_groups]: E_g of the group stream (module docstring)."""
    g = np.arange(n_groups, dtype=np.uint64)[None, :].repeat(rows, 0)
    r = np.arange(rows, dtype=np.uint64)[:, None].repeat(n_groups, 1)
    x = np.uint64(GROUP_COUNTER) + np.uint64(64) * (g // np.uint64(256)) + g % np.uint64(64)
    ctr = np.stack([x, r, np.full_like(g, offset & MASK32), np.full_like(g, (offset >> 32) & MASK32)], -1)
    key = np.stack([np.full_like(g, seed & MASK32), np.full_like(g, (seed >> 32) & MASK32)], -1)
    bits = philox4x32_10(ctr, key)
    word = ((g // np.uint64(64)) % np.uint64(4)).astype(np.int64)
    return _uniform_exp(np.take_along_axis(bits, word[..., None], -1)[..., 0])


def _neg_log2_clamped(e):
    return (-np.log2(np.maximum(e, np.float32(1e-10)))).astype(np.float32)


def sample_grouped(logits, temperatures, seed, offset):
    """The in-kernel draw of the GPU sampler.  logits: float array [R, V];
    temperatures: [R].  Returns (tokens int64 [R], group scores M float32
    [R, G], token scores float32 [R, V], filled for the tokens of each row's
    winning group and -inf elsewhere) -- the scores let a test tell a near
    tie from a wrong pick."""
    z = np.asarray(logits, dtype=np.float32)
    R, V = z.shape
    c1 = (np.float32(1.4426950408889634) / np.asarray(temperatures, dtype=np.float32)).astype(np.float32)
    zc = (z * c1[:, None]).astype(np.float32)
    G = (V + GROUP_TOK - 1) // GROUP_TOK
    pad = np.full((R, G * GROUP_TOK), -np.inf, dtype=np.float32)
    pad[:, :V] = zc
    zg = pad.reshape(R, G, GROUP_TOK)
    mx = zg.max(axis=-1)
    finite = mx > -np.inf
    safe_mx = np.where(finite, mx, np.float32(0)).astype(np.float32)
    s = np.zeros((R, G), dtype=np.float32)
    with np.errstate(invalid="ignore"):
        for i in range(GROUP_TOK):  # in token order, as the kernel sums
            s = (s + np.exp2((zg[..., i] - safe_mx).astype(np.float32))).astype(np.float32)
    with np.errstate(divide="ignore"):
        m = ((safe_mx + np.log2(s)).astype(np.float32) + _neg_log2_clamped(group_noise(seed, offset, R, G)))
    m = np.where(finite, m, np.float32(-np.inf)).astype(np.float32)
    gbest = m.argmax(axis=-1)
    # token stream, drawn only for the tokens of each row's winning group
    v = gbest[:, None].astype(np.int64) * GROUP_TOK + np.arange(GROUP_TOK)[None, :]
    inside = v < V
    vc = np.minimum(v, V - 1).astype(np.uint64)
    r = np.arange(R, dtype=np.uint64)[:, None].repeat(GROUP_TOK, 1)
    ctr = np.stack([vc // np.uint64(4), r, np.full_like(r, offset & MASK32), np.full_like(r, (offset >> 32) & MASK32)],
                   -1)
    key = np.stack([np.full_like(r, seed & MASK32), np.full_like(r, (seed >> 32) & MASK32)], -1)
    bits = np.take_along_axis(philox4x32_10(ctr, key), (vc % np.uint64(4)).astype(np.int64)[..., None], -1)[..., 0]
    sc = (np.take_along_axis(zc, np.minimum(v, V - 1), -1) + _neg_log2_clamped(_uniform_exp(bits))).astype(np.float32)
    sc = np.where(inside, sc, np.float32(-np.inf))
    tok_scores = np.full((R, V), -np.inf, dtype=np.float32)
    np.put_along_axis(tok_scores, np.minimum(v, V - 1), np.where(inside, sc, tok_scores[0, 0]), -1)
    tokens = (gbest.astype(np.int64) * GROUP_TOK + sc.argmax(axis=-1)).astype(np.int64)
    return tokens, m, tok_scores
