"""Pins the LM-head row selection and sampler oracle (nanovllm/layers/embed_head.py:56-72,
nanovllm/layers/sampler.py:7-12).

Independent checks: Random123's published known-answer vectors for
Philox4x32-10; torch's own CPU softmax and argmax on the same noise; the
Gumbel-max identity argmax(p / E) = argmax(y - log E); the empirical
distribution of samples against softmax(logits / T); the Exp(1) noise's
moments; and the row selection against torch's index_select of the index
tensors the reference builds.
"""
import numpy as np
import pytest
import torch

from oracle import lm_head as olh


@pytest.mark.parametrize("ctr,key,want", [
    ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
    ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
    ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
     [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
])
def test_philox_known_answers(ctr, key, want):
    got = olh.philox4x32_10(np.array(ctr, dtype=np.uint64), np.array(key, dtype=np.uint64))
    assert [int(v) for v in got] == want


def test_exponential_noise_moments():
    e = olh.exponential_noise(seed=123, offset=7, rows=4, vocab=50000).astype(np.float64)
    assert e.min() > 0 and np.isfinite(e).all()
    assert abs(e.mean() - 1.0) < 0.01 and abs(e.var() - 1.0) < 0.03
    assert not np.array_equal(e, olh.exponential_noise(seed=124, offset=7, rows=4, vocab=50000))


def _near_tie(q, a, b, rel=1e-5):
    return q[a] == q[b] or abs(q[a] - q[b]) <= rel * max(q[a], q[b])


def test_sample_matches_torch_softmax_argmax():
    g = torch.Generator().manual_seed(0)
    R, V = 12, 3001
    logits = (torch.randn(R, V, generator=g) * 4).to(torch.bfloat16)
    temps = torch.rand(R, generator=g) * 2 + 0.05
    noise = torch.empty(R, V).exponential_(1, generator=g)
    got, q = olh.sample(logits.float().numpy(), temps.numpy(), noise.numpy())
    probs = torch.softmax(logits.float() / temps[:, None], dim=-1)
    want = (probs / noise.clamp_min(1e-10)).argmax(dim=-1).numpy()
    for r in range(R):
        assert got[r] == want[r] or _near_tie(q[r], got[r], want[r])


def test_gumbel_max_identity():
    """argmax(softmax(y) / E) = argmax(y - log E): the division by the
    softmax sum and the exp are monotone."""
    rng = np.random.default_rng(1)
    R, V = 20, 5000
    y = rng.normal(size=(R, V)).astype(np.float32) * 3
    noise = rng.exponential(size=(R, V)).astype(np.float32)
    got, q = olh.sample(y, np.ones(R, np.float32), noise)
    gumbel = (y.astype(np.float64) - np.log(noise.astype(np.float64))).argmax(-1)
    for r in range(R):
        assert got[r] == gumbel[r] or _near_tie(q[r], got[r], gumbel[r])


def test_samples_follow_softmax():
    """Frequencies of 40,000 draws from 6 logits at T = 0.7 against softmax
    (chi-square with 5 degrees of freedom, p > 1e-4)."""
    from scipy.stats import chisquare
    logits = np.array([1.0, 0.2, -0.5, 2.0, 0.0, -3.0], dtype=np.float32)
    n = 40000
    noise = olh.exponential_noise(seed=99, offset=0, rows=n, vocab=6)
    tok, _ = olh.sample(np.tile(logits, (n, 1)), np.full(n, 0.7, np.float32), noise)
    p = np.exp(logits / 0.7) / np.exp(logits / 0.7).sum()
    counts = np.bincount(tok, minlength=6)
    assert chisquare(counts, p * n).pvalue > 1e-4


def test_select_rows_matches_the_reference_index_construction():
    """x[:split_pt], then varlen rows index_select'ed with arange(cu[nspec])
    and cu[nspec + 1:] - 1 (embed_head.py:62-72), built with torch ops."""
    g = torch.Generator().manual_seed(2)
    split_pt, nspec = 5, 2
    lq = [3, 4, 7, 1, 9]                       # 2 speculative sequences, 3 prefill ones
    cu = torch.tensor([0] + list(np.cumsum(lq)), dtype=torch.int32)
    x = torch.randn(split_pt + int(cu[-1]), 16, generator=g)
    varlen = x[split_pt:]
    keep = torch.cat([torch.arange(int(cu[nspec])), cu[nspec + 1:].long() - 1])
    want = torch.cat((x[:split_pt], varlen.index_select(0, keep)))
    got = olh.select_rows(x, split_pt, nspec, cu.tolist())
    assert torch.equal(got, want)
    assert olh.select_rows(x, split_pt, nspec, None) is x


def _chisquare_buckets(tok, p, n, min_expected=20):
    """Chi-square p-value of token counts against probabilities p, tokens with
    fewer than min_expected expected draws pooled into one bucket."""
    from scipy.stats import chisquare
    counts = np.bincount(tok, minlength=len(p)).astype(np.float64)
    big = p * n >= min_expected
    obs = np.concatenate([counts[big], [counts[~big].sum()]])
    exp = np.concatenate([p[big] * n, [p[~big].sum() * n]])
    if exp[-1] == 0:
        obs, exp = obs[:-1], exp[:-1]
    return chisquare(obs, exp).pvalue


@pytest.mark.parametrize("vocab,temp,scale,n", [(6, 0.7, 1.0, 30000), (40, 0.8, 1.5, 30000), (300, 0.5, 1.0, 30000),
                                                (5000, 0.25, 1.0, 8000)])
def test_grouped_draw_follows_softmax(vocab, temp, scale, n):
    """The top-down grouped draw (groups of 16; one partial group at vocab 6,
    40 and 300; two 4,096-token quads at 5,000) against softmax(z / T): n
    draws (rows of the same logits), chi-square p > 1e-4 (tokens expected
    fewer than 20 times pooled)."""
    rng = np.random.default_rng(vocab)
    z = (rng.normal(size=vocab) * scale).astype(np.float32)
    tok, _, _ = olh.sample_grouped(np.tile(z, (n, 1)), np.full(n, temp, np.float32), seed=vocab * 31 + 1, offset=5)
    y = z.astype(np.float64) / temp
    p = np.exp(y - y.max())
    p /= p.sum()
    assert _chisquare_buckets(tok, p, n) > 1e-4


def test_group_maximum_has_the_law_of_the_token_maxima():
    """M_g, drawn directly, against max_v (c z_v - log2 E_v) over the same 16
    tokens with one E per token (the token stream): both are Gumbel variables
    located at log2 sum_v 2^(c z_v) (two-sample Kolmogorov-Smirnov, 20,000
    each, p > 1e-3; a dropped log2-sum or a wrong sign shifts one by a full
    unit)."""
    from scipy.stats import ks_2samp
    rng = np.random.default_rng(3)
    z = (rng.normal(size=16) * 2).astype(np.float32)
    n = 20000
    _, m, tok_scores = olh.sample_grouped(np.tile(z, (n, 1)), np.ones(n, np.float32), seed=11, offset=0)
    direct = m[:, 0].astype(np.float64)
    per_token = tok_scores.max(axis=1).astype(np.float64)
    assert ks_2samp(direct, per_token).pvalue > 1e-3
    loc = np.log2(np.exp2(z.astype(np.float64) * 1.4426950408889634).sum())
    # Gumbel in log2 units: mean = loc + Euler-Mascheroni / ln 2
    assert abs(direct.mean() - (loc + 0.5772156649 / np.log(2))) < 0.03


def test_group_and_token_streams_are_distinct():
    """The group stream's counters start at 2^31, above every token counter
    (v / 4 < 2^29): the two draws of a row never share a Philox output."""
    e_tok = olh.exponential_noise(seed=5, offset=9, rows=2, vocab=64 * 4)
    e_grp = olh.group_noise(seed=5, offset=9, rows=2, n_groups=64)
    assert not np.isin(e_grp, e_tok).any()
    again = olh.group_noise(seed=5, offset=9, rows=2, n_groups=64)
    assert np.array_equal(e_grp, again) and e_grp.min() > 0
