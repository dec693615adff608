"""LM-head row selection and the sampler on the GPU against the oracle
(nanovllm/layers/embed_head.py:56-72, nanovllm/layers/sampler.py:7-12).

Selection is byte-exact.  Sampling is compared token by token with the
oracle on the same noise: a given matrix (the tokens agree unless the
oracle's two best scores p / E are within 1e-4 of each other: the kernel
ranks by the equivalent log2-domain score z log2(e) / T - log2(E), whose
rounding differs from the oracle's fp32 softmax by a few ulps), or the
in-kernel Philox4x32-10 draw, top down by groups of 16 tokens (the tokens
agree unless the two groups' maxima, or the two tokens' scores inside the
group, are within 1e-4 of each other).  The in-kernel noise is also checked
as a distribution against softmax(logits / T): 40,000 draws of 6 logits and
30,000 of 40 (three groups).
"""
from dataclasses import dataclass

import numpy as np
import pytest
import torch

from gpu_util import announce
from oracle import lm_head as olh
from oracle import metadata as om
from nanovllm_amd.engine import metadata as nm
from nanovllm_amd.layers.embed_head import select_lm_head_rows, lm_head_logits
from nanovllm_amd.layers.sampler import Sampler, sample_tokens
from nanovllm_amd.utils import context as ctxmod

pytestmark = pytest.mark.gpu


def _agree(got, want, q, rel=1e-4):
    bad = [r for r in range(len(want)) if got[r] != want[r] and
           abs(q[r][want[r]] - q[r][got[r]]) > rel * abs(q[r][want[r]])]
    assert not bad, f"{len(bad)} rows differ beyond a near tie, first {bad[0]}: gpu {got[bad[0]]} oracle {want[bad[0]]}"


@pytest.mark.parametrize("split_pt,lq,nspec", [(7, [5, 5, 3, 512, 40], 2), (0, [6, 100], 0), (12, [4, 4], 2),
                                                (0, [1000], 0)])
def test_select_rows_byte_exact(split_pt, lq, nspec):
    announce(f"lm head: row selection split_pt={split_pt} lq={lq} nspec={nspec}")
    g = torch.Generator().manual_seed(split_pt + len(lq))
    cu = [0] + list(np.cumsum(lq))
    x = torch.randn(split_pt + cu[-1], 4096, generator=g).to(torch.bfloat16)
    ctxmod.set_context(split_pt=split_pt, num_spec_seqs=nspec, num_spec_rows=cu[nspec],
                       cu_seqlens_q=torch.tensor(cu, dtype=torch.int32, device="cuda"))
    try:
        got = select_lm_head_rows(x.cuda(), ctxmod.get_context())
        torch.cuda.synchronize()
        assert torch.equal(got.cpu(), olh.select_rows(x, split_pt, nspec, cu))
        ctxmod.set_context(num_spec_rows=-1)          # the count read back from the GPU instead
        assert torch.equal(select_lm_head_rows(x.cuda(), ctxmod.get_context()).cpu(),
                           olh.select_rows(x, split_pt, nspec, cu))
        w = torch.randn(1000, 4096, generator=g).to(torch.bfloat16).cuda()
        want = torch.nn.functional.linear(olh.select_rows(x, split_pt, nspec, cu).cuda(), w)
        assert torch.equal(lm_head_logits(x.cuda(), w, ctxmod.get_context()), want)
    finally:
        ctxmod.reset_context()
    # no varlen rows: x itself
    assert select_lm_head_rows(x, ctxmod.get_context()) is x


@dataclass(slots=True)
class ReferenceShapedContext:
    """The fields of nanovllm/utils/context.py:5-15 and nothing else (no
    num_spec_rows), as the reference's runner fills them."""
    split_pt: int = 0
    num_spec_seqs: int = 0
    cu_seqlens_q: torch.Tensor | None = None
    cu_seqlens_k: torch.Tensor | None = None
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    slot_mapping: torch.Tensor | None = None
    context_lens: torch.Tensor | None = None
    block_tables: torch.Tensor | None = None


def test_select_rows_through_the_runners_context():
    """The step's metadata published through a setter with exactly the
    reference's keyword arguments (as model_runner.py:218 calls it), then the
    LM-head rows selected from that Context: the package's own Context is
    neither written nor read."""
    announce("lm head: row selection through a reference-shaped Context")
    ref = ReferenceShapedContext()

    def ref_set_context(split_pt, num_spec_seqs, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                        slot_mapping, context_lens, block_tables):
        ref.split_pt, ref.num_spec_seqs = split_pt, num_spec_seqs
        ref.cu_seqlens_q, ref.cu_seqlens_k = cu_seqlens_q, cu_seqlens_k
        ref.max_seqlen_q, ref.max_seqlen_k = max_seqlen_q, max_seqlen_k
        ref.slot_mapping, ref.context_lens, ref.block_tables = slot_mapping, context_lens, block_tables

    ctxmod.reset_context()
    rng = np.random.default_rng(5)
    pool = iter(rng.permutation(10000).tolist())
    dseqs = [om.SeqView(n, n - 1, 1, [next(pool) for _ in range(-(-n // 256))]) for n in (40, 700, 1300)]
    dseqs += [om.SeqView(n, n - 1, 5, [next(pool) for _ in range(-(-(n + 4) // 256))]) for n in (300, 900)]
    pseqs = [om.SeqView(n, c, n - c, [next(pool) for _ in range(-(-n // 256))]) for n, c in ((600, 0), (1000, 488))]
    want_md = om.prepare_sequence(dseqs, pseqs, 256)
    for build in (nm.prepare_sequence_device, nm.prepare_sequence):
        positions = build(dseqs, pseqs, 256, ref_set_context)
        n_tok = positions.numel()
        x = torch.randn(n_tok, 512, generator=torch.Generator().manual_seed(n_tok)).to(torch.bfloat16)
        got = select_lm_head_rows(x.cuda(), ref)
        torch.cuda.synchronize()
        assert ref.cu_seqlens_q.cpu().tolist() == want_md["cu_seqlens_q"]
        want = olh.select_rows(x, want_md["split_pt"], want_md["num_spec_seqs"], want_md["cu_seqlens_q"])
        assert got.shape[0] == 3 + 2 * 5 + 2 and torch.equal(got.cpu(), want), build.__name__
        assert ctxmod.get_context().cu_seqlens_q is None and ctxmod.get_context().slot_mapping is None


@pytest.mark.parametrize("dtype,vocab", [(torch.bfloat16, 151936), (torch.float16, 1003), (torch.float32, 4096)])
def test_sample_with_given_noise(dtype, vocab):
    announce(f"lm head: sampler, given noise, {dtype}, vocab {vocab}")
    g = torch.Generator().manual_seed(vocab)
    R = 24
    logits = (torch.randn(R, vocab, generator=g) * 5).to(dtype)
    temps = torch.rand(R, generator=g) * 1.5 + 0.05
    temps[0] = 1e-3                                   # nearly greedy
    noise = torch.empty(R, vocab).exponential_(1, generator=g)
    noise[1, :50] = 0.0                               # clamp_min(1e-10) path
    got = sample_tokens(logits.cuda(), temps.cuda(), noise=noise.cuda()).cpu().numpy()
    want, q = olh.sample(logits.float().numpy(), temps.numpy(), noise.numpy())
    _agree(got, want, q)


def _agree_grouped(got, want, m, tok_scores, rel=1e-4):
    G = olh.GROUP_TOK
    bad = []
    for r in range(len(want)):
        if got[r] == want[r]:
            continue
        gg, gw = int(got[r]) // G, int(want[r]) // G
        if gg != gw:
            tie = abs(m[r][gg] - m[r][gw]) <= rel * max(abs(m[r][gw]), 1.0)
        else:
            a, b = tok_scores[r][want[r]], tok_scores[r][got[r]]
            tie = abs(a - b) <= rel * max(abs(a), 1.0)
        if not tie:
            bad.append(r)
    assert not bad, f"{len(bad)} rows differ beyond a near tie, first {bad[0]}: gpu {got[bad[0]]} oracle {want[bad[0]]}"


@pytest.mark.parametrize("dtype,vocab,aligned", [(torch.bfloat16, 151936, True), (torch.float16, 32003, True),
                                                 (torch.float32, 4096, True), (torch.bfloat16, 5000, False)])
def test_sample_with_in_kernel_noise_matches_the_group_draw(dtype, vocab, aligned):
    """The kernel's top-down draw against the oracle's, token by token; the
    Qwen3 vocabulary, a vocabulary that leaves a partial group and a partial
    quad, fp32 logits, and rows whose start is not 4-element aligned (the
    element-wise load path)."""
    announce(f"lm head: sampler, in-kernel Philox noise, {dtype}, vocab {vocab}, aligned {aligned}")
    g = torch.Generator().manual_seed(vocab)
    R = 40
    full = (torch.randn(R, vocab + 1, generator=g) * 3).to(dtype)
    logits = full[:, :vocab] if aligned else full[:, 1:]
    temps = torch.rand(R, generator=g) + 0.3
    temps[0] = 1e-3                                   # nearly greedy
    seed, offset = 0x1234_5678_9ABC + vocab, 77
    lg = logits.cuda() if aligned else full.cuda()[:, 1:]
    got = sample_tokens(lg, temps.cuda(), seed=seed, offset=offset).cpu().numpy()
    want, m, tok_scores = olh.sample_grouped(logits.float().numpy(), temps.numpy(), seed, offset)
    _agree_grouped(got, want, m, tok_scores)


def test_in_kernel_samples_follow_softmax():
    from scipy.stats import chisquare
    announce("lm head: sampler distribution (40,000 draws)")
    logits = torch.tensor([1.0, 0.2, -0.5, 2.0, 0.0, -3.0])
    n = 40000
    tok = sample_tokens(logits.repeat(n, 1).cuda(), torch.full((n,), 0.7, device="cuda"), seed=2024).cpu().numpy()
    p = torch.softmax(logits / 0.7, 0).double().numpy()
    assert chisquare(np.bincount(tok, minlength=6), p * n).pvalue > 1e-4


def test_in_kernel_samples_follow_softmax_over_groups():
    """40 logits (groups of 16, the last partial) at T = 0.8, 30,000 draws:
    the winning group and the token inside it together follow softmax."""
    from scipy.stats import chisquare
    announce("lm head: sampler distribution over three groups (30,000 draws)")
    logits = torch.from_numpy((np.random.default_rng(40).normal(size=40) * 1.5).astype(np.float32))
    n = 30000
    tok = sample_tokens(logits.repeat(n, 1).cuda(), torch.full((n,), 0.8, device="cuda"), seed=77).cpu().numpy()
    p = torch.softmax(logits.double() / 0.8, 0).numpy()
    counts = np.bincount(tok, minlength=40)
    big = p * n >= 20
    obs = np.concatenate([counts[big], [counts[~big].sum()]])
    exp = np.concatenate([p[big] * n, [p[~big].sum() * n]])
    assert chisquare(obs, exp).pvalue > 1e-4


def test_sampler_module_is_repeatable_under_manual_seed():
    announce("lm head: Sampler module and torch.manual_seed")
    logits = torch.randn(8, 32000).to(torch.bfloat16).cuda()
    temps = torch.ones(8, device="cuda")
    torch.manual_seed(11)
    a = Sampler()(logits, temps)
    torch.manual_seed(11)
    b = Sampler()(logits, temps)
    c = Sampler()(logits, temps)
    assert torch.equal(a, b) and a.dtype == torch.int64 and a.shape == (8,)
    assert not torch.equal(b, c)
