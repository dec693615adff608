"""LM-head row selection and the sampler on the GPU against the oracle
(nanovllm/layers/embed_head.py:56-72, nanovllm/layers/sampler.py:7-12).

Selection is byte-exact.  Sampling is compared token by token with the
oracle on the same noise (a given matrix, or the Philox4x32-10 stream the
kernel draws in place): the tokens agree unless the oracle's two best scores
p / E are within 1e-4 of each other (the kernel ranks by the equivalent
log2-domain score z log2(e) / T - log2(E), whose rounding differs from the
oracle's fp32 softmax by a few ulps).  The in-kernel noise is also checked as a
distribution: 40,000 draws against softmax(logits / T).
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


def test_sample_with_in_kernel_noise_matches_the_philox_stream():
    announce("lm head: sampler, in-kernel Philox noise, vocab 151936")
    g = torch.Generator().manual_seed(5)
    R, V = 40, 151936
    logits = (torch.randn(R, V, generator=g) * 3).to(torch.bfloat16)
    temps = torch.rand(R, generator=g) + 0.3
    seed, offset = 0x1234_5678_9ABC, 77
    got = sample_tokens(logits.cuda(), temps.cuda(), seed=seed, offset=offset).cpu().numpy()
    noise = olh.exponential_noise(seed, offset, R, V)
    want, q = olh.sample(logits.float().numpy(), temps.numpy(), noise)
    _agree(got, want, q)


def test_in_kernel_samples_follow_softmax():
    from scipy.stats import chisquare
    announce("lm head: sampler distribution (40,000 draws)")
    logits = torch.tensor([1.0, 0.2, -0.5, 2.0, 0.0, -3.0])
    n = 40000
    tok = sample_tokens(logits.repeat(n, 1).cuda(), torch.full((n,), 0.7, device="cuda"), seed=2024).cpu().numpy()
    p = torch.softmax(logits / 0.7, 0).double().numpy()
    assert chisquare(np.bincount(tok, minlength=6), p * n).pvalue > 1e-4


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
