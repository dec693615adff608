"""On-device attention metadata (nanovllm/engine/model_runner.py:133-220):
nvamd_build_attention_metadata must equal the loop-for-loop oracle byte for
byte -- positions, slot mapping, context lengths, cu_seqlens, max lengths and
the -1 padded block tables -- over seeded random steps mixing plain decode,
speculative and prefill sequences, warm-up sequences without tables, tables
longer than needed, block sizes 16 .. 512, up to 2,048 sequences and
128K-token contexts."""
import numpy as np
import pytest
import torch

from gpu_util import announce
from oracle import metadata as om
from nanovllm_amd.engine import metadata as nm
from nanovllm_amd.utils import context as ctxmod

pytestmark = pytest.mark.gpu


def random_step(rng, bs, n_decode, n_prefill, max_len=3000, warm_frac=0.0, spare_blocks=0):
    """Sequences carry the step's block size, as nano-vLLM's Sequence does
    (Sequence.block_size = kvcache_block_size)."""
    pool = iter(rng.permutation(400000))
    dseqs, pseqs = [], []
    for _ in range(n_decode):
        n_tok = int(rng.integers(1, max_len))
        drafts = int(rng.integers(0, 5)) if rng.random() < 0.3 else 0
        nb = -(-(n_tok + drafts) // bs) + (spare_blocks if rng.random() < 0.2 else 0)
        table = [int(next(pool)) for _ in range(nb)]
        if drafts == 0:
            dseqs.append(om.SeqView(n_tok, n_tok - 1, 1, table[: max(-(-n_tok // bs), len(table) - spare_blocks)], bs))
        else:
            dseqs.append(om.SeqView(n_tok, n_tok - 1, 1 + drafts, table, bs))
    for _ in range(n_prefill):
        n_tok = int(rng.integers(1, max_len))
        cached = int(rng.integers(0, n_tok))
        lq = int(rng.integers(1, n_tok - cached + 1))
        table = [] if rng.random() < warm_frac else [int(next(pool)) for _ in range(-(-n_tok // bs))]
        pseqs.append(om.SeqView(n_tok, cached, lq, table, bs))
    return dseqs, pseqs


def check_step(dseqs, pseqs, bs):
    want = om.prepare_sequence(dseqs, pseqs, bs)
    got = nm.build_device_metadata(nm.pack_step(dseqs, pseqs, bs), bs)
    torch.cuda.synchronize()
    assert got["positions"].dtype == torch.int64 and got["positions"].cpu().tolist() == want["positions"]
    assert got["slot_mapping"].dtype == torch.int32 and got["slot_mapping"].cpu().tolist() == want["slot_mapping"]
    for key in ("context_lens", "cu_seqlens_q", "cu_seqlens_k"):
        if want[key] is None:
            assert got[key] is None, key
        else:
            assert got[key].cpu().tolist() == want[key], key
    assert (got["max_seqlen_q"], got["max_seqlen_k"]) == (want["max_seqlen_q"], want["max_seqlen_k"])
    assert (got["split_pt"], got["num_spec_seqs"]) == (want["split_pt"], want["num_spec_seqs"])
    if want["block_tables"] is None:
        assert got["block_tables"] is None
    else:
        assert got["block_tables"].cpu().tolist() == want["block_tables"]


@pytest.mark.parametrize("bs", [16, 32, 48, 256, 512])
def test_random_steps_match_oracle(bs):
    announce(f"metadata: random steps, block size {bs}")
    rng = np.random.default_rng(bs)
    for _ in range(12):
        dseqs, pseqs = random_step(rng, bs, int(rng.integers(0, 40)), int(rng.integers(0, 6)),
                                   warm_frac=0.15, spare_blocks=int(rng.integers(0, 3)))
        if dseqs or pseqs:
            check_step(dseqs, pseqs, bs)


def test_single_kind_steps_and_warmup():
    announce("metadata: decode-only, prefill-only, all-warm-up steps")
    rng = np.random.default_rng(7)
    check_step(*random_step(rng, 256, 64, 0), 256)                  # pure decode (graph path)
    check_step(*random_step(rng, 256, 0, 8), 256)                   # pure prefill
    check_step(*random_step(rng, 256, 0, 5, warm_frac=1.0), 256)    # warm-up: no tables, no slots
    check_step([om.SeqView(1, 0, 1, [3])], [], 256)                 # one token


def test_large_step_and_long_context():
    """2,048 sequences (the limit), and 32 sequences of up to 128K tokens."""
    announce("metadata: 2,048 sequences; 128K-token contexts")
    rng = np.random.default_rng(11)
    check_step(*random_step(rng, 256, 1900, 148, max_len=5000, warm_frac=0.05), 256)
    check_step(*random_step(rng, 256, 24, 8, max_len=128 * 1024), 256)


def test_prepare_sequence_device_sets_the_context():
    announce("metadata: prepare_sequence_device publishes the Context")
    rng = np.random.default_rng(3)
    dseqs, pseqs = random_step(rng, 256, 10, 3)
    want = om.prepare_sequence(dseqs, pseqs, 256)
    positions = nm.prepare_sequence_device(dseqs, pseqs, 256, ctxmod.set_context)
    c = ctxmod.get_context()
    torch.cuda.synchronize()
    assert positions.cpu().tolist() == want["positions"]
    assert c.slot_mapping.cpu().tolist() == want["slot_mapping"] and c.split_pt == want["split_pt"]
    assert c.block_tables.cpu().tolist() == want["block_tables"]
    ctxmod.reset_context()


def test_plain_row_without_a_table_gets_slot_minus_one():
    """The C ABI accepts a plain decode descriptor with table_len 0 (pack_step
    rejects it, as the reference's block_table[-1] would fail): its slot
    entry is written as -1, so a store skips it, instead of left unset."""
    announce("metadata: plain decode descriptor without a table")
    seqs = [om.SeqView(300, 299, 1, [7, 9]), om.SeqView(40, 39, 1, [11])]
    step = nm.pack_step(seqs, [], 256)
    desc = step.packed[:8].reshape(2, 4).copy()
    desc[1, 3] = 0                                    # second row: no table
    packed = np.concatenate([desc.reshape(-1), step.packed[8:10]]).astype(np.int32)
    bad = nm.PackedStep(packed=packed, num_seqs=2, num_plain=2, num_spec=0, num_tokens=2, num_slots=2,
                        num_table_rows=1, max_table_len=2, max_seqlen_q=0, max_seqlen_k=0, num_spec_rows=0)
    for _ in range(3):   # the slot buffer comes from the caching allocator, so it holds old values
        got = nm.build_device_metadata(bad, 256)
        torch.cuda.synchronize()
        assert got["slot_mapping"].cpu().tolist() == [9 * 256 + 43, -1]
        assert got["positions"].cpu().tolist() == [299, 39]
        assert got["context_lens"].cpu().tolist() == [300, 40]
        assert got["block_tables"].cpu().tolist() == [[7, 9]]
