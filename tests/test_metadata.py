"""Host attention metadata (nanovllm/engine/model_runner.py:133-220): the
package's numpy builder must equal the loop-for-loop oracle byte for byte,
and both must satisfy the closed forms."""
import numpy as np
from hypothesis import given, settings, strategies as st

from oracle import metadata as om
from nanovllm_amd.engine import metadata as nm
from nanovllm_amd.utils import context as ctxmod

BS = 256


@st.composite
def batches(draw):
    rng_blocks = draw(st.permutations(list(range(400))))
    pool = iter(rng_blocks)
    dseqs, pseqs = [], []
    for _ in range(draw(st.integers(0, 6))):            # decode (maybe speculative)
        n_tok = draw(st.integers(1, 3000))
        drafts = draw(st.integers(0, 4))
        nb = -(-(n_tok + drafts) // BS)
        table = [next(pool) for _ in range(nb)]
        if drafts == 0:
            seq = om.SeqView(num_tokens=n_tok, num_cached_tokens=n_tok - 1,
                             num_scheduled_tokens=1, block_table=table[: -(-n_tok // BS)])
        else:
            seq = om.SeqView(num_tokens=n_tok, num_cached_tokens=n_tok - 1,
                             num_scheduled_tokens=1 + drafts, block_table=table)
        dseqs.append(seq)
    for _ in range(draw(st.integers(0, 4))):            # prefill chunks
        n_tok = draw(st.integers(1, 3000))
        cached = draw(st.integers(0, n_tok - 1))
        lq = draw(st.integers(1, n_tok - cached))
        warm = draw(st.booleans()) and draw(st.booleans()) and draw(st.booleans())
        table = [] if warm else [next(pool) for _ in range(-(-n_tok // BS))]
        pseqs.append(om.SeqView(num_tokens=n_tok, num_cached_tokens=cached,
                                num_scheduled_tokens=lq, block_table=table))
    return dseqs, pseqs


@settings(max_examples=200, deadline=None)
@given(batches())
def test_builder_matches_oracle(batch):
    dseqs, pseqs = batch
    if not dseqs and not pseqs:
        return
    want = om.prepare_sequence(dseqs, pseqs, BS)
    got = nm.build_host_metadata(dseqs, pseqs, BS)
    assert got.positions.tolist() == want["positions"]
    assert got.slot_mapping.dtype == np.int32
    assert got.slot_mapping.tolist() == want["slot_mapping"]
    assert got.split_pt == want["split_pt"] and got.num_spec_seqs == want["num_spec_seqs"]
    if want["context_lens"] is None:
        assert got.context_lens.size == 0
    else:
        assert got.context_lens.tolist() == want["context_lens"]
    if want["cu_seqlens_q"] is None:
        assert got.cu_seqlens_q.size == 0
    else:
        assert got.cu_seqlens_q.tolist() == want["cu_seqlens_q"]
        assert got.cu_seqlens_k.tolist() == want["cu_seqlens_k"]
    assert (got.max_seqlen_q, got.max_seqlen_k) == (want["max_seqlen_q"], want["max_seqlen_k"])
    if want["block_tables"] is None:
        assert got.block_tables is None
    else:
        assert got.block_tables.tolist() == want["block_tables"]


@settings(max_examples=100, deadline=None)
@given(batches())
def test_slot_closed_form(batch):
    """slot(p) = bt[p // bs] * bs + p % bs for every scheduled position."""
    dseqs, pseqs = batch
    varlen = [s for s in dseqs if s.num_scheduled_tokens > 1] + pseqs
    plain = [s for s in dseqs if s.num_scheduled_tokens == 1]
    md = nm.build_host_metadata(dseqs, pseqs, BS)
    o = len(plain)
    for s in plain:
        assert md.slot_mapping[plain.index(s)] == s.block_table[(s.num_tokens - 1) // BS] * BS + (s.num_tokens - 1) % BS
    for s in varlen:
        if not s.block_table:
            continue
        for p in range(s.num_cached_tokens, s.num_cached_tokens + s.num_scheduled_tokens):
            assert md.slot_mapping[o] == s.block_table[p // BS] * BS + p % BS
            o += 1
    assert o == len(md.slot_mapping)


def test_graph_buffer_padding():
    slots, ctx, table = om.graph_decode_buffers([5, 700], [6, 1000], [[0], [2, 7, 9, 1]], 4, 8)
    assert slots == [5, 700, -1, -1] and ctx == [6, 1000, 0, 0]
    assert table[1][:4] == [2, 7, 9, 1] and table[2] == [0] * 8


def test_context_set_and_reset():
    ctxmod.reset_context()
    ctxmod.set_context(split_pt=3, max_seqlen_q=9)
    c = ctxmod.get_context()
    assert c.split_pt == 3 and c.max_seqlen_q == 9 and c.block_tables is None
    ctxmod.set_context(num_spec_seqs=2)
    assert c.split_pt == 3 and c.num_spec_seqs == 2     # unpassed fields keep their value
    ctxmod.reset_context()
    assert c.split_pt == 0 and c.num_spec_seqs == 0 and c.max_seqlen_q == 0


@settings(max_examples=200, deadline=None)
@given(batches())
def test_pack_step_sizes_match_oracle(batch):
    """The on-device build's upload: descriptors in the reference's row order,
    tables back to back, and output sizes equal to the oracle's lengths."""
    dseqs, pseqs = batch
    if not dseqs and not pseqs:
        return
    want = om.prepare_sequence(dseqs, pseqs, BS)
    st_ = nm.pack_step(dseqs, pseqs, BS)
    order = [s for s in dseqs if s.num_scheduled_tokens == 1] + \
            [s for s in dseqs if s.num_scheduled_tokens > 1] + pseqs
    desc = st_.packed[:4 * len(order)].reshape(-1, 4)
    assert desc.tolist() == [[s.num_tokens, s.num_cached_tokens, s.num_scheduled_tokens, len(s.block_table)]
                             for s in order]
    assert st_.packed[4 * len(order):].tolist() == [b for s in order for b in s.block_table]
    assert st_.num_tokens == len(want["positions"]) and st_.num_slots == len(want["slot_mapping"])
    assert st_.num_plain == want["split_pt"] and st_.num_spec == want["num_spec_seqs"]
    rows = want["block_tables"] or []
    assert st_.num_table_rows == len(rows) and (not rows or st_.max_table_len == len(rows[0]))
    assert (st_.max_seqlen_q, st_.max_seqlen_k) == (want["max_seqlen_q"], want["max_seqlen_k"])


def test_pack_step_rejects_what_the_reference_cannot_index():
    import pytest
    with pytest.raises(ValueError, match="plain decode"):
        nm.pack_step([om.SeqView(10, 9, 1, [])], [], BS)
    with pytest.raises(ValueError, match="does not cover"):
        nm.pack_step([], [om.SeqView(600, 0, 600, [1, 2])], BS)
