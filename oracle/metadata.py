"""Oracle: host attention metadata, restated with plain Python loops (TEST INFRASTRUCTURE ONLY).

Follows nanovllm/engine/model_runner.py:133-220 line by line in behaviour:

* prepare_decode (:188-201): per plain-decode sequence, ``positions = len-1``,
  ``context_lens = len`` and ``slot = block_table[-1] * bs +
  last_block_num_tokens - 1`` with ``last_block_num_tokens = len -
  (num_blocks - 1) * bs`` (nanovllm/engine/sequence.py:58-64).
* prepare_prefill (:144-186): per varlen sequence (speculative decode rows
  first, then prefill chunks), ``start = num_cached_tokens``, ``end = start +
  num_scheduled_tokens``; ``cu_seqlens_q`` accumulates ``end - start``,
  ``cu_seqlens_k`` accumulates ``end``; slots walk the blocks
  ``[start // bs, ceil(end / bs))`` (:172-182); a sequence with an empty
  block table (warm-up) contributes no slots (:170-171).
* prepare_sequence (:203-220): plain decode sequences (``num_scheduled_tokens
  == 1``) come first, then speculative ones, then prefill chunks; block
  tables follow that order, padded with -1 to the longest table (:133-142);
  ``split_pt`` is the number of plain decode sequences.
* the pure-decode graph buffers (:244-248, :300-305): slot_mapping padded
  with -1, context_lens with 0, block tables written into a zero-initialised
  ``[max_bs, max_num_blocks]`` buffer.
"""
from dataclasses import dataclass, field


@dataclass
class SeqView:
    """The fields of nanovllm's Sequence that the attention metadata reads."""
    num_tokens: int
    num_cached_tokens: int = 0
    num_scheduled_tokens: int = 1
    block_table: list = field(default_factory=list)
    block_size: int = 256

    @property
    def num_blocks(self):
        return (self.num_tokens + self.block_size - 1) // self.block_size

    @property
    def last_block_num_tokens(self):
        return self.num_tokens - (self.num_blocks - 1) * self.block_size


def prepare_decode(seqs, block_size):
    positions, slot_mapping, context_lens = [], [], []
    for seq in seqs:
        positions.append(seq.num_tokens - 1)
        context_lens.append(seq.num_tokens)
        slot_mapping.append(seq.block_table[-1] * block_size + seq.last_block_num_tokens - 1)
    return positions, slot_mapping, context_lens


def prepare_prefill(seqs, block_size):
    positions, slot_mapping = [], []
    cu_q, cu_k = [0], [0]
    max_q = max_k = 0
    for seq in seqs:
        start = seq.num_cached_tokens
        seqlen_q = seq.num_scheduled_tokens
        end = start + seqlen_q
        seqlen_k = end
        positions.extend(range(start, end))
        cu_q.append(cu_q[-1] + seqlen_q)
        cu_k.append(cu_k[-1] + seqlen_k)
        max_q = max(seqlen_q, max_q)
        max_k = max(seqlen_k, max_k)
        if not seq.block_table:
            continue
        start_block = start // block_size
        end_block = (end + block_size - 1) // block_size
        for i in range(start_block, end_block):
            slot_start = seq.block_table[i] * block_size
            if i == start_block:
                slot_start += start % block_size
            if i != end_block - 1:
                slot_end = seq.block_table[i] * block_size + block_size
            else:
                slot_end = seq.block_table[i] * block_size + end - i * block_size
            slot_mapping.extend(range(slot_start, slot_end))
    return positions, slot_mapping, cu_q, cu_k, max_q, max_k


def prepare_block_tables(seqs):
    max_len = max((len(seq.block_table) if seq.block_table else 0) for seq in seqs) if seqs else 0
    rows = []
    for seq in seqs:
        if seq.block_table:
            rows.append(list(seq.block_table) + [-1] * (max_len - len(seq.block_table)))
    return rows or None


def prepare_sequence(dseqs, pseqs, block_size):
    """Returns a dict with the same fields nanovllm's Context receives."""
    nd = [s for s in dseqs if s.num_scheduled_tokens == 1]
    sd = [s for s in dseqs if s.num_scheduled_tokens > 1]
    dpos, dslot, ctx_lens = prepare_decode(nd, block_size) if nd else ([], [], [])
    varlen = sd + pseqs
    if varlen:
        ppos, pslot, cu_q, cu_k, max_q, max_k = prepare_prefill(varlen, block_size)
    else:
        ppos, pslot, cu_q, cu_k, max_q, max_k = [], [], None, None, 0, 0
    return dict(
        positions=dpos + ppos,
        slot_mapping=dslot + pslot,
        context_lens=ctx_lens if nd else None,
        cu_seqlens_q=cu_q, cu_seqlens_k=cu_k,
        max_seqlen_q=max_q, max_seqlen_k=max_k,
        block_tables=prepare_block_tables(nd + sd + pseqs),
        split_pt=len(nd), num_spec_seqs=len(sd),
    )


def graph_decode_buffers(slot_mapping, context_lens, block_tables, max_bs, max_num_blocks):
    """Static decode-graph inputs after one replay's copies (model_runner.py:242-248)."""
    bs = len(slot_mapping)
    slots = [-1] * max_bs
    ctx = [0] * max_bs
    table = [[0] * max_num_blocks for _ in range(max_bs)]
    for i in range(bs):
        slots[i] = slot_mapping[i]
        ctx[i] = context_lens[i]
        for j, blk in enumerate(block_tables[i]):
            table[i][j] = blk
    return slots, ctx, table
