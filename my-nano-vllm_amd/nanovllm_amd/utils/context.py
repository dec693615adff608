"""Per-step attention metadata handed from the runner to the attention layers.

Same fields, defaults and setter semantics as nanovllm/utils/context.py:5-48:
``split_pt`` separates plain-decode rows (before) from varlen rows (after),
``num_spec_seqs`` counts the speculative sequences at the front of the varlen
group, and the tensors are int32 device tensors (block tables padded with -1).
One field is added to the reference's: ``num_spec_rows``, the host-side count
of the speculative sequences' query rows (``cu_seqlens_q[num_spec_seqs]``),
which the metadata builders know; -1 when unknown.
"""
from dataclasses import dataclass

import torch


@dataclass(slots=True)
class Context:
    split_pt: int = 0
    num_spec_seqs: int = 0
    cu_seqlens_q: torch.Tensor | None = None
    cu_seqlens_k: torch.Tensor | None = None
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    slot_mapping: torch.Tensor | None = None
    context_lens: torch.Tensor | None = None
    block_tables: torch.Tensor | None = None
    num_spec_rows: int = -1


_CONTEXT = Context()
_UNSET = object()
_FIELDS = Context.__slots__


def get_context() -> Context:
    return _CONTEXT


def set_context(split_pt=_UNSET, num_spec_seqs=_UNSET, cu_seqlens_q=_UNSET, cu_seqlens_k=_UNSET,
                max_seqlen_q=_UNSET, max_seqlen_k=_UNSET, slot_mapping=_UNSET,
                context_lens=_UNSET, block_tables=_UNSET, num_spec_rows=_UNSET):
    """Updates only the fields that are passed (unpassed fields keep their value)."""
    values = dict(split_pt=split_pt, num_spec_seqs=num_spec_seqs, cu_seqlens_q=cu_seqlens_q,
                  cu_seqlens_k=cu_seqlens_k, max_seqlen_q=max_seqlen_q, max_seqlen_k=max_seqlen_k,
                  slot_mapping=slot_mapping, context_lens=context_lens, block_tables=block_tables,
                  num_spec_rows=num_spec_rows)
    for name, value in values.items():
        if value is not _UNSET:
            setattr(_CONTEXT, name, value)


def reset_context():
    fresh = Context()
    for name in _FIELDS:
        setattr(_CONTEXT, name, getattr(fresh, name))
