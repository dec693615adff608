"""Host-side attention metadata: slot mapping, cu_seqlens, context lengths, block tables.

Behaviour of nanovllm/engine/model_runner.py:133-220, built per sequence with
numpy instead of per-token Python loops, then copied to the GPU from pinned
memory with non-blocking copies (as the reference does, :141, :183-184,
:199, :211-213):

* plain decode sequences (``num_scheduled_tokens == 1``, :205):
  ``position = len - 1``, ``context_len = len`` and
  ``slot = block_table[-1] * bs + last_block_num_tokens - 1`` (:195-198);
* varlen sequences (speculative-decode rows first, then prefill chunks,
  :206-209): query positions ``[num_cached, num_cached + num_scheduled)``,
  ``cu_seqlens_q`` / ``cu_seqlens_k`` prefix sums of ``num_scheduled`` and of
  ``num_cached + num_scheduled`` (:166-167) and, for every scheduled position
  p, ``slot = block_table[p // bs] * bs + p % bs`` (the block walk of
  :172-182); a sequence without a block table contributes no slots (:170);
* block tables in [plain decode | speculative | prefill] order, padded with
  -1 to the longest table (:133-142, :216).

``Seq``-like inputs need ``len(seq)``, ``num_cached_tokens``,
``num_scheduled_tokens`` and ``block_table`` -- nano-vLLM's ``Sequence``
qualifies.

``prepare_sequence_device`` builds the same tensors on the GPU instead: the
host packs one int32 descriptor per sequence ``{num_tokens, num_cached,
num_scheduled, len(block_table)}`` and the block tables back to back (work in
the number of sequences and blocks, none per token), uploads it with one
pinned non-blocking copy, and ``nvamd_build_attention_metadata`` expands it
into positions, slot mapping, context lengths, cu_seqlens and the padded
block tables.

Both builders publish the step through the ``set_context`` they are given:
the caller names the Context its attention and LM-head layers read.  Inside
nano-vLLM's runner that is ``nanovllm.utils.context.set_context``; the
package's own ``nanovllm_amd.utils.context.set_context`` also receives the
host-side ``num_spec_rows``.  There is no default, so a step is never
published to a Context nobody reads.
"""
import itertools
from dataclasses import dataclass

import numpy as np
import torch

from ..utils import context as _pkg_context

# the fields of nanovllm/utils/context.py:5-15 (what any Context accepts)
_REFERENCE_FIELDS = ("split_pt", "num_spec_seqs", "cu_seqlens_q", "cu_seqlens_k", "max_seqlen_q", "max_seqlen_k",
                     "slot_mapping", "context_lens", "block_tables")


def _publish(set_context, fields, num_spec_rows):
    if not callable(set_context):
        raise TypeError("set_context must be the Context setter the step's layers read "
                        "(nanovllm.utils.context.set_context inside nano-vLLM's runner)")
    values = {k: fields[k] for k in _REFERENCE_FIELDS}
    if set_context is _pkg_context.set_context:
        values["num_spec_rows"] = num_spec_rows
    set_context(**values)


def _seq_len(seq):
    return len(seq) if hasattr(seq, "__len__") else int(seq.num_tokens)


@dataclass
class HostMetadata:
    """Host (numpy) form of one step's attention metadata."""
    positions: np.ndarray          # int64 [num_tokens]
    slot_mapping: np.ndarray       # int32 [num_tokens]
    context_lens: np.ndarray       # int32 [num_plain_decode]
    cu_seqlens_q: np.ndarray       # int32 [num_varlen + 1] (empty if no varlen rows)
    cu_seqlens_k: np.ndarray
    max_seqlen_q: int
    max_seqlen_k: int
    block_tables: np.ndarray       # int32 [num_seqs_with_tables, max_len] (-1 padded) or None
    split_pt: int
    num_spec_seqs: int


def decode_rows(seqs, block_size):
    n = len(seqs)
    lens = np.fromiter((_seq_len(s) for s in seqs), dtype=np.int64, count=n)
    last_blk = np.fromiter((s.block_table[-1] for s in seqs), dtype=np.int64, count=n)
    num_blocks = (lens + block_size - 1) // block_size
    last_block_tokens = lens - (num_blocks - 1) * block_size
    slots = last_blk * block_size + last_block_tokens - 1
    return lens - 1, slots.astype(np.int32), lens.astype(np.int32)


def varlen_rows(seqs, block_size):
    starts = np.array([s.num_cached_tokens for s in seqs], dtype=np.int64)
    lq = np.array([s.num_scheduled_tokens for s in seqs], dtype=np.int64)
    ends = starts + lq
    cu_q = np.zeros(len(seqs) + 1, dtype=np.int64)
    cu_k = np.zeros(len(seqs) + 1, dtype=np.int64)
    np.cumsum(lq, out=cu_q[1:])
    np.cumsum(ends, out=cu_k[1:])
    positions = np.concatenate([np.arange(a, b, dtype=np.int64) for a, b in zip(starts, ends)]) \
        if len(seqs) else np.zeros(0, dtype=np.int64)
    slot_parts = []
    for s, a, b in zip(seqs, starts, ends):
        if not s.block_table:
            continue
        pos = np.arange(a, b, dtype=np.int64)
        table = np.asarray(s.block_table, dtype=np.int64)
        slot_parts.append(table[pos // block_size] * block_size + pos % block_size)
    slots = np.concatenate(slot_parts).astype(np.int32) if slot_parts else np.zeros(0, dtype=np.int32)
    max_q = int(lq.max()) if len(seqs) else 0
    max_k = int(ends.max()) if len(seqs) else 0
    return positions, slots, cu_q.astype(np.int32), cu_k.astype(np.int32), max_q, max_k


def padded_block_tables(seqs):
    tables = [s.block_table for s in seqs if s.block_table]
    if not tables:
        return None
    width = max(len(t) for t in tables)
    out = np.full((len(tables), width), -1, dtype=np.int32)
    for i, t in enumerate(tables):
        out[i, :len(t)] = t
    return out


def build_host_metadata(dseqs, pseqs, block_size) -> HostMetadata:
    nd = [s for s in dseqs if s.num_scheduled_tokens == 1]
    sd = [s for s in dseqs if s.num_scheduled_tokens > 1]
    varlen = sd + list(pseqs)
    if nd:
        dpos, dslot, ctx = decode_rows(nd, block_size)
    else:
        dpos, dslot, ctx = (np.zeros(0, np.int64), np.zeros(0, np.int32), np.zeros(0, np.int32))
    if varlen:
        ppos, pslot, cu_q, cu_k, max_q, max_k = varlen_rows(varlen, block_size)
    else:
        ppos, pslot = np.zeros(0, np.int64), np.zeros(0, np.int32)
        cu_q = cu_k = np.zeros(0, np.int32)
        max_q = max_k = 0
    return HostMetadata(
        positions=np.concatenate([dpos, ppos]),
        slot_mapping=np.concatenate([dslot, pslot]).astype(np.int32),
        context_lens=ctx, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k,
        max_seqlen_q=max_q, max_seqlen_k=max_k,
        block_tables=padded_block_tables(nd + sd + list(pseqs)),
        split_pt=len(nd), num_spec_seqs=len(sd))


def _to_device(arr, device):
    if arr is None:
        return None
    t = torch.from_numpy(np.ascontiguousarray(arr))
    if torch.device(device).type == "cuda":
        return t.pin_memory().to(device, non_blocking=True)
    return t.to(device)


def prepare_sequence(dseqs, pseqs, block_size, set_context, device="cuda"):
    """Builds the step's metadata, publishes it through ``set_context`` and
    returns the device positions (model_runner.prepare_sequence, :203-220)."""
    md = build_host_metadata(dseqs, pseqs, block_size)
    has_varlen = md.cu_seqlens_q.size > 0
    num_spec_rows = sum(s.num_scheduled_tokens for s in dseqs if s.num_scheduled_tokens > 1)
    _publish(set_context, dict(
        split_pt=md.split_pt, num_spec_seqs=md.num_spec_seqs,
        slot_mapping=_to_device(md.slot_mapping, device),
        context_lens=_to_device(md.context_lens, device) if md.split_pt else None,
        cu_seqlens_q=_to_device(md.cu_seqlens_q, device) if has_varlen else None,
        cu_seqlens_k=_to_device(md.cu_seqlens_k, device) if has_varlen else None,
        max_seqlen_q=md.max_seqlen_q, max_seqlen_k=md.max_seqlen_k,
        block_tables=_to_device(md.block_tables, device)), num_spec_rows)
    return _to_device(md.positions, device)


@dataclass
class PackedStep:
    """One step's upload for the on-device build and the output sizes it implies."""
    packed: np.ndarray       # int32: [num_seqs, 4] descriptors, then the block tables back to back
    num_seqs: int
    num_plain: int
    num_spec: int
    num_tokens: int          # positions
    num_slots: int           # slot_mapping entries
    num_table_rows: int      # sequences with a non-empty block table
    max_table_len: int
    max_seqlen_q: int
    max_seqlen_k: int
    num_spec_rows: int       # query rows of the speculative sequences


def pack_step(dseqs, pseqs, block_size) -> PackedStep:
    """Orders the sequences as the reference does (plain decode, speculative,
    prefill: model_runner.py:205-216) and packs their descriptors and block
    tables.  Raises where the reference's loops would fail: a plain decode
    sequence without a block table (``block_table[-1]``, :198), or a varlen
    sequence whose table does not cover its scheduled positions (:175-181)."""
    nd = [s for s in dseqs if s.num_scheduled_tokens == 1]
    sd = [s for s in dseqs if s.num_scheduled_tokens > 1]
    seqs = nd + sd + list(pseqs)
    n = len(seqs)
    desc = np.empty((n, 4), dtype=np.int64)
    desc[:, 0] = np.fromiter((_seq_len(s) for s in seqs), dtype=np.int64, count=n)
    desc[:, 1] = np.fromiter((s.num_cached_tokens for s in seqs), dtype=np.int64, count=n)
    desc[:, 2] = np.fromiter((s.num_scheduled_tokens for s in seqs), dtype=np.int64, count=n)
    desc[:, 3] = np.fromiter((len(s.block_table) if s.block_table else 0 for s in seqs), dtype=np.int64, count=n)
    n_plain = len(nd)
    tl = desc[:, 3]
    if n_plain and (tl[:n_plain] == 0).any():
        raise ValueError("a plain decode sequence has no block table")
    var = desc[n_plain:]
    ends = var[:, 1] + var[:, 2]
    has = var[:, 3] > 0
    if (has & ((ends + block_size - 1) // block_size > var[:, 3])).any():
        raise ValueError("a varlen sequence's block table does not cover its scheduled positions")
    total = int(tl.sum())
    tables = np.fromiter(itertools.chain.from_iterable(s.block_table for s in seqs if s.block_table),
                         dtype=np.int32, count=total)
    packed = np.concatenate([desc.astype(np.int32).reshape(-1), tables])
    return PackedStep(
        packed=packed, num_seqs=n, num_plain=n_plain, num_spec=len(sd),
        num_tokens=n_plain + int(var[:, 2].sum()),
        num_slots=n_plain + int(var[has, 2].sum()),
        num_table_rows=int((tl > 0).sum()), max_table_len=int(tl.max()) if n else 0,
        max_seqlen_q=int(var[:, 2].max()) if len(var) else 0,
        max_seqlen_k=int(ends.max()) if len(var) else 0,
        num_spec_rows=int(desc[n_plain:n_plain + len(sd), 2].sum()))


def build_device_metadata(step: PackedStep, block_size, device="cuda"):
    """Uploads a packed step and builds its tensors on the GPU (on torch's
    current stream).  Returns a dict with the fields nano-vLLM's Context
    receives plus ``positions``."""
    from .. import _native
    dev = torch.device(device)
    if dev.type != "cuda":
        raise ValueError(f"the on-device build needs a ROCm GPU (got {device})")
    lib = _native.load()
    n_var = step.num_seqs - step.num_plain
    packed = torch.from_numpy(step.packed).pin_memory().to(dev, non_blocking=True)
    i32 = dict(dtype=torch.int32, device=dev)
    positions = torch.empty(step.num_tokens, dtype=torch.int64, device=dev)
    slot_mapping = torch.empty(step.num_slots, **i32)
    context_lens = torch.empty(step.num_plain, **i32) if step.num_plain else None
    cu_q = torch.empty(n_var + 1, **i32) if n_var else None
    cu_k = torch.empty(n_var + 1, **i32) if n_var else None
    tables = torch.empty(step.num_table_rows, step.max_table_len, **i32) if step.num_table_rows else None
    ptr = lambda t: t.data_ptr() if t is not None else None  # noqa: E731
    st = lib.nvamd_build_attention_metadata(
        packed.data_ptr(), packed.numel(), step.num_seqs, step.num_plain, block_size, step.num_tokens,
        step.num_slots, step.num_table_rows, step.max_table_len, positions.data_ptr(), ptr(slot_mapping),
        ptr(context_lens), ptr(cu_q), ptr(cu_k), ptr(tables), torch.cuda.current_stream(dev).cuda_stream)
    _native.check(st, "build_attention_metadata")
    return dict(positions=positions, slot_mapping=slot_mapping, context_lens=context_lens,
                cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, max_seqlen_q=step.max_seqlen_q,
                max_seqlen_k=step.max_seqlen_k, block_tables=tables, split_pt=step.num_plain,
                num_spec_seqs=step.num_spec, num_spec_rows=step.num_spec_rows)


def prepare_sequence_device(dseqs, pseqs, block_size, set_context, device="cuda"):
    """prepare_sequence with the metadata built on the GPU: publishes it
    through ``set_context`` and returns the device positions."""
    md = build_device_metadata(pack_step(dseqs, pseqs, block_size), block_size, device)
    _publish(set_context, md, md["num_spec_rows"])
    return md["positions"]
