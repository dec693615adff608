"""Pure-decode HIP-graph capture and replay.

Restates the pure-decode graph path of nanovllm/engine/model_runner.py
(capture: :294-329, replay: :233-250) around any ``forward(input_ids,
positions) -> hidden`` that reads its attention metadata from the Context
(the FP8 store + decode kernels are launched inside it).  On ROCm,
``torch.cuda.CUDAGraph`` records a hipGraph; the kernels here use static
grids that depend only on tensor shapes, never on device values, so one
graph per batch size replays any contexts that fit ``max_num_blocks``.

Static buffers and padding match the reference: ``slot_mapping`` is filled
with -1 and ``context_lens`` zeroed before each replay's copies (padding rows
store nothing and attend to nothing -- the decode kernel writes zeros for
them), and ``block_tables`` is a zero-initialised ``[max_bs, max_num_blocks]``
buffer whose first columns are overwritten.
"""
import torch

from ..utils.context import get_context, reset_context, set_context


def graph_batch_sizes(max_bs):
    """1, 2, 4, 8, then multiples of 16 up to max_bs (model_runner.py:306)."""
    return [b for b in (1, 2, 4, 8) if b <= max_bs] + list(range(16, max_bs + 1, 16))


class DecodeGraphRunner:

    def __init__(self, forward, max_bs, max_num_blocks, hidden_size, dtype=torch.bfloat16,
                 device="cuda"):
        self.forward = forward
        self.max_bs = max_bs
        self.max_num_blocks = max_num_blocks
        dev = torch.device(device)
        self.vars = dict(
            input_ids=torch.zeros(max_bs, dtype=torch.int64, device=dev),
            positions=torch.zeros(max_bs, dtype=torch.int64, device=dev),
            slot_mapping=torch.zeros(max_bs, dtype=torch.int32, device=dev),
            context_lens=torch.zeros(max_bs, dtype=torch.int32, device=dev),
            block_tables=torch.zeros(max_bs, max_num_blocks, dtype=torch.int32, device=dev),
            outputs=torch.zeros(max_bs, hidden_size, dtype=dtype, device=dev),
        )
        self.graph_bs = graph_batch_sizes(max_bs)
        self.graphs = {}
        self.pool = None

    @torch.inference_mode()
    def capture(self):
        v = self.vars
        for bs in reversed(self.graph_bs):
            graph = torch.cuda.CUDAGraph()
            set_context(split_pt=bs, slot_mapping=v["slot_mapping"][:bs],
                        context_lens=v["context_lens"][:bs], block_tables=v["block_tables"][:bs])
            v["outputs"][:bs] = self.forward(v["input_ids"][:bs], v["positions"][:bs])  # warm-up
            with torch.cuda.graph(graph, self.pool):
                v["outputs"][:bs] = self.forward(v["input_ids"][:bs], v["positions"][:bs])
            if self.pool is None:
                self.pool = graph.pool()
            self.graphs[bs] = graph
            torch.cuda.synchronize()
            reset_context()
        return self

    def pick(self, bs):
        return next(x for x in self.graph_bs if x >= bs)

    @torch.inference_mode()
    def replay(self, input_ids, positions):
        """Runs a pure-decode step whose metadata is already in the Context."""
        bs = input_ids.size(0)
        if bs > self.max_bs:
            raise ValueError(f"batch {bs} exceeds the captured maximum {self.max_bs}")
        ctx = get_context()
        if ctx.block_tables.size(1) > self.max_num_blocks:
            raise ValueError("block table wider than the captured max_num_blocks")
        v = self.vars
        graph = self.graphs[self.pick(bs)]
        v["input_ids"][:bs] = input_ids
        v["positions"][:bs] = positions
        v["slot_mapping"].fill_(-1)
        v["slot_mapping"][:bs] = ctx.slot_mapping
        v["context_lens"].zero_()
        v["context_lens"][:bs] = ctx.context_lens
        v["block_tables"][:bs, :ctx.block_tables.size(1)] = ctx.block_tables
        graph.replay()
        return v["outputs"][:bs]
