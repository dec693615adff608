"""Pure-decode HIP-graph capture (nanovllm/engine/model_runner.py:233-250, 294-329):
store + decode captured per batch size, replayed with new metadata, must
equal eager execution on every replay."""
import pytest
import torch

from gpu_util import announce
import workloads as W
from nanovllm_amd.engine.graph import DecodeGraphRunner
from attention_layer import Attention
from nanovllm_amd.utils.context import get_context, reset_context, set_context

pytestmark = pytest.mark.gpu
SCALE = 128 ** -0.5


class TinyAttnStack(torch.nn.Module):
    """Embedding lookups -> L x (elementwise q/k/v, FP8 Attention).  Only row-wise
    ops besides the attention kernels, so eager and replay are bit-comparable
    whatever batch size the graph was captured for."""

    def __init__(self, L, Hq, Hkv, vocab=512):
        super().__init__()
        g = torch.Generator().manual_seed(0)
        self.Hq, self.Hkv, self.L = Hq, Hkv, L
        self.eq = torch.nn.Parameter(torch.randn(L, vocab, Hq * 128, generator=g).to(torch.bfloat16), requires_grad=False)
        self.ek = torch.nn.Parameter(torch.randn(L, vocab, Hkv * 128, generator=g).to(torch.bfloat16), requires_grad=False)
        self.ev = torch.nn.Parameter(torch.randn(L, vocab, Hkv * 128, generator=g).to(torch.bfloat16), requires_grad=False)
        self.attn = torch.nn.ModuleList([Attention(Hq, 128, SCALE) for _ in range(L)])

    def forward(self, input_ids, positions):
        B = input_ids.shape[0]
        h = torch.zeros(B, self.Hq * 128, dtype=torch.bfloat16, device=input_ids.device)
        kvw = self.Hkv * 128
        for l, attn in enumerate(self.attn):
            q = self.eq[l][input_ids] + h
            k = self.ek[l][input_ids] + h[:, :kvw]
            v = self.ev[l][input_ids] - h[:, :kvw]
            o = attn(q.view(B, self.Hq, 128), k.view(B, self.Hkv, 128), v.view(B, self.Hkv, 128))
            h = h + 0.5 * o.reshape(B, -1)
        return h


def _setup(model, L, P, bs=256):
    kv = torch.zeros(2, L, P, bs, model.Hkv, 128, dtype=torch.uint8, device="cuda").view(torch.float8_e4m3fn)
    kv.view(torch.uint8).random_(0, 0x78)
    for l, attn in enumerate(model.attn):
        attn.k_cache, attn.v_cache = kv[0, l], kv[1, l]
    return kv


def _step_inputs(wl, B):
    ctx = torch.from_numpy(wl.context_lens()[:B]).cuda()
    bt = torch.from_numpy(wl.block_tables[:B]).cuda()
    slot = torch.tensor([wl.slots_for(i, s.lk - 1, s.lk)[0] for i, s in enumerate(wl.seqs[:B])],
                        dtype=torch.int32, device="cuda")
    ids = torch.randint(0, 512, (B,), device="cuda")
    pos = ctx.long() - 1
    return ids, pos, slot, ctx, bt


def _replay_vs_eager(model, runner, kv, wl, B, reps=3):
    for rep in range(reps):
        ids, pos, slot, ctx, bt = _step_inputs(wl, B)
        ctx = torch.clamp(ctx - rep * 7, min=1)          # mutate contexts between replays
        slot = slot - 0                                   # same slots
        snapshot = kv.clone()
        set_context(split_pt=B, slot_mapping=slot, context_lens=ctx, block_tables=bt)
        with torch.inference_mode():
            eager = model(ids, pos)
        kv_eager = kv.clone()
        kv.copy_(snapshot)
        replayed = runner.replay(ids, pos).clone()
        torch.cuda.synchronize()
        reset_context()
        assert torch.equal(kv.view(torch.uint8), kv_eager.view(torch.uint8)), f"cache differs (replay {rep})"
        assert torch.equal(replayed, eager), f"replay {rep} differs from eager"


@pytest.mark.parametrize("B", [3, 16, 40])
def test_graph_replay_matches_eager(B):
    announce(f"graph: capture + replay B={B}")
    L, Hq, Hkv = 2, 16, 8
    model = TinyAttnStack(L, Hq, Hkv).cuda()
    wl = W.qwen3_0p6b_decode(B=64)
    max_nb = 8  # 2048 tokens
    runner = DecodeGraphRunner(model, max_bs=48, max_num_blocks=max_nb, hidden_size=Hq * 128)
    kv = _setup(model, L, wl.num_blocks)
    runner.capture()
    _replay_vs_eager(model, runner, kv, wl, B)


def test_graph_replay_qwen3_8b_headline_shapes():
    """The reference's capture list up to max_bs = 256 (1, 2, 4, 8, 16, ..., 256,
    model_runner.py:306) at Qwen3-8B heads (32/8) with 16-block tables (4,096
    tokens at block size 256); a 192-row step (the headline decode batch,
    context U[256, 4096]) replays the 192 graph and must equal eager, on three
    replays with mutated context lengths; then a 100-row step pads into the
    112 graph."""
    announce("graph: capture 1..256 at 32/8 heads, max_num_blocks 16; replay B=192 and B=100")
    L, Hq, Hkv = 2, 32, 8
    model = TinyAttnStack(L, Hq, Hkv).cuda()
    wl = W.qwen3_8b_decode()
    assert wl.num_seqs == 192 and wl.block_tables.shape[1] <= 16
    runner = DecodeGraphRunner(model, max_bs=256, max_num_blocks=16, hidden_size=Hq * 128)
    assert runner.graph_bs == [1, 2, 4, 8] + list(range(16, 257, 16))
    kv = _setup(model, L, wl.num_blocks)
    runner.capture()
    assert runner.pick(192) == 192 and runner.pick(100) == 112
    _replay_vs_eager(model, runner, kv, wl, 192)
    _replay_vs_eager(model, runner, kv, wl, 100, reps=1)
