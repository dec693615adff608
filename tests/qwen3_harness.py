"""Random-init Qwen3 harness for the greedy-decode check (test infrastructure).

A minimal Qwen3 decoder (the layer structure of nanovllm/models/qwen3.py:
q/k RMSNorm per head, neox RoPE, GQA attention, SiLU-gated MLP, pre-norm
residual blocks, final norm, LM head) whose attention is either

* ``attention_layer.Attention`` (the reference layer over the product path): FP8 KV
  store + HIP decode / prefill kernels on the GPU, or
* ``OracleAttention`` -- the same layer contract computed by the oracle on
  the CPU (oracle store into CPU caches, oracle decode / prefill).

Everything else (weights, linears, norms, RoPE, LM head) is the same bf16 GPU
code for both, so the two runs differ only in the attention implementation.
``GreedyRunner`` schedules sequences like the reference's scheduler does
(decode rows first, chunked prefill up to a per-step chunk, optional
speculative rows with drafts) and builds the step metadata with the product
metadata builder (nanovllm_amd.engine.metadata).
"""
from dataclasses import dataclass, field

import numpy as np
import torch
from torch import nn

from nanovllm_amd.engine.metadata import prepare_sequence
from attention_layer import Attention
from nanovllm_amd.utils.context import get_context, reset_context, set_context
from oracle import attention as oa
from oracle import fp8 as ofp8


@dataclass
class Qwen3TinyConfig:
    vocab_size: int = 2048
    hidden_size: int = 1024
    num_heads: int = 16
    num_kv_heads: int = 8
    head_dim: int = 128
    intermediate_size: int = 2048
    num_layers: int = 2
    rope_theta: float = 1e6
    rms_eps: float = 1e-6
    block_size: int = 256


def rms_norm(x, w, eps):
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (xf * w.float()).to(x.dtype)


class Rope:
    def __init__(self, head_dim, theta, device):
        self.inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=device, dtype=torch.float32) / head_dim))

    def __call__(self, x, positions):
        # x: [N, H, D] bf16; neox style (rotate halves)
        f = positions.float().unsqueeze(-1) * self.inv_freq          # [N, D/2]
        cos, sin = f.cos().unsqueeze(1), f.sin().unsqueeze(1)        # [N, 1, D/2]
        x1, x2 = x.float().chunk(2, dim=-1)
        return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1).to(x.dtype)


class OracleAttention(nn.Module):
    """The FP8 Attention layer contract (nanovllm/layers/attention.py:58-96)
    computed by the oracle on CPU caches."""

    def __init__(self, num_heads, head_dim, scale, k_cache, v_cache):
        super().__init__()
        self.num_heads, self.head_dim, self.scale = num_heads, head_dim, scale
        self.k_cache, self.v_cache = k_cache, v_cache   # uint8 CPU [P, bs, Hkv, D]

    def forward(self, q, k, v):
        ctx = get_context()
        ofp8.store_kvcache(k.cpu(), v.cpu(), self.k_cache, self.v_cache, ctx.slot_mapping.cpu())
        split = ctx.split_pt
        bt = ctx.block_tables.cpu() if ctx.block_tables is not None else None
        outs = []
        if split > 0:
            outs.append(oa.decode_attention(q[:split].cpu(), self.k_cache, self.v_cache, bt[:split],
                                            ctx.context_lens.cpu(), self.scale))
        if q.shape[0] > split:
            outs.append(oa.prefill_attention(q[split:].cpu(), self.k_cache, self.v_cache, bt[split:],
                                             ctx.cu_seqlens_q.cpu(), ctx.cu_seqlens_k.cpu(), self.scale))
        o = outs[0] if len(outs) == 1 else torch.cat(outs, 0)
        return o.to(q.device)


class Qwen3Tiny(nn.Module):
    def __init__(self, cfg: Qwen3TinyConfig, attn_factory, seed=0, device="cuda"):
        super().__init__()
        self.cfg = cfg
        g = torch.Generator(device="cpu").manual_seed(seed)
        H, Hq, Hkv, D, I = cfg.hidden_size, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.intermediate_size

        def w(*shape, std):
            return (torch.randn(*shape, generator=g) * std).to(device=device, dtype=torch.bfloat16)

        # unit-variance projections, so attention moves the residual stream by O(1)
        self.embed = w(cfg.vocab_size, H, std=1.0)
        self.layers = []
        for i in range(cfg.num_layers):
            self.layers.append(dict(
                in_norm=1.0 + w(H, std=0.1), post_norm=1.0 + w(H, std=0.1),
                qkv=w((Hq + 2 * Hkv) * D, H, std=H ** -0.5),
                q_norm=1.0 + w(D, std=0.1), k_norm=1.0 + w(D, std=0.1),
                o=w(H, Hq * D, std=(Hq * D) ** -0.5),
                gate_up=w(2 * I, H, std=H ** -0.5), down=w(H, I, std=I ** -0.5),
                attn=attn_factory(i)))
        self.norm = 1.0 + w(H, std=0.1)
        self.lm_head = w(cfg.vocab_size, H, std=3.0 * H ** -0.5)
        self.rope = Rope(D, cfg.rope_theta, device)
        self.scale = D ** -0.5

    @torch.inference_mode()
    def forward(self, input_ids, positions):
        cfg = self.cfg
        Hq, Hkv, D = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim
        h = self.embed[input_ids]
        for L in self.layers:
            x = rms_norm(h, L["in_norm"], cfg.rms_eps)
            qkv = x @ L["qkv"].T
            q, k, v = qkv.split([Hq * D, Hkv * D, Hkv * D], dim=-1)
            q = rms_norm(q.reshape(-1, Hq, D), L["q_norm"], cfg.rms_eps)
            k = rms_norm(k.reshape(-1, Hkv, D), L["k_norm"], cfg.rms_eps)
            v = v.reshape(-1, Hkv, D)          # strided view of qkv, as in the reference
            q, k = self.rope(q, positions), self.rope(k, positions)
            o = L["attn"](q, k, v)
            h = h + o.reshape(-1, Hq * D) @ L["o"].T
            x = rms_norm(h, L["post_norm"], cfg.rms_eps)
            gu = x @ L["gate_up"].T
            gt, up = gu.chunk(2, dim=-1)
            h = h + (torch.nn.functional.silu(gt.float()) * up.float()).to(h.dtype) @ L["down"].T
        return rms_norm(h, self.norm, cfg.rms_eps)

    def logits(self, hidden):
        return hidden.float() @ self.lm_head.float().T


def hip_model(cfg, num_blocks, seed=0):
    """Qwen3Tiny with the product attention and a GPU FP8 cache per layer."""
    caches = torch.zeros(2, cfg.num_layers, num_blocks, cfg.block_size, cfg.num_kv_heads, cfg.head_dim,
                         dtype=torch.uint8, device="cuda").view(torch.float8_e4m3fn)

    def make(i):
        a = Attention(cfg.num_heads, cfg.head_dim, cfg.head_dim ** -0.5)
        a.k_cache, a.v_cache = caches[0, i], caches[1, i]
        return a
    return Qwen3Tiny(cfg, make, seed=seed)


def oracle_model(cfg, num_blocks, seed=0):
    """Qwen3Tiny with oracle attention over CPU FP8 caches."""
    shape = (num_blocks, cfg.block_size, cfg.num_kv_heads, cfg.head_dim)

    def make(i):
        return OracleAttention(cfg.num_heads, cfg.head_dim, cfg.head_dim ** -0.5,
                               torch.zeros(shape, dtype=torch.uint8), torch.zeros(shape, dtype=torch.uint8))
    return Qwen3Tiny(cfg, make, seed=seed)


@dataclass
class Seq:
    """Sequence state with the attributes the metadata builder reads."""
    tokens: list
    block_table: list
    prompt_len: int
    num_cached_tokens: int = 0
    num_scheduled_tokens: int = 0
    drafts: list = field(default_factory=list)

    def __len__(self):
        return len(self.tokens)


class GreedyRunner:
    """Steps a model over a batch with the reference scheduler's shapes:
    decode rows first ([plain | speculative]), then prefill chunks."""

    def __init__(self, model, block_size, chunk):
        self.model, self.bs, self.chunk = model, block_size, chunk

    def step(self, seqs, spec_ids=()):
        """One forward.  Sequences still in prefill schedule their next chunk;
        finished ones decode one token (or 1 + drafts if in spec_ids).
        Returns {seq index: logits rows [n, vocab]} for the rows that predict."""
        dseqs, pseqs, ids = [], [], []
        for i, s in enumerate(seqs):
            if s.num_cached_tokens < s.prompt_len:
                s.num_scheduled_tokens = min(self.chunk, s.prompt_len - s.num_cached_tokens)
                s.drafts = []
                pseqs.append((i, s))
            else:
                s.drafts = list(s.drafts) if i in spec_ids else []
                s.num_scheduled_tokens = 1 + len(s.drafts)
                dseqs.append((i, s))
        plain = [(i, s) for i, s in dseqs if s.num_scheduled_tokens == 1]
        spec = [(i, s) for i, s in dseqs if s.num_scheduled_tokens > 1]
        order = plain + spec + pseqs
        prefilling = {i for i, _ in pseqs}
        # tokens the step feeds: the last token (plain), last + drafts (spec), the chunk (prefill)
        for i, s in order:
            if i in prefilling:
                ids += s.tokens[s.num_cached_tokens:s.num_cached_tokens + s.num_scheduled_tokens]
            else:
                ids += [s.tokens[-1]] + s.drafts
        # the builder reads len(seq) (decode) and num_cached_tokens (varlen rows)
        for _, s in spec:
            s.num_cached_tokens = len(s.tokens) - 1
            s.tokens = s.tokens + s.drafts
        positions = prepare_sequence([s for _, s in plain + spec], [s for _, s in pseqs], self.bs, set_context)
        input_ids = torch.tensor(ids, dtype=torch.int64, device="cuda")
        hidden = self.model.forward(input_ids, positions)
        logits = self.model.logits(hidden)
        reset_context()
        out, row = {}, 0
        for i, s in order:
            n = s.num_scheduled_tokens
            if i in prefilling:
                s.num_cached_tokens += n
                if s.num_cached_tokens == s.prompt_len:
                    out[i] = logits[row + n - 1:row + n]
            else:
                out[i] = logits[row:row + n]
                if s.drafts:  # drafts are never accepted: roll them back
                    s.tokens = s.tokens[:len(s.tokens) - len(s.drafts)]
                s.num_cached_tokens = len(s.tokens)
            row += n
        return out


def make_sequences(prompt_lens, max_new, vocab, block_size, num_blocks, seed):
    rng = np.random.default_rng(seed)
    pool = rng.permutation(num_blocks).tolist()
    seqs = []
    for L in prompt_lens:
        nb = -(-(L + max_new + 8) // block_size)
        table, pool = pool[:nb], pool[nb:]
        seqs.append(Seq(tokens=rng.integers(0, vocab, size=L).tolist(), block_table=table, prompt_len=L))
    return seqs


class GreedyComparison:
    """Row-by-row comparison of two greedy runs (product vs oracle) with a
    margin bound fixed in advance.  ``check(step, i, lh, lo)`` takes one
    sequence's predicting rows of one step ([n, vocab] logits of the product
    run and of the oracle run) and returns the token both runs feed back.

    * Every row must give the same greedy token in both runs unless the
      oracle's top-2 margin there is below ``margin_bound`` (a numerical tie);
      a flip at a larger margin raises AssertionError.
    * Each run feeds back its own greedy token (free-running).  Where the
      fed-back row (row 0) flips at a tie, both runs continue with the
      oracle's token from there (teacher-forced at that row), so their inputs
      stay identical and every later row is still compared.
    * Every row's logits must agree within ``logit_tol``.
    """

    def __init__(self, margin_bound, logit_tol):
        self.margin_bound, self.logit_tol = margin_bound, logit_tol
        self.flips, self.forced = [], []
        self.worst, self.n_rows, self.ties = 0.0, 0, 0

    def check(self, step, i, lh, lo):
        lh, lo = lh.float().cpu(), lo.float().cpu()
        assert lh.shape == lo.shape
        th, to = lh.argmax(-1).tolist(), lo.argmax(-1).tolist()
        dev = (lh - lo).abs().max(dim=-1).values
        self.worst = max(self.worst, float(dev.max()))
        assert torch.allclose(lh, lo, **self.logit_tol), \
            f"step {step} seq {i}: logits differ by up to {float(dev.max())}"
        top2 = lo.topk(2, dim=-1).values
        margins = (top2[:, 0] - top2[:, 1]).tolist()
        for r, (a, b, mg, dv) in enumerate(zip(th, to, margins, dev.tolist())):
            self.n_rows += 1
            self.ties += mg < self.margin_bound
            if a != b:
                assert mg < self.margin_bound, (
                    f"step {step} seq {i} row {r}: product greedy token {a} != oracle {b} at oracle top-2 margin "
                    f"{mg:.4f} >= {self.margin_bound} (row |dlogit| {dv:.4f})")
                self.flips.append((step, i, r, round(mg, 4), round(dv, 4)))
                print(f"[qwen3-greedy] tie flip: step {step} seq {i} row {r}: margin {mg:.4f}, "
                      f"|dlogit| {dv:.4f}", flush=True)
        if th[0] != to[0]:
            self.forced.append((step, i))
        return to[0]
