"""Seeded synthetic workloads at Qwen3 attention shapes, and their algorithmic units.

Each workload is a set of sequences over a paged FP8 KV pool:
  * per sequence: Lq query tokens and Lk = c + Lq keys (c = tokens already
    cached before this step; plain decode is Lq = 1, c = ctx - 1);
  * physical blocks are a shuffled subset of a pool 1.25x the blocks needed
    (or a caller-given pool size);
  * Q and the K/V values written into the cache are bf16 ~ N(0, 1); a
    fraction of K/V entries can be scaled (outliers) to exercise the E4M3
    range; K/V are quantised by whichever store function fills the cache.

The named constructors reproduce the benchmark configurations:
  tiny_decode      4 seqs, ctx [37, 256, 513, 1000], 4/2 heads, 16-block pool
  qwen3_0p6b_decode  B=256, 16/8 heads, ctx U[100, 2048]
  qwen3_8b_prefill  16 x 512-token chunks, 32/8 heads, cached U[0, 4096]
  qwen3_8b_mixed    192 decode + 32 spec x 5 + 3 x 512 chunks (+1024 contiguous)
  qwen3_8b_decode   the mixed batch's 192 plain-decode rows (32/8 heads, ctx U[256, 4096])
  qwen3_32b_long_decode  B=32, 64/8 heads, ctx U[32K, 128K], 1% x20 outliers
"""
from dataclasses import dataclass, field

import numpy as np
import torch

HEAD_DIM = 128
BLOCK_SIZE = 256


@dataclass
class SeqSpec:
    lq: int          # query tokens this step
    cached: int      # keys already in the cache before this step (c)

    @property
    def lk(self):
        return self.cached + self.lq


@dataclass
class PagedWorkload:
    name: str
    num_heads: int
    num_kv_heads: int
    seqs: list
    num_blocks: int
    block_tables: np.ndarray          # int32 [S, max_nb], -1 padded
    seed: int
    block_size: int = BLOCK_SIZE
    outlier_frac: float = 0.0
    outlier_scale: float = 20.0
    extra: dict = field(default_factory=dict)

    # ---- metadata --------------------------------------------------------
    @property
    def num_seqs(self):
        return len(self.seqs)

    def lq(self):
        return np.array([s.lq for s in self.seqs], dtype=np.int64)

    def lk(self):
        return np.array([s.lk for s in self.seqs], dtype=np.int64)

    def context_lens(self):
        """Decode view: keys per sequence (int32)."""
        return self.lk().astype(np.int32)

    def cu_seqlens(self):
        cu_q = np.concatenate([[0], np.cumsum(self.lq())]).astype(np.int32)
        cu_k = np.concatenate([[0], np.cumsum(self.lk())]).astype(np.int32)
        return cu_q, cu_k

    def num_q_tokens(self):
        return int(self.lq().sum())

    def slots_for(self, seq_idx, start, end):
        pos = np.arange(start, end, dtype=np.int64)
        table = self.block_tables[seq_idx].astype(np.int64)
        return (table[pos // self.block_size] * self.block_size + pos % self.block_size).astype(np.int32)

    def cache_slots(self, include_new=True):
        """Slots of every key that must be in the cache before attention runs."""
        parts = [self.slots_for(i, 0, s.lk if include_new else s.cached) for i, s in enumerate(self.seqs)]
        return np.concatenate(parts) if parts else np.zeros(0, np.int32)

    def new_token_slots(self):
        parts = [self.slots_for(i, s.cached, s.lk) for i, s in enumerate(self.seqs)]
        return np.concatenate(parts) if parts else np.zeros(0, np.int32)

    # ---- tensors ---------------------------------------------------------
    def make_q(self, device="cpu", seed_offset=0, dtype=torch.bfloat16):
        g = torch.Generator(device=device).manual_seed(self.seed * 1000 + 1 + seed_offset)
        return torch.randn(self.num_q_tokens(), self.num_heads, HEAD_DIM, generator=g,
                           device=device, dtype=torch.float32).to(dtype)

    def empty_caches(self, device):
        shape = (self.num_blocks, self.block_size, self.num_kv_heads, HEAD_DIM)
        k = torch.zeros(shape, dtype=torch.uint8, device=device)
        v = torch.zeros(shape, dtype=torch.uint8, device=device)
        return k.view(torch.float8_e4m3fn), v.view(torch.float8_e4m3fn)

    def kv_values(self, n_tokens, generator, device, which, dtype=torch.bfloat16):
        x = torch.randn(n_tokens, self.num_kv_heads, HEAD_DIM, generator=generator, device=device,
                        dtype=torch.float32)
        if self.outlier_frac > 0:
            mask = torch.rand(x.shape, generator=generator, device=device) < self.outlier_frac
            x = torch.where(mask, x * self.outlier_scale, x)
        return x.to(dtype)

    def fill_cache(self, k_cache, v_cache, store_fn, gen_device="cpu", include_new=True,
                   chunk_tokens=1 << 16, dtype=torch.bfloat16):
        """Writes N(0,1) K/V of ``dtype`` (bf16 or fp16) for every cached key
        through ``store_fn`` (signature of store_kvcache) in chunks of
        ``chunk_tokens`` tokens."""
        slots = self.cache_slots(include_new)
        g = torch.Generator(device=gen_device).manual_seed(self.seed * 1000 + 7)
        dev = k_cache.device
        for a in range(0, len(slots), chunk_tokens):
            b = min(a + chunk_tokens, len(slots))
            kk = self.kv_values(b - a, g, gen_device, "k", dtype).to(dev)
            vv = self.kv_values(b - a, g, gen_device, "v", dtype).to(dev)
            sm = torch.from_numpy(slots[a:b]).to(dev)
            store_fn(kk, vv, k_cache, v_cache, sm)

    # ---- algorithmic units -----------------------------------------------
    def decode_bytes(self):
        """HBM bytes of a decode step: FP8 K+V once, bf16 Q in + O out, block-table
        row and context length (per sequence)."""
        total = 0
        for s in self.seqs:
            total += (2 * s.lk * self.num_kv_heads * HEAD_DIM
                      + 2 * s.lq * self.num_heads * HEAD_DIM * 2
                      + 4 * -(-s.lk // self.block_size) + 4)
        return total

    def attention_flops(self):
        """QK^T + PV flops over the unmasked (causal) pairs only."""
        pairs = sum(s.lq * s.cached + s.lq * (s.lq + 1) // 2 for s in self.seqs)
        return 4 * HEAD_DIM * self.num_heads * pairs


def _assign_blocks(rng, seqs, block_size, pool_factor, num_blocks=None, max_num_blocks=None):
    nb = [-(-s.lk // block_size) for s in seqs]
    total = int(sum(nb))
    pool = num_blocks if num_blocks is not None else max(int(np.ceil(pool_factor * total)), total, 1)
    ids = rng.permutation(pool)[:total]
    width = max_num_blocks if max_num_blocks is not None else max(nb + [1])
    bt = np.full((len(seqs), width), -1, dtype=np.int32)
    o = 0
    for i, n in enumerate(nb):
        bt[i, :n] = ids[o:o + n]
        o += n
    return bt, pool


def make_workload(name, num_heads, num_kv_heads, seqs, seed, block_size=BLOCK_SIZE,
                  pool_factor=1.25, num_blocks=None, max_num_blocks=None, **kw):
    rng = np.random.default_rng(seed)
    bt, pool = _assign_blocks(rng, seqs, block_size, pool_factor, num_blocks, max_num_blocks)
    return PagedWorkload(name=name, num_heads=num_heads, num_kv_heads=num_kv_heads, seqs=seqs,
                         num_blocks=pool, block_tables=bt, seed=seed, block_size=block_size, **kw)


def decode_workload(name, B, num_heads, num_kv_heads, ctx_lo, ctx_hi, seed, **kw):
    rng = np.random.default_rng(seed + 12345)
    ctx = rng.integers(ctx_lo, ctx_hi + 1, size=B)
    seqs = [SeqSpec(lq=1, cached=int(c) - 1) for c in ctx]
    return make_workload(name, num_heads, num_kv_heads, seqs, seed, **kw)


def tiny_decode(seed=1):
    """4 sequences, ctx [37, 256, 513, 1000], 4 query / 2 kv heads, 16-block pool."""
    seqs = [SeqSpec(lq=1, cached=c - 1) for c in (37, 256, 513, 1000)]
    return make_workload("tiny_decode", 4, 2, seqs, seed, num_blocks=16)


def qwen3_0p6b_decode(seed=2, B=256):
    """B=256, 16/8 heads, ctx U[100, 2048], 1.25x pool."""
    return decode_workload("qwen3_0.6b_decode_b256", B, 16, 8, 100, 2048, seed)


def qwen3_8b_prefill(seed=3, S=16, chunk=512):
    """S x 512-token chunks, 32/8 heads, cached context U[0, 4096]."""
    rng = np.random.default_rng(seed + 12345)
    cached = rng.integers(0, 4096 + 1, size=S)
    seqs = [SeqSpec(lq=chunk, cached=int(c)) for c in cached]
    return make_workload("qwen3_8b_prefill_16x512", 32, 8, seqs, seed)


def qwen3_8b_mixed(seed=4):
    """Plain decode (192, ctx U[256, 4096]) + speculative (32 x 5 rows, c U[256, 4096])
    + 3 x 512-token chunks (c U[0, 4096]) sharing one paged pool; the
    1024-token contiguous prompt is in ``extra['contiguous_prompt_len']``."""
    rng = np.random.default_rng(seed + 12345)
    dec = [SeqSpec(lq=1, cached=int(c) - 1) for c in rng.integers(256, 4096 + 1, size=192)]
    spec = [SeqSpec(lq=5, cached=int(c)) for c in rng.integers(256, 4096 + 1, size=32)]
    chunks = [SeqSpec(lq=512, cached=int(c)) for c in rng.integers(0, 4096 + 1, size=3)]
    wl = make_workload("qwen3_8b_mixed", 32, 8, dec + spec + chunks, seed)
    wl.extra.update(split_pt=192, num_spec_seqs=32, contiguous_prompt_len=1024)
    return wl


def qwen3_8b_decode(seed=4):
    """The mixed batch's 192 plain-decode rows on their own (32/8 heads, ctx
    U[256, 4096]), over the mixed batch's paged pool."""
    full = qwen3_8b_mixed(seed)
    return sub_workload(full, range(full.extra["split_pt"]), name="qwen3_8b_decode_b192")


def qwen3_32b_long_decode(seed=5, B=32, ctx_lo=32 * 1024, ctx_hi=128 * 1024):
    """B=32, 64/8 heads, ctx U[32K, 128K], 1% of K/V entries x20."""
    return decode_workload("qwen3_32b_long_decode", B, 64, 8, ctx_lo, ctx_hi, seed,
                           outlier_frac=0.01, outlier_scale=20.0)


def sub_workload(wl, seq_indices, name=None, compact=False, seed=None):
    """The sequences ``seq_indices`` of ``wl`` (same blocks unless ``compact``,
    which renumbers them into a fresh pool of exactly the blocks needed)."""
    seqs = [wl.seqs[i] for i in seq_indices]
    bt = wl.block_tables[list(seq_indices)]
    num_blocks = wl.num_blocks
    if compact:
        used = np.unique(bt[bt >= 0])
        remap = {int(b): i for i, b in enumerate(used)}
        bt = np.where(bt >= 0, np.vectorize(lambda b: remap.get(int(b), -1))(bt), -1).astype(np.int32)
        num_blocks = len(used)
    return PagedWorkload(name=name or wl.name + "_sub", num_heads=wl.num_heads,
                         num_kv_heads=wl.num_kv_heads, seqs=seqs, num_blocks=num_blocks,
                         block_tables=bt, seed=wl.seed if seed is None else seed,
                         block_size=wl.block_size, outlier_frac=wl.outlier_frac,
                         outlier_scale=wl.outlier_scale, extra=dict(wl.extra))
