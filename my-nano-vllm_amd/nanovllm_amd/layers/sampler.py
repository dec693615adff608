"""Temperature sampler, the drop-in for nanovllm/layers/sampler.py.

``Sampler.forward(logits, temperatures)`` keeps the reference's signature and
result (sampler.py:7-12): token = argmax(softmax(logits / T) / max(E, 1e-10))
with E ~ Exp(1).  ``nvamd_sample`` computes the same argmax as that of
logits * log2(e) / T - log2(max(E, 1e-10)) in one sweep over the logits,
instead of the reference's fp32 copies of the whole [rows, vocab] matrix.  A
given noise matrix is used token by token; otherwise the noise is drawn in
the kernel from Philox4x32-10, top down by groups of 16 tokens (the group's
maximum score drawn directly, then the token inside the winning group; the
token distribution is softmax(logits / T) either way).  The generator is
keyed by a seed taken from torch's CPU generator on every call, so
``torch.manual_seed`` makes runs repeatable.
"""
import torch
from torch import nn

from .. import _native

_DTYPE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def sample_tokens(logits: torch.Tensor, temperatures: torch.Tensor, noise: torch.Tensor | None = None,
                  seed: int | None = None, offset: int = 0) -> torch.Tensor:
    """int64 [rows] tokens; ``noise`` (fp32 [rows, vocab]) replaces the in-kernel
    Exp(1) draws, ``seed`` the one taken from torch's CPU generator."""
    if not logits.is_cuda:
        raise ValueError(f"logits must be on a ROCm GPU (got {logits.device})")
    if logits.dtype not in _DTYPE:
        raise ValueError(f"logits must be bf16, fp16 or fp32 (got {logits.dtype})")
    if logits.stride(-1) != 1:
        logits = logits.contiguous()
    rows, vocab = logits.shape
    temperatures = temperatures.to(device=logits.device, dtype=torch.float32).contiguous()
    if temperatures.numel() != rows:
        raise ValueError("one temperature per row")
    if noise is not None:
        noise = noise.to(device=logits.device, dtype=torch.float32).contiguous()
        if tuple(noise.shape) != (rows, vocab):
            raise ValueError("noise must be [rows, vocab]")
    if seed is None:
        seed = int(torch.randint(0, 2 ** 62, (1,)).item())
    out = torch.empty(rows, dtype=torch.int64, device=logits.device)
    lib = _native.load()
    ws_bytes = lib.nvamd_sample_workspace_bytes(rows, vocab)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=logits.device)
    _native.check(lib.nvamd_sample(logits.data_ptr(), _DTYPE[logits.dtype], logits.stride(0), rows, vocab,
                                   temperatures.data_ptr(), noise.data_ptr() if noise is not None else None,
                                   seed, offset, out.data_ptr(), ws.data_ptr(), ws.numel(),
                                   torch.cuda.current_stream(logits.device).cuda_stream),
                  "sample")
    return out


class Sampler(nn.Module):

    def forward(self, logits: torch.Tensor, temperatures: torch.Tensor):
        return sample_tokens(logits, temperatures)
