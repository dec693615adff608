"""LM-head row selection, the drop-in for the selection in
ParallelLMHead.forward (nanovllm/layers/embed_head.py:56-72).

With varlen rows in the step, the LM head keeps the plain-decode rows, every
row of the speculative sequences (their drafts are verified against all of
them) and the last row of each prefill sequence.  ``select_lm_head_rows``
builds that matrix with one HIP gather (``nvamd_select_logit_rows``) from
the step's Context; ``lm_head_logits`` then applies the bf16 LM-head weight
(a plain library GEMM, as F.linear in the reference).

The Context is an argument: the caller passes the one its runner filled
(inside nano-vLLM, ``nanovllm.utils.context.get_context()``, the object
ParallelLMHead.forward reads at :57).  The speculative row count comes from
the Context's host-side ``num_spec_rows`` when it has one and the metadata
builder set it; otherwise ``cu_seqlens_q[nspec]`` is read back from the GPU,
as the reference does (:63).
"""
import torch
import torch.nn.functional as F

from .. import _native


def select_lm_head_rows(x: torch.Tensor, context) -> torch.Tensor:
    """The rows of ``x`` the LM head keeps under ``context`` (a Context with
    the fields of nanovllm/utils/context.py:5-15)."""
    cu = context.cu_seqlens_q
    if not isinstance(cu, torch.Tensor):
        return x
    if not x.is_cuda:
        raise ValueError(f"x must be on a ROCm GPU (got {x.device})")
    if x.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError(f"x must be bf16, fp16 or fp32 (got {x.dtype})")
    split_pt, nspec = context.split_pt, context.num_spec_seqs
    n_var = cu.numel() - 1
    n_spec_rows = getattr(context, "num_spec_rows", -1)
    if n_spec_rows < 0:
        n_spec_rows = int(cu[nspec].item())
    n_prefill = n_var - nspec
    if x.stride(-1) != 1 or (x.stride(0) * x.element_size()) % 16 or x.data_ptr() % 16:
        x = x.contiguous()
    out = torch.empty(split_pt + n_spec_rows + n_prefill, x.shape[1], dtype=x.dtype, device=x.device)
    cu = cu.to(torch.int32).contiguous()
    lib = _native.load()
    _native.check(lib.nvamd_select_logit_rows(
        x.data_ptr(), x.stride(0), x.shape[0], x.shape[1], x.element_size(), cu.data_ptr(), split_pt, nspec,
        n_spec_rows, n_prefill, out.data_ptr(), out.stride(0), torch.cuda.current_stream(x.device).cuda_stream),
        "select_logit_rows")
    return out


def lm_head_logits(x: torch.Tensor, weight: torch.Tensor, context) -> torch.Tensor:
    """The logits ParallelLMHead.forward returns on one GPU (embed_head.py:56-73)."""
    return F.linear(select_lm_head_rows(x, context), weight)
