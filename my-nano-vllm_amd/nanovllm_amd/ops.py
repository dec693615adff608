"""The attention path as operators of torch's dispatcher.

``torch.ops.nvamd.store_kvcache``, ``torch.ops.nvamd.decode`` and
``torch.ops.nvamd.prefill`` are registered by the C++ library
``libnvamd_torch_ops.so`` (``csrc/torch_ops.cpp``, a ``TORCH_LIBRARY`` block)
for the reference's three attention calls (store: attention.py:33-40; decode:
fp8_attention.py:173-207; prefill: fp8_attention.py:314-353), and
``torch.ops.nvamd.fp8_block_linear`` for its FP8 linear layer
(fp8_linear.py:93-139):

    store_kvcache(Tensor key, Tensor value, Tensor(a!) k_cache, Tensor(b!) v_cache, Tensor slot_mapping) -> ()
    decode(Tensor q, Tensor k_cache, Tensor v_cache, Tensor block_tables, Tensor context_lens, float scale) -> Tensor
    prefill(Tensor q, Tensor k, Tensor v, Tensor? block_tables, Tensor cu_q, Tensor cu_k, SymInt max_q,
            SymInt max_k, float scale) -> Tensor
    fp8_block_linear(Tensor x, Tensor weight, Tensor weight_scale) -> Tensor

Their ROCm kernels check the arguments, allocate the output and workspace
from torch's caching allocator and launch through the C ABI; the drop-in
Python functions (``nanovllm_amd.kernels.fp8_attention``,
``nanovllm_amd.layers.attention``, ``nanovllm_amd.kernels.fp8_linear``) call
them.  Their Meta kernels give
FakeTensor / torch.compile tracing the output shapes without running
anything.  There is no CPU kernel: a call on CPU tensors raises.

Importing this module loads the library when it is built; without it the
operators are absent and the Python entry points raise when called.
"""
from . import _native

try:
    _native.load_ops()
except RuntimeError:
    pass
