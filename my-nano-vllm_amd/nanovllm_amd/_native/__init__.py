"""ctypes binding of the gfx950 C-ABI library ``libnvamd_fp8attn.so``.

The library is built in-tree by ``make -C my-nano-vllm_amd`` (see
``__graft_entry__.build``), with ``libnvamd_torch_ops.so``, the dispatcher
operators over it (``load_ops``).  There is no fallback: importing the attention
functions works without a GPU, but calling them without the built library
raises ``RuntimeError``.

torch is imported before the library is loaded so that the HIP runtime torch
ships (soname ``libamdhip64.so.7``) is the one the library binds to; streams
handed over from torch are then valid in the library.
"""
import ctypes
import os

import torch  # noqa: F401  (loads torch's HIP runtime first)

LIB_NAME = "libnvamd_fp8attn.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
# the torch operators over the C ABI (csrc/torch_ops.cpp), linked against LIB_NAME
OPS_LIB_NAME = "libnvamd_torch_ops.so"
OPS_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), OPS_LIB_NAME)
ABI_VERSION = 7

_c_void_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float

# name -> (restype, argtypes); mirrors include/nvamd_fp8_attention.h, nvamd_fp8_linear.h and nvamd_lm_head.h
SIGNATURES = {
    "nvamd_abi_version": (_i32, []),
    "nvamd_last_error": (ctypes.c_char_p, []),
    "nvamd_store_kvcache": (_i32, [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _c_void_p,
                                   _c_void_p, _i64, _i32, _i32, _i64, _i32, _c_void_p]),
    "nvamd_qk_norm_rope_store": (_i32, [_c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p, _f32, _c_void_p, _i64,
                                        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i32, _i32,
                                        _i32, _i64, _c_void_p]),
    "nvamd_decode_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "nvamd_fp8_decode_attention": (_i32, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                          _c_void_p, _i32, _i32, _i32, _i32, _i64, _i32, _i32,
                                          _f32, _i32, _c_void_p, _i64, _i32, _c_void_p]),
    "nvamd_fp8_decode_attention_noalloc": (_i32, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                                  _c_void_p, _i32, _i32, _i32, _i32, _i64, _i32, _i32,
                                                  _f32, _i32, _c_void_p]),
    "nvamd_build_attention_metadata": (_i32, [_c_void_p, _i64, _i32, _i32, _i32, _i64, _i64, _i32, _i32,
                                              _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                              _c_void_p]),
    "nvamd_select_logit_rows": (_i32, [_c_void_p, _i64, _i64, _i32, _i32, _c_void_p, _i32, _i32, _i32, _i32,
                                       _c_void_p, _i64, _c_void_p]),
    "nvamd_sample_workspace_bytes": (_i64, [_i64, _i64]),
    "nvamd_sample": (_i32, [_c_void_p, _i32, _i64, _i64, _i64, _c_void_p, _c_void_p, ctypes.c_uint64,
                            ctypes.c_uint64, _c_void_p, _c_void_p, _i64, _c_void_p]),
    "nvamd_fp8_act_quant": (_i32, [_c_void_p, _i64, _i32, _c_void_p, _c_void_p, _i64, _i64, _c_void_p]),
    "nvamd_fp8_block_gemm": (_i32, [_c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p, _i64, _i32,
                                    _i64, _i64, _i64, _c_void_p, _i64, _c_void_p]),
    "nvamd_fp8_block_gemm_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "nvamd_prefill_workspace_bytes": (_i64, [_i64, _i32, _i32, _i32, _i64, _i32, _i32, _i32]),
    "nvamd_fp8_prefill_attention": (_i32, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                           _c_void_p, _c_void_p, _i64, _i32, _i32, _i32, _i32,
                                           _i64, _i32, _i32, _i32, _i32, _f32, _i32, _c_void_p,
                                           _i64, _i32, _c_void_p]),
}

_lib = None


def load():
    """Load (once) and return the ctypes library; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"nanovllm_amd: native library {LIB_PATH} is not built; run "
            "`make -C my-nano-vllm_amd` (or __graft_entry__.build()) first")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.nvamd_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"nanovllm_amd: ABI version {version} != expected {ABI_VERSION}; rebuild")
    _lib = lib
    return lib


_ops_loaded = False


def load_ops():
    """Load (once) the torch-operator library, which registers
    torch.ops.nvamd.store_kvcache / decode / prefill, and return
    torch.ops.nvamd; raises if it is not built."""
    global _ops_loaded
    if not _ops_loaded:
        load()  # the operators call into the C-ABI library (same file, loaded once)
        if not os.path.exists(OPS_LIB_PATH):
            raise RuntimeError(
                f"nanovllm_amd: operator library {OPS_LIB_PATH} is not built; run "
                "`make -C my-nano-vllm_amd` (or __graft_entry__.build()) first")
        torch.ops.load_library(OPS_LIB_PATH)
        _ops_loaded = True
    return torch.ops.nvamd


def check(status, what):
    if status != 0:
        msg = load().nvamd_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {status}): {msg}")
