"""The dispatcher operators torch.ops.nvamd.* (registered by nanovllm_amd.ops):
their schemas match the reference's three calls (attention.py:33,
fp8_attention.py:173-176,314-318), their fake implementations give the output
shapes without a GPU, and a CPU call raises instead of falling back."""
import pytest
import torch

import nanovllm_amd  # noqa: F401  (registers the operators)


def _schema(name):
    return str(getattr(torch.ops.nvamd, name).default._schema)


def test_store_schema_marks_the_cache_writes():
    s = _schema("store_kvcache")
    assert s.startswith("nvamd::store_kvcache(Tensor key, Tensor value, Tensor(")
    args = s[s.index("(") + 1:s.rindex(") ->")].split(", ")
    assert [a.split(" ")[-1] for a in args] == ["key", "value", "k_cache", "v_cache", "slot_mapping"]
    # k_cache and v_cache are written in place (distinct alias sets), nothing else is
    assert "!" in args[2] and "!" in args[3] and args[2].split(" ")[0] != args[3].split(" ")[0]
    assert all("!" not in a for a in (args[0], args[1], args[4]))
    assert s.endswith("-> ()")


def test_decode_and_prefill_schemas():
    assert _schema("decode") == ("nvamd::decode(Tensor q, Tensor k_cache, Tensor v_cache, Tensor block_tables, "
                                 "Tensor context_lens, float scale) -> Tensor")
    assert _schema("prefill") == ("nvamd::prefill(Tensor q, Tensor k, Tensor v, Tensor? block_tables, Tensor cu_q, "
                                  "Tensor cu_k, SymInt max_q, SymInt max_k, float scale) -> Tensor")


def test_fake_implementations_give_the_output_shapes():
    m = dict(device="meta")
    q = torch.empty(3, 32, 128, dtype=torch.bfloat16, **m)
    kc = torch.empty(16, 256, 8, 128, dtype=torch.float8_e4m3fn, **m)
    i32 = dict(dtype=torch.int32, **m)
    o = torch.ops.nvamd.decode(q, kc, kc, torch.empty(3, 2, **i32), torch.empty(3, **i32), 128 ** -0.5)
    assert o.shape == q.shape and o.dtype == torch.bfloat16 and o.device.type == "meta"
    o = torch.ops.nvamd.prefill(q, kc, kc, None, torch.empty(2, **i32), torch.empty(2, **i32), 3, 3, 128 ** -0.5)
    assert o.shape == q.shape and o.dtype == torch.bfloat16
    key = torch.empty(3, 8, 128, dtype=torch.bfloat16, **m)
    assert torch.ops.nvamd.store_kvcache(key, key, kc, kc, torch.empty(3, **i32)) is None


def test_cpu_tensors_raise():
    q = torch.zeros(2, 4, 128, dtype=torch.bfloat16)
    kc = torch.zeros(4, 256, 2, 128).to(torch.float8_e4m3fn)
    with pytest.raises(NotImplementedError):
        torch.ops.nvamd.decode(q, kc, kc, torch.zeros(2, 1, dtype=torch.int32), torch.ones(2, dtype=torch.int32),
                               128 ** -0.5)


def test_fp8_block_linear_schema_and_fake_shape():
    assert _schema("fp8_block_linear") == ("nvamd::fp8_block_linear(Tensor x, Tensor weight, Tensor weight_scale) "
                                           "-> Tensor")
    m = dict(device="meta")
    x = torch.empty(5, 256, dtype=torch.float16, **m)
    w = torch.empty(384, 256, dtype=torch.float8_e4m3fn, **m)
    o = torch.ops.nvamd.fp8_block_linear(x, w, torch.empty(3, 2, dtype=torch.bfloat16, **m))
    assert o.shape == (5, 384) and o.dtype == torch.float16 and o.device.type == "meta"
