"""FP8 KV store/quantise on the GPU: byte-exact against the golden table and the oracle."""
import os

import numpy as np
import pytest
import torch

from gpu_util import announce, cpu_store
from oracle import fp8 as ofp8
from nanovllm_amd.layers.attention import store_kvcache
import workloads as W

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "bf16_to_e4m3fn.bin")
FP8 = torch.float8_e4m3fn


def test_store_all_bf16_patterns_byte_exact():
    announce("store: all 65536 bf16 patterns")
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.int16)
    key = torch.from_numpy(bits.copy()).view(torch.bfloat16).reshape(512, 1, 128).cuda()
    value = key.flip(0).contiguous()
    kc = torch.zeros(2, 256, 1, 128, dtype=torch.uint8, device="cuda").view(FP8)
    vc = torch.zeros_like(kc)
    slots = torch.arange(512, dtype=torch.int32, device="cuda")
    store_kvcache(key, value, kc, vc, slots)
    torch.cuda.synchronize()
    golden = np.fromfile(GOLDEN, dtype=np.uint8)
    f = ofp8.bf16_bits_to_f32(bits.view(np.uint16))
    nan = np.isnan(f)
    got_k = kc.view(torch.uint8).cpu().numpy().reshape(-1)
    got_v = vc.view(torch.uint8).cpu().numpy().reshape(-1)[::-1].reshape(512, 128)[:, ::-1].reshape(-1)
    for got in (got_k, got_v):
        mism = np.nonzero((got != golden) & ~nan)[0]
        assert mism.size == 0, f"{mism.size} mismatches, first bf16 0x{int(bits.view(np.uint16)[mism[0]]):04x}: got 0x{got[mism[0]]:02x} want 0x{golden[mism[0]]:02x}"
        assert np.all((got[nan] & 0x7F) == 0x7F), "NaN inputs must give NaN codes"


def test_store_skips_padding_slots_and_reads_strided_rows():
    announce("store: slot -1, fused-qkv strided rows, canaries")
    torch.manual_seed(0)
    N, Hq, Hkv, D, P, bs = 37, 16, 8, 128, 6, 256
    qkv = torch.randn(N, (Hq + 2 * Hkv) * D, device="cuda").to(torch.bfloat16)
    k = qkv[:, Hq * D:(Hq + Hkv) * D].view(N, Hkv, D)
    v = qkv[:, (Hq + Hkv) * D:].view(N, Hkv, D)
    assert not v.is_contiguous() and v.stride(0) == (Hq + 2 * Hkv) * D
    kc = torch.full((P, bs, Hkv, D), 0xAB, dtype=torch.uint8, device="cuda").view(FP8)
    vc = torch.full((P, bs, Hkv, D), 0xCD, dtype=torch.uint8, device="cuda").view(FP8)
    slots = torch.randperm(P * bs)[:N].to(torch.int32)
    slots[::5] = -1
    store_kvcache(k, v, kc, vc, slots.cuda())
    kc_ref = torch.full((P, bs, Hkv, D), 0xAB, dtype=torch.uint8)
    vc_ref = torch.full((P, bs, Hkv, D), 0xCD, dtype=torch.uint8)
    ofp8.store_kvcache(k.cpu(), v.cpu(), kc_ref, vc_ref, slots)
    assert torch.equal(kc.view(torch.uint8).cpu(), kc_ref)
    assert torch.equal(vc.view(torch.uint8).cpu(), vc_ref)


def test_store_beyond_int32_offsets():
    announce("store: slots whose byte offset exceeds 2**31")
    Hkv, D, bs = 8, 128, 256
    P = 9000                                  # 9000*256*1024 B > 2**31
    kc = torch.zeros(P, bs, Hkv, D, dtype=torch.uint8, device="cuda").view(FP8)
    vc = torch.zeros_like(kc)
    slots = torch.tensor([P * bs - 1, 8192 * bs + 3, 5], dtype=torch.int32)
    k = torch.randn(3, Hkv, D).to(torch.bfloat16)
    v = torch.randn(3, Hkv, D).to(torch.bfloat16)
    store_kvcache(k.cuda(), v.cuda(), kc, vc, slots.cuda())
    kf, vf = kc.view(torch.uint8).view(-1, Hkv * D), vc.view(torch.uint8).view(-1, Hkv * D)
    for i, s in enumerate(slots.tolist()):
        assert torch.equal(kf[s].cpu(), ofp8.quantize_bf16_tensor(k[i].reshape(-1)))
        assert torch.equal(vf[s].cpu(), ofp8.quantize_bf16_tensor(v[i].reshape(-1)))


@pytest.mark.parametrize("make", [W.tiny_decode, W.qwen3_8b_prefill])
def test_store_workload_matches_oracle(make):
    wl = make()
    announce(f"store: workload {wl.name}")
    from gpu_util import build_pair
    build_pair(wl)


@pytest.mark.parametrize("hkv,d", [(2, 128), (1, 48), (3, 10)])
def test_store_each_kernel_path(hkv, d):
    """Rows of a multiple of 32 elements (two-chunk kernel), of 16 (one-chunk
    kernel) and of neither (one element per lane), with canaries around every
    written row and a slot of -1."""
    announce(f"store: row of {hkv}x{d} elements")
    torch.manual_seed(1)
    N, P, bs = 29, 3, 16
    k = (torch.randn(N, hkv, d) * 300).to(torch.bfloat16)
    v = (torch.randn(N, hkv, d) * 0.01).to(torch.bfloat16)
    slots = torch.randperm(P * bs)[:N].to(torch.int32)
    slots[3] = -1
    kc = torch.full((P, bs, hkv, d), 0x5A, dtype=torch.uint8, device="cuda").view(FP8)
    vc = torch.full((P, bs, hkv, d), 0xA5, dtype=torch.uint8, device="cuda").view(FP8)
    store_kvcache(k.cuda(), v.cuda(), kc, vc, slots.cuda())
    kc_ref = torch.full((P, bs, hkv, d), 0x5A, dtype=torch.uint8)
    vc_ref = torch.full((P, bs, hkv, d), 0xA5, dtype=torch.uint8)
    ofp8.store_kvcache(k, v, kc_ref, vc_ref, slots)
    assert torch.equal(kc.view(torch.uint8).cpu(), kc_ref)
    assert torch.equal(vc.view(torch.uint8).cpu(), vc_ref)
