"""Pins the FP8 block-scaled linear oracle (nanovllm/kernels/fp8_linear.py:11-139).

Independent checks: the committed bf16 -> E4M3FN golden table on groups whose
scale is exactly 1; torch's own CPU casts (float32 -> float8_e4m3fn, bfloat16,
float16); closed forms (amax element, zero and constant groups); the E4M3
error bound; torch float64 matmuls of the dequantised operands; an all-exact
integer GEMM that must agree bit for bit; and the locality of each block scale.
"""
import os

import numpy as np
import pytest
import torch

from oracle import fp8
from oracle import fp8_linear as ol

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "bf16_to_e4m3fn.bin")


def _bf16(a):
    return torch.from_numpy(np.asarray(a, dtype=np.float32)).to(torch.bfloat16)


def _bits(t):
    return t.view(torch.int16).numpy().view(np.uint16)


def test_unit_scale_groups_match_the_golden_table():
    """Every finite bf16 value with |x| <= 448, in groups that also hold 448:
    amax = 448, so the scale is exactly 1 and xq must be the reference's
    plain bf16 -> E4M3FN cast, i.e. the golden table."""
    golden = np.fromfile(GOLDEN, dtype=np.uint8)
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    vals = fp8.bf16_bits_to_f32(bits)
    keep = np.isfinite(vals) & (np.abs(vals) <= 448.0)
    bits, vals = bits[keep], vals[keep]
    n = len(vals)
    groups = -(-n // 127)
    x = np.full((groups, 128), 448.0, dtype=np.float32)
    flat = np.zeros(groups * 127, dtype=np.float32)
    flat[:n] = vals
    x[:, 1:] = flat.reshape(groups, 127)
    xq, x_scale, scale = ol.act_quant(_bf16(x))
    assert np.all(scale == 1.0) and np.all(x_scale == 0x3F80)
    got = xq.reshape(groups, 128)[:, 1:].reshape(-1)[:n]
    assert np.array_equal(got, golden[bits])
    assert np.all(xq.reshape(groups, 128)[:, 0] == 0x7E)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_quant_matches_torch_casts(dtype):
    """Groups spanning many binades (and fp16's range): the codes equal torch's
    float32 -> float8_e4m3fn cast of the clamped quotient, the scale bits
    torch's float32 -> bfloat16 cast."""
    g = torch.Generator().manual_seed(7)
    M, K = 48, 1024
    lo, hi = (-30, 30) if dtype == torch.bfloat16 else (-6, 4)
    mag = 10.0 ** torch.empty(M, K // 128, 1).uniform_(lo, hi, generator=g)
    x = (torch.randn(M, K // 128, 128, generator=g) * mag).reshape(M, K).to(dtype)
    xq, x_scale, scale = ol.act_quant(x)
    xf = x.float().reshape(M, K // 128, 128)
    s = xf.abs().amax(-1) / 448.0
    s = torch.where(s > 0, s, torch.ones_like(s))
    assert np.array_equal(scale, s.numpy())
    y = (xf / s[..., None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8)
    assert np.array_equal(xq, y.reshape(M, K).numpy())
    assert np.array_equal(x_scale, _bits(s.to(torch.bfloat16)))


def test_quant_closed_forms():
    """The amax element maps to +-448; an all-zero group has scale 1 and zero
    codes; a constant group is all +-448 with scale bf16(c / 448)."""
    x = np.zeros((3, 256), dtype=np.float32)
    x[0, :128] = np.linspace(-3.0, 2.0, 128)
    x[0, 128:] = 0.0
    x[1, :128] = -0.75
    x[1, 128:] = 1e-3
    x[2, 5] = -7.0
    xq, x_scale, scale = ol.act_quant(_bf16(x))
    assert xq[0, 0] == 0xFE and xq[2, 5] == 0xFE              # -amax -> -448
    assert np.all(xq[0, 128:] == 0) and x_scale[0, 1] == 0x3F80  # zero group
    assert np.all(xq[1, :128] == 0xFE) and np.all(xq[1, 128:] == 0x7E)
    c = np.float32(_bf16([1e-3]).float().item())
    assert x_scale[1, 1] == _bits(torch.tensor([c / np.float32(448.0)]).to(torch.bfloat16))[0]


def test_quant_error_bound():
    """|dequant(xq) * scale - x| <= 2^-4 |x| + 2^-10 scale (half an E4M3 ulp,
    relative in the normal range, absolute in the subnormal range)."""
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(64, 512, generator=g) * 10.0 ** torch.empty(64, 1).uniform_(-8, 8, generator=g)).to(torch.bfloat16)
    xq, _, scale = ol.act_quant(x)
    deq = fp8.dequant_table()[xq].reshape(64, 4, 128).astype(np.float64) * scale[..., None]
    xf = x.float().numpy().reshape(64, 4, 128).astype(np.float64)
    assert np.all(np.abs(deq - xf) <= 2.0 ** -4 * np.abs(xf) + 2.0 ** -10 * scale[..., None] * (1 + 1e-6))


def _rand_codes(g, shape):
    c = torch.randint(0, 256, shape, generator=g, dtype=torch.int32).to(torch.uint8)
    return torch.where((c & 0x7F) == 0x7F, c ^ 0x01, c).numpy()   # no NaN codes


def _rand_scales(g, shape):
    return _bits((10.0 ** torch.empty(shape).uniform_(-4, 1, generator=g)).to(torch.bfloat16))


def _f64_reference(xq, x_scale, w, w_scale):
    """Dequantise both operands (codes x block scales) and multiply in float64;
    also returns the sum of absolute terms (the accumulation error scale)."""
    t = torch.from_numpy(fp8.dequant_table().astype(np.float64))
    xs = torch.from_numpy(fp8.bf16_bits_to_f32(x_scale).astype(np.float64)).repeat_interleave(128, 1)
    ws = torch.from_numpy(fp8.bf16_bits_to_f32(w_scale).astype(np.float64)).repeat_interleave(128, 0).repeat_interleave(128, 1)
    xd = t[torch.from_numpy(xq).long()] * xs
    wd = t[torch.from_numpy(w).long()] * ws
    return (xd @ wd.T).numpy(), (xd.abs() @ wd.abs().T).numpy()


@pytest.mark.parametrize("M,N,K", [(1, 128, 128), (5, 256, 512), (33, 384, 1024)])
def test_gemm_matches_float64_matmul(M, N, K):
    g = torch.Generator().manual_seed(M * 7 + N + K)
    xq, w = _rand_codes(g, (M, K)), _rand_codes(g, (N, K))
    x_scale, w_scale = _rand_scales(g, (M, K // 128)), _rand_scales(g, (N // 128, K // 128))
    out, acc = ol.block_gemm(xq, x_scale, w, w_scale)
    ref, absum = _f64_reference(xq, x_scale, w, w_scale)
    kc = K // 128
    assert np.all(np.abs(acc - ref) <= (2 * kc + 2) * 2.0 ** -24 * absum + 1e-30)
    want = torch.from_numpy(ref).to(torch.float32).to(torch.bfloat16)
    o = torch.from_numpy(out.view(np.int16)).view(torch.bfloat16).float()
    assert torch.all((o - want.float()).abs() <= 2.0 ** -7 * want.float().abs() + 2.0 ** -22 * torch.from_numpy(absum).float())


def test_gemm_exact_integer_case():
    """Small-integer codes and power-of-two scales: every fp32 step is exact,
    so the oracle equals the float64 product rounded once to bf16 (a
    transposed operand or a misplaced scale fails this)."""
    g = torch.Generator().manual_seed(11)
    ints = torch.tensor([-4.0, -3.0, -2.0, -1.0, 0.0, 1.0, 2.0, 3.0, 4.0])
    M, N, K = 24, 256, 512
    xv = ints[torch.randint(0, 9, (M, K), generator=g)]
    wv = ints[torch.randint(0, 9, (N, K), generator=g)]
    xq = xv.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    w = wv.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    x_scale = _bits((2.0 ** torch.randint(-3, 4, (M, K // 128), generator=g).float()).to(torch.bfloat16))
    w_scale = _bits((2.0 ** torch.randint(-3, 4, (N // 128, K // 128), generator=g).float()).to(torch.bfloat16))
    out, acc = ol.block_gemm(xq, x_scale, w, w_scale)
    ref, _ = _f64_reference(xq, x_scale, w, w_scale)
    assert np.array_equal(acc.astype(np.float64), ref)
    assert np.array_equal(out, _bits(torch.from_numpy(ref).float().to(torch.bfloat16)))
    out16, _ = ol.block_gemm(xq, x_scale, w, w_scale, "fp16")
    assert np.array_equal(out16, torch.from_numpy(ref).float().to(torch.float16).view(torch.int16).numpy().view(np.uint16))


def test_gemm_scale_locality():
    """Doubling one weight-block scale sw[nb, kc] changes only columns of block
    nb, by that block's own contribution (its float64 partial x scales)."""
    g = torch.Generator().manual_seed(5)
    M, N, K = 8, 384, 384
    xq, w = _rand_codes(g, (M, K)), _rand_codes(g, (N, K))
    x_scale, w_scale = _rand_scales(g, (M, 3)), _rand_scales(g, (3, 3))
    _, acc0 = ol.block_gemm(xq, x_scale, w, w_scale)
    nb, kc = 1, 2
    w2 = w_scale.copy()
    w2[nb, kc] = _bits(torch.tensor([2 * fp8.bf16_bits_to_f32(w_scale[nb, kc])]).to(torch.bfloat16))[0]
    _, acc1 = ol.block_gemm(xq, x_scale, w, w2)
    cols = np.arange(N) // 128 == nb
    assert np.array_equal(acc0[:, ~cols], acc1[:, ~cols])
    t = fp8.dequant_table().astype(np.float64)
    blk = t[xq[:, kc * 128:(kc + 1) * 128]] @ t[w[cols, kc * 128:(kc + 1) * 128]].T
    contrib = blk * fp8.bf16_bits_to_f32(x_scale[:, kc])[:, None] * fp8.bf16_bits_to_f32(w_scale[nb, kc])
    assert np.allclose(acc1[:, cols] - acc0[:, cols], contrib, rtol=1e-5, atol=1e-5 * np.abs(acc0[:, cols]).max())
