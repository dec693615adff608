"""FP8 block-scaled linear on the GPU (nanovllm/kernels/fp8_linear.py:11-139)
against the oracle.

Activation quantisation is byte-exact (codes and bf16 scales).  The GEMM is
bit-exact where every step is exact (small-integer codes, power-of-two
scales).  Otherwise it is within one output ulp of the oracle's fp32
accumulator plus 2^-11 of the sum of absolute terms: the oracle sums each
128-wide block exactly, while gfx950's FP8 MFMA sums a block's products
aligned to the largest one in a window of 14 bits (a term more than 2^13
below the block's largest product is dropped: measured with cancelling
448 x 448 products beside one small term), the same kind of reduced-width
FP8 dot product NVIDIA's tensor cores compute for the reference, which is why
the reference promotes to fp32 every 128 elements.  On random codes the
largest error seen is 2^-15 of the sum of absolute terms; a misplaced or
missing K block errs by about 2^-3.5 of it.

Shapes are chosen so that on a 256-CU MI355X the library picks each of its
tile shapes (256x256, 128x64, 128x32, 64x16 features x tokens): it takes the
largest tile whose grid still covers the CUs.  65 to 192 tokens with at least
a CU's worth of 96-feature tiles take the 96x192 tile with a 4-stage ring
(tiles straddle the 128-row weight blocks, so fragments take their own
scales; K shorter than the ring).  Products with at most 256 tokens whose tile
grid would leave CUs idle take the small-M kernel instead (weights streamed
once; K split over workgroups with fp32 partials added in split order when the
workspace allows): its cases cover 1 to 256 tokens, 2, 4 and 8 compute waves,
splits and no workspace.
"""
import numpy as np
import pytest
import torch

from gpu_util import announce
from oracle import fp8
from oracle import fp8_linear as ol
from nanovllm_amd.kernels.fp8_linear import fp8_block_linear
from nanovllm_amd import _native

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def _codes(g, shape):
    c = torch.randint(0, 256, shape, generator=g, dtype=torch.int32).to(torch.uint8)
    return torch.where((c & 0x7F) == 0x7F, c ^ 0x01, c)   # no NaN codes


def _scales(g, shape, lo=-4, hi=1):
    return (10.0 ** torch.empty(shape).uniform_(lo, hi, generator=g)).to(torch.bfloat16)


# tolerance of the GEMM against the oracle's fp32 accumulator (module docstring)
ABS_TOL = 2.0 ** -11


def _gemm_gpu(xq, x_scale, w, w_scale, out_dtype=torch.bfloat16, w_stride=None, out_stride=None, ws_bytes=None):
    """Calls nvamd_fp8_block_gemm on device copies; optional padded row
    strides; ws_bytes: the workspace given (default: the size the library
    asks for)."""
    M, K = xq.shape
    N = w.shape[0]
    lib = _native.load()
    xq_d = xq.cuda().contiguous()
    xs_d = x_scale.cuda().contiguous()
    ws = w_stride or K
    w_buf = torch.zeros(N, ws, dtype=torch.uint8, device="cuda")
    w_buf[:, :K] = w.cuda()
    os_ = out_stride or N
    out_buf = torch.full((max(M, 1), os_), float("nan"), dtype=out_dtype, device="cuda")
    wsc = w_scale.cuda().contiguous()
    code = 0 if out_dtype == torch.bfloat16 else 1
    if ws_bytes is None:
        ws_bytes = lib.nvamd_fp8_block_gemm_workspace_bytes(M, N, K)
    gws = torch.full((max(ws_bytes, 16),), 0x7F, dtype=torch.uint8, device="cuda")  # NaN-filled partials
    st = lib.nvamd_fp8_block_gemm(xq_d.data_ptr(), xs_d.data_ptr(), w_buf.data_ptr(), ws, wsc.data_ptr(),
                                  out_buf.data_ptr(), os_, code, M, N, K, gws.data_ptr() if ws_bytes else None,
                                  ws_bytes, torch.cuda.current_stream().cuda_stream)
    _native.check(st, "fp8_block_gemm")
    torch.cuda.synchronize()
    if out_stride:
        assert torch.isnan(out_buf[:M, N:].float()).all(), "wrote past the row"
    return out_buf[:M, :N].cpu()


def _f64(xq, x_scale, w, w_scale):
    t = torch.from_numpy(fp8.dequant_table().astype(np.float64))
    xd = t[xq.long()] * x_scale.double().repeat_interleave(128, 1)
    wd = t[w.long()] * w_scale.double().repeat_interleave(128, 0).repeat_interleave(128, 1)
    return xd @ wd.T, xd.abs() @ wd.abs().T


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_act_quant_byte_exact(dtype):
    announce(f"fp8 linear: activation quant {dtype}")
    g = torch.Generator().manual_seed(21)
    M, K = 77, 2048
    lo, hi = (-30, 30) if dtype == torch.bfloat16 else (-5, 4)
    mag = 10.0 ** torch.empty(M, K // 128, 1).uniform_(lo, hi, generator=g)
    x = (torch.randn(M, K // 128, 128, generator=g) * mag).reshape(M, K)
    x[3, :128] = 0.0                    # zero group
    x[4, 128:256] = -1.25               # constant group
    x[5, 256:384] = 0.0
    x[5, 300] = 3.0                     # single non-zero element
    x = x.to(dtype)
    xq_ref, xs_ref, _ = ol.act_quant(x)
    lib = _native.load()
    xd = x.cuda()
    xq = torch.empty(M, K, dtype=torch.uint8, device="cuda")
    xs = torch.empty(M, K // 128, dtype=torch.bfloat16, device="cuda")
    _native.check(lib.nvamd_fp8_act_quant(xd.data_ptr(), K, 0 if dtype == torch.bfloat16 else 1, xq.data_ptr(),
                                          xs.data_ptr(), M, K, torch.cuda.current_stream().cuda_stream), "act_quant")
    torch.cuda.synchronize()
    assert np.array_equal(xq.cpu().numpy(), xq_ref)
    assert np.array_equal(_bits(xs), xs_ref)


def test_act_quant_unit_scale_all_patterns_and_strided_rows():
    """Every finite bf16 value with |x| <= 448 in groups holding 448 (scale
    exactly 1), read through a row stride wider than K."""
    announce("fp8 linear: activation quant, all bf16 patterns at scale 1, strided rows")
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    vals = fp8.bf16_bits_to_f32(bits)
    vals = vals[np.isfinite(vals) & (np.abs(vals) <= 448.0)]
    groups = -(-len(vals) // 127)
    groups += groups % 2
    x = np.full((groups, 128), 448.0, dtype=np.float32)
    flat = np.zeros(groups * 127, dtype=np.float32)
    flat[:len(vals)] = vals
    x[:, 1:] = flat.reshape(groups, 127)
    x = torch.from_numpy(x.reshape(groups // 2, 256)).to(torch.bfloat16)
    M, K = x.shape
    wide = torch.zeros(M, K + 64, dtype=torch.bfloat16)
    wide[:, :K] = x
    xq_ref, xs_ref, _ = ol.act_quant(x)
    lib = _native.load()
    wd = wide.cuda()
    xq = torch.empty(M, K, dtype=torch.uint8, device="cuda")
    xs = torch.empty(M, K // 128, dtype=torch.bfloat16, device="cuda")
    _native.check(lib.nvamd_fp8_act_quant(wd.data_ptr(), K + 64, 0, xq.data_ptr(), xs.data_ptr(), M, K,
                                          torch.cuda.current_stream().cuda_stream), "act_quant")
    torch.cuda.synchronize()
    assert np.array_equal(xq.cpu().numpy(), xq_ref)
    assert np.array_equal(_bits(xs), xs_ref)


# (M, N, K): tile chosen on 256 CUs -> 256x256: (4096, 4096, 256), and (4096, 4096, 640) with an odd
# number of K blocks (a token row's scale then sits in either half of its x_scale dword);
# 128x64: (1024, 2048, 256); 128x32: (1024, 1024, 128); 64x16: (300, 128, 256)
TILE_SHAPES = [(4096, 4096, 256), (4096, 4096, 640), (1024, 2048, 256), (1024, 1024, 128), (300, 128, 256)]
# at most 256 tokens: the Qwen3-8B qkv and down products at 192 tokens take the small-M kernel (down with K
# split over workgroups), gate/up the 96x192 ring tile; 256 tokens (16 token fragments), one token (K split),
# ragged token counts and odd K block counts on the small-M kernel
SKINNY_SHAPES = [(192, 6144, 4096), (192, 24576, 4096), (192, 4096, 12288), (256, 1024, 4096), (1, 4096, 4096),
                 (24, 256, 512), (1, 128, 128), (77, 2048, 1664), (130, 512, 3200)]
# the 96x192 ring tile: ragged tokens with an odd number of K blocks, K shorter than the ring (2 and 1 blocks),
# 65 tokens (its lower bound)
RING_SHAPES = [(100, 24576, 640), (150, 24576, 256), (192, 24576, 128), (65, 24576, 1024)]


@pytest.mark.parametrize("M,N,K", TILE_SHAPES + SKINNY_SHAPES + RING_SHAPES)
def test_gemm_exact_integer_case(M, N, K):
    """Small-integer codes, power-of-two scales: every fp32 step is exact, so
    the GPU must equal the oracle bit for bit (a transposed operand, a wrong
    K pairing between the MFMA operands or a misplaced scale fails)."""
    announce(f"fp8 linear: exact GEMM M={M} N={N} K={K}")
    g = torch.Generator().manual_seed(M + N + K)
    ints = torch.tensor([-4.0, -3.0, -2.0, -1.0, 0.0, 1.0, 2.0, 3.0, 4.0])
    xq = ints[torch.randint(0, 9, (M, K), generator=g)].to(torch.float8_e4m3fn).view(torch.uint8)
    w = ints[torch.randint(0, 9, (N, K), generator=g)].to(torch.float8_e4m3fn).view(torch.uint8)
    x_scale = (2.0 ** torch.randint(-3, 4, (M, K // 128), generator=g).float()).to(torch.bfloat16)
    w_scale = (2.0 ** torch.randint(-3, 4, (N // 128, K // 128), generator=g).float()).to(torch.bfloat16)
    got = _gemm_gpu(xq, x_scale, w, w_scale)
    want, _ = ol.block_gemm(xq.numpy(), _bits(x_scale), w.numpy(), _bits(w_scale))
    assert np.array_equal(_bits(got), want)


@pytest.mark.parametrize("M,N,K,out_dtype", [(4000, 4096, 384, torch.bfloat16), (1000, 2048, 512, torch.bfloat16),
                                             (77, 1024, 1024, torch.float16), (5, 384, 4096, torch.bfloat16),
                                             (130, 256, 12288, torch.bfloat16), (160, 24576, 768, torch.bfloat16),
                                             (96, 24576, 512, torch.float16)])
def test_gemm_matches_oracle(M, N, K, out_dtype):
    """Random codes (all finite E4M3FN values) and scales over five decades
    (two for the fp16 output, which must stay below 65504); ragged M, K up to
    12,288 (96 scale blocks)."""
    announce(f"fp8 linear: GEMM M={M} N={N} K={K} {out_dtype}")
    g = torch.Generator().manual_seed(M * 3 + N + K)
    xq, w = _codes(g, (M, K)), _codes(g, (N, K))
    lo, hi = (-4, 1) if out_dtype == torch.bfloat16 else (-4, -2)
    x_scale, w_scale = _scales(g, (M, K // 128), lo, hi), _scales(g, (N // 128, K // 128), lo, hi)
    got = _gemm_gpu(xq, x_scale, w, w_scale, out_dtype).double()
    _, acc = ol.block_gemm(xq.numpy(), _bits(x_scale), w.numpy(), _bits(w_scale),
                           "bf16" if out_dtype == torch.bfloat16 else "fp16")
    _, absum = _f64(xq, x_scale, w, w_scale)
    acc = torch.from_numpy(acc).double()
    ulp = 2.0 ** -7 if out_dtype == torch.bfloat16 else 2.0 ** -10
    bad = (got - acc).abs() > ulp * acc.abs() + ABS_TOL * absum
    assert not bad.any(), f"{int(bad.sum())} outputs off, first at {bad.nonzero()[0].tolist()}"


def test_gemm_large_tile_long_k_against_torch_fp32():
    """The 256x256 tile at the Qwen3-8B down-projection depth (K = 12,288, 96
    scale blocks; 4,000 tokens, ragged against the tile), against the same
    block-scaled sum in torch fp32 on the GPU (per K block an fp32 matmul of
    the dequantised codes, times x_scale * w_scale), at the oracle's
    tolerance.  The full-size oracle would take minutes on the host."""
    announce("fp8 linear: GEMM 4000 x 4096 x 12288 (256x256 tile) vs torch fp32")
    g = torch.Generator().manual_seed(12288)
    M, N, K = 4000, 4096, 12288
    xq, w = _codes(g, (M, K)), _codes(g, (N, K))
    x_scale, w_scale = _scales(g, (M, K // 128)), _scales(g, (N // 128, K // 128))
    got = _gemm_gpu(xq, x_scale, w, w_scale).cuda().double()
    t = torch.from_numpy(fp8.dequant_table().astype(np.float32)).cuda()
    xd, wd = t[xq.cuda().long()], t[w.cuda().long()]
    xs, ws = x_scale.cuda().float(), w_scale.cuda().float().repeat_interleave(128, 0)
    acc = torch.zeros(M, N, device="cuda")
    absum = torch.zeros(M, N, device="cuda")
    for kc in range(K // 128):
        xb, wb = xd[:, 128 * kc:128 * (kc + 1)], wd[:, 128 * kc:128 * (kc + 1)].T.contiguous()
        s = xs[:, kc:kc + 1] * ws[:, kc][None, :]
        acc += torch.matmul(xb, wb) * s
        absum += torch.matmul(xb.abs(), wb.abs()) * s
    bad = (got - acc.double()).abs() > 2.0 ** -7 * acc.double().abs() + ABS_TOL * absum.double()
    assert not bad.any(), f"{int(bad.sum())} outputs off, first at {bad.nonzero()[0].tolist()}"


def test_gemm_strided_weight_and_output_rows():
    """Weight rows with a padded stride, output rows with a padded stride (the
    padding must stay untouched)."""
    announce("fp8 linear: GEMM with strided weight and output rows")
    g = torch.Generator().manual_seed(9)
    M, N, K = 40, 384, 640
    xq, w = _codes(g, (M, K)), _codes(g, (N, K))
    x_scale, w_scale = _scales(g, (M, K // 128)), _scales(g, (N // 128, K // 128))
    got = _gemm_gpu(xq, x_scale, w, w_scale, w_stride=K + 128, out_stride=N + 8).double()
    _, acc = ol.block_gemm(xq.numpy(), _bits(x_scale), w.numpy(), _bits(w_scale))
    _, absum = _f64(xq, x_scale, w, w_scale)
    acc = torch.from_numpy(acc).double()
    assert not ((got - acc).abs() > 2.0 ** -7 * acc.abs() + ABS_TOL * absum).any()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fp8_block_linear_matches_oracle(dtype):
    """The drop-in fp8_block_linear (quant + GEMM) against the oracle's
    block_linear at K = 4096 (Qwen3-8B hidden size) with 300 tokens."""
    announce(f"fp8 linear: fp8_block_linear {dtype}")
    g = torch.Generator().manual_seed(4)
    M, N, K = 300, 1024, 4096
    x = (torch.randn(M, K, generator=g) * 3).to(dtype)
    w = _codes(g, (N, K))
    w_scale = (torch.rand(N // 128, K // 128, generator=g) * 2e-3).to(torch.bfloat16)
    got = fp8_block_linear(x.cuda(), w.cuda().view(torch.float8_e4m3fn), w_scale.cuda())
    torch.cuda.synchronize()
    assert got.dtype == dtype and got.shape == (M, N)
    xq, xs, _ = ol.act_quant(x)
    _, acc = ol.block_gemm(xq, xs, w.numpy(), _bits(w_scale), "bf16" if dtype == torch.bfloat16 else "fp16")
    _, absum = _f64(torch.from_numpy(xq), torch.from_numpy(xs.view(np.int16)).view(torch.bfloat16), w, w_scale)
    acc = torch.from_numpy(acc).double()
    ulp = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10
    assert not ((got.cpu().double() - acc).abs() > ulp * acc.abs() + ABS_TOL * absum).any()


def test_skinny_gemm_split_repeatable_and_without_workspace():
    """The Qwen3-8B down projection at 192 tokens (K = 12,288 split over
    workgroups): random codes and scales against the oracle, the same bits on
    a second call (partials added in split order), and the unsplit product
    (no workspace) within the same tolerance."""
    announce("fp8 linear: small-M GEMM 192 x 4096 x 12288, split and unsplit")
    lib = _native.load()
    g = torch.Generator().manual_seed(192)
    M, N, K = 192, 4096, 12288
    assert lib.nvamd_fp8_block_gemm_workspace_bytes(M, N, K) > 0, "this product splits K"
    xq, w = _codes(g, (M, K)), _codes(g, (N, K))
    x_scale, w_scale = _scales(g, (M, K // 128)), _scales(g, (N // 128, K // 128))
    got = _gemm_gpu(xq, x_scale, w, w_scale)
    again = _gemm_gpu(xq, x_scale, w, w_scale)
    assert torch.equal(got.view(torch.int16), again.view(torch.int16)), "split sums differ between calls"
    unsplit = _gemm_gpu(xq, x_scale, w, w_scale, ws_bytes=0)
    _, acc = ol.block_gemm(xq.numpy(), _bits(x_scale), w.numpy(), _bits(w_scale))
    _, absum = _f64(xq, x_scale, w, w_scale)
    acc = torch.from_numpy(acc).double()
    for name, out in (("split", got), ("unsplit", unsplit)):
        bad = (out.double() - acc).abs() > 2.0 ** -7 * acc.abs() + ABS_TOL * absum
        assert not bad.any(), f"{name}: {int(bad.sum())} outputs off, first at {bad.nonzero()[0].tolist()}"


@pytest.mark.parametrize("M,N,K,out_dtype", [(192, 6144, 4096, torch.bfloat16), (256, 2048, 4096, torch.float16),
                                             (33, 1024, 2048, torch.bfloat16)])
def test_skinny_gemm_matches_oracle(M, N, K, out_dtype):
    """Random codes and scales over five decades (two for fp16 outputs) on the
    small-M kernel, against the oracle's accumulator."""
    announce(f"fp8 linear: small-M GEMM M={M} N={N} K={K} {out_dtype}")
    g = torch.Generator().manual_seed(M * 7 + N + K)
    xq, w = _codes(g, (M, K)), _codes(g, (N, K))
    lo, hi = (-4, 1) if out_dtype == torch.bfloat16 else (-4, -2)
    x_scale, w_scale = _scales(g, (M, K // 128), lo, hi), _scales(g, (N // 128, K // 128), lo, hi)
    got = _gemm_gpu(xq, x_scale, w, w_scale, out_dtype).double()
    _, acc = ol.block_gemm(xq.numpy(), _bits(x_scale), w.numpy(), _bits(w_scale),
                           "bf16" if out_dtype == torch.bfloat16 else "fp16")
    _, absum = _f64(xq, x_scale, w, w_scale)
    acc = torch.from_numpy(acc).double()
    ulp = 2.0 ** -7 if out_dtype == torch.bfloat16 else 2.0 ** -10
    bad = (got - acc).abs() > ulp * acc.abs() + ABS_TOL * absum
    assert not bad.any(), f"{int(bad.sum())} outputs off, first at {bad.nonzero()[0].tolist()}"
