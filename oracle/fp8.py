"""Oracle: FP8 E4M3FN quantisation of the KV cache (TEST INFRASTRUCTURE ONLY).

The reference writes bf16 K/V into a ``float8_e4m3fn`` cache with a bare
``tl.store`` (nanovllm/layers/attention.py:27-31); the implicit cast is a
round-to-nearest-even downcast with no scale (scale == 1), and the decode /
prefill kernels dequantise with a plain ``.to(tl.float32)``
(nanovllm/kernels/fp8_attention.py:147-150, 262-263, 292-293).

Numerical contract restated here:
  * finite |x| rounds to the nearest E4M3FN value, ties to even mantissa,
    including the subnormal range (quantum 2**-9 below 2**-6);
  * results whose magnitude would exceed 448 saturate to +-448 (the
    saturating ``satfinite`` conversion of the reference's NVIDIA lowering);
    +-inf therefore also give +-448;
  * NaN gives a NaN code (0x7F with the input's sign bit);
  * -0.0 gives 0x80.

Pinned by (tests/test_oracle_fp8.py): torch's own CPU cast
``Tensor.to(torch.float8_e4m3fn)`` over every bf16 bit pattern with
|x| <= 448 (an independent implementation), an integer bit-manipulation
re-derivation over all 65,536 patterns, round trips of all 256 codes,
every midpoint between adjacent codes (tie -> even code) and the
saturation / NaN / signed-zero special cases.
"""
import numpy as np

E4M3_MAX = 448.0


def bf16_bits_to_f32(bits):
    """uint16 bf16 bit patterns -> float32 values (exact)."""
    b = np.asarray(bits).astype(np.uint32)
    return (b << np.uint32(16)).view(np.float32)


def e4m3_decode(codes):
    """uint8 E4M3FN codes -> float32 values (exact; NaN for S.1111.111)."""
    c = np.asarray(codes).astype(np.int64)
    s = (c >> 7) & 1
    e = (c >> 3) & 0xF
    m = c & 7
    mag = np.where(e == 0, m * 2.0 ** -9, (8 + m) * np.exp2(e - 10.0))
    val = np.where(s == 1, -mag, mag)
    val = np.where((e == 15) & (m == 7), np.nan, val)
    return val.astype(np.float32)


def e4m3_encode(x):
    """float values -> uint8 E4M3FN codes, RNE with saturation to +-448.

    Works in the value domain: pick the quantum of |x|'s binade (2**(E-3),
    or 2**-9 in the subnormal range), round |x|/quantum to the nearest
    integer with ties to even (np.rint), rebuild the value, saturate, then
    encode it.
    """
    with np.errstate(invalid="ignore"):
        x = np.asarray(x, dtype=np.float64)
    nan = np.isnan(x)
    neg = np.signbit(x)
    a = np.abs(np.where(nan, 0.0, x))
    a = np.minimum(a, 1e300)                   # inf -> large finite (saturates below)
    _, ex = np.frexp(a)                        # a = f * 2**ex, f in [0.5, 1)
    binade = np.maximum(ex - 1, -6)            # floor(log2 a), clamped to the normal minimum
    q_exp = binade - 3                         # 3 mantissa bits
    r = np.rint(np.ldexp(a, -q_exp))           # integer multiple of the quantum, RNE
    val = np.ldexp(r, q_exp)
    val = np.minimum(val, E4M3_MAX)            # satfinite
    # encode the (now representable) magnitude
    _, ex2 = np.frexp(np.where(val > 0, val, 1.0))
    e2 = ex2 - 1
    sub = val < 2.0 ** -6
    m_sub = np.rint(val * 2.0 ** 9)
    m_norm = np.rint((np.ldexp(val, -e2) - 1.0) * 8.0)
    code = np.where(sub, m_sub, ((e2 + 7) << 3) + m_norm)
    code = np.where(val == 0, 0, code).astype(np.int64)
    code = np.where(nan, 0x7F, code)
    code = code | (neg.astype(np.int64) << 7)
    return code.astype(np.uint8)


_LUT = None


def bf16_to_e4m3_lut():
    """The 65,536-entry table bf16 bit pattern -> E4M3FN code."""
    global _LUT
    if _LUT is None:
        bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
        _LUT = e4m3_encode(bf16_bits_to_f32(bits))
        _LUT.setflags(write=False)
    return _LUT


def quantize_bf16_bits(bits):
    """uint16 bf16 bit patterns (any shape) -> uint8 E4M3FN codes."""
    return bf16_to_e4m3_lut()[np.asarray(bits).astype(np.uint16).astype(np.int64)]


def quantize_bf16_tensor(t):
    """torch bf16 tensor (CPU) -> torch uint8 tensor of E4M3FN codes."""
    import torch
    bits = t.contiguous().view(torch.int16).numpy().view(np.uint16)
    return torch.from_numpy(quantize_bf16_bits(bits).reshape(tuple(t.shape)))


_DEQ = None


def dequant_table():
    """float32[256]: value of every E4M3FN code."""
    global _DEQ
    if _DEQ is None:
        _DEQ = e4m3_decode(np.arange(256, dtype=np.uint8))
        _DEQ.setflags(write=False)
    return _DEQ


def dequant_codes_tensor(codes):
    """torch uint8 (or float8_e4m3fn) tensor -> torch float32 tensor (exact)."""
    import torch
    if codes.dtype == torch.float8_e4m3fn:
        codes = codes.view(torch.uint8)
    table = torch.from_numpy(dequant_table().copy())
    return table[codes.long()]


def quantize_f16_tensor(t):
    """torch fp16 tensor (CPU) -> torch uint8 tensor of E4M3FN codes: the
    value widened to float32 (exact), then rounded as e4m3_encode does."""
    import torch
    vals = t.contiguous().to(torch.float32).numpy()
    return torch.from_numpy(e4m3_encode(vals).reshape(tuple(t.shape)))


def store_kvcache(key, value, k_cache, v_cache, slot_mapping):
    """CPU restatement of store_kvcache (nanovllm/layers/attention.py:11-40).

    key/value: torch bf16 or fp16 [N, Hkv, D] (any row stride); the
    reference's tl.store converts them to the cache's float8e4nv
    (attention.py:30-31), rounding to nearest even with saturation.
    k_cache/v_cache: torch uint8 [P, bs, Hkv, D] written in place;
    slot_mapping: int [N], rows with slot == -1 are skipped (attention.py:24).
    """
    import torch
    N = key.shape[0]
    D = key.shape[1] * key.shape[2]
    slots = slot_mapping.to(torch.int64)
    keep = slots != -1
    if N == 0 or not bool(keep.any()):
        return
    quant = quantize_f16_tensor if key.dtype == torch.float16 else quantize_bf16_tensor
    kq = quant(key.reshape(N, D)[keep])
    vq = quant(value.reshape(N, D)[keep])
    kf = k_cache.view(-1, D)
    vf = v_cache.view(-1, D)
    kf[slots[keep]] = kq
    vf[slots[keep]] = vq
