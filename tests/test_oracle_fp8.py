"""Pins the oracle's E4M3FN quantisation (nanovllm/layers/attention.py:27-31 semantics).

Independent checks: the committed golden table (PyTorch's own CPU cast plus
the saturation rule), an integer re-derivation from the bf16 bit fields,
round trips of every code, tie-to-even at every midpoint, and the special
cases (saturation, inf, NaN, signed zero, subnormals).
"""
import hashlib
import os

import numpy as np
import pytest
import torch

from oracle import fp8

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "bf16_to_e4m3fn.bin")
GOLDEN_SHA256 = "556222ae80c3498b4da64795f283e77962f1045e2525faaededd4e0a5b1ae212"

BITS = np.arange(65536, dtype=np.uint32).astype(np.uint16)
VALUES = fp8.bf16_bits_to_f32(BITS)


def _int_rederivation(bits):
    """bf16 bit fields -> E4M3FN code with integer rounding (RNE + sticky)."""
    out = np.zeros(bits.shape, dtype=np.uint8)
    for idx, b in enumerate(bits.tolist()):
        s, e, m = b >> 15, (b >> 7) & 0xFF, b & 0x7F
        sign = s << 7
        if e == 0xFF:
            out[idx] = (0x7F if m else 0x7E) | sign
            continue
        if e == 0:  # bf16 zero / subnormal (< 2**-126) rounds to zero
            out[idx] = sign
            continue
        E = e - 127
        sig = 128 + m                      # value = sig * 2**(E-7)
        if E >= -6:
            q, r = sig >> 4, sig & 15
            if r > 8 or (r == 8 and (q & 1)):
                q += 1
            if q == 16:
                q, E = 8, E + 1
            if E > 8 or (E == 8 and q > 14):
                code = 0x7E
            else:
                code = ((E + 7) << 3) | (q - 8)
        else:
            shift = -(E + 2)               # value / 2**-9 = sig >> shift
            if shift > 16:
                code = 0
            else:
                q, r, half = sig >> shift, sig & ((1 << shift) - 1), 1 << (shift - 1)
                if r > half or (r == half and (q & 1)):
                    q += 1
                code = q                   # q == 8 is the smallest normal (code 8)
        out[idx] = code | sign
    return out


def test_golden_table_is_intact():
    data = np.fromfile(GOLDEN, dtype=np.uint8)
    assert data.size == 65536
    assert hashlib.sha256(data.tobytes()).hexdigest() == GOLDEN_SHA256


def test_oracle_matches_golden_table_exhaustively():
    golden = np.fromfile(GOLDEN, dtype=np.uint8)
    lut = fp8.bf16_to_e4m3_lut()
    finite = ~np.isnan(VALUES)
    assert np.array_equal(lut[finite], golden[finite])
    # NaN patterns: both give a NaN code (exponent and mantissa all ones)
    nan = np.isnan(VALUES)
    assert np.all((lut[nan] & 0x7F) == 0x7F) and np.all((golden[nan] & 0x7F) == 0x7F)


def test_oracle_matches_torch_cast_in_range():
    rng = np.abs(VALUES) <= 448
    t = torch.from_numpy(VALUES.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(fp8.bf16_to_e4m3_lut()[rng], t[rng])


def test_oracle_matches_integer_rederivation():
    assert np.array_equal(fp8.bf16_to_e4m3_lut(), _int_rederivation(BITS))


def test_every_code_round_trips():
    codes = np.arange(256, dtype=np.uint8)
    vals = fp8.e4m3_decode(codes)
    ok = ~np.isnan(vals)
    assert ok.sum() == 254
    assert np.array_equal(fp8.e4m3_encode(vals[ok]), codes[ok])
    # decoding agrees with torch's fp8 -> fp32 conversion
    t = torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(vals[ok], t[ok])


def test_midpoints_round_to_even():
    codes = np.arange(0, 0x7E, dtype=np.uint8)       # positive finite codes except max
    lo, hi = fp8.e4m3_decode(codes), fp8.e4m3_decode(codes + 1)
    mid = (lo.astype(np.float64) + hi.astype(np.float64)) / 2
    got = fp8.e4m3_encode(mid)
    want = np.where(codes % 2 == 0, codes, codes + 1)  # even mantissa wins
    assert np.array_equal(got, want)
    # just off the midpoint goes to the nearer side
    assert np.array_equal(fp8.e4m3_encode(np.nextafter(mid, 0)), codes)
    assert np.array_equal(fp8.e4m3_encode(np.nextafter(mid, np.inf)), codes + 1)


@pytest.mark.parametrize("x,code", [
    (448.0, 0x7E), (-448.0, 0xFE), (464.0, 0x7E), (465.0, 0x7E), (1e6, 0x7E), (-1e30, 0xFE),
    (float("inf"), 0x7E), (float("-inf"), 0xFE), (0.0, 0x00), (-0.0, 0x80),
    (2.0 ** -9, 0x01), (2.0 ** -10, 0x00), (1.5 * 2.0 ** -10, 0x01), (2.0 ** -6, 0x08),
    (7 * 2.0 ** -9, 0x07), (7.5 * 2.0 ** -9, 0x08), (1.0, 0x38), (-2.0, 0xC0), (240.0, 0x77),
])
def test_special_values(x, code):
    assert int(fp8.e4m3_encode(np.array([x]))[0]) == code


def test_nan_keeps_sign_and_is_nan():
    assert int(fp8.e4m3_encode(np.array([np.nan]))[0]) == 0x7F
    assert int(fp8.e4m3_encode(np.array([-np.nan]))[0]) == 0xFF


def test_store_restatement_skips_padding_and_honours_row_stride():
    torch.manual_seed(0)
    Hkv, D, bs, P = 2, 128, 16, 4
    qkv = torch.randn(5, (4 + 2 * Hkv) * D).to(torch.bfloat16)
    k = qkv[:, 4 * D:(4 + Hkv) * D].view(5, Hkv, D)
    v = qkv[:, (4 + Hkv) * D:].view(5, Hkv, D)
    kc = torch.full((P, bs, Hkv, D), 0xAB, dtype=torch.uint8)
    vc = torch.full((P, bs, Hkv, D), 0xCD, dtype=torch.uint8)
    slots = torch.tensor([3, -1, 17, 63, 0], dtype=torch.int32)
    fp8.store_kvcache(k, v, kc, vc, slots)
    kf, vf = kc.view(-1, Hkv * D), vc.view(-1, Hkv * D)
    for i, s in enumerate(slots.tolist()):
        if s == -1:
            continue
        assert torch.equal(kf[s], fp8.quantize_bf16_tensor(k[i].reshape(-1)))
        assert torch.equal(vf[s], fp8.quantize_bf16_tensor(v[i].reshape(-1)))
    untouched = torch.ones(P * bs, dtype=torch.bool)
    untouched[[3, 17, 63, 0]] = False
    assert bool((kf[untouched] == 0xAB).all()) and bool((vf[untouched] == 0xCD).all())


F16_BITS = np.arange(65536, dtype=np.uint32).astype(np.uint16)
F16_VALUES = F16_BITS.view(np.float16).astype(np.float32)


def test_fp16_inputs_match_torch_cast_in_range():
    """fp16 K/V (every pattern): the oracle's encoding of the widened value
    against torch's own fp16 -> float8_e4m3fn cast (an independent
    implementation) wherever torch's cast is defined the same way
    (|x| <= 448; beyond it torch gives NaN, the reference saturates)."""
    ok = np.abs(F16_VALUES) <= 448
    half = torch.from_numpy(F16_BITS.view(np.int16).copy()).view(torch.float16)
    t = half.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = fp8.quantize_f16_tensor(half).numpy()
    assert np.array_equal(got[ok], t[ok])
    assert ok.sum() > 30000


def test_fp16_inputs_saturate_and_keep_nan():
    half = torch.tensor([449.0, 65504.0, -1000.0, float("inf"), float("-inf"), float("nan"), 2.0 ** -24],
                        dtype=torch.float16)
    got = fp8.quantize_f16_tensor(half).tolist()
    assert got[:5] == [0x7E, 0x7E, 0xFE, 0x7E, 0xFE]
    assert got[5] & 0x7F == 0x7F
    assert got[6] == 0x00  # 2^-24 is far below half of the smallest subnormal (2^-10)


def test_store_restatement_fp16_matches_bf16_on_shared_values():
    """Values exact in both 16-bit types give the same cache bytes."""
    Hkv, D = 2, 128
    g = torch.Generator().manual_seed(3)
    x = (torch.randint(-255, 256, (6, Hkv, D), generator=g).float() / 32)
    slots = torch.tensor([5, 0, -1, 9, 2, 7], dtype=torch.int32)
    caches = []
    for dt in (torch.float16, torch.bfloat16):
        kc = torch.zeros((3, 4, Hkv, D), dtype=torch.uint8)
        vc = torch.zeros_like(kc)
        fp8.store_kvcache(x.to(dt), (-x).to(dt), kc, vc, slots)
        caches.append((kc, vc))
    assert torch.equal(caches[0][0], caches[1][0]) and torch.equal(caches[0][1], caches[1][1])
    assert int(caches[0][0].count_nonzero()) > 0
