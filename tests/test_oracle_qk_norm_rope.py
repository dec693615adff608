"""Pins the oracle's q/k RMSNorm + RoPE + FP8 store (oracle/qk_norm_rope.py)
against independent formulations: torch's rms_norm in float64, a complex
rotation in float64, closed forms and invariants (CPU only)."""
import math

import numpy as np
import torch

from oracle import fp8 as ofp8
from oracle import qk_norm_rope as oq

D = 128


def _bf16(*shape, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def test_rms_norm_matches_float64_rms_norm_then_weight():
    x = _bf16(64, 8, D, seed=1, scale=3.0)
    w = (1.0 + 0.1 * _bf16(D, seed=2).float()).to(torch.bfloat16)
    eps = 1e-6
    got = oq.rms_norm_bf16(x, w, eps)
    ref = torch.nn.functional.rms_norm(x.double(), (D,), eps=eps).to(torch.bfloat16)
    want = (ref.float() * w.float()).to(torch.bfloat16)
    diff = (got.float() - want.float()).abs()
    ulp = want.float().abs().clamp(min=1e-30) * 2.0 ** -7
    assert bool((diff <= ulp).all()), float((diff / ulp).max())
    assert (got == want).float().mean() > 0.995  # fp32 vs fp64 only flips rare rounding boundaries


def test_fused_rms_norm_rounds_once():
    """The single-rounding form (inductor without emulated precision casts):
    within half a bf16 ulp of the float64 product rms_norm(x) * w (one
    rounding of a value computed in fp32), and the two-rounding form differs
    from it by at most one ulp, in a minority of elements."""
    x = _bf16(64, 8, D, seed=11, scale=3.0)
    w = (1.0 + 0.1 * _bf16(D, seed=12).float()).to(torch.bfloat16)
    eps = 1e-6
    fused = oq.rms_norm_bf16(x, w, eps, fused_norm=True)
    exact = torch.nn.functional.rms_norm(x.double(), (D,), eps=eps) * w.double()
    ulp = fused.double().abs().clamp(min=1e-30) * 2.0 ** -7
    assert bool(((fused.double() - exact).abs() <= 0.5 * ulp * 1.01).all())
    eager = oq.rms_norm_bf16(x, w, eps)
    assert bool(((eager.double() - fused.double()).abs() <= ulp * 1.01).all())
    same = (eager == fused).float().mean().item()
    assert 0.5 < same < 1.0, same  # double rounding moves some elements, not most


def test_rms_norm_constant_vector_gives_the_weight():
    w = _bf16(D, seed=3)
    for c in (0.5, -3.0, 100.0):
        x = torch.full((2, 1, D), c).to(torch.bfloat16)
        got = oq.rms_norm_bf16(x, w, 1e-6)
        want = (w.float() * math.copysign(1.0, c)).to(torch.bfloat16)
        assert torch.equal(got[0, 0], want) and torch.equal(got[1, 0], want)


def test_rope_is_a_complex_rotation_by_the_cached_angles():
    cache = oq.rope_cache(D, 4096, 1e6)
    x = _bf16(50, 4, D, seed=4)
    pos = torch.randint(0, 4096, (50,), generator=torch.Generator().manual_seed(5))
    got = oq.rope_bf16(x, pos, cache).double()
    z = torch.complex(x[..., :D // 2].double(), x[..., D // 2:].double())
    cs = cache[pos].double().unsqueeze(1)
    rot = torch.complex(cs[..., :D // 2], cs[..., D // 2:])
    zr = z * rot
    want = torch.cat((zr.real, zr.imag), dim=-1)
    diff = (got - want).abs()
    assert bool((diff <= want.abs() * 2.0 ** -8 + 1e-6).all())


def test_rope_cache_angles_are_position_times_inverse_frequency():
    base, maxp = 1e6, 2048
    cache = oq.rope_cache(D, maxp, base).double()
    j = np.arange(D // 2)
    inv = 1.0 / (base ** (2.0 * j / D))
    for p in (0, 1, 7, 1000, 2047):
        ang = p * inv
        assert np.allclose(cache[p, :D // 2].numpy(), np.cos(ang), atol=3e-4)
        assert np.allclose(cache[p, D // 2:].numpy(), np.sin(ang), atol=3e-4)


def test_rope_position_zero_is_the_identity_and_preserves_pair_norms():
    cache = oq.rope_cache(D, 512, 1e4)
    x = _bf16(16, 2, D, seed=6)
    assert torch.equal(oq.rope_bf16(x, torch.zeros(16, dtype=torch.int64), cache), x)
    y = oq.rope_bf16(x, torch.arange(16) * 31, cache).double()
    xd = x.double()
    n_in = xd[..., :D // 2] ** 2 + xd[..., D // 2:] ** 2
    n_out = y[..., :D // 2] ** 2 + y[..., D // 2:] ** 2
    assert torch.allclose(n_out, n_in, rtol=2e-2, atol=1e-4)


def test_qk_norm_rope_store_splits_and_stores():
    Hq, Hkv, N, bs, P = 8, 2, 40, 16, 8
    qkv = _bf16(N, (Hq + 2 * Hkv) * D, seed=7)
    wq, wk = _bf16(D, seed=8), _bf16(D, seed=9)
    cache = oq.rope_cache(D, 1024, 1e6)
    pos = torch.randint(0, 1024, (N,), generator=torch.Generator().manual_seed(10))
    slots = torch.randperm(P * bs, generator=torch.Generator().manual_seed(11))[:N].to(torch.int32)
    slots[::4] = -1
    kc = torch.full((P, bs, Hkv, D), 0x5A, dtype=torch.uint8)
    vc = torch.full((P, bs, Hkv, D), 0x5A, dtype=torch.uint8)
    q, k = oq.qk_norm_rope_store(qkv, Hq, Hkv, D, pos, wq, wk, 1e-6, cache, kc, vc, slots)
    want_q = oq.rope_bf16(oq.rms_norm_bf16(qkv[:, :Hq * D].reshape(N, Hq, D), wq, 1e-6), pos, cache)
    assert torch.equal(q, want_q)
    v = qkv[:, (Hq + Hkv) * D:].reshape(N, Hkv, D)
    kf, vf = kc.view(-1, Hkv * D), vc.view(-1, Hkv * D)
    for i in range(N):
        s = int(slots[i])
        if s < 0:
            continue
        assert torch.equal(kf[s], ofp8.quantize_bf16_tensor(k[i].reshape(-1)))
        assert torch.equal(vf[s], ofp8.quantize_bf16_tensor(v[i].reshape(-1)))
    untouched = torch.ones(P * bs, dtype=torch.bool)
    untouched[slots[slots >= 0].long()] = False
    assert bool((kf[untouched] == 0x5A).all()) and bool((vf[untouched] == 0x5A).all())
