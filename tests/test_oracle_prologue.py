"""Pins the oracle's indexer prologue (query RoPE/Hadamard/quant/gate and the key
LayerNorm/RoPE/Hadamard/quant) on the CPU.

The reference's own test of this stage (tests/test_indexer_transform.py:72-182)
needs CUDA and the fast_hadamard_transform package, neither present here; its
composition is restated below with independent routines: torch's LayerNorm and
bf16 casts, numpy complex multiplication for the rotation, scipy's Sylvester
Hadamard matrix in float64. The oracle computes in IEEE f32 in one fixed order,
so against these float64 routines it may differ by one fp8 step where a value
sits on a rounding boundary; the tests bound how often that happens.
"""
import numpy as np
import pytest
import scipy.linalg
import torch

import oracle as O


def _bf16(x):
    return O.f32_to_bf16(np.asarray(x, np.float32))


# ----------------------------------------------------------------- building blocks
def test_ue8m0_ceil_exact_at_and_just_above_powers_of_two():
    k = np.arange(-30, 10)
    p = np.ldexp(np.float32(1), k).astype(np.float32)
    assert np.array_equal(O.ue8m0_ceil(p), p)
    above = np.nextafter(p, np.float32(np.inf))
    assert np.array_equal(O.ue8m0_ceil(above), (2 * p).astype(np.float32))
    below = np.nextafter(p, np.float32(0))
    assert np.array_equal(O.ue8m0_ceil(below), p)


def test_interleaved_to_half_known_answer():
    got = O.interleaved_to_half(np.arange(64))
    assert np.array_equal(got, np.r_[np.arange(0, 64, 2), np.arange(1, 64, 2)])
    # on a batch, the permutation acts on the last axis only
    x = np.arange(3 * 64).reshape(3, 64)
    assert np.array_equal(O.interleaved_to_half(x)[2], got + 128)


def test_hadamard128_matches_sylvester_matrix():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((50, 128)).astype(np.float32)
    H = scipy.linalg.hadamard(128).astype(np.float64)
    ref = x.astype(np.float64) @ H.T / np.sqrt(128.0)
    np.testing.assert_allclose(O.hadamard128(x), ref, rtol=0, atol=2e-6 * np.abs(x).max() * 12)
    # orthonormal and an involution: applying it twice returns the input
    np.testing.assert_allclose(O.hadamard128(O.hadamard128(x)), x, atol=1e-5)
    # unit vectors give the (scaled) rows of H, sign pattern (-1)^popcount(o & i)
    for i in (0, 1, 37, 127):
        e = np.zeros(128, np.float32)
        e[i] = 1
        row = O.hadamard128(e)
        sign = np.array([(-1) ** bin(o & i).count("1") for o in range(128)], np.float64)
        np.testing.assert_allclose(row, sign / np.sqrt(128), rtol=1e-6)


def test_rope_neox_matches_complex_rotation():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((20, 64)).astype(np.float32)
    theta = rng.uniform(-np.pi, np.pi, (20, 32))
    cos, sin = np.cos(theta).astype(np.float32), np.sin(theta).astype(np.float32)
    got = O.rope_neox(x, cos, sin)
    z = (x[:, :32] + 1j * x[:, 32:]).astype(np.complex128) * (cos + 1j * sin.astype(np.float64))
    np.testing.assert_allclose(got[:, :32], z.real, atol=1e-5)
    np.testing.assert_allclose(got[:, 32:], z.imag, atol=1e-5)
    # rotation preserves each pair's norm; position 0 of the cache is the identity
    np.testing.assert_allclose(np.hypot(got[:, :32], got[:, 32:]), np.hypot(x[:, :32], x[:, 32:]), rtol=1e-5)
    cs = O.rope_cos_sin_cache(4)
    assert np.array_equal(O.rope_neox(x, cs[0, :32], cs[0, 32:]), x)


def test_rope_cache_matches_closed_form():
    cs = O.rope_cos_sin_cache(1000)
    t = np.arange(1000)[:, None]
    inv = 10000.0 ** (-np.arange(0, 64, 2) / 64.0)
    np.testing.assert_allclose(cs[:, :32], np.cos(t * inv), atol=2e-4)
    np.testing.assert_allclose(cs[:, 32:], np.sin(t * inv), atol=2e-4)


def test_tree_sum_matches_float64_sum():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((100, 128)).astype(np.float32)
    np.testing.assert_allclose(O.f32_tree_sum128(x), x.astype(np.float64).sum(-1), atol=1e-5)
    # integers small enough to be exact in f32 sum exactly in any order
    xi = rng.integers(-1000, 1000, (10, 128)).astype(np.float32)
    assert np.array_equal(O.f32_tree_sum128(xi), xi.sum(-1).astype(np.float32))


# ----------------------------------------------------------------- composed stages
def _torch_reference_q(q_u16, gate_u16, weight_scale, cs, positions, interleaved=True):
    """The composition of tests/test_indexer_transform.py:72-116 with float64 routines."""
    q = torch.from_numpy(q_u16.view(np.int16)).view(torch.bfloat16)
    half = q[..., :64].float().numpy()
    if interleaved:
        half = half.reshape(*half.shape[:-1], 32, 2).swapaxes(-1, -2).reshape(half.shape)
    c = cs[positions][:, None, :32].astype(np.float64)
    s = cs[positions][:, None, 32:].astype(np.float64)
    z = (half[..., :32] + 1j * half[..., 32:]) * (c + 1j * s)
    rot = np.concatenate([z.real, z.imag], -1)
    full = q.float().numpy().astype(np.float64)
    full[..., :64] = torch.from_numpy(rot).to(torch.bfloat16).double().numpy()
    H = scipy.linalg.hadamard(128).astype(np.float64)
    had = torch.from_numpy(full @ H.T * 128 ** -0.5).to(torch.bfloat16).float()
    amax = had.abs().amax(-1, keepdim=True).clamp(min=1e-4)
    scale = torch.exp2(torch.ceil(torch.log2(amax / 448.0)))
    codes = (had / scale).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    g = torch.from_numpy(gate_u16.view(np.int16)).view(torch.bfloat16).float()
    weights = (g.unsqueeze(-1) * weight_scale * scale).squeeze(-1).numpy()
    return codes, weights, scale.squeeze(-1).numpy()


def _assert_near_codes(got, ref, max_frac):
    diff = got != ref
    frac = diff.mean()
    assert frac <= max_frac, f"{frac:.2e} of codes differ"
    # a differing code is one fp8 step away (same sign, adjacent magnitude)
    g, r = got[diff].astype(np.int32), ref[diff].astype(np.int32)
    assert np.all((g & 0x80) == (r & 0x80)) and np.all(np.abs((g & 0x7F) - (r & 0x7F)) == 1)


@pytest.mark.parametrize("interleaved", [True, False])
def test_q_prologue_matches_float64_composition(interleaved):
    rng = np.random.default_rng(3)
    T, H = 6, 16
    q = _bf16(rng.standard_normal((T, H, 128)))
    gate = _bf16(rng.standard_normal((T, H)))
    cs = O.rope_cos_sin_cache(1024)
    pos = np.array([0, 3, 29, 511, 1000, 7])
    codes, weights = O.indexer_q_prologue(q, gate, 0.03125, cs, pos, interleaved)
    rc, rw, rs = _torch_reference_q(q, gate, 0.03125, cs, pos, interleaved)
    _assert_near_codes(codes, rc, 2e-3)
    # the scale is a power of two fixed by amax; weights = gate * weight_scale * scale exactly
    same_scale = np.isclose(weights, rw, rtol=0, atol=0)
    assert same_scale.mean() >= 0.98
    # round trip: decoded codes times the scale recover the Hadamard output within fp8 precision
    sf = rw / (O.bf16_to_f32(gate) * np.float32(0.03125))
    dec = O.fp8_e4m3fn_decode(codes) * sf[..., None]
    full = O.bf16_to_f32(q).astype(np.float64)
    assert np.all(np.abs(dec).max(-1) <= 448 * sf + 1e-12)
    assert np.linalg.norm(dec) > 0.9 * np.linalg.norm(full)   # orthonormal: energy is kept


def test_q_prologue_position_zero_is_pure_hadamard():
    rng = np.random.default_rng(4)
    q = _bf16(rng.standard_normal((1, 4, 128)))
    gate = _bf16(np.ones((1, 4)))
    cs = O.rope_cos_sin_cache(8)
    codes, w = O.indexer_q_prologue(q, gate, 1.0, cs, np.array([0]), rope_interleaved=False)
    y = O.bf16_to_f32(_bf16(O.hadamard128(O.bf16_to_f32(q))))
    c2, s2 = O.quantize_rows_ue8m0(y)
    assert np.array_equal(codes, c2) and np.array_equal(w, s2)


def test_k_transform_matches_float64_composition():
    rng = np.random.default_rng(5)
    T = 64
    key = _bf16(rng.standard_normal((T, 128)) * 3 + 0.5)
    w = rng.standard_normal(128).astype(np.float32)
    b = rng.standard_normal(128).astype(np.float32)
    cs = O.rope_cos_sin_cache(1024)
    pos = rng.integers(0, 1024, T)
    codes, scales = O.indexer_k_transform(key, w, b, 1e-5, cs, pos)
    # float64 composition of tests/test_indexer_transform.py:119-182
    kt = torch.from_numpy(key.view(np.int16)).view(torch.bfloat16)
    ln = torch.nn.functional.layer_norm(kt.double(), (128,), torch.from_numpy(w).double(),
                                        torch.from_numpy(b).double(), 1e-5).to(torch.bfloat16).double().numpy()
    half = O.interleaved_to_half(ln[:, :64])
    z = (half[:, :32] + 1j * half[:, 32:]) * (cs[pos, :32].astype(np.float64) + 1j * cs[pos, 32:])
    ln[:, :64] = torch.from_numpy(np.concatenate([z.real, z.imag], -1)).to(torch.bfloat16).double().numpy()
    had = ln @ scipy.linalg.hadamard(128).T * 128 ** -0.5
    amax = np.maximum(np.abs(had).max(-1), 1e-4)
    ref_scale = np.exp2(np.ceil(np.log2(amax / 448.0))).astype(np.float32)
    assert (scales == ref_scale).mean() >= 0.98
    ok = scales == ref_scale
    ref_codes = O.fp8_e4m3fn_encode(had[ok] / ref_scale[ok, None])
    _assert_near_codes(codes[ok], ref_codes, 5e-3)
