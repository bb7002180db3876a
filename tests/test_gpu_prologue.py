"""Indexer prologue on the GPU vs the oracle, bit for bit: the query transform
(RoPE -> Hadamard -> UE8M0 quant -> gate scaling) and the key transform + cache
store (LayerNorm -> RoPE -> Hadamard -> quant -> split page)."""
import numpy as np
import pytest
import torch

import oracle as O
from nanoengine_amd import deepseek_v4, indexer_transform, ops

pytestmark = pytest.mark.gpu


def _bf16(rng, shape, scale=1.0, shift=0.0):
    x = (rng.standard_normal(shape) * scale + shift).astype(np.float32)
    return torch.from_numpy(x).to(torch.bfloat16)


def _u16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _q_case(cuda, T, H, seed, pos_dtype=torch.int64, interleaved=True, gate_pad=0, max_pos=1024):
    rng = np.random.default_rng(seed)
    q = _bf16(rng, (T, H, 128))
    if T > 2:
        q[1] *= 1e-6          # amax below the 1e-4 floor
        q[2, 0] = 0           # an all-zero row
    gate_full = _bf16(rng, (T, H + gate_pad))
    gate = gate_full[:, :H]
    cs = O.rope_cos_sin_cache(max_pos)
    pos = torch.from_numpy(rng.integers(0, max_pos, T)).to(pos_dtype)
    if T > 0:
        pos[0] = 0
    ws = 64 ** -0.5 * 128 ** -0.5
    got_q, got_w = deepseek_v4.indexer_q_rope_hadamard_quant(
        q.to(cuda), gate_full.to(cuda)[:, :H], ws, torch.from_numpy(cs).to(cuda)[:, None, :], pos.to(cuda),
        rope_interleaved=interleaved)
    torch.cuda.synchronize()
    exp_q, exp_w = O.indexer_q_prologue(_u16(q), _u16(gate), ws, cs, pos.numpy(), interleaved)
    return got_q.view(torch.uint8).cpu().numpy(), got_w.cpu().numpy()[..., 0], exp_q, exp_w


@pytest.mark.parametrize("T,H", [(1, 64), (5, 8), (128, 64), (37, 16)])
@pytest.mark.parametrize("interleaved", [True, False])
def test_q_prologue_bit_exact(cuda, T, H, interleaved):
    print(f"q prologue T={T} H={H} interleaved={interleaved}", flush=True)
    gq, gw, eq, ew = _q_case(cuda, T, H, seed=T * 7 + H, interleaved=interleaved)
    assert np.array_equal(gq, eq), f"{(gq != eq).mean():.3e} of codes differ"
    assert np.array_equal(gw.view(np.uint32), ew.view(np.uint32))


def test_q_prologue_int32_positions_and_strided_gate(cuda):
    gq, gw, eq, ew = _q_case(cuda, 9, 64, seed=3, pos_dtype=torch.int32, gate_pad=5)
    assert np.array_equal(gq, eq)
    assert np.array_equal(gw.view(np.uint32), ew.view(np.uint32))


def test_q_prologue_large_batch_properties(cuda):
    """Decode-size batch (B=128, next_n=2, 64 heads): exact against the oracle."""
    gq, gw, eq, ew = _q_case(cuda, 256, 64, seed=99, max_pos=131072)
    assert np.array_equal(gq, eq)
    assert np.array_equal(gw.view(np.uint32), ew.view(np.uint32))


def test_q_prologue_empty_and_errors(cuda):
    q = torch.zeros(0, 64, 128, dtype=torch.bfloat16, device=cuda)
    g = torch.zeros(0, 64, dtype=torch.bfloat16, device=cuda)
    cs = torch.zeros(16, 64, dtype=torch.float32, device=cuda)
    q8, w = deepseek_v4.indexer_q_rope_hadamard_quant(q, g, 1.0, cs, torch.zeros(0, dtype=torch.int64, device=cuda))
    assert q8.shape == (0, 64, 128) and w.shape == (0, 64, 1)
    with pytest.raises(ValueError):
        deepseek_v4.indexer_q_rope_hadamard_quant(torch.zeros(2, 4, 64, dtype=torch.bfloat16, device=cuda),
                                                  g, 1.0, cs, torch.zeros(2, dtype=torch.int64, device=cuda))
    with pytest.raises(ValueError):
        deepseek_v4.indexer_q_rope_hadamard_quant(torch.zeros(2, 4, 128, dtype=torch.bfloat16, device=cuda),
                                                  torch.zeros(2, 3, dtype=torch.bfloat16, device=cuda), 1.0, cs,
                                                  torch.zeros(2, dtype=torch.int64, device=cuda))


def _k_case(cuda, T, seed, slot_dtype=torch.int32, row_pad=0, pages=4, neg=()):
    rng = np.random.default_rng(seed)
    key_full = _bf16(rng, (T, 128 + row_pad), scale=2.0, shift=0.3)
    if T > 3:
        key_full[3, :128] = 1.5   # constant row: variance 0
    key = key_full[:, :128]
    w = rng.standard_normal(128).astype(np.float32)
    b = rng.standard_normal(128).astype(np.float32) * 0.1
    cs = O.rope_cos_sin_cache(4096)
    pos = rng.integers(0, 4096, T)
    slots = rng.permutation(pages * 64)[:T].astype(np.int64)
    for i in neg:
        slots[i] = -1
    cache = torch.zeros(pages, 64 * 132, dtype=torch.uint8, device=cuda)
    indexer_transform.indexer_k_transform_store_fp8(
        key_full.to(cuda)[:, :128], torch.from_numpy(w).to(cuda), torch.from_numpy(b).to(cuda), 1e-6,
        torch.from_numpy(pos).to(cuda), torch.from_numpy(cs).to(cuda), cache,
        torch.from_numpy(slots).to(slot_dtype).to(cuda), 64)
    torch.cuda.synchronize()
    codes, sf = O.indexer_k_transform(_u16(key), w, b, 1e-6, cs, pos)
    keep = slots >= 0
    exp = O.pack_indexer_cache(codes[keep], sf[keep], slots[keep], pages)
    return cache.cpu().numpy(), exp


@pytest.mark.parametrize("T", [1, 17, 200])
def test_k_transform_store_bit_exact(cuda, T):
    print(f"k transform T={T}", flush=True)
    got, exp = _k_case(cuda, T, seed=T)
    assert np.array_equal(got, exp), f"{(got != exp).mean():.3e} of bytes differ"


def test_k_transform_store_int64_slots_strided_rows_and_skips(cuda):
    got, exp = _k_case(cuda, 40, seed=5, slot_dtype=torch.int64, row_pad=64, neg=(0, 7, 39))
    assert np.array_equal(got, exp)


def test_k_transform_rejects_bad_key(cuda):
    cache = torch.zeros(1, 64 * 132, dtype=torch.uint8, device=cuda)
    with pytest.raises(ValueError):
        indexer_transform.indexer_k_transform_store_fp8(
            torch.zeros(2, 64, dtype=torch.bfloat16, device=cuda), torch.ones(128, device=cuda),
            torch.zeros(128, device=cuda), 1e-6, torch.zeros(2, dtype=torch.int64, device=cuda),
            torch.zeros(8, 64, device=cuda), cache, torch.zeros(2, dtype=torch.int32, device=cuda), 64)
