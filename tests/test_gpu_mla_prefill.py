"""Sparse MLA prefill on the GPU vs the CPU oracle.

Tolerances (north star): o within bf16 atol 2e-2, LSE within 1e-3 (absolute,
natural log); max_logits within 1e-3. The rows and the query are bf16, exact
in the bf16 MFMA inputs; the differences are the bf16 rounding of P and the
fp32 accumulation order.
"""
import numpy as np
import pytest
import torch

import oracle as O
from nanoengine_amd import flash_mla, ops, synth

pytestmark = pytest.mark.gpu


def _case(T, H, K, s_kv, seed, invalid_frac=0.0, oob_frac=0.0, device="cuda"):
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(T, H, 576, generator=g).to(torch.bfloat16)
    kv = torch.randn(s_kv, 576, generator=g).to(torch.bfloat16)
    idx = torch.stack([torch.randperm(s_kv, generator=g)[:K] for _ in range(T)]).to(torch.int32)
    if invalid_frac:
        idx[torch.rand(T, K, generator=g) < invalid_frac] = -1
    if oob_frac:
        idx[torch.rand(T, K, generator=g) < oob_frac] = s_kv + 5
    return q.to(device), kv.to(device), idx.to(device)


def _check(o, mx, lse, eo, emx, elv):
    o = o.float().cpu().numpy()
    mx, lse = mx.cpu().numpy(), lse.cpu().numpy()
    assert np.abs(o - eo).max() <= 2e-2
    fin = np.isfinite(elv)
    assert np.array_equal(np.isfinite(lse), fin) and np.array_equal(np.isfinite(mx), fin)
    assert np.abs(lse[fin] - elv[fin]).max(initial=0.0) <= 1e-3
    assert np.abs(mx[fin] - emx[fin]).max(initial=0.0) <= 1e-3


@pytest.mark.parametrize("T,H,K,s_kv", [(3, 128, 2048, 5000), (5, 64, 512, 700), (4, 16, 96, 200),
                                        (2, 128, 128, 130)])
def test_matches_oracle(cuda, T, H, K, s_kv):
    print(f"mla prefill T={T} H={H} K={K} s_kv={s_kv}", flush=True)
    q, kv, idx = _case(T, H, K, s_kv, seed=T * 100 + K)
    scale = 192 ** -0.5
    o, mx, lse = ops.sparse_mla_prefill(q, kv, idx, scale)
    torch.cuda.synchronize()
    eo, emx, elv = O.sparse_mla_prefill(q.float().cpu().numpy(), kv.float().cpu().numpy(), idx.cpu().numpy(), scale)
    _check(o, mx, lse, eo, emx, elv)


def test_invalid_out_of_range_and_empty_rows(cuda):
    print("mla prefill invalid rows", flush=True)
    q, kv, idx = _case(4, 128, 256, 900, seed=4, invalid_frac=0.3, oob_frac=0.1)
    idx[1] = -1                  # no valid index: o = 0, lse = max_logits = -inf
    idx[2, 32:] = -1             # only the first block valid
    idx[3, :224] = 900           # only the last block valid (the rest is past s_kv)
    scale = 0.07
    o, mx, lse = ops.sparse_mla_prefill(q, kv, idx, scale)
    torch.cuda.synchronize()
    eo, emx, elv = O.sparse_mla_prefill(q.float().cpu().numpy(), kv.float().cpu().numpy(), idx.cpu().numpy(), scale)
    _check(o, mx, lse, eo, emx, elv)
    assert torch.all(o[1] == 0) and torch.all(torch.isneginf(lse[1])) and torch.all(torch.isneginf(mx[1]))


def test_flash_mla_sparse_fwd_signature_and_strided_kv(cuda):
    """flash_mla_sparse_fwd(q, kv [s_kv, 1, 576], indices [s_q, 1, topk], scale, d_v)
    as called at deepseek_v2.py:1644-1650; kv given as a strided view."""
    print("flash_mla_sparse_fwd", flush=True)
    q, kv, idx = _case(3, 128, 512, 1000, seed=9)
    big = torch.zeros(1000, 1, 640, dtype=torch.bfloat16, device=cuda)
    big[:, 0, :576] = kv
    kv_view = big[:, :, :576]
    out, mx, lse = flash_mla.flash_mla_sparse_fwd(q, kv_view, idx.unsqueeze(1), 192 ** -0.5, d_v=512)
    torch.cuda.synchronize()
    assert out.shape == (3, 128, 512) and mx.shape == (3, 128) and lse.shape == (3, 128)
    eo, emx, elv = O.sparse_mla_prefill(q.float().cpu().numpy(), kv.float().cpu().numpy(), idx.cpu().numpy(),
                                         192 ** -0.5)
    _check(out, mx, lse, eo, emx, elv)


def test_prefill_on_dequantised_rows_equals_decode_on_fp8_rows(cuda):
    """The same attention two ways: the prefill kernel over bf16 rows that are the
    exact dequantisation of fp8 cache rows, and the decode kernel over those fp8
    rows. Both must match each other to the decode tolerance."""
    print("mla prefill vs decode", flush=True)
    T, H, K = 4, 128, 1024
    kv8 = synth.make_mla_cache(40, seed=3, device=cuda)                  # [40, 64, 1, 656] view
    rows = kv8.reshape(-1, 656) if kv8.is_contiguous() else kv8.contiguous().reshape(-1, 656)
    deq = torch.from_numpy(O.dequant_mla_rows(rows.cpu().numpy())).to(torch.bfloat16).to(cuda)
    q = synth.make_mla_query(T, H, seed=3, device=cuda)
    g = torch.Generator(device="cpu").manual_seed(3)
    idx = torch.stack([torch.randperm(40 * 64, generator=g)[:K] for _ in range(T)]).to(torch.int32).to(cuda)
    o_p, _, l_p = ops.sparse_mla_prefill(q, deq, idx, 192 ** -0.5)
    o_d, l_d = ops.sparse_mla_decode(q, kv8, idx, 192 ** -0.5)
    torch.cuda.synchronize()
    assert (o_p.float() - o_d.float()).abs().max().item() <= 2e-2
    assert (l_p - l_d).abs().max().item() <= 1e-3
