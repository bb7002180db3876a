"""The sparse prefill's keys assembled from the paged fp8 MLA cache and the
fresh rows (dsa_mla_prefill_kv) against the oracle: bit-exact (the nope
dequantisation is exact in bf16, the rope and fresh rows are copies)."""
import numpy as np
import pytest
import torch

import oracle as O
from nanoengine_amd import mla_utils, ops, synth

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("cu_dtype", [torch.int32, torch.int64])
def test_assemble_prefill_kv_matches_oracle(cuda, cu_dtype):
    print(f"prefill kv assemble {cu_dtype}", flush=True)
    rng = np.random.default_rng(5)
    q_lens = np.array([40, 0, 129, 64, 1])
    k_lens = q_lens + np.array([300, 70, 0, 1000, 63])
    pages = (k_lens + 63) // 64
    num_blocks = int(pages.sum()) + 3
    perm = rng.permutation(num_blocks)
    bt = np.zeros((len(q_lens), pages.max()), np.int32)
    at = 0
    for b, p in enumerate(pages):
        bt[b, :p] = perm[at:at + p]
        at += p
    kv = synth.make_mla_cache(num_blocks, seed=9, device=cuda)          # [blocks, 64, 1, 656], stride 65 rows
    cu_q = np.concatenate([[0], np.cumsum(q_lens)])
    cu_k = np.concatenate([[0], np.cumsum(k_lens)])
    fresh = torch.randn(int(cu_q[-1]), 576, device=cuda).to(torch.bfloat16)
    t = lambda a: torch.from_numpy(a).to(cuda, cu_dtype)                 # noqa: E731
    out = mla_utils.assemble_prefill_kv(kv, torch.from_numpy(bt).to(cuda), t(cu_q), t(cu_k), fresh.unsqueeze(1))
    torch.cuda.synchronize()
    rows = kv.contiguous().reshape(-1, 656).cpu().numpy()
    exp = O.assemble_prefill_kv(rows, 64, bt, cu_q, cu_k, fresh.float().cpu().numpy())
    assert out.shape == (int(cu_k[-1]), 1, 576)
    assert np.array_equal(out[:, 0].float().cpu().numpy(), exp)


def _paged_case(cuda, seed=7, H=128, topk=256):
    rng = np.random.default_rng(seed)
    q_lens = np.array([40, 0, 129, 64, 3])
    k_lens = q_lens + np.array([300, 70, 0, 1000, 4000])
    pages = (k_lens + 63) // 64
    num_blocks = int(pages.sum()) + 5
    perm = rng.permutation(num_blocks)
    bt = np.zeros((len(q_lens), pages.max()), np.int32)
    at = 0
    for b, p in enumerate(pages):
        bt[b, :p] = perm[at:at + p]
        at += p
    cu_q = np.concatenate([[0], np.cumsum(q_lens)])
    cu_k = np.concatenate([[0], np.cumsum(k_lens)])
    T, total_k = int(cu_q[-1]), int(cu_k[-1])
    idx = np.full((T, topk), -1, np.int32)
    for b in range(len(q_lens)):
        cached = k_lens[b] - q_lens[b]
        for j in range(q_lens[b]):
            t = cu_q[b] + j
            win = cached + j + 1
            n = min(topk, win)
            sel = rng.choice(win, size=n, replace=False) + cu_k[b]
            idx[t, :n] = sel
            if n < topk:
                idx[t, n] = total_k + 5          # out of range: skipped
    idx[cu_q[3] + 1] = -1                        # a token with no valid index
    kv = synth.make_mla_cache(num_blocks, seed=seed, device=cuda)
    g = torch.Generator(device=cuda).manual_seed(seed)
    fresh = torch.randn(T, 576, device=cuda, generator=g).to(torch.bfloat16)
    q = synth.make_mla_query(T, H, seed=seed, device=cuda)
    t32 = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda, torch.int32)   # noqa: E731
    return q, kv, t32(bt), t32(cu_q), t32(cu_k), fresh, t32(idx), total_k, (bt, cu_q, cu_k, idx)


def test_paged_prefill_matches_assembled_rows(cuda):
    """The paged sparse prefill (one decode-kernel pass per token: its cached
    keys from the fp8 cache, then its fresh keys as bf16 rows in 32-row blocks)
    against the assembled bf16 keys through the bf16 prefill kernel and against
    the oracle. The sequences include one with no cached prefix (up to 129
    fresh keys per token: five fresh blocks, the last partly invalid), a token
    with no valid index and indices past the key count. A NaN row here has
    meant an invalid fresh key's P scaled to -inf (0 * -inf)."""
    print("paged sparse prefill", flush=True)
    q, kv, bt, cu_q, cu_k, fresh, idx, total_k, host = _paged_case(cuda)
    scale = 192 ** -0.5
    o, mx, lse = ops.sparse_mla_prefill_paged(q, kv, bt, cu_q, cu_k, fresh, idx, scale, total_k)
    asm = mla_utils.assemble_prefill_kv(kv, bt, cu_q, cu_k, fresh.unsqueeze(1), total_k)[:, 0]
    eo, emx, else_ = ops.sparse_mla_prefill(q, asm, idx, scale)
    torch.cuda.synchronize()
    # two GPU results, each rounded to bf16 on its own, with different summation
    # orders: a bf16 ulp of the value on top of atol
    assert torch.all((o.float() - eo.float()).abs() <= 2e-2 + eo.float().abs() * 2.0 ** -7)
    fin = torch.isfinite(else_)
    assert torch.equal(torch.isfinite(lse), fin) and torch.equal(torch.isfinite(mx), torch.isfinite(emx))
    assert (lse[fin] - else_[fin]).abs().max().item() <= 1e-3
    assert (mx[fin] - emx[fin]).abs().max().item() <= 1e-3
    bt_h, cu_q_h, cu_k_h, idx_h = host
    rows = kv.contiguous().reshape(-1, 656).cpu().numpy()
    kv_or = O.assemble_prefill_kv(rows, 64, bt_h, cu_q_h, cu_k_h, fresh.float().cpu().numpy())
    sample = np.array([0, 39, 40, 100, 168, 200, int(cu_q_h[3]) + 1, int(cu_q_h[-1]) - 1])
    oo, omx, olse = O.sparse_mla_prefill(q[sample].float().cpu().numpy(), kv_or, idx_h[sample], scale)
    err = np.abs(o[sample].float().cpu().numpy() - oo)
    print(f"paged prefill vs oracle: max |o err| {err.max():.4f} at |o| {np.abs(oo).flat[err.argmax()]:.3f}", flush=True)
    assert err.max() <= 2e-2
    ofin = np.isfinite(olse)
    assert np.array_equal(np.isfinite(lse[sample].cpu().numpy()), ofin)
    assert np.abs(lse[sample].cpu().numpy()[ofin] - olse[ofin]).max() <= 1e-3
    assert np.abs(mx[sample].cpu().numpy()[ofin] - omx[ofin]).max() <= 1e-3
    assert torch.all(o[int(cu_q_h[3]) + 1] == 0)


def test_flash_mla_sparse_fwd_paged_adapter(cuda):
    """The reference-shaped entry (indices [s_q, 1, topk], key_states
    [total_q, 1, 576], int64 cu_seqlens) gives the same result as the op."""
    from nanoengine_amd import flash_mla
    print("flash_mla_sparse_fwd_paged adapter", flush=True)
    q, kv, bt, cu_q, cu_k, fresh, idx, total_k, _ = _paged_case(cuda, seed=11)
    scale = 192 ** -0.5
    o, mx, lse = ops.sparse_mla_prefill_paged(q, kv, bt, cu_q, cu_k, fresh, idx, scale, total_k)
    o2, mx2, lse2 = flash_mla.flash_mla_sparse_fwd_paged(q, kv, bt, cu_q.to(torch.int64), cu_k.to(torch.int64),
                                                         fresh.unsqueeze(1), idx.unsqueeze(1).to(torch.int64),
                                                         scale)
    torch.cuda.synchronize()
    assert torch.equal(o, o2)
    assert torch.equal(torch.nan_to_num(lse, neginf=-1e30), torch.nan_to_num(lse2, neginf=-1e30))
    assert torch.equal(torch.nan_to_num(mx, neginf=-1e30), torch.nan_to_num(mx2, neginf=-1e30))
    with pytest.raises(ValueError):
        flash_mla.flash_mla_sparse_fwd_paged(q, kv, bt, cu_q, cu_k, fresh, idx, scale)   # indices not [s_q, 1, topk]


def test_bad_block_table_entries_are_skipped(cuda):
    """Block-table entries that point outside the cache (-1, past the block
    count) or columns past the table's width: the key assembly writes those
    cached rows as zeros, and the paged sparse prefill skips them like an
    index of -1. The table is passed as a narrowed view (row stride 63,
    width 40), so sequence 4's cached rows from 2560 on lie past its width."""
    print("prefill bad block-table entries", flush=True)
    q, kv, bt, cu_q, cu_k, fresh, idx, total_k, host = _paged_case(cuda, seed=13)
    bt_h, cu_q_h, cu_k_h, idx_h = host
    nblk = kv.shape[0]
    bad_bt = bt_h.copy()
    bad_bt[3, 2] = -1
    bad_bt[3, 5] = nblk + 7
    W = 40
    bt_view = torch.from_numpy(bad_bt).to(cuda)[:, :W]
    assert bt_view.stride(0) == bt_h.shape[1] and bt_view.shape[1] == W
    # which ragged key rows are unusable
    bad_row = np.zeros(total_k, bool)
    for b in range(len(cu_q_h) - 1):
        cached = (cu_k_h[b + 1] - cu_k_h[b]) - (cu_q_h[b + 1] - cu_q_h[b])
        for i in range(cached):
            col = i // 64
            bad_row[cu_k_h[b] + i] = col >= W or not (0 <= bad_bt[b, col] < nblk)
    assert bad_row.sum() > 1000
    rows = kv.contiguous().reshape(-1, 656).cpu().numpy()
    exp = O.assemble_prefill_kv(rows, 64, bt_h, cu_q_h, cu_k_h, fresh.float().cpu().numpy())
    exp[bad_row] = 0.0
    out = torch.empty(total_k, 576, dtype=torch.bfloat16, device=cuda)
    ops.mla_prefill_kv(kv, bt_view, cu_q, cu_k, fresh, total_k, out)
    scale = 192 ** -0.5
    o, mx, lse = ops.sparse_mla_prefill_paged(q, kv, bt_view, cu_q, cu_k, fresh, idx, scale, total_k)
    torch.cuda.synchronize()
    assert np.array_equal(out.float().cpu().numpy(), exp)
    idx_skip = np.where((idx_h >= 0) & (idx_h < total_k) & bad_row[np.clip(idx_h, 0, total_k - 1)], -1, idx_h)
    sample = np.array([int(cu_q_h[3]), int(cu_q_h[3]) + 30, int(cu_q_h[4]), int(cu_q_h[4]) + 2, 0, 50])
    oo, omx, olse = O.sparse_mla_prefill(q[sample].float().cpu().numpy(), exp, idx_skip[sample], scale)
    assert np.abs(o[sample].float().cpu().numpy() - oo).max() <= 2e-2
    assert np.abs(lse[sample].cpu().numpy() - olse).max() <= 1e-3
