"""The sparse prefill's keys assembled from the paged fp8 MLA cache and the
fresh rows (dsa_mla_prefill_kv) against the oracle: bit-exact (the nope
dequantisation is exact in bf16, the rope and fresh rows are copies)."""
import numpy as np
import pytest
import torch

import oracle as O
from nanoengine_amd import mla_utils, synth

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
