"""topk_indices_to_physical on the GPU: the reference's known-answer vectors
(tests/test_sparse_decode.py:98-161) and random cases vs the oracle."""
import numpy as np
import pytest
import torch

import oracle as O
from nanoengine_amd.mla_utils import topk_indices_to_physical

pytestmark = pytest.mark.gpu


def test_known_answers(cuda):
    bt = torch.tensor([[5, 10, 2, 8]], dtype=torch.int32, device=cuda)
    idx = torch.tensor([[0, 65, 192, 130]], dtype=torch.int32, device=cuda)
    assert topk_indices_to_physical(idx, bt, 64).cpu().tolist() == [[320, 641, 512, 130]]
    bt = torch.tensor([[3, 7]], dtype=torch.int32, device=cuda)
    idx = torch.tensor([[10, -1, 70, -1]], dtype=torch.int32, device=cuda)
    assert topk_indices_to_physical(idx, bt, 64).cpu().tolist() == [[3 * 64 + 10, -1, 7 * 64 + 6, -1]]
    bt = torch.tensor([[1, 2], [5, 6]], dtype=torch.int32, device=cuda)
    idx = torch.tensor([[0, 64], [63, 127]], dtype=torch.int32, device=cuda)
    assert topk_indices_to_physical(idx, bt, 64).cpu().tolist() == [[64, 128], [383, 447]]


@pytest.mark.parametrize("rows_per_table", [1, 2])
def test_random_vs_oracle(cuda, rows_per_table):
    rng = np.random.default_rng(rows_per_table)
    B, M, K, bs = 8, 1024, 2048, 64
    bt = rng.integers(0, 1 << 20, (B, M)).astype(np.int32)
    idx = rng.integers(-1, M * bs, (B * rows_per_table, K)).astype(np.int32)
    got = topk_indices_to_physical(torch.from_numpy(idx).to(cuda), torch.from_numpy(bt).to(cuda), bs)
    torch.cuda.synchronize()
    exp = O.topk_indices_to_physical(idx, np.repeat(bt, rows_per_table, axis=0), bs)
    assert np.array_equal(got.cpu().numpy(), exp)
