"""dsa_topk_transform_noalloc (the entry point that allocates nothing) against
dsa_topk_transform with a caller workspace, through the C ABI: two calls in a
row, the second smaller, on rows longer than 64K positions so that the
scratch-backed list path runs; then the row-limit error."""
import ctypes

import numpy as np
import pytest
import torch

from nanoengine_amd import _lib, ops

pytestmark = pytest.mark.gpu


def _noalloc(scores, lens, pt, out_page, out_raw, page_size, top_k):
    return _lib.load().dsa_topk_transform_noalloc(
        scores.data_ptr(), scores.stride(0), lens.data_ptr(), pt.data_ptr(), pt.stride(0), out_page.data_ptr(),
        out_raw.data_ptr(), scores.shape[0], scores.shape[1], page_size, top_k,
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


@pytest.mark.parametrize("first,second", [((8, 70000, 2048), (3, 66000, 512))])
def test_noalloc_matches_workspace_entry_point(cuda, first, second):
    for case, (B, W, K) in enumerate((first, second)):
        print(f"noalloc case {case}: B={B} W={W} K={K}", flush=True)
        g = torch.Generator(device="cpu").manual_seed(100 + case)
        scores = torch.randn(B, W, generator=g).to(cuda)
        lens = torch.tensor([W - 7 * b for b in range(B)], dtype=torch.int32).to(cuda)
        pages = (W + 63) // 64
        pt = torch.stack([torch.randperm(pages * 2, generator=g)[:pages] for _ in range(B)]).to(torch.int32).to(cuda)
        ref_page = torch.empty(B, K, dtype=torch.int32, device=cuda)
        ref_raw = torch.empty_like(ref_page)
        ws = torch.empty(ops.topk_workspace_bytes(B), dtype=torch.uint8, device=cuda)
        ops.topk_transform(scores, lens, pt, ref_page, 64, K, ref_raw, workspace=ws)
        got_page = torch.full_like(ref_page, -7)
        got_raw = torch.full_like(ref_page, -7)
        assert _noalloc(scores, lens, pt, got_page, got_raw, 64, K) == 0, _lib.load().dsa_last_error()
        torch.cuda.synchronize()
        assert torch.equal(got_page, ref_page)
        assert torch.equal(got_raw, ref_raw)
        assert int((got_raw[0] >= 0).sum()) == K


def test_noalloc_rejects_rows_beyond_scratch(cuda):
    B, W = 257, 70000
    scores = torch.zeros(B, W, device=cuda)
    lens = torch.full((B,), W, dtype=torch.int32, device=cuda)
    pt = torch.zeros(B, (W + 63) // 64, dtype=torch.int32, device=cuda)
    out = torch.empty(B, 2048, dtype=torch.int32, device=cuda)
    rc = _noalloc(scores, lens, pt, out, out, 64, 2048)
    assert rc == 2
    assert b"scratch maximum of 256 rows" in _lib.load().dsa_last_error()
