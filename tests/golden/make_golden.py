"""Writes tests/golden/config0_indexer.npz: the BASELINE config-0 indexer case.

Decode batch 4, next_n 1, 64 indexer heads x 128, contexts {1024, 2048, 3000,
4096} in a paged cache (page 64, block tables a seeded random permutation of
the 159 pages), q and k drawn N(0,1), rounded to bf16 and quantised to fp8
e4m3fn with one UE8M0 scale per 128-wide row, head weights
N(0,1) * 64^-0.5 * 128^-0.5 times the q scale. Expected outputs (logits, the
top-2048 positions and their physical slots) come from the numpy oracle.

Run from the repository root: ``python tests/golden/make_golden.py``.
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle as O  # noqa: E402


def bf16_round(x):
    return O.bf16_to_f32(O.f32_to_bf16(x.astype(np.float32)))


def main(seed: int = 0):
    rng = np.random.default_rng(seed)
    lens = np.array([1024, 2048, 3000, 4096], dtype=np.int32)
    B, H, D, P, K = 4, 64, 128, 64, 2048
    pages = (lens + P - 1) // P
    total = int(pages.sum())
    perm = rng.permutation(total).astype(np.int32)
    bt = np.zeros((B, pages.max()), dtype=np.int32)
    off = 0
    for b in range(B):
        bt[b, :pages[b]] = perm[off:off + pages[b]]
        off += pages[b]
    q = bf16_round(rng.standard_normal((B, 1, H, D)))
    q_fp8, q_scale = O.quantize_rows_ue8m0(q)
    w = (rng.standard_normal((B, H)) * H ** -0.5 * D ** -0.5).astype(np.float32)
    weights = (w * q_scale.reshape(B, H)).astype(np.float32)
    k = bf16_round(rng.standard_normal((total * P, D)))
    k_fp8, k_scale = O.quantize_rows_ue8m0(k)
    cache = O.pack_indexer_cache(k_fp8, k_scale, np.arange(total * P), total, P)
    ctx = lens.reshape(B, 1)
    max_ctx = bt.shape[1] * P
    logits = O.indexer_logits(q_fp8, cache, weights, ctx, bt, max_ctx)
    page_idx, raw = O.topk_transform(logits, lens, bt, P, K)
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "config0_indexer.npz")
    np.savez_compressed(out, q_fp8=q_fp8, weights=weights, cache=cache, context_lens=ctx,
                        block_tables=bt, logits=logits, topk_raw=raw, topk_page=page_idx)
    print(out, os.path.getsize(out))


if __name__ == "__main__":
    main()
