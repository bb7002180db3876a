"""BASELINE config 4 at its own shape, through the product route.

One 8192-token chunk attends causally over a 122880-token prefix that is
already in the paged fp8 caches: 131072 keys in all, top-2048, 64 indexer
heads x 128, 128 MLA heads x 576/512. The route is the one a chunked prefill
takes (lightning.py:1081-1250, deepseek_v2.py:1573-1650):

  compute_prefill_topk_paged (windows, paged->ragged key gather, fused logits
  + exact top-2048 with no logits buffer) -> flash_mla_sparse_fwd_paged (cached
  keys straight from the paged fp8 MLA cache, fresh keys as bf16 rows).

Eight query rows spread over the chunk are checked against the CPU oracle:
  * logits (ops.mqa_logits on the same gathered keys: the fused entry filters
    the very floats that kernel writes) within 1e-3 of max(|logit|, row RMS),
    or within the scaled fp8 MFMA's derived error bound where a head sum
    cancels (oracle ``indexer_logit_error_bound``);
  * the selected set equal to the oracle's exact top-2048 over the GPU's own
    logits, and differing from the top-2048 over the oracle's float64 logits
    only at ties within that tolerance of the k-th score (0 violations);
  * the assembled key rows those rows select (ops.mla_prefill_kv) bit-exact
    against the oracle's dequantisation of the fp8 cache;
  * MLA o within 2e-2 and LSE within 1e-3 of the oracle's sparse prefill.
Every row of the chunk must select exactly 2048 distinct in-window keys.
"""
import time

import numpy as np
import pytest
import torch

import oracle as O
from oracle import step_check as SC
from nanoengine_amd import flash_mla, ops, synth
from nanoengine_amd.indexer import compute_prefill_topk_paged, gather_indexer_cache

pytestmark = pytest.mark.gpu


def test_config4_chunk_sampled_rows_match_oracle(cuda):
    QN, KN, K, H, seed = 8192, 131072, 2048, 128, 0
    print(f"config4 QN={QN} KN={KN} K={K} H={H} seed={seed}", flush=True)
    t0 = time.time()
    inp = synth.make_indexer_inputs([KN], next_n=1, seed=seed, device=cuda)
    g = torch.Generator(device=cuda).manual_seed(seed + 3)
    q = torch.randn(QN, 64, 128, generator=g, device=cuda).to(torch.bfloat16)
    q_codes, q_scale = synth.ue8m0_quant_rows(q)
    w = (torch.randn(QN, 64, generator=g, device=cuda) * 64 ** -0.5 * 128 ** -0.5 * q_scale).float().contiguous()
    q8 = q_codes.view(torch.float8_e4m3fn)
    cu_q = torch.tensor([0, QN], dtype=torch.int32, device=cuda)
    cu_k = torch.tensor([0, KN], dtype=torch.int32, device=cuda)
    num_blocks = int(inp.block_tables.max().item()) + 1
    kv_cache = synth.make_mla_cache(num_blocks, seed=seed, device=cuda)
    fresh = torch.randn(QN, 576, generator=g, device=cuda).to(torch.bfloat16)
    q_mla = torch.randn(QN, H, 576, generator=g, device=cuda).to(torch.bfloat16)
    scale = 192 ** -0.5

    # the product route
    idx = compute_prefill_topk_paged(q8, w, cu_q, cu_k, inp.block_tables, inp.cache, page_size=64, index_topk=K)
    out, _, lse = flash_mla.flash_mla_sparse_fwd_paged(q_mla, kv_cache, inp.block_tables, cu_q, cu_k, fresh,
                                                       idx.unsqueeze(1), scale)
    torch.cuda.synchronize()
    print(f"gpu route done in {time.time() - t0:.1f} s", flush=True)

    # every row: 2048 distinct keys inside its causal window [0, KN - QN + 1 + i)
    ke = KN - QN + 1 + torch.arange(QN, device=cuda, dtype=torch.int32)
    assert bool((idx >= 0).all()) and bool((idx < ke[:, None]).all())
    assert bool((idx[:, 1:] > idx[:, :-1]).all()), "indices must be distinct (ascending)"

    rows = np.linspace(0, QN - 1, 8).round().astype(np.int64)
    rt = torch.as_tensor(rows, device=cuda)
    ks_r = np.zeros(len(rows), np.int32)
    ke_r = (KN - QN + 1 + rows).astype(np.int32)
    # the GPU logits of the sampled rows over the gathered keys
    keys, scales = gather_indexer_cache(inp.cache, inp.block_tables, cu_k, page_size=64, head_dim=128, total_k=KN)
    kvs = scales.view(torch.float32).reshape(-1)
    gl = torch.empty(len(rows), KN, dtype=torch.float32, device=cuda)
    ops.mqa_logits(q8[rt].contiguous(), keys.view(torch.float8_e4m3fn), kvs, w[rt].contiguous(),
                   torch.as_tensor(ks_r, device=cuda), torch.as_tensor(ke_r, device=cuda), gl, True)
    kv_bf16 = torch.empty(KN, 576, dtype=torch.bfloat16, device=cuda)
    ops.mla_prefill_kv(kv_cache, inp.block_tables, cu_q, cu_k, fresh, KN, kv_bf16)
    torch.cuda.synchronize()
    gpu_logits = gl.cpu().numpy()
    gpu_idx = idx[rt].cpu().numpy()

    # the oracle, on the host
    host_cache = inp.cache.cpu().numpy()
    bt = inp.block_tables.cpu().numpy()
    o_keys, o_scales = O.gather_indexer_cache(host_cache, bt, np.array([0, KN]))
    assert np.array_equal(o_keys, keys.cpu().numpy()) and np.array_equal(o_scales, kvs.cpu().numpy())
    exp_logits = O.mqa_logits(q_codes[rt].cpu().numpy(), o_keys, o_scales, w[rt].cpu().numpy(), ks_r, ke_r,
                              clean_logits=True)
    lg = SC.check_logits(gpu_logits, exp_logits, ke_r,
                         SC.ragged_logit_bound(q_codes[rt].cpu().numpy(), w[rt].cpu().numpy(), o_keys, o_scales))
    rel = lg["max_rel_err"]
    own = O.topk_transform_ragged(gpu_logits, ke_r - ks_r, ks_r, ks_r, K)
    topk_equal = bool(np.array_equal(own, gpu_idx))
    ties = SC.topk_tie_violations(gpu_idx, exp_logits, ke_r, K)
    kv_rows = O.assemble_prefill_kv(kv_cache.contiguous().reshape(-1, 656).cpu().numpy(), 64, bt,
                                    np.array([0, QN]), np.array([0, KN]), fresh.float().cpu().numpy())
    used = np.unique(gpu_idx[gpu_idx >= 0])
    kv_equal = bool(np.array_equal(kv_bf16[torch.as_tensor(used, device=cuda)].float().cpu().numpy(),
                                   kv_rows[used]))
    eo, _, el = O.sparse_mla_prefill(q_mla[rt].float().cpu().numpy(), kv_rows, gpu_idx, scale)
    o_err = float(np.abs(out[rt].float().cpu().numpy() - eo).max())
    lse_err = float(np.abs(lse[rt].cpu().numpy() - el).max())
    rep = {"rows": rows.tolist(), "logits_max_rel_err": rel, "logits_over_rtol": lg["over_rtol"],
           "logits_max_err_over_mfma_bound": lg["max_err_over_bound"], "topk_equal_on_gpu_logits": topk_equal,
           "topk_tie_violations": ties, "kv_rows_bit_exact": kv_equal, "o_max_abs_err": o_err,
           "lse_max_abs_err": lse_err, "fresh_keys_selected": int((gpu_idx >= KN - QN).sum()),
           "seconds": round(time.time() - t0, 1)}
    print(rep, flush=True)
    assert lg["ok"], rep
    assert topk_equal and ties == 0, rep
    assert kv_equal, rep
    assert o_err <= SC.O_ATOL and lse_err <= SC.LSE_ATOL, rep
