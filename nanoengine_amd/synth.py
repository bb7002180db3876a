"""Seeded synthetic DSA decode inputs, generated on the device with torch.

The shapes and distributions are the benchmark configurations: q and k drawn
N(0,1) in bf16 and quantised to fp8 e4m3fn with one UE8M0 scale per 128-wide
row (the rule of dlengine/runtime/layers/backends/dsa/indexer/lightning.py:78-101),
head weights N(0,1) * 64^-0.5 * 128^-0.5 with the q scale folded in
(lightning.py:1252-1273), MLA rows quantised into the 656-byte layout
(dlengine/runtime/kernel/triton/hopper/fp8_utils.py:32-108), and block tables
that are a random permutation of the page pool. All of it is input
preparation; none of it is on the measured path.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

PAGE = 64
IDX_HEADS = 64
IDX_DIM = 128
IDX_PAGE_BYTES = PAGE * (IDX_DIM + 4)
MLA_ROW = 656
MLA_BLOCK_ROWS = PAGE + 1          # one padding row per block (context/cache/mla.py:164-182)


def ue8m0_quant_rows(x: torch.Tensor, min_amax: float = 1e-4):
    """Per-row fp8 quantisation with a power-of-two scale: returns
    (fp8 codes as uint8 [..., D], scale f32 [...])."""
    amax = x.float().abs().amax(dim=-1).clamp(min=min_amax)
    sf = torch.exp2(torch.ceil(torch.log2(amax / 448.0)))
    codes = (x.float() * (1.0 / sf.unsqueeze(-1))).to(torch.float8_e4m3fn).view(torch.uint8)
    return codes, sf


def quantize_mla_rows(kv: torch.Tensor) -> torch.Tensor:
    """[N, 576] bf16 -> [N, 656] uint8 rows: 512 fp8 (4 tiles of 128, each with a
    UE8M0 f32 scale), 4 f32 scales, 64 bf16 rope."""
    n = kv.shape[0]
    nope = kv[:, :512].float().view(n, 4, 128)
    amax = nope.abs().amax(dim=-1)
    scales = torch.pow(2, torch.clamp_min(amax / 448.0, 1e-12).log2().ceil())
    codes = (nope / scales.unsqueeze(-1)).to(torch.float8_e4m3fn).view(torch.uint8).view(n, 512)
    out = torch.empty(n, MLA_ROW, dtype=torch.uint8, device=kv.device)
    out[:, :512] = codes
    out[:, 512:528] = scales.contiguous().view(torch.uint8).view(n, 16)
    out[:, 528:] = kv[:, 512:].contiguous().view(torch.uint8).view(n, 128)
    return out


@dataclass
class IndexerInputs:
    q_fp8: torch.Tensor          # [B*n, 64, 128] uint8 codes
    weights: torch.Tensor        # [B*n, 64] f32 (q scale folded in)
    cache: torch.Tensor          # [num_pages, 8448] uint8
    context_lens: torch.Tensor   # [B] int32, length after the last query token
    block_tables: torch.Tensor   # [B, M] int32
    next_n: int


def make_block_tables(lens: list[int], gen: torch.Generator, device, extra_pages: int = 0):
    """Random permutation of exactly the pages the sequences need."""
    pages = [(L + PAGE - 1) // PAGE for L in lens]
    total = sum(pages) + extra_pages
    perm = torch.randperm(total, generator=gen, device="cpu").to(torch.int32)
    M = max(pages)
    bt = torch.zeros(len(lens), M, dtype=torch.int32)
    off = 0
    for b, p in enumerate(pages):
        bt[b, :p] = perm[off:off + p]
        off += p
    return bt.to(device), total


def make_indexer_inputs(lens: list[int], next_n: int = 1, seed: int = 0, device="cuda",
                        chunk_tokens: int = 1 << 20) -> IndexerInputs:
    gen = torch.Generator(device="cpu").manual_seed(seed)
    B = len(lens)
    bt, num_pages = make_block_tables(lens, gen, device)
    dgen = torch.Generator(device=device).manual_seed(seed + 1)
    q = torch.randn(B * next_n, IDX_HEADS, IDX_DIM, generator=dgen, device=device).to(torch.bfloat16)
    q_codes, q_scale = ue8m0_quant_rows(q)
    w = torch.randn(B * next_n, IDX_HEADS, generator=dgen, device=device) * (IDX_HEADS ** -0.5) * (IDX_DIM ** -0.5)
    weights = (w * q_scale).float().contiguous()
    cache = torch.zeros(num_pages, IDX_PAGE_BYTES, dtype=torch.uint8, device=device)
    # keys for every page slot, written page by page in the split layout
    flat = cache.view(num_pages, PAGE * IDX_DIM + PAGE * 4)
    done = 0
    while done < num_pages:
        n_p = min(num_pages - done, max(1, chunk_tokens // PAGE))
        k = torch.randn(n_p * PAGE, IDX_DIM, generator=dgen, device=device).to(torch.bfloat16)
        codes, sf = ue8m0_quant_rows(k)
        flat[done:done + n_p, :PAGE * IDX_DIM] = codes.view(n_p, PAGE * IDX_DIM)
        flat[done:done + n_p, PAGE * IDX_DIM:] = sf.view(torch.uint8).view(n_p, PAGE * 4)
        done += n_p
    ctx = torch.tensor(lens, dtype=torch.int32, device=device)
    return IndexerInputs(q_codes.contiguous(), weights, cache, ctx, bt, next_n)


def make_mla_cache(num_blocks: int, seed: int = 0, device="cuda", chunk_blocks: int = 8192) -> torch.Tensor:
    """Padded fp8 MLA cache [num_blocks, 65, 1, 656] (uint8) filled from N(0,1)
    sources; returns the [num_blocks, 64, 1, 656] view the kernels consume."""
    buf = torch.zeros(num_blocks, MLA_BLOCK_ROWS, 1, MLA_ROW, dtype=torch.uint8, device=device)
    dgen = torch.Generator(device=device).manual_seed(seed + 7)
    done = 0
    while done < num_blocks:
        nb = min(num_blocks - done, chunk_blocks)
        kv = torch.randn(nb * PAGE, 576, generator=dgen, device=device).to(torch.bfloat16)
        buf[done:done + nb, :PAGE, 0] = quantize_mla_rows(kv).view(nb, PAGE, MLA_ROW)
        done += nb
    return buf[:, :PAGE]


def make_mla_query(tokens: int, heads: int = 128, seed: int = 0, device="cuda") -> torch.Tensor:
    dgen = torch.Generator(device=device).manual_seed(seed + 11)
    return torch.randn(tokens, heads, 576, generator=dgen, device=device).to(torch.bfloat16)


def random_topk_positions(lens: list[int], k: int, seed: int = 0, device="cuda") -> torch.Tensor:
    """[B, k] int32 distinct logical positions per row (ascending), -1 padded
    where the context is shorter than k."""
    gen = torch.Generator(device="cpu").manual_seed(seed + 13)
    out = torch.full((len(lens), k), -1, dtype=torch.int32)
    for b, L in enumerate(lens):
        n = min(L, k)
        sel = torch.randperm(L, generator=gen)[:n].sort().values
        out[b, :n] = sel.to(torch.int32)
    return out.to(device)
