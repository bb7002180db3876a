"""CPU checks of the C ABI: the library builds and loads, exports exactly the
symbols include/dsa_amd.h declares, and rejects bad arguments with the
documented status codes before touching a device."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dsa_amd.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"DSA_API\s+[\w\s\*]+?\b(dsa_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from nanoengine_amd import _lib
    if not _lib.LIB_PATH.exists():
        from nanoengine_amd import build
        build.build()
    return _lib.load()


def test_header_declares_the_reference_replacements():
    names = _declared()
    for n in ["dsa_indexer_logits", "dsa_indexer_schedule", "dsa_num_cus", "dsa_topk_transform",
              "dsa_topk_transform_ragged", "dsa_topk_to_physical", "dsa_sparse_mla_decode"]:
        assert n in names


def test_every_declared_symbol_is_exported_and_bound(lib):
    from nanoengine_amd import _lib
    for name in _declared():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(_declared())


def test_version_and_error_string(lib):
    assert lib.dsa_version() >= 100
    assert lib.dsa_topk_max_len() == 1 << 18


def test_argument_errors_return_status_without_a_device(lib):
    from nanoengine_amd import _lib
    P = None
    # top_k outside {512, 2048} -> invalid argument (1)
    rc = lib.dsa_topk_transform(P, 0, P, P, 0, P, P, 1, 10, 64, 1000, P, 0, P)
    assert rc == 1 and b"512 or 2048" in lib.dsa_last_error()
    # page size not a power of two
    assert lib.dsa_topk_transform(P, 0, P, P, 0, P, P, 1, 10, 48, 512, P, 0, P) == 1
    assert b"power of 2" in lib.dsa_last_error()
    # ragged top_k must be 2048
    assert lib.dsa_topk_transform_ragged(P, 0, P, P, P, P, 1, 10, 512, P, 0, P) == 1
    # rows longer than the bitmap -> unsupported (2)
    assert lib.dsa_topk_transform(P, 0, P, P, 0, P, P, 1, (1 << 18) + 1, 64, 2048, P, 0, P) in (1, 2)
    # indexer shape limits
    assert lib.dsa_indexer_logits(P, P, P, P, P, 0, 1, 1, 32, 128, 64, 64, P, 64, P) == 2
    assert lib.dsa_indexer_logits(P, P, P, P, P, 0, 1, 3, 64, 128, 64, 64, P, 64, P) == 2
    # sparse MLA: heads must be a multiple of 16, topk a multiple of 64
    assert lib.dsa_sparse_mla_decode(P, 0, 0, P, 42640, 64, 10, P, 0, 1, 24, 2048, ctypes.c_float(0.1), P, P,
                                     1, P, 0, P) == 2
    assert lib.dsa_sparse_mla_decode(P, 0, 0, P, 42640, 64, 10, P, 0, 1, 128, 100, ctypes.c_float(0.1), P, P,
                                     1, P, 0, P) == 2
    # a split count that does not split top-k into whole 64-row blocks
    assert lib.dsa_sparse_mla_decode(P, 0, 0, P, 42640, 64, 10, P, 0, 1, 128, 192, ctypes.c_float(0.1), P, P,
                                     2, P, 0, P) == 1
    # empty batches are a no-op success
    assert lib.dsa_topk_transform(P, 0, P, P, 0, P, P, 0, 0, 64, 2048, P, 0, P) == 0
    with pytest.raises(ValueError):
        _lib.check(1, "probe")


def test_workspace_size_queries(lib):
    assert lib.dsa_topk_workspace_bytes(0) == 0
    assert lib.dsa_topk_workspace_bytes(128) == 128 * (16 + 8 * 6144)
    # fused indexer + top-k: lists + full logits for rows the list select redoes
    assert lib.dsa_indexer_topk_workspace_bytes(0, 1, 65536) == 0
    assert lib.dsa_indexer_topk_workspace_bytes(128, 1, 65536) >= 128 * (16 + 8 * 6144) + 128 * 65536 * 4
    assert lib.dsa_sparse_mla_workspace_bytes(128, 128, 1) == 0
    assert lib.dsa_sparse_mla_workspace_bytes(32, 128, 4) == 4 * 32 * 128 * (512 + 1) * 4
    # splits grow until the grid (64 heads per workgroup) covers the CUs, in 64-row blocks of top-k
    assert lib.dsa_sparse_mla_num_splits(128, 128, 2048, 256) == 1
    assert lib.dsa_sparse_mla_num_splits(32, 128, 2048, 256) == 4
    assert lib.dsa_sparse_mla_num_splits(96, 128, 2048, 256) == 1   # two rounds of workgroups cost more
    assert lib.dsa_sparse_mla_num_splits(4, 128, 2048, 256) == 8    # at least 4 blocks per workgroup
    assert lib.dsa_sparse_mla_num_splits(1, 16, 128, 256) == 1      # two blocks: no split
    assert lib.dsa_sparse_mla_num_splits(1, 16, 512, 256) == 2      # eight blocks: two splits of four


def test_prefill_entry_points_reject_bad_arguments(lib):
    P = None
    # prefill windows: at least one sequence, non-negative sizes, pointers
    assert lib.dsa_prefill_windows(P, P, 0, 0, 4, 64, P, P, P, P) == 1
    assert lib.dsa_prefill_windows(P, P, 0, 2, 4, 0, P, P, P, P) == 1
    assert b"null pointer" in (lib.dsa_prefill_windows(P, P, 0, 2, 4, 64, P, P, P, P) == 1 and lib.dsa_last_error())
    # key assembly: rows of 576, a block stride that holds the block's rows, a
    # block count and table width that are not negative, 16-byte alignment
    assert lib.dsa_mla_prefill_kv(P, 64 * 656 - 1, 64, 8, P, 4, 4, P, P, 0, 1, 10, P, 576, P, 576, P) == 1
    assert lib.dsa_mla_prefill_kv(P, 42640, 64, 8, P, 4, 4, P, P, 0, 1, 10, P, 512, P, 576, P) == 1
    assert lib.dsa_mla_prefill_kv(P, 42640, 64, -1, P, 4, 4, P, P, 0, 1, 10, P, 576, P, 576, P) == 1
    assert lib.dsa_mla_prefill_kv(P, 42640, 64, 8, P, 4, -1, P, P, 0, 1, 10, P, 576, P, 576, P) == 1
    assert lib.dsa_mla_prefill_kv(P, 42640, 64, 8, P, 3, 4, P, P, 0, 1, 10, P, 576, P, 576, P) == 1   # stride < width
    assert lib.dsa_mla_prefill_kv(P, 42640, 64, 8, P, 4, 4, P, P, 0, 1, 0, P, 576, P, 576, P) == 0   # nothing to do
    # paged sparse prefill: workspace sizing and the workspace check come before any launch
    # cache-slot and fresh-row lists, 2048 wide each, and two counts per token
    assert lib.dsa_sparse_mla_prefill_paged_workspace_bytes(8192, 2048) == 2 * 8192 * 2048 * 4 + 8192 * 8
    assert lib.dsa_sparse_mla_prefill_paged_workspace_bytes(0, 2048) == 0
    ws = lib.dsa_sparse_mla_prefill_paged_workspace_bytes(10, 2048)
    f = ctypes.c_float(0.1)
    one = ctypes.c_void_p(16)  # a non-null address that is never dereferenced
    args = [one, 0, 0, one, 42640, 64, 10, one, 4, 4, one, one, 0, 1, 100, one, 576, 10, one, 2048, 10, 128, 2048,
            f, one, one, one, one]
    assert lib.dsa_sparse_mla_prefill_paged(*args, ws - 1, P) == 4          # workspace too small
    assert b"workspace" in lib.dsa_last_error()
    bad = list(args)
    bad[13] = 0                                                             # no sequences
    assert lib.dsa_sparse_mla_prefill_paged(*bad, ws, P) == 1
    bad = list(args)
    bad[27] = P                                                             # no workspace
    assert lib.dsa_sparse_mla_prefill_paged(*bad, ws, P) == 1
    bad = list(args)
    bad[9] = 5                                                              # table width > row stride
    assert lib.dsa_sparse_mla_prefill_paged(*bad, ws, P) == 1


def test_fused_prefill_topk_rejects_bad_arguments(lib):
    P = None
    one = ctypes.c_void_p(16)  # a non-null, aligned address that is never dereferenced
    rows, keys = 10, 5000
    ws = lib.dsa_mqa_topk_workspace_bytes(rows, keys, 2048)
    # the per-row candidate lists (6144 (key, position) pairs + 16-byte header) dominate
    assert ws >= rows * (16 + 6144 * 8)
    assert lib.dsa_mqa_topk_workspace_bytes(0, keys, 2048) == 0
    assert lib.dsa_mqa_topk_workspace_bytes(2 * rows, keys, 2048) > ws
    args = [one, one, one, one, 64, one, one, rows, keys, 64, keys, 2048, one, one]
    assert lib.dsa_mqa_topk(*args, ws - 1, P) == 4                         # workspace too small
    assert b"workspace" in lib.dsa_last_error()
    bad = list(args); bad[11] = 512                                        # ragged top-k is 2048 only
    assert lib.dsa_mqa_topk(*bad, ws, P) == 1
    bad = list(args); bad[9] = 32                                          # 64 indexer heads
    assert lib.dsa_mqa_topk(*bad, ws, P) == 2
    bad = list(args); bad[10] = (1 << 18) + 1                              # rows past the select's limit
    assert lib.dsa_mqa_topk(*bad, ws, P) == 2
    bad = list(args); bad[0] = P                                           # no query
    assert lib.dsa_mqa_topk(*bad, ws, P) == 1
    bad = list(args); bad[7] = 0                                           # nothing to do
    assert lib.dsa_mqa_topk(*bad, 0, P) == 0


def test_microbenchmark_library_exports_its_probes():
    """The measurements behind the kernels' design (bench.py --micro) come from
    a separate library; it loads without a device and exports every probe."""
    from nanoengine_amd.build import MICROBENCH_LIB
    if not MICROBENCH_LIB.exists():
        from nanoengine_amd import build
        build.build()
    mb = ctypes.CDLL(str(MICROBENCH_LIB))
    for name in ["dsa_mb_page_read", "dsa_mb_page_read_layout", "dsa_mb_row_gather", "dsa_mb_lds_read", "dsa_mb_valu_issue",
                 "dsa_mb_mfma_rate", "dsa_mb_mix", "dsa_mb_fp8_mfma_sum"]:
        assert hasattr(mb, name), name
