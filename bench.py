"""DSA decode step benchmark on one MI355X.

One step = fp8 lightning indexer (fp8 MFMA over the paged indexer cache) ->
exact top-2048 with page translation -> sparse MLA decode over the paged fp8
MLA cache, for batch 128, next_n 1, 64K context per sequence, 64 indexer heads
x 128, 128 MLA heads x 576/512. The indexer and the top-k run fused
(dsa_indexer_topk: the logits never reach memory); --unfused runs them as two
operators over a logits buffer instead. Inputs are seeded synthetic data
already resident in HBM; block tables are a random permutation of the page pool.

Prints ONE JSON line. `value` is decode tokens/s (= batch / step time);
`roofline` covers the dominant kernel (the indexer's filter pass over every key
page, HBM-bound), timed with HIP events that the library records on the stream
the kernels run on; `stages` reports every phase; `cpu_baseline` times the numpy
oracle of the same step on a bounded sample of the sequences on the host cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--unfused]
       python bench.py --copy-calib   (a plain 1 GiB device copy, for scaling
                                       rocprofv3 FETCH_SIZE/WRITE_SIZE)
       python bench.py --only {fused,indexer,topk,mla}   (profiling: one stage only)
       python bench.py --micro        (the microbenchmarks behind the kernels' design)
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "DSA decode µs/step & tokens/s at B=128,64K ctx,k=2048; % HBM / fp8-MFMA peak"
HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0
BF16_PEAK_TFLOPS = 2500.0
PMC_SUMMARY = os.path.join(ROOT, "profiles", "indexer_filter_config2_pmc.txt")


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--batch", type=int, default=128)
    p.add_argument("--ctx", type=int, default=65536)
    p.add_argument("--heads", type=int, default=128)
    p.add_argument("--topk", type=int, default=2048)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-sample", type=int, default=16, help="sequences in the CPU baseline sample")
    p.add_argument("--copy-calib", action="store_true")
    p.add_argument("--micro", action="store_true",
                   help="run the microbenchmarks of libdsa_microbench.so (one JSON line each)")
    p.add_argument("--unfused", action="store_true", help="indexer logits + top-k as two operators")
    p.add_argument("--config", type=int, choices=[1, 2, 3, 4], default=2,
                   help="1: sparse MLA decode alone, B=32 x 32K; 2: decode B=128 x 64K (the headline); "
                        "3: MTP verify, B=64, next_n=2, "
                        "lognormal lengths (median 16K, clipped to 2K-128K); 4: chunked prefill, "
                        "8192 queries over a 120K cached prefix (128K keys)")
    p.add_argument("--headline-only", action="store_true",
                   help="config 2 alone (without the embedded figures of configs 1, 3 and 4)")
    p.add_argument("--only", choices=["fused", "indexer", "topk", "mla", "logits", "kv", "mlabf16"], default=None,
                   help="profiling aid: launch only this stage in the timed loop (no JSON line)")
    return p.parse_args()


def pmc_traffic():
    """HBM bytes per filter-kernel launch from the committed rocprofv3 PMC summary, if any."""
    try:
        with open(PMC_SUMMARY) as f:
            m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", f.read(), re.M)
        return float(m.group(1)) if m else None
    except OSError:
        return None


def copy_calib():
    import torch
    n = 1 << 30
    a = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    b = torch.empty_like(a)
    for _ in range(5):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": n, "launches": 5}))


def micro():
    """The measurements behind the kernels' design (nanoengine_amd/csrc/microbench.hip)."""
    import ctypes

    import torch

    from nanoengine_amd.build import MICROBENCH_LIB

    lib = ctypes.CDLL(str(MICROBENCH_LIB))
    dev = torch.device("cuda:0")
    st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    sink = torch.zeros(16, dtype=torch.int32, device=dev)

    def timed(fn, reps=5):
        fn()
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            best = min(best, e0.elapsed_time(e1) * 1e-3)
        return best

    def check(rc, what):
        if rc != 0:
            raise RuntimeError(f"{what}: HIP error {rc}")

    g = torch.Generator(device=dev).manual_seed(1)
    # 1. random 8448-byte pages, the config-2 indexer pool (131072 pages = 1.107 GB)
    npages, grid = 131072, 512
    pool = torch.randint(0, 255, (npages * 8448,), dtype=torch.uint8, device=dev, generator=g)
    ids = torch.randperm(npages, device=dev, generator=g).to(torch.int32)
    per_wave = npages // (grid * 4)
    nbytes = npages * 8448
    for layout, name in ((0, "whole rows, plain loads"), (1, "whole rows, nontemporal loads"),
                         (2, "MFMA operand layout, nontemporal loads")):
        t = timed(lambda: check(lib.dsa_mb_page_read_layout(ctypes.c_void_p(pool.data_ptr()),
                                                            ctypes.c_void_p(ids.data_ptr()), per_wave, grid, layout,
                                                            ctypes.c_void_p(sink.data_ptr()), st), "page_read"))
        print(json.dumps({"micro": "page_read", "layout": name, "pages": npages, "page_bytes": 8448,
                          "waves": grid * 4, "us": round(t * 1e6, 1), "TBps": round(nbytes / t / 1e12, 3)}),
              flush=True)
    del pool, ids
    # 2. random 656-byte rows into LDS (5 GB pool, 64-row blocks, two in flight)
    nrows, nblk, grid = (5 << 30) // 656, 32, 256
    pool = torch.zeros(nrows * 656, dtype=torch.uint8, device=dev)
    t = timed(lambda: check(lib.dsa_mb_row_gather(ctypes.c_void_p(pool.data_ptr()), ctypes.c_int64(nrows), nblk,
                                                  grid, ctypes.c_void_p(sink.data_ptr()), st), "row_gather"))
    nbytes = grid * nblk * 64 * 656
    print(json.dumps({"micro": "row_gather_lds", "rows": grid * nblk * 64, "row_bytes": 656,
                      "workgroups": grid, "us": round(t * 1e6, 1), "TBps": round(nbytes / t / 1e12, 3)}), flush=True)
    del pool
    # 3. LDS read bandwidth per CU (clock64 cycles of each workgroup)
    cyc = torch.zeros(256 * 16, dtype=torch.int64, device=dev)
    iters = 4096
    for waves in (4, 8, 16):
        check(lib.dsa_mb_lds_read(waves, iters, 256, ctypes.c_void_p(sink.data_ptr()), ctypes.c_void_p(cyc.data_ptr()),
                                  st), "lds_read")
        torch.cuda.synchronize()
        c = float(cyc[:256].double().mean())
        print(json.dumps({"micro": "lds_read_b128", "waves_per_cu": waves,
                          "bytes_per_clk_per_cu": round(iters * 8 * 16 * 64 * waves / c, 1)}), flush=True)
    # 4. VALU issue: cycles per independent instruction of one wave
    for op, name in ((0, "v_fma_f32"), (1, "v_exp_f32")):
        for threads in (256, 512, 1024):
            iters = 2048
            check(lib.dsa_mb_valu_issue(op, threads, iters, 256, ctypes.c_void_p(sink.data_ptr()),
                                        ctypes.c_void_p(cyc.data_ptr()), st), "valu_issue")
            torch.cuda.synchronize()
            c = float(cyc[:256 * threads // 64].double().mean())
            print(json.dumps({"micro": "valu_issue", "op": name, "waves_per_simd": threads // 256,
                              "cycles_per_instr_per_wave": round(c / (iters * 12), 2)}), flush=True)
    # 5. MFMA rates (4 independent accumulators per wave, 4 waves per workgroup, 4 workgroups per CU)
    fsink = torch.zeros(16, dtype=torch.float32, device=dev)
    for shape, name, flop in ((0, "bf16_32x32x16", 2 * 32 * 32 * 16), (3, "bf16_16x16x32", 2 * 16 * 16 * 32),
                              (1, "fp8_scaled_32x32x64", 2 * 32 * 32 * 64), (2, "fp8_scaled_16x16x128", 2 * 16 * 16 * 128)):
        iters, grid = 2048, 1024
        t = timed(lambda: check(lib.dsa_mb_mfma_rate(shape, iters, grid, ctypes.c_void_p(fsink.data_ptr()), st),
                                "mfma_rate"))
        total = flop * 4 * iters * grid * 4
        peak = FP8_PEAK_TFLOPS if "fp8" in name else BF16_PEAK_TFLOPS
        print(json.dumps({"micro": "mfma_rate", "shape": name, "TFLOPs": round(total / t / 1e12, 1),
                          "frac_of_peak": round(total / t / 1e12 / peak, 3)}), flush=True)
    # 6. MFMA beside VALU on one SIMD: cycles per iteration (4 MFMAs / 16 VALU) of each kind of wave
    mcyc = torch.zeros(256 * 8, dtype=torch.int64, device=dev)
    for op, name in ((0, "v_fma_f32"), (1, "v_cvt_scalef32_pk_bf16_fp8")):
        res = {"micro": "mfma_beside_valu", "valu_op": name}
        for mode, tag in ((1, "mfma_alone"), (2, "valu_alone"), (3, "both")):
            iters = 2000
            check(lib.dsa_mb_mix(op, mode, iters, 256, ctypes.c_void_p(fsink.data_ptr()),
                                 ctypes.c_void_p(mcyc.data_ptr()), st), "mix")
            torch.cuda.synchronize()
            c = mcyc.view(256, 8).double()
            res[tag] = {"mfma_wave": round(float(c[:, :4].mean()) / iters, 1) if mode & 1 else None,
                        "valu_wave": round(float(c[:, 4:].mean()) / iters, 1) if mode & 2 else None}
        print(json.dumps(res), flush=True)
    # 8. summation error of each MFMA shape on random operands (values spread
    # over up to 16 binades), against the bound the oracle's logit checks use:
    # each product and each addition truncated toward zero at a quantum of
    # 2^(floor(log2 max|p|) - 13)
    import numpy as np
    rng = np.random.default_rng(0)
    for shape, name in ((0, "fp8_scaled_16x16x128"), (1, "fp8_scaled_32x32x64"), (2, "fp8_16x16x32"),
                        (3, "fp8_32x32x16"), (4, "bf16_32x32x16")):
        A, B, C = _mfma_probe_run(lib, st, dev, shape, rng, 400)
        print(json.dumps({"micro": "mfma_sum_bound", "shape": name, **_mfma_probe_stats(A, B, C)}), flush=True)
    # 7. summation precision of the scaled fp8 MFMA: products 2^p and +-1.875 in one output
    out = torch.zeros(17 * 64, dtype=torch.float32, device=dev)
    for sign in (1, -1):
        check(lib.dsa_mb_fp8_mfma_sum(sign, ctypes.c_void_p(out.data_ptr()), st), "fp8_mfma_sum")
        torch.cuda.synchronize()
        got = out.view(17, 64)[:, 0].cpu().tolist()
        exact = [2.0 ** p + sign * 1.875 for p in range(17)]
        print(json.dumps({"micro": "fp8_mfma_sum", "small_product": sign * 1.875,
                          "first_p_not_exact": next((p for p in range(17) if got[p] != exact[p]), None),
                          "small_part_kept": {p: got[p] - 2.0 ** p for p in range(17)}}), flush=True)


# Probed MFMA shapes: (M, N, K, bytes per element). Lane l of each operand holds
# row (A) or column (B) l % M and elements K/(64/M) * (l // M) .. of the k axis;
# the result layout is the standard 16x16 (4 registers) or 32x32 (16) one.
_PROBE_SHAPES = {0: (16, 16, 128, 1), 1: (32, 32, 64, 1), 2: (16, 16, 32, 1), 3: (32, 32, 16, 1),
                 4: (32, 32, 16, 2)}


def _mfma_probe_run(lib, st, dev, shape, rng, cases):
    """Random operands for one MFMA shape through dsa_mb_mfma_probe: returns the
    decoded A [c,M,K], B [c,K,N] (float64) and the GPU's C [c,M,N]."""
    import ctypes

    import numpy as np
    import torch
    M, N, K, eb = _PROBE_SHAPES[shape]
    spread = lambda *sh: np.exp2(rng.integers(-8, 8, sh))   # noqa: E731
    if eb == 1:
        x = np.clip(rng.standard_normal((cases, M, K)) * spread(cases, M, K), -448, 448)
        y = np.clip(rng.standard_normal((cases, K, N)) * spread(cases, 1, 1), -448, 448)
        Ac = torch.from_numpy(x.astype(np.float32)).to(torch.float8_e4m3fn)
        Bc = torch.from_numpy(y.astype(np.float32)).to(torch.float8_e4m3fn)
        raw = lambda t: t.view(torch.uint8).numpy()   # noqa: E731
    else:
        x = rng.standard_normal((cases, M, K)) * spread(cases, M, K)
        y = rng.standard_normal((cases, K, N))
        Ac = torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16)
        Bc = torch.from_numpy(y.astype(np.float32)).to(torch.bfloat16)
        raw = lambda t: t.view(torch.int16).numpy().view(np.uint16)   # noqa: E731
    a_el, b_el = raw(Ac), raw(Bc)
    groups = 64 // M
    kc = K // groups
    a = np.zeros((cases, 64, 32 // eb), a_el.dtype)
    b = np.zeros((cases, 64, 32 // eb), b_el.dtype)
    for l in range(64):
        r, g = l % M, l // M
        a[:, l, :kc] = a_el[:, r, g * kc:(g + 1) * kc]
        b[:, l, :kc] = b_el[:, g * kc:(g + 1) * kc, r]
    ta = torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).to(dev)
    tb = torch.from_numpy(np.ascontiguousarray(b).view(np.int32)).to(dev)
    out = torch.zeros(cases, 64, 16, dtype=torch.float32, device=dev)
    rc = lib.dsa_mb_mfma_probe(shape, cases, ctypes.c_void_p(ta.data_ptr()), ctypes.c_void_p(tb.data_ptr()),
                               ctypes.c_void_p(out.data_ptr()), st)
    if rc != 0:
        raise RuntimeError(f"mfma_probe: HIP error {rc}")
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    C = np.zeros((cases, M, N))
    for l in range(64):
        for i in range(4 if M == 16 else 16):
            row = 4 * (l // 16) + i if M == 16 else 8 * (i // 4) + 4 * (l // 32) + i % 4
            C[:, row, l % M] = o[:, l, i]
    return Ac.double().numpy(), Bc.double().numpy(), C


def _mfma_probe_stats(A, B, C):
    """Error of each dot against the exact sum, in units of q = 2^(E - 13)
    (E = floor(log2 of the largest product)) and against the bound
    B = sum_i (|p_i| - |trunc(p_i / q) q|) + (n - 1) q + one f32 rounding."""
    import numpy as np
    P = A[:, :, None, :] * np.transpose(B, (0, 2, 1))[:, None, :, :]
    err = np.abs(C - P.sum(-1))
    pm = np.abs(P).max(-1)
    ok = pm > 0
    q = np.exp2(np.floor(np.log2(np.where(ok, pm, 1.0))) - 13)
    n = (P != 0).sum(-1)
    R = (np.abs(P) - np.abs(np.trunc(P / q[..., None]) * q[..., None])).sum(-1) + np.maximum(n - 1, 0) * q \
        + 2.0 ** -24 * np.abs(P.sum(-1))
    return {"dots": int(ok.sum()), "exact_share": round(float((err[ok] == 0).mean()), 4),
            "max_err_over_quantum": round(float((err[ok] / q[ok]).max()), 3),
            "max_err_over_bound": round(float((err[ok] / np.maximum(R[ok], 1e-300)).max()), 4),
            "max_err_over_max_product": float((err[ok] / pm[ok]).max())}


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(inp, kv, q_mla, qlens, next_n, sample, scale, topk, step, reps=3, timed=True):
    """Times the numpy oracle of the full step (indexer logits, exact top-k with
    page translation, sparse MLA) on `sample` query rows spread over the batch,
    on every host core: one warm-up, then `reps` timed repetitions, median
    (``timed=False``: the parity check alone). Then checks the GPU step's
    outputs for the same rows against it (logits, top-k, physical slots, o,
    LSE) and returns (baseline or None, parity report). ``qlens`` holds each
    query token's own causal length [B * next_n]."""
    import numpy as np
    import torch
    from threadpoolctl import threadpool_limits

    import oracle as O
    from oracle import step_check as SC
    from nanoengine_amd import ops

    cores = os.cpu_count() or 1
    T = len(qlens)
    B = T // next_n
    rows = SC.spread_rows(T, sample)
    S = len(rows)
    max_ctx = inp.block_tables.shape[1] * 64
    # the GPU side of the parity check: the step's last outputs, plus the
    # standalone logits operator for the same inputs
    seq = torch.as_tensor(qlens, dtype=torch.int32, device=inp.cache.device)
    logits = ops.indexer_logits(inp.q_fp8.view(B, next_n, 64, 128), inp.cache, inp.weights, seq.view(B, next_n),
                                inp.block_tables, max_ctx)
    torch.cuda.synchronize()
    data = SC.sample_from_device(rows, q_idx_fp8=inp.q_fp8, weights=inp.weights, cache=inp.cache, lens=qlens,
                                 block_tables=inp.block_tables, q_mla=q_mla, kv=kv, logits=logits,
                                 logical=step.logical, physical=step.physical, o=step.out, lse=step.lse,
                                 next_n=next_n)
    del logits
    used, bt = SC.localize_pages(data["bt_global"], data["ctx"])
    kv_rows = kv[torch.as_tensor(used, dtype=torch.long, device=kv.device)].contiguous().reshape(-1, 656).cpu().numpy()
    ctx = data["ctx"].reshape(S, 1)

    def oracle_step():
        lg = O.indexer_logits(data["q_idx"], data["idx_pages"], data["weights"], ctx, bt, max_ctx)
        page, _ = O.topk_transform(lg, ctx.reshape(-1), bt, 64, topk)
        O.sparse_mla_decode(data["q_mla"], kv_rows, page, scale)
        return lg

    times = []
    with threadpool_limits(limits=cores):
        exp_logits = oracle_step()          # warm-up
        for _ in range(reps if timed else 0):
            t0 = time.perf_counter()
            oracle_step()
            times.append(time.perf_counter() - t0)
        rep = SC.check_step_rows(**data, sm_scale=scale, topk=topk, exp_logits=exp_logits)
    base = None
    if timed:
        dt = sorted(times)[len(times) // 2]
        base = {"value": round(S / dt, 3), "unit": "tokens/s", "cores": cores, "kind": "port",
                "cpu_model": cpu_model(),
                "sample": f"{S} of {T} query rows spread over the batch (rows {rows.tolist()}), same workload: "
                          f"numpy oracle of indexer logits + exact top-{topk} + transform + sparse MLA; "
                          f"median of {reps} timed runs after 1 warm-up, {dt:.2f} s each "
                          f"(runs: {', '.join(f'{t:.2f}' for t in times)})"}
    rep = {k: (round(v, 6) if isinstance(v, float) else v) for k, v in rep.items()}
    rep["rows"] = rows.tolist()
    return base, rep


def prologue_stages(T, dev, seed, reps=50):
    """Average launch time of the indexer prologue kernels for the step's T query
    tokens (they run before the step, so they are reported beside it, not in it):
    the query transform over T x 64 heads and the key transform + store of T keys."""
    import torch

    from nanoengine_amd import ops
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(T, 64, 128, generator=g).to(torch.bfloat16).to(dev)
    gate = torch.randn(T, 64, generator=g).to(torch.bfloat16).to(dev)
    key = torch.randn(T, 128, generator=g).to(torch.bfloat16).to(dev)
    cs = torch.randn(131072, 64, generator=g).to(dev)
    pos = torch.randint(0, 131072, (T,), generator=g).to(dev)
    slots = torch.randperm(T * 4, generator=g)[:T].to(torch.int32).to(dev)
    lw, lb = torch.ones(128, device=dev), torch.zeros(128, device=dev)
    q8 = torch.empty(T, 64, 128, dtype=torch.uint8, device=dev)
    w = torch.empty(T, 64, dtype=torch.float32, device=dev)
    cache = torch.zeros((T * 4 + 63) // 64 * 64 * 132, dtype=torch.uint8, device=dev)
    calls = {
        "indexer_q_prologue": (lambda: ops.indexer_q_prologue(q, gate, 0.01, cs, pos, q8, w),
                               T * 64 * (256 + 128 + 4 + 2) + T * 256),
        "indexer_k_transform_store": (lambda: ops.indexer_k_transform_store(key, lw, lb, 1e-6, pos, cs, cache,
                                                                            slots, 64), T * (256 + 132 + 256)),
    }
    out = {}
    for name, (fn, nbytes) in calls.items():
        for _ in range(5):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        out[name] = {"us": round(us, 2), "tokens": T, "bytes": nbytes,
                     "GBps": round(nbytes / (us * 1e-6) / 1e9, 1)}
    return out


def cpu_baseline_prefill(host, rows, scale, topk, gpu, reps=3):
    """The numpy oracle of config 4 on the host cores: the per-chunk work (the
    indexer key gather and the MLA key assembly from the fp8 cache) once, and
    the per-query work (ragged logits, exact top-k, sparse MLA prefill) for the
    sampled query rows; one warm-up, `reps` timed runs, medians. The reported
    rate is the chunk's queries over (per-chunk time + queries x per-query
    time). Then checks the GPU's outputs for the same rows against it: logits
    within each row's window, the top-k of the GPU's own logits, the assembled
    keys (bit-exact) and the MLA output."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    import oracle as O

    cores = os.cpu_count() or 1
    QN, KN = host["QN"], host["KN"]
    S = len(rows)
    ks = np.zeros(S, np.int32)
    ke = (KN - QN + 1 + rows).astype(np.int32)

    def chunk_part():
        keys, kscale = O.gather_indexer_cache(host["idx_cache"], host["bt"], host["cu_k"])
        kv = O.assemble_prefill_kv(host["mla_rows"], 64, host["bt"], host["cu_q"], host["cu_k"], host["fresh"])
        return keys, kscale, kv

    def row_part(keys, kscale, kv):
        lg = O.mqa_logits(host["q8"], keys, kscale, host["w"], ks, ke, clean_logits=True)
        idx = O.topk_transform_ragged(lg, ke - ks, ks, ks, topk)
        o, mx, lse = O.sparse_mla_prefill(host["q_mla"], kv, idx, scale)
        return lg, idx, o, lse

    t_chunk, t_rows = [], []
    with threadpool_limits(limits=cores):
        keys, kscale, kv = chunk_part()                 # warm-up
        exp = row_part(keys, kscale, kv)
        for _ in range(reps):
            t0 = time.perf_counter()
            keys, kscale, kv = chunk_part()
            t1 = time.perf_counter()
            row_part(keys, kscale, kv)
            t2 = time.perf_counter()
            t_chunk.append(t1 - t0)
            t_rows.append(t2 - t1)
        # parity: the GPU's rows against the oracle (1e-3 relative, or the
        # scaled fp8 MFMA's derived bound where a head sum cancels)
        from oracle import step_check as SC
        lg_exp = exp[0]
        lg = SC.check_logits(gpu["logits"], lg_exp, ke, SC.ragged_logit_bound(host["q8"], host["w"], keys, kscale))
        rel = lg["max_rel_err"]
        own = O.topk_transform_ragged(np.where(np.arange(KN)[None, :] < ke[:, None], gpu["logits"], -np.inf),
                                      ke - ks, ks, ks, topk)
        topk_equal = all(set(own[r][own[r] >= 0].tolist()) == set(gpu["idx"][r][gpu["idx"][r] >= 0].tolist())
                         for r in range(S))
        used = np.unique(gpu["idx"][gpu["idx"] >= 0])
        kv_equal = bool(np.array_equal(gpu["kv_rows"], kv[used]))
        o_exp, _, lse_exp = O.sparse_mla_prefill(host["q_mla"], kv, gpu["idx"], scale)
    o_err = float(np.abs(gpu["o"] - o_exp).max())
    lse_err = float(np.abs(gpu["lse"] - lse_exp).max())
    tc, tr = sorted(t_chunk)[len(t_chunk) // 2], sorted(t_rows)[len(t_rows) // 2]
    per_query = tr / S
    value = QN / (tc + QN * per_query)
    base = {"value": round(value, 3), "unit": "tokens/s", "cores": cores, "kind": "port", "cpu_model": cpu_model(),
            "sample": f"per-chunk work (indexer key gather + MLA key assembly from the fp8 cache, {KN} keys) "
                      f"in full, {tc:.2f} s; per-query work (ragged logits, exact top-{topk}, sparse MLA "
                      f"prefill) on {S} of {QN} queries spread over the chunk (rows {rows.tolist()}), "
                      f"{tr:.2f} s; medians of {reps} timed runs after 1 warm-up; value = {QN} / "
                      f"({tc:.2f} + {QN} x {per_query:.3f}) s"}
    ok = lg["ok"] and topk_equal and kv_equal and o_err <= 2e-2 and lse_err <= 1e-3
    parity = {"rows": rows.tolist(), "logits_max_rel_err": round(rel, 6), "logits_over_rtol": lg["over_rtol"],
              "logits_max_err_over_mfma_bound": lg["max_err_over_bound"], "topk_equal_on_gpu_logits": topk_equal,
              "kv_rows_bit_exact": kv_equal, "o_max_abs_err": round(o_err, 6), "lse_max_abs_err": round(lse_err, 6),
              "ok": bool(ok)}
    return base, parity


def bench_prefill(args):
    """one 8192-token chunk over a 122880-token cached prefix
    (131072 keys in all). Stages, each timed with HIP events on the launch
    stream over `steps` repetitions: the paged-to-ragged indexer key gather,
    the ragged fp8 MQA logits [8192 x 131072] (causal windows) fused with the
    exact ragged top-2048 (dsa_mqa_topk: no logits buffer), and the sparse MLA
    prefill: the selected keys of the cached prefix read from the paged fp8
    MLA cache, those of the chunk's fresh keys as bf16 rows
    (dsa_sparse_mla_prefill_paged). The reference's routes are timed beside
    them: logits into a buffer then the ragged top-k (whose indices must equal
    the fused entry's on every row), and the keys assembled as bf16 rows then
    the bf16 sparse prefill."""
    import numpy as np
    import torch

    from nanoengine_amd import _lib, mla_utils, ops, synth
    from nanoengine_amd.indexer import gather_indexer_cache

    _lib.load()
    dev = torch.device("cuda:0")
    QN, KN, K = 8192, 131072, args.topk
    inp = synth.make_indexer_inputs([KN], next_n=1, seed=args.seed, device=dev)
    dgen = torch.Generator(device=dev).manual_seed(args.seed + 3)
    q = torch.randn(QN, 64, 128, generator=dgen, device=dev).to(torch.bfloat16)
    q_codes, q_scale = synth.ue8m0_quant_rows(q)
    w = (torch.randn(QN, 64, generator=dgen, device=dev) * 64 ** -0.5 * 128 ** -0.5 * q_scale).float().contiguous()
    q8 = q_codes.view(torch.float8_e4m3fn)
    cu_q = torch.tensor([0, QN], dtype=torch.int32, device=dev)
    cu_k = torch.tensor([0, KN], dtype=torch.int32, device=dev)
    ks = torch.zeros(QN, dtype=torch.int32, device=dev)
    ke = (KN - QN + 1 + torch.arange(QN, dtype=torch.int32, device=dev)).contiguous()
    lens = (ke - ks).contiguous()
    logits = torch.empty(QN, KN, dtype=torch.float32, device=dev)
    idx = torch.empty(QN, K, dtype=torch.int32, device=dev)
    keys, scales = gather_indexer_cache(inp.cache, inp.block_tables, cu_k, page_size=64, head_dim=128, total_k=KN)
    ws = torch.empty(ops.topk_workspace_bytes(QN), dtype=torch.uint8, device=dev)
    kvs = scales.view(torch.float32).reshape(-1)
    # the MLA keys: the cached prefix lives in the paged fp8 MLA cache (same
    # block table as the indexer pages), the chunk's own keys arrive as bf16
    H = args.heads
    num_blocks = int(inp.block_tables.max().item()) + 1
    kv_cache = synth.make_mla_cache(num_blocks, seed=args.seed, device=dev)
    fresh = torch.randn(QN, 576, generator=dgen, device=dev).to(torch.bfloat16)
    kv_bf16 = torch.empty(KN, 576, dtype=torch.bfloat16, device=dev)
    q_mla = torch.randn(QN, H, 576, generator=dgen, device=dev).to(torch.bfloat16)
    mla_out = torch.empty(QN, H, 512, dtype=torch.bfloat16, device=dev)
    mla_max = torch.empty(QN, H, dtype=torch.float32, device=dev)
    mla_lse = torch.empty(QN, H, dtype=torch.float32, device=dev)
    scale = 192 ** -0.5
    pws = torch.empty(ops.sparse_mla_prefill_paged_workspace_bytes(QN, K), dtype=torch.uint8, device=dev)
    tws = torch.empty(ops.mqa_topk_workspace_bytes(QN, KN, K), dtype=torch.uint8, device=dev)
    idx2 = torch.empty_like(idx)
    stages = [
        ("gather_indexer_cache", lambda: ops.gather_indexer_cache(inp.cache, inp.block_tables, cu_k, 64, KN, keys,
                                                                  scales)),
        # logits and the exact top-2048 in one pass: no logits buffer
        ("mqa_topk", lambda: ops.mqa_topk(q8, keys.view(torch.float8_e4m3fn), kvs, w, ks, ke, KN, idx, K,
                                          workspace=tws)),
        # the cached keys straight from the paged fp8 cache, the fresh keys as bf16 rows
        ("sparse_mla_prefill_paged", lambda: ops.sparse_mla_prefill_paged(
            q_mla, kv_cache, inp.block_tables, cu_q, cu_k, fresh, idx, scale, KN, out=mla_out, max_logits=mla_max,
            lse=mla_lse, workspace=pws)),
    ]
    # the same attention through the assembled bf16 keys, timed beside the step
    alt_out = torch.empty_like(mla_out)
    alt_max, alt_lse = torch.empty_like(mla_max), torch.empty_like(mla_lse)
    alternative = [
        # the indexer as two operators over a [QN, KN] f32 logits buffer
        ("mqa_logits", lambda: ops.mqa_logits(q8, keys.view(torch.float8_e4m3fn), kvs, w, ks, ke, logits, False)),
        ("topk_transform_ragged", lambda: ops.topk_transform_ragged(logits, lens, ks, ks, idx2, K, workspace=ws)),
        ("mla_prefill_kv", lambda: ops.mla_prefill_kv(kv_cache, inp.block_tables, cu_q, cu_k, fresh, KN, kv_bf16)),
        ("sparse_mla_prefill", lambda: ops.sparse_mla_prefill(q_mla, kv_bf16, idx, scale, out=alt_out,
                                                              max_logits=alt_max, lse=alt_lse)),
    ]
    only = {"logits": "mqa_logits", "topk": "mqa_topk", "mla": "sparse_mla_prefill_paged", "kv": "mla_prefill_kv",
            "mlabf16": "sparse_mla_prefill"}.get(args.only)
    for _ in range(max(1, args.warmup)):
        for _, fn in stages:
            fn()
    torch.cuda.synchronize()
    steps = max(1, args.steps)
    for _, fn in alternative:
        fn()
    torch.cuda.synchronize()
    if only is not None:
        # profiling aid: the inputs are built, then only the named stage repeats
        fn = dict(stages + alternative)[only]
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        return
    t0 = time.perf_counter()
    for _ in range(steps):
        for _, fn in stages:
            fn()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    out = {}
    for name, fn in stages + alternative:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        out[name] = {"us": round(e0.elapsed_time(e1) * 1e3 / steps, 1)}
    pairs = int(lens.sum().item())
    flops = 2.0 * 64 * 128 * pairs
    ft = out["mqa_topk"]
    ft.update({"flops": flops, "TFLOPs": round(flops / (ft["us"] * 1e-6) / 1e12, 1),
               "fp8_mfma_frac": round(flops / (ft["us"] * 1e-6) / 1e12 / FP8_PEAK_TFLOPS, 4),
               "phases": ["prep", "sample keys", "sampled logits (1/64 of the keys)", "threshold",
                          "logits + filter", "list select", "fix-up of deferred rows (none here)"]})
    out["mqa_logits"].update({"flops": flops, "pairs": pairs,
                              "TFLOPs": round(flops / (out["mqa_logits"]["us"] * 1e-6) / 1e12, 1),
                              "fp8_mfma_frac": round(flops / (out["mqa_logits"]["us"] * 1e-6) / 1e12
                                                     / FP8_PEAK_TFLOPS, 4),
                              "logits_bytes": QN * KN * 4})
    mla_pairs = int((idx >= 0).sum().item())
    mla_flops = 2.0 * H * (576 + 512) * mla_pairs
    fresh_pairs = int((idx >= KN - QN).sum().item())
    for name in ("sparse_mla_prefill_paged", "sparse_mla_prefill"):
        mu = out[name]["us"]
        out[name].update({"flops": mla_flops, "TFLOPs": round(mla_flops / (mu * 1e-6) / 1e12, 1),
                          "bf16_mfma_frac": round(mla_flops / (mu * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4),
                          "heads": H})
    out["sparse_mla_prefill_paged"]["fresh_key_share"] = round(fresh_pairs / max(mla_pairs, 1), 4)
    out["alternative_assembled_bf16"] = {"us": round(out.pop("mla_prefill_kv")["us"] + out["sparse_mla_prefill"]["us"], 1),
                                         "stages": ["mla_prefill_kv", "sparse_mla_prefill"],
                                         "sparse_mla_prefill": out.pop("sparse_mla_prefill")}
    out["topk_transform_ragged"]["GBps"] = round(QN * KN * 4 / (out["topk_transform_ragged"]["us"] * 1e-6) / 1e9, 1)
    out["alternative_two_step_indexer"] = {
        "us": round(out["mqa_logits"]["us"] + out["topk_transform_ragged"]["us"], 1),
        "stages": ["mqa_logits", "topk_transform_ragged"],
        "mqa_logits": out.pop("mqa_logits"), "topk_transform_ragged": out.pop("topk_transform_ragged")}
    fused_equal = bool(torch.equal(idx, idx2))

    base, parity = None, None
    if not args.no_cpu_baseline:
        rows = np.linspace(0, QN - 1, 8).round().astype(np.int64)
        rt = torch.as_tensor(rows, device=dev)
        bt_np = inp.block_tables.cpu().numpy()
        host = {"QN": QN, "KN": KN, "idx_cache": inp.cache.cpu().numpy(), "bt": bt_np,
                "cu_q": np.array([0, QN]), "cu_k": np.array([0, KN]),
                "mla_rows": kv_cache.contiguous().reshape(-1, 656).cpu().numpy(),
                "fresh": fresh.float().cpu().numpy(), "q8": q_codes[rt].cpu().numpy(), "w": w[rt].cpu().numpy(),
                "q_mla": q_mla[rt].float().cpu().numpy()}
        used = torch.unique(idx[rt][idx[rt] >= 0])
        ops.mla_prefill_kv(kv_cache, inp.block_tables, cu_q, cu_k, fresh, KN, kv_bf16)   # rows for the key check
        gpu = {"logits": logits[rt].cpu().numpy(), "idx": idx[rt].cpu().numpy(),
               "kv_rows": kv_bf16[used].float().cpu().numpy(), "o": mla_out[rt].float().cpu().numpy(),
               "lse": mla_lse[rt].cpu().numpy()}
        base, parity = cpu_baseline_prefill(host, rows, scale, K, gpu)
    line = {
        "metric": METRIC, "value": round(QN / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": steps, "warmup": args.warmup, "ms_per_step": round(ms, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp8+bf16", "data": "synthetic",
        "config": {"workload": "BASELINE config 4: chunked prefill (indexer key gather + ragged fp8 MQA logits "
                               "fused with the exact ragged top-2048 + sparse MLA prefill over the paged fp8 cache and the fresh bf16 "
                               "rows), one layer", "queries": QN,
                   "keys": KN, "cached_prefix": KN - QN, "index_topk": K, "indexer_heads": 64,
                   "indexer_head_dim": 128, "mla_heads": H, "mla_dims": "576/512", "parallelism": "single GPU"},
        # the whole fused entry (every phase) priced as the logits contraction: a
        # lower bound on its dominant kernel's rate
        "roofline": {"bound": "mfma", "achieved": ft["TFLOPs"], "peak": FP8_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": ft["fp8_mfma_frac"], "traffic": None,
                     "kernel": "dsa_mqa_topk (mqa_logits_kernel<filter> + sample, threshold, list select)",
                     "flops_per_launch": flops, "avg_launch_us": ft["us"]},
        "stages": out, "cpu_baseline": base,
    }
    if parity is not None:
        line["parity"] = parity
    else:
        line["parity"] = {"ok": fused_equal}
    line["parity"]["fused_topk_equals_two_step_all_rows"] = fused_equal
    line["parity"]["ok"] = bool(line["parity"]["ok"] and fused_equal)
    return line


def bench_mla_decode(args):
    """sparse MLA decode alone, batch 32, 128 heads, 32K
    context, top-2048 indices per query from the config-0 generator scaled to
    32K (distinct positions, randomly paged). One call = one layer's decode
    attention; the key list is split so that the launch fills the CUs."""
    import torch

    from nanoengine_amd import _lib, mla_utils, ops, synth

    _lib.load()
    dev = torch.device("cuda:0")
    B, L, H, K = 32, 32768, args.heads, args.topk
    lens = [L] * B
    gen = torch.Generator(device="cpu").manual_seed(args.seed)
    bt, num_pages = synth.make_block_tables(lens, gen, dev)
    kv = synth.make_mla_cache(num_pages, seed=args.seed, device=dev)
    q = synth.make_mla_query(B, H, seed=args.seed, device=dev)
    pos = synth.random_topk_positions(lens, K, seed=args.seed, device=dev)
    idx = mla_utils.topk_indices_to_physical(pos, bt, 64)
    scale = 192 ** -0.5
    splits = ops.sparse_mla_num_splits(B, H, K, dev)
    ws = torch.empty(max(ops.sparse_mla_workspace_bytes(B, H, splits), 1), dtype=torch.uint8, device=dev)
    out = torch.empty(B, H, 512, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(B, H, dtype=torch.float32, device=dev)

    def call():
        ops.sparse_mla_decode(q, kv, idx, scale, out=out, lse=lse, num_splits=splits, workspace=ws)

    for _ in range(max(1, args.warmup)):
        call()
    torch.cuda.synchronize()
    steps = max(1, args.steps)
    # event-timed pass first (it also settles the GPU clock), then the wall loop
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        call()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / steps
    t0 = time.perf_counter()
    for _ in range(steps):
        call()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    # parity: eight tokens spread over the batch against the oracle
    import numpy as np

    import oracle as O
    from oracle import step_check as SC
    o_err, lse_err = 0.0, 0.0
    rows = SC.spread_rows(B, 8)
    for r in rows.tolist():
        sel = idx[r].long()
        kv_sel = kv[sel // 64, sel % 64, 0].cpu().numpy()
        eo, el = O.sparse_mla_decode(q[r:r + 1].float().cpu().numpy(), kv_sel, np.arange(K)[None, :], scale)
        o_err = max(o_err, float(np.abs(out[r].float().cpu().numpy() - eo[0]).max()))
        lse_err = max(lse_err, float(np.abs(lse[r].cpu().numpy() - el[0]).max()))
    parity = {"rows": rows.tolist(), "o_max_abs_err": round(o_err, 6), "lse_max_abs_err": round(lse_err, 6),
              "ok": bool(o_err <= SC.O_ATOL and lse_err <= SC.LSE_ATOL)}
    valid = int((idx >= 0).sum().item())
    nbytes = valid * 656 + B * H * 576 * 2 + B * H * 512 * 2 + B * H * 4 + B * K * 4
    flops = 2.0 * H * (576 + 512) * valid
    gbs = nbytes / (us * 1e-6) / 1e9
    return {
        "metric": METRIC, "value": round(B / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": steps, "warmup": args.warmup, "ms_per_step": round(ms, 4), "us_per_step": round(ms * 1e3, 1),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp8+bf16",
        "data": "synthetic",
        "config": {"workload": "BASELINE config 1: sparse MLA decode alone, one layer", "batch": B,
                   "context_len": L, "index_topk": K, "mla_heads": H, "mla_dims": "576/512", "page_size": 64,
                   "kv_cache": "fp8 656 B/token", "num_splits": splits, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "sparse_mla_kernel (+ split combine)", "bytes_per_launch": nbytes,
                     "avg_launch_us": round(us, 2)},
        "stages": {"sparse_mla_decode": {"us": round(us, 2), "bytes": nbytes, "GBps": round(gbs, 1),
                                         "bf16_mfma_frac": round(flops / (us * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4),
                                         "num_splits": splits}},
        "cpu_baseline": None, "parity": parity,
    }


def decode_line(args, config: int) -> dict | None:
    """BASELINE config 2 (the headline decode step) or 3 (MTP verify): the
    bench line as a dict (None for a --only profiling run)."""
    import torch

    from nanoengine_amd import _lib, synth
    from nanoengine_amd.pipeline import DsaDecodeStep

    _lib.load()
    dev = torch.device("cuda:0")
    B, L, H, K = args.batch, args.ctx, args.heads, args.topk
    n = 1
    if config == 3:
        import numpy as np
        B, n = 64, 2
        rng = np.random.default_rng(args.seed)
        lens = [int(x) for x in np.clip(np.exp(rng.normal(np.log(16384), 1.0, B)), 2048, 131072)]
    else:
        lens = [L] * B
    inp = synth.make_indexer_inputs(lens, next_n=n, seed=args.seed, device=dev)
    num_blocks = int(inp.block_tables.max().item()) + 1
    kv = synth.make_mla_cache(num_blocks, seed=args.seed, device=dev)
    q_mla = synth.make_mla_query(B * n, H, seed=args.seed, device=dev)
    scale = 192 ** -0.5
    max_ctx = inp.block_tables.shape[1] * 64
    step = DsaDecodeStep(B, n, max_ctx, num_heads=H, index_topk=K, device=dev, fused=not args.unfused)
    seq = step.expand_lens(inp.context_lens)   # per query token [B*n]
    bt = inp.block_tables
    pt = bt.repeat_interleave(n, dim=0).contiguous() if n > 1 else bt
    from nanoengine_amd import ops
    torch.cuda.synchronize()

    def run(ev=None):
        # ev: [start, after sample, after filter, after select, after MLA]
        if step.fused:
            ops.indexer_topk(inp.q_fp8.view(B, n, 64, 128), inp.cache, inp.weights, seq.view(B, n), bt, max_ctx, K,
                             step.physical, step.logical, workspace=step.fused_workspace,
                             phase_events=ev[0:4] + [None] if ev is not None else None)
        else:
            if ev is not None:
                ev[0].record()
            ops.indexer_logits(inp.q_fp8.view(B, n, 64, 128), inp.cache, inp.weights, seq.view(B, n), bt,
                               max_ctx, out=step.logits)
            if ev is not None:
                ev[1].record()
                ev[2].record()
            ops.topk_transform(step.logits, seq, pt, step.physical, 64, K, step.logical,
                               workspace=step.topk_workspace)
            if ev is not None:
                ev[3].record()
        ops.sparse_mla_decode(q_mla, kv, step.physical, scale, out=step.out, lse=step.lse,
                              num_splits=step.num_splits, workspace=step.workspace)
        if ev is not None:
            ev[4].record()

    if args.only:
        run()
        torch.cuda.synchronize()
        logits = torch.empty(B * n, max_ctx, dtype=torch.float32, device=dev) if args.only in ("indexer", "topk") else None
        if logits is not None:
            ops.indexer_logits(inp.q_fp8.view(B, n, 64, 128), inp.cache, inp.weights, seq.view(B, n), bt,
                               max_ctx, out=logits)
        for _ in range(args.steps):
            if args.only == "fused":
                ops.indexer_topk(inp.q_fp8.view(B, n, 64, 128), inp.cache, inp.weights, seq.view(B, n), bt,
                                 max_ctx, K, step.physical, step.logical,
                                 workspace=getattr(step, "fused_workspace", None))
            elif args.only == "indexer":
                ops.indexer_logits(inp.q_fp8.view(B, n, 64, 128), inp.cache, inp.weights, seq.view(B, n), bt,
                                   max_ctx, out=logits)
            elif args.only == "topk":
                ops.topk_transform(logits, seq, pt, step.physical, 64, K, step.logical)
            else:
                ops.sparse_mla_decode(q_mla, kv, step.physical, scale, out=step.out, lse=step.lse,
                                      num_splits=step.num_splits, workspace=step.workspace)
        torch.cuda.synchronize()
        print(f"ran {args.steps} launches of {args.only}", flush=True)
        return None

    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    # Per-phase durations with HIP events on the launch stream, in a pass of
    # its own before the wall-timed loop. It runs at least 300 steps (~0.1 s):
    # the GPU clock ramps over the first ~100 steps of load (325 -> 305
    # us/step at config 2), so this pass also hands the wall loop a settled
    # clock, and its averages are taken over its last `steps` steps.
    ev_steps = max(args.steps, 300)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(5)] for _ in range(ev_steps)]
    for e in evs:
        run(e)
    torch.cuda.synchronize()
    ph = [[e[i].elapsed_time(e[i + 1]) * 1e3 for e in evs[-args.steps:]] for i in range(4)]   # us
    med = [sorted(x)[len(x) // 2] for x in ph]
    avg = [sum(x) / len(x) for x in ph]
    idx_total = sum(avg[0:3])
    # timed region: exactly `steps` steps, synchronised on both sides
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps

    total_tokens = sum(lens)
    # the filter pass reads every key page of every sequence (+ q and head weights)
    idx_bytes = total_tokens * 132 + B * n * 64 * 128 + B * n * 64 * 4
    if not step.fused:
        idx_bytes += B * n * max_ctx * 4  # the logits written
    idx_flops = 2.0 * 64 * 128 * int(seq.sum().item())
    valid = int((step.physical >= 0).sum().item())
    mla_bytes = valid * 656 + B * n * H * 576 * 2 + B * n * H * 512 * 2 + B * n * H * 4 + B * n * K * 4
    mla_flops = 2.0 * H * (576 + 512) * valid

    def gbs(b, us):
        return b / (us * 1e-6) / 1e9

    r4 = lambda x: round(x, 4)
    stages = {
        "indexer_topk": {
            "us": round(idx_total, 2), "fused": step.fused,
            "phases_us": {"sample+threshold": round(avg[0], 2), "filter": round(avg[1], 2),
                          "select": round(avg[2], 2)},
            "filter_bytes": idx_bytes, "filter_GBps": round(gbs(idx_bytes, avg[1]), 1),
            "filter_hbm_frac": r4(gbs(idx_bytes, avg[1]) / HBM_PEAK_GBS),
            "filter_fp8_mfma_frac": r4(idx_flops / (avg[1] * 1e-6) / 1e12 / FP8_PEAK_TFLOPS)},
        "sparse_mla_decode": {"us": round(avg[3], 2), "us_median": round(med[3], 2), "bytes": mla_bytes,
                              "GBps": round(gbs(mla_bytes, avg[3]), 1),
                              "hbm_frac": r4(gbs(mla_bytes, avg[3]) / HBM_PEAK_GBS),
                              "bf16_mfma_frac": r4(mla_flops / (avg[3] * 1e-6) / 1e12 / BF16_PEAK_TFLOPS),
                              "num_splits": step.num_splits},
    }
    if not step.fused:
        stages["indexer_topk"] = {"us": round(idx_total, 2), "fused": False,
                                  "phases_us": {"indexer_logits": round(avg[0] + avg[1], 2),
                                                "topk_transform": round(avg[2], 2)},
                                  "indexer_bytes": idx_bytes,
                                  "indexer_GBps": round(gbs(idx_bytes, avg[0] + avg[1]), 1)}
    filt_us = avg[1] if step.fused else avg[0] + avg[1]
    achieved = gbs(idx_bytes, filt_us)
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": r4(achieved / HBM_PEAK_GBS), "traffic": pmc_traffic() if step.fused and config == 2 else None,
                "kernel": "indexer_filter_kernel<1> (persistent filter pass)" if step.fused else "indexer_logits_kernel<1, kIdxStore>",
                "bytes_per_launch": idx_bytes, "avg_launch_us": round(filt_us, 2)}

    stages["outside_step"] = prologue_stages(B * n, dev, args.seed)

    cpu, parity = None, None
    if not args.no_cpu_baseline:
        # config 2 times the oracle on a sample of sequences (the CPU baseline)
        # and checks those rows; config 3 checks 12 query rows, untimed
        cpu, parity = cpu_baseline(inp, kv, q_mla, seq.cpu().tolist(), n,
                                   min(args.cpu_sample, B) if config == 2 else 12, scale, K, step,
                                   timed=config == 2)

    return {
        "metric": METRIC, "value": round(B * n / (ms_per_step * 1e-3), 1), "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
        "us_per_step": round(ms_per_step * 1e3, 1), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp8+bf16", "data": "synthetic",
        "config": {"workload": ("BASELINE config 2: full DSA decode step, one layer" if n == 1 else
                                "BASELINE config 3: MTP verify step (next_n=2, causal draft lengths), one layer"),
                   "batch": B, "next_n": n, "context_len": L if n == 1 else
                   {"lognormal_median": 16384, "clip": [2048, 131072], "mean": round(sum(lens) / B)},
                   "index_topk": K, "indexer_heads": 64,
                   "indexer_head_dim": 128, "mla_heads": H, "mla_dims": "576/512", "page_size": 64,
                   "kv_cache": "fp8 656 B/token (block stride 65 rows)", "indexer_cache": "fp8 132 B/token",
                   "parallelism": "single GPU"},
        "untimed_before_wall_loop": {"warmup_steps": args.warmup, "stage_event_steps": ev_steps},
        "roofline": roofline, "stages": stages, "cpu_baseline": cpu, "parity": parity,
    }



def _summary(line: dict) -> dict:
    """The part of another config's bench line that the headline line carries."""
    keep = ("value", "unit", "ms_per_step", "us_per_step", "config", "roofline", "stages", "parity")
    out = {k: line[k] for k in keep if k in line}
    if line.get("cpu_baseline"):
        out["cpu_baseline"] = line["cpu_baseline"]
    return out


def _free_gpu():
    import gc

    import torch
    gc.collect()
    torch.cuda.empty_cache()


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}); the DSA decode path is "
              "rank-local and this build measures one GPU's share", file=sys.stderr)
        sys.exit(2)
    if args.copy_calib:
        copy_calib()
        return
    if args.micro:
        micro()
        return
    if args.config == 4:
        line = bench_prefill(args)
    elif args.config == 1:
        line = bench_mla_decode(args)
    else:
        line = decode_line(args, args.config)
        if args.config == 2 and not args.headline_only and not args.only:
            # the other BASELINE configs, each with its stage figures and its
            # parity check, as extra keys of the one line; the decode configs
            # (steps of ~0.04 and ~0.17 ms) time at least 200 steps, the
            # prefill chunk (~14 ms) at least 20, each after at least 20
            # warm-up steps
            _free_gpu()
            import copy
            line["other_configs"] = {}
            for cfg, fn, min_steps in ((1, bench_mla_decode, 200), (3, lambda a: decode_line(a, 3), 200),
                                       (4, bench_prefill, 20)):
                other = copy.copy(args)
                other.warmup, other.steps = max(args.warmup, 20), max(args.steps, min_steps)
                print(f"bench: config {cfg}", file=sys.stderr, flush=True)
                line["other_configs"][f"config{cfg}"] = _summary(fn(other))
                _free_gpu()
            # None: some config ran without its check (--no-cpu-baseline)
            checked = [v["parity"]["ok"] for v in line["other_configs"].values() if v.get("parity") is not None]
            line["other_configs_parity_ok"] = all(checked) if len(checked) == 3 else (False if not all(checked) else None)
    if line is None:   # a --only profiling run
        return
    print(json.dumps(line), flush=True)
    failed = [] if (line.get("parity") or {"ok": True})["ok"] else ["headline"]
    failed += [k for k, v in line.get("other_configs", {}).items()
               if v.get("parity") is not None and not v["parity"]["ok"]]
    if failed:
        print(f"PARITY FAILURE in {failed}: the GPU outputs do not match the oracle", file=sys.stderr)
        sys.exit(1)


if __name__ == "__main__":
    main()
