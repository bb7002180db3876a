// fp8 lightning-indexer logits over the paged indexer cache, for gfx950.
//
//   logits[b*n+j, t] = sum_h w[b*n+j, h] * relu(q[b,j,h,:] . k[t,:]) * scale[t]
//
// One wave owns one 64-token page at a time. The page's 64x128 fp8 keys are
// the B operand of v_mfma_scale_f32_16x16x128_f8f6f4 (fp8 x fp8 -> fp32, unit
// scales), 32 contiguous bytes of one token per lane, while the query heads
// (A operand, 16 heads per tile) stay resident in registers for the whole
// workgroup lifetime. indexer_logits_kernel loads the keys from HBM straight
// into that layout; the persistent filter pass loads whole 128-byte rows per
// instruction and reorders them through a per-wave LDS tile. Each page
// costs 16 MFMAs per query token (4 token tiles x 4 head tiles); the ReLU and
// the head weights are applied on the fp32 accumulators, and a 3-shuffle
// butterfly finishes the head sum so that lane l ends up owning token l of the
// page: the logits row segment and the per-token scales are then one
// coalesced 256-byte load/store each. Rotating register page buffers keep
// pages in flight while one is multiplied. The page primitives live in
// indexer_page.h.
//
// Launches: indexer_logits_kernel (one workgroup per 24 pages of a row) writes
// the logits (the fp8_paged_mqa_logits operator), samples 16 pages per row for
// the fused path's score threshold, or filters (batches above the persistent
// kernel's limit); indexer_filter_kernel is the fused path's persistent filter
// pass (one contiguous page range per wave, per-wave candidate staging).
#include <algorithm>
#include <type_traits>

#include "dsa_common.h"
#include "indexer_page.h"
#include "../../include/dsa_amd.h"

namespace dsa {

constexpr int kIdxThreads = 256;
constexpr int kIdxWaves = kIdxThreads / 64;
constexpr int kIdxPagesPerWave = 6;

// What a launch does with the logits of a page.
enum IdxMode : int {
  kIdxStore = 0,   // logits[row, t]
  kIdxSample = 1,  // every page_step-th page, one workgroup per row: the logits stay in LDS and
                   // give the row's score threshold ws[row].t_key (lists reset)
  kIdxFilter = 2,  // no logits: (key, t) of every token with key >= ws[row].t_key is appended
                   // to the row's candidate list (staged in LDS, one global atomic per WG)
};

struct IdxOut {
  float* logits;
  int64_t logits_stride;
  int page_step;            // kIdxSample: sampled page stride
  RowWs* ws;                // kIdxSample: thresholds out; kIdxFilter: thresholds in, lists out
  int top_k;                // kIdxSample
};

constexpr int kIdxWgTokens = kIdxWaves * kIdxPagesPerWave * kIdxPageTokens;  // 1536

struct IdxStoreLds {  // store mode: the waves' page tiles (rows_to_operands)
  __attribute__((aligned(16))) uint8_t tr[kIdxWaves][kIdxTrBytes];
};

constexpr int kSamplePages = 16;  // sampled pages per row, one workgroup
// The sample pass is latency-bound (one workgroup per row): its pages are
// spread one per wave (two per wave for two query tokens, which need twice the
// query registers).
template <int NQ>
constexpr int sample_threads() { return NQ == 1 ? 1024 : 512; }
template <int NQ, int MODE>
constexpr int idx_threads() { return MODE == kIdxSample ? sample_threads<NQ>() : kIdxThreads; }
constexpr int kSampleBinBits = 10;                              // threshold histogram of the sample
constexpr int kSampleBins = 1 << kSampleBinBits;
struct IdxSampleLds {
  uint8_t q[2][kIdxHeads * kIdxHeadDim];  // the row's query (staged once for all waves)
  float w[2][kIdxHeads];
  float logit[2][kSamplePages * kIdxPageTokens];
  uint32_t hist[kSampleBins];
  uint32_t wave_sum[2 * 16];
  uint32_t tb, above, eq;
};

struct IdxStage {  // per-WG LDS staging of kIdxFilter candidates, per query token
  uint32_t count[2];
  uint32_t base[2];
  uint32_t key[2][kIdxWgTokens];
  uint32_t pos[2][kIdxWgTokens];
  __attribute__((aligned(16))) uint8_t tr[kIdxWaves][kIdxTrBytes];  // the waves' page tiles
};

template <int NQ, int MODE>
__device__ __forceinline__ void compute_page(const PageRegs& cur, int p, int vp, int lane, const v8i (&qa)[NQ][4],
                                             const float (&w)[NQ][4][4], const int (&L)[NQ],
                                             const uint32_t (&tk)[NQ], int64_t max_ctx, const IdxOut& o,
                                             void* lds, int b) {
  IdxStage* stage = static_cast<IdxStage*>(lds);
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    const float v = page_head_sum<NQ>(cur, j, lane, qa, w);
    const int t = p * kIdxPageTokens + lane;
    const float logit = t < L[j] ? v * cur.scale : -__builtin_inff();
    if (MODE == kIdxFilter) {
      const bool pred = t < L[j] && order_key(logit) >= tk[j];
      const uint64_t m = __ballot(pred);
      if (m) {
        const int leader = __builtin_ctzll(m);
        uint32_t base = 0;
        if (lane == leader) base = atomicAdd(&stage->count[j], (uint32_t)__popcll(m));
        base = __shfl(base, leader, 64);
        if (pred) {
          const uint32_t slot = base + (uint32_t)__popcll(m & ((1ull << lane) - 1ull));
          stage->key[j][slot] = order_key(logit);
          stage->pos[j][slot] = (uint32_t)t;
        }
      }
    } else if (MODE == kIdxSample) {
      static_cast<IdxSampleLds*>(lds)->logit[j][vp * kIdxPageTokens + lane] = logit;
    } else {
      if (t < max_ctx) {
        float* dst = o.logits + (int64_t)(b * NQ + j) * o.logits_stride;
        // streaming store: the logits are consumed by a later kernel, not reused here
        __builtin_nontemporal_store(logit, dst + t);
      }
    }
  }
}

// Store and filter: 4 waves, two per SIMD: three 33-VGPR page buffers, the
// resident query tiles and head weights take ~180 VGPRs for one query token.
// Sample: one workgroup of 16 (8) waves per row.
template <int NQ, int MODE>
__global__ void __launch_bounds__((idx_threads<NQ, MODE>())) __attribute__((amdgpu_waves_per_eu(2)))
indexer_logits_kernel(const uint8_t* __restrict__ q, const uint8_t* __restrict__ kv,
                      const float* __restrict__ weights, const int32_t* __restrict__ ctx_lens,
                      const int32_t* __restrict__ block_tables, int64_t bt_stride, int64_t max_ctx,
                      const IdxOut o) {
  // LDS: candidate staging (filter) or the sampled logits (sample)
  __shared__ __align__(16) typename std::conditional<
      MODE == kIdxFilter, IdxStage,
      typename std::conditional<MODE == kIdxSample, IdxSampleLds, IdxStoreLds>::type>::type lds_mem;
  IdxStage* stage = reinterpret_cast<IdxStage*>(&lds_mem);
  constexpr int NT = idx_threads<NQ, MODE>();
  constexpr int NW = NT / 64;
  constexpr int PPW = MODE == kIdxSample ? kSamplePages / NW : kIdxPagesPerWave;
  static_assert(MODE != kIdxSample || PPW * NW == kSamplePages, "sample geometry");
  const int b = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int step = MODE == kIdxSample ? o.page_step : 1;
  const int vp_begin = blockIdx.x * (NW * PPW) + wave;
  // All of the wave's block-table entries in one load, issued before the
  // context lengths arrive: every table row holds ceil(max_ctx / 64) entries,
  // and entries past a row's context are loaded but never used.
  const int max_pages = (int)((max_ctx + kIdxPageTokens - 1) / kIdxPageTokens);
  const int spec_page = (vp_begin + NW * lane) * step;
  const int my_page =
      (lane < PPW && spec_page < max_pages) ? block_tables[(int64_t)b * bt_stride + spec_page] : 0;

  int L[NQ];
  uint32_t tk[NQ];
  int Lmax = 0;
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    L[j] = ctx_lens[b * NQ + j];
    Lmax = max(Lmax, L[j]);
    tk[j] = MODE == kIdxFilter ? o.ws[b * NQ + j].t_key : 0u;
  }
  // real pages of the row, and the virtual pages this launch walks (every
  // step-th real page)
  const int npages = (int)((min((int64_t)Lmax, max_ctx) + kIdxPageTokens - 1) / kIdxPageTokens);
  const int nvp = (npages + step - 1) / step;
  if (MODE != kIdxSample && blockIdx.x * (NW * PPW) >= nvp) return;

  if (MODE == kIdxFilter) {
    if (threadIdx.x < NQ) stage->count[threadIdx.x] = 0u;
    __syncthreads();
  }

  // Query heads as MFMA A operands: tile (j, ht) row i = head ht*16 + i.
  v8i qa[NQ][4];
  float w[NQ][4][4];
  auto load_q = [&](const uint8_t* qrows, const float* wrows) {
#pragma unroll
    for (int j = 0; j < NQ; ++j)
      load_query(qrows + j * kIdxHeads * kIdxHeadDim, wrows + j * kIdxHeads, lane, qa[j], w[j]);
  };
  if constexpr (MODE != kIdxSample)
    load_q(q + ((int64_t)b * NQ * kIdxHeads) * kIdxHeadDim, weights + (int64_t)b * NQ * kIdxHeads);

  // Three page buffers rotate so that two pages are in flight while one is
  // being multiplied; the wave's virtual pages are vp_begin + NW*i.
  [[maybe_unused]] PageRegs buf0, buf1, buf2;
  auto valid = [&](int i) { return i < PPW && vp_begin + NW * i < nvp; };
  auto page_ptr = [&](int i) {
    return kv + (int64_t)__builtin_amdgcn_readlane(my_page, i) * kIdxPageBytes;
  };
  auto compute = [&](const PageRegs& pr, int i) {
    const int vp = vp_begin + NW * i;
    compute_page<NQ, MODE>(pr, vp * step, vp, lane, qa, w, L, tk, max_ctx, o, &lds_mem, b);
  };
  if constexpr (MODE == kIdxSample) {
    // A latency-bound pass (one workgroup per row). The row's query and head
    // weights are read once per workgroup and staged in LDS, not once per
    // wave: 16 copies of the query would double the pass's bytes. They are
    // requested before the pages, so that waiting for them (loads complete
    // in order) does not wait for the pages too; then all of a wave's pages
    // go in flight at once, and the query reaches LDS while they load.
    constexpr int kQBytes = NQ * kIdxHeads * kIdxHeadDim;
    constexpr int kQPer = (kQBytes + 16 * NT - 1) / (16 * NT);
    const uint8_t* qsrc = q + ((int64_t)b * NQ * kIdxHeads) * kIdxHeadDim;
    v4i qv[kQPer];
#pragma unroll
    for (int u = 0; u < kQPer; ++u) {
      const int e = 16 * ((int)threadIdx.x + u * NT);
      if (e < kQBytes) qv[u] = *reinterpret_cast<const v4i*>(qsrc + e);
    }
    const float wv = threadIdx.x < NQ * kIdxHeads ? weights[(int64_t)b * NQ * kIdxHeads + threadIdx.x] : 0.f;
    PageRegs pb[PPW];
#pragma unroll
    for (int i = 0; i < PPW; ++i)
      if (valid(i)) load_page(pb[i], page_ptr(i), lane);
    IdxSampleLds& sq = *reinterpret_cast<IdxSampleLds*>(&lds_mem);
#pragma unroll
    for (int u = 0; u < kQPer; ++u) {
      const int e = 16 * ((int)threadIdx.x + u * NT);
      if (e < kQBytes) *reinterpret_cast<v4i*>(&sq.q[0][0] + e) = qv[u];
    }
    if (threadIdx.x < NQ * kIdxHeads) (&sq.w[0][0])[threadIdx.x] = wv;
    __syncthreads();
    load_q(&sq.q[0][0], &sq.w[0][0]);
#pragma unroll
    for (int i = 0; i < PPW; ++i)
      if (valid(i)) compute(pb[i], i);
  } else {
    // whole-row loads, reordered in the wave's LDS tile before each page's MFMAs
    uint8_t* tr = MODE == kIdxFilter ? stage->tr[wave] : reinterpret_cast<IdxStoreLds*>(&lds_mem)->tr[wave];
    auto compute_rows = [&](PageRegs& pr, int i) {
      rows_to_operands(pr, tr, lane);
      compute(pr, i);
    };
    if (valid(0)) load_page_rows(buf0, page_ptr(0), lane);
    if (valid(1)) load_page_rows(buf1, page_ptr(1), lane);
#pragma unroll
    for (int i = 0; i < PPW; i += 3) {
      if (valid(i + 2)) load_page_rows(buf2, page_ptr(i + 2), lane);
      if (valid(i)) compute_rows(buf0, i);
      if (valid(i + 3)) load_page_rows(buf0, page_ptr(i + 3), lane);
      if (valid(i + 1)) compute_rows(buf1, i + 1);
      if (valid(i + 4)) load_page_rows(buf1, page_ptr(i + 4), lane);
      if (valid(i + 2)) compute_rows(buf2, i + 2);
    }
  }

  if (MODE == kIdxSample) {
    // The row's score threshold from its sampled logits (one workgroup holds
    // them all in LDS): a key at or below the rank-r key of the sample,
    // r = f + 4 sqrt(f) + 8 with f = k * nsample / len, so that about k + margin
    // tokens of the whole row are expected at or above it. Two histogram levels
    // of 1024 bins over the sample's [min, max] key range (the second inside
    // the first's bin holding rank r): the threshold is the lower edge of the
    // final bin holding rank r. Any key at or below the rank-r key is a valid
    // threshold; resolution only trims the candidate list. The row's
    // candidate list is reset here.
    IdxSampleLds& sl = *reinterpret_cast<IdxSampleLds*>(&lds_mem);
    const int tid = threadIdx.x;
    const int span = step * kIdxPageTokens;
    __syncthreads();  // the sampled logits are in LDS
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      RowWs& rw = o.ws[b * NQ + j];
      const float* smp = sl.logit[j];
      const int len = (int)min((int64_t)max(L[j], 0), max_ctx);
      const int nv = (len + span - 1) / span;
      uint32_t nsample = 0;
      for (int v = 0; v < nv; ++v) nsample += (uint32_t)max(0, min(len - v * span, kIdxPageTokens));
      const float fk = (float)nsample / (float)max(len, 1) * (float)o.top_k;
      const uint32_t r = (uint32_t)(fk + 4.f * sqrtf(fk) + 8.f);
      uint32_t t_key = 0u;  // 0: every token is a candidate
      if (len > o.top_k && r < nsample) {
        // this thread's sampled keys (nv * 64 <= 1024 = 4 per thread)
        constexpr int kPer = kSamplePages * kIdxPageTokens / NT;
        uint32_t key[kPer];
        uint32_t kmin = 0xffffffffu, kmax = 0u;
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
          const int e = tid + u * NT;
          const bool ok = e < nv * kIdxPageTokens && (e >> 6) * span + (e & 63) < len;
          key[u] = ok ? order_key(smp[e]) : 0u;
          if (ok) {
            kmin = min(kmin, key[u]);
            kmax = max(kmax, key[u]);
          }
        }
        for (int i = tid; i < kSampleBins; i += NT) sl.hist[i] = 0u;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
          kmin = min(kmin, (uint32_t)__shfl_xor(kmin, off, 64));
          kmax = max(kmax, (uint32_t)__shfl_xor(kmax, off, 64));
        }
        if (lane == 0) {
          sl.wave_sum[wave] = kmin;
          sl.wave_sum[NW + wave] = kmax;
        }
        __syncthreads();
#pragma unroll
        for (int w2 = 0; w2 < NW; ++w2) {
          kmin = min(kmin, sl.wave_sum[w2]);
          kmax = max(kmax, sl.wave_sum[NW + w2]);
        }
        const uint32_t range = kmax - kmin;
        const int shift = max(0, 32 - (int)__clz(range) - kSampleBinBits);
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
          const int e = tid + u * NT;
          if (e < nv * kIdxPageTokens && (e >> 6) * span + (e & 63) < len)
            atomicAdd(&sl.hist[(key[u] - kmin) >> shift], 1u);
        }
        __syncthreads();
        find_threshold<NT>(sl.hist, sl.wave_sum, kSampleBins, r, &sl.tb, &sl.above, &sl.eq);
        const uint32_t tb0 = sl.tb;
        t_key = kmin + (tb0 << shift);
        if (shift > 0) {
          // second level inside bin tb0: 10 more bits of the range
          const uint32_t rem0 = r - sl.above;
          const int shift2 = max(0, shift - kSampleBinBits);
          __syncthreads();
          for (int i = tid; i < kSampleBins; i += NT) sl.hist[i] = 0u;
          __syncthreads();
#pragma unroll
          for (int u = 0; u < kPer; ++u) {
            const int e = tid + u * NT;
            const uint32_t dk = key[u] - kmin;
            if (e < nv * kIdxPageTokens && (e >> 6) * span + (e & 63) < len && (dk >> shift) == tb0)
              atomicAdd(&sl.hist[(dk >> shift2) & (kSampleBins - 1)], 1u);
          }
          __syncthreads();
          find_threshold<NT>(sl.hist, sl.wave_sum, kSampleBins, rem0, &sl.tb, &sl.above, &sl.eq);
          t_key += sl.tb << shift2;
        }
      }
      if (tid == 0) {
        rw.t_key = t_key;
        rw.count = 0u;
        rw.failed = 0u;
      }
      __syncthreads();
    }
  }

  if (MODE == kIdxFilter) {
    // one global atomic per workgroup and query token; entries past the
    // list's capacity are dropped and the count tells the finishing kernel
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      const uint32_t n = stage->count[j];
      RowWs& rw = o.ws[b * NQ + j];
      if (threadIdx.x == 0) stage->base[j] = n ? atomicAdd(&rw.count, n) : 0u;
      __syncthreads();
      const uint32_t base = stage->base[j];
      for (uint32_t e = threadIdx.x; e < n; e += NT)
        if (base + e < (uint32_t)kListCap) {
          rw.key[base + e] = stage->key[j][e];
          rw.pos[base + e] = stage->pos[j][e];
        }
    }
  }
}

// ---------------------------------------------------------------- persistent filter pass
// The filter pass as a persistent kernel: a fixed grid of waves (two
// workgroups per CU) where each wave streams one contiguous, balanced range
// of the flattened (batch entry, page) space through its rotating page
// buffers, with no barriers and no per-workgroup start-up or drain in the
// loop. Pages are read as whole rows (load_page_rows) and reordered into the
// MFMA operand layout in the wave's LDS tile (rows_to_operands). Candidates
// are staged per wave in LDS (wave-uniform counters, no LDS atomics) and
// flushed to the row's list with one global atomic when the batch entry
// changes, when the stage could overflow, and at the end.
constexpr int kFiltStageCap = 384;   // staged candidates per wave and query token
constexpr int kFiltWindow = 64;      // block-table entries a wave holds (one per lane)
constexpr int kFiltAdvance = 60;     // pages per window refill (a multiple of the 3- and 4-buffer rotations)
constexpr int kFiltMaxBatch = 4096;  // batch entries whose page prefix fits in LDS beside a second workgroup's
struct FiltWaveStage {
  uint32_t key[2][kFiltStageCap];
  uint32_t pos[2][kFiltStageCap];
  __attribute__((aligned(16))) uint8_t tr[kIdxTrBytes];  // the wave's page tile (rows_to_operands)
};
constexpr size_t filt_smem_bytes(int batch) {
  return sizeof(FiltWaveStage) * kIdxWaves + ((size_t)batch + 1 + kIdxWaves) * sizeof(int32_t);
}
static_assert(2 * filt_smem_bytes(kFiltMaxBatch) <= 160 * 1024, "two filter workgroups per CU at the largest batch");

template <int NQ>
__global__ void __launch_bounds__(kIdxThreads) __attribute__((amdgpu_waves_per_eu(2)))
indexer_filter_kernel(const uint8_t* __restrict__ q, const uint8_t* __restrict__ kv,
                      const float* __restrict__ weights, const int32_t* __restrict__ ctx_lens,
                      const int32_t* __restrict__ block_tables, int64_t bt_stride, int64_t max_ctx, int batch,
                      RowWs* __restrict__ ws) {
  extern __shared__ __align__(16) uint8_t fl_smem[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  FiltWaveStage& st = reinterpret_cast<FiltWaveStage*>(fl_smem)[wave];
  int32_t* prefix = reinterpret_cast<int32_t*>(fl_smem + sizeof(FiltWaveStage) * kIdxWaves);  // [batch + 1]
  int32_t* wsum = prefix + batch + 1;                                                         // [kIdxWaves]

  // 1. pages of each batch entry (the longest of its query tokens, capped at
  //    max_ctx) -> exclusive prefix in LDS, in tiles of kIdxThreads entries
  int32_t carry = 0;
  for (int base = 0; base < batch; base += kIdxThreads) {
    const int i = base + (int)threadIdx.x;
    int np = 0;
    if (i < batch) {
      int lm = 0;
#pragma unroll
      for (int j = 0; j < NQ; ++j) lm = max(lm, ctx_lens[i * NQ + j]);
      np = (int)((min((int64_t)lm, max_ctx) + kIdxPageTokens - 1) / kIdxPageTokens);
    }
    int v = np;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int n = __shfl_up(v, off, 64);
      if (lane >= off) v += n;
    }
    if (lane == 63) wsum[wave] = v;
    __syncthreads();
    int before = carry, tile = 0;
#pragma unroll
    for (int w2 = 0; w2 < kIdxWaves; ++w2) {
      if (w2 < wave) before += wsum[w2];
      tile += wsum[w2];
    }
    if (i < batch) prefix[i] = before + v - np;
    carry += tile;
    __syncthreads();
  }
  if (threadIdx.x == 0) prefix[batch] = carry;
  __syncthreads();
  const int64_t total = carry;

  // 2. this wave's range of the flattened pages
  const int64_t nwaves = (int64_t)gridDim.x * kIdxWaves;
  const int64_t gw = (int64_t)blockIdx.x * kIdxWaves + wave;
  const int64_t p0 = total * gw / nwaves, p1 = total * (gw + 1) / nwaves;
  const int n = (int)(p1 - p0);
  if (n <= 0) return;

  // block-table window: lane l holds page p0 + wb + l as (batch entry, table entry)
  int wb = 0, win_b = 0, win_page = 0;
  auto refill = [&](int from) {
    const int64_t p = p0 + from + lane;
    int bl = 0, page = 0;
    if (p < p1) {
      // last batch entry with prefix <= p
      int lo = 0, hi = batch - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (prefix[mid] <= p) lo = mid; else hi = mid - 1;
      }
      bl = lo;
      page = block_tables[(int64_t)bl * bt_stride + (int)(p - prefix[bl])];
    }
    win_b = bl;
    win_page = page;
  };
  refill(0);

  // state of the current batch entry
  int cur_b = -1;
  v8i qa[NQ][4];
  float w[NQ][4][4];
  int L[NQ];
  uint32_t tk[NQ];
  int cnt[NQ];
#pragma unroll
  for (int j = 0; j < NQ; ++j) cnt[j] = 0;

  auto flush = [&](int j) {
    const int c = cnt[j];
    if (c == 0) return;
    RowWs& rw = ws[cur_b * NQ + j];
    uint32_t base = 0;
    if (lane == 0) base = atomicAdd(&rw.count, (uint32_t)c);
    base = __shfl(base, 0, 64);
    for (int e = lane; e < c; e += 64)
      if (base + (uint32_t)e < (uint32_t)kListCap) {
        rw.key[base + e] = st.key[j][e];
        rw.pos[base + e] = st.pos[j][e];
      }
    cnt[j] = 0;
  };
  auto enter = [&](int b) {
#pragma unroll
    for (int j = 0; j < NQ; ++j) flush(j);
    cur_b = b;
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      const uint8_t* qb = q + ((int64_t)(b * NQ + j) * kIdxHeads) * kIdxHeadDim;
      const float* wq = weights + (int64_t)(b * NQ + j) * kIdxHeads;
#pragma unroll
      for (int ht = 0; ht < 4; ++ht) {
        qa[j][ht] = load32B(qb + (ht * 16 + (lane & 15)) * kIdxHeadDim + (lane >> 4) * 32);
#pragma unroll
        for (int r = 0; r < 4; ++r) w[j][ht][r] = wq[ht * 16 + (lane >> 4) * 4 + r];
      }
      L[j] = (int)min((int64_t)ctx_lens[b * NQ + j], max_ctx);
      tk[j] = ws[b * NQ + j].t_key;
    }
  };

  auto page_ptr = [&](int k) {
    return kv + (int64_t)__builtin_amdgcn_readlane(win_page, k - wb) * kIdxPageBytes;
  };
  auto compute = [&](PageRegs& pr, int k) {
    rows_to_operands(pr, st.tr, lane);
    const int b = __builtin_amdgcn_readlane(win_b, k - wb);
    if (b != cur_b) enter(b);
    const int page = (int)(p0 + k - prefix[b]);
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      if (cnt[j] > kFiltStageCap - kIdxPageTokens) flush(j);
      const float v = page_head_sum<NQ>(pr, j, lane, qa, w);
      const int t = page * kIdxPageTokens + lane;
      const uint32_t key = order_key(v * pr.scale);
      const bool pred = t < L[j] && key >= tk[j];
      const uint64_t m = __ballot(pred);
      if (pred) {
        const int slot = cnt[j] + (int)__popcll(m & ((1ull << lane) - 1ull));
        st.key[j][slot] = key;
        st.pos[j][slot] = (uint32_t)t;
      }
      cnt[j] += (int)__popcll(m);
    }
  };

  // NB rotating page buffers, NB - 1 pages in flight while one is multiplied
  constexpr int NB = NQ == 1 ? 4 : 3;
  static_assert(kFiltAdvance % NB == 0 && kFiltAdvance + NB - 1 < kFiltWindow, "window refill geometry");
  PageRegs buf[NB];
#pragma unroll
  for (int u = 0; u < NB - 1; ++u)
    if (u < n) load_page_rows(buf[u], page_ptr(u), lane);
  for (int k = 0; k < n; k += NB) {
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      if (k + u + NB - 1 < n) load_page_rows(buf[(u + NB - 1) % NB], page_ptr(k + u + NB - 1), lane);
      if (k + u < n) compute(buf[u], k + u);
    }
    if (k + NB - wb == kFiltAdvance) {
      // the NB - 1 pages loaded ahead came from this window's last used lanes
      wb += kFiltAdvance;
      refill(wb);
    }
  }
#pragma unroll
  for (int j = 0; j < NQ; ++j) flush(j);
}

static int filter_grid() {
  static int grid = 0;
  if (grid == 0) {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
    grid = 2 * cus;
  }
  return grid;
}

// The persistent filter pass; false when the batch does not fit its LDS prefix.
static bool launch_filter_persistent(const uint8_t* q, const uint8_t* kv, const float* weights,
                                     const int32_t* ctx_lens, const int32_t* bt, int64_t bt_stride, int batch,
                                     int next_n, int64_t max_ctx, RowWs* ws, hipStream_t stream) {
  if (batch > kFiltMaxBatch) return false;
  const size_t smem = filt_smem_bytes(batch);
  static bool attr_set = false;
  if (!attr_set) {
    const int max_smem = (int)filt_smem_bytes(kFiltMaxBatch);
    if (hipFuncSetAttribute((const void*)indexer_filter_kernel<1>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            max_smem) != hipSuccess ||
        hipFuncSetAttribute((const void*)indexer_filter_kernel<2>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            max_smem) != hipSuccess)
      return false;
    attr_set = true;
  }
  const dim3 grid((unsigned)filter_grid());
  if (next_n == 1)
    hipLaunchKernelGGL(indexer_filter_kernel<1>, grid, dim3(kIdxThreads), smem, stream, q, kv, weights, ctx_lens, bt,
                       bt_stride, max_ctx, batch, ws);
  else
    hipLaunchKernelGGL(indexer_filter_kernel<2>, grid, dim3(kIdxThreads), smem, stream, q, kv, weights, ctx_lens, bt,
                       bt_stride, max_ctx, batch, ws);
  return true;
}

template <int MODE>
void launch_indexer(const uint8_t* q, const uint8_t* kv, const float* weights, const int32_t* ctx_lens,
                    const int32_t* bt, int64_t bt_stride, int batch, int next_n, int64_t max_ctx, int64_t vpages,
                    const IdxOut& o, hipStream_t stream) {
  const int64_t per_block = MODE == kIdxSample ? kSamplePages : kIdxWaves * kIdxPagesPerWave;
  const dim3 grid((unsigned)((vpages + per_block - 1) / per_block), (unsigned)batch);
  if (next_n == 1)
    hipLaunchKernelGGL((indexer_logits_kernel<1, MODE>), grid, dim3(idx_threads<1, MODE>()), 0, stream, q, kv, weights, ctx_lens,
                       bt, bt_stride, max_ctx, o);
  else
    hipLaunchKernelGGL((indexer_logits_kernel<2, MODE>), grid, dim3(idx_threads<2, MODE>()), 0, stream, q, kv, weights, ctx_lens,
                       bt, bt_stride, max_ctx, o);
}

}  // namespace dsa

extern "C" int dsa_indexer_logits(const uint8_t* q_fp8, const uint8_t* kv_cache, const float* weights,
                                  const int32_t* context_lens, const int32_t* block_tables,
                                  int64_t block_table_stride, int batch, int next_n, int num_heads,
                                  int head_dim, int page_size, int64_t max_context_len, float* logits,
                                  int64_t logits_stride, void* stream) {
  using namespace dsa;
  if (num_heads != kIdxHeads || head_dim != kIdxHeadDim)
    return set_error(kUnsupported, "indexer: num_heads=%d head_dim=%d unsupported (need 64, 128)",
                     num_heads, head_dim);
  if (page_size != kIdxPageTokens)
    return set_error(kUnsupported, "indexer: page_size=%d unsupported (need 64)", page_size);
  if (next_n != 1 && next_n != 2)
    return set_error(kUnsupported, "indexer: next_n=%d unsupported (1 or 2)", next_n);
  if (batch < 0 || max_context_len < 0 || logits_stride < max_context_len)
    return set_error(kInvalidArgument, "indexer: bad sizes");
  if (batch == 0 || max_context_len == 0) return kOk;
  if (!q_fp8 || !kv_cache || !weights || !context_lens || !block_tables || !logits)
    return set_error(kInvalidArgument, "indexer: null pointer");
  if ((reinterpret_cast<uintptr_t>(q_fp8) | reinterpret_cast<uintptr_t>(kv_cache)) & 15)
    return set_error(kInvalidArgument, "indexer: q and kv_cache must be 16-byte aligned");
  const int64_t max_pages = (max_context_len + kIdxPageTokens - 1) / kIdxPageTokens;
  IdxOut o{logits, logits_stride, 1, nullptr, 0};
  launch_indexer<kIdxStore>(q_fp8, kv_cache, weights, context_lens, block_tables, block_table_stride, batch, next_n,
                            max_context_len, max_pages, o, (hipStream_t)stream);
  return check_launch("dsa_indexer_logits");
}

// ---------------------------------------------------------------- fused indexer + top-k
namespace dsa {
// Page step of the threshold sample: every step-th page, at most 16 pages (1024
// tokens) per row, so one workgroup holds a row's sample.
static inline int sample_step(int64_t max_pages) {
  return (int)std::max<int64_t>(1, (max_pages + kSamplePages - 1) / kSamplePages);
}

struct FusedWs {
  RowWs* ws;
  float* logits;  // full logits, written only for rows the list select redoes
  int64_t logits_stride;
  size_t bytes;
};

static inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static FusedWs fused_layout(void* base, int rows, int64_t max_ctx) {
  FusedWs f;
  f.logits_stride = (max_ctx + 3) & ~(int64_t)3;
  const size_t ws_b = align256((size_t)rows * sizeof(RowWs));
  const size_t logits_b = align256((size_t)rows * f.logits_stride * sizeof(float));
  uint8_t* p = static_cast<uint8_t*>(base);
  f.ws = reinterpret_cast<RowWs*>(p);
  f.logits = reinterpret_cast<float*>(p + ws_b);
  f.bytes = ws_b + logits_b;
  return f;
}
}  // namespace dsa

extern "C" size_t dsa_indexer_topk_workspace_bytes(int batch, int next_n, int64_t max_context_len) {
  if (batch <= 0 || next_n <= 0 || max_context_len <= 0) return 0;
  return dsa::fused_layout(nullptr, batch * next_n, max_context_len).bytes;
}

extern "C" int dsa_indexer_topk(const uint8_t* q_fp8, const uint8_t* kv_cache, const float* weights,
                                const int32_t* context_lens, const int32_t* block_tables,
                                int64_t block_table_stride, int batch, int next_n, int num_heads, int head_dim,
                                int page_size, int64_t max_context_len, int top_k, int32_t* out_physical,
                                int32_t* out_logical, void* workspace, size_t workspace_bytes, void* stream,
                                void* const* phase_events) {
  using namespace dsa;
  if (num_heads != kIdxHeads || head_dim != kIdxHeadDim)
    return set_error(kUnsupported, "indexer_topk: num_heads=%d head_dim=%d unsupported (need 64, 128)",
                     num_heads, head_dim);
  if (page_size != kIdxPageTokens)
    return set_error(kUnsupported, "indexer_topk: page_size=%d unsupported (need 64)", page_size);
  if (next_n != 1 && next_n != 2)
    return set_error(kUnsupported, "indexer_topk: next_n=%d unsupported (1 or 2)", next_n);
  if (top_k != 512 && top_k != 2048)
    return set_error(kInvalidArgument, "top_k must be 512 or 2048, got %d", top_k);
  if (batch < 0 || max_context_len < 0) return set_error(kInvalidArgument, "indexer_topk: bad sizes");
  if (max_context_len > dsa_topk_max_len())
    return set_error(kUnsupported, "indexer_topk: rows longer than %d are not supported", dsa_topk_max_len());
  if (batch == 0) return kOk;
  if (!q_fp8 || !kv_cache || !weights || !context_lens || !block_tables || !out_physical || !workspace)
    return set_error(kInvalidArgument, "indexer_topk: null pointer");
  if ((reinterpret_cast<uintptr_t>(q_fp8) | reinterpret_cast<uintptr_t>(kv_cache) |
       reinterpret_cast<uintptr_t>(workspace)) & 15)
    return set_error(kInvalidArgument, "indexer_topk: q, kv_cache and workspace must be 16-byte aligned");
  const int rows = batch * next_n;
  const FusedWs f = fused_layout(workspace, rows, max_context_len);
  if (workspace_bytes < f.bytes)
    return set_error(kWorkspaceTooSmall, "indexer_topk: workspace %zu B < %zu B", workspace_bytes, f.bytes);
  hipStream_t st = (hipStream_t)stream;
  // optional hipEvent_t[5]: before the first launch, then after the sample,
  // filter, finish and repair phases
  auto mark = [&](int i) {
    if (phase_events && phase_events[i]) (void)hipEventRecord((hipEvent_t)phase_events[i], st);
  };
  mark(0);
  const int64_t max_pages = (max_context_len + kIdxPageTokens - 1) / kIdxPageTokens;
  const int step = sample_step(max_pages);
  // 1-2. logits of every step-th page (one workgroup per row, kept in LDS) ->
  // the row's score threshold, lists reset
  IdxOut o_s{nullptr, 0, step, f.ws, top_k};
  launch_indexer<kIdxSample>(q_fp8, kv_cache, weights, context_lens, block_tables, block_table_stride, batch,
                             next_n, max_context_len, (max_pages + step - 1) / step, o_s, st);
  if (int rc = check_launch("dsa_indexer_topk(sample)")) return rc;
  mark(1);
  // 3. all pages: candidates at or above the threshold into the row lists
  if (!launch_filter_persistent(q_fp8, kv_cache, weights, context_lens, block_tables, block_table_stride, batch,
                                next_n, max_context_len, f.ws, st)) {
    IdxOut o_f{nullptr, 0, 1, f.ws, top_k};
    launch_indexer<kIdxFilter>(q_fp8, kv_cache, weights, context_lens, block_tables, block_table_stride, batch,
                               next_n, max_context_len, max_pages, o_f, st);
  }
  if (int rc = check_launch("dsa_indexer_topk(filter)")) return rc;
  mark(2);
  // 4. exact top-k of each row's list (with the page translation); a row
  // whose list is unusable is redone by its workgroup from its full logits
  const RowRepair rp{q_fp8, kv_cache, weights, f.logits, f.logits_stride, nullptr, nullptr};
  const int rc = launch_list_select(rp, context_lens, max_context_len, f.ws, block_tables, block_table_stride, next_n,
                                    6u, nullptr, out_physical, out_logical, top_k, rows, st);
  mark(3);
  mark(4);
  return rc;
}
