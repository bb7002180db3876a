// fp8 lightning-indexer logits over the paged indexer cache, for gfx950.
//
//   logits[b*n+j, t] = sum_h w[b*n+j, h] * relu(q[b,j,h,:] . k[t,:]) * scale[t]
//
// One wave owns one 64-token page at a time. The page's 64x128 fp8 keys are
// loaded straight from HBM into registers as the B operand of
// v_mfma_scale_f32_16x16x128_f8f6f4 (fp8 x fp8 -> fp32, unit scales), 32
// contiguous bytes per lane, while the query heads (A operand, 16 heads per
// tile) stay resident in registers for the whole workgroup lifetime. Each page
// costs 16 MFMAs per query token (4 token tiles x 4 head tiles); the ReLU and
// the head weights are applied on the fp32 accumulators, and a 3-shuffle
// butterfly finishes the head sum so that lane l ends up owning token l of the
// page: the logits row segment and the per-token scales are then one
// coalesced 256-byte load/store each. Each wave keeps two pages in flight
// (three rotating register buffers) so that HBM latency overlaps compute.
//
// Page layout (bytes): [64 tokens x 128 fp8][64 x f32 scale] = 8448.
#include <algorithm>
#include <type_traits>

#include "dsa_common.h"
#include "../../include/dsa_amd.h"

namespace dsa {

constexpr int kIdxThreads = 256;
constexpr int kIdxWaves = kIdxThreads / 64;
constexpr int kIdxPagesPerWave = 6;
constexpr int kIdxPageTokens = 64;
constexpr int kIdxHeadDim = 128;
constexpr int kIdxHeads = 64;
constexpr int kIdxPageBytes = kIdxPageTokens * (kIdxHeadDim + 4);

__device__ __forceinline__ v8i load32B(const uint8_t* p) {
  const v4i a = *reinterpret_cast<const v4i*>(p);
  const v4i b = *reinterpret_cast<const v4i*>(p + 16);
  v8i r;
  r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
  r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
  return r;
}

// max(x, 0) in one instruction (v_med3_f32 with bounds 0 and FLT_MAX).
__device__ __forceinline__ float relu(float x) { return __builtin_amdgcn_fmed3f(x, 0.f, 3.402823466e38f); }

struct PageRegs {
  v8i k[4];      // token tiles: lane holds token tt*16 + lane%16, bytes (lane/16)*32 .. +32
  float scale;   // scale of token `lane`
};

__device__ __forceinline__ void load_page(PageRegs& pr, const uint8_t* page, int lane) {
  const uint8_t* base = page + (lane & 15) * kIdxHeadDim + (lane >> 4) * 32;
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) pr.k[tt] = load32B(base + tt * 16 * kIdxHeadDim);
  pr.scale = reinterpret_cast<const float*>(page + kIdxPageTokens * kIdxHeadDim)[lane];
}

// What a launch does with the logits of a page.
enum IdxMode : int {
  kIdxStore = 0,   // logits[row, t] (and, with `only_failed`, only rows whose list failed)
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
  const RowWs* only_failed; // kIdxStore: skip rows whose list was usable (NULL: all rows)
  int top_k;                // kIdxSample
};

constexpr int kIdxWgTokens = kIdxWaves * kIdxPagesPerWave * kIdxPageTokens;  // 1536

struct IdxStageNone {
  uint32_t unused;
};

constexpr int kSamplePagesPerWave = 4;
constexpr int kSamplePages = kIdxWaves * kSamplePagesPerWave;  // 16 sampled pages per row, one workgroup
struct IdxSampleLds {
  float logit[2][kSamplePages * kIdxPageTokens];
  uint32_t hist[4096];
  uint32_t wave_sum[kIdxWaves];
  uint32_t tb, above, eq;
};

struct IdxStage {  // per-WG LDS staging of kIdxFilter candidates, per query token
  uint32_t count[2];
  uint32_t base[2];
  uint32_t key[2][kIdxWgTokens];
  uint32_t pos[2][kIdxWgTokens];
};

template <int NQ, int MODE>
__device__ __forceinline__ void compute_page(const PageRegs& cur, int p, int vp, int lane, const v8i (&qa)[NQ][4],
                                             const float (&w)[NQ][4][4], const int (&L)[NQ],
                                             const uint32_t (&tk)[NQ], int64_t max_ctx, const IdxOut& o,
                                             void* lds, int b) {
  IdxStage* stage = static_cast<IdxStage*>(lds);
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    float part[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      // four independent products per token tile keep the MFMA pipe busy
      v4f c[4];
#pragma unroll
      for (int ht = 0; ht < 4; ++ht)
        c[ht] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(qa[j][ht], cur.k[tt], (v4f){0.f, 0.f, 0.f, 0.f},
                                                                0, 0, 0, 127, 0, 127);
      // c[ht][r]: head ht*16 + (lane/16)*4 + r, token tt*16 + lane%16
      float acc = 0.f;
#pragma unroll
      for (int ht = 0; ht < 4; ++ht)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc = fmaf(w[j][ht][r], relu(c[ht][r]), acc);
      part[tt] = acc;
    }
    // Butterfly over the four 16-lane groups: lane group g keeps token tile g.
    const bool hi32 = lane & 32;
    const float s0 = hi32 ? part[0] : part[2];
    const float s1 = hi32 ? part[1] : part[3];
    const float k0 = (hi32 ? part[2] : part[0]) + shfl_xor(s0, 32);
    const float k1 = (hi32 ? part[3] : part[1]) + shfl_xor(s1, 32);
    const bool hi16 = lane & 16;
    const float v = (hi16 ? k1 : k0) + shfl_xor(hi16 ? k0 : k1, 16);
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

// Two waves per SIMD: three 33-VGPR page buffers, the resident query tiles
// and head weights take ~180 VGPRs for one query token.
template <int NQ, int MODE>
__global__ void __launch_bounds__(kIdxThreads) __attribute__((amdgpu_waves_per_eu(2)))
indexer_logits_kernel(const uint8_t* __restrict__ q, const uint8_t* __restrict__ kv,
                      const float* __restrict__ weights, const int32_t* __restrict__ ctx_lens,
                      const int32_t* __restrict__ block_tables, int64_t bt_stride, int64_t max_ctx,
                      const IdxOut o) {
  // LDS: candidate staging (filter) or the sampled logits (sample)
  __shared__ typename std::conditional<
      MODE == kIdxFilter, IdxStage,
      typename std::conditional<MODE == kIdxSample, IdxSampleLds, IdxStageNone>::type>::type lds_mem;
  IdxStage* stage = reinterpret_cast<IdxStage*>(&lds_mem);
  constexpr int PPW = MODE == kIdxSample ? kSamplePagesPerWave : kIdxPagesPerWave;
  const int b = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int step = MODE == kIdxSample ? o.page_step : 1;

  if (MODE == kIdxStore && o.only_failed) {
    bool any = false;
#pragma unroll
    for (int j = 0; j < NQ; ++j) any |= o.only_failed[b * NQ + j].failed != 0u;
    if (!any) return;
  }

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
  const int vp_begin = blockIdx.x * (kIdxWaves * PPW) + wave;
  if (MODE != kIdxSample && blockIdx.x * (kIdxWaves * PPW) >= nvp) return;

  if (MODE == kIdxFilter) {
    if (threadIdx.x < NQ) stage->count[threadIdx.x] = 0u;
    __syncthreads();
  }

  // Query heads as MFMA A operands: tile (j, ht) row i = head ht*16 + i.
  v8i qa[NQ][4];
  float w[NQ][4][4];
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    const uint8_t* qb = q + ((int64_t)(b * NQ + j) * kIdxHeads) * kIdxHeadDim;
    const float* wb = weights + (int64_t)(b * NQ + j) * kIdxHeads;
#pragma unroll
    for (int ht = 0; ht < 4; ++ht) {
      qa[j][ht] = load32B(qb + (ht * 16 + (lane & 15)) * kIdxHeadDim + (lane >> 4) * 32);
#pragma unroll
      for (int r = 0; r < 4; ++r) w[j][ht][r] = wb[ht * 16 + (lane >> 4) * 4 + r];
    }
  }

  const int32_t* bt = block_tables + (int64_t)b * bt_stride;
  // Three page buffers rotate so that two pages are in flight while one is
  // being multiplied; the wave's virtual pages are vp_begin + 4*i.
  PageRegs buf0, buf1, buf2;
  auto valid = [&](int i) { return i < PPW && vp_begin + kIdxWaves * i < nvp; };
  // All of the wave's block-table entries in one load up front, so no page
  // load waits behind a dependent table read.
  const int my_page = (lane < PPW && valid(lane)) ? bt[(vp_begin + kIdxWaves * lane) * step] : 0;
  auto page_ptr = [&](int i) {
    return kv + (int64_t)__builtin_amdgcn_readlane(my_page, i) * kIdxPageBytes;
  };
  auto compute = [&](const PageRegs& pr, int i) {
    const int vp = vp_begin + kIdxWaves * i;
    compute_page<NQ, MODE>(pr, vp * step, vp, lane, qa, w, L, tk, max_ctx, o, &lds_mem, b);
  };
  if (valid(0)) load_page(buf0, page_ptr(0), lane);
  if (valid(1)) load_page(buf1, page_ptr(1), lane);
#pragma unroll
  for (int i = 0; i < PPW; i += 3) {
    if (valid(i + 2)) load_page(buf2, page_ptr(i + 2), lane);
    if (valid(i)) compute(buf0, i);
    if (valid(i + 3)) load_page(buf0, page_ptr(i + 3), lane);
    if (valid(i + 1)) compute(buf1, i + 1);
    if (valid(i + 4)) load_page(buf1, page_ptr(i + 4), lane);
    if (valid(i + 2)) compute(buf2, i + 2);
  }

  if (MODE == kIdxSample) {
    // The row's score threshold from its sampled logits (one workgroup holds
    // them all in LDS): the rank-r key of the sample, r = f + 4 sqrt(f) + 8
    // with f = k * nsample / len (two radix digits, 12 + 10 bits), so that
    // about k + margin tokens of the whole row are expected at or above it. The
    // row's candidate list is reset here.
    IdxSampleLds& sl = *reinterpret_cast<IdxSampleLds*>(&lds_mem);
    const int tid = threadIdx.x;
    __syncthreads();
    const int span = step * kIdxPageTokens;
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      RowWs& rw = o.ws[b * NQ + j];
      const float* smp = sl.logit[j];
      const int len = (int)min((int64_t)max(L[j], 0), max_ctx);
      const int nv = (len + span - 1) / span;
      uint32_t t_key = 0u;  // 0: every token is a candidate
      if (len > o.top_k) {
        for (int i = tid; i < 4096; i += kIdxThreads) sl.hist[i] = 0u;
        __syncthreads();
        for (int e = tid; e < nv * kIdxPageTokens; e += kIdxThreads)
          if ((e >> 6) * span + (e & 63) < len) atomicAdd(&sl.hist[order_key(smp[e]) >> 20], 1u);
        uint32_t nsample = 0;
        for (int v = 0; v < nv; ++v) nsample += (uint32_t)max(0, min(len - v * span, kIdxPageTokens));
        const float fk = (float)nsample / (float)len * (float)o.top_k;
        const uint32_t r = (uint32_t)(fk + 4.f * sqrtf(fk) + 8.f);
        __syncthreads();
        if (r < nsample) {
          find_threshold<kIdxThreads>(sl.hist, sl.wave_sum, 4096, r, &sl.tb, &sl.above, &sl.eq);
          const uint32_t tb0 = sl.tb, rem0 = r - sl.above;
          __syncthreads();
          for (int i = tid; i < 1024; i += kIdxThreads) sl.hist[i] = 0u;
          __syncthreads();
          for (int e = tid; e < nv * kIdxPageTokens; e += kIdxThreads)
            if ((e >> 6) * span + (e & 63) < len) {
              const uint32_t k = order_key(smp[e]);
              if ((k >> 20) == tb0) atomicAdd(&sl.hist[(k >> 10) & 1023u], 1u);
            }
          __syncthreads();
          find_threshold<kIdxThreads>(sl.hist, sl.wave_sum, 1024, rem0, &sl.tb, &sl.above, &sl.eq);
          t_key = (tb0 << 20) | (sl.tb << 10);
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
      for (uint32_t e = threadIdx.x; e < n; e += kIdxThreads)
        if (base + e < (uint32_t)kListCap) {
          rw.key[base + e] = stage->key[j][e];
          rw.pos[base + e] = stage->pos[j][e];
        }
    }
  }
}

template <int MODE>
void launch_indexer(const uint8_t* q, const uint8_t* kv, const float* weights, const int32_t* ctx_lens,
                    const int32_t* bt, int64_t bt_stride, int batch, int next_n, int64_t max_ctx, int64_t vpages,
                    const IdxOut& o, hipStream_t stream) {
  const int64_t per_block = kIdxWaves * (MODE == kIdxSample ? kSamplePagesPerWave : kIdxPagesPerWave);
  const dim3 grid((unsigned)((vpages + per_block - 1) / per_block), (unsigned)batch);
  if (next_n == 1)
    hipLaunchKernelGGL((indexer_logits_kernel<1, MODE>), grid, dim3(kIdxThreads), 0, stream, q, kv, weights, ctx_lens,
                       bt, bt_stride, max_ctx, o);
  else
    hipLaunchKernelGGL((indexer_logits_kernel<2, MODE>), grid, dim3(kIdxThreads), 0, stream, q, kv, weights, ctx_lens,
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
  IdxOut o{logits, logits_stride, 1, nullptr, nullptr, 0};
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
  float* logits;  // full logits, written only for rows redone by the repair launches
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
  IdxOut o_s{nullptr, 0, step, f.ws, nullptr, top_k};
  launch_indexer<kIdxSample>(q_fp8, kv_cache, weights, context_lens, block_tables, block_table_stride, batch,
                             next_n, max_context_len, (max_pages + step - 1) / step, o_s, st);
  if (int rc = check_launch("dsa_indexer_topk(sample)")) return rc;
  mark(1);
  // 3. all pages: candidates at or above the threshold into the row lists
  IdxOut o_f{nullptr, 0, 1, f.ws, nullptr, top_k};
  launch_indexer<kIdxFilter>(q_fp8, kv_cache, weights, context_lens, block_tables, block_table_stride, batch, next_n,
                             max_context_len, max_pages, o_f, st);
  if (int rc = check_launch("dsa_indexer_topk(filter)")) return rc;
  mark(2);
  // 4. exact top-k of each usable list (with the page translation)
  if (int rc = launch_finish_fused(f.logits, f.logits_stride, context_lens, max_context_len, f.ws, block_tables,
                                   block_table_stride, next_n, 6u, out_physical, out_logical, top_k, rows, false, st))
    return rc;
  mark(3);
  // 5-6. rows whose list was unusable: their full logits, then the full select
  // (both launches return at once for every other row)
  IdxOut o_r{f.logits, f.logits_stride, 1, nullptr, f.ws, top_k};
  launch_indexer<kIdxStore>(q_fp8, kv_cache, weights, context_lens, block_tables, block_table_stride, batch, next_n,
                            max_context_len, max_pages, o_r, st);
  if (int rc = check_launch("dsa_indexer_topk(repair)")) return rc;
  const int rc = launch_finish_fused(f.logits, f.logits_stride, context_lens, max_context_len, f.ws, block_tables,
                                     block_table_stride, next_n, 6u, out_physical, out_logical, top_k, rows, true, st);
  mark(4);
  return rc;
}
