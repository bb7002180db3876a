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

template <int NQ>
__device__ __forceinline__ void compute_page(const PageRegs& cur, int p, int lane, const v8i (&qa)[NQ][4],
                                             const float (&w)[NQ][4][4], const int (&L)[NQ], int64_t max_ctx,
                                             float* __restrict__ logits, int64_t logits_stride, int b) {
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
    if (t < max_ctx) {
      float* dst = logits + (int64_t)(b * NQ + j) * logits_stride;
      // streaming store: the logits are consumed by a later kernel, not reused here
      __builtin_nontemporal_store(t < L[j] ? v * cur.scale : -__builtin_inff(), dst + t);
    }
  }
}

// Two waves per SIMD: three 33-VGPR page buffers, the resident query tiles
// and head weights take ~180 VGPRs for one query token.
template <int NQ>
__global__ void __launch_bounds__(kIdxThreads) __attribute__((amdgpu_waves_per_eu(2)))
indexer_logits_kernel(const uint8_t* __restrict__ q, const uint8_t* __restrict__ kv,
                      const float* __restrict__ weights, const int32_t* __restrict__ ctx_lens,
                      const int32_t* __restrict__ block_tables, int64_t bt_stride, int64_t max_ctx,
                      float* __restrict__ logits, int64_t logits_stride) {
  const int b = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;

  int L[NQ];
  int Lmax = 0;
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    L[j] = ctx_lens[b * NQ + j];
    Lmax = max(Lmax, L[j]);
  }
  const int npages = (int)((min((int64_t)Lmax, max_ctx) + kIdxPageTokens - 1) / kIdxPageTokens);
  const int p_begin = blockIdx.x * (kIdxWaves * kIdxPagesPerWave) + wave;
  if (blockIdx.x * (kIdxWaves * kIdxPagesPerWave) >= npages) return;

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
  // being multiplied; the wave's pages are p_begin + 4*i.
  PageRegs buf0, buf1, buf2;
  auto valid = [&](int i) { return i < kIdxPagesPerWave && p_begin + kIdxWaves * i < npages; };
  // All of the wave's block-table entries in one load up front, so no page
  // load waits behind a dependent table read.
  const int my_page = (lane < kIdxPagesPerWave && valid(lane)) ? bt[p_begin + kIdxWaves * lane] : 0;
  auto page_ptr = [&](int i) {
    return kv + (int64_t)__builtin_amdgcn_readlane(my_page, i) * kIdxPageBytes;
  };
  if (valid(0)) load_page(buf0, page_ptr(0), lane);
  if (valid(1)) load_page(buf1, page_ptr(1), lane);
#pragma unroll
  for (int i = 0; i < kIdxPagesPerWave; i += 3) {
    if (valid(i + 2)) load_page(buf2, page_ptr(i + 2), lane);
    if (valid(i)) compute_page<NQ>(buf0, p_begin + kIdxWaves * i, lane, qa, w, L, max_ctx, logits, logits_stride, b);
    if (valid(i + 3)) load_page(buf0, page_ptr(i + 3), lane);
    if (valid(i + 1)) compute_page<NQ>(buf1, p_begin + kIdxWaves * (i + 1), lane, qa, w, L, max_ctx, logits, logits_stride, b);
    if (valid(i + 4)) load_page(buf1, page_ptr(i + 4), lane);
    if (valid(i + 2)) compute_page<NQ>(buf2, p_begin + kIdxWaves * (i + 2), lane, qa, w, L, max_ctx, logits, logits_stride, b);
  }
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
  const int64_t per_block = kIdxWaves * kIdxPagesPerWave;
  const dim3 grid((unsigned)((max_pages + per_block - 1) / per_block), (unsigned)batch);
  if (next_n == 1)
    hipLaunchKernelGGL(indexer_logits_kernel<1>, grid, dim3(kIdxThreads), 0, (hipStream_t)stream, q_fp8,
                       kv_cache, weights, context_lens, block_tables, block_table_stride, max_context_len,
                       logits, logits_stride);
  else
    hipLaunchKernelGGL(indexer_logits_kernel<2>, grid, dim3(kIdxThreads), 0, (hipStream_t)stream, q_fp8,
                       kv_cache, weights, context_lens, block_tables, block_table_stride, max_context_len,
                       logits, logits_stride);
  return check_launch("dsa_indexer_logits");
}
