// Ragged fp8 MQA logits for the prefill indexer, for gfx950:
//
//   logits[i, j] = sum_h w[i, h] * relu(q[i, h, :] . kv[j, :]) * kv_scale[j],  ks[i] <= j < ke[i]
//
// (the contraction of deep_gemm.fp8_mqa_logits as called at
// dlengine/runtime/layers/backends/dsa/indexer/lightning.py:1212-1219; the
// score definition is lightning.py:116-162).
//
// This is a GEMM of the (token, head) rows of q [M*64, 128] against the keys
// [N, 128] with a ReLU-weighted head reduction in the epilogue, so it runs on
// v_mfma_scale_f32_32x32x64_f8f6f4 (unit scales), the fp8 shape that issues at
// the full fp8 rate on gfx950 (the 16x16x128 shape reaches ~78% of it). A
// workgroup (16 waves, four per SIMD) owns 16 query tokens and one chunk of
// keys; each wave keeps the A operands of its token (2 head tiles of 32 x 2
// k-steps of 64 dims) resident in registers for the whole chunk. Four waves
// per SIMD let the ReLU-weighted epilogue of one wave issue while another's
// MFMAs run. Keys stream through LDS in 128-key stages (16 KB, three buffers):
// each wave issues one 1 KB global->LDS copy per stage, already in the
// lane order of the MFMA B operand (32 keys x 64 dims per operand, lane half
// h holding bytes 32h .. 32h+31 of the 64-dim step), so an operand is two
// conflict-free ds_read_b128. Per 32 keys and token: 4 MFMAs (2 head tiles x
// 2 k-steps), ReLU + weight on the 16 heads a lane holds per head tile, then
// one shuffle pairs the two lane halves: lane l ends with key l of each 64-key
// half of the stage, one coalesced 256-byte store per token and half.
//
// Grid: token blocks x key chunks, with the chunk count a multiple of 8 and
// chunk c placed on XCD c % 8 (workgroups are dealt to the 8 XCDs round
// robin), so the workgroups sharing a chunk's keys share one L2; a short key
// set with many query blocks runs as one chunk (each query block read once).
//
// Filter mode (the fused top-k of prefill_topk.hip): instead of storing the
// logit, each wave compares the order key of its 64 logits with its row's
// threshold, appends the passing (key, position) pairs to a per-wave LDS
// stage (ballot + popcount slots) and moves the stage to the row's global
// list with one atomic when it could overflow and at the end. The stage is
// sized so that a typical chunk flushes once, at the end: a flush waits for
// the atomic's return, which also drains the wave's key prefetches.
#include <algorithm>
#include <type_traits>

#include "dsa_common.h"
#include "../../include/dsa_amd.h"

namespace dsa {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kPfThreads = 1024;
constexpr int kPfWaves = kPfThreads / 64;
constexpr int kPfTokens = kPfWaves;  // one token per wave, 16 per workgroup
constexpr int kPfStageKeys = 128;
constexpr int kPfStageBytes = kPfStageKeys * 128;       // 16 KB of keys
constexpr int kPfKeyTiles = kPfStageKeys / 32;
constexpr int kPfBufs = 3;
constexpr int kPfHeads = 64;

struct PfLds {
  uint8_t key[kPfBufs][kPfStageBytes];
  float scale[kPfBufs][kPfStageKeys];
};
// The filter mode's per-wave candidate stage: (order key, position in the
// row's window) of the keys at or above the row's threshold, moved to the
// row's list in RowWs with one global atomic per flush.
constexpr int kPfStageCap = 832;  // fills the LDS left by the key stages (157 KB of 160 KB)
struct PfLdsFilter : PfLds {
  uint32_t st_key[kPfWaves][kPfStageCap];
  uint32_t st_pos[kPfWaves][kPfStageCap];
};

__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}
__device__ __forceinline__ void dma4(const void* g, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)reinterpret_cast<uintptr_t>(p); }

__device__ __forceinline__ v8i load32B(const uint8_t* p) {
  const v4i a = *reinterpret_cast<const v4i*>(p);
  const v4i b = *reinterpret_cast<const v4i*>(p + 16);
  v8i r;
  r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
  r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
  return r;
}

// Lane l's 32-byte operand from two 1 KB chunks: bytes 0-15 at lo + 16l, 16-31 at hi + 16l.
__device__ __forceinline__ v8i load32B_lds(const uint8_t* lo, const uint8_t* hi, int lane) {
  const v4i a = *reinterpret_cast<const v4i*>(lo + 16 * lane);
  const v4i b = *reinterpret_cast<const v4i*>(hi + 16 * lane);
  v8i r;
  r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
  r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
  return r;
}

__device__ __forceinline__ float relu(float x) { return __builtin_amdgcn_fmed3f(x, 0.f, 3.402823466e38f); }

// Issue this wave's share of stage `kb` (keys kb .. kb+127) into LDS buffer
// `buf`: wave w copies chunk w = (key tile kt = w/4, k-step ks = (w/2)%2,
// half p = w%2): lane l takes key kb + 32kt + l%32, bytes 64ks + 32(l/32) +
// 16p .. +16, to key[buf] + 1024w + 16l. In the wave w of each group of
// eight, lanes 8(w%8) .. +8 copy the scales of keys kb + 64(w/8) + 8(w%8) .. +8.
// Keys past n_keys read key n_keys - 1 (their logits are never stored).
__device__ __forceinline__ void issue_stage(PfLds* lds, int buf, int64_t kb, int64_t n_keys, const uint8_t* kv,
                                            const float* kv_scale, int wave, int lane) {
  static_assert(kPfWaves * 1024 == kPfStageBytes, "one 1 KB chunk per wave");
  const int kt = wave >> 2, ks = (wave >> 1) & 1, hp = wave & 1;
  int64_t key = kb + kt * 32 + (lane & 31);
  key = key < n_keys ? key : n_keys - 1;
  dma16(kv + key * 128 + ks * 64 + (lane >> 5) * 32 + hp * 16, lds_addr(&lds->key[buf][wave * 1024]));
  const int half = wave >> 3;
  int64_t sk = kb + 64 * half + lane;
  sk = sk < n_keys ? sk : n_keys - 1;
  if ((lane >> 3) == (wave & 7)) dma4(kv_scale + sk, lds_addr(&lds->scale[buf][64 * half]));
}

// kFilter: no logits are stored; a key whose order key is at or above the
// row's threshold (ws[row].t_key) joins the row's candidate list instead.
template <bool kFilter>
__global__ void __launch_bounds__(kPfThreads)
mqa_logits_kernel(const uint8_t* __restrict__ q, const uint8_t* __restrict__ kv, const float* __restrict__ kv_scale,
                  const float* __restrict__ weights, int64_t w_stride, const int32_t* __restrict__ ks,
                  const int32_t* __restrict__ ke, int M, int64_t n_keys, int token_blocks, int64_t chunk_keys,
                  float* __restrict__ logits, int64_t logits_stride, RowWs* __restrict__ ws) {
  __shared__ typename std::conditional<kFilter, PfLdsFilter, PfLds>::type lds;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // workgroup -> (token block, chunk): XCD b % 8 takes chunks c with c % 8 == b % 8
  // (one chunk covers every key: workgroup b takes token block b; any
  // workgroup past the last token block exits)
  const int b = blockIdx.x;
  const bool one_chunk = chunk_keys >= n_keys;
  const int r = b >> 3;
  const int tb = one_chunk ? b : r % token_blocks;
  const int chunk = one_chunk ? 0 : (r / token_blocks) * 8 + (b & 7);
  const int r0 = tb * kPfTokens;
  // key range of the block's 16 rows, intersected with the chunk
  int lo_i = INT32_MAX, hi_i = INT32_MIN;
  if (lane < kPfTokens && r0 + lane < M) {
    lo_i = ks[r0 + lane];
    hi_i = ke[r0 + lane];
  }
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) {
    lo_i = min(lo_i, __shfl_xor(lo_i, m, 64));
    hi_i = max(hi_i, __shfl_xor(hi_i, m, 64));
  }
  lo_i = __builtin_amdgcn_readfirstlane(lo_i);
  hi_i = __builtin_amdgcn_readfirstlane(hi_i);
  const int64_t c0 = (int64_t)chunk * chunk_keys;
  int64_t lo = max((int64_t)lo_i, c0), hi = min(min((int64_t)hi_i, c0 + chunk_keys), n_keys);
  if (lo >= hi) return;
  lo &= ~(int64_t)(kPfStageKeys - 1);
  const int nstages = (int)((hi - lo + kPfStageKeys - 1) / kPfStageKeys);

  // this wave's token: A operands (head tile ht, k-step ks: head 32ht + lane%32,
  // bytes 64ks + 32(lane/32) .. +32) and the weights of the 16 heads a lane's
  // accumulator rows hold per head tile (32ht + 8(r/4) + 4(lane/32) + r%4)
  const int row = r0 + wave;
  const bool row_ok = row < M;
  const int rc = row_ok ? row : M - 1;
  const int rks = row_ok ? ks[rc] : 0, rke = row_ok ? ke[rc] : 0;
  v8i qa[2][2];
  float w[2][16];
  {
    const uint8_t* qb = q + (int64_t)rc * kPfHeads * 128;
    const float* wb = weights + (int64_t)rc * w_stride;
#pragma unroll
    for (int ht = 0; ht < 2; ++ht) {
#pragma unroll
      for (int kst = 0; kst < 2; ++kst) qa[ht][kst] = load32B(qb + (ht * 32 + (lane & 31)) * 128 + kst * 64 + (lane >> 5) * 32);
#pragma unroll
      for (int r = 0; r < 16; ++r) w[ht][r] = wb[ht * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)];
    }
  }
  uint32_t tk = 0;
  int cnt = 0;  // staged candidates of this wave's row (wave-uniform)
  if constexpr (kFilter) tk = row_ok ? ws[rc].t_key : 0u;
  auto flush = [&]() {
    if constexpr (kFilter) {
      if (cnt == 0) return;
      RowWs& rw = ws[rc];
      uint32_t base = 0;
      if (lane == 0) base = atomicAdd(&rw.count, (uint32_t)cnt);
      base = __builtin_amdgcn_readfirstlane(base);
      for (int e = lane; e < cnt; e += 64)
        if (base + (uint32_t)e < (uint32_t)kListCap) {
          rw.key[base + e] = lds.st_key[wave][e];
          rw.pos[base + e] = lds.st_pos[wave][e];
        }
      cnt = 0;
    }
  };
  issue_stage(&lds, 0, lo, n_keys, kv, kv_scale, wave, lane);
  if (nstages > 1) issue_stage(&lds, 1, lo + kPfStageKeys, n_keys, kv, kv_scale, wave, lane);
  // the query loads above are ordinary loads: make the compiler's count start from zero
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)

  for (int s = 0; s < nstages; ++s) {
    // stage s landed for every wave; every wave is done reading buffer (s + 2) % 3
    if (s + 1 < nstages) asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    const int buf = s % kPfBufs;
    const int64_t kb = lo + (int64_t)s * kPfStageKeys;
    const uint8_t* kbuf = lds.key[buf];
    // two 64-key halves per stage, each finished (stored) before the next, so
    // that the registers hold one half's operands and partial sums at a time
#pragma unroll
    for (int g = 0; g < kPfKeyTiles / 2; ++g) {
      __builtin_amdgcn_sched_barrier(0);
      float part[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int kt = 2 * g + t;
        const v8i kb0 = load32B_lds(kbuf + (kt * 4 + 0) * 1024, kbuf + (kt * 4 + 1) * 1024, lane);
        const v8i kb1 = load32B_lds(kbuf + (kt * 4 + 2) * 1024, kbuf + (kt * 4 + 3) * 1024, lane);
        const v16f z = {};
        v16f c0 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(qa[0][0], kb0, z, 0, 0, 0, 127, 0, 127);
        v16f c1 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(qa[1][0], kb0, z, 0, 0, 0, 127, 0, 127);
        c0 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(qa[0][1], kb1, c0, 0, 0, 0, 127, 0, 127);
        c1 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(qa[1][1], kb1, c1, 0, 0, 0, 127, 0, 127);
        // c_ht[r]: head 32ht + 8(r/4) + 4(lane/32) + r%4, key kb + 32kt + lane%32
        float a0 = 0.f, a1 = 0.f;  // two chains: no fma waits on the previous one
        // the epilogue issues ahead of the other waves' MFMAs (measured ~2-3% faster
        // than equal priority; raising the MFMA sequence instead gains ~1%)
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          a0 = fmaf(w[0][r], relu(c0[r]), a0);
          a1 = fmaf(w[1][r], relu(c1[r]), a1);
        }
        part[t] = a0 + a1;
        __builtin_amdgcn_s_setprio(0);
      }
      // the two lane halves hold the two halves of the heads: lane l < 32
      // keeps the half's first key tile (key l), lane l >= 32 its second
      // (key 32 + l%32 = l)
      const bool hi32 = lane & 32;
      const float v = (hi32 ? part[1] : part[0]) + __shfl_xor(hi32 ? part[0] : part[1], 32, 64);
      const float sc = lds.scale[buf][64 * g + lane];
      const int64_t key = kb + 64 * g + lane;
      if constexpr (kFilter) {
        const uint32_t okey = order_key(v * sc);
        const bool pred = row_ok && key >= rks && key < rke && key < hi && okey >= tk;
        const uint64_t m = __ballot(pred);
        if (m) {
          if (pred) {
            const int slot = cnt + (int)__popcll(m & ((1ull << lane) - 1ull));
            lds.st_key[wave][slot] = okey;
            lds.st_pos[wave][slot] = (uint32_t)(key - rks);
          }
          cnt += (int)__popcll(m);
          if (cnt > kPfStageCap - 64) flush();
        }
      } else {
        if (key >= rks && key < rke && key < hi)
          __builtin_nontemporal_store(v * sc, logits + (int64_t)row * logits_stride + key);
      }
    }
    if (s + 2 < nstages) issue_stage(&lds, (s + 2) % kPfBufs, kb + 2 * kPfStageKeys, n_keys, kv, kv_scale, wave, lane);
  }
  flush();
}

// logits[i, j] = -inf for j outside [ks[i], ke[i]), j < n_cols.
__global__ void __launch_bounds__(256)
mqa_logits_clean_kernel(const int32_t* __restrict__ ks, const int32_t* __restrict__ ke, int rows, int64_t n_cols,
                        float* __restrict__ logits, int64_t logits_stride) {
  for (int i = blockIdx.y; i < rows; i += gridDim.y) {
    const int64_t a = ks[i], e = ke[i];
    float* rowp = logits + (int64_t)i * logits_stride;
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < n_cols; j += (int64_t)gridDim.x * blockDim.x)
      if (j < a || j >= e) rowp[j] = -__builtin_inff();
  }
}


// Per-query key windows of a ragged prefill batch, on the device. Query i of
// sequence b (cu_q[b] <= i < cu_q[b+1]) sees the sequence's cached prefix and
// the fresh keys up to its own: [cu_k[b], i + 1 + (cu_k[b+1] - cu_q[b+1])), the
// causal rule of dlengine/runtime/layers/backends/dsa/indexer/lightning.py:
// 1190-1206 written in closed form. One thread per query finds b by binary
// search. Workgroup 0 also checks the batch and writes status[4] =
// {fault bits, total keys, longest key length, most pages of one sequence}
// (bit 0: cu_q or cu_k does not start at 0; bit 1: cu_q does not end at
// num_queries; bit 2: some q length < 0 or k length < q length), so the host
// validates with one read of 32 bytes.
__global__ void __launch_bounds__(256)
prefill_windows_kernel(const void* __restrict__ cu_q, const void* __restrict__ cu_k, int cu_is_64, int num_seqs,
                       int num_queries, int page_size, int32_t* __restrict__ ks, int32_t* __restrict__ ke,
                       int64_t* __restrict__ status) {
  auto cu = [&](const void* p, int i) -> int64_t {
    return cu_is_64 ? reinterpret_cast<const int64_t*>(p)[i] : (int64_t)reinterpret_cast<const int32_t*>(p)[i];
  };
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < num_queries) {
    int lo = 0, hi = num_seqs;  // largest b < num_seqs with cu_q[b] <= i
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (cu(cu_q, mid) <= i) lo = mid; else hi = mid;
    }
    ks[i] = (int32_t)cu(cu_k, lo);
    ke[i] = (int32_t)(i + 1 + cu(cu_k, lo + 1) - cu(cu_q, lo + 1));
  }
  if (blockIdx.x != 0) return;
  __shared__ unsigned long long s_bits, s_maxk, s_maxp;
  if (threadIdx.x == 0) s_bits = s_maxk = s_maxp = 0;
  __syncthreads();
  unsigned long long bits = 0, maxk = 0, maxp = 0;
  for (int b = threadIdx.x; b < num_seqs; b += 256) {
    const int64_t ql = cu(cu_q, b + 1) - cu(cu_q, b), kl = cu(cu_k, b + 1) - cu(cu_k, b);
    if (ql < 0 || kl < ql) bits |= 4;
    if (kl > 0) {
      maxk = max(maxk, (unsigned long long)kl);
      maxp = max(maxp, (unsigned long long)((kl + page_size - 1) / page_size));
    }
  }
  if (threadIdx.x == 0) {
    if (cu(cu_q, 0) != 0 || cu(cu_k, 0) != 0) bits |= 1;
    if (cu(cu_q, num_seqs) != num_queries) bits |= 2;
  }
  atomicOr(&s_bits, bits);
  atomicMax(&s_maxk, maxk);
  atomicMax(&s_maxp, maxp);
  __syncthreads();
  if (threadIdx.x == 0) {
    status[0] = (int64_t)s_bits;
    status[1] = cu(cu_k, num_seqs);
    status[2] = (int64_t)s_maxk;
    status[3] = (int64_t)s_maxp;
  }
}

}  // namespace

// Both modes of the logits kernel on one grid: token blocks x key chunks.
int launch_mqa_logits(bool filter, const uint8_t* q, const uint8_t* kv, const float* kv_scale, const float* weights,
                      int64_t weights_stride, const int32_t* ks, const int32_t* ke, int num_rows, int64_t num_keys,
                      float* logits, int64_t logits_stride, RowWs* ws, hipStream_t st) {
  const int token_blocks = (num_rows + kPfTokens - 1) / kPfTokens;
  int64_t chunks, chunk_keys;
  if (token_blocks >= 512 && num_keys <= 32 * kPfStageKeys) {
    // few keys, many rows: one chunk, so that each query block is read once
    chunks = 1;
    chunk_keys = std::max<int64_t>(num_keys, 1);
  } else {
    // chunks: a multiple of 8 (one XCD each), enough workgroups for the 256 CUs
    chunks = 8;
    while ((int64_t)token_blocks * chunks < 1024 && chunks * 64 * 8 <= num_keys) chunks *= 2;
    chunk_keys = (num_keys + chunks - 1) / chunks;
    chunk_keys = (chunk_keys + kPfStageKeys - 1) / kPfStageKeys * kPfStageKeys;
  }
  const int64_t grid = (int64_t)token_blocks * chunks;
  if (grid > INT32_MAX) return set_error(kInvalidArgument, "mqa logits: grid too large");
  if (filter)
    hipLaunchKernelGGL(mqa_logits_kernel<true>, dim3((unsigned)grid), dim3(kPfThreads), 0, st, q, kv, kv_scale,
                       weights, weights_stride, ks, ke, num_rows, num_keys, token_blocks, chunk_keys, logits,
                       logits_stride, ws);
  else
    hipLaunchKernelGGL(mqa_logits_kernel<false>, dim3((unsigned)grid), dim3(kPfThreads), 0, st, q, kv, kv_scale,
                       weights, weights_stride, ks, ke, num_rows, num_keys, token_blocks, chunk_keys, logits,
                       logits_stride, ws);
  return check_launch(filter ? "mqa logits (filter)" : "dsa_mqa_logits");
}

}  // namespace dsa

extern "C" {

int dsa_mqa_logits(const uint8_t* q, const uint8_t* kv, const float* kv_scale, const float* weights,
                   int64_t weights_stride, const int32_t* ks, const int32_t* ke, int num_rows, int64_t num_keys,
                   int num_heads, float* logits, int64_t logits_stride, int64_t num_cols, int clean_logits,
                   void* stream) {
  using namespace dsa;
  if (num_rows < 0 || num_keys < 0 || num_cols < num_keys || logits_stride < num_cols || weights_stride < num_heads)
    return set_error(kInvalidArgument, "dsa_mqa_logits: bad sizes");
  if (num_heads != kPfHeads) return set_error(kUnsupported, "dsa_mqa_logits: num_heads must be 64, got %d", num_heads);
  if (num_rows == 0) return kOk;
  if (!q || !weights || !ks || !ke || !logits || (num_keys > 0 && (!kv || !kv_scale)))
    return set_error(kInvalidArgument, "dsa_mqa_logits: null pointer");
  if ((reinterpret_cast<uintptr_t>(q) & 15) || (reinterpret_cast<uintptr_t>(kv) & 15) ||
      (reinterpret_cast<uintptr_t>(kv_scale) & 3) || (reinterpret_cast<uintptr_t>(weights) & 3))
    return set_error(kInvalidArgument, "dsa_mqa_logits: q and kv must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  if (clean_logits && num_cols > 0) {
    const int gx = (int)std::min<int64_t>((num_cols + 255) / 256, 64);
    hipLaunchKernelGGL(mqa_logits_clean_kernel, dim3(gx, std::min(num_rows, 65535)), dim3(256), 0, st, ks, ke,
                       num_rows, num_cols, logits, logits_stride);
    if (int rc = check_launch("dsa_mqa_logits (clean)")) return rc;
  }
  if (num_keys == 0) return kOk;
  return launch_mqa_logits(false, q, kv, kv_scale, weights, weights_stride, ks, ke, num_rows, num_keys, logits,
                           logits_stride, nullptr, st);
}

int dsa_prefill_windows(const void* cu_seqlens_q, const void* cu_seqlens_k, int cu_is_64, int num_seqs,
                        int num_queries, int page_size, int32_t* ks, int32_t* ke, int64_t* status, void* stream) {
  using namespace dsa;
  if (num_seqs < 1 || num_queries < 0 || page_size <= 0)
    return set_error(kInvalidArgument, "dsa_prefill_windows: bad sizes");
  if (!cu_seqlens_q || !cu_seqlens_k || !status || (num_queries > 0 && (!ks || !ke)))
    return set_error(kInvalidArgument, "dsa_prefill_windows: null pointer");
  const int grid = std::max(1, (num_queries + 255) / 256);
  hipLaunchKernelGGL(prefill_windows_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, cu_seqlens_q,
                     cu_seqlens_k, cu_is_64, num_seqs, num_queries, page_size, ks, ke, status);
  return check_launch("dsa_prefill_windows");
}

}  // extern "C"
