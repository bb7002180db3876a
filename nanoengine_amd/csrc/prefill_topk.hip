// Fused ragged fp8 MQA logits + exact top-2048 for the prefill indexer, for
// gfx950.
//
// The unfused path writes every logit of every row to HBM ([rows, keys] f32,
// 4.3 GB for an 8192-token chunk over 128K keys) and reads it back for the
// ragged top-k (lightning.py:1212-1246: deep_gemm.fp8_mqa_logits, then
// top_k_per_row_prefill). Here no logit is stored:
//
//   1. prep: clamped windows, the sampled windows and the defer counter;
//   2. sample: every 64th key (key 64j) is copied to a compact array and the
//      logits kernel scores it ([rows, keys/64] f32, 1/64 of the full work);
//   3. threshold: per row, from its sampled scores, an order key t such that
//      about top_k + 4 sqrt + 8 of the sampled keys lie at or above it
//      (expected ~1.7 top_k candidates in the row);
//   4. filter: the logits kernel again over all keys, its epilogue appending
//      (order key, position) of each key at or above t to the row's list;
//   5. list select: the exact top-k of each row's list (topk.hip), written as
//      position + ks;
//   6. fix-up: a row whose list holds fewer than top_k candidates (the sample
//      put t too high) or more than the list capacity is redone on the host's
//      order: its logits are scored into a chunk buffer and selected with the
//      ragged top-k. Needs one 4-byte device-to-host read per call.
//
// Exactness: a list with at least top_k entries, all at or above t, contains
// every key of the row's top-k (the k-th largest is >= t), ties included; the
// list select ranks by (score, lower position) exactly as the ragged top-k
// does, and both read the same float logit of the same kernel arithmetic. The
// result is therefore the ragged top-k's, bit for bit, whatever the sample.
#include <algorithm>
#include <cmath>

#include "dsa_common.h"
#include "../../include/dsa_amd.h"

namespace dsa {
namespace {

constexpr int kSampleStride = 64;  // keys per sampled key
constexpr int kHeads = 64;
constexpr int kHeadDim = 128;
constexpr size_t kAlign = 256;
constexpr int64_t kFixupLogitsBytes = int64_t(1) << 28;  // logits chunk of the fix-up

size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

// Windows clamped to max_len (as the ragged top-k clamps its row lengths), the
// sampled window [ceil(ks/64), ceil(ke'/64)) of each row, and the defer count.
__global__ void __launch_bounds__(256)
mqa_topk_prep_kernel(const int32_t* __restrict__ ks, const int32_t* __restrict__ ke, int rows, int64_t max_len,
                     int64_t samples, int32_t* __restrict__ ke_c, int32_t* __restrict__ lens,
                     int32_t* __restrict__ sks, int32_t* __restrict__ ske, uint32_t* __restrict__ defer_count) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i == 0) *defer_count = 0u;
  if (i >= rows) return;
  const int64_t a = ks[i];
  int64_t l = (int64_t)ke[i] - a;
  l = l < 0 ? 0 : (l > max_len ? max_len : l);
  ke_c[i] = (int32_t)(a + l);
  lens[i] = (int32_t)l;
  // inside [0, samples) whatever the window (the sampled scores are only a guide)
  auto clamp_s = [&](int64_t v) { return (int32_t)(v < 0 ? 0 : (v > samples ? samples : v)); };
  const int64_t s0 = clamp_s((a + kSampleStride - 1) / kSampleStride);
  ske[i] = (int32_t)std::max<int64_t>(s0, clamp_s((a + l + kSampleStride - 1) / kSampleStride));
  sks[i] = (int32_t)s0;
}

// Key 64j and its scale -> sample j. Eight lanes per 128-byte key.
__global__ void __launch_bounds__(256)
mqa_topk_sample_keys_kernel(const uint8_t* __restrict__ kv, const float* __restrict__ kv_scale, int64_t samples,
                            uint8_t* __restrict__ skv, float* __restrict__ sscale) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t j = t >> 3;
  const int part = (int)(t & 7);
  if (j >= samples) return;
  const int64_t key = j * kSampleStride;
  *reinterpret_cast<uint4*>(skv + j * kHeadDim + part * 16) =
      *reinterpret_cast<const uint4*>(kv + key * kHeadDim + part * 16);
  if (part == 0) sscale[j] = kv_scale[key];
}

// One workgroup per row: the threshold order key from the row's sampled
// scores (two histogram levels: 12 then 10 bits of the key). A row of at
// most top_k keys needs no list (the select writes it whole): its threshold
// is the largest key, which no score reaches (NaN ranks as -inf).
__global__ void __launch_bounds__(256)
mqa_topk_threshold_kernel(const float* __restrict__ slog, int64_t s_stride, const int32_t* __restrict__ sks,
                          const int32_t* __restrict__ ske, const int32_t* __restrict__ lens, int top_k,
                          RowWs* __restrict__ ws) {
  __shared__ __align__(16) uint32_t hist[4096];
  __shared__ uint32_t wave_sum[4];
  __shared__ uint32_t tb, above, eq;
  const int tid = threadIdx.x, b = blockIdx.x;
  const int len = lens[b];
  RowWs& w = ws[b];
  uint32_t t_key = 0xffffffffu;
  if (len > top_k) {
    const int a = sks[b];
    const int n = ske[b] - a;
    const float* row = slog + (int64_t)b * s_stride + a;
    const float f = (float)top_k * (float)n / (float)len;
    const uint32_t r = (uint32_t)(f + 4.f * sqrtf(f) + 8.f);
    t_key = 0u;  // every key of the row
    if (r < (uint32_t)n) {
      for (int i = tid; i < 4096; i += 256) hist[i] = 0u;
      __syncthreads();
      for (int i = tid; i < n; i += 256) atomicAdd(&hist[order_key(row[i]) >> 20], 1u);
      __syncthreads();
      find_threshold<256>(hist, wave_sum, 4096, r, &tb, &above, &eq);
      const uint32_t tb0 = tb, rem0 = r - above;
      __syncthreads();
      for (int i = tid; i < 1024; i += 256) hist[i] = 0u;
      __syncthreads();
      for (int i = tid; i < n; i += 256) {
        const uint32_t k = order_key(row[i]);
        if ((k >> 20) == tb0) atomicAdd(&hist[(k >> 10) & 1023u], 1u);
      }
      __syncthreads();
      find_threshold<256>(hist, wave_sum, 1024, rem0, &tb, &above, &eq);
      t_key = (tb0 << 20) | (tb << 10);
    }
  }
  if (tid == 0) {
    w.t_key = t_key;
    w.count = 0u;
    w.failed = 0u;
  }
}

// Rows rows[c0 .. c0 + n) of the inputs -> dense rows 0 .. n of the fix-up.
__global__ void __launch_bounds__(256)
mqa_topk_gather_rows_kernel(const int32_t* __restrict__ rows, int c0, const uint8_t* __restrict__ q,
                            const float* __restrict__ weights, int64_t w_stride, const int32_t* __restrict__ ks,
                            const int32_t* __restrict__ ke_c, const int32_t* __restrict__ lens,
                            uint8_t* __restrict__ qg, float* __restrict__ wg, int32_t* __restrict__ ksg,
                            int32_t* __restrict__ keg, int32_t* __restrict__ lensg) {
  const int i = blockIdx.x, tid = threadIdx.x;
  const int64_t r = rows[c0 + i];
  const uint4* src = reinterpret_cast<const uint4*>(q + r * kHeads * kHeadDim);
  uint4* dst = reinterpret_cast<uint4*>(qg + (int64_t)i * kHeads * kHeadDim);
  for (int e = tid; e < kHeads * kHeadDim / 16; e += 256) dst[e] = src[e];
  if (tid < kHeads) wg[(int64_t)i * kHeads + tid] = weights[r * w_stride + tid];
  if (tid == 0) {
    ksg[i] = ks[r];
    keg[i] = ke_c[r];
    lensg[i] = lens[r];
  }
}

__global__ void __launch_bounds__(256)
mqa_topk_scatter_rows_kernel(const int32_t* __restrict__ rows, int c0, const int32_t* __restrict__ outg, int top_k,
                             int32_t* __restrict__ out) {
  const int i = blockIdx.x;
  const int64_t r = rows[c0 + i];
  for (int e = threadIdx.x; e < top_k; e += 256) out[r * top_k + e] = outg[(int64_t)i * top_k + e];
}

// Workspace layout (each region 256-byte aligned).
struct MqaTopkLayout {
  int64_t samples, fix_rows;
  size_t ws, slog, skv, sscale, ke_c, lens, sks, ske, defer, count;
  size_t qg, wg, ksg, keg, lensg, logg, outg, total;
  MqaTopkLayout(int rows, int64_t keys, int top_k) {
    samples = (keys + kSampleStride - 1) / kSampleStride;
    fix_rows = std::max<int64_t>(1, std::min<int64_t>(rows, kFixupLogitsBytes / (4 * std::max<int64_t>(keys, 1))));
    size_t at = 0;
    auto take = [&](size_t bytes) { const size_t p = at; at += align_up(bytes); return p; };
    ws = take((size_t)rows * sizeof(RowWs));
    slog = take((size_t)rows * samples * 4);
    skv = take((size_t)samples * kHeadDim);
    sscale = take((size_t)samples * 4);
    ke_c = take((size_t)rows * 4);
    lens = take((size_t)rows * 4);
    sks = take((size_t)rows * 4);
    ske = take((size_t)rows * 4);
    defer = take((size_t)rows * 4);
    count = take(4);
    qg = take((size_t)fix_rows * kHeads * kHeadDim);
    wg = take((size_t)fix_rows * kHeads * 4);
    ksg = take((size_t)fix_rows * 4);
    keg = take((size_t)fix_rows * 4);
    lensg = take((size_t)fix_rows * 4);
    logg = take((size_t)fix_rows * keys * 4);
    outg = take((size_t)fix_rows * top_k * 4);
    total = at;
  }
};

}  // namespace
}  // namespace dsa

extern "C" {

size_t dsa_mqa_topk_workspace_bytes(int num_rows, int64_t num_keys, int top_k) {
  if (num_rows <= 0 || num_keys < 0 || top_k <= 0) return 0;
  return dsa::MqaTopkLayout(num_rows, num_keys, top_k).total;
}

int dsa_mqa_topk(const uint8_t* q, const uint8_t* kv, const float* kv_scale, const float* weights,
                 int64_t weights_stride, const int32_t* ks, const int32_t* ke, int num_rows, int64_t num_keys,
                 int num_heads, int64_t max_len, int top_k, int32_t* out, void* workspace, size_t workspace_bytes,
                 void* stream) {
  using namespace dsa;
  if (top_k != 2048) return set_error(kInvalidArgument, "ragged Indexer top_k must be 2048, got %d", top_k);
  if (num_heads != kHeads) return set_error(kUnsupported, "dsa_mqa_topk: num_heads must be 64, got %d", num_heads);
  if (num_rows < 0 || num_keys < 0 || max_len < 0 || weights_stride < num_heads)
    return set_error(kInvalidArgument, "dsa_mqa_topk: bad sizes");
  if (max_len > dsa_topk_max_len())
    return set_error(kUnsupported, "ragged rows longer than %d are not supported (got %lld)", dsa_topk_max_len(),
                     (long long)max_len);
  if (num_rows == 0) return kOk;
  if (!q || !weights || !ks || !ke || !out || (num_keys > 0 && (!kv || !kv_scale)))
    return set_error(kInvalidArgument, "dsa_mqa_topk: null pointer");
  if ((reinterpret_cast<uintptr_t>(q) & 15) || (reinterpret_cast<uintptr_t>(kv) & 15) ||
      (reinterpret_cast<uintptr_t>(kv_scale) & 3) || (reinterpret_cast<uintptr_t>(weights) & 3))
    return set_error(kInvalidArgument, "dsa_mqa_topk: q and kv must be 16-byte aligned");
  const MqaTopkLayout L(num_rows, num_keys, top_k);
  if (!workspace || workspace_bytes < L.total)
    return set_error(kWorkspaceTooSmall, "dsa_mqa_topk: workspace %zu B < %zu B", workspace_bytes, L.total);
  if (reinterpret_cast<uintptr_t>(workspace) & 255)
    return set_error(kInvalidArgument, "dsa_mqa_topk: workspace must be 256-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  uint8_t* base = static_cast<uint8_t*>(workspace);
  auto at = [&](size_t off) { return base + off; };
  RowWs* ws = reinterpret_cast<RowWs*>(at(L.ws));
  float* slog = reinterpret_cast<float*>(at(L.slog));
  int32_t* ke_c = reinterpret_cast<int32_t*>(at(L.ke_c));
  int32_t* lens = reinterpret_cast<int32_t*>(at(L.lens));
  int32_t* sks = reinterpret_cast<int32_t*>(at(L.sks));
  int32_t* ske = reinterpret_cast<int32_t*>(at(L.ske));
  int32_t* defer = reinterpret_cast<int32_t*>(at(L.defer));
  uint32_t* count = reinterpret_cast<uint32_t*>(at(L.count));

  hipLaunchKernelGGL(mqa_topk_prep_kernel, dim3((num_rows + 255) / 256), dim3(256), 0, st, ks, ke, num_rows, max_len,
                     L.samples, ke_c, lens, sks, ske, count);
  if (int rc = check_launch("dsa_mqa_topk (prep)")) return rc;
  if (num_keys > 0) {
    uint8_t* skv = at(L.skv);
    float* sscale = reinterpret_cast<float*>(at(L.sscale));
    hipLaunchKernelGGL(mqa_topk_sample_keys_kernel, dim3((unsigned)((L.samples * 8 + 255) / 256)), dim3(256), 0, st,
                       kv, kv_scale, L.samples, skv, sscale);
    if (int rc = check_launch("dsa_mqa_topk (sample keys)")) return rc;
    if (int rc = launch_mqa_logits(false, q, skv, sscale, weights, weights_stride, sks, ske, num_rows, L.samples,
                                   slog, L.samples, nullptr, st))
      return rc;
  }
  hipLaunchKernelGGL(mqa_topk_threshold_kernel, dim3(num_rows), dim3(256), 0, st, slog, L.samples, sks, ske, lens,
                     top_k, ws);
  if (int rc = check_launch("dsa_mqa_topk (threshold)")) return rc;
  if (num_keys > 0)
    if (int rc = launch_mqa_logits(true, q, kv, kv_scale, weights, weights_stride, ks, ke_c, num_rows, num_keys,
                                   nullptr, 0, ws, st))
      return rc;
  const RowRepair defer_only{nullptr, nullptr, nullptr, nullptr, 0, defer, count};
  if (int rc = launch_list_select(defer_only, lens, max_len, ws, nullptr, 0, 1, 0u, ks, out, nullptr, top_k,
                                  num_rows, st))
    return rc;

  // rows whose list could not give the exact top-k
  uint32_t n_defer = 0;
  if (hipMemcpyAsync(&n_defer, count, sizeof(n_defer), hipMemcpyDeviceToHost, st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess)
    return set_error(kLaunchFailed, "dsa_mqa_topk: reading the deferred-row count failed");
  if (n_defer > (uint32_t)num_rows)
    return set_error(kLaunchFailed, "dsa_mqa_topk: deferred-row count %u > rows %d", n_defer, num_rows);
  uint8_t* qg = at(L.qg);
  float* wg = reinterpret_cast<float*>(at(L.wg));
  int32_t* ksg = reinterpret_cast<int32_t*>(at(L.ksg));
  int32_t* keg = reinterpret_cast<int32_t*>(at(L.keg));
  int32_t* lensg = reinterpret_cast<int32_t*>(at(L.lensg));
  float* logg = reinterpret_cast<float*>(at(L.logg));
  int32_t* outg = reinterpret_cast<int32_t*>(at(L.outg));
  for (int64_t c0 = 0; c0 < (int64_t)n_defer; c0 += L.fix_rows) {
    const int n = (int)std::min<int64_t>(L.fix_rows, (int64_t)n_defer - c0);
    hipLaunchKernelGGL(mqa_topk_gather_rows_kernel, dim3(n), dim3(256), 0, st, defer, (int)c0, q, weights,
                       weights_stride, ks, ke_c, lens, qg, wg, ksg, keg, lensg);
    if (int rc = check_launch("dsa_mqa_topk (fix-up gather)")) return rc;
    if (int rc = launch_mqa_logits(false, qg, kv, kv_scale, wg, kHeads, ksg, keg, n, num_keys, logg, num_keys,
                                   nullptr, st))
      return rc;
    // the list workspace is free again: the fix-up's top-k reuses its first rows
    if (int rc = dsa_topk_transform_ragged(logg, num_keys, lensg, ksg, ksg, outg, n, max_len, top_k, ws,
                                           (size_t)n * sizeof(RowWs), st))
      return rc;
    hipLaunchKernelGGL(mqa_topk_scatter_rows_kernel, dim3(n), dim3(256), 0, st, defer, (int)c0, outg, top_k, out);
    if (int rc = check_launch("dsa_mqa_topk (fix-up scatter)")) return rc;
  }
  return kOk;
}

}  // extern "C"
