// Shared device helpers for the DSA decode kernels (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef float v2f __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

namespace dsa {

// Status codes shared by every C entry point (0 = success).
enum Status : int {
  kOk = 0,
  kInvalidArgument = 1,
  kUnsupported = 2,
  kLaunchFailed = 3,
  kWorkspaceTooSmall = 4,
};

// Records a human-readable message for dsa_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

// Monotone uint32 key of a float: larger float -> larger key. NaN ranks as -inf.
__device__ __forceinline__ uint32_t order_key(float x) {
  uint32_t u = __float_as_uint(x);
  if (x != x) u = 0xff800000u;  // -inf
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Round-to-nearest-even float -> bf16 bits.
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float x) {
  uint32_t u = __float_as_uint(x);
  if (x != x) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ uint32_t pack_bf16_rne(float lo, float hi) {
  return f32_to_bf16_rne(lo) | (f32_to_bf16_rne(hi) << 16);
}

// 2^ceil(log2(v)) for finite v > 0, exactly: v = 2^e * 1.m, ceil is e when the
// mantissa is zero and e + 1 otherwise.
__device__ __forceinline__ float pow2_ceil(float v) {
  const uint32_t u = __float_as_uint(v);
  int e = (int)((u >> 23) & 0xff);
  const uint32_t m = u & 0x7fffffu;
  if (e == 0) {  // subnormal: v = m * 2^-149
    const int msb = 31 - __clz(m);
    const int k = msb - 149 + ((m & (m - 1)) ? 1 : 0);
    return ldexpf(1.f, k);
  }
  const int k = e - 127 + (m ? 1 : 0);
  return ldexpf(1.f, k);
}

// Four floats -> four e4m3fn bytes (round to nearest even).
__device__ __forceinline__ uint32_t f32x4_to_fp8(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// Per-row candidate list of the exact top-k (device workspace): a score
// threshold t_key (order key), the number of candidates appended, a flag set
// when the list could not be used (fused indexer path), then the (key,
// position) pairs. Filled by the top-k gather kernel or by the fused indexer.
constexpr int kListCap = 6144;
struct RowWs {
  uint32_t t_key;
  uint32_t count;
  uint32_t failed;
  uint32_t pad;
  uint32_t key[kListCap];
  uint32_t pos[kListCap];
};

// What the list select needs to redo a row whose list is unusable: the
// indexer inputs of the row (query [rows, 64, 128] fp8, head weights
// [rows, 64], the paged key cache) and a logits row to write. With q NULL the
// row is not redone in the kernel: its index is appended to defer_rows
// (count in *defer_count) and its output is left for the caller to write.
struct RowRepair {
  const uint8_t* q;
  const uint8_t* kv;
  const float* weights;
  float* logits;
  int64_t logits_stride;
  int32_t* defer_rows;
  uint32_t* defer_count;
};

// Launcher of the list select of the fused indexer + top-k entry point
// (topk.hip): the exact top-k of each row's candidate list, with the page
// translation; a row whose list is unusable is redone in place from its
// full logits.
// Without a page table, row b's positions are written plus offsets[b] (NULL: 0).
int launch_list_select(const RowRepair& rp, const int32_t* seq_lens, int64_t max_len, RowWs* ws,
                       const int32_t* page_table, int64_t pt_stride, int pt_div, uint32_t page_bits,
                       const int32_t* offsets, int32_t* out_page, int32_t* out_raw, int top_k, int rows,
                       hipStream_t stream);

// The ragged fp8 MQA logits kernel (prefill_logits.hip). filter = false:
// logits[i, j] for j in [ks[i], ke[i]). filter = true: nothing is stored;
// key j of row i joins ws[i]'s candidate list (position j - ks[i]) when its
// order key is at least ws[i].t_key.
int launch_mqa_logits(bool filter, const uint8_t* q, const uint8_t* kv, const float* kv_scale, const float* weights,
                      int64_t weights_stride, const int32_t* ks, const int32_t* ke, int num_rows, int64_t num_keys,
                      float* logits, int64_t logits_stride, RowWs* ws, hipStream_t st);

// Sparse MLA decode over physical slots of the paged fp8 cache (the body of
// dsa_sparse_mla_decode). max_out (splits == 1 only) receives each head's
// largest scaled score in natural units; with compact set, each row's valid
// indices must come first and a workgroup stops at its first block with none.
// A chunked prefill's keys for the sparse MLA decode kernel: token t attends
// over the first counts[2t] entries of its cache-slot list (valid slots first)
// and over counts[2t+1] fresh bf16 rows rows[idx[t][i]] (row stride in
// elements, num_rows rows; idx row stride idx_stride, width >= counts rounded
// up to 32).
struct MlaFresh {
  const int32_t* counts;
  const void* rows;
  int64_t row_stride;
  int64_t num_rows;
  const int32_t* idx;
  int64_t idx_stride;
};
int sparse_mla_decode_impl(const void* q, int64_t q_token_stride, int64_t q_head_stride, const uint8_t* kv_cache,
                           int64_t kv_block_stride_bytes, int kv_block_size, int64_t kv_num_blocks,
                           const int32_t* indices, int64_t idx_stride, int num_tokens, int num_heads, int topk,
                           float sm_scale, void* out, float* lse, int num_splits, void* workspace,
                           size_t workspace_bytes, void* stream, float* max_out, const MlaFresh* fresh);

template <typename T>
__device__ __forceinline__ T shfl_xor(T v, int mask) {
  return __shfl_xor(v, mask, 64);
}

// Block-wide (NT threads): find the bin tb with S(tb+1) < remain <= S(tb),
// S(b) = sum of hist[b..nbins). Leaves tb, above = S(tb+1), eq = hist[tb] in
// the shared *tb_out, *above_out, *eq_out for every thread after the call.
// nbins is a power of two <= 4096; hist is 16-byte aligned. Thread t owns
// bins [t*per, t*per + per), read once (16-byte reads when per >= 4).
template <int NT>
__device__ void find_threshold(const uint32_t* hist, uint32_t* wave_sum, int nbins, uint32_t remain,
                               uint32_t* tb_out, uint32_t* above_out, uint32_t* eq_out) {
  constexpr int kWaves = NT / 64;
  constexpr int kMaxPer = 4096 / NT;
  static_assert(kMaxPer % 4 == 0, "4096 bins over at most 1024 threads");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = nbins >= NT ? nbins / NT : 1;
  const int first = tid * per;
  uint32_t v[kMaxPer];
#pragma unroll
  for (int i = 0; i < kMaxPer; ++i) v[i] = 0u;
  if (per >= 4) {
#pragma unroll
    for (int i = 0; i < kMaxPer; i += 4)
      if (i < per) {
        const uint4 x = *reinterpret_cast<const uint4*>(hist + first + i);
        v[i] = x.x; v[i + 1] = x.y; v[i + 2] = x.z; v[i + 3] = x.w;
      }
  } else if (first < nbins) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (i < per) v[i] = hist[first + i];
  }
  uint32_t local = 0;
#pragma unroll
  for (int i = 0; i < kMaxPer; ++i) local += v[i];
  // inclusive suffix sum inside the wave
  uint32_t sfx = local;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    uint32_t n = __shfl_down(sfx, off, 64);
    if (lane + off < 64) sfx += n;
  }
  if (lane == 0) wave_sum[wave] = sfx;
  __syncthreads();
  uint32_t higher = sfx - local;
#pragma unroll
  for (int w = 0; w < kWaves; ++w)
    if (w > wave) higher += wave_sum[w];
  if (first < nbins && higher < remain && higher + local >= remain) {
    uint32_t acc = higher;
#pragma unroll
    for (int i = kMaxPer - 1; i >= 0; --i) {
      if (i < per) {
        const uint32_t h = v[i];
        if (acc < remain && acc + h >= remain) {
          *tb_out = first + i;
          *above_out = acc;
          *eq_out = h;
        }
        acc += h;
      }
    }
  }
  __syncthreads();
}

}  // namespace dsa
