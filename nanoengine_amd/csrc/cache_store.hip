// fp8 cache writers for the DSA path, for gfx950: the 656-byte MLA row and the
// 132-byte indexer key (split page layout). One wave per token.
//
// MLA row (dlengine/runtime/kernel/triton/hopper/fp8_utils.py:32-108):
//   bytes [0,512)   e4m3fn(nope / s_t), four 128-dim tiles t
//   bytes [512,528) s_t = 2^ceil(log2(max(amax_t / 448, 1e-12))) as f32
//   bytes [528,656) the 64 rope values, bf16, unchanged
// Indexer key (dlengine/runtime/layers/backends/dsa/indexer/lightning.py:78-101,
// page layout :494-507): page = [page_size x 128 fp8][page_size x f32 scale],
//   sf = 2^ceil(log2(max(amax, 1e-4) / 448)), code = e4m3fn(x * (1/sf)).
// Slots < 0 are skipped (the reference writes them harmlessly or not at all).
#include "dsa_common.h"
#include "../../include/dsa_amd.h"

namespace dsa {

__device__ __forceinline__ int64_t load_slot(const void* slots, int slot_is_64, int i) {
  return slot_is_64 ? reinterpret_cast<const int64_t*>(slots)[i] : (int64_t)reinterpret_cast<const int32_t*>(slots)[i];
}

__global__ void __launch_bounds__(256)
mla_kv_store_kernel(const uint16_t* __restrict__ kv, int64_t row_stride, const void* __restrict__ slots,
                    int slot_is_64, int n, uint8_t* __restrict__ cache, int64_t block_stride, int block_size) {
  const int lane = threadIdx.x & 63;
  const int tok = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tok >= n) return;
  const int64_t slot = load_slot(slots, slot_is_64, tok);
  if (slot < 0) return;
  const uint16_t* src = kv + (int64_t)tok * row_stride;
  uint8_t* row = cache + (slot / block_size) * block_stride + (slot % block_size) * 656;
  // nope: lane l holds dims 8l .. 8l+7 (tile l/16)
  const v4i raw = *reinterpret_cast<const v4i*>(src + 8 * lane);
  float x[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[2 * i] = bf16_to_f32((uint16_t)raw[i]);
    x[2 * i + 1] = bf16_to_f32((uint16_t)((uint32_t)raw[i] >> 16));
  }
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(x[i]));
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) amax = fmaxf(amax, shfl_xor(amax, off));
  const float s = pow2_ceil(fmaxf(amax / 448.f, 1e-12f));
  uint2 codes;
  codes.x = f32x4_to_fp8(x[0] / s, x[1] / s, x[2] / s, x[3] / s);
  codes.y = f32x4_to_fp8(x[4] / s, x[5] / s, x[6] / s, x[7] / s);
  *reinterpret_cast<uint2*>(row + 8 * lane) = codes;
  if ((lane & 15) == 0) reinterpret_cast<float*>(row + 512)[lane >> 4] = s;
  // rope: lanes 0-15 copy 4 bf16 each
  if (lane < 16) *reinterpret_cast<uint2*>(row + 528 + 8 * lane) = *reinterpret_cast<const uint2*>(src + 512 + 4 * lane);
}

__global__ void __launch_bounds__(256)
indexer_k_store_kernel(const uint16_t* __restrict__ k, int64_t row_stride, const void* __restrict__ slots,
                       int slot_is_64, int n, uint8_t* __restrict__ cache, int page_size) {
  const int lane = threadIdx.x & 63;
  const int tok = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tok >= n) return;
  const int64_t slot = load_slot(slots, slot_is_64, tok);
  if (slot < 0) return;
  const uint32_t two = *reinterpret_cast<const uint32_t*>(k + (int64_t)tok * row_stride + 2 * lane);
  const float a = bf16_to_f32((uint16_t)two), b = bf16_to_f32((uint16_t)(two >> 16));
  float amax = fmaxf(fabsf(a), fabsf(b));
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) amax = fmaxf(amax, shfl_xor(amax, off));
  const float sf = pow2_ceil(fmaxf(amax, 1e-4f) / 448.f);
  const float inv = 1.f / sf;
  const int64_t page = slot / page_size, off = slot % page_size;
  uint8_t* base = cache + page * (int64_t)page_size * 132;
  const uint32_t w = f32x4_to_fp8(a * inv, b * inv, 0.f, 0.f);
  *reinterpret_cast<uint16_t*>(base + off * 128 + 2 * lane) = (uint16_t)w;
  if (lane == 0) reinterpret_cast<float*>(base + (int64_t)page_size * 128)[off] = sf;
}


// Paged split-layout indexer cache -> contiguous ragged keys and scales
// (dlengine/runtime/kernel/triton/generic/indexer_cache_gather.py:8-114).
// Ragged token cu[b] + i is token i of sequence b, read through block_table[b].
// Eight lanes copy one token's 128 key bytes (16 B each); the first of them
// also copies its 4-byte scale. The sequence of a token is found by binary
// search over cu_seqlens_k.
__global__ void __launch_bounds__(256)
gather_indexer_cache_kernel(const uint8_t* __restrict__ cache, int64_t page_bytes, int page_size,
                            const int32_t* __restrict__ block_table, int64_t bt_stride,
                            const void* __restrict__ cu, int cu_is_64, int num_seqs, int64_t total_k,
                            uint8_t* __restrict__ key_out, uint8_t* __restrict__ scale_out) {
  const int64_t tok = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
  const int piece = threadIdx.x & 7;
  if (tok >= total_k) return;
  int lo = 0, hi = num_seqs;  // largest b with cu[b] <= tok
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (load_slot(cu, cu_is_64, mid) <= tok) lo = mid; else hi = mid;
  }
  const int64_t i = tok - load_slot(cu, cu_is_64, lo);
  const int64_t page = block_table[(int64_t)lo * bt_stride + i / page_size];
  const int64_t off = i % page_size;
  const uint8_t* base = cache + page * page_bytes;
  *reinterpret_cast<v4i*>(key_out + tok * 128 + 16 * piece) =
      *reinterpret_cast<const v4i*>(base + off * 128 + 16 * piece);
  if (piece == 0)
    *reinterpret_cast<uint32_t*>(scale_out + tok * 4) =
        *reinterpret_cast<const uint32_t*>(base + (int64_t)page_size * 128 + off * 4);
}


// The sparse prefill's keys in ragged order, from the paged fp8 MLA cache and
// the chunk's fresh bf16 rows, in one pass: the gather of the cached prefix
// (dlengine/runtime/layers/backends/attention/mla_utils.py:200-234), its
// restore to bf16 (kernel/triton/hopper/fp8_utils.py:153-196) and the
// cached/fresh interleave (mla_utils.py:118-165) as the prefill calls them at
// dlengine/runtime/models/deepseek_v2/deepseek_v2.py:1573-1604.
// Key row r of sequence b (cu_k[b] <= r < cu_k[b+1]) at i = r - cu_k[b] is
// cached row i of the sequence when i < k_len - q_len (read through
// block_table[b]), else fresh row cu_q[b] + i - (k_len - q_len). One wave per
// row: for a cached row lane l dequantises nope bytes 8l .. 8l+7 with the
// scale of tile l/16 (exact: fp8 times a power of two is a bf16 value) and
// writes 16 bytes; lanes 0-7 copy the 128-byte bf16 rope tail. A fresh row is
// a 1152-byte copy in 16-byte pieces. A cached row whose block-table column is
// past the table's width, or whose block is negative or past the cache, is
// written as zeros (the row is never read).
__global__ void __launch_bounds__(256)
mla_prefill_kv_kernel(const uint8_t* __restrict__ cache, int64_t block_stride, int block_size, int64_t num_blocks,
                      const int32_t* __restrict__ block_table, int64_t bt_stride, int bt_width,
                      const void* __restrict__ cu_q,
                      const void* __restrict__ cu_k, int cu_is_64, int num_seqs, int64_t total_k,
                      const uint16_t* __restrict__ fresh, int64_t fresh_stride, uint16_t* __restrict__ out,
                      int64_t out_stride) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= total_k) return;
  int lo = 0, hi = num_seqs;  // largest b < num_seqs with cu_k[b] <= r
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (load_slot(cu_k, cu_is_64, mid) <= r) lo = mid; else hi = mid;
  }
  const int64_t k0 = load_slot(cu_k, cu_is_64, lo), k1 = load_slot(cu_k, cu_is_64, lo + 1);
  const int64_t q0 = load_slot(cu_q, cu_is_64, lo), q1 = load_slot(cu_q, cu_is_64, lo + 1);
  const int64_t i = r - k0, cached = (k1 - k0) - (q1 - q0);
  uint8_t* dst = reinterpret_cast<uint8_t*>(out + r * out_stride);
  if (i < cached) {
    const int64_t col = i / block_size;
    const int64_t blk = col < bt_width ? (int64_t)block_table[(int64_t)lo * bt_stride + col] : -1;
    if (blk < 0 || blk >= num_blocks) {
      *reinterpret_cast<v4i*>(dst + 16 * lane) = v4i{0, 0, 0, 0};
      if (lane < 8) *reinterpret_cast<v4i*>(dst + 1024 + 16 * lane) = v4i{0, 0, 0, 0};
      return;
    }
    const uint8_t* row = cache + blk * block_stride + (i % block_size) * 656;
    const uint2 codes = *reinterpret_cast<const uint2*>(row + 8 * lane);
    const float scale = reinterpret_cast<const float*>(row + 512)[lane >> 4];
    v4i o;
    o[0] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)codes.x, scale, false));
    o[1] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)codes.x, scale, true));
    o[2] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)codes.y, scale, false));
    o[3] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)codes.y, scale, true));
    *reinterpret_cast<v4i*>(dst + 16 * lane) = o;
    if (lane < 8) *reinterpret_cast<v4i*>(dst + 1024 + 16 * lane) = *reinterpret_cast<const v4i*>(row + 528 + 16 * lane);
  } else {
    const uint8_t* src = reinterpret_cast<const uint8_t*>(fresh + (q0 + i - cached) * fresh_stride);
    *reinterpret_cast<v4i*>(dst + 16 * lane) = *reinterpret_cast<const v4i*>(src + 16 * lane);
    if (lane < 8) *reinterpret_cast<v4i*>(dst + 1024 + 16 * lane) = *reinterpret_cast<const v4i*>(src + 1024 + 16 * lane);
  }
}

}  // namespace dsa

extern "C" {

int dsa_mla_kv_store(const void* kv, int64_t kv_row_stride, const void* slots, int slot_is_64, int num_tokens,
                     uint8_t* kv_cache, int64_t kv_block_stride_bytes, int kv_block_size, void* stream) {
  using namespace dsa;
  if (num_tokens < 0 || kv_block_size <= 0 || kv_block_stride_bytes < (int64_t)kv_block_size * 656)
    return set_error(kInvalidArgument, "dsa_mla_kv_store: bad sizes");
  if (num_tokens == 0) return kOk;
  if (!kv || !slots || !kv_cache) return set_error(kInvalidArgument, "dsa_mla_kv_store: null pointer");
  if ((reinterpret_cast<uintptr_t>(kv) & 15) || (kv_row_stride % 8) || (kv_block_stride_bytes % 8) ||
      (reinterpret_cast<uintptr_t>(kv_cache) & 7))
    return set_error(kInvalidArgument, "dsa_mla_kv_store: kv rows must be 16-byte aligned, cache 8-byte aligned");
  hipLaunchKernelGGL(mla_kv_store_kernel, dim3((num_tokens + 3) / 4), dim3(256), 0, (hipStream_t)stream,
                     static_cast<const uint16_t*>(kv), kv_row_stride, slots, slot_is_64, num_tokens, kv_cache,
                     kv_block_stride_bytes, kv_block_size);
  return check_launch("dsa_mla_kv_store");
}

int dsa_indexer_k_store(const void* k, int64_t k_row_stride, const void* slots, int slot_is_64, int num_tokens,
                        uint8_t* cache, int page_size, void* stream) {
  using namespace dsa;
  if (num_tokens < 0 || page_size <= 0) return set_error(kInvalidArgument, "dsa_indexer_k_store: bad sizes");
  if (num_tokens == 0) return kOk;
  if (!k || !slots || !cache) return set_error(kInvalidArgument, "dsa_indexer_k_store: null pointer");
  if ((reinterpret_cast<uintptr_t>(k) & 3) || (k_row_stride % 2))
    return set_error(kInvalidArgument, "dsa_indexer_k_store: key rows must be 4-byte aligned");
  hipLaunchKernelGGL(indexer_k_store_kernel, dim3((num_tokens + 3) / 4), dim3(256), 0, (hipStream_t)stream,
                     static_cast<const uint16_t*>(k), k_row_stride, slots, slot_is_64, num_tokens, cache, page_size);
  return check_launch("dsa_indexer_k_store");
}


int dsa_gather_indexer_cache(const uint8_t* cache, int64_t page_bytes, int page_size, int head_dim,
                             const int32_t* block_table, int64_t bt_stride, const void* cu_seqlens_k,
                             int cu_is_64, int num_seqs, int64_t total_k, uint8_t* key_out,
                             uint8_t* scale_out, void* stream) {
  using namespace dsa;
  if (head_dim != 128)
    return set_error(kUnsupported, "dsa_gather_indexer_cache: head_dim=%d (only 128 is supported)", head_dim);
  if (page_size <= 0 || num_seqs < 0 || total_k < 0 || page_bytes < (int64_t)page_size * 132)
    return set_error(kInvalidArgument, "dsa_gather_indexer_cache: bad sizes");
  if (total_k == 0) return kOk;
  if (!cache || !block_table || !cu_seqlens_k || !key_out || !scale_out || num_seqs == 0)
    return set_error(kInvalidArgument, "dsa_gather_indexer_cache: null pointer or no sequences");
  if (((reinterpret_cast<uintptr_t>(cache) | reinterpret_cast<uintptr_t>(key_out)) & 15) || (page_bytes & 15) ||
      (reinterpret_cast<uintptr_t>(scale_out) & 3))
    return set_error(kInvalidArgument, "dsa_gather_indexer_cache: cache and keys must be 16-byte aligned");
  const int64_t nwg = (total_k + 31) / 32;
  hipLaunchKernelGGL(gather_indexer_cache_kernel, dim3((unsigned)nwg), dim3(256), 0, (hipStream_t)stream, cache,
                     page_bytes, page_size, block_table, bt_stride, cu_seqlens_k, cu_is_64, num_seqs, total_k,
                     key_out, scale_out);
  return check_launch("dsa_gather_indexer_cache");
}

int dsa_mla_prefill_kv(const uint8_t* kv_cache, int64_t kv_block_stride_bytes, int kv_block_size,
                       int64_t kv_num_blocks, const int32_t* block_table, int64_t bt_stride, int bt_width,
                       const void* cu_seqlens_q,
                       const void* cu_seqlens_k, int cu_is_64, int num_seqs, int64_t total_k, const void* fresh,
                       int64_t fresh_row_stride, void* out, int64_t out_row_stride, void* stream) {
  using namespace dsa;
  if (num_seqs < 1 || total_k < 0 || kv_block_size <= 0 || fresh_row_stride < 576 || out_row_stride < 576 ||
      kv_block_stride_bytes < (int64_t)kv_block_size * 656 || kv_num_blocks < 0 || bt_width < 0 ||
      bt_stride < bt_width)
    return set_error(kInvalidArgument, "dsa_mla_prefill_kv: bad sizes");
  if (total_k == 0) return kOk;
  if (!kv_cache || !block_table || !cu_seqlens_q || !cu_seqlens_k || !fresh || !out)
    return set_error(kInvalidArgument, "dsa_mla_prefill_kv: null pointer");
  if (((reinterpret_cast<uintptr_t>(kv_cache) | reinterpret_cast<uintptr_t>(fresh) |
        reinterpret_cast<uintptr_t>(out)) & 15) || (kv_block_stride_bytes & 15) || (fresh_row_stride & 7) ||
      (out_row_stride & 7))
    return set_error(kInvalidArgument, "dsa_mla_prefill_kv: cache, fresh rows and output rows must be 16-byte aligned");
  const int64_t nwg = (total_k + 3) / 4;
  if (nwg > INT32_MAX) return set_error(kInvalidArgument, "dsa_mla_prefill_kv: too many rows");
  hipLaunchKernelGGL(mla_prefill_kv_kernel, dim3((unsigned)nwg), dim3(256), 0, (hipStream_t)stream, kv_cache,
                     kv_block_stride_bytes, kv_block_size, kv_num_blocks, block_table, bt_stride, bt_width,
                     cu_seqlens_q, cu_seqlens_k,
                     cu_is_64, num_seqs, total_k, static_cast<const uint16_t*>(fresh), fresh_row_stride,
                     static_cast<uint16_t*>(out), out_row_stride);
  return check_launch("dsa_mla_prefill_kv");
}

}  // extern "C"
