// Indexer prologue for gfx950: the query transform that produces the indexer's
// (q_fp8, weights) and the key transform that writes the indexer cache.
//
// Query (dlengine/runtime/kernel/jit/sgl/csrc/deepseek_v4/indexer_q.cuh:57-225,
// Python entry dlengine/runtime/kernel/jit/sgl/deepseek_v4.py:290-322, instantiated
// with RoPE on the leading 64 dims and the Hadamard rotation, :153-165):
//   1. dims 0..63 hold interleaved (re, im) pairs; reorder them to the half
//      layout [re 0..31 | im 0..31] (lightning.py:110-113) unless the caller
//      already provides that layout;
//   2. NeoX rotation of the 64 dims with cos/sin row `positions[t]` of the
//      [max_pos, 64] = [cos 0..31 | sin 0..31] cache (rotary_embedding.py:10-18,
//      33-40); every value rounded to bf16;
//   3. 128-point Hadamard, times 1/sqrt(128), rounded to bf16;
//   4. per (token, head) row: sf = 2^ceil(log2(max(amax, 1e-4) / 448)),
//      code = e4m3fn(x / sf); weights[t, h] = gate[t, h] * weight_scale * sf.
// Key (dlengine/runtime/kernel/triton/generic/indexer_transform.py:156-288):
//   LayerNorm(weight, bias, eps) rounded to bf16, steps 1-2 above, the
//   Hadamard of step 3 kept in f32, then the quantisation of step 4 written to
//   the split page layout [page_size x 128 fp8][page_size x f32 scale].
//
// Data layout: one row of 128 values per 16 lanes (8 consecutive values per
// lane, one 16-byte load), 4 rows per wave, 16 rows per 256-thread block. The
// Hadamard's first three stages are in-lane, the last four are xor shuffles
// inside the 16-lane group. Arithmetic is f32 without contraction, in a fixed
// order (Hadamard stages h = 1, 2, ..., 64; sums as an in-lane tree then a
// lane butterfly), so that a CPU restatement in IEEE f32 reproduces it bit
// for bit.
#include "dsa_common.h"
#include "../../include/dsa_amd.h"

namespace dsa {
namespace {

constexpr int kRowsPerBlock = 16;
constexpr float kInvSqrt128 = 0.0883883461356163f;  // f32 nearest to 128^-0.5

__device__ __forceinline__ float bf16_round(float x) { return __uint_as_float(f32_to_bf16_rne(x) << 16); }

__device__ __forceinline__ int64_t load_index(const void* p, int is_64, int i) {
  return is_64 ? reinterpret_cast<const int64_t*>(p)[i] : (int64_t)reinterpret_cast<const int32_t*>(p)[i];
}

// Rows of 128 bf16 as 4 packed words per lane (lane gl of the 16-lane group
// holds values 8gl .. 8gl+7). Reorder values 0..63 from interleaved pairs to
// the half layout: value d < 32 comes from 2d, value 32 + d from 2d + 1.
// Destination lane j < 8, value i takes source value 16(j & 3) + 2i + (j >> 2),
// i.e. word (i & 3) of lane 2(j & 3) + (i >> 2), half (j >> 2).
__device__ __forceinline__ void interleaved_to_half(uint32_t w[4], int lane, int gl) {
  const int src = (lane & ~15) + 2 * (gl & 3);
  uint32_t a[4], b[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    a[q] = (uint32_t)__shfl((int)w[q], src, 64);
    b[q] = (uint32_t)__shfl((int)w[q], src + 1, 64);
  }
  if (gl < 8) {
    const int sh = (gl >> 2) * 16;
    const uint32_t v0 = (a[0] >> sh) & 0xffffu, v1 = (a[1] >> sh) & 0xffffu;
    const uint32_t v2 = (a[2] >> sh) & 0xffffu, v3 = (a[3] >> sh) & 0xffffu;
    const uint32_t v4 = (b[0] >> sh) & 0xffffu, v5 = (b[1] >> sh) & 0xffffu;
    const uint32_t v6 = (b[2] >> sh) & 0xffffu, v7 = (b[3] >> sh) & 0xffffu;
    w[0] = v0 | (v1 << 16);
    w[1] = v2 | (v3 << 16);
    w[2] = v4 | (v5 << 16);
    w[3] = v6 | (v7 << 16);
  }
}

__device__ __forceinline__ void unpack8(const uint32_t w[4], float x[8]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    x[2 * q] = __uint_as_float(w[q] << 16);
    x[2 * q + 1] = __uint_as_float(w[q] & 0xffff0000u);
  }
}

// NeoX rotation of values 0..63 (half layout) by cos/sin row `cs`; lanes 0-3
// hold the first halves x1, lanes 4-7 the second halves x2 of the same pairs:
//   y1 = x1 cos - x2 sin,  y2 = x2 cos + x1 sin.  Results rounded to bf16.
__device__ __forceinline__ void rope_neox(float x[8], const float* __restrict__ cs, int gl) {
#pragma clang fp contract(off)
  float other[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) other[i] = shfl_xor(x[i], 4);
  if (gl < 8) {
    const float* c = cs + 8 * (gl & 3);
    const v4f c0 = *reinterpret_cast<const v4f*>(c), c1 = *reinterpret_cast<const v4f*>(c + 4);
    const v4f s0 = *reinterpret_cast<const v4f*>(c + 32), s1 = *reinterpret_cast<const v4f*>(c + 36);
    const float cv[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
    const float sv[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
    if (gl < 4) {
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = bf16_round(x[i] * cv[i] - other[i] * sv[i]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = bf16_round(x[i] * cv[i] + other[i] * sv[i]);
    }
  }
}

// Unnormalised 128-point Walsh-Hadamard transform (natural order, H[o, i] =
// (-1)^popcount(o & i)), stages h = 1, 2, 4 in-lane then 8 .. 64 across lanes,
// each stage (a, b) -> (a + b, a - b); then times 128^-0.5.
__device__ __forceinline__ void hadamard128(float x[8], int gl) {
#pragma clang fp contract(off)
#pragma unroll
  for (int h = 1; h < 8; h <<= 1) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (i & h) continue;
      const float a = x[i], b = x[i + h];
      x[i] = a + b;
      x[i + h] = a - b;
    }
  }
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float o = shfl_xor(x[i], m);
      x[i] = (gl & m) ? (o - x[i]) : (x[i] + o);
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = x[i] * kInvSqrt128;
}

// Sum over the row's 128 values: in-lane tree (i, i+4), (i, i+2), (i, i+1),
// then a butterfly over lanes xor 1, 2, 4, 8. Every lane of the group gets it.
__device__ __forceinline__ float row_sum(const float x[8]) {
#pragma clang fp contract(off)
  const float a0 = x[0] + x[4], a1 = x[1] + x[5], a2 = x[2] + x[6], a3 = x[3] + x[7];
  const float b0 = a0 + a2, b1 = a1 + a3;
  float s = b0 + b1;
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) s = s + shfl_xor(s, m);
  return s;
}

// Per-row UE8M0 quantisation: returns the scale and packs 8 e4m3fn codes.
__device__ __forceinline__ float quant_row(const float x[8], uint2& codes) {
  float amax = fabsf(x[0]);
#pragma unroll
  for (int i = 1; i < 8; ++i) amax = fmaxf(amax, fabsf(x[i]));
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) amax = fmaxf(amax, shfl_xor(amax, m));
  const float sf = pow2_ceil(fmaxf(amax, 1e-4f) / 448.f);
  const float inv = 1.f / sf;  // exact: sf is a power of two
  codes.x = f32x4_to_fp8(x[0] * inv, x[1] * inv, x[2] * inv, x[3] * inv);
  codes.y = f32x4_to_fp8(x[4] * inv, x[5] * inv, x[6] * inv, x[7] * inv);
  return sf;
}

__global__ void __launch_bounds__(256)
indexer_q_prologue_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ gate, int64_t gate_stride,
                          float weight_scale, const float* __restrict__ cos_sin, int64_t cache_positions,
                          const void* __restrict__ positions, int pos_is_64, int num_heads, int rows,
                          int interleaved, uint8_t* __restrict__ q_fp8, float* __restrict__ weights_out) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int gl = threadIdx.x & 15;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 4);
  if (row >= rows) return;  // whole 16-lane groups leave together
  const int tok = row / num_heads;
  const int head = row - tok * num_heads;
  const v4i raw = *reinterpret_cast<const v4i*>(q + (int64_t)row * 128 + 8 * gl);
  uint32_t w[4] = {(uint32_t)raw[0], (uint32_t)raw[1], (uint32_t)raw[2], (uint32_t)raw[3]};
  if (interleaved) interleaved_to_half(w, lane, gl);
  float x[8];
  unpack8(w, x);
  int64_t pos = load_index(positions, pos_is_64, tok);
  pos = pos < 0 ? 0 : (pos >= cache_positions ? cache_positions - 1 : pos);  // keep the read in bounds
  rope_neox(x, cos_sin + pos * 64, gl);
  hadamard128(x, gl);
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = bf16_round(x[i]);
  uint2 codes;
  const float sf = quant_row(x, codes);
  *reinterpret_cast<uint2*>(q_fp8 + (int64_t)row * 128 + 8 * gl) = codes;
  if (gl == 0) {
    const float g = bf16_to_f32(gate[(int64_t)tok * gate_stride + head]);
    weights_out[row] = g * weight_scale * sf;
  }
}

__global__ void __launch_bounds__(256)
indexer_k_transform_store_kernel(const uint16_t* __restrict__ key, int64_t key_stride,
                                 const float* __restrict__ ln_w, const float* __restrict__ ln_b, float eps,
                                 const float* __restrict__ cos_sin, int64_t cache_positions,
                                 const void* __restrict__ positions, int pos_is_64, const void* __restrict__ slots,
                                 int slot_is_64, int num_tokens, uint8_t* __restrict__ cache, int page_size) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int gl = threadIdx.x & 15;
  const int tok = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 4);
  if (tok >= num_tokens) return;
  const int64_t slot = load_index(slots, slot_is_64, tok);
  if (slot < 0) return;  // padded token: nothing to store
  const v4i raw = *reinterpret_cast<const v4i*>(key + (int64_t)tok * key_stride + 8 * gl);
  float x[8];
  {
    const uint32_t w[4] = {(uint32_t)raw[0], (uint32_t)raw[1], (uint32_t)raw[2], (uint32_t)raw[3]};
    unpack8(w, x);
  }
  // LayerNorm over the 128 values (biased variance), output rounded to bf16
  const float mean = row_sum(x) * (1.f / 128.f);
  float c[8], sq[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    c[i] = x[i] - mean;
    sq[i] = c[i] * c[i];
  }
  const float var = row_sum(sq) * (1.f / 128.f);
  const float inv_std = 1.f / sqrtf(var + eps);
  const v4f w0 = *reinterpret_cast<const v4f*>(ln_w + 8 * gl), w1 = *reinterpret_cast<const v4f*>(ln_w + 8 * gl + 4);
  const v4f b0 = *reinterpret_cast<const v4f*>(ln_b + 8 * gl), b1 = *reinterpret_cast<const v4f*>(ln_b + 8 * gl + 4);
  const float wv[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
  const float bv[8] = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
  uint32_t w[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float y0 = (c[2 * q] * inv_std) * wv[2 * q] + bv[2 * q];
    const float y1 = (c[2 * q + 1] * inv_std) * wv[2 * q + 1] + bv[2 * q + 1];
    w[q] = pack_bf16_rne(y0, y1);
  }
  // the projection's rope dims are interleaved pairs (indexer_transform.py:183-186)
  interleaved_to_half(w, lane, gl);
  unpack8(w, x);
  int64_t pos = load_index(positions, pos_is_64, tok);
  pos = pos < 0 ? 0 : (pos >= cache_positions ? cache_positions - 1 : pos);
  rope_neox(x, cos_sin + pos * 64, gl);
  hadamard128(x, gl);
  uint2 codes;
  const float sf = quant_row(x, codes);
  const int64_t page = slot / page_size, off = slot - page * page_size;
  uint8_t* base = cache + page * (int64_t)page_size * 132;
  *reinterpret_cast<uint2*>(base + off * 128 + 8 * gl) = codes;
  if (gl == 0) reinterpret_cast<float*>(base + (int64_t)page_size * 128)[off] = sf;
}

}  // namespace
}  // namespace dsa

extern "C" {

int dsa_indexer_q_prologue(const void* q, const void* gate, int64_t gate_token_stride, float weight_scale,
                           const float* cos_sin_cache, int64_t cache_positions, const void* positions, int pos_is_64,
                           int num_tokens, int num_heads, int rope_interleaved, uint8_t* q_fp8, float* weights_out,
                           void* stream) {
  using namespace dsa;
  if (num_tokens < 0 || num_heads <= 0 || cache_positions <= 0 || gate_token_stride < num_heads)
    return set_error(kInvalidArgument, "dsa_indexer_q_prologue: bad sizes");
  if (num_tokens == 0) return kOk;
  if (!q || !gate || !cos_sin_cache || !positions || !q_fp8 || !weights_out)
    return set_error(kInvalidArgument, "dsa_indexer_q_prologue: null pointer");
  if ((reinterpret_cast<uintptr_t>(q) & 15) || (reinterpret_cast<uintptr_t>(cos_sin_cache) & 15) ||
      (reinterpret_cast<uintptr_t>(q_fp8) & 7) || (reinterpret_cast<uintptr_t>(gate) & 1) ||
      (reinterpret_cast<uintptr_t>(weights_out) & 3))
    return set_error(kInvalidArgument,
                     "dsa_indexer_q_prologue: q and cos_sin_cache must be 16-byte aligned, q_fp8 8-byte aligned");
  const int64_t rows = (int64_t)num_tokens * num_heads;
  if (rows > INT32_MAX - kRowsPerBlock) return set_error(kInvalidArgument, "dsa_indexer_q_prologue: too many rows");
  hipLaunchKernelGGL(indexer_q_prologue_kernel, dim3((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock)),
                     dim3(256), 0, (hipStream_t)stream, static_cast<const uint16_t*>(q),
                     static_cast<const uint16_t*>(gate), gate_token_stride, weight_scale, cos_sin_cache,
                     cache_positions, positions, pos_is_64, num_heads, (int)rows, rope_interleaved, q_fp8,
                     weights_out);
  return check_launch("dsa_indexer_q_prologue");
}

int dsa_indexer_k_transform_store(const void* key, int64_t key_row_stride, const float* ln_weight,
                                  const float* ln_bias, float eps, const float* cos_sin_cache, int64_t cache_positions,
                                  const void* positions, int pos_is_64, const void* slots, int slot_is_64,
                                  int num_tokens, uint8_t* cache, int page_size, void* stream) {
  using namespace dsa;
  if (num_tokens < 0 || page_size <= 0 || cache_positions <= 0 || key_row_stride < 128)
    return set_error(kInvalidArgument, "dsa_indexer_k_transform_store: bad sizes");
  if (num_tokens == 0) return kOk;
  if (!key || !ln_weight || !ln_bias || !cos_sin_cache || !positions || !slots || !cache)
    return set_error(kInvalidArgument, "dsa_indexer_k_transform_store: null pointer");
  if ((reinterpret_cast<uintptr_t>(key) & 15) || (key_row_stride % 8) ||
      (reinterpret_cast<uintptr_t>(ln_weight) & 15) || (reinterpret_cast<uintptr_t>(ln_bias) & 15) ||
      (reinterpret_cast<uintptr_t>(cos_sin_cache) & 15) || (reinterpret_cast<uintptr_t>(cache) & 7))
    return set_error(kInvalidArgument,
                     "dsa_indexer_k_transform_store: key rows, LayerNorm parameters and cos_sin_cache must be "
                     "16-byte aligned, the cache 8-byte aligned");
  hipLaunchKernelGGL(indexer_k_transform_store_kernel, dim3((num_tokens + kRowsPerBlock - 1) / kRowsPerBlock),
                     dim3(256), 0, (hipStream_t)stream, static_cast<const uint16_t*>(key), key_row_stride, ln_weight,
                     ln_bias, eps, cos_sin_cache, cache_positions, positions, pos_is_64, slots, slot_is_64,
                     num_tokens, cache, page_size);
  return check_launch("dsa_indexer_k_transform_store");
}

}  // extern "C"
