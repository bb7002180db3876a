// Sparse MLA decode over the packed fp8 MLA cache, for gfx950.
//
// For each query token t and head h:
//   s_i = sm_scale * q[t,h,:576] . kv(idx_i)[:576]     (valid idx_i only)
//   o   = softmax(s) @ kv(idx)[:, :512],  lse = log(sum_i exp(s_i))
// where kv(slot) is a 656-byte row [512 e4m3fn][4 x f32 tile scale][64 bf16].
//
// Workgroup = 4 waves = 64 heads of one token over one key split; each wave
// owns 16 heads. Per block of 64 selected rows:
//   load   : lane = row; wave w gathers tile w of the 64 rows (8 x 16 B fp8 +
//            its f32 scale) and two 16 B rope chunks, a full block of compute
//            ahead of use (the row indices one block further ahead);
//   stage  : rows are dequantised in registers (fp8 * 2^k is exact in bf16,
//            one v_cvt_scalef32_pk_bf16_fp8 per pair) and written once,
//            row-major, into one of two LDS buffers [64][576] bf16 (double
//            buffering: one barrier per block), between the QK MFMAs;
//   QK     : S^T[64 keys x 16 heads] on v_mfma_f32_16x16x32_bf16, A = rows
//            from LDS (four independent accumulator chains), B = the wave's
//            16 query heads, resident in registers for the whole kernel;
//   softmax: online in the exp2 domain, with lazy rescaling: the running max
//            only moves (and O is only rescaled) when a block raises it by
//            more than 2^8, so P stays in [0, 256] and the rescale is rare;
//   PV     : O[16 heads x 512] += P . V, A = P straight from the QK
//            accumulators (two 16-key C tiles form one 32-key A operand), B =
//            V read from the same row-major LDS tile with ds_read_b64_tr_b16,
//            which hands each 16-lane group a transposed 4-key x 16-dv tile -
//            no separate transposed copy of V.
// Splits over the key list (for small batches) write normalised partial
// outputs and LSEs to a caller-provided workspace; a combine kernel merges
// them with the LSE rule of merge_attention_states.
#include <cmath>

#include "dsa_common.h"
#include "../../include/dsa_amd.h"

namespace dsa {

typedef short v4s __attribute__((ext_vector_type(4)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

constexpr int kMlaThreads = 256;
constexpr int kMlaHeadsPerWG = 64;
constexpr int kMlaKeys = 64;            // rows per block
constexpr int kMlaRowBytes = 656;
constexpr int kMlaDqk = 576;
constexpr int kMlaDv = 512;
// Staged row pitch: 576 bf16 + 32 B. 296 dwords is an odd multiple of 8
// banks, so 8 consecutive rows' 32-byte segments cover all 64 banks.
constexpr int kPitch = kMlaDqk * 2 + 32;
constexpr int kBufBytes = kMlaKeys * kPitch;
constexpr size_t kMlaSmemBytes = 2 * (size_t)kBufBytes;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kRescaleThreshold = 8.0f;  // log2 units

struct MlaParams {
  const uint16_t* q;
  int64_t q_tok_stride, q_head_stride;
  const uint8_t* kv;
  int64_t kv_blk_stride;
  int kv_block_size;
  const int32_t* idx;
  int64_t idx_stride;
  int T, H, topk, splits, head_groups;
  float scale_log2;
  uint16_t* out;
  float* lse;
  float* ws_o;    // [splits, T, H, 512] (splits > 1)
  float* ws_lse;  // [splits, T, H]
};

struct RowRegs {
  v4i nope[8];   // this wave's 128-dim tile of the lane's row
  v4i rope[2];   // rope chunks 2w, 2w+1
  float scale;
  bool valid;
};

__device__ __forceinline__ int32_t load_slot(const MlaParams& P, int t, int key0, int lane) {
  return P.idx[(int64_t)t * P.idx_stride + key0 + lane];
}

// Gather this wave's share of the lane's row (`slot` < 0: an invalid index, zeros).
__device__ __forceinline__ void load_rows(RowRegs& rr, const MlaParams& P, int32_t slot, int wave) {
  rr.valid = slot >= 0;
  if (rr.valid) {
    const uint8_t* row = P.kv + (int64_t)(slot / P.kv_block_size) * P.kv_blk_stride +
                         (int64_t)(slot % P.kv_block_size) * kMlaRowBytes;
    const v4i* nope = reinterpret_cast<const v4i*>(row + wave * 128);
#pragma unroll
    for (int i = 0; i < 8; ++i) rr.nope[i] = nope[i];
    rr.scale = reinterpret_cast<const float*>(row + 512)[wave];
    const v4i* rope = reinterpret_cast<const v4i*>(row + 528 + wave * 32);
    rr.rope[0] = rope[0];
    rr.rope[1] = rope[1];
  } else {
    const v4i z = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 8; ++i) rr.nope[i] = z;
    rr.rope[0] = z;
    rr.rope[1] = z;
    rr.scale = 0.f;
  }
}

// Stage piece i (0-7: a 16-dim nope chunk of the wave's tile; 8: the wave's
// two rope chunks) of the lane's row into the bf16 tile.
__device__ __forceinline__ void stage_piece(const RowRegs& rr, uint8_t* buf, int lane, int wave, int i) {
  uint8_t* krow = buf + lane * kPitch;
  if (i < 8) {
    const int c = wave * 8 + i;  // dims 16c .. 16c+15
    v4i lo, hi;
    dequant16_fp8_bf16(rr.nope[i], rr.scale, lo, hi);
    *reinterpret_cast<v4i*>(krow + c * 32) = lo;
    *reinterpret_cast<v4i*>(krow + c * 32 + 16) = hi;
  } else {
    *reinterpret_cast<v4i*>(krow + 1024 + wave * 32) = rr.rope[0];
    *reinterpret_cast<v4i*>(krow + 1024 + wave * 32 + 16) = rr.rope[1];
  }
}

__device__ __forceinline__ void stage_rows(const RowRegs& rr, uint8_t* buf, int lane, int wave) {
#pragma unroll
  for (int i = 0; i < 9; ++i) stage_piece(rr, buf, lane, wave, i);
}

__device__ __forceinline__ v8bf as_v8bf(v4i x) { return __builtin_bit_cast(v8bf, x); }

__device__ __forceinline__ int cvt_pk_bf16(float a, float b) {
  const v2f x = {a, b};
  return __builtin_bit_cast(int, __builtin_convertvector(x, v2bf));
}

__device__ __forceinline__ v4s lds_read_tr16(const uint8_t* p) {
  typedef __attribute__((address_space(3))) v4s lds_v4s;
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)p);
}

__global__ void __launch_bounds__(kMlaThreads)
sparse_mla_kernel(const MlaParams P) {
  extern __shared__ __align__(16) uint8_t smem[];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, c16 = lane & 15;

  // XCD-aware order: consecutive logical work items (the head groups and
  // splits of one token) land on the same XCD and share its L2.
  const int nwg = gridDim.x;
  int work = blockIdx.x;
  if ((nwg & 7) == 0) work = (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3);
  const int per_tok = P.head_groups * P.splits;
  const int t = work / per_tok;
  const int rem = work % per_tok;
  const int hg = rem / P.splits;
  const int split = rem % P.splits;
  const int chunk = P.topk / P.splits;
  const int key_begin = split * chunk;
  const int nblk = chunk / kMlaKeys;

  const int h0 = hg * kMlaHeadsPerWG + wave * 16;
  const bool active = h0 < P.H;

  // Query heads as B operands of S^T = K . Q^T: head h0 + lane%16, dims ks*32 + g*8 .. +8.
  v4i qb[18];
  if (active) {
    const uint16_t* qh = P.q + (int64_t)t * P.q_tok_stride + (int64_t)(h0 + c16) * P.q_head_stride + g * 8;
#pragma unroll
    for (int ks = 0; ks < 18; ++ks) qb[ks] = *reinterpret_cast<const v4i*>(qh + ks * 32);
  }

  // o[dt][r]: head h0 + 4g + r, dv dt*16 + c16
  v4f o[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) o[i] = (v4f){0.f, 0.f, 0.f, 0.f};
  float m_run = -__builtin_inff();  // per head c16, log2 domain
  float l_run = 0.f;                // per head c16, this lane's keys only

  // Pipeline: block n is multiplied from LDS while block n+1 (in registers)
  // is staged into the other buffer and block n+2's rows are in flight; the
  // row indices run one block further ahead.
  RowRegs rr;
  load_rows(rr, P, load_slot(P, t, key_begin, lane), wave);
  int32_t slot_pf = nblk > 1 ? load_slot(P, t, key_begin + kMlaKeys, lane) : -1;
  uint64_t vm_cur = __ballot(rr.valid);
  stage_rows(rr, smem, lane, wave);
  if (nblk > 1) load_rows(rr, P, slot_pf, wave);
  if (nblk > 2) slot_pf = load_slot(P, t, key_begin + 2 * kMlaKeys, lane);
  __syncthreads();

  for (int n = 0; n < nblk; ++n) {
    const uint8_t* buf = smem + (n & 1) * kBufBytes;
    uint8_t* next_buf = smem + ((n + 1) & 1) * kBufBytes;
    const bool stage_next = n + 1 < nblk;
    const uint64_t vm_next = stage_next ? __ballot(rr.valid) : 0ull;
    if (active && vm_cur) {
      // ---- S^T = K . Q^T: s[kt][r] = score(key kt*16 + 4g + r, head c16).
      // A operands are read two k-steps ahead of their MFMAs.
      v4f s[4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) s[kt] = (v4f){0.f, 0.f, 0.f, 0.f};
      const uint8_t* arow = buf + c16 * kPitch + g * 16;
      v4i a[3][4];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) a[ks][kt] = *reinterpret_cast<const v4i*>(arow + kt * 16 * kPitch + ks * 64);
#pragma unroll
      for (int ks = 0; ks < 18; ++ks) {
        if (ks + 2 < 18) {
#pragma unroll
          for (int kt = 0; kt < 4; ++kt)
            a[(ks + 2) % 3][kt] = *reinterpret_cast<const v4i*>(arow + kt * 16 * kPitch + (ks + 2) * 64);
        }
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
          s[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(a[ks % 3][kt]), as_v8bf(qb[ks]), s[kt], 0, 0, 0);
        if (stage_next && (ks & 1)) stage_piece(rr, next_buf, lane, wave, ks >> 1);
      }
      // block n+1 is staged: its registers take block n+2's rows now, which
      // leaves them a whole block of compute to arrive
      if (n + 2 < nblk) {
        load_rows(rr, P, slot_pf, wave);
        if (n + 3 < nblk) slot_pf = load_slot(P, t, key_begin + (n + 3) * kMlaKeys, lane);
      }

      // ---- online softmax (exp2 domain), lazy rescale
      float mloc = -__builtin_inff();
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = kt * 16 + g * 4 + r;
          const float x = ((vm_cur >> key) & 1ull) ? s[kt][r] * P.scale_log2 : -__builtin_inff();
          s[kt][r] = x;
          mloc = fmaxf(mloc, x);
        }
      mloc = fmaxf(mloc, shfl_xor(mloc, 16));
      mloc = fmaxf(mloc, shfl_xor(mloc, 32));
      const bool need = mloc > m_run + kRescaleThreshold;  // true on the first valid block
      if (__ballot(need)) {
        const float m_new = need ? mloc : m_run;
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 when m_run = -inf
        l_run *= alpha;
        m_run = m_new;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float ar = __shfl(alpha, g * 4 + r, 64);
#pragma unroll
          for (int dt = 0; dt < 32; ++dt) o[dt][r] *= ar;
        }
      }
      float psum = 0.f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pv = __builtin_amdgcn_exp2f(s[kt][r] - m_run);
          s[kt][r] = pv;
          psum += pv;
        }
      l_run += psum;

      // ---- O += P . V, V operands two tiles ahead
      v4i pa[2];
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        pa[kk][0] = cvt_pk_bf16(s[2 * kk][0], s[2 * kk][1]);
        pa[kk][1] = cvt_pk_bf16(s[2 * kk][2], s[2 * kk][3]);
        pa[kk][2] = cvt_pk_bf16(s[2 * kk + 1][0], s[2 * kk + 1][1]);
        pa[kk][3] = cvt_pk_bf16(s[2 * kk + 1][2], s[2 * kk + 1][3]);
      }
      // lane (g, c16) addresses key row 4g + c16/4 (+16, +32, +48), dv 4*(c16%4) of each 16-dv tile
      const uint8_t* vb = buf + (4 * g + (c16 >> 2)) * kPitch + (c16 & 3) * 8;
      v4s vv[3][4];
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int q = 0; q < 4; ++q) vv[dt][q] = lds_read_tr16(vb + q * 16 * kPitch + dt * 32);
#pragma unroll
      for (int dt = 0; dt < 32; ++dt) {
        if (dt + 2 < 32) {
#pragma unroll
          for (int q = 0; q < 4; ++q) vv[(dt + 2) % 3][q] = lds_read_tr16(vb + q * 16 * kPitch + (dt + 2) * 32);
        }
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const v8bf bop = __builtin_bit_cast(
              v8bf, __builtin_shufflevector(vv[dt % 3][2 * kk], vv[dt % 3][2 * kk + 1], 0, 1, 2, 3, 4, 5, 6, 7));
          o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(pa[kk]), bop, o[dt], 0, 0, 0);
        }
      }
    } else {
      if (stage_next) stage_rows(rr, next_buf, lane, wave);
      if (n + 2 < nblk) {
        load_rows(rr, P, slot_pf, wave);
        if (n + 3 < nblk) slot_pf = load_slot(P, t, key_begin + (n + 3) * kMlaKeys, lane);
      }
    }
    __syncthreads();
    vm_cur = vm_next;
  }

  if (!active) return;
  l_run += shfl_xor(l_run, 16);
  l_run += shfl_xor(l_run, 32);
  const bool any = l_run > 0.f;
  const float inv = any ? 1.f / l_run : 0.f;
  const float lse = any ? (m_run + __builtin_amdgcn_logf(l_run)) * kLn2 : -__builtin_inff();
  float inv_r[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) inv_r[r] = __shfl(inv, g * 4 + r, 64);

  if (P.splits == 1) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      uint16_t* orow = P.out + ((int64_t)t * P.H + h0 + g * 4 + r) * kMlaDv + c16;
#pragma unroll
      for (int dt = 0; dt < 32; ++dt) orow[dt * 16] = (uint16_t)f32_to_bf16_rne(o[dt][r] * inv_r[r]);
    }
    if (g == 0 && P.lse) P.lse[(int64_t)t * P.H + h0 + c16] = lse;
  } else {
    const int64_t row0 = ((int64_t)split * P.T + t) * P.H + h0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float* orow = P.ws_o + (row0 + g * 4 + r) * kMlaDv + c16;
#pragma unroll
      for (int dt = 0; dt < 32; ++dt) orow[dt * 16] = o[dt][r] * inv_r[r];
    }
    if (g == 0) P.ws_lse[row0 + c16] = lse;
  }
}

// One 64-thread workgroup per (token, head): merge the split partials.
__global__ void __launch_bounds__(64)
sparse_mla_combine_kernel(const float* __restrict__ ws_o, const float* __restrict__ ws_lse, int T, int H,
                          int splits, uint16_t* __restrict__ out, float* __restrict__ lse_out) {
  const int th = blockIdx.x;
  const int64_t stride = (int64_t)T * H;
  float m = -__builtin_inff();
  for (int s = 0; s < splits; ++s) m = fmaxf(m, ws_lse[s * stride + th]);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float wsum = 0.f;
  if (m != -__builtin_inff()) {
    for (int s = 0; s < splits; ++s) {
      const float l = ws_lse[s * stride + th];
      const float w = __expf(l - m);
      wsum += w;
      const v4f* src = reinterpret_cast<const v4f*>(ws_o + (s * stride + th) * kMlaDv + threadIdx.x * 8);
      const v4f a = src[0], b = src[1];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[e] = fmaf(w, a[e], acc[e]);
        acc[4 + e] = fmaf(w, b[e], acc[4 + e]);
      }
    }
  }
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
  v4i v;
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = (int)pack_bf16_rne(acc[2 * e] * inv, acc[2 * e + 1] * inv);
  *reinterpret_cast<v4i*>(out + (int64_t)th * kMlaDv + threadIdx.x * 8) = v;
  if (threadIdx.x == 0 && lse_out) lse_out[th] = wsum > 0.f ? m + logf(wsum) : -__builtin_inff();
}

}  // namespace dsa

extern "C" {

int dsa_sparse_mla_num_splits(int num_tokens, int num_heads, int topk, int num_cus) {
  if (num_tokens <= 0 || num_heads <= 0 || topk <= 0) return 1;
  if (num_cus <= 0) num_cus = 256;
  const int groups = (num_heads + dsa::kMlaHeadsPerWG - 1) / dsa::kMlaHeadsPerWG;
  const int64_t base = (int64_t)num_tokens * groups;
  int splits = 1;
  const int max_splits = topk / dsa::kMlaKeys;
  // grow until the grid covers the CUs once; splits must divide topk into 64-row blocks
  while (base * splits < num_cus && splits * 2 <= max_splits && (topk / (splits * 2)) % dsa::kMlaKeys == 0)
    splits *= 2;
  return splits;
}

size_t dsa_sparse_mla_workspace_bytes(int num_tokens, int num_heads, int num_splits) {
  if (num_splits <= 1 || num_tokens <= 0 || num_heads <= 0) return 0;
  const size_t rows = (size_t)num_splits * num_tokens * num_heads;
  return rows * dsa::kMlaDv * sizeof(float) + rows * sizeof(float);
}

int dsa_sparse_mla_decode(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                          const uint8_t* kv_cache, int64_t kv_block_stride_bytes, int kv_block_size,
                          const int32_t* indices, int64_t idx_stride, int num_tokens, int num_heads,
                          int topk, float sm_scale, void* out, float* lse, int num_splits, void* workspace,
                          size_t workspace_bytes, void* stream) {
  using namespace dsa;
  if (num_tokens < 0 || num_heads <= 0 || (num_heads % 16) != 0)
    return set_error(kUnsupported, "sparse_mla: num_heads=%d must be a positive multiple of 16", num_heads);
  if (topk <= 0 || topk % kMlaKeys != 0)
    return set_error(kUnsupported, "sparse_mla: topk=%d must be a positive multiple of %d", topk, kMlaKeys);
  if (kv_block_size <= 0 || kv_block_stride_bytes < (int64_t)kv_block_size * kMlaRowBytes)
    return set_error(kInvalidArgument, "sparse_mla: kv block stride %lld < %d rows x 656 B",
                     (long long)kv_block_stride_bytes, kv_block_size);
  if (kv_block_stride_bytes % 16 != 0)
    return set_error(kInvalidArgument, "sparse_mla: kv block stride must be a multiple of 16 bytes");
  if (num_tokens == 0) return kOk;
  if (!q || !kv_cache || !indices || !out)
    return set_error(kInvalidArgument, "sparse_mla: null pointer");
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(kv_cache) |
       reinterpret_cast<uintptr_t>(out)) & 15)
    return set_error(kInvalidArgument, "sparse_mla: q, kv_cache and out must be 16-byte aligned");
  if ((q_token_stride % 8) || (q_head_stride % 8))
    return set_error(kInvalidArgument, "sparse_mla: q strides must be multiples of 8 elements");
  if (num_splits <= 0) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    num_splits = dsa_sparse_mla_num_splits(num_tokens, num_heads, topk, dsa_num_cus(dev));
  }
  if (num_splits > topk / kMlaKeys || (topk / num_splits) % kMlaKeys != 0 || topk % num_splits != 0)
    return set_error(kInvalidArgument, "sparse_mla: num_splits=%d does not split topk=%d into 64-row blocks",
                     num_splits, topk);
  const size_t need = dsa_sparse_mla_workspace_bytes(num_tokens, num_heads, num_splits);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return set_error(kWorkspaceTooSmall, "sparse_mla: workspace %zu B < %zu B", workspace_bytes, need);

  static int smem_status = -1;
  if (smem_status < 0) {
    smem_status = hipFuncSetAttribute((const void*)sparse_mla_kernel,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMlaSmemBytes) == hipSuccess
                      ? 0 : 1;
  }
  if (smem_status) return set_error(kLaunchFailed, "sparse_mla: cannot reserve %zu B of LDS", kMlaSmemBytes);

  MlaParams P;
  P.q = static_cast<const uint16_t*>(q);
  P.q_tok_stride = q_token_stride;
  P.q_head_stride = q_head_stride;
  P.kv = kv_cache;
  P.kv_blk_stride = kv_block_stride_bytes;
  P.kv_block_size = kv_block_size;
  P.idx = indices;
  P.idx_stride = idx_stride;
  P.T = num_tokens;
  P.H = num_heads;
  P.topk = topk;
  P.splits = num_splits;
  P.head_groups = (num_heads + kMlaHeadsPerWG - 1) / kMlaHeadsPerWG;
  P.scale_log2 = sm_scale * kLog2e;
  P.out = static_cast<uint16_t*>(out);
  P.lse = lse;
  P.ws_o = nullptr;
  P.ws_lse = nullptr;
  if (num_splits > 1) {
    const size_t rows = (size_t)num_splits * num_tokens * num_heads;
    P.ws_o = static_cast<float*>(workspace);
    P.ws_lse = P.ws_o + rows * kMlaDv;
  }
  const int64_t nwg = (int64_t)num_tokens * P.head_groups * num_splits;
  hipLaunchKernelGGL(sparse_mla_kernel, dim3((unsigned)nwg), dim3(kMlaThreads), kMlaSmemBytes,
                     (hipStream_t)stream, P);
  if (int rc = check_launch("dsa_sparse_mla_decode")) return rc;
  if (num_splits > 1) {
    hipLaunchKernelGGL(sparse_mla_combine_kernel, dim3((unsigned)(num_tokens * num_heads)), dim3(64), 0,
                       (hipStream_t)stream, P.ws_o, P.ws_lse, num_tokens, num_heads, num_splits, P.out, lse);
    return check_launch("dsa_sparse_mla_decode(combine)");
  }
  return kOk;
}

}  // extern "C"
