// Sparse MLA prefill over ragged bf16 KV rows, for gfx950.
//
// For each query token t and head h:
//   s_i = sm_scale * q[t,h,:576] . kv[idx_i, :576]     (0 <= idx_i < s_kv only)
//   o   = softmax(s) @ kv[idx, :512],  lse = log(sum_i exp(s_i)),  max_logits = max_i s_i
// where kv is [s_kv, 576] bf16 (the ragged cached + fresh keys of a chunked
// prefill) and idx [topk] are packed logical indices into it.
//
// Workgroup = 8 waves (two per SIMD) = 64 heads of one token. Wave w = (head
// half hp = w/4, quarter q = w%4); its 32 heads are hp*32 + 0..31 of the
// workgroup's 64. Per block of 32 selected rows:
//   gather : the 1152-byte rows go straight from L2/HBM into LDS with
//            global_load_lds_dwordx4, three buffers, two blocks ahead. A block
//            is stored piece-major, [72 16-byte pieces][32 rows]: one load
//            instruction moves pieces 2i and 2i+1 of all 32 rows, and every
//            operand read below touches consecutive rows of one piece, so the
//            K reads are conflict-free. Invalid indices read a zero row.
//   QK     : wave q forms the partial S^T[32 keys x 32 heads] over nope dims
//            [128q, 128q+128) and rope dims [512+16q, 512+16q+16) on
//            v_mfma_f32_32x32x16_bf16 (A = rows from LDS, B = the wave's
//            query slice, resident in registers).
//   reduce : a four-way reduce-scatter through LDS leaves wave q with the full
//            scores of keys 8q .. 8q+7, so each score is exponentiated once.
//   softmax: per-head block maxima of the four key quarters are exchanged;
//            online softmax in the exp2 domain with lazy rescaling (the running
//            max moves only when a block raises it by more than 2^8). P goes
//            to LDS once, as bf16.
//   PV     : wave q produces output dims [128q, 128q+128) of its 32 heads:
//            O += P . V on v_mfma_f32_32x32x16_bf16, V read with
//            ds_read_b64_tr_b16 (each 16-lane group gets a transposed
//            4-key x 16-dim tile: the B operand layout).
#include <cmath>

#include "dsa_common.h"
#include "../../include/dsa_amd.h"

namespace dsa {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));

constexpr int kPrThreads = 512;
constexpr int kPrWaves = kPrThreads / 64;
constexpr int kPrHeadsPerWG = 64;
constexpr int kPrKeys = 32;                          // rows per block
constexpr int kPrDqk = 576;
constexpr int kPrDv = 512;
constexpr int kPrRowBytes = kPrDqk * 2;              // 1152
constexpr int kPrPieces = kPrRowBytes / 16;          // 72
constexpr int kPrBufBytes = kPrKeys * kPrRowBytes;   // 36864
constexpr int kPrDmaPerBlock = kPrBufBytes / 1024;   // 36 wave-wide loads per block
constexpr int kPrNumBufs = 3;
constexpr int kPrXsOff = kPrNumBufs * kPrBufBytes;           // partial scores [8 waves][4 quarters][64 lanes][4 f32]
constexpr int kPrMxOff = kPrXsOff + kPrWaves * 4 * 1024;     // block maxima / sums [2 hp][32 heads][4 quarters]
constexpr int kPrPOff = kPrMxOff + 2 * 32 * 4 * 4;           // P [2 hp][4 quarters][64 lanes][4 bf16]
constexpr int kPrRingOff = kPrPOff + 2 * 4 * 64 * 8;         // row indices, one 32-entry block per slot
constexpr int kPrRingSlots = 5;
constexpr size_t kPrSmemBytes = kPrRingOff + kPrRingSlots * 128;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kRescaleThreshold = 8.0f;  // log2 units
constexpr int kIdxWave = 7;                // the wave that fetches the row indices

static_assert(kPrBufBytes % 1024 == 0 && kPrPieces % 2 == 0, "a block of rows must be whole wave-wide loads");
static_assert(kPrSmemBytes <= 160 * 1024, "LDS budget");

// Source of the pieces of an invalid row: 1152 zero bytes.
__device__ __align__(16) uint8_t g_prefill_zero_row[kPrRowBytes];

struct PrParams {
  const uint16_t* q;
  int64_t q_tok_stride, q_head_stride;  // elements
  const uint16_t* kv;
  int64_t kv_row_stride;                // elements
  int64_t s_kv;
  const int32_t* idx;
  int64_t idx_stride;
  int T, H, topk, head_groups;
  float scale_log2;
  uint16_t* out;
  float* max_logits;
  float* lse;
};

__device__ __forceinline__ void dma4(const void* g, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}
__device__ __forceinline__ void barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)reinterpret_cast<uintptr_t>(p); }
__device__ __forceinline__ v8bf as_v8bf(v4i x) { return __builtin_bit_cast(v8bf, x); }

__device__ __forceinline__ int cvt_pk_bf16(float a, float b) {
  const v2f x = {a, b};
  typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(int, __builtin_convertvector(x, v2bf));
}

__device__ __forceinline__ v2i lds_read_tr16_at(uint32_t a) {
  typedef __attribute__((address_space(3))) v4s lds_v4s;
  return __builtin_bit_cast(v2i, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(uintptr_t)a));
}

// Loads of a block: wave w sends loads [first(w), first(w) + count(w)) of the
// block's 36, five for waves 0-3 and four for waves 4-7.
__device__ __forceinline__ int dma_count(int wave) {
  return kPrDmaPerBlock / kPrWaves + (wave < kPrDmaPerBlock % kPrWaves ? 1 : 0);
}
__device__ __forceinline__ int dma_first(int wave) {
  return wave * (kPrDmaPerBlock / kPrWaves) + min(wave, kPrDmaPerBlock % kPrWaves);
}
static_assert(kPrDmaPerBlock / kPrWaves == 4 && kPrDmaPerBlock % kPrWaves == 4, "wait counts assume 5 / 4 loads");

// Wait until at most n of this wave's copies are outstanding (n in {0, 4, 5, 6}).
__device__ __forceinline__ void wait_vm(int n) {
  if (n >= 6) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
  else if (n == 5) asm volatile("s_waitcnt vmcnt(5)" ::: "memory");
  else if (n == 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Send this wave's loads of block j into buffer `buf`. Load i covers LDS bytes
// [1024 i, 1024 i + 1024) of the block = pieces 2i and 2i + 1: lane l copies
// piece 2i + l/32 of row l%32.
__device__ __forceinline__ void issue_rows(const PrParams& P, const uint8_t* smem, int j, const uint8_t* buf,
                                           int lane, int wave) {
  const int32_t slot = reinterpret_cast<const int32_t*>(smem + kPrRingOff + (j % kPrRingSlots) * 128)[lane & 31];
  const bool ok = slot >= 0 && (int64_t)slot < P.s_kv;
  const uint64_t rowp = ok ? reinterpret_cast<uint64_t>(P.kv + (int64_t)slot * P.kv_row_stride)
                           : reinterpret_cast<uint64_t>(g_prefill_zero_row);
  const int first = dma_first(wave), cnt = dma_count(wave);
  const uint32_t base = lds_addr(buf) + 1024 * first;
  for (int i = 0; i < cnt; ++i) {
    const uint64_t g = rowp + 16 * (2 * (first + i) + (lane >> 5));
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g),
                 "{m0}"(__builtin_amdgcn_readfirstlane(base + 1024 * i)) : "memory");
  }
}

__device__ __forceinline__ void issue_index(const PrParams& P, uint8_t* smem, int t, int j, int lane) {
  if (lane < kPrKeys) {
    const int32_t* src = P.idx + (int64_t)t * P.idx_stride + j * kPrKeys + lane;
    dma4(src, __builtin_amdgcn_readfirstlane(lds_addr(smem + kPrRingOff + (j % kPrRingSlots) * 128)));
  }
}

__global__ void __launch_bounds__(kPrThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
sparse_mla_prefill_kernel(const PrParams P) {
  extern __shared__ __align__(16) uint8_t smem[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = lane >> 5, c32 = lane & 31;
  const int hp = wave >> 2, q4 = wave & 3;

  // XCD-aware order: the two head groups of a token land on the same XCD
  const int nwg = gridDim.x;
  int work = blockIdx.x;
  if ((nwg & 7) == 0) work = (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3);
  const int t = work / P.head_groups;
  const int hg = work % P.head_groups;
  const int nblk = P.topk / kPrKeys;
  const int h_half = hg * kPrHeadsPerWG + hp * 32;
  const int head = h_half + c32;
  const bool head_ok = head < P.H;

  // query B operands: k-step ks of the nope quarter = dims 128q + 16ks + 8h .. +8,
  // rope = dims 512 + 16q + 8h .. +8, of head c32
  v4i qn[8], qr;
  {
    const uint16_t* qh = P.q + (int64_t)t * P.q_tok_stride + (int64_t)(head_ok ? head : 0) * P.q_head_stride;
    const v4i z = {0, 0, 0, 0};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
      qn[ks] = head_ok ? *reinterpret_cast<const v4i*>(qh + 128 * q4 + 16 * ks + 8 * h) : z;
    qr = head_ok ? *reinterpret_cast<const v4i*>(qh + 512 + 16 * q4 + 8 * h) : z;
  }
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the query is in registers before any copy goes out

  v16f o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[i][r] = 0.f;
  float m_run = -__builtin_inff();  // per head c32, log2 domain (identical in the 4 waves of a head half)
  float m_max = -__builtin_inff();  // exact running maximum (log2 domain), for max_logits
  float l_run = 0.f;                // per head c32: this lane's keys only

  const int my_dma = dma_count(wave);
  if (wave == kIdxWave) {
    for (int j = 0; j < 4 && j < nblk; ++j) issue_index(P, smem, t, j, lane);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  barrier();
  issue_rows(P, smem, 0, smem, lane, wave);
  if (nblk > 1) issue_rows(P, smem, 1, smem + kPrBufBytes, lane, wave);

  float* xs = reinterpret_cast<float*>(smem + kPrXsOff);
  float* mx = reinterpret_cast<float*>(smem + kPrMxOff) + (hp * 32 + c32) * 4;
  uint8_t* pbuf = smem + kPrPOff + hp * 4 * 512;

  for (int n = 0; n < nblk; ++n) {
    // rows of block n (and, for the index wave, the indices of block n+2) have landed
    int allow = n + 1 < nblk ? my_dma : 0;
    if (wave == kIdxWave && n >= 1 && n + 3 < nblk) allow += 1;
    wait_vm(allow);
    barrier();
    const uint8_t* buf = smem + (n % kPrNumBufs) * kPrBufBytes;
    const int32_t slot_n = reinterpret_cast<const int32_t*>(smem + kPrRingOff + (n % kPrRingSlots) * 128)[c32];
    const uint32_t vmask = (uint32_t)__ballot(slot_n >= 0 && (int64_t)slot_n < P.s_kv);
    if (wave == kIdxWave && n + 4 < nblk) issue_index(P, smem, t, n + 4, lane);

    // ---- partial S^T[32 keys x 32 heads]: s[r] = key 8(r/4) + 4h + r%4, head c32.
    // Piece p of row r sits at buf + 512 p + 16 r.
    v16f s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.f;
    {
      const uint8_t* kb = buf + (16 * q4 + h) * 512 + 16 * c32;
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const v4i a = *reinterpret_cast<const v4i*>(kb + 2 * ks * 512);
        s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_v8bf(a), as_v8bf(qn[ks]), s, 0, 0, 0);
      }
      const v4i a = *reinterpret_cast<const v4i*>(buf + (64 + 2 * q4 + h) * 512 + 16 * c32);
      s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_v8bf(a), as_v8bf(qr), s, 0, 0, 0);
    }

    // ---- four-way reduce-scatter: this wave keeps keys 8 q4 + 4h + i (s[4 q4 + i])
    float sv[4];
#pragma unroll
    for (int o = 0; o < 4; ++o) {
      if (o == q4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[i] = s[4 * o + i];
      } else {
        *reinterpret_cast<v4f*>(xs + ((wave * 4 + o) * 64 + lane) * 4) = v4f{s[4 * o], s[4 * o + 1], s[4 * o + 2],
                                                                             s[4 * o + 3]};
      }
    }
    barrier();
#pragma unroll
    for (int k = 1; k < 4; ++k) {
      const int src = hp * 4 + ((q4 + k) & 3);
      const v4f v = *reinterpret_cast<const v4f*>(xs + ((src * 4 + q4) * 64 + lane) * 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) sv[i] += v[i];
    }
    const uint32_t vm = vmask >> (8 * q4 + 4 * h);
    if (vmask != 0xffffffffu) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (!((vm >> i) & 1u)) sv[i] = -__builtin_inff();
    }
    float mloc = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
    mloc = fmaxf(mloc, shfl_xor(mloc, 32));
    if (h == 0) mx[q4] = mloc;
    barrier();

    // ---- online softmax (exp2 domain), lazy rescale
    {
      const v4f m4 = *reinterpret_cast<const v4f*>(mx);
      const float mblk = fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3])) * P.scale_log2;
      m_max = fmaxf(m_max, mblk);
      const bool need = mblk > m_run + kRescaleThreshold;  // true on the first valid block
      if (__ballot(need)) {
        const float m_new = need ? mblk : m_run;
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 when m_run = -inf
        l_run *= alpha;
        m_run = m_new;
        int hh = 4 * h;
        asm volatile("" : "+v"(hh));
        float ar[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) ar[r] = __shfl(alpha, 8 * (r >> 2) + hh + (r & 3), 64);
#pragma unroll
        for (int nt = 0; nt < 4; ++nt)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[nt][r] *= ar[r];
      }
    }
    const float m_use = m_run == -__builtin_inff() ? 0.f : m_run;
    float pv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) pv[i] = __builtin_amdgcn_exp2f(fmaf(sv[i], P.scale_log2, -m_use));
    l_run += (pv[0] + pv[1]) + (pv[2] + pv[3]);
    *reinterpret_cast<v2i*>(pbuf + (q4 * 64 + lane) * 8) = v2i{cvt_pk_bf16(pv[0], pv[1]), cvt_pk_bf16(pv[2], pv[3])};
    barrier();

    // ---- O[32 heads x 128 dims] += P . V over the block's 32 keys (two k-steps of 16).
    // A: element e of lane half h is key 16ks + 8(e/4) + 4h + e%4 = quarters 2ks and
    // 2ks + 1 of P. B: lane (group G = lane/16, c16 = lane%16) addresses row
    // 16ks + 4h + c16/4 (+8 for elements 4-7) and dims 128q + 32nn + 16(G%2) + 4(c16%4).
    {
      const int c16 = lane & 15, G = lane >> 4;
      const int dvb = 128 * q4 + 16 * (G & 1) + 4 * (c16 & 3);
      uint32_t vb = lds_addr(buf) + (dvb >> 3) * 512 + (4 * h + (c16 >> 2)) * 16 + ((2 * dvb) & 15);
      asm volatile("" : "+v"(vb));
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const v2i p0 = *reinterpret_cast<const v2i*>(pbuf + ((2 * ks) * 64 + lane) * 8);
        const v2i p1 = *reinterpret_cast<const v2i*>(pbuf + ((2 * ks + 1) * 64 + lane) * 8);
        const v4i pa = {p0[0], p0[1], p1[0], p1[1]};
#pragma unroll
        for (int nn = 0; nn < 4; ++nn) {
          // 32 dims = 4 pieces further; 16 rows = 256 bytes further
          const uint32_t a = vb + nn * 4 * 512 + ks * 16 * 16;
          const v2i b0 = lds_read_tr16_at(a);
          const v2i b1 = lds_read_tr16_at(a + 8 * 16);
          const v4i bv = {b0[0], b0[1], b1[0], b1[1]};
          o[nn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_v8bf(pa), as_v8bf(bv), o[nn], 0, 0, 0);
        }
      }
    }
    // block n+2's rows, into the buffer of block n-1 that every wave left at the top
    if (n + 2 < nblk) issue_rows(P, smem, n + 2, smem + ((n + 2) % kPrNumBufs) * kPrBufBytes, lane, wave);
  }

  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  l_run += shfl_xor(l_run, 32);
  barrier();
  if (h == 0) mx[q4] = l_run;
  barrier();
  {
    const v4f l4 = *reinterpret_cast<const v4f*>(mx);
    l_run = (l4[0] + l4[1]) + (l4[2] + l4[3]);
  }
  if (h_half >= P.H) return;
  const bool any = l_run > 0.f;
  const float inv = any ? 1.f / l_run : 0.f;
  const float lse_new = any ? (m_run + __builtin_amdgcn_logf(l_run)) * kLn2 : -__builtin_inff();
  const float max_new = any ? m_max * kLn2 : -__builtin_inff();
  // o[nt][r]: head h_half + 8(r/4) + 4h + r%4, dim 128 q4 + 32nt + c32
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int hr = 8 * (r >> 2) + 4 * h + (r & 3);
    const float ir = __shfl(inv, hr, 64);
    if (h_half + hr < P.H) {
      uint16_t* orow = P.out + ((int64_t)t * P.H + h_half + hr) * kPrDv + 128 * q4 + c32;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) orow[32 * nt] = (uint16_t)f32_to_bf16_rne(o[nt][r] * ir);
    }
  }
  if (h == 0 && q4 == 0 && head_ok) {
    if (P.lse) P.lse[(int64_t)t * P.H + head] = lse_new;
    if (P.max_logits) P.max_logits[(int64_t)t * P.H + head] = max_new;
  }
}

// The chunked prefill's top-k split by where each key lives. Index g of token t
// is a position in the ragged key order (sequence b's keys at cu_k[b] ..): key
// i = g - cu_k[b] is cached row i of sequence b while i < k_len - q_len (its
// physical slot block_table[b][i / bs] * bs + i % bs in the paged fp8 cache),
// else fresh row cu_q[b] + i - (k_len - q_len). Each token's two lists are
// compacted in index order and padded with -1 to their widths, and their
// lengths go to counts[2t], counts[2t+1]. One 256-thread workgroup per token.
__global__ void __launch_bounds__(256)
prefill_split_kernel(const int32_t* __restrict__ idx, int64_t idx_stride, int topk, const void* __restrict__ cu_q,
                     const void* __restrict__ cu_k, int cu_is_64, int num_seqs, int64_t total_k,
                     const int32_t* __restrict__ bt, int64_t bt_stride, int bt_width, int block_size,
                     int32_t* __restrict__ cached, int cached_w, int32_t* __restrict__ fresh, int fresh_w,
                     int32_t* __restrict__ counts) {
  auto cu = [&](const void* p, int i) -> int64_t {
    return cu_is_64 ? reinterpret_cast<const int64_t*>(p)[i] : (int64_t)reinterpret_cast<const int32_t*>(p)[i];
  };
  __shared__ int s_cnt[2][4];
  __shared__ int s_base[2];
  const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int32_t* row = idx + (int64_t)t * idx_stride;
  int32_t* crow = cached + (int64_t)t * cached_w;
  int32_t* frow = fresh + (int64_t)t * fresh_w;
  if (tid == 0) s_base[0] = s_base[1] = 0;
  for (int e0 = 0; e0 < topk; e0 += 256) {
    const int e = e0 + tid;
    int kind = -1;  // 0 cached, 1 fresh
    int32_t v = -1;
    const int64_t g = e < topk ? (int64_t)row[e] : -1;
    if (g >= 0 && g < total_k) {
      int lo = 0, hi = num_seqs;  // largest b < num_seqs with cu_k[b] <= g
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (cu(cu_k, mid) <= g) lo = mid; else hi = mid;
      }
      const int64_t k0 = cu(cu_k, lo), k1 = cu(cu_k, lo + 1);
      const int64_t ncached = (k1 - k0) - (cu(cu_q, lo + 1) - cu(cu_q, lo));
      const int64_t i = g - k0;
      if (i < ncached) {
        // a block-table column past the table's width is skipped like -1; a
        // stale or negative block gives a slot the MLA kernel skips
        const int64_t col = i / block_size;
        if (col < bt_width) {
          kind = 0;
          v = bt[(int64_t)lo * bt_stride + col] * block_size + (int32_t)(i % block_size);
        }
      } else {
        kind = 1;
        v = (int32_t)(cu(cu_q, lo) + i - ncached);
      }
    }
    const uint64_t mc = __ballot(kind == 0), mf = __ballot(kind == 1);
    if (lane == 0) {
      s_cnt[0][wave] = __popcll(mc);
      s_cnt[1][wave] = __popcll(mf);
    }
    __syncthreads();
    int bc = s_base[0], bf = s_base[1];
    for (int w = 0; w < wave; ++w) {
      bc += s_cnt[0][w];
      bf += s_cnt[1][w];
    }
    const uint64_t below = (1ull << lane) - 1ull;
    if (kind == 0) crow[bc + __popcll(mc & below)] = v;
    if (kind == 1) frow[bf + __popcll(mf & below)] = v;
    __syncthreads();
    if (tid == 0) {
      s_base[0] += s_cnt[0][0] + s_cnt[0][1] + s_cnt[0][2] + s_cnt[0][3];
      s_base[1] += s_cnt[1][0] + s_cnt[1][1] + s_cnt[1][2] + s_cnt[1][3];
    }
    __syncthreads();
  }
  const int nc = s_base[0], nf = s_base[1];
  if (tid == 0) {
    counts[2 * t] = nc;
    counts[2 * t + 1] = nf;
  }
  for (int e = nc + tid; e < cached_w; e += 256) crow[e] = -1;
  for (int e = nf + tid; e < fresh_w; e += 256) frow[e] = -1;
}

}  // namespace

static int sparse_mla_prefill_impl(const void* q, int64_t q_token_stride, int64_t q_head_stride, const void* kv,
                                   int64_t kv_row_stride, int64_t s_kv, const int32_t* indices, int64_t idx_stride,
                                   int num_tokens, int num_heads, int topk, float sm_scale, void* out,
                                   float* max_logits, float* lse, void* stream);
}  // namespace dsa

extern "C" {

int dsa_sparse_mla_prefill(const void* q, int64_t q_token_stride, int64_t q_head_stride, const void* kv,
                           int64_t kv_row_stride, int64_t s_kv, const int32_t* indices, int64_t idx_stride,
                           int num_tokens, int num_heads, int topk, float sm_scale, void* out, float* max_logits,
                           float* lse, void* stream) {
  return dsa::sparse_mla_prefill_impl(q, q_token_stride, q_head_stride, kv, kv_row_stride, s_kv, indices,
                                      idx_stride, num_tokens, num_heads, topk, sm_scale, out, max_logits, lse,
                                      stream);
}

}  // extern "C"

namespace dsa {

static int sparse_mla_prefill_impl(const void* q, int64_t q_token_stride, int64_t q_head_stride, const void* kv,
                                   int64_t kv_row_stride, int64_t s_kv, const int32_t* indices, int64_t idx_stride,
                                   int num_tokens, int num_heads, int topk, float sm_scale, void* out,
                                   float* max_logits, float* lse, void* stream) {
  if (num_tokens < 0 || num_heads <= 0 || (num_heads % 16) != 0)
    return set_error(kUnsupported, "sparse_mla_prefill: num_heads=%d must be a positive multiple of 16", num_heads);
  if (topk <= 0 || topk % kPrKeys != 0)
    return set_error(kUnsupported, "sparse_mla_prefill: topk=%d must be a positive multiple of %d", topk, kPrKeys);
  if (s_kv < 0 || s_kv > INT32_MAX)
    return set_error(kInvalidArgument, "sparse_mla_prefill: s_kv=%lld out of range", (long long)s_kv);
  if (num_tokens == 0) return kOk;
  if (!q || !indices || !out || (s_kv > 0 && !kv))
    return set_error(kInvalidArgument, "sparse_mla_prefill: null pointer");
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(kv) | reinterpret_cast<uintptr_t>(out)) & 15)
    return set_error(kInvalidArgument, "sparse_mla_prefill: q, kv and out must be 16-byte aligned");
  if ((q_token_stride % 8) || (q_head_stride % 8) || (kv_row_stride % 8) || kv_row_stride < kPrDqk)
    return set_error(kInvalidArgument, "sparse_mla_prefill: strides must be multiples of 8 elements, kv rows >= 576");
  static int smem_status = -1;
  if (smem_status < 0)
    smem_status = hipFuncSetAttribute((const void*)sparse_mla_prefill_kernel,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)kPrSmemBytes) == hipSuccess
                      ? 0 : 1;
  if (smem_status) return set_error(kLaunchFailed, "sparse_mla_prefill: cannot reserve %zu B of LDS", kPrSmemBytes);
  PrParams P;
  P.q = static_cast<const uint16_t*>(q);
  P.q_tok_stride = q_token_stride;
  P.q_head_stride = q_head_stride;
  P.kv = static_cast<const uint16_t*>(kv);
  P.kv_row_stride = kv_row_stride;
  P.s_kv = s_kv;
  P.idx = indices;
  P.idx_stride = idx_stride;
  P.T = num_tokens;
  P.H = num_heads;
  P.topk = topk;
  P.head_groups = (num_heads + kPrHeadsPerWG - 1) / kPrHeadsPerWG;
  P.scale_log2 = sm_scale * kLog2e;
  P.out = static_cast<uint16_t*>(out);
  P.max_logits = max_logits;
  P.lse = lse;
  const int64_t nwg = (int64_t)num_tokens * P.head_groups;
  if (nwg > INT32_MAX) return set_error(kInvalidArgument, "sparse_mla_prefill: grid too large");
  hipLaunchKernelGGL(sparse_mla_prefill_kernel, dim3((unsigned)nwg), dim3(kPrThreads), kPrSmemBytes,
                     (hipStream_t)stream, P);
  return check_launch("dsa_sparse_mla_prefill");
}

static inline size_t pf_align(size_t x) { return (x + 255) & ~(size_t)255; }
static inline int cached_width(int topk) { return (topk + 63) / 64 * 64; }
static inline int fresh_width(int topk) { return (topk + 31) / 32 * 32; }

}  // namespace dsa

extern "C" {

size_t dsa_sparse_mla_prefill_paged_workspace_bytes(int num_tokens, int topk) {
  using namespace dsa;
  if (num_tokens <= 0 || topk <= 0) return 0;
  return pf_align((size_t)num_tokens * cached_width(topk) * 4) + pf_align((size_t)num_tokens * fresh_width(topk) * 4) +
         pf_align((size_t)num_tokens * 2 * 4);
}

int dsa_sparse_mla_prefill_paged(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                                 const uint8_t* kv_cache, int64_t kv_block_stride_bytes, int kv_block_size,
                                 int64_t kv_num_blocks, const int32_t* block_table, int64_t bt_stride,
                                 int bt_width, const void* cu_seqlens_q, const void* cu_seqlens_k, int cu_is_64, int num_seqs,
                                 int64_t total_k, const void* fresh, int64_t fresh_row_stride, int64_t total_q,
                                 const int32_t* indices, int64_t idx_stride, int num_tokens, int num_heads, int topk,
                                 float sm_scale, void* out, float* max_logits, float* lse, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  using namespace dsa;
  if (num_tokens < 0 || num_seqs < 1 || total_k < 0 || total_q < 0 || topk <= 0 || kv_block_size <= 0 ||
      bt_width < 0 || bt_stride < bt_width)
    return set_error(kInvalidArgument, "sparse_mla_prefill_paged: bad sizes");
  if (num_tokens == 0) return kOk;
  if (!indices || !block_table || !cu_seqlens_q || !cu_seqlens_k || !out || !max_logits || !lse || !workspace)
    return set_error(kInvalidArgument, "sparse_mla_prefill_paged: null pointer");
  const size_t need = dsa_sparse_mla_prefill_paged_workspace_bytes(num_tokens, topk);
  if (workspace_bytes < need)
    return set_error(kWorkspaceTooSmall, "sparse_mla_prefill_paged: workspace %zu B < %zu B", workspace_bytes, need);
  const int cw = cached_width(topk), fw = fresh_width(topk);
  int32_t* cached = static_cast<int32_t*>(workspace);
  int32_t* fresh_idx =
      reinterpret_cast<int32_t*>(static_cast<uint8_t*>(workspace) + pf_align((size_t)num_tokens * cw * 4));
  int32_t* counts = reinterpret_cast<int32_t*>(static_cast<uint8_t*>(workspace) + pf_align((size_t)num_tokens * cw * 4) +
                                               pf_align((size_t)num_tokens * fw * 4));
  hipStream_t st = (hipStream_t)stream;
  // 1. each token's indices split into cache slots and fresh rows, compacted and counted
  hipLaunchKernelGGL(prefill_split_kernel, dim3((unsigned)num_tokens), dim3(256), 0, st, indices, idx_stride, topk,
                     cu_seqlens_q, cu_seqlens_k, cu_is_64, num_seqs, total_k, block_table, bt_stride, bt_width,
                     kv_block_size,
                     cached, cw, fresh_idx, fw, counts);
  if (int rc = check_launch("dsa_sparse_mla_prefill_paged(split)")) return rc;
  // 2. the decode kernel over each token's cache slots (fp8 rows, exact
  // dequantisation in registers) followed by its fresh bf16 rows, one softmax
  const MlaFresh fr{counts, fresh, fresh_row_stride, total_q, fresh_idx, fw};
  return sparse_mla_decode_impl(q, q_token_stride, q_head_stride, kv_cache, kv_block_stride_bytes, kv_block_size,
                                kv_num_blocks, cached, cw, num_tokens, num_heads, cw, sm_scale, out, lse, 1, nullptr, 0,
                                stream, max_logits, &fr);
}

}  // extern "C"
