// Exact top-k selection (+ page-table translation) and the logical->physical
// index transform for the DSA decode path, written for gfx950.
//
// Order: a most-significant-digit radix select on a 50-bit composite key
//   [ order_key(score) : 32 bits ][ (2^18-1) - position : 18 bits ]
// so that every element is distinct and equal scores resolve to the lowest
// positions (NaN ranks as -inf). Digits are 12/10/10 bits of the score key and
// 9/9 bits of the inverted position.
//
// Rows of at most 64K positions take one launch (topk_onepass_kernel: the
// row in registers, a 1/8 sample for the threshold, the candidates listed in
// LDS). Longer or ragged rows take three launches on the caller's stream:
//   1. threshold (one workgroup per row): a 1/8 sample of the row (contiguous
//      1024-element chunks, one in eight) gives, by a two-digit radix on the
//      sample, a score threshold t with about k + 4 sqrt(k) elements expected
//      at or above it - a bound that holds with a wide margin;
//   2. gather (8192 positions per workgroup, 8 per 64K row): one coalesced
//      read of the scores, one compare per element, and the elements at or
//      above t are appended - (key, position) - to the row's candidate list in
//      the workspace (wave ballots into LDS, one global atomic per workgroup);
//   3. finish (one workgroup per row): if the list holds between k and its
//      capacity entries, the exact top-k of the row is the exact top-k of the
//      list, found by radix levels in LDS; otherwise the row falls back to
//      the full exact select, which re-reads the row from HBM per level and
//      needs no bound at all. The selected positions are marked in an LDS
//      bitmap, compacted with one block prefix scan (ascending order, so the
//      output is deterministic) and written with the page translation.
// No global sort, no bounded candidate buffer on the exact path. The list
// selects (one-launch kernel, the fused indexer's topk_list_kernel) radix over
// [ key - t : nb bits ][ (2^18-1) - position : 18 bits ] instead, nb the bit
// length of the largest key - t, so that their digits spread over the
// candidates' own range.
#include <mutex>

#include "dsa_common.h"
#include "indexer_page.h"
#include "../../include/dsa_amd.h"

namespace dsa {

constexpr int kTopkThreads = 512;
constexpr int kTopkMaxLen = 1 << 18;            // positions per row
constexpr int kBitmapWords = kTopkMaxLen / 32;  // 32 KB of LDS
constexpr int kHistBins = 4096;
constexpr uint32_t kIdxMax = (1u << 18) - 1;
constexpr int kLevels = 5;

// threshold / gather geometry
constexpr int kAuxThreads = 256;
constexpr int kSampleChunk = 1024;              // contiguous sampled chunk
constexpr int kSampleEvery = 8;                 // one chunk in eight
constexpr int kGatherPerThread = 32;
constexpr int kGatherSpan = kAuxThreads * kGatherPerThread;  // 8192 positions per workgroup
constexpr int kGatherLdsCap = 2048;             // candidates one gather workgroup can stage

struct TopkSmem {
  uint32_t hist[kHistBins];
  uint32_t bitmap[kBitmapWords];
  uint32_t list_key[2][kListCap];
  uint32_t list_pos[2][kListCap];
  uint32_t wave_sum[16];
  uint32_t list_count[2];
  uint32_t tb, above, eq;
};
constexpr size_t kTopkSmemBytes = sizeof(TopkSmem);

// LDS of the list select: the candidates of a level's threshold bin are kept
// as 16-bit indices into the row's list (values re-read from global), so two
// workgroups fit on a CU. A row the kernel repairs itself uses TopkSmem.
struct ListSmem {
  uint32_t hist[kHistBins];
  uint32_t bitmap[kBitmapWords];
  uint16_t list[2][kListCap];
  uint32_t wave_sum[16];
  uint32_t list_count[2];
  uint32_t tb, above, eq;
};
static_assert(kListCap <= 65536, "list indices are 16-bit");
static_assert(sizeof(ListSmem) <= sizeof(TopkSmem), "a repairing launch covers the list layout");

__device__ __forceinline__ uint32_t radix_digit(int level, uint32_t key, uint32_t pos) {
  switch (level) {
    case 0: return key >> 20;
    case 1: return (key >> 10) & 1023u;
    case 2: return key & 1023u;
    case 3: return ((kIdxMax - pos) >> 9) & 511u;
    default: return (kIdxMax - pos) & 511u;
  }
}

__device__ __forceinline__ int radix_bins(int level) {
  return level == 0 ? 4096 : (level < 3 ? 1024 : 512);
}

// Does (key, pos) carry the chosen digits of every level before `level`?
__device__ __forceinline__ bool in_bucket(int level, uint32_t key, uint32_t pos, const uint32_t* thr) {
  switch (level) {
    case 0: return true;
    case 1: return (key >> 20) == thr[0];
    case 2: return (key >> 10) == ((thr[0] << 10) | thr[1]);
    case 3: return key == ((thr[0] << 20) | (thr[1] << 10) | thr[2]);
    default:
      return key == ((thr[0] << 20) | (thr[1] << 10) | thr[2]) && (((kIdxMax - pos) >> 9) == thr[3]);
  }
}

// Inverse of order_key: the float whose key is k.
__device__ __forceinline__ float key_to_float(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k);
}

// Exclusive block prefix sum of one value per thread; returns the prefix and
// writes the block total to *total (all threads).
template <int NT>
__device__ uint32_t block_exclusive_scan(uint32_t* wave_sum, uint32_t x, uint32_t* total) {
  constexpr int kWaves = NT / 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t v = x;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    uint32_t n = __shfl_up(v, off, 64);
    if (lane >= off) v += n;
  }
  __syncthreads();
  if (lane == 63) wave_sum[wave] = v;
  __syncthreads();
  uint32_t before = 0, all = 0;
  for (int w = 0; w < kWaves; ++w) {
    uint32_t t = wave_sum[w];
    if (w < wave) before += t;
    all += t;
  }
  *total = all;
  return before + v - x;
}

// Positions of the set bits of bitmap[0, nwords) in ascending order into
// sel[0, top_k) (*total = all set bits). Thread t owns the 16-byte-aligned
// word range [4 q t, 4 q (t + 1)), q = ceil(nwords / 4NT), read with 16-byte
// loads (lanes 4q words apart: at most 2-way bank conflicts, where single
// words would conflict q-ways) and kept in registers for the second pass;
// words at or past nwords count as zero. Ends with a barrier.
template <int NT>
__device__ void compact_bitmap(const uint32_t* bitmap, int nwords, uint32_t* wave_sum, uint32_t* sel, int top_k,
                               uint32_t* total_out) {
  constexpr int kMaxQ = kBitmapWords / (4 * NT);
  static_assert(kMaxQ >= 1 && kBitmapWords % (4 * NT) == 0, "bitmap words per thread");
  const int tid = threadIdx.x;
  const int q = (nwords + 4 * NT - 1) / (4 * NT);
  const int w0 = tid * 4 * q;
  uint32_t v[4 * kMaxQ];
  uint32_t cnt = 0;
#pragma unroll
  for (int i = 0; i < kMaxQ; ++i) {
    uint4 x = {0u, 0u, 0u, 0u};
    if (i < q && w0 + 4 * i < nwords) x = *reinterpret_cast<const uint4*>(bitmap + w0 + 4 * i);
    v[4 * i] = x.x;
    v[4 * i + 1] = w0 + 4 * i + 1 < nwords ? x.y : 0u;
    v[4 * i + 2] = w0 + 4 * i + 2 < nwords ? x.z : 0u;
    v[4 * i + 3] = w0 + 4 * i + 3 < nwords ? x.w : 0u;
#pragma unroll
    for (int k = 0; k < 4; ++k) cnt += __popc(v[4 * i + k]);
  }
  uint32_t total = 0;
  uint32_t at = block_exclusive_scan<NT>(wave_sum, cnt, &total);
  __syncthreads();  // sel may alias buffers read before this call
#pragma unroll
  for (int k = 0; k < 4 * kMaxQ; ++k) {
    uint32_t bits = v[k];
    while (bits) {
      const int bit = __ffs(bits) - 1;
      bits &= bits - 1;
      if (at < (uint32_t)top_k) sel[at] = (uint32_t)(((w0 + k) << 5) + bit);
      ++at;
    }
  }
  __syncthreads();
  *total_out = total;
}


struct RowOut {
  int32_t* page;       // page-translated output (or the untranslated output)
  int32_t* raw;        // optional raw positions
  const int32_t* pt;   // page table row (NULL: write positions + offset)
  uint32_t page_bits;
  int32_t offset;      // ragged offset
  __device__ __forceinline__ void emit(int slot, int32_t p) const {
    if (pt) {
      int32_t v = -1;
      if (p >= 0) {
        const uint32_t mask = (1u << page_bits) - 1u;
        v = (pt[(uint32_t)p >> page_bits] << page_bits) | ((uint32_t)p & mask);
      }
      page[slot] = v;
      if (raw) raw[slot] = p;
    } else {
      page[slot] = p >= 0 ? p + offset : -1;
    }
  }
};

struct RowIn {
  const float* scores;
  int64_t stride;
  const int32_t* seq_lens;
  const int32_t* row_starts;
  int64_t max_len;
  // 1: scores that are not finite or have |x| >= 1e30 rank as -inf (the
  // portable selection tail of the indexer, lightning.py:1474-1478); 0: only
  // NaN does (topk_transform, topk.cuh).
  int mask_extreme;
  __device__ __forceinline__ uint32_t key(float x) const {
    return order_key(mask_extreme && !(fabsf(x) < 1e30f) ? -__builtin_inff() : x);
  }
  __device__ __forceinline__ int len(int b) const {
    int64_t l = seq_lens[b];
    return (int)(l < 0 ? 0 : (l > max_len ? max_len : l));
  }
  __device__ __forceinline__ const float* row(int b) const {
    return scores + (int64_t)b * stride + (row_starts ? row_starts[b] : 0);
  }
};

// ---------------------------------------------------------------- 1. threshold
__global__ void __launch_bounds__(kAuxThreads)
topk_threshold_kernel(const RowIn in, int top_k, RowWs* __restrict__ ws) {
  __shared__ __align__(16) uint32_t hist[kHistBins];
  __shared__ uint32_t wave_sum[kAuxThreads / 64];
  __shared__ uint32_t tb, above, eq;
  const int tid = threadIdx.x, b = blockIdx.x;
  const int len = in.len(b);
  RowWs& w = ws[b];
  if (len <= top_k) {
    if (tid == 0) { w.t_key = 0u; w.count = 0u; w.failed = 0u; }
    return;
  }
  const float* row = in.row(b);
  for (int i = tid; i < kHistBins; i += kAuxThreads) hist[i] = 0u;
  __syncthreads();
  // sampled chunks start at multiples of kSampleChunk * kSampleEvery
  constexpr int kStride = kSampleChunk * kSampleEvery;
  const int nchunks = (len + kStride - 1) / kStride;
  for (int c0 = 0; c0 < nchunks; c0 += 8) {
    float x[8][4];
#pragma unroll
    for (int c = 0; c < 8; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int pos = (c0 + c) * kStride + e * kAuxThreads + tid;
        x[c][e] = (c0 + c < nchunks && pos < len) ? row[pos] : 0.f;
      }
#pragma unroll
    for (int c = 0; c < 8; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int pos = (c0 + c) * kStride + e * kAuxThreads + tid;
        if (c0 + c < nchunks && pos < len) atomicAdd(&hist[in.key(x[c][e]) >> 20], 1u);
      }
  }
  uint32_t nsample = 0;
  for (int c = 0; c < nchunks; ++c) nsample += (uint32_t)max(0, min(len - c * kStride, kSampleChunk));
  const float fk = (float)nsample / (float)len * (float)top_k;
  const uint32_t r = (uint32_t)(fk + 4.f * sqrtf(fk) + 8.f);
  __syncthreads();
  uint32_t t_key = 0u;  // 0: gather everything
  if (r < nsample) {
    find_threshold<kAuxThreads>(hist, wave_sum, 4096, r, &tb, &above, &eq);
    const uint32_t tb0 = tb, rem0 = r - above;
    __syncthreads();
    for (int i = tid; i < 1024; i += kAuxThreads) hist[i] = 0u;
    __syncthreads();
    for (int c = 0; c < nchunks; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int pos = c * kStride + e * kAuxThreads + tid;
        if (pos < len) {
          const uint32_t k = in.key(row[pos]);  // second look at the sample: L2 hits
          if ((k >> 20) == tb0) atomicAdd(&hist[(k >> 10) & 1023u], 1u);
        }
      }
    __syncthreads();
    find_threshold<kAuxThreads>(hist, wave_sum, 1024, rem0, &tb, &above, &eq);
    t_key = (tb0 << 20) | (tb << 10);
  }
  if (tid == 0) {
    w.t_key = t_key;
    w.count = 0u;
    w.failed = 0u;
  }
}

// ---------------------------------------------------------------- 2. gather
__global__ void __launch_bounds__(kAuxThreads)
topk_gather_kernel(const RowIn in, int top_k, RowWs* __restrict__ ws) {
  __shared__ uint32_t s_key[kGatherLdsCap];
  __shared__ uint32_t s_pos[kGatherLdsCap];
  __shared__ uint32_t s_count, s_base;
  const int tid = threadIdx.x, lane = tid & 63, b = blockIdx.y;
  const int len = in.len(b);
  const int span0 = blockIdx.x * kGatherSpan;
  if (len <= top_k || span0 >= len) return;
  const float* row = in.row(b);
  RowWs& w = ws[b];
  if (tid == 0) s_count = 0u;
  const uint32_t t_key = w.t_key;
  // -inf and NaN share the lowest key; at or below it every element is gathered
  const bool all = t_key <= order_key(-__builtin_inff());
  const float t_f = key_to_float(t_key);
  float x[kGatherPerThread];
#pragma unroll
  for (int j = 0; j < kGatherPerThread; ++j) {
    const int pos = span0 + j * kAuxThreads + tid;
    x[j] = pos < len ? __builtin_nontemporal_load(row + pos) : 0.f;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kGatherPerThread; ++j) {
    const int pos = span0 + j * kAuxThreads + tid;
    // the float compare admits every key >= t_key (and -0.0 against +0.0,
    // which only adds a candidate)
    const bool pred = pos < len && (all || x[j] >= t_f);
    const uint64_t m = __ballot(pred);
    if (m) {
      const int leader = __builtin_ctzll(m);
      uint32_t base = 0;
      if (lane == leader) base = atomicAdd(&s_count, (uint32_t)__popcll(m));
      base = __shfl(base, leader, 64);
      if (pred) {
        const uint32_t slot = base + (uint32_t)__popcll(m & ((1ull << lane) - 1ull));
        if (slot < kGatherLdsCap) {
          s_key[slot] = in.key(x[j]);
          s_pos[slot] = (uint32_t)pos;
        }
      }
    }
  }
  __syncthreads();
  const uint32_t n = s_count;
  if (tid == 0) {
    // an overflowing workgroup poisons the count so that the row falls back
    s_base = n ? atomicAdd(&w.count, n > kGatherLdsCap ? (uint32_t)(kListCap + 1) : n) : 0u;
  }
  __syncthreads();
  const uint32_t base = s_base;
  if (n <= kGatherLdsCap)
    for (uint32_t e = tid; e < n; e += kAuxThreads)
      if (base + e < kListCap) {
        w.key[base + e] = s_key[e];
        w.pos[base + e] = s_pos[e];
      }
}

// ---------------------------------------------------------------- 3. finish
// The finish of row b by one workgroup of kTopkThreads threads (all of them
// call it): the list select when the row's list is usable, else the full
// exact select over the row's scores.
__device__ void finish_row(TopkSmem& s, const RowIn& in, RowWs* __restrict__ ws, const int32_t* __restrict__ offsets,
                           const int32_t* __restrict__ page_table, int64_t pt_stride, int pt_div, uint32_t page_bits,
                           int32_t* __restrict__ out_page, int32_t* __restrict__ out_raw, int top_k, int b) {
  const int tid = threadIdx.x;
  const int len = in.len(b);
  const float* row = in.row(b);

  RowOut out;
  out.page = out_page + (int64_t)b * top_k;
  out.raw = out_raw ? out_raw + (int64_t)b * top_k : nullptr;
  out.pt = page_table ? page_table + (int64_t)(b / pt_div) * pt_stride : nullptr;
  out.page_bits = page_bits;
  out.offset = offsets ? offsets[b] : 0;

  if (len <= top_k) {
    for (int i = tid; i < top_k; i += kTopkThreads) out.emit(i, i < len ? i : -1);
    return;
  }

  const int nwords = (len + 31) >> 5;
  for (int i = tid; i < nwords; i += kTopkThreads) s.bitmap[i] = 0u;
  for (int i = tid; i < kHistBins; i += kTopkThreads) s.hist[i] = 0u;
  if (tid < 2) s.list_count[tid] = 0u;
  const uint32_t cand = ws ? ws[b].count : 0u;
  const bool listed = ws && cand >= (uint32_t)top_k && cand <= (uint32_t)kListCap;
  __syncthreads();

  uint32_t thr[kLevels] = {0, 0, 0, 0, 0};
  uint32_t remain = (uint32_t)top_k;
  bool source_mode = !listed;  // level pass over the row (HBM) vs the LDS list
  int cur = 0;
  uint32_t list_n = 0;

  if (listed) {
    for (uint32_t e = tid; e < cand; e += kTopkThreads) {
      const uint32_t key = ws[b].key[e];
      s.list_key[0][e] = key;
      s.list_pos[0][e] = ws[b].pos[e];
      atomicAdd(&s.hist[key >> 20], 1u);
    }
    list_n = cand;
  } else {
    // Level-0 histogram: one coalesced pass over the row, 4 loads in flight per thread.
    for (int base = 0; base < len; base += 4 * kTopkThreads) {
      float x[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = base + j * kTopkThreads + tid;
        x[j] = i < len ? row[i] : 0.f;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = base + j * kTopkThreads + tid;
        if (i < len) atomicAdd(&s.hist[in.key(x[j]) >> 20], 1u);
      }
    }
  }
  __syncthreads();

  for (int level = 0; level < kLevels; ++level) {
    find_threshold<kTopkThreads>(s.hist, s.wave_sum, radix_bins(level), remain, &s.tb, &s.above, &s.eq);
    const uint32_t tb = s.tb, above = s.above, eq = s.eq;
    thr[level] = tb;
    remain -= above;
    const bool take_all = (eq == remain) || level == kLevels - 1;
    const bool collect = !take_all && (!source_mode || eq <= (uint32_t)kListCap);
    const int nxt = cur ^ 1;
    __syncthreads();  // everyone has read tb/above/eq and the old histogram
    if (!take_all) {
      for (int i = tid; i < radix_bins(level + 1); i += kTopkThreads) s.hist[i] = 0u;
      if (tid == 0) s.list_count[nxt] = 0u;
    }
    __syncthreads();

    // one element of the current bucket: mark, or pass on to the next digit
    auto visit = [&](uint32_t key, uint32_t pos) {
      const uint32_t d = radix_digit(level, key, pos);
      if (d > tb || (take_all && d == tb)) atomicOr(&s.bitmap[pos >> 5], 1u << (pos & 31));
      if (!take_all && d == tb) {
        atomicAdd(&s.hist[radix_digit(level + 1, key, pos)], 1u);
        if (collect) {
          const uint32_t slot = atomicAdd(&s.list_count[nxt], 1u);
          s.list_key[nxt][slot] = key;
          s.list_pos[nxt][slot] = pos;
        }
      }
    };

    if (source_mode) {
      // HBM pass over the row (the exact path with no bound)
      for (int base = 0; base < len; base += 4 * kTopkThreads) {
        float x[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int i = base + j * kTopkThreads + tid;
          x[j] = i < len ? row[i] : 0.f;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int i = base + j * kTopkThreads + tid;
          const uint32_t key = in.key(x[j]);
          if (i < len && in_bucket(level, key, (uint32_t)i, thr)) visit(key, (uint32_t)i);
        }
      }
    } else {
      for (uint32_t e = tid; e < list_n; e += kTopkThreads) visit(s.list_key[cur][e], s.list_pos[cur][e]);
    }
    __syncthreads();
    if (take_all) break;
    if (collect) {
      source_mode = false;
      cur = nxt;
      list_n = s.list_count[cur];
    }
  }

  // Compact the bitmap in position order: positions in ascending order into
  // LDS, then the page-table translation as independent loads spread over all
  // threads
  uint32_t* sel = s.list_pos[0];
  uint32_t total = 0;
  compact_bitmap<kTopkThreads>(s.bitmap, nwords, s.wave_sum, sel, top_k, &total);
  for (int i = tid; i < top_k; i += kTopkThreads) out.emit(i, i < (int)total ? (int32_t)sel[i] : -1);
}

__global__ void __launch_bounds__(kTopkThreads)
topk_finish_kernel(const RowIn in, RowWs* __restrict__ ws, const int32_t* __restrict__ offsets,
                   const int32_t* __restrict__ page_table, int64_t pt_stride, int pt_div, uint32_t page_bits,
                   int32_t* __restrict__ out_page, int32_t* __restrict__ out_raw, int top_k) {
  extern __shared__ __align__(16) uint8_t smem_raw[];
  finish_row(*reinterpret_cast<TopkSmem*>(smem_raw), in, ws, offsets, page_table, pt_stride, pt_div, page_bits,
             out_page, out_raw, top_k, blockIdx.x);
}

// ---------------------------------------------------------------- one launch
// Rows of up to 64K positions: one 512-thread workgroup per row holds the
// whole row in registers (128 order keys per thread), so every pass after the
// one HBM read runs on registers and LDS:
//   1. a 1/8 sample (every 8th register slot, spread over the row) gives the
//      score threshold t by a two-digit radix, exactly as the threshold kernel;
//   2. each thread counts its keys >= t; one block scan gives every thread its
//      place in the candidate list, which goes to LDS in thread order;
//   3. if the list holds between k and kListCap entries, the exact top-k is the
//      exact top-k of the list (radix levels in LDS); otherwise the levels run
//      over the registers (the same result without any bound);
//   4. bitmap compaction in position order and the page translation.
constexpr int kRegThreads = 512;
constexpr int kRegPerThread = 128;
constexpr int kRegMaxLen = kRegThreads * kRegPerThread;  // 65536

// Position of register slot i of thread t (slot i = element i%4 of float4 chunk i/4).
__device__ __forceinline__ int reg_pos(int t, int i) { return 4 * kRegThreads * (i >> 2) + 4 * t + (i & 3); }

// Exact selection of the `remain` largest of the n composites in list 0 of
// LDS (hi = key - t_key, lo = (2^18 - 1) - position, so every composite is
// distinct and equal keys favour the lower position): radix levels of 12
// bits from the top of the nb + 18 bit composite, nb = bit length of the
// largest hi (`hmax`), so that the digits spread over the candidates' own
// range. Marks the selected positions in the (cleared) LDS bitmap. All NT
// threads call it after a barrier; it ends with one.
template <int NT>
__device__ void composite_select(TopkSmem& s, uint32_t n, uint32_t remain, uint32_t hmax) {
  const int tid = threadIdx.x;
  const int nb = 32 - __clz(hmax);  // bits of the key part (0: all equal)
  const int total_bits = nb + 18;
  const int nlev = (total_bits + 11) / 12;
  auto digit = [&](uint32_t h, uint32_t p, int L) {
    const uint64_t c = ((uint64_t)h << 18) | p;
    const int top = total_bits - 12 * L;
    const int lo_b = max(top - 12, 0);
    return (uint32_t)((c >> lo_b) & ((1ull << (top - lo_b)) - 1ull));
  };
  int cur = 0;
  for (int L = 0; L < nlev; ++L) {
    const int top = total_bits - 12 * L;
    const int nbins = 1 << (top - max(top - 12, 0));
    const int nxt = cur ^ 1;
    // list_count[cur] (the length of this level's list) was read by every
    // thread before the previous barrier; list_count[nxt] is free
    for (int i = tid; i < nbins; i += NT) s.hist[i] = 0u;
    if (tid == 0) s.list_count[nxt] = 0u;
    __syncthreads();
    for (uint32_t e = tid; e < n; e += NT) atomicAdd(&s.hist[digit(s.list_key[cur][e], s.list_pos[cur][e], L)], 1u);
    __syncthreads();
    find_threshold<NT>(s.hist, s.wave_sum, nbins, remain, &s.tb, &s.above, &s.eq);
    const uint32_t tb = s.tb, above = s.above, eq = s.eq;
    remain -= above;
    const bool last = (eq == remain) || L == nlev - 1;
    for (uint32_t e = tid; e < n; e += NT) {
      const uint32_t h = s.list_key[cur][e], p = s.list_pos[cur][e];
      const uint32_t d = digit(h, p, L);
      if (d > tb || (last && d == tb)) {
        const uint32_t pos = kIdxMax - p;
        atomicOr(&s.bitmap[pos >> 5], 1u << (pos & 31));
      } else if (!last && d == tb) {
        const uint32_t slot = atomicAdd(&s.list_count[nxt], 1u);
        s.list_key[nxt][slot] = h;
        s.list_pos[nxt][slot] = p;
      }
    }
    __syncthreads();
    if (last) break;
    n = s.list_count[nxt];
    cur = nxt;
    __syncthreads();  // every thread has read the next level's length
  }
}

__global__ void __launch_bounds__(kRegThreads) __attribute__((amdgpu_waves_per_eu(1, 2)))
topk_onepass_kernel(const RowIn in, const int32_t* __restrict__ offsets, const int32_t* __restrict__ page_table,
                    int64_t pt_stride, uint32_t page_bits, int32_t* __restrict__ out_page,
                    int32_t* __restrict__ out_raw, int top_k) {
  extern __shared__ __align__(16) uint8_t smem_raw[];
  TopkSmem& s = *reinterpret_cast<TopkSmem*>(smem_raw);
  constexpr int NT = kRegThreads;
  const int tid = threadIdx.x;
  const int b = blockIdx.x;
  const int len = in.len(b);
  const float* row = in.row(b);

  RowOut out;
  out.page = out_page + (int64_t)b * top_k;
  out.raw = out_raw ? out_raw + (int64_t)b * top_k : nullptr;
  out.pt = page_table ? page_table + (int64_t)b * pt_stride : nullptr;
  out.page_bits = page_bits;
  out.offset = offsets ? offsets[b] : 0;

  if (len <= top_k) {
    for (int i = tid; i < top_k; i += NT) out.emit(i, i < len ? i : -1);
    return;
  }

  // ---- the row, as order keys (0 = beyond the row: below every real key).
  // The launcher guarantees 16-byte aligned rows.
  uint32_t key[kRegPerThread];
  // Every load is in bounds: a chunk past the row's storage re-reads the
  // row's last aligned chunk (len > top_k >= 4 here), and the keys of
  // positions >= len are masked to 0, so no load sits behind a branch.
  const int last = (int)((in.max_len - 4) & ~(int64_t)3);
#pragma unroll
  for (int j = 0; j < kRegPerThread / 4; ++j) {
    const int p = 4 * kRegThreads * j + 4 * tid;
    const v4f v = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(row + min(p, last)));
#pragma unroll
    for (int e = 0; e < 4; ++e) key[4 * j + e] = p + e < len ? in.key(v[e]) : 0u;
  }

  const int nwords = (len + 31) >> 5;
  for (int i = tid; i < nwords; i += NT) s.bitmap[i] = 0u;
  for (int i = tid; i < kHistBins; i += NT) s.hist[i] = 0u;
  if (tid < 2) s.list_count[tid] = 0u;
  __syncthreads();

  // ---- 1. threshold from the sample (slots 0, 8, 16, ...): a key at or
  // below the sample's rank-r key, from two 1024-bin histogram levels over the
  // sample's own [min, max] key range (binning raw order keys would put the
  // sample into the few bins its sign and exponent span, and the LDS atomics
  // would serialise)
  uint32_t my_samples = 0, kmin = 0xffffffffu, kmax = 0u;
#pragma unroll
  for (int m = 0; m < kRegPerThread / 8; ++m)
    if (key[8 * m]) {
      ++my_samples;
      kmin = min(kmin, key[8 * m]);
      kmax = max(kmax, key[8 * m]);
    }
  const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    kmin = min(kmin, (uint32_t)__shfl_xor(kmin, off, 64));
    kmax = max(kmax, (uint32_t)__shfl_xor(kmax, off, 64));
  }
  if (lane == 0) {
    s.list_count[0] = 0u;
    s.bitmap[kBitmapWords - 1 - wave] = kmin;  // scratch words far past any row of <= 64K positions
    s.bitmap[kBitmapWords - 1 - NT / 64 - wave] = kmax;
  }
  uint32_t nsample = 0;
  (void)block_exclusive_scan<NT>(s.wave_sum, my_samples, &nsample);
  __syncthreads();
#pragma unroll
  for (int w2 = 0; w2 < NT / 64; ++w2) {
    kmin = min(kmin, s.bitmap[kBitmapWords - 1 - w2]);
    kmax = max(kmax, s.bitmap[kBitmapWords - 1 - NT / 64 - w2]);
  }
  const float fk = (float)nsample / (float)len * (float)top_k;
  const uint32_t r = (uint32_t)(fk + 4.f * sqrtf(fk) + 8.f);
  uint32_t t_key = 1u;  // every real key is >= 0x007fffff
  if (r < nsample) {
    const int shift = max(0, 32 - (int)__clz(kmax - kmin) - 10);
#pragma unroll
    for (int m = 0; m < kRegPerThread / 8; ++m)
      if (key[8 * m]) atomicAdd(&s.hist[(key[8 * m] - kmin) >> shift], 1u);
    __syncthreads();
    find_threshold<NT>(s.hist, s.wave_sum, 1024, r, &s.tb, &s.above, &s.eq);
    const uint32_t tb0 = s.tb, rem0 = r - s.above;
    t_key = kmin + (tb0 << shift);
    if (shift > 0) {
      const int shift2 = max(0, shift - 10);
      __syncthreads();
      for (int i = tid; i < 1024; i += NT) s.hist[i] = 0u;
      __syncthreads();
#pragma unroll
      for (int m = 0; m < kRegPerThread / 8; ++m)
        if (key[8 * m] && ((key[8 * m] - kmin) >> shift) == tb0)
          atomicAdd(&s.hist[((key[8 * m] - kmin) >> shift2) & 1023u], 1u);
      __syncthreads();
      find_threshold<NT>(s.hist, s.wave_sum, 1024, rem0, &s.tb, &s.above, &s.eq);
      t_key += s.tb << shift2;
    }
    t_key = max(t_key, 1u);
  }

  // ---- 2. candidates >= t, written in thread order after one block scan; a
  // slot that no lane of the wave fills costs one compare and one ballot
  uint32_t mine = 0;
#pragma unroll
  for (int i = 0; i < kRegPerThread; ++i) mine += key[i] >= t_key ? 1u : 0u;
  uint32_t total_cand = 0;
  uint32_t put = block_exclusive_scan<NT>(s.wave_sum, mine, &total_cand);
  if (total_cand <= (uint32_t)kListCap) {
    // positions recomputed here from an opaque thread id: computed once and
    // kept, they would take as many registers as the keys
    int t_o = tid;
    uint32_t t_k = t_key;  // opaque too: the counting loop's compares are not kept
    asm volatile("" : "+v"(t_o), "+v"(t_k));
#pragma unroll
    for (int i = 0; i < kRegPerThread; ++i) {
      const bool pred = key[i] >= t_k;
      if (__ballot(pred)) {
        if (pred) {
          s.list_key[0][put] = key[i];
          s.list_pos[0][put] = (uint32_t)reg_pos(t_o, i);
        }
        put += pred ? 1u : 0u;
      }
    }
  }
  const uint32_t cand = total_cand;
  const bool listed = cand >= (uint32_t)top_k && cand <= (uint32_t)kListCap;
  if (listed) {
    // ---- 3. exact select over the list: composites in place, their max
    __syncthreads();  // the list is written
    uint32_t mx = 0;
    for (uint32_t e = tid; e < cand; e += NT) {
      const uint32_t h = s.list_key[0][e] - t_key;
      s.list_key[0][e] = h;
      s.list_pos[0][e] = kIdxMax - s.list_pos[0][e];
      mx = max(mx, h);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = max(mx, (uint32_t)__shfl_xor(mx, off, 64));
    if (lane == 0) s.wave_sum[wave] = mx;
    __syncthreads();
    mx = 0;
#pragma unroll
    for (int w2 = 0; w2 < NT / 64; ++w2) mx = max(mx, s.wave_sum[w2]);
    __syncthreads();  // wave_sum is read before composite_select reuses it
    composite_select<NT>(s, cand, (uint32_t)top_k, mx);
  } else {
  for (int i = tid; i < kHistBins; i += NT) s.hist[i] = 0u;
  __syncthreads();
  if (listed) {
    for (uint32_t e = tid; e < cand; e += NT) atomicAdd(&s.hist[s.list_key[0][e] >> 20], 1u);
  } else {
#pragma unroll
    for (int i = 0; i < kRegPerThread; ++i)
      if (key[i]) atomicAdd(&s.hist[key[i] >> 20], 1u);
  }
  __syncthreads();

  // ---- 3. exact radix levels over the list (LDS) or, when the sample missed,
  // over the row re-read from memory (the registers are free by then)
  uint32_t thr[kLevels] = {0, 0, 0, 0, 0};
  uint32_t remain = (uint32_t)top_k;
  bool source_mode = !listed;
  int cur = 0;
  uint32_t list_n = listed ? cand : 0u;
  for (int level = 0; level < kLevels; ++level) {
    find_threshold<NT>(s.hist, s.wave_sum, radix_bins(level), remain, &s.tb, &s.above, &s.eq);
    const uint32_t tb = s.tb, above = s.above, eq = s.eq;
    thr[level] = tb;
    remain -= above;
    const bool take_all = (eq == remain) || level == kLevels - 1;
    const bool collect = !take_all && (!source_mode || eq <= (uint32_t)kListCap);
    const int nxt = cur ^ 1;
    __syncthreads();
    if (!take_all) {
      for (int i = tid; i < radix_bins(level + 1); i += NT) s.hist[i] = 0u;
      if (tid == 0) s.list_count[nxt] = 0u;
    }
    __syncthreads();
    auto visit = [&](uint32_t k, uint32_t pos) {
      const uint32_t d = radix_digit(level, k, pos);
      if (d > tb || (take_all && d == tb)) atomicOr(&s.bitmap[pos >> 5], 1u << (pos & 31));
      if (!take_all && d == tb) {
        atomicAdd(&s.hist[radix_digit(level + 1, k, pos)], 1u);
        if (collect) {
          const uint32_t sl = atomicAdd(&s.list_count[nxt], 1u);
          s.list_key[nxt][sl] = k;
          s.list_pos[nxt][sl] = pos;
        }
      }
    };
    if (source_mode) {
      for (int base = 0; base < len; base += 4 * NT) {
        float x[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int i = base + j * NT + tid;
          x[j] = i < len ? row[i] : 0.f;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int i = base + j * NT + tid;
          const uint32_t k = in.key(x[j]);
          if (i < len && in_bucket(level, k, (uint32_t)i, thr)) visit(k, (uint32_t)i);
        }
      }
    } else {
      for (uint32_t e = tid; e < list_n; e += NT) visit(s.list_key[cur][e], s.list_pos[cur][e]);
    }
    __syncthreads();
    if (take_all) break;
    if (collect) {
      source_mode = false;
      cur = nxt;
      list_n = s.list_count[cur];
    }
  }

  }

  // ---- 4. compaction in position order (two words per thread) and output
  uint32_t* sel = s.list_pos[0];
  uint32_t total = 0;
  compact_bitmap<NT>(s.bitmap, nwords, s.wave_sum, sel, top_k, &total);
  for (int i = tid; i < top_k; i += NT) out.emit(i, i < (int)total ? (int32_t)sel[i] : -1);
}

// ---------------------------------------------------------------- list select
// Exact top-k of a row's candidate list (fused indexer path): every candidate
// has key >= t_key, so the radix runs over the 50-bit composite
//   [ key - t_key : nb bits ][ (2^18-1) - position : 18 bits ]
// where nb = bit length of (max key - t_key), in 12-bit digits from the top:
// the digits spread over the candidates' actual range instead of the fixed
// bit positions of the full select, where most candidates share the top
// digits. A row whose list is unusable (fewer than k or more than the list
// capacity) is flagged for the repair launches.
// Full indexer logits of one row by the calling workgroup (kTopkThreads
// threads): wave w computes pages w, w + 8, ... of the row through three
// rotating page buffers, logits[t] for t < len.
__device__ void repair_row_logits(const RowRepair& rp, const int32_t* __restrict__ bt_row, int row, int len) {
  constexpr int kWaves = kTopkThreads / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v8i qa[1][4];
  float w[1][4][4];
  load_query(rp.q + (int64_t)row * kIdxHeads * kIdxHeadDim, rp.weights + (int64_t)row * kIdxHeads, lane, qa[0],
             w[0]);
  float* out = rp.logits + (int64_t)row * rp.logits_stride;
  const int npages = (len + kIdxPageTokens - 1) / kIdxPageTokens;
  const int n = npages > wave ? (npages - wave + kWaves - 1) / kWaves : 0;  // this wave's pages
  auto page_ptr = [&](int i) { return rp.kv + (int64_t)bt_row[wave + kWaves * i] * kIdxPageBytes; };
  auto compute = [&](const PageRegs& pr, int i) {
    const float v = page_head_sum<1>(pr, 0, lane, qa, w);
    const int t = (wave + kWaves * i) * kIdxPageTokens + lane;
    if (t < len) out[t] = v * pr.scale;
  };
  PageRegs buf0, buf1, buf2;
  if (0 < n) load_page(buf0, page_ptr(0), lane);
  if (1 < n) load_page(buf1, page_ptr(1), lane);
  for (int i = 0; i < n; i += 3) {
    if (i + 2 < n) load_page(buf2, page_ptr(i + 2), lane);
    compute(buf0, i);
    if (i + 3 < n) load_page(buf0, page_ptr(i + 3), lane);
    if (i + 1 < n) compute(buf1, i + 1);
    if (i + 4 < n) load_page(buf1, page_ptr(i + 4), lane);
    if (i + 2 < n) compute(buf2, i + 2);
  }
}

// The list select of one row per workgroup. kRepair: a row whose list is
// unusable is redone in the kernel from its full logits (rp.q set, the launch
// reserves TopkSmem); otherwise it is appended to rp.defer_rows.
template <bool kRepair>
__device__ __forceinline__ void list_select_row(const int32_t* __restrict__ seq_lens, int64_t max_len,
                                                RowWs* __restrict__ ws, const int32_t* __restrict__ page_table,
                                                int64_t pt_stride, int pt_div, uint32_t page_bits,
                                                const int32_t* __restrict__ offsets, int32_t* __restrict__ out_page,
                                                int32_t* __restrict__ out_raw, int top_k, const RowRepair& rp) {
  extern __shared__ __align__(16) uint8_t smem_raw[];
  ListSmem& s = *reinterpret_cast<ListSmem*>(smem_raw);
  constexpr int NT = kTopkThreads;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = blockIdx.x;
  const int64_t l = seq_lens[b];
  const int len = (int)(l < 0 ? 0 : (l > max_len ? max_len : l));
  RowWs& w = ws[b];

  RowOut out;
  out.page = out_page + (int64_t)b * top_k;
  out.raw = out_raw ? out_raw + (int64_t)b * top_k : nullptr;
  out.pt = page_table ? page_table + (int64_t)(b / pt_div) * pt_stride : nullptr;
  out.page_bits = page_bits;
  out.offset = (!page_table && offsets) ? offsets[b] : 0;

  if (len <= top_k) {
    for (int i = tid; i < top_k; i += NT) out.emit(i, i < len ? i : -1);
    return;
  }
  const uint32_t cand = w.count;
  if (cand < (uint32_t)top_k || cand > (uint32_t)kListCap) {
    // The sample misjudged this row's threshold: its list cannot give the
    // exact top-k. Redo the row here, from its full logits, or leave it to
    // the caller.
    if (tid == 0) w.failed = 1u;
    if constexpr (kRepair) {
      repair_row_logits(rp, page_table + (int64_t)(b / pt_div) * pt_stride, b, len);
      __syncthreads();  // the row's logits (global) are visible to the whole workgroup
      const RowIn in{rp.logits, rp.logits_stride, seq_lens, nullptr, max_len};
      // a repairing launch reserves the full select's LDS
      finish_row(*reinterpret_cast<TopkSmem*>(smem_raw), in, nullptr, nullptr, page_table, pt_stride, pt_div,
                 page_bits, out_page, out_raw, top_k, b);
    } else {
      if (tid == 0) rp.defer_rows[atomicAdd(rp.defer_count, 1u)] = b;
    }
    return;
  }
  const uint32_t t_key = w.t_key;

  // Candidates into registers (element e = u * NT + tid), all loads in flight
  // at once: composite (hi = key - t_key, lo = inverted position), and the
  // block maximum of hi.
  constexpr int kPer = kListCap / NT;
  static_assert(kListCap % NT == 0, "list capacity must be whole rows of the block");
  uint32_t ch[kPer], cl[kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const uint32_t e = (uint32_t)(u * NT + tid);
    ch[u] = e < cand ? w.key[e] : t_key;
    cl[u] = e < cand ? w.pos[e] : 0u;
  }
  const int nwords = (len + 31) >> 5;
  // The row's page table, when it fits in the bitmap words past the row's,
  // is copied to LDS with the candidates so that the output's translation
  // reads LDS, not a dependent global load.
  const int npg = out.pt ? (len + (1 << page_bits) - 1) >> page_bits : 0;
  const int pt_off = (nwords + 3) & ~3;
  const bool pt_lds = out.pt && pt_off + npg <= kBitmapWords;
  int32_t* const ptc = reinterpret_cast<int32_t*>(s.bitmap + pt_off);
  if (pt_lds) {
    for (int i0 = 0; i0 < npg; i0 += 4 * NT) {
      int32_t v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + u * NT + tid;
        v[u] = i < npg ? out.pt[i] : 0;
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + u * NT + tid;
        if (i < npg) ptc[i] = v[u];
      }
    }
  }
  for (int i = tid; i < nwords; i += NT) s.bitmap[i] = 0u;
  for (int i = tid; i < kHistBins; i += NT) s.hist[i] = 0u;
  if (tid == 0) s.list_count[0] = 0u;
  uint32_t mx = 0;
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    ch[u] -= t_key;
    cl[u] = kIdxMax - cl[u];
    mx = max(mx, ch[u]);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = max(mx, (uint32_t)__shfl_xor(mx, off, 64));
  if (lane == 0) s.wave_sum[wave] = mx;
  __syncthreads();
  mx = 0;
  for (int i = 0; i < NT / 64; ++i) mx = max(mx, s.wave_sum[i]);
  const int nb = 32 - __clz(mx);            // bits of the key part (0: all equal)
  const int total_bits = nb + 18;
  const int nlev = (total_bits + 11) / 12;
  auto composite = [&](uint32_t h, uint32_t p) { return ((uint64_t)h << 18) | p; };
  // digit of level L: bits [total - 12(L+1), total - 12L) of the composite
  auto digit = [&](uint64_t c, int L) {
    const int top = total_bits - 12 * L;
    const int lo_b = max(top - 12, 0);
    return (uint32_t)((c >> lo_b) & ((1ull << (top - lo_b)) - 1ull));
  };
  auto mark = [&](uint32_t p) {
    const uint32_t pos = kIdxMax - p;
    atomicOr(&s.bitmap[pos >> 5], 1u << (pos & 31));
  };

  // level 0 straight from the registers
  uint32_t remain = (uint32_t)top_k;
  bool last;
  {
    const int nbins = 1 << (total_bits - max(total_bits - 12, 0));
#pragma unroll
    for (int u = 0; u < kPer; ++u)
      if ((uint32_t)(u * NT + tid) < cand) atomicAdd(&s.hist[digit(composite(ch[u], cl[u]), 0)], 1u);
    __syncthreads();
    find_threshold<NT>(s.hist, s.wave_sum, nbins, remain, &s.tb, &s.above, &s.eq);
    const uint32_t tb = s.tb, above = s.above, eq = s.eq;
    remain -= above;
    last = (eq == remain) || nlev == 1;
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      if ((uint32_t)(u * NT + tid) >= cand) continue;
      const uint32_t d = digit(composite(ch[u], cl[u]), 0);
      if (d > tb || (last && d == tb)) {
        mark(cl[u]);
      } else if (!last && d == tb) {
        const uint32_t slot = atomicAdd(&s.list_count[0], 1u);
        s.list[0][slot] = (uint16_t)(u * NT + tid);
      }
    }
    __syncthreads();
  }

  // further levels over the (short) list of the threshold bin, in LDS
  int cur = 0;
  for (int L = 1; L < nlev && !last; ++L) {
    const uint32_t n = s.list_count[cur];
    const int top = total_bits - 12 * L;
    const int lo_b = max(top - 12, 0);
    const int nbins = 1 << (top - lo_b);
    const int nxt = cur ^ 1;
    // list_count[cur] is read by every thread above; list_count[nxt] was last
    // read a level ago
    for (int i = tid; i < nbins; i += NT) s.hist[i] = 0u;
    if (tid == 0) s.list_count[nxt] = 0u;
    __syncthreads();
    // the threshold bin's candidates, re-read from the row's list (L2)
    auto cand_h = [&](uint32_t i) { return w.key[s.list[cur][i]] - t_key; };
    auto cand_p = [&](uint32_t i) { return kIdxMax - w.pos[s.list[cur][i]]; };
    for (uint32_t e = tid; e < n; e += NT) atomicAdd(&s.hist[digit(composite(cand_h(e), cand_p(e)), L)], 1u);
    __syncthreads();
    find_threshold<NT>(s.hist, s.wave_sum, nbins, remain, &s.tb, &s.above, &s.eq);
    const uint32_t tb = s.tb, above = s.above, eq = s.eq;
    remain -= above;
    last = (eq == remain) || L == nlev - 1;
    for (uint32_t e = tid; e < n; e += NT) {
      const uint32_t h = cand_h(e), p = cand_p(e);
      const uint32_t d = digit(composite(h, p), L);
      if (d > tb || (last && d == tb)) {
        mark(p);
      } else if (!last && d == tb) {
        const uint32_t slot = atomicAdd(&s.list_count[nxt], 1u);
        s.list[nxt][slot] = s.list[cur][e];
      }
    }
    __syncthreads();
    cur = nxt;
  }

  // compaction in position order and output
  uint32_t* sel = s.hist;  // 4096 entries >= top_k
  uint32_t total = 0;
  compact_bitmap<NT>(s.bitmap, nwords, s.wave_sum, sel, top_k, &total);
  if (pt_lds) {
    const uint32_t mask = (1u << page_bits) - 1u;
    for (int i = tid; i < top_k; i += NT) {
      const int32_t p = i < (int)total ? (int32_t)sel[i] : -1;
      out.page[i] = p >= 0 ? (int32_t)(((uint32_t)ptc[(uint32_t)p >> page_bits] << page_bits) | ((uint32_t)p & mask)) : -1;
      if (out.raw) out.raw[i] = p;
    }
  } else {
    for (int i = tid; i < top_k; i += NT) out.emit(i, i < (int)total ? (int32_t)sel[i] : -1);
  }
}

__global__ void __launch_bounds__(kTopkThreads)
topk_list_kernel(const int32_t* __restrict__ seq_lens, int64_t max_len, RowWs* __restrict__ ws,
                 const int32_t* __restrict__ page_table, int64_t pt_stride, int pt_div, uint32_t page_bits,
                 int32_t* __restrict__ out_page, int32_t* __restrict__ out_raw, int top_k, const RowRepair rp) {
  list_select_row<true>(seq_lens, max_len, ws, page_table, pt_stride, pt_div, page_bits, nullptr, out_page, out_raw,
                        top_k, rp);
}

// Four waves per SIMD (<= 128 VGPRs): with the list layout, two workgroups per CU.
__global__ void __launch_bounds__(kTopkThreads) __attribute__((amdgpu_waves_per_eu(4)))
topk_list_defer_kernel(const int32_t* __restrict__ seq_lens, int64_t max_len, RowWs* __restrict__ ws,
                       const int32_t* __restrict__ page_table, int64_t pt_stride, int pt_div, uint32_t page_bits,
                       const int32_t* __restrict__ offsets, int32_t* __restrict__ out_page,
                       int32_t* __restrict__ out_raw, int top_k, const RowRepair rp) {
  list_select_row<false>(seq_lens, max_len, ws, page_table, pt_stride, pt_div, page_bits, offsets, out_page, out_raw,
                         top_k, rp);
}

__global__ void topk_to_physical_kernel(const int32_t* __restrict__ topk, int64_t topk_stride,
                                        const int32_t* __restrict__ bt, int64_t bt_stride,
                                        int table_width, int rows, int k, int rows_per_table,
                                        int block_size, int32_t* __restrict__ out) {
  const int64_t n = (int64_t)rows * k;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int r = (int)(e / k), c = (int)(e % k);
    const int32_t p = topk[(int64_t)r * topk_stride + c];
    int32_t v = -1;
    if (p >= 0) {
      const int page = p / block_size;
      if (page < table_width)
        v = bt[(int64_t)(r / rows_per_table) * bt_stride + page] * block_size + p % block_size;
    }
    out[e] = v;
  }
}

static int prepare_topk_kernel() {
  static int status = -1;
  if (status < 0) {
    hipError_t e = hipFuncSetAttribute((const void*)topk_finish_kernel,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)kTopkSmemBytes);
    if (e == hipSuccess)
      e = hipFuncSetAttribute((const void*)topk_onepass_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)kTopkSmemBytes);
    if (e == hipSuccess)
      e = hipFuncSetAttribute((const void*)topk_list_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)kTopkSmemBytes);
    if (e == hipSuccess)
      e = hipFuncSetAttribute((const void*)topk_list_defer_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)sizeof(ListSmem));
    status = e == hipSuccess ? 0 : 1;
    if (status) return set_error(kLaunchFailed, "topk: cannot reserve %zu B of LDS: %s",
                                 kTopkSmemBytes, hipGetErrorString(e));
  }
  return status ? kLaunchFailed : kOk;
}

// The launches of one selection. `workspace` NULL: the exact full path only.
// Scratch of the no-allocation entry point: the per-row state (threshold,
// candidate count, candidate list) of up to kNoAllocRows rows, held by every
// GPU the library runs on until the process ends. Host code never passes the
// array's name to a kernel (on the host it is only a stand-in for the symbol):
// each device's address comes from hipGetSymbolAddress, once per device.
constexpr int kNoAllocRows = 256;
static __device__ __align__(256) uint8_t scratch[kNoAllocRows * sizeof(RowWs)];
constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

// This device's address of `scratch` (looked up on the first call with that
// device current, then cached).
static int device_scratch(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(kLaunchFailed, "dsa_topk_transform_noalloc: no usable current device (%d)", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return set_error(kLaunchFailed, "dsa_topk_transform_noalloc: hipGetSymbolAddress(scratch) failed: %s",
                       hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return kOk;
}

static int launch_topk(const RowIn& in, int batch, const int32_t* offsets, const int32_t* page_table,
                       int64_t pt_stride, uint32_t page_bits, int32_t* out_page, int32_t* out_raw,
                       int top_k, void* workspace, size_t workspace_bytes, hipStream_t stream,
                       const char* what) {
  if (int rc = prepare_topk_kernel()) return rc;
  const bool aligned = (reinterpret_cast<uintptr_t>(in.scores) & 15) == 0 && (in.stride & 3) == 0 && !in.row_starts;
  if (in.max_len <= kRegMaxLen && aligned) {
    // the whole row fits in one workgroup's registers: one launch, no workspace
    hipLaunchKernelGGL(topk_onepass_kernel, dim3(batch), dim3(kRegThreads), kTopkSmemBytes, stream, in, offsets,
                       page_table, pt_stride, page_bits, out_page, out_raw, top_k);
    return check_launch(what);
  }
  RowWs* ws = nullptr;
  if (workspace) {
    if (workspace_bytes < (size_t)batch * sizeof(RowWs))
      return set_error(kWorkspaceTooSmall, "%s: workspace %zu B < %zu B", what, workspace_bytes,
                       (size_t)batch * sizeof(RowWs));
    if (reinterpret_cast<uintptr_t>(workspace) & 15)
      return set_error(kInvalidArgument, "%s: workspace must be 16-byte aligned", what);
    ws = static_cast<RowWs*>(workspace);
    hipLaunchKernelGGL(topk_threshold_kernel, dim3(batch), dim3(kAuxThreads), 0, stream, in, top_k, ws);
    const int64_t spans = (in.max_len + kGatherSpan - 1) / kGatherSpan;
    if (spans > 0)
      hipLaunchKernelGGL(topk_gather_kernel, dim3((unsigned)spans, batch), dim3(kAuxThreads), 0, stream, in,
                         top_k, ws);
  }
  hipLaunchKernelGGL(topk_finish_kernel, dim3(batch), dim3(kTopkThreads), kTopkSmemBytes, stream, in, ws,
                     offsets, page_table, pt_stride, 1, page_bits, out_page, out_raw, top_k);
  return check_launch(what);
}

int launch_list_select(const RowRepair& rp, const int32_t* seq_lens, int64_t max_len, RowWs* ws,
                       const int32_t* page_table, int64_t pt_stride, int pt_div, uint32_t page_bits,
                       const int32_t* offsets, int32_t* out_page, int32_t* out_raw, int top_k, int rows,
                       hipStream_t stream) {
  if (int rc = prepare_topk_kernel()) return rc;
  if (rp.q)
    hipLaunchKernelGGL(topk_list_kernel, dim3(rows), dim3(kTopkThreads), kTopkSmemBytes, stream, seq_lens, max_len,
                       ws, page_table, pt_stride, pt_div, page_bits, out_page, out_raw, top_k, rp);
  else
    hipLaunchKernelGGL(topk_list_defer_kernel, dim3(rows), dim3(kTopkThreads), sizeof(ListSmem), stream, seq_lens,
                       max_len, ws, page_table, pt_stride, pt_div, page_bits, offsets, out_page, out_raw, top_k, rp);
  return check_launch("dsa_indexer_topk(select)");
}

}  // namespace dsa

extern "C" {

int dsa_topk_max_len(void) { return dsa::kTopkMaxLen; }

size_t dsa_topk_workspace_bytes(int batch) {
  return batch > 0 ? (size_t)batch * sizeof(dsa::RowWs) : 0;
}

int dsa_topk_transform(const float* scores, int64_t score_stride, const int32_t* seq_lens,
                       const int32_t* page_table, int64_t page_table_stride, int32_t* out_page,
                       int32_t* out_raw, int batch, int64_t max_len, int page_size, int top_k,
                       void* workspace, size_t workspace_bytes, void* stream) {
  using namespace dsa;
  if (top_k != 512 && top_k != 2048)
    return set_error(kInvalidArgument, "top_k must be 512 or 2048, got %d", top_k);
  if (page_size <= 0 || (page_size & (page_size - 1)))
    return set_error(kInvalidArgument, "page_size must be power of 2, got %d", page_size);
  if (batch < 0 || max_len < 0 || (batch > 0 && (!scores || !seq_lens || !out_page)))
    return set_error(kInvalidArgument, "dsa_topk_transform: bad arguments");
  if (max_len > kTopkMaxLen)
    return set_error(kUnsupported, "score rows longer than %d are not supported (got %lld)",
                     kTopkMaxLen, (long long)max_len);
  if (batch == 0) return kOk;
  const RowIn in{scores, score_stride, seq_lens, nullptr, max_len};
  const uint32_t bits = (uint32_t)__builtin_ctz((unsigned)page_size);
  return launch_topk(in, batch, nullptr, page_table, page_table_stride, bits, out_page,
                     page_table ? out_raw : nullptr, top_k, workspace, workspace_bytes, (hipStream_t)stream,
                     "dsa_topk_transform");
}

int dsa_topk_transform_noalloc(const float* scores, int64_t score_stride, const int32_t* seq_lens,
                               const int32_t* page_table, int64_t page_table_stride, int32_t* out_page,
                               int32_t* out_raw, int batch, int64_t max_len, int page_size, int top_k,
                               void* stream) {
  using namespace dsa;
  if (top_k != 512 && top_k != 2048)
    return set_error(kInvalidArgument, "top_k must be 512 or 2048, got %d", top_k);
  if (page_size <= 0 || (page_size & (page_size - 1)))
    return set_error(kInvalidArgument, "page_size must be power of 2, got %d", page_size);
  if (batch < 0 || max_len < 0 || (batch > 0 && (!scores || !seq_lens || !out_page)))
    return set_error(kInvalidArgument, "dsa_topk_transform_noalloc: bad arguments");
  if (batch > kNoAllocRows)
    return set_error(kUnsupported, "dsa_topk_transform_noalloc: %d rows exceed the scratch maximum of %d rows",
                     batch, kNoAllocRows);
  if (max_len > kTopkMaxLen)
    return set_error(kUnsupported, "score rows longer than %d are not supported (got %lld)",
                     kTopkMaxLen, (long long)max_len);
  if (batch == 0) return kOk;
  void* ws = nullptr;
  if (int rc = device_scratch(&ws)) return rc;
  const RowIn in{scores, score_stride, seq_lens, nullptr, max_len};
  const uint32_t bits = (uint32_t)__builtin_ctz((unsigned)page_size);
  return launch_topk(in, batch, nullptr, page_table, page_table_stride, bits, out_page,
                     page_table ? out_raw : nullptr, top_k, ws, (size_t)kNoAllocRows * sizeof(RowWs),
                     (hipStream_t)stream, "dsa_topk_transform_noalloc");
}

int dsa_indexer_select(const float* logits, int64_t logits_stride, const int32_t* context_lens,
                       int32_t* out, int rows, int64_t max_len, int top_k, void* workspace,
                       size_t workspace_bytes, void* stream) {
  using namespace dsa;
  if (top_k != 512 && top_k != 2048)
    return set_error(kInvalidArgument, "top_k must be 512 or 2048, got %d", top_k);
  if (rows < 0 || max_len < 0 || (rows > 0 && (!logits || !context_lens || !out)))
    return set_error(kInvalidArgument, "dsa_indexer_select: bad arguments");
  if (max_len > kTopkMaxLen)
    return set_error(kUnsupported, "logits rows longer than %d are not supported (got %lld)",
                     kTopkMaxLen, (long long)max_len);
  if (rows == 0) return kOk;
  const RowIn in{logits, logits_stride, context_lens, nullptr, max_len, 1};
  return launch_topk(in, rows, nullptr, nullptr, 0, 0u, out, nullptr, top_k, workspace, workspace_bytes,
                     (hipStream_t)stream, "dsa_indexer_select");
}

int dsa_topk_transform_ragged(const float* scores, int64_t score_stride, const int32_t* seq_lens,
                              const int32_t* row_starts, const int32_t* offsets, int32_t* out,
                              int batch, int64_t max_len, int top_k, void* workspace,
                              size_t workspace_bytes, void* stream) {
  using namespace dsa;
  if (top_k != 2048) return set_error(kInvalidArgument, "ragged Indexer top_k must be 2048, got %d", top_k);
  if (batch < 0 || max_len < 0 || (batch > 0 && (!scores || !seq_lens || !row_starts || !offsets || !out)))
    return set_error(kInvalidArgument, "dsa_topk_transform_ragged: bad arguments");
  if (max_len > kTopkMaxLen)
    return set_error(kUnsupported, "ragged rows longer than %d are not supported (got %lld)",
                     kTopkMaxLen, (long long)max_len);
  if (batch == 0) return kOk;
  const RowIn in{scores, score_stride, seq_lens, row_starts, max_len};
  return launch_topk(in, batch, offsets, nullptr, 0, 0u, out, nullptr, top_k, workspace, workspace_bytes,
                     (hipStream_t)stream, "dsa_topk_transform_ragged");
}

int dsa_topk_to_physical(const int32_t* topk_indices, int64_t topk_stride, const int32_t* block_table,
                         int64_t bt_stride, int table_width, int rows, int topk, int rows_per_table,
                         int block_size, int32_t* out, void* stream) {
  using namespace dsa;
  if (rows < 0 || topk < 0 || rows_per_table < 1 || block_size <= 0 || table_width < 0)
    return set_error(kInvalidArgument, "dsa_topk_to_physical: bad arguments");
  const int64_t n = (int64_t)rows * topk;
  if (n == 0) return kOk;
  if (!topk_indices || !block_table || !out)
    return set_error(kInvalidArgument, "dsa_topk_to_physical: null pointer");
  const int threads = 256;
  const int64_t blocks = std::min<int64_t>((n + threads - 1) / threads, 65536);
  hipLaunchKernelGGL(topk_to_physical_kernel, dim3((unsigned)blocks), dim3(threads), 0, (hipStream_t)stream,
                     topk_indices, topk_stride, block_table, bt_stride, table_width, rows, topk,
                     rows_per_table, block_size, out);
  return check_launch("dsa_topk_to_physical");
}

}  // extern "C"
