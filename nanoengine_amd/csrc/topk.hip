// Exact top-k selection (+ page-table translation) and the logical->physical
// index transform for the DSA decode path, written for gfx950.
//
// Selection is a most-significant-digit radix select on a 50-bit composite key
//   [ order_key(score) : 32 bits ][ (2^18-1) - position : 18 bits ]
// so that every element is distinct and equal scores resolve to the lowest
// positions. Digits are 12/10/10 bits of the score key and 9/9 bits of the
// inverted position. One 1024-thread workgroup owns one row:
//   1. one pass over the row in HBM builds the 4096-bin histogram of digit 0;
//   2. each level finds the threshold bin with a block suffix scan, marks every
//      element above it in an LDS bitmap (one bit per position), and gathers the
//      threshold bin's elements for the next digit - into an LDS candidate list
//      when they fit (4096 entries), otherwise by another filtered pass over
//      the row, so the result is exact for any distribution (no bounded
//      candidate buffer, unlike the reference's 16K limit);
//   3. the bitmap is compacted with one block prefix scan, which emits the
//      selected positions in ascending order (deterministic output), and the
//      page-table translation is applied while writing.
// Typical rows need two HBM passes (histogram, mark+gather) and no global sort.
#include "dsa_common.h"
#include "../../include/dsa_amd.h"

namespace dsa {

constexpr int kTopkThreads = 1024;
constexpr int kTopkWaves = kTopkThreads / 64;
constexpr int kTopkMaxLen = 1 << 18;            // positions per row
constexpr int kBitmapWords = kTopkMaxLen / 32;  // 32 KB of LDS
constexpr int kListCap = 4096;                  // candidates per list buffer
constexpr int kHistBins = 4096;
constexpr uint32_t kIdxMax = (1u << 18) - 1;
constexpr int kLevels = 5;

struct TopkSmem {
  uint32_t hist[kHistBins];
  uint32_t bitmap[kBitmapWords];
  uint32_t list_key[2][kListCap];
  uint32_t list_pos[2][kListCap];
  uint32_t wave_sum[kTopkWaves];
  uint32_t list_count[2];
  uint32_t tb, above, eq;
};
constexpr size_t kTopkSmemBytes = sizeof(TopkSmem);

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

// Block-wide: find the bin tb with S(tb+1) < remain <= S(tb), S(b) = sum of
// hist[b..nbins). Leaves tb, above = S(tb+1), eq = hist[tb] in shared memory.
__device__ void find_threshold(TopkSmem& s, int nbins, uint32_t remain) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = nbins >= kTopkThreads ? nbins / kTopkThreads : 1;
  const int first = tid * per;
  uint32_t local = 0;
  if (first < nbins)
    for (int i = 0; i < per; ++i) local += s.hist[first + i];
  // inclusive suffix sum inside the wave
  uint32_t v = local;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    uint32_t n = __shfl_down(v, off, 64);
    if (lane + off < 64) v += n;
  }
  if (lane == 0) s.wave_sum[wave] = v;
  __syncthreads();
  uint32_t higher = v - local;
  for (int w = wave + 1; w < kTopkWaves; ++w) higher += s.wave_sum[w];
  if (first < nbins) {
    uint32_t acc = higher;
    for (int i = per - 1; i >= 0; --i) {
      uint32_t h = s.hist[first + i];
      if (acc < remain && acc + h >= remain) {
        s.tb = first + i;
        s.above = acc;
        s.eq = h;
      }
      acc += h;
    }
  }
  __syncthreads();
}

// Exclusive block prefix sum of one value per thread; returns the prefix and
// writes the block total to *total (all threads).
__device__ uint32_t block_exclusive_scan(TopkSmem& s, uint32_t x, uint32_t* total) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t v = x;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    uint32_t n = __shfl_up(v, off, 64);
    if (lane >= off) v += n;
  }
  __syncthreads();
  if (lane == 63) s.wave_sum[wave] = v;
  __syncthreads();
  uint32_t before = 0, all = 0;
  for (int w = 0; w < kTopkWaves; ++w) {
    uint32_t t = s.wave_sum[w];
    if (w < wave) before += t;
    all += t;
  }
  *total = all;
  return before + v - x;
}

struct RowOut {
  int32_t* page;       // page-translated output (or the ragged output)
  int32_t* raw;        // optional raw positions
  const int32_t* pt;   // page table row (NULL for ragged)
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

__global__ void __launch_bounds__(kTopkThreads)
topk_select_kernel(const float* __restrict__ scores, int64_t score_stride,
                   const int32_t* __restrict__ seq_lens, const int32_t* __restrict__ row_starts,
                   const int32_t* __restrict__ offsets, const int32_t* __restrict__ page_table,
                   int64_t pt_stride, uint32_t page_bits, int32_t* __restrict__ out_page,
                   int32_t* __restrict__ out_raw, int64_t max_len, int top_k) {
  extern __shared__ __align__(16) uint8_t smem_raw[];
  TopkSmem& s = *reinterpret_cast<TopkSmem*>(smem_raw);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = blockIdx.x;

  int64_t len64 = seq_lens[b];
  if (len64 < 0) len64 = 0;
  if (len64 > max_len) len64 = max_len;
  const int len = (int)len64;
  const float* row = scores + (int64_t)b * score_stride + (row_starts ? row_starts[b] : 0);

  RowOut out;
  out.page = out_page + (int64_t)b * top_k;
  out.raw = out_raw ? out_raw + (int64_t)b * top_k : nullptr;
  out.pt = page_table ? page_table + (int64_t)b * pt_stride : nullptr;
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
  __syncthreads();

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
      if (i < len) atomicAdd(&s.hist[order_key(x[j]) >> 20], 1u);
    }
  }
  __syncthreads();

  uint32_t thr[kLevels] = {0, 0, 0, 0, 0};
  uint32_t remain = (uint32_t)top_k;
  bool global_mode = true;
  int cur = 0;
  uint32_t list_n = 0;

  for (int level = 0; level < kLevels; ++level) {
    find_threshold(s, radix_bins(level), remain);
    const uint32_t tb = s.tb, above = s.above, eq = s.eq;
    thr[level] = tb;
    remain -= above;
    const bool take_all = (eq == remain) || level == kLevels - 1;
    const bool collect = !take_all && (!global_mode || eq <= (uint32_t)kListCap);
    const int nxt = cur ^ 1;
    __syncthreads();  // everyone has read tb/above/eq and the old histogram
    if (!take_all) {
      for (int i = tid; i < radix_bins(level + 1); i += kTopkThreads) s.hist[i] = 0u;
      if (tid == 0) s.list_count[nxt] = 0u;
    }
    __syncthreads();

    if (global_mode) {
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
          const uint32_t key = order_key(x[j]);
          bool sel = false;
          if (i < len && in_bucket(level, key, (uint32_t)i, thr)) {
            const uint32_t d = radix_digit(level, key, (uint32_t)i);
            sel = d > tb || (take_all && d == tb);
            if (!take_all && d == tb) {
              atomicAdd(&s.hist[radix_digit(level + 1, key, (uint32_t)i)], 1u);
              if (collect) {
                const uint32_t slot = atomicAdd(&s.list_count[nxt], 1u);
                s.list_key[nxt][slot] = key;
                s.list_pos[nxt][slot] = (uint32_t)i;
              }
            }
          }
          // positions of one wave are 64 consecutive, 64-aligned -> two bitmap words
          const uint64_t m = __ballot(sel);
          if (lane == 0 && m) {
            const int w0 = (base + j * kTopkThreads + wave * 64) >> 5;
            if ((uint32_t)m) atomicOr(&s.bitmap[w0], (uint32_t)m);
            if ((uint32_t)(m >> 32)) atomicOr(&s.bitmap[w0 + 1], (uint32_t)(m >> 32));
          }
        }
      }
    } else {
      for (uint32_t e = tid; e < list_n; e += kTopkThreads) {
        const uint32_t key = s.list_key[cur][e], pos = s.list_pos[cur][e];
        const uint32_t d = radix_digit(level, key, pos);
        if (d > tb || (take_all && d == tb)) atomicOr(&s.bitmap[pos >> 5], 1u << (pos & 31));
        if (!take_all && d == tb) {
          atomicAdd(&s.hist[radix_digit(level + 1, key, pos)], 1u);
          const uint32_t slot = atomicAdd(&s.list_count[nxt], 1u);
          s.list_key[nxt][slot] = key;
          s.list_pos[nxt][slot] = pos;
        }
      }
    }
    __syncthreads();
    if (take_all) break;
    if (collect) {
      global_mode = false;
      cur = nxt;
      list_n = s.list_count[cur];
    }
  }

  // Compact the bitmap in position order: each thread owns a contiguous word range.
  const int wpt = (nwords + kTopkThreads - 1) / kTopkThreads;
  const int w_begin = min(tid * wpt, nwords), w_end = min(w_begin + wpt, nwords);
  uint32_t cnt = 0;
  for (int w = w_begin; w < w_end; ++w) cnt += __popc(s.bitmap[w]);
  uint32_t total = 0;
  uint32_t slot = block_exclusive_scan(s, cnt, &total);
  for (int w = w_begin; w < w_end; ++w) {
    uint32_t bits = s.bitmap[w];
    while (bits) {
      const int bit = __ffs(bits) - 1;
      bits &= bits - 1;
      if (slot < (uint32_t)top_k) out.emit((int)slot, (w << 5) + bit);
      ++slot;
    }
  }
  for (int i = (int)total + tid; i < top_k; i += kTopkThreads) out.emit(i, -1);
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
    hipError_t e = hipFuncSetAttribute((const void*)topk_select_kernel,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)kTopkSmemBytes);
    status = e == hipSuccess ? 0 : 1;
    if (status) return set_error(kLaunchFailed, "topk: cannot reserve %zu B of LDS: %s",
                                 kTopkSmemBytes, hipGetErrorString(e));
  }
  return status ? kLaunchFailed : kOk;
}

}  // namespace dsa

extern "C" {

int dsa_topk_max_len(void) { return dsa::kTopkMaxLen; }

int dsa_topk_transform(const float* scores, int64_t score_stride, const int32_t* seq_lens,
                       const int32_t* page_table, int64_t page_table_stride, int32_t* out_page,
                       int32_t* out_raw, int batch, int64_t max_len, int page_size, int top_k,
                       void* stream) {
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
  if (int rc = prepare_topk_kernel()) return rc;
  const uint32_t bits = (uint32_t)__builtin_ctz((unsigned)page_size);
  hipLaunchKernelGGL(topk_select_kernel, dim3(batch), dim3(kTopkThreads), kTopkSmemBytes,
                     (hipStream_t)stream, scores, score_stride, seq_lens, nullptr, nullptr, page_table,
                     page_table_stride, bits, out_page, out_raw, max_len, top_k);
  return check_launch("dsa_topk_transform");
}

int dsa_topk_transform_ragged(const float* scores, int64_t score_stride, const int32_t* seq_lens,
                              const int32_t* row_starts, const int32_t* offsets, int32_t* out,
                              int batch, int64_t max_len, int top_k, void* stream) {
  using namespace dsa;
  if (top_k != 2048) return set_error(kInvalidArgument, "ragged Indexer top_k must be 2048, got %d", top_k);
  if (batch < 0 || max_len < 0 || (batch > 0 && (!scores || !seq_lens || !row_starts || !offsets || !out)))
    return set_error(kInvalidArgument, "dsa_topk_transform_ragged: bad arguments");
  if (max_len > kTopkMaxLen)
    return set_error(kUnsupported, "ragged rows longer than %d are not supported (got %lld)",
                     kTopkMaxLen, (long long)max_len);
  if (batch == 0) return kOk;
  if (int rc = prepare_topk_kernel()) return rc;
  hipLaunchKernelGGL(topk_select_kernel, dim3(batch), dim3(kTopkThreads), kTopkSmemBytes,
                     (hipStream_t)stream, scores, score_stride, seq_lens, row_starts, offsets, nullptr,
                     (int64_t)0, 0u, out, nullptr, max_len, top_k);
  return check_launch("dsa_topk_transform_ragged");
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
