// Sparse MLA decode over the packed fp8 MLA cache, for gfx950.
//
// For each query token t and head h:
//   s_i = sm_scale * q[t,h,:576] . kv(idx_i)[:576]     (valid idx_i only)
//   o   = softmax(s) @ kv(idx)[:, :512],  lse = log(sum_i exp(s_i))
// where kv(slot) is a 656-byte row [512 e4m3fn][4 x f32 tile scale][64 bf16].
//
// Workgroup = 8 waves (two per SIMD) = 64 heads of one token over one key
// split, in blocks of 64 selected rows. The waves specialise, so that each
// SIMD pairs a wave in its score phase with a wave in its P.V phase instead
// of two waves in the same phase:
//   QK waves 0-3: wave (hp = w/2, kh = w%2) owns keys 32kh .. 32kh+31 of each
//            block for the 32 heads of head half hp, over all 576 dims:
//            S^T[32 keys x 32 heads] on 36 v_mfma_f32_32x32x16_bf16. A = the
//            key's fp8 nope bytes from LDS converted to bf16 with the row's
//            tile scale (v_cvt_scalef32_pk_bf16_fp8; exact, since an e4m3
//            value times a power of two is a bf16 value) and its bf16 rope;
//            B = the query's bf16 values as given, resident in registers.
//            Products are exact and sums are f32, as in a bf16
//            dequantise-then-multiply. (The scaled fp8 MFMA would take the
//            raw rows directly, but it sums its 64 products to only ~13 bits
//            below the largest one.) Then the wave's own online softmax over
//            its 32 keys: a lazy reference m (an integer, log2 units) per
//            head, P = 2^(s - m) to LDS as bf16, the reference beside it.
//   PV waves 4-7: wave dq owns O[all 64 heads x dims 128dq .. +128] (V
//            tile dq, two head tiles) and adds the previous block's P.V: the
//            two key halves' P come with their own references m0, m1; per head
//            tile the wave keeps O against R = max(m0, m1) (rescaling by a
//            power of two when R moves) and
//            forms P' = P * 2^(e + m_kh - R), e the tile scale exponent of
//            each key, by adding to the bf16 exponent field; V is read from
//            the raw rows with ds_read_b64_tr_b8 (8 keys x 1 dim per lane, the
//            B operand layout) and converted with unit scale.
//   rows   : the raw 656-byte rows go straight from HBM into LDS with
//            global_load_lds_dwordx4 - consecutive lanes take consecutive
//            16-byte pieces of the packed rows - into one of three buffers,
//            one block ahead of use (block t+1 while the QK waves read block t
//            and the PV waves block t-1). The row indices arrive the same way,
//            four blocks ahead, in a five-entry ring; one wave turns a block's
//            indices into a 64-entry row-address table in LDS, so a load costs
//            a table read and an add. Invalid indices read a zero row.
// One barrier per block: P, the references and the next block's rows change
// hands there; no score, maximum or sum is exchanged inside a block.
// Chunked prefill: after a token's cache-slot blocks come blocks of 32 fresh
// bf16 rows [576] (the chunk's own keys, not yet in the cache). They go to LDS
// the same way; the key half 0 QK waves read them as bf16 operands, and the
// PV waves read V with ds_read_b64_tr_b16 (no tile scale), so cached and
// fresh keys share one softmax.
// Splits over the key list (for small batches) write normalised partial
// outputs and LSEs to a caller-provided workspace; a combine kernel merges
// them with the LSE rule of merge_attention_states.
#include <algorithm>
#include <cmath>

#include "dsa_common.h"
#include "../../include/dsa_amd.h"

namespace dsa {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));

constexpr int kMlaThreads = 512;
constexpr int kMlaWaves = kMlaThreads / 64;
constexpr int kMlaHeadsPerWG = 64;
constexpr int kMlaKeys = 64;              // rows per block
constexpr int kMlaRowBytes = 656;
constexpr int kMlaRowPieces = kMlaRowBytes / 16;      // 41
constexpr int kMlaDv = 512;
constexpr int kBufBytes = kMlaKeys * kMlaRowBytes;    // 41984: one block of packed raw rows
// A chunked prefill's fresh keys are bf16 rows [576] (1152 B), 32 to a block:
// a fresh block is 36 wave-wide loads and fits a row buffer.
constexpr int kFreshKeys = 32;
constexpr int kFreshRowBytes = 576 * 2;
constexpr int kFreshRowPieces = kFreshRowBytes / 16;  // 72
constexpr int kFreshDma = kFreshKeys * kFreshRowBytes / 1024;  // 36
static_assert(kFreshKeys * kFreshRowBytes <= kBufBytes, "a fresh block must fit a row buffer");
constexpr int kDmaPerBlock = kBufBytes / 1024;        // 41 wave-wide 16-byte loads per block
constexpr int kNumBufs = 3;
// LDS map (bytes)
constexpr int kPOff = kNumBufs * kBufBytes;            // P, two blocks: [2][2 hp][4 k-steps][64 lanes][8 bf16]
constexpr int kEOff = kPOff + 2 * 2 * 4 * 64 * 16;     // exponent tables, one per PV wave: [4][2 tiles][4][2][8 u16]
constexpr int kRefOff = kEOff + 4 * 512;               // references of the two key halves, two blocks: [2][2 hp][2][32] f32
constexpr int kFinOff = kRefOff + 2 * 2 * 2 * 32 * 4;  // final sums, references, maxima: [3][2 hp][2][32] f32
constexpr int kRingOff = kFinOff + 3 * 128 * 4;        // row indices, one 64-entry block per slot
constexpr int kRingSlots = 5;
constexpr int kAddrOff = kRingOff + kRingSlots * 256;  // row addresses of blocks being gathered, [2][64] u64
constexpr size_t kMlaSmemBytes = kAddrOff + 2 * kMlaKeys * 8;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kRescaleThreshold = 8.0f;  // log2 units
// P' = P * 2^(e + m_kh - R) is formed by adding to the bf16 exponent field,
// which needs P' to stay a normal number: P of a valid key is kept at or above
// 2^-30 of its key half's reference, and a key half whose reference is more
// than 2^30 below R is scaled by 2^-30 instead of 2^(m_kh - R). Each of its
// keys then adds at most 2^-22 of R's scale where it should add less, the
// same bound as leaving the half out. With tile scales above 2^-66, P' stays
// above 2^-126.
constexpr float kMinLogP = -30.0f;
constexpr int kDropExp = -30;
constexpr int kIdxWave = 3;                // the wave that fetches the row indices (a QK wave)

static_assert(kBufBytes % 1024 == 0, "a block of rows must be whole wave-wide loads");
static_assert(kMlaSmemBytes <= 160 * 1024, "LDS budget");

// Source of the pieces of an invalid row (cache or fresh): zero bytes.
__device__ __align__(16) uint8_t g_mla_zero_row[kFreshRowBytes];

struct MlaParams {
  const uint16_t* q;
  int64_t q_tok_stride, q_head_stride;
  const uint8_t* kv;
  int64_t kv_blk_stride;
  int64_t kv_num_blocks;
  int kv_block_size;
  int kv_block_shift;  // log2(kv_block_size) when it is a power of two, else -1
  const int32_t* idx;
  int64_t idx_stride;
  int T, H, topk, splits, head_groups;
  float scale_log2;
  uint16_t* out;
  float* lse;
  float* ws_o;    // [splits, T, H, 512] (splits > 1)
  float* ws_lse;  // [splits, T, H]
  float* max_out; // [T, H] largest scaled score (natural units), or null (splits == 1 only)
  // chunked prefill (paged, splits == 1): token t attends over ceil(counts[2t] / 64)
  // blocks of cache slots from idx (valid slots first), then ceil(counts[2t+1] / 32)
  // blocks of fresh bf16 rows fresh[fresh_idx[t][i]] (null counts: topk / splits
  // blocks of cache slots)
  const int32_t* counts;
  const uint16_t* fresh;
  int64_t fresh_row_stride;  // elements
  int64_t fresh_rows;
  const int32_t* fresh_idx;
  int64_t fresh_idx_stride;
};

// ---- asynchronous global -> LDS copies. They are issued from inline asm so
// that the compiler neither inserts vmcnt(0) before every LDS read nor waits
// for them at barriers: the kernel waits for them itself (vmcnt).
// `lds` is the wave's destination base (M0); lane i writes lds + 4*size*i.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}
__device__ __forceinline__ void dma4(const void* g, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}
__device__ __forceinline__ void barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)reinterpret_cast<uintptr_t>(p);
}

__device__ __forceinline__ v8bf as_v8bf(v4i x) { return __builtin_bit_cast(v8bf, x); }

__device__ __forceinline__ int cvt_pk_bf16(float a, float b) {
  const v2f x = {a, b};
  return __builtin_bit_cast(int, __builtin_convertvector(x, v2bf));
}

typedef short v4s __attribute__((ext_vector_type(4)));
typedef short v8s __attribute__((ext_vector_type(8)));

// Four 16-bit elements per lane, transposed within each 16-lane group: lane m
// addresses row m/4, elements 4(m%4) .. +3 of a 4 x 16 tile and receives
// column m of its four rows.
__device__ __forceinline__ v4s lds_read_tr16_at(uint32_t a) {
  typedef __attribute__((address_space(3))) v4s lds_v4s;
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(uintptr_t)a);
}

__device__ __forceinline__ v2i lds_read_tr8_at(uint32_t a) {
  typedef __attribute__((address_space(3))) v2i lds_v2i;
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(uintptr_t)a);
}

// Eight fp8 bytes (one per key) -> the bf16 B operand, unit scale.
__device__ __forceinline__ v8bf fp8x8_to_bf16(v2i raw) {
  v4i r;
  r[0] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw[0], 1.f, false));
  r[1] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw[0], 1.f, true));
  r[2] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw[1], 1.f, false));
  r[3] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw[1], 1.f, true));
  return as_v8bf(r);
}

__device__ __forceinline__ v8i lds_read32(const uint8_t* p) {
  const v4i a = *reinterpret_cast<const v4i*>(p);
  const v4i b = *reinterpret_cast<const v4i*>(p + 16);
  v8i r;
  r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
  r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
  return r;
}

// The gather of one block. One wave writes the 64 row addresses of the block
// to a table in LDS (lane = row); every wave then sends its share of the 41
// wave-wide loads, lane l of load i taking 16-byte piece c = 64(first + i) + l
// of the packed block: row c / 41, byte 16 (c % 41) of it. Those (row, byte)
// pairs are loop invariants, computed once per lane (DmaLanes).
constexpr int kTabWave = 2;  // the wave that builds the row-address table (a QK wave: the PV waves' chain is longer)

// Wave-uniform state of one workgroup's loop. Blocks [0, ncached) are 64 cache
// slots each, blocks [ncached, nblk) 32 fresh bf16 rows each.
struct MlaCtx {
  int lane, wave, h, c32, hp, kh, t_tok, key_begin, nblk, ncached, h_half, head;
  bool head_ok;
};

// Cache block of a physical slot.
__device__ __forceinline__ int64_t slot_block(const MlaParams& P, int32_t slot) {
  return P.kv_block_shift >= 0 ? (int64_t)(slot >> P.kv_block_shift) : (int64_t)(slot / P.kv_block_size);
}

// A slot is used when it is >= 0 and inside the cache; any other index
// (-1 padding, or a stale value past the cache) is skipped.
__device__ __forceinline__ bool slot_valid(const MlaParams& P, int32_t slot) {
  return slot >= 0 && slot_block(P, slot) < P.kv_num_blocks;
}

__device__ __forceinline__ uint64_t row_address(const MlaParams& P, int32_t slot) {
  if (!slot_valid(P, slot)) return reinterpret_cast<uint64_t>(g_mla_zero_row);
  int64_t blk, in_blk;
  if (P.kv_block_shift >= 0) {
    blk = slot >> P.kv_block_shift;
    in_blk = slot & ((1 << P.kv_block_shift) - 1);
  } else {
    blk = slot / P.kv_block_size;
    in_blk = slot % P.kv_block_size;
  }
  return reinterpret_cast<uint64_t>(P.kv + blk * P.kv_blk_stride + in_blk * kMlaRowBytes);
}

// A fresh row index is used when it is in [0, fresh_rows); a fresh block's
// ring entries 32-63 are never used.
__device__ __forceinline__ bool fresh_valid(const MlaParams& P, int32_t r, int lane) {
  return lane < kFreshKeys && r >= 0 && r < P.fresh_rows;
}

// Table of block j's row addresses from ring slot j % 5 (lane = row), in table j % 2.
template <bool kFresh>
__device__ __forceinline__ void build_addr_table(const MlaParams& P, uint8_t* smem, const MlaCtx& c, int j) {
  const int lane = c.lane;
  const int32_t slot = reinterpret_cast<const int32_t*>(smem + kRingOff + (j % kRingSlots) * 256)[lane];
  uint64_t a;
  if (!kFresh || j < c.ncached)
    a = row_address(P, slot);
  else
    a = fresh_valid(P, slot, lane) ? reinterpret_cast<uint64_t>(P.fresh + (int64_t)slot * P.fresh_row_stride)
                                   : reinterpret_cast<uint64_t>(g_mla_zero_row);
  *reinterpret_cast<uint64_t*>(smem + kAddrOff + (j & 1) * 512 + 8 * lane) = a;
}

// Wave w sends loads [first(w), first(w) + count(w)) of the block: six for
// wave 0, five for the others, in runs that share one M0 (LDS base) value.
__device__ __forceinline__ int dma_count(int wave) {
  return kDmaPerBlock / kMlaWaves + (wave < kDmaPerBlock % kMlaWaves ? 1 : 0);
}
__device__ __forceinline__ int dma_first(int wave) {
  return wave * (kDmaPerBlock / kMlaWaves) + min(wave, kDmaPerBlock % kMlaWaves);
}
static_assert(kDmaPerBlock / kMlaWaves == 5 && kDmaPerBlock % kMlaWaves == 1,
              "six loads for wave 0, five for the others");

// Load i of this lane: table byte offset 8 * row in bits 0-15, byte offset
// within the row in bits 16-31.
struct DmaLanes {
  uint32_t pk[6];
};

__device__ __forceinline__ DmaLanes dma_lanes(int wave, int lane) {
  DmaLanes d;
#pragma unroll
  for (int i = 0; i < 6; ++i) {
    const int c = 64 * (dma_first(wave) + i) + lane;
    const int r = min(c / kMlaRowPieces, kMlaKeys - 1);
    d.pk[i] = (uint32_t)(8 * r) | ((uint32_t)(16 * (c - r * kMlaRowPieces)) << 16);
  }
  return d;
}

__device__ __forceinline__ uint64_t dma_addr(const uint8_t* tab, uint32_t pk) {
  return *reinterpret_cast<const uint64_t*>(tab + (pk & 0xffffu)) + (pk >> 16);
}

// Send this wave's loads of a block into `buf` (the table must hold its rows):
// runs of up to four share one M0 value, the immediate offset moving both the
// global and the LDS address by 1 KB steps.
__device__ __forceinline__ void issue_block(const uint8_t* smem, int j, const DmaLanes& d, const uint8_t* buf,
                                            int wave) {
  const uint8_t* tab = smem + kAddrOff + (j & 1) * 512;
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_addr(buf) + 1024 * dma_first(wave));
  const uint64_t a0 = dma_addr(tab, d.pk[0]);
  const uint64_t a1 = dma_addr(tab, d.pk[1]) - 1024;
  const uint64_t a2 = dma_addr(tab, d.pk[2]) - 2048;
  const uint64_t a3 = dma_addr(tab, d.pk[3]) - 3072;
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off\n\tglobal_load_lds_dwordx4 %1, off offset:1024\n\t"
               "global_load_lds_dwordx4 %2, off offset:2048\n\tglobal_load_lds_dwordx4 %3, off offset:3072"
               ::"v"(a0), "v"(a1), "v"(a2), "v"(a3), "{m0}"(m0) : "memory");
  const uint32_t m1 = __builtin_amdgcn_readfirstlane(lds_addr(buf) + 1024 * (dma_first(wave) + 4));
  const uint64_t b0 = dma_addr(tab, d.pk[4]);
  if (dma_count(wave) == 6) {
    const uint64_t b1 = dma_addr(tab, d.pk[5]) - 1024;
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off\n\tglobal_load_lds_dwordx4 %1, off offset:1024"
                 ::"v"(b0), "v"(b1), "{m0}"(m1) : "memory");
  } else {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(b0), "{m0}"(m1) : "memory");
  }
}

// A fresh block's 36 loads: five each for waves 0-3, four for waves 4-7; lane l
// of load i takes piece c = 64(first + i) + l of the packed 32 rows.
__device__ __forceinline__ void issue_fresh_block(const uint8_t* smem, int j, const uint8_t* buf, int wave,
                                                  int lane) {
  const uint8_t* tab = smem + kAddrOff + (j & 1) * 512;
  const int first = wave < 4 ? 5 * wave : 20 + 4 * (wave - 4);
  const int cnt = wave < 4 ? 5 : 4;
  for (int i = 0; i < cnt; ++i) {
    const int pc = 64 * (first + i) + lane;
    const int r = pc / kFreshRowPieces;
    const uint64_t g = *reinterpret_cast<const uint64_t*>(tab + 8 * r) + 16 * (pc - r * kFreshRowPieces);
    dma16(reinterpret_cast<const void*>(g), lds_addr(buf + 1024 * (first + i)));
  }
}
static_assert(4 * 5 + 4 * 4 == kFreshDma, "fresh block loads per wave");

// The row indices of block j into ring slot j % 5: 64 cache slots, or 32 fresh
// row indices (lanes 32-63 repeat lanes 0-31).
template <bool kFresh>
__device__ __forceinline__ void issue_index(const MlaParams& P, uint8_t* smem, const MlaCtx& c, int j) {
  const int32_t* src =
      !kFresh || j < c.ncached ? P.idx + (int64_t)c.t_tok * P.idx_stride + c.key_begin + j * kMlaKeys + c.lane
                    : P.fresh_idx + (int64_t)c.t_tok * P.fresh_idx_stride + (j - c.ncached) * kFreshKeys +
                          (c.lane & (kFreshKeys - 1));
  dma4(src, __builtin_amdgcn_readfirstlane(lds_addr(smem + kRingOff + (j % kRingSlots) * 256)));
}


// Start of iteration t (both roles, every wave): the index load of block t+4;
// this wave's share of block t+1's rows.
template <bool kFresh>
__device__ __forceinline__ void iteration_start(const MlaParams& P, uint8_t* smem, const MlaCtx& c,
                                                const DmaLanes& dl, int t) {
  if (c.wave == kIdxWave && t + 4 < c.nblk) issue_index<kFresh>(P, smem, c, t + 4);
  if (t + 1 < c.nblk) {
    uint8_t* buf = smem + ((t + 1) % kNumBufs) * kBufBytes;
    if (!kFresh || t + 1 < c.ncached) issue_block(smem, t + 1, dl, buf, c.wave);
    else issue_fresh_block(smem, t + 1, buf, c.wave, c.lane);
  }
}
// End of iteration t: this wave's loads (block t+1's rows, index loads) have
// landed; after the barrier every wave sees block t+1's rows and P(t).
__device__ __forceinline__ void iteration_end() {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  barrier();
}

// QK waves: S of block t over this wave's 32 keys, its lazy reference, P(t).
template <bool kFresh>
__device__ __forceinline__ void qk_waves(const MlaParams& P, uint8_t* smem, const MlaCtx& c, const DmaLanes& dl) {
  const int lane = c.lane, h = c.h, c32 = c.c32, hp = c.hp, kh = c.kh;
  // the query as the B operand over all dims: nope chunk k (64 dims), k-step j =
  // dims 64k + 32h + 8j .. +7, the same dims the key operand converts from its
  // row bytes; rope k-step r = bf16 dims 512 + 16r + 8h .. +7
  v4i qn[8][4];
  v4i qr[4];
  {
    const uint16_t* qh = P.q + (int64_t)c.t_tok * P.q_tok_stride + (int64_t)(c.head_ok ? c.head : 0) * P.q_head_stride;
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
      for (int j = 0; j < 4; ++j) qn[k][j] = *reinterpret_cast<const v4i*>(qh + 64 * k + 32 * h + 8 * j);
#pragma unroll
    for (int r = 0; r < 4; ++r) qr[r] = *reinterpret_cast<const v4i*>(qh + 512 + 16 * r + 8 * h);
  }
  // in registers before the loop: a wait the compiler places for these loads
  // inside the loop would also wait for every copy in flight (0x0f70 = vmcnt(0))
  __builtin_amdgcn_s_waitcnt(0x0f70);
  float* ref = reinterpret_cast<float*>(smem + kRefOff);
  float m_run = -__builtin_inff();  // this key half's reference per head c32 (an integer, log2 units)
  float m_max = -__builtin_inff();  // exact running maximum (log2 units), for max_out
  float l_run = 0.f;                // sum of P against m_run, this lane's keys only

  for (int t = 0; t <= c.nblk; ++t) {
    iteration_start<kFresh>(P, smem, c, dl, t);
    // row addresses of block t+2 (its indices landed two iterations ago); the
    // table slot was last read when block t was issued, before this iteration
    if (c.wave == kTabWave && t + 2 < c.nblk) build_addr_table<kFresh>(P, smem, c, t + 2);
    // a fresh block has 32 keys, all in key half 0
    const bool fresh = kFresh && t >= c.ncached;
    if (t < c.nblk && !(fresh && kh == 1)) {
      const uint8_t* buf = smem + (t % kNumBufs) * kBufBytes;
      const int32_t slot_t = reinterpret_cast<const int32_t*>(smem + kRingOff + (t % kRingSlots) * 256)[lane];
      const uint64_t vmask = __ballot(fresh ? fresh_valid(P, slot_t, lane) : slot_valid(P, slot_t));
      // s[r]: key 32kh + 8(r/4) + 4h + r%4, head c32
      v16f s;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = 0.f;
      if (fresh) {
        // bf16 rows: the key operand is read as is
        const uint8_t* frow = buf + c32 * kFreshRowBytes;
#pragma unroll
        for (int k = 0; k < 8; ++k)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const v4i kb = *reinterpret_cast<const v4i*>(frow + 2 * (64 * k + 32 * h + 8 * j));
            s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_v8bf(kb), as_v8bf(qn[k][j]), s, 0, 0, 0);
          }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const v4i rope = *reinterpret_cast<const v4i*>(frow + 2 * (512 + 16 * r + 8 * h));
          s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_v8bf(rope), as_v8bf(qr[r]), s, 0, 0, 0);
        }
      } else {
      const uint8_t* row = buf + (32 * kh + c32) * kMlaRowBytes;
      const v4f ksc = *reinterpret_cast<const v4f*>(row + 512);
      const uint8_t* krow = row + 32 * h;
      v8i kraw[2];
      kraw[0] = lds_read32(krow);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        if (k + 1 < 8) kraw[(k + 1) & 1] = lds_read32(krow + 64 * (k + 1));
        const float sc = ksc[k >> 1];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const v8i& kr = kraw[k & 1];
          v4i kb;
          kb[0] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(kr[2 * j], sc, false));
          kb[1] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(kr[2 * j], sc, true));
          kb[2] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(kr[2 * j + 1], sc, false));
          kb[3] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(kr[2 * j + 1], sc, true));
          s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_v8bf(kb), as_v8bf(qn[k][j]), s, 0, 0, 0);
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const v4i rope = *reinterpret_cast<const v4i*>(row + 528 + 32 * r + 16 * h);
        s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_v8bf(rope), as_v8bf(qr[r]), s, 0, 0, 0);
      }
      }
      // invalid keys score -inf (their rows are zeros); the masks are skipped
      // when every key of the block is valid, the usual case
      const bool all_valid = vmask == ~0ull;
      uint32_t vb16 = 0xffffu;  // bit r: key 32kh + 8(r/4) + 4h + r%4 valid
      if (!all_valid) {
        const uint64_t vm = vmask >> (32 * kh + 4 * h);
        vb16 = (uint32_t)(vm & 0xfu) | ((uint32_t)((vm >> 8) & 0xfu) << 4) | ((uint32_t)((vm >> 16) & 0xfu) << 8) |
               ((uint32_t)((vm >> 24) & 0xfu) << 12);
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (!((vb16 >> r) & 1u)) s[r] = -__builtin_inff();
      }
      float mloc = fmaxf(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])), fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
      mloc = fmaxf(mloc, fmaxf(fmaxf(fmaxf(s[8], s[9]), fmaxf(s[10], s[11])),
                               fmaxf(fmaxf(s[12], s[13]), fmaxf(s[14], s[15]))));
      mloc = fmaxf(mloc, shfl_xor(mloc, 32));
      const float mblk = mloc * P.scale_log2;
      m_max = fmaxf(m_max, mblk);
      // lazy reference: it moves (to an integer) only when a block exceeds it by 2^8
      const bool need = mblk > m_run + kRescaleThreshold;
      if (__ballot(need)) {
        const float m_new = need ? ceilf(mblk) : m_run;
        l_run *= __builtin_amdgcn_exp2f(m_run - m_new);  // a power of two (0 from -inf)
        m_run = m_new;
      }
      const float m_use = m_run == -__builtin_inff() ? 0.f : m_run;
      float pv[16];
#pragma unroll
      for (int r = 0; r < 16; ++r)
        pv[r] = __builtin_amdgcn_exp2f(fmaxf(fmaf(s[r], P.scale_log2, -m_use), kMinLogP));
      if (!all_valid) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (!((vb16 >> r) & 1u)) pv[r] = 0.f;
      }
      float lsum = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) lsum += pv[r];
      l_run += lsum;
      if (fresh && !all_valid) {
        // An invalid key's V is the zero row, so any finite P' leaves O alone.
        // The PV waves scale a fresh block's P by adding f in [-30, 0] to the
        // bf16 exponent field with no tile-scale term, which takes a P of 0 to
        // -inf for f = -1 (0 * -inf = NaN): write 1.0 instead (P' = 2^f).
        // (A cache block's term for the zero row's scale keeps 0 finite.)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (!((vb16 >> r) & 1u)) pv[r] = 1.f;
      }
      // P as the PV A operand of k-steps 2kh, 2kh+1: lane (c32, h) holds head
      // c32, keys 16ks + 8(j/4) + 4h + j%4 (j = 0..7)
      uint8_t* pb = smem + kPOff + (t & 1) * 8192 + hp * 4 * 1024;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const v4i pw = {cvt_pk_bf16(pv[8 * i], pv[8 * i + 1]), cvt_pk_bf16(pv[8 * i + 2], pv[8 * i + 3]),
                        cvt_pk_bf16(pv[8 * i + 4], pv[8 * i + 5]), cvt_pk_bf16(pv[8 * i + 6], pv[8 * i + 7])};
        *reinterpret_cast<v4i*>(pb + ((2 * kh + i) * 64 + lane) * 16) = pw;
      }
    }
    if (t < c.nblk && h == 0) ref[(((t & 1) * 2 + hp) * 2 + kh) * 32 + c32] = m_run;
    iteration_end();
  }
  // sums (both lane halves), references and maxima of this key half
  float* fin = reinterpret_cast<float*>(smem + kFinOff);
  const float l2 = l_run + shfl_xor(l_run, 32);
  if (h == 0) {
    fin[(hp * 2 + kh) * 32 + c32] = l2;
    fin[128 + (hp * 2 + kh) * 32 + c32] = m_run;
    fin[256 + (hp * 2 + kh) * 32 + c32] = m_max;
  }
  barrier();
}

// PV waves: O += P'(t-1) . V(t-1) against R, then the normalised output.
// Wave dq = w - 4 owns O[64 heads x dims 128dq .. 128dq+127], exactly V tile
// dq, as two head tiles (the head halves): each V byte is converted once per
// workgroup, and one exponent per key scales both tiles' P.
template <bool kFresh>
__device__ __forceinline__ void pv_waves(const MlaParams& P, uint8_t* smem, const MlaCtx& c, const DmaLanes& dl,
                                         int split) {
  const int lane = c.lane, h = c.h, c32 = c.c32, dq = c.wave - 4;
  const float* ref = reinterpret_cast<const float*>(smem + kRefOff);
  // this wave's exponent table (V tile dq): [4 k-steps][2 h][8 u16], written
  // as 16-bit entries and read back as 16-byte vectors through a type that
  // may alias them (so the reads stay after the writes)
  typedef int v4i_alias __attribute__((ext_vector_type(4), may_alias));
  uint16_t* et = reinterpret_cast<uint16_t*>(smem + kEOff) + dq * 256;
  v16f o[2][4];  // o[mt][nn][r]: head 32mt + 8(r/4) + 4h + r%4 of the workgroup, dim 128dq + 32nn + c32
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[mt][i][r] = 0.f;
  float R[2] = {-__builtin_inff(), -__builtin_inff()};  // reference of O per head tile, head c32 (log2 units)
  // transposing V reads: lane (G = lane/16, m = lane%16) addresses key row
  // 8(e/4) + 4h + e%4 (e = m/2) and dims (G%2)*16 + 8(m%2) of each 32-dim tile
  const int m16 = lane & 15, G = lane >> 4;
  const int e8 = m16 >> 1;
  const uint32_t vlane = (uint32_t)((8 * (e8 >> 2) + 4 * h + (e8 & 3)) * kMlaRowBytes + 128 * dq + (G & 1) * 16 +
                                    8 * (m16 & 1));
  // transposing bf16 reads of a fresh block: lane (G = lane/16, m = lane%16)
  // addresses key row 4h + m/4 (+8) and dims 16(G%2) + 4(m%4) .. +3 of each
  // 32-dim tile, and receives dim 16(G%2) + m of four consecutive keys
  const uint32_t flane = (uint32_t)((4 * h + (m16 >> 2)) * kFreshRowBytes +
                                    2 * (128 * dq + 16 * (G & 1) + 4 * (m16 & 3)));

  for (int t = 0; t <= c.nblk; ++t) {
    iteration_start<kFresh>(P, smem, c, dl, t);
    if (t >= 1) {
      const int par = (t - 1) & 1;
      const uint8_t* bufp = smem + ((t - 1) % kNumBufs) * kBufBytes;
      const bool fresh = kFresh && t - 1 >= c.ncached;
      if (!fresh) {
        // exponent table of block t-1, tile dq (lane = key): the tile scale's
        // exponent in the bf16 exponent field, at the PV A operand position of
        // the key (k-step key/16, lane half (key/4)%2, element 4((key/8)%2) + key%4)
        const int key = lane;
        const uint32_t sb = *reinterpret_cast<const uint32_t*>(bufp + key * kMlaRowBytes + 512 + 4 * dq);
        const int pos = ((key >> 4) * 2 + ((key >> 2) & 1)) * 8 + 4 * ((key >> 3) & 1) + (key & 3);
        et[pos] = (uint16_t)((uint32_t)((((int)((sb >> 23) & 0xffu)) - 127) << 7) & 0xffffu);
      }
      // each head tile's O follows the larger of its key-half references; O
      // moves by a power of two
      int fx[2][2];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const float m0 = ref[((par * 2 + mt) * 2 + 0) * 32 + c32];
        const float m1 = ref[((par * 2 + mt) * 2 + 1) * 32 + c32];
        const float mn = fmaxf(m0, m1);
        const bool up = mn > R[mt];
        if (__ballot(up)) {
          const float alpha = up ? __builtin_amdgcn_exp2f(R[mt] - mn) : 1.f;  // 0 from -inf
          R[mt] = up ? mn : R[mt];
          int hb = 4 * h;
          asm volatile("" : "+v"(hb));
          float ar[16];
#pragma unroll
          for (int r = 0; r < 16; ++r) ar[r] = __shfl(alpha, 8 * (r >> 2) + hb + (r & 3), 64);
#pragma unroll
          for (int nn = 0; nn < 4; ++nn)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[mt][nn][r] *= ar[r];
        }
        // per key half: m_kh - R (<= 0) for the bf16 exponent field (a key half
        // with no valid key yet has only zero rows in this block, so any finite
        // P' is fine there; a half more than 2^30 below R is scaled by 2^-30
        // instead of 2^f, which keeps P' a normal number)
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
          const float mk = k2 == 0 ? m0 : m1;
          const int f = mk == -__builtin_inff() ? 0 : max((int)(mk - R[mt]), kDropExp);
          fx[mt][k2] = (f << 7) & 0xffff;
          fx[mt][k2] |= fx[mt][k2] << 16;
        }
      }
      const uint8_t* pb = smem + kPOff + par * 8192;
      const uint32_t vb = lds_addr(bufp) + vlane;
      // The transposing reads take no immediate offset, so each address is
      // formed from an opaque base right before use; otherwise all of them
      // would be hoisted out of the loop into registers.
      auto vaddr = [&](int ks) {
        uint32_t a = vb + (16 * ks) * kMlaRowBytes;
        asm volatile("" : "+v"(a));
        return a;
      };
      // k-step ks: its P (both head tiles), exponent and V reads issued one
      // k-step ahead
      v2i vq[2][4];
      v4i pq[2][2], eq[2];
      {
        const uint32_t a0 = vaddr(0);
#pragma unroll
        for (int nn = 0; nn < 4; ++nn) vq[0][nn] = lds_read_tr8_at(a0 + 32 * nn);
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) pq[0][mt] = *reinterpret_cast<const v4i*>(pb + mt * 4096 + lane * 16);
        eq[0] = *reinterpret_cast<const v4i_alias*>(et + h * 8);
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int cur = ks & 1, nxt = cur ^ 1;
        if (ks + 1 < 4) {
          const uint32_t a1 = vaddr(ks + 1);
#pragma unroll
          for (int nn = 0; nn < 4; ++nn) vq[nxt][nn] = lds_read_tr8_at(a1 + 32 * nn);
#pragma unroll
          for (int mt = 0; mt < 2; ++mt)
            pq[nxt][mt] = *reinterpret_cast<const v4i*>(pb + mt * 4096 + ((ks + 1) * 64 + lane) * 16);
          eq[nxt] = *reinterpret_cast<const v4i_alias*>(et + ((ks + 1) * 2 + h) * 8);
        }
        const int k2 = ks >> 1;  // k-steps 0, 1: key half 0; 2, 3: key half 1
        if (fresh && ks >= 2) continue;  // a fresh block's 32 keys are k-steps 0, 1
        v4i pa[2];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            // (bit_cast of a vector element reads element 0; copy to scalars first)
            const int pe = pq[cur][mt][e], ee = fresh ? 0 : eq[cur][e];
            const v2u16 sum = __builtin_bit_cast(v2u16, pe) + __builtin_bit_cast(v2u16, ee) +
                              __builtin_bit_cast(v2u16, fx[mt][k2]);
            pa[mt][e] = __builtin_bit_cast(int, sum);
          }
#pragma unroll
        for (int nn = 0; nn < 4; ++nn) {
          v8bf vop;
          if (fresh) {
            // bf16 V, no tile scale: two transposing reads give keys 4h + 0..3 and 8 + 4h + 0..3
            uint32_t a = lds_addr(bufp) + flane + 16 * ks * kFreshRowBytes + 2 * (32 * nn);
            asm volatile("" : "+v"(a));
            const v4s lo = lds_read_tr16_at(a);
            const v4s hi = lds_read_tr16_at(a + 8 * kFreshRowBytes);
            const v8s vv = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            vop = __builtin_bit_cast(v8bf, vv);
          } else {
            vop = fp8x8_to_bf16(vq[cur][nn]);
          }
#pragma unroll
          for (int mt = 0; mt < 2; ++mt)
            o[mt][nn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_v8bf(pa[mt]), vop, o[mt][nn], 0, 0, 0);
        }
      }
    }
    iteration_end();
  }
  barrier();  // the QK waves' sums, references and maxima are in LDS
  const float* fin = reinterpret_cast<const float*>(smem + kFinOff);
  const int hg_base = c.h_half - c.hp * 32;  // the workgroup's first head
  int hb = 4 * h;
  asm volatile("" : "+v"(hb));
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    // total of P per head c32 of tile mt against R, and the exact maximum
    float lt = 0.f, mm = -__builtin_inff();
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      const float lk = fin[(mt * 2 + k2) * 32 + c32];
      const float mk = fin[128 + (mt * 2 + k2) * 32 + c32];
      if (mk != -__builtin_inff()) lt += lk * __builtin_amdgcn_exp2f(mk - R[mt]);
      mm = fmaxf(mm, fin[256 + (mt * 2 + k2) * 32 + c32]);
    }
    const bool any = lt > 0.f;
    const float inv = any ? 1.f / lt : 0.f;
    const float lse = any ? (R[mt] + __builtin_amdgcn_logf(lt)) * kLn2 : -__builtin_inff();
    const int h_half = hg_base + 32 * mt;
    if (h_half >= P.H) continue;
    const int head = h_half + c32;
    const bool head_ok = head < P.H;
    if (P.splits == 1) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int hr = 8 * (r >> 2) + 4 * h + (r & 3);
        const float ir = __shfl(inv, 8 * (r >> 2) + hb + (r & 3), 64);
        if (h_half + hr < P.H) {
          uint16_t* orow = P.out + ((int64_t)c.t_tok * P.H + h_half + hr) * kMlaDv + 128 * dq + c32;
#pragma unroll
          for (int nn = 0; nn < 4; ++nn) orow[32 * nn] = (uint16_t)f32_to_bf16_rne(o[mt][nn][r] * ir);
        }
      }
      if (dq == 0 && h == 0 && head_ok) {
        if (P.lse) P.lse[(int64_t)c.t_tok * P.H + head] = lse;
        if (P.max_out) P.max_out[(int64_t)c.t_tok * P.H + head] = any ? mm * kLn2 : -__builtin_inff();
      }
    } else {
      const int64_t row0 = ((int64_t)split * P.T + c.t_tok) * P.H + h_half;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int hr = 8 * (r >> 2) + 4 * h + (r & 3);
        const float ir = __shfl(inv, 8 * (r >> 2) + hb + (r & 3), 64);
        if (h_half + hr < P.H) {
          float* orow = P.ws_o + (row0 + hr) * kMlaDv + 128 * dq + c32;
#pragma unroll
          for (int nn = 0; nn < 4; ++nn) orow[32 * nn] = o[mt][nn][r] * ir;
        }
      }
      if (dq == 0 && h == 0 && head_ok) P.ws_lse[row0 + c32] = lse;
    }
  }
}

// kFresh: a chunked prefill's token lists (cache slots, then fresh bf16 rows);
// decode instantiates the kernel without that path.
template <bool kFresh>
__global__ void __launch_bounds__(kMlaThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
sparse_mla_kernel(const MlaParams P) {
  extern __shared__ __align__(16) uint8_t smem[];
  MlaCtx c;
  c.lane = threadIdx.x & 63;
  c.wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  c.h = c.lane >> 5;
  c.c32 = c.lane & 31;
  c.hp = (c.wave & 3) >> 1;
  c.kh = c.wave & 1;
  // XCD-aware order: consecutive logical work items (the head groups and
  // splits of one token) land on the same XCD and share its L2.
  const int nwg = gridDim.x;
  int work = blockIdx.x;
  if ((nwg & 7) == 0) work = (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3);
  const int per_tok = P.head_groups * P.splits;
  c.t_tok = work / per_tok;
  const int rem = work % per_tok;
  const int hg = rem / P.splits;
  const int split = rem % P.splits;
  const int chunk = P.topk / P.splits;
  c.key_begin = split * chunk;
  c.nblk = chunk / kMlaKeys;
  c.ncached = c.nblk;
  if (kFresh) {
    const int nc = __builtin_amdgcn_readfirstlane(P.counts[2 * c.t_tok]);
    const int nf = __builtin_amdgcn_readfirstlane(P.counts[2 * c.t_tok + 1]);
    c.ncached = (nc + kMlaKeys - 1) / kMlaKeys;
    c.nblk = c.ncached + (nf + kFreshKeys - 1) / kFreshKeys;
  }
  c.h_half = hg * kMlaHeadsPerWG + c.hp * 32;
  c.head = c.h_half + c.c32;
  c.head_ok = c.head < P.H;

  // prologue: the indices of blocks 0-3, the address tables of blocks 0 and
  // 1, block 0's rows
  if (c.wave == kIdxWave) {
    for (int j = 0; j < 4 && j < c.nblk; ++j) issue_index<kFresh>(P, smem, c, j);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  barrier();
  const DmaLanes dl = dma_lanes(c.wave, c.lane);
  if (c.wave == kTabWave) {
    if (c.nblk > 0) build_addr_table<kFresh>(P, smem, c, 0);
    if (c.nblk > 1) build_addr_table<kFresh>(P, smem, c, 1);
  }
  barrier();
  if (c.nblk > 0) {
    if (!kFresh || c.ncached > 0) issue_block(smem, 0, dl, smem, c.wave);
    else issue_fresh_block(smem, 0, smem, c.wave, c.lane);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  barrier();  // block 0's rows are in LDS
  // both roles run the same number of iterations and barriers
  if (c.wave < 4) qk_waves<kFresh>(P, smem, c, dl);
  else pv_waves<kFresh>(P, smem, c, dl, split);
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
  // A workgroup's time is a fixed start-up plus a cost per 64-row block, and
  // one workgroup runs per CU at a time: split as far as the grid still fits
  // the CUs in one round (a second round costs a whole workgroup's time), and
  // keep at least 4 blocks per workgroup (below that the start-up and the
  // combine outweigh the shorter key list). Splits must divide topk into
  // 64-row blocks.
  const int max_splits = std::min(8, topk / (4 * dsa::kMlaKeys));
  int splits = 1;
  while (splits * 2 <= max_splits && base * splits * 2 <= num_cus && (topk / (splits * 2)) % dsa::kMlaKeys == 0)
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
                          int64_t kv_num_blocks, const int32_t* indices, int64_t idx_stride, int num_tokens,
                          int num_heads, int topk, float sm_scale, void* out, float* lse, int num_splits,
                          void* workspace, size_t workspace_bytes, void* stream) {
  return dsa::sparse_mla_decode_impl(q, q_token_stride, q_head_stride, kv_cache, kv_block_stride_bytes,
                                     kv_block_size, kv_num_blocks, indices, idx_stride, num_tokens, num_heads, topk,
                                     sm_scale, out, lse, num_splits, workspace, workspace_bytes, stream, nullptr,
                                     nullptr);
}

}  // extern "C"

namespace dsa {

int sparse_mla_decode_impl(const void* q, int64_t q_token_stride, int64_t q_head_stride, const uint8_t* kv_cache,
                           int64_t kv_block_stride_bytes, int kv_block_size, int64_t kv_num_blocks,
                           const int32_t* indices, int64_t idx_stride, int num_tokens, int num_heads, int topk,
                           float sm_scale, void* out, float* lse, int num_splits, void* workspace,
                           size_t workspace_bytes, void* stream, float* max_out, const MlaFresh* fresh) {
  if (num_tokens < 0 || num_heads <= 0 || (num_heads % 16) != 0)
    return set_error(kUnsupported, "sparse_mla: num_heads=%d must be a positive multiple of 16", num_heads);
  if (topk <= 0 || topk % kMlaKeys != 0)
    return set_error(kUnsupported, "sparse_mla: topk=%d must be a positive multiple of %d", topk, kMlaKeys);
  if (kv_block_size <= 0 || kv_block_stride_bytes < (int64_t)kv_block_size * kMlaRowBytes)
    return set_error(kInvalidArgument, "sparse_mla: kv block stride %lld < %d rows x 656 B",
                     (long long)kv_block_stride_bytes, kv_block_size);
  if (kv_block_stride_bytes % 16 != 0)
    return set_error(kInvalidArgument, "sparse_mla: kv block stride must be a multiple of 16 bytes");
  if (kv_num_blocks < 0) return set_error(kInvalidArgument, "sparse_mla: kv_num_blocks < 0");
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
    smem_status = hipFuncSetAttribute((const void*)sparse_mla_kernel<false>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMlaSmemBytes) == hipSuccess &&
                          hipFuncSetAttribute((const void*)sparse_mla_kernel<true>,
                                              hipFuncAttributeMaxDynamicSharedMemorySize,
                                              (int)kMlaSmemBytes) == hipSuccess
                      ? 0 : 1;
  }
  if (smem_status) return set_error(kLaunchFailed, "sparse_mla: cannot reserve %zu B of LDS", kMlaSmemBytes);

  MlaParams P;
  P.kv_block_shift = (kv_block_size & (kv_block_size - 1)) == 0 ? __builtin_ctz((unsigned)kv_block_size) : -1;
  P.q = static_cast<const uint16_t*>(q);
  P.q_tok_stride = q_token_stride;
  P.q_head_stride = q_head_stride;
  P.kv = kv_cache;
  P.kv_blk_stride = kv_block_stride_bytes;
  P.kv_block_size = kv_block_size;
  P.kv_num_blocks = kv_num_blocks;
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
  P.max_out = num_splits == 1 ? max_out : nullptr;
  P.counts = nullptr;
  P.fresh = nullptr;
  P.fresh_row_stride = 0;
  P.fresh_rows = 0;
  P.fresh_idx = nullptr;
  P.fresh_idx_stride = 0;
  if (fresh) {
    if (num_splits != 1) return set_error(kInvalidArgument, "sparse_mla: fresh rows need num_splits == 1");
    if (!fresh->counts || (fresh->num_rows > 0 && (!fresh->rows || !fresh->idx)))
      return set_error(kInvalidArgument, "sparse_mla: null fresh-row pointer");
    if ((reinterpret_cast<uintptr_t>(fresh->rows) & 15) || (fresh->row_stride % 8) ||
        (fresh->num_rows > 0 && fresh->row_stride < 576))
      return set_error(kInvalidArgument, "sparse_mla: fresh rows must be 16-byte aligned bf16 rows of >= 576");
    P.counts = fresh->counts;
    P.fresh = static_cast<const uint16_t*>(fresh->rows);
    P.fresh_row_stride = fresh->row_stride;
    P.fresh_rows = fresh->num_rows;
    P.fresh_idx = fresh->idx;
    P.fresh_idx_stride = fresh->idx_stride;
  }
  if (num_splits > 1) {
    const size_t rows = (size_t)num_splits * num_tokens * num_heads;
    P.ws_o = static_cast<float*>(workspace);
    P.ws_lse = P.ws_o + rows * kMlaDv;
  }
  const int64_t nwg = (int64_t)num_tokens * P.head_groups * num_splits;
  if (fresh)
    hipLaunchKernelGGL(sparse_mla_kernel<true>, dim3((unsigned)nwg), dim3(kMlaThreads), kMlaSmemBytes,
                       (hipStream_t)stream, P);
  else
    hipLaunchKernelGGL(sparse_mla_kernel<false>, dim3((unsigned)nwg), dim3(kMlaThreads), kMlaSmemBytes,
                       (hipStream_t)stream, P);
  if (int rc = check_launch("dsa_sparse_mla_decode")) return rc;
  if (num_splits > 1) {
    hipLaunchKernelGGL(sparse_mla_combine_kernel, dim3((unsigned)(num_tokens * num_heads)), dim3(64), 0,
                       (hipStream_t)stream, P.ws_o, P.ws_lse, num_tokens, num_heads, num_splits, P.out, lse);
    return check_launch("dsa_sparse_mla_decode(combine)");
  }
  return kOk;
}

}  // namespace dsa
