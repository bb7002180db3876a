// Sparse MLA decode over the packed fp8 MLA cache, for gfx950.
//
// For each query token t and head h:
//   s_i = sm_scale * q[t,h,:576] . kv(idx_i)[:576]     (valid idx_i only)
//   o   = softmax(s) @ kv(idx)[:, :512],  lse = log(sum_i exp(s_i))
// where kv(slot) is a 656-byte row [512 e4m3fn][4 x f32 tile scale][64 bf16].
//
// Workgroup = 8 waves (two per SIMD) = 64 heads of one token over one key
// split. Two waves share each SIMD so that one wave's matrix work overlaps the
// other's vector work: a single wave issues a vector instruction only every
// ~7 cycles, so at one wave per SIMD this kernel would be bound by vector
// issue, not by the matrix cores. Each wave fits in 256 registers.
//
// Wave w = (head half hp = w/4, quarter q = w%4); its 32 heads are
// hp*32 + 0..31 of the workgroup's 64. Per block of 64 selected rows:
//   gather : the raw 656-byte rows go straight from HBM into LDS with
//            global_load_lds_dwordx4 - consecutive lanes take consecutive
//            16-byte pieces of the packed rows - into one of three buffers,
//            two blocks ahead of use. The row indices arrive the same way,
//            four blocks ahead, in a five-entry ring; one wave turns a block's
//            indices into a 64-entry row-address table in LDS, so a load costs
//            a table read and an add. Invalid indices read a zero row.
//   QK     : wave (kh = q/2, d = q%2) forms the partial S^T[32 keys x 32
//            heads] of keys 32kh..32kh+31 over nope dims [256d, 256d+256)
//            and rope dims [32d, 32d+32), all on v_mfma_f32_32x32x16_bf16:
//            A = the key's fp8 nope bytes from LDS converted to bf16 with the
//            row's tile scale (v_cvt_scalef32_pk_bf16_fp8; exact, since an
//            e4m3 value times a power of two is a bf16 value) and its bf16
//            rope; B = the query's bf16 values as given. Products are exact
//            and sums are f32, as in a bf16 dequantise-then-multiply. (The
//            scaled fp8 MFMA would take the raw rows directly, but it sums its
//            64 products to only ~14 bits below the largest one.)
//   reduce : the two dim halves are summed by a reduce-scatter through LDS:
//            wave (kh, d) ends with the full scores of keys 16o..16o+15,
//            o = 2kh + d, so each score is exponentiated exactly once.
//   softmax: per-head block maxima of the four key quarters are exchanged;
//            online softmax in the exp2 domain with lazy rescaling (the
//            running max moves only when a block raises it by more than 2^8).
//            P goes to LDS once, as bf16.
//   PV     : wave q produces output dims [128q, 128q+128) = V tile q of its
//            32 heads: O += P' . V on v_mfma_f32_32x32x16_bf16, P' = P * 2^e
//            with e the tile scale exponent of each key (a 16-bit add to the
//            bf16 exponent field, read from a per-block table), V read from
//            the raw rows with ds_read_b64_tr_b8 (8 keys x 1 dim per lane, the
//            B operand layout) and converted with unit scale.
// Splits over the key list (for small batches) write normalised partial
// outputs and LSEs to a caller-provided workspace; a combine kernel merges
// them with the LSE rule of merge_attention_states.
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
constexpr int kDmaPerBlock = kBufBytes / 1024;        // 41 wave-wide 16-byte loads per block
constexpr int kNumBufs = 3;
// LDS map (bytes)
constexpr int kXsOff = kNumBufs * kBufBytes;          // score partials: [8 waves][64 lanes][8 f32]
constexpr int kMxOff = kXsOff + kMlaWaves * 64 * 32;  // block maxima / final sums: [2 hp][32 heads][4 quarters] f32
constexpr int kPOff = kMxOff + 2 * 32 * 4 * 4;        // P: [2 hp][4 quarters][64 lanes][8 bf16]
constexpr int kEOff = kPOff + 2 * 4 * 64 * 16;        // exponent offsets, two blocks: [2][4 tiles][4 k-steps][2 halves][8 u16]
constexpr int kRingOff = kEOff + 2 * 4 * 4 * 2 * 16;  // row indices, one 64-entry block per slot
constexpr int kRingSlots = 5;
constexpr int kAddrOff = kRingOff + kRingSlots * 256;  // row addresses of blocks being gathered, [2][64] u64
constexpr size_t kMlaSmemBytes = kAddrOff + 2 * kMlaKeys * 8;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kRescaleThreshold = 8.0f;  // log2 units
// Smallest P kept for a valid key (log2): P' = P * 2^e is formed by adding e to
// the bf16 exponent field, which needs P to be a normal number.
constexpr float kMinLogP = -60.0f;
constexpr int kIdxWave = 7;                // the wave that fetches the row indices

static_assert(kBufBytes % 1024 == 0, "a block of rows must be whole wave-wide loads");
static_assert(kMlaSmemBytes <= 160 * 1024, "LDS budget");

// Source of the pieces of an invalid row: 656 zero bytes.
__device__ __align__(16) uint8_t g_mla_zero_row[kMlaRowBytes];

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
  int compact;    // the valid indices of a row come first: stop at the first block with none
};

// ---- asynchronous global -> LDS copies. They are issued from inline asm so
// that the compiler neither inserts vmcnt(0) before every LDS read nor waits
// for them at barriers: the kernel counts them itself with wait_vm().
// `lds` is the wave's destination base (M0); lane i writes lds + 4*size*i.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}
__device__ __forceinline__ void dma4(const void* g, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}
// Wait until at most n of this wave's copies are outstanding (n in {0, 1, 5, 6}).
__device__ __forceinline__ void wait_vm(int n) {
  if (n >= 6) asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
  else if (n == 5) asm volatile("s_waitcnt vmcnt(5)" ::: "memory");
  else if (n >= 1) asm volatile("s_waitcnt vmcnt(1)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
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

__device__ __forceinline__ v2i lds_read_tr8(const uint8_t* p) {
  typedef __attribute__((address_space(3))) v2i lds_v2i;
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)p);
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
constexpr int kTabWave = 6;  // the wave that builds the row-address table

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

// Table of block j's row addresses from ring slot j % 5 (lane = row), in table j % 2.
__device__ __forceinline__ void build_addr_table(const MlaParams& P, uint8_t* smem, int j, int lane) {
  const int32_t slot = reinterpret_cast<const int32_t*>(smem + kRingOff + (j % kRingSlots) * 256)[lane];
  *reinterpret_cast<uint64_t*>(smem + kAddrOff + (j & 1) * 512 + 8 * lane) = row_address(P, slot);
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
              "wait_vm() counts 6 / 5 loads per wave");

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

__device__ __forceinline__ void issue_index(const MlaParams& P, uint8_t* smem, int t, int key_begin, int j,
                                            int lane) {
  const int32_t* src = P.idx + (int64_t)t * P.idx_stride + key_begin + j * kMlaKeys + lane;
  dma4(src, __builtin_amdgcn_readfirstlane(lds_addr(smem + kRingOff + (j % kRingSlots) * 256)));
}

__global__ void __launch_bounds__(kMlaThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
sparse_mla_kernel(const MlaParams P) {
  extern __shared__ __align__(16) uint8_t smem[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = lane >> 5, c32 = lane & 31;
  const int hp = wave >> 2, q4 = wave & 3;
  const int kh = q4 >> 1, d = q4 & 1;  // QK: key half, dim half
  const int o4 = 2 * kh + d;           // owned key quarter after the reduce-scatter
  const int jt = q4;                   // PV: V tile (output dims [128 jt, 128 jt + 128))

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

  const int h_half = hg * kMlaHeadsPerWG + hp * 32;  // first head of this wave's 32
  const int head = h_half + c32;                     // this lane's head (score columns)
  const bool head_ok = head < P.H;

  // The indices of blocks 0-3 are fetched first, so that their round trip
  // overlaps the query's (the wait for the query below covers them too).
  if (wave == kIdxWave)
    for (int j = 0; j < 4 && j < nblk; ++j) issue_index(P, smem, t, key_begin, j, lane);

  // Query B operands, bf16 as given: nope chunk c (64 dims), k-step j holds
  // dims 256d + 64c + 32h + 8j .. +7 for lane half h, the same dims the key
  // operand converts from its row bytes. Rope k-step rho: bf16 dims
  // 32d + 16rho + 8h + 0..7.
  v4i qn[4][4];
  v4i qr[2];
  {
    const uint16_t* qh = P.q + (int64_t)t * P.q_tok_stride + (int64_t)(head_ok ? head : 0) * P.q_head_stride;
    const v4i z = {0, 0, 0, 0};
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        qn[c][j] = head_ok ? *reinterpret_cast<const v4i*>(qh + 256 * d + 64 * c + 32 * h + 8 * j) : z;
#pragma unroll
    for (int rho = 0; rho < 2; ++rho)
      qr[rho] = head_ok ? *reinterpret_cast<const v4i*>(qh + 512 + 32 * d + 16 * rho + 8 * h) : z;
  }
  // The query must be in registers before the first copy is issued: a wait
  // the compiler places for these loads inside the block loop would also wait
  // for every copy in flight. (The builtin, unlike inline asm, is seen by the
  // compiler's wait bookkeeping.) 0x0f70 = vmcnt(0) only.
  __builtin_amdgcn_s_waitcnt(0x0f70);

  v16f o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[i][r] = 0.f;
  float m_run = -__builtin_inff();  // per head c32, log2 domain (identical in the 4 waves of a head half)
  float m_max = -__builtin_inff();  // exact running maximum (log2 domain), for max_out
  float l_run = 0.f;                // per head c32: this lane's 8 keys of each block only

  const int my_dma = dma_count(wave);
  // prologue: the indices of blocks 0-3 have landed (issued first, waited
  // for with the query); then the rows of blocks 0 and 1
  barrier();
  const DmaLanes dl = dma_lanes(wave, lane);
  if (wave == kTabWave) {
    build_addr_table(P, smem, 0, lane);
    if (nblk > 1) build_addr_table(P, smem, 1, lane);
  }
  barrier();
  issue_block(smem, 0, dl, smem, wave);
  if (nblk > 1) issue_block(smem, 1, dl, smem + kBufBytes, wave);
  // rows of block 0 have landed
  wait_vm(nblk > 1 ? my_dma : 0);
  barrier();

  float* xs_mine = reinterpret_cast<float*>(smem + kXsOff) + (wave * 64 + lane) * 8;
  const float* xs_part = reinterpret_cast<const float*>(smem + kXsOff) + ((wave ^ 1) * 64 + lane) * 8;
  float* mx = reinterpret_cast<float*>(smem + kMxOff) + (hp * 32 + c32) * 4;
  uint8_t* pbuf = smem + kPOff + hp * 4 * 1024;
  uint16_t* etab = reinterpret_cast<uint16_t*>(smem + kEOff);

  for (int n = 0; n < nblk; ++n) {
    // Block n's rows landed (and are visible) at the last barrier of block n-1.
    // The buffers, tables and rings a wave touches before its first barrier of
    // block n are ones no wave still in block n-1 reads: the exponent and address
    // tables are double-buffered by block parity.
    const uint8_t* buf = smem + (n % kNumBufs) * kBufBytes;
    const int32_t slot_n = reinterpret_cast<const int32_t*>(smem + kRingOff + (n % kRingSlots) * 256)[lane];
    const uint64_t vmask = __ballot(slot_valid(P, slot_n));
    // every wave reads the same indices, so all of them leave at the same block
    if (P.compact && vmask == 0ull) break;
    if (wave == kIdxWave && n + 4 < nblk) issue_index(P, smem, t, key_begin, n + 4, lane);
    // row addresses of block n+2 (its indices landed before the last barrier), read after B3
    if (wave == kTabWave && n + 2 < nblk) build_addr_table(P, smem, n + 2, lane);
    uint16_t* et = etab + (n & 1) * 256;

    // Exponent table of this block: entry (tile, key) = the tile scale's
    // exponent shifted into the bf16 exponent field, at the position the PV
    // A operand holds that key (k-step key/16, lane half (key/4)%2, element
    // 4((key/8)%2) + key%4).
    if (wave < 4) {
      const int key = lane, tile = wave;
      const uint32_t sb = *reinterpret_cast<const uint32_t*>(buf + key * kMlaRowBytes + 512 + 4 * tile);
      const int e = (int)((sb >> 23) & 0xffu) - 127;
      const int pos = ((tile * 4 + (key >> 4)) * 2 + ((key >> 2) & 1)) * 8 + 4 * ((key >> 3) & 1) + (key & 3);
      et[pos] = (uint16_t)((uint32_t)(e << 7) & 0xffffu);
    }

    // ---- partial S^T[32 keys x 32 heads] over this wave's dims:
    // s[r] = key 32kh + 8(r/4) + 4h + r%4, head c32
    v16f s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.f;
    {
      const uint8_t* row = buf + (32 * kh + c32) * kMlaRowBytes;
      const v2f ksc = *reinterpret_cast<const v2f*>(row + 512 + 8 * d);
      // K chunk c: lane half h holds bytes 256d + 64c + 32h .. +32 of key
      // 32kh + c32, dequantised to bf16 with the tile scale (exact: an e4m3
      // value times a power of two is a bf16 value), 8 per k-step
      const uint8_t* krow = row + 256 * d + 32 * h;
      v8i kraw[2];
      kraw[0] = lds_read32(krow);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if (c + 1 < 4) kraw[(c + 1) & 1] = lds_read32(krow + 64 * (c + 1));
        const float sc = ksc[c >> 1];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const v8i& kr = kraw[c & 1];
          v4i kb;
          kb[0] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(kr[2 * j], sc, false));
          kb[1] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(kr[2 * j], sc, true));
          kb[2] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(kr[2 * j + 1], sc, false));
          kb[3] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(kr[2 * j + 1], sc, true));
          s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_v8bf(kb), as_v8bf(qn[c][j]), s, 0, 0, 0);
        }
      }
#pragma unroll
      for (int rho = 0; rho < 2; ++rho) {
        const v4i rope = *reinterpret_cast<const v4i*>(row + 528 + 64 * d + 32 * rho + 16 * h);
        s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_v8bf(rope), as_v8bf(qr[rho]), s, 0, 0, 0);
      }
    }

    // ---- reduce-scatter with the dim partner (wave ^ 1): this wave keeps
    // s[8d .. 8d+7] = keys 16 o4 + 8(i/4) + 4h + i%4 (i = 0..7) and sends the rest.
    float sv[8];
    if (d == 0) {
      *reinterpret_cast<v4f*>(xs_mine) = v4f{s[8], s[9], s[10], s[11]};
      *reinterpret_cast<v4f*>(xs_mine + 4) = v4f{s[12], s[13], s[14], s[15]};
#pragma unroll
      for (int i = 0; i < 8; ++i) sv[i] = s[i];
    } else {
      *reinterpret_cast<v4f*>(xs_mine) = v4f{s[0], s[1], s[2], s[3]};
      *reinterpret_cast<v4f*>(xs_mine + 4) = v4f{s[4], s[5], s[6], s[7]};
#pragma unroll
      for (int i = 0; i < 8; ++i) sv[i] = s[8 + i];
    }
    barrier();  // B1
    {
      const v4f a = *reinterpret_cast<const v4f*>(xs_part);
      const v4f b = *reinterpret_cast<const v4f*>(xs_part + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sv[i] += a[i];
        sv[4 + i] += b[i];
      }
    }
    // invalid keys score -inf (their rows are zeros, so P' . V gets exact zeros)
    const uint64_t vm = vmask >> (16 * o4 + 4 * h);
    if (vmask != ~0ull) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (!((vm >> (8 * (i >> 2) + (i & 3))) & 1ull)) sv[i] = -__builtin_inff();
    }
    float mloc = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])), fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
    mloc = fmaxf(mloc, shfl_xor(mloc, 32));
    if (h == 0) mx[o4] = mloc;
    barrier();  // B2

    // ---- online softmax (exp2 domain), lazy rescale; the block maximum is
    // the same in the four waves of a head half, so are m_run and alpha
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
        // o rows are heads 8(r/4) + 4h + r%4
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
    // m_run is -inf only while every key so far was invalid; then p = 0
    const float m_use = m_run == -__builtin_inff() ? 0.f : m_run;
    float pv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      pv[i] = __builtin_amdgcn_exp2f(fmaxf(fmaf(sv[i], P.scale_log2, -m_use), kMinLogP));
    if (vmask != ~0ull) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (!((vm >> (8 * (i >> 2) + (i & 3))) & 1ull)) pv[i] = 0.f;
    }
    l_run += ((pv[0] + pv[1]) + (pv[2] + pv[3])) + ((pv[4] + pv[5]) + (pv[6] + pv[7]));
    {
      const v4i pw = {cvt_pk_bf16(pv[0], pv[1]), cvt_pk_bf16(pv[2], pv[3]), cvt_pk_bf16(pv[4], pv[5]),
                      cvt_pk_bf16(pv[6], pv[7])};
      *reinterpret_cast<v4i*>(pbuf + (o4 * 64 + lane) * 16) = pw;
    }
    // rows of block n+1 have landed: issued at the end of block n-1 (or in the
    // prologue); only the index wave's load of block n+4 went out after them
    if (n + 1 < nblk) wait_vm(wave == kIdxWave && n + 4 < nblk ? 1 : 0);
    barrier();  // B3

    // ---- O[32 heads x 128 dims] += P' . V over the block's 64 keys (four k-steps of 16).
    // Lane (group G = lane/16, m = lane%16) addresses key row 8(e/4) + 4h + e%4
    // (e = m/2) and dims (G%2)*16 + 8(m%2) of each 32-dim tile.
    {
      const int m16 = lane & 15, G = lane >> 4;
      const int e8 = m16 >> 1;
      const uint8_t* vb = buf + (8 * (e8 >> 2) + 4 * h + (e8 & 3)) * kMlaRowBytes + 128 * jt + (G & 1) * 16 +
                          8 * (m16 & 1);
      // The transposing reads take no immediate offset, so each address is
      // formed from an opaque base right before use; otherwise all of them
      // would be hoisted out of the block loop into registers.
      auto vstep = [&](int ks) {
        uint32_t a = lds_addr(vb) + (16 * ks) * kMlaRowBytes;
        asm volatile("" : "+v"(a));
        return a;
      };
      v2i vr[2][4];
      {
        const uint32_t p = vstep(0);
#pragma unroll
        for (int nn = 0; nn < 4; ++nn) vr[0][nn] = lds_read_tr8_at(p + 32 * nn);
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        if (ks + 1 < 4) {
          const uint32_t p = vstep(ks + 1);
#pragma unroll
          for (int nn = 0; nn < 4; ++nn) vr[(ks + 1) & 1][nn] = lds_read_tr8_at(p + 32 * nn);
        }
        const v4i pr = *reinterpret_cast<const v4i*>(pbuf + (ks * 64 + lane) * 16);
        const v4i ev = *reinterpret_cast<const v4i*>(et + ((jt * 4 + ks) * 2 + h) * 8);
        v4i pa;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          // (bit_cast of a vector element reads element 0; copy to scalars first)
          const int pe = pr[e], ee = ev[e];
          pa[e] = __builtin_bit_cast(int, __builtin_bit_cast(v2u16, pe) + __builtin_bit_cast(v2u16, ee));
        }
        v8bf vb16[4];
#pragma unroll
        for (int nn = 0; nn < 4; ++nn) vb16[nn] = fp8x8_to_bf16(vr[ks & 1][nn]);
#pragma unroll
        for (int nn = 0; nn < 4; ++nn)
          o[nn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_v8bf(pa), vb16[nn], o[nn], 0, 0, 0);
      }
    }
    // block n+2's rows, into the buffer of block n-1, which every wave left before B3
    if (n + 2 < nblk) issue_block(smem, n + 2, dl, smem + ((n + 2) % kNumBufs) * kBufBytes, wave);
  }

  // drain: nothing may be left in flight when the workgroup ends
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  // total of P per head: both lane halves, then the four key quarters
  l_run += shfl_xor(l_run, 32);
  barrier();
  if (h == 0) mx[o4] = l_run;
  barrier();
  {
    const v4f l4 = *reinterpret_cast<const v4f*>(mx);
    l_run = (l4[0] + l4[1]) + (l4[2] + l4[3]);
  }
  if (h_half >= P.H) return;
  const bool any = l_run > 0.f;
  const float inv = any ? 1.f / l_run : 0.f;
  const float lse = any ? (m_run + __builtin_amdgcn_logf(l_run)) * kLn2 : -__builtin_inff();
  // o[nt][r]: head h_half + 8(r/4) + 4h + r%4, dim 128 jt + 32nt + c32
  if (P.splits == 1) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int hr = 8 * (r >> 2) + 4 * h + (r & 3);
      const float ir = __shfl(inv, hr, 64);
      if (h_half + hr < P.H) {
        uint16_t* orow = P.out + ((int64_t)t * P.H + h_half + hr) * kMlaDv + 128 * jt + c32;
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) orow[32 * nt] = (uint16_t)f32_to_bf16_rne(o[nt][r] * ir);
      }
    }
    if (h == 0 && jt == 0 && head_ok && P.lse) P.lse[(int64_t)t * P.H + head] = lse;
    if (h == 0 && jt == 0 && head_ok && P.max_out)
      P.max_out[(int64_t)t * P.H + head] = any ? m_max * kLn2 : -__builtin_inff();
  } else {
    const int64_t row0 = ((int64_t)split * P.T + t) * P.H + h_half;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int hr = 8 * (r >> 2) + 4 * h + (r & 3);
      const float ir = __shfl(inv, hr, 64);
      if (h_half + hr < P.H) {
        float* orow = P.ws_o + (row0 + hr) * kMlaDv + 128 * jt + c32;
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) orow[32 * nt] = o[nt][r] * ir;
      }
    }
    if (h == 0 && jt == 0 && head_ok) P.ws_lse[row0 + c32] = lse;
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
                          int64_t kv_num_blocks, const int32_t* indices, int64_t idx_stride, int num_tokens,
                          int num_heads, int topk, float sm_scale, void* out, float* lse, int num_splits,
                          void* workspace, size_t workspace_bytes, void* stream) {
  return dsa::sparse_mla_decode_impl(q, q_token_stride, q_head_stride, kv_cache, kv_block_stride_bytes,
                                     kv_block_size, kv_num_blocks, indices, idx_stride, num_tokens, num_heads, topk,
                                     sm_scale, out, lse, num_splits, workspace, workspace_bytes, stream, nullptr, 0);
}

}  // extern "C"

namespace dsa {

int sparse_mla_decode_impl(const void* q, int64_t q_token_stride, int64_t q_head_stride, const uint8_t* kv_cache,
                           int64_t kv_block_stride_bytes, int kv_block_size, int64_t kv_num_blocks,
                           const int32_t* indices, int64_t idx_stride, int num_tokens, int num_heads, int topk,
                           float sm_scale, void* out, float* lse, int num_splits, void* workspace,
                           size_t workspace_bytes, void* stream, float* max_out, int compact) {
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
    smem_status = hipFuncSetAttribute((const void*)sparse_mla_kernel,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMlaSmemBytes) == hipSuccess
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
  P.compact = compact;
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

}  // namespace dsa
