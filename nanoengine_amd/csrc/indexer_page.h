// One 64-token page of the fp8 lightning-indexer cache in registers, and the
// head-weighted ReLU sum of a query token over it (gfx950). Shared by the
// indexer passes and by the list select's in-place repair of a row.
//
// Page layout (bytes): [64 tokens x 128 fp8][64 x f32 scale] = 8448.
#pragma once

#include "dsa_common.h"

namespace dsa {

constexpr int kIdxPageTokens = 64;
constexpr int kIdxHeadDim = 128;
constexpr int kIdxHeads = 64;
constexpr int kIdxPageBytes = kIdxPageTokens * (kIdxHeadDim + 4);

__device__ __forceinline__ v8i load32B(const uint8_t* p) {
  const v4i a = *reinterpret_cast<const v4i*>(p);
  const v4i b = *reinterpret_cast<const v4i*>(p + 16);
  v8i r;
  r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
  r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
  return r;
}

// The same 32 bytes with nontemporal loads (global_load ... nt): key pages
// are read once per pass, and streaming them this way reads random 8448-byte
// pages at 6.6-6.8 TB/s against 5.9-6.0 TB/s for plain loads on MI355X.
__device__ __forceinline__ v8i load32B_stream(const uint8_t* p) {
  const v4i a = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p));
  const v4i b = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p + 16));
  v8i r;
  r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
  r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
  return r;
}

// max(x, 0) in one instruction (v_med3_f32 with bounds 0 and FLT_MAX).
__device__ __forceinline__ float relu(float x) { return __builtin_amdgcn_fmed3f(x, 0.f, 3.402823466e38f); }

struct PageRegs {
  v8i k[4];      // token tiles: lane holds token tt*16 + lane%16, bytes (lane/16)*32 .. +32
  float scale;   // scale of token `lane`
};

__device__ __forceinline__ void load_page(PageRegs& pr, const uint8_t* page, int lane) {
  const uint8_t* base = page + (lane & 15) * kIdxHeadDim + (lane >> 4) * 32;
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) pr.k[tt] = load32B_stream(base + tt * 16 * kIdxHeadDim);
  pr.scale = __builtin_nontemporal_load(reinterpret_cast<const float*>(page + kIdxPageTokens * kIdxHeadDim) + lane);
}

// A page as whole 128-byte rows per load instruction (nontemporal): chunk
// c = 2tt + h of the page (1 KB = rows 8c .. 8c+7) goes to pr.k[tt] dwords
// 4h .. 4h+3, lane l holding row 8c + l/8, bytes 16(l%8) .. +16. A load
// instruction of load_page touches 16 rows (half of each 128-byte line);
// one of these touches 8 whole rows, and the persistent filter pass reads
// its 1.1 GB ~12% faster this way. rows_to_operands turns the rows into
// load_page's operand layout through the wave's LDS tile.
constexpr int kIdxTrRow = 144;                                  // padded row stride of the tile
constexpr int kIdxTrBytes = kIdxPageTokens * kIdxTrRow;         // 9216 B per wave
__device__ __forceinline__ void load_page_rows(PageRegs& pr, const uint8_t* page, int lane) {
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    const v4i a = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(page + tt * 2048 + lane * 16));
    const v4i b = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(page + tt * 2048 + 1024 + lane * 16));
    pr.k[tt][0] = a[0]; pr.k[tt][1] = a[1]; pr.k[tt][2] = a[2]; pr.k[tt][3] = a[3];
    pr.k[tt][4] = b[0]; pr.k[tt][5] = b[1]; pr.k[tt][6] = b[2]; pr.k[tt][7] = b[3];
  }
  pr.scale = __builtin_nontemporal_load(reinterpret_cast<const float*>(page + kIdxPageTokens * kIdxHeadDim) + lane);
}

// The rows of load_page_rows -> the operand layout of load_page, through the
// calling wave's tile tr (kIdxTrBytes, 16-byte aligned, used by this wave
// alone). Rows are kIdxTrRow = 144 bytes apart, so the 16 rows one operand
// read touches fall on distinct LDS banks. A wave's LDS operations complete
// in issue order, and the compiler keeps the reads after the writes to the
// same tile, so no barrier is needed.
__device__ __forceinline__ void rows_to_operands(PageRegs& pr, uint8_t* tr, int lane) {
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const v4i x = {pr.k[tt][4 * h], pr.k[tt][4 * h + 1], pr.k[tt][4 * h + 2], pr.k[tt][4 * h + 3]};
      *reinterpret_cast<v4i*>(tr + (16 * tt + 8 * h + (lane >> 3)) * kIdxTrRow + (lane & 7) * 16) = x;
    }
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    const uint8_t* src = tr + (16 * tt + (lane & 15)) * kIdxTrRow + (lane >> 4) * 32;
    const v4i a = *reinterpret_cast<const v4i*>(src);
    const v4i b = *reinterpret_cast<const v4i*>(src + 16);
    pr.k[tt][0] = a[0]; pr.k[tt][1] = a[1]; pr.k[tt][2] = a[2]; pr.k[tt][3] = a[3];
    pr.k[tt][4] = b[0]; pr.k[tt][5] = b[1]; pr.k[tt][6] = b[2]; pr.k[tt][7] = b[3];
  }
}

// Query token j's heads as MFMA A operands (tile ht row i = head ht*16 + i)
// and this lane's head weights (head ht*16 + (lane/16)*4 + r).
__device__ __forceinline__ void load_query(const uint8_t* q_row, const float* w_row, int lane, v8i (&qa)[4],
                                           float (&w)[4][4]) {
#pragma unroll
  for (int ht = 0; ht < 4; ++ht) {
    qa[ht] = load32B(q_row + (ht * 16 + (lane & 15)) * kIdxHeadDim + (lane >> 4) * 32);
#pragma unroll
    for (int r = 0; r < 4; ++r) w[ht][r] = w_row[ht * 16 + (lane >> 4) * 4 + r];
  }
}

// Head-weighted ReLU sum of query token j over one page, before the token
// scale: lane l returns the value of token l of the page.
template <int NQ>
__device__ __forceinline__ float page_head_sum(const PageRegs& cur, int j, int lane, const v8i (&qa)[NQ][4],
                                               const float (&w)[NQ][4][4]) {
  float part[4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    // four independent products per token tile keep the MFMA pipe busy
    v4f c[4];
#pragma unroll
    for (int ht = 0; ht < 4; ++ht)
      c[ht] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(qa[j][ht], cur.k[tt], (v4f){0.f, 0.f, 0.f, 0.f},
                                                              0, 0, 0, 127, 0, 127);
    // c[ht][r]: head ht*16 + (lane/16)*4 + r, token tt*16 + lane%16
    float acc = 0.f;
#pragma unroll
    for (int ht = 0; ht < 4; ++ht)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc = fmaf(w[j][ht][r], relu(c[ht][r]), acc);
    part[tt] = acc;
  }
  // Butterfly over the four 16-lane groups: lane group g keeps token tile g.
  const bool hi32 = lane & 32;
  const float s0 = hi32 ? part[0] : part[2];
  const float s1 = hi32 ? part[1] : part[3];
  const float k0 = (hi32 ? part[2] : part[0]) + shfl_xor(s0, 32);
  const float k1 = (hi32 ? part[3] : part[1]) + shfl_xor(s1, 32);
  const bool hi16 = lane & 16;
  return (hi16 ? k1 : k0) + shfl_xor(hi16 ? k0 : k1, 16);
}

}  // namespace dsa
