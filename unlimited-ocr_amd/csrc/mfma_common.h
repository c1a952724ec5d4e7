// Shared pieces of the MFMA (matrix-core) gather-attention kernels for gfx950:
// operand types, the per-tile chunk plan (which 64-key chunks a 64-row query
// tile must visit) and per-row key masks.
//
// MFMA shape used throughout: v_mfma_f32_32x32x16_bf16 / _f16.  Per-lane
// layouts (lane l, h = l / 32):
//   A (32 x 16):  A[m = l % 32][k = 8h + j],            j = 0..7
//   B (16 x 32):  B[k = 8h + j][n = l % 32]
//   D (32 x 32):  D[m = 8(r / 4) + 4h + r % 4][n = l % 32], r = 0..15
// The kernels compute transposed products (S^T = K Q^T, O^T = V^T P^T, ...)
// so that every lane owns ONE query row (n = l % 32) and the D registers of a
// first product are directly the B operand of the next one: for the 16-key
// step ks of a 32-key D tile, B slot j holds key 16(ks%2) + 4h + j (j < 4) or
// 16(ks%2) + 8 + 4h + (j - 4) -- a fixed permutation of the reduction index
// that the A operand reproduces with two 8-byte LDS reads.
#pragma once

#include "common.h"

namespace srswa {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kChunk = 64;        // keys per chunk (MFMA key tile)
constexpr int kTileRows = 64;     // query rows per tile (two waves x 32)

template <typename T> struct Mfma;
template <> struct Mfma<bf16_t> {
  __device__ __forceinline__ static f32x16_t mac(const uint4& a, const uint4& b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static uint32_t pack2(float lo, float hi) { return pack_bf16x2(lo, hi); }
  __device__ __forceinline__ static float lo(uint32_t w) { return bf16_lo(w); }
  __device__ __forceinline__ static float hi(uint32_t w) { return bf16_hi(w); }
};
template <> struct Mfma<__half> {
  __device__ __forceinline__ static f32x16_t mac(const uint4& a, const uint4& b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
  __device__ __forceinline__ static uint32_t pack2(float lo, float hi) { return pack_h16x2(lo, hi); }
  __device__ __forceinline__ static float lo(uint32_t w) { return h16_lo(w); }
  __device__ __forceinline__ static float hi(uint32_t w) { return h16_hi(w); }
};

__device__ __forceinline__ f32x16_t zero16() {
  f32x16_t z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// key offset (0..31) inside a 32x32 D tile held by register r of lane half h
__device__ __forceinline__ int d_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

// Per-tile chunk plan built in LDS by all threads of the workgroup:
//   rows: key index qi, segment start seg, window start ls = max(qi-LW+1, seg)
//   ids:  the rows' slot block ids (S per row, -1 = none)
//   chunks: sorted list of 64-key chunks holding any window key or any key of a
//           selected block that can be a remote key of some row.
struct TilePlanSmem {
  int* qi;        // [64]
  int* seg;       // [64]
  int* ls;        // [64]
  int* ids;       // [64 * S]
  float* bias;    // [64 * S] or nullptr
  uint32_t* bits; // [nchunk_words]
  int* chunks;    // [umax]
  int* count;     // [1]
};

}  // namespace srswa
