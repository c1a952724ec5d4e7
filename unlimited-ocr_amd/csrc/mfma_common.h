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

#include <atomic>

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

// fp32 operands: a lane's 8 values (two 16-byte words) feed eight
// v_mfma_f32_32x32x2_f32, value j of lane half h being that product's k index
// h.  Both operands list their 8 values in one key order, so the eight
// products together sum the 16 k of a bf16 / fp16 step, in fp32 throughout.
struct F32x8 {
  uint4 lo, hi;
};
template <> struct Mfma<float> {
  __device__ __forceinline__ static f32x16_t mac(const F32x8& a, const F32x8& b, f32x16_t c) {
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.lo.x), __uint_as_float(b.lo.x), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.lo.y), __uint_as_float(b.lo.y), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.lo.z), __uint_as_float(b.lo.z), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.lo.w), __uint_as_float(b.lo.w), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.hi.x), __uint_as_float(b.hi.x), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.hi.y), __uint_as_float(b.hi.y), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.hi.z), __uint_as_float(b.hi.z), c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.hi.w), __uint_as_float(b.hi.w), c, 0, 0, 0);
  }
};
// a lane's operand fragment of one 16-wide k step: 8 values of T
template <typename T> using Frag = std::conditional_t<std::is_same<T, float>::value, F32x8, uint4>;
__device__ __forceinline__ F32x8 f32x8(const float* v) {
  return F32x8{make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])),
               make_uint4(__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]), __float_as_uint(v[7]))};
}

// The fp32 A operand X^T (M = feature d, K = 16 rows of X) in the key order of
// the MFMA output rows that form the B operand: lane (d = l % 32, h) value j
// is X[r0 + 4h + j][c0 + d] for j < 4 and X[r0 + 8 + 4h + (j - 4)][c0 + d]
// after (the order a_operand_tr gives the 16-bit forms), read as scalars.
template <int PITCH>
__device__ __forceinline__ F32x8 a_operand_f32(const float* x, int r0, int c0, int lane) {
  const int d = lane & 31, h = lane >> 5;
  const float* p = x + (r0 + 4 * h) * PITCH + c0 + d;
  float v[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[e] = p[e * PITCH];
    v[4 + e] = p[(8 + e) * PITCH];
  }
  return f32x8(v);
}

// Raw buffer loads (gfx9 buffer resource, byte offsets): one 32-bit lane
// offset plus a scalar offset per load instead of a 64-bit address per load,
// and a hardware range check -- bytes at or beyond `bytes` read as zero.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

__device__ __forceinline__ f32x16_t zero16() {
  f32x16_t z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// key offset (0..31) inside a 32x32 D tile held by register r of lane half h
__device__ __forceinline__ int d_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

// The same A operand (X^T, M = feature d, K = 16 rows of X in the permuted
// order) from two transposing LDS reads, ds_read_b64_tr_b16.  That instruction
// works on groups of 16 lanes: output lane L, element e is element L % 4 of
// the 8 bytes addressed by source lane 4e + L / 4 of its group.  Source lane
// s of group g (h = l / 32) therefore points at row r0 + 4h + s / 4, column
// c0 + 16(g % 2) + 4(s % 4), and lane (d = l % 32, h) receives
// X[r0 + 4h + e][c0 + d] (first read) and X[r0 + 8 + 4h + e][c0 + d]
// (second read, eight rows further), e = 0..3.
template <int PITCH>
__device__ __forceinline__ uint4 a_operand_tr(const uint16_t* x, int r0, int c0, int lane) {
  const int s = lane & 15, g = (lane >> 4) & 1, h = lane >> 5;
  const uint16_t* p = x + (r0 + 4 * h + (s >> 2)) * PITCH + c0 + 16 * g + 4 * (s & 3);
  const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)p);
  const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(p + 8 * PITCH));
  const uint2 a = __builtin_bit_cast(uint2, lo), b = __builtin_bit_cast(uint2, hi);
  return make_uint4(a.x, a.y, b.x, b.y);
}

// bits [lo, hi) of a 64-bit word, 0 <= lo, hi <= 64
__device__ __forceinline__ uint64_t range64(int lo, int hi) {
  if (hi <= lo) return 0ull;
  const uint64_t top = hi >= 64 ? ~0ull : ((1ull << hi) - 1ull);
  return top & ~((1ull << lo) - 1ull);
}

constexpr int kIdEnd = 0x7fffffff;   // sentinel closing a row's sorted id list

// One row's selected blocks, as the kernels walk them: the valid ids that hold
// at least one remote key of the row (seg <= j < ls, j <= qi), ascending, a
// repeated id kept once with its first slot's bias (and, when sslot is given,
// that slot's index), then kIdEnd padding up to SP = S + 1 entries (so a
// cursor never runs past the list).
//
// Up to 8 slots, from registers (id8 / b8: -1 / 0 past the row's slots): the
// (id, slot) keys are sorted by Batcher's odd-even merge network (19
// compare-exchanges); a repeated id then follows its first slot, which is the
// one kept.
__device__ inline void sort_row_ids8(const int* id8, const float* b8, int SP, int BS, int maxblk, int qi, int seg,
                                     int ls, int* sid, float* sb, int* sslot = nullptr) {
  uint32_t key[8];
  float bk[8];   // each key's bias, carried through the network with it
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const int id = id8[s];
    bool ok = id >= 0 && id <= maxblk;
    const int base = ok ? id * BS : 0;
    ok = ok && max(base, seg) < min(min(base + BS, ls), qi + 1);
    key[s] = ok ? ((uint32_t)id << 3) | (uint32_t)s : 0xffffffffu;
    bk[s] = b8[s];
  }
  auto cas = [&](int i, int j) __attribute__((always_inline)) {
    const bool sw = key[j] < key[i];
    const uint32_t ki = key[i];
    const float bi = bk[i];
    key[i] = sw ? key[j] : ki;
    key[j] = sw ? ki : key[j];
    bk[i] = sw ? bk[j] : bi;
    bk[j] = sw ? bi : bk[j];
  };
  cas(0, 1); cas(2, 3); cas(4, 5); cas(6, 7);
  cas(0, 2); cas(1, 3); cas(4, 6); cas(5, 7);
  cas(1, 2); cas(5, 6);
  cas(0, 4); cas(1, 5); cas(2, 6); cas(3, 7);
  cas(2, 4); cas(3, 5);
  cas(1, 2); cas(3, 4); cas(5, 6);
  int n = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t k = key[i];
    if (k == 0xffffffffu || (i > 0 && (key[i - 1] >> 3) == (k >> 3))) continue;
    sid[n] = (int)(k >> 3);
    if (sb) sb[n] = bk[i];
    if (sslot) sslot[n] = (int)(k & 7u);
    ++n;
  }
  for (int i = n; i < SP; ++i) {
    sid[i] = kIdEnd;
    if (sslot) sslot[i] = -1;
  }
}

// The same from the row's slots in memory (S of them, any number).
__device__ inline void sort_row_ids(const int32_t* ids, const float* bias, int S, int SP, int BS,
                                    int maxblk, int qi, int seg, int ls, int* sid, float* sb,
                                    int* sslot = nullptr) {
  if (S <= 8) {
    // every id (and bias) is loaded at once, so the row pays one memory latency
    int id8[8];
    float b8[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) id8[s] = s < S ? ids[s] : -1;
#pragma unroll
    for (int s = 0; s < 8; ++s) b8[s] = bias && s < S ? bias[s] : 0.f;
    sort_row_ids8(id8, b8, SP, BS, maxblk, qi, seg, ls, sid, sb, sslot);
    return;
  }
  int n = 0;
  for (int s = 0; s < S; ++s) {
    const int id = ids[s];
    if (id < 0 || id > maxblk) continue;
    const int lo = max(id * BS, seg), hi = min(min(id * BS + BS, ls), qi + 1);
    if (lo >= hi) continue;
    bool dup = false;
    for (int k = 0; k < n; ++k) dup |= sid[k] == id;
    if (dup) continue;
    const float bv = bias ? bias[s] : 0.f;
    int i = n;
    while (i > 0 && sid[i - 1] > id) {
      sid[i] = sid[i - 1];
      if (sb) sb[i] = sb[i - 1];
      if (sslot) sslot[i] = sslot[i - 1];
      --i;
    }
    sid[i] = id;
    if (sb) sb[i] = bv;
    if (sslot) sslot[i] = s;
    ++n;
  }
  for (int i = n; i < SP; ++i) {
    sid[i] = kIdEnd;
    if (sslot) sslot[i] = -1;
  }
}

// One row's walk over its sorted selected blocks, chunk by chunk (ascending).
struct RowWalk {
  const int* sid;      // sorted ids (kIdEnd-terminated)
  const float* sb;     // their bias (nullptr: no bias)
  int cur, nid;        // cursor and the id under it
  int ls, seg, hi, rem_hi;   // window [ls, hi), remote candidates [seg, rem_hi)
  bool ok;
};

// The row's keep mask over a chunk's 64 keys (bit k = key j0 + k), its remote
// part, the bias (log2 units) of each 16-key quarter and the sorted index of
// the block covering each quarter (-1: not selected).  Block sizes are powers
// of two >= 16, so a quarter never straddles two blocks.  Returns whether the
// row keeps the whole chunk with one bias for every key.
__device__ __forceinline__ bool chunk_mask(RowWalk& w, int j0, int bs_shift, bool blk64, uint64_t& keep,
                                           uint64_t& rm, float bq[4], int qix[4]) {
  uint32_t qmem = 0;
#pragma unroll
  for (int qq = 0; qq < 4; ++qq) {
    bq[qq] = 0.f;
    qix[qq] = -1;
  }
  if (blk64) {
    const int blk = j0 >> bs_shift;
    while (w.nid < blk) w.nid = w.sid[++w.cur];
    if (w.nid == blk) {
      qmem = 15u;
      const float bv = w.sb ? w.sb[w.cur] * kLog2e : 0.f;
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        bq[qq] = bv;
        qix[qq] = w.cur;
      }
    }
  } else {
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const int blk = (j0 + 16 * qq) >> bs_shift;
      while (w.nid < blk) w.nid = w.sid[++w.cur];
      if (w.nid == blk) {
        qmem |= 1u << qq;
        if (w.sb) bq[qq] = w.sb[w.cur] * kLog2e;
        qix[qq] = w.cur;
      }
    }
  }
  uint64_t qm = 0;
#pragma unroll
  for (int qq = 0; qq < 4; ++qq)
    if (qmem & (1u << qq)) qm |= 0xffffull << (16 * qq);
  const uint64_t wm = range64(min(max(w.ls - j0, 0), 64), min(max(w.hi - j0, 0), 64));
  rm = range64(min(max(w.seg - j0, 0), 64), min(max(w.rem_hi - j0, 0), 64)) & qm;
  keep = wm | rm;
  return !w.ok || (keep == ~0ull && (!w.sb || rm == 0ull || (rm == ~0ull && blk64)));
}

// Ascending list of the set bits of a bitmap (nwords words) by a prefix
// popcount in the first wavefront; every thread of the workgroup calls it
// after the bitmap is complete and gets the count.
__device__ inline int compact_bitmap(const uint32_t* s_bits, int nwords, uint16_t* s_chunks, int* s_count) {
  const int tid = threadIdx.x;
  if (tid < kWave) {
    int base = 0;
    for (int w0 = 0; w0 < nwords; w0 += kWave) {
      const int w = w0 + tid;
      const uint32_t bits = w < nwords ? s_bits[w] : 0u;
      const int cnt = __popc(bits);
      int incl = cnt;
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) {
        const int v = __shfl_up(incl, o, kWave);
        if (tid >= o) incl += v;
      }
      int pos = base + incl - cnt;
      uint32_t bb = bits;
      while (bb) {
        const int bit = __ffs(bb) - 1;
        bb &= bb - 1;
        s_chunks[pos++] = (uint16_t)(w * 32 + bit);
      }
      base += __shfl(incl, kWave - 1, kWave);
    }
    if (tid == 0) *s_count = base;
  }
  lds_barrier();
  return *s_count;
}

// Sorted list of the 64-key chunks a tile visits, from the rows' windows
// [ls, qi] and the remote keys of their sorted ids (sid, SP entries per row):
// a bitmap over chunks (s_bits, nwords words, zeroed here) compacted by a
// prefix popcount into s_chunks.  Every thread of the workgroup calls it;
// returns the chunk count.
__device__ inline int plan_chunks(const int* s_qi, const int* s_seg, const int* s_ls, const int* sid,
                                  int SP, int BS, int LW, int nrows, int nwords, uint32_t* s_bits,
                                  uint16_t* s_chunks, int* s_count) {
  const int tid = threadIdx.x, nthr = blockDim.x;
  for (int w = tid; w < nwords; w += nthr) s_bits[w] = 0u;
  lds_barrier();
  if (tid < kWave) {
    // the first wavefront, lane = row
    const int r = tid;
    const bool live = r < nrows;
    // windows: each row's chunks [ls / 64, qi / 64]; a row's range starts at
    // most one chunk past the previous row's end (ls <= qi = previous qi + 1),
    // so the union over the rows is the single range [min start, max end]
    const int c_lo = wave_min_int(live ? max(s_ls[r], 0) / kChunk : INT_MAX);
    const int c_hi = wave_max_int(live ? s_qi[r] / kChunk : INT_MIN);
    if (c_lo <= c_hi) {
      for (int w = (c_lo >> 5) + r; w <= (c_hi >> 5); w += kWave) {
        const int lo = max(c_lo - 32 * w, 0), hi = min(c_hi - 32 * w, 31);
        s_bits[w] |= (hi - lo == 31) ? 0xffffffffu : (((1u << (hi - lo + 1)) - 1u) << lo);
      }
    }
    // remote keys: the i-th listed block of every row; rows sharing a selection
    // list the same blocks, and then one lane sets the bits for the wave
    for (int i = 0; i < SP; ++i) {
      const int id = live ? sid[r * SP + i] : kIdEnd;
      const bool has = id != kIdEnd;
      const uint64_t m = __ballot(has);
      if (m == 0ull) break;   // every row's list has ended (kIdEnd pads each list)
      int c0 = 0, c1 = -1;
      if (has) {
        const int lo = max(id * BS, s_seg[r]);
        const int hi = min(min(id * BS + BS, s_ls[r]), s_qi[r] + 1);
        c0 = lo / kChunk;
        c1 = (hi - 1) / kChunk;
      }
      const int first = __ffsll((long long)m) - 1;
      const int f0 = __shfl(c0, first, kWave), f1 = __shfl(c1, first, kWave);
      const bool same = __all(!has || (c0 == f0 && c1 == f1));
      if (same) {
        if (r == first)
          for (int c = f0; c <= f1; ++c) atomicOr(&s_bits[c >> 5], 1u << (c & 31));
      } else if (has) {
        for (int c = c0; c <= c1; ++c) atomicOr(&s_bits[c >> 5], 1u << (c & 31));
      }
    }
  }
  lds_barrier();
  return compact_bitmap(s_bits, nwords, s_chunks, s_count);
}

// Raise a kernel's dynamic-LDS limit to `bytes` when it needs more than the
// default; returns false (error recorded) when the runtime refuses.  The grant
// is remembered per device (the attribute is set with that device current) in
// atomics, so calls from several host threads are safe.
constexpr int kMaxDevices = 64;
struct LdsGrant {
  std::atomic<size_t> bytes[kMaxDevices];   // zero-initialised in static storage
};
template <typename F>
inline bool ensure_dynamic_lds(F* kernel, size_t bytes, LdsGrant* g) {
  if (bytes <= 64 * 1024) return true;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    dev = -1;
  }
  const bool cached = dev >= 0 && dev < kMaxDevices;
  if (cached && bytes <= g->bytes[dev].load(std::memory_order_relaxed)) return true;
  const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    set_error("cannot grant %zu bytes of LDS: %s", bytes, hipGetErrorString(e));
    return false;
  }
  if (cached) {
    size_t cur = g->bytes[dev].load(std::memory_order_relaxed);
    while (cur < bytes && !g->bytes[dev].compare_exchange_weak(cur, bytes, std::memory_order_relaxed)) {
    }
  }
  return true;
}

// Compute units of the current device (0 when the runtime cannot say),
// remembered per device.
inline int device_cu_count() {
  static std::atomic<int> cached[kMaxDevices];   // zero-initialised in static storage
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  if (dev >= 0 && dev < kMaxDevices) {
    const int c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  if (dev >= 0 && dev < kMaxDevices) cached[dev].store(n, std::memory_order_relaxed);
  return n;
}

}  // namespace srswa
