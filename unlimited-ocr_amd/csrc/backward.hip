// Gather-attention backward on the matrix cores (gfx950).
//
// Replaces the reference's backward kernels
//   _gather_attn_bwd_dq_kernel  (K2)  HF/sparse_gather_triton.py:125-200
//   _gather_attn_bwd_dkv_kernel (K3)  HF/sparse_gather_triton.py:203-279
//   _e2e_attn_bwd_dq_kernel     (K6)  HF/sparse_gather_e2e_triton.py:124-206
//   _e2e_attn_bwd_dkv_kernel    (K7)  HF/sparse_gather_e2e_triton.py:209-275
// and the torch glue between them (delta = rowsum(O*dO), the dense
// [B, HI, T, M] block_mask scatter, HF/sparse_gather_triton.py:329,339-343).
//
// Kernels, in stream order:
//   1. zero + touch_kernel -- bit (chunk c, query tile tau) set when some row of
//      tau reads a REMOTE key of chunk c.  The bitmap is tile-granular (64x
//      smaller than the reference's per-token dense block mask) and its
//      content does not depend on the order of the atomic ORs.
//   2. dq_kernel  -- per 64-row query tile, the forward's chunk plan.  Its
//      set-up computes each row's delta = sum_d O*dO in fp32 and q*scale
//      rounded to the input dtype, and writes for the dK / dV kernel
//      q*scale [B, HQ, T, D], a 16-byte record per row (lse, delta, sample
//      start) and, per index head, the rows' first slot ids and biases.  Per chunk
//      S^T = K Q^T, dP^T = V dO^T, dS = P (dP - delta), dQ^T += K^T dS^T; the
//      bias gradient (sum of fp32 dS over the remote keys of a selected block)
//      is summed per (row, slot) in LDS and written once per query head --
//      no atomics (the reference uses tl.atomic_add).
//   3. dkv_kernel -- per 64-key chunk and kv head, every query tile whose
//      window covers the chunk or whose touch bit is set, in ascending order:
//      S = Q K^T, dP = dO V^T, dV^T += dO^T P, dK^T += Q^T dS, four waves split
//      by key half and role (S / softmax / dV, dP / dS / dK).  Deterministic
//      (fixed visiting order, no atomics).
// Rounding points follow the reference: q*scale and P / dS are rounded to the
// input dtype before their products; delta, P, dS and all accumulators are fp32.
#include <algorithm>
#include <type_traits>

#include "mfma_common.h"

namespace srswa {
namespace {

struct BwdK {
  srswa_bwd_args a;
  int ntiles, nchunk, nwords, umax, twords, SP, bs_shift;
  int G, IG;
  int nlogical, per_xcd;          // dQ workgroups (sequence, query head, tile), XCD-aware order
  int nlogical_kv;                // dK/dV workgroups (sequence, kv head, chunk)
  int chunks_off, sid_off;        // dQ LDS byte offsets of the chunk list and sorted ids
  int Tp;                         // T rounded up to whole tiles (rows of the row records)
  // row records, written by dQ, read by dK / dV (one buffer resource over all three):
  float4* rows;       // [B, HQ, Tp] {lse in log2 units (+inf past T), delta (0 past T), sample start, 0}
  uint32_t ids_off;   // byte offset from `rows` of the slot records [B, HI, Tp, kPreSlots] int32 (-1 padded)
  uint32_t bias_off;  // ... and of the bias records [B, HI, Tp, kPreSlots] fp32 (0 padded; with a bias)
  uint32_t rec_bytes; // bytes of the three
  uint32_t* touch;    // [B, HI, nchunk, twords]
  void* qs;           // [B, HQ, T, D] q * scale rounded to the input dtype (dK / dV operand)
};

constexpr int kPreSlots = 8;   // slots per row in the slot records (the dK / dV kernel's first look)

// -------------------------------------------------------------- 1. touch map
__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t* w, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) w[i] = 0u;
}

// One wavefront per (sequence, index head, query tile, slot), lane = row of
// the tile.  When every live lane's block maps to the same chunk range (rows
// of a tile sharing a selection), one lane sets the bits for the wave;
// otherwise each lane sets its own.  Either way the bitmap gets the same bits.
__global__ __launch_bounds__(256) void touch_kernel(BwdK p) {
  const srswa_bwd_args& a = p.a;
  const int lane = threadIdx.x % kWave;
  const int64_t w = (int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  const int64_t nw = (int64_t)a.B * a.HI * p.ntiles * a.S;
  if (w >= nw) return;
  const int s = (int)(w % a.S);
  int64_t r = w / a.S;
  const int tau = (int)(r % p.ntiles);
  r /= p.ntiles;
  const int ih = (int)(r % a.HI);
  const int b = (int)(r / a.HI);
  const int t = tau * kTileRows + lane;
  int c0 = 0, c1 = -1;                       // chunk range of this row's slot (empty: c1 < c0)
  if (t < a.T) {
    const int id = a.idx[(int64_t)b * a.idx_sb + (int64_t)ih * a.idx_sh + (int64_t)t * a.idx_st + s];
    const int BS = a.block_size;
    if (id >= 0 && id <= (a.Sk - 1) / BS) {
      const int qi = a.Sk - a.T + t;
      const int seg = a.seg ? a.seg[(int64_t)b * a.seg_sb + t] : 0;
      const int ls = max(qi - a.local_window + 1, seg);
      const int lo = max(id * BS, seg);
      const int hi = min(min(id * BS + BS, ls), qi + 1);
      if (lo < hi) {
        c0 = lo / kChunk;
        c1 = (hi - 1) / kChunk;
      }
    }
  }
  const bool live = c1 >= c0;
  const uint64_t lm = __ballot(live);
  if (lm == 0ull) return;
  const int first = __ffsll((long long)lm) - 1;
  const int f0 = __shfl(c0, first, kWave), f1 = __shfl(c1, first, kWave);
  const bool same = __all(!live || (c0 == f0 && c1 == f1));
  uint32_t* base = p.touch + ((int64_t)b * a.HI + ih) * p.nchunk * p.twords + (tau >> 5);
  if (same) {
    if (lane == first)
      for (int c = f0; c <= f1; ++c) atomicOr(base + (int64_t)c * p.twords, 1u << (tau & 31));
  } else if (live) {
    for (int c = c0; c <= c1; ++c) atomicOr(base + (int64_t)c * p.twords, 1u << (tau & 31));
  }
}

// -------------------------------------------------------------- 2. dQ
// ES: element bytes (2, or 4 for fp32, whose K^T operand is read as scalars:
// a 4-float pad keeps the lane halves' rows, 4 apart, on different banks)
template <int D, int ES = 2> struct DqLds {
  static constexpr int KP = ES == 4 ? D + 4 : D + 16;   // K: row reads (S^T) and K^T reads (dQ)
  static constexpr int VP = ES == 4 ? D + 4 : D + 8;    // V: row reads only
  static constexpr int vOff = kChunk * KP * ES;
  static constexpr int tileBytes = vOff + kChunk * VP * ES;
};

// One workgroup = (sequence, query head, 64-row tile), two waves of 32 rows,
// the forward's chunk plan; per chunk S^T = K Q^T and dP^T = V dO^T (lanes own
// rows, so lse and delta are per-lane registers), dS = P (dP - delta),
// dQ^T += K^T dS^T with the K^T operand read by transposing LDS reads.  The
// bias gradient (sum of fp32 dS over the remote keys of a selected block) is
// summed per (row, sorted block) in LDS in a fixed order and written per slot
// at the end (0 for repeated ids) -- no atomics.
// Two waves per SIMD (four workgroups per CU, LDS permitting).  At D = 128
// that fits the register file only without a staging prefetch: a chunk's K / V
// are loaded at the top of its own iteration, and the co-resident workgroups'
// waves cover the load latency (a one-chunk register prefetch needs 324
// registers, one wave per SIMD, and is slower).  At D = 64 the prefetch fits.
// The fp32 form (8 MFMAs per k step, twice the operand registers) runs one
// wave per SIMD at D = 128, with the accumulators in the second register file.
template <typename T, int D>
__global__ __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(std::is_same<T, float>::value && D == 128 ? 1 : 2)))
void dq_kernel(BwdK p) {
  constexpr bool F32 = std::is_same<T, float>::value;
  constexpr uint32_t ES = sizeof(T);
  using M = Mfma<T>;
  using L = DqLds<D, (int)sizeof(T)>;
  constexpr int KP = L::KP, VP = L::VP;
  constexpr int KS = D / 16, MT = D / 32, NT = 128;
  constexpr int PPT = kChunk * D / 8 / NT;
  constexpr int RPP = NT / (D / 8);
  extern __shared__ __align__(16) unsigned char smem[];
  const srswa_bwd_args& a = p.a;

  const int lid = (int)(blockIdx.x & 7) * p.per_xcd + (int)(blockIdx.x >> 3);
  if (lid >= p.nlogical) return;

  T* sK = reinterpret_cast<T*>(smem);
  T* sV = reinterpret_cast<T*>(smem + L::vOff);
  int* s_qi = reinterpret_cast<int*>(smem);          // set-up only (aliases the tiles)
  int* s_seg = s_qi + 64;
  int* s_ls = s_seg + 64;
  int* s_count = s_ls + 64;
  uint32_t* s_bits = reinterpret_cast<uint32_t*>(s_count + 4);
  uint16_t* s_chunks = reinterpret_cast<uint16_t*>(smem + p.chunks_off);
  int* s_sid = reinterpret_cast<int*>(smem + p.sid_off);
  float* s_sb = a.bias ? reinterpret_cast<float*>(s_sid + 64 * p.SP) : nullptr;
  int* s_sslot = a.dbias ? reinterpret_cast<int*>(s_sid + 64 * p.SP * (a.bias ? 2 : 1)) : nullptr;
  float* s_sdb = a.dbias ? reinterpret_cast<float*>(s_sslot + 64 * p.SP) : nullptr;

  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int h = lane >> 5, rl = lane & 31;
  const int tile = lid % p.ntiles;
  const int bh = lid / p.ntiles;
  const int hq = bh % a.HQ, b = bh / a.HQ;
  const int kvh = hq / p.G, ih = hq / p.IG;
  const int t0 = tile * kTileRows;
  const int nrows = min(kTileRows, a.T - t0);
  const int off = a.Sk - a.T;
  const int BS = a.block_size, LW = a.local_window, SP = p.SP;
  const int maxblk = (a.Sk - 1) >> p.bs_shift;
  const bool blk64 = BS >= kChunk;

  // Loads first, in the order their values are needed, and nothing computed
  // from a loaded value until all are issued (a use waits for its own load
  // and for every load issued before it): the set-up row's sample start and
  // first slots (tid < 64, row r = tid), then this lane's lse, q, dO and O
  // rows, which stay in flight across the sort and the chunk plan.  Rows past
  // T read row t0 (valid memory); their values are masked where used.
  const int row = wave * 32 + rl;
  const bool row_ok = row < nrows;
  const int trow = t0 + (row_ok ? row : 0);
  const int r = tid, rr = min(r, nrows - 1);
  const int smax = max(a.S - 1, 0);
  const int32_t* ids = a.S > 0 ? a.idx + (int64_t)b * a.idx_sb + (int64_t)ih * a.idx_sh + (int64_t)(t0 + rr) * a.idx_st
                               : reinterpret_cast<const int32_t*>(a.lse);   // a valid stand-in, never used
  const float* bias = a.bias ? a.bias + (int64_t)b * a.bias_sb + (int64_t)ih * a.bias_sh + (int64_t)(t0 + rr) * a.bias_st
                             : reinterpret_cast<const float*>(ids);
  const int* segp = a.seg ? a.seg + (int64_t)b * a.seg_sb + t0 + rr : ids;
  int seg_ld = 0, id8[kPreSlots];
  float b8[kPreSlots];
  if (tid < 64) {
    seg_ld = *segp;
#pragma unroll
    for (int s = 0; s < kPreSlots; ++s) {
      id8[s] = ids[min(s, smax)];
      b8[s] = bias[min(s, smax)];
    }
  }
  const float lse_ld = a.lse[(int64_t)b * a.lse_sb + (int64_t)trow * a.lse_st + (int64_t)hq * a.lse_sh];
  // lanes l and l ^ 32 hold the two halves of a row's head dims
  Frag<T> qf[KS], gf[KS], of[KS];
  {
    const T* qrow = reinterpret_cast<const T*>(a.q) + (int64_t)b * a.q_sb + (int64_t)trow * a.q_st + (int64_t)hq * a.q_sh;
    const T* grow = reinterpret_cast<const T*>(a.dout) + (int64_t)b * a.do_sb + (int64_t)trow * a.do_st + (int64_t)hq * a.do_sh;
    const T* orow = reinterpret_cast<const T*>(a.o) + (int64_t)b * a.o_sb + (int64_t)trow * a.o_st + (int64_t)hq * a.o_sh;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qf[ks] = *reinterpret_cast<const Frag<T>*>(qrow + 16 * ks + 8 * h);
      gf[ks] = *reinterpret_cast<const Frag<T>*>(grow + 16 * ks + 8 * h);
      of[ks] = *reinterpret_cast<const Frag<T>*>(orow + 16 * ks + 8 * h);
    }
  }
  if (tid < 64) {
    int qi = -1, seg = 0, ls = 0;
    if (r < nrows) {
      qi = off + t0 + r;
      seg = a.seg ? seg_ld : 0;
      ls = max(qi - LW + 1, seg);
    }
    s_qi[r] = qi;
    s_seg[r] = seg;
    s_ls[r] = ls;
    // the row's first slots, -1 / 0 past S and past T
#pragma unroll
    for (int s = 0; s < kPreSlots; ++s) {
      const bool in = r < nrows && s < a.S;
      id8[s] = in ? id8[s] : -1;
      b8[s] = in && a.bias ? b8[s] : 0.f;
    }
    if (a.S <= kPreSlots)
      sort_row_ids8(id8, b8, SP, BS, maxblk, qi, seg, ls, s_sid + r * SP, s_sb ? s_sb + r * SP : nullptr,
                    s_sslot ? s_sslot + r * SP : nullptr);
    else
      sort_row_ids(ids, a.bias ? bias : nullptr, r < nrows ? a.S : 0, SP, BS, maxblk, qi, seg, ls, s_sid + r * SP,
                   s_sb ? s_sb + r * SP : nullptr, s_sslot ? s_sslot + r * SP : nullptr);
    if (hq % p.IG == 0) {
      // the slot records of this index head's rows, for the dK / dV kernel
      // (one query head of the index head writes them)
      const int64_t rec = ((int64_t)b * a.HI + ih) * p.Tp + t0 + r;
      int4* ir = reinterpret_cast<int4*>(reinterpret_cast<char*>(p.rows) + p.ids_off) + rec * 2;
      ir[0] = make_int4(id8[0], id8[1], id8[2], id8[3]);
      ir[1] = make_int4(id8[4], id8[5], id8[6], id8[7]);
      if (a.bias) {
        float4* br = reinterpret_cast<float4*>(reinterpret_cast<char*>(p.rows) + p.bias_off) + rec * 2;
        br[0] = make_float4(b8[0], b8[1], b8[2], b8[3]);
        br[1] = make_float4(b8[4], b8[5], b8[6], b8[7]);
      }
    }
    if (s_sdb)
      for (int i = 0; i < SP; ++i) s_sdb[r * SP + i] = 0.f;
  }
  lds_barrier();   // the row loads above stay in flight across the plan
  const int U = plan_chunks(s_qi, s_seg, s_ls, s_sid, SP, BS, LW, nrows, p.nwords, s_bits, s_chunks, s_count);
  const float lse_l2 = row_ok ? lse_ld * kLog2e : INFINITY;   // log2 units; +inf past T, so every P is 0

  RowWalk w;
  w.ok = row_ok;
  w.ls = s_ls[row];
  w.seg = s_seg[row];
  w.hi = s_qi[row] + 1;
  w.rem_hi = min(w.ls, w.hi);
  w.sid = s_sid + row * SP;
  w.sb = s_sb ? s_sb + row * SP : nullptr;
  w.cur = 0;
  w.nid = w.sid[0];
  // wave-uniform bounds of the rows' windows: [w_ls_max, w_hi_min) lies in every one
  const int w_ls_max = wave_max_int(w.ok ? w.ls : INT_MIN);
  const int w_hi_min = wave_min_int(w.ok ? w.hi : INT_MAX);
  // delta = rowsum(O * dO) in fp32, published for the dK / dV kernel, and
  // q * scale rounded to the input dtype (the reference's rounding point of
  // the scaled query), kept here and written as [B, HQ, T, D] rows, which the
  // dK / dV kernel stages as they are
  float dpart = 0.f;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const uint32_t* o4 = reinterpret_cast<const uint32_t*>(&of[ks]);
    const uint32_t* g4 = reinterpret_cast<const uint32_t*>(&gf[ks]);
    if constexpr (F32) {
#pragma unroll
      for (int e = 0; e < 8; ++e) dpart += __uint_as_float(o4[e]) * __uint_as_float(g4[e]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) dpart += M::lo(o4[e]) * M::lo(g4[e]) + M::hi(o4[e]) * M::hi(g4[e]);
    }
  }
  const float drow = xor32_sum(dpart);   // every lane of the pair is active
  const float dlt = row_ok ? drow : 0.f;
  T* qsrow = reinterpret_cast<T*>(p.qs) + (((int64_t)b * a.HQ + hq) * a.T + trow) * D;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    uint32_t* xx = reinterpret_cast<uint32_t*>(&qf[ks]);
    if constexpr (F32) {
#pragma unroll
      for (int e = 0; e < 8; ++e) xx[e] = __float_as_uint(__uint_as_float(xx[e]) * a.scale);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) xx[e] = M::pack2(M::lo(xx[e]) * a.scale, M::hi(xx[e]) * a.scale);
    }
    if (row_ok) *reinterpret_cast<Frag<T>*>(qsrow + 16 * ks + 8 * h) = qf[ks];
  }
  // this row's record for the dK / dV kernel (rows past T too: +inf, 0, 0)
  if (h == 0) p.rows[((int64_t)b * a.HQ + hq) * p.Tp + t0 + row] = make_float4(lse_l2, dlt, __int_as_float(w.seg), 0.f);

  f32x16_t dq[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) dq[mt] = zero16();

  const __amdgpu_buffer_rsrc_t krs = make_rsrc(
      reinterpret_cast<const T*>(a.k) + (int64_t)b * a.k_sb + (int64_t)kvh * a.k_sh,
      (uint32_t)(((int64_t)(a.Sk - 1) * a.k_st + D) * ES));
  const __amdgpu_buffer_rsrc_t vrs = make_rsrc(
      reinterpret_cast<const T*>(a.v) + (int64_t)b * a.v_sb + (int64_t)kvh * a.v_sh,
      (uint32_t)(((int64_t)(a.Sk - 1) * a.v_st + D) * ES));
  const uint32_t kvo = (uint32_t)((tid / (D / 8)) * a.k_st + (tid % (D / 8)) * 8) * ES;
  const uint32_t vvo = (uint32_t)((tid / (D / 8)) * a.v_st + (tid % (D / 8)) * 8) * ES;
  T* sKw = sK + (tid / (D / 8)) * KP + (tid % (D / 8)) * 8;
  T* sVw = sV + (tid / (D / 8)) * VP + (tid % (D / 8)) * 8;
  Frag<T> kpre[PPT], vpre[PPT];
  auto fetch = [&](int c) {
    const uint32_t kso = (uint32_t)c * kChunk * (uint32_t)a.k_st * ES;
    const uint32_t vso = (uint32_t)c * kChunk * (uint32_t)a.v_st * ES;
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      if constexpr (F32) {     // both offsets in the lane part: the range check reads keys past Sk as zero
        const uint32_t ko = kvo + kso + (uint32_t)(i * RPP) * (uint32_t)a.k_st * ES;
        const uint32_t vo = vvo + vso + (uint32_t)(i * RPP) * (uint32_t)a.v_st * ES;
        kpre[i] = Frag<T>{buffer_load16(krs, ko, 0), buffer_load16(krs, ko + 16, 0)};
        vpre[i] = Frag<T>{buffer_load16(vrs, vo, 0), buffer_load16(vrs, vo + 16, 0)};
      } else {
        kpre[i] = buffer_load16(krs, kvo, kso + (uint32_t)(i * RPP) * (uint32_t)a.k_st * 2u);
        vpre[i] = buffer_load16(vrs, vvo, vso + (uint32_t)(i * RPP) * (uint32_t)a.v_st * 2u);
      }
    }
  };
  const uint16_t* k16 = reinterpret_cast<const uint16_t*>(sK);

  constexpr bool kPrefetch = D < 128 && !F32;   // fp32 at D = 64: the prefetch would spill
  if (kPrefetch && U > 0) fetch(s_chunks[0]);
  for (int u = 0; u < U; ++u) {
    const int j0 = (int)s_chunks[u] * kChunk;
    if (!kPrefetch) fetch(s_chunks[u]);   // in flight across the barrier
    __syncthreads();   // previous chunk fully consumed
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      *reinterpret_cast<Frag<T>*>(sKw + i * RPP * KP) = kpre[i];
      *reinterpret_cast<Frag<T>*>(sVw + i * RPP * VP) = vpre[i];
    }
    __syncthreads();
    if (kPrefetch && u + 1 < U) fetch(s_chunks[u + 1]);

    // a chunk inside every row's window needs no mask (and no walk of the ids)
    uint64_t keep = ~0ull, rm = 0ull;
    float bq[4] = {0.f, 0.f, 0.f, 0.f};
    int qix[4] = {-1, -1, -1, -1};
    bool fast = true;
    if (!(j0 >= w_ls_max && j0 + kChunk <= w_hi_min))
      fast = __all(chunk_mask(w, j0, p.bs_shift, blk64, keep, rm, bq, qix));
    const float addb = (fast && w.sb && rm != 0ull) ? bq[0] : 0.f;
    float dsum[4] = {0.f, 0.f, 0.f, 0.f};
    Frag<T> db[4];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      f32x16_t st = zero16(), dp = zero16();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        st = M::mac(*reinterpret_cast<const Frag<T>*>(sK + (32 * half + rl) * KP + 16 * ks + 8 * h), qf[ks], st);
        dp = M::mac(*reinterpret_cast<const Frag<T>*>(sV + (32 * half + rl) * VP + 16 * ks + 8 * h), gf[ks], dp);
      }
      if (fast) {
        const float sub = addb - lse_l2;
        float ds0 = 0.f;      // summed only for the bias gradient
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float pv = __builtin_amdgcn_exp2f(fmaf(st[r], kLog2e, sub));
          const float dsv = pv * (dp[r] - dlt);
          st[r] = dsv;
          ds0 += dsv;
        }
        if (s_sdb && rm != 0ull) dsum[0] += ds0;
      } else {
        const uint32_t k32 = (uint32_t)((keep >> (4 * h)) >> (32 * half));
        const uint32_t r32 = (uint32_t)((rm >> (4 * h)) >> (32 * half));
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int bit = 8 * (r >> 2) + (r & 3);
          const int qq = 2 * half + (r >> 3);
          const bool remb = (r32 >> bit) & 1u;
          const float x = fmaf(st[r], kLog2e, (remb ? bq[qq] : 0.f) - lse_l2);
          const float pv = ((k32 >> bit) & 1u) ? __builtin_amdgcn_exp2f(x) : 0.f;
          const float dsv = pv * (dp[r] - dlt);
          st[r] = dsv;
          if (remb) dsum[qq] += dsv;
        }
      }
      if constexpr (F32) {
        float v[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] = st[r];
        db[2 * half] = f32x8(v);
        db[2 * half + 1] = f32x8(v + 8);
      } else {
        db[2 * half] = make_uint4(M::pack2(st[0], st[1]), M::pack2(st[2], st[3]), M::pack2(st[4], st[5]),
                                  M::pack2(st[6], st[7]));
        db[2 * half + 1] = make_uint4(M::pack2(st[8], st[9]), M::pack2(st[10], st[11]), M::pack2(st[12], st[13]),
                                      M::pack2(st[14], st[15]));
      }
    }
    // dQ^T += K^T dS^T (k-step outer: MT interleaved accumulator chains)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      Frag<T> ka[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if constexpr (F32)
          ka[mt] = a_operand_f32<KP>(reinterpret_cast<const float*>(sK), 16 * ks, 32 * mt, lane);
        else
          ka[mt] = a_operand_tr<KP>(k16, 16 * ks, 32 * mt, lane);
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) dq[mt] = M::mac(ka[mt], db[ks], dq[mt]);
    }

    if (s_sdb) {
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const float tot = xor32_sum(dsum[qq]);
        if (h == 0 && w.ok && qix[qq] >= 0) s_sdb[row * SP + qix[qq]] += tot;
      }
    }
  }

  if (w.ok) {
    T* qrow = reinterpret_cast<T*>(a.dq) + (int64_t)b * a.dq_sb + (int64_t)(t0 + row) * a.dq_st + (int64_t)hq * a.dq_sh;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = 32 * mt + 8 * g + 4 * h;
        if constexpr (F32) {
          *reinterpret_cast<float4*>(qrow + d0) = make_float4(dq[mt][4 * g] * a.scale, dq[mt][4 * g + 1] * a.scale,
                                                              dq[mt][4 * g + 2] * a.scale, dq[mt][4 * g + 3] * a.scale);
        } else {
          uint2 x;
          x.x = M::pack2(dq[mt][4 * g] * a.scale, dq[mt][4 * g + 1] * a.scale);
          x.y = M::pack2(dq[mt][4 * g + 2] * a.scale, dq[mt][4 * g + 3] * a.scale);
          *reinterpret_cast<uint2*>(qrow + d0) = x;
        }
      }
  }
  if (s_sdb) {
    __syncthreads();
    for (int e = tid; e < nrows * a.S; e += NT) {
      const int r = e / a.S, s = e % a.S;
      float v = 0.f;
      for (int i = 0; i < SP; ++i)
        if (s_sslot[r * SP + i] == s) v = s_sdb[r * SP + i];
      a.dbias[(int64_t)b * a.db_sb + (int64_t)hq * a.db_sh + (int64_t)(t0 + r) * a.db_st + s] = v;
    }
  }
}

// -------------------------------------------------------------- 3. dK / dV

// bits [lo, hi) of a 32-bit word, the bounds clamped to [0, 32]
__device__ __forceinline__ uint32_t span32(int lo, int hi) {
  lo = min(max(lo, 0), 32);
  hi = min(max(hi, 0), 32);
  const uint32_t above = lo >= 32 ? 0u : (~0u << lo);
  const uint32_t below = hi >= 32 ? ~0u : ~(~0u << hi);
  return above & below;
}

// One workgroup = (sequence, kv head, 64-key chunk), four waves.  For every
// query head of the group, the query tiles whose windows cover the chunk or
// whose touch bit is set are visited in ascending order (deterministic: fixed
// order, no atomics).  The work of each 32-key half is split by role, so a
// wave holds one operand set and one accumulator set (two waves per SIMD):
//   role A (waves 0, 1): K of its keys; S = Q K^T, the masks, bias and
//     softmax -> P (fp32, published through LDS), dV^T += dO^T P;
//   role B (waves 2, 3): V of its keys; dP = dO V^T, then dS = P (dP - delta)
//     from the published P, dK^T += (q*scale)^T dS.
// Per visit: stage Q / dO | S (A) and dP (B) | the softmax (A) while the
// role-B waves (which wait for P anyway) derive the NEXT visit's row data
// (keep masks and biases of their key half, lse, delta) into the other of two
// buffers | barrier | dV (A), dS and dK (B).  A lane
// holds the same (row, key) elements in both roles (the same MFMA shape), so
// role B reads role A's P lane for lane.
template <int D, int ES = 2> struct DkvLds {
  // Q / dO tiles: row reads and transposed (fp32: scalar) reads
  static constexpr int QP = ES == 4 ? D + 4 : D + 16;
  static constexpr int gOff = kTileRows * QP * ES;  // dO tile
  static constexpr int pOff = 2 * gOff;             // P: [key half][8 x float4][64 lanes]
  static constexpr int rowOff = pOff + 2 * 8 * 64 * 16;
  // one row-data buffer: lse[64], delta[64], keep[2][64], remote[2][64] (32-bit
  // masks per key half), bias[4][64] per 16-key quarter, flag[4]
  static constexpr int rowBytes = (64 + 64 + 128 + 128 + 256) * 4 + 16;
  static constexpr int fixedBytes = rowOff + 2 * rowBytes;
};

template <typename T, int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(std::is_same<T, float>::value && D == 128 ? 1 : 2)))
void dkv_kernel(BwdK p) {
  constexpr bool F32 = std::is_same<T, float>::value;   // fp32: one wave per SIMD at D = 128
  constexpr uint32_t ES = sizeof(T);
  using M = Mfma<T>;
  using L = DkvLds<D, (int)sizeof(T)>;
  constexpr int QP = L::QP;
  constexpr int KS = D / 16, MT = D / 32, NT = 256;
  constexpr int PPT = kTileRows * D / 8 / NT;
  constexpr int RPP = NT / (D / 8);
  extern __shared__ __align__(16) unsigned char smem[];
  const srswa_bwd_args& a = p.a;

  // chunk-ascending dispatch (every (sequence, kv head) of chunk 0 first, ...,
  // consecutive workgroups on different XCDs): the early chunks, which every
  // later tile can select, have the longest visit lists and start first, so
  // the last workgroups to start are short ones
  const int g = (int)blockIdx.x, BK = p.nlogical_kv / p.nchunk;
  if (g >= p.nlogical_kv) return;
  const int lid = (g % BK) * p.nchunk + g / BK;

  T* sQ = reinterpret_cast<T*>(smem);
  T* sG = reinterpret_cast<T*>(smem + L::gOff);
  float4* sP = reinterpret_cast<float4*>(smem + L::pOff);
  int* s_tiles = reinterpret_cast<int*>(smem + L::fixedBytes);    // visit list
  // row-data buffer `buf`
  auto s_lse = [&](int buf) { return reinterpret_cast<float*>(smem + L::rowOff + buf * L::rowBytes); };
  auto s_dlt = [&](int buf) { return s_lse(buf) + 64; };
  auto s_keep = [&](int buf) { return reinterpret_cast<uint32_t*>(s_lse(buf) + 128); };   // [2][64]
  auto s_rem = [&](int buf) { return s_keep(buf) + 128; };                                 // [2][64]
  auto s_bq = [&](int buf) { return reinterpret_cast<float*>(s_keep(buf) + 256); };        // [4][64]
  auto s_flag = [&](int buf) { return reinterpret_cast<int*>(s_bq(buf) + 256); };

  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int kh = wave & 1, role = wave >> 1;     // key half, 0 = S / P / dV, 1 = dP / dS / dK
  const int h = lane >> 5, rl = lane & 31;
  const int c = lid % p.nchunk;
  const int bk = lid / p.nchunk;
  const int kvh = bk % a.HKV, b = bk / a.HKV;
  const int j0 = c * kChunk;
  const int kk = 32 * kh + rl;                 // this lane's key within the chunk
  const int jmine = j0 + kk;
  const bool key_ok = jmine < a.Sk;
  const int off = a.Sk - a.T;
  const int LW = a.local_window, S = a.S;
  const int myq = kk >> 4;                     // this key's 16-key quarter
  // role B: this key half's first key and the blocks of its two 16-key
  // quarters (a quarter past the keys has no remote bits, whatever matches it)
  const int hj0 = j0 + 32 * kh;
  const int qa = hj0 >> p.bs_shift, qb = (hj0 + 16) >> p.bs_shift;

  // role A: K of this lane's key; role B: V
  Frag<T> kv[KS];
  {
    const T* base = role == 0 ? reinterpret_cast<const T*>(a.k) + (int64_t)b * a.k_sb + (int64_t)kvh * a.k_sh
                              : reinterpret_cast<const T*>(a.v) + (int64_t)b * a.v_sb + (int64_t)kvh * a.v_sh;
    const int64_t st = role == 0 ? a.k_st : a.v_st;
    const T* row = base + (int64_t)(key_ok ? jmine : 0) * st;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      kv[ks] = key_ok ? *reinterpret_cast<const Frag<T>*>(row + 16 * ks + 8 * h) : Frag<T>{};
  }
  f32x16_t acc[MT];                            // role A: dV^T, role B: dK^T
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = zero16();

  // query tiles whose windows can reach this chunk: qi in [j0, j0 + 63 + LW - 1]
  const int wlo_t = j0 - off, whi_t = j0 + kChunk - 1 + LW - 1 - off;
  const int tau_a = max(wlo_t, 0) / kTileRows;
  const int tau_b = whi_t < 0 ? -1 : min(whi_t / kTileRows, p.ntiles - 1);

  T* sQw = sQ + (tid / (D / 8)) * QP + (tid % (D / 8)) * 8;
  T* sGw = sG + (tid / (D / 8)) * QP + (tid % (D / 8)) * 8;
  const uint16_t* q16 = reinterpret_cast<const uint16_t*>(sQ);
  const uint16_t* g16 = reinterpret_cast<const uint16_t*>(sG);
  const T* sX = role == 0 ? sQ : sG;           // the row operand of S (A) / dP (B)
  const uint16_t* x16 = role == 0 ? g16 : q16; // the transposed operand of dV (A) / dK (B)
  const float* x32 = reinterpret_cast<const float*>(role == 0 ? sG : sQ);   // the same, fp32
  float4* sPl = sP + kh * 8 * 64 + lane;       // this lane's P records
  __shared__ int s_ntiles;
  Frag<T> qpre[PPT], gpre[PPT];
  const __amdgpu_buffer_rsrc_t rrs = make_rsrc(p.rows, p.rec_bytes);   // row and slot records

  for (int gq = 0; gq < p.G; ++gq) {
    const int hq = kvh * p.G + gq;
    const int ih = hq / p.IG;
    const uint32_t* tb = p.touch + (((int64_t)b * a.HI + ih) * p.nchunk + c) * p.twords;
    __syncthreads();
    if (wave == 0) {
      // the visit list: window tiles | touched tiles, ascending; lane = 32-tile
      // word (all words loaded at once), positions from a prefix sum of counts
      int n = 0;
      for (int w0 = 0; w0 < p.twords; w0 += kWave) {
        const int wd = w0 + lane;
        uint32_t bits = 0u;
        if (wd < p.twords) {
          bits = tb[wd];
          const int lo = max(tau_a - 32 * wd, 0), hi = min(tau_b - 32 * wd, 31);
          if (lo <= hi) bits |= (hi - lo == 31) ? 0xffffffffu : (((1u << (hi - lo + 1)) - 1u) << lo);
          const int nvalid = p.ntiles - 32 * wd;
          if (nvalid < 32) bits &= (1u << nvalid) - 1u;
        }
        const int cnt = __popc(bits);
        int incl = cnt;
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) {
          const int y = __shfl_up(incl, o, kWave);
          if (lane >= o) incl += y;
        }
        int pos = n + incl - cnt;
        while (bits) {
          s_tiles[pos++] = 32 * wd + __ffs(bits) - 1;
          bits &= bits - 1;
        }
        n += __shfl(incl, kWave - 1, kWave);
      }
      if (lane == 0) s_ntiles = n;
    }
    __syncthreads();
    const int nt = s_ntiles;
    // the scaled query written by the dQ kernel ([T, D] rows of this head), dO as given
    const __amdgpu_buffer_rsrc_t qrs = make_rsrc(
        reinterpret_cast<const T*>(p.qs) + ((int64_t)b * a.HQ + hq) * a.T * D, (uint32_t)((int64_t)a.T * D * ES));
    const __amdgpu_buffer_rsrc_t grs = make_rsrc(
        reinterpret_cast<const T*>(a.dout) + (int64_t)b * a.do_sb + (int64_t)hq * a.do_sh,
        (uint32_t)(((int64_t)(a.T - 1) * a.do_st + D) * ES));
    const uint32_t qvo = (uint32_t)((tid / (D / 8)) * D + (tid % (D / 8)) * 8) * ES;
    const uint32_t gvo = (uint32_t)((tid / (D / 8)) * a.do_st + (tid % (D / 8)) * 8) * ES;
    auto fetch = [&](int tau) {
      const uint32_t qso = (uint32_t)tau * kTileRows * (uint32_t)D * ES;
      const uint32_t gso = (uint32_t)tau * kTileRows * (uint32_t)a.do_st * ES;
#pragma unroll
      for (int i = 0; i < PPT; ++i) {
        if constexpr (F32) {   // both offsets in the lane part: rows past T read as zero
          const uint32_t qo = qvo + qso + (uint32_t)(i * RPP) * (uint32_t)D * ES;
          const uint32_t go = gvo + gso + (uint32_t)(i * RPP) * (uint32_t)a.do_st * ES;
          qpre[i] = Frag<T>{buffer_load16(qrs, qo, 0), buffer_load16(qrs, qo + 16, 0)};
          gpre[i] = Frag<T>{buffer_load16(grs, go, 0), buffer_load16(grs, go + 16, 0)};
        } else {
          qpre[i] = buffer_load16(qrs, qvo, qso + (uint32_t)(i * RPP) * (uint32_t)D * 2u);
          gpre[i] = buffer_load16(grs, gvo, gso + (uint32_t)(i * RPP) * (uint32_t)a.do_st * 2u);
        }
      }
    };
    // row data of a tile for the role-B waves (lane = row): its row record
    // (lse, delta, sample start) and slot record (the first kPreSlots ids and
    // biases), five 16-byte buffer loads with scalar tile offsets.  Nothing is
    // computed from a loaded value here: that would wait for the load at once,
    // and with it for the Q / dO prefetch issued just before.  Without a bias
    // the bias loads read the slot record again (row_masks then ignores them).
    const uint32_t row_so = (uint32_t)(((int64_t)b * a.HQ + hq) * p.Tp) * 16u;
    const uint32_t ids_so = p.ids_off + (uint32_t)(((int64_t)b * a.HI + ih) * p.Tp) * 32u;
    const uint32_t bias_so = (a.bias ? p.bias_off - p.ids_off : 0u) + ids_so;
    uint4 pf_rec, pf_i0, pf_i1, pf_b0, pf_b1;
    auto rfetch = [&](int tau) {
      const uint32_t t16 = (uint32_t)tau * kTileRows * 16u, t32 = 2u * t16;
      pf_rec = buffer_load16(rrs, lane * 16u, row_so + t16);
      pf_i0 = buffer_load16(rrs, lane * 32u, ids_so + t32);
      pf_i1 = buffer_load16(rrs, lane * 32u + 16u, ids_so + t32);
      pf_b0 = buffer_load16(rrs, lane * 32u, bias_so + t32);
      pf_b1 = buffer_load16(rrs, lane * 32u + 16u, bias_so + t32);
    };
    // the role-B wave of key half kh: row data of visit v for the half's 32
    // keys into buffer v & 1 -- keep / remote bits, the biases of its two
    // 16-key quarters, the lse (kh 0) or delta (kh 1), whether every row keeps
    // the half whole -- then the loads of visit v + 1's row data.  Both role-B
    // waves wait for P in this phase anyway.
    auto row_masks = [&](int v) {
      const int buf = v & 1;
      const int t0 = s_tiles[v] * kTileRows;
      const int nrows = min(kTileRows, a.T - t0);
      const int r = lane;
      uint32_t keep = 0u, rm = 0u;
      float b0 = 0.f, b1 = 0.f;
      if (r < nrows) {
        const int qi = off + t0 + r;
        const int seg = (int)pf_rec.z;
        const int ls = max(qi - LW + 1, seg);
        const int pf_id[kPreSlots] = {(int)pf_i0.x, (int)pf_i0.y, (int)pf_i0.z, (int)pf_i0.w,
                                      (int)pf_i1.x, (int)pf_i1.y, (int)pf_i1.z, (int)pf_i1.w};
        const uint32_t pf_b[kPreSlots] = {pf_b0.x, pf_b0.y, pf_b0.z, pf_b0.w, pf_b1.x, pf_b1.y, pf_b1.z, pf_b1.w};
        // the first slot holding each quarter's block (the scan runs down, so
        // the lowest matching slot's bias stays)
        bool m0 = false, m1 = false;
#pragma unroll
        for (int s = kPreSlots - 1; s >= 0; --s) {
          const bool h0 = pf_id[s] == qa, h1 = pf_id[s] == qb;
          b0 = h0 ? __uint_as_float(pf_b[s]) : b0;
          b1 = h1 ? __uint_as_float(pf_b[s]) : b1;
          m0 = m0 || h0;
          m1 = m1 || h1;
        }
        b0 *= kLog2e;
        b1 *= kLog2e;
        if (S > kPreSlots && !(m0 && m1)) {
          // the remaining slots (read here; each value is used, and waited
          // for, inside this branch, so the common path keeps its short wait)
          const int32_t* ids = a.idx + (int64_t)b * a.idx_sb + (int64_t)ih * a.idx_sh + (int64_t)(t0 + r) * a.idx_st;
          const float* bias = a.bias ? a.bias + (int64_t)b * a.bias_sb + (int64_t)ih * a.bias_sh + (int64_t)(t0 + r) * a.bias_st : nullptr;
          for (int s = kPreSlots; s < S && !(m0 && m1); ++s) {
            const int id = ids[s];
            if (!m0 && id == qa) {
              m0 = true;
              b0 = bias ? bias[s] * kLog2e : 0.f;
            }
            if (!m1 && id == qb) {
              m1 = true;
              b1 = bias ? bias[s] * kLog2e : 0.f;
            }
          }
          __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): nothing of this branch left in flight
        }
        b0 = (m0 && a.bias) ? b0 : 0.f;
        b1 = (m1 && a.bias) ? b1 : 0.f;
        const uint32_t qm = (m0 ? 0x0000ffffu : 0u) | (m1 ? 0xffff0000u : 0u);
        rm = span32(seg - hj0, min(ls, qi + 1) - hj0) & qm;
        keep = span32(ls - hj0, qi + 1 - hj0) | rm;
      }
      s_keep(buf)[64 * kh + r] = keep;
      s_rem(buf)[64 * kh + r] = rm;
      s_bq(buf)[(2 * kh) * 64 + r] = b0;
      s_bq(buf)[(2 * kh + 1) * 64 + r] = b1;
      if (kh == 0)
        s_lse(buf)[r] = __uint_as_float(pf_rec.x);   // log2 units, +inf past T
      else
        s_dlt(buf)[r] = __uint_as_float(pf_rec.y);
      const bool whole = r >= nrows || (keep == ~0u && (!a.bias || rm == 0u));
      const bool all = __all(whole);
      if (r == 0) s_flag(buf)[kh] = all ? 1 : 0;
      if (v + 1 < nt) rfetch(s_tiles[v + 1]);
    };
    if (nt > 0) {
      fetch(s_tiles[0]);
      if (role == 1) {
        rfetch(s_tiles[0]);
        row_masks(0);
      }
    }
    for (int it = 0; it < nt; ++it) {
      const int buf = it & 1;
      __syncthreads();   // previous tile consumed (Q, dO, P); this visit's row data written
#pragma unroll
      for (int i = 0; i < PPT; ++i) {
        *reinterpret_cast<Frag<T>*>(sQw + i * RPP * QP) = qpre[i];
        *reinterpret_cast<Frag<T>*>(sGw + i * RPP * QP) = gpre[i];
      }
      // issued on every visit (the last one fetches its own tile again, unused):
      // with a fetch on some paths only, the row-data reads of phase 2 would
      // wait for every load in flight, this prefetch included
      fetch(s_tiles[min(it + 1, nt - 1)]);
      __syncthreads();

      // S = Q K^T (A) or dP = dO V^T (B): 64 rows x this lane's key; register r
      // of half `half` is row 32 half + 8 (r / 4) + 4h + r % 4
      f32x16_t sg[2] = {zero16(), zero16()};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
        for (int half = 0; half < 2; ++half)
          sg[half] = M::mac(*reinterpret_cast<const Frag<T>*>(sX + (32 * half + rl) * QP + 16 * ks + 8 * h), kv[ks], sg[half]);
      }
      if (role == 0) {
        const bool fast = s_flag(buf)[kh] != 0;   // every row keeps this key half whole
        const float* lse = s_lse(buf);
        // keep / remote bits of this lane's key for the 32 rows it holds in the
        // MFMA layout (bit 16 half + 4 r4 + e <-> row 32 half + 8 r4 + 4 h + e),
        // from the rows' 32-bit masks of this key half, four rows per read
        uint32_t km32 = ~0u, rm32 = 0u;
        if (!fast) {
          km32 = 0u;
          const uint32_t* kw = s_keep(buf) + 64 * kh;
          const uint32_t* rw = s_rem(buf) + 64 * kh;
#pragma unroll
          for (int half = 0; half < 2; ++half)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
              const int row0 = 32 * half + 8 * r4 + 4 * h;
              const int b0 = 16 * half + 4 * r4;
              const uint4 k4 = *reinterpret_cast<const uint4*>(kw + row0);
              km32 |= (((k4.x >> rl) & 1u) | (((k4.y >> rl) & 1u) << 1) | (((k4.z >> rl) & 1u) << 2) |
                       (((k4.w >> rl) & 1u) << 3)) << b0;
              if (a.bias) {
                const uint4 r4v = *reinterpret_cast<const uint4*>(rw + row0);
                rm32 |= (((r4v.x >> rl) & 1u) | (((r4v.y >> rl) & 1u) << 1) | (((r4v.z >> rl) & 1u) << 2) |
                         (((r4v.w >> rl) & 1u) << 3)) << b0;
              }
            }
        }
        // sg <- P in place; two straight-line copies (every row keeps the
        // chunk whole / masked): a uniform test per element would split the
        // unrolled loop into one basic block per exp
        auto softmax = [&](auto fast_tag) {
          constexpr bool FAST = decltype(fast_tag)::value;
#pragma unroll
          for (int half = 0; half < 2; ++half)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
              const int row0 = 32 * half + 8 * r4 + 4 * h;
              const float4 l4 = *reinterpret_cast<const float4*>(lse + row0);
              float4 b4 = make_float4(0.f, 0.f, 0.f, 0.f);
              if constexpr (!FAST)
                if (a.bias) b4 = *reinterpret_cast<const float4*>(s_bq(buf) + myq * 64 + row0);
              const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
              const float bv[4] = {b4.x, b4.y, b4.z, b4.w};
              float pv[4];
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const int r = 4 * r4 + e;
                float x;
                if constexpr (FAST) {
                  x = fmaf(sg[half][r], kLog2e, -lv[e]);
                } else {
                  const int bit = 16 * half + 4 * r4 + e;
                  const bool remb = (rm32 >> bit) & 1u;
                  x = fmaf(sg[half][r], kLog2e, (remb ? bv[e] : 0.f) - lv[e]);
                  x = ((km32 >> bit) & 1u) ? x : -INFINITY;      // exp2(-inf) = 0
                }
                // a key past Sk needs no test: no row keeps it (windows and
                // remote ranges end at qi + 1 <= Sk), so it is -inf above and
                // never in a half every row keeps whole (the fast form); and
                // its P only reaches its own dK / dV, which are not written
                pv[e] = __builtin_amdgcn_exp2f(x);
                sg[half][r] = pv[e];
              }
              sPl[(4 * half + r4) * 64] = make_float4(pv[0], pv[1], pv[2], pv[3]);
            }
        };
        if (fast)
          softmax(std::true_type{});
        else
          softmax(std::false_type{});
      }
      // the next visit's row data (the other buffer), on the role-B waves while
      // role A runs the softmax that role B waits for
      if (role == 1 && it + 1 < nt) row_masks(it + 1);
      __syncthreads();   // P published; the next visit's row data written
      if (role == 1) {
        // sg <- dS = P (dP - delta) in place
        const float* dlt = s_dlt(buf);
#pragma unroll
        for (int half = 0; half < 2; ++half)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
            const int row0 = 32 * half + 8 * r4 + 4 * h;
            const float4 d4 = *reinterpret_cast<const float4*>(dlt + row0);
            const float4 p4 = sPl[(4 * half + r4) * 64];
            const float dv4[4] = {d4.x, d4.y, d4.z, d4.w}, pv[4] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) sg[half][4 * r4 + e] = pv[e] * (sg[half][4 * r4 + e] - dv4[e]);
          }
      }
      Frag<T> pk[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int hf = ks >> 1, r0 = 8 * (ks & 1);
        if constexpr (F32) {
          float v[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] = sg[hf][r0 + j];
          pk[ks] = f32x8(v);
        } else {
          pk[ks] = make_uint4(M::pack2(sg[hf][r0], sg[hf][r0 + 1]), M::pack2(sg[hf][r0 + 2], sg[hf][r0 + 3]),
                              M::pack2(sg[hf][r0 + 4], sg[hf][r0 + 5]), M::pack2(sg[hf][r0 + 6], sg[hf][r0 + 7]));
        }
      }
      // A: dV^T += dO^T P; B: dK^T += (q*scale)^T dS (k-step outer, a step's
      // operands read before its MFMAs)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        Frag<T> xa[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          if constexpr (F32)
            xa[mt] = a_operand_f32<QP>(x32, 16 * ks, 32 * mt, lane);
          else
            xa[mt] = a_operand_tr<QP>(x16, 16 * ks, 32 * mt, lane);
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt] = M::mac(xa[mt], pk[ks], acc[mt]);
      }
    }
  }

  if (!key_ok) return;
  T* out = role == 0
               ? reinterpret_cast<T*>(a.dv) + (int64_t)b * a.dv_sb + (int64_t)jmine * a.dv_st + (int64_t)kvh * a.dv_sh
               : reinterpret_cast<T*>(a.dk) + (int64_t)b * a.dk_sb + (int64_t)jmine * a.dk_st + (int64_t)kvh * a.dk_sh;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * mt + 8 * g + 4 * h;
      if constexpr (F32) {
        *reinterpret_cast<float4*>(out + d0) =
            make_float4(acc[mt][4 * g], acc[mt][4 * g + 1], acc[mt][4 * g + 2], acc[mt][4 * g + 3]);
      } else {
        uint2 w;
        w.x = M::pack2(acc[mt][4 * g], acc[mt][4 * g + 1]);
        w.y = M::pack2(acc[mt][4 * g + 2], acc[mt][4 * g + 3]);
        *reinterpret_cast<uint2*>(out + d0) = w;
      }
    }
}

// -------------------------------------------------------------- host side
bool al16b(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int check_bwd(const srswa_bwd_args* a) {
  if (!a || !a->q || !a->k || !a->v || !a->o || !a->lse || !a->dout || !a->dq || !a->dk || !a->dv ||
      (!a->idx && a->S > 0)) {
    set_error("bwd: null argument");
    return SRSWA_INVALID;
  }
  if (a->B < 0 || a->T < 0 || a->Sk < a->T || a->HQ <= 0 || a->HKV <= 0 || a->HI <= 0 || a->S < 0 ||
      a->block_size <= 0 || a->local_window <= 0) {
    set_error("bwd: bad sizes (need Sk >= T)");
    return SRSWA_INVALID;
  }
  if (a->HQ % a->HKV || a->HQ % a->HI) {
    set_error("bwd: HQ must be a multiple of HKV and HI");
    return SRSWA_UNSUPPORTED;
  }
  if (a->dtype != SRSWA_BF16 && a->dtype != SRSWA_F16 && a->dtype != SRSWA_F32) {
    set_error("bwd: dtype %d not supported (bf16, fp16, fp32)", a->dtype);
    return SRSWA_UNSUPPORTED;
  }
  const int es = a->dtype == SRSWA_F32 ? 4 : 2;   // element bytes
  if (!(a->D == 64 || a->D == 128) || a->block_size < 16 || (a->block_size & (a->block_size - 1)) || a->S > 64) {
    set_error("bwd: D in {64,128}, block size a power of two >= 16, <= 64 slots");
    return SRSWA_UNSUPPORTED;
  }
  if (a->dbias && !a->bias) {
    set_error("bwd: a bias gradient needs the bias");
    return SRSWA_INVALID;
  }
  if (ceil_div(a->Sk, kChunk) > 65536) {
    set_error("bwd: key length above 4M");
    return SRSWA_UNSUPPORTED;
  }
  const int64_t span = ((int64_t)ceil_div(a->Sk, kChunk) * kChunk * std::max(a->k_st, a->v_st) + a->D) * es;
  const int64_t qspan = ((int64_t)ceil_div(a->T, kTileRows) * kTileRows * std::max(a->q_st, a->do_st) + a->D) * es;
  if (span >= ((int64_t)1 << 32) || qspan >= ((int64_t)1 << 32)) {
    set_error("bwd: one sequence's tensors span 4 GiB or more");
    return SRSWA_UNSUPPORTED;
  }
  const int64_t st[] = {a->q_sb, a->q_st, a->q_sh, a->k_sb, a->k_st, a->k_sh, a->v_sb, a->v_st, a->v_sh,
                        a->o_sb, a->o_st, a->o_sh, a->do_sb, a->do_st, a->do_sh, a->dq_sb, a->dq_st,
                        a->dq_sh, a->dk_sb, a->dk_st, a->dk_sh, a->dv_sb, a->dv_st, a->dv_sh};
  for (int64_t s : st)
    if ((s * es) % 16) {
      set_error("bwd: rows must be 16-byte aligned");
      return SRSWA_UNSUPPORTED;
    }
  const void* ptrs[] = {a->q, a->k, a->v, a->o, a->dout, a->dq, a->dk, a->dv};
  for (const void* q : ptrs)
    if (!al16b(q)) {
      set_error("bwd: pointers must be 16-byte aligned");
      return SRSWA_UNSUPPORTED;
    }
  return SRSWA_OK;
}

void plan_bwd(const srswa_bwd_args* a, BwdK& k) {
  k.a = *a;
  k.ntiles = ceil_div(a->T, kTileRows);
  k.nchunk = ceil_div(a->Sk, kChunk);
  k.nwords = ceil_div(k.nchunk, 32);
  k.Tp = k.ntiles * kTileRows;
  const int64_t per_tile = (int64_t)kTileRows * a->S * (ceil_div(a->block_size, kChunk) + 1) +
                           ceil_div(a->local_window + kTileRows - 1, kChunk) + 1;
  k.umax = (int)std::min<int64_t>((int64_t)k.nchunk, per_tile);
  k.twords = ceil_div(k.ntiles, 32);
  k.SP = a->S + 1;
  k.bs_shift = __builtin_ctz((unsigned)std::max(a->block_size, 1));
  k.G = a->HQ / a->HKV;
  k.IG = a->HQ / a->HI;
  k.nlogical = (int)std::min<int64_t>((int64_t)a->B * a->HQ * k.ntiles, INT32_MAX);
  k.per_xcd = ceil_div(k.nlogical, 8);
  k.nlogical_kv = (int)std::min<int64_t>((int64_t)a->B * a->HKV * k.nchunk, INT32_MAX);
  // dQ LDS: K / V tiles (the set-up arrays alias them), chunk list, sorted ids
  // (+ bias, + slot map and bias-gradient sums)
  const bool f32 = a->dtype == SRSWA_F32;
  const size_t tile = a->D == 128 ? (f32 ? DqLds<128, 4>::tileBytes : DqLds<128>::tileBytes)
                                  : (f32 ? DqLds<64, 4>::tileBytes : DqLds<64>::tileBytes);
  const size_t setup = (3 * 64 + 4) * 4 + (size_t)k.nwords * 4;
  size_t n = std::max(tile, setup);
  k.chunks_off = (int)n;
  n += ((size_t)k.umax * 2 + 15) / 16 * 16;
  k.sid_off = (int)n;
}

// the row records [B, HQ, Tp] x 16 B, then the slot and bias records [B, HI, Tp] x 32 B each
size_t rec_bytes(const BwdK& k) {
  const size_t rows = (size_t)k.a.B * k.a.HQ * k.Tp * 16, slots = (size_t)k.a.B * k.a.HI * k.Tp * 32;
  return (rows + 2 * slots + 255) / 256 * 256;
}
size_t touch_words(const BwdK& k) { return (size_t)k.a.B * k.a.HI * k.nchunk * k.twords; }
size_t qs_bytes(const BwdK& k) {
  const size_t es = k.a.dtype == SRSWA_F32 ? 4 : 2;
  return ((size_t)k.a.B * k.a.HQ * k.a.T * k.a.D * es + 255) / 256 * 256;
}

size_t dq_smem(const BwdK& k) {
  const size_t n = (size_t)k.sid_off + (size_t)64 * k.SP * 4 * (1 + (k.a.bias ? 1 : 0) + (k.a.dbias ? 2 : 0));
  return (n + 15) / 16 * 16;
}

size_t dkv_smem(const BwdK& k) {
  const bool f32 = k.a.dtype == SRSWA_F32;
  const size_t fixed = k.a.D == 128 ? (f32 ? DkvLds<128, 4>::fixedBytes : DkvLds<128>::fixedBytes)
                                    : (f32 ? DkvLds<64, 4>::fixedBytes : DkvLds<64>::fixedBytes);  // + visit list
  return (fixed + (size_t)k.ntiles * 4 + 15) / 16 * 16;
}

template <typename T, int D>
int launch_bwd(const BwdK& k, hipStream_t st) {
  static LdsGrant granted_dq, granted_dkv;
  if (!ensure_dynamic_lds(&dq_kernel<T, D>, dq_smem(k), &granted_dq) ||
      !ensure_dynamic_lds(&dkv_kernel<T, D>, dkv_smem(k), &granted_dkv))
    return SRSWA_UNSUPPORTED;
  const srswa_bwd_args& a = k.a;
  const int64_t nw = (int64_t)touch_words(k);
  if (nw > 0) hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)((nw + 255) / 256)), dim3(256), 0, st, k.touch, nw);
  const int64_t ne = (int64_t)a.B * a.HI * k.ntiles * a.S;     // one wavefront each
  if (ne > 0) hipLaunchKernelGGL(touch_kernel, dim3((unsigned)((ne + 3) / 4)), dim3(256), 0, st, k);
  hipLaunchKernelGGL((dq_kernel<T, D>), dim3((unsigned)(8 * k.per_xcd)), dim3(128), dq_smem(k), st, k);
  hipLaunchKernelGGL((dkv_kernel<T, D>), dim3((unsigned)k.nlogical_kv), dim3(256), dkv_smem(k), st, k);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("bwd launch failed: %s", hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}

}  // namespace
}  // namespace srswa

using namespace srswa;

extern "C" size_t srswa_gather_bwd_workspace(const srswa_bwd_args* a) {
  if (!a || a->B <= 0 || a->T <= 0 || a->HQ <= 0 || a->HI <= 0 || a->Sk <= 0) return 0;
  BwdK k{};
  plan_bwd(a, k);
  return rec_bytes(k) + qs_bytes(k) + touch_words(k) * 4;
}

extern "C" int srswa_gather_bwd(const srswa_bwd_args* a, void* scratch, size_t scratch_bytes,
                                void* stream) {
  int st = check_bwd(a);
  if (st != SRSWA_OK) return st;
  if (a->B == 0 || a->T == 0) return SRSWA_OK;
  BwdK k{};
  plan_bwd(a, k);
  const size_t need = rec_bytes(k) + qs_bytes(k) + touch_words(k) * 4;
  if (!scratch || scratch_bytes < need) {
    set_error("bwd: scratch of %zu bytes required (got %zu)", need, scratch_bytes);
    return SRSWA_WORKSPACE;
  }
  if (dq_smem(k) > 156 * 1024 || dkv_smem(k) > 156 * 1024) {
    set_error("bwd: LDS budget exceeded (key length too large)");
    return SRSWA_UNSUPPORTED;
  }
  if (rec_bytes(k) >= ((size_t)1 << 31)) {
    set_error("bwd: row records of 2 GiB or more");
    return SRSWA_UNSUPPORTED;
  }
  k.rows = reinterpret_cast<float4*>(scratch);
  k.ids_off = (uint32_t)((size_t)k.a.B * k.a.HQ * k.Tp * 16);
  k.bias_off = k.ids_off + (uint32_t)((size_t)k.a.B * k.a.HI * k.Tp * 32);
  k.rec_bytes = (uint32_t)rec_bytes(k);
  k.qs = reinterpret_cast<char*>(scratch) + rec_bytes(k);
  k.touch = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(scratch) + rec_bytes(k) + qs_bytes(k));
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (a->dtype == SRSWA_F32)
    return a->D == 128 ? launch_bwd<float, 128>(k, s) : launch_bwd<float, 64>(k, s);
  if (a->dtype == SRSWA_BF16)
    return a->D == 128 ? launch_bwd<bf16_t, 128>(k, s) : launch_bwd<bf16_t, 64>(k, s);
  return a->D == 128 ? launch_bwd<__half, 128>(k, s) : launch_bwd<__half, 64>(k, s);
}
