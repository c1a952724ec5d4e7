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
//   1. delta_kernel  -- delta[b,t,hq] = sum_d O*dO in fp32.
//   2. zero + touch_kernel -- bit (chunk c, query tile tau) set when some row of
//      tau reads a REMOTE key of chunk c.  The bitmap is tile-granular (64x
//      smaller than the reference's per-token dense block mask) and its
//      content does not depend on the order of the atomic ORs.
//   3. dq_kernel  -- per 64-row query tile, the forward's chunk plan; per chunk
//      S^T = K Q^T, dP^T = V dO^T, dS = P (dP - delta), dQ^T += K^T dS^T; the
//      bias gradient (sum of fp32 dS over the remote keys of a selected block)
//      is summed per (row, slot) in LDS and written once per query head --
//      no atomics (the reference uses tl.atomic_add).
//   4. dkv_kernel -- per 64-key chunk and kv head, every query tile whose
//      window covers the chunk or whose touch bit is set, in ascending order:
//      S = Q K^T, dP = dO V^T, dV^T += dO^T P, dK^T += Q^T dS.  Deterministic
//      (fixed visiting order, no atomics).
// Rounding points follow the reference: q*scale and P / dS are rounded to the
// input dtype before their products; delta, P, dS and all accumulators are fp32.
#include <algorithm>

#include "mfma_common.h"

namespace srswa {
namespace {

struct BwdK {
  srswa_bwd_args a;
  int ntiles, nchunk, nwords, umax, twords;
  int G, IG;
  float* delta;       // [B, T, HQ]
  uint32_t* touch;    // [B, HI, nchunk, twords]
};

// -------------------------------------------------------------- 1. delta
template <typename T, int D>
__global__ __launch_bounds__(256) void delta_kernel(BwdK p) {
  constexpr int LPR = D / 8;                 // lanes per row (16-byte pieces)
  constexpr int RPW = kWave / LPR;           // rows per wave
  const srswa_bwd_args& a = p.a;
  using M = Mfma<T>;
  const int lane = threadIdx.x % kWave;
  const int64_t row = ((int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave) * RPW + lane / LPR;
  const int64_t rows = (int64_t)a.B * a.T * a.HQ;
  const int c = lane % LPR;
  float s = 0.f;
  if (row < rows) {
    const int hq = (int)(row % a.HQ);
    const int64_t bt = row / a.HQ;
    const int t = (int)(bt % a.T);
    const int b = (int)(bt / a.T);
    const uint4 ow = *reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(a.o) + (int64_t)b * a.o_sb +
                                                     (int64_t)t * a.o_st + (int64_t)hq * a.o_sh + c * 8);
    const uint4 gw = *reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(a.dout) + (int64_t)b * a.do_sb +
                                                     (int64_t)t * a.do_st + (int64_t)hq * a.do_sh + c * 8);
    const uint32_t* o4 = reinterpret_cast<const uint32_t*>(&ow);
    const uint32_t* g4 = reinterpret_cast<const uint32_t*>(&gw);
#pragma unroll
    for (int e = 0; e < 4; ++e) s += M::lo(o4[e]) * M::lo(g4[e]) + M::hi(o4[e]) * M::hi(g4[e]);
  }
#pragma unroll
  for (int o = LPR / 2; o >= 1; o >>= 1) s += __shfl_xor(s, o, kWave);
  if (row < rows && c == 0) p.delta[row] = s;
}

// -------------------------------------------------------------- 2. touch map
__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t* w, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) w[i] = 0u;
}

__global__ __launch_bounds__(256) void touch_kernel(BwdK p) {
  const srswa_bwd_args& a = p.a;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t n = (int64_t)a.B * a.HI * a.T * a.S;
  if (e >= n) return;
  const int s = (int)(e % a.S);
  int64_t r = e / a.S;
  const int t = (int)(r % a.T);
  r /= a.T;
  const int ih = (int)(r % a.HI);
  const int b = (int)(r / a.HI);
  const int id = a.idx[(int64_t)b * a.idx_sb + (int64_t)ih * a.idx_sh + (int64_t)t * a.idx_st + s];
  const int BS = a.block_size;
  if (id < 0 || id > (a.Sk - 1) / BS) return;
  const int qi = a.Sk - a.T + t;
  const int seg = a.seg ? a.seg[(int64_t)b * a.seg_sb + t] : 0;
  const int ls = max(qi - a.local_window + 1, seg);
  const int lo = max(id * BS, seg);
  const int hi = min(min(id * BS + BS, ls), qi + 1);
  if (lo >= hi) return;
  const int tau = t / kTileRows;
  uint32_t* base = p.touch + ((int64_t)b * a.HI + ih) * p.nchunk * p.twords;
  for (int c = lo / kChunk; c <= (hi - 1) / kChunk; ++c)
    atomicOr(base + (int64_t)c * p.twords + (tau >> 5), 1u << (tau & 31));
}

// -------------------------------------------------------------- 3. dQ
constexpr int kSlotCap = 32;   // planned chunks per tile covered by the slot table

template <typename T, int D>
__global__ __launch_bounds__(128) void dq_kernel(BwdK p) {
  using M = Mfma<T>;
  constexpr int KP = D + 8;
  constexpr int KS = D / 16;
  constexpr int MT = D / 32;
  constexpr int NT = 128;
  extern __shared__ __align__(16) unsigned char smem[];
  const srswa_bwd_args& a = p.a;
  T* sK = reinterpret_cast<T*>(smem);
  T* sV = sK + kChunk * KP;
  int8_t* s_tab = reinterpret_cast<int8_t*>(sV + kChunk * KP);
  int* s_qi = reinterpret_cast<int*>(s_tab + kSlotCap * 64 * 8);
  int* s_seg = s_qi + 64;
  int* s_ls = s_seg + 64;
  int* s_ids = s_ls + 64;
  float* s_bias = reinterpret_cast<float*>(s_ids + 64 * a.S);
  float* s_dbias = s_bias + 64 * a.S;
  uint32_t* s_bits = reinterpret_cast<uint32_t*>(s_dbias + 64 * a.S);
  int* s_chunks = reinterpret_cast<int*>(s_bits + p.nwords);
  int* s_count = s_chunks + p.umax;

  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int h = lane / 32, rl = lane % 32;
  const int tile = blockIdx.x % p.ntiles;
  const int64_t bh = blockIdx.x / p.ntiles;
  const int hq = (int)(bh % a.HQ);
  const int b = (int)(bh / a.HQ);
  const int kvh = hq / p.G, ih = hq / p.IG;
  const int t0 = tile * kTileRows;
  const int nrows = min(kTileRows, a.T - t0);
  const int off = a.Sk - a.T;
  const int BS = a.block_size, LW = a.local_window, S = a.S;

  for (int r = tid; r < 64; r += NT) {
    int qi = -1, seg = 0, ls = 0;
    if (r < nrows) {
      qi = off + t0 + r;
      seg = a.seg ? a.seg[(int64_t)b * a.seg_sb + t0 + r] : 0;
      ls = max(qi - LW + 1, seg);
    }
    s_qi[r] = qi;
    s_seg[r] = seg;
    s_ls[r] = ls;
  }
  for (int e = tid; e < 64 * S; e += NT) {
    const int r = e / S, s = e % S;
    int id = -1;
    float bv = 0.f;
    if (r < nrows) {
      id = a.idx[(int64_t)b * a.idx_sb + (int64_t)ih * a.idx_sh + (int64_t)(t0 + r) * a.idx_st + s];
      if (a.bias) bv = a.bias[(int64_t)b * a.bias_sb + (int64_t)ih * a.bias_sh + (int64_t)(t0 + r) * a.bias_st + s];
    }
    s_ids[e] = id;
    s_bias[e] = bv;
    s_dbias[e] = 0.f;
  }
  for (int w = tid; w < p.nwords; w += NT) s_bits[w] = 0u;
  __syncthreads();
  const int U = build_chunk_plan(s_qi, s_seg, s_ls, s_ids, S, BS, nrows, p.nchunk, p.nwords,
                                 s_bits, s_chunks, s_count, LW, a.Sk);
  build_slot_table(s_qi, s_seg, s_ls, s_ids, s_chunks, U, kSlotCap, S, BS, a.Sk, nrows, s_tab);

  const int row = wave * 32 + rl;
  const bool row_ok = row < nrows;
  const int my_qi = s_qi[row], my_seg = s_seg[row], my_ls = s_ls[row];
  const uint32_t wlen = (uint32_t)max(my_qi - my_ls + 1, 0);
  const uint32_t rlen = (uint32_t)max(min(my_ls, my_qi + 1) - my_seg, 0);
  const int trow = t0 + (row_ok ? row : 0);
  uint4 qf[KS], gf[KS];
  {
    const T* qrow = reinterpret_cast<const T*>(a.q) + (int64_t)b * a.q_sb + (int64_t)trow * a.q_st + (int64_t)hq * a.q_sh;
    const T* grow = reinterpret_cast<const T*>(a.dout) + (int64_t)b * a.do_sb + (int64_t)trow * a.do_st + (int64_t)hq * a.do_sh;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      uint4 w = row_ok ? *reinterpret_cast<const uint4*>(qrow + 16 * ks + 8 * h) : make_uint4(0, 0, 0, 0);
      uint32_t* ww = reinterpret_cast<uint32_t*>(&w);
#pragma unroll
      for (int e = 0; e < 4; ++e) ww[e] = M::pack2(M::lo(ww[e]) * a.scale, M::hi(ww[e]) * a.scale);
      qf[ks] = w;
      gf[ks] = row_ok ? *reinterpret_cast<const uint4*>(grow + 16 * ks + 8 * h) : make_uint4(0, 0, 0, 0);
    }
  }
  const float lse_l2 = row_ok ? a.lse[(int64_t)b * a.lse_sb + (int64_t)trow * a.lse_st + (int64_t)hq * a.lse_sh] * kLog2e
                              : INFINITY;
  const float dlt = row_ok ? p.delta[((int64_t)b * a.T + trow) * a.HQ + hq] : 0.f;

  f32x16_t dq[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) dq[mt] = zero16();

  const T* kg = reinterpret_cast<const T*>(a.k) + (int64_t)b * a.k_sb + (int64_t)kvh * a.k_sh;
  const T* vg = reinterpret_cast<const T*>(a.v) + (int64_t)b * a.v_sb + (int64_t)kvh * a.v_sh;
  constexpr int PPT = kChunk * D / 8 / NT;
  uint4 kpre[PPT], vpre[PPT];
  auto fetch = [&](int c) {
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int pc = tid + i * NT;
      const int j = c * kChunk + pc / (D / 8), col = pc % (D / 8);
      const bool in = j < a.Sk;
      kpre[i] = in ? *reinterpret_cast<const uint4*>(kg + (int64_t)j * a.k_st + col * 8) : make_uint4(0, 0, 0, 0);
      vpre[i] = in ? *reinterpret_cast<const uint4*>(vg + (int64_t)j * a.v_st + col * 8) : make_uint4(0, 0, 0, 0);
    }
  };
  const bool one_blk = (BS % kChunk) == 0;
  const bool sub_blk = (kChunk % BS) == 0;
  const int bs_shift = __ffs(BS) - 1;

  if (U > 0) fetch(s_chunks[0]);
  for (int u = 0; u < U; ++u) {
    const int c = s_chunks[u];
    const int j0 = c * kChunk;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int pc = tid + i * NT;
      const int key = pc / (D / 8), col = pc % (D / 8);
      *reinterpret_cast<uint4*>(sK + key * KP + col * 8) = kpre[i];
      *reinterpret_cast<uint4*>(sV + key * KP + col * 8) = vpre[i];
    }
    __syncthreads();
    if (u + 1 < U) fetch(s_chunks[u + 1]);

    f32x16_t st[2] = {zero16(), zero16()}, dp[2] = {zero16(), zero16()};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      st[0] = M::mac(*reinterpret_cast<const uint4*>(sK + rl * KP + 16 * ks + 8 * h), qf[ks], st[0]);
      st[1] = M::mac(*reinterpret_cast<const uint4*>(sK + (32 + rl) * KP + 16 * ks + 8 * h), qf[ks], st[1]);
      dp[0] = M::mac(*reinterpret_cast<const uint4*>(sV + rl * KP + 16 * ks + 8 * h), gf[ks], dp[0]);
      dp[1] = M::mac(*reinterpret_cast<const uint4*>(sV + (32 + rl) * KP + 16 * ks + 8 * h), gf[ks], dp[1]);
    }

    const int blo = j0 / BS;
    bool memb[5];
    float mbias[5];
    int mslot[5];
    if (u < kSlotCap) {
      const uint2 tw = *reinterpret_cast<const uint2*>(s_tab + (u * 64 + row) * 8);
      const int8_t* t8 = reinterpret_cast<const int8_t*>(&tw);
#pragma unroll
      for (int q = 0; q < 5; ++q) {
        mslot[q] = t8[q];
        memb[q] = t8[q] >= 0;
        mbias[q] = memb[q] ? s_bias[row * S + t8[q]] : 0.f;
      }
    } else {
      const int nq = min(j0 + kChunk - 1, a.Sk - 1) / BS - blo + 1;
#pragma unroll
      for (int q = 0; q < 5; ++q) {
        memb[q] = false;
        mbias[q] = 0.f;
        mslot[q] = -1;
        if (q < nq && row_ok) {
          for (int s = 0; s < S; ++s)
            if (s_ids[row * S + s] == blo + q) {
              memb[q] = true;
              mbias[q] = s_bias[row * S + s];
              mslot[q] = s;
              break;
            }
        }
      }
    }

    float dsum[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int half = 0; half < 2; ++half)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int offk = 32 * half + d_row(r, h);
        const int j = j0 + offk;
        const bool win = (uint32_t)(j - my_ls) < wlen;
        bool rem = (uint32_t)(j - my_seg) < rlen;
        int qb = 0;
        float bb;
        if (one_blk) {
          rem = rem && memb[0];
          bb = mbias[0];
        } else {
          qb = sub_blk ? (offk >> bs_shift) : (j / BS - blo);
          bb = 0.f;
          bool mm = false;
#pragma unroll
          for (int qq = 0; qq < 5; ++qq)
            if (qb == qq) { mm = memb[qq]; bb = mbias[qq]; }
          rem = rem && mm;
        }
        const float sv = st[half][r];
        const float pv = (win || rem) ? exp2f((rem ? sv + bb : sv) * kLog2e - lse_l2) : 0.f;
        const float dsv = pv * (dp[half][r] - dlt);
        st[half][r] = dsv;
        if (rem) {
#pragma unroll
          for (int qq = 0; qq < 5; ++qq)
            if (qb == qq) dsum[qq] += dsv;
        }
      }
    if (a.dbias) {
#pragma unroll
      for (int qq = 0; qq < 5; ++qq) {
        const float tot = dsum[qq] + __shfl_xor(dsum[qq], 32, kWave);
        if (h == 0 && mslot[qq] >= 0) s_dbias[row * S + mslot[qq]] += tot;
      }
    }
    uint4 db[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int hf = ks >> 1, r0 = 8 * (ks & 1);
      db[ks] = make_uint4(M::pack2(st[hf][r0], st[hf][r0 + 1]), M::pack2(st[hf][r0 + 2], st[hf][r0 + 3]),
                          M::pack2(st[hf][r0 + 4], st[hf][r0 + 5]), M::pack2(st[hf][r0 + 6], st[hf][r0 + 7]));
    }
    // dQ^T += K^T dS^T  (K^T operands read column-wise from the natural K tile)
    const uint16_t* k16 = reinterpret_cast<const uint16_t*>(sK);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        dq[mt] = M::mac(a_operand_t<KP>(k16, 32 * mt + rl, ks, h), db[ks], dq[mt]);
  }

  if (row_ok) {
    T* qrow = reinterpret_cast<T*>(a.dq) + (int64_t)b * a.dq_sb + (int64_t)(t0 + row) * a.dq_st + (int64_t)hq * a.dq_sh;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = 32 * mt + 8 * g + 4 * h;
        uint2 w;
        w.x = M::pack2(dq[mt][4 * g] * a.scale, dq[mt][4 * g + 1] * a.scale);
        w.y = M::pack2(dq[mt][4 * g + 2] * a.scale, dq[mt][4 * g + 3] * a.scale);
        *reinterpret_cast<uint2*>(qrow + d0) = w;
      }
  }
  if (a.dbias) {
    __syncthreads();
    for (int e = tid; e < nrows * S; e += NT) {
      const int r = e / S, s = e % S;
      a.dbias[(int64_t)b * a.db_sb + (int64_t)hq * a.db_sh + (int64_t)(t0 + r) * a.db_st + s] = s_dbias[e];
    }
  }
}

// -------------------------------------------------------------- 4. dK / dV
template <typename T, int D>
__global__ __launch_bounds__(128) void dkv_kernel(BwdK p) {
  using M = Mfma<T>;
  constexpr int KP = D + 8;
  constexpr int KS = D / 16;
  constexpr int MT = D / 32;
  constexpr int NQ = 5;                       // blocks a 64-key chunk can overlap (BS >= 16)
  extern __shared__ __align__(16) unsigned char smem[];
  const srswa_bwd_args& a = p.a;
  T* sQ = reinterpret_cast<T*>(smem);         // [64][KP]  q * scale, rounded
  T* sG = sQ + kTileRows * KP;                // [64][KP]  dO
  int4* s_row = reinterpret_cast<int4*>(sG + kTileRows * KP);   // {qi, ls, seg, lse*log2e bits}
  float* s_dlt = reinterpret_cast<float*>(s_row + 64);
  float* s_mb = s_dlt + 64;                   // [64][NQ] bias if member else NaN
  int* s_ids = reinterpret_cast<int*>(s_mb + 64 * NQ);   // [64 * S]
  float* s_bias = reinterpret_cast<float*>(s_ids + 64 * a.S);

  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int h = lane / 32, rl = lane % 32;
  const int c = blockIdx.x % p.nchunk;
  const int64_t bk = blockIdx.x / p.nchunk;
  const int kvh = (int)(bk % a.HKV);
  const int b = (int)(bk / a.HKV);
  const int j0 = c * kChunk;
  const int jmine = j0 + 32 * wave + rl;       // this lane's key
  const bool key_ok = jmine < a.Sk;
  const int off = a.Sk - a.T;
  const int BS = a.block_size, LW = a.local_window, S = a.S;
  const int blo = j0 / BS;
  const int bhi = min(j0 + kChunk - 1, a.Sk - 1) / BS;
  const int qmine = jmine / BS - blo;

  uint4 kf[KS], vf[KS];
  {
    const T* krow = reinterpret_cast<const T*>(a.k) + (int64_t)b * a.k_sb + (int64_t)(key_ok ? jmine : 0) * a.k_st + (int64_t)kvh * a.k_sh;
    const T* vrow = reinterpret_cast<const T*>(a.v) + (int64_t)b * a.v_sb + (int64_t)(key_ok ? jmine : 0) * a.v_st + (int64_t)kvh * a.v_sh;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      kf[ks] = key_ok ? *reinterpret_cast<const uint4*>(krow + 16 * ks + 8 * h) : make_uint4(0, 0, 0, 0);
      vf[ks] = key_ok ? *reinterpret_cast<const uint4*>(vrow + 16 * ks + 8 * h) : make_uint4(0, 0, 0, 0);
    }
  }
  f32x16_t dk[MT], dv[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) { dk[mt] = zero16(); dv[mt] = zero16(); }

  // query tiles whose windows can reach this chunk: qi in [j0, j0 + 63 + LW - 1]
  const int wlo_t = j0 - off, whi_t = j0 + kChunk - 1 + LW - 1 - off;
  const int tau_a = max(wlo_t, 0) / kTileRows;
  const int tau_b = whi_t < 0 ? -1 : min(whi_t / kTileRows, p.ntiles - 1);

  constexpr int NT = 128;
  constexpr int PPT = kTileRows * D / 8 / NT;
  uint4 qpre[PPT], gpre[PPT];   // one tile's Q / dO pieces (loaded together, then staged)
  int* s_tiles = reinterpret_cast<int*>(s_bias + 64 * a.S);    // visit list
  __shared__ int s_ntiles;

  for (int gq = 0; gq < p.G; ++gq) {
    const int hq = kvh * p.G + gq;
    const int ih = hq / p.IG;
    const uint32_t* tb = p.touch + (((int64_t)b * a.HI + ih) * p.nchunk + c) * p.twords;
    // visit list: window tiles [tau_a, tau_b] plus every touched tile, ascending
    __syncthreads();
    if (tid == 0) {
      int n = 0;
      for (int w = 0; w < p.twords; ++w) {
        uint32_t bits = tb[w];
        const int lo = max(tau_a - 32 * w, 0), hi = min(tau_b - 32 * w, 31);
        if (lo <= hi) bits |= (hi - lo == 31) ? 0xffffffffu : (((1u << (hi - lo + 1)) - 1u) << lo);
        while (bits) {
          const int tau = 32 * w + __ffs(bits) - 1;
          bits &= bits - 1;
          if (tau < p.ntiles) s_tiles[n++] = tau;
        }
      }
      s_ntiles = n;
    }
    __syncthreads();
    const int nt = s_ntiles;
    auto fetch = [&](int tau) {
      const int t0 = tau * kTileRows;
      const int nrows = min(kTileRows, a.T - t0);
#pragma unroll
      for (int i = 0; i < PPT; ++i) {
        const int pc = tid + i * NT;
        const int r = pc / (D / 8), col = pc % (D / 8);
        const bool in = r < nrows;
        qpre[i] = in ? *reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(a.q) + (int64_t)b * a.q_sb +
                                                       (int64_t)(t0 + r) * a.q_st + (int64_t)hq * a.q_sh + col * 8)
                     : make_uint4(0, 0, 0, 0);
        gpre[i] = in ? *reinterpret_cast<const uint4*>(reinterpret_cast<const T*>(a.dout) + (int64_t)b * a.do_sb +
                                                       (int64_t)(t0 + r) * a.do_st + (int64_t)hq * a.do_sh + col * 8)
                     : make_uint4(0, 0, 0, 0);
      }
    };
    for (int it = 0; it < nt; ++it) {
      const int tau = s_tiles[it];
      {
        const int t0 = tau * kTileRows;
        const int nrows = min(kTileRows, a.T - t0);
        fetch(tau);        // all loads of the tile in flight at once
        __syncthreads();   // previous tile consumed
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
          const int pc = tid + i * NT;
          const int r = pc / (D / 8), col = pc % (D / 8);
          uint4 qw = qpre[i];
          uint32_t* ww = reinterpret_cast<uint32_t*>(&qw);
#pragma unroll
          for (int e = 0; e < 4; ++e) ww[e] = M::pack2(M::lo(ww[e]) * a.scale, M::hi(ww[e]) * a.scale);
          *reinterpret_cast<uint4*>(sQ + r * KP + col * 8) = qw;
          *reinterpret_cast<uint4*>(sG + r * KP + col * 8) = gpre[i];
        }
        for (int r = tid; r < 64; r += NT) {
          int4 ri = make_int4(INT_MIN, 0, 0, 0);   // invalid row: qi < every key
          float dl = 0.f;
          if (r < nrows) {
            const int t = t0 + r;
            const int qi = off + t;
            const int seg = a.seg ? a.seg[(int64_t)b * a.seg_sb + t] : 0;
            const float lse = a.lse[(int64_t)b * a.lse_sb + (int64_t)t * a.lse_st + (int64_t)hq * a.lse_sh];
            ri = make_int4(qi, max(qi - LW + 1, seg), seg, __float_as_int(lse * kLog2e));
            dl = p.delta[((int64_t)b * a.T + t) * a.HQ + hq];
          }
          s_row[r] = ri;
          s_dlt[r] = dl;
        }
        for (int e = tid; e < 64 * S; e += NT) {
          const int r = e / S, s = e % S;
          int id = -1;
          float bv = 0.f;
          if (r < nrows) {
            id = a.idx[(int64_t)b * a.idx_sb + (int64_t)ih * a.idx_sh + (int64_t)(t0 + r) * a.idx_st + s];
            if (a.bias) bv = a.bias[(int64_t)b * a.bias_sb + (int64_t)ih * a.bias_sh + (int64_t)(t0 + r) * a.bias_st + s];
          }
          s_ids[e] = id;
          s_bias[e] = bv;
        }
        __syncthreads();
        // membership of every row in the chunk's blocks (first slot's bias)
        for (int e = tid; e < 64 * NQ; e += NT) {
          const int r = e / NQ, qq = e % NQ;
          float mb = __int_as_float(0x7fc00000);   // NaN: not selected
          const int blk = blo + qq;
          if (r < nrows && blk <= bhi) {
            for (int s = 0; s < S; ++s)
              if (s_ids[r * S + s] == blk) { mb = s_bias[r * S + s]; break; }
          }
          s_mb[e] = mb;
        }
        __syncthreads();

        // S = Q K^T and dP = dO V^T for the 64 rows x this lane's key
        f32x16_t sp[2] = {zero16(), zero16()}, gd[2] = {zero16(), zero16()};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          sp[0] = M::mac(*reinterpret_cast<const uint4*>(sQ + rl * KP + 16 * ks + 8 * h), kf[ks], sp[0]);
          sp[1] = M::mac(*reinterpret_cast<const uint4*>(sQ + (32 + rl) * KP + 16 * ks + 8 * h), kf[ks], sp[1]);
          gd[0] = M::mac(*reinterpret_cast<const uint4*>(sG + rl * KP + 16 * ks + 8 * h), vf[ks], gd[0]);
          gd[1] = M::mac(*reinterpret_cast<const uint4*>(sG + (32 + rl) * KP + 16 * ks + 8 * h), vf[ks], gd[1]);
        }
        // in place: sp <- P, gd <- dS
#pragma unroll
        for (int half = 0; half < 2; ++half)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = 32 * half + d_row(r, h);
            const int4 ri = s_row[row];
            const float mb = s_mb[row * NQ + qmine];
            const bool win = jmine >= ri.y && jmine <= ri.x;
            const bool rem = !win && jmine >= ri.z && jmine < ri.y && jmine <= ri.x && !(mb != mb);
            const float sv = sp[half][r];
            const float pv = (key_ok && (win || rem)) ? exp2f((rem ? sv + mb : sv) * kLog2e - __int_as_float(ri.w)) : 0.f;
            sp[half][r] = pv;
            gd[half][r] = pv * (gd[half][r] - s_dlt[row]);
          }
        uint4 pb[4], db[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const int hf = ks >> 1, r0 = 8 * (ks & 1);
          pb[ks] = make_uint4(M::pack2(sp[hf][r0], sp[hf][r0 + 1]), M::pack2(sp[hf][r0 + 2], sp[hf][r0 + 3]),
                              M::pack2(sp[hf][r0 + 4], sp[hf][r0 + 5]), M::pack2(sp[hf][r0 + 6], sp[hf][r0 + 7]));
          db[ks] = make_uint4(M::pack2(gd[hf][r0], gd[hf][r0 + 1]), M::pack2(gd[hf][r0 + 2], gd[hf][r0 + 3]),
                              M::pack2(gd[hf][r0 + 4], gd[hf][r0 + 5]), M::pack2(gd[hf][r0 + 6], gd[hf][r0 + 7]));
        }
        // dV^T += dO^T P ; dK^T += (q*scale)^T dS  (transposed operands read
        // column-wise from the natural Q / dO tiles)
        const uint16_t* g16 = reinterpret_cast<const uint16_t*>(sG);
        const uint16_t* q16 = reinterpret_cast<const uint16_t*>(sQ);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) {
            dv[mt] = M::mac(a_operand_t<KP>(g16, 32 * mt + rl, ks, h), pb[ks], dv[mt]);
            dk[mt] = M::mac(a_operand_t<KP>(q16, 32 * mt + rl, ks, h), db[ks], dk[mt]);
          }
      }
    }
  }

  if (!key_ok) return;
  T* kout = reinterpret_cast<T*>(a.dk) + (int64_t)b * a.dk_sb + (int64_t)jmine * a.dk_st + (int64_t)kvh * a.dk_sh;
  T* vout = reinterpret_cast<T*>(a.dv) + (int64_t)b * a.dv_sb + (int64_t)jmine * a.dv_st + (int64_t)kvh * a.dv_sh;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * mt + 8 * g + 4 * h;
      uint2 wk, wv;
      wk.x = M::pack2(dk[mt][4 * g], dk[mt][4 * g + 1]);
      wk.y = M::pack2(dk[mt][4 * g + 2], dk[mt][4 * g + 3]);
      wv.x = M::pack2(dv[mt][4 * g], dv[mt][4 * g + 1]);
      wv.y = M::pack2(dv[mt][4 * g + 2], dv[mt][4 * g + 3]);
      *reinterpret_cast<uint2*>(kout + d0) = wk;
      *reinterpret_cast<uint2*>(vout + d0) = wv;
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
  if (a->dtype != SRSWA_BF16 && a->dtype != SRSWA_F16) {
    set_error("bwd: matrix-core path takes bf16 / fp16");
    return SRSWA_UNSUPPORTED;
  }
  if (!(a->D == 64 || a->D == 128) || a->block_size < 16 || a->S > 64) {
    set_error("bwd: D in {64,128}, block size >= 16, <= 64 slots");
    return SRSWA_UNSUPPORTED;
  }
  const int64_t st[] = {a->q_sb, a->q_st, a->q_sh, a->k_sb, a->k_st, a->k_sh, a->v_sb, a->v_st, a->v_sh,
                        a->o_sb, a->o_st, a->o_sh, a->do_sb, a->do_st, a->do_sh, a->dq_sb, a->dq_st,
                        a->dq_sh, a->dk_sb, a->dk_st, a->dk_sh, a->dv_sb, a->dv_st, a->dv_sh};
  for (int64_t s : st)
    if ((s * 2) % 16) {
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
  const int per_row = a->S * (ceil_div(a->block_size, kChunk) + 1) + ceil_div(a->local_window, kChunk) + 1;
  k.umax = (int)std::min<int64_t>((int64_t)k.nchunk, (int64_t)kTileRows * per_row);
  k.twords = ceil_div(k.ntiles, 32);
  k.G = a->HQ / a->HKV;
  k.IG = a->HQ / a->HI;
}

size_t delta_bytes(const BwdK& k) {
  return ((size_t)k.a.B * k.a.T * k.a.HQ * 4 + 255) / 256 * 256;
}
size_t touch_words(const BwdK& k) { return (size_t)k.a.B * k.a.HI * k.nchunk * k.twords; }

size_t dq_smem(const BwdK& k) {
  const int D = k.a.D;
  size_t n = (size_t)kChunk * (D + 8) * 2 * 2 + (size_t)kSlotCap * 64 * 8;
  n += 3 * 64 * 4 + (size_t)64 * k.a.S * 4 * 3 + (size_t)k.nwords * 4 + (size_t)k.umax * 4 + 16;
  return (n + 15) / 16 * 16;
}
size_t dkv_smem(const BwdK& k) {
  const int D = k.a.D;
  size_t n = (size_t)kTileRows * (D + 8) * 2 * 2;
  n += 64 * 16 + 64 * 4 + 64 * 5 * 4 + (size_t)64 * k.a.S * 4 * 2 + (size_t)k.ntiles * 4 + 16;
  return (n + 15) / 16 * 16;
}

template <typename T, int D>
int launch_bwd(const BwdK& k, hipStream_t st) {
  static size_t granted_dq = 0, granted_dkv = 0;
  if (!ensure_dynamic_lds(&dq_kernel<T, D>, dq_smem(k), &granted_dq) ||
      !ensure_dynamic_lds(&dkv_kernel<T, D>, dkv_smem(k), &granted_dkv))
    return SRSWA_UNSUPPORTED;
  const srswa_bwd_args& a = k.a;
  const int rpw = kWave / (D / 8);
  const int64_t rows = (int64_t)a.B * a.T * a.HQ;
  hipLaunchKernelGGL((delta_kernel<T, D>), dim3((unsigned)((rows + 4 * rpw - 1) / (4 * rpw))), dim3(256), 0, st, k);
  const int64_t nw = (int64_t)touch_words(k);
  if (nw > 0) hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)((nw + 255) / 256)), dim3(256), 0, st, k.touch, nw);
  const int64_t ne = (int64_t)a.B * a.HI * a.T * a.S;
  if (ne > 0) hipLaunchKernelGGL(touch_kernel, dim3((unsigned)((ne + 255) / 256)), dim3(256), 0, st, k);
  hipLaunchKernelGGL((dq_kernel<T, D>), dim3((unsigned)((int64_t)a.B * a.HQ * k.ntiles)), dim3(128),
                     dq_smem(k), st, k);
  hipLaunchKernelGGL((dkv_kernel<T, D>), dim3((unsigned)((int64_t)a.B * a.HKV * k.nchunk)), dim3(128),
                     dkv_smem(k), st, k);
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
  return delta_bytes(k) + touch_words(k) * 4;
}

extern "C" int srswa_gather_bwd(const srswa_bwd_args* a, void* scratch, size_t scratch_bytes,
                                void* stream) {
  int st = check_bwd(a);
  if (st != SRSWA_OK) return st;
  if (a->B == 0 || a->T == 0) return SRSWA_OK;
  BwdK k{};
  plan_bwd(a, k);
  const size_t need = delta_bytes(k) + touch_words(k) * 4;
  if (!scratch || scratch_bytes < need) {
    set_error("bwd: scratch of %zu bytes required (got %zu)", need, scratch_bytes);
    return SRSWA_WORKSPACE;
  }
  if (dq_smem(k) > 156 * 1024 || dkv_smem(k) > 156 * 1024) {
    set_error("bwd: LDS budget exceeded (key length too large)");
    return SRSWA_UNSUPPORTED;
  }
  k.delta = reinterpret_cast<float*>(scratch);
  k.touch = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(scratch) + delta_bytes(k));
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (a->dtype == SRSWA_BF16)
    return a->D == 128 ? launch_bwd<bf16_t, 128>(k, s) : launch_bwd<bf16_t, 64>(k, s);
  return a->D == 128 ? launch_bwd<__half, 128>(k, s) : launch_bwd<__half, 64>(k, s);
}
