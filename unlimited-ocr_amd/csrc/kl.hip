// Gather-KL of the indexer's distillation loss on the matrix cores (gfx950).
//
// Replaces the KL term of the DASH / "sparse" stage training step:
//   the n_idx_heads == 1 gather branch of select_and_kl_loss  HF/_sparse_base_impl.py:3413-3478
//   _kl_chunk_core / _KLChunkFn (multi-index-head form)       HF/_sparse_base_impl.py:2071-2190
// For query row t of index head ih, over its selected blocks' keys j with
// seg_t <= j < max(pos_t - LW + 1, 0) (the token window excluded):
//   teacher  p_j = mean over the G query heads h of ih of softmax_j(scaling * bf16(q_h . k_j))
//   student  log q_j = log_softmax_j(bf16(qi . ki_j))
//   kl_t = sum_j p_j (log max(p_j, 1e-12) - log q_j),  valid_t = any key kept
// and, for the backward, dsel[t, slot, u] = q_j - p_j for key j = 64 id + u of
// each selected slot (0 where not kept): d kl / d s_j.
//
// Forward: one workgroup per (sequence, index head, 64-row tile), two waves of
// 32 rows (lane = row, S^T = K Q^T as in the attention forward).  The tile
// visits the union of its rows' selected 64-key blocks that hold kept keys:
//   pass 1, head-outer: each head's (max, sum) softmax statistics per row
//            (the G teacher heads, then the student);
//   pass 2, block-outer: every head's logits again, p mixed over the heads in
//            registers, the student's log-softmax, the KL terms and dsel.
// Keys are staged per (head, block) in LDS from registers fetched one stage
// ahead (with the next stage's query fragments).
// Backward (student path only, the teacher carries no gradient):
//   dq_kernel -- one wavefront per row: dq = sum_j bf16(g dsel_j) ki_j;
//   dk_kernel -- one workgroup per (sequence, block): the rows that selected
//                the block, in row order (deterministic), dk_u += bf16(g dsel_u) qi.
#include <algorithm>

#include "mfma_common.h"

namespace srswa {
namespace {

struct KlK {
  srswa_kl_args a;
  int ntiles, nwords, G, KV;     // G = query heads per index head, KV = query heads per kv head
  int nlogical, per_xcd;
  int ids_off, bits_off, chunks_off, stats_off;   // LDS byte offsets
};

template <int D> struct KlLds {
  static constexpr int KP = D + 8;                 // conflict-free 16-byte row reads
  static constexpr int tileBytes = kChunk * KP * 2;
};

template <typename T> __device__ __forceinline__ float round_to(float v);
template <> __device__ __forceinline__ float round_to<bf16_t>(float v) { return bf16_lo(pack_bf16x2(v, 0.f)); }
template <> __device__ __forceinline__ float round_to<__half>(float v) {
  return __half2float(__float2half_rn(v));
}

template <typename T, int D>
__global__ __launch_bounds__(128, 1) void kl_fwd_kernel(KlK p) {
  using M = Mfma<T>;
  using L = KlLds<D>;
  constexpr int KP = L::KP, KS = D / 16, NT = 128;
  constexpr int PPT = kChunk * D / 8 / NT;
  constexpr int RPP = NT / (D / 8);
  extern __shared__ __align__(16) unsigned char smem[];
  const srswa_kl_args& a = p.a;

  const int lid = (int)(blockIdx.x & 7) * p.per_xcd + (int)(blockIdx.x >> 3);
  if (lid >= p.nlogical) return;
  T* sK = reinterpret_cast<T*>(smem);
  int* s_ids = reinterpret_cast<int*>(smem + p.ids_off);          // [64][K], -1 = no kept key
  uint32_t* s_bits = reinterpret_cast<uint32_t*>(smem + p.bits_off);
  uint16_t* s_chunks = reinterpret_cast<uint16_t*>(smem + p.chunks_off);
  int* s_count = reinterpret_cast<int*>(s_bits + p.nwords);
  float2* s_st = reinterpret_cast<float2*>(smem + p.stats_off);   // [G + 1][64] (max, sum)

  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int h = lane >> 5, rl = lane & 31;
  const int tile = lid % p.ntiles;
  const int bh = lid / p.ntiles;
  const int ih = bh % a.HI, b = bh / a.HI;
  const int t0 = tile * kTileRows;
  const int nrows = min(kTileRows, a.T - t0);
  const int K = a.K, G = p.G, LW = a.local_window;
  const int64_t ds_tile = (int64_t)b * a.ds_sb + (int64_t)ih * a.ds_sh;

  auto row_range = [&](int r, int& lo, int& hi) {
    const int t = t0 + r;
    const int pos = a.pos[(int64_t)b * a.pos_sb + t];
    lo = a.seg ? a.seg[(int64_t)b * a.seg_sb + t] : 0;
    hi = min(max(pos - LW + 1, 0), a.Sk);
  };

  // set-up: the rows' selected blocks that hold kept keys, and their union
  for (int w = tid; w < p.nwords; w += NT) s_bits[w] = 0u;
  __syncthreads();
  for (int e = tid; e < kTileRows * K; e += NT) {
    const int r = e / K, s = e % K;
    int id = -1;
    if (r < nrows) {
      int lo, hi;
      row_range(r, lo, hi);
      const int32_t* ids = a.sel + (int64_t)b * a.sel_sb + (int64_t)ih * a.sel_sh + (int64_t)(t0 + r) * a.sel_st;
      id = ids[s];
      if (id < 0 || (int64_t)id * kChunk >= hi || (int64_t)id * kChunk + kChunk <= lo) id = -1;
      for (int s2 = 0; s2 < s && id >= 0; ++s2)          // a repeated id counts once (first slot)
        if (ids[s2] == id) id = -1;
      if (id < 0 && a.dsel) {             // a slot with nothing kept: its dsel row is zero
        float4* z = reinterpret_cast<float4*>(a.dsel + ds_tile + (int64_t)(t0 + r) * a.ds_st + (int64_t)s * kChunk);
#pragma unroll
        for (int i = 0; i < kChunk / 4; ++i) z[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    s_ids[e] = id;
    if (id >= 0) atomicOr(&s_bits[id >> 5], 1u << (id & 31));
  }
  __syncthreads();
  const int U = compact_bitmap(s_bits, p.nwords, s_chunks, s_count);

  const int row = wave * 32 + rl;
  const bool row_ok = row < nrows;
  int lo = 0, hi = 0;
  if (row_ok) row_range(row, lo, hi);
  const int* my_ids = s_ids + row * K;

  // stages: pass 1 (hh, u) head-outer, pass 2 (u, hh) block-outer; hh == G is the student
  const int per_pass = (G + 1) * U;
  const int nstage = 2 * per_pass;
  auto stage_of = [&](int i, int& hh, int& u) {
    if (i < per_pass) {
      hh = i / U;
      u = i % U;
    } else {
      u = (i - per_pass) / (G + 1);
      hh = (i - per_pass) % (G + 1);
    }
  };
  auto key_base = [&](int hh, int64_t& st) -> const T* {
    if (hh == G) {
      st = a.ik_st;
      return reinterpret_cast<const T*>(a.idx_k) + (int64_t)b * a.ik_sb;
    }
    const int kvh = (ih * G + hh) / p.KV;
    st = a.km_st;
    return reinterpret_cast<const T*>(a.k_main) + (int64_t)b * a.km_sb + (int64_t)kvh * a.km_sh;
  };
  auto q_row = [&](int hh) -> const T* {
    const int t = t0 + (row_ok ? row : 0);
    if (hh == G)
      return reinterpret_cast<const T*>(a.q_idx) + (int64_t)b * a.qi_sb + (int64_t)ih * a.qi_sh + (int64_t)t * a.qi_st;
    return reinterpret_cast<const T*>(a.q_main) + (int64_t)b * a.qm_sb + (int64_t)(ih * G + hh) * a.qm_sh +
           (int64_t)t * a.qm_st;
  };

  T* sKw = sK + (tid / (D / 8)) * KP + (tid % (D / 8)) * 8;
  uint4 kpre[PPT], qpre[KS], qf[KS];
  auto fetch = [&](int i) {
    int hh, u;
    stage_of(i, hh, u);
    int64_t st;
    const T* base = key_base(hh, st);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(base, (uint32_t)(((int64_t)(a.Sk - 1) * st + D) * 2));
    const uint32_t vo = (uint32_t)((tid / (D / 8)) * st + (tid % (D / 8)) * 8) * 2;
    const uint32_t so = (uint32_t)s_chunks[u] * kChunk * (uint32_t)st * 2u;
#pragma unroll
    for (int k = 0; k < PPT; ++k) kpre[k] = buffer_load16(rs, vo, so + (uint32_t)(k * RPP) * (uint32_t)st * 2u);
    const T* qr = q_row(hh);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qpre[ks] = row_ok ? *reinterpret_cast<const uint4*>(qr + 16 * ks + 8 * h) : make_uint4(0, 0, 0, 0);
  };

  float m_run = -INFINITY, l_run = 0.f;   // pass 1: this lane's keys of the current head
  float pacc[32];                         // pass 2: teacher p of this lane's 32 keys of the block
#pragma unroll
  for (int r = 0; r < 32; ++r) pacc[r] = 0.f;
  float kl_acc = 0.f;
  int slot = -1;
  uint64_t keep = 0ull;

  if (nstage > 0) fetch(0);
  for (int i = 0; i < nstage; ++i) {
    int hh, u;
    stage_of(i, hh, u);
    const bool pass2 = i >= per_pass;
    __syncthreads();                       // previous stage's keys consumed
#pragma unroll
    for (int k = 0; k < PPT; ++k) *reinterpret_cast<uint4*>(sKw + k * RPP * KP) = kpre[k];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = qpre[ks];
    __syncthreads();
    if (i + 1 < nstage) fetch(i + 1);

    const int c = s_chunks[u];
    const int j0 = c * kChunk;
    if (!pass2 || hh == 0) {              // the row's slot of this block and its kept keys
      slot = -1;
      for (int s = 0; s < K; ++s)
        if (my_ids[s] == c) {
          slot = s;
          break;
        }
      keep = (row_ok && slot >= 0) ? range64(min(max(lo - j0, 0), 64), min(max(hi - j0, 0), 64)) : 0ull;
    }
    f32x16_t st[2] = {zero16(), zero16()};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      st[0] = M::mac(*reinterpret_cast<const uint4*>(sK + rl * KP + 16 * ks + 8 * h), qf[ks], st[0]);
      st[1] = M::mac(*reinterpret_cast<const uint4*>(sK + (32 + rl) * KP + 16 * ks + 8 * h), qf[ks], st[1]);
    }
    // logits in the reference's rounding: the product rounded to the input
    // dtype, the teacher's then scaled; key of register r of half `half`:
    // 32 half + 8 (r / 4) + 4h + r % 4
    const float mul = hh == G ? 1.f : a.scaling;
    const uint64_t kh = keep >> (4 * h);
    if (!pass2) {
      float mloc = -INFINITY;
#pragma unroll
      for (int half = 0; half < 2; ++half)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float x = round_to<T>(st[half][r]) * mul;
          st[half][r] = x;
          if ((kh >> (32 * half + 8 * (r >> 2) + (r & 3))) & 1ull) mloc = fmaxf(mloc, x);
        }
      if (mloc > -INFINITY) {
        const float mn = fmaxf(m_run, mloc);
        float l = m_run > -INFINITY ? l_run * __builtin_amdgcn_exp2f((m_run - mn) * kLog2e) : 0.f;
#pragma unroll
        for (int half = 0; half < 2; ++half)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if ((kh >> (32 * half + 8 * (r >> 2) + (r & 3))) & 1ull)
              l += __builtin_amdgcn_exp2f((st[half][r] - mn) * kLog2e);
        m_run = mn;
        l_run = l;
      }
      if (u == U - 1) {                    // the head's statistics for the row: merge the lane pair
        const float mo = __shfl_xor(m_run, 32, kWave), lo2 = __shfl_xor(l_run, 32, kWave);
        const float mm = fmaxf(m_run, mo);
        float ll = 0.f;
        if (mm > -INFINITY) {
          if (m_run > -INFINITY) ll += l_run * __builtin_amdgcn_exp2f((m_run - mm) * kLog2e);
          if (mo > -INFINITY) ll += lo2 * __builtin_amdgcn_exp2f((mo - mm) * kLog2e);
        }
        if (h == 0) s_st[hh * 64 + row] = make_float2(mm, ll);
        m_run = -INFINITY;
        l_run = 0.f;
      }
      continue;
    }
    // pass 2
    const float2 ml = s_st[hh * 64 + row];
    if (hh < G) {
      if (ml.y > 0.f) {
        const float inv = 1.f / ml.y;
#pragma unroll
        for (int half = 0; half < 2; ++half)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const bool kp = (kh >> (32 * half + 8 * (r >> 2) + (r & 3))) & 1ull;
            const float x = round_to<T>(st[half][r]) * mul;
            pacc[16 * half + r] += kp ? __builtin_amdgcn_exp2f((x - ml.x) * kLog2e) * inv : 0.f;
          }
      }
      continue;
    }
    // student: log-softmax, KL terms, dsel; then the next block starts from zero
    const float lse = ml.y > 0.f ? ml.x + logf(ml.y) : 0.f;
    const float invg = 1.f / (float)G;
    float dsv[32];
#pragma unroll
    for (int half = 0; half < 2; ++half)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const bool kp = (kh >> (32 * half + 8 * (r >> 2) + (r & 3))) & 1ull;
        const float x = round_to<T>(st[half][r]);
        const float pv = pacc[16 * half + r] * invg;
        const float logq = x - lse;
        if (kp) kl_acc += pv * (logf(fmaxf(pv, 1e-12f)) - logq);
        dsv[16 * half + r] = kp ? __builtin_amdgcn_exp2f(logq * kLog2e) - pv : 0.f;
        pacc[16 * half + r] = 0.f;
      }
    if (a.dsel && row_ok && slot >= 0) {
      float* drow = a.dsel + ds_tile + (int64_t)(t0 + row) * a.ds_st + (int64_t)slot * kChunk;
#pragma unroll
      for (int half = 0; half < 2; ++half)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
          *reinterpret_cast<float4*>(drow + 32 * half + 8 * r4 + 4 * h) =
              make_float4(dsv[16 * half + 4 * r4], dsv[16 * half + 4 * r4 + 1], dsv[16 * half + 4 * r4 + 2],
                          dsv[16 * half + 4 * r4 + 3]);
    }
  }

  const float kl_row = kl_acc + __shfl_xor(kl_acc, 32, kWave);
  if (row_ok && h == 0) {
    const float2 sst = U > 0 ? s_st[G * 64 + row] : make_float2(-INFINITY, 0.f);
    const bool valid = sst.y > 0.f;
    a.kl[(int64_t)b * a.kl_sb + (int64_t)ih * a.kl_sh + t0 + row] = valid ? kl_row : 0.f;
    a.valid[(int64_t)b * a.va_sb + (int64_t)ih * a.va_sh + t0 + row] = valid ? 1 : 0;
  }
}

// -------------------------------------------------------------- backward
// dq: one wavefront per (sequence, index head, row); lane l owns head-dim
// elements 2l, 2l + 1 (D = 128) or l (D = 64); ds broadcast by shuffles.
template <typename T, int D>
__global__ __launch_bounds__(256) void kl_dq_kernel(srswa_kl_bwd_args a) {
  constexpr int EPL = D / kWave;                   // elements per lane (1 or 2)
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int64_t rowi = (int64_t)blockIdx.x * 4 + wave;
  if (rowi >= (int64_t)a.B * a.HI * a.T) return;
  const int t = (int)(rowi % a.T);
  const int ih = (int)((rowi / a.T) % a.HI);
  const int b = (int)(rowi / ((int64_t)a.T * a.HI));
  const float g = a.grad[(int64_t)b * a.g_sb + (int64_t)ih * a.g_sh + t];
  float acc[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
  const T* kb = reinterpret_cast<const T*>(a.idx_k) + (int64_t)b * a.ik_sb;
  if (g != 0.f) {
    const int32_t* ids = a.sel + (int64_t)b * a.sel_sb + (int64_t)ih * a.sel_sh + (int64_t)t * a.sel_st;
    const float* drow = a.dsel + (int64_t)b * a.ds_sb + (int64_t)ih * a.ds_sh + (int64_t)t * a.ds_st;
    for (int s = 0; s < a.K; ++s) {
      const int id = ids[s];
      if (id < 0 || (int64_t)id * kChunk >= a.Sk) continue;
      const float dsl = round_to<T>(g * drow[s * kChunk + lane]);   // d s in the input dtype
      const int nk = min(kChunk, a.Sk - id * kChunk);
      for (int u = 0; u < nk; ++u) {
        const float dsu = __shfl(dsl, u, kWave);
        if (dsu == 0.f) continue;
        const T* kr = kb + (int64_t)(id * kChunk + u) * a.ik_st + lane * EPL;
        if constexpr (EPL == 2) {
          const uint32_t w = *reinterpret_cast<const uint32_t*>(kr);
          acc[0] += dsu * Mfma<T>::lo(w);
          acc[1] += dsu * Mfma<T>::hi(w);
        } else {
          const uint16_t w = *reinterpret_cast<const uint16_t*>(kr);
          acc[0] += dsu * Mfma<T>::lo((uint32_t)w);
        }
      }
    }
  }
  T* out = reinterpret_cast<T*>(a.dq_idx) + (int64_t)b * a.dq_sb + (int64_t)ih * a.dq_sh + (int64_t)t * a.dq_st +
           lane * EPL;
  if constexpr (EPL == 2) {
    *reinterpret_cast<uint32_t*>(out) = Mfma<T>::pack2(acc[0], acc[1]);
  } else {
    *reinterpret_cast<uint16_t*>(out) = (uint16_t)(Mfma<T>::pack2(acc[0], 0.f) & 0xffffu);
  }
}

// dk: one workgroup of 256 threads per (sequence, block); thread (u, q) owns
// key u's head-dim quarter q.  The rows of every index head are scanned in
// order, 256 at a time; the rows that selected the block are compacted into
// LDS and applied in order (deterministic).
constexpr int kDkThreads = 256;

template <typename T, int D>
__global__ __launch_bounds__(kDkThreads) void kl_dk_kernel(srswa_kl_bwd_args a, int nblk) {
  constexpr int DQ = D / 4;                        // head-dim elements per thread
  __shared__ int s_row[kDkThreads];                // (ih * T + t) of a matching row
  __shared__ int s_slot[kDkThreads];
  __shared__ int s_n;
  __shared__ int s_wc[kDkThreads / kWave];
  const int tid = threadIdx.x;
  const int c = blockIdx.x % nblk, b = blockIdx.x / nblk;
  const int u = tid / 4, q = tid % 4;
  float acc[DQ];
#pragma unroll
  for (int e = 0; e < DQ; ++e) acc[e] = 0.f;
  const int64_t nrow = (int64_t)a.HI * a.T;
  for (int64_t r0 = 0; r0 < nrow; r0 += kDkThreads) {
    if (tid == 0) s_n = 0;
    __syncthreads();
    const int64_t r = r0 + tid;
    int found = -1;
    if (r < nrow) {
      const int ih = (int)(r / a.T), t = (int)(r % a.T);
      const int32_t* ids = a.sel + (int64_t)b * a.sel_sb + (int64_t)ih * a.sel_sh + (int64_t)t * a.sel_st;
      for (int s = 0; s < a.K; ++s)
        if (ids[s] == c) {
          found = s;
          break;
        }
      if (found >= 0 && a.grad[(int64_t)b * a.g_sb + (int64_t)ih * a.g_sh + t] == 0.f) found = -1;
    }
    // order-preserving compaction: the prefix count of matches before this thread
    const uint64_t bal = __ballot(found >= 0);
    const int w = tid / kWave;
    if ((tid % kWave) == 0) s_wc[w] = __popcll(bal);
    __syncthreads();
    int base = 0;
    for (int i = 0; i < w; ++i) base += s_wc[i];
    if (found >= 0) {
      const int idx = base + __popcll(bal & ((1ull << (tid % kWave)) - 1ull));
      s_row[idx] = (int)r;
      s_slot[idx] = found;
    }
    if (tid == 0) {
      int n = 0;
      for (int i = 0; i < kDkThreads / kWave; ++i) n += s_wc[i];
      s_n = n;
    }
    __syncthreads();
    const int n = s_n;
    for (int e = 0; e < n; ++e) {
      const int rr = s_row[e], s = s_slot[e];
      const int ih = rr / a.T, t = rr % a.T;
      const float g = a.grad[(int64_t)b * a.g_sb + (int64_t)ih * a.g_sh + t];
      const float ds = round_to<T>(g * a.dsel[(int64_t)b * a.ds_sb + (int64_t)ih * a.ds_sh + (int64_t)t * a.ds_st +
                                             (int64_t)s * kChunk + u]);
      if (ds == 0.f) continue;
      const T* qr = reinterpret_cast<const T*>(a.q_idx) + (int64_t)b * a.qi_sb + (int64_t)ih * a.qi_sh +
                    (int64_t)t * a.qi_st + q * DQ;
#pragma unroll
      for (int e8 = 0; e8 < DQ / 8; ++e8) {
        const uint4 w4 = *reinterpret_cast<const uint4*>(qr + 8 * e8);
        const uint32_t ww[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          acc[8 * e8 + 2 * k] += ds * Mfma<T>::lo(ww[k]);
          acc[8 * e8 + 2 * k + 1] += ds * Mfma<T>::hi(ww[k]);
        }
      }
    }
    __syncthreads();
  }
  const int key = c * kChunk + u;
  if (key >= a.Sk) return;
  T* out = reinterpret_cast<T*>(a.dk_idx) + (int64_t)b * a.dk_sb + (int64_t)key * a.dk_st + q * DQ;
#pragma unroll
  for (int e8 = 0; e8 < DQ / 8; ++e8) {
    uint4 w4;
    w4.x = Mfma<T>::pack2(acc[8 * e8], acc[8 * e8 + 1]);
    w4.y = Mfma<T>::pack2(acc[8 * e8 + 2], acc[8 * e8 + 3]);
    w4.z = Mfma<T>::pack2(acc[8 * e8 + 4], acc[8 * e8 + 5]);
    w4.w = Mfma<T>::pack2(acc[8 * e8 + 6], acc[8 * e8 + 7]);
    *reinterpret_cast<uint4*>(out + 8 * e8) = w4;
  }
}

bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int check_common(int dtype, int D, int block_size, int K, const char* what) {
  if (dtype != SRSWA_BF16 && dtype != SRSWA_F16) {
    set_error("%s: dtype %d not supported (bf16, fp16)", what, dtype);
    return SRSWA_UNSUPPORTED;
  }
  if (D != 64 && D != 128) {
    set_error("%s: head dim %d not supported (64, 128)", what, D);
    return SRSWA_UNSUPPORTED;
  }
  if (block_size != kChunk) {
    set_error("%s: block_size %d not supported (64)", what, block_size);
    return SRSWA_UNSUPPORTED;
  }
  if (K <= 0 || K > 64) {
    set_error("%s: %d selected blocks per row not supported (1..64)", what, K);
    return SRSWA_UNSUPPORTED;
  }
  return SRSWA_OK;
}

}  // namespace
}  // namespace srswa

using namespace srswa;

extern "C" int srswa_gather_kl_fwd(const srswa_kl_args* a, void* stream) {
  if (!a || !a->q_idx || !a->idx_k || !a->q_main || !a->k_main || !a->sel || !a->pos || !a->kl || !a->valid) {
    set_error("gather kl: null argument");
    return SRSWA_INVALID;
  }
  if (a->B < 0 || a->HI <= 0 || a->HQ <= 0 || a->HKV <= 0 || a->T < 0 || a->Sk <= 0 || a->local_window < 1 ||
      a->HQ % a->HI || a->HQ % a->HKV) {
    set_error("gather kl: bad sizes (HQ must be a multiple of HI and HKV)");
    return SRSWA_INVALID;
  }
  int rc = check_common(a->dtype, a->D, a->block_size, a->K, "gather kl");
  if (rc != SRSWA_OK) return rc;
  const int eb = 2;
  bool ok = al16(a->q_idx) && al16(a->idx_k) && al16(a->q_main) && al16(a->k_main) && (!a->dsel || al16(a->dsel));
  for (int64_t st : {a->qi_sb, a->qi_sh, a->qi_st, a->ik_sb, a->ik_st, a->qm_sb, a->qm_sh, a->qm_st, a->km_sb,
                     a->km_sh, a->km_st})
    ok = ok && (st * eb) % 16 == 0;
  if (a->dsel) ok = ok && (a->ds_sb * 4) % 16 == 0 && (a->ds_sh * 4) % 16 == 0 && (a->ds_st * 4) % 16 == 0;
  if (!ok) {
    set_error("gather kl: rows must be 16-byte aligned");
    return SRSWA_UNSUPPORTED;
  }
  const int64_t kspan = (int64_t)(a->Sk - 1) * std::max(a->ik_st, a->km_st) + a->D;
  if (kspan * eb >= (int64_t)1 << 32) {
    set_error("gather kl: a sequence's key span exceeds 4 GiB");
    return SRSWA_UNSUPPORTED;
  }
  if (a->T == 0 || a->B == 0) return SRSWA_OK;
  KlK k;
  k.a = *a;
  k.ntiles = ceil_div(a->T, kTileRows);
  const int nblk = ceil_div(a->Sk, kChunk);
  k.nwords = ceil_div(nblk, 32);
  k.G = a->HQ / a->HI;
  k.KV = a->HQ / a->HKV;
  k.nlogical = a->B * a->HI * k.ntiles;
  k.per_xcd = ceil_div(k.nlogical, 8);
  const int tile_bytes = a->D == 64 ? KlLds<64>::tileBytes : KlLds<128>::tileBytes;
  k.ids_off = tile_bytes;
  k.bits_off = k.ids_off + kTileRows * a->K * 4;
  k.chunks_off = k.bits_off + (k.nwords + 4) * 4;
  const int nchunk_max = std::min(kTileRows * a->K, nblk);
  k.stats_off = (k.chunks_off + nchunk_max * 2 + 15) & ~15;
  const size_t lds = (size_t)k.stats_off + (size_t)(k.G + 1) * kTileRows * 8;
  if (lds > 160 * 1024) {
    set_error("gather kl: %zu bytes of LDS needed", lds);
    return SRSWA_UNSUPPORTED;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)(8 * k.per_xcd)), block(128);
  static size_t granted[4] = {0, 0, 0, 0};
  bool lds_ok = true;
#define KL_LAUNCH(T_, D_, I_)                                                                    \
  lds_ok = ensure_dynamic_lds(kl_fwd_kernel<T_, D_>, lds, &granted[I_]);                       \
  if (lds_ok) hipLaunchKernelGGL((kl_fwd_kernel<T_, D_>), grid, block, lds, st, k);
  if (a->dtype == SRSWA_BF16) {
    if (a->D == 128) { KL_LAUNCH(bf16_t, 128, 0) } else { KL_LAUNCH(bf16_t, 64, 1) }
  } else {
    if (a->D == 128) { KL_LAUNCH(__half, 128, 2) } else { KL_LAUNCH(__half, 64, 3) }
  }
#undef KL_LAUNCH
  if (!lds_ok) return SRSWA_LAUNCH;
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("gather kl launch failed: %s", hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}

extern "C" int srswa_gather_kl_bwd(const srswa_kl_bwd_args* a, void* stream) {
  if (!a || !a->q_idx || !a->idx_k || !a->sel || !a->dsel || !a->grad || !a->dq_idx || !a->dk_idx) {
    set_error("gather kl backward: null argument");
    return SRSWA_INVALID;
  }
  if (a->B < 0 || a->HI <= 0 || a->T < 0 || a->Sk <= 0) {
    set_error("gather kl backward: bad sizes");
    return SRSWA_INVALID;
  }
  int rc = check_common(a->dtype, a->D, a->block_size, a->K, "gather kl backward");
  if (rc != SRSWA_OK) return rc;
  bool ok = al16(a->q_idx) && al16(a->dk_idx) && al16(a->idx_k) && al16(a->dq_idx);
  for (int64_t st : {a->qi_sb, a->qi_sh, a->qi_st, a->dk_sb, a->dk_st, a->ik_sb, a->ik_st, a->dq_sb, a->dq_sh,
                     a->dq_st})
    ok = ok && (st * 2) % 16 == 0;
  if (!ok) {
    set_error("gather kl backward: rows must be 16-byte aligned");
    return SRSWA_UNSUPPORTED;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int nblk = ceil_div(a->Sk, kChunk);
  const int64_t rows = (int64_t)a->B * a->HI * a->T;
  if (a->B > 0) {
    const dim3 gdk((unsigned)((int64_t)a->B * nblk));
    if (a->dtype == SRSWA_BF16) {
      if (a->D == 128) hipLaunchKernelGGL((kl_dk_kernel<bf16_t, 128>), gdk, dim3(kDkThreads), 0, st, *a, nblk);
      else hipLaunchKernelGGL((kl_dk_kernel<bf16_t, 64>), gdk, dim3(kDkThreads), 0, st, *a, nblk);
    } else {
      if (a->D == 128) hipLaunchKernelGGL((kl_dk_kernel<__half, 128>), gdk, dim3(kDkThreads), 0, st, *a, nblk);
      else hipLaunchKernelGGL((kl_dk_kernel<__half, 64>), gdk, dim3(kDkThreads), 0, st, *a, nblk);
    }
  }
  if (rows > 0) {
    const dim3 gdq((unsigned)((rows + 3) / 4));
    if (a->dtype == SRSWA_BF16) {
      if (a->D == 128) hipLaunchKernelGGL((kl_dq_kernel<bf16_t, 128>), gdq, dim3(256), 0, st, *a);
      else hipLaunchKernelGGL((kl_dq_kernel<bf16_t, 64>), gdq, dim3(256), 0, st, *a);
    } else {
      if (a->D == 128) hipLaunchKernelGGL((kl_dq_kernel<__half, 128>), gdq, dim3(256), 0, st, *a);
      else hipLaunchKernelGGL((kl_dq_kernel<__half, 64>), gdq, dim3(256), 0, st, *a);
    }
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("gather kl backward launch failed: %s", hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}
