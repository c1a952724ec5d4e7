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
// Forward: one workgroup per (sequence, index head, 64-row tile), four waves:
// two teams, team t owning keys [32 t, 32 t + 32) of every block, each team's
// two waves 32 rows (lane = row, S^T = K Q^T as in the attention forward).
// The tile visits the union of its rows' selected 64-key blocks that hold
// kept keys:
//   pass 1, head-outer: each head's (max, sum) softmax statistics per row and
//            key half (the G teacher heads, then the student), merged when read;
//   pass 2, block-outer: every head's logits again, p mixed over the heads in
//            registers, the student's log-softmax, the KL terms and dsel.
// Logits are carried in log2 units (scale * log2 e folded in once) so every
// probability is one fused multiply-add and exp2; masked keys enter the sums
// as exp2(-inf) = 0, and a wave whose rows all keep its key half takes a copy
// without per-key tests.  Keys are staged per (head, block) in LDS from
// registers fetched one stage ahead (with the next stage's query fragments;
// pass 1 reloads the query only when the head changes).
// Backward (student path only, the teacher carries no gradient): tile
// products on the matrix cores with ds = bf16(g dsel), see below.
#include <algorithm>

#include <type_traits>

#include "mfma_common.h"

namespace srswa {
namespace {

struct KlK {
  srswa_kl_args a;
  int ntiles, nwords, G, KV;     // G = query heads per index head, KV = query heads per kv head
  int nlogical, per_xcd;
  int ids_off, bits_off, chunks_off, stats_off;   // LDS byte offsets
  const uint32_t* rs_flag;       // [B, HI, ntiles]: tile taken by the row-sparse kernels, or NULL
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
__global__ __launch_bounds__(256, 2) void kl_fwd_kernel(KlK p) {
  using M = Mfma<T>;
  using L = KlLds<D>;
  constexpr int KP = L::KP, KS = D / 16, NT = 256;
  constexpr int PPT = kChunk * D / 8 / NT;
  constexpr int RPP = NT / (D / 8);
  extern __shared__ __align__(16) unsigned char smem[];
  const srswa_kl_args& a = p.a;

  const int lid = (int)(blockIdx.x & 7) * p.per_xcd + (int)(blockIdx.x >> 3);
  if (lid >= p.nlogical) return;
  T* sK = reinterpret_cast<T*>(smem);
  // [64][K] kept ids (-1 = none), or with slots_are_blocks [64][ceil(K / 32)]
  // bitmaps of the kept blocks (slot = block)
  int* s_ids = reinterpret_cast<int*>(smem + p.ids_off);
  uint32_t* s_bits = reinterpret_cast<uint32_t*>(smem + p.bits_off);
  uint16_t* s_chunks = reinterpret_cast<uint16_t*>(smem + p.chunks_off);
  int* s_count = reinterpret_cast<int*>(s_bits + p.nwords);
  float2* s_st = reinterpret_cast<float2*>(smem + p.stats_off);   // [2][G + 1][64] (max, sum) per key half
  float* s_kl = reinterpret_cast<float*>(s_st + 2 * (p.G + 1) * 64);  // [64] key half 1's KL sums

  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int h = lane >> 5, rl = lane & 31;
  // two teams of two waves: team `team` owns keys [32 team, 32 team + 32) of
  // every block for the tile's 64 rows (wave rw of the team: rows 32 rw ..)
  const int team = wave >> 1, rw = wave & 1;
  const int tile = lid % p.ntiles;
  const int bh = lid / p.ntiles;
  if (p.rs_flag && p.rs_flag[(int64_t)bh * p.ntiles + tile]) return;   // the row-sparse kernels take it
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
  const bool dense = a.slots_are_blocks != 0;
  const int nwk = (K + 31) >> 5;                  // bitmap words per row (slots_are_blocks)
  uint32_t* s_kb = reinterpret_cast<uint32_t*>(s_ids);
  for (int w = tid; w < p.nwords; w += NT) s_bits[w] = 0u;
  __syncthreads();
  // slot = block: a row lists block s as sel[s] == s (no repeats possible);
  // a listed block with no kept key gets a zero dsel row (the backward reads
  // every listed slot), unlisted slots are left alone
  for (int e = tid; dense && e < kTileRows * nwk; e += NT) {
    const int r = e / nwk, w = e % nwk;
    uint32_t bits = 0u;
    if (r < nrows) {
      int lo, hi;
      row_range(r, lo, hi);
      const int32_t* ids = a.sel + (int64_t)b * a.sel_sb + (int64_t)ih * a.sel_sh + (int64_t)(t0 + r) * a.sel_st;
      for (int j = 0; j < 32; ++j) {
        const int s = 32 * w + j;
        if (s >= K || ids[s] != s) continue;
        if ((int64_t)s * kChunk < hi && (int64_t)s * kChunk + kChunk > lo) {
          bits |= 1u << j;
        } else if (a.dsel) {
          float4* z = reinterpret_cast<float4*>(a.dsel + ds_tile + (int64_t)(t0 + r) * a.ds_st + (int64_t)s * kChunk);
#pragma unroll
          for (int i = 0; i < kChunk / 4; ++i) z[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
    }
    s_kb[e] = bits;
    if (bits) atomicOr(&s_bits[w], bits);
  }
  for (int e = tid; !dense && e < kTileRows * K; e += NT) {
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

  const int row = rw * 32 + rl;
  const bool row_ok = row < nrows;
  // a row's softmax statistics of head hh (max in log2 units, sum), merged
  // over the two key halves
  auto stats = [&](int hh) __attribute__((always_inline)) {
    const float2 s0 = s_st[hh * 64 + row], s1 = s_st[((p.G + 1) + hh) * 64 + row];
    const float mm = fmaxf(s0.x, s1.x);
    float ll = 0.f;
    if (mm > -INFINITY) {
      if (s0.x > -INFINITY) ll += s0.y * __builtin_amdgcn_exp2f(s0.x - mm);
      if (s1.x > -INFINITY) ll += s1.y * __builtin_amdgcn_exp2f(s1.x - mm);
    }
    return make_float2(mm, ll);
  };
  int lo = 0, hi = 0;
  if (row_ok) row_range(row, lo, hi);
  const int* my_ids = s_ids + (dense ? 0 : row * K);
  // the row's first kKlIdRegs filtered ids in registers (the slot search of
  // every stage then has no LDS round trip); slots past them are read from LDS
  constexpr int kKlIdRegs = 8;
  int id_reg[kKlIdRegs];
#pragma unroll
  for (int s = 0; s < kKlIdRegs; ++s) id_reg[s] = (!dense && s < K) ? my_ids[s] : -1;
  auto find_slot_of = [&](int c) __attribute__((always_inline)) {
    if (dense) return ((s_kb[row * nwk + (c >> 5)] >> (c & 31)) & 1u) ? c : -1;
    int found = -1;
#pragma unroll
    for (int s = kKlIdRegs - 1; s >= 0; --s) found = id_reg[s] == c ? s : found;   // first slot wins
    for (int s = kKlIdRegs; s < K && found < 0; ++s)
      if (my_ids[s] == c) found = s;
    return found;
  };

  // stages: pass 1 (hh, u) head-outer, pass 2 (u, hh) block-outer; hh == G is the student
  const int per_pass = (G + 1) * U;
  const int nstage = 2 * per_pass;
  // (hh, u) of stage i -> of stage i + 1 (counters instead of divisions by U)
  auto next_of = [&](int i, int& hh, int& u) {
    if (i + 1 < per_pass) {
      if (++u == U) {
        u = 0;
        ++hh;
      }
    } else if (i + 1 == per_pass) {
      hh = 0;
      u = 0;
    } else if (++hh == G + 1) {
      hh = 0;
      ++u;
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
  auto fetch = [&](int hh, int u, bool with_q) {
    int64_t st;
    const T* base = key_base(hh, st);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(base, (uint32_t)(((int64_t)(a.Sk - 1) * st + D) * 2));
    const uint32_t vo = (uint32_t)((tid / (D / 8)) * st + (tid % (D / 8)) * 8) * 2;
    const uint32_t so = (uint32_t)s_chunks[u] * kChunk * (uint32_t)st * 2u;
#pragma unroll
    for (int k = 0; k < PPT; ++k) kpre[k] = buffer_load16(rs, vo, so + (uint32_t)(k * RPP) * (uint32_t)st * 2u);
    // the query of a row past the tile end is row t0's (its keys are never kept)
    if (with_q) {
      const T* qr = q_row(hh);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) qpre[ks] = *reinterpret_cast<const uint4*>(qr + 16 * ks + 8 * h);
    }
  };

  float m_run = -INFINITY, l_run = 0.f;   // pass 1: this lane's keys of the current head
  float pacc[16];                         // pass 2: teacher p of this lane's 16 keys of the block
#pragma unroll
  for (int r = 0; r < 16; ++r) pacc[r] = 0.f;
  float kl_acc = 0.f;
  int slot = -1;
  uint64_t keep = 0ull;
  bool full = false;

  int hh_c = 0, u_c = 0;                 // stage i
  int hh_f = 0, u_f = 0;                 // stage i + 1, the next fetch
  if (nstage > 0) fetch(0, 0, true);
  next_of(0, hh_f, u_f);
  for (int i = 0; i < nstage; ++i) {
    const int hh = hh_c, u = u_c;
    const bool pass2 = i >= per_pass;
    __syncthreads();                       // previous stage's keys consumed
#pragma unroll
    for (int k = 0; k < PPT; ++k) *reinterpret_cast<uint4*>(sKw + k * RPP * KP) = kpre[k];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = qpre[ks];
    __syncthreads();
    // pass 1 runs head-outer: the query changes only with the head
    if (i + 1 < nstage) fetch(hh_f, u_f, i + 1 >= per_pass || u_f == 0);

    const int c = s_chunks[u];
    const int j0 = c * kChunk;
    if (!pass2 || hh == 0) {              // the row's slot of this block and its kept keys
      slot = find_slot_of(c);
      keep = (row_ok && slot >= 0) ? range64(min(max(lo - j0, 0), 64), min(max(hi - j0, 0), 64)) : 0ull;
      full = __all((uint32_t)(keep >> (32 * team)) == ~0u);   // every row keeps the team's half whole
    }
    f32x16_t st = zero16();
    __builtin_amdgcn_s_setprio(1);   // matrix work first; the other wave of the SIMD fills it with VALU
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      st = M::mac(*reinterpret_cast<const uint4*>(sK + (32 * team + rl) * KP + 16 * ks + 8 * h), qf[ks], st);
    __builtin_amdgcn_s_setprio(0);
    // logits in the reference's rounding: the product rounded to the input
    // dtype, the teacher's then scaled; key of register r:
    // 32 team + 8 (r / 4) + 4h + r % 4
    const float mul2 = (hh == G ? 1.f : a.scaling) * kLog2e;   // logits in log2 units
    const uint32_t kh = (uint32_t)(keep >> (32 * team + 4 * h));   // bit 8 (r / 4) + r % 4 <-> register r
    // two straight-line copies: every row of the wave keeps the whole block
    // (no per-key tests) / masked
    auto compute = [&](auto full_tag) __attribute__((always_inline)) {
      constexpr bool FULL = decltype(full_tag)::value;
      auto kept = [&](int bit) __attribute__((always_inline)) { return FULL || ((kh >> bit) & 1u) != 0; };
      if (!pass2) {
        float mloc = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float x = round_to<T>(st[r]) * mul2;
          st[r] = x;
          if (kept(8 * (r >> 2) + (r & 3))) mloc = fmaxf(mloc, x);
        }
        if (mloc > -INFINITY) {
          const float mn = fmaxf(m_run, mloc);
          float l = m_run > -INFINITY ? l_run * __builtin_amdgcn_exp2f(m_run - mn) : 0.f;
#pragma unroll
          for (int r = 0; r < 16; ++r)   // a masked key adds exp2(-inf) = 0 (no branch)
            l += __builtin_amdgcn_exp2f(kept(8 * (r >> 2) + (r & 3)) ? st[r] - mn : -INFINITY);
          m_run = mn;
          l_run = l;
        }
        if (u == U - 1) {                    // the head's statistics for the row: merge the lane pair
          const float mo = __shfl_xor(m_run, 32, kWave), lo2 = __shfl_xor(l_run, 32, kWave);
          const float mm = fmaxf(m_run, mo);
          float ll = 0.f;
          if (mm > -INFINITY) {
            if (m_run > -INFINITY) ll += l_run * __builtin_amdgcn_exp2f(m_run - mm);
            if (mo > -INFINITY) ll += lo2 * __builtin_amdgcn_exp2f(mo - mm);
          }
          if (h == 0) s_st[(team * (G + 1) + hh) * 64 + row] = make_float2(mm, ll);
          m_run = -INFINITY;
          l_run = 0.f;
        }
        return;
      }
      // pass 2
      const float2 ml = stats(hh);
      if (hh < G) {
        if (ml.y > 0.f) {
          // p = exp2(x - m) / l = exp2(x - (m + log2 l))
          const float c = ml.x + __builtin_amdgcn_logf(ml.y);
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const bool kp = kept(8 * (r >> 2) + (r & 3));
            pacc[r] += __builtin_amdgcn_exp2f(kp ? fmaf(round_to<T>(st[r]), mul2, -c) : -INFINITY);
          }
        }
        return;
      }
      // student: log-softmax, KL terms, dsel (4 keys per store); then the
      // next block starts from zero.  log via the hardware log2.
      const float lse2 = ml.y > 0.f ? ml.x + __builtin_amdgcn_logf(ml.y) : 0.f;   // log2 units
      const float invg = 1.f / (float)G;
      const bool wr = a.dsel && row_ok && slot >= 0;
      float* drow = wr ? a.dsel + ds_tile + (int64_t)(t0 + row) * a.ds_st + (int64_t)slot * kChunk : nullptr;
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        float dv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * r4 + e;
          const bool kp = kept(8 * r4 + e);
          const float pv = pacc[r] * invg;
          const float logq2 = fmaf(round_to<T>(st[r]), kLog2e, -lse2);
          const float lp2 = __builtin_amdgcn_logf(fmaxf(pv, 1e-12f));
          const float term = pv * (lp2 - logq2), d = __builtin_amdgcn_exp2f(logq2) - pv;
          kl_acc += kp ? term : 0.f;                               // log2 units
          dv[e] = kp ? d : 0.f;
          pacc[r] = 0.f;
        }
        if (wr) *reinterpret_cast<float4*>(drow + 32 * team + 8 * r4 + 4 * h) = make_float4(dv[0], dv[1], dv[2], dv[3]);
      }
    };
    if (full)
      compute(std::true_type{});
    else
      compute(std::false_type{});
    hh_c = hh_f;
    u_c = u_f;
    next_of(i + 1, hh_f, u_f);
  }

  // the row's KL: the lane pair, then the two key halves (team 0 writes)
  const float kl_half = (kl_acc + __shfl_xor(kl_acc, 32, kWave)) * kLn2;
  if (team == 1 && h == 0) s_kl[row] = kl_half;
  __syncthreads();
  if (team == 0 && row_ok && h == 0) {
    const float kl_row = kl_half + s_kl[row];
    const float2 sst = U > 0 ? stats(G) : make_float2(-INFINITY, 0.f);
    const bool valid = sst.y > 0.f;
    a.kl[(int64_t)b * a.kl_sb + (int64_t)ih * a.kl_sh + t0 + row] = valid ? kl_row : 0.f;
    a.valid[(int64_t)b * a.va_sb + (int64_t)ih * a.va_sh + t0 + row] = valid ? 1 : 0;
  }
}

// -------------------------------------------------------------- row-sparse forward
// Rows that select unrelated blocks (per-row top-k, as the indexer's own
// selections are) give a 64-row tile a block union near the whole prefix, and
// the tile kernel would spend most of its work on (row, block) pairs that no
// row of the pair keeps.  Tiles whose union exceeds K blocks (rows that do not
// all share one selection) are flagged on the device and taken block-major: for every key block, the rows of flagged
// tiles that selected it are gathered 64 at a time, so each (row, block) pair
// is computed once.
//   kl_rs_flag_kernel    per tile: the union size and the flag; for a flagged
//                        tile, bit t of block c's row bitmap for every kept
//                        (row t, block c) pair;
//   kl_rs_pass_kernel    per (block, 2048-row window), over the same row groups
//                        twice: STATS writes each pair's (max, sum) per head,
//                        MIX (after the combine) mixes the teacher over the
//                        heads, takes the student's log-softmax and writes the
//                        pair's KL sum and its dsel row;
//   kl_rs_combine_kernel per (row, head): the pairs' statistics merged in slot
//                        order; dsel zeroed for slots with nothing kept;
//   kl_rs_final_kernel   per row: the KL as the sum of its pairs in slot order.
// Every (row, slot) pair writes its own records, so no result depends on how
// the rows are grouped.
constexpr int kRsRange = 2048;   // row window of a block-major workgroup (64 bitmap words)
constexpr int kRsWin = 2048;     // rows per window of the dK scan (64 bitmap words)

struct KlRsK {
  srswa_kl_args a;
  int ntiles, nblk, nwords, rwords, nrange, G, KV;
  int per_xcd;        // block-major workgroups per XCD
  uint32_t* flag;     // [B, HI, ntiles]
  uint32_t* rbm;      // [B, HI, nblk, rwords] rows of flagged tiles per block
  float2* srec;       // [B, HI, T, K, G + 1] per pair and head: (max in log2 units, sum)
  float2* rst;        // [B, HI, T, G + 1] per row and head: merged (max, sum)
  float* klp;         // [B, HI, T, K] per pair: sum of the KL terms (log2 units)
};

// The row's kept key range [lo, hi): its sample start to the window start.
__device__ __forceinline__ void kl_row_range(const srswa_kl_args& a, int b, int t, int& lo, int& hi) {
  const int pos = a.pos[(int64_t)b * a.pos_sb + t];
  lo = a.seg ? a.seg[(int64_t)b * a.seg_sb + t] : 0;
  hi = min(max(pos - a.local_window + 1, 0), a.Sk);
}

// Block id of slot s of row t when it holds kept keys and is the id's first
// slot (a repeated id counts once), else -1.  With slots_are_blocks (dense)
// slot s holds block s exactly when ids[s] == s (no repeats to look for).
__device__ __forceinline__ int kl_slot_block(const int32_t* ids, int s, int lo, int hi, bool dense = false) {
  int id = ids[s];
  if (dense && id != s) return -1;
  if (id < 0 || (int64_t)id * kChunk >= hi || (int64_t)id * kChunk + kChunk <= lo) return -1;
  if (!dense)
    for (int s2 = 0; s2 < s; ++s2)
      if (ids[s2] == id) return -1;
  return id;
}

__device__ __forceinline__ const int32_t* kl_row_ids(const srswa_kl_args& a, int b, int ih, int t) {
  return a.sel + (int64_t)b * a.sel_sb + (int64_t)ih * a.sel_sh + (int64_t)t * a.sel_st;
}

// Rows of one window of NW bitmap words (32 NW rows) of a block's row bitmap,
// ascending, as offsets from the window's first row (lanes < NW of wave 0 one
// word each); returns the count.  Every thread of the workgroup calls it.
template <int NW>
__device__ __forceinline__ int window_rows(const uint32_t* words, int w0, int rwords, uint16_t* s_rows, int* s_n) {
  static_assert(NW <= kWave, "one word per lane of wave 0");
  const int tid = threadIdx.x, lane = tid % kWave;
  if (tid < kWave) {
    const int w = w0 + lane;
    const uint32_t bits = (lane < NW && w < rwords) ? words[w] : 0u;
    const int cnt = __popc(bits);
    int incl = cnt;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int v = __shfl_up(incl, o, kWave);
      if (lane >= o) incl += v;
    }
    int pos = incl - cnt;
    uint32_t bb = bits;
    while (bb) {
      const int bit = __ffs(bb) - 1;
      bb &= bb - 1;
      s_rows[pos++] = (uint16_t)(lane * 32 + bit);
    }
    if (lane == kWave - 1) *s_n = incl;
  }
  __syncthreads();
  return *s_n;
}

// Bits of a 64-row tile's (block, row) pairs into row bitmaps: per block of the
// tile's union (s_chunks, U entries), one wave ballots the rows whose kept ids
// (s_ids, -1 = none) include it and ORs the two 32-row words once.
__device__ __forceinline__ void tile_row_bits(const int* s_ids, int K, bool dense, int nrows, const uint16_t* s_chunks,
                                              int U, uint32_t* bm0, uint32_t* bm1, int rwords, int tile) {
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave, nw = blockDim.x / kWave;
  const int nwk = (K + 31) >> 5;
  for (int u = wave; u < U; u += nw) {
    const int c = s_chunks[u];
    bool mine = false;
    if (lane < nrows && dense)     // s_ids: per-row bitmaps of the listed blocks (slot = block)
      mine = (reinterpret_cast<const uint32_t*>(s_ids)[lane * nwk + (c >> 5)] >> (c & 31)) & 1u;
    else if (lane < nrows)
      for (int s = 0; s < K; ++s) mine = mine || s_ids[lane * K + s] == c;
    const uint64_t m = __ballot(mine);
    if (lane < 2) {
      const uint32_t w = (uint32_t)(m >> (32 * lane));
      const int64_t at = (int64_t)c * rwords + 2 * tile + lane;
      if (w && 2 * tile + lane < rwords) {
        atomicOr(&bm0[at], w);
        if (bm1) atomicOr(&bm1[at], w);
      }
    }
  }
}

__global__ __launch_bounds__(256) void kl_rs_flag_kernel(KlRsK p) {
  // LDS: [nwords] union bits, [1] count, [64 K] kept ids, [1] list length,
  // then the union as a block list
  extern __shared__ uint32_t s_u[];
  const srswa_kl_args& a = p.a;
  const int tile = (int)(blockIdx.x % p.ntiles);
  const int bh = (int)(blockIdx.x / p.ntiles);
  const int ih = bh % a.HI, b = bh / a.HI;
  const int t0 = tile * kTileRows, nrows = min(kTileRows, a.T - t0);
  const int K = a.K, tid = threadIdx.x;
  uint32_t* s_bits = s_u;
  uint32_t* s_cnt = s_u + p.nwords;
  int* s_ids = reinterpret_cast<int*>(s_u + p.nwords + 1);
  // with slots_are_blocks the ids region holds [64][ceil(K / 32)] bitmaps of
  // the kept blocks
  const bool dense = a.slots_are_blocks != 0;
  const int nwk = (K + 31) >> 5;
  int* s_len = s_ids + kTileRows * (dense ? nwk : K);
  uint16_t* s_chunks = reinterpret_cast<uint16_t*>(s_len + 1);
  for (int w = tid; w <= p.nwords; w += blockDim.x) s_u[w] = 0u;
  __syncthreads();
  for (int e = tid; dense && e < kTileRows * nwk; e += blockDim.x) {
    const int r = e / nwk, w = e % nwk;
    uint32_t bits = 0u;
    if (r < nrows) {
      int lo, hi;
      kl_row_range(a, b, t0 + r, lo, hi);
      const int32_t* ids = kl_row_ids(a, b, ih, t0 + r);
      for (int j = 0; j < 32; ++j) {
        const int s = 32 * w + j;
        if (s >= K) break;
        if (kl_slot_block(ids, s, lo, hi, true) >= 0) {
          bits |= 1u << j;
        } else if (ids[s] == s && a.dsel) {          // listed, nothing kept: a zero dsel row
          float4* z = reinterpret_cast<float4*>(a.dsel + (int64_t)b * a.ds_sb + (int64_t)ih * a.ds_sh +
                                                (int64_t)(t0 + r) * a.ds_st + (int64_t)s * kChunk);
#pragma unroll
          for (int i = 0; i < kChunk / 4; ++i) z[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
    }
    reinterpret_cast<uint32_t*>(s_ids)[e] = bits;
    if (bits) atomicOr(&s_bits[w], bits);
  }
  for (int e = tid; !dense && e < kTileRows * K; e += blockDim.x) {
    const int r = e / K, s = e % K;
    int id = -1;
    if (r < nrows) {
      int lo, hi;
      kl_row_range(a, b, t0 + r, lo, hi);
      id = kl_slot_block(kl_row_ids(a, b, ih, t0 + r), s, lo, hi);
      if (id >= 0) atomicOr(&s_bits[id >> 5], 1u << (id & 31));
    }
    s_ids[e] = id;
  }
  __syncthreads();
  for (int w = tid; w < p.nwords; w += blockDim.x) atomicAdd(s_cnt, (uint32_t)__popc(s_bits[w]));
  __syncthreads();
  // slot = block: the host runs these kernels only when every tile goes
  // block-major (too few tiles to fill the chip)
  const bool rs = dense || (int)*s_cnt > K;
  if (tid == 0) p.flag[(int64_t)bh * p.ntiles + tile] = rs ? 1u : 0u;
  if (!rs) return;                                    // uniform: no barrier below is skipped by part of the group
  const int U = compact_bitmap(s_bits, p.nwords, s_chunks, s_len);
  tile_row_bits(s_ids, K, dense, nrows, s_chunks, U, p.rbm + (int64_t)bh * p.nblk * p.rwords, nullptr, p.rwords,
                tile);
}

// One workgroup per (sequence, index head, block c, 2048-row window): the
// window's rows that selected c, ascending, two waves.  Logical order: window
// major, block fastest, dealt to the XCDs in contiguous runs, so the workgroups
// on one XCD gather query rows of the same windows from its L2.
// of 32 rows per group of 64 (lane = row, S^T = K Q^T over the block's 64
// keys as in the tile kernel).  Stage (group, head): K of the head's block
// staged in LDS, the rows' query fragments in registers, both fetched one
// stage ahead.
template <typename T, int D, bool MIX>
__global__ __launch_bounds__(128, 2) void kl_rs_pass_kernel(KlRsK p) {
  using M = Mfma<T>;
  using L = KlLds<D>;
  constexpr int KP = L::KP, KS = D / 16, NT = 128;
  constexpr int PPT = kChunk * D / 8 / NT;
  constexpr int RPP = NT / (D / 8);
  __shared__ __align__(16) T sK[kChunk * KP];
  __shared__ uint16_t s_rows[kRsRange];             // the window's rows of block c, offsets from its first
  __shared__ int s_n;
  // MIX: the student's log q (log2 units) of the group's rows, [row][key] with
  // a 68-float pitch (conflict-free 16-byte accesses)
  constexpr int LQP = 68;
  __shared__ __align__(16) float s_lq[MIX ? kTileRows * LQP : 4];
  const srswa_kl_args& a = p.a;
  const int64_t lid = (int64_t)(blockIdx.x & 7) * p.per_xcd + (blockIdx.x >> 3);
  if (lid >= (int64_t)a.B * a.HI * p.nrange * p.nblk) return;
  const int c = (int)(lid % p.nblk);
  const int range = (int)((lid / p.nblk) % p.nrange);
  const int bh = (int)(lid / ((int64_t)p.nblk * p.nrange));
  const int ih = bh % a.HI, b = bh / a.HI;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int h = lane >> 5, rl = lane & 31;
  const int G = p.G, K = a.K;
  const int j0 = c * kChunk;

  // the window's rows of block c, ascending
  const int r0 = range * kRsRange;
  const int n = window_rows<kRsRange / 32>(p.rbm + ((int64_t)bh * p.nblk + c) * p.rwords, range * (kRsRange / 32),
                                           p.rwords, s_rows, &s_n);
  if (n == 0) return;
  const int ngroups = (n + kTileRows - 1) / kTileRows;
  const int nst = ngroups * (G + 1);
  const int row = wave * 32 + rl;                    // row of the group this lane owns
  // head of a stage's position j in its group: the student first (its log q
  // is parked in LDS), then the teachers; the last teacher forms the terms
  auto head_of = [&](int j) { return j == 0 ? G : j - 1; };

  auto key_base = [&](int hh, int64_t& st) -> const T* {
    if (hh == G) {
      st = a.ik_st;
      return reinterpret_cast<const T*>(a.idx_k) + (int64_t)b * a.ik_sb;
    }
    const int kvh = (ih * G + hh) / p.KV;
    st = a.km_st;
    return reinterpret_cast<const T*>(a.k_main) + (int64_t)b * a.km_sb + (int64_t)kvh * a.km_sh;
  };
  // the row of group g this lane owns, or -1 past the list (it then reads
  // row s_rows[0]'s query and keeps nothing)
  auto group_row = [&](int g) { const int i = g * kTileRows + row; return i < n ? r0 + (int)s_rows[i] : -1; };
  auto q_row = [&](int hh, int t) -> const T* {
    const int tt = t >= 0 ? t : r0 + (int)s_rows[0];
    if (hh == G)
      return reinterpret_cast<const T*>(a.q_idx) + (int64_t)b * a.qi_sb + (int64_t)ih * a.qi_sh + (int64_t)tt * a.qi_st;
    return reinterpret_cast<const T*>(a.q_main) + (int64_t)b * a.qm_sb + (int64_t)(ih * G + hh) * a.qm_sh +
           (int64_t)tt * a.qm_st;
  };
  T* sKw = sK + (tid / (D / 8)) * KP + (tid % (D / 8)) * 8;
  uint4 kpre[PPT], qpre[KS], qf[KS];
  auto fetch = [&](int i) {
    const int g = i / (G + 1), hh = head_of(i % (G + 1));
    int64_t st;
    const T* base = key_base(hh, st);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(base, (uint32_t)(((int64_t)(a.Sk - 1) * st + D) * 2));
    const uint32_t vo = (uint32_t)((tid / (D / 8)) * st + (tid % (D / 8)) * 8) * 2;
    const uint32_t so = (uint32_t)j0 * (uint32_t)st * 2u;
#pragma unroll
    for (int k = 0; k < PPT; ++k) kpre[k] = buffer_load16(rs, vo, so + (uint32_t)(k * RPP) * (uint32_t)st * 2u);
    const T* qr = q_row(hh, group_row(g));
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qpre[ks] = *reinterpret_cast<const uint4*>(qr + 16 * ks + 8 * h);
  };

  const int64_t rowbase = (int64_t)bh * a.T;       // (b, ih) row offset of the per-row records
  int t = -1, slot = -1;
  uint64_t keep = 0ull;
  float pacc[32];
  fetch(0);
  for (int i = 0; i < nst; ++i) {
    const int g = i / (G + 1), j = i % (G + 1), hh = head_of(j);
    __syncthreads();                                  // the previous stage's keys consumed
#pragma unroll
    for (int k = 0; k < PPT; ++k) *reinterpret_cast<uint4*>(sKw + k * RPP * KP) = kpre[k];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = qpre[ks];
    __syncthreads();
    if (i + 1 < nst) fetch(i + 1);
    if (j == 0) {                                     // a new group: the lane's row, slot and kept keys
      t = group_row(g);
      slot = -1;
      keep = 0ull;
      if (t >= 0) {
        int lo, hi;
        kl_row_range(a, b, t, lo, hi);
        const int32_t* ids = kl_row_ids(a, b, ih, t);
        if (a.slots_are_blocks) slot = c;           // the bitmap holds kept pairs
        for (int s = 0; s < K && slot < 0; ++s)
          if (ids[s] == c) slot = s;                  // the first slot holding c (the bitmap holds kept pairs)
        keep = range64(min(max(lo - j0, 0), 64), min(max(hi - j0, 0), 64));
      }
      if constexpr (MIX) {
#pragma unroll
        for (int r = 0; r < 32; ++r) pacc[r] = 0.f;
      }
    }
    f32x16_t st[2] = {zero16(), zero16()};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
        st[kh] = M::mac(*reinterpret_cast<const uint4*>(sK + (32 * kh + rl) * KP + 16 * ks + 8 * h), qf[ks], st[kh]);
    }
    // logits in the reference's rounding, in log2 units; register r of key
    // half kh is key 32 kh + 8 (r / 4) + 4h + r % 4
    const float mul2 = (hh == G ? 1.f : a.scaling) * kLog2e;
    // logit of element r (0..31) of the lane: -inf where the key is not kept
    auto xat = [&](int r) __attribute__((always_inline)) {
      const int kh = r >> 4, rr = r & 15;
      const int key = 32 * kh + 8 * (rr >> 2) + 4 * h + (rr & 3);
      return ((keep >> key) & 1ull) ? round_to<T>(st[kh][rr]) * mul2 : -INFINITY;
    };
    if constexpr (!MIX) {
      float x[32];
#pragma unroll
      for (int r = 0; r < 32; ++r) x[r] = xat(r);
      float m = -INFINITY;
#pragma unroll
      for (int r = 0; r < 32; ++r) m = fmaxf(m, x[r]);
      m = fmaxf(m, __shfl_xor(m, 32, kWave));
      float l = 0.f;
      if (m > -INFINITY) {
#pragma unroll
        for (int r = 0; r < 32; ++r) l += __builtin_amdgcn_exp2f(x[r] - m);   // a masked key adds 0
      }
      l += __shfl_xor(l, 32, kWave);
      if (t >= 0 && h == 0) p.srec[((rowbase + t) * K + slot) * (G + 1) + hh] = make_float2(m, l);
    } else {
      const float2 ml = t >= 0 ? p.rst[(rowbase + t) * (G + 1) + hh] : make_float2(-INFINITY, 0.f);
      float* lq = s_lq + row * LQP;
      if (hh == G) {
        // student: log q (log2 units) of the lane's keys into LDS, 4 keys per store
        const float lse2 = ml.y > 0.f ? ml.x + __builtin_amdgcn_logf(ml.y) : 0.f;
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = xat(16 * kh + 4 * r4 + e) - lse2;
            *reinterpret_cast<float4*>(lq + 32 * kh + 8 * r4 + 4 * h) = make_float4(v[0], v[1], v[2], v[3]);
          }
      } else if (ml.y > 0.f) {
        const float cc = ml.x + __builtin_amdgcn_logf(ml.y);    // p = exp2(x - (m + log2 l))
#pragma unroll
        for (int r = 0; r < 32; ++r) pacc[r] += __builtin_amdgcn_exp2f(xat(r) - cc);
      }
      if (j == G) {
        // the group's last teacher: the pair's KL terms and its dsel row
        const float invg = 1.f / (float)G;
        float kl_acc = 0.f;
        float* drow = (a.dsel && t >= 0)
                          ? a.dsel + (int64_t)b * a.ds_sb + (int64_t)ih * a.ds_sh + (int64_t)t * a.ds_st +
                                (int64_t)slot * kChunk
                          : nullptr;
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
            const float4 q4 = *reinterpret_cast<const float4*>(lq + 32 * kh + 8 * r4 + 4 * h);
            const float lqv[4] = {q4.x, q4.y, q4.z, q4.w};
            float dv[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int r = 16 * kh + 4 * r4 + e;
              const int key = 32 * kh + 8 * r4 + 4 * h + e;
              const bool kp = (keep >> key) & 1ull;
              const float pv = pacc[r] * invg;
              const float logq2 = lqv[e];
              const float lp2 = __builtin_amdgcn_logf(fmaxf(pv, 1e-12f));
              const float term = pv * (lp2 - logq2), d = __builtin_amdgcn_exp2f(logq2) - pv;
              kl_acc += kp ? term : 0.f;
              dv[e] = kp ? d : 0.f;
            }
            if (drow) *reinterpret_cast<float4*>(drow + 32 * kh + 8 * r4 + 4 * h) = make_float4(dv[0], dv[1], dv[2], dv[3]);
          }
        kl_acc += __shfl_xor(kl_acc, 32, kWave);
        if (t >= 0 && h == 0) p.klp[(rowbase + t) * K + slot] = kl_acc;
      }
    }
  }
}

// Per (row, head) of a flagged tile: the head's statistics merged over the
// row's kept slots in slot order; the head-0 thread also zeroes the dsel rows
// of slots with nothing kept (with slots_are_blocks the flag kernel does).
__global__ __launch_bounds__(256) void kl_rs_combine_kernel(KlRsK p) {
  const srswa_kl_args& a = p.a;
  const int G1 = p.G + 1;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)a.B * a.HI * a.T * G1) return;
  const int hh = (int)(gid % G1);
  const int64_t rowi = gid / G1;                   // (b, ih, t) row index
  const int t = (int)(rowi % a.T);
  const int bh = (int)(rowi / a.T);
  const int ih = bh % a.HI, b = bh / a.HI;
  if (!p.flag[(int64_t)bh * p.ntiles + t / kTileRows]) return;
  const int K = a.K;
  const bool dense = a.slots_are_blocks != 0;
  int lo, hi;
  kl_row_range(a, b, t, lo, hi);
  const int32_t* ids = kl_row_ids(a, b, ih, t);
  // the kept slots: a bitmap (at most 64 slots), or with slots_are_blocks the
  // constant-time test of the slot itself
  // (dense: kl_rs_flag_kernel zeroes the dsel rows of listed slots with
  // nothing kept)
  uint64_t live = 0ull;
  for (int s = 0; s < K && !dense; ++s) {
    if (kl_slot_block(ids, s, lo, hi) >= 0) {
      live |= 1ull << s;
    } else if (hh == 0 && a.dsel) {
      float4* z = reinterpret_cast<float4*>(a.dsel + (int64_t)b * a.ds_sb + (int64_t)ih * a.ds_sh +
                                            (int64_t)t * a.ds_st + (int64_t)s * kChunk);
#pragma unroll
      for (int i = 0; i < kChunk / 4; ++i) z[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  auto is_live = [&](int s) { return dense ? kl_slot_block(ids, s, lo, hi, true) >= 0 : ((live >> s) & 1ull) != 0; };
  // dense: only the blocks of the row's kept key range can be live
  const int s0 = dense ? lo / kChunk : 0, s1 = dense ? min(K, (hi + kChunk - 1) / kChunk) : K;
  const float2* rec = p.srec + rowi * K * G1 + hh;
  float mm = -INFINITY;
  for (int s = s0; s < s1; ++s)
    if (is_live(s)) mm = fmaxf(mm, rec[s * G1].x);
  float ll = 0.f;
  if (mm > -INFINITY)
    for (int s = s0; s < s1; ++s)
      if (is_live(s)) {
        const float2 v = rec[s * G1];                // a second read, from cache
        if (v.x > -INFINITY) ll += v.y * __builtin_amdgcn_exp2f(v.x - mm);
      }
  p.rst[rowi * G1 + hh] = make_float2(mm, ll);
}

// Per row of a flagged tile: kl = the sum of its pairs' KL sums in slot order.
__global__ __launch_bounds__(256) void kl_rs_final_kernel(KlRsK p) {
  const srswa_kl_args& a = p.a;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)a.B * a.HI * a.T) return;
  const int t = (int)(gid % a.T);
  const int bh = (int)(gid / a.T);
  const int ih = bh % a.HI, b = bh / a.HI;
  if (!p.flag[(int64_t)bh * p.ntiles + t / kTileRows]) return;
  int lo, hi;
  kl_row_range(a, b, t, lo, hi);
  const int32_t* ids = kl_row_ids(a, b, ih, t);
  float kl = 0.f;
  const bool dense = a.slots_are_blocks != 0;   // only the blocks of the kept key range can hold a pair
  const int s0 = dense ? lo / kChunk : 0, s1 = dense ? min(a.K, (hi + kChunk - 1) / kChunk) : a.K;
  for (int s = s0; s < s1; ++s)
    if (kl_slot_block(ids, s, lo, hi, dense) >= 0) kl += p.klp[gid * a.K + s];
  const bool valid = p.rst[gid * (p.G + 1) + p.G].y > 0.f;
  a.kl[(int64_t)b * a.kl_sb + (int64_t)ih * a.kl_sh + t] = valid ? kl * kLn2 : 0.f;
  a.valid[(int64_t)b * a.va_sb + (int64_t)ih * a.va_sh + t] = valid ? 1 : 0;
}

// -------------------------------------------------------------- backward
// Tile products on the matrix cores with ds = rnd(g * dsel) (the reference's
// bf16 gradient of the logits) staged in LDS.  kl_bwd_flag_kernel first
// marks, per 64-row tile, whether its rows' selected blocks form a union of
// more than K blocks (rows that do not share one selection) and fills two row
// bitmaps per block: every row that selected it, and those of flagged tiles.
//   dq_kernel:    per (sequence, index head, 64-row tile) not flagged, over
//                 the tile's selected blocks: dQ[rows, d] += DS[rows, keys] K[keys, d];
//   rs_dq_kernel: per (sequence, index head, block, 2048-row range), the
//                 flagged rows that selected the block, 64 at a time: each
//                 (row, slot) pair's product DS K written as an fp32 partial,
//                 then summed per row in slot order (rs_dq_reduce_kernel);
//   dk_kernel:    per (sequence, block, 2048-row window), the window's rows
//                 that selected the block, ascending, 64 at a time:
//                 dK[keys, d] += DS^T[keys, rows] Q[rows, d] as an fp32
//                 partial; dk_reduce_kernel sums the windows in order
//                 (deterministic).
// Four waves; wave w owns output tiles (w / TPW halves of 32 rows / keys,
// 32-wide head-dim slices); K and Q rows are read as B operands with
// ds_read_b64_tr_b16 from their natural layout.
constexpr int kBwdThreads = 256;

struct KlBwdK {
  srswa_kl_bwd_args a;
  int ntiles, nblk, nwords, rwords, nrange;
  int per_xcd;              // rs_dq workgroups per XCD (window major, block fastest)
  uint32_t* flag;           // [B, HI, ntiles]: rows of the tile taken by rs_dq_kernel
  uint32_t* rbm;            // [B, HI, nblk, rwords] rows of flagged tiles per block
  uint32_t* rbm_all;        // [B, HI, nblk, rwords] every row per block
  float* dqp;               // [B, HI, T, K, D] per (row, slot): dQ partial of a flagged row
  float* dkp;               // [B, nblk, nwin, 64, D] per (block, 2048-row window): dK partial
  uint32_t* dkw;            // [B, nblk, nwin]: the window wrote a partial
  int nwin;
};

template <int D> struct KlBwdLds {
  static constexpr int XP = D + 16;          // K / Q rows: conflict-free transposing reads
  static constexpr int SP = kChunk + 8;      // DS rows: 16-byte row reads
  static constexpr int dsOff = kChunk * XP * 2;
  static constexpr int bytes = dsOff + 64 * SP * 2;
};

// the slot of block c among row (b, ih, t)'s ids (first occurrence), -1 if
// none; with slots_are_blocks slot c itself when the row lists block c
__device__ __forceinline__ int find_slot(const srswa_kl_bwd_args& a, int b, int ih, int t, int c) {
  const int32_t* ids = a.sel + (int64_t)b * a.sel_sb + (int64_t)ih * a.sel_sh + (int64_t)t * a.sel_st;
  if (a.slots_are_blocks) return (c < a.K && ids[c] == c) ? c : -1;
  for (int s = 0; s < a.K; ++s)
    if (ids[s] == c) return s;
  return -1;
}

// The B operand comes from a_operand_tr, whose lane half h holds the 16-row
// group's rows 4h .. 4h + 3 and 8 + 4h .. 8 + 4h + 3 (the MFMA output order);
// the A operand read as 8 contiguous values from LDS must list its k index in
// that same order, so DS is staged with element x of each 16-group at
// position slot_of_key(x): bits 2 and 3 swapped.
__device__ __forceinline__ int slot_of_key(int x) { return (x & ~12) | ((x & 4) << 1) | ((x & 8) >> 1); }

// 16 values ds = rnd(g * dsel[t, slot, k0 .. k0 + 15]) (zeros without a slot)
template <typename T>
__device__ __forceinline__ void ds16(const srswa_kl_bwd_args& a, int b, int ih, int t, int slot, int k0,
                                     float* out) {
  if (slot < 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) out[i] = 0.f;
    return;
  }
  const float g = a.grad[(int64_t)b * a.g_sb + (int64_t)ih * a.g_sh + t];
  const float4* src = reinterpret_cast<const float4*>(a.dsel + (int64_t)b * a.ds_sb + (int64_t)ih * a.ds_sh +
                                                      (int64_t)t * a.ds_st + (int64_t)slot * kChunk + k0);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 v = src[i];
    out[4 * i] = round_to<T>(g * v.x);
    out[4 * i + 1] = round_to<T>(g * v.y);
    out[4 * i + 2] = round_to<T>(g * v.z);
    out[4 * i + 3] = round_to<T>(g * v.w);
  }
}

// 64 rows of D elements (row r at base + r * st, rows >= n zero) into LDS
template <typename T, int D>
__device__ __forceinline__ void stage_rows(T* dst, const T* base, int64_t st, int n) {
  constexpr int XP = KlBwdLds<D>::XP;
  constexpr int PR = D / 8;                       // 16-byte pieces per row
  for (int e = threadIdx.x; e < 64 * PR; e += kBwdThreads) {
    const int r = e / PR, c = (e % PR) * 8;
    const uint4 v = r < n ? *reinterpret_cast<const uint4*>(base + (int64_t)r * st + c) : make_uint4(0, 0, 0, 0);
    *reinterpret_cast<uint4*>(dst + r * XP + c) = v;
  }
}

__global__ __launch_bounds__(256) void kl_zero_kernel(uint32_t* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

template <typename T, int D>
__device__ __forceinline__ void store_tiles(T* base, int64_t st, int nvalid, const f32x16_t* acc, int wave,
                                            int lane) {
  // acc[i] = output tile (rows / keys half = i0 >> ..., dims 32 * dt): see the callers' mapping
  constexpr int MT = D / 32;
  constexpr int TPW = 2 * MT / 4;                 // output tiles per wave
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int tix = wave * TPW + i;
    const int half = tix / MT, dt = tix % MT;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = 32 * half + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      if (m < nvalid) {
        const uint32_t w = Mfma<T>::pack2(acc[i][r], 0.f);
        *reinterpret_cast<uint16_t*>(base + (int64_t)m * st + 32 * dt + (lane & 31)) = (uint16_t)(w & 0xffffu);
      }
    }
  }
}

template <typename T, int D>
__global__ __launch_bounds__(kBwdThreads) void kl_dq_kernel(KlBwdK p) {
  using M = Mfma<T>;
  using L = KlBwdLds<D>;
  constexpr int XP = L::XP, SP = L::SP, MT = D / 32, TPW = 2 * MT / 4;
  extern __shared__ __align__(16) unsigned char smem[];
  T* sK = reinterpret_cast<T*>(smem);
  T* sDS = reinterpret_cast<T*>(smem + L::dsOff);
  __shared__ uint32_t s_bits[64];
  __shared__ uint16_t s_chunks[64 * 64];
  __shared__ int s_count;
  const srswa_kl_bwd_args& a = p.a;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int tile = blockIdx.x % p.ntiles;
  const int bh = blockIdx.x / p.ntiles;
  if (p.flag[(int64_t)bh * p.ntiles + tile]) return;   // rs_dq_kernel takes the tile's rows
  const int ih = bh % a.HI, b = bh / a.HI;
  const int t0 = tile * kTileRows;
  const int nrows = min(kTileRows, a.T - t0);
  // the tile's selected blocks (rows with a nonzero gradient)
  const int nwords = p.nwords;
  for (int w = tid; w < nwords; w += kBwdThreads) s_bits[w] = 0u;
  __syncthreads();
  for (int e = tid; e < nrows * a.K; e += kBwdThreads) {
    const int r = e / a.K, s = e % a.K;
    const int id = a.sel[(int64_t)b * a.sel_sb + (int64_t)ih * a.sel_sh + (int64_t)(t0 + r) * a.sel_st + s];
    if (id >= 0 && id < p.nblk && (!a.slots_are_blocks || id == s)) atomicOr(&s_bits[id >> 5], 1u << (id & 31));
  }
  __syncthreads();
  const int U = compact_bitmap(s_bits, nwords, s_chunks, &s_count);

  f32x16_t acc[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i) acc[i] = zero16();
  const uint16_t* k16 = reinterpret_cast<const uint16_t*>(sK);
  const int rr = tid / 4, kq = (tid % 4) * 16;    // DS staging: row, 16-key quarter
  for (int u = 0; u < U; ++u) {
    const int c = s_chunks[u];
    __syncthreads();
    stage_rows<T, D>(sK, reinterpret_cast<const T*>(a.idx_k) + (int64_t)b * a.ik_sb + (int64_t)c * kChunk * a.ik_st,
                     a.ik_st, min(kChunk, a.Sk - c * kChunk));
    {
      float v[16];
      const int slot = rr < nrows ? find_slot(a, b, ih, t0 + rr, c) : -1;
      ds16<T>(a, b, ih, t0 + rr, slot, kq, v);
      // keys in the transposing read's order (slot_of_key): 0-3, 8-11 | 4-7, 12-15
      uint4 w0, w1;
      w0 = make_uint4(M::pack2(v[0], v[1]), M::pack2(v[2], v[3]), M::pack2(v[8], v[9]), M::pack2(v[10], v[11]));
      w1 = make_uint4(M::pack2(v[4], v[5]), M::pack2(v[6], v[7]), M::pack2(v[12], v[13]), M::pack2(v[14], v[15]));
      *reinterpret_cast<uint4*>(sDS + rr * SP + kq) = w0;
      *reinterpret_cast<uint4*>(sDS + rr * SP + kq + 8) = w1;
    }
    __syncthreads();
    // dQ[row, d] += DS[row, key] K[key, d]: A = DS rows, B = K via transposing reads
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int i = 0; i < TPW; ++i) {
        const int tix = wave * TPW + i;
        const int half = tix / MT, dt = tix % MT;
        const uint4 av = *reinterpret_cast<const uint4*>(sDS + (32 * half + (lane & 31)) * SP + 16 * ks + 8 * (lane >> 5));
        acc[i] = M::mac(av, a_operand_tr<XP>(k16, 16 * ks, 32 * dt, lane), acc[i]);
      }
    }
  }
  store_tiles<T, D>(reinterpret_cast<T*>(a.dq_idx) + (int64_t)b * a.dq_sb + (int64_t)ih * a.dq_sh +
                        (int64_t)t0 * a.dq_st,
                    a.dq_st, nrows, acc, wave, lane);
}

// Per (sequence, index head, 64-row tile): the union of the rows' selected
// blocks (0 <= id < nblk, an id's first slot) and the flag; a bit per (block,
// row) pair in the all-rows bitmap, and in the flagged-rows bitmap for a
// flagged tile.
__global__ __launch_bounds__(256) void kl_bwd_flag_kernel(KlBwdK p) {
  // LDS as kl_rs_flag_kernel's
  extern __shared__ uint32_t s_u[];
  const srswa_kl_bwd_args& a = p.a;
  const int tile = (int)(blockIdx.x % p.ntiles);
  const int bh = (int)(blockIdx.x / p.ntiles);
  const int ih = bh % a.HI, b = bh / a.HI;
  const int t0 = tile * kTileRows, nrows = min(kTileRows, a.T - t0);
  const int K = a.K, tid = threadIdx.x;
  uint32_t* s_bits = s_u;
  uint32_t* s_cnt = s_u + p.nwords;
  int* s_ids = reinterpret_cast<int*>(s_u + p.nwords + 1);
  // with slots_are_blocks the ids region holds [64][ceil(K / 32)] bitmaps
  int* s_len = s_ids + kTileRows * (a.slots_are_blocks ? (K + 31) >> 5 : K);
  uint16_t* s_chunks = reinterpret_cast<uint16_t*>(s_len + 1);
  for (int w = tid; w <= p.nwords; w += blockDim.x) s_u[w] = 0u;
  __syncthreads();
  const bool dense = a.slots_are_blocks != 0;
  const int nwk = (K + 31) >> 5;
  // slot = block: per-row bitmaps of the listed blocks in place of the ids
  for (int e = tid; dense && e < kTileRows * nwk; e += blockDim.x) {
    const int r = e / nwk, w = e % nwk;
    uint32_t bits = 0u;
    if (r < nrows) {
      const int32_t* ids = a.sel + (int64_t)b * a.sel_sb + (int64_t)ih * a.sel_sh + (int64_t)(t0 + r) * a.sel_st;
      for (int j = 0; j < 32; ++j) {
        const int s = 32 * w + j;
        if (s < K && s < p.nblk && ids[s] == s) bits |= 1u << j;
      }
    }
    reinterpret_cast<uint32_t*>(s_ids)[e] = bits;
    if (bits) atomicOr(&s_bits[w], bits);
  }
  for (int e = tid; !dense && e < kTileRows * K; e += blockDim.x) {
    const int r = e / K, s = e % K;
    int id = -1;
    if (r < nrows) {
      const int32_t* ids = a.sel + (int64_t)b * a.sel_sb + (int64_t)ih * a.sel_sh + (int64_t)(t0 + r) * a.sel_st;
      id = ids[s];
      if (id < 0 || id >= p.nblk) id = -1;
      for (int s2 = 0; s2 < s && id >= 0; ++s2)
        if (ids[s2] == id) id = -1;
      if (id >= 0) atomicOr(&s_bits[id >> 5], 1u << (id & 31));
    }
    s_ids[e] = id;
  }
  __syncthreads();
  for (int w = tid; w < p.nwords; w += blockDim.x) atomicAdd(s_cnt, (uint32_t)__popc(s_bits[w]));
  __syncthreads();
  const bool rs = !dense && (int)*s_cnt > K;   // slot = block: a union never exceeds K
  if (tid == 0) p.flag[(int64_t)bh * p.ntiles + tile] = rs ? 1u : 0u;
  const int U = compact_bitmap(s_bits, p.nwords, s_chunks, s_len);
  const int64_t base = (int64_t)bh * p.nblk * p.rwords;
  tile_row_bits(s_ids, K, dense, nrows, s_chunks, U, p.rbm_all + base, rs ? p.rbm + base : nullptr, p.rwords, tile);
}

// Per (sequence, index head, block c, 2048-row window): the window's flagged
// rows that selected c, 64 at a time; each (row, slot) pair's dQ partial
// DS K, fp32.
template <typename T, int D>
__global__ __launch_bounds__(kBwdThreads) void kl_rs_dq_kernel(KlBwdK p) {
  using M = Mfma<T>;
  using L = KlBwdLds<D>;
  constexpr int XP = L::XP, SP = L::SP, MT = D / 32, TPW = 2 * MT / 4;
  extern __shared__ __align__(16) unsigned char smem[];
  T* sK = reinterpret_cast<T*>(smem);
  T* sDS = reinterpret_cast<T*>(smem + L::dsOff);
  __shared__ uint16_t s_rows[kRsRange];
  __shared__ int s_n, s_t[kTileRows], s_slot[kTileRows];
  const srswa_kl_bwd_args& a = p.a;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int64_t lid = (int64_t)(blockIdx.x & 7) * p.per_xcd + (blockIdx.x >> 3);
  if (lid >= (int64_t)a.B * a.HI * p.nrange * p.nblk) return;
  const int c = (int)(lid % p.nblk);
  const int range = (int)((lid / p.nblk) % p.nrange);
  const int bh = (int)(lid / ((int64_t)p.nblk * p.nrange));
  const int ih = bh % a.HI, b = bh / a.HI;
  const int r0 = range * kRsRange;
  const int n = window_rows<kRsRange / 32>(p.rbm + ((int64_t)bh * p.nblk + c) * p.rwords, range * (kRsRange / 32),
                                           p.rwords, s_rows, &s_n);
  if (n == 0) return;
  stage_rows<T, D>(sK, reinterpret_cast<const T*>(a.idx_k) + (int64_t)b * a.ik_sb + (int64_t)c * kChunk * a.ik_st,
                   a.ik_st, min(kChunk, a.Sk - c * kChunk));
  const uint16_t* k16 = reinterpret_cast<const uint16_t*>(sK);
  const int rr = tid / 4, kq = (tid % 4) * 16;    // DS staging: row, 16-key quarter
  for (int g0 = 0; g0 < n; g0 += kTileRows) {
    __syncthreads();                              // the previous group's DS consumed
    {
      const int i = g0 + rr;
      const int t = i < n ? r0 + (int)s_rows[i] : -1;
      const int slot = t >= 0 ? find_slot(a, b, ih, t, c) : -1;
      if (kq == 0) {
        s_t[rr] = t;
        s_slot[rr] = slot;
      }
      float v[16];
      ds16<T>(a, b, ih, t, slot, kq, v);
      uint4 w0, w1;                               // keys in the transposing read's order (slot_of_key)
      w0 = make_uint4(M::pack2(v[0], v[1]), M::pack2(v[2], v[3]), M::pack2(v[8], v[9]), M::pack2(v[10], v[11]));
      w1 = make_uint4(M::pack2(v[4], v[5]), M::pack2(v[6], v[7]), M::pack2(v[12], v[13]), M::pack2(v[14], v[15]));
      *reinterpret_cast<uint4*>(sDS + rr * SP + kq) = w0;
      *reinterpret_cast<uint4*>(sDS + rr * SP + kq + 8) = w1;
    }
    __syncthreads();
    f32x16_t acc[TPW];
#pragma unroll
    for (int i = 0; i < TPW; ++i) acc[i] = zero16();
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int i = 0; i < TPW; ++i) {
        const int tix = wave * TPW + i;
        const int half = tix / MT, dt = tix % MT;
        const uint4 av = *reinterpret_cast<const uint4*>(sDS + (32 * half + (lane & 31)) * SP + 16 * ks + 8 * (lane >> 5));
        acc[i] = M::mac(av, a_operand_tr<XP>(k16, 16 * ks, 32 * dt, lane), acc[i]);
      }
    }
    // row m of output tile (half, dt): 32 half + 8 (r / 4) + 4 (lane / 32) + r % 4
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int tix = wave * TPW + i;
      const int half = tix / MT, dt = tix % MT;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = 32 * half + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        const int t = s_t[m];
        if (t >= 0)
          p.dqp[(((int64_t)bh * a.T + t) * a.K + s_slot[m]) * D + 32 * dt + (lane & 31)] = acc[i][r];
      }
    }
  }
}

// dQ of a flagged row: its pairs' partials summed in slot order (an id's
// first slot, 0 <= id < nblk), rounded once to the input dtype; four head
// dims per thread.
template <typename T, int D>
__global__ __launch_bounds__(256) void kl_rs_dq_reduce_kernel(KlBwdK p) {
  const srswa_kl_bwd_args& a = p.a;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)a.B * a.HI * a.T * (D / 4)) return;
  const int d = (int)(gid % (D / 4)) * 4;
  const int64_t rowi = gid / (D / 4);
  const int t = (int)(rowi % a.T);
  const int bh = (int)(rowi / a.T);
  const int ih = bh % a.HI, b = bh / a.HI;
  if (!p.flag[(int64_t)bh * p.ntiles + t / kTileRows]) return;
  const int32_t* ids = a.sel + (int64_t)b * a.sel_sb + (int64_t)ih * a.sel_sh + (int64_t)t * a.sel_st;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s = 0; s < a.K; ++s) {
    int id = ids[s];
    if (id < 0 || id >= p.nblk) continue;
    bool first = true;
    for (int s2 = 0; s2 < s; ++s2) first = first && ids[s2] != id;
    if (first) {
      const float4 v = *reinterpret_cast<const float4*>(p.dqp + (rowi * a.K + s) * D + d);
      acc.x += v.x;
      acc.y += v.y;
      acc.z += v.z;
      acc.w += v.w;
    }
  }
  uint2 w;
  w.x = Mfma<T>::pack2(acc.x, acc.y);
  w.y = Mfma<T>::pack2(acc.z, acc.w);
  *reinterpret_cast<uint2*>(reinterpret_cast<T*>(a.dq_idx) + (int64_t)b * a.dq_sb + (int64_t)ih * a.dq_sh +
                            (int64_t)t * a.dq_st + d) = w;
}

template <typename T, int D>
__global__ __launch_bounds__(kBwdThreads) void kl_dk_kernel(KlBwdK p) {
  using M = Mfma<T>;
  using L = KlBwdLds<D>;
  constexpr int XP = L::XP, SP = L::SP, MT = D / 32, TPW = 2 * MT / 4;
  constexpr int PR = D / 8;                         // 16-byte pieces per Q row
  extern __shared__ __align__(16) unsigned char smem[];
  T* sQ = reinterpret_cast<T*>(smem);
  T* sDT = reinterpret_cast<T*>(smem + L::dsOff);   // DS^T [key][row]
  __shared__ uint16_t s_rows[kRsWin];
  __shared__ int s_n;
  const srswa_kl_bwd_args& a = p.a;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int win = (int)(blockIdx.x % p.nwin);
  const int c = (int)((blockIdx.x / p.nwin) % p.nblk), b = (int)(blockIdx.x / ((int64_t)p.nwin * p.nblk));
  f32x16_t acc[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i) acc[i] = zero16();
  const uint16_t* q16 = reinterpret_cast<const uint16_t*>(sQ);
  const int rr = tid / 4, kq = (tid % 4) * 16;
  const int w0 = win * (kRsWin / 32), r0 = win * kRsWin;
  int any = 0;
  for (int ih = 0; ih < a.HI; ++ih) {
    const uint32_t* words = p.rbm_all + (((int64_t)b * a.HI + ih) * p.nblk + c) * p.rwords;
    const T* qbase = reinterpret_cast<const T*>(a.q_idx) + (int64_t)b * a.qi_sb + (int64_t)ih * a.qi_sh;
    __syncthreads();                                // the previous head's list consumed
    const int n = window_rows<kRsWin / 32>(words, w0, p.rwords, s_rows, &s_n);
    any |= n;
    for (int g0 = 0; g0 < n; g0 += kTileRows) {
      __syncthreads();
      // the group's Q rows (gathered) and DS^T
      for (int e = tid; e < kTileRows * PR; e += kBwdThreads) {
        const int r = e / PR, cc = (e % PR) * 8;
        const int i = g0 + r;
        const uint4 v = i < n ? *reinterpret_cast<const uint4*>(qbase + (int64_t)(r0 + s_rows[i]) * a.qi_st + cc)
                              : make_uint4(0, 0, 0, 0);
        *reinterpret_cast<uint4*>(sQ + r * XP + cc) = v;
      }
      {
        const int i = g0 + rr;
        const int t = i < n ? r0 + (int)s_rows[i] : -1;
        const int slot = t >= 0 ? find_slot(a, b, ih, t, c) : -1;
        float v[16];
        ds16<T>(a, b, ih, t, slot, kq, v);
#pragma unroll
        for (int k = 0; k < 16; ++k)   // rows in the transposing read's order (slot_of_key)
          reinterpret_cast<uint16_t*>(sDT)[(kq + k) * SP + slot_of_key(rr)] = (uint16_t)(M::pack2(v[k], 0.f) & 0xffffu);
      }
      __syncthreads();
      // dK[key, d] += DS^T[key, row] Q[row, d]
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
        for (int i = 0; i < TPW; ++i) {
          const int tix = wave * TPW + i;
          const int half = tix / MT, dt = tix % MT;
          const uint4 av = *reinterpret_cast<const uint4*>(sDT + (32 * half + (lane & 31)) * SP + 16 * ks + 8 * (lane >> 5));
          acc[i] = M::mac(av, a_operand_tr<XP>(q16, 16 * ks, 32 * dt, lane), acc[i]);
        }
      }
    }
  }
  const int64_t wi = ((int64_t)b * p.nblk + c) * p.nwin + win;
  if (tid == 0) p.dkw[wi] = any ? 1u : 0u;
  if (!any) return;
  // the fp32 partial: key m of output tile (half, dt) is 32 half + 8 (r / 4) + 4 (lane / 32) + r % 4
  float* out = p.dkp + wi * kChunk * D;
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int tix = wave * TPW + i;
    const int half = tix / MT, dt = tix % MT;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = 32 * half + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      out[m * D + 32 * dt + (lane & 31)] = acc[i][r];
    }
  }
}

// dK of a block: its windows' partials summed in window order, rounded once to
// the input dtype; four head dims per thread.
template <typename T, int D>
__global__ __launch_bounds__(256) void kl_dk_reduce_kernel(KlBwdK p) {
  const srswa_kl_bwd_args& a = p.a;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)a.B * p.nblk * kChunk * (D / 4)) return;
  const int d = (int)(gid % (D / 4)) * 4;
  const int key = (int)((gid / (D / 4)) % kChunk);
  const int64_t bc = gid / ((int64_t)(D / 4) * kChunk);   // b * nblk + c
  const int c = (int)(bc % p.nblk), b = (int)(bc / p.nblk);
  if (c * kChunk + key >= a.Sk) return;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int w = 0; w < p.nwin; ++w) {
    const int64_t wi = bc * p.nwin + w;
    if (!p.dkw[wi]) continue;
    const float4 v = *reinterpret_cast<const float4*>(p.dkp + (wi * kChunk + key) * D + d);
    acc.x += v.x;
    acc.y += v.y;
    acc.z += v.z;
    acc.w += v.w;
  }
  uint2 w;
  w.x = Mfma<T>::pack2(acc.x, acc.y);
  w.y = Mfma<T>::pack2(acc.z, acc.w);
  *reinterpret_cast<uint2*>(reinterpret_cast<T*>(a.dk_idx) + (int64_t)b * a.dk_sb +
                            (int64_t)(c * kChunk + key) * a.dk_st + d) = w;
}

bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int check_common(int dtype, int D, int block_size, int K, int Sk, int slots_are_blocks, const char* what) {
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
  if (slots_are_blocks) {
    const int nblk = (int)ceil_div(Sk, kChunk);
    if (K != nblk || nblk > 64 * 32) {
      set_error("%s: slots_are_blocks needs K = ceil(Sk / 64) = %d <= 2048 (got K = %d)", what, nblk, K);
      return SRSWA_UNSUPPORTED;
    }
  } else if (K <= 0 || K > 64) {
    set_error("%s: %d selected blocks per row not supported (1..64)", what, K);
    return SRSWA_UNSUPPORTED;
  }
  return SRSWA_OK;
}

}  // namespace
}  // namespace srswa

using namespace srswa;

namespace srswa {
namespace {

// Workspace of the row-sparse kernels, in 256-byte aligned pieces.
struct KlRsLayout {
  size_t flag, rbm, srec, rst, klp, total;
};
KlRsLayout kl_rs_layout(const srswa_kl_args* a) {
  auto al = [](size_t n) { return (n + 255) / 256 * 256; };
  const int64_t bh = (int64_t)a->B * a->HI, rows = bh * a->T, G = a->HQ / std::max(a->HI, 1);
  const int64_t ntiles = ceil_div(a->T, kTileRows), nblk = ceil_div(a->Sk, kChunk), rwords = ceil_div(a->T, 32);
  KlRsLayout L{};
  L.flag = 0;
  L.rbm = L.flag + al((size_t)(bh * ntiles) * 4);
  L.srec = L.rbm + al((size_t)(bh * nblk * rwords) * 4);
  L.rst = L.srec + al((size_t)(rows * a->K * (G + 1)) * 8);
  L.klp = L.rst + al((size_t)(rows * (G + 1)) * 8);
  L.total = L.klp + al((size_t)(rows * a->K) * 4);
  return L;
}

int kl_fwd_impl(const srswa_kl_args* a, void* scratch, size_t scratch_bytes, void* stream);

// slots_are_blocks: every tile goes block-major when the tiles alone cannot
// fill the chip (a chunk of the warmup stage's rows), else the tile kernel
// runs alone (a tile's union never exceeds K)
bool kl_dense_block_major(const srswa_kl_args* a) {
  return a->slots_are_blocks && (int64_t)a->B * a->HI * ceil_div(a->T, kTileRows) < 512;
}

}  // namespace
}  // namespace srswa

extern "C" size_t srswa_gather_kl_fwd_workspace(const srswa_kl_args* a) {
  if (!a || a->B <= 0 || a->HI <= 0 || a->T <= 0 || a->Sk <= 0 || a->K <= 0) return 0;
  if (a->slots_are_blocks && !kl_dense_block_major(a)) return 0;
  return kl_rs_layout(a).total;
}

extern "C" int srswa_gather_kl_fwd(const srswa_kl_args* a, void* stream) {
  return kl_fwd_impl(a, nullptr, 0, stream);
}

extern "C" int srswa_gather_kl_fwd_ws(const srswa_kl_args* a, void* scratch, size_t scratch_bytes, void* stream) {
  if (!scratch) {
    set_error("gather kl: null workspace (srswa_gather_kl_fwd runs without one)");
    return SRSWA_INVALID;
  }
  return kl_fwd_impl(a, scratch, scratch_bytes, stream);
}

namespace srswa {
namespace {

// The tile kernels (tiles whose rows share their selection) and the
// block-major kernels (flagged tiles) write disjoint rows, and on per-row
// selections the tile kernels occupy few CUs for a long time.  When the caller
// passes a second stream and two events, the tile kernels run on that stream,
// forked from the caller's stream after the flag pass and joined back before
// the call returns; without them everything runs on the caller's stream in
// turn.  The library owns no stream or event and keeps no state between calls.
struct KlSide {
  hipStream_t s;
  hipEvent_t fork, join;
};

// the caller's side stream and events: all three or none
bool kl_side_of(void* s, void* fork, void* join, const char* what, KlSide* out) {
  if (!s && !fork && !join) {
    *out = KlSide{nullptr, nullptr, nullptr};
    return true;
  }
  if (!s || !fork || !join) {
    set_error("%s: side_stream, fork_event and join_event are given together or not at all", what);
    return false;
  }
  *out = KlSide{reinterpret_cast<hipStream_t>(s), reinterpret_cast<hipEvent_t>(fork),
                reinterpret_cast<hipEvent_t>(join)};
  return true;
}

// launches `side_work` on the side stream beside `main_work` on st (both
// after everything already queued on st); st then waits for both.  Without a
// side stream both run on st in turn.
template <typename SideF, typename MainF>
hipError_t kl_fork(hipStream_t st, const KlSide& sd, SideF side_work, MainF main_work) {
  if (!sd.s) {
    side_work(st);
    main_work(st);
    return hipSuccess;   // launch errors are the caller's hipGetLastError()
  }
  hipError_t e = hipEventRecord(sd.fork, st);
  if (e == hipSuccess) e = hipStreamWaitEvent(sd.s, sd.fork, 0);
  if (e != hipSuccess) return e;
  side_work(sd.s);
  main_work(st);
  e = hipEventRecord(sd.join, sd.s);
  if (e == hipSuccess) e = hipStreamWaitEvent(st, sd.join, 0);
  return e;
}

int kl_fwd_impl(const srswa_kl_args* a, void* scratch, size_t scratch_bytes, void* stream) {
  if (!a || !a->q_idx || !a->idx_k || !a->q_main || !a->k_main || !a->sel || !a->pos || !a->kl || !a->valid) {
    set_error("gather kl: null argument");
    return SRSWA_INVALID;
  }
  if (a->B < 0 || a->HI <= 0 || a->HQ <= 0 || a->HKV <= 0 || a->T < 0 || a->Sk <= 0 || a->local_window < 1 ||
      a->HQ % a->HI || a->HQ % a->HKV) {
    set_error("gather kl: bad sizes (HQ must be a multiple of HI and HKV)");
    return SRSWA_INVALID;
  }
  int rc = check_common(a->dtype, a->D, a->block_size, a->K, a->Sk, a->slots_are_blocks, "gather kl");
  if (rc != SRSWA_OK) return rc;
  KlSide side;
  if (!kl_side_of(a->side_stream, a->fork_event, a->join_event, "gather kl", &side)) return SRSWA_INVALID;
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
  if (a->slots_are_blocks && !kl_dense_block_major(a)) scratch = nullptr;   // the tile kernel alone
  KlRsLayout rl{};
  if (scratch) {
    rl = kl_rs_layout(a);
    if (scratch_bytes < rl.total) {
      set_error("gather kl: workspace too small (%zu < %zu)", scratch_bytes, rl.total);
      return SRSWA_WORKSPACE;
    }
  }
  KlK k;
  k.a = *a;
  k.ntiles = ceil_div(a->T, kTileRows);
  const int nblk = ceil_div(a->Sk, kChunk);
  k.nwords = ceil_div(nblk, 32);
  k.G = a->HQ / a->HI;
  k.KV = a->HQ / a->HKV;
  k.nlogical = a->B * a->HI * k.ntiles;
  k.per_xcd = ceil_div(k.nlogical, 8);
  k.rs_flag = nullptr;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  KlRsK rk{};
  if (scratch) {
    // the per-tile decision and the row bitmap first: the tile kernel skips
    // the tiles the row-sparse kernels take
    char* base = static_cast<char*>(scratch);
    rk.a = *a;
    rk.ntiles = k.ntiles;
    rk.nblk = nblk;
    rk.nwords = k.nwords;
    rk.rwords = ceil_div(a->T, 32);
    rk.nrange = ceil_div(a->T, kRsRange);
    rk.per_xcd = (int)ceil_div((int64_t)a->B * a->HI * nblk * rk.nrange, (int64_t)8);
    rk.G = k.G;
    rk.KV = k.KV;
    rk.flag = reinterpret_cast<uint32_t*>(base + rl.flag);
    rk.rbm = reinterpret_cast<uint32_t*>(base + rl.rbm);
    rk.srec = reinterpret_cast<float2*>(base + rl.srec);
    rk.rst = reinterpret_cast<float2*>(base + rl.rst);
    rk.klp = reinterpret_cast<float*>(base + rl.klp);
    const int64_t rbm_words = (int64_t)a->B * a->HI * nblk * rk.rwords;
    hipLaunchKernelGGL(kl_zero_kernel, dim3((unsigned)((rbm_words + 255) / 256)), dim3(256), 0, st, rk.rbm, rbm_words);
    const size_t idw = a->slots_are_blocks ? (size_t)ceil_div(a->K, 32) : (size_t)a->K;
    const size_t flds = ((size_t)k.nwords + 2 + (size_t)kTileRows * idw) * 4 + (size_t)nblk * 2 + 16;
    hipLaunchKernelGGL(kl_rs_flag_kernel, dim3((unsigned)k.nlogical), dim3(256), flds, st, rk);
    k.rs_flag = rk.flag;
  }

  const int tile_bytes = a->D == 64 ? KlLds<64>::tileBytes : KlLds<128>::tileBytes;
  k.ids_off = tile_bytes;
  // per row: K ids, or with slots_are_blocks a bitmap of ceil(K / 32) words
  k.bits_off = k.ids_off + kTileRows * (a->slots_are_blocks ? (int)ceil_div(a->K, 32) : a->K) * 4;
  k.chunks_off = k.bits_off + (k.nwords + 4) * 4;
  const int nchunk_max = std::min(kTileRows * a->K, nblk);
  k.stats_off = (k.chunks_off + nchunk_max * 2 + 15) & ~15;
  const size_t lds = (size_t)k.stats_off + 2 * (size_t)(k.G + 1) * kTileRows * 8 + kTileRows * 4;
  if (lds > 160 * 1024) {
    set_error("gather kl: %zu bytes of LDS needed", lds);
    return SRSWA_UNSUPPORTED;
  }
  const dim3 grid((unsigned)(8 * k.per_xcd)), block(256);
  static LdsGrant granted[4];
  bool lds_ok = true;
#define KL_GRANT(T_, D_, I_) lds_ok = ensure_dynamic_lds(kl_fwd_kernel<T_, D_>, lds, &granted[I_]);
  if (a->dtype == SRSWA_BF16) {
    if (a->D == 128) { KL_GRANT(bf16_t, 128, 0) } else { KL_GRANT(bf16_t, 64, 1) }
  } else {
    if (a->D == 128) { KL_GRANT(__half, 128, 2) } else { KL_GRANT(__half, 64, 3) }
  }
#undef KL_GRANT
  if (!lds_ok) return SRSWA_LAUNCH;
  auto tile_work = [&](hipStream_t s) {
#define KL_LAUNCH(T_, D_) hipLaunchKernelGGL((kl_fwd_kernel<T_, D_>), grid, block, lds, s, k);
    if (a->dtype == SRSWA_BF16) {
      if (a->D == 128) { KL_LAUNCH(bf16_t, 128) } else { KL_LAUNCH(bf16_t, 64) }
    } else {
      if (a->D == 128) { KL_LAUNCH(__half, 128) } else { KL_LAUNCH(__half, 64) }
    }
#undef KL_LAUNCH
  };
  auto rs_work = [&](hipStream_t s) {
    const dim3 gp((unsigned)(8 * (int64_t)rk.per_xcd));
    const dim3 gr((unsigned)(((int64_t)a->B * a->HI * a->T + 255) / 256));
    const dim3 gc((unsigned)(((int64_t)a->B * a->HI * a->T * (k.G + 1) + 255) / 256));
#define KL_RS(T_, D_)                                                                  \
  hipLaunchKernelGGL((kl_rs_pass_kernel<T_, D_, false>), gp, dim3(128), 0, s, rk);    \
  hipLaunchKernelGGL(kl_rs_combine_kernel, gc, dim3(256), 0, s, rk);                   \
  hipLaunchKernelGGL((kl_rs_pass_kernel<T_, D_, true>), gp, dim3(128), 0, s, rk);     \
  hipLaunchKernelGGL(kl_rs_final_kernel, gr, dim3(256), 0, s, rk);
    if (a->dtype == SRSWA_BF16) {
      if (a->D == 128) { KL_RS(bf16_t, 128) } else { KL_RS(bf16_t, 64) }
    } else {
      if (a->D == 128) { KL_RS(__half, 128) } else { KL_RS(__half, 64) }
    }
#undef KL_RS
  };
  if (scratch && kl_dense_block_major(a)) {
    rs_work(st);   // every tile is flagged: the tile kernel would have nothing to do
  } else if (scratch) {
    const hipError_t fe = kl_fork(st, side, tile_work, rs_work);
    if (fe != hipSuccess) {
      set_error("gather kl: side stream failed: %s", hipGetErrorString(fe));
      return SRSWA_LAUNCH;
    }
  } else {
    tile_work(st);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("gather kl launch failed: %s", hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}

}  // namespace
}  // namespace srswa

namespace srswa {
namespace {
// Backward workspace, in 256-byte aligned pieces.
struct KlBwdLayout {
  size_t flag, rbm, rbm_all, dqp, dkp, dkw, total;
};
KlBwdLayout kl_bwd_layout(const srswa_kl_bwd_args* a) {
  auto al = [](size_t n) { return (n + 255) / 256 * 256; };
  const int64_t bh = (int64_t)std::max(a->B, 0) * std::max(a->HI, 0), T = std::max(a->T, 0);
  const int64_t ntiles = ceil_div(T, kTileRows), nblk = ceil_div(std::max(a->Sk, 0), kChunk), rwords = ceil_div(T, 32);
  KlBwdLayout L{};
  L.flag = 0;
  L.rbm = L.flag + al((size_t)(bh * ntiles) * 4);
  L.rbm_all = L.rbm + al((size_t)(bh * nblk * rwords) * 4);
  L.dqp = L.rbm_all + al((size_t)(bh * nblk * rwords) * 4);
  const int64_t kp = a->slots_are_blocks ? 0 : std::max(a->K, 0);   // flagged rows' dQ partials
  L.dkp = L.dqp + al((size_t)(bh * T * kp * std::max(a->D, 0)) * 4);
  const int64_t nwin = ceil_div(T, kRsWin), bb = std::max(a->B, 0);
  L.dkw = L.dkp + al((size_t)(bb * nblk * nwin * kChunk * std::max(a->D, 0)) * 4);
  L.total = L.dkw + al((size_t)(bb * nblk * nwin) * 4);
  return L;
}
}  // namespace
}  // namespace srswa

extern "C" int srswa_gather_kl_bwd_workspace(const srswa_kl_bwd_args* a, size_t* scratch_bytes) {
  if (!a || !scratch_bytes) {
    set_error("gather kl backward workspace: null argument");
    return SRSWA_INVALID;
  }
  *scratch_bytes = kl_bwd_layout(a).total;
  return SRSWA_OK;
}

extern "C" int srswa_gather_kl_bwd(const srswa_kl_bwd_args* a, void* scratch, size_t scratch_bytes, void* stream) {
  if (!a || !a->q_idx || !a->idx_k || !a->sel || !a->dsel || !a->grad || !a->dq_idx || !a->dk_idx) {
    set_error("gather kl backward: null argument");
    return SRSWA_INVALID;
  }
  if (a->B < 0 || a->HI <= 0 || a->T < 0 || a->Sk <= 0) {
    set_error("gather kl backward: bad sizes");
    return SRSWA_INVALID;
  }
  int rc = check_common(a->dtype, a->D, a->block_size, a->K, a->Sk, a->slots_are_blocks, "gather kl backward");
  if (rc != SRSWA_OK) return rc;
  KlSide side;
  if (!kl_side_of(a->side_stream, a->fork_event, a->join_event, "gather kl backward", &side)) return SRSWA_INVALID;
  bool ok = al16(a->q_idx) && al16(a->idx_k) && al16(a->dsel) && ((uintptr_t)a->dq_idx & 7u) == 0;
  for (int64_t st : {a->qi_sb, a->qi_sh, a->qi_st, a->ik_sb, a->ik_st}) ok = ok && (st * 2) % 16 == 0;
  for (int64_t st : {a->dq_sb, a->dq_sh, a->dq_st, a->dk_sb, a->dk_st}) ok = ok && (st * 2) % 8 == 0;   // 4-element stores
  ok = ok && ((uintptr_t)a->dk_idx & 7u) == 0;
  ok = ok && (a->ds_sb * 4) % 16 == 0 && (a->ds_sh * 4) % 16 == 0 && (a->ds_st * 4) % 16 == 0;
  if (!ok) {
    set_error("gather kl backward: rows must be 16-byte aligned");
    return SRSWA_UNSUPPORTED;
  }
  if (ceil_div(a->Sk, kChunk) > 64 * 32) {
    set_error("gather kl backward: more than 2048 key blocks");
    return SRSWA_UNSUPPORTED;
  }
  size_t need = 0;
  srswa_gather_kl_bwd_workspace(a, &need);
  if (a->B == 0 || a->T == 0) return SRSWA_OK;
  if (!scratch || scratch_bytes < need) {
    set_error("gather kl backward: workspace too small (%zu < %zu)", scratch_bytes, need);
    return SRSWA_WORKSPACE;
  }
  const KlBwdLayout bl = kl_bwd_layout(a);
  char* base = static_cast<char*>(scratch);
  KlBwdK k;
  k.a = *a;
  k.ntiles = ceil_div(a->T, kTileRows);
  k.nblk = ceil_div(a->Sk, kChunk);
  k.nwords = ceil_div(k.nblk, 32);
  k.rwords = ceil_div(a->T, 32);
  k.nrange = ceil_div(a->T, kRsRange);
  k.per_xcd = (int)ceil_div((int64_t)a->B * a->HI * k.nblk * k.nrange, (int64_t)8);
  k.flag = reinterpret_cast<uint32_t*>(base + bl.flag);
  k.rbm = reinterpret_cast<uint32_t*>(base + bl.rbm);
  k.rbm_all = reinterpret_cast<uint32_t*>(base + bl.rbm_all);
  k.dqp = reinterpret_cast<float*>(base + bl.dqp);
  k.dkp = reinterpret_cast<float*>(base + bl.dkp);
  k.dkw = reinterpret_cast<uint32_t*>(base + bl.dkw);
  k.nwin = ceil_div(a->T, kRsWin);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int64_t words = (int64_t)(bl.dqp - bl.rbm) / 4;       // both row bitmaps
  hipLaunchKernelGGL(kl_zero_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, st, k.rbm, words);
  const int64_t ntl = (int64_t)a->B * a->HI * k.ntiles;
  const size_t idw = a->slots_are_blocks ? (size_t)ceil_div(a->K, 32) : (size_t)a->K;
  const size_t flds = ((size_t)k.nwords + 2 + (size_t)kTileRows * idw) * 4 + (size_t)k.nblk * 2 + 16;
  hipLaunchKernelGGL(kl_bwd_flag_kernel, dim3((unsigned)ntl), dim3(256), flds, st, k);
  const dim3 gdq((unsigned)ntl), gdk((unsigned)((int64_t)a->B * k.nblk * k.nwin));
  const dim3 gdr((unsigned)(((int64_t)a->B * k.nblk * kChunk * (a->D / 4) + 255) / 256));
  const dim3 grs((unsigned)(8 * (int64_t)k.per_xcd));
  const dim3 grd((unsigned)(((int64_t)a->B * a->HI * a->T * (a->D / 4) + 255) / 256));
  const size_t lds = a->D == 128 ? KlBwdLds<128>::bytes : KlBwdLds<64>::bytes;
  // dQ of the unflagged tiles beside the block-major dQ and dK (disjoint outputs)
  auto dq_work = [&](hipStream_t s) {
#define KL_DQ(T_, D_) hipLaunchKernelGGL((kl_dq_kernel<T_, D_>), gdq, dim3(kBwdThreads), lds, s, k);
    if (a->dtype == SRSWA_BF16) {
      if (a->D == 128) { KL_DQ(bf16_t, 128) } else { KL_DQ(bf16_t, 64) }
    } else {
      if (a->D == 128) { KL_DQ(__half, 128) } else { KL_DQ(__half, 64) }
    }
#undef KL_DQ
  };
  auto rest_work = [&](hipStream_t s) {
    // slot = block: no tile is flagged, so the block-major dQ has no rows
    const bool rs = !a->slots_are_blocks;
#define KL_BWD(T_, D_)                                                                              \
  if (rs) hipLaunchKernelGGL((kl_rs_dq_kernel<T_, D_>), grs, dim3(kBwdThreads), lds, s, k);        \
  if (rs) hipLaunchKernelGGL((kl_rs_dq_reduce_kernel<T_, D_>), grd, dim3(256), 0, s, k);           \
  hipLaunchKernelGGL((kl_dk_kernel<T_, D_>), gdk, dim3(kBwdThreads), lds, s, k);                   \
  hipLaunchKernelGGL((kl_dk_reduce_kernel<T_, D_>), gdr, dim3(256), 0, s, k);
    if (a->dtype == SRSWA_BF16) {
      if (a->D == 128) { KL_BWD(bf16_t, 128) } else { KL_BWD(bf16_t, 64) }
    } else {
      if (a->D == 128) { KL_BWD(__half, 128) } else { KL_BWD(__half, 64) }
    }
#undef KL_BWD
  };
  const hipError_t fe = kl_fork(st, side, dq_work, rest_work);
  if (fe != hipSuccess) {
    set_error("gather kl backward: side stream failed: %s", hipGetErrorString(fe));
    return SRSWA_LAUNCH;
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("gather kl backward launch failed: %s", hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}
