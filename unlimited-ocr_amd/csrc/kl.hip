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
  int* s_ids = reinterpret_cast<int*>(smem + p.ids_off);          // [64][K], -1 = no kept key
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
  const int* my_ids = s_ids + row * K;
  // the row's first kKlIdRegs filtered ids in registers (the slot search of
  // every stage then has no LDS round trip); slots past them are read from LDS
  constexpr int kKlIdRegs = 8;
  int id_reg[kKlIdRegs];
#pragma unroll
  for (int s = 0; s < kKlIdRegs; ++s) id_reg[s] = s < K ? my_ids[s] : -1;
  auto find_slot_of = [&](int c) __attribute__((always_inline)) {
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

// -------------------------------------------------------------- backward
// Both kernels are tile products on the matrix cores with ds = rnd(g * dsel)
// (the reference's bf16 gradient of the logits) staged in LDS:
//   dq_kernel: per (sequence, index head, 64-row tile), over the tile's
//              selected blocks: dQ[rows, d] += DS[rows, keys] K[keys, d];
//   dk_kernel: per (sequence, block), over the 64-row tiles that selected it
//              (a touch bitmap that dq_kernel sets; ascending: deterministic):
//              dK[keys, d] += DS^T[keys, rows] Q[rows, d].
// Four waves; wave w owns output tiles (w / TPW halves of 32 rows / keys,
// 32-wide head-dim slices); K and Q rows are read as B operands with
// ds_read_b64_tr_b16 from their natural layout.
constexpr int kBwdThreads = 256;

struct KlBwdK {
  srswa_kl_bwd_args a;
  int ntiles, nblk, twords;
  uint32_t* touch;          // [B, HI, nblk, twords]
};

template <int D> struct KlBwdLds {
  static constexpr int XP = D + 16;          // K / Q rows: conflict-free transposing reads
  static constexpr int SP = kChunk + 8;      // DS rows: 16-byte row reads
  static constexpr int dsOff = kChunk * XP * 2;
  static constexpr int bytes = dsOff + 64 * SP * 2;
};

// the slot of block c among row (b, ih, t)'s ids (first occurrence), -1 if none
__device__ __forceinline__ int find_slot(const srswa_kl_bwd_args& a, int b, int ih, int t, int c) {
  const int32_t* ids = a.sel + (int64_t)b * a.sel_sb + (int64_t)ih * a.sel_sh + (int64_t)t * a.sel_st;
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
  const int ih = bh % a.HI, b = bh / a.HI;
  const int t0 = tile * kTileRows;
  const int nrows = min(kTileRows, a.T - t0);
  // the tile's selected blocks (rows with a nonzero gradient)
  const int nwords = (p.nblk + 31) / 32;
  for (int w = tid; w < nwords; w += kBwdThreads) s_bits[w] = 0u;
  __syncthreads();
  for (int e = tid; e < nrows * a.K; e += kBwdThreads) {
    const int r = e / a.K, s = e % a.K;
    const int id = a.sel[(int64_t)b * a.sel_sb + (int64_t)ih * a.sel_sh + (int64_t)(t0 + r) * a.sel_st + s];
    if (id >= 0 && id < p.nblk) atomicOr(&s_bits[id >> 5], 1u << (id & 31));
  }
  __syncthreads();
  const int U = compact_bitmap(s_bits, nwords, s_chunks, &s_count);
  // this tile touches these blocks: one bit per (block, tile) for dk_kernel
  for (int u = tid; u < U; u += kBwdThreads)
    atomicOr(&p.touch[(((int64_t)b * a.HI + ih) * p.nblk + s_chunks[u]) * p.twords + (tile >> 5)], 1u << (tile & 31));

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

template <typename T, int D>
__global__ __launch_bounds__(kBwdThreads) void kl_dk_kernel(KlBwdK p) {
  using M = Mfma<T>;
  using L = KlBwdLds<D>;
  constexpr int XP = L::XP, SP = L::SP, MT = D / 32, TPW = 2 * MT / 4;
  extern __shared__ __align__(16) unsigned char smem[];
  T* sQ = reinterpret_cast<T*>(smem);
  T* sDT = reinterpret_cast<T*>(smem + L::dsOff);   // DS^T [key][row]
  const srswa_kl_bwd_args& a = p.a;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int c = blockIdx.x % p.nblk, b = blockIdx.x / p.nblk;
  f32x16_t acc[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i) acc[i] = zero16();
  const uint16_t* q16 = reinterpret_cast<const uint16_t*>(sQ);
  const int rr = tid / 4, kq = (tid % 4) * 16;
  for (int ih = 0; ih < a.HI; ++ih) {
    const uint32_t* tb = p.touch + (((int64_t)b * a.HI + ih) * p.nblk + c) * p.twords;
    for (int wd = 0; wd < p.twords; ++wd) {
      uint32_t bits = tb[wd];
      while (bits) {
        const int tile = 32 * wd + __ffs(bits) - 1;
        bits &= bits - 1;
        const int t0 = tile * kTileRows;
        const int nrows = min(kTileRows, a.T - t0);
        __syncthreads();
        stage_rows<T, D>(sQ, reinterpret_cast<const T*>(a.q_idx) + (int64_t)b * a.qi_sb + (int64_t)ih * a.qi_sh +
                                 (int64_t)t0 * a.qi_st,
                         a.qi_st, nrows);
        {
          float v[16];
          const int slot = rr < nrows ? find_slot(a, b, ih, t0 + rr, c) : -1;
          ds16<T>(a, b, ih, t0 + rr, slot, kq, v);
#pragma unroll
          for (int i = 0; i < 16; ++i)   // rows in the transposing read's order (slot_of_key)
            reinterpret_cast<uint16_t*>(sDT)[(kq + i) * SP + slot_of_key(rr)] =
                (uint16_t)(M::pack2(v[i], 0.f) & 0xffffu);
        }
        __syncthreads();
        // dK[key, d] += DS^T[key, row] Q[row, d]
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
          for (int i = 0; i < TPW; ++i) {
            const int tix = wave * TPW + i;
            const int half = tix / MT, dt = tix % MT;
            const uint4 av =
                *reinterpret_cast<const uint4*>(sDT + (32 * half + (lane & 31)) * SP + 16 * ks + 8 * (lane >> 5));
            acc[i] = M::mac(av, a_operand_tr<XP>(q16, 16 * ks, 32 * dt, lane), acc[i]);
          }
        }
      }
    }
  }
  store_tiles<T, D>(reinterpret_cast<T*>(a.dk_idx) + (int64_t)b * a.dk_sb + (int64_t)c * kChunk * a.dk_st, a.dk_st,
                    min(kChunk, a.Sk - c * kChunk), acc, wave, lane);
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
  const size_t lds = (size_t)k.stats_off + 2 * (size_t)(k.G + 1) * kTileRows * 8 + kTileRows * 4;
  if (lds > 160 * 1024) {
    set_error("gather kl: %zu bytes of LDS needed", lds);
    return SRSWA_UNSUPPORTED;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)(8 * k.per_xcd)), block(256);
  static LdsGrant granted[4];
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

extern "C" int srswa_gather_kl_bwd_workspace(const srswa_kl_bwd_args* a, size_t* scratch_bytes) {
  if (!a || !scratch_bytes) {
    set_error("gather kl backward workspace: null argument");
    return SRSWA_INVALID;
  }
  const int64_t words = (int64_t)a->B * a->HI * ceil_div(a->Sk, kChunk) * ceil_div(ceil_div(a->T, kTileRows), 32);
  *scratch_bytes = (size_t)std::max<int64_t>(words, 0) * 4;
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
  int rc = check_common(a->dtype, a->D, a->block_size, a->K, "gather kl backward");
  if (rc != SRSWA_OK) return rc;
  bool ok = al16(a->q_idx) && al16(a->idx_k) && al16(a->dsel);
  for (int64_t st : {a->qi_sb, a->qi_sh, a->qi_st, a->ik_sb, a->ik_st}) ok = ok && (st * 2) % 16 == 0;
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
  KlBwdK k;
  k.a = *a;
  k.ntiles = ceil_div(a->T, kTileRows);
  k.nblk = ceil_div(a->Sk, kChunk);
  k.twords = ceil_div(k.ntiles, 32);
  k.touch = static_cast<uint32_t*>(scratch);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int64_t words = (int64_t)need / 4;
  hipLaunchKernelGGL(kl_zero_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, st, k.touch, words);
  const dim3 gdq((unsigned)((int64_t)a->B * a->HI * k.ntiles)), gdk((unsigned)((int64_t)a->B * k.nblk));
  const size_t lds = a->D == 128 ? KlBwdLds<128>::bytes : KlBwdLds<64>::bytes;
#define KL_BWD(T_, D_)                                                                      \
  hipLaunchKernelGGL((kl_dq_kernel<T_, D_>), gdq, dim3(kBwdThreads), lds, st, k);          \
  hipLaunchKernelGGL((kl_dk_kernel<T_, D_>), gdk, dim3(kBwdThreads), lds, st, k);
  if (a->dtype == SRSWA_BF16) {
    if (a->D == 128) { KL_BWD(bf16_t, 128) } else { KL_BWD(bf16_t, 64) }
  } else {
    if (a->D == 128) { KL_BWD(__half, 128) } else { KL_BWD(__half, 64) }
  }
#undef KL_BWD
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("gather kl backward launch failed: %s", hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}
