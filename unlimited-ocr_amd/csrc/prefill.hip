// Gather-attention forward on the matrix cores (gfx950): prefill / training /
// chunked prefill with a prefix cache.
//
// Replaces the reference's fused forward kernels
//   _gather_attn_fwd_kernel (K1)  HF/sparse_gather_triton.py:35-122
//   _e2e_attn_fwd_kernel   (K5)  HF/sparse_gather_e2e_triton.py:36-121
// and extends them to a query chunk at the tail of a longer KV cache (the
// reference wrapper returns None there, HF/sparse_gather_triton.py:409-410).
//
// Semantics per query row t (key index qi = Sk - T + t, sample start seg,
// window start ls = max(qi - LW + 1, seg)):
//   window keys ls <= j <= qi                       logit = scale*q.k
//   remote keys j in a selected block, seg <= j < ls  logit = scale*q.k + bias
// one softmax over both (disjoint) sets, O in the input dtype, LSE in fp32.
// Duplicate block ids count once (the first slot's bias is used).  The block
// size is a power of two >= 16, as the reference's tl.arange(0, BS) requires
// (HF/sparse_gather_triton.py:86), so every aligned 16-key quarter of a
// 64-key chunk lies inside one block.
//
// One workgroup = (sequence, query head, 64-row query tile), two waves of 32
// rows; at most ~40 KB of LDS and 256 registers per lane, so four workgroups
// (two waves per SIMD) share a CU and hide each other's latencies.
// Set-up: every row's block ids are sorted and deduplicated into LDS, and the
// sorted list of 64-key chunks the tile visits is built (window ranges and
// selected blocks of all 64 rows: bitmap + prefix popcount), so a tile whose
// rows share their selection visits |selected| + |window| chunks once.
// Per chunk:
//   * K (row pitch D+8) and V (row pitch D+16) are staged in LDS from
//     registers fetched one chunk ahead;
//   * S^T = K Q^T on v_mfma_f32_32x32x16_{bf16,f16}: every lane owns one
//     query row and 32 of the chunk's keys;
//   * each lane derives its row's 64-bit keep mask for the chunk (window range
//     | remote range & selected quarters); a chunk that every row of the wave
//     keeps whole (the common case) skips all per-key masking;
//   * softmax in the log2 domain with lazy rescaling: the running max moves
//     only when a chunk exceeds it by more than 2^8, so the O accumulators are
//     rescaled only on those rare chunks;
//   * O^T += V^T P^T, the V^T operand read from the natural V tile by
//     ds_read_b64_tr_b16 (two transposing reads per operand).
// q*scale and P are rounded to the input dtype before their products, the
// same rounding points as the reference kernels (HF/sparse_gather_triton.py:68,94).
#include <algorithm>
#include <cmath>

#include "mfma_common.h"

namespace srswa {
namespace {

struct FwdK {
  srswa_fwd_args a;
  int ntiles, nwords, SP, G, IG, bs_shift;
  int nlogical, per_xcd;       // XCD-aware workgroup order
  int chunks_off, sid_off;     // LDS byte offsets of the chunk list and sorted ids
  int pages_off;               // paged: LDS byte offset of the visited chunks' page ids
  int ppc, page_cap;           // paged: page ids per chunk (1 when BS >= 64, else 4); chunks held in LDS
  // paged form (the serving prefill): request b's queries are rows cu[b] ..
  // cu[b + 1) of q / out / ids / bias, query t sits at key prefix[b] + t, the
  // request holds seqlen[b] keys, and key j is row j % BS of page bt[b, j / BS]
  const int32_t* cu;
  const int32_t* prefix;
  const int32_t* seqlen;
  const int32_t* bt;
  int64_t bt_sr, k_pst, v_pst;
  int kv8;                     // FP8: the caches' fp8 format (srswa_dtype)
  // tail split: the last ntail logical tiles run as nsplit workgroups each, part
  // p taking chunks [U p / nsplit, U (p + 1) / nsplit) of the tile's plan and
  // writing an unnormalised record (O fp32 [64][D], then m, l per row) that
  // fwd_merge_kernel combines.  The whole tiles come first in dispatch order.
  int nsplit, ntail, per_xcd_p;
  float* part;                 // [ntail * nsplit][64 * D + 128]
};

// ES: element bytes (2, or 4 for fp32, whose V^T operand is read as scalars:
// a 4-float pad keeps the two lane halves' rows, 4 apart, on different banks)
template <int D, int ES = 2> struct FwdLds {
  static constexpr int KP = D + 8;                  // K row pitch (elements): conflict-free row reads
  static constexpr int VP = ES == 4 ? D + 4 : D + 16;   // V row pitch: conflict-free V^T reads
  static constexpr int kOff = 0;
  static constexpr int vOff = kChunk * KP * ES;
  static constexpr int tileBytes = vOff + kChunk * VP * ES;
};

// Two waves per SIMD; the fp32 form at D = 128 (twice the operand registers)
// one, with the accumulators in the second register file.
template <typename T, int D, bool PAGED, bool FP8 = false>
__global__ __launch_bounds__(128) __attribute__((amdgpu_waves_per_eu(std::is_same<T, float>::value && D == 128 ? 1 : 2)))
void fwd_kernel(FwdK p) {
  static_assert(!FP8 || PAGED, "fp8 caches: the paged form");
  constexpr bool F32 = std::is_same<T, float>::value;   // fp32: the unpaged form, 8 MFMAs per k step
  static_assert(!F32 || !PAGED, "fp32: the unpaged form");
  using KE = std::conditional_t<FP8, uint8_t, T>;   // cache element
  // a staged piece: 8 cache elements
  using Pre = std::conditional_t<FP8, uint2, Frag<T>>;
  using M = Mfma<T>;
  using L = FwdLds<D, (int)sizeof(T)>;
  constexpr int KP = L::KP, VP = L::VP;
  constexpr int KS = D / 16;         // k-steps over the head dim
  constexpr int MT = D / 32;         // 32-row tiles of O^T
  constexpr int NT = 128;
  constexpr int PPT = kChunk * D / 8 / NT;   // 16-byte pieces of K (and of V) per thread
  extern __shared__ __align__(16) unsigned char smem[];
  const srswa_fwd_args& a = p.a;

  // The hardware deals workgroups to the 8 XCDs round-robin; logical tile
  // xcd * per_xcd + k keeps neighbouring tiles of one (sequence, head), which
  // share most of their window keys, on the same L2.
  const int nwhole = p.nlogical - p.ntail;
  int lid, part = 0, rec = -1;
  if ((int)blockIdx.x < 8 * p.per_xcd) {
    lid = (int)(blockIdx.x & 7) * p.per_xcd + (int)(blockIdx.x >> 3);
    if (lid >= nwhole) return;
  } else {
    const int pid = (int)blockIdx.x - 8 * p.per_xcd;
    rec = (pid & 7) * p.per_xcd_p + (pid >> 3);
    if (rec >= p.ntail * p.nsplit) return;
    lid = nwhole + rec / p.nsplit;
    part = rec % p.nsplit;
  }

  T* sK = reinterpret_cast<T*>(smem + L::kOff);
  T* sV = reinterpret_cast<T*>(smem + L::vOff);
  // set-up arrays alias the K/V tiles (dead once the chunk loop starts)
  int* s_qi = reinterpret_cast<int*>(smem);
  int* s_seg = s_qi + 64;
  int* s_ls = s_seg + 64;
  int* s_count = s_ls + 64;
  uint32_t* s_bits = reinterpret_cast<uint32_t*>(s_count + 4);
  uint16_t* s_chunks = reinterpret_cast<uint16_t*>(smem + p.chunks_off);
  int* s_sid = reinterpret_cast<int*>(smem + p.sid_off);
  float* s_sb = a.bias ? reinterpret_cast<float*>(s_sid + 64 * p.SP) : nullptr;

  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int h = lane >> 5, rl = lane & 31;
  const int tile = lid % p.ntiles;
  const int bh = lid / p.ntiles;
  const int hq = bh % a.HQ, b = bh / a.HQ;
  const int kvh = hq / p.G, ih = hq / p.IG;
  const int t0 = tile * kTileRows;
  // this tile's sequence: its query rows (q0 = first row in q / out / ids),
  // key count and the key index of its first query
  int q0 = 0, Tb = a.T, Skb = a.Sk;
  if constexpr (PAGED) {
    q0 = p.cu[b];
    Tb = p.cu[b + 1] - q0;
    Skb = p.seqlen[b];
    if (t0 >= Tb) return;             // the grid covers the longest request
  }
  const int nrows = min(kTileRows, Tb - t0);
  const int off = PAGED ? p.prefix[b] : a.Sk - a.T;
  const int BS = a.block_size, LW = a.local_window, SP = p.SP;
  const int maxblk = (Skb - 1) >> p.bs_shift;
  // logits to log2 units: the matrix-core prefill rounds q * scale to the input
  // dtype first (K1 / K5, HF/sparse_gather_triton.py:68); the serving prefill
  // scales the fp32 product (attend_triton.py:204)
  const float l2s = PAGED ? a.scale * kLog2e : kLog2e;

  // Loads first, and nothing computed from a loaded value until all are
  // issued (a use waits for its own load and every load issued before it):
  // the set-up row's sample start and first 8 slots (tid < 64, row r = tid),
  // then this lane's query row, in flight across the sort and the chunk plan.
  // Rows past T read row t0 (valid memory) and are masked where used (their
  // output and lse are never written).
  const int row = wave * 32 + rl;
  const bool row_ok = row < nrows;
  const int r = tid, rr = min(r, nrows - 1);
  const int smax = max(a.S - 1, 0);
  const int32_t* ids = a.S > 0 ? a.idx + (int64_t)b * a.idx_sb + (int64_t)ih * a.idx_sh + (int64_t)(q0 + t0 + rr) * a.idx_st
                               : reinterpret_cast<const int32_t*>(a.q);   // a valid stand-in, never used
  const float* bias = a.bias ? a.bias + (int64_t)b * a.bias_sb + (int64_t)ih * a.bias_sh + (int64_t)(q0 + t0 + rr) * a.bias_st
                             : reinterpret_cast<const float*>(ids);
  const int* segp = a.seg ? a.seg + (int64_t)b * a.seg_sb + t0 + rr : ids;
  int seg_ld = 0, id8[8];
  float b8[8];
  if (tid < 64) {
    seg_ld = *segp;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      id8[s] = ids[min(s, smax)];
      b8[s] = bias[min(s, smax)];
    }
  }
  Frag<T> qf[KS];
  {
    const T* qrow = reinterpret_cast<const T*>(a.q) + (int64_t)b * a.q_sb +
                    (int64_t)(q0 + t0 + (row_ok ? row : 0)) * a.q_st + (int64_t)hq * a.q_sh;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = *reinterpret_cast<const Frag<T>*>(qrow + 16 * ks + 8 * h);
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
    if (a.S <= 8) {
#pragma unroll
      for (int s = 0; s < 8; ++s) {   // -1 / 0 past S and past T
        const bool in = r < nrows && s < a.S;
        id8[s] = in ? id8[s] : -1;
        b8[s] = in && a.bias ? b8[s] : 0.f;
      }
      sort_row_ids8(id8, b8, SP, BS, maxblk, qi, seg, ls, s_sid + r * SP, s_sb ? s_sb + r * SP : nullptr);
    } else {
      sort_row_ids(ids, a.bias ? bias : nullptr, r < nrows ? a.S : 0, SP, BS, maxblk, qi, seg, ls, s_sid + r * SP,
                   s_sb ? s_sb + r * SP : nullptr);
    }
  }
  lds_barrier();
  const int U = plan_chunks(s_qi, s_seg, s_ls, s_sid, SP, BS, LW, nrows, p.nwords, s_bits, s_chunks, s_count);
  // paged: the page of each 16-key quarter of every visited chunk, looked up
  // once here, so a prefetch issues its K / V loads without a dependent read
  // (the first page_cap chunks; a longer list reads the rest from the table)
  int* s_pages = PAGED ? reinterpret_cast<int*>(smem + p.pages_off) : nullptr;
  const int32_t* bt_r = PAGED ? p.bt + (int64_t)b * p.bt_sr : nullptr;
  const int nblk_live = (Skb + BS - 1) >> p.bs_shift;
  auto page_of = [&](int c, int qq) {    // page of quarter qq of chunk c
    const int blk = (c * kChunk + 16 * qq) >> p.bs_shift;
    return blk < nblk_live ? bt_r[blk] : 0;
  };
  if constexpr (PAGED) {
    const int held = min(U, p.page_cap);
    for (int e = tid; e < held * p.ppc; e += 128) s_pages[e] = page_of(s_chunks[e / p.ppc], e % p.ppc);
    __syncthreads();
  }

  // this lane's row: window [ls, qi], remote candidates [seg, min(ls, qi + 1))
  const int my_ls = s_ls[row], my_seg = s_seg[row];
  const int my_hi = s_qi[row] + 1;
  const int rem_hi = min(my_ls, my_hi);
  const int* my_sid = s_sid + row * SP;
  const float* my_sb = s_sb ? s_sb + row * SP : nullptr;
  // a chunk inside the window of every row of the wave, [w_ls_max, w_hi_min),
  // takes no per-key mask, no bias and no walk of the selected ids (the
  // bounds are wave-uniform)
  const int w_ls_max = wave_max_int(row_ok ? my_ls : INT_MIN);
  const int w_hi_min = wave_min_int(row_ok ? my_hi : INT_MAX);
  const float inv_l2s = PAGED ? 1.f / a.scale * kLn2 : kLn2;


  if constexpr (F32) {
    // fp32: q * scale, each product rounded once (as the reference's fp32 q * scale)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      uint32_t* ww = reinterpret_cast<uint32_t*>(&qf[ks]);
#pragma unroll
      for (int e = 0; e < 8; ++e) ww[e] = __float_as_uint(__uint_as_float(ww[e]) * a.scale);
    }
  } else if constexpr (!PAGED) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      uint32_t* ww = reinterpret_cast<uint32_t*>(&qf[ks]);
#pragma unroll
      for (int e = 0; e < 4; ++e) ww[e] = M::pack2(M::lo(ww[e]) * a.scale, M::hi(ww[e]) * a.scale);
    }
  }

  f32x16_t o[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) o[mt] = zero16();
  float m_b = -INFINITY, l_run = 0.f;     // running max (log2 units) and row sum
  int cur = 0, nid = my_sid[0];           // cursor into the row's sorted ids

  // K / V of this (sequence, kv head) as buffer resources ending at key Sk - 1
  // (keys of a chunk beyond Sk read as zero)
  constexpr uint32_t ES = sizeof(T);
  const __amdgpu_buffer_rsrc_t krs = make_rsrc(
      reinterpret_cast<const T*>(a.k) + (int64_t)b * a.k_sb + (int64_t)kvh * a.k_sh,
      (uint32_t)(((int64_t)(a.Sk - 1) * a.k_st + D) * ES));
  const __amdgpu_buffer_rsrc_t vrs = make_rsrc(
      reinterpret_cast<const T*>(a.v) + (int64_t)b * a.v_sb + (int64_t)kvh * a.v_sh,
      (uint32_t)(((int64_t)(a.Sk - 1) * a.v_st + D) * ES));
  constexpr int RPP = NT / (D / 8);            // rows per pass of the 128 threads
  const uint32_t kvo = (uint32_t)((tid / (D / 8)) * a.k_st + (tid % (D / 8)) * 8) * ES;
  const uint32_t vvo = (uint32_t)((tid / (D / 8)) * a.v_st + (tid % (D / 8)) * 8) * ES;
  // this thread's 16-byte piece of the first staged row; later pieces are RPP rows apart
  T* sKw = sK + (tid / (D / 8)) * KP + (tid % (D / 8)) * 8;
  T* sVw = sV + (tid / (D / 8)) * VP + (tid % (D / 8)) * 8;
  Pre kpre[PPT], vpre[PPT];
  // paged: the kv head's base (uniform) and this thread's column byte offset.
  // Piece i of a thread covers chunk row tid / (D/8) + i * RPP, whose 16-key
  // quarter is (i * RPP) / 16 for every thread (tid / (D/8) < RPP <= 16), so
  // the page of each piece is uniform: its base goes to scalar registers
  // (readfirstlane) and only a 32-bit in-page offset stays per lane.
  const char* kpg = reinterpret_cast<const char*>(reinterpret_cast<const KE*>(a.k) + (int64_t)kvh * a.k_sh);
  const char* vpg = reinterpret_cast<const char*>(reinterpret_cast<const KE*>(a.v) + (int64_t)kvh * a.v_sh);
  const uint32_t col_b = (uint32_t)(tid % (D / 8)) * 8u * (uint32_t)sizeof(KE);
  auto fetch = [&](int u) {
    const int c = s_chunks[u];
    if constexpr (PAGED) {
      static_assert(RPP <= 16 && 16 % RPP == 0, "a piece's quarter must not depend on the thread");
      // the chunk's (up to) four quarter pages, uniform: from LDS, or past the
      // held list from the block table
      int qpg[4];
      if (u < p.page_cap) {
        if (p.ppc == 1) {
          qpg[0] = qpg[1] = qpg[2] = qpg[3] = __builtin_amdgcn_readfirstlane(s_pages[u]);
        } else {
#pragma unroll
          for (int qq = 0; qq < 4; ++qq) qpg[qq] = __builtin_amdgcn_readfirstlane(s_pages[4 * u + qq]);
        }
      } else {
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) qpg[qq] = __builtin_amdgcn_readfirstlane(page_of(c, qq));
      }
#pragma unroll
      for (int i = 0; i < PPT; ++i) {
        const int row = tid / (D / 8) + i * RPP;
        const int j = c * kChunk + row;
        const int pg = qpg[(i * RPP) >> 4];
        const uint32_t jr = (uint32_t)(j & (BS - 1));
        const char* kb = kpg + (int64_t)pg * p.k_pst * (int64_t)sizeof(KE);
        const char* vb = vpg + (int64_t)pg * p.v_pst * (int64_t)sizeof(KE);
        if (j < Skb) {
          kpre[i] = *reinterpret_cast<const Pre*>(kb + (jr * (uint32_t)a.k_st * (uint32_t)sizeof(KE) + col_b));
          vpre[i] = *reinterpret_cast<const Pre*>(vb + (jr * (uint32_t)a.v_st * (uint32_t)sizeof(KE) + col_b));
        } else {
          kpre[i] = Pre{};
          vpre[i] = Pre{};
        }
      }
    } else if constexpr (F32) {
      // two 16-byte words per 8-float piece, both offsets in the lane part
      // (the buffer range check reads keys past Sk as zero)
      const uint32_t kso = (uint32_t)c * kChunk * (uint32_t)a.k_st * ES;
      const uint32_t vso = (uint32_t)c * kChunk * (uint32_t)a.v_st * ES;
#pragma unroll
      for (int i = 0; i < PPT; ++i) {
        const uint32_t ko = kvo + kso + (uint32_t)(i * RPP) * (uint32_t)a.k_st * ES;
        const uint32_t vo = vvo + vso + (uint32_t)(i * RPP) * (uint32_t)a.v_st * ES;
        kpre[i] = Pre{buffer_load16(krs, ko, 0), buffer_load16(krs, ko + 16, 0)};
        vpre[i] = Pre{buffer_load16(vrs, vo, 0), buffer_load16(vrs, vo + 16, 0)};
      }
    } else if constexpr (!FP8) {
      const uint32_t kso = (uint32_t)c * kChunk * (uint32_t)a.k_st * 2u;
      const uint32_t vso = (uint32_t)c * kChunk * (uint32_t)a.v_st * 2u;
#pragma unroll
      for (int i = 0; i < PPT; ++i) {
        kpre[i] = buffer_load16(krs, kvo, kso + (uint32_t)(i * RPP) * (uint32_t)a.k_st * 2u);
        vpre[i] = buffer_load16(vrs, vvo, vso + (uint32_t)(i * RPP) * (uint32_t)a.v_st * 2u);
      }
    }
  };
  const uint16_t* v16 = reinterpret_cast<const uint16_t*>(sV);

  // this workgroup's share of the plan (all of it unless the tile is split)
  const int nsp = rec >= 0 ? p.nsplit : 1;
  const int u_lo = (int)((int64_t)U * part / nsp), u_hi = (int)((int64_t)U * (part + 1) / nsp);
  if (u_lo < u_hi) fetch(u_lo);
  for (int u = u_lo; u < u_hi; ++u) {
    const int j0 = (int)s_chunks[u] * kChunk;
    __syncthreads();   // previous chunk fully consumed
    if constexpr (FP8) {
      fp8_dispatch(p.kv8, [&](auto F) {
        constexpr int FF = decltype(F)::value;
        uint32_t sp = 0u;
#pragma unroll
        for (int i = 0; i < PPT; ++i) sp |= fp8_special_bits<FF>(kpre[i]) | fp8_special_bits<FF>(vpre[i]);
        if (__builtin_expect(!fp8_any_special(sp), 1)) {
#pragma unroll
          for (int i = 0; i < PPT; ++i) {
            *reinterpret_cast<uint4*>(sKw + i * RPP * KP) = fp8x8_to_fast<FF, T>(kpre[i]);
            *reinterpret_cast<uint4*>(sVw + i * RPP * VP) = fp8x8_to_fast<FF, T>(vpre[i]);
          }
        } else {
#pragma unroll
          for (int i = 0; i < PPT; ++i) {
            *reinterpret_cast<uint4*>(sKw + i * RPP * KP) = fp8x8_to_exact<FF, T>(kpre[i]);
            *reinterpret_cast<uint4*>(sVw + i * RPP * VP) = fp8x8_to_exact<FF, T>(vpre[i]);
          }
        }
      });
    } else {
#pragma unroll
      for (int i = 0; i < PPT; ++i) {
        *reinterpret_cast<Pre*>(sKw + i * RPP * KP) = kpre[i];
        *reinterpret_cast<Pre*>(sVw + i * RPP * VP) = vpre[i];
      }
    }
    __syncthreads();
    if (u + 1 < u_hi) fetch(u + 1);

    // S^T (keys x rows) for the two 32-key halves of the chunk
    f32x16_t st[2] = {zero16(), zero16()};
    // the wave's issue priority is raised over its MFMA blocks: of the two waves
    // of a SIMD, the one with matrix work issues it first and the other's
    // softmax VALU fills the MFMA execution time
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const Frag<T> a0 = *reinterpret_cast<const Frag<T>*>(sK + rl * KP + 16 * ks + 8 * h);
      const Frag<T> a1 = *reinterpret_cast<const Frag<T>*>(sK + (32 + rl) * KP + 16 * ks + 8 * h);
      st[0] = M::mac(a0, qf[ks], st[0]);
      st[1] = M::mac(a1, qf[ks], st[1]);
    }
    __builtin_amdgcn_s_setprio(0);

    // the row's keep mask: window keys | remote keys of its selected 16-key
    // quarters (with their bias).  A chunk that every row of the wave keeps
    // whole with one bias (always one inside every row's window) leaves the
    // raw logits as they are; otherwise the masks and the bias are folded into
    // them: a dropped key becomes -inf, a kept remote key's bias is added as
    // bias / l2s (l2s > 0), so one softmax form below serves both.
    float addb = 0.f;
    uint64_t keep = ~0ull, rm = 0ull;
    float bq[4] = {0.f, 0.f, 0.f, 0.f};
    int masked = 0;
    if (!(j0 >= w_ls_max && j0 + kChunk <= w_hi_min)) {
      uint32_t qmem = 0;
      if (BS >= kChunk) {
        const int blk = j0 >> p.bs_shift;
        while (nid < blk) nid = my_sid[++cur];
        if (nid == blk) {
          qmem = 15u;
          if (my_sb) bq[0] = bq[1] = bq[2] = bq[3] = my_sb[cur] * kLog2e;
        }
      } else {
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const int blk = (j0 + 16 * qq) >> p.bs_shift;
          while (nid < blk) nid = my_sid[++cur];
          if (nid == blk) {
            qmem |= 1u << qq;
            if (my_sb) bq[qq] = my_sb[cur] * kLog2e;
          }
        }
      }
      uint64_t qm = 0;
#pragma unroll
      for (int qq = 0; qq < 4; ++qq)
        if (qmem & (1u << qq)) qm |= 0xffffull << (16 * qq);
      const uint64_t wm = range64(min(max(my_ls - j0, 0), 64), min(max(my_hi - j0, 0), 64));
      rm = range64(min(max(my_seg - j0, 0), 64), min(max(rem_hi - j0, 0), 64)) & qm;
      keep = wm | rm;
      const bool whole = !row_ok || (keep == ~0ull && (!my_sb || rm == 0ull || (rm == ~0ull && BS >= kChunk)));
      if (__all(whole)) {
        if (my_sb && rm != 0ull) addb = bq[0];
      } else {
        masked = 1;
      }
    }
    // The mask is applied under an opaque per-lane flag, so the compiler
    // predicates the update in place instead of branching around it (a
    // uniform branch made it keep the raw logits in a second register set and
    // copy all 32 back at the join, on every unmasked chunk).
    asm volatile("" : "+v"(masked));
    if (masked) {
      const uint64_t kh = keep >> (4 * h), rh = rm >> (4 * h);
      float bs[4];
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) bs[qq] = bq[qq] * inv_l2s;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const uint32_t k32 = (uint32_t)(kh >> (32 * half)), r32 = (uint32_t)(rh >> (32 * half));
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int bit = 8 * (r >> 2) + (r & 3);
          float x = st[half][r];
          if (my_sb) x += ((r32 >> bit) & 1u) ? bs[2 * half + (r >> 3)] : 0.f;
          st[half][r] = ((k32 >> bit) & 1u) ? x : -INFINITY;
        }
      }
    }

    // row max of the chunk's logits (log2 units); lane (l, h) holds keys
    // 32 half + 8 (r / 4) + 4h + r % 4
    float mq[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x16_t& s = st[g >> 1];
      const int r0 = 8 * (g & 1);
      mq[g] = fmaxf(fmaxf(fmaxf(s[r0], s[r0 + 1]), fmaxf(s[r0 + 2], s[r0 + 3])),
                    fmaxf(fmaxf(s[r0 + 4], s[r0 + 5]), fmaxf(s[r0 + 6], s[r0 + 7])));
    }
    float mloc = fmaf(fmaxf(fmaxf(mq[0], mq[1]), fmaxf(mq[2], mq[3])), l2s, addb);
    mloc = xor32_max(mloc);
    // lazy rescaling: the reference point m_b moves only when the chunk's max
    // exceeds it by more than 8 (p <= 2^8 stays exact in fp32 and in P's
    // rounding), so O is rescaled only on the rare chunks where a row's max jumps
    const bool grow = mloc > m_b + 8.f;
    if (__any(grow)) {
      float alpha = 1.f;
      if (grow) {
        alpha = exp2f(m_b - mloc);    // 0 on a row's first non-empty chunk
        m_b = mloc;
      }
      l_run *= alpha;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[mt][r] *= alpha;
    }
    const float sub = addb - (m_b == -INFINITY ? 0.f : m_b);
    float ps[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int half = 0; half < 2; ++half)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pv = __builtin_amdgcn_exp2f(fmaf(st[half][r], l2s, sub));
        st[half][r] = pv;
        ps[2 * half + (r >> 3)] += pv;
      }
    l_run += (ps[0] + ps[1]) + (ps[2] + ps[3]);

    // P^T as B operands (4 steps of 16 keys), rounded to the input dtype
    Frag<T> pb[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int hf = ks >> 1, r0 = 8 * (ks & 1);
      if constexpr (F32) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = st[hf][r0 + j];
        pb[ks] = f32x8(v);
      } else {
        pb[ks] = make_uint4(M::pack2(st[hf][r0], st[hf][r0 + 1]), M::pack2(st[hf][r0 + 2], st[hf][r0 + 3]),
                            M::pack2(st[hf][r0 + 4], st[hf][r0 + 5]), M::pack2(st[hf][r0 + 6], st[hf][r0 + 7]));
      }
    }
    // O^T += V^T P^T, k-step outer: the MT accumulators form independent
    // chains that interleave, and a step's operands are read before its MFMAs
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      Frag<T> va[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if constexpr (F32)
          va[mt] = a_operand_f32<VP>(reinterpret_cast<const float*>(sV), 16 * ks, 32 * mt, lane);
        else
          va[mt] = a_operand_tr<VP>(v16, 16 * ks, 32 * mt, lane);
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) o[mt] = M::mac(va[mt], pb[ks], o[mt]);
    }
    __builtin_amdgcn_s_setprio(0);
  }

  const float l_tot = xor32_sum(l_run);
  if (rec >= 0) {
    // a part of a split tile: the unnormalised record, merged by fwd_merge_kernel
    float* pr = p.part + (int64_t)rec * (64 * D + 128);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<float4*>(pr + row * D + 32 * mt + 8 * g + 4 * h) =
            make_float4(o[mt][4 * g], o[mt][4 * g + 1], o[mt][4 * g + 2], o[mt][4 * g + 3]);
    if (h == 0) *reinterpret_cast<float2*>(pr + 64 * D + 2 * row) = make_float2(m_b, l_tot);
    return;
  }
  if (!row_ok) return;
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  T* orow = reinterpret_cast<T*>(a.out) + (int64_t)b * a.o_sb + (int64_t)(q0 + t0 + row) * a.o_st +
            (int64_t)hq * a.o_sh;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * mt + 8 * g + 4 * h;
      if constexpr (F32) {
        *reinterpret_cast<float4*>(orow + d0) =
            make_float4(o[mt][4 * g] * inv, o[mt][4 * g + 1] * inv, o[mt][4 * g + 2] * inv, o[mt][4 * g + 3] * inv);
      } else {
        uint2 w;
        w.x = M::pack2(o[mt][4 * g] * inv, o[mt][4 * g + 1] * inv);
        w.y = M::pack2(o[mt][4 * g + 2] * inv, o[mt][4 * g + 3] * inv);
        *reinterpret_cast<uint2*>(orow + d0) = w;
      }
    }
  if (!PAGED && a.lse && h == 0)
    a.lse[(int64_t)b * a.lse_sb + (int64_t)(t0 + row) * a.lse_st + (int64_t)hq * a.lse_sh] =
        l_tot > 0.f ? (m_b + log2f(l_tot)) * kLn2 : -INFINITY;
}

// Combines the nsplit (<= 4) part records of each split tile: m = max m_p,
// O = sum 2^(m_p - m) O_p, l = sum 2^(m_p - m) l_p, out = O / l in the input
// dtype, lse = (m + log2 l) ln 2.  A row with no keys in any part (l = 0)
// writes zeros and lse = -inf, as the unsplit kernel does.  Four workgroups
// per tile (16 rows each), 16 threads per row, every part's loads issued
// before the combine.
template <typename T, int D>
__global__ __launch_bounds__(256) void fwd_merge_kernel(FwdK p) {
  using M = Mfma<T>;
  constexpr int TPR = 16, DPT = D / TPR;         // threads per row, dims per thread (8 or 4)
  constexpr int REC = 64 * D + 128;              // floats per part record
  const srswa_fwd_args& a = p.a;
  const int ti = (int)blockIdx.x >> 2;
  const int lid = p.nlogical - p.ntail + ti;
  const int tile = lid % p.ntiles, bh = lid / p.ntiles;
  const int hq = bh % a.HQ, b = bh / a.HQ;
  const int t0 = tile * kTileRows;
  const int nrows = min(kTileRows, a.T - t0);
  const int r = 16 * ((int)blockIdx.x & 3) + (int)threadIdx.x / TPR, c = (int)threadIdx.x % TPR;
  if (r >= nrows) return;
  const float* rec = p.part + (int64_t)ti * p.nsplit * REC;
  float2 ml[4];
  float4 ov[4][DPT / 4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const bool live = q < p.nsplit;
    const float* pq = rec + (int64_t)(live ? q : 0) * REC;
    ml[q] = live ? *reinterpret_cast<const float2*>(pq + 64 * D + 2 * r) : make_float2(-INFINITY, 0.f);
#pragma unroll
    for (int d = 0; d < DPT / 4; ++d)
      ov[q][d] = live ? reinterpret_cast<const float4*>(pq + r * D + c * DPT)[d] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const float mx = fmaxf(fmaxf(ml[0].x, ml[1].x), fmaxf(ml[2].x, ml[3].x));
  float l = 0.f, acc[DPT];
#pragma unroll
  for (int d = 0; d < DPT; ++d) acc[d] = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float w = ml[q].x == -INFINITY ? 0.f : exp2f(ml[q].x - mx);
    l += ml[q].y * w;
#pragma unroll
    for (int d = 0; d < DPT / 4; ++d) {
      acc[4 * d] += w * ov[q][d].x;
      acc[4 * d + 1] += w * ov[q][d].y;
      acc[4 * d + 2] += w * ov[q][d].z;
      acc[4 * d + 3] += w * ov[q][d].w;
    }
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  T* orow = reinterpret_cast<T*>(a.out) + (int64_t)b * a.o_sb + (int64_t)(t0 + r) * a.o_st + (int64_t)hq * a.o_sh +
            c * DPT;
  if constexpr (std::is_same<T, float>::value) {
#pragma unroll
    for (int d = 0; d < DPT / 4; ++d)
      reinterpret_cast<float4*>(orow)[d] =
          make_float4(acc[4 * d] * inv, acc[4 * d + 1] * inv, acc[4 * d + 2] * inv, acc[4 * d + 3] * inv);
  } else if constexpr (DPT == 8) {
    *reinterpret_cast<uint4*>(orow) =
        make_uint4(M::pack2(acc[0] * inv, acc[1] * inv), M::pack2(acc[2] * inv, acc[3] * inv),
                   M::pack2(acc[4] * inv, acc[5] * inv), M::pack2(acc[6] * inv, acc[7] * inv));
  } else {
    *reinterpret_cast<uint2*>(orow) = make_uint2(M::pack2(acc[0] * inv, acc[1] * inv), M::pack2(acc[2] * inv, acc[3] * inv));
  }
  if (c == 0 && a.lse)
    a.lse[(int64_t)b * a.lse_sb + (int64_t)(t0 + r) * a.lse_st + (int64_t)hq * a.lse_sh] =
        l > 0.f ? (mx + log2f(l)) * kLn2 : -INFINITY;
}

bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int check_fwd(const srswa_fwd_args* a) {
  if (!a || !a->q || !a->k || !a->v || !a->out || (!a->idx && a->S > 0)) {
    set_error("fwd: null argument");
    return SRSWA_INVALID;
  }
  if (a->B < 0 || a->T < 0 || a->Sk < a->T || a->HQ <= 0 || a->HKV <= 0 || a->HI <= 0 || a->S < 0 ||
      a->block_size <= 0 || a->local_window <= 0) {
    set_error("fwd: bad sizes (need Sk >= T)");
    return SRSWA_INVALID;
  }
  if (a->HQ % a->HKV || a->HQ % a->HI) {
    set_error("fwd: HQ must be a multiple of HKV and HI");
    return SRSWA_UNSUPPORTED;
  }
  if (a->dtype != SRSWA_BF16 && a->dtype != SRSWA_F16 && a->dtype != SRSWA_F32) {
    set_error("fwd: dtype %d not supported (bf16, fp16, fp32)", a->dtype);
    return SRSWA_UNSUPPORTED;
  }
  if (!(a->D == 64 || a->D == 128)) {
    set_error("fwd: head dim %d not supported (64, 128)", a->D);
    return SRSWA_UNSUPPORTED;
  }
  const int es = a->dtype == SRSWA_F32 ? 4 : 2;   // element bytes
  if (a->block_size < 16 || (a->block_size & (a->block_size - 1)) || a->S > 64) {
    set_error("fwd: block size must be a power of two >= 16, at most 64 slots");
    return SRSWA_UNSUPPORTED;
  }
  if (ceil_div(a->Sk, kChunk) > 65536) {
    set_error("fwd: key length above 4M");
    return SRSWA_UNSUPPORTED;
  }
  // K / V of one (sequence, kv head) are addressed with 32-bit byte offsets
  const int64_t span = ((int64_t)ceil_div(a->Sk, kChunk) * kChunk * std::max(a->k_st, a->v_st) + a->D) * es;
  if (span >= ((int64_t)1 << 32)) {
    set_error("fwd: one sequence's K / V span 4 GiB or more");
    return SRSWA_UNSUPPORTED;
  }
  const int64_t st[] = {a->q_sb, a->q_st, a->q_sh, a->k_sb, a->k_st, a->k_sh, a->v_sb, a->v_st,
                        a->v_sh, a->o_sb, a->o_st, a->o_sh};
  for (int64_t s : st)
    if ((s * es) % 16) {
      set_error("fwd: rows must be 16-byte aligned");
      return SRSWA_UNSUPPORTED;
    }
  if (!al16(a->q) || !al16(a->k) || !al16(a->v) || !al16(a->out)) {
    set_error("fwd: pointers must be 16-byte aligned");
    return SRSWA_UNSUPPORTED;
  }
  return SRSWA_OK;
}

template <typename T, int D, bool PAGED, bool FP8 = false>
int launch_fwd(const FwdK& k, size_t smem, hipStream_t st) {
  static LdsGrant granted;
  if (!ensure_dynamic_lds(&fwd_kernel<T, D, PAGED, FP8>, smem, &granted)) return SRSWA_UNSUPPORTED;
  hipLaunchKernelGGL((fwd_kernel<T, D, PAGED, FP8>), dim3((unsigned)(8 * k.per_xcd + 8 * k.per_xcd_p)), dim3(128),
                     smem, st, k);
  if constexpr (!PAGED)
    if (k.ntail > 0) hipLaunchKernelGGL((fwd_merge_kernel<T, D>), dim3((unsigned)(4 * k.ntail)), dim3(256), 0, st, k);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("fwd launch failed: %s", hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}

}  // namespace
}  // namespace srswa

using namespace srswa;

namespace srswa {
namespace {

// The forward's launch plan (no device work).  Returns SRSWA_OK with k, smem
// and the split's workspace bytes filled in.
int plan_fwd(const srswa_fwd_args* a, FwdK& k, size_t& smem, size_t& ws_bytes) {
  k = FwdK{};
  k.a = *a;
  k.ntiles = ceil_div(a->T, kTileRows);
  const int nchunk = ceil_div(a->Sk, kChunk);
  k.nwords = ceil_div(nchunk, 32);
  k.SP = a->S + 1;
  k.G = a->HQ / a->HKV;
  k.IG = a->HQ / a->HI;
  k.bs_shift = __builtin_ctz((unsigned)a->block_size);
  const int64_t nlogical = (int64_t)a->B * a->HQ * k.ntiles;
  if (nlogical > (int64_t)1 << 30) {
    set_error("fwd: too many query tiles");
    return SRSWA_UNSUPPORTED;
  }
  k.nlogical = (int)nlogical;
  // distinct chunks one tile can visit: the selected blocks of 64 rows plus
  // the window span of 64 consecutive rows
  const int64_t per_tile = (int64_t)kTileRows * a->S * (ceil_div(a->block_size, kChunk) + 1) +
                           ceil_div(a->local_window + kTileRows - 1, kChunk) + 1;
  const int umax = (int)std::min<int64_t>(nchunk, per_tile);
  const bool f32 = a->dtype == SRSWA_F32;
  const size_t tile = a->D == 128 ? (f32 ? FwdLds<128, 4>::tileBytes : FwdLds<128>::tileBytes)
                                  : (f32 ? FwdLds<64, 4>::tileBytes : FwdLds<64>::tileBytes);
  const size_t setup = (3 * 64 + 4) * 4 + (size_t)k.nwords * 4;
  size_t n = std::max(tile, setup);
  k.chunks_off = (int)n;
  n += ((size_t)umax * 2 + 15) / 16 * 16;
  k.sid_off = (int)n;
  n += (size_t)64 * k.SP * 4 * (a->bias ? 2 : 1);
  smem = (n + 15) / 16 * 16;
  if (smem > 156 * 1024) {
    set_error("fwd: %zu bytes of LDS needed (key length too large)", smem);
    return SRSWA_UNSUPPORTED;
  }
  // Tail split.  The GPU holds `slots` workgroups at once (four per CU at two
  // waves per SIMD, fewer when LDS runs out).  When the last round of tiles
  // fills at most a fifth of them, its tiles run as four workgroups each over
  // quarters of their chunk plans, so that round takes about a quarter of a
  // tile's time.  A fuller last round is left whole: each part pays the
  // tile's set-up and first-load latency again, and its fp32 record costs
  // 8x the tile's output bytes, which outweighs the shorter round.  Measured
  // (4 x 10 heads, 65536 keys, D 128): 80 tiles 39.5 -> 27.6 us, 200 tiles
  // 40.9 -> 38.6 us, 1,040 tiles 110 -> 92 us split; 1,280 tiles on 1,024
  // slots 129 us whole against 134 us split.
  k.nsplit = 1;
  k.ntail = 0;
  ws_bytes = 0;
  const int cus = device_cu_count();
  const int per_cu = std::min<int>(4, (int)((160 * 1024) / smem));
  if (cus > 0 && per_cu > 0) {
    const int64_t slots = (int64_t)cus * per_cu;
    const int64_t rounds = (nlogical + slots - 1) / slots;
    const int64_t tail = nlogical - (rounds - 1) * slots;
    const int64_t f = 4;
    if (tail * 5 <= slots) {
      k.nsplit = (int)f;
      k.ntail = (int)tail;
      ws_bytes = (size_t)tail * f * (64 * a->D + 128) * sizeof(float);
    }
  }
  k.per_xcd = ceil_div(k.nlogical - k.ntail, 8);
  k.per_xcd_p = ceil_div(k.ntail * k.nsplit, 8);
  return SRSWA_OK;
}

}  // namespace
}  // namespace srswa

extern "C" size_t srswa_gather_fwd_workspace(const srswa_fwd_args* a) {
  if (check_fwd(a) != SRSWA_OK || a->B == 0 || a->T == 0) return 0;
  FwdK k;
  size_t smem = 0, ws = 0;
  return plan_fwd(a, k, smem, ws) == SRSWA_OK ? ws : 0;
}

extern "C" int srswa_gather_fwd_ws(const srswa_fwd_args* a, void* ws, size_t ws_bytes, void* stream) {
  int st = check_fwd(a);
  if (st != SRSWA_OK) return st;
  if (a->B == 0 || a->T == 0) return SRSWA_OK;
  FwdK k;
  size_t smem = 0, need = 0;
  st = plan_fwd(a, k, smem, need);
  if (st != SRSWA_OK) return st;
  if (k.ntail > 0 && (!ws || ws_bytes < need || ((uintptr_t)ws & 15u))) {
    // no (usable) workspace: every tile runs whole
    k.nsplit = 1;
    k.ntail = 0;
    k.per_xcd = ceil_div(k.nlogical, 8);
    k.per_xcd_p = 0;
  }
  k.part = reinterpret_cast<float*>(ws);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (a->dtype == SRSWA_F32)
    return a->D == 128 ? launch_fwd<float, 128, false>(k, smem, s) : launch_fwd<float, 64, false>(k, smem, s);
  if (a->dtype == SRSWA_BF16)
    return a->D == 128 ? launch_fwd<bf16_t, 128, false>(k, smem, s) : launch_fwd<bf16_t, 64, false>(k, smem, s);
  return a->D == 128 ? launch_fwd<__half, 128, false>(k, smem, s) : launch_fwd<__half, 64, false>(k, smem, s);
}

extern "C" int srswa_gather_fwd(const srswa_fwd_args* a, void* stream) {
  return srswa_gather_fwd_ws(a, nullptr, 0, stream);
}

extern "C" int srswa_gather_fwd_paged(const srswa_paged_fwd_args* a, void* stream) {
  if (!a || !a->q || !a->k_cache || !a->v_cache || !a->out || !a->block_table || !a->cu_seqlens_q ||
      !a->seq_lens || !a->prefix_lens || (!a->topk && a->S > 0)) {
    set_error("paged fwd: null argument");
    return SRSWA_INVALID;
  }
  if (a->R < 0 || a->max_query_len < 0 || a->HQ <= 0 || a->HKV <= 0 || a->S < 0 || a->max_blocks <= 0 ||
      a->page_size <= 0 || a->local_blocks < 0) {
    set_error("paged fwd: bad sizes");
    return SRSWA_INVALID;
  }
  if (a->R == 0 || a->max_query_len == 0) return SRSWA_OK;
  if (a->HQ % a->HKV) {
    set_error("paged fwd: HQ must be a multiple of HKV");
    return SRSWA_UNSUPPORTED;
  }
  if (a->dtype != SRSWA_BF16 && a->dtype != SRSWA_F16) {
    set_error("paged fwd: matrix-core path takes bf16 / fp16");
    return SRSWA_UNSUPPORTED;
  }
  if (!(a->D == 64 || a->D == 128)) {
    set_error("paged fwd: head dim %d not supported (64, 128)", a->D);
    return SRSWA_UNSUPPORTED;
  }
  if (a->page_size < 16 || (a->page_size & (a->page_size - 1)) || a->S > 64) {
    set_error("paged fwd: page size must be a power of two >= 16, at most 64 slots");
    return SRSWA_UNSUPPORTED;
  }
  const int64_t keys = (int64_t)a->max_blocks * a->page_size;
  if (ceil_div((int)std::min<int64_t>(keys, 1 << 30), kChunk) > 65536 || keys > (1 << 30)) {
    set_error("paged fwd: block table spans more than 4M keys");
    return SRSWA_UNSUPPORTED;
  }
  // the kernel takes a chunk's row max before scaling (max(s) * scale = max(s * scale))
  if (!(a->scale > 0.f) || !std::isfinite(a->scale)) {
    set_error("paged fwd: scale must be positive and finite");
    return SRSWA_UNSUPPORTED;
  }
  const bool fp8 = a->kv_fp8 != 0;
  if (fp8 && (a->kv_fp8 < SRSWA_FP8_E4M3FN || a->kv_fp8 > SRSWA_FP8_E5M2FNUZ)) {
    set_error("paged fwd: kv_fp8 %d is not an fp8 format", a->kv_fp8);
    return SRSWA_UNSUPPORTED;
  }
  const int64_t st[] = {a->q_sn, a->q_sh, a->o_sn, a->o_sh};
  for (int64_t v : st)
    if ((v * 2) % 16) {
      set_error("paged fwd: rows must be 16-byte aligned");
      return SRSWA_UNSUPPORTED;
    }
  // a staged piece is 8 cache elements: 16 bytes, 8 with fp8
  const int64_t kvst[] = {a->k_sp, a->k_st, a->k_sh, a->v_sp, a->v_st, a->v_sh};
  for (int64_t v : kvst)
    if ((v * (fp8 ? 1 : 2)) % (fp8 ? 8 : 16)) {
      set_error("paged fwd: cache rows must be %d-byte aligned", fp8 ? 8 : 16);
      return SRSWA_UNSUPPORTED;
    }
  if (!al16(a->q) || !al16(a->k_cache) || !al16(a->v_cache) || !al16(a->out)) {
    set_error("paged fwd: pointers must be 16-byte aligned");
    return SRSWA_UNSUPPORTED;
  }
  FwdK k{};
  srswa_fwd_args& f = k.a;
  f.q = a->q;  f.q_sb = 0;  f.q_st = a->q_sn;  f.q_sh = a->q_sh;
  f.k = a->k_cache;  f.k_sb = 0;  f.k_st = a->k_st;  f.k_sh = a->k_sh;
  f.v = a->v_cache;  f.v_sb = 0;  f.v_st = a->v_st;  f.v_sh = a->v_sh;
  f.idx = a->topk;  f.idx_sb = 0;  f.idx_sh = a->t_sh;  f.idx_st = a->t_sn;
  f.bias = a->bias;  f.bias_sb = 0;  f.bias_sh = a->b_sh;  f.bias_st = a->b_sn;
  f.seg = nullptr;
  f.out = a->out;  f.o_sb = 0;  f.o_st = a->o_sn;  f.o_sh = a->o_sh;
  f.lse = nullptr;
  f.B = a->R;  f.T = a->max_query_len;  f.Sk = (int)keys;  f.HQ = a->HQ;  f.HKV = a->HKV;  f.HI = a->HKV;
  f.D = a->D;  f.S = a->S;  f.block_size = a->page_size;  f.local_window = a->local_blocks * a->page_size;
  f.scale = a->scale;  f.dtype = a->dtype;
  k.cu = a->cu_seqlens_q;
  k.prefix = a->prefix_lens;
  k.seqlen = a->seq_lens;
  k.bt = a->block_table;
  k.bt_sr = a->bt_sr;
  k.k_pst = a->k_sp;
  k.v_pst = a->v_sp;
  k.kv8 = a->kv_fp8;
  k.ntiles = ceil_div(a->max_query_len, kTileRows);
  const int nchunk = ceil_div((int)keys, kChunk);
  k.nwords = ceil_div(nchunk, 32);
  k.SP = a->S + 1;
  k.G = a->HQ / a->HKV;
  k.IG = k.G;                      // one selection per kv head
  k.bs_shift = __builtin_ctz((unsigned)a->page_size);
  const int64_t nlogical = (int64_t)a->R * a->HQ * k.ntiles;
  if (nlogical > (int64_t)1 << 30) {
    set_error("paged fwd: too many query tiles");
    return SRSWA_UNSUPPORTED;
  }
  k.nlogical = (int)nlogical;
  k.per_xcd = ceil_div(k.nlogical, 8);
  k.nsplit = 1;                    // no tail split: the live tiles depend on device-side lengths
  const int64_t per_tile = (int64_t)kTileRows * a->S * (ceil_div(a->page_size, kChunk) + 1) +
                           ceil_div(f.local_window + kTileRows - 1, kChunk) + 1;
  const int umax = (int)std::min<int64_t>(nchunk, per_tile);
  const size_t tile = a->D == 128 ? FwdLds<128>::tileBytes : FwdLds<64>::tileBytes;
  const size_t setup = (3 * 64 + 4) * 4 + (size_t)k.nwords * 4;
  size_t n = std::max(tile, setup);
  k.chunks_off = (int)n;
  n += ((size_t)umax * 2 + 15) / 16 * 16;
  k.sid_off = (int)n;
  n += (size_t)64 * k.SP * 4 * (a->bias ? 2 : 1);
  // page ids of the visited chunks in the LDS left below 40 KB (four
  // workgroups per CU), or below 52 KB when the rest already exceeds it
  k.ppc = a->page_size >= kChunk ? 1 : 4;
  k.pages_off = (int)((n + 15) / 16 * 16);
  const size_t budget = k.pages_off <= 40 * 1024 - 64 ? 40 * 1024 : 52 * 1024;
  k.page_cap = (int)std::min<int64_t>(umax, k.pages_off < (int)budget ? (budget - k.pages_off) / (4 * k.ppc) : 0);
  n = k.pages_off + (size_t)k.page_cap * 4 * k.ppc;
  const size_t smem = (n + 15) / 16 * 16;
  if (smem > 156 * 1024) {
    set_error("paged fwd: %zu bytes of LDS needed (block table too wide)", smem);
    return SRSWA_UNSUPPORTED;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (fp8) {
    if (a->dtype == SRSWA_BF16)
      return a->D == 128 ? launch_fwd<bf16_t, 128, true, true>(k, smem, s)
                         : launch_fwd<bf16_t, 64, true, true>(k, smem, s);
    return a->D == 128 ? launch_fwd<__half, 128, true, true>(k, smem, s) : launch_fwd<__half, 64, true, true>(k, smem, s);
  }
  if (a->dtype == SRSWA_BF16)
    return a->D == 128 ? launch_fwd<bf16_t, 128, true>(k, smem, s) : launch_fwd<bf16_t, 64, true>(k, smem, s);
  return a->D == 128 ? launch_fwd<__half, 128, true>(k, smem, s) : launch_fwd<__half, 64, true>(k, smem, s);
}
