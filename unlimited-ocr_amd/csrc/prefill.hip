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
// Duplicate block ids count once (the first slot's bias is used).
//
// One workgroup = (sequence, query head, 64-row query tile), two waves of 32
// rows.  Set-up builds in LDS the sorted list of 64-key chunks the tile must
// visit (window ranges and selected blocks of all 64 rows, as a bitmap then a
// prefix-popcount compaction), so a tile whose rows share their selection (the
// indexer selects per 64-query tile) visits |selected| + |window| chunks once
// instead of once per row.  Per chunk: K and V (row pitch D+8) are staged in
// LDS, S^T = K Q^T and O^T += V^T P^T (V^T operands read column-wise from the
// natural V tile, bank-conflict free) run on
// v_mfma_f32_32x32x16_{bf16,f16}; q is pre-multiplied by the scale and rounded
// to the input dtype and P is rounded to it before the PV product, the same
// rounding points as the reference kernels (HF/sparse_gather_triton.py:68,94).
#include <algorithm>

#include "mfma_common.h"

namespace srswa {
namespace {

struct FwdK {
  srswa_fwd_args a;
  int ntiles, nchunk, nwords, umax;
  int G, IG;
};

constexpr int kSlotCap = 32;   // planned chunks per tile covered by the slot table

struct FwdSmem {
  static size_t bytes(int D, int S, bool bias, int nwords, int umax, int esz) {
    size_t n = (size_t)kChunk * (D + 8) * esz * 2;                 // K, V (natural)
    n += (size_t)kSlotCap * 64 * 8;                                // slot table
    n += 3 * 64 * 4 + (size_t)64 * S * 4 * (bias ? 2 : 1) + (size_t)nwords * 4 + (size_t)umax * 4 + 16;
    return (n + 15) / 16 * 16;
  }
};

template <typename T, int D>
__global__ __launch_bounds__(128) void fwd_kernel(FwdK p) {
  using M = Mfma<T>;
  constexpr int KP = D + 8;          // K / V row pitch (elements)
  constexpr int KS = D / 16;         // k-steps over the head dim
  constexpr int MT = D / 32;         // 32-row tiles of O^T
  extern __shared__ __align__(16) unsigned char smem[];
  const srswa_fwd_args& a = p.a;
  T* sK = reinterpret_cast<T*>(smem);
  T* sV = sK + kChunk * KP;
  int8_t* s_tab = reinterpret_cast<int8_t*>(sV + kChunk * KP);
  int* s_qi = reinterpret_cast<int*>(s_tab + kSlotCap * 64 * 8);
  int* s_seg = s_qi + 64;
  int* s_ls = s_seg + 64;
  int* s_ids = s_ls + 64;
  float* s_bias = reinterpret_cast<float*>(s_ids + 64 * a.S);
  uint32_t* s_bits = reinterpret_cast<uint32_t*>(s_bias + (a.bias ? 64 * a.S : 0));
  int* s_chunks = reinterpret_cast<int*>(s_bits + p.nwords);
  int* s_count = s_chunks + p.umax;

  constexpr int NT = 128;
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
    if (a.bias) s_bias[e] = bv;
  }
  for (int w = tid; w < p.nwords; w += NT) s_bits[w] = 0u;
  __syncthreads();
  const int U = build_chunk_plan(s_qi, s_seg, s_ls, s_ids, S, BS, nrows, p.nchunk, p.nwords,
                                 s_bits, s_chunks, s_count, LW, a.Sk);
  build_slot_table(s_qi, s_seg, s_ls, s_ids, s_chunks, U, kSlotCap, S, BS, a.Sk, nrows, s_tab);

  // this lane's row: window [ls, qi] and remote range [seg, min(ls, qi+1))
  const int row = wave * 32 + rl;
  const bool row_ok = row < nrows;
  const int my_qi = s_qi[row], my_seg = s_seg[row], my_ls = s_ls[row];
  const uint32_t wlen = (uint32_t)max(my_qi - my_ls + 1, 0);
  const uint32_t rlen = (uint32_t)max(min(my_ls, my_qi + 1) - my_seg, 0);
  uint4 qf[KS];
  {
    const T* qrow = reinterpret_cast<const T*>(a.q) + (int64_t)b * a.q_sb +
                    (int64_t)(t0 + (row_ok ? row : 0)) * a.q_st + (int64_t)hq * a.q_sh;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      uint4 w = row_ok ? *reinterpret_cast<const uint4*>(qrow + 16 * ks + 8 * h) : make_uint4(0, 0, 0, 0);
      uint32_t* ww = reinterpret_cast<uint32_t*>(&w);
#pragma unroll
      for (int e = 0; e < 4; ++e) ww[e] = M::pack2(M::lo(ww[e]) * a.scale, M::hi(ww[e]) * a.scale);
      qf[ks] = w;
    }
  }

  f32x16_t o[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) o[mt] = zero16();
  float m_run = -INFINITY, l_run = 0.f;

  const T* kg = reinterpret_cast<const T*>(a.k) + (int64_t)b * a.k_sb + (int64_t)kvh * a.k_sh;
  const T* vg = reinterpret_cast<const T*>(a.v) + (int64_t)b * a.v_sb + (int64_t)kvh * a.v_sh;
  // chunk staging: every thread owns PPT 16-byte pieces of K and of V; the next
  // chunk's pieces are fetched into registers while the current one computes
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
  const bool one_blk = (BS % kChunk) == 0;      // every chunk lies inside one block
  const bool sub_blk = (kChunk % BS) == 0;      // every chunk holds 64/BS whole blocks
  const int bs_shift = __ffs(BS) - 1;

  if (U > 0) fetch(s_chunks[0]);
  for (int u = 0; u < U; ++u) {
    const int c = s_chunks[u];
    const int j0 = c * kChunk;
    __syncthreads();   // previous chunk fully consumed
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int pc = tid + i * NT;
      const int key = pc / (D / 8), col = pc % (D / 8);
      *reinterpret_cast<uint4*>(sK + key * KP + col * 8) = kpre[i];
      *reinterpret_cast<uint4*>(sV + key * KP + col * 8) = vpre[i];
    }
    __syncthreads();
    if (u + 1 < U) fetch(s_chunks[u + 1]);

    // S^T (keys x rows) for the two 32-key halves of the chunk
    f32x16_t st[2] = {zero16(), zero16()};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const uint4 a0 = *reinterpret_cast<const uint4*>(sK + rl * KP + 16 * ks + 8 * h);
      const uint4 a1 = *reinterpret_cast<const uint4*>(sK + (32 + rl) * KP + 16 * ks + 8 * h);
      st[0] = M::mac(a0, qf[ks], st[0]);
      st[1] = M::mac(a1, qf[ks], st[1]);
    }

    // this row's selected blocks among the (<= 5) the chunk overlaps
    const int blo = j0 / BS;
    bool memb[5];
    float mbias[5];
    if (u < kSlotCap) {
      const uint2 tw = *reinterpret_cast<const uint2*>(s_tab + (u * 64 + row) * 8);
      const int8_t* t8 = reinterpret_cast<const int8_t*>(&tw);
#pragma unroll
      for (int q = 0; q < 5; ++q) {
        memb[q] = t8[q] >= 0;
        mbias[q] = (a.bias && memb[q]) ? s_bias[row * S + t8[q]] : 0.f;
      }
    } else {
      const int nq = min(j0 + kChunk - 1, a.Sk - 1) / BS - blo + 1;
#pragma unroll
      for (int q = 0; q < 5; ++q) {
        memb[q] = false;
        mbias[q] = 0.f;
        if (q < nq && row_ok) {
          for (int s = 0; s < S; ++s)
            if (s_ids[row * S + s] == blo + q) {
              memb[q] = true;
              if (a.bias) mbias[q] = s_bias[row * S + s];
              break;
            }
        }
      }
    }

    // masked logits (log2 domain) in place, row max over the chunk
    float mloc = -INFINITY;
#pragma unroll
    for (int half = 0; half < 2; ++half)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int offk = 32 * half + d_row(r, h);
        const int j = j0 + offk;
        const bool win = (uint32_t)(j - my_ls) < wlen;
        bool rem = (uint32_t)(j - my_seg) < rlen;
        float bb;
        if (one_blk) {
          rem = rem && memb[0];
          bb = mbias[0];
        } else {
          const int qb = sub_blk ? (offk >> bs_shift) : (j / BS - blo);
          bb = 0.f;
          bool mm = false;
#pragma unroll
          for (int qq = 0; qq < 5; ++qq)
            if (qb == qq) { mm = memb[qq]; bb = mbias[qq]; }
          rem = rem && mm;
        }
        const float x = win ? st[half][r] * kLog2e : (rem ? (st[half][r] + bb) * kLog2e : -INFINITY);
        st[half][r] = x;
        mloc = fmaxf(mloc, x);
      }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32, kWave));
    const float m_new = fmaxf(m_run, mloc);
    const float alpha = m_new == -INFINITY ? 1.f : exp2f(m_run - m_new);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    float psum = 0.f;
#pragma unroll
    for (int half = 0; half < 2; ++half)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pv = exp2f(st[half][r] - m_use);
        st[half][r] = pv;
        psum += pv;
      }
    l_run = l_run * alpha + psum;
    m_run = m_new;
    if (alpha != 1.f) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[mt][r] *= alpha;
    }

    // P^T as B operands (4 steps of 16 keys), rounded to the input dtype
    uint4 pb[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int hf = ks >> 1, r0 = 8 * (ks & 1);
      pb[ks] = make_uint4(M::pack2(st[hf][r0], st[hf][r0 + 1]), M::pack2(st[hf][r0 + 2], st[hf][r0 + 3]),
                          M::pack2(st[hf][r0 + 4], st[hf][r0 + 5]), M::pack2(st[hf][r0 + 6], st[hf][r0 + 7]));
    }
    // O^T += V^T P^T  (V^T operands read column-wise from the natural V tile)
    const uint16_t* v16 = reinterpret_cast<const uint16_t*>(sV);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        o[mt] = M::mac(a_operand_t<KP>(v16, 32 * mt + rl, ks, h), pb[ks], o[mt]);
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32, kWave);
  if (!row_ok) return;
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  T* orow = reinterpret_cast<T*>(a.out) + (int64_t)b * a.o_sb + (int64_t)(t0 + row) * a.o_st +
            (int64_t)hq * a.o_sh;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * mt + 8 * g + 4 * h;
      uint2 w;
      w.x = M::pack2(o[mt][4 * g] * inv, o[mt][4 * g + 1] * inv);
      w.y = M::pack2(o[mt][4 * g + 2] * inv, o[mt][4 * g + 3] * inv);
      *reinterpret_cast<uint2*>(orow + d0) = w;
    }
  if (a.lse && h == 0)
    a.lse[(int64_t)b * a.lse_sb + (int64_t)(t0 + row) * a.lse_st + (int64_t)hq * a.lse_sh] =
        l_tot > 0.f ? (m_run + log2f(l_tot)) * kLn2 : -INFINITY;
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
  if (a->dtype != SRSWA_BF16 && a->dtype != SRSWA_F16) {
    set_error("fwd: matrix-core path takes bf16 / fp16");
    return SRSWA_UNSUPPORTED;
  }
  if (!(a->D == 64 || a->D == 128)) {
    set_error("fwd: head dim %d not supported (64, 128)", a->D);
    return SRSWA_UNSUPPORTED;
  }
  if (a->block_size < 16 || a->S > 64) {
    set_error("fwd: block size >= 16 and <= 64 slots required");
    return SRSWA_UNSUPPORTED;
  }
  const int64_t st[] = {a->q_sb, a->q_st, a->q_sh, a->k_sb, a->k_st, a->k_sh, a->v_sb, a->v_st,
                        a->v_sh, a->o_sb, a->o_st, a->o_sh};
  for (int64_t s : st)
    if ((s * 2) % 16) {
      set_error("fwd: rows must be 16-byte aligned");
      return SRSWA_UNSUPPORTED;
    }
  if (!al16(a->q) || !al16(a->k) || !al16(a->v) || !al16(a->out)) {
    set_error("fwd: pointers must be 16-byte aligned");
    return SRSWA_UNSUPPORTED;
  }
  return SRSWA_OK;
}

template <typename T, int D>
int launch_fwd(const FwdK& k, size_t smem, hipStream_t st) {
  static size_t granted = 0;
  if (!ensure_dynamic_lds(&fwd_kernel<T, D>, smem, &granted)) return SRSWA_UNSUPPORTED;
  const int64_t grid = (int64_t)k.a.B * k.a.HQ * k.ntiles;
  hipLaunchKernelGGL((fwd_kernel<T, D>), dim3((unsigned)grid), dim3(128), smem, st, k);
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

extern "C" int srswa_gather_fwd(const srswa_fwd_args* a, void* stream) {
  int st = check_fwd(a);
  if (st != SRSWA_OK) return st;
  if (a->B == 0 || a->T == 0) return SRSWA_OK;
  FwdK k{};
  k.a = *a;
  k.ntiles = ceil_div(a->T, kTileRows);
  k.nchunk = ceil_div(a->Sk, kChunk);
  k.nwords = ceil_div(k.nchunk, 32);
  const int per_row = a->S * (ceil_div(a->block_size, kChunk) + 1) + ceil_div(a->local_window, kChunk) + 1;
  k.umax = (int)std::min<int64_t>((int64_t)k.nchunk, (int64_t)kTileRows * per_row);
  k.G = a->HQ / a->HKV;
  k.IG = a->HQ / a->HI;
  const size_t smem = FwdSmem::bytes(a->D, a->S, a->bias != nullptr, k.nwords, k.umax, 2);
  if (smem > 156 * 1024) {
    set_error("fwd: %zu bytes of LDS needed (key length too large)", smem);
    return SRSWA_UNSUPPORTED;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (a->dtype == SRSWA_BF16)
    return a->D == 128 ? launch_fwd<bf16_t, 128>(k, smem, s) : launch_fwd<bf16_t, 64>(k, smem, s);
  return a->D == 128 ? launch_fwd<__half, 128>(k, smem, s) : launch_fwd<__half, 64>(k, smem, s);
}
