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
// instead of once per row.  Per chunk: K (row pitch D+8) and V^T (pitch 72)
// are staged in LDS, S^T = K Q^T and O^T += V^T P^T run on
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

struct FwdSmem {
  static size_t bytes(int D, int S, bool bias, int nwords, int umax, int esz) {
    size_t n = (size_t)kChunk * (D + 8) * esz + (size_t)D * (kChunk + 8) * esz;
    n += 3 * 64 * 4 + (size_t)64 * S * 4 * (bias ? 2 : 1) + (size_t)nwords * 4 + (size_t)umax * 4 + 16;
    return (n + 15) / 16 * 16;
  }
};

template <typename T, int D>
__global__ __launch_bounds__(128) void fwd_kernel(FwdK p) {
  using M = Mfma<T>;
  constexpr int KP = D + 8;          // K row pitch (elements)
  constexpr int VP = kChunk + 8;     // V^T row pitch
  constexpr int KS = D / 16;         // k-steps over the head dim
  constexpr int MT = D / 32;         // 32-row tiles of O^T
  extern __shared__ __align__(16) unsigned char smem[];
  const srswa_fwd_args& a = p.a;
  T* sK = reinterpret_cast<T*>(smem);
  T* sVt = sK + kChunk * KP;
  int* s_qi = reinterpret_cast<int*>(sVt + D * VP);
  int* s_seg = s_qi + 64;
  int* s_ls = s_seg + 64;
  int* s_ids = s_ls + 64;
  float* s_bias = reinterpret_cast<float*>(s_ids + 64 * a.S);
  uint32_t* s_bits = reinterpret_cast<uint32_t*>(s_bias + (a.bias ? 64 * a.S : 0));
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

  for (int r = tid; r < 64; r += blockDim.x) {
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
  for (int e = tid; e < 64 * S; e += blockDim.x) {
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
  for (int w = tid; w < p.nwords; w += blockDim.x) s_bits[w] = 0u;
  __syncthreads();
  const int U = build_chunk_plan(s_qi, s_seg, s_ls, s_ids, S, BS, nrows, p.nchunk, p.nwords,
                                 s_bits, s_chunks, s_count, LW, a.Sk);

  // this lane's row and its pre-scaled q fragments (B operand of S^T = K Q^T)
  const int row = wave * 32 + rl;
  const bool row_ok = row < nrows;
  const int my_qi = s_qi[row], my_seg = s_seg[row], my_ls = s_ls[row];
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
  constexpr int PIECES = kChunk * D / 8;     // 16-byte pieces per chunk and tensor

  for (int u = 0; u < U; ++u) {
    const int c = s_chunks[u];
    const int j0 = c * kChunk;
    __syncthreads();   // previous chunk fully consumed
    for (int pc = tid; pc < PIECES; pc += blockDim.x) {
      const int key = pc / (D / 8), col = pc % (D / 8);
      const int j = j0 + key;
      uint4 kw = make_uint4(0, 0, 0, 0), vw = make_uint4(0, 0, 0, 0);
      if (j < a.Sk) {
        kw = *reinterpret_cast<const uint4*>(kg + (int64_t)j * a.k_st + col * 8);
        vw = *reinterpret_cast<const uint4*>(vg + (int64_t)j * a.v_st + col * 8);
      }
      *reinterpret_cast<uint4*>(sK + key * KP + col * 8) = kw;
      const uint16_t* vv = reinterpret_cast<const uint16_t*>(&vw);
#pragma unroll
      for (int e = 0; e < 8; ++e) reinterpret_cast<uint16_t*>(sVt)[(col * 8 + e) * VP + key] = vv[e];
    }
    __syncthreads();

    // S^T (keys x rows) for the two 32-key halves of the chunk
    f32x16_t st0 = zero16(), st1 = zero16();
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const uint4 a0 = *reinterpret_cast<const uint4*>(sK + rl * KP + 16 * ks + 8 * h);
      const uint4 a1 = *reinterpret_cast<const uint4*>(sK + (32 + rl) * KP + 16 * ks + 8 * h);
      st0 = M::mac(a0, qf[ks], st0);
      st1 = M::mac(a1, qf[ks], st1);
    }

    // membership of this row in the (<= 5) blocks the chunk overlaps
    const int blo = j0 / BS;
    const int bhi = min(j0 + kChunk - 1, a.Sk - 1) / BS;
    bool memb[5];
    float mbias[5];
#pragma unroll
    for (int q = 0; q < 5; ++q) {
      memb[q] = false;
      mbias[q] = 0.f;
      const int blk = blo + q;
      if (blk <= bhi && row_ok) {
        for (int s = 0; s < S; ++s) {
          if (s_ids[row * S + s] == blk) {
            memb[q] = true;
            if (a.bias) mbias[q] = s_bias[row * S + s];
            break;
          }
        }
      }
    }

    float lg[32];
    float mloc = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int key = 32 * half + d_row(r, h);
        const int j = j0 + key;
        const float s = half ? st1[r] : st0[r];
        const bool win = j >= my_ls && j <= my_qi;
        const int q = j / BS - blo;
        bool rem = !win && j >= my_seg && j < my_ls && j <= my_qi;
        float bb = 0.f;
#pragma unroll
        for (int qq = 0; qq < 5; ++qq)
          if (q == qq) { rem = rem && memb[qq]; bb = mbias[qq]; }
        const float x = win ? s * kLog2e : (rem ? (s + bb) * kLog2e : -INFINITY);
        lg[half * 16 + r] = x;
        mloc = fmaxf(mloc, x);
      }
    }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32, kWave));
    const float m_new = fmaxf(m_run, mloc);
    const float alpha = m_new == -INFINITY ? 1.f : exp2f(m_run - m_new);
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const float pv = m_new == -INFINITY ? 0.f : exp2f(lg[i] - m_new);
      lg[i] = pv;
      psum += pv;
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[mt][r] *= alpha;

    // P^T as B operands (4 steps of 16 keys), rounded to the input dtype
    uint4 pb[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const float* src = lg + (ks >> 1) * 16 + 8 * (ks & 1);
      pb[ks] = make_uint4(M::pack2(src[0], src[1]), M::pack2(src[2], src[3]),
                          M::pack2(src[4], src[5]), M::pack2(src[6], src[7]));
    }
    // O^T += V^T P^T
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const T* vrow = sVt + (32 * mt + rl) * VP;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const uint2 lo = *reinterpret_cast<const uint2*>(vrow + 16 * ks + 4 * h);
        const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 16 * ks + 8 + 4 * h);
        o[mt] = M::mac(make_uint4(lo.x, lo.y, hi.x, hi.y), pb[ks], o[mt]);
      }
    }
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
  static bool attr = false;
  if (!attr) {
    hipFuncSetAttribute(reinterpret_cast<const void*>(&fwd_kernel<T, D>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    attr = true;
  }
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
  if (smem > 160 * 1024) {
    set_error("fwd: %zu bytes of LDS needed (key length too large)", smem);
    return SRSWA_UNSUPPORTED;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (a->dtype == SRSWA_BF16)
    return a->D == 128 ? launch_fwd<bf16_t, 128>(k, smem, s) : launch_fwd<bf16_t, 64>(k, smem, s);
  return a->D == 128 ? launch_fwd<__half, 128>(k, smem, s) : launch_fwd<__half, 64>(k, smem, s);
}
