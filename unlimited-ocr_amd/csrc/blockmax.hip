// Fused indexer block-max score on the matrix cores (gfx950).
//
// Replaces _block_max_score_kernel / triton_block_max_score (K4,
// HF/sparse_gather_triton.py:445-524), the fused form of the eager
// "token_future | local_token" masked block amax of DeepseekV2Indexer.forward
// (HF/_sparse_base_impl.py:3076-3094):
//   out[b, c, blk] = max over keys j of blk with seg[b,c] <= j < min(max(pos[b,c]-LW+1, 0), Sk)
//                    of q[b,c] . k[b,j]      (unscaled, fp32 accumulation; -inf if none)
// One workgroup = (sequence, kBmaxRows = 256 query rows, slab of keys); eight
// waves of 32 rows (two per SIMD) share every staged chunk, each lane owning
// one row.  The blocks are independent, so the keys are
// cut into slabs of whole blocks (>= 16 chunks of 64 keys) spread over the
// grid, and every workgroup writes exactly its slab's blocks.  Keys stream in
// 64-key chunks through LDS (the next chunk prefetched into registers), S^T =
// K Q^T on v_mfma_f32_32x32x16; a chunk every row of the wave scores whole
// skips the per-key masking; chunks past the tile's last remote key are
// skipped and their blocks written as -inf.  No dense [B, C, Sk] score tensor
// exists.  fp32 operands (the inference router's fp32 index q / k,
// HF/modeling_deepseekv2.py:419-430) run the same tiling on
// v_mfma_f32_32x32x2_f32: lane half h supplies head-dim elements 8m + 4h .. +3
// of step group m to both operands, from one 16-byte read each.
#include <algorithm>
#include <type_traits>

#include "mfma_common.h"

namespace srswa {
namespace {

constexpr int kBmaxRows = 256;              // query rows per workgroup (8 waves)
constexpr int kBmaxThreads = 2 * kBmaxRows;

struct BmaxK {
  srswa_blockmax_args a;
  int ntiles;
  int nslab, slab_chunks;   // key slabs per (sequence, tile); chunks per slab (whole blocks)
};

// S^T tile (keys x 32 rows) of one 32-key half from the staged chunk
template <typename T, int D> struct BmaxMac {
  static constexpr int EPP = 8;                       // elements per 16-byte piece
  static constexpr int KP = D + 8;
  static constexpr int NQ = D / 16;                   // query fragments (uint4) per lane
  __device__ __forceinline__ static void load_q(uint4* qf, const T* qrow, int h, bool ok) {
#pragma unroll
    for (int ks = 0; ks < NQ; ++ks)
      qf[ks] = ok ? *reinterpret_cast<const uint4*>(qrow + 16 * ks + 8 * h) : make_uint4(0, 0, 0, 0);
  }
  __device__ __forceinline__ static f32x16_t tile(const T* sK, int key, const uint4* qf, int h) {
    f32x16_t s = zero16();
#pragma unroll
    for (int ks = 0; ks < NQ; ++ks)
      s = Mfma<T>::mac(*reinterpret_cast<const uint4*>(sK + key * KP + 16 * ks + 8 * h), qf[ks], s);
    return s;
  }
};
template <int D> struct BmaxMac<float, D> {
  static constexpr int EPP = 4;
  static constexpr int KP = D + 4;
  static constexpr int NQ = D / 8;
  __device__ __forceinline__ static void load_q(uint4* qf, const float* qrow, int h, bool ok) {
#pragma unroll
    for (int m = 0; m < NQ; ++m)
      qf[m] = ok ? *reinterpret_cast<const uint4*>(qrow + 8 * m + 4 * h) : make_uint4(0, 0, 0, 0);
  }
  __device__ __forceinline__ static f32x16_t tile(const float* sK, int key, const uint4* qf, int h) {
    f32x16_t s = zero16();
#pragma unroll
    for (int m = 0; m < NQ; ++m) {
      const float4 kv = *reinterpret_cast<const float4*>(sK + key * KP + 8 * m + 4 * h);
      const float4 qv = __builtin_bit_cast(float4, qf[m]);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, qv.x, s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, qv.y, s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.z, qv.z, s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.w, qv.w, s, 0, 0, 0);
    }
    return s;
  }
};

template <typename T, int D>
__global__ __launch_bounds__(kBmaxThreads) void block_max_kernel(BmaxK p) {
  using MC = BmaxMac<T, D>;
  constexpr int KP = MC::KP;
  constexpr int EPP = MC::EPP;
  __shared__ __align__(16) T sK[kChunk * KP];
  __shared__ int s_maxls;
  const srswa_blockmax_args& a = p.a;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int h = lane / 32, rl = lane % 32;
  const int slab = blockIdx.x % p.nslab;
  const int bt = blockIdx.x / p.nslab;
  const int tile = bt % p.ntiles;
  const int b = bt / p.ntiles;
  const int row = tile * kBmaxRows + wave * 32 + rl;
  const bool row_ok = row < a.C;
  const int BS = a.block_size;

  int ls = 0, seg = 0;
  if (row_ok) {
    const int pos = a.pos[(int64_t)b * a.pos_sb + (int64_t)row * a.pos_sc];
    seg = a.seg ? a.seg[(int64_t)b * a.seg_sb + (int64_t)row * a.seg_sc] : 0;
    // remote keys end at the local window's start and at the last key (j < Sk)
    ls = min(max(pos - (a.local_window - 1), 0), a.Sk);
  }
  if (tid == 0) s_maxls = 0;
  __syncthreads();
  if (row_ok) atomicMax(&s_maxls, ls);
  __syncthreads();
  const int kend = s_maxls;                       // no row has a remote key >= kend
  const int nchunks = ceil_div(kend, kChunk);
  // this slab: chunks [c_lo, c_hi) visited, blocks [blk_lo, blk_hi) written
  const int c_lo = slab * p.slab_chunks;
  const int c_hi = min(c_lo + p.slab_chunks, nchunks);
  const int blk_lo = c_lo * kChunk / BS;
  const int blk_hi = slab == p.nslab - 1 ? a.nblk : min(a.nblk, (c_lo + p.slab_chunks) * kChunk / BS);

  uint4 qf[MC::NQ];
  MC::load_q(qf, reinterpret_cast<const T*>(a.q) + (int64_t)b * a.q_sb + (int64_t)(row_ok ? row : 0) * a.q_sc, h,
             row_ok);
  float* orow = a.out + (int64_t)b * a.o_sb + (int64_t)(row_ok ? row : 0) * a.o_sc;
  const T* kg = reinterpret_cast<const T*>(a.k) + (int64_t)b * a.k_sb;
  constexpr int PR = D / EPP;                     // 16-byte pieces per key row
  constexpr int PPT = kChunk * PR / kBmaxThreads; // per thread
  float run = -INFINITY;                          // running max of the open block (BS >= 64)
  uint4 pre[PPT];
  auto fetch = [&](int c) {
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int pc = tid + kBmaxThreads * i;
      const int j = c * kChunk + pc / PR, col = pc % PR;
      pre[i] = j < a.Sk ? *reinterpret_cast<const uint4*>(kg + (int64_t)j * a.k_sk + col * EPP)
                        : make_uint4(0, 0, 0, 0);
    }
  };

  if (c_lo < c_hi) fetch(c_lo);
  for (int c = c_lo; c < c_hi; ++c) {
    const int j0 = c * kChunk;
    __syncthreads();   // the previous chunk is consumed
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int pc = tid + kBmaxThreads * i;
      *reinterpret_cast<uint4*>(sK + (pc / PR) * KP + (pc % PR) * EPP) = pre[i];
    }
    __syncthreads();
    if (c + 1 < c_hi) fetch(c + 1);
    const f32x16_t s0 = MC::tile(sK, rl, qf, h);
    const f32x16_t s1 = MC::tile(sK, 32 + rl, qf, h);
    // every row of the wave scores the whole chunk: no per-key masks
    const bool whole = __all(!row_ok || (j0 >= seg && j0 + kChunk <= ls));
    if (BS >= kChunk) {
      float mx = -INFINITY;
      if (whole) {
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, fmaxf(s0[r], s1[r]));
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r)
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            const int j = j0 + 32 * half + d_row(r, h);
            if (j >= seg && j < ls) mx = fmaxf(mx, half ? s1[r] : s0[r]);
          }
      }
      run = fmaxf(run, mx);
      const bool closes = ((j0 + kChunk) % BS == 0) || (c == c_hi - 1);
      if (closes) {
        run = fmaxf(run, __shfl_xor(run, 32, kWave));
        const int blk = j0 / BS;
        if (row_ok && h == 0 && blk < a.nblk) orow[(int64_t)blk * a.o_sn] = run;
        run = -INFINITY;
      }
    } else {
      // BS in {16, 32}: 64 / BS whole blocks per chunk
      const int nsub = kChunk / BS;
      for (int sb = 0; sb < nsub; ++sb) {
        float mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r)
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            const int off = 32 * half + d_row(r, h);
            const int j = j0 + off;
            if (off / BS == sb && j >= seg && j < ls) mx = fmaxf(mx, half ? s1[r] : s0[r]);
          }
        mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
        const int blk = j0 / BS + sb;
        if (row_ok && h == 0 && blk < a.nblk) orow[(int64_t)blk * a.o_sn] = mx;
      }
    }
  }
  // the slab's blocks after the last visited chunk hold no remote key of any row
  if (row_ok && h == 0) {
    const int first = c_hi > c_lo ? c_hi * kChunk / BS + ((c_hi * kChunk) % BS ? 1 : 0) : blk_lo;
    for (int blk = max(first, blk_lo); blk < blk_hi; ++blk) orow[(int64_t)blk * a.o_sn] = -INFINITY;
  }
}

template <typename T, int D>
int launch_bmax(const BmaxK& k, hipStream_t st) {
  hipLaunchKernelGGL((block_max_kernel<T, D>), dim3((unsigned)((int64_t)k.a.B * k.ntiles * k.nslab)), dim3(kBmaxThreads), 0, st,
                     k);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("block max launch failed: %s", hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}

}  // namespace
}  // namespace srswa

using namespace srswa;

extern "C" int srswa_block_max_score(const srswa_blockmax_args* a, void* stream) {
  if (!a || !a->q || !a->k || !a->pos || !a->out) {
    set_error("block max: null argument");
    return SRSWA_INVALID;
  }
  if (a->B < 0 || a->C < 0 || a->Sk < 0 || a->nblk < 0 || a->block_size <= 0 || a->local_window <= 0) {
    set_error("block max: bad sizes");
    return SRSWA_INVALID;
  }
  if (a->B == 0 || a->C == 0 || a->nblk == 0) return SRSWA_OK;
  if (a->dtype != SRSWA_BF16 && a->dtype != SRSWA_F16 && a->dtype != SRSWA_F32) {
    set_error("block max: dtype %d not supported (bf16, fp16, fp32)", a->dtype);
    return SRSWA_UNSUPPORTED;
  }
  const int64_t eb = a->dtype == SRSWA_F32 ? 4 : 2;
  if (!(a->D == 64 || a->D == 128)) {
    set_error("block max: head dim %d not supported", a->D);
    return SRSWA_UNSUPPORTED;
  }
  const int BS = a->block_size;
  if (!(BS == 16 || BS == 32 || BS % kChunk == 0)) {
    set_error("block max: block size must be 16, 32 or a multiple of 64");
    return SRSWA_UNSUPPORTED;
  }
  if (((uintptr_t)a->q & 15) || ((uintptr_t)a->k & 15) || (a->q_sb * eb) % 16 || (a->q_sc * eb) % 16 ||
      (a->k_sb * eb) % 16 || (a->k_sk * eb) % 16) {
    set_error("block max: rows must be 16-byte aligned");
    return SRSWA_UNSUPPORTED;
  }
  BmaxK k{};
  k.a = *a;
  k.ntiles = ceil_div(a->C, kBmaxRows);
  // slabs of whole blocks, at least 16 chunks (1024 keys) each
  const int cpb = BS >= kChunk ? BS / kChunk : 1;          // chunks per block
  k.slab_chunks = cpb * ceil_div(16, cpb);
  k.nslab = std::max(1, ceil_div(ceil_div(a->Sk, kChunk), k.slab_chunks));
  if ((int64_t)a->B * k.ntiles * k.nslab > 0x7fffffff) {
    set_error("block max: grid too large");
    return SRSWA_UNSUPPORTED;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (a->dtype == SRSWA_BF16) return a->D == 128 ? launch_bmax<bf16_t, 128>(k, s) : launch_bmax<bf16_t, 64>(k, s);
  if (a->dtype == SRSWA_F32) return a->D == 128 ? launch_bmax<float, 128>(k, s) : launch_bmax<float, 64>(k, s);
  return a->D == 128 ? launch_bmax<__half, 128>(k, s) : launch_bmax<__half, 64>(k, s);
}
