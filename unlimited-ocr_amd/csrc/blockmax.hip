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

// 16-bit operands, blocks of whole chunks (BS % 64 == 0): one workgroup =
// (sequence, 256 rows, slab of kBm2Slab chunks), four waves of 64 rows.  A
// wave holds two 32-row query tiles, so every K fragment it reads from LDS
// feeds two MFMAs.  K chunks reach LDS by direct-to-LDS buffer loads
// (buffer_load_dwordx4 ... lds) into a three-slot ring: two chunks in flight, no
// staging registers, one barrier per chunk.  A key row is D * 2 bytes without
// padding; its 16-byte pieces are XOR-swizzled so the A-operand reads (32
// keys, one piece each) hit distinct banks.  Block maxima are staged in LDS
// and written once per slab, so no global store sits between the ring's loads
// and the vmcnt waits that count them.
constexpr int kBm2Rows = 256;
constexpr int kBm2Threads = 256;
constexpr int kBm2Slab = 24;        // chunks per slab
constexpr int kBm2Out = kBm2Slab + 1;   // staged maxima: row pitch (odd: no bank conflicts)

template <int D> struct Bm2Layout {
  static constexpr int NP = D / 8;                    // 16-byte pieces per key row
  static constexpr int RPL = 256 / (D * 2);           // key rows per 256 bytes (1 or 2)
  static constexpr int kStage = kChunk * D;           // elements per ring slot
  static constexpr int LPT = kChunk * NP / kBm2Threads;   // direct-to-LDS loads per thread per chunk
  // element offset of piece p of key row r in a slot
  __device__ __forceinline__ static int at(int r, int p) { return r * D + 8 * (p ^ ((r / RPL) % NP)); }
};

// max of three (IEEE maxNum: a quiet NaN operand is ignored, like fmaxf);
// written out because fmaxf on MFMA results first canonicalises every input.
// The compiler's hazard checks do not see into inline asm, so a caller that
// feeds it MFMA results first waits them out with mfma_result_wait().
__device__ __forceinline__ float max3f(float a, float b, float c) {
  float d;
  asm volatile("v_max3_f32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
  return d;
}
// A VALU read of an MFMA result needs the MFMA's passes + 2 wait states; the
// 32x32 16-bit MFMAs take at most 16 passes.  s_nop N waits N + 1 states.
constexpr int kMfmaMaxPasses = 16;
constexpr int kMfmaReadWait = kMfmaMaxPasses + 2;
constexpr int kNopWaits = (7 + 1) + (7 + 1) + (3 + 1);
static_assert(kNopWaits >= kMfmaReadWait, "s_nop sequence shorter than the MFMA read hazard");
// The wait takes one result register of each of the four MFMAs as operands, so
// it cannot be scheduled before any of them has issued; the max3f statements
// are volatile asm too, so they stay after it in program order.
__device__ __forceinline__ void mfma_result_wait(float r0, float r1, float r2, float r3) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" ::"v"(r0), "v"(r1), "v"(r2), "v"(r3));
}

// s_waitcnt vmcnt(N), the other counters left alone (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
template <int N> __device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 16, "vmcnt");
  __builtin_amdgcn_s_waitcnt(N | (0x7 << 4) | (0xF << 8));
}

template <typename T, int D>
__global__ __launch_bounds__(kBm2Threads, 2) void block_max16_kernel(BmaxK p) {
  using L = Bm2Layout<D>;
  using M = Mfma<T>;
  constexpr int NQ = D / 16;
  __shared__ __align__(16) T sK0[L::kStage];
  __shared__ __align__(16) T sK1[L::kStage];
  __shared__ __align__(16) T sK2[L::kStage];
  __shared__ float s_out[kBm2Rows * kBm2Out];     // [row][block of the slab]
  __shared__ int s_maxls;
  const srswa_blockmax_args& a = p.a;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int h = lane / 32, rl = lane % 32;
  const int total = a.B * p.ntiles * p.nslab;
  const int per_xcd = (int)(gridDim.x / 8);
  const int lid = (int)(blockIdx.x & 7) * per_xcd + (int)(blockIdx.x >> 3);
  if (lid >= total) return;
  // tile fastest: one XCD's workgroups score consecutive tiles against the same key slab
  const int tile = lid % p.ntiles;
  const int slab = (lid / p.ntiles) % p.nslab;
  const int b = lid / (p.ntiles * p.nslab);
  const int cpb = a.block_size / kChunk;

  int ls[2], seg[2];
  bool ok[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int row = tile * kBm2Rows + wave * 64 + 32 * rt + rl;
    ok[rt] = row < a.C;
    const int pos = ok[rt] ? a.pos[(int64_t)b * a.pos_sb + (int64_t)row * a.pos_sc] : 0;
    seg[rt] = ok[rt] && a.seg ? a.seg[(int64_t)b * a.seg_sb + (int64_t)row * a.seg_sc] : 0;
    ls[rt] = ok[rt] ? min(max(pos - (a.local_window - 1), 0), a.Sk) : 0;
  }

  // the slab's first two chunks are requested before the rows' extent is known
  // (a chunk past it is loaded for nothing; buffer loads past the keys read zeros)
  const int c_lo = slab * p.slab_chunks;
  const int c_top = min(c_lo + p.slab_chunks, ceil_div(a.Sk, kChunk));
  const T* kg = reinterpret_cast<const T*>(a.k) + (int64_t)b * a.k_sb;
  // the sequence's keys (the host checks that a chunk past them stays < 4 GiB)
  const __amdgpu_buffer_rsrc_t krs =
      make_rsrc(kg, a.Sk > 0 ? (uint32_t)(((int64_t)(a.Sk - 1) * a.k_sk + D) * (int64_t)sizeof(T)) : 0u);
  // load i of this thread fills the slot's 16-byte piece wave * 64 * LPT + 64 i + lane
  // (a wave's load covers 1 KiB of the slot): key row r, swizzled piece
  uint32_t voff[L::LPT];
#pragma unroll
  for (int i = 0; i < L::LPT; ++i) {
    const int piece = (wave * L::LPT + i) * kWave + lane;
    const int r = piece / L::NP, q = piece % L::NP;
    voff[i] = (uint32_t)(((int64_t)r * a.k_sk + 8 * (q ^ ((r / L::RPL) % L::NP))) * (int64_t)sizeof(T));
  }
  const uint32_t chunk_bytes = (uint32_t)((int64_t)kChunk * a.k_sk * (int64_t)sizeof(T));
  auto issue = [&](int c, T* slot) {
    const uint32_t cb = (uint32_t)c * chunk_bytes;
#pragma unroll
    for (int i = 0; i < L::LPT; ++i) {
      const uint32_t off = voff[i] + cb;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          krs, (__attribute__((address_space(3))) void*)(slot + (wave * L::LPT + i) * kWave * 8), 16, off, 0, 0, 0);
    }
  };
  if (c_lo < c_top) issue(c_lo, sK0);
  if (c_lo + 1 < c_top) issue(c_lo + 1, sK1);

  uint4 qf[2][NQ];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int row = tile * kBm2Rows + wave * 64 + 32 * rt + rl;
    const T* qrow = reinterpret_cast<const T*>(a.q) + (int64_t)b * a.q_sb + (int64_t)(ok[rt] ? row : 0) * a.q_sc;
#pragma unroll
    for (int ks = 0; ks < NQ; ++ks)
      qf[rt][ks] = ok[rt] ? *reinterpret_cast<const uint4*>(qrow + 16 * ks + 8 * h) : make_uint4(0, 0, 0, 0);
  }

  // wave-uniform bounds: a chunk inside [wlo, whi) is scored whole by every row of the wave
  const int wlo = wave_max_int(max(ok[0] ? seg[0] : INT_MIN, ok[1] ? seg[1] : INT_MIN));
  const int whi = wave_min_int(min(ok[0] ? ls[0] : INT_MAX, ok[1] ? ls[1] : INT_MAX));
  const int wls = wave_max_int(max(ls[0], ls[1]));
  if (tid == 0) s_maxls = 0;
  for (int i = tid; i < kBm2Rows * kBm2Out; i += kBm2Threads) s_out[i] = -INFINITY;
  __syncthreads();
  if (lane == 0) atomicMax(&s_maxls, wls);
  __syncthreads();
  const int c_hi = min(c_top, ceil_div(s_maxls, kChunk));   // no row has a remote key past this chunk
  const int blk_lo = c_lo / cpb;
  const int blk_hi = slab == p.nslab - 1 ? a.nblk : min(a.nblk, (c_lo + p.slab_chunks) / cpb);

  float run[2] = {-INFINITY, -INFINITY};
  int cib = 0, lb = 0;                            // chunk inside the open block, its slab-local index
  float* srow = s_out + (wave * 64 + 32 * h + rl) * kBm2Out;   // lane half h stages tile h's row
  auto compute = [&](int c, const T* slot) {
    const int j0 = c * kChunk;
    f32x16_t acc[2][2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) acc[rt][0] = acc[rt][1] = zero16();
    // the fragments of step ks + 1 are read before the MFMAs of step ks
    uint4 a0 = *reinterpret_cast<const uint4*>(slot + L::at(rl, h));
    uint4 a1 = *reinterpret_cast<const uint4*>(slot + L::at(32 + rl, h));
#pragma unroll
    for (int ks = 0; ks < NQ; ++ks) {
      uint4 n0 = a0, n1 = a1;
      if (ks + 1 < NQ) {
        n0 = *reinterpret_cast<const uint4*>(slot + L::at(rl, 2 * (ks + 1) + h));
        n1 = *reinterpret_cast<const uint4*>(slot + L::at(32 + rl, 2 * (ks + 1) + h));
      }
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        acc[rt][0] = M::mac(a0, qf[rt][ks], acc[rt][0]);
        acc[rt][1] = M::mac(a1, qf[rt][ks], acc[rt][1]);
      }
      a0 = n0;
      a1 = n1;
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);     // DS reads of step 0
#pragma unroll
    for (int ks = 0; ks < NQ; ++ks) {
      if (ks + 1 < NQ) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);   // step ks + 1's reads
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);                    // step ks's MFMAs
    }
    if (j0 >= wlo && j0 + kChunk <= whi) {
      mfma_result_wait(acc[0][0][15], acc[0][1][15], acc[1][0][15], acc[1][1][15]);
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        float mx = max3f(run[rt], acc[rt][0][0], acc[rt][1][0]);
#pragma unroll
        for (int r = 1; r < 16; ++r) mx = max3f(mx, acc[rt][0][r], acc[rt][1][r]);
        run[rt] = mx;
      }
    } else {
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        // key offset 32 half + 8 (r / 4) + 4 h + r % 4 of the chunk is kept when
        // seg <= j0 + offset < ls; the bounds pass an empty asm so the compiler
        // keeps this rare path's arithmetic inside the branch
        int lo = seg[rt] - j0 - 4 * h, hi = ls[rt] - j0 - 4 * h;
        asm volatile("" : "+v"(lo), "+v"(hi));
        float mx = run[rt];
#pragma unroll
        for (int r = 0; r < 16; ++r)
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            const int off = 32 * half + 8 * (r >> 2) + (r & 3);
            if (off >= lo && off < hi) mx = fmaxf(mx, acc[rt][half][r]);
          }
        run[rt] = mx;
      }
    }
    if (++cib == cpb || c == c_hi - 1) {
      // both lane halves end with both tiles' maxima; half h stages tile h
      const float m0 = xor32_max(run[0]), m1 = xor32_max(run[1]);
      srow[lb] = h ? m1 : m0;
      run[0] = run[1] = -INFINITY;
      cib = 0;
      ++lb;
    }
  };
  // one step: chunk c's loads landed for every thread, slot `nxt` (read two
  // steps ago) refilled with chunk c + 2, chunk c scored from slot `cur`
  auto step = [&](int c, const T* cur, T* nxt) {
    // chunk c + 1 is in flight (issued after chunk c) when the prologue asked for
    // it or, later, when it lies before c_hi
    if (c == c_lo ? c_lo + 1 < c_top : c + 1 < c_hi) wait_vm<L::LPT>(); else wait_vm<0>();
    // an execution barrier only: the wait above already covers this thread's
    // ring loads, and __syncthreads()'s fence would also wait for the chunk
    // still in flight (LDS-DMA counts as an LDS store); the empty asm keeps
    // the compiler from moving LDS accesses across it
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (c + 2 < c_hi) issue(c + 2, nxt);
    compute(c, cur);
  };
  for (int c = c_lo; c < c_hi; c += 3) {
    step(c, sK0, sK2);
    if (c + 1 >= c_hi) break;
    step(c + 1, sK1, sK0);
    if (c + 2 >= c_hi) break;
    step(c + 2, sK2, sK1);
  }
  wait_vm<0>();      // a speculative chunk still in flight must land before the workgroup ends
  __syncthreads();
  // the slab's blocks: 16 lanes per row; blocks past the staged ones (the last
  // slab's tail when nblk exceeds the keys) hold no key
  const int nb = blk_hi - blk_lo;
  const int sb = p.slab_chunks / cpb;
  for (int k = tid & 15; k < nb; k += 16)
    for (int rw = tid >> 4; rw < kBm2Rows; rw += kBm2Threads / 16) {
      const int row = tile * kBm2Rows + rw;
      if (row < a.C)
        a.out[(int64_t)b * a.o_sb + (int64_t)row * a.o_sc + (int64_t)(blk_lo + k) * a.o_sn] =
            k < sb ? s_out[rw * kBm2Out + k] : -INFINITY;
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
  // the ring kernel addresses one sequence's keys with 32-bit byte offsets
  const bool keys32 = ((int64_t)(a->Sk + kChunk) * a->k_sk + a->D) * eb < ((int64_t)1 << 32);
  if (a->dtype != SRSWA_F32 && BS % kChunk == 0 && keys32) {
    // 16-bit operands, whole-chunk blocks: the ring kernel (slabs of kBm2Slab chunks)
    k.ntiles = ceil_div(a->C, kBm2Rows);
    k.slab_chunks = cpb * ceil_div(kBm2Slab, cpb);
    k.nslab = std::max(1, ceil_div(ceil_div(a->Sk, kChunk), k.slab_chunks));
    const int64_t total = (int64_t)a->B * k.ntiles * k.nslab;
    if (total > 0x7ffffff0) {
      set_error("block max: grid too large");
      return SRSWA_UNSUPPORTED;
    }
    const dim3 grid((unsigned)((total + 7) / 8 * 8));
    if (a->dtype == SRSWA_BF16) {
      if (a->D == 128) hipLaunchKernelGGL((block_max16_kernel<bf16_t, 128>), grid, dim3(kBm2Threads), 0, s, k);
      else hipLaunchKernelGGL((block_max16_kernel<bf16_t, 64>), grid, dim3(kBm2Threads), 0, s, k);
    } else {
      if (a->D == 128) hipLaunchKernelGGL((block_max16_kernel<__half, 128>), grid, dim3(kBm2Threads), 0, s, k);
      else hipLaunchKernelGGL((block_max16_kernel<__half, 64>), grid, dim3(kBm2Threads), 0, s, k);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
      set_error("block max launch failed: %s", hipGetErrorString(e));
      return SRSWA_LAUNCH;
    }
    return SRSWA_OK;
  }
  if (a->dtype == SRSWA_BF16) return a->D == 128 ? launch_bmax<bf16_t, 128>(k, s) : launch_bmax<bf16_t, 64>(k, s);
  if (a->dtype == SRSWA_F32) return a->D == 128 ? launch_bmax<float, 128>(k, s) : launch_bmax<float, 64>(k, s);
  return a->D == 128 ? launch_bmax<__half, 128>(k, s) : launch_bmax<__half, 64>(k, s);
}
