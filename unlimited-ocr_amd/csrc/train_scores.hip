// DASH training block scorers (gfx950), forward and backward.
//
// Replaces the stage-0 scoring of the DASH training router, from the index
// queries / keys the layer's projections, RMSNorms, RoPE and nan_to_num
// produced (those stay the caller's torch ops):
//   DashAttention._block_scores_headcls  HF/dash_attention.py:1053-1143 (stage0 "head_cls", the shipped one)
//   DashAttention._block_scores          HF/dash_attention.py:1005-1050 (stage0 "indexer")
//
// head_cls (fp32 throughout; q, k [B, S, D], position p[i] of query row i):
//   block c holds keys [c BS, min(c BS + BS, S)) (the "valid" ones; none past S)
//   pre_t = (k_t . hc) / sqrt(D), aw_t = clamp(pre_t, +-1e4)
//   m = max over valid aw (0 for a block without keys), e_t = exp(aw_t - m) on valid keys
//   w_t = e_t / max(sum e, 1e-6), kbar_c = nan_to_num(sum_t w_t k_t)
//   z[i, c] = clamp(q_i . kbar_c / sqrt(D), +-1e4)  if c <= p[i] / BS - LB and block c holds a key
//           = -1e9                                   otherwise
// The reference pads the last block with zero keys; exp of a padding logit
// (0 - m) overflows when m < -88.72, and inf * 0 makes that block's k_bar NaN
// (zeroed by nan_to_num) and head_cls's gradient NaN: both kept here.
//
// Backward, for g = d loss / d z as the caller's hook leaves it:
//   dz_raw[i, c] = sanitize(g[i, c] / sqrt(D)) where -1e4 < z[i, c] < 1e4 (kept and
//                  inside the clamp), else 0  (sanitize: nan/inf -> 0, clamp +-1e4: the
//                  reference's hook on the matmul output)
//   dq_i   = sum_c dz_raw[i, c] kbar_c
//   dkbar_c = [kbar_c finite] sum_i dz_raw[i, c] q_i
//   dw_t = dkbar_c . k_t, dden = -[sum e >= 1e-6] sum_t dw_t e_t / max(sum e, 1e-6)^2
//   de_t = dw_t / max(sum e, 1e-6) + dden, ds_t = [|pre_t| <= 1e4] de_t e_t / sqrt(D)
//   dk_t = w_t dkbar_c + ds_t hc,  dhc = sum over every block and key of ds_t k_t
// (the row max m carries sum_t de_t e_t = 0 exactly in real arithmetic; its
// rounding residue is not propagated).
//
// block-max ("indexer" stage 0; fp32 q, k [B, S, D], no scaling):
//   z[i, c] = max over keys j of block c with j <= p[i] - LW of clamp(q_i . k_j, +-1e4),
//             -1e9 when the block holds no such key (and for blocks past the keys)
// Backward (torch's amax rule): the gradient of z[i, c] is split evenly over
// the keys attaining the maximum (count n), and reaches those whose
// unclamped score lies in [-1e4, 1e4]: dq_i += g / n k_j, dk_j += g / n q_i.
// The forward records per (row, block) an int32 code -- the first such key's
// offset, n, and flags for "several keys take the gradient" (their 64-bit mask
// is then written to a side array) and "none does" -- in block-major order.
//
// Kernels: hc_summary_fwd (one workgroup per block, its key rows read once
// into registers), hc_score_fwd (64 query
// rows per workgroup, Z = Q K_bar^T as 32 x 32 fp32 MFMA tiles against groups
// of 64 blocks staged in LDS), hc_score_bwd_dq (dQ = dZ K_bar, one row tile and
// 64 head dims per workgroup), hc_score_bwd_dkbar (dK_bar = dZ^T Q as fp32
// partials per 256-row chunk, one block group and 64 head dims per
// workgroup), hc_summary_bwd (one workgroup per block: the partials summed in
// a fixed chunk order, stage 0 redone, then its backward), and hc_dhc_reduce
// (block partials of d head_cls summed in a fixed order);
// bm_fwd (128 rows per workgroup, 64-key chunks through LDS, S^T = K Q^T on
// v_mfma_f32_32x32x2_f32 as the inference block-max kernel, then per block the
// clamped max, its tie and in-range masks), bm_bwd_dq (4 rows per wave, 16
// waves per 64-row tile, the arg-max key rows of two blocks gathered
// together) and bm_bwd_dk (four keys per wave, 16 lanes each, scanning the
// block's codes in row order).  No atomics: every result is deterministic.
#include <algorithm>
#include <type_traits>

#include "mfma_common.h"
#include "summary.h"

namespace srswa {
namespace {

constexpr int kTsRows = 64;      // query rows per score tile
constexpr int kTsGroup = 64;     // blocks per staged group
constexpr int kTsChunk = 256;    // query rows per d k_bar partial
constexpr int kTsPad = kTsGroup + 1;

__device__ __forceinline__ float clamp_act(float v) { return fminf(fmaxf(v, -kActClamp), kActClamp); }
// nan_to_num(nan=0, posinf=0, neginf=0) then clamp to +-1e4: _sanitize_grad, HF/dash_attention.py:749-755
__device__ __forceinline__ float sanitize(float g) { return isfinite(g) ? clamp_act(g) : 0.f; }

// the last remote block of a query row at position p (none: -1)
__device__ __forceinline__ int last_remote_block(int p, int BS, int LB) { return p >= 0 ? p / BS - LB : -1; }

// ---------------------------------------------------------------- stage 0
// One workgroup (256 threads) per block c of sequence b: nv valid keys
// (nv <= BS), rows at kg, k_st apart.  Each key row is read once, into
// registers: key t belongs to threads TPK t .. TPK t + TPK - 1 (TPK = 256 / BS),
// thread j of them holding the float4 chunks j, j + TPK, j + 2 TPK, ... of the
// row (D / TPK dims; a key's threads read consecutive chunks).  A
// per-key dot product is summed over the key's threads by a butterfly (every
// lane of the key ends with the same bits: each step adds a pair in both
// orders, and fp32 addition commutes); per-dim sums over the keys go through
// an LDS tile of the weighted rows, summed column-wise in key order.
template <int D, int BS> struct HcKeys {
  static constexpr int TPK = 256 / BS, NV4 = D / (4 * TPK);
  // first head dim of this thread's chunk i
  static __device__ __forceinline__ int dim(int i) { return 4 * ((int)threadIdx.x % TPK + TPK * i); }
  float4 v[NV4];
};

template <int D, int BS> struct HcWgLds {
  static constexpr int WP = D + 4;           // row pitch of wk (rows start 4 banks apart)
  float wk[BS * WP];                         // weighted key rows [t][e]
  float hc[128], dkb[128];
  float part[256];                           // slice partials of the chunk sums [NQ][D]
  float red[4];
};

// the block's key rows into registers (rows past nv repeat row nv - 1; they are
// masked wherever they could count)
template <int D, int BS>
__device__ __forceinline__ void load_keys(const float* kg, int64_t k_st, int nv, HcKeys<D, BS>& K) {
  using KS = HcKeys<D, BS>;
  const int t = threadIdx.x / KS::TPK;
  if (nv > 0) {
    const float* row = kg + (int64_t)min(t, nv - 1) * k_st;
#pragma unroll
    for (int i = 0; i < KS::NV4; ++i) K.v[i] = *reinterpret_cast<const float4*>(row + KS::dim(i));
  } else {
#pragma unroll
    for (int i = 0; i < KS::NV4; ++i) K.v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

// k_t . v (v in LDS, D entries) for this thread's key t, on every lane of the key
template <int D, int BS>
__device__ __forceinline__ float key_dot(const HcKeys<D, BS>& K, const float* v) {
  using KS = HcKeys<D, BS>;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < KS::NV4; ++i) {
    const float4 w = *reinterpret_cast<const float4*>(v + KS::dim(i));
    s = fmaf(K.v[i].x, w.x, s);
    s = fmaf(K.v[i].y, w.y, s);
    s = fmaf(K.v[i].z, w.z, s);
    s = fmaf(K.v[i].w, w.w, s);
  }
#pragma unroll
  for (int o = 1; o < KS::TPK; o <<= 1) s += __shfl_xor(s, o, kWave);
  return s;
}

// the workgroup's max / sum of v (waves combined in wave order; every thread
// gets the result)
__device__ __forceinline__ float wg_max(float v, float* red) {
  v = wave_max(v);
  if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  const float r = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  return r;
}
__device__ __forceinline__ float wg_sum(float v, float* red) {
  v = wave_sum(v);
  if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  const float r = ((red[0] + red[1]) + red[2]) + red[3];
  __syncthreads();
  return r;
}

// sum over keys t < nv of coef_t k_t[e] for head dim e = tid (threads tid < D),
// coef_t this thread's key's coefficient, summed in key order
template <int D, int BS>
__device__ __forceinline__ float keys_weighted(const HcKeys<D, BS>& K, int nv, float coef, HcWgLds<D, BS>& L) {
  using KS = HcKeys<D, BS>;
  using LS = HcWgLds<D, BS>;
  float* dst = L.wk + (threadIdx.x / KS::TPK) * LS::WP;
#pragma unroll
  for (int i = 0; i < KS::NV4; ++i)
    *reinterpret_cast<float4*>(dst + KS::dim(i)) =
        make_float4(coef * K.v[i].x, coef * K.v[i].y, coef * K.v[i].z, coef * K.v[i].w);
  __syncthreads();
  float s = 0.f;
  if (threadIdx.x < D)
    for (int u = 0; u < nv; ++u) s += L.wk[u * LS::WP + threadIdx.x];
  __syncthreads();
  return s;
}

struct HcBlockOut {
  float den, rowmax;
  bool pad_overflow;
  float kb;          // kbar_raw of head dim tid (threads tid < D)
  float pre, e, w;   // this thread's key: unclamped logit, exp, weight (0 past nv)
};

// The block's stage-0 forward from the keys in registers: the weighted summary
// kbar_raw, the softmax statistics and the thread's key's logit, exp and weight.
// L.hc holds head_cls.
template <int D, int BS>
__device__ void hc_block_forward(const HcKeys<D, BS>& K, int nv, float isd, HcWgLds<D, BS>& L, HcBlockOut& out) {
  using KS = HcKeys<D, BS>;
  const int t = threadIdx.x / KS::TPK, j = threadIdx.x % KS::TPK;
  const bool valid = t < nv;
  const float dot = key_dot<D, BS>(K, L.hc);
  const float pre = valid ? dot * isd : 0.f;
  const float cl = valid ? clamp_act(pre) : -INFINITY;
  const float mx = wg_max(cl, L.red);
  const float rowmax = nv > 0 ? mx : 0.f;
  const float e = valid ? expf(cl - rowmax) : 0.f;
  const float den = wg_sum(j == 0 ? e : 0.f, L.red);
  const float dn = fmaxf(den, 1e-6f);
  const float w = e / dn;
  out.kb = keys_weighted<D, BS>(K, nv, w, L);
  out.den = den;
  out.rowmax = rowmax;
  out.pre = pre;
  out.e = e;
  out.w = w;
  // a padding key's weight is exp(0 - m) * 0: NaN once exp(-m) overflows
  out.pad_overflow = nv > 0 && nv < BS && isinf(expf(-rowmax));
}

struct HcK {
  srswa_hc_score_args a;
  float isd;
  int ngroups;
};

template <int D, int BS>
__global__ __launch_bounds__(256) void hc_summary_fwd_kernel(HcK p) {
  __shared__ __align__(16) HcWgLds<D, BS> L;
  const srswa_hc_score_args& a = p.a;
  const int b = (int)(blockIdx.x / (unsigned)a.nblk), c = (int)(blockIdx.x % (unsigned)a.nblk);
  const int t0 = c * BS;
  const int nv = max(0, min(BS, a.S - t0));
  HcKeys<D, BS> K;
  load_keys<D, BS>(a.k + (int64_t)b * a.k_sb + (int64_t)t0 * a.k_st, a.k_st, nv, K);
  if (threadIdx.x < D) L.hc[threadIdx.x] = a.head_cls[threadIdx.x];
  __syncthreads();
  HcBlockOut hb;
  hc_block_forward<D, BS>(K, nv, p.isd, L, hb);
  if (threadIdx.x < D)
    a.kbar[(int64_t)b * a.kb_sb + (int64_t)c * D + threadIdx.x] = (isfinite(hb.kb) && !hb.pad_overflow) ? hb.kb : 0.f;
}

// ---------------------------------------------------------------- scores
// the last block holding a key (chunk_valid) and the last one scored
__device__ __forceinline__ int last_valid_block(const srswa_hc_score_args& a) {
  return min(a.nblk - 1, (a.S - 1) / a.block_size);
}

// Workgroup blockIdx.x's work item and part: items are dealt to the 8 XCDs
// round-robin by workgroup index, and the `parts` workgroups of one item go to
// one XCD one after another, so what they share stays in that XCD's L2.
// Launched over ceil(nitems / 8) * 8 * parts workgroups; false past the last item.
__device__ __forceinline__ bool xcd_item(int nitems, int parts, int& item, int& part) {
  const int j = (int)blockIdx.x, x = j % 8, k = j / 8;
  part = k % parts;
  item = (k / parts) * 8 + x;
  return item < nitems;
}

// Scores of 64 query rows per workgroup on fp32 MFMA.  Per group of 64 blocks
// the k_bar rows are staged in LDS (the next group's loaded ahead), and wave w
// computes the 32 x 32 tile of rows 32 (w & 1) .. + 31 against blocks
// 32 (w >> 1) .. + 31 as Q K_bar^T (v_mfma_f32_32x32x2f32; in step group m
// lane half h supplies head dims 8 m + 4 h .. + 3 to both operands), its query
// rows held in registers for the whole tile.  A lane's accumulators are one
// block's scores for 16 rows, so a store instruction writes 32 consecutive
// blocks of two rows.  Waves whose rows reach none of their blocks, and groups
// past the tile's last remote block, store -1e9 without scoring.  Tiles go
// heaviest (last rows) first.
template <int D>
__global__ __launch_bounds__(256) void hc_score_fwd_kernel(HcK p) {
  constexpr int KP = D + 4;                         // k_bar row pitch in LDS
  constexpr int PR = D / 4;                         // 16-byte pieces per k_bar row
  constexpr int PPT = kTsGroup * PR / 256;          // pieces per thread
  __shared__ __align__(16) float s_kb[kTsGroup * KP];
  __shared__ int s_rm[kTsRows];
  __shared__ int s_trm;
  const srswa_hc_score_args& a = p.a;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / kWave), lane = tid % kWave;
  const int h = lane / 32, rl = lane % 32;
  const int ntiles = ceil_div(a.S, kTsRows);
  const int b = (int)(blockIdx.x % (unsigned)a.B), tile = ntiles - 1 - (int)(blockIdx.x / (unsigned)a.B);
  const int row0 = tile * kTsRows;
  const int lastv = last_valid_block(a);
  if (tid < kTsRows) {                              // wave 0: the rows' last scored blocks
    const int row = row0 + tid;
    const int rm = row < a.S ? min(last_remote_block(a.pos[(int64_t)b * a.pos_sb + (int64_t)row * a.pos_st],
                                                     a.block_size, a.local_blocks), lastv)
                             : -1;
    s_rm[tid] = rm;
    const int wm = wave_max_int(rm);
    if (tid == 0) s_trm = wm;
  }
  const int wr = 32 * (wave & 1), wc = 32 * (wave >> 1);
  float4 qf[D / 8];
  {                                                 // rows past S: loaded from row S - 1, never stored
    const float* qrow = a.q + (int64_t)b * a.q_sb + (int64_t)min(row0 + wr + rl, a.S - 1) * a.q_st + 4 * h;
#pragma unroll
    for (int m = 0; m < D / 8; ++m) qf[m] = *reinterpret_cast<const float4*>(qrow + 8 * m);
  }
  // k_bar rows of a group: blocks past nblk read as zero
  const auto rkb = make_rsrc(a.kbar + (int64_t)b * a.kb_sb, (uint32_t)a.nblk * D * 4);
  uint4 pre[PPT];
  auto fetch = [&](int g0) {
#pragma unroll
    for (int i = 0; i < PPT; ++i) pre[i] = buffer_load16(rkb, 4 * ((uint32_t)g0 * D + tid * 4 + 1024 * i), 0);
  };
  lds_barrier();
  const int trm = __builtin_amdgcn_readfirstlane(s_trm);
  int rmv[16];
  int wrm = -1;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    rmv[r] = s_rm[wr + d_row(r, h)];
    wrm = max(wrm, rmv[r]);
  }
  wrm = __builtin_amdgcn_readfirstlane(max(wrm, __shfl_xor(wrm, 32, kWave)));
  const int ngs = trm >= 0 ? trm / kTsGroup + 1 : 0;      // groups holding a scored block
  if (ngs > 0) fetch(0);
  // z through unconditional buffer stores (a conditional store would make each
  // wait for the prefetch wait for every store): the range ends at the tile's
  // last row's last block, so rows past S fall outside it; blocks past nblk
  // are sent past it
  const int nr = min(kTsRows, a.S - row0);
  const auto rzs = make_rsrc(a.z + (int64_t)b * a.z_sb + (int64_t)row0 * a.z_st,
                             (uint32_t)(((int64_t)(nr - 1) * a.z_st + a.nblk) * 4));
  const uint32_t zst4 = 4 * (uint32_t)a.z_st;
  const uint32_t zoff = (uint32_t)(wr + 4 * h) * zst4 + 4 * (uint32_t)(wc + rl);
  for (int gi = 0; gi < p.ngroups; ++gi) {
    const int g0 = gi * kTsGroup, c = g0 + wc + rl;
    f32x16_t s = zero16();
    if (gi < ngs) {
      lds_barrier();                                // the previous group's k_bar is consumed
#pragma unroll
      for (int i = 0; i < PPT; ++i) {
        const int pc = tid + 256 * i;
        *reinterpret_cast<uint4*>(s_kb + (pc / PR) * KP + 4 * (pc % PR)) = pre[i];
      }
      lds_barrier();
      if (gi + 1 < ngs) fetch(g0 + kTsGroup);
      if (g0 + wc <= wrm) {
        const float* kr = s_kb + (wc + rl) * KP + 4 * h;
#pragma unroll
        for (int m = 0; m < D / 8; ++m) {
          const float4 kv = *reinterpret_cast<const float4*>(kr + 8 * m);
          s = __builtin_amdgcn_mfma_f32_32x32x2f32(qf[m].x, kv.x, s, 0, 0, 0);
          s = __builtin_amdgcn_mfma_f32_32x32x2f32(qf[m].y, kv.y, s, 0, 0, 0);
          s = __builtin_amdgcn_mfma_f32_32x32x2f32(qf[m].z, kv.z, s, 0, 0, 0);
          s = __builtin_amdgcn_mfma_f32_32x32x2f32(qf[m].w, kv.w, s, 0, 0, 0);
        }
      }
    }
    const uint32_t off = c < a.nblk ? zoff + 4 * (uint32_t)g0 : 0x80000000u;
#pragma unroll
    for (int r = 0; r < 16; ++r)
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(c <= rmv[r] ? clamp_act(s[r] * p.isd) : kScoreNeg), rzs,
                                            off + (uint32_t)d_row(r, 0) * zst4, 0, 0);
  }
}

// ---------------------------------------------------------------- backward
struct HcBK {
  srswa_hc_score_bwd_args a;
  float isd;
  int nchunks;
  float* dkb_part;     // [nchunks, B, nblk, D]
  float* dhc_part;     // [B, nblk, D]
};

// dz_raw of one (row, block) from g and the forward's z
__device__ __forceinline__ float dz_raw(float g, float z, float isd) {
  return (z > -kActClamp && z < kActClamp) ? sanitize(g * isd) : 0.f;
}

// the rows' last scored blocks (min'd with the last valid block) for rows
// r0 .. r0 + 63, by wave 0: each lane its row, the wave's maximum returned
__device__ __forceinline__ int rows_reach(const srswa_hc_score_bwd_args& a, int b, int row, int lastv) {
  return row < a.S ? min(last_remote_block(a.pos[(int64_t)b * a.pos_sb + (int64_t)row * a.pos_st], a.block_size,
                                           a.local_blocks),
                         lastv)
                   : -1;
}

// dZ of a 64 x 64 (rows x blocks) tile, loaded ahead: a thread's entries are
// rows tid / 64 + 4 i and block tid % 64.  Buffer loads from the tile's first
// row: the range ends at the last row's last block, so rows past S read as
// zero (and give dZ = 0); blocks past nblk are dropped when stored.
constexpr int kZpt = kTsRows * kTsGroup / 256;

struct DzAhead {
  float g[kZpt], z[kZpt];
  __device__ __forceinline__ void fetch(const srswa_hc_score_bwd_args& a, int b, int r0, int g0) {
    const int nr = min(kTsRows, a.S - r0);
    const auto rg = make_rsrc(a.gz + (int64_t)b * a.gz_sb + (int64_t)r0 * a.gz_st + g0,
                              (uint32_t)(((int64_t)(nr - 1) * a.gz_st + a.nblk - g0) * 4));
    const auto rz = make_rsrc(a.z + (int64_t)b * a.z_sb + (int64_t)r0 * a.z_st + g0,
                              (uint32_t)(((int64_t)(nr - 1) * a.z_st + a.nblk - g0) * 4));
    const uint32_t r = threadIdx.x / kTsGroup, c = threadIdx.x % kTsGroup;
#pragma unroll
    for (int i = 0; i < kZpt; ++i) {
      g[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rg, 4 * ((r + 4 * i) * (uint32_t)a.gz_st + c), 0, 0));
      z[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rz, 4 * ((r + 4 * i) * (uint32_t)a.z_st + c), 0, 0));
    }
  }
  // dZ into s_dz[row * pitch + block]
  __device__ __forceinline__ void store(const srswa_hc_score_bwd_args& a, int g0, float isd, float* s_dz,
                                        int pitch) const {
    const int r = threadIdx.x / kTsGroup, c = threadIdx.x % kTsGroup;
    const uint32_t keep = g0 + c < a.nblk ? ~0u : 0u;      // a mask, not a branch
#pragma unroll
    for (int i = 0; i < kZpt; ++i)
      s_dz[(r + 4 * i) * pitch + c] = __uint_as_float(__float_as_uint(dz_raw(g[i], z[i], isd)) & keep);
  }
};

// dQ = dZ K_bar over the remote blocks on fp32 MFMA, one 64-row tile and a
// 64-dim slice of the head dims per workgroup: per group of 64 blocks up to
// the tile's last remote one, dZ (from the upstream gradient and the
// forward's scores) and the slice of the blocks' k_bar rows are staged in
// LDS, the next group's loaded ahead.  Wave w accumulates the 32 x 32 tile of
// rows 32 (w & 1) .. + 31 and slice dims 32 (w >> 1) .. + 31; in step group m
// lane half h supplies blocks 8 m + 4 h .. + 3 (dZ one 16-byte read, k_bar
// single reads whose lane halves fall 32 banks apart).  The D / 64 slices of a
// tile run on one XCD one after another (dZ stays in that L2); tiles go
// heaviest (last rows) first.
template <int D>
__global__ __launch_bounds__(256) void hc_score_bwd_dq_kernel(HcBK p) {
  constexpr int NS = D / 64;                       // dim slices
  constexpr int KBP = 64 + 8;                      // k_bar slice pitch
  constexpr int DZP = kTsGroup + 4;                // dZ row pitch
  constexpr int KPT = kTsGroup * 16 / 256;         // 16-byte k_bar pieces per thread
  __shared__ __align__(16) float s_kb[kTsGroup * KBP];
  __shared__ __align__(16) float s_dz[kTsRows * DZP];
  __shared__ int s_trm;
  const srswa_hc_score_bwd_args& a = p.a;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / kWave), lane = tid % kWave;
  const int h = lane / 32, rl = lane % 32;
  const int ntiles = ceil_div(a.S, kTsRows);
  int item, ds;
  if (!xcd_item(a.B * ntiles, NS, item, ds)) return;
  const int b = item % a.B, tile = ntiles - 1 - item / a.B;
  const int r0 = tile * kTsRows, d0 = 64 * ds;
  const int lastv = min(a.nblk - 1, (a.S - 1) / a.block_size);
  if (tid < kTsRows) {
    const int wm = wave_max_int(rows_reach(a, b, r0 + tid, lastv));
    if (tid == 0) s_trm = wm;
  }
  const int wr = 32 * (wave & 1), wd = 32 * (wave >> 1);
  // the slice of the k_bar rows: blocks past nblk read as zero
  const auto rkb = make_rsrc(a.kbar + (int64_t)b * a.kb_sb + d0, (uint32_t)(a.nblk * D - d0) * 4);
  uint4 kpre[KPT];
  DzAhead dza;
  auto fetch = [&](int g0) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const uint32_t pc = tid + 256 * i;
      kpre[i] = buffer_load16(rkb, 4 * (((uint32_t)g0 + pc / 16) * D + 4 * (pc % 16)), 0);
    }
    dza.fetch(a, b, r0, g0);
  };
  lds_barrier();
  const int trm = __builtin_amdgcn_readfirstlane(s_trm);
  const int ngs = trm >= 0 ? trm / kTsGroup + 1 : 0;
  f32x16_t acc = zero16();
  if (ngs > 0) fetch(0);
  for (int gi = 0; gi < ngs; ++gi) {
    const int g0 = gi * kTsGroup;
    lds_barrier();                                 // the previous group is consumed
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int pc = tid + 256 * i;
      *reinterpret_cast<uint4*>(s_kb + (pc / 16) * KBP + 4 * (pc % 16)) = kpre[i];
    }
    dza.store(a, g0, p.isd, s_dz, DZP);
    lds_barrier();
    if (gi + 1 < ngs) fetch(g0 + kTsGroup);
    // every block of the group (dZ is zero past the rows' reach): a skip per
    // step would split the accumulator chain
    const float* dzr = s_dz + (wr + rl) * DZP + 4 * h;
    const float* kbr = s_kb + 4 * h * KBP + wd + rl;
#pragma unroll
    for (int m = 0; m < kTsGroup / 8; ++m) {
      const float4 d4 = *reinterpret_cast<const float4*>(dzr + 8 * m);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(d4.x, kbr[(8 * m) * KBP], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(d4.y, kbr[(8 * m + 1) * KBP], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(d4.z, kbr[(8 * m + 2) * KBP], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(d4.w, kbr[(8 * m + 3) * KBP], acc, 0, 0, 0);
    }
  }
  float* dq = a.dq + (int64_t)b * a.dq_sb + d0 + wd + rl;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = r0 + wr + d_row(r, h);
    if (row < a.S) dq[(int64_t)row * a.dq_st] = acc[r];
  }
}

// d k_bar partial of one 256-row chunk, 64 blocks and a 64-dim slice of the
// head dims per workgroup on fp32 MFMA: per 64-row sub-chunk whose rows reach
// the group, dZ and the slice of the query rows are staged in LDS (the next
// such sub-chunk loaded ahead).  Wave w accumulates the 32 x 32 tile of
// blocks 32 (w & 1) .. + 31 and slice dims 32 (w >> 1) .. + 31 (dZ^T Q); in
// step group m lane half h supplies rows 8 m + 4 h .. + 3, both operands as
// single reads whose lane halves fall 32 banks apart.  The partial is summed
// over the sub-chunks in row order.  The D / 64 slices of a (chunk, group)
// run on one XCD one after another.
template <int D>
__global__ __launch_bounds__(256) void hc_score_bwd_dkbar_kernel(HcBK p) {
  constexpr int NS = D / 64;
  constexpr int DZP = kTsGroup + 8;                // dZ row pitch
  constexpr int QP = 64 + 8;                       // query slice pitch
  constexpr int QPT = kTsRows * 16 / 256;          // 16-byte query pieces per thread
  constexpr int NSUB = kTsChunk / kTsRows;
  __shared__ __align__(16) float s_q[kTsRows * QP];
  __shared__ __align__(16) float s_dz[kTsRows * DZP];
  __shared__ int s_srm[NSUB];
  const srswa_hc_score_bwd_args& a = p.a;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / kWave), lane = tid % kWave;
  const int h = lane / 32, rl = lane % 32;
  const int ngroups = ceil_div(a.nblk, kTsGroup);
  int item, ds;
  if (!xcd_item(a.B * ngroups * p.nchunks, NS, item, ds)) return;
  const int chunk = item % p.nchunks;
  const int g0 = ((item / p.nchunks) % ngroups) * kTsGroup;
  const int b = item / (p.nchunks * ngroups);
  const int d0 = 64 * ds;
  const int lastv = min(a.nblk - 1, (a.S - 1) / a.block_size);
  {                                                // wave s: sub-chunk s's rows
    const int wm = wave_max_int(rows_reach(a, b, chunk * kTsChunk + tid, lastv));
    if (lane == 0) s_srm[wave] = wm;
  }
  const int wc = 32 * (wave & 1), wd = 32 * (wave >> 1);
  uint4 qpre[QPT];
  DzAhead dza;
  auto fetch = [&](int r0) {          // the sub-chunk's query slice: rows past S read as zero
    const int nr = min(kTsRows, a.S - r0);
    const auto rq = make_rsrc(a.q + (int64_t)b * a.q_sb + (int64_t)r0 * a.q_st + d0,
                              (uint32_t)(((int64_t)(nr - 1) * a.q_st + 64) * 4));
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
      const uint32_t pc = tid + 256 * i;
      qpre[i] = buffer_load16(rq, 4 * ((pc / 16) * (uint32_t)a.q_st + 4 * (pc % 16)), 0);
    }
    dza.fetch(a, b, r0, g0);
  };
  lds_barrier();
  unsigned live = 0;                               // sub-chunks whose rows reach the group
#pragma unroll
  for (int s = 0; s < NSUB; ++s)
    if (chunk * kTsChunk + s * kTsRows < a.S && s_srm[s] >= g0) live |= 1u << s;
  live = __builtin_amdgcn_readfirstlane(live);
  f32x16_t acc = zero16();
  if (live) fetch(chunk * kTsChunk + kTsRows * __builtin_ctz(live));
  while (live) {
    live &= live - 1;                              // this sub-chunk's rows are the ones loaded ahead
    lds_barrier();                                 // the previous sub-chunk is consumed
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
      const int pc = tid + 256 * i;
      *reinterpret_cast<uint4*>(s_q + (pc / 16) * QP + 4 * (pc % 16)) = qpre[i];
    }
    dza.store(a, g0, p.isd, s_dz, DZP);
    lds_barrier();
    if (live) fetch(chunk * kTsChunk + kTsRows * __builtin_ctz(live));
    const float* dzc = s_dz + 4 * h * DZP + wc + rl;
    const float* qc = s_q + 4 * h * QP + wd + rl;
#pragma unroll
    for (int m = 0; m < kTsRows / 8; ++m)
#pragma unroll
      for (int x = 0; x < 4; ++x)
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(dzc[(8 * m + x) * DZP], qc[(8 * m + x) * QP], acc, 0, 0, 0);
  }
  float* dst = p.dkb_part + ((int64_t)chunk * a.B + b) * a.nblk * D + d0 + wd + rl;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int c = g0 + wc + d_row(r, h);
    if (c < a.nblk) dst[(int64_t)c * D] = acc[r];
  }
}

// stage-0 backward, one workgroup per block: d idx_k rows of the block and
// the block's partial of d head_cls (the key rows read once, into registers)
template <int D, int BS>
__global__ __launch_bounds__(256) void hc_summary_bwd_kernel(HcBK p) {
  constexpr int NQ = 256 / D;
  using KS = HcKeys<D, BS>;
  __shared__ __align__(16) HcWgLds<D, BS> L;
  const srswa_hc_score_bwd_args& a = p.a;
  const int tid = threadIdx.x;
  const int b = (int)(blockIdx.x / (unsigned)a.nblk), c = (int)(blockIdx.x % (unsigned)a.nblk);
  const int t0 = c * BS;
  const int nv = max(0, min(BS, a.S - t0));
  HcKeys<D, BS> K;
  load_keys<D, BS>(a.k + (int64_t)b * a.k_sb + (int64_t)t0 * a.k_st, a.k_st, nv, K);
  if (tid < D) L.hc[tid] = a.head_cls[tid];
  {
    // d k_bar: the chunk partials, slice q taking chunks q, q + NQ, ... in
    // order, the slices then added in order
    const int e = tid % D, q = tid / D;
    constexpr int kAhead = 16;
    float acc = 0.f;
    for (int ch0 = q; ch0 < p.nchunks; ch0 += NQ * kAhead) {
      float v[kAhead];
#pragma unroll
      for (int u = 0; u < kAhead; ++u)
        v[u] = p.dkb_part[(((int64_t)min(ch0 + u * NQ, p.nchunks - 1) * a.B + b) * a.nblk + c) * D + e];
#pragma unroll
      for (int u = 0; u < kAhead; ++u)
        if (ch0 + u * NQ < p.nchunks) acc += v[u];
    }
    L.part[q * D + e] = acc;
  }
  __syncthreads();
  float dkb = 0.f;
  if (tid < D) {
    dkb = L.part[tid];
#pragma unroll
    for (int r = 1; r < NQ; ++r) dkb += L.part[r * D + tid];
  }
  __syncthreads();
  HcBlockOut hb;
  hc_block_forward<D, BS>(K, nv, p.isd, L, hb);
  // nan_to_num(k_bar) passes no gradient where k_bar_raw is not finite
  if (tid < D) L.dkb[tid] = (!isfinite(hb.kb) || hb.pad_overflow) ? 0.f : dkb;
  __syncthreads();
  const int t = tid / KS::TPK, j = tid % KS::TPK;
  const bool valid = t < nv;
  const float dn = fmaxf(hb.den, 1e-6f);
  const float dw = key_dot<D, BS>(K, L.dkb);                 // dw_t = dkbar . k_t
  const float se = wg_sum((valid && j == 0) ? dw * hb.e : 0.f, L.red);
  const float dden = hb.den >= 1e-6f ? -se / (dn * dn) : 0.f;
  float ds = 0.f;
  if (valid) {
    const float de = dw / dn + dden;
    ds = (hb.pre >= -kActClamp && hb.pre <= kActClamp) ? de * hb.e * p.isd : 0.f;
  }
  const float dh = keys_weighted<D, BS>(K, nv, ds, L);       // the block's d head_cls
  if (tid < D) p.dhc_part[((int64_t)b * a.nblk + c) * D + tid] = hb.pad_overflow ? __builtin_nanf("") : dh;
  if (valid) {                                               // this thread's dims of d k_t
    float* dst = a.dk + (int64_t)b * a.dk_sb + (int64_t)(t0 + t) * a.dk_st;
#pragma unroll
    for (int i = 0; i < KS::NV4; ++i) {
      const int e0 = KS::dim(i);
      float o[4];
#pragma unroll
      for (int x = 0; x < 4; ++x) o[x] = hb.pad_overflow ? 0.f : fmaf(hb.w, L.dkb[e0 + x], ds * L.hc[e0 + x]);
      *reinterpret_cast<float4*>(dst + e0) = make_float4(o[0], o[1], o[2], o[3]);
    }
  }
}

// d head_cls: a workgroup per 16 head dims; sixteen interleaved slices of the
// block partials, each summed in block order, then the slice sums in slice
// order (fixed order)
constexpr int kDhcDims = 16, kDhcParts = 16;

template <int D>
__global__ __launch_bounds__(kDhcDims * kDhcParts) void hc_dhc_reduce_kernel(HcBK p) {
  __shared__ float s_part[kDhcParts][kDhcDims];
  const int el = threadIdx.x % kDhcDims, part = threadIdx.x / kDhcDims;
  const int e = blockIdx.x * kDhcDims + el;
  const int64_t n = (int64_t)p.a.B * p.a.nblk;
  float s = 0.f;
  constexpr int kAhead = 16;                       // partials loaded together, then added in order
  for (int64_t i0 = part; i0 < n; i0 += (int64_t)kAhead * kDhcParts) {
    float v[kAhead];
#pragma unroll
    for (int u = 0; u < kAhead; ++u) v[u] = p.dhc_part[min(i0 + (int64_t)u * kDhcParts, n - 1) * D + e];
#pragma unroll
    for (int u = 0; u < kAhead; ++u)
      if (i0 + (int64_t)u * kDhcParts < n) s += v[u];
  }
  s_part[part][el] = s;
  __syncthreads();
  if (part == 0) {
    float t = s_part[0][el];
#pragma unroll
    for (int k = 1; k < kDhcParts; ++k) t += s_part[k][el];
    p.a.dhc[e] = t;
  }
}

// ---------------------------------------------------------------- block max
constexpr int kBmRows = 128;                 // query rows per workgroup (4 waves of 32)
constexpr int kBmThreads = 2 * kBmRows;
constexpr int kBmSlab = 16;                  // chunks of 64 keys per workgroup
constexpr int kCodeMulti = 1 << 16;          // several keys take the gradient: mask in the side array
constexpr int kCodeNone = 1 << 17;           // no key takes the gradient

struct BmK {
  srswa_bm_score_args a;
  int ntiles, nslab;
};

// S^T tile (32 keys x 32 rows) from the staged chunk, fp32 operands: lane half
// h supplies head dims 8 m + 4 h .. + 3 of step group m to both operands
template <int D>
__device__ __forceinline__ f32x16_t bm_tile(const float* sK, int key, const float4* qf, int h) {
  constexpr int KP = D + 4;
  f32x16_t s = zero16();
#pragma unroll
  for (int m = 0; m < D / 8; ++m) {
    const float4 kv = *reinterpret_cast<const float4*>(sK + key * KP + 8 * m + 4 * h);
    s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, qf[m].x, s, 0, 0, 0);
    s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, qf[m].y, s, 0, 0, 0);
    s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.z, qf[m].z, s, 0, 0, 0);
    s = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.w, qf[m].w, s, 0, 0, 0);
  }
  return s;
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  const uint32_t lo = __shfl_xor((uint32_t)v, m, kWave), hi = __shfl_xor((uint32_t)(v >> 32), m, kWave);
  return ((uint64_t)hi << 32) | lo;
}

template <int D, int BS>
__global__ __launch_bounds__(kBmThreads, 2) void bm_fwd_kernel(BmK p) {
  constexpr int KP = D + 4;
  constexpr int NSUB = kChunk / BS;
  __shared__ __align__(16) float sK[kChunk * KP];
  __shared__ int s_maxls;
  const srswa_bm_score_args& a = p.a;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / kWave), lane = tid % kWave;
  const int h = lane / 32, rl = lane % 32;
  const int slab = blockIdx.x % p.nslab;
  const int bt = blockIdx.x / p.nslab;
  const int tile = p.ntiles - 1 - bt % p.ntiles;   // heaviest (last rows) first
  const int b = bt / p.ntiles;
  const int row = tile * kBmRows + wave * 32 + rl;
  const bool row_ok = row < a.S;
  int ls = 0;                                   // remote keys: j < ls
  if (row_ok) {
    const int pos = a.pos[(int64_t)b * a.pos_sb + (int64_t)row * a.pos_st];
    ls = min(max(pos - a.local_window + 1, 0), a.S);
  }
  if (tid == 0) s_maxls = 0;
  __syncthreads();
  if (row_ok && h == 0) atomicMax(&s_maxls, ls);
  __syncthreads();
  const int nchunks = ceil_div(s_maxls, kChunk);
  const int c_lo = slab * kBmSlab;
  const int c_hi = min(c_lo + kBmSlab, nchunks);
  const int blk_lo = c_lo * NSUB;
  const int blk_hi = slab == p.nslab - 1 ? a.nblk : min(a.nblk, (c_lo + kBmSlab) * NSUB);

  float4 qf[D / 8];
  {
    const float* qrow = a.q + (int64_t)b * a.q_sb + (int64_t)(row_ok ? row : 0) * a.q_st;
#pragma unroll
    for (int m = 0; m < D / 8; ++m)
      qf[m] = row_ok ? *reinterpret_cast<const float4*>(qrow + 8 * m + 4 * h) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float* zrow = a.z + (int64_t)b * a.z_sb + (int64_t)(row_ok ? row : 0) * a.z_st;
  int32_t* code = a.code + (int64_t)b * a.nblk * a.S + (row_ok ? row : 0);      // [b][blk][row]
  uint64_t* tm = a.tiemask + ((int64_t)b * a.S + (row_ok ? row : 0)) * a.nblk;   // [b][row][blk]
  const float* kg = a.k + (int64_t)b * a.k_sb;
  constexpr int PR = D / 4;                       // 16-byte pieces per key row
  constexpr int PPT = kChunk * PR / kBmThreads;   // per thread
  float4 pre[PPT];
  auto fetch = [&](int c) {
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int pc = tid + kBmThreads * i;
      const int j = c * kChunk + pc / PR, col = pc % PR;
      pre[i] = j < a.S ? *reinterpret_cast<const float4*>(kg + (int64_t)j * a.k_st + 4 * col)
                       : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  if (c_lo < c_hi) fetch(c_lo);
  for (int c = c_lo; c < c_hi; ++c) {
    const int j0 = c * kChunk;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int pc = tid + kBmThreads * i;
      *reinterpret_cast<float4*>(sK + (pc / PR) * KP + (pc % PR) * 4) = pre[i];
    }
    __syncthreads();
    if (c + 1 < c_hi) fetch(c + 1);
    const f32x16_t s0 = bm_tile<D>(sK, rl, qf, h);
    const f32x16_t s1 = bm_tile<D>(sK, 32 + rl, qf, h);
#pragma unroll
    for (int sb = 0; sb < NSUB; ++sb) {
      float mx = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r)
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const int off = 32 * half + d_row(r, h);
          if (off / BS == sb && j0 + off < ls) mx = fmaxf(mx, clamp_act(half ? s1[r] : s0[r]));
        }
      mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
      uint64_t tie = 0, grad = 0;                 // block-relative key bits
#pragma unroll
      for (int r = 0; r < 16; ++r)
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const int off = 32 * half + d_row(r, h);
          if (off / BS == sb && j0 + off < ls) {
            const float raw = half ? s1[r] : s0[r];
            const float cv = clamp_act(raw);
            const uint64_t bit = 1ull << (off - sb * BS);
            if (cv == mx) {
              tie |= bit;
              if (raw == cv) grad |= bit;
            }
          }
        }
      tie |= shfl_xor_u64(tie, 32);
      grad |= shfl_xor_u64(grad, 32);
      const int blk = c * NSUB + sb;
      if (row_ok && h == 0 && blk < a.nblk) {
        const int ng = __popcll(grad);
        int cd = kCodeNone;
        if (ng > 0) cd = (int)__builtin_ctzll(grad) | (__popcll(tie) << 8) | (ng > 1 ? kCodeMulti : 0);
        zrow[blk] = mx == -INFINITY ? kScoreNeg : mx;
        code[(int64_t)blk * a.S] = cd;
        if (ng > 1) tm[blk] = grad;
      }
    }
  }
  // the slab's blocks after the last visited chunk hold no remote key of any row
  if (row_ok && h == 0) {
    for (int blk = max(c_hi > c_lo ? c_hi * NSUB : blk_lo, blk_lo); blk < blk_hi; ++blk) {
      zrow[blk] = kScoreNeg;
      code[(int64_t)blk * a.S] = kCodeNone;
    }
  }
}

// The block-max backward's weights w[b, c, i] = gz[b, i, c] / n (0 where no key
// of block c takes row i's gradient), block-major: written by bm_bwd_dq, read
// by bm_bwd_dk.
struct BmBK {
  srswa_bm_score_bwd_args a;
  float* wT;                 // [B, nblk, S]
};

// the last block holding a key at or below p - LW (-1: none)
__device__ __forceinline__ int bm_last_remote(int p, int LW, int BS) { return p - LW >= 0 ? (p - LW) / BS : -1; }

// dq: 4 rows per wave, 16 waves per workgroup (64 rows); per group of 64
// blocks the codes and weights g / n are staged in LDS (and the weights
// stored block-major for bm_bwd_dk), then for each kBmBpi blocks up to the
// tile's last remote one the wave's key rows of all of them are loaded
// together (lanes over the head dims) and accumulated in block order.
constexpr int kBmRpw = 4;                               // rows per wave
constexpr int kBmDqWaves = kTsRows / kBmRpw;
constexpr int kBmBpi = 2;                               // blocks gathered together (divides kTsGroup)

template <int D, int BS>
__global__ __launch_bounds__(kBmDqWaves * kWave) void bm_bwd_dq_kernel(BmBK p) {
  constexpr int EPL = D / kWave;
  __shared__ int s_code[kTsGroup * kTsPad];     // [block][row]
  __shared__ float s_w[kTsGroup * kTsPad];      // [block][row]
  __shared__ int s_red[kBmDqWaves];
  const srswa_bm_score_bwd_args& a = p.a;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int ntiles = (a.S + kTsRows - 1) / kTsRows;
  const int b = blockIdx.x / ntiles, tile = blockIdx.x % ntiles;
  const int r0 = tile * kTsRows;
  const int nr = min(kTsRows, a.S - r0);
  const float* kg = a.k + (int64_t)b * a.k_sb + EPL * lane;
  const int nblk_keys = min(a.nblk, ceil_div(a.S, BS));   // blocks that can hold a key
  int trm;                                                // the tile's last remote block
  {
    const int row = r0 + (int)(threadIdx.x % kTsRows);
    const int rm = row < a.S ? bm_last_remote(a.pos[(int64_t)b * a.pos_sb + (int64_t)row * a.pos_st], a.local_window,
                                              BS)
                             : -1;
    const int wm = wave_max_int(rm);
    if (lane == 0) s_red[wave] = wm;
    __syncthreads();
    trm = s_red[0];
#pragma unroll
    for (int w = 1; w < kBmDqWaves; ++w) trm = max(trm, s_red[w]);
    trm = min(trm, nblk_keys - 1);
  }
  float acc[kBmRpw][EPL];
#pragma unroll
  for (int r = 0; r < kBmRpw; ++r)
#pragma unroll
    for (int j = 0; j < EPL; ++j) acc[r][j] = 0.f;
  for (int g0 = 0; g0 < nblk_keys; g0 += kTsGroup) {
    const int gn = min(kTsGroup, nblk_keys - g0);
    float* wdst = p.wT + ((int64_t)b * a.nblk + g0) * a.S + r0;
    if (g0 > trm) {                       // no row of the tile reaches these blocks
      for (int i = threadIdx.x; i < gn * kTsRows; i += blockDim.x) {
        const int c = i / kTsRows, r = i % kTsRows;
        if (r < nr) wdst[(int64_t)c * a.S + r] = 0.f;
      }
      continue;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < gn * kTsRows; i += blockDim.x) {
      const int c = i / kTsRows, r = i % kTsRows;           // codes: rows contiguous
      s_code[c * kTsPad + r] = r < nr ? a.code[((int64_t)b * a.nblk + g0 + c) * a.S + r0 + r] : kCodeNone;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < gn * kTsRows; i += blockDim.x) {
      const int r = i / gn, c = i % gn;                     // upstream gradient: blocks contiguous
      const int cd = s_code[c * kTsPad + r];
      float w = 0.f;
      if (r < nr && !(cd & kCodeNone))
        w = a.gz[(int64_t)b * a.gz_sb + (int64_t)(r0 + r) * a.gz_st + g0 + c] / (float)((cd >> 8) & 0xff);
      s_w[c * kTsPad + r] = w;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < gn * kTsRows; i += blockDim.x) {
      const int c = i / kTsRows, r = i % kTsRows;           // weights, block-major
      if (r < nr) wdst[(int64_t)c * a.S + r] = s_w[c * kTsPad + r];
    }
    const int cn = min(gn, trm - g0 + 1);
    for (int c0 = 0; c0 < cn; c0 += kBmBpi) {               // c0 + kBmBpi <= 64: in the staged arrays
      float kv[kBmBpi][kBmRpw][EPL];
#pragma unroll
      for (int u = 0; u < kBmBpi; ++u)
#pragma unroll
        for (int r = 0; r < kBmRpw; ++r) {
          const int c = c0 + u, rr = kBmRpw * wave + r;
          const int cd = s_code[c * kTsPad + rr];
          const float w = s_w[c * kTsPad + rr];
#pragma unroll
          for (int e = 0; e < EPL; ++e) kv[u][r][e] = 0.f;
          if (c < cn && w != 0.f && !(cd & kCodeMulti)) {
            const int j = (g0 + c) * BS + (cd & 0xff);
#pragma unroll
            for (int e = 0; e < EPL; ++e) kv[u][r][e] = kg[(int64_t)j * a.k_st + e];
          }
        }
#pragma unroll
      for (int u = 0; u < kBmBpi; ++u) {
        const int c = c0 + u;
        if (c >= cn) break;
        const int blk = g0 + c;
#pragma unroll
        for (int r = 0; r < kBmRpw; ++r) {
          const int rr = kBmRpw * wave + r;
          const int cd = s_code[c * kTsPad + rr];
          const float w = s_w[c * kTsPad + rr];
          if (w == 0.f) continue;
          if (!(cd & kCodeMulti)) {
#pragma unroll
            for (int e = 0; e < EPL; ++e) acc[r][e] = fmaf(w, kv[u][r][e], acc[r][e]);
          } else {
            // several keys share the gradient: each one in key order
            uint64_t m = a.tiemask[((int64_t)b * a.S + r0 + rr) * a.nblk + blk];
            while (m) {
              const int off = __builtin_ctzll(m);
              m &= m - 1;
              const int j = blk * BS + off;
#pragma unroll
              for (int e = 0; e < EPL; ++e) acc[r][e] = fmaf(w, kg[(int64_t)j * a.k_st + e], acc[r][e]);
            }
          }
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kBmRpw; ++r) {
    const int rr = kBmRpw * wave + r;
    if (rr < nr) {
      float* dst = a.dq + (int64_t)b * a.dq_sb + (int64_t)(r0 + rr) * a.dq_st + EPL * lane;
#pragma unroll
      for (int e = 0; e < EPL; ++e) dst[e] = acc[r][e];
    }
  }
}

// dk: one wave per (sequence, block, four keys); lane group k (16 lanes)
// owns key 4 w + k's D / 16 head dims per lane.  The block's codes and
// weights are scanned 64 rows at a time in row order (the next batch loaded
// while this one is taken); the rows whose gradient reaches a key are taken
// one per lane group per step (four rows per load instruction).
template <int D, int BS>
__global__ __launch_bounds__(256) void bm_bwd_dk_kernel(BmBK p) {
  constexpr int DPL = D / 16;                    // head dims per lane
  constexpr int QPB = BS / 4;                    // key quads per block
  const srswa_bm_score_bwd_args& a = p.a;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  // workgroups are dealt to the eight XCDs round-robin: consecutive logical
  // ids (the quads of one block) are kept on one XCD so its L2 serves the
  // block's code column to all of them
  const int per_xcd = (int)(gridDim.x / 8);
  const int64_t lid = (int64_t)(blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  const int64_t gw = lid * 4 + wave;
  const int nblk_keys = min(a.nblk, ceil_div(a.S, BS));
  if (gw >= (int64_t)a.B * nblk_keys * QPB) return;
  const int quad = (int)(gw % QPB);
  const int blk = (int)((gw / QPB) % nblk_keys);
  const int b = (int)(gw / ((int64_t)QPB * nblk_keys));
  const int kgrp = lane / 16, dl = lane % 16;
  const int off0 = 4 * quad;                      // first key offset of the quad
  const int my_key = off0 + kgrp;
  const int32_t* col = a.code + ((int64_t)b * a.nblk + blk) * a.S;
  const float* wcol = p.wT + ((int64_t)b * a.nblk + blk) * a.S;
  const float* qb = a.q + (int64_t)b * a.q_sb + DPL * dl;
  float acc[DPL];
#pragma unroll
  for (int e = 0; e < DPL; ++e) acc[e] = 0.f;
  int cd_n = lane < a.S ? col[lane] : kCodeNone;
  float w_n = lane < a.S ? wcol[lane] : 0.f;
  for (int i0 = 0; i0 < a.S; i0 += kWave) {
    const int i = i0 + lane;
    const int cd = cd_n;
    const float w = w_n;
    if (i + kWave < a.S) {
      cd_n = col[i + kWave];
      w_n = wcol[i + kWave];
    } else {
      cd_n = kCodeNone;
      w_n = 0.f;
    }
    // which keys of the quad this row's gradient reaches (bit k)
    uint32_t hit = 0;
    if (w != 0.f) {
      if (cd & kCodeMulti) {
        const uint64_t m = a.tiemask[((int64_t)b * a.S + i) * a.nblk + blk];
        hit = (uint32_t)((m >> off0) & 0xfu);
      } else {
        const int f = (cd & 0xff) - off0;
        hit = (f >= 0 && f < 4) ? 1u << f : 0u;
      }
    }
    if (!__any(hit != 0)) continue;
    uint64_t bal[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) bal[k] = __ballot((hit >> k) & 1u);
    uint64_t mine = bal[kgrp];
    // step n: every lane group takes its n-th row (rows in ascending order)
    while (__any(mine != 0)) {
      const int rsel = mine ? (int)__builtin_ctzll(mine) : 0;
      const float wr = __shfl(w, rsel, kWave);
      if (mine) {
        mine &= mine - 1;
        const float* qrow = qb + (int64_t)(i0 + rsel) * a.q_st;
#pragma unroll
        for (int e = 0; e < DPL; e += 4) {
          const float4 qv = *reinterpret_cast<const float4*>(qrow + e);
          acc[e] = fmaf(wr, qv.x, acc[e]);
          acc[e + 1] = fmaf(wr, qv.y, acc[e + 1]);
          acc[e + 2] = fmaf(wr, qv.z, acc[e + 2]);
          acc[e + 3] = fmaf(wr, qv.w, acc[e + 3]);
        }
      }
    }
  }
  const int j = blk * BS + my_key;
  if (j < a.S) {                                  // the last block may end past the keys
    float* dst = a.dk + (int64_t)b * a.dk_sb + (int64_t)j * a.dk_st + DPL * dl;
#pragma unroll
    for (int e = 0; e < DPL; e += 4)
      *reinterpret_cast<float4*>(dst + e) = make_float4(acc[e], acc[e + 1], acc[e + 2], acc[e + 3]);
  }
}

// the head_cls block size as a template argument (16, 32, 64 or 128; checked by hc_check)
template <int D, typename F>
void hc_dispatch_bs(int BS, F&& f) {
  if (BS == 16) f(std::integral_constant<int, 16>{});
  else if (BS == 32) f(std::integral_constant<int, 32>{});
  else if (BS == 64) f(std::integral_constant<int, 64>{});
  else f(std::integral_constant<int, 128>{});
}

int hc_check(int B, int S, int D, int nblk, int BS, int LB, const char* what) {
  if (B < 0 || S < 0 || nblk < 0 || BS <= 0 || LB < 0) {
    set_error("%s: bad sizes", what);
    return SRSWA_INVALID;
  }
  if (!(D == 64 || D == 128)) {
    set_error("%s: head dim %d not supported (64, 128)", what, D);
    return SRSWA_UNSUPPORTED;
  }
  if (!(BS == 16 || BS == 32 || BS == 64 || BS == 128)) {
    set_error("%s: block size %d not supported (16, 32, 64, 128)", what, BS);
    return SRSWA_UNSUPPORTED;
  }
  return SRSWA_OK;
}

bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace
}  // namespace srswa

using namespace srswa;

extern "C" int srswa_hc_score_fwd(const srswa_hc_score_args* a, void* stream) {
  if (!a || !a->q || !a->k || !a->head_cls || !a->pos || !a->kbar || !a->z) {
    set_error("head_cls scores: null argument");
    return SRSWA_INVALID;
  }
  int rc = hc_check(a->B, a->S, a->D, a->nblk, a->block_size, a->local_blocks, "head_cls scores");
  if (rc != SRSWA_OK) return rc;
  if (a->B == 0 || a->S == 0 || a->nblk == 0) return SRSWA_OK;
  if (!al16(a->q) || !al16(a->k) || !al16(a->kbar) || (a->q_sb % 4) || (a->q_st % 4) || (a->k_sb % 4) ||
      (a->k_st % 4) || (a->kb_sb % 4) || a->kb_sb < (int64_t)a->nblk * a->D) {
    set_error("head_cls scores: rows must be 16-byte aligned and k_bar [B, nblk, D] dense per sequence");
    return SRSWA_UNSUPPORTED;
  }
  // 32-bit buffer offsets into k_bar and a 64-row tile of z
  if ((int64_t)a->nblk * a->D >= (int64_t(1) << 23) || a->z_st < a->nblk || a->z_st >= (int64_t(1) << 23)) {
    set_error("head_cls scores: score rows must not overlap (z_st >= nblk) and z_st, nblk * D must stay below 2^23");
    return SRSWA_UNSUPPORTED;
  }
  HcK k{};
  k.a = *a;
  k.isd = 1.0f / sqrtf((float)a->D);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  k.ngroups = ceil_div(a->nblk, kTsGroup);
  const unsigned gs = (unsigned)((int64_t)a->B * a->nblk);     // a workgroup per block
  const int64_t gz64 = (int64_t)a->B * ceil_div(a->S, kTsRows);
  if (gz64 > 0x7fffffff) {
    set_error("head_cls scores: too many row tiles");
    return SRSWA_UNSUPPORTED;
  }
  const unsigned gz = (unsigned)gz64;
  if (a->D == 128) {
    hc_dispatch_bs<128>(a->block_size, [&](auto bs) {
      hipLaunchKernelGGL((hc_summary_fwd_kernel<128, decltype(bs)::value>), dim3(gs), dim3(256), 0, st, k);
    });
    hipLaunchKernelGGL(hc_score_fwd_kernel<128>, dim3(gz), dim3(256), 0, st, k);
  } else {
    hc_dispatch_bs<64>(a->block_size, [&](auto bs) {
      hipLaunchKernelGGL((hc_summary_fwd_kernel<64, decltype(bs)::value>), dim3(gs), dim3(256), 0, st, k);
    });
    hipLaunchKernelGGL(hc_score_fwd_kernel<64>, dim3(gz), dim3(256), 0, st, k);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("head_cls scores launch failed: %s", hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}

namespace srswa {
namespace {
int hc_bwd_chunks(const srswa_hc_score_bwd_args* a) { return (a->S + kTsChunk - 1) / kTsChunk; }
}  // namespace
}  // namespace srswa

extern "C" int srswa_hc_score_bwd_workspace(const srswa_hc_score_bwd_args* a, size_t* scratch_bytes) {
  if (!a || !scratch_bytes) {
    set_error("head_cls scores backward: null argument");
    return SRSWA_INVALID;
  }
  int rc = hc_check(a->B, a->S, a->D, a->nblk, a->block_size, a->local_blocks, "head_cls scores backward");
  if (rc != SRSWA_OK) return rc;
  const size_t blocks = (size_t)a->B * a->nblk * a->D;
  *scratch_bytes = (size_t)(hc_bwd_chunks(a) + 1) * blocks * sizeof(float);
  return SRSWA_OK;
}

extern "C" int srswa_hc_score_bwd(const srswa_hc_score_bwd_args* a, void* scratch, size_t scratch_bytes,
                                  void* stream) {
  if (!a || !a->q || !a->k || !a->head_cls || !a->pos || !a->kbar || !a->z || !a->gz || !a->dq || !a->dk ||
      !a->dhc) {
    set_error("head_cls scores backward: null argument");
    return SRSWA_INVALID;
  }
  size_t need = 0;
  int rc = srswa_hc_score_bwd_workspace(a, &need);
  if (rc != SRSWA_OK) return rc;
  if (a->B == 0 || a->S == 0 || a->nblk == 0) return SRSWA_OK;
  if (!scratch || scratch_bytes < need || !al16(scratch)) {
    set_error("head_cls scores backward: scratch of %zu bytes required (got %zu)", need, scratch_bytes);
    return SRSWA_WORKSPACE;
  }
  if (!al16(a->q) || !al16(a->k) || !al16(a->kbar) || !al16(a->dq) || !al16(a->dk) || (a->q_sb % 4) ||
      (a->q_st % 4) || (a->k_sb % 4) || (a->k_st % 4) || (a->kb_sb % 4) || (a->dq_sb % 4) || (a->dq_st % 4) ||
      (a->dk_sb % 4) || (a->dk_st % 4) || a->kb_sb < (int64_t)a->nblk * a->D) {
    set_error("head_cls scores backward: rows must be 16-byte aligned and k_bar [B, nblk, D] dense per sequence");
    return SRSWA_UNSUPPORTED;
  }
  // 32-bit buffer offsets within a 64-row tile
  constexpr int64_t kMaxStride = int64_t(1) << 23;
  if (a->z_st < a->nblk || a->gz_st < a->nblk || a->q_st < a->D || a->z_st >= kMaxStride ||
      a->gz_st >= kMaxStride || a->q_st >= kMaxStride || (int64_t)a->nblk * a->D >= kMaxStride) {
    set_error("head_cls scores backward: rows must not overlap (z_st, gz_st >= nblk, q_st >= D) and q_st, z_st, "
              "gz_st, nblk * D must stay below 2^23");
    return SRSWA_UNSUPPORTED;
  }
  HcBK k{};
  k.a = *a;
  k.isd = 1.0f / sqrtf((float)a->D);
  k.nchunks = hc_bwd_chunks(a);
  k.dkb_part = reinterpret_cast<float*>(scratch);
  k.dhc_part = k.dkb_part + (size_t)k.nchunks * a->B * a->nblk * a->D;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  // work items dealt to the XCDs with their D / 64 dim slices: (row tile) for
  // dQ, (256-row chunk, block group) for d k_bar
  const int64_t nq = (int64_t)a->B * ceil_div(a->S, kTsRows);
  const int64_t nk = (int64_t)a->B * ceil_div(a->nblk, kTsGroup) * k.nchunks;
  const int64_t gq64 = (nq + 7) / 8 * 8 * (a->D / 64), gk64 = (nk + 7) / 8 * 8 * (a->D / 64);
  if (gq64 > 0x7fffffff || gk64 > 0x7fffffff) {
    set_error("head_cls scores backward: too many work items");
    return SRSWA_UNSUPPORTED;
  }
  const dim3 gq((unsigned)gq64), gk((unsigned)gk64);
  const dim3 gs((unsigned)((int64_t)a->B * a->nblk));          // a workgroup per block
  if (a->D == 128) {
    hipLaunchKernelGGL(hc_score_bwd_dq_kernel<128>, gq, dim3(256), 0, st, k);
    hipLaunchKernelGGL(hc_score_bwd_dkbar_kernel<128>, gk, dim3(256), 0, st, k);
    hc_dispatch_bs<128>(a->block_size, [&](auto bs) {
      hipLaunchKernelGGL((hc_summary_bwd_kernel<128, decltype(bs)::value>), gs, dim3(256), 0, st, k);
    });
    hipLaunchKernelGGL(hc_dhc_reduce_kernel<128>, dim3(128 / kDhcDims), dim3(kDhcDims * kDhcParts), 0, st, k);
  } else {
    hipLaunchKernelGGL(hc_score_bwd_dq_kernel<64>, gq, dim3(256), 0, st, k);
    hipLaunchKernelGGL(hc_score_bwd_dkbar_kernel<64>, gk, dim3(256), 0, st, k);
    hc_dispatch_bs<64>(a->block_size, [&](auto bs) {
      hipLaunchKernelGGL((hc_summary_bwd_kernel<64, decltype(bs)::value>), gs, dim3(256), 0, st, k);
    });
    hipLaunchKernelGGL(hc_dhc_reduce_kernel<64>, dim3(64 / kDhcDims), dim3(kDhcDims * kDhcParts), 0, st, k);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("head_cls scores backward launch failed: %s", hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}

namespace srswa {
namespace {

int bm_check(const srswa_bm_score_args* a, const char* what) {
  if (a->B < 0 || a->S < 0 || a->nblk < 0 || a->block_size <= 0 || a->local_window < 1) {
    set_error("%s: bad sizes", what);
    return SRSWA_INVALID;
  }
  if (!(a->D == 64 || a->D == 128)) {
    set_error("%s: head dim %d not supported (64, 128)", what, a->D);
    return SRSWA_UNSUPPORTED;
  }
  if (!(a->block_size == 16 || a->block_size == 32 || a->block_size == 64)) {
    set_error("%s: block size %d not supported (16, 32, 64)", what, a->block_size);
    return SRSWA_UNSUPPORTED;
  }
  return SRSWA_OK;
}

template <int D, int BS>
void bm_launch_fwd(const BmK& k, hipStream_t st) {
  const dim3 grid((unsigned)((int64_t)k.a.B * k.ntiles * k.nslab));
  hipLaunchKernelGGL((bm_fwd_kernel<D, BS>), grid, dim3(kBmThreads), 0, st, k);
}

template <int D, int BS>
void bm_launch_bwd(const BmBK& k, hipStream_t st) {
  const srswa_bm_score_bwd_args& a = k.a;
  const int ntiles = (a.S + kTsRows - 1) / kTsRows;
  hipLaunchKernelGGL((bm_bwd_dq_kernel<D, BS>), dim3((unsigned)((int64_t)a.B * ntiles)), dim3(kBmDqWaves * kWave), 0,
                     st, k);
  const int64_t waves = (int64_t)a.B * std::min(a.nblk, (a.S + BS - 1) / BS) * (BS / 4);
  if (waves > 0)   // a multiple of 8 workgroups (the XCD deal), surplus ones exit at once
    hipLaunchKernelGGL((bm_bwd_dk_kernel<D, BS>), dim3((unsigned)(((waves + 3) / 4 + 7) / 8 * 8)), dim3(256), 0,
                       st, k);
}

template <typename F>
void bm_dispatch(int D, int BS, F&& f) {
  if (D == 128) {
    if (BS == 16) f(std::integral_constant<int, 128>{}, std::integral_constant<int, 16>{});
    else if (BS == 32) f(std::integral_constant<int, 128>{}, std::integral_constant<int, 32>{});
    else f(std::integral_constant<int, 128>{}, std::integral_constant<int, 64>{});
  } else {
    if (BS == 16) f(std::integral_constant<int, 64>{}, std::integral_constant<int, 16>{});
    else if (BS == 32) f(std::integral_constant<int, 64>{}, std::integral_constant<int, 32>{});
    else f(std::integral_constant<int, 64>{}, std::integral_constant<int, 64>{});
  }
}

}  // namespace
}  // namespace srswa

extern "C" int srswa_bm_score_fwd(const srswa_bm_score_args* a, void* stream) {
  if (!a || !a->q || !a->k || !a->pos || !a->z || !a->code || !a->tiemask) {
    set_error("block-max scores: null argument");
    return SRSWA_INVALID;
  }
  int rc = bm_check(a, "block-max scores");
  if (rc != SRSWA_OK) return rc;
  if (a->B == 0 || a->S == 0 || a->nblk == 0) return SRSWA_OK;
  if (!al16(a->q) || !al16(a->k) || (a->q_sb % 4) || (a->q_st % 4) || (a->k_sb % 4) || (a->k_st % 4)) {
    set_error("block-max scores: rows must be 16-byte aligned");
    return SRSWA_UNSUPPORTED;
  }
  BmK k{};
  k.a = *a;
  k.ntiles = ceil_div(a->S, kBmRows);
  k.nslab = std::max(1, ceil_div(ceil_div(a->S, kChunk), kBmSlab));
  if ((int64_t)a->B * k.ntiles * k.nslab > 0x7fffffff) {
    set_error("block-max scores: grid too large");
    return SRSWA_UNSUPPORTED;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  bm_dispatch(a->D, a->block_size, [&](auto d, auto bs) { bm_launch_fwd<decltype(d)::value, decltype(bs)::value>(k, st); });
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("block-max scores launch failed: %s", hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}

extern "C" int srswa_bm_score_bwd_workspace(const srswa_bm_score_bwd_args* a, size_t* scratch_bytes) {
  if (!a || !scratch_bytes) {
    set_error("block-max scores backward: null argument");
    return SRSWA_INVALID;
  }
  srswa_bm_score_args f{};
  f.B = a->B; f.S = a->S; f.D = a->D; f.nblk = a->nblk; f.block_size = a->block_size;
  f.local_window = a->local_window;
  int rc = bm_check(&f, "block-max scores backward");
  if (rc != SRSWA_OK) return rc;
  *scratch_bytes = (size_t)a->B * a->nblk * a->S * sizeof(float);
  return SRSWA_OK;
}

extern "C" int srswa_bm_score_bwd(const srswa_bm_score_bwd_args* a, void* scratch, size_t scratch_bytes,
                                  void* stream) {
  if (!a || !a->q || !a->k || !a->pos || !a->code || !a->tiemask || !a->gz || !a->dq || !a->dk) {
    set_error("block-max scores backward: null argument");
    return SRSWA_INVALID;
  }
  size_t need = 0;
  int rc = srswa_bm_score_bwd_workspace(a, &need);
  if (rc != SRSWA_OK) return rc;
  if (a->B == 0 || a->S == 0 || a->nblk == 0) return SRSWA_OK;
  if (!scratch || scratch_bytes < need || !al16(scratch)) {
    set_error("block-max scores backward: scratch of %zu bytes required (got %zu)", need, scratch_bytes);
    return SRSWA_WORKSPACE;
  }
  if (!al16(a->q) || !al16(a->k) || !al16(a->dk) || (a->q_sb % 4) || (a->q_st % 4) || (a->k_sb % 4) ||
      (a->k_st % 4) || (a->dk_sb % 4) || (a->dk_st % 4)) {
    set_error("block-max scores backward: rows must be 16-byte aligned");
    return SRSWA_UNSUPPORTED;
  }
  BmBK k{};
  k.a = *a;
  k.wT = reinterpret_cast<float*>(scratch);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  bm_dispatch(a->D, a->block_size, [&](auto d, auto bs) { bm_launch_bwd<decltype(d)::value, decltype(bs)::value>(k, st); });
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("block-max scores backward launch failed: %s", hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}
