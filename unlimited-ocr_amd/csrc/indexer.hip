// Block indexer for gfx950: head_cls / mean-pool block summaries, remote
// block scores and the wavefront top-k selection.
//
// Replaces the reference's block scoring + selection:
//   _block_scores_infer (stage0 "head_cls")  HF/modeling_deepseekv2.py:380-417
//   DashAttention._block_scores_headcls       HF/dash_attention.py:1053-1143
//   _summary_keys / _score_rows               WHL!layers/attention/unlimited_dash_ops/dash_stage0.py:25-58
//   _kbar_page_kernel / _score_kernel (K11/K12) WHL!layers/attention/unlimited_dash_ops/route_triton.py:37-126
//   block_scores.topk(k) -> -1 for empty     HF/_sparse_base_impl.py:3100-3105
//
// index_summary_kernel: one wavefront per (b, index head, block).  The
// block's real keys (position < kv_len) are streamed once with 16-byte loads
// (16 lanes per 256-byte bf16 row, whole 128-byte lines per instruction) and
// reduced to k_bar in fp32 registers: a plain mean when head_cls is absent
// (the reference's zero-initialised head_cls), else the head_cls softmax
// weights (q.k-style reduce-scatter to per-key logits, wave max/sum, LDS
// broadcast).  k_bar is optionally stored (the per-page summary cache) and
// dotted with every query row: z = clamp(q.k_bar / sqrt(d), +-1e4) on remote
// blocks (blk <= q_pos / BS - local_blocks), SCORE_NEG elsewhere.
//
// topk_rows_kernel: one wavefront per score row.  Scores are mapped to
// order-preserving 64-bit keys (score bits, then the complemented block id so
// equal scores rank the LOWER id first); K rounds of "largest key below the
// previous winner" (per-lane scan + 64-lane max) give the K best in
// descending order, exactly and deterministically; invalid rows pad with -1.
// Rows up to 2048 wide take topk_rows_regs_kernel: the same rounds over keys
// held in registers.
#include "summary.h"

namespace srswa {
namespace {

constexpr int kIdxWaves = 4;

struct IndexK {
  srswa_index_args a;
  float inv_sqrt_d;
  float* scores;        // resolved output / scratch for scores
  int64_t sc_sb, sc_sh, sc_sq;
};

template <typename T, int D, bool HC>
__global__ __launch_bounds__(kIdxWaves * kWave) void index_summary_kernel(IndexK p) {
  using V = Vec16<T>;
  constexpr int EPV = V::N;
  constexpr int LPR = D / EPV;         // lanes per key row
  constexpr int RPI = kWave / LPR;     // rows per load instruction
  static_assert(LPR <= kWave && kWave % LPR == 0, "");
  __shared__ float s_w[kIdxWaves][64];

  const srswa_index_args& a = p.a;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int r = lane / LPR, c = lane % LPR;
  const int nbw = ceil_div(a.nblk, kIdxWaves);
  const int blk = (blockIdx.x % nbw) * kIdxWaves + wave;
  const int64_t bh = blockIdx.x / nbw;
  const int h = (int)(bh % a.HI);
  const int b = (int)(bh / a.HI);
  if (blk >= a.nblk) return;
  const int BS = a.block_size;
  const int kvl = a.kv_len ? min(a.kv_len[b], a.L) : a.L;
  const int k0 = blk * BS;
  const int k1 = min(k0 + BS, kvl);     // real keys of this block

  // is the block remote for at least one query row?
  bool needed = a.kbar_out != nullptr;
  for (int lq0 = 0; !needed && lq0 < a.Lq; lq0 += kWave) {
    const int lq = lq0 + lane;
    bool rem = false;
    if (lq < a.Lq) {
      const int qp = a.q_pos[(int64_t)b * a.pos_sb + (int64_t)lq * a.pos_sq];
      rem = (qp >= 0) && (blk <= qp / BS - a.local_blocks);
    }
    needed = __any(rem);
  }

  float kb[EPV];   // k_bar slice: dims [c*EPV, c*EPV+EPV), valid on every lane after the reduce
#pragma unroll
  for (int e = 0; e < EPV; ++e) kb[e] = 0.f;
  const bool has_keys = k1 > k0;
  if (needed && has_keys)
    summarize_rows<T, D, HC>(reinterpret_cast<const T*>(a.k) + (int64_t)b * a.k_sb + (int64_t)h * a.k_sh +
                                 (int64_t)k0 * a.k_st + c * EPV,
                             a.k_st, k1 - k0, HC ? a.head_cls + c * EPV : nullptr, p.inv_sqrt_d, s_w[wave], kb);

  if (a.kbar_out && r == 0) {
    float* dst = a.kbar_out + (int64_t)b * a.kb_sb + (int64_t)h * a.kb_sh + (int64_t)blk * a.kb_sn + c * EPV;
#pragma unroll
    for (int e = 0; e < EPV; e += 4)
      *reinterpret_cast<uint4*>(dst + e) = Vec16<float>::pack(kb + e);
  }
  if (!p.scores) return;

  // scores for every query row
  for (int lq = 0; lq < a.Lq; ++lq) {
    const int qp = a.q_pos[(int64_t)b * a.pos_sb + (int64_t)lq * a.pos_sq];
    const bool remote = has_keys && qp >= 0 && blk <= qp / BS - a.local_blocks;
    float z = kScoreNeg;
    if (remote) {
      const float* qrow = a.q + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh + (int64_t)lq * a.q_sq + c * EPV;
      float s = 0.f;
      if (r == 0) {
#pragma unroll
        for (int e = 0; e < EPV; ++e) s = fmaf(qrow[e], kb[e], s);
      }
#pragma unroll
      for (int o = LPR / 2; o >= 1; o >>= 1) s += __shfl_xor(s, o, kWave);
      z = fminf(fmaxf(s * p.inv_sqrt_d, -kActClamp), kActClamp);
    }
    if (lane == 0)
      p.scores[(int64_t)b * p.sc_sb + (int64_t)h * p.sc_sh + (int64_t)lq * p.sc_sq + blk] = z;
  }
}

__device__ __forceinline__ uint64_t order_key(float s, int idx) {
  uint32_t u = __float_as_uint(s);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)u << 32) | (uint64_t)(0xffffffffu - (uint32_t)idx);
}

struct TopkK {
  const float* scores;
  int64_t rows, row_stride;
  int32_t n, K, ascending;
  float invalid_at;
  int32_t* out_idx; int64_t out_stride;
  float* out_val;
};

// The K winners held one per lane (lane k the k-th largest): optionally
// reordered by ascending id, then written with -1 / -inf padding.
__device__ __forceinline__ void topk_write(const TopkK& p, int64_t row, int lane, int my_id, float my_val, int nsel) {
  if (p.ascending && nsel > 1) {
    // rank of this lane's id among the selected ids (ids are distinct)
    int rank = 0;
    for (int j = 0; j < nsel; ++j) {
      const int o = __shfl(my_id, j, kWave);
      rank += (lane < nsel && o < my_id) ? 1 : 0;
    }
    const int dst = lane < nsel ? rank : lane;
    // scatter via LDS-free shuffle: lane t takes the element whose rank is t
    int got_id = -1;
    float got_val = 0.f;
    for (int j = 0; j < nsel; ++j) {
      const int rj = __shfl(dst, j, kWave);
      const int ij = __shfl(my_id, j, kWave);
      const float vj = __shfl(my_val, j, kWave);
      if (rj == lane) { got_id = ij; got_val = vj; }
    }
    my_id = lane < nsel ? got_id : -1;
    my_val = got_val;
  }
  for (int k = lane; k < p.K; k += kWave) {
    const int id = k < nsel ? (k < kWave ? my_id : -1) : -1;
    p.out_idx[row * p.out_stride + k] = id;
    if (p.out_val) p.out_val[row * p.out_stride + k] = id >= 0 ? my_val : -INFINITY;
  }
}

// one wavefront per row; 4 rows per workgroup (rows of any width)
__global__ __launch_bounds__(256) void topk_rows_kernel(TopkK p) {
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= p.rows) return;
  const float* s = p.scores + row * p.row_stride;
  uint64_t prev = ~0ull;
  int my_id = -1;             // lane k keeps the k-th winner
  float my_val = 0.f;
  int nsel = 0;
  for (int k = 0; k < p.K; ++k) {
    uint64_t best = 0;
    for (int j = lane; j < p.n; j += kWave) {
      const float v = s[j];
      if (!(v > p.invalid_at)) continue;                 // invalid, -inf or NaN
      const uint64_t key = order_key(v, j);
      if (key < prev && key > best) best = key;
    }
    best = wave_max_u64(best);
    if (best == 0) break;                                // no valid entry left
    prev = best;
    const int id = (int)(0xffffffffu - (uint32_t)(best & 0xffffffffu));
    if (lane == k) {
      my_id = id;
      my_val = s[id];
    }
    ++nsel;
  }
  topk_write(p, row, lane, my_id, my_val, nsel);
}

// The same selection with the row held in registers (column j = lane + 64 i,
// i < NPL; rows up to 64 NPL wide): one read of the scores, then each round a
// register max, a DPP wave max and the winner's key cleared where it lives.
// The winner's score comes back exactly from its key's upper half.
template <int NPL>
__global__ __launch_bounds__(256) void topk_rows_regs_kernel(TopkK p) {
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= p.rows) return;
  const float* s = p.scores + row * p.row_stride;
  // the row's scores as one unconditional batch of loads (column clamped to the
  // row, the tail masked below): under a per-column branch each load would
  // wait out its own round trip
  float sv[NPL];
  if (p.n > 0) {
#pragma unroll
    for (int i = 0; i < NPL; ++i) sv[i] = s[min(lane + kWave * i, p.n - 1)];
  }
  uint64_t key[NPL];
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int j = lane + kWave * i;
    const float v = j < p.n ? sv[i] : -INFINITY;
    key[i] = v > p.invalid_at ? order_key(v, j) : 0ull;  // invalid, -inf or NaN: never selected
  }
  int my_id = -1;
  float my_val = 0.f;
  int nsel = 0;
  for (int k = 0; k < p.K; ++k) {
    uint64_t best = 0;
#pragma unroll
    for (int i = 0; i < NPL; ++i) best = key[i] > best ? key[i] : best;
    best = wave_max_u64(best);
    if (best == 0) break;
#pragma unroll
    for (int i = 0; i < NPL; ++i) key[i] = key[i] == best ? 0ull : key[i];
    if (lane == k) {
      my_id = (int)(0xffffffffu - (uint32_t)(best & 0xffffffffu));
      const uint32_t u = (uint32_t)(best >> 32);
      my_val = __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
    }
    ++nsel;
  }
  topk_write(p, row, lane, my_id, my_val, nsel);
}

int elem_bytes_i(int dt) { return dt == SRSWA_F32 ? 4 : 2; }

template <typename T, bool HC>
int launch_summary(const IndexK& k, hipStream_t st) {
  const int64_t grid = (int64_t)k.a.B * k.a.HI * ceil_div(k.a.nblk, kIdxWaves);
  if (k.a.D == 64)
    hipLaunchKernelGGL((index_summary_kernel<T, 64, HC>), dim3((unsigned)grid), dim3(kIdxWaves * kWave), 0, st, k);
  else
    hipLaunchKernelGGL((index_summary_kernel<T, 128, HC>), dim3((unsigned)grid), dim3(kIdxWaves * kWave), 0, st, k);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("index summary launch failed: %s", hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}

template <typename T>
int dispatch_summary(const IndexK& k, hipStream_t st) {
  return k.a.head_cls ? launch_summary<T, true>(k, st) : launch_summary<T, false>(k, st);
}

int run_topk(const TopkK& t, hipStream_t st) {
  if (t.rows == 0) return SRSWA_OK;
  const int64_t grid = (t.rows + 3) / 4;
  if (t.n <= 256)
    hipLaunchKernelGGL(topk_rows_regs_kernel<4>, dim3((unsigned)grid), dim3(256), 0, st, t);
  else if (t.n <= 512)
    hipLaunchKernelGGL(topk_rows_regs_kernel<8>, dim3((unsigned)grid), dim3(256), 0, st, t);
  else if (t.n <= 1024)
    hipLaunchKernelGGL(topk_rows_regs_kernel<16>, dim3((unsigned)grid), dim3(256), 0, st, t);
  else if (t.n <= 2048)
    hipLaunchKernelGGL(topk_rows_regs_kernel<32>, dim3((unsigned)grid), dim3(256), 0, st, t);
  else
    hipLaunchKernelGGL(topk_rows_kernel, dim3((unsigned)grid), dim3(256), 0, st, t);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("topk launch failed: %s", hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}

bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int validate_index(const srswa_index_args* a, bool need_k) {
  if (!a || !a->q_pos || (need_k && !a->k)) {
    set_error("index: null argument");
    return SRSWA_INVALID;
  }
  if (a->B < 0 || a->HI <= 0 || a->Lq < 0 || a->L <= 0 || a->nblk <= 0 || a->block_size <= 0 ||
      a->local_blocks < 0 || a->K < 0) {
    set_error("index: bad sizes");
    return SRSWA_INVALID;
  }
  if (!(a->D == 64 || a->D == 128)) {
    set_error("index: head dim %d not supported (64, 128)", a->D);
    return SRSWA_UNSUPPORTED;
  }
  if (a->K > 64) {
    set_error("index: top-k of at most 64 blocks per row (got %d)", a->K);
    return SRSWA_UNSUPPORTED;
  }
  const int eb = elem_bytes_i(a->k_dtype);
  if (need_k && (!al16(a->k) || (a->k_sb * eb) % 16 || (a->k_st * eb) % 16 || (a->k_sh * eb) % 16)) {
    set_error("index: key rows must be 16-byte aligned");
    return SRSWA_UNSUPPORTED;
  }
  if (a->kbar_out && (!al16(a->kbar_out) || (a->kb_sb * 4) % 16 || (a->kb_sh * 4) % 16 || (a->kb_sn * 4) % 16)) {
    set_error("index: k_bar rows must be 16-byte aligned");
    return SRSWA_UNSUPPORTED;
  }
  return SRSWA_OK;
}

}  // namespace
}  // namespace srswa

using namespace srswa;

extern "C" size_t srswa_index_workspace(const srswa_index_args* a) {
  if (!a || a->scores || a->B <= 0 || a->Lq <= 0) return 0;
  return (size_t)a->B * a->HI * a->Lq * a->nblk * sizeof(float);
}

extern "C" int srswa_index_meanpool_topk(const srswa_index_args* a, void* scratch,
                                         size_t scratch_bytes, void* stream) {
  int st = validate_index(a, true);
  if (st != SRSWA_OK) return st;
  if (a->B == 0 || a->Lq == 0) return SRSWA_OK;
  if (!a->q && (a->scores || a->topk_idx)) {
    set_error("index: q required for scores");
    return SRSWA_INVALID;
  }
  IndexK k{};
  k.a = *a;
  k.inv_sqrt_d = 1.0f / sqrtf((float)a->D);
  if (a->scores) {
    k.scores = a->scores;
    k.sc_sb = a->sc_sb; k.sc_sh = a->sc_sh; k.sc_sq = a->sc_sq;
  } else if (a->topk_idx) {
    const size_t need = srswa_index_workspace(a);
    if (!scratch || scratch_bytes < need) {
      set_error("index: scratch of %zu bytes required (got %zu)", need, scratch_bytes);
      return SRSWA_WORKSPACE;
    }
    k.scores = reinterpret_cast<float*>(scratch);
    k.sc_sq = a->nblk; k.sc_sh = (int64_t)a->Lq * a->nblk; k.sc_sb = (int64_t)a->HI * a->Lq * a->nblk;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (a->k_dtype) {
    case SRSWA_F32: st = dispatch_summary<float>(k, s); break;
    case SRSWA_BF16: st = dispatch_summary<bf16_t>(k, s); break;
    case SRSWA_F16: st = dispatch_summary<__half>(k, s); break;
    default: set_error("index: bad k dtype"); return SRSWA_UNSUPPORTED;
  }
  if (st != SRSWA_OK || !a->topk_idx || a->K == 0) return st;
  // rows (b, h, lq) are contiguous in the score buffer when it is ours; for a
  // caller buffer each row is at b*sc_sb + h*sc_sh + lq*sc_sq, contiguous when
  // sc_sh == Lq*sc_sq and sc_sb == HI*sc_sh.
  if (k.sc_sh != (int64_t)a->Lq * k.sc_sq || k.sc_sb != (int64_t)a->HI * k.sc_sh ||
      a->ti_sh != (int64_t)a->Lq * a->ti_sq || a->ti_sb != (int64_t)a->HI * a->ti_sh) {
    set_error("index: score / top-k rows must be packed [B, HI, Lq, *]");
    return SRSWA_UNSUPPORTED;
  }
  TopkK t{};
  t.scores = k.scores;
  t.rows = (int64_t)a->B * a->HI * a->Lq;
  t.row_stride = k.sc_sq;
  t.n = a->nblk;
  t.K = a->K;
  t.ascending = a->ascending;
  t.invalid_at = kScoreNeg * 0.5f;
  t.out_idx = a->topk_idx;
  t.out_stride = a->ti_sq;
  t.out_val = a->topk_val;
  return run_topk(t, s);
}

extern "C" int srswa_topk_rows(const float* scores, int64_t rows, int32_t n, int64_t row_stride,
                               int32_t K, int32_t ascending, float invalid_at, int32_t* out_idx,
                               float* out_val, int64_t out_stride, void* stream) {
  if (!scores || !out_idx || rows < 0 || n <= 0 || K < 0) {
    set_error("topk: bad arguments");
    return SRSWA_INVALID;
  }
  if (K > 64) {
    set_error("topk: K <= 64 supported (got %d)", K);
    return SRSWA_UNSUPPORTED;
  }
  if (K == 0) return SRSWA_OK;
  TopkK t{scores, rows, row_stride, n, K, ascending, invalid_at, out_idx, out_stride, out_val};
  return run_topk(t, reinterpret_cast<hipStream_t>(stream));
}
