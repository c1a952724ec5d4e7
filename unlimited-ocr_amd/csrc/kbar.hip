// head_cls summary cache over a paged index-key cache: the serving stage 0 of
// the DASH router on gfx950.
//
// Replaces (WHL!layers/attention/unlimited_dash_ops/dash_stage0.py):
//   KBarCache.put + headcls_scores_prefill's summaries  :62-121
//   KBarCache.refresh_tail                               :123-148
//   headcls_scores_decode / _score_rows                  :45-58, :151-199
// and the Triton pair K11/K12 that serves them (route_triton.py:37-126).
//
// kbar_pages_kernel: one wavefront per (request, logical block); the page's
//   real keys are streamed once and reduced to an fp32 summary row written
//   at the page id (summary.h).
// kbar_scores_kernel: one wavefront per (query row, 64 blocks), every summary
//   row of the chunk in flight at once, the dots finished by a transposing
//   butterfly.
#include "summary.h"

namespace srswa {
namespace {

constexpr int kKbWaves = 4;

// One summary row slice (EPV floats) to memory; a NaN component is stored as 0
// (a page whose head_cls weights are NaN, route_triton.py:68).
template <int EPV>
__device__ __forceinline__ void store_summary(float* dst, const float* kb, bool write) {
  if (!write) return;
  float o[EPV];
#pragma unroll
  for (int e = 0; e < EPV; ++e) o[e] = kb[e] == kb[e] ? kb[e] : 0.f;
#pragma unroll
  for (int e = 0; e < EPV; e += 4) *reinterpret_cast<uint4*>(dst + e) = Vec16<float>::pack(o + e);
}

// 1/sqrt(D) rounded once to fp32 from the double value, as the reference
// passes it (route_triton.py:665, 723, 803)
float inv_sqrt(int D) { return (float)(1.0 / sqrt((double)D)); }

template <typename T, int D, bool HC>
__global__ __launch_bounds__(kKbWaves * kWave) void kbar_pages_kernel(srswa_kbar_pages_args a, int per_req,
                                                                      float inv_sqrt_d) {
  using V = Vec16<T>;
  constexpr int EPV = V::N;
  constexpr int LPR = D / EPV;
  __shared__ float s_w[kKbWaves][64];
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int64_t w = (int64_t)blockIdx.x * kKbWaves + wave;
  if (w >= (int64_t)a.R * per_req) return;
  const int r = (int)(w / per_req), j = (int)(w % per_req);
  const int sl = a.seq_lens[r];
  const int nb = min(ceil_div(max(sl, 0), a.page_size), a.max_blocks);
  const int blk = a.tail_blocks > 0 ? nb - a.tail_blocks + j : j;
  if (blk < 0 || blk >= nb) return;
  const int page = a.block_table[(int64_t)r * a.bt_sr + blk];
  const int nkeys = min(a.page_size, sl - blk * a.page_size);
  const int c = lane % LPR;
  float kb[EPV];
  summarize_rows<T, D, HC>(reinterpret_cast<const T*>(a.keys) + (int64_t)page * a.k_sp + c * EPV, a.k_st, nkeys,
                           HC ? a.head_cls + c * EPV : nullptr, inv_sqrt_d, s_w[wave], kb);
  store_summary<EPV>(a.kbar + (int64_t)page * a.kb_sp + c * EPV, kb, lane < LPR);
}

// kbar_plan_kernel: one wavefront per plan entry (page id, live keys); entries
//   with no live key are skipped (they mark slots of a dense plan that hold no
//   page, and writing them would clobber another request's page).
template <typename T, int D, bool HC>
__global__ __launch_bounds__(kKbWaves * kWave) void kbar_plan_kernel(srswa_kbar_plan_args a, float inv_sqrt_d) {
  using V = Vec16<T>;
  constexpr int EPV = V::N;
  constexpr int LPR = D / EPV;
  __shared__ float s_w[kKbWaves][64];
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int64_t i = (int64_t)blockIdx.x * kKbWaves + wave;
  if (i >= a.n) return;
  const int nkeys = min(a.tok[i], a.page_size);
  const int64_t page = a.pages[i];
  if (nkeys <= 0 || page < 0 || page >= a.num_pages) return;
  const int c = lane % LPR;
  float kb[EPV];
  summarize_rows<T, D, HC>(reinterpret_cast<const T*>(a.keys) + page * a.k_sp + c * EPV, a.k_st, nkeys,
                           HC ? a.head_cls + c * EPV : nullptr, inv_sqrt_d, s_w[wave], kb);
  store_summary<EPV>(a.kbar + page * a.kb_sp + c * EPV, kb, lane < LPR);
}

// kbar_scores_kernel: one wavefront per (query row, 64 blocks).  Lane l reads
//   the block-table entry of block b0 + l once; then every summary row of the
//   chunk is fetched at once (LPB = D/4 lanes x 16 bytes per row, BPS = 64/LPB
//   rows per step, STEPS = LPB steps, all loads in flight before the first
//   product), and the LPB-lane dot products are finished by a transposing
//   butterfly: at each level a lane keeps half of its partial sums and adds its
//   partner's matching half, so after log2(LPB) levels lane (sub, c) holds the
//   full dot of step c, block b0 + BPS c + sub (31 exchanges for D = 128
//   instead of 5 per step).
template <int D>
__global__ __launch_bounds__(kKbWaves * kWave) void kbar_scores_kernel(srswa_kbar_scores_args a, int chunks,
                                                                       float inv_sqrt_d) {
  constexpr int LPB = D / 4;               // lanes per summary row
  constexpr int BPS = kWave / LPB;         // blocks per step
  constexpr int STEPS = kWave / BPS;       // == LPB
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int64_t w = (int64_t)blockIdx.x * kKbWaves + wave;
  if (w >= (int64_t)a.nrows * chunks) return;
  const int n = (int)(w / chunks), ch = (int)(w % chunks);
  const bool prefill = a.cu_q && a.ctx && !a.row_pos;    // chunk-local row n = query row_off + n
  const int m = prefill ? a.row_off + n : n;
  const int r = a.row_req ? a.row_req[m] : n / a.dql;
  const int sl = a.seq_lens[r];
  const int pos = prefill ? a.ctx[r] + (m - a.cu_q[r]) : a.row_pos ? a.row_pos[n] : sl - a.dql + n % a.dql;
  const int qblk = pos >= 0 ? pos / a.page_size : -1;
  const int lim = min(min(qblk - a.local_blocks, ceil_div(max(sl, 0), a.page_size) - 1), a.max_blocks - 1);
  const int sub = lane / LPB, c = lane % LPB;
  const float* qrow = a.q + (int64_t)n * a.q_sn + c * 4;
  const float4 qv = *reinterpret_cast<const float4*>(qrow);
  const int b0 = ch * kWave;
  // lane l: page of block b0 + l (-1 = not a remote block)
  const int lb = b0 + lane;
  const int lpage = (pos >= 0 && lb <= lim) ? a.block_table[(int64_t)r * a.bt_sr + lb] : -1;
  float4 kv[STEPS];
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const int pg = __shfl(lpage, s * BPS + sub, kWave);
    // a non-remote block reads the row's own query (in bounds) and is dropped below
    const float* src = pg >= 0 ? a.kbar + (int64_t)pg * a.kb_sp + c * 4 : qrow;
    kv[s] = *reinterpret_cast<const float4*>(src);
  }
  float z[STEPS];
#pragma unroll
  for (int s = 0; s < STEPS; ++s) z[s] = qv.x * kv[s].x + qv.y * kv[s].y + qv.z * kv[s].z + qv.w * kv[s].w;
  reduce_scatter<STEPS, LPB / 2>(z, c);
  const int blk = b0 + BPS * c + sub;
  const bool remote = blk <= lim && pos >= 0;
  if (blk < a.width)
    a.scores[(int64_t)n * a.sc_sn + blk] =
        remote ? fminf(fmaxf(z[0] * inv_sqrt_d, -kActClamp), kActClamp) : kScoreNeg;
}

bool al16k(const void* p) { return ((uintptr_t)p & 15u) == 0; }

template <typename T, bool HC>
void launch_pages(const srswa_kbar_pages_args& a, int per_req, float inv, hipStream_t st) {
  const int64_t waves = (int64_t)a.R * per_req;
  const dim3 grid((unsigned)((waves + kKbWaves - 1) / kKbWaves));
  if (a.D == 64)
    hipLaunchKernelGGL((kbar_pages_kernel<T, 64, HC>), grid, dim3(kKbWaves * kWave), 0, st, a, per_req, inv);
  else
    hipLaunchKernelGGL((kbar_pages_kernel<T, 128, HC>), grid, dim3(kKbWaves * kWave), 0, st, a, per_req, inv);
}

template <typename T>
void launch_pages_hc(const srswa_kbar_pages_args& a, int per_req, float inv, hipStream_t st) {
  if (a.head_cls) launch_pages<T, true>(a, per_req, inv, st);
  else launch_pages<T, false>(a, per_req, inv, st);
}

}  // namespace
}  // namespace srswa

using namespace srswa;

extern "C" int srswa_kbar_pages(const srswa_kbar_pages_args* a, void* stream) {
  if (!a || !a->keys || !a->block_table || !a->seq_lens || !a->kbar) {
    set_error("kbar pages: null argument");
    return SRSWA_INVALID;
  }
  if (a->R < 0 || a->max_blocks <= 0 || a->page_size <= 0 || a->tail_blocks < 0) {
    set_error("kbar pages: bad sizes");
    return SRSWA_INVALID;
  }
  if (!(a->D == 64 || a->D == 128) || a->k_dtype < 0 || a->k_dtype > 2) {
    set_error("kbar pages: D=%d / dtype not supported", a->D);
    return SRSWA_UNSUPPORTED;
  }
  const int eb = a->k_dtype == SRSWA_F32 ? 4 : 2;
  if (!al16k(a->keys) || !al16k(a->kbar) || (a->k_sp * eb) % 16 || (a->k_st * eb) % 16 || (a->kb_sp * 4) % 16 ||
      (a->head_cls && !al16k(a->head_cls))) {
    set_error("kbar pages: rows must be 16-byte aligned");
    return SRSWA_UNSUPPORTED;
  }
  if (a->R == 0) return SRSWA_OK;
  const int per_req = a->tail_blocks > 0 ? std::min(a->tail_blocks, a->max_blocks) : a->max_blocks;
  const float inv = inv_sqrt(a->D);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (a->k_dtype) {
    case SRSWA_F32: launch_pages_hc<float>(*a, per_req, inv, st); break;
    case SRSWA_BF16: launch_pages_hc<bf16_t>(*a, per_req, inv, st); break;
    default: launch_pages_hc<__half>(*a, per_req, inv, st); break;
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("kbar pages launch failed: %s", hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}

extern "C" int srswa_kbar_scores(const srswa_kbar_scores_args* a, void* stream) {
  if (!a || !a->q || !a->kbar || !a->block_table || !a->seq_lens || !a->scores) {
    set_error("kbar scores: null argument");
    return SRSWA_INVALID;
  }
  const bool prefill = a->cu_q && a->ctx && !a->row_pos && a->row_req;
  const bool explicit_rows = a->row_req && a->row_pos;
  if (a->nrows < 0 || a->R <= 0 || a->max_blocks <= 0 || a->width <= 0 || a->page_size <= 0 ||
      a->local_blocks < 0 || a->row_off < 0 ||
      (!prefill && !explicit_rows && (a->dql <= 0 || a->nrows != a->R * a->dql))) {
    set_error("kbar scores: bad sizes");
    return SRSWA_INVALID;
  }
  if (!(a->D == 64 || a->D == 128)) {
    set_error("kbar scores: D=%d not supported (64, 128)", a->D);
    return SRSWA_UNSUPPORTED;
  }
  if (!al16k(a->q) || !al16k(a->kbar) || (a->q_sn * 4) % 16 || (a->kb_sp * 4) % 16) {
    set_error("kbar scores: rows must be 16-byte aligned");
    return SRSWA_UNSUPPORTED;
  }
  if (a->nrows == 0) return SRSWA_OK;
  const int chunks = ceil_div(a->width, kWave);
  const int64_t waves = (int64_t)a->nrows * chunks;
  const dim3 grid((unsigned)((waves + kKbWaves - 1) / kKbWaves));
  const float inv = inv_sqrt(a->D);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (a->D == 64)
    hipLaunchKernelGGL(kbar_scores_kernel<64>, grid, dim3(kKbWaves * kWave), 0, st, *a, chunks, inv);
  else
    hipLaunchKernelGGL(kbar_scores_kernel<128>, grid, dim3(kKbWaves * kWave), 0, st, *a, chunks, inv);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("kbar scores launch failed: %s", hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}

namespace srswa {
namespace {
template <typename T, bool HC>
void launch_plan(const srswa_kbar_plan_args& a, float inv, hipStream_t st) {
  const dim3 grid((unsigned)((a.n + kKbWaves - 1) / kKbWaves));
  if (a.D == 64)
    hipLaunchKernelGGL((kbar_plan_kernel<T, 64, HC>), grid, dim3(kKbWaves * kWave), 0, st, a, inv);
  else
    hipLaunchKernelGGL((kbar_plan_kernel<T, 128, HC>), grid, dim3(kKbWaves * kWave), 0, st, a, inv);
}
template <typename T>
void launch_plan_hc(const srswa_kbar_plan_args& a, float inv, hipStream_t st) {
  if (a.head_cls) launch_plan<T, true>(a, inv, st);
  else launch_plan<T, false>(a, inv, st);
}
}  // namespace
}  // namespace srswa

extern "C" int srswa_kbar_plan(const srswa_kbar_plan_args* a, void* stream) {
  if (!a || !a->keys || !a->kbar || (a->n > 0 && (!a->pages || !a->tok))) {
    set_error("kbar plan: null argument");
    return SRSWA_INVALID;
  }
  if (a->n < 0 || a->num_pages <= 0 || a->page_size <= 0) {
    set_error("kbar plan: bad sizes");
    return SRSWA_INVALID;
  }
  if (!(a->D == 64 || a->D == 128) || a->k_dtype < 0 || a->k_dtype > 2) {
    set_error("kbar plan: D=%d / dtype not supported", a->D);
    return SRSWA_UNSUPPORTED;
  }
  const int eb = a->k_dtype == SRSWA_F32 ? 4 : 2;
  if (!al16k(a->keys) || !al16k(a->kbar) || (a->k_sp * eb) % 16 || (a->k_st * eb) % 16 || (a->kb_sp * 4) % 16 ||
      (a->head_cls && !al16k(a->head_cls))) {
    set_error("kbar plan: rows must be 16-byte aligned");
    return SRSWA_UNSUPPORTED;
  }
  if (a->n == 0) return SRSWA_OK;
  const float inv = inv_sqrt(a->D);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (a->k_dtype) {
    case SRSWA_F32: launch_plan_hc<float>(*a, inv, st); break;
    case SRSWA_BF16: launch_plan_hc<bf16_t>(*a, inv, st); break;
    default: launch_plan_hc<__half>(*a, inv, st); break;
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("kbar plan launch failed: %s", hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}
