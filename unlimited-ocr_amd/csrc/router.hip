// DASH router on the GPU: block scores -> (block ids, bias, valid) for the
// gather-attention kernels.
//
// Replaces _infer_route_select (HF/modeling_deepseekv2.py:338-362), the
// vLLM DashRouterMath.route_and_select path with budget_topk=True that the
// DASH decode step runs between the block scorer and the attend
// (HF/modeling_deepseekv2.py:535-546).  Per (sequence, query) row:
//   1. candidates: remote blocks (score > _SCORE_NEG / 2) that the page mask
//      allows, or every remote block when the mask leaves none;
//      x = candidate ? score * idx_scale : _ENTMAX_NEG, non-finite -> _ENTMAX_NEG;
//   2. top-M window of x, descending, equal x -> lower block id (the
//      reference's torch.topk leaves the order of equal values open);
//   3. 1.5-entmax over the M values (Peters, Niculae & Martins 2019; the
//      sort-based threshold of HF/dash_attention.py:772-795): z = (x - max)/2,
//      prefix means of z and z^2, tau_rho = mean - sqrt(max((1 - ss)/rho, 0)),
//      support = #{tau_rho <= z_rho}, prior = max(z - tau_support, 0)^2;
//   4. the first K slots: valid = candidate, bias = valid ?
//      (log(max(prior, floor)) - mean over valid) / sigma : 0.
// One wavefront per row (M <= 64: lane k holds the k-th window entry).  The
// prefix sums run left to right in double, rounded per prefix to fp32, the
// order and accumulation of torch's CPU cumsum; no mul+add contraction, and
// fp32 division / sqrt are correctly rounded, so the threshold follows the
// reference's fp32 arithmetic step by step.
#include "common.h"

namespace srswa {
namespace {

constexpr float kScoreNeg = -1.0e9f;    // _SCORE_NEG, HF/dash_attention.py:741
constexpr float kEntmaxNeg = -1.0e4f;   // _ENTMAX_NEG, HF/modeling_deepseekv2.py:65

// Order key of a window entry: the fp32 x mapped to an order-preserving
// unsigned (high word), then 0x7fffffff - idx (equal x: the lower block id is
// the larger key), then the candidate flag in bit 0 so the selected key alone
// gives back x, the block id and the flag.  Every key of a real block is > 0.
__device__ __forceinline__ uint64_t route_key(float x, int idx, bool cand) {
  uint32_t u = __float_as_uint(x);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)u << 32) | ((uint64_t)(0x7fffffffu - (uint32_t)idx) << 1) | (cand ? 1u : 0u);
}
__device__ __forceinline__ float key_x(uint64_t k) {
  const uint32_t u = (uint32_t)(k >> 32);
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}
__device__ __forceinline__ int key_id(uint64_t k) { return (int)(0x7fffffffu - ((uint32_t)k >> 1)); }
__device__ __forceinline__ bool key_cand(uint64_t k) { return (k & 1u) != 0; }
__device__ __forceinline__ uint64_t kmax(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t wave_max_key(uint64_t v) { return wave_max_u64(v); }

__device__ __forceinline__ float readlane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

struct RouteK {
  srswa_route_args a;
  int M, K;
  float inv_sigma;
};

// NPL > 0: each lane keeps the keys of its NPL blocks (j = lane + 64 i) in
// registers.  The window is found without M rounds over every key: the M-th
// largest of the 64 lane maxima is a threshold T with at least M keys >= T
// (those M maxima); the keys >= T (at most 64 in any ordinary row) are
// compacted through LDS and sorted across the wave, lane k then holding the
// k-th largest key.  A row with more than 64 keys >= T takes the M rounds of
// "largest key below the previous one" instead.  NPL == 0 rescans the row
// from memory every round (rows above 4096 blocks).
template <int NPL>
__global__ __launch_bounds__(256) void dash_route_kernel(RouteK p) {
#pragma clang fp contract(off)
  const srswa_route_args& a = p.a;
  __shared__ uint64_t s_sel[4][kWave];
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= (int64_t)a.B * a.Lq) return;
  const int b = (int)(row / a.Lq), q = (int)(row % a.Lq);
  const float* s = a.scores + (int64_t)b * a.sc_sb + (int64_t)q * a.sc_sq;
  const uint8_t* c = a.cand ? a.cand + (int64_t)b * a.cd_sb + (int64_t)q * a.cd_sq : nullptr;
  const int n = a.nblk, M = p.M, K = p.K;

  // the row's scores (and mask bytes) in one batch, past-end lanes reading the
  // last block (in bounds) and dropped below
  constexpr int NR = NPL > 0 ? NPL : 1;
  float sv[NR];
  uint8_t cv[NR];
  bool any = false;
  if (NPL > 0) {
#pragma unroll
    for (int i = 0; i < NPL; ++i) sv[i] = s[min(lane + i * kWave, n - 1)];
    if (c) {
#pragma unroll
      for (int i = 0; i < NPL; ++i) cv[i] = c[min(lane + i * kWave, n - 1)];
#pragma unroll
      for (int i = 0; i < NPL; ++i) any |= lane + i * kWave < n && sv[i] > kScoreNeg * 0.5f && cv[i] != 0;
    } else {
#pragma unroll
      for (int i = 0; i < NPL; ++i) cv[i] = 1;
    }
  } else if (c) {
    for (int j = lane; j < n; j += kWave) any |= (s[j] > kScoreNeg * 0.5f) && c[j] != 0;
  }
  const bool use_c = c != nullptr && __any(any);
  auto key_of = [&](float v, bool cbit, int j) {
    const bool isc = (v > kScoreNeg * 0.5f) && (!use_c || cbit);
    const float x = v * a.idx_scale;
    return route_key((isc && isfinite(x)) ? x : kEntmaxNeg, j, isc);
  };

  uint64_t my_key = 0;
  bool sorted = false;
  uint64_t keys[NR];
  if (NPL > 0) {
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const int j = lane + i * kWave;
      const uint64_t k = key_of(sv[i], cv[i] != 0, j);
      keys[i] = j < n ? k : 0ull;
    }
    uint64_t m0 = 0, m1 = 0, m2 = 0, m3 = 0;
#pragma unroll
    for (int i = 0; i < NPL; i += 4) {
      m0 = kmax(m0, keys[i]);
      m1 = kmax(m1, keys[i + 1]);
      m2 = kmax(m2, keys[i + 2]);
      m3 = kmax(m3, keys[i + 3]);
    }
    // min(n, 64) >= M lanes hold a real key, so T > 0
    const uint64_t lanes_sorted = wave_sort_desc<uint64_t>(kmax(kmax(m0, m1), kmax(m2, m3)), lane);
    const uint64_t T = __shfl(lanes_sorted, M - 1, kWave);
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < NPL; ++i) cnt += keys[i] >= T ? 1 : 0;
    int incl = cnt;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int t = __shfl_up(incl, o, kWave);
      incl += lane >= o ? t : 0;
    }
    const int total = __shfl(incl, kWave - 1, kWave);
    if (total <= kWave) {
      int off = incl - cnt;
#pragma unroll
      for (int i = 0; i < NPL; ++i)
        if (keys[i] >= T) s_sel[wave][off++] = keys[i];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      my_key = wave_sort_desc<uint64_t>(lane < total ? s_sel[wave][lane] : 0ull, lane);
      sorted = true;
    }
  }
  if (!sorted) {
    // M rounds of "largest key below the previous one"
    uint64_t prev = ~0ull;
    for (int k = 0; k < M; ++k) {
      uint64_t best = 0;
      if (NPL > 0) {
#pragma unroll
        for (int i = 0; i < NPL; ++i) {
          const uint64_t key = keys[i];
          best = (key < prev && key > best) ? key : best;
        }
      } else {
        for (int j = lane; j < n; j += kWave) {
          const uint64_t key = key_of(s[j], c == nullptr || c[j] != 0, j);
          if (key < prev && key > best) best = key;
        }
      }
      best = wave_max_key(best);
      prev = best;
      if (lane == k) my_key = best;
    }
  }
  const int my_id = key_id(my_key);
  const bool my_c = lane < M && key_cand(my_key);
  const float my_x = lane < M ? key_x(my_key) : kEntmaxNeg;

  // 1.5-entmax over the window (descending already)
  const float xmax = readlane_f(my_x, 0);
  const float z = (my_x - xmax) / 2.f;
  const float zsq = z * z;
  double cs = 0.0, cs2 = 0.0;
  float my_cs = 0.f, my_cs2 = 0.f;
#pragma unroll
  for (int k = 0; k < kWave; ++k) {
    if (k >= M) break;
    cs += (double)readlane_f(z, k);
    cs2 += (double)readlane_f(zsq, k);
    if (lane == k) {
      my_cs = (float)cs;
      my_cs2 = (float)cs2;
    }
  }
  const float rho = (float)(lane + 1);
  const float mean = my_cs / rho;
  const float mean_sq = my_cs2 / rho;
  const float msq = mean * mean;
  const float ss = rho * (mean_sq - msq);
  const float delta = (1.f - ss) / rho;
  const float tau = mean - sqrtf(fmaxf(delta, 0.f));
  int support = __popcll(__ballot(lane < M && tau <= z));
  support = support < 1 ? 1 : support;
  const float tau_star = __shfl(tau, support - 1, kWave);
  const float y = fmaxf(z - tau_star, 0.f);
  const float prior = y * y;

  // the first K slots: centred log-prior bias over the valid ones
  const bool v = lane < K && my_c;
  const float logp = logf(fmaxf(prior, a.floor));
  int cnt = __popcll(__ballot(v));
  cnt = cnt < 1 ? 1 : cnt;
  const float lv = v ? logp : 0.f;
  float sum = 0.f;
#pragma unroll
  for (int k = 0; k < kWave; ++k) {
    if (k >= K) break;
    sum += readlane_f(lv, k);
  }
  const float mu = sum / (float)cnt;
  const float diff = logp - mu;
  const float bias = v ? diff * p.inv_sigma : 0.f;
  if (lane < K) {
    a.topi[(int64_t)b * a.ti_sb + (int64_t)q * a.ti_sq + lane] = (a.mask_ids && !v) ? -1 : my_id;
    a.bias[(int64_t)b * a.bi_sb + (int64_t)q * a.bi_sq + lane] = bias;
    a.valid[(int64_t)b * a.va_sb + (int64_t)q * a.va_sq + lane] = v ? 1 : 0;
  }
}

}  // namespace
}  // namespace srswa

using namespace srswa;

extern "C" int srswa_dash_route(const srswa_route_args* a, void* stream) {
  if (!a || (!a->scores && a->B * a->Lq > 0) || (a->B * a->Lq > 0 && (!a->topi || !a->bias || !a->valid))) {
    set_error("route: null argument");
    return SRSWA_INVALID;
  }
  if (a->B < 0 || a->Lq < 0 || a->nblk <= 0 || !(a->sigma != 0.0)) {
    set_error("route: bad sizes or sigma");
    return SRSWA_INVALID;
  }
  const int M = a->topm > 0 ? std::max(1, std::min(a->topm, a->nblk)) : a->nblk;
  if (M > kWave) {
    set_error("route: top-M window of %d above 64", M);
    return SRSWA_UNSUPPORTED;
  }
  if (a->B == 0 || a->Lq == 0) return SRSWA_OK;
  RouteK k{};
  k.a = *a;
  k.M = M;
  k.K = std::max(1, std::min(a->K, M));
  k.inv_sigma = (float)(1.0 / a->sigma);
  const int64_t rows = (int64_t)a->B * a->Lq;
  const dim3 grid((unsigned)((rows + 3) / 4));
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (a->nblk <= 8 * kWave) hipLaunchKernelGGL(dash_route_kernel<8>, grid, dim3(256), 0, st, k);
  else if (a->nblk <= 32 * kWave) hipLaunchKernelGGL(dash_route_kernel<32>, grid, dim3(256), 0, st, k);
  else if (a->nblk <= 64 * kWave) hipLaunchKernelGGL(dash_route_kernel<64>, grid, dim3(256), 0, st, k);
  else hipLaunchKernelGGL(dash_route_kernel<0>, grid, dim3(256), 0, st, k);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("route launch failed: %s", hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}
