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

__device__ __forceinline__ uint64_t route_key(float s, int idx) {
  uint32_t u = __float_as_uint(s);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)u << 32) | (uint64_t)(0xffffffffu - (uint32_t)idx);
}

__device__ __forceinline__ uint64_t wave_max_key(uint64_t v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const uint64_t w = __shfl_xor(v, o, kWave);
    v = w > v ? w : v;
  }
  return v;
}

struct RouteK {
  srswa_route_args a;
  int M, K;
  float inv_sigma;
};

// NPL > 0: each lane keeps the order keys of its NPL blocks (j = lane + 64 i)
// in registers, built once, so the M selection rounds never touch memory;
// NPL == 0 rescans the row from memory every round (rows above 4096 blocks).
template <int NPL>
__global__ __launch_bounds__(256) void dash_route_kernel(RouteK p) {
#pragma clang fp contract(off)
  const srswa_route_args& a = p.a;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= (int64_t)a.B * a.Lq) return;
  const int b = (int)(row / a.Lq), q = (int)(row % a.Lq);
  const float* s = a.scores + (int64_t)b * a.sc_sb + (int64_t)q * a.sc_sq;
  const uint8_t* c = a.cand ? a.cand + (int64_t)b * a.cd_sb + (int64_t)q * a.cd_sq : nullptr;
  const int n = a.nblk, M = p.M, K = p.K;

  bool any = false;
  if (c)
    for (int j = lane; j < n; j += kWave) any |= (s[j] > kScoreNeg * 0.5f) && c[j] != 0;
  const bool use_c = c != nullptr && __any(any);
  auto xval = [&](int j, bool& isc) {
    const float v = s[j];
    isc = (v > kScoreNeg * 0.5f) && (!use_c || c[j] != 0);
    const float x = v * a.idx_scale;
    return (isc && isfinite(x)) ? x : kEntmaxNeg;
  };

  // top-M window: M rounds of "largest key below the previous one"
  uint64_t keys[NPL > 0 ? NPL : 1];
  if (NPL > 0) {
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const int j = lane + i * kWave;
      bool isc;
      keys[i] = j < n ? route_key(xval(j, isc), j) : 0ull;   // real keys are > 0
    }
  }
  uint64_t prev = ~0ull;
  int my_id = 0;
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
        bool isc;
        const uint64_t key = route_key(xval(j, isc), j);
        if (key < prev && key > best) best = key;
      }
    }
    best = wave_max_key(best);
    prev = best;
    if (lane == k) my_id = (int)(0xffffffffu - (uint32_t)(best & 0xffffffffu));
  }
  bool my_c = false;
  const float my_x = lane < M ? xval(my_id, my_c) : kEntmaxNeg;
  my_c = my_c && lane < M;

  // 1.5-entmax over the window (descending already)
  const float xmax = __shfl(my_x, 0, kWave);
  const float z = (my_x - xmax) / 2.f;
  const float zsq = z * z;
  double cs = 0.0, cs2 = 0.0;
  float my_cs = 0.f, my_cs2 = 0.f;
  for (int k = 0; k < M; ++k) {
    cs += (double)__shfl(z, k, kWave);
    cs2 += (double)__shfl(zsq, k, kWave);
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
  for (int k = 0; k < K; ++k) sum += __shfl(lv, k, kWave);
  const float mu = sum / (float)cnt;
  const float diff = logp - mu;
  const float bias = v ? diff * p.inv_sigma : 0.f;
  if (lane < K) {
    a.topi[(int64_t)b * a.ti_sb + (int64_t)q * a.ti_sq + lane] = my_id;
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
