// Serving DASH router for gfx950: block scores -> 1.5-entmax prior over every
// candidate block -> hard top-K budget -> centred log-prior bias, packed in
// ascending block order into caller-owned slots.
//
// Replaces the Triton routers of the SGLang backend
// (WHL!layers/attention/unlimited_dash_ops/route_triton.py): _entmax_kernel
// :129-221 and _entmax_tiled_kernel :280-463 (the same selection over the
// page-mask window), and _win_bounds_kernel :466-505.
//
// route_entmax_regs_kernel (rows up to 2048 columns) holds the row in
// registers and runs every step below as register loops; route_entmax_kernel
// (wider rows): one wavefront per query row, the row's scores read in
// streaming passes (64 columns per step, L2-resident after the first):
//   1. candidate counts (remote, remote & page mask), max and min of x;
//   2. the candidates with z > -1 -- the only ones a bisection midpoint in
//      [-1, 0] can count -- are compacted into LDS; the 24 tau steps then sum
//      a few values per lane in fp64 and reduce them across the wave (every
//      lane ends with the same bits, so every lane takes the same branch);
//   3. budget: the reference's 40-step count bisection moves lo up exactly
//      when the (K+1)-th largest candidate z exceeds mid, so that order
//      statistic is selected exactly (lane maxima -> threshold -> compaction
//      -> wave sort or a bitwise search) and the 40 steps are replayed on it;
//   4. mu over the active blocks (fp64 sum), then the packed write (ballot
//      prefix counts give each active block its ascending slot).
// Compiled without FP contraction: every product and sum is rounded as the
// reference's fp32 Triton arithmetic rounds it.
#include <algorithm>

#include "mfma_common.h"   // device_cu_count
#include "summary.h"

namespace srswa {
namespace {

constexpr float kEntmaxNeg = -1.0e4f;   // ENTMAX_NEG, route_triton.py:25
constexpr int kRsWaves = 4;             // rows per workgroup
constexpr int kCap = 512;               // compacted values per wave (8 per lane)
constexpr int kPerLane = kCap / kWave;
constexpr int kTauIters = 24;           // ENTMAX_ITERS, route_triton.py:12
constexpr int kCapIters = 40;           // ENTMAX_ITERS_CAP, route_triton.py:14

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

struct RowView {
  const float* sc;
  const int8_t* im;
  int W;
  float idx_scale;
  bool use_img;
  float xm;
  // column j (< W): candidate flag and z
  __device__ __forceinline__ bool load(int j, float& z) const {
    const float s = sc[j];
    const bool remote = s > kScoreNeg * 0.5f;             // NaN: not remote
    const bool cand = remote && (!use_img || im[j] != 0);
    float x = s * idx_scale;
    x = x == x ? x : kEntmaxNeg;
    z = (x - xm) * 0.5f;
    return cand;
  }
};

__global__ __launch_bounds__(kRsWaves * kWave) void route_entmax_kernel(srswa_route_serve_args a) {
  __shared__ float s_val[kRsWaves][kCap];
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int64_t row = (int64_t)blockIdx.x * kRsWaves + wave;
  if (row >= a.rows) return;
  const unsigned long long lt = (1ull << lane) - 1ull;
  float* buf = s_val[wave];
  uint32_t* ubuf = reinterpret_cast<uint32_t*>(buf);

  RowView v{a.scores + row * a.sc_sn, a.img ? a.img + row * a.img_sn : nullptr, a.W, a.idx_scale, false, 0.f};

  // ---- pass 1: candidate sets, max / min of x over them
  int n_rem = 0, n_img = 0;
  float mx_r = -INFINITY, mn_r = INFINITY, mx_i = -INFINITY, mn_i = INFINITY;
  for (int j0 = 0; j0 < a.W; j0 += kWave) {
    const int j = j0 + lane;
    bool remote = false, ci = false;
    float x = 0.f;
    if (j < a.W) {
      const float s = v.sc[j];
      remote = s > kScoreNeg * 0.5f;
      ci = remote && v.im && v.im[j] != 0;
      x = s * a.idx_scale;
      x = x == x ? x : kEntmaxNeg;
    }
    n_rem += __popcll(__ballot(remote));
    n_img += __popcll(__ballot(ci));
    if (remote) { mx_r = fmaxf(mx_r, x); mn_r = fminf(mn_r, x); }
    if (ci) { mx_i = fmaxf(mx_i, x); mn_i = fminf(mn_i, x); }
  }
  // per-row fallback: a page mask that leaves no candidate is dropped
  v.use_img = n_img > 0;
  const int n_cand = v.use_img ? n_img : n_rem;
  const bool has_any = n_cand > 0;
  const float xmax = wave_max(v.use_img ? mx_i : mx_r);
  const float xmin = wave_min(v.use_img ? mn_i : mn_r);
  v.xm = has_any ? xmax : 0.f;
  // min over the candidates of z = (x - xm) * 0.5: rounding is monotone
  const float zmin = (xmin - v.xm) * 0.5f;

  // ---- pass 2: tau over the candidates with z > -1
  int n_act = 0;
  for (int j0 = 0; j0 < a.W; j0 += kWave) {
    const int j = j0 + lane;
    float z = -INFINITY;
    const bool act = j < a.W && v.load(j, z) && z > -1.f;
    const unsigned long long bal = __ballot(act);
    const int pos = n_act + __popcll(bal & lt);
    if (act && pos < kCap) buf[pos] = z;
    n_act += __popcll(bal);
  }
  wave_sync_lds();
  float zz[kPerLane];
#pragma unroll
  for (int i = 0; i < kPerLane; ++i) {
    const int k = lane + i * kWave;
    zz[i] = k < n_act ? buf[k] : -INFINITY;
  }
  float lo = -1.f, hi = 0.f;
  for (int it = 0; it < kTauIters; ++it) {
    const float mid = (lo + hi) * 0.5f;
    double acc = 0.0;
    if (n_act <= kCap) {
#pragma unroll
      for (int i = 0; i < kPerLane; ++i) {
        const float p = fmaxf(zz[i] - mid, 0.f);
        acc += (double)(p * p);
      }
    } else {   // more than kCap values above -1: sum straight from the row
      for (int j0 = 0; j0 < a.W; j0 += kWave) {
        const int j = j0 + lane;
        float z;
        if (j < a.W && v.load(j, z)) {
          const float p = fmaxf(z - mid, 0.f);
          acc += (double)(p * p);
        }
      }
    }
    const float ssum = (float)wave_sum_f64(acc);
    if (ssum > 1.f) lo = mid;
    else hi = mid;
  }
  const float tau = (lo + hi) * 0.5f;

  // ---- pass 3: the budget threshold
  float zthr = -INFINITY;
  if (n_cand > a.K) {
    // lane maxima of the candidates' order keys; T = the (K+1)-th largest of
    // them leaves at least K + 1 keys >= T
    uint32_t lmax = 0;
    for (int j0 = 0; j0 < a.W; j0 += kWave) {
      const int j = j0 + lane;
      float z;
      if (j < a.W && v.load(j, z)) lmax = max(lmax, f32_order_key(z));
    }
    wave_sync_lds();   // buf is reused
    uint32_t T = 0;
    if (a.K + 1 <= kWave) T = __shfl(wave_sort_desc<uint32_t>(lmax, lane), a.K, kWave);
    int C = 0;
    for (int j0 = 0; j0 < a.W; j0 += kWave) {
      const int j = j0 + lane;
      float z;
      uint32_t key = 0;
      const bool sel = j < a.W && v.load(j, z) && (key = f32_order_key(z)) >= T;
      const unsigned long long bal = __ballot(sel);
      const int pos = C + __popcll(bal & lt);
      if (sel && pos < kCap) ubuf[pos] = key;
      C += __popcll(bal);
    }
    wave_sync_lds();
    uint32_t kth;   // key of the (K+1)-th largest candidate z
    if (C <= kWave) {
      const uint32_t mine = lane < C ? ubuf[lane] : 0u;
      kth = __shfl(wave_sort_desc<uint32_t>(mine, lane), a.K, kWave);
    } else {
      // largest t with at least K + 1 keys >= t, bit by bit from the top
      uint32_t kv[kPerLane];
#pragma unroll
      for (int i = 0; i < kPerLane; ++i) {
        const int k = lane + i * kWave;
        kv[i] = (C <= kCap && k < C) ? ubuf[k] : 0u;
      }
      kth = 0;
      for (int bit = 31; bit >= 0; --bit) {
        const uint32_t t = kth | (1u << bit);
        int cnt = 0;
        if (C <= kCap) {
#pragma unroll
          for (int i = 0; i < kPerLane; ++i) cnt += __popcll(__ballot(kv[i] >= t));
        } else {
          for (int j0 = 0; j0 < a.W; j0 += kWave) {
            const int j = j0 + lane;
            float z;
            const bool ge = j < a.W && v.load(j, z) && f32_order_key(z) >= t;
            cnt += __popcll(__ballot(ge));
          }
        }
        if (cnt >= a.K + 1) kth = t;
      }
    }
    const float zk1 = f32_from_order_key(kth);
    // the reference's bisection, replayed: cnt(z > mid) > K <=> zk1 > mid
    float lo2 = zmin - 1.f, hi2 = 0.f;
    for (int it = 0; it < kCapIters; ++it) {
      const float mid = (lo2 + hi2) * 0.5f;
      if (zk1 > mid) lo2 = mid;
      else hi2 = mid;
    }
    zthr = hi2;
  }

  // ---- pass 4: mu over the active blocks
  double lsum = 0.0;
  int n_sel = 0;
  for (int j0 = 0; j0 < a.W; j0 += kWave) {
    const int j = j0 + lane;
    float z = 0.f;
    const bool act = j < a.W && v.load(j, z) && z > zthr;
    if (act) {
      float pr = fmaxf(z - tau, 0.f);
      pr = pr * pr;
      lsum += (double)logf(fmaxf(pr, a.prior_floor));
    }
    n_sel += __popcll(__ballot(act));
  }
  const float mu = (float)wave_sum_f64(lsum) / (float)max(n_sel, 1);

  // ---- pass 5: packed write, ascending block ids
  int32_t* oi = a.out_idx + row * a.oi_sn;
  float* ob = a.out_bias + row * a.ob_sn;
  int base = 0;
  for (int j0 = 0; j0 < a.W && base < a.M; j0 += kWave) {
    const int j = j0 + lane;
    float z = 0.f;
    const bool act = j < a.W && v.load(j, z) && z > zthr;
    const unsigned long long bal = __ballot(act);
    const int pos = base + __popcll(bal & lt);
    if (act && pos < a.M) {
      float pr = fmaxf(z - tau, 0.f);
      pr = pr * pr;
      const float lp = logf(fmaxf(pr, a.prior_floor));
      oi[pos] = j;
      ob[pos] = (lp - mu) * a.inv_sigma;
    }
    base += __popcll(bal);
  }
  for (int s = min(base, a.M) + lane; s < a.M; s += kWave) {
    oi[s] = -1;
    ob[s] = 0.f;
  }
}

// The same router with the row held in registers (column j = lane + 64 i,
// i < NPL): one read of the scores and page mask, every later pass a register
// loop.  Rows up to 64 NPL columns (2048 with NPL = 32).  The tau sums keep
// four fp64 partial sums per lane (independent add chains); as in the
// streaming kernel their order differs from the reference's reduction tree
// only below fp64 resolution, and the sum is then rounded to fp32.
// SPLIT (few rows, a GPU mostly idle, as in a decode step): two waves per row.
// The tau bisection (role 0) and the budget threshold (role 1) depend only on
// the row's z, so they run side by side; role 1 hands its threshold to role 0
// through LDS, and role 0 finishes the row.  Otherwise (a prefill chunk, the
// GPU full) one wave per row runs both stages.
template <int NPL, bool SPLIT>
__global__ __launch_bounds__(kRsWaves * kWave) void route_entmax_regs_kernel(srswa_route_serve_args a) {
  static_assert(NPL % 4 == 0 && NPL <= 32, "NPL: a multiple of 4, at most 32");
  constexpr int kRows = SPLIT ? kRsWaves / 2 : kRsWaves;   // rows per workgroup
  __shared__ uint32_t s_key[kRows][kWave];
  __shared__ float s_live[kRows][4 * kWave];
  __shared__ float s_thr[kRows];
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int pr = SPLIT ? wave >> 1 : wave;
  const int row_role = SPLIT ? wave & 1 : -1;      // -1: both stages
  const int64_t row0 = (int64_t)blockIdx.x * kRows + pr;
  // a pair past the last row works on the last row and writes nothing, so
  // every wave reaches the barrier below
  const bool live_row = row0 < a.rows;
  const int64_t row = live_row ? row0 : a.rows - 1;
  const unsigned long long lt = (1ull << lane) - 1ull;
  const float* sc = a.scores + row * a.sc_sn;
  const int8_t* im = a.img ? a.img + row * a.img_sn : nullptr;

  // The row's scores and page-mask bytes are loaded as two unconditional
  // batches (column index clamped to the row, the tail masked afterwards), so
  // all of a lane's loads are in flight together: loads under a per-column
  // branch each wait out their own round trip.
  float x[NPL];
  int8_t iv[NPL];
  if (a.W > 0) {
    const int wl = a.W - 1;
#pragma unroll
    for (int i = 0; i < NPL; ++i) x[i] = sc[min(lane + kWave * i, wl)];
    if (im) {
#pragma unroll
      for (int i = 0; i < NPL; ++i) iv[i] = im[min(lane + kWave * i, wl)];
    }
  }
  uint32_t rem_bits = 0, img_bits = 0;
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int j = lane + kWave * i;
    const float s = j < a.W ? x[i] : -INFINITY;
    const bool remote = s > kScoreNeg * 0.5f;             // NaN / -inf: not remote
    const bool ci = remote && im && iv[i] != 0;
    float xv = s * a.idx_scale;
    x[i] = xv == xv ? xv : kEntmaxNeg;
    rem_bits |= remote ? 1u << i : 0u;
    img_bits |= ci ? 1u << i : 0u;
  }
  const int n_img = wave_sum_int(__popc(img_bits));
  const bool use_img = n_img > 0;
  const uint32_t cand = use_img ? img_bits : rem_bits;
  const int n_cand = use_img ? n_img : wave_sum_int(__popc(rem_bits));
  float mx = -INFINITY, mn = INFINITY;
#pragma unroll
  for (int i = 0; i < NPL; ++i)
    if ((cand >> i) & 1u) {
      mx = fmaxf(mx, x[i]);
      mn = fminf(mn, x[i]);
    }
  const float xm = n_cand > 0 ? wave_max(mx) : 0.f;
  const float zmin = (wave_min(mn) - xm) * 0.5f;
  // x -> z in place; non-candidates -inf
#pragma unroll
  for (int i = 0; i < NPL; ++i) x[i] = ((cand >> i) & 1u) ? (x[i] - xm) * 0.5f : -INFINITY;
  float* z = x;

  float tau = 0.f, zthr = -INFINITY;
  if (row_role != 1) {
  // tau: the reference's 24 bisection steps.  Every midpoint lies in (-1, 0),
  // so a z <= -1 adds exactly 0 to every step's sum: the live values (z > -1,
  // usually the few near the row's max) are compacted through LDS into
  // NC <= 4 per lane first, and the steps loop over those alone (the whole row
  // when more than 256 are live).
  uint32_t live = 0;
#pragma unroll
  for (int i = 0; i < NPL; ++i) live |= z[i] > -1.f ? 1u << i : 0u;
  const int n_live = wave_sum_int(__popc(live));
  float lo = -1.f, hi = 0.f;
  if (n_live <= 4 * kWave) {
    int base = 0;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const bool lv = (live >> i) & 1u;
      const unsigned long long bal = __ballot(lv);
      if (lv) s_live[pr][base + __popcll(bal & lt)] = z[i];
      base += __popcll(bal);
    }
    wave_sync_lds();
    auto bisect = [&](auto nc_tag) __attribute__((always_inline)) {
      constexpr int NC = decltype(nc_tag)::value;
      float zc[NC];
#pragma unroll
      for (int k = 0; k < NC; ++k) zc[k] = lane + kWave * k < n_live ? s_live[pr][lane + kWave * k] : -INFINITY;
      for (int it = 0; it < kTauIters; ++it) {
        const float mid = (lo + hi) * 0.5f;
        double acc = 0.0;
#pragma unroll
        for (int k = 0; k < NC; ++k) {
          const float p = fmaxf(zc[k] - mid, 0.f);
          acc += (double)(p * p);
        }
        const float ssum = (float)wave_sum_f64(acc);
        if (ssum > 1.f) lo = mid;
        else hi = mid;
      }
    };
    if (n_live <= kWave) bisect(std::integral_constant<int, 1>{});
    else if (n_live <= 2 * kWave) bisect(std::integral_constant<int, 2>{});
    else bisect(std::integral_constant<int, 4>{});
  } else {
    for (int it = 0; it < kTauIters; ++it) {
      const float mid = (lo + hi) * 0.5f;
      double acc[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
      for (int i = 0; i < NPL; ++i) {
        const float p = fmaxf(z[i] - mid, 0.f);
        acc[i & 3] += (double)(p * p);
      }
      const float ssum = (float)wave_sum_f64((acc[0] + acc[1]) + (acc[2] + acc[3]));
      if (ssum > 1.f) lo = mid;
      else hi = mid;
    }
  }
  tau = (lo + hi) * 0.5f;
  }
  if (row_role != 0) {
  // budget: the (K+1)-th largest candidate z, then the reference's 40 steps
  if (n_cand > a.K) {
    uint32_t keys[NPL];
    uint32_t lmax = 0;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      keys[i] = ((cand >> i) & 1u) ? f32_order_key(z[i]) : 0u;
      lmax = max(lmax, keys[i]);
    }
    uint32_t kth = 0;
    bool found = false;
    if (a.K + 1 <= kWave) {
      const uint32_t T = __shfl(wave_sort_desc<uint32_t>(lmax, lane), a.K, kWave);
      int cnt = 0;
#pragma unroll
      for (int i = 0; i < NPL; ++i) cnt += keys[i] >= T ? 1 : 0;
      int incl = cnt;
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) {
        const int v = __shfl_up(incl, o, kWave);
        incl += lane >= o ? v : 0;
      }
      const int C = __shfl(incl, kWave - 1, kWave);
      if (C <= kWave) {
        int off = incl - cnt;
#pragma unroll
        for (int i = 0; i < NPL; ++i)
          if (keys[i] >= T) s_key[pr][off++] = keys[i];
        wave_sync_lds();
        kth = __shfl(wave_sort_desc<uint32_t>(lane < C ? s_key[pr][lane] : 0u, lane), a.K, kWave);
        found = true;
      }
    }
    if (!found) {   // largest t with at least K + 1 keys >= t, bit by bit from the top
      for (int bit = 31; bit >= 0; --bit) {
        const uint32_t t = kth | (1u << bit);
        int cnt = 0;
#pragma unroll
        for (int i = 0; i < NPL; ++i) cnt += keys[i] >= t ? 1 : 0;
        if (wave_sum_int(cnt) >= a.K + 1) kth = t;
      }
    }
    const float zk1 = f32_from_order_key(kth);
    float lo2 = zmin - 1.f, hi2 = 0.f;
    for (int it = 0; it < kCapIters; ++it) {
      const float mid = (lo2 + hi2) * 0.5f;
      if (zk1 > mid) lo2 = mid;
      else hi2 = mid;
    }
    zthr = hi2;
  }
  if (SPLIT && lane == 0) s_thr[pr] = zthr;
  }
  if constexpr (SPLIT) {
    __syncthreads();
    if (row_role == 1 || !live_row) return;
    zthr = s_thr[pr];
  } else if (!live_row) {
    return;
  }

  // mu over the active blocks (the log prior of those alone), then the packed
  // write
  float lp[NPL];
  uint32_t act = 0;
  double lsum = 0.0;
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const bool ac = ((cand >> i) & 1u) && z[i] > zthr;
    act |= ac ? 1u << i : 0u;
    lp[i] = 0.f;
    if (ac) {
      float pv = fmaxf(z[i] - tau, 0.f);
      pv = pv * pv;
      lp[i] = logf(fmaxf(pv, a.prior_floor));
      lsum += (double)lp[i];
    }
  }
  const int n_sel = wave_sum_int(__popc(act));
  const float mu = (float)wave_sum_f64(lsum) / (float)max(n_sel, 1);
  int32_t* oi = a.out_idx + row * a.oi_sn;
  float* ob = a.out_bias + row * a.ob_sn;
  int base = 0;
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const bool ac = (act >> i) & 1u;
    const unsigned long long bal = __ballot(ac);
    const int pos = base + __popcll(bal & lt);
    if (ac && pos < a.M) {
      oi[pos] = lane + kWave * i;
      ob[pos] = (lp[i] - mu) * a.inv_sigma;
    }
    base += __popcll(bal);
  }
  for (int s2 = min(base, a.M) + lane; s2 < a.M; s2 += kWave) {
    oi[s2] = -1;
    ob[s2] = 0.f;
  }
}

// One wavefront per decode query row.
__global__ __launch_bounds__(kRsWaves * kWave) void win_bounds_kernel(srswa_win_bounds_args a) {
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int row = blockIdx.x * kRsWaves + wave;
  if (row >= a.rows) return;
  const int r = row / a.dql;
  const int seq = a.seq_lens[r];
  const int q_pos = seq - a.dql + row % a.dql;
  const int q_blk = q_pos / a.block_size;
  const int8_t* al = a.allow + (int64_t)row * a.a_sn;
  const int lim = min(a.W, a.WQ);
  int lo = a.W, hi = -1;
  for (int j0 = 0; j0 < lim; j0 += kWave) {
    const int j = j0 + lane;
    const bool keep = j < lim && al[j] != 0 && j <= q_blk - a.local_blocks && (int64_t)j * a.block_size < seq;
    if (keep) { lo = min(lo, j); hi = max(hi, j); }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    lo = min(lo, __shfl_xor(lo, o, kWave));
    hi = max(hi, __shfl_xor(hi, o, kWave));
  }
  if (lane != 0) return;
  const bool any_r = hi >= 0;
  const int n_blk = (seq + a.block_size - 1) / a.block_size;
  const int w_seq = min(a.W, max(n_blk, 1));
  const bool no_remote = seq <= 0 || q_blk - a.local_blocks < 0;
  const int lo_v = any_r ? lo : 0;
  const int hi_v = any_r ? hi + 1 : (no_remote ? 0 : w_seq);
  a.lo[row] = lo_v;
  a.hi[row] = hi_v;
  a.fit[row] = (hi_v - lo_v) <= a.tile ? 1 : 0;
}

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s launch failed: %s", what, hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}

}  // namespace
}  // namespace srswa

using namespace srswa;

extern "C" int srswa_route_serve(const srswa_route_serve_args* a, void* stream) {
  if (!a || (a->rows > 0 && (!a->scores || !a->out_idx || !a->out_bias))) {
    set_error("route serve: null argument");
    return SRSWA_INVALID;
  }
  if (a->rows < 0 || a->W < 0 || a->M < 1 || a->K < 1) {
    set_error("route serve: bad sizes (rows %d, W %d, K %d, M %d)", a->rows, a->W, a->K, a->M);
    return SRSWA_INVALID;
  }
  if (a->rows == 0) return SRSWA_OK;
  const dim3 grid((unsigned)((a->rows + kRsWaves - 1) / kRsWaves));
  const dim3 grid2((unsigned)((a->rows + kRsWaves / 2 - 1) / (kRsWaves / 2)));
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  // two waves per row while those waves fit one per SIMD (a decode step); a
  // prefill chunk, which fills the GPU, keeps one wave per row
  const int cus = device_cu_count();
  const bool split = cus > 0 && (int64_t)a->rows * 2 <= (int64_t)cus * 4;
  if (a->W <= 8 * kWave) {
    if (split) hipLaunchKernelGGL((route_entmax_regs_kernel<8, true>), grid2, dim3(kRsWaves * kWave), 0, st, *a);
    else hipLaunchKernelGGL((route_entmax_regs_kernel<8, false>), grid, dim3(kRsWaves * kWave), 0, st, *a);
  } else if (a->W <= 32 * kWave) {
    if (split) hipLaunchKernelGGL((route_entmax_regs_kernel<32, true>), grid2, dim3(kRsWaves * kWave), 0, st, *a);
    else hipLaunchKernelGGL((route_entmax_regs_kernel<32, false>), grid, dim3(kRsWaves * kWave), 0, st, *a);
  } else
    hipLaunchKernelGGL(route_entmax_kernel, grid, dim3(kRsWaves * kWave), 0, st, *a);
  return launch_status("route serve");
}

extern "C" int srswa_win_bounds(const srswa_win_bounds_args* a, void* stream) {
  if (!a || (a->rows > 0 && (!a->allow || !a->seq_lens || !a->lo || !a->hi || !a->fit))) {
    set_error("win bounds: null argument");
    return SRSWA_INVALID;
  }
  if (a->rows < 0 || a->W < 0 || a->WQ < 0 || a->block_size <= 0 || a->local_blocks < 0 || a->dql <= 0) {
    set_error("win bounds: bad sizes");
    return SRSWA_INVALID;
  }
  if (a->rows == 0) return SRSWA_OK;
  const dim3 grid((unsigned)((a->rows + kRsWaves - 1) / kRsWaves));
  hipLaunchKernelGGL(win_bounds_kernel, grid, dim3(kRsWaves * kWave), 0, reinterpret_cast<hipStream_t>(stream), *a);
  return launch_status("win bounds");
}
