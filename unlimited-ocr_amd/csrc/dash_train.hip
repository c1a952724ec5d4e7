// Training DASH router on the GPU: DashAttention._route / _select_and_bias
// (HF/dash_attention.py:1145-1204) with the 1.5-entmax of :764-810, forward
// and backward.  Between the block scorer and the e2e gather kernels of the
// sparse training step (:1302-1303): block scores [rows, nblk] -> prior
// [rows, nblk] -> (top-K ids, centred log-prior bias, valid) and back.
//
// One wavefront per query row.  Elementwise steps round to the storage dtype
// where the reference's tensors do (bf16 training runs the whole router in
// bf16); reductions accumulate in fp32, the entmax threshold in fp64:
//   route:  candidates (score > -5e8, under the row's block / image mask,
//           falling back to every remote block), x, z = (x - max) / 2; the z
//           above -1 (every support member: tau >= max z - 1) are compacted and
//           sorted descending (bitonic: across the wave when at most 64, else
//           in LDS), their fp64 prefix sums give each
//           rank's closed-form threshold tau_r = mean - sqrt(max((1 - ss) / r,
//           0)), support = #{r : tau_r <= z_(r)}, prior = max(z - tau_support, 0)^2;
//   select: the top K of the 64-bit keys (order key of the masked prior,
//           ~block id) by a lane-maximum threshold and a wave sort, then the
//           bias of the K slots by wave reductions;
//   backward: select scatters d topv into a dense LDS row (one wave per
//           workgroup), route applies the entmax Jacobian-vector product.
#include <algorithm>

#include "common.h"

namespace srswa {
namespace {

constexpr float kRemoteCut = -5.0e8f;   // _SCORE_NEG * 0.5, HF/dash_attention.py:741, 1158
constexpr float kActClamp = 1.0e4f;     // _ACT_CLAMP

template <typename T> __device__ __forceinline__ float ldv(const void* p, int64_t i);
template <> __device__ __forceinline__ float ldv<float>(const void* p, int64_t i) {
  return reinterpret_cast<const float*>(p)[i];
}
template <> __device__ __forceinline__ float ldv<bf16_t>(const void* p, int64_t i) {
  return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(p)[i] << 16);
}
template <> __device__ __forceinline__ float ldv<__half>(const void* p, int64_t i) {
  return __half2float(reinterpret_cast<const __half*>(p)[i]);
}

// v rounded to the storage dtype (and back to fp32)
template <typename T> __device__ __forceinline__ float rnd(float v);
template <> __device__ __forceinline__ float rnd<float>(float v) { return v; }
template <> __device__ __forceinline__ float rnd<bf16_t>(float v) { return bf16_lo(pack_bf16x2(v, 0.f)); }
template <> __device__ __forceinline__ float rnd<__half>(float v) { return __half2float(__float2half_rn(v)); }

template <typename T> __device__ __forceinline__ void stv(void* p, int64_t i, float v);
template <> __device__ __forceinline__ void stv<float>(void* p, int64_t i, float v) {
  reinterpret_cast<float*>(p)[i] = v;
}
template <> __device__ __forceinline__ void stv<bf16_t>(void* p, int64_t i, float v) {
  reinterpret_cast<uint16_t*>(p)[i] = f32_to_bf16_rne(v);
}
template <> __device__ __forceinline__ void stv<__half>(void* p, int64_t i, float v) {
  reinterpret_cast<__half*>(p)[i] = __float2half_rn(v);
}

// closed-form 1.5-entmax threshold of the r largest z (sums s1, s2 of z, z^2)
__device__ __forceinline__ double entmax_tau(double s1, double s2, int r) {
  const double mean = s1 / r, msq = s2 / r;
  const double ss = r * (msq - mean * mean);
  const double delta = (1.0 - ss) / r;
  return mean - sqrt(delta > 0.0 ? delta : 0.0);
}

// ------------------------------------------------------------ route forward
// x of one block (before the max shift) from its score and mask bit
template <typename T>
__device__ __forceinline__ float route_x(const srswa_dash_route_train_args& a, float s, bool m, bool& cand) {
  cand = s > kRemoteCut && m;
  float x = cand ? rnd<T>(s * a.scale) : rnd<T>(a.neg);
  if (!__builtin_isfinite(x)) x = rnd<T>(a.neg);
  return x;
}

// Sort the c (<= pcap) floats of s_z descending in LDS (bitonic over the
// next power of two >= max(c, 64), padded with -inf); one wave per workgroup.
__device__ __forceinline__ int lds_sort_desc(float* s_z, int c, int lane) {
  int P = kWave;
  while (P < c) P <<= 1;
  for (int i = c + lane; i < P; i += kWave) s_z[i] = -INFINITY;
  __syncthreads();
  for (int k = 2; k <= P; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int t = lane; t < P / 2; t += kWave) {
        const int i = 2 * j * (t / j) + (t % j), l = i + j;
        const float vi = s_z[i], vl = s_z[l];
        const bool desc = (i & k) == 0;
        if (desc ? (vi < vl) : (vi > vl)) {
          s_z[i] = vl;
          s_z[l] = vi;
        }
      }
      __syncthreads();
    }
  }
  return P;
}

// tau of the c largest z, sorted descending: E per lane in s_z (lane-major),
// or one per lane in `mine` (E == 0)
__device__ __forceinline__ double entmax_threshold(const float* s_z, float mine, int c, int E, int lane) {
  const int per = E > 0 ? E : 1;
  auto val = [&](int e) __attribute__((always_inline)) { return E > 0 ? (double)s_z[lane * E + e] : (double)mine; };
  double l1 = 0.0, l2 = 0.0;
  for (int e = 0; e < per; ++e)
    if (lane * per + e < c) {
      const double v = val(e);
      l1 += v;
      l2 += v * v;
    }
  double i1 = l1, i2 = l2;                          // inclusive scan over lanes
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const double t1 = __shfl_up(i1, o, kWave), t2 = __shfl_up(i2, o, kWave);
    if (lane >= o) {
      i1 += t1;
      i2 += t2;
    }
  }
  double b1 = __shfl_up(i1, 1, kWave), b2 = __shfl_up(i2, 1, kWave);
  if (lane == 0) b1 = b2 = 0.0;
  // support = #{ranks r with tau_r <= z_(r)}; tau_r of every rank this lane holds
  int cnt = 0;
  double s1 = b1, s2 = b2;
  for (int e = 0; e < per; ++e)
    if (lane * per + e < c) {
      const double v = val(e);
      s1 += v;
      s2 += v * v;
      cnt += entmax_tau(s1, s2, lane * per + e + 1) <= v ? 1 : 0;
    }
  const int support = max(wave_sum_int(cnt), 1);
  const int owner = (support - 1) / per;
  double tau = 0.0;
  if (lane == owner) {
    s1 = b1;
    s2 = b2;
    for (int e = 0; lane * per + e < support; ++e) {
      const double v = val(e);
      s1 += v;
      s2 += v * v;
    }
    tau = entmax_tau(s1, s2, support);
  }
  return __shfl(tau, owner, kWave);
}

// NPL > 0: the row's scores and mask bits stay in registers (block i = lane +
// 64 t); NPL == 0 re-reads the row for every pass (rows above 1024 blocks).
// The z above -1 (usually few) are sorted across the wave when at most 64,
// else in LDS.
template <typename T, int NPL>
__global__ __launch_bounds__(kWave) void route_train_kernel(srswa_dash_route_train_args a, int pcap) {
  extern __shared__ float s_z[];                    // [pcap]
  const int lane = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int n = a.nblk;
  const void* sr = reinterpret_cast<const char*>(a.scores) + row * a.sc_sr * (int64_t)sizeof(T);
  const uint8_t* bc = a.block_cand ? a.block_cand + row * a.bc_sr : nullptr;
  const uint8_t* im = (!bc && a.img) ? a.img + (row / a.rows_per_seq) * a.img_sb : nullptr;
  constexpr int NR = NPL > 0 ? NPL : 1;
  float sv[NR];
  bool mv[NR];
  auto score = [&](int t, int i) __attribute__((always_inline)) { return NPL > 0 ? sv[t] : ldv<T>(sr, i); };
  auto maskb = [&](int t, int i) __attribute__((always_inline)) {
    return NPL > 0 ? mv[t] : (bc ? bc[i] != 0 : (im ? im[i] != 0 : true));
  };
  if constexpr (NPL > 0) {
    // two unconditional batches of loads (block clamped to the row, the tail
    // masked after): under a per-block branch each load waits out its own
    // round trip
    const uint8_t* mrow = bc ? bc : im;
    uint8_t mb[NR];
    if (n > 0) {
#pragma unroll
      for (int t = 0; t < NPL; ++t) sv[t] = ldv<T>(sr, min(lane + kWave * t, n - 1));
      if (mrow) {
#pragma unroll
        for (int t = 0; t < NPL; ++t) mb[t] = mrow[min(lane + kWave * t, n - 1)];
      }
    }
#pragma unroll
    for (int t = 0; t < NPL; ++t) {
      const int i = lane + kWave * t;
      sv[t] = i < n ? sv[t] : -INFINITY;
      mv[t] = i < n && (mrow ? mb[t] != 0 : true);
    }
  }
  const int nt = NPL > 0 ? NPL : ceil_div(n, kWave);

  // the row's mask applies when it leaves a candidate (HF/dash_attention.py:1159-1165)
  bool any_masked = false;
  if (bc || im) {
    for (int t = 0; t < nt; ++t) {
      const int i = lane + kWave * t;
      if (i < n) any_masked |= score(t, i) > kRemoteCut && maskb(t, i);
    }
  }
  const bool use_mask = (bc || im) && __any(any_masked);

  float xm = -INFINITY;
  for (int t = 0; t < nt; ++t) {
    const int i = lane + kWave * t;
    bool cd;
    if (i < n) xm = fmaxf(xm, route_x<T>(a, score(t, i), !use_mask || maskb(t, i), cd));
  }
  xm = wave_max(xm);

  // z = (x - max) / 2 (kept in sv for NPL > 0), cand written, the z > -1 counted
  uint8_t* cr = a.cand + row * a.c_sr;
  int cnt_hi = 0;
  for (int t = 0; t < nt; ++t) {
    const int i = lane + kWave * t;
    if (i < n) {
      bool cd;
      const float z = rnd<T>(route_x<T>(a, score(t, i), !use_mask || maskb(t, i), cd) - xm) * 0.5f;
      cr[i] = cd ? 1 : 0;
      cnt_hi += z > -1.f ? 1 : 0;
      if constexpr (NPL > 0) sv[t] = z;
    }
  }
  const int c = wave_sum_int(cnt_hi);
  // compaction of the z > -1 into s_z (ascending block order)
  {
    int base = 0;
    for (int t = 0; t < nt; ++t) {
      const int i = lane + kWave * t;
      float z = -INFINITY;
      if (i < n) {
        if constexpr (NPL > 0) {
          z = sv[t];
        } else {
          bool cd;
          z = rnd<T>(route_x<T>(a, score(t, i), !use_mask || maskb(t, i), cd) - xm) * 0.5f;
        }
      }
      const bool keep = z > -1.f;
      const uint64_t bal = __ballot(keep);
      if (keep) s_z[base + __popcll(bal & ((1ull << lane) - 1ull))] = z;
      base += __popcll(bal);
    }
  }
  double tau;
  if (c <= kWave) {
    __syncthreads();
    const float mine = wave_sort_desc<float>(lane < c ? s_z[lane] : -INFINITY, lane);
    tau = entmax_threshold(nullptr, mine, c, 0, lane);
  } else {
    const int P = lds_sort_desc(s_z, c, lane);
    tau = entmax_threshold(s_z, 0.f, c, P / kWave, lane);
  }

  void* pr = reinterpret_cast<char*>(a.prior) + row * a.p_sr * (int64_t)sizeof(T);
  for (int t = 0; t < nt; ++t) {
    const int i = lane + kWave * t;
    if (i < n) {
      float z;
      if constexpr (NPL > 0) {
        z = sv[t];
      } else {
        bool cd;
        z = rnd<T>(route_x<T>(a, score(t, i), !use_mask || maskb(t, i), cd) - xm) * 0.5f;
      }
      const float d = rnd<T>(fmaxf((float)((double)z - tau), 0.f));
      stv<T>(pr, i, d * d);
    }
  }
}

// ----------------------------------------------------------- route backward
template <typename T>
__global__ __launch_bounds__(256) void route_train_bwd_kernel(srswa_dash_route_train_bwd_args a) {
  const int lane = threadIdx.x % kWave;
  const int64_t row = (int64_t)blockIdx.x * 4 + threadIdx.x / kWave;
  if (row >= a.rows) return;
  const int n = a.nblk;
  const int64_t es = sizeof(T);
  const void* dyr = reinterpret_cast<const char*>(a.d_prior) + row * a.dp_sr * es;
  const void* yr = reinterpret_cast<const char*>(a.prior) + row * a.p_sr * es;
  const uint8_t* cr = a.cand + row * a.c_sr;
  void* dsr = reinterpret_cast<char*>(a.d_scores) + row * a.ds_sr * es;
  float sdx = 0.f, sg = 0.f;
  for (int i = lane; i < n; i += kWave) {
    const float g = rnd<T>(sqrtf(ldv<T>(yr, i)));
    sdx += rnd<T>(ldv<T>(dyr, i) * g);
    sg += g;
  }
  sdx = rnd<T>(wave_sum(sdx));
  sg = rnd<T>(wave_sum(sg));
  const float q = rnd<T>(sdx / fmaxf(sg, rnd<T>(1e-12f)));
  for (int i = lane; i < n; i += kWave) {
    const float g = rnd<T>(sqrtf(ldv<T>(yr, i)));
    const float dx = rnd<T>(rnd<T>(ldv<T>(dyr, i) * g) - rnd<T>(q * g));
    stv<T>(dsr, i, cr[i] ? dx * a.scale : 0.f);
  }
}

// ----------------------------------------------------------------- select
// The K slots of the row: lane j < K ends with slot j's key (order key of sel
// << 32 | ~block id, unique per block).  NPL > 0 keeps the row's keys in
// registers and finds them without K rounds over every key: the K-th largest
// of the 64 lane maxima is a threshold with at least K keys at or above it;
// those keys (at most 64 in an ordinary row) are compacted through LDS and
// sorted across the wave.  More than 64, or NPL == 0 (rows above 1024
// blocks): K rounds of "largest key below the previous one".
template <typename T, int NPL>
__device__ __forceinline__ uint64_t select_keys(const srswa_dash_select_train_args& a, int64_t row, int lane,
                                                uint64_t* s_sel) {
  const int n = a.nblk;
  const int64_t es = sizeof(T);
  const void* pr = reinterpret_cast<const char*>(a.prior) + row * a.p_sr * es;
  const uint8_t* cr = a.cand + row * a.c_sr;
  auto key_of = [&](int i) __attribute__((always_inline)) {
    const float sel = cr[i] ? ldv<T>(pr, i) : -1.f;
    return ((uint64_t)f32_order_key(sel) << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
  };
  constexpr int NR = NPL > 0 ? NPL : 1;
  uint64_t keys[NR];
  if constexpr (NPL > 0) {
    // candidate bytes and priors as two unconditional batches of loads (block
    // clamped to the row, the tail masked after), so they are in flight together
    uint8_t cb[NPL];
    float pv[NPL];
    if (n > 0) {
#pragma unroll
      for (int t = 0; t < NPL; ++t) cb[t] = cr[min(lane + kWave * t, n - 1)];
#pragma unroll
      for (int t = 0; t < NPL; ++t) pv[t] = ldv<T>(pr, min(lane + kWave * t, n - 1));
    }
    uint64_t lmax = 0ull;
#pragma unroll
    for (int t = 0; t < NPL; ++t) {
      const int i = lane + kWave * t;
      const float sel = cb[t] ? pv[t] : -1.f;
      keys[t] = i < n ? ((uint64_t)f32_order_key(sel) << 32) | (uint64_t)(0xffffffffu - (uint32_t)i) : 0ull;
      lmax = keys[t] > lmax ? keys[t] : lmax;
    }
    // K <= min(n, 64) lanes hold a real key, so the threshold is a real key
    const uint64_t T_ = __shfl(wave_sort_desc<uint64_t>(lmax, lane), a.K - 1, kWave);
    int cnt = 0;
#pragma unroll
    for (int t = 0; t < NPL; ++t) cnt += keys[t] >= T_ ? 1 : 0;
    int incl = cnt;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int v = __shfl_up(incl, o, kWave);
      incl += lane >= o ? v : 0;
    }
    const int total = __shfl(incl, kWave - 1, kWave);
    if (total <= kWave) {
      int off = incl - cnt;
#pragma unroll
      for (int t = 0; t < NPL; ++t)
        if (keys[t] >= T_) s_sel[off++] = keys[t];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      return wave_sort_desc<uint64_t>(lane < total ? s_sel[lane] : 0ull, lane);
    }
  }
  uint64_t prev = ~0ull, mine = 0ull;
  for (int s = 0; s < a.K; ++s) {
    uint64_t best = 0ull;
    if constexpr (NPL > 0) {
#pragma unroll
      for (int t = 0; t < NPL; ++t) best = (keys[t] < prev && keys[t] > best) ? keys[t] : best;
    } else {
      for (int i = lane; i < n; i += kWave) {
        const uint64_t k = key_of(i);
        best = (k < prev && k > best) ? k : best;
      }
    }
    best = wave_max_u64(best);
    if (lane == s) mine = best;
    prev = best;
  }
  return mine;
}

// bias terms of slot `lane` (< K) from its key
template <typename T>
struct SlotBias {
  float topv, clamped, logp, mu, pre;
  bool valid;
  int cnt;
};

template <typename T>
__device__ __forceinline__ SlotBias<T> slot_bias(const srswa_dash_select_train_args& a, float topv, bool live) {
  SlotBias<T> b;
  b.topv = topv;
  b.valid = live && topv >= 0.f;
  b.clamped = rnd<T>(fmaxf(topv, a.floor));        // clamp_min(floor) in the storage dtype
  b.logp = rnd<T>(logf(b.clamped));
  b.cnt = __popcll(__ballot(b.valid));
  const float sum = rnd<T>(wave_sum(b.valid ? b.logp : 0.f));
  b.mu = rnd<T>(sum / (float)max(b.cnt, 1));
  b.pre = rnd<T>(rnd<T>(b.logp - b.mu) * a.inv_sigma);
  return b;
}

template <typename T, int NPL>
__global__ __launch_bounds__(256) void select_train_kernel(srswa_dash_select_train_args a) {
  __shared__ uint64_t s_sel[4][kWave];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int64_t row = (int64_t)blockIdx.x * 4 + wave;
  if (row >= a.rows) return;
  const uint64_t key = select_keys<T, NPL>(a, row, lane, s_sel[wave]);
  const bool live = lane < a.K;
  const int id = (int)(0xffffffffu - (uint32_t)key);
  const float topv = f32_from_order_key((uint32_t)(key >> 32));
  const SlotBias<T> b = slot_bias<T>(a, topv, live);
  if (live) {
    a.topi[row * a.ti_sr + lane] = id;
    a.valid[row * a.v_sr + lane] = b.valid ? 1 : 0;
    if (a.bias) {
      const float v = b.valid ? fminf(fmaxf(b.pre, -kActClamp), kActClamp) : 0.f;
      stv<T>(reinterpret_cast<char*>(a.bias) + row * a.b_sr * (int64_t)sizeof(T), lane, v);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kWave) void select_train_bwd_kernel(srswa_dash_select_train_args a) {
  extern __shared__ float s_row[];                 // [nblk] d prior of the row
  const int lane = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int n = a.nblk;
  const int64_t es = sizeof(T);
  for (int i = lane; i < n; i += kWave) s_row[i] = 0.f;
  const bool live = lane < a.K;
  int id = 0;
  float topv = -1.f, g = 0.f;
  if (live) {
    id = (int)a.topi[row * a.ti_sr + lane];
    id = min(max(id, 0), n - 1);                   // ids come from the forward: 0 <= id < nblk
    const bool cd = a.cand[row * a.c_sr + id] != 0;
    topv = cd ? ldv<T>(reinterpret_cast<const char*>(a.prior) + row * a.p_sr * es, id) : -1.f;
    g = ldv<T>(reinterpret_cast<const char*>(a.d_bias) + row * a.db_sr * es, lane);
  }
  const SlotBias<T> b = slot_bias<T>(a, topv, live);
  const bool pass = b.valid && b.pre >= -kActClamp && b.pre <= kActClamp;
  const float u = pass ? g * a.inv_sigma : 0.f;
  const float U = wave_sum(u);
  const float dlogp = u - (b.valid ? U / (float)max(b.cnt, 1) : 0.f);
  // log backward divides by the clamped value; clamp_min passes where topv >= floor
  const float dtop = (live && topv >= a.floor) ? dlogp / b.clamped : 0.f;
  __syncthreads();
  if (live) s_row[id] = dtop;
  __syncthreads();
  void* dr = reinterpret_cast<char*>(a.d_prior) + row * a.dp_sr * es;
  for (int i = lane; i < n; i += kWave) stv<T>(dr, i, s_row[i]);
}

size_t esize(int dtype) { return dtype == SRSWA_F32 ? 4 : 2; }

int check_dtype(int dtype, const char* what) {
  if (dtype != SRSWA_F32 && dtype != SRSWA_BF16 && dtype != SRSWA_F16) {
    set_error("%s: dtype %d not supported", what, dtype);
    return SRSWA_UNSUPPORTED;
  }
  return SRSWA_OK;
}

constexpr int kMaxBlocks = 8192;    // LDS row of one wavefront: 32 KB

template <typename T>
void launch_route(const srswa_dash_route_train_args& a, int pcap, hipStream_t s) {
  const size_t lds = (size_t)pcap * sizeof(float);
  if (a.nblk <= 4 * kWave)
    hipLaunchKernelGGL((route_train_kernel<T, 4>), dim3(a.rows), dim3(kWave), lds, s, a, pcap);
  else if (a.nblk <= 16 * kWave)
    hipLaunchKernelGGL((route_train_kernel<T, 16>), dim3(a.rows), dim3(kWave), lds, s, a, pcap);
  else
    hipLaunchKernelGGL((route_train_kernel<T, 0>), dim3(a.rows), dim3(kWave), lds, s, a, pcap);
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

extern "C" int srswa_dash_route_train(const srswa_dash_route_train_args* a, void* stream) {
  if (!a || !a->scores || !a->prior || !a->cand || a->rows < 0 || a->nblk < 0) {
    set_error("dash route train: bad arguments");
    return SRSWA_INVALID;
  }
  if (a->img && !a->block_cand && a->rows_per_seq <= 0) {
    set_error("dash route train: rows_per_seq must be positive with an image mask");
    return SRSWA_INVALID;
  }
  int rc = check_dtype(a->dtype, "dash route train");
  if (rc != SRSWA_OK) return rc;
  if (a->nblk > kMaxBlocks) {
    set_error("dash route train: %d blocks per row (at most %d)", a->nblk, kMaxBlocks);
    return SRSWA_UNSUPPORTED;
  }
  if (a->rows == 0 || a->nblk == 0) return SRSWA_OK;
  int pcap = kWave;
  while (pcap < a->nblk) pcap <<= 1;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (a->dtype == SRSWA_F32) launch_route<float>(*a, pcap, s);
  else if (a->dtype == SRSWA_BF16) launch_route<bf16_t>(*a, pcap, s);
  else launch_route<__half>(*a, pcap, s);
  return launch_status("dash route train");
}

extern "C" int srswa_dash_route_train_bwd(const srswa_dash_route_train_bwd_args* a, void* stream) {
  if (!a || !a->d_prior || !a->prior || !a->cand || !a->d_scores || a->rows < 0 || a->nblk < 0) {
    set_error("dash route train bwd: bad arguments");
    return SRSWA_INVALID;
  }
  int rc = check_dtype(a->dtype, "dash route train bwd");
  if (rc != SRSWA_OK) return rc;
  if (a->rows == 0 || a->nblk == 0) return SRSWA_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)ceil_div(a->rows, 4));
  if (a->dtype == SRSWA_F32)
    hipLaunchKernelGGL(route_train_bwd_kernel<float>, grid, dim3(256), 0, s, *a);
  else if (a->dtype == SRSWA_BF16)
    hipLaunchKernelGGL(route_train_bwd_kernel<bf16_t>, grid, dim3(256), 0, s, *a);
  else
    hipLaunchKernelGGL(route_train_bwd_kernel<__half>, grid, dim3(256), 0, s, *a);
  return launch_status("dash route train bwd");
}

namespace {
int check_select(const srswa_dash_select_train_args* a, bool bwd) {
  if (!a || !a->prior || !a->cand || !a->topi || a->rows < 0 || a->nblk < 0 || a->K < 0 ||
      (!bwd && !a->valid) || (bwd && (!a->d_bias || !a->d_prior))) {
    set_error("dash select train: bad arguments");
    return SRSWA_INVALID;
  }
  int rc = check_dtype(a->dtype, "dash select train");
  if (rc != SRSWA_OK) return rc;
  if (a->K > kWave || a->K > a->nblk) {
    set_error("dash select train: K = %d (at most 64 and nblk = %d)", a->K, a->nblk);
    return SRSWA_UNSUPPORTED;
  }
  if (a->nblk > kMaxBlocks) {
    set_error("dash select train: %d blocks per row (at most %d)", a->nblk, kMaxBlocks);
    return SRSWA_UNSUPPORTED;
  }
  return SRSWA_OK;
}

template <typename T>
void launch_select(const srswa_dash_select_train_args& a, hipStream_t s) {
  const dim3 grid((unsigned)ceil_div(a.rows, 4));
  if (a.nblk <= 4 * kWave)
    hipLaunchKernelGGL((select_train_kernel<T, 4>), grid, dim3(256), 0, s, a);
  else if (a.nblk <= 16 * kWave)
    hipLaunchKernelGGL((select_train_kernel<T, 16>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((select_train_kernel<T, 0>), grid, dim3(256), 0, s, a);
}
}  // namespace

extern "C" int srswa_dash_select_train(const srswa_dash_select_train_args* a, void* stream) {
  int rc = check_select(a, false);
  if (rc != SRSWA_OK) return rc;
  if (a->rows == 0 || a->K == 0) return SRSWA_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (a->dtype == SRSWA_F32) launch_select<float>(*a, s);
  else if (a->dtype == SRSWA_BF16) launch_select<bf16_t>(*a, s);
  else launch_select<__half>(*a, s);
  return launch_status("dash select train");
}

extern "C" int srswa_dash_select_train_bwd(const srswa_dash_select_train_args* a, void* stream) {
  int rc = check_select(a, true);
  if (rc != SRSWA_OK) return rc;
  if (a->rows == 0 || a->nblk == 0) return SRSWA_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const size_t lds = (size_t)a->nblk * sizeof(float);
  if (a->dtype == SRSWA_F32)
    hipLaunchKernelGGL(select_train_bwd_kernel<float>, dim3(a->rows), dim3(kWave), lds, s, *a);
  else if (a->dtype == SRSWA_BF16)
    hipLaunchKernelGGL(select_train_bwd_kernel<bf16_t>, dim3(a->rows), dim3(kWave), lds, s, *a);
  else
    hipLaunchKernelGGL(select_train_bwd_kernel<__half>, dim3(a->rows), dim3(kWave), lds, s, *a);
  return launch_status("dash select train bwd");
}
