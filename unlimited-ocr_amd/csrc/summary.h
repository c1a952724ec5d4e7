// Block summary keys k_bar for the DASH stage-0 scorer (gfx950): the mean of
// a block's keys, or their head_cls softmax-weighted mean.
//
// Restates _summary_keys (WHL!layers/attention/unlimited_dash_ops/
// dash_stage0.py:25-43) and the head_cls branch of _block_scores_infer
// (HF/modeling_deepseekv2.py:391-404): logits aw = clamp(k.head_cls / sqrt(d),
// +-1e4) over the block's real keys, w = softmax(aw), k_bar = sum w k (fp32).
// A zero head_cls gives uniform weights, the plain mean.
#pragma once

#include "common.h"

namespace srswa {

constexpr float kScoreNeg = -1.0e9f;   // _SCORE_NEG, HF/dash_attention.py:741
constexpr float kActClamp = 1.0e4f;    // _ACT_CLAMP, HF/dash_attention.py:747

// One wavefront summarises nkeys (>= 1) key rows: row j at kbase + j * k_st,
// where kbase already points at this lane's column slice (c * EPV, c = lane %
// LPR).  16-byte loads, LPR lanes per row (whole 128-byte lines per
// instruction); with HC the per-key logits are finished by a reduce-scatter
// over the LPR lanes of a row and folded in by an online softmax (the weights
// broadcast through s_w, 64 floats of LDS).  On return kb[] holds this lane's
// slice of k_bar on every lane.
template <typename T, int D, bool HC>
__device__ __forceinline__ void summarize_rows(const T* kbase, int64_t k_st, int nkeys, const float* hc,
                                               float inv_sqrt_d, float* s_w, float* kb) {
  using V = Vec16<T>;
  constexpr int EPV = V::N;
  constexpr int LPR = D / EPV;         // lanes per key row
  constexpr int RPI = kWave / LPR;     // rows per load instruction
  constexpr int NI = kWave / RPI;      // instructions per 64-row chunk (== LPR)
  const int lane = threadIdx.x % kWave;
  const int r = lane / LPR, c = lane % LPR;
#pragma unroll
  for (int e = 0; e < EPV; ++e) kb[e] = 0.f;
  float hcf[EPV];
  if (HC) {
#pragma unroll
    for (int e = 0; e < EPV; ++e) hcf[e] = hc[e];
  }
  float wsum = 0.f, wmax = -INFINITY;  // head_cls softmax state (HC)
  for (int j0 = 0; j0 < nkeys; j0 += NI * RPI) {
    uint4 kr[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int key = j0 + i * RPI + r;
      kr[i] = key < nkeys ? *reinterpret_cast<const uint4*>(kbase + (int64_t)key * k_st) : make_uint4(0, 0, 0, 0);
    }
    if (!HC) {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        float f[EPV];
        V::unpack(kr[i], f);
#pragma unroll
        for (int e = 0; e < EPV; ++e) kb[e] += f[e];
      }
    } else {
      // per-key logits k.hc / sqrt(d): reduce-scatter over the LPR lanes of a row
      float part[NI];
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        float f[EPV];
        V::unpack(kr[i], f);
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < EPV; ++e) s = fmaf(f[e], hcf[e], s);
        part[i] = s;
      }
      reduce_scatter<NI, LPR / 2>(part, c);
      const int key = j0 + c * RPI + r;                 // the key this lane owns
      float aw = fminf(fmaxf(part[0] * inv_sqrt_d, -kActClamp), kActClamp);
      aw = key < nkeys ? aw : -INFINITY;
      const float mnew = fmaxf(wmax, wave_max(aw));
      const float alpha = exp2f((wmax - mnew) * kLog2e);
      const float w = key < nkeys ? exp2f((aw - mnew) * kLog2e) : 0.f;
      wsum = wsum * alpha + wave_sum(w);
      wmax = mnew;
#pragma unroll
      for (int e = 0; e < EPV; ++e) kb[e] *= alpha;
      s_w[r * NI + c] = w;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const float wi = s_w[r * NI + i];
        float f[EPV];
        V::unpack(kr[i], f);
#pragma unroll
        for (int e = 0; e < EPV; ++e) kb[e] = fmaf(wi, f[e], kb[e]);
      }
      __builtin_amdgcn_wave_barrier();
    }
  }
  // sum the RPI row groups, then normalise
#pragma unroll
  for (int o = LPR; o < kWave; o <<= 1)
#pragma unroll
    for (int e = 0; e < EPV; ++e) kb[e] += __shfl_xor(kb[e], o, kWave);
  const float norm = HC ? 1.f / fmaxf(wsum, 1e-6f) : 1.f / (float)nkeys;
#pragma unroll
  for (int e = 0; e < EPV; ++e) kb[e] *= norm;
}

}  // namespace srswa
