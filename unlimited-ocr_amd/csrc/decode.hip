// Decode gather-attention for gfx950 (MI355X).
//
// Replaces the reference's decode attend: _decode_attend
// (HF/modeling_deepseekv2.py:454-481) and SGLang's dash_sparse_attn_decode
// (WHL!layers/attention/unlimited_dash_ops/attend_triton.py:307-518 + the LSE
// merge in WHL!layers/attention/unlimited_dash_ops/common.py:44-89).
//
// Work decomposition.  The keys one query row reads are cut into "units" of
// UK keys: ceil(BS/UK) units per selected remote block slot, then
// ceil(LW/UK) units tiling the token window (q_pos-LW, q_pos] from its first
// key (the window is contiguous, so its units need not be block aligned).  A
// paged window's units sit on the UK grid inside one page each; its first
// unit also carries the window's last keys, so it still takes LW/UK units.
// One wavefront streams one or more units:
//   * K and V rows are read straight into VGPRs with 16-byte loads, LPR lanes
//     per key row (bf16, D=128: 16 lanes x 16 B = the row's two 128-byte
//     lines), so every load instruction moves whole cache lines;
//   * q.k partial sums are finished by a butterfly reduce-scatter across the
//     LPR lanes of a row (each lane ends holding one key's score);
//   * online softmax in the log2 domain (wave max/sum via shuffles), p is
//     broadcast back through 256 bytes of LDS per wave, then o += p v;
// Four waves (one workgroup; eight with fp8 caches) merge their (m, l, o) in LDS; the workgroups of
// one (row, head) write (O, M, L) records to a scratch buffer, and a second
// small kernel combines them (decode_merge_kernel).
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include <atomic>
#include <mutex>

#include "common.h"

namespace srswa {

static thread_local char g_err[512];
void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}
const char* last_error() { return g_err; }

namespace {

constexpr int kDecodeWaves = 4;   // waves per workgroup

struct DecodePlan {
  int UK;              // keys per unit
  int upb;             // units per remote block slot
  int n_remote_units;  // S * upb
  int n_units;         // + window units
  int upw;             // units per wave
  int nsplit;          // workgroups per (row, head)
  int pstride;         // floats per partial record (128-byte multiple)
  int64_t rowheads;    // B * Lq * HQ
  int gq;              // query heads per workgroup (gqa_heads)
  int nw;              // waves per workgroup
};

struct DecodeK {
  srswa_decode_args a;
  int G, IG;
  int UK, upb, n_remote_units, n_units, upw, nsplit, pstride;
  float scale_l2;      // scale * log2(e)
  int64_t rowheads;
  float* part;
  // paged cache (PAGED kernels): key j of sequence b lives in page
  // bt[b * bt_sb + j / block_size] at row j % block_size; q positions come
  // from kv_len: q_pos = kv_len[b] - Lq + lq
  const int32_t* bt;
  int64_t bt_sb, k_pst, v_pst;   // block-table row stride, page strides (elements)
  int bs_shift, max_blocks;
  int kv8;                       // FP8 kernels: the caches' fp8 format (srswa_dtype)
  int gq;                        // query heads per workgroup (gqa_heads)
  int nw;                        // waves per workgroup (4; the fp8 paged form 8)
};

template <typename TO>
__device__ __forceinline__ void store_out(TO* dst, const float* f, int n);
template <>
__device__ __forceinline__ void store_out<float>(float* dst, const float* f, int n) {
  if (n % 4 != 0) {
    for (int e = 0; e < n; ++e) dst[e] = f[e];
    return;
  }
  for (int e = 0; e < n; e += 4)
    *reinterpret_cast<uint4*>(dst + e) = Vec16<float>::pack(f + e);
}
template <>
__device__ __forceinline__ void store_out<bf16_t>(bf16_t* dst, const float* f, int n) {
  if (n == 8) {
    *reinterpret_cast<uint4*>(dst) = Vec16<bf16_t>::pack(f);
  } else if (n == 1) {
    dst->bits = f32_to_bf16_rne(f[0]);
  } else {
    for (int e = 0; e < n; e += 2)
      *reinterpret_cast<uint32_t*>(dst + e) = pack_bf16x2(f[e], f[e + 1]);
  }
}
template <>
__device__ __forceinline__ void store_out<__half>(__half* dst, const float* f, int n) {
  if (n == 8) {
    *reinterpret_cast<uint4*>(dst) = Vec16<__half>::pack(f);
  } else if (n == 1) {
    *dst = __float2half_rn(f[0]);
  } else {
    for (int e = 0; e < n; e += 2)
      *reinterpret_cast<uint32_t*>(dst + e) = pack_h16x2(f[e], f[e + 1]);
  }
}

// q.k over one 16-byte chunk: packed bf16/fp16 dot2 (v_dot2_f32_bf16 /
// v_dot2_f32_f16: exact products, fp32 accumulation) or fp32 FMAs.
template <typename T> struct QFrag;
template <> struct QFrag<float> {
  float f[4];
  __device__ __forceinline__ void load(const float* p) {
    Vec16<float>::unpack(*reinterpret_cast<const uint4*>(p), f);
  }
  __device__ __forceinline__ float dot(const uint4& w) const {
    float s = f[0] * __uint_as_float(w.x);
    s = fmaf(f[1], __uint_as_float(w.y), s);
    s = fmaf(f[2], __uint_as_float(w.z), s);
    return fmaf(f[3], __uint_as_float(w.w), s);
  }
};
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
template <> struct QFrag<bf16_t> {
  uint4 w;
  __device__ __forceinline__ void load(const bf16_t* p) { w = *reinterpret_cast<const uint4*>(p); }
  __device__ __forceinline__ float dot(const uint4& k) const {
    float s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.x), __builtin_bit_cast(bf16x2_t, k.x), 0.f, false);
    s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.y), __builtin_bit_cast(bf16x2_t, k.y), s, false);
    s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.z), __builtin_bit_cast(bf16x2_t, k.z), s, false);
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.w), __builtin_bit_cast(bf16x2_t, k.w), s, false);
  }
};
template <> struct QFrag<__half> {
  uint4 w;
  __device__ __forceinline__ void load(const __half* p) { w = *reinterpret_cast<const uint4*>(p); }
  __device__ __forceinline__ float dot(const uint4& k) const {
    float s = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, w.x), __builtin_bit_cast(f16x2_t, k.x), 0.f, false);
    s = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, w.y), __builtin_bit_cast(f16x2_t, k.y), s, false);
    s = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, w.z), __builtin_bit_cast(f16x2_t, k.z), s, false);
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, w.w), __builtin_bit_cast(f16x2_t, k.w), s, false);
  }
};

// streaming 16-byte load (K/V rows are read once per call)
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_stream(const void* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint2 load_stream8(const void* p) {
  const u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
  return make_uint2(v.x, v.y);
}

// A lane's 8 (16-bit) or 4 (fp32) elements of a K / V row: one 16-byte load,
// or with an fp8 cache (FP8) one 8-byte load, converted after the loads are
// issued (the raw words wait here).
template <typename T, bool FP8> struct KVRaw {
  uint4 w;
  __device__ __forceinline__ void load(const void* p) { w = load_stream(p); }
  __device__ __forceinline__ void zero() { w = make_uint4(0, 0, 0, 0); }
};
template <typename T> struct KVRaw<T, true> {
  uint2 w;
  __device__ __forceinline__ void load(const void* p) { w = load_stream8(p); }
  __device__ __forceinline__ void zero() { w = make_uint2(0, 0); }
};

// GQ query heads per workgroup (GQA: heads of one kv head that read one id
// row): each K / V row is loaded once and scored for all GQ heads.
template <typename T, typename TO, int D, int NI, bool PAGED, bool FP8 = false, int GQ = 1, int NW = kDecodeWaves>
__global__ __launch_bounds__(NW * kWave) void decode_kernel(DecodeK p) {
  using V = Vec16<T>;
  using KE = std::conditional_t<FP8, uint8_t, T>;   // cache element
  static_assert(!FP8 || (PAGED && sizeof(T) == 2), "fp8 caches: paged, 16-bit queries");
  constexpr int EPV = V::N;           // elements per 16-byte vector
  constexpr int LPR = D / EPV;        // lanes per key row
  constexpr int RPI = kWave / LPR;    // key rows per load instruction
  constexpr int UK = NI * RPI;        // keys per unit
  constexpr int DUP = LPR / NI;       // lanes sharing one finished score
  static_assert(LPR <= kWave && kWave % LPR == 0, "row must fit a wavefront");
  static_assert(NI <= LPR && LPR % NI == 0, "NI must divide LPR");

  __shared__ float s_p[NW][GQ][64];
  __shared__ float s_o[NW][GQ][D];
  __shared__ float s_m[NW][GQ], s_l[NW][GQ];

  const srswa_decode_args& a = p.a;
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int r = lane / LPR;
  const int c = lane % LPR;

  const int split = blockIdx.x % p.nsplit;
  const int64_t rg = blockIdx.x / p.nsplit;     // ((b * Lq) + lq) * (HQ / GQ) + head group
  const int hq0 = (int)(rg % (a.HQ / GQ)) * GQ; // the group's first query head
  const int64_t bl = rg / (a.HQ / GQ);
  const int64_t rh0 = bl * a.HQ + hq0;          // ((b * Lq) + lq) * HQ + hq0
  const int lq = (int)(bl % a.Lq);
  const int b = (int)(bl / a.Lq);
  const int kvh = hq0 / p.G;
  const int ih = hq0 / p.IG;

  const int kvl = a.kv_len ? min(a.kv_len[b], a.L) : a.L;
  const int qp = PAGED ? a.kv_len[b] - a.Lq + lq : a.q_pos[b * a.pos_sb + lq * a.pos_sq];
  const int last = min(qp, kvl - 1);                   // last key this row may read
  const int ws = max(qp - a.local_window + 1, 0);      // first window key
  const int remote_end = min(ws, last + 1);            // remote keys are < this

  // this lane's slice of each head's q
  QFrag<T> qf[GQ];
#pragma unroll
  for (int g = 0; g < GQ; ++g)
    qf[g].load(reinterpret_cast<const T*>(a.q) + (int64_t)b * a.q_sb + (int64_t)lq * a.q_sq +
               (int64_t)(hq0 + g) * a.q_sh + c * EPV);
  const int32_t* idx_row = a.idx + (int64_t)b * a.idx_sb + (int64_t)ih * a.idx_sh +
                           (int64_t)lq * a.idx_sq;
  const int64_t aux_off = (int64_t)b * a.idx_sb + (int64_t)ih * a.idx_sh +
                          (int64_t)lq * a.idx_sq;

  const KE* kbase = reinterpret_cast<const KE*>(a.k) + (PAGED ? 0 : (int64_t)b * a.k_sb) +
                    (int64_t)kvh * a.k_sh + c * EPV;
  const KE* vbase = reinterpret_cast<const KE*>(a.v) + (PAGED ? 0 : (int64_t)b * a.v_sb) +
                    (int64_t)kvh * a.v_sh + c * EPV;
  int max_blk = kvl > 0 ? (kvl - 1) / a.block_size : -1;
  if (PAGED) max_blk = min(max_blk, p.max_blocks - 1);
  const int32_t* bt_row = PAGED ? p.bt + (int64_t)b * p.bt_sb : nullptr;
  // paged window: units on the UK grid from ws_al (each inside one block);
  // lane i holds the page of the window's i-th block
  const int ws_al = PAGED ? (ws & ~(p.UK - 1)) : ws;
  const int wblk0 = ws_al >> (PAGED ? p.bs_shift : 0);
  int win_page = 0;
  if (PAGED && a.local_window > 0) {
    const int wb = wblk0 + lane;
    if (wb <= max_blk) win_page = bt_row[wb];
  }

  float m[GQ], l[GQ];
  float acc[GQ][EPV];
#pragma unroll
  for (int g = 0; g < GQ; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < EPV; ++e) acc[g][e] = 0.f;
  }

  // Slot metadata in one round trip: lane s holds slot s (S <= 64) -- its id,
  // whether it survives (valid, in range, first slot holding that id) and its
  // bias.  Wider rows (S > 64) re-read the slots per unit instead.
  const bool slots_in_regs = a.S <= kWave;
  int my_bid = -1, my_page = 0;
  bool my_ok = false;
  float my_bias = 0.f;
  if (slots_in_regs && lane < a.S) {
    my_bid = idx_row[(int64_t)lane * a.idx_ss];
    my_ok = my_bid >= 0 && my_bid <= max_blk &&
            (!a.valid || a.valid[aux_off + (int64_t)lane * a.idx_ss]);
    if (a.bias) my_bias = a.bias[aux_off + (int64_t)lane * a.idx_ss];
    if (PAGED && my_ok) my_page = bt_row[my_bid];
  }
  if (slots_in_regs) {
    bool dup = false;
    for (int j = 0; j < a.S - 1; ++j) {
      const int bj = __shfl(my_bid, j, kWave);
      const bool okj = __shfl(my_ok ? 1 : 0, j, kWave) != 0;
      dup |= (j < lane) && okj && (bj == my_bid);
    }
    my_ok = my_ok && !dup;
  }

  // the workgroup's units, dealt round-robin to its waves so that every wave
  // mixes remote (scattered) and window (contiguous) units
  const int u_base = split * NW * p.upw;
  for (int i = 0; i < p.upw; ++i) {
    const int u = u_base + wave + i * NW;
    if (u >= p.n_units) break;
    int k0, k1, klo;
    int page = 0, page2 = 0;
    int wrap = 0;            // keys k0 + kk, kk < wrap, are read LW keys further on
    float bias_l2 = 0.f;
    if (u < p.n_remote_units) {
      const int slot = u / p.upb, sub = u % p.upb;
      int bid;
      bool ok;
      float bias = 0.f;
      if (slots_in_regs) {
        bid = __shfl(my_bid, slot, kWave);
        ok = __shfl(my_ok ? 1 : 0, slot, kWave) != 0;
        bias = __shfl(my_bias, slot, kWave);
        if (PAGED) page = __shfl(my_page, slot, kWave);
      } else {
        bid = idx_row[(int64_t)slot * a.idx_ss];
        ok = bid >= 0 && bid <= max_blk && (!a.valid || a.valid[aux_off + (int64_t)slot * a.idx_ss]);
        // a repeat of an id held by an earlier valid slot is skipped
        for (int s0 = 0; ok && s0 < slot; s0 += kWave) {
          const int s = s0 + lane;
          bool d = false;
          if (s < slot) {
            const int o = idx_row[(int64_t)s * a.idx_ss];
            d = (o == bid) && (!a.valid || a.valid[aux_off + (int64_t)s * a.idx_ss]);
          }
          if (__any(d)) ok = false;
        }
        if (ok && a.bias) bias = a.bias[aux_off + (int64_t)slot * a.idx_ss];
        if (PAGED && ok) page = bt_row[bid];
      }
      k0 = ok ? bid * a.block_size + sub * UK : 0;
      k1 = ok ? min(min(k0 + UK, bid * a.block_size + a.block_size), remote_end) : 0;
      klo = k0;
      bias_l2 = bias * kLog2e;
    } else {
      const int j = u - p.n_remote_units;
      k0 = ws_al + j * UK;
      k1 = min(k0 + UK, last + 1);
      klo = PAGED ? max(k0, ws) : k0;
      if (PAGED) {
        page = __shfl(win_page, (k0 >> p.bs_shift) - wblk0, kWave);
        // The paged window [ws, ws + LW) on the UK grid: units j = 1.. are
        // whole; unit 0 holds its first UK - (ws - ws_al) keys and, in the
        // slots before them, the window's last ws - ws_al keys (LW further
        // on, another page), so LW / UK units cover any window
        wrap = j == 0 ? ws - ws_al : 0;
        if (wrap > 0) {
          page2 = __shfl(win_page, ((k0 + a.local_window) >> p.bs_shift) - wblk0, kWave);
          klo = ws;
          k1 = last + 1;
        }
      }
    }
    if (k1 <= klo) continue;   // uniform across the wave

    // unit base: the sequence's K / V rows (contiguous) or the unit's page
    const KE* kb = kbase;
    const KE* vb = vbase;
    int kr0 = k0;              // row of key k0 in kb / vb
    if (PAGED) {
      kb += (int64_t)page * p.k_pst;
      vb += (int64_t)page * p.v_pst;
      kr0 = k0 & (a.block_size - 1);
    }
    KVRaw<T, FP8> kw[NI], vw[NI];
    // key of unit slot kk (wrapped slots: LW further on, in page2)
    auto key_of = [&](int kk) { return k0 + kk + (PAGED && kk < wrap ? a.local_window : 0); };
    if (PAGED && wrap > 0) {
      const int64_t dk = (int64_t)(page2 - page) * p.k_pst, dv = (int64_t)(page2 - page) * p.v_pst;
      const int w0 = (k0 + a.local_window) & (a.block_size - 1);   // row of the first wrapped key
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int kk = i * RPI + r;
        const int key = key_of(kk);
        const int64_t ro = kk < wrap ? dk + (int64_t)(w0 + kk) * a.k_st : (int64_t)(kr0 + kk) * a.k_st;
        if (key >= klo && key < k1) kw[i].load(kb + ro);
        else kw[i].zero();
      }
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int kk = i * RPI + r;
        const int key = key_of(kk);
        const int64_t ro = kk < wrap ? dv + (int64_t)(w0 + kk) * a.v_st : (int64_t)(kr0 + kk) * a.v_st;
        if (key >= klo && key < k1) vw[i].load(vb + ro);
        else vw[i].zero();
      }
    } else {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int key = k0 + i * RPI + r;
        if ((!PAGED || key >= klo) && key < k1) kw[i].load(kb + (int64_t)(kr0 + i * RPI + r) * a.k_st);
        else kw[i].zero();
      }
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int key = k0 + i * RPI + r;
        if ((!PAGED || key >= klo) && key < k1) vw[i].load(vb + (int64_t)(kr0 + i * RPI + r) * a.v_st);
        else vw[i].zero();
      }
    }

    float part[GQ][NI];
    if constexpr (FP8) {
      fp8_dispatch(p.kv8, [&](auto F) {
        constexpr int FF = decltype(F)::value;
        uint32_t sp = 0u;
#pragma unroll
        for (int i = 0; i < NI; ++i) sp |= fp8_special_bits<FF>(kw[i].w);
        if (__builtin_expect(!fp8_any_special(sp), 1)) {
#pragma unroll
          for (int i = 0; i < NI; ++i) {
            const uint4 kc = fp8x8_to_fast<FF, T>(kw[i].w);
#pragma unroll
            for (int g = 0; g < GQ; ++g) part[g][i] = qf[g].dot(kc);
          }
        } else {
#pragma unroll
          for (int i = 0; i < NI; ++i) {
            const uint4 kc = fp8x8_to_exact<FF, T>(kw[i].w);
#pragma unroll
            for (int g = 0; g < GQ; ++g) part[g][i] = qf[g].dot(kc);
          }
        }
      });
    } else {
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int g = 0; g < GQ; ++g) part[g][i] = qf[g].dot(kw[i].w);
    }
    const int i_own = c / DUP;                    // which instruction's key this lane holds
    const int key = key_of(i_own * RPI + r);
    const bool owner = (c % DUP) == 0;
    const bool kept = (!PAGED || key >= klo) && key < k1;
#pragma unroll
    for (int g = 0; g < GQ; ++g) {
      // reduce-scatter across the LPR lanes of a row: NI partials -> 1 score
      reduce_scatter<NI, LPR / 2>(part[g], c);
#pragma unroll
      for (int o = DUP / 2; o >= 1; o >>= 1) part[g][0] += __shfl_xor(part[g][0], o, kWave);
      const float t = kept ? part[g][0] * p.scale_l2 + bias_l2 : -INFINITY;
      const float mnew = fmaxf(m[g], wave_max(t));     // finite: key klo is always kept
      const float alpha = exp2f(m[g] - mnew);
      const float pj = exp2f(t - mnew);
      l[g] = l[g] * alpha + (owner ? pj : 0.f);   // per-lane; summed over the wave once at the end
      m[g] = mnew;
#pragma unroll
      for (int e = 0; e < EPV; ++e) acc[g][e] *= alpha;
      if (owner) s_p[wave][g][r * NI + i_own] = pj;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float pv[GQ][NI];
#pragma unroll
    for (int g = 0; g < GQ; ++g)
#pragma unroll
      for (int i = 0; i < NI; ++i) pv[g][i] = s_p[wave][g][r * NI + i];
    if constexpr (FP8) {
      fp8_dispatch(p.kv8, [&](auto F) {
        constexpr int FF = decltype(F)::value;
        uint32_t sp = 0u;
#pragma unroll
        for (int i = 0; i < NI; ++i) sp |= fp8_special_bits<FF>(vw[i].w);
        if (__builtin_expect(!fp8_any_special(sp), 1)) {
#pragma unroll
          for (int i = 0; i < NI; ++i) {
            float f[8];
            fp8x8_to_f32_fast<FF>(vw[i].w, f);
#pragma unroll
            for (int g = 0; g < GQ; ++g)
#pragma unroll
              for (int e = 0; e < EPV; ++e) acc[g][e] = fmaf(pv[g][i], f[e], acc[g][e]);
          }
        } else {
#pragma unroll
          for (int i = 0; i < NI; ++i) {
            float f[8];
            fp8x8_to_f32_exact<FF>(vw[i].w, f);
#pragma unroll
            for (int g = 0; g < GQ; ++g)
#pragma unroll
              for (int e = 0; e < EPV; ++e) acc[g][e] = fmaf(pv[g][i], f[e], acc[g][e]);
          }
        }
      });
    } else {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        float f[EPV];
        V::unpack(vw[i].w, f);
#pragma unroll
        for (int g = 0; g < GQ; ++g)
#pragma unroll
          for (int e = 0; e < EPV; ++e) acc[g][e] = fmaf(pv[g][i], f[e], acc[g][e]);
      }
    }
    __builtin_amdgcn_wave_barrier();
  }

  // sum the RPI row groups of the wave
#pragma unroll
  for (int g = 0; g < GQ; ++g)
#pragma unroll
    for (int o = LPR; o < kWave; o <<= 1)
#pragma unroll
      for (int e = 0; e < EPV; ++e) acc[g][e] += __shfl_xor(acc[g][e], o, kWave);

  if (r == 0) {
#pragma unroll
    for (int g = 0; g < GQ; ++g)
#pragma unroll
      for (int e = 0; e < EPV; ++e) s_o[wave][g][c * EPV + e] = acc[g][e];
  }
#pragma unroll
  for (int g = 0; g < GQ; ++g) l[g] = wave_sum(l[g]);
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < GQ; ++g) { s_m[wave][g] = m[g]; s_l[wave][g] = l[g]; }
  }
  __syncthreads();
  if (wave != 0) return;

  // merge the workgroup's waves (wave 0), head by head
#pragma unroll
  for (int g = 0; g < GQ; ++g) {
    const int64_t rh = rh0 + g;
    const int hq = hq0 + g;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, s_m[w][g]);
    float L = 0.f, O[EPV];
#pragma unroll
    for (int e = 0; e < EPV; ++e) O[e] = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float wt = s_m[w][g] == -INFINITY ? 0.f : exp2f(s_m[w][g] - M);
      L += s_l[w][g] * wt;
      if (r == 0) {
#pragma unroll
        for (int e = 0; e < EPV; ++e) O[e] = fmaf(s_o[w][g][c * EPV + e], wt, O[e]);
      }
    }

    if (p.nsplit > 1) {
      // record: O[0..D) then M, L; records are 128-byte aligned
      float* rec = p.part + (rh * p.nsplit + split) * p.pstride;
      if (r == 0) store_out<float>(rec + c * EPV, O, EPV);
      if (lane == 0) { rec[D] = M; rec[D + 1] = L; }
      continue;   // decode_merge_kernel combines the records
    }

    const float inv = L > 0.f ? 1.f / L : 0.f;
    if (r == 0) {
#pragma unroll
      for (int e = 0; e < EPV; ++e) O[e] *= inv;
      TO* orow = reinterpret_cast<TO*>(a.out) + (int64_t)b * a.o_sb + (int64_t)lq * a.o_sq +
                 (int64_t)hq * a.o_sh + c * EPV;
      store_out<TO>(orow, O, EPV);
    }
    if (a.lse && lane == 0) {
      a.lse[(int64_t)b * a.lse_sb + (int64_t)lq * a.lse_sq + (int64_t)hq * a.lse_sh] =
          L > 0.f ? fmaf(M, kLn2, logf(L)) : -INFINITY;   // one rounding wherever it is inlined
    }
  }
}

// Combines the per-workgroup (O, M, L) records of every (row, head): one
// wavefront per (row, head), D/64 dims per lane.
template <typename TO, int D>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeK p) {
  constexpr int DPL = D / kWave;   // dims per lane
  const srswa_decode_args& a = p.a;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int64_t rh = (int64_t)blockIdx.x * 4 + wave;
  if (rh >= p.rowheads) return;
  const float* recs = p.part + rh * p.nsplit * p.pstride;
  float M = -INFINITY, L = 0.f, O[DPL];
#pragma unroll
  for (int e = 0; e < DPL; ++e) O[e] = 0.f;
  for (int s0 = 0; s0 < p.nsplit; s0 += 8) {
    // all loads of up to 8 records issued before any is used: unconditional,
    // from clamped record indices (a load behind a branch per record would be
    // waited for on its own); the records past nsplit are masked afterwards
    float ms[8], ls[8], os[8][DPL];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float* rec = recs + (int64_t)min(s0 + j, p.nsplit - 1) * p.pstride;
      ms[j] = rec[D];
      ls[j] = rec[D + 1];
#pragma unroll
      for (int e = 0; e < DPL; ++e) os[j][e] = rec[lane * DPL + e];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (s0 + j >= p.nsplit) ms[j] = -INFINITY;    // wave-uniform
    float Mn = M;
#pragma unroll
    for (int j = 0; j < 8; ++j) Mn = fmaxf(Mn, ms[j]);
    const float r0 = M == -INFINITY ? 0.f : exp2f(M - Mn);
    L *= r0;
#pragma unroll
    for (int e = 0; e < DPL; ++e) O[e] *= r0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (ms[j] == -INFINITY) continue;            // an empty or masked record adds nothing
      const float wt = exp2f(ms[j] - Mn);
      L = fmaf(ls[j], wt, L);
#pragma unroll
      for (int e = 0; e < DPL; ++e) O[e] = fmaf(os[j][e], wt, O[e]);
    }
    M = Mn;
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
#pragma unroll
  for (int e = 0; e < DPL; ++e) O[e] *= inv;
  const int hq = (int)(rh % a.HQ);
  const int64_t bl = rh / a.HQ;
  const int lq = (int)(bl % a.Lq);
  const int b = (int)(bl / a.Lq);
  TO* orow = reinterpret_cast<TO*>(a.out) + (int64_t)b * a.o_sb + (int64_t)lq * a.o_sq +
             (int64_t)hq * a.o_sh + lane * DPL;
  store_out<TO>(orow, O, DPL);
  if (a.lse && lane == 0)
    a.lse[(int64_t)b * a.lse_sb + (int64_t)lq * a.lse_sq + (int64_t)hq * a.lse_sh] =
        L > 0.f ? fmaf(M, kLn2, logf(L)) : -INFINITY;   // one rounding wherever it is inlined
}

int elem_bytes(int dt) { return dt == SRSWA_F32 ? 4 : 2; }

// Tuning knobs (environment, read once): SRSWA_DECODE_NI = 8 (default) | 16
// load instructions per unit (bf16 D=128: 32 | 64 keys); SRSWA_DECODE_UPW =
// units per wave (default 2, 4 with fp8 caches).
int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return (v && *v) ? atoi(v) : dflt;
}

// row instructions per unit for (dtype, D)
int decode_ni(int dt, int D) {
  static const int want = env_int("SRSWA_DECODE_NI", 8);
  const int lpr = D * elem_bytes(dt) / 16;
  const int ni = lpr < 16 ? lpr : 16;
  return (want == 8 && ni == 16) ? 8 : ni;
}

// Query heads served per workgroup: under GQA the heads of one kv head that
// also share one id row (G and IG multiples of the group) are scored together,
// so each K / V row is read once per group instead of once per head.  Groups
// take 16-bit queries with outputs of the same dtype and units of at most 8
// loads; SRSWA_DECODE_GQA=0 turns them off.
int gqa_heads(const srswa_decode_args* a, int ni) {
  static const int on = env_int("SRSWA_DECODE_GQA", 1);
  if (!on || a->in_dtype == SRSWA_F32 || a->out_dtype != a->in_dtype || ni > 8) return 1;
  const int G = a->HQ / a->HKV, IG = a->HQ / a->HI;
  for (int gq : {4, 2})
    if (G % gq == 0 && IG % gq == 0) return gq;
  return 1;
}

DecodePlan make_plan(const srswa_decode_args* a, bool paged = false, bool fp8 = false) {
  DecodePlan pl{};
  const int lpr = a->D * elem_bytes(a->in_dtype) / 16;
  int ni = decode_ni(a->in_dtype, a->D);
  // a paged unit must stay inside one block (one page): UK <= block size
  while (paged && ni > 1 && ni * (kWave / lpr) > a->block_size) ni >>= 1;
  pl.UK = ni * (kWave / lpr);
  pl.upb = ceil_div(a->block_size, pl.UK);
  pl.n_remote_units = a->S * pl.upb;
  // paged windows run on the UK grid, LW / UK units with the first one
  // wrapped (UK divides the page size, which divides LW)
  pl.n_units = pl.n_remote_units + ceil_div(a->local_window, pl.UK);
  // an fp8 unit holds half the bytes: a workgroup takes four times the
  // units, as eight waves of four (at config 3 one workgroup per row, so no
  // split-K merge; eight waves of four beat four of eight by about 1%, and
  // sixteen of two lose a quarter)
  pl.nw = fp8 && paged ? 8 : kDecodeWaves;
  static const int upw = env_int("SRSWA_DECODE_UPW", 0);
  pl.upw = upw > 0 ? upw : (fp8 ? 4 : 2);
  pl.nsplit = ceil_div(pl.n_units, pl.nw * pl.upw);
  pl.pstride = ceil_div(a->D + 2, 32) * 32;
  pl.rowheads = (int64_t)a->B * a->Lq * a->HQ;
  pl.gq = gqa_heads(a, ni);
  return pl;
}

size_t scratch_bytes(const DecodePlan& pl) {
  return pl.nsplit <= 1 ? 0 : (size_t)pl.rowheads * pl.nsplit * pl.pstride * 4;
}

template <typename T, typename TO, int D, int NI, int GQ>
void launch_decode_gq(const DecodeK& k, int64_t grid, hipStream_t st) {
  if constexpr (sizeof(T) == 2 && std::is_same_v<T, TO>) {
    if (k.kv8 && k.bt) {
      if (k.nw == 8)
        hipLaunchKernelGGL((decode_kernel<T, TO, D, NI, true, true, GQ, 8>), dim3((unsigned)grid),
                           dim3(8 * kWave), 0, st, k);
      else
        hipLaunchKernelGGL((decode_kernel<T, TO, D, NI, true, true, GQ>), dim3((unsigned)grid),
                           dim3(kDecodeWaves * kWave), 0, st, k);
    }
  }
  if (k.kv8) {
    // fp8 caches take the 16-bit paged kernels only (checked by the caller)
  } else if (k.bt)
    hipLaunchKernelGGL((decode_kernel<T, TO, D, NI, true, false, GQ>), dim3((unsigned)grid),
                       dim3(kDecodeWaves * kWave), 0, st, k);
  else
    hipLaunchKernelGGL((decode_kernel<T, TO, D, NI, false, false, GQ>), dim3((unsigned)grid),
                       dim3(kDecodeWaves * kWave), 0, st, k);
}

template <typename T, typename TO, int D, int NI>
int launch_decode_ni(const DecodeK& k, int64_t grid, hipStream_t st) {
  // head groups: 16-bit queries with 16-bit outputs of their dtype, units of
  // at most 8 load instructions (gqa_heads never picks a group otherwise)
  constexpr bool kGroups = sizeof(T) == 2 && std::is_same_v<T, TO> && NI <= 8;
  if (kGroups && k.gq == 4) launch_decode_gq<T, TO, D, NI, kGroups ? 4 : 1>(k, grid / 4, st);
  else if (kGroups && k.gq == 2) launch_decode_gq<T, TO, D, NI, kGroups ? 2 : 1>(k, grid / 2, st);
  else launch_decode_gq<T, TO, D, NI, 1>(k, grid, st);
  if (k.nsplit > 1)
    hipLaunchKernelGGL((decode_merge_kernel<TO, D>), dim3((unsigned)((k.rowheads + 3) / 4)),
                       dim3(256), 0, st, k);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("decode launch failed: %s", hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}

template <typename T, typename TO, int D>
int launch_decode(const DecodeK& k, int64_t grid, hipStream_t st) {
  constexpr int LPR = D / Vec16<T>::N;
  constexpr int NI_MAX = LPR < 16 ? LPR : 16;
  const int ni = k.UK / (kWave / LPR);
  if (NI_MAX >= 16 && ni == 16) return launch_decode_ni<T, TO, D, 16 <= NI_MAX ? 16 : NI_MAX>(k, grid, st);
  if (ni == 8) return launch_decode_ni<T, TO, D, 8 <= NI_MAX ? 8 : NI_MAX>(k, grid, st);
  if (ni == 4) return launch_decode_ni<T, TO, D, 4>(k, grid, st);
  if (ni == 2) return launch_decode_ni<T, TO, D, 2>(k, grid, st);
  return launch_decode_ni<T, TO, D, 1>(k, grid, st);
}

template <typename T>
int dispatch_out(const DecodeK& k, int64_t grid, hipStream_t st) {
  const int D = k.a.D;
  const int od = k.a.out_dtype;
  if (od == SRSWA_F32) {
    if (D == 64) return launch_decode<T, float, 64>(k, grid, st);
    if (D == 128) return launch_decode<T, float, 128>(k, grid, st);
  } else if (od == SRSWA_BF16) {
    if (D == 64) return launch_decode<T, bf16_t, 64>(k, grid, st);
    if (D == 128) return launch_decode<T, bf16_t, 128>(k, grid, st);
  } else if (od == SRSWA_F16) {
    if (D == 64) return launch_decode<T, __half, 64>(k, grid, st);
    if (D == 128) return launch_decode<T, __half, 128>(k, grid, st);
  }
  set_error("decode: unsupported out dtype %d / D %d", od, D);
  return SRSWA_UNSUPPORTED;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace
}  // namespace srswa

using namespace srswa;

extern "C" int srswa_version(void) { return 100; }
extern "C" const char* srswa_last_error(void) { return srswa::last_error(); }

extern "C" size_t srswa_gather_decode_workspace(const srswa_decode_args* a) {
  if (a && a->B > 0 && a->Lq > 0 && a->HQ > 0 && a->D > 0 && a->block_size > 0 && a->S >= 0 &&
      a->local_window > 0)
    return scratch_bytes(make_plan(a));
  return 0;
}

extern "C" int srswa_gather_decode(const srswa_decode_args* a, void* ws, size_t ws_bytes,
                                   void* stream) {
  if (!a || !a->q || !a->k || !a->v || !a->out || !a->q_pos || (!a->idx && a->S > 0)) {
    set_error("decode: null argument");
    return SRSWA_INVALID;
  }
  if (a->B < 0 || a->Lq < 0 || a->HQ <= 0 || a->HKV <= 0 || a->HI <= 0 || a->S < 0 ||
      a->L <= 0 || a->block_size <= 0 || a->local_window <= 0) {
    set_error("decode: bad sizes");
    return SRSWA_INVALID;
  }
  if (a->B == 0 || a->Lq == 0) return SRSWA_OK;
  if (a->HQ % a->HKV != 0 || a->HQ % a->HI != 0) {
    set_error("decode: HQ=%d must be a multiple of HKV=%d and HI=%d", a->HQ, a->HKV, a->HI);
    return SRSWA_UNSUPPORTED;
  }
  const int ib = elem_bytes(a->in_dtype);
  if (!(a->D == 64 || a->D == 128) || a->in_dtype < 0 || a->in_dtype > 2 ||
      a->out_dtype < 0 || a->out_dtype > 2) {
    set_error("decode: unsupported D=%d / dtype", a->D);
    return SRSWA_UNSUPPORTED;
  }
  // every row must start on a 16-byte boundary
  const int64_t strides[] = {a->q_sb, a->q_sq, a->q_sh, a->k_sb, a->k_st, a->k_sh,
                             a->v_sb, a->v_st, a->v_sh};
  for (int64_t s : strides)
    if ((s * ib) % 16 != 0) {
      set_error("decode: strides must keep rows 16-byte aligned");
      return SRSWA_UNSUPPORTED;
    }
  const int ob = elem_bytes(a->out_dtype);
  if (((a->o_sb * ob) % 16) || ((a->o_sq * ob) % 16) || ((a->o_sh * ob) % 16) ||
      !aligned16(a->q) || !aligned16(a->k) || !aligned16(a->v) || !aligned16(a->out)) {
    set_error("decode: pointers must be 16-byte aligned");
    return SRSWA_UNSUPPORTED;
  }
  if (a->S > 1024) {
    set_error("decode: at most 1024 slots per row (got %d)", a->S);
    return SRSWA_UNSUPPORTED;
  }
  const DecodePlan pl = make_plan(a);
  const size_t need = scratch_bytes(pl);
  if (need > 0 && (!ws || ws_bytes < need)) {
    set_error("decode: scratch of %zu bytes required (got %zu)", need, ws_bytes);
    return SRSWA_WORKSPACE;
  }
  DecodeK k{};
  k.a = *a;
  k.G = a->HQ / a->HKV;
  k.IG = a->HQ / a->HI;
  k.UK = pl.UK;
  k.upb = pl.upb;
  k.n_remote_units = pl.n_remote_units;
  k.n_units = pl.n_units;
  k.upw = pl.upw;
  k.nw = pl.nw;
  k.nsplit = pl.nsplit;
  k.pstride = pl.pstride;
  k.scale_l2 = a->scale * kLog2e;
  k.rowheads = pl.rowheads;
  k.gq = pl.gq;
  if (need > 0) k.part = reinterpret_cast<float*>(ws);
  const int64_t grid = pl.rowheads * pl.nsplit;
  if (grid > 0x7fffffff) {
    set_error("decode: grid too large");
    return SRSWA_UNSUPPORTED;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (a->in_dtype) {
    case SRSWA_F32: return dispatch_out<float>(k, grid, st);
    case SRSWA_BF16: return dispatch_out<bf16_t>(k, grid, st);
    case SRSWA_F16: return dispatch_out<__half>(k, grid, st);
  }
  return SRSWA_UNSUPPORTED;
}

namespace {

// The paged arguments as a decode over R sequences of dql query rows, the
// caches addressed per page (k_sb / v_sb unused) and positions from seq_lens.
srswa_decode_args paged_as_decode(const srswa_paged_decode_args* a) {
  srswa_decode_args d{};
  d.q = a->q;  d.q_sb = (int64_t)a->dql * a->q_sn;  d.q_sq = a->q_sn;  d.q_sh = a->q_sh;
  d.k = a->k_cache;  d.k_sb = 0;  d.k_st = a->k_st;  d.k_sh = a->k_sh;
  d.v = a->v_cache;  d.v_sb = 0;  d.v_st = a->v_st;  d.v_sh = a->v_sh;
  d.idx = a->topk;  d.idx_sb = (int64_t)a->dql * a->t_sn;  d.idx_sh = a->t_sh;  d.idx_sq = a->t_sn;
  d.idx_ss = a->t_sk;
  d.bias = a->bias;  d.valid = nullptr;
  d.q_pos = nullptr;  d.kv_len = a->seq_lens;
  d.out = a->out;  d.o_sb = (int64_t)a->dql * a->o_sn;  d.o_sq = a->o_sn;  d.o_sh = a->o_sh;
  d.lse = nullptr;
  d.B = a->R;  d.Lq = a->dql;  d.HQ = a->HQ;  d.HKV = a->HKV;  d.HI = a->HKV;  d.D = a->D;
  d.S = a->topk_n;  d.L = a->max_blocks * a->page_size;
  d.block_size = a->page_size;  d.local_window = a->local_blocks * a->page_size;
  d.scale = a->scale;  d.in_dtype = a->in_dtype;  d.out_dtype = a->out_dtype;
  return d;
}

}  // namespace

extern "C" size_t srswa_gather_decode_paged_workspace(const srswa_paged_decode_args* a) {
  if (a && a->R > 0 && a->dql > 0 && a->HQ > 0 && a->D > 0 && a->page_size > 0 && a->topk_n >= 0 &&
      a->local_blocks >= 0) {
    const srswa_decode_args d = paged_as_decode(a);
    return scratch_bytes(make_plan(&d, true, a->kv_fp8 != 0));
  }
  return 0;
}

extern "C" int srswa_gather_decode_paged(const srswa_paged_decode_args* a, void* ws, size_t ws_bytes,
                                         void* stream) {
  if (!a || !a->q || !a->k_cache || !a->v_cache || !a->out || !a->block_table || !a->seq_lens ||
      (!a->topk && a->topk_n > 0)) {
    set_error("paged decode: null argument");
    return SRSWA_INVALID;
  }
  if (a->R < 0 || a->dql <= 0 || a->HQ <= 0 || a->HKV <= 0 || a->topk_n < 0 || a->max_blocks <= 0 ||
      a->page_size <= 0 || a->local_blocks < 0) {
    set_error("paged decode: bad sizes");
    return SRSWA_INVALID;
  }
  if (a->R == 0) return SRSWA_OK;
  if (a->HQ % a->HKV != 0) {
    set_error("paged decode: HQ=%d must be a multiple of HKV=%d", a->HQ, a->HKV);
    return SRSWA_UNSUPPORTED;
  }
  if (!(a->D == 64 || a->D == 128) || a->in_dtype < 0 || a->in_dtype > 2 || a->out_dtype < 0 ||
      a->out_dtype > 2) {
    set_error("paged decode: unsupported D=%d / dtype", a->D);
    return SRSWA_UNSUPPORTED;
  }
  const int ib = elem_bytes(a->in_dtype), ob = elem_bytes(a->out_dtype);
  const bool fp8 = a->kv_fp8 != 0;
  if (fp8 && (a->kv_fp8 < SRSWA_FP8_E4M3FN || a->kv_fp8 > SRSWA_FP8_E5M2FNUZ || a->in_dtype == SRSWA_F32 ||
              a->out_dtype != a->in_dtype)) {
    set_error("paged decode: fp8 caches (kv_fp8 %d) take bf16 / fp16 queries and outputs of the same dtype",
              a->kv_fp8);
    return SRSWA_UNSUPPORTED;
  }
  const int kvb = fp8 ? 1 : ib;            // cache element bytes
  const int rpi = kWave / (a->D * ib / 16);
  if ((a->page_size & (a->page_size - 1)) || a->page_size < rpi) {
    set_error("paged decode: page size %d must be a power of two >= %d", a->page_size, rpi);
    return SRSWA_UNSUPPORTED;
  }
  if (a->local_blocks > kWave - 1 || a->topk_n > 1024) {
    set_error("paged decode: at most 63 local blocks and 1024 slots");
    return SRSWA_UNSUPPORTED;
  }
  const int64_t qstrides[] = {a->q_sn, a->q_sh};
  for (int64_t st : qstrides)
    if ((st * ib) % 16 != 0) {
      set_error("paged decode: strides must keep rows 16-byte aligned");
      return SRSWA_UNSUPPORTED;
    }
  // a lane reads 8 (16-bit) elements of a cache row: 16 bytes, 8 with fp8
  const int64_t kvstrides[] = {a->k_sp, a->k_st, a->k_sh, a->v_sp, a->v_st, a->v_sh};
  for (int64_t st : kvstrides)
    if ((st * kvb) % (fp8 ? 8 : 16) != 0) {
      set_error("paged decode: cache strides must keep rows %d-byte aligned", fp8 ? 8 : 16);
      return SRSWA_UNSUPPORTED;
    }
  if (((a->o_sn * ob) % 16) || ((a->o_sh * ob) % 16) || !aligned16(a->q) || !aligned16(a->k_cache) ||
      !aligned16(a->v_cache) || !aligned16(a->out)) {
    set_error("paged decode: pointers must be 16-byte aligned");
    return SRSWA_UNSUPPORTED;
  }
  const srswa_decode_args d = paged_as_decode(a);
  const DecodePlan pl = make_plan(&d, true, a->kv_fp8 != 0);
  const size_t need = scratch_bytes(pl);
  if (need > 0 && (!ws || ws_bytes < need)) {
    set_error("paged decode: scratch of %zu bytes required (got %zu)", need, ws_bytes);
    return SRSWA_WORKSPACE;
  }
  DecodeK k{};
  k.a = d;
  k.G = d.HQ / d.HKV;
  k.IG = d.HQ / d.HI;
  k.UK = pl.UK;
  k.upb = pl.upb;
  k.n_remote_units = pl.n_remote_units;
  k.n_units = pl.n_units;
  k.upw = pl.upw;
  k.nw = pl.nw;
  k.nsplit = pl.nsplit;
  k.pstride = pl.pstride;
  k.scale_l2 = d.scale * kLog2e;
  k.rowheads = pl.rowheads;
  k.gq = pl.gq;
  if (need > 0) k.part = reinterpret_cast<float*>(ws);
  k.bt = a->block_table;
  k.bt_sb = a->bt_sr;
  k.k_pst = a->k_sp;
  k.v_pst = a->v_sp;
  k.bs_shift = __builtin_ctz((unsigned)a->page_size);
  k.max_blocks = a->max_blocks;
  k.kv8 = a->kv_fp8;
  const int64_t grid = pl.rowheads * pl.nsplit;
  if (grid > 0x7fffffff) {
    set_error("paged decode: grid too large");
    return SRSWA_UNSUPPORTED;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (a->in_dtype) {
    case SRSWA_F32: return dispatch_out<float>(k, grid, st);
    case SRSWA_BF16: return dispatch_out<bf16_t>(k, grid, st);
    case SRSWA_F16: return dispatch_out<__half>(k, grid, st);
  }
  return SRSWA_UNSUPPORTED;
}

// ---------------------------------------------------------------------------
// Allocation-free decode.  The split-K records live in `scratch`, a file-scope
// device array of kStaticScratchBytes that each GPU the library runs on holds
// until the process ends.  Host code never passes the array's name to a
// kernel (on the host it is only a stand-in for the symbol): its device
// address is looked up once per device with hipGetSymbolAddress, with that
// device current, and cached.  Every call on one GPU shares that GPU's array,
// so calls that overlap on one GPU (several streams, several host threads)
// race; calls on one stream are ordered and safe.  Nothing needs clearing:
// every call writes each record it reads.
// ---------------------------------------------------------------------------
namespace {
constexpr size_t kStaticScratchBytes = size_t(8) << 20;   // 8 MiB per device
constexpr int kMaxDevices = 64;
}  // namespace

static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace {
std::atomic<void*> g_static_scratch[kMaxDevices];
std::mutex g_static_scratch_mu;

// The device address of `scratch` on the device `stream` runs on, which must
// be the current device.
int static_scratch(void* stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("decode (no alloc): no usable current device (%s)", hipGetErrorString(e));
    return SRSWA_INVALID;
  }
  if (stream) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(reinterpret_cast<hipStream_t>(stream), &sdev);
    if (e != hipSuccess || sdev != dev) {
      set_error("decode (no alloc): the stream belongs to device %d, the current device is %d", (int)sdev, dev);
      return SRSWA_INVALID;
    }
  }
  void* p = g_static_scratch[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_static_scratch_mu);
    p = g_static_scratch[dev].load(std::memory_order_relaxed);
    if (!p) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p) {
        set_error("decode (no alloc): hipGetSymbolAddress of the static scratch failed on device %d: %s", dev,
                  hipGetErrorString(e));
        return SRSWA_LAUNCH;
      }
      g_static_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return SRSWA_OK;
}
}  // namespace

extern "C" int srswa_gather_decode_noalloc(const srswa_decode_args* a, void* stream) {
  const size_t need = srswa_gather_decode_workspace(a);
  if (need > kStaticScratchBytes) {
    set_error("decode (no alloc): this call needs %zu bytes of split-K scratch, above the static %zu bytes; "
              "use srswa_gather_decode with a caller-owned workspace", need, kStaticScratchBytes);
    return SRSWA_WORKSPACE;
  }
  void* ws = nullptr;
  if (need > 0) {
    const int st = static_scratch(stream, &ws);
    if (st != SRSWA_OK) return st;
  }
  return srswa_gather_decode(a, ws, need > 0 ? kStaticScratchBytes : 0, stream);
}
