// Page2D rotary embedding on the device: the per-token cos/sin table of the
// two-axis (token-in-page, page) coordinates and its application to one or
// two tensors (q / k of the main branch, idx_q / idx_k of the indexer).
//
// Replaces
//   _cos_sin_2d_kernel / cos_sin_2d_fused  WHL!layers/attention/unlimited_dash_ops/decode_meta_triton.py:166-209,354-389
//   PageRope2D.cos_sin                     WHL!…/page2d_rope.py:108-127
//   DeepseekV2IndexerRotary2D.forward      HF/_sparse_base_impl.py:2046-2061
//   apply_page2d_rope(_pair) and kernels   WHL!…/page2d_rope.py:130-324
//   transformers' llama apply_rotary_pos_emb as the HF indexer applies it
//                                          HF/_sparse_base_impl.py:39-41,3049
//
// The rotary application is a streaming elementwise pass (HBM-bound: read x
// and write o once; the cos/sin rows are shared by every head of a token and
// come from L2).  Each lane owns VE consecutive elements of the first half of
// a head and the matching VE of the second half, so both rotate_half partners
// arrive in one pair of 16-byte loads and nothing is exchanged between lanes.
// Rounding follows the eager torch order the reference kernels reproduce:
// x*cos and rotate_half(x)*sin are each rounded to the tensor dtype, their sum
// is formed in fp32 and rounded again.
#include "common.h"

#pragma clang fp contract(off)

namespace srswa {
namespace {

__device__ __forceinline__ int64_t ld_ix(const void* p, int64_t i, int is64) {
  return is64 ? reinterpret_cast<const int64_t*>(p)[i] : (int64_t)reinterpret_cast<const int32_t*>(p)[i];
}

// dtype traits: round an fp32 value to the storage type and back
template <typename T> struct Rt;
template <> struct Rt<float> {
  __device__ __forceinline__ static float r(float v) { return v; }
  __device__ __forceinline__ static void store(float* p, float v) { *p = v; }
};
template <> struct Rt<bf16_t> {
  __device__ __forceinline__ static float r(float v) { return bf16_lo(pack_bf16x2(v, 0.f)); }
  __device__ __forceinline__ static void store(bf16_t* p, float v) { p->bits = f32_to_bf16_rne(v); }
};
template <> struct Rt<__half> {
  __device__ __forceinline__ static float r(float v) { return __half2float(__float2half_rn(v)); }
  __device__ __forceinline__ static void store(__half* p, float v) { *p = __float2half_rn(v); }
};

// ------------------------------------------------------------ cos / sin
// One thread per (token, frequency pair i < dim/2): the angle is formed once
// and written to columns i and i + dim/2 of both tables (the reference's
// cat(ang, ang)).
template <typename T>
__global__ __launch_bounds__(256) void cos_sin_kernel(srswa_cos_sin_args a) {
  const int half = a.dim / 2;
  const int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= (int64_t)a.T * half) return;
  const int64_t t = item / half;
  const int i = (int)(item % half);
  float ang;
  if (i < a.n_tok) {
    const float tf = (float)ld_ix(a.tok, t, a.tok_i64);
    ang = __fmul_rn(tf, a.inv_tok[i]);
  } else {
    int64_t p = ld_ix(a.page, t, a.page_i64);
    if (a.page_mod > 0) {
      p %= a.page_mod;
      if (p < 0) p += a.page_mod;       // non-negative remainder (torch.remainder)
    }
    ang = __fmul_rn((float)p, a.inv_page[i - a.n_tok]);
  }
  float s, c;
  sincosf(ang, &s, &c);
  T* co = reinterpret_cast<T*>(a.cos) + t * a.c_st;
  T* so = reinterpret_cast<T*>(a.sin) + t * a.s_st;
  Rt<T>::store(co + i, c);
  Rt<T>::store(co + i + half, c);
  Rt<T>::store(so + i, s);
  Rt<T>::store(so + i + half, s);
}

// ------------------------------------------------------------ rotary apply
struct RopeK {
  srswa_rope_args a;
  int lph;          // lanes per head: (head_dim / 2) / VE
  int heads;        // HX + HY
};

template <typename T>
__global__ __launch_bounds__(256) void rope_kernel(RopeK p) {
  using V = Vec16<T>;
  constexpr int VE = V::N;
  const srswa_rope_args& a = p.a;
  const int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_tok = (int64_t)p.heads * p.lph;
  if (item >= (int64_t)a.B * a.S * per_tok) return;
  const int64_t n = item / per_tok;
  const int rem = (int)(item % per_tok);
  const int h = rem / p.lph;
  const int e0 = (rem % p.lph) * VE;
  const int half = a.head_dim / 2;
  const int64_t b = n / a.S, s = n % a.S;

  const T* src;
  T* dst;
  if (h < a.HX) {
    src = reinterpret_cast<const T*>(a.x) + b * a.x_sb + s * a.x_ss + (int64_t)h * a.x_sh;
    dst = reinterpret_cast<T*>(a.ox) + b * a.ox_sb + s * a.ox_ss + (int64_t)h * a.ox_sh;
  } else {
    const int hy = h - a.HX;
    src = reinterpret_cast<const T*>(a.y) + b * a.y_sb + s * a.y_ss + (int64_t)hy * a.y_sh;
    dst = reinterpret_cast<T*>(a.oy) + b * a.oy_sb + s * a.oy_ss + (int64_t)hy * a.oy_sh;
  }
  const T* cr = reinterpret_cast<const T*>(a.cos) + b * a.c_sb + s * a.c_ss;
  const T* sr = reinterpret_cast<const T*>(a.sin) + b * a.s_sb + s * a.s_ss;

  float x1[VE], x2[VE], c1[VE], c2[VE], s1[VE], s2[VE], o1[VE], o2[VE];
  V::unpack(*reinterpret_cast<const uint4*>(src + e0), x1);
  V::unpack(*reinterpret_cast<const uint4*>(src + half + e0), x2);
  V::unpack(*reinterpret_cast<const uint4*>(cr + e0), c1);
  V::unpack(*reinterpret_cast<const uint4*>(cr + half + e0), c2);
  V::unpack(*reinterpret_cast<const uint4*>(sr + e0), s1);
  V::unpack(*reinterpret_cast<const uint4*>(sr + half + e0), s2);
#pragma unroll
  for (int e = 0; e < VE; ++e) {
    // first half: x1*cos + (-x2)*sin; second half: x2*cos + x1*sin
    const float a1 = Rt<T>::r(__fmul_rn(x1[e], c1[e]));
    const float b1 = Rt<T>::r(__fmul_rn(-x2[e], s1[e]));
    const float a2 = Rt<T>::r(__fmul_rn(x2[e], c2[e]));
    const float b2 = Rt<T>::r(__fmul_rn(x1[e], s2[e]));
    o1[e] = __fadd_rn(a1, b1);
    o2[e] = __fadd_rn(a2, b2);
  }
  *reinterpret_cast<uint4*>(dst + e0) = V::pack(o1);
  *reinterpret_cast<uint4*>(dst + half + e0) = V::pack(o2);
}

bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace
}  // namespace srswa

using namespace srswa;

extern "C" int srswa_page2d_cos_sin(const srswa_cos_sin_args* a, void* stream) {
  if (!a || !a->tok || !a->page || !a->inv_tok || !a->cos || !a->sin) {
    set_error("page2d cos/sin: null argument");
    return SRSWA_INVALID;
  }
  if (a->T < 0 || a->dim <= 0 || (a->dim & 1) || a->n_tok <= 0 || a->n_tok > a->dim / 2 ||
      (a->n_tok < a->dim / 2 && !a->inv_page) || a->page_mod < 0 || (a->tok_i64 != 0 && a->tok_i64 != 1) ||
      (a->page_i64 != 0 && a->page_i64 != 1) || a->c_st < a->dim || a->s_st < a->dim) {
    set_error("page2d cos/sin: bad sizes or flags");
    return SRSWA_INVALID;
  }
  if (a->out_dtype < 0 || a->out_dtype > 2) {
    set_error("page2d cos/sin: dtype %d not supported", a->out_dtype);
    return SRSWA_UNSUPPORTED;
  }
  const int64_t items = (int64_t)a->T * (a->dim / 2);
  if (items == 0) return SRSWA_OK;
  const dim3 grid((unsigned)((items + 255) / 256));
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (a->out_dtype) {
    case SRSWA_F32: hipLaunchKernelGGL(cos_sin_kernel<float>, grid, dim3(256), 0, st, *a); break;
    case SRSWA_BF16: hipLaunchKernelGGL(cos_sin_kernel<bf16_t>, grid, dim3(256), 0, st, *a); break;
    default: hipLaunchKernelGGL(cos_sin_kernel<__half>, grid, dim3(256), 0, st, *a); break;
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("page2d cos/sin launch failed: %s", hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}

extern "C" int srswa_page2d_rope(const srswa_rope_args* a, void* stream) {
  if (!a || !a->x || !a->ox || !a->cos || !a->sin || (a->y && !a->oy)) {
    set_error("page2d rope: null argument");
    return SRSWA_INVALID;
  }
  const int HY = a->y ? a->HY : 0;
  if (a->B < 0 || a->S < 0 || a->HX <= 0 || HY < 0 || a->head_dim <= 0) {
    set_error("page2d rope: bad sizes");
    return SRSWA_INVALID;
  }
  if (a->dtype < 0 || a->dtype > 2) {
    set_error("page2d rope: dtype %d not supported", a->dtype);
    return SRSWA_UNSUPPORTED;
  }
  const int eb = a->dtype == SRSWA_F32 ? 4 : 2;
  const int ve = 16 / eb;
  const int half = a->head_dim / 2;
  if ((a->head_dim & 1) || half % ve) {
    set_error("page2d rope: head_dim=%d must be a multiple of %d", a->head_dim, 2 * ve);
    return SRSWA_UNSUPPORTED;
  }
  bool ok = al16(a->x) && al16(a->ox) && al16(a->cos) && al16(a->sin);
  for (int64_t st : {a->x_sb, a->x_ss, a->x_sh, a->ox_sb, a->ox_ss, a->ox_sh, a->c_sb, a->c_ss, a->s_sb, a->s_ss})
    ok = ok && (st * eb) % 16 == 0;
  if (a->y) {
    ok = ok && al16(a->y) && al16(a->oy);
    for (int64_t st : {a->y_sb, a->y_ss, a->y_sh, a->oy_sb, a->oy_ss, a->oy_sh}) ok = ok && (st * eb) % 16 == 0;
  }
  if (!ok) {
    set_error("page2d rope: rows and heads must be 16-byte aligned");
    return SRSWA_UNSUPPORTED;
  }
  RopeK k;
  k.a = *a;
  k.a.HY = HY;
  k.lph = half / ve;
  k.heads = a->HX + HY;
  const int64_t items = (int64_t)a->B * a->S * k.heads * k.lph;
  if (items == 0) return SRSWA_OK;
  const dim3 grid((unsigned)((items + 255) / 256));
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (a->dtype) {
    case SRSWA_F32: hipLaunchKernelGGL(rope_kernel<float>, grid, dim3(256), 0, st, k); break;
    case SRSWA_BF16: hipLaunchKernelGGL(rope_kernel<bf16_t>, grid, dim3(256), 0, st, k); break;
    default: hipLaunchKernelGGL(rope_kernel<__half>, grid, dim3(256), 0, st, k); break;
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("page2d rope launch failed: %s", hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}
