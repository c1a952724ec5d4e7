// Shared device helpers for the SR-SWA gfx950 kernels: bf16/fp16 <-> fp32,
// 64-lane wavefront reductions, error recording for the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <limits.h>
#include <stdint.h>

#include <type_traits>

#include "srswa.h"

namespace srswa {

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// record an error message for srswa_last_error() (host side, per thread)
void set_error(const char* fmt, ...);

struct bf16_t { uint16_t bits; };

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16, round to nearest even (gfx950 v_cvt_pk_bf16_f32)
typedef __bf16 bf16x2_native_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2_native_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  return (uint16_t)(pack_bf16x2(f, 0.f) & 0xffffu);
}

__device__ __forceinline__ float h16_lo(uint32_t w) {
  return __half2float(__ushort_as_half((unsigned short)(w & 0xffffu)));
}
__device__ __forceinline__ float h16_hi(uint32_t w) {
  return __half2float(__ushort_as_half((unsigned short)(w >> 16)));
}
__device__ __forceinline__ uint32_t pack_h16x2(float lo, float hi) {
  return (uint32_t)__half_as_ushort(__float2half_rn(lo)) |
         ((uint32_t)__half_as_ushort(__float2half_rn(hi)) << 16);
}

// 16-byte vector of storage elements <-> fp32 values.
template <typename T> struct Vec16;
template <> struct Vec16<float> {
  static constexpr int N = 4;
  __device__ __forceinline__ static void unpack(const uint4& w, float* f) {
    f[0] = __uint_as_float(w.x); f[1] = __uint_as_float(w.y);
    f[2] = __uint_as_float(w.z); f[3] = __uint_as_float(w.w);
  }
  __device__ __forceinline__ static uint4 pack(const float* f) {
    return make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]),
                      __float_as_uint(f[3]));
  }
};
template <> struct Vec16<bf16_t> {
  static constexpr int N = 8;
  __device__ __forceinline__ static void unpack(const uint4& w, float* f) {
    f[0] = bf16_lo(w.x); f[1] = bf16_hi(w.x); f[2] = bf16_lo(w.y); f[3] = bf16_hi(w.y);
    f[4] = bf16_lo(w.z); f[5] = bf16_hi(w.z); f[6] = bf16_lo(w.w); f[7] = bf16_hi(w.w);
  }
  __device__ __forceinline__ static uint4 pack(const float* f) {
    return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                      pack_bf16x2(f[6], f[7]));
  }
};
template <> struct Vec16<__half> {
  static constexpr int N = 8;
  __device__ __forceinline__ static void unpack(const uint4& w, float* f) {
    f[0] = h16_lo(w.x); f[1] = h16_hi(w.x); f[2] = h16_lo(w.y); f[3] = h16_hi(w.y);
    f[4] = h16_lo(w.z); f[5] = h16_hi(w.z); f[6] = h16_lo(w.w); f[7] = h16_hi(w.w);
  }
  __device__ __forceinline__ static uint4 pack(const float* f) {
    return make_uint4(pack_h16x2(f[0], f[1]), pack_h16x2(f[2], f[3]), pack_h16x2(f[4], f[5]),
                      pack_h16x2(f[6], f[7]));
  }
};

// fp8 K/V cache formats (srswa_dtype codes of the k_cache / v_cache of the
// paged serving kernels).  Every fp8 value is exact in bf16 and fp16, so the
// kernels convert at load time and run their 16-bit paths unchanged, as the
// reference's `k.to(q.dtype)` does, on gfx950's scaled conversions
// (v_cvt_scalef32_pk_{f32,bf16,f16}_{fp8,bf8}: two bytes of a word per
// instruction, read as the OCP e4m3fn / e5m2 formats and multiplied by a power
// of two).
constexpr int kFp8E4M3FN = 3, kFp8E4M3FNUZ = 4, kFp8E5M2 = 5, kFp8E5M2FNUZ = 6;

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_native_t __attribute__((ext_vector_type(2)));

// An FNUZ byte is the same OCP byte's value halved (its exponent bias is one
// higher), so the FNUZ formats convert with scale 1/2, except three kinds of
// byte that OCP reads differently: 0x80 (FNUZ NaN, OCP -0) and the codes OCP
// keeps for NaN / infinity, which FNUZ uses for ordinary values (|b| = 0x7f in
// e4m3: 240; exponent 31 in e5m2: (1 + m/4) 2^15).
template <int F>
struct Fp8Fmt {
  static constexpr bool E4 = F == kFp8E4M3FN || F == kFp8E4M3FNUZ;
  static constexpr bool FNUZ = F == kFp8E4M3FNUZ || F == kFp8E5M2FNUZ;
  static constexpr float kScale = FNUZ ? 0.5f : 1.f;
};

// Bit 7 of a byte of the result is set when that byte of w may be one of the
// FNUZ bytes above (never missed; a borrow between bytes can flag a harmless
// neighbour), so a word whose result is 0 takes the fast conversion as is.
//   (~w & e) - 1: a byte with all exponent bits set (and, for e4m3, all
//                 mantissa bits) is 0 before the subtraction and 0xff after;
//                 any other byte stays below 0x80;
//   ((w & 0x7f) - 1) & w: bit 7 of 0x80 (magnitude 0, sign set).
template <bool E4>
__device__ __forceinline__ uint32_t fnuz_special_bits(uint32_t w) {
  constexpr uint32_t kE = E4 ? 0x7f7f7f7fu : 0x7c7c7c7cu;
  const uint32_t t1 = (~w & kE) - 0x01010101u;
  const uint32_t t2 = ((w & 0x7f7f7f7fu) - 0x01010101u) & w;
  return t1 | t2;
}

// the FNUZ value of byte i of w when it is one of the bytes OCP reads
// differently, else v (that byte's fast conversion)
template <bool E4>
__device__ __forceinline__ float fnuz_fix(uint32_t w, int i, float v) {
  const uint32_t b = (w >> (8 * i)) & 0xffu;
  if constexpr (E4) {
    v = (b & 0x7fu) == 0x7fu ? ((b & 0x80u) ? -240.f : 240.f) : v;
  } else {
    const float big = (float)(4u + (b & 3u)) * 8192.f;   // (1 + m/4) 2^15
    v = (b & 0x7cu) == 0x7cu ? ((b & 0x80u) ? -big : big) : v;
  }
  return b == 0x80u ? __uint_as_float(0x7fc00000u) : v;
}

// two bytes (the low half of w, or the high half when HI) -> fp32 pair
template <int F, bool HI>
__device__ __forceinline__ f32x2_t fp8x2_f32(uint32_t w) {
  if constexpr (Fp8Fmt<F>::E4) return __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, Fp8Fmt<F>::kScale, HI);
  else return __builtin_amdgcn_cvt_scalef32_pk_f32_bf8(w, Fp8Fmt<F>::kScale, HI);
}

// The FNUZ special-byte flags of an 8-byte piece (bit 7 of a byte, as
// fnuz_special_bits; constant 0 for the OCP formats).  A loop ORs the flags of
// all its pieces and takes one branch: the fast conversions below when no bit
// 7 is set, the exact ones (per-byte fix-up) otherwise.
template <int F>
__device__ __forceinline__ uint32_t fp8_special_bits(const uint2& w) {
  if constexpr (Fp8Fmt<F>::FNUZ)
    return fnuz_special_bits<Fp8Fmt<F>::E4>(w.x) | fnuz_special_bits<Fp8Fmt<F>::E4>(w.y);
  else
    return 0u;
}
__device__ __forceinline__ bool fp8_any_special(uint32_t bits) { return (bits & 0x80808080u) != 0u; }

// eight fp8 bytes (byte 0 of w.x first) -> fp32, without the FNUZ fix-up
template <int F>
__device__ __forceinline__ void fp8x8_to_f32_fast(const uint2& w, float* f) {
  const f32x2_t p0 = fp8x2_f32<F, false>(w.x), p1 = fp8x2_f32<F, true>(w.x);
  const f32x2_t p2 = fp8x2_f32<F, false>(w.y), p3 = fp8x2_f32<F, true>(w.y);
  f[0] = p0[0]; f[1] = p0[1]; f[2] = p1[0]; f[3] = p1[1];
  f[4] = p2[0]; f[5] = p2[1]; f[6] = p3[0]; f[7] = p3[1];
}

// eight fp8 bytes -> fp32, exact for every byte
template <int F>
__device__ __forceinline__ void fp8x8_to_f32_exact(const uint2& w, float* f) {
  fp8x8_to_f32_fast<F>(w, f);
  if constexpr (Fp8Fmt<F>::FNUZ) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[i] = fnuz_fix<Fp8Fmt<F>::E4>(w.x, i, f[i]);
      f[4 + i] = fnuz_fix<Fp8Fmt<F>::E4>(w.y, i, f[4 + i]);
    }
  }
}

// two bytes (the low half of w, or the high half when HI) -> a packed pair of T
// (bf16 / fp16)
template <int F, typename T, bool HI>
__device__ __forceinline__ uint32_t fp8x2_to(uint32_t w) {
  constexpr bool E4 = Fp8Fmt<F>::E4;
  constexpr float s = Fp8Fmt<F>::kScale;
  if constexpr (std::is_same<T, bf16_t>::value) {
    if constexpr (E4) return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, s, HI));
    else return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, s, HI));
  } else {
    static_assert(std::is_same<T, __half>::value, "fp8 caches convert to bf16 or fp16");
    if constexpr (E4) return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, s, HI));
    else return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_bf8(w, s, HI));
  }
}

// eight fp8 bytes -> eight values of T as one 16-byte vector, one instruction
// per pair, without the FNUZ fix-up
template <int F, typename T>
__device__ __forceinline__ uint4 fp8x8_to_fast(const uint2& w) {
  return make_uint4(fp8x2_to<F, T, false>(w.x), fp8x2_to<F, T, true>(w.x), fp8x2_to<F, T, false>(w.y),
                    fp8x2_to<F, T, true>(w.y));
}

// eight fp8 bytes -> eight values of T, exact for every byte (through fp32)
template <int F, typename T>
__device__ __forceinline__ uint4 fp8x8_to_exact(const uint2& w) {
  if constexpr (Fp8Fmt<F>::FNUZ) {
    float f[8];
    fp8x8_to_f32_exact<F>(w, f);
    return Vec16<T>::pack(f);
  } else {
    return fp8x8_to_fast<F, T>(w);
  }
}

// Runs fn(std::integral_constant<int, F>) for the fp8 format fmt: one uniform
// branch around a whole loop instead of one per converted vector.
template <typename Fn>
__device__ __forceinline__ void fp8_dispatch(int fmt, Fn&& fn) {
  switch (fmt) {
    case kFp8E4M3FN: fn(std::integral_constant<int, kFp8E4M3FN>{}); break;
    case kFp8E5M2: fn(std::integral_constant<int, kFp8E5M2>{}); break;
    case kFp8E4M3FNUZ: fn(std::integral_constant<int, kFp8E4M3FNUZ>{}); break;
    default: fn(std::integral_constant<int, kFp8E5M2FNUZ>{}); break;
  }
}

// Full-wavefront reductions (64 lanes, every lane active) on DPP: each level
// is a VALU operand modifier instead of an LDS permute round trip.  Within each
// 16-lane row: quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror,
// row_mirror leave every lane with its row's total; row_bcast:15 then adds row
// 0's total into row 1 and row 2's into row 3, row_bcast:31 adds lane 31's
// (rows 0 + 1) into rows 2 and 3, so lane 63 holds the wave's total, which
// readlane hands to every lane (the same bits everywhere).
namespace dpp {
constexpr int kXor1 = 0xb1;      // quad_perm [1, 0, 3, 2]
constexpr int kXor2 = 0x4e;      // quad_perm [2, 3, 0, 1]
constexpr int kHalfMirror = 0x141;
constexpr int kMirror = 0x140;
constexpr int kBcast15 = 0x142;
constexpr int kBcast31 = 0x143;

template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ uint32_t mov(uint32_t identity, uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)identity, (int)v, CTRL, ROWS, 0xf, false);
}
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ float movf(float identity, float v) {
  return __uint_as_float(mov<CTRL, ROWS>(__float_as_uint(identity), __float_as_uint(v)));
}
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ uint64_t mov64(uint64_t identity, uint64_t v) {
  const uint32_t lo = mov<CTRL, ROWS>((uint32_t)identity, (uint32_t)v);
  const uint32_t hi = mov<CTRL, ROWS>((uint32_t)(identity >> 32), (uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}

// op over the wave; T is float, double (as its bits) or uint64_t
template <typename T, typename Op>
__device__ __forceinline__ T reduce(T v, T identity, Op op) {
  auto m = [&](auto ctrl_tag, auto rows_tag, T x) __attribute__((always_inline)) {
    constexpr int C = decltype(ctrl_tag)::value, R = decltype(rows_tag)::value;
    if constexpr (sizeof(T) == 8) {
      return __builtin_bit_cast(T, mov64<C, R>(__builtin_bit_cast(uint64_t, identity), __builtin_bit_cast(uint64_t, x)));
    } else {
      return __builtin_bit_cast(T, mov<C, R>(__builtin_bit_cast(uint32_t, identity), __builtin_bit_cast(uint32_t, x)));
    }
  };
  using I = int;
  v = op(v, m(std::integral_constant<I, kXor1>{}, std::integral_constant<I, 0xf>{}, v));
  v = op(v, m(std::integral_constant<I, kXor2>{}, std::integral_constant<I, 0xf>{}, v));
  v = op(v, m(std::integral_constant<I, kHalfMirror>{}, std::integral_constant<I, 0xf>{}, v));
  v = op(v, m(std::integral_constant<I, kMirror>{}, std::integral_constant<I, 0xf>{}, v));
  v = op(v, m(std::integral_constant<I, kBcast15>{}, std::integral_constant<I, 0xa>{}, v));
  v = op(v, m(std::integral_constant<I, kBcast31>{}, std::integral_constant<I, 0xc>{}, v));
  if constexpr (sizeof(T) == 8) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), 63);
    return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
  } else {
    return __builtin_bit_cast(T, (uint32_t)__builtin_amdgcn_readlane((int)__builtin_bit_cast(uint32_t, v), 63));
  }
}
}  // namespace dpp

// max / sum of this lane's value and lane (l ^ 32)'s, on the VALU:
// v_permlane32_swap exchanges the upper half of its first operand with the
// lower half of its second, so with both operands v every lane ends holding
// {v[l], v[l ^ 32]} (the two orders give the same bits: fmaxf and a two-term
// sum are commutative)
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// A workgroup barrier for LDS traffic only: this wave's LDS operations are
// complete (lgkmcnt(0)) and every wave has arrived, while its global loads stay
// in flight (__syncthreads()'s fence also waits for those).  One volatile asm
// with a memory clobber, so no memory access is moved across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ int wave_max_int(int v) {
  return dpp::reduce<int>(v, INT_MIN, [](int a, int b) { return a > b ? a : b; });
}
__device__ __forceinline__ int wave_min_int(int v) {
  return dpp::reduce<int>(v, INT_MAX, [](int a, int b) { return a < b ? a : b; });
}

__device__ __forceinline__ float wave_max(float v) {
  return dpp::reduce<float>(v, -INFINITY, [](float a, float b) { return fmaxf(a, b); });
}
__device__ __forceinline__ float wave_sum(float v) {
  return dpp::reduce<float>(v, 0.f, [](float a, float b) { return a + b; });
}
__device__ __forceinline__ float wave_min(float v) {
  return dpp::reduce<float>(v, INFINITY, [](float a, float b) { return fminf(a, b); });
}
__device__ __forceinline__ double wave_sum_f64(double v) {
  return dpp::reduce<double>(v, 0.0, [](double a, double b) { return a + b; });
}
__device__ __forceinline__ int wave_sum_int(int v) {
  return dpp::reduce<int>(v, 0, [](int a, int b) { return a + b; });
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  return dpp::reduce<uint64_t>(v, 0ull, [](uint64_t a, uint64_t b) { return a > b ? a : b; });
}

// Bitonic sort of one unsigned value per lane, descending over the wave (lane 0
// the largest): stage (K, J) compares lanes J apart; blocks with bit K of the
// lane clear end descending, the others ascending, and K = 64 makes one run.
// Lane (l ^ J)'s value for J in {1, 2, 4, 8, 16, 32}, on the VALU: DPP
// quad_perm [1,0,3,2] / [2,3,0,1]; xor 4 as row_half_mirror of the quad
// reversal [3,2,1,0] (lane i of an 8-lane half reads 7 - i after the quad
// flip, which is i ^ 4); xor 8 as row_ror:8 (a 16-lane row rotated by half);
// xor 16 / 32 by v_permlane16_swap / v_permlane32_swap, which exchange the odd
// rows of the first operand with the even rows of the second (16 / 32-lane
// rows): with both operands v, a lane whose row bit is clear finds the partner
// in the second result, the others in the first.
template <int J>
__device__ __forceinline__ uint32_t xor_lane_u32(uint32_t v, int lane) {
  if constexpr (J == 1) return dpp::mov<dpp::kXor1>(v, v);
  else if constexpr (J == 2) return dpp::mov<dpp::kXor2>(v, v);
  else if constexpr (J == 4) return dpp::mov<dpp::kHalfMirror>(v, dpp::mov<0x1b>(v, v));
  else if constexpr (J == 8) return dpp::mov<0x128>(v, v);
  else if constexpr (J == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (lane & 16) ? r[0] : r[1];
  } else {
    static_assert(J == 32, "J: a power of two below 64");
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (lane & 32) ? r[0] : r[1];
  }
}
template <int J, typename U>
__device__ __forceinline__ U xor_lane(U v, int lane) {
  if constexpr (sizeof(U) == 8) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = xor_lane_u32<J>((uint32_t)b, lane), hi = xor_lane_u32<J>((uint32_t)(b >> 32), lane);
    return __builtin_bit_cast(U, ((uint64_t)hi << 32) | lo);
  } else {
    return __builtin_bit_cast(U, xor_lane_u32<J>(__builtin_bit_cast(uint32_t, v), lane));
  }
}

template <typename U, int K, int J>
__device__ __forceinline__ U bitonic_merge(U v, int lane) {
  const U w = xor_lane<J>(v, lane);
  const bool take_max = ((lane & J) == 0) == ((lane & K) == 0);
  v = take_max ? (w > v ? w : v) : (w > v ? v : w);
  if constexpr (J > 1) return bitonic_merge<U, K, J / 2>(v, lane);
  else return v;
}
template <typename U, int K = 2>
__device__ __forceinline__ U wave_sort_desc(U v, int lane) {
  v = bitonic_merge<U, K, K / 2>(v, lane);
  if constexpr (K < kWave) return wave_sort_desc<U, K * 2>(v, lane);
  else return v;
}

// Order-preserving map of an fp32 value to an unsigned key (a > b <=> key(a) >
// key(b) for non-NaN values) and back.
__device__ __forceinline__ uint32_t f32_order_key(float x) {
  const uint32_t u = __float_as_uint(x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float f32_from_order_key(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Reduce-scatter of N partial sums per lane over the 2 O lanes of a row (c =
// the lane's index in the row): at each level the lanes differing in bit O of c
// swap the halves of part they do not keep and add them to the halves they do.
// After log2(N) levels, part[0] of lane c holds the row-wide sum of partial
// c / (2 O / N).  The levels are template arguments: a run-time-halving loop
// is left rolled by hipcc and turns part[] into a compare / select chain.
template <int N, int O, int NA>
__device__ __forceinline__ void reduce_scatter(float (&part)[NA], int c) {
  if constexpr (N > 1) {
    static_assert(O >= 1 && N <= NA, "reduce_scatter: a level without a lane bit");
    const bool upper = (c & O) != 0;
#pragma unroll
    for (int j = 0; j < N / 2; ++j) {
      const float send = upper ? part[j] : part[j + N / 2];
      const float keep = upper ? part[j + N / 2] : part[j];
      part[j] = keep + __shfl_xor(send, O, kWave);
    }
    reduce_scatter<N / 2, O / 2>(part, c);
  }
}

__host__ __device__ constexpr int ceil_div(int a, int b) { return (a + b - 1) / b; }

}  // namespace srswa
