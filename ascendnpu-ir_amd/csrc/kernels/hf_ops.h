// Scalar semantics of HFusion/linalg region bodies on CDNA4 (gfx950).
//
// Every function here is the device-side meaning of one op of the region
// builders in bishengir/lib/Dialect/HFusion/IR/HFusionOps.cpp:434-862
// (unary/binary/compare/ternary fns, cast with RoundMode) and
// :1507-1595 (reduce_with_index).  Kernels are compiled with
// -ffp-contract=off so that mul/add stay separately rounded as in the
// reference's CPU lowering; fp32 division and sqrt are the correctly rounded
// HIP defaults.
//
// Storage types in registers: f32 -> float, f64 -> double, bf16/f16 -> the
// 16-bit pattern in uint16_t, iN -> intN_t, i1 -> bool.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <type_traits>

#pragma clang fp contract(off)

namespace hf {

// RoundMode numbering of HFusionEnums.td:122-141
enum RoundMode : int { RINT = 0, ROUND = 1, FLOOR = 2, CEIL = 3, TRUNC = 4, ODD = 5, TRUNCWO = 6 };

__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }
__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }

// ---------------------------------------------------------------- bf16/f16
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

// Round-to-nearest-even f32 -> bf16 (gfx950 v_cvt_pk_bf16_f32); NaN stays NaN.
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

// Rounds the exact value `a` (given as double; every f32/int32 value is exact
// in double) onto a binary format with `p` significand bits and exponent range
// [emin, emax] under `mode`.  Directed modes and round-to-odd follow the
// IEEE-754 definitions; overflow goes to inf or to the largest finite value as
// the mode dictates.
__device__ inline double round_to_format(double x, int p, int emin, int emax, int mode) {
  if (x != x || x == 0.0 || __builtin_isinf(x)) return x;
  bool neg = x < 0;
  double a = neg ? -x : x;
  int lead = ilogb(a);
  if (lead < emin) lead = emin;
  double q = ldexp(1.0, lead - (p - 1));
  double s = a / q;
  double fl = floor(s), fr = s - fl;
  bool odd = fmod(fl, 2.0) != 0.0;
  double r;
  switch (mode) {
  case RINT: r = (fr > 0.5 || (fr == 0.5 && odd)) ? fl + 1 : fl; break;
  case ROUND: r = fr >= 0.5 ? fl + 1 : fl; break;
  case FLOOR: r = (neg && fr > 0) ? fl + 1 : fl; break;
  case CEIL: r = (!neg && fr > 0) ? fl + 1 : fl; break;
  case ODD: r = (fr > 0 && !odd) ? fl + 1 : fl; break;
  default: r = fl;
  }
  double v = r * q;
  double maxf = ldexp(2.0 - ldexp(1.0, -(p - 1)), emax);
  if (v > maxf) {
    bool to_inf = (mode == RINT || mode == ROUND) || (mode == FLOOR && neg) ||
                  (mode == CEIL && !neg);
    v = to_inf ? __builtin_inf() : maxf;
  }
  return neg ? -v : v;
}

template <int MODE> __device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  if constexpr (MODE == RINT) {
    return f32_to_bf16_rne(f);
  } else {
    if (f != f) return f32_to_bf16_rne(f);
    float v = (float)round_to_format((double)f, 8, -126, 127, MODE);
    return (uint16_t)(f2u(v) >> 16);
  }
}

template <int MODE> __device__ __forceinline__ uint16_t f32_to_f16(float f) {
  if constexpr (MODE == RINT) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
  } else {
    if (f != f) return __builtin_bit_cast(uint16_t, (_Float16)f);
    double v = round_to_format((double)f, 11, -14, 15, MODE);
    // v is on the f16 grid (or +-inf), so the RNE conversion is exact
    return __builtin_bit_cast(uint16_t, (_Float16)(float)v);
  }
}

// ---------------------------------------------------------------- fp8
// FMT 0: f8E4M3FN (sign, 4 exponent bits, bias 7, 3 mantissa bits; no
// infinities, S.1111.111 is NaN, largest finite 448); FMT 1: f8E5M2 (bias 15,
// 2 mantissa bits, IEEE-style infinities and NaNs, largest finite 57344).
template <int FMT> __device__ __forceinline__ float fp8_to_f32(uint8_t b) {
  const float sgn = (b & 0x80) ? -1.0f : 1.0f;
  if constexpr (FMT == 0) {
    const int e = (b >> 3) & 15, m = b & 7;
    if (e == 15 && m == 7) return __builtin_nanf("");
    return sgn * (e == 0 ? (float)m * 0x1p-9f : __builtin_ldexpf(1.0f + (float)m * 0.125f, e - 7));
  } else {
    const int e = (b >> 2) & 31, m = b & 3;
    if (e == 31) return m == 0 ? sgn * __builtin_inff() : __builtin_nanf("");
    return sgn * (e == 0 ? (float)m * 0x1p-16f : __builtin_ldexpf(1.0f + (float)m * 0.25f, e - 15));
  }
}

// Rounds the exact value x to the fp8 precision under MODE with no upper
// exponent bound (round_to_format above), then IEEE 754 overflow (7.4) past the
// largest finite value: nearest modes give infinity (NaN in E4M3FN), trunc and
// odd the largest finite value, floor / ceil one or the other by sign; SAT
// clamps to the largest finite value instead.  NaN maps to 0x7F (NaN in both).
template <int FMT, int MODE, bool SAT> __device__ __forceinline__ uint8_t to_fp8(double x) {
  constexpr int P = FMT == 0 ? 4 : 3, EMIN = FMT == 0 ? -6 : -14;
  constexpr double MAXF = FMT == 0 ? 448.0 : 57344.0;
  if (x != x) return 0x7F;
  const bool neg = __builtin_signbit(x);
  const uint8_t s = neg ? 0x80 : 0;
  double v = __builtin_fabs(round_to_format(x, P, EMIN, 1023, MODE));
  if (v > MAXF) {
    const bool to_inf = !SAT && (MODE == RINT || MODE == ROUND || (MODE == FLOOR && neg) || (MODE == CEIL && !neg));
    if (!to_inf) return (uint8_t)(s | (FMT == 0 ? 0x7E : 0x7B));
    return (uint8_t)(s | (FMT == 0 ? 0x7F : 0x7C));
  }
  if (v == 0.0) return s;
  int e = ilogb(v);
  if (e < EMIN) return (uint8_t)(s | (uint8_t)(v * ldexp(1.0, (P - 1) - EMIN)));  // subnormal
  const int m = (int)((v * ldexp(1.0, -e) - 1.0) * (double)(1 << (P - 1)));
  return (uint8_t)(s | ((e + (FMT == 0 ? 7 : 15)) << (P - 1)) | m);
}
template <int FMT, int MODE, bool SAT> __device__ __forceinline__ uint8_t f32_to_fp8(float f) {
  return to_fp8<FMT, MODE, SAT>((double)f);
}

// ---------------------------------------------------------------- ints
template <int MODE> __device__ __forceinline__ float round_integral(float x) {
  if constexpr (MODE == RINT) return __builtin_roundevenf(x);
  else if constexpr (MODE == ROUND) return __builtin_roundf(x);
  else if constexpr (MODE == FLOOR) return __builtin_floorf(x);
  else if constexpr (MODE == CEIL) return __builtin_ceilf(x);
  else if constexpr (MODE == ODD) {
    float t = __builtin_truncf(x);
    if (t != x && __builtin_fmodf(t, 2.0f) == 0.0f) t += (x < 0 ? -1.0f : 1.0f);
    return t;
  } else return __builtin_truncf(x);
}

// hfusion.cast float -> signed integer of type T: round per MODE, then either
// clamp (saturate; NaN -> 0) or keep the low bits (two's-complement wrap).
template <typename T, int MODE, bool SAT> __device__ __forceinline__ T f32_to_int(float f) {
  float r = round_integral<MODE>(f);
  if constexpr (SAT) {
    constexpr double lo = -(double)(1ull << (sizeof(T) * 8 - 1));
    constexpr double hi = (double)(1ull << (sizeof(T) * 8 - 1)) - 1.0;
    if (r != r) return (T)0;
    double d = (double)r;
    d = d < lo ? lo : (d > hi ? hi : d);
    return (T)(int64_t)d;
  } else {
    if constexpr (sizeof(T) == 1) {
      // |r| >= 2^31 is a multiple of 256: its low byte is 0
      return __builtin_fabsf(r) < 2147483648.0f ? (T)(int32_t)r : (T)0;
    } else if constexpr (sizeof(T) <= 4) {
      if (__builtin_expect(__builtin_fabsf(r) < 2147483648.0f, 1)) return (T)(int32_t)r;
      return (T)(int64_t)r;
    } else {
      return (T)(int64_t)r;
    }
  }
}

// arith.fptosi (the CPU lowering's f32 -> iN): truncation toward zero.
template <typename T> __device__ __forceinline__ T fptosi(float f) { return (T)(int64_t)__builtin_truncf(f); }

// integer -> f32 under MODE (sitofp is RINT)
template <int MODE> __device__ __forceinline__ float int_to_f32(int64_t v) {
  if constexpr (MODE == RINT) return (float)v;
  else return (float)round_to_format((double)v, 24, -126, 127, MODE);
}

// ---------------------------------------------------------------- float fns
__device__ __forceinline__ float maximumf(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float minimumf(float a, float b) { return __builtin_elementwise_minimum(a, b); }
__device__ __forceinline__ float maxnumf(float a, float b) { return __builtin_fmaxf(a, b); }
__device__ __forceinline__ float minnumf(float a, float b) { return __builtin_fminf(a, b); }

__device__ __forceinline__ float add(float a, float b) { return a + b; }
__device__ __forceinline__ float sub(float a, float b) { return a - b; }
__device__ __forceinline__ float mul(float a, float b) { return a * b; }
__device__ __forceinline__ float div(float a, float b) { return a / b; }
__device__ __forceinline__ float rec(float a) { return 1.0f / a; }

// mathExt.ilogb (MathExtOps.td:79-91): floor(log2|x|) as a float; -inf at
// zero, +inf at infinity, NaN kept.  The frexp exponent e has |x| = m * 2^e
// with m in [0.5, 1), denormals included, so floor(log2|x|) = e - 1.
__device__ __forceinline__ float ilogb_f(float x) {
  if (__builtin_isnan(x)) return x;
  if (x == 0.0f) return -__builtin_inff();
  if (__builtin_isinf(x)) return __builtin_inff();
  int e;
  (void)__builtin_frexpf(x, &e);
  return (float)(e - 1);
}
// mathExt.ldexp folder (MathExtOps.cpp:70-85): ldexpf(a, int(b)); the count
// saturates to int and NaN counts as 0.
__device__ __forceinline__ float ldexp_f(float a, float b) {
  const int n = __builtin_isnan(b) ? 0 : b >= 2147483647.0f ? 2147483647 : b <= -2147483648.0f ? (-2147483647 - 1) : (int)b;
  return __builtin_ldexpf(a, n);
}
// math.ipowi: a^b in two's complement (the caller truncates to its width);
// a negative exponent gives the integer 1 / a^|b|: 1, +-1 or 0 (0 for a == 0).
__device__ __forceinline__ int64_t ipowi(int64_t a, int64_t b) {
  if (b < 0) return a == 1 ? 1 : a == -1 ? ((b & 1) ? -1 : 1) : 0;
  uint64_t acc = 1, base = (uint64_t)a;
  for (uint64_t e = (uint64_t)b; e; e >>= 1) {
    if (e & 1) acc *= base;
    base *= base;
  }
  return (int64_t)acc;
}
// hfusion.hypot, f32 (the lowering of Normalize.cpp:8969-9036): the largest
// magnitude s scales the others, terms (a_i / s)^2 (1 for a_i == s, 0 when
// s == 0) are summed in operand order, result s * sqrt(sum); any NaN operand
// gives NaN and any infinite one +inf, infinity winning.
__device__ __forceinline__ float hypot_scaled(float x, float y, float z, int n) {
  const float a0 = __builtin_fabsf(x), a1 = __builtin_fabsf(y), a2 = n == 3 ? __builtin_fabsf(z) : 0.0f;
  const bool nan = __builtin_isnan(x) || __builtin_isnan(y) || (n == 3 && __builtin_isnan(z));
  const bool inf = a0 == __builtin_inff() || a1 == __builtin_inff() || (n == 3 && a2 == __builtin_inff());
  float s = a0 > a1 ? a0 : a1;
  if (n == 3) s = s > a2 ? s : a2;
  const float safe = s == 0.0f ? 1.0f : s;
  auto term = [&](float a) -> float {
    if (s == 0.0f) return 0.0f;
    if (a == s) return 1.0f;
    const float q = a / safe;
    return q * q;
  };
  float sum = term(a0) + term(a1);
  if (n == 3) sum = sum + term(a2);
  float r = s * __builtin_sqrtf(sum);
  if (nan) r = __builtin_nanf("");
  if (inf) r = __builtin_inff();
  return r;
}
// f16 hypot: the direct path in f32, sqrt(sum_i a_i * a_i) (then rounded to
// f16 by the caller), with the same NaN / infinity rules.
__device__ __forceinline__ float hypot_direct(float x, float y, float z, int n) {
  const float a0 = __builtin_fabsf(x), a1 = __builtin_fabsf(y), a2 = n == 3 ? __builtin_fabsf(z) : 0.0f;
  const bool nan = __builtin_isnan(x) || __builtin_isnan(y) || (n == 3 && __builtin_isnan(z));
  const bool inf = a0 == __builtin_inff() || a1 == __builtin_inff() || (n == 3 && a2 == __builtin_inff());
  float sum = a0 * a0 + a1 * a1;
  if (n == 3) sum = sum + a2 * a2;
  float r = __builtin_sqrtf(sum);
  if (nan) r = __builtin_nanf("");
  if (inf) r = __builtin_inff();
  return r;
}
// nextafter on f16 bits (IEEE nextafter: NaN in, NaN out; x == y gives y;
// from zero the smallest denormal with y's sign; else one ulp toward y).
__device__ __forceinline__ uint16_t nextafter_h(uint16_t x, uint16_t y) {
  const bool xn = (x & 0x7FFF) > 0x7C00, yn = (y & 0x7FFF) > 0x7C00;
  if (xn) return x;
  if (yn) return y;
  const float fx = hf::f16_to_f32(x), fy = hf::f16_to_f32(y);
  if (fx == fy) return y;
  if ((x & 0x7FFF) == 0) return (uint16_t)((y & 0x8000) | 1);
  const bool away = (__builtin_fabsf(fx) < __builtin_fabsf(fy)) && ((x ^ y) & 0x8000) == 0;
  return (uint16_t)(away ? x + 1 : x - 1);
}
// erfinv(y) in f32: Winitzki's closed-form estimate (a = 0.147), then Newton
// steps on erf(x) - y in double, x -= (erf(x) - y) / (2/sqrt(pi) exp(-x^2)),
// rounded once to f32.  |y| > 1 and NaN give NaN, y = +-1 gives +-inf.
__device__ __forceinline__ float erfinv_f(float yf);

// Modified Bessel function of the first kind, order 0: the power series
// sum_k (x^2/4)^k / (k!)^2, every term positive (no cancellation), summed in
// double until a term no longer changes the sum, rounded once to f32.  i0 is
// even.  The reference lowering forms exp(|x|) * i0e(|x|) in f32
// (Normalize.cpp:8549-8573), so from |x| = 88.72283935546875 on, where the
// f32 exp overflows, its result is +inf although i0 itself stays below
// FLT_MAX up to |x| ~ 91.9: those inputs give +inf here too.  +-inf gives NaN,
// as that form does (exp(inf) * 0).
__device__ __forceinline__ float cyl_bessel_i0_f(float xf) {
  if (__builtin_isnan(xf) || __builtin_isinf(xf)) return __builtin_nanf("");
  double x = __builtin_fabs((double)xf);
  if (x >= 88.72283935546875) return __builtin_inff();
  double q = 0.25 * x * x, term = 1.0, sum = 1.0;
  for (int k = 1; k < 400; ++k) {
    term *= q / ((double)k * (double)k);
    sum += term;
    if (term < sum * 1e-17) break;
  }
  return (float)sum;
}

__device__ __forceinline__ float erfinv_f(float yf) {
  if (__builtin_isnan(yf) || __builtin_fabsf(yf) > 1.0f) return __builtin_nanf("");
  if (yf == 1.0f) return __builtin_inff();
  if (yf == -1.0f) return -__builtin_inff();
  if (yf == 0.0f) return yf;
  const double y = (double)yf, a = 0.147, pi = 3.14159265358979323846;
  const double l = log((1.0 - y) * (1.0 + y));
  const double t = 2.0 / (pi * a) + 0.5 * l;
  double x = sqrt(sqrt(t * t - l / a) - t);
  if (y < 0) x = -x;
  const double k = 2.0 / sqrt(pi);
  for (int i = 0; i < 4; ++i) x -= (erf(x) - y) / (k * exp(-x * x));
  return (float)x;
}
// arith.ceildivui / arith.remui on unsigned operand bits (0 for a zero divisor)
__device__ __forceinline__ uint64_t ceildivu(uint64_t a, uint64_t b) { return b == 0 ? 0 : a / b + (a % b != 0); }
__device__ __forceinline__ uint64_t remu(uint64_t a, uint64_t b) { return b == 0 ? 0 : a % b; }
__device__ __forceinline__ float relu(float a) { return maximumf(0.0f, a); }
__device__ __forceinline__ float rsqrt(float a) { return 1.0f / __builtin_sqrtf(a); }

// exp(x) in fp32 as 2^t with t = RN(x*log2(e)) and the hardware base-2
// exponential.  The rounding of t moves the result by a relative
// ln(2)*|t|*2^-24 (<= 5.2e-6 for results in the normal range, |t| < 126), the
// rounded log2(e) constant (relative 1.3e-8) by ln(2)*|t|*1.3e-8 (<= 1.1e-6),
// plus one ulp of v_exp_f32: at most 6.5e-6 relative, inside the 1e-5 fp32
// tolerance and far inside one bf16 ulp.  Results below 2^-64 are computed as 2^(t+64) * 2^-64
// (one rounding into the denormal range).
__device__ __forceinline__ float exp_f32(float x) {
  const float t = x * 0x1.715476p+0f;
  const bool tiny = t < -64.0f;
  const float r = __builtin_amdgcn_exp2f(tiny ? t + 64.0f : t);
  return tiny ? r * 0x1p-64f : r;
}

// exp(x) in fp32 for an op whose result is rounded (to nearest even) onto a
// narrower format with P significand bits (bf16: 8, f16: 11) and normal range
// [LO, HI].  The CPU computes expf in f32 and rounds that; glibc's expf is
// within 0.51 f32 ulp of exp(x), so it rounds onto the P-bit grid as exp(x)
// itself does unless exp(x) lies within about 0.01 f32 ulp of a midpoint of
// that grid.  exp_f32 is within 6.5e-6 relative (at most 55 f32 ulps) of
// exp(x): when no midpoint lies within 128 f32 ulps of it, it rounds like
// exp(x).  Otherwise (about 0.4 % of bf16 results, 3 % of f16 ones), and
// outside the normal range, exp is evaluated in double and rounded to f32.
template <int P>
__device__ __forceinline__ float exp_narrow(float x) {
  constexpr int D = 24 - P; // f32 significand bits below the P-bit grid
  constexpr float LO = P == 8 ? 0x1p-126f : 0x1p-14f, HI = P == 8 ? 0x1.fffffep127f : 65504.0f;
  const float e = exp_f32(x);
  const uint32_t f = __float_as_uint(e) & ((1u << D) - 1);
  const uint32_t half = 1u << (D - 1);
  const uint32_t dist = f > half ? f - half : half - f;
  if (__builtin_expect(dist > 128u && e >= LO && e <= HI, 1)) return e;
  return (float)exp((double)x);
}

// Exactness switch of the element functions below: kExact evaluates the
// IEEE result directly; kFast takes the cheap path and records in a Guard when the
// cheap path cannot vouch for the exact result, in which case the caller
// re-evaluates that phase with kExact (rare: out-of-range magnitudes or
// quotients within a rounding error of a half-integer).
using kFast = std::integral_constant<bool, false>;
using kExact = std::integral_constant<bool, true>;

// Running evidence of the fast paths (plain arithmetic, issued in program
// order): the largest quotient magnitude seen (NaN-propagating) and the
// exponent range of the per-row reciprocals.
struct Guard {
  float qmax = 0.0f;
  int emin = 0, emax = 0;
  int dmin = 0, dmax = 0; // exponent range of div_rn dividends and quotients
  // quant8x4: range of the biased quotients next to the clamp bounds they
  // must respect
  float tmin = __builtin_inff(), tmax = -__builtin_inff();
  float tmin_need = -__builtin_inff(), tmax_need = __builtin_inff();
  __device__ __forceinline__ bool bad() const {
    return !(qmax <= 0x1p+100f) || emin < -96 || emax > 40 || dmin < -96 || dmax > 100 ||
           !(tmin >= tmin_need) || !(tmax <= tmax_need);
  }
  // per-row divisor check: r = RN(1/b) must be a finite normal number with
  // exponent in [-96, 40] (so |b| >= 2^-41 and the reciprocal is
  // exact-rounded normal); frexp reports 0 for inf/NaN, hence the extra test
  __device__ __forceinline__ void divisor(float r) {
    const int er = __builtin_fabsf(r) <= 0x1.fffffep+127f ? __builtin_amdgcn_frexp_expf(r) : -1000;
    asm volatile("v_min3_i32 %0, %0, %2, %2\n\tv_max3_i32 %1, %1, %2, %2" : "+v"(emin), "+v"(emax) : "v"(er));
  }
};

// rint(RN(a / b)) (round-half-even of the correctly rounded quotient) given
// r = RN(1/b), computed once per row.  q0 = RN(a*r) is within one ulp of a/b
// (r has relative error <= 2^-24), so one Markstein correction
// q1 = RN(q0 + (a - b*q0)*r), with the residual exact by FMA, is RN(a/b)
// (Markstein's theorem for a correctly rounded reciprocal and a faithful
// quotient; checked on the CPU for every b mantissa against 48 random a each,
// 4e8 pairs, with no mismatch).
// Exactness envelope: the row's reciprocal passed Guard::divisor (|b| >=
// 2^-41, normal r) and |q| <= 2^100 (recorded, NaN-propagating: an infinite
// or NaN a or b gives a NaN or infinite q).  Inside it the residual is exact
// unless |a| < 2^-96; then |q| < 2^-55, whose round-to-integral is +-0 with the
// sign of a/b whatever the last bits (round to nearest keeps the sign of every
// intermediate).  Outside it the caller recomputes with IEEE division.
template <typename EX>
__device__ __forceinline__ float rint_div(float a, float b, float r, Guard &g, EX) {
  if constexpr (EX::value) {
    return __builtin_roundevenf(a / b);
  } else {
    float q = a * r;
    const float e = __builtin_fmaf(-q, b, a);
    q = __builtin_fmaf(e, r, q);
    asm volatile("v_maximum3_f32 %0, %0, |%1|, |%1|" : "+v"(g.qmax) : "v"(q));
    return __builtin_roundevenf(q);
  }
}

// int8 dynamic quantisation, four elements to one packed word:
//   (int8)clamp(rint(RN(a_i / b)), LO, HI),  LO >= -128, HI <= 127,
// given r = RN(1/b) (passed Guard::divisor).  With Q = a/b exact,
// tl = RN(a*r + 128 - 2^-15) and th = RN(a*r + 128 + 2^-15) bracket Q + 128:
// a*r = Q(1 + e) with |e| <= 2^-24, so for |Q| < 128 the product is within
// 2^-17 of Q and each sum within 2^-17 more of its target, while RN(Q) + 128
// is within 2^-18 of Q + 128 -- strictly between tl and th.
// v_cvt_pk_u8_f32 rounds half to even and clamps to [0, 255]; RNE is
// monotonic, so when the two packed words agree every byte is
// RNE(RN(Q) + 128) = rint(RN(Q)) + 128 (128 is even) and XOR 0x80 gives the
// int8 value.  A word that disagrees holds a quotient near a half-integer
// (about one element in 10^4): its four elements are recomputed with the
// exact quotient (rint_div) in place.
// Clamps: HI = 127 is the converter's own upper clamp (+inf included);
// LO > -128 and HI < 127 are checked on the tracked extremes, and the
// NaN-propagating minimum also catches NaN quotients: those blocks take the
// exact path.
template <int LO, int HI>
__device__ __forceinline__ uint32_t quant8x4(const float (&a)[4], float b, float r, Guard &g) {
  static_assert(-128 <= LO && LO <= HI && HI <= 127, "int8 clamp bounds");
  constexpr float D = 0x1p-15f;
  float tl[4], th[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    tl[i] = __builtin_fmaf(a[i], r, 128.0f - D);
    th[i] = __builtin_fmaf(a[i], r, 128.0f + D);
  }
  uint32_t wl = __builtin_amdgcn_cvt_pk_u8_f32(tl[0], 0, 0u), wh = __builtin_amdgcn_cvt_pk_u8_f32(th[0], 0, 0u);
#pragma unroll
  for (int i = 1; i < 4; ++i) {
    wl = __builtin_amdgcn_cvt_pk_u8_f32(tl[i], i, wl);
    wh = __builtin_amdgcn_cvt_pk_u8_f32(th[i], i, wh);
  }
  asm volatile("v_minimum3_f32 %0, %0, %1, %2\n\tv_minimum3_f32 %0, %0, %3, %4"
               : "+v"(g.tmin) : "v"(tl[0]), "v"(tl[1]), "v"(tl[2]), "v"(tl[3]));
  g.tmin_need = (float)LO + 127.5f + 0x1p-12f;
  if constexpr (HI < 127) {
    asm volatile("v_maximum3_f32 %0, %0, %1, %2\n\tv_maximum3_f32 %0, %0, %3, %4"
                 : "+v"(g.tmax) : "v"(th[0]), "v"(th[1]), "v"(th[2]), "v"(th[3]));
    g.tmax_need = (float)HI + 128.5f - 0x1p-12f;
  }
  uint32_t w = wl ^ 0x80808080u;
  if (__builtin_expect(wl != wh, 0)) {
    w = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float q = __builtin_amdgcn_fmed3f(rint_div(a[i], b, r, g, kFast{}), (float)LO, (float)HI);
      w |= ((uint32_t)(int32_t)q & 0xFFu) << (8 * i);
    }
  }
  return w;
}

// float already holding an integral value (or +-inf/NaN) -> integer type T:
// no rounding step; saturating or wrapping as the cast requests.
// RN(a / b) given r = RN(1/b), computed once per row: one Markstein
// correction of a*r (see rint_div), then v_div_fixup_f32 for the IEEE results
// of zero, infinite and NaN operands (it also keeps the sign of a zero
// quotient).  Exactness envelope: the row's reciprocal passed Guard::divisor,
// and the dividend and quotient have frexp exponents in [-96, 100] (zero
// counts as 0): then q0 = a*r is normal, the FMA residual a - q0*b is a
// multiple of 2^(ea-47) >= 2^-149 below 2^(ea-23), hence representable, and
// q1 is normal.  Outside it the caller recomputes with IEEE division.
template <typename EX>
__device__ __forceinline__ float div_rn(float a, float b, float r, Guard &g, EX) {
  if constexpr (EX::value) {
    return a / b;
  } else {
    float q = a * r;
    const float e = __builtin_fmaf(-q, b, a);
    q = __builtin_fmaf(e, r, q);
    q = __builtin_amdgcn_div_fixupf(q, b, a);
    const int ea = __builtin_amdgcn_frexp_expf(a), eq = __builtin_amdgcn_frexp_expf(q);
    asm volatile("v_min3_i32 %0, %0, %2, %3\n\tv_max_i32 %1, %1, %3" : "+v"(g.dmin), "+v"(g.dmax) : "v"(ea), "v"(eq));
    return q;
  }
}

template <typename T, bool SAT> __device__ __forceinline__ T integral_to_int(float r) {
  if constexpr (SAT) {
    return f32_to_int<T, TRUNC, true>(r);
  } else if constexpr (sizeof(T) == 1) {
    return __builtin_fabsf(r) < 2147483648.0f ? (T)(int32_t)r : (T)0;
  } else {
    return f32_to_int<T, TRUNC, false>(r);
  }
}

// ---------------------------------------------------------------- wave64
// Butterfly exchange across the 64 lanes of a wavefront.
template <typename T> __device__ __forceinline__ T shfl_xor(T v, int m) { return __shfl_xor(v, m, 64); }

} // namespace hf
