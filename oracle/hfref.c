/*
 * hfref.c — CPU restatement of the reference's CPU lowering for HFusion op
 * groups.  TEST INFRASTRUCTURE ONLY (the parity checker and the timed CPU
 * baseline); the product never links it.  See hfref.h for the contract.
 *
 * Build: -O2 -ffp-contract=off -fno-fast-math (no FMA contraction, IEEE
 * division/sqrt, libm for transcendental math), as the MLIR CPU pipeline
 * produces (bishengir/lib/ExecutionEngine/ExecutionEnginePipelines.cpp:54-89).
 */
#define _GNU_SOURCE
#include "hfref.h"

#include <fenv.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------------ */
/* bf16 / f16 conversions                                                    */
/* ------------------------------------------------------------------------ */

float hfref_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* arith.truncf f32->bf16: round to nearest even; NaN stays a (quiet) NaN. */
uint16_t hfref_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float hfref_f16_to_f32(uint16_t h) {
  uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff;
  if (e == 0x1f) return u2f(s | 0x7f800000u | (m << 13));
  if (e == 0) {
    float v = ldexpf((float)m, -24);
    return s ? -v : v;
  }
  return u2f(s | ((e + 112) << 23) | (m << 13));
}

/* Generic rounding of an exact value `x` onto a binary floating format with
 * `p` significand bits and exponent range [emin, emax], under round mode
 * `mode` (HFusionEnums.td:122-141 numbering).  Returns the rounded value as a
 * long double (exactly representable), or +-inf on overflow.  Written from the
 * IEEE-754 definition of the directed/nearest modes and of round-to-odd
 * ("jamming": truncate, then set the last bit when inexact). */
static long double round_to_format(long double x, int p, int emin, int emax,
                                   int mode) {
  if (isnan(x) || isinf(x) || x == 0) return x;
  int neg = signbit(x) != 0;
  long double a = neg ? -x : x;
  int E;
  frexpl(a, &E); /* a = m * 2^E, m in [0.5, 1): leading bit at 2^(E-1) */
  int lead = E - 1;
  if (lead < emin) lead = emin;
  long double q = ldexpl(1.0L, lead - (p - 1)); /* quantum */
  long double s = a / q;                        /* exact (power of 2) */
  long double fl = floorl(s), fr = s - fl;
  long double r;
  switch (mode) {
  case 0: /* rint: nearest, ties to even */
    r = (fr > 0.5L || (fr == 0.5L && fmodl(fl, 2.0L) != 0)) ? fl + 1 : fl;
    break;
  case 1: /* round: nearest, ties away */
    r = fr >= 0.5L ? fl + 1 : fl;
    break;
  case 2: /* floor */
    r = (neg && fr > 0) ? fl + 1 : fl;
    break;
  case 3: /* ceil */
    r = (!neg && fr > 0) ? fl + 1 : fl;
    break;
  case 5: /* odd */
    r = (fr > 0 && fmodl(fl, 2.0L) == 0) ? fl + 1 : fl;
    break;
  default: /* trunc / truncwithoverflow */
    r = fl;
  }
  long double v = r * q;
  long double maxf = ldexpl(2.0L - ldexpl(1.0L, -(p - 1)), emax);
  if (v > maxf) {
    int to_inf;
    switch (mode) {
    case 0: case 1: to_inf = 1; break;
    case 2: to_inf = neg; break;
    case 3: to_inf = !neg; break;
    default: to_inf = 0;
    }
    v = to_inf ? (long double)INFINITY : maxf;
  }
  return neg ? -v : v;
}

uint16_t hfref_f32_to_bf16_mode(float f, int mode) {
  if (isnan(f)) return hfref_f32_to_bf16(f);
  long double v = round_to_format((long double)f, 8, -126, 127, mode);
  return (uint16_t)(f2u((float)v) >> 16); /* exact: v is on the bf16 grid */
}

uint16_t hfref_f32_to_f16_mode(float f, int mode) {
  uint32_t u = f2u(f);
  uint16_t sgn = (uint16_t)((u >> 16) & 0x8000u);
  if (isnan(f)) return (uint16_t)(sgn | 0x7e00u | ((u >> 13) & 0x3ffu));
  long double v = round_to_format((long double)f, 11, -14, 15, mode);
  if (isinf(v)) return (uint16_t)(sgn | 0x7c00u);
  if (v == 0) return sgn;
  long double a = fabsl(v);
  int E;
  frexpl(a, &E);
  int lead = E - 1;
  uint16_t bits;
  if (lead < -14) { /* subnormal: a = m * 2^-24 */
    bits = (uint16_t)(a / ldexpl(1.0L, -24));
  } else {
    long double mant = a / ldexpl(1.0L, lead) - 1.0L; /* [0,1) */
    bits = (uint16_t)(((lead + 15) << 10) | (uint16_t)(mant * 1024.0L));
  }
  return (uint16_t)(sgn | bits);
}

uint16_t hfref_f32_to_f16(float f) { return hfref_f32_to_f16_mode(f, 0); }

static inline int64_t wrap_bits(int64_t v, int bits) {
  if (bits >= 64) return v;
  uint64_t m = (1ull << bits) - 1ull;
  uint64_t u = (uint64_t)v & m;
  if (u >> (bits - 1)) u |= ~m;
  return (int64_t)u;
}

static long double round_int(long double x, int mode) {
  long double fl = floorl(x), fr = x - fl;
  int neg = x < 0;
  switch (mode) {
  case 0: return (fr > 0.5L || (fr == 0.5L && fmodl(fl, 2.0L) != 0)) ? fl + 1 : fl;
  case 1: return neg ? -floorl(-x + 0.5L) : floorl(x + 0.5L);
  case 2: return fl;
  case 3: return fr > 0 ? fl + 1 : fl;
  case 5: { /* von Neumann: truncate toward zero, jam the last bit */
    long double t = truncl(x);
    if (t != x && fmodl(t, 2.0L) == 0) t += neg ? -1 : 1;
    return t;
  }
  default: return truncl(x);
  }
}

int64_t hfref_f32_to_int_mode(float f, int mode, int bits, int saturate) {
  long double lo = -ldexpl(1.0L, bits - 1), hi = ldexpl(1.0L, bits - 1) - 1;
  if (isnan(f)) return 0;
  long double r = isinf(f) ? (long double)f : round_int((long double)f, mode);
  if (saturate) {
    if (r < lo) r = lo;
    if (r > hi) r = hi;
    return (int64_t)r;
  }
  if (isinf(r) || fabsl(r) >= ldexpl(1.0L, 63)) return INT64_MIN; /* poison */
  return wrap_bits((int64_t)r, bits);
}

float hfref_int_to_f32_mode(int64_t v, int mode) {
  return (float)round_to_format((long double)v, 24, -126, 127, mode);
}

/* HFusionOps.cpp:1926-1938 ConstantFolding::roundToOdd, evaluated in double. */
int64_t hfref_fold_round_to_odd(double x) {
  double rounded = round(x);
  const double epsilon = 1e-9;
  if (fabs(fabs(x - floor(x)) - 0.5) < epsilon) {
    if (((int)rounded) % 2 != 0) rounded = x > 0 ? floor(x) : ceil(x);
  }
  return (int64_t)rounded;
}

/* ------------------------------------------------------------------------ */
/* scalar region bodies (RegionBuilderHelper, HFusionOps.cpp:434-640)        */
/* ------------------------------------------------------------------------ */

/* arith.maximumf / minimumf: NaN-propagating, -0 < +0 */
static inline float maximumf(float a, float b) {
  if (isnan(a) || isnan(b)) return NAN;
  if (a == 0 && b == 0) return (signbit(a) && signbit(b)) ? -0.0f : 0.0f;
  return a > b ? a : b;
}
static inline float minimumf(float a, float b) {
  if (isnan(a) || isnan(b)) return NAN;
  if (a == 0 && b == 0) return (signbit(a) || signbit(b)) ? -0.0f : 0.0f;
  return a < b ? a : b;
}
/* arith.maxnumf / minnumf: a NaN operand yields the other operand */
static inline float maxnumf(float a, float b) {
  if (isnan(a)) return b;
  if (isnan(b)) return a;
  return maximumf(a, b);
}
static inline float minnumf(float a, float b) {
  if (isnan(a)) return b;
  if (isnan(b)) return a;
  return minimumf(a, b);
}

static inline int ldexp_count(float b) {
  if (isnan(b)) return 0;
  if (b >= 2147483647.0f) return 2147483647;
  if (b <= -2147483648.0f) return -2147483647 - 1;
  return (int)b;
}

static inline float unary_f32(int fn, float x) {
  switch (fn) {
  case HFU_SQRT: return sqrtf(x);
  case HFU_RSQRT: { volatile float s = sqrtf(x); return 1.0f / s; }
  case HFU_EXP: return expf(x);
  case HFU_EXP2: return exp2f(x);
  case HFU_LOG: return logf(x);
  case HFU_LOG2: return log2f(x);
  case HFU_LOG10: return log10f(x);
  case HFU_LOG1P: return log1pf(x);
  case HFU_EXPM1: return expm1f(x);
  case HFU_ABS: return fabsf(x);
  case HFU_NEG: return -x;
  case HFU_RELU: return maximumf(0.0f, x);
  case HFU_REC: return 1.0f / x;
  case HFU_TANH: return tanhf(x);
  case HFU_SIN: return sinf(x);
  case HFU_COS: return cosf(x);
  case HFU_ERF: return erff(x);
  case HFU_NEARBYINT: return roundevenf(x);
  case HFU_CEIL: return ceilf(x);
  case HFU_FLOOR: return floorf(x);
  case HFU_ROUND: return roundf(x);
  case HFU_SQUARE: return x * x;
  case HFU_TRUNC: return truncf(x);
  /* math.tan .. math.cosh lower through MathToLLVM to the libm calls
     (HFusionOps.cpp:443-480) */
  case HFU_TAN: return tanf(x);
  case HFU_ACOS: return acosf(x);
  case HFU_ACOSH: return acoshf(x);
  case HFU_ASIN: return asinf(x);
  case HFU_ASINH: return asinhf(x);
  case HFU_ATAN: return atanf(x);
  case HFU_ATANH: return atanhf(x);
  case HFU_SINH: return sinhf(x);
  case HFU_COSH: return coshf(x);
  /* mathExt.lgamma: log|Gamma(x)| (MathExtOps.td:96-106) */
  case HFU_LGAMMA: return lgammaf(x);
  /* mathExt.ilogb: floor(log2|x|) as a float of the operand's type
     (MathExtOps.td:79-91): -inf at zero, +inf at infinity, NaN kept */
  case HFU_ILOGB:
    if (isnan(x)) return x;
    if (x == 0.0f) return -INFINITY;
    if (isinf(x)) return INFINITY;
    return (float)ilogbf(x);
  }
  abort();
}

static inline float binary_f32(int fn, float a, float b) {
  switch (fn) {
  case HFB_ADD: return a + b;
  case HFB_SUB: return a - b;
  case HFB_MUL: return a * b;
  case HFB_DIV: return a / b;
  case HFB_MAXF: return maximumf(a, b);
  case HFB_MINF: return minimumf(a, b);
  case HFB_MAXNUMF: return maxnumf(a, b);
  case HFB_MINNUMF: return minnumf(a, b);
  case HFB_POWF: return powf(a, b);
  case HFB_MODF: return fmodf(a, b);
  case HFB_COPYSIGN: return copysignf(a, b);
  case HFB_ATAN2: return atan2f(a, b);
  /* mathExt.ldexp folder: ldexpf(a, static_cast<int>(b))
     (MathExtOps.cpp:70-85); the conversion saturates, NaN -> 0 */
  case HFB_LDEXP: return ldexpf(a, ldexp_count(b));
  /* mathExt.divfhp folder: IEEE division, nearest-even (MathExtOps.cpp:91-99) */
  case HFB_DIVFHP: return a / b;
  }
  abort();
}

static inline uint64_t ubits(int64_t v, int bits) {
  return bits >= 64 ? (uint64_t)v : ((uint64_t)v & ((1ull << bits) - 1ull));
}

static inline int64_t binary_i64(int fn, int64_t a, int64_t b, int bits) {
  int64_t r;
  switch (fn) {
  case HFB_IADD: r = (int64_t)((uint64_t)a + (uint64_t)b); break;
  case HFB_ISUB: r = (int64_t)((uint64_t)a - (uint64_t)b); break;
  case HFB_IMUL: r = (int64_t)((uint64_t)a * (uint64_t)b); break;
  case HFB_IDIV: r = b == 0 ? 0 : a / b; break;
  case HFB_IREM: r = b == 0 ? 0 : a % b; break;
  case HFB_IMAX: r = a > b ? a : b; break;
  case HFB_IMIN: r = a < b ? a : b; break;
  case HFB_IMAXU: r = ubits(a, bits) > ubits(b, bits) ? a : b; break;
  case HFB_IMINU: r = ubits(a, bits) < ubits(b, bits) ? a : b; break;
  case HFB_IAND: r = a & b; break;
  case HFB_IOR: r = a | b; break;
  case HFB_IXOR: r = a ^ b; break;
  case HFB_ISHL: r = (b < 0 || b >= bits) ? 0 : (int64_t)((uint64_t)a << b); break;
  case HFB_ISHRS: r = (b < 0 || b >= bits) ? 0 : (a >> b); break;
  case HFB_ISHRU: r = (b < 0 || b >= bits) ? 0 : (int64_t)(ubits(a, bits) >> b); break;
  case HFB_IFLOORDIV:
    if (b == 0) { r = 0; break; }
    r = a / b;
    if ((a % b != 0) && ((a < 0) != (b < 0))) r -= 1;
    break;
  case HFB_ICEILDIV:
    if (b == 0) { r = 0; break; }
    r = a / b;
    if ((a % b != 0) && ((a < 0) == (b < 0))) r += 1;
    break;
  /* math.ipowi (HFusionOps.cpp:588-591): a^b with wrap-around; a negative
     exponent gives 1 / a^|b| in integers (0 unless |a| == 1; 0 for a == 0) */
  case HFB_IPOW:
    if (b < 0) {
      r = a == 1 ? 1 : a == -1 ? ((b & 1) ? -1 : 1) : 0;
    } else {
      uint64_t acc = 1, base = (uint64_t)a;
      for (uint64_t e = (uint64_t)b; e; e >>= 1) {
        if (e & 1) acc *= base;
        base *= base;
      }
      r = (int64_t)acc;
    }
    break;
  /* arith.ceildivui / arith.remui on the operands' unsigned bits */
  case HFB_ICEILDIVU: {
    uint64_t ua = ubits(a, bits), ub = ubits(b, bits);
    r = ub == 0 ? 0 : (int64_t)(ua / ub + (ua % ub != 0));
    break;
  }
  case HFB_IREMU: {
    uint64_t ua = ubits(a, bits), ub = ubits(b, bits);
    r = ub == 0 ? 0 : (int64_t)(ua % ub);
    break;
  }
  default: abort();
  }
  return wrap_bits(r, bits);
}

/* ------------------------------------------------------------------------ */
/* array primitives                                                          */
/* ------------------------------------------------------------------------ */

void hfref_unary_f32(int fn, const float *in, float *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = unary_f32(fn, in[i]);
}
void hfref_binary_f32(int fn, const float *a, const float *b, float *out,
                      int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = binary_f32(fn, a[i], b[i]);
}
void hfref_fma_f32(const float *a, const float *b, const float *c, float *out,
                   int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = fmaf(a[i], b[i], c[i]);
}
void hfref_binary_i64(int fn, const int64_t *a, const int64_t *b,
                      int64_t *out, int64_t n, int bits) {
  for (int64_t i = 0; i < n; ++i) out[i] = binary_i64(fn, a[i], b[i], bits);
}
void hfref_compare_f32(int fn, const float *a, const float *b, uint8_t *out,
                       int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    float x = a[i], y = b[i];
    int r;
    switch (fn) {
    case HFC_EQ: r = x == y; break;          /* OEQ */
    case HFC_NE: r = !(x == y); break;       /* UNE */
    case HFC_LT: r = x < y; break;           /* OLT */
    case HFC_LE: r = x <= y; break;          /* OLE */
    case HFC_GT: r = x > y; break;           /* OGT */
    default: r = x >= y;                     /* OGE */
    }
    out[i] = (uint8_t)r;
  }
}
void hfref_compare_i64(int fn, const int64_t *a, const int64_t *b,
                       uint8_t *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    int64_t x = a[i], y = b[i];
    int r;
    switch (fn) {
    case HFC_EQ: r = x == y; break;
    case HFC_NE: r = x != y; break;
    case HFC_LT: r = x < y; break;
    case HFC_LE: r = x <= y; break;
    case HFC_GT: r = x > y; break;
    default: r = x >= y;
    }
    out[i] = (uint8_t)r;
  }
}

/* fp8 (fmt 0: f8E4M3FN, 4-bit exponent bias 7, 3 mantissa bits, no
   infinities, S.1111.111 = NaN, max 448; fmt 1: f8E5M2, bias 15, 2 mantissa
   bits, IEEE-style inf/NaN, max 57344).  Encoding rounds the exact value to
   the format's precision with no upper exponent bound (round_to_format, with
   subnormals below 2^emin), then applies IEEE 754 overflow (section 7.4) when
   the result passes the largest finite value: nearest modes give infinity,
   toward-zero modes (trunc, odd) the largest finite value, floor/ceil one or
   the other by sign; "infinity" is NaN in E4M3FN.  Saturation clamps to the
   largest finite value instead. */
float hfref_fp8_to_f32(uint8_t b, int fmt) {
  const float sgn = (b & 0x80) ? -1.0f : 1.0f;
  if (fmt == 0) {
    int e = (b >> 3) & 15, m = b & 7;
    if (e == 15 && m == 7) return NAN;
    return sgn * (e == 0 ? (float)m * 0x1p-9f : ldexpf(1.0f + (float)m / 8.0f, e - 7));
  }
  int e = (b >> 2) & 31, m = b & 3;
  if (e == 31) return m == 0 ? sgn * INFINITY : NAN;
  return sgn * (e == 0 ? (float)m * 0x1p-16f : ldexpf(1.0f + (float)m / 4.0f, e - 15));
}

static uint8_t to_fp8(long double x, int fmt, int mode, int sat) {
  const int P = fmt == 0 ? 4 : 3, EMIN = fmt == 0 ? -6 : -14;
  const long double MAXF = fmt == 0 ? 448.0L : 57344.0L;
  if (isnan(x)) return 0x7F;
  const int neg = signbit(x) != 0;
  const uint8_t s = neg ? 0x80 : 0;
  const uint8_t big = (uint8_t)(s | (fmt == 0 ? 0x7E : 0x7B));  /* largest finite */
  const uint8_t inf = (uint8_t)(s | (fmt == 0 ? 0x7F : 0x7C));  /* inf, or NaN in E4M3FN */
  long double v = fabsl(round_to_format(x, P, EMIN, 16383, mode)); /* unbounded above */
  if (v > MAXF) {
    if (sat) return big;
    int to_inf;
    switch (mode) {
    case 0: case 1: to_inf = 1; break; /* nearest */
    case 2: to_inf = neg; break;       /* floor */
    case 3: to_inf = !neg; break;      /* ceil */
    default: to_inf = 0;               /* trunc, odd */
    }
    return to_inf ? inf : big;
  }
  if (v == 0.0L) return s;
  int e = ilogbl(v);
  if (e < EMIN) return (uint8_t)(s | (uint8_t)ldexpl(v, (P - 1) - EMIN));
  int m = (int)((ldexpl(v, -e) - 1.0L) * (long double)(1 << (P - 1)));
  return (uint8_t)(s | ((e + (fmt == 0 ? 7 : 15)) << (P - 1)) | m);
}

void hfref_fp8_to_f32_n(const uint8_t *in, float *out, int64_t n, int fmt) {
  for (int64_t i = 0; i < n; ++i) out[i] = hfref_fp8_to_f32(in[i], fmt);
}
void hfref_f32_to_fp8_n(const float *in, uint8_t *out, int64_t n, int fmt, int mode, int sat) {
  for (int64_t i = 0; i < n; ++i) out[i] = to_fp8((long double)in[i], fmt, mode, sat);
}
void hfref_int_to_fp8_n(const int64_t *in, uint8_t *out, int64_t n, int fmt, int mode, int sat) {
  for (int64_t i = 0; i < n; ++i) out[i] = to_fp8((long double)in[i], fmt, mode, sat);
}

void hfref_bf16_to_f32_n(const uint16_t *in, float *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = hfref_bf16_to_f32(in[i]);
}
void hfref_f32_to_bf16_n(const float *in, uint16_t *out, int64_t n, int mode) {
  if (mode == 0)
    for (int64_t i = 0; i < n; ++i) out[i] = hfref_f32_to_bf16(in[i]);
  else
    for (int64_t i = 0; i < n; ++i) out[i] = hfref_f32_to_bf16_mode(in[i], mode);
}
void hfref_f16_to_f32_n(const uint16_t *in, float *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = hfref_f16_to_f32(in[i]);
}
void hfref_f32_to_f16_n(const float *in, uint16_t *out, int64_t n, int mode) {
  for (int64_t i = 0; i < n; ++i) out[i] = hfref_f32_to_f16_mode(in[i], mode);
}
/* arith.fptosi: rounds toward zero; a result outside the target range (or a
 * NaN/inf input) is poison in LLVM — flagged here, value unspecified. */
void hfref_fptosi_n(const float *in, int64_t *out, int64_t n, int bits,
                    int *poison) {
  long double lo = -ldexpl(1.0L, bits - 1), hi = ldexpl(1.0L, bits - 1) - 1;
  int p = 0;
  for (int64_t i = 0; i < n; ++i) {
    float f = in[i];
    if (isnan(f) || isinf(f)) { p = 1; out[i] = 0; continue; }
    long double t = truncl((long double)f);
    if (t < lo || t > hi) { p = 1; out[i] = 0; continue; }
    out[i] = (int64_t)t;
  }
  if (poison) *poison = p;
}
void hfref_f32_to_int_mode_n(const float *in, int64_t *out, int64_t n,
                             int mode, int bits, int saturate) {
  for (int64_t i = 0; i < n; ++i)
    out[i] = hfref_f32_to_int_mode(in[i], mode, bits, saturate);
}
void hfref_int_to_f32_n(const int64_t *in, float *out, int64_t n, int mode) {
  for (int64_t i = 0; i < n; ++i) out[i] = hfref_int_to_f32_mode(in[i], mode);
}
void hfref_roundeven_n(const float *in, float *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = roundevenf(in[i]);
}
void hfref_round_n(const float *in, float *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = roundf(in[i]);
}

/* linalg.reduce region `op(%in, %init)` folded serially along the reduced
 * index (ConvertHIVMToUpstream.cpp:573-752; convert-linalg-to-loops). */
void hfref_reduce_f32(int op, const float *x, float *acc, int64_t K,
                      int64_t N) {
  for (int64_t k = 0; k < K; ++k) {
    const float *row = x + k * N;
    for (int64_t j = 0; j < N; ++j) {
      float in = row[j], a = acc[j];
      switch (op) {
      case 0: a = in + a; break;
      case 1: a = in * a; break;
      case 2: a = maximumf(in, a); break;
      case 3: a = minimumf(in, a); break;
      case 4: a = maxnumf(in, a); break;
      default: a = minnumf(in, a);
      }
      acc[j] = a;
    }
  }
}

void hfref_reduce_i64(int op, const int64_t *x, int64_t *acc, int64_t K,
                      int64_t N, int bits) {
  static const int map[] = {HFB_IADD, HFB_IMUL, HFB_IMAX, HFB_IMIN, HFB_IAND,
                            HFB_IOR,  HFB_IXOR, HFB_IMAXU, HFB_IMINU};
  for (int64_t k = 0; k < K; ++k)
    for (int64_t j = 0; j < N; ++j)
      acc[j] = binary_i64(map[op], x[k * N + j], acc[j], bits);
}

/* hfusion.reduce_with_index region (HFusionOps.cpp:1507-1595):
 *   res = maximumf(in, outV); pred = res OGT outV;
 *   outI = pred ? index : outI; outV = res                                  */
void hfref_reduce_with_index_f32(int kind, const float *x, const int64_t *in_idx,
                                 float *val, int64_t *idx, int64_t K,
                                 int64_t N) {
  for (int64_t k = 0; k < K; ++k)
    for (int64_t j = 0; j < N; ++j) {
      float in = x[k * N + j], ov = val[j];
      float res = kind == 0 ? maximumf(in, ov) : minimumf(in, ov);
      int pred = kind == 0 ? (res > ov) : (res < ov);
      if (pred) idx[j] = in_idx ? in_idx[k * N + j] : k;
      val[j] = res;
    }
}

void hfref_reduce_with_index_i64(int kind, const int64_t *x,
                                 const int64_t *in_idx, int64_t *val,
                                 int64_t *idx, int64_t K, int64_t N, int bits) {
  for (int64_t k = 0; k < K; ++k)
    for (int64_t j = 0; j < N; ++j) {
      int64_t in = x[k * N + j], ov = val[j], res;
      int pred;
      switch (kind) {
      case 0: res = in > ov ? in : ov; pred = res > ov; break;
      case 1: res = in < ov ? in : ov; pred = res < ov; break;
      case 2: res = ubits(in, bits) > ubits(ov, bits) ? in : ov;
        pred = ubits(res, bits) > ubits(ov, bits); break;
      default: res = ubits(in, bits) < ubits(ov, bits) ? in : ov;
        pred = ubits(res, bits) < ubits(ov, bits);
      }
      if (pred) idx[j] = in_idx ? in_idx[k * N + j] : k;
      val[j] = res;
    }
}

/* upstream linalg.matmul region: out = out + cast(a) * cast(b), k innermost */
void hfref_matmul_i8_i32(const int8_t *A, const int8_t *B, int32_t *C,
                         int64_t M, int64_t N, int64_t K, int b_transposed) {
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      int32_t acc = C[m * N + n];
      const int8_t *a = A + m * K;
      if (b_transposed) {
        const int8_t *b = B + n * K;
        for (int64_t k = 0; k < K; ++k) acc += (int32_t)a[k] * (int32_t)b[k];
      } else {
        for (int64_t k = 0; k < K; ++k)
          acc += (int32_t)a[k] * (int32_t)B[k * N + n];
      }
      C[m * N + n] = acc;
    }
}

void hfref_matmul_f32(const float *A, const float *B, float *C, int64_t M,
                      int64_t N, int64_t K, int b_transposed) {
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      float acc = C[m * N + n];
      for (int64_t k = 0; k < K; ++k) {
        float b = b_transposed ? B[n * K + k] : B[k * N + n];
        float p = A[m * K + k] * b;
        acc = acc + p;
      }
      C[m * N + n] = acc;
    }
}

/* e2m1 (OCP MX fp4): sign, two exponent bits (bias 1), one mantissa bit;
 * exponent 0 is the subnormal 0.5 m.  The 16 values are +-{0, 0.5, 1, 1.5,
 * 2, 3, 4, 6}. */
float hfref_fp4_to_f32(uint8_t v) {
  const float sgn = (v & 8) ? -1.0f : 1.0f;
  const int e = (v >> 1) & 3, m = v & 1;
  return sgn * (e == 0 ? 0.5f * (float)m : ldexpf(1.0f + 0.5f * (float)m, e - 1));
}

/* hfusion.matmul_mx (HFusionOps.td:1233-1291): C = C + (A * 2^(sa-127)) x
 * (B * 2^(sb-127)), A [M, K] and B [K, N] of formats fa / fb (0 e4m3, 1
 * e5m2: one byte each; 4 e2m1: two values per byte, the even k in the low
 * nibble, so A is [M, K/2] and B [K/2, N] bytes -- the packing of the
 * reference's fp4x2_e2m1_t, LocalMmadMx.cpp:131-133, whose K factor is 2),
 * sa [M, ceil(K/32)] and sb [N, ceil(K/32)] e8m0 bytes, one per 32 k of the
 * K logical values.  Each scaled operand is rounded to f32, the product is an f32
 * multiply and the sum runs serially over k from C's value, as the linalg.matmul
 * region the reference's decomposition ends in (HFusionOps.cpp:3590-3790:
 * operand * broadcast scale, then linalg.matmul).  Where the
 * decomposition's f16 steps are exact (scaled operands inside f16's range)
 * this is the decomposition's value bit for bit.
 * e8m0 255 is NaN here, as in the OCP MX format and the MI355X's scaled MFMA.
 * The reference decomposition instead shifts the byte into a bf16 exponent
 * (ui8 -> i16, << 7, bitcast), so 255 reads as +inf there and a block of
 * nonzero same-sign products gives +-inf rather than NaN: the 255 case is
 * parity unpinned against the reference. */
static float mx_scale(uint8_t e) {
  return e == 255 ? NAN : ldexpf(1.0f, (int)e - 127);
}
static float mx_scaled(uint8_t v, int fmt, uint8_t e) {
  const float x = fmt == 4 ? hfref_fp4_to_f32(v) : hfref_fp8_to_f32(v, fmt);
  return (float)((double)x * (double)mx_scale(e));
}
/* element k of a row of packed values (fmt 4: nibbles, low one first) */
static uint8_t mx_elem(const uint8_t *row, int64_t k, int64_t stride, int fmt) {
  if (fmt != 4) return row[k * stride];
  const uint8_t b = row[(k / 2) * stride];
  return (k & 1) ? (uint8_t)(b >> 4) : (uint8_t)(b & 15);
}
void hfref_matmul_mx(const uint8_t *A, const uint8_t *B, const uint8_t *sa, const uint8_t *sb, float *C, int64_t M,
                     int64_t N, int64_t K, int fa, int fb) {
  const int64_t kb = (K + 31) / 32;
  const int64_t Ka = fa == 4 ? (K + 1) / 2 : K; /* bytes per row of A */
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      float acc = C[m * N + n];
      for (int64_t k = 0; k < K; ++k) {
        const float x = mx_scaled(mx_elem(A + m * Ka, k, 1, fa), fa, sa[m * kb + k / 32]);
        const float y = mx_scaled(mx_elem(B + n, k, N, fb), fb, sb[n * kb + k / 32]);
        const float p = x * y;
        acc = acc + p;
      }
      C[m * N + n] = acc;
    }
}

/* ------------------------------------------------------------------------ */
/* composed groups (op-by-op loop nests, temporaries materialised)           */
/* ------------------------------------------------------------------------ */

void hfref_vecadd_f32(const float *a, const float *b, float *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}

/* The RMSNorm + dynamic per-token int8 quant group, op by op as authored in
 * the group IR (rms_norm structure of
 * bishengir/test/bishengir-compile/hfusion/compile-rms-norm-fp32-split-n.mlir:5-47,
 * followed by absmax / scale / nearbyint / clamp / cast). */
void hfref_rmsnorm_quant(const uint16_t *x_bf16, const uint16_t *gamma_bf16,
                         float eps, int8_t *q, float *scale, int64_t R,
                         int64_t C) {
  size_t n = (size_t)R * (size_t)C;
  float *xf = malloc(n * 4), *t = malloc(n * 4), *g = malloc((size_t)C * 4);
  float *ss = malloc((size_t)R * 4), *inv = malloc((size_t)R * 4);
  float *amax = malloc((size_t)R * 4);
  for (size_t i = 0; i < n; ++i) xf[i] = hfref_bf16_to_f32(x_bf16[i]);
  for (size_t i = 0; i < n; ++i) t[i] = xf[i] * xf[i];
  for (int64_t r = 0; r < R; ++r) {
    float acc = 0.0f;
    for (int64_t c = 0; c < C; ++c) acc = t[r * C + c] + acc;
    ss[r] = acc;
  }
  float cf = (float)C;
  for (int64_t r = 0; r < R; ++r) {
    float mean = ss[r] / cf;
    float ms = mean + eps;
    float rt = sqrtf(ms);
    inv[r] = 1.0f / rt;
  }
  for (int64_t c = 0; c < C; ++c) g[c] = hfref_bf16_to_f32(gamma_bf16[c]);
  for (int64_t r = 0; r < R; ++r)
    for (int64_t c = 0; c < C; ++c) {
      float y1 = xf[r * C + c] * inv[r];
      t[r * C + c] = y1 * g[c];
    }
  for (int64_t r = 0; r < R; ++r) {
    float acc = 0.0f;
    for (int64_t c = 0; c < C; ++c) acc = maximumf(fabsf(t[r * C + c]), acc);
    amax[r] = acc;
  }
  for (int64_t r = 0; r < R; ++r) scale[r] = amax[r] / 127.0f;
  for (int64_t r = 0; r < R; ++r)
    for (int64_t c = 0; c < C; ++c) {
      float v = t[r * C + c] / scale[r];
      v = roundevenf(v);
      v = minimumf(v, 127.0f);
      v = maximumf(v, -127.0f);
      q[r * C + c] = (int8_t)(int32_t)v; /* fptosi: value is integral, in range */
    }
  free(xf); free(t); free(g); free(ss); free(inv); free(amax);
}

/* Safe softmax group (bishengir/test/Dialect/HFusion/regbase/Normalize/
 * hfusion-normalize-reduction-ops.mlir:262-277 structure, maximumf reduce),
 * then truncf to bf16. */
void hfref_softmax_bf16(const float *x, uint16_t *out, int64_t R, int64_t C) {
  size_t n = (size_t)R * (size_t)C;
  float *e = malloc(n * 4), *m = malloc((size_t)R * 4), *s = malloc((size_t)R * 4);
  for (int64_t r = 0; r < R; ++r) {
    float acc = -INFINITY;
    for (int64_t c = 0; c < C; ++c) acc = maximumf(x[r * C + c], acc);
    m[r] = acc;
  }
  for (int64_t r = 0; r < R; ++r)
    for (int64_t c = 0; c < C; ++c) e[r * C + c] = x[r * C + c] - m[r];
  for (size_t i = 0; i < n; ++i) e[i] = expf(e[i]);
  for (int64_t r = 0; r < R; ++r) {
    float acc = 0.0f;
    for (int64_t c = 0; c < C; ++c) acc = e[r * C + c] + acc;
    s[r] = acc;
  }
  for (int64_t r = 0; r < R; ++r)
    for (int64_t c = 0; c < C; ++c)
      out[r * C + c] = hfref_f32_to_bf16(e[r * C + c] / s[r]);
  free(e); free(m); free(s);
}

/* reduce_with_index <max> over the last axis, init (-inf, 0), i32 indices. */
void hfref_argmax(const float *x, float *val, int32_t *idx, int64_t R,
                  int64_t C) {
  for (int64_t r = 0; r < R; ++r) {
    float ov = -INFINITY;
    int32_t oi = 0;
    const float *row = x + r * C;
    for (int64_t c = 0; c < C; ++c) {
      float res = maximumf(row[c], ov);
      if (res > ov) oi = (int32_t)c;
      ov = res;
    }
    val[r] = ov;
    idx[r] = oi;
  }
}

/* W8A8: C = matmul_transpose_b(A, B) in i32 (init 0), then
 * bf16( (sitofp(C) * s_tok[m]) * s_ch[n] ). */
void hfref_w8a8_dequant_rows(const int8_t *A, const int8_t *Bt,
                             const float *s_tok, const float *s_ch,
                             uint16_t *out, int64_t M, int64_t N, int64_t K,
                             int64_t m0, int64_t m1) {
  (void)M;
  int32_t *acc = malloc((size_t)N * 4);
  for (int64_t m = m0; m < m1; ++m) {
    memset(acc, 0, (size_t)N * 4);
    hfref_matmul_i8_i32(A + m * K, Bt, acc, 1, N, K, 1);
    for (int64_t n = 0; n < N; ++n) {
      float c = (float)acc[n];
      float t = c * s_tok[m];
      float u = t * s_ch[n];
      out[m * N + n] = hfref_f32_to_bf16(u);
    }
  }
  free(acc);
}


/* ---------------------------------------------------------------- memref ABI
 * Ranked descriptors as the MLIR C interface lays them out
 * (BiShengIRRunnerUtils.cpp:99-110 passes them to `_mlir_ciface_` entries):
 * two pointers, the offset, then R sizes and R strides, all 64-bit. */
typedef struct {
  char *allocated, *aligned;
  int64_t offset;
  int64_t dims[]; /* sizes[R] then strides[R] */
} hfref_memref;

static int64_t memref_numel(const hfref_memref *m, int rank) {
  int64_t n = 1;
  for (int k = 0; k < rank; ++k) n *= m->dims[k];
  return n;
}

/* walks the elements in row-major order, copying between the strided view and
 * a dense buffer (to_dense != 0: view -> dense) */
static void memref_copy(const hfref_memref *m, int rank, int esz, char *dense, int to_dense) {
  const int64_t n = memref_numel(m, rank);
  int64_t idx[8] = {0};
  for (int64_t e = 0; e < n; ++e) {
    int64_t off = m->offset;
    for (int k = 0; k < rank; ++k) off += idx[k] * m->dims[rank + k];
    char *p = m->aligned + off * esz;
    if (to_dense) memcpy(dense + e * esz, p, (size_t)esz);
    else memcpy(p, dense + e * esz, (size_t)esz);
    for (int k = rank - 1; k >= 0; --k) {
      if (++idx[k] < m->dims[k]) break;
      idx[k] = 0;
    }
  }
}

int hfref_memref_gather(const void *desc, int rank, int elem_size, void *dense) {
  if (!desc || !dense || rank < 0 || rank > 8) return -1;
  memref_copy((const hfref_memref *)desc, rank, elem_size, (char *)dense, 1);
  return 0;
}

int hfref_memref_scatter(const void *dense, const void *desc, int rank, int elem_size) {
  if (!desc || !dense || rank < 0 || rank > 8) return -1;
  memref_copy((const hfref_memref *)desc, rank, elem_size, (char *)(uintptr_t)dense, 0);
  return 0;
}

static int dims_are(const void *desc, int rank, const int64_t *want) {
  const hfref_memref *m = (const hfref_memref *)desc;
  if (!m) return 0;
  for (int k = 0; k < rank; ++k)
    if (m->dims[k] != want[k]) return 0;
  return 1;
}

static void *gathered(const void *desc, int rank, int esz) {
  const hfref_memref *m = (const hfref_memref *)desc;
  void *d = malloc((size_t)(memref_numel(m, rank) * esz) + 1);
  memref_copy(m, rank, esz, (char *)d, 1);
  return d;
}

static void *dense_for(const void *desc, int rank, int esz) {
  return malloc((size_t)(memref_numel((const hfref_memref *)desc, rank) * esz) + 1);
}

static void put_back(void *dense, const void *desc, int rank, int esz) {
  memref_copy((const hfref_memref *)desc, rank, esz, (char *)dense, 0);
  free(dense);
}

int hfref_vecadd_f32_memref(const void *a, const void *b, const void *out) {
  if (!a) return -1;
  const int64_t n[1] = {((const hfref_memref *)a)->dims[0]};
  if (!dims_are(b, 1, n) || !dims_are(out, 1, n)) return -1;
  float *da = gathered(a, 1, 4), *db = gathered(b, 1, 4), *dout = dense_for(out, 1, 4);
  hfref_vecadd_f32(da, db, dout, n[0]);
  put_back(dout, out, 1, 4);
  free(da);
  free(db);
  return 0;
}

int hfref_rmsnorm_quant_memref(const void *x, const void *gamma, float eps, const void *q, const void *scale) {
  if (!x) return -1;
  const hfref_memref *mx = (const hfref_memref *)x;
  const int64_t rc[2] = {mx->dims[0], mx->dims[1]}, c[1] = {rc[1]}, r[1] = {rc[0]};
  if (!dims_are(gamma, 1, c) || !dims_are(q, 2, rc) || !dims_are(scale, 1, r)) return -1;
  uint16_t *dx = gathered(x, 2, 2), *dg = gathered(gamma, 1, 2);
  int8_t *dq = dense_for(q, 2, 1);
  float *ds = dense_for(scale, 1, 4);
  hfref_rmsnorm_quant(dx, dg, eps, dq, ds, rc[0], rc[1]);
  put_back(dq, q, 2, 1);
  put_back(ds, scale, 1, 4);
  free(dx);
  free(dg);
  return 0;
}

int hfref_softmax_bf16_memref(const void *x, const void *out) {
  if (!x) return -1;
  const hfref_memref *mx = (const hfref_memref *)x;
  const int64_t rc[2] = {mx->dims[0], mx->dims[1]};
  if (!dims_are(out, 2, rc)) return -1;
  float *dx = gathered(x, 2, 4);
  uint16_t *dout = dense_for(out, 2, 2);
  hfref_softmax_bf16(dx, dout, rc[0], rc[1]);
  put_back(dout, out, 2, 2);
  free(dx);
  return 0;
}

int hfref_argmax_memref(const void *x, const void *val, const void *idx) {
  if (!x) return -1;
  const hfref_memref *mx = (const hfref_memref *)x;
  const int64_t rc[2] = {mx->dims[0], mx->dims[1]}, r[1] = {rc[0]};
  if (!dims_are(val, 1, r) || !dims_are(idx, 1, r)) return -1;
  float *dx = gathered(x, 2, 4), *dv = dense_for(val, 1, 4);
  int32_t *di = dense_for(idx, 1, 4);
  hfref_argmax(dx, dv, di, rc[0], rc[1]);
  put_back(dv, val, 1, 4);
  put_back(di, idx, 1, 4);
  free(dx);
  return 0;
}

int hfref_w8a8_dequant_memref(const void *a, const void *bt, const void *s_tok, const void *s_ch, const void *out) {
  if (!a || !bt) return -1;
  const hfref_memref *ma = (const hfref_memref *)a, *mb = (const hfref_memref *)bt;
  const int64_t M = ma->dims[0], K = ma->dims[1], N = mb->dims[0];
  const int64_t nk[2] = {N, K}, m1[1] = {M}, n1[1] = {N}, mn[2] = {M, N};
  if (!dims_are(bt, 2, nk) || !dims_are(s_tok, 1, m1) || !dims_are(s_ch, 1, n1) || !dims_are(out, 2, mn)) return -1;
  int8_t *da = gathered(a, 2, 1), *db = gathered(bt, 2, 1);
  float *dst = gathered(s_tok, 1, 4), *dsc = gathered(s_ch, 1, 4);
  uint16_t *dout = dense_for(out, 2, 2);
  hfref_w8a8_dequant_rows(da, db, dst, dsc, dout, M, N, K, 0, M);
  put_back(dout, out, 2, 2);
  free(da);
  free(db);
  free(dst);
  free(dsc);
  return 0;
}

/* ---- hfusion.sort ----
 * The reference decomposes a value sort along the last axis into a bubble
 * sort (bishengir/lib/Dialect/HFusion/Transforms/DecomposeOpInterfaceImpl.cpp:
 * 740-830): n-1 passes, each comparing elements j and j+1 for j = 0..n-2 in
 * order and swapping them when `cmpf ugt` (ascending) / `cmpf ult`
 * (descending) holds -- unordered predicates, so any comparison with a NaN
 * swaps -- or, for integers, `cmpi sgt` / `cmpi slt`.  Restated literally. */
static double sort_key(const void *row, int64_t j, int kind) {
  switch (kind) {
  case 0: return ((const float *)row)[j];
  case 1: return hfref_f16_to_f32(((const uint16_t *)row)[j]);
  case 2: return hfref_bf16_to_f32(((const uint16_t *)row)[j]);
  case 8: return ((const int8_t *)row)[j];
  case 16: return ((const int16_t *)row)[j];
  case 32: return ((const int32_t *)row)[j];
  default: return 0;
  }
}

static int sort_need_swap(const void *row, int64_t j, int kind, int descending) {
  if (kind == 64) {
    const int64_t a = ((const int64_t *)row)[j], b = ((const int64_t *)row)[j + 1];
    return descending ? a < b : a > b;
  }
  const double a = sort_key(row, j, kind), b = sort_key(row, j + 1, kind);
  if (kind <= 2 && (a != a || b != b)) return 1; /* unordered: ugt / ult hold */
  return descending ? a < b : a > b;
}

int hfref_sort_rows(void *data, int64_t R, int64_t L, int kind, int descending) {
  int esz;
  switch (kind) {
  case 0: case 32: esz = 4; break;
  case 1: case 2: case 16: esz = 2; break;
  case 8: esz = 1; break;
  case 64: esz = 8; break;
  default: return -1;
  }
  for (int64_t r = 0; r < R; ++r) {
    char *row = (char *)data + r * L * esz;
    for (int64_t pass = 0; pass + 1 < L; ++pass)
      for (int64_t j = 0; j + 1 < L; ++j)
        if (sort_need_swap(row, j, kind, descending)) {
          char t[8];
          memcpy(t, row + j * esz, esz);
          memcpy(row + j * esz, row + (j + 1) * esz, esz);
          memcpy(row + (j + 1) * esz, t, esz);
        }
  }
  return 0;
}
