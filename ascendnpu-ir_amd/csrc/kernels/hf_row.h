// Row-resident building blocks for LAST_AXIS_PBR / elementwise groups on
// CDNA4.
//
// A row group is TR consecutive threads (TR = 64 * WPR, or a power of two
// below 64) owning one row of C elements; thread `lt` holds EPL = NCH * VEC
// elements, chunk j of VEC contiguous columns starting at
// j * TR * VEC + lt * VEC, so each chunk is one 16-byte (or narrower) global
// access and a wave's accesses are fully coalesced.
//
// This replaces the Ascend UB-tiled vector library behind hivm.hir.v* ops
// (bishengir/lib/Template/lib/Vector/Reduction/ReduceAR.cpp and
// Elementwise/EltWise*.cpp) — no data is staged through a scratchpad except
// for the cross-wave combine and the serial-order chain below.
#pragma once
#include "hf_ops.h"

namespace hf {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
template <int BYTES> struct vec_bits;
template <> struct vec_bits<16> { using t = u32x4; };
template <> struct vec_bits<8> { using t = u32x2; };
template <> struct vec_bits<4> { using t = uint32_t; };
template <> struct vec_bits<2> { using t = uint16_t; };
template <> struct vec_bits<1> { using t = uint8_t; };

// VEC contiguous elements through one global access of VEC * sizeof(T) bytes
// (callers guarantee the alignment: row length and chunk offsets are
// multiples of VEC).
template <typename T, int VEC> __device__ __forceinline__ void vec_load(const T *__restrict__ p, T *out) {
  constexpr int B = VEC * (int)sizeof(T);
  if constexpr (B == 16 || B == 8 || B == 4 || B == 2 || B == 1) {
    using V = typename vec_bits<B>::t;
    V v = __builtin_nontemporal_load(reinterpret_cast<const V *>(p));
    __builtin_memcpy(out, &v, B);
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) out[i] = p[i];
  }
}

template <typename T, int VEC> __device__ __forceinline__ void vec_store(T *__restrict__ p, const T *in) {
  constexpr int B = VEC * (int)sizeof(T);
  if constexpr (B == 16 || B == 8 || B == 4 || B == 2 || B == 1) {
    using V = typename vec_bits<B>::t;
    V v;
    __builtin_memcpy(&v, in, B);
    __builtin_nontemporal_store(v, reinterpret_cast<V *>(p));
  } else {
#pragma unroll
    for (int i = 0; i < VEC; ++i) p[i] = in[i];
  }
}

// Opaque redefinition of a register array: values computed from it after this
// point are not merged (CSE) with values computed before, so cheap element
// chains are recomputed per phase instead of being kept live across a
// reduction (which would exhaust the VGPRs).
template <typename T, int N> __device__ __forceinline__ void launder(T (&a)[N]) {
  if constexpr ((N * sizeof(T)) % 4 == 0 && sizeof(T) < 4) {
    // launder whole dwords so packed 8/16-bit elements stay packed
    constexpr int W = N * sizeof(T) / 4;
    uint32_t w[W];
    __builtin_memcpy(w, a, sizeof(w));
#pragma unroll
    for (int i = 0; i < W; ++i) asm volatile("" : "+v"(w[i]));
    __builtin_memcpy(a, w, sizeof(w));
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) asm volatile("" : "+v"(a[i]));
  }
}

template <typename T, int VEC, int NCH, int TR, bool MASKED>
__device__ __forceinline__ void row_load(const T *__restrict__ rowp, int lt, int64_t C, T *out) {
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int64_t c0 = (int64_t)j * TR * VEC + (int64_t)lt * VEC;
    if constexpr (!MASKED) {
      vec_load<T, VEC>(rowp + c0, &out[j * VEC]);
    } else {
      if (c0 + VEC <= C) {
        vec_load<T, VEC>(rowp + c0, &out[j * VEC]);
      } else {
#pragma unroll
        for (int v = 0; v < VEC; ++v) out[j * VEC + v] = (c0 + v < C) ? rowp[c0 + v] : T(0);
      }
    }
  }
}

// The RPW rows of a row group, issued chunk-major (chunk j of every row before
// chunk j+1), so consumers of the first columns wait only for those loads.
template <typename T, int VEC, int NCH, int TR, int RPW, bool MASKED>
__device__ __forceinline__ void rows_load(const T *__restrict__ base, const int64_t (&row)[RPW], int64_t C, int lt, T *out) {
#pragma unroll
  for (int j = 0; j < NCH; ++j)
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
      const T *rowp = base + row[rr] * C;
      T *o = out + rr * (NCH * VEC) + j * VEC;
      const int64_t c0 = (int64_t)j * TR * VEC + (int64_t)lt * VEC;
      if constexpr (!MASKED) {
        vec_load<T, VEC>(rowp + c0, o);
      } else {
        if (c0 + VEC <= C) {
          vec_load<T, VEC>(rowp + c0, o);
        } else {
#pragma unroll
          for (int v = 0; v < VEC; ++v) o[v] = (c0 + v < C) ? rowp[c0 + v] : T(0);
        }
      }
    }
}

// Vector chunks [j0, j1) of the RPW rows of a row group (chunk-major).
template <typename T, int VEC, int NCH, int TR, int RPW, bool MASKED>
__device__ __forceinline__ void rows_load_range(const T *__restrict__ base, const int64_t (&row)[RPW], int64_t C, int lt,
                                                T *out, int j0, int j1) {
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    if (j < j0 || j >= j1) continue;
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) {
      const T *rowp = base + row[rr] * C;
      T *o = out + rr * (NCH * VEC) + j * VEC;
      const int64_t c0 = (int64_t)j * TR * VEC + (int64_t)lt * VEC;
      if constexpr (!MASKED) {
        vec_load<T, VEC>(rowp + c0, o);
      } else {
        if (c0 + VEC <= C) {
          vec_load<T, VEC>(rowp + c0, o);
        } else {
#pragma unroll
          for (int v = 0; v < VEC; ++v) o[v] = (c0 + v < C) ? rowp[c0 + v] : T(0);
        }
      }
    }
  }
}

template <typename T, int VEC, int NCH, int TR, bool MASKED>
__device__ __forceinline__ void row_store(T *__restrict__ rowp, int lt, int64_t C, const T *in) {
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int64_t c0 = (int64_t)j * TR * VEC + (int64_t)lt * VEC;
    if constexpr (!MASKED) {
      vec_store<T, VEC>(rowp + c0, &in[j * VEC]);
    } else {
      if (c0 + VEC <= C) {
        vec_store<T, VEC>(rowp + c0, &in[j * VEC]);
      } else {
#pragma unroll
        for (int v = 0; v < VEC; ++v)
          if (c0 + v < C) rowp[c0 + v] = in[j * VEC + v];
      }
    }
  }
}

// Stores vector chunk j (VEC elements) of this lane's share of a row.
template <typename T, int VEC, int TR, bool MASKED>
__device__ __forceinline__ void row_store_chunk(T *__restrict__ rowp, int lt, int64_t C, int j, const T *in) {
  const int64_t c0 = (int64_t)j * TR * VEC + (int64_t)lt * VEC;
  if constexpr (!MASKED) {
    vec_store<T, VEC>(rowp + c0, in);
  } else {
    if (c0 + VEC <= C) {
      vec_store<T, VEC>(rowp + c0, in);
    } else {
#pragma unroll
      for (int v = 0; v < VEC; ++v)
        if (c0 + v < C) rowp[c0 + v] = in[v];
    }
  }
}

// All-reduce of one value per thread across the TR threads of a row group.
// In-wave: xor butterfly over min(TR, 64) lanes (every lane ends with the same
// bits because all combiners are commutative).  Across the WPR waves of a
// row: one LDS slot per wave, then a fixed-order fold.  `lds` holds
// RB * WPR entries and is private to this call site.
template <int TR, int RB, typename T, typename F>
__device__ __forceinline__ T row_allreduce(T v, F comb, T *lds, int rloc, int lt) {
  constexpr int W = TR < 64 ? TR : 64;
#pragma unroll
  for (int m = W / 2; m >= 1; m >>= 1) v = comb(v, shfl_xor(v, m));
  if constexpr (TR > 64) {
    constexpr int WPR = TR / 64;
    if ((lt & 63) == 0) lds[rloc * WPR + lt / 64] = v;
    __syncthreads();
    T r = lds[rloc * WPR];
#pragma unroll
    for (int w = 1; w < WPR; ++w) r = comb(r, lds[rloc * WPR + w]);
    v = r;
  }
  return v;
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// acc + rp[0] + rp[1] + ... + rp[N-1], strictly in that order, from LDS.
// The dependent adds run at the v_add_f32 latency (7.3-7.7 cycles on gfx950)
// only if the LDS reads never stall them.  The compiler, short of registers
// in this kernel, reuses one 4-register buffer and waits on every read, so
// the 512-float case is one asm statement: two fixed buffers, the reads of the
// next 16 floats in flight while the 16 adds of the current ones run (about
// 10 -> 7.7 cycles per add measured in the RMSNorm kernel).
template <int N>
__device__ __forceinline__ float lds_chain_sum(const float *rp, float acc) {
  static_assert(N % 64 == 0, "chunk must be a multiple of 64 floats");
  if constexpr (N == 512) {
    // 32 groups of 16 floats through two fixed register buffers
    // (v224-v239, v240-v255): the four reads of group g+1 are in flight
    // while the 16 dependent adds of group g run, so the LDS latency stays
    // hidden behind the chain.  One asm statement, so no compiler code runs
    // between a read and the wait that covers it.
    const uint32_t p = (uint32_t)(uintptr_t)rp;
    asm volatile(
      "ds_read_b128 v[224:227], %[p] offset:0\n"
      "ds_read_b128 v[228:231], %[p] offset:16\n"
      "ds_read_b128 v[232:235], %[p] offset:32\n"
      "ds_read_b128 v[236:239], %[p] offset:48\n"
      "ds_read_b128 v[240:243], %[p] offset:64\n"
      "ds_read_b128 v[244:247], %[p] offset:80\n"
      "ds_read_b128 v[248:251], %[p] offset:96\n"
      "ds_read_b128 v[252:255], %[p] offset:112\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v224, %[acc]\n"
      "v_add_f32 %[acc], v225, %[acc]\n"
      "v_add_f32 %[acc], v226, %[acc]\n"
      "v_add_f32 %[acc], v227, %[acc]\n"
      "v_add_f32 %[acc], v228, %[acc]\n"
      "v_add_f32 %[acc], v229, %[acc]\n"
      "v_add_f32 %[acc], v230, %[acc]\n"
      "v_add_f32 %[acc], v231, %[acc]\n"
      "v_add_f32 %[acc], v232, %[acc]\n"
      "v_add_f32 %[acc], v233, %[acc]\n"
      "v_add_f32 %[acc], v234, %[acc]\n"
      "v_add_f32 %[acc], v235, %[acc]\n"
      "v_add_f32 %[acc], v236, %[acc]\n"
      "v_add_f32 %[acc], v237, %[acc]\n"
      "v_add_f32 %[acc], v238, %[acc]\n"
      "v_add_f32 %[acc], v239, %[acc]\n"
      "ds_read_b128 v[224:227], %[p] offset:128\n"
      "ds_read_b128 v[228:231], %[p] offset:144\n"
      "ds_read_b128 v[232:235], %[p] offset:160\n"
      "ds_read_b128 v[236:239], %[p] offset:176\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v240, %[acc]\n"
      "v_add_f32 %[acc], v241, %[acc]\n"
      "v_add_f32 %[acc], v242, %[acc]\n"
      "v_add_f32 %[acc], v243, %[acc]\n"
      "v_add_f32 %[acc], v244, %[acc]\n"
      "v_add_f32 %[acc], v245, %[acc]\n"
      "v_add_f32 %[acc], v246, %[acc]\n"
      "v_add_f32 %[acc], v247, %[acc]\n"
      "v_add_f32 %[acc], v248, %[acc]\n"
      "v_add_f32 %[acc], v249, %[acc]\n"
      "v_add_f32 %[acc], v250, %[acc]\n"
      "v_add_f32 %[acc], v251, %[acc]\n"
      "v_add_f32 %[acc], v252, %[acc]\n"
      "v_add_f32 %[acc], v253, %[acc]\n"
      "v_add_f32 %[acc], v254, %[acc]\n"
      "v_add_f32 %[acc], v255, %[acc]\n"
      "ds_read_b128 v[240:243], %[p] offset:192\n"
      "ds_read_b128 v[244:247], %[p] offset:208\n"
      "ds_read_b128 v[248:251], %[p] offset:224\n"
      "ds_read_b128 v[252:255], %[p] offset:240\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v224, %[acc]\n"
      "v_add_f32 %[acc], v225, %[acc]\n"
      "v_add_f32 %[acc], v226, %[acc]\n"
      "v_add_f32 %[acc], v227, %[acc]\n"
      "v_add_f32 %[acc], v228, %[acc]\n"
      "v_add_f32 %[acc], v229, %[acc]\n"
      "v_add_f32 %[acc], v230, %[acc]\n"
      "v_add_f32 %[acc], v231, %[acc]\n"
      "v_add_f32 %[acc], v232, %[acc]\n"
      "v_add_f32 %[acc], v233, %[acc]\n"
      "v_add_f32 %[acc], v234, %[acc]\n"
      "v_add_f32 %[acc], v235, %[acc]\n"
      "v_add_f32 %[acc], v236, %[acc]\n"
      "v_add_f32 %[acc], v237, %[acc]\n"
      "v_add_f32 %[acc], v238, %[acc]\n"
      "v_add_f32 %[acc], v239, %[acc]\n"
      "ds_read_b128 v[224:227], %[p] offset:256\n"
      "ds_read_b128 v[228:231], %[p] offset:272\n"
      "ds_read_b128 v[232:235], %[p] offset:288\n"
      "ds_read_b128 v[236:239], %[p] offset:304\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v240, %[acc]\n"
      "v_add_f32 %[acc], v241, %[acc]\n"
      "v_add_f32 %[acc], v242, %[acc]\n"
      "v_add_f32 %[acc], v243, %[acc]\n"
      "v_add_f32 %[acc], v244, %[acc]\n"
      "v_add_f32 %[acc], v245, %[acc]\n"
      "v_add_f32 %[acc], v246, %[acc]\n"
      "v_add_f32 %[acc], v247, %[acc]\n"
      "v_add_f32 %[acc], v248, %[acc]\n"
      "v_add_f32 %[acc], v249, %[acc]\n"
      "v_add_f32 %[acc], v250, %[acc]\n"
      "v_add_f32 %[acc], v251, %[acc]\n"
      "v_add_f32 %[acc], v252, %[acc]\n"
      "v_add_f32 %[acc], v253, %[acc]\n"
      "v_add_f32 %[acc], v254, %[acc]\n"
      "v_add_f32 %[acc], v255, %[acc]\n"
      "ds_read_b128 v[240:243], %[p] offset:320\n"
      "ds_read_b128 v[244:247], %[p] offset:336\n"
      "ds_read_b128 v[248:251], %[p] offset:352\n"
      "ds_read_b128 v[252:255], %[p] offset:368\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v224, %[acc]\n"
      "v_add_f32 %[acc], v225, %[acc]\n"
      "v_add_f32 %[acc], v226, %[acc]\n"
      "v_add_f32 %[acc], v227, %[acc]\n"
      "v_add_f32 %[acc], v228, %[acc]\n"
      "v_add_f32 %[acc], v229, %[acc]\n"
      "v_add_f32 %[acc], v230, %[acc]\n"
      "v_add_f32 %[acc], v231, %[acc]\n"
      "v_add_f32 %[acc], v232, %[acc]\n"
      "v_add_f32 %[acc], v233, %[acc]\n"
      "v_add_f32 %[acc], v234, %[acc]\n"
      "v_add_f32 %[acc], v235, %[acc]\n"
      "v_add_f32 %[acc], v236, %[acc]\n"
      "v_add_f32 %[acc], v237, %[acc]\n"
      "v_add_f32 %[acc], v238, %[acc]\n"
      "v_add_f32 %[acc], v239, %[acc]\n"
      "ds_read_b128 v[224:227], %[p] offset:384\n"
      "ds_read_b128 v[228:231], %[p] offset:400\n"
      "ds_read_b128 v[232:235], %[p] offset:416\n"
      "ds_read_b128 v[236:239], %[p] offset:432\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v240, %[acc]\n"
      "v_add_f32 %[acc], v241, %[acc]\n"
      "v_add_f32 %[acc], v242, %[acc]\n"
      "v_add_f32 %[acc], v243, %[acc]\n"
      "v_add_f32 %[acc], v244, %[acc]\n"
      "v_add_f32 %[acc], v245, %[acc]\n"
      "v_add_f32 %[acc], v246, %[acc]\n"
      "v_add_f32 %[acc], v247, %[acc]\n"
      "v_add_f32 %[acc], v248, %[acc]\n"
      "v_add_f32 %[acc], v249, %[acc]\n"
      "v_add_f32 %[acc], v250, %[acc]\n"
      "v_add_f32 %[acc], v251, %[acc]\n"
      "v_add_f32 %[acc], v252, %[acc]\n"
      "v_add_f32 %[acc], v253, %[acc]\n"
      "v_add_f32 %[acc], v254, %[acc]\n"
      "v_add_f32 %[acc], v255, %[acc]\n"
      "ds_read_b128 v[240:243], %[p] offset:448\n"
      "ds_read_b128 v[244:247], %[p] offset:464\n"
      "ds_read_b128 v[248:251], %[p] offset:480\n"
      "ds_read_b128 v[252:255], %[p] offset:496\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v224, %[acc]\n"
      "v_add_f32 %[acc], v225, %[acc]\n"
      "v_add_f32 %[acc], v226, %[acc]\n"
      "v_add_f32 %[acc], v227, %[acc]\n"
      "v_add_f32 %[acc], v228, %[acc]\n"
      "v_add_f32 %[acc], v229, %[acc]\n"
      "v_add_f32 %[acc], v230, %[acc]\n"
      "v_add_f32 %[acc], v231, %[acc]\n"
      "v_add_f32 %[acc], v232, %[acc]\n"
      "v_add_f32 %[acc], v233, %[acc]\n"
      "v_add_f32 %[acc], v234, %[acc]\n"
      "v_add_f32 %[acc], v235, %[acc]\n"
      "v_add_f32 %[acc], v236, %[acc]\n"
      "v_add_f32 %[acc], v237, %[acc]\n"
      "v_add_f32 %[acc], v238, %[acc]\n"
      "v_add_f32 %[acc], v239, %[acc]\n"
      "ds_read_b128 v[224:227], %[p] offset:512\n"
      "ds_read_b128 v[228:231], %[p] offset:528\n"
      "ds_read_b128 v[232:235], %[p] offset:544\n"
      "ds_read_b128 v[236:239], %[p] offset:560\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v240, %[acc]\n"
      "v_add_f32 %[acc], v241, %[acc]\n"
      "v_add_f32 %[acc], v242, %[acc]\n"
      "v_add_f32 %[acc], v243, %[acc]\n"
      "v_add_f32 %[acc], v244, %[acc]\n"
      "v_add_f32 %[acc], v245, %[acc]\n"
      "v_add_f32 %[acc], v246, %[acc]\n"
      "v_add_f32 %[acc], v247, %[acc]\n"
      "v_add_f32 %[acc], v248, %[acc]\n"
      "v_add_f32 %[acc], v249, %[acc]\n"
      "v_add_f32 %[acc], v250, %[acc]\n"
      "v_add_f32 %[acc], v251, %[acc]\n"
      "v_add_f32 %[acc], v252, %[acc]\n"
      "v_add_f32 %[acc], v253, %[acc]\n"
      "v_add_f32 %[acc], v254, %[acc]\n"
      "v_add_f32 %[acc], v255, %[acc]\n"
      "ds_read_b128 v[240:243], %[p] offset:576\n"
      "ds_read_b128 v[244:247], %[p] offset:592\n"
      "ds_read_b128 v[248:251], %[p] offset:608\n"
      "ds_read_b128 v[252:255], %[p] offset:624\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v224, %[acc]\n"
      "v_add_f32 %[acc], v225, %[acc]\n"
      "v_add_f32 %[acc], v226, %[acc]\n"
      "v_add_f32 %[acc], v227, %[acc]\n"
      "v_add_f32 %[acc], v228, %[acc]\n"
      "v_add_f32 %[acc], v229, %[acc]\n"
      "v_add_f32 %[acc], v230, %[acc]\n"
      "v_add_f32 %[acc], v231, %[acc]\n"
      "v_add_f32 %[acc], v232, %[acc]\n"
      "v_add_f32 %[acc], v233, %[acc]\n"
      "v_add_f32 %[acc], v234, %[acc]\n"
      "v_add_f32 %[acc], v235, %[acc]\n"
      "v_add_f32 %[acc], v236, %[acc]\n"
      "v_add_f32 %[acc], v237, %[acc]\n"
      "v_add_f32 %[acc], v238, %[acc]\n"
      "v_add_f32 %[acc], v239, %[acc]\n"
      "ds_read_b128 v[224:227], %[p] offset:640\n"
      "ds_read_b128 v[228:231], %[p] offset:656\n"
      "ds_read_b128 v[232:235], %[p] offset:672\n"
      "ds_read_b128 v[236:239], %[p] offset:688\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v240, %[acc]\n"
      "v_add_f32 %[acc], v241, %[acc]\n"
      "v_add_f32 %[acc], v242, %[acc]\n"
      "v_add_f32 %[acc], v243, %[acc]\n"
      "v_add_f32 %[acc], v244, %[acc]\n"
      "v_add_f32 %[acc], v245, %[acc]\n"
      "v_add_f32 %[acc], v246, %[acc]\n"
      "v_add_f32 %[acc], v247, %[acc]\n"
      "v_add_f32 %[acc], v248, %[acc]\n"
      "v_add_f32 %[acc], v249, %[acc]\n"
      "v_add_f32 %[acc], v250, %[acc]\n"
      "v_add_f32 %[acc], v251, %[acc]\n"
      "v_add_f32 %[acc], v252, %[acc]\n"
      "v_add_f32 %[acc], v253, %[acc]\n"
      "v_add_f32 %[acc], v254, %[acc]\n"
      "v_add_f32 %[acc], v255, %[acc]\n"
      "ds_read_b128 v[240:243], %[p] offset:704\n"
      "ds_read_b128 v[244:247], %[p] offset:720\n"
      "ds_read_b128 v[248:251], %[p] offset:736\n"
      "ds_read_b128 v[252:255], %[p] offset:752\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v224, %[acc]\n"
      "v_add_f32 %[acc], v225, %[acc]\n"
      "v_add_f32 %[acc], v226, %[acc]\n"
      "v_add_f32 %[acc], v227, %[acc]\n"
      "v_add_f32 %[acc], v228, %[acc]\n"
      "v_add_f32 %[acc], v229, %[acc]\n"
      "v_add_f32 %[acc], v230, %[acc]\n"
      "v_add_f32 %[acc], v231, %[acc]\n"
      "v_add_f32 %[acc], v232, %[acc]\n"
      "v_add_f32 %[acc], v233, %[acc]\n"
      "v_add_f32 %[acc], v234, %[acc]\n"
      "v_add_f32 %[acc], v235, %[acc]\n"
      "v_add_f32 %[acc], v236, %[acc]\n"
      "v_add_f32 %[acc], v237, %[acc]\n"
      "v_add_f32 %[acc], v238, %[acc]\n"
      "v_add_f32 %[acc], v239, %[acc]\n"
      "ds_read_b128 v[224:227], %[p] offset:768\n"
      "ds_read_b128 v[228:231], %[p] offset:784\n"
      "ds_read_b128 v[232:235], %[p] offset:800\n"
      "ds_read_b128 v[236:239], %[p] offset:816\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v240, %[acc]\n"
      "v_add_f32 %[acc], v241, %[acc]\n"
      "v_add_f32 %[acc], v242, %[acc]\n"
      "v_add_f32 %[acc], v243, %[acc]\n"
      "v_add_f32 %[acc], v244, %[acc]\n"
      "v_add_f32 %[acc], v245, %[acc]\n"
      "v_add_f32 %[acc], v246, %[acc]\n"
      "v_add_f32 %[acc], v247, %[acc]\n"
      "v_add_f32 %[acc], v248, %[acc]\n"
      "v_add_f32 %[acc], v249, %[acc]\n"
      "v_add_f32 %[acc], v250, %[acc]\n"
      "v_add_f32 %[acc], v251, %[acc]\n"
      "v_add_f32 %[acc], v252, %[acc]\n"
      "v_add_f32 %[acc], v253, %[acc]\n"
      "v_add_f32 %[acc], v254, %[acc]\n"
      "v_add_f32 %[acc], v255, %[acc]\n"
      "ds_read_b128 v[240:243], %[p] offset:832\n"
      "ds_read_b128 v[244:247], %[p] offset:848\n"
      "ds_read_b128 v[248:251], %[p] offset:864\n"
      "ds_read_b128 v[252:255], %[p] offset:880\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v224, %[acc]\n"
      "v_add_f32 %[acc], v225, %[acc]\n"
      "v_add_f32 %[acc], v226, %[acc]\n"
      "v_add_f32 %[acc], v227, %[acc]\n"
      "v_add_f32 %[acc], v228, %[acc]\n"
      "v_add_f32 %[acc], v229, %[acc]\n"
      "v_add_f32 %[acc], v230, %[acc]\n"
      "v_add_f32 %[acc], v231, %[acc]\n"
      "v_add_f32 %[acc], v232, %[acc]\n"
      "v_add_f32 %[acc], v233, %[acc]\n"
      "v_add_f32 %[acc], v234, %[acc]\n"
      "v_add_f32 %[acc], v235, %[acc]\n"
      "v_add_f32 %[acc], v236, %[acc]\n"
      "v_add_f32 %[acc], v237, %[acc]\n"
      "v_add_f32 %[acc], v238, %[acc]\n"
      "v_add_f32 %[acc], v239, %[acc]\n"
      "ds_read_b128 v[224:227], %[p] offset:896\n"
      "ds_read_b128 v[228:231], %[p] offset:912\n"
      "ds_read_b128 v[232:235], %[p] offset:928\n"
      "ds_read_b128 v[236:239], %[p] offset:944\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v240, %[acc]\n"
      "v_add_f32 %[acc], v241, %[acc]\n"
      "v_add_f32 %[acc], v242, %[acc]\n"
      "v_add_f32 %[acc], v243, %[acc]\n"
      "v_add_f32 %[acc], v244, %[acc]\n"
      "v_add_f32 %[acc], v245, %[acc]\n"
      "v_add_f32 %[acc], v246, %[acc]\n"
      "v_add_f32 %[acc], v247, %[acc]\n"
      "v_add_f32 %[acc], v248, %[acc]\n"
      "v_add_f32 %[acc], v249, %[acc]\n"
      "v_add_f32 %[acc], v250, %[acc]\n"
      "v_add_f32 %[acc], v251, %[acc]\n"
      "v_add_f32 %[acc], v252, %[acc]\n"
      "v_add_f32 %[acc], v253, %[acc]\n"
      "v_add_f32 %[acc], v254, %[acc]\n"
      "v_add_f32 %[acc], v255, %[acc]\n"
      "ds_read_b128 v[240:243], %[p] offset:960\n"
      "ds_read_b128 v[244:247], %[p] offset:976\n"
      "ds_read_b128 v[248:251], %[p] offset:992\n"
      "ds_read_b128 v[252:255], %[p] offset:1008\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v224, %[acc]\n"
      "v_add_f32 %[acc], v225, %[acc]\n"
      "v_add_f32 %[acc], v226, %[acc]\n"
      "v_add_f32 %[acc], v227, %[acc]\n"
      "v_add_f32 %[acc], v228, %[acc]\n"
      "v_add_f32 %[acc], v229, %[acc]\n"
      "v_add_f32 %[acc], v230, %[acc]\n"
      "v_add_f32 %[acc], v231, %[acc]\n"
      "v_add_f32 %[acc], v232, %[acc]\n"
      "v_add_f32 %[acc], v233, %[acc]\n"
      "v_add_f32 %[acc], v234, %[acc]\n"
      "v_add_f32 %[acc], v235, %[acc]\n"
      "v_add_f32 %[acc], v236, %[acc]\n"
      "v_add_f32 %[acc], v237, %[acc]\n"
      "v_add_f32 %[acc], v238, %[acc]\n"
      "v_add_f32 %[acc], v239, %[acc]\n"
      "ds_read_b128 v[224:227], %[p] offset:1024\n"
      "ds_read_b128 v[228:231], %[p] offset:1040\n"
      "ds_read_b128 v[232:235], %[p] offset:1056\n"
      "ds_read_b128 v[236:239], %[p] offset:1072\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v240, %[acc]\n"
      "v_add_f32 %[acc], v241, %[acc]\n"
      "v_add_f32 %[acc], v242, %[acc]\n"
      "v_add_f32 %[acc], v243, %[acc]\n"
      "v_add_f32 %[acc], v244, %[acc]\n"
      "v_add_f32 %[acc], v245, %[acc]\n"
      "v_add_f32 %[acc], v246, %[acc]\n"
      "v_add_f32 %[acc], v247, %[acc]\n"
      "v_add_f32 %[acc], v248, %[acc]\n"
      "v_add_f32 %[acc], v249, %[acc]\n"
      "v_add_f32 %[acc], v250, %[acc]\n"
      "v_add_f32 %[acc], v251, %[acc]\n"
      "v_add_f32 %[acc], v252, %[acc]\n"
      "v_add_f32 %[acc], v253, %[acc]\n"
      "v_add_f32 %[acc], v254, %[acc]\n"
      "v_add_f32 %[acc], v255, %[acc]\n"
      "ds_read_b128 v[240:243], %[p] offset:1088\n"
      "ds_read_b128 v[244:247], %[p] offset:1104\n"
      "ds_read_b128 v[248:251], %[p] offset:1120\n"
      "ds_read_b128 v[252:255], %[p] offset:1136\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v224, %[acc]\n"
      "v_add_f32 %[acc], v225, %[acc]\n"
      "v_add_f32 %[acc], v226, %[acc]\n"
      "v_add_f32 %[acc], v227, %[acc]\n"
      "v_add_f32 %[acc], v228, %[acc]\n"
      "v_add_f32 %[acc], v229, %[acc]\n"
      "v_add_f32 %[acc], v230, %[acc]\n"
      "v_add_f32 %[acc], v231, %[acc]\n"
      "v_add_f32 %[acc], v232, %[acc]\n"
      "v_add_f32 %[acc], v233, %[acc]\n"
      "v_add_f32 %[acc], v234, %[acc]\n"
      "v_add_f32 %[acc], v235, %[acc]\n"
      "v_add_f32 %[acc], v236, %[acc]\n"
      "v_add_f32 %[acc], v237, %[acc]\n"
      "v_add_f32 %[acc], v238, %[acc]\n"
      "v_add_f32 %[acc], v239, %[acc]\n"
      "ds_read_b128 v[224:227], %[p] offset:1152\n"
      "ds_read_b128 v[228:231], %[p] offset:1168\n"
      "ds_read_b128 v[232:235], %[p] offset:1184\n"
      "ds_read_b128 v[236:239], %[p] offset:1200\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v240, %[acc]\n"
      "v_add_f32 %[acc], v241, %[acc]\n"
      "v_add_f32 %[acc], v242, %[acc]\n"
      "v_add_f32 %[acc], v243, %[acc]\n"
      "v_add_f32 %[acc], v244, %[acc]\n"
      "v_add_f32 %[acc], v245, %[acc]\n"
      "v_add_f32 %[acc], v246, %[acc]\n"
      "v_add_f32 %[acc], v247, %[acc]\n"
      "v_add_f32 %[acc], v248, %[acc]\n"
      "v_add_f32 %[acc], v249, %[acc]\n"
      "v_add_f32 %[acc], v250, %[acc]\n"
      "v_add_f32 %[acc], v251, %[acc]\n"
      "v_add_f32 %[acc], v252, %[acc]\n"
      "v_add_f32 %[acc], v253, %[acc]\n"
      "v_add_f32 %[acc], v254, %[acc]\n"
      "v_add_f32 %[acc], v255, %[acc]\n"
      "ds_read_b128 v[240:243], %[p] offset:1216\n"
      "ds_read_b128 v[244:247], %[p] offset:1232\n"
      "ds_read_b128 v[248:251], %[p] offset:1248\n"
      "ds_read_b128 v[252:255], %[p] offset:1264\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v224, %[acc]\n"
      "v_add_f32 %[acc], v225, %[acc]\n"
      "v_add_f32 %[acc], v226, %[acc]\n"
      "v_add_f32 %[acc], v227, %[acc]\n"
      "v_add_f32 %[acc], v228, %[acc]\n"
      "v_add_f32 %[acc], v229, %[acc]\n"
      "v_add_f32 %[acc], v230, %[acc]\n"
      "v_add_f32 %[acc], v231, %[acc]\n"
      "v_add_f32 %[acc], v232, %[acc]\n"
      "v_add_f32 %[acc], v233, %[acc]\n"
      "v_add_f32 %[acc], v234, %[acc]\n"
      "v_add_f32 %[acc], v235, %[acc]\n"
      "v_add_f32 %[acc], v236, %[acc]\n"
      "v_add_f32 %[acc], v237, %[acc]\n"
      "v_add_f32 %[acc], v238, %[acc]\n"
      "v_add_f32 %[acc], v239, %[acc]\n"
      "ds_read_b128 v[224:227], %[p] offset:1280\n"
      "ds_read_b128 v[228:231], %[p] offset:1296\n"
      "ds_read_b128 v[232:235], %[p] offset:1312\n"
      "ds_read_b128 v[236:239], %[p] offset:1328\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v240, %[acc]\n"
      "v_add_f32 %[acc], v241, %[acc]\n"
      "v_add_f32 %[acc], v242, %[acc]\n"
      "v_add_f32 %[acc], v243, %[acc]\n"
      "v_add_f32 %[acc], v244, %[acc]\n"
      "v_add_f32 %[acc], v245, %[acc]\n"
      "v_add_f32 %[acc], v246, %[acc]\n"
      "v_add_f32 %[acc], v247, %[acc]\n"
      "v_add_f32 %[acc], v248, %[acc]\n"
      "v_add_f32 %[acc], v249, %[acc]\n"
      "v_add_f32 %[acc], v250, %[acc]\n"
      "v_add_f32 %[acc], v251, %[acc]\n"
      "v_add_f32 %[acc], v252, %[acc]\n"
      "v_add_f32 %[acc], v253, %[acc]\n"
      "v_add_f32 %[acc], v254, %[acc]\n"
      "v_add_f32 %[acc], v255, %[acc]\n"
      "ds_read_b128 v[240:243], %[p] offset:1344\n"
      "ds_read_b128 v[244:247], %[p] offset:1360\n"
      "ds_read_b128 v[248:251], %[p] offset:1376\n"
      "ds_read_b128 v[252:255], %[p] offset:1392\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v224, %[acc]\n"
      "v_add_f32 %[acc], v225, %[acc]\n"
      "v_add_f32 %[acc], v226, %[acc]\n"
      "v_add_f32 %[acc], v227, %[acc]\n"
      "v_add_f32 %[acc], v228, %[acc]\n"
      "v_add_f32 %[acc], v229, %[acc]\n"
      "v_add_f32 %[acc], v230, %[acc]\n"
      "v_add_f32 %[acc], v231, %[acc]\n"
      "v_add_f32 %[acc], v232, %[acc]\n"
      "v_add_f32 %[acc], v233, %[acc]\n"
      "v_add_f32 %[acc], v234, %[acc]\n"
      "v_add_f32 %[acc], v235, %[acc]\n"
      "v_add_f32 %[acc], v236, %[acc]\n"
      "v_add_f32 %[acc], v237, %[acc]\n"
      "v_add_f32 %[acc], v238, %[acc]\n"
      "v_add_f32 %[acc], v239, %[acc]\n"
      "ds_read_b128 v[224:227], %[p] offset:1408\n"
      "ds_read_b128 v[228:231], %[p] offset:1424\n"
      "ds_read_b128 v[232:235], %[p] offset:1440\n"
      "ds_read_b128 v[236:239], %[p] offset:1456\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v240, %[acc]\n"
      "v_add_f32 %[acc], v241, %[acc]\n"
      "v_add_f32 %[acc], v242, %[acc]\n"
      "v_add_f32 %[acc], v243, %[acc]\n"
      "v_add_f32 %[acc], v244, %[acc]\n"
      "v_add_f32 %[acc], v245, %[acc]\n"
      "v_add_f32 %[acc], v246, %[acc]\n"
      "v_add_f32 %[acc], v247, %[acc]\n"
      "v_add_f32 %[acc], v248, %[acc]\n"
      "v_add_f32 %[acc], v249, %[acc]\n"
      "v_add_f32 %[acc], v250, %[acc]\n"
      "v_add_f32 %[acc], v251, %[acc]\n"
      "v_add_f32 %[acc], v252, %[acc]\n"
      "v_add_f32 %[acc], v253, %[acc]\n"
      "v_add_f32 %[acc], v254, %[acc]\n"
      "v_add_f32 %[acc], v255, %[acc]\n"
      "ds_read_b128 v[240:243], %[p] offset:1472\n"
      "ds_read_b128 v[244:247], %[p] offset:1488\n"
      "ds_read_b128 v[248:251], %[p] offset:1504\n"
      "ds_read_b128 v[252:255], %[p] offset:1520\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v224, %[acc]\n"
      "v_add_f32 %[acc], v225, %[acc]\n"
      "v_add_f32 %[acc], v226, %[acc]\n"
      "v_add_f32 %[acc], v227, %[acc]\n"
      "v_add_f32 %[acc], v228, %[acc]\n"
      "v_add_f32 %[acc], v229, %[acc]\n"
      "v_add_f32 %[acc], v230, %[acc]\n"
      "v_add_f32 %[acc], v231, %[acc]\n"
      "v_add_f32 %[acc], v232, %[acc]\n"
      "v_add_f32 %[acc], v233, %[acc]\n"
      "v_add_f32 %[acc], v234, %[acc]\n"
      "v_add_f32 %[acc], v235, %[acc]\n"
      "v_add_f32 %[acc], v236, %[acc]\n"
      "v_add_f32 %[acc], v237, %[acc]\n"
      "v_add_f32 %[acc], v238, %[acc]\n"
      "v_add_f32 %[acc], v239, %[acc]\n"
      "ds_read_b128 v[224:227], %[p] offset:1536\n"
      "ds_read_b128 v[228:231], %[p] offset:1552\n"
      "ds_read_b128 v[232:235], %[p] offset:1568\n"
      "ds_read_b128 v[236:239], %[p] offset:1584\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v240, %[acc]\n"
      "v_add_f32 %[acc], v241, %[acc]\n"
      "v_add_f32 %[acc], v242, %[acc]\n"
      "v_add_f32 %[acc], v243, %[acc]\n"
      "v_add_f32 %[acc], v244, %[acc]\n"
      "v_add_f32 %[acc], v245, %[acc]\n"
      "v_add_f32 %[acc], v246, %[acc]\n"
      "v_add_f32 %[acc], v247, %[acc]\n"
      "v_add_f32 %[acc], v248, %[acc]\n"
      "v_add_f32 %[acc], v249, %[acc]\n"
      "v_add_f32 %[acc], v250, %[acc]\n"
      "v_add_f32 %[acc], v251, %[acc]\n"
      "v_add_f32 %[acc], v252, %[acc]\n"
      "v_add_f32 %[acc], v253, %[acc]\n"
      "v_add_f32 %[acc], v254, %[acc]\n"
      "v_add_f32 %[acc], v255, %[acc]\n"
      "ds_read_b128 v[240:243], %[p] offset:1600\n"
      "ds_read_b128 v[244:247], %[p] offset:1616\n"
      "ds_read_b128 v[248:251], %[p] offset:1632\n"
      "ds_read_b128 v[252:255], %[p] offset:1648\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v224, %[acc]\n"
      "v_add_f32 %[acc], v225, %[acc]\n"
      "v_add_f32 %[acc], v226, %[acc]\n"
      "v_add_f32 %[acc], v227, %[acc]\n"
      "v_add_f32 %[acc], v228, %[acc]\n"
      "v_add_f32 %[acc], v229, %[acc]\n"
      "v_add_f32 %[acc], v230, %[acc]\n"
      "v_add_f32 %[acc], v231, %[acc]\n"
      "v_add_f32 %[acc], v232, %[acc]\n"
      "v_add_f32 %[acc], v233, %[acc]\n"
      "v_add_f32 %[acc], v234, %[acc]\n"
      "v_add_f32 %[acc], v235, %[acc]\n"
      "v_add_f32 %[acc], v236, %[acc]\n"
      "v_add_f32 %[acc], v237, %[acc]\n"
      "v_add_f32 %[acc], v238, %[acc]\n"
      "v_add_f32 %[acc], v239, %[acc]\n"
      "ds_read_b128 v[224:227], %[p] offset:1664\n"
      "ds_read_b128 v[228:231], %[p] offset:1680\n"
      "ds_read_b128 v[232:235], %[p] offset:1696\n"
      "ds_read_b128 v[236:239], %[p] offset:1712\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v240, %[acc]\n"
      "v_add_f32 %[acc], v241, %[acc]\n"
      "v_add_f32 %[acc], v242, %[acc]\n"
      "v_add_f32 %[acc], v243, %[acc]\n"
      "v_add_f32 %[acc], v244, %[acc]\n"
      "v_add_f32 %[acc], v245, %[acc]\n"
      "v_add_f32 %[acc], v246, %[acc]\n"
      "v_add_f32 %[acc], v247, %[acc]\n"
      "v_add_f32 %[acc], v248, %[acc]\n"
      "v_add_f32 %[acc], v249, %[acc]\n"
      "v_add_f32 %[acc], v250, %[acc]\n"
      "v_add_f32 %[acc], v251, %[acc]\n"
      "v_add_f32 %[acc], v252, %[acc]\n"
      "v_add_f32 %[acc], v253, %[acc]\n"
      "v_add_f32 %[acc], v254, %[acc]\n"
      "v_add_f32 %[acc], v255, %[acc]\n"
      "ds_read_b128 v[240:243], %[p] offset:1728\n"
      "ds_read_b128 v[244:247], %[p] offset:1744\n"
      "ds_read_b128 v[248:251], %[p] offset:1760\n"
      "ds_read_b128 v[252:255], %[p] offset:1776\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v224, %[acc]\n"
      "v_add_f32 %[acc], v225, %[acc]\n"
      "v_add_f32 %[acc], v226, %[acc]\n"
      "v_add_f32 %[acc], v227, %[acc]\n"
      "v_add_f32 %[acc], v228, %[acc]\n"
      "v_add_f32 %[acc], v229, %[acc]\n"
      "v_add_f32 %[acc], v230, %[acc]\n"
      "v_add_f32 %[acc], v231, %[acc]\n"
      "v_add_f32 %[acc], v232, %[acc]\n"
      "v_add_f32 %[acc], v233, %[acc]\n"
      "v_add_f32 %[acc], v234, %[acc]\n"
      "v_add_f32 %[acc], v235, %[acc]\n"
      "v_add_f32 %[acc], v236, %[acc]\n"
      "v_add_f32 %[acc], v237, %[acc]\n"
      "v_add_f32 %[acc], v238, %[acc]\n"
      "v_add_f32 %[acc], v239, %[acc]\n"
      "ds_read_b128 v[224:227], %[p] offset:1792\n"
      "ds_read_b128 v[228:231], %[p] offset:1808\n"
      "ds_read_b128 v[232:235], %[p] offset:1824\n"
      "ds_read_b128 v[236:239], %[p] offset:1840\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v240, %[acc]\n"
      "v_add_f32 %[acc], v241, %[acc]\n"
      "v_add_f32 %[acc], v242, %[acc]\n"
      "v_add_f32 %[acc], v243, %[acc]\n"
      "v_add_f32 %[acc], v244, %[acc]\n"
      "v_add_f32 %[acc], v245, %[acc]\n"
      "v_add_f32 %[acc], v246, %[acc]\n"
      "v_add_f32 %[acc], v247, %[acc]\n"
      "v_add_f32 %[acc], v248, %[acc]\n"
      "v_add_f32 %[acc], v249, %[acc]\n"
      "v_add_f32 %[acc], v250, %[acc]\n"
      "v_add_f32 %[acc], v251, %[acc]\n"
      "v_add_f32 %[acc], v252, %[acc]\n"
      "v_add_f32 %[acc], v253, %[acc]\n"
      "v_add_f32 %[acc], v254, %[acc]\n"
      "v_add_f32 %[acc], v255, %[acc]\n"
      "ds_read_b128 v[240:243], %[p] offset:1856\n"
      "ds_read_b128 v[244:247], %[p] offset:1872\n"
      "ds_read_b128 v[248:251], %[p] offset:1888\n"
      "ds_read_b128 v[252:255], %[p] offset:1904\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v224, %[acc]\n"
      "v_add_f32 %[acc], v225, %[acc]\n"
      "v_add_f32 %[acc], v226, %[acc]\n"
      "v_add_f32 %[acc], v227, %[acc]\n"
      "v_add_f32 %[acc], v228, %[acc]\n"
      "v_add_f32 %[acc], v229, %[acc]\n"
      "v_add_f32 %[acc], v230, %[acc]\n"
      "v_add_f32 %[acc], v231, %[acc]\n"
      "v_add_f32 %[acc], v232, %[acc]\n"
      "v_add_f32 %[acc], v233, %[acc]\n"
      "v_add_f32 %[acc], v234, %[acc]\n"
      "v_add_f32 %[acc], v235, %[acc]\n"
      "v_add_f32 %[acc], v236, %[acc]\n"
      "v_add_f32 %[acc], v237, %[acc]\n"
      "v_add_f32 %[acc], v238, %[acc]\n"
      "v_add_f32 %[acc], v239, %[acc]\n"
      "ds_read_b128 v[224:227], %[p] offset:1920\n"
      "ds_read_b128 v[228:231], %[p] offset:1936\n"
      "ds_read_b128 v[232:235], %[p] offset:1952\n"
      "ds_read_b128 v[236:239], %[p] offset:1968\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v240, %[acc]\n"
      "v_add_f32 %[acc], v241, %[acc]\n"
      "v_add_f32 %[acc], v242, %[acc]\n"
      "v_add_f32 %[acc], v243, %[acc]\n"
      "v_add_f32 %[acc], v244, %[acc]\n"
      "v_add_f32 %[acc], v245, %[acc]\n"
      "v_add_f32 %[acc], v246, %[acc]\n"
      "v_add_f32 %[acc], v247, %[acc]\n"
      "v_add_f32 %[acc], v248, %[acc]\n"
      "v_add_f32 %[acc], v249, %[acc]\n"
      "v_add_f32 %[acc], v250, %[acc]\n"
      "v_add_f32 %[acc], v251, %[acc]\n"
      "v_add_f32 %[acc], v252, %[acc]\n"
      "v_add_f32 %[acc], v253, %[acc]\n"
      "v_add_f32 %[acc], v254, %[acc]\n"
      "v_add_f32 %[acc], v255, %[acc]\n"
      "ds_read_b128 v[240:243], %[p] offset:1984\n"
      "ds_read_b128 v[244:247], %[p] offset:2000\n"
      "ds_read_b128 v[248:251], %[p] offset:2016\n"
      "ds_read_b128 v[252:255], %[p] offset:2032\n"
      "s_waitcnt lgkmcnt(4)\n"
      "v_add_f32 %[acc], v224, %[acc]\n"
      "v_add_f32 %[acc], v225, %[acc]\n"
      "v_add_f32 %[acc], v226, %[acc]\n"
      "v_add_f32 %[acc], v227, %[acc]\n"
      "v_add_f32 %[acc], v228, %[acc]\n"
      "v_add_f32 %[acc], v229, %[acc]\n"
      "v_add_f32 %[acc], v230, %[acc]\n"
      "v_add_f32 %[acc], v231, %[acc]\n"
      "v_add_f32 %[acc], v232, %[acc]\n"
      "v_add_f32 %[acc], v233, %[acc]\n"
      "v_add_f32 %[acc], v234, %[acc]\n"
      "v_add_f32 %[acc], v235, %[acc]\n"
      "v_add_f32 %[acc], v236, %[acc]\n"
      "v_add_f32 %[acc], v237, %[acc]\n"
      "v_add_f32 %[acc], v238, %[acc]\n"
      "v_add_f32 %[acc], v239, %[acc]\n"
      "s_waitcnt lgkmcnt(0)\n"
      "v_add_f32 %[acc], v240, %[acc]\n"
      "v_add_f32 %[acc], v241, %[acc]\n"
      "v_add_f32 %[acc], v242, %[acc]\n"
      "v_add_f32 %[acc], v243, %[acc]\n"
      "v_add_f32 %[acc], v244, %[acc]\n"
      "v_add_f32 %[acc], v245, %[acc]\n"
      "v_add_f32 %[acc], v246, %[acc]\n"
      "v_add_f32 %[acc], v247, %[acc]\n"
      "v_add_f32 %[acc], v248, %[acc]\n"
      "v_add_f32 %[acc], v249, %[acc]\n"
      "v_add_f32 %[acc], v250, %[acc]\n"
      "v_add_f32 %[acc], v251, %[acc]\n"
      "v_add_f32 %[acc], v252, %[acc]\n"
      "v_add_f32 %[acc], v253, %[acc]\n"
      "v_add_f32 %[acc], v254, %[acc]\n"
      "v_add_f32 %[acc], v255, %[acc]\n"
      : [acc] "+v"(acc)
      : [p] "v"(p)
      : "v224", "v225", "v226", "v227", "v228", "v229", "v230", "v231", "v232", "v233", "v234", "v235", "v236", "v237", "v238", "v239", "v240", "v241", "v242", "v243", "v244", "v245", "v246", "v247", "v248", "v249", "v250", "v251", "v252", "v253", "v254", "v255", "memory");
    return acc;
  } else {
#pragma unroll 16
    for (int c = 0; c < N; c += 4) {
      const f32x4 q = *reinterpret_cast<const f32x4 *>(rp + c);
      acc = q.x + acc;
      acc = q.y + acc;
      acc = q.z + acc;
      acc = q.w + acc;
    }
    return acc;
  }
}

// Serial-order fp32 sums of the RB*RPW rows of a block, bit-identical to the
// reference CPU lowering's `for c in 0..C-1: acc = x[c] + acc` starting from
// `init` (convert-linalg-to-loops on linalg.reduce {arith.addf}).
// The rows' values (produced lazily by `val(e)`, e = rr*EPL + element) are
// staged through a double-buffered LDS ring in CHUNK-column pieces; lane t of
// wave 0 (t < RB*RPW) walks row t of the block in column order.  While wave 0
// folds chunk k, the other waves write chunk k+1 into the other buffer, so one
// barrier per chunk suffices.  The sums are broadcast back to every thread of
// each row group through `bcast` (RB*RPW floats).  `lds` holds
// 2 * RB*RPW * (CHUNK + 4) floats.
//
// `prefetch(k)` issues the global loads of LDS chunk k; it is called for chunk
// k + LA at the start of step k, so each CU keeps only LA chunks of loads in
// flight and the first chunks are not queued behind the whole tensor.
template <int TR, int RB, int RPW, int VEC, int EPL, int CHUNK, int LA, typename F, typename PF>
__device__ __forceinline__ void row_sum_ordered(F val, PF prefetch, const float (&init)[RPW], float (&out)[RPW], float *lds,
                                                float *bcast, int rloc, int lt, int64_t C) {
  constexpr int SPAN = TR * VEC;
  constexpr int JPC = CHUNK / SPAN;       // vector chunks per LDS chunk
  constexpr int NCH = EPL / VEC;          // vector chunks per row per lane
  constexpr int NK = (NCH + JPC - 1) / JPC;
  constexpr int STRIDE = CHUNK + 4;
  constexpr int NROWS = RB * RPW;
  static_assert(NROWS <= 64, "one chain lane per row, all in wave 0");
  const int tid = threadIdx.x;
  const bool wave0 = tid < 64;
  auto write = [&](int k, float *buf) {
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr)
#pragma unroll
      for (int jj = 0; jj < JPC; ++jj) {
        const int j = k * JPC + jj;
        if (j < NCH) {
          float *dst = buf + (rloc * RPW + rr) * STRIDE + jj * SPAN + lt * VEC;
#pragma unroll
          for (int v = 0; v < VEC; ++v) dst[v] = val(rr * EPL + j * VEC + v);
        }
      }
  };
  if (lt == 0)
#pragma unroll
    for (int rr = 0; rr < RPW; ++rr) bcast[rloc * RPW + rr] = init[rr];
  write(0, lds);
  __syncthreads();
  float acc = tid < NROWS ? bcast[tid] : 0.0f;
  // fully unrolled: every lane's element index stays a compile-time constant,
  // so the row values stay in VGPRs
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    if (k + LA < NK) prefetch(k + LA);
    float *cur = lds + (k & 1) * NROWS * STRIDE;
    float *nxt = lds + ((k + 1) & 1) * NROWS * STRIDE;
    if (k + 1 < NK && !wave0) write(k + 1, nxt);
    if (tid < NROWS) {
      const float *rp = cur + tid * STRIDE;
      const int64_t cbase = (int64_t)k * CHUNK;
      const int n = (int)((C - cbase) < CHUNK ? (C - cbase) : CHUNK);
      if (n == CHUNK) {
        acc = lds_chain_sum<CHUNK>(rp, acc);
      } else {
        for (int c = 0; c < n; ++c) acc = rp[c] + acc;
      }
    }
    if (k + 1 < NK && wave0) write(k + 1, nxt);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0); // keep each chunk's conversions local to its step
  }
  if (tid < NROWS) bcast[tid] = acc;
  __syncthreads();
#pragma unroll
  for (int rr = 0; rr < RPW; ++rr) out[rr] = bcast[rloc * RPW + rr];
}

} // namespace hf

__device__ __forceinline__ int64_t hf_floordiv(int64_t a, int64_t b) {
  if (b == 0) return 0;
  int64_t q = a / b;
  if ((a % b != 0) && ((a < 0) != (b < 0))) --q;
  return q;
}
__device__ __forceinline__ int64_t hf_ceildiv(int64_t a, int64_t b) {
  if (b == 0) return 0;
  int64_t q = a / b;
  if ((a % b != 0) && ((a < 0) == (b < 0))) ++q;
  return q;
}
