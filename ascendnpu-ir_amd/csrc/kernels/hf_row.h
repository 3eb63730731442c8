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

template <typename T, int VEC, int NCH, int TR, bool MASKED>
__device__ __forceinline__ void row_load(const T *__restrict__ rowp, int lt, int64_t C, T (&out)[VEC * NCH]) {
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

template <typename T, int VEC, int NCH, int TR, bool MASKED>
__device__ __forceinline__ void row_store(T *__restrict__ rowp, int lt, int64_t C, const T (&in)[VEC * NCH]) {
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

// Serial-order fp32 sum of a row, bit-identical to the reference CPU
// lowering's `for c in 0..C-1: acc = x[c] + acc` starting from `init`
// (convert-linalg-to-loops on linalg.reduce {arith.addf}).  The row's values
// are staged through LDS in CHUNK-column pieces; lane r < RB of the block
// (one lane per row) walks its row in column order.  The result is broadcast
// back to every thread of the row.
template <int TR, int RB, int VEC, int EPL, int CHUNK>
__device__ __forceinline__ float row_sum_ordered(const float (&x)[EPL], float init, float *lds, float *bcast, int rloc,
                                                 int lt, int64_t C) {
  constexpr int SPAN = TR * VEC;
  constexpr int JPC = CHUNK / SPAN; // vector chunks per LDS chunk
  constexpr int NCH = EPL / VEC;
  constexpr int STRIDE = CHUNK + 4;
  static_assert(NCH % JPC == 0, "chunking must tile the row");
  const int tid = threadIdx.x;
  float acc = init;
#pragma unroll
  for (int k = 0; k < NCH / JPC; ++k) {
#pragma unroll
    for (int jj = 0; jj < JPC; ++jj)
#pragma unroll
      for (int v = 0; v < VEC; ++v)
        lds[rloc * STRIDE + jj * SPAN + lt * VEC + v] = x[(k * JPC + jj) * VEC + v];
    __syncthreads();
    if (tid < RB) {
      const float *rp = lds + tid * STRIDE;
      const int64_t cbase = (int64_t)k * CHUNK;
      const int n = (int)((C - cbase) < CHUNK ? (C - cbase) : CHUNK);
      if (n == CHUNK) {
#pragma unroll 8
        for (int c = 0; c < CHUNK; c += 4) {
          const float4 q = *reinterpret_cast<const float4 *>(rp + c);
          acc = q.x + acc;
          acc = q.y + acc;
          acc = q.z + acc;
          acc = q.w + acc;
        }
      } else {
        for (int c = 0; c < n; ++c) acc = rp[c] + acc;
      }
    }
    __syncthreads();
  }
  if (tid < RB) bcast[tid] = acc;
  __syncthreads();
  return bcast[rloc];
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
