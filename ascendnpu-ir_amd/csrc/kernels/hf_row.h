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
// The dependent adds run at the VALU latency; to keep LDS latency off that
// path, PF ds_read_b128 are kept in flight with explicit lgkmcnt waits (the
// compiler would otherwise wait for each read right after issuing it when
// registers are scarce).  Each wait names the register it guards as an
// in/out operand, so the adds that consume it cannot move above the wait, and
// each refill names the running sum, so it cannot move above those adds.
// Serial fold of N floats of one LDS row into acc, left to right.  Plain
// code on purpose: with a 16-read unroll the compiler keeps enough
// ds_read_b128 in flight to hide their latency behind the dependent adds
// (measured on gfx950: 7.3-7.7 cycles per add, the v_add_f32 dependency
// latency), while hand-placed s_waitcnt variants ran at 12-14 cycles.
template <int N>
__device__ __forceinline__ float lds_chain_sum(const float *rp, float acc) {
  static_assert(N % 64 == 0, "chunk must be a multiple of 64 floats");
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
