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
#define HF_ADD(r) "v_add_f32 %[acc], v" #r ", %[acc]\n"
#define HF_ADD16_A HF_ADD(224) HF_ADD(225) HF_ADD(226) HF_ADD(227) HF_ADD(228) HF_ADD(229) HF_ADD(230) HF_ADD(231) \
  HF_ADD(232) HF_ADD(233) HF_ADD(234) HF_ADD(235) HF_ADD(236) HF_ADD(237) HF_ADD(238) HF_ADD(239)
#define HF_ADD16_B HF_ADD(240) HF_ADD(241) HF_ADD(242) HF_ADD(243) HF_ADD(244) HF_ADD(245) HF_ADD(246) HF_ADD(247) \
  HF_ADD(248) HF_ADD(249) HF_ADD(250) HF_ADD(251) HF_ADD(252) HF_ADD(253) HF_ADD(254) HF_ADD(255)
#define HF_RD(lo, hi, off) "ds_read_b128 v[" #lo ":" #hi "], %[p] offset:" #off "\n"
// group g's 16 floats (bytes 64g .. 64g+63) into buffer A (v224-v239) or B (v240-v255)
#define HF_RD_A(o0, o1, o2, o3) HF_RD(224, 227, o0) HF_RD(228, 231, o1) HF_RD(232, 235, o2) HF_RD(236, 239, o3)
#define HF_RD_B(o0, o1, o2, o3) HF_RD(240, 243, o0) HF_RD(244, 247, o1) HF_RD(248, 251, o2) HF_RD(252, 255, o3)
#define HF_W4 "s_waitcnt lgkmcnt(4)\n" // the older group has landed; the newer stays in flight
    asm volatile(
      HF_RD_A(0, 16, 32, 48) HF_RD_B(64, 80, 96, 112)
      HF_W4 HF_ADD16_A HF_RD_A(128, 144, 160, 176) // group 0; read group 2
      HF_W4 HF_ADD16_B HF_RD_B(192, 208, 224, 240) // group 1; read group 3
      HF_W4 HF_ADD16_A HF_RD_A(256, 272, 288, 304) // group 2; read group 4
      HF_W4 HF_ADD16_B HF_RD_B(320, 336, 352, 368) // group 3; read group 5
      HF_W4 HF_ADD16_A HF_RD_A(384, 400, 416, 432) // group 4; read group 6
      HF_W4 HF_ADD16_B HF_RD_B(448, 464, 480, 496) // group 5; read group 7
      HF_W4 HF_ADD16_A HF_RD_A(512, 528, 544, 560) // group 6; read group 8
      HF_W4 HF_ADD16_B HF_RD_B(576, 592, 608, 624) // group 7; read group 9
      HF_W4 HF_ADD16_A HF_RD_A(640, 656, 672, 688) // group 8; read group 10
      HF_W4 HF_ADD16_B HF_RD_B(704, 720, 736, 752) // group 9; read group 11
      HF_W4 HF_ADD16_A HF_RD_A(768, 784, 800, 816) // group 10; read group 12
      HF_W4 HF_ADD16_B HF_RD_B(832, 848, 864, 880) // group 11; read group 13
      HF_W4 HF_ADD16_A HF_RD_A(896, 912, 928, 944) // group 12; read group 14
      HF_W4 HF_ADD16_B HF_RD_B(960, 976, 992, 1008) // group 13; read group 15
      HF_W4 HF_ADD16_A HF_RD_A(1024, 1040, 1056, 1072) // group 14; read group 16
      HF_W4 HF_ADD16_B HF_RD_B(1088, 1104, 1120, 1136) // group 15; read group 17
      HF_W4 HF_ADD16_A HF_RD_A(1152, 1168, 1184, 1200) // group 16; read group 18
      HF_W4 HF_ADD16_B HF_RD_B(1216, 1232, 1248, 1264) // group 17; read group 19
      HF_W4 HF_ADD16_A HF_RD_A(1280, 1296, 1312, 1328) // group 18; read group 20
      HF_W4 HF_ADD16_B HF_RD_B(1344, 1360, 1376, 1392) // group 19; read group 21
      HF_W4 HF_ADD16_A HF_RD_A(1408, 1424, 1440, 1456) // group 20; read group 22
      HF_W4 HF_ADD16_B HF_RD_B(1472, 1488, 1504, 1520) // group 21; read group 23
      HF_W4 HF_ADD16_A HF_RD_A(1536, 1552, 1568, 1584) // group 22; read group 24
      HF_W4 HF_ADD16_B HF_RD_B(1600, 1616, 1632, 1648) // group 23; read group 25
      HF_W4 HF_ADD16_A HF_RD_A(1664, 1680, 1696, 1712) // group 24; read group 26
      HF_W4 HF_ADD16_B HF_RD_B(1728, 1744, 1760, 1776) // group 25; read group 27
      HF_W4 HF_ADD16_A HF_RD_A(1792, 1808, 1824, 1840) // group 26; read group 28
      HF_W4 HF_ADD16_B HF_RD_B(1856, 1872, 1888, 1904) // group 27; read group 29
      HF_W4 HF_ADD16_A HF_RD_A(1920, 1936, 1952, 1968) // group 28; read group 30
      HF_W4 HF_ADD16_B HF_RD_B(1984, 2000, 2016, 2032) // group 29; read group 31
      HF_W4 HF_ADD16_A                                            // group 30
      "s_waitcnt lgkmcnt(0)\n" HF_ADD16_B                          // group 31
      : [acc] "+v"(acc)
      : [p] "v"(p)
      : "v224", "v225", "v226", "v227", "v228", "v229", "v230", "v231", "v232", "v233", "v234", "v235", "v236", "v237", "v238", "v239", "v240", "v241", "v242", "v243", "v244", "v245", "v246", "v247", "v248", "v249", "v250", "v251", "v252", "v253", "v254", "v255", "memory");
#undef HF_ADD
#undef HF_ADD16_A
#undef HF_ADD16_B
#undef HF_RD
#undef HF_RD_A
#undef HF_RD_B
#undef HF_W4
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
