// RMSNorm + dynamic per-row int8 quantisation on CDNA4, one wavefront per
// row, with the reference's serial fp32 sum of squares computed exactly but
// without a 4096-long dependent add chain.
//
// Group (compile-rms-norm-fp32-split-n.mlir:5-47 followed by the dynamic
// quantisation ops, LAST_AXIS_PBR):
//   xf = extf(x); ss = fold_k RN(ss + RN(xf_k^2)) from s0 (serial, k = 0..C-1);
//   inv = 1 / sqrt(ss / K + eps); y = RN(RN(xf * inv) * gammaf);
//   amax = maximumf over |y| from a0; scale = amax / QD;
//   q = (int8) max(min(rint(y / scale), HI), LO).
//
// Exact serial sum.  Every addend x^2 of a bf16 x is exact in f32 and >= 0,
// so the running sum never decreases.  While the running sum s stays inside
// one binade [2^p, 2^(p+1)), each step is s' = s + (x^2 rounded to the binade's
// grid u = 2^(p-23)), ties to even: in units of u, n' = n + d(n & 1).  A run of
// steps inside one binade is therefore the map n -> n + D[n & 1], fixed by two
// values; runs compose (f then g: D[b] = Df[b] + Dg[b ^ (Df[b] & 1)]).  The
// kernel:
//   1. each lane owns C/64 consecutive elements of the row (the row lands in
//      LDS by DMA, prefetched one row ahead, in a line-swizzled order that
//      keeps the DMA reads coalesced and the segment reads free of bank
//      conflicts), split into sub-segments of 16;
//   2. an approximate prefix (fp32 partial sums and a wave scan) predicts the
//      binade p of every sub-segment; sub-segments whose prediction is not
//      clear by a 2^-10 margin are marked dirty;
//   3. for each clean sub-segment two candidate chains, started at 2^p (n = 0)
//      and 2^p + u (n = 1), give D[0] and D[1]: fmaf(x, x, c) = RN(x^2 + c)
//      because x^2 is exact (for |x| < 2^-63 the square is below half an ulp
//      of c >= 2^-60 either way);
//   4. runs (maximal sequences of clean sub-segments of one binade, in row
//      order) compose inside the lane, then across lanes with a segmented
//      scan over runs of whole lanes; a lane keeps an event per run that
//      ends in it and per dirty sub-segment;
//   5. lane 0's elements take their serial steps from s0 ahead of the rest;
//      a wave-uniform stitch walks the other lanes' events: a run applies when the
//      exact running sum lies in its binade and the result stays below
//      2^(p+1) (the addends are >= 0, so every intermediate value is inside);
//      a dirty sub-segment takes its 16 serial steps; if a run does not
//      apply (a mispredicted binade), the row is walked again sub-segment by
//      sub-segment.
//   The result is the bit pattern of the serial sum for every input,
//   including NaN and infinity (which always take the serial steps).
// Quantisation: y stays in registers; the row maximum is a wave reduction;
// the int8 codes go through a bracketed fast path (exact recomputation of
// near-tie words), a row whose Guard reports an unsafe magnitude is
// recomputed with IEEE division, and the codes leave as whole lines.
#pragma once
#include "hf_ops.h"

namespace hf {

typedef unsigned rq_u4 __attribute__((ext_vector_type(4)));

// n -> n + D[n & 1] inside one binade (units of its ulp)
struct BandFn {
  int32_t d0, d1;
};
__device__ __forceinline__ int32_t band_pick(int32_t d, int32_t odd, int32_t even) {
  // odd if d is odd, else even: a bit-field insert under the mask -(d & 1)
  int32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(__builtin_amdgcn_sbfe(d, 0, 1)), "v"(odd), "v"(even));
  return r;
}
__device__ __forceinline__ BandFn band_compose(BandFn f, BandFn g) {
  BandFn h;
  h.d0 = f.d0 + band_pick(f.d0, g.d1, g.d0);
  h.d1 = f.d1 + band_pick(f.d1, g.d0, g.d1);
  return h;
}

// ---- wave64 DPP primitives (gfx9 DPP: row shifts, row broadcasts, wave shifts)
template <int CTRL, int ROWMASK = 0xf>
__device__ __forceinline__ int dpp(int old, int v) {
  return __builtin_amdgcn_update_dpp(old, v, CTRL, ROWMASK, 0xf, false);
}
constexpr int DPP_ROW_SHR1 = 0x111, DPP_ROW_SHR2 = 0x112, DPP_ROW_SHR4 = 0x114, DPP_ROW_SHR8 = 0x118;
constexpr int DPP_ROW_BCAST15 = 0x142, DPP_ROW_BCAST31 = 0x143, DPP_WAVE_SHR1 = 0x138, DPP_WAVE_SHL1 = 0x130;

// inclusive prefix sum over the 64 lanes (f32, any association: approximate)
__device__ __forceinline__ float wave_scan_add(float v, int lane) {
  const int l16 = lane & 15;
  float t;
  t = __int_as_float(dpp<DPP_ROW_SHR1>(0, __float_as_int(v))); if (l16 >= 1) v += t;
  t = __int_as_float(dpp<DPP_ROW_SHR2>(0, __float_as_int(v))); if (l16 >= 2) v += t;
  t = __int_as_float(dpp<DPP_ROW_SHR4>(0, __float_as_int(v))); if (l16 >= 4) v += t;
  t = __int_as_float(dpp<DPP_ROW_SHR8>(0, __float_as_int(v))); if (l16 >= 8) v += t;
  t = __int_as_float(dpp<DPP_ROW_BCAST15, 0xa>(0, __float_as_int(v))); if (lane & 16) v += t;
  t = __int_as_float(dpp<DPP_ROW_BCAST31, 0xc>(0, __float_as_int(v))); if (lane >= 32) v += t;
  return v;
}

// NaN-propagating maximum over the 64 lanes, returned uniform
__device__ __forceinline__ float wave_max(float v) {
  v = maximumf(v, __int_as_float(dpp<DPP_ROW_SHR1>(__float_as_int(v), __float_as_int(v))));
  v = maximumf(v, __int_as_float(dpp<DPP_ROW_SHR2>(__float_as_int(v), __float_as_int(v))));
  v = maximumf(v, __int_as_float(dpp<DPP_ROW_SHR4>(__float_as_int(v), __float_as_int(v))));
  v = maximumf(v, __int_as_float(dpp<DPP_ROW_SHR8>(__float_as_int(v), __float_as_int(v))));
  v = maximumf(v, __int_as_float(dpp<DPP_ROW_BCAST15, 0xa>(__float_as_int(v), __float_as_int(v))));
  v = maximumf(v, __int_as_float(dpp<DPP_ROW_BCAST31, 0xc>(__float_as_int(v), __float_as_int(v))));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Segmented inclusive composition scan over the lanes: lane j ends with the
// composition of lanes start..j (start <= j: the head of j's run).
__device__ __forceinline__ BandFn wave_seg_compose(BandFn g, int start, int lane) {
  const int l16 = lane & 15, row0 = lane & ~15;
#define HF_SEG_STEP(CTRL, MASK, COND)                                                                 \
  {                                                                                                   \
    const BandFn pv = {dpp<CTRL, MASK>(g.d0, g.d0), dpp<CTRL, MASK>(g.d1, g.d1)};                     \
    const BandFn cg = band_compose(pv, g);                                                            \
    const bool c_ = (COND);                                                                           \
    g.d0 = c_ ? cg.d0 : g.d0;                                                                         \
    g.d1 = c_ ? cg.d1 : g.d1;                                                                         \
  }
  HF_SEG_STEP(DPP_ROW_SHR1, 0xf, l16 >= 1 && lane - 1 >= start)
  HF_SEG_STEP(DPP_ROW_SHR2, 0xf, l16 >= 2 && lane - 2 >= start)
  HF_SEG_STEP(DPP_ROW_SHR4, 0xf, l16 >= 4 && lane - 4 >= start)
  HF_SEG_STEP(DPP_ROW_SHR8, 0xf, l16 >= 8 && lane - 8 >= start)
  HF_SEG_STEP(DPP_ROW_BCAST15, 0xa, (lane & 16) && start <= row0 - 1)
  HF_SEG_STEP(DPP_ROW_BCAST31, 0xc, lane >= 32 && start <= 31)
#undef HF_SEG_STEP
  return g;
}

// An item of the stitch: a binade map packed in two words,
//   w0 = d0 | (p + 127) << 23 | valid << 31,  w1 = d1
// (p + 127 in [67, 247]; d0, d1 < 2^23).
__device__ __forceinline__ uint32_t band_pack(int p, int32_t d0, bool valid) {
  return (uint32_t)d0 | ((uint32_t)(p + 127) << 23) | (valid ? 0x80000000u : 0u);
}
// applies a packed map; false when s is outside its binade or leaves it
__device__ __forceinline__ bool band_apply_packed(uint32_t &s, uint32_t w0, uint32_t w1) {
  const uint32_t lo = w0 & 0x7f800000u, hi = lo + (1u << 23);
  const uint32_t ns = s + ((s & 1u) ? w1 : (w0 & 0x7fffffu));
  const bool ok = (w0 >> 31) && s >= lo && ns < hi;
  s = ok ? ns : s;
  return ok;
}

// 16 serial steps s = RN(s + RN(x_k^2)) over lane j's elements x[0..15] (every
// lane runs its own; lane j's result is returned).  From s >= 2^-100 on, one
// FMA per step is the same: x^2 is exact unless |x| < 2^-63, and then it is
// below half an ulp of s on both paths.
__device__ __forceinline__ uint32_t serial16(uint32_t s, const float *x, int j) {
  float sf = __uint_as_float(s);
  if (s >= 0x0d800000u && s <= 0x7f800000u) { // [2^-100, inf]
#pragma unroll
    for (int k = 0; k < 16; ++k) sf = __builtin_fmaf(x[k], x[k], sf);
  } else {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      float xk = x[k];
      asm volatile("" : "+v"(xk)); // squared here, not hoisted out of the stitch
      const float sq = xk * xk;
      sf = sf + sq;
    }
  }
  return (uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(sf), j);
}

// int8 codes of four quotients a_i / b, as quant8x4 but without tracking the
// clamp bounds: for callers whose quotients cannot reach them (|a_i| <= |b| * QD
// with the clamps outside [-QD, QD]) and whose rows with a non-finite maximum
// take the exact path.
__device__ __forceinline__ uint32_t quant8x4_inner(const float (&a)[4], float b, float r, Guard &g) {
  constexpr float D = 0x1p-15f;
  uint32_t wl = 0, wh = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    wl = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_fmaf(a[i], r, 128.0f - D), i, wl);
    wh = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_fmaf(a[i], r, 128.0f + D), i, wh);
  }
  uint32_t w = wl ^ 0x80808080u;
  if (__builtin_expect(wl != wh, 0)) {
    w = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float q = rint_div(a[i], b, r, g, kFast{});
      w |= ((uint32_t)(int32_t)q & 0xFFu) << (8 * i);
    }
  }
  return w;
}

// a wave-uniform value the compiler cannot prove uniform, moved to SGPRs
__device__ __forceinline__ int64_t uniform_i64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

template <int C, int LO, int HI, int WPB>
__device__ __forceinline__ void rmsq_rows(const uint16_t *__restrict__ x, const uint16_t *__restrict__ gamma,
                                          int8_t *__restrict__ q, float *__restrict__ scale, int64_t R, float s0,
                                          float K, float eps, float a0, float qd, float *dbg = nullptr) {
  static_assert(C == 1024 || C == 2048 || C == 4096, "rows of 1024, 2048 or 4096 elements");
  constexpr int SEG = C / 64;      // elements per lane
  constexpr int NG = SEG / 8;      // 16-byte granules per lane
  constexpr int NS = SEG / 16;     // sub-segments per lane
  __shared__ rq_u4 lds_all[WPB][C / 8];
  const int lane0 = threadIdx.x & 63;
  rq_u4 *lds = lds_all[threadIdx.x / 64];
  // rows in rounds of W = grid * WPB: in a full round, wave w of workgroup b
  // takes row b WPB + w of it; the last, partial round of Rl rows is split
  // as evenly: workgroup b takes PL = ceil(Rl / grid) of its rows, on its
  // first PL waves (with one workgroup per CU, every SIMD gets the same
  // number of rows to within one, and the rows in flight stay together)
  const int64_t W = (int64_t)gridDim.x * WPB;
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / 64)); // wave-uniform
  const int64_t lastBase = (R / W) * W, PL = (R - lastBase + gridDim.x - 1) / gridDim.x;
  auto rowOf = [&](int64_t base) -> int64_t {
    if (base < lastBase) return base + (int64_t)blockIdx.x * WPB + wv;
    return wv < PL ? base + (int64_t)blockIdx.x * PL + wv : R;
  };
  int64_t base = 0;
  int64_t row = rowOf(0);
  // gamma as f32 in LDS for the workgroup (lane j's 4-float groups at
  // stride 64 so that the reads are free of bank conflicts), read where used
  __shared__ float4 lds_gamma[C / 4];
  for (int i = threadIdx.x; i < C / 4; i += WPB * 64) {
    const uint2 w = reinterpret_cast<const uint2 *>(gamma)[i]; // columns 4i .. 4i+3
    const int j = i / (SEG / 4), g4 = i % (SEG / 4);
    lds_gamma[g4 * 64 + j] = make_float4(__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u),
                                         __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xffff0000u));
  }
  __syncthreads();
  // row DMA straight into this wave's LDS row buffer.  Granule G (16 bytes,
  // columns 8G .. 8G+7) of the row sits at slot G ^ ((G >> 4) & 7): a
  // permutation inside every 128-byte line, so DMA instruction k, lane l
  // fills slot 64k + l from one line per eight lanes (coalesced), and lane j's
  // granule g (G = NG*j + g) is read with the 64 lanes spread over the banks.
  // Slot 64k + l holds G = 64k + 8(l/8) + ((l % 8) ^ ((4k + l/16) & 7)); its
  // byte offset is 1024k + off[k & 1] with off[1] = off[0] ^ 64.
  const uint32_t ldsBase = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
  const uint32_t dmaOff0 = 128u * (lane0 / 8) + 16u * ((lane0 % 8) ^ (lane0 / 16)), dmaOff1 = dmaOff0 ^ 64u;
  const rq_u4 *rdPtr[NG];
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    const uint32_t G = NG * lane0 + g;
    rdPtr[g] = lds + (G ^ ((G >> 4) & 7u));
  }
  auto issueRow = [&](int64_t r) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); // this wave's reads of the buffer are done
    const uint16_t *rowp = x + uniform_i64(r) * C;
#pragma unroll
    for (int k = 0; k < NG; ++k) {
      asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"((k & 1) ? dmaOff1 : dmaOff0),
                   "s"(rowp + 512 * k), "s"(ldsBase + 1024u * k)
                   : "memory");
    }
  };
  // staggered start: the second wave on each SIMD (w / 4 = 1) issues its
  // first row C/2 cycles late and the third (which has one row fewer) 2C
  // cycles late, so that the first waves' rows arrive without the whole
  // grid's first rows competing with them and work starts sooner
  if (wv / 4 == 1) __builtin_amdgcn_s_sleep(C / 128); // 64 cycles a unit
  if (wv / 4 == 2) {
    __builtin_amdgcn_s_sleep(C / 64);
    __builtin_amdgcn_s_sleep(C / 64);
  }
  if (row < R) issueRow(row);
  for (; row < R; base += W, row = rowOf(base)) {
    const int lane = lane0;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); // the row's DMA has landed
    __builtin_amdgcn_wave_barrier();
    rq_u4 seg[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) seg[g] = *rdPtr[g];
    // prefetch the next row into the buffer once these reads are done
    const int64_t next = rowOf(base + W);
    if (next < R) issueRow(next);

    // ---- 2. approximate prefix: sub-segment sums and a wave scan
    float xf[SEG];
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xf[8 * g + 2 * i] = __uint_as_float(seg[g][i] << 16);
        xf[8 * g + 2 * i + 1] = __uint_as_float(seg[g][i] & 0xffff0000u);
      }
    float a[NS];
    float tot = 0.0f;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      float e0 = 0.0f, e1 = 0.0f; // two chains: half the latency
#pragma unroll
      for (int k = 16 * s; k < 16 * s + 16; k += 2) {
        e0 = __builtin_fmaf(xf[k], xf[k], e0);
        e1 = __builtin_fmaf(xf[k + 1], xf[k + 1], e1);
      }
      a[s] = e0 + e1;
      tot += a[s];
    }
    const float incl = wave_scan_add(tot, lane);
    float ps = s0 + (incl - tot);
    // ---- 3. per sub-segment (item): binade prediction and candidate chains
    int kt[NS];          // item key: its binade if clean, else unique
    uint32_t w0[NS], w1[NS];
#pragma unroll
    for (int t = 0; t < NS; ++t) {
      // predicted binade: the biased exponent of the approximate start and
      // end agree (2^-10 margin), within [2^-60, 2^120]
      const uint32_t elo = __float_as_uint(ps * (1.0f - 0x1p-10f)) >> 23;
      ps += a[t];
      const uint32_t ehi = __float_as_uint(ps * (1.0f + 0x1p-10f)) >> 23;
      bool clean = elo == ehi && elo - 67u <= 180u;
      const uint32_t base = (clean ? elo : 127u) << 23;
      float c0 = __uint_as_float(base), c1 = __uint_as_float(base + 1u);
#pragma unroll
      for (int k = 16 * t; k < 16 * t + 16; ++k) {
        c0 = __builtin_fmaf(xf[k], xf[k], c0);
        c1 = __builtin_fmaf(xf[k], xf[k], c1);
      }
      const uint32_t d0 = __float_as_uint(c0) - base, d1 = __float_as_uint(c1) - base - 1u;
      clean = clean && (d0 | d1) < (1u << 23);
      kt[t] = clean ? (int)elo - 127 : -1000 - NS * lane - t;
      w0[t] = d0 | base | (clean ? 0x80000000u : 0u); // band_pack(p, d0, clean)
      w1[t] = d1;
    }
    // lane 0's elements serially from s0, the one start known before the
    // stitch (the running sum crosses a binade every few elements there, so
    // its sub-segments are mostly dirty; as a chain of its own the steps
    // overlap the work below instead of lengthening the stitch): every lane
    // runs the steps over its own elements, lane 0's result is kept
    uint32_t p0 = __float_as_uint(s0);
#pragma unroll
    for (int t = 0; t < NS; ++t) p0 = serial16(p0, &xf[16 * t], 0);
    // ---- 4. runs: maximal sequences of clean items of one binade, in row
    //         order.  Q[t] composes the run that ends at item t from its start
    //         in this lane; a segmented scan over the lanes composes the runs
    //         that pass through whole lanes.
    BandFn Q[NS];
    Q[0] = {(int32_t)(w0[0] & 0x7fffffu), (int32_t)w1[0]};
#pragma unroll
    for (int t = 1; t < NS; ++t) {
      const BandFn f = {(int32_t)(w0[t] & 0x7fffffu), (int32_t)w1[t]};
      const BandFn c = band_compose(Q[t - 1], f);
      const bool join = kt[t] == kt[t - 1]; // dirty keys are unique: never joined
      Q[t].d0 = join ? c.d0 : f.d0;
      Q[t].d1 = join ? c.d1 : f.d1;
    }
    // h: the leading items that share item 0's key
    int h = 1;
#pragma unroll
    for (int t = 1; t < NS; ++t) h += (h == t && kt[t] == kt[0]) ? 1 : 0;
    const bool whole = h == NS && kt[0] > -1000;
    const int lastKeyPrev = dpp<DPP_WAVE_SHR1>(-2000, kt[NS - 1]);
    const bool connIn = lane > 1 && kt[0] == lastKeyPrev; // item 0 continues a run (lane 0 is summed apart)
    const bool connOut = __builtin_amdgcn_update_dpp(0, (int)connIn, DPP_WAVE_SHL1, 0xf, 0xf, false) != 0 && lane < 63;
    const bool segHead = !(whole && connIn);
    const uint64_t heads = __ballot(segHead);
    const int start = 63 - __builtin_clzll(heads & (lane == 63 ? ~0ull : ((2ull << lane) - 1)));
    // the run ending at the lane's last item, from its head in this or an earlier lane
    const BandFn A = wave_seg_compose(Q[NS - 1], start, lane);
    // the head run (items 0 .. h-1) from its head in an earlier lane
    const BandFn Aprev = {dpp<DPP_WAVE_SHR1>(0, A.d0), dpp<DPP_WAVE_SHR1>(0, A.d1)};
    BandFn Qh = Q[0];
#pragma unroll
    for (int t = 1; t < NS; ++t) {
      Qh.d0 = h == t + 1 ? Q[t].d0 : Qh.d0;
      Qh.d1 = h == t + 1 ? Q[t].d1 : Qh.d1;
    }
    const BandFn H = band_compose(Aprev, Qh);
    // the lane's stitch events, item by item: a packed map (bit 31 set) where
    // a run ends, the serial marker 0x40000000 for a dirty item, 0 otherwise
    uint32_t ev0[NS], ev1[NS], evmask = 0;
#pragma unroll
    for (int t = 0; t < NS; ++t) {
      const bool end = t < NS - 1 ? kt[t] != kt[t + 1] : !connOut;
      const bool useH = connIn && t == h - 1;
      const int32_t m0 = useH ? H.d0 : Q[t].d0, m1 = useH ? H.d1 : Q[t].d1;
      const bool ok = ((uint32_t)m0 | (uint32_t)m1) < (1u << 23);
      const uint32_t pk = ((uint32_t)m0 & 0x7fffffu) | (w0[t] & 0x7f800000u) | (ok ? 0x80000000u : 0u);
      ev0[t] = kt[t] <= -1000 ? 0x40000000u : end ? pk : 0u;
      ev1[t] = (uint32_t)m1;
      evmask |= ev0[t] ? (1u << t) : 0u;
    }
    const uint64_t visit = __ballot(evmask != 0) & ~1ull;
    // ---- 5. wave-uniform stitch from s0 (scalar code: a wave issues one
    //         instruction per four cycles, so the step is kept short)
    uint32_t s = p0; // the stitch starts at lane 1
    int nslow = 0;
    uint32_t runBad = 0;
    // (raised issue priority: the stitch is the wave's latency-bound part,
    // and the SIMD's other waves fill the VALU around it)
    __builtin_amdgcn_s_setprio(1);
    for (uint64_t vm = visit; vm; vm &= vm - 1) {
      const int j = __builtin_ctzll(vm);
      const uint32_t m = __builtin_amdgcn_readlane(evmask, j);
#pragma unroll
      for (int t = 0; t < NS; ++t) {
        if (!(m & (1u << t))) continue;
        const uint32_t a0 = __builtin_amdgcn_readlane(ev0[t], j);
        if (a0 == 0x40000000u) {
          // a dirty item: its own serial steps (every lane runs its own
          // elements from s; lane j's result is kept)
          s = serial16(s, &xf[16 * t], j);
          ++nslow;
          continue;
        }
        const uint32_t a1 = __builtin_amdgcn_readlane(ev1[t], j);
        const uint32_t lo = a0 & 0x7f800000u;
        const uint32_t ns = s + ((s & 1u) ? a1 : (a0 & 0x7fffffu));
        // zero iff the map is valid and s and its image lie in the binade
        const uint32_t chk = ((s - lo) | (ns - lo) | (~a0 & 0x80000000u)) >> 23;
        runBad |= chk;
        s = chk ? s : ns;
      }
    }
    __builtin_amdgcn_s_setprio(0);
    const bool fail = runBad != 0; // a run did not hold (its binade was mispredicted)
    if (fail) {
      // a run did not hold (its binade was mispredicted): item by item
      s = __float_as_uint(s0);
      for (int j = 0; j < 64; ++j) {
#pragma unroll
        for (int t = 0; t < NS; ++t) {
          if (!band_apply_packed(s, __builtin_amdgcn_readlane(w0[t], j), __builtin_amdgcn_readlane(w1[t], j))) {
            s = serial16(s, &xf[16 * t], j);
            nslow += 1000;
          }
        }
      }
    }
    // ---- tail: inv, y, amax, scale, codes
    const float ss = __uint_as_float(s);
    if (dbg && lane == 0) {
      dbg[2 * row] = ss;
      dbg[2 * row + 1] = (float)nslow;
    }
    const float inv = 1.0f / __builtin_sqrtf(ss / K + eps);
    float m = 0.0f;
#pragma unroll
    for (int g4 = 0; g4 < SEG / 4; ++g4) {
      const float4 gw = lds_gamma[g4 * 64 + lane];
      xf[4 * g4] = (xf[4 * g4] * inv) * gw.x;
      xf[4 * g4 + 1] = (xf[4 * g4 + 1] * inv) * gw.y;
      xf[4 * g4 + 2] = (xf[4 * g4 + 2] * inv) * gw.z;
      xf[4 * g4 + 3] = (xf[4 * g4 + 3] * inv) * gw.w;
    }
#pragma unroll
    for (int k = 0; k < SEG; k += 2)
      asm volatile("v_maximum3_f32 %0, %0, |%1|, |%2|" : "+v"(m) : "v"(xf[k]), "v"(xf[k + 1]));
    const float amax = maximumf(wave_max(m), a0);
    const float sc = amax / qd;
    if (lane == 0) __builtin_nontemporal_store(sc, &scale[row]);
    const float r = 1.0f / sc;
    Guard gd;
    gd.divisor(r);
    // codes as words: cw[c][d] = word d of lane's 16-byte chunk c
    constexpr int NCH = SEG / 16;
    uint32_t cw[NCH][4];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      // 16 codes: the bracketing pair of packed words, one test for the chunk
      constexpr float D = 0x1p-15f;
      uint32_t wl[4], wh[4];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        wl[w] = 0;
        wh[w] = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float a = xf[16 * c + 4 * w + e];
          wl[w] = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_fmaf(a, r, 128.0f - D), e, wl[w]);
          wh[w] = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_fmaf(a, r, 128.0f + D), e, wh[w]);
        }
      }
      if (__builtin_expect(((wl[0] ^ wh[0]) | (wl[1] ^ wh[1]) | (wl[2] ^ wh[2]) | (wl[3] ^ wh[3])) != 0, 0)) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float a4[4] = {xf[16 * c + 4 * w], xf[16 * c + 4 * w + 1], xf[16 * c + 4 * w + 2], xf[16 * c + 4 * w + 3]};
          wl[w] = quant8x4_inner(a4, sc, r, gd) ^ 0x80808080u;
        }
      }
#pragma unroll
      for (int w = 0; w < 4; ++w) cw[c][w] = wl[w] ^ 0x80808080u;
    }
    if (__ballot(gd.bad()) != 0 || !(amax <= 0x1.fffffep+127f)) {
      // rare: an unsafe magnitude or a NaN quotient -- IEEE division
#pragma unroll
      for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          uint32_t v = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float qf = maximumf(minimumf(__builtin_roundevenf(xf[16 * c + 4 * w + e] / sc), (float)HI), (float)LO);
            v |= ((uint32_t)(int32_t)qf & 0xFFu) << (8 * e);
          }
          cw[c][w] = v;
        }
    }
    // The row's codes leave in NCH stores of 1024 contiguous bytes each (whole
    // 128-byte lines per instruction), non-temporal, so that no dirty lines
    // of them are left in the L2 for the end-of-kernel write-back to wait
    // on.  Lane L's chunk c holds row bytes 16 (NCH L + c) .. +15; a transpose
    // of the chunk index with the lane's 16-lane row (NCH = 4: permlane32 and
    // permlane16 swaps) or 32-lane half (NCH = 2) gives store i, lane (h, m)
    // the chunk h of lane (i, m).
    int8_t *qr = q + row * C;
    if constexpr (NCH == 4) {
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        auto r02 = __builtin_amdgcn_permlane32_swap(cw[0][d], cw[2][d], false, false);
        auto r13 = __builtin_amdgcn_permlane32_swap(cw[1][d], cw[3][d], false, false);
        auto r01 = __builtin_amdgcn_permlane16_swap(r02[0], r13[0], false, false);
        auto r23 = __builtin_amdgcn_permlane16_swap(r02[1], r13[1], false, false);
        cw[0][d] = r01[0];
        cw[1][d] = r01[1];
        cw[2][d] = r23[0];
        cw[3][d] = r23[1];
      }
      // lane 16h + m, store i: bytes 1024 i + 64 m + 16 h (chunk h of lane 16 i + m)
      rq_u4 *dst = reinterpret_cast<rq_u4 *>(qr + 64 * (lane & 15) + 16 * (lane >> 4));
#pragma unroll
      for (int i = 0; i < 4; ++i)
        __builtin_nontemporal_store(rq_u4{cw[i][0], cw[i][1], cw[i][2], cw[i][3]}, dst + 64 * i);
    } else if constexpr (NCH == 2) {
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        auto r01 = __builtin_amdgcn_permlane32_swap(cw[0][d], cw[1][d], false, false);
        cw[0][d] = r01[0];
        cw[1][d] = r01[1];
      }
      // lane 32h + m, store i: bytes 1024 i + 32 m + 16 h (chunk h of lane 32 i + m)
      rq_u4 *dst = reinterpret_cast<rq_u4 *>(qr + 32 * (lane & 31) + 16 * (lane >> 5));
#pragma unroll
      for (int i = 0; i < 2; ++i)
        __builtin_nontemporal_store(rq_u4{cw[i][0], cw[i][1], cw[i][2], cw[i][3]}, dst + 64 * i);
    } else {
      __builtin_nontemporal_store(rq_u4{cw[0][0], cw[0][1], cw[0][2], cw[0][3]}, reinterpret_cast<rq_u4 *>(qr) + lane);
    }
  }
}

} // namespace hf
