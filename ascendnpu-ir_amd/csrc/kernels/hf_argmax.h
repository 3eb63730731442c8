// hfusion.reduce_with_index over the last axis on CDNA4.
//
// Meaning (HFusionOps.cpp:1507-1595, region of the 3-argument form), folded
// serially by the CPU lowering over c = 0..C-1 starting from (init_v, init_i):
//     res = maximumf(x[c], v); if (res OGT v) i = c; v = res;      (<max>)
//     res = minimumf(x[c], v); if (res OLT v) i = c; v = res;      (<min>)
// Closed form used here (order-independent, hence tree-safe):
//   * let p = index of the first NaN (or C); only x[0..p) can move the index;
//   * M = maximumf over x[0..p), J = lowest c < p with x[c] == M (IEEE ==,
//     so -0 and +0 are one class);
//   * i = (M OGT init_v) ? J : init_i;  v = NaN if p < C, else
//     maximumf(M, init_v).
// Schedule: each row is split into SEG segments, one workgroup each; a
// segment produces the record (M, J, has_nan) of its prefix before its first
// NaN.  With SEG == 1 the workgroup folds it into the init and writes the row.
// Otherwise the last workgroup of a row (arrival counter in the workspace)
// folds the records left to right with the serial rule above and resets the
// counter.
// Cross-workgroup protocol: records and counters are accessed only through
// agent-scope relaxed atomics, which the gfx942/gfx950 memory model keeps
// coherent across the XCDs' L2 caches (sc1 accesses).  A writer waits for
// its record stores to complete (s_waitcnt vmcnt(0)) before the counter RMW;
// the last arriver issues its record loads only after the RMW has returned.
// An acq_rel RMW would add an L2 writeback and an L2 invalidate per
// workgroup (measured: 4x slower over a 256 x 152064 launch), needed only
// for plain stores, of which this protocol has none.
// Replaces the Ascend ReduceAR_With_Index template
// (bishengir/lib/Template/lib/Vector/Reduction/ReduceAR_With_Index.cpp).
#pragma once
#include "hf_ops.h"

namespace hf {

struct ArgRec {
  float m;
  int32_t has_nan;
  int64_t j; // INT64_MAX when the prefix is empty
};

__device__ __forceinline__ void rec_store(ArgRec *slot, const ArgRec &r) {
  uint64_t *w = reinterpret_cast<uint64_t *>(slot);
  const uint64_t w0 = (uint64_t)__builtin_bit_cast(uint32_t, r.m) | ((uint64_t)(uint32_t)r.has_nan << 32);
  __hip_atomic_store(w, w0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(w + 1, (uint64_t)r.j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ ArgRec rec_load(ArgRec *slot) {
  uint64_t *w = reinterpret_cast<uint64_t *>(slot);
  const uint64_t w0 = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t w1 = __hip_atomic_load(w + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  ArgRec r;
  r.m = __builtin_bit_cast(float, (uint32_t)w0);
  r.has_nan = (int32_t)(w0 >> 32);
  r.j = (int64_t)w1;
  return r;
}

template <int KIND> __device__ __forceinline__ bool arg_better(float a, float b) { return KIND == 0 ? (a > b) : (a < b); }
template <int KIND> __device__ __forceinline__ float arg_fold(float a, float b) {
  return KIND == 0 ? maximumf(a, b) : minimumf(a, b);
}

// (value, index) combine: strictly better value wins; equal values keep the
// lower index and fold the value (so +0 absorbs -0 for <max>).
template <int KIND> __device__ __forceinline__ void arg_combine(float &v, int64_t &i, float v2, int64_t i2) {
  if (arg_better<KIND>(v2, v)) { v = v2; i = i2; }
  else if (!(arg_better<KIND>(v, v2))) { // equal (neither better; NaN excluded by construction)
    v = arg_fold<KIND>(v, v2);
    i = i2 < i ? i2 : i;
  }
}

template <int KIND, int BLOCK>
__device__ __forceinline__ void arg_block_reduce(float &v, int64_t &i, float *sv, int64_t *si) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    float v2 = __shfl_xor(v, m, 64);
    int64_t i2 = __shfl_xor(i, m, 64);
    arg_combine<KIND>(v, i, v2, i2);
  }
  constexpr int NW = BLOCK / 64;
  const int w = threadIdx.x / 64, l = threadIdx.x % 64;
  if (l == 0) { sv[w] = v; si[w] = i; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < NW; ++k) arg_combine<KIND>(v, i, sv[k], si[k]);
  }
}

// Scans [s0, s1) of a row; elements at or past `limit` are ignored; NaNs are
// excluded from (v, i) and the first NaN position is tracked in `nan_at`.
template <int KIND, int BLOCK, bool ALIGNED>
__device__ __forceinline__ void arg_scan(const float *__restrict__ row, int64_t s0, int64_t s1, int64_t limit, float &v,
                                         int64_t &i, int64_t &nan_at) {
  const float ident = KIND == 0 ? -__builtin_inff() : __builtin_inff();
  v = ident;
  i = INT64_MAX;
  nan_at = INT64_MAX;
  const int64_t e1 = s1 < limit ? s1 : limit;
  auto visit = [&](float x, int64_t c) {
    if (x != x) { nan_at = c < nan_at ? c : nan_at; return; }
    arg_combine<KIND>(v, i, x, c);
  };
  if constexpr (ALIGNED) {
    const int64_t n4 = (e1 - s0) / 4;
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const f32x4 *p4 = reinterpret_cast<const f32x4 *>(row + s0);
#pragma unroll 4
    for (int64_t q = threadIdx.x; q < n4; q += BLOCK) {
      const f32x4 x = __builtin_nontemporal_load(p4 + q);
      const int64_t c = s0 + q * 4;
      visit(x.x, c);
      visit(x.y, c + 1);
      visit(x.z, c + 2);
      visit(x.w, c + 3);
    }
    for (int64_t c = s0 + n4 * 4 + threadIdx.x; c < e1; c += BLOCK) visit(row[c], c);
  } else {
    for (int64_t c = s0 + threadIdx.x; c < e1; c += BLOCK) visit(row[c], c);
  }
}

// Segment record without NaNs, in one streaming pass: every lane walks its
// elements in increasing index order, CH float4 (or 4*CH scalars) per round
// with all loads of a round in flight together, keeping
//   m = fold (maximumf / minimumf, NaN-propagating) of what it has seen,
//   j = its first position whose value beats every earlier one (strictly),
// which is its first position holding a value IEEE-equal to its final m
// (equal values, and -0/+0, never replace j).  Lanes are then combined by
// (better value; for IEEE-equal values the lower position).  Returns false
// when the segment holds a NaN (m is NaN); the caller takes the general path.
template <int KIND, int BLOCK, bool ALIGNED>
__device__ __forceinline__ bool arg_segment_fast(const float *__restrict__ row, int64_t s0, int64_t e1, float &v, int64_t &i,
                                                 float *sv, int *si) {
  constexpr int CH = 8;
  const float ident = KIND == 0 ? -__builtin_inff() : __builtin_inff();
  const int tid = threadIdx.x;
  const int n = (int)(e1 - s0);
  float m = ident;
  int j = 0x7fffffff;
  auto visit = [&](float x, int pos) {
    j = arg_better<KIND>(x, m) ? pos : j;
    m = arg_fold<KIND>(x, m);
  };
  if constexpr (ALIGNED) {
    // n % 4 == 0 (C % 4 == 0): no partial float4; lanes past the end read a
    // clamped in-range address and see the identity
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const f32x4 *p4 = reinterpret_cast<const f32x4 *>(row + s0);
    const int n4 = n / 4;
    for (int q0 = 0; q0 < n4; q0 += CH * BLOCK) {
      f32x4 t[CH];
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int o4 = q0 + c * BLOCK + tid;
        t[c] = __builtin_nontemporal_load(p4 + (o4 < n4 ? o4 : n4 - 1));
      }
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int o4 = q0 + c * BLOCK + tid;
        const bool in = o4 < n4;
        visit(in ? t[c].x : ident, 4 * o4);
        visit(in ? t[c].y : ident, 4 * o4 + 1);
        visit(in ? t[c].z : ident, 4 * o4 + 2);
        visit(in ? t[c].w : ident, 4 * o4 + 3);
      }
    }
  } else {
    for (int o0 = 0; o0 < n; o0 += 4 * CH * BLOCK) {
      float t[4 * CH];
#pragma unroll
      for (int c = 0; c < 4 * CH; ++c) {
        const int o = o0 + c * BLOCK + tid;
        t[c] = __builtin_nontemporal_load(row + s0 + (o < n ? o : n - 1));
      }
#pragma unroll
      for (int c = 0; c < 4 * CH; ++c) {
        const int o = o0 + c * BLOCK + tid;
        visit(o < n ? t[c] : ident, o);
      }
    }
  }
  // a lane whose in-range values all equal the identity (e.g. -inf for
  // <max>) never saw a strictly better one: its answer is its first position
  {
    const int first = ALIGNED ? 4 * tid : tid;
    if (j == 0x7fffffff && m == ident && first < n) j = first;
  }
  // lanes with no element in range keep j = 0x7fffffff; a real position is
  // always lower
  auto combine = [&](float m2, int j2) {
    if (arg_better<KIND>(m2, m)) { m = m2; j = j2; }
    else if (!arg_better<KIND>(m, m2)) { m = arg_fold<KIND>(m, m2); j = j2 < j ? j2 : j; }
  };
#pragma unroll
  for (int sh = 32; sh >= 1; sh >>= 1) {
    const float m2 = __shfl_xor(m, sh, 64);
    const int j2 = __shfl_xor(j, sh, 64);
    combine(m2, j2);
  }
  constexpr int NW = BLOCK / 64;
  if (tid % 64 == 0) { sv[tid / 64] = m; si[tid / 64] = j; }
  __syncthreads();
  m = sv[0];
  j = si[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) combine(sv[w], si[w]);
  if (m != m) return false; // a NaN somewhere in the segment
  v = m;
  i = j == 0x7fffffff ? INT64_MAX : s0 + j;
  return true;
}

// One work item: segment `item % SEG` of row `item / SEG` (SEG segments of
// SEGLEN elements per row); with SEG > 1 the last of a row's segments to
// arrive folds the row's records.
template <int KIND, int BLOCK, bool ALIGNED, typename IdxT>
__device__ void arg_item(const float *__restrict__ x, int64_t R, int64_t C, int64_t SEG, int64_t SEGLEN, int64_t item,
                         float init_v, IdxT init_i, float *__restrict__ out_v, IdxT *__restrict__ out_i, void *ws) {
  __shared__ float sv[BLOCK / 64];
  __shared__ int64_t si[BLOCK / 64];
  __shared__ int64_t snan[BLOCK / 64];
  __shared__ float fv[BLOCK / 64];
  __shared__ int fi[BLOCK / 64];
  __shared__ int last;
  ArgRec *recs = reinterpret_cast<ArgRec *>(ws);
  unsigned *counters = reinterpret_cast<unsigned *>(recs + R * SEG);
  const int64_t row = item / SEG, seg = item % SEG;
  const float *rp = x + row * C;
  const int64_t s0 = seg * SEGLEN, s1 = (s0 + SEGLEN < C) ? s0 + SEGLEN : C;
  float v;
  int64_t i;
  bool has_nan = false;
  if (!arg_segment_fast<KIND, BLOCK, ALIGNED>(rp, s0, s1, v, i, fv, fi)) {
    // rare path: locate the first NaN, then rescan the prefix before it
    int64_t nan_at;
    arg_scan<KIND, BLOCK, ALIGNED>(rp, s0, s1, s1, v, i, nan_at);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      int64_t o = __shfl_xor(nan_at, m, 64);
      nan_at = o < nan_at ? o : nan_at;
    }
    if (threadIdx.x % 64 == 0) snan[threadIdx.x / 64] = nan_at;
    __syncthreads();
    int64_t p = snan[0];
    for (int k = 1; k < BLOCK / 64; ++k) p = snan[k] < p ? snan[k] : p;
    int64_t dummy;
    arg_scan<KIND, BLOCK, ALIGNED>(rp, s0, s1, p, v, i, dummy);
    arg_block_reduce<KIND, BLOCK>(v, i, sv, si);
    has_nan = true;
  }
  if (SEG == 1) {
    // the whole row in this workgroup: fold the record into the init directly
    if (threadIdx.x == 0) {
      float V = init_v;
      int64_t I = (int64_t)init_i;
      if (V == V) {
        if (i != INT64_MAX) {
          if (arg_better<KIND>(v, V)) I = i;
          V = arg_fold<KIND>(v, V);
        }
        if (has_nan) V = __builtin_nanf("");
      }
      if (out_v) out_v[row] = V;
      if (out_i) out_i[row] = (IdxT)I;
    }
    return;
  }
  if (threadIdx.x == 0) {
    ArgRec r;
    r.m = v;
    r.has_nan = has_nan;
    r.j = i;
    rec_store(&recs[item], r);
    // release: the record happens-before the count that the last arriver
    // reads; acquire: the last arriver's reads of the other records follow it
    unsigned prev = __hip_atomic_fetch_add(&counters[row], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    last = prev == (unsigned)(SEG - 1);
  }
  __syncthreads();
  if (!last) return;
  // every thread of the last arriver loads records: order its loads after
  // thread 0's acquire (the barrier above) at agent scope
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  // serial fold of the segment records, left to right: the whole workgroup
  // loads BLOCK records at a time into LDS (independent loads in flight
  // together), thread 0 folds them
  __shared__ ArgRec fold[BLOCK];
  float V = init_v;
  int64_t I = (int64_t)init_i;
  bool vnan = V != V;
  for (int64_t s0 = 0; s0 < SEG; s0 += BLOCK) {
    const int64_t s = s0 + threadIdx.x;
    if (s < SEG) fold[threadIdx.x] = rec_load(&recs[row * SEG + s]); // issued after the counter RMW returned
    __syncthreads();
    if (threadIdx.x == 0) {
      const int64_t n = SEG - s0 < BLOCK ? SEG - s0 : BLOCK;
      for (int64_t t = 0; t < n && !vnan; ++t) {
        const ArgRec r = fold[t];
        if (r.j != INT64_MAX) {
          if (arg_better<KIND>(r.m, V)) I = r.j;
          V = arg_fold<KIND>(r.m, V);
        }
        if (r.has_nan) { V = __builtin_nanf(""); vnan = true; }
      }
    }
    __syncthreads();
  }
  if (threadIdx.x != 0) return;
  if (out_v) out_v[row] = V;
  if (out_i) out_i[row] = (IdxT)I;
  __hip_atomic_store(&counters[row], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int KIND, int BLOCK, bool ALIGNED, typename IdxT>
__device__ void argreduce_rows(const float *__restrict__ x, int64_t R, int64_t C, int64_t SEG, int64_t SEGLEN, float init_v,
                               IdxT init_i, float *__restrict__ out_v, IdxT *__restrict__ out_i, void *ws) {
  arg_item<KIND, BLOCK, ALIGNED, IdxT>(x, R, C, SEG, SEGLEN, blockIdx.x, init_v, init_i, out_v, out_i, ws);
}

// The split of a row into segments for R rows of C elements: about two
// workgroups per CU when there are fewer rows than CUs, segments a multiple
// of 4 elements (aligned float4 loads) and at least min(C, 4096) long.  The
// compiler uses the same rule for a static R (lower.cpp, REDUCE_WITH_INDEX).
__device__ __forceinline__ void arg_schedule(int64_t R, int64_t C, int64_t &segs, int64_t &segLen) {
  constexpr int64_t CUS = 256;
  segs = R >= CUS ? 1 : ((2 * CUS + R - 1) / R > 1 ? (2 * CUS + R - 1) / R : 1);
  segLen = ((C + segs - 1) / segs + 3) / 4 * 4;
  const int64_t minLen = (C + 3) / 4 * 4 < 4096 ? (C + 3) / 4 * 4 : 4096;
  segLen = segLen > minLen ? segLen : minLen;
  segs = (C + segLen - 1) / segLen;
}

// A runtime row count R: the segments follow arg_schedule (one segment per
// row when the workspace of WS bytes could not hold the records), and the
// grid walks the R * SEG work items.  init(row) gives the row's init value
// and index.
template <int KIND, int BLOCK, bool ALIGNED, typename IdxT, typename Init>
__device__ void argreduce_rows_dyn(const float *__restrict__ x, int64_t R, int64_t C, uint64_t WS, Init init,
                                   float *__restrict__ out_v, IdxT *__restrict__ out_i, void *ws) {
  int64_t SEG, SEGLEN;
  arg_schedule(R, C, SEG, SEGLEN);
  if ((uint64_t)(R * SEG * 16 + R * 4 + 256) > WS) {
    SEG = 1;
    SEGLEN = (C + 3) / 4 * 4;
  }
  for (int64_t item = blockIdx.x; item < R * SEG; item += gridDim.x) {
    float init_v;
    IdxT init_i;
    init(item / SEG, init_v, init_i);
    arg_item<KIND, BLOCK, ALIGNED, IdxT>(x, R, C, SEG, SEGLEN, item, init_v, init_i, out_v, out_i, ws);
    __syncthreads(); // the item's shared scratch is free
  }
}

} // namespace hf
