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
// NaN; the last workgroup of a row (arrival counter in the workspace) folds the
// records left to right with the serial rule above and resets the counter.
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

// Segment record without NaNs, from registers: every lane loads its NV
// float4 (or 4*NV scalars) of the segment at once, then
//   pass 1: M = fold (maximumf / minimumf, NaN-propagating) over the block;
//   pass 2: J = lowest index c with x[c] == M (IEEE ==) over the block.
// Returns false (and leaves v, i unset) when the segment holds a NaN; the
// caller then takes the general path.  Indices inside a segment are 32-bit.
template <int KIND, int BLOCK, bool ALIGNED, int NV>
__device__ __forceinline__ bool arg_segment_fast(const float *__restrict__ row, int64_t s0, int64_t e1, float &v, int64_t &i,
                                                 float *sv, int *si) {
  const float ident = KIND == 0 ? -__builtin_inff() : __builtin_inff();
  const int tid = threadIdx.x;
  const int n = (int)(e1 - s0);
  float x[4 * NV];
  // element k of lane tid sits at offset off(k) of the segment
  auto off = [&](int k) -> int {
    return ALIGNED ? ((k / 4) * BLOCK + tid) * 4 + (k % 4) : (k / 4) * 4 * BLOCK + (k % 4) * BLOCK + tid;
  };
  // branch-free loads (a branch per load would make the compiler wait for
  // each): lanes past the end read a clamped in-range address and select the
  // identity.  ALIGNED means C % 4 == 0, so n % 4 == 0 and no float4 is partial.
  if constexpr (ALIGNED) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const f32x4 *p4 = reinterpret_cast<const f32x4 *>(row + s0);
    const int last4 = n / 4 - 1;
#pragma unroll
    for (int q = 0; q < NV; ++q) {
      const int o4 = q * BLOCK + tid;
      const f32x4 t = __builtin_nontemporal_load(p4 + (o4 < last4 ? o4 : last4));
      const bool in = o4 <= last4;
      x[4 * q + 0] = in ? t.x : ident;
      x[4 * q + 1] = in ? t.y : ident;
      x[4 * q + 2] = in ? t.z : ident;
      x[4 * q + 3] = in ? t.w : ident;
    }
  } else {
#pragma unroll
    for (int k = 0; k < 4 * NV; ++k) {
      const int o = off(k);
      const float t = __builtin_nontemporal_load(row + s0 + (o < n ? o : n - 1));
      x[k] = o < n ? t : ident;
    }
  }
  float m = ident;
#pragma unroll
  for (int k = 0; k < 4 * NV; ++k) m = arg_fold<KIND>(x[k], m);
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) m = arg_fold<KIND>(__shfl_xor(m, s, 64), m);
  constexpr int NW = BLOCK / 64;
  if (tid % 64 == 0) sv[tid / 64] = m;
  __syncthreads();
  m = sv[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) m = arg_fold<KIND>(sv[w], m);
  if (m != m) return false; // a NaN somewhere in the segment
  int j = 0x7fffffff;
#pragma unroll
  for (int k = 4 * NV - 1; k >= 0; --k) {
    const int o = off(k);
    j = (x[k] == m && o < n) ? o : j; // lane offsets grow with k: the last hit kept is the lowest
  }
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) {
    const int o = __shfl_xor(j, s, 64);
    j = o < j ? o : j;
  }
  if (tid % 64 == 0) si[tid / 64] = j;
  __syncthreads();
  j = si[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) j = si[w] < j ? si[w] : j;
  v = m;
  i = j == 0x7fffffff ? INT64_MAX : s0 + j;
  return true;
}

template <int KIND, int BLOCK, bool ALIGNED, typename IdxT, int NV>
__device__ void argreduce_rows(const float *__restrict__ x, int64_t R, int64_t C, int64_t SEG, int64_t SEGLEN, float init_v,
                               IdxT init_i, float *__restrict__ out_v, IdxT *__restrict__ out_i, void *ws) {
  static_assert(NV >= 1, "segment of at least 4*BLOCK elements");
  __shared__ float sv[BLOCK / 64];
  __shared__ int64_t si[BLOCK / 64];
  __shared__ int64_t snan[BLOCK / 64];
  __shared__ float fv[BLOCK / 64];
  __shared__ int fi[BLOCK / 64];
  __shared__ int last;
  ArgRec *recs = reinterpret_cast<ArgRec *>(ws);
  unsigned *counters = reinterpret_cast<unsigned *>(recs + R * SEG);
  const int64_t row = blockIdx.x / SEG, seg = blockIdx.x % SEG;
  const float *rp = x + row * C;
  const int64_t s0 = seg * SEGLEN, s1 = (s0 + SEGLEN < C) ? s0 + SEGLEN : C;
  float v;
  int64_t i;
  bool has_nan = false;
  if (!arg_segment_fast<KIND, BLOCK, ALIGNED, NV>(rp, s0, s1, v, i, fv, fi)) {
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
  if (threadIdx.x == 0) {
    ArgRec r;
    r.m = v;
    r.has_nan = has_nan;
    r.j = i;
    rec_store(&recs[blockIdx.x], r);
    __builtin_amdgcn_s_waitcnt(0); // the record stores have completed
    unsigned prev = __hip_atomic_fetch_add(&counters[row], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = prev == (unsigned)(SEG - 1);
  }
  __syncthreads();
  if (!last || threadIdx.x != 0) return;
  // serial fold of the segment records, left to right
  float V = init_v;
  int64_t I = (int64_t)init_i;
  bool vnan = V != V;
  for (int64_t s = 0; s < SEG && !vnan; ++s) {
    const ArgRec r = rec_load(&recs[row * SEG + s]); // issued after the counter RMW returned
    if (r.j != INT64_MAX) {
      if (arg_better<KIND>(r.m, V)) I = r.j;
      V = arg_fold<KIND>(r.m, V);
    }
    if (r.has_nan) { V = __builtin_nanf(""); vnan = true; }
  }
  if (out_v) out_v[row] = V;
  if (out_i) out_i[row] = (IdxT)I;
  __hip_atomic_store(&counters[row], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

} // namespace hf
