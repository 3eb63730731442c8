// HFusion ops lowered one op per kernel: histogram (the cumulative ops and
// (de)interleave are generated in full by the lowering; they need no library
// code beyond hf_ops.h).
#pragma once
#include "hf_ops.h"

namespace hf {

// hfusion.histogram (HFusionOps.td:637-660; CPU meaning
// ConvertHFusionToUpstream.cpp:39-160): for every element v of the flattened
// input with 0 <= v < bins (and mask != 0 when a mask is given),
// hist[v] += 1, starting from zero; the counts wrap to the output width as
// arith.addi does.  Counting is order-free, so the result is exact in any
// order: each workgroup counts its grid-strided share in LDS (LDSB > 0, bins
// <= LDSB) or straight into the workspace, then adds its counts into the
// u64 workspace with agent-scope atomics.  The last workgroup to arrive
// (arrival counter after the bins) copies the totals to the output and
// clears the workspace for the next launch; the workspace starts zeroed.
template <int BLOCK, int LDSB, bool MASK, typename IT, typename MT, typename OT>
__device__ void histogram(const IT *__restrict__ x, const MT *__restrict__ mask, int64_t n, int64_t bins,
                          OT *__restrict__ out, unsigned long long *ws) {
  __shared__ unsigned h[LDSB > 0 ? LDSB : 1];
  __shared__ int last;
  if constexpr (LDSB > 0)
    for (int64_t b = threadIdx.x; b < bins; b += BLOCK) h[b] = 0;
  __syncthreads();
  for (int64_t i = (int64_t)blockIdx.x * BLOCK + threadIdx.x; i < n; i += (int64_t)gridDim.x * BLOCK) {
    const int64_t v = (int64_t)x[i];
    bool ok = v >= 0 && v < bins;
    if constexpr (MASK) ok = ok && mask[i] != 0;
    if (ok) {
      if constexpr (LDSB > 0) atomicAdd(&h[v], 1u);
      else __hip_atomic_fetch_add(&ws[v], 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  if constexpr (LDSB > 0)
    for (int64_t b = threadIdx.x; b < bins; b += BLOCK)
      if (h[b]) __hip_atomic_fetch_add(&ws[b], (unsigned long long)h[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // every thread's adds complete before the arrival is counted
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __syncthreads();
  unsigned *arrived = reinterpret_cast<unsigned *>(ws + bins);
  if (threadIdx.x == 0)
    last = __hip_atomic_fetch_add(arrived, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
  __syncthreads();
  if (!last) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  for (int64_t b = threadIdx.x; b < bins; b += BLOCK) {
    const unsigned long long c = __hip_atomic_load(&ws[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    out[b] = (OT)c;
    __hip_atomic_store(&ws[b], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (threadIdx.x == 0) __hip_atomic_store(arrived, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

} // namespace hf
