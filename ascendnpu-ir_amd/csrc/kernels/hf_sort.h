// hfusion.sort: the values of each row sorted along the last axis.
//
// The reference decomposes the op into a bubble sort
// (bishengir/lib/Dialect/HFusion/Transforms/DecomposeOpInterfaceImpl.cpp:
// 740-830): n-1 passes over j = 0..n-2, swapping elements j and j+1 when
// `cmpf ugt` holds (descending: `ult`; integers: `sgt` / `slt`).  Its result
// has a closed form, which is what runs here:
//   * values that are not NaN never swap when equal, so they come out stably
//     sorted (in particular +0 and -0, which compare equal, keep their input
//     order);
//   * every pass moves each NaN one slot to the left (a compare with a NaN on
//     the right always swaps, and the carried element passes it), except that
//     a pass starting with a NaN carries that NaN to the end (every compare
//     with it on the left swaps).  A NaN starting at p <= n-2 reaches slot 0
//     at pass p and wraps once, so after the n-1 passes the NaN that started
//     at p sits at (p + 1) mod n, bits unchanged;
//   * the sorted non-NaN values fill the remaining slots in order.
// (There are always enough passes for the non-NaN values to be fully sorted:
// only passes that start with a NaN skip sorting work, at most one per NaN.)
//
// One workgroup sorts RPW = max(1, 2048 / P) rows, P = L rounded up to a
// power of two, in LDS: 64-bit keys (order key << 32 | index) through a
// bitonic network per P-element segment.  The index makes every key unique,
// so the network's unstable exchanges still give the stable order.  The
// order key maps the values to unsigned integers in ascending order
// (descending: complemented); NaNs take 0xffffffff and end up after every
// value, in index order; padding takes ~0.  The output is gathered from the
// input row (L2-resident) by the sorted indices.
#pragma once
#include "hf_ops.h"

namespace hf {

// element kinds: 0 f32, 1 f16, 2 bf16, 8/16/32 signed integers of that width
template <int KIND> struct SortElem;
template <> struct SortElem<0> { using T = float; };
template <> struct SortElem<1> { using T = uint16_t; };
template <> struct SortElem<2> { using T = uint16_t; };
template <> struct SortElem<8> { using T = int8_t; };
template <> struct SortElem<16> { using T = int16_t; };
template <> struct SortElem<32> { using T = int32_t; };

template <int KIND> __device__ __forceinline__ bool sort_isnan(typename SortElem<KIND>::T v) {
  if constexpr (KIND == 0) return __builtin_isnan(v);
  else if constexpr (KIND == 1) return (v & 0x7c00) == 0x7c00 && (v & 0x03ff) != 0;
  else if constexpr (KIND == 2) return (v & 0x7f80) == 0x7f80 && (v & 0x007f) != 0;
  else return false;
}

// ascending order key of a value that is not NaN
template <int KIND> __device__ __forceinline__ uint32_t sort_order_key(typename SortElem<KIND>::T v) {
  if constexpr (KIND == 0 || KIND == 1 || KIND == 2) {
    uint32_t b;
    if constexpr (KIND == 0) b = __float_as_uint(v);
    else if constexpr (KIND == 1) b = (uint32_t)v << 16;  // f16 order = order of its bits as the high half
    else b = (uint32_t)v << 16;                            // bf16: the f32 with these high bits
    if ((b & 0x7fffffffu) == 0) b = 0;                     // -0 == +0
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  } else {
    return (uint32_t)(int32_t)v ^ 0x80000000u;
  }
}

template <int KIND, bool DESC, int P, int NT>
__device__ void sort_rows(const typename SortElem<KIND>::T *__restrict__ src, typename SortElem<KIND>::T *__restrict__ dst,
                          int64_t R, int L) {
  using T = typename SortElem<KIND>::T;
  constexpr int RPW = P >= 2048 ? 1 : 2048 / P;
  constexpr int E = RPW * P;
  constexpr bool FLOAT = KIND <= 2;
  __shared__ unsigned long long key[E];
  const int64_t r0 = (int64_t)blockIdx.x * RPW;

  for (int e = threadIdx.x; e < E; e += NT) {
    const int64_t r = r0 + e / P;
    const int j = e % P;
    unsigned long long k = ~0ull;
    if (r < R && j < L) {
      const T v = src[r * L + j];
      uint32_t hi;
      if (FLOAT && sort_isnan<KIND>(v)) hi = 0xffffffffu;
      else hi = DESC ? ~sort_order_key<KIND>(v) : sort_order_key<KIND>(v);
      k = ((unsigned long long)hi << 32) | (uint32_t)j;
    }
    key[e] = k;
  }
  __syncthreads();

  // bitonic network over each P-element segment (ascending keys)
  for (int k = 2; k <= P; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int t = threadIdx.x; t < E / 2; t += NT) {
        const int i = 2 * t - (t & (j - 1));
        const int q = i + j;
        const bool up = k == P || (i & k) == 0;
        const unsigned long long a = key[i], b = key[q];
        if ((a > b) == up) {
          key[i] = b;
          key[q] = a;
        }
      }
      __syncthreads();
    }
  }

  for (int e = threadIdx.x; e < E; e += NT) {
    const int64_t r = r0 + e / P;
    const int q = e % P;
    if (r >= R || q >= L) continue;
    const T *row = src + r * L;
    const unsigned long long *seg = key + (e / P) * P;
    int rank = q;
    if constexpr (FLOAT) {
      // first sorted position holding a NaN (keys ascend; NaN keys and
      // padding are the only ones with the high word all ones)
      int lo = 0, hi = L;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if ((uint32_t)(seg[mid] >> 32) == 0xffffffffu) hi = mid;
        else lo = mid + 1;
      }
      const int first_nan = lo;
      if (first_nan < L) {
        const int p = q == 0 ? L - 1 : q - 1;
        const T pv = row[p];
        if (sort_isnan<KIND>(pv)) {
          dst[r * L + q] = pv;  // the NaN that started at p
          continue;
        }
        // NaN slots before q: slot 0 when the last input is NaN, and slot
        // s in [1, q-1] when input s-1 is NaN (NaN indices <= q-2, found in
        // the NaN keys, which are in index order)
        int c = 0;
        if (q >= 1) {
          c = sort_isnan<KIND>(row[L - 1]) ? 1 : 0;
          int a = first_nan, b = L;
          while (a < b) {
            const int mid = (a + b) >> 1;
            if ((int)(uint32_t)seg[mid] <= q - 2) a = mid + 1;
            else b = mid;
          }
          c += a - first_nan;
        }
        rank = q - c;
      }
    }
    dst[r * L + q] = row[(uint32_t)seg[rank]];
  }
}

} // namespace hf
