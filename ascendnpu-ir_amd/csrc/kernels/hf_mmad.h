// Dense contraction (hivm.hir.mmadL1 / linalg.matmul) with a fused epilogue on
// CDNA4 matrix cores.
//
// C[m, n] = sum_k A[m, k] * B(k, n), A row-major [M, K], B either [N, K]
// (matmul_transpose_b, the weight layout) or [K, N] (linalg.matmul).
//   * int8 x int8 -> int32 with v_mfma_i32_32x32x32_i8 (exact integer sums);
//   * bf16 x bf16 -> fp32 with v_mfma_f32_32x32x16_bf16.
// One 256x256 macro-tile per workgroup of 4 waves (2 x 2, 128x128 each =
// 4 x 4 MFMA tiles of 32x32), K advanced 64 bytes at a time through a
// double-buffered LDS stage with register prefetch of the next K slice.
// Macro-tiles are numbered so that the workgroups the dispatcher sends to one
// XCD (blockIdx % 8) cover a compact 2-D block of C and share A/B panels in
// that XCD's L2.  The epilogue functor receives the raw accumulator and the
// (m, n) coordinate: this is where the reference's fixpipe dequant
// (bishengir/lib/Template/lib/Fixpipe/Fixpipe.cpp, descale modes of
// HIVMAttrs.td:1061-1071) is fused.
#pragma once
#include "hf_ops.h"

namespace hf {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

constexpr int MM_TM = 256, MM_TN = 256, MM_BK = 64; // BK in bytes
constexpr int MM_LDS_STRIDE = MM_BK + 16;             // 80 B rows: conflict-free b128 reads

template <bool I8> struct MfmaOp;
template <> struct MfmaOp<true> {
  using acc_t = v16i;
  using scalar_t = int32_t;
  __device__ __forceinline__ static acc_t run(v4i a, v4i b, acc_t c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  }
};
template <> struct MfmaOp<false> {
  using acc_t = v16f;
  using scalar_t = float;
  __device__ __forceinline__ static acc_t run(v4i a, v4i b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), c, 0, 0, 0);
  }
};

// XCD-aware macro-tile numbering: workgroup b runs on XCD b % 8; give each XCD
// a contiguous (TMt/4) x (TNt/2) block of tiles when the grid allows it.
__device__ __forceinline__ void mm_tile_of(int b, int tmt, int tnt, int &ti, int &tj) {
  if (tmt % 4 == 0 && tnt % 2 == 0 && tmt * tnt >= 64) {
    const int xcd = b % 8, local = b / 8;
    const int bh = tmt / 4, bw = tnt / 2;
    ti = (xcd / 2) * bh + local / bw;
    tj = (xcd % 2) * bw + local % bw;
  } else {
    ti = b / tnt;
    tj = b % tnt;
  }
}

// Loads this thread's share of one [256 rows x 64 B] K-major slice of a
// row-major operand (rows = M or N, row length K bytes) into registers.
// Thread t owns 16-byte chunks (row t/4 + 64 i, byte (t%4)*16), i = 0..3.
template <typename T>
__device__ __forceinline__ void mm_load_kmajor(const T *__restrict__ base, int64_t rows, int64_t row0, int64_t Kbytes,
                                               int64_t k0, v4i (&r)[4]) {
  const int t = threadIdx.x;
  const int64_t kb = k0 + (t % 4) * 16;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t row = row0 + t / 4 + 64 * i;
    if (row < rows && kb < Kbytes) {
      r[i] = __builtin_nontemporal_load(reinterpret_cast<const v4i *>(reinterpret_cast<const char *>(base) + row * Kbytes + kb));
    } else {
      r[i] = v4i{0, 0, 0, 0};
    }
  }
}

__device__ __forceinline__ void mm_store_kmajor(char *lds, const v4i (&r)[4]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    *reinterpret_cast<v4i *>(lds + (t / 4 + 64 * i) * MM_LDS_STRIDE + (t % 4) * 16) = r[i];
}

// [K x N] row-major operand (linalg.matmul B): load a 64(k-bytes) x 256(n)
// slice and write it transposed (n-major) into LDS.  ESZ is the element size.
template <int ESZ>
__device__ __forceinline__ void mm_load_nmajor(const char *__restrict__ B, int64_t N, int64_t K, int64_t n0, int64_t k0,
                                               v4i (&r)[4]) {
  // slice has 64/ESZ k-rows of 256*ESZ bytes: 16-byte chunks, thread t loads 4
  constexpr int KR = MM_BK / ESZ;          // k rows in the slice
  constexpr int CPR = MM_TN * ESZ / 16;    // 16-byte chunks per k row
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = t + 256 * i;             // chunk id in [0, KR*CPR)
    const int kr = c / CPR, ch = c % CPR;
    const int64_t k = k0 / ESZ + kr, n = n0 + (int64_t)ch * (16 / ESZ);
    if (c < KR * CPR && k < K && n < N)
      r[i] = *reinterpret_cast<const v4i *>(B + (k * N + n) * ESZ);
    else
      r[i] = v4i{0, 0, 0, 0};
  }
}

template <int ESZ> __device__ __forceinline__ void mm_store_nmajor(char *lds, const v4i (&r)[4]) {
  constexpr int CPR = MM_TN * ESZ / 16;
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = t + 256 * i;
    const int kr = c / CPR, ch = c % CPR;
    const char *src = reinterpret_cast<const char *>(&r[i]);
#pragma unroll
    for (int e = 0; e < 16 / ESZ; ++e) {
      const int n = ch * (16 / ESZ) + e;
#pragma unroll
      for (int b = 0; b < ESZ; ++b) lds[n * MM_LDS_STRIDE + kr * ESZ + b] = src[e * ESZ + b];
    }
  }
}

template <bool I8, typename Epi, bool BT, typename ElemT, typename Args>
__device__ void mmad_core(const ElemT *__restrict__ A, const ElemT *__restrict__ B, typename Epi::out_t *__restrict__ out,
                          int64_t M, int64_t N, int64_t K, const Args &P) {
  using Op = MfmaOp<I8>;
  using acc_t = typename Op::acc_t;
  constexpr int ESZ = sizeof(ElemT);
  __shared__ __attribute__((aligned(16))) char lds[2][2][MM_TM * MM_LDS_STRIDE]; // [buf][A/B]
  const int tmt = (int)((M + MM_TM - 1) / MM_TM), tnt = (int)((N + MM_TN - 1) / MM_TN);
  int ti, tj;
  mm_tile_of(blockIdx.x, tmt, tnt, ti, tj);
  const int64_t m0 = (int64_t)ti * MM_TM, n0 = (int64_t)tj * MM_TN;
  const int64_t Kb = K * ESZ;
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int wm = wave / 2, wn = wave % 2;

  acc_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = acc_t{};

  v4i ra[4], rb[4];
  mm_load_kmajor(A, M, m0, Kb, 0, ra);
  if constexpr (BT) mm_load_kmajor(B, N, n0, Kb, 0, rb);
  else mm_load_nmajor<ESZ>(reinterpret_cast<const char *>(B), N, K, n0, 0, rb);
  mm_store_kmajor(lds[0][0], ra);
  if constexpr (BT) mm_store_kmajor(lds[0][1], rb);
  else mm_store_nmajor<ESZ>(lds[0][1], rb);
  __syncthreads();

  const int nsteps = (int)((Kb + MM_BK - 1) / MM_BK);
  for (int s = 0; s < nsteps; ++s) {
    const int cur = s & 1;
    const bool more = s + 1 < nsteps;
    if (more) {
      const int64_t k0 = (int64_t)(s + 1) * MM_BK;
      mm_load_kmajor(A, M, m0, Kb, k0, ra);
      if constexpr (BT) mm_load_kmajor(B, N, n0, Kb, k0, rb);
      else mm_load_nmajor<ESZ>(reinterpret_cast<const char *>(B), N, K, n0, k0, rb);
    }
    const char *la = lds[cur][0], *lb = lds[cur][1];
#pragma unroll
    for (int kk = 0; kk < MM_BK; kk += 32) {
      v4i fa[4], fb[4];
      const int koff = kk + (lane / 32) * 16;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        fa[i] = *reinterpret_cast<const v4i *>(la + (wm * 128 + i * 32 + lane % 32) * MM_LDS_STRIDE + koff);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        fb[j] = *reinterpret_cast<const v4i *>(lb + (wn * 128 + j * 32 + lane % 32) * MM_LDS_STRIDE + koff);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = Op::run(fa[i], fb[j], acc[i][j]);
    }
    if (more) {
      mm_store_kmajor(lds[cur ^ 1][0], ra);
      if constexpr (BT) mm_store_kmajor(lds[cur ^ 1][1], rb);
      else mm_store_nmajor<ESZ>(lds[cur ^ 1][1], rb);
    }
    __syncthreads();
  }

  // epilogue: accumulator register r of a 32x32 tile holds
  // row 8*(r/4) + 4*(lane/32) + r%4, column lane%32
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t n = n0 + wn * 128 + j * 32 + lane % 32;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m0 + wm * 128 + i * 32 + 8 * (r / 4) + 4 * (lane / 32) + r % 4;
        if (m < M && n < N) out[m * N + n] = Epi::apply(acc[i][j][r], m, n, P);
      }
    }
}

template <typename Epi, bool BT, typename Args>
__device__ __forceinline__ void mmad_i8(const int8_t *A, const int8_t *B, typename Epi::out_t *out, int64_t M, int64_t N,
                                        int64_t K, const Args &P) {
  mmad_core<true, Epi, BT>(A, B, out, M, N, K, P);
}

template <typename Epi, bool BT, typename Args>
__device__ __forceinline__ void mmad_bf16(const uint16_t *A, const uint16_t *B, typename Epi::out_t *out, int64_t M,
                                          int64_t N, int64_t K, const Args &P) {
  mmad_core<false, Epi, BT>(A, B, out, M, N, K, P);
}

} // namespace hf
