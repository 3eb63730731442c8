// Dense contraction (hivm.hir.mmadL1 / linalg.matmul) with a fused epilogue on
// CDNA4 matrix cores.
//
// C[m, n] = sum_k A(m, k) * B(k, n), A row-major [M, K] (or [K, M],
// hivm a_transpose), B either [N, K] (matmul_transpose_b / b_transpose, the
// weight layout) or [K, N] (linalg.matmul).
//   * int8 x int8 -> int32 with v_mfma_i32_32x32x32_i8 (exact integer sums);
//   * bf16 x bf16 -> fp32 with v_mfma_f32_32x32x16_bf16;
//   * f16 x f16 -> fp32 with v_mfma_f32_32x32x16_f16.
// One 256x256 macro-tile per workgroup of 4 waves (2 x 2, 128x128 each =
// 4 x 4 MFMA tiles of 32x32), K advanced 64 bytes at a time.
//   * DMA path (B [N, K], K spanning a multiple of 64 bytes): a 4-slot LDS
//     ring filled by global_load_lds_dwordx4 four steps ahead of the MFMAs,
//     fragments double-buffered in registers (one barrier per step);
//   * register path (the rest): a double-buffered LDS stage with register
//     prefetch of the next K slice.
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

// Matrix-core kinds: int8 -> int32, bf16 -> fp32, f16 -> fp32 (32x32 tiles;
// each lane feeds 16 bytes of A and of B per instruction, 32 bytes of K).
// MK_MX + 2 * fa + fb: block-scaled fp8 (fa, fb: 0 e4m3, 1 e5m2, the
// matrix core's format codes), 32 k per e8m0 scale; MK_MX4: block-scaled
// fp4 (e2m1, format code 4) on both sides, two values per byte along K
enum MmadKind : int { MK_I8 = 0, MK_BF16 = 1, MK_F16 = 2, MK_MX = 3, MK_MX4 = 7 };
constexpr bool mk_is_mx(int mk) { return mk >= MK_MX && mk <= MK_MX4; }
constexpr bool mk_is_fp4(int mk) { return mk == MK_MX4; }
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

template <int MK> struct MfmaOp;
template <> struct MfmaOp<MK_I8> {
  using acc_t = v16i;
  using scalar_t = int32_t;
  __device__ __forceinline__ static acc_t run(v4i a, v4i b, acc_t c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  }
};
template <> struct MfmaOp<MK_BF16> {
  using acc_t = v16f;
  using scalar_t = float;
  __device__ __forceinline__ static acc_t run(v4i a, v4i b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), c, 0, 0, 0);
  }
};
typedef int v8i __attribute__((ext_vector_type(8)));
// v_mfma_scale_f32_32x32x64_f8f6f4.  Operand layout (measured on gfx950):
// lane l holds row (col) l % 32; its bytes 0-15 are k = 16 (l / 32) + 0..15
// and bytes 16-31 are k = 32 + 16 (l / 32) + 0..15 of the 64; the scale
// byte of lane l applies to row (col) l % 32 at k = 32 (l / 32) .. +31, i.e.
// to bytes 0-15 of lanes 32 (l / 32) / 32 and bytes 16-31 alike.  SEL picks
// the byte of the scale register.
// For fp4 each lane's 16 bytes hold its 32 k (k = 32 (l / 32) + 0..31, the
// even k in the low nibble): exactly the int8 fragment of one 32-byte k-block,
// in the operand's low four registers.
template <int MK> struct MfmaMx {
  static_assert(mk_is_mx(MK), "block-scaled kind");
  using acc_t = v16f;
  static constexpr int FA = mk_is_fp4(MK) ? 4 : (MK - MK_MX) / 2, FB = mk_is_fp4(MK) ? 4 : (MK - MK_MX) % 2;
  template <int SEL>
  __device__ __forceinline__ static acc_t run(v8i a, v8i b, acc_t c, int sa, int sb) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, FA, FB, SEL, sa, SEL, sb);
  }
};
__device__ __forceinline__ v8i mx_cat(v4i lo, v4i hi) { return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]}; }
__device__ __forceinline__ v8i mx_lo(v4i lo) { return v8i{lo[0], lo[1], lo[2], lo[3], 0, 0, 0, 0}; }
template <> struct MfmaOp<MK_F16> {
  using acc_t = v16f;
  using scalar_t = float;
  __device__ __forceinline__ static acc_t run(v4i a, v4i b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), c, 0, 0, 0);
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

// Epilogue: accumulator register r of a 32x32 tile holds row
// 8*(r/4) + 4*(lane/32) + r%4 and column lane%32 of that tile.  The
// functor's per-row operands are loaded once per accumulator row and its
// per-column operands once per column; bounds are tested per element only
// in tiles that cross the edge of C.
template <typename Epi, typename acc_t, typename Args>
__device__ __forceinline__ void mm_epilogue(acc_t (&acc)[4][4], typename Epi::out_t *__restrict__ out, int64_t M,
                                            int64_t N, int64_t m0, int64_t n0, int wm, int wn, int lane, const Args &P) {
  const bool full = m0 + MM_TM <= M && n0 + MM_TN <= N;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    typename Epi::row_t rv[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t m = m0 + wm * 128 + i * 32 + 8 * (r / 4) + 4 * (lane / 32) + r % 4;
      rv[r] = Epi::row(m < M ? m : M - 1, P);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t n = n0 + wn * 128 + j * 32 + lane % 32;
      const typename Epi::col_t cv = Epi::col(n < N ? n : N - 1, P);
      // the tile leaves the accumulator registers only here: one tile's
      // values in VGPRs at a time
      acc_t a = acc[i][j];
      asm volatile("" : "+a"(a)::"memory");
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t m = m0 + wm * 128 + i * 32 + 8 * (r / 4) + 4 * (lane / 32) + r % 4;
        if (full || (m < M && n < N)) out[m * N + n] = Epi::apply(a[r], m, n, rv[r], cv, P);
      }
    }
  }
}

// Epilogue through LDS (the DMA path's ring is free by then): the tile's
// outputs are computed into a row-major out_t stage, then the whole
// workgroup (NT threads) writes them out as 16-byte row segments (a
// 256-column row is one contiguous run of C).  Each wave holds 128 rows x
// 32*JT columns.  When the whole 256x256 tile fits the stage (2-byte
// outputs) all waves compute at once; otherwise the two row halves (waves
// wm = 0, then wm = 1) take turns.
template <typename Epi, int JT = 4, int NT = 256, typename acc_t, typename Args>
__device__ __forceinline__ void mm_epilogue_lds(acc_t (&acc)[4][JT], typename Epi::out_t *__restrict__ out, int64_t M,
                                                int64_t N, int64_t m0, int64_t n0, int wm, int wn, int lane, const Args &P,
                                                char *stage, int stage_bytes) {
  using O = typename Epi::out_t;
  constexpr int RB = 256 * (int)sizeof(O);       // bytes of one staged row
  constexpr int CPR = RB / 16;                    // 16-byte chunks per row
  constexpr int EPC = 16 / (int)sizeof(O);        // elements per chunk
  const bool one_pass = 256 * RB <= stage_bytes;
  const int rows_per_pass = one_pass ? 256 : 128;
  const int RS = rows_per_pass * (RB + 16) <= stage_bytes ? RB + 16 : RB; // padded when it fits
  const int tid = threadIdx.x;
  for (int h = 0; h < (one_pass ? 1 : 2); ++h) {
    __syncthreads(); // the stage is free
    if (one_pass || wm == h) {
      const int rbase = one_pass ? wm * 128 : 0; // this wave's first staged row
      // FULL: every tile lies inside C (M and N multiples of the tile and
      // compile-time constants), so the operand indices
      // need no clamping and the functor's per-row loads of 4 consecutive
      // rows merge into one vector load
      auto stage_tiles = [&](auto full_c) {
        constexpr bool FULL = decltype(full_c)::value;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          typename Epi::row_t rv[16];
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int64_t m = m0 + wm * 128 + i * 32 + 8 * (r / 4) + 4 * (lane / 32) + r % 4;
            rv[r] = Epi::row(FULL || m < M ? m : M - 1, P);
          }
#pragma unroll
          for (int j = 0; j < JT; ++j) {
            const int col = wn * (32 * JT) + j * 32 + lane % 32;
            const int64_t n = n0 + col;
            const typename Epi::col_t cv = Epi::col(FULL || n < N ? n : N - 1, P);
            acc_t a = acc[i][j];
            asm volatile("" : "+a"(a)::"memory"); // one tile in VGPRs at a time
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int row = i * 32 + 8 * (r / 4) + 4 * (lane / 32) + r % 4;
              const int64_t m = m0 + wm * 128 + row;
              // rows and columns past C are staged (from clamped operand
              // indices) but never stored
              *reinterpret_cast<O *>(stage + (rbase + row) * RS + col * (int)sizeof(O)) =
                  Epi::apply(a[r], FULL || m < M ? m : M - 1, FULL || n < N ? n : N - 1, rv[r], cv, P);
            }
          }
        }
      };
      // (a runtime M keeps one epilogue: both would not fit the registers)
      if (__builtin_constant_p(M) && __builtin_constant_p(N) && M % 256 == 0 && N % 256 == 0)
        stage_tiles(std::true_type{});
      else
        stage_tiles(std::false_type{});
    }
    __syncthreads();
    const int64_t mrow0 = m0 + (one_pass ? 0 : h * 128);
#pragma unroll 4
    for (int c = tid; c < rows_per_pass * CPR; c += NT) {
      const int row = c / CPR, ch = c % CPR;
      const int64_t m = mrow0 + row, n = n0 + (int64_t)ch * EPC;
      if (m >= M) continue;
      const v4i v = *reinterpret_cast<const v4i *>(stage + row * RS + ch * 16);
      if (n + EPC <= N) {
        __builtin_nontemporal_store(v, reinterpret_cast<v4i *>(out + m * N + n));
      } else {
        const O *e = reinterpret_cast<const O *>(&v);
        for (int k = 0; k < EPC && n + k < N; ++k) out[m * N + n + k] = e[k];
      }
    }
  }
}

template <int MK, typename Epi, bool AT, bool BT, typename ElemT, typename Args>
__device__ void mmad_core(const ElemT *__restrict__ A, const ElemT *__restrict__ B, typename Epi::out_t *__restrict__ out,
                          int64_t M, int64_t N, int64_t K, const Args &P) {
  using Op = MfmaOp<MK>;
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
  if constexpr (!AT) mm_load_kmajor(A, M, m0, Kb, 0, ra);
  else mm_load_nmajor<ESZ>(reinterpret_cast<const char *>(A), M, K, m0, 0, ra);
  if constexpr (BT) mm_load_kmajor(B, N, n0, Kb, 0, rb);
  else mm_load_nmajor<ESZ>(reinterpret_cast<const char *>(B), N, K, n0, 0, rb);
  if constexpr (!AT) mm_store_kmajor(lds[0][0], ra);
  else mm_store_nmajor<ESZ>(lds[0][0], ra);
  if constexpr (BT) mm_store_kmajor(lds[0][1], rb);
  else mm_store_nmajor<ESZ>(lds[0][1], rb);
  __syncthreads();

  const int nsteps = (int)((Kb + MM_BK - 1) / MM_BK);
  for (int s = 0; s < nsteps; ++s) {
    const int cur = s & 1;
    const bool more = s + 1 < nsteps;
    if (more) {
      const int64_t k0 = (int64_t)(s + 1) * MM_BK;
      if constexpr (!AT) mm_load_kmajor(A, M, m0, Kb, k0, ra);
      else mm_load_nmajor<ESZ>(reinterpret_cast<const char *>(A), M, K, m0, k0, ra);
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
      if constexpr (!AT) mm_store_kmajor(lds[cur ^ 1][0], ra);
      else mm_store_nmajor<ESZ>(lds[cur ^ 1][0], ra);
      if constexpr (BT) mm_store_kmajor(lds[cur ^ 1][1], rb);
      else mm_store_nmajor<ESZ>(lds[cur ^ 1][1], rb);
    }
    __syncthreads();
  }

  mm_epilogue<Epi>(acc, out, M, N, m0, n0, wm, wn, lane, P);
}

// ---- DMA path --------------------------------------------------------------
// LDS layout of one operand slice (256 rows x 64 bytes = 1024 granules of 16
// bytes): granule g of row r sits at position 4r + (g ^ ((r >> 2) & 3)).  A
// fragment read touches one logical granule of 32 consecutive rows, and any
// 16 consecutive rows then cover all 16 granule slots of a 256-byte bank
// line.  global_load_lds_dwordx4 writes lane l of a wave to position
// base + l, so the swizzle is applied by choosing which global granule each
// lane fetches.
constexpr int MMD_STAGES = 4;
constexpr int MMD_SLICE = 256 * 64;  // bytes per operand per stage

__device__ __forceinline__ void mmd_dma16(const void *g, uint32_t lds_addr) {
  // M0 holds the wave's LDS destination; written here and read by the next
  // instruction only
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds_addr) : "memory");
}

// 16 bytes per lane from the wave-uniform base + the lane's 32-bit offset
// into LDS at M0 + 16 * lane
__device__ __forceinline__ void mmd_dma16_off(const char *base, uint32_t off, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds_addr) : "memory");
}
// 4 bytes per lane into LDS at M0 + 4 * lane
__device__ __forceinline__ void mmd_dma4(const void *g, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(lds_addr) : "memory");
}
template <int N> __device__ __forceinline__ void mmd_wait_vm() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }

// Issues this wave's 4 DMA instructions (rows 64*wave .. +63) of one operand
// slice: rows row0.., K bytes k0..k0+63; rows past `rows` re-read the last row.
__device__ __forceinline__ void mmd_issue_operand(const char *__restrict__ base, int64_t rows, int64_t row0, int64_t Kbytes,
                                                  int64_t k0, uint32_t lds_slice) {
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int blk = wave * 4 + i;            // 1 KB block: rows 16*blk .. +15
    const int r = 16 * blk + lane / 4;
    const int g = (lane % 4) ^ ((r >> 2) & 3);
    int64_t row = row0 + r;
    row = row < rows ? row : rows - 1;
    mmd_dma16(base + row * Kbytes + k0 + g * 16, __builtin_amdgcn_readfirstlane(lds_slice + blk * 1024));
  }
}

template <int MK, typename Epi, typename ElemT, typename Args>
__device__ void mmad_core_dma(const ElemT *__restrict__ A, const ElemT *__restrict__ B, typename Epi::out_t *__restrict__ out,
                              int64_t M, int64_t N, int64_t K, const Args &P) {
  using Op = MfmaOp<MK>;
  using acc_t = typename Op::acc_t;
  constexpr int ESZ = sizeof(ElemT);
  __shared__ __attribute__((aligned(1024))) char lds[MMD_STAGES][2][MMD_SLICE]; // [stage][A/B]
  const int tmt = (int)((M + MM_TM - 1) / MM_TM), tnt = (int)((N + MM_TN - 1) / MM_TN);
  int ti, tj;
  mm_tile_of(blockIdx.x, tmt, tnt, ti, tj);
  const int64_t m0 = (int64_t)ti * MM_TM, n0 = (int64_t)tj * MM_TN;
  const int64_t Kb = K * ESZ;
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int wm = wave / 2, wn = wave % 2;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)&lds[0][0][0];
  const char *Ab = reinterpret_cast<const char *>(A), *Bb = reinterpret_cast<const char *>(B);
  const int nsteps = (int)(Kb / 64);

  // every step issues the same number of DMAs (8 per wave), so one fixed
  // vmcnt finds a stage complete; steps past the end re-read the last slice
  // into a ring slot that is never read again
  auto issue = [&](int s) {
    const int sk = s < nsteps ? s : nsteps - 1;
    const uint32_t st = lds0 + (uint32_t)((s % MMD_STAGES) * 2 * MMD_SLICE);
    mmd_issue_operand(Ab, M, m0, Kb, (int64_t)sk * 64, st);
    mmd_issue_operand(Bb, N, n0, Kb, (int64_t)sk * 64, st + MMD_SLICE);
  };
  // one of the 8 DMA instructions of stage s (d < 4: A, else B)
  auto issue_one = [&](int s, int d) {
    const int sk = s < nsteps ? s : nsteps - 1;
    const uint32_t st = lds0 + (uint32_t)((s % MMD_STAGES) * 2 * MMD_SLICE) + (d < 4 ? 0u : (uint32_t)MMD_SLICE);
    const int blk = wave * 4 + (d & 3);
    const int r = 16 * blk + lane / 4;
    const int g = (lane % 4) ^ ((r >> 2) & 3);
    const int64_t rows = d < 4 ? M : N, row0 = d < 4 ? m0 : n0;
    int64_t row = row0 + r;
    row = row < rows ? row : rows - 1;
    mmd_dma16((d < 4 ? Ab : Bb) + row * Kb + (int64_t)sk * 64 + g * 16, __builtin_amdgcn_readfirstlane(st + blk * 1024));
  };

  acc_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = acc_t{};

  // fragment of MFMA tile row/col block `blk` (32 rows), logical granule g
  auto frag = [&](const char *slice, int blk, int g) -> v4i {
    const int r = blk * 32 + lane % 32;
    return *reinterpret_cast<const v4i *>(slice + (4 * r + (g ^ ((r >> 2) & 3))) * 16);
  };
  // all 16 fragments (2 k-halves x (4 A + 4 B)) of one stage
  auto fetch = [&](int stage, v4i (&f)[2][8]) {
    const char *la = lds[stage % MMD_STAGES][0], *lb = lds[stage % MMD_STAGES][1];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
#pragma unroll
      for (int i = 0; i < 4; ++i) f[q][i] = frag(la, wm * 4 + i, 2 * q + lane / 32);
#pragma unroll
      for (int j = 0; j < 4; ++j) f[q][4 + j] = frag(lb, wn * 4 + j, 2 * q + lane / 32);
    }
  };
  auto mfmas = [&](const v4i (&f)[2][8]) {
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = Op::run(f[q][i], f[q][4 + j], acc[i][j]);
  };
  // Step s: the fragments of stage s are already in registers; the wave
  // multiplies them while it reads stage s+1's fragments into the other set,
  // so the matrix core never waits on LDS.  The barrier at the top of step s
  // makes stage s+1 visible and frees the slot of stage s (its fragments were
  // read during step s-1) for the DMA of stage s+4: three stages are in
  // flight while one is multiplied.
  auto step = [&](int s, const v4i (&cur)[2][8], v4i (&nxt)[2][8]) {
    __builtin_amdgcn_sched_barrier(0);
    mmd_wait_vm<16>();   // this wave's DMAs of stage s+1 are complete
    __syncthreads();     // everyone's are; stage s is no longer read
    // 8 groups: one DMA of stage s+4, two fragment reads of stage s+1, four
    // MFMAs of stage s -- a DMA that waits for a free memory queue slot
    // then holds back at most one group's MFMAs
    const char *la = lds[(s + 1) % MMD_STAGES][0], *lb = lds[(s + 1) % MMD_STAGES][1];
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      __builtin_amdgcn_sched_barrier(0);
      issue_one(s + 4, g);
      const int q = g / 4, i = g % 4;
      nxt[q][i] = frag(la, wm * 4 + i, 2 * q + lane / 32);
      nxt[q][4 + i] = frag(lb, wn * 4 + i, 2 * q + lane / 32);
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = Op::run(cur[q][i], cur[q][4 + j], acc[i][j]);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  issue(0);
  issue(1);
  issue(2);
  mmd_wait_vm<16>();     // stage 0 (this wave)
  __syncthreads();
  issue(3);
  v4i f0[2][8], f1[2][8];
  fetch(0, f0);
#pragma unroll 1
  for (int s = 0; s < nsteps; s += 2) {
    step(s, f0, f1);
    if (s + 1 >= nsteps) break;
    step(s + 1, f1, f0);
  }
  mmd_wait_vm<0>();      // drain the trailing re-reads before the LDS is reused
  mm_epilogue_lds<Epi>(acc, out, M, N, m0, n0, wm, wn, lane, P, &lds[0][0][0], (int)sizeof(lds));
}

// ---- DMA path, 128-byte K slices --------------------------------------------
// Same tile and MFMA layout as above, but each stage carries 128 bytes of K
// per row: every row read is a whole 128-byte line, which on gfx950 feeds a
// CU about 1.5x faster than 64-byte halves (the per-CU feed is bounded by the
// L1's outstanding requests).  Two stages of 2 x 32 KB (mmad_core_pp below).
// Slice layout: 256 rows x 8 granules of 16 bytes; logical granule g of row r
// sits at 8r + (g ^ ((r >> 1) & 7)), so the 16 lanes a ds_read_b128 serves
// per cycle (16 consecutive rows, one logical granule) cover 16 distinct
// 4-bank groups.  A DMA instruction writes 8 rows (lane l -> row l/8,
// position l%8), and each lane fetches the global granule that belongs there.
constexpr int MMD2_SLICE = 256 * 128;

// ---- DMA path, 128-byte K slices, two waves per SIMD -------------------------
// With one wave per SIMD, a DMA that waits for a free memory-queue slot also
// holds back that wave's MFMAs, so feed and multiply add up instead of
// overlapping.  Here 8 waves (512 threads) share the 256x256 tile, two per
// SIMD, each 128 rows x 64 columns (4 x 2 MFMA tiles, 128 accumulator
// registers): while one wave of a SIMD waits on memory, the other issues
// MFMAs.  Ring: two stages of 128-byte K slices, swizzled as described above;
// each wave issues 8 DMAs per stage (its 32 rows of A and of B).
// BKN: B is [K, N] (linalg.matmul; int8, fp8, or bf16 / f16 with 64 k-rows of
// 512 bytes per stage as below): a byte stage of B is 128 k-rows x 256
// columns, each DMA instruction 4 whole 256-byte k-rows, kept K-major in LDS
// (granule g of k-row r at position g ^ kn_swz(r), so the 8 k-rows x 2
// granules one half-wave reads sit on 16 different positions).  A B fragment is read with
// two ds_read_b64_tr_b8: in each group of 16 lanes, lane i's byte b comes from
// the 8 bytes addressed by lane 2b + i/8, byte i % 8; so lane j addressing
// k-row k0 + j/2 at column c0 + 8 (j % 2) gives lane i the column c0 + i at
// k-rows k0 .. k0+7 -- eight consecutive k-bytes of one column, as the matrix
// core takes them.
// Block-scaled fp8 (MK_MX..): B [K, N] as above; SA [M, K/32] and SB
// [N, K/32] hold the e8m0 scales.  One 128-byte slice is 2 scaled MFMAs of
// 64 k per tile, each taking the int8 path's fragments of two k-blocks.  The
// slice's scales (bytes 4s .. 4s+3 of each row: 1 KB for the tile's 256 A
// rows, 1 KB for its 256 B columns) ride the same ring, one 4-byte-per-lane
// DMA per wave per stage, so every load of a stage is covered by the ring's
// own wait.  Block-scaled fp4 (MK_MX4): a 128-byte slice holds 256 k, four
// scaled fp4 MFMAs of 64 k per tile, each taking the int8 path's fragment of
// one k-block (16 bytes, 32 k per lane); the slice's scales are 8 bytes of
// each row, two 4-byte DMAs per wave per stage into two planes.
// AKM: A is [K, M] (hivm a_transpose), staged and read exactly as a [K, N] B
// (its M columns in place of N).
template <int MK, typename Epi, bool BKN, bool AKM = false, typename ElemT, typename Args>
__device__ void mmad_core_pp(const ElemT *__restrict__ A, const ElemT *__restrict__ B, typename Epi::out_t *__restrict__ out,
                             int64_t M, int64_t N, int64_t K, const Args &P, const uint8_t *__restrict__ SA = nullptr,
                             const uint8_t *__restrict__ SB = nullptr) {
  constexpr bool MX = mk_is_mx(MK), FP4 = mk_is_fp4(MK);
  constexpr int NW = FP4 ? 2 : 1; // scale words per row per stage (32 k per byte)
  static_assert(!AKM || !MX, "block-scaled A is [M, K]");
  static_assert(!(BKN || AKM) || (((MK == MK_I8 || MX) && sizeof(ElemT) == 1) ||
                                  ((MK == MK_BF16 || MK == MK_F16) && sizeof(ElemT) == 2)),
                "the K-major operand path takes bytes or 16-bit floats");
  static_assert(!MX || BKN, "block-scaled operands come with B [K, N]");
  using Op = typename std::conditional<MX, MfmaMx<(MX ? MK : MK_MX)>, MfmaOp<(MX ? MK_I8 : MK)>>::type;
  using acc_t = typename Op::acc_t;
  constexpr int ESZ = sizeof(ElemT);
  __shared__ __attribute__((aligned(1024))) char lds[2][2][MMD2_SLICE]; // [stage][A/B]
  __shared__ __attribute__((aligned(1024))) uint32_t lds_sc[MX ? 2 : 1][2 * NW][MX ? 256 : 1]; // [stage][A/B x word][row]
  const int tmt = (int)((M + MM_TM - 1) / MM_TM), tnt = (int)((N + MM_TN - 1) / MM_TN);
  int ti, tj;
  mm_tile_of(blockIdx.x, tmt, tnt, ti, tj);
  const int64_t m0 = (int64_t)ti * MM_TM, n0 = (int64_t)tj * MM_TN;
  const int64_t Kb = K * ESZ;
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int wm = wave / 4, wn = wave % 4; // waves w and w+4 share a SIMD
  constexpr int DPS = 8 + (MX ? NW : 0); // DMA instructions per wave per stage
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)&lds[0][0][0];
  const char *Ab = reinterpret_cast<const char *>(A), *Bb = reinterpret_cast<const char *>(B);
  const int nsteps = (int)(Kb / 128);
  auto kn_swz = [](int kr) { return ((kr & 7) << 1) | ((kr >> 3) & 1); };
  // 16-bit [K, N]: the 4 k-rows of one transposing read on 4 different
  // 64-byte bank groups
  auto kn16_swz = [](int kr) { return (kr & 3) << 2; };

  // DMA d (0..7) of K slice s into ring slot `slot`: d < 4 this wave's A
  // rows (32 * wave ..), else its B rows, 8 rows per instruction.  Each lane's
  // source is a 32-bit offset, fixed for the whole loop, from a wave-uniform
  // base that advances by one K slice per step, so a step's DMAs cost no
  // vector address arithmetic.
  //   row-major operand: offset (row - row0) * Kb + 16 g from the tile's
  //     first row (rows past the end re-read the last row);
  //   K-major operand (int8): 4 k-rows of 256 columns per instruction, lane l
  //     filling position l % 16 of k-row 4 blk + l / 16 with logical granule
  //     (l % 16) ^ kn_swz(k-row); offset k-row * cols + column from the
  //     slice's first k-row (columns past the end re-read valid bytes,
  //     masked later);
  //   K-major 16-bit: a 128-byte slice is 64 k-rows of 512 bytes, lane l
  //     filling position l % 32 of k-row 2 blk + l / 32 with logical granule
  //     (8 columns) (l % 32) ^ kn16_swz(k-row).
  // The lowering keeps these offsets below 2^32 (256 rows of K bytes, or
  // 128 bytes' worth of k-rows).
  uint32_t dofs[8];
#pragma unroll
  for (int d = 0; d < 8; ++d) {
    const int blk = wave * 4 + (d & 3);
    const bool kmaj = d >= 4 ? BKN : AKM; // this operand is stored [K, columns]
    if (kmaj) {
      const int64_t cols = d >= 4 ? N : M, c0 = d >= 4 ? n0 : m0;
      if constexpr (ESZ == 1) {
        const int kr = 4 * blk + lane / 16;
        const int gg = (lane % 16) ^ kn_swz(kr);
        int64_t col = c0 + 16 * gg;
        col = col + 16 <= cols ? col : cols - 16;
        dofs[d] = (uint32_t)(kr * cols + col);
      } else {
        const int kr = 2 * blk + lane / 32;
        const int gg = (lane % 32) ^ kn16_swz(kr);
        int64_t col = c0 + 8 * gg;
        col = col + 8 <= cols ? col : cols - 8;
        dofs[d] = (uint32_t)((kr * cols + col) * 2);
      }
    } else {
      const int r = 8 * blk + lane / 8;
      const int g = (lane % 8) ^ ((r >> 1) & 7);
      const int64_t rows = d < 4 ? M : N, row0 = d < 4 ? m0 : n0;
      int64_t row = row0 + r;
      row = row < rows ? row : rows - 1;
      dofs[d] = (uint32_t)((row - row0) * Kb + g * 16);
    }
  }
  const char *const dbase[2] = {AKM ? Ab : Ab + m0 * Kb, BKN ? Bb : Bb + n0 * Kb};
  const int64_t dstride[2] = {AKM ? 128 * M : 128, BKN ? 128 * N : 128};
  auto issue_one = [&](int s, int slot, int d) {
    const uint32_t st = lds0 + (uint32_t)(slot * 2 * MMD2_SLICE) + (d < 4 ? 0u : (uint32_t)MMD2_SLICE) +
                        (uint32_t)((wave * 4 + (d & 3)) * 1024);
    mmd_dma16_off(dbase[d >= 4] + (int64_t)s * dstride[d >= 4], dofs[d], __builtin_amdgcn_readfirstlane(st));
  };
  // the scales of K slice s: wave w carries 64 rows (w < 4: A rows 64 w ..,
  // else B columns 64 (w - 4) ..), 4 bytes each (fp4: 8 bytes, as two words
  // in two planes); a row of scales has K/32 bytes (fp4: K/16, K in bytes)
  const uint32_t lds_sc0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint32_t *)&lds_sc[0][0][0];
  auto issue_scales = [&](int s, int slot) {
    if constexpr (MX) {
      const int op = wave / 4, r = 64 * (wave % 4) + lane;
      const int64_t rows = op ? N : M, row0 = op ? n0 : m0;
      int64_t row = row0 + r;
      row = row < rows ? row : rows - 1;
#pragma unroll
      for (int w = 0; w < NW; ++w)
        mmd_dma4((op ? SB : SA) + row * (K / (32 / NW)) + 4 * NW * (int64_t)s + 4 * w,
                 __builtin_amdgcn_readfirstlane(lds_sc0 + (uint32_t)(((slot * 2 + op) * NW + w) * 1024 + 256 * (wave % 4))));
    }
  };
  auto issue_stage = [&](int s) {
#pragma unroll
    for (int d = 0; d < 8; ++d) issue_one(s < nsteps ? s : nsteps - 1, s & 1, d);
    issue_scales(s < nsteps ? s : nsteps - 1, s & 1);
  };

  acc_t acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = acc_t{};

  auto frag = [&](const char *slice, int blk, int g) -> v4i {
    const int r = blk * 32 + lane % 32;
    return *reinterpret_cast<const v4i *>(slice + (8 * r + (g ^ ((r >> 1) & 7))) * 16);
  };
  // B fragment from the K-major slice: 32 columns blk * 32 .., k-block kb
  auto frag_kn = [&](const char *slice, int blk, int kb) -> v4i {
    const int q = lane / 16, j = lane % 16;
    const int col = blk * 32 + 16 * (q % 2) + 8 * (j % 2);
    v4i r;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int kr = kb * 32 + 16 * (q / 2) + 8 * h + j / 2;
      const int pos = kr * 256 + (((col >> 4) ^ kn_swz(kr)) << 4) + (col & 15);
      typedef int v2i_ __attribute__((ext_vector_type(2)));
      const v2i_ t = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
          (__attribute__((address_space(3))) v2i_ *)(uintptr_t)((uint32_t)(uintptr_t)(__attribute__((address_space(3))) const char *)slice + pos));
      r[2 * h] = t.x;
      r[2 * h + 1] = t.y;
    }
    return r;
  };
  // 16-bit B fragment from the K-major slice: columns blk * 32 .., k-block
  // kb (16 k).  ds_read_b64_tr_b16: in each group of 16 lanes, lane i's
  // element e is element i % 4 of the 4 addressed by lane 4 e + i / 4, so
  // lane j addressing k-row k0 + j / 4 at column c0 + 4 (j % 4) gives lane i
  // the column c0 + i at k-rows k0 .. k0+3 (measured on gfx950)
  auto frag_kn16 = [&](const char *slice, int blk, int kb) -> v4i {
    const int q = lane / 16, j = lane % 16;
    const int col = blk * 32 + 16 * (q % 2) + 4 * (j % 4);
    v4i r;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int kr = kb * 16 + 8 * (q / 2) + 4 * h + j / 4;
      const int pos = kr * 512 + (((col >> 3) ^ kn16_swz(kr)) << 4) + (col & 7) * 2;
      typedef short v4s_ __attribute__((ext_vector_type(4)));
      const v4s_ t = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) v4s_ *)(uintptr_t)((uint32_t)(uintptr_t)(__attribute__((address_space(3))) const char *)slice + pos));
      typedef int v2i_ __attribute__((ext_vector_type(2)));
      const v2i_ u = __builtin_bit_cast(v2i_, t);
      r[2 * h] = u.x;
      r[2 * h + 1] = u.y;
    }
    return r;
  };
  // the 12 fragments (2 k-blocks x (4 A + 2 B)) of half h of stage s
  auto fetch = [&](int s, int h, v4i (&f)[2][6]) {
    const char *la = lds[s & 1][0], *lb = lds[s & 1][1];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        f[q][i] = !AKM ? frag(la, wm * 4 + i, 4 * h + 2 * q + lane / 32)
                  : ESZ == 1 ? frag_kn(la, wm * 4 + i, 2 * h + q) : frag_kn16(la, wm * 4 + i, 2 * h + q);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        f[q][4 + j] = !BKN ? frag(lb, wn * 2 + j, 4 * h + 2 * q + lane / 32)
                      : ESZ == 1 ? frag_kn(lb, wn * 2 + j, 2 * h + q) : frag_kn16(lb, wn * 2 + j, 2 * h + q);
    }
  };

  // this lane's scale words for stage s, shifted so that byte 2h is the scale
  // of its k-half in half h of the slice (fp4: word w, byte 2q, of its
  // k-half in k-block 2w + q; word 1 is read for the second half, after the
  // first half's fragments are dead)
  uint32_t sa_w[4], sb_w[2];
  auto read_scales = [&](int s, int w) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      sa_w[i] = lds_sc[MX ? (s & 1) : 0][w][MX ? wm * 128 + i * 32 + lane % 32 : 0] >> (8 * (lane / 32));
#pragma unroll
    for (int j = 0; j < 2; ++j)
      sb_w[j] = lds_sc[MX ? (s & 1) : 0][NW + w][MX ? (wn * 2 + j) * 32 + lane % 32 : 0] >> (8 * (lane / 32));
  };

  // Step s: wait for stage s (stage s+1 may be in flight); multiply its first
  // half while reading the second half's fragments; after a barrier (all of
  // stage s is in registers everywhere) issue stage s+2 into the freed slot
  // while the second half is multiplied.
  v4i f0[2][6], f1[2][6];
  issue_stage(0);
  issue_stage(1);
#pragma unroll 1
  for (int s = 0; s < nsteps; ++s) {
    __builtin_amdgcn_sched_barrier(0);
    mmd_wait_vm<DPS>();
    __syncthreads();
    fetch(s, 0, f0);
    fetch(s, 1, f1);
    if constexpr (FP4) {
      // k-blocks 0 and 1 of the slice: one scaled fp4 MFMA each
      read_scales(s, 0);
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = q == 0 ? Op::template run<0>(mx_lo(f0[0][i]), mx_lo(f0[0][4 + j]), acc[i][j], (int)sa_w[i], (int)sb_w[j])
                               : Op::template run<2>(mx_lo(f0[1][i]), mx_lo(f0[1][4 + j]), acc[i][j], (int)sa_w[i], (int)sb_w[j]);
    } else if constexpr (MX) {
      read_scales(s, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = Op::template run<0>(mx_cat(f0[0][i], f0[1][i]), mx_cat(f0[0][4 + j], f0[1][4 + j]), acc[i][j],
                                          (int)sa_w[i], (int)sb_w[j]);
    } else {
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[i][j] = Op::run(f0[q][i], f0[q][4 + j], acc[i][j]);
    }
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads(); // every wave holds stage s in registers: its slot is free
    const int s2 = s + 2 < nsteps ? s + 2 : nsteps - 1;
    if constexpr (FP4) {
      // k-blocks 2 and 3
      read_scales(s, 1);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          __builtin_amdgcn_sched_barrier(0);
          issue_one(s2, s & 1, i * 2 + j);
          acc[i][j] = Op::template run<0>(mx_lo(f1[0][i]), mx_lo(f1[0][4 + j]), acc[i][j], (int)sa_w[i], (int)sb_w[j]);
          acc[i][j] = Op::template run<2>(mx_lo(f1[1][i]), mx_lo(f1[1][4 + j]), acc[i][j], (int)sa_w[i], (int)sb_w[j]);
        }
      issue_scales(s2, s & 1);
    } else if constexpr (MX) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          __builtin_amdgcn_sched_barrier(0);
          issue_one(s2, s & 1, i * 2 + j);
          acc[i][j] = Op::template run<2>(mx_cat(f1[0][i], f1[1][i]), mx_cat(f1[0][4 + j], f1[1][4 + j]), acc[i][j],
                                          (int)sa_w[i], (int)sb_w[j]);
        }
      issue_scales(s2, s & 1);
    } else {
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          __builtin_amdgcn_sched_barrier(0);
          issue_one(s2, s & 1, q * 4 + i);
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[i][j] = Op::run(f1[q][i], f1[q][4 + j], acc[i][j]);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  mmd_wait_vm<0>();
  __syncthreads();
  mm_epilogue_lds<Epi, 2, 512>(acc, out, M, N, m0, n0, wm, wn, lane, P, &lds[0][0][0], (int)sizeof(lds));
}

// [R, C] row-major operand of ESZ-byte elements -> its [C, R] transpose, one
// tile of 128 bytes x 128 bytes (T = 128 / ESZ elements each way) per
// workgroup of 256 threads, staged through LDS: every global read is a whole
// 128-byte line segment, so no line is fetched by two workgroups (both row
// lengths span a multiple of 16 bytes; ragged edges are masked in 16-byte
// chunks).  Used to re-lay a [K, N] (or [K, M]) matmul operand K-contiguous
// ahead of the DMA ring.  Bytes (ESZ 1): each thread reads a 16-row x 4-column
// block as 16 dwords and transposes it in registers (v_perm); wider elements
// are gathered element by element.
// matmul_mx operands to bf16 for the exact contraction (compiler option
// mx_exact=1): element (r, c) of a [R, C] byte operand in fp8 format FMT
// becomes fp8(v) * 2^(s - 127), with s the e8m0 scale of its row r
// (ROWSCALE, A [M, K]: k = c) or of its column c (B [K, N]: k = r), one per
// 32 k (scale row length K/32); e8m0 255 gives NaN.  The scaled value has at
// most 3 significant bits, so it is exact in bf16 wherever its exponent is
// inside bf16's normal range (the range of f32).  Eight bytes per thread
// and step, 16-byte stores.
template <int FMT, bool ROWSCALE>
__device__ __forceinline__ void mx_to_bf16(const uint8_t *__restrict__ src, const uint8_t *__restrict__ sc,
                                           uint16_t *__restrict__ dst, int64_t R, int64_t C, int64_t K) {
  const int64_t n8 = R * C / 8, ks = K / 32;
  if constexpr (!ROWSCALE) {
    // B [K, N]: a thread owns 8 columns of 8 rows inside one 32-row scale
    // block; their 8 scales are loaded once for the 8 rows
    const int64_t cg = C / 8, items = (R / 8) * cg;
    for (int64_t it = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; it < items; it += (int64_t)gridDim.x * blockDim.x) {
      const int64_t r8 = it / cg, kb = r8 / 4, c0 = (it % cg) * 8;
      int sx[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) sx[j] = sc[(c0 + j) * ks + kb];
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int64_t e0 = (r8 * 8 + r) * C + c0;
        const uint2 w = *reinterpret_cast<const uint2 *>(src + e0);
        uint16_t o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint8_t b = (uint8_t)((j < 4 ? w.x : w.y) >> (8 * (j % 4)));
          const float f = sx[j] == 255 ? __builtin_nanf("") : __builtin_ldexpf(fp8_to_f32<FMT>(b), sx[j] - 127);
          o[j] = f32_to_bf16_rne(f);
        }
        uint4 v;
        __builtin_memcpy(&v, o, 16);
        *reinterpret_cast<uint4 *>(dst + e0) = v;
      }
    }
    return;
  }
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t e0 = i * 8, r = e0 / C, c0 = e0 % C;
    const uint2 w = *reinterpret_cast<const uint2 *>(src + e0);
    uint16_t o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint8_t b = (uint8_t)((j < 4 ? w.x : w.y) >> (8 * (j % 4)));
      const int64_t c = c0 + j;
      const uint8_t s = ROWSCALE ? sc[r * ks + c / 32] : sc[c * ks + r / 32];
      const float f = s == 255 ? __builtin_nanf("") : __builtin_ldexpf(fp8_to_f32<FMT>(b), (int)s - 127);
      o[j] = f32_to_bf16_rne(f);
    }
    uint4 v;
    __builtin_memcpy(&v, o, 16);
    *reinterpret_cast<uint4 *>(dst + e0) = v;
  }
}

template <int ESZ>
__device__ __forceinline__ void mm_transpose(const char *__restrict__ src, char *__restrict__ dst, int64_t R, int64_t C) {
  constexpr int T = 128 / ESZ, CH = 8, EPC = 16 / ESZ, PITCH = 136; // row pitch: the two half-waves' rows on other banks
  __shared__ __attribute__((aligned(16))) char tile[T][PITCH];
  const int64_t tilesC = (C + T - 1) / T;
  const int64_t r0 = (int64_t)(blockIdx.x / tilesC) * T, c0 = (int64_t)(blockIdx.x % tilesC) * T;
  for (int i = threadIdx.x; i < T * CH; i += 256) {
    const int r = i / CH, ch = i % CH;
    const int64_t gr = r0 + r, gc = c0 + (int64_t)ch * EPC;
    v4i v = {0, 0, 0, 0};
    if (gr < R && gc < C) v = *reinterpret_cast<const v4i *>(src + (gr * C + gc) * ESZ);
    uint2 *t2 = reinterpret_cast<uint2 *>(&tile[r][ch * 16]);
    t2[0] = make_uint2((uint32_t)v[0], (uint32_t)v[1]);
    t2[1] = make_uint2((uint32_t)v[2], (uint32_t)v[3]);
  }
  __syncthreads();
  if constexpr (ESZ == 1) {
    // columns 4 c4 .. +3, rows 16 rb .. +15; eight consecutive lanes (rb) hold
    // one destination row's 128 bytes, so each 16-byte store instruction
    // writes whole lines
    const int rb = threadIdx.x % 8, c4 = threadIdx.x / 8;
    uint32_t d[16];
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) d[rr] = *reinterpret_cast<const uint32_t *>(&tile[16 * rb + rr][4 * c4]);
    uint32_t o[4][4]; // o[t][w]: column 4 c4 + t, rows 16 rb + 4w .. +3
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t lo01 = __builtin_amdgcn_perm(d[4 * w + 1], d[4 * w], 0x05010400u);
      const uint32_t hi01 = __builtin_amdgcn_perm(d[4 * w + 1], d[4 * w], 0x07030602u);
      const uint32_t lo23 = __builtin_amdgcn_perm(d[4 * w + 3], d[4 * w + 2], 0x05010400u);
      const uint32_t hi23 = __builtin_amdgcn_perm(d[4 * w + 3], d[4 * w + 2], 0x07030602u);
      o[0][w] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);
      o[1][w] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);
      o[2][w] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
      o[3][w] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
    }
    const int64_t gr = r0 + 16 * rb;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int64_t gc = c0 + 4 * c4 + t;
      if (gc < C && gr < R)
        *reinterpret_cast<v4i *>(dst + gc * R + gr) = v4i{(int)o[t][0], (int)o[t][1], (int)o[t][2], (int)o[t][3]};
    }
  } else {
    for (int i = threadIdx.x; i < T * CH; i += 256) {
      const int c = i / CH, ch = i % CH;
      const int64_t gc = c0 + c, gr = r0 + (int64_t)ch * EPC;
      if (gc >= C || gr >= R) continue;
      union { v4i v; char b[16]; } u;
#pragma unroll
      for (int e = 0; e < EPC; ++e)
#pragma unroll
        for (int b = 0; b < ESZ; ++b) u.b[e * ESZ + b] = tile[ch * EPC + e][c * ESZ + b];
      *reinterpret_cast<v4i *>(dst + (gc * R + gr) * ESZ) = u.v;
    }
  }
}

// Entry: MK selects the matrix-core kind; A is [M, K] (or [K, M] with AT), B is
// [N, K] with BT (the weight layout) or [K, N]; DMA selects the LDS DMA ring:
// 0 none (register staging), 1 with 64-byte K slices (256 threads), 3 with
// 128-byte slices and two waves per SIMD (512 threads); both require !AT, BT
// and K spanning a multiple of 64 resp. 128 bytes; 4 as 3 with a B [K, N]
// (!BT) and / or an A [K, M] (AT), rows of a multiple of 16 bytes, staged
// K-major and read by transposing LDS reads.
template <int MK, typename Epi, bool AT, bool BT, int DMA, typename ElemT, typename Args>
__device__ __forceinline__ void mmad(const ElemT *A, const ElemT *B, typename Epi::out_t *out, int64_t M, int64_t N, int64_t K,
                                     const Args &P) {
  static_assert(DMA == 0 || DMA == 4 || (!AT && BT), "the DMA rings 1 and 3 take K-contiguous A and B");
  static_assert(DMA == 0 || DMA == 1 || DMA == 3 || DMA == 4, "DMA mode");
  if constexpr (DMA == 4) mmad_core_pp<MK, Epi, !BT, AT>(A, B, out, M, N, K, P);
  else if constexpr (mk_is_mx(MK)) static_assert(DMA == 4, "block-scaled kinds run on the [K, N] ring");
  else if constexpr (DMA == 3) mmad_core_pp<MK, Epi, false>(A, B, out, M, N, K, P);
  else if constexpr (DMA == 1) mmad_core_dma<MK, Epi>(A, B, out, M, N, K, P);
  else mmad_core<MK, Epi, AT, BT>(A, B, out, M, N, K, P);
}

// Block-scaled fp8 / fp4 contraction: A [M, K], B [K, N] (bytes of the
// formats MK encodes; K counts bytes), SA [M, K/32], SB [N, K/32] e8m0 (fp4:
// two values per byte, so [M, K/16] and [N, K/16]); K a multiple of 128, N
// of 16.
template <int MK, typename Epi, typename Args>
__device__ __forceinline__ void mmad_mx(const uint8_t *A, const uint8_t *B, const uint8_t *SA, const uint8_t *SB,
                                        typename Epi::out_t *out, int64_t M, int64_t N, int64_t K, const Args &P) {
  static_assert(mk_is_mx(MK), "block-scaled kind");
  mmad_core_pp<MK, Epi, true>(A, B, out, M, N, K, P, SA, SB);
}

} // namespace hf
