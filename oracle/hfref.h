/*
 * hfref — CPU restatement of BiShengIR's CPU lowering of HFusion op groups.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity oracle: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it, and only as
 * the checker (or the timed CPU baseline).  The product path never links it.
 *
 * What it restates: `lower-for-cpu-runner-pipeline`
 * (bishengir/lib/ExecutionEngine/ExecutionEnginePipelines.cpp:39-90), i.e.
 * every linalg/hfusion structured op becomes a serial scalar loop nest
 * (`convert-linalg-to-loops`, :73) whose body is the op's region as built by
 * RegionBuilderHelper (bishengir/lib/Dialect/HFusion/IR/HFusionOps.cpp:428-862)
 * and then lowered arith/math -> LLVM -> libm on x86-64.
 *
 * Compile with -O2 -ffp-contract=off -fno-fast-math: the CPU lowering emits
 * separate fmul/fadd (no `contract` flag), correctly rounded div/sqrt, and
 * calls glibc expf/logf/... for math.* ops.
 */
#ifndef HFREF_H
#define HFREF_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions (pinned by closed forms in tests) ---- */
float hfref_bf16_to_f32(uint16_t h);
uint16_t hfref_f32_to_bf16(float f);          /* arith.truncf: RNE, NaN stays NaN */
float hfref_f16_to_f32(uint16_t h);
uint16_t hfref_f32_to_f16(float f);           /* arith.truncf: RNE */

/* Declared hfusion.cast semantics (HFusionEnums.td:122-141).
 * mode: 0 rint, 1 round, 2 floor, 3 ceil, 4 trunc, 5 odd, 6 truncwithoverflow */
uint16_t hfref_f32_to_bf16_mode(float f, int mode);
uint16_t hfref_f32_to_f16_mode(float f, int mode);
/* float -> integer of `bits` width (8/16/32/64), declared round mode; saturate
 * clamps to the signed range (NaN -> 0); otherwise two's-complement wrap. */
int64_t hfref_f32_to_int_mode(float f, int mode, int bits, int saturate);
/* signed integer -> f32 with declared round mode */
float hfref_int_to_f32_mode(int64_t v, int mode);
/* the reference constant folder's float->int "odd" (HFusionOps.cpp:1926-1938) */
int64_t hfref_fold_round_to_odd(double x);

/* ---- array primitives used by the IR interpreter (oracle/interp.py) ---- */
/* unary fn codes */
enum {
  HFU_SQRT = 0, HFU_RSQRT, HFU_EXP, HFU_EXP2, HFU_LOG, HFU_LOG2, HFU_LOG10,
  HFU_LOG1P, HFU_EXPM1, HFU_ABS, HFU_NEG, HFU_RELU, HFU_REC, HFU_TANH,
  HFU_SIN, HFU_COS, HFU_ERF, HFU_NEARBYINT, HFU_CEIL, HFU_FLOOR, HFU_ROUND,
  HFU_SQUARE, HFU_TRUNC, HFU_TAN, HFU_ACOS, HFU_ACOSH, HFU_ASIN, HFU_ASINH,
  HFU_ATAN, HFU_ATANH, HFU_SINH, HFU_COSH, HFU_LGAMMA, HFU_ILOGB
};
/* binary fn codes */
enum {
  HFB_ADD = 0, HFB_SUB, HFB_MUL, HFB_DIV, HFB_MAXF, HFB_MINF, HFB_MAXNUMF,
  HFB_MINNUMF, HFB_POWF, HFB_MODF, HFB_COPYSIGN, HFB_ATAN2, HFB_LDEXP,
  HFB_DIVFHP,
  /* integer */
  HFB_IADD = 32, HFB_ISUB, HFB_IMUL, HFB_IDIV, HFB_IMAX, HFB_IMIN, HFB_IAND,
  HFB_IOR, HFB_IXOR, HFB_ISHL, HFB_ISHRS, HFB_ISHRU, HFB_IREM,
  HFB_IFLOORDIV, HFB_ICEILDIV, HFB_IMAXU, HFB_IMINU, HFB_IPOW, HFB_ICEILDIVU,
  HFB_IREMU
};
/* compare fn codes */
enum { HFC_EQ = 0, HFC_NE, HFC_LT, HFC_LE, HFC_GT, HFC_GE };

void hfref_unary_f32(int fn, const float *in, float *out, int64_t n);
void hfref_binary_f32(int fn, const float *a, const float *b, float *out,
                      int64_t n);
void hfref_fma_f32(const float *a, const float *b, const float *c, float *out,
                   int64_t n);
/* integer binary on int64 lanes, result wrapped to `bits` */
void hfref_binary_i64(int fn, const int64_t *a, const int64_t *b,
                      int64_t *out, int64_t n, int bits);
void hfref_compare_f32(int fn, const float *a, const float *b, uint8_t *out,
                       int64_t n);
void hfref_compare_i64(int fn, const int64_t *a, const int64_t *b,
                       uint8_t *out, int64_t n);

/* conversions over arrays */
/* fp8: fmt 0 = f8E4M3FN, 1 = f8E5M2 */
float hfref_fp8_to_f32(uint8_t b, int fmt);
void hfref_fp8_to_f32_n(const uint8_t *in, float *out, int64_t n, int fmt);
void hfref_f32_to_fp8_n(const float *in, uint8_t *out, int64_t n, int fmt, int mode, int sat);
void hfref_int_to_fp8_n(const int64_t *in, uint8_t *out, int64_t n, int fmt, int mode, int sat);
void hfref_bf16_to_f32_n(const uint16_t *in, float *out, int64_t n);
void hfref_f32_to_bf16_n(const float *in, uint16_t *out, int64_t n, int mode);
void hfref_f16_to_f32_n(const uint16_t *in, float *out, int64_t n);
void hfref_f32_to_f16_n(const float *in, uint16_t *out, int64_t n, int mode);
/* fptosi (CPU lowering: truncation toward zero; *poison set when out of range) */
void hfref_fptosi_n(const float *in, int64_t *out, int64_t n, int bits,
                    int *poison);
void hfref_f32_to_int_mode_n(const float *in, int64_t *out, int64_t n,
                             int mode, int bits, int saturate);
void hfref_int_to_f32_n(const int64_t *in, float *out, int64_t n, int mode);
void hfref_roundeven_n(const float *in, float *out, int64_t n);
void hfref_round_n(const float *in, float *out, int64_t n); /* math.round */

/* serial reduction: x is [K, N] (reduced index outermost, row-major), acc [N]
 * is updated in place: for k in 0..K-1: for j: acc[j] = op(x[k,j], acc[j]).
 * op: 0 addf 1 mulf 2 maximumf 3 minimumf 4 maxnumf 5 minnumf */
void hfref_reduce_f32(int op, const float *x, float *acc, int64_t K, int64_t N);
/* op: 0 addi 1 muli 2 maxsi 3 minsi 4 andi 5 ori 6 xori 7 maxui 8 minui */
void hfref_reduce_i64(int op, const int64_t *x, int64_t *acc, int64_t K,
                      int64_t N, int bits);
/* reduce_with_index, region of HFusionOps.cpp:1507-1595.  x [K, N] with the
 * reduced index k outermost; (val, idx) [N] carry the init and are updated.
 * kind: 0 max 1 min.  in_idx may be NULL (then idx = k, the linalg.index). */
void hfref_reduce_with_index_f32(int kind, const float *x, const int64_t *in_idx,
                                 float *val, int64_t *idx, int64_t K,
                                 int64_t N);
/* kind: 0 max(si) 1 min(si) 2 maxui 3 minui */
void hfref_reduce_with_index_i64(int kind, const int64_t *x,
                                 const int64_t *in_idx, int64_t *val,
                                 int64_t *idx, int64_t K, int64_t N, int bits);

/* linalg.matmul region: C[m,n] = C[m,n] + cast(A[m,k]) * cast(B[k,n]), k serial */
void hfref_matmul_i8_i32(const int8_t *A, const int8_t *B, int32_t *C,
                         int64_t M, int64_t N, int64_t K, int b_transposed);
void hfref_matmul_f32(const float *A, const float *B, float *C, int64_t M,
                      int64_t N, int64_t K, int b_transposed);
/* hfusion.matmul_mx: fp8 (fa/fb 0 e4m3, 1 e5m2) or packed fp4 (4 e2m1, two
 * per byte) operands with e8m0 scales per 32 k, f32 serial sum; K counts
 * logical values */
float hfref_fp4_to_f32(uint8_t v);
void hfref_matmul_mx(const uint8_t *A, const uint8_t *B, const uint8_t *sa, const uint8_t *sb, float *C, int64_t M,
                     int64_t N, int64_t K, int fa, int fb);

/* ---- composed groups: op-by-op loop nests with materialised temporaries,
 * as the CPU lowering executes them (used for the timed CPU baseline) ---- */
void hfref_vecadd_f32(const float *a, const float *b, float *out, int64_t n);
void hfref_rmsnorm_quant(const uint16_t *x_bf16, const uint16_t *gamma_bf16,
                         float eps, int8_t *q, float *scale, int64_t R,
                         int64_t C);
void hfref_softmax_bf16(const float *x, uint16_t *out, int64_t R, int64_t C);
void hfref_argmax(const float *x, float *val, int32_t *idx, int64_t R,
                  int64_t C);
/* rows [m0, m1) of the W8A8 mmad + dequant group, B given as [N, K] */
void hfref_w8a8_dequant_rows(const int8_t *A, const int8_t *Bt,
                             const float *s_tok, const float *s_ch,
                             uint16_t *out, int64_t M, int64_t N, int64_t K,
                             int64_t m0, int64_t m1);

/* hfusion.sort of the values along the last axis of R rows of L elements, in
 * place: the bubble sort the reference decomposes the op into.  kind: 0 f32,
 * 1 f16, 2 bf16 (float compare after the exact widening), 8/16/32/64 signed
 * integers of that width.  Returns 0, or -1 for an unknown kind. */
int hfref_sort_rows(void *data, int64_t R, int64_t L, int kind, int descending);

/* ---- host-entry ABI: MLIR ranked memref descriptors ----
 * The reference's runner calls `_mlir_ciface_<func>` with memref descriptors
 * (bishengir/lib/ExecutionEngine/BiShengIRRunnerUtils.cpp:99-110): for rank R
 * the standard layout is { T *allocated; T *aligned; int64_t offset;
 * int64_t sizes[R]; int64_t strides[R]; } (element strides).  Every
 * descriptor argument here is a pointer to such a struct; element (i0..iR-1)
 * lives at aligned + offset + sum_k i_k * strides[k].  Any strides are
 * accepted (views, slices, transposes); sizes must match the group's shapes.
 * Returns 0, or -1 when a shape does not match. */
int hfref_memref_gather(const void *desc, int rank, int elem_size, void *dense);
int hfref_memref_scatter(const void *dense, const void *desc, int rank, int elem_size);
int hfref_vecadd_f32_memref(const void *a, const void *b, const void *out);
int hfref_rmsnorm_quant_memref(const void *x, const void *gamma, float eps, const void *q, const void *scale);
int hfref_softmax_bf16_memref(const void *x, const void *out);
int hfref_argmax_memref(const void *x, const void *val, const void *idx);
int hfref_w8a8_dequant_memref(const void *a, const void *bt, const void *s_tok, const void *s_ch, const void *out);

#ifdef __cplusplus
}
#endif
#endif
