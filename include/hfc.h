/*
 * hfc — C-ABI of the MI355X HFusion compiler (ConvertHFusionToHIP + HIP code
 * object emission).
 *
 * Replaces, for the HFusion op-group path, the reference's device compile
 * entry `bishengir-compile <in.mlir> ... -o <out>`
 * (bishengir/tools/bishengir-compile/bishengir-compile.cpp:103-191 ->
 * runBiShengIRPipeline, bishengir/lib/Tools/bishengir-compile/
 * BiShengIRCompileMain.cpp:265-356, which ends by exec'ing the external
 * `hivmc`, :188-262).  Here the final step runs `hipcc --genco` for gfx950.
 *
 * Outputs for an output prefix P:
 *   P.hip       generated HIP translation unit (kernels of every entry func)
 *   P.hsaco     gfx950 code object (hipModuleLoad-able)
 *   P.manifest  launch manifest(s): one "hfr-manifest 1" block per entry func,
 *               then one "hfr-program 1" block per host function that the
 *               fusion front-end split into groups
 *
 * Fusion front-end (the reference's HFusion auto-fusion: InferFuncFusionKind
 * + HFusionOpFusion + OutlineSingleOp, bishengir/lib/Dialect/HFusion/
 * Transforms/InferFuncFusionKind.cpp:70-103, OpFusion.cpp:68-229): a function
 * without `hfusion.fusion_kind` that is marked
 * `hacc.function_kind = #hacc.function_kind<HOST>`, or whose ops fit no single
 * fusion kind, is outlined into fused groups (`<func>_g<k>`, each one kernel)
 * and a launch program named after the function (see hfr_program_* in hfr.h).
 *
 * Options string: ';'-separated key=value pairs
 *   hipcc=<path>            (default /opt/rocm/bin/hipcc)
 *   include=<dir>           kernel library headers (default: located next to
 *                           this library, ../csrc/kernels)
 *   arch=<gfx>              (default gfx950)
 *   emit=hip|hsaco|outlined stop after writing P.hip, or build the code object,
 *                           or stop after the fusion front-end, writing the
 *                           outlined module (P.outlined.mlir) and the launch
 *                           programs (P.programs)
 *   fusion_kind=<KIND>      outline every function without a declared kind
 *                           by this one kind (PURE_ELEMWISE, ANY_PB,
 *                           LAST_AXIS_PBR, ANY_PBR, MIX_CV), as the
 *                           reference's --test-assign-fusion-kind does
 *   ordered_fp_sums=0|1     serial-order fp32 sums for every linalg.reduce addf
 *   rmsq_kernel=0|1         RMSNorm + dynamic int8 quantisation groups: 1 (the
 *                           default) through the one-wave-per-row exact
 *                           parallel sum where the widths allow, 0 through the
 *                           generic row program
 *   rmsn_kernel=1           the same groups through the chain-wave kernel
 *   mx_exact=1              fp8 hfusion.matmul_mx through scaled bf16 operands
 *                           and the bf16 matrix core (exact products, f32 sums)
 *   dyn=<func>:<arg>.<dim>=<size>,...  sizes of dynamic dims
 *   dyn=runtime             one kernel for every row count (every dynamic dim
 *                           is dim 0 of the arguments; row programs, RMSNorm +
 *                           quant, streaming elementwise of rank >= 2,
 *                           contractions over M, reduce_with_index over
 *                           rows): launch with
 *                           hfr_group_launch_rows
 *
 * Returns 0 on success; a negative code with a message in `err` otherwise
 * (mirrors the reference's "[ERROR] ..." + EXIT_FAILURE convention).
 */
#ifndef HFC_H
#define HFC_H
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HFC_OK 0
#define HFC_ERR_PARSE -1     /* input is not in the accepted HFusion subset */
#define HFC_ERR_LOWER -2     /* group shape/ops not supported by the lowering */
#define HFC_ERR_IO -3        /* cannot read input / write outputs */
#define HFC_ERR_TOOLCHAIN -4 /* hipcc failed */

/* Compile IR text held in memory. */
int hfc_compile(const char *ir_text, const char *out_prefix, const char *options, char *err, size_t errlen);
/* Compile an .mlir file. */
int hfc_compile_file(const char *mlir_path, const char *out_prefix, const char *options, char *err, size_t errlen);
/* Library version string. */
const char *hfc_version(void);

#ifdef __cplusplus
}
#endif
#endif
