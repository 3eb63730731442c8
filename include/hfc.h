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
 *   P.manifest  launch manifest(s): one "hfr-manifest 1" block per entry func
 *
 * Options string: ';'-separated key=value pairs
 *   hipcc=<path>            (default /opt/rocm/bin/hipcc)
 *   include=<dir>           kernel library headers (default: located next to
 *                           this library, ../csrc/kernels)
 *   arch=<gfx>              (default gfx950)
 *   emit=hip|hsaco          stop after writing P.hip, or build the code object
 *   ordered_fp_sums=0|1     serial-order fp32 sums for every linalg.reduce addf
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
