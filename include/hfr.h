/*
 * hfr — C-ABI runtime that loads and launches HFusion group kernels on one
 * MI355X (one GPU, caller-provided stream).
 *
 * Replaces the host launch sequence the reference's integration test drives
 * through CANN (bishengir/test/Integration/HIVM/VecAdd/main.cpp:
 * rtDevBinaryRegister + rtFunctionRegister -> rtKernelLaunch(stub, blockDim,
 * args = {in0, in1, out}, stream) -> aclrtSynchronizeStream).  Kernel
 * arguments are bare device pointers in the group function's argument order
 * (destination-passing style, HFusionStructuredOps.td:38-44), followed by
 * buffers for results that are not written into an argument.
 *
 * Ownership: the caller allocates and frees every tensor buffer.  The runtime
 * owns module/group handles and one zero-initialised workspace per group
 * handle that needs one, allocated by hfr_group_load on the current device
 * (launches never allocate).
 * Threading: launches are asynchronous on the given stream; the caller
 * synchronises.  A handle must not be used from two threads at once, and two
 * in-flight launches of one group handle that both use its internal workspace
 * must be on the same stream.
 * Errors: every call returns 0 or a negative HFR_ERR_* code; hfr_last_error()
 * gives the message for the calling thread.
 */
#ifndef HFR_H
#define HFR_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HFR_OK 0
#define HFR_ERR_INVALID -1  /* bad argument (null handle/pointer, count mismatch) */
#define HFR_ERR_HIP -2      /* HIP runtime call failed */
#define HFR_ERR_IO -3       /* file missing or unreadable */
#define HFR_ERR_MANIFEST -4 /* malformed manifest */
#define HFR_ERR_NOT_FOUND -5/* kernel or function name not present */

typedef struct hfr_module *hfr_module_t;
typedef struct hfr_kernel *hfr_kernel_t;
typedef struct hfr_group *hfr_group_t;
typedef struct hfr_program *hfr_program_t;

typedef struct hfr_launch_cfg {
  unsigned grid[3];
  unsigned block[3];
  unsigned lds_bytes;
} hfr_launch_cfg;

typedef struct hfr_group_info {
  int nparams;
  int nresults;
  int nkargs;
  uint64_t workspace_bytes;
  uint64_t algo_bytes; /* algorithmic HBM bytes per launch */
  uint64_t algo_ops;   /* algorithmic ops per launch (contractions) */
  hfr_launch_cfg cfg;
} hfr_group_info;

/* ---- code objects and kernels (replaces rtDevBinaryRegister / rtFunctionRegister) */
int hfr_module_load(const char *hsaco_path, hfr_module_t *out);
int hfr_module_unload(hfr_module_t m);
int hfr_kernel_get(hfr_module_t m, const char *name, hfr_kernel_t *out);
/* args: one 8-byte slot per kernel parameter (device pointer or raw scalar
 * bits); replaces rtKernelLaunch. */
int hfr_launch(hfr_kernel_t k, const hfr_launch_cfg *cfg, const uint64_t *args, size_t nargs, void *stream);

/* ---- manifest-driven groups (what bishengir-compile --target=mi355x emits) */
/* func may be NULL when the manifest holds one group. */
int hfr_group_load(const char *manifest_path, const char *func, hfr_group_t *out);
int hfr_group_unload(hfr_group_t g);
int hfr_group_info_get(hfr_group_t g, hfr_group_info *info);
/* params: one slot per group argument (device pointer, or the raw bits of a
 * scalar argument); results: one pointer per group result (ignored — may be
 * NULL — for results written into an argument); workspace: NULL to use the
 * group's own, or a caller buffer of workspace_bytes (zeroed before its first
 * use when the group requires it). */
int hfr_group_launch(hfr_group_t g, const uint64_t *params, size_t nparams, void *const *results, size_t nresults,
                     void *workspace, void *stream);
/* A group compiled with runtime row counts (compiler option dyn=runtime; its
 * manifest holds `rows_dyn`, and -1 for the row dim of each shape): the same
 * launch over `rows` rows (0: no launch).  One compiled kernel serves every
 * row count, where the reference schedules a dynamic-shape kernel once and
 * reads the sizes at run time from its memref descriptors
 * (bishengir/lib/Dialect/HFusion/Transforms/AutoSchedule/AnyPBRSchedule.cpp).
 * hfr_group_launch refuses such a group; this entry refuses a static group
 * unless rows is -1. */
int hfr_group_launch_rows(hfr_group_t g, const uint64_t *params, size_t nparams, void *const *results,
                          size_t nresults, int64_t rows, void *workspace, void *stream);

/* ---- launch programs (an un-fused function split into fused groups)
 * Replaces the host function the reference's HFusion auto-fusion leaves
 * behind after outlining: a sequence of `func.call`s to the outlined groups
 * with tensors passed between them
 * (bishengir/lib/Dialect/HFusion/Transforms/OpFusion.cpp:68-229,
 * OpFusion/FusibleBlockOutliner.cpp:211-290).  Here the steps launch the
 * groups' kernels in order on one stream; tensors passed between groups live
 * in one program workspace. */
typedef struct hfr_program_info {
  int nparams;
  int nresults;
  int nsteps;
  uint64_t workspace_bytes; /* intermediate tensors, 256-byte aligned */
} hfr_program_info;

/* name may be NULL when the manifest holds one program. */
int hfr_program_load(const char *manifest_path, const char *name, hfr_program_t *out);
int hfr_program_unload(hfr_program_t p);
int hfr_program_info_get(hfr_program_t p, hfr_program_info *info);
/* params: one slot per argument of the original function; results: one
 * pointer per result (ignored for results written into an argument);
 * workspace: NULL to use the program's own (allocated at load), or a
 * caller buffer of workspace_bytes.  Steps are enqueued on `stream`; each
 * group uses its own internal workspace. */
int hfr_program_launch(hfr_program_t p, const uint64_t *params, size_t nparams, void *const *results, size_t nresults,
                       void *workspace, void *stream);

/* ---- MLIR C-interface form of a group launch
 * descs: one pointer per group argument, in the IR's argument order, to the
 * argument's ranked memref descriptor as an `_mlir_ciface_*` function receives
 * it, then one per result not written into an argument:
 *     struct { T *allocated; T *aligned; int64_t offset;
 *              int64_t sizes[R]; int64_t strides[R]; }
 * (R = the tensor's rank; a scalar argument passes a pointer to its value).
 * The device buffer is aligned + offset elements.  Sizes must equal the
 * group's static shape (otherwise HFR_ERR_INVALID); a group with a runtime
 * row count takes its rows from the descriptors' row dims, which must agree.  Dense row-major views are
 * used in place; any other strides (row pitches, transposed or broadcast
 * views) go through a dense staging copy on `stream`: gathered before the
 * group's kernels when the group reads the view, scattered back after them
 * when it writes it.  A written view that overlaps itself is refused.  The
 * staging buffer belongs to the group: allocated on the first strided launch,
 * grown when a later one needs more (which waits for the device), freed by
 * hfr_group_unload; calls that overlap on one group race.  Replaces the reference runner's memref entry points
 * (`_mlir_ciface_getData*` / `printData*` over UnrankedMemRefType, whose
 * descriptor field points at this ranked layout:
 * bishengir/lib/ExecutionEngine/BiShengIRRunnerUtils.cpp:99-110). */
int hfr_group_launch_memref(hfr_group_t g, void *const *descs, size_t ndescs, void *stream);

/* ---- launch without allocation (no counterpart in the reference)
 * For callers that cannot allocate device memory: code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.  Same
 * arguments as hfr_group_launch without a workspace: a group that needs one
 * uses the library's static per-device scratch array of HFR_SCRATCH_BYTES
 * (held by each GPU until the process ends; groups needing more are refused
 * with HFR_ERR_INVALID).  The scratch is cleared with a fill kernel on
 * `stream` before the group's kernel when the group needs zeroed workspace.
 * Calls on one GPU share its scratch: calls that overlap on one GPU (two
 * streams, or two threads) race.  The call allocates nothing on the device
 * (the first call on a device looks up the scratch address once). */
#define HFR_SCRATCH_BYTES (4u << 20)
int hfr_group_launch_noalloc(hfr_group_t g, const uint64_t *params, size_t nparams, void *const *results,
                             size_t nresults, void *stream);
uint64_t hfr_scratch_bytes(void);

const char *hfr_last_error(void);
const char *hfr_version(void);

#ifdef __cplusplus
}
#endif
#endif
