// ConvertHFusionToHIP: maps one outlined HFusion op group (a `func.func`) onto
// a CDNA4 HIP kernel plus a launch manifest.
//
// This takes the place of the reference's HFusion->HIVM->Template path
// (bishengir/lib/Conversion/HFusionToHIVM/HFusionToHIVM.cpp:1785-1933,
// bishengir/lib/Dialect/HIVM/Pipelines/HIVMPipelines.cpp:516-546) and of the
// external `hivmc` step (bishengir/lib/Tools/bishengir-compile/
// BiShengIRCompileMain.cpp:188-262).
#pragma once
#include "ir.h"

#include <string>
#include <vector>

namespace hfc {

struct BufferDesc {
  std::string role;  // "in", "out", "inout", "scalar"
  Elem elem = Elem::None;
  std::vector<int64_t> shape;
  int tiedParam = -1; // results: the func argument they are written into
};

struct KernelPlan {
  std::string funcName;
  std::string kernelName;
  std::string kind;           // PURE_ELEMWISE | LAST_AXIS_PBR | REDUCE_WITH_INDEX | SINGLE_CUBE
  std::string variant;        // schedule detail, e.g. "ordered-sum"
  std::string source;         // HIP translation-unit body (kernel only)
  unsigned grid[3] = {1, 1, 1};
  unsigned block[3] = {1, 1, 1};
  unsigned ldsBytes = 0;      // dynamic LDS
  uint64_t workspaceBytes = 0;
  bool workspaceZeroInit = false; // workspace must be zero when first used
  std::vector<BufferDesc> params;  // func arguments, in order
  std::vector<BufferDesc> results; // func results, in order
  // kernel argument list, each "param:<i>", "result:<i>", "ws"
  std::vector<std::string> kargs;
  double algoBytes = 0;       // algorithmic HBM bytes per launch
  double algoOps = 0;         // algorithmic ops per launch (cube groups)
  // kernels launched before the main one on the same stream (operand
  // re-layouts into the workspace); argument lists as `kargs`
  struct PreKernel {
    std::string name;
    unsigned grid = 1, block = 256;
    std::vector<std::string> kargs;
  };
  std::vector<PreKernel> pre;
  // runtime row count (compiler option dyn=runtime): the kernel takes the
  // row count R as its last argument (karg "rows"); the launch grid is
  // min(ceil(R * rowsA / rowsB) * rowsC, rowsCap) blocks (rowsCap 0: no cap),
  // or the static grid when rowsA is 0.  Shapes hold -1 for the row dim, and
  // algoBytes is per row.
  bool rowsDyn = false;
  int64_t rowsA = 0, rowsB = 1, rowsC = 1, rowsCap = 0;
};

struct LowerOptions {
  // fp sums in the reference's serial order: 1 everywhere the row fits the
  // serial schedule's registers, 0 only where an integer output depends on
  // the sum (tree order elsewhere); the default (-1) is the serial order for
  // rows of at most 4096 elements
  int orderedFloatSums = -1;
  // RMSNorm + dynamic quantisation (matchRmsQuant) through hf_rmsq.h, the
  // default for rows it takes (option rmsq_kernel=0: the generic row program)
  bool rmsqKernel = true;
  bool mxExact = false;          // matmul_mx through scaled bf16 operands and the bf16 matrix core
  bool rmsnKernel = false;       // ... through hf_rmsn.h (chain wave + product maxima; opt-in)
  // dynamic dims specialised to kRuntimeRows (option dyn=runtime): the row
  // count becomes a kernel argument where the group kind allows it
  bool runtimeRows = false;
};

// Ops lowered as a kernel of their own (cumulative ops, histogram,
// (de)interleave): they never fuse with other ops.
bool isSingleOpKernel(const std::string &opName);

// Lowers every `hacc.entry` function (or every function if none is tagged).
std::vector<KernelPlan> lowerModule(Module &m, const LowerOptions &opt);

// The text of the HIP source file holding all `plans` (includes the kernel
// library headers).
std::string emitTranslationUnit(const std::vector<KernelPlan> &plans);

// The launch manifest (line-oriented text, read by libhfr and the host API).
std::string emitManifest(const KernelPlan &p, const std::string &hsacoName);

} // namespace hfc
