// HFusion fusion front-end: splits an un-fused function into fusible op
// groups, each outlined as its own `func.func` (one kernel), plus the launch
// program that runs them in order.
//
// Follows the reference's grouping (bishengir/lib/Dialect/HFusion/Transforms/
// InferFuncFusionKind.cpp:70-103, OpFusion.cpp:68-133, OutlineSingleOp via
// OpFusion.cpp:165-229, and the union-find analyzer of
// OpFusion/FusibleBlockAnalyzer.cpp with the fusion rules of
// OpFusion/FusibleHelper.cpp):
//   1. a function whose ops all fit one fusion kind (tried in enum order) stays
//      one group;
//   2. otherwise blocks are grown per kind in the multi-kernel order (MixCV,
//      LastAxisPBR, AnyPB; the Ascend-only shallow / C2 kinds are skipped);
//   3. every important op left over becomes a group of its own.
#pragma once
#include "ir.h"

#include <string>
#include <vector>

namespace hfc {

// One buffer of a launch program: "p<i>" a program parameter, "t<j>" a
// temporary in the program workspace, "r<k>" a program result.
struct ProgramStep {
  std::string group;                 // outlined func name
  std::vector<std::string> args;     // binding per group argument
  std::vector<std::string> results;  // binding per group result
};

struct ProgramBuffer {
  Elem elem = Elem::None;
  std::vector<int64_t> shape;
  std::string role;    // params: in | out | inout | scalar; results: binding ("p<i>" when written into a param, else "r")
  uint64_t offset = 0; // temps: byte offset in the workspace
  uint64_t bytes = 0;
};

struct ProgramPlan {
  std::string name; // the host function
  std::vector<ProgramBuffer> params, results, temps;
  std::vector<ProgramStep> steps;
  std::vector<std::string> groupKinds; // fusion kind of each step's group
  uint64_t workspaceBytes = 0;
};

// Fusion kind of a whole function as InferFuncFusionKind computes it
// ("PURE_ELEMWISE", ..., "UNKNOWN").
std::string inferFusionKind(const Func &f);

// Rewrites every function without an `hfusion.fusion_kind` whose ops do not
// fit one kind into its outlined groups (programs describe how to launch
// them).  Returns the new module text, or the input text when nothing was
// split.
// `forceKind` (a FusionKind name) outlines every function without a declared
// kind by that one kind, as `--test-assign-fusion-kind` does in the
// reference's tests; groups left over become single-op groups.
std::string outlineFusedGroups(const Module &m, std::vector<ProgramPlan> &programs,
                               const std::string &forceKind = "");

// The launch-program section of the manifest.
std::string emitProgramManifest(const ProgramPlan &p);

} // namespace hfc
