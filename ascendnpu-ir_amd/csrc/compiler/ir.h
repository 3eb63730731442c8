// In-memory form of the HFusion op subset read from textual MLIR.
//
// The reference keeps HFusion groups as MLIR `func.func`s tagged
// `hacc.entry` / `hfusion.fusion_kind` (bishengir/include/bishengir/Dialect/
// HFusion/IR/HFusionEnums.td:210-233) whose bodies are destination-passing
// linalg/hfusion structured ops (HFusionStructuredOps.td:38-44).  No MLIR is
// available on the target machines, so this is a self-contained reader for the
// ops the MI355X lowering accepts.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace hfc {

struct CompileError : std::runtime_error {
  using std::runtime_error::runtime_error;
};

enum class Elem { F32, F16, BF16, F64, F8E4M3FN, F8E5M2, I1, I8, I16, I32, I64, Index, None };

const char *elemName(Elem e);
int elemBytes(Elem e);
int elemBits(Elem e);
bool isFloat(Elem e);
bool isInt(Elem e);
Elem parseElem(const std::string &s); // throws on unknown

struct Type {
  bool tensor = false;
  bool memref = false; // a memref<...> (read as a tensor of the same shape)
  Elem elem = Elem::None;
  bool uns = false;           // written ui8: bytes read unsigned (matmul_mx scales only)
  std::vector<int64_t> shape; // tensor only
  int64_t numel() const {
    int64_t n = 1;
    for (auto d : shape) n *= d;
    return n;
  }
  std::string str() const;
};

struct Op;

struct Value {
  std::string name; // "%x", "%4#1" for multi-result
  Type type;
  Op *def = nullptr;   // producing op (null for func args)
  int resultIdx = 0;
  int argIdx = -1;     // func argument position
  // folded scalar constant (arith.constant or foldable scalar arith)
  bool isConst = false;
  double fconst = 0;
  int64_t iconst = 0;
  uint64_t constBits = 0; // exact bit pattern for float constants given in hex
  bool constHasBits = false;
  std::vector<Op *> users;
};

struct Op {
  std::string name;                       // e.g. "hfusion.elemwise_binary"
  size_t srcBegin = 0, srcEnd = 0;        // the statement's span in Module::source
  std::vector<Value *> ins, outs, operands; // operands: non ins/outs operands
  std::vector<Type> insTypes, outsTypes;
  std::vector<Value *> results;
  std::map<std::string, std::string> attrs; // key -> raw value ("mul", "true")
  std::vector<int64_t> dims;                // `dimensions = [...]`
  bool hasDims = false;
  std::string angleKind;  // `<max>` of reduce_with_index
  std::string combiner;   // region / {arith.addf} combiner of linalg.reduce
  std::vector<std::string> regionOps; // op names inside the region
  std::string literal;    // arith.constant literal text
  Type literalType;       // type after ':' (arith ops / constants)
  Type toType;            // `to T` of casts
  int line = 0;
  std::string attr(const std::string &k, const std::string &dflt = "") const {
    auto it = attrs.find(k);
    return it == attrs.end() ? dflt : it->second;
  }
};

struct Func {
  std::string name;
  std::vector<Value *> args;
  std::vector<Type> resultTypes;
  std::map<std::string, std::string> attrs;
  std::vector<Op *> ops;
  std::vector<Value *> returns;
  size_t srcBegin = 0, srcEnd = 0; // `func.func ... }` span in Module::source
  bool isEntry() const { return attrs.count("hacc.entry") != 0; }
  std::string fusionKind() const {
    auto it = attrs.find("hfusion.fusion_kind");
    return it == attrs.end() ? "" : it->second;
  }
};

struct Module {
  std::string source; // the text the module was read from
  std::map<std::string, std::string> aliases; // `#map = affine_map<...>` -> "affine_map<...>"
  std::vector<std::unique_ptr<Func>> funcs;
  std::vector<std::unique_ptr<Value>> values;
  std::vector<std::unique_ptr<Op>> ops;
  Value *newValue() {
    values.emplace_back(new Value());
    return values.back().get();
  }
  Op *newOp() {
    ops.emplace_back(new Op());
    return ops.back().get();
  }
};

// Parses textual MLIR (the subset above).  Throws CompileError with a line
// number on anything it does not understand.
std::unique_ptr<Module> parseModule(const std::string &text);

// Dynamic dims (shape -1 after parsing): true when any value has one.
bool hasDynamicDims(const Module &m);
// Makes every type static from the sizes of the functions' dynamic argument
// dims, spec "<func>:<arg>.<dim>=<size>,..." (dynamic.cpp).  Spec "runtime":
// every dynamic dim must be the row count (dim 0 of the arguments, and only
// that size where it flows); it becomes kRuntimeRows, which the lowering
// turns into a kernel argument (LowerOptions::runtimeRows).
void specializeDynamic(Module &m, const std::string &spec);
constexpr int64_t kRuntimeRows = int64_t(1) << 30;

} // namespace hfc
