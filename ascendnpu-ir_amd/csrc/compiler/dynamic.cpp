// Dynamic dims (`?` in tensor / memref types): shape specialisation.
//
// The reference compiles a dynamic-shape kernel once and reads the sizes at
// run time from the memref descriptors, with host tiling functions choosing
// the schedule.  Here a group is compiled per size: the caller names the size
// of every dynamic dim of the function's arguments (compiler option
// `dyn=<func>:<arg>.<dim>=<size>,...`), this pass makes every type of the
// function static, and the lowering runs unchanged.  Compiled groups are
// cached by content, so a serving loop that buckets its sizes compiles each
// bucket once.
//
// Sizes flow the way the IR spells them: tensor.dim folds to the argument's
// size, index arithmetic folds, tensor.empty takes its dynamic dims from its
// index operands in order, a destination-style op's result takes its `outs`
// shape, an op without `outs` takes its first input's shape, and a reshape
// (expand_shape / collapse_shape) with one dynamic dim takes it from the
// element count.
#include "ir.h"

#include <set>

#include <map>
#include <sstream>

namespace hfc {

bool hasDynamicDims(const Module &m) {
  for (auto &v : m.values)
    for (auto d : v->type.shape)
      if (d < 0) return true;
  return false;
}

namespace {

bool isDynamic(const Type &t) {
  for (auto d : t.shape)
    if (d < 0) return true;
  return false;
}

int64_t numelOf(const std::vector<int64_t> &s) {
  int64_t n = 1;
  for (auto d : s) n *= d;
  return n;
}

// folds the index-typed scalar arithmetic that dynamic sizes go through
void foldIndex(Op *op) {
  if (op->results.empty()) return;
  Value *r = op->results[0];
  const std::string &n = op->name;
  if (n == "arith.constant") {
    // integer / index literals (the lowering folds every constant later)
    if (!r->type.tensor && !isFloat(r->type.elem) && !op->literal.empty()) {
      try {
        r->iconst = std::stoll(op->literal, nullptr, 0);
        r->fconst = (double)r->iconst;
        r->isConst = true;
      } catch (const std::exception &) {
      }
    }
    return;
  }
  if (n == "tensor.dim") {
    if (op->operands.size() == 2 && op->operands[1]->isConst) {
      const auto &sh = op->operands[0]->type.shape;
      const int64_t i = op->operands[1]->iconst;
      if (i < 0 || i >= (int64_t)sh.size()) throw CompileError("tensor.dim index out of range at line " + std::to_string(op->line));
      if (sh[i] >= 0) {
        r->isConst = true;
        r->iconst = sh[i];
        r->fconst = (double)sh[i];
      }
    }
    return;
  }
  if (r->type.tensor || r->isConst || op->operands.empty()) return;
  for (auto *o : op->operands)
    if (!o->isConst) return;
  const int64_t a = op->operands[0]->iconst, b = op->operands.size() > 1 ? op->operands[1]->iconst : 0;
  bool ok = true;
  int64_t v = 0;
  if (n == "arith.index_cast" || n == "arith.index_castui" || n == "arith.extsi" || n == "arith.extui" ||
      n == "arith.trunci") v = a;
  else if (n == "arith.addi") v = a + b;
  else if (n == "arith.subi") v = a - b;
  else if (n == "arith.muli") v = a * b;
  else if (n == "arith.divsi" && b) v = a / b; // truncating
  else if (n == "arith.divui" && b) v = (int64_t)((uint64_t)a / (uint64_t)b);
  else if ((n == "arith.floordivsi" || n == "arith.ceildivsi") && b) {
    // rounding toward -inf / +inf for any signs
    v = a / b;
    const bool inexact = v * b != a, neg = (a < 0) != (b < 0);
    if (inexact && n == "arith.floordivsi" && neg) --v;
    if (inexact && n == "arith.ceildivsi" && !neg) ++v;
  }
  else if (n == "arith.maxsi") v = a > b ? a : b;
  else if (n == "arith.minsi") v = a < b ? a : b;
  else ok = false;
  if (ok && (r->type.elem == Elem::Index || !isFloat(r->type.elem))) {
    r->isConst = true;
    r->iconst = v;
    r->fconst = (double)v;
  }
}

[[noreturn]] void cannot(const Op *op, const Value *v) {
  throw CompileError("cannot infer the dynamic shape of " + v->name + " ('" + op->name + "' at line " +
                     std::to_string(op->line) + ")");
}

void specializeFunc(Func &f, const std::map<std::pair<int, int>, int64_t> &sizes) {
  for (Value *a : f.args) {
    for (size_t d = 0; d < a->type.shape.size(); ++d) {
      if (a->type.shape[d] >= 0) continue;
      auto it = sizes.find({a->argIdx, (int)d});
      if (it == sizes.end())
        throw CompileError("dynamic dim " + std::to_string(d) + " of argument " + std::to_string(a->argIdx) + " of @" +
                           f.name + " has no size (compile with dyn=" + f.name + ":" + std::to_string(a->argIdx) + "." +
                           std::to_string(d) + "=<size>)");
      if (it->second < 0) throw CompileError("negative size for a dynamic dim of @" + f.name);
      a->type.shape[d] = it->second;
    }
  }
  for (Op *op : f.ops) {
    foldIndex(op);
    for (size_t ri = 0; ri < op->results.size(); ++ri) {
      Value *r = op->results[ri];
      if (!isDynamic(r->type)) continue;
      auto &sh = r->type.shape;
      const std::string &n = op->name;
      if (n == "tensor.empty") {
        size_t k = 0;
        for (auto &d : sh) {
          if (d >= 0) continue;
          if (k >= op->operands.size() || !op->operands[k]->isConst) cannot(op, r);
          d = op->operands[k++]->iconst;
        }
      } else if (n == "tensor.expand_shape" || n == "tensor.collapse_shape") {
        const Value *src = op->operands.empty() ? nullptr : op->operands[0];
        int unknown = 0;
        int64_t known = 1;
        for (auto d : sh) {
          if (d < 0) ++unknown;
          else known *= d;
        }
        if (!src || isDynamic(src->type) || unknown != 1 || known == 0) cannot(op, r);
        for (auto &d : sh)
          if (d < 0) d = numelOf(src->type.shape) / known;
      } else if (ri < op->outs.size() && !isDynamic(op->outs[ri]->type) &&
                 op->outs[ri]->type.shape.size() == sh.size()) {
        sh = op->outs[ri]->type.shape;
      } else if (op->outs.empty() && !op->ins.empty() && !isDynamic(op->ins[0]->type) &&
                 op->ins[0]->type.shape.size() == sh.size()) {
        sh = op->ins[0]->type.shape;
      } else if (op->outs.empty() && op->ins.empty() && !op->operands.empty() && op->operands[0]->type.tensor &&
                 !isDynamic(op->operands[0]->type) && op->operands[0]->type.shape.size() == sh.size()) {
        sh = op->operands[0]->type.shape;
      } else {
        cannot(op, r);
      }
    }
    // elementwise ops take operands of one shape: sizes given for different
    // arguments must agree where the IR joins them
    if (!op->outs.empty() && (op->name.find("elemwise") != std::string::npos || op->name == "hfusion.cast" ||
                              op->name == "hfusion.compare" || op->name == "hfusion.select")) {
      const auto &want = op->outs[0]->type.shape;
      for (Value *v : op->ins)
        if (v->type.tensor && v->type.shape.size() == want.size() && v->type.shape != want)
          throw CompileError("the sizes given for the dynamic dims disagree: '" + op->name + "' at line " +
                             std::to_string(op->line) + " joins " + v->type.str() + " and " + op->outs[0]->type.str());
    }
    for (size_t i = 0; i < op->results.size() && i < op->outs.size(); ++i)
      if (op->outs[i]->type.tensor && op->results[i]->type.shape != op->outs[i]->type.shape)
        throw CompileError("the sizes given for the dynamic dims disagree: the result of '" + op->name + "' at line " +
                           std::to_string(op->line) + " is " + op->results[i]->type.str() + ", its destination " +
                           op->outs[i]->type.str());
    // the types kept beside the operands follow their values
    for (size_t i = 0; i < op->ins.size() && i < op->insTypes.size(); ++i) op->insTypes[i] = op->ins[i]->type;
    for (size_t i = 0; i < op->outs.size() && i < op->outsTypes.size(); ++i) op->outsTypes[i] = op->outs[i]->type;
    if (isDynamic(op->literalType) && !op->results.empty()) op->literalType.shape = op->results[0]->type.shape;
    if (isDynamic(op->toType) && !op->results.empty()) op->toType.shape = op->results[0]->type.shape;
  }
  for (size_t i = 0; i < f.resultTypes.size() && i < f.returns.size(); ++i) f.resultTypes[i] = f.returns[i]->type;
}

} // namespace

// spec "runtime": the row count stays a launch-time value
void specializeRuntimeRows(Module &m) {
  for (auto &f : m.funcs) {
    std::vector<Value *> vals(f->args.begin(), f->args.end());
    for (Op *op : f->ops)
      for (Value *r : op->results) vals.push_back(r);
    // the dims that are dynamic now: each must end up as the row count itself
    std::vector<std::pair<Value *, size_t>> dyn;
    for (Value *v : vals)
      for (size_t d = 0; d < v->type.shape.size(); ++d) {
        if (v->type.shape[d] == kRuntimeRows)
          throw CompileError("@" + f->name + " has a static dim of " + std::to_string(kRuntimeRows) +
                             ", the placeholder of runtime row counts");
        if (v->type.shape[d] < 0) dyn.push_back({v, d});
      }
    if (dyn.empty()) continue;
    std::map<std::pair<int, int>, int64_t> sizes;
    for (Value *a : f->args)
      for (size_t d = 0; d < a->type.shape.size(); ++d) {
        if (a->type.shape[d] >= 0) continue;
        if (d != 0)
          throw CompileError("runtime row counts: dynamic dim " + std::to_string(d) + " of argument " +
                             std::to_string(a->argIdx) + " of @" + f->name + " is not dim 0");
        sizes[{a->argIdx, 0}] = kRuntimeRows;
      }
    specializeFunc(*f, sizes);
    for (auto &vd : dyn)
      if (vd.first->type.shape[vd.second] != kRuntimeRows)
        throw CompileError("runtime row counts: dim " + std::to_string(vd.second) + " of " + vd.first->name + " in @" +
                           f->name + " is derived from the row count, not the row count itself (compile per size)");
  }
}

void specializeDynamic(Module &m, const std::string &spec) {
  if (spec == "runtime") {
    specializeRuntimeRows(m);
    return;
  }
  // spec: <func>:<arg>.<dim>=<size>, comma-separated
  std::map<std::string, std::map<std::pair<int, int>, int64_t>> sizes;
  std::stringstream ss(spec);
  std::string item;
  while (std::getline(ss, item, ',')) {
    if (item.empty()) continue;
    const auto colon = item.rfind(':'), dot = item.find('.', colon == std::string::npos ? 0 : colon),
               eq = item.find('=');
    if (colon == std::string::npos || dot == std::string::npos || eq == std::string::npos || !(colon < dot && dot < eq))
      throw CompileError("bad dyn entry '" + item + "' (expected <func>:<arg>.<dim>=<size>)");
    try {
      sizes[item.substr(0, colon)][{std::stoi(item.substr(colon + 1, dot - colon - 1)),
                                    std::stoi(item.substr(dot + 1, eq - dot - 1))}] = std::stoll(item.substr(eq + 1));
    } catch (const std::exception &) {
      throw CompileError("bad dyn entry '" + item + "'");
    }
  }
  // every entry names a function with a dynamic argument dim at that place
  for (const auto &fe : sizes) {
    const Func *fn = nullptr;
    for (auto &f : m.funcs)
      if (f->name == fe.first) fn = f.get();
    if (!fn) throw CompileError("dyn entry for @" + fe.first + ", which is not a function of the module");
  }
  std::set<std::string> used;
  for (auto &f : m.funcs) {
    bool dyn = false;
    for (Value *a : f->args) dyn |= isDynamic(a->type);
    for (Op *op : f->ops)
      for (Value *r : op->results) dyn |= isDynamic(r->type);
    if (!dyn) continue;
    auto it = sizes.find(f->name);
    if (it != sizes.end()) {
      // every entry must name a dynamic dim of an argument
      for (const auto &kv : it->second) {
        const int ai = kv.first.first, di = kv.first.second;
        if (ai < 0 || ai >= (int)f->args.size() || di < 0 || di >= (int)f->args[ai]->type.shape.size() ||
            f->args[ai]->type.shape[di] >= 0)
          throw CompileError("dyn entry " + f->name + ":" + std::to_string(ai) + "." + std::to_string(di) +
                             " names no dynamic dim of @" + f->name);
      }
      used.insert(f->name);
    }
    specializeFunc(*f, sizes[f->name]);
  }
  for (const auto &kv : sizes)
    if (!used.count(kv.first))
      throw CompileError("dyn entry for @" + kv.first + ", which has no dynamic dims (or does not exist)");
}

} // namespace hfc
