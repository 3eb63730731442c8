// ConvertHFusionToHIP — see lower.h.
//
// Group classification follows the reference's fusion kinds
// (FusibleHelper.cpp:51-70 pattern -> kind; HFusionEnums.td:210-233):
//   * a `linalg.matmul[_transpose_b]` + elementwise epilogue -> SINGLE_CUBE
//     (hand-written MFMA kernel, hf_mmad.h, with a generated epilogue);
//   * `hfusion.reduce_with_index` -> split-row arg-reduction (hf_argmax.h);
//   * last-axis `linalg.reduce` chains -> LAST_AXIS_PBR row programs (one row
//     group of threads keeps its row resident in VGPRs, hf_row.h helpers);
//   * everything else (elementwise + broadcast) -> PURE_ELEMWISE / ANY_PB
//     streaming kernels with 128-bit accesses.
// Scalar meaning of each op: hf_ops.h (region builders of
// bishengir/lib/Dialect/HFusion/IR/HFusionOps.cpp:434-862).
#include "lower.h"

#include <algorithm>
#include <cctype>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <set>
#include <sstream>

namespace hfc {
namespace {

[[noreturn]] void unsupported(const Op *op, const std::string &why) {
  throw CompileError("unsupported: " + why + (op ? " ('" + op->name + "' at line " + std::to_string(op->line) + ")" : std::string()));
}

std::string ctype(Elem e) {
  switch (e) {
  case Elem::F32: return "float";
  case Elem::F64: return "double";
  case Elem::F16: case Elem::BF16: return "uint16_t";
  case Elem::F8E4M3FN: case Elem::F8E5M2: return "uint8_t";
  case Elem::I1: return "bool";
  case Elem::I8: return "int8_t";
  case Elem::I16: return "int16_t";
  case Elem::I32: return "int32_t";
  case Elem::I64: case Elem::Index: return "int64_t";
  default: throw CompileError("no storage type for element type");
  }
}
// in-memory element type (i1 is one byte)
std::string mtype(Elem e) { return e == Elem::I1 ? "uint8_t" : ctype(e); }

std::string floatLit(float f) {
  if (std::isnan(f)) return "__builtin_nanf(\"\")";
  if (std::isinf(f)) return f > 0 ? "__builtin_inff()" : "(-__builtin_inff())";
  char buf[64];
  std::snprintf(buf, sizeof buf, "%af", (double)f);
  return std::string("(") + buf + ")";
}
std::string doubleLit(double d) {
  if (std::isnan(d)) return "__builtin_nan(\"\")";
  if (std::isinf(d)) return d > 0 ? "__builtin_inf()" : "(-__builtin_inf())";
  char buf[64];
  std::snprintf(buf, sizeof buf, "%a", d);
  return std::string("(") + buf + ")";
}

// --------------------------------------------------------------- constants
bool parseLiteral(const std::string &lit, Elem e, Value *v) {
  std::string s = lit;
  if (s.rfind("dense<", 0) == 0) s = s.substr(6, s.size() - 7);
  if (s.empty()) return false;
  if (s == "true" || s == "false") {
    v->isConst = true;
    v->iconst = s == "true";
    v->fconst = (double)v->iconst;
    return true;
  }
  bool hex = s.size() > 2 && (s.compare(0, 2, "0x") == 0 || s.compare(0, 2, "0X") == 0);
  v->isConst = true;
  if (isFloat(e)) {
    if (hex) {
      uint64_t bits = std::stoull(s, nullptr, 16);
      v->constBits = bits;
      v->constHasBits = true;
      if (e == Elem::F32) { float f; uint32_t u = (uint32_t)bits; std::memcpy(&f, &u, 4); v->fconst = f; }
      else if (e == Elem::F64) { double d; std::memcpy(&d, &bits, 8); v->fconst = d; }
      else if (e == Elem::BF16) { float f; uint32_t u = (uint32_t)bits << 16; std::memcpy(&f, &u, 4); v->fconst = f; }
      else throw CompileError("hex f16 constants are not supported");
    } else if (e == Elem::F32 || e == Elem::BF16 || e == Elem::F16) {
      v->fconst = std::strtof(s.c_str(), nullptr);
    } else {
      v->fconst = std::strtod(s.c_str(), nullptr);
    }
    v->iconst = (int64_t)v->fconst;
  } else {
    v->iconst = hex ? (int64_t)std::stoull(s, nullptr, 16) : std::stoll(s);
    v->fconst = (double)v->iconst;
  }
  return true;
}

float roundF32(double d) { return (float)d; }

void foldConstants(Func &f) {
  for (Op *op : f.ops) {
    if (op->results.empty()) continue;
    Value *r = op->results[0];
    const std::string &n = op->name;
    auto allConst = [&]() {
      for (auto *o : op->operands) if (!o->isConst) return false;
      return !op->operands.empty();
    };
    if (n == "arith.constant") {
      if (!parseLiteral(op->literal, r->type.elem, r))
        unsupported(op, "constant literal '" + op->literal + "'");
      continue;
    }
    if (n == "tensor.dim") {
      r->type = Type();
      r->type.elem = Elem::Index;
      if (op->operands.size() == 2 && op->operands[1]->isConst) {
        auto &sh = op->operands[0]->type.shape;
        int64_t i = op->operands[1]->iconst;
        if (i < 0 || i >= (int64_t)sh.size()) unsupported(op, "dimension index");
        r->isConst = true;
        r->iconst = sh[i];
        r->fconst = (double)sh[i];
      }
      continue;
    }
    if (r->type.tensor || !allConst()) continue;
    Value *a = op->operands[0];
    Value *b = op->operands.size() > 1 ? op->operands[1] : nullptr;
    Elem e = r->type.elem;
    bool f32 = e == Elem::F32;
    auto setF = [&](double d) { r->isConst = true; r->fconst = f32 ? (double)roundF32(d) : d; r->iconst = (int64_t)r->fconst; };
    auto setI = [&](int64_t i) { r->isConst = true; r->iconst = i; r->fconst = (double)i; };
    if (n == "arith.index_cast" || n == "arith.index_castui" || n == "arith.extsi" ||
        n == "arith.extui" || n == "arith.trunci") setI(a->iconst);
    else if (n == "arith.sitofp" || n == "arith.uitofp") setF((double)a->iconst);
    else if (n == "arith.extf" || n == "arith.truncf") setF(a->fconst);
    else if (n == "arith.fptosi" || n == "arith.fptoui") setI((int64_t)std::trunc(a->fconst));
    else if (n == "arith.negf") setF(-a->fconst);
    else if (b && f32 && n == "arith.addf") setF(roundF32(a->fconst) + roundF32(b->fconst));
    else if (b && f32 && n == "arith.subf") setF(roundF32(a->fconst) - roundF32(b->fconst));
    else if (b && f32 && n == "arith.mulf") setF(roundF32(a->fconst) * roundF32(b->fconst));
    else if (b && f32 && n == "arith.divf") setF(roundF32(a->fconst) / roundF32(b->fconst));
    else if (b && n == "arith.addf") setF(a->fconst + b->fconst);
    else if (b && n == "arith.subf") setF(a->fconst - b->fconst);
    else if (b && n == "arith.mulf") setF(a->fconst * b->fconst);
    else if (b && n == "arith.divf") setF(a->fconst / b->fconst);
    else if (b && n == "arith.addi") setI(a->iconst + b->iconst);
    else if (b && n == "arith.subi") setI(a->iconst - b->iconst);
    else if (b && n == "arith.muli") setI(a->iconst * b->iconst);
    else if (b && n == "arith.divsi" && b->iconst) setI(a->iconst / b->iconst);
  }
}

// A scalar literal expression for a constant value of element type e.
std::string constExpr(const Value *v, Elem e) {
  if (!v->isConst) throw CompileError("value " + v->name + " is not a constant");
  switch (e) {
  case Elem::F32:
    if (v->constHasBits && v->type.elem == Elem::F32) {
      char b[64];
      std::snprintf(b, sizeof b, "__uint_as_float(0x%08xu)", (unsigned)v->constBits);
      return b;
    }
    return floatLit((float)v->fconst);
  case Elem::F64: return doubleLit(v->fconst);
  case Elem::BF16: {
    char b[64];
    float f = (float)v->fconst;
    uint32_t u; std::memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) u = (u >> 16) | 0x40u;
    else u = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
    std::snprintf(b, sizeof b, "((uint16_t)0x%04x)", u & 0xffffu);
    return b;
  }
  case Elem::F16: return "hf::f32_to_f16<0>(" + floatLit((float)v->fconst) + ")";
  case Elem::I1: return v->iconst ? "true" : "false";
  case Elem::I8: return "((int8_t)" + std::to_string(v->iconst) + ")";
  case Elem::I16: return "((int16_t)" + std::to_string(v->iconst) + ")";
  case Elem::I32: return "((int32_t)" + std::to_string(v->iconst) + ")";
  default: return "((int64_t)" + std::to_string(v->iconst) + "ll)";
  }
}

// --------------------------------------------------------------- scalar ops
// convertScalarToDtype (upstream MLIR), used by the `cast` type_fn of named ops.
std::string castExpr(const std::string &x, Elem from, Elem to, bool unsignedCast) {
  if (from == to) return x;
  if (from == Elem::Index) from = Elem::I64;
  if (to == Elem::Index) to = Elem::I64;
  if (from == to) return x;
  auto toF32 = [&](const std::string &s, Elem f) -> std::string {
    if (f == Elem::F32) return s;
    if (f == Elem::BF16) return "hf::bf16_to_f32(" + s + ")";
    if (f == Elem::F16) return "hf::f16_to_f32(" + s + ")";
    if (f == Elem::F64) return "((float)(" + s + "))";
    if (f == Elem::F8E4M3FN) return "hf::fp8_to_f32<0>(" + s + ")";
    if (f == Elem::F8E5M2) return "hf::fp8_to_f32<1>(" + s + ")";
    throw CompileError("internal: toF32");
  };
  if (isFloat(from) && isFloat(to)) {
    if (to == Elem::F64) return "((double)" + toF32(x, from) + ")";
    std::string f = toF32(x, from);
    if (to == Elem::F32) return f;
    if (to == Elem::BF16) return "hf::f32_to_bf16<0>(" + f + ")";
    if (to == Elem::F8E4M3FN) return "hf::f32_to_fp8<0, 0, false>(" + f + ")";
    if (to == Elem::F8E5M2) return "hf::f32_to_fp8<1, 0, false>(" + f + ")";
    return "hf::f32_to_f16<0>(" + f + ")";
  }
  if (isInt(from) && isFloat(to)) {
    bool uns = unsignedCast || from == Elem::I1;
    std::string iv = uns ? "(int64_t)(uint" + std::to_string(std::max(8, elemBits(from))) + "_t)(" + x + ")"
                         : "(int64_t)(" + x + ")";
    if (from == Elem::I1) iv = "(int64_t)(" + x + ")";
    if (to == Elem::F64) return "((double)" + iv + ")";
    if (to == Elem::F32) return "hf::int_to_f32<0>(" + iv + ")";
    if (to == Elem::F8E4M3FN) return "hf::to_fp8<0, 0, false>((double)" + iv + ")";
    if (to == Elem::F8E5M2) return "hf::to_fp8<1, 0, false>((double)" + iv + ")";
    if (to == Elem::BF16) return "hf::f32_to_bf16<0>((float)hf::round_to_format((double)" + iv + ", 8, -126, 127, 0))";
    return "hf::f32_to_f16<0>((float)hf::round_to_format((double)" + iv + ", 11, -14, 15, 0))";
  }
  if (isFloat(from) && isInt(to)) {
    std::string f = from == Elem::F64 ? x : toF32(x, from);
    if (to == Elem::I1) return "((" + f + ") != 0)";
    return "hf::fptosi<" + ctype(to) + ">(" + f + ")";
  }
  // int -> int
  if (to == Elem::I1) return "((" + x + ") & 1)";
  if (from == Elem::I1 || (unsignedCast && elemBits(to) > elemBits(from)))
    return "(" + ctype(to) + ")(uint" + std::to_string(std::max(8, elemBits(from))) + "_t)(" + x + ")";
  return "(" + ctype(to) + ")(" + x + ")";
}

// hfusion.cast with its declared RoundMode (HFusionEnums.td:122-141) and
// enable_saturate (HFusionNamedStructuredOps.yaml:375-432).
std::string declaredCastExpr(const std::string &x, Elem from, Elem to, int mode, bool sat, bool uns) {
  if (from == Elem::Index) from = Elem::I64;
  if (to == Elem::Index) to = Elem::I64;
  std::string M = std::to_string(mode);
  if (isFloat(from) && isFloat(to)) {
    std::string f = castExpr(x, from, Elem::F32, false);
    if (from == to) {
      if (to == Elem::F32) return "hf::round_integral<" + M + ">(" + f + ")";
      std::string r = "hf::round_integral<" + M + ">(" + f + ")";
      return castExpr(r, Elem::F32, to, false);
    }
    if (to == Elem::F32) return f;
    if (to == Elem::F64) return "((double)" + f + ")";
    if (from == Elem::F64) f = "((float)(" + x + "))";
    if (to == Elem::BF16) return "hf::f32_to_bf16<" + M + ">(" + f + ")";
    if (to == Elem::F8E4M3FN || to == Elem::F8E5M2)
      return std::string("hf::f32_to_fp8<") + (to == Elem::F8E4M3FN ? "0" : "1") + ", " + M + ", " + (sat ? "true" : "false") +
             ">(" + f + ")";
    return "hf::f32_to_f16<" + M + ">(" + f + ")";
  }
  if (isFloat(from) && isInt(to)) {
    std::string f = castExpr(x, from, Elem::F32, false);
    if (to == Elem::I1) return "((" + f + ") != 0)";
    return "hf::f32_to_int<" + ctype(to) + ", " + M + ", " + (sat ? "true" : "false") + ">(" + f + ")";
  }
  if (isInt(from) && isFloat(to)) {
    std::string iv = (uns || from == Elem::I1) && from != Elem::I64
                         ? "(int64_t)(uint" + std::to_string(std::max(8, elemBits(from))) + "_t)(" + x + ")"
                         : "(int64_t)(" + x + ")";
    if (to == Elem::F32) return "hf::int_to_f32<" + M + ">(" + iv + ")";
    if (to == Elem::F64) return "((double)" + iv + ")";
    if (to == Elem::F8E4M3FN || to == Elem::F8E5M2)
      return std::string("hf::to_fp8<") + (to == Elem::F8E4M3FN ? "0" : "1") + ", " + M + ", " + (sat ? "true" : "false") +
             ">((double)" + iv + ")";
    if (to == Elem::BF16) return "hf::f32_to_bf16<0>((float)hf::round_to_format((double)" + iv + ", 8, -126, 127, " + M + "))";
    return "hf::f32_to_f16<0>((float)hf::round_to_format((double)" + iv + ", 11, -14, 15, " + M + "))";
  }
  // int -> int
  if (sat && elemBits(to) < elemBits(from) && to != Elem::I1) {
    int b = elemBits(to);
    std::string lo = "(-(int64_t)1 << " + std::to_string(b - 1) + ")";
    std::string hi = "(((int64_t)1 << " + std::to_string(b - 1) + ") - 1)";
    return "(" + ctype(to) + ")(((int64_t)(" + x + ")) < " + lo + " ? " + lo + " : (((int64_t)(" + x + ")) > " + hi + " ? " + hi + " : (int64_t)(" + x + ")))";
  }
  return castExpr(x, from, to, uns);
}

std::string f32UnaryFn(const std::string &fn, const std::string &x, const Op *op) {
  if (fn == "sqrt") return "__builtin_sqrtf(" + x + ")";
  if (fn == "rsqrt") return "hf::rsqrt(" + x + ")";
  if (fn == "exp") return "hf::exp_f32(" + x + ")";
  if (fn == "exp2") return "exp2f(" + x + ")";
  if (fn == "log") return "logf(" + x + ")";
  if (fn == "log2") return "log2f(" + x + ")";
  if (fn == "log10") return "log10f(" + x + ")";
  if (fn == "log1p") return "log1pf(" + x + ")";
  if (fn == "expm1") return "expm1f(" + x + ")";
  if (fn == "abs" || fn == "absf") return "__builtin_fabsf(" + x + ")";
  if (fn == "negf" || fn == "neg") return "(-(" + x + "))";
  if (fn == "relu") return "hf::relu(" + x + ")";
  if (fn == "rec" || fn == "reciprocal") return "hf::rec(" + x + ")";
  if (fn == "tanh") return "tanhf(" + x + ")";
  if (fn == "sin") return "sinf(" + x + ")";
  if (fn == "cos") return "cosf(" + x + ")";
  if (fn == "erf") return "erff(" + x + ")";
  if (fn == "nearbyint") return "__builtin_roundevenf(" + x + ")";
  if (fn == "ceil") return "__builtin_ceilf(" + x + ")";
  if (fn == "floor") return "__builtin_floorf(" + x + ")";
  if (fn == "round") return "__builtin_roundf(" + x + ")";
  if (fn == "square") return "((" + x + ") * (" + x + "))";
  if (fn == "trunc") return "__builtin_truncf(" + x + ")";
  // math.tan .. math.cosh: the device libm (HFusionOps.cpp:443-480)
  static const std::set<std::string> libm = {"tan", "acos", "acosh", "asin", "asinh", "atan", "atanh",
                                             "sinh", "cosh", "lgamma"};
  if (libm.count(fn)) return fn + "f(" + x + ")";
  if (fn == "ilogb") return "hf::ilogb_f(" + x + ")";
  unsupported(op, "unary function '" + fn + "' on f32");
}

std::string f32BinaryFn(const std::string &fn, const std::string &a, const std::string &b, const Op *op) {
  if (fn == "add") return "(" + a + " + " + b + ")";
  if (fn == "sub") return "(" + a + " - " + b + ")";
  if (fn == "mul") return "(" + a + " * " + b + ")";
  if (fn == "div" || fn == "div_unsigned") return "(" + a + " / " + b + ")";
  if (fn == "maxf" || fn == "max_signed" || fn == "max_unsigned") return "hf::maximumf(" + a + ", " + b + ")";
  if (fn == "minf" || fn == "min_signed" || fn == "min_unsigned") return "hf::minimumf(" + a + ", " + b + ")";
  if (fn == "maxnumf") return "hf::maxnumf(" + a + ", " + b + ")";
  if (fn == "minnumf") return "hf::minnumf(" + a + ", " + b + ")";
  if (fn == "powf") return "powf(" + a + ", " + b + ")";
  if (fn == "mod" || fn == "modui") return "fmodf(" + a + ", " + b + ")";
  if (fn == "copysign") return "copysignf(" + a + ", " + b + ")";
  if (fn == "atan2") return "atan2f(" + a + ", " + b + ")";
  if (fn == "ldexp") return "hf::ldexp_f(" + a + ", " + b + ")";
  if (fn == "divfhp") return "(" + a + " / " + b + ")";
  unsupported(op, "binary function '" + fn + "' on floats");
}

std::string intBinaryFn(const std::string &fn, const std::string &a, const std::string &b, Elem t, const Op *op) {
  std::string T = ctype(t);
  std::string A = "(int64_t)(" + a + ")", B = "(int64_t)(" + b + ")";
  std::string U = "uint" + std::to_string(std::max(8, elemBits(t))) + "_t";
  if (fn == "add") return "(" + T + ")((uint64_t)" + A + " + (uint64_t)" + B + ")";
  if (fn == "sub") return "(" + T + ")((uint64_t)" + A + " - (uint64_t)" + B + ")";
  if (fn == "mul") return "(" + T + ")((uint64_t)" + A + " * (uint64_t)" + B + ")";
  if (fn == "div") return "(" + T + ")(" + B + " == 0 ? 0 : " + A + " / " + B + ")";
  if (fn == "mod") return "(" + T + ")(" + B + " == 0 ? 0 : " + A + " % " + B + ")";
  if (fn == "max_signed" || fn == "maxsi") return "(" + A + " > " + B + " ? (" + T + ")(" + a + ") : (" + T + ")(" + b + "))";
  if (fn == "min_signed" || fn == "minsi") return "(" + A + " < " + B + " ? (" + T + ")(" + a + ") : (" + T + ")(" + b + "))";
  if (fn == "max_unsigned") return "((" + U + ")(" + a + ") > (" + U + ")(" + b + ") ? (" + T + ")(" + a + ") : (" + T + ")(" + b + "))";
  if (fn == "min_unsigned") return "((" + U + ")(" + a + ") < (" + U + ")(" + b + ") ? (" + T + ")(" + a + ") : (" + T + ")(" + b + "))";
  if (fn == "vand") return "(" + T + ")(" + A + " & " + B + ")";
  if (fn == "vor") return "(" + T + ")(" + A + " | " + B + ")";
  if (fn == "vxor") return "(" + T + ")(" + A + " ^ " + B + ")";
  if (fn == "shli") return "(" + T + ")((uint64_t)" + A + " << " + B + ")";
  if (fn == "shrsi") return "(" + T + ")(" + A + " >> " + B + ")";
  if (fn == "shrui") return "(" + T + ")((" + U + ")(" + a + ") >> " + B + ")";
  if (fn == "floordivsi") return "(" + T + ")hf_floordiv(" + A + ", " + B + ")";
  if (fn == "ceildivsi") return "(" + T + ")hf_ceildiv(" + A + ", " + B + ")";
  if (fn == "powi") return "(" + T + ")hf::ipowi(" + A + ", " + B + ")";
  if (fn == "ceildivui") return "(" + T + ")hf::ceildivu((" + U + ")(" + a + "), (" + U + ")(" + b + "))";
  if (fn == "modui") return "(" + T + ")hf::remu((" + U + ")(" + a + "), (" + U + ")(" + b + "))";
  unsupported(op, "binary function '" + fn + "' on integers");
}

// Applies a float-domain expression builder in element type U (f16/bf16/fp8
// are computed in f32 and rounded back, as LLVM promotes them on the CPU).
std::string inFloatType(Elem U, const std::vector<std::string> &xs,
                        const std::function<std::string(const std::vector<std::string> &)> &f32fn) {
  if (U == Elem::F32) return f32fn(xs);
  // bf16, f16 and the fp8 formats compute in f32 and round back to nearest
  // even after each op, as the CPU lowering's float emulation does
  if (U == Elem::BF16 || U == Elem::F16 || U == Elem::F8E4M3FN || U == Elem::F8E5M2) {
    std::vector<std::string> ys;
    for (auto &x : xs) ys.push_back(castExpr(x, U, Elem::F32, false));
    return castExpr(f32fn(ys), Elem::F32, U, false);
  }
  if (U == Elem::F64) {
    // f64 math: the f32 builders with double arguments resolve to the double
    // overloads of the arithmetic operators; named libm calls are mapped.
    std::string s = f32fn(xs);
    const char *pairs[][2] = {{"__builtin_sqrtf", "__builtin_sqrt"}, {"expf", "exp"}, {"logf", "log"},
                              {"__builtin_fabsf", "__builtin_fabs"}, {"hf::maximumf", "__builtin_elementwise_maximum"},
                              {"hf::minimumf", "__builtin_elementwise_minimum"}, {"__builtin_roundevenf", "__builtin_roundeven"},
                              {"__builtin_floorf", "__builtin_floor"}, {"__builtin_ceilf", "__builtin_ceil"}};
    for (auto &p : pairs) {
      size_t pos;
      while ((pos = s.find(p[0])) != std::string::npos) s.replace(pos, std::strlen(p[0]), p[1]);
    }
    return s;
  }
  throw CompileError("float function on non-float type");
}

int roundModeOf(const std::string &s) {
  if (s.empty() || s == "rint") return 0;
  if (s == "round") return 1;
  if (s == "floor") return 2;
  if (s == "ceil") return 3;
  if (s == "trunc") return 4;
  if (s == "odd") return 5;
  if (s == "truncwithoverflow") return 6;
  throw CompileError("unknown round_mode '" + s + "'");
}

// ---- linalg.generic (elementwise subset) ---------------------------------
// A map `affine_map<(d0, d1) -> (d1)>` as its result dims ({1}); false for
// results that are not plain dims.
bool parseAffineMap(const std::string &txt, int &nd, std::vector<int> &res) {
  const size_t arrow = txt.find("->");
  if (arrow == std::string::npos) return false;
  const std::string lhs = txt.substr(0, arrow), rhs = txt.substr(arrow + 2);
  nd = 0;
  for (size_t i = 0; i + 1 < lhs.size(); ++i) if (lhs[i] == 'd' && std::isdigit((unsigned char)lhs[i + 1])) ++nd;
  res.clear();
  const size_t a = rhs.find('('), b = rhs.rfind(')');
  if (a == std::string::npos || b == std::string::npos || b < a) return false;
  std::stringstream ss(rhs.substr(a + 1, b - a - 1));
  std::string tok;
  while (std::getline(ss, tok, ',')) {
    tok.erase(std::remove_if(tok.begin(), tok.end(), [](char c) { return std::isspace((unsigned char)c); }), tok.end());
    if (tok.empty()) continue;
    if (tok.size() < 2 || tok[0] != 'd') return false;
    for (size_t i = 1; i < tok.size(); ++i) if (!std::isdigit((unsigned char)tok[i])) return false;
    res.push_back(std::stoi(tok.substr(1)));
  }
  return true;
}

// indexing maps of a linalg.generic, one per ins then outs operand
bool genericMaps(const Op *op, std::vector<std::vector<int>> &maps, int &nd) {
  const std::string s = op->attr("indexing_maps");
  maps.clear();
  size_t q = 0;
  while ((q = s.find("affine_map<", q)) != std::string::npos) {
    const size_t arrow = s.find("->", q);
    if (arrow == std::string::npos) return false;
    size_t e = s.find('>', arrow + 2);
    if (e == std::string::npos) return false;
    std::vector<int> r;
    int n;
    if (!parseAffineMap(s.substr(q + 11, e - q - 11), n, r)) return false;
    nd = n;
    maps.push_back(r);
    q = e;
  }
  return maps.size() == op->ins.size() + op->outs.size();
}

// a linalg.generic the elementwise emitters take: parallel loops only, every
// output indexed by the identity map, inputs by plain-dim projections in
// increasing order (broadcasts; a transposed input is rejected)
bool genericIsElementwise(const Op *op) {
  if (op->name != "linalg.generic" || op->attr("region").empty() || op->outs.size() != 1) return false;
  if (op->attr("iterator_types").find("reduction") != std::string::npos) return false;
  std::vector<std::vector<int>> maps;
  int nd = 0;
  if (!genericMaps(op, maps, nd)) return false;
  const auto &om = maps.back();
  if ((int)om.size() != nd) return false;
  for (int i = 0; i < nd; ++i) if (om[i] != i) return false;
  // inputs: dims in increasing order (broadcasts, no transposes)
  for (size_t i = 0; i + 1 < maps.size(); ++i)
    for (size_t k = 1; k < maps[i].size(); ++k) if (maps[i][k] <= maps[i][k - 1]) return false;
  return true;
}

bool isElementwiseOp(const Op *op) {
  if (op->name == "linalg.generic") return genericIsElementwise(op);
  static const std::set<std::string> s = {
      "hfusion.elemwise_unary", "hfusion.elemwise_binary", "hfusion.elemwise_ternary",
      "linalg.elemwise_unary",  "linalg.elemwise_binary",  "hfusion.compare",
      "hfusion.select",         "hfusion.cast",            "arith.addf", "arith.subf",
      "arith.mulf",             "arith.divf",              "arith.maximumf", "arith.minimumf",
      "arith.negf",             "arith.extf",              "arith.truncf", "arith.sitofp",
      "arith.fptosi",           "arith.addi",              "arith.subi", "arith.muli",
      "linalg.add", "linalg.sub", "linalg.mul", "linalg.div", "linalg.max", "linalg.min",
      "linalg.exp", "linalg.abs", "linalg.negf", "linalg.sqrt", "linalg.rsqrt", "linalg.reciprocal",
      "hfusion.isinf", "hfusion.isnan", "hfusion.isfinite", "hfusion.nextafter", "hfusion.hypot", "hfusion.erfinv",
      "hfusion.bitcast", "hfusion.signbit", "hfusion.cyl_bessel_i0"};
  return s.count(op->name) != 0;
}

// arith.bitcast (the `bitcast` type_fn, HFusionOps.cpp:752-756): the same
// bits read as a type of the same width.
std::string bitcastExpr(const std::string &x, Elem from, Elem to, const Op *op) {
  if (from == to) return x;
  if (from == Elem::I1 || to == Elem::I1 || elemBits(from) != elemBits(to)) unsupported(op, "bitcast between widths");
  return "__builtin_bit_cast(" + ctype(to) + ", (" + ctype(from) + ")(" + x + "))";
}

// Element expression of a linalg.generic's result: its region's scalar
// arith / math statements, each translated with the same helpers as the
// named ops (f16/bf16/fp8 computed in f32 and rounded back per op).
// `a`/`at` hold the ins operands, then the captured outer values in the
// order of attrs["captures"].
std::string genericExpr(const Op *op, const std::vector<std::string> &a, const std::vector<Elem> &at, Elem U) {
  const std::string body = op->attr("region");
  const size_t lp = body.find('('), rp = body.find(')');
  if (lp == std::string::npos || rp == std::string::npos) unsupported(op, "linalg.generic region header");
  struct V { std::string e; Elem t; };
  std::map<std::string, V> env;
  {
    std::stringstream ss(body.substr(lp + 1, rp - lp - 1));
    std::string arg;
    size_t i = 0;
    while (std::getline(ss, arg, ',')) {
      const size_t c = arg.find(':');
      if (c == std::string::npos) continue;
      std::string nm = arg.substr(0, c), ty = arg.substr(c + 1);
      nm.erase(std::remove_if(nm.begin(), nm.end(), ::isspace), nm.end());
      ty.erase(std::remove_if(ty.begin(), ty.end(), ::isspace), ty.end());
      if (i < op->ins.size()) env[nm] = {a.at(i), parseElem(ty)};
      else env[nm] = {"", Elem::None}; // the output's block argument: not readable here
      ++i;
    }
  }
  {
    std::stringstream ss(op->attr("captures"));
    std::string nm;
    size_t j = op->ins.size();
    while (ss >> nm) { env[nm] = {a.at(j), at.at(j)}; ++j; }
  }
  auto get = [&](const std::string &nm) -> V {
    auto it = env.find(nm);
    if (it == env.end()) unsupported(op, "region value " + nm);
    if (it->second.t == Elem::None) unsupported(op, "a region that reads its output");
    return it->second;
  };
  static const std::map<std::string, std::string> fbin = {
      {"arith.addf", "add"}, {"arith.subf", "sub"}, {"arith.mulf", "mul"}, {"arith.divf", "div"},
      {"arith.maximumf", "maxf"}, {"arith.minimumf", "minf"}, {"arith.maxnumf", "maxnumf"}, {"arith.minnumf", "minnumf"},
      {"arith.remf", "mod"}, {"math.powf", "powf"}, {"math.atan2", "atan2"}, {"math.copysign", "copysign"}};
  static const std::map<std::string, std::string> fun = {
      {"arith.negf", "negf"}, {"math.exp", "exp"}, {"math.exp2", "exp2"}, {"math.log", "log"}, {"math.log2", "log2"},
      {"math.log10", "log10"}, {"math.log1p", "log1p"}, {"math.expm1", "expm1"}, {"math.sqrt", "sqrt"},
      {"math.rsqrt", "rsqrt"}, {"math.tanh", "tanh"}, {"math.sin", "sin"}, {"math.cos", "cos"}, {"math.tan", "tan"},
      {"math.erf", "erf"}, {"math.absf", "abs"}, {"math.floor", "floor"}, {"math.ceil", "ceil"}, {"math.round", "round"},
      {"math.roundeven", "nearbyint"}, {"math.trunc", "trunc"}, {"math.atan", "atan"}, {"math.asin", "asin"},
      {"math.acos", "acos"}, {"math.sinh", "sinh"}, {"math.cosh", "cosh"}, {"math.asinh", "asinh"},
      {"math.acosh", "acosh"}, {"math.atanh", "atanh"}};
  static const std::map<std::string, std::string> ibin = {
      {"arith.addi", "add"}, {"arith.subi", "sub"}, {"arith.muli", "mul"}, {"arith.divsi", "div"}, {"arith.remsi", "mod"},
      {"arith.remui", "modui"}, {"arith.andi", "vand"}, {"arith.ori", "vor"}, {"arith.xori", "vxor"},
      {"arith.shli", "shli"}, {"arith.shrsi", "shrsi"}, {"arith.shrui", "shrui"}, {"arith.maxsi", "max_signed"},
      {"arith.minsi", "min_signed"}, {"arith.maxui", "max_unsigned"}, {"arith.minui", "min_unsigned"},
      {"arith.ceildivsi", "ceildivsi"}, {"arith.floordivsi", "floordivsi"}, {"arith.ceildivui", "ceildivui"},
      {"math.ipowi", "powi"}};
  std::stringstream lines(body.substr(body.find(':', rp) == std::string::npos ? rp + 1 : body.find(':', rp) + 1));
  std::string line;
  while (std::getline(lines, line)) {
    const size_t b0 = line.find_first_not_of(" \t");
    if (b0 == std::string::npos) continue;
    line = line.substr(b0);
    // strip `fastmath<...>` and attribute dictionaries
    for (size_t q; (q = line.find("fastmath<")) != std::string::npos;) line.erase(q, line.find('>', q) - q + 1);
    for (size_t q; (q = line.find('{')) != std::string::npos;) line.erase(q, line.find('}', q) - q + 1);
    const size_t colon = line.rfind(':');
    std::string head = colon == std::string::npos ? line : line.substr(0, colon);
    std::string tail = colon == std::string::npos ? "" : line.substr(colon + 1);
    auto trim = [](std::string x) {
      x.erase(0, x.find_first_not_of(" \t"));
      x.erase(x.find_last_not_of(" \t") + 1);
      return x;
    };
    std::string toTy;
    if (tail.find(" to ") != std::string::npos) {
      toTy = trim(tail.substr(tail.find(" to ") + 4));
      tail = tail.substr(0, tail.find(" to "));
    }
    tail = trim(tail);
    std::vector<std::string> names;
    for (size_t q = 0; (q = head.find('%', q)) != std::string::npos;) {
      size_t e = q + 1;
      while (e < head.size() && (std::isalnum((unsigned char)head[e]) || head[e] == '_' || head[e] == '.' || head[e] == '#')) ++e;
      names.push_back(head.substr(q, e - q));
      q = e;
    }
    if (line.rfind("linalg.yield", 0) == 0) {
      if (names.size() != 1) unsupported(op, "linalg.yield of other than one value");
      V y = get(names[0]);
      return castExpr(y.e, y.t, U, false);
    }
    const size_t eq = head.find('=');
    if (eq == std::string::npos || names.empty()) unsupported(op, "region statement '" + line + "'");
    const std::string res = names[0];
    std::string rest = trim(head.substr(eq + 1));
    const std::string opn = rest.substr(0, rest.find_first_of(" \t"));
    rest = trim(rest.substr(opn.size()));
    std::vector<V> xs;
    for (size_t i = 1; i < names.size(); ++i) xs.push_back(get(names[i]));
    const Elem ty = tail.empty() ? (xs.empty() ? Elem::None : xs[0].t) : parseElem(tail);
    V out;
    if (opn == "arith.constant") {
      Value tmp;
      tmp.type.elem = ty;
      std::string lit = rest;
      if (!parseLiteral(lit, ty, &tmp)) unsupported(op, "region constant '" + lit + "'");
      out = {constExpr(&tmp, ty), ty};
    } else if (fbin.count(opn)) {
      out = {inFloatType(ty, {xs.at(0).e, xs.at(1).e}, [&](const std::vector<std::string> &y) {
               return f32BinaryFn(fbin.at(opn), y[0], y[1], op); }), ty};
    } else if (fun.count(opn)) {
      out = {inFloatType(ty, {xs.at(0).e}, [&](const std::vector<std::string> &y) { return f32UnaryFn(fun.at(opn), y[0], op); }), ty};
    } else if (opn == "math.fma") {
      out = {inFloatType(ty, {xs.at(0).e, xs.at(1).e, xs.at(2).e}, [&](const std::vector<std::string> &y) {
               return "fmaf(" + y[0] + ", " + y[1] + ", " + y[2] + ")"; }), ty};
    } else if (ibin.count(opn)) {
      out = {intBinaryFn(ibin.at(opn), xs.at(0).e, xs.at(1).e, ty, op), ty};
    } else if (opn == "arith.select") {
      const Elem vt = xs.at(1).t;
      out = {"(" + xs.at(0).e + " ? " + xs.at(1).e + " : " + xs.at(2).e + ")", vt};
    } else if (opn == "arith.cmpf" || opn == "arith.cmpi") {
      const std::string pred = trim(rest.substr(0, rest.find(',')));
      const Elem ot = xs.at(0).t;
      std::string e;
      if (opn == "arith.cmpf") {
        const std::string x = castExpr(xs[0].e, ot, Elem::F32, false), y = castExpr(xs[1].e, ot, Elem::F32, false);
        static const std::map<std::string, std::string> P = {
            {"oeq", "(@X == @Y)"}, {"one", "(@X < @Y || @X > @Y)"}, {"olt", "(@X < @Y)"}, {"ole", "(@X <= @Y)"},
            {"ogt", "(@X > @Y)"}, {"oge", "(@X >= @Y)"}, {"ord", "(@X == @X && @Y == @Y)"},
            {"ueq", "!(@X < @Y || @X > @Y)"}, {"une", "!(@X == @Y)"}, {"ult", "!(@X >= @Y)"}, {"ule", "!(@X > @Y)"},
            {"ugt", "!(@X <= @Y)"}, {"uge", "!(@X < @Y)"}, {"uno", "(@X != @X || @Y != @Y)"}, {"true", "true"},
            {"false", "false"}};
        if (!P.count(pred)) unsupported(op, "cmpf predicate " + pred);
        e = P.at(pred);
        for (size_t q; (q = e.find("@X")) != std::string::npos;) e.replace(q, 2, "(" + x + ")");
        for (size_t q; (q = e.find("@Y")) != std::string::npos;) e.replace(q, 2, "(" + y + ")");
      } else {
        const std::string x = "(int64_t)(" + xs[0].e + ")", y = "(int64_t)(" + xs[1].e + ")";
        const int bits = elemBits(ot == Elem::Index ? Elem::I64 : ot);
        const std::string mask = bits >= 64 ? "" : " & " + std::to_string((1ull << bits) - 1) + "ull";
        const std::string UX = "((uint64_t)(" + x + ")" + mask + ")", UY = "((uint64_t)(" + y + ")" + mask + ")";
        static const std::map<std::string, std::string> P = {
            {"eq", "=="}, {"ne", "!="}, {"slt", "<"}, {"sle", "<="}, {"sgt", ">"}, {"sge", ">="},
            {"ult", "<"}, {"ule", "<="}, {"ugt", ">"}, {"uge", ">="}};
        if (!P.count(pred)) unsupported(op, "cmpi predicate " + pred);
        e = pred[0] == 'u' ? "(" + UX + " " + P.at(pred) + " " + UY + ")" : "(" + x + " " + P.at(pred) + " " + y + ")";
      }
      out = {"(bool)" + e, Elem::I1};
    } else if (opn == "arith.extf" || opn == "arith.truncf" || opn == "arith.sitofp" || opn == "arith.uitofp" ||
               opn == "arith.fptosi" || opn == "arith.fptoui" || opn == "arith.extsi" || opn == "arith.extui" ||
               opn == "arith.trunci" || opn == "arith.index_cast" || opn == "arith.index_castui") {
      const Elem to = parseElem(toTy);
      const bool uns = opn == "arith.uitofp" || opn == "arith.fptoui" || opn == "arith.extui" || opn == "arith.index_castui";
      out = {castExpr(xs.at(0).e, xs.at(0).t, to, uns), to};
    } else if (opn == "arith.bitcast") {
      const Elem to = parseElem(toTy);
      out = {bitcastExpr(xs.at(0).e, xs.at(0).t, to, op), to};
    } else {
      unsupported(op, "region op '" + opn + "'");
    }
    env[res] = out;
  }
  unsupported(op, "linalg.generic region without linalg.yield");
}

// Element expression of an elementwise op's result from operand expressions.
std::string elementExpr(const Op *op, const std::vector<std::string> &a, const std::vector<Elem> &at, Elem U) {
  const std::string &n = op->name;
  if (n == "linalg.generic") return genericExpr(op, a, at, U);
  bool uns = op->attr("cast") == "cast_unsigned";
  bool bits = op->attr("cast") == "bitcast";
  auto named = [&](const std::string &fn, int arity) -> std::string {
    if ((int)a.size() != arity) unsupported(op, "operand count");
    std::vector<std::string> xs;
    for (int i = 0; i < arity; ++i) xs.push_back(bits ? bitcastExpr(a[i], at[i], U, op) : castExpr(a[i], at[i], U, uns));
    if (isFloat(U)) {
      // exp rounded onto bf16 / f16: the guarded evaluation that rounds as
      // the CPU's f32 expf does
      if (arity == 1 && fn == "exp" && (U == Elem::BF16 || U == Elem::F16))
        return castExpr("hf::exp_narrow<" + std::string(U == Elem::BF16 ? "8" : "11") + ">(" + castExpr(xs[0], U, Elem::F32, false) + ")",
                        Elem::F32, U, false);
      if (arity == 1) return inFloatType(U, xs, [&](const std::vector<std::string> &y) { return f32UnaryFn(fn, y[0], op); });
      if (arity == 2) return inFloatType(U, xs, [&](const std::vector<std::string> &y) { return f32BinaryFn(fn, y[0], y[1], op); });
      if (fn == "fma")
        return inFloatType(U, xs, [&](const std::vector<std::string> &y) { return "fmaf(" + y[0] + ", " + y[1] + ", " + y[2] + ")"; });
      if (fn == "select") return "(" + a[0] + " ? " + xs[1] + " : " + xs[2] + ")";
      unsupported(op, "ternary function '" + fn + "'");
    }
    std::string T = ctype(U);
    if (arity == 1) {
      if (fn == "relu") return "(" + T + ")((int64_t)(" + xs[0] + ") > 0 ? (int64_t)(" + xs[0] + ") : 0)";
      if (fn == "vnot") return "(" + T + ")(~(int64_t)(" + xs[0] + "))";
      if (fn == "absi" || fn == "abs") return "(" + T + ")((int64_t)(" + xs[0] + ") < 0 ? -(int64_t)(" + xs[0] + ") : (int64_t)(" + xs[0] + "))";
      if (fn == "rec") return "(" + T + ")((int64_t)(" + xs[0] + ") == 0 ? 0 : 1 / (int64_t)(" + xs[0] + "))";
      unsupported(op, "unary function '" + fn + "' on integers");
    }
    if (arity == 2) return intBinaryFn(fn, xs[0], xs[1], U, op);
    if (fn == "select") return "(" + a[0] + " ? " + xs[1] + " : " + xs[2] + ")";
    unsupported(op, "ternary function '" + fn + "' on integers");
  };
  if (n == "hfusion.elemwise_unary") return named(op->attr("fun", "sqrt"), 1);
  if (n == "linalg.elemwise_unary") return named(op->attr("fun", "exp"), 1);
  if (n == "hfusion.elemwise_binary") return named(op->attr("fun", "vand"), 2);
  if (n == "linalg.elemwise_binary") return named(op->attr("fun", "add"), 2);
  if (n == "hfusion.elemwise_ternary") {
    std::string fn = op->attr("fun", "fma");
    if (fn == "select") {
      // select keeps the i1 condition uncast
      std::vector<std::string> xs = {a[0], castExpr(a[1], at[1], U, uns), castExpr(a[2], at[2], U, uns)};
      return "(" + xs[0] + " ? " + xs[1] + " : " + xs[2] + ")";
    }
    return named(fn, 3);
  }
  // float predicates and math ops of HFusionOps.td:251-305, 1309-1400 (no outs:
  // operands and result type come from the op's own syntax)
  if (n == "hfusion.isinf" || n == "hfusion.isnan" || n == "hfusion.isfinite") {
    if (a.size() != 1 || !isFloat(at[0])) unsupported(op, "operand of " + n);
    std::string f = castExpr(a[0], at[0], Elem::F32, false);
    std::string pred = n == "hfusion.isinf" ? "__builtin_isinf" : n == "hfusion.isnan" ? "__builtin_isnan" : "__builtin_isfinite";
    return castExpr("(bool)" + pred + "(" + f + ")", Elem::I1, U, false);
  }
  if (n == "hfusion.signbit") {
    // HFusionOps.td:1295: 1 / true where the sign bit is set (f16 -> f32 keeps it)
    if (a.size() != 1 || (at[0] != Elem::F32 && at[0] != Elem::F16)) unsupported(op, "operand of hfusion.signbit");
    if (U != Elem::I1 && U != Elem::I8) unsupported(op, "result type of hfusion.signbit");
    std::string f = castExpr(a[0], at[0], Elem::F32, false);
    return castExpr("(bool)__builtin_signbitf(" + f + ")", Elem::I1, U, false);
  }
  if (n == "hfusion.nextafter") {
    if (a.size() != 2 || at[0] != U || at[1] != U) unsupported(op, "operands of hfusion.nextafter");
    if (U == Elem::F32) return "nextafterf(" + a[0] + ", " + a[1] + ")";
    if (U == Elem::F16) return "hf::nextafter_h(" + a[0] + ", " + a[1] + ")";
    unsupported(op, "hfusion.nextafter on this type");
  }
  if (n == "hfusion.hypot") {
    if ((a.size() != 2 && a.size() != 3)) unsupported(op, "operand count of hfusion.hypot");
    for (auto e : at) if (e != U) unsupported(op, "mixed operand types of hfusion.hypot");
    if (U != Elem::F32 && U != Elem::F16) unsupported(op, "hfusion.hypot on this type");
    std::vector<std::string> f;
    for (size_t i = 0; i < a.size(); ++i) f.push_back(castExpr(a[i], at[i], Elem::F32, false));
    std::string z = a.size() == 3 ? f[2] : "0.0f";
    std::string e = std::string(U == Elem::F32 ? "hf::hypot_scaled(" : "hf::hypot_direct(") + f[0] + ", " + f[1] + ", " + z +
                    ", " + std::to_string(a.size()) + ")";
    return castExpr(e, Elem::F32, U, false);
  }
  if (n == "hfusion.cyl_bessel_i0") {
    if (a.size() != 1 || at[0] != U || (U != Elem::F32 && U != Elem::F16)) unsupported(op, "operand of hfusion.cyl_bessel_i0");
    return castExpr("hf::cyl_bessel_i0_f(" + castExpr(a[0], U, Elem::F32, false) + ")", Elem::F32, U, false);
  }
  if (n == "hfusion.erfinv") {
    if (a.size() != 1 || at[0] != U || (U != Elem::F32 && U != Elem::F16)) unsupported(op, "operand of hfusion.erfinv");
    return castExpr("hf::erfinv_f(" + castExpr(a[0], U, Elem::F32, false) + ")", Elem::F32, U, false);
  }
  if (n == "hfusion.bitcast") return bitcastExpr(a[0], at[0], U, op);
  if (n == "hfusion.select") return "(" + a[0] + " ? " + a[1] + " : " + a[2] + ")";
  if (n == "hfusion.compare") {
    std::string fn = op->attr("compare_fn", "veq");
    Elem T = at[0];
    std::string x = a[0], y = a[1];
    if (T == Elem::BF16 || T == Elem::F16) { x = castExpr(x, T, Elem::F32, false); y = castExpr(y, T, Elem::F32, false); }
    if (fn == "veq") return "(" + x + " == " + y + ")";
    if (fn == "vne") return "!(" + x + " == " + y + ")";
    if (fn == "vlt") return "(" + x + " < " + y + ")";
    if (fn == "vle") return "(" + x + " <= " + y + ")";
    if (fn == "vgt") return "(" + x + " > " + y + ")";
    if (fn == "vge") return "(" + x + " >= " + y + ")";
    std::string U2 = "uint" + std::to_string(std::max(8, elemBits(T))) + "_t";
    if (fn == "vult") return "((" + U2 + ")(" + x + ") < (" + U2 + ")(" + y + "))";
    if (fn == "vule") return "((" + U2 + ")(" + x + ") <= (" + U2 + ")(" + y + "))";
    if (fn == "vugt") return "((" + U2 + ")(" + x + ") > (" + U2 + ")(" + y + "))";
    if (fn == "vuge") return "((" + U2 + ")(" + x + ") >= (" + U2 + ")(" + y + "))";
    unsupported(op, "compare function '" + fn + "'");
  }
  if (n == "hfusion.cast") {
    int mode = roundModeOf(op->attr("round_mode", "rint"));
    bool sat = op->attr("enable_saturate") == "true";
    bool u = uns || op->attr("unsigned_mode").find("ui2") != std::string::npos;
    return declaredCastExpr(a[0], at[0], U, mode, sat, u);
  }
  // plain arith / linalg named ops on tensors
  static const std::map<std::string, std::string> bin = {
      {"arith.addf", "add"}, {"arith.subf", "sub"}, {"arith.mulf", "mul"}, {"arith.divf", "div"},
      {"arith.maximumf", "maxf"}, {"arith.minimumf", "minf"}, {"arith.addi", "add"},
      {"arith.subi", "sub"}, {"arith.muli", "mul"}, {"linalg.add", "add"}, {"linalg.sub", "sub"},
      {"linalg.mul", "mul"}, {"linalg.div", "div"}, {"linalg.max", "maxf"}, {"linalg.min", "minf"}};
  static const std::map<std::string, std::string> un = {
      {"arith.negf", "negf"}, {"linalg.exp", "exp"}, {"linalg.abs", "abs"}, {"linalg.negf", "negf"},
      {"linalg.sqrt", "sqrt"}, {"linalg.rsqrt", "rsqrt"}, {"linalg.reciprocal", "reciprocal"}};
  if (bin.count(n)) return named(bin.at(n), 2);
  if (un.count(n)) return named(un.at(n), 1);
  if (n == "arith.extf" || n == "arith.truncf" || n == "arith.sitofp" || n == "arith.fptosi")
    return castExpr(a[0], at[0], U, false);
  unsupported(op, "elementwise op");
}

struct Combiner {
  std::string name;     // arith op
  std::string expr;     // with placeholders A (in) and B (acc)
  std::string identity; // neutral element in the value type
  bool isAddF = false;
};

Combiner combinerFor(const Op *op, const std::string &arith, Elem t) {
  Combiner c;
  c.name = arith;
  std::string T = ctype(t);
  auto lim = [&](bool mx) -> std::string {
    int b = elemBits(t);
    if (b >= 64) return mx ? "(int64_t)0x7fffffffffffffffll" : "(int64_t)(-0x7fffffffffffffffll - 1)";
    return mx ? "(" + T + ")" + std::to_string((1ll << (b - 1)) - 1) : "(" + T + ")(" + std::to_string(-(1ll << (b - 1))) + ")";
  };
  if (t == Elem::F32) {
    if (arith == "arith.addf") { c.expr = "(A + B)"; c.identity = "(-0.0f)"; c.isAddF = true; }
    else if (arith == "arith.mulf") { c.expr = "(A * B)"; c.identity = "1.0f"; }
    else if (arith == "arith.maximumf") { c.expr = "hf::maximumf(A, B)"; c.identity = "(-__builtin_inff())"; }
    else if (arith == "arith.minimumf") { c.expr = "hf::minimumf(A, B)"; c.identity = "__builtin_inff()"; }
    else if (arith == "arith.maxnumf") { c.expr = "hf::maxnumf(A, B)"; c.identity = "__builtin_nanf(\"\")"; }
    else if (arith == "arith.minnumf") { c.expr = "hf::minnumf(A, B)"; c.identity = "__builtin_nanf(\"\")"; }
    else unsupported(op, "reduction combiner '" + arith + "' on f32");
    return c;
  }
  if (isInt(t) && t != Elem::I1) {
    if (arith == "arith.addi") { c.expr = "(" + T + ")((uint64_t)(A) + (uint64_t)(B))"; c.identity = "(" + T + ")0"; }
    else if (arith == "arith.muli") { c.expr = "(" + T + ")((uint64_t)(A) * (uint64_t)(B))"; c.identity = "(" + T + ")1"; }
    else if (arith == "arith.maxsi") { c.expr = "((A) > (B) ? (A) : (B))"; c.identity = lim(false); }
    else if (arith == "arith.minsi") { c.expr = "((A) < (B) ? (A) : (B))"; c.identity = lim(true); }
    else if (arith == "arith.andi") { c.expr = "(" + T + ")((A) & (B))"; c.identity = "(" + T + ")(-1)"; }
    else if (arith == "arith.ori") { c.expr = "(" + T + ")((A) | (B))"; c.identity = "(" + T + ")0"; }
    else if (arith == "arith.xori") { c.expr = "(" + T + ")((A) ^ (B))"; c.identity = "(" + T + ")0"; }
    else unsupported(op, "reduction combiner '" + arith + "' on integers");
    return c;
  }
  unsupported(op, std::string("reductions over ") + elemName(t));
}

std::string subst(std::string e, const std::string &a, const std::string &b) {
  std::string out;
  for (char ch : e) {
    if (ch == 'A') out += a;
    else if (ch == 'B') out += b;
    else out += ch;
  }
  return out;
}

// --------------------------------------------------------------- analysis
struct Analysis {
  Func *f = nullptr;
  std::vector<int64_t> D;                     // iteration domain
  std::map<const Value *, std::vector<int>> map; // tensor value -> D dims it spans
  std::vector<BufferDesc> params, results;
  std::vector<int> resultTied;                 // tied param per result (-1: own buffer)
  std::set<int> paramsRead, paramsWritten;
  // dim 0 is the runtime row count (kRuntimeRows): kernels take it as their
  // last argument, hf_rows
  bool rowsDyn = false;
};

// The func argument a destination operand finally writes into (through
// linalg.fill / tensor.empty chains), or -1.
int tiedArgOf(const Value *v) {
  while (v) {
    if (v->argIdx >= 0) return v->argIdx;
    const Op *d = v->def;
    if (!d || d->outs.empty()) return -1;
    v = d->outs[std::min<size_t>(v->resultIdx, d->outs.size() - 1)];
  }
  return -1;
}

const Op *findOp(const Func &f, const std::function<bool(const Op *)> &p) {
  for (const Op *op : f.ops) if (p(op)) return op;
  return nullptr;
}

void describeBuffers(Analysis &A) {
  Func &f = *A.f;
  for (Value *a : f.args) {
    BufferDesc b;
    b.elem = a->type.elem;
    b.shape = a->type.shape;
    b.role = a->type.tensor ? "in" : "scalar";
    A.params.push_back(b);
  }
  for (size_t i = 0; i < f.returns.size(); ++i) {
    Value *r = f.returns[i];
    BufferDesc b;
    b.elem = r->type.elem;
    b.shape = r->type.shape;
    b.role = "out";
    int t = r->def ? tiedArgOf(r->def->outs.empty() ? nullptr : r->def->outs[std::min<size_t>(r->resultIdx, r->def->outs.size() - 1)])
                   : r->argIdx;
    if (t >= 0 && f.args[t]->type.elem != r->type.elem) t = -1;
    b.tiedParam = t;
    if (t >= 0) {
      A.paramsWritten.insert(t);
      A.params[t].role = "out";
    }
    A.results.push_back(b);
    A.resultTied.push_back(t);
  }
  // params that are read: used as `ins`/operands anywhere
  for (const Op *op : f.ops) {
    for (auto *v : op->ins) if (v->argIdx >= 0) A.paramsRead.insert(v->argIdx);
    for (auto *v : op->operands) if (v->argIdx >= 0) A.paramsRead.insert(v->argIdx);
  }
  for (int p : A.paramsRead) if (A.params[p].role == "out") A.params[p].role = "inout";
}

bool isAlias(const Op *op) {
  return op->name == "linalg.broadcast" || op->name == "tensor.empty" || op->name == "linalg.fill" ||
         op->name == "arith.constant" || op->name == "tensor.dim" || op->name.rfind("arith.index", 0) == 0;
}

// `permutation = [...]` of a linalg.transpose (out dim i is in dim perm[i]).
std::vector<int64_t> permutationOf(const Op *op) {
  std::vector<int64_t> perm;
  std::string p = op->attr("permutation");
  for (size_t i = 0; i < p.size();) {
    size_t j = p.find(',', i);
    if (j == std::string::npos) j = p.size();
    perm.push_back(std::stoll(p.substr(i, j - i)));
    i = j + 1;
  }
  if (op->ins.size() != 1 || op->outs.size() != 1) unsupported(op, "transpose operand form");
  const size_t n = op->ins[0]->type.shape.size();
  std::vector<bool> seen(n, false);
  if (perm.size() != n) unsupported(op, "permutation length");
  for (auto d : perm) {
    if (d < 0 || d >= (int64_t)n || seen[d]) unsupported(op, "not a permutation");
    seen[d] = true;
  }
  for (size_t i = 0; i < n; ++i)
    if (op->outs[0]->type.shape[i] != op->ins[0]->type.shape[perm[i]]) unsupported(op, "transpose shapes");
  return perm;
}

// `m` without the entries at `positions` (tensor dims of a reduce or
// broadcast op's `dimensions`).
std::vector<int> dropPositions(const std::vector<int> &m, const std::vector<int64_t> &positions) {
  std::vector<int> o;
  for (size_t i = 0; i < m.size(); ++i)
    if (std::find(positions.begin(), positions.end(), (int64_t)i) == positions.end()) o.push_back(m[i]);
  return o;
}

// Propagates D-dim maps through broadcasts, reductions and elementwise ops.
void inferMaps(Analysis &A, const std::set<const Value *> &exclude) {
  Func &f = *A.f;
  int r = (int)A.D.size();
  std::vector<int> all;
  for (int i = 0; i < r; ++i) all.push_back(i);
  auto setMap = [&](const Value *v, const std::vector<int> &m, const Op *op) -> bool {
    if (!v->type.tensor || exclude.count(v)) return false;
    if ((int)m.size() != (int)v->type.shape.size()) unsupported(op, "shape does not match its broadcast/reduce dimensions");
    for (size_t i = 0; i < m.size(); ++i)
      if (v->type.shape[i] != A.D[m[i]]) unsupported(op, "tensor shape inconsistent with the group's iteration domain");
    auto it = A.map.find(v);
    if (it != A.map.end()) {
      if (it->second != m) unsupported(op, "value used with two different broadcast layouts");
      return false;
    }
    A.map[v] = m;
    return true;
  };
  // seeds: full-rank tensors (in a group with transposes, only its results:
  // a tensor of the domain's shape may reach them through a permutation)
  bool hasTranspose = false;
  for (Op *op : f.ops) hasTranspose |= op->name == "linalg.transpose";
  if (hasTranspose) {
    for (Value *v : f.returns)
      if (v->type.tensor && v->type.shape == A.D && !exclude.count(v)) A.map[v] = all;
    // a reducing group whose results are all reduced: the first reduction's
    // input spans the domain (largestShape chose its shape)
    if (A.map.empty())
      for (Op *op : f.ops)
        if ((op->name == "linalg.reduce" || op->name == "hfusion.reduce_with_index") && !op->ins.empty()) {
          if (op->ins[0]->type.shape == A.D && !exclude.count(op->ins[0])) A.map[op->ins[0]] = all;
          break;
        }
  } else {
    for (Value *a : f.args)
      if (a->type.tensor && a->type.shape == A.D && !exclude.count(a)) A.map[a] = all;
    for (Op *op : f.ops)
      for (Value *v : op->results)
        if (v->type.tensor && v->type.shape == A.D && !exclude.count(v)) A.map[v] = all;
  }
  bool changed = true;
  while (changed) {
    changed = false;
    for (Op *op : f.ops) {
      const std::string &n = op->name;
      auto minus = [&](const std::vector<int64_t> &dims) {
        std::vector<int> m;
        for (int i = 0; i < r; ++i)
          if (std::find(dims.begin(), dims.end(), i) == dims.end()) m.push_back(i);
        return m;
      };
      // the operand's map is the result's without the broadcast dims (with
      // identity maps: D minus `dimensions`)
      if (n == "linalg.broadcast") {
        if (op->ins.empty()) continue;
        const Value *o = op->results.empty() ? op->outs[0] : op->results[0];
        if (A.map.count(o)) changed |= setMap(op->ins[0], dropPositions(A.map[o], op->dims), op);
        else if (!hasTranspose) changed |= setMap(op->ins[0], minus(op->dims), op);
        continue;
      }
      if (n == "linalg.transpose") {
        // out dim i is in dim perm[i]: in[perm[i]] spans what out[i] spans
        std::vector<int64_t> perm = permutationOf(op);
        const Value *o = op->results.empty() ? op->outs[0] : op->results[0];
        const Value *in = op->ins[0];
        if (A.map.count(o)) {
          std::vector<int> mi(perm.size());
          for (size_t i = 0; i < perm.size(); ++i) mi[perm[i]] = A.map[o][i];
          changed |= setMap(in, mi, op);
          for (auto *v : op->results) changed |= setMap(v, A.map[o], op);
          changed |= setMap(op->outs[0], A.map[o], op);
        } else if (A.map.count(in)) {
          std::vector<int> mo(perm.size());
          for (size_t i = 0; i < perm.size(); ++i) mo[i] = A.map[in][perm[i]];
          changed |= setMap(o, mo, op);
          for (auto *v : op->results) changed |= setMap(v, mo, op);
        }
        continue;
      }
      // the result's map is the input's without the reduced dims
      if (n == "linalg.reduce" || n == "hfusion.reduce_with_index") {
        const Value *x = op->ins.empty() ? nullptr : op->ins[0];
        if (x && A.map.count(x)) {
          const std::vector<int> mo = dropPositions(A.map[x], op->dims);
          for (auto *o : op->outs) changed |= setMap(o, mo, op);
          for (auto *o : op->results) changed |= setMap(o, mo, op);
          for (auto *i : op->ins) changed |= setMap(i, A.map[x], op);
        } else if (!hasTranspose) {
          for (auto *o : op->outs) changed |= setMap(o, minus(op->dims), op);
          for (auto *o : op->results) changed |= setMap(o, minus(op->dims), op);
        }
        continue;
      }
      if (n == "linalg.generic" && genericIsElementwise(op)) {
        std::vector<std::vector<int>> maps;
        int nd = 0;
        genericMaps(op, maps, nd);
        const Value *o = op->results.empty() ? op->outs[0] : op->results[0];
        const std::vector<int> *known = A.map.count(o) ? &A.map[o] : (A.map.count(op->outs[0]) ? &A.map[op->outs[0]] : nullptr);
        if (known) {
          std::vector<int> mo = *known;
          changed |= setMap(op->outs[0], mo, op);
          for (auto *v : op->results) changed |= setMap(v, mo, op);
          for (size_t i = 0; i < op->ins.size(); ++i) {
            if (!op->ins[i]->type.tensor) continue;
            std::vector<int> mi;
            for (int d : maps[i]) mi.push_back(mo.at(d));
            changed |= setMap(op->ins[i], mi, op);
          }
        }
        continue;
      }
      if (n == "linalg.fill") {
        if (A.map.count(op->results[0])) changed |= setMap(op->outs[0], A.map[op->results[0]], op);
        if (A.map.count(op->outs[0])) changed |= setMap(op->results[0], A.map[op->outs[0]], op);
        continue;
      }
      if (isElementwiseOp(op)) {
        std::vector<Value *> vs;
        for (auto *v : op->ins) if (v->type.tensor) vs.push_back(v);
        for (auto *v : op->operands) if (v->type.tensor) vs.push_back(v);
        for (auto *v : op->outs) vs.push_back(v);
        for (auto *v : op->results) vs.push_back(v);
        const std::vector<int> *known = nullptr;
        for (auto *v : vs) if (A.map.count(v)) { known = &A.map[v]; break; }
        if (known) {
          std::vector<int> m = *known;
          for (auto *v : vs) changed |= setMap(v, m, op);
        }
      }
    }
  }
  for (Value *a : f.args)
    if (a->type.tensor && !exclude.count(a) && !A.map.count(a)) {
      bool used = !a->users.empty();
      if (used) throw CompileError("cannot place argument " + a->name + " in the group's iteration domain");
    }
}

std::string resultKind(const Func &f, bool *hasMatmul, bool *hasRWI, bool *hasReduce) {
  *hasMatmul = *hasRWI = *hasReduce = false;
  for (const Op *op : f.ops) {
    if (op->name == "linalg.matmul" || op->name == "linalg.matmul_transpose_b" || op->name == "hivm.hir.matmul" ||
        op->name == "hfusion.matmul_mx")
      *hasMatmul = true;
    if (op->name == "hfusion.reduce_with_index") *hasRWI = true;
    if (op->name == "linalg.reduce") *hasReduce = true;
  }
  if (*hasMatmul) return "SINGLE_CUBE";
  if (*hasRWI) return "REDUCE_WITH_INDEX";
  if (*hasReduce) return "LAST_AXIS_PBR";
  return "PURE_ELEMWISE";
}

std::vector<int64_t> largestShape(const Func &f, const std::set<const Value *> &exclude) {
  std::vector<int64_t> best;
  auto consider = [&](const Value *v) {
    if (!v->type.tensor || exclude.count(v)) return;
    const auto &s = v->type.shape;
    if (s.size() > best.size() || (s.size() == best.size() && v->type.numel() > 0 && best.empty())) best = s;
  };
  for (auto *a : f.args) consider(a);
  for (auto *op : f.ops) for (auto *v : op->results) consider(v);
  bool hasTranspose = false;
  for (auto *op : f.ops) hasTranspose |= op->name == "linalg.transpose";
  if (hasTranspose) {
    // the domain is the results' shape (results are stored contiguously), or
    // in a group whose results are reduced, the first reduction's input
    for (auto *r : f.returns)
      if (r->type.tensor && r->type.shape.size() == best.size()) return r->type.shape;
    for (auto *op : f.ops)
      if ((op->name == "linalg.reduce" || op->name == "hfusion.reduce_with_index") && !op->ins.empty() &&
          op->ins[0]->type.shape.size() == best.size())
        return op->ins[0]->type.shape;
    return best;
  }
  for (auto *op : f.ops) for (auto *v : op->results)
    if (v->type.tensor && !exclude.count(v) && v->type.shape.size() == best.size() && v->type.shape != best)
      throw CompileError("group mixes full-rank tensors of different shapes (" + v->type.str() + ")");
  return best;
}

// A tensor value a kernel would read that no op of the group defines and that
// is no group argument: an uninitialised tensor.empty (its contents are
// undefined in the reference too), or an internal error.
[[noreturn]] void undefinedValue(const Value *v) {
  if (v->def && v->def->name == "tensor.empty")
    throw CompileError("unsupported: the group reads the uninitialised contents of tensor.empty " + v->name);
  throw CompileError("internal: value " + v->name + " used before definition");
}

std::string kernelParamList(const Analysis &A, std::vector<std::string> &kargs, bool withWs) {
  std::ostringstream s;
  bool first = true;
  for (size_t i = 0; i < A.params.size(); ++i) {
    if (!first) s << ", ";
    first = false;
    if (A.params[i].role == "scalar") s << "uint64_t s" << i;
    else s << "void* __restrict__ p" << i;
    kargs.push_back("param:" + std::to_string(i));
  }
  for (size_t i = 0; i < A.results.size(); ++i) {
    if (A.resultTied[i] >= 0) continue;
    if (!first) s << ", ";
    first = false;
    s << "void* __restrict__ r" << i;
    kargs.push_back("result:" + std::to_string(i));
  }
  if (withWs) {
    if (!first) s << ", ";
    first = false;
    s << "void* __restrict__ ws";
    kargs.push_back("ws");
  }
  if (A.rowsDyn) {
    if (!first) s << ", ";
    s << "int64_t hf_rows";
    kargs.push_back("rows");
  }
  return s.str();
}

// Pointer expression of the buffer holding func result i.
std::string resultPtr(const Analysis &A, size_t i) {
  return A.resultTied[i] >= 0 ? "p" + std::to_string(A.resultTied[i]) : "r" + std::to_string(i);
}

std::string scalarArgExpr(const Analysis &A, int i) {
  Elem e = A.params[i].elem;
  std::string s = "s" + std::to_string(i);
  if (e == Elem::F32) return "__uint_as_float((uint32_t)" + s + ")";
  if (e == Elem::F64) return "__longlong_as_double((long long)" + s + ")";
  if (e == Elem::BF16 || e == Elem::F16) return "((uint16_t)" + s + ")";
  return "((" + ctype(e) + ")" + s + ")";
}

double bytesOf(const BufferDesc &b) {
  double n = elemBytes(b.elem);
  for (auto d : b.shape) n *= (double)d;
  return n;
}

double algoBytes(const Analysis &A) {
  double t = 0;
  for (int p : A.paramsRead) if (A.params[p].role != "scalar") t += bytesOf(A.params[p]);
  for (auto &r : A.results) t += bytesOf(r);
  return t;
}

// ======================================================================
// Row-program emitter (LAST_AXIS_PBR).  Domain [R, C] (1-D groups use R = 1).
// A row group of TR threads owns RPW consecutive rows; a block holds RB row
// groups.  Values live in one of four spaces:
//   Full  — per element; either an array of RPW*EPL lane elements or a lazy
//           expression re-evaluated at each use (cheap chains are recomputed
//           rather than kept in VGPRs);
//   Row   — per row: an array of RPW scalars;
//   Col   — per column: an array of EPL (input) or a lazy expression;
//   Scalar— a constant or kernel argument.
// ======================================================================
enum class Sp { Full, Row, Col, Scalar };

struct RowEmitter {
  Analysis &A;
  const LowerOptions &opt;
  std::ostringstream pre, body;
  struct V {
    Sp sp;
    std::string name;
    bool lazy = false;     // Full/Col: `name(e, ex)` instead of `name[e]`
    bool fast = false;     // evaluation may raise hf_bad (fast-path ops inside)
    bool integral = false; // holds integral values (or inf/NaN) only
    bool guarded = false;  // non-NaN in fast mode (a NaN raises the Guard)
    bool ranged = false;   // known to lie in [lo, hi] (or be NaN)
    double lo = 0, hi = 0;
    // set when the value is min/max(x, constant) of a guarded x
    std::string clampX;
    bool clampIsMin = false;
    double clampC = 0;
    // set when the value is an invariant-divisor division a / b (lazy)
    std::string divA, divB, divR;
    // set along rint(a / b) -> clamp -> cast: the dividend and the reciprocal
    // (`qRcp` indexed by row when qRcpRow), for the packed int8 fast path
    const Value *qSrc = nullptr;
    std::string qRcp, qDiv; // reciprocal array (or scalar) and the divisor's per-row access
    bool qRcpRow = false;
    bool quant8 = false; // an int8 cast of clamp(rint(a / b)), lo/hi the clamp
  };
  std::map<const Value *, V> val;
  std::vector<std::string> arrays; // loaded element/column input arrays
  std::vector<std::string> prefetchStmts; // chunk loads issued inside the serial chain
  static constexpr int LOOKAHEAD = 2;   // LDS chunks of loads in flight per CU
  std::map<std::string, std::set<std::string>> lazyDeps; // lazy value -> input arrays it reads
  std::set<const Value *> orderedReduce;
  int tmp = 0;
  int nred = 0; // LDS slots (per row of a row group) for tree reductions
  bool needOrdered = false;
  bool progressive = false; // Full inputs streamed in by the first (serial) reduction
  // after the serial chain, inputs are loaded where first used: the chain's
  // LDS reads need the registers an early load would hold through it
  bool afterOrdered = false;
  std::map<std::string, size_t> declaredAt; // array -> body offset of its declaration (pre: 0)
  int64_t R = 1, C = 1;
  int TR = 64, RB = 1, RPW = 1, VEC = 4, EPL = 4, CH = 0;
  bool masked = false;

  RowEmitter(Analysis &a, const LowerOptions &o) : A(a), opt(o) {}

  Sp spaceOfMap(const std::vector<int> &m) const {
    if (A.D.size() == 1) return m.empty() ? Sp::Scalar : Sp::Full;
    if (m.size() == 2) return Sp::Full;
    if (m.size() == 1) return m[0] == 0 ? Sp::Row : Sp::Col;
    return Sp::Scalar;
  }
  std::string fresh() { return "v" + std::to_string(tmp++); }

  // value of v at full element index e (0 <= e < RPW*EPL); `ex` names the
  // exactness switch (hf::kFast{} / hf::kExact{} or a lambda's `ex`)
  std::string at(const Value *v, const std::string &e, const std::string &ex = "ex") const {
    const V &x = val.at(v);
    switch (x.sp) {
    case Sp::Full: return x.lazy ? x.name + "(" + e + ", " + ex + ")" : x.name + "[" + e + "]";
    case Sp::Col: return x.lazy ? x.name + "(" + e + ", " + ex + ")" : x.name + "[(" + e + ") % EPL]";
    case Sp::Row: return x.name + "[(" + e + ") / EPL]";
    default: return x.name;
    }
  }
  bool isFast(const Value *v) const { return val.at(v).lazy && val.at(v).fast; }
  // an element expression written for a lambda (`ex`) evaluated in a loop
  static std::string replaceEx(const std::string &expr, const std::string &with) {
    std::string out;
    for (size_t i = 0; i < expr.size();) {
      bool word = expr.compare(i, 2, "ex") == 0 && (i == 0 || !(std::isalnum((unsigned char)expr[i - 1]) || expr[i - 1] == '_')) &&
                  (i + 2 >= expr.size() || !(std::isalnum((unsigned char)expr[i + 2]) || expr[i + 2] == '_'));
      if (word) { out += with; i += 2; }
      else out += expr[i++];
    }
    return out;
  }
  // value of a Row/Scalar value for row rr of the group
  std::string atRow(const Value *v, const std::string &rr) const {
    const V &x = val.at(v);
    if (x.sp == Sp::Row) return x.name + "[" + rr + "]";
    if (x.sp == Sp::Scalar) return x.name;
    throw CompileError("internal: per-row access to an element value");
  }

  std::string colExpr(const std::string &e) const {
    return "((int64_t)(((" + e + ") % EPL) / VEC) * (TR * VEC) + lt * VEC + (" + e + ") % VEC)";
  }

  int uses(const Value *v) const {
    int n = 0;
    for (const Op *u : v->users) {
      for (auto *i : u->ins) n += i == v;
      for (auto *i : u->operands) n += i == v;
    }
    for (auto *r : A.f->returns) n += r == v;
    return n;
  }

  static bool expensive(const Op *op) {
    std::string fn = op->attr("fun");
    static const std::set<std::string> costly = {"exp", "exp2", "log", "log2", "log10", "log1p", "expm1", "tanh",
                                                 "sin", "cos", "erf", "powf", "sqrt", "rsqrt", "div", "rec",
                                                 "reciprocal", "mod", "modui", "tan", "acos", "acosh", "asin",
                                                 "asinh", "atan", "atanh", "sinh", "cosh", "lgamma", "atan2",
                                                 "divfhp", "powi"};
    if (op->name == "hfusion.hypot" || op->name == "hfusion.erfinv" ||
        op->name == "hfusion.cyl_bessel_i0")
      return true;
    return costly.count(fn) || op->name == "arith.divf" || op->name == "linalg.div";
  }

  // Float sums are folded in the reference's serial order (the CPU loop's
  // left-to-right fold from the init) wherever the row fits the serial
  // schedule (at most 4096 elements: 4 resident rows per wave), and always
  // when the result reaches an integer-typed group output (bit-exact integer
  // outputs depend on it).  Wider rows use tree order.
  void markOrdered() {
    Func &f = *A.f;
    std::set<const Value *> intOut;
    for (auto *r : f.returns) if (isInt(r->type.elem)) intOut.insert(r);
    const int64_t width = A.D.empty() ? 1 : A.D.back();
    const bool everywhere = opt.orderedFloatSums == 1 || (opt.orderedFloatSums < 0 && width <= 4096);
    for (Op *op : f.ops) {
      if (op->name != "linalg.reduce" || op->combiner != "arith.addf") continue;
      if (op->results.empty() || op->results[0]->type.elem != Elem::F32) continue;
      bool reaches = everywhere;
      std::vector<const Value *> stack(op->results.begin(), op->results.end());
      std::set<const Value *> seen;
      while (!stack.empty() && !reaches) {
        const Value *v = stack.back();
        stack.pop_back();
        if (!seen.insert(v).second) continue;
        if (intOut.count(v)) reaches = true;
        for (const Op *u : v->users)
          for (auto *r : u->results) stack.push_back(r);
      }
      if (reaches) orderedReduce.insert(op->results[0]);
    }
    needOrdered = !orderedReduce.empty();
    // progressive loading is valid only when the serial chain is the first
    // consumer that needs whole rows (no earlier reduction)
    for (Op *op : f.ops)
      if (op->name == "linalg.reduce") {
        progressive = orderedReduce.count(op->results[0]) != 0;
        break;
      }
  }

  void chooseSchedule() {
    if (A.D.size() == 2) { R = A.D[0]; C = A.D[1]; }
    else if (A.D.size() == 1) { R = 1; C = A.D[0]; }
    else throw CompileError("row programs support rank-1 and rank-2 groups");
    // vector width from the tensors that travel through HBM
    int maxBytes = 1;
    auto consider = [&](const Value *v) {
      if (!v->type.tensor || !A.map.count(v)) return;
      Sp s = spaceOfMap(A.map.at(v));
      if (s == Sp::Full || s == Sp::Col) maxBytes = std::max(maxBytes, elemBytes(v->type.elem));
    };
    for (auto *a : A.f->args) consider(a);
    for (auto *r : A.f->returns) consider(r);
    VEC = std::max(1, 16 / maxBytes);
    if (VEC > 8) VEC = 8;
    while (VEC > 1 && C % VEC) VEC /= 2;
    if (needOrdered) {
      // one wave per row group, 4 rows each, 8 waves: 32 rows per block with
      // a single serial chain lane per row in wave 0 (2 waves per SIMD leave
      // 256 VGPRs per lane for the resident rows)
      TR = 64;
      RB = 8;
      RPW = 4;
    } else {
      int64_t perLaneTarget = VEC * 4;
      int tr = 64;
      while (tr < 1024 && (int64_t)tr * perLaneTarget < C) tr *= 2;
      TR = tr;
      RB = std::max(1, 256 / TR);
      RPW = 1;
    }
    int64_t span = (int64_t)TR * VEC;
    int64_t nch = (C + span - 1) / span;
    EPL = (int)(nch * VEC);
    masked = (C % span) != 0;
    if (EPL * RPW > 256)
      throw CompileError("row of " + std::to_string(C) + " elements does not fit one row group");
    if (needOrdered) {
      int jpc = std::max<int64_t>(1, 512 / span);
      if (jpc > nch) jpc = (int)nch;
      CH = (int)(jpc * span);
      // two LDS buffers of RB*RPW rows must fit next to the other stages
      while ((int64_t)2 * RB * RPW * (CH + 4) * 4 > 140 * 1024 && jpc > 1) { --jpc; CH = (int)(jpc * span); }
      if ((int64_t)2 * RB * RPW * (CH + 4) * 4 > 140 * 1024)
        throw CompileError("row too wide for the serial-order staging buffer");
    }
  }

  std::string rowExpr(const std::string &rr) const { return "row[" + rr + "]"; }

  void loadInput(const Value *a) {
    int i = a->argIdx;
    Sp s = spaceOfMap(A.map.at(a));
    std::string T = ctype(a->type.elem), M = mtype(a->type.elem);
    std::string nm = "in" + std::to_string(i);
    val[a] = {s, nm, false};
    std::string P = "(const " + M + "*)p" + std::to_string(i);
    std::ostringstream &pre = afterOrdered ? this->body : this->pre;
    if ((s == Sp::Full || s == Sp::Col) && a->type.elem != Elem::I1) {
      arrays.push_back(nm);
      declaredAt[nm] = afterOrdered ? (size_t)this->body.tellp() : 0;
    }
    if (s == Sp::Full && progressive && a->type.elem != Elem::I1) {
      // loaded progressively by the serial chain (LOOKAHEAD chunks ahead)
      const int jpc = CH / (TR * VEC);
      pre << "  " << M << " " << nm << "[RPW * EPL];\n"
          << "  hf::rows_load_range<" << M << ", VEC, EPL / VEC, TR, RPW, MASKED>(" << P << ", row, C, lt, " << nm << ", 0, "
          << LOOKAHEAD * jpc << ");\n";
      prefetchStmts.push_back("hf::rows_load_range<" + M + ", VEC, EPL / VEC, TR, RPW, MASKED>(" + P + ", row, C, lt, " + nm +
                              ", kk * " + std::to_string(jpc) + ", kk * " + std::to_string(jpc) + " + " + std::to_string(jpc) + ");");
    } else if (s == Sp::Full) {
      pre << "  " << M << " " << nm << (a->type.elem == Elem::I1 ? "_raw" : "") << "[RPW * EPL];\n"
          << "  hf::rows_load<" << M << ", VEC, EPL / VEC, TR, RPW, MASKED>(" << P << ", row, C, lt, "
          << nm << (a->type.elem == Elem::I1 ? "_raw" : "") << ");\n";
      if (a->type.elem == Elem::I1)
        pre << "  bool " << nm << "[RPW * EPL];\n  for (int e = 0; e < RPW * EPL; ++e) " << nm << "[e] = " << nm << "_raw[e] != 0;\n";
    } else if (s == Sp::Col) {
      pre << "  " << M << " " << nm << (a->type.elem == Elem::I1 ? "_raw" : "") << "[EPL];\n"
          << "  hf::row_load<" << M << ", VEC, EPL / VEC, TR, MASKED>(" << P << ", lt, C, " << nm
          << (a->type.elem == Elem::I1 ? "_raw" : "") << ");\n";
      if (a->type.elem == Elem::I1)
        pre << "  bool " << nm << "[EPL];\n  for (int e = 0; e < EPL; ++e) " << nm << "[e] = " << nm << "_raw[e] != 0;\n";
    } else if (s == Sp::Row) {
      pre << "  " << T << " " << nm << "[RPW];\n"
          << "#pragma unroll\n  for (int rr = 0; rr < RPW; ++rr) " << nm << "[rr] = (" << P << ")[row[rr]];\n";
    } else {
      pre << "  const " << T << " " << nm << " = (" << P << ")[0];\n";
    }
  }

  void bindScalar(const Value *v) {
    if (v->isConst) { val[v] = {Sp::Scalar, constExpr(v, v->type.elem)}; return; }
    if (v->argIdx >= 0) { val[v] = {Sp::Scalar, scalarArgExpr(A, v->argIdx)}; return; }
    throw CompileError("non-constant scalar " + v->name + " in a tensor group");
  }

  void ensure(const Value *v) {
    if (val.count(v)) return;
    if (!v->type.tensor) { bindScalar(v); return; }
    if (v->argIdx >= 0) { loadInput(v); return; }
    if (v->isConst) { val[v] = {Sp::Scalar, constExpr(v, v->type.elem)}; return; }
    undefinedValue(v);
  }

  // division of an element value by a per-row (or constant) f32 divisor:
  // reciprocal once per row (consumed by hf::rint_div for a rounding consumer)
  bool isInvariantDiv(const Op *op, const std::vector<const Value *> &opsv, Elem U) const {
    bool div = (op->name == "linalg.elemwise_binary" && op->attr("fun") == "div") || op->name == "arith.divf" ||
               op->name == "linalg.div";
    if (!div || U != Elem::F32 || opsv.size() != 2) return false;
    if (opsv[0]->type.elem != Elem::F32 || opsv[1]->type.elem != Elem::F32) return false;
    Sp s1 = val.at(opsv[1]).sp, s0 = val.at(opsv[0]).sp;
    return (s1 == Sp::Row || s1 == Sp::Scalar) && (s0 == Sp::Full || s0 == Sp::Col);
  }

  void emitElementwise(const Op *op) {
    std::vector<const Value *> opsv;
    for (auto *v : op->ins) opsv.push_back(v);
    for (auto *v : op->operands) opsv.push_back(v);
    bool anyFull = false, anyRow = false, anyCol = false;
    for (auto *v : opsv) {
      ensure(v);
      Sp s = val[v].sp;
      anyFull |= s == Sp::Full;
      anyRow |= s == Sp::Row;
      anyCol |= s == Sp::Col;
    }
    Sp out = anyFull || (anyRow && anyCol) ? Sp::Full : anyCol ? Sp::Col : anyRow ? Sp::Row : Sp::Scalar;
    const Value *res = op->results[0];
    if (A.map.count(res) && spaceOfMap(A.map.at(res)) == Sp::Full) out = Sp::Full;
    Elem U = res->type.elem;
    std::vector<Elem> at_;
    for (auto *v : opsv) at_.push_back(v->type.elem);
    std::string nm = fresh();
    std::string T = ctype(U);
    if (out == Sp::Full || out == Sp::Col) {
      std::string expr;
      bool fast = false, integral = false;
      V nv{out, nm, true};
      for (auto *v : opsv) fast |= val[v].fast;
      const std::string fn = op->attr("fun");
      if (isInvariantDiv(op, opsv, U)) {
        const Value *b = opsv[1];
        std::string rn = nm + "_rcp";
        std::string bAt, rAt;
        if (val[b].sp == Sp::Row) {
          body << "  float " << rn << "[RPW];\n#pragma unroll\n  for (int rr = 0; rr < RPW; ++rr) { " << rn << "[rr] = 1.0f / "
               << atRow(b, "rr") << "; if constexpr (!EXM::value) hf_g.divisor(" << rn << "[rr]); }\n";
          bAt = at(b, "e");
          rAt = rn + "[(e) / EPL]";
        } else {
          body << "  const float " << rn << " = 1.0f / " << val[b].name << ";\n  if constexpr (!EXM::value) hf_g.divisor(" << rn << ");\n";
          bAt = val[b].name;
          rAt = rn;
        }
        // the quotient is RN(a/b) from the row reciprocal (hf::div_rn, exact
        // or re-executed); a consuming nearbyint takes hf::rint_div instead
        expr = "hf::div_rn(" + at(opsv[0], "e") + ", " + bAt + ", " + rAt + ", hf_g, ex)";
        fast = true;
        nv.divA = at(opsv[0], "e");
        nv.divB = bAt;
        nv.divR = rAt;
        nv.qSrc = opsv[0];
        nv.qRcp = rn;
        nv.qRcpRow = val[b].sp == Sp::Row;
        nv.qDiv = val[b].sp == Sp::Row ? atRow(b, "rr") : val[b].name;
      } else if ((op->name == "hfusion.elemwise_unary" && fn == "nearbyint") && U == Elem::F32 && opsv[0]->type.elem == Elem::F32 &&
                 val[opsv[0]].lazy && !val[opsv[0]].divA.empty() && uses(opsv[0]) == 1) {
        // rint of a division by a per-row divisor (dynamic quantisation)
        const V &d = val[opsv[0]];
        expr = "hf::rint_div(" + d.divA + ", " + d.divB + ", " + d.divR + ", hf_g, ex)";
        fast = true;
        integral = true;
        nv.guarded = true;
        nv.qSrc = d.qSrc;
        nv.qRcp = d.qRcp;
        nv.qRcpRow = d.qRcpRow;
        nv.qDiv = d.qDiv;
      } else if ((fn == "maxf" || fn == "minf") && U == Elem::F32 && opsv.size() == 2 && opsv[1]->isConst &&
                 val[opsv[0]].lazy && val[opsv[0]].guarded) {
        // clamp of a guarded (non-NaN in fast mode) value: min/max pairs fold
        // into one v_med3_f32
        const V &x = val[opsv[0]];
        double c = opsv[1]->fconst;
        bool isMin = fn == "minf";
        if (!x.clampX.empty() && x.clampIsMin != isMin && uses(opsv[0]) == 1 &&
            (isMin ? x.clampC <= c : c <= x.clampC)) {
          double lo = isMin ? x.clampC : c, hi = isMin ? c : x.clampC;
          expr = "(ex.value ? " + elementExpr(op, {at(opsv[0], "e"), val[opsv[1]].name}, at_, U) + " : __builtin_amdgcn_fmed3f(" +
                 x.clampX + ", " + floatLit((float)lo) + ", " + floatLit((float)hi) + "))";
          nv.ranged = true;
          nv.lo = lo;
          nv.hi = hi;
        } else {
          expr = elementExpr(op, {at(opsv[0], "e"), val[opsv[1]].name}, at_, U);
          nv.clampX = at(opsv[0], "e");
          nv.clampIsMin = isMin;
          nv.clampC = c;
        }
        fast = true;
        integral = x.integral && std::floor(c) == c;
        nv.guarded = true;
        if (integral && uses(opsv[0]) == 1) {
          nv.qSrc = x.qSrc;
          nv.qRcp = x.qRcp;
          nv.qRcpRow = x.qRcpRow;
          nv.qDiv = x.qDiv;
        }
      } else {
        std::vector<std::string> args;
        for (auto *v : opsv) args.push_back(at(v, "e"));
        if (op->name == "hfusion.cast" && U != Elem::I1 && isInt(U) && opsv[0]->type.elem == Elem::F32 && val[opsv[0]].integral) {
          bool sat = op->attr("enable_saturate") == "true";
          const V &x = val[opsv[0]];
          double tlo = -std::ldexp(1.0, elemBits(U) - 1), thi = std::ldexp(1.0, elemBits(U) - 1) - 1;
          if (x.ranged && x.lo >= tlo && x.hi <= thi && elemBits(U) <= 32)
            // integral and inside the target range: one convert (NaN -> 0)
            expr = "(" + ctype(U) + ")(int32_t)(" + args[0] + ")";
          if (U == Elem::I8 && x.ranged && x.qSrc && x.lo >= -128 && x.hi <= 127 && x.lo <= x.hi &&
              std::floor(x.lo) == x.lo && std::floor(x.hi) == x.hi && uses(opsv[0]) == 1) {
            nv.quant8 = true;
            nv.qSrc = x.qSrc;
            nv.qRcp = x.qRcp;
            nv.qRcpRow = x.qRcpRow;
            nv.qDiv = x.qDiv;
            nv.lo = x.lo;
            nv.hi = x.hi;
          }
          else
            expr = "hf::integral_to_int<" + ctype(U) + ", " + (sat ? "true" : "false") + ">(" + args[0] + ")";
        } else {
          expr = elementExpr(op, args, at_, U);
        }
        // integral-valued results: rounding functions, and min/max/select of
        // integral values and integral constants
        auto integ = [&](const Value *v) {
          if (v->isConst) return std::floor(v->fconst) == v->fconst;
          return val[v].integral;
        };
        if (fn == "nearbyint" || fn == "floor" || fn == "ceil" || fn == "round" || fn == "trunc") integral = true;
        if ((fn == "maxf" || fn == "minf" || fn == "maxnumf" || fn == "minnumf") && integ(opsv[0]) && integ(opsv[1])) integral = true;
        if (op->name == "hfusion.select" && integ(opsv[1]) && integ(opsv[2])) integral = true;
      }
      nv.fast = fast;
      nv.integral = integral;
      bool materialise = expensive(op) && uses(res) > 1;
      if (materialise) {
        std::string n = out == Sp::Full ? "RPW * EPL" : "EPL";
        body << "  " << T << " " << nm << "[" << n << "];\n#pragma unroll\n  for (int e = 0; e < " << n << "; ++e) " << nm
             << "[e] = " << expr << ";\n";
        val[res] = {out, nm, false};
        val[res].integral = integral;
      } else {
        body << "  auto " << nm << " = [&](int e, auto ex) -> " << T << " { return " << expr << "; };\n";
        val[res] = nv;
        std::set<std::string> deps;
        for (auto *v : opsv) {
          const V &x = val[v];
          if (x.lazy) deps.insert(lazyDeps[x.name].begin(), lazyDeps[x.name].end());
          else if (std::find(arrays.begin(), arrays.end(), x.name) != arrays.end()) deps.insert(x.name);
        }
        lazyDeps[nm] = deps;
      }
      return;
    }
    if (out == Sp::Row) {
      std::vector<std::string> args;
      for (auto *v : opsv) args.push_back(atRow(v, "rr"));
      body << "  " << T << " " << nm << "[RPW];\n#pragma unroll\n  for (int rr = 0; rr < RPW; ++rr) " << nm
           << "[rr] = " << elementExpr(op, args, at_, U) << ";\n";
      val[res] = {Sp::Row, nm};
      return;
    }
    std::vector<std::string> args;
    for (auto *v : opsv) args.push_back(val[v].name);
    body << "  const " << T << " " << nm << " = " << elementExpr(op, args, at_, U) << ";\n";
    val[res] = {Sp::Scalar, nm};
  }

  void emitReduce(const Op *op) {
    if (op->ins.size() != 1 || op->outs.size() != 1) unsupported(op, "multi-operand linalg.reduce");
    int last = (int)A.D.size() - 1;
    if (op->dims.size() != 1 || op->dims[0] != last) unsupported(op, "reduction over a non-last axis");
    const Value *x = op->ins[0];
    ensure(x);
    if (val[x].sp != Sp::Full) unsupported(op, "reduction of a broadcast value");
    const Value *init = op->outs[0];
    Elem t = x->type.elem;
    Combiner cb = combinerFor(op, op->combiner, t);
    std::string T = ctype(t);
    // init per row: a fill of a constant/scalar, a row tensor argument, or an
    // uninitialised tensor.empty (the combiner's identity)
    std::string initAt;
    if (init->def && init->def->name == "linalg.fill") {
      const Value *c = init->def->ins[0];
      ensure(c);
      initAt = c->isConst ? constExpr(c, t) : val[c].name;
    } else if (init->argIdx >= 0) {
      ensure(init);
      initAt = atRow(init, "rr");
    } else if (init->isConst) {
      initAt = constExpr(init, t);
    } else if (init->def && init->def->name == "tensor.empty") {
      initAt = cb.identity;
    } else {
      unsupported(op, "reduction init must be a linalg.fill, an argument or tensor.empty");
    }
    const Value *res = op->results[0];
    std::string nm = fresh();
    val[res] = {A.D.size() == 1 ? Sp::Row : Sp::Row, nm};
    std::string xe = at(x, "e");
    if (orderedReduce.count(res)) {
      body << "  float " << nm << "_init[RPW];\n#pragma unroll\n  for (int rr = 0; rr < RPW; ++rr) " << nm << "_init[rr] = " << initAt
           << ";\n  float " << nm << "[RPW];\n  hf::row_sum_ordered<TR, RB, RPW, VEC, EPL, CHUNK, " << LOOKAHEAD
           << ">([&](int e) -> float { return " << xe << "; }, [&](int kk) {";
      for (auto &st : prefetchStmts) body << " " << st;
      prefetchStmts.clear(); // later chains find every chunk loaded
      body << " }, " << nm << "_init, " << nm << ", lds_chain, lds_bcast, rloc, lt, C);\n";
      body << "@@LAUNDER@@\n";
      afterOrdered = true;
      return;
    }
    std::string p = nm + "_p";
    body << "  " << T << " " << p << "[RPW];\n#pragma unroll\n  for (int rr = 0; rr < RPW; ++rr) " << p << "[rr] = " << cb.identity << ";\n";
    body << "#pragma unroll\n  for (int e = 0; e < RPW * EPL; ++e) ";
    if (masked) body << "if (" << colExpr("e") << " < C) ";
    body << p << "[e / EPL] = " << subst(cb.expr, xe, p + "[e / EPL]") << ";\n";
    int slot = nred++;
    body << "#pragma unroll\n  for (int rr = 0; rr < RPW; ++rr) " << p << "[rr] = hf::row_allreduce<TR, RB>(" << p << "[rr], [](" << T
         << " A, " << T << " B) { return " << cb.expr << "; }, (" << T << "*)(lds_red + (" << slot << " * RPW + rr) * RB * WPR), rloc, lt);\n";
    body << "  " << T << " " << nm << "[RPW];\n#pragma unroll\n  for (int rr = 0; rr < RPW; ++rr) " << nm << "[rr] = "
         << subst(cb.expr, p + "[rr]", initAt) << ";\n";
    body << "@@LAUNDER@@\n";
  }

  void emitStore(size_t i) {
    const Value *v = A.f->returns[i];
    if (v->argIdx >= 0 && A.resultTied[i] == v->argIdx) return;
    ensure(v);
    Elem e = v->type.elem;
    std::string ptr = resultPtr(A, i);
    std::string M = mtype(e);
    Sp s = val[v].sp;
    Sp ms = A.map.count(v) ? spaceOfMap(A.map.at(v)) : s;
    if (ms == Sp::Full) {
      // chunk by chunk: VEC values are computed, then stored with one access.
      // Rows past R were clamped to row R-1 and recompute its exact values, so
      // the store needs no (divergent) row guard.
      auto storeLoop = [&](const std::string &ex, const std::string &ind) {
        body << ind << "#pragma unroll\n" << ind << "for (int rr = 0; rr < RPW; ++rr)\n#pragma unroll\n" << ind
             << "  for (int j = 0; j < EPL / VEC; ++j) {\n" << ind << "    " << M << " st_[VEC];\n#pragma unroll\n" << ind
             << "    for (int v = 0; v < VEC; ++v) st_[v] = (" << M << ")(" << at(v, "rr * EPL + j * VEC + v", ex) << ");\n"
             << ind << "    hf::row_store_chunk<" << M << ", VEC, TR, MASKED>((" << M << "*)" << ptr
             << " + row[rr] * C, lt, C, j, st_);\n" << ind
             << "    __builtin_amdgcn_sched_barrier(0); // bound the live range to one chunk\n" << ind << "  }\n";
      };
      const V &q = val[v];
      if (q.quant8 && e == Elem::I8) {
        // int8 quantisation: four elements per packed word through
        // hf::quant8x4 in the fast pass; the exact pass stores element-wise
        body << "  if constexpr (EXM::value || VEC % 4 != 0) {\n";
        storeLoop("ex", "    ");
        const std::string rcp = q.qRcpRow ? q.qRcp + "[rr]" : q.qRcp;
        body << "  } else {\n#pragma unroll\n    for (int rr = 0; rr < RPW; ++rr)\n#pragma unroll\n"
             << "      for (int j = 0; j < EPL / VEC; ++j) {\n        uint32_t st_[VEC / 4];\n#pragma unroll\n"
             << "        for (int w = 0; w < VEC / 4; ++w) {\n          float a_[4];\n#pragma unroll\n"
             << "          for (int i = 0; i < 4; ++i) a_[i] = " << at(q.qSrc, "rr * EPL + j * VEC + 4 * w + i") << ";\n"
             << "          st_[w] = hf::quant8x4<" << (int)q.lo << ", " << (int)q.hi << ">(a_, " << q.qDiv << ", " << rcp
             << ", hf_g);\n"
             << "        }\n        hf::row_store_chunk<int8_t, VEC, TR, MASKED>((int8_t*)" << ptr
             << " + row[rr] * C, lt, C, j, (const int8_t*)st_);\n"
             << "        __builtin_amdgcn_sched_barrier(0); // bound the live range to one chunk\n      }\n  }\n";
      } else {
        storeLoop("ex", "  ");
      }
    } else if (ms == Sp::Row || (ms == Sp::Scalar && A.D.size() == 1)) {
      std::string idx = ms == Sp::Row ? "row[rr]" : "0";
      body << "#pragma unroll\n  for (int rr = 0; rr < RPW; ++rr) if (row_ok[rr] && lt == 0) ((" << M << "*)" << ptr << ")[" << idx
           << "] = " << (s == Sp::Scalar ? val[v].name : atRow(v, "rr")) << ";\n";
    } else if (ms == Sp::Col) {
      body << "  if (blockIdx.x == 0 && rloc == 0) {\n    " << M << " st_[EPL];\n    for (int ee = 0; ee < EPL; ++ee) st_[ee] = (" << M
           << ")(" << at(v, "ee") << ");\n    hf::row_store<" << M << ", VEC, EPL / VEC, TR, MASKED>((" << M << "*)" << ptr
           << ", lt, C, st_);\n  }\n";
    } else {
      throw CompileError("cannot store a scalar result");
    }
  }

  KernelPlan run(const std::string &kname, const std::string &kind) {
    markOrdered();
    chooseSchedule();
    Func &f = *A.f;
    for (Op *op : f.ops) {
      const std::string &n = op->name;
      if (n == "tensor.empty" || n == "arith.constant" || n == "tensor.dim" ||
          (n.rfind("arith.", 0) == 0 && !op->results.empty() && !op->results[0]->type.tensor))
        continue;
      if (n == "linalg.fill") {
        const Value *c = op->ins[0];
        ensure(c);
        val[op->results[0]] = {Sp::Scalar, c->isConst ? constExpr(c, op->results[0]->type.elem) : val[c].name};
        continue;
      }
      if (n == "linalg.broadcast") {
        ensure(op->ins[0]);
        val[op->results[0]] = val[op->ins[0]];
        continue;
      }
      if (n == "linalg.reduce") { emitReduce(op); continue; }
      if (isElementwiseOp(op)) { emitElementwise(op); continue; }
      unsupported(op, "op in a " + kind + " group");
    }
    for (size_t i = 0; i < f.returns.size(); ++i) emitStore(i);

    KernelPlan p;
    p.kernelName = kname;
    p.kind = kind;
    p.variant = needOrdered ? "row-resident, serial-order fp32 sum" : "row-resident";
    int block = TR * RB;
    int64_t rowsPerBlock = (int64_t)RB * RPW;
    int64_t grid = (R + rowsPerBlock - 1) / rowsPerBlock;
    std::ostringstream k;
    std::string params = kernelParamList(A, p.kargs, false);
    std::string argNames;
    for (size_t i = 0; i < A.params.size(); ++i) argNames += (A.params[i].role == "scalar" ? "s" : "p") + std::to_string(i) + ", ";
    for (size_t i = 0; i < A.results.size(); ++i)
      if (A.resultTied[i] < 0) argNames += "r" + std::to_string(i) + ", ";
    if (A.rowsDyn) {
      if (R != kRuntimeRows) throw CompileError("runtime row counts: the row program's rows are not the row count");
      argNames += "hf_rows, ";
      p.rowsDyn = true;
      p.rowsA = 1;
      p.rowsB = rowsPerBlock;
    }
    std::string ldsParams = "uint64_t* lds_red, float* lds_chain, float* lds_bcast";
    std::string ldsArgs = "lds_red_, lds_chain_, lds_bcast_";
    // the row program, instantiated for a fast (kFast) and an exact (kExact) mode
    k << "template <typename EXM>\n__device__ __forceinline__ bool " << kname << "_body(" << params << ", " << ldsParams << ") {\n"
      << "  const EXM ex{};\n  (void)ex; (void)lds_red; (void)lds_chain; (void)lds_bcast;\n"
      << "  constexpr int TR = " << TR << ", RB = " << RB << ", RPW = " << RPW << ", VEC = " << VEC << ", EPL = " << EPL
      << ", WPR = " << std::max(1, TR / 64) << ";\n"
      << "  constexpr bool MASKED = " << (masked ? "true" : "false") << ";\n"
      << (A.rowsDyn ? std::string("  const int64_t R = hf_rows;\n  constexpr int64_t C = ") + std::to_string(C) + "ll;\n"
                    : "  constexpr int64_t R = " + std::to_string(R) + "ll, C = " + std::to_string(C) + "ll;\n")
      << "  const int tid = threadIdx.x, rloc = tid / TR, lt = tid % TR;\n"
      << "  int64_t row[RPW];\n  bool row_ok[RPW];\n"
      << "#pragma unroll\n  for (int rr = 0; rr < RPW; ++rr) {\n"
      << "    // a row group of whole waves has wave-uniform rows: keep them in SGPRs\n"
      << "    const int rl_ = TR % 64 == 0 ? __builtin_amdgcn_readfirstlane(rloc) : rloc;\n"
      << "    const int64_t r_ = ((int64_t)blockIdx.x * RB + rl_) * RPW + rr;\n"
      << "    row_ok[rr] = r_ < R;\n    row[rr] = r_ < R ? r_ : R - 1;\n  }\n"
      << "  (void)row_ok; (void)lt;\n"
      << "  hf::Guard hf_g; // evidence that every fast-path element is exact\n";
    if (needOrdered) k << "  constexpr int CHUNK = " << CH << ";\n";
    k << pre.str() << resolveLaunder(body.str()) << "  return hf_g.bad();\n}\n";
    // LDS of the kernel, shared by both instantiations
    int redWords = std::max(1, nred * RPW * RB * std::max(1, TR / 64));
    int chainWords = needOrdered ? 2 * RB * RPW * (CH + 4) : 1;
    int bcastWords = needOrdered ? RB * RPW : 1;
    bool anyFast = false;
    for (auto &kv : val) anyFast |= kv.second.fast;
    if (anyFast)
      k << "__device__ __attribute__((noinline)) void " << kname << "_exact(" << params << ", " << ldsParams << ") {\n"
        << "  " << kname << "_body<hf::kExact>(" << argNames << "lds_red, lds_chain, lds_bcast);\n}\n";
    // row programs without a serial chain: ask for two resident blocks per CU
    // so that one block's loads overlap the other's arithmetic
    std::string occ;
    if (!needOrdered && block >= 256)
      occ = " __attribute__((amdgpu_waves_per_eu(" + std::to_string(std::min(8, block / 128)) + ")))";
    k << "extern \"C\" __global__ __launch_bounds__(" << block << ")" << occ << " void " << kname << "(" << params << ") {\n"
      << "  __shared__ uint64_t lds_red_[" << redWords << "];\n"
      << "  __shared__ __attribute__((aligned(16))) float lds_chain_[" << chainWords << "];\n"
      << "  __shared__ float lds_bcast_[" << bcastWords << "];\n"
      << "  const bool bad = " << kname << "_body<hf::kFast>(" << argNames << ldsArgs << ");\n";
    if (anyFast)
      k << "  // rare: some element's fast path could not vouch for its exact value;\n"
        << "  // the whole block recomputes its rows with IEEE division\n"
        << "  if (__syncthreads_or(bad)) " << kname << "_exact(" << argNames << ldsArgs << ");\n";
    else
      k << "  (void)bad;\n";
    k << "}\n";
    p.source = k.str();
    p.grid[0] = (unsigned)grid;
    p.block[0] = (unsigned)block;
    return p;
  }

  // At each reduction boundary, launder the input arrays that are still read
  // afterwards (and only those, so dead arrays are not kept alive).
  std::string resolveLaunder(const std::string &b) const {
    std::string out;
    size_t pos = 0;
    const std::string mark = "@@LAUNDER@@\n";
    while (true) {
      size_t m = b.find(mark, pos);
      if (m == std::string::npos) { out += b.substr(pos); break; }
      out += b.substr(pos, m - pos);
      std::string rest = b.substr(m + mark.size());
      auto mentions = [&](const std::string &id) {
        for (size_t q = rest.find(id); q != std::string::npos; q = rest.find(id, q + 1)) {
          char nx = q + id.size() < rest.size() ? rest[q + id.size()] : ' ';
          char pv = q ? rest[q - 1] : ' ';
          if (!std::isalnum((unsigned char)nx) && nx != '_' && !std::isalnum((unsigned char)pv) && pv != '_') return true;
        }
        return false;
      };
      for (auto &a : arrays) {
        if (declaredAt.count(a) && declaredAt.at(a) > m) continue; // declared later
        bool used = mentions(a);
        for (auto &kv : lazyDeps)
          if (!used && kv.second.count(a) && mentions(kv.first)) used = true;
        if (used) out += "  hf::launder(" + a + ");\n";
      }
      pos = m + mark.size();
    }
    return out;
  }
};

// ======================================================================
// PURE_ELEMWISE / ANY_PB: streaming kernel over the flattened domain.
// ======================================================================
struct EltwiseEmitter {
  Analysis &A;
  std::ostringstream body;
  std::map<const Value *, std::string> name;
  std::map<const Value *, bool> vec; // per-element array vs. uniform scalar
  int tmp = 0;
  int VEC = 4;
  int64_t N = 1;
  // transposed inputs: tiles of 64 (dim TQ) x 64 (last dim) staged through
  // LDS, read along TQ (their contiguous dim) and consumed along the last dim
  int TQ = -1;
  std::vector<const Value *> staged;
  // a tile spans TILE positions of the staged inputs' contiguous dim and TL of
  // the output's; PITCH = TL + 1 words (the odd pitch spreads both access
  // patterns over all banks)
  static constexpr int TILE = 64;
  int TL = 64, PITCH = 65;

  EltwiseEmitter(Analysis &a) : A(a) {}
  std::string fresh() { return "v" + std::to_string(tmp++); }

  std::string at(const Value *v) { return vec.at(v) ? name.at(v) + "[e]" : name.at(v); }

  // flat index of the chunk base inside an input spanning dims `m`
  std::string indexFor(const std::vector<int> &m) {
    int r = (int)A.D.size();
    if ((int)m.size() == r) {
      bool ident = true;
      for (int i = 0; i < r; ++i) ident &= m[i] == i;
      if (ident) return "base";
    }
    if (m.empty()) return "0";
    std::string s;
    int64_t stride = 1;
    for (int i = (int)m.size() - 1; i >= 0; --i) {
      std::string term = "c" + std::to_string(m[i]) + " * " + std::to_string(stride) + "ll";
      s = s.empty() ? term : term + " + " + s;
      stride *= A.D[m[i]];
    }
    return s;
  }
  // element stride of D dim d inside a tensor spanning dims `m` (0: absent)
  int64_t strideOf(const std::vector<int> &m, int d) const {
    int64_t stride = 1;
    for (int i = (int)m.size() - 1; i >= 0; --i) {
      if (m[i] == d) return stride;
      stride *= A.D[m[i]];
    }
    return 0;
  }
  static std::string wordType(Elem e) { return elemBytes(e) == 8 ? "uint64_t" : "uint32_t"; }
  static std::string uintOf(Elem e) {
    switch (elemBytes(e)) {
    case 1: return "uint8_t";
    case 2: return "uint16_t";
    case 4: return "uint32_t";
    default: return "uint64_t";
    }
  }
  std::string ldsName(const Value *v) const { return "lds_in" + std::to_string(v->argIdx); }

  void ensure(const Value *v) {
    if (name.count(v)) return;
    if (!v->type.tensor || v->isConst) {
      if (v->isConst) name[v] = constExpr(v, v->type.elem);
      else if (v->argIdx >= 0) name[v] = scalarArgExpr(A, v->argIdx);
      else throw CompileError("non-constant scalar " + v->name);
      vec[v] = false;
      return;
    }
    if (v->argIdx < 0) undefinedValue(v);
    int i = v->argIdx;
    const auto &m = A.map.at(v);
    int r = (int)A.D.size();
    std::string T = ctype(v->type.elem), M = mtype(v->type.elem);
    std::string nm = "in" + std::to_string(i);
    name[v] = nm;
    bool hasLast = !m.empty() && m.back() == r - 1;
    int64_t sLast = r ? strideOf(m, r - 1) : 0;
    const bool isStaged = std::find(staged.begin(), staged.end(), v) != staged.end();
    std::string P = "((const " + M + "*)p" + std::to_string(i) + ")";
    std::string cvt = v->type.elem == Elem::I1 ? " != 0" : "";
    if (isStaged) {
      vec[v] = true;
      body << "    " << T << " " << nm << "[VEC];\n#pragma unroll\n    for (int e = 0; e < VEC; ++e) " << nm
           << "[e] = __builtin_bit_cast(" << M << ", (" << uintOf(v->type.elem) << ")" << ldsName(v) << "[lq * " << PITCH
           << " + ll + e])" << cvt << ";\n";
    } else if (hasLast) {
      vec[v] = true;
      if (v->type.elem == Elem::I1) {
        body << "    " << T << " " << nm << "[VEC]; { uint8_t t_[VEC]; hf::vec_load<uint8_t, VEC>((const uint8_t*)p" << i << " + " << indexFor(m)
             << ", t_); for (int e = 0; e < VEC; ++e) " << nm << "[e] = t_[e] != 0; }\n";
      } else {
        body << "    " << T << " " << nm << "[VEC]; hf::vec_load<" << M << ", VEC>((const " << M << "*)p" << i << " + " << indexFor(m) << ", " << nm << ");\n";
      }
    } else if (sLast) {
      // a permuted input not staged through LDS: one load per element
      vec[v] = true;
      body << "    " << T << " " << nm << "[VEC];\n#pragma unroll\n    for (int e = 0; e < VEC; ++e) " << nm << "[e] = " << P << "["
           << indexFor(m) << " + (int64_t)e * " << sLast << "ll]" << cvt << ";\n";
    } else {
      vec[v] = false;
      body << "    const " << T << " " << nm << " = " << P << "[" << indexFor(m) << "]" << cvt << ";\n";
    }
  }

  // Inputs whose contiguous dim is not the domain's last one (transposed
  // loads): the most common such dim becomes TQ and its inputs are staged.
  void chooseStaging() {
    const int r = (int)A.D.size();
    if (r < 2) return;
    std::map<int, int> count;
    for (const Value *a : A.f->args) {
      if (!a->type.tensor || !A.map.count(a) || a->users.empty()) continue;
      const auto &m = A.map.at(a);
      if (m.empty() || m.back() == r - 1 || !strideOf(m, r - 1)) continue;
      if (elemBytes(a->type.elem) > 8) continue;
      ++count[m.back()];
    }
    if (count.empty()) return;
    int best = -1, bc = 0;
    for (auto &kv : count) if (kv.second > bc) { best = kv.first; bc = kv.second; }
    TQ = best;
    for (const Value *a : A.f->args) {
      if (!a->type.tensor || !A.map.count(a) || a->users.empty()) continue;
      const auto &m = A.map.at(a);
      if (!m.empty() && m.back() == TQ && strideOf(m, r - 1)) staged.push_back(a);
    }
  }

  void emitOps() {
    Func &f = *A.f;
    for (Op *op : f.ops) {
      const std::string &n = op->name;
      if (n == "tensor.empty" || n == "arith.constant" || n == "tensor.dim" || (n.rfind("arith.", 0) == 0 && !op->results[0]->type.tensor))
        continue;
      if (n == "linalg.fill") {
        ensure(op->ins[0]);
        name[op->results[0]] = name[op->ins[0]];
        vec[op->results[0]] = false;
        continue;
      }
      if (n == "linalg.broadcast" || n == "linalg.transpose") {
        // both are views: the value at a domain point is the operand's value
        // at the point its own map selects
        const Value *in = op->ins[0];
        ensure(in);
        const Value *res = op->results.empty() ? op->outs[0] : op->results[0];
        name[res] = name[in];
        vec[res] = vec[in];
        continue;
      }
      if (!isElementwiseOp(op)) unsupported(op, "op in an elementwise group");
      std::vector<const Value *> opsv;
      for (auto *v : op->ins) opsv.push_back(v);
      for (auto *v : op->operands) opsv.push_back(v);
      bool anyVec = false;
      for (auto *v : opsv) { ensure(v); anyVec |= vec[v]; }
      const Value *res = op->results[0];
      Elem U = res->type.elem;
      std::vector<Elem> at_;
      for (auto *v : opsv) at_.push_back(v->type.elem);
      std::string nm = fresh();
      name[res] = nm;
      vec[res] = anyVec;
      std::vector<std::string> args;
      for (auto *v : opsv) args.push_back(at(v));
      if (anyVec)
        body << "    " << ctype(U) << " " << nm << "[VEC];\n#pragma unroll\n    for (int e = 0; e < VEC; ++e) " << nm << "[e] = "
             << elementExpr(op, args, at_, U) << ";\n";
      else
        body << "    const " << ctype(U) << " " << nm << " = " << elementExpr(op, args, at_, U) << ";\n";
    }
    for (size_t i = 0; i < f.returns.size(); ++i) {
      const Value *v = f.returns[i];
      if (v->argIdx >= 0) continue;
      if (v->type.shape != A.D) throw CompileError("elementwise group result must span the whole domain");
      if (A.map.count(v)) {
        const auto &m = A.map.at(v);
        for (size_t d = 0; d < m.size(); ++d)
          if (m[d] != (int)d) throw CompileError("elementwise group result stored in a permuted layout");
      }
      ensure(v);
      std::string src = name[v];
      Elem e = v->type.elem;
      if (!vec[v] || e == Elem::I1) {
        std::string t = fresh();
        body << "    " << mtype(e) << " " << t << "[VEC];\n    for (int e = 0; e < VEC; ++e) " << t << "[e] = " << at(v) << ";\n";
        src = t;
      }
      body << "    hf::vec_store<" << mtype(e) << ", VEC>((" << mtype(e) << "*)" << resultPtr(A, i) << " + base, " << src << ");\n";
    }
  }

  KernelPlan run(const std::string &kname, const std::string &kind) {
    int r = (int)A.D.size();
    N = 1;
    for (auto d : A.D) N *= d;
    int maxBytes = 1;
    for (auto &kv : A.map) maxBytes = std::max(maxBytes, elemBytes(kv.first->type.elem));
    VEC = std::max(1, 16 / maxBytes);
    if (VEC > 8) VEC = 8;
    int64_t L = r ? A.D[r - 1] : 1;
    while (VEC > 1 && L % VEC) VEC /= 2;
    chooseStaging();
    if (TQ >= 0) return runTiled(kname, kind);
    // a runtime row count: dim 0 is the row count, the rest a static row
    const bool dynRows = A.rowsDyn && r >= 2 && A.D[0] == kRuntimeRows;
    // coordinates of the chunk base
    std::ostringstream coords;
    if (r > 1) {
      coords << "    int64_t t_ = base;\n";
      for (int d = r - 1; d >= 0; --d) {
        if (d == 0 && dynRows) {
          coords << "    const int64_t c0 = t_;\n";
          continue;
        }
        coords << "    const int64_t c" << d << " = t_ % " << A.D[d] << "ll; t_ /= " << A.D[d] << "ll;\n";
      }
      coords << "    (void)t_;\n";
      for (int d = 0; d < r; ++d) coords << "    (void)c" << d << ";\n";
    } else if (r == 1) {
      coords << "    const int64_t c0 = base; (void)c0;\n";
    }
    body << coords.str();
    emitOps();
    KernelPlan p;
    p.kernelName = kname;
    p.kind = kind;
    p.variant = "streaming";
    int block = 256;
    int64_t nch = N / VEC;
    // chunks of VEC elements per row (a row's length is a multiple of VEC)
    const int64_t nchRow = dynRows ? N / kRuntimeRows / VEC : 0;
    if (dynRows) {
      p.rowsDyn = true;
      p.rowsA = nchRow;
      p.rowsB = block;
      p.rowsCap = 1 << 20;
    }
    std::ostringstream k;
    k << "extern \"C\" __global__ __launch_bounds__(" << block << ") void " << kname << "("
      << kernelParamList(A, p.kargs, false) << ") {\n"
      << "  constexpr int VEC = " << VEC << ";\n"
      << (dynRows ? "  const int64_t NCH = hf_rows * " + std::to_string(nchRow) + "ll;\n"
                  : "  constexpr int64_t NCH = " + std::to_string(nch) + "ll;\n")
      << "  for (int64_t ch = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; ch < NCH; ch += (int64_t)gridDim.x * blockDim.x) {\n"
      << "    const int64_t base = ch * VEC;\n"
      << body.str() << "  }\n}\n";
    p.source = k.str();
    int64_t grid = (nch + block - 1) / block;
    if (grid > (1 << 20)) grid = 1 << 20;
    if (grid < 1) grid = 1;
    p.grid[0] = (unsigned)grid;
    p.block[0] = block;
    return p;
  }

  // Tiles of 64 (TQ) x 64 (last dim) of the domain.  Each staged input's
  // tile is read with loads along TQ (its own contiguous dim, VQ elements a
  // lane) into an LDS tile [TQ][last] of 32/64-bit words; then each lane
  // computes VEC consecutive elements along the last dim from LDS and the
  // other inputs, and stores them with one access.  Replaces the Ascend
  // Transpose2D / Transpose3D templates
  // (bishengir/lib/Template/lib/Vector/Transpose/Transpose2D.cpp).
  KernelPlan runTiled(const std::string &kname, const std::string &kind) {
    const int r = (int)A.D.size(), LD = r - 1;
    const int64_t DQ = A.D[TQ], DL = A.D[LD];
    // 128 output positions per tile when the output dim is long enough: the
    // concurrently running workgroups (consecutive tiles run along the output's
    // contiguous dim) then extend each output row in 512-byte runs
    TL = DL >= 128 && staged.size() <= 2 ? 128 : 64;
    PITCH = TL + 1;
    const int64_t NTQ = (DQ + TILE - 1) / TILE, NTL = (DL + TL - 1) / TL;
    int64_t NO = 1;
    for (int d = 0; d < r; ++d) if (d != TQ && d != LD) NO *= A.D[d];
    const int64_t NT = NO * NTQ * NTL;
    const int block = 256;
    // the per-element body (coordinates c<d> and `base` set by the loop)
    emitOps();
    std::ostringstream k;
    KernelPlan p;
    p.kernelName = kname;
    p.kind = kind;
    p.variant = "LDS-staged transpose tiles (64x" + std::to_string(TL) + ")";
    k << "extern \"C\" __global__ __launch_bounds__(" << block << ") void " << kname << "("
      << kernelParamList(A, p.kargs, false) << ") {\n"
      << "  constexpr int VEC = " << VEC << ";\n";
    for (const Value *v : staged)
      k << "  __shared__ " << wordType(v->type.elem) << " " << ldsName(v) << "[" << TILE * PITCH << "];\n";
    // Workgroup b runs on XCD b % 8.  Each run of 8 G consecutive tiles is
    // dealt out so that XCD x takes G consecutive tiles of it (G = NTL / 8
    // when a row of tiles splits evenly: each XCD then extends its own
    // stretch of every output row).  Measured at [4096, 8192] bf16 -> f32:
    // 37.7 us dealt one tile at a time, 36.1 us with G = 4 (2 and 8: 36.4,
    // 36.5; 16 and 64: 37.2, 38.1).
    const int64_t G = NTL % 8 == 0 && NTL / 8 <= 8 ? NTL / 8 : NTL >= 32 ? 4 : 1;
    const int64_t NTF = NT / (8 * G) * (8 * G);
    k << "  for (int64_t tile = blockIdx.x; tile < " << NT << "ll; tile += gridDim.x) {\n"
      << "    int64_t t_ = tile;\n";
    if (G > 1)
      k << "    if (tile < " << NTF << "ll) t_ = tile / " << 8 * G << "ll * " << 8 * G << "ll + tile % 8 * " << G
        << "ll + tile % " << 8 * G << "ll / 8;\n";
    k << "    const int64_t tl_ = t_ % " << NTL << "ll; t_ /= " << NTL << "ll;\n"
      << "    const int64_t tq_ = t_ % " << NTQ << "ll; t_ /= " << NTQ << "ll;\n";
    for (int d = r - 1; d >= 0; --d) {
      if (d == TQ || d == LD) continue;
      k << "    const int64_t c" << d << " = t_ % " << A.D[d] << "ll; t_ /= " << A.D[d] << "ll; (void)c" << d << ";\n";
    }
    k << "    __syncthreads(); // the previous tile's LDS reads are done\n";
    for (const Value *v : staged) {
      const auto &m = A.map.at(v);
      std::string M = mtype(v->type.elem), U = uintOf(v->type.elem), W = wordType(v->type.elem);
      int VQ = std::max(1, 16 / elemBytes(v->type.elem));
      if (VQ > 8) VQ = 8;
      while (VQ > 1 && DQ % VQ) VQ /= 2;
      const int lanesPerRow = TILE / VQ;
      const int nItems = TL * lanesPerRow, nLd = (nItems + block - 1) / block;
      // every load of the tile in flight before the first LDS write
      k << "    {\n      " << M << " w_[" << nLd << "][" << VQ << "];\n      bool ok_[" << nLd << "];\n"
        << "#pragma unroll\n      for (int it_ = 0; it_ < " << nLd << "; ++it_) {\n"
        << "        const int i_ = threadIdx.x + it_ * " << block << ";\n"
        << "        const int lq0 = (i_ % " << lanesPerRow << ") * " << VQ << ", ll = i_ / " << lanesPerRow << ";\n"
        << "        const int64_t c" << TQ << " = tq_ * " << TILE << " + lq0, c" << LD << " = tl_ * " << TL << " + ll;\n"
        << "        ok_[it_] = i_ < " << nItems << " && c" << LD << " < " << DL << "ll && c" << TQ << " < " << DQ << "ll;\n"
        << "        if (!ok_[it_]) continue;\n"
        << "        const " << M << "* src_ = (const " << M << "*)p" << v->argIdx << " + (" << indexFor(m) << ");\n";
      if (VQ > 1)
        k << "        hf::vec_load<" << M << ", " << VQ << ">(src_, w_[it_]);\n";
      else
        k << "        w_[it_][0] = src_[0];\n";
      k << "      }\n#pragma unroll\n      for (int it_ = 0; it_ < " << nLd << "; ++it_) {\n"
        << "        if (!ok_[it_]) continue;\n"
        << "        const int i_ = threadIdx.x + it_ * " << block << ";\n"
        << "        const int lq0 = (i_ % " << lanesPerRow << ") * " << VQ << ", ll = i_ / " << lanesPerRow << ";\n"
        << "#pragma unroll\n        for (int j = 0; j < " << VQ << "; ++j) " << ldsName(v) << "[(lq0 + j) * " << PITCH
        << " + ll] = (" << W << ")__builtin_bit_cast(" << U << ", w_[it_][j]);\n"
        << "      }\n    }\n";
    }
    const int lanesPerRow = TL / VEC;
    k << "    __syncthreads();\n"
      << "    for (int i_ = threadIdx.x; i_ < " << TILE * lanesPerRow << "; i_ += " << block << ") {\n"
      << "      const int lq = i_ / " << lanesPerRow << ", ll = (i_ % " << lanesPerRow << ") * VEC;\n"
      << "      const int64_t c" << TQ << " = tq_ * " << TILE << " + lq, c" << LD << " = tl_ * " << TL << " + ll;\n"
      << "      if (c" << LD << " >= " << DL << "ll || c" << TQ << " >= " << DQ << "ll) continue;\n"
      << "      (void)lq; (void)ll;\n"
      << "      int64_t base = 0;\n";
    for (int d = 0; d < r; ++d) k << "      base = base * " << A.D[d] << "ll + c" << d << ";\n";
    k << "      {\n" << body.str() << "      }\n    }\n  }\n}\n";
    p.source = k.str();
    p.grid[0] = (unsigned)std::max<int64_t>(1, std::min<int64_t>(NT, 8192));
    p.block[0] = block;
    return p;
  }
};

// ======================================================================
// REDUCE_WITH_INDEX
// ======================================================================
KernelPlan lowerReduceWithIndex(Analysis &A, const std::string &kname) {
  Func &f = *A.f;
  const Op *rw = findOp(f, [](const Op *o) { return o->name == "hfusion.reduce_with_index"; });
  for (const Op *op : f.ops) {
    const std::string &n = op->name;
    if (op == rw || n == "tensor.empty" || n == "linalg.fill" || n == "arith.constant" || n == "tensor.dim") continue;
    unsupported(op, "op fused with hfusion.reduce_with_index");
  }
  if (rw->ins.size() != 1) unsupported(rw, "reduce_with_index with an index input");
  const Value *x = rw->ins[0];
  if (x->argIdx < 0) unsupported(rw, "reduce_with_index input must be a group argument");
  int rank = (int)x->type.shape.size();
  if (rw->dims.size() != 1 || rw->dims[0] != rank - 1) unsupported(rw, "reduce_with_index over a non-last axis");
  std::string kindS = rw->angleKind.empty() ? rw->attr("reduce_kind", "max") : rw->angleKind;
  int kind;
  if (kindS == "max") kind = 0;
  else if (kindS == "min") kind = 1;
  else unsupported(rw, "reduce_with_index kind '" + kindS + "'");
  if (x->type.elem != Elem::F32) unsupported(rw, "reduce_with_index over non-f32 values");
  int64_t C = x->type.shape.back(), R = 1;
  for (int i = 0; i + 1 < rank; ++i) R *= x->type.shape[i];
  Elem idxE = rw->outs[1]->type.elem;
  if (idxE != Elem::I32 && idxE != Elem::I64) unsupported(rw, "index type");
  auto initOf = [&](const Value *o, Elem e) -> std::string {
    if (o->def && o->def->name == "linalg.fill") {
      const Value *c = o->def->ins[0];
      if (c->isConst) return constExpr(c, e);
      if (c->argIdx >= 0) return scalarArgExpr(A, c->argIdx);
    }
    if (o->argIdx >= 0) return "INIT_FROM_ARG";
    unsupported(rw, "reduce_with_index init must be a linalg.fill");
  };
  std::string iv = initOf(rw->outs[0], Elem::F32), ii = initOf(rw->outs[1], idxE);
  std::string ivArg, iiArg;
  if (iv == "INIT_FROM_ARG") { ivArg = "p" + std::to_string(rw->outs[0]->argIdx); iv = ""; }
  if (ii == "INIT_FROM_ARG") { iiArg = "p" + std::to_string(rw->outs[1]->argIdx); ii = ""; }
  // output pointers
  std::string outV = "nullptr", outI = "nullptr";
  for (size_t i = 0; i < f.returns.size(); ++i) {
    const Value *v = f.returns[i];
    if (v->def != rw) unsupported(rw, "group returns a value other than the reduction results");
    (v->resultIdx == 0 ? outV : outI) = resultPtr(A, i);
  }
  // schedule: with at least one row per CU, one workgroup per row (no
  // cross-workgroup step); otherwise about two workgroups per CU, each on a
  // segment of a row (a multiple of 4 elements, so float4 loads stay aligned).
  // hf::arg_schedule (hf_argmax.h) is the same rule for a runtime row count.
  const int64_t CUS = 256;
  auto schedule = [&](int64_t rows, int64_t &segs, int64_t &segLen) {
    segs = rows >= CUS ? 1 : std::max<int64_t>(1, (2 * CUS + rows - 1) / rows);
    segLen = ((C + segs - 1) / segs + 3) / 4 * 4;
    segLen = std::max<int64_t>(segLen, std::min<int64_t>((C + 3) / 4 * 4, 4096)); // no tiny segments
    segs = (C + segLen - 1) / segLen;
  };
  int64_t segs, segLen;
  schedule(A.rowsDyn ? CUS : R, segs, segLen);
  const int BLOCK = segLen >= 32768 ? 1024 : (segLen >= 8192 ? 512 : 256);
  bool aligned = (C % 4) == 0;
  KernelPlan p;
  p.kernelName = kname;
  p.kind = "REDUCE_WITH_INDEX";
  std::ostringstream k;
  std::string IT = ctype(idxE);
  if (A.rowsDyn) {
    if (R != kRuntimeRows) unsupported(rw, "a runtime row count that is not the rows of the input");
    // the largest workspace any row count asks for (from CUS rows on, one
    // segment per row and no records)
    uint64_t ws = 256;
    for (int64_t r = 1; r < CUS; ++r) {
      int64_t sg, sl;
      schedule(r, sg, sl);
      ws = std::max<uint64_t>(ws, (uint64_t)(r * sg * 16 + r * 4 + 256));
    }
    p.variant = "runtime rows: split rows below one per CU, a workgroup per row above";
    k << "extern \"C\" __global__ __launch_bounds__(" << BLOCK << ") void " << kname << "("
      << kernelParamList(A, p.kargs, true) << ") {\n"
      << "  constexpr int64_t C = " << C << "ll;\n"
      << "  auto init = [&](int64_t row, float &v, " << IT << " &i) {\n"
      << "    v = " << (ivArg.empty() ? iv : "((const float*)" + ivArg + ")[row]") << ";\n"
      << "    i = " << (iiArg.empty() ? ii : "((const " + IT + "*)" + iiArg + ")[row]") << ";\n  };\n"
      << "  hf::argreduce_rows_dyn<" << kind << ", " << BLOCK << ", " << (aligned ? "true" : "false") << ", " << IT
      << ">((const float*)p" << x->argIdx << ", hf_rows, C, " << ws << "ull, init, (float*)" << outV << ", (" << IT << "*)"
      << outI << ", ws);\n}\n";
    p.source = k.str();
    // R * SEG work items (at most ceil(C / min(C, 4096)) segments a row)
    p.rowsDyn = true;
    p.rowsA = (C + std::min<int64_t>(C, 4096) - 1) / std::min<int64_t>(C, 4096);
    p.rowsB = 1;
    p.rowsCap = 2048;
    p.block[0] = BLOCK;
    p.workspaceBytes = ws;
    p.workspaceZeroInit = true;
    return p;
  }
  p.variant = segs == 1 ? "one workgroup per row, streaming" : "split-row two-level, last-block combine";
  k << "extern \"C\" __global__ __launch_bounds__(" << BLOCK << ") void " << kname << "("
    << kernelParamList(A, p.kargs, true) << ") {\n"
    << "  constexpr int64_t R = " << R << "ll, C = " << C << "ll, SEG = " << segs << "ll, SEGLEN = " << segLen << "ll;\n"
    << "  const float init_v = " << (ivArg.empty() ? iv : "((const float*)" + ivArg + ")[blockIdx.x / SEG]") << ";\n"
    << "  const " << IT << " init_i = " << (iiArg.empty() ? ii : "((const " + IT + "*)" + iiArg + ")[blockIdx.x / SEG]") << ";\n"
    << "  hf::argreduce_rows<" << kind << ", " << BLOCK << ", " << (aligned ? "true" : "false") << ", " << IT
    << ">((const float*)p" << x->argIdx << ", R, C, SEG, SEGLEN, init_v, init_i, (float*)" << outV << ", (" << IT << "*)" << outI
    << ", ws);\n}\n";
  p.source = k.str();
  p.grid[0] = (unsigned)(R * segs);
  p.block[0] = BLOCK;
  // workspace: per-segment partial records + one arrival counter per row
  p.workspaceBytes = (uint64_t)(R * segs * 16 + R * 4 + 256);
  p.workspaceZeroInit = true;
  return p;
}

// ======================================================================
// SINGLE_CUBE: matmul + elementwise epilogue
// ======================================================================
// Epilogue of hivm.hir.matmul (HIVMMacroOps.td:373-398): C = descale * (A*B + bias),
// descale per channel ([N]) or per tensor ([1]) (HIVMAttrs.td:1061-1071).  The
// op has no CPU lowering in the reference (ConvertHIVMToUpstream has no mmad
// pattern); the arithmetic here is its documented formula with the accumulator
// type of the inputs: an integer bias joins the int32 accumulator exactly, then
// the sum goes to fp32 (round to nearest even); a float bias is added in fp32;
// the descale multiplies in fp32; the result is rounded to C's type (nearest
// even, saturating for integer C).
void hivmMatmulEpilogue(const Op *mm, bool intAcc, std::ostringstream &epi, std::ostringstream &colFields,
                        std::ostringstream &colLoads, std::string &outExpr) {
  auto named = [&](const char *k) -> const Value * {
    auto it = mm->attrs.find(std::string("operand.") + k);
    return it == mm->attrs.end() ? nullptr : mm->operands.at(std::stoul(it->second));
  };
  const Value *bias = named("bias"), *descale = named("descale");
  const std::string mode = mm->attr("descale_mode", descale ? "DescalePerChannel" : "DescaleNull");
  if (mode != "DescaleNull" && mode != "DescalePerChannel" && mode != "DescalePerTensor")
    unsupported(mm, "descale_mode " + mode);
  if ((mode == "DescaleNull") != (descale == nullptr)) unsupported(mm, "descale operand and descale_mode disagree");
  auto colLoad = [&](const Value *v, const std::string &nm) {
    if (v->argIdx < 0) unsupported(mm, "bias/descale must be group arguments");
    colFields << " " << ctype(v->type.elem) << " " << nm << ";";
    colLoads << "    Cv." << nm << " = ((const " << mtype(v->type.elem) << "*)P.p" << v->argIdx << ")[n];\n";
  };
  auto toF32 = [&](Elem e, const std::string &x) -> std::string {
    if (e == Elem::BF16) return "hf::bf16_to_f32(" + x + ")";
    if (e == Elem::F16) return "hf::f16_to_f32(" + x + ")";
    if (e == Elem::F32) return x;
    if (isInt(e)) return "hf::int_to_f32<0>((int64_t)(" + x + "))";
    unsupported(mm, "epilogue operand type");
  };
  std::string t = "acc";
  if (bias) {
    if (bias->type.shape.size() != 1) unsupported(mm, "bias must be a vector of shape [n]");
    colLoad(bias, "bias");
  }
  if (intAcc && bias && isInt(bias->type.elem)) {
    epi << "    const int32_t ib = acc + (int32_t)Cv.bias;\n";
    t = "ib";
  }
  epi << "    float t = " << (intAcc ? "hf::int_to_f32<0>((int64_t)(" + t + "))" : t) << ";\n";
  if (bias && !(intAcc && isInt(bias->type.elem))) epi << "    t = t + " << toF32(bias->type.elem, "Cv.bias") << ";\n";
  if (descale) {
    if (mode == "DescalePerChannel") {
      colLoad(descale, "descale");
      epi << "    t = t * " << toF32(descale->type.elem, "Cv.descale") << ";\n";
    } else {
      if (descale->argIdx < 0) unsupported(mm, "descale must be a group argument");
      epi << "    t = t * " << toF32(descale->type.elem, "((const " + mtype(descale->type.elem) + "*)P.p" +
                                                        std::to_string(descale->argIdx) + ")[0]") << ";\n";
    }
  }
  Elem oe = mm->outs[0]->type.elem;
  if (oe == Elem::F32) outExpr = "t";
  else if (oe == Elem::BF16) outExpr = "hf::f32_to_bf16<0>(t)";
  else if (oe == Elem::F16) outExpr = "hf::f32_to_f16<0>(t)";
  else if (oe == Elem::I8 || oe == Elem::I16 || oe == Elem::I32)
    outExpr = "hf::f32_to_int<" + ctype(oe) + ", 0, true>(t)";
  else unsupported(mm, "matmul output type");
}

constexpr int MK_BF16_CODE = 1; // hf::MK_BF16
KernelPlan lowerMatmul(Analysis &A, const std::string &kname, const LowerOptions &opt) {
  Func &f = *A.f;
  const Op *mm = findOp(f, [](const Op *o) {
    return o->name == "linalg.matmul" || o->name == "linalg.matmul_transpose_b" || o->name == "hivm.hir.matmul" ||
           o->name == "hfusion.matmul_mx";
  });
  const bool hivm = mm->name == "hivm.hir.matmul";
  const bool mx = mm->name == "hfusion.matmul_mx";
  const bool bT = hivm ? mm->attrs.count("b_transpose") != 0 : mm->name == "linalg.matmul_transpose_b";
  const bool aT = hivm && mm->attrs.count("a_transpose") != 0;
  // matmul_mx (HFusionOps.td:1233-1291): A [M, K], B [K, N] fp8 (or bytes
  // reinterpreted by hfusion.bitcast or by lhsFormat / rhsFormat), scales
  // [M, K/32] and [N, K/32] e8m0
  const Op *castA = nullptr, *castB = nullptr;
  auto throughBitcast = [&](const Value *v, const Op *&cast) {
    if (mx && v->def && v->def->name == "hfusion.bitcast" && !v->def->ins.empty()) {
      if (elemBits(v->def->ins[0]->type.elem) != 8 || v->def->ins[0]->type.shape != v->type.shape)
        unsupported(v->def, "matmul_mx operand bitcast from other than same-shape bytes");
      cast = v->def;
      return (const Value *)v->def->ins[0];
    }
    return v;
  };
  const Value *a = throughBitcast(mm->ins[0], castA), *b = throughBitcast(mm->ins[1], castB);
  if (a->argIdx < 0 || b->argIdx < 0) unsupported(mm, "matmul operands must be group arguments");
  if (a->type.shape.size() != 2 || b->type.shape.size() != 2) unsupported(mm, "matmul operands must be rank 2");
  int64_t M = aT ? a->type.shape[1] : a->type.shape[0], K = aT ? a->type.shape[0] : a->type.shape[1];
  int64_t N = bT ? b->type.shape[0] : b->type.shape[1];
  if ((bT ? b->type.shape[1] : b->type.shape[0]) != K) unsupported(mm, "matmul shapes");
  Elem ae = a->type.elem, be = b->type.elem;
  int mk = -1;
  bool fp4 = false;
  int64_t Kl = K; // logical K (fp4 packs two values per byte)
  const Value *sa = nullptr, *sb = nullptr;
  if (mx) {
    // the matrix core's format codes: 0 e4m3, 1 e5m2, 4 e2m1 (fp4).  The
    // lhsFormat / rhsFormat attribute (HFusionAttrs.td:131-137: FP8E5M2_T = 1,
    // FP8E4M3_T = 2, FP4E2M1_T = 3) decides over the element type when
    // present, as HFusionToHIVM keeps it for the HIVM op when the type does
    // not match it (Matmul.cpp:62-70); fp4 operands are bytes holding two
    // values along K, the even k in the low nibble (LocalMmadMx.cpp:131-133,
    // K factor 2)
    auto fmt = [&](const Value *orig, const char *attr) -> int {
      auto it = mm->attrs.find(attr);
      if (it != mm->attrs.end()) {
        int code = -1;
        size_t used = 0;
        try { code = std::stoi(it->second, &used); } catch (...) { code = -1; }
        if (used == 0) code = -1;
        if (code == 1) return 1;
        if (code == 2) return 0;
        if (code == 3) return 4;
        unsupported(mm, std::string("matmul_mx operand without a valid ") + attr);
      }
      const Elem e = orig->type.elem;
      if (e == Elem::F8E4M3FN) return 0;
      if (e == Elem::F8E5M2) return 1;
      if (e == Elem::I8) unsupported(mm, std::string("matmul_mx byte operand without a valid ") + attr);
      unsupported(mm, "matmul_mx operand type (f8E4M3FN, f8E5M2 or bytes with a format)");
      return -1;
    };
    const int fa = fmt(mm->ins[0], "lhsFormat"), fb = fmt(mm->ins[1], "rhsFormat");
    if ((fa == 4) != (fb == 4)) unsupported(mm, "matmul_mx mixing fp4 (e2m1) and fp8 operands");
    fp4 = fa == 4;
    mk = fp4 ? 7 : 3 + 2 * fa + fb;
    Kl = fp4 ? 2 * K : K;
    if (mm->ins.size() != 4) unsupported(mm, "matmul_mx takes A, B and two scale operands");
    sa = mm->ins[2];
    sb = mm->ins[3];
    if (sa->argIdx < 0 || sb->argIdx < 0) unsupported(mm, "matmul_mx scales must be group arguments");
    if (sa->type.elem != Elem::I8 || sb->type.elem != Elem::I8) unsupported(mm, "matmul_mx scales are ui8 / i8 (e8m0)");
    if (Kl % 32 != 0 || sa->type.shape != std::vector<int64_t>{M, Kl / 32} || sb->type.shape != std::vector<int64_t>{N, Kl / 32})
      unsupported(mm, "matmul_mx scales must be [M, K/32] and [N, K/32]");
    if (K % 128 != 0) unsupported(mm, fp4 ? "matmul_mx fp4 K must be a multiple of 256" : "matmul_mx K must be a multiple of 128");
    if (N % 16 != 0) unsupported(mm, "matmul_mx N must be a multiple of 16");
    if (mm->results[0]->type.elem != Elem::F32) unsupported(mm, "matmul_mx accumulates in f32");
    ae = be = Elem::I8; // bytes from here on
  } else if (ae == Elem::I8 && be == Elem::I8) mk = 0;
  else if (ae == Elem::BF16 && be == Elem::BF16) mk = 1;
  else if (ae == Elem::F16 && be == Elem::F16) mk = 2;
  if (mk < 0) unsupported(mm, "matmul element types (supported: i8 x i8, bf16 x bf16, f16 x f16, matmul_mx fp8 / fp4)");
  const bool i8 = mk == 0;
  if (!hivm && !mx) {
    Elem ce = mm->results[0]->type.elem;
    if (ce != (i8 ? Elem::I32 : Elem::F32)) unsupported(mm, "matmul accumulator type (i32 for i8, f32 for bf16/f16)");
  }
  const int esz = elemBytes(ae);
  if ((K * esz) % 16 != 0) unsupported(mm, "matmul K must span a multiple of 16 bytes");
  if (!bT && (N * esz) % 16 != 0) unsupported(mm, "matmul N must span a multiple of 16 bytes when B is [K, N]");
  if (aT && (M * esz) % 16 != 0) unsupported(mm, "matmul M must span a multiple of 16 bytes when A is [K, M]");
  // LDS DMA ring (operands K-contiguous: A [M, K], B [N, K]): 128-byte K
  // slices with two waves per SIMD when K allows, else 64-byte slices.  An
  // operand stored the other way round (B [K, N], A [K, M]) is first copied
  // K-contiguous into the workspace by a transpose kernel of its own, when
  // the DMA ring applies; otherwise the register-staging path reads it as is.
  // A B [K, N] with 128-byte K slices goes through the ring as it is
  // (mode 4): whole 256-byte k-rows are staged and the matrix-core operand is
  // formed by transposing LDS reads, so no re-layout pass is needed.
  // The 128-byte ring addresses each lane's source as a 32-bit offset from
  // a per-step base: 256 rows of K bytes, or 128 bytes' worth of k-rows of a
  // [K, N] / [K, M] operand, must stay below 2^32 bytes.
  // (a row-major operand's offsets count from its tile's first row, so only
  // a K-major operand's column count is bounded)
  const bool offs32 = K * esz <= (int64_t(1) << 24) && (!aT || M <= (int64_t(1) << 25)) && (bT || N <= (int64_t(1) << 25));
  if (mx && !offs32) unsupported(mm, "matmul_mx with K above 2^24 bytes or M, N above 2^25");
  const int dma0 = (K * esz) % 128 == 0 && offs32 ? 3 : (K * esz) % 64 == 0 ? 1 : 0;
  // The same holds for a bf16 / f16 B [K, N] (512-byte k-rows, 16-bit
  // transposing reads).
  // An A [K, M] is staged and read the same way.
  const bool kmajOk = (bT || (N * esz) % 16 == 0) && (!aT || (M * esz) % 16 == 0);
  const int dma = mx ? 4 : dma0 == 3 && (!bT || aT) && kmajOk ? 4 : dma0;
  const bool preB = dma != 0 && dma != 4 && !bT, preA = dma != 0 && dma != 4 && aT;
  const bool kT = (dma != 0 && dma != 4) || bT; // the main kernel's B is [N, K]
  const bool mT = (dma == 0 || dma == 4) && aT; // the main kernel's A is [K, M]
  const int threads = dma >= 3 ? 512 : 256;
  auto align256 = [](uint64_t v) { return (v + 255) / 256 * 256; };
  const uint64_t wsB = preB ? align256((uint64_t)(N * K * esz)) : 0, wsA = preA ? align256((uint64_t)(M * K * esz)) : 0;
  // matmul_mx with mx_exact=1: both operands scaled into bf16 by pre kernels
  // (workspace: A' [M, K] then B' [K, N]), then the bf16 contraction, whose
  // products are exact and whose sums are f32 (the fp8 matrix core's 64-k dot
  // product is not: about 2^-11 of the products' magnitude sum)
  const bool mxExact = mx && opt.mxExact;
  if (mxExact && fp4) unsupported(mm, "mx_exact=1 with fp4 operands (the option is for fp8)");
  // a runtime row count is M, the rows of a row-major A and of C
  if (A.rowsDyn && (aT || M != kRuntimeRows || mxExact))
    unsupported(mm, "a runtime row count other than the rows of A [M, K] (or with mx_exact=1)");
  const std::string Mx = A.rowsDyn ? std::string("hf_rows") : std::to_string(M) + "ll";
  const uint64_t wsXA = mxExact ? align256((uint64_t)(M * K * 2)) : 0, wsXB = mxExact ? align256((uint64_t)(K * N * 2)) : 0;
  // matmul_mx accumulates onto its `outs`: a tensor.empty (taken as zero) or
  // a constant fill, added after the contraction
  std::string accInit;
  if (mx) {
    const Value *acc0 = mm->outs.empty() ? nullptr : mm->outs[0];
    if (!acc0 || !acc0->def) unsupported(mm, "matmul_mx accumulator must be a tensor.empty or a constant linalg.fill");
    if (acc0->def->name == "linalg.fill") {
      if (!acc0->def->ins[0]->isConst) unsupported(mm, "matmul_mx accumulator fill must be a constant");
      if (acc0->def->ins[0]->fconst != 0.0) accInit = constExpr(acc0->def->ins[0], Elem::F32);
    } else if (acc0->def->name != "tensor.empty") {
      unsupported(mm, "matmul_mx accumulator must be a tensor.empty or a constant linalg.fill");
    }
  } else if (!hivm) {
    const Value *acc0 = mm->outs[0];
    if (!(acc0->def && acc0->def->name == "linalg.fill" && acc0->def->ins[0]->isConst && acc0->def->ins[0]->fconst == 0.0))
      unsupported(mm, "matmul accumulator must start from a zero linalg.fill");
  } else if (mm->outs.empty() || mm->outs[0]->argIdx < 0 || mm->outs[0]->type.shape != std::vector<int64_t>{M, N}) {
    unsupported(mm, "hivm.hir.matmul writes a [M, N] group argument");
  }
  // epilogue over D = [M, N] with the matmul result as the accumulator
  std::set<const Value *> excl = {a, b};
  if (mx) excl.insert({sa, sb, mm->ins[0], mm->ins[1]});
  A.D = {M, N};
  if (!hivm) inferMaps(A, excl);
  // per-element code, plus the operand loads split by their index: [m] once
  // per accumulator row, [n] once per column, [m, n] per element
  std::ostringstream epi, rowFields, rowLoads, colFields, colLoads;
  std::map<const Value *, std::string> name;
  int tmp = 0;
  auto ensure = [&](const Value *v) {
    if (name.count(v)) return;
    if (v == mm->results[0]) { name[v] = accInit.empty() ? "acc" : "(acc + " + accInit + ")"; return; }
    if (v->isConst || !v->type.tensor) {
      if (v->isConst) name[v] = constExpr(v, v->type.elem);
      else if (v->argIdx >= 0) name[v] = scalarArgExpr(A, v->argIdx);
      else throw CompileError("non-constant scalar in epilogue");
      return;
    }
    if (v->argIdx < 0) throw CompileError("internal: epilogue value " + v->name);
    const auto &m = A.map.at(v);
    std::string nm = "e" + std::to_string(tmp++);
    std::string T = ctype(v->type.elem), Mt = mtype(v->type.elem), P = "((const " + Mt + "*)P.p" + std::to_string(v->argIdx) + ")";
    if (m.size() == 2) {
      epi << "    const " << T << " " << nm << " = " << P << "[m * " << N << "ll + n];\n";
      name[v] = nm;
    } else if (m.empty()) {
      epi << "    const " << T << " " << nm << " = " << P << "[0];\n";
      name[v] = nm;
    } else if (m[0] == 0) {
      rowFields << " " << T << " " << nm << ";";
      rowLoads << "    R." << nm << " = " << P << "[m];\n";
      name[v] = "R." + nm;
    } else {
      colFields << " " << T << " " << nm << ";";
      colLoads << "    Cv." << nm << " = " << P << "[n];\n";
      name[v] = "Cv." + nm;
    }
  };
  std::string hivmOut;
  if (hivm) {
    for (const Op *op : f.ops)
      if (op != mm && !isAlias(op)) unsupported(op, "op beside hivm.hir.matmul in a group");
    hivmMatmulEpilogue(mm, i8, epi, colFields, colLoads, hivmOut);
  }
  for (const Op *op : f.ops) {
    if (hivm) break;
    const std::string &n = op->name;
    if (op == mm || op == castA || op == castB || n == "tensor.empty" || n == "arith.constant" || n == "tensor.dim" ||
        n == "linalg.fill")
      continue;
    if (n.rfind("arith.", 0) == 0 && !op->results[0]->type.tensor) continue;
    if (n == "linalg.broadcast") {
      ensure(op->ins[0]);
      name[op->results[0]] = name[op->ins[0]];
      continue;
    }
    if (!isElementwiseOp(op)) unsupported(op, "op in a matmul epilogue");
    std::vector<const Value *> opsv;
    for (auto *v : op->ins) opsv.push_back(v);
    for (auto *v : op->operands) opsv.push_back(v);
    std::vector<std::string> args;
    std::vector<Elem> at_;
    for (auto *v : opsv) { ensure(v); args.push_back(name[v]); at_.push_back(v->type.elem); }
    std::string nm = "t" + std::to_string(tmp++);
    Elem U = op->results[0]->type.elem;
    epi << "    const " << ctype(U) << " " << nm << " = " << elementExpr(op, args, at_, U) << ";\n";
    name[op->results[0]] = nm;
  }
  if (f.returns.size() != 1) unsupported(mm, "matmul groups must return exactly one tensor");
  const Value *outv = f.returns[0];
  if (outv->type.shape != std::vector<int64_t>{M, N}) unsupported(mm, "matmul group result shape");
  if (hivm) name[outv] = hivmOut;
  else ensure(outv);
  Elem oe = outv->type.elem;
  KernelPlan p;
  p.kernelName = kname;
  p.kind = "SINGLE_CUBE";
  std::ostringstream k;
  std::string params = kernelParamList(A, p.kargs, preA || preB || mxExact);
  // epilogue functor receives all kernel pointer arguments
  k << "namespace {\nstruct " << kname << "_args {";
  for (size_t i = 0; i < A.params.size(); ++i)
    k << (A.params[i].role == "scalar" ? " uint64_t s" : " const void* p") << i << ";";
  k << " };\n"
    << "struct " << kname << "_epi {\n"
    << "  using out_t = " << mtype(oe) << ";\n"
    << "  using args_t = " << kname << "_args;\n"
    << "  struct row_t {" << rowFields.str() << " int unused_; };\n"
    << "  struct col_t {" << colFields.str() << " int unused_; };\n"
    << "  __device__ __forceinline__ static row_t row(int64_t m, const args_t& P) {\n    row_t R{};\n" << rowLoads.str()
    << "    return R;\n  }\n"
    << "  __device__ __forceinline__ static col_t col(int64_t n, const args_t& P) {\n    col_t Cv{};\n" << colLoads.str()
    << "    return Cv;\n  }\n"
    << "  __device__ __forceinline__ static out_t apply(" << (i8 ? "int32_t" : "float")
    << " acc, int64_t m, int64_t n, const row_t& R, const col_t& Cv, const args_t& P) {\n";
  for (size_t i = 0; i < A.params.size(); ++i)
    if (A.params[i].role == "scalar") k << "    const uint64_t s" << i << " = P.s" << i << ";\n";
  k << epi.str() << "    return (out_t)" << name[outv] << ";\n  }\n};\n}\n";
  k << "extern \"C\" __global__ __launch_bounds__(" << threads << ") void " << kname << "(" << params << ") {\n"
    << "  " << kname << "_args P;\n";
  for (size_t i = 0; i < A.params.size(); ++i)
    k << "  P." << (A.params[i].role == "scalar" ? "s" : "p") << i << " = " << (A.params[i].role == "scalar" ? "s" : "p") << i << ";\n";
  const std::string et = i8 ? "int8_t" : "uint16_t";
  const std::string aPtr = preA ? "(const " + et + "*)((char*)ws + " + std::to_string(wsB) + ")" : "(const " + et + "*)p" + std::to_string(a->argIdx);
  const std::string bPtr = preB ? "(const " + et + "*)ws" : "(const " + et + "*)p" + std::to_string(b->argIdx);
  if (mxExact)
    k << "  hf::mmad<" << MK_BF16_CODE << ", " << kname << "_epi, false, false, 4>((const uint16_t*)ws, (const uint16_t*)((char*)ws + "
      << wsXA << "), (" << mtype(oe) << "*)" << resultPtr(A, 0) << ", " << Mx << ", " << N << "ll, " << K << "ll, P);\n}\n";
  else if (mx)
    k << "  hf::mmad_mx<" << mk << ", " << kname << "_epi>((const uint8_t*)p" << a->argIdx << ", (const uint8_t*)p" << b->argIdx
      << ", (const uint8_t*)p" << sa->argIdx << ", (const uint8_t*)p" << sb->argIdx << ", (" << mtype(oe) << "*)"
      << resultPtr(A, 0) << ", " << Mx << ", " << N << "ll, " << K << "ll, P);\n}\n";
  else
    k << "  hf::mmad<" << mk << ", " << kname << "_epi, " << (mT ? "true" : "false") << ", " << (kT ? "true" : "false") << ", "
      << dma << ">(" << aPtr << ", " << bPtr << ", (" << mtype(oe) << "*)" << resultPtr(A, 0) << ", " << Mx << ", " << N
      << "ll, " << K << "ll, P);\n}\n";
  // the re-layout kernels: [K, X] -> [X, K], 128 x 128-byte tiles
  auto preKernel = [&](const char *suffix, const Value *src, int64_t X, uint64_t off) {
    KernelPlan::PreKernel pk;
    pk.name = kname + suffix;
    const int64_t T = 128 / esz; // tile edge in elements (128 bytes)
    pk.grid = (unsigned)(((K + T - 1) / T) * ((X + T - 1) / T));
    pk.block = 256;
    pk.kargs = {"param:" + std::to_string(src->argIdx), "ws"};
    k << "extern \"C\" __global__ __launch_bounds__(256) void " << pk.name << "(const void* __restrict__ src, void* __restrict__ ws) {\n"
      << "  hf::mm_transpose<" << esz << ">((const char*)src, (char*)ws + " << off << ", " << K << "ll, " << X << "ll);\n}\n";
    p.pre.push_back(pk);
  };
  if (preB) preKernel("_relayout_b", b, N, 0);
  if (preA) preKernel("_relayout_a", a, M, wsB);
  p.workspaceBytes = wsB + wsA;
  if (mxExact) {
    auto mxPre = [&](const char *suffix, const Value *src, const Value *scl, int fmt, bool rowScale, int64_t R, int64_t Cc,
                     uint64_t off) {
      KernelPlan::PreKernel pk;
      pk.name = kname + suffix;
      pk.grid = (unsigned)std::min<int64_t>(((rowScale ? R * Cc / 8 : R / 8 * (Cc / 8)) + 255) / 256, 8192);
      pk.block = 256;
      pk.kargs = {"param:" + std::to_string(src->argIdx), "param:" + std::to_string(scl->argIdx), "ws"};
      k << "extern \"C\" __global__ __launch_bounds__(256) void " << pk.name
        << "(const void* __restrict__ src, const void* __restrict__ sc, void* __restrict__ ws) {\n"
        << "  hf::mx_to_bf16<" << fmt << ", " << (rowScale ? "true" : "false") << ">((const uint8_t*)src, (const uint8_t*)sc, "
        << "(uint16_t*)((char*)ws + " << off << "), " << R << "ll, " << Cc << "ll, " << K << "ll);\n}\n";
      p.pre.push_back(pk);
    };
    mxPre("_mx_a", a, sa, (mk - 3) / 2, true, M, K, 0);
    mxPre("_mx_b", b, sb, (mk - 3) % 2, false, K, N, wsXA);
    p.workspaceBytes = wsXA + wsXB;
  }
  p.source = k.str();
  // 256x256 macro-tiles, one workgroup each (XCD-aware order inside the kernel)
  const int64_t TM = 256, TN = 256;
  p.grid[0] = (unsigned)(((M + TM - 1) / TM) * ((N + TN - 1) / TN));
  if (A.rowsDyn) {
    // ceil(M / 256) row tiles of ceil(N / 256) tiles each
    p.rowsDyn = true;
    p.rowsA = 1;
    p.rowsB = TM;
    p.rowsC = (N + TN - 1) / TN;
  }
  p.block[0] = (unsigned)threads;
  static const char *mxName[5] = {"e4m3 x e4m3", "e4m3 x e5m2", "e5m2 x e4m3", "e5m2 x e5m2", "e2m1 x e2m1, fp4 two per byte"};
  p.variant = std::string(mxExact ? std::string("exact matmul_mx: ") + mxName[mk - 3] +
                                         " with e8m0 scales per 32 k, scaled into bf16 by pre kernels, mfma_f32_32x32x16_bf16"
                          : mx ? std::string("mfma_scale_f32_32x32x64_f8f6f4 (") + mxName[mk - 3] + ", e8m0 scales per 32 k)"
                          : mk == 0 ? "mfma_i32_32x32x32_i8" : mk == 1 ? "mfma_f32_32x32x16_bf16" : "mfma_f32_32x32x16_f16") +
              (aT ? ", A [K,M]" : "") + (bT ? ", B [N,K]" : ", B [K,N]") +
              (preA || preB ? " (re-laid K-contiguous by a transpose kernel)" : "") +
              (dma == 4 ? std::string(", LDS DMA ring (128-byte slices, 2 waves/SIMD; ") + (aT && bT ? "A" : aT ? "A and B" : "B") +
                              " k-rows staged whole, transposing LDS reads)" :
               dma == 3 ? ", LDS DMA ring (128-byte slices, 2 waves/SIMD)" : dma == 1 ? ", LDS DMA ring" : ", register staging");
  p.algoOps = 2.0 * (double)M * (double)N * (double)Kl;
  return p;
}

} // namespace

// ======================================================================
// Single-op kernels: cumulative ops, histogram, (de)interleave
// ======================================================================
bool isSingleOpKernel(const std::string &n) {
  return n == "hfusion.cumsum" || n == "hfusion.cumprod" || n == "hfusion.cummax" || n == "hfusion.cummin" ||
         n == "hfusion.histogram" || n == "hfusion.deinterleave" || n == "hfusion.interleave" || n == "hfusion.flip" ||
         n == "hfusion.mulext" || n == "hfusion.mulextui" || n == "hfusion.arange" || n == "hfusion.gather" || n == "hfusion.sort";
}

static std::vector<int64_t> intList(const std::string &s) {
  std::vector<int64_t> v;
  std::stringstream ss(s);
  std::string tok;
  while (std::getline(ss, tok, ',')) if (!tok.empty()) v.push_back(std::stoll(tok));
  return v;
}

static KernelPlan lowerSingleOp(Analysis &A, const std::string &kname, const Op *op) {
  Func &f = *A.f;
  for (const Op *o : f.ops)
    if (o != op && o->name != "tensor.empty" && o->name != "arith.constant" && o->name.rfind("arith.index", 0) != 0)
      unsupported(o, "op in a group with " + op->name);
  if (op->name == "hfusion.gather" || op->name == "hfusion.sort")
    for (const Value *v : op->ins)
      if (v->argIdx < 0) unsupported(op, "operand that is not a group argument");
  if (op->name != "hfusion.arange")
    for (const Value *v : op->operands)
      if (v->argIdx < 0) unsupported(op, "operand that is not a group argument");
  std::vector<std::string> outPtr(op->results.size());
  for (size_t i = 0; i < f.returns.size(); ++i) {
    const Value *v = f.returns[i];
    if (v->def != op) unsupported(op, "group returns a value other than the op's results");
    outPtr[v->resultIdx] = resultPtr(A, i);
  }
  for (auto &s : outPtr) if (s.empty()) unsupported(op, "a result the group does not return");
  auto inPtr = [&](size_t i) { return "p" + std::to_string(op->operands.at(i)->argIdx); };
  for (const Value *v : op->operands)
    if (v->type.tensor && v->type.shape.empty()) unsupported(op, "rank-0 operand");
  for (const Value *v : op->ins)
    if (v->type.tensor && v->type.shape.empty()) unsupported(op, "rank-0 operand");
  auto numel = [](const std::vector<int64_t> &sh) { int64_t n = 1; for (auto d : sh) n *= d; return n; };
  const std::string n = op->name.substr(std::string("hfusion.").size());
  KernelPlan p;
  p.kernelName = kname;
  std::ostringstream k;
  if (n == "cumsum" || n == "cumprod" || n == "cummax" || n == "cummin") {
    // CPU meaning (cumprod: ConvertHFusionToUpstream.cpp:385-450): along the
    // cumulation dim, in index order (reverse: from the end), acc_0 = x_0 and
    // acc_l = acc_{l-1} (op) x_l, each step rounded to the element type.
    const Value *x = op->operands.at(0);
    Elem ie = x->type.elem, oe = op->results[0]->type.elem;
    auto dims = intList(op->attr("cum_dims"));
    const auto &sh = x->type.shape;
    if (dims.size() != 1 || dims[0] < 0 || dims[0] >= (int64_t)sh.size()) unsupported(op, "one cumulation dim");
    if (ie != oe && !(n == "cumsum" && !isFloat(ie) && !isFloat(oe) && elemBits(oe) >= elemBits(ie)))
      unsupported(op, "result type differing from the input");
    int64_t d = dims[0], L = sh[d], outer = 1, inner = 1;
    for (int64_t i = 0; i < d; ++i) outer *= sh[i];
    for (size_t i = d + 1; i < sh.size(); ++i) inner *= sh[i];
    const bool rev = op->attr("reverse") == "true", nan = op->attr("propagate_nan", "true") != "false";
    std::string comb;
    if (isFloat(oe)) {
      std::string fn = n == "cumsum" ? "add" : n == "cumprod" ? "mul" : n == "cummax" ? (nan ? "maxf" : "maxnumf")
                                                                                      : (nan ? "minf" : "minnumf");
      comb = inFloatType(oe, {"acc", "xv"}, [&](const std::vector<std::string> &y) { return f32BinaryFn(fn, y[0], y[1], op); });
    } else {
      std::string fn = n == "cumsum" ? "add" : n == "cumprod" ? "mul" : n == "cummax" ? "max_signed" : "min_signed";
      comb = intBinaryFn(fn, "acc", "xv", oe, op);
    }
    const std::string IT = mtype(ie), OT = ctype(oe);
    k << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "(" << kernelParamList(A, p.kargs, false) << ") {\n"
      << "  constexpr int64_t OUTER = " << outer << "ll, L = " << L << "ll, INNER = " << inner << "ll;\n"
      << "  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;\n"
      << "  if (t >= OUTER * INNER) return;\n"
      << "  const int64_t o = t / INNER, i = t % INNER;\n"
      << "  const " << IT << " *src = (const " << IT << " *)" << inPtr(0) << " + o * L * INNER + i;\n"
      << "  " << OT << " *dst = (" << OT << " *)" << outPtr[0] << " + o * L * INNER + i;\n"
      << "  " << OT << " acc = 0;\n"
      << "  for (int64_t s = 0; s < L; ++s) {\n"
      << "    const int64_t l = " << (rev ? "L - 1 - s" : "s") << ";\n"
      << "    const " << OT << " xv = " << castExpr("(" + ctype(ie) + ")src[l * INNER]", ie, oe, false) << ";\n"
      << "    acc = s == 0 ? xv : (" << OT << ")(" << comb << ");\n"
      << "    dst[l * INNER] = acc;\n  }\n}\n";
    p.kind = "SCAN";
    p.variant = "one thread per line, " + std::string(rev ? "reverse" : "forward") + " serial order";
    p.grid[0] = (unsigned)std::max<int64_t>(1, (outer * inner + 255) / 256);
    p.block[0] = 256;
  } else if (n == "flip") {
    // reverse along flip_axis (HFusionOps.td:226-245: the last dimension)
    const Value *x = op->operands.at(0);
    const auto &sh = x->type.shape;
    int64_t ax = op->attrs.count("flip_axis") ? std::stoll(op->attr("flip_axis")) : (int64_t)sh.size() - 1;
    if (ax < 0) ax += (int64_t)sh.size();
    if (ax < 0 || ax >= (int64_t)sh.size()) unsupported(op, "flip_axis");
    if (op->results[0]->type.elem != x->type.elem) unsupported(op, "flip result type");
    int64_t L = sh[ax], outer = 1, inner = 1;
    for (int64_t i = 0; i < ax; ++i) outer *= sh[i];
    for (size_t i = ax + 1; i < sh.size(); ++i) inner *= sh[i];
    const std::string T = mtype(x->type.elem);
    k << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "(" << kernelParamList(A, p.kargs, false) << ") {\n"
      << "  constexpr int64_t L = " << L << "ll, INNER = " << inner << "ll, N = " << outer * L * inner << "ll;\n"
      << "  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;\n"
      << "  if (t >= N) return;\n"
      << "  const int64_t i = t % INNER, l = (t / INNER) % L, o = t / (INNER * L);\n"
      << "  ((" << T << " *)" << outPtr[0] << ")[t] = ((const " << T << " *)" << inPtr(0) << ")[(o * L + (L - 1 - l)) * INNER + i];\n}\n";
    p.kind = "FLIP";
    p.variant = "one thread per element";
    p.grid[0] = (unsigned)std::max<int64_t>(1, (outer * L * inner + 255) / 256);
    p.block[0] = 256;
  } else if (n == "mulext" || n == "mulextui") {
    // (2N)-bit product of sign- (mulext) or zero-extended (mulextui) operands,
    // low and high N-bit halves (HFusionOps.td:114-158)
    const Value *a0 = op->operands.at(0), *b0 = op->operands.at(1);
    Elem e = a0->type.elem;
    if (isFloat(e) || e == Elem::I1 || b0->type.elem != e || a0->type.shape != b0->type.shape) unsupported(op, "operands");
    const int bits = elemBits(e);
    const bool sgn = n == "mulext";
    const std::string T = ctype(e), U = "uint" + std::to_string(bits) + "_t";
    std::string lo, hi;
    if (bits == 64) {
      lo = "(" + T + ")((uint64_t)a * (uint64_t)b)";
      hi = sgn ? "(" + T + ")__mul64hi((long long)a, (long long)b)" : "(" + T + ")__umul64hi((unsigned long long)a, (unsigned long long)b)";
    } else {
      std::string pr = sgn ? "((int64_t)a * (int64_t)b)" : "(int64_t)((uint64_t)(" + U + ")a * (uint64_t)(" + U + ")b)";
      lo = "(" + T + ")" + pr;
      hi = "(" + T + ")(" + pr + " >> " + std::to_string(bits) + ")";
    }
    const int64_t N = numel(a0->type.shape);
    k << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "(" << kernelParamList(A, p.kargs, false) << ") {\n"
      << "  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;\n"
      << "  if (t >= " << N << "ll) return;\n"
      << "  const " << T << " a = ((const " << T << " *)" << inPtr(0) << ")[t], b = ((const " << T << " *)" << inPtr(1) << ")[t];\n";
    if (op->results.size() != 2) unsupported(op, "mulext without both results");
    k << "  ((" << T << " *)" << outPtr[0] << ")[t] = " << lo << ";\n"
      << "  ((" << T << " *)" << outPtr[1] << ")[t] = " << hi << ";\n}\n";
    p.kind = "MULEXT";
    p.variant = sgn ? "signed" : "unsigned";
    p.grid[0] = (unsigned)std::max<int64_t>(1, (N + 255) / 256);
    p.block[0] = 256;
  } else if (n == "arange") {
    // value at index (i0, i1, ...) = offset + sum_d stride_d * i_d
    // (HFusionStructuredOps.td:163-175), converted to the element type
    if (op->outs.size() != 1) unsupported(op, "arange without one outs");
    const Value *o = op->outs[0];
    const auto &sh = o->type.shape;
    const bool hasOff = op->attr("arange.offset") == "1";
    if (op->operands.size() != sh.size() + (hasOff ? 1 : 0)) unsupported(op, "arange needs one stride per dimension");
    auto idx = [&](const Value *v) -> std::string {
      if (v->isConst) return "(int64_t)" + std::to_string(v->iconst) + "ll";
      if (v->argIdx >= 0 && A.params[v->argIdx].role == "scalar") return "(int64_t)" + scalarArgExpr(A, v->argIdx);
      unsupported(op, "arange offset/stride that is not a constant or scalar argument");
    };
    std::string off = hasOff ? idx(op->operands[0]) : "(int64_t)0";
    std::ostringstream val;
    val << off;
    int64_t inner = 1;
    for (int d = (int)sh.size() - 1; d >= 0; --d) {
      val << " + " << idx(op->operands[(hasOff ? 1 : 0) + d]) << " * ((t / " << inner << "ll) % " << sh[d] << "ll)";
      inner *= sh[d];
    }
    Elem e = o->type.elem;
    const int64_t N = numel(sh);
    k << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "(" << kernelParamList(A, p.kargs, false) << ") {\n"
      << "  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;\n"
      << "  if (t >= " << N << "ll) return;\n"
      << "  const int64_t v = " << val.str() << ";\n"
      << "  ((" << mtype(e) << " *)" << outPtr[0] << ")[t] = " << castExpr("v", Elem::I64, e, false) << ";\n}\n";
    p.kind = "ARANGE";
    p.variant = "one thread per element";
    p.grid[0] = (unsigned)std::max<int64_t>(1, (N + 255) / 256);
    p.block[0] = 256;
  } else if (n == "gather") {
    // out[p] = src[p with the axis coordinate replaced by index[p]] when
    // 0 <= index[p] < src.shape[axis], else the init value (the loop of
    // HFusionStructuredOps.td:222-238 assigns only on a matching k)
    if (op->ins.size() != 2 || op->outs.size() != 1) unsupported(op, "gather operands");
    const Value *src = op->ins[0], *ix = op->ins[1], *init = op->outs[0];
    const auto &ss = src->type.shape, &is = ix->type.shape;
    const int64_t rank = (int64_t)is.size();
    int64_t ax = op->attrs.count("axis") ? std::stoll(op->attr("axis")) : rank - 1;
    if (ax < 0) ax += rank;
    if ((int64_t)ss.size() != rank || ax < 0 || ax >= rank || init->type.shape != is) unsupported(op, "gather shapes");
    for (int64_t d = 0; d < rank; ++d)
      if (d != ax && ss[d] != is[d]) unsupported(op, "gather shapes differing off the axis");
    if (isFloat(ix->type.elem) || ix->type.elem == Elem::I1) unsupported(op, "gather index type");
    const std::string T = mtype(src->type.elem);
    // strides of the index/output and of src
    std::vector<int64_t> istr(rank, 1), sstr(rank, 1);
    for (int64_t d = rank - 2; d >= 0; --d) { istr[d] = istr[d + 1] * is[d + 1]; sstr[d] = sstr[d + 1] * ss[d + 1]; }
    const int64_t N = numel(is);
    std::ostringstream sofs;
    sofs << "(int64_t)0";
    for (int64_t d = 0; d < rank; ++d) {
      if (d == ax) sofs << " + k * " << sstr[d] << "ll";
      else sofs << " + ((t / " << istr[d] << "ll) % " << is[d] << "ll) * " << sstr[d] << "ll";
    }
    // out-of-range positions keep the init: the outs argument when it is one,
    // else (a tensor.empty, whose contents are unspecified) the result buffer
    const std::string fallback = init->argIdx >= 0 ? "((const " + T + " *)p" + std::to_string(init->argIdx) + ")[t]"
                                                   : "((" + T + " *)" + outPtr[0] + ")[t]";
    k << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "(" << kernelParamList(A, p.kargs, false) << ") {\n"
      << "  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;\n"
      << "  if (t >= " << N << "ll) return;\n"
      << "  const int64_t k = (int64_t)((const " << mtype(ix->type.elem) << " *)p" << ix->argIdx << ")[t];\n"
      << "  const " << T << " v = (k >= 0 && k < " << ss[ax] << "ll) ? ((const " << T << " *)p" << src->argIdx << ")[" << sofs.str()
      << "] : " << fallback << ";\n"
      << "  ((" << T << " *)" << outPtr[0] << ")[t] = v;\n}\n";
    p.kind = "GATHER";
    p.variant = "one thread per output element";
    p.grid[0] = (unsigned)std::max<int64_t>(1, (N + 255) / 256);
    p.block[0] = 256;
  } else if (n == "sort") {
    // value sort along the last axis (HFusionOps.cpp:3341-3348 accepts only
    // the tail axis); the reference's bubble-sort decomposition
    // (DecomposeOpInterfaceImpl.cpp:740-830) handles one result only
    if (op->ins.size() != 1) unsupported(op, "sort without exactly one input");
    if (op->results.size() != 1) unsupported(op, "sort with an index result (the reference decomposes only the value sort)");
    const Value *x = op->ins[0];
    const Elem e = x->type.elem;
    if (op->results[0]->type.elem != e || op->results[0]->type.shape != x->type.shape)
      unsupported(op, "sort result type differing from the input");
    const auto &sh = x->type.shape;
    const int64_t rank = (int64_t)sh.size(), ax = std::stoll(op->attr("sort_axis", "-1"));
    if (ax != -1 && ax != rank - 1) unsupported(op, "sort along an axis other than the last");
    int kind;
    switch (e) {
    case Elem::F32: kind = 0; break;
    case Elem::F16: kind = 1; break;
    case Elem::BF16: kind = 2; break;
    case Elem::I8: kind = 8; break;
    case Elem::I16: kind = 16; break;
    case Elem::I32: kind = 32; break;
    default: unsupported(op, std::string("sort of ") + elemName(e) + " (f32, f16, bf16 and i8/i16/i32 are lowered)");
    }
    const int64_t L = sh.back(), R = numel(sh) / std::max<int64_t>(1, L);
    if (L > 16384) unsupported(op, "sort axis longer than 16384 (one row is sorted in LDS)");
    int64_t P = 1;
    while (P < L) P <<= 1;
    const int64_t rpw = P >= 2048 ? 1 : 2048 / P, E = rpw * P;
    const int nt = E <= 2048 ? 256 : 1024;
    const bool desc = op->attr("descending", "false") == "true";
    const std::string T = mtype(e);
    if (L <= 1) {
      k << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "(" << kernelParamList(A, p.kargs, false) << ") {\n"
        << "  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;\n"
        << "  if (t < " << R << "ll) ((" << T << " *)" << outPtr[0] << ")[t] = ((const " << T << " *)p" << x->argIdx << ")[t];\n}\n";
      p.variant = "copy (one element per row)";
      p.grid[0] = (unsigned)std::max<int64_t>(1, (R + 255) / 256);
      p.block[0] = 256;
    } else {
      k << "extern \"C\" __global__ __launch_bounds__(" << nt << ") void " << kname << "(" << kernelParamList(A, p.kargs, false)
        << ") {\n  hf::sort_rows<" << kind << ", " << (desc ? "true" : "false") << ", " << P << ", " << nt << ">((const " << T
        << " *)p" << x->argIdx << ", (" << T << " *)" << outPtr[0] << ", " << R << "ll, " << L << ");\n}\n";
      p.variant = "bitonic network, " + std::to_string(rpw) + " row(s) of " + std::to_string(P) +
                  " keys per workgroup in LDS, " + (desc ? "descending" : "ascending");
      p.grid[0] = (unsigned)std::max<int64_t>(1, (R + rpw - 1) / rpw);
      p.block[0] = (unsigned)nt;
    }
    p.kind = "SORT";
  } else if (n == "histogram") {
    const Value *x = op->operands.at(0);
    const Value *mk = op->operands.size() > 1 ? op->operands[1] : nullptr;
    if (op->literal.empty()) unsupported(op, "histogram without num_bins");
    const int64_t bins = std::stoll(op->literal);
    Elem ie = x->type.elem, oe = op->results[0]->type.elem;
    if (isFloat(ie) || ie == Elem::I1) unsupported(op, "histogram of a non-integer input");
    if (isFloat(oe) || oe == Elem::I1) unsupported(op, "histogram counts of a non-integer type");
    if (op->results[0]->type.shape.size() != 1 || op->results[0]->type.shape[0] != bins)
      unsupported(op, "histogram output must be [num_bins]");
    const int64_t N = numel(x->type.shape);
    const int ldsb = bins <= 8192 ? (int)bins : 0;
    const int64_t grid = std::max<int64_t>(1, std::min<int64_t>(1024, (N + 256 * 16 - 1) / (256 * 16)));
    const std::string MT = mk ? mtype(mk->type.elem) : "uint8_t";
    k << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "(" << kernelParamList(A, p.kargs, true) << ") {\n"
      << "  hf::histogram<256, " << ldsb << ", " << (mk ? "true" : "false") << ">((const " << mtype(ie) << " *)" << inPtr(0)
      << ", (const " << MT << " *)" << (mk ? inPtr(1) : "nullptr") << ", " << N << "ll, " << bins << "ll, (" << ctype(oe)
      << " *)" << outPtr[0] << ", (unsigned long long *)ws);\n}\n";
    p.kind = "HISTOGRAM";
    p.variant = ldsb ? "LDS bins, last-workgroup copy" : "global bins, last-workgroup copy";
    p.grid[0] = (unsigned)grid;
    p.block[0] = 256;
    p.workspaceBytes = (uint64_t)bins * 8 + 256;
    p.workspaceZeroInit = true;
  } else {
    // (de)interleave along the last dim (HFusionOps.td:160-220; CPU meaning of
    // deinterleave ConvertHFusionToUpstream.cpp:268-335: out[.., j] =
    // in[.., 2j + channel])
    const bool de = n == "deinterleave";
    const Value *x = op->operands.at(0);
    Elem e = x->type.elem;
    for (auto *v : op->operands) if (v->type.elem != e) unsupported(op, "operands of different types");
    for (auto *r : op->results) if (r->type.elem != e) unsupported(op, "result type differing from the input");
    const std::string T = mtype(e);
    int64_t R = 1, J;
    const auto &sh = x->type.shape;
    for (size_t i = 0; i + 1 < sh.size(); ++i) R *= sh[i];
    std::ostringstream body;
    if (de) {
      if (sh.back() % 2) unsupported(op, "deinterleave of an odd last dim");
      J = sh.back() / 2;
      int ch = op->angleKind == "all" ? -1 : (op->literal.empty() ? -1 : std::stoi(op->literal));
      if (ch < -1 || ch > 1) unsupported(op, "deinterleave channel");
      if ((ch == -1) != (op->results.size() == 2)) unsupported(op, "deinterleave result count for its channel");
      body << "  const " << T << " *src = (const " << T << " *)" << inPtr(0) << " + r * (2 * J) + 2 * j;\n";
      if (ch == -1)
        body << "  ((" << T << " *)" << outPtr[0] << ")[t] = src[0];\n  ((" << T << " *)" << outPtr[1] << ")[t] = src[1];\n";
      else
        body << "  ((" << T << " *)" << outPtr[0] << ")[t] = src[" << ch << "];\n";
      p.variant = "deinterleave channel " + std::string(ch == -1 ? "all" : std::to_string(ch));
    } else {
      if (op->operands.size() != 2) unsupported(op, "interleave of other than two tensors");
      if (op->operands[1]->type.shape != sh) unsupported(op, "interleave operands of different shapes");
      J = sh.back();
      body << "  " << T << " *dst = (" << T << " *)" << outPtr[0] << " + r * (2 * J) + 2 * j;\n"
           << "  dst[0] = ((const " << T << " *)" << inPtr(0) << ")[t];\n"
           << "  dst[1] = ((const " << T << " *)" << inPtr(1) << ")[t];\n";
      p.variant = "interleave";
    }
    k << "extern \"C\" __global__ __launch_bounds__(256) void " << kname << "(" << kernelParamList(A, p.kargs, false) << ") {\n"
      << "  constexpr int64_t R = " << R << "ll, J = " << J << "ll;\n"
      << "  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;\n"
      << "  if (t >= R * J) return;\n"
      << "  const int64_t r = t / J, j = t % J;\n  (void)r; (void)j;\n"
      << body.str() << "}\n";
    p.kind = de ? "DEINTERLEAVE" : "INTERLEAVE";
    p.grid[0] = (unsigned)std::max<int64_t>(1, (R * J + 255) / 256);
    p.block[0] = 256;
  }
  p.source = k.str();
  return p;
}

// A group of elementwise ops whose tensors are reshaped views of each other
// (tensor.expand_shape / collapse_shape of row-major data) and all hold the
// same number of elements: every tensor shares the flat element index, so the
// group runs over one flat dimension and the reshapes vanish.  The buffer
// descriptors (taken before this) keep the arguments' own shapes.
// A linalg.transpose that only moves unit dims keeps the row-major element
// order: it becomes a reshape view (as compile-pure-elemwise-with-foldable-
// transpose.mlir:5-12 has it, between an expand and a collapse).
static void foldTrivialTransposes(Func &f) {
  for (Op *op : f.ops) {
    if (op->name != "linalg.transpose") continue;
    std::vector<int64_t> perm = permutationOf(op);
    const auto &in = op->ins[0]->type.shape;
    std::vector<int64_t> order;
    for (auto d : perm) if (in[d] != 1) order.push_back(d);
    if (!std::is_sorted(order.begin(), order.end())) continue;
    Value *src = op->ins[0], *dst = op->outs[0];
    auto &du = dst->users;
    du.erase(std::remove(du.begin(), du.end(), op), du.end());
    op->name = "tensor.collapse_shape";
    op->operands = {src};
    op->ins.clear();
    op->outs.clear();
    if (op->results.empty()) unsupported(op, "transpose without a result");
  }
}

static void flattenReshapeGroup(Func &f) {
  bool anyReshape = false;
  int64_t n = -1;
  auto numelOf = [](const Type &t) { int64_t k = 1; for (auto d : t.shape) k *= d; return k; };
  auto same = [&](const Value *v) {
    if (!v->type.tensor) return true;
    int64_t k = numelOf(v->type);
    if (n < 0) n = k;
    return k == n;
  };
  for (const Op *op : f.ops) {
    const std::string &nm = op->name;
    const bool reshape = nm == "tensor.expand_shape" || nm == "tensor.collapse_shape";
    anyReshape |= reshape;
    // (a linalg.generic's maps name the dims of its own rank: not flattened)
    if (!reshape && (!isElementwiseOp(op) || nm == "linalg.generic") && nm != "tensor.empty" &&
        nm != "arith.constant" && nm != "linalg.fill")
      return;
    for (auto *lst : {&op->ins, &op->outs, &op->operands, &op->results})
      for (const Value *v : *lst) if (!same(v)) return;
  }
  for (const Value *v : f.args) if (!same(v)) return;
  if (!anyReshape || n <= 0) return;
  for (size_t i = 0; i < f.ops.size();) {
    Op *op = f.ops[i];
    if (op->name != "tensor.expand_shape" && op->name != "tensor.collapse_shape") { ++i; continue; }
    Value *src = op->operands.at(0), *dst = op->results.at(0);
    auto &su = src->users;
    su.erase(std::remove(su.begin(), su.end(), op), su.end());
    for (Op *u : dst->users) {
      for (auto *lst : {&u->ins, &u->outs, &u->operands})
        for (Value *&v : *lst) if (v == dst) v = src;
      su.push_back(u);
    }
    for (Value *&r : f.returns) if (r == dst) r = src;
    f.ops.erase(f.ops.begin() + i);
  }
  auto flat = [&](Value *v) { if (v->type.tensor) v->type.shape = {n}; };
  for (Value *v : f.args) flat(v);
  for (Op *op : f.ops)
    for (auto *lst : {&op->ins, &op->outs, &op->operands, &op->results})
      for (Value *v : *lst) flat(v);
}

// Reshapes (tensor.expand_shape / collapse_shape) inside a group that also
// broadcasts or reduces.  A reshape of row-major data keeps the element
// order, so it is a view; what it changes is which dims the reduce and
// broadcast ops name.  The full-size tensors' shapes are refined to one
// common factorisation, the union of their dim boundaries (which must nest:
// [24,512,16,12] and [24,512,192] refine to [24,512,16,12]).  Every tensor
// is re-typed onto the fine dims it spans (unit dims dropped), the
// `dimensions` of reduce and broadcast ops are rewritten on those dims, and
// the reshapes vanish; the normal domain inference and collapsing follow.
// The reference admits reshapes into LAST_AXIS_PBR, ANY_PBR and ANY_PB
// groups (bishengir/lib/Dialect/HFusion/Transforms/OpFusion/
// FusibleHelper.cpp:617-629); its model-derived group
// bishengir/test/Dialect/HFusion/hfusion-pipeline.mlir:56-125 collapses
// [24,512,16,12] to [24,512,192] before row sums and expands [24,512] to
// [24,512,1,1] after them.
static void resolveReshapes(Func &f) {
  auto isReshape = [](const Op *op) { return op->name == "tensor.expand_shape" || op->name == "tensor.collapse_shape"; };
  bool any = false;
  for (const Op *op : f.ops) any |= isReshape(op);
  if (!any) return;
  for (const Op *op : f.ops)
    if (op->name == "linalg.transpose" || op->name == "linalg.generic")
      unsupported(op, "a reshape beside a transpose or linalg.generic in a reducing or broadcasting group");
  std::vector<Value *> vals;
  std::set<const Value *> seen;
  auto add = [&](Value *v) { if (v->type.tensor && seen.insert(v).second) vals.push_back(v); };
  for (Value *a : f.args) add(a);
  for (Op *op : f.ops)
    for (auto *lst : {&op->ins, &op->outs, &op->operands, &op->results})
      for (Value *v : *lst) add(v);
  int64_t N = 1;
  for (const Value *v : vals) N = std::max(N, v->type.numel());
  // fine dims, outermost first: the ratios of consecutive suffix products
  std::set<int64_t> cuts;
  for (const Value *v : vals) {
    if (v->type.numel() != N) continue;
    int64_t s = 1;
    for (size_t i = v->type.shape.size(); i-- > 0;) {
      s *= v->type.shape[i];
      if (s > 1) cuts.insert(s);
    }
  }
  std::vector<int64_t> F;
  int64_t prev = 1;
  for (int64_t c : cuts) {
    if (c % prev) throw CompileError("unsupported: reshapes whose dim boundaries do not nest (" + std::to_string(prev) + " and " + std::to_string(c) + " elements)");
    F.insert(F.begin(), c / prev);
    prev = c;
  }
  using Layout = std::vector<std::vector<int>>; // fine dims spanned by each tensor dim
  auto flat = [](const Layout &L) {
    std::vector<int> o;
    for (auto &g : L) o.insert(o.end(), g.begin(), g.end());
    return o;
  };
  // the fine dims `fl` cut into consecutive runs of the sizes `shape`
  auto split = [&](const std::vector<int> &fl, const std::vector<int64_t> &shape, Layout &out) {
    out.assign(shape.size(), {});
    size_t k = 0;
    for (size_t i = 0; i < shape.size(); ++i) {
      int64_t p = 1;
      while (p < shape[i] && k < fl.size()) { out[i].push_back(fl[k]); p *= F[fl[k]]; ++k; }
      if (p != shape[i]) return false;
    }
    return k == fl.size();
  };
  std::map<const Value *, Layout> lay;
  bool changed = false;
  auto set = [&](const Value *v, const Layout &L, const Op *op) {
    if (!v->type.tensor) return;
    auto it = lay.find(v);
    if (it != lay.end()) {
      if (it->second != L) unsupported(op, "a tensor placed on two different dims across reshapes");
      return;
    }
    if (L.size() != v->type.shape.size()) unsupported(op, "internal: layout rank");
    lay[v] = L;
    changed = true;
  };
  std::vector<int> all;
  for (size_t d = 0; d < F.size(); ++d) all.push_back((int)d);
  for (const Value *v : vals) {
    Layout L;
    if (v->type.numel() == 1) set(v, Layout(v->type.shape.size()), nullptr);
    else if (v->type.numel() == N && split(all, v->type.shape, L)) set(v, L, nullptr);
  }
  auto minus = [](const Layout &L, const std::vector<int64_t> &dims) {
    Layout o;
    for (size_t i = 0; i < L.size(); ++i)
      if (std::find(dims.begin(), dims.end(), (int64_t)i) == dims.end()) o.push_back(L[i]);
    return o;
  };
  changed = true;
  while (changed) {
    changed = false;
    for (Op *op : f.ops) {
      const std::string &n = op->name;
      if (isReshape(op)) {
        const Value *src = op->operands.at(0), *dst = op->results.at(0);
        Layout L;
        if (lay.count(src) && !lay.count(dst)) {
          if (!split(flat(lay[src]), dst->type.shape, L))
            unsupported(op, "reshape splits a dim that the group's full-size tensors keep whole");
          set(dst, L, op);
        } else if (lay.count(dst) && !lay.count(src)) {
          if (!split(flat(lay[dst]), src->type.shape, L))
            unsupported(op, "reshape splits a dim that the group's full-size tensors keep whole");
          set(src, L, op);
        } else if (lay.count(src) && flat(lay[src]) != flat(lay[dst])) {
          unsupported(op, "reshape between tensors on different dims");
        }
        continue;
      }
      if (n == "linalg.broadcast") {
        const Value *o = op->results.empty() ? op->outs.at(0) : op->results[0];
        if (!lay.count(o) && lay.count(op->outs.at(0))) o = op->outs[0];
        if (!lay.count(o)) continue;
        const Layout Lo = lay[o];
        set(op->ins.at(0), minus(Lo, op->dims), op);
        set(op->outs[0], Lo, op);
        for (auto *v : op->results) set(v, Lo, op);
        continue;
      }
      if (n == "linalg.reduce" || n == "hfusion.reduce_with_index") {
        const Value *known = nullptr;
        for (auto *v : op->ins) if (lay.count(v)) known = v;
        if (!known) continue;
        const Layout Li = lay[known];
        for (auto *v : op->ins) set(v, Li, op);
        const Layout Lo = minus(Li, op->dims);
        for (auto *v : op->outs) set(v, Lo, op);
        for (auto *v : op->results) set(v, Lo, op);
        continue;
      }
      if (n == "linalg.fill" || isElementwiseOp(op)) {
        std::vector<const Value *> vs;
        for (auto *lst : {&op->ins, &op->operands, &op->outs, &op->results})
          for (auto *v : *lst) if (v->type.tensor && v->type.numel() != 1) vs.push_back(v);
        const Value *known = nullptr;
        for (auto *v : vs) if (lay.count(v)) { known = v; break; }
        if (!known) continue;
        const Layout L = lay[known];
        for (auto *v : vs) if (v->type.shape == known->type.shape) set(v, L, op);
      }
    }
  }
  for (const Value *v : vals)
    if (!lay.count(v) && (!v->users.empty() || std::find(f.returns.begin(), f.returns.end(), v) != f.returns.end()))
      throw CompileError("unsupported: cannot place tensor " + v->name + " (" + v->type.str() + ") on the group's dims across its reshapes");
  // dims of reduce / broadcast ops on the fine shapes (they need the old layouts)
  for (Op *op : f.ops) {
    if (op->name == "linalg.reduce" || op->name == "hfusion.reduce_with_index") {
      const std::vector<int> fl = flat(lay.at(op->ins.at(0)));
      const Layout &Li = lay.at(op->ins[0]);
      std::vector<int64_t> nd;
      for (size_t k = 0; k < fl.size(); ++k)
        for (int64_t d : op->dims)
          if (d >= 0 && d < (int64_t)Li.size() && std::count(Li[d].begin(), Li[d].end(), fl[k])) nd.push_back((int64_t)k);
      if (nd.empty()) unsupported(op, "reduction over unit dimensions only");
      op->dims = nd;
    } else if (op->name == "linalg.broadcast") {
      const Value *o = op->results.empty() ? op->outs.at(0) : op->results[0];
      const std::vector<int> fo = flat(lay.at(o)), fi = flat(lay.at(op->ins.at(0)));
      std::vector<int64_t> nd;
      for (size_t k = 0; k < fo.size(); ++k)
        if (std::find(fi.begin(), fi.end(), fo[k]) == fi.end()) nd.push_back((int64_t)k);
      op->dims = nd;
    }
  }
  // the reshapes become aliases of their sources
  for (size_t i = 0; i < f.ops.size();) {
    Op *op = f.ops[i];
    if (!isReshape(op)) { ++i; continue; }
    Value *src = op->operands.at(0), *dst = op->results.at(0);
    auto &su = src->users;
    su.erase(std::remove(su.begin(), su.end(), op), su.end());
    for (Op *u : dst->users) {
      for (auto *lst : {&u->ins, &u->outs, &u->operands})
        for (Value *&v : *lst) if (v == dst) v = src;
      su.push_back(u);
    }
    for (Value *&r : f.returns) if (r == dst) r = src;
    f.ops.erase(f.ops.begin() + i);
  }
  for (const auto &kv : lay) {
    Value *v = const_cast<Value *>(kv.first);
    std::vector<int64_t> s;
    for (int d : flat(kv.second)) s.push_back(F[d]);
    v->type.shape = s;
  }
}

// linalg.generic with a reduction over the last loop dim whose region ends
// in `%y = <combine> %v, %out` (or `%out, %v`), %out read nowhere else:
// rewritten as an elementwise linalg.generic computing %v over the full loop
// domain, then linalg.reduce with that combiner into the original outs.  The
// row programs then schedule it like any row reduction.
static void splitGenericReductions(Module &m, Func &f) {
  static const std::map<std::string, std::string> comb = {
      {"arith.addf", "arith.addf"}, {"arith.mulf", "arith.mulf"}, {"arith.maximumf", "arith.maximumf"},
      {"arith.minimumf", "arith.minimumf"}, {"arith.maxnumf", "arith.maxnumf"}, {"arith.minnumf", "arith.minnumf"},
      {"arith.addi", "arith.addi"}, {"arith.muli", "arith.muli"}, {"arith.maxsi", "arith.maxsi"},
      {"arith.minsi", "arith.minsi"}, {"arith.andi", "arith.andi"}, {"arith.ori", "arith.ori"},
      {"arith.xori", "arith.xori"}};
  for (size_t oi = 0; oi < f.ops.size(); ++oi) {
    Op *g = f.ops[oi];
    if (g->name != "linalg.generic" || g->attr("iterator_types").find("reduction") == std::string::npos) continue;
    if (g->outs.size() != 1 || g->results.size() != 1) continue;
    std::vector<std::vector<int>> maps;
    int nd = 0;
    if (!genericMaps(g, maps, nd) || nd < 1) continue;
    // reduction over exactly the last loop dim; outs indexed by d0..d(nd-2)
    std::vector<std::string> it;
    {
      std::string its = g->attr("iterator_types");
      for (size_t q = 0; q < its.size();) {
        size_t p = its.find_first_of("pr", q);
        if (p == std::string::npos) break;
        if (its.compare(p, 8, "parallel") == 0) { it.push_back("parallel"); q = p + 8; }
        else if (its.compare(p, 9, "reduction") == 0) { it.push_back("reduction"); q = p + 9; }
        else q = p + 1;
      }
    }
    if ((int)it.size() != nd || it.back() != "reduction") continue;
    bool ok = true;
    for (int i = 0; i + 1 < nd; ++i) ok &= it[i] == "parallel";
    const auto &om = maps.back();
    ok &= (int)om.size() == nd - 1;
    for (int i = 0; ok && i < nd - 1; ++i) ok = om[i] == i;
    if (!ok) continue;
    int64_t L = -1;
    for (size_t i = 0; i < g->ins.size(); ++i)
      for (size_t ax = 0; ax < maps[i].size(); ++ax)
        if (maps[i][ax] == nd - 1 && g->ins[i]->type.tensor) L = g->ins[i]->type.shape[ax];
    if (L < 0) continue;
    // the region: header, statements, yield
    const std::string region = g->attr("region");
    const size_t hp = region.find(')'), colon = region.find(':', hp);
    if (hp == std::string::npos || colon == std::string::npos) continue;
    std::string header = region.substr(0, colon + 1);
    std::vector<std::string> lines;
    {
      std::stringstream ss(region.substr(colon + 1));
      std::string ln;
      while (std::getline(ss, ln)) {
        const size_t b0 = ln.find_first_not_of(" \t");
        if (b0 != std::string::npos) lines.push_back(ln.substr(b0));
      }
    }
    // block argument names; the last one is %out
    std::vector<std::string> bnames;
    {
      const size_t lp = header.find('(');
      std::stringstream ss(header.substr(lp + 1, hp - lp - 1));
      std::string arg;
      while (std::getline(ss, arg, ',')) {
        std::string nm = arg.substr(0, arg.find(':'));
        nm.erase(std::remove_if(nm.begin(), nm.end(), ::isspace), nm.end());
        bnames.push_back(nm);
      }
    }
    if (bnames.size() != g->ins.size() + 1 || lines.empty() || lines.back().rfind("linalg.yield", 0) != 0) continue;
    const std::string outArg = bnames.back();
    auto valueNames = [](const std::string &t) {
      std::vector<std::string> v;
      for (size_t q = 0; (q = t.find('%', q)) != std::string::npos;) {
        size_t e = q + 1;
        while (e < t.size() && (std::isalnum((unsigned char)t[e]) || t[e] == '_' || t[e] == '.' || t[e] == '#')) ++e;
        v.push_back(t.substr(q, e - q));
        q = e;
      }
      return v;
    };
    const auto yv = valueNames(lines.back());
    if (yv.size() != 1) continue;
    int si = -1;
    for (int i = 0; i + 1 < (int)lines.size(); ++i)
      if (lines[i].rfind(yv[0] + " ", 0) == 0 || lines[i].rfind(yv[0] + "=", 0) == 0) si = i;
    if (si < 0) continue;
    const std::string &S = lines[si];
    const size_t eq = S.find('=');
    std::string rest = S.substr(eq + 1);
    rest.erase(0, rest.find_first_not_of(" \t"));
    const std::string opn = rest.substr(0, rest.find_first_of(" \t"));
    if (!comb.count(opn)) continue;
    const auto sv = valueNames(S);
    if (sv.size() != 3) continue;
    std::string v;
    if (sv[1] == outArg && sv[2] != outArg) v = sv[2];
    else if (sv[2] == outArg && sv[1] != outArg) v = sv[1];
    else continue;
    bool outElsewhere = false;
    for (int i = 0; i + 1 < (int)lines.size(); ++i)
      if (i != si) for (auto &nm : valueNames(lines[i])) outElsewhere |= nm == outArg;
    if (outElsewhere) continue;
    const std::string ty = S.substr(S.rfind(':') + 1);
    Elem vt;
    try { std::string t = ty; t.erase(std::remove_if(t.begin(), t.end(), ::isspace), t.end()); vt = parseElem(t); }
    catch (const CompileError &) { continue; }
    // build: %e = tensor.empty, %V = linalg.generic (elementwise), linalg.reduce
    Type full;
    full.tensor = true;
    full.elem = vt;
    full.shape = g->outs[0]->type.shape;
    full.shape.push_back(L);
    Op *empty = m.newOp();
    empty->name = "tensor.empty";
    Value *ev = m.newValue();
    ev->type = full;
    ev->def = empty;
    ev->name = g->results[0]->name + "#elem_init";
    empty->results.push_back(ev);
    Op *eg = m.newOp();
    eg->name = "linalg.generic";
    eg->line = g->line;
    eg->ins = g->ins;
    eg->insTypes = g->insTypes;
    eg->operands = g->operands;
    eg->outs = {ev};
    eg->attrs = g->attrs;
    // maps: the ins maps, then the identity over all nd loops
    std::string im = "[";
    for (size_t i = 0; i < g->ins.size(); ++i) {
      im += "affine_map<(";
      for (int d = 0; d < nd; ++d) im += (d ? ", d" : "d") + std::to_string(d);
      im += ") -> (";
      for (size_t k = 0; k < maps[i].size(); ++k) im += (k ? ", d" : "d") + std::to_string(maps[i][k]);
      im += ")>, ";
    }
    im += "affine_map<(";
    for (int d = 0; d < nd; ++d) im += (d ? ", d" : "d") + std::to_string(d);
    im += ") -> (";
    for (int d = 0; d < nd; ++d) im += (d ? ", d" : "d") + std::to_string(d);
    im += ")>]";
    eg->attrs["indexing_maps"] = im;
    eg->attrs["iterator_types"] = "[parallel]";
    std::string nr = header + "\n";
    for (int i = 0; i + 1 < (int)lines.size(); ++i)
      if (i != si) nr += "  " + lines[i] + "\n";
    nr += "  linalg.yield " + v + " : " + elemName(vt) + "\n";
    eg->attrs["region"] = nr;
    Value *vv = m.newValue();
    vv->type = full;
    vv->def = eg;
    vv->name = g->results[0]->name + "#elem";
    eg->results.push_back(vv);
    ev->users.push_back(eg);
    Op *rd = m.newOp();
    rd->name = "linalg.reduce";
    rd->line = g->line;
    rd->ins = {vv};
    rd->outs = g->outs;
    rd->dims = {nd - 1};
    rd->hasDims = true;
    rd->combiner = comb.at(opn);
    rd->results = g->results;
    for (Value *r : rd->results) r->def = rd;
    vv->users.push_back(rd);
    for (auto *lst : {&g->ins, &g->operands})
      for (Value *x : *lst) std::replace(x->users.begin(), x->users.end(), (Op *)g, eg);
    for (Value *x : g->outs) std::replace(x->users.begin(), x->users.end(), (Op *)g, rd);
    f.ops[oi] = rd;
    f.ops.insert(f.ops.begin() + oi, eg);
    f.ops.insert(f.ops.begin() + oi, empty);
    oi += 2;
  }
}

// ======================================================================
// Domain collapse.  Unit dims are dropped and adjacent dims that every
// tensor of the group treats alike (spans both, consecutively, or neither)
// merge into one, so a rank-N group becomes the smallest equivalent domain:
// a last-axis reduction over [B, S, H] becomes rows x H, a middle-axis one
// over [A, R, B] keeps three dims.  Value shapes and the `dimensions` of
// reduce / broadcast ops follow; buffer descriptors (taken before) keep the
// arguments' own shapes, and row-major buffers are unchanged by the merge.
// ======================================================================
bool collapseDomain(Analysis &A) {
  const std::vector<int64_t> D = A.D;
  const int r = (int)D.size();
  if (r == 0) return false;
  // indexing maps of generics and transposes are not rewritten: such groups
  // keep their domain
  for (const Op *op : A.f->ops)
    if (op->name == "linalg.generic" || op->name == "linalg.transpose") return false;
  auto nonUnit = [&](const std::vector<int> &m) {
    std::vector<int> k;
    for (int x : m) if (D[x] != 1) k.push_back(x);
    return k;
  };
  std::vector<int> keep;
  for (int d = 0; d < r; ++d) if (D[d] != 1) keep.push_back(d);
  std::vector<int> grp(r, -1);
  int g = -1;
  for (size_t idx = 0; idx < keep.size(); ++idx) {
    const int d = keep[idx];
    bool merge = idx > 0;
    if (merge) {
      const int p = keep[idx - 1];
      for (auto &kv : A.map) {
        std::vector<int> mk = nonUnit(kv.second);
        auto ip = std::find(mk.begin(), mk.end(), p), id = std::find(mk.begin(), mk.end(), d);
        const bool hp = ip != mk.end(), hd = id != mk.end();
        if (hp != hd || (hp && id != ip + 1)) { merge = false; break; }
      }
    }
    if (!merge) ++g;
    grp[d] = g;
  }
  const int ng = g + 1;
  std::vector<int64_t> nD(std::max(ng, 1), 1);
  for (int d = 0; d < r; ++d) if (grp[d] >= 0) nD[grp[d]] *= D[d];
  auto newMap = [&](const std::vector<int> &m) {
    std::vector<int> out;
    for (int x : m) {
      if (D[x] == 1) continue;
      if (out.empty() || out.back() != grp[x]) out.push_back(grp[x]);
    }
    if (ng == 0 && !m.empty()) out.push_back(0);
    return out;
  };
  if (nD == D) return false;
  // op dims first (they need the old maps)
  for (Op *op : A.f->ops) {
    if (op->name == "linalg.reduce" || op->name == "hfusion.reduce_with_index") {
      if (op->ins.empty() || !A.map.count(op->ins[0])) continue;
      const auto &mi = A.map.at(op->ins[0]);
      std::vector<int> nm = newMap(mi);
      std::vector<int64_t> nd;
      for (int64_t pos : op->dims) {
        if (pos < 0 || pos >= (int64_t)mi.size()) unsupported(op, "reduction dimension out of range");
        int x = mi[pos];
        if (D[x] == 1) continue;
        int q = (int)(std::find(nm.begin(), nm.end(), grp[x]) - nm.begin());
        if (nd.empty() || nd.back() != q) nd.push_back(q);
      }
      if (nd.empty()) unsupported(op, "reduction over unit dimensions only");
      op->dims = nd;
    } else if (op->name == "linalg.broadcast") {
      if (op->results.empty() || !A.map.count(op->results[0]) || !A.map.count(op->ins[0])) continue;
      std::vector<int> no = newMap(A.map.at(op->results[0])), ni = newMap(A.map.at(op->ins[0]));
      std::vector<int64_t> nd;
      for (size_t q = 0; q < no.size(); ++q)
        if (std::find(ni.begin(), ni.end(), no[q]) == ni.end()) nd.push_back((int64_t)q);
      op->dims = nd;
    }
  }
  for (auto &kv : A.map) {
    Value *v = const_cast<Value *>(kv.first);
    kv.second = newMap(kv.second);
    std::vector<int64_t> s;
    for (int x : kv.second) s.push_back(nD[x]);
    v->type.shape = s;
  }
  A.D = nD;
  return true;
}

// ======================================================================
// Column programs (ANY_PBR): reductions over one (collapsed) dim k that is
// not the innermost one, reduce_with_index along any dim, and row groups
// whose broadcast layout the row programs do not take.  Each thread owns
// one point of the other dims and walks dim k in increasing order, so every
// fold runs in the CPU loop nest's order (linalg-to-loops visits the reduced
// index serially per output element); consecutive threads take consecutive
// points of the innermost kept dim, so each step's loads coalesce.  Values
// that vary along k are lambdas of r re-evaluated in each pass (inputs are
// re-read from memory rather than kept); values that do not are computed
// once per thread.  Replaces the Ascend ReduceRA / ReduceARA /
// ReduceRA_With_Index templates
// (bishengir/lib/Template/lib/Vector/Reduction/ReduceRA.cpp, ReduceARA.cpp,
// ReduceRA_With_Index.cpp); kind inference "other reduce -> ANY_PBR" is
// FusibleHelper.cpp:63-64.
// ======================================================================
struct ColumnEmitter {
  Analysis &A;
  int K = -1; // the reduced dim of D
  std::ostringstream body;
  struct CV {
    std::string name;
    bool lazy = false; // a lambda of r
  };
  std::map<const Value *, CV> val;
  int tmp = 0;

  explicit ColumnEmitter(Analysis &a) : A(a) {}
  std::string fresh() { return "v" + std::to_string(tmp++); }

  // element strides of a tensor spanning D dims `m` (row-major)
  std::vector<int64_t> strides(const std::vector<int> &m) const {
    std::vector<int64_t> s(m.size(), 1);
    for (int i = (int)m.size() - 2; i >= 0; --i) s[i] = s[i + 1] * A.D[m[i + 1]];
    return s;
  }
  // flat offset of the thread's point (coordinate of K excluded) and the
  // stride along K
  std::pair<std::string, int64_t> offsetOf(const std::vector<int> &m) const {
    std::vector<int64_t> s = strides(m);
    std::string off;
    int64_t sk = 0;
    for (size_t i = 0; i < m.size(); ++i) {
      if (m[i] == K) { sk = s[i]; continue; }
      std::string t = "c" + std::to_string(m[i]) + " * " + std::to_string(s[i]) + "ll";
      off = off.empty() ? t : off + " + " + t;
    }
    return {off.empty() ? "0ll" : off, sk};
  }
  bool spansK(const Value *v) const {
    auto it = A.map.find(v);
    return it != A.map.end() && std::find(it->second.begin(), it->second.end(), K) != it->second.end();
  }
  std::string at(const Value *v, const std::string &r = "r") const {
    const CV &x = val.at(v);
    return x.lazy ? x.name + "(" + r + ")" : x.name;
  }

  void ensure(const Value *v) {
    if (val.count(v)) return;
    if (!v->type.tensor || v->isConst) {
      if (v->isConst) val[v] = {constExpr(v, v->type.elem), false};
      else if (v->argIdx >= 0) val[v] = {scalarArgExpr(A, v->argIdx), false};
      else throw CompileError("non-constant scalar " + v->name);
      return;
    }
    if (v->argIdx < 0) undefinedValue(v);
    const int i = v->argIdx;
    auto [off, sk] = offsetOf(A.map.at(v));
    std::string T = ctype(v->type.elem), M = mtype(v->type.elem);
    std::string nm = "in" + std::to_string(i);
    std::string P = "((const " + M + "*)p" + std::to_string(i) + ")";
    std::string cvt = v->type.elem == Elem::I1 ? " != 0" : "";
    if (spansK(v)) {
      body << "    const int64_t " << nm << "_o = " << off << ";\n"
           << "    auto " << nm << " = [&](int64_t r) -> " << T << " { return " << P << "[" << nm << "_o + r * " << sk << "ll]" << cvt
           << "; };\n";
      val[v] = {nm, true};
    } else {
      body << "    const " << T << " " << nm << " = " << P << "[" << off << "]" << cvt << ";\n";
      val[v] = {nm, false};
    }
  }

  std::string initOf(const Op *op, const Value *init, Elem t, const std::string &identity) {
    if (init->def && init->def->name == "linalg.fill") {
      const Value *c = init->def->ins[0];
      ensure(c);
      return c->isConst ? constExpr(c, t) : val[c].name;
    }
    if (init->argIdx >= 0) {
      ensure(init);
      if (val[init].lazy) unsupported(op, "reduction init varying along the reduced dim");
      return val[init].name;
    }
    if (init->isConst) return constExpr(init, t);
    if (init->def && init->def->name == "tensor.empty") return identity;
    unsupported(op, "reduction init must be a linalg.fill, an argument or tensor.empty");
  }

  void emitReduce(const Op *op, int64_t RK) {
    if (op->ins.size() != 1 || op->outs.size() != 1) unsupported(op, "multi-operand linalg.reduce");
    const Value *x = op->ins[0];
    ensure(x);
    Elem t = x->type.elem;
    Combiner cb = combinerFor(op, op->combiner, t);
    std::string T = ctype(t), nm = fresh();
    std::string init = initOf(op, op->outs[0], t, cb.identity);
    body << "    " << T << " " << nm << " = " << init << ";\n";
    if (val[x].lazy)
      body << "    for (int64_t r = 0; r < " << RK << "ll; ++r) " << nm << " = " << subst(cb.expr, at(x), nm) << ";\n";
    else // a value constant along the reduced dim still folds RK times
      body << "    for (int64_t r = 0; r < " << RK << "ll; ++r) " << nm << " = " << subst(cb.expr, val[x].name, nm) << ";\n";
    val[op->results[0]] = {nm, false};
  }

  // hfusion.reduce_with_index: the region of HFusionOps.cpp:1507-1653 folded
  // serially from the init: res = max/min(in, v); upd = res OGT/OLT v (sgt,
  // slt, ugt, ult for integers); i = upd ? index : i; v = res.
  void emitReduceWithIndex(const Op *op, int64_t RK) {
    if (op->ins.empty() || op->ins.size() > 2 || op->outs.size() != 2 || op->results.size() != 2)
      unsupported(op, "reduce_with_index operand form");
    const Value *x = op->ins[0];
    ensure(x);
    const Value *xi = op->ins.size() == 2 ? op->ins[1] : nullptr;
    if (xi) ensure(xi);
    Elem t = x->type.elem, it = op->outs[1]->type.elem;
    std::string kindS = op->angleKind.empty() ? op->attr("reduce_kind", "max") : op->angleKind;
    // bf16 / f16 fold in f32: the conversion is exact and monotone, and the
    // folded value is one of the inputs or the init, so it converts back exactly
    const bool narrow = t == Elem::BF16 || t == Elem::F16;
    std::string T = narrow ? "float" : ctype(t), IT = ctype(it);
    std::string fold, cmp;
    if (t == Elem::F32 || narrow) {
      if (kindS == "max") { fold = "hf::maximumf(X, V)"; cmp = "(R_ > V)"; }
      else if (kindS == "min") { fold = "hf::minimumf(X, V)"; cmp = "(R_ < V)"; }
      else unsupported(op, "reduce_with_index kind '" + kindS + "' on floats");
    } else if (isInt(t) && t != Elem::I1) {
      std::string UT = t == Elem::I8 ? "uint8_t" : t == Elem::I16 ? "uint16_t" : t == Elem::I32 ? "uint32_t" : "uint64_t";
      if (kindS == "max") { fold = "((X) > (V) ? (X) : (V))"; cmp = "(R_ > V)"; }
      else if (kindS == "min") { fold = "((X) < (V) ? (X) : (V))"; cmp = "(R_ < V)"; }
      else if (kindS == "max_unsigned" || kindS == "maxui") {
        fold = "((" + UT + ")(X) > (" + UT + ")(V) ? (X) : (V))"; cmp = "((" + UT + ")R_ > (" + UT + ")V)";
      } else if (kindS == "min_unsigned" || kindS == "minui") {
        fold = "((" + UT + ")(X) < (" + UT + ")(V) ? (X) : (V))"; cmp = "((" + UT + ")R_ < (" + UT + ")V)";
      } else unsupported(op, "reduce_with_index kind '" + kindS + "'");
    } else {
      unsupported(op, std::string("reduce_with_index over ") + elemName(t));
    }
    if (!isInt(it) || it == Elem::I1) unsupported(op, "reduce_with_index index type");
    auto repl = [](std::string e, const std::string &from, const std::string &to) {
      for (size_t p = e.find(from); p != std::string::npos; p = e.find(from, p + to.size())) e.replace(p, from.size(), to);
      return e;
    };
    std::string nv = fresh(), ni = fresh();
    const std::string init = initOf(op, op->outs[0], t, "0");
    body << "    " << T << " " << nv << " = " << (narrow ? castExpr(init, t, Elem::F32, false) : init) << ";\n"
         << "    " << IT << " " << ni << " = " << initOf(op, op->outs[1], it, "0") << ";\n"
         << "    for (int64_t r = 0; r < " << RK << "ll; ++r) {\n"
         << "      const " << T << " x_ = " << (narrow ? castExpr(at(x), t, Elem::F32, false) : at(x)) << ";\n"
         << "      const " << T << " R_ = " << repl(repl(fold, "X", "x_"), "V", nv) << ";\n"
         << "      if (" << repl(cmp, "V", nv) << ") " << ni << " = (" << IT << ")("
         << (xi ? at(xi) : std::string("r")) << ");\n"
         << "      " << nv << " = R_;\n    }\n";
    if (narrow) {
      const std::string nn = fresh();
      body << "    const " << ctype(t) << " " << nn << " = " << castExpr(nv, Elem::F32, t, false) << ";\n";
      nv = nn;
    }
    val[op->results[0]] = {nv, false};
    val[op->results[1]] = {ni, false};
  }

  void emitElementwise(const Op *op) {
    std::vector<const Value *> opsv;
    for (auto *v : op->ins) opsv.push_back(v);
    for (auto *v : op->operands) opsv.push_back(v);
    bool lazy = false;
    for (auto *v : opsv) { ensure(v); lazy |= val[v].lazy; }
    const Value *res = op->results[0];
    Elem U = res->type.elem;
    std::vector<Elem> at_;
    std::vector<std::string> args;
    for (auto *v : opsv) { at_.push_back(v->type.elem); args.push_back(at(v)); }
    std::string nm = fresh(), T = ctype(U);
    if (lazy)
      body << "    auto " << nm << " = [&](int64_t r) -> " << T << " { return " << elementExpr(op, args, at_, U) << "; };\n";
    else
      body << "    const " << T << " " << nm << " = " << elementExpr(op, args, at_, U) << ";\n";
    val[res] = {nm, lazy};
  }

  KernelPlan run(const std::string &kname, const std::string &kind) {
    Func &f = *A.f;
    const int n = (int)A.D.size();
    // the reduced dim: the one every reduction folds
    for (const Op *op : f.ops) {
      if (op->name != "linalg.reduce" && op->name != "hfusion.reduce_with_index") continue;
      if (!A.map.count(op->ins[0])) unsupported(op, "reduction input outside the group's domain");
      const auto &mi = A.map.at(op->ins[0]);
      if (op->dims.size() != 1) unsupported(op, "reduction over non-adjacent dimensions");
      int d = mi.at(op->dims[0]);
      if (K >= 0 && K != d) unsupported(op, "reductions over different dimensions in one group");
      K = d;
    }
    if (K < 0) throw CompileError("internal: column program without a reduction");
    const int64_t RK = A.D[K];
    // thread -> point of the other dims (innermost kept dim fastest)
    int64_t P = 1;
    for (int d = 0; d < n; ++d) if (d != K) P *= A.D[d];
    std::ostringstream coords;
    coords << "    int64_t t_ = pt; (void)t_;\n";
    for (int d = n - 1; d >= 0; --d) {
      if (d == K) continue;
      coords << "    const int64_t c" << d << " = t_ % " << A.D[d] << "ll; t_ /= " << A.D[d] << "ll; (void)c" << d << ";\n";
    }
    body << coords.str();
    for (Op *op : f.ops) {
      const std::string &nmo = op->name;
      if (nmo == "tensor.empty" || nmo == "arith.constant" || nmo == "tensor.dim" ||
          (nmo.rfind("arith.", 0) == 0 && !op->results.empty() && !op->results[0]->type.tensor))
        continue;
      if (nmo == "linalg.fill") {
        ensure(op->ins[0]);
        val[op->results[0]] = val[op->ins[0]];
        continue;
      }
      if (nmo == "linalg.broadcast") {
        ensure(op->ins[0]);
        val[op->results[0]] = val[op->ins[0]];
        continue;
      }
      if (nmo == "linalg.transpose") {
        // the same function of the point: the operand's map holds the permutation
        ensure(op->ins[0]);
        val[op->results.at(0)] = val[op->ins[0]];
        continue;
      }
      if (nmo == "linalg.reduce") { emitReduce(op, RK); continue; }
      if (nmo == "hfusion.reduce_with_index") { emitReduceWithIndex(op, RK); continue; }
      if (!isElementwiseOp(op)) unsupported(op, "op in a reduction group");
      emitElementwise(op);
    }
    for (size_t i = 0; i < f.returns.size(); ++i) {
      const Value *v = f.returns[i];
      if (v->argIdx >= 0 && A.resultTied[i] == v->argIdx) continue;
      ensure(v);
      if (!A.map.count(v)) throw CompileError("cannot place result " + v->name + " in the group's domain");
      auto [off, sk] = offsetOf(A.map.at(v));
      Elem e = v->type.elem;
      std::string M = mtype(e), ptr = "((" + M + "*)" + resultPtr(A, i) + ")";
      if (spansK(v))
        body << "    for (int64_t r = 0; r < " << RK << "ll; ++r) " << ptr << "[" << off << " + r * " << sk << "ll] = (" << M << ")("
             << at(v) << ");\n";
      else
        body << "    " << ptr << "[" << off << "] = (" << M << ")(" << at(v) << ");\n";
    }
    KernelPlan p;
    p.kernelName = kname;
    p.kind = kind;
    p.variant = "column program, serial along dim " + std::to_string(K) + " of " + std::to_string(n);
    const int block = 256;
    std::ostringstream k;
    k << "extern \"C\" __global__ __launch_bounds__(" << block << ") void " << kname << "(" << kernelParamList(A, p.kargs, false)
      << ") {\n"
      << "  for (int64_t pt = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; pt < " << P
      << "ll; pt += (int64_t)gridDim.x * blockDim.x) {\n"
      << body.str() << "  }\n}\n";
    p.source = k.str();
    int64_t grid = (P + block - 1) / block;
    p.grid[0] = (unsigned)std::max<int64_t>(1, std::min<int64_t>(grid, 1 << 20));
    p.block[0] = block;
    return p;
  }
};

// ======================================================================
// RMSNorm + dynamic int8 quantisation (hf_rmsq.h).  The group's ops are
// matched one by one, in the order and form of the configs' IR
// (compile-rms-norm-fp32-split-n.mlir:5-47 followed by the quantisation):
// any deviation leaves the group to the generic row program.
// ======================================================================
struct RmsqMatch {
  int x = -1, gamma = -1; // argument positions
  size_t qRes = 0, sRes = 0;
  double s0 = 0, K = 0, eps = 0, a0 = 0, qd = 0;
  int lo = 0, hi = 0;
};

const Op *defOp(const Value *v) { return v ? v->def : nullptr; }
bool isFun(const Op *op, std::initializer_list<const char *> names, const char *fn) {
  if (!op) return false;
  bool nm = false;
  for (const char *n : names) nm |= op->name == n;
  return nm && op->attr("fun") == fn && op->attr("cast").empty();
}
bool binOp(const Op *op, const char *fn) {
  return isFun(op, {"linalg.elemwise_binary", "hfusion.elemwise_binary"}, fn) && op->ins.size() == 2;
}
bool unOp(const Op *op, const char *fn) {
  return isFun(op, {"linalg.elemwise_unary", "hfusion.elemwise_unary"}, fn) && op->ins.size() == 1;
}
bool constF32(const Value *v, double &out) {
  if (!v || !v->isConst || v->type.tensor || v->type.elem != Elem::F32) return false;
  out = v->fconst;
  return std::isfinite(out);
}
// value = broadcast of `src` along `dims`
const Value *broadcastOf(const Value *v, std::vector<int64_t> dims) {
  const Op *b = defOp(v);
  if (!b || b->name != "linalg.broadcast" || b->dims != dims || b->ins.size() != 1) return nullptr;
  return b->ins[0];
}
// exact widening cast of a bf16 group argument to f32
int bf16ArgCast(const Value *v) {
  const Op *c = defOp(v);
  if (!c || c->name != "hfusion.cast" || c->ins.size() != 1 || v->type.elem != Elem::F32) return -1;
  const Value *a = c->ins[0];
  if (a->argIdx < 0 || a->type.elem != Elem::BF16) return -1;
  return a->argIdx;
}
// linalg.reduce <combiner> over dim 1 with init fill(constant)
const Value *reduceOf(const Value *v, const char *comb, double &init) {
  const Op *r = defOp(v);
  if (!r || r->name != "linalg.reduce" || r->combiner != comb || r->dims != std::vector<int64_t>{1} || r->ins.size() != 1)
    return nullptr;
  const Op *f = defOp(r->outs[0]);
  if (!f || f->name != "linalg.fill" || !constF32(f->ins[0], init)) return nullptr;
  return r->ins[0];
}

bool matchRmsQuant(const Analysis &A, RmsqMatch &m) {
  const Func &f = *A.f;
  if (A.D.size() != 2 || f.returns.size() != 2) return false;
  const int64_t C = A.D[1];
  if (C != 1024 && C != 2048 && C != 4096) return false;
  for (size_t i = 0; i < 2; ++i) {
    if (f.returns[i]->type.elem == Elem::I8) m.qRes = i;
    else m.sRes = i;
  }
  if (m.qRes == m.sRes) return false;
  const Value *qv = f.returns[m.qRes], *sc = f.returns[m.sRes];
  if (A.resultTied[m.qRes] < 0 || sc->type.elem != Elem::F32 || qv->type.shape != A.D ||
      sc->type.shape != std::vector<int64_t>{A.D[0]})
    return false;
  // q = cast_i8(maxf(minf(nearbyint(y / bcast(sc)), HI), LO))
  const Op *cq = defOp(qv);
  if (!cq || cq->name != "hfusion.cast" || cq->attr("round_mode", "rint") != "rint" || cq->ins.size() != 1 ||
      cq->attr("cast") == "cast_unsigned")
    return false;
  const Op *mx = defOp(cq->ins[0]);
  double lo, hi;
  if (!binOp(mx, "maxf") || !constF32(mx->ins[1], lo)) return false;
  const Op *mn = defOp(mx->ins[0]);
  if (!binOp(mn, "minf") || !constF32(mn->ins[1], hi)) return false;
  if (lo != std::floor(lo) || hi != std::floor(hi) || lo < -128 || hi > 127 || lo > hi) return false;
  const Op *rn = defOp(mn->ins[0]);
  if (!unOp(rn, "nearbyint")) return false;
  const Op *dv = defOp(rn->ins[0]);
  if (!binOp(dv, "div") || broadcastOf(dv->ins[1], {1}) != sc) return false;
  const Value *y = dv->ins[0];
  // sc = amax / QD; amax = reduce maximumf |y| from a0
  const Op *sd = defOp(sc);
  if (!binOp(sd, "div") || !constF32(sd->ins[1], m.qd)) return false;
  const Value *ay = reduceOf(sd->ins[0], "arith.maximumf", m.a0);
  if (!ay || !unOp(defOp(ay), "abs") || defOp(ay)->ins[0] != y) return false;
  // y = (xf * bcast(inv)) * bcast(gammaf)
  const Op *ym = defOp(y);
  if (!binOp(ym, "mul")) return false;
  const Value *gf = broadcastOf(ym->ins[1], {0});
  if (!gf || (m.gamma = bf16ArgCast(gf)) < 0) return false;
  const Op *y1 = defOp(ym->ins[0]);
  if (!binOp(y1, "mul")) return false;
  const Value *xf = y1->ins[0];
  if ((m.x = bf16ArgCast(xf)) < 0) return false;
  // inv = rec(sqrt(ss / K + eps)); ss = reduce addf (xf * xf) from s0
  const Value *inv = broadcastOf(y1->ins[1], {1});
  const Op *rc = defOp(inv);
  if (!unOp(rc, "rec")) return false;
  const Op *sq = defOp(rc->ins[0]);
  if (!unOp(sq, "sqrt")) return false;
  const Op *ad = defOp(sq->ins[0]);
  if (!binOp(ad, "add") || !constF32(ad->ins[1], m.eps)) return false;
  const Op *md = defOp(ad->ins[0]);
  if (!binOp(md, "div") || !constF32(md->ins[1], m.K)) return false;
  const Value *x2 = reduceOf(md->ins[0], "arith.addf", m.s0);
  const Op *mul2 = defOp(x2);
  if (!x2 || !binOp(mul2, "mul") || mul2->ins[0] != xf || mul2->ins[1] != xf) return false;
  if (!(m.s0 >= 0)) return false;
  // the quotients y / (amax / QD) lie in [-QD, QD] (to a rounding): the clamps
  // must not bind there, and the biased codes must fit a byte
  if (!(m.qd > 0 && m.qd <= 127 && lo <= -m.qd && hi >= m.qd)) return false;
  m.lo = (int)lo;
  m.hi = (int)hi;
  return A.params[m.gamma].shape == std::vector<int64_t>{C} || A.map.at(f.args[m.gamma]) == std::vector<int>{1};
}

KernelPlan lowerRmsQuant(Analysis &A, const RmsqMatch &m, const std::string &kname) {
  const int64_t R = A.D[0], C = A.D[1];
  // one workgroup per CU: 12 waves, three per SIMD (the occupancy the
  // register budget allows); 12 row buffers and gamma fill 112 KB of LDS at
  // 4096 columns
  constexpr int WPB = 12;
  KernelPlan p;
  p.kernelName = kname;
  p.kind = "LAST_AXIS_PBR";
  p.variant = "rmsnorm-quant: one wave per row, binade-run exact serial sum";
  std::ostringstream k;
  k << "extern \"C\" __global__ __launch_bounds__(" << WPB * 64 << ") __attribute__((amdgpu_waves_per_eu(3))) void " << kname
    << "(" << kernelParamList(A, p.kargs, false) << ") {\n"
    << "  hf::rmsq_rows<" << C << ", " << m.lo << ", " << m.hi << ", " << WPB << ">((const uint16_t*)p" << m.x
    << ", (const uint16_t*)p" << m.gamma << ", (int8_t*)" << resultPtr(A, m.qRes) << ", (float*)" << resultPtr(A, m.sRes)
    << ", " << (A.rowsDyn ? std::string("hf_rows") : std::to_string(R) + "ll") << ", " << floatLit((float)m.s0) << ", "
    << floatLit((float)m.K) << ", " << floatLit((float)m.eps) << ", "
    << floatLit((float)m.a0) << ", " << floatLit((float)m.qd) << ");\n}\n";
  p.source = k.str();
  // a runtime row count keeps the full grid: waves past the last row exit
  if (A.rowsDyn) p.rowsDyn = true;
  p.grid[0] = (unsigned)(A.rowsDyn ? 256 : std::min<int64_t>(R, 256));
  p.block[0] = WPB * 64;
  return p;
}

// The chain-wave kernel for the pattern (hf_rmsn.h, option rmsn_kernel=1):
// the serial chain in a wave of its own, the product maxima reduced beside
// it, the quantisation from registers.
KernelPlan lowerRmsNorm(Analysis &A, const RmsqMatch &m, const std::string &kname) {
  const int64_t R = A.D[0], C = A.D[1];
  KernelPlan p;
  p.kernelName = kname;
  p.kind = "LAST_AXIS_PBR";
  p.variant = "rmsnorm-quant: serial-order fp32 sum in a chain wave, product maxima beside it";
  std::ostringstream k;
  k << "extern \"C\" __global__ __launch_bounds__(576) void " << kname << "(" << kernelParamList(A, p.kargs, false) << ") {\n"
    << "  hf::rmsn_rows<" << C << ", " << m.lo << ", " << m.hi << ">((const uint16_t*)p" << m.x << ", (const uint16_t*)p"
    << m.gamma << ", (int8_t*)" << resultPtr(A, m.qRes) << ", (float*)" << resultPtr(A, m.sRes) << ", " << R << "ll, "
    << floatLit((float)m.s0) << ", " << floatLit((float)m.K) << ", " << floatLit((float)m.eps) << ", "
    << floatLit((float)m.a0) << ", " << floatLit((float)m.qd) << ");\n}\n";
  p.source = k.str();
  p.grid[0] = (unsigned)((R + 31) / 32);
  p.block[0] = 576;
  return p;
}

// Every linalg.reduce of the group folds exactly the last dim of its input,
// which spans the whole domain.
bool reducesLastDimOnly(const Analysis &A) {
  const int last = (int)A.D.size() - 1;
  for (const Op *op : A.f->ops) {
    if (op->name == "hfusion.reduce_with_index") return false;
    if (op->name != "linalg.reduce") continue;
    if (op->ins.empty() || !A.map.count(op->ins[0])) return false;
    const auto &mi = A.map.at(op->ins[0]);
    if ((int)mi.size() != last + 1 || op->dims.size() != 1 || mi.at(op->dims[0]) != last) return false;
  }
  return true;
}

// A lone reduce_with_index (max/min, f32, no index input) over the last dim of
// a group argument: the split-row streaming kernel of hf_argmax.h.
bool isRowArgReduce(const Func &f) {
  const Op *rw = nullptr;
  for (const Op *op : f.ops) {
    const std::string &n = op->name;
    if (n == "tensor.empty" || n == "linalg.fill" || n == "arith.constant" || n == "tensor.dim") continue;
    if (n != "hfusion.reduce_with_index" || rw) return false;
    rw = op;
  }
  if (!rw || rw->ins.size() != 1 || rw->outs.size() != 2) return false;
  const Value *x = rw->ins[0];
  if (x->argIdx < 0 || x->type.elem != Elem::F32) return false;
  const int rank = (int)x->type.shape.size();
  if (rw->dims.size() != 1 || rw->dims[0] != rank - 1) return false;
  std::string k = rw->angleKind.empty() ? rw->attr("reduce_kind", "max") : rw->angleKind;
  Elem ie = rw->outs[1]->type.elem;
  return (k == "max" || k == "min") && (ie == Elem::I32 || ie == Elem::I64);
}

std::vector<KernelPlan> lowerModule(Module &m, const LowerOptions &opt) {
  std::vector<KernelPlan> out;
  bool anyEntry = false;
  for (auto &f : m.funcs) anyEntry |= f->isEntry();
  for (auto &fp : m.funcs) {
    Func &f = *fp;
    if (anyEntry && !f.isEntry()) continue;
    foldConstants(f);
    Analysis A;
    A.f = &f;
    // annotation.mark {overflow_mode = "saturate"} on a cast's result makes
    // that cast saturate (Normalize.cpp:4285-4301); the mark itself is dropped
    for (size_t i = 0; i < f.ops.size();) {
      Op *op = f.ops[i];
      if (op->name != "annotation.mark") { ++i; continue; }
      const std::string mode = op->attr("overflow_mode");
      for (Value *v : op->operands) {
        if (mode.find("saturate") != std::string::npos && v->def && v->def->name == "hfusion.cast")
          v->def->attrs["enable_saturate"] = "true";
        auto &u = v->users;
        u.erase(std::remove(u.begin(), u.end(), op), u.end());
      }
      f.ops.erase(f.ops.begin() + i);
    }
    // destination-style ops on memrefs (no SSA result): each write gives the
    // `outs` buffer a new value, later reads of the buffer see the latest
    // value, and with no `return` operands the last value of every written
    // argument is a group result tied to that argument
    {
      std::map<Value *, Value *> latest; // buffer (func argument) -> its current value
      std::vector<Value *> written;      // written arguments in first-write order
      const bool noReturns = f.returns.empty();
      for (Op *op : f.ops) {
        for (auto *lst : {&op->ins, &op->operands})
          for (Value *&v : *lst) {
            auto it = latest.find(v);
            if (it == latest.end()) continue;
            auto &u = v->users;
            u.erase(std::remove(u.begin(), u.end(), op), u.end());
            v = it->second;
            v->users.push_back(op);
          }
        if (!op->results.empty() || op->outs.empty()) continue;
        for (size_t j = 0; j < op->outs.size(); ++j) {
          Value *buf = op->outs[j];
          Value *r = m.newValue();
          r->type = buf->type;
          r->def = op;
          r->resultIdx = (int)j;
          r->name = buf->name + "#written";
          op->results.push_back(r);
          if (buf->argIdx >= 0) {
            if (!latest.count(buf)) written.push_back(buf);
            latest[buf] = r;
          }
        }
      }
      if (noReturns)
        for (Value *b : written) f.returns.push_back(latest[b]);
    }
    splitGenericReductions(m, f);
    // ui8 is read as raw bytes: only matmul_mx's e8m0 scales may be ui8
    for (const Op *op : f.ops) {
      if (op->name == "hfusion.matmul_mx" || op->name == "func.return") continue;
      for (const Value *v : op->ins)
        if (v->type.uns) unsupported(op, "ui8 operand outside matmul_mx scales");
      for (const Value *v : op->operands)
        if (v->type.uns) unsupported(op, "ui8 operand outside matmul_mx scales");
    }
    describeBuffers(A);
    if (opt.runtimeRows) {
      for (auto &b : A.params)
        for (auto d : b.shape) A.rowsDyn |= d == kRuntimeRows;
      for (auto &b : A.results)
        for (auto d : b.shape) A.rowsDyn |= d == kRuntimeRows;
    }
    std::string kname = "hf_" + f.name;
    KernelPlan p;
    const Op *single = findOp(f, [](const Op *o) { return isSingleOpKernel(o->name); });
    bool hasMM = false, hasRWI = false, hasRed = false;
    std::string kind = single ? "" : resultKind(f, &hasMM, &hasRWI, &hasRed);
    if (single) {
      p = lowerSingleOp(A, kname, single);
    } else if (kind == "SINGLE_CUBE") {
      p = lowerMatmul(A, kname, opt);
    } else if (kind == "REDUCE_WITH_INDEX" && isRowArgReduce(f)) {
      p = lowerReduceWithIndex(A, kname);
    } else {
      foldTrivialTransposes(f);
      flattenReshapeGroup(f);
      resolveReshapes(f);
      A.D = largestShape(f, {});
      if (A.D.empty()) {
        // rank-0 tensors only: one element
        bool anyTensor = false;
        for (const Value *v : f.args) anyTensor |= v->type.tensor;
        for (const Value *v : f.returns) anyTensor |= v->type.tensor;
        if (!anyTensor) throw CompileError("group @" + f.name + " has no tensor to iterate over");
      }
      inferMaps(A, {});
      if (kind == "LAST_AXIS_PBR" || kind == "REDUCE_WITH_INDEX") {
        // row programs take rank <= 2 groups reducing the last dim; a higher
        // rank collapses first; anything else is a column program
        // (a transposed operand: the column program, which indexes every
        // tensor through its own map)
        bool rows = kind == "LAST_AXIS_PBR" && !findOp(f, [](const Op *o) { return o->name == "linalg.transpose"; });
        if (rows && (A.D.size() > 2 || !reducesLastDimOnly(A))) {
          collapseDomain(A);
          rows = A.D.size() <= 2 && reducesLastDimOnly(A);
        }
        RmsqMatch rq;
        if (rows && opt.rmsnKernel && matchRmsQuant(A, rq)) {
          p = lowerRmsNorm(A, rq, kname);
        } else if (rows && opt.rmsqKernel && matchRmsQuant(A, rq)) {
          p = lowerRmsQuant(A, rq, kname);
        } else if (rows) {
          RowEmitter e(A, opt);
          p = e.run(kname, "LAST_AXIS_PBR");
        } else {
          collapseDomain(A);
          ColumnEmitter e(A);
          p = e.run(kname, "ANY_PBR");
        }
      } else {
        bool anyBrc = false;
        for (auto &kv : A.map) anyBrc |= kv.second.size() != A.D.size();
        EltwiseEmitter e(A);
        p = e.run(kname, anyBrc ? "ANY_PB" : "PURE_ELEMWISE");
      }
    }
    p.funcName = f.name;
    p.params = A.params;
    p.results = A.results;
    p.algoBytes = algoBytes(A);
    if (A.rowsDyn) {
      if (!p.rowsDyn)
        throw CompileError("runtime row counts: @" + f.name + " lowers to a " + p.kind + " kernel (" + p.variant +
                           "), which is compiled per size (dyn=<func>:<arg>.<dim>=<size>)");
      // the row count must not be baked into the kernel anywhere else
      if (p.source.find(std::to_string(kRuntimeRows)) != std::string::npos ||
          p.source.find(std::to_string(kRuntimeRows - 1)) != std::string::npos)
        throw CompileError("runtime row counts: the kernel of @" + f.name + " depends on the row count");
      for (auto *bufs : {&p.params, &p.results})
        for (auto &b : *bufs)
          for (auto &d : b.shape)
            if (d == kRuntimeRows) d = -1;
      p.algoBytes /= (double)kRuntimeRows;
      if (p.rowsA > 0) p.grid[0] = 1; // set at launch from the row count
    }
    std::string declared = f.fusionKind();
    if (!declared.empty() && declared != p.kind && !(declared == "PURE_ELEMWISE" && p.kind == "ANY_PB") &&
        !(declared == "ANY_PB" && p.kind == "PURE_ELEMWISE") && !(declared == "ANY_PBR" && p.kind == "LAST_AXIS_PBR") &&
        !(declared == "LAST_AXIS_PBR" && p.kind == "REDUCE_WITH_INDEX") &&
        !(declared == "LAST_AXIS_PBR" && p.kind == "ANY_PBR"))
      p.variant += " (declared " + declared + ")";
    out.push_back(p);
  }
  if (out.empty()) throw CompileError("no kernel functions in module");
  return out;
}

std::string emitTranslationUnit(const std::vector<KernelPlan> &plans) {
  std::ostringstream s;
  s << "// Generated by bishengir-compile --target=mi355x (ConvertHFusionToHIP).\n"
    << "#include \"hf_ops.h\"\n#include \"hf_row.h\"\n#include \"hf_argmax.h\"\n#include \"hf_mmad.h\"\n#include \"hf_misc.h\"\n"
    << "#include \"hf_rmsq.h\"\n#include \"hf_rmsn.h\"\n#include \"hf_sort.h\"\n\n";
  for (auto &p : plans) s << "// group @" << p.funcName << ": " << p.kind << " (" << p.variant << ")\n" << p.source << "\n";
  return s.str();
}

std::string emitManifest(const KernelPlan &p, const std::string &hsacoName) {
  std::ostringstream s;
  s << "hfr-manifest 1\n"
    << "func " << p.funcName << "\n"
    << "kernel " << p.kernelName << "\n"
    << "hsaco " << hsacoName << "\n"
    << "kind " << p.kind << "\n"
    << "grid " << p.grid[0] << " " << p.grid[1] << " " << p.grid[2] << "\n"
    << "block " << p.block[0] << " " << p.block[1] << " " << p.block[2] << "\n"
    << "lds " << p.ldsBytes << "\n"
    << "workspace " << p.workspaceBytes << " " << (p.workspaceZeroInit ? 1 : 0) << "\n"
    << "algo_bytes " << (uint64_t)p.algoBytes << "\n"
    << "algo_ops " << (uint64_t)p.algoOps << "\n";
  if (p.rowsDyn) s << "rows_dyn " << p.rowsA << " " << p.rowsB << " " << p.rowsC << " " << p.rowsCap << "\n";
  auto shp = [](const std::vector<int64_t> &v) {
    std::string r = std::to_string(v.size());
    for (auto d : v) r += " " + std::to_string(d);
    return r;
  };
  for (size_t i = 0; i < p.params.size(); ++i)
    s << "param " << i << " " << p.params[i].role << " " << elemName(p.params[i].elem) << " " << shp(p.params[i].shape) << "\n";
  for (size_t i = 0; i < p.results.size(); ++i)
    s << "result " << i << " " << p.results[i].tiedParam << " " << elemName(p.results[i].elem) << " " << shp(p.results[i].shape) << "\n";
  for (auto &k : p.kargs) s << "karg " << k << "\n";
  for (auto &pk : p.pre) {
    s << "pre " << pk.name << " " << pk.grid << " 1 1 " << pk.block << " 1 1 " << pk.kargs.size();
    for (auto &k : pk.kargs) s << " " << k;
    s << "\n";
  }
  s << "variant " << p.variant << "\n";
  return s.str();
}

} // namespace hfc
