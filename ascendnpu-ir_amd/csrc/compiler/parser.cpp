// Reader for the textual-MLIR subset of HFusion op groups.
//
// Accepted syntax follows the printers of the ops the reference defines or
// uses: hfusion named structured ops (HFusionNamedStructuredOps.yaml:72-470),
// hfusion.reduce_with_index (HFusionStructuredOps.td:69-157), upstream
// linalg.{elemwise_unary,elemwise_binary,fill,broadcast,reduce,matmul,
// matmul_transpose_b}, tensor.{empty,dim}, arith scalar ops and func.func with
// hacc/hfusion attributes (e.g. bishengir/test/bishengir-compile/hfusion/
// compile-rms-norm-fp32-split-n.mlir:5-47).
#include "ir.h"

#include <cctype>
#include <cstring>
#include <sstream>

namespace hfc {

const char *elemName(Elem e) {
  switch (e) {
  case Elem::F32: return "f32";
  case Elem::F16: return "f16";
  case Elem::BF16: return "bf16";
  case Elem::F64: return "f64";
  case Elem::F8E4M3FN: return "f8E4M3FN";
  case Elem::F8E5M2: return "f8E5M2";
  case Elem::I1: return "i1";
  case Elem::I8: return "i8";
  case Elem::I16: return "i16";
  case Elem::I32: return "i32";
  case Elem::I64: return "i64";
  case Elem::Index: return "index";
  default: return "none";
  }
}
int elemBits(Elem e) {
  switch (e) {
  case Elem::F32: case Elem::I32: return 32;
  case Elem::F16: case Elem::BF16: case Elem::I16: return 16;
  case Elem::F64: case Elem::I64: case Elem::Index: return 64;
  case Elem::I8: case Elem::F8E4M3FN: case Elem::F8E5M2: return 8;
  case Elem::I1: return 1;
  default: return 0;
  }
}
int elemBytes(Elem e) {
  int b = elemBits(e);
  return b == 1 ? 1 : b / 8;
}
bool isFloat(Elem e) {
  return e == Elem::F32 || e == Elem::F16 || e == Elem::BF16 || e == Elem::F64 || e == Elem::F8E4M3FN ||
         e == Elem::F8E5M2;
}
bool isInt(Elem e) {
  return e == Elem::I1 || e == Elem::I8 || e == Elem::I16 || e == Elem::I32 ||
         e == Elem::I64 || e == Elem::Index;
}
Elem parseElem(const std::string &s) {
  static const std::map<std::string, Elem> m = {
      {"f32", Elem::F32}, {"f16", Elem::F16},   {"bf16", Elem::BF16},
      {"f64", Elem::F64}, {"i1", Elem::I1},     {"i8", Elem::I8},
      {"i16", Elem::I16}, {"i32", Elem::I32},   {"i64", Elem::I64},
      {"index", Elem::Index}, {"f8E4M3FN", Elem::F8E4M3FN}, {"f8E5M2", Elem::F8E5M2}};
  auto it = m.find(s);
  if (it == m.end()) throw CompileError("unsupported element type '" + s + "'");
  return it->second;
}

std::string Type::str() const {
  if (!tensor) return elemName(elem);
  std::string s = "tensor<";
  for (auto d : shape) s += std::to_string(d) + "x";
  return s + elemName(elem) + ">";
}

namespace {

enum class Tok { Ident, Value, Symbol, Hash, Number, String, Punct, Raw, End };

struct Token {
  Tok kind;
  std::string text;
  int line;
  size_t off = 0, end = 0; // source span [off, end)
};

bool identStart(char c) { return std::isalpha((unsigned char)c) || c == '_'; }
bool identChar(char c) {
  return std::isalnum((unsigned char)c) || c == '_' || c == '.' || c == '$';
}

// Reads a balanced <...> group starting at text[i] == '<'; returns inner text.
std::string readAngle(const std::string &t, size_t &i, int &line) {
  int depth = 0;
  size_t start = i;
  for (; i < t.size(); ++i) {
    if (t[i] == '\n') ++line;
    if (t[i] == '<') ++depth;
    else if (t[i] == '>' && !(i > 0 && t[i - 1] == '-')) {
      if (--depth == 0) {
        ++i;
        return t.substr(start + 1, i - start - 2);
      }
    }
  }
  throw CompileError("unterminated '<' at line " + std::to_string(line));
}

std::vector<Token> lex(const std::string &t) {
  std::vector<Token> out;
  int line = 1;
  size_t i = 0;
  while (i < t.size()) {
    char c = t[i];
    if (c == '\n') { ++line; ++i; continue; }
    if (std::isspace((unsigned char)c)) { ++i; continue; }
    if (c == '/' && i + 1 < t.size() && t[i + 1] == '/') {
      while (i < t.size() && t[i] != '\n') ++i;
      continue;
    }
    if (c == '%' || c == '@' || c == '^') {
      size_t j = i + 1;
      while (j < t.size() && (identChar(t[j]) || t[j] == '-' || t[j] == '#'))
        ++j;
      out.push_back({c == '%' ? Tok::Value : Tok::Symbol, t.substr(i, j - i), line, i, j});
      i = j;
      continue;
    }
    if (c == '#') {
      size_t j = i + 1;
      while (j < t.size() && identChar(t[j])) ++j;
      std::string name = t.substr(i, j - i);
      if (j < t.size() && t[j] == '<') {
        std::string inner = readAngle(t, j, line);
        out.push_back({Tok::Hash, name + "<" + inner + ">", line, i, j});
      } else {
        out.push_back({Tok::Hash, name, line, i, j});
      }
      i = j;
      continue;
    }
    if (c == '"') {
      size_t j = i + 1;
      while (j < t.size() && t[j] != '"') ++j;
      out.push_back({Tok::String, t.substr(i + 1, j - i - 1), line, i, j + 1});
      i = j + 1;
      continue;
    }
    if (std::isdigit((unsigned char)c) ||
        (c == '-' && i + 1 < t.size() && std::isdigit((unsigned char)t[i + 1]))) {
      size_t j = i + (c == '-' ? 1 : 0);
      if (t.compare(j, 2, "0x") == 0 || t.compare(j, 2, "0X") == 0) {
        j += 2;
        while (j < t.size() && std::isxdigit((unsigned char)t[j])) ++j;
      } else {
        while (j < t.size() && std::isdigit((unsigned char)t[j])) ++j;
        if (j < t.size() && t[j] == '.') {
          ++j;
          while (j < t.size() && std::isdigit((unsigned char)t[j])) ++j;
        }
        if (j < t.size() && (t[j] == 'e' || t[j] == 'E') && j + 1 < t.size() &&
            (std::isdigit((unsigned char)t[j + 1]) || t[j + 1] == '+' || t[j + 1] == '-')) {
          j += 2;
          while (j < t.size() && std::isdigit((unsigned char)t[j])) ++j;
        }
      }
      out.push_back({Tok::Number, t.substr(i, j - i), line, i, j});
      i = j;
      continue;
    }
    if (identStart(c)) {
      size_t j = i;
      while (j < t.size() && identChar(t[j])) ++j;
      std::string id = t.substr(i, j - i);
      if ((id == "tensor" || id == "memref" || id == "dense" ||
           id == "affine_map" || id == "vector") &&
          j < t.size() && t[j] == '<') {
        std::string inner = readAngle(t, j, line);
        out.push_back({Tok::Raw, id + "<" + inner + ">", line, i, j});
      } else {
        out.push_back({Tok::Ident, id, line, i, j});
      }
      i = j;
      continue;
    }
    if (c == '-' && i + 1 < t.size() && t[i + 1] == '>') {
      out.push_back({Tok::Punct, "->", line, i, i + 2});
      i += 2;
      continue;
    }
    out.push_back({Tok::Punct, std::string(1, c), line, i, i + 1});
    ++i;
  }
  out.push_back({Tok::End, "", line, t.size(), t.size()});
  return out;
}

Type parseTypeText(const std::string &s, int line) {
  Type ty;
  // memref<...> (destination-style hivm ops on global memory) reads like a
  // tensor: the shape and element type; the layout / address space after the
  // first comma is dropped
  const bool isMemref = s.rfind("memref<", 0) == 0;
  if (s.rfind("tensor<", 0) == 0 || isMemref) {
    std::string inner = isMemref ? s.substr(7, s.size() - 8) : s.substr(7, s.size() - 8);
    // strip optional encoding ", #enc"
    auto comma = inner.find(',');
    if (comma != std::string::npos) inner = inner.substr(0, comma);
    std::string cleaned;
    for (char c : inner)
      if (!std::isspace((unsigned char)c)) cleaned += c;
    ty.tensor = true;
    ty.memref = isMemref;
    size_t p = 0;
    while (true) {
      size_t x = cleaned.find('x', p);
      if (x == std::string::npos) break;
      std::string d = cleaned.substr(p, x - p);
      if (d == "?") { // a dynamic dim: -1 until specialised (dynamic.cpp)
        ty.shape.push_back(-1);
        p = x + 1;
        continue;
      }
      if (!std::isdigit((unsigned char)cleaned[p])) break;
      bool alldig = !d.empty();
      for (char c : d) alldig &= std::isdigit((unsigned char)c) != 0;
      if (!alldig) break;
      ty.shape.push_back(std::stoll(d));
      p = x + 1;
    }
    std::string e = cleaned.substr(p);
    if (e.find('?') != std::string::npos)
      throw CompileError("unsupported dynamic type '" + s + "' at line " + std::to_string(line));
    try {
      if (e == "ui8") ty.uns = true;
      ty.elem = parseElem(e == "ui8" ? "i8" : e);
    } catch (CompileError &) {
      throw CompileError("unsupported tensor type '" + s + "' at line " +
                         std::to_string(line));
    }
    return ty;
  }
  try {
    ty.elem = parseElem(s);
  } catch (CompileError &) {
    throw CompileError("unsupported type '" + s + "' at line " + std::to_string(line));
  }
  return ty;
}

// Strip "#dialect.kind<inner>" to "inner"; other values unchanged.
std::string normAttr(const std::string &v) {
  if (!v.empty() && v[0] == '#') {
    auto lt = v.find('<');
    if (lt != std::string::npos && v.back() == '>')
      return v.substr(lt + 1, v.size() - lt - 2);
  }
  return v;
}

class Parser {
public:
  Parser(const std::string &text) : toks_(lex(text)), src_(text) {}

  std::unique_ptr<Module> run() {
    mod_.reset(new Module());
    while (peek().kind != Tok::End) {
      if (peek().kind == Tok::Ident && peek().text == "func.func") {
        parseFunc();
      } else if (peek().kind == Tok::Hash && isP(peek(1), "=") && peek(2).kind == Tok::Raw) {
        // attribute alias, e.g. `#map = affine_map<(d0, d1) -> (d1)>`
        mod_->aliases[peek().text] = peek(2).text;
        pos_ += 3;
      } else {
        ++pos_;
      }
    }
    if (mod_->funcs.empty()) throw CompileError("no func.func found in input");
    return std::move(mod_);
  }

private:
  std::vector<Token> toks_;
  std::string src_;
  size_t pos_ = 0;
  std::unique_ptr<Module> mod_;
  std::map<std::string, Value *> scope_;

  const Token &peek(size_t k = 0) const {
    size_t i = pos_ + k;
    return i < toks_.size() ? toks_[i] : toks_.back();
  }
  const Token &next() { return toks_[pos_ < toks_.size() - 1 ? pos_++ : pos_]; }
  bool isP(const Token &t, const char *p) const {
    return t.kind == Tok::Punct && t.text == p;
  }
  [[noreturn]] void fail(const std::string &msg) {
    throw CompileError(msg + " at line " + std::to_string(peek().line));
  }
  void expectP(const char *p) {
    if (!isP(peek(), p)) fail(std::string("expected '") + p + "' but found '" + peek().text + "'");
    ++pos_;
  }

  Type parseType() {
    const Token &t = next();
    if (t.kind == Tok::Raw || t.kind == Tok::Ident) return parseTypeText(t.text, t.line);
    throw CompileError("expected a type at line " + std::to_string(t.line) + ", found '" + t.text + "'");
  }

  // Parses `{k = v, k2, ...}`; the opening brace is the current token.
  std::map<std::string, std::string> parseAttrDict() {
    std::map<std::string, std::string> m;
    expectP("{");
    while (!isP(peek(), "}")) {
      if (peek().kind == Tok::End) fail("unterminated attribute dictionary");
      std::string key = next().text;
      std::string val;
      if (isP(peek(), "=")) {
        ++pos_;
        int depth = 0;
        while (true) {
          const Token &t = peek();
          if (t.kind == Tok::End) fail("unterminated attribute value");
          if (depth == 0 && (isP(t, ",") || isP(t, "}"))) break;
          if (isP(t, "[") || isP(t, "{") || isP(t, "(")) ++depth;
          if (isP(t, "]") || isP(t, "}") || isP(t, ")")) --depth;
          if (!val.empty()) val += " ";
          val += t.text;
          ++pos_;
        }
      } else {
        val = "unit";
      }
      m[key] = normAttr(val);
      if (isP(peek(), ",")) ++pos_;
    }
    expectP("}");
    return m;
  }

  Value *lookup(const std::string &name, int line) {
    auto it = scope_.find(name);
    if (it == scope_.end())
      throw CompileError("use of undefined value " + name + " at line " + std::to_string(line));
    return it->second;
  }

  void define(const std::string &name, Value *v) {
    if (scope_.count(name))
      throw CompileError("redefinition of " + name);
    v->name = name;
    scope_[name] = v;
  }

  // After the `)` of an unnamed-argument list: an optional `-> type` or
  // `-> (types)` and an optional `attributes {...}` of an external declaration.
  void skipSignatureTail() {
    if (isP(peek(), "->")) {
      ++pos_;
      if (isP(peek(), "(")) {
        int depth = 0;
        do {
          if (isP(peek(), "(")) ++depth;
          if (isP(peek(), ")")) --depth;
          ++pos_;
        } while (depth > 0 && peek().kind != Tok::End);
      } else {
        parseType();
      }
    }
    if (peek().kind == Tok::Ident && peek().text == "attributes") {
      ++pos_;
      parseAttrDict();
    }
  }

  void parseFunc() {
    const size_t begin = toks_[pos_].off;
    ++pos_; // func.func
    scope_.clear();
    auto f = std::make_unique<Func>();
    f->srcBegin = begin;
    if (peek().kind == Tok::Ident) ++pos_; // visibility
    if (peek().kind != Tok::Symbol) fail("expected function name");
    f->name = next().text.substr(1);
    expectP("(");
    if (peek().kind != Tok::Value && !isP(peek(), ")")) {
      // an external declaration (`func.func private @f(f32) -> f32`): no
      // body, nothing to lower
      int depth = 1;
      while (depth > 0 && peek().kind != Tok::End) {
        if (isP(peek(), "(")) ++depth;
        if (isP(peek(), ")")) --depth;
        ++pos_;
      }
      skipSignatureTail();
      if (isP(peek(), "{")) fail("function body with unnamed arguments");
      return;
    }
    while (!isP(peek(), ")")) {
      if (peek().kind != Tok::Value) fail("expected function argument");
      std::string nm = next().text;
      expectP(":");
      Value *v = mod_->newValue();
      v->type = parseType();
      v->argIdx = (int)f->args.size();
      define(nm, v);
      f->args.push_back(v);
      if (isP(peek(), "{")) parseAttrDict();
      if (isP(peek(), ",")) ++pos_;
    }
    expectP(")");
    if (isP(peek(), "->")) {
      ++pos_;
      if (isP(peek(), "(")) {
        ++pos_;
        while (!isP(peek(), ")")) {
          f->resultTypes.push_back(parseType());
          if (isP(peek(), "{")) parseAttrDict();
          if (isP(peek(), ",")) ++pos_;
        }
        expectP(")");
      } else {
        f->resultTypes.push_back(parseType());
      }
    }
    if (peek().kind == Tok::Ident && peek().text == "attributes") {
      ++pos_;
      f->attrs = parseAttrDict();
    }
    // a declaration with named (or no) arguments and no body
    if (!isP(peek(), "{")) return;
    expectP("{");
    while (!isP(peek(), "}")) {
      if (peek().kind == Tok::End) fail("unterminated function body");
      if (peek().kind == Tok::Ident &&
          (peek().text == "return" || peek().text == "func.return")) {
        ++pos_;
        while (peek().kind == Tok::Value) {
          int line = peek().line;
          f->returns.push_back(lookup(next().text, line));
          if (isP(peek(), ",")) ++pos_;
        }
        if (isP(peek(), ":")) {
          ++pos_;
          parseType();
          while (isP(peek(), ",")) { ++pos_; parseType(); }
        }
        continue;
      }
      parseStatement(*f);
    }
    expectP("}");
    f->srcEnd = toks_[pos_ - 1].end;
    if (f->returns.size() != f->resultTypes.size())
      throw CompileError("function @" + f->name + ": return arity does not match its signature");
    mod_->funcs.push_back(std::move(f));
  }

  // Is the token at position p the start of a statement (`%a = `, `%a, %b =`,
  // `%a:2 =`)?
  bool statementStart(size_t p) const {
    if (toks_[p].kind != Tok::Value) return false;
    size_t q = p + 1;
    while (q < toks_.size()) {
      const Token &t = toks_[q];
      if (isP(t, "=")) return true;
      if (isP(t, ",") && q + 1 < toks_.size() && toks_[q + 1].kind == Tok::Value) { q += 2; continue; }
      if (isP(t, ":") && q + 1 < toks_.size() && toks_[q + 1].kind == Tok::Number) { q += 2; continue; }
      return false;
    }
    return false;
  }

  void parseOperandList(std::vector<Value *> &vals, std::vector<Type> &types) {
    expectP("(");
    std::vector<std::pair<std::string, int>> names;
    while (peek().kind == Tok::Value) {
      names.push_back({peek().text, peek().line});
      ++pos_;
      if (isP(peek(), ",")) ++pos_;
    }
    if (isP(peek(), ":")) {
      ++pos_;
      while (!isP(peek(), ")")) {
        types.push_back(parseType());
        if (isP(peek(), ",")) ++pos_;
      }
    }
    expectP(")");
    for (auto &n : names) vals.push_back(lookup(n.first, n.second));
  }

  void parseStatement(Func &f) {
    int line = peek().line;
    const size_t firstTok = pos_;
    std::vector<std::string> resNames;
    int multi = 0;
    if (peek().kind == Tok::Value) {
      while (true) {
        std::string nm = next().text;
        if (isP(peek(), ":") && peek(1).kind == Tok::Number) {
          ++pos_;
          multi = std::stoi(next().text);
        }
        resNames.push_back(nm);
        if (isP(peek(), ",")) { ++pos_; continue; }
        break;
      }
      expectP("=");
    }
    if (peek().kind == Tok::String && isP(peek(1), "(")) {
      // generic form: "dialect.op"(%a, %b) {attrs} : (T1, T2) -> T3
      Op *op = mod_->newOp();
      op->name = next().text;
      if (op->name.size() >= 2 && op->name.front() == '"') op->name = op->name.substr(1, op->name.size() - 2);
      op->line = line;
      expectP("(");
      while (!isP(peek(), ")")) {
        if (peek().kind == Tok::Value) op->operands.push_back(lookup(peek().text, peek().line));
        ++pos_;
      }
      expectP(")");
      if (isP(peek(), "{")) {
        auto m = parseAttrDict();
        for (auto &kv : m) op->attrs[kv.first] = kv.second;
      }
      expectP(":");
      expectP("(");
      while (!isP(peek(), ")")) {
        if (!isP(peek(), ",")) parseType();
        else ++pos_;
      }
      expectP(")");
      if (!isP(peek(), "->")) fail("expected '->' in a generic operation type");
      ++pos_;
      std::vector<Type> rtypes;
      if (isP(peek(), "(")) {
        ++pos_;
        while (!isP(peek(), ")")) {
          if (isP(peek(), ",")) { ++pos_; continue; }
          rtypes.push_back(parseType());
        }
        ++pos_;
      } else {
        rtypes.push_back(parseType());
      }
      size_t nres = multi ? (size_t)multi : resNames.size();
      if (nres > rtypes.size()) fail("result count of '" + op->name + "'");
      for (size_t i = 0; i < nres; ++i) {
        Value *v = mod_->newValue();
        v->type = rtypes[i];
        v->def = op;
        v->resultIdx = (int)i;
        op->results.push_back(v);
        if (multi) define(resNames[0] + "#" + std::to_string(i), v);
        else define(resNames[i], v);
      }
      if (multi) scope_[resNames[0]] = op->results[0];
      for (auto *v : op->operands) v->users.push_back(op);
      op->srcBegin = toks_[firstTok].off;
      op->srcEnd = toks_[pos_ - 1].end;
      f.ops.push_back(op);
      return;
    }
    if (peek().kind != Tok::Ident) fail("expected an operation name");
    Op *op = mod_->newOp();
    op->name = next().text;
    op->line = line;
    std::vector<Type> arrowTypes;
    bool sawRegionArgs = false;
    while (true) {
      const Token &t = peek();
      if (t.kind == Tok::End) break;
      if (isP(t, "}")) break; // end of function body
      if (t.kind == Tok::Ident && (t.text == "return" || t.text == "func.return")) break;
      if (t.kind == Tok::Value && statementStart(pos_)) break;
      // an op name on a later line starts the next statement (ops without
      // results, such as annotation.mark or hivm.hir.*)
      if (t.kind == Tok::Ident && t.line > line && t.text.find('.') != std::string::npos) break;
      if (t.kind == Tok::Ident && (t.text == "ins" || t.text == "outs") && isP(peek(1), "(")) {
        bool isIns = t.text == "ins";
        ++pos_;
        if (isIns) parseOperandList(op->ins, op->insTypes);
        else parseOperandList(op->outs, op->outsTypes);
        continue;
      }
      // named operand of an hivm op: `bias = %v : type`, `descale = %v : type`
      if (t.kind == Tok::Ident && isP(peek(1), "=") && peek(2).kind == Tok::Value) {
        op->attrs["operand." + t.text] = std::to_string(op->operands.size());
        pos_ += 2;
        op->operands.push_back(lookup(peek().text, peek().line));
        ++pos_;
        if (isP(peek(), ":")) { ++pos_; parseType(); }
        continue;
      }
      // `descale_mode = #hivm.descale_mode<DescalePerChannel>`
      if (t.kind == Tok::Ident && isP(peek(1), "=") && peek(2).kind == Tok::Hash) {
        op->attrs[t.text] = normAttr(peek(2).text);
        pos_ += 3;
        continue;
      }
      // unit flags of hivm matmuls
      if (t.kind == Tok::Ident && (t.text == "a_transpose" || t.text == "b_transpose")) {
        op->attrs[t.text] = "unit";
        ++pos_;
        continue;
      }
      if (t.kind == Tok::Ident && t.text == "dimensions" && isP(peek(1), "=")) {
        pos_ += 2;
        expectP("[");
        while (!isP(peek(), "]")) {
          if (peek().kind == Tok::Number) op->dims.push_back(std::stoll(peek().text));
          ++pos_;
        }
        expectP("]");
        op->hasDims = true;
        continue;
      }
      // hfusion.arange `offset[%o] strides[%s0, ...]`: the offset operand
      // comes first when present
      if (t.kind == Tok::Ident && t.text == "offset" && isP(peek(1), "[")) {
        op->attrs["arange.offset"] = "1";
        ++pos_;
        continue;
      }
      // `cum_dims = [1]` (integer list) and `reverse = false` / `num = 4`
      // operands written outside the attribute dictionary
      if (t.kind == Tok::Ident && isP(peek(1), "=") && isP(peek(2), "[")) {
        const std::string key = t.text;
        pos_ += 3;
        std::string v;
        while (!isP(peek(), "]") && peek().kind != Tok::End) {
          if (peek().kind == Tok::Number) v += (v.empty() ? "" : ",") + peek().text;
          ++pos_;
        }
        expectP("]");
        op->attrs[key] = v;
        continue;
      }
      if (t.kind == Tok::Ident && isP(peek(1), "=") &&
          (peek(2).kind == Tok::Number || (peek(2).kind == Tok::Ident && (peek(2).text == "true" || peek(2).text == "false")))) {
        op->attrs[t.text] = peek(2).text;
        pos_ += 3;
        continue;
      }
      if (isP(t, "(") && peek(1).kind == Tok::Value && isP(peek(2), ":")) {
        // region block arguments `(%in: f32, %init: f32)` (an operand list
        // such as tensor.empty(%d0, %d1) falls through to the value case)
        int depth = 0;
        do {
          if (isP(peek(), "(")) ++depth;
          if (isP(peek(), ")")) --depth;
          ++pos_;
        } while (depth > 0);
        sawRegionArgs = true;
        continue;
      }
      // the body of a linalg.generic: kept as text (attrs["region"]); values
      // of the enclosing function it reads become operands (attrs["captures"])
      if (isP(t, "{") && peek(1).kind == Tok::Symbol && peek(1).text.rfind("^", 0) == 0) {
        const size_t open = pos_;
        int depth = 0;
        std::string caps;
        do {
          const Token &r = peek();
          if (r.kind == Tok::End) fail("unterminated region");
          if (isP(r, "{")) ++depth;
          if (isP(r, "}")) --depth;
          if (r.kind == Tok::Value && scope_.count(r.text) && caps.find(" " + r.text + " ") == std::string::npos) {
            caps += " " + r.text + " ";
            op->operands.push_back(scope_[r.text]);
          }
          ++pos_;
        } while (depth > 0);
        op->attrs["region"] = src_.substr(toks_[open].end, toks_[pos_ - 1].off - toks_[open].end);
        op->attrs["captures"] = caps;
        continue;
      }
      if (isP(t, "{")) {
        if (sawRegionArgs) {
          int depth = 0;
          do {
            const Token &r = peek();
            if (isP(r, "{")) ++depth;
            if (isP(r, "}")) --depth;
            if (r.kind == Tok::Ident && r.text.find('.') != std::string::npos)
              op->regionOps.push_back(r.text);
            ++pos_;
          } while (depth > 0);
          sawRegionArgs = false;
          continue;
        }
        auto m = parseAttrDict();
        for (auto &kv : m) {
          if (kv.first.rfind("arith.", 0) == 0 && kv.second == "unit") op->combiner = kv.first;
          std::string v = kv.second;
          if (kv.first == "indexing_maps")
            for (auto &al : mod_->aliases) {
              // whole alias names only (#map vs #map1)
              size_t q = 0;
              while ((q = v.find(al.first, q)) != std::string::npos) {
                size_t e = q + al.first.size();
                if (e < v.size() && (std::isalnum((unsigned char)v[e]) || v[e] == '_')) { q = e; continue; }
                v.replace(q, al.first.size(), al.second);
                q += al.second.size();
              }
            }
          op->attrs[kv.first] = v;
        }
        continue;
      }
      if (isP(t, "<") && peek(1).kind == Tok::Ident && isP(peek(2), ">")) {
        op->angleKind = peek(1).text;
        pos_ += 3;
        continue;
      }
      if (isP(t, "->")) {
        ++pos_;
        arrowTypes.push_back(parseType());
        while (isP(peek(), ",")) { ++pos_; arrowTypes.push_back(parseType()); }
        continue;
      }
      if (isP(t, ":")) {
        ++pos_;
        op->literalType = parseType();
        while (isP(peek(), ",")) { ++pos_; parseType(); }
        if (peek().kind == Tok::Ident && (peek().text == "to" || peek().text == "into")) {
          ++pos_;
          op->toType = parseType();
        }
        continue;
      }
      if (t.kind == Tok::Value) {
        op->operands.push_back(lookup(t.text, t.line));
        ++pos_;
        continue;
      }
      if (t.kind == Tok::Number || (t.kind == Tok::Raw && t.text.rfind("dense<", 0) == 0) ||
          (t.kind == Tok::Ident && (t.text == "true" || t.text == "false"))) {
        op->literal = t.text;
        ++pos_;
        continue;
      }
      ++pos_; // punctuation such as '(' ')' of tensor.empty(), ',' separators
    }
    if (op->combiner.empty()) {
      for (auto &r : op->regionOps)
        if (r.rfind("arith.", 0) == 0 || r.rfind("math.", 0) == 0) { op->combiner = r; break; }
    }
    // result types
    std::vector<Type> rtypes = arrowTypes;
    if (rtypes.empty()) {
      if (!op->outsTypes.empty()) rtypes = op->outsTypes;
      else if (op->toType.elem != Elem::None) rtypes.push_back(op->toType);
      else if (op->literalType.elem != Elem::None) rtypes.push_back(op->literalType);
    }
    // hfusion.mulext / mulextui: two results of the operands' type
    if ((op->name == "hfusion.mulext" || op->name == "hfusion.mulextui") && rtypes.size() == 1) rtypes.push_back(rtypes[0]);
    size_t nres = multi ? (size_t)multi : resNames.size();
    if (nres > rtypes.size() && !resNames.empty())
      throw CompileError("cannot infer result types of '" + op->name + "' at line " + std::to_string(line));
    for (size_t i = 0; i < nres; ++i) {
      Value *v = mod_->newValue();
      v->type = rtypes[i];
      v->def = op;
      v->resultIdx = (int)i;
      op->results.push_back(v);
      if (multi) define(resNames[0] + "#" + std::to_string(i), v);
      else define(resNames[i], v);
    }
    if (multi) scope_[resNames[0]] = op->results[0];
    for (auto *v : op->ins) v->users.push_back(op);
    for (auto *v : op->outs) v->users.push_back(op);
    for (auto *v : op->operands) v->users.push_back(op);
    op->srcBegin = toks_[firstTok].off;
    op->srcEnd = pos_ > firstTok ? toks_[pos_ - 1].end : toks_[firstTok].end;
    f.ops.push_back(op);
  }
};

} // namespace

std::unique_ptr<Module> parseModule(const std::string &text) {
  Parser p(text);
  auto m = p.run();
  m->source = text;
  return m;
}

} // namespace hfc
