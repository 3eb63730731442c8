// HFusion fusion front-end (see fusion.h).
#include "fusion.h"
#include "lower.h"

#include <algorithm>
#include <climits>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <queue>
#include <set>
#include <sstream>

namespace hfc {
namespace {

// Op patterns (OpFusion/FusibleHelper.cpp:getOpPattern, restricted to the op
// vocabulary this backend reads).
enum class Pat { EW, ZR, LB, OB, LR, OR, MM, TR, RS, Aux, Buffer, Opaque };

// FusionKind numbering of HFusionEnums.td:210-233.
enum Kind { PureElemwise = 1, AnyPB, LastAxisPBR, AnyPBR, SingleCube, ShallowCV, ShallowVV, MixCV, MixC2, Unknown };

const char *kindName(int k) {
  static const char *n[] = {"", "PURE_ELEMWISE", "ANY_PB", "LAST_AXIS_PBR", "ANY_PBR", "SINGLE_CUBE",
                            "SHALLOW_CV", "SHALLOW_VV", "MIX_CV", "MIX_C2", "UNKNOWN"};
  return n[k];
}

size_t rankOf(const Value *v) { return v->type.tensor ? v->type.shape.size() : 0; }

bool isElementwiseName(const std::string &n) {
  static const std::set<std::string> s = {"linalg.elemwise_unary", "linalg.elemwise_binary", "linalg.fill",
                                          "hfusion.elemwise_unary", "hfusion.elemwise_binary", "hfusion.compare",
                                          "hfusion.cast", "hfusion.select", "hfusion.bitcast", "hfusion.signbit", "hfusion.cyl_bessel_i0", "hfusion.isinf",
                                          "hfusion.isnan", "hfusion.isfinite", "hfusion.nextafter", "hfusion.hypot",
                                          "hfusion.erfinv"};
  return s.count(n) != 0;
}

Pat patternOf(const Op *op) {
  const std::string &n = op->name;
  if (isElementwiseName(n)) {
    bool zero = true;
    for (auto *v : op->ins) zero &= rankOf(v) == 0;
    for (auto *v : op->outs) zero &= rankOf(v) == 0;
    for (auto *v : op->operands) zero &= rankOf(v) == 0;
    return zero ? Pat::ZR : Pat::EW;
  }
  if (n == "linalg.reduce" || n == "hfusion.reduce_with_index") {
    if (op->dims.size() != 1 || op->outs.empty()) return Pat::OR;
    return (size_t)op->dims[0] == rankOf(op->outs[0]) ? Pat::LR : Pat::OR;
  }
  if (n == "linalg.broadcast") {
    if (op->dims.size() != 1 || op->ins.empty()) return Pat::OB;
    return (size_t)op->dims[0] == rankOf(op->ins[0]) ? Pat::LB : Pat::OB;
  }
  if (n == "linalg.matmul" || n == "linalg.matmul_transpose_a" || n == "linalg.matmul_transpose_b" ||
      n == "hfusion.matmul_mx")
    return Pat::MM;
  if (n == "linalg.transpose") return Pat::TR;
  if (n == "tensor.expand_shape" || n == "tensor.collapse_shape") return Pat::RS;
  if (n == "tensor.empty") return Pat::Buffer;
  if (n == "tensor.dim" || n == "annotation.mark") return Pat::Aux;
  if (n == "arith.constant") return (!op->results.empty() && op->results[0]->type.tensor) ? Pat::Opaque : Pat::Aux;
  // scalar arith / math feeding the groups (index casts of tensor.dim, ...)
  if ((n.rfind("arith.", 0) == 0 || n.rfind("math.", 0) == 0) && !op->results.empty() && !op->results[0]->type.tensor)
    return Pat::Aux;
  return Pat::Opaque;
}

bool important(Pat p) {
  return p == Pat::EW || p == Pat::ZR || p == Pat::LB || p == Pat::OB || p == Pat::LR || p == Pat::OR || p == Pat::MM ||
         p == Pat::TR;
}

bool inSet(Pat p, std::initializer_list<Pat> s) { return std::find(s.begin(), s.end(), p) != s.end(); }

// Producer -> consumer fusibility per kind (FusibleHelper.cpp:isFusible and the
// per-kind tables).
bool fusible(int kind, Pat a, Pat b) {
  switch (kind) {
  case PureElemwise:
    return inSet(a, {Pat::EW, Pat::ZR, Pat::TR, Pat::RS}) && inSet(b, {Pat::EW, Pat::ZR, Pat::TR, Pat::RS});
  case AnyPB: {
    auto s = {Pat::EW, Pat::ZR, Pat::LB, Pat::OB, Pat::TR, Pat::RS};
    return inSet(a, s) && inSet(b, s);
  }
  case LastAxisPBR:
    if (inSet(a, {Pat::EW, Pat::ZR, Pat::TR, Pat::RS}))
      return inSet(b, {Pat::EW, Pat::ZR, Pat::LB, Pat::LR, Pat::OB, Pat::TR, Pat::RS});
    if (inSet(a, {Pat::LB, Pat::LR, Pat::OB})) return inSet(b, {Pat::EW, Pat::ZR, Pat::LB, Pat::OB, Pat::TR, Pat::RS});
    return false;
  case AnyPBR: {
    auto s = {Pat::EW, Pat::ZR, Pat::LB, Pat::LR, Pat::OB, Pat::OR, Pat::TR, Pat::RS};
    return inSet(a, s) && inSet(b, s);
  }
  case MixCV:
    if (inSet(a, {Pat::EW, Pat::ZR, Pat::TR, Pat::RS})) return inSet(b, {Pat::EW, Pat::ZR, Pat::TR, Pat::RS});
    if (a == Pat::MM) return inSet(b, {Pat::EW, Pat::ZR});
    return false;
  default: // SingleCube holds one op; the shallow / C2 kinds are Ascend-only
    return false;
  }
}

// Ops a kind can schedule as a group of one (FusibleHelper.cpp:schedulable).
bool schedulable(int kind, Pat p) {
  switch (kind) {
  case PureElemwise: return inSet(p, {Pat::EW, Pat::ZR});
  case AnyPB: return inSet(p, {Pat::EW, Pat::ZR, Pat::LB, Pat::OB});
  case LastAxisPBR: return inSet(p, {Pat::EW, Pat::ZR, Pat::LR, Pat::LB, Pat::OB});
  case AnyPBR: return inSet(p, {Pat::EW, Pat::ZR, Pat::LR, Pat::LB, Pat::OB, Pat::OR});
  case MixCV: return inSet(p, {Pat::EW, Pat::ZR, Pat::MM});
  default: return false;
  }
}

int singleKind(Pat p) {
  switch (p) {
  case Pat::EW: case Pat::ZR: case Pat::TR: return PureElemwise;
  case Pat::LR: return LastAxisPBR;
  case Pat::OR: return AnyPBR;
  case Pat::MM: return SingleCube;
  case Pat::LB: case Pat::OB: return AnyPB;
  default: return Unknown;
  }
}

// MixCV node types (FusibleHelper.cpp:obtainType / adjustType).
enum Ty { TyOpaque = 0, TyPureEW = 1, TyPureMM = 2, TySuffixEW = 3 };

// Union-find over the ops of one function body, growing fusible blocks of one
// kind (the algorithm of FusibleBlockAnalyzer.cpp).  Ops already placed in
// groups are pre-joined into opaque nodes.
class Analyzer {
public:
  // Nodes are the function's ops in program order plus the return (last).
  Analyzer(const Func &f, int kind, int maxHorizontal, const std::vector<std::vector<int>> &placed)
      : f_(f), kind_(kind), maxH_(maxHorizontal < 0 ? INT_MAX : maxHorizontal) {
    const size_t n = f.ops.size() + 1;
    ret_ = (int)f.ops.size();
    for (size_t i = 0; i + 1 < n; ++i) idx_[f.ops[i]] = (int)i;
    par_.assign(n, -1);
    pat_.assign(n, Pat::Opaque);
    opaque_.assign(n, false);
    ty_.assign(n, TyOpaque);
    rank_.assign(n, -1);
    rdim_.assign(n, -1);
    imp_.assign(n, 0);
    pivot_.assign(n, -1);
    topo_.assign(n, 0);
    edge_.resize(n);
    rev_.resize(n);
    users_.resize(n);
    for (size_t i = 0; i + 1 < n; ++i) {
      const Op *op = f.ops[i];
      Pat p = patternOf(op);
      pat_[i] = p;
      imp_[i] = important(p) ? 1 : 0;
      if (p == Pat::LR) {
        int r = 0;
        for (auto *v : op->ins) r = std::max(r, (int)rankOf(v));
        rank_[i] = r;
      }
      if ((p == Pat::LR || p == Pat::OR) && op->dims.size() == 1) rdim_[i] = (int)op->dims[0];
      ty_[i] = inSet(p, {Pat::EW, Pat::ZR}) ? TyPureEW : p == Pat::MM ? TyPureMM : TyOpaque;
      if (isPivot(p, op)) pivot_[i] = (int)i;
      // users in MLIR use-list order: per result, most recent use first
      // (the return, created last, leads)
      for (auto *r : op->results) {
        for (auto it = f.returns.rbegin(); it != f.returns.rend(); ++it)
          if (*it == r) users_[i].push_back(ret_);
        for (auto it = r->users.rbegin(); it != r->users.rend(); ++it)
          if (idx_.count(*it)) users_[i].push_back(idx_.at(*it));
      }
    }
    opaque_[ret_] = true;
    // earlier groups: one opaque node each
    for (auto &g : placed) {
      for (size_t k = 1; k < g.size(); ++k) {
        int a = find(g[0]), b = find(g[k]);
        if (a != b) { par_[a] += par_[b]; par_[b] = a; }
      }
      for (int i : g) opaque_[i] = true;
      imp_[find(g[0])] = 0;
    }
  }

  // Blocks of this kind with more than one important op.
  std::vector<std::vector<int>> blocks() {
    initEdges();
    initTopo();
    // candidate (producer, user) pairs by the user's then the producer's
    // topological rank; std::sort as the reference's llvm::sort
    std::vector<std::pair<int, int>> cand;
    for (size_t u = 0; u < users_.size(); ++u)
      for (int v : users_[u]) cand.emplace_back((int)u, v);
    std::sort(cand.begin(), cand.end(), [&](const std::pair<int, int> &a, const std::pair<int, int> &b) {
      if (topo_[a.second] != topo_[b.second]) return topo_[a.second] < topo_[b.second];
      return topo_[a.first] < topo_[b.first];
    });
    for (auto &c : cand)
      if (!opaque_[c.first] && !opaque_[c.second] && fusible(kind_, pat_[c.first], pat_[c.second]))
        tryJoin(c.first, c.second, false);
    // horizontal merging of independent blocks
    std::vector<int> heads;
    for (size_t i = 0; i < f_.ops.size(); ++i) {
      int p = find((int)i);
      if (p != (int)i || imp_[p] < 1 || opaque_[i]) continue;
      if (size(p) == 1 && !schedulable(kind_, pat_[i])) continue;
      heads.push_back((int)i);
    }
    std::sort(heads.begin(), heads.end(), [&](int a, int b) { return topo_[a] < topo_[b]; });
    int merged = 0;
    if (trace_) {
      std::fprintf(stderr, "[fusion %s] heads:", kindName(kind_));
      for (int h : heads) std::fprintf(stderr, " %d(topo %d)", h, topo_[h]);
      std::fprintf(stderr, "\n");
    }
    for (size_t u = 0; u < heads.size() && merged < maxH_; ++u)
      for (size_t v = u + 1; v < heads.size() && merged < maxH_; ++v) merged += tryJoin(heads[u], heads[v], true) ? 1 : 0;
    std::map<int, std::vector<int>> sets;
    for (size_t i = 0; i < f_.ops.size(); ++i)
      if (!opaque_[i]) sets[find((int)i)].push_back((int)i);
    std::vector<std::vector<int>> out;
    for (auto &kv : sets) {
      const auto &g = kv.second;
      if (g.size() < 2) continue;
      int nImp = 0, nMM = 0;
      for (int i : g) { nImp += important(pat_[i]); nMM += pat_[i] == Pat::MM; }
      if (nImp <= 1) continue;
      if (kind_ == MixCV && nMM == 0) continue;
      out.push_back(g);
    }
    return out;
  }

private:
  const Func &f_;
  int kind_, maxH_;
  std::map<const Op *, int> idx_;
  std::vector<int> par_; // < 0: head with -size
  std::vector<Pat> pat_;
  std::vector<bool> opaque_;
  std::vector<int> ty_, rank_, rdim_, imp_, pivot_, topo_;
  std::vector<std::map<int, bool>> edge_; // head -> (head, fusible)
  std::vector<std::set<int>> rev_;
  std::vector<std::vector<int>> users_; // per node, user nodes in use-list order
  int ret_ = 0;                         // the return node
  bool trace_ = std::getenv("HFC_FUSION_TRACE") != nullptr;

  bool isPivot(Pat p, const Op *op) const {
    switch (kind_) {
    case MixCV: return p == Pat::MM;
    case AnyPB: case LastAxisPBR: case AnyPBR: return p == Pat::LB || p == Pat::OB || op->name == "linalg.fill";
    case PureElemwise: return p == Pat::EW || p == Pat::ZR;
    default: return false;
    }
  }

  int find(int x) { return par_[x] < 0 ? x : par_[x] = find(par_[x]); }
  int size(int x) { return -par_[find(x)]; }

  void initEdges() {
    for (auto &e : edge_) e.clear();
    for (auto &r : rev_) r.clear();
    for (size_t i = 0; i < users_.size(); ++i) {
      int a = find((int)i);
      for (int ui : users_[i]) {
        int b = find(ui);
        if (a == b) continue;
        bool ok = !opaque_[i] && !opaque_[ui] && fusible(kind_, pat_[i], pat_[ui]);
        auto it = edge_[a].find(b);
        edge_[a][b] = (it == edge_[a].end() || it->second) && ok;
        rev_[b].insert(a);
      }
    }
  }

  void initTopo() {
    const size_t n = users_.size();
    std::vector<int> indeg(n, 0);
    for (size_t i = 0; i < n; ++i)
      for (auto &e : edge_[i]) ++indeg[e.first];
    std::queue<int> q;
    for (size_t i = 0; i < n; ++i)
      if (indeg[i] == 0) q.push((int)i);
    int rank = 0;
    while (!q.empty()) {
      size_t cnt = q.size();
      while (cnt--) {
        int x = q.front();
        q.pop();
        topo_[x] = rank;
        for (auto &e : edge_[x])
          if (--indeg[e.first] == 0) q.push(e.first);
      }
      ++rank;
    }
  }

  static bool sameOutShape(const Op *a, const Op *b) {
    size_t na = a->ins.size() + a->outs.size() + a->operands.size();
    size_t nb = b->ins.size() + b->outs.size() + b->operands.size();
    if (na != nb || a->outs.size() != b->outs.size()) return false;
    for (size_t i = 0; i < a->outs.size(); ++i)
      if (a->outs[i]->type.shape != b->outs[i]->type.shape) return false;
    return true;
  }

  static bool sameMatmulShape(const Op *a, const Op *b) {
    if (a->outs.empty() || b->outs.empty() || a->ins.empty() || b->ins.empty()) return false;
    if (a->outs[0]->type.shape != b->outs[0]->type.shape) return false;
    auto fa = a->ins[0]->type.shape, fb = b->ins[0]->type.shape;
    if (a->name == "linalg.matmul_transpose_a" && fa.size() == 2) std::swap(fa[0], fa[1]);
    if (b->name == "linalg.matmul_transpose_a" && fb.size() == 2) std::swap(fb[0], fb[1]);
    return fa == fb;
  }

  // True when the two blocks may not merge because of another path between
  // them (FusibleBlockAnalyzer.cpp:isRestrictedByDependency).
  bool restrictedByDependency(int s, int t, bool horizontal) {
    if (!horizontal) {
      auto it = edge_[s].find(t);
      if (it == edge_[s].end() || !it->second) return true;
      if (edge_[s].size() == 1) return false;
    }
    std::vector<int> indeg(users_.size(), 0);
    std::vector<bool> seen(users_.size(), false);
    std::queue<int> q;
    seen[s] = true;
    q.push(s);
    while (!q.empty()) {
      int x = q.front();
      q.pop();
      for (auto &e : edge_[x]) {
        ++indeg[e.first];
        if (seen[e.first]) continue;
        seen[e.first] = true;
        if (horizontal || topo_[e.first] <= topo_[t]) q.push(e.first);
      }
    }
    return horizontal ? indeg[t] > 0 : indeg[t] > 1;
  }

  bool tryJoin(int u, int v, bool horizontal) {
    int pu = find(u), pv = find(v);
    if (pu == pv) return false;
    if (kind_ == LastAxisPBR || kind_ == AnyPBR) {
      if (rank_[pu] >= 0 && rank_[pv] >= 0 && rank_[pu] != rank_[pv]) return false;
      if (rdim_[pu] >= 0 && rdim_[pv] >= 0 && rdim_[pu] != rdim_[pv]) return false;
    }
    if (kind_ == MixCV && !horizontal) {
      int a = ty_[pu], b = ty_[pv];
      bool ok = ((a == TyPureEW || a == TyPureMM) && b == TyPureEW) || (a == TySuffixEW && b == TyPureEW);
      if (!ok) return false;
    }
    if (horizontal && pivot_[pu] >= 0 && pivot_[pv] >= 0 &&
        !(kind_ == MixCV ? sameMatmulShape(f_.ops[pivot_[pu]], f_.ops[pivot_[pv]])
                         : sameOutShape(f_.ops[pivot_[pu]], f_.ops[pivot_[pv]])))
      return false;
    if (restrictedByDependency(pu, pv, horizontal)) {
      if (trace_ && horizontal) std::fprintf(stderr, "  dep %d->%d\n", pu, pv);
      return false;
    }
    if (horizontal) {
      if (restrictedByDependency(pv, pu, true)) {
        if (trace_) std::fprintf(stderr, "  dep %d->%d\n", pv, pu);
        return false;
      }
      if (imp_[pu] == 0 || imp_[pv] == 0) return false;
    }
    if (trace_) std::fprintf(stderr, "[fusion %s] join %d %d%s\n", kindName(kind_), u, v, horizontal ? " (horizontal)" : "");
    join(pu, pv, horizontal);
    return true;
  }

  void mergeEdges(int a, int b) {
    edge_[a].erase(b);
    edge_[b].erase(a);
    for (auto &e : edge_[b]) {
      rev_[e.first].erase(b);
      rev_[e.first].insert(a);
      if (!e.second) edge_[a][e.first] = false;
      else edge_[a].emplace(e.first, true);
    }
    edge_[b].clear();
    rev_[a].erase(b);
    rev_[b].erase(a);
    for (int p : rev_[b]) {
      auto it = edge_[p].find(b);
      bool ok = it != edge_[p].end() && it->second;
      if (!ok) edge_[p][a] = false;
      else edge_[p].emplace(a, true);
      edge_[p].erase(b);
      rev_[a].insert(p);
    }
    rev_[b].clear();
  }

  void join(int a, int b, bool horizontal) {
    const int preA = a, preB = b;
    if (par_[a] > par_[b]) std::swap(a, b); // larger set stays the head
    mergeEdges(a, b);
    par_[a] += par_[b];
    imp_[a] += imp_[b];
    if (pivot_[b] != -1) pivot_[a] = pivot_[b];
    par_[b] = a;
    if (rank_[a] < 0) rank_[a] = rank_[b];
    if (rdim_[a] < 0) rdim_[a] = rdim_[b];
    topo_[a] = std::max(topo_[a], topo_[b]);
    int ta = ty_[preA], tb = ty_[preB], t = TyOpaque;
    if (horizontal) {
      if (ta == TyPureMM || ta == TySuffixEW) t = ta;
      if (tb == TyPureMM || tb == TySuffixEW) t = tb;
    } else if (ta == TyPureEW && tb == TyPureEW) {
      t = TyPureEW;
    } else if ((ta == TyPureMM || ta == TySuffixEW) && tb == TyPureEW) {
      t = TySuffixEW;
    }
    ty_[a] = t;
  }
};

int countImportant(const Func &f) {
  int n = 0;
  for (const Op *op : f.ops) n += important(patternOf(op));
  return n;
}

std::set<const Value *> blockOutputs(const Func &f, const std::set<const Op *> &members) {
  std::set<const Value *> out;
  for (const Op *op : members)
    for (auto *r : op->results) {
      bool used = std::find(f.returns.begin(), f.returns.end(), r) != f.returns.end();
      for (const Op *u : r->users) used |= !members.count(u) && patternOf(u) != Pat::Aux;
      if (used) out.insert(r);
    }
  return out;
}

int inferKind(const Func &f) {
  int nImp = countImportant(f);
  if (nImp == 0) return AnyPB;
  if (nImp == 1) {
    for (const Op *op : f.ops)
      if (important(patternOf(op))) return singleKind(patternOf(op));
  }
  for (int k = PureElemwise; k < Unknown; ++k) {
    if (k == SingleCube || k == ShallowCV || k == ShallowVV || k == MixC2) continue;
    Analyzer a(f, k, -1, {});
    auto bs = a.blocks();
    if (bs.size() != 1) continue;
    int n = 0;
    std::set<const Op *> members;
    for (int i : bs[0]) { n += important(patternOf(f.ops[i])); members.insert(f.ops[i]); }
    if (n != nImp) continue;
    if (k == MixCV && blockOutputs(f, members).size() != 1) continue;
    return k;
  }
  return Unknown;
}

// Follows the destination operand chain of v to a value of `inputs`, if any.
const Value *tiedInput(const Value *v, const std::set<const Value *> &inputs) {
  while (v) {
    if (inputs.count(v)) return v;
    const Op *d = v->def;
    if (!d || d->outs.empty()) return nullptr;
    v = d->outs[std::min<size_t>((size_t)std::max(v->resultIdx, 0), d->outs.size() - 1)];
  }
  return nullptr;
}

uint64_t bytesOf(const Type &t) {
  uint64_t n = 1;
  for (auto d : t.shape) n *= (uint64_t)d;
  return n * (uint64_t)elemBytes(t.elem);
}

std::string sanitize(const std::string &v) {
  std::string s;
  for (char c : v) s += (std::isalnum((unsigned char)c) || c == '_') ? c : '_';
  return s;
}

// Splits a block into single-output blocks: from each output op, walk the
// producers in reverse program order and take those whose every user is
// already taken (FusibleBlockOutliner.cpp:46-160, OutputMode::Single).
std::vector<std::vector<int>> splitSingleOutput(const Func &f, const std::vector<int> &block) {
  std::set<const Op *> inBlock;
  std::map<const Op *, int> index;
  for (int i : block) { inBlock.insert(f.ops[i]); index[f.ops[i]] = i; }
  std::set<const Value *> outs = blockOutputs(f, inBlock);
  std::vector<int> outOps;
  for (int i : block)
    for (auto *r : f.ops[i]->results)
      if (outs.count(r) && std::find(outOps.begin(), outOps.end(), i) == outOps.end()) outOps.push_back(i);
  std::vector<std::vector<int>> res;
  for (int o : outOps) {
    std::set<int> taken = {o};
    std::priority_queue<int> q; // op index = program order
    q.push(o);
    while (!q.empty()) {
      const Op *cur = f.ops[q.top()];
      q.pop();
      std::vector<const Value *> opnds(cur->ins.begin(), cur->ins.end());
      opnds.insert(opnds.end(), cur->outs.begin(), cur->outs.end());
      opnds.insert(opnds.end(), cur->operands.begin(), cur->operands.end());
      for (const Value *v : opnds) {
        const Op *d = v->def;
        if (!d || !inBlock.count(d) || taken.count(index[d])) continue;
        bool safe = true;
        for (auto *r : d->results) {
          if (std::find(f.returns.begin(), f.returns.end(), r) != f.returns.end()) safe = false;
          for (const Op *u : r->users) safe &= index.count(u) && taken.count(index[u]);
        }
        if (safe) { taken.insert(index[d]); q.push(index[d]); }
      }
    }
    if (taken.size() > 1) res.emplace_back(taken.begin(), taken.end());
  }
  return res;
}

bool isHostMarked(const Func &f) {
  auto fk = f.attrs.find("hacc.function_kind");
  return fk != f.attrs.end() && fk->second.find("HOST") != std::string::npos;
}

std::string declaredKind(const Func &f) {
  std::string k = f.fusionKind();
  auto lt = k.find('<'), gt = k.rfind('>');
  if (lt != std::string::npos && gt != std::string::npos && gt > lt) k = k.substr(lt + 1, gt - lt - 1);
  return k;
}

// Functions the front-end splits: host functions (OpFusion.cpp:280-318) and,
// when the input marks no function as host, entry functions whose ops fit
// no single fusion kind.
bool isHostFunction(const Func &f, bool anyEntry) {
  if (isHostMarked(f)) return true;
  if (!declaredKind(f).empty() && declaredKind(f) != "UNKNOWN") return false;
  if (anyEntry && !f.isEntry()) return false; // not compiled at all
  return inferKind(f) == Unknown;
}

int kindFromName(const std::string &n) {
  for (int k = PureElemwise; k <= Unknown; ++k)
    if (n == kindName(k)) return k;
  throw CompileError("unknown fusion kind '" + n + "'");
}

} // namespace

std::string inferFusionKind(const Func &f) { return kindName(inferKind(f)); }

std::string outlineFusedGroups(const Module &m, std::vector<ProgramPlan> &programs, const std::string &forceKind) {
  std::ostringstream text;
  bool changed = false, anyEntry = false;
  for (auto &fp : m.funcs) anyEntry |= fp->isEntry();
  const int forced = forceKind.empty() ? 0 : kindFromName(forceKind);
  text << "module {\n";
  for (auto &fp : m.funcs) {
    const Func &f = *fp;
    if (!isHostFunction(f, anyEntry) && !(forced && declaredKind(f).empty())) {
      text << "  " << m.source.substr(f.srcBegin, f.srcEnd - f.srcBegin) << "\n";
      continue;
    }
    changed = true;
    std::vector<std::vector<int>> groups;
    std::vector<int> kinds;
    std::vector<std::string> names;
    // the kind: forced, else the function's label, else inferred
    // (InferFuncFusionKind.cpp:70-103)
    const std::string label = declaredKind(f);
    int whole = forced ? forced : (!label.empty() && label != "UNKNOWN") ? kindFromName(label) : inferKind(f);
    // the Ascend-only shallow / C2 labels go through the multi-kernel split
    if (whole == ShallowCV || whole == ShallowVV || whole == MixC2) whole = Unknown;
    if (whole != Unknown) {
      // outline by the function's one kind (OpFusion.cpp:136-168)
      Analyzer a(f, whole, -1, {});
      for (auto &b : a.blocks()) {
        names.push_back(f.name + "_" + std::to_string(groups.size()));
        groups.push_back(b);
        kinds.push_back(whole);
      }
    } else {
      // blocks per kind in the multi-kernel order (OpFusion.cpp:68-133);
      // MixCV blocks are split to single outputs and never merged sideways
      for (int k : {MixCV, LastAxisPBR, AnyPB}) {
        Analyzer a(f, k, k == MixCV ? 0 : -1, groups);
        std::vector<std::vector<int>> bs = a.blocks(), split;
        if (k == MixCV)
          for (auto &b : bs)
            for (auto &s : splitSingleOutput(f, b)) split.push_back(s);
        int cnt = 0;
        for (auto &b : k == MixCV ? split : bs) {
          names.push_back(f.name + "_multi_" + kindName(k) + "_" + std::to_string(cnt++));
          groups.push_back(b);
          kinds.push_back(k);
        }
      }
    }
    std::set<int> placed;
    for (auto &g : groups) placed.insert(g.begin(), g.end());
    int singles = 0;
    for (size_t i = 0; i < f.ops.size(); ++i) {
      Pat p = patternOf(f.ops[i]);
      if (placed.count((int)i)) continue;
      // what is left becomes a group of one (OpFusion.cpp:171-229)
      if (important(p)) {
        names.push_back(f.name + "_single_outlined_" + std::to_string(singles++) + "_0");
        groups.push_back({(int)i});
        kinds.push_back(singleKind(p));
        continue;
      }
      if (p == Pat::RS) {
        // a reshape left between kernels is a view of its operand's buffer
        names.push_back("");
        groups.push_back({(int)i});
        kinds.push_back(-1);
        continue;
      }
      if (p == Pat::Opaque && isSingleOpKernel(f.ops[i]->name)) {
        // an op with a kernel of its own (scan, histogram, (de)interleave)
        names.push_back(f.name + "_single_outlined_" + std::to_string(singles++) + "_0");
        groups.push_back({(int)i});
        kinds.push_back(Unknown);
        continue;
      }
      if (p == Pat::Opaque && f.ops[i]->name != "arith.constant")
        throw CompileError("@" + f.name + ": op '" + f.ops[i]->name + "' (line " + std::to_string(f.ops[i]->line) +
                           ") cannot be placed in a fused group");
    }
    // A linalg.fill left as a group of one whose only use is the
    // destination of one op in another group initialises that op's buffer:
    // it is emitted inside the consumer's kernel instead of as a kernel that
    // writes the constant to memory (matmul accumulators, reduction inits).
    std::set<const Op *> initFills;
    {
      std::map<const Op *, int> owner;
      for (size_t g = 0; g < groups.size(); ++g)
        for (int i : groups[g]) owner[f.ops[i]] = (int)g;
      for (size_t g = 0; g < groups.size(); ++g) {
        if (groups[g].size() != 1 || kinds[g] < 0) continue;
        const Op *fill = f.ops[groups[g][0]];
        if (fill->name != "linalg.fill" || fill->results.size() != 1) continue;
        const Value *r = fill->results[0];
        if (r->users.size() != 1 || std::find(f.returns.begin(), f.returns.end(), r) != f.returns.end()) continue;
        const Op *u = r->users[0];
        if (!owner.count(u) || owner[u] == (int)g) continue;
        if (std::find(u->outs.begin(), u->outs.end(), r) == u->outs.end()) continue;
        if (std::find(u->ins.begin(), u->ins.end(), r) != u->ins.end()) continue;
        initFills.insert(fill);
      }
      std::vector<std::vector<int>> g2;
      std::vector<int> k2;
      std::vector<std::string> n2;
      for (size_t g = 0; g < groups.size(); ++g) {
        if (groups[g].size() == 1 && initFills.count(f.ops[groups[g][0]])) continue;
        g2.push_back(groups[g]);
        k2.push_back(kinds[g]);
        n2.push_back(names[g]);
      }
      groups.swap(g2);
      kinds.swap(k2);
      names.swap(n2);
    }
    // the groups' members and the auxiliary ops each one needs
    std::map<const Op *, int> groupOf;
    for (size_t g = 0; g < groups.size(); ++g)
      for (int i : groups[g]) groupOf[f.ops[i]] = (int)g;
    std::map<const Op *, size_t> order;
    for (size_t i = 0; i < f.ops.size(); ++i) order[f.ops[i]] = i;
    // topological order of the groups (producer group before consumer group)
    std::vector<std::set<int>> deps(groups.size());
    for (size_t g = 0; g < groups.size(); ++g)
      for (int i : groups[g]) {
        const Op *op = f.ops[i];
        std::vector<const Value *> opnds(op->ins.begin(), op->ins.end());
        opnds.insert(opnds.end(), op->outs.begin(), op->outs.end());
        opnds.insert(opnds.end(), op->operands.begin(), op->operands.end());
        for (const Value *v : opnds)
          if (v->def && groupOf.count(v->def) && groupOf[v->def] != (int)g) deps[g].insert(groupOf[v->def]);
      }
    std::vector<int> seq, state(groups.size(), 0);
    std::function<void(int)> visit = [&](int g) {
      if (state[g] == 2) return;
      if (state[g] == 1) throw CompileError("internal: cyclic op groups in @" + f.name);
      state[g] = 1;
      for (int d : deps[g]) visit(d);
      state[g] = 2;
      seq.push_back(g);
    };
    for (size_t g = 0; g < groups.size(); ++g) visit((int)g);
    std::vector<int> seqPos(groups.size());
    for (size_t k = 0; k < seq.size(); ++k) seqPos[seq[k]] = (int)k;

    ProgramPlan prog;
    prog.name = f.name;
    std::map<const Value *, std::string> binding; // value -> buffer binding
    for (size_t i = 0; i < f.args.size(); ++i) {
      const Value *a = f.args[i];
      ProgramBuffer b;
      b.elem = a->type.elem;
      b.shape = a->type.shape;
      b.role = a->type.tensor ? "in" : "scalar";
      prog.params.push_back(b);
      binding[a] = "p" + std::to_string(i);
    }
    // program results; a value reaching a result only through reshape views
    // is written straight into that result's buffer
    std::map<const Value *, int> resultIdx;
    for (size_t k = 0; k < f.returns.size(); ++k) {
      const Value *v = f.returns[k];
      while (true) {
        if (!resultIdx.count(v)) resultIdx[v] = (int)k;
        const Op *d = v->def;
        if (!d || groupOf.count(d) == 0 || kinds[groupOf[d]] >= 0) break;
        v = !d->ins.empty() ? d->ins[0] : !d->operands.empty() ? d->operands[0] : nullptr;
        if (!v || v->argIdx >= 0) break;
      }
    }
    prog.results.resize(f.returns.size());
    for (int g : seq) {
      if (kinds[g] < 0) {
        const Op *rs = f.ops[groups[g][0]];
        const Value *src = !rs->ins.empty() ? rs->ins[0] : !rs->operands.empty() ? rs->operands[0] : nullptr;
        if (!src || rs->results.empty() || !binding.count(src))
          throw CompileError("@" + f.name + ": cannot bind the operand of " + rs->name + " (line " +
                             std::to_string(rs->line) + ")");
        binding[rs->results[0]] = binding[src];
        continue;
      }
      std::set<const Op *> members;
      for (int i : groups[g]) members.insert(f.ops[i]);
      // auxiliary ops (constants, tensor.empty, tensor.dim, scalar arith,
      // annotation.mark) needed by the members, transitively
      std::set<const Op *> emitted(members);
      std::vector<const Op *> work(members.begin(), members.end());
      while (!work.empty()) {
        const Op *op = work.back();
        work.pop_back();
        std::vector<const Value *> opnds(op->ins.begin(), op->ins.end());
        opnds.insert(opnds.end(), op->outs.begin(), op->outs.end());
        opnds.insert(opnds.end(), op->operands.begin(), op->operands.end());
        for (const Value *v : opnds) {
          const Op *d = v->def;
          if (!d || emitted.count(d) || groupOf.count(d)) continue;
          Pat p = patternOf(d);
          if (p == Pat::Aux || p == Pat::Buffer || d->name == "arith.constant" || initFills.count(d)) {
            emitted.insert(d);
            work.push_back(d);
          }
        }
      }
      for (const Op *op : f.ops) // marks on member results travel with them
        if (op->name == "annotation.mark" && !op->operands.empty() && op->operands[0]->def &&
            members.count(op->operands[0]->def))
          emitted.insert(op);
      std::vector<const Op *> ops(emitted.begin(), emitted.end());
      std::sort(ops.begin(), ops.end(), [&](const Op *a, const Op *b) { return order[a] < order[b]; });
      // inputs: values the emitted ops use that they do not define
      std::vector<const Value *> inputs;
      std::set<const Value *> inputSet;
      for (const Op *op : ops) {
        std::vector<const Value *> opnds(op->ins.begin(), op->ins.end());
        opnds.insert(opnds.end(), op->outs.begin(), op->outs.end());
        opnds.insert(opnds.end(), op->operands.begin(), op->operands.end());
        for (const Value *v : opnds)
          if ((!v->def || !emitted.count(v->def)) && !inputSet.count(v)) { inputSet.insert(v); inputs.push_back(v); }
      }
      std::set<const Value *> outSet = blockOutputs(f, members);
      std::vector<const Value *> outputs(outSet.begin(), outSet.end());
      std::sort(outputs.begin(), outputs.end(), [&](const Value *a, const Value *b) {
        if (a->def != b->def) return order[a->def] < order[b->def];
        return a->resultIdx < b->resultIdx;
      });
      const std::string gname = names[g];
      ProgramStep ps;
      ps.group = gname;
      text << "  func.func @" << gname << "(";
      for (size_t i = 0; i < inputs.size(); ++i) {
        if (!binding.count(inputs[i])) throw CompileError("internal: unbound group input in @" + f.name);
        text << (i ? ", " : "") << "%" << sanitize(inputs[i]->name.substr(1)) << "_in: " << inputs[i]->type.str();
        ps.args.push_back(binding[inputs[i]]);
      }
      text << ")";
      if (!outputs.empty()) {
        text << " -> (";
        for (size_t i = 0; i < outputs.size(); ++i) text << (i ? ", " : "") << outputs[i]->type.str();
        text << ")";
      }
      text << " attributes {" << (anyEntry ? "hacc.entry, " : "") << "hfusion.fusion_kind = #hfusion.fusion_kind<"
           << kindName(kinds[g]) << ">} {\n";
      // inputs keep their names through a rename of the argument list
      std::map<std::string, std::string> rename;
      for (const Value *v : inputs) rename[v->name] = "%" + sanitize(v->name.substr(1)) + "_in";
      for (const Op *op : ops) {
        std::string st = m.source.substr(op->srcBegin, op->srcEnd - op->srcBegin);
        // rename uses of the inputs (whole SSA names only)
        std::string outStr;
        for (size_t i = 0; i < st.size();) {
          if (st[i] == '%') {
            size_t j = i + 1;
            while (j < st.size() && (std::isalnum((unsigned char)st[j]) || st[j] == '_' || st[j] == '.' || st[j] == '$' ||
                                     st[j] == '-' || st[j] == '#'))
              ++j;
            std::string nm = st.substr(i, j - i), base = nm;
            auto hash = nm.find('#');
            if (hash != std::string::npos) base = nm.substr(0, hash);
            auto it = rename.find(nm);
            if (it == rename.end() && base != nm) it = rename.find(nm);
            outStr += it != rename.end() ? it->second : nm;
            i = j;
          } else {
            outStr += st[i++];
          }
        }
        text << "    " << outStr << "\n";
      }
      if (!outputs.empty()) {
        text << "    return ";
        for (size_t i = 0; i < outputs.size(); ++i) text << (i ? ", " : "") << outputs[i]->name;
        text << " : ";
        for (size_t i = 0; i < outputs.size(); ++i) text << (i ? ", " : "") << outputs[i]->type.str();
        text << "\n";
      } else {
        text << "    return\n";
      }
      text << "  }\n";
      // result buffers: written into an input's buffer, a program result or
      // a temporary
      for (const Value *o : outputs) {
        const Value *t = tiedInput(o, inputSet);
        std::string b;
        if (t && t->type.elem == o->type.elem) {
          // the group writes into its input's buffer: no later group may
          // still read the value that buffer held
          for (const Op *u : t->users)
            if (groupOf.count(u) && seqPos[groupOf[u]] > seqPos[g])
              throw CompileError("@" + f.name + ": " + t->name + " is updated in place by one fused group (line " +
                                 std::to_string(o->def->line) + ") and read by a later one; give the op a fresh "
                                 "tensor.empty destination");
          b = binding[t];
        } else if (resultIdx.count(o)) {
          b = "r" + std::to_string(resultIdx[o]);
        } else {
          ProgramBuffer tb;
          tb.elem = o->type.elem;
          tb.shape = o->type.shape;
          tb.bytes = bytesOf(o->type);
          tb.offset = (prog.workspaceBytes + 255) / 256 * 256;
          prog.workspaceBytes = tb.offset + tb.bytes;
          b = "t" + std::to_string(prog.temps.size());
          prog.temps.push_back(tb);
        }
        binding[o] = b;
        ps.results.push_back(b);
        if (b[0] == 'p') prog.params[std::stoi(b.substr(1))].role = "out";
      }
      prog.steps.push_back(ps);
      prog.groupKinds.push_back(kindName(kinds[g]));
    }
    for (size_t k = 0; k < f.returns.size(); ++k) {
      const Value *r = f.returns[k];
      ProgramBuffer b;
      b.elem = r->type.elem;
      b.shape = r->type.shape;
      b.bytes = bytesOf(r->type);
      if (!binding.count(r)) throw CompileError("@" + f.name + " returns a value no group produces");
      b.role = binding[r][0] == 'p' ? binding[r] : (binding[r] == "r" + std::to_string(k) ? "r" : "");
      if (b.role.empty() && binding[r][0] == 'r')
        throw CompileError("@" + f.name + ": results " + binding[r].substr(1) + " and " + std::to_string(k) +
                           " share one buffer");
      if (b.role.empty())
        throw CompileError("@" + f.name + ": result " + std::to_string(k) + " is written in place into an "
                           "intermediate tensor; give its op a tensor.empty destination");
      prog.results[k] = b;
    }
    // written params that an op also reads (as `ins` / plain operand)
    for (const Op *op : f.ops) {
      std::vector<const Value *> rd(op->ins.begin(), op->ins.end());
      rd.insert(rd.end(), op->operands.begin(), op->operands.end());
      for (const Value *v : rd)
        if (v->argIdx >= 0 && prog.params[v->argIdx].role == "out") prog.params[v->argIdx].role = "inout";
    }
    programs.push_back(prog);
  }
  text << "}\n";
  return changed ? text.str() : m.source;
}

std::string emitProgramManifest(const ProgramPlan &p) {
  std::ostringstream s;
  auto shp = [](const std::vector<int64_t> &v) {
    std::string r = std::to_string(v.size());
    for (auto d : v) r += " " + std::to_string(d);
    return r;
  };
  s << "hfr-program 1\n"
    << "program " << p.name << "\n"
    << "pworkspace " << p.workspaceBytes << "\n";
  for (size_t i = 0; i < p.params.size(); ++i)
    s << "pparam " << i << " " << p.params[i].role << " " << elemName(p.params[i].elem) << " " << shp(p.params[i].shape) << "\n";
  for (size_t i = 0; i < p.results.size(); ++i)
    s << "presult " << i << " " << p.results[i].role << " " << elemName(p.results[i].elem) << " " << shp(p.results[i].shape)
      << "\n";
  for (size_t i = 0; i < p.temps.size(); ++i)
    s << "ptemp " << i << " " << p.temps[i].offset << " " << p.temps[i].bytes << " " << elemName(p.temps[i].elem) << " "
      << shp(p.temps[i].shape) << "\n";
  for (size_t i = 0; i < p.steps.size(); ++i) {
    const auto &st = p.steps[i];
    s << "pstep " << st.group << " " << p.groupKinds[i] << " " << st.args.size();
    for (auto &a : st.args) s << " " << a;
    s << " " << st.results.size();
    for (auto &r : st.results) s << " " << r;
    s << "\n";
  }
  return s.str();
}

} // namespace hfc
