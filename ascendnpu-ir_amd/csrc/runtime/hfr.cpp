// hfr — C-ABI HIP runtime for HFusion group kernels.  See include/hfr.h.
//
// hipModuleLoad / hipModuleGetFunction / hipModuleLaunchKernel take the place
// of the CANN rtDevBinaryRegister / rtFunctionRegister / rtKernelLaunch calls
// of bishengir/test/Integration/HIVM/VecAdd/main.cpp.
#include "../../../include/hfr.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <mutex>
#include <sstream>
#include <string>
#include <vector>

struct hfr_module {
  hipModule_t mod = nullptr;
  std::string path;
  int refs = 1;
};

struct hfr_kernel {
  hipFunction_t fn = nullptr;
  hfr_module *owner = nullptr;
};

// element size of a manifest element type name (i1 is one byte)
int elemSize(const std::string &e) {
  if (e == "f64" || e == "i64" || e == "index") return 8;
  if (e == "f32" || e == "i32") return 4;
  if (e == "f16" || e == "bf16" || e == "i16") return 2;
  return 1;
}

struct Buf {
  std::string elem;
  std::vector<int64_t> shape;
};

struct Karg {
  enum Kind { Param, Result, Workspace, Rows } kind;
  int index;
};

// A kernel the group runs before its main kernel (an operand re-layout into
// the workspace, e.g. the [N, K] copy of a [K, N] matmul operand).
struct PreLaunch {
  std::string kernel;
  hipFunction_t fn = nullptr;
  hfr_launch_cfg cfg{};
  std::vector<Karg> kargs;
};

struct hfr_group {
  std::string func, kernel, hsaco;
  std::vector<PreLaunch> pre;
  hfr_module *mod = nullptr;
  hipFunction_t fn = nullptr;
  hfr_launch_cfg cfg{};
  uint64_t wsBytes = 0;
  bool wsZero = false;
  uint64_t algoBytes = 0, algoOps = 0;
  // runtime row count (manifest `rows_dyn a b c cap`): grid.x =
  // min(ceil(R * a / b) * c, cap) (cap 0: none), or the static grid when a is 0
  bool rowsDyn = false;
  int64_t rowsA = 0, rowsB = 1, rowsC = 1, rowsCap = 0;
  std::vector<std::string> paramRoles;
  std::vector<Buf> paramBufs, resultBufs;
  std::vector<int> resultTied;
  std::vector<Karg> kargs;
  void *ownWs = nullptr;
  int ownWsDevice = -1;
  // dense staging copies of strided memref views (hfr_group_launch_memref)
  void *stage = nullptr;
  size_t stageBytes = 0;
  int stageDevice = -1;
};

// A buffer binding inside a launch program: program parameter, workspace
// temporary or program result.
struct Binding {
  enum Kind { Param, Temp, Result } kind;
  int index;
};

struct ProgramStep {
  hfr_group *group = nullptr;
  std::vector<Binding> args, results;
};

struct hfr_program {
  std::string name;
  std::vector<std::string> paramRoles;  // in | out | inout | scalar
  std::vector<int> resultParam;         // param a result is written into, or -1
  std::vector<uint64_t> tempOffset;
  uint64_t wsBytes = 0;
  std::vector<ProgramStep> steps;
  void *ownWs = nullptr;
  int ownWsDevice = -1;
};

namespace {

constexpr size_t HFR_MAX_KARGS = 64;

thread_local std::string g_err;

int fail(int code, const std::string &msg) {
  g_err = msg;
  return code;
}

int hipFail(hipError_t e, const char *what) {
  // the error is reported through the return code; clear HIP's last-error
  // state so it does not resurface in the caller's next, unrelated HIP call
  (void)hipGetLastError();
  return fail(HFR_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

std::string dirOf(const std::string &p) {
  auto s = p.find_last_of('/');
  return s == std::string::npos ? "." : p.substr(0, s);
}

bool parseKarg(const std::string &k, Karg &a) {
  if (k == "ws") { a.kind = Karg::Workspace; a.index = 0; return true; }
  if (k == "rows") { a.kind = Karg::Rows; a.index = 0; return true; }
  if (k.rfind("param:", 0) == 0) { a.kind = Karg::Param; a.index = std::atoi(k.c_str() + 6); return true; }
  if (k.rfind("result:", 0) == 0) { a.kind = Karg::Result; a.index = std::atoi(k.c_str() + 7); return true; }
  return false;
}

// Parses one manifest block (lines after "hfr-manifest 1" until the next one).
int parseBlock(const std::vector<std::string> &lines, hfr_group &g) {
  for (const auto &ln : lines) {
    std::istringstream is(ln);
    std::string key;
    is >> key;
    if (key == "func") is >> g.func;
    else if (key == "kernel") is >> g.kernel;
    else if (key == "hsaco") is >> g.hsaco;
    else if (key == "grid") is >> g.cfg.grid[0] >> g.cfg.grid[1] >> g.cfg.grid[2];
    else if (key == "block") is >> g.cfg.block[0] >> g.cfg.block[1] >> g.cfg.block[2];
    else if (key == "lds") is >> g.cfg.lds_bytes;
    else if (key == "workspace") { int z = 0; is >> g.wsBytes >> z; g.wsZero = z != 0; }
    else if (key == "algo_bytes") is >> g.algoBytes;
    else if (key == "algo_ops") is >> g.algoOps;
    else if (key == "rows_dyn") {
      is >> g.rowsA >> g.rowsB >> g.rowsC >> g.rowsCap;
      g.rowsDyn = true;
      if (g.rowsA < 0 || g.rowsB <= 0 || g.rowsC <= 0 || g.rowsCap < 0)
        return fail(HFR_ERR_MANIFEST, "bad rows_dyn line: " + ln);
    }
    else if (key == "param" || key == "result") {
      int i, tied = -1, rank = 0;
      std::string role;
      Buf b;
      is >> i;
      if (key == "param") is >> role;
      else is >> tied;
      is >> b.elem >> rank;
      for (int d = 0; d < rank && is; ++d) { int64_t x; is >> x; b.shape.push_back(x); }
      if (key == "param") { g.paramRoles.push_back(role); g.paramBufs.push_back(b); }
      else { g.resultTied.push_back(tied); g.resultBufs.push_back(b); }
    }
    else if (key == "karg") {
      std::string k;
      is >> k;
      Karg a;
      if (!parseKarg(k, a)) return fail(HFR_ERR_MANIFEST, "bad karg '" + k + "'");
      g.kargs.push_back(a);
    }
    else if (key == "pre") {
      // pre <kernel> <grid x y z> <block x y z> <n> <karg>...
      PreLaunch pl;
      int n = 0;
      is >> pl.kernel >> pl.cfg.grid[0] >> pl.cfg.grid[1] >> pl.cfg.grid[2] >> pl.cfg.block[0] >> pl.cfg.block[1] >>
          pl.cfg.block[2] >> n;
      for (int i = 0; i < n && is; ++i) {
        std::string k;
        is >> k;
        Karg a;
        if (!parseKarg(k, a)) return fail(HFR_ERR_MANIFEST, "bad karg '" + k + "'");
        pl.kargs.push_back(a);
      }
      if (!pl.cfg.grid[0] || !pl.cfg.block[0]) return fail(HFR_ERR_MANIFEST, "pre kernel without launch shape");
      g.pre.push_back(pl);
    }
    if (is.fail()) return fail(HFR_ERR_MANIFEST, "malformed manifest line: " + ln);
  }
  if (g.kernel.empty() || g.hsaco.empty()) return fail(HFR_ERR_MANIFEST, "manifest block without kernel/hsaco");
  if (!g.cfg.block[0] || !g.cfg.grid[0]) return fail(HFR_ERR_MANIFEST, "manifest block without launch shape");
  auto check = [&](const std::vector<Karg> &ks) {
    for (auto &a : ks) {
      if (a.kind == Karg::Param && (a.index < 0 || a.index >= (int)g.paramRoles.size()))
        return fail(HFR_ERR_MANIFEST, "karg refers to a missing param");
      if (a.kind == Karg::Result && (a.index < 0 || a.index >= (int)g.resultTied.size()))
        return fail(HFR_ERR_MANIFEST, "karg refers to a missing result");
      if (a.kind == Karg::Workspace && !g.wsBytes) return fail(HFR_ERR_MANIFEST, "karg ws without a workspace");
      if (a.kind == Karg::Rows && !g.rowsDyn) return fail(HFR_ERR_MANIFEST, "karg rows without rows_dyn");
    }
    return (int)HFR_OK;
  };
  int rc = check(g.kargs);
  for (auto &pl : g.pre)
    if (!rc) rc = check(pl.kargs);
  return rc;
}

// Splits a manifest into group blocks ("hfr-manifest 1") and launch-program
// blocks ("hfr-program 1").
int readManifest(const char *path, std::vector<std::vector<std::string>> &groups,
                 std::vector<std::vector<std::string>> &programs) {
  std::ifstream f(path);
  if (!f) return fail(HFR_ERR_IO, std::string("cannot open manifest ") + path);
  std::vector<std::string> *cur = nullptr;
  std::string ln;
  while (std::getline(f, ln)) {
    if (ln.rfind("hfr-manifest", 0) == 0) {
      if (ln != "hfr-manifest 1") return fail(HFR_ERR_MANIFEST, "unsupported manifest version: " + ln);
      groups.emplace_back();
      cur = &groups.back();
      continue;
    }
    if (ln.rfind("hfr-program", 0) == 0) {
      if (ln != "hfr-program 1") return fail(HFR_ERR_MANIFEST, "unsupported program version: " + ln);
      programs.emplace_back();
      cur = &programs.back();
      continue;
    }
    if (!cur) return fail(HFR_ERR_MANIFEST, "manifest must start with 'hfr-manifest 1'");
    if (!ln.empty()) cur->push_back(ln);
  }
  if (groups.empty() && programs.empty()) return fail(HFR_ERR_MANIFEST, "empty manifest");
  return HFR_OK;
}

int launchRaw(hipFunction_t fn, const hfr_launch_cfg &cfg, const uint64_t *args, size_t nargs, void *stream) {
  // the argument buffer is copied by hipModuleLaunchKernel; a fixed array
  // keeps launches free of heap allocation
  uint64_t buf[HFR_MAX_KARGS];
  if (nargs > HFR_MAX_KARGS) return fail(HFR_ERR_INVALID, "too many kernel arguments");
  for (size_t i = 0; i < nargs; ++i) buf[i] = args[i];
  size_t sz = nargs * sizeof(uint64_t);
  void *extra[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, nargs ? buf : nullptr, HIP_LAUNCH_PARAM_BUFFER_SIZE, &sz,
                   HIP_LAUNCH_PARAM_END};
  hipError_t e = hipModuleLaunchKernel(fn, cfg.grid[0], cfg.grid[1] ? cfg.grid[1] : 1, cfg.grid[2] ? cfg.grid[2] : 1,
                                       cfg.block[0], cfg.block[1] ? cfg.block[1] : 1, cfg.block[2] ? cfg.block[2] : 1,
                                       cfg.lds_bytes, (hipStream_t)stream, nullptr, extra);
  if (e != hipSuccess) return hipFail(e, "hipModuleLaunchKernel");
  return HFR_OK;
}

// Checks a group launch's arguments (counts, null pointers).
int checkGroupArgs(const hfr_group *g, const uint64_t *params, size_t nparams, void *const *results, size_t nresults) {
  if (!g) return fail(HFR_ERR_INVALID, "null group");
  if (nparams != g->paramRoles.size())
    return fail(HFR_ERR_INVALID, "group @" + g->func + " takes " + std::to_string(g->paramRoles.size()) +
                                     " arguments, got " + std::to_string(nparams));
  if (nresults != g->resultTied.size())
    return fail(HFR_ERR_INVALID, "group @" + g->func + " has " + std::to_string(g->resultTied.size()) +
                                     " results, got " + std::to_string(nresults));
  if (nparams && !params) return fail(HFR_ERR_INVALID, "null params array");
  for (size_t i = 0; i < nparams; ++i)
    if (g->paramRoles[i] != "scalar" && params[i] == 0)
      return fail(HFR_ERR_INVALID, "null device pointer for argument " + std::to_string(i));
  for (size_t i = 0; i < nresults; ++i)
    if (g->resultTied[i] < 0 && (!results || !results[i]))
      return fail(HFR_ERR_INVALID, "null device pointer for result " + std::to_string(i));
  return HFR_OK;
}

// Assembles the kernel arguments (params, own result buffers, workspace) and
// launches the group's kernels: its pre kernels in order, then the main one,
// all on `stream`.
int launchGroup(const hfr_group *g, const uint64_t *params, void *const *results, void *ws, void *stream,
                int64_t rows = -1) {
  auto launch = [&](hipFunction_t fn, hfr_launch_cfg cfg, const std::vector<Karg> &kargs) {
    if (g->rowsDyn && g->rowsA > 0) {
      int64_t blocks = (rows * g->rowsA + g->rowsB - 1) / g->rowsB * g->rowsC;
      if (g->rowsCap > 0 && blocks > g->rowsCap) blocks = g->rowsCap;
      cfg.grid[0] = (unsigned)(blocks > 0 ? blocks : 1);
    }
    uint64_t args[HFR_MAX_KARGS];
    if (kargs.size() > HFR_MAX_KARGS) return fail(HFR_ERR_INVALID, "too many kernel arguments");
    size_t n = 0;
    for (auto &a : kargs) {
      switch (a.kind) {
      case Karg::Param: args[n++] = params[a.index]; break;
      case Karg::Result: args[n++] = (uint64_t)(uintptr_t)results[a.index]; break;
      case Karg::Workspace: args[n++] = (uint64_t)(uintptr_t)ws; break;
      case Karg::Rows: args[n++] = (uint64_t)rows; break;
      }
    }
    return launchRaw(fn, cfg, args, n, stream);
  };
  for (auto &pl : g->pre) {
    const int rc = launch(pl.fn, pl.cfg, pl.kargs);
    if (rc) return rc;
  }
  return launch(g->fn, g->cfg, g->kargs);
}

} // namespace

extern "C" {

const char *hfr_version(void) { return "hfr 0.1 (gfx950)"; }
const char *hfr_last_error(void) { return g_err.c_str(); }

int hfr_module_load(const char *hsaco_path, hfr_module_t *out) {
  if (!hsaco_path || !out) return fail(HFR_ERR_INVALID, "null argument to hfr_module_load");
  std::ifstream probe(hsaco_path, std::ios::binary);
  if (!probe) return fail(HFR_ERR_IO, std::string("cannot open code object ") + hsaco_path);
  auto m = std::make_unique<hfr_module>();
  hipError_t e = hipModuleLoad(&m->mod, hsaco_path);
  if (e != hipSuccess) return hipFail(e, "hipModuleLoad");
  m->path = hsaco_path;
  *out = m.release();
  return HFR_OK;
}

int hfr_module_unload(hfr_module_t m) {
  if (!m) return fail(HFR_ERR_INVALID, "null module");
  if (--m->refs > 0) return HFR_OK;
  hipError_t e = hipModuleUnload(m->mod);
  delete m;
  if (e != hipSuccess) return hipFail(e, "hipModuleUnload");
  return HFR_OK;
}

int hfr_kernel_get(hfr_module_t m, const char *name, hfr_kernel_t *out) {
  if (!m || !name || !out) return fail(HFR_ERR_INVALID, "null argument to hfr_kernel_get");
  hipFunction_t fn;
  hipError_t e = hipModuleGetFunction(&fn, m->mod, name);
  if (e != hipSuccess) {
    (void)hipGetLastError(); // reported here, not by the caller's next HIP call
    return fail(HFR_ERR_NOT_FOUND, std::string("kernel '") + name + "' not in " + m->path);
  }
  auto k = new hfr_kernel();
  k->fn = fn;
  k->owner = m;
  *out = k;
  return HFR_OK;
}

int hfr_launch(hfr_kernel_t k, const hfr_launch_cfg *cfg, const uint64_t *args, size_t nargs, void *stream) {
  if (!k || !cfg || (nargs && !args)) return fail(HFR_ERR_INVALID, "null argument to hfr_launch");
  return launchRaw(k->fn, *cfg, args, nargs, stream);
}

int hfr_group_load(const char *manifest_path, const char *func, hfr_group_t *out) {
  if (!manifest_path || !out) return fail(HFR_ERR_INVALID, "null argument to hfr_group_load");
  std::vector<std::vector<std::string>> blocks, programs;
  int rc = readManifest(manifest_path, blocks, programs);
  if (rc) return rc;
  if (blocks.empty()) return fail(HFR_ERR_MANIFEST, "manifest holds no group");
  auto g = std::make_unique<hfr_group>();
  bool found = false;
  for (auto &b : blocks) {
    hfr_group cand;
    int rc = parseBlock(b, cand);
    if (rc) return rc;
    if (!func || cand.func == func) {
      if (!func && blocks.size() > 1) return fail(HFR_ERR_INVALID, "manifest holds several groups; name one");
      *g = cand;
      found = true;
      break;
    }
  }
  if (!found) return fail(HFR_ERR_NOT_FOUND, std::string("group '") + (func ? func : "") + "' not in manifest");
  std::string hsaco = g->hsaco[0] == '/' ? g->hsaco : dirOf(manifest_path) + "/" + g->hsaco;
  rc = hfr_module_load(hsaco.c_str(), &g->mod);
  if (rc) return rc;
  hipError_t e = hipModuleGetFunction(&g->fn, g->mod->mod, g->kernel.c_str());
  for (size_t i = 0; e == hipSuccess && i < g->pre.size(); ++i)
    e = hipModuleGetFunction(&g->pre[i].fn, g->mod->mod, g->pre[i].kernel.c_str());
  if (e != hipSuccess) {
    (void)hipGetLastError();
    hfr_module_unload(g->mod);
    return fail(HFR_ERR_NOT_FOUND, "kernel of group '" + g->func + "' not in " + hsaco);
  }
  // the group's own workspace lives on the device current at load time, so
  // that launches stay asynchronous
  if (g->wsBytes) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    e = hipMalloc(&g->ownWs, g->wsBytes);
    if (e == hipSuccess) e = hipMemset(g->ownWs, 0, g->wsBytes);
    if (e != hipSuccess) {
      if (g->ownWs) (void)hipFree(g->ownWs);
      hfr_module_unload(g->mod);
      return hipFail(e, "workspace allocation");
    }
    g->ownWsDevice = dev;
  }
  *out = g.release();
  return HFR_OK;
}

int hfr_group_unload(hfr_group_t g) {
  if (!g) return fail(HFR_ERR_INVALID, "null group");
  int rc = HFR_OK;
  if (g->ownWs) {
    int cur = 0;
    (void)hipGetDevice(&cur);
    if (g->ownWsDevice >= 0) (void)hipSetDevice(g->ownWsDevice);
    hipError_t e = hipFree(g->ownWs);
    (void)hipSetDevice(cur);
    if (e != hipSuccess) rc = hipFail(e, "hipFree(workspace)");
  }
  if (g->stage) {
    int cur = 0;
    (void)hipGetDevice(&cur);
    if (g->stageDevice >= 0) (void)hipSetDevice(g->stageDevice);
    hipError_t e = hipFree(g->stage);
    (void)hipSetDevice(cur);
    if (e != hipSuccess && !rc) rc = hipFail(e, "hipFree(staging)");
  }
  if (g->mod) {
    int r2 = hfr_module_unload(g->mod);
    if (!rc) rc = r2;
  }
  delete g;
  return rc;
}

int hfr_group_info_get(hfr_group_t g, hfr_group_info *info) {
  if (!g || !info) return fail(HFR_ERR_INVALID, "null argument to hfr_group_info_get");
  info->nparams = (int)g->paramRoles.size();
  info->nresults = (int)g->resultTied.size();
  info->nkargs = (int)g->kargs.size();
  info->workspace_bytes = g->wsBytes;
  info->algo_bytes = g->algoBytes;
  info->algo_ops = g->algoOps;
  info->cfg = g->cfg;
  return HFR_OK;
}

int hfr_group_launch(hfr_group_t g, const uint64_t *params, size_t nparams, void *const *results, size_t nresults,
                     void *workspace, void *stream) {
  if (g && g->rowsDyn)
    return fail(HFR_ERR_INVALID, "group @" + g->func + " takes its row count at launch (hfr_group_launch_rows)");
  return hfr_group_launch_rows(g, params, nparams, results, nresults, -1, workspace, stream);
}

int hfr_group_launch_rows(hfr_group_t g, const uint64_t *params, size_t nparams, void *const *results, size_t nresults,
                          int64_t rows, void *workspace, void *stream) {
  if (g && !g->rowsDyn && rows != -1)
    return fail(HFR_ERR_INVALID, "group @" + g->func + " has a static row count");
  if (g && g->rowsDyn && rows < 0) return fail(HFR_ERR_INVALID, "negative row count for group @" + g->func);
  int rc = checkGroupArgs(g, params, nparams, results, nresults);
  if (rc) return rc;
  if (g->rowsDyn && rows == 0) return HFR_OK; // nothing to do
  void *ws = workspace;
  if (g->wsBytes && !ws) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (dev != g->ownWsDevice) return fail(HFR_ERR_INVALID, "group workspace belongs to another device");
    ws = g->ownWs;
  }
  return launchGroup(g, params, results, ws, stream, rows);
}

} // extern "C"

namespace {

int parseBinding(const std::string &s, const hfr_program &p, Binding &b) {
  if (s.size() < 2) return fail(HFR_ERR_MANIFEST, "bad binding '" + s + "'");
  int i = std::atoi(s.c_str() + 1);
  switch (s[0]) {
  case 'p': b = {Binding::Param, i}; return i >= 0 && i < (int)p.paramRoles.size() ? HFR_OK : fail(HFR_ERR_MANIFEST, "binding " + s + " out of range");
  case 't': b = {Binding::Temp, i}; return i >= 0 && i < (int)p.tempOffset.size() ? HFR_OK : fail(HFR_ERR_MANIFEST, "binding " + s + " out of range");
  case 'r': b = {Binding::Result, i}; return i >= 0 && i < (int)p.resultParam.size() ? HFR_OK : fail(HFR_ERR_MANIFEST, "binding " + s + " out of range");
  default: return fail(HFR_ERR_MANIFEST, "bad binding '" + s + "'");
  }
}

bool sameBinding(const Binding &a, const Binding &b) { return a.kind == b.kind && a.index == b.index; }

void freeProgram(hfr_program *p) {
  for (auto &st : p->steps)
    if (st.group) hfr_group_unload(st.group);
  if (p->ownWs) {
    int cur = 0;
    (void)hipGetDevice(&cur);
    if (p->ownWsDevice >= 0) (void)hipSetDevice(p->ownWsDevice);
    (void)hipFree(p->ownWs);
    (void)hipSetDevice(cur);
  }
  delete p;
}

} // namespace

extern "C" {

int hfr_program_load(const char *manifest_path, const char *name, hfr_program_t *out) {
  if (!manifest_path || !out) return fail(HFR_ERR_INVALID, "null argument to hfr_program_load");
  std::vector<std::vector<std::string>> groups, programs;
  int rc = readManifest(manifest_path, groups, programs);
  if (rc) return rc;
  const std::vector<std::string> *blk = nullptr;
  for (auto &b : programs) {
    std::string pname;
    for (auto &ln : b)
      if (ln.rfind("program ", 0) == 0) pname = ln.substr(8);
    if (!name || pname == name) {
      if (!name && programs.size() > 1) return fail(HFR_ERR_INVALID, "manifest holds several programs; name one");
      blk = &b;
      break;
    }
  }
  if (!blk) return fail(HFR_ERR_NOT_FOUND, std::string("program '") + (name ? name : "") + "' not in manifest");
  auto *p = new hfr_program();
  std::vector<std::vector<std::string>> stepLines;
  for (auto &ln : *blk) {
    std::istringstream is(ln);
    std::string key;
    is >> key;
    if (key == "program") is >> p->name;
    else if (key == "pworkspace") is >> p->wsBytes;
    else if (key == "pparam") { int i; std::string role; is >> i >> role; p->paramRoles.push_back(role); }
    else if (key == "presult") {
      int i; std::string role;
      is >> i >> role;
      p->resultParam.push_back(role[0] == 'p' ? std::atoi(role.c_str() + 1) : -1);
    } else if (key == "ptemp") { int i; uint64_t off; is >> i >> off; p->tempOffset.push_back(off); }
    else if (key == "pstep") {
      std::vector<std::string> toks;
      std::string t;
      while (is >> t) toks.push_back(t);
      stepLines.push_back(toks);
    }
    if (is.fail() && key != "pstep") { freeProgram(p); return fail(HFR_ERR_MANIFEST, "malformed program line: " + ln); }
  }
  for (int rp : p->resultParam)
    if (rp >= (int)p->paramRoles.size()) { freeProgram(p); return fail(HFR_ERR_MANIFEST, "program result bound to a missing param"); }
  // pstep <group> <kind> <nargs> <bindings...> <nresults> <bindings...>
  for (auto &toks : stepLines) {
    ProgramStep st;
    size_t k = 2;
    auto bad = [&]() { freeProgram(p); return fail(HFR_ERR_MANIFEST, "malformed pstep line"); };
    if (toks.size() < 4) return bad();
    int na = std::atoi(toks[k++].c_str());
    if (na < 0 || k + na >= toks.size()) return bad();
    for (int i = 0; i < na; ++i) {
      Binding b;
      if ((rc = parseBinding(toks[k++], *p, b))) { freeProgram(p); return rc; }
      st.args.push_back(b);
    }
    int nr = std::atoi(toks[k++].c_str());
    if (nr < 0 || k + nr != toks.size()) return bad();
    for (int i = 0; i < nr; ++i) {
      Binding b;
      if ((rc = parseBinding(toks[k++], *p, b))) { freeProgram(p); return rc; }
      st.results.push_back(b);
    }
    p->steps.push_back(st);
    if ((rc = hfr_group_load(manifest_path, toks[0].c_str(), &p->steps.back().group))) {
      p->steps.back().group = nullptr;
      freeProgram(p);
      return rc;
    }
    hfr_group *g = p->steps.back().group;
    if (g->paramRoles.size() != st.args.size() || g->resultTied.size() != st.results.size()) {
      freeProgram(p);
      return fail(HFR_ERR_MANIFEST, "step @" + toks[0] + " does not match its group's signature");
    }
    // a result the group writes into one of its arguments must be bound to
    // that argument's buffer
    for (size_t j = 0; j < st.results.size(); ++j) {
      int t = g->resultTied[j];
      if (t >= 0 && !sameBinding(st.args[t], st.results[j])) {
        freeProgram(p);
        return fail(HFR_ERR_MANIFEST, "step @" + toks[0] + " result " + std::to_string(j) + " is written into argument " +
                                          std::to_string(t) + " but bound elsewhere");
      }
    }
  }
  if (p->wsBytes) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    hipError_t e = hipMalloc(&p->ownWs, p->wsBytes);
    if (e != hipSuccess) {
      p->ownWs = nullptr;
      freeProgram(p);
      return hipFail(e, "hipMalloc(program workspace)");
    }
    p->ownWsDevice = dev;
  }
  *out = p;
  return HFR_OK;
}

int hfr_program_unload(hfr_program_t p) {
  if (!p) return fail(HFR_ERR_INVALID, "null program");
  freeProgram(p);
  return HFR_OK;
}

int hfr_program_info_get(hfr_program_t p, hfr_program_info *info) {
  if (!p || !info) return fail(HFR_ERR_INVALID, "null argument to hfr_program_info_get");
  info->nparams = (int)p->paramRoles.size();
  info->nresults = (int)p->resultParam.size();
  info->nsteps = (int)p->steps.size();
  info->workspace_bytes = p->wsBytes;
  return HFR_OK;
}

int hfr_program_launch(hfr_program_t p, const uint64_t *params, size_t nparams, void *const *results, size_t nresults,
                       void *workspace, void *stream) {
  if (!p) return fail(HFR_ERR_INVALID, "null program");
  if (nparams != p->paramRoles.size())
    return fail(HFR_ERR_INVALID, "program @" + p->name + " takes " + std::to_string(p->paramRoles.size()) +
                                     " arguments, got " + std::to_string(nparams));
  if (nresults != p->resultParam.size())
    return fail(HFR_ERR_INVALID, "program @" + p->name + " has " + std::to_string(p->resultParam.size()) +
                                     " results, got " + std::to_string(nresults));
  if (nparams && !params) return fail(HFR_ERR_INVALID, "null params array");
  for (size_t i = 0; i < nparams; ++i)
    if (p->paramRoles[i] != "scalar" && params[i] == 0)
      return fail(HFR_ERR_INVALID, "null device pointer for argument " + std::to_string(i));
  for (size_t i = 0; i < nresults; ++i)
    if (p->resultParam[i] < 0 && (!results || !results[i]))
      return fail(HFR_ERR_INVALID, "null device pointer for result " + std::to_string(i));
  char *ws = (char *)workspace;
  if (p->wsBytes && !ws) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (dev != p->ownWsDevice) return fail(HFR_ERR_INVALID, "program workspace belongs to another device");
    ws = (char *)p->ownWs;
  }
  auto resolve = [&](const Binding &b) -> uint64_t {
    switch (b.kind) {
    case Binding::Param: return params[b.index];
    case Binding::Temp: return (uint64_t)(uintptr_t)(ws + p->tempOffset[b.index]);
    case Binding::Result:
      return p->resultParam[b.index] >= 0 ? params[p->resultParam[b.index]] : (uint64_t)(uintptr_t)results[b.index];
    }
    return 0;
  };
  std::vector<uint64_t> args;
  std::vector<void *> res;
  for (auto &st : p->steps) {
    args.clear();
    res.clear();
    for (auto &b : st.args) args.push_back(resolve(b));
    for (auto &b : st.results) res.push_back((void *)(uintptr_t)resolve(b));
    int rc = hfr_group_launch(st.group, args.data(), args.size(), res.data(), res.size(), nullptr, stream);
    if (rc) return rc;
  }
  return HFR_OK;
}

} // extern "C"

// ---------------------------------------------------------------------------
// MLIR C-interface entry: ranked memref descriptors in the IR's argument order
// (the layout `_mlir_ciface_*` functions receive; the reference runner's
// UnrankedMemRefType wraps a pointer to one of these,
// bishengir/lib/ExecutionEngine/BiShengIRRunnerUtils.cpp:99-110).
// { T *allocated; T *aligned; int64_t offset; int64_t sizes[R]; int64_t strides[R]; }
namespace {

constexpr int HFR_MAX_RANK = 8;

// A view of a memref descriptor: base address, sizes and element strides.
struct View {
  char *base = nullptr;
  int rank = 0;
  int64_t sizes[HFR_MAX_RANK] = {}, strides[HFR_MAX_RANK] = {};
  bool dense = true;
  int64_t numel = 1;
};

// A dim the group gives as -1 (a runtime row count) takes the descriptor's
// size, which must agree with every other such dim (`rows`, -1 until the
// first).
int readDesc(const Buf &b, const void *desc, const char *what, size_t idx, View &v, int64_t &rows) {
  if (!desc) return fail(HFR_ERR_INVALID, std::string("null descriptor for ") + what + " " + std::to_string(idx));
  const char *d = (const char *)desc;
  char *aligned = *(char *const *)(d + sizeof(void *));
  const int64_t offset = *(const int64_t *)(d + 2 * sizeof(void *));
  const int64_t *sizes = (const int64_t *)(d + 2 * sizeof(void *) + sizeof(int64_t));
  const int64_t *strides = sizes + b.shape.size();
  if (b.shape.size() > (size_t)HFR_MAX_RANK)
    return fail(HFR_ERR_INVALID, std::string(what) + " " + std::to_string(idx) + ": rank above " + std::to_string(HFR_MAX_RANK));
  v.rank = (int)b.shape.size();
  int64_t expect = 1;
  for (int k = v.rank; k-- > 0;) {
    if (b.shape[k] == -1) {
      if (sizes[k] < 0) return fail(HFR_ERR_INVALID, std::string(what) + " " + std::to_string(idx) + ": negative size");
      if (rows >= 0 && sizes[k] != rows)
        return fail(HFR_ERR_INVALID, std::string(what) + " " + std::to_string(idx) + ": " + std::to_string(sizes[k]) +
                                         " rows, another view has " + std::to_string(rows));
      rows = sizes[k];
    } else if (sizes[k] != b.shape[k])
      return fail(HFR_ERR_INVALID, std::string(what) + " " + std::to_string(idx) + ": size " + std::to_string(sizes[k]) +
                                       " in dim " + std::to_string(k) + ", the group expects " + std::to_string(b.shape[k]));
    v.sizes[k] = sizes[k];
    v.strides[k] = strides[k];
    if (sizes[k] != 1 && strides[k] != expect) v.dense = false;
    expect *= sizes[k];
    v.numel *= sizes[k];
  }
  if (!aligned) return fail(HFR_ERR_INVALID, std::string("null aligned pointer for ") + what + " " + std::to_string(idx));
  if (offset < 0) return fail(HFR_ERR_INVALID, std::string("negative offset for ") + what + " " + std::to_string(idx));
  v.base = aligned + offset * elemSize(b.elem);
  return HFR_OK;
}

// A written view must not alias itself: ordered by stride, each dim's stride
// covers the extent of the dims below it (zero or negative strides refused).
bool nonOverlapping(const View &v) {
  int order[HFR_MAX_RANK];
  int n = 0;
  for (int k = 0; k < v.rank; ++k)
    if (v.sizes[k] != 1) order[n++] = k;
  std::sort(order, order + n, [&](int a, int b) { return v.strides[a] < v.strides[b]; });
  int64_t extent = 1;
  for (int i = 0; i < n; ++i) {
    const int k = order[i];
    if (v.strides[k] < extent) return false;
    extent = v.strides[k] * v.sizes[k];
  }
  return true;
}

struct ViewArg {
  int rank;
  int64_t sizes[HFR_MAX_RANK], strides[HFR_MAX_RANK];
};

// Element i of the dense row-major order <-> the view's element at the
// same coordinates: GATHER copies view -> dense, otherwise dense -> view.
// Consecutive threads take consecutive dense elements.
template <typename T, bool GATHER>
__global__ void hfr_strided_copy(T *view, T *dense, ViewArg v, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    int64_t r = i, off = 0;
    for (int k = v.rank - 1; k >= 0; --k) {
      off += (r % v.sizes[k]) * v.strides[k];
      r /= v.sizes[k];
    }
    if (GATHER) dense[i] = view[off];
    else view[off] = dense[i];
  }
}

int stridedCopy(const View &v, int eb, void *dense, bool gather, hipStream_t st) {
  ViewArg a;
  a.rank = v.rank;
  for (int k = 0; k < v.rank; ++k) { a.sizes[k] = v.sizes[k]; a.strides[k] = v.strides[k]; }
  if (v.numel == 0) return HFR_OK;
  const unsigned block = 256, grid = (unsigned)std::min<int64_t>((v.numel + block - 1) / block, 65536);
#define HFR_COPY(T)                                                                                             \
  do {                                                                                                          \
    if (gather)                                                                                                 \
      hipLaunchKernelGGL((hfr_strided_copy<T, true>), dim3(grid), dim3(block), 0, st, (T *)v.base, (T *)dense, a, v.numel); \
    else                                                                                                        \
      hipLaunchKernelGGL((hfr_strided_copy<T, false>), dim3(grid), dim3(block), 0, st, (T *)v.base, (T *)dense, a, v.numel); \
  } while (0)
  switch (eb) {
  case 1: HFR_COPY(uint8_t); break;
  case 2: HFR_COPY(uint16_t); break;
  case 4: HFR_COPY(uint32_t); break;
  case 8: HFR_COPY(uint64_t); break;
  default: return fail(HFR_ERR_INVALID, "element size " + std::to_string(eb));
  }
#undef HFR_COPY
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? HFR_OK : hipFail(e, "strided copy launch");
}

} // namespace

extern "C" int hfr_group_launch_memref(hfr_group_t g, void *const *descs, size_t ndescs, void *stream) {
  if (!g) return fail(HFR_ERR_INVALID, "null group");
  size_t nown = 0;
  for (int t : g->resultTied) nown += t < 0;
  if (ndescs != g->paramRoles.size() + nown)
    return fail(HFR_ERR_INVALID, "group @" + g->func + " takes " + std::to_string(g->paramRoles.size() + nown) +
                                     " descriptors, got " + std::to_string(ndescs));
  if (ndescs && !descs) return fail(HFR_ERR_INVALID, "null descriptor array");
  uint64_t params[HFR_MAX_KARGS];
  void *results[HFR_MAX_KARGS];
  if (g->paramRoles.size() > HFR_MAX_KARGS || g->resultTied.size() > HFR_MAX_KARGS)
    return fail(HFR_ERR_INVALID, "too many group arguments");
  // a strided view is staged through a dense copy: gathered before the launch
  // when the group reads it, scattered back after when the group writes it
  struct Staged {
    View v;
    int eb;
    size_t off;
    bool read, written;
  };
  std::vector<Staged> staged;
  std::vector<std::pair<int, size_t>> stagedParam, stagedResult; // index -> staged slot
  size_t total = 0;
  int64_t rows = -1; // a runtime row count, read from the descriptors
  auto stage = [&](const View &v, const std::string &elem, bool read, bool written, const char *what, size_t idx) -> int {
    if (written && !nonOverlapping(v))
      return fail(HFR_ERR_INVALID, std::string(what) + " " + std::to_string(idx) + ": the written view overlaps itself");
    const int eb = elemSize(elem);
    staged.push_back({v, eb, total, read, written});
    total += ((size_t)v.numel * eb + 255) & ~(size_t)255;
    return HFR_OK;
  };
  for (size_t i = 0; i < g->paramRoles.size(); ++i) {
    if (g->paramRoles[i] == "scalar") {
      if (!descs[i]) return fail(HFR_ERR_INVALID, "null scalar pointer for argument " + std::to_string(i));
      uint64_t bits = 0;
      std::memcpy(&bits, descs[i], (size_t)elemSize(g->paramBufs[i].elem));
      params[i] = bits;
      continue;
    }
    View v;
    int rc = readDesc(g->paramBufs[i], descs[i], "argument", i, v, rows);
    if (rc) return rc;
    params[i] = (uint64_t)(uintptr_t)v.base;
    if (!v.dense) {
      const std::string &role = g->paramRoles[i];
      rc = stage(v, g->paramBufs[i].elem, role != "out", role != "in", "argument", i);
      if (rc) return rc;
      stagedParam.push_back({(int)i, staged.size() - 1});
    }
  }
  size_t k = g->paramRoles.size();
  for (size_t j = 0; j < g->resultTied.size(); ++j) {
    results[j] = nullptr;
    if (g->resultTied[j] >= 0) continue;
    View v;
    int rc = readDesc(g->resultBufs[j], descs[k++], "result", j, v, rows);
    if (rc) return rc;
    results[j] = v.base;
    if (!v.dense) {
      rc = stage(v, g->resultBufs[j].elem, false, true, "result", j);
      if (rc) return rc;
      stagedResult.push_back({(int)j, staged.size() - 1});
    }
  }
  if (g->rowsDyn && rows < 0) return fail(HFR_ERR_INVALID, "group @" + g->func + ": no view carries the row count");
  if (!g->rowsDyn) rows = -1;
  if (staged.empty())
    return hfr_group_launch_rows(g, params, g->paramRoles.size(), results, g->resultTied.size(), rows, nullptr, stream);
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hipFail(e, "hipGetDevice");
  if (g->stage && (g->stageBytes < total || g->stageDevice != dev)) {
    // grown (or moved): the old copy is released once the device is idle
    int cur = dev;
    if (g->stageDevice >= 0) (void)hipSetDevice(g->stageDevice);
    e = hipFree(g->stage);
    (void)hipSetDevice(cur);
    g->stage = nullptr;
    g->stageBytes = 0;
    if (e != hipSuccess) return hipFail(e, "hipFree(staging)");
  }
  if (!g->stage) {
    e = hipMalloc(&g->stage, total);
    if (e != hipSuccess) return hipFail(e, "hipMalloc(staging)");
    g->stageBytes = total;
    g->stageDevice = dev;
  }
  hipStream_t st = (hipStream_t)stream;
  char *base = (char *)g->stage;
  for (auto &pi : stagedParam) params[pi.first] = (uint64_t)(uintptr_t)(base + staged[pi.second].off);
  for (auto &rj : stagedResult) results[rj.first] = base + staged[rj.second].off;
  for (auto &sv : staged)
    if (sv.read) {
      int rc = stridedCopy(sv.v, sv.eb, base + sv.off, true, st);
      if (rc) return rc;
    }
  int rc = hfr_group_launch_rows(g, params, g->paramRoles.size(), results, g->resultTied.size(), rows, nullptr, stream);
  if (rc) return rc;
  for (auto &sv : staged)
    if (sv.written) {
      rc = stridedCopy(sv.v, sv.eb, base + sv.off, false, st);
      if (rc) return rc;
    }
  return HFR_OK;
}

// ---------------------------------------------------------------------------
// Launch without allocation.  `scratch` is a device array of this library's
// own code object; each GPU holds its own copy, whose address is looked up
// once per device (hipGetSymbolAddress) and used in place of the array's
// host-side name.
namespace {

static __device__ __align__(256) unsigned char scratch[HFR_SCRATCH_BYTES];

__global__ void hfr_zero_fill(uint4 *p, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

constexpr int HFR_MAX_DEVICES = 64;
std::mutex g_scratchMu;
void *g_scratchPtr[HFR_MAX_DEVICES];

int scratchFor(int dev, void **out) {
  if (dev < 0 || dev >= HFR_MAX_DEVICES) return fail(HFR_ERR_INVALID, "device ordinal out of range");
  std::lock_guard<std::mutex> lk(g_scratchMu);
  if (!g_scratchPtr[dev]) {
    void *ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hipFail(e, "hipGetSymbolAddress(scratch)");
    g_scratchPtr[dev] = ptr;
  }
  *out = g_scratchPtr[dev];
  return HFR_OK;
}

} // namespace

extern "C" uint64_t hfr_scratch_bytes(void) { return HFR_SCRATCH_BYTES; }

extern "C" int hfr_group_launch_noalloc(hfr_group_t g, const uint64_t *params, size_t nparams, void *const *results,
                                        size_t nresults, void *stream) {
  int rc = checkGroupArgs(g, params, nparams, results, nresults);
  if (rc) return rc;
  if (g->rowsDyn)
    return fail(HFR_ERR_INVALID, "group @" + g->func + " takes its row count at launch (hfr_group_launch_rows)");
  if (g->wsBytes > HFR_SCRATCH_BYTES)
    return fail(HFR_ERR_INVALID, "group @" + g->func + " needs " + std::to_string(g->wsBytes) +
                                     " workspace bytes; the static scratch holds " + std::to_string(HFR_SCRATCH_BYTES));
  void *ws = nullptr;
  if (g->wsBytes) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hipFail(e, "hipGetDevice");
    if ((rc = scratchFor(dev, &ws))) return rc;
    if (g->wsZero) {
      // a fill kernel, not hipMemsetAsync: callers may capture this launch
      const size_t n16 = (g->wsBytes + 15) / 16;
      const unsigned blocks = (unsigned)std::min<size_t>((n16 + 255) / 256, 1024);
      hipLaunchKernelGGL(hfr_zero_fill, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (uint4 *)ws, n16);
      e = hipGetLastError();
      if (e != hipSuccess) return hipFail(e, "scratch fill");
    }
  }
  return launchGroup(g, params, results, ws, stream);
}
