// hfc C-ABI: parse -> ConvertHFusionToHIP -> write P.hip / P.manifest ->
// hipcc --genco for gfx950 -> P.hsaco.  See include/hfc.h.
#include "../../../include/hfc.h"
#include "fusion.h"
#include "lower.h"

#include <dlfcn.h>
#include <sys/stat.h>
#include <sys/wait.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <fstream>
#include <sstream>

namespace {

std::map<std::string, std::string> parseOptions(const char *s) {
  std::map<std::string, std::string> m;
  if (!s) return m;
  std::stringstream ss(s);
  std::string item;
  while (std::getline(ss, item, ';')) {
    if (item.empty()) continue;
    auto eq = item.find('=');
    if (eq == std::string::npos) m[item] = "1";
    else m[item.substr(0, eq)] = item.substr(eq + 1);
  }
  return m;
}

void setErr(char *err, size_t n, const std::string &msg) {
  if (!err || !n) return;
  std::snprintf(err, n, "%s", msg.c_str());
}

std::string dirOf(const std::string &p) {
  auto s = p.find_last_of('/');
  return s == std::string::npos ? "." : p.substr(0, s);
}

std::string defaultInclude() {
  Dl_info info;
  if (dladdr((void *)&hfc_version, &info) && info.dli_fname) {
    std::string d = dirOf(info.dli_fname) + "/../csrc/kernels";
    struct stat st;
    if (stat((d + "/hf_ops.h").c_str(), &st) == 0) return d;
  }
  const char *env = std::getenv("HFC_KERNEL_INCLUDE");
  return env ? env : "";
}

bool writeFile(const std::string &path, const std::string &text) {
  std::ofstream f(path, std::ios::binary);
  if (!f) return false;
  f << text;
  return (bool)f;
}

// Runs argv, stderr+stdout captured into `log`; returns exit status.
int runTool(const std::vector<std::string> &argv, std::string &log) {
  char tmpl[] = "/tmp/hfc_log_XXXXXX";
  int fd = mkstemp(tmpl);
  if (fd < 0) { log = "cannot create a temporary file"; return -1; }
  pid_t pid = fork();
  if (pid < 0) { close(fd); unlink(tmpl); log = "fork failed"; return -1; }
  if (pid == 0) {
    dup2(fd, 1);
    dup2(fd, 2);
    std::vector<char *> a;
    for (auto &s : argv) a.push_back(const_cast<char *>(s.c_str()));
    a.push_back(nullptr);
    execvp(a[0], a.data());
    _exit(127);
  }
  int status = 0;
  waitpid(pid, &status, 0);
  close(fd);
  std::ifstream in(tmpl);
  std::stringstream ss;
  ss << in.rdbuf();
  log = ss.str();
  unlink(tmpl);
  if (WIFEXITED(status)) return WEXITSTATUS(status);
  return -1;
}

int compileText(const std::string &text, const char *outPrefix, const char *options, char *err, size_t errlen) {
  if (!outPrefix || !*outPrefix) { setErr(err, errlen, "no output prefix"); return HFC_ERR_IO; }
  auto opts = parseOptions(options);
  std::unique_ptr<hfc::Module> mod;
  try {
    mod = hfc::parseModule(text);
  } catch (const hfc::CompileError &e) {
    setErr(err, errlen, std::string("parse error: ") + e.what());
    return HFC_ERR_PARSE;
  } catch (const std::exception &e) {
    setErr(err, errlen, std::string("parse error (internal): ") + e.what());
    return HFC_ERR_PARSE;
  }
  // dynamic dims: specialised to the sizes the caller names (option dyn=...)
  const bool dynamic = hfc::hasDynamicDims(*mod);
  if (dynamic) {
    try {
      hfc::specializeDynamic(*mod, opts.count("dyn") ? opts["dyn"] : "");
    } catch (const hfc::CompileError &e) {
      setErr(err, errlen, std::string("dynamic shapes: ") + e.what());
      return HFC_ERR_PARSE;
    }
  }
  // fusion front-end: functions that are not one group yet are split into
  // outlined groups plus a launch program
  std::vector<hfc::ProgramPlan> programs;
  try {
    std::string outlined = hfc::outlineFusedGroups(*mod, programs, opts.count("fusion_kind") ? opts["fusion_kind"] : "");
    if (dynamic && !programs.empty())
      throw hfc::CompileError("a function with dynamic dims must be one group (the fusion front-end re-reads "
                              "outlined groups from their source text, which keeps the dynamic types)");
    if (opts.count("emit") && opts["emit"] == "outlined") {
      std::string man;
      for (auto &p : programs) man += hfc::emitProgramManifest(p);
      if (!writeFile(std::string(outPrefix) + ".outlined.mlir", outlined) ||
          !writeFile(std::string(outPrefix) + ".programs", man)) {
        setErr(err, errlen, "cannot write outputs with prefix " + std::string(outPrefix));
        return HFC_ERR_IO;
      }
      return HFC_OK;
    }
    if (!programs.empty()) {
      // kept beside the code object for inspection
      writeFile(std::string(outPrefix) + ".outlined.mlir", outlined);
      mod = hfc::parseModule(outlined);
    }
  } catch (const hfc::CompileError &e) {
    setErr(err, errlen, std::string("fusion error: ") + e.what());
    return HFC_ERR_LOWER;
  } catch (const std::exception &e) {
    setErr(err, errlen, std::string("fusion error (internal): ") + e.what());
    return HFC_ERR_LOWER;
  }
  std::vector<hfc::KernelPlan> plans;
  try {
    hfc::LowerOptions lo;
    if (opts.count("ordered_fp_sums")) lo.orderedFloatSums = opts["ordered_fp_sums"] == "1" ? 1 : 0;
    lo.rmsqKernel = !(opts.count("rmsq_kernel") && opts["rmsq_kernel"] == "0");
    lo.rmsnKernel = opts.count("rmsn_kernel") && opts["rmsn_kernel"] == "1";
    lo.mxExact = opts.count("mx_exact") && opts["mx_exact"] == "1";
    lo.runtimeRows = opts.count("dyn") && opts["dyn"] == "runtime";
    plans = hfc::lowerModule(*mod, lo);
  } catch (const hfc::CompileError &e) {
    setErr(err, errlen, std::string("lowering error: ") + e.what());
    return HFC_ERR_LOWER;
  } catch (const std::exception &e) {
    setErr(err, errlen, std::string("lowering error (internal): ") + e.what());
    return HFC_ERR_LOWER;
  }
  std::string prefix = outPrefix;
  std::string hipPath = prefix + ".hip", hsacoPath = prefix + ".hsaco", manPath = prefix + ".manifest";
  std::string hsacoName = hsacoPath.substr(hsacoPath.find_last_of('/') == std::string::npos ? 0 : hsacoPath.find_last_of('/') + 1);
  std::string man;
  for (auto &p : plans) man += hfc::emitManifest(p, hsacoName);
  for (auto &p : programs) man += hfc::emitProgramManifest(p);
  if (!writeFile(hipPath, hfc::emitTranslationUnit(plans)) || !writeFile(manPath, man)) {
    setErr(err, errlen, "cannot write outputs with prefix " + prefix);
    return HFC_ERR_IO;
  }
  if (opts.count("emit") && opts["emit"] == "hip") return HFC_OK;
  std::string inc = opts.count("include") ? opts["include"] : defaultInclude();
  if (inc.empty()) { setErr(err, errlen, "kernel library headers not found (set include=...)"); return HFC_ERR_IO; }
  std::string hipcc = opts.count("hipcc") ? opts["hipcc"] : "/opt/rocm/bin/hipcc";
  std::string arch = opts.count("arch") ? opts["arch"] : "gfx950";
  std::vector<std::string> argv = {hipcc, "--genco", "--offload-arch=" + arch, "-O3", "-std=c++17",
                                   "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                                   "-I" + inc, "-o", hsacoPath, hipPath};
  std::string log;
  int rc = runTool(argv, log);
  if (rc != 0) {
    if (log.size() > 4000) log = log.substr(0, 4000) + "\n...";
    setErr(err, errlen, "hipcc failed (exit " + std::to_string(rc) + "):\n" + log);
    return HFC_ERR_TOOLCHAIN;
  }
  return HFC_OK;
}

} // namespace

extern "C" {

const char *hfc_version(void) { return "hfc 0.1 (gfx950)"; }

int hfc_compile(const char *ir_text, const char *out_prefix, const char *options, char *err, size_t errlen) {
  if (!ir_text) { setErr(err, errlen, "null IR text"); return HFC_ERR_IO; }
  return compileText(ir_text, out_prefix, options, err, errlen);
}

int hfc_compile_file(const char *mlir_path, const char *out_prefix, const char *options, char *err, size_t errlen) {
  if (!mlir_path) { setErr(err, errlen, "null input path"); return HFC_ERR_IO; }
  std::ifstream f(mlir_path, std::ios::binary);
  if (!f) { setErr(err, errlen, std::string("cannot open input file ") + mlir_path); return HFC_ERR_IO; }
  std::stringstream ss;
  ss << f.rdbuf();
  return compileText(ss.str(), out_prefix, options, err, errlen);
}

} // extern "C"
