// bishengir-compile — device-compile entry kept as the drop-in CLI.
//
// Same shape as the reference tool (bishengir/tools/bishengir-compile/
// bishengir-compile.cpp:103-191): `bishengir-compile <input.mlir> [flags]
// -o <output>`; errors go to stderr as "[ERROR] ..." with EXIT_FAILURE.
// With --target=mi355x (the default of this build) the output is a gfx950
// code object <output>.hsaco plus <output>.manifest and <output>.hip instead
// of the Ascend ELF produced through `hivmc`.
//
// --enable-cpu-runner[=<options>], --enable-cpu-runner-before=<pass>[,<n>][,<options>]
// and --enable-cpu-runner-after=… (BiShengIRCompileConfig.cpp:100-125,
// PassManager.cpp:56-93) run the input after compiling it: the host function
// (or the only group) is executed with generated inputs and the arguments and
// results are written in the reference runner's text format (runner.cpp).  The
// execution happens on the MI355X; every cut point of the pipeline computes the
// same function, so <pass> and <n> are checked for form only.  The files are
// --runner-inputs=<path> and --runner-outputs=<path> (defaults
// <output>.runner_inputs.txt / <output>.runner_outputs.txt), --runner-func
// picks a function when the module holds several.
//
// Reference flags that configure the Ascend pipeline (-enable-hfusion-compile,
// -enable-hivm-compile, -enable-lir-compile, -block-dim, ...;
// bishengir/include/bishengir/Tools/bishengir-compile/Options.td) are
// accepted and have no effect here: fusion kinds, tiling and block counts are
// chosen by the MI355X lowering.
#include "../../../include/hfc.h"
#include "../runtime/runner.h"

#include <algorithm>
#include <cctype>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

static bool startsWith(const std::string &s, const char *p) { return s.rfind(p, 0) == 0; }

static int compileMain(int argc, char **argv);

// Any exception escaping the compiler or the runner is reported the way the
// reference tool reports errors: `[ERROR] ...` on stderr and EXIT_FAILURE.
int main(int argc, char **argv) {
  try {
    return compileMain(argc, argv);
  } catch (const std::exception &e) {
    std::fprintf(stderr, "[ERROR] internal error: %s\n", e.what());
    return EXIT_FAILURE;
  }
}

static int compileMain(int argc, char **argv) {
  std::string input, output, target = "mi355x";
  std::string opts;
  int runnerFlags = 0;
  std::string runnerIn, runnerOut, runnerFunc;
  static const char *ignored[] = {"-enable-hfusion-compile", "-enable-hivm-compile", "-enable-lir-compile",
                                  "-block-dim", "-enable-auto-multi-buffer", "-enable-static-bare-ptr",
                                  "-enable-triton-kernel-compile", "-enable-bin-relocation", "-enable-sanitizer",
                                  "-enable-debug-info", "-enable-cpu-trace-intrinsic", "-enable-hfusion-auto-schedule"};
  for (int i = 1; i < argc; ++i) {
    std::string a = argv[i];
    std::string b = startsWith(a, "--") ? a.substr(1) : a;
    if (b == "-o") {
      if (i + 1 >= argc) { std::fprintf(stderr, "[ERROR] -o needs a value\n"); return EXIT_FAILURE; }
      output = argv[++i];
    } else if (startsWith(b, "-o=")) {
      output = b.substr(3);
    } else if (startsWith(b, "-target=")) {
      target = b.substr(8);
    } else if (startsWith(b, "-hipcc=")) {
      opts += "hipcc=" + b.substr(7) + ";";
    } else if (startsWith(b, "-dyn=")) {
      opts += "dyn=" + b.substr(5) + ";";
    } else if (startsWith(b, "-emit=")) {
      opts += "emit=" + b.substr(6) + ";";
    } else if (b == "-enable-cpu-runner" || startsWith(b, "-enable-cpu-runner=")) {
      ++runnerFlags;
    } else if (startsWith(b, "-enable-cpu-runner-before") || startsWith(b, "-enable-cpu-runner-after")) {
      ++runnerFlags;
      auto eq = b.find('=');
      std::string spec = eq == std::string::npos ? "" : b.substr(eq + 1);
      std::string pass = spec.substr(0, spec.find(','));
      if (pass.empty()) { std::fprintf(stderr, "[ERROR] At least the pass name should be provided!\n"); return EXIT_FAILURE; }
      for (char c : pass)
        if (!(std::isalnum((unsigned char)c) || c == '-' || c == '_' || c == '.')) {
          std::fprintf(stderr, "[ERROR] \"%s\" is not a pass!\n", pass.c_str());
          return EXIT_FAILURE;
        }
      std::string rest = spec.find(',') == std::string::npos ? "" : spec.substr(spec.find(',') + 1);
      std::string idx = rest.substr(0, rest.find(','));
      if (!idx.empty() && std::all_of(idx.begin(), idx.end(), [](char c) { return std::isdigit((unsigned char)c) || c == '-'; })) {
        if (std::atol(idx.c_str()) <= 0) {
          std::fprintf(stderr, "[ERROR] Pass index should be a positive non-zero integer, but found %s!\n", idx.c_str());
          return EXIT_FAILURE;
        }
      }
    } else if (startsWith(b, "-runner-inputs=")) {
      runnerIn = b.substr(15);
    } else if (startsWith(b, "-runner-outputs=")) {
      runnerOut = b.substr(16);
    } else if (startsWith(b, "-runner-func=")) {
      runnerFunc = b.substr(13);
    } else if (startsWith(b, "-fusion-kind=")) {
      opts += "fusion_kind=" + b.substr(13) + ";";
    } else if (b == "-ordered-fp-sums") {
      opts += "ordered_fp_sums=1;";
    } else if (startsWith(b, "-kernel-include=")) {
      opts += "include=" + b.substr(16) + ";";
    } else if (!a.empty() && a[0] == '-') {
      bool ok = false;
      for (const char *ig : ignored)
        if (b == ig || startsWith(b, (std::string(ig) + "=").c_str())) ok = true;
      if (!ok) { std::fprintf(stderr, "[ERROR] unknown option '%s'\n", a.c_str()); return EXIT_FAILURE; }
    } else if (input.empty()) {
      input = a;
    } else {
      std::fprintf(stderr, "[ERROR] more than one input file\n");
      return EXIT_FAILURE;
    }
  }
  if (input.empty()) { std::fprintf(stderr, "[ERROR] no input file\n"); return EXIT_FAILURE; }
  if (runnerFlags > 1) {
    std::fprintf(stderr, "[ERROR] Cannot combine any of multible cpu-runner options.\n");
    return EXIT_FAILURE;
  }
  if (target != "mi355x" && target != "gfx950") {
    std::fprintf(stderr, "[ERROR] unsupported target '%s' (this build targets mi355x)\n", target.c_str());
    return EXIT_FAILURE;
  }
  if (output.empty()) {
    output = input;
    auto dot = output.find_last_of('.');
    if (dot != std::string::npos) output = output.substr(0, dot);
  }
  if (output.size() > 6 && output.compare(output.size() - 6, 6, ".hsaco") == 0) output.resize(output.size() - 6);
  std::vector<char> err(8192);
  int rc = hfc_compile_file(input.c_str(), output.c_str(), opts.c_str(), err.data(), err.size());
  if (rc != HFC_OK) {
    std::fprintf(stderr, "[ERROR] %s\n", err.data());
    return EXIT_FAILURE;
  }
  if (runnerFlags) {
    std::string msg;
    if (runnerIn.empty()) runnerIn = output + ".runner_inputs.txt";
    if (runnerOut.empty()) runnerOut = output + ".runner_outputs.txt";
    if (hfusionRun(output + ".manifest", runnerFunc, runnerIn, runnerOut, msg) != 0) {
      std::fprintf(stderr, "[ERROR] [Runner] %s\n", msg.c_str());
      return EXIT_FAILURE;
    }
  }
  return EXIT_SUCCESS;
}
