// bishengir-compile — device-compile entry kept as the drop-in CLI.
//
// Same shape as the reference tool (bishengir/tools/bishengir-compile/
// bishengir-compile.cpp:103-191): `bishengir-compile <input.mlir> [flags]
// -o <output>`; errors go to stderr as "[ERROR] ..." with EXIT_FAILURE.
// With --target=mi355x (the default of this build) the output is a gfx950
// code object <output>.hsaco plus <output>.manifest and <output>.hip instead
// of the Ascend ELF produced through `hivmc`.
//
// Reference flags that configure the Ascend pipeline (-enable-hfusion-compile,
// -enable-hivm-compile, -enable-lir-compile, -block-dim, ...;
// bishengir/include/bishengir/Tools/bishengir-compile/Options.td) are
// accepted and have no effect here: fusion kinds, tiling and block counts are
// chosen by the MI355X lowering.
#include "../../../include/hfc.h"

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

static bool startsWith(const std::string &s, const char *p) { return s.rfind(p, 0) == 0; }

int main(int argc, char **argv) {
  std::string input, output, target = "mi355x";
  std::string opts;
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
    } else if (startsWith(b, "-emit=")) {
      opts += "emit=" + b.substr(6) + ";";
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
  return EXIT_SUCCESS;
}
