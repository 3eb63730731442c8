// Device runner used by `bishengir-compile --enable-cpu-runner*` (runner.cpp).
#pragma once
#include <string>

// Runs the host function (launch program) or group `func` of a compiled
// manifest (empty: the only one) on the current GPU with generated inputs,
// writing the arguments to `inputsPath` and the results to `outputsPath` in
// the reference runner's printData format.  Returns 0, or 1 with `err` set.
int hfusionRun(const std::string &manifest, const std::string &func, const std::string &inputsPath,
               const std::string &outputsPath, std::string &err);
