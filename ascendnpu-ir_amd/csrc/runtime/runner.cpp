// Device runner behind `bishengir-compile --enable-cpu-runner[-before|-after]`.
//
// The reference's runner wraps the host entry function in a `main` that
// (bishengir/lib/ExecutionEngine/CreateHostMain.cpp:342-388)
//   1. fills every argument with pseudo-random data: one std::mt19937(1)
//      stream per element type, uniform over a fixed range per type
//      (BiShengIRRunnerUtils.cpp:62-68, 103-125);
//   2. prints the arguments to one file and, after the call, the results to
//      a second file in the `printData` text format (:72-97): rank, the sizes,
//      then the elements (integers in decimal — int8 as its raw byte —, floats
//      as `%.9e` of their float value).
// Here the same steps run the compiled groups on the MI355X through libhfr
// instead of the CPU lowering, so both runs can be compared file to file.
#include "runner.h"

#include "../../../include/hfr.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iomanip>
#include <map>
#include <random>
#include <sstream>
#include <string>
#include <vector>

namespace {

struct Buf {
  std::string role, elem;
  std::vector<int64_t> shape;
  int tied = -1; // results: the argument they are written into
  int64_t numel() const {
    int64_t n = 1;
    for (auto d : shape) n *= d;
    return n;
  }
};

struct Entry {
  bool program = false;
  std::string name;
  std::vector<Buf> params, results;
};

int elemSize(const std::string &e) {
  if (e == "f32" || e == "i32") return 4;
  if (e == "f64" || e == "i64" || e == "index") return 8;
  if (e == "f16" || e == "bf16" || e == "i16") return 2;
  if (e == "i8" || e == "i1") return 1;
  return 0;
}

std::vector<int64_t> readShape(std::istringstream &is) {
  int n = 0;
  is >> n;
  std::vector<int64_t> s(n > 0 ? n : 0);
  for (auto &d : s) is >> d;
  return s;
}

// Reads the entries of a manifest: launch programs first (a split host
// function), then groups.
std::vector<Entry> readEntries(const std::string &path, std::string &err) {
  std::ifstream f(path);
  if (!f) { err = "cannot open " + path; return {}; }
  std::vector<Entry> groups, programs;
  Entry *cur = nullptr;
  std::string ln;
  while (std::getline(f, ln)) {
    if (ln.rfind("hfr-manifest", 0) == 0) { groups.emplace_back(); cur = &groups.back(); continue; }
    if (ln.rfind("hfr-program", 0) == 0) {
      programs.emplace_back();
      cur = &programs.back();
      cur->program = true;
      continue;
    }
    if (!cur) continue;
    std::istringstream is(ln);
    std::string key;
    is >> key;
    if (key == "func" || key == "program") is >> cur->name;
    else if (key == "param" || key == "pparam") {
      Buf b;
      int i;
      is >> i >> b.role >> b.elem;
      b.shape = readShape(is);
      cur->params.push_back(b);
    } else if (key == "result" || key == "presult") {
      Buf b;
      int i;
      std::string tied;
      is >> i >> tied >> b.elem;
      b.shape = readShape(is);
      if (key == "result") b.tied = std::atoi(tied.c_str());
      else b.tied = tied[0] == 'p' ? std::atoi(tied.c_str() + 1) : -1;
      cur->results.push_back(b);
    }
  }
  programs.insert(programs.end(), groups.begin(), groups.end());
  return programs;
}

uint16_t floatToBf16(float v) {
  if (std::isnan(v)) return std::signbit(v) ? 0xFFC0 : 0x7FC0;
  uint32_t u;
  std::memcpy(&u, &v, 4);
  u += 0x7FFF + ((u >> 16) & 1);
  return (uint16_t)(u >> 16);
}

float bf16ToFloat(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// IEEE binary16 from binary32, round to nearest even (subnormals and
// overflow to infinity included).
uint16_t floatToHalf(float v) {
  uint32_t u;
  std::memcpy(&u, &v, 4);
  const uint32_t sign = (u >> 16) & 0x8000;
  const int32_t exp = (int32_t)((u >> 23) & 0xFF);
  uint32_t man = u & 0x7FFFFF;
  if (exp == 0xFF) return (uint16_t)(sign | 0x7C00 | (man ? 0x200 : 0));
  int32_t e = exp - 127 + 15;
  if (e >= 0x1F) return (uint16_t)(sign | 0x7C00);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    man |= 0x800000;
    const int shift = 14 - e;
    uint32_t h = man >> shift, rem = man & ((1u << shift) - 1), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1))) ++h;
    return (uint16_t)(sign | h);
  }
  uint32_t h = ((uint32_t)e << 10) | (man >> 13), rem = man & 0x1FFF;
  if (rem > 0x1000 || (rem == 0x1000 && (h & 1))) ++h; // a carry into the exponent is still exact
  return (uint16_t)(sign | h);
}

float halfToFloat(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000) << 16;
  const int exp = (h >> 10) & 0x1F;
  const uint32_t man = h & 0x3FF;
  float f;
  if (exp == 0) f = std::ldexp((float)man, -24);
  else if (exp == 0x1F) f = man ? NAN : INFINITY;
  else f = std::ldexp((float)(man | 0x400), exp - 25);
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u |= sign;
  std::memcpy(&f, &u, 4);
  return f;
}

// One generator stream per element type for the whole run, as the
// reference's function-local static generators are per instantiation.
struct Streams {
  std::map<std::string, std::mt19937> gen;
  std::mt19937 &of(const std::string &e) {
    auto it = gen.find(e);
    if (it == gen.end()) it = gen.emplace(e, std::mt19937(1)).first;
    return it->second;
  }
};

bool fill(Streams &S, const Buf &b, std::vector<unsigned char> &host, std::string &err) {
  const int64_t n = b.numel();
  host.assign((size_t)n * elemSize(b.elem), 0);
  std::mt19937 &g = S.of(b.elem);
  if (b.elem == "f32") {
    std::uniform_real_distribution<float> d(-1000., 1000.);
    float *p = (float *)host.data();
    for (int64_t i = 0; i < n; ++i) p[i] = d(g);
  } else if (b.elem == "f64") {
    std::uniform_real_distribution<double> d(-10000., 10000.);
    double *p = (double *)host.data();
    for (int64_t i = 0; i < n; ++i) p[i] = d(g);
  } else if (b.elem == "bf16") {
    std::uniform_real_distribution<float> d(-100., 100.);
    uint16_t *p = (uint16_t *)host.data();
    for (int64_t i = 0; i < n; ++i) p[i] = floatToBf16(d(g));
  } else if (b.elem == "f16") {
    std::uniform_real_distribution<float> d(-100., 100.);
    uint16_t *p = (uint16_t *)host.data();
    for (int64_t i = 0; i < n; ++i) p[i] = floatToHalf(d(g));
  } else if (b.elem == "i1") {
    std::uniform_int_distribution<uint8_t> d(0, 1);
    for (int64_t i = 0; i < n; ++i) host[i] = d(g) ? 1 : 0;
  } else if (b.elem == "i8") {
    std::uniform_int_distribution<int8_t> d(-100, 100);
    int8_t *p = (int8_t *)host.data();
    for (int64_t i = 0; i < n; ++i) p[i] = d(g);
  } else if (b.elem == "i16") {
    std::uniform_int_distribution<int16_t> d(-1000, 1000);
    int16_t *p = (int16_t *)host.data();
    for (int64_t i = 0; i < n; ++i) p[i] = d(g);
  } else if (b.elem == "i32") {
    std::uniform_int_distribution<int32_t> d(-10000, 10000);
    int32_t *p = (int32_t *)host.data();
    for (int64_t i = 0; i < n; ++i) p[i] = d(g);
  } else if (b.elem == "i64" || b.elem == "index") {
    std::uniform_int_distribution<int64_t> d(-100000, 100000);
    int64_t *p = (int64_t *)host.data();
    for (int64_t i = 0; i < n; ++i) p[i] = d(g);
  } else {
    err = "the runner has no data generator for element type " + b.elem;
    return false;
  }
  return true;
}

void print(std::ostream &out, const Buf &b, const std::vector<unsigned char> &host) {
  out << b.shape.size();
  for (size_t i = 0; i < b.shape.size(); ++i) out << (i == 0 ? '\n' : ' ') << b.shape[i];
  const int64_t n = b.numel();
  auto sci = [](double v) {
    std::ostringstream ss;
    ss << std::scientific << std::setprecision(9) << v;
    return ss.str();
  };
  for (int64_t i = 0; i < n; ++i) {
    out << (i == 0 ? '\n' : ' ');
    if (b.elem == "f32") out << sci(((const float *)host.data())[i]);
    else if (b.elem == "f64") out << sci(((const double *)host.data())[i]);
    else if (b.elem == "bf16") out << sci(bf16ToFloat(((const uint16_t *)host.data())[i]));
    else if (b.elem == "f16") out << sci(halfToFloat(((const uint16_t *)host.data())[i]));
    else if (b.elem == "i1") out << (int)host[i];
    else if (b.elem == "i8") out << (char)host[i];
    else if (b.elem == "i16") out << ((const int16_t *)host.data())[i];
    else if (b.elem == "i32") out << ((const int32_t *)host.data())[i];
    else out << ((const int64_t *)host.data())[i];
  }
  out << '\n';
}

bool hipOk(hipError_t e, const char *what, std::string &err) {
  if (e == hipSuccess) return true;
  err = std::string(what) + ": " + hipGetErrorString(e);
  return false;
}

} // namespace

int hfusionRun(const std::string &manifest, const std::string &func, const std::string &inputsPath,
               const std::string &outputsPath, std::string &err) {
  std::vector<Entry> entries = readEntries(manifest, err);
  if (entries.empty()) {
    if (err.empty()) err = "manifest holds nothing to run";
    return 1;
  }
  const Entry *e = nullptr;
  if (func.empty()) {
    if (entries[0].program) {
      int np = 0;
      for (auto &x : entries) np += x.program;
      if (np > 1) { err = "several host functions; name one with --runner-func"; return 1; }
      e = &entries[0];
    } else if (entries.size() == 1) {
      e = &entries[0];
    } else {
      err = "several groups; name one with --runner-func";
      return 1;
    }
  } else {
    for (auto &x : entries)
      if (x.name == func) { e = &x; break; }
    if (!e) { err = "no function @" + func + " in " + manifest; return 1; }
  }
  for (auto &p : e->params)
    if (p.role == "scalar") { err = "the runner passes tensors only (@" + e->name + " takes a scalar)"; return 1; }

  // 1. inputs, generated and printed in argument order
  Streams S;
  std::vector<std::vector<unsigned char>> host(e->params.size());
  for (size_t i = 0; i < e->params.size(); ++i)
    if (!fill(S, e->params[i], host[i], err)) return 1;
  {
    std::ofstream out(inputsPath);
    if (!out) { err = "cannot write " + inputsPath; return 1; }
    for (size_t i = 0; i < e->params.size(); ++i) print(out, e->params[i], host[i]);
  }
  // 2. device buffers, launch, results
  std::vector<void *> dev(e->params.size(), nullptr), rdev(e->results.size(), nullptr);
  auto release = [&]() {
    for (void *p : dev) if (p) (void)hipFree(p);
    for (void *p : rdev) if (p) (void)hipFree(p);
  };
  for (size_t i = 0; i < e->params.size(); ++i) {
    size_t bytes = host[i].size() ? host[i].size() : 1;
    if (!hipOk(hipMalloc(&dev[i], bytes), "hipMalloc", err) ||
        !hipOk(hipMemcpy(dev[i], host[i].data(), host[i].size(), hipMemcpyHostToDevice), "hipMemcpy", err)) {
      release();
      return 1;
    }
  }
  std::vector<uint64_t> slots(e->params.size());
  for (size_t i = 0; i < dev.size(); ++i) slots[i] = (uint64_t)(uintptr_t)dev[i];
  for (size_t j = 0; j < e->results.size(); ++j) {
    const Buf &r = e->results[j];
    if (r.tied >= 0) continue;
    size_t bytes = (size_t)r.numel() * elemSize(r.elem);
    if (!hipOk(hipMalloc(&rdev[j], bytes ? bytes : 1), "hipMalloc", err)) { release(); return 1; }
  }
  int rc = 0;
  if (e->program) {
    hfr_program_t p = nullptr;
    rc = hfr_program_load(manifest.c_str(), e->name.c_str(), &p);
    if (!rc) rc = hfr_program_launch(p, slots.data(), slots.size(), rdev.data(), rdev.size(), nullptr, nullptr);
    if (!rc && !hipOk(hipDeviceSynchronize(), "hipDeviceSynchronize", err)) rc = -2;
    if (p) hfr_program_unload(p);
  } else {
    hfr_group_t g = nullptr;
    rc = hfr_group_load(manifest.c_str(), e->name.c_str(), &g);
    if (!rc) rc = hfr_group_launch(g, slots.data(), slots.size(), rdev.data(), rdev.size(), nullptr, nullptr);
    if (!rc && !hipOk(hipDeviceSynchronize(), "hipDeviceSynchronize", err)) rc = -2;
    if (g) hfr_group_unload(g);
  }
  if (rc) {
    if (err.empty()) err = hfr_last_error();
    release();
    return 1;
  }
  std::ofstream out(outputsPath);
  if (!out) { err = "cannot write " + outputsPath; release(); return 1; }
  for (size_t j = 0; j < e->results.size(); ++j) {
    const Buf &r = e->results[j];
    std::vector<unsigned char> h((size_t)r.numel() * elemSize(r.elem));
    void *src = r.tied >= 0 ? dev[r.tied] : rdev[j];
    if (!hipOk(hipMemcpy(h.data(), src, h.size(), hipMemcpyDeviceToHost), "hipMemcpy", err)) { release(); return 1; }
    print(out, r, h);
  }
  release();
  return 0;
}
