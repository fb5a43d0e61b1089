// Minimal test registry shared by the C++ test files of this binary.
#pragma once

#include <stdio.h>

#include <functional>
#include <vector>

inline int g_failures = 0;
#define CHECK(cond)                                                                 \
  do {                                                                              \
    if (!(cond)) {                                                                  \
      fprintf(stderr, "  CHECK failed %s:%d: %s\n", __FILE__, __LINE__, #cond);   \
      ++g_failures;                                                                 \
    }                                                                               \
  } while (0)

struct Case {
  const char* name;
  bool gpu;
  std::function<void()> fn;
};
inline std::vector<Case>& cases() {
  static std::vector<Case> c;
  return c;
}
struct Reg {
  Reg(const char* n, bool gpu, std::function<void()> f) { cases().push_back({n, gpu, f}); }
};
#define TEST(name, gpu) \
  static void name();   \
  static Reg reg_##name(#name, gpu, name); \
  static void name()
