// Minimal test harness for the C++ tests: CHECK* record a failure with its
// location and keep going inside a test; run() prints one line per test and
// main() returns the number of failed tests (0 = all passed).
#pragma once

#include <cmath>
#include <cstdio>
#include <exception>
#include <functional>
#include <string>
#include <vector>

namespace harness {

inline int &failures() {
  static int n = 0;
  return n;
}
inline int &current_failures() {
  static int n = 0;
  return n;
}

inline void fail(const char *file, int line, const std::string &msg) {
  std::printf("\n  FAILED %s:%d: %s", file, line, msg.c_str());
  current_failures() += 1;
}

inline void run(const char *name, const std::function<void()> &test) {
  std::printf("%s ... ", name);
  std::fflush(stdout);
  current_failures() = 0;
  try {
    test();
  } catch (const std::exception &e) {
    fail(__FILE__, __LINE__, std::string("unexpected exception: ") + e.what());
  }
  if (current_failures()) {
    failures() += 1;
    std::printf("\n%s: FAILED\n", name);
  } else {
    std::printf("PASSED\n");
  }
  std::fflush(stdout);
}

} // namespace harness

#define CHECK(cond)                                                            \
  do {                                                                         \
    if (!(cond)) harness::fail(__FILE__, __LINE__, #cond);                     \
  } while (0)

#define CHECK_NEAR(actual, expected, tol)                                      \
  do {                                                                         \
    const double a_ = (actual), e_ = (expected);                               \
    if (!(std::fabs(a_ - e_) <= (tol)))                                        \
      harness::fail(__FILE__, __LINE__,                                        \
                    std::string(#actual) + " = " + std::to_string(a_) +       \
                        ", expected " + std::to_string(e_));                   \
  } while (0)

#define CHECK_THROWS(Exception, expr)                                          \
  do {                                                                         \
    bool threw_ = false;                                                       \
    try {                                                                      \
      expr;                                                                    \
    } catch (const Exception &) {                                              \
      threw_ = true;                                                           \
    } catch (...) {                                                            \
    }                                                                          \
    if (!threw_)                                                               \
      harness::fail(__FILE__, __LINE__, "expected " #Exception " from " #expr); \
  } while (0)
