#pragma once
// mini_test.hpp -- a small self-registering test runner for the C++ API tests.
// Outcomes: pass, fail, skip. `--filter=<prefix>` selects tests by "suite.name"
// prefix; a filter that matches nothing exits with status 2 (as the
// reference's runner does, tests/test_framework.cpp:300-308).

#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

namespace mt {

struct Skip {
  std::string why;
};

struct Context {
  std::vector<std::string> failures;
  void fail(const char* file, int line, const std::string& msg) {
    std::ostringstream oss;
    oss << file << ":" << line << ": " << msg;
    failures.push_back(oss.str());
  }
};

struct Test {
  std::string name;
  std::function<void(Context&)> fn;
};

inline std::vector<Test>& registry() {
  static std::vector<Test> r;
  return r;
}

struct Registrar {
  Registrar(const char* suite, const char* name, std::function<void(Context&)> fn) {
    registry().push_back({std::string(suite) + "." + name, std::move(fn)});
  }
};

inline int run_all(int argc, char** argv) {
  std::string filter;
  bool list = false;
  for (int i = 1; i < argc; ++i) {
    if (std::strncmp(argv[i], "--filter=", 9) == 0) filter = argv[i] + 9;
    if (std::strcmp(argv[i], "--list") == 0) list = true;
  }
  int passed = 0, failed = 0, skipped = 0, matched = 0;
  for (auto& t : registry()) {
    if (!filter.empty() && t.name.compare(0, filter.size(), filter) != 0) continue;
    ++matched;
    if (list) {
      std::printf("%s\n", t.name.c_str());
      continue;
    }
    Context ctx;
    try {
      t.fn(ctx);
    } catch (const Skip& s) {
      std::printf("[ SKIP ] %s: %s\n", t.name.c_str(), s.why.c_str());
      ++skipped;
      continue;
    } catch (const std::exception& e) {
      ctx.failures.push_back(std::string("uncaught exception: ") + e.what());
    }
    if (ctx.failures.empty()) {
      std::printf("[ PASS ] %s\n", t.name.c_str());
      ++passed;
    } else {
      std::printf("[ FAIL ] %s\n", t.name.c_str());
      for (auto& f : ctx.failures) std::printf("    %s\n", f.c_str());
      ++failed;
    }
    std::fflush(stdout);
  }
  if (matched == 0) {
    std::printf("no test matches filter '%s'\n", filter.c_str());
    return 2;
  }
  if (!list) std::printf("%d passed, %d failed, %d skipped\n", passed, failed, skipped);
  return failed == 0 ? 0 : 1;
}

}  // namespace mt

#define MT_CAT2(a, b) a##b
#define MT_CAT(a, b) MT_CAT2(a, b)
#define TEST(suite, name)                                                         \
  static void MT_CAT(test_, MT_CAT(suite, MT_CAT(_, name)))(mt::Context & ctx);   \
  static mt::Registrar MT_CAT(reg_, MT_CAT(suite, MT_CAT(_, name)))(              \
      #suite, #name, MT_CAT(test_, MT_CAT(suite, MT_CAT(_, name))));              \
  static void MT_CAT(test_, MT_CAT(suite, MT_CAT(_, name)))(mt::Context & ctx)

#define EXPECT_TRUE(c) \
  do { if (!(c)) ctx.fail(__FILE__, __LINE__, "expected true: " #c); } while (0)
#define ASSERT_TRUE(c)                                                  \
  do {                                                                  \
    if (!(c)) {                                                         \
      ctx.fail(__FILE__, __LINE__, "required: " #c);                    \
      return;                                                           \
    }                                                                   \
  } while (0)
#define EXPECT_EQ(a, b)                                                              \
  do {                                                                               \
    if (!((a) == (b))) {                                                             \
      std::ostringstream oss_;                                                       \
      oss_ << "expected " #a " == " #b " (" << (a) << " vs " << (b) << ")";          \
      ctx.fail(__FILE__, __LINE__, oss_.str());                                      \
    }                                                                                \
  } while (0)
#define EXPECT_THROWS_MSG(expr, substr)                                              \
  do {                                                                               \
    bool thrown_ = false;                                                            \
    try {                                                                            \
      (void)(expr);                                                                  \
    } catch (const std::exception& e_) {                                             \
      thrown_ = true;                                                                \
      if (std::string(e_.what()).find(substr) == std::string::npos)                  \
        ctx.fail(__FILE__, __LINE__,                                                 \
                 std::string("message of " #expr " lacks '") + (substr) + "': " + e_.what()); \
    }                                                                                \
    if (!thrown_) ctx.fail(__FILE__, __LINE__, "expected a throw from " #expr);      \
  } while (0)
#define EXPECT_NO_THROW(expr)                                                        \
  do {                                                                               \
    try {                                                                            \
      (void)(expr);                                                                  \
    } catch (const std::exception& e_) {                                             \
      ctx.fail(__FILE__, __LINE__, std::string("unexpected throw from " #expr ": ") + e_.what()); \
    }                                                                                \
  } while (0)
#define SKIP(why) throw mt::Skip{why}
