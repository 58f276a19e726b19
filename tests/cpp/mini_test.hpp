// mini_test.hpp -- a small GTest-shaped test runner for the C++ drop-in.
//
// GoogleTest is not available in this toolchain, so the C++ tests register
// with TEST_F(Fixture, Name) and check with EXPECT_* / ASSERT_* macros of
// the same names and meaning; the test bodies therefore read like the
// reference's GTest suites.  `dnn_tests --list` prints the registered tests
// without touching a GPU; `dnn_tests [filter]` runs those whose
// "Fixture.Name" contains the filter and exits non-zero on any failure.
#pragma once

#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <exception>
#include <functional>
#include <iostream>
#include <sstream>
#include <string>
#include <vector>

namespace mini_test {

struct Failure {};  // thrown by ASSERT_* to end the current test

struct Registry {
    struct Entry {
        std::string name;
        std::function<void()> run;
    };
    std::vector<Entry> tests;
    int failures = 0;  // failed checks in the running test
    static Registry& get() {
        static Registry r;
        return r;
    }
};

// SCOPED_TRACE: messages that a failure inside their scope also prints
inline std::vector<std::string>& traces() {
    static thread_local std::vector<std::string> t;
    return t;
}
struct ScopedTrace {
    explicit ScopedTrace(std::string m) { traces().push_back(std::move(m)); }
    ~ScopedTrace() { traces().pop_back(); }
    ScopedTrace(const ScopedTrace&) = delete;
    ScopedTrace& operator=(const ScopedTrace&) = delete;
};

inline void fail(const char* file, int line, const std::string& msg) {
    std::cout << file << ":" << line << ": Failure\n  " << msg << std::endl;
    for (const std::string& t : traces()) std::cout << "  (trace: " << t << ")" << std::endl;
    ++Registry::get().failures;
}

template <typename A, typename B>
std::string describe(const char* op, const char* ea, const char* eb, const A& a, const B& b) {
    std::ostringstream os;
    os << "Expected: (" << ea << ") " << op << " (" << eb << "), actual: " << a << " vs " << b;
    return os.str();
}

struct Registrar {
    Registrar(const char* fixture, const char* name, std::function<void()> fn) {
        Registry::get().tests.push_back({std::string(fixture) + "." + name, std::move(fn)});
    }
};

class Test {
public:
    virtual ~Test() = default;
    virtual void SetUp() {}
    virtual void TearDown() {}
    virtual void Body() = 0;
};

inline int run_all(int argc, char** argv) {
    auto& reg = Registry::get();
    const std::string filter = argc > 1 ? argv[1] : "";
    if (filter == "--list") {
        for (auto& t : reg.tests) std::cout << t.name << "\n";
        return 0;
    }
    int run = 0, failed = 0;
    std::vector<std::string> failed_names;
    for (auto& t : reg.tests) {
        if (!filter.empty() && t.name.find(filter) == std::string::npos) continue;
        ++run;
        reg.failures = 0;
        std::cout << "[ RUN      ] " << t.name << std::endl;
        try {
            t.run();
        } catch (const Failure&) {
        } catch (const std::exception& e) {
            fail(__FILE__, __LINE__, std::string("uncaught exception: ") + e.what());
        }
        if (reg.failures) {
            ++failed;
            failed_names.push_back(t.name);
            std::cout << "[  FAILED  ] " << t.name << std::endl;
        } else {
            std::cout << "[       OK ] " << t.name << std::endl;
        }
    }
    std::cout << "[==========] " << run << " tests ran, " << (run - failed) << " passed, " << failed << " failed"
              << std::endl;
    for (auto& n : failed_names) std::cout << "[  FAILED  ] " << n << std::endl;
    return (failed || run == 0) ? 1 : 0;
}

}  // namespace mini_test

#define MT_CAT2(a, b) a##b
#define MT_CAT(a, b) MT_CAT2(a, b)
#define SCOPED_TRACE(msg) mini_test::ScopedTrace MT_CAT(mt_trace_, __LINE__)(msg)

#define MT_CLASS(F, N) F##_##N##_Test
#define TEST_F(F, N)                                                                       \
    class MT_CLASS(F, N) : public F {                                                      \
    public:                                                                                \
        void Body() override;                                                              \
        void mt_set_up() { this->SetUp(); }                                                \
        void mt_tear_down() { this->TearDown(); }                                          \
    };                                                                                     \
    static mini_test::Registrar F##_##N##_registrar(#F, #N, [] {                           \
        MT_CLASS(F, N) t;                                                                  \
        t.mt_set_up();                                                                     \
        try {                                                                              \
            t.Body();                                                                      \
        } catch (...) {                                                                    \
            t.mt_tear_down();                                                              \
            throw;                                                                         \
        }                                                                                  \
        t.mt_tear_down();                                                                  \
    });                                                                                    \
    void MT_CLASS(F, N)::Body()

#define MT_CMP(fatal, op, a, b)                                                              \
    do {                                                                                     \
        const auto mt_a = (a); /* copies: (a) may be an element of a temporary */          \
        const auto mt_b = (b);                                                               \
        if (!(mt_a op mt_b)) {                                                               \
            mini_test::fail(__FILE__, __LINE__, mini_test::describe(#op, #a, #b, mt_a, mt_b)); \
            if (fatal) throw mini_test::Failure{};                                           \
        }                                                                                    \
    } while (0)

#define EXPECT_EQ(a, b) MT_CMP(false, ==, a, b)
#define EXPECT_NE(a, b) MT_CMP(false, !=, a, b)
#define EXPECT_LE(a, b) MT_CMP(false, <=, a, b)
#define EXPECT_LT(a, b) MT_CMP(false, <, a, b)
#define EXPECT_GT(a, b) MT_CMP(false, >, a, b)
#define ASSERT_EQ(a, b) MT_CMP(true, ==, a, b)
#define ASSERT_LE(a, b) MT_CMP(true, <=, a, b)
#define EXPECT_TRUE(c) MT_CMP(false, ==, static_cast<bool>(c), true)
#define EXPECT_FALSE(c) MT_CMP(false, ==, static_cast<bool>(c), false)
#define ASSERT_TRUE(c) MT_CMP(true, ==, static_cast<bool>(c), true)

#define EXPECT_NEAR(a, b, tol)                                                                   \
    do {                                                                                         \
        const double mt_a = (a), mt_b = (b), mt_t = (tol);                                       \
        if (!(std::fabs(mt_a - mt_b) <= mt_t)) {                                                 \
            std::ostringstream mt_os;                                                            \
            mt_os << "|" #a " - " #b "| = " << std::fabs(mt_a - mt_b) << " > " << mt_t << " (" << mt_a \
                  << " vs " << mt_b << ")";                                                      \
            mini_test::fail(__FILE__, __LINE__, mt_os.str());                                    \
        }                                                                                        \
    } while (0)

// equal within 4 units in the last place (GTest's EXPECT_FLOAT_EQ)
inline bool mt_float_eq(float a, float b) {
    if (std::isnan(a) || std::isnan(b)) return false;
    if (a == b) return true;
    int32_t ia, ib;
    std::memcpy(&ia, &a, 4);
    std::memcpy(&ib, &b, 4);
    if ((ia < 0) != (ib < 0)) return false;
    return std::abs((int64_t)ia - (int64_t)ib) <= 4;
}
#define EXPECT_FLOAT_EQ(a, b)                                                                       \
    do {                                                                                            \
        const float mt_a = (a), mt_b = (b);                                                         \
        if (!mt_float_eq(mt_a, mt_b))                                                               \
            mini_test::fail(__FILE__, __LINE__, mini_test::describe("~=", #a, #b, mt_a, mt_b));     \
    } while (0)

#define MT_THROWS(fatal, stmt, ExcT)                                                              \
    do {                                                                                          \
        bool mt_caught = false;                                                                   \
        try {                                                                                     \
            stmt;                                                                                 \
        } catch (const ExcT&) {                                                                   \
            mt_caught = true;                                                                     \
        } catch (...) {                                                                           \
        }                                                                                         \
        if (!mt_caught) {                                                                         \
            mini_test::fail(__FILE__, __LINE__, "Expected " #stmt " to throw " #ExcT);            \
            if (fatal) throw mini_test::Failure{};                                                \
        }                                                                                         \
    } while (0)
#define EXPECT_THROW(stmt, ExcT) MT_THROWS(false, stmt, ExcT)
#define EXPECT_ANY_THROW(stmt) MT_THROWS(false, stmt, std::exception)
#define EXPECT_NO_THROW(stmt)                                                                     \
    do {                                                                                          \
        try {                                                                                     \
            stmt;                                                                                 \
        } catch (const std::exception& mt_e) {                                                    \
            mini_test::fail(__FILE__, __LINE__, std::string("Unexpected exception: ") + mt_e.what()); \
        }                                                                                         \
    } while (0)
