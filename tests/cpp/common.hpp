// common.hpp — test helpers of the C++ drop-in tests: the counterpart of the reference's
// test::DeviceGuard and assert helpers (autograd/common.hpp:22-81), without a device handle
// (libttperf_hip selects device 0 per store) and with exact (bitwise) checks.
#pragma once

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "ttperf/ttperf.h"

namespace test {

inline int g_failures = 0;

// Fails the process early (exit 2) when no GPU is visible, so the caller can tell
// "skipped" from "failed".
struct DeviceGuard {
    DeviceGuard() {
        int n = 0;
        if (ttp_device_count(&n) != TTP_OK || n < 1) {
            std::printf("SKIP: no HIP device\n");
            std::exit(2);
        }
    }
};

inline uint32_t bits(float x) {
    uint32_t u;
    std::memcpy(&u, &x, 4);
    return u;
}

inline float bf16_round(float x) {  // value of the round-to-nearest-even bf16 of x
    uint32_t u = bits(x);
    u = ((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16) << 16;
    float r;
    std::memcpy(&r, &u, 4);
    return r;
}

inline void check(bool ok, const std::string& what) {
    if (!ok) {
        std::printf("FAIL: %s\n", what.c_str());
        ++g_failures;
    }
}

// every element bit-identical to the expected value
inline void assert_bits(const std::vector<float>& got, const std::vector<float>& want,
                        const std::string& what) {
    if (got.size() != want.size()) {
        check(false, what + ": size " + std::to_string(got.size()) + " != " +
                         std::to_string(want.size()));
        return;
    }
    size_t bad = 0, first = 0;
    for (size_t i = 0; i < got.size(); ++i)
        if (bits(got[i]) != bits(want[i]) && !(std::isnan(got[i]) && std::isnan(want[i]))) {
            if (!bad) first = i;
            ++bad;
        }
    if (bad) {
        char buf[256];
        std::snprintf(buf, sizeof buf, "%s: %zu of %zu differ (first [%zu] got %.9g want %.9g)",
                      what.c_str(), bad, got.size(), first, got[first], want[first]);
        check(false, buf);
    }
}

inline void assert_all_close(const std::vector<float>& got, float expected, float tol,
                             const std::string& what) {
    for (size_t i = 0; i < got.size(); ++i)
        if (!(std::fabs(got[i] - expected) <= tol)) {
            char buf[256];
            std::snprintf(buf, sizeof buf, "%s: [%zu] = %.9g, expected %.9g +- %g", what.c_str(), i,
                          got[i], expected, tol);
            check(false, buf);
            return;
        }
}

// the pass/fail line is flushed at once: what the runtimes do at exit cannot lose it
inline int finish(const char* name) {
    if (g_failures) {
        std::printf("%s: %d check(s) failed\n", name, g_failures);
        std::fflush(stdout);
        return 1;
    }
    std::printf("%s: PASS\n", name);
    std::fflush(stdout);
    return 0;
}

}  // namespace test
