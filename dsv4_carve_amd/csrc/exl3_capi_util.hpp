// Host-side helpers shared by the C-ABI entry points: a thread-local error
// message (no error codes cross the ABI other than a negative return), launch
// checking and a per-device CU count cache.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <mutex>

namespace exl3 {

inline thread_local char g_last_error[512] = {0};

inline void clear_error() { g_last_error[0] = 0; }

inline int fail(const char* msg) {
    snprintf(g_last_error, sizeof(g_last_error), "%s", msg);
    return -1;
}

inline int check_launch() {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        snprintf(g_last_error, sizeof(g_last_error), "kernel launch failed: %s", hipGetErrorString(e));
        return -1;
    }
    return 0;
}

inline int64_t align_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

constexpr int MAX_DEVICES = 64;

inline int device_cus() {
    static int cache[MAX_DEVICES] = {0};
    static std::mutex mu;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return 256;
    std::lock_guard<std::mutex> lock(mu);
    if (!cache[dev]) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        cache[dev] = cus;
    }
    return cache[dev];
}

}  // namespace exl3
