// api_util.hpp -- host helpers shared by the loom_amd_* entry points.
#pragma once

#include <mutex>
#include <string>

#include "lamd.hpp"

struct loom_amd_matrix {
    lamd::Matrix m;
};

namespace lamd {

extern thread_local std::string g_amd_error;

inline int fail(const std::string& msg) {
    g_amd_error = msg;
    return -1;
}

inline int fail_hip(const char* what, hipError_t e) {
    return fail(std::string(what) + ": " + hipGetErrorString(e));
}

// Restores the caller's current device on scope exit.
struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) (void)hipSetDevice(dev);
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

bool is_gfx950(int dev);
int visible_gfx950();

// Lock serializing the v2 plugin's calls on one device (amd_api.hip).
std::mutex& device_mutex(int device);

// Bump layout of one allocation's sub-buffers, 256-byte aligned.
struct Layout {
    size_t off = 0;
    size_t take(size_t bytes) {
        size_t at = off;
        off += (bytes + 255) & ~(size_t)255;
        return at;
    }
};

}  // namespace lamd
