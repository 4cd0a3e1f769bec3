// Error state and version of the C ABI (include/primus_turbo_amd.h).
#include <unistd.h>

#include <atomic>
#include <chrono>
#include <cstdarg>
#include <cstdio>

#include "common.h"

namespace pta {

static thread_local char g_last_error[1024] = {0};

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
}

static thread_local uint64_t g_wait_tag    = 0;
static thread_local int64_t  g_wait_offset = -1;
static std::atomic<int>      g_force_giveup{0};

void clear_error() {
    g_last_error[0] = '\0';
    g_wait_tag      = 0;
    g_wait_offset   = -1;
}

void record_wait(uint64_t tag, int64_t status_offset) {
    g_wait_tag    = tag;
    g_wait_offset = status_offset;
}

WaitPlan wait_plan(uint64_t tag, uint32_t default_limit) {
    if (g_force_giveup.load(std::memory_order_relaxed)) return WaitPlan{~tag, 64u};
    return WaitPlan{tag, default_limit};
}

uint64_t next_call_tag() {
    static std::atomic<uint64_t> ctr{0};
    static const uint64_t        salt =
        (static_cast<uint64_t>(getpid()) << 40) ^
        (static_cast<uint64_t>(std::chrono::steady_clock::now().time_since_epoch().count()) << 16);
    return salt ^ (ctr.fetch_add(1, std::memory_order_relaxed) + 1);
}

bool stream_capturing(hipStream_t st) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    // an error (e.g. a legacy-stream query during another stream's capture)
    // counts as capturing: the caller then takes its graph-safe form
    if (hipStreamIsCapturing(st, &cs) != hipSuccess) return true;
    return cs != hipStreamCaptureStatusNone;
}

int device_cu_count() {
    constexpr int   kMax = 64;
    static std::atomic<int> cus[kMax] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
    if (dev < kMax) {
        if (int c = cus[dev].load(std::memory_order_relaxed)) return c;
    }
    int c = 0;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
    if (dev < kMax) cus[dev].store(c, std::memory_order_relaxed);
    return c;
}

} // namespace pta

extern "C" const char *pta_last_error(void) { return pta::g_last_error; }

extern "C" int pta_abi_version(void) { return 6; }

extern "C" int pta_last_wait_status(uint64_t *tag, int64_t *status_offset) {
    if (tag == nullptr || status_offset == nullptr) return PTA_ERR_INVALID_ARG;
    *tag           = pta::g_wait_tag;
    *status_offset = pta::g_wait_offset;
    return PTA_OK;
}

extern "C" void pta_test_force_wait_giveup(int on) { pta::g_force_giveup.store(on != 0, std::memory_order_relaxed); }
