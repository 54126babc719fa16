// Kernel timing for benchmarks. ct_profile_begin creates a pool of HIP event pairs; each
// launch of an enabled family takes the next pair and records it around the launch on the
// launch's own stream, so the measured interval is that kernel's execution (consecutive
// kernels on one stream do not overlap). ct_profile_read synchronises on the events and
// sums their elapsed times; ct_profile_end releases the pool. This is the only state the library keeps
// between calls, and only between begin and end.

#include <atomic>
#include <mutex>
#include <vector>

#include "common.hpp"
#include "profile.hpp"

namespace ct {
namespace {

struct Slot {
    hipEvent_t start, stop;
    int family;
    double work;
    bool closed;
};

std::mutex g_mutex;
std::atomic<int> g_families{0};
std::vector<Slot> g_slots;
size_t g_used = 0;

}  // namespace

int profile_open(int family, hipStream_t stream) {
    if (!(g_families.load(std::memory_order_relaxed) & family)) return -1;
    std::lock_guard<std::mutex> lock(g_mutex);
    if (!(g_families.load() & family) || g_used >= g_slots.size()) return -1;
    const int slot = (int)g_used++;
    g_slots[slot].family = family;
    g_slots[slot].work = 0.0;
    g_slots[slot].closed = false;
    if (hipEventRecord(g_slots[slot].start, stream) != hipSuccess) return -1;
    return slot;
}

void profile_close(int slot, hipStream_t stream, double work) {
    if (slot < 0) return;
    std::lock_guard<std::mutex> lock(g_mutex);
    if ((size_t)slot >= g_slots.size()) return;
    if (hipEventRecord(g_slots[slot].stop, stream) == hipSuccess) {
        g_slots[slot].work = work;
        g_slots[slot].closed = true;
    }
}

}  // namespace ct

using namespace ct;

extern "C" int ct_profile_begin(int32_t families, int32_t capacity) {
    if (families <= 0 || capacity <= 0) return -CT_EINVAL_SHAPE;
    std::lock_guard<std::mutex> lock(g_mutex);
    if (g_families.load() != 0) return -CT_EINVAL_POINTER;  // already profiling
    // Build the pool aside and publish it only when every event exists; on a failure the
    // events created so far are destroyed and the profiler stays closed.
    std::vector<Slot> slots((size_t)capacity, Slot{});
    size_t created = 0;
    hipError_t e = hipSuccess;
    for (; created < slots.size(); ++created) {
        e = hipEventCreate(&slots[created].start);
        if (e != hipSuccess) break;
        e = hipEventCreate(&slots[created].stop);
        if (e != hipSuccess) {
            hipEventDestroy(slots[created].start);
            break;
        }
    }
    if (e != hipSuccess) {
        for (size_t i = 0; i < created; ++i) {
            hipEventDestroy(slots[i].start);
            hipEventDestroy(slots[i].stop);
        }
        return (int)e;
    }
    g_slots.swap(slots);
    g_used = 0;
    g_families.store(families);
    return 0;
}

extern "C" int ct_profile_read(int32_t family, double *total_ms, int64_t *launches, double *work) {
    std::lock_guard<std::mutex> lock(g_mutex);
    double ms_sum = 0.0, work_sum = 0.0;
    int64_t count = 0;
    int status = 0;
    for (size_t i = 0; i < g_used; ++i) {
        Slot &s = g_slots[i];
        if (!s.closed || !(s.family & family)) continue;
        hipError_t e = hipEventSynchronize(s.stop);
        float ms = 0.f;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, s.start, s.stop);
        if (e != hipSuccess) {
            status = (int)e;
            continue;
        }
        ms_sum += ms;
        work_sum += s.work;
        ++count;
    }
    if (total_ms) *total_ms = ms_sum;
    if (launches) *launches = count;
    if (work) *work = work_sum;
    return status;
}

extern "C" int ct_profile_end(void) {
    std::lock_guard<std::mutex> lock(g_mutex);
    g_families.store(0);
    for (size_t i = 0; i < g_used; ++i) hipEventSynchronize(g_slots[i].stop);
    for (auto &s : g_slots) {
        hipEventDestroy(s.start);
        hipEventDestroy(s.stop);
    }
    g_slots.clear();
    g_used = 0;
    return 0;
}
