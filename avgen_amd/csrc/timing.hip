// Opt-in per-kernel launch timing with HIP events recorded on the launch
// stream (diagnostics for benchmarks; off by default, zero cost when off
// beyond one relaxed atomic load per launch).
#include <atomic>
#include <mutex>
#include <vector>

#include "avattn.h"
#include "avattn_kernels.h"

namespace avattn {
namespace {

std::atomic<bool> g_on{false};
std::mutex g_mu;
std::vector<hipEvent_t> g_start, g_stop;
std::vector<int> g_kid;
int g_used = 0;
int g_dropped = 0;

void destroy_locked() {
  for (auto e : g_start) (void)hipEventDestroy(e);
  for (auto e : g_stop) (void)hipEventDestroy(e);
  g_start.clear();
  g_stop.clear();
  g_kid.clear();
  g_used = 0;
  g_dropped = 0;
}

}  // namespace

LaunchTimer::LaunchTimer(int kernel_id, hipStream_t stream) : slot_(-1), stream_(stream) {
  if (!g_on.load(std::memory_order_relaxed)) return;
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_used >= (int)g_start.size()) {
    ++g_dropped;
    return;
  }
  slot_ = g_used++;
  g_kid[slot_] = kernel_id;
  if (hipEventRecord(g_start[slot_], stream_) != hipSuccess) slot_ = -1;
}

LaunchTimer::~LaunchTimer() {
  if (slot_ < 0) return;
  (void)hipEventRecord(g_stop[slot_], stream_);
}

}  // namespace avattn

using namespace avattn;

extern "C" {

int avattn_timing_begin(int32_t capacity) {
  if (capacity <= 0 || capacity > (1 << 20)) return AVATTN_ERR_ARGUMENT;
  std::lock_guard<std::mutex> lock(g_mu);
  destroy_locked();
  g_start.resize(capacity);
  g_stop.resize(capacity);
  g_kid.assign(capacity, -1);
  for (int i = 0; i < capacity; ++i) {
    if (hipEventCreate(&g_start[i]) != hipSuccess || hipEventCreate(&g_stop[i]) != hipSuccess) {
      g_start.resize(i);
      g_stop.resize(i);
      destroy_locked();
      return AVATTN_ERR_LAUNCH;
    }
  }
  g_on.store(true);
  return AVATTN_OK;
}

int avattn_timing_end(void) {
  g_on.store(false);
  return AVATTN_OK;
}

int avattn_timing_read(int32_t kernel_id, double* total_ms, int32_t* launches) {
  if (!total_ms || !launches) return AVATTN_ERR_NULL_POINTER;
  std::lock_guard<std::mutex> lock(g_mu);
  double sum = 0.0;
  int n = 0;
  for (int i = 0; i < g_used; ++i) {
    if (g_kid[i] != kernel_id) continue;
    if (hipEventSynchronize(g_stop[i]) != hipSuccess) return AVATTN_ERR_LAUNCH;
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, g_start[i], g_stop[i]) != hipSuccess) return AVATTN_ERR_LAUNCH;
    sum += ms;
    ++n;
  }
  *total_ms = sum;
  *launches = n;
  return g_dropped ? AVATTN_ERR_WORKSPACE : AVATTN_OK;
}

int avattn_timing_reset(void) {
  g_on.store(false);
  std::lock_guard<std::mutex> lock(g_mu);
  destroy_locked();
  return AVATTN_OK;
}

}  // extern "C"
