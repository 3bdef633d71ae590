// Error reporting, launch counters and optional per-launch event timing.
#include "runtime.hpp"

#include <atomic>
#include <mutex>
#include <vector>

namespace odde {

namespace {
thread_local std::string g_error;
std::atomic<int64_t> g_launches[ODDE_K_COUNT];

struct TimingState {
  std::mutex mu;
  bool enabled = false;
  std::vector<hipEvent_t> pool;        // idle events
  struct Rec { int id; hipEvent_t a, b; };
  std::vector<Rec> recs;
};
TimingState& timing() {
  static TimingState t;
  return t;
}

hipEvent_t get_event(TimingState& t) {
  if (!t.pool.empty()) {
    hipEvent_t e = t.pool.back();
    t.pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}
}  // namespace

int set_error(int code, const std::string& msg) {
  g_error = msg;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(ODDE_EHIP, std::string(what) + ": " + hipGetErrorString(e));
  return ODDE_OK;
}

int resident_grid(const void* kernel, int threads) {
  int dev = 0, cus = 0, per = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, threads, 0) != hipSuccess) {
    (void)hipGetLastError();
    return 256;  // one workgroup per CU of an MI355X
  }
  return (per > 0 ? per : 1) * (cus > 0 ? cus : 1);
}

int proj_split(int64_t wgs, int max_split) {
  static const int forced = [] {
    const char* e = getenv("ODDE_PROJ_SPLIT");
    return e ? atoi(e) : 0;
  }();
  int s = 1;
  while (max_split % (2 * s) == 0 && (forced > 0 ? 2 * s <= forced : wgs * s < 1024)) s *= 2;
  return s;
}

LaunchScope::LaunchScope(int kernel_id, hipStream_t s, bool events)
    : id(kernel_id), stream(s), slot(-1) {
  g_launches[id].fetch_add(1, std::memory_order_relaxed);
  if (!events) return;
  TimingState& t = timing();
  std::lock_guard<std::mutex> lk(t.mu);
  if (!t.enabled) return;
  hipEvent_t a = get_event(t), b = get_event(t);
  if (!a || !b) return;
  (void)hipEventRecord(a, stream);
  t.recs.push_back({id, a, b});
  slot = static_cast<int>(t.recs.size()) - 1;
}

LaunchScope::~LaunchScope() {
  if (slot < 0) return;
  TimingState& t = timing();
  std::lock_guard<std::mutex> lk(t.mu);
  if (slot < static_cast<int>(t.recs.size())) (void)hipEventRecord(t.recs[slot].b, stream);
}

}  // namespace odde

extern "C" {

int odde_abi_version(void) { return ODDE_ABI_VERSION; }

const char* odde_last_error(void) { return odde::g_error.c_str(); }

int64_t odde_launch_count(int kernel_id) {
  if (kernel_id < 0 || kernel_id >= ODDE_K_COUNT) return -1;
  return odde::g_launches[kernel_id].load();
}

int odde_timing_enable(int on) {
  auto& t = odde::timing();
  std::lock_guard<std::mutex> lk(t.mu);
  t.enabled = on != 0;
  return ODDE_OK;
}

int odde_timing_reset(void) {
  auto& t = odde::timing();
  std::lock_guard<std::mutex> lk(t.mu);
  for (auto& r : t.recs) {
    (void)hipEventSynchronize(r.b);
    t.pool.push_back(r.a);
    t.pool.push_back(r.b);
  }
  t.recs.clear();
  return ODDE_OK;
}

int odde_timing_query(int kernel_id, double* total_ms, int64_t* launches) {
  if (kernel_id < 0 || kernel_id >= ODDE_K_COUNT || !total_ms || !launches)
    return odde::set_error(ODDE_EINVAL, "odde_timing_query: bad argument");
  auto& t = odde::timing();
  std::lock_guard<std::mutex> lk(t.mu);
  double tot = 0.0;
  int64_t cnt = 0;
  for (auto& r : t.recs) {
    if (r.id != kernel_id) continue;
    if (hipEventSynchronize(r.b) != hipSuccess)
      return odde::set_error(ODDE_EHIP, "odde_timing_query: event sync failed");
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, r.a, r.b) != hipSuccess)
      return odde::set_error(ODDE_EHIP, "odde_timing_query: elapsed time failed");
    tot += ms;
    ++cnt;
  }
  *total_ms = tot;
  *launches = cnt;
  return ODDE_OK;
}

}  // extern "C"
