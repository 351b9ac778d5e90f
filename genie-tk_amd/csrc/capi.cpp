// Error state, version and per-kernel timing of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <atomic>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "capi_util.hpp"

namespace gtk {
static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

namespace {
struct Record {
  const char* name;
  hipEvent_t begin, end;
};
std::atomic<bool> g_timing{false};
std::mutex g_mu;
std::vector<Record> g_records;
std::vector<hipEvent_t> g_pool;

hipEvent_t take_event() {
  if (!g_pool.empty()) {
    hipEvent_t e = g_pool.back();
    g_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}
}  // namespace

StageTimer::StageTimer(const char* name, hipStream_t st) : name_(name), st_(st) {
  if (!g_timing.load(std::memory_order_relaxed)) return;
  std::lock_guard<std::mutex> lk(g_mu);
  begin_ = take_event();
  if (begin_) (void)hipEventRecord(begin_, st_);
}

StageTimer::~StageTimer() {
  if (!begin_) return;
  std::lock_guard<std::mutex> lk(g_mu);
  hipEvent_t end = take_event();
  if (!end) {
    g_pool.push_back(begin_);
    return;
  }
  (void)hipEventRecord(end, st_);
  g_records.push_back({name_, begin_, end});
}
int device_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}
}  // namespace gtk

using namespace gtk;

extern "C" const char* gtk_last_error(void) { return g_err; }
extern "C" int gtk_version(void) { return 100; }

extern "C" int gtk_timing_enable(int on) {
  std::lock_guard<std::mutex> lk(g_mu);
  for (auto& r : g_records) {
    (void)hipEventSynchronize(r.end);
    g_pool.push_back(r.begin);
    g_pool.push_back(r.end);
  }
  g_records.clear();
  g_timing.store(on != 0);
  return GTK_OK;
}

extern "C" int gtk_timing_report(char* buf, size_t buf_bytes) {
  GTK_REQUIRE(buf && buf_bytes > 0, GTK_EINVAL, "gtk_timing_report: null buffer");
  struct Agg {
    int n = 0;
    double total = 0, mn = 1e30, mx = 0;
  };
  std::map<std::string, Agg> agg;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    for (auto& r : g_records) {
      float ms = 0.f;
      (void)hipEventSynchronize(r.end);
      if (hipEventElapsedTime(&ms, r.begin, r.end) == hipSuccess) {
        Agg& a = agg[r.name];
        a.n += 1;
        a.total += ms;
        a.mn = ms < a.mn ? ms : a.mn;
        a.mx = ms > a.mx ? ms : a.mx;
      }
      g_pool.push_back(r.begin);
      g_pool.push_back(r.end);
    }
    g_records.clear();
  }
  size_t off = 0;
  buf[0] = 0;
  for (auto& kv : agg) {
    int w = snprintf(buf + off, buf_bytes - off, "%s %d %.6f %.6f %.6f\n", kv.first.c_str(),
                     kv.second.n, kv.second.total, kv.second.mn, kv.second.mx);
    if (w < 0 || (size_t)w >= buf_bytes - off) break;
    off += (size_t)w;
  }
  return GTK_OK;
}
