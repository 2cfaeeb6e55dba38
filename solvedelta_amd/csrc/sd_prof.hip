// Opt-in per-kernel timing with HIP events on the launch stream (used by the
// benchmark to measure each kernel's average duration inside its timed region).
// Disabled by default; when disabled every hook is a branch on a flag.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>
#include <map>
#include <string>
#include <vector>
#include "sd_internal.h"

namespace sd {
namespace {
struct Rec { const char* name; hipEvent_t a, b; };
bool g_on = false;
std::vector<Rec> g_recs;
std::vector<hipEvent_t> g_pool;
std::map<std::string, std::pair<double, long>> g_acc;  // name -> (total ms, count)
const char* g_pending = nullptr;
hipEvent_t g_start;

hipEvent_t get_event() {
  if (!g_pool.empty()) { hipEvent_t e = g_pool.back(); g_pool.pop_back(); return e; }
  hipEvent_t e;
  (void)hipEventCreate(&e);
  return e;
}
void drain() {
  for (Rec& r : g_recs) {
    (void)hipEventSynchronize(r.b);
    float ms = 0.f;
    (void)hipEventElapsedTime(&ms, r.a, r.b);
    auto& acc = g_acc[r.name];
    acc.first += ms;
    acc.second += 1;
    g_pool.push_back(r.a);
    g_pool.push_back(r.b);
  }
  g_recs.clear();
}
}  // namespace

void prof_begin(const char* name, hipStream_t st) {
  if (!g_on) return;
  g_pending = name;
  g_start = get_event();
  (void)hipEventRecord(g_start, st);
}

void prof_end(hipStream_t st) {
  if (!g_on || !g_pending) return;
  hipEvent_t e = get_event();
  (void)hipEventRecord(e, st);
  g_recs.push_back({g_pending, g_start, e});
  g_pending = nullptr;
  if (g_recs.size() > 4096) drain();
}

}  // namespace sd

extern "C" {
// Enables (1) or disables (0) per-kernel timing; enabling clears the totals.
int sd_profile_enable(int on) {
  sd::drain();
  if (on) sd::g_acc.clear();
  sd::g_on = on != 0;
  return 0;
}

// Writes "name total_ms count" lines into buf; returns the bytes needed.
size_t sd_profile_read(char* buf, size_t len) {
  sd::drain();
  std::string out;
  char line[256];
  for (auto& kv : sd::g_acc) {
    snprintf(line, sizeof line, "%s %.6f %ld\n", kv.first.c_str(), kv.second.first,
             kv.second.second);
    out += line;
  }
  if (buf && len) {
    size_t n = out.size() < len - 1 ? out.size() : len - 1;
    memcpy(buf, out.data(), n);
    buf[n] = 0;
  }
  return out.size() + 1;
}
}
