// Per-kernel HIP-event timing of the library's own launches.
//
// When enabled, every kernel launch of the library is bracketed by two hipEvents
// recorded on the launch stream; moe_mi355x_profile_read() synchronises those events
// and returns count and summed duration per kernel slot.  Disabled (the default), the
// brackets cost one branch.  Host-side only; thread-safe.
#include <atomic>
#include <mutex>
#include <vector>

#include "common.h"

namespace {

struct Rec {
  int slot;
  hipEvent_t a, b;
};

std::mutex g_mu;
std::atomic<bool> g_enabled{false};  // read on every launch without taking the lock
std::vector<Rec> g_recs;
std::vector<hipEvent_t> g_free;

hipEvent_t take_event() {
  if (!g_free.empty()) {
    hipEvent_t e = g_free.back();
    g_free.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

void recycle_all() {
  for (auto& r : g_recs) {
    if (r.a) g_free.push_back(r.a);
    if (r.b) g_free.push_back(r.b);
  }
  g_recs.clear();
}

}  // namespace

int moe_prof_begin(int slot, hipStream_t s) {
  if (!g_enabled.load(std::memory_order_relaxed)) return -1;
  std::lock_guard<std::mutex> lk(g_mu);
  Rec r{slot, take_event(), take_event()};
  if (!r.a || !r.b) return -1;
  if (hipEventRecord(r.a, s) != hipSuccess) return -1;
  g_recs.push_back(r);
  return (int)g_recs.size() - 1;
}

void moe_prof_end(int id, hipStream_t s) {
  if (id < 0) return;
  std::lock_guard<std::mutex> lk(g_mu);
  if (id < (int)g_recs.size()) (void)hipEventRecord(g_recs[id].b, s);
}

extern "C" int moe_mi355x_profile_enable(int on) {
  std::lock_guard<std::mutex> lk(g_mu);
  recycle_all();
  g_enabled.store(on != 0, std::memory_order_relaxed);
  return MOE_OK;
}

extern "C" int moe_mi355x_profile_read(int slot, int* count, double* total_ms) {
  MOE_RETURN_IF(!count || !total_ms || slot < 0 || slot >= MOE_PROF_SLOTS, MOE_ERR_INVALID_ARG);
  std::lock_guard<std::mutex> lk(g_mu);
  int n = 0;
  double tot = 0.0;
  for (auto& r : g_recs) {
    if (r.slot != slot) continue;
    hipError_t e = hipEventSynchronize(r.b);
    if (e != hipSuccess) return (int)e;
    float ms = 0.f;
    e = hipEventElapsedTime(&ms, r.a, r.b);
    if (e != hipSuccess) return (int)e;
    ++n;
    tot += ms;
  }
  *count = n;
  *total_ms = tot;
  return MOE_OK;
}

extern "C" const char* moe_mi355x_profile_slot_name(int slot) {
  static const char* names[MOE_PROF_SLOTS] = {"router_gemm", "topk_softmax", "quant_act", "align",
                                              "gemm_gate_up", "quant_h", "gemm_down", "combine", "linear"};
  return (slot >= 0 && slot < MOE_PROF_SLOTS) ? names[slot] : "";
}
