// Status plumbing, version string and the per-device scratch allocator.
//
// The reference reports shape errors as Err(String) (e.g. src/kernels.rs:98-109);
// the C ABI returns a negative status and keeps the same message in a
// thread-local string readable through bh_last_error().
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <mutex>
#include <string>
#include <vector>

#include "common.hpp"

namespace bh {

namespace {
thread_local std::string g_last_error;

struct Scratch {
  void *ptr = nullptr;
  size_t bytes = 0;
};
std::mutex g_scratch_mu;
std::vector<Scratch> g_scratch;  // indexed by device ordinal * kScratchSlots + slot
// Buffers replaced by a larger one.  They are never freed: a HIP graph
// captured while one was current still holds its address, and replaying that
// graph must find the memory alive.  Growth is at least twofold, so the
// retired buffers of a slot add up to less than its current one.
struct Retired {
  void *ptr;
  size_t bytes;
  int dev;
};
std::vector<Retired> g_retired;
}  // namespace

int fail(int code, const std::string &msg) {
  g_last_error = msg;
  return code;
}

int ok() {
  g_last_error.clear();
  return BH_OK;
}

int check_hip(hipError_t e, const char *what) {
  if (e == hipSuccess) return BH_OK;
  return fail(BH_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

int check_launch(const char *what) {
  return check_hip(hipGetLastError(), what);
}

void *device_scratch(size_t bytes, int slot, hipStream_t stream) {
  int dev = 0;
  if (check_hip(hipGetDevice(&dev), "hipGetDevice") != BH_OK) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  const size_t idx = static_cast<size_t>(dev) * kScratchSlots + slot;
  if (g_scratch.size() <= idx) g_scratch.resize(idx + 1);
  Scratch &s = g_scratch[idx];
  if (s.bytes >= bytes) return s.ptr;
  // Growth allocates.  Under stream capture that would put an allocation
  // (and the new address) into the graph being recorded, so it is refused:
  // the caller runs the call once eagerly at its largest shape first.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (check_hip(hipStreamIsCapturing(stream, &cap), "hipStreamIsCapturing") != BH_OK)
    return nullptr;
  if (cap != hipStreamCaptureStatusNone) {
    fail(BH_ERR_HIP, "scratch of " + std::to_string(bytes) + " bytes needed but " +
                         std::to_string(s.bytes) +
                         " reserved, and the stream is capturing: run this call once outside "
                         "capture at its largest shape before capturing it");
    return nullptr;
  }
  size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
  if (s.bytes <= SIZE_MAX / 2 && want < 2 * s.bytes) want = 2 * s.bytes;
  void *p = nullptr;
  if (check_hip(hipMalloc(&p, want), "scratch hipMalloc") != BH_OK) return nullptr;
  // queued work and captured graphs may still use the old buffer: keep it
  if (s.ptr != nullptr) g_retired.push_back(Retired{s.ptr, s.bytes, dev});
  s.ptr = p;
  s.bytes = want;
  return p;
}

size_t scratch_bytes(int slot) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  const size_t idx = static_cast<size_t>(dev) * kScratchSlots + slot;
  return idx < g_scratch.size() ? g_scratch[idx].bytes : 0;
}

size_t device_cu_count() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return static_cast<size_t>(n);
}

}  // namespace bh

extern "C" const char *bh_last_error(void) { return bh::g_last_error.c_str(); }

extern "C" size_t bh_scratch_retired_bytes(void) {
  std::lock_guard<std::mutex> lock(bh::g_scratch_mu);
  size_t n = 0;
  for (const auto &r : bh::g_retired) n += r.bytes;
  return n;
}

extern "C" int bh_scratch_release(void) {
  std::lock_guard<std::mutex> lock(bh::g_scratch_mu);
  if (bh::g_retired.empty()) return bh::ok();
  int cur = 0;
  if (int e = bh::check_hip(hipGetDevice(&cur), "hipGetDevice")) return e;
  int status = BH_OK;
  std::vector<bh::Retired> keep;
  std::vector<int> synced;
  for (const auto &r : bh::g_retired) {
    bool ok = true;
    if (std::find(synced.begin(), synced.end(), r.dev) == synced.end()) {
      ok = bh::check_hip(hipSetDevice(r.dev), "hipSetDevice") == BH_OK &&
           bh::check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize") == BH_OK;
      if (ok) synced.push_back(r.dev);
    } else {
      ok = bh::check_hip(hipSetDevice(r.dev), "hipSetDevice") == BH_OK;
    }
    if (ok && bh::check_hip(hipFree(r.ptr), "scratch hipFree") == BH_OK) continue;
    status = BH_ERR_HIP;
    keep.push_back(r);
  }
  bh::g_retired.swap(keep);
  (void)hipSetDevice(cur);
  return status == BH_OK ? bh::ok() : status;
}

extern "C" const char *bh_version(void) {
  return "bonsai-hip 0.1.0 (gfx950)";
}

extern "C" size_t bh_pq2_row_bytes(size_t ne0) { return (ne0 + 127) / 128 * 34; }
