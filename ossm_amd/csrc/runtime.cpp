// Host runtime of libossm_scan: error strings and scratch management.
#include "runtime.hpp"

#include <cstdlib>
#include <map>
#include <mutex>
#include <utility>

#include "../../include/ossm_scan.h"

namespace ossm {
namespace {

thread_local std::string g_last_error;

struct Scratch {
  void* base = nullptr;       // device buffer: header + payload
  size_t payload = 0;         // payload capacity in bytes
  unsigned int epoch = 0;     // tag of the most recent launch
  unsigned long long next_ticket = 0;  // value of the device counter after all queued launches
};

struct Workspace {
  void* base = nullptr;
  size_t bytes = 0;
};

std::mutex g_mu;
std::map<std::pair<int, hipStream_t>, Scratch> g_scratch;
std::map<std::pair<int, hipStream_t>, Workspace> g_workspace;

}  // namespace

int set_error(int status, const std::string& msg) {
  g_last_error = msg;
  return status;
}

int clear_error() {
  g_last_error.clear();
  return OSSM_OK;
}

int hip_check(hipError_t e, const char* what) {
  if (e == hipSuccess) return OSSM_OK;
  return set_error(OSSM_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

int launch_check(const char* what) {
  return hip_check(hipGetLastError(), what);
}

bool scan_order_by_ticket() {
  static const bool by_ticket = [] {
    const char* v = std::getenv("OSSM_SCAN_ORDER");
    return v == nullptr || std::string(v) != "dispatch";
  }();
  return by_ticket;
}

int acquire_scratch(hipStream_t stream, size_t payload_bytes, uint64_t n_workgroups,
                    void** payload, LaunchSync* sync) {
  const bool by_ticket = scan_order_by_ticket();
  if (!by_ticket) n_workgroups = 0;  // no ticket is drawn
  int dev = 0;
  if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
  std::lock_guard<std::mutex> lock(g_mu);
  Scratch& s = g_scratch[{dev, stream}];
  if (s.base == nullptr || s.payload < payload_bytes) {
    // Grow: earlier launches on this stream may still read the old buffer.
    if (s.base != nullptr) {
      if (int rc = hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize")) return rc;
      if (int rc = hip_check(hipFree(s.base), "hipFree(scratch)")) return rc;
      s.base = nullptr;
    }
    size_t cap = payload_bytes < (size_t(1) << 20) ? (size_t(1) << 20) : payload_bytes;
    cap = (cap + (size_t(1) << 20) - 1) & ~((size_t(1) << 20) - 1);
    void* p = nullptr;
    if (int rc = hip_check(hipMalloc(&p, kHdrBytes + cap), "hipMalloc(scratch)")) return rc;
    if (int rc = hip_check(hipMemset(p, 0, kHdrBytes + cap), "hipMemset(scratch)")) {
      (void)hipFree(p);
      return rc;
    }
    s.base = p;
    s.payload = cap;
    s.epoch = 0;
    s.next_ticket = 0;
  }
  s.epoch += 1;
  if (s.epoch == 0) s.epoch = 1;  // 0 is the tag of never-written memory
  char* b = static_cast<char*>(s.base);
  sync->ticket = reinterpret_cast<unsigned long long*>(b + kHdrTicket);
  sync->err = reinterpret_cast<unsigned int*>(b + kHdrErr);
  sync->base = s.next_ticket;
  sync->tag = s.epoch;
  sync->use_ticket = by_ticket ? 1 : 0;
  s.next_ticket += n_workgroups;
  *payload = b + kHdrBytes;
  return OSSM_OK;
}

int acquire_workspace(hipStream_t stream, size_t bytes, void** ptr) {
  int dev = 0;
  if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
  std::lock_guard<std::mutex> lock(g_mu);
  Workspace& w = g_workspace[{dev, stream}];
  if (w.base == nullptr || w.bytes < bytes) {
    if (w.base != nullptr) {
      if (int rc = hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize")) return rc;
      if (int rc = hip_check(hipFree(w.base), "hipFree(workspace)")) return rc;
      w.base = nullptr;
      w.bytes = 0;
    }
    size_t cap = bytes < (size_t(1) << 20) ? (size_t(1) << 20) : bytes;
    cap = (cap + (size_t(1) << 20) - 1) & ~((size_t(1) << 20) - 1);
    void* p = nullptr;
    if (int rc = hip_check(hipMalloc(&p, cap), "hipMalloc(workspace)")) return rc;
    w.base = p;
    w.bytes = cap;
  }
  *ptr = w.base;
  return OSSM_OK;
}

void release_unlaunched(hipStream_t stream, uint64_t n_workgroups) {
  if (!scan_order_by_ticket()) return;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return;
  std::lock_guard<std::mutex> lock(g_mu);
  auto it = g_scratch.find({dev, stream});
  if (it != g_scratch.end() && it->second.next_ticket >= n_workgroups)
    it->second.next_ticket -= n_workgroups;
}

}  // namespace ossm

extern "C" {

int ossm_abi_version(void) { return 10; }

const char* ossm_last_error(void) { return ossm::g_last_error.c_str(); }

uint32_t ossm_device_error_bits(ossm_stream_t stream_v) {
  hipStream_t stream = static_cast<hipStream_t>(stream_v);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0xffffffffu;
  void* base = nullptr;
  {
    std::lock_guard<std::mutex> lock(ossm::g_mu);
    auto it = ossm::g_scratch.find({dev, stream});
    if (it == ossm::g_scratch.end()) return 0;
    base = it->second.base;
  }
  if (hipStreamSynchronize(stream) != hipSuccess) return 0xffffffffu;
  uint32_t bits = 0;
  char* err = static_cast<char*>(base) + ossm::kHdrErr;
  if (hipMemcpy(&bits, err, sizeof(bits), hipMemcpyDeviceToHost) != hipSuccess) return 0xffffffffu;
  if (bits != 0) (void)hipMemset(err, 0, sizeof(bits));
  return bits;
}

}  // extern "C"
