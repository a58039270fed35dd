// Host runtime of libossm_scan: error strings and scratch management.
#include "runtime.hpp"

#include <atomic>
#include <cstdlib>
#include <map>
#include <memory>
#include <mutex>
#include <utility>
#include <vector>

#include "../../include/ossm_scan.h"

namespace ossm {

thread_local LaunchTiming t_launch_timing;

namespace {

thread_local std::string g_last_error;

int release_buffer(void* p, bool captured, const char* what);

struct Scratch {
  void* base = nullptr;       // device buffer: header + payload
  size_t payload = 0;         // payload capacity in bytes
  unsigned int epoch = 0;     // counter of the dispatch-order tags (next_dispatch_tag)
  bool captured = false;      // a HIP graph holds this buffer's address
};

struct Workspace {
  void* base = nullptr;
  size_t bytes = 0;
  bool captured = false;
};

// Buffers a captured graph may still use: never freed (the graph keeps their
// addresses and may be replayed until the process ends).
std::mutex g_retired_mu;
std::vector<void*> g_retired;

// Everything the library keeps for one (device, stream).  `call` is held by a
// StreamCall for the whole of one C call; `scratch` and `workspace` are only
// touched under it.
struct StreamState {
  std::recursive_mutex call;
  Scratch scratch;
  Workspace workspace;
};

std::mutex g_mu;  // guards the map itself (never held while waiting on `call`)
std::map<std::pair<int, hipStream_t>, std::unique_ptr<StreamState>> g_streams;

StreamState& state_of(int dev, hipStream_t stream) {
  std::lock_guard<std::mutex> lock(g_mu);
  auto& slot = g_streams[{dev, stream}];
  if (!slot) slot.reset(new StreamState());
  return *slot;  // never erased: the address stays valid
}

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

int take_launch_timing(const StreamCall& call, LaunchTiming* out) {
  *out = LaunchTiming{};
  if (t_launch_timing.start == nullptr) return OSSM_OK;
  if (call.capturing())
    return set_error(OSSM_ERR_UNSUPPORTED,
                     "ossm_time_next_launch: timing events cannot be recorded under stream capture");
  *out = t_launch_timing;
  t_launch_timing = LaunchTiming{};
  return OSSM_OK;
}

int device_cu_count(int dev) {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> counts[kMaxDevices] = {};
  if (dev < 0 || dev >= kMaxDevices) return 0;
  int n = counts[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
      (void)hipGetLastError();
      return 0;
    }
    counts[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

int choose_scan_order(int dev, bool capturing, int64_t n_workgroups, bool* by_ticket) {
  const char* v = std::getenv("OSSM_SCAN_ORDER");
  const std::string mode = v == nullptr ? std::string("auto") : std::string(v);
  if (mode == "ticket") {
    *by_ticket = true;
  } else if (mode == "dispatch") {
    if (capturing)
      return set_error(OSSM_ERR_UNSUPPORTED,
                       "ossm_scan: OSSM_SCAN_ORDER=dispatch chooses look-back tags on the host per "
                       "call, which a replayed HIP graph would reuse: capture needs ticket order");
    *by_ticket = false;
  } else if (mode == "auto" || mode.empty()) {
    *by_ticket = capturing || n_workgroups * 4 > device_cu_count(dev);
  } else {
    return set_error(OSSM_ERR_INVALID_ARGUMENT,
                     "ossm_scan: OSSM_SCAN_ORDER must be auto, ticket or dispatch, not '" + mode + "'");
  }
  return OSSM_OK;
}

unsigned int next_dispatch_tag(unsigned int& epoch) {
  epoch = (epoch + 1) & (kDispatchTagBase - 1);
  if (epoch == 0) epoch = 1;
  return kDispatchTagBase | epoch;
}

StreamCall::StreamCall(hipStream_t stream) : stream_(stream) {
  if ((status_ = hip_check(hipGetDevice(&device_), "hipGetDevice"))) return;
  lock_ = std::unique_lock<std::recursive_mutex>(state_of(device_, stream).call);
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  const hipError_t e = hipStreamIsCapturing(stream, &cap);
  if (e != hipSuccess) {
    (void)hipGetLastError();  // keep a refused call from surfacing as a later launch error
    status_ = set_error(OSSM_ERR_HIP, std::string("hipStreamIsCapturing: ") + hipGetErrorString(e));
    return;
  }
  capturing_ = cap == hipStreamCaptureStatusActive;
  if (cap == hipStreamCaptureStatusInvalidated)
    status_ = set_error(OSSM_ERR_UNSUPPORTED, "ossm_scan: the stream's graph capture was invalidated");
}

namespace {

int refuse_capture(const char* what) {
  return set_error(OSSM_ERR_UNSUPPORTED,
                   std::string("ossm_scan: the stream is being captured into a HIP graph and the ") +
                       what + "; run this call once eagerly on the stream before capturing it");
}

}  // namespace

int acquire_scratch(StreamCall& call, size_t payload_bytes, int64_t n_workgroups, void** payload,
                    LaunchSync* sync) {
  if (call.status()) return call.status();
  bool by_ticket = true;
  if (int rc = choose_scan_order(call.device(), call.capturing(), n_workgroups, &by_ticket)) return rc;
  Scratch& s = state_of(call.device(), call.stream()).scratch;
  if (s.base == nullptr || s.payload < payload_bytes) {
    if (call.capturing()) return refuse_capture("look-back scratch would have to grow");
    // Grow: earlier launches on this stream may still read the old buffer.
    if (s.base != nullptr) {
      if (int rc = hip_check(hipStreamSynchronize(call.stream()), "hipStreamSynchronize")) return rc;
      if (int rc = release_buffer(s.base, s.captured, "hipFree(scratch)")) return rc;
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
    s.captured = false;
  }
  if (call.capturing()) s.captured = true;
  char* b = static_cast<char*>(s.base);
  sync->ticket = reinterpret_cast<unsigned long long*>(b + kHdrTicket);
  sync->err = reinterpret_cast<unsigned int*>(b + kHdrErr);
  sync->flag = reinterpret_cast<unsigned long long*>(b + kHdrFlag);
  sync->use_ticket = by_ticket ? 1 : 0;
  sync->poison = 0;
  sync->tag = by_ticket ? 0 : next_dispatch_tag(s.epoch);  // ticket order: drawn on the device
  *payload = b + kHdrBytes;
  return OSSM_OK;
}

int acquire_workspace(StreamCall& call, size_t bytes, void** ptr) {
  if (call.status()) return call.status();
  Workspace& w = state_of(call.device(), call.stream()).workspace;
  if (w.base == nullptr || w.bytes < bytes) {
    if (call.capturing()) return refuse_capture("workspace would have to grow");
    if (w.base != nullptr) {
      if (int rc = hip_check(hipStreamSynchronize(call.stream()), "hipStreamSynchronize")) return rc;
      if (int rc = release_buffer(w.base, w.captured, "hipFree(workspace)")) return rc;
      w.base = nullptr;
      w.bytes = 0;
    }
    size_t cap = bytes < (size_t(1) << 20) ? (size_t(1) << 20) : bytes;
    cap = (cap + (size_t(1) << 20) - 1) & ~((size_t(1) << 20) - 1);
    void* p = nullptr;
    if (int rc = hip_check(hipMalloc(&p, cap), "hipMalloc(workspace)")) return rc;
    w.base = p;
    w.bytes = cap;
    w.captured = false;
  }
  if (call.capturing()) w.captured = true;
  *ptr = w.base;
  return OSSM_OK;
}

namespace {

int release_buffer(void* p, bool captured, const char* what) {
  if (captured) {
    std::lock_guard<std::mutex> lock(g_retired_mu);
    g_retired.push_back(p);
    return OSSM_OK;
  }
  return hip_check(hipFree(p), what);
}

}  // namespace

}  // namespace ossm

extern "C" {

int ossm_abi_version(void) { return 16; }

const char* ossm_last_error(void) { return ossm::g_last_error.c_str(); }

uint32_t ossm_device_error_bits(ossm_stream_t stream_v) {
  hipStream_t stream = static_cast<hipStream_t>(stream_v);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0xffffffffu;
  const uint32_t fixed_bits = ossm::noalloc_error_bits(dev);
  if (fixed_bits == 0xffffffffu) return fixed_bits;
  ossm::StreamState& st = ossm::state_of(dev, stream);
  std::lock_guard<std::recursive_mutex> hold(st.call);
  ossm::Scratch& s = st.scratch;
  if (s.base == nullptr) return fixed_bits;
  if (hipStreamSynchronize(stream) != hipSuccess) return 0xffffffffu;
  uint32_t bits = 0;
  char* base = static_cast<char*>(s.base);
  if (hipMemcpy(&bits, base + ossm::kHdrErr, sizeof(bits), hipMemcpyDeviceToHost) != hipSuccess)
    return 0xffffffffu;
  // With the stream drained, every launch on this scratch has run to its end
  // and left the ticket counter at a multiple of 2^32.  A launch that did not
  // (an aborted kernel) leaves it out of step; move it to the next multiple,
  // so that later launches start in step.
  unsigned long long t = 0;
  if (hipMemcpy(&t, base + ossm::kHdrTicket, sizeof(t), hipMemcpyDeviceToHost) == hipSuccess &&
      (t & (ossm::kEpochSpan - 1)) != 0) {
    t = (t | (ossm::kEpochSpan - 1)) + 1;
    (void)hipMemcpy(base + ossm::kHdrTicket, &t, sizeof(t), hipMemcpyHostToDevice);
  }
  if (bits != 0) (void)hipMemset(base + ossm::kHdrErr, 0, sizeof(bits));
  return bits | fixed_bits;
}

int ossm_time_next_launch(void* start_event, void* stop_event) {
  ossm::clear_error();
  if ((start_event == nullptr) != (stop_event == nullptr))
    return ossm::set_error(OSSM_ERR_INVALID_ARGUMENT,
                           "ossm_time_next_launch: give both events or neither");
  ossm::t_launch_timing = {static_cast<hipEvent_t>(start_event), static_cast<hipEvent_t>(stop_event)};
  return OSSM_OK;
}

int ossm_test_skew_tickets(ossm_stream_t stream_v, uint64_t delta) {
  ossm::clear_error();
  hipStream_t stream = static_cast<hipStream_t>(stream_v);
  int dev = 0;
  if (int rc = ossm::hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
  ossm::StreamState& st = ossm::state_of(dev, stream);
  std::lock_guard<std::recursive_mutex> hold(st.call);
  ossm::Scratch& s = st.scratch;
  if (s.base == nullptr)
    return ossm::set_error(OSSM_ERR_INVALID_ARGUMENT,
                           "ossm_test_skew_tickets: no scan has run on this stream yet");
  if (int rc = ossm::hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize")) return rc;
  char* base = static_cast<char*>(s.base);
  unsigned long long t = 0;
  if (int rc = ossm::hip_check(hipMemcpy(&t, base + ossm::kHdrTicket, sizeof(t), hipMemcpyDeviceToHost),
                               "hipMemcpy"))
    return rc;
  t += delta;
  return ossm::hip_check(hipMemcpy(base + ossm::kHdrTicket, &t, sizeof(t), hipMemcpyHostToDevice),
                         "hipMemcpy");
}

}  // extern "C"
