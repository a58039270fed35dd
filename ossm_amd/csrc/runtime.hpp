// Host-side runtime shared by the scan entry points: error reporting and the
// per-(device, stream) scratch buffer that carries look-back records, tickets
// and partial sums between workgroups.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>
#include <string>

namespace ossm {

// Error bits a kernel may raise in the scratch header (see ossm_device_error_bits).
constexpr uint32_t kErrSpinTimeout = 1u;
constexpr uint32_t kErrBadTicket = 2u;

// Layout of the scratch header (bytes from the buffer start).
constexpr size_t kHdrTicket = 0;    // uint64_t monotonically increasing ticket counter
constexpr size_t kHdrErr = 64;      // uint32_t error bits
constexpr size_t kHdrBytes = 256;   // payload starts here, 256-byte aligned

// Per-launch synchronisation arguments handed to a look-back kernel.
struct LaunchSync {
  unsigned long long* ticket;  // device counter, shared by all launches on this scratch
  unsigned int* err;           // device error bits
  unsigned long long base;     // value of *ticket when this launch starts
  unsigned int tag;            // epoch tag of this launch's records (never 0)
  int use_ticket;              // 1: chunks follow the ticket counter, 0: dispatch order
};

// Whether look-back kernels order their chunks by the ticket counter (the
// default) or by workgroup index (environment OSSM_SCAN_ORDER=dispatch).
bool scan_order_by_ticket();

// Records the message for ossm_last_error() and returns `status`.
int set_error(int status, const std::string& msg);
int clear_error();

// Checks a HIP call, records "<what>: <hipGetErrorString>" on failure.
int hip_check(hipError_t e, const char* what);

// One C call's hold on a (device, stream).  An entry point that uses the
// stream's scratch or workspace creates one first and keeps it until its last
// launch is enqueued: the ticket base and tag drawn for a launch, and the
// partial sums one launch leaves for the next, then belong to launches that
// reach the stream in the order they were drawn, whatever other host threads
// do on the same stream.  The lock is recursive (an entry point may call
// another on the same stream).  status() is nonzero when the device could not
// be read or the stream is being captured into a graph (launch tags and
// ticket bases are chosen on the host per call, so a replayed graph would
// reuse them: capture is refused with OSSM_ERR_UNSUPPORTED before anything is
// enqueued).
class StreamCall {
 public:
  explicit StreamCall(hipStream_t stream);
  StreamCall(const StreamCall&) = delete;
  StreamCall& operator=(const StreamCall&) = delete;
  int status() const { return status_; }
  hipStream_t stream() const { return stream_; }
  int device() const { return device_; }

 private:
  hipStream_t stream_;
  int device_ = 0;
  int status_ = 0;
  std::unique_lock<std::recursive_mutex> lock_;
};

// Returns a scratch payload of at least `payload_bytes` for the call's stream
// and the launch bookkeeping for a grid of `n_workgroups` look-back
// workgroups.  The payload is zero-filled when first allocated and is never
// cleared again: kernels tag what they write with sync.tag.
int acquire_scratch(StreamCall& call, size_t payload_bytes, uint64_t n_workgroups,
                    void** payload, LaunchSync* sync);

// Returns a plain device workspace of at least `bytes` for the call's stream,
// separate from the tagged look-back records: partial sums written here can
// never be mistaken for a record.  Contents are unspecified; kernels write
// before they read.  Grows on demand (synchronising the stream before freeing
// the old one).
int acquire_workspace(StreamCall& call, size_t bytes, void** ptr);

// Undo the ticket reservation of the last acquire_scratch of this call when
// its kernel failed to launch (the device counter never advanced).
void release_unlaunched(StreamCall& call, uint64_t n_workgroups);

// Launch-error check after a kernel launch (reference: C10_CUDA_KERNEL_LAUNCH_CHECK).
int launch_check(const char* what);

// Error bits of the allocation-free forward's fixed scratch on device `dev`
// (0 if that path never ran there); synchronises the device, clears the bits
// and re-reads its ticket counter.  Defined beside that scratch.
uint32_t noalloc_error_bits(int dev);

}  // namespace ossm
