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
constexpr size_t kHdrFlag = 128;    // uint64_t: tag of the launch whose outputs are zeroed
constexpr size_t kHdrBytes = 256;   // payload starts here, 256-byte aligned

// Per-launch synchronisation arguments handed to a look-back kernel.
//
// Ticket order (the default): every workgroup draws t = ticket++ when it
// starts.  Each launch starts with the counter at a multiple of 2^32
// (kEpochSpan): the low 32 bits of t are the workgroup's order in the launch,
// the high 32 bits the launch's epoch, and the records' tag is the epoch + 1.
// The workgroup that draws the launch's last order advances the counter to
// the next multiple of 2^32.  Nothing per launch is chosen on the host, so a
// launch captured into a HIP graph draws fresh tags and orders on every
// replay.  Dispatch order draws no ticket: the order is the workgroup index
// and the host chooses the tag per call.  The two tag ranges are disjoint
// (ticket order 1 .. 2^31 - 1, dispatch order 2^31 .. 2^32 - 1), so launches
// of either order can follow each other on one scratch.
struct LaunchSync {
  unsigned long long* ticket;  // device counter, shared by all launches on this scratch
  unsigned int* err;           // device error bits
  unsigned long long* flag;    // tag of the launch whose accumulated outputs are zeroed
  unsigned int tag;            // records' tag: set on the device in ticket order, by the host in dispatch order
  int use_ticket;              // 1: chunks follow the ticket counter, 0: dispatch order
  int poison;                  // 0 from the host; 1 on the device when the ticket was out of range
};

constexpr unsigned long long kEpochSpan = 1ull << 32;

// First tag of the host-chosen (dispatch-order) range.
constexpr unsigned int kDispatchTagBase = 0x80000000u;

// Whether a look-back launch of `n_workgroups` workgroups on device `dev`
// orders its chunks by the ticket counter (*by_ticket = true) or by workgroup
// index.  Environment OSSM_SCAN_ORDER, read per call: "ticket" or "dispatch"
// forces one; unset or "auto" takes dispatch order for a grid of at most a
// quarter as many workgroups as the device has CUs, outside stream capture,
// and ticket order otherwise.  Such a grid is resident at once on an idle
// device, and the ticket's atomic round trip is ~1 us of a ~10 us launch.
//
// The quarter bounds what concurrent launches can do.  A dispatch-order
// workgroup may wait on one of lower index that another XCD has not yet
// dispatched; dispatch-order launches on other streams whose waiting
// workgroups fill the XCDs each other's next workgroup needs would stall
// until the bounded spin gives up (NaN, error bit).  Ticket-order launches
// always drain, since they wait only on workgroups already running.  With a
// launch's share of an XCD at most a quarter of its CUs, filling one XCD
// takes four other such launches, five at once, each of workgroups that hold
// a whole CU.  Forced dispatch order under capture returns
// OSSM_ERR_UNSUPPORTED (its tag is chosen on the host, which a replay would
// reuse).
int choose_scan_order(int dev, bool capturing, int64_t n_workgroups, bool* by_ticket);

// Compute units of device `dev`, looked up once per device (0 when the query
// fails).
int device_cu_count(int dev);

// Next host-chosen tag of a dispatch-order launch from the counter `epoch`:
// kDispatchTagBase .. 2^32 - 1, never a ticket-order tag.
unsigned int next_dispatch_tag(unsigned int& epoch);

// Events that the next oscillatory-scan launch on this host thread records as
// its own start and end (ossm_time_next_launch); both null when unset.
struct LaunchTiming {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
};
extern thread_local LaunchTiming t_launch_timing;

// Takes (and clears) this thread's launch timing for a launch on `call`'s
// stream.  A set timing under stream capture is refused: returns
// OSSM_ERR_UNSUPPORTED and leaves it set.
class StreamCall;
int take_launch_timing(const StreamCall& call, LaunchTiming* out);

// Records the message for ossm_last_error() and returns `status`.
int set_error(int status, const std::string& msg);
int clear_error();

// Checks a HIP call, records "<what>: <hipGetErrorString>" on failure.
int hip_check(hipError_t e, const char* what);

// One C call's hold on a (device, stream).  An entry point that uses the
// stream's scratch or workspace creates one first and keeps it until its last
// launch is enqueued: the partial sums one launch leaves for the next then
// belong to launches that reach the stream in the order they were enqueued,
// whatever other host threads do on the same stream.  The lock is recursive
// (an entry point may call another on the same stream).  status() is nonzero
// when the device could not be read.  capturing() is true while the stream is
// being captured into a HIP graph: the scratch and workspace are then used as
// they are (a capture that would need them to grow is refused with
// OSSM_ERR_UNSUPPORTED) and are never freed afterwards, since the graph keeps
// their addresses.
class StreamCall {
 public:
  explicit StreamCall(hipStream_t stream);
  StreamCall(const StreamCall&) = delete;
  StreamCall& operator=(const StreamCall&) = delete;
  int status() const { return status_; }
  hipStream_t stream() const { return stream_; }
  int device() const { return device_; }
  bool capturing() const { return capturing_; }

 private:
  hipStream_t stream_;
  int device_ = 0;
  int status_ = 0;
  bool capturing_ = false;
  std::unique_lock<std::recursive_mutex> lock_;
};

// Returns a scratch payload of at least `payload_bytes` for the call's stream
// and the launch bookkeeping of a look-back kernel of `n_workgroups`
// workgroups (its order from choose_scan_order).  The payload is zero-filled
// when first allocated and is never cleared again: kernels tag what they
// write with sync.tag.  Under capture, forced dispatch order is refused (its
// tag is chosen on the host) and so is a payload larger than the current one.
int acquire_scratch(StreamCall& call, size_t payload_bytes, int64_t n_workgroups, void** payload,
                    LaunchSync* sync);

// Returns a plain device workspace of at least `bytes` for the call's stream,
// separate from the tagged look-back records: partial sums written here can
// never be mistaken for a record.  Contents are unspecified; kernels write
// before they read.  Grows on demand (synchronising the stream before freeing
// the old one, unless a graph captured it); refused under capture when it
// would have to grow.
int acquire_workspace(StreamCall& call, size_t bytes, void** ptr);

// Launch-error check after a kernel launch (reference: C10_CUDA_KERNEL_LAUNCH_CHECK).
int launch_check(const char* what);

// Error bits of the allocation-free forward's fixed scratch on device `dev`
// (0 if that path never ran there); synchronises the device, clears the bits
// and re-reads its ticket counter.  Defined beside that scratch.
uint32_t noalloc_error_bits(int dev);

}  // namespace ossm
