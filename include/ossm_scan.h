/*
 * ossm_scan.h — C ABI of the MI355X (gfx950) scan library libossm_scan.so.
 *
 * Drop-in device side of the reference extension `ossm._kernels`
 * (src/ossm/csrc/bindings.cpp:159-224).  Every entry point takes plain device
 * pointers, sizes and a HIP stream (passed as void*), launches asynchronously
 * on that stream, and returns 0 on success or a nonzero status with a message
 * available from ossm_last_error().  Outputs are written, never allocated:
 * the caller (e.g. the Python binding ossm_amd._kernels) allocates them.
 *
 * Layouts (all contiguous, complex = interleaved float re/im = complex64):
 *   D-LinOSS:   a_diag, g_diag, step [P] f32;  bu [L,B,P] c64;
 *               states [L,B,P,2] c64 (component 0 = auxiliary w, 1 = x)
 *   LinOSS:     m11, m12, m21, m22 [P] c64;  b_seq, states [L,B,P,2] c64
 *   sel. D-LinOSS: A, G, step [L|1, B|1, M] f32;  bu [L,B,M] c64;  states [L,B,M,2] c64
 *   selective:  u, dt, gate, out [B,D,L] f32;  A [D,N] f32;  Bm, Cm [B,L,N] f32
 *               (the _bf16 entries: the same layouts with bf16 except A, dA, chunk_states)
 *
 * Scratch: the library keeps, per (device, stream), one zero-initialised
 * buffer of tagged look-back records (never cleared between calls) and one
 * plain workspace for partial sums; both grow on demand (hipMalloc outside
 * the kernels, after synchronising the stream) and live until process exit.
 *
 * Threads and graphs: a call holds its (device, stream) from the launch
 * bookkeeping (scratch, workspace) through its last launch, so calls from
 * several host threads on one stream are safe and reach the stream whole.
 * Each look-back launch draws its chunk order and record tag on the device
 * from the scratch's ticket counter, so a call may be captured into a HIP
 * graph and the graph replayed.  (Outside capture, a launch of at most a
 * quarter as many workgroups as the device has CUs takes the workgroup index
 * as its chunk order and a host-chosen tag instead, saving the ticket's
 * atomic round trip.)  Under capture the scratch and workspace are used as
 * they are: a call that would need them to grow returns OSSM_ERR_UNSUPPORTED
 * before enqueuing anything (run it once eagerly on the stream first), as
 * does OSSM_SCAN_ORDER=dispatch (host-chosen tags for every launch).
 * Buffers a graph captured are never freed.  Replays use the capture
 * stream's scratch: replay the graph on that stream, or ordered with
 * everything else that uses it.
 */
#ifndef OSSM_SCAN_H
#define OSSM_SCAN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* ossm_stream_t; /* hipStream_t */

enum {
  OSSM_OK = 0,
  OSSM_ERR_INVALID_ARGUMENT = 1, /* shape / pointer / variant problem (reference: TORCH_CHECK) */
  OSSM_ERR_HIP = 2,              /* HIP runtime error (reference: AT_CUDA_CHECK) */
  OSSM_ERR_UNSUPPORTED = 3       /* valid request this build does not implement */
};

enum { OSSM_DLINOSS_IMEX1 = 0, OSSM_DLINOSS_IMEX2 = 1, OSSM_DLINOSS_IM = 2, OSSM_DLINOSS_EX = 3 };

/* Library ABI version (bumped on any change of the entry points or their
   behaviour; currently 16). */
int ossm_abi_version(void);

/* Message of the last failing call on this host thread ("" if none). */
const char* ossm_last_error(void);

/*
 * Synchronises `stream` and returns (then clears) the device-side error bits
 * of its scratch buffer: bit 0 = a look-back wait gave up (bounded spin
 * exceeded), bit 1 = a workgroup drew an out-of-range ticket.  0 means every
 * launch on this stream since the last check completed its protocol.  Either
 * failure also makes the affected outputs NaN (the chunk carries that could
 * not be read are NaN), so a failed protocol never returns plausible values.  Once
 * ossm_dlinoss_forward_noalloc has run on the current device, the device is
 * synchronised and the bits of its fixed array are included too.
 */
uint32_t ossm_device_error_bits(ossm_stream_t stream);

/*
 * Test hook, no counterpart in the reference: synchronises `stream` and adds
 * `delta` to the ticket counter of its scratch, as a launch that did not run
 * to its end would leave it.  The next ticket-order look-back launches on
 * the stream then draw out-of-range tickets: they raise bit 1 of
 * ossm_device_error_bits and their carries are NaN, while every kernel still
 * exits normally;
 * ossm_device_error_bits puts the counter back in step.  For tests of the
 * failure path only.
 */
int ossm_test_skew_tickets(ossm_stream_t stream, uint64_t delta);

/*
 * Measurement hook, no counterpart in the reference (for benchmarks and
 * profilers): the next oscillatory-scan kernel that this host thread launches
 * through ossm_dlinoss_{forward,backward} or ossm_linoss_{forward,backward}
 * records `start_event` and `stop_event` (hipEvent_t, created by the caller)
 * as its own start and end, through hipExtLaunchKernel, so no event packet is
 * queued between kernels.
 * hipEventElapsedTime of the pair is then that kernel's duration.  The setting
 * is used once; passing two nulls clears it.  A launch under stream capture
 * does not take it and fails with OSSM_ERR_UNSUPPORTED while it is set.
 */
int ossm_time_next_launch(void* start_event, void* stop_event);

/*
 * D-LinOSS forward, replaces dlinoss_<v>_forward:
 *   dlinoss_imex1.cpp:317-352, dlinoss_imex2.cpp:329-364,
 *   dlinoss_im.cpp:347-382,    dlinoss_ex.cpp:264-299.
 * s_t = M(a,g,dt) s_{t-1} + f(a,g,dt) bu_t per (b,p), s_{-1} = 0; writes all
 * L states, both components.
 */
int ossm_dlinoss_forward(int variant, const float* a_diag, const float* g_diag,
                         const float* step, const void* bu, void* states, int64_t length,
                         int64_t batch, int64_t ssm, ossm_stream_t stream);

/*
 * Allocation-free D-LinOSS forward.  No counterpart in the reference: for
 * callers that cannot allocate device memory (tight serving loops, harnesses
 * that forbid hipMalloc).  Same arguments, results and errors as
 * ossm_dlinoss_forward, but the look-back records live in a fixed 16 MiB
 * device array (plus a 256-byte header) that the library holds on each GPU it
 * runs on until the process ends, so the call allocates nothing.  Limit: half
 * a byte of records per state-step, i.e. at most 33,554,432 state-steps
 * (L*B*P) per call; larger problems return OSSM_ERR_UNSUPPORTED with a
 * message.  Every call on a GPU shares that array: calls that overlap on one
 * GPU (two streams, or two host threads' streams) race and must be ordered by
 * the caller.  May be captured into a HIP graph once it has run eagerly on the
 * device (the first call looks up the array's address).  Its device error
 * bits are reported by ossm_device_error_bits.
 */
int ossm_dlinoss_forward_noalloc(int variant, const float* a_diag, const float* g_diag,
                                 const float* step, const void* bu, void* states,
                                 int64_t length, int64_t batch, int64_t ssm,
                                 ossm_stream_t stream);

/*
 * Sequence sharding of the D-LinOSS forward (context parallelism), the part one
 * GPU runs; no counterpart in the reference, which scans each sequence in one
 * piece.  The sequence is split into n_shards consecutive shards (lengths
 * shard_lengths[0 .. n_shards-1], summing to `length`, at most 64 shards) and
 * each shard's rows of `states` [length, batch, ssm, 2] complex64 were
 * computed by ossm_dlinoss_forward from a zero state.  The true state entering
 * shard k is c_0 = 0, c_{k+1} = M^len_k c_k + z_k, where z_k is shard k's last
 * zero-start state and M the oscillator's transition: ossm_dlinoss_shard_carries
 * writes every c_k to `carries` [n_shards, batch, ssm, 2] complex64 (the
 * exclusive scan over shards that would run across GPUs; powers and sums in
 * fp64).  ossm_dlinoss_shard_fixup then corrects one shard in place,
 * states[t] += M^(t+1) carry for t = 0 .. length-1 of that shard (`states` and
 * `length` the shard's rows, `carry` its c_k [batch, ssm, 2] complex64), after
 * which the states equal those of one ossm_dlinoss_forward over the whole
 * sequence, to rounding.  Neither allocates or uses look-back scratch.
 */
int ossm_dlinoss_shard_carries(int variant, const float* a_diag, const float* g_diag,
                               const float* step, const void* states, int64_t length,
                               const int64_t* shard_lengths, int n_shards, void* carries,
                               int64_t batch, int64_t ssm, ossm_stream_t stream);
int ossm_dlinoss_shard_fixup(int variant, const float* a_diag, const float* g_diag,
                             const float* step, const void* carry, void* states, int64_t length,
                             int64_t batch, int64_t ssm, ossm_stream_t stream);

/*
 * D-LinOSS backward, replaces dlinoss_<v>_backward:
 *   dlinoss_imex1.cpp:354-390, dlinoss_imex2.cpp:366-402,
 *   dlinoss_im.cpp:384-420,    dlinoss_ex.cpp:301-365.
 * grad_output is the gradient w.r.t. component 1 (x) of the states, [L,B,P] c64.
 * Only the state before each chunk (128 or 256 steps, by the launch's tile)
 * is read; the rest is recomputed from bu.  grad_a/grad_g/grad_step [P] f32 are overwritten (not accumulated).
 */
int ossm_dlinoss_backward(int variant, const float* a_diag, const float* g_diag,
                          const float* step, const void* bu, const void* states,
                          const void* grad_output, float* grad_a, float* grad_g,
                          float* grad_step, void* grad_bu, int64_t length, int64_t batch,
                          int64_t ssm, ossm_stream_t stream);

/*
 * complex128 forms of ossm_dlinoss_forward / ossm_dlinoss_backward: the
 * reference's device dispatchers take complex64 and complex128
 * (AT_DISPATCH_COMPLEX_TYPES, dlinoss_imex1_cuda.cu:196, 234; dlinoss_imex2_cuda.cu,
 * dlinoss_im_cuda.cu, dlinoss_ex_cuda.cu alike), with a_diag, g_diag, step of the
 * complex type's value type.  a_diag, g_diag, step [P] fp64; bu, grad_output,
 * grad_bu [L,B,P] c128; states [L,B,P,2] c128; grad_a, grad_g, grad_step [P] fp64
 * (overwritten).  One lane per channel walks the sequence (as the reference's
 * kernels do); the backward reads every step's previous state from states, and
 * the per-oscillator sums run over batch rows in order.
 */
int ossm_dlinoss_forward_f64(int variant, const double* a_diag, const double* g_diag,
                             const double* step, const void* bu, void* states, int64_t length,
                             int64_t batch, int64_t ssm, ossm_stream_t stream);
int ossm_dlinoss_backward_f64(int variant, const double* a_diag, const double* g_diag,
                              const double* step, const void* bu, const void* states,
                              const void* grad_output, double* grad_a, double* grad_g,
                              double* grad_step, void* grad_bu, int64_t length, int64_t batch,
                              int64_t ssm, ossm_stream_t stream);

/*
 * LinOSS scan forward, replaces linoss_scan (linoss_scan.cpp:115-146):
 * s_t = M s_{t-1} + b_t with complex M = [[m11, m12], [m21, m22]] per oscillator.
 */
int ossm_linoss_forward(const void* m11, const void* m12, const void* m21, const void* m22,
                        const void* b_seq, void* states, int64_t length, int64_t batch,
                        int64_t ssm, ossm_stream_t stream);

/*
 * LinOSS scan backward.  The reference has no native backward; this replaces
 * the Python loop of _LinossScanFn.backward (models/linoss.py:83-151):
 * g_t = grad_t + M^H g_{t+1};  grad_b_t = g_t;  grad_M_ij = sum g_i conj(s_j,t-1).
 * grad_output, grad_b: [L,B,P,2] c64;  grad_m: [P,2,2] c64 (overwritten).
 */
int ossm_linoss_backward(const void* m11, const void* m12, const void* m21, const void* m22,
                         const void* states, const void* grad_output, void* grad_m,
                         void* grad_b, int64_t length, int64_t batch, int64_t ssm,
                         ossm_stream_t stream);

/* Number of rows of the selective scan's checkpoint tensor (ceil(length / 32); 0 for length 0). */
int64_t ossm_selective_num_chunks(int64_t length);

/*
 * Selective scan forward, replaces selective_scan_cuda_forward
 * (selective_scan_cuda.cu:253-310) and, on the device, selective_scan_cpu
 * (selective_scan_cpu.cpp:78-166):
 *   h_t = exp(dt_t A_dn) h_{t-1} + dt_t Bm_tn u_t,  y_t = sum_n Cm_tn h_t,
 *   out_t = y_t * silu(gate_t)  (out = y when gate == NULL).
 * raw_out [B,D,L] receives y (may be NULL, or equal to out when gate == NULL).
 * chunk_states [B,D,n_chunks,2N] f32 (may be NULL) receives checkpoints of the
 * state: row c holds h after step 32c+15 (first N) and after step 32c+31
 * (last N); a checkpoint past the end of the sequence holds the final state.
 * 1 <= dstate <= 256.
 */
int ossm_selective_forward(const float* u, const float* dt, const float* A, const float* Bm,
                           const float* Cm, const float* gate, float* out, float* raw_out,
                           float* chunk_states, int64_t batch, int64_t dim, int64_t length,
                           int64_t dstate, ossm_stream_t stream);

/*
 * Selective scan backward, replaces selective_scan_cuda_backward
 * (selective_scan_cuda.cu:312-393) and selective_scan_cpu_backward
 * (selective_scan_cpu.cpp:168-360).  chunk_states and raw_out must come from
 * ossm_selective_forward on the same inputs (raw_out is read only when a gate
 * is given, for dgate).  Writes du, ddt [B,D,L], dA [D,N], dB, dC [B,L,N]
 * (all overwritten) and dgate [B,D,L] (zeros when gate == NULL; may be NULL
 * then).  The sums over channels (dB, dC) and over batch and time (dA) are
 * formed in a fixed order: results are deterministic.
 */
int ossm_selective_backward(const float* grad_out, const float* u, const float* dt,
                            const float* A, const float* Bm, const float* Cm, const float* gate,
                            const float* chunk_states, const float* raw_out, float* du,
                            float* ddt, float* dA, float* dB, float* dC, float* dgate,
                            int64_t batch, int64_t dim, int64_t length, int64_t dstate,
                            ossm_stream_t stream);

/*
 * Selective D-LinOSS forward, replaces sdlinoss_<v>_forward (bindings.cpp:60-106,
 * 169-176; dispatcher sdlinoss_imex1.cpp:317-355, CPU kernel :33-97, and siblings).
 * Per step, dt = clamp(step, 1e-6, 1): comb = -a x + bu, tmpw = alpha w + dt^2 comb,
 * w' = tmpw / S, x' = x + w', with (alpha, S) per variant:
 *   imex1 (1, max(1 + dt g, 1e-6)), imex2 (1 - dt g, max(1 + dt^2 a, 1e-6)),
 *   im (1, max(1 + dt g + dt^2 a, 1e-6)), ex (1 - dt g, 1).
 * A, G, step are fp32 [X_len, X_batch, M] contiguous with X_len in {1, length} and
 * X_batch in {1, batch} (broadcast over time / batch); bu [L,B,M] c64; states
 * [L,B,M,2] c64 (component 0 = w, 1 = x).  With all three broadcast over time
 * the scan runs on the D-LinOSS kernels (per-channel constant coefficients);
 * environment OSSM_SDL_TB_OSC=0 keeps the selective kernels.
 */
int ossm_sdlinoss_forward(int variant, const float* A, int64_t a_len, int64_t a_batch,
                          const float* G, int64_t g_len, int64_t g_batch, const float* step,
                          int64_t s_len, int64_t s_batch, const void* bu, void* states,
                          int64_t length, int64_t batch, int64_t ssm, ossm_stream_t stream);

/*
 * Selective D-LinOSS backward, replaces sdlinoss_<v>_backward (dispatcher
 * sdlinoss_imex1.cpp:357-425, CPU kernel :99-231, and siblings).  states must be the forward's output on the same inputs (the
 * backward reads it at sub-chunk starts only and recomputes the steps in between).
 * Writes grad_bu [L,B,M] c64 and grad_A, grad_G, grad_step with the shapes of A, G,
 * step: per-step gradients summed over the broadcast axes (sdlinoss_cpu_utils.h:84-97)
 * in a fixed order.  grad_step is zero where step was clamped.
 */
int ossm_sdlinoss_backward(int variant, const float* A, int64_t a_len, int64_t a_batch,
                           const float* G, int64_t g_len, int64_t g_batch, const float* step,
                           int64_t s_len, int64_t s_batch, const void* bu, const void* states,
                           const void* grad_output, float* grad_A, float* grad_G,
                           float* grad_step, void* grad_bu, int64_t length, int64_t batch,
                           int64_t ssm, ossm_stream_t stream);

/*
 * complex128 forms of ossm_linoss_forward / ossm_linoss_backward: the reference's
 * device kernel dispatches complex128 too (linoss_scan_cuda.cu:139).  m_ij [P],
 * b_seq, states, grad_output, grad_b [L,B,P,2], grad_m [P,2,2], all c128.  One lane
 * per channel walks the sequence; grad_m is summed over batch rows in order.
 */
int ossm_linoss_forward_f64(const void* m11, const void* m12, const void* m21, const void* m22,
                            const void* b_seq, void* states, int64_t length, int64_t batch,
                            int64_t ssm, ossm_stream_t stream);
int ossm_linoss_backward_f64(const void* m11, const void* m12, const void* m21, const void* m22,
                             const void* states, const void* grad_output, void* grad_m,
                             void* grad_b, int64_t length, int64_t batch, int64_t ssm,
                             ossm_stream_t stream);

/*
 * complex128 forms of ossm_sdlinoss_forward / ossm_sdlinoss_backward: the reference's device kernels
 * dispatch complex128 too (sdlinoss_imex1_cuda.cu:232, 271, and siblings).  A, G,
 * step are fp64 [X_len, X_batch, M]; bu, states, grad_output, grad_bu are c128
 * with the layouts above; grad_A, grad_G, grad_step fp64.  One lane per channel
 * walks the sequence (the backward reads every step's previous state from states);
 * broadcast gradients are summed in a fixed order.
 */
int ossm_sdlinoss_forward_f64(int variant, const double* A, int64_t a_len, int64_t a_batch,
                              const double* G, int64_t g_len, int64_t g_batch, const double* step,
                              int64_t s_len, int64_t s_batch, const void* bu, void* states,
                              int64_t length, int64_t batch, int64_t ssm, ossm_stream_t stream);
int ossm_sdlinoss_backward_f64(int variant, const double* A, int64_t a_len, int64_t a_batch,
                               const double* G, int64_t g_len, int64_t g_batch,
                               const double* step, int64_t s_len, int64_t s_batch, const void* bu,
                               const void* states, const void* grad_output, double* grad_A,
                               double* grad_G, double* grad_step, void* grad_bu, int64_t length,
                               int64_t batch, int64_t ssm, ossm_stream_t stream);

/*
 * bf16 storage variants of the two entries above.  No counterpart in the
 * reference, whose selective-scan extension is fp32 only
 * (selective_scan_cuda.cu:253-393); they serve callers that keep activations
 * in bf16 (the reference's bridge upcasts them to fp32 first,
 * _selective_scan.py:141-160).  u, dt, gate, out, raw_out, Bm, Cm, grad_out,
 * du, ddt, dgate, dB, dC are bf16 (pointers as void*); A, dA and chunk_states
 * stay fp32.  Loads widen exactly to fp32, the recurrence and every sum run in
 * fp32 (also across the 16-state passes), and each stored value is rounded to
 * nearest-even once.
 */
int ossm_selective_forward_bf16(const void* u, const void* dt, const float* A, const void* Bm,
                                const void* Cm, const void* gate, void* out, void* raw_out,
                                float* chunk_states, int64_t batch, int64_t dim, int64_t length,
                                int64_t dstate, ossm_stream_t stream);

int ossm_selective_backward_bf16(const void* grad_out, const void* u, const void* dt,
                                 const float* A, const void* Bm, const void* Cm, const void* gate,
                                 const float* chunk_states, const void* raw_out, void* du,
                                 void* ddt, float* dA, void* dB, void* dC, void* dgate,
                                 int64_t batch, int64_t dim, int64_t length, int64_t dstate,
                                 ossm_stream_t stream);

/*
 * Selective scan with a per-channel skip D, an extension with no counterpart in
 * the reference (whose selective kernels take no D, selective_scan_cuda.cu:
 * 253-393; BASELINE configs 3 and 4 name a D skip): the forward of
 * ossm_selective_forward (elem OSSM_ELEM_F32) or ossm_selective_forward_bf16
 * (OSSM_ELEM_BF16) with y_t = sum_n Cm_tn h_t + D u_t, i.e.
 *   raw_out = y + D u,  out = raw_out * silu(gate)  (out = raw_out without a gate),
 * fused into the scan kernel.  d_skip [dim] f32, not null.
 */
enum { OSSM_ELEM_F32 = 0, OSSM_ELEM_BF16 = 1 };
int ossm_selective_forward_skip(int elem, const void* u, const void* dt, const float* A,
                                const void* Bm, const void* Cm, const float* d_skip,
                                const void* gate, void* out, void* raw_out, float* chunk_states,
                                int64_t batch, int64_t dim, int64_t length, int64_t dstate,
                                ossm_stream_t stream);

/*
 * Backward of ossm_selective_forward_skip: the gradients of
 * ossm_selective_backward / _bf16 (raw_out from the skip forward, which holds
 * y + D u) with du += D gy and dD[d] = sum over batch and time of gy u, where
 * gy = grad_out * silu(gate) (grad_out without a gate).  dD [dim] f32, summed
 * in a fixed order (deterministic).  Both run in the scan kernel.
 */
int ossm_selective_backward_skip(int elem, const void* grad_out, const void* u, const void* dt,
                                 const float* A, const void* Bm, const void* Cm,
                                 const float* d_skip, const void* gate, const float* chunk_states,
                                 const void* raw_out, void* du, void* ddt, float* dA, void* dB,
                                 void* dC, float* dD, void* dgate, int64_t batch, int64_t dim,
                                 int64_t length, int64_t dstate, ossm_stream_t stream);

/*
 * Diagonal complex scan x_t = lambda_p * x_{t-1} + b_t, x_{-1} = 0, per channel
 * (b, p): replaces lru_scan and s5_scan (dispatchers lru_scan.cpp:126-146 and
 * s5_scan.cpp:126-146, CPU kernels lru_scan.cpp:10-58 / s5_scan.cpp:10-66, CUDA
 * lru_scan_cuda.cu:77-115).  lambda_real, lambda_imag [state]; b_seq and out
 * [L, B, state] complex64 (the reference's [L, B, state, 2] real view).
 */
int ossm_diag_scan_forward(const float* lambda_real, const float* lambda_imag, const void* b_seq,
                           void* out, int64_t length, int64_t batch, int64_t state,
                           ossm_stream_t stream);

/*
 * Native backward of the diagonal scan; the reference runs it as a Python loop
 * (_LRUScanFn.backward lru.py:52-80, _S5ScanFn.backward s5.py:137-165).  From the
 * forward's states and grad_output [L, B, state] complex64: grad_b_t = g_t with
 * g_t = grad_output_t + conj(lambda) g_{t+1}, and grad_lambda [state] complex64 =
 * sum over t, b of g_t conj(x_{t-1}) (summed in fp64 in a fixed order).
 */
int ossm_diag_scan_backward(const float* lambda_real, const float* lambda_imag, const void* states,
                            const void* grad_output, void* grad_lambda, void* grad_b,
                            int64_t length, int64_t batch, int64_t state, ossm_stream_t stream);

/* fp64 (complex128) twins of the two entries above (the reference dispatches
 * lru_scan / s5_scan over float and double, lru_scan_cuda.cu:102). */
int ossm_diag_scan_forward_f64(const double* lambda_real, const double* lambda_imag,
                               const void* b_seq, void* out, int64_t length, int64_t batch,
                               int64_t state, ossm_stream_t stream);

int ossm_diag_scan_backward_f64(const double* lambda_real, const double* lambda_imag,
                                const void* states, const void* grad_output, void* grad_lambda,
                                void* grad_b, int64_t length, int64_t batch, int64_t state,
                                ossm_stream_t stream);

/*
 * Fused D-LinOSS layer forward, replaces the body of DampedLinOSSLayer.forward
 * after the parameter projection (dlinoss.py:210-247: bu = u B^T as two real
 * GEMMs, permutes, run_dlinoss, y = Re(x C^T) + D u).  inputs / outputs
 * [batch, length, hidden] fp32 row-major; B [ssm, hidden, 2] and C
 * [hidden, ssm, 2] (real, imaginary parts last, the layer's parameter layout);
 * D [hidden]; a_diag, g_diag, step [ssm] as returned by _project_parameters
 * (dlinoss.py:249-264).  bu and the states stay on chip.  carries (may be
 * null): [batch, ceil(length / 32), ssm] complex 2-vectors (4 floats), the
 * state entering each 32-step chunk, for ossm_dlinoss_layer_backward.  hidden
 * and ssm up to 256 (OSSM_ERR_UNSUPPORTED beyond).
 */
int ossm_dlinoss_layer_forward(int variant, const float* inputs, const float* B, const float* C,
                               const float* D, const float* a_diag, const float* g_diag,
                               const float* step, float* outputs, void* carries, int64_t batch,
                               int64_t length, int64_t hidden, int64_t ssm, ossm_stream_t stream);

/*
 * Backward of ossm_dlinoss_layer_forward (the reference differentiates
 * dlinoss.py:210-247 with autograd around dlinoss_<v>_backward): from the
 * inputs, grad_output [batch, length, hidden] and the forward's carries,
 * writes grad_inputs [batch, length, hidden], grad_a / grad_g / grad_step
 * [ssm], and the two factors of the weight gradients, grad_bu and x_conj
 * [batch, length, ssm] complex (grad of bu; x with its imaginary part
 * negated): grad_B[p, h, c] = sum_{b,t} grad_bu[b,t,p].c u[b,t,h] and
 * grad_C[h, p, c] = sum_{b,t} grad_output[b,t,h] x_conj[b,t,p].c, plain GEMMs
 * the caller runs; grad_D = sum grad_output * inputs.  OSSM_ERR_UNSUPPORTED
 * when hidden and ssm need more LDS than one workgroup has (e.g. both 256).
 */
int ossm_dlinoss_layer_backward(int variant, const float* inputs, const float* grad_output,
                                const float* B, const float* C, const float* D,
                                const float* a_diag, const float* g_diag, const float* step,
                                const void* carries, float* grad_inputs, void* grad_bu,
                                void* x_conj, float* grad_a, float* grad_g, float* grad_step,
                                int64_t batch, int64_t length, int64_t hidden, int64_t ssm,
                                ossm_stream_t stream);

/*
 * Selective scan in the Mamba mixer's layout (mambarec.py:136-184 feeds the
 * scan transposed copies; this reads the mixer's tensors in place).  u, dt,
 * gate [batch, length, dim] with row strides ld_u, ld_dt, ld_z (>= dim); dt is
 * given before its softplus: the scan uses softplus(dt + dt_bias[d])
 * (mambarec.py:155, torch's threshold 20; dt_bias may be null); B, C
 * [batch, length, dstate] views with row stride ld_bc (the x_proj output
 * split, mambarec.py:153); A [dim, dstate].  out, raw_out dense
 * [batch, length, dim]; chunk_states as ossm_selective_forward.  Same
 * recurrence and gate as ossm_selective_forward (selective_scan_cuda.cu:253-310).
 */
int ossm_selective_mamba_forward(const float* u, int64_t ld_u, const float* dt, int64_t ld_dt,
                                 const float* dt_bias, const float* A, const float* B,
                                 const float* C, int64_t ld_bc, const float* gate, int64_t ld_z,
                                 float* out, float* raw_out, float* chunk_states, int64_t batch,
                                 int64_t dim, int64_t length, int64_t dstate, ossm_stream_t stream);

/*
 * Backward of ossm_selective_mamba_forward (selective_scan_cuda.cu:312-393 in
 * this layout).  du, ddt, dgate dense [batch, length, dim]; ddt is the gradient
 * w.r.t. dt before the softplus (the dt_bias gradient is its sum over batch and
 * length); dA [dim, dstate]; dB, dC dense [batch, length, dstate].
 */
int ossm_selective_mamba_backward(const float* grad_out, const float* u, int64_t ld_u,
                                  const float* dt, int64_t ld_dt, const float* dt_bias,
                                  const float* A, const float* B, const float* C, int64_t ld_bc,
                                  const float* gate, int64_t ld_z, const float* chunk_states,
                                  const float* raw_out, float* du, float* ddt, float* dA,
                                  float* dB, float* dC, float* dgate, int64_t batch, int64_t dim,
                                  int64_t length, int64_t dstate, ossm_stream_t stream);

/*
 * The Mamba mixer's causal depthwise convolution + SiLU (mambarec.py:143-150:
 * pad K-1 on the left, Conv1d(groups=D), SiLU), in the [batch, length, dim]
 * layout: out[b,t,d] = silu(bias[d] + sum_k weight[d,k] x[b,t-K+1+k,d]).  x has
 * row stride ld_x (the x half of in_proj's output); weight [dim, width]
 * (Conv1d's [dim, 1, width]); bias [dim] or null; out dense.  width 1..8.
 */
int ossm_mamba_conv_forward(const float* x, int64_t ld_x, const float* weight, const float* bias,
                            float* out, int64_t batch, int64_t length, int64_t dim, int64_t width,
                            ossm_stream_t stream);

/* Backward of the above: grad_x dense [batch, length, dim]; grad_weight
 * [dim, width] and grad_bias [dim] (may be null) summed in a fixed order. */
int ossm_mamba_conv_backward(const float* x, int64_t ld_x, const float* weight, const float* bias,
                             const float* grad_out, float* grad_x, float* grad_weight,
                             float* grad_bias, int64_t batch, int64_t length, int64_t dim,
                             int64_t width, ossm_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* OSSM_SCAN_H */
