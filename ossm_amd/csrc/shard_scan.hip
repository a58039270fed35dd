// Sequence (context-parallel) sharding of the D-LinOSS forward: the part of it
// that one GPU can show.  No counterpart in the reference, which runs one
// process per sequence.
//
// With the sequence split into G consecutive shards of lengths len_0 ..
// len_{G-1}, each shard is scanned by the ordinary forward from a zero state
// (on its own GPU in a multi-GPU run).  The recurrence s_t = M s_{t-1} + F bu_t
// is linear, so the true states differ from those by M^(t+1) c_k, where t is
// the step within shard k and c_k the true state entering it.  The carries
// follow from each shard's last zero-start state z_k alone:
//     c_0 = 0,   c_{k+1} = M^(len_k) c_k + z_k,
// an exclusive scan of affine maps over the shards (what would travel between
// GPUs: one complex 2-vector per channel and shard, B*P*16 bytes), after which
// every shard is corrected independently by the fix-up pass
//     s_t += M^(t+1) c_k.
// shard_carry_kernel is that scan (one lane per channel, fp64 powers and
// accumulation), shard_fixup_kernel the fix-up (16 B read and 16 B written per
// state-step: HBM-bound).
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>
#include <string>

#include "../../include/ossm_scan.h"
#include "dlinoss_model.hpp"
#include "runtime.hpp"
#include "scan_device.hpp"

namespace ossm {
namespace {

constexpr int kMaxShards = 64;

struct ShardTable {
  long long start[kMaxShards];  // first row of each shard in the [L, B*P] states
  long long len[kMaxShards];
  int count;
};

// c_k for every shard k, written to carries[k * nc + ch] as (w, x) complex
// pairs; z_k is read from the states row start_k + len_k - 1.
template <int V>
__global__ __launch_bounds__(256) void shard_carry_kernel(typename Dlinoss<V>::Params prm,
                                                          const float4* __restrict__ states,
                                                          ShardTable tab,
                                                          float4* __restrict__ carries, int nc) {
  const int ch = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
  if (ch >= nc) return;
  const auto k = Dlinoss<V>::coef(prm, ch);
  const RMatD M = widen(Dlinoss<V>::matrix(k));
  double cr0 = 0.0, ci0 = 0.0, cr1 = 0.0, ci1 = 0.0;  // (w, x), real and imaginary parts
  // the shards' last states are read kBatch at a time, all in flight before
  // the chain uses them (the chain itself is serial over shards)
  constexpr int kBatch = 8;
  for (int s0 = 0; s0 < tab.count; s0 += kBatch) {
    float4 z[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j)
      if (s0 + j < tab.count)
        z[j] = states[static_cast<size_t>(tab.start[s0 + j] + tab.len[s0 + j] - 1) * nc + ch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int s = s0 + j;
      if (s >= tab.count) break;
      carries[static_cast<size_t>(s) * nc + ch] =
          make_float4(static_cast<float>(cr0), static_cast<float>(ci0), static_cast<float>(cr1),
                      static_cast<float>(ci1));
      // M^len by binary powering in fp64
      RMatD P = mat_identity(M), b = M;
      for (long long n = tab.len[s]; n > 0; n >>= 1) {
        if (n & 1) P = mat_mul(P, b);
        if (n > 1) b = mat_mul(b, b);
      }
      const double nr0 = P.a * cr0 + P.b * cr1 + z[j].x, ni0 = P.a * ci0 + P.b * ci1 + z[j].y;
      const double nr1 = P.c * cr0 + P.d * cr1 + z[j].z, ni1 = P.c * ci0 + P.d * ci1 + z[j].w;
      cr0 = nr0; ci0 = ni0; cr1 = nr1; ci1 = ni1;
    }
  }
}

// s_t += M^(t+1) c for the L rows of one shard.  Workgroup = W waves over
// W*T consecutive steps of 64 channels; each lane forms M^(t0+1) c once (fp64
// power) and then steps it with M, adding it to each of its T states.
template <int V, int T, int W>
__global__ __launch_bounds__(W * kWave) void shard_fixup_kernel(typename Dlinoss<V>::Params prm,
                                                                const float4* __restrict__ carry,
                                                                float4* __restrict__ states, int L,
                                                                int nc, int n_groups) {
  const int lane = threadIdx.x & (kWave - 1);
  const int w = wave_id();
  const int chunk = static_cast<int>(blockIdx.x) / n_groups;
  const int g = static_cast<int>(blockIdx.x) - chunk * n_groups;
  const int ch = g * kWave + lane;
  if (ch >= nc) return;
  const long long t0 = static_cast<long long>(chunk) * (T * W) + static_cast<long long>(w) * T;
  if (t0 >= L) return;
  const auto k = Dlinoss<V>::coef(prm, ch);
  const RMat M = Dlinoss<V>::matrix(k);
  float4 v = mat_apply(mat_pow(M, static_cast<int>(t0) + 1), carry[ch]);
  const int n = static_cast<int>(min(static_cast<long long>(T), L - t0));
  float4 s[T];
#pragma unroll
  for (int i = 0; i < T; ++i)
    if (i < n) s[i] = group_row(states, t0 + i, nc, g)[lane];
#pragma unroll
  for (int i = 0; i < T; ++i) {
    if (i < n) {
      stream_store(&group_row(states, t0 + i, nc, g)[lane], f4add(s[i], v));
      v = mat_apply(M, v);
    }
  }
}

constexpr int kFixT = 16, kFixW = 8;

template <int V>
int shard_carries_v(const float* a, const float* g, const float* dt, const void* states,
                    const ShardTable& tab, void* carries, int64_t nc, int64_t P, hipStream_t stream) {
  const typename Dlinoss<V>::Params prm{a, g, dt, static_cast<int>(P)};
  hipLaunchKernelGGL((shard_carry_kernel<V>), dim3(static_cast<unsigned>((nc + 255) / 256)), dim3(256),
                     0, stream, prm, static_cast<const float4*>(states), tab,
                     static_cast<float4*>(carries), static_cast<int>(nc));
  return launch_check("shard_carry_kernel");
}

template <int V>
int shard_fixup_v(const float* a, const float* g, const float* dt, const void* carry, void* states,
                  int64_t L, int64_t nc, int64_t P, hipStream_t stream) {
  const typename Dlinoss<V>::Params prm{a, g, dt, static_cast<int>(P)};
  const int64_t n_groups = (nc + kWave - 1) / kWave;
  const int64_t n_chunks = (L + kFixT * kFixW - 1) / (kFixT * kFixW);
  if (n_groups * n_chunks > INT_MAX)
    return set_error(OSSM_ERR_UNSUPPORTED, "dlinoss_shard_fixup: problem too large for one launch grid");
  hipLaunchKernelGGL((shard_fixup_kernel<V, kFixT, kFixW>),
                     dim3(static_cast<unsigned>(n_groups * n_chunks)), dim3(kFixW * kWave), 0, stream,
                     prm, static_cast<const float4*>(carry), static_cast<float4*>(states),
                     static_cast<int>(L), static_cast<int>(nc), static_cast<int>(n_groups));
  return launch_check("shard_fixup_kernel");
}

int check_shard_sizes(int64_t L, int64_t B, int64_t P, const char* what) {
  if (L < 0 || B < 0 || P < 0)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, std::string(what) + ": negative size");
  if (L > INT_MAX || B * P > INT_MAX / 2 || P > INT_MAX || L * B * P > (int64_t(1) << 40))
    return set_error(OSSM_ERR_UNSUPPORTED, std::string(what) + ": size exceeds 32-bit indexing");
  return OSSM_OK;
}

}  // namespace
}  // namespace ossm

using namespace ossm;

extern "C" {

int ossm_dlinoss_shard_carries(int variant, const float* a_diag, const float* g_diag,
                               const float* step, const void* states, int64_t length,
                               const int64_t* shard_lengths, int n_shards, void* carries,
                               int64_t batch, int64_t ssm, ossm_stream_t stream_v) {
  clear_error();
  if (int rc = check_shard_sizes(length, batch, ssm, "dlinoss_shard_carries")) return rc;
  if (n_shards < 1 || n_shards > kMaxShards)
    return set_error(OSSM_ERR_INVALID_ARGUMENT,
                     "dlinoss_shard_carries: n_shards must be 1 .. " + std::to_string(kMaxShards));
  if (!shard_lengths) return set_error(OSSM_ERR_INVALID_ARGUMENT, "dlinoss_shard_carries: null shard_lengths");
  ShardTable tab{};
  tab.count = n_shards;
  long long at = 0;
  for (int s = 0; s < n_shards; ++s) {
    if (shard_lengths[s] < 1)
      return set_error(OSSM_ERR_INVALID_ARGUMENT, "dlinoss_shard_carries: every shard needs at least one step");
    tab.start[s] = at;
    tab.len[s] = shard_lengths[s];
    at += shard_lengths[s];
  }
  if (at != length)
    return set_error(OSSM_ERR_INVALID_ARGUMENT,
                     "dlinoss_shard_carries: shard lengths sum to " + std::to_string(at) +
                         ", not the states' length " + std::to_string(length));
  if (batch == 0 || ssm == 0) return OSSM_OK;
  if (!a_diag || !g_diag || !step || !states || !carries)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "dlinoss_shard_carries: null pointer");
  hipStream_t stream = static_cast<hipStream_t>(stream_v);
  const int64_t nc = batch * ssm;
  switch (variant) {
    case OSSM_DLINOSS_IMEX1: return shard_carries_v<OSSM_DLINOSS_IMEX1>(a_diag, g_diag, step, states, tab, carries, nc, ssm, stream);
    case OSSM_DLINOSS_IMEX2: return shard_carries_v<OSSM_DLINOSS_IMEX2>(a_diag, g_diag, step, states, tab, carries, nc, ssm, stream);
    case OSSM_DLINOSS_IM: return shard_carries_v<OSSM_DLINOSS_IM>(a_diag, g_diag, step, states, tab, carries, nc, ssm, stream);
    case OSSM_DLINOSS_EX: return shard_carries_v<OSSM_DLINOSS_EX>(a_diag, g_diag, step, states, tab, carries, nc, ssm, stream);
    default: return set_error(OSSM_ERR_INVALID_ARGUMENT, "Unknown D-LinOSS variant code");
  }
}

int ossm_dlinoss_shard_fixup(int variant, const float* a_diag, const float* g_diag,
                             const float* step, const void* carry, void* states, int64_t length,
                             int64_t batch, int64_t ssm, ossm_stream_t stream_v) {
  clear_error();
  if (int rc = check_shard_sizes(length, batch, ssm, "dlinoss_shard_fixup")) return rc;
  if (length == 0 || batch == 0 || ssm == 0) return OSSM_OK;
  if (!a_diag || !g_diag || !step || !carry || !states)
    return set_error(OSSM_ERR_INVALID_ARGUMENT, "dlinoss_shard_fixup: null pointer");
  hipStream_t stream = static_cast<hipStream_t>(stream_v);
  const int64_t nc = batch * ssm;
  switch (variant) {
    case OSSM_DLINOSS_IMEX1: return shard_fixup_v<OSSM_DLINOSS_IMEX1>(a_diag, g_diag, step, carry, states, length, nc, ssm, stream);
    case OSSM_DLINOSS_IMEX2: return shard_fixup_v<OSSM_DLINOSS_IMEX2>(a_diag, g_diag, step, carry, states, length, nc, ssm, stream);
    case OSSM_DLINOSS_IM: return shard_fixup_v<OSSM_DLINOSS_IM>(a_diag, g_diag, step, carry, states, length, nc, ssm, stream);
    case OSSM_DLINOSS_EX: return shard_fixup_v<OSSM_DLINOSS_EX>(a_diag, g_diag, step, carry, states, length, nc, ssm, stream);
    default: return set_error(OSSM_ERR_INVALID_ARGUMENT, "Unknown D-LinOSS variant code");
  }
}

}  // extern "C"
