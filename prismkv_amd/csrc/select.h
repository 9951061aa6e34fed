// Top-16 selection primitives shared by the route, decode and compat
// kernels: 44-bit bucket keys and a single-wave exact Top-16.
#pragma once

#include "common.h"

namespace prismkv {
namespace {

__device__ __forceinline__ uint64_t make_key(float prob, int bucket) {
  return ((uint64_t)__float_as_uint(prob) << 12) | (uint64_t)(4095 - bucket);
}
__device__ __forceinline__ int key_bucket(uint64_t k) { return 4095 - (int)(k & 4095u); }

// Number of keys greater than x among v[0 .. 16 * ceil(n / 16)), n uniform
// across the wave; entries past n must be zero (a zero key is never
// greater).  Reads go in chunks of 8 pairs with no branch between them.
__device__ __forceinline__ int count_greater(const unsigned long long* v, int n, unsigned long long x) {
  const ulonglong2* v2 = reinterpret_cast<const ulonglong2*>(v);
  int r = 0;
  for (int j0 = 0; 2 * j0 < n; j0 += 8) {
    ulonglong2 o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = v2[j0 + j];
#pragma unroll
    for (int j = 0; j < 8; ++j) r += (o[j].x > x) + (o[j].y > x);
  }
  return r;
}

// Inclusive prefix sum over the lanes of one wave (int).
__device__ __forceinline__ int wave_scan_i(int v) { return (int)wave_incl_scan((unsigned)v); }

// Top-16 of the keys keys[0..64*K) (0 = empty; nonzero keys unique), in rank
// order, into out[0..16) (0 padding); run by one whole wave, no barriers.
// tau = the 16th largest per-lane maximum (lane maxima ranked against each
// other with broadcast LDS reads): at least 16 keys are >= tau and at most 16
// lanes hold such keys, so the <= 16K candidates >= tau are ranked exactly.
// `scratch` holds 64 + 16K keys rounded up to 16 (16-byte aligned).  Returns
// the number of winners.
template <int K>
__device__ int wave_top16(const unsigned long long* keys, unsigned long long* scratch, unsigned long long* out) {
  const int lane = threadIdx.x & 63;
  unsigned long long kk[K], lm = 0;
#pragma unroll
  for (int i = 0; i < K; ++i) {
    kk[i] = keys[lane + 64 * i];
    lm = kk[i] > lm ? kk[i] : lm;
  }
  unsigned long long* mx = scratch;        // [64]
  unsigned long long* cand = scratch + 64; // [16K]
  mx[lane] = lm;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_s_waitcnt(0);
  const int r = lm > 0 ? count_greater(mx, 64, lm) : 64;
  const unsigned long long at15 = __ballot(r == kTop - 1);
  unsigned long long tau = 1;  // dead keys (0) never qualify
  if (at15) {
    const int src = __ffsll((long long)at15) - 1;
    // readlane returns int: widen through unsigned so the low word is not sign-extended
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(lm >> 32), src);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)lm, src);
    tau = ((unsigned long long)hi << 32) | (unsigned long long)lo;
  }
  int mine = 0;
#pragma unroll
  for (int i = 0; i < K; ++i) mine += kk[i] >= tau;
  int nc;
  int at = wave_excl_small<(K < 2 ? 1 : K < 4 ? 2 : K < 8 ? 3 : K < 16 ? 4 : 6)>(mine, &nc);
#pragma unroll
  for (int i = 0; i < K; ++i)
    if (kk[i] >= tau) cand[at++] = kk[i];
  for (int c = nc + lane; c < ((nc + 15) & ~15); c += 64) cand[c] = 0;  // zero tail of the last chunk
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_s_waitcnt(0);
  for (int c = lane; c < nc; c += 64) {
    const unsigned long long k = cand[c];
    const int rk = count_greater(cand, nc, k);
    if (rk < kTop) out[rk] = k;
  }
  const int need = nc < kTop ? nc : kTop;
  if (lane >= need && lane < kTop) out[lane] = 0;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_s_waitcnt(0);
  return need;
}

// Writes the winners (sel, rank order) from one wave: features[r] = bucket,
// valid[r] = 1 for r < need; remaining slots id 0 / valid 0
// (route_parallel.cu:23,29); raw = sum of winner counts.
template <typename CountT>
__device__ void write_selection(const unsigned long long* sel, int need, const CountT* counts, int64_t* features,
                                float* valid, int* raw) {
  const int tid = threadIdx.x;
  if (tid < 64) {
    const bool hit = tid < need;
    const int b = hit ? key_bucket(sel[tid]) : 0;
    if (tid < kTop) {
      features[tid] = b;
      valid[tid] = hit ? 1.0f : 0.0f;
    }
    const int n = wave_sum_i(hit ? (int)counts[b] : 0);
    if (tid == 0) *raw = n;
  }
}

}  // namespace
}  // namespace prismkv
