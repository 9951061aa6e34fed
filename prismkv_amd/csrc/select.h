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

// ---------------------------------------------------------------------------
// Register-resident Top-16 by bitonic networks.  A wave holds 64 keys per
// "set" (one per lane); rows are the four 16-lane groups.  Exchanges within a
// row go through DPP (a few cycles), across rows through a lane permute, so
// a Top-16 of 64 keys is ~20 dependent compare-exchange steps and touches
// no LDS.  Keys are unique except 0 (empty), which sorts last.
// ---------------------------------------------------------------------------
template <int kCtrl>
__device__ __forceinline__ unsigned long long dpp_u64(unsigned long long v) {
  const int lo = __builtin_amdgcn_mov_dpp((int)(unsigned)v, kCtrl, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_mov_dpp((int)(unsigned)(v >> 32), kCtrl, 0xF, 0xF, false);
  return ((unsigned long long)(unsigned)hi << 32) | (unsigned long long)(unsigned)lo;
}
// The key held by lane `src` (uniform), in every lane.
__device__ __forceinline__ unsigned long long readlane_u64(unsigned long long v, int src) {
  const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(v >> 32), src);
  const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)v, src);
  return ((unsigned long long)hi << 32) | (unsigned long long)lo;
}
// The key of lane (lane ^ M) for M = 16 or 32 (permlane swaps, no LDS).
template <int M>
__device__ __forceinline__ unsigned long long xor_rows_u64(unsigned long long v) {
  const unsigned lo = M == 32 ? xor32_u((unsigned)v) : xor16_u((unsigned)v);
  const unsigned hi = M == 32 ? xor32_u((unsigned)(v >> 32)) : xor16_u((unsigned)(v >> 32));
  return ((unsigned long long)hi << 32) | (unsigned long long)lo;
}
// The key of lane (lane ^ D) for D in {1, 2, 4, 8} (within the row).
template <int D>
__device__ __forceinline__ unsigned long long xor_lane_u64(unsigned long long v) {
  if constexpr (D == 1) return dpp_u64<0xB1>(v);   // quad_perm [1,0,3,2]
  if constexpr (D == 2) return dpp_u64<0x4E>(v);   // quad_perm [2,3,0,1]
  if constexpr (D == 8) return dpp_u64<0x128>(v);  // row_ror:8
  if constexpr (D == 4) {
    const unsigned long long up = dpp_u64<0x104>(v);    // row_shl:4: lane i reads lane i + 4
    const unsigned long long down = dpp_u64<0x114>(v);  // row_shr:4: lane i reads lane i - 4
    return (threadIdx.x & 4) ? down : up;
  }
  return v;
}
// Compare-exchange with lane ^ D: keep the larger key where keep_max, else the smaller.
template <int D>
__device__ __forceinline__ unsigned long long cx_u64(unsigned long long v, bool keep_max) {
  const unsigned long long o = xor_lane_u64<D>(v);
  return ((v > o) == keep_max) ? v : o;
}
// Bitonic sequence in each row -> descending row (lane 16r + j holds rank j).
__device__ __forceinline__ unsigned long long row_merge_desc(unsigned long long v) {
  const int i = threadIdx.x & 15;
  v = cx_u64<8>(v, (i & 8) == 0);
  v = cx_u64<4>(v, (i & 4) == 0);
  v = cx_u64<2>(v, (i & 2) == 0);
  return cx_u64<1>(v, (i & 1) == 0);
}
// Any keys -> each row sorted descending.
__device__ __forceinline__ unsigned long long row_sort_desc(unsigned long long v) {
  const int i = threadIdx.x & 15;
  v = cx_u64<1>(v, ((i & 1) == 0) == ((i & 2) == 0));
  v = cx_u64<2>(v, ((i & 2) == 0) == ((i & 4) == 0));
  v = cx_u64<1>(v, ((i & 1) == 0) == ((i & 4) == 0));
  v = cx_u64<4>(v, ((i & 4) == 0) == ((i & 8) == 0));
  v = cx_u64<2>(v, ((i & 2) == 0) == ((i & 8) == 0));
  v = cx_u64<1>(v, ((i & 1) == 0) == ((i & 8) == 0));
  return row_merge_desc(v);
}
// Two descending 16-lists a, b (same lanes) -> the descending top 16 of both.
__device__ __forceinline__ unsigned long long merge_top16(unsigned long long a, unsigned long long b) {
  const unsigned long long r = dpp_u64<0x140>(b);  // row_mirror: b ascending along the row
  return row_merge_desc(a > r ? a : r);
}
// Rows sorted descending -> every row holds the descending top 16 of the wave.
__device__ __forceinline__ unsigned long long rows_top16(unsigned long long v) {
  v = merge_top16(v, xor_rows_u64<16>(v));
  return merge_top16(v, xor_rows_u64<32>(v));
}
// Top-16 of K sets of 64 keys whose rows are already sorted descending:
// lane j < 16 of every row ends with the rank-j key (0 if fewer keys).
template <int K>
__device__ __forceinline__ unsigned long long sorted_rows_top16(unsigned long long (&v)[K]) {
#pragma unroll
  for (int k = 0; k < K; ++k) v[k] = rows_top16(v[k]);
#pragma unroll
  for (int w = 1; w < K; w *= 2)
#pragma unroll
    for (int k = 0; k + w < K; k += 2 * w) v[k] = merge_top16(v[k], v[k + w]);
  return v[0];
}
// Top-16 of K sets of 64 arbitrary keys.
template <int K>
__device__ __forceinline__ unsigned long long bitonic_top16(unsigned long long (&v)[K]) {
#pragma unroll
  for (int k = 0; k < K; ++k) v[k] = row_sort_desc(v[k]);
  return sorted_rows_top16<K>(v);
}

// Full descending sort of one wave's 64 keys (lane r ends with rank r):
// the bitonic network over the lane index, exchanges with lane ^ j through
// DPP (j < 16) or a lane permute (j = 16, 32).
template <int J>
__device__ __forceinline__ unsigned long long xor_any_u64(unsigned long long v) {
  if constexpr (J >= 16) return xor_rows_u64<J>(v);
  else return xor_lane_u64<J>(v);
}
template <int K, int J>
__device__ __forceinline__ unsigned long long sort_step(unsigned long long v) {
  const int lane = threadIdx.x & 63;
  const bool keep_max = ((lane & K) == 0) == ((lane & J) == 0);  // descending blocks of K
  const unsigned long long o = xor_any_u64<J>(v);
  return ((v > o) == keep_max) ? v : o;
}
template <int K>
__device__ __forceinline__ unsigned long long sort_merge(unsigned long long v) {
  if constexpr (K >= 64) v = sort_step<K, 32>(v);
  if constexpr (K >= 32) v = sort_step<K, 16>(v);
  if constexpr (K >= 16) v = sort_step<K, 8>(v);
  if constexpr (K >= 8) v = sort_step<K, 4>(v);
  if constexpr (K >= 4) v = sort_step<K, 2>(v);
  return sort_step<K, 1>(v);
}
__device__ __forceinline__ unsigned long long wave_sort_desc(unsigned long long v) {
  v = sort_merge<2>(v);
  v = sort_merge<4>(v);
  v = sort_merge<8>(v);
  v = sort_merge<16>(v);
  v = sort_merge<32>(v);
  return sort_merge<64>(v);
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
    const int b = hit ? min(key_bucket(sel[tid]), kF - 1) : 0;  // in range even for a key read after a give-up
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
