// Moment scoring of one 32-bucket tile, shared by the route kernels and the
// fused decode kernel so that both produce bit-identical logits, chunk
// statistics and probability keys.
//
// Semantics: src/prismkv/core.py:119-128 (router="moments"): logit =
// (log(count) + (q @ mean^T) / sqrt(d)) + (q^2 @ var^T) / (2d) in this
// accumulation order, dead buckets -inf; per-head softmax exp(l - M) / Z and
// the sum over heads in head order.
//
// A tile is f32 [256 rows][32 buckets] (rows k < 128: mean dim k, k >= 128:
// variance dim k - 128).  256 threads score it: thread t = bucket quad
// (t & 7) x row phase (t >> 3) issues 8 independent 16-byte loads; the
// 2 parts x 4 heads x 4 buckets products are reduced across the 8 row lanes
// of a wave with a transpose-reduce and across the 4 waves in LDS, in a fixed
// order, so results are run-to-run identical.
#pragma once

#include "select.h"

namespace prismkv {
namespace {

constexpr float kSqrtD = 11.3137084989847604f;  // fp32(sqrt(128)), core.py:125

// Transpose-reduce step over lane bit M (32, 16 or 8): `x` holds 2N partial
// sums; lanes with the bit set keep the upper half, the others the lower
// half, and add the partner's copy of the kept half (own term first).  After
// the step x[0..N) holds the new partial sums.
template <int N, int M>
__device__ __forceinline__ void treduce(float* x) {
  if constexpr (M == 32 || M == 16) {
#pragma unroll
    for (int j = 0; j < N; ++j) x[j] = swap_add<M>(x[j], x[j + N]);
  } else {
    const unsigned long long hi = __ballot((threadIdx.x & M) != 0);
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const float keep = lane_select(hi, x[j + N], x[j]);
      const float send = lane_select(hi, x[j], x[j + N]);
      x[j] = keep + xor8(send);
    }
  }
}

// LDS of one 256-thread tile scorer.
struct TileLds {
  float4 red[4][64];            // cross-wave partials
  float dots[2][kHq][kChunk];   // [part][head][bucket]
};

// q (rows k < 128) and q*q (rows k >= 128) of group g, 4 heads per float4:
// thread t of nt stages entries t, t + nt, ... of the 512.
__device__ __forceinline__ void stage_query(const uint16_t* q, int g, float4* qq, int t, int nt) {
  for (int i = t; i < kHq * kD; i += nt) {
    const int h = i >> 7, k = i & (kD - 1);
    const float x = bf16_to_f32(q[((size_t)g * kHq + h) * kD + k]);
    reinterpret_cast<float*>(&qq[k])[h] = x;
    reinterpret_cast<float*>(&qq[kD + k])[h] = x * x;  // core.py:127 q.square() in fp32
  }
}
// The same for exactly 512 threads, split so the caller can issue the q load
// before its tile loads (its wait then leaves those in flight): the raw bf16
// bits are loaded first and converted only in store_query512.
__device__ __forceinline__ unsigned load_query512(const uint16_t* q, int g, int t) {
  return q[((size_t)g * kHq + (t >> 7)) * kD + (t & (kD - 1))];
}
__device__ __forceinline__ void store_query512(unsigned bits, float4* qq, int t) {
  const float x = __uint_as_float(bits << 16);
  const int h = t >> 7, k = t & (kD - 1);
  reinterpret_cast<float*>(&qq[k])[h] = x;
  reinterpret_cast<float*>(&qq[kD + k])[h] = x * x;  // core.py:127 q.square() in fp32
}

// The 16-byte loads of tile (g, c) for thread t (0..255); c must be a valid
// tile (no branch, so every load of the caller stays in flight together).
__device__ __forceinline__ void load_tile(const float* moments, int g, int c, int t, float4 (&m4)[8]) {
  const int quad = t & 7, r = t >> 3;
  const float4* tile = reinterpret_cast<const float4*>(moments + (size_t)(g * kChunks + c) * kRow * kChunk);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(tile + (r + 32 * i) * (kChunk / 4) + quad));
    m4[i] = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
  }
}

// Products and reductions of one tile; returns, in thread t < 128, the logit
// of head t >> 5 for bucket 32c + (t & 31) whose size is `n` (loaded by the
// caller with the tile, so no load waits here; -inf for a dead bucket).
// Every thread of the workgroup must call it (two barriers); t is the
// thread's index within its 256-thread scorer, whose 4 waves are consecutive.
__device__ __forceinline__ float tile_logit(const float4* qq, const float4 (&m4)[8], int t, TileLds& s, int n,
                                            bool has) {
  const int r = t >> 3, w = t >> 6, lane = t & 63;
  // acc[part*16 + head*4 + j]: part 0 = mean rows, 1 = variance rows
  float acc[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) acc[i] = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float4 qv = qq[r + 32 * i];
    const float* hq = reinterpret_cast<const float*>(&qv);
    const float* mv = reinterpret_cast<const float*>(&m4[i]);
    const int part = i >> 2;
#pragma unroll
    for (int h = 0; h < kHq; ++h)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[part * 16 + h * 4 + j] = fmaf(hq[h], mv[j], acc[part * 16 + h * 4 + j]);
  }
  // reduce over the 8 row lanes of the wave (lane bits 5,4,3)
  treduce<16, 32>(acc);
  treduce<8, 16>(acc);
  treduce<4, 8>(acc);
  // lane now holds part (lane>>5)&1, head (lane>>3)&3, buckets 4*quad .. +3
  s.red[w][lane] = make_float4(acc[0], acc[1], acc[2], acc[3]);
  __syncthreads();
  {
    const int l = t >> 2, j = t & 3;
    const float v = ((reinterpret_cast<const float*>(&s.red[0][l])[j] + reinterpret_cast<const float*>(&s.red[1][l])[j]) +
                     reinterpret_cast<const float*>(&s.red[2][l])[j]) +
                    reinterpret_cast<const float*>(&s.red[3][l])[j];
    s.dots[(l >> 5) & 1][(l >> 3) & 3][4 * (l & 7) + j] = v;
  }
  __syncthreads();
  float l = -INFINITY;
  if (t < kHq * kChunk && has) {
    const int h = t >> 5, b = t & 31;
    if (n > 0) {
      // core.py:122-127: log(count) + (q @ mean^T) / sqrt(d) + (q^2 @ var^T) / (2d)
      const float lc = logf((float)n);
      l = (lc + s.dots[0][h][b] / kSqrtD) + s.dots[1][h][b] / (2.0f * kD);
    }
  }
  return l;
}

// One tile scored by both halves of a 512-thread workgroup: half h takes
// part h (h = 0: mean rows 0..127, 1: variance rows 128..255) with 4 loads
// per thread.  Every dot product is the same tree of additions as in
// tile_logit (row lanes paired by lane bit 5, then 4, then 3; each pair sum
// is commutative; then the 4 waves in order), so the logits are bit-identical.
struct SplitLds {
  float2 red[2][4][64];
  float dots[2][kHq][kChunk];
};

__device__ __forceinline__ void load_half_tile(const float* moments, int g, int c, int part, int t, float4 (&m4)[4]) {
  const int quad = t & 7, r = t >> 3;
  const float4* tile = reinterpret_cast<const float4*>(moments + (size_t)(g * kChunks + c) * kRow * kChunk);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u32x4 v = __builtin_nontemporal_load(
        reinterpret_cast<const u32x4*>(tile + (r + 32 * i + 128 * part) * (kChunk / 4) + quad));
    m4[i] = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
  }
}

// Returns the logit in threads tid < 128 (head tid >> 5, bucket 32c + (tid & 31),
// size n); every thread of the 512 must call it (two barriers).
__device__ __forceinline__ float tile_logit_split(const float4* qq, const float4 (&m4)[4], int tid, SplitLds& s, int n,
                                                  bool has) {
  const int half = tid >> 8, t = tid & 255, r = t >> 3, w = t >> 6, lane = t & 63;
  float acc[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 qv = qq[r + 32 * i + 128 * half];
    const float* hq = reinterpret_cast<const float*>(&qv);
    const float* mv = reinterpret_cast<const float*>(&m4[i]);
#pragma unroll
    for (int h = 0; h < kHq; ++h)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[h * 4 + j] = fmaf(hq[h], mv[j], acc[h * 4 + j]);
  }
  // lane bit 5 -> head bit 1, bit 4 -> head bit 0, bit 3 -> bucket bit 1
  treduce<8, 32>(acc);
  treduce<4, 16>(acc);
  treduce<2, 8>(acc);
  s.red[half][w][lane] = make_float2(acc[0], acc[1]);
  __syncthreads();
  if (t < kHq * kChunk) {
    const int h = t >> 5, b = t & 31;
    const int L = ((h >> 1) << 5) | ((h & 1) << 4) | (((b & 3) >> 1) << 3) | (b >> 2);
    const bool hi = b & 1;
    const float v = (((hi ? s.red[half][0][L].y : s.red[half][0][L].x) + (hi ? s.red[half][1][L].y : s.red[half][1][L].x)) +
                     (hi ? s.red[half][2][L].y : s.red[half][2][L].x)) +
                    (hi ? s.red[half][3][L].y : s.red[half][3][L].x);
    s.dots[half][h][b] = v;
  }
  __syncthreads();
  float l = -INFINITY;
  if (tid < kHq * kChunk && has) {
    const int h = tid >> 5, b = tid & 31;
    if (n > 0) {
      // core.py:122-127: log(count) + (q @ mean^T) / sqrt(d) + (q^2 @ var^T) / (2d)
      const float lc = logf((float)n);
      l = (lc + s.dots[0][h][b] / kSqrtD) + s.dots[1][h][b] / (2.0f * kD);
    }
  }
  return l;
}

// (max, sum of exp(l - max)) over the 32 lanes of a head (lanes 0-31 or
// 32-63 of a wave, all active).
__device__ __forceinline__ float2 chunk_stats(float l) {
  float m = l;
  m = fmaxf(m, xor16(m));
  m = fmaxf(m, xor8(m));
  m = fmaxf(m, xor4(m));
  m = fmaxf(m, xor2(m));
  m = fmaxf(m, xor1(m));
  float e = (l == -INFINITY) ? 0.f : expf(l - m);
  e += xor16(e);
  e += xor8(e);
  e += xor4(e);
  e += xor2(e);
  e += xor1(e);
  return make_float2(m, e);
}

// Merge of the 94 chunk statistics of one head by one wave (lane i reads
// chunks i and i + 64 through `ld(chunk)`): M = max, Z = sum z_c e^{m_c - M};
// returns (M, 1/Z) in every lane (1/Z = 0 when Z = 0).
template <typename Load2>
__device__ __forceinline__ float2 merge_chunk_stats(Load2 ld) {
  const int lane = threadIdx.x & 63;
  const float2 s0 = lane < kChunks ? ld(lane) : make_float2(-INFINITY, 0.f);
  const float2 s1 = lane + 64 < kChunks ? ld(lane + 64) : make_float2(-INFINITY, 0.f);
  const float m = wave_max(fmaxf(s0.x, s1.x));
  float z = (s0.x == -INFINITY ? 0.f : s0.y * expf(s0.x - m)) + (s1.x == -INFINITY ? 0.f : s1.y * expf(s1.x - m));
  z = wave_sum(z);
  return make_float2(m, z > 0.f ? 1.0f / z : 0.f);
}

// Key of a live bucket: per-head softmax exp(l - M) / Z summed over heads in
// head order (core.py:128); equal logits give bit-equal keys, so exact ties
// fall to the lower bucket id.  0 for a dead bucket.
__device__ __forceinline__ uint64_t bucket_key(const float (&l)[kHq], const float* gmax, const float* grz, int bucket) {
  if (l[0] == -INFINITY) return 0;
  const float p0 = expf(l[0] - gmax[0]) * grz[0];
  const float p1 = expf(l[1] - gmax[1]) * grz[1];
  const float p2 = expf(l[2] - gmax[2]) * grz[2];
  const float p3 = expf(l[3] - gmax[3]) * grz[3];
  return make_key(((p0 + p1) + p2) + p3, bucket);
}

}  // namespace
}  // namespace prismkv
