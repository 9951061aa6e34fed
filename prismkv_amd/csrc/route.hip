// Stage 1 -- route: score the F=3000 buckets of each KV group from stored
// count / mean / diagonal-variance moments against the 4 query heads, softmax
// per head, average over heads, select the Top-16 live buckets.
//
// Semantics: src/prismkv/core.py:106-130 (router="moments"),
//            kernels/ppu_8b/route_parallel.cu:12-32 (tie rule, padding, raw).
//
// Design (two launches per layer, no vendor GEMM):
//   * Moment tables live in HBM as 32-bucket tiles [g][chunk][k][32] (k < 128:
//     mean, k >= 128: variance; 128-byte tile rows).  Scoring workgroup
//     (chunk, g) streams its 32 KB tile with eight independent 16-byte loads
//     per thread (thread = 4 buckets x 8 k-rows), so ~750 workgroups keep the
//     whole 24.6 MB table in flight at once.  The per-thread products for
//     2 parts x 4 heads x 4 buckets are reduced across the 8 k-row lanes of a
//     wave with a transpose-reduce (28 shuffles) and across the 4 waves in
//     LDS, in a fixed order, so results are run-to-run identical.
//   * Logit = (log(count) + mean_term / sqrt(d)) + var_term / (2d): the
//     accumulation order of core.py:122-127.  Each scoring workgroup stores
//     its 4x32 logits and per-head (max, sum-exp) chunk statistics with
//     plain stores and exits: the kernel boundary is the only inter-workgroup
//     synchronisation (a per-group arrival counter would serialise 94
//     device-scope atomics on one address).
//   * The part kernel (8 workgroups per group, 376 buckets each) merges the
//     94 chunk statistics, forms the head-summed probabilities exp(l - M) / Z
//     -- equal logits give bit-equal probabilities, so exact ties fall to the
//     lower bucket id as in the reference -- and keeps its 16 best 44-bit
//     keys (probability bits << 12 | 4095 - bucket: value descending, bucket
//     id ascending on ties); the final kernel ranks the 128 candidates of a
//     group.  Each select ranks per-thread maxima with LDS broadcast reads to
//     find a threshold, then ranks the few keys above it (no histogram
//     atomics, no sorting network).
#include "score.h"

namespace prismkv {
namespace {

constexpr int kRT = 256;                      // route workgroup size
constexpr int kKeys = (kFP + kRT - 1) / kRT;  // 12 candidate keys per thread

// ---------------------------------------------------------------------------
// Route, pass 1 (moment scoring): grid (kChunks, G) x 256.
// ---------------------------------------------------------------------------
struct RouteWork {
  float* logits;  // [G][4][kFP]
  float* stats;   // [G][kChunks][4][2] (chunk max, chunk sum of exp)
};

__global__ __launch_bounds__(kRT) void route_score_kernel(const uint16_t* __restrict__ q,
                                                          const float* __restrict__ moments,
                                                          const int* __restrict__ counts, RouteWork work) {
  const int c = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
  __shared__ float4 qq[kRow];  // [k] -> 4 heads; k < 128: q, k >= 128: q*q
  __shared__ TileLds lds;
  float4 m4[8];
  load_tile(moments, g, c, tid, m4);  // 16-byte tile loads first
  const int n = tid < kHq * kChunk ? counts[(size_t)g * kFP + c * kChunk + (tid & 31)] : 0;
  stage_query(q, g, qq, tid, kRT);
  __syncthreads();
  const float l = tile_logit(qq, m4, tid, lds, n, true);
  if (tid < kHq * kChunk) {
    // thread = (head tid>>5, bucket tid&31); 32 lanes per head
    const int h = tid >> 5, b = tid & 31;
    work.logits[((size_t)g * kHq + h) * kFP + c * kChunk + b] = l;
    const float2 st = chunk_stats(l);
    if (b == 0) *reinterpret_cast<float2*>(&work.stats[(((size_t)g * kChunks + c) * kHq + h) * 2]) = st;
  }
}

// ---------------------------------------------------------------------------
// Route, pass 2 (normalise, aggregate, local Top-16): grid (kParts, G) x 256.
// Part j of group g turns the logits of buckets [j*kPartB, (j+1)*kPartB)
// into probabilities exp(l - M) / Z -- bit-equal for equal logits, so exact
// ties fall to the lower bucket id as in the reference -- and keeps its 16
// best keys; the union of the parts' bests holds the group's Top-16.
// ---------------------------------------------------------------------------
constexpr int kParts = 8;
constexpr int kPartB = kFP / kParts;  // 376 buckets per part
constexpr int kPartKeys = (kPartB + kRT - 1) / kRT;  // 2

__global__ __launch_bounds__(kRT) void route_part_kernel(RouteWork work, unsigned long long* __restrict__ cand,
                                                         float* __restrict__ scores) {
  const int part = blockIdx.x, g = blockIdx.y, tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  __shared__ float gmax[kHq], grz[kHq];
  __shared__ __align__(16) unsigned long long keys[kPartKeys * kRT];
  __shared__ __align__(16) unsigned long long scratch[64 + 16 * kPartKeys * 4 + 2];
  // every load of the workgroup is issued before any is used
  const float* lg = work.logits + (size_t)g * kHq * kFP;
  float lv[kPartKeys][kHq];
#pragma unroll
  for (int i = 0; i < kPartKeys; ++i) {
    const int b = part * kPartB + min(tid + i * kRT, kPartB - 1);
#pragma unroll
    for (int h = 0; h < kHq; ++h) lv[i][h] = lg[h * kFP + b];
  }
  {
    // merge chunk statistics: wave h handles head h, lanes cover the 94 chunks
    const int h = w;
    const float2* st = reinterpret_cast<const float2*>(work.stats) + (size_t)g * kChunks * kHq + h;
    const float2 mz = merge_chunk_stats([&](int ch) { return st[ch * kHq]; });
    if (lane == 0) {
      gmax[h] = mz.x;
      grz[h] = mz.y;
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kPartKeys; ++i) {
    const int off = tid + i * kRT, b = part * kPartB + off;
    const uint64_t key = off < kPartB ? bucket_key(lv[i], gmax, grz, b) : 0;
    keys[off] = key;
    // optional: the head-mean score of core.py:128 (the key's probability sum / 4)
    if (scores && off < kPartB && b < kF) scores[(size_t)g * kF + b] = __uint_as_float((unsigned)(key >> 12)) * 0.25f;
  }
  __syncthreads();
  // wave w keeps the 16 best of keys[128w, 128w + 128); wave 0 then the 16 best of those 64
  __shared__ __align__(16) unsigned long long best[4 * kTop];
  __shared__ __align__(16) unsigned long long sc[4][64 + 2 * 16 + 2];
  wave_top16<2>(keys + 128 * w, sc[w], best + kTop * w);
  __syncthreads();
  if (w == 0) {
    __shared__ __align__(16) unsigned long long win[kTop];
    wave_top16<1>(best, scratch, win);
    if (lane < kTop) cand[((size_t)g * kParts + part) * kTop + lane] = win[lane];
  }
}

// ---------------------------------------------------------------------------
// Route, pass 3: the Top-16 of the kParts x 16 candidates of each group.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void route_final_kernel(const unsigned long long* __restrict__ cand,
                                                         const int* __restrict__ counts,
                                                         int64_t* __restrict__ features, float* __restrict__ valid,
                                                         int* __restrict__ raw) {
  const int g = blockIdx.x, lane = threadIdx.x;
  __shared__ __align__(16) unsigned long long keys[kParts * kTop];
  __shared__ __align__(16) unsigned long long scratch[64 + 2 * 16 + 2];
  __shared__ __align__(16) unsigned long long win[kTop];
  static_assert(kParts * kTop == 128, "two candidates per lane");
  keys[lane] = cand[(size_t)g * kParts * kTop + lane];
  keys[lane + 64] = cand[(size_t)g * kParts * kTop + lane + 64];
  __syncthreads();
  const int need = wave_top16<2>(keys, scratch, win);
  write_selection(win, need, counts + (size_t)g * kFP, features + (size_t)g * kTop, valid + (size_t)g * kTop,
                  raw + g);
}

// ---------------------------------------------------------------------------
// Compat: fused_norm_top (kernels/ppu_8b/route_parallel.cu:13-35).
// prod f32 [8][4][3000], ln f32 [8][3000], ct i32 [8][3000] -> ids i64 [8][16],
// vals f32 [8][16], raw i32 [8].  One workgroup per group.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kRT) void norm_top_kernel(const float* __restrict__ prod, const float* __restrict__ ln,
                                                       const int* __restrict__ ct, int64_t* __restrict__ ids,
                                                       float* __restrict__ vals, int* __restrict__ raw) {
  const int g = blockIdx.x, tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  __shared__ float red[kHq][4];
  __shared__ float hmax[kHq], hsum[kHq];
  __shared__ __align__(16) unsigned long long keys[kKeys * kRT];
  __shared__ __align__(16) unsigned long long sc[kRT / 64][64 + 16 * kKeys];
  __shared__ __align__(16) unsigned long long best[kRT / 64 * kTop], win[kTop];
  const int* cg = ct + (size_t)g * kF;
  const float* lng = ln + (size_t)g * kF;
  float lv[kHq][kKeys];
#pragma unroll
  for (int h = 0; h < kHq; ++h) {
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < kKeys; ++i) {
      const int b = tid + i * kRT;
      float l = -INFINITY;
      if (b < kF && cg[b] > 0) l = prod[((size_t)g * kHq + h) * kF + b] + lng[b];
      lv[h][i] = l;
      m = fmaxf(m, l);
    }
    m = wave_max(m);
    if (lane == 0) red[h][w] = m;
  }
  __syncthreads();
  if (tid < kHq) hmax[tid] = fmaxf(fmaxf(red[tid][0], red[tid][1]), fmaxf(red[tid][2], red[tid][3]));
  __syncthreads();
#pragma unroll
  for (int h = 0; h < kHq; ++h) {
    const float m = hmax[h];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kKeys; ++i) {
      const float e = (m == -INFINITY || lv[h][i] == -INFINITY) ? 0.f : expf(lv[h][i] - m);
      lv[h][i] = e;
      s += e;
    }
    s = wave_sum(s);
    if (lane == 0) red[h][w] = s;
  }
  __syncthreads();
  if (tid < kHq) hsum[tid] = (red[tid][0] + red[tid][1]) + (red[tid][2] + red[tid][3]);
  __syncthreads();
  // keys laid out so that wave w's 768 keys are contiguous: slot i of thread t at 768 w + 64 i + lane
#pragma unroll
  for (int i = 0; i < kKeys; ++i) {
    const int b = tid + i * kRT;
    uint64_t key = 0;
    if (b < kF && cg[b] > 0) {
      float a = 0.f;
#pragma unroll
      for (int h = 0; h < kHq; ++h) a += hsum[h] > 0.f ? lv[h][i] / hsum[h] : 0.f;
      key = make_key(a, b);
    }
    keys[w * 64 * kKeys + 64 * i + lane] = key;
  }
  __syncthreads();
  wave_top16<kKeys>(keys + w * 64 * kKeys, sc[w], best + kTop * w);
  __syncthreads();
  if (w == 0) {
    const int need = wave_top16<1>(best, sc[0], win);
    write_selection(win, need, cg, ids + (size_t)g * kTop, vals + (size_t)g * kTop, raw + g);
  }
}

// Compat: pack (kernels/ppu_8b/pack.cu:3-4): bf16 q[32][128] -> a[32][256] = [q, q*q].
__global__ void pack_kernel(const uint16_t* __restrict__ q, float* __restrict__ a) {
  const int r = blockIdx.x, d = threadIdx.x;
  const float v = bf16_to_f32(q[r * kD + d]);
  a[r * kRow + d] = v;
  a[r * kRow + kD + d] = v * v;
}

}  // namespace
}  // namespace prismkv

using namespace prismkv;

static void launch_route_score(const uint16_t* q, const float* moments, const int* counts, float* logits,
                               float* stats, int groups, hipStream_t stream) {
  hipLaunchKernelGGL(route_score_kernel, dim3(kChunks, groups), dim3(kRT), 0, stream, q, moments, counts,
                     RouteWork{logits, stats});
}

static size_t route_logits_bytes(int groups) { return (size_t)groups * kHq * kFP * sizeof(float); }
static size_t route_stats_bytes(int groups) { return (size_t)groups * kChunks * kHq * 2 * sizeof(float); }

extern "C" {

static size_t route_cand_bytes(int groups) { return (size_t)groups * kParts * kTop * sizeof(unsigned long long); }

size_t prismkv_route_work_bytes(int groups) {
  if (groups < 1) return 0;
  return route_logits_bytes(groups) + route_stats_bytes(groups) + route_cand_bytes(groups);
}

static int route_impl(uint64_t q, uint64_t moments, uint64_t counts, uint64_t work, uint64_t features,
                      uint64_t valid, uint64_t raw, float* scores, int groups, uint64_t stream) {
  if (groups < 1 || groups > 65535) return kBadSize;
  if (!q || !moments || !counts || !work || !features || !valid || !raw) return kBadSize;
  char* base = reinterpret_cast<char*>(work);
  RouteWork rw{reinterpret_cast<float*>(base), reinterpret_cast<float*>(base + route_logits_bytes(groups))};
  hipStream_t s = (hipStream_t)stream;
  launch_route_score(reinterpret_cast<const uint16_t*>(q), reinterpret_cast<const float*>(moments),
                     reinterpret_cast<const int*>(counts), rw.logits, rw.stats, groups, s);
  unsigned long long* cand =
      reinterpret_cast<unsigned long long*>(base + route_logits_bytes(groups) + route_stats_bytes(groups));
  hipLaunchKernelGGL(route_part_kernel, dim3(kParts, groups), dim3(kRT), 0, s, rw, cand, scores);
  hipLaunchKernelGGL(route_final_kernel, dim3(groups), dim3(64), 0, s, cand, reinterpret_cast<const int*>(counts),
                     reinterpret_cast<int64_t*>(features), reinterpret_cast<float*>(valid),
                     reinterpret_cast<int*>(raw));
  return (int)hipGetLastError();
}

int prismkv_route(uint64_t q, uint64_t moments, uint64_t counts, uint64_t work, uint64_t features, uint64_t valid,
                  uint64_t raw, int groups, uint64_t stream) {
  return route_impl(q, moments, counts, work, features, valid, raw, nullptr, groups, stream);
}

int prismkv_route_scores(uint64_t q, uint64_t moments, uint64_t counts, uint64_t work, uint64_t features,
                         uint64_t valid, uint64_t raw, uint64_t scores, int groups, uint64_t stream) {
  if (!scores) return kBadSize;
  return route_impl(q, moments, counts, work, features, valid, raw, reinterpret_cast<float*>(scores), groups,
                    stream);
}

int pack(uint64_t q, uint64_t a, uint64_t stream) {
  hipLaunchKernelGGL(pack_kernel, dim3(32), dim3(kD), 0, (hipStream_t)stream, reinterpret_cast<const uint16_t*>(q),
                     reinterpret_cast<float*>(a));
  return (int)hipGetLastError();
}

int fused_norm_top(uint64_t prod, uint64_t ln, uint64_t ct, uint64_t ids, uint64_t vals, uint64_t raw,
                   uint64_t stream) {
  hipLaunchKernelGGL(norm_top_kernel, dim3(8), dim3(kRT), 0, (hipStream_t)stream,
                     reinterpret_cast<const float*>(prod), reinterpret_cast<const float*>(ln),
                     reinterpret_cast<const int*>(ct), reinterpret_cast<int64_t*>(ids), reinterpret_cast<float*>(vals),
                     reinterpret_cast<int*>(raw));
  return (int)hipGetLastError();
}

}  // extern "C"
