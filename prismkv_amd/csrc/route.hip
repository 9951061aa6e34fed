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

template <typename QT>
__global__ __launch_bounds__(kRT) void route_score_kernel(const QT* __restrict__ q,
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
// Route by query activations (router "q_activation", core.py:131-139):
//   a = relu((q / query_scale) W^T + b), the SAE encode of the 4 queries;
//   per head the 16 largest activations (value descending, bucket ascending:
//   the stable descending argsort), weights val / max(sum val, 1e-20) / 4
//   with the sum taken in rank order; score[bucket] = the weights of the
//   bucket summed in head order (scatter_add over the flattened [4][16]
//   lists); the order = buckets of positive score and nonzero size, by score
//   descending and bucket ascending -- up to 64.
// qact_part_kernel: grid (12, G) x 256: workgroup j encodes buckets
//   [256 j, 256 j + 256) for the 4 heads (thread = bucket, fp32 dot products
//   in dim order) and keeps each head's 16 best keys;
// qact_final_kernel: grid G x 256: wave h ranks head h's 12 x 16 candidates;
//   wave 0 forms the weights and scores, keeps the first entry of each bucket,
//   sorts and writes the selection (features / valid [G][64], raw) and the
//   score vector.
// ---------------------------------------------------------------------------
constexpr int kQaParts = (kF + kRT - 1) / kRT;  // 12
constexpr int kQaSel = kHq * kTop;               // 64

template <typename QT>
__global__ __launch_bounds__(kRT) void qact_part_kernel(const QT* __restrict__ q, const float* __restrict__ W,
                                                        const float* __restrict__ b, const float* __restrict__ qscale,
                                                        unsigned long long* __restrict__ cand) {
  const int j = blockIdx.x, g = blockIdx.y, tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  __shared__ float xs[kHq][kD];
  __shared__ __align__(16) unsigned long long keys[kHq][kRT];
  const float qs = qscale[g];
  for (int i = tid; i < kHq * kD; i += kRT) xs[i / kD][i % kD] = to_f32(q[(size_t)g * kHq * kD + i]) / qs;
  __syncthreads();
  const int f = j * kRT + tid;
  float acc[kHq] = {0.f, 0.f, 0.f, 0.f};
  if (f < kF) {
    const float4* wr = reinterpret_cast<const float4*>(W + ((size_t)g * kF + f) * kD);
#pragma unroll 8
    for (int d4 = 0; d4 < kD / 4; ++d4) {
      const float4 wv = wr[d4];
#pragma unroll
      for (int h = 0; h < kHq; ++h) {
        acc[h] = fmaf(xs[h][4 * d4], wv.x, acc[h]);
        acc[h] = fmaf(xs[h][4 * d4 + 1], wv.y, acc[h]);
        acc[h] = fmaf(xs[h][4 * d4 + 2], wv.z, acc[h]);
        acc[h] = fmaf(xs[h][4 * d4 + 3], wv.w, acc[h]);
      }
    }
  }
  const float bias = f < kF ? b[(size_t)g * kF + f] : 0.f;
#pragma unroll
  for (int h = 0; h < kHq; ++h) {
    const float x = acc[h] + bias;
    keys[h][tid] = f < kF ? make_key(x > 0.f ? x : 0.f, f) : 0ull;  // relu; slots past F stay empty
  }
  __syncthreads();
  if (w < kHq) {
    unsigned long long v[kRT / 64];
#pragma unroll
    for (int k = 0; k < kRT / 64; ++k) v[k] = keys[w][64 * k + lane];
    const unsigned long long best = bitonic_top16<kRT / 64>(v);
    if (lane < kTop) cand[(((size_t)g * kHq + w) * kQaParts + j) * kTop + lane] = best;
  }
}

__global__ __launch_bounds__(kRT) void qact_final_kernel(const unsigned long long* __restrict__ cand,
                                                         const int* __restrict__ counts, int64_t* __restrict__ features,
                                                         float* __restrict__ valid, int* __restrict__ raw,
                                                         float* __restrict__ scores) {
  const int g = blockIdx.x, tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  __shared__ __align__(16) unsigned long long top[kHq][kTop];
  __shared__ float sc_lds[kFP];
  __shared__ int ent_b[kQaSel];
  __shared__ float ent_c[kQaSel];
  for (int i = tid; i < kFP; i += kRT) sc_lds[i] = 0.f;
  static_assert(kQaParts * kTop == 3 * 64, "three 64-key sets per head");
  if (w < kHq) {
    unsigned long long v[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) v[k] = cand[((size_t)g * kHq + w) * kQaParts * kTop + 64 * k + lane];
    const unsigned long long best = sorted_rows_top16<3>(v);  // each 16-lane row is one part's ranked list
    if (lane < kTop) top[w][lane] = best;
  }
  __syncthreads();
  if (w == 0) {
    // entry e = 16 h + r: head h's rank-r activation (the flattened order of core.py:136-137)
    const int h = lane >> 4, r = lane & 15;
    const unsigned long long key = top[h][r];  // never 0: every part holds at least 16 real buckets
    const float val = __uint_as_float((unsigned)(key >> 12));
    const int bucket = key ? key_bucket(key) : 0;
    float s = 0.f;
#pragma unroll
    for (int rr = 0; rr < kTop; ++rr) s += __uint_as_float((unsigned)(top[h][rr] >> 12));
    s = fmaxf(s, 1e-20f);
    const float c = (val / s) / (float)kHq;
    ent_b[lane] = bucket;
    ent_c[lane] = c;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_s_waitcnt(0);
    // the bucket's score: its entries' weights added in entry order, from 0
    float sc = 0.f;
    bool first = true;
    for (int e = 0; e < kQaSel; ++e)
      if (ent_b[e] == bucket) {
        sc += ent_c[e];
        first = first && e >= lane;
      }
    if (first) sc_lds[bucket] = sc;
    const bool keep = first && sc > 0.f && counts[(size_t)g * kFP + bucket] > 0;
    const unsigned long long k2 = wave_sort_desc(keep ? make_key(sc, bucket) : 0ull);
    const int n = __popcll(__ballot(k2 != 0));
    const int fb = k2 ? key_bucket(k2) : 0;
    features[(size_t)g * kQaSel + lane] = lane < n ? fb : 0;
    valid[(size_t)g * kQaSel + lane] = lane < n ? 1.f : 0.f;
    const int rs = wave_sum_i(lane < n ? counts[(size_t)g * kFP + fb] : 0);
    if (lane == 0) raw[g] = rs;
  }
  __syncthreads();
  if (scores)
    for (int i = tid; i < kF; i += kRT) scores[(size_t)g * kF + i] = sc_lds[i];
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

template <typename QT>
static void launch_route_score(const QT* q, const float* moments, const int* counts, float* logits, float* stats,
                               int groups, hipStream_t stream) {
  hipLaunchKernelGGL(route_score_kernel<QT>, dim3(kChunks, groups), dim3(kRT), 0, stream, q, moments, counts,
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

}  // extern "C"

template <typename QT>
static int route_impl(uint64_t q, uint64_t moments, uint64_t counts, uint64_t work, uint64_t features,
                      uint64_t valid, uint64_t raw, float* scores, int groups, size_t work_bytes, uint64_t stream) {
  if (groups < 1 || groups > 65535) return kBadSize;
  if (!q || !moments || !counts || !work || !features || !valid || !raw) return kBadSize;
  if (work_bytes < prismkv_route_work_bytes(groups)) return kBadSize;
  char* base = reinterpret_cast<char*>(work);
  RouteWork rw{reinterpret_cast<float*>(base), reinterpret_cast<float*>(base + route_logits_bytes(groups))};
  hipStream_t s = (hipStream_t)stream;
  launch_route_score(reinterpret_cast<const QT*>(q), reinterpret_cast<const float*>(moments),
                     reinterpret_cast<const int*>(counts), rw.logits, rw.stats, groups, s);
  unsigned long long* cand =
      reinterpret_cast<unsigned long long*>(base + route_logits_bytes(groups) + route_stats_bytes(groups));
  hipLaunchKernelGGL(route_part_kernel, dim3(kParts, groups), dim3(kRT), 0, s, rw, cand, scores);
  hipLaunchKernelGGL(route_final_kernel, dim3(groups), dim3(64), 0, s, cand, reinterpret_cast<const int*>(counts),
                     reinterpret_cast<int64_t*>(features), reinterpret_cast<float*>(valid),
                     reinterpret_cast<int*>(raw));
  return (int)hipGetLastError();
}

extern "C" {

int prismkv_route(uint64_t q, uint64_t moments, uint64_t counts, uint64_t work, uint64_t features, uint64_t valid,
                  uint64_t raw, int groups, size_t work_bytes, uint64_t stream) {
  return route_impl<uint16_t>(q, moments, counts, work, features, valid, raw, nullptr, groups, work_bytes, stream);
}

int prismkv_route_scores(uint64_t q, uint64_t moments, uint64_t counts, uint64_t work, uint64_t features,
                         uint64_t valid, uint64_t raw, uint64_t scores, int groups, size_t work_bytes,
                         uint64_t stream) {
  if (!scores) return kBadSize;
  return route_impl<uint16_t>(q, moments, counts, work, features, valid, raw, reinterpret_cast<float*>(scores),
                              groups, work_bytes, stream);
}

int prismkv_route_scores_f32(uint64_t q, uint64_t moments, uint64_t counts, uint64_t work, uint64_t features,
                             uint64_t valid, uint64_t raw, uint64_t scores, int groups, size_t work_bytes,
                             uint64_t stream) {
  if (!scores) return kBadSize;
  return route_impl<float>(q, moments, counts, work, features, valid, raw, reinterpret_cast<float*>(scores), groups,
                           work_bytes, stream);
}

size_t prismkv_route_qact_work_bytes(int groups) {
  if (groups < 1 || groups > 65535) return 0;
  return (size_t)groups * kHq * kQaParts * kTop * sizeof(unsigned long long);
}

}  // extern "C"

template <typename QT>
static int route_qact_impl(uint64_t q, uint64_t W, uint64_t b, uint64_t qscale, uint64_t counts, uint64_t work,
                           uint64_t features, uint64_t valid, uint64_t raw, uint64_t scores, int groups,
                           size_t work_bytes, uint64_t stream) {
  if (groups < 1 || groups > 65535) return kBadSize;
  if (!q || !W || !b || !qscale || !counts || !work || !features || !valid || !raw || (W & 15u)) return kBadSize;
  if (work_bytes < prismkv_route_qact_work_bytes(groups)) return kBadSize;
  hipStream_t s = (hipStream_t)stream;
  unsigned long long* cand = reinterpret_cast<unsigned long long*>(work);
  hipLaunchKernelGGL(qact_part_kernel<QT>, dim3(kQaParts, groups), dim3(kRT), 0, s, reinterpret_cast<const QT*>(q),
                     reinterpret_cast<const float*>(W), reinterpret_cast<const float*>(b),
                     reinterpret_cast<const float*>(qscale), cand);
  hipLaunchKernelGGL(qact_final_kernel, dim3(groups), dim3(kRT), 0, s, cand, reinterpret_cast<const int*>(counts),
                     reinterpret_cast<int64_t*>(features), reinterpret_cast<float*>(valid),
                     reinterpret_cast<int*>(raw), reinterpret_cast<float*>(scores));
  return (int)hipGetLastError();
}

extern "C" {

int prismkv_route_qact(uint64_t q, uint64_t W, uint64_t b, uint64_t qscale, uint64_t counts, uint64_t work,
                       uint64_t features, uint64_t valid, uint64_t raw, uint64_t scores, int groups, size_t work_bytes,
                       uint64_t stream) {
  return route_qact_impl<uint16_t>(q, W, b, qscale, counts, work, features, valid, raw, scores, groups, work_bytes,
                                   stream);
}

int prismkv_route_qact_f32(uint64_t q, uint64_t W, uint64_t b, uint64_t qscale, uint64_t counts, uint64_t work,
                           uint64_t features, uint64_t valid, uint64_t raw, uint64_t scores, int groups,
                           size_t work_bytes, uint64_t stream) {
  return route_qact_impl<float>(q, W, b, qscale, counts, work, features, valid, raw, scores, groups, work_bytes,
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
