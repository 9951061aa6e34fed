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
#include "launch.h"
#include "select.h"

namespace prismkv {
namespace {

constexpr int kRT = 256;                      // route workgroup size
constexpr int kKeys = (kFP + kRT - 1) / kRT;  // 12 candidate keys per thread
constexpr float kSqrtD = 11.3137084989847604f;  // fp32(sqrt(128)), core.py:125

// Transpose-reduce step: `x` holds 2n partial sums; lanes whose `mask` bit is
// set keep the upper half, the others the lower half, and add the partner's
// copy of the kept half.  After the step x[0..n) holds the new partial sums.
template <int N>
__device__ __forceinline__ void treduce(float* x, int mask) {
  const unsigned long long hi = __ballot((threadIdx.x & mask) != 0);
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const float keep = lane_select(hi, x[j + N], x[j]);
    const float send = lane_select(hi, x[j], x[j + N]);
    x[j] = keep + __shfl_xor(send, mask);
  }
}

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
  const int w = tid >> 6, lane = tid & 63;
  __shared__ float4 qq[kRow];                 // [k] -> 4 heads; k < 128: q, k >= 128: q*q
  __shared__ float4 red[kRT / 64][64];        // cross-wave partials
  __shared__ float dots[2][kHq][kChunk];      // [part][head][bucket]

  // 16-byte tile loads first: thread = bucket quad (tid & 7) x k-row phase (tid >> 3)
  const int quad = tid & 7, r = tid >> 3;
  const float4* tile = reinterpret_cast<const float4*>(moments + (size_t)(g * kChunks + c) * kRow * kChunk);
  float4 m4[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(tile + (r + 32 * i) * (kChunk / 4) + quad));
    m4[i] = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
  }
  for (int i = tid; i < kHq * kD; i += kRT) {
    const int h = i >> 7, k = i & (kD - 1);
    const float x = bf16_to_f32(q[((size_t)g * kHq + h) * kD + k]);
    reinterpret_cast<float*>(&qq[k])[h] = x;
    reinterpret_cast<float*>(&qq[kD + k])[h] = x * x;  // core.py:127 q.square() in fp32
  }
  __syncthreads();

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
  // reduce over the 8 k-row lanes of the wave (lane bits 5,4,3)
  treduce<16>(acc, 32);
  treduce<8>(acc, 16);
  treduce<4>(acc, 8);
  // lane now holds part (lane>>5)&1, head (lane>>3)&3, buckets 4*quad .. +3
  red[w][lane] = make_float4(acc[0], acc[1], acc[2], acc[3]);
  __syncthreads();
  {
    const int l = tid >> 2, j = tid & 3;
    const float s = ((reinterpret_cast<const float*>(&red[0][l])[j] + reinterpret_cast<const float*>(&red[1][l])[j]) +
                     reinterpret_cast<const float*>(&red[2][l])[j]) +
                    reinterpret_cast<const float*>(&red[3][l])[j];
    dots[(l >> 5) & 1][(l >> 3) & 3][4 * (l & 7) + j] = s;
  }
  __syncthreads();

  if (tid < kHq * kChunk) {
    // thread = (head tid>>5, bucket tid&31); 32 lanes per head
    const int h = tid >> 5, b = tid & 31, bucket = c * kChunk + b;
    const int n = counts[(size_t)g * kFP + bucket];
    float l = -INFINITY;
    if (n > 0) {
      // core.py:122-127: log(count) + (q @ mean^T) / sqrt(d) + (q^2 @ var^T) / (2d)
      const float lc = logf((float)n);
      l = (lc + dots[0][h][b] / kSqrtD) + dots[1][h][b] / (2.0f * kD);
    }
    work.logits[((size_t)g * kHq + h) * kFP + bucket] = l;
    float m = l;
#pragma unroll
    for (int o = 16; o; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    float e = (l == -INFINITY) ? 0.f : expf(l - m);
#pragma unroll
    for (int o = 16; o; o >>= 1) e += __shfl_xor(e, o);
    if (b == 0) *reinterpret_cast<float2*>(&work.stats[(((size_t)g * kChunks + c) * kHq + h) * 2]) = make_float2(m, e);
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

__global__ __launch_bounds__(kRT) void route_part_kernel(RouteWork work, unsigned long long* __restrict__ cand) {
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
    const float2 s0 = lane < kChunks ? st[lane * kHq] : make_float2(-INFINITY, 0.f);
    const float2 s1 = lane + 64 < kChunks ? st[(lane + 64) * kHq] : make_float2(-INFINITY, 0.f);
    const float m = wave_max(fmaxf(s0.x, s1.x));
    float z = (s0.x == -INFINITY ? 0.f : s0.y * expf(s0.x - m)) + (s1.x == -INFINITY ? 0.f : s1.y * expf(s1.x - m));
    z = wave_sum(z);
    if (lane == 0) {
      gmax[h] = m;
      grz[h] = z > 0.f ? 1.0f / z : 0.f;
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kPartKeys; ++i) {
    const int off = tid + i * kRT, b = part * kPartB + off;
    uint64_t key = 0;
    if (off < kPartB && lv[i][0] != -INFINITY) {
      // per-head softmax exp(l - M) / Z, then the sum over heads in head order (core.py:128)
      const float p0 = expf(lv[i][0] - gmax[0]) * grz[0];
      const float p1 = expf(lv[i][1] - gmax[1]) * grz[1];
      const float p2 = expf(lv[i][2] - gmax[2]) * grz[2];
      const float p3 = expf(lv[i][3] - gmax[3]) * grz[3];
      key = make_key(((p0 + p1) + p2) + p3, b);
    }
    keys[off] = key;
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

void prismkv::launch_route_score(const uint16_t* q, const float* moments, const int* counts, float* logits,
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

int prismkv_route(uint64_t q, uint64_t moments, uint64_t counts, uint64_t work, uint64_t features, uint64_t valid,
                  uint64_t raw, int groups, uint64_t stream) {
  if (groups < 1 || groups > 65535) return kBadSize;
  if (!q || !moments || !counts || !work || !features || !valid || !raw) return kBadSize;
  char* base = reinterpret_cast<char*>(work);
  RouteWork rw{reinterpret_cast<float*>(base), reinterpret_cast<float*>(base + route_logits_bytes(groups))};
  hipStream_t s = (hipStream_t)stream;
  launch_route_score(reinterpret_cast<const uint16_t*>(q), reinterpret_cast<const float*>(moments),
                     reinterpret_cast<const int*>(counts), rw.logits, rw.stats, groups, s);
  unsigned long long* cand =
      reinterpret_cast<unsigned long long*>(base + route_logits_bytes(groups) + route_stats_bytes(groups));
  hipLaunchKernelGGL(route_part_kernel, dim3(kParts, groups), dim3(kRT), 0, s, rw, cand);
  hipLaunchKernelGGL(route_final_kernel, dim3(groups), dim3(64), 0, s, cand, reinterpret_cast<const int*>(counts),
                     reinterpret_cast<int64_t*>(features), reinterpret_cast<float*>(valid),
                     reinterpret_cast<int*>(raw));
  return (int)hipGetLastError();
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
