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
//   * The select kernel (one workgroup per group) merges the 94 chunk
//     statistics, forms the head-summed probabilities exp(l - M) / Z -- equal
//     logits give bit-equal probabilities, so exact ties fall to the lower
//     bucket id as in the reference -- and picks the Top-16 on 44-bit keys
//     (probability bits << 12 | 4095 - bucket): value descending, bucket id
//     ascending on ties.  The select ranks per-thread maxima with LDS
//     broadcast reads to find a threshold, then ranks the few keys above it
//     (no histogram atomics, no sorting network).
#include "common.h"

namespace prismkv {
namespace {

constexpr int kRT = 256;                      // route workgroup size
constexpr int kKeys = (kFP + kRT - 1) / kRT;  // 12 candidate keys per thread
constexpr float kSqrtD = 11.3137084989847604f;  // fp32(sqrt(128)), core.py:125

struct SelectLds {
  unsigned long long tm[kRT];    // per-thread maxima
  unsigned long long cand[kRT];  // keys >= tau
  unsigned long long sel[kTop];  // the winners, rank order
  unsigned long long tau;
  int ncand;
};

__device__ __forceinline__ uint64_t make_key(float prob, int bucket) {
  return ((uint64_t)__float_as_uint(prob) << 12) | (uint64_t)(4095 - bucket);
}
__device__ __forceinline__ int key_bucket(uint64_t k) { return 4095 - (int)(k & 4095u); }

// Top-16 of the nonzero keys of the workgroup (unique by construction), in
// rank order, into lds.sel; returns how many (min(16, live)).  No histogram
// and no sorting network: tau = the 16th largest per-thread maximum, found by
// ranking the 256 maxima against each other with LDS broadcast reads; at
// least 16 keys are >= tau and at most 16 threads hold such keys (15 when
// fewer than 16 threads hold a live key and tau falls back to 1), so the
// <= 192 candidates >= tau are ranked exactly the same way.
__device__ int select_top(const uint64_t (&key)[kKeys], SelectLds& lds) {
  const int tid = threadIdx.x;
  unsigned long long lm = 0;
#pragma unroll
  for (int i = 0; i < kKeys; ++i) lm = key[i] > lm ? key[i] : lm;
  lds.tm[tid] = lm;
  if (tid == 0) {
    lds.tau = 1;  // dead keys (0) never qualify
    lds.ncand = 0;
  }
  __syncthreads();
  int r = 0;
  const ulonglong2* tm2 = reinterpret_cast<const ulonglong2*>(lds.tm);
#pragma unroll 8
  for (int j = 0; j < kRT / 2; ++j) {
    const ulonglong2 o = tm2[j];
    r += (o.x > lm) + (o.y > lm);
  }
  if (r == kTop - 1 && lm > 0) lds.tau = lm;  // unique: nonzero maxima are distinct
  __syncthreads();
  const unsigned long long tau = lds.tau;
  int mine = 0;
#pragma unroll
  for (int i = 0; i < kKeys; ++i) mine += key[i] >= tau;
  if (mine) {
    int at = atomicAdd(&lds.ncand, mine);
#pragma unroll
    for (int i = 0; i < kKeys; ++i)
      if (key[i] >= tau && at < kRT) lds.cand[at++] = key[i];
  }
  __syncthreads();
  const int nc = lds.ncand < kRT ? lds.ncand : kRT;
  if (tid < nc) {
    const unsigned long long k = lds.cand[tid];
    int rk = 0;
    for (int j = 0; j < nc; ++j) rk += lds.cand[j] > k;
    if (rk < kTop) lds.sel[rk] = k;
  }
  __syncthreads();
  return nc < kTop ? nc : kTop;
}

// Writes the winners (lds.sel, rank order): features[r] = bucket, valid[r] =
// 1 for r < need; remaining slots id 0 / valid 0 (route_parallel.cu:23,29);
// raw = sum of winner counts.
template <typename CountT>
__device__ void write_selection(const SelectLds& lds, int need, const CountT* counts, int64_t* features,
                                float* valid, int* raw) {
  const int tid = threadIdx.x;
  if (tid < 64) {
    const bool hit = tid < need;
    const int b = hit ? key_bucket(lds.sel[tid]) : 0;
    if (tid < kTop) {
      features[tid] = b;
      valid[tid] = hit ? 1.0f : 0.0f;
    }
    const int n = wave_sum_i(hit ? (int)counts[b] : 0);
    if (tid == 0) *raw = n;
  }
}

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
// Route, pass 2 (normalise, aggregate, Top-16): grid G x 256.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kRT) void route_select_kernel(RouteWork work, const int* __restrict__ counts,
                                                           int64_t* __restrict__ features,
                                                           float* __restrict__ valid, int* __restrict__ raw) {
  const int g = blockIdx.x, tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  __shared__ float gmax[kHq], grz[kHq];
  __shared__ SelectLds lds;
  // every load of the workgroup is issued before any is used
  const float* lg = work.logits + (size_t)g * kHq * kFP;
  float lv[kKeys][kHq];
#pragma unroll
  for (int i = 0; i < kKeys; ++i) {
    const int b = min(tid + i * kRT, kFP - 1);
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
  uint64_t key[kKeys];
#pragma unroll
  for (int i = 0; i < kKeys; ++i) {
    const int b = tid + i * kRT;
    key[i] = 0;
    if (b < kFP && lv[i][0] != -INFINITY) {
      // per-head softmax exp(l - M) / Z, then the sum over heads in head order (core.py:128)
      const float p0 = expf(lv[i][0] - gmax[0]) * grz[0];
      const float p1 = expf(lv[i][1] - gmax[1]) * grz[1];
      const float p2 = expf(lv[i][2] - gmax[2]) * grz[2];
      const float p3 = expf(lv[i][3] - gmax[3]) * grz[3];
      key[i] = make_key(((p0 + p1) + p2) + p3, b);
    }
  }
  const int need = select_top(key, lds);
  write_selection(lds, need, counts + (size_t)g * kFP, features + (size_t)g * kTop, valid + (size_t)g * kTop,
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
  __shared__ SelectLds lds;
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
  uint64_t key[kKeys];
#pragma unroll
  for (int i = 0; i < kKeys; ++i) {
    const int b = tid + i * kRT;
    key[i] = 0;
    if (b < kF && cg[b] > 0) {
      float a = 0.f;
#pragma unroll
      for (int h = 0; h < kHq; ++h) a += hsum[h] > 0.f ? lv[h][i] / hsum[h] : 0.f;
      key[i] = make_key(a, b);
    }
  }
  const int need = select_top(key, lds);
  write_selection(lds, need, cg, ids + (size_t)g * kTop, vals + (size_t)g * kTop, raw + g);
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

static size_t route_logits_bytes(int groups) { return (size_t)groups * kHq * kFP * sizeof(float); }
static size_t route_stats_bytes(int groups) { return (size_t)groups * kChunks * kHq * 2 * sizeof(float); }

extern "C" {

size_t prismkv_route_work_bytes(int groups) {
  if (groups < 1) return 0;
  return route_logits_bytes(groups) + route_stats_bytes(groups);
}

int prismkv_route(uint64_t q, uint64_t moments, uint64_t counts, uint64_t work, uint64_t features, uint64_t valid,
                  uint64_t raw, int groups, uint64_t stream) {
  if (groups < 1 || groups > 65535) return kBadSize;
  if (!q || !moments || !counts || !work || !features || !valid || !raw) return kBadSize;
  char* base = reinterpret_cast<char*>(work);
  RouteWork rw{reinterpret_cast<float*>(base), reinterpret_cast<float*>(base + route_logits_bytes(groups))};
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(route_score_kernel, dim3(kChunks, groups), dim3(kRT), 0, s, reinterpret_cast<const uint16_t*>(q),
                     reinterpret_cast<const float*>(moments), reinterpret_cast<const int*>(counts), rw);
  hipLaunchKernelGGL(route_select_kernel, dim3(groups), dim3(kRT), 0, s, rw, reinterpret_cast<const int*>(counts),
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
