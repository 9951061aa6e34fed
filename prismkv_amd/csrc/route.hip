// Stage 1 -- route: score the F=3000 buckets of each KV group from stored
// count / mean / diagonal-variance moments against the 4 query heads, softmax
// per head, average over heads, select the Top-16 live buckets.
//
// Semantics: src/prismkv/core.py:106-130 (router="moments"),
//            kernels/ppu_8b/route_parallel.cu:12-32 (tie rule, padding, raw).
//
// Design (one launch per layer, no vendor GEMM):
//   * Moment tables live in HBM as 64-bucket tiles [g][chunk][k][64] (k < 128:
//     mean, k >= 128: variance), so one wave64 reads 256 contiguous bytes per
//     k-row and each lane owns one bucket -- the 4-head dot products need no
//     cross-lane reduction.  A workgroup of 4 waves splits k into quarters and
//     combines the partial sums in LDS in a fixed order (ties stay exact).
//   * Each workgroup writes its 64x4 logits plus per-head (max, sum-exp) chunk
//     statistics; the last workgroup of the group (device-scope counter)
//     merges the 47 chunk statistics, forms the head-averaged probabilities
//     and selects the Top-16 with an LDS radix select on 64-bit keys
//     (probability bits << 32 | ~bucket), i.e. value descending, bucket id
//     ascending on ties -- the reference order.  The counter is restored to
//     zero by that workgroup, so the launch can be replayed from a graph.
#include "common.h"

namespace prismkv {
namespace {

constexpr int kRT = 256;                    // route workgroup size
constexpr int kKeys = (kFP + kRT - 1) / kRT;  // 12 candidate keys per thread

struct SelectLds {
  unsigned hist[256];
  unsigned wsum[4];
  unsigned long long sel[kTop];
  int nsel, digit, rem, stop, live;
};

// Writes the min(kTop, live) largest nonzero keys of the workgroup into
// lds.sel (unordered) and returns that count.  Keys are unique by
// construction, so the selected set has exactly `need` members.
__device__ int select_top(const uint64_t (&key)[kKeys], SelectLds& lds) {
  const int tid = threadIdx.x;
  int nl = 0;
#pragma unroll
  for (int i = 0; i < kKeys; ++i) nl += key[i] != 0;
  if (tid == 0) { lds.live = 0; lds.nsel = 0; }
  __syncthreads();
  if (nl) atomicAdd(&lds.live, nl);
  __syncthreads();
  const int live = lds.live;
  const int need = live < kTop ? live : kTop;
  uint64_t prefix = 0;
  int shift = 64;
  if (live > need) {
    // MSB-first radix select over 8-bit digits of the 64-bit key.
    unsigned rem = (unsigned)need;
    for (;;) {
      shift -= 8;
      lds.hist[tid] = 0;
      __syncthreads();
#pragma unroll
      for (int i = 0; i < kKeys; ++i) {
        const uint64_t k = key[i];
        if (k != 0 && (shift == 56 || (k >> (shift + 8)) == prefix))
          atomicAdd(&lds.hist[(unsigned)(k >> shift) & 255u], 1u);
      }
      __syncthreads();
      // thread t looks at digit 255-t: inclusive scan = keys with digit >= 255-t
      const unsigned c = lds.hist[255 - tid];
      const unsigned incl = block_incl_scan<kRT>(c, lds.wsum);
      const unsigned excl = incl - c;
      if (excl < rem && incl >= rem) {
        lds.digit = 255 - tid;
        lds.rem = (int)(rem - excl);
        lds.stop = (c == rem - excl);
      }
      __syncthreads();
      prefix = (prefix << 8) | (uint64_t)lds.digit;
      rem = (unsigned)lds.rem;
      const bool stop = lds.stop != 0;
      __syncthreads();
      if (stop || shift == 0) break;
    }
  }
#pragma unroll
  for (int i = 0; i < kKeys; ++i) {
    const uint64_t k = key[i];
    if (k != 0 && (live <= need || (k >> shift) >= prefix)) {
      const int s = atomicAdd(&lds.nsel, 1);
      if (s < kTop) lds.sel[s] = k;
    }
  }
  __syncthreads();
  return need;
}

// Writes the selected keys in rank order: features[r] = bucket, valid[r] = 1
// for r < need; remaining slots id 0 / valid 0; raw = sum of winner counts.
template <typename CountT>
__device__ void write_selection(const SelectLds& lds, int need, const CountT* counts, int64_t* features,
                                float* valid, int* raw) {
  const int tid = threadIdx.x;
  if (tid < need) {
    const unsigned long long k = lds.sel[tid];
    int r = 0;
    for (int j = 0; j < need; ++j) r += lds.sel[j] > k;
    features[r] = (int64_t)(0xffffffffu - (unsigned)(k & 0xffffffffu));
    valid[r] = 1.0f;
  } else if (tid < kTop) {
    features[tid] = 0;
    valid[tid] = 0.0f;
  }
  if (tid == 0) {
    int total = 0;
    for (int j = 0; j < need; ++j) total += (int)counts[0xffffffffu - (unsigned)(lds.sel[j] & 0xffffffffu)];
    *raw = total;
  }
}

__device__ __forceinline__ uint64_t make_key(float prob, int bucket) {
  return ((uint64_t)__float_as_uint(prob) << 32) | (uint64_t)(0xffffffffu - (unsigned)bucket);
}

// ---------------------------------------------------------------------------
// Fused route: grid (kChunks, G) x 256.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kRT) void route_kernel(const uint16_t* __restrict__ q,
                                                    const float* __restrict__ moments,
                                                    const int* __restrict__ counts,
                                                    float* __restrict__ logits, float* __restrict__ stats,
                                                    unsigned* __restrict__ sync, int64_t* __restrict__ features,
                                                    float* __restrict__ valid, int* __restrict__ raw) {
  const int c = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
  const int w = tid >> 6, lane = tid & 63;
  __shared__ float4 qq[kRow];            // [k] -> 4 heads; k < 128: q, k >= 128: q*q
  __shared__ float part[4][kHq][kChunk];  // [k quarter][head][bucket]
  __shared__ int is_last;
  __shared__ float gmax[kHq], gsum[kHq];
  __shared__ SelectLds lds;

  for (int i = tid; i < kHq * kD; i += kRT) {
    const int h = i >> 7, k = i & (kD - 1);
    const float x = bf16_to_f32(q[((size_t)g * kHq + h) * kD + k]);
    reinterpret_cast<float*>(&qq[k])[h] = x;
    reinterpret_cast<float*>(&qq[kD + k])[h] = x * x;
  }
  __syncthreads();

  // wave w covers moment rows [64w, 64w+64) of this chunk's tile
  const float* tile = moments + ((size_t)(g * kChunks + c) * kRow + w * 64) * kChunk + lane;
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll 16
  for (int kk = 0; kk < 64; ++kk) {
    const float t = __builtin_nontemporal_load(tile + kk * kChunk);
    const float4 qv = qq[w * 64 + kk];
    a0 = fmaf(qv.x, t, a0);
    a1 = fmaf(qv.y, t, a1);
    a2 = fmaf(qv.z, t, a2);
    a3 = fmaf(qv.w, t, a3);
  }
  part[w][0][lane] = a0;
  part[w][1][lane] = a1;
  part[w][2][lane] = a2;
  part[w][3][lane] = a3;
  __syncthreads();

  {
    // wave h finalises head h for the 64 buckets of the chunk
    const int h = w, b = c * kChunk + lane;
    const int n = counts[(size_t)g * kFP + b];
    const float dm = part[0][h][lane] + part[1][h][lane];
    const float dv = part[2][h][lane] + part[3][h][lane];
    // core.py:122-127 order: log(count) + mean term + variance term
    const float l = n > 0 ? (logf((float)n) + dm / 11.3137084989847604f) + dv * (1.0f / 256.0f) : -INFINITY;
    logits[((size_t)g * kHq + h) * kFP + b] = l;
    const float m = wave_max(l);
    const float e = (l == -INFINITY) ? 0.f : expf(l - m);
    const float z = wave_sum(e);
    if (lane == 0) {
      stats[(((size_t)g * kChunks + c) * kHq + h) * 2 + 0] = m;
      stats[(((size_t)g * kChunks + c) * kHq + h) * 2 + 1] = z;
    }
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) is_last = atomic_add_agent(&sync[g], 1u) == (unsigned)(kChunks - 1);
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  if (tid == 0) atomic_store_agent(&sync[g], 0u);

  {
    // merge chunk statistics: wave h handles head h, lane = chunk
    const int h = w;
    const float mc = lane < kChunks ? stats[(((size_t)g * kChunks + lane) * kHq + h) * 2 + 0] : -INFINITY;
    const float zc = lane < kChunks ? stats[(((size_t)g * kChunks + lane) * kHq + h) * 2 + 1] : 0.f;
    const float m = wave_max(mc);
    const float z = wave_sum(mc == -INFINITY ? 0.f : zc * expf(mc - m));
    if (lane == 0) {
      gmax[h] = m;
      gsum[h] = z;
    }
  }
  __syncthreads();

  uint64_t key[kKeys];
  const float* lg = logits + (size_t)g * kHq * kFP;
#pragma unroll
  for (int i = 0; i < kKeys; ++i) {
    const int b = tid + i * kRT;
    key[i] = 0;
    if (b < kFP) {
      const float l0 = lg[b];
      if (l0 != -INFINITY) {
        const float p0 = expf(l0 - gmax[0]) / gsum[0];
        const float p1 = expf(lg[kFP + b] - gmax[1]) / gsum[1];
        const float p2 = expf(lg[2 * kFP + b] - gmax[2]) / gsum[2];
        const float p3 = expf(lg[3 * kFP + b] - gmax[3]) / gsum[3];
        key[i] = make_key(((p0 + p1) + p2) + p3, b);
      }
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

extern "C" {

size_t prismkv_route_work_bytes(int groups) {
  if (groups < 1) return 0;
  const size_t logits = (size_t)groups * kHq * kFP * sizeof(float);
  const size_t stats = (size_t)groups * kChunks * kHq * 2 * sizeof(float);
  const size_t sync = (size_t)groups * sizeof(unsigned);
  return logits + stats + ((sync + 255) & ~(size_t)255);
}

int prismkv_route(uint64_t q, uint64_t moments, uint64_t counts, uint64_t work, uint64_t features, uint64_t valid,
                  uint64_t raw, int groups, uint64_t stream) {
  if (groups < 1 || groups > 65535) return kBadSize;
  if (!q || !moments || !counts || !work || !features || !valid || !raw) return kBadSize;
  float* logits = reinterpret_cast<float*>(work);
  float* stats = logits + (size_t)groups * kHq * kFP;
  unsigned* sync = reinterpret_cast<unsigned*>(stats + (size_t)groups * kChunks * kHq * 2);
  hipLaunchKernelGGL(route_kernel, dim3(kChunks, groups), dim3(kRT), 0, (hipStream_t)stream,
                     reinterpret_cast<const uint16_t*>(q), reinterpret_cast<const float*>(moments),
                     reinterpret_cast<const int*>(counts), logits, stats, sync, reinterpret_cast<int64_t*>(features),
                     reinterpret_cast<float*>(valid), reinterpret_cast<int*>(raw));
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
