// Stage 3 -- sparse attention over the selected ORIGINAL bf16 KV rows plus the
// whole unindexed tail, read in place (no gather copy), 4 query heads of a KV
// group sharing every row.
//
// Semantics: src/prismkv/core.py:170-183 (exact softmax over selected rows and
//            tail [H, H+T), scale 1/sqrt(d)), kernels/ppu_8b/av_tuned.cu:16,31,60
//            (row j < count -> ids[j], else H + j - count; den == 0 -> 0).
//
// Design: grid (splits, G) x 256.  Split p of group g owns a contiguous range
// of the group's row list (the range is derived on device from count[g], so
// no host sync).  Each wave64 takes 4 rows per step; 16 lanes share a row and
// each lane loads 16 bytes (8 dims) of K and of V -- 256 contiguous bytes per
// row, fully used.  QK dot products reduce across the 16 lanes with xor
// shuffles; softmax is online in fp32 (no bf16 rounding of P); P.V
// accumulates in fp32.  The 16 row-slot states of a workgroup merge in LDS to
// one (max, denominator, acc[128]) per head, stored in the reference's split
// state layout [(g*4+h)*S + p][130].  The last workgroup of a group (device
// counter, restored to zero afterwards) merges the S split states and writes
// the bf16 output; the compat entry point uses a separate merge launch instead.
#include "common.h"

namespace prismkv {
namespace {

constexpr int kAT = 256;
constexpr int kStateW = kD + 2;                    // {max, den, acc[128]}
constexpr float kScale = 0.08838834764831845f;     // 1/sqrt(128)

struct AttendArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const int32_t* ids;
  const int32_t* cnt;
  int64_t ks, vs, ids_stride;
  int H, T, S;
  float* state;
};

__device__ __forceinline__ void unpack8(const uint4 r, float (&f)[8]) {
  f[0] = bf16_lo(r.x); f[1] = bf16_hi(r.x);
  f[2] = bf16_lo(r.y); f[3] = bf16_hi(r.y);
  f[4] = bf16_lo(r.z); f[5] = bf16_hi(r.z);
  f[6] = bf16_lo(r.w); f[7] = bf16_hi(r.w);
}

// Computes this workgroup's split state and writes it to a.state.
__device__ __forceinline__ void attend_split(const AttendArgs& a, int g, int p) {
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int r = lane >> 4, s = lane & 15;
  int n_old = a.cnt[g];
  n_old = n_old < 0 ? 0 : (n_old > a.H ? a.H : n_old);
  const int total = n_old + a.T;
  const int span = (total + a.S - 1) / a.S;
  const int j0 = min(total, p * span), j1 = min(total, j0 + span);
  const int last_row = a.H + a.T - 1;

  float qf[kHq][8];
#pragma unroll
  for (int h = 0; h < kHq; ++h)
    unpack8(*reinterpret_cast<const uint4*>(a.q + ((size_t)g * kHq + h) * kD + 8 * s), qf[h]);

  float acc[kHq][8], m[kHq], z[kHq];
#pragma unroll
  for (int h = 0; h < kHq; ++h) {
    m[h] = -INFINITY;
    z[h] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[h][i] = 0.f;
  }
  const uint16_t* kg = a.k + (size_t)g * a.ks + 8 * s;
  const uint16_t* vg = a.v + (size_t)g * a.vs + 8 * s;
  const int32_t* idg = a.ids + (size_t)g * a.ids_stride;

  for (int jb = j0 + w * 4; jb < j1; jb += 16) {
    const int j = jb + r;
    const bool ok = j < j1;
    float kf[8], vf[8];
    if (ok) {
      int pos = j < n_old ? idg[j] : a.H + (j - n_old);
      pos = pos < 0 ? 0 : (pos > last_row ? last_row : pos);
      unpack8(load_nt16(kg + (size_t)pos * kD), kf);
      unpack8(load_nt16(vg + (size_t)pos * kD), vf);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) kf[i] = vf[i] = 0.f;
    }
    float dot[kHq];
#pragma unroll
    for (int h = 0; h < kHq; ++h) {
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) d = fmaf(qf[h][i], kf[i], d);
      dot[h] = d;
    }
#pragma unroll
    for (int o = 8; o; o >>= 1)
#pragma unroll
      for (int h = 0; h < kHq; ++h) dot[h] += __shfl_xor(dot[h], o);
    if (ok) {
#pragma unroll
      for (int h = 0; h < kHq; ++h) {
        const float sc = dot[h] * kScale;
        const float nm = fmaxf(m[h], sc);
        const float alpha = __expf(m[h] - nm);
        const float pw = __expf(sc - nm);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[h][i] = fmaf(acc[h][i], alpha, pw * vf[i]);
        z[h] = fmaf(z[h], alpha, pw);
        m[h] = nm;
      }
    }
  }

  // merge the 16 row slots of the workgroup
  __shared__ float sm[16][kHq], sz[16][kHq];
  __shared__ float sacc[16][kHq][kD];
  const int slot = w * 4 + r;
  if (s == 0) {
#pragma unroll
    for (int h = 0; h < kHq; ++h) {
      sm[slot][h] = m[h];
      sz[slot][h] = z[h];
    }
  }
#pragma unroll
  for (int h = 0; h < kHq; ++h)
#pragma unroll
    for (int i = 0; i < 8; ++i) sacc[slot][h][8 * s + i] = acc[h][i];
  __syncthreads();
  {
    const int h = tid >> 6, d0 = (tid & 63) * 2;
    float M = -INFINITY;
#pragma unroll
    for (int sl = 0; sl < 16; ++sl) M = fmaxf(M, sm[sl][h]);
    float den = 0.f, v0 = 0.f, v1 = 0.f;
#pragma unroll
    for (int sl = 0; sl < 16; ++sl) {
      const float ms = sm[sl][h];
      const float wgt = ms == -INFINITY ? 0.f : __expf(ms - M);
      den = fmaf(wgt, sz[sl][h], den);
      v0 = fmaf(wgt, sacc[sl][h][d0], v0);
      v1 = fmaf(wgt, sacc[sl][h][d0 + 1], v1);
    }
    float* st = a.state + (((size_t)g * kHq + h) * a.S + p) * kStateW;
    if ((tid & 63) == 0) {
      st[0] = M;
      st[1] = den;
    }
    st[2 + d0] = v0;
    st[3 + d0] = v1;
  }
}

// Merges the S split states of head row `hh` (= g*4 + h) for dims d0, d0+1.
__device__ __forceinline__ void merge_head(const float* state, int S, int hh, int d0, uint16_t* out) {
  const float* st = state + (size_t)hh * S * kStateW;
  float M = -INFINITY;
  for (int pp = 0; pp < S; ++pp) M = fmaxf(M, st[(size_t)pp * kStateW]);
  float den = 0.f, v0 = 0.f, v1 = 0.f;
  for (int pp = 0; pp < S; ++pp) {
    const float* sp = st + (size_t)pp * kStateW;
    const float mp = sp[0];
    const float wgt = mp == -INFINITY ? 0.f : __expf(mp - M);
    den = fmaf(wgt, sp[1], den);
    v0 = fmaf(wgt, sp[2 + d0], v0);
    v1 = fmaf(wgt, sp[3 + d0], v1);
  }
  out[(size_t)hh * kD + d0] = f32_to_bf16(den > 0.f ? v0 / den : 0.f);
  out[(size_t)hh * kD + d0 + 1] = f32_to_bf16(den > 0.f ? v1 / den : 0.f);
}

__global__ __launch_bounds__(kAT) void attend_fused(AttendArgs a, unsigned* __restrict__ sync,
                                                    uint16_t* __restrict__ out) {
  const int p = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
  __shared__ int is_last;
  attend_split(a, g, p);
  __threadfence();
  __syncthreads();
  if (tid == 0) is_last = atomic_add_agent(&sync[g], 1u) == (unsigned)(a.S - 1);
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  if (tid == 0) atomic_store_agent(&sync[g], 0u);
  merge_head(a.state, a.S, g * kHq + (tid >> 6), (tid & 63) * 2, out);
}

__global__ __launch_bounds__(kAT) void attend_split_only(AttendArgs a) { attend_split(a, blockIdx.y, blockIdx.x); }

// Compat merge: grid (8*4) x 64, one head row per workgroup.
__global__ __launch_bounds__(64) void attend_merge(const float* __restrict__ state, uint16_t* __restrict__ out,
                                                   int S) {
  merge_head(state, S, blockIdx.x, threadIdx.x * 2, out);
}

}  // namespace
}  // namespace prismkv

using namespace prismkv;

extern "C" {

size_t prismkv_attend_work_bytes(int groups, int splits) {
  if (groups < 1 || splits < 1) return 0;
  return (size_t)groups * kHq * splits * kStateW * sizeof(float) + (size_t)groups * sizeof(unsigned);
}

int prismkv_attend(uint64_t q, uint64_t k, uint64_t v, uint64_t ids, uint64_t count, uint64_t work, uint64_t out,
                   int groups, int H, int T, int64_t ks, int64_t vs, int64_t ids_stride, int splits,
                   uint64_t stream) {
  if (groups < 1 || groups > 65535 || H < 0 || T < 0 || splits < 1 || splits > 1024) return kBadSize;
  if (ks < (int64_t)(H + T) * kD || vs < (int64_t)(H + T) * kD || ids_stride < H) return kBadSize;
  if (!q || !k || !v || !ids || !count || !work || !out) return kBadSize;
  AttendArgs a{reinterpret_cast<const uint16_t*>(q), reinterpret_cast<const uint16_t*>(k),
               reinterpret_cast<const uint16_t*>(v), reinterpret_cast<const int32_t*>(ids),
               reinterpret_cast<const int32_t*>(count), ks, vs, ids_stride, H, T, splits,
               reinterpret_cast<float*>(work)};
  unsigned* sync = reinterpret_cast<unsigned*>(reinterpret_cast<float*>(work) +
                                               (size_t)groups * kHq * splits * kStateW);
  hipLaunchKernelGGL(attend_fused, dim3(splits, groups), dim3(kAT), 0, (hipStream_t)stream, a, sync,
                     reinterpret_cast<uint16_t*>(out));
  return (int)hipGetLastError();
}

// kernels/ppu_8b/av_tuned.cu:62-67 contract; state is the caller's
// f32 [32][128][130] buffer, used as [(g*4+h)*S + p][130].
int attention_tuned(uint64_t q, uint64_t k, uint64_t v, uint64_t ids, uint64_t cnt, uint64_t state, uint64_t out,
                    int H, int T, int KS, int VS, int S, int mode, uint64_t stream) {
  if (S < 1 || S > 128 || H < 1 || T < 0 || KS < (H + T) * kD || VS < (H + T) * kD) return kBadSize;
  if (mode < 0 || mode > 2) return kBadMode;
  AttendArgs a{reinterpret_cast<const uint16_t*>(q), reinterpret_cast<const uint16_t*>(k),
               reinterpret_cast<const uint16_t*>(v), reinterpret_cast<const int32_t*>(ids),
               reinterpret_cast<const int32_t*>(cnt), KS, VS, H, H, T, S, reinterpret_cast<float*>(state)};
  hipLaunchKernelGGL(attend_split_only, dim3(S, 8), dim3(kAT), 0, (hipStream_t)stream, a);
  hipLaunchKernelGGL(attend_merge, dim3(8 * kHq), dim3(64), 0, (hipStream_t)stream,
                     reinterpret_cast<const float*>(state), reinterpret_cast<uint16_t*>(out), S);
  return (int)hipGetLastError();
}

}  // extern "C"
