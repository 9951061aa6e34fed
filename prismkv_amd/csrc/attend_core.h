// Sparse-attention core shared by the attend and decode kernels: the
// per-slot online softmax step, the workgroup state merge and the split merge.
#pragma once

#include "common.h"

namespace prismkv {
namespace {

constexpr int kAT = 512;                           // 8 waves
constexpr int kStateW = kD + 2;                    // {max, den, acc[128]}
constexpr float kLog2eScale = 0.12751743082459868f;  // log2(e) / sqrt(128): scores in the exp2 domain
constexpr float kSlack = 8.0f;                     // lazy-rescale threshold (log2 units)
constexpr int kStepRows = 16;                      // rows per wave step (4 slots x 4 rows)

// E: the element type of q, K, V and the output (uint16_t = bf16 bits, or float).
template <typename E>
struct AttendArgs {
  const E* q;
  const E* k;
  const E* v;
  const int32_t* ids;
  const int32_t* cnt;
  int64_t ks, vs, ids_stride;
  int H, T, S;
  float* state;
  unsigned* err = nullptr;  // error word (kErrIds for an id or count out of range), or none
};

__device__ __forceinline__ void unpack8(const uint4 r, float (&f)[8]) {
  f[0] = bf16_lo(r.x); f[1] = bf16_hi(r.x);
  f[2] = bf16_lo(r.y); f[3] = bf16_hi(r.y);
  f[4] = bf16_lo(r.z); f[5] = bf16_hi(r.z);
  f[6] = bf16_lo(r.w); f[7] = bf16_hi(r.w);
}

// 8 consecutive fp32 dims as loaded (two 16-byte loads).
struct F32x8 {
  uint4 a, b;
};
__device__ __forceinline__ void unpack8(const F32x8& r, float (&f)[8]) {
  f[0] = __uint_as_float(r.a.x); f[1] = __uint_as_float(r.a.y);
  f[2] = __uint_as_float(r.a.z); f[3] = __uint_as_float(r.a.w);
  f[4] = __uint_as_float(r.b.x); f[5] = __uint_as_float(r.b.y);
  f[6] = __uint_as_float(r.b.z); f[7] = __uint_as_float(r.b.w);
}

// The raw 8-dim load of one element type, and the output conversion.
template <typename E>
struct Row8;
template <>
struct Row8<uint16_t> {
  typedef uint4 Raw;
  static __device__ __forceinline__ Raw load(const uint16_t* p) { return load_nt16(p); }
  static __device__ __forceinline__ uint16_t out(float x) { return f32_to_bf16(x); }
};
template <>
struct Row8<float> {
  typedef F32x8 Raw;
  static __device__ __forceinline__ Raw load(const float* p) { return F32x8{load_nt16(p), load_nt16(p + 4)}; }
  static __device__ __forceinline__ float out(float x) { return x; }
};

__device__ __forceinline__ float exp2_or_zero(float x) { return x == -INFINITY ? 0.f : exp2f(x); }

constexpr int kSlotRows = 9;                 // rows per slot per round
constexpr int kWaveRows = 4 * kSlotRows;     // rows per wave per round

constexpr int kSlots = kAT / 16;             // 32 slots of 16 lanes

// LDS of one workgroup: the slot merge, then the split weights of the final merge.
struct AttendLds {
  union {
    struct {
      float sm[kSlots][kHq], sz[kSlots][kHq], wt[kSlots][kHq], mx[kHq];
      float sacc[kSlots][kHq][kD];
    } red;
    float wts[kAT / 64][64];               // split weights of the final merge
  };
};

// Per-lane running state of one slot: head-h scores live in lanes with
// (lane & 3) == h; acc holds all 4 heads x this lane's 8 dims.
struct SlotState {
  float m, z;            // running max / denominator of head (lane & 3)
  float acc[kHq][8];
};

// One step: 4 rows per slot (row b of slot = rows[b]); kr/vr hold the loaded
// lines (R: uint4 of 8 bf16 dims or F32x8); rows b >= nvalid are masked.
template <typename R>
__device__ __forceinline__ void attend_step(const float (&qf)[kHq][8], const R (&kr)[4], const R (&vr)[4],
                                            int nvalid, SlotState& s) {
  const int lane = threadIdx.x & 63, q16 = lane & 15, slot0 = lane & 48;
  float x[16];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    float kf[8];
    unpack8(kr[b], kf);
#pragma unroll
    for (int h = 0; h < kHq; ++h) {
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) d = fmaf(qf[h][i], kf[i], d);
      x[b * 4 + h] = d;
    }
  }
  // transpose-reduce over the 16 lanes of the slot: lane q16 ends with (row q16>>2, head q16&3)
#pragma unroll
  for (int stage = 0; stage < 4; ++stage) {
    const int mask = 8 >> stage, n = 8 >> stage;
    const unsigned long long hi = __ballot((q16 & mask) != 0);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (j < n) {
        const float keep = lane_select(hi, x[j + n], x[j]);
        const float send = lane_select(hi, x[j], x[j + n]);
        const float got = mask == 8 ? xor8(send) : mask == 4 ? xor4(send) : mask == 2 ? xor2(send) : xor1(send);
        x[j] = keep + got;
      }
    }
  }
  float sc = ((q16 >> 2) < nvalid) ? x[0] : -INFINITY;
  // batch max of this head over the 4 rows (lane bits 2, 3)
  float bm = fmaxf(sc, xor4(sc));
  bm = fmaxf(bm, xor8(bm));
  const bool grow = bm > s.m + kSlack || (s.m == -INFINITY && bm != -INFINITY);
  if (__ballot(grow)) {
    const float nm = grow ? bm : s.m;
    const float alpha = grow ? exp2_or_zero(s.m - nm) : 1.0f;
    s.m = nm;
    s.z *= alpha;
#pragma unroll
    for (int h = 0; h < kHq; ++h) {
      const float ah = __shfl(alpha, slot0 + h);
#pragma unroll
      for (int i = 0; i < 8; ++i) s.acc[h][i] *= ah;
    }
  }
  const float p = sc == -INFINITY ? 0.f : exp2f(sc - s.m);
  float ps = p + xor4(p);
  ps += xor8(ps);
  s.z += ps;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    if (b < nvalid) {
      float vf[8];
      unpack8(vr[b], vf);
#pragma unroll
      for (int h = 0; h < kHq; ++h) {
        const float pb = __shfl(p, slot0 + b * 4 + h);
#pragma unroll
        for (int i = 0; i < 8; ++i) s.acc[h][i] = fmaf(pb, vf[i], s.acc[h][i]);
      }
    }
  }
}

// Merges the 32 slot states of the workgroup in LDS and stores the result as
// split state `stp` ((max, den, acc[128]) per head; head h at stp + h * hstride).
__device__ inline void store_wg_state(const SlotState& s, AttendLds& lds, float* stp, size_t hstride) {
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, q16 = lane & 15, slot = lane >> 4;
  __syncthreads();  // LDS shared with the caller's earlier phases is free again
  // gather the slot's per-head max / denominator into every lane
  float mm[kHq], zz[kHq];
#pragma unroll
  for (int h = 0; h < kHq; ++h) {
    mm[h] = __shfl(s.m, (lane & 48) + h);
    zz[h] = __shfl(s.z, (lane & 48) + h);
  }
  const int sl = w * 4 + slot;
  if (q16 == 0) {
#pragma unroll
    for (int h = 0; h < kHq; ++h) {
      lds.red.sm[sl][h] = mm[h];
      lds.red.sz[sl][h] = zz[h];
    }
  }
#pragma unroll
  for (int h = 0; h < kHq; ++h) {
    float4* dst = reinterpret_cast<float4*>(&lds.red.sacc[sl][h][8 * q16]);
    dst[0] = make_float4(s.acc[h][0], s.acc[h][1], s.acc[h][2], s.acc[h][3]);
    dst[1] = make_float4(s.acc[h][4], s.acc[h][5], s.acc[h][6], s.acc[h][7]);
  }
  __syncthreads();
  if (tid < kSlots * kHq) {
    // slot weights e^(m_slot - M) per head, once: thread = (slot tid >> 2, head tid & 3)
    const int k = tid >> 2, h = tid & 3;
    float M = -INFINITY;
#pragma unroll
    for (int j = 0; j < kSlots; ++j) M = fmaxf(M, lds.red.sm[j][h]);
    const float m = lds.red.sm[k][h];
    lds.red.wt[k][h] = m == -INFINITY ? 0.f : exp2f(m - M);
    if (k == 0) lds.red.mx[h] = M;
  }
  __syncthreads();
  {
    // thread = (head tid >> 7, dim tid & 127)
    const int h = tid >> 7, d = tid & (kD - 1);
    const float M = lds.red.mx[h];
    float den = 0.f, v = 0.f;
#pragma unroll
    for (int k = 0; k < kSlots; ++k) {
      const float wgt = lds.red.wt[k][h];
      den = fmaf(wgt, lds.red.sz[k][h], den);
      v = fmaf(wgt, lds.red.sacc[k][h][d], v);
    }
    float* sh = stp + (size_t)h * hstride;
    if (d == 0) st_dev2(sh, M, den);
    st_dev(sh + 2 + d, v);
  }
}

// Merges the S split states of group g into out[g] (thread = head tid >> 7,
// dim tid & 127; out of element type E).  Splits go in batches of 32: each thread issues its 32
// accumulator loads and each wave its 32 (max, den) loads before any is
// used, so S <= 32 costs one memory round trip.  The caller has seen every
// split's arrival (the states are complete when this runs).
template <typename E>
__device__ void merge_group(const float* state, int S, int g, E* out, float (&wts)[kAT / 64][64]) {
  const int tid = threadIdx.x, h = tid >> 7, d = tid & (kD - 1), w = tid >> 6, lane = tid & 63;
  const float* st = state + (size_t)(g * kHq + h) * S * kStateW;
  float M = -INFINITY, den = 0.f, v = 0.f;
  for (int p0 = 0; p0 < S; p0 += 32) {
    const int n = min(32, S - p0);
    const float* mzp = st + (size_t)(p0 + min(lane & 31, n - 1)) * kStateW;
    const float2 mz = ld_dev2(mzp);
    float av[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) av[i] = ld_dev(st + (size_t)(p0 + min(i, n - 1)) * kStateW + 2 + d);
    // online merge across batches: rescale what is accumulated when the max grows
    const bool mine = lane < n;  // lanes 32..63 duplicate lanes 0..31 and stay out
    const float bm = wave_max(mine ? mz.x : -INFINITY);
    const float nM = fmaxf(M, bm);
    const float scale = (M == -INFINITY) ? 0.f : exp2f(M - nM);
    den *= scale;
    v *= scale;
    M = nM;
    const float wgt = (mine && mz.x != -INFINITY) ? exp2f(mz.x - M) : 0.f;
    den += wave_sum(wgt * mz.y);
    __syncthreads();  // previous batch's weights are consumed
    wts[w][lane] = wgt;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 32; ++i) v = fmaf(wts[w][i], av[i], v);
  }
  out[((size_t)g * kHq + h) * kD + d] = Row8<E>::out(den > 0.f ? v / den : 0.f);
}

}  // namespace
}  // namespace prismkv
