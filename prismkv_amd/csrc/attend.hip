// Stage 3 -- sparse attention over the selected ORIGINAL bf16 KV rows plus the
// whole unindexed tail, read in place (no gather copy), 4 query heads of a KV
// group sharing every row.
//
// Semantics: src/prismkv/core.py:170-183 (exact softmax over selected rows and
//            tail [H, H+T), scale 1/sqrt(d)), kernels/ppu_8b/av_tuned.cu:16,31,60
//            (row j < count -> ids[j], else H + j - count; den == 0 -> 0).
//
// Design: grid (splits, G) x 256.  Split p of group g owns a contiguous range
// of the group's row list (derived on device from count[g]: no host sync).
// Row positions of the range are staged in LDS first, so K/V loads never wait
// on an index load.  Each wave64 is 4 slots of 16 lanes; a slot takes 4 rows
// per step and each lane loads 16 bytes (8 dims) of K and of V per row --
// every row is one fully used 256-byte line pair.  Loads of the next step are
// issued before the current step is computed (register double buffering).
// The 16 (row, head) partial dot products of a lane are reduced across the
// slot with a transpose-reduce (15 shuffles), leaving one score per lane.
// Softmax runs online in the exp2 domain with a lazy rescale (the running
// max moves only when a score exceeds it by more than 2^8), P stays fp32 and
// P.V accumulates in fp32.  The 16 slot states of a workgroup merge in LDS to
// one (max, denominator, acc[128]) per head, stored in the reference's split
// state layout [(g*4+h)*S + p][130].  The last workgroup of a group (device
// counter, restored to zero afterwards) merges the S split states and writes
// the bf16 output; the compat entry point uses a separate merge launch.
// Split states cross workgroups through write-through stores, not fences.
#include "common.h"

namespace prismkv {
namespace {

constexpr int kAT = 256;
constexpr int kStateW = kD + 2;                    // {max, den, acc[128]}
constexpr float kLog2eScale = 0.12751743082459868f;  // log2(e) / sqrt(128): scores in the exp2 domain
constexpr float kSlack = 8.0f;                     // lazy-rescale threshold (log2 units)
constexpr int kPosChunk = 1024;                    // row positions staged in LDS per round
constexpr int kStepRows = 16;                      // rows per wave step (4 slots x 4 rows)

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

__device__ __forceinline__ float exp2_or_zero(float x) { return x == -INFINITY ? 0.f : exp2f(x); }

struct AttendLds {
  int pos[kPosChunk];
  float sm[16][kHq], sz[16][kHq];
  float sacc[16][kHq][kD];
};

// Per-lane running state of one slot: head-h scores live in lanes with
// (lane & 3) == h; acc holds all 4 heads x this lane's 8 dims.
struct SlotState {
  float m, z;            // running max / denominator of head (lane & 3)
  float acc[kHq][8];
};

// One step: 4 rows per slot (row b of slot = rows[b]); kr/vr hold the loaded
// lines; ok[b] marks real rows.
__device__ __forceinline__ void attend_step(const float (&qf)[kHq][8], const uint4 (&kr)[4], const uint4 (&vr)[4],
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
    const bool hi = (q16 & mask) != 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (j < n) {
        const float keep = hi ? x[j + n] : x[j];
        const float send = hi ? x[j] : x[j + n];
        x[j] = keep + __shfl_xor(send, mask);
      }
    }
  }
  float sc = ((q16 >> 2) < nvalid) ? x[0] : -INFINITY;
  // batch max of this head over the 4 rows (lane bits 2, 3)
  float bm = fmaxf(sc, __shfl_xor(sc, 4));
  bm = fmaxf(bm, __shfl_xor(bm, 8));
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
  float ps = p + __shfl_xor(p, 4);
  ps += __shfl_xor(ps, 8);
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

// Computes this workgroup's split state and writes it to a.state.
__device__ void attend_split(const AttendArgs& a, int g, int p, AttendLds& lds) {
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int q16 = lane & 15, slot = lane >> 4;
  int n_old = a.cnt[g];
  n_old = n_old < 0 ? 0 : (n_old > a.H ? a.H : n_old);
  const int total = n_old + a.T;
  const int span = (total + a.S - 1) / a.S;
  const int j0 = min(total, p * span), j1 = min(total, j0 + span);
  const int last_row = a.H + a.T - 1;

  float qf[kHq][8];
#pragma unroll
  for (int h = 0; h < kHq; ++h) {
    unpack8(*reinterpret_cast<const uint4*>(a.q + ((size_t)g * kHq + h) * kD + 8 * q16), qf[h]);
#pragma unroll
    for (int i = 0; i < 8; ++i) qf[h][i] *= kLog2eScale;
  }
  SlotState s;
  s.m = -INFINITY;
  s.z = 0.f;
#pragma unroll
  for (int h = 0; h < kHq; ++h)
#pragma unroll
    for (int i = 0; i < 8; ++i) s.acc[h][i] = 0.f;

  const uint16_t* kg = a.k + (size_t)g * a.ks + 8 * q16;
  const uint16_t* vg = a.v + (size_t)g * a.vs + 8 * q16;
  const int32_t* idg = a.ids + (size_t)g * a.ids_stride;

  for (int c0 = j0; c0 < j1; c0 += kPosChunk) {
    const int n = min(kPosChunk, j1 - c0);
    __syncthreads();  // previous chunk's positions are consumed
    for (int i = tid; i < n; i += kAT) {
      const int j = c0 + i;
      int pos = j < n_old ? idg[j] : a.H + (j - n_old);
      lds.pos[i] = pos < 0 ? 0 : (pos > last_row ? last_row : pos);
    }
    __syncthreads();
    // wave w takes steps w, w+4, ...; a step is 16 rows = 4 slots x 4 rows
    const int steps = (n + kStepRows - 1) / kStepRows;
    int st = w;
    if (st >= steps) continue;
    uint4 kc[4], vc[4];
    auto issue = [&](int step, uint4 (&kr)[4], uint4 (&vr)[4]) {
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int i = step * kStepRows + slot * 4 + b;
        const int pos = lds.pos[i < n ? i : n - 1];
        kr[b] = load_nt16(kg + (size_t)pos * kD);
        vr[b] = load_nt16(vg + (size_t)pos * kD);
      }
    };
    issue(st, kc, vc);
    for (;;) {
      const int nxt = st + kAT / 64;
      uint4 kn[4], vn[4];
      if (nxt < steps) issue(nxt, kn, vn);
      const int rem = n - (st * kStepRows + slot * 4);
      attend_step(qf, kc, vc, rem < 0 ? 0 : (rem > 4 ? 4 : rem), s);
      if (nxt >= steps) break;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        kc[b] = kn[b];
        vc[b] = vn[b];
      }
      st = nxt;
    }
  }

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
      lds.sm[sl][h] = mm[h];
      lds.sz[sl][h] = zz[h];
    }
  }
#pragma unroll
  for (int h = 0; h < kHq; ++h) {
    float4* dst = reinterpret_cast<float4*>(&lds.sacc[sl][h][8 * q16]);
    dst[0] = make_float4(s.acc[h][0], s.acc[h][1], s.acc[h][2], s.acc[h][3]);
    dst[1] = make_float4(s.acc[h][4], s.acc[h][5], s.acc[h][6], s.acc[h][7]);
  }
  __syncthreads();
  {
    const int h = tid >> 6, d0 = (tid & 63) * 2;
    float M = -INFINITY;
#pragma unroll
    for (int k = 0; k < 16; ++k) M = fmaxf(M, lds.sm[k][h]);
    float den = 0.f, v0 = 0.f, v1 = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const float wgt = exp2_or_zero(lds.sm[k][h] == -INFINITY ? -INFINITY : lds.sm[k][h] - M);
      den = fmaf(wgt, lds.sz[k][h], den);
      v0 = fmaf(wgt, lds.sacc[k][h][d0], v0);
      v1 = fmaf(wgt, lds.sacc[k][h][d0 + 1], v1);
    }
    float* stp = a.state + (((size_t)g * kHq + h) * a.S + p) * kStateW;
    if ((tid & 63) == 0) st_dev2(stp, M, den);
    st_dev2(stp + 2 + d0, v0, v1);
  }
}

// Merges the S split states of head row hh (= g*4 + h) for dims d0, d0+1.
// All state loads of a batch of 16 splits are issued before any is used.
__device__ __forceinline__ void merge_head(const float* state, int S, int hh, int d0, uint16_t* out) {
  const float* st = state + (size_t)hh * S * kStateW;
  float M = -INFINITY;
  for (int p0 = 0; p0 < S; p0 += 16) {
    float mv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) mv[i] = p0 + i < S ? ld_dev(st + (size_t)(p0 + i) * kStateW) : -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) M = fmaxf(M, mv[i]);
  }
  float den = 0.f, v0 = 0.f, v1 = 0.f;
  for (int p0 = 0; p0 < S; p0 += 16) {
    float mv[16], zv[16];
    float2 av[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (p0 + i < S) {
        const float* sp = st + (size_t)(p0 + i) * kStateW;
        const float2 mz = ld_dev2(sp);
        mv[i] = mz.x;
        zv[i] = mz.y;
        av[i] = ld_dev2(sp + 2 + d0);
      } else {
        mv[i] = -INFINITY;
        zv[i] = 0.f;
        av[i] = make_float2(0.f, 0.f);
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float wgt = mv[i] == -INFINITY ? 0.f : exp2f(mv[i] - M);
      den = fmaf(wgt, zv[i], den);
      v0 = fmaf(wgt, av[i].x, v0);
      v1 = fmaf(wgt, av[i].y, v1);
    }
  }
  out[(size_t)hh * kD + d0] = f32_to_bf16(den > 0.f ? v0 / den : 0.f);
  out[(size_t)hh * kD + d0 + 1] = f32_to_bf16(den > 0.f ? v1 / den : 0.f);
}

__global__ __launch_bounds__(kAT) void attend_fused(AttendArgs a, unsigned* __restrict__ sync,
                                                    uint16_t* __restrict__ out) {
  const int p = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
  __shared__ AttendLds lds;
  __shared__ int is_last;
  attend_split(a, g, p, lds);
  drain();
  __syncthreads();
  if (tid == 0) is_last = inc_dev(&sync[g]) == (unsigned)(a.S - 1);
  __syncthreads();
  if (!is_last) return;
  if (tid == 0) st_dev(&sync[g], 0u);
  merge_head(a.state, a.S, g * kHq + (tid >> 6), (tid & 63) * 2, out);
}

__global__ __launch_bounds__(kAT) void attend_split_only(AttendArgs a) {
  __shared__ AttendLds lds;
  attend_split(a, blockIdx.y, blockIdx.x, lds);
}

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
