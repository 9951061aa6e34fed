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

constexpr int kAT = 512;                           // 8 waves
constexpr int kStateW = kD + 2;                    // {max, den, acc[128]}
constexpr float kLog2eScale = 0.12751743082459868f;  // log2(e) / sqrt(128): scores in the exp2 domain
constexpr float kSlack = 8.0f;                     // lazy-rescale threshold (log2 units)
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

constexpr int kSlotRows = 9;                 // rows per slot per round
constexpr int kWaveRows = 4 * kSlotRows;     // rows per wave per round

// LDS of one workgroup: the gather staging area of the 4 waves, reused for
// the slot merge once every wave is done with it.
constexpr int kSlots = kAT / 16;             // 32 slots of 16 lanes

struct AttendLds {
  union {
    uint4 kv[kAT / 64][2][kSlotRows][64];  // [wave][K, V][row of slot][lane] (147456 B)
    struct {
      float sm[kSlots][kHq], sz[kSlots][kHq];
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
    const unsigned long long hi = __ballot((q16 & mask) != 0);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (j < n) {
        const float keep = lane_select(hi, x[j + n], x[j]);
        const float send = lane_select(hi, x[j], x[j + n]);
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
//
// The group's row list (count[g] selected rows, then the T tail rows) is
// dealt row by row to the 8*S waves of the group's S workgroups: wave
// gw = 8p + w owns rows gw, gw + 8S, gw + 16S, ... -- every wave gets the
// same number of rows to within one.  Row positions of the list do not depend on
// count[g], so the id loads are issued together with the count load; then
// every K and V row of the round (up to 36 per wave) is gathered straight
// into the wave's LDS region with global_load_lds (16 bytes per lane, no
// registers held by loads in flight) before any is consumed.
__device__ void attend_split(const AttendArgs& a, int g, int p, AttendLds& lds) {
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int q16 = lane & 15, slot = lane >> 4;
  const int last_row = a.H + a.T - 1;
  const int nwaves = (kAT / 64) * a.S, gw = (kAT / 64) * p + w;
  const int32_t* idg = a.ids + (size_t)g * a.ids_stride;
  const uint16_t* kg = a.k + (size_t)g * a.ks + 8 * q16;
  const uint16_t* vg = a.v + (size_t)g * a.vs + 8 * q16;

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

  __attribute__((address_space(3))) void* kdst =
      (__attribute__((address_space(3))) void*)&lds.kv[w][0][0][0];
  __attribute__((address_space(3))) void* vdst =
      (__attribute__((address_space(3))) void*)&lds.kv[w][1][0][0];
  int n_old = -1, total = 0;
  for (int round = 0;; ++round) {
    // row i of this lane's slot in the round: list index j[i]
    int jr[kSlotRows], idv[kSlotRows];
#pragma unroll
    for (int i = 0; i < kSlotRows; ++i) {
      const int j = gw + nwaves * (round * kWaveRows + i * 4 + slot);
      jr[i] = j;
      idv[i] = a.H > 0 ? idg[j < a.H ? j : a.H - 1] : 0;  // speculative: meaningful only if j < count
    }
    if (n_old < 0) {
      n_old = a.cnt[g];
      n_old = n_old < 0 ? 0 : (n_old > a.H ? a.H : n_old);
      total = n_old + a.T;
    }
    if (!__ballot(jr[0] < total)) break;  // rows grow with i and round: nothing left for this wave
#pragma unroll
    for (int i = 0; i < kSlotRows; ++i) {
      const int j = jr[i];
      if (j < total) {
        int pos = j < n_old ? idv[i] : a.H + (j - n_old);
        pos = pos < 0 ? 0 : (pos > last_row ? last_row : pos);
        __builtin_amdgcn_global_load_lds(kg + (size_t)pos * kD, (char __attribute__((address_space(3)))*)kdst + i * 1024,
                                         16, 0, 0);
        __builtin_amdgcn_global_load_lds(vg + (size_t)pos * kD, (char __attribute__((address_space(3)))*)vdst + i * 1024,
                                         16, 0, 0);
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const int base = gw + nwaves * (round * kWaveRows + slot);  // list index of row i: base + 4 * nwaves * i
#pragma unroll 1
    for (int st = 0; st < (kSlotRows + 3) / 4; ++st) {
      int nv = 0;
      uint4 kr[4], vr[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int i = min(st * 4 + b, kSlotRows - 1);
        nv += (st * 4 + b < kSlotRows) && (base + 4 * nwaves * (st * 4 + b) < total);
        kr[b] = lds.kv[w][0][i][lane];
        vr[b] = lds.kv[w][1][i][lane];
      }
      if (__ballot(nv > 0)) attend_step(qf, kr, vr, nv, s);
    }
    asm volatile("" ::: "memory");  // LDS reads of this round precede the next round's gathers
  }

  // gather the slot's per-head max / denominator into every lane
  float mm[kHq], zz[kHq];
#pragma unroll
  for (int h = 0; h < kHq; ++h) {
    mm[h] = __shfl(s.m, (lane & 48) + h);
    zz[h] = __shfl(s.z, (lane & 48) + h);
  }
  __syncthreads();  // every wave is done with the staging area
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
  {
    // thread = (head tid >> 7, dim tid & 127)
    const int h = tid >> 7, d = tid & (kD - 1);
    float M = -INFINITY;
#pragma unroll
    for (int k = 0; k < kSlots; ++k) M = fmaxf(M, lds.red.sm[k][h]);
    float den = 0.f, v = 0.f;
#pragma unroll
    for (int k = 0; k < kSlots; ++k) {
      const float wgt = lds.red.sm[k][h] == -INFINITY ? 0.f : exp2f(lds.red.sm[k][h] - M);
      den = fmaf(wgt, lds.red.sz[k][h], den);
      v = fmaf(wgt, lds.red.sacc[k][h][d], v);
    }
    float* stp = a.state + (((size_t)g * kHq + h) * a.S + p) * kStateW;
    if (d == 0) st_dev2(stp, M, den);
    st_dev(stp + 2 + d, v);
  }
}

// Merges the S split states of group g into out[g] (thread = head tid >> 7,
// dim tid & 127).  Splits go in batches of 32: each thread issues its 32
// accumulator loads and each wave its 32 (max, den) loads before any is
// used, so S <= 32 costs one memory round trip.
__device__ void merge_group(const float* state, int S, int g, uint16_t* out, AttendLds& lds) {
  const int tid = threadIdx.x, h = tid >> 7, d = tid & (kD - 1), w = tid >> 6, lane = tid & 63;
  const float* st = state + (size_t)(g * kHq + h) * S * kStateW;
  float M = -INFINITY, den = 0.f, v = 0.f;
  for (int p0 = 0; p0 < S; p0 += 32) {
    const int n = min(32, S - p0);
    const float2 mz = ld_dev2(st + (size_t)(p0 + min(lane & 31, n - 1)) * kStateW);
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
    lds.wts[w][lane] = wgt;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 32; ++i) v = fmaf(lds.wts[w][i], av[i], v);
  }
  out[((size_t)g * kHq + h) * kD + d] = f32_to_bf16(den > 0.f ? v / den : 0.f);
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
  merge_group(a.state, a.S, g, out, lds);
}

__global__ __launch_bounds__(kAT) void attend_split_only(AttendArgs a) {
  __shared__ AttendLds lds;
  attend_split(a, blockIdx.y, blockIdx.x, lds);
}

// Compat merge: one workgroup per group.
__global__ __launch_bounds__(kAT) void attend_merge(const float* __restrict__ state, uint16_t* __restrict__ out,
                                                    int S) {
  __shared__ AttendLds lds;
  merge_group(state, S, blockIdx.x, out, lds);
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
  hipLaunchKernelGGL(attend_merge, dim3(8), dim3(kAT), 0, (hipStream_t)stream,
                     reinterpret_cast<const float*>(state), reinterpret_cast<uint16_t*>(out), S);
  return (int)hipGetLastError();
}

}  // extern "C"
