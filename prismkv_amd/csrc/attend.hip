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
//
// prismkv_attend_f32 runs the same kernel on fp32 q / K / V (fp32 output):
// each lane's 8 dims of a row are two 16-byte loads, and a slot takes 5 rows
// per round instead of 9 so the rows in flight fit the same registers.
#include "attend_core.h"

namespace prismkv {
namespace {

// Computes this workgroup's split state and writes it to a.state.
//
// The group's row list (count[g] selected rows, then the T tail rows) is
// dealt row by row to the 8*S waves of the group's S workgroups: wave
// gw = 8p + w owns rows gw, gw + 8S, gw + 16S, ... -- every wave gets the
// same number of rows to within one.  Row positions of the list do not depend on
// count[g], so the id loads are issued together with the count load; then
// every K and V row of the round (up to 36 per wave, 16 bytes per lane per
// row) is requested before any is consumed.
template <typename E>
__device__ void attend_split(const AttendArgs<E>& a, int g, int p, AttendLds& lds) {
  typedef Row8<E> RL;
  constexpr int kRows = sizeof(E) == 2 ? kSlotRows : 5;  // rows per slot per round
  constexpr int kRoundRows = 4 * kRows;                  // rows per wave per round
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int q16 = lane & 15, slot = lane >> 4;
  const int last_row = a.H + a.T - 1;
  const int nwaves = (kAT / 64) * a.S, gw = (kAT / 64) * p + w;
  const int32_t* idg = a.ids + (size_t)g * a.ids_stride;
  const E* kg = a.k + (size_t)g * a.ks + 8 * q16;
  const E* vg = a.v + (size_t)g * a.vs + 8 * q16;

  float qf[kHq][8];
#pragma unroll
  for (int h = 0; h < kHq; ++h) {
    unpack8(RL::load(a.q + ((size_t)g * kHq + h) * kD + 8 * q16), qf[h]);
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

  int n_old = -1, total = 0;
  bool bad = false;  // an id outside [0, H) or a count outside [0, H]
  for (int round = 0;; ++round) {
    // row i of this lane's slot in the round: list index j[i]
    int jr[kRows], idv[kRows];
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      const int j = gw + nwaves * (round * kRoundRows + i * 4 + slot);
      jr[i] = j;
      idv[i] = a.H > 0 ? idg[j < a.H ? j : a.H - 1] : 0;  // speculative: meaningful only if j < count
    }
    if (n_old < 0) {
      const int given = a.cnt[g];
      n_old = given < 0 ? 0 : (given > a.H ? a.H : given);
      bad = given != n_old;
      total = n_old + a.T;
    }
    if (!__ballot(jr[0] < total)) break;  // rows grow with i and round: nothing left for this wave
    // every lane issues all 2 * kRows gathers at once (rows past the end
    // re-read row 0 and are masked); the compiler waits per load, so step st
    // computes as soon as its own rows have landed, while later rows fly
    typename RL::Raw kr[kRows], vr[kRows];
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
      const int j = jr[i];
      const int p = j < n_old ? idv[i] : a.H + (j - n_old);
      bad |= j < n_old && (p < 0 || p >= a.H);
      const int pos = (j < total && p >= 0) ? (p > last_row ? last_row : p) : 0;
      kr[i] = RL::load(kg + (size_t)pos * kD);
      vr[i] = RL::load(vg + (size_t)pos * kD);
      if ((i & 3) == 3) asm volatile("" ::: "memory");  // issue the rows step by step, in order
    }
    const int base = gw + nwaves * (round * kRoundRows + slot);  // list index of row i: base + 4 * nwaves * i
#pragma unroll
    for (int st = 0; st < (kRows + 3) / 4; ++st) {
      int nv = 0;
      typename RL::Raw ks[4], vs[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int i = st * 4 + b;
        nv += (i < kRows) && (base + 4 * nwaves * i < total);
        ks[b] = kr[i < kRows ? i : kRows - 1];
        vs[b] = vr[i < kRows ? i : kRows - 1];
      }
      if (__ballot(nv > 0)) attend_step(qf, ks, vs, nv, s);
    }
    asm volatile("" ::: "memory");  // LDS reads of this round precede the next round's gathers
  }

  if (a.err && __ballot(bad) && lane == 0) report_error(a.err, error_host_slot(a.err), kErrIds);
  store_wg_state(s, lds, a.state + (((size_t)g * kHq) * a.S + p) * kStateW, (size_t)a.S * kStateW);
}

template <typename E>
__global__ __launch_bounds__(kAT) void attend_fused(AttendArgs<E> a, unsigned* __restrict__ sync, E* __restrict__ out) {
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
  merge_group(a.state, a.S, g, out, lds.wts);
}

__global__ __launch_bounds__(kAT) void attend_split_only(AttendArgs<uint16_t> a) {
  __shared__ AttendLds lds;
  attend_split(a, blockIdx.y, blockIdx.x, lds);
}

// Compat merge: one workgroup per group.
__global__ __launch_bounds__(kAT) void attend_merge(const float* __restrict__ state, uint16_t* __restrict__ out,
                                                    int S) {
  __shared__ AttendLds lds;
  merge_group(state, S, blockIdx.x, out, lds.wts);
}

}  // namespace
}  // namespace prismkv

using namespace prismkv;

extern "C" size_t prismkv_attend_work_bytes(int groups, int splits);

// The split kernel with the last-arriving workgroup's merge over the work's
// split states (after the decode-phase region, whose error word comes first).
template <typename E>
static int attend_split_launch(uint64_t q, uint64_t k, uint64_t v, uint64_t ids, uint64_t count, uint64_t work,
                               uint64_t out, int groups, int H, int T, int64_t ks, int64_t vs, int64_t ids_stride,
                               int splits, uint64_t stream) {
  float* state = reinterpret_cast<float*>(reinterpret_cast<char*>(work) + attend_list_work_bytes(groups));
  AttendArgs<E> a{reinterpret_cast<const E*>(q), reinterpret_cast<const E*>(k), reinterpret_cast<const E*>(v),
                  reinterpret_cast<const int32_t*>(ids), reinterpret_cast<const int32_t*>(count), ks, vs, ids_stride,
                  H, T, splits, state};
  a.err = reinterpret_cast<unsigned*>(work);
  unsigned* sync = reinterpret_cast<unsigned*>(state + (size_t)groups * kHq * splits * kStateW);
  hipLaunchKernelGGL(attend_fused<E>, dim3(splits, groups), dim3(kAT), 0, (hipStream_t)stream, a, sync,
                     reinterpret_cast<E*>(out));
  return (int)hipGetLastError();
}

extern "C" {

// Work: the decode-phase region (attend_list_work_bytes: its error word
// first), then this file's split states and arrival counters, disjoint, so
// either launch finds its region as it left it.
size_t prismkv_attend_work_bytes(int groups, int splits) {
  if (groups < 1 || splits < 1) return 0;
  return attend_list_work_bytes(groups) + (size_t)groups * kHq * splits * kStateW * sizeof(float) +
         (size_t)groups * sizeof(unsigned);
}

int prismkv_attend(uint64_t q, uint64_t k, uint64_t v, uint64_t ids, uint64_t count, uint64_t work, uint64_t out,
                   int groups, int H, int T, int64_t ks, int64_t vs, int64_t ids_stride, int splits,
                   size_t work_bytes, uint64_t stream) {
  if (groups < 1 || groups > 65535 || H < 0 || T < 0 || splits < 1 || splits > 1024) return kBadSize;
  if (ks < (int64_t)(H + T) * kD || vs < (int64_t)(H + T) * kD || ids_stride < H) return kBadSize;
  if (!q || !k || !v || !ids || !count || !work || !out) return kBadSize;
  if (work_bytes < prismkv_attend_work_bytes(groups, splits)) return kBadSize;
  // the decode's attention phases when the lists fit them; the split count
  // does not change the result (exact softmax), only the partition
  const int rc = attend_list(q, k, v, ids, count, work, out, groups, H, T, ks, vs, ids_stride, stream);
  if (rc != kBadSize) return rc;
  return attend_split_launch<uint16_t>(q, k, v, ids, count, work, out, groups, H, T, ks, vs, ids_stride, splits,
                                      stream);
}

// fp32 q / K / V rows and fp32 output; the same work layout (error word first).
int prismkv_attend_f32(uint64_t q, uint64_t k, uint64_t v, uint64_t ids, uint64_t count, uint64_t work, uint64_t out,
                       int groups, int H, int T, int64_t ks, int64_t vs, int64_t ids_stride, int splits,
                       size_t work_bytes, uint64_t stream) {
  if (groups < 1 || groups > 65535 || H < 0 || T < 0 || splits < 1 || splits > 1024) return kBadSize;
  if (ks < (int64_t)(H + T) * kD || vs < (int64_t)(H + T) * kD || ids_stride < H) return kBadSize;
  if (!q || !k || !v || !ids || !count || !work || !out || ((q | k | v | (uint64_t)(ks | vs) * 4) & 15u))
    return kBadSize;
  if (work_bytes < prismkv_attend_work_bytes(groups, splits)) return kBadSize;
  return attend_split_launch<float>(q, k, v, ids, count, work, out, groups, H, T, ks, vs, ids_stride, splits, stream);
}

// kernels/ppu_8b/av_tuned.cu:62-67 contract; state is the caller's
// f32 [32][128][130] buffer, used as [(g*4+h)*S + p][130].
int attention_tuned(uint64_t q, uint64_t k, uint64_t v, uint64_t ids, uint64_t cnt, uint64_t state, uint64_t out,
                    int H, int T, int KS, int VS, int S, int mode, uint64_t stream) {
  if (S < 1 || S > 128 || H < 1 || T < 0 || KS < (H + T) * kD || VS < (H + T) * kD) return kBadSize;
  if (mode < 0 || mode > 2) return kBadMode;
  AttendArgs<uint16_t> a{reinterpret_cast<const uint16_t*>(q), reinterpret_cast<const uint16_t*>(k),
                         reinterpret_cast<const uint16_t*>(v), reinterpret_cast<const int32_t*>(ids),
                         reinterpret_cast<const int32_t*>(cnt), KS, VS, H, H, T, S, reinterpret_cast<float*>(state)};
  hipLaunchKernelGGL(attend_split_only, dim3(S, 8), dim3(kAT), 0, (hipStream_t)stream, a);
  hipLaunchKernelGGL(attend_merge, dim3(8), dim3(kAT), 0, (hipStream_t)stream,
                     reinterpret_cast<const float*>(state), reinterpret_cast<uint16_t*>(out), S);
  return (int)hipGetLastError();
}

}  // extern "C"
