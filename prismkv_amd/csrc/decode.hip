// Fused routed decode of one layer: bucket selection (stages 1b), bitmap
// union (stage 2) and sparse attention (stage 3) in ONE launch after the
// moment-scoring launch of route.hip.  Same results as prismkv_route +
// prismkv_union + prismkv_attend; it exists because every kernel boundary in
// a HIP graph costs ~1.75 us on MI355X, more than most of these stages' work.
//
// Semantics: src/prismkv/core.py:106-183 (route, union, attend), the tie and
// padding rules of kernels/ppu_8b/route_parallel.cu:12,23,29 and the ascending
// emission of kernels/ppu_8b/union.cu:26.
//
// Grid (S, G) x 512, S = ceil(ceil(H/32) / 64): workgroup p of group g owns
// bitmap words [64p, 64p + 64) (tokens [2048p, 2048p + 2048)) and tail rows
// [p * ceil(T/S), ...).  Phases:
//   1. every workgroup turns the group's logits into head-summed
//      probabilities and selects the Top-16 itself (~1 us of VALU per
//      workgroup; the same bits everywhere, so all agree) -- cheaper than
//      handing candidates between workgroups; workgroup 0 writes
//      features / valid / raw;
//   2. union tile: one wave ORs the selected rows over its 64 words and
//      compacts the set bits into an LDS token list, publishing the tile's
//      count;
//   3. attention over the tile's tokens plus its tail share, 36 rows per
//      wave per round, every load of a round in flight at once;
//   4. the tile's ids go to ids[g][prefix ...], prefix = sum of the counts of
//      the lower tiles (published in phase 2, long before; lower-numbered
//      workgroups are dispatched earlier, so the bounded wait ends);
//   5. the last workgroup of the group (arrival counter) merges the S split
//      states into out[g] and clears the counters, so the launch can be
//      replayed from a graph without memset nodes.
#include <algorithm>

#include "attend_core.h"
#include "launch.h"
#include "select.h"

namespace prismkv {
namespace {

constexpr int kDT = kAT;           // 512 threads, 8 waves
constexpr int kTileWords = 64;     // bitmap words per workgroup
constexpr int kTileTokens = 32 * kTileWords;
constexpr unsigned kReady = 1u << 31;

struct DecodeArgs {
  const uint16_t* q;
  const float* logits;  // [G][4][kFP] from the scoring launch
  const float* stats;   // [G][kChunks][4][2]
  const int* counts;    // [G][kFP]
  const uint32_t* bits;
  int64_t row_words;
  const uint16_t* k;
  const uint16_t* v;
  int64_t ks, vs;
  int H, T, S, tail_per;
  unsigned* status;          // [G][S] kReady | tile count
  unsigned* sync;            // [G]
  unsigned* err;
  float* state;  // [G*4][S][130]
  int64_t* features;
  float* valid;
  int* raw;
  int32_t* ids;
  int64_t ids_stride;
  int32_t* count;
  uint16_t* out;
};

struct DecodeLds {
  int rows[kTileTokens];  // the tile's selected tokens, ascending
  alignas(16) unsigned long long win[kTop];
  int sel_rows[kTop];
  int need, nsel, base;
  int is_last;
  float gmax[kHq], grz[kHq];
  union alignas(16) {
    struct {
      alignas(16) unsigned long long keys[kDT * 6];   // 6 keys per thread
      unsigned long long best[kDT / 64 * kTop];
      unsigned long long sc[kDT / 64][64 + 16 * 6];
    } sel;
    AttendLds att;
  };
};

// Bounded spin until `pred` holds for every lane of the calling wave; sets
// the error word and gives up instead of hanging.
template <typename Pred>
__device__ __forceinline__ void wait_all(Pred pred, unsigned* err) {
  for (int spins = 0;; ++spins) {
    if (__ballot(!pred()) == 0) return;
    if (spins >= kSpinLimit) {
      if ((threadIdx.x & 63) == 0) atomicOr(err, 1u);
      return;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// Phases 1-2: the group's Top-16 (rank order) into lds.win / lds.sel_rows /
// lds.need, computed by this workgroup alone from the scoring launch's logits
// and chunk statistics: probabilities exp(l - M) / Z summed over heads in head
// order (core.py:128), keys value-descending / id-ascending.  Every
// workgroup of the group computes the same bits, so all of them agree.
constexpr int kSelKeys = (kFP + kDT - 1) / kDT;  // 6 buckets per thread

__device__ void decode_select(const DecodeArgs& a, int g, DecodeLds& lds) {
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const float* lg = a.logits + (size_t)g * kHq * kFP;
  float lv[kSelKeys][kHq];
#pragma unroll
  for (int i = 0; i < kSelKeys; ++i) {
    const int b = min(tid + kDT * i, kFP - 1);
#pragma unroll
    for (int h = 0; h < kHq; ++h) lv[i][h] = lg[h * kFP + b];
  }
  if (w < kHq) {
    // merge chunk statistics: wave h handles head h, lanes cover the 94 chunks
    const int h = w;
    const float2* st = reinterpret_cast<const float2*>(a.stats) + (size_t)g * kChunks * kHq + h;
    const float2 s0 = lane < kChunks ? st[lane * kHq] : make_float2(-INFINITY, 0.f);
    const float2 s1 = lane + 64 < kChunks ? st[(lane + 64) * kHq] : make_float2(-INFINITY, 0.f);
    const float m = wave_max(fmaxf(s0.x, s1.x));
    float z = (s0.x == -INFINITY ? 0.f : s0.y * expf(s0.x - m)) + (s1.x == -INFINITY ? 0.f : s1.y * expf(s1.x - m));
    z = wave_sum(z);
    if (lane == 0) {
      lds.gmax[h] = m;
      lds.grz[h] = z > 0.f ? 1.0f / z : 0.f;
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kSelKeys; ++i) {
    const int b = tid + kDT * i;
    uint64_t key = 0;
    if (b < kFP && lv[i][0] != -INFINITY) {
      const float p0 = expf(lv[i][0] - lds.gmax[0]) * lds.grz[0];
      const float p1 = expf(lv[i][1] - lds.gmax[1]) * lds.grz[1];
      const float p2 = expf(lv[i][2] - lds.gmax[2]) * lds.grz[2];
      const float p3 = expf(lv[i][3] - lds.gmax[3]) * lds.grz[3];
      key = make_key(((p0 + p1) + p2) + p3, b);
    }
    lds.sel.keys[w * 64 * kSelKeys + 64 * i + lane] = key;  // wave w's keys contiguous
  }
  __syncthreads();
  wave_top16<kSelKeys>(lds.sel.keys + w * 64 * kSelKeys, lds.sel.sc[w], lds.sel.best + kTop * w);
  __syncthreads();
  if (w == 0) {
    const int need = wave_top16<2>(lds.sel.best, lds.sel.sc[0], lds.win);
    if (lane < kTop) lds.sel_rows[lane] = key_bucket(lds.win[lane < need ? lane : 0]);
    if (lane == 0) lds.need = need;
  }
  __syncthreads();
}

__global__ __launch_bounds__(kDT) void decode_kernel(DecodeArgs a) {
  const int p = blockIdx.x, g = blockIdx.y, tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  __shared__ DecodeLds lds;

  // ---- 1-2. the group's Top-16, computed here
  decode_select(a, g, lds);
  if (p == 0 && w == 0)
    write_selection(lds.win, lds.need, a.counts + (size_t)g * kFP, a.features + (size_t)g * kTop,
                    a.valid + (size_t)g * kTop, a.raw + g);

  // ---- 3. union tile: OR the selected rows over words [64p, 64p + 64), compact
  const int nw = (a.H + 31) / 32;
  const int nr = lds.need;
  if (w == 0) {
    const int wd = p * kTileWords + lane;
    uint32_t m = 0;
    if (nr > 0 && wd < nw) {
      const uint32_t* gb = a.bits + (size_t)g * kF * a.row_words + wd;
      uint32_t v[kTop];
#pragma unroll
      for (int r = 0; r < kTop; ++r) v[r] = __builtin_nontemporal_load(gb + (size_t)lds.sel_rows[r < nr ? r : nr - 1] * a.row_words);
#pragma unroll
      for (int r = 0; r < kTop; ++r) m |= v[r];
      if (wd == nw - 1 && (a.H & 31)) m &= (1u << (a.H & 31)) - 1u;
    }
    const int n = __popc(m);
    const int incl = wave_scan_i(n);
    int at = incl - n;
    while (m) {
      lds.rows[at++] = wd * 32 + (int)__builtin_ctz(m);
      m &= m - 1u;
    }
    const int total = __shfl(incl, 63);
    if (lane == 0) {
      lds.nsel = total;
      st_dev(&a.status[(size_t)g * a.S + p], kReady | (unsigned)total);
    }
  }
  __syncthreads();

  // ---- 4. attention over the tile's tokens, then its tail rows
  const int n_sel = lds.nsel;
  const int t_lo = min(a.T, p * a.tail_per), t_hi = min(a.T, t_lo + a.tail_per);
  const int n_rows = n_sel + (t_hi - t_lo);
  {
    const int q16 = lane & 15, slot = lane >> 4;
    const int last_row = a.H + a.T - 1;
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
    // row r of the workgroup's list: wave w takes r = w + 8 (36 round + 4 i + slot)
    for (int round = 0; round * (kDT / 64) * kWaveRows < n_rows; ++round) {
      const int base = w + (kDT / 64) * (round * kWaveRows + slot);
      uint4 kr[kSlotRows], vr[kSlotRows];
#pragma unroll
      for (int i = 0; i < kSlotRows; ++i) {
        const int r = base + (kDT / 64) * 4 * i;
        int pos = 0;
        if (r < n_sel) pos = lds.rows[r];
        else if (r < n_rows) pos = a.H + t_lo + (r - n_sel);
        pos = pos < 0 ? 0 : (pos > last_row ? last_row : pos);
        kr[i] = load_nt16(kg + (size_t)pos * kD);
        vr[i] = load_nt16(vg + (size_t)pos * kD);
        if ((i & 3) == 3) asm volatile("" ::: "memory");  // issue the rows step by step, in order
      }
#pragma unroll
      for (int st = 0; st < (kSlotRows + 3) / 4; ++st) {
        int nv = 0;
        uint4 ks[4], vs[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const int i = st * 4 + b;
          nv += (i < kSlotRows) && (base + (kDT / 64) * 4 * i < n_rows);
          ks[b] = kr[i < kSlotRows ? i : kSlotRows - 1];
          vs[b] = vr[i < kSlotRows ? i : kSlotRows - 1];
        }
        if (__ballot(nv > 0)) attend_step(qf, ks, vs, nv, s);
      }
    }
    store_wg_state(s, lds.att, a.state + ((size_t)g * kHq * a.S + p) * kStateW, (size_t)a.S * kStateW);
  }

  // ---- 5. the tile's ids at their global offset
  if (w == 0) {
    const unsigned* st = a.status + (size_t)g * a.S;
    unsigned prefix = 0;
    for (int c0 = 0; c0 < p; c0 += 64) {
      const int qq = c0 + lane;
      wait_all([&] { return qq >= p || (ld_dev(st + qq) & kReady) != 0u; }, a.err);
      prefix += (unsigned)wave_sum_i(qq < p ? (int)(ld_dev(st + qq) & ~kReady) : 0);
    }
    if (lane == 0) {
      lds.base = (int)prefix;
      if (p == a.S - 1) a.count[g] = (int32_t)(prefix + (unsigned)n_sel);
    }
  }
  __syncthreads();
  {
    int32_t* dst = a.ids + (size_t)g * a.ids_stride + lds.base;
    for (int i = tid; i < n_sel; i += kDT) dst[i] = lds.rows[i];
  }

  // ---- 6. arrival; the last workgroup merges and resets
  drain();
  __syncthreads();
  if (tid == 0) lds.is_last = inc_dev(&a.sync[g]) == (unsigned)(a.S - 1);
  __syncthreads();
  if (!lds.is_last) return;
  for (int i = tid; i < a.S; i += kDT) st_dev(&a.status[(size_t)g * a.S + i], 0u);
  if (tid == 0) st_dev(&a.sync[g], 0u);
  merge_group(a.state, a.S, g, a.out, lds.att);
}

}  // namespace
}  // namespace prismkv

using namespace prismkv;

static int decode_tiles(int H) { return std::max(1, ((H + 31) / 32 + kTileWords - 1) / kTileWords); }

// Work layout (bytes): route logits | route stats | status | sync | err | state
struct DecodeWorkLayout {
  size_t logits, stats, status, sync, err, state, total;
  DecodeWorkLayout(int groups, int S) {
    size_t o = 0;
    auto take = [&](size_t n) { const size_t at = o; o += (n + 255) & ~(size_t)255; return at; };
    logits = take((size_t)groups * kHq * kFP * sizeof(float));
    stats = take((size_t)groups * kChunks * kHq * 2 * sizeof(float));
    status = take((size_t)groups * S * sizeof(unsigned));
    sync = take((size_t)groups * sizeof(unsigned));
    err = take(sizeof(unsigned));
    state = take((size_t)groups * kHq * S * kStateW * sizeof(float));
    total = o;
  }
};

extern "C" {

size_t prismkv_decode_work_bytes(int groups, int capacity) {
  if (groups < 1 || capacity < 1) return 0;
  return DecodeWorkLayout(groups, decode_tiles(capacity)).total;
}

int prismkv_decode_score(uint64_t q, uint64_t moments, uint64_t counts, uint64_t work, int groups, int capacity,
                         uint64_t stream) {
  if (groups < 1 || groups > 65535 || capacity < 1) return kBadSize;
  if (!q || !moments || !counts || !work) return kBadSize;
  const DecodeWorkLayout L(groups, decode_tiles(capacity));
  char* w = reinterpret_cast<char*>(work);
  launch_route_score(reinterpret_cast<const uint16_t*>(q), reinterpret_cast<const float*>(moments),
                     reinterpret_cast<const int*>(counts), reinterpret_cast<float*>(w + L.logits),
                     reinterpret_cast<float*>(w + L.stats), groups, (hipStream_t)stream);
  return (int)hipGetLastError();
}

int prismkv_decode_attend(uint64_t q, uint64_t counts, uint64_t bits, uint64_t k, uint64_t v, uint64_t work,
                          uint64_t features, uint64_t valid, uint64_t raw, uint64_t ids, uint64_t count, uint64_t out,
                          int groups, int H, int T, int capacity, int64_t row_words, int64_t ks, int64_t vs,
                          int64_t ids_stride, uint64_t stream) {
  if (groups < 1 || groups > 65535 || H < 1 || T < 0 || capacity < H) return kBadSize;
  if (row_words < (H + 31) / 32 || ids_stride < H) return kBadSize;
  if (ks < (int64_t)(H + T) * kD || vs < (int64_t)(H + T) * kD) return kBadSize;
  if (!q || !counts || !bits || !k || !v || !work || !features || !valid || !raw || !ids || !count || !out)
    return kBadSize;
  const int S = decode_tiles(H);
  const DecodeWorkLayout L(groups, decode_tiles(capacity));
  char* w = reinterpret_cast<char*>(work);
  DecodeArgs a;
  a.q = reinterpret_cast<const uint16_t*>(q);
  a.logits = reinterpret_cast<const float*>(w + L.logits);
  a.stats = reinterpret_cast<const float*>(w + L.stats);
  a.counts = reinterpret_cast<const int*>(counts);
  a.bits = reinterpret_cast<const uint32_t*>(bits);
  a.row_words = row_words;
  a.k = reinterpret_cast<const uint16_t*>(k);
  a.v = reinterpret_cast<const uint16_t*>(v);
  a.ks = ks;
  a.vs = vs;
  a.H = H;
  a.T = T;
  a.S = S;
  a.tail_per = (T + S - 1) / S;
  a.status = reinterpret_cast<unsigned*>(w + L.status);
  a.sync = reinterpret_cast<unsigned*>(w + L.sync);
  a.err = reinterpret_cast<unsigned*>(w + L.err);
  a.state = reinterpret_cast<float*>(w + L.state);
  a.features = reinterpret_cast<int64_t*>(features);
  a.valid = reinterpret_cast<float*>(valid);
  a.raw = reinterpret_cast<int*>(raw);
  a.ids = reinterpret_cast<int32_t*>(ids);
  a.ids_stride = ids_stride;
  a.count = reinterpret_cast<int32_t*>(count);
  a.out = reinterpret_cast<uint16_t*>(out);
  hipLaunchKernelGGL(decode_kernel, dim3(S, groups), dim3(kDT), 0, (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

int prismkv_decode(uint64_t q, uint64_t moments, uint64_t counts, uint64_t bits, uint64_t k, uint64_t v,
                   uint64_t work, uint64_t features, uint64_t valid, uint64_t raw, uint64_t ids, uint64_t count,
                   uint64_t out, int groups, int H, int T, int capacity, int64_t row_words, int64_t ks, int64_t vs,
                   int64_t ids_stride, uint64_t stream) {
  if (groups < 1 || groups > 65535 || H < 1 || T < 0 || capacity < H) return kBadSize;
  if (row_words < (H + 31) / 32 || ids_stride < H) return kBadSize;
  if (ks < (int64_t)(H + T) * kD || vs < (int64_t)(H + T) * kD) return kBadSize;
  if (!moments) return kBadSize;
  const int rc = prismkv_decode_score(q, moments, counts, work, groups, capacity, stream);
  if (rc) return rc;
  return prismkv_decode_attend(q, counts, bits, k, v, work, features, valid, raw, ids, count, out, groups, H, T,
                               capacity, row_words, ks, vs, ids_stride, stream);
}

}  // extern "C"
