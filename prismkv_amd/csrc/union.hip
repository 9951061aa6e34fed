// Stage 2 -- union: OR the membership bitmap rows of the selected buckets and
// compact the set bits into an ascending token-ID list.  Also the bitmap
// build (CSR lists -> bits) used at index construction.
//
// Semantics: kernels/ppu_8b/union.cu:14-27 (OR of rows with valid > 0,
//            ascending emission of w*32+bit), kernels/ppu_8b/pack.cu:5 (bit
//            order: token t <-> word t>>5, bit t&31), src/prismkv/core.py:142-167.
//
// Design: one launch.  Workgroup (tile, group) ORs the selected rows over its
// 256 x WPT words.  Rows are padded to 16 by repeating the last selected row
// (OR is idempotent), so every thread issues 16 independent vector loads at
// once.  The tile's output offset comes from a decoupled look-back in which
// one wave inspects up to 64 predecessor status words per round in parallel;
// tiles only wait on lower-numbered tiles of the same group, which the
// in-order dispatcher has already started, and every wait is bounded (it
// reports through an error word instead of hanging).  The last tile to finish
// restores the status words to zero, so the launch is replayable from a graph
// without memset nodes.
#include "common.h"

namespace prismkv {
namespace {

constexpr int kUT = 256;                 // union workgroup size
constexpr unsigned kFlagAgg = 1u << 30;  // status: tile aggregate available
constexpr unsigned kFlagInc = 2u << 30;  // status: inclusive prefix available
constexpr unsigned kValMask = (1u << 30) - 1;

struct UnionWork {
  unsigned* status;  // [groups][tiles]
  unsigned* done;    // [groups]
  unsigned* err;     // [1] sticky error word; its host-word slot at byte 8
  int spin;          // bound of every wait (sleeps)
};

__host__ __device__ inline int union_tiles(int H, int wpt) {
  const int nw = (H + 31) / 32;
  const int tw = kUT * wpt;
  return (nw + tw - 1) / tw;
}

template <int WPT>
struct Words;
template <>
struct Words<1> {
  static __device__ __forceinline__ void load(const uint32_t* p, uint32_t* m) { m[0] = __builtin_nontemporal_load(p); }
};
template <>
struct Words<2> {
  static __device__ __forceinline__ void load(const uint32_t* p, uint32_t* m) {
    typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
    m[0] = v.x;
    m[1] = v.y;
  }
};
template <>
struct Words<4> {
  static __device__ __forceinline__ void load(const uint32_t* p, uint32_t* m) {
    const uint4 v = load_nt16(p);
    m[0] = v.x; m[1] = v.y; m[2] = v.z; m[3] = v.w;
  }
};

// Exclusive prefix of tile t of a group by decoupled look-back (run by wave 0).
// Returns the prefix; publishes the inclusive status of tile t.
__device__ unsigned look_back(unsigned* st, int t, unsigned total, const UnionWork& work) {
  const int lane = threadIdx.x & 63;
  if (t == 0) {
    if (lane == 0) st_dev(&st[0], kFlagInc | total);
    return 0;
  }
  if (lane == 0) st_dev(&st[t], kFlagAgg | total);
  unsigned prefix = 0;
  int end = t;  // window: tiles end-64 .. end-1, lane i looks at tile end-1-i
  for (;;) {
    const int p = end - 1 - lane;
    unsigned s = p >= 0 ? ld_dev(&st[p]) : (kFlagInc | 0u);
    for (int spins = 0;; ++spins) {
      if (!__ballot((s >> 30) == 0)) break;
      if (spins >= work.spin) {  // a predecessor never published: report, do not hang
        if (lane == 0) report_error(work.err, error_host_slot(work.err));
        s = kFlagInc | 0u;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
      if ((s >> 30) == 0) s = ld_dev(&st[p]);
    }
    const unsigned long long inc = __ballot((s >> 30) == 2u);
    if (inc) {
      const int first = __ffsll((long long)inc) - 1;  // nearest predecessor with an inclusive prefix
      prefix += (unsigned)wave_sum_i(lane <= first ? (int)(s & kValMask) : 0);
      break;
    }
    prefix += (unsigned)wave_sum_i((int)(s & kValMask));
    end -= 64;
  }
  if (lane == 0) st_dev(&st[t], kFlagInc | ((prefix + total) & kValMask));
  return prefix;
}

template <int WPT, int kSel>
__global__ __launch_bounds__(kUT) void union_kernel(const uint32_t* __restrict__ bits, int64_t row_words,
                                                    const int64_t* __restrict__ features,
                                                    const float* __restrict__ valid, int32_t* __restrict__ ids,
                                                    int64_t ids_stride, int32_t* __restrict__ count, UnionWork work,
                                                    int H, int tiles) {
  static_assert(kSel % kTop == 0 && kSel <= 64, "selections of up to 64 rows, 16 at a time");
  const int t = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
  __shared__ int rows[kSel];
  __shared__ int nrows;
  __shared__ unsigned wsum[kUT / 64];
  __shared__ unsigned base;
  __shared__ int last;
  if (tid < 64) {
    // wave 0 compacts the valid, in-range selections (an out-of-range id selects nothing)
    bool ok = false;
    int f = 0;
    if (tid < kSel) {
      // both requested at once (not the id only where valid holds)
      const float vl = valid[(size_t)g * kSel + tid];
      const int64_t fe = features[(size_t)g * kSel + tid];
      ok = vl > 0.f && fe >= 0 && fe < kF;
      f = (int)fe;
    }
    const unsigned long long m = __ballot(ok);
    if (ok) rows[__popcll(m & ((1ull << tid) - 1))] = f;
    if (tid == 0) nrows = __popcll(m);
  }
  __syncthreads();
  const int nr = nrows;
  const int nw = (H + 31) / 32;
  const int w0 = (t * kUT + tid) * WPT;
  uint32_t m[WPT];
#pragma unroll
  for (int i = 0; i < WPT; ++i) m[i] = 0;
  const uint32_t* gb = bits + (size_t)g * kF * row_words;
  if (nr > 0) {
    if (w0 + WPT <= nw) {
      // 16 rows at a time, all loads of a round issued together (rows past nr
      // repeat the last selected one: OR is idempotent)
      for (int r0 = 0; r0 < nr; r0 += kTop) {  // uniform
        uint32_t v[kTop][WPT];
#pragma unroll
        for (int r = 0; r < kTop; ++r)
          Words<WPT>::load(gb + (size_t)rows[r0 + r < nr ? r0 + r : nr - 1] * row_words + w0, v[r]);
#pragma unroll
        for (int r = 0; r < kTop; ++r)
#pragma unroll
          for (int i = 0; i < WPT; ++i) m[i] |= v[r][i];
      }
    } else {
      for (int r = 0; r < nr; ++r) {
        const uint32_t* src = gb + (size_t)rows[r] * row_words;
#pragma unroll
        for (int i = 0; i < WPT; ++i)
          if (w0 + i < nw) m[i] |= src[w0 + i];
      }
    }
  }
  // tokens at or beyond H are never members; clear them defensively
#pragma unroll
  for (int i = 0; i < WPT; ++i) {
    const int w = w0 + i;
    if (w >= nw) m[i] = 0;
    else if (w == nw - 1 && (H & 31)) m[i] &= (1u << (H & 31)) - 1u;
  }
  unsigned n = 0;
#pragma unroll
  for (int i = 0; i < WPT; ++i) n += __popc(m[i]);
  const unsigned incl = block_incl_scan<kUT>(n, wsum);  // wsum[3] = tile total afterwards
  const unsigned excl = incl - n;
  unsigned* st = work.status + (size_t)g * tiles;
  if (tid < 64) {
    const unsigned total = wsum[0] + wsum[1] + wsum[2] + wsum[3];
    const unsigned prefix = look_back(st, t, total, work);
    if (tid == 0) {
      base = prefix;
      if (t == tiles - 1) count[g] = (int32_t)(prefix + total);
    }
  }
  __syncthreads();
  int at = (int)(base + excl);
  int32_t* out = ids + (size_t)g * ids_stride;
#pragma unroll
  for (int i = 0; i < WPT; ++i) {
    uint32_t v = m[i];
    const int wb = (w0 + i) * 32;
    while (v) {
      out[at++] = wb + (int)__builtin_ctz(v);
      v &= v - 1u;
    }
  }
  // the last tile of the group to get here clears the status words for reuse
  if (tid == 0) last = inc_dev(&work.done[g]) == (unsigned)(tiles - 1);
  __syncthreads();
  if (last) {
    for (int i = tid; i < tiles; i += kUT) st_dev(&st[i], 0u);
    if (tid == 0) st_dev(&work.done[g], 0u);
  }
}

// Compat two-pass union (kernels/ppu_8b/union.cu:14-27 contract): pass 1 ORs
// and counts 128-word tiles into the caller's mask/tiles scratch, pass 2 sums
// the preceding tile counts and emits.  Used by launch_union_warp only.
constexpr int kCT = 128;

__global__ __launch_bounds__(kCT) void compat_count(const uint32_t* __restrict__ bits,
                                                    const int64_t* __restrict__ ids,
                                                    const float* __restrict__ vals, uint32_t* __restrict__ mask,
                                                    int* __restrict__ tiles, int nw, int nb) {
  const int u = blockIdx.y, tid = threadIdx.x, w = blockIdx.x * kCT + tid;
  __shared__ unsigned wsum[kCT / 64];
  uint32_t v = 0;
  if (w < nw) {
    for (int j = 0; j < kTop; ++j) {
      const int64_t f = ids[u * kTop + j];
      if (vals[u * kTop + j] > 0.f && f >= 0 && f < kF) v |= bits[((size_t)u * kF + f) * nw + w];
    }
    mask[(size_t)u * nw + w] = v;
  }
  const unsigned incl = block_incl_scan<kCT>(__popc(v), wsum);
  if (tid == kCT - 1) tiles[u * nb + blockIdx.x] = (int)incl;
}

__global__ __launch_bounds__(kCT) void compat_extract(const uint32_t* __restrict__ mask,
                                                      const int* __restrict__ tiles, int* __restrict__ selected,
                                                      int* __restrict__ counts, int H, int nw, int nb) {
  const int u = blockIdx.y, tid = threadIdx.x, w = blockIdx.x * kCT + tid;
  __shared__ unsigned wsum[kCT / 64];
  __shared__ int base;
  uint32_t v = w < nw ? mask[(size_t)u * nw + w] : 0u;
  if (w == nw - 1 && (H & 31)) v &= (1u << (H & 31)) - 1u;
  const unsigned n = __popc(v);
  const unsigned incl = block_incl_scan<kCT>(n, wsum);
  if (tid == 0) {
    int s = 0;
    for (int j = 0; j < (int)blockIdx.x; ++j) s += tiles[u * nb + j];
    base = s;
    if ((int)blockIdx.x == nb - 1) counts[u] = s + tiles[u * nb + blockIdx.x];
  }
  __syncthreads();
  int at = base + (int)(incl - n);
  while (v) {
    selected[(size_t)u * H + at++] = w * 32 + (int)__builtin_ctz(v);
    v &= v - 1u;
  }
}

// Bitmap build from CSR lists (kernels/ppu_8b/pack.cu:5-6 contract):
// bits[(g*F + f)*row_words + t/32] |= 1 << (t%32) for each member t of f.
__global__ __launch_bounds__(256) void bits_kernel(const int* __restrict__ ids, const int* __restrict__ offsets,
                                                   uint32_t* __restrict__ bits, int64_t cap, int64_t row_words) {
  const int g = blockIdx.y, f = blockIdx.x;
  const int lo = offsets[(size_t)g * (kF + 1) + f], hi = offsets[(size_t)g * (kF + 1) + f + 1];
  uint32_t* row = bits + ((size_t)g * kF + f) * row_words;
  for (int j = lo + (int)threadIdx.x; j < hi; j += 256) {
    const int t = ids[(size_t)g * cap + j];
    atomicOr(row + (t >> 5), 1u << (t & 31));
  }
}

// Strict unique-ID budget (src/prismkv/core.py:149-163): walk the ranked
// buckets (rows with valid > 0, in rank order) and accept a bucket only if
// the tokens it adds to the running union keep the union within `limit`;
// a bucket that would overflow is skipped and the walk continues.  Rewrites
// features / valid / raw with the accepted buckets compacted to the front in
// rank order (unused slots id 0, valid 0), which the union then consumes.

// Raw buffer loads (gfx9 resource word 3: 32-bit data format) with the
// non-temporal hint.
constexpr int kRawBufferWord3 = 0x00020000;
constexpr int kLoadNonTemporal = 2;
template <int V>
__device__ __forceinline__ void load_run(__amdgpu_buffer_rsrc_t r, unsigned byte_offset, uint32_t* m);
template <>
__device__ __forceinline__ void load_run<1>(__amdgpu_buffer_rsrc_t r, unsigned byte_offset, uint32_t* m) {
  m[0] = __builtin_amdgcn_raw_buffer_load_b32(r, byte_offset, 0, kLoadNonTemporal);
}
template <>
__device__ __forceinline__ void load_run<4>(__amdgpu_buffer_rsrc_t r, unsigned byte_offset, uint32_t* m) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_offset, 0, kLoadNonTemporal);
  m[0] = v.x; m[1] = v.y; m[2] = v.z; m[3] = v.w;
}

// Row register sets of the walk: an even number of rows, as many as the load
// counter (63 loads in flight) and about 128 registers hold, at most 16.
constexpr int cap_row_sets(int loads_per_row, int words_per_row) {
  int sets = 63 / loads_per_row;
  if (128 / words_per_row < sets) sets = 128 / words_per_row;
  return (sets < 16 ? sets : 16) & ~1;
}

// Workgroups past the groups' walkers pull the selected rows into L2 so
// that the walker's loads hit there: workgroup b >= groups serves group
// b % groups (with groups a multiple of 8, the walker's XCD under the
// round-robin dispatch) and touches one word per 64 bytes of its part of
// every selected row.  It reads the selection the walker rewrites at its
// end; a helper that starts that late only touches other rows.
template <int kSel>
__device__ void touch_rows(const uint32_t* bits, int64_t row_words, const int64_t* features, const float* valid,
                           int g, int part, int parts, int nw) {
  const int lines = (nw + 15) >> 4, per = (lines + parts - 1) / parts;
  const int lo = part * per, hi = lo + per < lines ? lo + per : lines;
  const uint32_t* bg = bits + (size_t)g * kF * row_words;
  unsigned acc = 0;
  for (int j = 0; j < kSel; ++j) {
    const int64_t f = features[(size_t)g * kSel + j];
    if (!(valid[(size_t)g * kSel + j] > 0.f && f >= 0 && f < kF)) continue;
    const uint32_t* row = bg + (size_t)f * row_words;
    for (int l = lo + (int)threadIdx.x; l < hi; l += blockDim.x) acc ^= row[16 * l];
  }
  asm volatile("" ::"v"(acc));  // keeps the loads
}

// The budgeted walk, one workgroup of kCapT threads per group (workgroups
// past `groups` are row-touching helpers).  Thread tid owns runs of V
// consecutive words, V (tid + kCapT u) .. + V - 1 for u < R, of every row
// (V = 4: one 16-byte load per run), and keeps its slice of the running
// union U in registers.  Decisions go in pairs, one block-wide reduction per
// pair: for ranked rows a, b with x = a \ U and y = b \ U the block sums
// |x|, |y \ x| and |y ∩ x|; a is kept when total + |x| fits the limit, and b
// when its size over the union as it then stands, |y \ x| if a was kept and
// |y \ x| + |y ∩ x| if not, fits what is left -- the decisions of the
// one-bucket-at-a-time walk.
// Loads: every wave holds the selection in a register (lane j: ranked
// bucket j), so a row's address is one lane read.  Each pair step requests
// the rows kSets - 2 ranks ahead into register sets that rotate by name (a
// copy would wait for the load), through a buffer resource whose range is
// empty past the selection (such loads return 0 without a memory request).
// kSets R loads in flight stay within the 63 that a wave's load counter
// tracks, so the wait for a pair's rows is exact.
template <int kCapT, int V, int R, int kSel>
__global__ __launch_bounds__(kCapT) void cap_kernel(const uint32_t* __restrict__ bits, int64_t row_words,
                                                    const int* __restrict__ counts, int64_t* features, float* valid,
                                                    int* raw, int H, long long limit, int groups) {
  constexpr int WPT = V * R;
  if ((int)blockIdx.x >= groups) {
    touch_rows<kSel>(bits, row_words, features, valid, blockIdx.x % groups, blockIdx.x / groups - 1,
                     gridDim.x / groups - 1, (H + 31) >> 5);
    return;
  }
  const int g = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  __shared__ int sel[kSel], nsel_s;
  __shared__ u32x4 part[2][kCapT / 64];  // per wave and pair: |x|, |y \ x|, |y ∩ x|
  // wave 0, lane j < kSel: ranked entry j, its rank among the valid ones and its size
  bool ok = false;
  int at = 0, cnt = 0;
  if (w == 0) {
    // the valid, in-range selections in rank order (an out-of-range id selects nothing)
    const int j = lane < kSel ? lane : kSel - 1;
    const int64_t fe = features[(size_t)g * kSel + j];
    const float va = valid[(size_t)g * kSel + j];
    ok = lane < kSel && va > 0.f && fe >= 0 && fe < kF;
    const int f = ok ? (int)fe : 0;
    cnt = counts[(size_t)g * kFP + f];  // used after the walk
    const unsigned long long m = __ballot(ok);
    at = __popcll(m & ((1ull << lane) - 1ull));
    if (ok) sel[at] = f;
    if (lane == 0) nsel_s = __popcll(m);
  }
  __syncthreads();
  const int n = __builtin_amdgcn_readfirstlane(nsel_s);  // uniform: the row resources live in scalars
  const int selv = sel[lane < kSel ? lane : kSel - 1];   // lane j < n: ranked bucket j
  const int lim = limit < H ? (int)limit : H;            // a union never exceeds H
  const int nw = (H + 31) >> 5;
  const int last_run = (nw - 1) / V;  // the last run that holds a word below nw
  const uint32_t tail_mask = (H & 31) ? (1u << (H & 31)) - 1u : ~0u;
  const uint32_t* bg = bits + (size_t)g * kF * row_words;
  uint32_t wmask[WPT];
  unsigned rcol[R];
#pragma unroll
  for (int u = 0; u < R; ++u) {
    const int run = tid + u * kCapT;
    rcol[u] = (unsigned)(V * (run <= last_run ? run : last_run));
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const int wd = V * run + e;
      wmask[V * u + e] = run <= last_run && wd < nw ? (wd == nw - 1 ? tail_mask : ~0u) : 0u;
    }
  }
  const int row_bytes = (int)(4 * row_words);
  auto load_row = [&](int j, uint32_t (&r)[WPT]) {  // j uniform
    const int b = __builtin_amdgcn_readlane(selv, j < n ? j : n - 1);
    const uint64_t a = reinterpret_cast<uint64_t>(bg + (size_t)b * row_words);
    const uint64_t base = (uint64_t)__builtin_amdgcn_readfirstlane((unsigned)(a >> 32)) << 32 |
                          (unsigned)__builtin_amdgcn_readfirstlane((unsigned)a);
    const __amdgpu_buffer_rsrc_t rows = __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<void*>(base), (short)0, __builtin_amdgcn_readfirstlane(j < n ? row_bytes : 0),
        kRawBufferWord3);
#pragma unroll
    for (int u = 0; u < R; ++u) load_run<V>(rows, 4 * rcol[u], r + V * u);
  };
  constexpr int kSets = cap_row_sets(R, WPT), kAhead = kSets - 2;
  static_assert(kSets >= 4 && kSets * R <= 63, "rows in flight exceed the load counter");
  uint32_t chosen[WPT], rs[kSets][WPT];
#pragma unroll
  for (int u = 0; u < WPT; ++u) chosen[u] = 0u;
  int total = 0;
  unsigned long long accepted = 0;
  // decisions j and j + 1 (j < n) on rows ra, rb, requesting rows j + kAhead, j + kAhead + 1
  auto pair = [&](int j, uint32_t (&ra)[WPT], uint32_t (&rb)[WPT], uint32_t (&fa)[WPT], uint32_t (&fb)[WPT]) {
    load_row(j + kAhead, fa);
    load_row(j + kAhead + 1, fb);
    __builtin_amdgcn_sched_barrier(0);  // the requests go out before this pair waits
    int cx = 0, cy = 0, cxy = 0;
#pragma unroll
    for (int u = 0; u < WPT; ++u) {
      const uint32_t x = ra[u] & wmask[u] & ~chosen[u], y = rb[u] & wmask[u] & ~chosen[u];
      cx += __popc(x);
      cy += __popc(y & ~x);
      cxy += __popc(y & x);
    }
    cx = wave_sum_dpp(cx);
    cy = wave_sum_dpp(cy);
    cxy = wave_sum_dpp(cxy);
    u32x4* slot = part[(j >> 1) & 1];
    if (lane == 0) slot[w] = u32x4{(unsigned)cx, (unsigned)cy, (unsigned)cxy, 0u};
    __syncthreads();
    // part[(j >> 1) & 1] is rewritten two pairs later, after the next barrier
    int sx = 0, sy = 0, sxy = 0;
#pragma unroll
    for (int i = 0; i < kCapT / 64; ++i) {
      const u32x4 p = slot[i];
      sx += (int)p.x;
      sy += (int)p.y;
      sxy += (int)p.z;
    }
    // uniform: every thread holds the same sums
    const bool take_a = total + sx <= lim;
    const int base = take_a ? total + sx : total, size_b = take_a ? sy : sy + sxy;
    const bool take_b = j + 1 < n && base + size_b <= lim;
    total = take_b ? base + size_b : base;
    if (take_a) {
#pragma unroll
      for (int u = 0; u < WPT; ++u) chosen[u] |= ra[u] & wmask[u];
      accepted |= 1ull << j;
    }
    if (take_b) {
#pragma unroll
      for (int u = 0; u < WPT; ++u) chosen[u] |= rb[u] & wmask[u];
      accepted |= 1ull << (j + 1);
    }
  };
  if (n > 0) {
    // rows requested in rank order, as the loop requests them: the counter
    // wait for a pair then covers exactly the rows before it
#pragma unroll
    for (int i = 0; i < kAhead; ++i) {
      load_row(i, rs[i]);
      __builtin_amdgcn_sched_barrier(0);
    }
    // the walk leaves after its last decision (n is uniform); the loads
    // still pending then are of empty ranges
    for (int j = 0; j < n; j += kSets) {
#pragma unroll
      for (int i = 0; i < kSets; i += 2) {
        if (j + i >= n) break;
        pair(j + i, rs[i], rs[i + 1], rs[(i + kAhead) % kSets], rs[(i + kAhead + 1) % kSets]);
      }
    }
  }
  // wave 0 writes the kept buckets in rank order, lane j its own
  if (w == 0) {
    const int raw_sum = wave_sum_dpp(ok && (accepted >> at & 1ull) ? cnt : 0);
    const int kept = __popcll(accepted);
    if (lane < kSel) {
      int64_t* fg = features + (size_t)g * kSel;
      if (lane < n && (accepted >> lane & 1ull)) fg[__popcll(accepted & ((1ull << lane) - 1ull))] = selv;
      if (lane >= kept) fg[lane] = 0;
      valid[(size_t)g * kSel + lane] = lane < kept ? 1.f : 0.f;
    }
    if (lane == 0) raw[g] = raw_sum;
  }
}

// The same walk for histories up to 2^20 tokens: the running union lives in
// LDS (up to 32768 words) and an accepted bucket's words are read a second
// time (from L2) to merge them in.
constexpr int kCapBigT = 1024;
constexpr int kCapMaxWords = 32768;

template <int kSel>
__global__ __launch_bounds__(kCapBigT) void cap_big_kernel(const uint32_t* __restrict__ bits, int64_t row_words,
                                                           const int* __restrict__ counts, int64_t* features,
                                                           float* valid, int* raw, int H, long long limit) {
  const int g = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  __shared__ int sel[kSel], nsel_s;
  __shared__ int part[2][kCapBigT / 64];
  __shared__ uint32_t chosen[kCapMaxWords];
  const int nw = (H + 31) >> 5;
  for (int i = tid; i < nw; i += kCapBigT) chosen[i] = 0u;
  if (tid == 0) {
    int n = 0;
    for (int j = 0; j < kSel; ++j) {
      const int64_t f = features[(size_t)g * kSel + j];
      if (valid[(size_t)g * kSel + j] > 0.f && f >= 0 && f < kF) sel[n++] = (int)f;
    }
    nsel_s = n;
  }
  __syncthreads();
  const int n = nsel_s;
  const uint32_t tail_mask = (H & 31) ? (1u << (H & 31)) - 1u : ~0u;
  const uint32_t* bg = bits + (size_t)g * kF * row_words;
  long long total = 0;
  int raw_sum = 0;
  unsigned long long accepted = 0;
  for (int j = 0; j < n; ++j) {
    const uint32_t* row = bg + (size_t)sel[j] * row_words;
    int c = 0;
    for (int i = tid; i < nw; i += kCapBigT) {
      const uint32_t m = i == nw - 1 ? (row[i] & tail_mask) : row[i];
      c += __popc(m & ~chosen[i]);
    }
    c = wave_sum_i(c);
    if (lane == 0) part[j & 1][w] = c;
    __syncthreads();
    long long add = 0;
#pragma unroll
    for (int i = 0; i < kCapBigT / 64; ++i) add += part[j & 1][i];
    if (total + add <= limit) {  // uniform
      // each thread merges exactly the words it counted: no other thread touches them
      for (int i = tid; i < nw; i += kCapBigT) chosen[i] |= i == nw - 1 ? (row[i] & tail_mask) : row[i];
      total += add;
      raw_sum += counts[(size_t)g * kFP + sel[j]];
      accepted |= 1ull << j;
    }
  }
  if (tid == 0) {
    int at = 0;
    for (int j = 0; j < n; ++j)
      if (accepted >> j & 1ull) features[(size_t)g * kSel + at++] = sel[j];
    for (int j = 0; j < kSel; ++j) {
      if (j >= at) features[(size_t)g * kSel + j] = 0;
      valid[(size_t)g * kSel + j] = j < at ? 1.f : 0.f;
    }
    raw[g] = raw_sum;
  }
}

}  // namespace
}  // namespace prismkv

using namespace prismkv;

// Words per thread: the widest vector load that still leaves at least 8
// tiles per group (and fits the row alignment).
static int union_wpt(int H, int64_t row_words) {
  const int nw = (H + 31) / 32;
  if (nw >= 8 * kUT * 4 && (row_words & 3) == 0) return 4;
  if (nw >= 8 * kUT * 2 && (row_words & 1) == 0) return 2;
  return 1;
}

extern "C" {

}  // extern "C"

template <int kSel>
static void launch_cap(const uint32_t* b, int64_t row_words, const int* c, int64_t* f, float* v, int* r, int groups,
                       int H, long long lim, hipStream_t s) {
  const int nw = (H + 31) / 32;
  // 16-byte runs where every row starts 16-byte aligned
  const bool quads = (row_words & 3) == 0 && (reinterpret_cast<uintptr_t>(b) & 15) == 0;
  // 512 threads: half the waves to synchronise per decision of 1024, and the
  // registers for 16 words per thread; above 2048 words a row, one
  // row-touching workgroup per group for every 1024 words
  const int parts = nw > 2048 ? (nw + 1023) / 1024 : 0;
  const dim3 grid(groups * (1 + parts)), block(512);
  if (nw > 16 * 512 || (!quads && nw > 4 * 512))  // up to 2^20 tokens
    hipLaunchKernelGGL(cap_big_kernel<kSel>, dim3(groups), dim3(kCapBigT), 0, s, b, row_words, c, f, v, r, H, lim);
  else if (!quads)
    hipLaunchKernelGGL((cap_kernel<512, 1, 4, kSel>), grid, block, 0, s, b, row_words, c, f, v, r, H, lim, groups);
  else if (nw <= 4 * 512)
    hipLaunchKernelGGL((cap_kernel<512, 4, 1, kSel>), grid, block, 0, s, b, row_words, c, f, v, r, H, lim, groups);
  else if (nw <= 8 * 512)
    hipLaunchKernelGGL((cap_kernel<512, 4, 2, kSel>), grid, block, 0, s, b, row_words, c, f, v, r, H, lim, groups);
  else
    hipLaunchKernelGGL((cap_kernel<512, 4, 4, kSel>), grid, block, 0, s, b, row_words, c, f, v, r, H, lim, groups);
}

static int select_cap(uint64_t bits, uint64_t counts, uint64_t features, uint64_t valid, uint64_t raw, int groups,
                      int H, int64_t limit, int64_t row_words, int width, uint64_t stream) {
  if (groups < 1 || groups > 65535 || H < 1 || H > (1 << 20) || limit < 0) return kBadSize;
  if (row_words < (H + 31) / 32 || (width != kTop && width != 64)) return kBadSize;
  if (!bits || !counts || !features || !valid || !raw) return kBadSize;
  const uint32_t* b = reinterpret_cast<const uint32_t*>(bits);
  const int* c = reinterpret_cast<const int*>(counts);
  int64_t* f = reinterpret_cast<int64_t*>(features);
  float* v = reinterpret_cast<float*>(valid);
  int* r = reinterpret_cast<int*>(raw);
  hipStream_t s = (hipStream_t)stream;
  if (width == kTop) launch_cap<kTop>(b, row_words, c, f, v, r, groups, H, (long long)limit, s);
  else launch_cap<64>(b, row_words, c, f, v, r, groups, H, (long long)limit, s);
  return (int)hipGetLastError();
}

extern "C" {

int prismkv_select_cap(uint64_t bits, uint64_t counts, uint64_t features, uint64_t valid, uint64_t raw, int groups,
                       int H, int64_t limit, int64_t row_words, uint64_t stream) {
  return select_cap(bits, counts, features, valid, raw, groups, H, limit, row_words, kTop, stream);
}

int prismkv_select_cap_n(uint64_t bits, uint64_t counts, uint64_t features, uint64_t valid, uint64_t raw, int groups,
                         int H, int64_t limit, int64_t row_words, int width, uint64_t stream) {
  return select_cap(bits, counts, features, valid, raw, groups, H, limit, row_words, width, stream);
}

size_t prismkv_union_work_bytes(int groups, int H) {
  if (groups < 1 || H < 1) return 0;
  const int tiles = union_tiles(H, 1);  // the largest tile count of any variant
  return ((size_t)groups * tiles + groups + 4) * sizeof(unsigned);
}

}  // extern "C"

template <int kSel>
static void launch_union(const uint32_t* b, int64_t row_words, const int64_t* f, const float* v, int32_t* o,
                         int64_t ids_stride, int32_t* c, UnionWork uw, int H, int wpt, dim3 grid, hipStream_t s) {
  const int tiles = (int)grid.x;
  const dim3 block(kUT);
  if (wpt == 4)
    hipLaunchKernelGGL((union_kernel<4, kSel>), grid, block, 0, s, b, row_words, f, v, o, ids_stride, c, uw, H, tiles);
  else if (wpt == 2)
    hipLaunchKernelGGL((union_kernel<2, kSel>), grid, block, 0, s, b, row_words, f, v, o, ids_stride, c, uw, H, tiles);
  else
    hipLaunchKernelGGL((union_kernel<1, kSel>), grid, block, 0, s, b, row_words, f, v, o, ids_stride, c, uw, H, tiles);
}

static int union_impl(uint64_t bits, uint64_t features, uint64_t valid, uint64_t work, uint64_t ids, uint64_t count,
                      int groups, int H, int64_t row_words, int64_t ids_stride, int width, size_t work_bytes,
                      uint64_t stream) {
  if (groups < 1 || groups > 65535 || H < 1 || H > (1 << 29)) return kBadSize;
  if (row_words < (H + 31) / 32 || ids_stride < H || (width != kTop && width != 64)) return kBadSize;
  if (!bits || !features || !valid || !work || !ids || !count) return kBadSize;
  if (work_bytes < prismkv_union_work_bytes(groups, H)) return kBadSize;
  const int wpt = union_wpt(H, row_words);
  const int tiles = union_tiles(H, wpt);
  // fixed layout for any H: err word, its host-word slot (bytes 8-15),
  // done[groups], then status[groups][tiles]
  if (work % 8) return kBadSize;
  unsigned* w = reinterpret_cast<unsigned*>(work);
  UnionWork uw{w + 4 + groups, w + 4, w, spin_limit()};
  const dim3 grid(tiles, groups);
  const uint32_t* b = reinterpret_cast<const uint32_t*>(bits);
  const int64_t* f = reinterpret_cast<const int64_t*>(features);
  const float* v = reinterpret_cast<const float*>(valid);
  int32_t* o = reinterpret_cast<int32_t*>(ids);
  int32_t* c = reinterpret_cast<int32_t*>(count);
  hipStream_t s = (hipStream_t)stream;
  if (width == kTop) launch_union<kTop>(b, row_words, f, v, o, ids_stride, c, uw, H, wpt, grid, s);
  else launch_union<64>(b, row_words, f, v, o, ids_stride, c, uw, H, wpt, grid, s);
  return (int)hipGetLastError();
}

extern "C" {

int prismkv_union(uint64_t bits, uint64_t features, uint64_t valid, uint64_t work, uint64_t ids, uint64_t count,
                  int groups, int H, int64_t row_words, int64_t ids_stride, size_t work_bytes, uint64_t stream) {
  return union_impl(bits, features, valid, work, ids, count, groups, H, row_words, ids_stride, kTop, work_bytes,
                    stream);
}

int prismkv_union_n(uint64_t bits, uint64_t features, uint64_t valid, uint64_t work, uint64_t ids, uint64_t count,
                    int groups, int H, int64_t row_words, int64_t ids_stride, int width, size_t work_bytes,
                    uint64_t stream) {
  return union_impl(bits, features, valid, work, ids, count, groups, H, row_words, ids_stride, width, work_bytes,
                    stream);
}

int prismkv_build_bits(uint64_t ids, uint64_t offsets, uint64_t bits, int groups, int64_t cap, int64_t row_words,
                       uint64_t stream) {
  if (groups < 1 || groups > 65535 || cap < 0 || row_words < 1) return kBadSize;
  hipLaunchKernelGGL(bits_kernel, dim3(kF, groups), dim3(256), 0, (hipStream_t)stream,
                     reinterpret_cast<const int*>(ids), reinterpret_cast<const int*>(offsets),
                     reinterpret_cast<uint32_t*>(bits), cap, row_words);
  return (int)hipGetLastError();
}

int build_bits(uint64_t ids, uint64_t offsets, uint64_t bits, int H, int C, uint64_t stream) {
  if (H < 1 || C < 0) return kBadSize;
  return prismkv_build_bits(ids, offsets, bits, 8, C, (H + 31) / 32, stream);
}

int launch_union_warp(uint64_t bits, uint64_t ids, uint64_t vals, uint64_t mask, uint64_t tiles, uint64_t selected,
                      uint64_t counts, int U, int H, int mode, uint64_t stream) {
  if (U < 1 || U > 8 || H < 1 || H > 131072) return kBadSize;
  if (mode < 0 || mode > 2) return kBadMode;
  const int nw = (H + 31) / 32, nb = (nw + kCT - 1) / kCT;
  hipLaunchKernelGGL(compat_count, dim3(nb, U), dim3(kCT), 0, (hipStream_t)stream,
                     reinterpret_cast<const uint32_t*>(bits), reinterpret_cast<const int64_t*>(ids),
                     reinterpret_cast<const float*>(vals), reinterpret_cast<uint32_t*>(mask),
                     reinterpret_cast<int*>(tiles), nw, nb);
  hipLaunchKernelGGL(compat_extract, dim3(nb, U), dim3(kCT), 0, (hipStream_t)stream,
                     reinterpret_cast<const uint32_t*>(mask), reinterpret_cast<const int*>(tiles),
                     reinterpret_cast<int*>(selected), reinterpret_cast<int*>(counts), H, nw, nb);
  return (int)hipGetLastError();
}

}  // extern "C"
