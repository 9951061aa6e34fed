// Stage 4 -- the index update (append_index) and the prefill index build
// (build_index): encode keys with the group's SAE, take the exact batch-wide
// positive Top-k of the activations, set the members' bitmap bits and
// (re)compute the bucket moments.
//
// Semantics: src/prismkv/core.py:186-201 (append_index) on top of
//   build_index  core.py:92-103  center = keys.float().mean(0) unless given
//                                (append: the ORIGINAL center);
//                                x = (k - center) / key_scale;
//                                a = relu(x W^T + b) (SharedSAE.dense,
//                                core.py:47-48);
//   positive_global_topk core.py:13-26  budget N * key_mean over the keys
//                                indexed: keep a > tau and a > 0, then, if
//                                tau > 0, values == tau in ascending flat
//                                index (token * F + feature) up to the budget;
//   summarize    core.py:76-89   per-bucket mean / population variance of
//                                the ORIGINAL keys (two-pass);
//   the merge    core.py:190-199 mean = (a m_a + b m_b) / max(a+b, 1),
//                                var = (a v_a + b v_b) / max(a+b, 1)
//                                      + a b / max(a+b, 1)^2 (m_a - m_b)^2,
//                                in fp32 and in that operation order;
//   lists        core.py:200     new members are tokens H + t: here bits
//                                H + t of the bucket's bitmap row
//                                (kernels/ppu_8b/pack.cu:5 bit order).
//
// Launches of one update (all G groups at once; the update runs every
// `interval` tokens, its cost is amortised):
//   encode   LDS-tiled fp32 GEMM, 64 tokens x 64 buckets per workgroup,
//            writes a = relu(...) [G][N][F] and a histogram of the positive
//            values' top 11 bits (4 replicas of each global bin, so the
//            flushes of ~750 workgroups do not queue on one address);
//   digit    one workgroup per group picks the histogram bin holding the
//            budget-th largest value (3 levels: bits 30..20, 19..9, 8..0);
//   refine   re-reads a, histograms the values inside the chosen prefix;
//   emit     sets bitmap bits for a > tau (or all positives when fewer
//            than the budget are positive) and for a == tau when every tie
//            fits the budget;
//   ties     only when ties overflow the budget: per contiguous range of a,
//            count the ties, then take the first `need` in flat order;
//   moments  per 32-bucket tile: new members from the bitmap, two-pass
//            moments of their keys, merge, counts += new.
// Keys are the model's bf16 K cache or fp32 rows (the `_f32` entry points):
// the kernels that read keys take the element type as a template argument
// and widen every key to fp32 at the load, so both compute the same fp32 /
// double arithmetic on the values they are given.
// The build runs the same selection over all H keys of a group (in batches
// of groups, so the activations of one batch fit the workspace) after a
// center pass and a bitmap clear, and computes every bucket's moments from
// scratch (build_moments: one workgroup per bucket, any member count).
#include <algorithm>

#include "common.h"

namespace prismkv {
namespace {

constexpr int kUT = 256;
constexpr int kTT = 64;        // tokens per encode tile
constexpr int kFT = 64;        // buckets per encode tile
constexpr int kFTiles = (kF + kFT - 1) / kFT;  // 47
constexpr int kBins = 2048;
constexpr int kRep = 4;        // global histogram replicas
constexpr int kLevels = 3;
constexpr int kRefineBlocks = 256;  // workgroups per group of a pass over a
constexpr int kMaxTieBlocks = 4096;  // contiguous ranges of a per group for the ordered ties
constexpr int kTieMinLen = 65536;    // values per range at least (multiple of 4 * kUT)
constexpr int kTieGrid = 256;        // workgroups per group of the tie kernels
constexpr int kCenterParts = 64;     // row ranges of the center sum
constexpr int kListChunk = 256;      // list entries a wave reserves at once once its workgroup's buffer is full
constexpr unsigned kListSlack = (unsigned)kRefineBlocks * (kUT / 64) * kListChunk;  // unfilled chunk tails, at most
constexpr int kMaxBuild = 1 << 20;   // keys per group of a build (N * F < 2^32 flat indices)
constexpr int kBuildCenter = 1;      // prismkv_build flag: compute the center (else it is an input)

// ctl words per group
enum { kMode = 0, kPrefix, kRem, kTau, kNeed, kTies, kOrdered, kCount, kListed, kListLen, kCtl = 16 };
enum { kModeTopK = 0, kModeAllPositive = 1 };

// Key loads of the two key element types: 2, 4 or 8 consecutive dims as the
// raw loaded bits (kept packed while in flight) and their fp32 values.
template <typename KT>
struct KeyLoad;

template <>
struct KeyLoad<uint16_t> {  // bf16
  typedef uint32_t Raw2;
  typedef uint2 Raw4;
  static __device__ __forceinline__ Raw2 load2(const uint16_t* p) { return *reinterpret_cast<const uint32_t*>(p); }
  static __device__ __forceinline__ float lo(Raw2 r) { return bf16_lo(r); }
  static __device__ __forceinline__ float hi(Raw2 r) { return bf16_hi(r); }
  static __device__ __forceinline__ Raw4 load4(const uint16_t* p) { return *reinterpret_cast<const uint2*>(p); }
  static __device__ __forceinline__ float4 f4(Raw4 r) {
    return make_float4(bf16_lo(r.x), bf16_hi(r.x), bf16_lo(r.y), bf16_hi(r.y));
  }
  static __device__ __forceinline__ void load8(const uint16_t* p, float (&x)[8]) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    x[0] = bf16_lo(v.x); x[1] = bf16_hi(v.x); x[2] = bf16_lo(v.y); x[3] = bf16_hi(v.y);
    x[4] = bf16_lo(v.z); x[5] = bf16_hi(v.z); x[6] = bf16_lo(v.w); x[7] = bf16_hi(v.w);
  }
};

template <>
struct KeyLoad<float> {
  typedef float2 Raw2;
  typedef float4 Raw4;
  static __device__ __forceinline__ Raw2 load2(const float* p) { return *reinterpret_cast<const float2*>(p); }
  static __device__ __forceinline__ float lo(Raw2 r) { return r.x; }
  static __device__ __forceinline__ float hi(Raw2 r) { return r.y; }
  static __device__ __forceinline__ Raw4 load4(const float* p) { return *reinterpret_cast<const float4*>(p); }
  static __device__ __forceinline__ float4 f4(Raw4 r) { return r; }
  static __device__ __forceinline__ void load8(const float* p, float (&x)[8]) {
    const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  }
};

struct UpdateArgs {
  const void* k;      // K rows (bf16 or fp32); the block is rows [H, H+N) of each group
  int64_t ks;         // group stride (elements)
  const float* W;     // [G][F][128]
  const float* b;     // [G][F]
  const float* center;  // [G][128]
  const float* scale;   // [G]
  uint32_t* bits;
  int64_t row_words;
  int* counts;     // [G][kFP]
  float* moments;  // [G][kChunks][256][32]
  float* act;      // [G][N][F]
  unsigned* hist;  // [G][kLevels][kRep][kBins]
  unsigned* ctl;   // [G][kCtl]
  unsigned* tcount;  // [G][tie_blocks] ties per contiguous range of a
  uint2* list;       // [G][list_cap] (flat index, value bits) of the values at or above tau's first digit
  unsigned list_cap;  // entries per group (0 bits: an unfilled chunk entry)
  int H, N;          // first key row / bitmap column, keys indexed
  long long budget;  // N * key_mean
  int tie_blocks;
  long long tie_len;  // values per range, a multiple of 4 * kUT
};

__device__ __forceinline__ unsigned* hist_of(const UpdateArgs& a, int g, int level) {
  return a.hist + ((size_t)g * kLevels + level) * kRep * kBins;
}

// ---------------------------------------------------------------------------
// encode: grid (ceil(N / 128), P, G) x 512.  Workgroup (y, part) takes the
// tokens [128 y, 128 y + 128), wave w the 16 rows 128 y + 16 w + i, and the
// bucket tiles part, part + P, ... (64 buckets each).  The wave's
// x = (k - center) / scale is computed once, into registers, and each bucket
// tile's W streams through LDS, double-buffered: the next tile's W is
// requested into registers while the current tile is multiplied, then
// stored to the other buffer.  Products run on fp32 MFMA
// (v_mfma_f32_16x16x4f32: lane l feeds A[i = l % 16][k = l / 16],
// B[k][j = l % 16] and holds D[4 (l / 16) + r][l % 16]).  A is W (bucket
// rows) and B is x (token columns), so D is [bucket][token] and lane (i, q)
// ends with buckets 4 q .. 4 q + 3 of token i, stored as one 16-byte store.
// Lane (i, q) = (l % 16, l / 16) supplies the dims 16 kb + 4 q + t of dim
// block kb to step t: its W values are one 16-byte LDS read per 16-bucket
// column and block, its x values those of token row i at its 32 dims.  A and
// B always pair the same dim, so the steps only reorder the sum over the 128
// dims (the same order for every token and bucket).  P is the smallest count that gives the launch
// kEncMinWgs workgroups (two per CU), so the x of a token is computed P times
// in all rather than once per bucket tile.
// ---------------------------------------------------------------------------
typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int kET = 512;                          // encode workgroup
constexpr int kRowTile = 16;                      // tokens per wave
constexpr int kEncTokens = kET / 64 * kRowTile;   // tokens per workgroup (128)
constexpr int kEncMinWgs = 512;                   // workgroups the bucket-tile parts aim for
constexpr int kWLoads = kFT * kD / 4 / kET;       // float4 of a W tile per thread (4)

// K chunk kb (4 dims 16 kb + 4 q ..) of token row t0 + i for lane (i, q).
template <typename KT>
__device__ __forceinline__ typename KeyLoad<KT>::Raw4 key_chunk(const UpdateArgs& a, int g, int t0, int kb) {
  const int li = threadIdx.x & 15, lq = (threadIdx.x >> 4) & 3;
  const int row = min(t0 + li, a.N - 1);  // rows past the block repeat the last one (masked at the store)
  const KT* k = static_cast<const KT*>(a.k);
  return KeyLoad<KT>::load4(k + (size_t)g * a.ks + (size_t)(a.H + row) * kD + 16 * kb + 4 * lq);
}

template <typename KT>
__global__ __launch_bounds__(kET) void encode_kernel(UpdateArgs a) {
  const int y = blockIdx.x, part = blockIdx.y, parts = gridDim.y, g = blockIdx.z, tid = threadIdx.x;
  const int w = tid >> 6, lane = tid & 63, li = lane & 15, lq = lane >> 4;
  __shared__ __align__(16) float ws[2][kFT][kD + 4];  // [buffer][bucket][dim], padded against bank conflicts
  __shared__ __align__(16) float cs[kD];              // center
  __shared__ unsigned hist[kBins];
  const int t0 = y * kEncTokens + w * kRowTile;  // the wave's first token
  typename KeyLoad<KT>::Raw4 kr[kD / 16];
#pragma unroll
  for (int kb = 0; kb < kD / 16; ++kb) kr[kb] = key_chunk<KT>(a, g, t0, kb);
  const float* wg = a.W + (size_t)g * kF * kD;
  // thread tid moves float4 tid + kET u of a 64 x 128 W tile (bucket i / 32, dims 4 (i % 32) ..)
  auto load_w = [&](int ft, float4 (&r)[kWLoads]) {
#pragma unroll
    for (int u = 0; u < kWLoads; ++u) {
      const int i = tid + kET * u, f = ft * kFT + i / (kD / 4);
      r[u] = f < kF ? *reinterpret_cast<const float4*>(wg + (size_t)f * kD + 4 * (i % (kD / 4)))
                    : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  auto store_w = [&](int buf, const float4 (&r)[kWLoads]) {
#pragma unroll
    for (int u = 0; u < kWLoads; ++u) {
      const int i = tid + kET * u;
      *reinterpret_cast<float4*>(&ws[buf][i / (kD / 4)][4 * (i % (kD / 4))]) = r[u];
    }
  };
  float4 wr[kWLoads];
  load_w(part, wr);
  for (int i = tid; i < kBins; i += kET) hist[i] = 0;
  if (tid < kD) cs[tid] = a.center[(size_t)g * kD + tid];
  __syncthreads();
  // x = (k - center) / key_scale in fp32 (core.py:98) for this lane's row and 32 dims
  const float sc = a.scale[g];
  float4 xs[kD / 16];
#pragma unroll
  for (int kb = 0; kb < kD / 16; ++kb) {
    const float4 r = KeyLoad<KT>::f4(kr[kb]);
    const float4 c = *reinterpret_cast<const float4*>(&cs[16 * kb + 4 * lq]);
    xs[kb] = make_float4((r.x - c.x) / sc, (r.y - c.y) / sc, (r.z - c.z) / sc, (r.w - c.w) / sc);
  }
  store_w(0, wr);
  __syncthreads();
  const float* bg = a.b + (size_t)g * kF;
  float* ag = a.act + (size_t)g * a.N * kF;
  int buf = 0;
  for (int ft = part; ft < kFTiles; ft += parts) {  // uniform
    const bool more = ft + parts < kFTiles;
    if (more) load_w(ft + parts, wr);  // in flight while this tile is multiplied
    const int f0 = ft * kFT;
    // the output is bucket-major (lane (i, q): buckets f0 + 16 j + 4 q .. + 3
    // of token t0 + i), so each lane's 4 values of a j go out as one 16-byte
    // store; kF is a multiple of 4, so those 4 buckets are live together
    float4 bias[kFT / 16];
#pragma unroll
    for (int j = 0; j < kFT / 16; ++j) {
      const int f = f0 + 16 * j + 4 * lq;
      bias[j] = f < kF ? *reinterpret_cast<const float4*>(bg + f) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    f32x4 acc[kFT / 16];
#pragma unroll
    for (int j = 0; j < kFT / 16; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < kD / 16; ++kb) {
      const float4 xa = xs[kb];
      float4 bv[kFT / 16];
#pragma unroll
      for (int j = 0; j < kFT / 16; ++j)
        bv[j] = *reinterpret_cast<const float4*>(&ws[buf][16 * j + li][16 * kb + 4 * lq]);
      // the four accumulators interleaved: no MFMA waits on the one before it.
      // A = W (bucket rows), B = x (token columns): D[bucket][token], the
      // same products in the same order as x W^T, transposed
#pragma unroll
      for (int j = 0; j < kFT / 16; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(bv[j].x, xa.x, acc[j], 0, 0, 0);
#pragma unroll
      for (int j = 0; j < kFT / 16; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(bv[j].y, xa.y, acc[j], 0, 0, 0);
#pragma unroll
      for (int j = 0; j < kFT / 16; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(bv[j].z, xa.z, acc[j], 0, 0, 0);
#pragma unroll
      for (int j = 0; j < kFT / 16; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(bv[j].w, xa.w, acc[j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    // bias, relu, histogram of the positive values, store: lane (i, q) holds
    // buckets f0 + 16 j + 4 q + r of token t0 + i
    const int tok = t0 + li;
#pragma unroll
    for (int j = 0; j < kFT / 16; ++j) {
      const int f = f0 + 16 * j + 4 * lq;
      const float b4[4] = {bias[j].x, bias[j].y, bias[j].z, bias[j].w};
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float x = acc[j][r] + b4[r];
        v[r] = x > 0.f ? x : 0.f;  // relu; non-positive values are never selected
      }
      if (tok < a.N && f < kF) {
        *reinterpret_cast<float4*>(&ag[(size_t)tok * kF + f]) = make_float4(v[0], v[1], v[2], v[3]);
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (v[r] > 0.f) atomicAdd(&hist[__float_as_uint(v[r]) >> 20], 1u);
      }
    }
    if (more) {  // the other buffer was last read before the previous barrier
      store_w(buf ^ 1, wr);
      __syncthreads();
      buf ^= 1;
    }
  }
  __syncthreads();
  unsigned* hg = hist_of(a, g, 0) + ((part + y) % kRep) * kBins;
  for (int i = tid; i < kBins; i += kET)
    if (hist[i]) atomicAdd(&hg[i], hist[i]);
}

// ---------------------------------------------------------------------------
// digit: grid G x 256.  Level L consumes hist level L (all replicas, then
// zeroes them for the next update) and narrows the threshold prefix.
// Level widths: 11 bits (30..20), 11 bits (19..9), 9 bits (8..0); positive
// floats order like their bit patterns, so the prefix after level 2 is the
// exact bit pattern of tau, the budget-th largest value.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kUT) void digit_kernel(UpdateArgs a, int level) {
  const int g = blockIdx.x, tid = threadIdx.x;
  __shared__ unsigned wsum[kUT / 64];
  __shared__ unsigned found_digit, found_rem, found_ties;
  unsigned* ctl = a.ctl + (size_t)g * kCtl;
  unsigned* h = hist_of(a, g, level);
  constexpr int kPer = kBins / kUT;  // 8 bins per thread, descending digits
  unsigned c[kPer], tot = 0;
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int d = kBins - 1 - (tid * kPer + u);
    unsigned s = 0;
#pragma unroll
    for (int r = 0; r < kRep; ++r) {
      s += h[r * kBins + d];
      h[r * kBins + d] = 0;
    }
    c[u] = s;
    tot += s;
  }
  const long long total_vals = (long long)a.N * kF;
  const unsigned count = (unsigned)(a.budget < total_vals ? a.budget : total_vals);
  const unsigned incl = block_incl_scan<kUT>(tot, wsum);
  unsigned rem, prefix_in;
  if (level == 0) {
    // wsum holds the per-wave totals: their sum is the number of positive values
    const unsigned npos = wsum[0] + wsum[1] + wsum[2] + wsum[3];
    if (npos < count || count == 0) {
      // fewer positives than the budget: tau = 0 and every positive value is
      // kept (core.py:22-26); an empty budget keeps nothing
      if (tid == 0) {
        ctl[kMode] = count == 0 ? kModeTopK : kModeAllPositive;
        ctl[kPrefix] = 0;
        ctl[kRem] = 0;
        ctl[kTau] = count == 0 ? 0x7f800000u : 0u;
        ctl[kNeed] = 0;
        ctl[kTies] = 0;
        ctl[kOrdered] = 0;
        ctl[kCount] = count;
        ctl[kListed] = 0;
      }
      return;
    }
    rem = count;
    prefix_in = 0;
  } else {
    if (ctl[kMode] != kModeTopK || ctl[kTau] == 0x7f800000u) return;
    rem = ctl[kRem];
    prefix_in = ctl[kPrefix];
  }
  const int width = level < 2 ? 11 : 9;
  unsigned run = incl - tot;
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int d = kBins - 1 - (tid * kPer + u);
    if (d < (1 << width) && run < rem && run + c[u] >= rem) {
      found_digit = (unsigned)d;
      found_rem = rem - run;
      found_ties = c[u];
    }
    run += c[u];
  }
  __syncthreads();
  if (tid == 0) {
    const unsigned prefix = (prefix_in << width) | found_digit;
    if (level == 0) {
      // every value the selection can take lies in the first digit's bin or
      // above it: (count - found_rem) above, found_ties in it.  If they fit,
      // the first refine pass collects them and the later passes read only them.
      ctl[kListed] = (unsigned long long)(count - found_rem) + found_ties + kListSlack <= (unsigned long long)a.list_cap;
      ctl[kListLen] = 0;
    }
    ctl[kMode] = kModeTopK;
    ctl[kPrefix] = prefix;
    ctl[kRem] = found_rem;
    ctl[kCount] = count;
    if (level == kLevels - 1) {
      // prefix is the exact tau; found_rem of its found_ties ties are taken
      ctl[kTau] = prefix;
      ctl[kNeed] = found_rem;
      ctl[kTies] = found_ties;
      ctl[kOrdered] = found_ties > found_rem;
    } else {
      ctl[kTau] = 0;
    }
  }
}

// ---------------------------------------------------------------------------
// refine: grid (kRefineBlocks, G) x 256; histogram of the next digit of the
// positive values whose higher bits equal the prefix.  Level 1 reads a and,
// when the digit kernel found that they fit (ctl kListed), also collects every
// positive value whose first digit is at or above tau's into the group's
// compact list: a workgroup gathers its own in LDS (slots by LDS atomics) and
// reserves its range of the list with one global atomic at its end; once the
// LDS buffer is full, each wave writes into chunks of kListChunk entries of
// the list that it reserves one at a time and zero-fills the unused tail of
// its last one (an index build's candidates, about 8 per key, overflow every
// buffer).  Level 2 and the emit then read only the list, skipping zero
// entries.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kUT) void refine_kernel(UpdateArgs a, int level) {
  const int g = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
  unsigned* ctl = a.ctl + (size_t)g * kCtl;
  if (ctl[kMode] != kModeTopK || ctl[kTau] == 0x7f800000u) return;
  constexpr int kBuf = 1024;  // LDS list entries per workgroup
  __shared__ unsigned hist[kBins];
  __shared__ uint2 buf[kBuf];
  __shared__ unsigned nbuf, first_miss, base_s;
  for (int i = tid; i < kBins; i += kUT) hist[i] = 0;
  if (tid == 0) {
    nbuf = 0u;
    first_miss = kBuf;
  }
  __syncthreads();
  const unsigned prefix = ctl[kPrefix];
  const bool listed = ctl[kListed] != 0u;
  const int shift_hi = level == 1 ? 20 : 9;  // bits above this level's digit
  const int shift = level == 1 ? 9 : 0;
  const unsigned dmask = level == 1 ? 0x7ffu : 0x1ffu;
  uint2* list = a.list + (size_t)g * a.list_cap;
  if (level == 2 && listed) {
    const unsigned len = min(ctl[kListLen], a.list_cap);
    for (unsigned i = blockIdx.x * kUT + tid; i < len; i += gridDim.x * kUT) {
      const unsigned u = list[i].y;
      if (u != 0u && (u >> shift_hi) == prefix) atomicAdd(&hist[(u >> shift) & dmask], 1u);
    }
  } else {
    const size_t n = (size_t)a.N * kF;
    const float4* ag = reinterpret_cast<const float4*>(a.act + (size_t)g * n);
    const bool collect = level == 1 && listed;
    // this wave's chunk of the list, once the workgroup's buffer is full:
    // entries [c_at, c_at + c_n) are filled (c_n = kListChunk: none to fill)
    unsigned c_at = 0u, c_n = (unsigned)kListChunk;
    for (size_t i = (size_t)blockIdx.x * kUT + tid; i < (n / 4 + kUT - 1) / kUT * kUT;
         i += (size_t)gridDim.x * kUT) {  // every lane of a wave iterates alike (the list's ballot)
      const bool in = i < n / 4;
      const float4 v4 = in ? ag[i] : make_float4(0.f, 0.f, 0.f, 0.f);
      const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const unsigned u = __float_as_uint(vv[j]);
        if (vv[j] > 0.f && (u >> shift_hi) == prefix) atomicAdd(&hist[(u >> shift) & dmask], 1u);
        if (collect) {
          const bool take = vv[j] > 0.f && (u >> 20) >= prefix;
          const unsigned long long m = __ballot(take);
          if (m) {  // uniform
            const unsigned cnt = (unsigned)__popcll(m), rank = (unsigned)__popcll(m & ((1ull << lane) - 1ull));
            unsigned at = 0u;
            if (lane == 0) at = atomicAdd(&nbuf, cnt);
            at = __shfl(at, 0);
            if (at + cnt <= (unsigned)kBuf) {  // uniform
              if (take) buf[at + rank] = make_uint2((unsigned)(4 * i + j), u);
            } else {
              // the buffer is full: into the wave's chunk of the list, a new
              // chunk reserved (one global atomic per kListChunk entries) for
              // what does not fit.  Reservations come in increasing order, so
              // every one that fitted the buffer lies below the first that did
              // not, and the buffer's valid entries are those below it.
              if (lane == 0) atomicMin(&first_miss, at);
              const unsigned room = (unsigned)kListChunk - c_n;  // uniform
              unsigned nat = 0u;
              if (cnt > room) {  // uniform
                if (lane == 0) nat = atomicAdd(&ctl[kListLen], (unsigned)kListChunk);
                nat = __shfl(nat, 0);
              }
              if (take) {
                const unsigned dst = rank < room ? c_at + c_n + rank : nat + (rank - room);
                if (dst < a.list_cap) list[dst] = make_uint2((unsigned)(4 * i + j), u);
              }
              if (cnt > room) {
                c_at = nat;
                c_n = cnt - room;
              } else {
                c_n += cnt;
              }
            }
          }
        }
      }
    }
    // the unfilled tail of the wave's chunk reads as no entry (value bits 0)
    for (unsigned e = c_n + lane; e < (unsigned)kListChunk; e += 64)
      if (c_at + e < a.list_cap) list[c_at + e] = make_uint2(0u, 0u);
  }
  __syncthreads();
  unsigned* hg = hist_of(a, g, level) + (blockIdx.x % kRep) * kBins;
  for (int i = tid; i < kBins; i += kUT)
    if (hist[i]) atomicAdd(&hg[i], hist[i]);
  // the workgroup's buffered candidates
  const unsigned nb = min(nbuf, first_miss);
  if (nb == 0u) return;  // uniform
  if (tid == 0) base_s = atomicAdd(&ctl[kListLen], nb);
  __syncthreads();
  for (unsigned i = tid; i < nb; i += kUT)
    if (base_s + i < a.list_cap) list[base_s + i] = buf[i];
}

__device__ __forceinline__ void set_member(const UpdateArgs& a, int g, unsigned flat) {
  const int tok = (int)(flat / kF), f = (int)(flat % kF);
  const int t = a.H + tok;
  atomicOr(a.bits + ((size_t)g * kF + f) * a.row_words + (t >> 5), 1u << (t & 31));
}

// ---------------------------------------------------------------------------
// emit: grid (kRefineBlocks, G) x 256 over a.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kUT) void emit_kernel(UpdateArgs a) {
  const int g = blockIdx.y, tid = threadIdx.x;
  const unsigned* ctl = a.ctl + (size_t)g * kCtl;
  const unsigned mode = ctl[kMode];
  const float tau = __uint_as_float(ctl[kTau]);
  const bool take_ties = mode == kModeTopK && !ctl[kOrdered] && tau > 0.f;
  if (mode == kModeTopK && ctl[kListed]) {  // every candidate is in the compact list
    const uint2* list = a.list + (size_t)g * a.list_cap;
    const unsigned len = min(ctl[kListLen], a.list_cap);
    for (unsigned i = blockIdx.x * kUT + tid; i < len; i += gridDim.x * kUT) {
      const uint2 e = list[i];
      const float v = __uint_as_float(e.y);
      if (e.y != 0u && (v > tau || (take_ties && v == tau))) set_member(a, g, e.x);
    }
    return;
  }
  const size_t n = (size_t)a.N * kF;
  const float4* ag = reinterpret_cast<const float4*>(a.act + (size_t)g * n);
  for (size_t i = (size_t)blockIdx.x * kUT + tid; i < n / 4; i += (size_t)gridDim.x * kUT) {
    const float4 v4 = ag[i];
    const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float v = vv[j];
      const bool sel = mode == kModeAllPositive ? v > 0.f : ((v > tau && v > 0.f) || (take_ties && v == tau));
      if (sel) set_member(a, g, (unsigned)(4 * i + j));
    }
  }
}

// ---------------------------------------------------------------------------
// ties, only when the ties at tau overflow the budget: the first `need` of
// them in ascending flat index (core.py:23-24).  The activations of a group
// are cut into tie_blocks contiguous ranges [r L, (r + 1) L), dealt to the
// workgroups r = x, x + kTieGrid, ...  tie_count_kernel counts each range's
// ties; tie_take_kernel skips the ties of the lower ranges and takes the
// range's own in flat order (4 consecutive values per thread) while the
// budget lasts.  Grid (min(tie_blocks, kTieGrid), G) x 256 each.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool ordered_ties(const UpdateArgs& a, int g) {
  const unsigned* ctl = a.ctl + (size_t)g * kCtl;
  return ctl[kMode] == kModeTopK && ctl[kOrdered];
}

__global__ __launch_bounds__(kUT) void tie_count_kernel(UpdateArgs a) {
  const int g = blockIdx.y, tid = threadIdx.x;
  if (!ordered_ties(a, g)) return;
  __shared__ unsigned wsum[kUT / 64];
  const float tau = __uint_as_float(a.ctl[(size_t)g * kCtl + kTau]);
  const size_t n = (size_t)a.N * kF;
  const float4* ag = reinterpret_cast<const float4*>(a.act + (size_t)g * n);
  for (int r = blockIdx.x; r < a.tie_blocks; r += gridDim.x) {  // uniform
    const size_t lo = min(n, (size_t)r * a.tie_len), hi = min(n, lo + a.tie_len);
    unsigned c = 0;
    constexpr int kU = 8;  // loads in flight per thread
    for (size_t i0 = lo / 4 + tid; i0 < hi / 4; i0 += kU * kUT) {
      float4 v[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const size_t i = i0 + (size_t)u * kUT;
        v[u] = ag[i < hi / 4 ? i : i0];  // a repeated value is not counted twice below
      }
#pragma unroll
      for (int u = 0; u < kU; ++u)
        if (i0 + (size_t)u * kUT < hi / 4)
          c += (unsigned)(v[u].x == tau) + (unsigned)(v[u].y == tau) + (unsigned)(v[u].z == tau) +
               (unsigned)(v[u].w == tau);
    }
    block_incl_scan<kUT>(c, wsum);
    if (tid == 0) a.tcount[(size_t)g * a.tie_blocks + r] = wsum[0] + wsum[1] + wsum[2] + wsum[3];
    __syncthreads();  // wsum is rewritten by the next range's scan
  }
}

__global__ __launch_bounds__(kUT) void tie_take_kernel(UpdateArgs a) {
  const int g = blockIdx.y, tid = threadIdx.x;
  if (!ordered_ties(a, g)) return;
  __shared__ unsigned wsum[kUT / 64];
  const unsigned* ctl = a.ctl + (size_t)g * kCtl;
  const float tau = __uint_as_float(ctl[kTau]);  // > 0: only positive values reach the histogram
  const unsigned need = ctl[kNeed];
  const size_t n = (size_t)a.N * kF;
  const float4* ag = reinterpret_cast<const float4*>(a.act + (size_t)g * n);
  for (int r = blockIdx.x; r < a.tie_blocks; r += gridDim.x) {  // uniform
    unsigned below = 0;
    for (int j = tid; j < r; j += kUT) below += a.tcount[(size_t)g * a.tie_blocks + j];
    block_incl_scan<kUT>(below, wsum);
    unsigned taken = wsum[0] + wsum[1] + wsum[2] + wsum[3];  // ties of the lower ranges, all ranked first
    __syncthreads();  // every thread has read wsum before the next scan rewrites it
    const size_t lo = min(n, (size_t)r * a.tie_len), hi = min(n, lo + a.tie_len);
    for (size_t base = lo / 4; base < hi / 4 && taken < need; base += kUT) {  // uniform condition
      const size_t i = base + tid;
      const float4 v = i < hi / 4 ? ag[i] : make_float4(0.f, 0.f, 0.f, 0.f);
      const bool h[4] = {v.x == tau, v.y == tau, v.z == tau, v.w == tau};
      const unsigned c = (unsigned)h[0] + (unsigned)h[1] + (unsigned)h[2] + (unsigned)h[3];
      const unsigned incl = block_incl_scan<kUT>(c, wsum);
      unsigned rank = taken + incl - c;  // rank of this thread's first tie among all ties
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (h[j]) {
          if (rank < need) set_member(a, g, (unsigned)(4 * i + j));
          ++rank;
        }
      taken += wsum[0] + wsum[1] + wsum[2] + wsum[3];
      __syncthreads();  // wsum is rewritten by the next scan
    }
  }
}

// ---------------------------------------------------------------------------
// moments: grid (kChunks, G) x 256.  Wave w handles buckets 32c + 8w + j:
// members from the bitmap, two-pass moments of their keys; then the tile
// merge, thread = (dim k, bucket col) pairs of mean row k and var row 128+k.
// ---------------------------------------------------------------------------
constexpr int kMaxBlock = 4096;  // new tokens per update (LDS member list per wave)
constexpr int kMomBatch = 16;    // member key words requested at once

__device__ __forceinline__ float merge_mean(float a, float b, float den, float ma, float mb) {
#pragma clang fp contract(off)
  return (a * ma + b * mb) / den;
}
__device__ __forceinline__ float merge_var(float a, float b, float den, float ma, float mb, float va, float vb) {
#pragma clang fp contract(off)
  const float v = (a * va + b * vb) / den;
  const float d = ma - mb;
  return v + ((a * b) / (den * den)) * (d * d);
}

template <typename KT>
__global__ __launch_bounds__(kUT) void moments_kernel(UpdateArgs a) {
  const int c = blockIdx.x, g = blockIdx.y, tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  __shared__ float nm[kChunk][kD], nv[kChunk][kD];
  __shared__ int nb[kChunk];
  // the wave's member list, in dynamic LDS sized by the block (N tokens per
  // wave at most), so that several workgroups share a CU
  extern __shared__ int toks_all[];
  int* toks = toks_all + (size_t)w * a.N;
  const int w_lo = a.H >> 5, w_hi = (a.H + a.N - 1) >> 5;
  typedef KeyLoad<KT> KL;
  const KT* kg = static_cast<const KT*>(a.k) + (size_t)g * a.ks;
  // the first 64 bitmap words of the wave's 8 buckets, all requested at once
  // (the whole block's words up to 2016 tokens)
  constexpr int kCols = kChunk / 4;
  uint32_t first[kCols];
#pragma unroll
  for (int j = 0; j < kCols; ++j) {
    const int f = c * kChunk + w * kCols + j;
    const int wd = w_lo + lane;
    first[j] = f < kF && wd <= w_hi ? a.bits[((size_t)g * kF + f) * a.row_words + wd] : 0u;
  }
#pragma unroll
  for (int j = 0; j < kCols; ++j) {
    const int col = w * kCols + j, f = c * kChunk + col;
    int b = 0;
    if (f < kF) {
      const uint32_t* row = a.bits + ((size_t)g * kF + f) * a.row_words;
      for (int w0 = w_lo; w0 <= w_hi; w0 += 64) {
        const int wd = w0 + lane;
        uint32_t m = w0 == w_lo ? first[j] : (wd <= w_hi ? row[wd] : 0u);
        if (wd == w_lo) m &= ~0u << (a.H & 31);                               // tokens before H
        if (wd == w_hi && ((a.H + a.N) & 31)) m &= (1u << ((a.H + a.N) & 31)) - 1u;  // tokens past H+N
        const int pc = __popc(m);
        const int incl = (int)wave_incl_scan((unsigned)pc);
        int at = b + incl - pc;
        while (m) {
          toks[at++] = wd * 32 + (int)__builtin_ctz(m);
          m &= m - 1u;
        }
        b += __shfl(incl, 63);
      }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_s_waitcnt(0);
    // two-pass moments of the ORIGINAL keys (core.py:84-88); lane owns dims
    // 2l, 2l+1.  Members are summed in ascending order; their key words are
    // requested kMomBatch at a time, and a bucket of at most kMomBatch members
    // keeps them in registers for the second pass.
    auto key_word = [&](int i) { return KL::load2(kg + (size_t)toks[i] * kD + 2 * lane); };
    float s0 = 0.f, s1 = 0.f;
    typename KL::Raw2 kept[kMomBatch];
    for (int i0 = 0; i0 < b; i0 += kMomBatch) {  // uniform
      typename KL::Raw2 r[kMomBatch];
#pragma unroll
      for (int u = 0; u < kMomBatch; ++u) r[u] = key_word(min(i0 + u, b - 1));  // unconditional: one round trip
#pragma unroll
      for (int u = 0; u < kMomBatch; ++u) {
        if (i0 + u < b) {
          s0 += KL::lo(r[u]);
          s1 += KL::hi(r[u]);
        }
        kept[u] = r[u];
      }
    }
    const float m0 = b ? s0 / (float)b : 0.f, m1 = b ? s1 / (float)b : 0.f;
    float q0 = 0.f, q1 = 0.f;
    if (b <= kMomBatch) {
#pragma unroll
      for (int u = 0; u < kMomBatch; ++u)
        if (u < b) {
          const float d0 = KL::lo(kept[u]) - m0, d1 = KL::hi(kept[u]) - m1;
          q0 += d0 * d0;
          q1 += d1 * d1;
        }
    } else {
      for (int i0 = 0; i0 < b; i0 += kMomBatch) {
        typename KL::Raw2 r[kMomBatch];
#pragma unroll
        for (int u = 0; u < kMomBatch; ++u) r[u] = key_word(min(i0 + u, b - 1));
#pragma unroll
        for (int u = 0; u < kMomBatch; ++u)
          if (i0 + u < b) {
            const float d0 = KL::lo(r[u]) - m0, d1 = KL::hi(r[u]) - m1;
            q0 += d0 * d0;
            q1 += d1 * d1;
          }
      }
    }
    nm[col][2 * lane] = m0;
    nm[col][2 * lane + 1] = m1;
    nv[col][2 * lane] = b ? q0 / (float)b : 0.f;
    nv[col][2 * lane + 1] = b ? q1 / (float)b : 0.f;
    if (lane == 0) nb[col] = b;
    __builtin_amdgcn_wave_barrier();
  }
  __syncthreads();
  float* tile = a.moments + (size_t)(g * kChunks + c) * kRow * kChunk;
  const int col = tid & (kChunk - 1), f = c * kChunk + col;
  if (f >= kF) return;  // padding columns stay zero
  const int na = a.counts[(size_t)g * kFP + f], nbn = nb[col];
  const float fa = (float)na, fb = (float)nbn;
  const float total = fa + fb, den = total < 1.f ? 1.f : total;
  // every old mean and variance of the thread's 16 dims is requested before
  // the first merge, so the tile costs one memory round trip
  constexpr int kRowsPerThread = kD / (kUT / kChunk);  // 16
  float ma[kRowsPerThread], va[kRowsPerThread];
#pragma unroll
  for (int i = 0; i < kRowsPerThread; ++i) {
    const int k = (tid >> 5) + (kUT / kChunk) * i;
    ma[i] = tile[k * kChunk + col];
    va[i] = tile[(kD + k) * kChunk + col];
  }
#pragma unroll
  for (int i = 0; i < kRowsPerThread; ++i) {
    const int k = (tid >> 5) + (kUT / kChunk) * i;
    const float mb = nm[col][k], vb = nv[col][k];
    tile[k * kChunk + col] = merge_mean(fa, fb, den, ma[i], mb);
    tile[(kD + k) * kChunk + col] = merge_var(fa, fb, den, ma[i], mb, va[i], vb);
  }
  if (tid < kChunk) a.counts[(size_t)g * kFP + f] = na + nbn;
}

// ---------------------------------------------------------------------------
// Build-only kernels.
// center (build without a given center, core.py:95): keys.float().mean(0)
// over K rows [H, H + N).  center_part_kernel: grid (kCenterParts, G) x 256,
// part p sums rows [p R, (p + 1) R), R = ceil(N / kCenterParts), in double
// (thread = row step tid >> 4 of 16, dims 8 (tid & 15) ..);
// center_final_kernel: grid G x 128 adds the parts in order, divides by N.
// ---------------------------------------------------------------------------
template <typename KT>
__global__ __launch_bounds__(kUT) void center_part_kernel(UpdateArgs a, double* part) {
  const int p = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
  __shared__ double red[kUT / 16][kD];
  const int R = (a.N + kCenterParts - 1) / kCenterParts;
  const int lo = min(a.N, p * R), hi = min(a.N, lo + R);
  const int r = tid >> 4, d0 = (tid & 15) * 8;
  const KT* kg = static_cast<const KT*>(a.k) + (size_t)g * a.ks + (size_t)a.H * kD;
  double acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.0;
  for (int t = lo + r; t < hi; t += kUT / 16) {
    float x[8];
    KeyLoad<KT>::load8(kg + (size_t)t * kD + d0, x);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] += x[j];
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) red[r][d0 + j] = acc[j];
  __syncthreads();
  if (tid < kD) {
    double t = 0.0;
#pragma unroll
    for (int i = 0; i < kUT / 16; ++i) t += red[i][tid];
    part[((size_t)g * kCenterParts + p) * kD + tid] = t;
  }
}

__global__ __launch_bounds__(kD) void center_final_kernel(UpdateArgs a, const double* part, float* center) {
  const int g = blockIdx.x, d = threadIdx.x;
  double t = 0.0;
  for (int p = 0; p < kCenterParts; ++p) t += part[((size_t)g * kCenterParts + p) * kD + d];
  center[(size_t)g * kD + d] = (float)(t / (double)a.N);
}

// clear: grid (blocks, G) x 256 zeroes the group's F bitmap rows (row_words
// is a multiple of 4 words and the rows are 16-byte aligned).
__global__ __launch_bounds__(kUT) void clear_bits_kernel(UpdateArgs a) {
  const int g = blockIdx.y;
  const size_t n4 = (size_t)kF * a.row_words / 4;
  uint4* bg = reinterpret_cast<uint4*>(a.bits + (size_t)g * kF * a.row_words);
  for (size_t i = (size_t)blockIdx.x * kUT + threadIdx.x; i < n4; i += (size_t)gridDim.x * kUT)
    bg[i] = make_uint4(0u, 0u, 0u, 0u);
}

// ---------------------------------------------------------------------------
// build_moments: grid (F, G) x 256, one workgroup per bucket f, any member
// count.  Members are the set bits of the bucket's bitmap row below N (a
// build indexes K rows = bitmap columns [0, N)).  Chunks of 256 words (one
// per thread) are compacted into an LDS token list; while the whole list
// fits in kList tokens it is kept and both passes read it, otherwise each
// pass re-scans the row chunk by chunk.  Thread = (member slot tid >> 4 of
// 16, dims 8 (tid & 15) ..): 16 key rows per step with 16-byte loads,
// double accumulation, fixed order.  mean = sum / n rounded to fp32; var =
// sum (x - mean)^2 / n with that rounded mean; empty bucket -> 0
// (core.py:84-88).  Counts and moments are written, not merged.
// ---------------------------------------------------------------------------
constexpr int kList = 8192;
constexpr int kSlots = kUT / 16;

struct BuildMomentsLds {
  int toks[kList];
  double red[kSlots][kD];
  unsigned wsum[kUT / 64];
  float mean[kD];
};

// Members among words [w0, w0 + 256) of the row -> toks[at ..] when they all
// fit below kList.  Returns the chunk's member count (uniform); the caller
// barriers before the list is read and before the next chunk.
__device__ __forceinline__ unsigned compact_chunk(const uint32_t* row, int w0, int nw, int N, int* toks, unsigned at,
                                                  unsigned* wsum) {
  const int wd = w0 + threadIdx.x;
  uint32_t m = wd < nw ? row[wd] : 0u;
  if (wd == nw - 1 && (N & 31)) m &= (1u << (N & 31)) - 1u;
  const unsigned pc = (unsigned)__popc(m);
  const unsigned incl = block_incl_scan<kUT>(pc, wsum);
  const unsigned total = wsum[0] + wsum[1] + wsum[2] + wsum[3];
  if (at + total <= (unsigned)kList) {
    unsigned p = at + incl - pc;
    while (m) {
      toks[p++] = wd * 32 + (int)__builtin_ctz(m);
      m &= m - 1u;
    }
  }
  return total;
}

template <bool kDev, typename KT>
__device__ __forceinline__ void accumulate_rows(const KT* kg, const int* toks, unsigned n, int slot, int d0,
                                                const float (&m)[8], double (&acc)[8]) {
#pragma unroll 4
  for (unsigned i = slot; i < n; i += kSlots) {
    float x[8];
    KeyLoad<KT>::load8(kg + (size_t)toks[i] * kD + d0, x);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if constexpr (kDev) {
        const double t = (double)x[j] - (double)m[j];
        acc[j] += t * t;
      } else {
        acc[j] += (double)x[j];
      }
    }
  }
}

// One pass over the members (kDev: squared deviations from m), reduced over
// the slots into red[0][..] order-fixed sums for tid < kD (returned).
template <bool kDev, typename KT>
__device__ double bucket_pass(BuildMomentsLds& L, const uint32_t* row, const KT* kg, int nw, int N, bool kept,
                              unsigned n, const float (&m)[8]) {
  const int tid = threadIdx.x, slot = tid >> 4, d0 = (tid & 15) * 8;
  double acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.0;
  if (kept) {
    accumulate_rows<kDev>(kg, L.toks, n, slot, d0, m, acc);
  } else {
    for (int w0 = 0; w0 < nw; w0 += kUT) {
      __syncthreads();  // the previous chunk's list has been read
      const unsigned c = compact_chunk(row, w0, nw, N, L.toks, 0u, L.wsum);  // <= 8192: always fits
      __syncthreads();
      accumulate_rows<kDev>(kg, L.toks, c, slot, d0, m, acc);
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) L.red[slot][d0 + j] = acc[j];
  __syncthreads();
  double t = 0.0;
  if (tid < kD)
#pragma unroll
    for (int i = 0; i < kSlots; ++i) t += L.red[i][tid];
  __syncthreads();  // red is free again
  return t;
}

template <typename KT>
__global__ __launch_bounds__(kUT) void build_moments_kernel(UpdateArgs a) {
  const int f = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
  __shared__ BuildMomentsLds L;
  const uint32_t* row = a.bits + ((size_t)g * kF + f) * a.row_words;
  const KT* kg = static_cast<const KT*>(a.k) + (size_t)g * a.ks;
  const int nw = (a.N + 31) >> 5;
  // count the members, keeping the list while it fits
  unsigned n = 0;
  bool kept = true;
  for (int w0 = 0; w0 < nw; w0 += kUT) {
    const unsigned c = compact_chunk(row, w0, nw, a.N, L.toks, n, L.wsum);
    __syncthreads();
    if (n + c > (unsigned)kList) {
      kept = false;
      n = 0;
      for (int w1 = 0; w1 < nw; w1 += kUT) {  // count only: the list is rebuilt per chunk in the passes
        const int wd = w1 + tid;
        uint32_t m = wd < nw ? row[wd] : 0u;
        if (wd == nw - 1 && (a.N & 31)) m &= (1u << (a.N & 31)) - 1u;
        block_incl_scan<kUT>((unsigned)__popc(m), L.wsum);
        n += L.wsum[0] + L.wsum[1] + L.wsum[2] + L.wsum[3];
        __syncthreads();
      }
      break;
    }
    n += c;
  }
  float zero[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) zero[j] = 0.f;
  const double sum = bucket_pass<false>(L, row, kg, nw, a.N, kept, n, zero);
  if (tid < kD) L.mean[tid] = n ? (float)(sum / (double)n) : 0.f;
  __syncthreads();
  float m[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) m[j] = L.mean[(tid & 15) * 8 + j];
  const double dev = bucket_pass<true>(L, row, kg, nw, a.N, kept, n, m);
  if (tid < kD) {
    float* tile = a.moments + (size_t)(g * kChunks + f / kChunk) * kRow * kChunk;
    const int col = f % kChunk;
    tile[tid * kChunk + col] = L.mean[tid];
    tile[(kD + tid) * kChunk + col] = n ? (float)(dev / (double)n) : 0.f;
  }
  if (tid == 0) a.counts[(size_t)g * kFP + f] = (int)n;
}

// ---------------------------------------------------------------------------
// positive_global_topk on a given [N][F] fp32 matrix (core.py:13-26), for
// callers of the Python surface: the same threshold kernels (digit / refine)
// after a level-0 histogram, then the flat indices in the reference's order
// -- every strict value (a > tau and a > 0; every positive one when fewer
// than the budget are positive) in ascending flat index, then the first
// `need` values equal to tau in ascending flat index.  The matrix is cut
// into the contiguous ranges of the tie kernels; flat_count_kernel counts
// each range's strict values and ties (tcount[2r], tcount[2r + 1]),
// flat_emit_kernel writes them after the lower ranges' ones.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kUT) void hist0_kernel(UpdateArgs a) {
  const int g = blockIdx.y, tid = threadIdx.x;
  __shared__ unsigned hist[kBins];
  for (int i = tid; i < kBins; i += kUT) hist[i] = 0;
  __syncthreads();
  const size_t n = (size_t)a.N * kF;
  const float4* ag = reinterpret_cast<const float4*>(a.act + (size_t)g * n);
  for (size_t i = (size_t)blockIdx.x * kUT + tid; i < n / 4; i += (size_t)gridDim.x * kUT) {
    const float4 v4 = ag[i];
    const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (vv[j] > 0.f) atomicAdd(&hist[__float_as_uint(vv[j]) >> 20], 1u);
  }
  __syncthreads();
  unsigned* hg = hist_of(a, g, 0) + (blockIdx.x % kRep) * kBins;
  for (int i = tid; i < kBins; i += kUT)
    if (hist[i]) atomicAdd(&hg[i], hist[i]);
}

struct FlatRule {
  float tau;
  bool all_pos, ties;
  __device__ bool strict(float v) const { return all_pos ? v > 0.f : (v > tau && v > 0.f); }
  __device__ bool tie(float v) const { return ties && v == tau; }
};

__device__ __forceinline__ FlatRule flat_rule(const UpdateArgs& a, int g) {
  const unsigned* ctl = a.ctl + (size_t)g * kCtl;
  FlatRule r;
  r.tau = __uint_as_float(ctl[kTau]);  // +inf (nothing) for an empty budget
  r.all_pos = ctl[kMode] == kModeAllPositive;
  r.ties = !r.all_pos && r.tau > 0.f && ctl[kTau] != 0x7f800000u;
  return r;
}

__global__ __launch_bounds__(kUT) void flat_count_kernel(UpdateArgs a) {
  const int g = blockIdx.y, tid = threadIdx.x;
  __shared__ unsigned wsum[kUT / 64];
  const FlatRule rule = flat_rule(a, g);
  const size_t n = (size_t)a.N * kF;
  const float4* ag = reinterpret_cast<const float4*>(a.act + (size_t)g * n);
  for (int r = blockIdx.x; r < a.tie_blocks; r += gridDim.x) {  // uniform
    const size_t lo = min(n, (size_t)r * a.tie_len), hi = min(n, lo + a.tie_len);
    unsigned cs = 0, ct = 0;
    for (size_t i = lo / 4 + tid; i < hi / 4; i += kUT) {
      const float4 v = ag[i];
      const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        cs += rule.strict(vv[j]);
        ct += rule.tie(vv[j]);
      }
    }
    block_incl_scan<kUT>(cs, wsum);
    if (tid == 0) a.tcount[((size_t)g * a.tie_blocks + r) * 2] = wsum[0] + wsum[1] + wsum[2] + wsum[3];
    __syncthreads();
    block_incl_scan<kUT>(ct, wsum);
    if (tid == 0) a.tcount[((size_t)g * a.tie_blocks + r) * 2 + 1] = wsum[0] + wsum[1] + wsum[2] + wsum[3];
    __syncthreads();
  }
}

__global__ __launch_bounds__(kUT) void flat_emit_kernel(UpdateArgs a, int64_t* out, int* out_len) {
  const int g = blockIdx.y, tid = threadIdx.x;
  __shared__ unsigned wsum[kUT / 64];
  const FlatRule rule = flat_rule(a, g);
  const unsigned need = rule.ties ? a.ctl[(size_t)g * kCtl + kNeed] : 0u;
  const unsigned* tc = a.tcount + (size_t)g * a.tie_blocks * 2;
  // all strict values come first: their total over every range
  unsigned all_s = 0, all_t = 0;
  for (int j = tid; j < a.tie_blocks; j += kUT) {
    all_s += tc[2 * j];
    all_t += tc[2 * j + 1];
  }
  block_incl_scan<kUT>(all_s, wsum);
  const unsigned strict_total = wsum[0] + wsum[1] + wsum[2] + wsum[3];
  __syncthreads();
  block_incl_scan<kUT>(all_t, wsum);
  const unsigned ties_total = wsum[0] + wsum[1] + wsum[2] + wsum[3];
  __syncthreads();
  if (blockIdx.x == 0 && tid == 0) out_len[g] = (int)(strict_total + min(ties_total, need));
  const size_t n = (size_t)a.N * kF;
  const float4* ag = reinterpret_cast<const float4*>(a.act + (size_t)g * n);
  for (int r = blockIdx.x; r < a.tie_blocks; r += gridDim.x) {  // uniform
    unsigned bs = 0, bt = 0;
    for (int j = tid; j < r; j += kUT) {
      bs += tc[2 * j];
      bt += tc[2 * j + 1];
    }
    block_incl_scan<kUT>(bs, wsum);
    unsigned at_s = wsum[0] + wsum[1] + wsum[2] + wsum[3];
    __syncthreads();
    block_incl_scan<kUT>(bt, wsum);
    unsigned at_t = wsum[0] + wsum[1] + wsum[2] + wsum[3];
    __syncthreads();
    const size_t lo = min(n, (size_t)r * a.tie_len), hi = min(n, lo + a.tie_len);
    for (size_t base = lo / 4; base < hi / 4; base += kUT) {  // uniform
      const size_t i = base + tid;
      const float4 v = i < hi / 4 ? ag[i] : make_float4(0.f, 0.f, 0.f, 0.f);
      const float vv[4] = {v.x, v.y, v.z, v.w};
      bool hs[4], ht[4];
      unsigned cs = 0, ct = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        hs[j] = i < hi / 4 && rule.strict(vv[j]);
        ht[j] = i < hi / 4 && rule.tie(vv[j]);
        cs += hs[j];
        ct += ht[j];
      }
      const unsigned is = block_incl_scan<kUT>(cs, wsum);
      const unsigned ts = wsum[0] + wsum[1] + wsum[2] + wsum[3];
      __syncthreads();
      const unsigned it = block_incl_scan<kUT>(ct, wsum);
      const unsigned tt = wsum[0] + wsum[1] + wsum[2] + wsum[3];
      __syncthreads();
      unsigned ks = at_s + is - cs, kt = at_t + it - ct;  // ranks of this thread's first strict value / tie
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t flat = (int64_t)(4 * i + j);
        if (hs[j]) out[ks++] = flat;
        if (ht[j]) {
          if (kt < need) out[strict_total + kt] = flat;
          ++kt;
        }
      }
      at_s += ts;
      at_t += tt;
    }
  }
}

}  // namespace
}  // namespace prismkv

using namespace prismkv;

// Work layout (bytes) for `groups` groups and blocks of N keys: the regions
// that must start at zero (histograms, control words) and the other scratch
// first, at offsets that depend on the group count only, then the block's
// activations [groups][N][3000] f32 and the compact candidate list
// [groups][list_cap] (sized by N).  A workspace sized for the largest block
// therefore serves every smaller block: no call finds another call's
// activations or list where it expects zeroed histograms.
struct UpdateLayout {
  size_t hist, ctl, tcount, part, act, list, total;
  unsigned list_cap;
  UpdateLayout(int groups, int N) {
    size_t o = 0;
    auto take = [&](size_t n) { const size_t at = o; o += (n + 255) & ~(size_t)255; return at; };
    hist = take((size_t)groups * kLevels * kRep * kBins * sizeof(unsigned));
    ctl = take((size_t)groups * kCtl * sizeof(unsigned));
    tcount = take((size_t)groups * kMaxTieBlocks * 2 * sizeof(unsigned));
    part = take((size_t)groups * kCenterParts * kD * sizeof(double));
    act = take((size_t)groups * N * kF * sizeof(float));
    // the compact list: room for 16 candidates per key (twice the 8 H
    // budget of an index build) plus the chunk tails, at least 2^19
    list_cap = N > 0 ? std::max(1u << 19, 16u * (unsigned)N + kListSlack) : 0u;
    list = take((size_t)groups * list_cap * sizeof(uint2));
    total = o;
  }
};

static UpdateArgs make_args(uint64_t k, uint64_t W, uint64_t b, uint64_t center, uint64_t scale, uint64_t bits,
                            uint64_t counts, uint64_t moments, uint64_t work, int groups, int H, int N, int key_mean,
                            int64_t ks, int64_t row_words, const UpdateLayout& L) {
  char* w = reinterpret_cast<char*>(work);
  UpdateArgs a;
  a.k = reinterpret_cast<const void*>(k);
  a.ks = ks;
  a.W = reinterpret_cast<const float*>(W);
  a.b = reinterpret_cast<const float*>(b);
  a.center = reinterpret_cast<const float*>(center);
  a.scale = reinterpret_cast<const float*>(scale);
  a.bits = reinterpret_cast<uint32_t*>(bits);
  a.row_words = row_words;
  a.counts = reinterpret_cast<int*>(counts);
  a.moments = reinterpret_cast<float*>(moments);
  a.act = reinterpret_cast<float*>(w + L.act);
  a.hist = reinterpret_cast<unsigned*>(w + L.hist);
  a.ctl = reinterpret_cast<unsigned*>(w + L.ctl);
  a.tcount = reinterpret_cast<unsigned*>(w + L.tcount);
  a.list = reinterpret_cast<uint2*>(w + L.list);
  a.list_cap = L.list_cap;
  a.H = H;
  a.N = N;
  a.budget = (long long)N * key_mean;
  // ordered-tie ranges: at most kMaxTieBlocks per group, each a multiple of 4 * kUT values
  const long long n = (long long)N * kF;
  long long len = std::max<long long>(kTieMinLen, (n + kMaxTieBlocks - 1) / kMaxTieBlocks);
  len = (len + 4 * kUT - 1) / (4 * kUT) * (4 * kUT);
  a.tie_len = len;
  a.tie_blocks = (int)((n + len - 1) / len);
  (void)groups;
  return a;
}

// encode .. ties: the exact batch-wide positive Top-k of the N keys' activations
// and their bitmap bits.
template <typename KT>
static void launch_selection(const UpdateArgs& a, int groups, hipStream_t s) {
  const int token_tiles = (a.N + kEncTokens - 1) / kEncTokens;
  const int parts = std::max(1, std::min(kFTiles, (kEncMinWgs + token_tiles * groups - 1) / (token_tiles * groups)));
  hipLaunchKernelGGL(encode_kernel<KT>, dim3(token_tiles, parts, groups), dim3(kET), 0, s, a);
  hipLaunchKernelGGL(digit_kernel, dim3(groups), dim3(kUT), 0, s, a, 0);
  for (int level = 1; level < kLevels; ++level) {
    hipLaunchKernelGGL(refine_kernel, dim3(kRefineBlocks, groups), dim3(kUT), 0, s, a, level);
    hipLaunchKernelGGL(digit_kernel, dim3(groups), dim3(kUT), 0, s, a, level);
  }
  hipLaunchKernelGGL(emit_kernel, dim3(kRefineBlocks, groups), dim3(kUT), 0, s, a);
  const int tie_grid = std::min(a.tie_blocks, kTieGrid);
  hipLaunchKernelGGL(tie_count_kernel, dim3(tie_grid, groups), dim3(kUT), 0, s, a);
  hipLaunchKernelGGL(tie_take_kernel, dim3(tie_grid, groups), dim3(kUT), 0, s, a);
}

template <typename KT>
static bool aligned16(uint64_t p, int64_t stride_elems) {
  return ((p | (uint64_t)(stride_elems * (int64_t)sizeof(KT))) & 15u) == 0;
}

template <typename KT>
static int update_impl(uint64_t k, uint64_t W, uint64_t b, uint64_t center, uint64_t scale, uint64_t bits,
                       uint64_t counts, uint64_t moments, uint64_t work, int groups, int H, int N, int key_mean,
                       int64_t ks, int64_t row_words, size_t work_bytes, uint64_t stream) {
  if (groups < 1 || groups > 65535 || H < 0 || N < 1 || N > kMaxBlock || key_mean < 1 || key_mean > kF)
    return kBadSize;
  if (ks < (int64_t)(H + N) * kD || row_words < (H + N + 31) / 32) return kBadSize;
  if (!k || !W || !b || !center || !scale || !bits || !counts || !moments || !work) return kBadSize;
  if (!aligned16<KT>(k, ks) || ((W | b) & 15u)) return kBadSize;
  const UpdateLayout L(groups, N);
  if (work_bytes < L.total) return kBadSize;  // prismkv_update_work_bytes(groups, N)
  const UpdateArgs a = make_args(k, W, b, center, scale, bits, counts, moments, work, groups, H, N, key_mean, ks,
                                 row_words, L);
  hipStream_t s = (hipStream_t)stream;
  launch_selection<KT>(a, groups, s);
  // member lists: N ints per wave of dynamic LDS (up to 64 KB, allowed once per key type)
  static const hipError_t lds_ok = hipFuncSetAttribute(reinterpret_cast<const void*>(moments_kernel<KT>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                                       (int)(kUT / 64 * kMaxBlock * sizeof(int)));
  if (lds_ok != hipSuccess) return (int)lds_ok;
  hipLaunchKernelGGL(moments_kernel<KT>, dim3(kChunks, groups), dim3(kUT), (size_t)(kUT / 64) * N * sizeof(int), s,
                     a);
  return (int)hipGetLastError();
}

template <typename KT>
static int build_impl(uint64_t k, uint64_t W, uint64_t b, uint64_t center, uint64_t scale, uint64_t bits,
                      uint64_t counts, uint64_t moments, uint64_t work, int groups, int batch, int H, int key_mean,
                      int flags, int64_t ks, int64_t row_words, size_t work_bytes, uint64_t stream) {
  if (groups < 1 || groups > 65535 || batch < 1 || batch > groups || H < 1 || H > kMaxBuild || key_mean < 1 ||
      key_mean > kF)
    return kBadSize;
  if (flags & ~kBuildCenter) return kBadMode;
  if (ks < (int64_t)H * kD || row_words < (H + 31) / 32 || (row_words & 3)) return kBadSize;
  if (!k || !W || !b || !center || !scale || !bits || !counts || !moments || !work) return kBadSize;
  if (!aligned16<KT>(k, ks) || ((bits | W | b) & 15u)) return kBadSize;
  const UpdateLayout L(batch, H);
  if (work_bytes < L.total) return kBadSize;  // prismkv_build_work_bytes(batch, H)
  hipStream_t s = (hipStream_t)stream;
  for (int g0 = 0; g0 < groups; g0 += batch) {
    const int nb = std::min(batch, groups - g0);
    const uint64_t kg = k + (uint64_t)g0 * ks * sizeof(KT);
    const uint64_t cg = center + (uint64_t)g0 * kD * sizeof(float);
    UpdateArgs a = make_args(kg, W + (uint64_t)g0 * kF * kD * sizeof(float), b + (uint64_t)g0 * kF * sizeof(float),
                             cg, scale + (uint64_t)g0 * sizeof(float),
                             bits + (uint64_t)g0 * kF * row_words * sizeof(uint32_t),
                             counts + (uint64_t)g0 * kFP * sizeof(int),
                             moments + (uint64_t)g0 * kChunks * kRow * kChunk * sizeof(float), work, nb, 0, H,
                             key_mean, ks, row_words, L);
    if (flags & kBuildCenter) {
      double* part = reinterpret_cast<double*>(reinterpret_cast<char*>(work) + L.part);
      hipLaunchKernelGGL(center_part_kernel<KT>, dim3(kCenterParts, nb), dim3(kUT), 0, s, a, part);
      hipLaunchKernelGGL(center_final_kernel, dim3(nb), dim3(kD), 0, s, a, (const double*)part,
                         reinterpret_cast<float*>(cg));
    }
    hipLaunchKernelGGL(clear_bits_kernel, dim3(512, nb), dim3(kUT), 0, s, a);
    launch_selection<KT>(a, nb, s);
    hipLaunchKernelGGL(build_moments_kernel<KT>, dim3(kF, nb), dim3(kUT), 0, s, a);
  }
  return (int)hipGetLastError();
}

template <typename KT>
static int summarize_impl(uint64_t k, uint64_t bits, uint64_t center, uint64_t counts, uint64_t moments,
                          uint64_t work, int groups, int H, int flags, int64_t ks, int64_t row_words,
                          size_t work_bytes, uint64_t stream) {
  if (groups < 1 || groups > 65535 || H < 1 || H > kMaxBuild) return kBadSize;
  if (flags & ~kBuildCenter) return kBadMode;
  if (ks < (int64_t)H * kD || row_words < (H + 31) / 32) return kBadSize;
  if (!k || !bits || !center || !counts || !moments || !work || !aligned16<KT>(k, ks)) return kBadSize;
  const UpdateLayout L(groups, 0);
  if (work_bytes < L.total) return kBadSize;  // prismkv_summarize_work_bytes(groups)
  const UpdateArgs a = make_args(k, 0, 0, center, 0, bits, counts, moments, work, groups, 0, H, 1, ks, row_words, L);
  hipStream_t s = (hipStream_t)stream;
  if (flags & kBuildCenter) {
    double* part = reinterpret_cast<double*>(reinterpret_cast<char*>(work) + L.part);
    hipLaunchKernelGGL(center_part_kernel<KT>, dim3(kCenterParts, groups), dim3(kUT), 0, s, a, part);
    hipLaunchKernelGGL(center_final_kernel, dim3(groups), dim3(kD), 0, s, a, (const double*)part,
                       reinterpret_cast<float*>(center));
  }
  hipLaunchKernelGGL(build_moments_kernel<KT>, dim3(kF, groups), dim3(kUT), 0, s, a);
  return (int)hipGetLastError();
}

extern "C" {

size_t prismkv_update_work_bytes(int groups, int max_block) {
  if (groups < 1 || groups > 65535 || max_block < 1 || max_block > kMaxBlock) return 0;
  return UpdateLayout(groups, max_block).total;
}

size_t prismkv_update_act_offset(int groups) {
  if (groups < 1 || groups > 65535) return 0;
  return UpdateLayout(groups, 0).act;
}

int prismkv_update(uint64_t k, uint64_t W, uint64_t b, uint64_t center, uint64_t scale, uint64_t bits,
                   uint64_t counts, uint64_t moments, uint64_t work, int groups, int H, int N, int key_mean,
                   int64_t ks, int64_t row_words, size_t work_bytes, uint64_t stream) {
  return update_impl<uint16_t>(k, W, b, center, scale, bits, counts, moments, work, groups, H, N, key_mean, ks,
                               row_words, work_bytes, stream);
}

int prismkv_update_f32(uint64_t k, uint64_t W, uint64_t b, uint64_t center, uint64_t scale, uint64_t bits,
                       uint64_t counts, uint64_t moments, uint64_t work, int groups, int H, int N, int key_mean,
                       int64_t ks, int64_t row_words, size_t work_bytes, uint64_t stream) {
  return update_impl<float>(k, W, b, center, scale, bits, counts, moments, work, groups, H, N, key_mean, ks,
                            row_words, work_bytes, stream);
}

size_t prismkv_build_work_bytes(int batch, int H) {
  if (batch < 1 || batch > 65535 || H < 1 || H > kMaxBuild) return 0;
  return UpdateLayout(batch, H).total;
}

int prismkv_build(uint64_t k, uint64_t W, uint64_t b, uint64_t center, uint64_t scale, uint64_t bits,
                  uint64_t counts, uint64_t moments, uint64_t work, int groups, int batch, int H, int key_mean,
                  int flags, int64_t ks, int64_t row_words, size_t work_bytes, uint64_t stream) {
  return build_impl<uint16_t>(k, W, b, center, scale, bits, counts, moments, work, groups, batch, H, key_mean, flags,
                              ks, row_words, work_bytes, stream);
}

int prismkv_build_f32(uint64_t k, uint64_t W, uint64_t b, uint64_t center, uint64_t scale, uint64_t bits,
                      uint64_t counts, uint64_t moments, uint64_t work, int groups, int batch, int H, int key_mean,
                      int flags, int64_t ks, int64_t row_words, size_t work_bytes, uint64_t stream) {
  return build_impl<float>(k, W, b, center, scale, bits, counts, moments, work, groups, batch, H, key_mean, flags,
                           ks, row_words, work_bytes, stream);
}

size_t prismkv_topk_work_bytes(void) { return UpdateLayout(1, 0).total; }

int prismkv_topk(uint64_t act, uint64_t out, uint64_t out_len, uint64_t work, int N, int64_t count,
                 size_t work_bytes, uint64_t stream) {
  if (N < 1 || N > kMaxBuild || count < 0) return kBadSize;
  if (!act || !out || !out_len || !work || (act & 15u)) return kBadSize;
  const UpdateLayout L(1, 0);
  if (work_bytes < L.total) return kBadSize;  // prismkv_topk_work_bytes()
  const int64_t n = (int64_t)N * kF;
  UpdateArgs a = make_args(0, 0, 0, 0, 0, 0, 0, 0, work, 1, 0, N, 1, 0, 0, L);
  a.act = reinterpret_cast<float*>(act);  // read only here
  a.budget = count < n ? count : n;
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(hist0_kernel, dim3(kRefineBlocks, 1), dim3(kUT), 0, s, a);
  hipLaunchKernelGGL(digit_kernel, dim3(1), dim3(kUT), 0, s, a, 0);
  for (int level = 1; level < kLevels; ++level) {
    hipLaunchKernelGGL(refine_kernel, dim3(kRefineBlocks, 1), dim3(kUT), 0, s, a, level);
    hipLaunchKernelGGL(digit_kernel, dim3(1), dim3(kUT), 0, s, a, level);
  }
  const int grid = std::min(a.tie_blocks, kTieGrid);
  hipLaunchKernelGGL(flat_count_kernel, dim3(grid, 1), dim3(kUT), 0, s, a);
  hipLaunchKernelGGL(flat_emit_kernel, dim3(grid, 1), dim3(kUT), 0, s, a, reinterpret_cast<int64_t*>(out),
                     reinterpret_cast<int*>(out_len));
  return (int)hipGetLastError();
}

size_t prismkv_summarize_work_bytes(int groups) {
  if (groups < 1 || groups > 65535) return 0;
  return UpdateLayout(groups, 0).total;
}

int prismkv_summarize(uint64_t k, uint64_t bits, uint64_t center, uint64_t counts, uint64_t moments, uint64_t work,
                      int groups, int H, int flags, int64_t ks, int64_t row_words, size_t work_bytes,
                      uint64_t stream) {
  return summarize_impl<uint16_t>(k, bits, center, counts, moments, work, groups, H, flags, ks, row_words, work_bytes,
                                  stream);
}

int prismkv_summarize_f32(uint64_t k, uint64_t bits, uint64_t center, uint64_t counts, uint64_t moments,
                          uint64_t work, int groups, int H, int flags, int64_t ks, int64_t row_words,
                          size_t work_bytes, uint64_t stream) {
  return summarize_impl<float>(k, bits, center, counts, moments, work, groups, H, flags, ks, row_words, work_bytes,
                               stream);
}

}  // extern "C"
