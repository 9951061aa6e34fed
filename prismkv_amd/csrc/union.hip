// Stage 2 -- union: OR the membership bitmap rows of the selected buckets and
// compact the set bits into an ascending token-ID list.  Also the bitmap
// build (CSR lists -> bits) used at index construction.
//
// Semantics: kernels/ppu_8b/union.cu:14-27 (OR of rows with valid > 0,
//            ascending emission of w*32+bit), kernels/ppu_8b/pack.cu:5 (bit
//            order: token t <-> word t>>5, bit t&31), src/prismkv/core.py:142-167.
//
// Design: one launch.  Workgroup (tile, group) ORs up to 16 rows over its
// 256 x WPT words (coalesced 4 or 16 bytes per lane), counts bits, and finds
// its output offset with a decoupled look-back over the preceding tiles of the
// same group (status words in caller-provided work memory, tiles only wait on
// lower-numbered tiles, which the in-order dispatcher has already started;
// the wait is bounded and reports through an error word instead of hanging).
// The last tile to finish restores the status words to zero, so the launch
// is replayable from a graph without memset nodes.
#include "common.h"

namespace prismkv {
namespace {

constexpr int kUT = 256;                 // union workgroup size
constexpr unsigned kFlagAgg = 1u << 30;  // status: tile aggregate available
constexpr unsigned kFlagInc = 2u << 30;  // status: inclusive prefix available
constexpr unsigned kValMask = (1u << 30) - 1;
constexpr int kSpinLimit = 1 << 20;

struct UnionWork {
  unsigned* status;  // [groups][tiles]
  unsigned* done;    // [groups]
  unsigned* err;     // [1]
};

__host__ __device__ inline int union_tiles(int H, int wpt) {
  const int nw = (H + 31) / 32;
  const int tw = kUT * wpt;
  return (nw + tw - 1) / tw;
}

template <int WPT>
__global__ __launch_bounds__(kUT) void union_kernel(const uint32_t* __restrict__ bits, int64_t row_words,
                                                    const int64_t* __restrict__ features,
                                                    const float* __restrict__ valid, int32_t* __restrict__ ids,
                                                    int64_t ids_stride, int32_t* __restrict__ count, UnionWork work,
                                                    int H, int tiles) {
  const int t = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
  __shared__ int rows[kTop];
  __shared__ int nrows;
  __shared__ unsigned wsum[kUT / 64];
  __shared__ unsigned base;
  if (tid == 0) {
    int n = 0;
    for (int j = 0; j < kTop; ++j)
      if (valid[(size_t)g * kTop + j] > 0.f) {
        const int64_t f = features[(size_t)g * kTop + j];
        if (f >= 0 && f < kF) rows[n++] = (int)f;  // an out-of-range id selects nothing
      }
    nrows = n;
  }
  __syncthreads();
  const int nw = (H + 31) / 32;
  const int w0 = (t * kUT + tid) * WPT;
  uint32_t m[WPT];
#pragma unroll
  for (int i = 0; i < WPT; ++i) m[i] = 0;
  const uint32_t* gb = bits + (size_t)g * kF * row_words;
  const int nr = nrows;
  if (w0 + WPT <= nw) {
    for (int r = 0; r < nr; ++r) {
      const uint32_t* src = gb + (size_t)rows[r] * row_words + w0;
      if constexpr (WPT == 4) {
        const uint4 v = load_nt16(src);
        m[0] |= v.x; m[1] |= v.y; m[2] |= v.z; m[3] |= v.w;
      } else {
#pragma unroll
        for (int i = 0; i < WPT; ++i) m[i] |= __builtin_nontemporal_load(src + i);
      }
    }
  } else {
    for (int r = 0; r < nr; ++r) {
      const uint32_t* src = gb + (size_t)rows[r] * row_words;
#pragma unroll
      for (int i = 0; i < WPT; ++i)
        if (w0 + i < nw) m[i] |= src[w0 + i];
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
  const unsigned incl = block_incl_scan<kUT>(n, wsum);
  const unsigned excl = incl - n;

  if (tid == kUT - 1) {
    // incl of the last thread is the tile total
    unsigned* st = work.status + (size_t)g * tiles;
    const unsigned total = incl;
    unsigned prefix = 0;
    if (t == 0) {
      atomic_store_agent(&st[0], kFlagInc | total);
    } else {
      atomic_store_agent(&st[t], kFlagAgg | total);
      int p = t - 1;
      while (p >= 0) {
        unsigned s = atomic_load_agent(&st[p]);
        int spins = 0;
        while ((s >> 30) == 0 && spins < kSpinLimit) {
          __builtin_amdgcn_s_sleep(1);
          s = atomic_load_agent(&st[p]);
          ++spins;
        }
        if ((s >> 30) == 0) {  // predecessor never published: report, do not hang
          atomicOr(work.err, 1u);
          break;
        }
        prefix += s & kValMask;
        if ((s >> 30) == 2u) break;
        --p;
      }
      atomic_store_agent(&st[t], kFlagInc | ((prefix + total) & kValMask));
    }
    base = prefix;
    if (t == tiles - 1) count[g] = (int32_t)(prefix + total);
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
  // last tile of the group to get here clears the status words for reuse
  if (tid == kUT - 1) {
    if (atomic_add_agent(&work.done[g], 1u) == (unsigned)(tiles - 1)) {
      unsigned* st = work.status + (size_t)g * tiles;
      for (int i = 0; i < tiles; ++i) atomic_store_agent(&st[i], 0u);
      atomic_store_agent(&work.done[g], 0u);
    }
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
    for (int j = 0; j < kTop; ++j)
      if (vals[u * kTop + j] > 0.f) v |= bits[((size_t)u * kF + ids[u * kTop + j]) * nw + w];
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

}  // namespace
}  // namespace prismkv

using namespace prismkv;

// 16-byte row loads once a group has at least 8 such tiles and rows are 16-byte aligned.
static int union_wpt(int H, int64_t row_words) {
  return ((H + 31) / 32) >= 8 * kUT * 4 && (row_words & 3) == 0 ? 4 : 1;
}

extern "C" {

size_t prismkv_union_work_bytes(int groups, int H) {
  if (groups < 1 || H < 1) return 0;
  const int tiles = union_tiles(H, 1);  // the largest tile count of any variant
  return ((size_t)groups * tiles + groups + 1) * sizeof(unsigned);
}

int prismkv_union(uint64_t bits, uint64_t features, uint64_t valid, uint64_t work, uint64_t ids, uint64_t count,
                  int groups, int H, int64_t row_words, int64_t ids_stride, uint64_t stream) {
  if (groups < 1 || groups > 65535 || H < 1 || H > (1 << 29)) return kBadSize;
  if (row_words < (H + 31) / 32 || ids_stride < H) return kBadSize;
  if (!bits || !features || !valid || !work || !ids || !count) return kBadSize;
  const int wpt = union_wpt(H, row_words);
  const int tiles = union_tiles(H, wpt);
  unsigned* w = reinterpret_cast<unsigned*>(work);
  UnionWork uw{w, w + (size_t)groups * tiles, w + (size_t)groups * tiles + groups};
  const dim3 grid(tiles, groups), block(kUT);
  if (wpt == 4)
    hipLaunchKernelGGL(union_kernel<4>, grid, block, 0, (hipStream_t)stream,
                       reinterpret_cast<const uint32_t*>(bits), row_words, reinterpret_cast<const int64_t*>(features),
                       reinterpret_cast<const float*>(valid), reinterpret_cast<int32_t*>(ids), ids_stride,
                       reinterpret_cast<int32_t*>(count), uw, H, tiles);
  else
    hipLaunchKernelGGL(union_kernel<1>, grid, block, 0, (hipStream_t)stream,
                       reinterpret_cast<const uint32_t*>(bits), row_words, reinterpret_cast<const int64_t*>(features),
                       reinterpret_cast<const float*>(valid), reinterpret_cast<int32_t*>(ids), ids_stride,
                       reinterpret_cast<int32_t*>(count), uw, H, tiles);
  return (int)hipGetLastError();
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
