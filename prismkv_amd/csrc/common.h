// Shared constants and device helpers for the PrismKV routed-decode kernels
// (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace prismkv {

// Qwen3-8B native geometry (src/prismkv/native8b.py:1-6).
constexpr int kF = 3000;         // SAE feature buckets per KV group
constexpr int kD = 128;          // head dimension
constexpr int kHq = 4;           // query heads per KV group
constexpr int kTop = 16;         // selected buckets per group
constexpr int kChunk = 32;       // buckets per moment tile (128-byte tile rows)
constexpr int kChunks = (kF + kChunk - 1) / kChunk;  // 94
constexpr int kFP = kChunks * kChunk;                // 3008, padded bucket count
constexpr int kRow = 2 * kD;     // per-bucket moment row: mean[128] then var[128]

// Error convention of the C ABI (kernels/ppu_8b/union.cu:40,47, av_tuned.cu:63,65).
constexpr int kBadSize = -1;
constexpr int kBadMode = -2;

__device__ __forceinline__ float bf16_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
// An input element (bf16 bits or fp32) as fp32: the widening is exact.
__device__ __forceinline__ float to_f32(uint16_t h) { return bf16_to_f32(h); }
__device__ __forceinline__ float to_f32(float x) { return x; }

// fp32 -> bf16, round to nearest even, NaN kept quiet.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// 16-byte streaming load (non-temporal hint: data read once per decode step).
__device__ __forceinline__ uint4 load_nt16(const void* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// 16-byte streaming load through a raw buffer resource (gfx9 resource word 3
// 0x00020000: 32-bit data format; aux 2: non-temporal).  The 32-bit offset
// takes one address register per load instead of two.
__device__ __forceinline__ uint4 load_nt16_buf(__amdgpu_buffer_rsrc_t r, unsigned byte_offset) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_offset, 0, 2);
  return make_uint4(v.x, v.y, v.z, v.w);
}
// 4-byte streaming load through a raw buffer resource.
__device__ __forceinline__ uint32_t load_nt4_buf(__amdgpu_buffer_rsrc_t r, unsigned byte_offset) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, byte_offset, 0, 2);
}
// A raw buffer resource over [base, base + bytes).  Reads past `bytes` return
// 0 without a memory access, so a resource of 0 bytes turns a load into a
// no-op that still counts as issued (kernels use this to keep a load sequence
// unconditional, so the compiler's wait counts stay exact).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_buffer(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}

// Per-lane select by a wave lane mask: lane i gets `if_set` when bit i of
// `lanes` is set, else `if_clear` (one v_cndmask).  Written out so that the
// compiler cannot fold `c ? x[a] : x[b]` over a register array into a
// dynamically indexed array, which it lowers to long compare/select chains.
__device__ __forceinline__ float lane_select(unsigned long long lanes, float if_set, float if_clear) {
  float r;
  asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(r) : "v"(if_clear), "v"(if_set), "s"(lanes));
  return r;
}

// In-row (16-lane) exchanges through DPP: a few cycles instead of an LDS
// round trip.  xor 1 / xor 2 are quad permutations, xor 8 is a rotation of
// the row by 8; xor 4 combines a left and a right row shift by 4.
template <int kCtrl>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), kCtrl, 0xF, 0xF, false));
}
__device__ __forceinline__ float xor1(float v) { return dpp_f<0xB1>(v); }   // quad_perm [1,0,3,2]
__device__ __forceinline__ float xor2(float v) { return dpp_f<0x4E>(v); }   // quad_perm [2,3,0,1]
__device__ __forceinline__ float xor8(float v) { return dpp_f<0x128>(v); }  // row_ror:8
__device__ __forceinline__ float xor4(float v) {
  const float up = dpp_f<0x104>(v);    // row_shl:4: lane i reads lane i + 4
  const float down = dpp_f<0x114>(v);  // row_shr:4: lane i reads lane i - 4
  return (threadIdx.x & 4) ? down : up;
}
__device__ __forceinline__ float row_mirror(float v) { return dpp_f<0x140>(v); }       // lane i <- 15 - i
__device__ __forceinline__ float row_half_mirror(float v) { return dpp_f<0x141>(v); }  // lane i <- 7 - i (in 8)

// Exchanges across rows through the gfx950 permlane swaps (VALU, no LDS).
// permlane32_swap(a, b) returns {a', b'}: a' = a in lanes 0-31 and b of lane
// l - 32 in lanes 32-63; b' = a of lane l + 32 in lanes 0-31 and b in lanes
// 32-63.  permlane16_swap does the same between rows 0/1 and 2/3.
__device__ __forceinline__ unsigned xor32_u(unsigned v) {
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return (threadIdx.x & 32) ? r[0] : r[1];
}
__device__ __forceinline__ unsigned xor16_u(unsigned v) {
  const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return (threadIdx.x & 16) ? r[0] : r[1];
}
__device__ __forceinline__ float xor32(float v) { return __uint_as_float(xor32_u(__float_as_uint(v))); }
__device__ __forceinline__ float xor16(float v) { return __uint_as_float(xor16_u(__float_as_uint(v))); }
// Transpose-reduce step across lane bit 5 (M = 32) or 4 (M = 16): lanes with
// the bit clear return lo + lo of lane l ^ M, lanes with it set hi + hi of
// lane l ^ M.  After the swap one register holds the own term and the other
// the partner's (which is which depends on the lane); IEEE addition is
// commutative, so one add gives both lanes of a pair the same bits.
template <int M>
__device__ __forceinline__ float swap_add(float lo, float hi) {
  const unsigned a = __float_as_uint(lo), b = __float_as_uint(hi);
  if constexpr (M == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
}

// Wave reductions: within each 16-lane row by DPP (pairs i^1, i^2, then the
// mirrors i <-> 7-i and i <-> 15-i), then the 4 row results by readlane.
// Fixed order, so results are run-to-run identical; the result is uniform.
__device__ __forceinline__ float row_max(float v) {
  v = fmaxf(v, xor1(v));
  v = fmaxf(v, xor2(v));
  v = fmaxf(v, row_half_mirror(v));
  return fmaxf(v, row_mirror(v));
}
__device__ __forceinline__ float row_sum(float v) {
  v += xor1(v);
  v += xor2(v);
  v += row_half_mirror(v);
  return v + row_mirror(v);
}
__device__ __forceinline__ float lane_bcast(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ float wave_max(float v) {
  v = row_max(v);
  return fmaxf(fmaxf(lane_bcast(v, 0), lane_bcast(v, 16)), fmaxf(lane_bcast(v, 32), lane_bcast(v, 48)));
}
__device__ __forceinline__ float wave_sum(float v) {
  v = row_sum(v);
  return (lane_bcast(v, 0) + lane_bcast(v, 16)) + (lane_bcast(v, 32) + lane_bcast(v, 48));
}

// Exclusive prefix over the lanes of a wave for small nonnegative counts
// (v < 2^kBits): one ballot per bit plane and a lane-masked popcount.
template <int kBits>
__device__ __forceinline__ int wave_excl_small(int v, int* total) {
  int pre = 0, tot = 0;
#pragma unroll
  for (int b = 0; b < kBits; ++b) {
    const unsigned long long m = __ballot((v >> b) & 1);
    pre += (int)__builtin_amdgcn_mbcnt_hi((unsigned)(m >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)m, 0u)) << b;
    tot += __popcll(m) << b;
  }
  *total = tot;
  return pre;
}


// Sum of v over the 64 lanes of a wave through DPP moves (no LDS round
// trips): pairs, quads (quad_perm), 8 (row_half_mirror), 16 (row_mirror),
// then row 0 into row 1 and row 2 into row 3 (row_bcast:15), rows 0-1 into
// rows 2-3 (row_bcast:31); lane 63 holds the total.
__device__ __forceinline__ int wave_sum_dpp(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
  v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
  v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);  // row_half_mirror
  v += __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false);  // row_mirror
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15 into rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31 into rows 2, 3
  return __builtin_amdgcn_readlane(v, 63);
}

// Wave sums of 8 integers at once by a transpose-reduce: pairs of lanes
// 32, 16 and 8 apart swap halves of the set and add (permlane swaps, then a
// DPP row rotation), which leaves lane l holding partial sums of value l >> 3
// over its 8-lane group's partners; three in-row DPP steps then add the
// group.  Returns, in lane 8j, the sum of p[j] over the wave (other lanes
// hold the same sum for j = l >> 3).  Integer sums are exact in any order.
__device__ __forceinline__ int wave_sum8(int (&p)[8]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const auto r = __builtin_amdgcn_permlane32_swap((unsigned)p[j], (unsigned)p[j + 4], false, false);
    p[j] = (int)(r[0] + r[1]);  // bit 5 clear: value j, set: value j + 4
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const auto r = __builtin_amdgcn_permlane16_swap((unsigned)p[j], (unsigned)p[j + 2], false, false);
    p[j] = (int)(r[0] + r[1]);  // bit 4 clear: value j (+4), set: value j + 2 (+4)
  }
  const bool b3 = lane & 8;
  const int keep = b3 ? p[1] : p[0], send = b3 ? p[0] : p[1];
  int v = keep + __float_as_int(xor8(__int_as_float(send)));  // value lane >> 3
  v += __float_as_int(xor4(__int_as_float(v)));
  v += __float_as_int(xor2(__int_as_float(v)));
  v += __float_as_int(xor1(__int_as_float(v)));
  return v;
}

// The wave's integer sum, in every lane.
__device__ __forceinline__ int wave_sum_i(int v) { return wave_sum_dpp(v); }

// Inclusive prefix sum over the lanes of a wave64 by DPP (no LDS traffic):
// in-row shifts by 1, 2, 4 and 8 (lanes without a source add 0), then row
// 0's total into row 1 and row 2's into row 3, then rows 0-1's total into
// rows 2 and 3.
__device__ __forceinline__ unsigned wave_incl_scan(unsigned x) {
  x += __builtin_amdgcn_update_dpp(0u, x, 0x111, 0xF, 0xF, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0u, x, 0x112, 0xF, 0xF, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0u, x, 0x114, 0xF, 0xF, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0u, x, 0x118, 0xF, 0xF, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0u, x, 0x142, 0xA, 0xF, false);  // row_bcast:15 into rows 1, 3
  x += __builtin_amdgcn_update_dpp(0u, x, 0x143, 0xC, 0xF, false);  // row_bcast:31 into rows 2, 3
  return x;
}

// Inclusive prefix sum over a workgroup of NT threads (NT a multiple of 64).
// `wsum` is NT/64 words of LDS.  Contains two barriers.
template <int NT>
__device__ __forceinline__ unsigned block_incl_scan(unsigned v, unsigned* wsum) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_incl_scan(v);
  if (lane == 63) wsum[w] = v;
  __syncthreads();
  unsigned add = 0;
#pragma unroll
  for (int j = 0; j < NT / 64; ++j) add += (j < w) ? wsum[j] : 0u;
  __syncthreads();
  return v + add;
}

// Bounded spin used by every inter-workgroup wait: by default about 2^20
// sleeps of 64 clocks (tens of milliseconds) before the waiter gives up and
// reports.  The limit is process-wide and host-settable
// (prismkv_set_spin_limit); every launch passes the current value to its
// kernel as an argument.
constexpr int kSpinLimit = 1 << 20;
int spin_limit();  // the current process-wide limit (defined in decode.hip)

// Stage 3 on the fused decode's attention phases (defined in decode.hip):
// the bytes its workspace region takes for `groups` groups, and the launch
// over the given id lists; -1 when the geometry does not fit it (the caller
// then uses its own split-K kernel).
size_t attend_list_work_bytes(int groups);
int attend_list(uint64_t q, uint64_t k, uint64_t v, uint64_t ids, uint64_t count, uint64_t work, uint64_t out,
                int groups, int H, int T, int64_t ks, int64_t vs, int64_t ids_stride, uint64_t stream);

// Error words.  A workspace's first 32-bit word is its sticky error word; its
// 8-byte slot at byte offset 8 optionally holds the device address of a
// host-mapped 32-bit word (0 = none), so a host binding can notice an error
// without copying or synchronising.  A wait that gives up writes kErrWait to
// both (system scope: the host word lives in host memory); an attention over
// a caller's id list that finds an id outside [0, H) or a count outside
// [0, H] writes kErrIds (and reads the id clamped into range).
constexpr unsigned kErrWait = 1u, kErrIds = 2u;
__device__ __forceinline__ void report_error(unsigned* err, unsigned* const* host_slot, unsigned code = kErrWait) {
  __hip_atomic_store(err, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  if (host_slot) {
    unsigned* host = __hip_atomic_load(host_slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (host) __hip_atomic_store(host, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}
// The host-pointer slot of a workspace whose error word is `err`.
__host__ __device__ inline unsigned* const* error_host_slot(unsigned* err) {
  return reinterpret_cast<unsigned* const*>(reinterpret_cast<char*>(err) + 8);
}

// Cross-workgroup communication.  Data one workgroup hands to another is
// written through to the device coherence point and read back from it with
// relaxed agent-scope atomics (global_store/load ... sc1); a writer drains its
// stores (s_waitcnt 0) before the workgroup barrier that precedes the
// arrival-counter increment, and a reader only loads after it has observed
// the counter.  No agent-scope fences: on gfx950 each one writes back or
// invalidates the whole L2 of the XCD, which costs tens of microseconds when
// hundreds of workgroups do it.
template <typename T>
__device__ __forceinline__ void st_dev(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T ld_dev(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned inc_dev(unsigned* p) {
  return __hip_atomic_fetch_add(p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Waits until every memory operation this thread issued has completed.
__device__ __forceinline__ void drain() { __builtin_amdgcn_s_waitcnt(0); }

__device__ __forceinline__ void st_dev2(float* p, float a, float b) {
  st_dev(reinterpret_cast<unsigned long long*>(p),
         ((unsigned long long)__float_as_uint(b) << 32) | (unsigned long long)__float_as_uint(a));
}
__device__ __forceinline__ float2 ld_dev2(const float* p) {
  const unsigned long long v = ld_dev(reinterpret_cast<const unsigned long long*>(p));
  return make_float2(__uint_as_float((unsigned)v), __uint_as_float((unsigned)(v >> 32)));
}

}  // namespace prismkv
