// Sparse attention of one wave on the matrix cores in 16-row blocks: QK^T
// as v_mfma_f32_16x16x32_bf16, PV as v_mfma_f32_16x16x16_bf16, online
// softmax in fp32.
//
// Semantics: src/prismkv/core.py:170-183 (exact softmax over the selected
// rows and the tail, scale 1/sqrt(d)): scores are fp32 sums of exact bf16
// products; probabilities stay fp32 up to the PV product, where each is
// split into a bf16 head and a bf16 remainder (two products), so P.V carries
// ~16 significant bits of P instead of bf16's 8; accumulation is fp32.
//
// Operand layouts (lane l, j = l % 16, q = l / 16; r = 0..3 fp32 results,
// D[i][jj] with i = 4q + r, jj = j for both shapes):
//   QK (16x16x32: A[i][k] with i = j, k = 8q + t; B[k][jj] with jj = j):
//        D[row][head] = K . Q^T over 4 chunks of 32 dims.  Lane l supplies
//        row j of the block, dims 32c + 8q .. +8 -- one 16-byte load per
//        chunk of its own row -- and Q[head j] (zero for j >= 4).  The scores
//        of rows 4q + r for head j land in lane l.
//   PV (16x16x16: A[i][k] with i = j, k = 4q + t; B[k][jj] with jj = j):
//        D[head][dim] = P . V with the reduction index k = 4q + t exactly
//        the rows the lane scored, so P needs no lane exchange; the 8 column
//        blocks n map dim 8j + n to column j, so lane l reads rows 4q + t at
//        dims 8j .. 8j + 8 (16-byte loads; each load instruction covers 4
//        whole rows) and pairs them per dim with v_perm.  Lanes 0-15 end
//        with out[head r][8j + n] in acc[n][r].
#pragma once

#include "attend_core.h"

namespace prismkv {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct MfmaAttn {
  bf16x8 qop[4];  // Q^T operand per 32-dim chunk (zero in lanes with j >= 4)
  f32x4 acc[8];   // PV accumulators
  float m;        // running max (exp2 domain) of head j (lanes with j < 4)
  float z;        // this lane's share of head j's denominator
};

// Per-wave states of a workgroup, merged in LDS.
template <int kWaves>
struct MfmaLds {
  float sm[kWaves][kHq], sz[kWaves][kHq], wt[kWaves][kHq], mx[kHq];
  float sacc[kWaves][kHq][kD];
};

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) {
  const u32x4 u = {v.x, v.y, v.z, v.w};
  return __builtin_bit_cast(bf16x8, u);
}

__device__ __forceinline__ void mfma_init(MfmaAttn& st, const uint16_t* qg) {
  const int lane = threadIdx.x & 63, j = lane & 15, q = lane >> 4;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (j < kHq) v = *reinterpret_cast<const uint4*>(qg + j * kD + 32 * c + 8 * q);
    st.qop[c] = as_bf16x8(v);
  }
#pragma unroll
  for (int n = 0; n < 8; ++n) st.acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
  st.m = -INFINITY;
  st.z = 0.f;
}

// bf16 pair (lo = a's dim n, hi = b's dim n) of two 8-dim rows.
template <int N>
__device__ __forceinline__ unsigned dim_pair(const uint4& a, const uint4& b) {
  const unsigned wa = (N >> 1) == 0 ? a.x : (N >> 1) == 1 ? a.y : (N >> 1) == 2 ? a.z : a.w;
  const unsigned wb = (N >> 1) == 0 ? b.x : (N >> 1) == 1 ? b.y : (N >> 1) == 2 ? b.z : b.w;
  return __builtin_amdgcn_perm(wb, wa, (N & 1) ? 0x07060302u : 0x05040100u);
}

typedef short s16x4 __attribute__((ext_vector_type(4)));

// Up to NB blocks of 16 rows as ONE step of the online softmax: the QK
// products of every block first (independent MFMA chains), then one
// running-max update for all of them (lazy: the max moves only when a score
// exceeds it by kSlack), then the PV products, so the blocks of a round
// share one max reduction and one rescale instead of waiting on each
// other's.  kr[i][c]: lane's row j of block i, dims 32c + 8q; vr[i][t]: row
// 4q + t, dims 8j .. 8j + 8.  Block i has nvalid[i] live rows (0: no block
// i; uniform per wave); rows >= nvalid[i] are masked (their loads may repeat
// any row), and its loads must be valid whenever nvalid[i] > 0.
template <int NB>
__device__ __forceinline__ void mfma_blocks16(MfmaAttn& st, const uint4 (&kr)[NB][4], const uint4 (&vr)[NB][4],
                                              const int (&nvalid)[NB]) {
  const int lane = threadIdx.x & 63, j = lane & 15, q = lane >> 4;
  f32x4 d[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    d[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (nvalid[i] > 0) {
#pragma unroll
      for (int c = 0; c < 4; ++c) d[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kr[i][c]), st.qop[c], d[i], 0, 0, 0);
    }
  }
  float s[NB][4];
  float bm = -INFINITY;
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      s[i][r] = (j < kHq && 4 * q + r < nvalid[i]) ? d[i][r] * kLog2eScale : -INFINITY;
      bm = fmaxf(bm, s[i][r]);
    }
  bm = fmaxf(bm, xor16(bm));
  bm = fmaxf(bm, xor32(bm));
  const bool grow = bm > st.m + kSlack || (st.m == -INFINITY && bm != -INFINITY);
  if (__ballot(grow)) {
    const float nm = grow ? bm : st.m;
    const float alpha = grow ? exp2_or_zero(st.m - nm) : 1.0f;
    st.m = nm;
    st.z *= alpha;
    float ah[kHq];
#pragma unroll
    for (int r = 0; r < kHq; ++r) ah[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(alpha), r));
#pragma unroll
    for (int n = 0; n < 8; ++n)
#pragma unroll
      for (int r = 0; r < kHq; ++r) st.acc[n][r] *= ah[r];
  }
  typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    if (nvalid[i] <= 0) continue;  // uniform
    float p[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) p[t] = s[i][t] == -INFINITY ? 0.f : exp2f(s[i][t] - st.m);
    st.z += (p[0] + p[1]) + (p[2] + p[3]);
    // P = head + remainder, both bf16: head = the top 16 bits, remainder rounded to nearest
    unsigned hi[4], lo[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const unsigned b = __float_as_uint(p[t]);
      hi[t] = b >> 16;
      lo[t] = f32_to_bf16(p[t] - __uint_as_float(b & 0xffff0000u));
    }
    const u32x2 uh = {hi[0] | hi[1] << 16, hi[2] | hi[3] << 16};
    const u32x2 ul = {lo[0] | lo[1] << 16, lo[2] | lo[3] << 16};
    const s16x4 ph = __builtin_bit_cast(s16x4, uh), pl = __builtin_bit_cast(s16x4, ul);
#define PRISMKV_PVB(N)                                                                   \
    {                                                                                    \
      const u32x2 vu = {dim_pair<N>(vr[i][0], vr[i][1]), dim_pair<N>(vr[i][2], vr[i][3])}; \
      const s16x4 vb = __builtin_bit_cast(s16x4, vu);                                    \
      st.acc[N] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ph, vb, st.acc[N], 0, 0, 0); \
      st.acc[N] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pl, vb, st.acc[N], 0, 0, 0); \
    }
    PRISMKV_PVB(0) PRISMKV_PVB(1) PRISMKV_PVB(2) PRISMKV_PVB(3)
    PRISMKV_PVB(4) PRISMKV_PVB(5) PRISMKV_PVB(6) PRISMKV_PVB(7)
#undef PRISMKV_PVB
  }
}

// Writes wave w's state (max, denominator, acc[4][128]) into LDS.
template <int kWaves>
__device__ __forceinline__ void mfma_stash(const MfmaAttn& st, MfmaLds<kWaves>& lds, int w) {
  const int lane = threadIdx.x & 63;
  float zt = st.z + xor16(st.z);
  zt += xor32(zt);
  if (lane < kHq) {
    lds.sm[w][lane] = st.m;
    lds.sz[w][lane] = zt;
  }
  if (lane < 16) {
#pragma unroll
    for (int r = 0; r < kHq; ++r) {
      float4* dst = reinterpret_cast<float4*>(&lds.sacc[w][r][8 * lane]);
      dst[0] = make_float4(st.acc[0][r], st.acc[1][r], st.acc[2][r], st.acc[3][r]);
      dst[1] = make_float4(st.acc[4][r], st.acc[5][r], st.acc[6][r], st.acc[7][r]);
    }
  }
}

}  // namespace
}  // namespace prismkv
