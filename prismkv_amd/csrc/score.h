// Moment scoring of one 32-bucket tile, shared by the route kernels and the
// fused decode kernel so that both produce bit-identical logits, chunk
// statistics and probability keys.
//
// Semantics: src/prismkv/core.py:119-128 (router="moments"): logit =
// (log(count) + (q @ mean^T) / sqrt(d)) + (q^2 @ var^T) / (2d) in this
// accumulation order, dead buckets -inf; per-head softmax exp(l - M) / Z and
// the sum over heads in head order.
//
// A tile is f32 [256 rows][32 buckets] (rows k < 128: mean dim k, k >= 128:
// variance dim k - 128).  256 threads score it: thread t = bucket quad
// (t & 7) x row phase (t >> 3) issues 8 independent 16-byte loads.  The
// products run on the matrix cores as v_mfma_f32_4x4x1_16b_f32 outer
// products (block = 4 lanes of one row: 4 buckets x 4 heads, K = 1), each a
// chain of exact fused multiply-adds over the thread's rows, bit for bit the
// fmaf chain; the partial sums are then reduced across the 8 row lanes of a
// wave with a transpose-reduce and across the 4 waves in LDS, in a fixed
// order, so results are run-to-run identical.
#pragma once

#include "select.h"

namespace prismkv {
namespace {

constexpr float kSqrtD = 11.3137084989847604f;  // fp32(sqrt(128)), core.py:125

// Transpose-reduce step over lane bit M (32, 16 or 8): `x` holds 2N partial
// sums; lanes with the bit set keep the upper half, the others the lower
// half, and add the partner's copy of the kept half (own term first).  After
// the step x[0..N) holds the new partial sums.
template <int N, int M>
__device__ __forceinline__ void treduce(float* x) {
  if constexpr (M == 32 || M == 16) {
#pragma unroll
    for (int j = 0; j < N; ++j) x[j] = swap_add<M>(x[j], x[j + N]);
  } else {
    const unsigned long long hi = __ballot((threadIdx.x & M) != 0);
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const float keep = lane_select(hi, x[j + N], x[j]);
      const float send = lane_select(hi, x[j], x[j + N]);
      x[j] = keep + xor8(send);
    }
  }
}

// LDS of one 256-thread tile scorer.
struct TileLds {
  float4 red[4][64];            // cross-wave partials
  float dots[2][kHq][kChunk];   // [part][head][bucket]
};

// q (rows k < 128) and q*q (rows k >= 128) of group g, 4 heads per float4,
// from bf16 or fp32 queries: thread t of nt stages entries t, t + nt, ... of
// the 512.
template <typename QT>
__device__ __forceinline__ void stage_query(const QT* q, int g, float4* qq, int t, int nt) {
  for (int i = t; i < kHq * kD; i += nt) {
    const int h = i >> 7, k = i & (kD - 1);
    const float x = to_f32(q[((size_t)g * kHq + h) * kD + k]);
    reinterpret_cast<float*>(&qq[k])[h] = x;
    reinterpret_cast<float*>(&qq[kD + k])[h] = x * x;  // core.py:127 q.square() in fp32
  }
}
// The same for exactly 512 threads, split so the caller can issue the q load
// before its tile loads (its wait then leaves those in flight): the raw bf16
// bits are loaded first and converted only in store_query512.
__device__ __forceinline__ unsigned load_query512(const uint16_t* q, int g, int t) {
  return q[((size_t)g * kHq + (t >> 7)) * kD + (t & (kD - 1))];
}
__device__ __forceinline__ void store_query512(unsigned bits, float4* qq, int t) {
  const float x = __uint_as_float(bits << 16);
  const int h = t >> 7, k = t & (kD - 1);
  reinterpret_cast<float*>(&qq[k])[h] = x;
  reinterpret_cast<float*>(&qq[kD + k])[h] = x * x;  // core.py:127 q.square() in fp32
}

// The 16-byte loads of tile (g, c) for thread t (0..255); c must be a valid
// tile (no branch, so every load of the caller stays in flight together).
__device__ __forceinline__ void load_tile(const float* moments, int g, int c, int t, float4 (&m4)[8]) {
  const int quad = t & 7, r = t >> 3;
  const float4* tile = reinterpret_cast<const float4*>(moments + (size_t)(g * kChunks + c) * kRow * kChunk);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(tile + (r + 32 * i) * (kChunk / 4) + quad));
    m4[i] = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
  }
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// One K = 1 step of 16 independent 4 x 4 outer products: block b = lanes
// 4b..4b+3; D[b][i][j] += A[b][i] B[b][j] with A[b][i] = `a` of lane 4b + i
// and B[b][j] = `b` of lane 4b + j; VGPR v of lane 4b + j holds D[b][v][j].
// Each step is an exact fused multiply-add (a chain equals the fmaf chain).
__device__ __forceinline__ f32x4 outer4(float a, float b, f32x4 d) {
  return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, d, 0, 0, 0);
}

// The row products of one thread's loads as 4 x 4 blocks: load i of lane l
// holds buckets 4 (l & 7) .. +3 of its row, so component c of the lanes of
// block b = l >> 2 (same row, quads 4 (b & 1) + i) gives A = buckets
// 16 (b & 1) + 4 i + c, and B = q of head l & 3 at that row (from `qq`).
// d[c] then holds, in VGPR v of lane l, the partial over the loaded rows of
// bucket 16 ((l >> 2) & 1) + 4 v + c, head l & 3.
template <int N>
__device__ __forceinline__ void row_products(const float4* qq, const float4* m, const int* rows, int lane,
                                             f32x4 (&d)[4]) {
  const float* qf = reinterpret_cast<const float*>(qq);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const float qb = qf[rows[i] * 4 + (lane & 3)];
    d[0] = outer4(m[i].x, qb, d[0]);
    d[1] = outer4(m[i].y, qb, d[1]);
    d[2] = outer4(m[i].z, qb, d[2]);
    d[3] = outer4(m[i].w, qb, d[3]);
  }
}

// Products and reductions of one tile; returns, in thread t < 128, the logit
// of head t >> 5 for bucket 32c + (t & 31) whose size is `n` (loaded by the
// caller with the tile, so no load waits here; -inf for a dead bucket).
// Every thread of the workgroup must call it (two barriers); t is the
// thread's index within its 256-thread scorer, whose 4 waves are consecutive.
__device__ __forceinline__ float tile_logit(const float4* qq, const float4 (&m4)[8], int t, TileLds& s, int n,
                                            bool has) {
  const int r = t >> 3, w = t >> 6, lane = t & 63;
  // acc[part * 16 + c * 4 + v]: part 0 = mean rows r + 32 i (i < 4), 1 = variance rows
  float acc[32];
#pragma unroll
  for (int part = 0; part < 2; ++part) {
    f32x4 d[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) d[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int rows[4] = {r + 128 * part, r + 32 + 128 * part, r + 64 + 128 * part, r + 96 + 128 * part};
    row_products<4>(qq, m4 + 4 * part, rows, lane, d);
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[part * 16 + c * 4 + v] = d[c][v];
  }
  // reduce over the 8 row lanes of the wave (lane bits 5,4,3 = row bits 2,1,0)
  treduce<16, 32>(acc);
  treduce<8, 16>(acc);
  treduce<4, 8>(acc);
  // lane now holds part (lane >> 5) & 1, c = 2 ((lane >> 4) & 1) + ((lane >> 3) & 1),
  // head lane & 3: buckets 16 ((lane >> 2) & 1) + 4 v + c, v = 0..3
  s.red[w][lane] = make_float4(acc[0], acc[1], acc[2], acc[3]);
  __syncthreads();
  {
    const int l = t >> 2, v = t & 3;
    const float x = ((reinterpret_cast<const float*>(&s.red[0][l])[v] + reinterpret_cast<const float*>(&s.red[1][l])[v]) +
                     reinterpret_cast<const float*>(&s.red[2][l])[v]) +
                    reinterpret_cast<const float*>(&s.red[3][l])[v];
    const int c = 2 * ((l >> 4) & 1) + ((l >> 3) & 1);
    s.dots[(l >> 5) & 1][l & 3][16 * ((l >> 2) & 1) + 4 * v + c] = x;
  }
  __syncthreads();
  float l = -INFINITY;
  if (t < kHq * kChunk && has) {
    const int h = t >> 5, b = t & 31;
    if (n > 0) {
      // core.py:122-127: log(count) + (q @ mean^T) / sqrt(d) + (q^2 @ var^T) / (2d)
      const float lc = logf((float)n);
      l = (lc + s.dots[0][h][b] / kSqrtD) + s.dots[1][h][b] / (2.0f * kD);
    }
  }
  return l;
}

// One tile scored by both halves of a 512-thread workgroup: half h takes
// part h (h = 0: mean rows 0..127, 1: variance rows 128..255) with 4 loads
// per thread.  Every dot product is the same tree of additions as in
// tile_logit (the same fused chain over a thread's 4 rows, row lanes paired
// by lane bit 5, then 4, then 3; each pair sum is commutative; then the 4
// waves in order), so the logits are bit-identical.
struct SplitLds {
  float2 red[2][4][64];
  float dots[2][kHq][kChunk];
};

__device__ __forceinline__ void load_half_tile(const float* moments, int g, int c, int part, int t, float4 (&m4)[4]) {
  const int quad = t & 7, r = t >> 3;
  const float4* tile = reinterpret_cast<const float4*>(moments + (size_t)(g * kChunks + c) * kRow * kChunk);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u32x4 v = __builtin_nontemporal_load(
        reinterpret_cast<const u32x4*>(tile + (r + 32 * i + 128 * part) * (kChunk / 4) + quad));
    m4[i] = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
  }
}

// Three tiles scored by a 512-thread workgroup in one pass: half h takes all
// of tile A_h (8 loads per thread, m8) and part h of tile B (4 loads, m4),
// so the two reductions interleave and share their 2 barriers.  The log of
// each bucket size is taken before the products, off the chain that follows
// the last load.  Returns (x) the logit of tile A_h in threads t < 128 of
// half h (head t >> 5, bucket t & 31) and (y) tile B's in threads
// 128 <= tid < 256 (head (tid - 128) >> 5, bucket tid & 31), -inf for a
// dead bucket; na / nb are the sizes of bucket tid & 31 of A_h / B.  Every
// dot product is the same tree of additions as in tile_logit (the same
// fused chains over a thread's rows, row lanes paired by lane bit 5, then
// 4, then 3, each pair sum commutative, then the 4 waves in order), so the
// logits are bit-identical to tile_logit's.
__device__ __forceinline__ float2 tile_logits3(const float4* qq, const float4 (&m8)[8], const float4 (&m4)[4], int tid,
                                               TileLds (&sa)[2], SplitLds& sb, int na, int nb) {
  const int half = tid >> 8, t = tid & 255, r = t >> 3, w = t >> 6, lane = t & 63;
  const float lca = logf((float)na), lcb = logf((float)nb);
  float a[32];  // a[part * 16 + c * 4 + v]
  float b[16];  // b[c * 4 + v], part = half
#pragma unroll
  for (int part = 0; part < 2; ++part) {
    f32x4 d[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) d[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int rows[4] = {r + 128 * part, r + 32 + 128 * part, r + 64 + 128 * part, r + 96 + 128 * part};
    row_products<4>(qq, m8 + 4 * part, rows, lane, d);
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int v = 0; v < 4; ++v) a[part * 16 + c * 4 + v] = d[c][v];
  }
  {
    f32x4 d[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) d[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int rows[4] = {r + 128 * half, r + 32 + 128 * half, r + 64 + 128 * half, r + 96 + 128 * half};
    row_products<4>(qq, m4, rows, lane, d);
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int v = 0; v < 4; ++v) b[c * 4 + v] = d[c][v];
  }
  treduce<16, 32>(a);
  treduce<8, 32>(b);
  treduce<8, 16>(a);
  treduce<4, 16>(b);
  treduce<4, 8>(a);
  treduce<2, 8>(b);
  sa[half].red[w][lane] = make_float4(a[0], a[1], a[2], a[3]);
  sb.red[half][w][lane] = make_float2(b[0], b[1]);
  __syncthreads();
  {
    const int l = t >> 2, v = t & 3;
    const float x = ((reinterpret_cast<const float*>(&sa[half].red[0][l])[v] +
                      reinterpret_cast<const float*>(&sa[half].red[1][l])[v]) +
                     reinterpret_cast<const float*>(&sa[half].red[2][l])[v]) +
                    reinterpret_cast<const float*>(&sa[half].red[3][l])[v];
    const int c = 2 * ((l >> 4) & 1) + ((l >> 3) & 1);
    sa[half].dots[(l >> 5) & 1][l & 3][16 * ((l >> 2) & 1) + 4 * v + c] = x;
  }
  if (t < kHq * kChunk) {
    const int h = t >> 5, bk = t & 31;
    const int qh = bk >> 4, v = (bk >> 2) & 3, c = bk & 3;
    const int L = h | (qh << 2) | ((v >> 1) << 3) | ((c & 1) << 4) | ((c >> 1) << 5);
    const bool hi = v & 1;
    const float x = (((hi ? sb.red[half][0][L].y : sb.red[half][0][L].x) + (hi ? sb.red[half][1][L].y : sb.red[half][1][L].x)) +
                     (hi ? sb.red[half][2][L].y : sb.red[half][2][L].x)) +
                    (hi ? sb.red[half][3][L].y : sb.red[half][3][L].x);
    sb.dots[half][h][bk] = x;
  }
  __syncthreads();
  float2 out = make_float2(-INFINITY, -INFINITY);
  const int h = (t >> 5) & 3, bk = t & 31;
  if (t < kHq * kChunk) {
    // core.py:122-127: log(count) + (q @ mean^T) / sqrt(d) + (q^2 @ var^T) / (2d)
    if (na > 0) out.x = (lca + sa[half].dots[0][h][bk] / kSqrtD) + sa[half].dots[1][h][bk] / (2.0f * kD);
  } else if (half == 0) {
    if (nb > 0) out.y = (lcb + sb.dots[0][h][bk] / kSqrtD) + sb.dots[1][h][bk] / (2.0f * kD);
  }
  return out;
}

// (max, sum of exp(l - max)) over the 32 lanes of a head (lanes 0-31 or
// 32-63 of a wave, all active).
__device__ __forceinline__ float2 chunk_stats(float l) {
  float m = l;
  m = fmaxf(m, xor16(m));
  m = fmaxf(m, xor8(m));
  m = fmaxf(m, xor4(m));
  m = fmaxf(m, xor2(m));
  m = fmaxf(m, xor1(m));
  float e = (l == -INFINITY) ? 0.f : expf(l - m);
  e += xor16(e);
  e += xor8(e);
  e += xor4(e);
  e += xor2(e);
  e += xor1(e);
  return make_float2(m, e);
}

// Merge of the 94 chunk statistics of one head by one wave (lane i reads
// chunks i and i + 64 through `ld(chunk)`): M = max, Z = sum z_c e^{m_c - M};
// returns (M, 1/Z) in every lane (1/Z = 0 when Z = 0).
template <typename Load2>
__device__ __forceinline__ float2 merge_chunk_stats(Load2 ld) {
  const int lane = threadIdx.x & 63;
  const float2 s0 = lane < kChunks ? ld(lane) : make_float2(-INFINITY, 0.f);
  const float2 s1 = lane + 64 < kChunks ? ld(lane + 64) : make_float2(-INFINITY, 0.f);
  const float m = wave_max(fmaxf(s0.x, s1.x));
  float z = (s0.x == -INFINITY ? 0.f : s0.y * expf(s0.x - m)) + (s1.x == -INFINITY ? 0.f : s1.y * expf(s1.x - m));
  z = wave_sum(z);
  return make_float2(m, z > 0.f ? 1.0f / z : 0.f);
}

// Key of a live bucket: per-head softmax exp(l - M) / Z summed over heads in
// head order (core.py:128); equal logits give bit-equal keys, so exact ties
// fall to the lower bucket id.  0 for a dead bucket.
__device__ __forceinline__ uint64_t bucket_key(const float (&l)[kHq], const float* gmax, const float* grz, int bucket) {
  if (l[0] == -INFINITY) return 0;
  const float p0 = expf(l[0] - gmax[0]) * grz[0];
  const float p1 = expf(l[1] - gmax[1]) * grz[1];
  const float p2 = expf(l[2] - gmax[2]) * grz[2];
  const float p3 = expf(l[3] - gmax[3]) * grz[3];
  return make_key(((p0 + p1) + p2) + p3, bucket);
}

}  // namespace
}  // namespace prismkv
