// Fused routed decode of one layer in ONE launch: moment scoring (stage 1a),
// bucket selection (stage 1b), bitmap union (stage 2) and sparse attention
// (stage 3).  Same results as prismkv_route + prismkv_union + prismkv_attend;
// it exists because every kernel boundary in a HIP graph costs ~1.75 us on
// MI355X, more than most of these stages' work, and because the selection
// is cheapest when each workgroup ranks only the buckets it scored.
//
// Semantics: src/prismkv/core.py:106-183 (route, union, attend), the tie and
// padding rules of kernels/ppu_8b/route_parallel.cu:12,23,29 and the ascending
// emission of kernels/ppu_8b/union.cu:26.
//
// Other launches share these phases: route_kernel runs phases 1-4 alone
// (prismkv_route_single); decode_kernel<KW, true> runs phases 5-9 on a
// selection read from features / valid (prismkv_union_attend, after a strict
// unique cap has walked it) or phases 6-9 on a given id list (prismkv_attend);
// the capped variant runs the budgeted walk between phases 4 and 6
// (prismkv_decode_capped); the route-only variant stops after the ids
// (prismkv_route_union).
//
// Grid (S, G) x 512, S = clamp(256 / G, 32, 256) (32 for 8 groups: the whole
// launch is resident at once, one workgroup per CU, at any history).  Workgroup p
// of group g owns the contiguous moment tiles kp .. kp + k - 1 of the 94
// (k = ceil(94 / S) <= 3: one 96 KB stream per workgroup),
// bitmap words [tw p, tw (p + 1)), tw = ceil(ceil(H/32) / S) <= 512 (tokens
// [32 tw p, 32 tw (p + 1)), so every workgroup gathers its share of the
// selected rows at any history) and tail rows [p * ceil(T/S), ...).  Phases:
//   1. score its tiles (two 256-thread scorers side by side, every tile load
//      issued up front) into LDS logits; publish each tile's per-head
//      (max, sum-exp) statistics;
//   2. read the group's 94 chunk statistics as they land and merge them into
//      the per-head (M, 1/Z) -- every workgroup merges the same 94 pairs in
//      the same order, so all hold the same bits;
//   3. rank its own buckets' keys (head-summed probability, bucket id) and
//      publish its 16 best;
//   4. read the group's S x 16 candidates as they land and rank them: the
//      group's Top-16 is among them, and every workgroup computes the same
//      winners; meanwhile each wave requests the tile's bitmap words of its
//      best candidates' rows (and, for long tails, its first tail block);
//   5. union tile: OR the winners' rows over the tile's words (prefetched in
//      phase 4 for tiles of up to 128 words) and compact the set bits into
//      an LDS token list, publishing the tile's count;
//   6. attention over the tile's tokens plus its tail share in 16-row MFMA
//      blocks dealt round-robin to the waves, the K/V loads of up to four
//      blocks per wave in flight at once (a wave's early tail block,
//      requested in phase 4, takes one slot of its first round; the lower
//      tiles' counts requested meanwhile);
//   7. the tile's ids offset: prefix = sum of the counts of the lower tiles;
//   8. its split state (per head max, denominator, acc[128]) is published,
//      then the tile's ids go to ids[g][prefix ...], and the group's last
//      workgroup writes features / valid / raw;
//   9. workgroups 0..15 each read one (head, 32-dim slice) of the S split
//      states as they land, merge it into out[g] and clear the words they
//      read; workgroup 0 also clears the group's statistics, candidates and
//      tile counts, so the launch replays from a graph without memset nodes.
// Published words hold the bitwise complement of their value, so a zero
// word (as cleared, or as the zero-filled workspace starts) reads as "not
// yet written": readers poll the data itself, one memory round trip after
// the writer's store, with no flags and no fences.  Waits only involve the
// workgroups of one group, which the in-order dispatcher starts back to back
// (S <= 256 fit on the GPU at once); every wait is bounded and reports
// through the error word instead of hanging.  Data crosses workgroups only
// through write-through (agent-scope) stores and loads, never through
// device-scope fences.
#include <algorithm>
#include <mutex>

#include "attend_mfma.h"
#include "score.h"

// The attention phase runs on the matrix cores (v_mfma_f32_16x16x32_bf16 for
// QK, 16x16x16 for PV).  Building with -DPRISMKV_VALU_ATTENTION=1 swaps in the
// fp32 VALU attention of attend_core.h (same loads, online softmax, state
// layout and merge) for the A/B that chose the matrix cores: 26.9 against
// 30.3 us per layer at H = 65536 on MI355X.
#ifndef PRISMKV_VALU_ATTENTION
#define PRISMKV_VALU_ATTENTION 0
#endif

namespace prismkv {
namespace {

constexpr int kDT = kAT;           // 512 threads, 8 waves
constexpr int kTileWords = 64;     // bitmap words per union chunk (one wave, one word per lane)
constexpr int kPrefetchChunks = 2; // union chunks the wide variant requests in phase 4 (tiles of 65-128 words)
constexpr int kMaxTileWords = 512; // bitmap words per workgroup at most (8 chunks, one per wave)
constexpr int kTileTokens = 32 * kMaxTileWords;
constexpr int kMinSplits = 32;     // at least one workgroup per CU for the scoring
constexpr int kMaxSplits = 256;    // one group's workgroups must fit on the GPU at once
constexpr int kMaxOwn = (kChunks + kMinSplits - 1) / kMinSplits;  // moment tiles per workgroup (3)
constexpr unsigned kReady = 1u << 31;
constexpr int kSlices = 4;                    // 32-dim slices of a head's output
constexpr int kSliceW = 2 + kD / kSlices;     // {max, den, acc[32]} per (split, head, slice)
constexpr int kMergers = kHq * kSlices;       // workgroups 0..15 each merge one (head, slice)
constexpr int kEarlyRows = 16 * (kAT / 64);   // early tail rows per workgroup: one 16-row block per wave

struct DecodeArgs {
  const uint16_t* q;
  const float* moments;  // [G][94][256][32]
  const int* counts;     // [G][kFP]
  const uint32_t* bits;
  int64_t row_words;
  const uint16_t* k;
  const uint16_t* v;
  int64_t ks, vs;
  int H, T, S;          // T: the tail length, or its upper bound when tail_dev is set
  int tw;               // bitmap words per workgroup, ceil(ceil(H / 32) / S) <= 512
  const int* tail_dev;  // optional: the tail length in device memory (read at launch; graph replays)
  unsigned long long* stats;  // [G][kChunks][4] published (max, sum-exp) per chunk and head
  unsigned long long* cand;   // [G][S][16] published best keys of each workgroup
  unsigned* status;           // [G][S] kReady | tile count
  unsigned* err;                  // sticky error word (a wait gave up)
  unsigned* const* err_host;      // optional slot holding a host-mapped error word's address
  int spin;                       // bound of every wait (sleeps), prismkv_set_spin_limit
  float* state;  // [G][S][4 heads][4 slices][34] published split states
  unsigned* walk;  // [G][4 windows][S][8] published pattern counts (capped launch)
  int limit;       // the strict unique cap's limit (capped launch)
  int rows16;      // capped launch: rows and tiles 16-byte aligned (the walk reads its words 4 a lane)
  int64_t* features;
  float* valid;
  int* raw;
  int32_t* ids;
  int64_t ids_stride;
  int32_t* count;
  uint16_t* out;
  // attention over a given id list (prismkv_attend; given-selection
  // instantiation only): the group's ids [G][ids_stride] and counts [G]
  // replace the selection and the union; ids / count are then not written
  const int32_t* ids_in;
  const int32_t* count_in;
};

// The tile's selected tokens live in dynamic LDS after this struct, sized
// per launch (32 tw ints): a launch allocates only what its history needs
// (8 KB at 64K), since a larger LDS allocation slows every launch.
struct DecodeLds {
  float tl[kMaxOwn][kHq][kChunk];  // logits of this workgroup's moment tiles
  alignas(16) unsigned long long win[kTop];
  int sel_rows[kTop];
  int need, nsel, base;
  unsigned cover[kDT / 64];  // per wave: the winners' ranks whose rows it prefetched
  int chunk_rows[kDT / 64];  // per union chunk: its selected tokens
  float gmax[kHq], grz[kHq];
  int walk_part[kDT / 64][8];  // capped launch: per wave, its packed pattern counts
  unsigned walk_keep;          // capped launch: the window's kept rows
  union alignas(16) {
    struct {
      float4 qq[kRow];
      TileLds tile[2];
      SplitLds split;
    } score;
    struct {
      alignas(16) unsigned long long own[2 * 64];  // this workgroup's keys (<= 96 used)
      alignas(16) unsigned long long best[kDT / 64 * kTop];
      unsigned ors[kDT / 64][kTileWords];  // per wave: OR of its prefetched winning rows over the tile's words
      unsigned ors2[kDT / 64][kTileWords];  // the same over the second chunk (wide variant)
    } sel;
    MfmaLds<kDT / 64> mf;
    struct {
      float2 mz[kMaxSplits];                 // (max, den) of every split
      float red[kDT / 64];                    // per-wave partial max / den
      float part[kDT / 32][kD / kSlices];    // per split-group partial sums
    } fin;
  };
};

// Bounded spin until `pred` holds for every lane of the calling wave; sets
// the error words and gives up instead of hanging.  A wait that gives up
// leaves the unlanded words at zero; every reader maps a zero word to an
// in-range value (bucket 0, count 0, NaN state), so the launch still ends
// normally, with the error reported.
template <typename Pred, typename Args>
__device__ __forceinline__ void wait_all(Pred pred, const Args& a) {
  for (int spins = 0;; ++spins) {
    if (__ballot(!pred()) == 0) return;
    if (spins >= a.spin) {
      if ((threadIdx.x & 63) == 0) report_error(a.err, a.err_host);
      return;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// s_waitcnt immediate waiting until at most n vector memory operations of
// the wave are outstanding (expcnt and lgkmcnt left open).
constexpr int vmcnt_wait(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }

#ifndef PRISMKV_POLL_STAGGER
#define PRISMKV_POLL_STAGGER 16
#endif
// The two generations of a poll: after the first is issued, the second waits
// PRISMKV_POLL_STAGGER x 64 cycles (about 0.4 us), so that thereafter they
// land that far apart and a published word is seen a quarter of a round trip
// after it lands on average, not half of one.  Measured at 64K (36 layers,
// four alternations): 0 -> 25.28, 8 -> 25.13, 12 -> 24.97, 16 -> 24.90,
// 20 -> 24.95, 24 -> 25.11, 32 -> 25.63 us per layer.
__device__ __forceinline__ void poll_stagger() {
  if constexpr (PRISMKV_POLL_STAGGER > 0) __builtin_amdgcn_s_sleep(PRISMKV_POLL_STAGGER);
}

#ifndef PRISMKV_POLL_GENS
#define PRISMKV_POLL_GENS 2
#endif
constexpr int kPollGens = PRISMKV_POLL_GENS;  // generations of a poll's loads in flight

// Polls published words with kPollGens generations of kLoads unconditional
// loads each in flight (issue(g) requests generation g, ready(g) takes it
// and returns whether every word has landed, uniform).  Nothing else is in flight
// after the drain, so each generation is waited for exactly with
// vmcnt((kPollGens - 1) kLoads), leaving the later ones outstanding; the
// generations are issued poll_stagger() apart and so keep landing apart.
// Gives up (report(), once) after `limit` + 1 generations found short.
template <int kLoads, typename Issue, typename Ready, typename Report>
__device__ __forceinline__ void poll_generations(Issue&& issue, Ready&& ready, Report&& report, int limit) {
  drain();
#pragma unroll
  for (int g = 0; g + 1 < kPollGens; ++g) {
    issue(g);
    poll_stagger();
  }
  for (int tries = 0;;) {
#pragma unroll
    for (int g = 0; g < kPollGens; ++g) {
      issue((g + kPollGens - 1) % kPollGens);
      __builtin_amdgcn_s_waitcnt(vmcnt_wait((kPollGens - 1) * kLoads));  // generation g has landed
      if (ready(g)) return;
      if (tries++ >= limit) {  // (a limit of 0 gives up at the first generation found short)
        report();
        return;
      }
    }
  }
}

// Bitmap row of a candidate key.  Landed keys always name a bucket below
// 3000; the clamp keeps a key read after a wait gave up in range too.
__device__ __forceinline__ int row_of(unsigned long long key) { return min(key_bucket(key), kF - 1); }

// Published words: the complement of the value's bits, so 0 = not yet.
__device__ __forceinline__ void pub2(unsigned long long* p, float a, float b) {
  st_dev(p, ~(((unsigned long long)__float_as_uint(b) << 32) | (unsigned long long)__float_as_uint(a)));
}
__device__ __forceinline__ float2 unpub2(unsigned long long r) {
  r = ~r;
  return make_float2(__uint_as_float((unsigned)r), __uint_as_float((unsigned)(r >> 32)));
}

// Phase 8: merges the 8 wave states stashed in LDS and publishes
// them per (head, 32-dim slice) as complemented words {max, den, acc[32]}:
// each slice has its own copy of (max, den), so every published word has
// exactly one reader.  Thread = (head tid >> 7, dim tid & 127).
__device__ __forceinline__ void publish_sliced(MfmaLds<kDT / 64>& lds, float* stp) {
  const int tid = threadIdx.x;
  __syncthreads();
  if (tid < (kDT / 64) * kHq) {
    const int k = tid >> 2, h = tid & 3;
    float M = -INFINITY;
#pragma unroll
    for (int i = 0; i < kDT / 64; ++i) M = fmaxf(M, lds.sm[i][h]);
    const float m = lds.sm[k][h];
    lds.wt[k][h] = m == -INFINITY ? 0.f : exp2f(m - M);
    if (k == 0) lds.mx[h] = M;
  }
  __syncthreads();
  const int h = tid >> 7, d = tid & (kD - 1);
  const float M = lds.mx[h];
  float den = 0.f, v = 0.f;
#pragma unroll
  for (int k = 0; k < kDT / 64; ++k) {
    const float wgt = lds.wt[k][h];
    den = fmaf(wgt, lds.sz[k][h], den);
    v = fmaf(wgt, lds.sacc[k][h][d], v);
  }
  float* sl = stp + (h * kSlices + (d >> 5)) * kSliceW;
  if ((d & 31) == 0)
    st_dev(reinterpret_cast<unsigned long long*>(sl),
           ~(((unsigned long long)__float_as_uint(den) << 32) | (unsigned long long)__float_as_uint(M)));
  st_dev(reinterpret_cast<unsigned*>(sl + 2 + (d & 31)), ~__float_as_uint(v));
}

// Phase 9 for (head h, slice c): polls the S published (max, den) pairs and
// the S x 32 accumulators of the slice, merges them exactly
// (out = sum_k e^(m_k - M) acc_k / sum_k e^(m_k - M) den_k, 0 if the
// denominator is 0), writes out[g][h][32c .. 32c + 32) and clears the words.
// Thread = (dim tid & 31, split group tid >> 5): splits k = group + 16 i.
template <int KW>
__device__ __forceinline__ void merge_slice(const DecodeArgs& a, int g, int h, int c, DecodeLds& lds) {
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, d = tid & 31, sg = tid >> 5;
  const int S = a.S;
  constexpr int kGroups = kDT / 32;  // 16
  const size_t stride = (size_t)kHq * kSlices * kSliceW;  // floats per split
  float* base = a.state + (size_t)g * S * stride + (h * kSlices + c) * kSliceW;
  // Polled with two generations of loads in flight: a word that lands just
  // after one generation was issued is seen by the next, half a round trip
  // later.  Every load is unconditional (published words keep their value
  // until this merge clears them), and nothing else is in flight (drained
  // first), so the explicit wait for a generation leaves the other one
  // outstanding; the compiler's own waits would otherwise take both.
  constexpr int kPer = 2 * KW;  // S <= 32 KW splits: thread (d, sg) reads splits sg + 16 i, i < kPer
  const unsigned long long* mzp =
      reinterpret_cast<const unsigned long long*>(base + (size_t)min(tid, S - 1) * stride);
  const unsigned* accp[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i)
    accp[i] = reinterpret_cast<const unsigned*>(base + (size_t)min(sg + kGroups * i, S - 1) * stride + 2 + d);
  unsigned long long rmz = 0, gmz[kPollGens];
  unsigned racc[kPer], gacc[kPollGens][kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) racc[i] = 0u;
  auto issue = [&](int gen) {
    gmz[gen] = ld_dev(mzp);
#pragma unroll
    for (int i = 0; i < kPer; ++i) gacc[gen][i] = ld_dev(accp[i]);
  };
  auto take = [&](int gen) {  // keep the first nonzero value of every word; true when all landed
    bool ok = true;
    if (tid < S) {
      rmz = rmz ? rmz : gmz[gen];
      ok = rmz != 0;
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i)
      if (sg + kGroups * i < S) {
        racc[i] = racc[i] ? racc[i] : gacc[gen][i];
        ok = ok && racc[i] != 0u;
      }
    return ok;
  };
  // each wave waits for its own words only: the first barrier below then
  // waits for every wave
  poll_generations<1 + kPer>(issue, [&](int gen) { return __ballot(!take(gen)) == 0; },
                              [&] { if (lane == 0) report_error(a.err, a.err_host); }, a.spin);
  if constexpr (KW <= 2) {
    // S <= 64: wave 0 holds every split's (max, den), so it derives M, the
    // splits' weights and the denominator alone and the other waves read the
    // weights behind one barrier (the same values and order as below)
    if (w == 0) {
      float2 mz = make_float2(-INFINITY, 0.f);
      if (tid < S) {
        const unsigned long long r = ~rmz;
        mz = make_float2(__uint_as_float((unsigned)r), __uint_as_float((unsigned)(r >> 32)));
      }
      const float M = wave_max(mz.x);
      const float wk = (tid < S && mz.x != -INFINITY) ? exp2f(mz.x - M) : 0.f;
      const float dsum = wave_sum(wk * mz.y);
      if (tid < S) lds.fin.mz[tid].x = wk;
      if (lane == 0) lds.fin.red[0] = dsum;
    }
    __syncthreads();
    float v = 0.f;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int k = sg + kGroups * i;
      if (k < S) v = fmaf(lds.fin.mz[k].x, __uint_as_float(~racc[i]), v);
    }
    lds.fin.part[sg][d] = v;
    __syncthreads();
    if (tid < 32) {
      const float den = lds.fin.red[0];
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < kGroups; ++i) acc += lds.fin.part[i][tid];
      if (a.out)  // the route-and-union launch merges only to clear (no output)
        a.out[((size_t)g * kHq + h) * kD + c * (kD / kSlices) + tid] = f32_to_bf16(den > 0.f ? acc / den : 0.f);
    }
  } else {
    // M = max over splits, den = sum of weighted denominators (fixed order)
    float2 mz = make_float2(-INFINITY, 0.f);
    if (tid < S) {
      const unsigned long long r = ~rmz;
      mz = make_float2(__uint_as_float((unsigned)r), __uint_as_float((unsigned)(r >> 32)));
      lds.fin.mz[tid] = mz;
    }
    float m = wave_max(mz.x);
    if (lane == 0) lds.fin.red[w] = m;
    __syncthreads();
    float M = -INFINITY;
  #pragma unroll
    for (int i = 0; i < kDT / 64; ++i) M = fmaxf(M, lds.fin.red[i]);
    const float wk = (tid < S && mz.x != -INFINITY) ? exp2f(mz.x - M) : 0.f;
    const float dsum = wave_sum(wk * mz.y);
    __syncthreads();  // everyone has read red[] as maxima
    if (lane == 0) lds.fin.red[w] = dsum;
    // weighted accumulators of this thread's splits
    float v = 0.f;
  #pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int k = sg + kGroups * i;
      if (k < S) {
        const float mk = lds.fin.mz[k].x;
        const float wgt = mk == -INFINITY ? 0.f : exp2f(mk - M);
        v = fmaf(wgt, __uint_as_float(~racc[i]), v);
      }
    }
    lds.fin.part[sg][d] = v;
    __syncthreads();
    if (tid < 32) {
      float den = 0.f;
  #pragma unroll
      for (int i = 0; i < kDT / 64; ++i) den += lds.fin.red[i];
      float acc = 0.f;
  #pragma unroll
      for (int i = 0; i < kGroups; ++i) acc += lds.fin.part[i][tid];
      if (a.out)  // the route-and-union launch merges only to clear (no output)
        a.out[((size_t)g * kHq + h) * kD + c * (kD / kSlices) + tid] = f32_to_bf16(den > 0.f ? acc / den : 0.f);
    }
  }
  // every word read above has been consumed (the barrier follows the last use)
  for (int i = tid; i < S * kSliceW; i += kDT) {
    const int k = i / kSliceW, e = i - k * kSliceW;
    st_dev(reinterpret_cast<unsigned*>(base + (size_t)k * stride + e), 0u);
  }
}

// Phase 4 for KW sets of 64 candidates per wave: wave w polls the published
// keys [64 KW w, 64 KW (w + 1)) straight into registers (each 16-lane row is
// one workgroup's list, already in rank order) and keeps their top 16.  The
// group's Top-16 lies within these 8 lists (a key with fewer than 16 greater
// keys overall has fewer than 16 in its own wave), so the rank of a listed
// key among all candidates, when below 16, is its rank among the 128 listed
// ones: thread t < 128 counts, for its key, the greater keys of each sorted
// list by binary search and writes the key to win[rank].
//
// The union's bitmap words are requested early: as soon as it has its list,
// each wave loads words [tw p, tw (p + 1)) of the rows of its kPrefetch best
// keys, which land while the ranks are counted; the group's winners are
// usually among them.  Once the ranks are known, each wave ORs the rows of its
// prefetched keys that won into lds.sel.ors[w] and marks their ranks in
// lds.cover[w]; the union loads only the winners no wave prefetched.
// Without kPrefetchRows (the route-only and the capped launch) nothing is
// prefetched.
//
// `early` lets the fused decode request its early tail rows here (phase 6
// consumes them): prepare() once the candidates have landed, issue() after
// the barrier that follows the bitmap-word requests -- so every wave's words
// are ahead of every wave's tail rows in the CU's memory queue and the
// selection never waits for the tail -- and wait_words() before the words
// are used (a wait that leaves the tail rows in flight).
constexpr int kPrefetch = 6;

// Phase 5's tile count, published for the ids offsets.  The decode publishes
// one status word per tile (cleared by workgroup 0 after the final merge).
// The route-only launch has no final hand-off, so it publishes the count to
// each later tile r in a slot of r's own ([G][S][S] words in the split-state
// region, which it does not otherwise use): every slot has one reader, which
// clears it once read.
template <bool kSlots>
__device__ __forceinline__ void publish_count(const DecodeArgs& a, int g, int p, int total, int lane) {
  if constexpr (kSlots) {
    unsigned* slots = reinterpret_cast<unsigned*>(a.state) + (size_t)g * a.S * a.S + p;
    for (int r = p + 1 + lane; r < a.S; r += 64) st_dev(slots + (size_t)r * a.S, kReady | (unsigned)total);
  } else if (lane == 0) {
    st_dev(&a.status[(size_t)g * a.S + p], kReady | (unsigned)total);
  }
}

template <bool B>
struct BoolTag {
  static constexpr bool value = B;
};

struct NoEarly {
  __device__ void prepare() {}
  __device__ void barrier() { __syncthreads(); }
  __device__ void issue() {}
  __device__ void wait_words() const {}
};
template <int KW, bool kPrefetchRows = true, class Early = NoEarly, int kPfChunks = 1>
__device__ __forceinline__ void final_top16(const DecodeArgs& a, int g, int p, DecodeLds& lds, Early& early) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nk = a.S * kTop;
  const unsigned long long* cg = a.cand + (size_t)g * a.S * kTop;
  unsigned long long v[KW];
  {
    // two generations of unconditional loads in flight (nothing else is,
    // after the drain), each waited for explicitly: a key that lands just
    // after one generation was issued is seen by the next
    unsigned long long r[KW], gen[kPollGens][KW];
    auto issue = [&](int gg) {
#pragma unroll
      for (int k = 0; k < KW; ++k) gen[gg][k] = ld_dev(cg + min((w * KW + k) * 64 + lane, nk - 1));
    };
    auto take = [&](int gg) {
      bool ok = true;
#pragma unroll
      for (int k = 0; k < KW; ++k) {
        r[k] = r[k] ? r[k] : gen[gg][k];
        ok = ok && ((w * KW + k) * 64 + lane >= nk || r[k] != 0);
      }
      return __ballot(!ok) == 0;
    };
#pragma unroll
    for (int k = 0; k < KW; ++k) r[k] = 0;
    poll_generations<KW>(issue, take, [&] { if (lane == 0) report_error(a.err, a.err_host); }, a.spin);
#pragma unroll
    for (int k = 0; k < KW; ++k) v[k] = (w * KW + k) * 64 + lane < nk ? ~r[k] : 0ull;
  }
  early.prepare();
  const unsigned long long best = sorted_rows_top16<KW>(v);
  if (lane < kTop) lds.sel.best[kTop * w + lane] = best;
  if (threadIdx.x < kTop) lds.win[threadIdx.x] = 0ull;  // ranks no key fills stay empty
  const int nw = (a.H + 31) / 32;
  const int wd = p * a.tw + lane;
  const bool word = lane < a.tw && wd < nw;
  // kPfChunks = 2 (tiles of more than one chunk): the second chunk's words
  // are requested too
  constexpr bool two = kPrefetchRows && kPfChunks > 1;
  const bool word2 = kTileWords + lane < a.tw && wd + kTileWords < nw;
  unsigned long long pk[kPrefetch];
  uint32_t pw[kPrefetch], pw2[kPrefetch];
#pragma unroll
  for (int r = 0; r < kPrefetch; ++r) {
    pk[r] = readlane_u64(best, r);  // rank r of this wave's list (uniform)
    pw[r] = 0u;
    pw2[r] = 0u;
    if constexpr (kPrefetchRows) {
      // every rank issues its loads (an empty key's through an empty resource),
      // so the loads after these are counted exactly when pw is waited for
      const uint32_t* row = a.bits + ((size_t)g * kF + row_of(pk[r])) * a.row_words;
      const __amdgpu_buffer_rsrc_t res = raw_buffer(row, pk[r] ? (int)a.row_words * 4 : 0);
      pw[r] = load_nt4_buf(res, (unsigned)min(wd, nw - 1) * 4u);
      if constexpr (two) pw2[r] = load_nt4_buf(res, (unsigned)min(wd + kTileWords, nw - 1) * 4u);
    }
  }
  early.barrier();
  early.issue();
  constexpr int kListed = kDT / 64 * kTop;  // 128
  if (threadIdx.x < kListed) {
    const unsigned long long x = lds.sel.best[threadIdx.x];
    if (x != 0ull) {  // nonzero keys are unique, so their ranks are
      // binary searches of the 8 descending lists, step by step across the
      // lists, so each step's 8 LDS reads are in flight together
      constexpr int kLists = kDT / 64;
      int pos[kLists];
#pragma unroll
      for (int L = 0; L < kLists; ++L) pos[L] = 0;
#pragma unroll
      for (int step = kTop / 2; step > 0; step >>= 1) {
        unsigned long long y[kLists];
#pragma unroll
        for (int L = 0; L < kLists; ++L) y[L] = lds.sel.best[kTop * L + pos[L] + step - 1];
#pragma unroll
        for (int L = 0; L < kLists; ++L) pos[L] += y[L] > x ? step : 0;
      }
      unsigned long long y[kLists];
#pragma unroll
      for (int L = 0; L < kLists; ++L) y[L] = lds.sel.best[kTop * L + pos[L]];
      int rank = 0;
#pragma unroll
      for (int L = 0; L < kLists; ++L) rank += pos[L] + (y[L] > x ? 1 : 0);  // 16 when the whole list is greater
      if (rank < kTop) lds.win[rank] = x;
    }
  }
  __syncthreads();
  // the winners are exactly the candidates >= the last winner's key (nonzero
  // keys are unique); a prefetched winner's rank = the winners above it
  const unsigned long long win = lane < kTop ? lds.win[lane] : 0ull;
  const int need = __popcll(__ballot(win != 0ull));
  const unsigned long long last = need ? readlane_u64(win, need - 1) : ~0ull;
  uint32_t part = 0u, part2 = 0u;
  unsigned covered = 0u;
  early.wait_words();
#pragma unroll
  for (int r = 0; r < kPrefetch; ++r)
    if (pk[r] != 0ull && pk[r] >= last) {  // uniform
      part |= pw[r];
      part2 |= pw2[r];
      covered |= 1u << __popcll(__ballot(lane < need && win > pk[r]));
    }
  lds.sel.ors[w][lane] = word ? part : 0u;
  if constexpr (two) lds.sel.ors2[w][lane] = word2 ? part2 : 0u;
  if (lane == 0) lds.cover[w] = kPrefetchRows ? covered : 0u;
  if (w == 0) {
    if (lane < kTop) lds.sel_rows[lane] = lane < need ? row_of(win) : 0;  // the union reads rows < need only
    if (lane == 0) lds.need = need;
  }
  __syncthreads();
}

// Phases 1-4: the group's Top-16 (rank order) into lds.win (every wave) and
// lds.sel_rows / lds.need.  Without kUnion only workgroup 0 runs phase 4;
// kPrefetchRows requests the union's bitmap words in phase 4.
template <int KW, bool kUnion = true, bool kPrefetchRows = kUnion, class Early = NoEarly, int kPfChunks = 1>
__device__ __forceinline__ void decode_select(const DecodeArgs& a, int g, int p, DecodeLds& lds, Early& early) {
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int S = a.S;
  // moment tiles kper * p + j, j < own: contiguous 32 KB tiles, one stream per workgroup
  const int kper = (kChunks + S - 1) / S;
  const int own = max(0, min(kper, kChunks - kper * p));
  auto tile = [&](int j) { return kper * p + j; };
  // ---- 1. score the own tiles: half 0 takes tile 0, half 1 tile 1, and
  // both halves tile 2 (half h its part h), in one pass.  Loads go out in one
  // batch with no branch: q first (so staging it waits for nothing else),
  // then the bucket sizes, then the tiles (a missing tile repeats a valid
  // one), so the products of the first tiles run while the rest lands.
  {
    const int half = tid >> 8, t = tid & 255;
    unsigned qv = load_query512(a.q, g, tid);
    asm volatile("" ::: "memory");  // q is issued first, whatever the scheduler's pressure estimate
    const int c0 = min(tile(half), kChunks - 1), c2 = min(tile(2), kChunks - 1);
    const int* cg = a.counts + (size_t)g * kFP + (t & 31);
    const int n0 = __builtin_nontemporal_load(cg + c0 * kChunk), n2 = __builtin_nontemporal_load(cg + c2 * kChunk);
    float4 m4[8], m2[4];
    load_tile(a.moments, g, c0, t, m4);
    load_half_tile(a.moments, g, c2, half, t, m2);
    // every load above is issued before q is first used (the asm takes q as
    // an operand, so even its conversion cannot move up between the loads)
    asm volatile("" : "+v"(qv) :: "memory");
    store_query512(qv, lds.score.qq, tid);
    __syncthreads();
    // logits: tile `half` in threads t < 128 of each half, tile 2 in threads
    // 128..255 of half 0; each head's 32 buckets fill half a wave
    const float2 l = tile_logits3(lds.score.qq, m4, m2, tid, lds.score.tile, lds.score.split, n0, n2);
    const bool mine = t < kHq * kChunk ? half < own : half == 0 && own > 2;  // uniform per wave
    if (mine) {
      const int j = t < kHq * kChunk ? half : 2, h = (t >> 5) & 3;
      const float x = t < kHq * kChunk ? l.x : l.y;
      lds.tl[j][h][t & 31] = x;
      const float2 st = chunk_stats(x);
      if ((t & 31) == 0) pub2(&a.stats[((size_t)g * kChunks + tile(j)) * kHq + h], st.x, st.y);
    }
  }
  __syncthreads();
  // ---- 2. the group's per-head (M, 1/Z), from the statistics as they land
  if (w < kHq) {
    const int h = w;
    const unsigned long long* st = a.stats + (size_t)g * kChunks * kHq + h;
    // two generations of unconditional loads in flight, as in final_top16
    unsigned long long r0 = 0, r1 = 0, gen[kPollGens][2];
    auto issue = [&](int gg) {
      gen[gg][0] = ld_dev(st + min(lane, kChunks - 1) * kHq);
      gen[gg][1] = ld_dev(st + min(lane + 64, kChunks - 1) * kHq);
    };
    auto take = [&](int gg) {
      r0 = r0 ? r0 : gen[gg][0];
      r1 = r1 ? r1 : gen[gg][1];
      return __ballot(!((lane >= kChunks || r0 != 0) && (lane + 64 >= kChunks || r1 != 0))) == 0;
    };
    poll_generations<2>(issue, take, [&] { if (lane == 0) report_error(a.err, a.err_host); }, a.spin);
    const float2 mz = merge_chunk_stats([&](int ch) { return unpub2(ch == lane ? r0 : r1); });
    if (lane == 0) {
      lds.gmax[h] = mz.x;
      lds.grz[h] = mz.y;
    }
  }
  __syncthreads();
  // ---- 3. this workgroup's 16 best keys: wave j < own ranks tile j's 32
  // keys (row sorts, then rows 0 and 1 merged), wave 0 merges the tiles'
  // lists (row j = tile j, empty rows zero)
  if (w < own) {  // uniform
    const int b = lane & 31;
    uint64_t key = 0;
    if (lane < kChunk) {
      const float lv[kHq] = {lds.tl[w][0][b], lds.tl[w][1][b], lds.tl[w][2][b], lds.tl[w][3][b]};
      key = bucket_key(lv, lds.gmax, lds.grz, tile(w) * kChunk + b);
    }
    unsigned long long v = row_sort_desc(key);
    v = merge_top16(v, xor_rows_u64<16>(v));  // rows 0, 1: the tile's top 16
    if (lane < kTop) lds.sel.own[kTop * w + lane] = v;
  }
  __syncthreads();
  if (w == 0) {
    const unsigned long long best = rows_top16(lane < kTop * own ? lds.sel.own[lane] : 0ull);  // lane j < 16: rank j
    if (lane < kTop) st_dev(&a.cand[((size_t)g * S + p) * kTop + lane], ~best);
  }
  // ---- 4. the group's Top-16 from its S x 16 candidates, as they land
  if constexpr (!kUnion) {
    if (p != 0) return;
  }
  final_top16<KW, kUnion && kPrefetchRows, Early, kPfChunks>(a, g, p, lds, early);
}
template <int KW, bool kUnion = true, bool kPrefetchRows = kUnion>
__device__ __forceinline__ void decode_select(const DecodeArgs& a, int g, int p, DecodeLds& lds) {
  NoEarly none;
  decode_select<KW, kUnion, kPrefetchRows>(a, g, p, lds, none);
}

// ---- 4b. (capped launch) the strict unique cap's budgeted walk over the
// group's ranked buckets (src/prismkv/core.py:149-163), spread over the
// group's workgroups: workgroup p owns words [tw p, tw (p + 1)) of every
// ranked row, thread t word tw p + t, and keeps its word of the union U of
// the kept rows.  The ranks go in windows of 4.  For the window's rows,
// x_i = row_i \ U, each workgroup counts its tokens of every membership
// pattern m = 1..15 (the tokens in exactly the rows of m among the 4),
// publishes the 15 counts and reads every workgroup's: row i then adds the
// tokens whose pattern holds i and no row kept before it in the window,
// which decides the window's rows in rank order exactly as the
// one-bucket-at-a-time walk does, and every workgroup decides the same from
// the same sums.
// The greedy walk never drops a kept row, so the union only grows: the
// tokens a window adds are final once it is decided.  Each window's new
// tokens are appended to the workgroup's row list (rows[], in window order)
// and attended by segment(lo, n) while the NEXT window's counts cross
// between the workgroups (segment(-1, 0), the tail share, goes with the
// first window), so the gather runs during the walk's hand-offs instead of
// after the last one.  Returns this thread's word of U (0 past the tile),
// the kept ranks in *keep, the rows listed in *listed and the first row not
// yet attended in *attended (the caller attends [*attended, *listed) after a
// barrier).
constexpr int kWindow = 4;
constexpr int kWindows = kTop / kWindow;
constexpr int kPacked = 8;  // 15 pattern counts, two 16-bit counts per word
// The ranked rows' words of the tile wait in dynamic LDS after the row list
// ([kTop][kDT], thread t's at t), not in registers: the attention between
// the windows needs those.
constexpr int kWalkWordsBytes = kTop * kDT * (int)sizeof(uint32_t);

template <typename Segment>
__device__ __forceinline__ uint32_t capped_walk(const DecodeArgs& a, int g, int p, DecodeLds& lds, int* rows,
                                                unsigned* keep, int* listed_out, int* attended_out,
                                                Segment&& segment) {
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int nr = lds.need;
  const int nw = (a.H + 31) / 32, wd = p * a.tw + tid;
  const bool col = tid < a.tw && wd < nw;
  const uint32_t wmask = !col ? 0u : (wd == nw - 1 && (a.H & 31)) ? (1u << (a.H & 31)) - 1u : ~0u;
  // every ranked row's word, all requested at once, kept in LDS
  uint32_t* words = reinterpret_cast<uint32_t*>(rows + 32 * a.tw);
  if (a.rows16) {
    // aligned rows and tiles: wave w takes ranks w and w + 8, lane l words
    // 4 l .. 4 l + 3 of each 256-word part of the tile (16-byte loads: a
    // CU's load instructions, not their bytes, bound this)
    constexpr int kRanks = kTop / (kDT / 64), kParts = kDT / 256;  // 2, 2
    uint4 q[kRanks][kParts];
#pragma unroll
    for (int i = 0; i < kRanks; ++i) {
      const int r = w + (kDT / 64) * i;
      const uint32_t* row = a.bits + ((size_t)g * kF + (r < nr ? lds.sel_rows[r] : 0)) * a.row_words;
      const __amdgpu_buffer_rsrc_t res = raw_buffer(row, r < nr ? (int)a.row_words * 4 : 0);  // past the row: 0
#pragma unroll
      for (int j = 0; j < kParts; ++j)
        q[i][j] = 256 * j < a.tw ? load_nt16_buf(res, (unsigned)(p * a.tw + 256 * j + 4 * lane) * 4u)
                                 : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int i = 0; i < kRanks; ++i)
#pragma unroll
      for (int j = 0; j < kParts; ++j) {
        const int t = 256 * j + 4 * lane, wt = p * a.tw + t;
        uint32_t m[4] = {q[i][j].x, q[i][j].y, q[i][j].z, q[i][j].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          m[e] = t + e < a.tw && wt + e < nw ? m[e] : 0u;
          if (wt + e == nw - 1 && (a.H & 31)) m[e] &= (1u << (a.H & 31)) - 1u;
        }
        *reinterpret_cast<uint4*>(&words[(w + (kDT / 64) * i) * kDT + t]) = make_uint4(m[0], m[1], m[2], m[3]);
      }
    __syncthreads();  // every rank's words, for every thread
  } else {
    uint32_t v[kTop];
    const uint32_t* gb = a.bits + (size_t)g * kF * a.row_words + (col ? wd : 0);
#pragma unroll
    for (int r = 0; r < kTop; ++r)
      v[r] = nr > 0 ? __builtin_nontemporal_load(gb + (size_t)lds.sel_rows[r < nr ? r : nr - 1] * a.row_words) : 0u;
#pragma unroll
    for (int r = 0; r < kTop; ++r) words[r * kDT + tid] = v[r] & (r < nr ? wmask : 0u);
  }
  const int lim = a.limit < a.H ? a.limit : a.H;  // a union never exceeds H
  unsigned* rec = a.walk + (size_t)g * kWindows * a.S * kPacked;
  uint32_t U = 0u;
  int total = 0, listed = 0, attended = 0;
  unsigned kept = 0u;
  bool tail_done = false;
#pragma unroll
  for (int k = 0; k < kWindows; ++k) {
    if (kWindow * k >= nr) break;  // uniform
    uint32_t x[kWindow];
#pragma unroll
    for (int i = 0; i < kWindow; ++i) x[i] = words[(kWindow * k + i) * kDT + tid] & ~U;
    // pattern m = (rows 0, 1: m & 3) x (rows 2, 3: m >> 2)
    const uint32_t lo[4] = {~x[0] & ~x[1], x[0] & ~x[1], ~x[0] & x[1], x[0] & x[1]};
    const uint32_t hi[4] = {~x[2] & ~x[3], x[2] & ~x[3], ~x[2] & x[3], x[2] & x[3]};
    int packed[kPacked];  // per wave: <= 2048 per count, so two fit a word
#pragma unroll
    for (int j = 0; j < kPacked; ++j) {
      const int m0 = 2 * j + 1, m1 = 2 * j + 2;
      const int c0 = __popc(lo[m0 & 3] & hi[m0 >> 2]);
      const int c1 = m1 < 16 ? __popc(lo[m1 & 3] & hi[(m1 >> 2) & 3]) : 0;
      packed[j] = c0 | c1 << 16;
    }
    const int wsum = wave_sum8(packed);  // lane 8j: the wave's packed word j
    if ((lane & 7) == 0) lds.walk_part[w][lane >> 3] = wsum;
    __syncthreads();
    // the workgroup's counts (<= 16384 each: no carry between the halves),
    // published complemented
    if (w == 0 && lane < kPacked) {
      unsigned sum = 0u;
#pragma unroll
      for (int ww = 0; ww < kDT / 64; ++ww) sum += (unsigned)lds.walk_part[ww][lane];
      st_dev(&rec[((size_t)k * a.S + p) * kPacked + lane], ~sum);
    }
    // while they cross: the rows decided so far (before the first window,
    // the tail share), by every wave
    if (!tail_done) {
      segment(-1, 0);
      tail_done = true;
    } else {
      segment(attended, listed - attended);
      attended = listed;
    }
    if (w == 0) {
      // every workgroup's counts, lane l summing word l & 7 of workgroups
      // (l >> 3) + 8 i
      const int j = lane & 7;
      int s0 = 0, s1 = 0;
      for (int q0 = lane >> 3; q0 < a.S; q0 += 32) {
        // two generations of unconditional loads in flight (nothing else
        // is, after the drain), each waited for explicitly, as in the
        // final merge
        unsigned r[4] = {0u, 0u, 0u, 0u}, gen[kPollGens][4];
        auto issue = [&](int gg) {
#pragma unroll
          for (int t = 0; t < 4; ++t)
            gen[gg][t] = ld_dev(&rec[((size_t)k * a.S + min(q0 + 8 * t, a.S - 1)) * kPacked + j]);
        };
        auto take = [&](int gg) {
          bool done = true;
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            r[t] = r[t] ? r[t] : gen[gg][t];
            done = done && (q0 + 8 * t >= a.S || r[t] != 0u);
          }
          return __ballot(!done) == 0;
        };
        poll_generations<4>(issue, take, [&] { if (lane == 0) report_error(a.err, a.err_host); }, a.spin);
#pragma unroll
        for (int t = 0; t < 4; ++t)
          if (q0 + 8 * t < a.S) {
            const unsigned c = ~r[t];
            s0 += (int)(c & 0xFFFFu);
            s1 += (int)(c >> 16);
          }
      }
      // across lane bits 3, 4, 5 (DPP row rotation, then permlane swaps)
      s0 += __float_as_int(xor8(__int_as_float(s0)));
      s1 += __float_as_int(xor8(__int_as_float(s1)));
      s0 += (int)xor16_u((unsigned)s0);
      s1 += (int)xor16_u((unsigned)s1);
      s0 += (int)xor32_u((unsigned)s0);
      s1 += (int)xor32_u((unsigned)s1);
      // lane j < 8: the group's counts of patterns 2j + 1 (s0) and 2j + 2 (s1)
      int cnt[16];
      cnt[0] = 0;
#pragma unroll
      for (int jj = 0; jj < kPacked; ++jj) {
        cnt[2 * jj + 1] = __builtin_amdgcn_readlane(s0, jj);
        if (2 * jj + 2 < 16) cnt[2 * jj + 2] = __builtin_amdgcn_readlane(s1, jj);
      }
      unsigned kw = 0u;  // the window's kept rows so far
#pragma unroll
      for (int i = 0; i < kWindow; ++i) {
        if (kWindow * k + i >= nr) break;
        int add = 0;
#pragma unroll
        for (int m = 1; m < 16; ++m) add += ((m >> i) & 1) && !(m & kw) ? cnt[m] : 0;
        if (total + add <= lim) {
          kw |= 1u << i;
          total += add;
        }
      }
      if (lane == 0) lds.walk_keep = kw;
    }
    __syncthreads();
    const unsigned kw = lds.walk_keep;
    uint32_t inc = 0u;  // this word's tokens the window adds
#pragma unroll
    for (int i = 0; i < kWindow; ++i) inc |= (kw >> i) & 1u ? x[i] : 0u;
    U |= inc;
    kept |= kw << (kWindow * k);
    // append them to the row list (the next segment reads it after the
    // next window's first barrier; the caller barriers after the last)
    const int c = __popc(inc), incl = wave_scan_i(c);
    if (lane == 63) lds.chunk_rows[w] = incl;
    __syncthreads();
    int at = listed, add = 0;
#pragma unroll
    for (int ww = 0; ww < kDT / 64; ++ww) {
      const int t = lds.chunk_rows[ww];
      at += ww < w ? t : 0;
      add += t;
    }
    at += incl - c;
    for (uint32_t m = inc; m; m &= m - 1u) rows[at++] = wd * 32 + (int)__builtin_ctz(m);
    listed += add;
  }
  if (!tail_done) segment(-1, 0);  // nothing ranked: the tail share alone
  *keep = kept;
  *listed_out = listed;
  *attended_out = attended;
  return U;
}

// KW = 64-key candidate sets per wave, ceil(S / 32): one instantiation per
// range of S, so a launch carries only the selection code it runs.  With
// kGiven the selection is not computed but read from features / valid (as
// a strict unique cap leaves them) and phases 5-9 run on it.  With kCap the
// strict unique cap's walk (phase 4b) runs between the selection and the
// union, on the same launch.
// The early tail request of the fused decode: wave w's 16-row block of the
// workgroup's tail rows, [t_lo + 16 w, t_lo + 16 w + 16) clipped to its share
// [t_lo, t_hi), into ek / ev in the MFMA operand layouts of mfma_blocks16.
// prepare() derives the rows from the tail word (long landed by then);
// issue() requests them: 8 loads in every wave, through empty resources
// for a wave without early rows.  A load costs its CU issue time even then,
// so the host takes this kernel only for tails that give most waves a block.
struct EarlyTail {
  const DecodeArgs& a;
  int g, p, tail_word;
  int& n;  // this wave's early rows (uniform), for phase 6
  uint4 (&ek)[1][4];
  uint4 (&ev)[1][4];
  int r0 = 0, T = 0;
  __device__ void prepare() {
    T = a.tail_dev ? min(max(tail_word, 0), a.T) : a.T;
    const int per = (T + a.S - 1) / a.S;
    const int lo = min(T, p * per), hi = min(T, lo + per);
    const int wu = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    n = __builtin_amdgcn_readfirstlane(max(0, min(16, hi - (lo + 16 * wu))));
    r0 = a.H + lo + 16 * wu;  // the K/V row of the block's first row
  }
  __device__ void issue() {
    {  // every wave (an empty resource for a wave without early rows: no memory access)
      const int lane = threadIdx.x & 63, j = lane & 15, qd = lane >> 4;
      const int kv_bytes = __builtin_amdgcn_readfirstlane(n > 0 ? (a.H + T) * 2 * kD : 0);
      const __amdgpu_buffer_rsrc_t kb = raw_buffer(a.k + (size_t)g * a.ks, kv_bytes);
      const __amdgpu_buffer_rsrc_t vb = raw_buffer(a.v + (size_t)g * a.vs, kv_bytes);
      const unsigned ko = (unsigned)(r0 + (j < n ? j : 0)) * (2 * kD) + 16 * qd;
#pragma unroll
      for (int c = 0; c < 4; ++c) ek[0][c] = load_nt16_buf(kb, ko + 64 * c);
#pragma unroll
      for (int t = 0; t < 4; ++t)
        ev[0][t] = load_nt16_buf(vb, (unsigned)(r0 + (4 * qd + t < n ? 4 * qd + t : 0)) * (2 * kD) + 16 * j);
    }
  }
  __device__ void barrier() { __syncthreads(); }
  // Loads complete in order: with at most the 8 early loads outstanding,
  // everything requested before them (the bitmap words) has landed.  The
  // explicit wait keeps the compiler from waiting for every load instead.
  __device__ void wait_words() const { __builtin_amdgcn_s_waitcnt(8 | (0x7 << 4) | (0xf << 8)); }
};

// The route-only launch after phase 5 (what Native8B.route() runs: the
// selection, the union tiles and the ids, no attention): wave 0 polls the
// lower tiles' counts from this tile's slots (clearing each once read), the
// tile writes its ids, and the group's last workgroup writes count, features /
// valid / raw and clears the statistics and candidates -- every workgroup
// published its count after its phase 4, so none reads them any more.
template <int KW>
__device__ __forceinline__ void route_finish(const DecodeArgs& a, int g, int p, DecodeLds& lds, const int* rows) {
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, S = a.S;
  const int n_sel = lds.nsel;
  if (w == 0) {
    constexpr int kC = (KW + 1) / 2;  // 64-lane chunks of S <= 32 KW lower tiles
    unsigned* slots = reinterpret_cast<unsigned*>(a.state) + ((size_t)g * S + p) * S;  // tile p's slots
    unsigned v[kC], gen[kPollGens][kC];
#pragma unroll
    for (int c = 0; c < kC; ++c) v[c] = 0u;
    auto issue = [&](int gg) {
#pragma unroll
      for (int c = 0; c < kC; ++c) gen[gg][c] = ld_dev(slots + min(64 * c + lane, S - 1));
    };
    auto take = [&](int gg) {
      bool ok = true;
#pragma unroll
      for (int c = 0; c < kC; ++c)
        if (64 * c + lane < p) {
          v[c] = v[c] ? v[c] : gen[gg][c];
          ok = ok && v[c] != 0u;
        }
      return __ballot(!ok) == 0;
    };
    poll_generations<kC>(issue, take, [&] { if (lane == 0) report_error(a.err, a.err_host); }, a.spin);
    unsigned prefix = 0;
#pragma unroll
    for (int c = 0; c < kC; ++c) {
      const int q = 64 * c + lane;
      prefix += (unsigned)wave_sum_i(q < p ? (int)(v[c] & ~kReady) : 0);
      if (q < p) st_dev(slots + q, 0u);  // read: clear for the next launch
    }
    if (lane == 0) {
      lds.base = (int)prefix;
      if (p == S - 1) a.count[g] = (int32_t)(prefix + (unsigned)n_sel);
    }
  }
  __syncthreads();
  int32_t* dst = a.ids + (size_t)g * a.ids_stride + lds.base;
  for (int i = tid; i < n_sel; i += kDT) dst[i] = rows[i];
  if (p == S - 1) {
    if (w == 0)
      write_selection(lds.win, lds.need, a.counts + (size_t)g * kFP, a.features + (size_t)g * kTop,
                      a.valid + (size_t)g * kTop, a.raw + g);
    for (int i = tid; i < kChunks * kHq; i += kDT) st_dev(&a.stats[(size_t)g * kChunks * kHq + i], 0ull);
    for (int i = tid; i < S * kTop; i += kDT) st_dev(&a.cand[(size_t)g * S * kTop + i], 0ull);
  }
}

// kWide: union tiles of 65-128 words (the host's choice when tw > 64), whose
// two chunks' words phase 4 requests.
template <int KW, bool kGiven = false, bool kCap = false, bool kEarlyTail = false, bool kRouteOnly = false,
          bool kWide = false>
__global__ __launch_bounds__(kDT) void decode_kernel(DecodeArgs a) {
  const int p = blockIdx.x, g = blockIdx.y, tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  __shared__ DecodeLds lds;
  extern __shared__ __align__(16) int rows[];  // the tile's selected tokens, ascending (32 tw of them)
  // the tail length: the host's T, or the device word clamped to it (the
  // host checked the K/V extents for T).  The word is requested now, with
  // no branch (without a device word the load reads q and is ignored), so
  // it has long landed when the attention first uses it.
  const int tail_word = ld_dev(a.tail_dev ? a.tail_dev : reinterpret_cast<const int*>(a.q));
  // Early tail (the uncapped decode): each wave's 16-row block of the
  // workgroup's tail rows is requested in phase 4, behind the bitmap words,
  // so it streams in while the selection finishes and the union is built
  // (HBM is otherwise idle then); in phase 6 it takes one slot of the
  // wave's first round, whose other blocks' loads are issued before it is
  // waited for (it can land after the union is built).
  constexpr bool kEarly = kEarlyTail && !kGiven && !kCap && !kRouteOnly && !PRISMKV_VALU_ATTENTION;
  constexpr int kPfChunks = kWide && !kGiven && !kCap ? 2 : 1;  // union chunks prefetched in phase 4
  int early_n = 0;
  uint4 ek[1][4], ev[1][4];

  // attention over a given id list: no selection, no union (uniform)
  const bool id_list = kGiven && a.ids_in != nullptr;
  if constexpr (kGiven) {
    // ---- 1-4. the given selection: the valid, in-range buckets in order (an
    // out-of-range id selects nothing, as in union_kernel); no row is
    // prefetched, so the union loads every selected row
    if (w == 0 && !id_list) {
      bool ok = false;
      int f = 0;
      if (lane < kTop) {
        // both requested at once (not the id only where valid holds)
        const float vl = a.valid[(size_t)g * kTop + lane];
        const int64_t fe = a.features[(size_t)g * kTop + lane];
        ok = vl > 0.f && fe >= 0 && fe < kF;
        f = (int)fe;
      }
      const unsigned long long m = __ballot(ok);
      if (ok) lds.sel_rows[__popcll(m & ((1ull << lane) - 1ull))] = f;
      if (lane == 0) lds.need = __popcll(m);
    }
    lds.sel.ors[w][lane] = 0u;
    if (lane == 0) lds.cover[w] = 0u;
    __syncthreads();
  } else if constexpr (!kCap) {
    // ---- 1-4. the group's Top-16 (and the early tail rows requested)
    if constexpr (kEarly) {
      EarlyTail early{a, g, p, tail_word, early_n, ek, ev};
      decode_select<KW, true, true, EarlyTail, kPfChunks>(a, g, p, lds, early);
    } else {
      NoEarly none;
      decode_select<KW, true, true, NoEarly, kPfChunks>(a, g, p, lds, none);
    }
  }
  // ---- 1-4b. (capped) the group's Top-16; the budgeted walk over it runs
  // in phase 6, interleaved with the attention of the rows it has decided
  if constexpr (kCap) decode_select<KW, true, false>(a, g, p, lds);

  // ---- 5. union tile: OR the selected rows over words [tw p, tw (p + 1)), compact.
  // One 64-word chunk (histories up to 64K at 8 groups): wave 0 ORs the rows
  // the waves prefetched in phase 4 and loads any winner none prefetched.
  // More chunks: wave w < ceil(tw / 64) takes chunk w -- in the wide variant
  // (two chunks, both prefetched) as wave 0 does its one chunk, otherwise by
  // loading every selected row; the chunks' counts give each its offset.
  // (Phase 4's final barrier publishes need and sel_rows.)
  const int nw = (a.H + 31) / 32;
  if constexpr (kCap) {
    // the capped launch lists its rows during the walk (phase 6)
  } else if (id_list) {
    // ---- 5'. the workgroup's entries of the group's list (count ids, then
    // the T tail rows H .. H + T - 1).  A list of at most kDT S entries (a
    // sparse union) goes in 16-position chunks p, p + S, p + 2S, ... (kDT
    // entries a workgroup at most), positions that do not depend on count,
    // so their ids are requested together with count instead of after it
    // lands.  A longer list goes in contiguous even shares, which keep each
    // workgroup's K/V reads local; its ids are read once count has landed.
    const int32_t* idg = a.ids_in + (size_t)g * a.ids_stride;
    const int given_cnt = a.count_in[g];
    const int id0 = idg[min((p + a.S * (tid >> 4)) * 16 + (tid & 15), (int)a.ids_stride - 1)];  // in the id row
    const int cnt = min(max(given_cnt, 0), a.H), total = cnt + a.T;
    const bool inter = total <= kDT * a.S;  // uniform
    const int chunks = (total + 15) / 16, per = (total + a.S - 1) / a.S;
    const int mine = chunks > p ? (chunks - p + a.S - 1) / a.S : 0;  // interleaved: this workgroup's chunks
    const int lo = min(total, p * per);                             // contiguous: the first position
    const int n = inter ? (mine ? 16 * (mine - 1) + min(16, total - 16 * (p + a.S * (mine - 1))) : 0)
                        : min(total, lo + per) - lo;
    auto pos_of = [&](int k) { return inter ? (p + a.S * (k >> 4)) * 16 + (k & 15) : lo + k; };
    bool bad = p == 0 && tid == 0 && given_cnt != cnt;
    for (int k = tid; k < n; k += kDT) {
      const int j = pos_of(k);
      int r = a.H + (j - cnt);
      if (j < cnt) {
        const int id = inter && k == tid ? id0 : idg[j];
        bad |= id < 0 || id >= a.H;
        r = min(max(id, 0), a.H - 1);
      }
      rows[k] = r;
    }
    if (bad) report_error(a.err, a.err_host, kErrIds);  // the rows stay in range (clamped)
    if (tid == 0) lds.nsel = n;
  } else if (a.tw <= kTileWords) {
    if (w == 0) {
      const int nr = lds.need;
      const int wd = p * a.tw + lane;
      uint32_t m = 0u;
      unsigned covered = 0u;
#pragma unroll
      for (int k = 0; k < kDT / 64; ++k) {
        m |= lds.sel.ors[k][lane];
        covered |= lds.cover[k];
      }
      const unsigned missing = ((1u << nr) - 1u) & ~covered;  // winners' ranks no wave prefetched (uniform)
      if (missing && lane < a.tw && wd < nw) {
        // one round of loads: every rank loads (a covered one repeats the first
        // missing row) and only the missing ones are kept
        const uint32_t* gb = a.bits + (size_t)g * kF * a.row_words + wd;
        const int first = __builtin_ctz(missing);
        uint32_t v[kTop];
#pragma unroll
        for (int r = 0; r < kTop; ++r)
          v[r] = __builtin_nontemporal_load(gb + (size_t)lds.sel_rows[(missing >> r) & 1u ? r : first] * a.row_words);
#pragma unroll
        for (int r = 0; r < kTop; ++r) m |= (missing >> r) & 1u ? v[r] : 0u;
      }
      if (wd == nw - 1 && (a.H & 31)) m &= (1u << (a.H & 31)) - 1u;
      const int n = __popc(m);
      const int incl = wave_scan_i(n);
      int at = incl - n;
      while (m) {
        rows[at++] = wd * 32 + (int)__builtin_ctz(m);
        m &= m - 1u;
      }
      const int total = __builtin_amdgcn_readlane(incl, 63);
      if (lane == 0) lds.nsel = total;
      publish_count<kRouteOnly>(a, g, p, total, lane);
    }
  } else {
    const int chunks = (a.tw + kTileWords - 1) / kTileWords;  // <= 8
    const int cw = w * kTileWords + lane, wd = p * a.tw + cw;
    const int nr = lds.need;
    uint32_t m = 0u;
    int n = 0, incl = 0;
    if (w < chunks) {
      if constexpr (kPfChunks > 1) {
        // chunk w < 2 (both prefetched): the waves' ORs, then one round of
        // loads for the winners no wave prefetched (every rank loads, a
        // covered one repeating the first missing row, and only the missing
        // ones are kept)
        unsigned covered = 0u;
#pragma unroll
        for (int k = 0; k < kDT / 64; ++k) {
          m |= w ? lds.sel.ors2[k][lane] : lds.sel.ors[k][lane];
          covered |= lds.cover[k];
        }
        const unsigned missing = ((1u << nr) - 1u) & ~covered;  // uniform
        if (missing && cw < a.tw && wd < nw) {
          const uint32_t* gb = a.bits + (size_t)g * kF * a.row_words + wd;
          const int first = __builtin_ctz(missing);
          uint32_t v[kTop];
#pragma unroll
          for (int r = 0; r < kTop; ++r)
            v[r] = __builtin_nontemporal_load(gb + (size_t)lds.sel_rows[(missing >> r) & 1u ? r : first] * a.row_words);
#pragma unroll
          for (int r = 0; r < kTop; ++r) m |= (missing >> r) & 1u ? v[r] : 0u;
        }
      } else if (nr > 0 && cw < a.tw && wd < nw) {
        const uint32_t* gb = a.bits + (size_t)g * kF * a.row_words + wd;
        uint32_t v[kTop];
#pragma unroll
        for (int r = 0; r < kTop; ++r)
          v[r] = __builtin_nontemporal_load(gb + (size_t)lds.sel_rows[r < nr ? r : nr - 1] * a.row_words);
#pragma unroll
        for (int r = 0; r < kTop; ++r) m |= v[r];
      }
      if (wd == nw - 1 && (a.H & 31)) m &= (1u << (a.H & 31)) - 1u;
      n = __popc(m);
      incl = wave_scan_i(n);
      if (lane == 63) lds.chunk_rows[w] = incl;
    }
    __syncthreads();  // every chunk's count, for the offsets
    if (w < chunks) {
      int off = 0;
      for (int k = 0; k < w; ++k) off += lds.chunk_rows[k];
      int at = off + incl - n;
      while (m) {
        rows[at++] = wd * 32 + (int)__builtin_ctz(m);
        m &= m - 1u;
      }
      if (w == chunks - 1) {
        const int total = __builtin_amdgcn_readlane(off + incl, 63);
        if (lane == 0) lds.nsel = total;
        publish_count<kRouteOnly>(a, g, p, total, lane);
      }
    }
  }
  __syncthreads();
  if constexpr (kRouteOnly) {
    route_finish<KW>(a, g, p, lds, rows);
    return;
  }
  // the lower tiles' counts, requested once this workgroup's first K/V loads
  // are in flight and used after the attention (no barrier in between)
  unsigned lower[kMaxSplits / 64];  // 0 = not loaded yet (a workgroup without rows never prefetches)
#pragma unroll
  for (int c = 0; c < kMaxSplits / 64; ++c) lower[c] = (64 * c + lane < p) ? 0u : kReady;

  // ---- 6. attention over the tile's tokens, then its tail rows, in 16-row
  // blocks dealt round-robin from the last wave down (block b to wave
  // 7 - b % 8, so wave 0, which also sums the ids offset, gets the fewest),
  // four blocks per round with every K/V load of the round issued up front
  // and the round's blocks taken as one step of the online softmax.  Only
  // the list's last block is partial: a wave's block whose lanes mostly
  // repeat one row still costs about a third of a full block's load time,
  // so whole blocks are dealt rather than equal row counts.
  int tail_now = tail_word;
  // (the given-selection kernels: without this the compiler converts the word
  // to a scalar right after its load, which waits a whole round trip at launch)
  if constexpr (kGiven) asm volatile("" : "+v"(tail_now));
  const int T = a.tail_dev ? min(max(tail_now, 0), a.T) : a.T;
  const int tail_per = id_list ? 0 : (T + a.S - 1) / a.S;  // an id list holds its tail rows
  const int t_lo = min(T, p * tail_per), t_hi = min(T, t_lo + tail_per);
  // the list: the tile's tokens, then the tail rows the early blocks did not take
  const int early_rows = kEarly ? min(t_hi - t_lo, kEarlyRows) : 0;
  int n_sel = kCap ? 0 : lds.nsel;  // the capped launch's: the walk's final list
  uint32_t walked = 0u;             // the capped launch's word of the kept rows' union (thread = tile word)
  int walked_at = 0;                // ... and its tokens' offset in the tile's ascending ids
  {
    const int j = lane & 15, qd = lane >> 4;
    const int last_row = a.H + T - 1;
    const uint16_t* kg = a.k + (size_t)g * a.ks;
    const uint16_t* vg = a.v + (size_t)g * a.vs;
    constexpr int kWaves = kDT / 64;
#if PRISMKV_VALU_ATTENTION
    // VALU attention (the A/B alternative, built with -DPRISMKV_VALU_ATTENTION=1):
    // lane (q16, slot) holds dims 8 q16 .. 8 q16 + 8 of the rows of its slot
    // (4 slots of 16 lanes, 4 rows each per 16-row block); P stays fp32
    const int q16 = j, slot = qd;
    float qf[kHq][8];
#pragma unroll
    for (int h = 0; h < kHq; ++h) {
      unpack8(*reinterpret_cast<const uint4*>(a.q + ((size_t)g * kHq + h) * kD + 8 * q16), qf[h]);
#pragma unroll
      for (int i = 0; i < 8; ++i) qf[h][i] *= kLog2eScale;
    }
    SlotState st;
    st.m = -INFINITY;
    st.z = 0.f;
#pragma unroll
    for (int h = 0; h < kHq; ++h)
#pragma unroll
      for (int i = 0; i < 8; ++i) st.acc[h][i] = 0.f;
#else
    MfmaAttn st;
    mfma_init(st, a.q + (size_t)g * kHq * kD);
    // the group's K and V rows [0, last_row] as buffer resources (row
    // positions are clamped into that range, so every offset is in bounds)
    const int kv_bytes = __builtin_amdgcn_readfirstlane((last_row + 1) * 2 * kD);
    const __amdgpu_buffer_rsrc_t kbuf = raw_buffer(kg, kv_bytes), vbuf = raw_buffer(vg, kv_bytes);
#endif
    // blocks per wave per round (the capped launch keeps the walk's state
    // live across its segments: two blocks, 256 rows per workgroup in
    // flight, still cover HBM's latency)
    constexpr int kPerRound = kCap ? 2 : 4;
    // the wave index made explicitly uniform keeps the block indices in
    // scalar registers (fewer VGPRs for the round's loads)
    const int wu = __builtin_amdgcn_readfirstlane(w);
    // attends n rows, row r at K/V row pos_of(r) (clamped into the group's
    // rows; rows past n repeat the block's first row and are masked); with
    // `look`, wave 0 requests the lower tiles' counts once its first K/V
    // loads are in flight.  pre_n > 0: the wave's early tail block (ek / ev,
    // pre_n rows, requested in phase 4 and possibly still in flight) takes
    // slot 0 of the first round, whose other slots take the list's first
    // blocks, so the round's loads are issued before the early rows are
    // waited for.
    auto attend_rows = [&](auto&& pos_of, int n, bool look, auto pre_tag, int pre_n) {
      const int n_blocks = (n + 15) >> 4;
      auto row_pos = [&](int r, int base) {
        const int pos = pos_of(r < n ? r : base);
        return pos < 0 ? 0 : (pos > last_row ? last_row : pos);
      };
      // one round: the list's blocks k0 + 8 i in slots i (slots i + 1 with
      // the early block in slot 0)
      auto round = [&](int k0, auto pre_tag) {
        constexpr int kShift = decltype(pre_tag)::value ? 1 : 0;
        uint4 kr[kPerRound][4], vr[kPerRound][4];
#pragma unroll
        for (int i = 0; i < kPerRound; ++i) {
          if (i < kShift) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              kr[i][c] = ek[0][c];
              vr[i][c] = ev[0][c];
            }
            continue;
          }
          const int base = 16 * (k0 + kWaves * (i - kShift));
          if (base < n) {  // uniform per wave
#if PRISMKV_VALU_ATTENTION
#pragma unroll
            for (int b = 0; b < 4; ++b) {
              const size_t at = (size_t)row_pos(base + 4 * slot + b, base) * kD + 8 * q16;
              kr[i][b] = load_nt16(kg + at);
              vr[i][b] = load_nt16(vg + at);
            }
#else
            const unsigned ko = (unsigned)row_pos(base + j, base) * (2 * kD) + 16 * qd;
#pragma unroll
            for (int c = 0; c < 4; ++c) kr[i][c] = load_nt16_buf(kbuf, ko + 64 * c);
#pragma unroll
            for (int t = 0; t < 4; ++t)
              vr[i][t] = load_nt16_buf(vbuf, (unsigned)row_pos(base + 4 * qd + t, base) * (2 * kD) + 16 * j);
#endif
          }
        }
        asm volatile("" ::: "memory");  // every load of the round is in flight before any is used
        if (look && k0 == kWaves - 1 - wu && wu == 0) {
#pragma unroll
          for (int c = 0; c < kMaxSplits / 64; ++c) {
            const int qq = 64 * c + lane;
            if (qq < p) lower[c] = ld_dev(&a.status[(size_t)g * a.S + qq]);
          }
        }
#if PRISMKV_VALU_ATTENTION
#pragma unroll
        for (int i = 0; i < kPerRound; ++i) {
          const int base = 16 * (k0 + kWaves * i);
          if (base < n) attend_step(qf, kr[i], vr[i], max(0, min(4, n - base - 4 * slot)), st);
        }
#else
        int nv[kPerRound];
#pragma unroll
        for (int i = 0; i < kPerRound; ++i)
          nv[i] = i < kShift ? pre_n : max(0, min(16, n - 16 * (k0 + kWaves * (i - kShift))));
        mfma_blocks16<kPerRound>(st, kr, vr, nv);
#endif
      };
      int k0 = kWaves - 1 - wu;
#if !PRISMKV_VALU_ATTENTION
      if constexpr (decltype(pre_tag)::value) {
        if (pre_n > 0) {  // uniform
          round(k0, BoolTag<true>{});
          k0 += (kPerRound - 1) * kWaves;
        }
      }
#endif
      if constexpr (kCap || kGiven) {
        // (the rounds written out: as calls of `round` the capped launch's
        // code is scheduled differently and measured 0.14 us slower, the
        // all-read control's 0.6 us)
        for (; k0 < n_blocks; k0 += kPerRound * kWaves) {  // blocks k0 + 8 i
          uint4 kr[kPerRound][4], vr[kPerRound][4];
#pragma unroll
          for (int i = 0; i < kPerRound; ++i) {
            const int base = 16 * (k0 + kWaves * i);
            if (base < n) {  // uniform per wave
#if PRISMKV_VALU_ATTENTION
#pragma unroll
              for (int b = 0; b < 4; ++b) {
                const size_t at = (size_t)row_pos(base + 4 * slot + b, base) * kD + 8 * q16;
                kr[i][b] = load_nt16(kg + at);
                vr[i][b] = load_nt16(vg + at);
              }
#else
              const unsigned ko = (unsigned)row_pos(base + j, base) * (2 * kD) + 16 * qd;
#pragma unroll
              for (int c = 0; c < 4; ++c) kr[i][c] = load_nt16_buf(kbuf, ko + 64 * c);
#pragma unroll
              for (int t = 0; t < 4; ++t)
                vr[i][t] = load_nt16_buf(vbuf, (unsigned)row_pos(base + 4 * qd + t, base) * (2 * kD) + 16 * j);
#endif
            }
          }
          asm volatile("" ::: "memory");  // every load of the round is in flight before any is used
          if (look && k0 == kWaves - 1 - wu && wu == 0) {
#pragma unroll
            for (int c = 0; c < kMaxSplits / 64; ++c) {
              const int qq = 64 * c + lane;
              if (qq < p) lower[c] = ld_dev(&a.status[(size_t)g * a.S + qq]);
            }
          }
#if PRISMKV_VALU_ATTENTION
#pragma unroll
          for (int i = 0; i < kPerRound; ++i) {
            const int base = 16 * (k0 + kWaves * i);
            if (base < n) attend_step(qf, kr[i], vr[i], max(0, min(4, n - base - 4 * slot)), st);
          }
#else
          int nv[kPerRound];
#pragma unroll
          for (int i = 0; i < kPerRound; ++i) nv[i] = max(0, min(16, n - 16 * (k0 + kWaves * i)));
          mfma_blocks16<kPerRound>(st, kr, vr, nv);
#endif
        }
      } else {
        for (; k0 < n_blocks; k0 += kPerRound * kWaves) round(k0, BoolTag<false>{});
      }
    };
    if constexpr (kCap) {
      // ---- 4b + 6. the walk, each window's hand-off overlapped with the
      // attention of the rows decided before it (the tail share first)
      unsigned keep = 0u;
      int listed = 0, attended = 0;
      walked = capped_walk(a, g, p, lds, rows, &keep, &listed, &attended, [&](int lo, int n) {
        if (lo < 0)
          attend_rows([&](int r) { return a.H + t_lo + r; }, t_hi - t_lo, false, BoolTag<false>{}, 0);
        else
          attend_rows([&](int r) { return rows[lo + r]; }, n, false, BoolTag<false>{}, 0);
      });
      // the tile's count for the look-back, and its ascending ids' offsets
      const int c = __popc(walked), incl = wave_scan_i(c);
      if (lane == 63) lds.chunk_rows[w] = incl;
      __syncthreads();  // also: the last window's rows are listed
#pragma unroll
      for (int ww = 0; ww < kWaves; ++ww) walked_at += ww < w ? lds.chunk_rows[ww] : 0;
      walked_at += incl - c;
      n_sel = listed;
      if (tid == 0) st_dev(&a.status[(size_t)g * a.S + p], kReady | (unsigned)listed);
      attend_rows([&](int r) { return rows[attended + r]; }, listed - attended, true, BoolTag<false>{}, 0);
      // the kept buckets (in rank order, compacted) into features / valid /
      // raw, by a workgroup that merges nothing
      if (p == a.S - 1 && w == 0) {
        const int nkept = __popc(keep);
        const bool kept = lane < kTop && ((keep >> lane) & 1u);
        const int b = lane < kTop ? lds.sel_rows[lane] : 0;
        if (lane < kTop) {
          int64_t* fg = a.features + (size_t)g * kTop;
          if (kept) fg[__popc(keep & ((1u << lane) - 1u))] = b;
          if (lane >= nkept) fg[lane] = 0;
          a.valid[(size_t)g * kTop + lane] = lane < nkept ? 1.f : 0.f;
        }
        const int nb = wave_sum_i(kept ? a.counts[(size_t)g * kFP + b] : 0);
        if (lane == 0) a.raw[g] = nb;
      }
    } else {
      // the tile's tokens and the tail rows the early blocks did not take;
      // the early block goes with the first round
      const int n_rows = n_sel + (t_hi - t_lo) - early_rows;
      attend_rows([&](int r) { return r < n_sel ? rows[r] : a.H + t_lo + early_rows + (r - n_sel); }, n_rows,
                  !id_list, BoolTag<true>{}, early_n);
    }

    // each wave stashes its state as soon as its attention ends: the LDS
    // union's earlier users (phases 1-5) are done, and no wave reads it
    // during the attention
#if PRISMKV_VALU_ATTENTION
    {
      // merge the wave's 4 slot states (lane bits 4, 5) into the stash layout
      const int h = q16 & 3;
      float M = fmaxf(st.m, xor16(st.m));
      M = fmaxf(M, xor32(M));  // head h's max over the slots (lanes with q16 & 3 == h)
      const float wgt = st.m == -INFINITY ? 0.f : exp2f(st.m - M);
      float z = wgt * st.z;
      z += xor16(z);
      z += xor32(z);
      if (slot == 0 && q16 < kHq) {
        lds.mf.sm[w][h] = M;
        lds.mf.sz[w][h] = z;
      }
#pragma unroll
      for (int hh = 0; hh < kHq; ++hh) {
        const float wh = __shfl(wgt, slot * 16 + hh);  // weight of head hh in this lane's slot
        float acc[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          acc[i] = wh * st.acc[hh][i];
          acc[i] += xor16(acc[i]);
          acc[i] += xor32(acc[i]);
        }
        if (slot == 0) {
          float4* dst = reinterpret_cast<float4*>(&lds.mf.sacc[w][hh][8 * q16]);
          dst[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
          dst[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
        }
      }
    }
#else
    mfma_stash(st, lds.mf, w);
#endif

    // ---- 7. the tile's global ids offset (ids are written after phase 8)
    if (w == 0 && !id_list) {
      const unsigned* tiles = a.status + (size_t)g * a.S;
      unsigned prefix = 0;
#pragma unroll
      for (int c = 0; c < kMaxSplits / 64; ++c) {
        const int qq = 64 * c + lane;
        unsigned v = lower[c];
        wait_all([&] {
          if (qq < p && !(v & kReady)) v = ld_dev(tiles + qq);
          return (v & kReady) != 0u;
        }, a);
        prefix += (unsigned)wave_sum_i(qq < p ? (int)(v & ~kReady) : 0);
      }
      if (lane == 0) {
        lds.base = (int)prefix;
        if (p == a.S - 1) a.count[g] = (int32_t)(prefix + (unsigned)n_sel);
      }
    }

    // ---- 8. the split state (after the look-back: its publication tells
    // workgroup 0 that this workgroup no longer reads any published word);
    // publish_sliced's first barrier waits for every wave's stash and also
    // publishes lds.base to every wave
    publish_sliced(lds.mf, a.state + (size_t)(g * a.S + p) * kHq * kSlices * kSliceW);
  }
  if constexpr (kCap) {
    // ascending, from the union word: rows[] holds them in window order
    int32_t* dst = a.ids + (size_t)g * a.ids_stride + lds.base + walked_at;
    const int wd = p * a.tw + tid;
    for (uint32_t m = walked; m; m &= m - 1u) *dst++ = wd * 32 + (int)__builtin_ctz(m);
  } else if (!id_list) {
    int32_t* dst = a.ids + (size_t)g * a.ids_stride + lds.base;
    for (int i = tid; i < n_sel; i += kDT) dst[i] = rows[i];
  }
  // the selection (features / valid / raw) is written here, after the
  // attention, by the group's last workgroup (not a merger), so that its
  // bucket-size loads neither wait behind the early tail rows nor delay a merge
  if constexpr (!kGiven && !kCap)
    if (p == a.S - 1 && w == 0)
      write_selection(lds.win, lds.need, a.counts + (size_t)g * kFP, a.features + (size_t)g * kTop,
                      a.valid + (size_t)g * kTop, a.raw + g);
  // ---- 9. workgroups 0..15 each merge one (head, 32-dim slice) of the S
  // split states into out[g] and clear the words they read; workgroup 0
  // also clears the group's statistics, candidates and tile counts (every
  // workgroup has published its state, so none reads them any more)
  if (p >= kMergers) return;
  merge_slice<KW>(a, g, p >> 2, p & 3, lds);
  if (p == 0) {
    for (int i = tid; i < kChunks * kHq; i += kDT) st_dev(&a.stats[(size_t)g * kChunks * kHq + i], 0ull);
    for (int i = tid; i < a.S * kTop; i += kDT) st_dev(&a.cand[(size_t)g * a.S * kTop + i], 0ull);
    for (int i = tid; i < a.S; i += kDT) st_dev(&a.status[(size_t)g * a.S + i], 0u);
    if constexpr (kCap)
      for (int i = tid; i < kWindows * a.S * kPacked; i += kDT) st_dev(&a.walk[(size_t)g * kWindows * a.S * kPacked + i], 0u);
  }
}

// Stage 1 alone in one launch (the separate route of the capped and
// compatibility paths): phases 1-4 as in decode_kernel, except that only
// workgroup 0 ranks the group's candidates.  It writes features / valid /
// raw and clears the group's statistics and candidates: every workgroup read
// the statistics before publishing its candidates, and no other reads those,
// so the workspace is all zero again when the launch ends.
template <int KW>
__global__ __launch_bounds__(kDT) void route_kernel(DecodeArgs a) {
  const int p = blockIdx.x, g = blockIdx.y, tid = threadIdx.x, w = tid >> 6;
  __shared__ DecodeLds lds;
  decode_select<KW, false>(a, g, p, lds);
  if (p != 0) return;
  if (w == 0)
    write_selection(lds.win, lds.need, a.counts + (size_t)g * kFP, a.features + (size_t)g * kTop,
                    a.valid + (size_t)g * kTop, a.raw + g);
  for (int i = tid; i < kChunks * kHq; i += kDT) st_dev(&a.stats[(size_t)g * kChunks * kHq + i], 0ull);
  for (int i = tid; i < a.S * kTop; i += kDT) st_dev(&a.cand[(size_t)g * a.S * kTop + i], 0ull);
}

}  // namespace
}  // namespace prismkv

using namespace prismkv;

// Workgroups per group: 256 / groups (32 for 8 groups), so the whole launch is
// resident at once, one workgroup per CU, at any history; the union tile
// grows with H instead (tw <= 512 words up to kFusedMaxHistory).
static int decode_splits(int groups) { return std::min(kMaxSplits, std::max(kMinSplits, 256 / std::max(groups, 1))); }
static constexpr int kFusedMaxHistory = kMinSplits * kTileTokens;  // 524288

// The process-wide bound of every inter-workgroup wait, passed to each launch.
static int g_spin_limit = kSpinLimit;
namespace prismkv {
int spin_limit() { return __atomic_load_n(&g_spin_limit, __ATOMIC_RELAXED); }
}  // namespace prismkv

// Work layout (bytes) for the split count of `groups` groups:
// err (the error word, then the host-word slot at byte 8) | stats | candidates | status | state | walk.
// The capped walk's records come last: the other launches touch the first
// `walk` bytes only (the route-and-union launch keeps its count slots in the
// state region).
struct DecodeWorkLayout {
  size_t err, stats, cand, status, state, walk, total;
  DecodeWorkLayout(int groups, int S) {
    size_t o = 0;
    auto take = [&](size_t n) { const size_t at = o; o += (n + 255) & ~(size_t)255; return at; };
    err = take(sizeof(unsigned));
    stats = take((size_t)groups * kChunks * kHq * sizeof(unsigned long long));
    cand = take((size_t)groups * S * kTop * sizeof(unsigned long long));
    status = take((size_t)groups * S * sizeof(unsigned));
    state = take((size_t)groups * S * kHq * kSlices * kSliceW * sizeof(float));
    walk = take((size_t)groups * kWindows * S * kPacked * sizeof(unsigned));
    total = o;
  }
};

// Workgroups of decode_kernel resident on device `dev` at once (CUs x blocks
// per CU) with the largest row list (64 KB of dynamic LDS) and the capped
// walk's words (32 KB), queried once per device; the instantiations are
// allowed that much dynamic LDS here.  The
// route-only kernels (no dynamic LDS) are counted at the same size, which
// can only understate them.
static int resident_workgroups() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cached[dev] == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    // the instantiations differ only in the selection code; take the least resident
    int least = 1 << 30;
    const void* fns[] = {reinterpret_cast<const void*>(decode_kernel<1>), reinterpret_cast<const void*>(decode_kernel<2>),
                         reinterpret_cast<const void*>(decode_kernel<4>), reinterpret_cast<const void*>(decode_kernel<8>),
                         reinterpret_cast<const void*>(route_kernel<1>),  reinterpret_cast<const void*>(route_kernel<2>),
                         reinterpret_cast<const void*>(route_kernel<4>),  reinterpret_cast<const void*>(route_kernel<8>),
                         reinterpret_cast<const void*>(decode_kernel<1, true>),
                         reinterpret_cast<const void*>(decode_kernel<2, true>),
                         reinterpret_cast<const void*>(decode_kernel<4, true>),
                         reinterpret_cast<const void*>(decode_kernel<8, true>),
                         reinterpret_cast<const void*>(decode_kernel<1, false, true>),
                         reinterpret_cast<const void*>(decode_kernel<2, false, true>),
                         reinterpret_cast<const void*>(decode_kernel<4, false, true>),
                         reinterpret_cast<const void*>(decode_kernel<8, false, true>),
                         reinterpret_cast<const void*>(decode_kernel<1, false, false, true>),
                         reinterpret_cast<const void*>(decode_kernel<2, false, false, true>),
                         reinterpret_cast<const void*>(decode_kernel<4, false, false, true>),
                         reinterpret_cast<const void*>(decode_kernel<8, false, false, true>),
                         reinterpret_cast<const void*>(decode_kernel<1, false, false, false, true>),
                         reinterpret_cast<const void*>(decode_kernel<2, false, false, false, true>),
                         reinterpret_cast<const void*>(decode_kernel<4, false, false, false, true>),
                         reinterpret_cast<const void*>(decode_kernel<8, false, false, false, true>),
                         reinterpret_cast<const void*>(decode_kernel<1, false, false, false, false, true>),
                         reinterpret_cast<const void*>(decode_kernel<2, false, false, false, false, true>),
                         reinterpret_cast<const void*>(decode_kernel<4, false, false, false, false, true>),
                         reinterpret_cast<const void*>(decode_kernel<1, false, false, true, false, true>),
                         reinterpret_cast<const void*>(decode_kernel<2, false, false, true, false, true>),
                         reinterpret_cast<const void*>(decode_kernel<4, false, false, true, false, true>),
                         reinterpret_cast<const void*>(decode_kernel<1, false, false, false, true, true>),
                         reinterpret_cast<const void*>(decode_kernel<2, false, false, false, true, true>),
                         reinterpret_cast<const void*>(decode_kernel<4, false, false, false, true, true>)};
    // (the capped launches' row list is followed by the walk's words)
    const int dyn = kTileTokens * (int)sizeof(int) + kWalkWordsBytes;
    for (const void* fn : fns) {
      if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, dyn) != hipSuccess) return 0;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kDT, dyn) != hipSuccess) return 0;
      least = std::min(least, per_cu);
    }
    per_cu = least;
    cached[dev] = cus * per_cu;
  }
  return cached[dev];
}

// Every host-side check of a decode launch, before anything is enqueued:
// 0, or -1 for a size, range, pointer or residency the launch cannot take.
// limit >= 0: the capped launch (route, the strict unique cap's walk, union + attention).
static int decode_check(uint64_t q, uint64_t moments, uint64_t counts, uint64_t bits, uint64_t k, uint64_t v,
                        uint64_t work, uint64_t features, uint64_t valid, uint64_t raw, uint64_t ids, uint64_t count,
                        uint64_t out, bool given, int groups, int H, int T, int capacity, int64_t row_words,
                        int64_t ks, int64_t vs, int64_t ids_stride, int64_t limit, bool route_only = false) {
  if (groups < 1 || groups > 65535 || H < 1 || H > kFusedMaxHistory || T < 0 || capacity < H) return kBadSize;
  if (given && limit >= 0) return kBadSize;
  if (row_words < (H + 31) / 32 || ids_stride < H) return kBadSize;
  if (!route_only) {  // the route-and-union launch reads no K/V and writes no out
    if (ks < (int64_t)(H + T) * kD || vs < (int64_t)(H + T) * kD) return kBadSize;
    if (((int64_t)H + T) * 2 * kD > INT32_MAX) return kBadSize;  // K/V rows are read through 32-bit buffer offsets
    if (!k || !v || !out) return kBadSize;
  }
  // a given selection needs neither the moment tables nor raw
  if (!q || (!given && (!moments || !counts || !raw)) || !bits || !work || !features || !valid || !ids || !count)
    return kBadSize;
  if (decode_splits(groups) > resident_workgroups()) return kBadSize;  // a group's workgroups must be resident together
  return 0;
}

// One fused variant's launch for S workgroups per group: KW = ceil(S / 32)
// 64-key candidate sets per wave (the wide variant is never taken above
// S = 128, so it has no KW = 8 instantiation).
template <bool kGiven, bool kCap, bool kEarlyTail, bool kRouteOnly, bool kWide>
static void launch_decode(int S, dim3 grid, size_t dyn, hipStream_t s, const DecodeArgs& a) {
  const dim3 block(kDT);
  if (S <= 32) hipLaunchKernelGGL((decode_kernel<1, kGiven, kCap, kEarlyTail, kRouteOnly, kWide>), grid, block, dyn, s, a);
  else if (S <= 64) hipLaunchKernelGGL((decode_kernel<2, kGiven, kCap, kEarlyTail, kRouteOnly, kWide>), grid, block, dyn, s, a);
  else if (S <= 128) hipLaunchKernelGGL((decode_kernel<4, kGiven, kCap, kEarlyTail, kRouteOnly, kWide>), grid, block, dyn, s, a);
  else if constexpr (!kWide) hipLaunchKernelGGL((decode_kernel<8, kGiven, kCap, kEarlyTail, kRouteOnly, false>), grid, block, dyn, s, a);
}

// Enqueues a decode launch whose arguments decode_check accepted.
static int decode_launch(uint64_t q, uint64_t moments, uint64_t counts, uint64_t bits, uint64_t k, uint64_t v,
                         uint64_t work, uint64_t features, uint64_t valid, uint64_t raw, uint64_t ids, uint64_t count,
                         uint64_t out, const int* tail_dev, bool given, int groups, int H, int T, int64_t row_words,
                         int64_t ks, int64_t vs, int64_t ids_stride, uint64_t stream, unsigned* err, int64_t limit,
                         bool route_only = false) {
  const int S = decode_splits(groups);
  const DecodeWorkLayout L(groups, S);
  char* w = reinterpret_cast<char*>(work);
  DecodeArgs a;
  a.q = reinterpret_cast<const uint16_t*>(q);
  a.moments = reinterpret_cast<const float*>(moments);
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
  a.tw = ((H + 31) / 32 + S - 1) / S;
  // the capped walk reads its words 4 a lane: a tile of a multiple of 4
  // words, and rows16 when the rows are of a multiple of 4 words too
  if (limit >= 0) a.tw = (a.tw + 3) & ~3;
  a.rows16 = limit >= 0 && row_words % 4 == 0;
  a.tail_dev = tail_dev;
  a.stats = reinterpret_cast<unsigned long long*>(w + L.stats);
  a.cand = reinterpret_cast<unsigned long long*>(w + L.cand);
  a.status = reinterpret_cast<unsigned*>(w + L.status);
  // the workspace's own error word and host-word slot, or the caller's word
  a.err = err ? err : reinterpret_cast<unsigned*>(w + L.err);
  a.err_host = err ? nullptr : error_host_slot(a.err);
  a.spin = spin_limit();
  a.state = reinterpret_cast<float*>(w + L.state);
  a.walk = reinterpret_cast<unsigned*>(w + L.walk);
  a.limit = (int)std::min<int64_t>(limit, H);
  a.features = reinterpret_cast<int64_t*>(features);
  a.valid = reinterpret_cast<float*>(valid);
  a.raw = reinterpret_cast<int*>(raw);
  a.ids = reinterpret_cast<int32_t*>(ids);
  a.ids_stride = ids_stride;
  a.count = reinterpret_cast<int32_t*>(count);
  a.out = reinterpret_cast<uint16_t*>(out);
  a.ids_in = nullptr;
  a.count_in = nullptr;
  const dim3 grid(S, groups);
  hipStream_t s = (hipStream_t)stream;
  const size_t rows_bytes = (size_t)32 * a.tw * sizeof(int);  // the tile's row list (dynamic LDS)
  // wide: union tiles of 65-128 words, both chunks prefetched (S <= 128 at
  // every history the single launch takes, 8 groups above 64K)
  const bool wide = a.tw > kTileWords && a.tw <= kPrefetchChunks * kTileWords && S <= 128;
  if (route_only) {
    if (wide) launch_decode<false, false, false, true, true>(S, grid, rows_bytes, s, a);
    else launch_decode<false, false, false, true, false>(S, grid, rows_bytes, s, a);
  } else if (limit >= 0) {
    launch_decode<false, true, false, false, false>(S, grid, rows_bytes + kWalkWordsBytes, s, a);
  } else if (given) {
    launch_decode<true, false, false, false, false>(S, grid, rows_bytes, s, a);
  } else if ((T + S - 1) / S >= kEarlyRows / 2) {
    // tails that give most waves an early block: the early-tail variant
    if (wide) launch_decode<false, false, true, false, true>(S, grid, rows_bytes, s, a);
    else launch_decode<false, false, true, false, false>(S, grid, rows_bytes, s, a);
  } else {
    if (wide) launch_decode<false, false, false, false, true>(S, grid, rows_bytes, s, a);
    else launch_decode<false, false, false, false, false>(S, grid, rows_bytes, s, a);
  }
  return (int)hipGetLastError();
}

// A decode launch on a caller's workspace of work_bytes bytes, which must
// hold prismkv_decode_work_bytes(groups, capacity).
static int decode_impl(uint64_t q, uint64_t moments, uint64_t counts, uint64_t bits, uint64_t k, uint64_t v,
                       uint64_t work, uint64_t features, uint64_t valid, uint64_t raw, uint64_t ids, uint64_t count,
                       uint64_t out, const int* tail_dev, bool given, int groups, int H, int T, int capacity,
                       int64_t row_words, int64_t ks, int64_t vs, int64_t ids_stride, size_t work_bytes,
                       uint64_t stream, int64_t limit = -1) {
  if (groups < 1 || groups > 65535) return kBadSize;
  if (work_bytes < DecodeWorkLayout(groups, decode_splits(groups)).total) return kBadSize;
  const int rc = decode_check(q, moments, counts, bits, k, v, work, features, valid, raw, ids, count, out, given,
                              groups, H, T, capacity, row_words, ks, vs, ids_stride, limit);
  if (rc) return rc;
  return decode_launch(q, moments, counts, bits, k, v, work, features, valid, raw, ids, count, out, tail_dev, given,
                       groups, H, T, row_words, ks, vs, ids_stride, stream, nullptr, limit);
}

// ---- stage 3 over a given id list ---------------------------------------
// The decode's phases 6-9 with each workgroup's rows read from the group's id
// list (count[g] ids, then the T tail rows: every S-th 16-row chunk of a list
// of at most 512 S entries, even contiguous shares of a longer one) instead
// of a union tile: round-robin 16-row MFMA blocks, the sliced split
// states and the 16 merging workgroups, with the decode's bounded waits and
// error word (word 0 of the region, its host-word slot at byte 8).
namespace prismkv {

size_t attend_list_work_bytes(int groups) {
  return groups < 1 ? 0 : DecodeWorkLayout(groups, decode_splits(groups)).total;
}

int attend_list(uint64_t q, uint64_t k, uint64_t v, uint64_t ids, uint64_t count, uint64_t work, uint64_t out,
                int groups, int H, int T, int64_t ks, int64_t vs, int64_t ids_stride, uint64_t stream) {
  const int S = decode_splits(groups);
  // every row of a workgroup's share must fit its dynamic LDS list
  if (H + T < 1 || (int64_t)(H + T) > (int64_t)kTileTokens * S || S > resident_workgroups()) return kBadSize;
  const DecodeWorkLayout L(groups, S);
  char* w = reinterpret_cast<char*>(work);
  DecodeArgs a{};
  a.q = reinterpret_cast<const uint16_t*>(q);
  a.k = reinterpret_cast<const uint16_t*>(k);
  a.v = reinterpret_cast<const uint16_t*>(v);
  a.ks = ks;
  a.vs = vs;
  a.H = H;
  a.T = T;
  a.S = S;
  a.tw = 0;
  a.stats = reinterpret_cast<unsigned long long*>(w + L.stats);
  a.cand = reinterpret_cast<unsigned long long*>(w + L.cand);
  a.status = reinterpret_cast<unsigned*>(w + L.status);
  a.err = reinterpret_cast<unsigned*>(w + L.err);
  a.err_host = error_host_slot(a.err);
  a.spin = spin_limit();
  a.state = reinterpret_cast<float*>(w + L.state);
  a.walk = reinterpret_cast<unsigned*>(w + L.walk);
  a.ids_stride = ids_stride;
  a.out = reinterpret_cast<uint16_t*>(out);
  a.ids_in = reinterpret_cast<const int32_t*>(ids);
  a.count_in = reinterpret_cast<const int32_t*>(count);
  const dim3 grid(S, groups), block(kDT);
  hipStream_t s = (hipStream_t)stream;
  // a workgroup's list: at most kDT interleaved entries, or a contiguous
  // share of ceil((H + T) / S)
  const size_t rows_bytes = (size_t)std::max(kDT, (H + T + S - 1) / S) * sizeof(int);
  if (S <= 32) hipLaunchKernelGGL((decode_kernel<1, true>), grid, block, rows_bytes, s, a);
  else if (S <= 64) hipLaunchKernelGGL((decode_kernel<2, true>), grid, block, rows_bytes, s, a);
  else if (S <= 128) hipLaunchKernelGGL((decode_kernel<4, true>), grid, block, rows_bytes, s, a);
  else hipLaunchKernelGGL((decode_kernel<8, true>), grid, block, rows_bytes, s, a);
  return (int)hipGetLastError();
}

}  // namespace prismkv

// ---- the allocation-free decode ----------------------------------------
// Callers that cannot allocate (code under graph capture, tight serving
// loops) get the decode workspace from this file-scope array instead of a
// caller-owned buffer: 1 MiB, which holds the workspace of up to 13 groups.
// Every GPU the library runs on holds its own copy until the process ends;
// its device address is looked up once per device (hipGetSymbolAddress, with
// that device current) and only that address is handed to kernels.
constexpr size_t kScratchBytes = 1u << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// The address of this device's scratch array, or nullptr if the lookup fails.
static char* scratch_address() {
  static std::mutex mu;
  static char* address[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  if (!address[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
    address[dev] = static_cast<char*>(p);
  }
  return address[dev];
}

// Zero-fills n16 16-byte words (a kernel rather than a memset, so the call
// stays capturable into a graph).
__global__ __launch_bounds__(256) void clear_words(uint4* p, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

extern "C" {

size_t prismkv_scratch_bytes(void) { return kScratchBytes; }

int prismkv_decode_noalloc(uint64_t q, uint64_t moments, uint64_t counts, uint64_t bits, uint64_t k, uint64_t v,
                           uint64_t features, uint64_t valid, uint64_t raw, uint64_t ids, uint64_t count,
                           uint64_t out, uint64_t err, int groups, int H, int T, int capacity, int64_t row_words,
                           int64_t ks, int64_t vs, int64_t ids_stride, uint64_t stream) {
  if (groups < 1 || groups > 65535 || !err || err % 4) return kBadSize;
  // the uncapped launch touches the layout's first L.walk bytes only
  const DecodeWorkLayout L(groups, decode_splits(groups));
  if (L.walk > kScratchBytes) return kBadSize;  // the workspace of more than 13 groups does not fit
  char* work = scratch_address();
  if (!work) return (int)hipErrorInvalidSymbol;
  // every check before the clear: a rejected call enqueues nothing
  int rc = decode_check(q, moments, counts, bits, k, v, reinterpret_cast<uint64_t>(work), features, valid, raw, ids,
                        count, out, false, groups, H, T, capacity, row_words, ks, vs, ids_stride, -1);
  if (rc) return rc;
  // a call that gave up may have left published words behind: start from zero
  hipLaunchKernelGGL(clear_words, dim3((unsigned)std::min<size_t>(1024, (L.walk / 16 + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, reinterpret_cast<uint4*>(work), L.walk / 16);
  rc = (int)hipGetLastError();
  if (rc) return rc;
  return decode_launch(q, moments, counts, bits, k, v, reinterpret_cast<uint64_t>(work), features, valid, raw, ids,
                       count, out, nullptr, false, groups, H, T, row_words, ks, vs, ids_stride, stream,
                       reinterpret_cast<unsigned*>(err), -1);
}

int prismkv_set_spin_limit(int limit) {
  if (limit < 0) return kBadSize;
  return __atomic_exchange_n(&g_spin_limit, limit, __ATOMIC_RELAXED);
}

int prismkv_get_spin_limit(void) { return spin_limit(); }

uint64_t prismkv_mapped_pointer(uint64_t host) {
  void* dev = nullptr;
  if (!host || hipHostGetDevicePointer(&dev, reinterpret_cast<void*>(host), 0) != hipSuccess) return 0;
  return reinterpret_cast<uint64_t>(dev);
}

size_t prismkv_decode_work_bytes(int groups, int capacity) {
  if (groups < 1 || groups > 65535 || capacity < 1) return 0;
  return DecodeWorkLayout(groups, decode_splits(groups)).total;
}

int prismkv_decode(uint64_t q, uint64_t moments, uint64_t counts, uint64_t bits, uint64_t k, uint64_t v,
                   uint64_t work, uint64_t features, uint64_t valid, uint64_t raw, uint64_t ids, uint64_t count,
                   uint64_t out, int groups, int H, int T, int capacity, int64_t row_words, int64_t ks, int64_t vs,
                   int64_t ids_stride, size_t work_bytes, uint64_t stream) {
  return decode_impl(q, moments, counts, bits, k, v, work, features, valid, raw, ids, count, out, nullptr, false, groups,
                     H, T, capacity, row_words, ks, vs, ids_stride, work_bytes, stream);
}

int prismkv_union_attend(uint64_t q, uint64_t bits, uint64_t k, uint64_t v, uint64_t work, uint64_t features,
                         uint64_t valid, uint64_t ids, uint64_t count, uint64_t out, int groups, int H, int T,
                         int capacity, int64_t row_words, int64_t ks, int64_t vs, int64_t ids_stride,
                         size_t work_bytes, uint64_t stream) {
  return decode_impl(q, 0, 0, bits, k, v, work, features, valid, 0, ids, count, out, nullptr, true, groups, H, T,
                     capacity, row_words, ks, vs, ids_stride, work_bytes, stream);
}

int prismkv_union_attend_tail(uint64_t q, uint64_t bits, uint64_t k, uint64_t v, uint64_t work, uint64_t features,
                              uint64_t valid, uint64_t ids, uint64_t count, uint64_t out, uint64_t tail, int groups, int H,
                              int max_tail, int capacity, int64_t row_words, int64_t ks, int64_t vs, int64_t ids_stride,
                              size_t work_bytes, uint64_t stream) {
  if (!tail || tail % 4) return kBadSize;
  return decode_impl(q, 0, 0, bits, k, v, work, features, valid, 0, ids, count, out, reinterpret_cast<const int*>(tail),
                     true, groups, H, max_tail, capacity, row_words, ks, vs, ids_stride, work_bytes, stream);
}

int prismkv_route_union(uint64_t q, uint64_t moments, uint64_t counts, uint64_t bits, uint64_t work,
                        uint64_t features, uint64_t valid, uint64_t raw, uint64_t ids, uint64_t count, int groups,
                        int H, int capacity, int64_t row_words, int64_t ids_stride, size_t work_bytes,
                        uint64_t stream) {
  if (groups < 1 || groups > 65535) return kBadSize;
  if (work_bytes < DecodeWorkLayout(groups, decode_splits(groups)).total) return kBadSize;
  const int rc = decode_check(q, moments, counts, bits, 0, 0, work, features, valid, raw, ids, count, 0, false,
                              groups, H, 0, capacity, row_words, 0, 0, ids_stride, -1, true);
  if (rc) return rc;
  return decode_launch(q, moments, counts, bits, 0, 0, work, features, valid, raw, ids, count, 0, nullptr, false,
                       groups, H, 0, row_words, 0, 0, ids_stride, stream, nullptr, -1, true);
}

int prismkv_route_single(uint64_t q, uint64_t moments, uint64_t counts, uint64_t work, uint64_t features,
                         uint64_t valid, uint64_t raw, int groups, size_t work_bytes, uint64_t stream) {
  if (groups < 1 || groups > 65535) return kBadSize;
  if (!q || !moments || !counts || !work || !features || !valid || !raw) return kBadSize;
  const int S = decode_splits(groups);
  const DecodeWorkLayout L(groups, S);
  if (work_bytes < L.total) return kBadSize;  // prismkv_decode_work_bytes(groups, .)
  if (S > resident_workgroups()) return kBadSize;  // a group's workgroups must be resident together
  char* w = reinterpret_cast<char*>(work);
  DecodeArgs a{};  // no bitmap, K/V, ids or split states: phases 1-4 only
  a.q = reinterpret_cast<const uint16_t*>(q);
  a.moments = reinterpret_cast<const float*>(moments);
  a.counts = reinterpret_cast<const int*>(counts);
  a.H = 1;
  a.S = S;
  a.stats = reinterpret_cast<unsigned long long*>(w + L.stats);
  a.cand = reinterpret_cast<unsigned long long*>(w + L.cand);
  a.status = reinterpret_cast<unsigned*>(w + L.status);
  a.err = reinterpret_cast<unsigned*>(w + L.err);
  a.err_host = error_host_slot(a.err);
  a.spin = spin_limit();
  a.state = reinterpret_cast<float*>(w + L.state);
  a.features = reinterpret_cast<int64_t*>(features);
  a.valid = reinterpret_cast<float*>(valid);
  a.raw = reinterpret_cast<int*>(raw);
  const dim3 grid(S, groups), block(kDT);
  hipStream_t s = (hipStream_t)stream;
  if (S <= 32) hipLaunchKernelGGL(route_kernel<1>, grid, block, 0, s, a);
  else if (S <= 64) hipLaunchKernelGGL(route_kernel<2>, grid, block, 0, s, a);
  else if (S <= 128) hipLaunchKernelGGL(route_kernel<4>, grid, block, 0, s, a);
  else hipLaunchKernelGGL(route_kernel<8>, grid, block, 0, s, a);
  return (int)hipGetLastError();
}

int prismkv_decode_tail(uint64_t q, uint64_t moments, uint64_t counts, uint64_t bits, uint64_t k, uint64_t v,
                        uint64_t work, uint64_t features, uint64_t valid, uint64_t raw, uint64_t ids, uint64_t count,
                        uint64_t out, uint64_t tail, int groups, int H, int max_tail, int capacity, int64_t row_words,
                        int64_t ks, int64_t vs, int64_t ids_stride, size_t work_bytes, uint64_t stream) {
  if (!tail || tail % 4) return kBadSize;
  return decode_impl(q, moments, counts, bits, k, v, work, features, valid, raw, ids, count, out,
                     reinterpret_cast<const int*>(tail), false, groups, H, max_tail, capacity, row_words, ks, vs,
                     ids_stride, work_bytes, stream);
}

int prismkv_decode_capped(uint64_t q, uint64_t moments, uint64_t counts, uint64_t bits, uint64_t k, uint64_t v,
                          uint64_t work, uint64_t features, uint64_t valid, uint64_t raw, uint64_t ids, uint64_t count,
                          uint64_t out, int groups, int H, int T, int capacity, int64_t limit, int64_t row_words,
                          int64_t ks, int64_t vs, int64_t ids_stride, size_t work_bytes, uint64_t stream) {
  if (limit < 0) return kBadSize;
  return decode_impl(q, moments, counts, bits, k, v, work, features, valid, raw, ids, count, out, nullptr, false, groups,
                     H, T, capacity, row_words, ks, vs, ids_stride, work_bytes, stream, limit);
}

int prismkv_decode_capped_tail(uint64_t q, uint64_t moments, uint64_t counts, uint64_t bits, uint64_t k, uint64_t v,
                               uint64_t work, uint64_t features, uint64_t valid, uint64_t raw, uint64_t ids,
                               uint64_t count, uint64_t out, uint64_t tail, int groups, int H, int max_tail,
                               int capacity, int64_t limit, int64_t row_words, int64_t ks, int64_t vs,
                               int64_t ids_stride, size_t work_bytes, uint64_t stream) {
  if (!tail || tail % 4 || limit < 0) return kBadSize;
  return decode_impl(q, moments, counts, bits, k, v, work, features, valid, raw, ids, count, out,
                     reinterpret_cast<const int*>(tail), false, groups, H, max_tail, capacity, row_words, ks, vs,
                     ids_stride, work_bytes, stream, limit);
}

}  // extern "C"
