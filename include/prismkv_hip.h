/*
 * prismkv_hip.h -- C ABI of libprismkv_hip.so, the MI355X (gfx950) kernels of
 * PrismKV's routed decode path.
 *
 * Conventions (kept from the reference binding, src/prismkv/native8b.py:46-51):
 *   - every device pointer is passed as uint64_t (torch `tensor.data_ptr()`),
 *     then int / int64 sizes, then a trailing uint64_t hipStream_t;
 *   - return 0 on success, -1 for an invalid size/range, -2 for an invalid
 *     mode (kernels/ppu_8b/union.cu:40,47, av_tuned.cu:63,65), otherwise the
 *     hipError_t of the launch;
 *   - arguments are validated on the host before anything is enqueued; the
 *     library allocates nothing, never synchronises and only enqueues work on
 *     the given stream.  `work` buffers are caller-owned scratch, sized by the
 *     matching *_work_bytes() call, zero-filled once before first use; the
 *     kernels leave their counters at zero again, so launches can be replayed
 *     from a captured graph.  Calls sharing a work buffer must not overlap.
 *     Every entry point that takes `work` also takes its size, `work_bytes`
 *     (the last argument before the stream), and returns -1 without enqueuing
 *     anything when it is below what the matching *_work_bytes() query returns
 *     for the call's own sizes: an undersized or stale workspace is refused
 *     instead of being written past its end.  (No reference counterpart: the
 *     reference's kernels take no workspace.)
 *
 * Geometry is the native 8B specialisation: F = 3000 buckets, d = 128,
 * 4 query heads per KV group, Top-16 buckets (src/prismkv/native8b.py:1-6).
 *
 * Device layouts (per layer; G = groups):
 *   q        bf16 [G][4][128]
 *   moments  f32  [G][94][256][32]  bucket tiles: k < 128 mean, k >= 128 var;
 *                                   bucket b -> tile b/32, column b%32 (3008 padded)
 *   counts   i32  [G][3008]         bucket sizes, padding buckets 0
 *   bits     u32  [G][3000][row_words]  token t of bucket f: word t>>5, bit t&31
 *   features i64  [G][16], valid f32 [G][16], raw i32 [G]
 *   ids      i32  [G][ids_stride] (first count[g] valid, ascending), count i32 [G]
 *   K, V     bf16 rows of 128, group stride ks / vs elements; rows [H, H+T) are the tail
 *   out      bf16 [G][4][128]
 */
#ifndef PRISMKV_HIP_H
#define PRISMKV_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- reference-compatible entry points (same names and signatures) ---- */

/* kernels/ppu_8b/pack.cu:4 -- bf16 q[32][128] -> f32 a[32][256] = [q, q*q]. */
int pack(uint64_t q, uint64_t a, uint64_t stream);

/* kernels/ppu_8b/pack.cu:6 -- CSR lists (ids i32 [8][C], offsets i32 [8][3001])
 * -> bits u32 [8][3000][ceil(H/32)] (bits must be zeroed by the caller). */
int build_bits(uint64_t ids, uint64_t offsets, uint64_t bits, int H, int C, uint64_t stream);

/* kernels/ppu_8b/route_parallel.cu:33 -- prod f32 [8][4][3000], ln f32 [8][3000],
 * ct i32 [8][3000] -> ids i64 [8][16], vals f32 [8][16], raw i32 [8]. */
int fused_norm_top(uint64_t prod, uint64_t ln, uint64_t ct, uint64_t ids, uint64_t vals, uint64_t raw,
                   uint64_t stream);

/* kernels/ppu_8b/union.cu:39 -- bits u32 [U][3000][NW], mask u32 [U][NW] and
 * tiles i32 [U][ceil(NW/128)] scratch -> selected i32 [U][H], counts i32 [U].
 * U in [1,8], H in [1,131072], mode in {0,1,2} (all give identical output). */
int launch_union_warp(uint64_t bits, uint64_t ids, uint64_t vals, uint64_t mask, uint64_t tiles,
                      uint64_t selected, uint64_t counts, int U, int H, int mode, uint64_t stream);

/* kernels/ppu_8b/av_tuned.cu:62 -- 8 groups; state f32 [32][S][130] scratch;
 * S in [1,128]; KS, VS >= (H+T)*128; mode in {0,1,2} (identical output). */
int attention_tuned(uint64_t q, uint64_t k, uint64_t v, uint64_t ids, uint64_t cnt, uint64_t state,
                    uint64_t out, int H, int T, int KS, int VS, int S, int mode, uint64_t stream);

/* ---- MI355X-native entry points ---- */

/* Stage 1 (replaces pack + torch.bmm + fused_norm_top, src/prismkv/native8b.py:85-87;
 * semantics src/prismkv/core.py:106-130): moment scoring, per-part Top-16
 * candidates and the final Top-16, three launches for G groups. */
size_t prismkv_route_work_bytes(int groups);
int prismkv_route(uint64_t q, uint64_t moments, uint64_t counts, uint64_t work, uint64_t features,
                  uint64_t valid, uint64_t raw, int groups, size_t work_bytes, uint64_t stream);
/* Stage 1 in ONE launch (the same replacement and semantics as prismkv_route,
 * identical features / valid / raw): the selection phases of prismkv_decode
 * alone.  `work` is prismkv_decode's workspace (prismkv_decode_work_bytes,
 * zero-filled once; the launch leaves it zero) and its first 32-bit word the
 * same error word; -1 when one group's workgroups cannot be resident at once,
 * as for prismkv_decode. */
int prismkv_route_single(uint64_t q, uint64_t moments, uint64_t counts, uint64_t work, uint64_t features,
                         uint64_t valid, uint64_t raw, int groups, size_t work_bytes, uint64_t stream);
/* Stages 1-2 in ONE launch (replaces Native8B.route = pack + torch.bmm +
 * fused_norm_top + launch_union_warp, src/prismkv/native8b.py:82-89;
 * semantics src/prismkv/core.py:106-130, :142-148 with cap None): the
 * selection, union and id phases of prismkv_decode without the attention.
 * Writes the same features / valid / raw / ids / count as prismkv_decode;
 * no K/V is read and no output written.  The limits, workspace and -1 are
 * prismkv_decode's. */
int prismkv_route_union(uint64_t q, uint64_t moments, uint64_t counts, uint64_t bits, uint64_t work,
                        uint64_t features, uint64_t valid, uint64_t raw, uint64_t ids, uint64_t count, int groups,
                        int H, int capacity, int64_t row_words, int64_t ids_stride, size_t work_bytes,
                        uint64_t stream);

/* Stage 2 (replaces launch_union_warp, src/prismkv/native8b.py:88-89;
 * semantics kernels/ppu_8b/union.cu:14-27): one launch, any H up to 2^29. */
size_t prismkv_union_work_bytes(int groups, int H);
int prismkv_union(uint64_t bits, uint64_t features, uint64_t valid, uint64_t work, uint64_t ids,
                  uint64_t count, int groups, int H, int64_t row_words, int64_t ids_stride, size_t work_bytes,
                  uint64_t stream);

/* Stage 2, strict unique-ID budget (src/prismkv/core.py:149-163, select_buckets
 * with unique_cap): walks the ranked buckets (rows with valid > 0, in rank
 * order) and keeps a bucket only if the union of the kept buckets stays within
 * `limit` = floor(H * unique_cap) tokens, skipping one that would overflow;
 * rewrites features / valid / raw with the kept buckets compacted to the front
 * in rank order (then run prismkv_union).  H <= 2^20; counts i32 [G][3008]. */
int prismkv_select_cap(uint64_t bits, uint64_t counts, uint64_t features, uint64_t valid, uint64_t raw, int groups,
                       int H, int64_t limit, int64_t row_words, uint64_t stream);

/* Bitmap build from CSR (replaces build_bits, src/prismkv/native8b.py:66-70):
 * ids i32 [G][cap], offsets i32 [G][3001]; bits must be zeroed by the caller. */
int prismkv_build_bits(uint64_t ids, uint64_t offsets, uint64_t bits, int groups, int64_t cap,
                       int64_t row_words, uint64_t stream);

/* Stage 3 (replaces attention_tuned, src/prismkv/native8b.py:91-102;
 * semantics src/prismkv/core.py:170-183): when H + T <= 16384 x S (S =
 * min(256, max(32, 256 / groups)) workgroups per group, all resident), the
 * fused decode's attention phases over each group's count + T rows (every
 * S-th 16-row chunk per workgroup; contiguous shares past 512 S rows); otherwise split-K with the merge fused into
 * the last workgroup of each group.  splits in [1,1024] (the partition does
 * not change the result).  `work` (prismkv_attend_work_bytes) is zero-filled
 * once before first use and left zeroed; its first 32-bit word is the error
 * word (1 if a bounded inter-workgroup wait gave up; 2 if an id outside
 * [0, H) or a count outside [0, H] was found, which is then read clamped into
 * range), with the optional host-word slot at byte 8.  The ids of a group
 * must be distinct (the reference's attend rejects duplicates on the host,
 * src/prismkv/core.py:176-179). */
size_t prismkv_attend_work_bytes(int groups, int splits);
int prismkv_attend(uint64_t q, uint64_t k, uint64_t v, uint64_t ids, uint64_t count, uint64_t work,
                   uint64_t out, int groups, int H, int T, int64_t ks, int64_t vs, int64_t ids_stride,
                   int splits, size_t work_bytes, uint64_t stream);

/* Stages 1-3 fused (replaces Native8B.__call__ = route + attention,
 * src/prismkv/native8b.py:104-106): ONE launch per layer for moment scoring,
 * selection, union and sparse attention; writes the same features / valid /
 * raw / ids / count as prismkv_route + prismkv_union and the same out as
 * prismkv_attend.  H <= 524288, (H + T) * 256 < 2^31 (the K/V rows are
 * read through 32-bit byte offsets).  `work` is sized for the largest history the
 * caller will use (`capacity` >= H) by prismkv_decode_work_bytes and is
 * zero-filled once before first use; its first 32-bit word is the error word
 * (nonzero if a bounded inter-workgroup wait gave up; see the bounded-wait
 * section below).  The workgroups of one
 * group wait on each other: it returns -1 if one group's
 * min(256, max(32, 256 / groups)) workgroups cannot be resident on the device
 * at once. */
size_t prismkv_decode_work_bytes(int groups, int capacity);
int prismkv_decode(uint64_t q, uint64_t moments, uint64_t counts, uint64_t bits, uint64_t k, uint64_t v,
                   uint64_t work, uint64_t features, uint64_t valid, uint64_t raw, uint64_t ids, uint64_t count,
                   uint64_t out, int groups, int H, int T, int capacity, int64_t row_words, int64_t ks, int64_t vs,
                   int64_t ids_stride, size_t work_bytes, uint64_t stream);
/* prismkv_decode with the tail length read from device memory at launch
 * (`tail`: one int32, 4-byte aligned), clamped to [0, max_tail]; the K/V
 * extents are checked for max_tail.  For a decode step captured once in a
 * HIP graph and replayed as the tail grows (the caller advances the word on
 * the stream between or inside replays): the reference binding has no
 * counterpart (its Native8B.__call__, src/prismkv/native8b.py:104-106,
 * takes the length from K's shape on the host). */
int prismkv_decode_tail(uint64_t q, uint64_t moments, uint64_t counts, uint64_t bits, uint64_t k, uint64_t v,
                        uint64_t work, uint64_t features, uint64_t valid, uint64_t raw, uint64_t ids, uint64_t count,
                        uint64_t out, uint64_t tail, int groups, int H, int max_tail, int capacity, int64_t row_words,
                        int64_t ks, int64_t vs, int64_t ids_stride, size_t work_bytes, uint64_t stream);
/* Stages 2-3 fused from a given selection (replaces launch_union_warp +
 * attention_tuned, src/prismkv/native8b.py:88-89 and :100-101): ONE launch
 * for the union and the sparse attention of prismkv_decode, over the
 * selection in features / valid read as prismkv_union reads it (the valid
 * entries with in-range bucket ids, in order; up to 16 per group), e.g. as
 * prismkv_select_cap left it.  Writes the same ids / count as prismkv_union
 * and the same out as prismkv_attend; features / valid / raw are not
 * touched.  `work` is prismkv_decode's workspace; the limits and the -1 for
 * a group that cannot be resident are prismkv_decode's. */
int prismkv_union_attend(uint64_t q, uint64_t bits, uint64_t k, uint64_t v, uint64_t work, uint64_t features,
                         uint64_t valid, uint64_t ids, uint64_t count, uint64_t out, int groups, int H, int T,
                         int capacity, int64_t row_words, int64_t ks, int64_t vs, int64_t ids_stride,
                         size_t work_bytes, uint64_t stream);
/* prismkv_union_attend with the tail length read from device memory at
 * launch (`tail`: one int32, 4-byte aligned), clamped to [0, max_tail], as
 * prismkv_decode_tail: the capped step (route, budgeted walk, union +
 * attention) of a decode captured once in a HIP graph and replayed as the
 * tail grows.  No reference counterpart (the reference takes the tail length
 * from K's shape on the host). */
int prismkv_union_attend_tail(uint64_t q, uint64_t bits, uint64_t k, uint64_t v, uint64_t work, uint64_t features,
                              uint64_t valid, uint64_t ids, uint64_t count, uint64_t out, uint64_t tail, int groups, int H,
                              int max_tail, int capacity, int64_t row_words, int64_t ks, int64_t vs, int64_t ids_stride,
                              size_t work_bytes, uint64_t stream);
/* The capped step in ONE launch (replaces the strict unique cap branch of
 * select_buckets, src/prismkv/core.py:149-163, between route and union,
 * src/prismkv/native8b.py:104-106 with a cap): prismkv_decode with the
 * budgeted walk between the selection and the union.  The group's Top-16 in
 * rank order is walked with limit `limit` (>= 0; floor(H * unique_cap) in
 * the reference): a bucket is kept when the union of the kept buckets,
 * itself included, stays within the limit.  Writes features / valid / raw
 * for the kept buckets (compacted in rank order, as prismkv_select_cap
 * leaves them), their union's ids / count and the attention over it, the
 * same results as prismkv_route_single + prismkv_select_cap +
 * prismkv_union_attend.  The limits, workspace and -1 are prismkv_decode's. */
int prismkv_decode_capped(uint64_t q, uint64_t moments, uint64_t counts, uint64_t bits, uint64_t k, uint64_t v,
                          uint64_t work, uint64_t features, uint64_t valid, uint64_t raw, uint64_t ids, uint64_t count,
                          uint64_t out, int groups, int H, int T, int capacity, int64_t limit, int64_t row_words,
                          int64_t ks, int64_t vs, int64_t ids_stride, size_t work_bytes, uint64_t stream);
/* prismkv_decode_capped with the tail length read from device memory at
 * launch, as prismkv_decode_tail (no reference counterpart: a captured capped
 * step replayed as the tail grows). */
int prismkv_decode_capped_tail(uint64_t q, uint64_t moments, uint64_t counts, uint64_t bits, uint64_t k, uint64_t v,
                               uint64_t work, uint64_t features, uint64_t valid, uint64_t raw, uint64_t ids,
                               uint64_t count, uint64_t out, uint64_t tail, int groups, int H, int max_tail,
                               int capacity, int64_t limit, int64_t row_words, int64_t ks, int64_t vs,
                               int64_t ids_stride, size_t work_bytes, uint64_t stream);

/* The allocation-free decode.  No counterpart in the reference: for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  Same launch and outputs as
 * prismkv_decode, but the workspace is the library's own file-scope device
 * array of prismkv_scratch_bytes() = 1 MiB (one copy per GPU, held until the
 * process ends), which holds the workspace of up to 13 groups; -1 for more
 * groups or a null / misaligned `err`.  `err` (one int32, device or
 * host-mapped memory) receives 1 if a bounded wait gave up; it is not
 * cleared by the call.  Each call first clears the array with a small kernel
 * (no memset node, so the call can be captured), then decodes; it calls no
 * hipMalloc, hipFree or allocating library routine.  Calls on one GPU share
 * the array: calls that overlap on one GPU (other streams) race. */
size_t prismkv_scratch_bytes(void);
int prismkv_decode_noalloc(uint64_t q, uint64_t moments, uint64_t counts, uint64_t bits, uint64_t k, uint64_t v,
                           uint64_t features, uint64_t valid, uint64_t raw, uint64_t ids, uint64_t count,
                           uint64_t out, uint64_t err, int groups, int H, int T, int capacity, int64_t row_words,
                           int64_t ks, int64_t vs, int64_t ids_stride, uint64_t stream);

/* ---- bounded waits and their error words (no reference counterpart: the
 * reference kernels never wait across workgroups) --------------------------
 * Every inter-workgroup wait of prismkv_decode, prismkv_decode_tail,
 * prismkv_decode_capped(_tail), prismkv_union_attend, prismkv_route_single
 * and prismkv_union gives up after
 * a process-wide number of sleeps (64 clocks each; default 2^20, tens of
 * milliseconds), writes 1 to its workspace's first 32-bit word (the sticky
 * error word, cleared only by the caller) and lets the launch run to its end
 * with every access in range; the results of such a launch are invalid and
 * the workspace must be zero-filled again before the next launch.  If the
 * workspace's 8-byte slot at byte offset 8 holds a nonzero device address (of
 * a host-mapped 32-bit word, see prismkv_mapped_pointer), the wait also writes
 * 1 there, so a host binding can notice it without synchronising.
 * prismkv_set_spin_limit sets the bound for launches enqueued afterwards and
 * returns the previous one (-1 for a negative limit). */
int prismkv_set_spin_limit(int limit);
int prismkv_get_spin_limit(void);
/* The device address of a host pointer from hipHostMalloc (e.g. a pinned
 * torch tensor), 0 if it is not device-accessible. */
uint64_t prismkv_mapped_pointer(uint64_t host);

/* ---- stage 4: incremental index update ---------------------------------
 * append_index (src/prismkv/core.py:186-201) for all groups at once, on the
 * device tables in place.  The new block is K rows [H, H+N) of each group
 * (bf16, group stride `ks` elements, rows of 128).  Per group:
 *   x = (k - center[g]) / scale[g] (fp32), a = relu(x W[g]^T + b[g])
 *     (SharedSAE.dense, core.py:47-48), W f32 [G][3000][128], b f32 [G][3000],
 *     center f32 [G][128] (the index's ORIGINAL center), scale f32 [G];
 *   BatchTopK over the block (positive_global_topk, core.py:13-26) with the
 *     budget N * key_mean: values above the budget-th largest tau, then ties
 *     at tau in ascending flat index (token * 3000 + bucket) up to the budget,
 *     or every positive value when fewer are positive;
 *   bits: member (token t, bucket f) sets bit H + t of row f (columns
 *     [H, H+N) must be zero on entry; rows of `row_words` >= (H+N+31)/32);
 *   counts i32 [G][3008] += new members; moments (the tiled [G][94][256][32]
 *     table) <- Chan merge of the old moments with the block's population
 *     moments, in fp32 and the operation order of core.py:190-199.
 * `work` is prismkv_update_work_bytes(groups, N) bytes, zero-filled once
 * before first use and left zeroed; a workspace sized for the largest block
 * serves every smaller one.  N <= 4096; K rows, W and b 16-byte aligned;
 * returns -1 on bad sizes.  The block's dense activations [G][N][3000] f32
 * stay in the workspace from byte prismkv_update_act_offset(groups) on until
 * the next call (the same offset, for `batch` groups, in prismkv_build's).
 * The caller guarantees K holds rows [0, H+N) for every group. */
size_t prismkv_update_work_bytes(int groups, int max_block);
size_t prismkv_update_act_offset(int groups);
int prismkv_update(uint64_t k, uint64_t W, uint64_t b, uint64_t center, uint64_t scale, uint64_t bits,
                   uint64_t counts, uint64_t moments, uint64_t work, int groups, int H, int N, int key_mean,
                   int64_t ks, int64_t row_words, size_t work_bytes, uint64_t stream);

/* ---- prefill index build -----------------------------------------------
 * build_index (src/prismkv/core.py:92-103) of every group from K rows
 * [0, H) (replaces the host build before Native8B(indices), i.e.
 * src/prismkv/hf_reference.py:196-198 followed by src/prismkv/native8b.py:35-74).
 * Per group: center[g] = mean of the rows (computed when flags & 1, else an
 * input); x = (k - center[g]) / scale[g]; a = relu(x W[g]^T + b[g]); BatchTopK
 * over all H keys with the budget H * key_mean (the same rule as
 * prismkv_update); the bitmap rows are cleared and member (t, f) sets bit t
 * of row f; counts[g][f] = members and the tiled moments get each bucket's
 * population mean and variance of the ORIGINAL keys (core.py:76-89), written
 * directly.  Groups are processed `batch` at a time; `work` is
 * prismkv_build_work_bytes(batch, H) bytes (H x 3000 fp32 activations per
 * group of a batch), zero-filled once before first use and left zeroed.
 * H <= 2^20, row_words a multiple of 4 and >= (H+31)/32, bits, W, b and K
 * rows 16-byte aligned; -1 on bad sizes, -2 on unknown flags. */
size_t prismkv_build_work_bytes(int batch, int H);
int prismkv_build(uint64_t k, uint64_t W, uint64_t b, uint64_t center, uint64_t scale, uint64_t bits,
                  uint64_t counts, uint64_t moments, uint64_t work, int groups, int batch, int H, int key_mean,
                  int flags, int64_t ks, int64_t row_words, size_t work_bytes, uint64_t stream);

/* ---- the prismkv.core surface (src/prismkv/core.py) ---------------------
 * Stage 1 with the score vector of bucket_scores (core.py:106-130): as
 * prismkv_route, and scores f32 [G][3000] <- the per-head softmax
 * probabilities' mean over the 4 heads (0 for a dead bucket). */
int prismkv_route_scores(uint64_t q, uint64_t moments, uint64_t counts, uint64_t work, uint64_t features,
                         uint64_t valid, uint64_t raw, uint64_t scores, int groups, size_t work_bytes,
                         uint64_t stream);

/* Stage 1 by query activations (router "q_activation", core.py:131-139):
 * a = relu((q / qscale[g]) W[g]^T + b[g]) for the 4 heads (W f32 [G][3000][128],
 * b f32 [G][3000], qscale f32 [G]); per head the 16 largest activations
 * (value descending, bucket ascending), weights val / max(sum, 1e-20) / 4;
 * score = the weights of a bucket summed in head order; the selection is the
 * buckets of positive score and nonzero size by score descending, bucket
 * ascending: features i64 [G][64], valid f32 [G][64], raw i32 [G]; scores
 * f32 [G][3000] (optional, 0 to skip).  Then prismkv_union_n / _select_cap_n
 * with width 64. */
size_t prismkv_route_qact_work_bytes(int groups);
int prismkv_route_qact(uint64_t q, uint64_t W, uint64_t b, uint64_t qscale, uint64_t counts, uint64_t work,
                       uint64_t features, uint64_t valid, uint64_t raw, uint64_t scores, int groups, size_t work_bytes,
                       uint64_t stream);

/* prismkv_union / prismkv_select_cap over selections of `width` rows per
 * group (features / valid [G][width]), width 16 or 64. */
int prismkv_union_n(uint64_t bits, uint64_t features, uint64_t valid, uint64_t work, uint64_t ids, uint64_t count,
                    int groups, int H, int64_t row_words, int64_t ids_stride, int width, size_t work_bytes,
                    uint64_t stream);
int prismkv_select_cap_n(uint64_t bits, uint64_t counts, uint64_t features, uint64_t valid, uint64_t raw, int groups,
                         int H, int64_t limit, int64_t row_words, int width, uint64_t stream);

/* positive_global_topk (core.py:13-26) of a device matrix act f32 [N][3000]
 * (16-byte aligned, N <= 2^20) with budget `count`: out i64 [min(count,
 * 3000 N)] <- every value above the budget-th largest tau (and above 0) in
 * ascending flat index (row * 3000 + column), then the values equal to
 * tau > 0 in ascending flat index up to the budget (every positive value when
 * fewer are positive); out_len i32 [1] <- how many were written.  `work` is
 * prismkv_topk_work_bytes() bytes, zero-filled once and left zeroed. */
size_t prismkv_topk_work_bytes(void);
int prismkv_topk(uint64_t act, uint64_t out, uint64_t out_len, uint64_t work, int N, int64_t count,
                 size_t work_bytes, uint64_t stream);

/* summarize (core.py:76-89) of every group from its bitmap rows: counts and
 * the tiled moments get each bucket's member count and the population mean
 * and variance of the member K rows (bit t of row f: row t of K, t < H);
 * center[g] <- mean of K rows [0, H) when flags & 1.  `work` is
 * prismkv_summarize_work_bytes(groups) bytes, zero-filled once. */
size_t prismkv_summarize_work_bytes(int groups);
int prismkv_summarize(uint64_t k, uint64_t bits, uint64_t center, uint64_t counts, uint64_t moments, uint64_t work,
                      int groups, int H, int flags, int64_t ks, int64_t row_words, size_t work_bytes,
                      uint64_t stream);

/* ---- fp32 inputs ---------------------------------------------------------
 * The reference's core functions take tensors of any float dtype and compute
 * in fp32 (src/prismkv/core.py:92-103,106-139,170-183; examples/replay.py:15-21
 * runs them on fp32 keys, queries and values).  These entry points are the
 * ones above with fp32 in place of bf16: the same arguments, work sizes,
 * error words and results, except that
 *   prismkv_build_f32 / prismkv_update_f32 / prismkv_summarize_f32: K rows are
 *     fp32 (ks in elements; rows 16-byte aligned);
 *   prismkv_route_scores_f32 / prismkv_route_qact_f32: q is fp32 [G][4][128];
 *   prismkv_attend_f32: q, K and V rows are fp32 and out is fp32 [G][4][128]
 *     (always the split-K kernel; q, K, V and the row strides 16-byte
 *     aligned).
 * Every key, query and value is used at full fp32 precision. */
int prismkv_build_f32(uint64_t k, uint64_t W, uint64_t b, uint64_t center, uint64_t scale, uint64_t bits,
                      uint64_t counts, uint64_t moments, uint64_t work, int groups, int batch, int H, int key_mean,
                      int flags, int64_t ks, int64_t row_words, size_t work_bytes, uint64_t stream);
int prismkv_update_f32(uint64_t k, uint64_t W, uint64_t b, uint64_t center, uint64_t scale, uint64_t bits,
                       uint64_t counts, uint64_t moments, uint64_t work, int groups, int H, int N, int key_mean,
                       int64_t ks, int64_t row_words, size_t work_bytes, uint64_t stream);
int prismkv_summarize_f32(uint64_t k, uint64_t bits, uint64_t center, uint64_t counts, uint64_t moments,
                          uint64_t work, int groups, int H, int flags, int64_t ks, int64_t row_words,
                          size_t work_bytes, uint64_t stream);
int prismkv_route_scores_f32(uint64_t q, uint64_t moments, uint64_t counts, uint64_t work, uint64_t features,
                             uint64_t valid, uint64_t raw, uint64_t scores, int groups, size_t work_bytes,
                             uint64_t stream);
int prismkv_route_qact_f32(uint64_t q, uint64_t W, uint64_t b, uint64_t qscale, uint64_t counts, uint64_t work,
                           uint64_t features, uint64_t valid, uint64_t raw, uint64_t scores, int groups,
                           size_t work_bytes, uint64_t stream);
int prismkv_attend_f32(uint64_t q, uint64_t k, uint64_t v, uint64_t ids, uint64_t count, uint64_t work,
                       uint64_t out, int groups, int H, int T, int64_t ks, int64_t vs, int64_t ids_stride,
                       int splits, size_t work_bytes, uint64_t stream);

#ifdef __cplusplus
}
#endif

#endif /* PRISMKV_HIP_H */
