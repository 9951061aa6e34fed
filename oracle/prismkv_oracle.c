/*
 * prismkv_oracle.c -- CPU restatement of PrismKV's routed-decode semantics.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package links, loads or
 * calls this file: it is the checker that tests/, the smoke entry point and
 * the cpu_baseline leg of bench.py compare the HIP path against.
 *
 * Every function restates one piece of the reference algorithm and names the
 * reference file:line it follows (paths relative to the reference repository).
 * Floating-point work is carried in double precision and rounded once to the
 * output type, so the oracle gives the mathematically intended value rather
 * than one particular fp32 summation order; integer/index work is exact.
 * Where a result is an ordering of floating-point scores, the functions also
 * return the smallest relative gap between neighbouring ranks ("margin"), so a
 * test can tell a genuine disagreement from a rounding-order near-tie.
 *
 * Build: gcc -O2 -shared -fPIC -o oracle/liboracle.so oracle/prismkv_oracle.c -lm
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* helpers                                                            */
/* ------------------------------------------------------------------ */

/* Order-preserving map float -> uint32 (larger float -> larger key). */
static inline uint32_t float_key(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

static inline float key_float(uint32_t k)
{
    uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* Round-to-nearest-even fp32 -> bf16 bits (NaN kept quiet). */
uint16_t orc_f32_to_bf16(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u)
        return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/*
 * k-th largest (1-based) of n floats by exact radix selection on the
 * order-preserving key (11/11/10-bit digits).  Equivalent to
 * `flat.topk(k).values.min()` for finite inputs.
 */
static float kth_largest(const float *a, int64_t n, int64_t k)
{
    static const int shifts[3] = {21, 10, 0};
    static const int widths[3] = {11, 11, 10};
    uint32_t prefix = 0, prefix_mask = 0;
    int64_t need = k;
    int64_t *hist = (int64_t *)malloc(sizeof(int64_t) * 2048);
    for (int pass = 0; pass < 3; ++pass) {
        int nb = 1 << widths[pass];
        memset(hist, 0, sizeof(int64_t) * nb);
        for (int64_t i = 0; i < n; ++i) {
            uint32_t key = float_key(a[i]);
            if ((key & prefix_mask) == prefix)
                hist[(key >> shifts[pass]) & (uint32_t)(nb - 1)]++;
        }
        int64_t above = 0;
        int digit = nb - 1;
        for (; digit > 0; --digit) {
            if (above + hist[digit] >= need)
                break;
            above += hist[digit];
        }
        need -= above;
        prefix |= (uint32_t)digit << shifts[pass];
        prefix_mask |= (uint32_t)(nb - 1) << shifts[pass];
    }
    free(hist);
    return key_float(prefix);
}

/* ------------------------------------------------------------------ */
/* stage 4 pieces: BatchTopK, SAE encode, moments, build and append   */
/* ------------------------------------------------------------------ */

/*
 * positive_global_topk -- src/prismkv/core.py:13-26.
 * count = min(count, n); threshold = the count-th largest value.  Keep every
 * element > threshold and > 0 (ascending flat index); if threshold > 0, fill
 * the remaining budget with elements == threshold in ascending flat index.
 * Output order is "strict, then ties", as the reference concatenates them.
 * Returns the number of indices written, or -1 for a negative count.
 */
int64_t orc_positive_global_topk(const float *a, int64_t n, int64_t count, int64_t *out)
{
    if (count < 0 || n < 0)
        return -1;
    if (count > n)
        count = n;
    if (count == 0)
        return 0;
    float thr = kth_largest(a, n, count);
    int64_t len = 0;
    for (int64_t i = 0; i < n; ++i)
        if (a[i] > thr && a[i] > 0.0f)
            out[len++] = i;
    if (thr > 0.0f) {
        int64_t need = count - len;
        for (int64_t i = 0; i < n && need > 0; ++i)
            if (a[i] == thr) {
                out[len++] = i;
                --need;
            }
    }
    return len;
}

/*
 * Margin of the BatchTopK threshold: smallest relative gap between the
 * count-th largest value and its neighbours that differ from it.  When the
 * GEMM feeding the selection is computed in another summation order, the
 * memberships can only differ if rounding moves a value across this gap.
 */
double orc_topk_margin(const float *a, int64_t n, int64_t count)
{
    if (count <= 0 || count >= n)
        return INFINITY;
    float thr = kth_largest(a, n, count);
    float above = INFINITY, below = -INFINITY;
    for (int64_t i = 0; i < n; ++i) {
        if (a[i] > thr && a[i] < above)
            above = a[i];
        if (a[i] < thr && a[i] > below)
            below = a[i];
    }
    double g1 = isinf(above) ? INFINITY : ((double)above - thr);
    double g2 = isinf(below) ? INFINITY : ((double)thr - below);
    double g = g1 < g2 ? g1 : g2;
    double s = fabs((double)thr) > 1e-30 ? fabs((double)thr) : 1e-30;
    return g / s;
}

/* SharedSAE.dense -- src/prismkv/core.py:47-48: relu(x @ W^T + b). */
void orc_sae_dense(const float *x, int64_t N, int d, const float *W, const float *b, int F, float *out)
{
    for (int64_t i = 0; i < N; ++i) {
        const float *xi = x + i * d;
        for (int f = 0; f < F; ++f) {
            const float *wf = W + (int64_t)f * d;
            double acc = 0.0;
            for (int k = 0; k < d; ++k)
                acc += (double)xi[k] * (double)wf[k];
            acc += (double)b[f];
            out[i * F + f] = acc > 0.0 ? (float)acc : 0.0f;
        }
    }
}

/*
 * summarize -- src/prismkv/core.py:76-89: per-bucket population mean and
 * diagonal variance of the ORIGINAL keys (two-pass), empty bucket -> 0.
 * Lists are CSR: bucket b owns ids[offsets[b] .. offsets[b+1]).
 */
void orc_summarize(const float *keys, int d, const int64_t *offsets, const int64_t *ids, int F,
                   int64_t *counts, float *mean, float *var)
{
    double *m = (double *)malloc(sizeof(double) * d);
    for (int f = 0; f < F; ++f) {
        int64_t lo = offsets[f], hi = offsets[f + 1], n = hi - lo;
        counts[f] = n;
        for (int k = 0; k < d; ++k)
            m[k] = 0.0;
        if (n == 0) {
            for (int k = 0; k < d; ++k)
                mean[(int64_t)f * d + k] = var[(int64_t)f * d + k] = 0.0f;
            continue;
        }
        for (int64_t j = lo; j < hi; ++j)
            for (int k = 0; k < d; ++k)
                m[k] += keys[ids[j] * d + k];
        for (int k = 0; k < d; ++k) {
            m[k] /= (double)n;
            mean[(int64_t)f * d + k] = (float)m[k];
        }
        for (int k = 0; k < d; ++k) {
            double s = 0.0, mk = (double)mean[(int64_t)f * d + k];
            for (int64_t j = lo; j < hi; ++j) {
                double t = keys[ids[j] * d + k] - mk;
                s += t * t;
            }
            var[(int64_t)f * d + k] = (float)(s / (double)n);
        }
    }
    free(m);
}

/* Per-dimension mean of the keys (torch `keys.float().mean(0)`). */
void orc_mean_rows(const float *keys, int64_t N, int d, float *out)
{
    for (int k = 0; k < d; ++k) {
        double s = 0.0;
        for (int64_t i = 0; i < N; ++i)
            s += keys[i * d + k];
        out[k] = (float)(s / (double)N);
    }
}

/*
 * build_index -- src/prismkv/core.py:92-103.
 * center = mean(keys) unless given; x = (k - center) / key_scale (fp32 ops);
 * a = dense(x); flat = positive_global_topk(a, N * key_mean);
 * token = flat // F, feature = flat % F; per-feature ascending token lists.
 * Writes CSR offsets[F+1] and ids (capacity N*key_mean), the center used and
 * summarize() moments.  `act` is caller scratch of N*F floats (kept so the
 * caller can inspect the threshold margin).  Returns the membership count.
 */
int64_t orc_build_index(const float *keys, int64_t N, int d, const float *W, const float *b, int F,
                        int key_mean, float key_scale, const float *center_in, float *center_out,
                        float *act, int64_t *offsets, int64_t *ids, int64_t *counts, float *mean,
                        float *var)
{
    if (N <= 0 || !(key_scale > 0.0f))
        return -1;
    if (center_in)
        memcpy(center_out, center_in, sizeof(float) * d);
    else
        orc_mean_rows(keys, N, d, center_out);
    float *x = (float *)malloc(sizeof(float) * N * d);
    for (int64_t i = 0; i < N; ++i)
        for (int k = 0; k < d; ++k)
            x[i * d + k] = (keys[i * d + k] - center_out[k]) / key_scale;
    orc_sae_dense(x, N, d, W, b, F, act);
    free(x);
    int64_t budget = N * (int64_t)key_mean;
    int64_t *flat = (int64_t *)malloc(sizeof(int64_t) * (budget > 0 ? budget : 1));
    int64_t len = orc_positive_global_topk(act, N * (int64_t)F, budget, flat);
    /* counting sort by feature; tokens ascend within a feature because the
       flat indices are visited in ascending token order after sorting */
    int64_t *cnt = (int64_t *)calloc((size_t)F + 1, sizeof(int64_t));
    for (int64_t j = 0; j < len; ++j)
        cnt[flat[j] % F + 1]++;
    offsets[0] = 0;
    for (int f = 0; f < F; ++f)
        offsets[f + 1] = offsets[f] + cnt[f + 1];
    /* mark selection on a dense byte map so tokens come out sorted */
    unsigned char *sel = (unsigned char *)calloc((size_t)(N * F), 1);
    for (int64_t j = 0; j < len; ++j)
        sel[flat[j]] = 1;
    int64_t *fill = (int64_t *)malloc(sizeof(int64_t) * F);
    for (int f = 0; f < F; ++f)
        fill[f] = offsets[f];
    for (int64_t t = 0; t < N; ++t)
        for (int f = 0; f < F; ++f)
            if (sel[t * F + f])
                ids[fill[f]++] = t;
    free(sel);
    free(fill);
    free(cnt);
    free(flat);
    orc_summarize(keys, d, offsets, ids, F, counts, mean, var);
    return len;
}

/*
 * append_index moment merge -- src/prismkv/core.py:186-201 (lines 190-199).
 * Given the old per-bucket (count, mean, var) and the new block's (count,
 * mean, var), write the merged values (Chan et al. pairwise update):
 *   mean = (a m_a + b m_b) / max(a+b, 1)
 *   var  = (a v_a + b v_b) / max(a+b, 1) + a b / max(a+b,1)^2 (m_a - m_b)^2
 * The new block's lists are the block-local lists shifted by the old history
 * (core.py:200); callers concatenate them after the old lists.
 */
void orc_merge_moments(int F, int d, const int64_t *ca, const float *ma, const float *va,
                       const int64_t *cb, const float *mb, const float *vb, int64_t *cout,
                       float *mout, float *vout)
{
    for (int f = 0; f < F; ++f) {
        double a = (double)ca[f], b = (double)cb[f], total = a + b;
        double den = total < 1.0 ? 1.0 : total;
        cout[f] = ca[f] + cb[f];
        for (int k = 0; k < d; ++k) {
            int64_t i = (int64_t)f * d + k;
            double m = (a * ma[i] + b * mb[i]) / den;
            double dm = (double)ma[i] - (double)mb[i];
            double v = (a * va[i] + b * vb[i]) / den + (a * b) / (den * den) * dm * dm;
            mout[i] = (float)m;
            vout[i] = (float)v;
        }
    }
}

/* ------------------------------------------------------------------ */
/* stage 1: routing                                                   */
/* ------------------------------------------------------------------ */

typedef struct {
    double v;
    int64_t id;
} scored_t;

static int cmp_scored_desc(const void *x, const void *y)
{
    const scored_t *a = (const scored_t *)x, *b = (const scored_t *)y;
    if (a->v > b->v)
        return -1;
    if (a->v < b->v)
        return 1;
    return a->id < b->id ? -1 : (a->id > b->id);
}

/*
 * Ranks `live` buckets by (score desc, id asc) and writes the first topk ids.
 * margin = min relative gap (s_i - s_{i+1}) / s_i over neighbouring ranks
 * i = 0 .. min(topk, live)-1 (the last pair is rank topk-1 vs rank topk);
 * exactly equal neighbours are ties that any implementation breaks by id,
 * they are skipped and counted in *ties.
 */
static int rank_live(const double *score, const unsigned char *live, int F, int topk, int64_t *order,
                     double *margin, int *ties)
{
    scored_t *s = (scored_t *)malloc(sizeof(scored_t) * (F > 0 ? F : 1));
    int n = 0;
    for (int b = 0; b < F; ++b)
        if (live[b]) {
            s[n].v = score[b];
            s[n].id = b;
            ++n;
        }
    qsort(s, (size_t)n, sizeof(scored_t), cmp_scored_desc);
    int k = n < topk ? n : topk;
    for (int i = 0; i < k; ++i)
        order[i] = s[i].id;
    double mg = INFINITY;
    int nt = 0;
    int last = n > topk ? topk : n - 1; /* compare pairs (i, i+1), i < last */
    for (int i = 0; i < last; ++i) {
        double hi = s[i].v, lo = s[i + 1].v;
        if (hi == lo) {
            ++nt;
            continue;
        }
        double g = (hi - lo) / (fabs(hi) > 1e-300 ? fabs(hi) : 1e-300);
        if (g < mg)
            mg = g;
    }
    if (margin)
        *margin = mg;
    if (ties)
        *ties = nt;
    free(s);
    return k;
}

/*
 * bucket_scores(router="moments") -- src/prismkv/core.py:106-130.
 * logits[h,b] = [log(max(n_b,1))] + [q_h . mu_b / sqrt(d)] + [(q_h*q_h) . nu_b / (2d)]
 * (terms bitmask: 1 count, 2 mean, 4 variance); empty buckets -> -inf;
 * softmax over buckets per head; mean over heads; stable argsort descending;
 * keep live buckets; first topk.  No live bucket -> zero scores, empty order.
 * Writes score[F]; returns the number of ordered buckets.
 */
int orc_bucket_scores(const float *q, int Hq, int d, const int64_t *counts, const float *mean,
                      const float *var, int F, int terms, int topk, double *score, int64_t *order,
                      double *margin, int *ties)
{
    unsigned char *live = (unsigned char *)malloc((size_t)F + 1);
    double *lg = (double *)malloc(sizeof(double) * (size_t)F);
    int any = 0;
    for (int b = 0; b < F; ++b) {
        live[b] = counts[b] > 0;
        any |= live[b];
        score[b] = 0.0;
    }
    if (!any) {
        free(live);
        free(lg);
        if (margin)
            *margin = INFINITY;
        if (ties)
            *ties = 0;
        return 0;
    }
    double rs = 1.0 / sqrt((double)d);
    for (int h = 0; h < Hq; ++h) {
        const float *qh = q + (int64_t)h * d;
        double mx = -INFINITY;
        for (int b = 0; b < F; ++b) {
            if (!live[b]) {
                lg[b] = -INFINITY;
                continue;
            }
            double l = 0.0;
            if (terms & 1)
                l += log((double)(counts[b] > 1 ? counts[b] : 1));
            if (terms & 2) {
                double s = 0.0;
                for (int k = 0; k < d; ++k)
                    s += (double)qh[k] * mean[(int64_t)b * d + k];
                l += s * rs;
            }
            if (terms & 4) {
                double s = 0.0;
                for (int k = 0; k < d; ++k)
                    s += (double)qh[k] * qh[k] * var[(int64_t)b * d + k];
                l += s / (2.0 * d);
            }
            lg[b] = l;
            if (l > mx)
                mx = l;
        }
        double z = 0.0;
        for (int b = 0; b < F; ++b)
            if (live[b])
                z += exp(lg[b] - mx);
        for (int b = 0; b < F; ++b)
            if (live[b])
                score[b] += exp(lg[b] - mx) / z / Hq;
    }
    int k = rank_live(score, live, F, topk, order, margin, ties);
    free(live);
    free(lg);
    return k;
}

/*
 * Native route from precomputed products -- kernels/ppu_8b/route_parallel.cu:13-32
 * (`fused_parallel`): l = prod + ln where ct > 0 else -inf; per-head softmax
 * (den > 0 ? v/den : 0); aggregate = sum over heads of live buckets; Top-k by
 * (value desc, id asc); unused slots padded with id 0 / valid 0; raw = sum of
 * ct over winners.  prod is [Hq][F] for one group.
 */
int orc_norm_top(const float *prod, const float *ln, const int32_t *ct, int Hq, int F, int topk,
                 int64_t *ids, float *vals, int32_t *raw, double *margin, int *ties)
{
    unsigned char *live = (unsigned char *)malloc((size_t)F + 1);
    double *agg = (double *)calloc((size_t)F, sizeof(double));
    double *lg = (double *)malloc(sizeof(double) * (size_t)F);
    for (int b = 0; b < F; ++b)
        live[b] = ct[b] > 0;
    for (int h = 0; h < Hq; ++h) {
        double mx = -INFINITY, den = 0.0;
        for (int b = 0; b < F; ++b) {
            lg[b] = live[b] ? (double)prod[(int64_t)h * F + b] + ln[b] : -INFINITY;
            if (lg[b] > mx)
                mx = lg[b];
        }
        if (isinf(mx))
            continue;
        for (int b = 0; b < F; ++b)
            den += live[b] ? exp(lg[b] - mx) : 0.0;
        for (int b = 0; b < F; ++b)
            if (live[b] && den > 0)
                agg[b] += exp(lg[b] - mx) / den;
    }
    int64_t *order = (int64_t *)malloc(sizeof(int64_t) * (size_t)topk);
    int k = rank_live(agg, live, F, topk, order, margin, ties);
    int32_t total = 0;
    for (int i = 0; i < topk; ++i) {
        ids[i] = i < k ? order[i] : 0;
        vals[i] = i < k ? 1.0f : 0.0f;
        if (i < k)
            total += ct[order[i]];
    }
    *raw = total;
    free(order);
    free(live);
    free(agg);
    free(lg);
    return k;
}

/*
 * bucket_scores(router="q_activation") -- src/prismkv/core.py:131-139.
 * a = relu((q / query_scale) W^T + b) per query row (x in fp32, the dot
 * product accumulated in double and rounded to fp32, as orc_sae_dense);
 * per row the `topk` largest activations (value descending, index ascending:
 * the stable descending argsort); weights val / max(sum val, 1e-20) / Hq in
 * fp32 with the sum taken in rank order (torch's own 16-element summation
 * order is not fixed by the reference); score[f] = the weights of f added
 * in the flattened [Hq][topk] order, from 0, in fp32; order = buckets with
 * score > 0 and counts > 0, score descending, index ascending.  Writes
 * score[F]; returns the order length.  *margin = the smallest relative gap
 * that decides the result: between a row's topk-th and next activation
 * (when positive) and between consecutive ordered scores.
 */
int orc_qact_scores(const float *q, int Hq, int d, const float *W, const float *b, int F, float query_scale,
                    const int64_t *counts, int topk, float *score, int64_t *order, double *margin)
{
    float *x = (float *)malloc(sizeof(float) * Hq * d);
    float *a = (float *)malloc(sizeof(float) * Hq * F);
    scored_t *s = (scored_t *)malloc(sizeof(scored_t) * (F > 0 ? F : 1));
    for (int i = 0; i < Hq * d; ++i)
        x[i] = q[i] / query_scale;
    orc_sae_dense(x, Hq, d, W, b, F, a);
    double gap = INFINITY;
    for (int f = 0; f < F; ++f)
        score[f] = 0.0f;
    int k = topk < F ? topk : F;
    for (int h = 0; h < Hq; ++h) {
        for (int f = 0; f < F; ++f) {
            s[f].v = a[(int64_t)h * F + f];
            s[f].id = f;
        }
        qsort(s, F, sizeof(scored_t), cmp_scored_desc);
        if (k < F && s[k - 1].v > 0.0) {
            double g = (s[k - 1].v - s[k].v) / fabs(s[k - 1].v);
            if (g < gap)
                gap = g;
        }
        float sum = 0.0f;
        for (int r = 0; r < k; ++r)
            sum += (float)s[r].v;
        if (sum < 1e-20f)
            sum = 1e-20f;
        for (int r = 0; r < k; ++r) {
            float c = ((float)s[r].v / sum) / (float)Hq;
            score[s[r].id] += c;
        }
    }
    int n = 0;
    for (int f = 0; f < F; ++f)
        if (score[f] > 0.0f && counts[f] > 0) {
            s[n].v = score[f];
            s[n].id = f;
            ++n;
        }
    qsort(s, n, sizeof(scored_t), cmp_scored_desc);
    for (int i = 0; i < n; ++i) {
        order[i] = s[i].id;
        if (i + 1 < n) {
            double g = (s[i].v - s[i + 1].v) / fabs(s[i].v);
            if (g < gap)
                gap = g;
        }
    }
    *margin = gap;
    free(x);
    free(a);
    free(s);
    return n;
}

/* pack -- kernels/ppu_8b/pack.cu:3: a[r] = [q_r, q_r * q_r] in fp32. */
void orc_pack(const uint16_t *q, int rows, int d, float *a)
{
    for (int r = 0; r < rows; ++r)
        for (int k = 0; k < d; ++k) {
            uint32_t u = (uint32_t)q[r * d + k] << 16;
            float v;
            memcpy(&v, &u, 4);
            a[(int64_t)r * 2 * d + k] = v;
            a[(int64_t)r * 2 * d + d + k] = v * v;
        }
}

/* ------------------------------------------------------------------ */
/* stage 2: bucket selection / union                                  */
/* ------------------------------------------------------------------ */

/*
 * select_buckets -- src/prismkv/core.py:142-167.
 * Walk `order`; with no cap (unique_cap < 0) accept every bucket; with a cap,
 * limit = floor(H * cap) and SKIP (continue past) any bucket whose count of
 * not-yet-chosen ids would overflow the limit.  Output: ascending unique ids,
 * accepted features in rank order, raw = sum of accepted list lengths.
 * Returns the unique count, or -1 for a cap outside [0, 1].
 */
int64_t orc_select_buckets(const int64_t *order, int n_order, const int64_t *offsets, const int64_t *ids,
                           int64_t H, double unique_cap, int64_t *out_ids, int64_t *features,
                           int *n_features, int64_t *raw, int64_t *limit_out)
{
    if (unique_cap >= 0.0 && unique_cap > 1.0)
        return -1;
    int64_t limit = unique_cap < 0.0 ? H : (int64_t)floor((double)H * unique_cap);
    unsigned char *chosen = (unsigned char *)calloc((size_t)(H > 0 ? H : 1), 1);
    int64_t count = 0, rawc = 0;
    int nf = 0;
    for (int i = 0; i < n_order; ++i) {
        int64_t b = order[i], lo = offsets[b], hi = offsets[b + 1], fresh = 0;
        for (int64_t j = lo; j < hi; ++j)
            fresh += !chosen[ids[j]];
        if (count + fresh > limit)
            continue;
        for (int64_t j = lo; j < hi; ++j)
            chosen[ids[j]] = 1;
        count += fresh;
        rawc += hi - lo;
        features[nf++] = b;
    }
    int64_t n = 0;
    for (int64_t t = 0; t < H; ++t)
        if (chosen[t])
            out_ids[n++] = t;
    free(chosen);
    *n_features = nf;
    *raw = rawc;
    *limit_out = limit;
    return n;
}

/*
 * build_bits -- kernels/ppu_8b/pack.cu:5: bits[f][t >> 5] |= 1 << (t & 31)
 * for every member t of bucket f; rows are row_words uint32 apart.
 */
void orc_build_bits(const int64_t *offsets, const int64_t *ids, int F, int64_t row_words, uint32_t *bits)
{
    for (int f = 0; f < F; ++f)
        for (int64_t j = offsets[f]; j < offsets[f + 1]; ++j) {
            int64_t t = ids[j];
            bits[(int64_t)f * row_words + (t >> 5)] |= 1u << (t & 31);
        }
}

/*
 * Bitmap union -- kernels/ppu_8b/union.cu:14-27: OR the rows of the selected
 * buckets whose valid flag is > 0, then emit w*32+bit in ascending order for
 * tokens below H.  Returns the unique count.
 */
int64_t orc_union_bits(const uint32_t *bits, int64_t row_words, int64_t H, const int64_t *features,
                       const float *valid, int k, int32_t *out_ids)
{
    int64_t nw = (H + 31) / 32, n = 0;
    for (int64_t w = 0; w < nw; ++w) {
        uint32_t m = 0;
        for (int j = 0; j < k; ++j)
            if (valid[j] > 0.0f)
                m |= bits[features[j] * row_words + w];
        for (int bit = 0; bit < 32; ++bit)
            if (((m >> bit) & 1u) && w * 32 + bit < H)
                out_ids[n++] = (int32_t)(w * 32 + bit);
    }
    return n;
}

/* ------------------------------------------------------------------ */
/* stage 3: attention                                                 */
/* ------------------------------------------------------------------ */

/*
 * attend -- src/prismkv/core.py:170-183: exact softmax(q K^T / sqrt(d)) V over
 * the selected old rows plus every tail row [H, L).  old_ids must be unique
 * and in [0, H) (returns -1 otherwise, the reference raises ValueError); no
 * row at all -> zeros.  q is [Hq][d]; K, V are [L][d] rows with row stride
 * `stride` floats.  Output in double, [Hq][d].
 */
int orc_attend(const float *q, int Hq, int d, const float *K, const float *V, int64_t stride, int64_t L,
               const int64_t *old_ids, int64_t n_old, int64_t H, double *out)
{
    if (H < 0 || H > L)
        return -1;
    if (n_old > 0) {
        unsigned char *seen = (unsigned char *)calloc((size_t)(H > 0 ? H : 1), 1);
        for (int64_t j = 0; j < n_old; ++j) {
            int64_t t = old_ids[j];
            if (t < 0 || t >= H || seen[t]) {
                free(seen);
                return -1;
            }
            seen[t] = 1;
        }
        free(seen);
    }
    int64_t rows = n_old + (L - H);
    for (int i = 0; i < Hq * d; ++i)
        out[i] = 0.0;
    if (rows == 0)
        return 0;
    double *s = (double *)malloc(sizeof(double) * (size_t)rows);
    double rs = 1.0 / sqrt((double)d);
    for (int h = 0; h < Hq; ++h) {
        const float *qh = q + (int64_t)h * d;
        double mx = -INFINITY;
        for (int64_t r = 0; r < rows; ++r) {
            int64_t pos = r < n_old ? old_ids[r] : H + (r - n_old);
            double acc = 0.0;
            for (int k = 0; k < d; ++k)
                acc += (double)qh[k] * K[pos * stride + k];
            s[r] = acc * rs;
            if (s[r] > mx)
                mx = s[r];
        }
        double z = 0.0;
        for (int64_t r = 0; r < rows; ++r) {
            s[r] = exp(s[r] - mx);
            z += s[r];
        }
        double *oh = out + (int64_t)h * d;
        for (int64_t r = 0; r < rows; ++r) {
            int64_t pos = r < n_old ? old_ids[r] : H + (r - n_old);
            double p = s[r] / z;
            for (int k = 0; k < d; ++k)
                oh[k] += p * V[pos * stride + k];
        }
    }
    free(s);
    return 0;
}
