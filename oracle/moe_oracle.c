/*
 * moe_oracle.c -- CPU restatement of hy-nomas-rs `MoeLayer::forward` and of the
 * deterministic generator its tests and random weights use.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker, never the product: only
 * the tests, the smoke check and the CPU-baseline leg of the benchmark load it.
 * The product library never links or calls it.
 *
 * Reference files restated (paths relative to the reference repository):
 *   nomas-core/src/tensor_utils.rs:65-106   SplitMix64 + Box-Muller
 *   nomas-core/src/tensor_utils.rs:123-155  deterministic_randn_affine / uniform
 *   nomas-core/src/tensor_utils.rs:159-162  xavier
 *   nomas-core/src/modules/mod.rs:47-55     Weights::path_seed (FNV-1a)
 *   nomas-core/src/modules/mod.rs:122-142   Lin::fwd  (x @ W^T + b, rows folded)
 *   nomas-core/src/modules/moe.rs:65-109    MoeLayer::forward
 *   nomas-core/src/modules/mlp.rs:39-48     FeedForward::SwiGlu (orc_ffn_f64, and each expert)
 *   nomas-core/src/modules/norm.rs:55-65     RmsNorm::forward     (orc_norm_modulate)
 *   nomas-core/src/modules/modulate.rs:69-79 modulate             (orc_norm_modulate)
 *   nomas-core/src/modules/block.rs:96,101   the FFN seams of DiTBlock::forward
 *                                            (orc_norm_modulate, orc_gated_residual)
 *
 * Two evaluation modes:
 *   - sparse f64  (orc_forward_sparse_f64): routing from f64 logits, only the
 *     selected experts, f64 accumulation.  Used for parity at any size because
 *     rows are independent, so any subset of rows can be checked exactly.
 *   - faithful dense f32 (orc_forward_dense_f32): the reference algorithm as
 *     written -- f32 routing composed as max/sub/exp/sum/div, iterative argmax,
 *     every expert on every row, combine in ascending expert order.  This is
 *     also the timed CPU baseline.
 *
 * Weight layout everywhere is the reference's (out, in), experts concatenated:
 *   router wr (E, D); gate wg (E, H, D), bg (E, H); up wu (E, H, D), bu (E, H);
 *   down wd (E, D, H), bd (E, D).  The optional shared dense branch uses the
 *   same layout with E = 1 (moe.rs:44-54,103-106).
 *
 * `orc_mutation` plants one known mistake so the pin tests can prove they
 * would catch it (0 = faithful).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int orc_mutation = 0;

enum {
    MUT_NONE = 0,
    MUT_BOXMULLER_SWAP = 1,   /* sin/cos order of the Box-Muller pair swapped   */
    MUT_TIE_HIGH_INDEX = 2,   /* argmax ties resolved to the highest index      */
    MUT_NO_RENORM = 3,        /* weights = raw softmax probs (no renormalise)   */
    MUT_SWAP_GATE_UP = 4,     /* silu applied to the up projection              */
    MUT_DROP_DOWN_BIAS = 5,   /* down-projection bias ignored                   */
    MUT_DOWN_TRANSPOSED = 6,  /* down weight indexed (in, out) instead of (out, in) */
    MUT_FNV_PRIME = 7,        /* FNV-1a with a wrong multiplier                 */
    MUT_SPLITMIX_SHIFT = 8,   /* SplitMix64 first xor-shift 31 instead of 30    */
    MUT_MODULATE_NO_ONE = 9,  /* modulate multiplies by scale, not 1 + scale    */
    MUT_VAR_D_MINUS_1 = 10,   /* RMSNorm mean over D - 1 elements               */
    MUT_NORM_NO_ROUND = 11,   /* norm output not rounded to the model dtype     */
    MUT_UNGATED_RESIDUAL = 12, /* residual adds y without the gate              */
    MUT_H_UNROUNDED = 13,     /* rounded mode: SwiGLU intermediate kept in f64  */
    MUT_COMBINE_UNFUSED = 14, /* rounded mode: combine as f32 mul, then add     */
    /* a simulated GPU-path fault (tests/test_parity_bars.py), not an oracle
     * mistake: the gate/up GEMM skips x[32..39] for hidden units 0..15, one
     * 16-byte operand fragment of one k step of one 16-row MFMA block */
    MUT_GATE_UP_LOSES_FRAGMENT = 15
};

/* ------------------------------------------------------------------ */
/* Generator: tensor_utils.rs:65-106, mod.rs:47-55                     */
/* ------------------------------------------------------------------ */

/* SplitMix64::next_u64 (tensor_utils.rs:76-83). */
uint64_t orc_splitmix64_next(uint64_t *state)
{
    *state += 0x9E3779B97F4A7C15ull;
    uint64_t z = *state;
    z = (z ^ (z >> (orc_mutation == MUT_SPLITMIX_SHIFT ? 31 : 30))) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* SplitMix64::next_f64 (tensor_utils.rs:86-89): 53 high bits scaled to [0, 1). */
static double next_f64(uint64_t *state)
{
    return (double)(orc_splitmix64_next(state) >> 11) * (1.0 / 9007199254740992.0);
}

/* Weights::path_seed (mod.rs:47-55): FNV-1a over the path bytes, offset basis
 * xor'ed with the base seed. */
uint64_t orc_path_seed(uint64_t seed, const char *path)
{
    uint64_t h = 0xcbf29ce484222325ull ^ seed;
    const uint64_t prime = orc_mutation == MUT_FNV_PRIME ? 0x100000001b5ull : 0x100000001b3ull;
    for (const unsigned char *p = (const unsigned char *)path; *p; ++p) {
        h ^= (uint64_t)*p;
        h *= prime;
    }
    return h;
}

/* deterministic_randn_affine (tensor_utils.rs:123-138) with next_normal
 * (tensor_utils.rs:93-106): each pair of draws (u1, u2) yields r*cos(theta)
 * first and caches r*sin(theta) for the next element. */
void orc_randn_affine(uint64_t seed, double mean, double std, int64_t n, float *out)
{
    uint64_t st = seed;
    for (int64_t i = 0; i < n; i += 2) {
        double u1 = next_f64(&st);
        if (u1 < 2.2250738585072014e-308) /* f64::MIN_POSITIVE */
            u1 = 2.2250738585072014e-308;
        double u2 = next_f64(&st);
        double r = sqrt(-2.0 * log(u1));
        double theta = 2.0 * 3.14159265358979323846 * u2;
        double a = r * cos(theta), b = r * sin(theta);
        if (orc_mutation == MUT_BOXMULLER_SWAP) { double t = a; a = b; b = t; }
        out[i] = (float)(a * std + mean);
        if (i + 1 < n)
            out[i + 1] = (float)(b * std + mean);
    }
}

/* deterministic_uniform (tensor_utils.rs:141-155). */
void orc_uniform(uint64_t seed, double lo, double hi, int64_t n, float *out)
{
    uint64_t st = seed;
    for (int64_t i = 0; i < n; ++i)
        out[i] = (float)(lo + next_f64(&st) * (hi - lo));
}

/* xavier (tensor_utils.rs:159-162): N(0, sqrt(2/(out+in))) of shape (out, in). */
void orc_xavier(int64_t out_f, int64_t in_f, uint64_t seed, float *w)
{
    orc_randn_affine(seed, 0.0, sqrt(2.0 / (double)(out_f + in_f)), out_f * in_f, w);
}

/* f32 -> bf16 round-to-nearest-even, returned widened back to f32
 * (candle's to_dtype(BF16) goes through half::bf16::from_f32, which is RNE). */
void orc_round_bf16(float *a, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) {
        uint32_t u;
        memcpy(&u, &a[i], 4);
        if ((u & 0x7fffffffu) > 0x7f800000u) {
            u = (u | 0x00400000u) & 0xffff0000u;
        } else {
            u += 0x7fffu + ((u >> 16) & 1u);
            u &= 0xffff0000u;
        }
        memcpy(&a[i], &u, 4);
    }
}

/* ------------------------------------------------------------------ */
/* Routing: moe.rs:67-95                                               */
/* ------------------------------------------------------------------ */

/* Route one row in f64.  logits_e = sum_d x_d * wr[e][d] (ascending d),
 * probs = softmax composed max/sub/exp/sum/div, top-k by k passes of argmax
 * over the remaining probs (first maximum wins), weights = top / (sum + 1e-9).
 * Writes the k selected experts in ascending index order with their weights,
 * the E logits, and the logit gap between the k-th selected and the best
 * unselected expert (+inf when k == E). */
static void route_row_f64(int64_t D, int64_t E, int64_t k, const float *x, const float *wr,
                          int32_t *idx, double *w, double *logits, double *gap, double *scratch)
{
    double *p = scratch;            /* E */
    double *rem = scratch + E;      /* E */
    double *top = scratch + 2 * E;  /* E */
    for (int64_t e = 0; e < E; ++e) {
        double s = 0.0;
        const float *we = wr + e * D;
        for (int64_t d = 0; d < D; ++d)
            s += (double)x[d] * (double)we[d];
        logits[e] = s;
    }
    double m = logits[0];
    for (int64_t e = 1; e < E; ++e)
        if (logits[e] > m) m = logits[e];
    double sum = 0.0;
    for (int64_t e = 0; e < E; ++e) {
        p[e] = exp(logits[e] - m);
        sum += p[e];
    }
    for (int64_t e = 0; e < E; ++e) {
        p[e] /= sum;
        rem[e] = p[e];
        top[e] = 0.0;
    }
    for (int64_t it = 0; it < k; ++it) {
        int64_t best = 0;
        for (int64_t e = 1; e < E; ++e) {
            if (orc_mutation == MUT_TIE_HIGH_INDEX ? rem[e] >= rem[best] : rem[e] > rem[best])
                best = e;
        }
        top[best] += rem[best];
        rem[best] = 0.0;
    }
    /* A selected expert is one whose remaining prob was zeroed; with no
     * underflowed probabilities every selected entry of `top` is > 0. */
    double norm = 0.0;
    for (int64_t e = 0; e < E; ++e)
        norm += top[e];
    double kth = INFINITY, best_un = -INFINITY;
    int64_t j = 0;
    for (int64_t e = 0; e < E; ++e) {
        if (top[e] > 0.0) {
            if (j < k) {
                idx[j] = (int32_t)e;
                w[j] = orc_mutation == MUT_NO_RENORM ? top[e] : top[e] / (norm + 1e-9);
            }
            ++j;
            if (logits[e] < kth) kth = logits[e];
        } else if (logits[e] > best_un) {
            best_un = logits[e];
        }
    }
    for (; j < k; ++j) { idx[j] = -1; w[j] = 0.0; }
    *gap = (k == E) ? INFINITY : kth - best_un;
}

/* Route T rows (x: T x D, wr: E x D).  Any output pointer may be NULL. */
void orc_route_f64(int64_t T, int64_t D, int64_t E, int64_t k, const float *x, const float *wr,
                   int32_t *idx, double *w, double *logits, double *gap)
{
#pragma omp parallel
    {
        double *scr = (double *)malloc(sizeof(double) * (size_t)(4 * E + 2 * k + 1));
        int32_t *li = (int32_t *)malloc(sizeof(int32_t) * (size_t)k);
#pragma omp for schedule(static)
        for (int64_t t = 0; t < T; ++t) {
            double *lg = scr + 3 * E, *lw = scr + 4 * E, g;
            route_row_f64(D, E, k, x + t * D, wr, li, lw, lg, &g, scr);
            if (idx) memcpy(idx + t * k, li, sizeof(int32_t) * (size_t)k);
            if (w) memcpy(w + t * k, lw, sizeof(double) * (size_t)k);
            if (logits) memcpy(logits + t * E, lg, sizeof(double) * (size_t)E);
            if (gap) gap[t] = g;
        }
        free(scr);
        free(li);
    }
}

/* ------------------------------------------------------------------ */
/* Sparse f64 forward of selected rows                                 */
/* ------------------------------------------------------------------ */

static double silu(double g) { return g / (1.0 + exp(-g)); }

static float round_dt(float v, int dt);

/* The kernels' storage of an intermediate in the model dtype: the f64 value
 * rounded to f32 (their accumulators), then to the model dtype; rdt < 0
 * keeps the f64 value. */
static double stored(double v, int rdt)
{
    return rdt < 0 ? v : (double)round_dt((float)v, rdt);
}

/* One SwiGLU FFN (mlp.rs:42-46) on one row, f64: y = down(silu(gate x) * up x).
 * rdt >= 0 stores the SwiGLU intermediate a and the output y in the model
 * dtype rdt, as the GPU path's buffers hold them (see stored()). */
static void swiglu_row_f64(int64_t D, int64_t H, const float *x, const float *wg, const float *bg,
                           const float *wu, const float *bu, const float *wd, const float *bd,
                           double *a, double *y, int rdt)
{
    for (int64_t h = 0; h < H; ++h) {
        double g = bg ? (double)bg[h] : 0.0, u = bu ? (double)bu[h] : 0.0;
        const float *gr = wg + h * D, *ur = wu + h * D;
        for (int64_t d = 0; d < D; ++d) {
            if (orc_mutation == MUT_GATE_UP_LOSES_FRAGMENT && h < 16 && d >= 32 && d < 40) continue;
            g += (double)x[d] * (double)gr[d];
            u += (double)x[d] * (double)ur[d];
        }
        if (orc_mutation == MUT_SWAP_GATE_UP) { double t = g; g = u; u = t; }
        a[h] = orc_mutation == MUT_H_UNROUNDED ? silu(g) * u : stored(silu(g) * u, rdt);
    }
    for (int64_t d = 0; d < D; ++d) {
        double s = (bd && orc_mutation != MUT_DROP_DOWN_BIAS) ? (double)bd[d] : 0.0;
        if (orc_mutation == MUT_DOWN_TRANSPOSED) {
            /* reads wd as if it were laid out (in, out) = (H, D) */
            for (int64_t h = 0; h < H; ++h)
                s += a[h] * (double)wd[h * D + d];
        } else {
            const float *dr = wd + d * H;
            for (int64_t h = 0; h < H; ++h)
                s += a[h] * (double)dr[h];
        }
        y[d] = stored(s, rdt);
    }
}

/* FeedForward::SwiGlu::forward (mlp.rs:39-48) on the listed rows (NULL:
 * 0..nrows-1), f64: the dense FFN of the blocks without MoE. */
void orc_ffn_f64(int64_t D, int64_t H, const float *x, const float *wg, const float *bg,
                 const float *wu, const float *bu, const float *wd, const float *bd,
                 const int64_t *rows, int64_t nrows, double *out)
{
#pragma omp parallel
    {
        double *a = (double *)malloc(sizeof(double) * (size_t)H);
#pragma omp for schedule(dynamic, 1)
        for (int64_t r = 0; r < nrows; ++r) {
            int64_t t = rows ? rows[r] : r;
            swiglu_row_f64(D, H, x + t * D, wg, bg, wu, bu, wd, bd, a, out + r * D, -1);
        }
        free(a);
    }
}

/* out[r] = MoeLayer::forward(x)[rows[r]] for the listed rows, in f64.
 * `rows` may be NULL to mean rows 0..nrows-1.  The shared dense branch
 * (dense_* pointers, coefficient s) is added after the experts when s > 0,
 * additively as moe.rs:103-106 does.  Also writes each row's routing when
 * idx/w/gap are non-NULL (k entries per row, ascending expert index). */
static void forward_sparse(int64_t D, int64_t E, int64_t k, int64_t H,
                           const float *x, const float *wr,
                           const float *wg, const float *bg, const float *wu, const float *bu,
                           const float *wd, const float *bd,
                           double s, const float *dwg, const float *dbg, const float *dwu,
                           const float *dbu, const float *dwd, const float *dbd,
                           const int64_t *rows, int64_t nrows, double *out,
                           int32_t *idx_out, double *w_out, double *gap_out, int rdt)
{
#pragma omp parallel
    {
        double *scr = (double *)malloc(sizeof(double) * (size_t)(4 * E + 2 * k + H + D + 1));
        int32_t *li = (int32_t *)malloc(sizeof(int32_t) * (size_t)k);
#pragma omp for schedule(dynamic, 1)
        for (int64_t r = 0; r < nrows; ++r) {
            int64_t t = rows ? rows[r] : r;
            const float *xr = x + t * D;
            double *lg = scr + 3 * E, *lw = scr + 4 * E, *a = lw + k, *y = a + H, g;
            route_row_f64(D, E, k, xr, wr, li, lw, lg, &g, scr);
            double *o = out + r * D;
            for (int64_t d = 0; d < D; ++d) o[d] = 0.0;
            /* rdt >= 0: the GPU combine -- per element, an f32 fused
             * multiply-add of the stored y by the f32 gate, slot by slot in
             * ascending expert order (then the dense slot), the sum rounded
             * once to the model dtype */
            for (int64_t j = 0; j < k; ++j) {
                int64_t e = li[j];
                if (e < 0) continue;
                swiglu_row_f64(D, H, xr, wg + e * H * D, bg ? bg + e * H : NULL,
                               wu + e * H * D, bu ? bu + e * H : NULL,
                               wd + e * D * H, bd ? bd + e * D : NULL, a, y, rdt);
                if (rdt < 0)
                    for (int64_t d = 0; d < D; ++d) o[d] += lw[j] * y[d];
                else if (orc_mutation == MUT_COMBINE_UNFUSED)
                    for (int64_t d = 0; d < D; ++d) {
                        const float m = (float)y[d] * (float)lw[j];
                        o[d] = (double)((float)o[d] + m);
                    }
                else
                    for (int64_t d = 0; d < D; ++d)
                        o[d] = (double)fmaf((float)y[d], (float)lw[j], (float)o[d]);
            }
            if (s > 0.0 && dwg) {
                swiglu_row_f64(D, H, xr, dwg, dbg, dwu, dbu, dwd, dbd, a, y, rdt);
                if (rdt < 0)
                    for (int64_t d = 0; d < D; ++d) o[d] += s * y[d];
                else
                    for (int64_t d = 0; d < D; ++d)
                        o[d] = (double)fmaf((float)y[d], (float)s, (float)o[d]);
            }
            if (rdt >= 0)
                for (int64_t d = 0; d < D; ++d) o[d] = (double)round_dt((float)o[d], rdt);
            if (idx_out) memcpy(idx_out + r * k, li, sizeof(int32_t) * (size_t)k);
            if (w_out) memcpy(w_out + r * k, lw, sizeof(double) * (size_t)k);
            if (gap_out) gap_out[r] = g;
        }
        free(scr);
        free(li);
    }
}

void orc_forward_sparse_f64(int64_t D, int64_t E, int64_t k, int64_t H,
                            const float *x, const float *wr,
                            const float *wg, const float *bg, const float *wu, const float *bu,
                            const float *wd, const float *bd,
                            double s, const float *dwg, const float *dbg, const float *dwu,
                            const float *dbu, const float *dwd, const float *dbd,
                            const int64_t *rows, int64_t nrows, double *out,
                            int32_t *idx_out, double *w_out, double *gap_out)
{
    forward_sparse(D, E, k, H, x, wr, wg, bg, wu, bu, wd, bd, s, dwg, dbg, dwu, dbu, dwd, dbd,
                   rows, nrows, out, idx_out, w_out, gap_out, -1);
}

/* The same forward with the GPU path's storage roundings: the SwiGLU
 * intermediate and each expert's output held in the model dtype dt (0 f32,
 * 1 bf16, 2 f16), the combine an f32 fused multiply-add per slot, the output
 * rounded to dt.  Not the reference's arithmetic (candle rounds after every
 * op): it isolates the kernels' own error from the storage roundings, so a
 * tight bar against it catches mistakes (a lost k step, a stale partial)
 * that the loose bar against the f64 forward would let through. */
void orc_forward_sparse_rounded(int64_t D, int64_t E, int64_t k, int64_t H,
                                const float *x, const float *wr,
                                const float *wg, const float *bg, const float *wu, const float *bu,
                                const float *wd, const float *bd,
                                double s, const float *dwg, const float *dbg, const float *dwu,
                                const float *dbu, const float *dwd, const float *dbd,
                                const int64_t *rows, int64_t nrows, double *out, int dt)
{
    forward_sparse(D, E, k, H, x, wr, wg, bg, wu, bu, wd, bd, s, dwg, dbg, dwu, dbu, dwd, dbd,
                   rows, nrows, out, NULL, NULL, NULL, dt < 0 ? 0 : dt);
}

/* Routing of a model in dtype dt (0 f32, 1 bf16, 2 f16) as the reference
 * evaluates it, op by op in the tensor dtype (moe.rs:67-95): PARITY UNPINNED.
 * candle cannot be built or imported here, so its per-op semantics are
 * restated from its documented behaviour and not checked against it:
 *   logits = x . wr^T accumulated in f32, rounded to dt (candle's CPU matmul
 *            of half types accumulates in f32);
 *   softmax composed (candle_nn::ops::softmax): m = max; diff = dt(l - m);
 *            num = dt(exp(diff)); den = the num summed one add at a time in
 *            dt, ascending expert; p = dt(num / den);
 *   top-k:   k passes of argmax over the remaining p (first maximum wins),
 *            each pass zeroing the chosen entry (moe.rs:77-91);
 *   gates:   norm = the chosen p summed in dt; w = dt(p / dt(norm + dt(1e-9)))
 *            (moe.rs:92-95).
 * Used to measure how often a model-dtype router would choose another expert
 * set than the f64 routing the GPU path follows.  idx (T x k, ascending), w
 * (T x k) may be NULL. */
void orc_route_model_dtype(int64_t T, int64_t D, int64_t E, int64_t k, const float *x,
                           const float *wr, int dt, int32_t *idx, float *w)
{
#pragma omp parallel
    {
        float *p = (float *)malloc(sizeof(float) * (size_t)(3 * E));
        float *rem = p + E, *top = p + 2 * E;
#pragma omp for schedule(static)
        for (int64_t t = 0; t < T; ++t) {
            const float *xr = x + t * D;
            for (int64_t e = 0; e < E; ++e) {
                float s = 0.0f;
                const float *we = wr + e * D;
                for (int64_t d = 0; d < D; ++d) s += xr[d] * we[d];
                p[e] = round_dt(s, dt);
            }
            float m = p[0];
            for (int64_t e = 1; e < E; ++e) if (p[e] > m) m = p[e];
            float den = 0.0f;
            for (int64_t e = 0; e < E; ++e) {
                p[e] = round_dt(expf(round_dt(p[e] - m, dt)), dt);
                den = round_dt(den + p[e], dt);
            }
            for (int64_t e = 0; e < E; ++e) {
                rem[e] = round_dt(p[e] / den, dt);
                top[e] = 0.0f;
            }
            for (int64_t it = 0; it < k; ++it) {
                int64_t best = 0;
                for (int64_t e = 1; e < E; ++e) if (rem[e] > rem[best]) best = e;
                top[best] = rem[best];
                rem[best] = 0.0f;
            }
            float norm = 0.0f;
            for (int64_t e = 0; e < E; ++e) norm = round_dt(norm + top[e], dt);
            const float dnorm = round_dt(norm + round_dt(1e-9f, dt), dt);
            int64_t j = 0;
            for (int64_t e = 0; e < E && j < k; ++e) {
                /* chosen entries: zeroed in rem; a chosen p of 0 (underflow) is
                 * listed too, by the order of the passes */
                if (rem[e] == 0.0f && (top[e] > 0.0f || p[e] == 0.0f)) {
                    if (idx) idx[t * k + j] = (int32_t)e;
                    if (w) w[t * k + j] = round_dt(top[e] / dnorm, dt);
                    ++j;
                }
            }
            for (; j < k; ++j) {
                if (idx) idx[t * k + j] = -1;
                if (w) w[t * k + j] = 0.0f;
            }
        }
        free(p);
    }
}

/* ------------------------------------------------------------------ */
/* Faithful dense f32 forward (the reference algorithm; CPU baseline)   */
/* ------------------------------------------------------------------ */

typedef float v16f __attribute__((vector_size(64)));

/* C (M x N, row-major, ldc) = A (M x K) . B (N x K)^T, both K-contiguous, as
 * Lin::fwd's x.matmul(W^T) (mod.rs:135).  Cache-blocked with a 4x4 register
 * tile of 16-wide dot-product accumulators; OpenMP over row/column blocks. */
static void sgemm_nt(int64_t M, int64_t N, int64_t K, const float *A, const float *B, float *C,
                     int64_t ldc)
{
    const int64_t MB = 64, NB = 64;
    int64_t mblocks = (M + MB - 1) / MB, nblocks = (N + NB - 1) / NB;
    int64_t K16 = K & ~(int64_t)15;
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
    for (int64_t mb = 0; mb < mblocks; ++mb) {
        for (int64_t nb = 0; nb < nblocks; ++nb) {
            int64_t m1 = mb * MB + MB < M ? mb * MB + MB : M;
            int64_t n1 = nb * NB + NB < N ? nb * NB + NB : N;
            for (int64_t m = mb * MB; m < m1; m += 4) {
                for (int64_t n = nb * NB; n < n1; n += 4) {
                    int64_t mr = m1 - m < 4 ? m1 - m : 4, nr = n1 - n < 4 ? n1 - n : 4;
                    v16f acc[4][4];
                    memset(acc, 0, sizeof(acc));
                    const float *ap[4], *bp[4];
                    for (int i = 0; i < 4; ++i) ap[i] = A + (m + (i < mr ? i : 0)) * K;
                    for (int j = 0; j < 4; ++j) bp[j] = B + (n + (j < nr ? j : 0)) * K;
                    for (int64_t kk = 0; kk < K16; kk += 16) {
                        v16f av[4], bv[4];
                        for (int i = 0; i < 4; ++i) memcpy(&av[i], ap[i] + kk, 64);
                        for (int j = 0; j < 4; ++j) memcpy(&bv[j], bp[j] + kk, 64);
                        for (int i = 0; i < 4; ++i)
                            for (int j = 0; j < 4; ++j)
                                acc[i][j] += av[i] * bv[j];
                    }
                    for (int i = 0; i < mr; ++i) {
                        for (int j = 0; j < nr; ++j) {
                            float s = 0.0f;
                            for (int l = 0; l < 16; ++l) s += acc[i][j][l];
                            for (int64_t kk = K16; kk < K; ++kk) s += ap[i][kk] * bp[j][kk];
                            C[(m + i) * ldc + n + j] = s;
                        }
                    }
                }
            }
        }
    }
}

/* SwiGLU on all T rows in f32 (mlp.rs:42-46 via Lin::fwd, mod.rs:122-142):
 * each op rounded to f32 as candle does. G and U are T x H scratch. */
static void swiglu_dense_f32(int64_t T, int64_t D, int64_t H, const float *x, const float *wg,
                             const float *bg, const float *wu, const float *bu, const float *wd,
                             const float *bd, float *G, float *U, float *Y)
{
    sgemm_nt(T, H, D, x, wg, G, H);
    sgemm_nt(T, H, D, x, wu, U, H);
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < T; ++t) {
        for (int64_t h = 0; h < H; ++h) {
            float g = G[t * H + h] + (bg ? bg[h] : 0.0f);
            float u = U[t * H + h] + (bu ? bu[h] : 0.0f);
            float sg = g / (1.0f + expf(-g));
            G[t * H + h] = sg * u;
        }
    }
    sgemm_nt(T, D, H, G, wd, Y, D);
    if (bd) {
#pragma omp parallel for schedule(static)
        for (int64_t t = 0; t < T; ++t)
            for (int64_t d = 0; d < D; ++d) Y[t * D + d] += bd[d];
    }
}

/* The reference MoeLayer::forward (moe.rs:65-109) in f32, every expert on
 * every row.  Routing: f32 logits, softmax max/sub/exp/sum/div, k passes of
 * argmax (first max wins) with the selected entry zeroed, weights
 * top / (sum_E top + 1e-9).  Combine: out = out + y_e * w_e in ascending e,
 * then out + s * dense(x).  Writes the dense (T x E) weights when w_dense is
 * non-NULL.  Scratch is allocated internally (3 * T * max(H, D) floats). */
int orc_forward_dense_f32(int64_t T, int64_t D, int64_t E, int64_t k, int64_t H,
                          const float *x, const float *wr,
                          const float *wg, const float *bg, const float *wu, const float *bu,
                          const float *wd, const float *bd,
                          double s, const float *dwg, const float *dbg, const float *dwu,
                          const float *dbu, const float *dwd, const float *dbd,
                          float *out, float *w_dense)
{
    int64_t HD = H > D ? H : D;
    float *logits = (float *)malloc(sizeof(float) * (size_t)(T * E));
    float *wts = (float *)malloc(sizeof(float) * (size_t)(T * E));
    float *G = (float *)malloc(sizeof(float) * (size_t)(T * HD));
    float *U = (float *)malloc(sizeof(float) * (size_t)(T * HD));
    float *Y = (float *)malloc(sizeof(float) * (size_t)(T * D));
    if (!logits || !wts || !G || !U || !Y) {
        free(logits); free(wts); free(G); free(U); free(Y);
        return -1;
    }
    sgemm_nt(T, E, D, x, wr, logits, E);
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < T; ++t) {
        float *l = logits + t * E, *w = wts + t * E;
        float m = l[0];
        for (int64_t e = 1; e < E; ++e) if (l[e] > m) m = l[e];
        float sum = 0.0f;
        for (int64_t e = 0; e < E; ++e) { w[e] = expf(l[e] - m); sum += w[e]; }
        for (int64_t e = 0; e < E; ++e) w[e] = w[e] / sum;  /* w holds probs = remaining */
        float top[1024];
        float *tp = E <= 1024 ? top : (float *)malloc(sizeof(float) * (size_t)E);
        for (int64_t e = 0; e < E; ++e) tp[e] = 0.0f;
        for (int64_t it = 0; it < k; ++it) {
            int64_t best = 0;
            for (int64_t e = 1; e < E; ++e)
                if (orc_mutation == MUT_TIE_HIGH_INDEX ? w[e] >= w[best] : w[e] > w[best]) best = e;
            float sel = w[best];
            tp[best] = tp[best] + sel;
            w[best] = w[best] - sel;
        }
        float norm = 0.0f;
        for (int64_t e = 0; e < E; ++e) norm += tp[e];
        for (int64_t e = 0; e < E; ++e)
            w[e] = orc_mutation == MUT_NO_RENORM ? tp[e] : tp[e] / (norm + 1e-9f);
        if (tp != top) free(tp);
    }
    if (w_dense) memcpy(w_dense, wts, sizeof(float) * (size_t)(T * E));
    memset(out, 0, sizeof(float) * (size_t)(T * D));
    for (int64_t ei = 0; ei < E; ++ei) {
        int64_t e = ei;
        swiglu_dense_f32(T, D, H, x, wg + e * H * D, bg ? bg + e * H : NULL, wu + e * H * D,
                         bu ? bu + e * H : NULL, wd + e * D * H, bd ? bd + e * D : NULL, G, U, Y);
#pragma omp parallel for schedule(static)
        for (int64_t t = 0; t < T; ++t) {
            float we = wts[t * E + e];
            for (int64_t d = 0; d < D; ++d) {
                float prod = Y[t * D + d] * we;
                out[t * D + d] = out[t * D + d] + prod;
            }
        }
    }
    if (s > 0.0 && dwg) {
        swiglu_dense_f32(T, D, H, x, dwg, dbg, dwu, dbu, dwd, dbd, G, U, Y);
        float sf = (float)s;
#pragma omp parallel for schedule(static)
        for (int64_t t = 0; t < T; ++t)
            for (int64_t d = 0; d < D; ++d) out[t * D + d] = out[t * D + d] + Y[t * D + d] * sf;
    }
    free(logits); free(wts); free(G); free(U); free(Y);
    return 0;
}

/* ------------------------------------------------------------------ */
/* Block seams: block.rs:96,101, norm.rs:55-65, modulate.rs:69-79      */
/* ------------------------------------------------------------------ */

/* f32 -> f16 round-to-nearest-even, widened back (candle's to_dtype(F16) goes
 * through half::f16::from_f32).  Written from the definition: the result is a
 * multiple of the f16 quantum at the value's binade (2^(e-10), and 2^-24 below
 * the normal range), chosen by rint (ties to even in the default rounding
 * mode); magnitudes that round past 65504 become infinity; NaN stays NaN. */
static float round_f16_1(float v)
{
    if (isnan(v) || isinf(v) || v == 0.0f) return v;
    int ex;
    (void)frexpf(v, &ex);            /* |v| = m * 2^ex, m in [0.5, 1) */
    int q = ex - 11;                  /* quantum 2^q of an 11-bit significand */
    if (q < -24) q = -24;             /* subnormal f16: fixed quantum 2^-24 */
    float r = ldexpf(rintf(ldexpf(v, -q)), q);
    if (fabsf(r) > 65504.0f) r = copysignf(INFINITY, v);
    return r;
}

void orc_round_f16(float *a, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) a[i] = round_f16_1(a[i]);
}

/* dt: 0 f32 (no rounding), 1 bf16, 2 f16 (DataType, config.rs:30-39) */
static float round_dt(float v, int dt)
{
    if (dt == 1) {
        orc_round_bf16(&v, 1);
        return v;
    }
    if (dt == 2) return round_f16_1(v);
    return v;
}

/* h = modulate(norm2(x), shift, scale) for rows x D activations already in the
 * model dtype (widened to f32); row r in sequence r / seq, shift and scale
 * (rows / seq, D), norm_w (D) or NULL (RmsNorm::no_affine).  Each step is one
 * candle-core 0.11.1 f32 op rounded to f32, in the reference's order:
 *   norm.rs:58-65   sq = x.powf(2); ss = sum (one add at a time, ascending d);
 *                   var = ss * f32(1/D) (mean_keepdim = sum * (1/D));
 *                   t = var + f32(eps); inv = t.powf(-0.5);
 *                   n = x * inv; n = n * w; n -> model dtype
 *   modulate.rs:76-78  m = n * (scale + 1) + shift in f32; m -> model dtype
 * pow_mode 0 calls libm powf as the reference's f32::powf does; pow_mode 1
 * uses the correctly rounded forms (x*x, and 1/sqrt in double rounded once),
 * which powf matches except where its result lands within its error bound of
 * a rounding midpoint.  inv_out (rows) may be NULL. */
void orc_norm_modulate(int64_t rows, int64_t D, int64_t seq, const float *x,
                       const float *norm_w, double eps, const float *shift,
                       const float *scale, int dt, int pow_mode, float *h, float *inv_out)
{
    volatile float two = 2.0f, mhalf = -0.5f; /* runtime exponents: no folding */
    const float p2 = two, pm = mhalf;
    const float inv_d = (float)(1.0 / (double)(orc_mutation == MUT_VAR_D_MINUS_1 ? D - 1 : D));
    const float eps_f = (float)eps;
    for (int64_t r = 0; r < rows; ++r) {
        const float *xr = x + r * D;
        float ss = 0.0f;
        for (int64_t d = 0; d < D; ++d) {
            const float sq = pow_mode ? xr[d] * xr[d] : powf(xr[d], p2);
            ss = ss + sq;
        }
        const float var = ss * inv_d;
        const float t = var + eps_f;
        const float inv = pow_mode ? (float)(1.0 / sqrt((double)t)) : powf(t, pm);
        if (inv_out) inv_out[r] = inv;
        const int64_t b = r / seq;
        const float *sc = scale + b * D, *sh = shift + b * D;
        float *hr = h + r * D;
        for (int64_t d = 0; d < D; ++d) {
            float n = xr[d] * inv;
            if (norm_w) n = n * norm_w[d];
            if (orc_mutation != MUT_NORM_NO_ROUND) n = round_dt(n, dt);
            const float opl = orc_mutation == MUT_MODULATE_NO_ONE ? sc[d] : sc[d] + 1.0f;
            float m = n * opl;
            m = m + sh[d];
            hr[d] = round_dt(m, dt);
        }
    }
}

/* out = x + y * gate (block.rs:101): y is the FFN output in the model dtype,
 * gate (rows / seq, D); the product and the sum each rounded to the model
 * dtype, as tensor ops in that dtype do. */
void orc_gated_residual(int64_t rows, int64_t D, int64_t seq, const float *x, const float *y,
                        const float *gate, int dt, float *out)
{
    for (int64_t r = 0; r < rows; ++r) {
        const float *g = gate + (r / seq) * D;
        for (int64_t d = 0; d < D; ++d) {
            const float t = round_dt(orc_mutation == MUT_UNGATED_RESIDUAL ? y[r * D + d]
                                                                       : y[r * D + d] * g[d], dt);
            out[r * D + d] = round_dt(x[r * D + d] + t, dt);
        }
    }
}

int orc_num_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void orc_set_num_threads(int n)
{
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}
