/*
 * orda_oracle.c — CPU restatement of malcolmgreaves/orda-cutile-rs's
 * `distillation_loss` path. TEST INFRASTRUCTURE ONLY: it is the parity
 * oracle of the HIP library's tests and the CPU baseline of bench.py; the
 * product never links it.
 *
 * Each function cites the reference file:line it restates. Types follow the
 * reference exactly (Rust f32 -> float, f64 -> double, usize -> size_t), loops
 * keep the reference's order, and the file is built with -ffp-contract=off
 * so that a*b+c is never fused (Rust does not fuse). libm's exp/log are the
 * ones Rust's f64::exp/ln call on Linux.
 *
 * Pins (what checks this restatement; see tests/test_oracle_*.py):
 *   resolver   — every integer known answer of resolver.rs:133-189 plus the
 *                closed-form plans of the five benchmark shapes;
 *   mat        — mat.rs:152-176 known answers, brute-force f64 GEMM;
 *   CE row     — cross_entropy.rs:92-148 closed forms (textbook softmax);
 *   KL         — kl.rs:160-223 closed forms (2-class sigmoid, KL(p||p)=0,
 *                KL>=0, temperature-scaled gradient);
 *   quant      — quant.rs:209-275 (RNE table, 0.5*scale bound, unbiased
 *                stochastic mean, exact target rows) and the published
 *                SplitMix64 reference outputs;
 *   api        — tests/end_to_end.rs:90-417 restated: finite-difference
 *                gradients for all teacher modes against the independent f64
 *                forward, chunk invariance, component identity, sum = mean*n,
 *                INT8 bounds.
 */
#include "orda_oracle.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ======================================================================
 * resolver.rs
 * ==================================================================== */

/* resolver.rs:18-21 */
size_t ora_ceil_div(size_t a, size_t b) { return a / b + (a % b != 0); }

/* resolver.rs:27-36 — 1 below 1.5, else 2^(floor(log2(raw/1.5))+1). */
size_t ora_chunks_from_raw(double raw) {
    if (raw < 1.5) return 1;
    double e = floor(log2(raw / 1.5));
    /* Rust `as i64` saturates; clamp(0, 60) follows. */
    long long ei;
    if (isnan(e)) ei = 0;
    else if (e > 1e18) ei = 1000000000000000000LL;
    else if (e < -1e18) ei = -1000000000000000000LL;
    else ei = (long long)e;
    ei += 1;
    if (ei < 0) ei = 0;
    if (ei > 60) ei = 60;
    return (size_t)1 << (unsigned)ei;
}

static size_t min_sz(size_t a, size_t b) { return a < b ? a : b; }
static size_t max_sz(size_t a, size_t b) { return a > b ? a : b; }

/* resolver.rs:53-99 */
void ora_resolve_chunk_size(size_t bt, int fixed, size_t fixed_rows, int has_v,
                            size_t v, int has_max_chunks, size_t max_chunks,
                            size_t *chunk_size, size_t *num_chunks) {
    if (bt == 0) { /* the reference asserts bt > 0 */
        *chunk_size = 0;
        *num_chunks = 0;
        return;
    }
    if (fixed) {
        size_t cs = max_sz(min_sz(fixed_rows, bt), 1);
        *chunk_size = cs;
        *num_chunks = ora_ceil_div(bt, cs);
        return;
    }
    if (!has_v) {
        *chunk_size = bt;
        *num_chunks = 1;
        return;
    }
    size_t max_useful = max_sz(bt / 512, 1);
    size_t mc = has_max_chunks ? max_chunks : 2 * max_useful;
    double vr = (double)v / 32768.0;
    double raw_pressure = ((double)bt / 1024.0) * (vr * vr); /* powi(2) */
    double raw_bt_floor = (double)bt / 4096.0;
    double raw = fmax(raw_pressure, raw_bt_floor);
    size_t n = ora_chunks_from_raw(raw);
    n = min_sz(n, mc);
    n = min_sz(n, max_useful);
    n = min_sz(n, bt);
    n = max_sz(n, 1);
    *chunk_size = ora_ceil_div(bt, n);
    *num_chunks = n;
}

/* resolver.rs:103-105 */
size_t ora_default_max_chunks_limit(size_t bt) { return 2 * max_sz(bt / 512, 1); }

/* resolver.rs:114-126 */
size_t ora_chunk_doubling_schedule(size_t bt, size_t start, size_t limit,
                                   size_t *out, size_t cap) {
    limit = min_sz(max_sz(limit, 1), bt);
    if (limit < 1) return 0; /* bt == 0: the reference's clamp panics */
    size_t n = start < 1 ? 1 : (start > limit ? limit : start);
    size_t len = 0;
    if (len < cap) out[len] = n;
    len++;
    while (n < bt && n < limit) {
        n = min_sz(min_sz(n * 2, bt), limit);
        if (len < cap) out[len] = n;
        len++;
        if (n >= bt || n >= limit) break;
    }
    return len;
}

/* config.rs:123-125 */
int ora_is_power_of_two(size_t v) { return v > 0 && (v & (v - 1)) == 0; }

/* ======================================================================
 * mat.rs
 * ==================================================================== */

/* Threads for the three products below and for the element-wise and
 * row-wise loops over whole matrices (add/scale, deterministic INT8 rows);
 * 1, the default, is the reference's single thread. With more, output rows or
 * elements are shared out between threads; every output element still
 * accumulates its terms in the reference's order, so the results are bitwise
 * the same (the oracle's tests check this). Only the CPU baseline's all-core
 * timing sets it. */
static int g_threads = 1;

void ora_set_threads(int n) { g_threads = n > 1 ? n : 1; }

/* mat.rs:63-80 — out = a @ bᵀ, sequential f32 dot from 0. */
void ora_matmul_nt(const float *a, const float *b, float *out, size_t m, size_t k,
                   size_t n) {
#pragma omp parallel for if (g_threads > 1) num_threads(g_threads) schedule(static)
    for (size_t i = 0; i < m; i++) {
        const float *arow = a + i * k;
        float *orow = out + i * n;
        for (size_t j = 0; j < n; j++) {
            const float *brow = b + j * k;
            float acc = 0.0f;
            for (size_t p = 0; p < k; p++) acc += arow[p] * brow[p];
            orow[j] = acc;
        }
    }
}

/* mat.rs:86-105 — out = a @ b, zero entries of a skipped. */
void ora_matmul_nn(const float *a, const float *b, float *out, size_t m, size_t k,
                   size_t n) {
    memset(out, 0, m * n * sizeof(float));
#pragma omp parallel for if (g_threads > 1) num_threads(g_threads) schedule(static)
    for (size_t i = 0; i < m; i++) {
        const float *arow = a + i * k;
        float *orow = out + i * n;
        for (size_t p = 0; p < k; p++) {
            float aip = arow[p];
            if (aip == 0.0f) continue;
            const float *brow = b + p * n;
            for (size_t j = 0; j < n; j++) orow[j] += aip * brow[j];
        }
    }
}

/* mat.rs:111-130 — out = aᵀ @ b with a [k,m], b [k,n]. */
void ora_matmul_tn(const float *a, const float *b, float *out, size_t k, size_t m,
                   size_t n) {
    memset(out, 0, m * n * sizeof(float));
    if (g_threads > 1) {
        /* Output row i on one thread: its terms arrive in p order, as below. */
#pragma omp parallel for num_threads(g_threads) schedule(static)
        for (size_t i = 0; i < m; i++) {
            float *orow = out + i * n;
            for (size_t p = 0; p < k; p++) {
                float aip = a[p * m + i];
                if (aip == 0.0f) continue;
                const float *brow = b + p * n;
                for (size_t j = 0; j < n; j++) orow[j] += aip * brow[j];
            }
        }
        return;
    }
    for (size_t p = 0; p < k; p++) {
        const float *arow = a + p * m;
        const float *brow = b + p * n;
        for (size_t i = 0; i < m; i++) {
            float aip = arow[i];
            if (aip == 0.0f) continue;
            float *orow = out + i * n;
            for (size_t j = 0; j < n; j++) orow[j] += aip * brow[j];
        }
    }
}

/* mat.rs:133-138 */
static void add_assign(float *dst, const float *src, size_t len) {
#pragma omp parallel for if (g_threads > 1) num_threads(g_threads) schedule(static)
    for (size_t i = 0; i < len; i++) dst[i] += src[i];
}

/* mat.rs:141-145 */
static void scale_assign(float *m, size_t len, float s) {
#pragma omp parallel for if (g_threads > 1) num_threads(g_threads) schedule(static)
    for (size_t i = 0; i < len; i++) m[i] *= s;
}

/* ======================================================================
 * reference/cross_entropy.rs
 * ==================================================================== */

/* cross_entropy.rs:20-74 — f64 row math; grad (length v) always written. */
float ora_ce_fwdbwd_row(const float *x, size_t v, int64_t y, int64_t ignore_index,
                        float label_smoothing, float scale, float *grad) {
    int ignored = (y == ignore_index);
    double alpha = (double)label_smoothing;

    double m = -INFINITY;
    for (size_t j = 0; j < v; j++)
        if ((double)x[j] > m) m = (double)x[j];
    double d = 0.0, sum_x = 0.0;
    for (size_t j = 0; j < v; j++) {
        d += exp((double)x[j] - m);
        if (alpha > 0.0) sum_x += (double)x[j];
    }
    double lse = m + log(d);

    size_t y_safe = ignored ? 0 : (size_t)y;
    double logit_tgt = (double)x[y_safe];
    double nll;
    if (alpha > 0.0)
        nll = lse - (1.0 - alpha) * logit_tgt - (alpha / (double)v) * sum_x;
    else
        nll = lse - logit_tgt;
    if (ignored) nll = 0.0;

    double eff_scale = ignored ? 0.0 : (double)scale;
    double eps = alpha / (double)v;
    for (size_t j = 0; j < v; j++) grad[j] = 0.0f;
    if (eff_scale != 0.0) {
        for (size_t j = 0; j < v; j++) {
            double p = exp((double)x[j] - m) / d;
            double prob = alpha > 0.0 ? p - eps : p;
            if (j == y_safe) prob -= 1.0 - alpha;
            grad[j] = (float)(prob * eff_scale);
        }
    }
    return (float)nll;
}

/* ======================================================================
 * reference/kl.rs
 * ==================================================================== */

/* kl.rs:20-41 */
void ora_softmax_logsoftmax(const float *x, size_t v, double inv_t, double *p,
                            double *log_p) {
    double m = -INFINITY;
    for (size_t j = 0; j < v; j++) {
        double z = (double)x[j] * inv_t;
        if (z > m) m = z;
    }
    double d = 0.0;
    for (size_t j = 0; j < v; j++) d += exp(((double)x[j] * inv_t) - m);
    double log_d = log(d);
    for (size_t j = 0; j < v; j++) {
        double zc = ((double)x[j] * inv_t) - m;
        p[j] = exp(zc) / d;
        log_p[j] = zc - log_d;
    }
}

/* kl.rs:45-54 */
double ora_forward_kl_row(const float *s, const float *t, size_t v, double temperature) {
    double inv_t = 1.0 / temperature;
    double *buf = (double *)malloc(4 * v * sizeof(double));
    double *ps = buf, *lps = buf + v, *pt = buf + 2 * v, *lpt = buf + 3 * v;
    ora_softmax_logsoftmax(s, v, inv_t, ps, lps);
    ora_softmax_logsoftmax(t, v, inv_t, pt, lpt);
    double kl = 0.0;
    for (size_t j = 0; j < v; j++) kl += pt[j] * (lpt[j] - lps[j]);
    free(buf);
    return kl;
}

/* kl.rs:66-127 — logits_chunk is [2*n_rows, v], student rows first. */
float ora_kl_chunk(const float *logits_chunk, const int64_t *targets, size_t n_rows,
                   size_t v, float kl_weight, float temperature, int64_t ignore_index,
                   float grad_denom, float *grad) {
    double inv_t = 1.0 / (double)temperature;
    float gs32 = kl_weight * temperature / grad_denom; /* f32, then widened */
    double grad_scale = (double)gs32;
    float tsq32 = temperature * temperature;
    double t_sq = (double)tsq32;

    double *buf = (double *)malloc(4 * v * sizeof(double));
    double *ps = buf, *lps = buf + v, *pt = buf + 2 * v, *lpt = buf + 3 * v;
    double kl_accum = 0.0;
    if (grad) memset(grad, 0, n_rows * v * sizeof(float));
    for (size_t i = 0; i < n_rows; i++) {
        int ignored = targets[i] == ignore_index;
        const float *s = logits_chunk + i * v;
        const float *t = logits_chunk + (n_rows + i) * v;
        ora_softmax_logsoftmax(s, v, inv_t, ps, lps);
        ora_softmax_logsoftmax(t, v, inv_t, pt, lpt);
        double kl_row = 0.0;
        for (size_t j = 0; j < v; j++) kl_row += pt[j] * (lpt[j] - lps[j]);
        if (ignored) kl_row = 0.0;
        kl_accum += kl_row * t_sq;
        if (grad) {
            float *grow = grad + i * v;
            if (ignored) {
                for (size_t j = 0; j < v; j++) grow[j] = 0.0f;
            } else {
                for (size_t j = 0; j < v; j++) grow[j] = (float)(grad_scale * (ps[j] - pt[j]));
            }
        }
    }
    free(buf);
    return (float)kl_accum;
}

/* Per-row variant used to expose per-row KL (same arithmetic as the loop
 * body above; returns kl_row * t_sq, 0 for an ignored row). */
static double kl_row_scaled(const float *s, const float *t, size_t v, int ignored,
                            double inv_t, double t_sq, double *buf) {
    double *ps = buf, *lps = buf + v, *pt = buf + 2 * v, *lpt = buf + 3 * v;
    ora_softmax_logsoftmax(s, v, inv_t, ps, lps);
    ora_softmax_logsoftmax(t, v, inv_t, pt, lpt);
    double kl_row = 0.0;
    for (size_t j = 0; j < v; j++) kl_row += pt[j] * (lpt[j] - lps[j]);
    if (ignored) kl_row = 0.0;
    return kl_row * t_sq;
}

/* ======================================================================
 * quant.rs
 * ==================================================================== */

#define GOLDEN_GAMMA 0x9E3779B97F4A7C15ULL

/* quant.rs:23-27 */
uint64_t ora_rng_new(uint64_t seed) { return seed + GOLDEN_GAMMA; }

/* quant.rs:29-37 — SplitMix64 (Steele, Lea & Flood, OOPSLA 2014). */
uint64_t ora_rng_next_u64(uint64_t *state) {
    *state += GOLDEN_GAMMA;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

/* quant.rs:39-43 */
float ora_rng_next_f32(uint64_t *state) {
    return (float)(ora_rng_next_u64(state) >> 40) * (1.0f / (float)(1u << 24));
}

/* quant.rs:48-63 */
float ora_round_half_even(float x) {
    float f = floorf(x);
    float diff = x - f;
    if (diff < 0.5f) return f;
    if (diff > 0.5f) return f + 1.0f;
    if (isnan(f)) return f; /* Rust: NaN as i64 == 0 (even) -> f */
    long long fi = (long long)f;
    return (fi % 2 == 0) ? f : f + 1.0f;
}

/* Rust f32::clamp then `as i8` (saturating, NaN -> 0). */
static int8_t clamp_to_i8(float v) {
    if (isnan(v)) return 0;
    if (v < -127.0f) v = -127.0f;
    if (v > 127.0f) v = 127.0f;
    return (int8_t)v;
}

/* quant.rs:90-94 — f32::max ignores NaN, like fmaxf. */
float ora_row_scale(const float *row, size_t cols) {
    float amax = 0.0f;
    for (size_t c = 0; c < cols; c++) amax = fmaxf(amax, fabsf(row[c]));
    return fmaxf(amax, 1e-12f) / 127.0f;
}

/* quant.rs:96-117 */
void ora_quantize_rowwise_int8(const float *m, size_t rows, size_t cols, int8_t *q,
                               float *scale) {
#pragma omp parallel for if (g_threads > 1) num_threads(g_threads) schedule(static)
    for (size_t r = 0; r < rows; r++) {
        const float *row = m + r * cols;
        float s = ora_row_scale(row, cols);
        scale[r] = s;
        for (size_t c = 0; c < cols; c++)
            q[r * cols + c] = clamp_to_i8(ora_round_half_even(row[c] / s));
    }
}

/* quant.rs:120-144 — one uniform per element, row-major. */
void ora_quantize_rowwise_int8_stochastic(const float *m, size_t rows, size_t cols,
                                          uint64_t *rng_state, int8_t *q,
                                          float *scale) {
    for (size_t r = 0; r < rows; r++) {
        const float *row = m + r * cols;
        float s = ora_row_scale(row, cols);
        scale[r] = s;
        for (size_t c = 0; c < cols; c++) {
            float scaled = row[c] / s;
            float floor_v = floorf(scaled);
            float frac = scaled - floor_v;
            float bump = frac > ora_rng_next_f32(rng_state) ? 1.0f : 0.0f;
            q[r * cols + c] = clamp_to_i8(floor_v + bump);
        }
    }
}

static int cmp_size(const void *a, const void *b) {
    size_t x = *(const size_t *)a, y = *(const size_t *)b;
    return (x > y) - (x < y);
}

/* quant.rs:163-171 */
size_t ora_unique_targets(const int64_t *target, size_t n, int64_t ignore_index,
                          size_t rows, size_t *out) {
    size_t cnt = 0;
    for (size_t i = 0; i < n; i++) {
        int64_t t = target[i];
        if (t != ignore_index && t >= 0 && (uint64_t)t < rows) out[cnt++] = (size_t)t;
    }
    qsort(out, cnt, sizeof(size_t), cmp_size);
    size_t u = 0;
    for (size_t i = 0; i < cnt; i++)
        if (u == 0 || out[u - 1] != out[i]) out[u++] = out[i];
    return u;
}

/* quant.rs:157-202 (quantize_grad_w followed by dequantize_grad_w). */
void ora_quant_dequant_grad_w(const float *grad_w, size_t rows, size_t cols,
                              const int64_t *target, size_t n_target,
                              int64_t ignore_index, int stochastic, uint64_t seed,
                              float grad_output, float *out, int8_t *q, float *scale) {
    size_t *uniq = (size_t *)malloc((n_target ? n_target : 1) * sizeof(size_t));
    size_t nu = ora_unique_targets(target, n_target, ignore_index, rows, uniq);
    if (stochastic) {
        uint64_t st = ora_rng_new(seed);
        ora_quantize_rowwise_int8_stochastic(grad_w, rows, cols, &st, q, scale);
    } else {
        ora_quantize_rowwise_int8(grad_w, rows, cols, q, scale);
    }
    /* QuantRows::dequantize (quant.rs:77-87) */
#pragma omp parallel for if (g_threads > 1) num_threads(g_threads) schedule(static)
    for (size_t r = 0; r < rows; r++) {
        float s = scale[r];
        for (size_t c = 0; c < cols; c++) out[r * cols + c] = (float)q[r * cols + c] * s;
    }
    for (size_t i = 0; i < nu; i++)
        memcpy(out + uniq[i] * cols, grad_w + uniq[i] * cols, cols * sizeof(float));
    scale_assign(out, rows * cols, grad_output);
    free(uniq);
}

/* ======================================================================
 * api.rs
 * ==================================================================== */

/* api.rs:49-64, config.rs:68-90 (Profile::Balanced) */
void ora_options_default(ora_options *o) {
    memset(o, 0, sizeof(*o));
    o->student_ce_weight = 1.0f;
    o->has_teacher_ce_weight = 0;
    o->kd_weight = 0.0f;
    o->temperature = 1.0f;
    o->ignore_index = -100;
    o->label_smoothing = 0.0f;
    o->reduction = ORA_MEAN;
    o->chunk_fixed = 0;
    o->backend = ORA_BACKEND_AUTO;
    o->max_fused_size = 65536 / 2;
}

static void set_err(char *err, size_t len, const char *fmt, ...) {
    if (!err || !len) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, len, fmt, ap);
    va_end(ap);
}

/* api.rs:104-181 and config.rs:106-119. Returns 0 when valid. */
static int validate(size_t bt, size_t h, size_t wv, size_t wh, const int64_t *labels,
                    size_t n_labels, const ora_teacher *t, const ora_options *o,
                    char *err, size_t err_len) {
    if (o->max_fused_size < 1 || !ora_is_power_of_two(o->max_fused_size)) {
        set_err(err, err_len, "max_fused_size must be a power of two >= 1, got %zu",
                o->max_fused_size);
        return 1;
    }
    if (o->has_max_chunks && o->max_chunks < 1) {
        set_err(err, err_len, "max_chunks must be >= 1, got %zu", o->max_chunks);
        return 1;
    }
    if (bt == 0) {
        set_err(err, err_len, "student_hidden has 0 rows (BT must be > 0)");
        return 1;
    }
    if (wh != h) {
        set_err(err, err_len, "weight must have shape (V, %zu), got (%zu, %zu)", h, wv, wh);
        return 1;
    }
    size_t v = wv;
    if (n_labels != bt) {
        set_err(err, err_len, "labels must have length BT=%zu, got %zu", bt, n_labels);
        return 1;
    }
    for (size_t i = 0; i < n_labels; i++) {
        int64_t tl = labels[i];
        if (tl != o->ignore_index && (tl < 0 || (uint64_t)tl >= v)) {
            set_err(err, err_len, "label %lld out of range [0, %zu) and != ignore_index %lld",
                    (long long)tl, v, (long long)o->ignore_index);
            return 1;
        }
    }
    if (!(o->label_smoothing >= 0.0f && o->label_smoothing <= 1.0f)) {
        set_err(err, err_len, "label_smoothing must be in [0,1], got %g",
                (double)o->label_smoothing);
        return 1;
    }
    if (o->kd_weight < 0.0f) {
        set_err(err, err_len, "kd_weight must be >= 0, got %g", (double)o->kd_weight);
        return 1;
    }
    if (o->temperature <= 0.0f) {
        set_err(err, err_len, "temperature must be > 0, got %g", (double)o->temperature);
        return 1;
    }
    switch (t->mode) {
    case ORA_TIED:
        if (t->hidden_rows != bt || t->hidden_cols != h) {
            set_err(err, err_len, "Tied teacher hidden must be (%zu, %zu), got (%zu, %zu)",
                    bt, h, t->hidden_rows, t->hidden_cols);
            return 1;
        }
        break;
    case ORA_SEPARATE:
        if (t->hidden_rows != bt) {
            set_err(err, err_len, "Separate teacher hidden must have BT=%zu rows", bt);
            return 1;
        }
        if (t->weight_rows != v || t->weight_cols != t->hidden_cols) {
            set_err(err, err_len, "Separate teacher weight must be (%zu, %zu), got (%zu, %zu)",
                    v, t->hidden_cols, t->weight_rows, t->weight_cols);
            return 1;
        }
        break;
    case ORA_PRECOMPUTED:
        if (t->logits_rows != bt || t->logits_cols != v) {
            set_err(err, err_len,
                    "Precomputed teacher logits must be (%zu, %zu), got (%zu, %zu)", bt, v,
                    t->logits_rows, t->logits_cols);
            return 1;
        }
        break;
    default:
        set_err(err, err_len, "unknown teacher mode %d", t->mode);
        return 1;
    }
    return 0;
}

/* teacher.rs:54-59 */
static float default_teacher_ce_weight(int mode) { return mode == ORA_TIED ? 1.0f : 0.0f; }

/* api.rs:188-422 */
int ora_distillation_loss(const float *student_hidden, size_t bt, size_t h,
                          const float *weight, size_t wv, size_t wh,
                          const int64_t *labels, size_t n_labels,
                          const ora_teacher *teacher, const ora_options *opts,
                          ora_output *out, char *err, size_t err_len) {
    if (validate(bt, h, wv, wh, labels, n_labels, teacher, opts, err, err_len)) return 1;
    size_t v = wv;
    if (opts->backend == ORA_BACKEND_GPU) {
        set_err(err, err_len, "the CPU oracle serves Backend::Auto and Backend::Cpu only");
        return 1;
    }
    int mode = teacher->mode;
    float w_s = opts->student_ce_weight;
    float w_t = opts->has_teacher_ce_weight ? opts->teacher_ce_weight
                                            : default_teacher_ce_weight(mode);
    if (w_t < 0.0f) {
        set_err(err, err_len, "teacher_ce_weight must be >= 0, got %g", (double)w_t);
        return 1;
    }
    float kd = opts->kd_weight;
    float temperature = opts->temperature;
    float ls = opts->label_smoothing;
    int64_t ignore = opts->ignore_index;
    int need_teacher = kd > 0.0f || w_t > 0.0f;

    size_t n_non_ignore = 0;
    for (size_t i = 0; i < bt; i++) n_non_ignore += labels[i] != ignore;
    size_t denom = opts->reduction == ORA_MEAN ? max_sz(n_non_ignore, 1) : 1;
    float mean_scale = 1.0f / (float)denom;

    size_t cs, nc;
    ora_resolve_chunk_size(bt, opts->chunk_fixed, opts->chunk_rows, 1, v,
                           opts->has_max_chunks, opts->max_chunks, &cs, &nc);

    size_t ht_dim = mode == ORA_SEPARATE ? teacher->hidden_cols : h;
    int has_ght = w_t > 0.0f && (mode == ORA_TIED || mode == ORA_SEPARATE);
    int has_gwt = w_t > 0.0f && mode == ORA_SEPARATE;

    float *grad_h_s = out->grad_student_hidden;
    float *grad_w = out->grad_weight;
    float *grad_h_t = out->grad_teacher_hidden;
    float *grad_w_t = out->grad_teacher_weight;
    memset(grad_h_s, 0, bt * h * sizeof(float));
    memset(grad_w, 0, v * h * sizeof(float));
    if (has_ght) memset(grad_h_t, 0, bt * ht_dim * sizeof(float));
    if (has_gwt) memset(grad_w_t, 0, v * ht_dim * sizeof(float));

    double sum_nll_s = 0.0, sum_nll_t = 0.0, kl_accum = 0.0;

    size_t hmax = h > ht_dim ? h : ht_dim;
    float *logits_chunk = (float *)malloc(2 * cs * v * sizeof(float));
    float *grad_kl = (float *)malloc(cs * v * sizeof(float));
    float *g = (float *)malloc(v * sizeof(float));
    float *gh_chunk = (float *)malloc(cs * hmax * sizeof(float));
    float *tn_tmp = (float *)malloc(v * hmax * sizeof(float));
    double *klbuf = (double *)malloc(4 * v * sizeof(double));

    for (size_t c = 0; c < nc; c++) {
        size_t start = c * cs;
        if (start >= bt) break;
        size_t end = min_sz(start + cs, bt);
        size_t n = end - start;

        const float *h_s_chunk = student_hidden + start * h;     /* sub_rows */
        ora_matmul_nt(h_s_chunk, weight, logits_chunk, n, h, v); /* student rows */

        const float *h_t_chunk = NULL;
        if (need_teacher) {
            float *lt = logits_chunk + n * v;
            if (mode == ORA_TIED) {
                h_t_chunk = teacher->hidden + start * h;
                ora_matmul_nt(h_t_chunk, weight, lt, n, h, v);
            } else if (mode == ORA_SEPARATE) {
                h_t_chunk = teacher->hidden + start * ht_dim;
                ora_matmul_nt(h_t_chunk, teacher->weight, lt, n, ht_dim, v);
            } else {
                memcpy(lt, teacher->logits + start * v, n * v * sizeof(float));
            }
        }

        /* KL reads clean logits (api.rs:301-316). */
        int have_kl = 0;
        if (kd > 0.0f) {
            float kl_sum_chunk = ora_kl_chunk(logits_chunk, labels + start, n, v, kd,
                                              temperature, ignore, 1.0f, grad_kl);
            kl_accum += (double)kl_sum_chunk;
            have_kl = 1;
            if (out->row_kl) {
                double inv_t = 1.0 / (double)temperature;
                double t_sq = (double)(temperature * temperature);
                for (size_t r = 0; r < n; r++)
                    out->row_kl[start + r] = (float)kl_row_scaled(
                        logits_chunk + r * v, logits_chunk + (n + r) * v, v,
                        labels[start + r] == ignore, inv_t, t_sq, klbuf);
            }
        } else if (out->row_kl) {
            for (size_t r = 0; r < n; r++) out->row_kl[start + r] = 0.0f;
        }

        /* CE student rows, in place (api.rs:318-323). */
        for (size_t r = 0; r < n; r++) {
            float nll = ora_ce_fwdbwd_row(logits_chunk + r * v, v, labels[start + r], ignore,
                                          ls, w_s, g);
            sum_nll_s += (double)nll;
            if (out->row_nll_s) out->row_nll_s[start + r] = nll;
            memcpy(logits_chunk + r * v, g, v * sizeof(float));
        }
        /* CE teacher rows (api.rs:325-333). */
        if (w_t > 0.0f) {
            for (size_t r = 0; r < n; r++) {
                float nll = ora_ce_fwdbwd_row(logits_chunk + (n + r) * v, v, labels[start + r],
                                              ignore, ls, w_t, g);
                sum_nll_t += (double)nll;
                if (out->row_nll_t) out->row_nll_t[start + r] = nll;
                memcpy(logits_chunk + (n + r) * v, g, v * sizeof(float));
            }
        } else if (out->row_nll_t) {
            for (size_t r = 0; r < n; r++) out->row_nll_t[start + r] = 0.0f;
        }
        /* KL merge (api.rs:335-344). */
        if (have_kl) {
            for (size_t r = 0; r < n; r++) {
                float *row = logits_chunk + r * v;
                const float *krow = grad_kl + r * v;
                for (size_t j = 0; j < v; j++) row[j] += krow[j];
            }
        }

        /* GEMM backward (api.rs:346-377). */
        const float *dS = logits_chunk;
        ora_matmul_nn(dS, weight, gh_chunk, n, v, h);
        memcpy(grad_h_s + start * h, gh_chunk, n * h * sizeof(float));
        ora_matmul_tn(dS, h_s_chunk, tn_tmp, n, v, h);
        add_assign(grad_w, tn_tmp, v * h);

        if (w_t > 0.0f) {
            const float *dT = logits_chunk + n * v;
            if (mode == ORA_TIED) {
                ora_matmul_nn(dT, weight, gh_chunk, n, v, h);
                memcpy(grad_h_t + start * ht_dim, gh_chunk, n * ht_dim * sizeof(float));
                ora_matmul_tn(dT, h_t_chunk, tn_tmp, n, v, h);
                add_assign(grad_w, tn_tmp, v * h);
            } else if (mode == ORA_SEPARATE) {
                ora_matmul_nn(dT, teacher->weight, gh_chunk, n, v, ht_dim);
                memcpy(grad_h_t + start * ht_dim, gh_chunk, n * ht_dim * sizeof(float));
                ora_matmul_tn(dT, h_t_chunk, tn_tmp, n, v, ht_dim);
                add_assign(grad_w_t, tn_tmp, v * ht_dim);
            }
        }
    }

    /* Deferred mean (api.rs:380-388). */
    scale_assign(grad_h_s, bt * h, mean_scale);
    scale_assign(grad_w, v * h, mean_scale);
    if (has_ght) scale_assign(grad_h_t, bt * ht_dim, mean_scale);
    if (has_gwt) scale_assign(grad_w_t, v * ht_dim, mean_scale);

    /* Optional INT8 round trip (api.rs:390-399). */
    if (opts->quantize_grad_weight) {
        int8_t *q = out->q_codes ? out->q_codes : (int8_t *)malloc(v * h);
        float *sc = out->q_scales ? out->q_scales : (float *)malloc(v * sizeof(float));
        float *deq = (float *)malloc(v * h * sizeof(float));
        uint64_t seed = opts->has_stochastic_seed ? opts->stochastic_seed : 0;
        ora_quant_dequant_grad_w(grad_w, v, h, labels, bt, ignore,
                                 opts->stochastic_rounding, seed, 1.0f, deq, q, sc);
        memcpy(grad_w, deq, v * h * sizeof(float));
        free(deq);
        if (!out->q_codes) free(q);
        if (!out->q_scales) free(sc);
    }

    /* api.rs:401-405 */
    double ms = (double)mean_scale;
    out->student_ce = (float)(sum_nll_s * ms);
    out->teacher_ce = (float)(sum_nll_t * ms);
    out->kl = (float)(kl_accum * ms);
    out->loss = (float)(((double)w_s * sum_nll_s + (double)w_t * sum_nll_t +
                         (double)kd * kl_accum) * ms);
    out->has_grad_teacher_hidden = has_ght;
    out->has_grad_teacher_weight = has_gwt;
    out->chunk_size = cs;
    out->num_chunks = nc;

    free(logits_chunk);
    free(grad_kl);
    free(g);
    free(gh_chunk);
    free(tn_tmp);
    free(klbuf);
    return 0;
}

/* ---- f64 forward oracle (api.rs:424-584) ------------------------------ */

/* api.rs:427-438 */
static void logits_row_f64(const float *h_row, size_t hdim, const float *w, size_t wrows,
                           double *out) {
    for (size_t vr = 0; vr < wrows; vr++) {
        const float *wr = w + vr * hdim;
        double acc = 0.0;
        for (size_t k = 0; k < hdim; k++) acc += (double)h_row[k] * (double)wr[k];
        out[vr] = acc;
    }
}

/* api.rs:441-462 */
static double nll_f64(const double *logits, size_t v, int64_t y, int64_t ignore_index,
                      double ls) {
    if (y == ignore_index) return 0.0;
    double m = -INFINITY;
    for (size_t j = 0; j < v; j++) m = fmax(m, logits[j]);
    double d = 0.0, sum_x = 0.0;
    for (size_t j = 0; j < v; j++) {
        d += exp(logits[j] - m);
        if (ls > 0.0) sum_x += logits[j];
    }
    double lse = m + log(d);
    double logit_tgt = logits[(size_t)y];
    if (ls > 0.0) return lse - (1.0 - ls) * logit_tgt - (ls / (double)v) * sum_x;
    return lse - logit_tgt;
}

/* api.rs:465-485 */
static double kl_f64(const double *s, const double *t, size_t v, double temperature,
                     double *buf) {
    double inv_t = 1.0 / temperature;
    const double *xs[2] = {s, t};
    double *lp[2] = {buf, buf + v};
    double *pt = buf + 2 * v;
    for (int w = 0; w < 2; w++) {
        const double *x = xs[w];
        double m = -INFINITY;
        for (size_t j = 0; j < v; j++) m = fmax(m, x[j] * inv_t);
        double d = 0.0;
        for (size_t j = 0; j < v; j++) d += exp(x[j] * inv_t - m);
        double log_d = log(d);
        for (size_t j = 0; j < v; j++) {
            if (w == 1) pt[j] = exp(x[j] * inv_t - m) / d;
            lp[w][j] = (x[j] * inv_t - m) - log_d;
        }
    }
    double kl = 0.0;
    for (size_t j = 0; j < v; j++) kl += pt[j] * (lp[1][j] - lp[0][j]);
    return kl;
}

/* api.rs:511-572 */
int ora_forward_loss_f64(const float *student_hidden, size_t bt, size_t h,
                         const float *weight, size_t wv, size_t wh,
                         const int64_t *labels, size_t n_labels,
                         const ora_teacher *teacher, const ora_options *opts,
                         const float *kl_teacher_logits, double *loss, char *err,
                         size_t err_len) {
    if (validate(bt, h, wv, wh, labels, n_labels, teacher, opts, err, err_len)) return 1;
    if (opts->backend == ORA_BACKEND_GPU) {
        set_err(err, err_len, "the CPU oracle serves Backend::Auto and Backend::Cpu only");
        return 1;
    }
    size_t v = wv;
    int mode = teacher->mode;
    double w_s = (double)opts->student_ce_weight;
    double w_t = (double)(opts->has_teacher_ce_weight ? opts->teacher_ce_weight
                                                      : default_teacher_ce_weight(mode));
    double kd = (double)opts->kd_weight;
    double temperature = (double)opts->temperature;
    double ls = (double)opts->label_smoothing;
    int64_t ignore = opts->ignore_index;
    double t_sq = temperature * temperature;

    size_t n_non_ignore = 0;
    for (size_t i = 0; i < bt; i++) n_non_ignore += labels[i] != ignore;
    double denom = (double)(opts->reduction == ORA_MEAN ? max_sz(n_non_ignore, 1) : 1);

    double *ls_row = (double *)malloc(v * sizeof(double));
    double *lt_row = (double *)malloc(v * sizeof(double));
    double *kt_row = (double *)malloc(v * sizeof(double));
    double *buf = (double *)malloc(3 * v * sizeof(double));
    double sum_nll_s = 0.0, sum_nll_t = 0.0, sum_kl = 0.0;
    size_t ht = mode == ORA_SEPARATE ? teacher->hidden_cols : h;

    for (size_t r = 0; r < bt; r++) {
        logits_row_f64(student_hidden + r * h, h, weight, v, ls_row);
        sum_nll_s += nll_f64(ls_row, v, labels[r], ignore, ls);
        int need_teacher = kd > 0.0 || w_t > 0.0;
        if (need_teacher) {
            if (mode == ORA_TIED)
                logits_row_f64(teacher->hidden + r * h, h, weight, v, lt_row);
            else if (mode == ORA_SEPARATE)
                logits_row_f64(teacher->hidden + r * ht, ht, teacher->weight, v, lt_row);
            else
                for (size_t j = 0; j < v; j++) lt_row[j] = (double)teacher->logits[r * v + j];
            if (w_t > 0.0) sum_nll_t += nll_f64(lt_row, v, labels[r], ignore, ls);
            if (kd > 0.0 && labels[r] != ignore) {
                const double *kt = lt_row;
                if (kl_teacher_logits) {
                    for (size_t j = 0; j < v; j++)
                        kt_row[j] = (double)kl_teacher_logits[r * v + j];
                    kt = kt_row;
                }
                sum_kl += kl_f64(ls_row, kt, v, temperature, buf) * t_sq;
            }
        }
    }
    *loss = (w_s * sum_nll_s + w_t * sum_nll_t + kd * sum_kl) / denom;
    free(ls_row);
    free(lt_row);
    free(kt_row);
    free(buf);
    return 0;
}
