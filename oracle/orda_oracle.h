/*
 * orda_oracle.h — CPU restatement of the reference crate's distillation-loss
 * path (malcolmgreaves/orda-cutile-rs), used ONLY as the parity oracle.
 *
 * TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load this library. The product (liborda_hip.so) never
 * links or calls it.
 *
 * Every function names the reference file:line it restates. The arithmetic
 * keeps the reference's types (f32 GEMMs with sequential accumulation, f64
 * row math) and loop orders; the library is compiled with
 * -ffp-contract=off so no multiply-add is fused, as in Rust.
 */
#ifndef ORDA_ORACLE_H
#define ORDA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- resolver.rs ------------------------------------------------------ */
size_t ora_ceil_div(size_t a, size_t b);                       /* resolver.rs:18-21  */
size_t ora_chunks_from_raw(double raw);                        /* resolver.rs:27-36  */
/* fixed==0 → ChunkSize::Auto, else ChunkSize::Fixed(fixed_rows).
 * has_v/has_max_chunks encode the Option<usize> arguments.     resolver.rs:53-99  */
void ora_resolve_chunk_size(size_t bt, int fixed, size_t fixed_rows, int has_v,
                            size_t v, int has_max_chunks, size_t max_chunks,
                            size_t *chunk_size, size_t *num_chunks);
size_t ora_default_max_chunks_limit(size_t bt);                /* resolver.rs:103-105 */
/* Returns the schedule length; writes up to cap entries.       resolver.rs:114-126 */
size_t ora_chunk_doubling_schedule(size_t bt, size_t start, size_t limit,
                                   size_t *out, size_t cap);

/* ---- config.rs -------------------------------------------------------- */
int ora_is_power_of_two(size_t v);                             /* config.rs:123-125  */

/* ---- mat.rs (row-major f32) ------------------------------------------- */
void ora_set_threads(int n);   /* threads of the three products; default 1 */
void ora_matmul_nt(const float *a, const float *b, float *out, size_t m,
                   size_t k, size_t n);                        /* mat.rs:63-80   */
void ora_matmul_nn(const float *a, const float *b, float *out, size_t m,
                   size_t k, size_t n);                        /* mat.rs:86-105  */
void ora_matmul_tn(const float *a, const float *b, float *out, size_t k,
                   size_t m, size_t n);                        /* mat.rs:111-130 */

/* ---- reference/cross_entropy.rs ---------------------------------------- */
float ora_ce_fwdbwd_row(const float *x, size_t v, int64_t y, int64_t ignore_index,
                        float label_smoothing, float scale, float *grad);
                                                     /* cross_entropy.rs:20-74 */

/* ---- reference/kl.rs --------------------------------------------------- */
void ora_softmax_logsoftmax(const float *x, size_t v, double inv_t, double *p,
                            double *log_p);                    /* kl.rs:20-41   */
double ora_forward_kl_row(const float *s, const float *t, size_t v,
                          double temperature);                 /* kl.rs:45-54   */
/* grad may be NULL (compute_grad=false).                       kl.rs:66-127  */
float ora_kl_chunk(const float *logits_chunk, const int64_t *targets, size_t n_rows,
                   size_t v, float kl_weight, float temperature, int64_t ignore_index,
                   float grad_denom, float *grad);

/* ---- quant.rs ---------------------------------------------------------- */
uint64_t ora_rng_new(uint64_t seed);                            /* quant.rs:23-27 */
uint64_t ora_rng_next_u64(uint64_t *state);                     /* quant.rs:29-37 */
float ora_rng_next_f32(uint64_t *state);                        /* quant.rs:39-43 */
float ora_round_half_even(float x);                             /* quant.rs:48-63 */
float ora_row_scale(const float *row, size_t cols);             /* quant.rs:90-94 */
void ora_quantize_rowwise_int8(const float *m, size_t rows, size_t cols, int8_t *q,
                               float *scale);                   /* quant.rs:96-117 */
void ora_quantize_rowwise_int8_stochastic(const float *m, size_t rows, size_t cols,
                                          uint64_t *rng_state, int8_t *q,
                                          float *scale);        /* quant.rs:120-144 */
/* Sorted, de-duplicated in-range non-ignored targets; returns count. quant.rs:163-171 */
size_t ora_unique_targets(const int64_t *target, size_t n, int64_t ignore_index,
                          size_t rows, size_t *out);
/* quantize_grad_w + dequantize_grad_w(·, grad_output) in one call: writes the
 * dequantized matrix to out (may alias nothing), codes and scales.
 * stochastic: 0 = RNE, 1 = SplitMix64 seeded with seed.        quant.rs:157-202 */
void ora_quant_dequant_grad_w(const float *grad_w, size_t rows, size_t cols,
                              const int64_t *target, size_t n_target,
                              int64_t ignore_index, int stochastic, uint64_t seed,
                              float grad_output, float *out, int8_t *q, float *scale);

/* ---- api.rs ------------------------------------------------------------ */
enum { ORA_TIED = 0, ORA_SEPARATE = 1, ORA_PRECOMPUTED = 2 };
enum { ORA_MEAN = 0, ORA_SUM = 1 };
enum { ORA_BACKEND_AUTO = 0, ORA_BACKEND_CPU = 1, ORA_BACKEND_GPU = 2 };

/* LossOptions + KernelConfig (api.rs:25-64, config.rs:45-90). Option<T>
 * fields carry a has_* flag. */
typedef struct {
    float student_ce_weight;
    int has_teacher_ce_weight;
    float teacher_ce_weight;
    float kd_weight;
    float temperature;
    int64_t ignore_index;
    float label_smoothing;
    int reduction;
    int chunk_fixed;          /* 0 = Auto, 1 = Fixed(chunk_rows) */
    size_t chunk_rows;
    int backend;
    /* KernelConfig */
    int online_softmax, fast_math, quantize_grad_weight, stochastic_rounding,
        fp32_grad_weight_accumulation;
    int has_max_chunks;
    size_t max_chunks;
    size_t max_fused_size;
    int has_stochastic_seed;
    uint64_t stochastic_seed;
} ora_options;

void ora_options_default(ora_options *o);                       /* api.rs:49-64 */

/* Teacher (teacher.rs:11-32). Fields not used by the mode are ignored. */
typedef struct {
    int mode;
    const float *hidden; size_t hidden_rows, hidden_cols;     /* Tied / Separate */
    const float *weight; size_t weight_rows, weight_cols;     /* Separate        */
    const float *logits; size_t logits_rows, logits_cols;     /* Precomputed     */
} ora_teacher;

/* DistillationLossOutput (api.rs:71-92). Caller allocates the gradient
 * buffers: grad_student_hidden [BT,H], grad_weight [V,H], and, when the
 * corresponding has_* flag will be set, grad_teacher_hidden [BT,Ht] and
 * grad_teacher_weight [V,Ht]. Optional extras (NULL to skip):
 * row_nll_s / row_nll_t / row_kl [BT] per-row values (kl with T² applied, 0
 * for ignored rows), q_codes [V,H] and q_scales [V] when quantizing. */
typedef struct {
    float loss, student_ce, teacher_ce, kl;
    float *grad_student_hidden;
    float *grad_weight;
    float *grad_teacher_hidden; int has_grad_teacher_hidden;
    float *grad_teacher_weight; int has_grad_teacher_weight;
    size_t chunk_size, num_chunks;
    float *row_nll_s, *row_nll_t, *row_kl;
    int8_t *q_codes; float *q_scales;
} ora_output;

/* Returns 0 on success, 1 on a validation error (message in err). */
int ora_distillation_loss(const float *student_hidden, size_t bt, size_t h,
                          const float *weight, size_t wv, size_t wh,
                          const int64_t *labels, size_t n_labels,
                          const ora_teacher *teacher, const ora_options *opts,
                          ora_output *out, char *err, size_t err_len);   /* api.rs:188-422 */

/* f64 forward (api.rs:511-572). kl_teacher_logits [BT,V] may be NULL. */
int ora_forward_loss_f64(const float *student_hidden, size_t bt, size_t h,
                         const float *weight, size_t wv, size_t wh,
                         const int64_t *labels, size_t n_labels,
                         const ora_teacher *teacher, const ora_options *opts,
                         const float *kl_teacher_logits, double *loss, char *err,
                         size_t err_len);

#ifdef __cplusplus
}
#endif
#endif
