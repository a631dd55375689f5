/*
 * orda.h — C ABI of liborda_hip.so, the MI355X (gfx950) backend of the
 * chunked fused cross-entropy + forward-KL distillation loss of
 * malcolmgreaves/orda-cutile-rs.
 *
 * This is the boundary a binding of the reference crate would call from a
 * `Backend::Hip` arm of `distillation_loss` (src/api.rs:197-207, the slot the
 * crate reserves for `Backend::Cuda`). Plain pointers, sizes and POD structs
 * only; no exceptions or panics cross it. Every entry point returns an
 * orda_status and, on failure, copies a message into `err` (the reference's
 * `Err(String)`).
 *
 * Threading: an orda_ctx owns one HIP stream, a device workspace and timing
 * state; use one context per host thread. Calls are synchronous at return,
 * like the reference.
 */
#ifndef ORDA_ORDA_H
#define ORDA_ORDA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORDA_ABI_VERSION 2

typedef enum {
    ORDA_OK = 0,
    ORDA_ERR_INVALID = 1,      /* validation failure (api.rs:104-181, :214-216) */
    ORDA_ERR_OOM = 2,          /* device memory exhausted after the doubling schedule */
    ORDA_ERR_HIP = 3,          /* a HIP runtime call failed */
    ORDA_ERR_UNAVAILABLE = 4,  /* no usable gfx950 device */
    ORDA_ERR_INTERNAL = 5
} orda_status;

typedef enum { ORDA_F32 = 0, ORDA_BF16 = 1, ORDA_I8 = 2 } orda_dtype;
typedef enum { ORDA_HOST = 0, ORDA_DEVICE = 1 } orda_location;

/* Teacher::{Tied, Separate, Precomputed} (src/teacher.rs:11-32). */
typedef enum { ORDA_TEACHER_TIED = 0, ORDA_TEACHER_SEPARATE = 1, ORDA_TEACHER_PRECOMPUTED = 2 } orda_teacher_mode;
/* Reduction (src/config.rs:10-17). */
typedef enum { ORDA_REDUCTION_MEAN = 0, ORDA_REDUCTION_SUM = 1 } orda_reduction;
/* Backend (src/config.rs:19-31); ORDA_BACKEND_HIP takes the Cuda slot. */
typedef enum { ORDA_BACKEND_AUTO = 0, ORDA_BACKEND_CPU = 1, ORDA_BACKEND_HIP = 2 } orda_backend;
/* Profile (src/config.rs:33-42). */
typedef enum { ORDA_PROFILE_BALANCED = 0, ORDA_PROFILE_FAST = 1, ORDA_PROFILE_DEBUG = 2 } orda_profile;

/* A dense row-major matrix: element (r, c) at data + (r*ld + c)*sizeof(dtype).
 * ld == 0 means ld == cols (the reference's Mat, src/mat.rs:10-14). */
typedef struct {
    void *data;
    int64_t rows, cols, ld;
    int32_t dtype;      /* orda_dtype */
    int32_t location;   /* orda_location */
} orda_tensor;

/* src/teacher.rs:11-32. Fields not used by the mode are ignored. */
typedef struct {
    int32_t mode;           /* orda_teacher_mode */
    orda_tensor hidden;     /* Tied [BT,H]; Separate [BT,Ht] */
    orda_tensor weight;     /* Separate [V,Ht] */
    orda_tensor logits;     /* Precomputed [BT,V], fp32 or bf16; beside bf16
                               inputs read in place when 16-byte aligned
                               with ld a multiple of 4 (fp32) or 8 (bf16),
                               else copied into the staging buffer */
} orda_teacher;

/* KernelConfig (src/config.rs:45-63). Option<T> fields carry has_* flags.
 * The reference's CPU path ignores the tuning fields (src/config.rs:3-7); on
 * this GPU path they act as follows:
 *   fast_math       (Profile::Fast, src/config.rs:37-40,93-103) the per-row
 *                   logs and divisions of the row pass use the hardware
 *                   approximations (v_log_f32, v_rcp_f32 then a multiply);
 *                   exponentials are the hardware exp2 in every profile.
 *                   Inputs keep their dtype: fp32 inputs run the fp32 GEMMs,
 *                   and the result matches the reference to the fp32
 *                   tolerance.
 *   profile         ORDA_PROFILE_DEBUG (the precise preset): bf16 inputs are
 *                   widened to fp32 and run the fp32 pipeline (fp32 logits,
 *                   fp32 GEMMs), matching the reference to the fp32
 *                   tolerance. Set by orda_kernel_config_from_profile; the
 *                   reference records the preset only through the fields
 *                   it sets, so this one field is new.
 *   online_softmax  row statistics of Precomputed teacher logits that the
 *                   logits GEMM does not read (fp32 inputs, or logits that
 *                   are unaligned or at a pitch that is not a multiple of 4
 *                   (fp32) or 8 (bf16); with bf16 inputs and a KL term,
 *                   aligned logits are read in the GEMM's epilogue) by the
 *                   online-softmax merge: per 8192-column segment, each
 *                   thread's sums relative to its own maximum, rescaled to
 *                   the larger maximum as they merge, instead of a
 *                   segment-wide maximum first. (The chunk-launcher slot
 *                   takes no KernelConfig; it always uses the max first.)
 *   fp32_grad_weight_accumulation, max_fused_size: accepted and validated;
 *                   grad_W always accumulates in fp32 (the reference's
 *                   output is f32) and the tile widths are fixed. */
typedef struct {
    int32_t online_softmax;
    int32_t fast_math;
    int32_t quantize_grad_weight;
    int32_t stochastic_rounding;
    int32_t fp32_grad_weight_accumulation;
    int32_t has_max_chunks;
    int64_t max_chunks;
    int64_t max_fused_size;
    int32_t has_stochastic_seed;
    uint64_t stochastic_seed;
    int32_t profile;            /* orda_profile the config was made from */
} orda_kernel_config;

/* LossOptions (src/api.rs:25-47). */
typedef struct {
    float student_ce_weight;
    int32_t has_teacher_ce_weight;
    float teacher_ce_weight;
    float kd_weight;
    float temperature;
    int64_t ignore_index;
    float label_smoothing;
    int32_t reduction;          /* orda_reduction */
    int32_t chunk_fixed;        /* 0: ChunkSize::Auto, 1: ChunkSize::Fixed(chunk_rows) */
    int64_t chunk_rows;
    orda_kernel_config config;
    int32_t backend;            /* orda_backend */
} orda_loss_options;

/* DistillationLossOutput (src/api.rs:71-92). The caller owns every buffer:
 * grad_* tensors must be float32 and are written on success.
 * grad_teacher_hidden / grad_teacher_weight are needed exactly when the
 * reference returns Some (api.rs:244-258); has_* report that on return.
 * The remaining tensors are optional diagnostics (data == NULL skips them):
 * per-row losses [BT] (float32; kl includes T², 0 for ignored rows) and the
 * INT8 codes [V,H] / scales [V] of grad_weight when quantize_grad_weight is
 * set (the reference's internal QuantRows, src/quant.rs:66-73). */
typedef struct {
    float loss, student_ce, teacher_ce, kl;
    orda_tensor grad_student_hidden;
    orda_tensor grad_weight;
    orda_tensor grad_teacher_hidden;
    orda_tensor grad_teacher_weight;
    int32_t has_grad_teacher_hidden;
    int32_t has_grad_teacher_weight;
    int64_t chunk_size, num_chunks;      /* ChunkPlan actually used */
    orda_tensor row_nll_student;
    orda_tensor row_nll_teacher;
    orda_tensor row_kl;
    orda_tensor quant_codes;
    orda_tensor quant_scales;
} orda_loss_output;

typedef struct orda_ctx orda_ctx;

/* ---- library ------------------------------------------------------------ */
int32_t orda_abi_version(void);
/* is_available() (src/lib.rs:70-79, src/cuda/mod.rs:51-53): a gfx950 device
 * is visible. */
int32_t orda_is_available(void);

/* ---- options ------------------------------------------------------------ */
/* LossOptions::default() (src/api.rs:49-64). */
void orda_loss_options_default(orda_loss_options *opts);
/* KernelConfig::from_profile (src/config.rs:78-90). */
void orda_kernel_config_from_profile(int32_t profile, orda_kernel_config *cfg);
/* KernelConfig::validate (src/config.rs:106-119). */
int32_t orda_kernel_config_validate(const orda_kernel_config *cfg, char *err, size_t err_len);

/* ---- chunk resolver (src/resolver.rs) ----------------------------------- */
/* resolve_chunk_size (resolver.rs:53-99). has_v/has_max_chunks encode the
 * Option arguments. bt must be > 0. */
int32_t orda_resolve_chunk_size(int64_t bt, int32_t chunk_fixed, int64_t chunk_rows,
                                int32_t has_v, int64_t v, int32_t has_max_chunks,
                                int64_t max_chunks, int64_t *chunk_size, int64_t *num_chunks);
/* chunks_from_raw (resolver.rs:27-36). */
int64_t orda_chunks_from_raw(double raw);
/* default_max_chunks_limit (resolver.rs:103-105). */
int64_t orda_default_max_chunks_limit(int64_t bt);
/* chunk_doubling_schedule (resolver.rs:114-126); returns the length, writes
 * at most cap entries. */
int64_t orda_chunk_doubling_schedule(int64_t bt, int64_t start, int64_t limit, int64_t *out,
                                     int64_t cap);

/* ---- context -------------------------------------------------------------- */
int32_t orda_ctx_create(int32_t device, orda_ctx **out, char *err, size_t err_len);
void orda_ctx_destroy(orda_ctx *ctx);
/* Run on a caller-owned hipStream_t (NULL: the context's own stream, a
 * blocking stream, so it is ordered after work queued on the null stream). */
int32_t orda_ctx_set_stream(orda_ctx *ctx, void *hip_stream);
/* Upper bound, in bytes, on device memory the context may hold (workspace
 * and staging). 0 = no bound. Allocations past it fail like a device OOM,
 * which drives the chunk-doubling retry (resolver.rs:107-126). */
int32_t orda_ctx_set_memory_limit(orda_ctx *ctx, int64_t bytes);
/* Bytes of logits staging the context may use per group of chunks
 * (default 16 GiB). Consecutive chunks up to this size share one logits
 * GEMM, row pass and backward GEMMs; a smaller budget runs more groups, each
 * accumulating into grad_W. The split-K partials of backward GEMMs with
 * fewer output tiles than CUs (at most 256 MB) come on top of it. No
 * counterpart in the reference, which runs one chunk at a time
 * (src/api.rs:263-378). */
int32_t orda_ctx_set_staging_budget(orda_ctx *ctx, int64_t bytes);
/* Release the cached workspace. */
int32_t orda_ctx_trim(orda_ctx *ctx);
/* Device bytes the context's workspace holds (what orda_ctx_set_memory_limit
 * bounds): staged inputs, the logits group, statistics, split-K partials. */
int32_t orda_ctx_workspace_bytes(orda_ctx *ctx, int64_t *bytes);
/* Per-kernel timing with HIP events on the context's stream. */
typedef enum {
    ORDA_KERNEL_GEMM_LOGITS = 0,
    ORDA_KERNEL_ROW_PASS = 1,
    ORDA_KERNEL_GEMM_GRAD_HIDDEN = 2,
    ORDA_KERNEL_GEMM_GRAD_WEIGHT = 3,
    ORDA_KERNEL_QUANT = 4,
    ORDA_KERNEL_OTHER = 5,
    ORDA_KERNEL_KINDS = 6
} orda_kernel_kind;
int32_t orda_ctx_set_timing(orda_ctx *ctx, int32_t enable);
int32_t orda_ctx_get_kernel_time(orda_ctx *ctx, int32_t kind, double *total_ms,
                                 int64_t *launches);
int32_t orda_ctx_reset_kernel_time(orda_ctx *ctx);

/* ---- the loss --------------------------------------------------------------- */
/* distillation_loss(student_hidden, weight, labels, teacher, opts)
 * (src/api.rs:188-422). student_hidden [BT,H], weight [V,H] (f32 or bf16,
 * host or device; all float inputs share one dtype), labels [BT] int64 at
 * labels_location. ctx may be NULL (a temporary context on device 0).
 * Labels on the device are validated on the device and the result is read
 * back with the loss at the call's one synchronisation, so an out-of-range
 * label is reported (with the reference's message, and ahead of any later
 * validation error, as in src/api.rs:104-181) after the kernels have run:
 * the output buffers then hold unspecified values. As in the reference, BT
 * must be > 0 while H, a Separate teacher's width and V may be 0 (V = 0
 * leaves only ignored labels: every term and gradient is 0). */
int32_t orda_distillation_loss(orda_ctx *ctx, const orda_tensor *student_hidden,
                               const orda_tensor *weight, const int64_t *labels,
                               int64_t n_labels, int32_t labels_location,
                               const orda_teacher *teacher, const orda_loss_options *opts,
                               orda_loss_output *out, char *err, size_t err_len);

/* ---- the GPU row-kernel slot (src/cuda/launch.rs:51-158) ----------------- */
/* kl_ce_on_logits_chunk: the KL kernel then the CE kernel over a prepared
 * logits_chunk [2*n_rows, V] (student rows first), with the outputs of
 * KlCeChunkOutput (launch.rs:28-37) in separate buffers: grad_kl_student
 * [n_rows,V], kl_per_row [n_rows], grad_ce [grid_rows,V], ce_loss
 * [grid_rows], grid_rows = student_only ? n_rows : 2*n_rows. Any V (no
 * V % BLOCK requirement); a device logits_chunk is read in place at any
 * pitch. Tensors may live on host or device; targets are int32 like the
 * reference's launcher. */
int32_t orda_kl_ce_on_logits_chunk(orda_ctx *ctx, const orda_tensor *logits_chunk,
                                   const int32_t *targets, int32_t targets_location,
                                   int64_t n_rows, float inv_t, float kl_grad_scale, float t_sq,
                                   float student_ce_weight, float teacher_ce_weight,
                                   float label_smoothing, int32_t ignore_index,
                                   int32_t student_only, int32_t compute_kl,
                                   orda_tensor *grad_kl_student, orda_tensor *kl_per_row,
                                   orda_tensor *grad_ce, orda_tensor *ce_loss, char *err,
                                   size_t err_len);

/* The same slot with no device allocation: no counterpart in the reference.
 * For callers that cannot allocate during the call (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). ctx is
 * required; every tensor and the targets must be on the device; n_rows is at
 * most 32768 (ORDA_ERR_INVALID beyond). The per-row scratch is one 1.75 MiB
 * array per GPU held until the process ends and shared by every call on that
 * GPU: calls that overlap on one GPU race. On a stream under HIP graph
 * capture (the context's stream, orda_ctx_set_stream) the call records its
 * kernels and returns without waiting or timing; every replay of the graph
 * uses the same per-GPU scratch, so a replay overlapping another call or
 * replay on that GPU races too. Otherwise the call is synchronous. */
int32_t orda_kl_ce_on_logits_chunk_noalloc(orda_ctx *ctx, const orda_tensor *logits_chunk,
                                           const int32_t *targets, int32_t targets_location,
                                           int64_t n_rows, float inv_t, float kl_grad_scale,
                                           float t_sq, float student_ce_weight,
                                           float teacher_ce_weight, float label_smoothing,
                                           int32_t ignore_index, int32_t student_only,
                                           int32_t compute_kl, orda_tensor *grad_kl_student,
                                           orda_tensor *kl_per_row, orda_tensor *grad_ce,
                                           orda_tensor *ce_loss, char *err, size_t err_len);

/* ---- INT8 row-wise quantization (src/quant.rs:96-202) --------------------- */
/* quantize_grad_w followed by dequantize_grad_w(·, grad_output): m [rows,cols]
 * float32; out receives the dequantized matrix (may alias m) with the rows
 * named by non-ignored in-range targets kept exact; codes (int8 [rows,cols])
 * and scales (float32 [rows]) are optional. stochastic=1 uses the SplitMix64
 * stream of Rng::new(seed), bit-exact. */
int32_t orda_quant_rows_int8(orda_ctx *ctx, const orda_tensor *m, const int64_t *targets,
                             int64_t n_targets, int32_t targets_location, int64_t ignore_index,
                             int32_t stochastic, uint64_t seed, float grad_output,
                             orda_tensor *out, orda_tensor *codes, orda_tensor *scales, char *err,
                             size_t err_len);

#ifdef __cplusplus
}
#endif
#endif /* ORDA_ORDA_H */
