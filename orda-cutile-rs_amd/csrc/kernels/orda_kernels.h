// orda_kernels.h — launchers for the gfx950 kernels of the fused
// cross-entropy + forward-KL distillation loss. Internal to liborda_hip.so;
// the public surface is include/orda/orda.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace orda {

enum class DType : int { F32 = 0, BF16 = 1 };

inline int dtype_size(DType t) { return t == DType::F32 ? 4 : 2; }

// ---------------------------------------------------------------- GEMM
// One launch computes up to two problems that share M, N, K and pitches:
//   C_p[M,N] (op)= alpha * A_p · B_p
// A is K-major ([M][lda], element (m,k) at m*lda+k). B is K-major ([N][ldb],
// (n,k) at n*ldb+k) for the Logits epilogue and N-major ([K][ldb], (n,k) at
// k*ldb+n) for Store/Accum; other layouts are rejected.
// Pitches are in elements and must be multiples of 8; base pointers 16-byte
// aligned. Out-of-range rows/columns/K are zero-filled on load and masked on
// store.
enum class GemmEpilogue : int {
  StoreF32 = 0,    // C = alpha*acc                       (C is float)
  AccumF32 = 1,    // C = alpha*(C + acc)                 (C is float)
  Logits = 2,      // C = acc stored in the logits dtype, plus per-row
                   // partial softmax statistics for every 256-column tile
  LogitsTeacher = 3,   // internal: a Logits product with fp32 lg.teacher_logits
  LogitsTeacher16 = 4, // internal: a Logits product with bf16 lg.teacher_logits
                       // (launch_gemm selects it; callers pass Logits)
};

struct GemmProblem {
  const void* a;
  const void* b;
  void* c;
};

struct LogitStatsArgs {
  // stats[(p*M + m) * stats_ld + n_tile] = {max, Σe^(x-max), Σe^((x-max)/T), Σx}
  float4* stats;
  int64_t stats_ld;       // in float4 units, >= ceil(N/256)
  float* xy;              // xy[p*M + m] = fp32 logit at the row's label column
  const int64_t* labels;  // label of row m of either problem = labels[m]
  int64_t ignore_index;
  float inv_t;            // 1/T
  // Paired rows (one problem, bf16): pair_rows > 0 means the GEMM's rows
  // are student and teacher rows in blocks of 16 (student rows 16b..16b+15
  // as rows 32b..32b+15, the same teacher rows as 32b+16..32b+31),
  // M = 2*round16(pair_rows), read in place: student rows from prob[0].a,
  // teacher rows from pair_teacher, both with pitch lda. Student row r is
  // stored as row r of C / stats / xy, teacher row r as row pair_rows + r, and
  //   cross[r * stats_ld + n_tile] = {Σ e^((t_j - max_t)/T) · (t_j - s_j),
  //                                  Σ (e^((s_j - max_t)/T) - e^((t_j - max_t)/T))}
  // over the tile's columns, max_t being the teacher row's tile maximum; the
  // second sum forms each element's difference before adding it (NaN where
  // the student's maximum exceeds the teacher's by more than 64·T·ln 2 in a
  // half tile: the row pass then uses the two rows' own sums).
  int64_t pair_rows;
  float2* cross;
  const void* pair_teacher;
  // bf16 logits (required then): each logit is stored relative to the
  // maximum m of its 128-column half tile k (k = 2*n_tile + h), in log2
  // units, C = bf16((x - m) * log2(e)), so the bf16 rounding error of a
  // stored logit scales with its distance below that maximum, not with its
  // magnitude. m goes to hmax[r * hmax_ld + 2*k + side], r the row within
  // its block (student rows side 0, teacher rows side 1: the paired rows,
  // or problem p as side p; a teacher-only launch passes hmax + 1), so a
  // row pair's two maxima of one half are adjacent. hmax_ld >= 4*ceil(N/256),
  // even. fp32 logits are stored as they are.
  float* hmax;
  int64_t hmax_ld;
  // Teacher logits beside the product (one problem, bf16 inputs and bf16
  // logits, no paired rows): teacher_logits[r * teacher_ld + n], of type
  // teacher_type (fp32: 16-byte aligned, teacher_ld a multiple of 4; bf16:
  // 8-byte aligned, teacher_ld a multiple of 4), is the teacher logit of the
  // product's row r. The epilogue reads the tile's teacher logits and writes,
  // as for paired rows, the teacher rows' statistics (stats row M + r), label
  // logits (xy[M + r]) and the two KL sums (cross[r]); the teacher logits are
  // not stored, and hmax holds the student rows' maxima (side 0) only.
  const void* teacher_logits;
  int64_t teacher_ld;
  DType teacher_type;
};

struct GemmArgs {
  int nprob;              // 1 or 2
  GemmProblem prob[2];
  int64_t M, N, K;
  int64_t lda, ldb, ldc;
  bool a_kmajor, b_kmajor;
  DType in_type;          // dtype of A and B
  DType logits_type;      // dtype of C for the Logits epilogue
  GemmEpilogue epi;
  float alpha;
  // When set, the epilogue scales by alpha * *alpha_ptr (a device value, e.g.
  // the deferred mean computed on the device by launch_label_check).
  const float* alpha_ptr;
  int group_m;            // M-tiles per raster group (L2 reuse of B)
  // Rounds spanning all N-tiles, the XCDs of a round on the same operand
  // strips (launch_gemm picks the blocks; shapes it cannot fill: ignored).
  bool share_rounds;
  // Set by launch_gemm when share_rounds applies: each XCD takes an
  // sh_a (M) x sh_b (N) block of a round, sh_xn XCDs side by side in N.
  int sh_a, sh_b, sh_xn;
  // Store/Accum only: C is stored transposed, element (m, n) of the
  // product at C[n*ldc + m] (C is [N][ldc]).
  bool c_trans;
  LogitStatsArgs lg;
  // Split-K workspace for Store/Accum GEMMs with fewer tiles than CUs: when
  // given (gemm_split_bytes(g) bytes), launch_gemm splits K over several
  // workgroups per tile and sums their fp32 partials in a fixed order.
  float* split_ws;
  int64_t split_ws_bytes;
  // Set by launch_gemm for the split launch: K range s*split_len.. of the
  // workgroups of split s, partials of split s at split_ws + s*split_stride.
  int split_k;
  int64_t split_len, split_stride;
  // With split_ws: the split launch writes the partials only and skips the
  // reduction (the caller reduces them, e.g. launch_row_stats with
  // src_splits). Only for products gemm_split_plan splits whole.
  bool partials_only;
};

hipError_t launch_gemm(const GemmArgs& g, hipStream_t stream);
// How launch_gemm splits K for g when it splits the whole product (no part
// in whole rounds) and the workspace suffices: splits > 1, split s's
// partial of problem p at split_ws + s*stride + p*rows*ldp (rows x ldp, in
// C's orientation, fp32); otherwise splits = 0.
struct GemmSplit {
  int splits;
  int64_t stride, ldp;
};
GemmSplit gemm_split_plan(const GemmArgs& g);
// Transposed staging of hidden rows for a K-major operand over rows:
//   dst[c*ldd + r]          = a[r*lda + c]   (r < rows)
//   dst[c*ldd + rows + r]   = b[r*ldb + c]   (r < rows, when b is set)
// for c < cols; ldd >= rows (or 2*rows), a multiple of 8.
hipError_t launch_transpose_rows(const void* a, int64_t lda, const void* b, int64_t ldb,
                                 int64_t rows, int64_t cols, void* dst, int64_t ldd, DType t,
                                 hipStream_t stream);
// Workspace bytes launch_gemm uses to split K for this GEMM (0: no split).
int64_t gemm_split_bytes(const GemmArgs& g);
// Whether launch_gemm runs this Store/Accum GEMM on 128 x 128 tiles (fp32
// inputs, at most 64 tiles of 256 x 256): splits and partials as given by
// gemm_split_plan / gemm_split_bytes.
bool gemm_small_tiles(const GemmArgs& g);
int64_t gemm_stat_tiles(int64_t n);   // ceil(n/256)

// ---------------------------------------------------------------- row pass
// Fused KL + CE + merge over row pairs of a logits chunk, gradient written
// in place (or to split outputs for the chunk-launcher entry point).
struct RowPassArgs {
  DType ltype;             // logits storage dtype
  void* student;           // row r of the student block at student + r*ld
  void* teacher;           // row r of the teacher block (may be null)
  int64_t ld;              // pitch (elements) of both blocks, multiple of 8
  int64_t ld_t;            // teacher pitch when it differs (read-only teacher
                           // rows, e.g. Precomputed logits in place); 0: ld
  int64_t n_rows;          // row pairs
  int64_t v;               // vocabulary
  const float4* stats_s;   // per-row partial stats of student rows
  const float4* stats_t;   // ... of teacher rows (may be null)
  int64_t stats_ld;        // float4 entries per row
  int64_t stats_tiles;     // entries filled per student row
  int64_t stats_tiles_t;   // entries filled per teacher row
  const float* xy_s;       // fp32 target logit of each student row
  const float* xy_t;
  const int64_t* labels;   // [n_rows]
  int64_t ignore_index;
  float w_s, w_t, kd, temperature, label_smoothing;
  bool teacher_ce;         // w_t > 0: compute teacher CE loss
  bool teacher_grad;       // write the teacher CE gradient into teacher rows
  bool kl;                 // kd > 0: KL loss and student KL gradient
  float* row_nll_s;        // [n_rows] outputs (never null)
  float* row_nll_t;
  float* row_kl;           // KL_row * T^2 (T^2 in f32), 0 when ignored
  // Per-tile KL partials of the teacher rows from a paired logits GEMM
  // (LogitStatsArgs::cross, same pitch as the stats), or null: then the
  // pass accumulates the KL sums from the logits it reads.
  const float2* cross;
  // Scratch of n_rows float4 for the chunked passes: over paired bf16
  // logits (cross set, gradient in place), and over fp32 logits (cross
  // null); may be null (then the row-per-workgroup pass runs).
  float4* row_consts;
  // fp32 chunked pass with a KL term: n_rows * row_pass_kl_blocks(v)
  // float4, each column block's share of the row's three KL sums.
  float4* kl_part;
  // bf16 logits stored relative to their half-tile maxima by the logits
  // GEMM (LogitStatsArgs::hmax): half k of row r has its maximum at
  // hmax_s[r*hmax_ld + 2*k] (student) and hmax_t[r*hmax_ld + 2*k]
  // (teacher, hmax_s + 1 for the GEMM's paired layout), or null for rows
  // stored as they are (Precomputed teacher logits, the chunk-launcher
  // entry point). The chunked pass over paired bf16 rows runs only with
  // them, interleaved.
  const float* hmax_s;
  const float* hmax_t;
  int64_t hmax_ld;
  // Gradient rows: written at grad_s/grad_t + r*ld in gtype. Null grad_s
  // means in place (gtype == ltype).
  void* grad_s;
  void* grad_t;
  DType gtype;
  // Split mode (chunk-launcher entry point): gradients go to separate
  // buffers instead of overwriting the logits, and are not merged.
  bool split;
  float* grad_kl;          // [n_rows][v] (split mode)
  float* grad_ce;          // [n_rows or 2*n_rows][v] (split mode)
  float* ce_loss;          // [n_rows or 2*n_rows] (split mode)
  float kl_grad_scale;     // split mode: KL gradient scale as given
  float t_sq;              // split mode: T^2 as given
  float inv_t;             // split mode: 1/T as given
  bool student_only;       // split mode: CE over student rows only
  bool fast_math;          // per-row logs and divisions by the hardware approximations
  // The teacher rows are logits as they are, fp32 (Precomputed teacher
  // logits, or a Separate teacher's) or bf16 (teacher_bf16: Precomputed
  // teacher logits), read in place at pitch ld_t (a teacher gradient goes to
  // the bf16 rows grad_t at pitch ld), beside bf16 student rows relative to
  // their half-tile maxima, with the paired KL sums in cross
  // (LogitStatsArgs::teacher_logits).
  bool teacher_f32;
  bool teacher_bf16;
};

hipError_t launch_row_pass(const RowPassArgs& a, hipStream_t stream);
// float4 entries per row of RowPassArgs::kl_part (ceil(v/512)).
int64_t row_pass_kl_blocks(int64_t v);

// Per-row statistics of rows that were not produced by the GEMM (Precomputed
// teacher logits, the chunk-launcher entry point). Reads src (fp32 or bf16,
// any pitch), writes one stats entry per row and the fp32 target logit, and
// optionally copies the row into dst (logits dtype, pitch ldd, zero padding
// up to the next multiple of 8).
struct RowStatsArgs {
  DType src_type;
  const void* src;
  int64_t lds;
  DType dst_type;
  void* dst;               // may be null
  int64_t ldd;
  int64_t n_rows, v;
  float4* stats;           // stats[r * stats_ld]
  int64_t stats_ld;
  float* xy;
  const int64_t* labels;   // may be null (then xy is not written)
  int64_t label_rows;      // > 0: row r's label is labels[r % label_rows]
  int64_t ignore_index;
  float inv_t;
  bool online;             // one online pass; else a max pass, then a sum pass
  // With segmented (and !online): one workgroup per 8192-column segment of a
  // row, held in registers for both passes (one read), statistics of
  // segment s at stats[r * stats_ld + s]; stats_ld >= row_stats_segments(v).
  bool segmented;
  // segmented fp32 rows only: src holds src_splits split-K partials, split s
  // at src + s*src_split_stride; each element is their sum in split order
  // (the reduction launch_gemm would run), written to dst.
  int src_splits;
  int64_t src_split_stride;
};
hipError_t launch_row_stats(const RowStatsArgs& a, hipStream_t stream);
int64_t row_stats_segments(int64_t v);

// ---------------------------------------------------------------- reductions
// Sums per-row losses into the reference's scalars (api.rs:401-405):
// out[0..3] = loss, student_ce, teacher_ce, kl (as float).
struct FinalizeArgs {
  const float* row_nll_s;
  const float* row_nll_t;
  const float* row_kl;
  int64_t bt;
  int64_t chunk_size;      // KL is summed per chunk then rounded to f32
  float w_s, w_t, kd;
  float mean_scale;
  const float* mean_scale_ptr;   // when set, *mean_scale_ptr replaces mean_scale
  float* out;              // 4 floats
};
hipError_t launch_finalize(const FinalizeArgs& a, hipStream_t stream);

// ---------------------------------------------------------------- INT8 quant
struct QuantArgs {
  const float* src;        // [rows][cols]
  int64_t lds;
  float* dst;              // dequantized output (may equal src)
  int64_t ldd;
  int8_t* codes;           // may be null
  int64_t ldq;
  float* scales;           // may be null
  const uint8_t* keep_exact;  // per-row flag: copy the source row exactly
  int64_t rows, cols;
  bool stochastic;
  uint64_t seed;
  float grad_output;
};
hipError_t launch_quant(const QuantArgs& a, hipStream_t stream);

// Label validation on the device (src/api.rs:125-133) and the deferred-mean
// scale (src/api.rs:225-230): n_valid counts labels != ignore_index; the
// first label (lowest index) that is neither ignore_index nor in [0, v) is
// reported with its value (bad_index -1: none); mean_scale =
// 1 / max(n_valid, 1) as f32 for the Mean reduction, 1 for Sum.
struct LabelStatus {
  int64_t n_valid;
  int64_t bad_index;
  int64_t bad_label;
  float mean_scale;
  float pad;
};
hipError_t launch_label_check(const int64_t* labels, int64_t n, int64_t v, int64_t ignore_index,
                              bool mean, LabelStatus* out, hipStream_t stream);

// out64[i] = in32[i] for i < n, and zero[i] = 0 for i < n_zero (the targets of
// the chunk-launcher entry point widened to the kernels' int64 labels).
hipError_t launch_widen_targets(const int32_t* in32, int64_t n, int64_t* out64, float* zero,
                                int64_t n_zero, hipStream_t stream);

// keep[labels[i]] = 1 for every in-range, non-ignored label.
hipError_t launch_mark_targets(const int64_t* labels, int64_t n, int64_t ignore_index,
                               uint8_t* keep, int64_t rows, hipStream_t stream);

// Strided 2-D copy with dtype conversion (f32<->bf16) and zero padding of
// columns [cols, ldd).
hipError_t launch_convert_rows(DType src_t, const void* src, int64_t lds, DType dst_t,
                               void* dst, int64_t ldd, int64_t rows, int64_t cols,
                               hipStream_t stream);

}  // namespace orda
