/* C++ mirror of the reference crate's public API (src/lib.rs:53-79) over the
 * C ABI of liborda_hip.so (orda/orda.h): the same type names, fields,
 * defaults and argument meanings, so that C++ code reads like a caller of the
 * crate. Header-only (C++17); link with -lorda_hip.
 *
 * Errors: where the crate returns Err(String) (src/api.rs:188-194,
 * src/config.rs:106-119) or asserts (src/resolver.rs:53-59, src/mat.rs:17-23),
 * these functions throw: orda::Error carries the reference's message in
 * what() and the orda_status code in status(); Mat::from_vec throws
 * std::invalid_argument. Every computation runs on the GPU; there is no host
 * fallback (Backend::Cpu is refused, as the C ABI documents). */
#ifndef ORDA_ORDA_HPP
#define ORDA_ORDA_HPP

#include <cstddef>
#include <cstdint>
#include <optional>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "orda/orda.h"

namespace orda {

class Error : public std::runtime_error {
 public:
  Error(int32_t status, const std::string& message)
      : std::runtime_error(message), status_(status) {}
  int32_t status() const noexcept { return status_; }

 private:
  int32_t status_;
};

namespace detail {
inline void check(int32_t rc, const char* err) {
  if (rc != ORDA_OK) throw Error(rc, err);
}
}  // namespace detail

/* Mat (src/mat.rs:8-57): a dense row-major f32 matrix on the host. */
struct Mat {
  size_t rows = 0;
  size_t cols = 0;
  std::vector<float> data;

  /* src/mat.rs:17-23 (the reference panics on a length mismatch) */
  static Mat from_vec(size_t rows, size_t cols, std::vector<float> data) {
    if (data.size() != rows * cols)
      throw std::invalid_argument("data length must equal rows*cols");
    Mat m;
    m.rows = rows;
    m.cols = cols;
    m.data = std::move(data);
    return m;
  }
  static Mat zeros(size_t rows, size_t cols) {
    return from_vec(rows, cols, std::vector<float>(rows * cols, 0.0f));
  }
  std::pair<size_t, size_t> shape() const { return {rows, cols}; }
  const float* row(size_t r) const { return data.data() + r * cols; }
  float* row_mut(size_t r) { return data.data() + r * cols; }
  float get(size_t r, size_t c) const { return data[r * cols + c]; }
  bool operator==(const Mat& o) const {
    return rows == o.rows && cols == o.cols && data == o.data;
  }

  /* The C ABI's view of this matrix (host memory, f32). */
  orda_tensor view() const {
    return orda_tensor{const_cast<float*>(data.data()), static_cast<int64_t>(rows),
                       static_cast<int64_t>(cols), 0, ORDA_F32, ORDA_HOST};
  }
};

/* src/config.rs:10-42. Backend::Hip takes the place of Backend::Cuda. */
enum class Reduction : int32_t { Mean = ORDA_REDUCTION_MEAN, Sum = ORDA_REDUCTION_SUM };
enum class Backend : int32_t { Auto = ORDA_BACKEND_AUTO, Cpu = ORDA_BACKEND_CPU, Hip = ORDA_BACKEND_HIP };
enum class Profile : int32_t {
  Balanced = ORDA_PROFILE_BALANCED,
  Fast = ORDA_PROFILE_FAST,
  Debug = ORDA_PROFILE_DEBUG
};

constexpr size_t DEFAULT_MAX_FUSED_SIZE = 65536 / 2;   // src/config.rs:65

/* src/config.rs:122-125 */
inline bool is_power_of_two(size_t value) { return value > 0 && (value & (value - 1)) == 0; }

/* KernelConfig (src/config.rs:45-121). `profile` records the preset the
 * config was made from: on this GPU path Profile::Debug widens bf16 inputs to
 * the fp32 pipeline (the reference keeps a preset only through the fields it
 * sets). */
struct KernelConfig {
  bool online_softmax = false;
  bool fast_math = false;
  bool quantize_grad_weight = false;
  bool stochastic_rounding = false;
  bool fp32_grad_weight_accumulation = false;
  std::optional<size_t> max_chunks;
  size_t max_fused_size = DEFAULT_MAX_FUSED_SIZE;
  std::optional<uint64_t> stochastic_seed;
  Profile profile = Profile::Balanced;

  /* src/config.rs:78-90 */
  static KernelConfig from_profile(Profile p) {
    orda_kernel_config c{};
    orda_kernel_config_from_profile(static_cast<int32_t>(p), &c);
    return from_c(c);
  }
  bool fast_math_exp() const { return fast_math; }
  bool fast_math_log() const { return fast_math; }
  bool fast_math_mul() const { return fast_math; }
  /* src/config.rs:106-119 */
  void validate() const {
    const orda_kernel_config c = to_c();
    char err[512] = {0};
    detail::check(orda_kernel_config_validate(&c, err, sizeof err), err);
  }

  orda_kernel_config to_c() const {
    orda_kernel_config c{};
    c.online_softmax = online_softmax;
    c.fast_math = fast_math;
    c.quantize_grad_weight = quantize_grad_weight;
    c.stochastic_rounding = stochastic_rounding;
    c.fp32_grad_weight_accumulation = fp32_grad_weight_accumulation;
    c.has_max_chunks = max_chunks.has_value();
    c.max_chunks = static_cast<int64_t>(max_chunks.value_or(0));
    c.max_fused_size = static_cast<int64_t>(max_fused_size);
    c.has_stochastic_seed = stochastic_seed.has_value();
    c.stochastic_seed = stochastic_seed.value_or(0);
    c.profile = static_cast<int32_t>(profile);
    return c;
  }
  static KernelConfig from_c(const orda_kernel_config& c) {
    KernelConfig k;
    k.online_softmax = c.online_softmax != 0;
    k.fast_math = c.fast_math != 0;
    k.quantize_grad_weight = c.quantize_grad_weight != 0;
    k.stochastic_rounding = c.stochastic_rounding != 0;
    k.fp32_grad_weight_accumulation = c.fp32_grad_weight_accumulation != 0;
    if (c.has_max_chunks) k.max_chunks = static_cast<size_t>(c.max_chunks);
    k.max_fused_size = static_cast<size_t>(c.max_fused_size);
    if (c.has_stochastic_seed) k.stochastic_seed = c.stochastic_seed;
    k.profile = static_cast<Profile>(c.profile);
    return k;
  }
};

/* ChunkSize (src/resolver.rs:9-17) */
struct ChunkSize {
  bool is_auto = true;
  size_t fixed = 0;
  static ChunkSize Auto() { return ChunkSize{}; }
  static ChunkSize Fixed(size_t rows) { return ChunkSize{false, rows}; }
  bool operator==(const ChunkSize& o) const {
    return is_auto == o.is_auto && (is_auto || fixed == o.fixed);
  }
};

/* ChunkPlan (src/resolver.rs:38-45) */
struct ChunkPlan {
  size_t chunk_size = 0;
  size_t num_chunks = 0;
  bool operator==(const ChunkPlan& o) const {
    return chunk_size == o.chunk_size && num_chunks == o.num_chunks;
  }
};

/* src/resolver.rs:19-22 */
inline size_t ceil_div(size_t a, size_t b) { return a / b + (a % b != 0); }

/* src/resolver.rs:27-36 */
inline size_t chunks_from_raw(double raw) {
  return static_cast<size_t>(orda_chunks_from_raw(raw));
}

/* src/resolver.rs:53-99 (bt must be > 0: the reference asserts it) */
inline ChunkPlan resolve_chunk_size(size_t bt, ChunkSize chunk_size, std::optional<size_t> v,
                                    std::optional<size_t> max_chunks) {
  int64_t cs = 0, nc = 0;
  const int32_t rc = orda_resolve_chunk_size(
      static_cast<int64_t>(bt), chunk_size.is_auto ? 0 : 1, static_cast<int64_t>(chunk_size.fixed),
      v.has_value(), static_cast<int64_t>(v.value_or(0)), max_chunks.has_value(),
      static_cast<int64_t>(max_chunks.value_or(0)), &cs, &nc);
  if (rc != ORDA_OK) throw Error(rc, "BT (batch * sequence length) must be > 0");
  return ChunkPlan{static_cast<size_t>(cs), static_cast<size_t>(nc)};
}

/* src/resolver.rs:103-105 */
inline size_t default_max_chunks_limit(size_t bt) {
  return static_cast<size_t>(orda_default_max_chunks_limit(static_cast<int64_t>(bt)));
}

/* src/resolver.rs:114-126 */
inline std::vector<size_t> chunk_doubling_schedule(size_t bt, size_t start, size_t limit) {
  const int64_t n = orda_chunk_doubling_schedule(static_cast<int64_t>(bt), static_cast<int64_t>(start),
                                                 static_cast<int64_t>(limit), nullptr, 0);
  std::vector<int64_t> tmp(static_cast<size_t>(n > 0 ? n : 0));
  orda_chunk_doubling_schedule(static_cast<int64_t>(bt), static_cast<int64_t>(start),
                               static_cast<int64_t>(limit), tmp.data(), n);
  return std::vector<size_t>(tmp.begin(), tmp.end());
}

/* TeacherMode and Teacher (src/teacher.rs:11-60) */
enum class TeacherMode : int32_t {
  Tied = ORDA_TEACHER_TIED,
  Separate = ORDA_TEACHER_SEPARATE,
  Precomputed = ORDA_TEACHER_PRECOMPUTED
};

class Teacher {
 public:
  static Teacher Tied(Mat hidden) { return Teacher(TeacherMode::Tied, std::move(hidden), {}, {}); }
  static Teacher Separate(Mat hidden, Mat weight) {
    return Teacher(TeacherMode::Separate, std::move(hidden), std::move(weight), {});
  }
  static Teacher Precomputed(Mat logits) {
    return Teacher(TeacherMode::Precomputed, {}, {}, std::move(logits));
  }
  TeacherMode mode() const { return mode_; }
  float default_teacher_ce_weight() const { return mode_ == TeacherMode::Tied ? 1.0f : 0.0f; }
  const Mat& hidden() const { return hidden_; }
  const Mat& weight() const { return weight_; }
  const Mat& logits() const { return logits_; }

  orda_teacher to_c() const {
    orda_teacher t{};
    t.mode = static_cast<int32_t>(mode_);
    if (mode_ != TeacherMode::Precomputed) t.hidden = hidden_.view();
    if (mode_ == TeacherMode::Separate) t.weight = weight_.view();
    if (mode_ == TeacherMode::Precomputed) t.logits = logits_.view();
    return t;
  }

 private:
  Teacher(TeacherMode m, Mat h, Mat w, Mat l)
      : mode_(m), hidden_(std::move(h)), weight_(std::move(w)), logits_(std::move(l)) {}
  TeacherMode mode_;
  Mat hidden_, weight_, logits_;
};

/* LossOptions and its Default (src/api.rs:25-64) */
struct LossOptions {
  float student_ce_weight = 1.0f;
  std::optional<float> teacher_ce_weight;
  float kd_weight = 0.0f;
  float temperature = 1.0f;
  int64_t ignore_index = -100;
  float label_smoothing = 0.0f;
  Reduction reduction = Reduction::Mean;
  ChunkSize chunk_size = ChunkSize::Auto();
  KernelConfig config;
  Backend backend = Backend::Auto;

  orda_loss_options to_c() const {
    orda_loss_options o{};
    o.student_ce_weight = student_ce_weight;
    o.has_teacher_ce_weight = teacher_ce_weight.has_value();
    o.teacher_ce_weight = teacher_ce_weight.value_or(0.0f);
    o.kd_weight = kd_weight;
    o.temperature = temperature;
    o.ignore_index = ignore_index;
    o.label_smoothing = label_smoothing;
    o.reduction = static_cast<int32_t>(reduction);
    o.chunk_fixed = chunk_size.is_auto ? 0 : 1;
    o.chunk_rows = static_cast<int64_t>(chunk_size.fixed);
    o.config = config.to_c();
    o.backend = static_cast<int32_t>(backend);
    return o;
  }
};

/* DistillationLossOutput (src/api.rs:66-92) */
struct DistillationLossOutput {
  float loss = 0.0f;
  float student_ce = 0.0f;
  float teacher_ce = 0.0f;
  float kl = 0.0f;
  Mat grad_student_hidden;
  Mat grad_weight;
  std::optional<Mat> grad_teacher_hidden;
  std::optional<Mat> grad_teacher_weight;
  ChunkPlan chunk_plan;
};

/* is_available() (src/lib.rs:70-79): a gfx950 device is visible. */
inline bool is_available() { return orda_is_available() != 0; }

/* A device context (orda_ctx): its stream, workspace and memory bound. The
 * functions below also take none, running on a temporary context on device 0
 * as the crate's free functions do. */
class Context {
 public:
  explicit Context(int32_t device = 0) {
    char err[512] = {0};
    detail::check(orda_ctx_create(device, &ctx_, err, sizeof err), err);
  }
  ~Context() { orda_ctx_destroy(ctx_); }
  Context(const Context&) = delete;
  Context& operator=(const Context&) = delete;
  Context(Context&& o) noexcept : ctx_(std::exchange(o.ctx_, nullptr)) {}
  Context& operator=(Context&& o) noexcept {
    std::swap(ctx_, o.ctx_);
    return *this;
  }
  orda_ctx* get() const { return ctx_; }
  /* a caller-owned hipStream_t, or nullptr for the context's own stream */
  void set_stream(void* hip_stream) { orda_ctx_set_stream(ctx_, hip_stream); }
  void set_memory_limit(int64_t bytes) {
    detail::check(orda_ctx_set_memory_limit(ctx_, bytes), "memory limit must be >= 0");
  }
  void set_staging_budget(int64_t bytes) {
    detail::check(orda_ctx_set_staging_budget(ctx_, bytes), "staging budget must be positive");
  }
  void trim() { orda_ctx_trim(ctx_); }

 private:
  orda_ctx* ctx_ = nullptr;
};

/* distillation_loss (src/api.rs:188-422) on host matrices, like the crate:
 * the gradients come back as new host matrices, grad_teacher_hidden and
 * grad_teacher_weight present exactly where the reference returns Some
 * (src/api.rs:244-258). */
inline DistillationLossOutput distillation_loss(Context* ctx, const Mat& student_hidden,
                                                const Mat& weight,
                                                const std::vector<int64_t>& labels,
                                                const Teacher& teacher, const LossOptions& opts) {
  const float w_t = opts.teacher_ce_weight.value_or(teacher.default_teacher_ce_weight());
  const bool want_ght = w_t > 0.0f && teacher.mode() != TeacherMode::Precomputed;
  const bool want_gwt = w_t > 0.0f && teacher.mode() == TeacherMode::Separate;
  DistillationLossOutput r;
  r.grad_student_hidden = Mat::zeros(student_hidden.rows, student_hidden.cols);
  r.grad_weight = Mat::zeros(weight.rows, weight.cols);
  if (want_ght) r.grad_teacher_hidden = Mat::zeros(teacher.hidden().rows, teacher.hidden().cols);
  if (want_gwt) r.grad_teacher_weight = Mat::zeros(teacher.weight().rows, teacher.weight().cols);

  orda_loss_output out{};
  out.grad_student_hidden = r.grad_student_hidden.view();
  out.grad_weight = r.grad_weight.view();
  if (want_ght) out.grad_teacher_hidden = r.grad_teacher_hidden->view();
  if (want_gwt) out.grad_teacher_weight = r.grad_teacher_weight->view();
  const orda_tensor s = student_hidden.view(), w = weight.view();
  const orda_teacher t = teacher.to_c();
  const orda_loss_options o = opts.to_c();
  char err[1024] = {0};
  detail::check(orda_distillation_loss(ctx ? ctx->get() : nullptr, &s, &w, labels.data(),
                                       static_cast<int64_t>(labels.size()), ORDA_HOST, &t, &o,
                                       &out, err, sizeof err),
                err);
  r.loss = out.loss;
  r.student_ce = out.student_ce;
  r.teacher_ce = out.teacher_ce;
  r.kl = out.kl;
  if (!out.has_grad_teacher_hidden) r.grad_teacher_hidden.reset();
  if (!out.has_grad_teacher_weight) r.grad_teacher_weight.reset();
  r.chunk_plan = ChunkPlan{static_cast<size_t>(out.chunk_size), static_cast<size_t>(out.num_chunks)};
  return r;
}

inline DistillationLossOutput distillation_loss(const Mat& student_hidden, const Mat& weight,
                                                const std::vector<int64_t>& labels,
                                                const Teacher& teacher, const LossOptions& opts) {
  return distillation_loss(nullptr, student_hidden, weight, labels, teacher, opts);
}

/* KlCeChunkOutput and kl_ce_on_logits_chunk (src/cuda/launch.rs:27-158):
 * the KL then the CE row kernels over a prepared [2*n_rows, V] logits_chunk
 * (student rows first). `block` is accepted for the reference's signature;
 * any V works here (the reference requires V % block == 0). */
struct KlCeChunkOutput {
  std::vector<float> grad_kl_student;   // [n_rows, V]
  std::vector<float> kl_per_row;        // [n_rows]
  std::vector<float> grad_ce;           // [grid_rows, V]
  std::vector<float> ce_loss;           // [grid_rows]
};

inline KlCeChunkOutput kl_ce_on_logits_chunk(const std::vector<float>& logits_chunk,
                                             const std::vector<int32_t>& targets, size_t n_rows,
                                             size_t v, size_t /*block*/, float inv_t,
                                             float kl_grad_scale, float t_sq,
                                             float student_ce_weight, float teacher_ce_weight,
                                             float label_smoothing, int32_t ignore_index,
                                             bool student_only, bool compute_kl,
                                             Context* ctx = nullptr) {
  if (logits_chunk.size() != 2 * n_rows * v)
    throw std::invalid_argument("logits_chunk must be [2*n_rows, V]");
  if (targets.size() != n_rows) throw std::invalid_argument("targets must have n_rows entries");
  const size_t grid = student_only ? n_rows : 2 * n_rows;
  KlCeChunkOutput r;
  r.grad_kl_student.assign(n_rows * v, 0.0f);
  r.kl_per_row.assign(n_rows, 0.0f);
  r.grad_ce.assign(grid * v, 0.0f);
  r.ce_loss.assign(grid, 0.0f);
  auto host = [](std::vector<float>& x, size_t rows, size_t cols) {
    return orda_tensor{x.data(), static_cast<int64_t>(rows), static_cast<int64_t>(cols), 0,
                       ORDA_F32, ORDA_HOST};
  };
  const orda_tensor lc{const_cast<float*>(logits_chunk.data()), static_cast<int64_t>(2 * n_rows),
                       static_cast<int64_t>(v), 0, ORDA_F32, ORDA_HOST};
  orda_tensor gk = host(r.grad_kl_student, n_rows, v), kr = host(r.kl_per_row, n_rows, 1);
  orda_tensor gc = host(r.grad_ce, grid, v), cl = host(r.ce_loss, grid, 1);
  char err[1024] = {0};
  detail::check(orda_kl_ce_on_logits_chunk(ctx ? ctx->get() : nullptr, &lc, targets.data(),
                                           ORDA_HOST, static_cast<int64_t>(n_rows), inv_t,
                                           kl_grad_scale, t_sq, student_ce_weight,
                                           teacher_ce_weight, label_smoothing, ignore_index,
                                           student_only, compute_kl, &gk, &kr, &gc, &cl, err,
                                           sizeof err),
                err);
  return r;
}

/* quantize_grad_w then dequantize_grad_w(·, grad_output) (src/quant.rs:147-202):
 * the dequantized matrix with the rows named by non-ignored in-range targets
 * kept exact, and the INT8 codes and per-row scales. Stochastic rounding
 * draws from Rng::new(seed) (src/quant.rs:18-44). */
struct QuantDequant {
  Mat dequantized;
  std::vector<int8_t> codes;    // [rows, cols]
  std::vector<float> scales;    // [rows]
};

inline QuantDequant quant_dequant_grad_w(const Mat& grad_w, const std::vector<int64_t>& targets,
                                         int64_t ignore_index, bool stochastic, uint64_t seed,
                                         float grad_output = 1.0f, Context* ctx = nullptr) {
  QuantDequant r;
  r.dequantized = Mat::zeros(grad_w.rows, grad_w.cols);
  r.codes.assign(grad_w.rows * grad_w.cols, 0);
  r.scales.assign(grad_w.rows, 0.0f);
  const orda_tensor m = grad_w.view();
  orda_tensor out = r.dequantized.view();
  orda_tensor codes{r.codes.data(), static_cast<int64_t>(grad_w.rows),
                    static_cast<int64_t>(grad_w.cols), 0, ORDA_I8, ORDA_HOST};
  orda_tensor scales{r.scales.data(), static_cast<int64_t>(grad_w.rows), 1, 0, ORDA_F32, ORDA_HOST};
  char err[1024] = {0};
  detail::check(orda_quant_rows_int8(ctx ? ctx->get() : nullptr, &m, targets.data(),
                                     static_cast<int64_t>(targets.size()), ORDA_HOST, ignore_index,
                                     stochastic, seed, grad_output, &out, &codes, &scales, err,
                                     sizeof err),
                err);
  return r;
}

}  // namespace orda

#endif  // ORDA_ORDA_HPP
