// api.cpp — host orchestration of liborda_hip.so: the C ABI of
// include/orda/orda.h over the gfx950 kernels.
//
// distillation_loss follows src/api.rs:188-422 step for step: validate, pick
// the teacher-CE weight, count non-ignored labels for the deferred mean,
// resolve the chunk plan, then per chunk build the [student; teacher]
// logits (one MFMA GEMM with a fused statistics epilogue), run the fused
// KL + CE row pass that overwrites the logits with their gradient, and
// finally run the backward GEMMs, the deferred mean (fused as GEMM alpha),
// the optional INT8 round trip and the f64 loss assembly.
//
// Device-first layout: the logits of consecutive chunks are kept side by
// side in one staging buffer (student block, then teacher block, each
// [rows, pitch]); each chunk's logits_chunk is a slice of it. Every loss
// term comes from fp32 values (GEMM statistics, label logits, the KL cross
// term), so the logits are stored in bf16 for bf16 inputs wherever the row
// pass need not form the KL cross term from them: a Tied teacher (the GEMM
// runs over interleaved student/teacher rows and forms it) or no KL term;
// otherwise fp32. The logits GEMM and the row pass run once per group of
// chunks, and so do the backward GEMMs, which read the gradient rows (in
// place when the logits have the input dtype, else a bf16 copy); grad_W is
// therefore written once per group instead of read-modified-written per
// chunk. The group size is bounded by the context's staging budget (16 GiB
// by default); an out-of-memory failure first halves the group, then walks
// the reference's chunk-doubling schedule (resolver.rs:107-126).
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <chrono>
#include <map>
#include <memory>

#include "orda_host.h"

using orda::DType;
using orda::Error;

struct orda_ctx {
  int device = 0;
  hipStream_t own = nullptr;
  hipStream_t stream = nullptr;
  int64_t mem_limit = 0;
  int64_t held = 0;
  int64_t staging_budget = int64_t(16) << 30;
  struct Buf {
    void* p = nullptr;
    int64_t bytes = 0;
  };
  std::map<std::string, Buf> bufs;
  // Pinned host staging for small device-to-host reads (the labels, which
  // the host validates and counts): a copy into pageable memory costs
  // several times as long.
  void* pinned = nullptr;
  int64_t pinned_bytes = 0;
  bool timing = false;
  struct Pending {
    int kind;
    hipEvent_t a, b;
  };
  std::vector<Pending> pending;
  std::vector<hipEvent_t> pool;
  double total_ms[ORDA_KERNEL_KINDS] = {};
  int64_t launches[ORDA_KERNEL_KINDS] = {};
  // Recorded at the end of a call and polled by wait_stream.
  hipEvent_t done = nullptr;
};

namespace {

[[noreturn]] void fail(int32_t status, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  throw Error{status, buf};
}

void hip_check(hipError_t e, const char* what) {
  if (e == hipSuccess) return;
  (void)hipGetLastError();
  if (e == hipErrorOutOfMemory) fail(ORDA_ERR_OOM, "%s: device out of memory", what);
  fail(ORDA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

// The end-of-call wait for the context's stream. It polls an event for up
// to kSpinMicros, then blocks in hipStreamSynchronize: a short call's wait
// ends sooner after its last operation when polled (Tied BT=256 H=512
// V=8192 fp32: 0.216 against 0.223 ms per call), and a long call does not
// hold a host core for its whole duration.
constexpr int64_t kSpinMicros = 1000;

void wait_stream(orda_ctx* c) {
  hip_check(hipEventRecord(c->done, c->stream), "hipEventRecord");
  const auto t0 = std::chrono::steady_clock::now();
  for (;;) {
    const hipError_t q = hipEventQuery(c->done);
    if (q == hipSuccess) return;
    if (q != hipErrorNotReady) hip_check(q, "hipEventQuery");
    if (std::chrono::steady_clock::now() - t0 > std::chrono::microseconds(kSpinMicros)) break;
    __builtin_ia32_pause();
  }
  hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
}

void copy_err(const Error& e, char* err, size_t len) {
  if (!err || !len) return;
  snprintf(err, len, "%s", e.msg.c_str());
}

// Rust's `{}` Display of an f32 (shortest round-trip digits, no exponent).
std::string fmt_f32(float x) {
  if (isnan(x)) return "NaN";
  if (isinf(x)) return x > 0 ? "inf" : "-inf";
  char buf[128];
  int p = 1;
  for (; p <= 9; ++p) {
    snprintf(buf, sizeof buf, "%.*g", p, static_cast<double>(x));
    if (strtof(buf, nullptr) == x) break;
  }
  if (!strchr(buf, 'e')) return buf;
  // expand exponent notation to a plain decimal
  double d = strtod(buf, nullptr);
  int exp10 = static_cast<int>(floor(log10(fabs(d))));
  int decimals = exp10 < 0 ? (p - 1 - exp10) : std::max(0, p - 1 - exp10);
  snprintf(buf, sizeof buf, "%.*f", decimals, d);
  return buf;
}

int64_t round8(int64_t x) { return (x + 7) / 8 * 8; }
int64_t round64(int64_t x) { return (x + 63) / 64 * 64; }

// Pitch of the logits staging rows: V rounded up to 64 elements, so that every
// row starts on a 128-byte line (the backward GEMMs read these rows in
// 128-byte K-slabs: at V = 50257 a pitch of round8(V) put every slab across two
// lines, grad_hidden 0.524 of peak against 0.60, the row pass 0.65 against
// 0.75). fp32 rows: plus 64 when that is a multiple of 1024, so that rows (and
// the many row streams the row pass and the GEMMs walk in step) do not sit a
// power of two apart. bf16 rows: further up to 64 past a multiple of 1024,
// which measured the bf16 row pass (BT = 8192, paired rows, TB/s, two passes)
// at V = 151936 5.9 against 5.0, at 50257 6.0 against 5.7, at 100000 and 128256
// 1-2 % faster, at 32000 and 200064 1-3 % slower, elsewhere equal; the
// backward GEMMs equal. (fp32 rows at V = 32000: the row pass 1.5 % slower,
// so fp32 keeps the first rule.)
int64_t logits_pitch(int64_t v, orda::DType lt) {
  int64_t p = round64(v);
  if (lt == orda::DType::BF16) {
    while (p % 1024 != 64) p += 64;
    return p;
  }
  return p % 1024 == 0 ? p + 64 : p;
}

int64_t tensor_ld(const orda_tensor& t) { return t.ld ? t.ld : t.cols; }

DType to_dtype(int32_t d, const char* what) {
  if (d == ORDA_F32) return DType::F32;
  if (d == ORDA_BF16) return DType::BF16;
  fail(ORDA_ERR_INVALID, "%s must be float32 or bfloat16", what);
}

// ------------------------------------------------------------ workspace
void* ws(orda_ctx* c, const std::string& name, int64_t bytes) {
  orda_ctx::Buf& b = c->bufs[name];
  if (bytes <= 0) return b.p;
  if (b.p && b.bytes >= bytes) return b.p;
  if (b.p) {
    hip_check(hipFree(b.p), "hipFree");
    c->held -= b.bytes;
    b = orda_ctx::Buf{};
  }
  const int64_t rounded = (bytes + 255) / 256 * 256;
  if (c->mem_limit > 0 && c->held + rounded > c->mem_limit)
    fail(ORDA_ERR_OOM, "workspace '%s' (%lld bytes) exceeds the context memory limit",
         name.c_str(), static_cast<long long>(rounded));
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, rounded);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    if (e == hipErrorOutOfMemory)
      fail(ORDA_ERR_OOM, "hipMalloc of workspace '%s' (%lld bytes): out of memory", name.c_str(),
           static_cast<long long>(rounded));
    hip_check(e, "hipMalloc");
  }
  b.p = p;
  b.bytes = rounded;
  c->held += rounded;
  return p;
}

void ws_release(orda_ctx* c, const std::string& name) {
  auto it = c->bufs.find(name);
  if (it == c->bufs.end() || !it->second.p) return;
  (void)hipFree(it->second.p);
  c->held -= it->second.bytes;
  it->second = orda_ctx::Buf{};
}

void ws_trim(orda_ctx* c) {
  for (auto& kv : c->bufs)
    if (kv.second.p) (void)hipFree(kv.second.p);
  c->bufs.clear();
  c->held = 0;
}

// ------------------------------------------------------------ timing
hipEvent_t get_event(orda_ctx* c) {
  if (!c->pool.empty()) {
    hipEvent_t e = c->pool.back();
    c->pool.pop_back();
    return e;
  }
  hipEvent_t e;
  hip_check(hipEventCreate(&e), "hipEventCreate");
  return e;
}

template <class F>
void timed(orda_ctx* c, int kind, F&& f) {
  if (!c->timing) {
    hip_check(f(), "kernel launch");
    return;
  }
  hipEvent_t a = get_event(c), b = get_event(c);
  hip_check(hipEventRecord(a, c->stream), "hipEventRecord");
  hip_check(f(), "kernel launch");
  hip_check(hipEventRecord(b, c->stream), "hipEventRecord");
  c->pending.push_back({kind, a, b});
}

void collect_timing(orda_ctx* c) {
  for (auto& p : c->pending) {
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) {
      c->total_ms[p.kind] += ms;
      c->launches[p.kind] += 1;
    }
    c->pool.push_back(p.a);
    c->pool.push_back(p.b);
  }
  c->pending.clear();
}

// ------------------------------------------------------------ staging
struct DMat {
  const void* p = nullptr;
  int64_t ld = 0, rows = 0, cols = 0;
  DType t = DType::F32;
};

// The checks every caller tensor passes before any kernel reads it: a
// non-negative shape, a data pointer when it has elements, ld >= cols.
void check_view(const orda_tensor& t, const char* what) {
  if (t.rows < 0 || t.cols < 0) fail(ORDA_ERR_INVALID, "%s has a negative shape", what);
  if (t.rows > 0 && t.cols > 0 && !t.data) fail(ORDA_ERR_INVALID, "%s has a null data pointer", what);
  if (tensor_ld(t) < t.cols) fail(ORDA_ERR_INVALID, "%s has ld < cols", what);
}

// Device-resident view of an input matrix with a pitch that is a multiple of
// 8 elements and a 16-byte aligned base; copies only when needed. A matrix
// of no columns is staged as one column of zeros (pitch 8), so that a
// product over an empty hidden width reads zeros (exactly 0 logits).
DMat stage(orda_ctx* c, const orda_tensor& t, const std::string& name, const char* what) {
  DMat d;
  d.t = to_dtype(t.dtype, what);
  d.rows = t.rows;
  d.cols = t.cols;
  const int64_t ld = tensor_ld(t);
  const int es = orda::dtype_size(d.t);
  check_view(t, what);
  // Pass-through needs whole 16-byte chunks inside every row, including the
  // last one: pitch and width both multiples of 8 elements.
  if (t.location == ORDA_DEVICE && t.cols > 0 && ld % 8 == 0 && t.cols % 8 == 0 &&
      (reinterpret_cast<uintptr_t>(t.data) % 16) == 0) {
    d.p = t.data;
    d.ld = ld;
    return d;
  }
  d.ld = round8(t.cols > 0 ? t.cols : 1);
  void* buf = ws(c, name, t.rows * d.ld * es);
  d.p = buf;
  if (t.rows == 0) return d;
  if (t.location == ORDA_DEVICE) {
    hip_check(orda::launch_convert_rows(d.t, t.data, ld, d.t, buf, d.ld, t.rows, t.cols, c->stream),
              "stage input");
  } else {
    if (d.ld != t.cols)
      hip_check(hipMemsetAsync(buf, 0, t.rows * d.ld * es, c->stream), "hipMemsetAsync");
    if (t.cols > 0)
      hip_check(hipMemcpy2DAsync(buf, d.ld * es, t.data, ld * es, t.cols * es, t.rows,
                                 hipMemcpyHostToDevice, c->stream),
                "upload input");
  }
  return d;
}

// Output matrix: the caller's device buffer, or a device temporary copied
// back to the caller's host buffer at the end.
struct OutMat {
  float* p = nullptr;
  int64_t ld = 0;
  const orda_tensor* t = nullptr;
  bool host = false;
};

OutMat out_mat(orda_ctx* c, const orda_tensor& t, int64_t rows, int64_t cols,
               const std::string& name, const char* what) {
  if (t.dtype != ORDA_F32) fail(ORDA_ERR_INVALID, "%s must be float32", what);
  if (t.rows != rows || t.cols != cols)
    fail(ORDA_ERR_INVALID, "%s must be (%lld, %lld), got (%lld, %lld)", what,
         static_cast<long long>(rows), static_cast<long long>(cols),
         static_cast<long long>(t.rows), static_cast<long long>(t.cols));
  check_view(t, what);
  OutMat o;
  o.t = &t;
  if (t.location == ORDA_DEVICE) {
    o.p = static_cast<float*>(t.data);
    o.ld = tensor_ld(t);
  } else {
    o.host = true;
    o.ld = cols;
    o.p = static_cast<float*>(ws(c, name, rows * cols * 4));
  }
  return o;
}

void download(orda_ctx* c, const OutMat& o) {
  if (!o.host) return;
  const orda_tensor& t = *o.t;
  if (t.rows == 0 || t.cols == 0) return;
  hip_check(hipMemcpy2DAsync(t.data, tensor_ld(t) * 4, o.p, o.ld * 4, t.cols * 4, t.rows,
                             hipMemcpyDeviceToHost, c->stream),
            "download output");
}

// Copy a contiguous device array into an optional caller tensor (1-D data
// viewed as rows x cols with the tensor's pitch).
void deliver(orda_ctx* c, const orda_tensor& t, const void* src, int64_t rows, int64_t cols,
             int es, const char* what) {
  if (!t.data) return;
  if (t.rows != rows || t.cols != cols)
    fail(ORDA_ERR_INVALID, "%s must be (%lld, %lld)", what, static_cast<long long>(rows),
         static_cast<long long>(cols));
  const hipMemcpyKind k = t.location == ORDA_DEVICE ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost;
  hip_check(hipMemcpy2DAsync(t.data, tensor_ld(t) * es, src, cols * es, cols * es, rows, k,
                             c->stream),
            what);
}

// Pinned host staging of at least `bytes` (small device-to-host reads).
void* pinned(orda_ctx* c, int64_t bytes) {
  if (c->pinned_bytes < bytes) {
    if (c->pinned) hip_check(hipHostFree(c->pinned), "hipHostFree");
    c->pinned = nullptr;
    c->pinned_bytes = 0;
    const int64_t b = std::max<int64_t>(bytes, 256);
    hip_check(hipHostMalloc(&c->pinned, b, hipHostMallocDefault), "hipHostMalloc");
    c->pinned_bytes = b;
  }
  return c->pinned;
}

// A host copy of the labels. For labels on the device this reads them back on
// the context's stream and waits: only the error path of distillation_loss
// does that (to report a bad label ahead of a later validation failure).
std::vector<int64_t> host_labels(orda_ctx* c, const int64_t* labels, int64_t n, int32_t loc) {
  std::vector<int64_t> h(static_cast<size_t>(n));
  if (n == 0) return h;
  if (!labels) fail(ORDA_ERR_INVALID, "labels is null");
  if (loc == ORDA_DEVICE) {
    void* p = pinned(c, n * 8);
    hip_check(hipMemcpyAsync(p, labels, n * 8, hipMemcpyDeviceToHost, c->stream), "read labels");
    hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    memcpy(h.data(), p, n * 8);
  } else {
    memcpy(h.data(), labels, n * 8);
  }
  return h;
}

// The labels as a device array the kernels can read: device labels in place
// (8-byte aligned) or copied on the stream; host labels uploaded.
const int64_t* device_labels(orda_ctx* c, const int64_t* labels, int64_t n, int32_t loc,
                             const std::string& name) {
  if (n > 0 && !labels) fail(ORDA_ERR_INVALID, "labels is null");
  if (loc == ORDA_DEVICE && (reinterpret_cast<uintptr_t>(labels) % 8) == 0) return labels;
  void* d = ws(c, name, std::max<int64_t>(8, n * 8));
  if (n > 0)
    hip_check(hipMemcpyAsync(d, labels, n * 8,
                             loc == ORDA_DEVICE ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice,
                             c->stream),
              "stage labels");
  return static_cast<const int64_t*>(d);
}

// api.rs:125-133 on host labels.
void check_labels_host(const std::vector<int64_t>& hl, int64_t v, int64_t ignore) {
  for (int64_t t : hl)
    if (t != ignore && (t < 0 || t >= v))
      fail(ORDA_ERR_INVALID, "label %lld out of range [0, %lld) and != ignore_index %lld",
           static_cast<long long>(t), static_cast<long long>(v), static_cast<long long>(ignore));
}

void config_validate(const orda_kernel_config& k) {
  const int64_t mf = k.max_fused_size;
  if (mf < 1 || (mf & (mf - 1)) != 0)
    fail(ORDA_ERR_INVALID, "max_fused_size must be a power of two >= 1, got %lld",
         static_cast<long long>(mf));
  if (k.has_max_chunks && k.max_chunks < 1)
    fail(ORDA_ERR_INVALID, "max_chunks must be >= 1, got %lld", static_cast<long long>(k.max_chunks));
  if (k.profile < ORDA_PROFILE_BALANCED || k.profile > ORDA_PROFILE_DEBUG)
    fail(ORDA_ERR_INVALID, "unknown profile %d", k.profile);
}

// The dtype the GEMMs and the logits run in: the inputs' own, except bf16
// inputs under the Debug profile (fp32, the precise preset). fast_math
// (Profile::Fast) changes only how the row pass forms its per-row logs and
// divisions (src/config.rs:37-40,93-103), never the inputs.
DType compute_dtype(const orda_kernel_config& k, DType in) {
  if (k.profile == ORDA_PROFILE_DEBUG) return DType::F32;
  return in;
}

// A device copy of an input view in another dtype (pitch round8(cols)).
DMat convert(orda_ctx* c, const DMat& src, DType want, const std::string& name) {
  DMat d = src;
  d.t = want;
  d.ld = round8(src.cols > 0 ? src.cols : 1);
  d.p = ws(c, name, std::max<int64_t>(1, src.rows) * d.ld * orda::dtype_size(want));
  hip_check(orda::launch_convert_rows(src.t, src.p, src.ld, want, const_cast<void*>(d.p), d.ld,
                                      src.rows, src.cols, c->stream),
            "convert input");
  return d;
}

const char* dt_name(DType t) { return t == DType::F32 ? "float32" : "bfloat16"; }

// ------------------------------------------------------------ the loss
struct LossPlan {
  int mode;
  float w_s, w_t, kd, T, ls;
  int64_t ignore;
  bool need_teacher, has_ght, has_gwt;
  bool mean;                // Reduction::Mean; the scale itself is computed on the device
  int64_t bt, h, v, ht;
  DType dt;
  bool quant, stochastic;
  uint64_t seed;
  bool fast_math;           // approximate per-row logs and divisions
  bool online;              // one-pass row statistics (KernelConfig::online_softmax)
};

struct Inputs {
  DMat hs, W, th, tw, tl;
  const int64_t* labels = nullptr;
  OutMat gh, gw, ght, gwt;
};

struct RunResult {
  float scal[4];
};

char* at(const void* base, int64_t elems, DType t) {
  return static_cast<char*>(const_cast<void*>(base)) + elems * orda::dtype_size(t);
}

// Tied teacher with bf16 inputs: the logits GEMM runs over student and
// teacher rows interleaved in blocks of 16, so that it forms the KL cross
// term Σ p_t^T·(x_t − x_s) from its fp32 accumulators.
bool paired_rows(const LossPlan& P, const Inputs& in) {
  return P.need_teacher && P.mode == ORDA_TEACHER_TIED && in.th.ld == in.hs.ld &&
         P.dt == orda::DType::BF16;
}

// Precomputed teacher logits beside bf16 inputs with a KL term, fp32 with a
// pitch of a multiple of 4 elements or bf16 with a pitch of a multiple of 8,
// on a 16-byte aligned base: the logits GEMM reads each tile's teacher logits
// in its epilogue and forms the teacher's statistics and the KL sums there
// (as for paired rows), so that the student logits are stored in bf16 and the
// row pass reads the teacher rows in place.
bool teacher_beside_gemm(const LossPlan& P, const Inputs& in) {
  if (!P.need_teacher || P.mode != ORDA_TEACHER_PRECOMPUTED || P.kd <= 0.f ||
      P.dt != orda::DType::BF16 || reinterpret_cast<uintptr_t>(in.tl.p) % 16)
    return false;
  return (in.tl.t == orda::DType::F32 && in.tl.ld % 4 == 0) ||
         (in.tl.t == orda::DType::BF16 && in.tl.ld % 8 == 0);
}

// A Separate teacher beside bf16 inputs with a KL term: the teacher's logits
// GEMM runs first and stores its logits in fp32, and the student's logits
// GEMM reads them in its epilogue as it reads Precomputed logits; with
// teacher CE the row pass writes the teacher's gradient rows to a bf16
// buffer. Staging bytes per column 6 (8 with teacher CE) instead of 12 for
// fp32 logits of both rows and their bf16 gradients; the same HBM traffic.
bool separate_beside_gemm(const LossPlan& P) {
  return P.need_teacher && P.mode == ORDA_TEACHER_SEPARATE && P.kd > 0.f &&
         P.dt == orda::DType::BF16;
}

// Logits storage: bf16 for bf16 inputs wherever only the gradient reads the
// stored logits (every loss term comes from the GEMM's fp32 statistics, and
// the KL sums from the paired GEMM or from Precomputed teacher logits read in
// its epilogue); fp32 when the row pass must form the KL sums from them.
orda::DType logits_dtype(const LossPlan& P, bool paired) {
  return P.dt == orda::DType::BF16 && (paired || P.kd <= 0.f) ? orda::DType::BF16
                                                             : orda::DType::F32;
}

// Precomputed teacher logits that the row pass reads where they are instead
// of from a copy in the staging buffer: those read beside the logits GEMM
// (teacher_beside_gemm; the row pass takes single elements past a row's
// end), or logits already in the logits dtype with a pitch and a width of a
// multiple of 8 elements and a 16-byte aligned base (that row pass reads
// whole 16-byte vectors of 8 logits, so a narrower last vector would read
// past the row, and past the tensor's storage on its last row).
bool teacher_logits_direct(const LossPlan& P, const Inputs& in) {
  return teacher_beside_gemm(P, in) ||
         (P.need_teacher && P.mode == ORDA_TEACHER_PRECOMPUTED && in.tl.t == logits_dtype(P, false) &&
          in.tl.ld % 8 == 0 && in.tl.cols % 8 == 0 && reinterpret_cast<uintptr_t>(in.tl.p) % 16 == 0);
}

// Device bytes the loss stages per chunk row: the buffers run_loss sizes by
// the group's rows. (The split-K partials of small backward GEMMs are sized
// by the GEMM, at most 256 MB, and come on top.)
int64_t staged_bytes_per_row(const LossPlan& P, const Inputs& in) {
  const bool sep_epi = separate_beside_gemm(P);
  const bool paired = paired_rows(P, in) || teacher_beside_gemm(P, in) || sep_epi;
  const orda::DType lt = logits_dtype(P, paired);
  const int64_t blocks = P.need_teacher && !teacher_logits_direct(P, in) && !sep_epi ? 2 : 1;
  const int64_t nst = orda::gemm_stat_tiles(P.v);
  const int64_t ldl = logits_pitch(P.v, lt);
  int64_t b = blocks * ldl *
              (orda::dtype_size(lt) + (lt == P.dt ? 0 : orda::dtype_size(P.dt)));
  // the teacher's fp32 logits, and its bf16 gradient rows with teacher CE
  if (sep_epi) b += ldl * (P.w_t > 0.f ? 6 : 4);
  b += 2 * nst * 16 + 2 * 4;   // statistics, label logits
  b += 16;                         // row constants
  if (paired) b += nst * 8;        // KL partials
  if (lt == orda::DType::BF16) b += 4 * nst * 4;   // half-tile maxima of both rows
  // fp32 logits with a KL term: the gradient blocks' KL sums
  if (!paired && lt == orda::DType::F32 && P.kd > 0.f) b += orda::row_pass_kl_blocks(P.v) * 16;
  // hcat: the hidden rows transposed for grad_W ([h_s; h_t] with a Tied
  // teacher and teacher CE; else the student's, then the Separate teacher's).
  b += (P.mode == ORDA_TEACHER_TIED && P.w_t > 0.f ? 2 * P.h
                                                   : std::max(P.h, P.has_gwt ? P.ht : int64_t{0})) *
       orda::dtype_size(P.dt);
  return b;
}

// The split-K workspace a backward GEMM asks for, if any (one buffer shared
// by the GEMMs of a call: they run in order on one stream).
void attach_split_ws(orda_ctx* c, orda::GemmArgs& g) {
  const int64_t b = orda::gemm_split_bytes(g);
  if (b <= 0) return;
  const orda_ctx::Buf& cur = c->bufs["splitk"];
  // Growing the buffer frees the old one, which launches already queued on
  // the stream may still use.
  if (cur.p && cur.bytes < b) hip_check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
  g.split_ws = static_cast<float*>(ws(c, "splitk", b));
  g.split_ws_bytes = b;
}

// ms_dev: the deferred-mean scale on the device (LabelStatus::mean_scale).
void run_loss(orda_ctx* c, const LossPlan& P, const Inputs& in, orda::ChunkPlan plan, int64_t G,
              float* row3_out, float* scal_dev, const float* ms_dev) {
  using namespace orda;
  const int64_t cs = plan.chunk_size, nc = plan.num_chunks;
  const int64_t bt = P.bt, v = P.v, h = P.h;
  const DType dt = P.dt;
  const int es = dtype_size(dt);
  const int64_t nst = gemm_stat_tiles(v);
  const int64_t cap = std::min(bt, G * cs);
  const bool tl_direct = teacher_logits_direct(P, in);
  const bool sep_epi = separate_beside_gemm(P);
  const int blocks = P.need_teacher && !tl_direct && !sep_epi ? 2 : 1;
  const bool tied_tce = P.mode == ORDA_TEACHER_TIED && P.w_t > 0.f;

  // Every loss term comes from fp32 values: the GEMM's tile statistics and
  // label logits, and the KL cross term either from the paired GEMM or from
  // fp32 logits read back by the row pass (lt = F32). The gradient rows the
  // backward GEMMs read are in the input dtype: in place when lt == dt,
  // else a separate bf16 buffer.
  const bool paired = paired_rows(P, in);
  // fp32 teacher logits read in the student's logits-GEMM epilogue:
  // Precomputed ones in place, or a Separate teacher's from its own GEMM
  const bool t_epi = teacher_beside_gemm(P, in) || sep_epi;
  const DType lt = logits_dtype(P, paired || t_epi);
  const int64_t ldl = logits_pitch(v, lt);
  void* L = ws(c, "logits", blocks * cap * ldl * dtype_size(lt));
  void* TL = sep_epi ? ws(c, "tlogits", cap * ldl * 4) : nullptr;
  void* TG = sep_epi && P.w_t > 0.f ? ws(c, "tgrad", cap * ldl * es) : nullptr;
  void* Gb = dt == lt ? L : ws(c, "dlogits", blocks * cap * ldl * es);
  // Statistics and label logits of a whole group: student rows, then teacher
  // rows (the logits GEMM of problem p writes row p*M + r).
  float4* stats = static_cast<float4*>(ws(c, "stats", 2 * cap * nst * 16));
  // Written for every non-ignored row by the tile or segment holding its
  // label column (ignored rows are never read).
  float* xy = static_cast<float*>(ws(c, "xy", 2 * cap * 4));
  float* rnll_s = row3_out;
  float* rnll_t = row3_out + bt;
  float* rkl = row3_out + 2 * bt;
  // The hidden rows of a group transposed ([width][rows], pitch ldh_cat):
  // the K-major A operand of grad_Wᵀ.
  const int64_t ldh_cat = round64(tied_tce ? 2 * cap : cap);   // rows on 128-byte lines
  void* hcat = ws(c, "hcat", std::max(h, P.has_gwt ? P.ht : int64_t{0}) * ldh_cat * es);
  float2* cross = paired || t_epi ? static_cast<float2*>(ws(c, "cross", cap * nst * 8)) : nullptr;
  // bf16 logits are stored relative to their half-tile maxima: per row
  // pair and 128-column half, the student's and the teacher's maximum side
  // by side (LogitStatsArgs::hmax).
  const int64_t hld = 4 * nst;
  float* hmax = lt == DType::BF16 ? static_cast<float*>(ws(c, "hmax", cap * hld * 4)) : nullptr;
  // Row constants of the chunked row passes, and for fp32 logits with a KL
  // term the per-block KL sums.
  const bool f32_rows = !paired && lt == DType::F32;
  float4* rconst = static_cast<float4*>(ws(c, "rconst", cap * 16));
  float4* klpart = f32_rows && P.kd > 0.f
                       ? static_cast<float4*>(ws(c, "klpart", cap * row_pass_kl_blocks(v) * 16))
                       : nullptr;
  const float inv_t = 1.0f / P.T;
  // The logits products' K: an empty hidden width (H = 0, or a Separate
  // teacher's Ht = 0) runs over the single zero column its operands are
  // staged with, so the logits are exactly 0; the backward products keep the
  // true width (no output columns, nothing launched).
  const int64_t kh = std::max<int64_t>(h, 1);

  if (v == 0) {
    // An empty vocabulary: every label is ignore_index (validated), so every
    // loss term and every gradient is 0, and grad_W has no rows.
    auto zero_out = [&](const OutMat& o, int64_t cols) {
      if (cols > 0)
        hip_check(hipMemset2DAsync(o.p, o.ld * 4, 0, cols * 4, bt, c->stream), "hipMemset2DAsync");
    };
    zero_out(in.gh, h);
    if (P.has_ght) zero_out(in.ght, P.ht);
    hip_check(hipMemsetAsync(row3_out, 0, 3 * bt * 4, c->stream), "hipMemsetAsync");
  }
  for (int64_t g0 = 0; v > 0 && g0 < nc; g0 += G) {
    const int64_t g1 = std::min(nc, g0 + G);
    const int64_t gs = g0 * cs;
    if (gs >= bt) break;
    const int64_t ge = std::min(bt, g1 * cs);
    const int64_t btg = ge - gs;
    void* Ls = L;
    void* Lt = sep_epi ? TL : at(L, btg * ldl, lt);
    void* Gs = Gb;
    void* Gt = sep_epi ? TG : at(Gb, btg * ldl, dt);
    const bool first = g0 == 0;
    const bool last = ge >= bt;

    // The chunks of a group are computed together: each logit, each row's
    // statistics and each row's gradient depend on that row alone, so one
    // launch over the group's rows gives the per-chunk results of
    // src/api.rs:263-344 exactly; the per-chunk sums are formed from the
    // per-row values in finalize.

    // ---- logits = [h_s; h_t] · Wᵀ (api.rs:272-299) with tile statistics
    GemmArgs f{};
    f.M = btg;
    f.N = v;
    f.K = kh;
    f.lda = in.hs.ld;
    f.ldb = in.W.ld;
    f.ldc = ldl;
    f.a_kmajor = f.b_kmajor = true;
    f.in_type = dt;
    f.logits_type = lt;
    f.epi = GemmEpilogue::Logits;
    f.alpha = 1.f;
    f.lg.stats = stats;
    f.lg.stats_ld = nst;
    f.lg.xy = xy;
    f.lg.labels = in.labels + gs;
    f.lg.ignore_index = P.ignore;
    f.lg.inv_t = inv_t;
    f.lg.hmax = hmax;
    f.lg.hmax_ld = hld;
    f.nprob = 1;
    f.prob[0] = {at(in.hs.p, gs * in.hs.ld, dt), in.W.p, Ls};
    const bool fuse_t = P.need_teacher && P.mode == ORDA_TEACHER_TIED && in.th.ld == in.hs.ld;
    if (paired) {
      // One problem over student and teacher rows in blocks of 16, read in
      // place from both tensors (one pitch); C rows, statistics and label
      // logits come out in the usual order (student rows, then teacher rows).
      f.prob[0] = {at(in.hs.p, gs * in.hs.ld, dt), in.W.p, L};
      f.lg.pair_teacher = at(in.th.p, gs * in.th.ld, dt);
      f.M = 2 * ((btg + 15) / 16 * 16);
      f.lg.pair_rows = btg;
      f.lg.cross = cross;
    } else if (fuse_t) {
      f.nprob = 2;
      f.prob[1] = {at(in.th.p, gs * in.th.ld, dt), in.W.p, Lt};
    } else if (t_epi) {
      // the group's teacher logits, read in the epilogue beside the student
      // rows' accumulators: teacher statistics at rows btg + r, KL sums
      f.lg.teacher_logits = sep_epi ? Lt : at(in.tl.p, gs * in.tl.ld, in.tl.t);
      f.lg.teacher_ld = sep_epi ? ldl : in.tl.ld;
      f.lg.teacher_type = sep_epi ? DType::F32 : in.tl.t;
      f.lg.cross = cross;
    }
    f.group_m = 8;
    // fp32 logits of fp32 inputs, for a product with fewer output tiles than
    // CUs (small BT·V): stored plainly, on 128 x 128 tiles where the product
    // has at most 64 of 256 x 256 and/or with K split over the CUs
    // (launch_gemm's ordered split K), then each row's statistics and label
    // logit from the stored rows, per 8192-column segment. The statistics
    // epilogue needs all of K and 256-wide tiles in one workgroup, so it can
    // neither split nor take the small tiles. Returns whether that path ran.
    auto logits_gemm = [&](const GemmArgs& g) {
      GemmArgs sg = g;
      sg.epi = GemmEpilogue::StoreF32;
      sg.lg = LogitStatsArgs{};
      if (lt != DType::F32 || g.in_type != DType::F32 || paired ||
          (gemm_split_bytes(sg) <= 0 && !gemm_small_tiles(sg))) {
        timed(c, ORDA_KERNEL_GEMM_LOGITS, [&] { return launch_gemm(g, c->stream); });
        return false;
      }
      attach_split_ws(c, sg);
      const GemmSplit sp = gemm_split_plan(sg);
      const bool contiguous =
          g.nprob == 1 || static_cast<float*>(g.prob[1].c) == static_cast<float*>(g.prob[0].c) + g.M * g.ldc;
      if (sp.splits > 1 && contiguous) {
        // The whole product splits: its partials only, then one launch over
        // every problem's rows that sums them in split order, writes the
        // logits and forms each 8192-column segment's statistics and the
        // label logit (the reduction and the statistics of the path below
        // in one pass; timed with the logits GEMM, as the statistics of the
        // fused epilogue are).
        sg.partials_only = true;
        timed(c, ORDA_KERNEL_GEMM_LOGITS, [&] { return launch_gemm(sg, c->stream); });
        RowStatsArgs r{};
        r.src_type = DType::F32;
        r.src = sg.split_ws;
        r.lds = sp.ldp;
        r.src_splits = sp.splits;
        r.src_split_stride = sp.stride;
        r.dst_type = DType::F32;
        r.dst = g.prob[0].c;
        r.ldd = g.ldc;
        r.n_rows = g.M * g.nprob;
        r.v = g.N;
        r.stats = g.lg.stats;
        r.stats_ld = g.lg.stats_ld;
        r.xy = g.lg.xy;
        r.labels = g.lg.labels;
        r.label_rows = g.M;
        r.ignore_index = g.lg.ignore_index;
        r.inv_t = g.lg.inv_t;
        r.segmented = true;
        timed(c, ORDA_KERNEL_GEMM_LOGITS, [&] { return launch_row_stats(r, c->stream); });
        return true;
      }
      timed(c, ORDA_KERNEL_GEMM_LOGITS, [&] { return launch_gemm(sg, c->stream); });
      // the statistics of every problem's rows in one launch where the
      // problems' rows follow each other
      const int groups = contiguous ? 1 : g.nprob;
      for (int p = 0; p < groups; ++p) {
        RowStatsArgs r{};
        r.src_type = DType::F32;
        r.src = g.prob[p].c;
        r.lds = g.ldc;
        r.dst_type = DType::F32;
        r.ldd = g.ldc;
        r.n_rows = contiguous ? g.M * g.nprob : g.M;
        r.v = g.N;
        r.stats = g.lg.stats + p * g.M * g.lg.stats_ld;
        r.stats_ld = g.lg.stats_ld;
        r.xy = g.lg.xy + p * g.M;
        r.labels = g.lg.labels;
        r.label_rows = g.M;
        r.ignore_index = g.lg.ignore_index;
        r.inv_t = g.lg.inv_t;
        r.segmented = true;
        // timed with the logits GEMM, as the fused epilogue's statistics are
        timed(c, ORDA_KERNEL_GEMM_LOGITS, [&] { return launch_row_stats(r, c->stream); });
      }
      return true;
    };
    // A Separate (or Tied at another pitch) teacher's own logits GEMM. With
    // sep_epi it runs first and stores fp32 logits, which the student's
    // epilogue then reads (it writes the teacher statistics again, from the
    // same fp32 values).
    auto teacher_gemm = [&] {
      GemmArgs t = f;
      t.nprob = 1;
      const bool sep = P.mode == ORDA_TEACHER_SEPARATE;
      t.K = sep ? std::max<int64_t>(P.ht, 1) : kh;
      t.lda = in.th.ld;
      t.ldb = sep ? in.tw.ld : in.W.ld;
      t.prob[0] = {at(in.th.p, gs * in.th.ld, dt), sep ? in.tw.p : in.W.p, Lt};
      t.lg.stats = stats + btg * nst;
      t.lg.xy = xy + btg;
      t.lg.hmax = hmax ? hmax + 1 : nullptr;   // the teacher side
      if (sep_epi) {
        t.logits_type = DType::F32;
        t.lg.hmax = nullptr;
        t.lg.teacher_logits = nullptr;
        t.lg.teacher_ld = 0;
        t.lg.cross = nullptr;
      }
      return logits_gemm(t);
    };
    if (sep_epi) teacher_gemm();
    const bool seg_s = logits_gemm(f);
    bool seg_t = fuse_t && seg_s;
    if (P.need_teacher && !fuse_t && !t_epi) {
      if (P.mode == ORDA_TEACHER_PRECOMPUTED) {
        RowStatsArgs r{};
        r.src_type = in.tl.t;
        r.src = at(in.tl.p, gs * in.tl.ld, in.tl.t);
        r.lds = in.tl.ld;
        r.dst_type = lt;
        r.dst = tl_direct ? nullptr : Lt;
        r.ldd = ldl;
        r.n_rows = btg;
        r.v = v;
        r.stats = stats + btg * nst;
        r.stats_ld = nst;
        r.xy = xy + btg;
        r.labels = in.labels + gs;
        r.ignore_index = P.ignore;
        r.inv_t = inv_t;
        r.online = P.online;
        r.segmented = true;
        timed(c, ORDA_KERNEL_OTHER, [&] { return launch_row_stats(r, c->stream); });
      } else {
        seg_t = teacher_gemm();
      }
    }

    // ---- KL + CE + merge, in place (api.rs:301-344)
    {
      RowPassArgs r{};
      r.ltype = lt;
      r.student = Ls;
      r.teacher = !P.need_teacher ? nullptr : tl_direct ? at(in.tl.p, gs * in.tl.ld, in.tl.t) : Lt;
      r.ld_t = tl_direct ? in.tl.ld : sep_epi ? ldl : 0;
      r.grad_s = dt == lt ? nullptr : Gs;
      r.grad_t = sep_epi || dt != lt ? Gt : nullptr;
      r.gtype = dt;
      r.ld = ldl;
      r.n_rows = btg;
      r.v = v;
      r.stats_s = stats;
      r.stats_t = stats + btg * nst;
      r.stats_ld = nst;
      const int64_t nseg = row_stats_segments(v);
      r.stats_tiles = seg_s ? nseg : nst;
      r.stats_tiles_t = t_epi ? nst
                        : P.mode == ORDA_TEACHER_PRECOMPUTED ? nseg
                        : seg_t ? nseg : nst;
      r.xy_s = xy;
      r.xy_t = xy + btg;
      r.cross = cross;
      // Rows of the logits GEMM in bf16 are relative to their half-tile
      // maxima; Precomputed teacher rows (converted or in place) and fp32
      // teacher rows read beside the student GEMM are not.
      r.hmax_s = hmax;
      r.hmax_t = hmax && P.need_teacher && P.mode != ORDA_TEACHER_PRECOMPUTED && !t_epi ? hmax + 1
                                                                                      : nullptr;
      r.hmax_ld = hld;
      r.row_consts = rconst;
      r.kl_part = klpart;
      // the teacher rows as they are: a Separate teacher's fp32 logits, or the
      // caller's Precomputed logits in their own dtype
      r.teacher_f32 = t_epi && (sep_epi || in.tl.t == DType::F32);
      r.teacher_bf16 = t_epi && !sep_epi && in.tl.t == DType::BF16;
      r.labels = in.labels + gs;
      r.ignore_index = P.ignore;
      r.w_s = P.w_s;
      r.w_t = P.w_t;
      r.kd = P.kd;
      r.temperature = P.T;
      r.label_smoothing = P.ls;
      r.teacher_ce = P.w_t > 0.f;
      r.teacher_grad = P.w_t > 0.f && P.mode != ORDA_TEACHER_PRECOMPUTED;
      r.kl = P.kd > 0.f;
      r.row_nll_s = rnll_s + gs;
      r.row_nll_t = rnll_t + gs;
      r.row_kl = rkl + gs;
      r.split = false;
      r.fast_math = P.fast_math;
      timed(c, ORDA_KERNEL_ROW_PASS, [&] { return launch_row_pass(r, c->stream); });
    }

    // ---- grad_hidden = dlogits · W, scaled by the deferred mean (api.rs:347-366, 381-388)
    {
      GemmArgs d{};
      d.M = btg;
      d.N = h;
      d.K = v;
      d.lda = ldl;
      d.ldb = in.W.ld;
      d.ldc = in.gh.ld;
      d.a_kmajor = true;
      d.b_kmajor = false;
      d.in_type = dt;
      d.epi = GemmEpilogue::StoreF32;
      d.alpha = 1.f;
      d.alpha_ptr = ms_dev;
      d.group_m = 4;
      d.share_rounds = true;
      d.nprob = 1;
      d.prob[0] = {Gs, in.W.p, in.gh.p + gs * in.gh.ld};
      const bool fuse = P.has_ght && P.mode == ORDA_TEACHER_TIED && in.ght.ld == in.gh.ld;
      if (fuse) {
        d.nprob = 2;
        d.prob[1] = {Gt, in.W.p, in.ght.p + gs * in.ght.ld};
      }
      attach_split_ws(c, d);
      timed(c, ORDA_KERNEL_GEMM_GRAD_HIDDEN, [&] { return launch_gemm(d, c->stream); });
      if (P.has_ght && !fuse) {
        GemmArgs t = d;
        t.nprob = 1;
        const bool sep = P.mode == ORDA_TEACHER_SEPARATE;
        t.N = sep ? P.ht : h;
        t.ldb = sep ? in.tw.ld : in.W.ld;
        t.ldc = in.ght.ld;
        t.prob[0] = {Gt, sep ? in.tw.p : in.W.p, in.ght.p + gs * in.ght.ld};
        attach_split_ws(c, t);
        timed(c, ORDA_KERNEL_GEMM_GRAD_HIDDEN, [&] { return launch_gemm(t, c->stream); });
      }
    }

    // ---- grad_W (+)= dlogitsᵀ · hidden (api.rs:350, 360, 367-370), computed
    // as grad_Wᵀ = hiddenᵀ · dlogits: the group's hidden rows are transposed
    // into hcat (a K-major A over K = rows), the gradient rows are an N-major
    // B read in place, and C is stored transposed, i.e. as grad_W. With a
    // Tied teacher and teacher CE, [h_s; h_t]ᵀ · [dS; dT] is one GEMM over
    // K = 2·rows (the teacher gradient rows follow the student rows).
    auto grad_weight = [&](const void* ha, int64_t lda_h, const void* hb, int64_t ldb_h,
                           int64_t width, const void* D, float* C, int64_t ldc) {
      const int64_t k = hb != nullptr ? 2 * btg : btg;
      timed(c, ORDA_KERNEL_OTHER, [&] {
        return launch_transpose_rows(ha, lda_h, hb, ldb_h, btg, width, hcat, ldh_cat, dt,
                                     c->stream);
      });
      GemmArgs w{};
      w.M = width;
      w.N = v;
      w.K = k;
      w.lda = ldh_cat;
      w.ldb = ldl;
      w.ldc = ldc;
      w.a_kmajor = true;
      w.b_kmajor = false;
      w.c_trans = true;
      w.in_type = dt;
      w.epi = first ? GemmEpilogue::StoreF32 : GemmEpilogue::AccumF32;
      w.alpha = 1.f;
      w.alpha_ptr = last ? ms_dev : nullptr;
      w.group_m = 8;
      w.nprob = 1;
      w.prob[0] = {hcat, D, C};
      attach_split_ws(c, w);
      timed(c, ORDA_KERNEL_GEMM_GRAD_WEIGHT, [&] { return launch_gemm(w, c->stream); });
    };
    grad_weight(at(in.hs.p, gs * in.hs.ld, dt), in.hs.ld,
                tied_tce ? at(in.th.p, gs * in.th.ld, dt) : nullptr, in.th.ld, h, Gs, in.gw.p,
                in.gw.ld);
    if (P.has_gwt)
      grad_weight(at(in.th.p, gs * in.th.ld, dt), in.th.ld, nullptr, 0, P.ht, Gt, in.gwt.p,
                  in.gwt.ld);
  }

  // ---- loss assembly (api.rs:401-405)
  FinalizeArgs fa{};
  fa.row_nll_s = rnll_s;
  fa.row_nll_t = rnll_t;
  fa.row_kl = rkl;
  fa.bt = bt;
  fa.chunk_size = cs;
  fa.w_s = P.w_s;
  fa.w_t = P.w_t;
  fa.kd = P.kd;
  fa.mean_scale = 1.f;
  fa.mean_scale_ptr = ms_dev;
  fa.out = scal_dev;
  timed(c, ORDA_KERNEL_OTHER, [&] { return launch_finalize(fa, c->stream); });
}

void loss_impl(orda_ctx* c, const orda_tensor* sh, const orda_tensor* w, const int64_t* labels,
               int64_t n_labels, int32_t lab_loc, const orda_teacher* teacher,
               const orda_loss_options* o, orda_loss_output* out) {
  using namespace orda;
  if (!sh || !w || !teacher || !o || !out) fail(ORDA_ERR_INVALID, "null argument");
  // ---- validate (api.rs:104-181)
  config_validate(o->config);
  const int64_t bt = sh->rows, h = sh->cols;
  if (bt == 0) fail(ORDA_ERR_INVALID, "student_hidden has 0 rows (BT must be > 0)");
  if (bt < 0 || h < 0 || w->rows < 0 || w->cols < 0) fail(ORDA_ERR_INVALID, "negative shape");
  if (w->cols != h)
    fail(ORDA_ERR_INVALID, "weight must have shape (V, %lld), got (%lld, %lld)",
         static_cast<long long>(h), static_cast<long long>(w->rows), static_cast<long long>(w->cols));
  const int64_t v = w->rows;
  if (n_labels != bt)
    fail(ORDA_ERR_INVALID, "labels must have length BT=%lld, got %lld", static_cast<long long>(bt),
         static_cast<long long>(n_labels));
  if (!labels) fail(ORDA_ERR_INVALID, "labels is null");
  // Labels on the host are range-checked here (api.rs:125-133). Labels on the
  // device are checked by a kernel with the non-ignored count, and the
  // result is read back with the loss at the end of the call: no wait before
  // the first kernel. If one of the later checks fails first, the device
  // labels are read back then, so that a bad label is still the error
  // reported, as in the reference's order.
  const bool dev_labels = lab_loc == ORDA_DEVICE;
  if (!dev_labels) check_labels_host(host_labels(c, labels, n_labels, lab_loc), v, o->ignore_index);

  LossPlan P{};
  Inputs in;
  const int mode = teacher->mode;
  int64_t ht = h;
  try {
    if (!(o->label_smoothing >= 0.f && o->label_smoothing <= 1.f))
      fail(ORDA_ERR_INVALID, "label_smoothing must be in [0,1], got %s",
           fmt_f32(o->label_smoothing).c_str());
    if (o->kd_weight < 0.f)
      fail(ORDA_ERR_INVALID, "kd_weight must be >= 0, got %s", fmt_f32(o->kd_weight).c_str());
    if (o->temperature <= 0.f)
      fail(ORDA_ERR_INVALID, "temperature must be > 0, got %s", fmt_f32(o->temperature).c_str());
    switch (mode) {
      case ORDA_TEACHER_TIED:
        if (teacher->hidden.rows != bt || teacher->hidden.cols != h)
          fail(ORDA_ERR_INVALID, "Tied teacher hidden must be (%lld, %lld), got (%lld, %lld)",
               static_cast<long long>(bt), static_cast<long long>(h),
               static_cast<long long>(teacher->hidden.rows),
               static_cast<long long>(teacher->hidden.cols));
        break;
      case ORDA_TEACHER_SEPARATE:
        if (teacher->hidden.rows != bt)
          fail(ORDA_ERR_INVALID, "Separate teacher hidden must have BT=%lld rows",
               static_cast<long long>(bt));
        ht = teacher->hidden.cols;
        if (teacher->weight.rows != v || teacher->weight.cols != ht)
          fail(ORDA_ERR_INVALID, "Separate teacher weight must be (%lld, %lld), got (%lld, %lld)",
               static_cast<long long>(v), static_cast<long long>(ht),
               static_cast<long long>(teacher->weight.rows),
               static_cast<long long>(teacher->weight.cols));
        break;
      case ORDA_TEACHER_PRECOMPUTED:
        if (teacher->logits.rows != bt || teacher->logits.cols != v)
          fail(ORDA_ERR_INVALID, "Precomputed teacher logits must be (%lld, %lld), got (%lld, %lld)",
               static_cast<long long>(bt), static_cast<long long>(v),
               static_cast<long long>(teacher->logits.rows),
               static_cast<long long>(teacher->logits.cols));
        break;
      default:
        fail(ORDA_ERR_INVALID, "unknown teacher mode %d", mode);
    }
    // ---- backend (api.rs:197-207)
    if (o->backend == ORDA_BACKEND_CPU)
      fail(ORDA_ERR_INVALID,
           "Backend::Cpu is the reference crate's CPU path; liborda_hip serves Backend::Auto and "
           "Backend::Hip");
    if (o->backend != ORDA_BACKEND_AUTO && o->backend != ORDA_BACKEND_HIP)
      fail(ORDA_ERR_INVALID, "unknown backend %d", o->backend);

    P.mode = mode;
    P.w_s = o->student_ce_weight;
    P.w_t = o->has_teacher_ce_weight ? o->teacher_ce_weight : (mode == ORDA_TEACHER_TIED ? 1.f : 0.f);
    if (P.w_t < 0.f)
      fail(ORDA_ERR_INVALID, "teacher_ce_weight must be >= 0, got %s", fmt_f32(P.w_t).c_str());
    P.kd = o->kd_weight;
    P.T = o->temperature;
    P.ls = o->label_smoothing;
    P.ignore = o->ignore_index;
    P.need_teacher = P.kd > 0.f || P.w_t > 0.f;
    P.has_ght = P.w_t > 0.f && (mode == ORDA_TEACHER_TIED || mode == ORDA_TEACHER_SEPARATE);
    P.has_gwt = P.w_t > 0.f && mode == ORDA_TEACHER_SEPARATE;
    P.mean = o->reduction == ORDA_REDUCTION_MEAN;
    P.bt = bt;
    P.h = h;
    P.v = v;
    P.ht = ht;
    P.quant = o->config.quantize_grad_weight != 0;
    P.stochastic = o->config.stochastic_rounding != 0;
    P.seed = o->config.has_stochastic_seed ? o->config.stochastic_seed : 0;

    // ---- dtypes: every float input shares the student's dtype
    P.dt = to_dtype(sh->dtype, "student_hidden");
    if (to_dtype(w->dtype, "weight") != P.dt)
      fail(ORDA_ERR_INVALID, "weight must be %s like student_hidden", dt_name(P.dt));
    if (P.need_teacher && (mode == ORDA_TEACHER_TIED || mode == ORDA_TEACHER_SEPARATE) &&
        to_dtype(teacher->hidden.dtype, "teacher hidden") != P.dt)
      fail(ORDA_ERR_INVALID, "teacher hidden must be %s like student_hidden", dt_name(P.dt));
    if (P.need_teacher && mode == ORDA_TEACHER_SEPARATE &&
        to_dtype(teacher->weight.dtype, "teacher weight") != P.dt)
      fail(ORDA_ERR_INVALID, "teacher weight must be %s like student_hidden", dt_name(P.dt));

    hip_check(hipSetDevice(c->device), "hipSetDevice");
    // ---- device inputs and outputs
    in.hs = stage(c, *sh, "in.student", "student_hidden");
    in.W = stage(c, *w, "in.weight", "weight");
    if (P.need_teacher && (mode == ORDA_TEACHER_TIED || mode == ORDA_TEACHER_SEPARATE))
      in.th = stage(c, teacher->hidden, "in.t_hidden", "teacher hidden");
    if (P.need_teacher && mode == ORDA_TEACHER_SEPARATE)
      in.tw = stage(c, teacher->weight, "in.t_weight", "teacher weight");
    if (P.need_teacher && mode == ORDA_TEACHER_PRECOMPUTED) {
      const orda_tensor& tl = teacher->logits;
      if (tl.location == ORDA_DEVICE) {
        check_view(tl, "teacher logits");
        in.tl.p = tl.data;
        in.tl.ld = tensor_ld(tl);
        in.tl.t = to_dtype(tl.dtype, "teacher logits");
        in.tl.rows = tl.rows;
        in.tl.cols = tl.cols;
      } else {
        in.tl = stage(c, tl, "in.t_logits", "teacher logits");
      }
    }
    in.gh = out_mat(c, out->grad_student_hidden, bt, h, "out.gh", "grad_student_hidden");
    in.gw = out_mat(c, out->grad_weight, v, h, "out.gw", "grad_weight");
    if (P.has_ght) in.ght = out_mat(c, out->grad_teacher_hidden, bt, ht, "out.ght", "grad_teacher_hidden");
    if (P.has_gwt) in.gwt = out_mat(c, out->grad_teacher_weight, v, ht, "out.gwt", "grad_teacher_weight");
  } catch (const Error& e) {
    if (dev_labels && e.status == ORDA_ERR_INVALID)
      check_labels_host(host_labels(c, labels, n_labels, lab_loc), v, o->ignore_index);
    throw;
  }
  // ---- compute dtype (Profile::Debug)
  {
    const DType ct = compute_dtype(o->config, P.dt);
    if (ct != P.dt) {
      in.hs = convert(c, in.hs, ct, "cv.student");
      in.W = convert(c, in.W, ct, "cv.weight");
      if (in.th.p) in.th = convert(c, in.th, ct, "cv.t_hidden");
      if (in.tw.p) in.tw = convert(c, in.tw, ct, "cv.t_weight");
      P.dt = ct;
    }
  }
  P.fast_math = o->config.fast_math != 0;
  P.online = o->config.online_softmax != 0;
  in.labels = device_labels(c, labels, n_labels, lab_loc, "in.labels");
  float* row3 = static_cast<float*>(ws(c, "rows", 3 * bt * 4));
  // Loss scalars (4 floats) followed by the label status, read back together.
  char* scal_blk = static_cast<char*>(ws(c, "scalars", 64));
  float* scal = reinterpret_cast<float*>(scal_blk);
  LabelStatus* lstat = reinterpret_cast<LabelStatus*>(scal_blk + 16);
  static_assert(16 + sizeof(LabelStatus) <= 64, "scalar block");
  hip_check(launch_label_check(in.labels, bt, v, P.ignore, P.mean, lstat, c->stream), "label check");

  const orda::ChunkPlan plan0 = resolve_chunk_size(bt, o->chunk_fixed != 0, o->chunk_rows, true, v,
                                                   o->config.has_max_chunks != 0,
                                                   o->config.max_chunks);

  // ---- chunk plan, staging group, OOM retry (resolver.rs:103-126)
  orda::ChunkPlan plan = plan0;
  const int64_t limit = o->config.has_max_chunks ? o->config.max_chunks : default_max_chunks_limit(bt);
  const int64_t chunk_bytes = plan.chunk_size * staged_bytes_per_row(P, in);
  int64_t G = std::max<int64_t>(1, std::min<int64_t>(plan.num_chunks, c->staging_budget / std::max<int64_t>(chunk_bytes, 1)));
  for (;;) {
    try {
      run_loss(c, P, in, plan, G, row3, scal, &lstat->mean_scale);
      break;
    } catch (const Error& e) {
      if (e.status != ORDA_ERR_OOM) throw;
      (void)hipStreamSynchronize(c->stream);
      (void)hipGetLastError();
      ws_release(c, "logits");
      ws_release(c, "hcat");
      ws_release(c, "hmax");
      ws_release(c, "stats");
      ws_release(c, "xy");
      ws_release(c, "dlogits");
      ws_release(c, "cross");
      ws_release(c, "rconst");
      ws_release(c, "klpart");
      ws_release(c, "tlogits");
      ws_release(c, "tgrad");
      ws_release(c, "splitk");
      if (G > 1) {
        G /= 2;
        continue;
      }
      const std::vector<int64_t> sched = chunk_doubling_schedule(bt, plan.num_chunks, limit);
      int64_t next = -1;
      for (int64_t s : sched)
        if (s > plan.num_chunks) {
          next = s;
          break;
        }
      if (next < 0)
        fail(ORDA_ERR_OOM, "out of device memory at num_chunks=%lld (limit %lld): %s",
             static_cast<long long>(plan.num_chunks), static_cast<long long>(limit), e.msg.c_str());
      plan = orda::ChunkPlan{ceil_div(bt, next), next};
      G = 1;
    }
  }

  // ---- optional INT8 round trip of grad_W (api.rs:390-399)
  // (V = 0: no rows to quantize; H = 0: rows of no codes, each with the
  // scale of an all-zero row.)
  if (P.quant) {
    uint8_t* keep = nullptr;
    if (v > 0) {
      keep = static_cast<uint8_t*>(ws(c, "keep", v));
      hip_check(hipMemsetAsync(keep, 0, v, c->stream), "hipMemsetAsync");
      hip_check(launch_mark_targets(in.labels, bt, P.ignore, keep, v, c->stream), "mark targets");
    }
    const bool want_codes = out->quant_codes.data != nullptr;
    const bool want_scales = out->quant_scales.data != nullptr;
    int8_t* codes = nullptr;
    float* scales = nullptr;
    int64_t ldq = h;
    if (want_codes) {
      if (out->quant_codes.dtype != ORDA_I8 || out->quant_codes.rows != v || out->quant_codes.cols != h)
        fail(ORDA_ERR_INVALID, "quant_codes must be int8 (%lld, %lld)", static_cast<long long>(v),
             static_cast<long long>(h));
      if (v * h == 0) {
        // no codes to write
      } else if (out->quant_codes.location == ORDA_DEVICE) {
        codes = static_cast<int8_t*>(out->quant_codes.data);
        ldq = tensor_ld(out->quant_codes);
      } else {
        codes = static_cast<int8_t*>(ws(c, "out.codes", v * h));
      }
    }
    if (want_scales) {
      if (out->quant_scales.dtype != ORDA_F32 || out->quant_scales.rows * std::max<int64_t>(out->quant_scales.cols, 1) != v)
        fail(ORDA_ERR_INVALID, "quant_scales must be float32 with V=%lld entries", static_cast<long long>(v));
      scales = out->quant_scales.location == ORDA_DEVICE
                   ? static_cast<float*>(out->quant_scales.data)
                   : static_cast<float*>(ws(c, "out.scales", v * 4));
    }
    QuantArgs q{};
    q.src = in.gw.p;
    q.lds = in.gw.ld;
    q.dst = in.gw.p;
    q.ldd = in.gw.ld;
    q.codes = codes;
    q.ldq = ldq;
    q.scales = scales;
    q.keep_exact = keep;
    q.rows = v;
    q.cols = h;
    q.stochastic = P.stochastic;
    q.seed = P.seed;
    q.grad_output = 1.0f;
    timed(c, ORDA_KERNEL_QUANT, [&] { return launch_quant(q, c->stream); });
    if (codes && out->quant_codes.location != ORDA_DEVICE)
      hip_check(hipMemcpy2DAsync(out->quant_codes.data, tensor_ld(out->quant_codes), codes, h, h, v,
                                 hipMemcpyDeviceToHost, c->stream),
                "download codes");
    if (want_scales && v > 0 && out->quant_scales.location != ORDA_DEVICE)
      hip_check(hipMemcpyAsync(out->quant_scales.data, scales, v * 4, hipMemcpyDeviceToHost,
                               c->stream),
                "download scales");
  }

  // ---- outputs
  download(c, in.gh);
  download(c, in.gw);
  if (P.has_ght) download(c, in.ght);
  if (P.has_gwt) download(c, in.gwt);
  deliver(c, out->row_nll_student, row3, bt, 1, 4, "row_nll_student");
  deliver(c, out->row_nll_teacher, row3 + bt, bt, 1, 4, "row_nll_teacher");
  deliver(c, out->row_kl, row3 + 2 * bt, bt, 1, 4, "row_kl");
  // The one wait of the call: loss scalars and label status together.
  char* hblk = static_cast<char*>(pinned(c, 64));
  hip_check(hipMemcpyAsync(hblk, scal_blk, 64, hipMemcpyDeviceToHost, c->stream), "read loss");
  wait_stream(c);
  collect_timing(c);
  float hs[4];
  LabelStatus ls;
  memcpy(hs, hblk, 16);
  memcpy(&ls, hblk + 16, sizeof ls);
  if (ls.bad_index >= 0)
    fail(ORDA_ERR_INVALID, "label %lld out of range [0, %lld) and != ignore_index %lld",
         static_cast<long long>(ls.bad_label), static_cast<long long>(v),
         static_cast<long long>(P.ignore));
  out->loss = hs[0];
  out->student_ce = hs[1];
  out->teacher_ce = hs[2];
  out->kl = hs[3];
  out->has_grad_teacher_hidden = P.has_ght;
  out->has_grad_teacher_weight = P.has_gwt;
  out->chunk_size = plan.chunk_size;
  out->num_chunks = plan.num_chunks;
}

struct TempCtx {
  orda_ctx* c = nullptr;
  bool owned = false;
  ~TempCtx() {
    if (owned) orda_ctx_destroy(c);
  }
};

orda_ctx* ensure_ctx(orda_ctx* ctx, TempCtx& tmp) {
  if (ctx) return ctx;
  char err[256];
  if (orda_ctx_create(0, &tmp.c, err, sizeof err) != ORDA_OK) fail(ORDA_ERR_UNAVAILABLE, "%s", err);
  tmp.owned = true;
  return tmp.c;
}

}  // namespace

namespace orda {

int32_t ctx_device(const orda_ctx* c) { return c->device; }

// kl_ce_on_logits_chunk (src/cuda/launch.rs:51-158): row statistics of both
// halves of the chunk, then the split row pass. Device logits are read in
// place at any pitch; host tensors are staged. With `sc`, every tensor must
// be on the device and the per-row scratch comes from sc instead of the
// context's workspace (nothing is allocated).
void kl_ce_slot(orda_ctx* c, const orda_tensor* logits_chunk, const int32_t* targets,
                int32_t targets_location, int64_t n_rows, float inv_t, float kl_grad_scale,
                float t_sq, float student_ce_weight, float teacher_ce_weight,
                float label_smoothing, int32_t ignore_index, int32_t student_only,
                int32_t compute_kl, orda_tensor* grad_kl_student, orda_tensor* kl_per_row,
                orda_tensor* grad_ce, orda_tensor* ce_loss, const SlotScratch* sc) {
  if (!logits_chunk || !grad_kl_student || !kl_per_row || !grad_ce || !ce_loss)
    fail(ORDA_ERR_INVALID, "null argument");
  // launch.rs:67-73
  const int64_t v = logits_chunk->cols;
  if (n_rows < 0 || v < 1) fail(ORDA_ERR_INVALID, "empty logits_chunk");
  if (logits_chunk->rows != 2 * n_rows) fail(ORDA_ERR_INVALID, "logits_chunk must be [2*n_rows, V]");
  if (n_rows > 0 && !targets) fail(ORDA_ERR_INVALID, "targets is null");
  check_view(*logits_chunk, "logits_chunk");
  const int64_t grid_rows = student_only ? n_rows : 2 * n_rows;
  if (sc) {
    if (n_rows > sc->max_rows)
      fail(ORDA_ERR_INVALID, "n_rows=%lld exceeds the no-allocation scratch limit of %lld rows",
           static_cast<long long>(n_rows), static_cast<long long>(sc->max_rows));
    const orda_tensor* dev_only[] = {logits_chunk, grad_kl_student, kl_per_row, grad_ce, ce_loss};
    for (const orda_tensor* t : dev_only)
      if (t->location != ORDA_DEVICE)
        fail(ORDA_ERR_INVALID, "the no-allocation entry point takes device tensors only");
    if (targets_location != ORDA_DEVICE)
      fail(ORDA_ERR_INVALID, "the no-allocation entry point takes device targets only");
  }
  hip_check(hipSetDevice(c->device), "hipSetDevice");
  // Under HIP graph capture (the no-allocation form only: every tensor is on
  // the device, so nothing is copied back) the call records its kernels and
  // returns without waiting: a synchronize would invalidate the capture.
  // Per-kernel timing is skipped then too (its events would be replayed
  // with the graph, not read).
  bool capturing = false;
  if (sc) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    hip_check(hipStreamIsCapturing(c->stream, &cs), "hipStreamIsCapturing");
    capturing = cs != hipStreamCaptureStatusNone;
  }
  auto launch = [&](int kind, auto&& f) {
    if (capturing)
      hip_check(f(), "kernel launch");
    else
      timed(c, kind, f);
  };
  DMat L;
  if (logits_chunk->location == ORDA_DEVICE) {
    L.p = logits_chunk->data;
    L.ld = tensor_ld(*logits_chunk);
    L.t = to_dtype(logits_chunk->dtype, "logits_chunk");
    L.rows = logits_chunk->rows;
    L.cols = v;
  } else {
    L = stage(c, *logits_chunk, "slot.logits", "logits_chunk");
  }
  OutMat gk = out_mat(c, *grad_kl_student, n_rows, v, "slot.gkl", "grad_kl_student");
  OutMat gc = out_mat(c, *grad_ce, grid_rows, v, "slot.gce", "grad_ce");
  OutMat kr = out_mat(c, *kl_per_row, n_rows, 1, "slot.klr", "kl_per_row");
  OutMat cl = out_mat(c, *ce_loss, grid_rows, 1, "slot.cel", "ce_loss");
  if (gk.ld != v || gc.ld != v) fail(ORDA_ERR_INVALID, "gradient outputs must be dense");
  const int64_t n2 = std::max<int64_t>(1, 2 * n_rows);
  int64_t* lab;
  float4* stats;
  float* xy;
  float* nll_unused;
  if (sc) {
    lab = sc->labels;
    stats = sc->stats;
    xy = sc->xy;
    nll_unused = sc->nll;
  } else {
    lab = static_cast<int64_t*>(ws(c, "slot.labels", std::max<int64_t>(1, n_rows) * 8));
    stats = static_cast<float4*>(ws(c, "slot.stats", n2 * 16));
    xy = static_cast<float*>(ws(c, "slot.xy", n2 * 4));
    nll_unused = static_cast<float*>(ws(c, "slot.unused", n2 * 4));
  }
  // Targets widened to the kernels' int64 labels on the stream (device
  // targets), or on the host and uploaded; the label logits start at zero.
  std::vector<int64_t> hl;   // lives until the stream is synchronized below
  if (targets_location == ORDA_DEVICE) {
    hip_check(launch_widen_targets(targets, n_rows, lab, xy, 2 * n_rows, c->stream), "targets");
  } else {
    hl.resize(static_cast<size_t>(n_rows));
    for (int64_t i = 0; i < n_rows; ++i) hl[i] = targets[i];
    if (n_rows > 0)
      hip_check(hipMemcpyAsync(lab, hl.data(), n_rows * 8, hipMemcpyHostToDevice, c->stream),
                "upload targets");
    hip_check(launch_widen_targets(nullptr, 0, nullptr, xy, 2 * n_rows, c->stream), "targets");
  }
  for (int half = 0; half < 2; ++half) {
    RowStatsArgs r{};
    r.src_type = L.t;
    r.src = at(L.p, half * n_rows * L.ld, L.t);
    r.lds = L.ld;
    r.dst = nullptr;
    r.n_rows = n_rows;
    r.v = v;
    r.stats = stats + half * n_rows;
    r.stats_ld = 1;
    r.xy = xy + half * n_rows;
    r.labels = lab;
    r.ignore_index = ignore_index;
    r.inv_t = inv_t;
    launch(ORDA_KERNEL_OTHER, [&] { return launch_row_stats(r, c->stream); });
  }
  RowPassArgs a{};
  a.ltype = L.t;
  a.student = const_cast<void*>(L.p);
  a.teacher = at(L.p, n_rows * L.ld, L.t);
  a.ld = L.ld;
  a.n_rows = n_rows;
  a.v = v;
  a.stats_s = stats;
  a.stats_t = stats + n_rows;
  a.stats_ld = 1;
  a.stats_tiles = 1;
  a.stats_tiles_t = 1;
  a.xy_s = xy;
  a.xy_t = xy + n_rows;
  a.labels = lab;
  a.ignore_index = ignore_index;
  a.w_s = student_ce_weight;
  a.w_t = teacher_ce_weight;
  a.kd = 0.f;
  a.temperature = 1.f / inv_t;
  a.label_smoothing = label_smoothing;
  a.kl = compute_kl != 0;
  a.row_nll_s = nll_unused;
  a.row_nll_t = nll_unused + n_rows;
  a.row_kl = kr.p;
  a.split = true;
  a.grad_kl = gk.p;
  a.grad_ce = gc.p;
  a.ce_loss = cl.p;
  a.kl_grad_scale = kl_grad_scale;
  a.t_sq = t_sq;
  a.inv_t = inv_t;
  a.student_only = student_only != 0;
  launch(ORDA_KERNEL_ROW_PASS, [&] { return launch_row_pass(a, c->stream); });
  download(c, gk);
  download(c, gc);
  download(c, kr);
  download(c, cl);
  if (capturing) return;
  wait_stream(c);
  collect_timing(c);
}

}  // namespace orda

extern "C" {

int32_t orda_abi_version(void) { return ORDA_ABI_VERSION; }

int32_t orda_is_available(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n < 1) {
    (void)hipGetLastError();
    return 0;
  }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, 0) != hipSuccess) return 0;
  return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

void orda_kernel_config_from_profile(int32_t profile, orda_kernel_config* cfg) {
  if (!cfg) return;
  memset(cfg, 0, sizeof *cfg);
  cfg->fast_math = profile == ORDA_PROFILE_FAST;
  cfg->max_fused_size = 65536 / 2;
  cfg->profile = profile;
}

void orda_loss_options_default(orda_loss_options* o) {
  if (!o) return;
  memset(o, 0, sizeof *o);
  o->student_ce_weight = 1.0f;
  o->kd_weight = 0.0f;
  o->temperature = 1.0f;
  o->ignore_index = -100;
  o->label_smoothing = 0.0f;
  o->reduction = ORDA_REDUCTION_MEAN;
  o->chunk_fixed = 0;
  orda_kernel_config_from_profile(ORDA_PROFILE_BALANCED, &o->config);
  o->backend = ORDA_BACKEND_AUTO;
}

int32_t orda_kernel_config_validate(const orda_kernel_config* cfg, char* err, size_t err_len) {
  try {
    if (!cfg) fail(ORDA_ERR_INVALID, "null config");
    config_validate(*cfg);
    return ORDA_OK;
  } catch (const Error& e) {
    copy_err(e, err, err_len);
    return e.status;
  }
}

int32_t orda_ctx_create(int32_t device, orda_ctx** out, char* err, size_t err_len) {
  try {
    if (!out) fail(ORDA_ERR_INVALID, "null output pointer");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n < 1) {
      (void)hipGetLastError();
      fail(ORDA_ERR_UNAVAILABLE, "no HIP device is visible");
    }
    if (device < 0 || device >= n) fail(ORDA_ERR_INVALID, "device %d out of range [0, %d)", device, n);
    std::unique_ptr<orda_ctx> c(new orda_ctx());
    c->device = device;
    hip_check(hipSetDevice(device), "hipSetDevice");
    // A blocking stream: it waits for work the caller queued on the legacy
    // null stream (torch's default stream, whose handle is NULL) before it
    // reads the inputs, and the null stream waits for it in turn.
    hip_check(hipStreamCreateWithFlags(&c->own, hipStreamDefault), "hipStreamCreate");
    c->stream = c->own;
    hip_check(hipEventCreateWithFlags(&c->done, hipEventDisableTiming), "hipEventCreate");
    // The no-allocation entry point's scratch address on this device.
    hip_check(orda::noalloc_scratch_init(device), "no-allocation scratch");
    *out = c.release();
    return ORDA_OK;
  } catch (const Error& e) {
    copy_err(e, err, err_len);
    return e.status;
  }
}

void orda_ctx_destroy(orda_ctx* c) {
  if (!c) return;
  (void)hipSetDevice(c->device);
  if (c->stream) (void)hipStreamSynchronize(c->stream);
  for (auto& p : c->pending) {
    c->pool.push_back(p.a);
    c->pool.push_back(p.b);
  }
  for (hipEvent_t e : c->pool) (void)hipEventDestroy(e);
  if (c->pinned) (void)hipHostFree(c->pinned);
  if (c->done) (void)hipEventDestroy(c->done);
  ws_trim(c);
  if (c->own) (void)hipStreamDestroy(c->own);
  delete c;
}

int32_t orda_ctx_set_stream(orda_ctx* c, void* s) {
  if (!c) return ORDA_ERR_INVALID;
  c->stream = s ? static_cast<hipStream_t>(s) : c->own;
  return ORDA_OK;
}

int32_t orda_ctx_set_memory_limit(orda_ctx* c, int64_t bytes) {
  if (!c || bytes < 0) return ORDA_ERR_INVALID;
  c->mem_limit = bytes;
  return ORDA_OK;
}

int32_t orda_ctx_set_staging_budget(orda_ctx* c, int64_t bytes) {
  if (!c || bytes <= 0) return ORDA_ERR_INVALID;
  c->staging_budget = bytes;
  return ORDA_OK;
}

int32_t orda_ctx_workspace_bytes(orda_ctx* c, int64_t* bytes) {
  if (!c || !bytes) return ORDA_ERR_INVALID;
  *bytes = c->held;
  return ORDA_OK;
}

int32_t orda_ctx_trim(orda_ctx* c) {
  if (!c) return ORDA_ERR_INVALID;
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->stream);
  ws_trim(c);
  return ORDA_OK;
}

int32_t orda_ctx_set_timing(orda_ctx* c, int32_t enable) {
  if (!c) return ORDA_ERR_INVALID;
  c->timing = enable != 0;
  return ORDA_OK;
}

int32_t orda_ctx_get_kernel_time(orda_ctx* c, int32_t kind, double* total_ms, int64_t* launches) {
  if (!c || kind < 0 || kind >= ORDA_KERNEL_KINDS) return ORDA_ERR_INVALID;
  if (total_ms) *total_ms = c->total_ms[kind];
  if (launches) *launches = c->launches[kind];
  return ORDA_OK;
}

int32_t orda_ctx_reset_kernel_time(orda_ctx* c) {
  if (!c) return ORDA_ERR_INVALID;
  for (int k = 0; k < ORDA_KERNEL_KINDS; ++k) {
    c->total_ms[k] = 0;
    c->launches[k] = 0;
  }
  return ORDA_OK;
}

int32_t orda_distillation_loss(orda_ctx* ctx, const orda_tensor* student_hidden,
                               const orda_tensor* weight, const int64_t* labels, int64_t n_labels,
                               int32_t labels_location, const orda_teacher* teacher,
                               const orda_loss_options* opts, orda_loss_output* out, char* err,
                               size_t err_len) {
  TempCtx tmp;
  try {
    orda_ctx* c = ensure_ctx(ctx, tmp);
    loss_impl(c, student_hidden, weight, labels, n_labels, labels_location, teacher, opts, out);
    return ORDA_OK;
  } catch (const Error& e) {
    copy_err(e, err, err_len);
    return e.status;
  } catch (const std::exception& e) {
    copy_err(Error{ORDA_ERR_INTERNAL, e.what()}, err, err_len);
    return ORDA_ERR_INTERNAL;
  }
}

int32_t orda_kl_ce_on_logits_chunk(orda_ctx* ctx, const orda_tensor* logits_chunk,
                                   const int32_t* targets, int32_t targets_location, int64_t n_rows,
                                   float inv_t, float kl_grad_scale, float t_sq,
                                   float student_ce_weight, float teacher_ce_weight,
                                   float label_smoothing, int32_t ignore_index,
                                   int32_t student_only, int32_t compute_kl,
                                   orda_tensor* grad_kl_student, orda_tensor* kl_per_row,
                                   orda_tensor* grad_ce, orda_tensor* ce_loss, char* err,
                                   size_t err_len) {
  TempCtx tmp;
  try {
    orda_ctx* c = ensure_ctx(ctx, tmp);
    orda::kl_ce_slot(c, logits_chunk, targets, targets_location, n_rows, inv_t, kl_grad_scale,
                     t_sq, student_ce_weight, teacher_ce_weight, label_smoothing, ignore_index,
                     student_only, compute_kl, grad_kl_student, kl_per_row, grad_ce, ce_loss,
                     nullptr);
    return ORDA_OK;
  } catch (const Error& e) {
    copy_err(e, err, err_len);
    return e.status;
  } catch (const std::exception& e) {
    copy_err(Error{ORDA_ERR_INTERNAL, e.what()}, err, err_len);
    return ORDA_ERR_INTERNAL;
  }
}

int32_t orda_quant_rows_int8(orda_ctx* ctx, const orda_tensor* m, const int64_t* targets,
                             int64_t n_targets, int32_t targets_location, int64_t ignore_index,
                             int32_t stochastic, uint64_t seed, float grad_output,
                             orda_tensor* outp, orda_tensor* codes, orda_tensor* scales, char* err,
                             size_t err_len) {
  using namespace orda;
  TempCtx tmp;
  try {
    orda_ctx* c = ensure_ctx(ctx, tmp);
    if (!m || !outp) fail(ORDA_ERR_INVALID, "null argument");
    if (m->dtype != ORDA_F32) fail(ORDA_ERR_INVALID, "m must be float32");
    hip_check(hipSetDevice(c->device), "hipSetDevice");
    const int64_t rows = m->rows, cols = m->cols;
    const DMat src = stage(c, *m, "q.src", "m");
    OutMat o = out_mat(c, *outp, rows, cols, "q.out", "out");
    const int64_t* lab = device_labels(c, targets, n_targets, targets_location, "q.labels");
    uint8_t* keep = static_cast<uint8_t*>(ws(c, "q.keep", std::max<int64_t>(rows, 1)));
    hip_check(hipMemsetAsync(keep, 0, std::max<int64_t>(rows, 1), c->stream), "hipMemsetAsync");
    hip_check(launch_mark_targets(lab, n_targets, ignore_index, keep, rows, c->stream), "mark targets");
    int8_t* q = nullptr;
    int64_t ldq = cols;
    if (codes && codes->data) {
      if (codes->dtype != ORDA_I8 || codes->rows != rows || codes->cols != cols)
        fail(ORDA_ERR_INVALID, "codes must be int8 [rows, cols]");
      if (codes->location == ORDA_DEVICE) {
        q = static_cast<int8_t*>(codes->data);
        ldq = tensor_ld(*codes);
      } else {
        q = static_cast<int8_t*>(ws(c, "q.codes", std::max<int64_t>(1, rows * cols)));
      }
    }
    float* s = nullptr;
    if (scales && scales->data) {
      if (scales->dtype != ORDA_F32 || scales->rows * std::max<int64_t>(scales->cols, 1) != rows)
        fail(ORDA_ERR_INVALID, "scales must be float32 with one entry per row");
      s = scales->location == ORDA_DEVICE ? static_cast<float*>(scales->data)
                                          : static_cast<float*>(ws(c, "q.scales", std::max<int64_t>(1, rows) * 4));
    }
    QuantArgs a{};
    a.src = static_cast<const float*>(src.p);
    a.lds = src.ld;
    a.dst = o.p;
    a.ldd = o.ld;
    a.codes = q;
    a.ldq = ldq;
    a.scales = s;
    a.keep_exact = keep;
    a.rows = rows;
    a.cols = cols;
    a.stochastic = stochastic != 0;
    a.seed = seed;
    a.grad_output = grad_output;
    timed(c, ORDA_KERNEL_QUANT, [&] { return launch_quant(a, c->stream); });
    download(c, o);
    if (q && codes->location != ORDA_DEVICE && rows * cols > 0)
      hip_check(hipMemcpy2DAsync(codes->data, tensor_ld(*codes), q, cols, cols, rows,
                                 hipMemcpyDeviceToHost, c->stream),
                "download codes");
    if (s && scales->location != ORDA_DEVICE && rows > 0)
      hip_check(hipMemcpyAsync(scales->data, s, rows * 4, hipMemcpyDeviceToHost, c->stream),
                "download scales");
    wait_stream(c);
    collect_timing(c);
    return ORDA_OK;
  } catch (const Error& e) {
    copy_err(e, err, err_len);
    return e.status;
  } catch (const std::exception& e) {
    copy_err(Error{ORDA_ERR_INTERNAL, e.what()}, err, err_len);
    return ORDA_ERR_INTERNAL;
  }
}

}  // extern "C"
