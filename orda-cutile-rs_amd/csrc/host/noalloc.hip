// noalloc.hip — orda_kl_ce_on_logits_chunk_noalloc: the chunk-launcher entry
// point without any device allocation, for callers that cannot allocate
// during the call (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).
//
// The per-row scratch the kernels need (int64 labels, row statistics of both
// halves of the chunk, label logits, row losses: 56 bytes per row) lives in
// one file-scope device array of kMaxRows rows (1.75 MiB), which every GPU
// the library runs on holds until the process ends. Host code never passes
// the array's name to a kernel: its device address is looked up once per
// device with hipGetSymbolAddress (at context creation, with that device
// current) and only that address is used. Every call on a GPU shares that
// GPU's array, so calls that overlap on one GPU (two streams, two threads)
// race; each call writes every scratch entry it reads first.
#include <mutex>

#include "orda_host.h"

namespace {

constexpr int64_t kMaxRows = 32768;
// labels 8 B, stats 2 x 16 B, label logits 2 x 4 B, row losses 2 x 4 B
constexpr int64_t kBytesPerRow = 8 + 2 * 16 + 2 * 4 + 2 * 4;
constexpr int64_t kScratchBytes = kMaxRows * kBytesPerRow;
constexpr int kMaxDevices = 64;

}  // namespace

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

std::mutex g_mu;
void* g_scratch[kMaxDevices] = {};   // device address of `scratch` per device

}  // namespace

namespace orda {

hipError_t noalloc_scratch_init(int device) {
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_scratch[device] != nullptr) return hipSuccess;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return e;
  g_scratch[device] = p;
  return hipSuccess;
}

}  // namespace orda

namespace {

void* scratch_of(int device) {
  std::lock_guard<std::mutex> lock(g_mu);
  return g_scratch[device];
}

}  // namespace

extern "C" int32_t orda_kl_ce_on_logits_chunk_noalloc(
    orda_ctx* ctx, const orda_tensor* logits_chunk, const int32_t* targets,
    int32_t targets_location, int64_t n_rows, float inv_t, float kl_grad_scale, float t_sq,
    float student_ce_weight, float teacher_ce_weight, float label_smoothing,
    int32_t ignore_index, int32_t student_only, int32_t compute_kl, orda_tensor* grad_kl_student,
    orda_tensor* kl_per_row, orda_tensor* grad_ce, orda_tensor* ce_loss, char* err,
    size_t err_len) {
  auto report = [&](int32_t status, const std::string& msg) {
    if (err && err_len) snprintf(err, err_len, "%s", msg.c_str());
    return status;
  };
  try {
    if (!ctx) return report(ORDA_ERR_INVALID, "the no-allocation entry point needs a context");
    const int dev = orda::ctx_device(ctx);
    hipError_t e = hipSetDevice(dev);
    if (e == hipSuccess) e = orda::noalloc_scratch_init(dev);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return report(ORDA_ERR_HIP, std::string("no-allocation scratch: ") + hipGetErrorString(e));
    }
    unsigned char* base = static_cast<unsigned char*>(scratch_of(dev));
    orda::SlotScratch sc;
    sc.max_rows = kMaxRows;
    sc.labels = reinterpret_cast<int64_t*>(base);
    sc.stats = reinterpret_cast<float4*>(base + 8 * kMaxRows);
    sc.xy = reinterpret_cast<float*>(base + 40 * kMaxRows);
    sc.nll = reinterpret_cast<float*>(base + 48 * kMaxRows);
    orda::kl_ce_slot(ctx, logits_chunk, targets, targets_location, n_rows, inv_t, kl_grad_scale,
                     t_sq, student_ce_weight, teacher_ce_weight, label_smoothing, ignore_index,
                     student_only, compute_kl, grad_kl_student, kl_per_row, grad_ce, ce_loss, &sc);
    return ORDA_OK;
  } catch (const orda::Error& e) {
    return report(e.status, e.msg);
  } catch (const std::exception& e) {
    return report(ORDA_ERR_INTERNAL, e.what());
  }
}
