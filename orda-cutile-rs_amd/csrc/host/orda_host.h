// orda_host.h — internal host-side declarations of liborda_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "../../../include/orda/orda.h"
#include "../kernels/orda_kernels.h"

namespace orda {

struct ChunkPlan {
  int64_t chunk_size;
  int64_t num_chunks;
};

int64_t ceil_div(int64_t a, int64_t b);
int64_t chunks_from_raw(double raw);
ChunkPlan resolve_chunk_size(int64_t bt, bool fixed, int64_t fixed_rows, bool has_v, int64_t v,
                             bool has_max_chunks, int64_t max_chunks);
int64_t default_max_chunks_limit(int64_t bt);
std::vector<int64_t> chunk_doubling_schedule(int64_t bt, int64_t start, int64_t limit);

// Error carried to the C ABI boundary.
struct Error {
  int32_t status;
  std::string msg;
};

// Caller-provided per-row scratch of the chunk-launcher entry point (rows up
// to max_rows): int64 labels [max_rows], float4 stats [2*max_rows], float
// label logits [2*max_rows], float row losses [2*max_rows].
struct SlotScratch {
  int64_t max_rows;
  int64_t* labels;
  float4* stats;
  float* xy;
  float* nll;
};

// kl_ce_on_logits_chunk (src/cuda/launch.rs:51-158) behind both C entry
// points; throws Error. With sc every tensor must be on the device and
// nothing is allocated.
void kl_ce_slot(orda_ctx* c, const orda_tensor* logits_chunk, const int32_t* targets,
                int32_t targets_location, int64_t n_rows, float inv_t, float kl_grad_scale,
                float t_sq, float student_ce_weight, float teacher_ce_weight,
                float label_smoothing, int32_t ignore_index, int32_t student_only,
                int32_t compute_kl, orda_tensor* grad_kl_student, orda_tensor* kl_per_row,
                orda_tensor* grad_ce, orda_tensor* ce_loss, const SlotScratch* sc);

int32_t ctx_device(const orda_ctx* c);

// Looks up, once per device, the device address of the no-allocation entry
// point's scratch array (call with that device current). Returns a HIP error.
hipError_t noalloc_scratch_init(int device);

}  // namespace orda
