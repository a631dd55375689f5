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

}  // namespace orda
