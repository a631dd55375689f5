// resolver.cpp — chunk-size resolution and the OOM-retry doubling schedule
// (src/resolver.rs:9-126). Pure integer/f64 arithmetic; identical results to
// the reference for every input.
#include <math.h>

#include "orda_host.h"

namespace orda {

int64_t ceil_div(int64_t a, int64_t b) { return a / b + (a % b != 0); }

// resolver.rs:27-36
int64_t chunks_from_raw(double raw) {
  if (raw < 1.5) return 1;
  const double e = floor(log2(raw / 1.5));
  long long ei;
  if (isnan(e)) ei = 0;                       // Rust `as i64` saturates
  else if (e > 1e18) ei = 1000000000000000000LL;
  else if (e < -1e18) ei = -1000000000000000000LL;
  else ei = static_cast<long long>(e);
  ei += 1;
  if (ei < 0) ei = 0;
  if (ei > 60) ei = 60;
  return static_cast<int64_t>(1ull << ei);
}

// resolver.rs:53-99
ChunkPlan resolve_chunk_size(int64_t bt, bool fixed, int64_t fixed_rows, bool has_v, int64_t v,
                             bool has_max_chunks, int64_t max_chunks) {
  if (fixed) {
    int64_t cs = fixed_rows < bt ? fixed_rows : bt;
    if (cs < 1) cs = 1;
    return {cs, ceil_div(bt, cs)};
  }
  if (!has_v) return {bt, 1};
  const int64_t max_useful = bt / 512 > 1 ? bt / 512 : 1;
  const int64_t mc = has_max_chunks ? max_chunks : 2 * max_useful;
  const double vr = static_cast<double>(v) / 32768.0;
  const double raw_pressure = (static_cast<double>(bt) / 1024.0) * (vr * vr);
  const double raw_bt_floor = static_cast<double>(bt) / 4096.0;
  const double raw = fmax(raw_pressure, raw_bt_floor);
  int64_t n = chunks_from_raw(raw);
  if (n > mc) n = mc;
  if (n > max_useful) n = max_useful;
  if (n > bt) n = bt;
  if (n < 1) n = 1;
  return {ceil_div(bt, n), n};
}

// resolver.rs:103-105
int64_t default_max_chunks_limit(int64_t bt) { return 2 * (bt / 512 > 1 ? bt / 512 : 1); }

// resolver.rs:114-126
std::vector<int64_t> chunk_doubling_schedule(int64_t bt, int64_t start, int64_t limit) {
  std::vector<int64_t> out;
  limit = limit < 1 ? 1 : limit;
  limit = limit < bt ? limit : bt;
  if (limit < 1) return out;
  int64_t n = start < 1 ? 1 : (start > limit ? limit : start);
  out.push_back(n);
  while (n < bt && n < limit) {
    int64_t d = n * 2;
    if (d > bt) d = bt;
    if (d > limit) d = limit;
    n = d;
    out.push_back(n);
    if (n >= bt || n >= limit) break;
  }
  return out;
}

}  // namespace orda

extern "C" {

int32_t orda_resolve_chunk_size(int64_t bt, int32_t chunk_fixed, int64_t chunk_rows,
                                int32_t has_v, int64_t v, int32_t has_max_chunks,
                                int64_t max_chunks, int64_t* chunk_size, int64_t* num_chunks) {
  if (bt <= 0 || !chunk_size || !num_chunks) return ORDA_ERR_INVALID;
  const orda::ChunkPlan p = orda::resolve_chunk_size(bt, chunk_fixed != 0, chunk_rows,
                                                     has_v != 0, v, has_max_chunks != 0,
                                                     max_chunks);
  *chunk_size = p.chunk_size;
  *num_chunks = p.num_chunks;
  return ORDA_OK;
}

int64_t orda_chunks_from_raw(double raw) { return orda::chunks_from_raw(raw); }

int64_t orda_default_max_chunks_limit(int64_t bt) { return orda::default_max_chunks_limit(bt); }

int64_t orda_chunk_doubling_schedule(int64_t bt, int64_t start, int64_t limit, int64_t* out,
                                     int64_t cap) {
  const std::vector<int64_t> s = orda::chunk_doubling_schedule(bt, start, limit);
  for (int64_t i = 0; i < static_cast<int64_t>(s.size()) && i < cap; ++i) out[i] = s[i];
  return static_cast<int64_t>(s.size());
}

}  // extern "C"
