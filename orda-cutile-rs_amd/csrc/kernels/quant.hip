// quant.hip — INT8 row-wise quantize/dequantize of grad_W on gfx950, and the
// small element-wise helpers of the host orchestration.
//
// One workgroup per row (src/quant.rs:96-144, 157-202); rows that fit in
// registers are read once (quant_vec_kernel), longer ones twice:
//   s    = max(amax, 1e-12) / 127                (f32, IEEE division)
//   code = clamp(RNE(x / s), -127, 127)           deterministic
//   code = clamp(floor(x/s) + (frac > u), ...)    stochastic, u from SplitMix64
//   out  = (target row ? x : code * s) * grad_output
// The reference draws one SplitMix64 uniform per element in row-major order
// over the whole matrix. SplitMix64 advances its state by a constant, so the
// draw for flat element e is mix(seed + (e + 2)·γ) — computed here per
// element, which reproduces the sequential stream bit for bit.
#include <math.h>

#include "orda_kernels.h"

namespace orda {
namespace {

constexpr int kThreads = 256;
typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;

__device__ __forceinline__ uint64_t splitmix_mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// quant.rs:39-43 for the draw with index e of Rng::new(seed).
__device__ __forceinline__ float uniform_at(uint64_t seed, uint64_t e) {
  const uint64_t z = splitmix_mix(seed + (e + 2) * kGamma);
  return static_cast<float>(z >> 40) * (1.0f / 16777216.0f);
}

__device__ __forceinline__ int8_t to_code(float v) {
  if (isnan(v)) return 0;
  v = fminf(fmaxf(v, -127.0f), 127.0f);
  return static_cast<int8_t>(v);
}

__global__ __launch_bounds__(kThreads) void quant_kernel(QuantArgs a) {
  __shared__ float red[kThreads / 64];
  const int64_t r = blockIdx.x;
  const float* src = a.src + r * a.lds;
  float amax = 0.f;
  for (int64_t c = threadIdx.x; c < a.cols; c += kThreads) amax = fmaxf(amax, fabsf(src[c]));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = red[0];
#pragma unroll
  for (int w = 1; w < kThreads / 64; ++w) amax = fmaxf(amax, red[w]);
  const float s = fmaxf(amax, 1e-12f) / 127.0f;
  const bool keep = a.keep_exact && a.keep_exact[r];
  float* dst = a.dst + r * a.ldd;
  int8_t* q = a.codes ? a.codes + r * a.ldq : nullptr;
  const uint64_t ebase = static_cast<uint64_t>(r) * static_cast<uint64_t>(a.cols);
  for (int64_t c = threadIdx.x; c < a.cols; c += kThreads) {
    const float x = src[c];
    const float scaled = x / s;
    int8_t code;
    if (a.stochastic) {
      const float fl = floorf(scaled);
      const float u = uniform_at(a.seed, ebase + static_cast<uint64_t>(c));
      code = to_code(fl + ((scaled - fl) > u ? 1.0f : 0.0f));
    } else {
      code = to_code(rintf(scaled));
    }
    if (q) q[c] = code;
    const float deq = keep ? x : static_cast<float>(code) * s;
    dst[c] = deq * a.grad_output;
  }
  if (a.scales && threadIdx.x == 0) a.scales[r] = s;
}

// One code and its dequantized value (quant.rs:109-144, 186-199).
__device__ __forceinline__ float quant_one(const QuantArgs& a, float x, float s, bool keep,
                                           uint64_t e, int8_t& code) {
  const float scaled = x / s;
  if (a.stochastic) {
    const float fl = floorf(scaled);
    code = to_code(fl + ((scaled - fl) > uniform_at(a.seed, e) ? 1.0f : 0.0f));
  } else {
    code = to_code(rintf(scaled));
  }
  return (keep ? x : static_cast<float>(code) * s) * a.grad_output;
}

// Rows of at most kThreads·4·NV elements with 16-byte aligned rows: each row
// is read once into registers (float4 per load), reduced to its scale and
// written once. A kept row written in place with grad_output 1 is already
// exact and is not written at all.
template <int NV>
__global__ __launch_bounds__(kThreads) void quant_vec_kernel(QuantArgs a) {
  __shared__ float red[kThreads / 64];
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  const int cols = static_cast<int>(a.cols);
  const float* src = a.src + r * a.lds;
  float4 x[NV];
  float amax = 0.f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int c = (tid + k * kThreads) * 4;
    // grad_W streams through once: non-temporal loads and stores
    if (c < cols) {
      const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(src + c));
      x[k] = make_float4(v[0], v[1], v[2], v[3]);
    } else {
      x[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(x[k].x), fabsf(x[k].y)), fmaxf(fabsf(x[k].z), fabsf(x[k].w))));
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  if ((tid & 63) == 0) red[tid >> 6] = amax;
  __syncthreads();
  amax = red[0];
#pragma unroll
  for (int w = 1; w < kThreads / 64; ++w) amax = fmaxf(amax, red[w]);
  const float s = fmaxf(amax, 1e-12f) / 127.0f;             // quant.rs:54-57
  const bool keep = a.keep_exact && a.keep_exact[r];
  const bool write = !(keep && a.dst == a.src && a.ldd == a.lds && a.grad_output == 1.0f);
  float* dst = a.dst + r * a.ldd;
  int8_t* q = a.codes ? a.codes + r * a.ldq : nullptr;
  const uint64_t ebase = static_cast<uint64_t>(r) * static_cast<uint64_t>(a.cols);
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int c = (tid + k * kThreads) * 4;
    if (c >= cols) continue;
    int8_t c0, c1, c2, c3;
    float4 o;
    o.x = quant_one(a, x[k].x, s, keep, ebase + c, c0);
    o.y = quant_one(a, x[k].y, s, keep, ebase + c + 1, c1);
    o.z = quant_one(a, x[k].z, s, keep, ebase + c + 2, c2);
    o.w = quant_one(a, x[k].w, s, keep, ebase + c + 3, c3);
    if (write) __builtin_nontemporal_store(f32x4{o.x, o.y, o.z, o.w}, reinterpret_cast<f32x4*>(dst + c));
    if (q) {
      const uint32_t packed = static_cast<uint32_t>(static_cast<uint8_t>(c0)) |
                              (static_cast<uint32_t>(static_cast<uint8_t>(c1)) << 8) |
                              (static_cast<uint32_t>(static_cast<uint8_t>(c2)) << 16) |
                              (static_cast<uint32_t>(static_cast<uint8_t>(c3)) << 24);
      __builtin_nontemporal_store(packed, reinterpret_cast<uint32_t*>(q + c));
    }
  }
  if (a.scales && tid == 0) a.scales[r] = s;
}

__global__ void mark_targets_kernel(const int64_t* labels, int64_t n, int64_t ignore,
                                    uint8_t* keep, int64_t rows) {
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t t = labels[i];
    if (t != ignore && t >= 0 && t < rows) keep[t] = 1;
  }
}

// One workgroup: the label count, the first invalid label and the mean
// scale, reduced over the block (no atomics, nothing to clear beforehand).
constexpr int kCheckThreads = 1024;
__global__ __launch_bounds__(kCheckThreads) void label_check_kernel(const int64_t* labels, int64_t n,
                                                                    int64_t v, int64_t ignore,
                                                                    bool mean, LabelStatus* out) {
  __shared__ int64_t cnt[kCheckThreads / 64], first[kCheckThreads / 64];
  int64_t c = 0, f = INT64_MAX;
  for (int64_t i = threadIdx.x; i < n; i += kCheckThreads) {
    const int64_t t = labels[i];
    if (t != ignore) {
      ++c;
      if ((t < 0 || t >= v) && i < f) f = i;
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    c += __shfl_xor(c, o);
    const int64_t g = __shfl_xor(f, o);
    f = g < f ? g : f;
  }
  if ((threadIdx.x & 63) == 0) {
    cnt[threadIdx.x >> 6] = c;
    first[threadIdx.x >> 6] = f;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    c = 0;
    f = INT64_MAX;
    for (int w = 0; w < kCheckThreads / 64; ++w) {
      c += cnt[w];
      f = first[w] < f ? first[w] : f;
    }
    LabelStatus s;
    s.n_valid = c;
    s.bad_index = f == INT64_MAX ? -1 : f;
    s.bad_label = f == INT64_MAX ? 0 : labels[f];
    const int64_t denom = mean ? (c > 1 ? c : 1) : 1;
    s.mean_scale = 1.0f / static_cast<float>(denom);   // api.rs:230
    s.pad = 0.f;
    *out = s;
  }
}

__global__ void widen_targets_kernel(const int32_t* in32, int64_t n, int64_t* out64, float* zero,
                                     int64_t n_zero) {
  const int64_t total = n > n_zero ? n : n_zero;
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    if (i < n) out64[i] = in32[i];
    if (i < n_zero) zero[i] = 0.f;
  }
}

// Rows of src (any pitch and alignment) into dst rows of pitch ldd, a
// multiple of 8 elements, zero past `cols`: one workgroup per (row, 2048
// columns), eight columns a thread, stored as one (bf16) or two (fp32)
// 16-byte vectors. (One element per thread with a 64-bit division by the
// pitch each ran at a quarter of this rate.)
constexpr int kConvCols = 2048;
template <typename S, typename D>
__global__ __launch_bounds__(256) void convert_rows_kernel(const S* src, int64_t lds, D* dst,
                                                           int64_t ldd, int64_t cols, int64_t cpr) {
  const int64_t r = blockIdx.x / cpr;
  const int64_t c0 = (blockIdx.x - r * cpr) * kConvCols + threadIdx.x * 8;
  if (c0 >= ldd) return;
  const S* s = src + r * lds + c0;
  float x[8];
  // the widest loads the source row's alignment allows (a row at an odd
  // pitch may start on any boundary)
  const uintptr_t sa = reinterpret_cast<uintptr_t>(s);
  if (c0 + 8 <= cols && sa % 16 == 0) {
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int h = 0; h < static_cast<int>(sizeof(S)) * 8 / 16; ++h) {
      const u4 w = reinterpret_cast<const u4*>(s)[h];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (sizeof(S) == 4) {
          x[4 * h + i] = __uint_as_float(w[i]);
        } else {
          x[2 * i] = __uint_as_float(w[i] << 16);
          x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
      }
    }
  } else if (c0 + 8 <= cols && sa % 8 == 0) {
    typedef uint32_t u2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int h = 0; h < static_cast<int>(sizeof(S)) * 8 / 8; ++h) {
      const u2 w = reinterpret_cast<const u2*>(s)[h];
      if constexpr (sizeof(S) == 4) {
        x[2 * h] = __uint_as_float(w[0]);
        x[2 * h + 1] = __uint_as_float(w[1]);
      } else {
        x[4 * h] = __uint_as_float(w[0] << 16);
        x[4 * h + 1] = __uint_as_float(w[0] & 0xffff0000u);
        x[4 * h + 2] = __uint_as_float(w[1] << 16);
        x[4 * h + 3] = __uint_as_float(w[1] & 0xffff0000u);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = c0 + i < cols ? static_cast<float>(s[i]) : 0.f;
  }
  D* d = dst + r * ldd + c0;
  if constexpr (sizeof(D) == 4) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    reinterpret_cast<f4*>(d)[0] = f4{x[0], x[1], x[2], x[3]};
    reinterpret_cast<f4*>(d)[1] = f4{x[4], x[5], x[6], x[7]};
  } else {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    u4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = __builtin_bit_cast(uint32_t, bf16x2{static_cast<__bf16>(x[2 * i]),
                                                 static_cast<__bf16>(x[2 * i + 1])});
    *reinterpret_cast<u4*>(d) = w;
  }
}

unsigned grid_for(int64_t total) {
  int64_t b = (total + 255) / 256;
  if (b > 65536) b = 65536;
  if (b < 1) b = 1;
  return static_cast<unsigned>(b);
}

}  // namespace

hipError_t launch_quant(const QuantArgs& a, hipStream_t s) {
  if (a.rows <= 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(a.rows)), block(kThreads);
  const auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const bool vec = a.cols % 4 == 0 && a.lds % 4 == 0 && a.ldd % 4 == 0 && al16(a.src) &&
                   al16(a.dst) && (a.codes == nullptr || (a.ldq % 4 == 0 && (reinterpret_cast<uintptr_t>(a.codes) & 3) == 0));
  const int64_t per = kThreads * 4;   // elements per float4 of every thread
  if (vec && a.cols <= per) hipLaunchKernelGGL(quant_vec_kernel<1>, grid, block, 0, s, a);
  else if (vec && a.cols <= 2 * per) hipLaunchKernelGGL(quant_vec_kernel<2>, grid, block, 0, s, a);
  else if (vec && a.cols <= 4 * per) hipLaunchKernelGGL(quant_vec_kernel<4>, grid, block, 0, s, a);
  else if (vec && a.cols <= 8 * per) hipLaunchKernelGGL(quant_vec_kernel<8>, grid, block, 0, s, a);
  else hipLaunchKernelGGL(quant_kernel, grid, block, 0, s, a);
  return hipGetLastError();
}

hipError_t launch_mark_targets(const int64_t* labels, int64_t n, int64_t ignore_index,
                               uint8_t* keep, int64_t rows, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(mark_targets_kernel, dim3(grid_for(n)), dim3(256), 0, s, labels, n,
                     ignore_index, keep, rows);
  return hipGetLastError();
}

hipError_t launch_label_check(const int64_t* labels, int64_t n, int64_t v, int64_t ignore_index,
                              bool mean, LabelStatus* out, hipStream_t s) {
  hipLaunchKernelGGL(label_check_kernel, dim3(1), dim3(kCheckThreads), 0, s, labels, n, v,
                     ignore_index, mean, out);
  return hipGetLastError();
}

hipError_t launch_widen_targets(const int32_t* in32, int64_t n, int64_t* out64, float* zero,
                                int64_t n_zero, hipStream_t s) {
  const int64_t total = n > n_zero ? n : n_zero;
  if (total <= 0) return hipSuccess;
  hipLaunchKernelGGL(widen_targets_kernel, dim3(grid_for(total)), dim3(256), 0, s, in32, n, out64,
                     zero, n_zero);
  return hipGetLastError();
}

hipError_t launch_convert_rows(DType st, const void* src, int64_t lds, DType dt, void* dst,
                               int64_t ldd, int64_t rows, int64_t cols, hipStream_t s) {
  if (rows <= 0 || ldd <= 0) return hipSuccess;
  // dst rows start on 16-byte boundaries and hold whole 8-element vectors
  if (ldd % 8 != 0 || reinterpret_cast<uintptr_t>(dst) % 16 != 0) return hipErrorInvalidValue;
  const int64_t cpr = (ldd + kConvCols - 1) / kConvCols;
  if (rows * cpr > 0x7fffffff) return hipErrorInvalidValue;
  const dim3 g(static_cast<unsigned>(rows * cpr)), b(256);
  if (st == DType::F32 && dt == DType::F32)
    hipLaunchKernelGGL((convert_rows_kernel<float, float>), g, b, 0, s,
                       static_cast<const float*>(src), lds, static_cast<float*>(dst), ldd, cols, cpr);
  else if (st == DType::F32)
    hipLaunchKernelGGL((convert_rows_kernel<float, __bf16>), g, b, 0, s,
                       static_cast<const float*>(src), lds, static_cast<__bf16*>(dst), ldd, cols, cpr);
  else if (dt == DType::F32)
    hipLaunchKernelGGL((convert_rows_kernel<__bf16, float>), g, b, 0, s,
                       static_cast<const __bf16*>(src), lds, static_cast<float*>(dst), ldd, cols, cpr);
  else
    hipLaunchKernelGGL((convert_rows_kernel<__bf16, __bf16>), g, b, 0, s,
                       static_cast<const __bf16*>(src), lds, static_cast<__bf16*>(dst), ldd, cols, cpr);
  return hipGetLastError();
}

}  // namespace orda
