// mfma_power.hip — measurement probe, not part of the library: bf16 MFMA
// throughput on all CUs with operands that change every iteration (as a
// GEMM's do) or stay fixed, for the two bf16 MFMA shapes of gfx950.
// One wave per SIMD (256 threads per workgroup, 256 workgroups). Each wave
// keeps 256 fp32 accumulators per lane (64 blocks of 16x16 or 16 of 32x32)
// and 16 operand registers (8 bf16 each) holding random N(0,1)-like bf16
// values, which a VALU XOR changes once per iteration (CHANGE=1) or never
// (CHANGE=0). Both shapes do the same flops per iteration. Build with
// `make -C orda-cutile-rs_amd probes`; prints TFLOP/s per variant.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
#define CHECK(x) do { hipError_t e = (x); if (e != hipSuccess) { printf("err %s %d\n", hipGetErrorString(e), __LINE__); exit(1);} } while (0)

template <int CHANGE>
__global__ __launch_bounds__(256, 1) void mfma16(const u32x4* src, float* out, int iters) {
  const int tid = threadIdx.x;
  u32x4 a[8], b[8];
  for (int i = 0; i < 8; ++i) { a[i] = src[(blockIdx.x * 256 + tid) * 16 + i]; b[i] = src[(blockIdx.x * 256 + tid) * 16 + 8 + i]; }
  f32x4 acc[8][8];
  for (int i = 0; i < 8; ++i) for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0, 0, 0, 0};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[i]), __builtin_bit_cast(bf16x8, b[j]), acc[i][j], 0, 0, 0);
    if (CHANGE) {
#pragma unroll
      for (int i = 0; i < 8; ++i) { a[i] ^= u32x4{0x00550055u, 0x00aa00aau, 0x00330033u, 0x00cc00ccu}; b[i] ^= u32x4{0x00cc00ccu, 0x00330033u, 0x00aa00aau, 0x00550055u}; }
    }
  }
  float s = 0.f;
  for (int i = 0; i < 8; ++i) for (int j = 0; j < 8; ++j) s += acc[i][j][0] + acc[i][j][3];
  out[blockIdx.x * 256 + tid] = s;
}

template <int CHANGE>
__global__ __launch_bounds__(256, 1) void mfma32(const u32x4* src, float* out, int iters) {
  const int tid = threadIdx.x;
  u32x4 a[8], b[8];
  for (int i = 0; i < 8; ++i) { a[i] = src[(blockIdx.x * 256 + tid) * 16 + i]; b[i] = src[(blockIdx.x * 256 + tid) * 16 + 8 + i]; }
  f32x16 acc[4][4];
  for (int i = 0; i < 4; ++i) for (int j = 0; j < 4; ++j) for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a[i * 2 + k]), __builtin_bit_cast(bf16x8, b[j * 2 + k]), acc[i][j], 0, 0, 0);
    if (CHANGE) {
#pragma unroll
      for (int i = 0; i < 8; ++i) { a[i] ^= u32x4{0x00550055u, 0x00aa00aau, 0x00330033u, 0x00cc00ccu}; b[i] ^= u32x4{0x00cc00ccu, 0x00330033u, 0x00aa00aau, 0x00550055u}; }
    }
  }
  float s = 0.f;
  for (int i = 0; i < 4; ++i) for (int j = 0; j < 4; ++j) s += acc[i][j][0] + acc[i][j][15];
  out[blockIdx.x * 256 + tid] = s;
}

template <typename K>
float timeit(K k, const u32x4* src, float* out, int iters) {
  hipEvent_t a, b;
  CHECK(hipEventCreate(&a)); CHECK(hipEventCreate(&b));
  hipLaunchKernelGGL(k, dim3(256), dim3(256), 0, 0, src, out, 64);
  CHECK(hipEventRecord(a));
  hipLaunchKernelGGL(k, dim3(256), dim3(256), 0, 0, src, out, iters);
  CHECK(hipEventRecord(b));
  CHECK(hipEventSynchronize(b));
  float ms; CHECK(hipEventElapsedTime(&ms, a, b));
  return ms;
}

int main() {
  const size_t n = 256 * 256 * 16;
  u32x4* h = (u32x4*)malloc(n * sizeof(u32x4));
  uint64_t s = 12345;
  for (size_t i = 0; i < n; ++i) {
    u32x4 v;
    for (int e = 0; e < 4; ++e) {
      // two random bf16 values, N(0,1)-like exponents: sign random, exponent 125..128
      s = s * 6364136223846793005ull + 1442695040888963407ull;
      uint32_t r = (uint32_t)(s >> 32);
      uint32_t lo = ((r & 1) << 15) | ((125 + ((r >> 1) & 3)) << 7) | ((r >> 3) & 0x7f);
      uint32_t hi = (((r >> 10) & 1) << 15) | ((125 + ((r >> 11) & 3)) << 7) | ((r >> 13) & 0x7f);
      v[e] = lo | (hi << 16);
    }
    h[i] = v;
  }
  u32x4* src; float* out;
  CHECK(hipMalloc(&src, n * sizeof(u32x4))); CHECK(hipMalloc(&out, 256 * 256 * 4));
  CHECK(hipMemcpy(src, h, n * sizeof(u32x4), hipMemcpyHostToDevice));
  const int iters = 40000;   // per wave: 64 MFMA x 16384 flop x iters
  const double flops = 256.0 * 4 * iters * 64 * 16384.0;
  for (int rep = 0; rep < 2; ++rep) {
    float t16c = timeit(mfma16<1>, src, out, iters);
    float t16s = timeit(mfma16<0>, src, out, iters);
    float t32c = timeit(mfma32<1>, src, out, iters);
    float t32s = timeit(mfma32<0>, src, out, iters);
    printf("16x16x32 changing %.2f ms %.0f TF | static %.2f ms %.0f TF || 32x32x16 changing %.2f ms %.0f TF | static %.2f ms %.0f TF\n",
           t16c, flops / t16c / 1e9, t16s, flops / t16s / 1e9, t32c, flops / t32c / 1e9, t32s, flops / t32s / 1e9);
    fflush(stdout);
  }
  return 0;
}
