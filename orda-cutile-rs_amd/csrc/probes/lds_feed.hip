// lds_feed.hip — measurement probe, not part of the library: the GEMM's
// global->LDS DMA pattern alone (global_load_lds_dwordx4, no MFMA, no LDS
// reads). Each of 256 workgroups streams stages of 32 KB (or 16 KB) through
// a ring of LDS slots, waiting for the oldest outstanding stage and a barrier
// per stage like the GEMM main loop. Source rows: `rowb` bytes per row and
// stage (64 = a K-major stage, 128 = a K-major stage pair, 512 = an MN-major
// row of 256 bf16), row pitch 262272 bytes (the padded pitch of a 131072-wide
// bf16 logits row). `groups` distinct row blocks are read: 32 gives 4 blocks
// per XCD (8 workgroups share each), 8 gives one block per XCD. A last set
// of runs reads every stage as one contiguous block instead. Build with
// `make -C orda-cutile-rs_amd probes`; prints TB/s per configuration.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
#include <vector>

#define CHECK(x) do { hipError_t e = (x); if (e != hipSuccess) { printf("err %s line %d\n", hipGetErrorString(e), __LINE__); exit(1);} } while (0)

template <int RING, int XF>   // XF: 16-byte transfers per thread per stage
__global__ __launch_bounds__(256, 1) void feed(const unsigned char* src, int64_t pitch, int rowb,
                                               int stages, int groups, unsigned long long* sink, int mn) {
  __shared__ __attribute__((aligned(1024))) unsigned char lds[RING * XF * 4096];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int rows_per_stage = XF * 4096 / rowb;
  const int cpr = rowb / 16;
  const int64_t wg = blockIdx.x % groups;
  const unsigned char* base = src + wg * rows_per_stage * pitch;
  uint32_t goff[XF];
  for (int t = 0; t < XF; ++t) {
    const int P = (t * 4 + wave) * 64 + lane;
    goff[t] = (P / cpr) * (mn == 2 ? rowb : pitch) + (P % cpr) * 16;
  }
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds;
  auto issue = [&](int st, int slot) {
    // mn 1: MN-major rows; mn 2: blocked, each stage one contiguous block
    const unsigned char* s = mn == 1 ? src + (int64_t)(blockIdx.x % groups) * 512 + (int64_t)st * rows_per_stage * pitch
                           : mn == 2 ? src + ((int64_t)(blockIdx.x % groups) * stages + st) * (XF * 4096)
                                     : base + (int64_t)st * rowb;
    uint64_t p = (uint64_t)s;
    uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p), hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
    uint64_t ps = ((uint64_t)hi << 32) | lo;
    for (int t = 0; t < XF; ++t) {
      uint32_t m0 = __builtin_amdgcn_readfirstlane(lds0 + slot * XF * 4096 + (t * 4 + wave) * 1024);
      asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %0" :: "s"(ps), "v"(goff[t]), "s"(m0) : "memory", "m0");
    }
  };
  for (int t = 0; t < RING - 1; ++t) issue(t, t);
  for (int st = 0; st < stages; ++st) {
    // stage st landed: outstanding = stages st+1 .. st+RING-2
    asm volatile("s_waitcnt vmcnt(%0)" :: "n"((RING - 2) * XF));
    __builtin_amdgcn_s_barrier();
    const int nx = st + RING - 1;
    issue(nx < stages ? nx : 0, nx % RING);
  }
  asm volatile("s_waitcnt vmcnt(0)");
  if (tid == 0 && lds[0] == 0x5a && lds[1] == 0xa5) sink[blockIdx.x] = 1;
}

template <int RING, int XF>
float run(const unsigned char* src, int64_t pitch, int rowb, int stages, int groups, int nwg, unsigned long long* sink, int mn) {
  hipEvent_t a, b;
  CHECK(hipEventCreate(&a)); CHECK(hipEventCreate(&b));
  hipLaunchKernelGGL((feed<RING, XF>), dim3(nwg), dim3(256), 0, 0, src, pitch, rowb, stages, groups, sink, mn);
  CHECK(hipEventRecord(a));
  hipLaunchKernelGGL((feed<RING, XF>), dim3(nwg), dim3(256), 0, 0, src, pitch, rowb, stages, groups, sink, mn);
  CHECK(hipEventRecord(b));
  CHECK(hipEventSynchronize(b));
  float ms; CHECK(hipEventElapsedTime(&ms, a, b));
  return ms;
}

int main() {
  const int64_t total_rows = 16384;
  for (int64_t pitch : {(int64_t)262272}) {
  const size_t bytes = (size_t)total_rows * pitch;
  unsigned char* src; CHECK(hipMalloc(&src, bytes));
  CHECK(hipMemset(src, 1, bytes));
  unsigned long long* sink; CHECK(hipMalloc(&sink, 4096 * 8));
  const int nwg = 256;
  for (int groups : {32, 8}) {
    for (int rowb : {64, 128, 512}) {
      const int mn = rowb == 512;
      // K-major: stages cover one row's 262144 bytes; MN-major: stages cover all rows
      const int nst = mn ? 0 : (int)(262144 / rowb);
      for (int xf : {8, 4}) {
        const int rps = xf * 4096 / rowb;
        if (!mn && ((int64_t)groups * rps > total_rows || (int64_t)nst * rowb > pitch)) { printf("bounds\n"); return 1; }
      }
      // MN-major: rows per stage = xf*4096/512 (64 or 32); stages = total_rows / rps;
      // columns: group g reads bytes [g*512, g*512+512) of each row, g < groups <= 32 -> 16 KB < pitch
      const int nst8 = mn ? (int)(total_rows / (8 * 4096 / 512)) : nst;
      const int nst4 = mn ? (int)(total_rows / (4 * 4096 / 512)) : nst;
      if (mn && (int64_t)groups * 512 > pitch) { printf("bounds\n"); return 1; }
      const double tot8 = (double)nwg * nst8 * 32768.0, tot4 = (double)nwg * nst4 * 16384.0;
      float t44 = run<4, 8>(src, pitch, rowb, nst8, groups, nwg, sink, mn);
      float t84 = run<8, 4>(src, pitch, rowb, nst4, groups, nwg, sink, mn);
      printf("pitch %lld rowb %3d groups %3d: ring 4x32KB %.1f TB/s | ring 8x16KB %.1f TB/s\n",
             (long long)pitch, rowb, groups, tot8 / t44 / 1e9, tot4 / t84 / 1e9);
      fflush(stdout);
    }
  }
  // blocked: group g's stages are consecutive contiguous blocks of the stage size
  for (int groups : {32, 8}) {
    const int rowb = 128;
    const int nst8 = (int)(bytes / ((size_t)groups * 32768)) < 2048 ? (int)(bytes / ((size_t)groups * 32768)) : 2048;
    const int nst4 = nst8;
    const double tot8 = (double)nwg * nst8 * 32768.0, tot4 = (double)nwg * nst4 * 16384.0;
    float t44 = run<4, 8>(src, pitch, rowb, nst8, groups, nwg, sink, 2);
    float t84 = run<8, 4>(src, pitch, rowb, nst4, groups, nwg, sink, 2);
    printf("blocked 32KB/16KB stages   groups %3d: ring 4x32KB %.1f TB/s | ring 8x16KB %.1f TB/s\n",
           groups, tot8 / t44 / 1e9, tot4 / t84 / 1e9);
    fflush(stdout);
  }
  CHECK(hipFree(src)); CHECK(hipFree(sink));
  }
  return 0;
}
