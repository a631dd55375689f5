// gemm.hip — MFMA GEMMs of the distillation loss on gfx950.
//
// The three products of the reference's chunk loop (src/api.rs:273-292 and
// :346-377, via src/mat.rs:63-130) all run through one kernel template:
//   logits      C[2n,V]  = [h_s;h_t] · Wᵀ      A K-major, B K-major
//   grad_hidden C[rows,H] = dlogits · W         A K-major, B N-major
//   grad_W      C[V,H]   = dlogitsᵀ · hidden    A M-major, B N-major
//
// Workgroup tile 256x256, 4 waves each owning 128x128, K staged 128 bytes at a
// time (64 bf16 or 32 fp32) through a double-buffered, XOR-swizzled LDS tile
// laid out [row][k]. MN-major operands are transposed in registers
// (v_perm_b32 for bf16) on their way into LDS so every MFMA operand read is
// one conflict-free ds_read_b128. bf16 uses v_mfma_f32_16x16x32_bf16, fp32
// uses v_mfma_f32_16x16x4_f32 (four per 16-byte k-group); accumulation is
// fp32 in both.
//
// The Logits epilogue fuses the statistics the row pass needs: for every row
// and every 256-column tile it writes {max, Σe^(x-max), Σe^((x-max)/T), Σx}
// computed from the fp32 accumulators, and the fp32 logit at the row's label,
// so the row pass reads each logit exactly once.
#include <float.h>
#include <math.h>

#include "orda_kernels.h"

namespace orda {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kTile = 256;           // BM = BN
constexpr int kSlab = 128;           // bytes of K per LDS stage
constexpr int kThreads = 256;
constexpr int kFrag = 8;             // 8x8 MFMA 16x16 fragments per wave
constexpr int kStageBytes = kTile * kSlab;   // 32 KB per operand per stage
constexpr float kLog2e = 1.4426950408889634f;

// Physical 16-byte chunk of (row, chunk) in a [256][128 B] LDS tile. Rows
// r..r+7 (aligned) reading one chunk, and rows r, r+8, ..., r+56 writing one
// chunk, both land on 8 distinct chunks (all 32 banks).
__device__ __forceinline__ int lds_off(int row, int chunk) {
  return row * kSlab + ((chunk ^ ((row ^ (row >> 3)) & 7)) << 4);
}

__device__ __forceinline__ u32x4 lds_read16(const unsigned char* base, int off) {
  return *reinterpret_cast<const u32x4*>(base + off);
}
__device__ __forceinline__ void lds_write16(unsigned char* base, int off, u32x4 v) {
  *reinterpret_cast<u32x4*>(base + off) = v;
}

__device__ __forceinline__ u32x4 gload16(const unsigned char* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

template <typename T>
struct Elem;
template <>
struct Elem<float> {
  static constexpr int kSize = 4;
};
template <>
struct Elem<__bf16> {
  static constexpr int kSize = 2;
};

__device__ __forceinline__ float wave16_max(float v) {
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 16));
  return v;
}
__device__ __forceinline__ float wave16_sum(float v) {
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) v += __shfl_xor(v, o, 16);
  return v;
}

// Operand loader: global -> registers -> (transpose) -> swizzled LDS tile.
// KMAJOR: the operand is stored [rows=M or N][ld], one stage is rows
// [r0, r0+256) x bytes [k0*ES, k0*ES+128).
// !KMAJOR: the operand is stored [K][ld]; one stage is K rows [k0, k0+SK) x
// columns [c0, c0+256).
template <typename T, bool KMAJOR>
struct Loader {
  static constexpr int ES = Elem<T>::kSize;
  static constexpr int EPC = 16 / ES;     // elements per 16-byte chunk
  static constexpr int SK = kSlab / ES;   // K elements per stage

  const unsigned char* base;   // operand base (uniform)
  int64_t ld_bytes;
  int64_t extent;              // rows (KMAJOR) or columns (!KMAJOR) that exist
  int64_t K;
  int r0;                      // tile origin along M/N
  uint32_t voff[8];            // per-thread byte offsets within a stage
  uint32_t valid;              // per-load bit: row/column in range

  __device__ __forceinline__ void init(const void* p, int64_t ld, int64_t ext, int64_t k,
                                       int origin, int tid) {
    base = static_cast<const unsigned char*>(p);
    ld_bytes = ld * ES;
    extent = ext;
    K = k;
    r0 = origin;
    valid = 0;
    if (KMAJOR) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        int row = (tid >> 3) + 32 * i;
        voff[i] = static_cast<uint32_t>(row * ld_bytes + (tid & 7) * 16);
        if (origin + row < ext) valid |= 1u << i;
      }
    } else if (ES == 2) {
      int kb = tid >> 5, mb = tid & 31;
#pragma unroll
      for (int i = 0; i < 8; ++i) voff[i] = static_cast<uint32_t>((kb * 8 + i) * ld_bytes + mb * 16);
      if (origin + mb * 8 < ext) valid = 0xffu;
    } else {
      int mb = tid & 63;
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        int kb = (tid >> 6) + 4 * b;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          voff[b * 4 + i] = static_cast<uint32_t>((kb * 4 + i) * ld_bytes + mb * 16);
      }
      if (origin + mb * 4 < ext) valid = 0xffu;
    }
  }

  // Issue the global loads of stage kt.
  __device__ __forceinline__ void load(u32x4 (&r)[8], int kt, int tid) const {
    const int64_t k0 = static_cast<int64_t>(kt) * SK;
    const int64_t krem = K - k0;
    if (KMAJOR) {
      const unsigned char* s = base + r0 * ld_bytes + k0 * ES;
      const bool kok = (tid & 7) * EPC < krem;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        r[i] = u32x4{0, 0, 0, 0};
        if (kok && ((valid >> i) & 1)) r[i] = gload16(s + voff[i]);
      }
    } else {
      const unsigned char* s = base + k0 * ld_bytes + static_cast<int64_t>(r0) * ES;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        int krow;
        if (ES == 2) krow = (tid >> 5) * 8 + i;
        else krow = ((tid >> 6) + 4 * (i >> 2)) * 4 + (i & 3);
        r[i] = u32x4{0, 0, 0, 0};
        if (krow < krem && ((valid >> i) & 1)) r[i] = gload16(s + voff[i]);
      }
    }
  }

  // Write stage registers to an LDS tile (transposing MN-major data).
  __device__ __forceinline__ void store(unsigned char* tile, const u32x4 (&r)[8], int tid) const {
    if (KMAJOR) {
#pragma unroll
      for (int i = 0; i < 8; ++i) lds_write16(tile, lds_off((tid >> 3) + 32 * i, tid & 7), r[i]);
    } else if (ES == 2) {
      // r[i] holds 8 bf16 of K-row kb*8+i at columns mb*8..mb*8+7; chunk j of
      // the output holds K-rows kb*8..kb*8+7 of column mb*8+j.
      const int kb = tid >> 5, mb = tid & 31;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
        u32x4 o;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          o[q] = __builtin_amdgcn_perm(r[2 * q + 1][j >> 1], r[2 * q][j >> 1], sel);
        lds_write16(tile, lds_off(mb * 8 + j, kb), o);
      }
    } else {
      const int mb = tid & 63;
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const int kb = (tid >> 6) + 4 * b;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          u32x4 o = {r[b * 4 + 0][j], r[b * 4 + 1][j], r[b * 4 + 2][j], r[b * 4 + 3][j]};
          lds_write16(tile, lds_off(mb * 4 + j, kb), o);
        }
      }
    }
  }
};

template <typename T>
__device__ __forceinline__ void mfma_step(f32x4 (&acc)[kFrag][kFrag], const u32x4 (&a)[kFrag],
                                          const u32x4 (&b)[kFrag]) {
#pragma unroll
  for (int i = 0; i < kFrag; ++i) {
#pragma unroll
    for (int j = 0; j < kFrag; ++j) {
      if constexpr (Elem<T>::kSize == 2) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8, a[i]), __builtin_bit_cast(bf16x8, b[j]), acc[i][j], 0, 0, 0);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[i][q]),
                                                           __uint_as_float(b[j][q]), acc[i][j],
                                                           0, 0, 0);
      }
    }
  }
}

struct TileCoord {
  int p, m0, n0, ntile;
};

__device__ __forceinline__ TileCoord map_tile(const GemmArgs& g) {
  const int64_t Mt = (g.M + kTile - 1) / kTile;
  const int64_t Nt = (g.N + kTile - 1) / kTile;
  const int64_t Mv = Mt * g.nprob;
  const int64_t T = Mv * Nt;
  int64_t t = blockIdx.x;
  // Consecutive workgroups land on consecutive XCDs; give each XCD a
  // contiguous range of the raster so tiles sharing operands share an L2.
  const int64_t per = T / 8;
  if (per > 0 && t < per * 8) t = (t % 8) * per + t / 8;
  const int64_t gm = g.group_m > 0 ? g.group_m : 1;
  const int64_t in_group = gm * Nt;
  const int64_t gid = t / in_group;
  const int64_t first = gid * gm;
  const int64_t gsize = (Mv - first) < gm ? (Mv - first) : gm;
  const int64_t r = t % in_group;
  const int64_t pm = first + r % gsize;
  const int64_t pn = r / gsize;
  TileCoord c;
  c.p = static_cast<int>(pm / Mt);
  c.m0 = static_cast<int>((pm % Mt) * kTile);
  c.n0 = static_cast<int>(pn * kTile);
  c.ntile = static_cast<int>(pn);
  return c;
}

template <typename T, bool AK, bool BK, GemmEpilogue EPI, typename LT>
__global__ __launch_bounds__(kThreads, 1) void gemm_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) unsigned char smem[4 * kStageBytes];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const TileCoord tc = map_tile(g);
  const GemmProblem& pr = g.prob[tc.p];

  Loader<T, AK> la;
  Loader<T, BK> lb;
  la.init(pr.a, g.lda, g.M, g.K, tc.m0, tid);
  lb.init(pr.b, g.ldb, g.N, g.K, tc.n0, tid);

  f32x4 acc[kFrag][kFrag];
#pragma unroll
  for (int i = 0; i < kFrag; ++i)
#pragma unroll
    for (int j = 0; j < kFrag; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  constexpr int SK = kSlab / Elem<T>::kSize;
  const int nk = static_cast<int>((g.K + SK - 1) / SK);

  // Stage s of operand A lives at smem + s*2*kStageBytes, of B one stage later.

  u32x4 ra[8], rb[8];
  if (nk > 0) {
    la.load(ra, 0, tid);
    lb.load(rb, 0, tid);
    la.store(smem, ra, tid);
    lb.store(smem + kStageBytes, rb, tid);
  }
  __syncthreads();

  const int lrow = lane & 15;
  const int lgrp = lane >> 4;
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) {
      la.load(ra, kt + 1, tid);
      lb.load(rb, kt + 1, tid);
    }
    const unsigned char* ta = smem + cur * 2 * kStageBytes;
    const unsigned char* tb = ta + kStageBytes;
#pragma unroll
    for (int kg = 0; kg < 2; ++kg) {
      u32x4 af[kFrag], bfr[kFrag];
#pragma unroll
      for (int i = 0; i < kFrag; ++i) af[i] = lds_read16(ta, lds_off(wm * 128 + i * 16 + lrow, kg * 4 + lgrp));
#pragma unroll
      for (int j = 0; j < kFrag; ++j) bfr[j] = lds_read16(tb, lds_off(wn * 128 + j * 16 + lrow, kg * 4 + lgrp));
      mfma_step<T>(acc, af, bfr);
    }
    if (kt + 1 < nk) {
      unsigned char* na = smem + (cur ^ 1) * 2 * kStageBytes;
      la.store(na, ra, tid);
      lb.store(na + kStageBytes, rb, tid);
    }
    __syncthreads();
  }

  // ------------------------------------------------------------ epilogue
  const int row_w = tc.m0 + wm * 128;          // first row of this wave
  const int col_l = tc.n0 + wn * 128 + lrow;   // this lane's column for fragment j=0
  if constexpr (EPI == GemmEpilogue::StoreF32 || EPI == GemmEpilogue::AccumF32) {
    float* C = static_cast<float*>(pr.c);
#pragma unroll
    for (int i = 0; i < kFrag; ++i) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t row = row_w + i * 16 + lgrp * 4 + e;
        if (row >= g.M) continue;
        float* crow = C + row * g.ldc;
#pragma unroll
        for (int j = 0; j < kFrag; ++j) {
          const int64_t col = col_l + j * 16;
          if (col < g.N) {
            float v = acc[i][j][e];
            if constexpr (EPI == GemmEpilogue::AccumF32) v = g.alpha * (crow[col] + v);
            else v = g.alpha * v;
            crow[col] = v;
          }
        }
      }
    }
  } else {
    // Logits: store, then per-row partial softmax statistics of this tile.
    LT* C = static_cast<LT*>(pr.c);
    int64_t* lab = reinterpret_cast<int64_t*>(smem);              // [256] labels
    float4* part = reinterpret_cast<float4*>(smem + 4096);        // [2][256]
    {
      const int64_t row = tc.m0 + tid;
      lab[tid] = row < g.M ? g.lg.labels[row] : g.lg.ignore_index;
    }
    __syncthreads();
    const float it2 = g.lg.inv_t * kLog2e;
    bool cv[kFrag];
#pragma unroll
    for (int j = 0; j < kFrag; ++j) cv[j] = (col_l + j * 16) < g.N;
#pragma unroll
    for (int i = 0; i < kFrag; ++i) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int rl = wm * 128 + i * 16 + lgrp * 4 + e;   // row within tile
        const int64_t row = tc.m0 + rl;
        const bool rv = row < g.M;
        const int64_t y = lab[rl];
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < kFrag; ++j)
          if (cv[j]) mx = fmaxf(mx, acc[i][j][e]);
        mx = wave16_max(mx);
        float d1 = 0.f, dT = 0.f, sx = 0.f;
        if (mx != -INFINITY) {
#pragma unroll
          for (int j = 0; j < kFrag; ++j) {
            if (cv[j]) {
              const float x = acc[i][j][e];
              const float dx = x - mx;
              d1 += __builtin_amdgcn_exp2f(dx * kLog2e);
              dT += __builtin_amdgcn_exp2f(dx * it2);
              sx += x;
            }
          }
        }
        d1 = wave16_sum(d1);
        dT = wave16_sum(dT);
        sx = wave16_sum(sx);
        if (lrow == 0) part[wn * 256 + rl] = make_float4(mx, d1, dT, sx);
        if (rv) {
          LT* crow = C + row * g.ldc;
#pragma unroll
          for (int j = 0; j < kFrag; ++j) {
            const int64_t col = col_l + j * 16;
            if (cv[j]) {
              crow[col] = static_cast<LT>(acc[i][j][e]);
              if (col == y) g.lg.xy[tc.p * g.M + row] = acc[i][j][e];
            }
          }
        }
      }
    }
    __syncthreads();
    {
      const int64_t row = tc.m0 + tid;
      if (row < g.M) {
        const float4 a = part[tid], b = part[256 + tid];
        const float m = fmaxf(a.x, b.x);
        float4 s;
        s.x = m;
        s.w = a.w + b.w;
        if (m == -INFINITY) {
          s.y = 0.f;
          s.z = 0.f;
        } else {
          const float ea = __builtin_amdgcn_exp2f((a.x - m) * kLog2e);
          const float eb = __builtin_amdgcn_exp2f((b.x - m) * kLog2e);
          const float fa = __builtin_amdgcn_exp2f((a.x - m) * it2);
          const float fb = __builtin_amdgcn_exp2f((b.x - m) * it2);
          s.y = a.y * ea + b.y * eb;
          s.z = a.z * fa + b.z * fb;
        }
        g.lg.stats[(static_cast<int64_t>(tc.p) * g.M + row) * g.lg.stats_ld + tc.ntile] = s;
      }
    }
  }
}

template <typename T, bool AK, bool BK, GemmEpilogue EPI, typename LT>
hipError_t launch_t(const GemmArgs& g, hipStream_t s) {
  const int64_t Mt = (g.M + kTile - 1) / kTile;
  const int64_t Nt = (g.N + kTile - 1) / kTile;
  const int64_t tiles = Mt * Nt * g.nprob;
  if (tiles == 0) return hipSuccess;
  hipLaunchKernelGGL((gemm_kernel<T, AK, BK, EPI, LT>), dim3(static_cast<unsigned>(tiles)),
                     dim3(kThreads), 0, s, g);
  return hipGetLastError();
}

template <typename T>
hipError_t dispatch_layout(const GemmArgs& g, hipStream_t s) {
  using E = GemmEpilogue;
  if (g.epi == E::Logits) {
    if (!g.a_kmajor || !g.b_kmajor) return hipErrorInvalidValue;
    if (g.logits_type == DType::BF16) return launch_t<T, true, true, E::Logits, __bf16>(g, s);
    return launch_t<T, true, true, E::Logits, float>(g, s);
  }
  if (g.a_kmajor && !g.b_kmajor) {
    if (g.epi == E::StoreF32) return launch_t<T, true, false, E::StoreF32, float>(g, s);
    return launch_t<T, true, false, E::AccumF32, float>(g, s);
  }
  if (!g.a_kmajor && !g.b_kmajor) {
    if (g.epi == E::StoreF32) return launch_t<T, false, false, E::StoreF32, float>(g, s);
    return launch_t<T, false, false, E::AccumF32, float>(g, s);
  }
  if (g.a_kmajor && g.b_kmajor) {
    if (g.epi == E::StoreF32) return launch_t<T, true, true, E::StoreF32, float>(g, s);
    return launch_t<T, true, true, E::AccumF32, float>(g, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace

int64_t gemm_stat_tiles(int64_t n) { return (n + kTile - 1) / kTile; }

hipError_t launch_gemm(const GemmArgs& g, hipStream_t stream) {
  if (g.nprob < 1 || g.nprob > 2) return hipErrorInvalidValue;
  if ((g.lda % 8) || (g.ldb % 8) || (g.ldc % 8 && g.epi == GemmEpilogue::Logits))
    return hipErrorInvalidValue;
  if (g.in_type == DType::BF16) return dispatch_layout<__bf16>(g, stream);
  return dispatch_layout<float>(g, stream);
}

}  // namespace orda
