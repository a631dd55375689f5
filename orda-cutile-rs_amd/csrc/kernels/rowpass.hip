// rowpass.hip — the row pass of the distillation loss on gfx950.
//
// For each (student row, teacher row) pair of a logits chunk (layout of
// src/api.rs:276-299: student rows, then teacher rows) it forms, from the
// per-tile softmax statistics written by the logits GEMM, lse at T=1 and at
// temperature T, then streams the two rows once:
//   student grad = w_s·((p_s − α/V) − [j=y](1−α)) + kd·T·(p_s^T − p_t^T)
//                                          (cross_entropy.rs:58-71, kl.rs:83-124,
//                                           merge api.rs:335-344)
//   teacher grad = w_t·((p_t − α/V) − [j=y](1−α))   (api.rs:325-333)
// overwriting both rows in place, and the KL term
//   KL_row = Σ p_t^T (x_t − x_s)/T + lse_s^T − lse_t^T,
// where lse_s^T − lse_t^T = log(Σ e^(x_s/T) / Σ e^(x_t/T)) is formed as
// log1p(D/S) from a sum D of per-element differences of the two rows'
// terms (each difference rounded once) over the teacher's sum S: for nearly
// equal rows, two separately rounded sums of V terms would leave an error of
// a few 1e-7 in a KL that may itself be that small.
// Three forms:
//   * paired bf16 logits: the KL cross sum comes per tile from the logits
//     GEMM's fp32 accumulators (the stored logits only feed the gradient);
//     a per-row kernel merges the statistics, an elementwise kernel over
//     (row, column block) writes the gradient;
//   * large fp32 chunks: the same two kernels, the elementwise one also
//     summing each block's share of the KL cross sum, then a per-row sum;
//   * otherwise one workgroup per row pair, fused.
// The per-row NLL uses the fp32 label logit and Σx from the GEMM epilogue and
// is formed in f64 like the reference. Exponentials are exp2 with log2(e)
// folded into one FMA per element.
#include <math.h>

#include "kl_sums.h"
#include "orda_kernels.h"

namespace orda {
namespace {

constexpr int kThreads = 256;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Per-row constants: precise logf / IEEE division, or with fast_math the
// hardware approximations (v_log_f32 times ln 2, v_rcp_f32 then a multiply).
__device__ __forceinline__ float rlog(float x, bool fast) {
  return fast ? __builtin_amdgcn_logf(x) * kLn2 : logf(x);
}
__device__ __forceinline__ float rlog2(float x, bool fast) {
  return fast ? __builtin_amdgcn_logf(x) : log2f(x);
}
__device__ __forceinline__ float rdiv(float a, float b, bool fast) {
  return fast ? a * __builtin_amdgcn_rcpf(b) : a / b;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct Stat {
  float m, d1, dT, sx;
};

__device__ __forceinline__ Stat merge(Stat a, Stat b, float it2) {
  Stat r;
  r.m = fmaxf(a.m, b.m);
  r.sx = a.sx + b.sx;
  if (r.m == -INFINITY) {
    r.d1 = 0.f;
    r.dT = 0.f;
  } else {
    r.d1 = a.d1 * __builtin_amdgcn_exp2f((a.m - r.m) * kLog2e) +
           b.d1 * __builtin_amdgcn_exp2f((b.m - r.m) * kLog2e);
    r.dT = a.dT * __builtin_amdgcn_exp2f((a.m - r.m) * it2) +
           b.dT * __builtin_amdgcn_exp2f((b.m - r.m) * it2);
  }
  return r;
}

__device__ __forceinline__ Stat shfl_xor_stat(Stat s, int o) {
  Stat r;
  r.m = __shfl_xor(s.m, o);
  r.d1 = __shfl_xor(s.d1, o);
  r.dT = __shfl_xor(s.dT, o);
  r.sx = __shfl_xor(s.sx, o);
  return r;
}

// Block-wide merge of per-thread partial stats; every thread gets the result.
template <int TPB = kThreads>
__device__ Stat block_merge(Stat s, float it2, Stat* scratch) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) s = merge(s, shfl_xor_stat(s, o), it2);
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[wave] = s;
  __syncthreads();
  Stat r = scratch[0];
#pragma unroll
  for (int w = 1; w < TPB / 64; ++w) r = merge(r, scratch[w], it2);
  return r;
}

template <int TPB = kThreads>
__device__ float block_sum(float v, float* scratch) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[wave] = v;
  __syncthreads();
  float r = 0.f;
#pragma unroll
  for (int w = 0; w < TPB / 64; ++w) r += scratch[w];
  return r;
}

template <int TPB = kThreads>
__device__ Stat load_row_stats(const float4* st, int64_t tiles, float it2, Stat* scratch) {
  Stat s{-INFINITY, 0.f, 0.f, 0.f};
  for (int64_t t = threadIdx.x; t < tiles; t += TPB) {
    const float4 v = st[t];
    s = merge(s, Stat{v.x, v.y, v.z, v.w}, it2);
  }
  return block_merge<TPB>(s, it2, scratch);
}

// Vector of logits in storage type LT <-> fp32.
template <typename LT>
struct Vec;
template <>
struct Vec<float> {
  static constexpr int N = 4;
  typedef u32x4 raw;
  static __device__ __forceinline__ void unpack(raw r, float (&x)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] = __uint_as_float(r[i]);
  }
  static __device__ __forceinline__ raw pack(const float (&x)[N]) {
    raw r;
#pragma unroll
    for (int i = 0; i < N; ++i) r[i] = __float_as_uint(x[i]);
    return r;
  }
};
template <>
struct Vec<__bf16> {
  static constexpr int N = 8;
  typedef u32x4 raw;
  static __device__ __forceinline__ void unpack(raw r, float (&x)[N]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = __uint_as_float(r[i] << 16);
      x[2 * i + 1] = __uint_as_float(r[i] & 0xffff0000u);
    }
  }
  static __device__ __forceinline__ raw pack(const float (&x)[N]) {
    // one v_cvt_pk_bf16_f32 (round to nearest even) per pair
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    raw r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bf16x2 p = {static_cast<__bf16>(x[2 * i]), static_cast<__bf16>(x[2 * i + 1])};
      r[i] = __builtin_bit_cast(uint32_t, p);
    }
    return r;
  }
};

// KL_row (without T²) of a row pair from its merged statistics s, t and the
// paired GEMM's merged KL sums x (kl_sums.h): the mean of the centred
// difference under p_t^T plus log1p(x.y / t.dT) = lse_s^T - lse_t^T (with
// the shift between the two maxima taken out of both). Precise log1p and
// division of the sums in every profile (they carry the small-KL
// precision; one per row). Should x.y / t.dT not lie in (-1, inf), the two
// rows' own sums instead.
__device__ __forceinline__ float kl_paired(float2 x, const Stat& s, const Stat& t, float inv_t,
                                           bool fast) {
  const float z = x.y / t.dT;
  const float lr = isfinite(z) && z > -1.f ? log1pf(z) : rlog(rdiv(s.dT, t.dT, fast), fast);
  return rdiv(x.x, t.dT, fast) * (kLn2 * inv_t) + lr;
}

// KL_row (without T²) from the sums of a pass that forms p_s^T and p_t^T
// itself as 2^(x·log2(e)/T − o) (scaled by the same factor g in both):
// cross = g·Σ p_t^T (x_t − x_s), sum_t = g·Σ p_t^T, sum_d = g·Σ (p_s^T − p_t^T)
// (each difference formed before it is summed), and do = o_s − o_t, the
// difference of the two exponent offsets as the pass used them (log2
// units). Exact in those terms: KL = E_t[x_t − x_s]/T + (lse_s^T − lse_t^T),
// with lse_s^T − lse_t^T = do·ln2 + log(Σ p_s^T / Σ p_t^T).
__device__ __forceinline__ float kl_from_sums(float cross, float sum_t, float sum_d, float d_off,
                                              float inv_t, bool fast) {
  return rdiv(cross, sum_t, fast) * inv_t + d_off * kLn2 + log1pf(sum_d / sum_t);
}

// nll of cross_entropy.rs:46-56 from merged stats, in f64.
__device__ __forceinline__ double row_nll(const Stat& s, float xy, double alpha, int64_t v) {
  const double lse = static_cast<double>(s.m) + log(static_cast<double>(s.d1));
  if (alpha > 0.0)
    return lse - (1.0 - alpha) * static_cast<double>(xy) -
           (alpha / static_cast<double>(v)) * static_cast<double>(s.sx);
  return lse - static_cast<double>(xy);
}

template <typename LT, bool SPLIT, int TPB>
__global__ __launch_bounds__(TPB) void row_pass_kernel(RowPassArgs a) {
  __shared__ Stat sstat[TPB / 64];
  __shared__ float ssum[TPB / 64];
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t y = a.labels[r];
  // A label outside [0, V) that is not ignore_index is an error the host
  // reports; the row is then treated as ignored so no access leaves the row.
  const bool ignored = y == a.ignore_index || y < 0 || y >= a.v;
  const bool has_t = a.teacher != nullptr;
  const float T = a.temperature;
  const float inv_t = SPLIT ? a.inv_t : 1.0f / T;
  const float it2 = inv_t * kLog2e;

  const Stat ss = load_row_stats<TPB>(a.stats_s + r * a.stats_ld, a.stats_tiles, it2, sstat);
  Stat st{-INFINITY, 0.f, 0.f, 0.f};
  if (has_t) st = load_row_stats<TPB>(a.stats_t + r * a.stats_ld, a.stats_tiles_t, it2, sstat);

  const double alpha = static_cast<double>(a.label_smoothing);
  // Per-row constants: p = exp2(x*log2e - off).
  const float lse1_s = ss.m + logf(ss.d1);
  const float lseT_s = ss.m * inv_t + logf(ss.dT);
  const float lse1_t = st.m + logf(st.d1);
  const float lseT_t = st.m * inv_t + logf(st.dT);
  const float o1s = lse1_s * kLog2e, oTs = lseT_s * kLog2e;
  const float o1t = lse1_t * kLog2e, oTt = lseT_t * kLog2e;

  const float eps = static_cast<float>(alpha / static_cast<double>(a.v));
  const float one_m_a = 1.0f - a.label_smoothing;
  // CE scales (ignored rows -> 0, cross_entropy.rs:59).
  const float ws = ignored ? 0.f : a.w_s;
  const float wt = ignored ? 0.f : a.w_t;
  const bool do_kl = a.kl && has_t;
  const float gsc = ignored ? 0.f : (SPLIT ? a.kl_grad_scale : a.kd * T);  // kl.rs:85
  const bool do_tgrad = SPLIT ? (!a.student_only && has_t) : (a.teacher_grad && has_t);

  LT* srow = static_cast<LT*>(a.student) + r * a.ld;
  LT* trow = has_t ? static_cast<LT*>(a.teacher) + r * a.ld : nullptr;
  float* gkl = SPLIT ? a.grad_kl + r * a.v : nullptr;
  float* gce_s = SPLIT ? a.grad_ce + r * a.v : nullptr;
  float* gce_t = (SPLIT && do_tgrad) ? a.grad_ce + (a.n_rows + r) * a.v : nullptr;

  using VT = Vec<LT>;
  constexpr int NV = VT::N;
  float cross = 0.f, sum_pt = 0.f, sum_d = 0.f;
  const int64_t vpad = (a.v + NV - 1) / NV * NV;
  // Rows are read where they are, at any pitch: 16-byte vectors where the
  // row is 16-byte aligned and the vector lies inside the row, single
  // elements otherwise (nothing past column V is read).
  const bool vec = (reinterpret_cast<uintptr_t>(srow) & 15) == 0 &&
                   (!has_t || (reinterpret_cast<uintptr_t>(trow) & 15) == 0);
  // SPLIT outputs (dense fp32 rows) leave as 16-byte stores where this
  // row's outputs are 16-byte aligned.
  const bool ovec = SPLIT && (reinterpret_cast<uintptr_t>(gce_s) & 15) == 0 &&
                    (!do_kl || (reinterpret_cast<uintptr_t>(gkl) & 15) == 0) &&
                    (!do_tgrad || (reinterpret_cast<uintptr_t>(gce_t) & 15) == 0);
  for (int64_t j0 = static_cast<int64_t>(tid) * NV; j0 < vpad; j0 += TPB * NV) {
    float xs[NV], xt[NV], gs[NV], gt[NV], gk[NV];
    const bool whole = vec && j0 + NV <= a.v;
    if (whole) {
      VT::unpack(*reinterpret_cast<const typename VT::raw*>(srow + j0), xs);
      if (has_t) VT::unpack(*reinterpret_cast<const typename VT::raw*>(trow + j0), xt);
    } else {
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const bool in = j0 + i < a.v;
        xs[i] = in ? static_cast<float>(srow[j0 + i]) : 0.f;
        xt[i] = in && has_t ? static_cast<float>(trow[j0 + i]) : 0.f;
      }
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int64_t j = j0 + i;
      const bool valid = j < a.v;
      float g = 0.f, gkv = 0.f, gtv = 0.f;
      if (valid) {
        const float p = __builtin_amdgcn_exp2f(fmaf(xs[i], kLog2e, -o1s));
        float prob = p - eps;
        if (j == y) prob -= one_m_a;
        g = prob * ws;
        if (do_kl) {
          const float ps = __builtin_amdgcn_exp2f(fmaf(xs[i], it2, -oTs));
          const float pt = __builtin_amdgcn_exp2f(fmaf(xt[i], it2, -oTt));
          const float d = ps - pt;
          gkv = gsc * d;
          cross = fmaf(pt, xt[i] - xs[i], cross);
          sum_pt += pt;
          sum_d += d;
        }
        if (do_tgrad) {
          const float q = __builtin_amdgcn_exp2f(fmaf(xt[i], kLog2e, -o1t));
          float pr = q - eps;
          if (j == y) pr -= one_m_a;
          gtv = pr * wt;
        }
      }
      if (SPLIT) {
        gs[i] = g;
        gk[i] = gkv;
        gt[i] = gtv;
      } else {
        gs[i] = ignored ? 0.f : g + gkv;
        gt[i] = gtv;
      }
    }
    if (SPLIT) {
      if (whole && ovec) {
        typedef float f4 __attribute__((ext_vector_type(4)));
        // Non-temporal only where a store instruction covers whole lines
        // (fp32 logits: 16 bytes a lane, lanes adjacent). With bf16 logits a
        // lane's 8 outputs are two stores 16 bytes apart, each instruction
        // covering half of every line: as non-temporal stores the pass took
        // 0.55 ms at 512 x 131072, as ordinary ones 0.24 ms.
        auto st4 = [&](float* p, const float* g) {
          const f4 w = f4{g[0], g[1], g[2], g[3]};
          if (NV == 4) __builtin_nontemporal_store(w, reinterpret_cast<f4*>(p));
          else *reinterpret_cast<f4*>(p) = w;
        };
#pragma unroll
        for (int h = 0; h < NV / 4; ++h) {
          st4(gce_s + j0 + 4 * h, gs + 4 * h);
          if (do_kl) st4(gkl + j0 + 4 * h, gk + 4 * h);
          if (do_tgrad) st4(gce_t + j0 + 4 * h, gt + 4 * h);
        }
      } else {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          if (j0 + i >= a.v) break;
          gce_s[j0 + i] = gs[i];
          if (do_kl) gkl[j0 + i] = gk[i];
          if (do_tgrad) gce_t[j0 + i] = gt[i];
        }
      }
    } else {
      if (whole) {
        *reinterpret_cast<typename VT::raw*>(srow + j0) = VT::pack(gs);
        if (do_tgrad) *reinterpret_cast<typename VT::raw*>(trow + j0) = VT::pack(gt);
      } else {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          if (j0 + i >= a.v) break;
          srow[j0 + i] = static_cast<LT>(gs[i]);
          if (do_tgrad) trow[j0 + i] = static_cast<LT>(gt[i]);
        }
      }
    }
  }
  if (SPLIT && !do_kl && a.grad_kl) {
    for (int64_t j = tid; j < a.v; j += TPB) gkl[j] = 0.f;
  }

  if (do_kl) {
    cross = block_sum<TPB>(cross, ssum);
    sum_pt = block_sum<TPB>(sum_pt, ssum);
    sum_d = block_sum<TPB>(sum_d, ssum);
  }
  if (tid == 0) {
    const float xy_s = ignored ? 0.f : a.xy_s[r];
    const double nll_s = ignored ? 0.0 : row_nll(ss, xy_s, alpha, a.v);
    float kl_row = 0.f;
    if (do_kl && !ignored) {
      const float t_sq = SPLIT ? a.t_sq : T * T;   // kl.rs:86
      kl_row = kl_from_sums(cross, sum_pt, sum_d, oTs - oTt, inv_t, false) * t_sq;
    }
    double nll_t = 0.0;
    const bool tce = SPLIT ? (!a.student_only && has_t) : (a.teacher_ce && has_t);
    if (tce && !ignored) nll_t = row_nll(st, a.xy_t[r], alpha, a.v);
    if (SPLIT) {
      a.ce_loss[r] = static_cast<float>(nll_s);
      if (tce) a.ce_loss[a.n_rows + r] = static_cast<float>(nll_t);
      if (a.row_kl) a.row_kl[r] = kl_row;
    } else {
      a.row_nll_s[r] = static_cast<float>(nll_s);
      a.row_nll_t[r] = static_cast<float>(nll_t);
      a.row_kl[r] = kl_row;
    }
  }
}

// Eight consecutive logits (16-byte aligned) as fp32, and eight gradients
// back in the storage type.
template <typename T>
__device__ __forceinline__ void load8(const T* p, float (&x)[8]);
template <>
__device__ __forceinline__ void load8(const float* p, float (&x)[8]) {
  const u32x4 a = reinterpret_cast<const u32x4*>(p)[0], b = reinterpret_cast<const u32x4*>(p)[1];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[i] = __uint_as_float(a[i]);
    x[4 + i] = __uint_as_float(b[i]);
  }
}
template <>
__device__ __forceinline__ void load8(const __bf16* p, float (&x)[8]) {
  Vec<__bf16>::unpack(*reinterpret_cast<const u32x4*>(p), x);
}
template <typename T>
__device__ __forceinline__ void store8(T* p, const float (&g)[8]);
template <>
__device__ __forceinline__ void store8(float* p, const float (&g)[8]) {
  reinterpret_cast<u32x4*>(p)[0] = u32x4{__float_as_uint(g[0]), __float_as_uint(g[1]),
                                         __float_as_uint(g[2]), __float_as_uint(g[3])};
  reinterpret_cast<u32x4*>(p)[1] = u32x4{__float_as_uint(g[4]), __float_as_uint(g[5]),
                                         __float_as_uint(g[6]), __float_as_uint(g[7])};
}
template <>
__device__ __forceinline__ void store8(__bf16* p, const float (&g)[8]) {
  *reinterpret_cast<u32x4*>(p) = Vec<__bf16>::pack(g);
}
// Streaming forms for data touched once (non-temporal hint on the access).
__device__ __forceinline__ void store8_nt(__bf16* p, const float (&g)[8]) {
  __builtin_nontemporal_store(Vec<__bf16>::pack(g), reinterpret_cast<u32x4*>(p));
}

// The half-tile maxima of one row pair (RowPassArgs::hmax_s / hmax_t), or
// 0 where the rows are stored as they are.
struct HalfRel {
  const float* ps;
  const float* pt;
  bool rs, rt;
  __device__ HalfRel(const RowPassArgs& a, int64_t r, bool teacher)
      : ps(a.hmax_s ? a.hmax_s + r * a.hmax_ld : nullptr),
        pt(teacher && a.hmax_t ? a.hmax_t + r * a.hmax_ld : nullptr),
        rs(a.hmax_s != nullptr),
        rt(teacher && a.hmax_t != nullptr) {}
  __device__ float s(int64_t col) const { return rs ? ps[2 * (col >> 7)] : 0.f; }
  __device__ float t(int64_t col) const { return rt ? pt[2 * (col >> 7)] : 0.f; }
};

// The row pass of distillation_loss, specialised on the logits type LT, the
// gradient type GT and whether the KL term (KL) and the teacher CE gradient
// (TG) are present. Same results as the unsplit row_pass_kernel, with the
// per-element work cut down for the bandwidth-bound case:
//  * the CE and KL weights are folded into the exponents,
//      w_s·p_s = 2^(x_s·log2e − lse_s·log2e + log2|w_s|), likewise kd·T·p_s^T,
//      kd·T·p_t^T and w_t·p_t, and Σp_t^T(x_t − x_s), Σp_t^T are formed from
//      kd·T·p_t^T and divided by kd·T once;
//  * the label column is fixed up by the one thread that holds it, and only
//    the last, partial group of a row checks column bounds;
//  * two 8-element groups per row and thread are in flight per iteration;
//  * an ignored row is a zero fill.
// Logits are read in LT (fp32, or bf16 only when the inputs are bf16 and
// the loss terms do not need fp32 logits; bf16 rows of the logits GEMM are
// relative to their half-tile maxima) and gradients written in GT, in place
// when grad_s is null.
template <typename LT, typename GT, bool KL, bool TG>
__global__ __launch_bounds__(kThreads) void row_pass_fused_kernel(RowPassArgs a) {
  __shared__ Stat sstat[kThreads / 64];
  __shared__ float ssum[kThreads / 64];
  constexpr int NV = 8;
  constexpr bool HT = KL || TG;   // the teacher row is read
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t y = a.labels[r];
  const int64_t v = a.v;
  const int nvec = static_cast<int>((v + NV - 1) / NV);
  const int nfull = static_cast<int>(v / NV);
  const LT* srow = static_cast<const LT*>(a.student) + r * a.ld;
  const LT* trow = HT ? static_cast<const LT*>(a.teacher) + r * (a.ld_t ? a.ld_t : a.ld) : nullptr;
  GT* gsrow = static_cast<GT*>(a.grad_s ? a.grad_s : a.student) + r * a.ld;
  GT* gtrow = TG ? static_cast<GT*>(a.grad_s ? a.grad_t : a.teacher) + r * a.ld : nullptr;

  // cross_entropy.rs:59, kl.rs:92: zero gradient and losses (also for a
  // label outside [0, V), which the host reports as an error).
  if (y == a.ignore_index || y < 0 || y >= v) {
    const float z[NV] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int vi = tid; vi < nvec; vi += kThreads) {
      store8(gsrow + static_cast<int64_t>(vi) * NV, z);
      if (TG) store8(gtrow + static_cast<int64_t>(vi) * NV, z);
    }
    if (tid == 0) {
      a.row_nll_s[r] = 0.f;
      a.row_nll_t[r] = 0.f;
      a.row_kl[r] = 0.f;
    }
    return;
  }

  const bool fm = a.fast_math;
  const float T = a.temperature;
  const float inv_t = rdiv(1.0f, T, fm);
  const float it2 = inv_t * kLog2e;
  const Stat ss = load_row_stats(a.stats_s + r * a.stats_ld, a.stats_tiles, it2, sstat);
  Stat st{-INFINITY, 0.f, 0.f, 0.f};
  if (HT || a.teacher_ce) st = load_row_stats(a.stats_t + r * a.stats_ld, a.stats_tiles_t, it2, sstat);
  // KL sums from a paired logits GEMM (kl_sums.h), each tile's taken to
  // the row's merged maxima and added.
  float2 xc = make_float2(0.f, 0.f);
  if (KL && a.cross != nullptr) {
    const float4* srow_s = a.stats_s + r * a.stats_ld;
    const float4* srow_t = a.stats_t + r * a.stats_ld;
    const float2* crow = a.cross + r * a.stats_ld;
    float px = 0.f, pd = 0.f;
    for (int64_t t = tid; t < a.stats_tiles_t; t += kThreads) {
      const float4 vs = srow_s[t], vt = srow_t[t];
      const float2 c = kl_rebase(crow[t], vs.x, vt.x, vs.z, vt.z, ss.m, st.m, inv_t);
      px += c.x;
      pd += c.y;
    }
    xc.x = block_sum(px, ssum);
    xc.y = block_sum(pd, ssum);
  }

  const double alpha = static_cast<double>(a.label_smoothing);
  const float lse1_s = ss.m + rlog(ss.d1, fm);
  const float lseT_s = ss.m * inv_t + rlog(ss.dT, fm);
  const float lse1_t = st.m + rlog(st.d1, fm);
  const float lseT_t = st.m * inv_t + rlog(st.dT, fm);
  const float eps = static_cast<float>(alpha / static_cast<double>(v));
  const float one_m_a = 1.0f - a.label_smoothing;
  const float ws = a.w_s, wt = a.w_t;
  const float gsc = a.kd * T;                              // kl.rs:85
  // w_s·p_s (w_s may be any sign; w_t, kd >= 0 are validated by the caller)
  const float ca = rlog2(fabsf(ws), fm) - lse1_s * kLog2e;
  const float sgn = ws < 0.f ? -1.f : 1.f;
  const float cb = KL ? rlog2(gsc, fm) - lseT_s * kLog2e : 0.f;   // kd·T·p_s^T
  const float cc = KL ? rlog2(gsc, fm) - lseT_t * kLog2e : 0.f;   // kd·T·p_t^T
  const float cd = TG ? rlog2(wt, fm) - lse1_t * kLog2e : 0.f;    // w_t·p_t
  const float k0 = -ws * eps, kt0 = -wt * eps;
  const float ky = ws * one_m_a, kyt = wt * one_m_a;
  // bf16 rows stored relative to their half-tile maxima (log2 units; the
  // launcher keeps such rows away from the KL cross term below, which needs
  // the logits themselves): scale 1 (1/T) instead of log2(e) (log2(e)/T),
  // and each 128-column half's maximum folded into the offsets.
  const HalfRel hr(a, r, HT);
  const float e1s = hr.rs ? 1.f : kLog2e, eTs = hr.rs ? inv_t : it2;
  const float e1t = hr.rt ? 1.f : kLog2e, eTt = hr.rt ? inv_t : it2;
  auto offs = [&](float hs, float ht) {
    return float4{fmaf(hs, kLog2e, ca), fmaf(hs, it2, cb), fmaf(ht, it2, cc), fmaf(ht, kLog2e, cd)};
  };

  float cross = 0.f, sum_c = 0.f, sum_d = 0.f;
  // Gradient of one element pair, without the label term.
  auto elem = [&](float xs, float xt, const float4& o, float& g, float& gt, float& cx, float& c,
                  float& d) {
    g = fmaf(sgn, __builtin_amdgcn_exp2f(fmaf(xs, e1s, o.x)), k0);
    if (KL) {
      const float b = __builtin_amdgcn_exp2f(fmaf(xs, eTs, o.y));
      c = __builtin_amdgcn_exp2f(fmaf(xt, eTt, o.z));
      d = b - c;
      g += d;
      cx = c * (xt - xs);
    }
    if (TG) gt = __builtin_amdgcn_exp2f(fmaf(xt, e1t, o.w)) + kt0;
  };
  auto compute = [&](int j0, const float (&xs)[NV], const float (&xt)[NV], float hs, float ht,
                     bool full) {
    float g[NV], gt[NV];
    const float4 o = offs(hs, ht);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const bool valid = full || j0 + i < v;
      float gi = 0.f, ti = 0.f, cx = 0.f, c = 0.f, d = 0.f;
      elem(xs[i], xt[i], o, gi, ti, cx, c, d);
      if (KL) {
        cross += valid ? cx : 0.f;
        sum_c += valid ? c : 0.f;
        sum_d += valid ? d : 0.f;
      }
      g[i] = valid ? gi : 0.f;
      gt[i] = valid ? ti : 0.f;
    }
    store8(gsrow + j0, g);
    if (TG) store8(gtrow + j0, gt);
  };
  // The label column's logits, read by its owner before the row is
  // overwritten (the gradient may go in place).
  const bool owner = tid == (y / NV) % kThreads;
  float xs_y = 0.f, xt_y = 0.f;
  if (owner) {
    xs_y = static_cast<float>(srow[y]);
    if (HT) xt_y = static_cast<float>(trow[y]);
  }
  // Offsets within a row fit 32 bits (V < 2^31). Every thread has at least
  // nk full groups; those run software pipelined over two register buffers
  // with a uniform trip count, so each group's loads are in flight while the
  // previous group computes and every wait covers loads only.
  constexpr int kStep = kThreads * NV;
  const int jfull = nfull * NV;
  const int nk = nfull / kThreads;
  int j = tid * NV;
  if (nk > 0) {
    // Both buffers are loaded before the loop and each is refilled right
    // after its group is stored, so every compute finds its loads issued
    // one compute earlier on all paths into it.
    float as[NV], at[NV], bs[NV], bt[NV];
    const int jb0 = nk > 1 ? j + kStep : j;
    load8(srow + j, as);
    if (HT) load8(trow + j, at);
    float ahs = hr.s(j), aht = hr.t(j);
    load8(srow + jb0, bs);
    if (HT) load8(trow + jb0, bt);
    float bhs = hr.s(jb0), bht = hr.t(jb0);
    int k = 0;
    for (; k + 1 < nk; k += 2) {
      compute(j, as, at, ahs, aht, true);
      const int ja = k + 2 < nk ? j + 2 * kStep : j;   // re-read when past the end
      load8(srow + ja, as);
      if (HT) load8(trow + ja, at);
      ahs = hr.s(ja);
      aht = hr.t(ja);
      compute(j + kStep, bs, bt, bhs, bht, true);
      const int jb = k + 3 < nk ? j + 3 * kStep : j;
      load8(srow + jb, bs);
      if (HT) load8(trow + jb, bt);
      bhs = hr.s(jb);
      bht = hr.t(jb);
      j += 2 * kStep;
    }
    if (k < nk) {
      compute(j, as, at, ahs, aht, true);
      j += kStep;
    }
  }
  for (; j < nvec * NV; j += kStep) {
    float s0[NV], t0[NV];
    load8(srow + j, s0);
    if (HT) load8(trow + j, t0);
    const float hs0 = hr.s(j), ht0 = hr.t(j);
    if (j < jfull) compute(j, s0, t0, hs0, ht0, true);
    else compute(j, s0, t0, hs0, ht0, false);
  }
  // The label column: its owner (the thread that wrote it, so in program
  // order) rewrites it with the −(1−α)·w term included.
  if (owner) {
    float gy = 0.f, ty = 0.f, cx = 0.f, c = 0.f, d = 0.f;
    elem(xs_y, xt_y, offs(hr.s(y), hr.t(y)), gy, ty, cx, c, d);
    gsrow[y] = static_cast<GT>(gy - ky);
    if (TG) gtrow[y] = static_cast<GT>(ty - kyt);
  }

  if (KL && a.cross == nullptr) {
    cross = block_sum(cross, ssum);
    sum_c = block_sum(sum_c, ssum);
    sum_d = block_sum(sum_d, ssum);
  }
  if (tid == 0) {
    a.row_nll_s[r] = static_cast<float>(row_nll(ss, a.xy_s[r], alpha, v));
    float kl_row = 0.f;
    if (KL && a.cross != nullptr)
      kl_row = kl_paired(xc, ss, st, inv_t, fm) * (T * T);
    else if (KL)   // offsets as used: p_s^T·kd·T = 2^(x·eTs + cb + ...), p_t^T likewise with cc
      kl_row = kl_from_sums(cross, sum_c, sum_d, cc - cb, inv_t, fm) * (T * T);
    a.row_kl[r] = kl_row;
    a.row_nll_t[r] = a.teacher_ce ? static_cast<float>(row_nll(st, a.xy_t[r], alpha, v)) : 0.f;
  }
}

// ------------------------------------------------- chunked row pass (paired)
// With the KL cross term from a paired logits GEMM nothing in the row pass
// needs a reduction over a row: every loss term comes from the GEMM's tile
// statistics. The pass then splits into a per-row kernel that merges the
// statistics, writes the row's losses and four exponent constants, and an
// elementwise gradient kernel over (row, 8192-column chunk) blocks, so that
// consecutive workgroups stream consecutive memory (the row-per-workgroup
// kernel keeps ~2000 rows 256 KB apart open at once).
//   consts[r] = {ca, cb, cc, cd}: log2|w_s| - lse1_s·log2e,
//   log2(kd·T) - lseT_s·log2e, log2(kd·T) - lseT_t·log2e, log2(w_t) - lse1_t·log2e.
template <bool KL, bool TG>
__global__ __launch_bounds__(kThreads) void row_consts_kernel(RowPassArgs a) {
  // One wave per row, kThreads / 64 rows per workgroup: each lane merges
  // every 64th tile entry, then a butterfly over the wave. No LDS, no
  // barrier. The teacher's KL cross partials are merged with its
  // statistics, rescaled like Σe^((x-max)/T).
  const int lane = threadIdx.x & 63;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
  if (r >= a.n_rows) return;
  const int64_t y = a.labels[r];
  if (y == a.ignore_index || y < 0 || y >= a.v) {   // cross_entropy.rs:59, kl.rs:92
    if (lane == 0) {
      a.row_nll_s[r] = 0.f;
      a.row_nll_t[r] = 0.f;
      a.row_kl[r] = 0.f;
      a.row_consts[r] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    return;
  }
  const bool fm = a.fast_math;
  const float T = a.temperature;
  const float inv_t = rdiv(1.0f, T, fm);
  const float it2 = inv_t * kLog2e;
  Stat ss{-INFINITY, 0.f, 0.f, 0.f}, st{-INFINITY, 0.f, 0.f, 0.f};
  float2 xc = make_float2(0.f, 0.f);
  const float4* rs = a.stats_s + r * a.stats_ld;
  const bool teacher = KL || TG || a.teacher_ce;
  const float4* rt = a.stats_t + r * a.stats_ld;
  // Without a paired GEMM's cross partials (fp32 logits), the KL cross sums
  // come from row_grad_f32_kernel's blocks instead.
  const bool xk = KL && a.cross != nullptr;
  const float2* rc = xk ? a.cross + r * a.stats_ld : nullptr;
  const int64_t nt = a.stats_tiles > a.stats_tiles_t ? a.stats_tiles : a.stats_tiles_t;
  // The row's two maxima first, then every tile's entries taken to them once
  // and added (no pairwise merges). kPer entries per lane are loaded at a
  // time; a missing entry is {-inf, 0, 0, 0}, which adds nothing. Rows of up
  // to 64·kPer tiles (V <= 131072) keep their entries in registers between
  // the two steps; longer rows read them again.
  constexpr int kPer = 8;
  const float4 none = make_float4(-INFINITY, 0.f, 0.f, 0.f);
  float4 vs[kPer], vt[kPer];
  float2 vc[kPer];
  auto load = [&](int64_t t0) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int64_t t = t0 + i * 64 + lane;
      vs[i] = t < a.stats_tiles ? rs[t] : none;
      const bool tok = teacher && t < a.stats_tiles_t;
      vt[i] = tok ? rt[t] : none;
      vc[i] = xk && tok ? rc[t] : make_float2(0.f, 0.f);
    }
  };
  const bool one = nt <= 64 * kPer;
  float ms = -INFINITY, mt = -INFINITY;
  for (int64_t t0 = 0; t0 < nt; t0 += 64 * kPer) {
    load(t0);
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      ms = fmaxf(ms, vs[i].x);
      mt = fmaxf(mt, vt[i].x);
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    ms = fmaxf(ms, __shfl_xor(ms, o));
    mt = fmaxf(mt, __shfl_xor(mt, o));
  }
  ss.m = ms;
  st.m = mt;
  for (int64_t t0 = 0; t0 < nt; t0 += 64 * kPer) {
    if (!one) load(t0);
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      if (vs[i].x != -INFINITY) {
        ss.d1 = fmaf(vs[i].y, __builtin_amdgcn_exp2f((vs[i].x - ms) * kLog2e), ss.d1);
        ss.dT = fmaf(vs[i].z, __builtin_amdgcn_exp2f((vs[i].x - ms) * it2), ss.dT);
        ss.sx += vs[i].w;
      }
      if (vt[i].x != -INFINITY) {
        st.d1 = fmaf(vt[i].y, __builtin_amdgcn_exp2f((vt[i].x - mt) * kLog2e), st.d1);
        st.dT = fmaf(vt[i].z, __builtin_amdgcn_exp2f((vt[i].x - mt) * it2), st.dT);
        st.sx += vt[i].w;
      }
      if (xk) {
        const float2 c = kl_rebase(vc[i], vs[i].x, vt[i].x, vs[i].z, vt[i].z, ms, mt, inv_t);
        xc.x += c.x;
        xc.y += c.y;
      }
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    ss.d1 += __shfl_xor(ss.d1, o);
    ss.dT += __shfl_xor(ss.dT, o);
    ss.sx += __shfl_xor(ss.sx, o);
    st.d1 += __shfl_xor(st.d1, o);
    st.dT += __shfl_xor(st.dT, o);
    st.sx += __shfl_xor(st.sx, o);
    if (xk) {
      xc.x += __shfl_xor(xc.x, o);
      xc.y += __shfl_xor(xc.y, o);
    }
  }
  if (lane == 0) {
    const double alpha = static_cast<double>(a.label_smoothing);
    const float lse1_s = ss.m + rlog(ss.d1, fm);
    const float lseT_s = ss.m * inv_t + rlog(ss.dT, fm);
    const float lse1_t = st.m + rlog(st.d1, fm);
    const float lseT_t = st.m * inv_t + rlog(st.dT, fm);
    const float gsc = a.kd * T;                              // kl.rs:85
    float4 k;
    k.x = rlog2(fabsf(a.w_s), fm) - lse1_s * kLog2e;
    k.y = KL ? rlog2(gsc, fm) - lseT_s * kLog2e : 0.f;
    k.z = KL ? rlog2(gsc, fm) - lseT_t * kLog2e : 0.f;
    k.w = TG ? rlog2(a.w_t, fm) - lse1_t * kLog2e : 0.f;
    a.row_consts[r] = k;
    a.row_nll_s[r] = static_cast<float>(row_nll(ss, a.xy_s[r], alpha, a.v));
    // Without the GEMM's KL partials, row_kl_kernel forms the row's KL
    // from the gradient blocks' sums and these constants.
    a.row_kl[r] = xk ? kl_paired(xc, ss, st, inv_t, fm) * (T * T) : 0.f;
    a.row_nll_t[r] = a.teacher_ce ? static_cast<float>(row_nll(st, a.xy_t[r], alpha, a.v)) : 0.f;
  }
}

// Gradient of one (row, chunk) block, in place in bf16 (the paired layout):
// student g = w_s·((p_s − α/V) − [j=y](1−α)) + kd·T·(p_s^T − p_t^T),
// teacher g = w_t·((p_t − α/V) − [j=y](1−α)) (when TG).
// Small blocks: 128 threads, one 8-element vector each (1024 columns). A
// block's loads are few, but many blocks fit (51 VGPRs), and the rows the
// chip streams at once stay close together: measured 1.40 ms at the
// BT=8192, V=131072 workload, against 1.42 ms for 256 threads x 1 vector,
// 1.52 ms for 256 x 2, 1.57 ms for 256 x 4 (84 VGPRs, five waves per SIMD)
// and 1.45 ms for 64 x 1.
constexpr int kChunkVec = 1;                             // 8-element vectors per thread
constexpr int kGradThreads = 128;
constexpr int kChunk = kGradThreads * 8 * kChunkVec;     // columns per workgroup
template <bool KL, bool TG, int TT>
__global__ __launch_bounds__(kGradThreads) void row_grad_kernel(RowPassArgs a, int64_t chunks) {
  // TT: the teacher rows' form. 0: bf16 relative to their half-tile maxima
  // (the paired GEMM's rows, pitch ld, gradient in place); 1 (fp32) or 2
  // (bf16): logits as they are, read in place at pitch ld_t (Precomputed
  // teacher logits, or a Separate teacher's), the gradient (TG) to the bf16
  // rows grad_t at pitch ld.
  constexpr bool kRaw = TT != 0;
  constexpr int NV = 8;
  const int64_t r = blockIdx.x / chunks;
  const int64_t c0 = (blockIdx.x - r * chunks) * kChunk;
  const int tid = threadIdx.x;
  const int64_t y = a.labels[r];
  const int64_t v = a.v;
  __bf16* srow = static_cast<__bf16*>(a.student) + r * a.ld;
  __bf16* trow = (KL || TG) && TT == 0 ? static_cast<__bf16*>(a.teacher) + r * a.ld : nullptr;
  const float* trowf = TT == 1 ? static_cast<const float*>(a.teacher) + r * a.ld_t : nullptr;
  const __bf16* trowh = TT == 2 ? static_cast<const __bf16*>(a.teacher) + r * a.ld_t : nullptr;
  __bf16* gtrow = kRaw ? (TG ? static_cast<__bf16*>(a.grad_t) + r * a.ld : nullptr) : trow;
  if (y == a.ignore_index || y < 0 || y >= v) {   // zero gradient rows
    const float z[NV] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < kChunkVec; ++q) {
      const int64_t j = c0 + (static_cast<int64_t>(q) * kGradThreads + tid) * NV;
      if (j < v) {
        store8_nt(srow + j, z);
        if (TG) store8_nt(gtrow + j, z);
      }
    }
    return;
  }
  const float4 k = a.row_consts[r];
  const float inv_t = rdiv(1.0f, a.temperature, a.fast_math);
  const float it2 = kLog2e * inv_t;
  const float eps = static_cast<float>(static_cast<double>(a.label_smoothing) / static_cast<double>(v));
  const float one_m_a = 1.0f - a.label_smoothing;
  const float sgn = a.w_s < 0.f ? -1.f : 1.f;
  const float k0 = -a.w_s * eps, kt0 = -a.w_t * eps;
  // Both rows are stored relative to their half-tile maxima, in log2 units
  // (LogitStatsArgs::hmax): each 128-column half's maximum is folded into
  // the exponent offsets, and the T terms scale by 1/T. fp32 teacher rows
  // (kRaw) are logits as they are: scale log2(e)/T, no maximum.
  auto offs = [&](float hs, float ht) {
    return float4{fmaf(hs, kLog2e, k.x), fmaf(hs, it2, k.y), kRaw ? k.z : fmaf(ht, it2, k.z),
                  kRaw ? k.w : fmaf(ht, kLog2e, k.w)};
  };
  const float eTt = kRaw ? it2 : inv_t;
  const float e1t = kRaw ? kLog2e : 1.f;
  auto elem = [&](float xs, float xt, const float4& o, float& g, float& gt) {
    g = fmaf(sgn, __builtin_amdgcn_exp2f(xs + o.x), k0);
    if (KL) g += __builtin_amdgcn_exp2f(fmaf(xs, inv_t, o.y)) - __builtin_amdgcn_exp2f(fmaf(xt, eTt, o.z));
    if (TG) gt = __builtin_amdgcn_exp2f(fmaf(xt, e1t, o.w)) + kt0;
  };
  // The label column's logits, read by the thread that writes that column.
  const int64_t yl = y - c0;
  const bool owner = yl >= 0 && yl < kChunk && tid == (yl / NV) % kGradThreads;
  float xs_y = 0.f, xt_y = 0.f;
  if (owner) {
    xs_y = static_cast<float>(srow[y]);
    if (TT == 1) xt_y = trowf[y];
    else if (TT == 2) xt_y = static_cast<float>(trowh[y]);
    else if (KL || TG) xt_y = static_cast<float>(trow[y]);
  }
  // Half-tile maxima, loaded first (ahead of the logits, so that no wait
  // comes between): the student's and the teacher's maxima of a half are
  // adjacent, one float2 per lane (lanes of one half share it). A lane past
  // the row's end reads the row's last half, which it does not use.
  float hs[kChunkVec], ht[kChunkVec];
#pragma unroll
  for (int q = 0; q < kChunkVec; ++q) {
    const int64_t hk = (c0 + (static_cast<int64_t>(q) * kGradThreads + tid) * NV) >> 7;
    const int64_t hl = (v - 1) >> 7;
    const float2 m = *reinterpret_cast<const float2*>(a.hmax_s + r * a.hmax_ld + 2 * (hk < hl ? hk : hl));
    hs[q] = m.x;
    ht[q] = m.y;
  }
  // The loads stay packed (bf16 pairs) until their group is computed. An
  // fp32 teacher vector is two 16-byte loads, or single elements where it
  // would pass the row's end (its pitch is only a multiple of 4).
  u32x4 rs[kChunkVec], rt[kChunkVec], rt2[kChunkVec];
#pragma unroll
  for (int q = 0; q < kChunkVec; ++q) {
    const int64_t j = c0 + (static_cast<int64_t>(q) * kGradThreads + tid) * NV;
    if (j < v) {
      rs[q] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(srow + j));
      if (TT == 1) {
        if (j + NV <= v) {
          rt[q] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(trowf + j));
          rt2[q] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(trowf + j) + 1);
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            rt[q][i] = j + i < v ? __float_as_uint(trowf[j + i]) : 0u;
            rt2[q][i] = j + 4 + i < v ? __float_as_uint(trowf[j + 4 + i]) : 0u;
          }
        }
      } else if (TT == 2) {
        // 8 bf16 logits a 16-byte vector; single elements where it would
        // pass the row's end (the pitch is only a multiple of 8 elements)
        if (j + NV <= v) {
          rt[q] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(trowh + j));
        } else {
          const uint16_t* h16 = reinterpret_cast<const uint16_t*>(trowh + j);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t lo = j + 2 * i < v ? h16[2 * i] : 0u;
            const uint32_t hi = j + 2 * i + 1 < v ? h16[2 * i + 1] : 0u;
            rt[q][i] = lo | (hi << 16);
          }
        }
      } else if (KL || TG) {
        rt[q] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(trow + j));
      }
    }
  }
#pragma unroll
  for (int q = 0; q < kChunkVec; ++q) {
    const int64_t j = c0 + (static_cast<int64_t>(q) * kGradThreads + tid) * NV;
    if (j >= v) continue;
    float xs[NV], xt[NV] = {};
    Vec<__bf16>::unpack(rs[q], xs);
    if (TT == 1) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xt[i] = __uint_as_float(rt[q][i]);
        xt[4 + i] = __uint_as_float(rt2[q][i]);
      }
    } else if (KL || TG) {
      Vec<__bf16>::unpack(rt[q], xt);
    }
    float g[NV], gt[NV];
    const float4 o = offs(hs[q], ht[q]);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      float gi = 0.f, ti = 0.f;
      elem(xs[i], xt[i], o, gi, ti);
      const bool valid = j + i < v;
      g[i] = valid ? gi : 0.f;
      gt[i] = valid ? ti : 0.f;
    }
    store8_nt(srow + j, g);
    if (TG) store8_nt(gtrow + j, gt);
  }
  if (owner) {   // the label term, after this thread's own store of that column
    float gy = 0.f, ty = 0.f;
    elem(xs_y, xt_y, offs(hs[0], ht[0]), gy, ty);   // column y is in this thread's vector
    srow[y] = static_cast<__bf16>(gy - a.w_s * one_m_a);
    if (TG) gtrow[y] = static_cast<__bf16>(ty - a.w_t * one_m_a);
  }
}

// The same chunked pass over fp32 logits (fp32 inputs; bf16 inputs whose
// KL term needs fp32 logits), where the KL cross term is not available from
// the GEMM: each (row, kF32Chunk-column) block also writes its share of the
// three KL sums of row_pass_fused_kernel,
//   kl_part[r * chunks + c] = {Σ kd·T·p_t^T·(x_t − x_s), Σ kd·T·p_t^T,
//                              Σ kd·T·(p_s^T − p_t^T), 0},
// and row_kl_kernel adds a row's shares. Gradients go in place (GT float)
// or to the separate gradient rows grad_s/grad_t; the teacher rows may have
// their own pitch (Precomputed logits read in place). One wave per block,
// one 16-byte vector (4 logits) of each row per thread, non-temporal loads
// and stores: measured at the fp32 workloads (BT x V = 2048 x 32000,
// 4096 x 32000, 4096 x 65536, two alternating passes) 0.174 / 0.338 /
// 0.520 ms per pass, against 0.189 / 0.400 / 0.585 ms with two vectors per
// row and thread and ordinary accesses, 0.212 / 0.418 / 0.613 ms with two
// vectors and non-temporal accesses, 0.174 / 0.364 / 0.553 ms with one
// vector and ordinary accesses. (The paired bf16 pass moves one 16-byte
// vector per row and thread too, non-temporally.)
constexpr int kF32Threads = 64;
constexpr int kF32Vec = 1;                                 // NV-element vectors per thread
constexpr int kF32NV = 4;
constexpr bool kF32Nt = true;
constexpr int kF32Chunk = kF32Threads * kF32NV * kF32Vec;  // columns per workgroup
// N gradient values to p (aligned to their size), as fp32 or packed bf16.
template <bool NT, int N>
__device__ __forceinline__ void store_vec(float* p, const float (&g)[N]) {
#pragma unroll
  for (int h = 0; h < N / 4; ++h) {
    const u32x4 w = u32x4{__float_as_uint(g[4 * h]), __float_as_uint(g[4 * h + 1]),
                          __float_as_uint(g[4 * h + 2]), __float_as_uint(g[4 * h + 3])};
    if (NT) __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(p) + h);
    else reinterpret_cast<u32x4*>(p)[h] = w;
  }
}
template <bool NT, int N>
__device__ __forceinline__ void store_vec(__bf16* p, const float (&g)[N]) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  uint32_t w[N / 2];
#pragma unroll
  for (int i = 0; i < N / 2; ++i)
    w[i] = __builtin_bit_cast(uint32_t, bf16x2{static_cast<__bf16>(g[2 * i]),
                                               static_cast<__bf16>(g[2 * i + 1])});
  if constexpr (N == 8) {
    const u32x4 v = u32x4{w[0], w[1], w[2], w[3]};
    if (NT) __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
    else *reinterpret_cast<u32x4*>(p) = v;
  } else {
    static_assert(N == 4, "4 or 8 values");
    const u32x2 v = u32x2{w[0], w[1]};
    if (NT) __builtin_nontemporal_store(v, reinterpret_cast<u32x2*>(p));
    else *reinterpret_cast<u32x2*>(p) = v;
  }
}
template <bool NT>
__device__ __forceinline__ u32x4 load_vec(const float* p) {
  if (NT) return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return *reinterpret_cast<const u32x4*>(p);
}
template <typename GT, bool KL, bool TG>
__global__ __launch_bounds__(kF32Threads) void row_grad_f32_kernel(RowPassArgs a, int64_t chunks) {
  constexpr int NV = kF32NV;
  constexpr int NH = NV / 4;   // 16-byte loads per row and thread
  __shared__ float sred[3][kF32Threads / 64];
  const int64_t r = blockIdx.x / chunks;
  const int64_t ci = blockIdx.x - r * chunks;
  const int64_t c0 = ci * kF32Chunk;
  const int tid = threadIdx.x;
  const int64_t y = a.labels[r];
  const int64_t v = a.v;
  const float* srow = static_cast<const float*>(a.student) + r * a.ld;
  const float* trow =
      (KL || TG) ? static_cast<const float*>(a.teacher) + r * (a.ld_t ? a.ld_t : a.ld) : nullptr;
  GT* gsrow = static_cast<GT*>(a.grad_s ? a.grad_s : a.student) + r * a.ld;
  GT* gtrow = TG ? static_cast<GT*>(a.grad_s ? a.grad_t : a.teacher) + r * a.ld : nullptr;
  auto col = [&](int q) { return c0 + (static_cast<int64_t>(q) * kF32Threads + tid) * NV; };
  if (y == a.ignore_index || y < 0 || y >= v) {   // zero gradient rows, no KL
    float z[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) z[i] = 0.f;
#pragma unroll
    for (int q = 0; q < kF32Vec; ++q) {
      const int64_t j = col(q);
      if (j < v) {
        store_vec<kF32Nt>(gsrow + j, z);
        if (TG) store_vec<kF32Nt>(gtrow + j, z);
      }
    }
    if (KL && tid == 0) a.kl_part[r * chunks + ci] = make_float4(0.f, 0.f, 0.f, 0.f);
    return;
  }
  const float4 k = a.row_consts[r];
  const float it2 = kLog2e * rdiv(1.0f, a.temperature, a.fast_math);
  const float eps = static_cast<float>(static_cast<double>(a.label_smoothing) / static_cast<double>(v));
  const float one_m_a = 1.0f - a.label_smoothing;
  const float sgn = a.w_s < 0.f ? -1.f : 1.f;
  const float k0 = -a.w_s * eps, kt0 = -a.w_t * eps;
  // Gradient of one element pair without the label term; c = kd·T·p_t^T,
  // d = kd·T·(p_s^T − p_t^T).
  auto elem = [&](float xs, float xt, float& g, float& gt, float& c, float& d) {
    g = fmaf(sgn, __builtin_amdgcn_exp2f(fmaf(xs, kLog2e, k.x)), k0);
    if (KL) {
      c = __builtin_amdgcn_exp2f(fmaf(xt, it2, k.z));
      d = __builtin_amdgcn_exp2f(fmaf(xs, it2, k.y)) - c;
      g += d;
    }
    if (TG) gt = __builtin_amdgcn_exp2f(fmaf(xt, kLog2e, k.w)) + kt0;
  };
  // The label column's logits, read by the thread that writes that column.
  const int64_t yl = y - c0;
  const bool owner = yl >= 0 && yl < kF32Chunk && tid == (yl / NV) % kF32Threads;
  float xs_y = 0.f, xt_y = 0.f;
  if (owner) {
    xs_y = srow[y];
    if (KL || TG) xt_y = trow[y];
  }
  u32x4 rs[kF32Vec][NH], rt[kF32Vec][NH];
#pragma unroll
  for (int q = 0; q < kF32Vec; ++q) {
    const int64_t j = col(q);
    if (j < v) {
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        rs[q][h] = load_vec<kF32Nt>(srow + j + 4 * h);
        if (KL || TG) rt[q][h] = load_vec<kF32Nt>(trow + j + 4 * h);
      }
    }
  }
  float cross = 0.f, sum_c = 0.f, sum_d = 0.f;
#pragma unroll
  for (int q = 0; q < kF32Vec; ++q) {
    const int64_t j = col(q);
    if (j >= v) continue;
    float g[NV], gt[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const float xs = __uint_as_float(rs[q][i >> 2][i & 3]);
      const float xt = (KL || TG) ? __uint_as_float(rt[q][i >> 2][i & 3]) : 0.f;
      float gi = 0.f, ti = 0.f, c = 0.f, d = 0.f;
      elem(xs, xt, gi, ti, c, d);
      const bool valid = j + i < v;
      if (KL) {
        cross += valid ? c * (xt - xs) : 0.f;
        sum_c += valid ? c : 0.f;
        sum_d += valid ? d : 0.f;
      }
      g[i] = valid ? gi : 0.f;
      gt[i] = valid ? ti : 0.f;
    }
    store_vec<kF32Nt>(gsrow + j, g);
    if (TG) store_vec<kF32Nt>(gtrow + j, gt);
  }
  if (owner) {   // the label term, after this thread's own store of that column
    float gy = 0.f, ty = 0.f, c = 0.f, d = 0.f;
    elem(xs_y, xt_y, gy, ty, c, d);
    gsrow[y] = static_cast<GT>(gy - a.w_s * one_m_a);
    if (TG) gtrow[y] = static_cast<GT>(ty - a.w_t * one_m_a);
  }
  if (KL) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      cross += __shfl_xor(cross, o);
      sum_c += __shfl_xor(sum_c, o);
      sum_d += __shfl_xor(sum_d, o);
    }
    if ((tid & 63) == 0) {
      sred[0][tid >> 6] = cross;
      sred[1][tid >> 6] = sum_c;
      sred[2][tid >> 6] = sum_d;
    }
    __syncthreads();
    if (tid == 0) {
      float x = 0.f, sm = 0.f, sd = 0.f;
#pragma unroll
      for (int w = 0; w < kF32Threads / 64; ++w) {
        x += sred[0][w];
        sm += sred[1][w];
        sd += sred[2][w];
      }
      a.kl_part[r * chunks + ci] = make_float4(x, sm, sd, 0.f);
    }
  }
}

// KL_row·T² of every non-ignored row from its gradient blocks' sums and the
// exponent offsets of row_consts_kernel (kl_from_sums, as in
// row_pass_fused_kernel). One wave per row: lanes take every 64th block,
// then a butterfly.
__global__ __launch_bounds__(kThreads) void row_kl_kernel(RowPassArgs a, int64_t chunks) {
  const int lane = threadIdx.x & 63;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
  if (r >= a.n_rows) return;
  const int64_t y = a.labels[r];
  if (y == a.ignore_index || y < 0 || y >= a.v) return;   // row_kl is already 0
  const float4* p = a.kl_part + r * chunks;
  float x = 0.f, s = 0.f, d = 0.f;
  for (int64_t c = lane; c < chunks; c += 64) {
    const float4 q = p[c];
    x += q.x;
    s += q.y;
    d += q.z;
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    x += __shfl_xor(x, o);
    s += __shfl_xor(s, o);
    d += __shfl_xor(d, o);
  }
  if (lane == 0) {
    const bool fm = a.fast_math;
    const float T = a.temperature;
    const float inv_t = rdiv(1.0f, T, fm);
    // the offsets the gradient blocks used: p_s^T = 2^(x·log2(e)/T + k.y),
    // p_t^T = 2^(x·log2(e)/T + k.z), both scaled by kd·T
    const float4 k = a.row_consts[r];
    a.row_kl[r] = kl_from_sums(x, s, d, k.z - k.y, inv_t, fm) * (T * T);
  }
}

// ------------------------------------------------------------------ row stats
template <int TPB = kThreads>
__device__ float block_max(float v, float* scratch) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) scratch[wave] = v;
  __syncthreads();
  float r = scratch[0];
#pragma unroll
  for (int w = 1; w < TPB / 64; ++w) r = fmaxf(r, scratch[w]);
  return r;
}

// Per-row statistics {max, Σe^(x-max), Σe^((x-max)/T), Σx} of rows the GEMM
// did not produce. ONLINE: one read, each element merged into running
// statistics (two exponentials per statistic); otherwise a max pass, then a
// pass summing e^(x-max) and e^((x-max)/T) (the second read of a row mostly
// hits the cache).
template <typename ST, typename DT, bool ONLINE>
__global__ __launch_bounds__(kThreads) void row_stats_kernel(RowStatsArgs a) {
  __shared__ Stat sstat[kThreads / 64];
  __shared__ float sred[kThreads / 64];
  const int64_t r = blockIdx.x;
  const ST* src = static_cast<const ST*>(a.src) + r * a.lds;
  DT* dst = a.dst ? static_cast<DT*>(a.dst) + r * a.ldd : nullptr;
  const float it2 = a.inv_t * kLog2e;
  Stat s{-INFINITY, 0.f, 0.f, 0.f};
  if constexpr (ONLINE) {
    for (int64_t j = threadIdx.x; j < a.v; j += kThreads) {
      const float x = static_cast<float>(src[j]);
      if (dst) dst[j] = static_cast<DT>(x);
      s = merge(s, Stat{x, 1.f, 1.f, x}, it2);
    }
    s = block_merge(s, it2, sstat);
  } else {
    float m = -INFINITY, sx = 0.f;
    for (int64_t j = threadIdx.x; j < a.v; j += kThreads) {
      const float x = static_cast<float>(src[j]);
      if (dst) dst[j] = static_cast<DT>(x);
      m = fmaxf(m, x);
      sx += x;
    }
    m = block_max(m, sred);
    const float o1 = -m * kLog2e, oT = -m * it2;
    float d1 = 0.f, dT = 0.f;
    for (int64_t j = threadIdx.x; j < a.v; j += kThreads) {
      const float x = static_cast<float>(src[j]);
      d1 += __builtin_amdgcn_exp2f(fmaf(x, kLog2e, o1));
      dT += __builtin_amdgcn_exp2f(fmaf(x, it2, oT));
    }
    s.m = m;
    s.sx = block_sum(sx, sred);
    s.d1 = block_sum(d1, sred);
    s.dT = block_sum(dT, sred);
  }
  if (dst)
    for (int64_t j = a.v + threadIdx.x; j < a.ldd; j += kThreads) dst[j] = static_cast<DT>(0.f);
  if (threadIdx.x == 0) {
    a.stats[r * a.stats_ld] = make_float4(s.m, s.d1, s.dT, s.sx);
    if (a.labels) {
      const int64_t y = a.labels[a.label_rows > 0 ? r % a.label_rows : r];
      if (y != a.ignore_index && y >= 0 && y < a.v) a.xy[r] = static_cast<float>(src[y]);
    }
  }
}

// The chunk-launcher slot's statistics of whole rows (no converted copy):
// two passes over the row, max then the exponential sums, by 1024 threads,
// with 16-byte loads where every row is 16-byte aligned. (With 256 threads
// and single-element loads the slot ran at 1.0-2.0 TB/s at 512-1024 rows.)
constexpr int kWideThreads = 1024;
template <typename ST, bool VEC>
__global__ __launch_bounds__(kWideThreads) void row_stats_wide_kernel(RowStatsArgs a) {
  __shared__ float sred[kWideThreads / 64];
  const int64_t r = blockIdx.x;
  const ST* src = static_cast<const ST*>(a.src) + r * a.lds;
  const float it2 = a.inv_t * kLog2e;
  using VT = Vec<ST>;
  constexpr int NV = VT::N;
  const int64_t nfull = VEC ? a.v / NV : 0;
  auto each = [&](auto&& f) {
    if constexpr (VEC) {
      for (int64_t q = threadIdx.x; q < nfull; q += kWideThreads) {
        float x[NV];
        VT::unpack(*reinterpret_cast<const typename VT::raw*>(src + q * NV), x);
#pragma unroll
        for (int i = 0; i < NV; ++i) f(x[i]);
      }
    }
    for (int64_t j = nfull * NV + threadIdx.x; j < a.v; j += kWideThreads)
      f(static_cast<float>(src[j]));
  };
  float m = -INFINITY, sx = 0.f;
  each([&](float x) {
    m = fmaxf(m, x);
    sx += x;
  });
  m = block_max<kWideThreads>(m, sred);
  const float o1 = -m * kLog2e, oT = -m * it2;
  float d1 = 0.f, dT = 0.f;
  each([&](float x) {
    d1 += __builtin_amdgcn_exp2f(fmaf(x, kLog2e, o1));
    dT += __builtin_amdgcn_exp2f(fmaf(x, it2, oT));
  });
  sx = block_sum<kWideThreads>(sx, sred);
  d1 = block_sum<kWideThreads>(d1, sred);
  dT = block_sum<kWideThreads>(dT, sred);
  if (threadIdx.x == 0) {
    a.stats[r * a.stats_ld] = make_float4(m, d1, dT, sx);
    if (a.labels) {
      const int64_t y = a.labels[a.label_rows > 0 ? r % a.label_rows : r];
      if (y != a.ignore_index && y >= 0 && y < a.v) a.xy[r] = static_cast<float>(src[y]);
    }
  }
}

// Segmented two-pass statistics: one workgroup per (row, 8192-column
// segment); each thread holds its 32 columns in registers, so the max pass
// and the sum pass read HBM once.
constexpr int kSegCols = 8192;
constexpr int kSegPer = kSegCols / kThreads;   // 32 columns per thread
template <typename ST, typename DT, bool VEC, bool ONLINE>
__global__ __launch_bounds__(kThreads) void row_stats_seg_kernel(RowStatsArgs a, int64_t nseg) {
  __shared__ float sred[kThreads / 64];
  __shared__ Stat sstat[kThreads / 64];
  const int64_t r = blockIdx.x / nseg;
  const int64_t sg = blockIdx.x - r * nseg;
  const int64_t c0 = sg * kSegCols;
  const ST* src = static_cast<const ST*>(a.src) + r * a.lds;
  DT* dst = a.dst ? static_cast<DT*>(a.dst) + r * a.ldd : nullptr;
  const float it2 = a.inv_t * kLog2e;
  // Element k of this thread is column col(k). VEC (fp32 rows, 16-byte
  // aligned, pitches a multiple of 4): four consecutive columns per 16-byte
  // load, so each load instruction of a wave reads one contiguous kilobyte;
  // a vector that starts below V may end past it inside the row's pitch.
  // Otherwise one column per load, 64 consecutive elements per wave. Split-K
  // partials are summed in split order, as splitk_reduce_kernel does.
  auto col = [&](int k) -> int64_t {
    return VEC ? c0 + (k >> 2) * (4 * kThreads) + 4 * threadIdx.x + (k & 3)
               : c0 + k * kThreads + threadIdx.x;
  };
  float x[kSegPer];
  float m = -INFINITY, sx = 0.f;
  if constexpr (VEC) {
    typedef float f4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int q = 0; q < kSegPer / 4; ++q) {
      const int64_t j = col(4 * q);
      f4 v = {0.f, 0.f, 0.f, 0.f};
      if (j < a.v) {
        v = *reinterpret_cast<const f4*>(src + j);
        for (int sp = 1; sp < a.src_splits; ++sp)
          v += *reinterpret_cast<const f4*>(src + sp * a.src_split_stride + j);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) x[4 * q + e] = j + e < a.v ? v[e] : -INFINITY;
    }
  } else {
#pragma unroll
    for (int k = 0; k < kSegPer; ++k) {
      const int64_t j = col(k);
      x[k] = j < a.v ? static_cast<float>(src[j]) : -INFINITY;
    }
  }
  // the row's label column, when it lies in this segment: its thread writes
  // the fp32 label logit
  int64_t yy = -1;
  if (a.labels) {
    yy = a.labels[a.label_rows > 0 ? r % a.label_rows : r];
    if (yy == a.ignore_index || yy < c0 || yy >= c0 + kSegCols || yy >= a.v) yy = -1;
  }
#pragma unroll
  for (int k = 0; k < kSegPer; ++k) {
    const int64_t j = col(k);
    if (j < a.v) {
      m = fmaxf(m, x[k]);
      sx += x[k];
      if (j == yy) a.xy[r] = x[k];
    }
  }
  if (dst) {
    if constexpr (VEC) {
      typedef float f4 __attribute__((ext_vector_type(4)));
#pragma unroll
      for (int q = 0; q < kSegPer / 4; ++q) {
        const int64_t j = col(4 * q);
        if (j + 4 <= a.v) {
          *reinterpret_cast<f4*>(dst + j) = f4{x[4 * q], x[4 * q + 1], x[4 * q + 2], x[4 * q + 3]};
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (j + e < a.v) dst[j + e] = static_cast<DT>(x[4 * q + e]);
        }
      }
    } else {
#pragma unroll
      for (int k = 0; k < kSegPer; ++k) {
        const int64_t j = col(k);
        if (j < a.v) dst[j] = static_cast<DT>(x[k]);
      }
    }
  }
  if (dst && sg == nseg - 1)
    for (int64_t j = a.v + threadIdx.x; j < a.ldd; j += kThreads) dst[j] = static_cast<DT>(0.f);
  if constexpr (ONLINE) {
    // KernelConfig::online_softmax: no block-wide maximum before the sums.
    // Each thread forms {max, sums} of its own columns relative to its own
    // maximum, and the block merges the threads' states, rescaling each
    // state's sums to the larger maximum (the online softmax merge).
    float d1 = 0.f, dT = 0.f;
    if (m != -INFINITY) {
      const float o1 = -m * kLog2e, oT = -m * it2;
#pragma unroll
      for (int k = 0; k < kSegPer; ++k) {
        // e^(-inf) = 0 for the columns past V
        d1 += __builtin_amdgcn_exp2f(fmaf(x[k], kLog2e, o1));
        dT += __builtin_amdgcn_exp2f(fmaf(x[k], it2, oT));
      }
    }
    const Stat st = block_merge(Stat{m, d1, dT, sx}, it2, sstat);
    if (threadIdx.x == 0) a.stats[r * a.stats_ld + sg] = make_float4(st.m, st.d1, st.dT, st.sx);
    return;
  }
  m = block_max(m, sred);
  const float o1 = -m * kLog2e, oT = -m * it2;
  float d1 = 0.f, dT = 0.f;
#pragma unroll
  for (int k = 0; k < kSegPer; ++k) {
    // e^(-inf) = 0 for the columns past V
    d1 += __builtin_amdgcn_exp2f(fmaf(x[k], kLog2e, o1));
    dT += __builtin_amdgcn_exp2f(fmaf(x[k], it2, oT));
  }
  sx = block_sum(sx, sred);
  d1 = block_sum(d1, sred);
  dT = block_sum(dT, sred);
  if (threadIdx.x == 0) a.stats[r * a.stats_ld + sg] = make_float4(m, d1, dT, sx);
}

// ------------------------------------------------------------------ finalize
__global__ __launch_bounds__(kThreads) void finalize_kernel(FinalizeArgs a) {
  __shared__ double red[3][kThreads];
  double s_nll = 0.0, t_nll = 0.0, kl = 0.0;
  // Unrolled so that a thread's loads are in flight together; the
  // additions keep their order.
#pragma unroll 8
  for (int64_t i = threadIdx.x; i < a.bt; i += kThreads) {
    s_nll += static_cast<double>(a.row_nll_s[i]);
    t_nll += static_cast<double>(a.row_nll_t[i]);
  }
  // KL is accumulated per chunk and rounded to f32 (api.rs:304-314 with
  // kl.rs:126): one wave per chunk, lane partials summed across the wave.
  const int64_t nc = (a.bt + a.chunk_size - 1) / a.chunk_size;
  const int lane = threadIdx.x & 63;
  for (int64_t c = threadIdx.x >> 6; c < nc; c += kThreads / 64) {
    const int64_t e = (c + 1) * a.chunk_size < a.bt ? (c + 1) * a.chunk_size : a.bt;
    double k = 0.0;
#pragma unroll 8
    for (int64_t i = c * a.chunk_size + lane; i < e; i += 64) k += static_cast<double>(a.row_kl[i]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) k += __shfl_xor(k, o);
    if (lane == 0) kl += static_cast<double>(static_cast<float>(k));
  }
  red[0][threadIdx.x] = s_nll;
  red[1][threadIdx.x] = t_nll;
  red[2][threadIdx.x] = kl;
  __syncthreads();
  for (int w = kThreads / 2; w > 0; w >>= 1) {
    if (threadIdx.x < w)
      for (int q = 0; q < 3; ++q) red[q][threadIdx.x] += red[q][threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const double ms = static_cast<double>(a.mean_scale_ptr ? *a.mean_scale_ptr : a.mean_scale);
    const double S = red[0][0], Tt = red[1][0], K = red[2][0];
    a.out[0] = static_cast<float>((static_cast<double>(a.w_s) * S +
                                   static_cast<double>(a.w_t) * Tt +
                                   static_cast<double>(a.kd) * K) * ms);
    a.out[1] = static_cast<float>(S * ms);
    a.out[2] = static_cast<float>(Tt * ms);
    a.out[3] = static_cast<float>(K * ms);
  }
}

}  // namespace

hipError_t launch_row_pass(const RowPassArgs& a, hipStream_t s) {
  if (a.n_rows <= 0) return hipSuccess;
  // Half-tile-relative rows: bf16 logits of the logits GEMM only, and never
  // where the KL cross term is formed from the stored logits.
  if ((a.hmax_s != nullptr || a.hmax_t != nullptr) &&
      (a.split || a.ltype != DType::BF16 || (a.kl && a.cross == nullptr) ||
       a.hmax_ld < 4 * ((a.v + 255) / 256)))
    return hipErrorInvalidValue;
  dim3 grid(static_cast<unsigned>(a.n_rows));
  if (a.split) {   // any pitch and alignment
    // 512 threads a row: at 512 x 131072 and 1024 x 32000 fp32 logits
    // 0.470 and 0.220 ms per slot call, against 0.50 and 0.220 ms with 256
    // threads and 0.468 and 0.242 ms with 1024 (bf16 within 3 % of each other).
    constexpr int kSplitThreads = 512;
    if (a.ltype == DType::BF16)
      hipLaunchKernelGGL((row_pass_kernel<__bf16, true, kSplitThreads>), grid, dim3(kSplitThreads), 0, s, a);
    else
      hipLaunchKernelGGL((row_pass_kernel<float, true, kSplitThreads>), grid, dim3(kSplitThreads), 0, s, a);
    return hipGetLastError();
  }
  if (a.ld % 8) return hipErrorInvalidValue;
  const bool has_t = a.teacher != nullptr;
  const bool kl = a.kl && has_t;
  const bool tg = a.teacher_grad && has_t;
  if ((a.teacher_ce || kl || tg) && a.stats_t == nullptr) return hipErrorInvalidValue;
  if (a.teacher_f32 || a.teacher_bf16) {
    // bf16 student rows (relative to their half-tile maxima) beside fp32 or
    // bf16 teacher logits read in place at pitch ld_t; the statistics and KL sums
    // of both come from the logits GEMM's epilogue. The teacher gradient, if
    // any, goes to the bf16 rows grad_t (pitch ld).
    if (!has_t || a.grad_s != nullptr || (tg && a.grad_t == nullptr) || a.cross == nullptr ||
        a.row_consts == nullptr || a.ltype != DType::BF16 || a.hmax_s == nullptr ||
        a.hmax_t != nullptr || a.hmax_ld % 2 || reinterpret_cast<uintptr_t>(a.hmax_s) % 8 ||
        a.ld_t % (a.teacher_bf16 ? 8 : 4) || a.ld_t < a.v ||
        reinterpret_cast<uintptr_t>(a.teacher) % 16 || (a.teacher_f32 && a.teacher_bf16))
      return hipErrorInvalidValue;
    const int64_t chunks = (a.v + kChunk - 1) / kChunk;
    const int64_t blocks = a.n_rows * chunks;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 cgrid(static_cast<unsigned>((a.n_rows + kThreads / 64 - 1) / (kThreads / 64)));
    const dim3 ggrid(static_cast<unsigned>(blocks));
    if (kl && tg) {
      hipLaunchKernelGGL((row_consts_kernel<true, true>), cgrid, dim3(kThreads), 0, s, a);
      hipLaunchKernelGGL((a.teacher_bf16 ? row_grad_kernel<true, true, 2> : row_grad_kernel<true, true, 1>), ggrid,
                         dim3(kGradThreads), 0, s, a, chunks);
    } else if (kl) {
      hipLaunchKernelGGL((row_consts_kernel<true, false>), cgrid, dim3(kThreads), 0, s, a);
      hipLaunchKernelGGL((a.teacher_bf16 ? row_grad_kernel<true, false, 2> : row_grad_kernel<true, false, 1>), ggrid,
                         dim3(kGradThreads), 0, s, a, chunks);
    } else if (tg) {
      hipLaunchKernelGGL((row_consts_kernel<false, true>), cgrid, dim3(kThreads), 0, s, a);
      hipLaunchKernelGGL((a.teacher_bf16 ? row_grad_kernel<false, true, 2> : row_grad_kernel<false, true, 1>), ggrid,
                         dim3(kGradThreads), 0, s, a, chunks);
    } else {
      hipLaunchKernelGGL((row_consts_kernel<false, false>), cgrid, dim3(kThreads), 0, s, a);
      hipLaunchKernelGGL((a.teacher_bf16 ? row_grad_kernel<false, false, 2> : row_grad_kernel<false, false, 1>), ggrid,
                         dim3(kGradThreads), 0, s, a, chunks);
    }
    return hipGetLastError();
  }
  const DType gt = a.grad_s ? a.gtype : a.ltype;
  if (a.grad_s && (tg && a.grad_t == nullptr)) return hipErrorInvalidValue;
  if (a.ld_t && ((a.ld_t % 8) || (tg && a.grad_s == nullptr))) return hipErrorInvalidValue;
  // Blocks of at least 20·2^20 logits take the chunked passes below where
  // both forms apply (bf16 logits without a KL term; fp32 logits).
  const bool big = a.n_rows * a.v >= (int64_t{20} << 20);
  const bool pairs_rel = a.hmax_t == a.hmax_s + 1;   // teacher maxima beside the student's
  if (a.row_consts != nullptr && a.ltype == DType::BF16 && a.grad_s == nullptr && a.ld_t == 0 &&
      (!(kl || tg || a.teacher_ce) || has_t) && a.hmax_s != nullptr && a.hmax_ld % 2 == 0 &&
      reinterpret_cast<uintptr_t>(a.hmax_s) % 8 == 0 &&
      (a.cross != nullptr ? pairs_rel : !kl && (!tg || pairs_rel) && big)) {
    // bf16 in place (rows relative to their half-tile maxima): per-row
    // constants, then the chunked elementwise gradient. The paired layout
    // (KL sums from the logits GEMM), or no KL term at all (student CE, and
    // teacher CE from the teacher's own statistics): at BT x V = 8192 x
    // 131072, student CE only, this pass took 0.78 ms against 0.89 ms for
    // the row-per-workgroup kernel.
    const int64_t chunks = (a.v + kChunk - 1) / kChunk;
    const int64_t blocks = a.n_rows * chunks;
    const dim3 cgrid(static_cast<unsigned>((a.n_rows + kThreads / 64 - 1) / (kThreads / 64)));
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    if (kl && tg) {
      hipLaunchKernelGGL((row_consts_kernel<true, true>), cgrid, dim3(kThreads), 0, s, a);
      hipLaunchKernelGGL((row_grad_kernel<true, true, 0>), dim3(static_cast<unsigned>(blocks)),
                         dim3(kGradThreads), 0, s, a, chunks);
    } else if (kl) {
      hipLaunchKernelGGL((row_consts_kernel<true, false>), cgrid, dim3(kThreads), 0, s, a);
      hipLaunchKernelGGL((row_grad_kernel<true, false, 0>), dim3(static_cast<unsigned>(blocks)),
                         dim3(kGradThreads), 0, s, a, chunks);
    } else if (tg) {
      hipLaunchKernelGGL((row_consts_kernel<false, true>), cgrid, dim3(kThreads), 0, s, a);
      hipLaunchKernelGGL((row_grad_kernel<false, true, 0>), dim3(static_cast<unsigned>(blocks)),
                         dim3(kGradThreads), 0, s, a, chunks);
    } else {
      hipLaunchKernelGGL((row_consts_kernel<false, false>), cgrid, dim3(kThreads), 0, s, a);
      hipLaunchKernelGGL((row_grad_kernel<false, false, 0>), dim3(static_cast<unsigned>(blocks)),
                         dim3(kGradThreads), 0, s, a, chunks);
    }
    return hipGetLastError();
  }
  // The chunked fp32 pass costs two more launches (~12 us) and streams
  // faster: the row-per-workgroup kernel serves blocks of fewer than 20·2^20
  // logits (Tied, fp32, one block of rows x V; fused against chunked:
  // 256 x 8192 14.6 / 23.5 us, 512 x 16384 29.6 / 36.7 us, 1024 x 16000
  // 48.4 / 58.4 us, 512 x 32000 54.0 / 55.9 us, 768 x 32000 90.2 / 79.1 us,
  // 1024 x 32000 118.2 / 98.2 us).
  if (big && a.ltype == DType::F32 && a.cross == nullptr && a.row_consts != nullptr &&
      (a.kl_part != nullptr || !kl) && (!(kl || tg || a.teacher_ce) || has_t)) {
    // fp32 logits: per-row constants, the chunked elementwise gradient with
    // per-block KL sums, then each row's KL from those sums.
    const int64_t chunks = row_pass_kl_blocks(a.v);
    const int64_t blocks = a.n_rows * chunks;
    const dim3 cgrid(static_cast<unsigned>((a.n_rows + kThreads / 64 - 1) / (kThreads / 64)));
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 bgrid(static_cast<unsigned>(blocks));
#define ORDA_ROWGRAD_F32(GT)                                                                          \
  if (kl && tg) {                                                                                     \
    hipLaunchKernelGGL((row_consts_kernel<true, true>), cgrid, dim3(kThreads), 0, s, a);              \
    hipLaunchKernelGGL((row_grad_f32_kernel<GT, true, true>), bgrid, dim3(kF32Threads), 0, s, a, chunks); \
  } else if (kl) {                                                                                    \
    hipLaunchKernelGGL((row_consts_kernel<true, false>), cgrid, dim3(kThreads), 0, s, a);             \
    hipLaunchKernelGGL((row_grad_f32_kernel<GT, true, false>), bgrid, dim3(kF32Threads), 0, s, a, chunks); \
  } else if (tg) {                                                                                    \
    hipLaunchKernelGGL((row_consts_kernel<false, true>), cgrid, dim3(kThreads), 0, s, a);             \
    hipLaunchKernelGGL((row_grad_f32_kernel<GT, false, true>), bgrid, dim3(kF32Threads), 0, s, a, chunks); \
  } else {                                                                                            \
    hipLaunchKernelGGL((row_consts_kernel<false, false>), cgrid, dim3(kThreads), 0, s, a);            \
    hipLaunchKernelGGL((row_grad_f32_kernel<GT, false, false>), bgrid, dim3(kF32Threads), 0, s, a, chunks); \
  }
    if (gt == DType::F32) {
      ORDA_ROWGRAD_F32(float)
    } else {
      ORDA_ROWGRAD_F32(__bf16)
    }
#undef ORDA_ROWGRAD_F32
    if (kl) hipLaunchKernelGGL(row_kl_kernel, cgrid, dim3(kThreads), 0, s, a, chunks);
    return hipGetLastError();
  }
#define ORDA_ROWPASS(LT, GT)                                                                          \
  if (kl && tg) hipLaunchKernelGGL((row_pass_fused_kernel<LT, GT, true, true>), grid, dim3(kThreads), 0, s, a);   \
  else if (kl) hipLaunchKernelGGL((row_pass_fused_kernel<LT, GT, true, false>), grid, dim3(kThreads), 0, s, a);  \
  else if (tg) hipLaunchKernelGGL((row_pass_fused_kernel<LT, GT, false, true>), grid, dim3(kThreads), 0, s, a);  \
  else hipLaunchKernelGGL((row_pass_fused_kernel<LT, GT, false, false>), grid, dim3(kThreads), 0, s, a);
  if (a.ltype == DType::F32 && gt == DType::BF16) {
    ORDA_ROWPASS(float, __bf16)
  } else if (a.ltype == DType::F32 && gt == DType::F32) {
    ORDA_ROWPASS(float, float)
  } else if (a.ltype == DType::BF16 && gt == DType::BF16) {
    ORDA_ROWPASS(__bf16, __bf16)
  } else {
    return hipErrorInvalidValue;
  }
#undef ORDA_ROWPASS
  return hipGetLastError();
}

int64_t row_stats_segments(int64_t v) { return (v + kSegCols - 1) / kSegCols; }

int64_t row_pass_kl_blocks(int64_t v) { return (v + kF32Chunk - 1) / kF32Chunk; }

hipError_t launch_row_stats(const RowStatsArgs& a, hipStream_t s) {
  if (a.n_rows <= 0) return hipSuccess;
  if (a.src_splits > 1 && (!a.segmented || a.online || a.src_type != DType::F32 || a.dst == nullptr))
    return hipErrorInvalidValue;
  dim3 grid(static_cast<unsigned>(a.n_rows));
  const bool sf = a.src_type == DType::F32;
  const bool df = a.dst_type == DType::F32;
  if (a.segmented) {
    const int64_t nseg = row_stats_segments(a.v);
    if (a.stats_ld < nseg) return hipErrorInvalidValue;
    const int64_t blocks = a.n_rows * nseg;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 g(static_cast<unsigned>(blocks));
    // 16-byte fp32 vectors where the rows allow them (split-K partials
    // always do; a row of any pitch otherwise goes element by element)
    const bool vec = sf && a.lds % 4 == 0 && reinterpret_cast<uintptr_t>(a.src) % 16 == 0 &&
                     a.src_split_stride % 4 == 0 &&
                     (a.dst == nullptr ||
                      (df && a.ldd % 4 == 0 && reinterpret_cast<uintptr_t>(a.dst) % 16 == 0));
    if (a.src_splits > 1 && !vec) return hipErrorInvalidValue;
#define ORDA_ROWSTATS_SEG(ON)                                                                            \
  if (vec) hipLaunchKernelGGL((row_stats_seg_kernel<float, float, true, ON>), g, dim3(kThreads), 0, s, a, nseg); \
  else if (sf && df) hipLaunchKernelGGL((row_stats_seg_kernel<float, float, false, ON>), g, dim3(kThreads), 0, s, a, nseg); \
  else if (sf) hipLaunchKernelGGL((row_stats_seg_kernel<float, __bf16, false, ON>), g, dim3(kThreads), 0, s, a, nseg); \
  else if (df) hipLaunchKernelGGL((row_stats_seg_kernel<__bf16, float, false, ON>), g, dim3(kThreads), 0, s, a, nseg); \
  else hipLaunchKernelGGL((row_stats_seg_kernel<__bf16, __bf16, false, ON>), g, dim3(kThreads), 0, s, a, nseg);
    if (a.online) {
      ORDA_ROWSTATS_SEG(true)
    } else {
      ORDA_ROWSTATS_SEG(false)
    }
#undef ORDA_ROWSTATS_SEG
    return hipGetLastError();
  }
  if (!a.online && a.dst == nullptr) {
    const int es = sf ? 4 : 2;
    const bool vec = reinterpret_cast<uintptr_t>(a.src) % 16 == 0 && (a.lds * es) % 16 == 0;
    if (sf && vec) hipLaunchKernelGGL((row_stats_wide_kernel<float, true>), grid, dim3(kWideThreads), 0, s, a);
    else if (sf) hipLaunchKernelGGL((row_stats_wide_kernel<float, false>), grid, dim3(kWideThreads), 0, s, a);
    else if (vec) hipLaunchKernelGGL((row_stats_wide_kernel<__bf16, true>), grid, dim3(kWideThreads), 0, s, a);
    else hipLaunchKernelGGL((row_stats_wide_kernel<__bf16, false>), grid, dim3(kWideThreads), 0, s, a);
    return hipGetLastError();
  }
#define ORDA_ROWSTATS(ONLINE)                                                                        \
  if (sf && df) hipLaunchKernelGGL((row_stats_kernel<float, float, ONLINE>), grid, dim3(kThreads), 0, s, a);   \
  else if (sf) hipLaunchKernelGGL((row_stats_kernel<float, __bf16, ONLINE>), grid, dim3(kThreads), 0, s, a);  \
  else if (df) hipLaunchKernelGGL((row_stats_kernel<__bf16, float, ONLINE>), grid, dim3(kThreads), 0, s, a);  \
  else hipLaunchKernelGGL((row_stats_kernel<__bf16, __bf16, ONLINE>), grid, dim3(kThreads), 0, s, a);
  if (a.online) {
    ORDA_ROWSTATS(true)
  } else {
    ORDA_ROWSTATS(false)
  }
#undef ORDA_ROWSTATS
  return hipGetLastError();
}

hipError_t launch_finalize(const FinalizeArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(finalize_kernel, dim3(1), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace orda
