// gemm.hip — MFMA GEMMs of the distillation loss on gfx950.
//
// The three products of the reference's chunk loop (src/api.rs:273-292 and
// :346-377, via src/mat.rs:63-130) all run through one kernel template:
//   logits      C[2n,V]   = [h_s;h_t] · Wᵀ     A K-major, B K-major
//   grad_hidden C[rows,H] = dlogits · W        A K-major, B N-major
//   grad_W      C[V,H]    = (hiddenᵀ · dlogits)ᵀ, computed as
//               Cᵀ[H,V]   = hiddenᵀ · dlogits  A K-major (the hidden rows
//               transposed by transpose_rows_kernel), B N-major, C stored
//               transposed
//
// Workgroup tile 256x256, 4 waves each owning 128x128 as 8x8 fragments of
// 16x16. K advances 64 bytes per stage (32 bf16 / 16 fp32) through a ring of
// four 32 KB LDS stages. Operands travel global -> LDS by DMA
// (global_load_lds_dwordx4, 16 bytes per lane, written lane-linearly). In
// the bf16 loops the fragments of stage s+1 are read into a second register
// set while the 64 MFMAs of stage s run, so the MFMAs start at once after a
// barrier (one per stage). When both operands are K-major the bf16 loop
// moves stages in pairs (128 bytes of K per row: 8 lanes fetch one full
// cache line, half the L1 requests of single stages); otherwise it moves
// single stages four ahead. The fp32 loop moves single stages three ahead:
//   * K-major tiles are stored [row][64 B] (a pair: [row][128 B]) with the
//     16-byte chunks XOR-swizzled by row; the swizzle is applied by choosing
//     which global chunk each lane fetches. Fragment reads are conflict-free
//     ds_read_b128.
//   * MN-major tiles are stored [k][256 elements] (bf16: 512 B rows) with an
//     8-byte-pair swizzle and read with ds_read_b64_tr_b16, the gfx950 LDS
//     transpose read: lanes 4j..4j+3 of each 16-lane group name row j and
//     lane i receives column i of those 4 rows, i.e. four consecutive k of
//     one column — exactly an MFMA operand. fp32 MN-major tiles use
//     ds_read_b32.
// bf16 uses v_mfma_f32_16x16x32_bf16, fp32 v_mfma_f32_16x16x4_f32 (four per
// 16-byte k-group); accumulation is fp32 in both. Workgroups are rastered in
// groups of M-tiles and each XCD receives a contiguous range, so tiles that
// share an operand strip share that XCD's L2; products with few N-tiles
// (grad_hidden) instead run rounds that all XCDs spend on the same operand
// strips (map_tile).
//
// The Logits epilogue fuses the statistics the row pass needs: for every row
// and every 256-column tile it writes {max, Σe^(x-max), Σe^((x-max)/T), Σx}
// from the fp32 accumulators, plus the fp32 logit at the row's label, so the
// row pass reads each logit exactly once. With paired rows (student and
// teacher rows interleaved in blocks of 16) it also writes the tile's KL
// KL sums Σ e^((t-max_t)/T)·((t - max_t) - (s - max_s)) and
// Σ (e^((s-max_s)/T) - e^((t-max_t)/T)), each element's terms taken
// relative to its own row's maximum and its difference formed before it is
// summed (with log1p of the second over Σe^((t-max_t)/T), the row pass gets
// lse_s^T - lse_t^T without the cancellation of two separately rounded
// sums, and a constant offset between the rows cancels element by element),
// so that every loss term comes from fp32 accumulators and the stored
// logits (then bf16) only feed the gradient. Each lane stores its 4 consecutive columns directly. bf16 logits
// are stored relative to the maximum of their 128-column half tile, in log2
// units, with those maxima beside the statistics: their rounding error then
// follows their distance below the maximum, not their magnitude.
#include <float.h>
#include <math.h>

#include "kl_sums.h"
#include "orda_kernels.h"

namespace orda {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef __attribute__((address_space(3))) const u32x4 lds_u32x4;

constexpr int kTile = 256;                     // BM = BN
constexpr int kSlab = 64;                      // bytes of K per stage (K-major rows)
constexpr int kThreads = 256;
constexpr int kFrag = 8;                       // 8x8 fragments of 16x16 per wave
constexpr int kOpBytes = 16384;                // one operand, one stage
constexpr int kStageBytes = 2 * kOpBytes;      // A then B
constexpr int kRing = 4;                       // stages in flight
constexpr int kXfers = kOpBytes / (kThreads * 16);   // DMA transfers per thread per operand
static_assert(kXfers == 4, "the main loop's DMA schedule assumes four transfers per operand");
constexpr int kEpiLds = 16384;                 // epilogue scratch beside the ring
constexpr float kLog2e = 1.4426950408889634f;

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

// ---------------------------------------------------------------- swizzles
// K-major tile [256 rows][4 chunks of 16 B]: two rows share a 128-byte bank
// line, and rows r..r+7 (aligned) reading one logical chunk land on 8
// distinct 16-byte bank windows.
__device__ __forceinline__ int kmaj_swz(int r) { return (r >> 1) & 3; }
__device__ __forceinline__ int kmaj_off(int r, int c) { return r * kSlab + ((c ^ kmaj_swz(r)) << 4); }

// MN-major bf16 tile [32 k-rows][32 chunks of 16 B]. The four rows a 16-lane
// transpose read touches (k0..k0+3) and the groups 8 rows apart use distinct
// 32-byte windows.
__device__ __forceinline__ int mnb_swz(int r) { return 2 * (r & 3) + 8 * ((r >> 3) & 1); }
// MN-major fp32 tile [16 k-rows][64 chunks of 16 B].
__device__ __forceinline__ int mnf_swz(int r) { return 4 * ((r >> 2) & 3); }

// s_waitcnt encodings (gfx9): vmcnt in bits 3:0 and 15:14, expcnt 6:4,
// lgkmcnt 11:8. Both wait for every LDS operation.
constexpr int kWaitAll = 0x0070;                              // vmcnt(0) lgkmcnt(0)
constexpr int vm_wait(int n) { return 0x0070 | (n & 15) | ((n >> 4) << 14); }
constexpr int kWaitTwoStages = vm_wait(2 * 2 * kXfers);     // stage s+1 landed
constexpr int kWaitLds = 0xC07F;                              // lgkmcnt(0) only

// One DMA transfer: every active lane copies the 16 bytes at sbase + voff
// into LDS at M0 + 16 * lane (global_load_lds_dwordx4, saddr form). Written as
// inline asm so that the compiler's memory-counter bookkeeping does not see
// the transfers: it would otherwise make every later LDS transpose read wait
// for all of them (vmcnt(0)). The kernel orders DMA and reads itself with
// explicit s_waitcnt + s_barrier. M0 is reserved by the compiler, hence the
// clobber (nothing else in these kernels keeps a value in M0).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const unsigned char* sbase, uint32_t voff, unsigned char* l) {
  // sbase and the LDS destination are wave-uniform; readfirstlane states it
  // to the compiler so that they live in SGPRs also inside divergent code.
  // (readfirstlane returns int: each half goes through uint32_t so that the
  // low half is not sign-extended into the high one.)
  const uint64_t p = reinterpret_cast<uint64_t>(sbase);
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p)));
  const uint32_t hi =
      static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p >> 32)));
  const uint64_t ps = (static_cast<uint64_t>(hi) << 32) | lo;
  const uint32_t m0 = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void*)l))));
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %0"
               :
               : "s"(ps), "v"(voff), "s"(m0)
               : "memory", "m0");
}
// Main-loop form: M0 = m0base + imm in one SALU add (the caller keeps
// m0base = the stage slot's LDS offset + this wave's 1 KB block).
template <int IMM>
__device__ __forceinline__ void dma16_at(uint64_t sbase, uint32_t voff, uint32_t m0base) {
  asm volatile("s_add_u32 m0, %2, %3\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %0"
               :
               : "s"(sbase), "v"(voff), "s"(m0base), "n"(IMM)
               : "memory", "m0", "scc");
}
#pragma clang diagnostic pop
// A wave-uniform 64-bit value in an SGPR pair.
__device__ __forceinline__ uint64_t uniform64(const void* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v)));
  const uint32_t hi =
      static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32)));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// ---------------------------------------------------------------- loaders
// Per-thread description of one operand's 8 DMA transfers per stage.
// KMAJOR: operand stored [rows of M or N][ld], a stage covers rows
//         [origin, origin+256) x elements [k0, k0+SK).
// !KMAJOR: operand stored [K][ld], a stage covers K rows [k0, k0+SK) x
//         columns [origin, origin+256).
// Rows/columns past the operand's edge are clamped to the last one that
// exists: they only feed output rows/columns that are never stored.
template <typename T, bool KMAJOR>
struct Loader {
  static constexpr int ES = Elem<T>::kSize;
  static constexpr int EPC = 16 / ES;       // elements per 16-byte chunk
  static constexpr int SK = kSlab / ES;     // K per stage
  static constexpr int CPR = KMAJOR ? kSlab / 16 : (kTile * ES / 16);   // chunks per LDS row

  const unsigned char* base;   // operand origin: KMAJOR row origin, else column origin
  int64_t ld_bytes;
  int64_t K;
  uint32_t goff[kXfers];       // byte offset of each transfer within a stage
  int kidx[kXfers];            // K coordinate of each transfer within the stage

  __device__ __forceinline__ void init(const void* p, int64_t ld, int64_t ext, int64_t k,
                                       int origin, int wave, int lane) {
    ld_bytes = ld * ES;
    K = k;
    if (KMAJOR) {
      base = static_cast<const unsigned char*>(p) + static_cast<int64_t>(origin) * ld_bytes;
      const int rmax = static_cast<int>(ext - 1 - origin);
#pragma unroll
      for (int i = 0; i < kXfers; ++i) {
        const int P = (i * 4 + wave) * 64 + lane;
        const int r = P / CPR;
        const int c = (P % CPR) ^ kmaj_swz(r);
        const int rr = r < rmax ? r : rmax;
        goff[i] = static_cast<uint32_t>(rr * ld_bytes + c * 16);
        kidx[i] = c * EPC;
      }
    } else {
      base = static_cast<const unsigned char*>(p) + static_cast<int64_t>(origin) * ES;
      const int cmax = static_cast<int>((ext - 1 - origin) / EPC);
#pragma unroll
      for (int i = 0; i < kXfers; ++i) {
        const int P = (i * 4 + wave) * 64 + lane;
        const int r = P / CPR;
        const int pc = P % CPR;
        const int c = pc ^ (ES == 2 ? mnb_swz(r) : mnf_swz(r));
        const int cc = c < cmax ? c : cmax;
        goff[i] = static_cast<uint32_t>(r * ld_bytes + cc * 16);
        kidx[i] = r;
      }
    }
  }

  // K-major paired rows read in place (LogitStatsArgs::pair_teacher), as
  // PairLoader::init_paired for the single-stage layout: transfer i of wave
  // w covers tile rows 16(4i + w) .. +15, so odd waves move teacher rows
  // only. Used for the K left after the stage pairs.
  __device__ __forceinline__ void init_paired(const void* ps, const void* pt, int64_t ld,
                                              int64_t rows, int64_t k, int64_t origin, int wave,
                                              int lane) {
    static_assert(KMAJOR && ES == 2, "paired rows are bf16 and K-major");
    ld_bytes = ld * ES;
    K = k;
    const int64_t last = rows - 1;
    const int64_t b0 = origin < last ? origin : last;
    base = static_cast<const unsigned char*>((wave & 1) ? pt : ps) + b0 * ld_bytes;
#pragma unroll
    for (int i = 0; i < kXfers; ++i) {
      const int P = (i * 4 + wave) * 64 + lane;
      const int r = P / CPR;
      const int c = (P % CPR) ^ kmaj_swz(r);
      const int64_t src = origin + 16 * (r >> 5) + (r & 15);
      const int64_t rr = src < last ? src : last;
      goff[i] = static_cast<uint32_t>((rr - b0) * ld_bytes + c * 16);
      kidx[i] = c * EPC;
    }
  }

  // Source of stage kt (from its first K element on).
  __device__ __forceinline__ const unsigned char* stage_src(int kt) const {
    const int64_t k0 = static_cast<int64_t>(kt) * SK;
    return KMAJOR ? base + k0 * ES : base + k0 * ld_bytes;
  }

  // Issue the DMA of stage kt into the LDS operand tile `tile`. Transfers past
  // K write zeros instead, so the tail stage contributes nothing.
  __device__ __forceinline__ void issue(unsigned char* tile, int kt, int wave, int lane) const {
    const int64_t k0 = static_cast<int64_t>(kt) * SK;
    const unsigned char* s = stage_src(kt);
    const int64_t krem = K - k0;
    if (krem >= SK) {
#pragma unroll
      for (int i = 0; i < kXfers; ++i)
        dma16(s, goff[i], tile + (i * 4 + wave) * 1024);
    } else {
#pragma unroll
      for (int i = 0; i < kXfers; ++i) {
        unsigned char* l = tile + (i * 4 + wave) * 1024;
        if (kidx[i] < krem) {
          dma16(s, goff[i], l);
        } else {
          *reinterpret_cast<u32x4*>(l + lane * 16) = u32x4{0, 0, 0, 0};
        }
      }
    }
  }
};

// Per-thread description of one bf16 operand's DMA transfers for a stage
// pair (64 elements of K) of the main loop; the pair lands in a double slot
// of 32 KB:
//   K-major:  [256 rows][8 chunks of 16 B], chunk q of row r stored at
//             q ^ (r & 7), so 8 lanes fetch one full 128-byte line of a row;
//   MN-major: [64 k-rows][32 chunks of 16 B] with the single-stage swizzle,
//             i.e. two consecutive single-stage slots.
// Rows/columns past the operand's edge are clamped as in Loader.
template <bool KMAJOR>
struct PairLoader {
  static constexpr int kX = 2 * kXfers;   // transfers per thread per pair
  const unsigned char* base;
  int64_t step;                           // bytes from one pair to the next
  uint32_t goff[kX];

  __device__ __forceinline__ void init(const void* p, int64_t ld, int64_t ext, int origin, int wave,
                                       int lane) {
    const int64_t ldb = ld * 2;
    if (KMAJOR) {
      base = static_cast<const unsigned char*>(p) + static_cast<int64_t>(origin) * ldb;
      step = 128;
      const int rmax = static_cast<int>(ext - 1 - origin);
#pragma unroll
      for (int t = 0; t < kX; ++t) {
        const int P = (t * 4 + wave) * 64 + lane;
        const int r = P >> 3;
        const int q = (P & 7) ^ (r & 7);
        const int rr = r < rmax ? r : rmax;
        goff[t] = static_cast<uint32_t>(rr * ldb + q * 16);
      }
    } else {
      base = static_cast<const unsigned char*>(p) + static_cast<int64_t>(origin) * 2;
      step = 64 * ldb;
      const int cmax = static_cast<int>((ext - 1 - origin) / 8);
#pragma unroll
      for (int t = 0; t < kX; ++t) {
        const int P = (t * 4 + wave) * 64 + lane;
        const int r = P >> 5;
        const int c = (P & 31) ^ mnb_swz(r);
        const int cc = c < cmax ? c : cmax;
        goff[t] = static_cast<uint32_t>(r * ldb + cc * 16);
      }
    }
  }
  // K-major paired rows read in place (LogitStatsArgs::pair_teacher): tile
  // row r of 32-row block b = r/32 is row origin + 16b + r%16 of the student
  // tensor ps (r%32 < 16) or of the teacher tensor pt. Transfer t of wave w
  // covers tile rows 32t + 8w .. 32t + 8w + 7, so waves 0-1 move student
  // rows only and waves 2-3 teacher rows only: one base per wave. Rows past
  // `rows` are clamped to the last one (their outputs are not stored).
  __device__ __forceinline__ void init_paired(const void* ps, const void* pt, int64_t ld,
                                              int64_t rows, int64_t origin, int wave, int lane) {
    static_assert(KMAJOR, "paired rows are K-major");
    const int64_t ldb = ld * 2;
    const int64_t last = rows - 1;
    const int64_t b0 = origin < last ? origin : last;   // base row, within the tensor
    base = static_cast<const unsigned char*>(wave < 2 ? ps : pt) + b0 * ldb;
    step = 128;
#pragma unroll
    for (int t = 0; t < kX; ++t) {
      const int P = (t * 4 + wave) * 64 + lane;
      const int r = P >> 3;
      const int q = (P & 7) ^ (r & 7);
      const int64_t src = origin + 16 * (r >> 5) + (r & 15);
      const int64_t rr = src < last ? src : last;
      goff[t] = static_cast<uint32_t>((rr - b0) * ldb + q * 16);
    }
  }
  __device__ __forceinline__ const unsigned char* src(int pair) const { return base + pair * step; }
};

// ---------------------------------------------------------------- fragments
// Operand fragment of a stage (64 bytes of K) for 16 rows (or columns)
// starting at r0 of the tile: lane (m = lane%16, g = lane/16) holds the K
// elements [g*KG/4, +KG/4) of row r0+m, KG = 32 (bf16) or 16 (fp32).
template <typename T, bool KMAJOR>
__device__ __forceinline__ u32x4 read_frag(const unsigned char* tile, int r0, int lane) {
  const int m = lane & 15, g = lane >> 4;
  constexpr int kg = 0;
  if constexpr (KMAJOR) {
    return *reinterpret_cast<const u32x4*>(tile + kmaj_off(r0 + m, kg * 4 + g));
  } else if constexpr (Elem<T>::kSize == 2) {
    // two transpose reads: K rows 8g + {0..3} and 8g + {4..7}
    u32x4 out;
    const int col = r0 + 4 * (m & 3);
    const int c = col >> 3;
    const int byte = (m & 1) * 8;   // (col % 8) * 2, col % 4 == 0
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int kr = kg * 32 + 8 * g + 4 * h + (m >> 2);
      const int off = kr * 512 + ((c ^ mnb_swz(kr)) << 4) + byte;
      const u32x2 w = __builtin_bit_cast(
          u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(tile + off)));
      out[2 * h] = w[0];
      out[2 * h + 1] = w[1];
    }
    return out;
  } else {
    u32x4 out;
    const int col = r0 + m;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int kr = kg * 16 + 4 * g + q;
      const int off = kr * 1024 + (((col >> 2) ^ mnf_swz(kr)) << 4) + (col & 3) * 4;
      out[q] = *reinterpret_cast<const uint32_t*>(tile + off);
    }
    return out;
  }
}

// Fragment reader of one bf16 operand for the interleaved main loops. Each
// lane keeps its LDS byte addresses of the reads of ring stage 0 (and, for a
// paired K-major tile, of stage 1); the rest is the read's immediate:
//   K-major, single stages (slot s at s * kOpBytes): fragment i sits 1024*i
//             bytes after fragment 0 (the row swizzle depends on the row's
//             low bits only) — one ds_read_b128 each;
//   K-major, paired (PairLoader's double slots; stage s is half s%2 of
//             double slot s/2): fragment i sits 2048*i bytes after fragment
//             0; the stage half selects chunk bit 2, which the swizzle XORs,
//             hence one base address per half;
//   MN-major (either ring; stage s at s * kOpBytes): two transpose reads per
//             fragment (h = 0, 1); fragment i of read h sits at
//             off[h] ^ (i << 5), because i only moves chunk bits 1-3 of the
//             row, which are the bits the swizzle XORs.
// read_op<SLOT>(o) issues LDS instruction o of a stage: fragment o (K-major)
// or half o%2 of fragment o/2 (MN-major).
template <bool KMAJOR, bool PAIRED>
struct FragReader {
  static constexpr int kOps = KMAJOR ? kFrag : 2 * kFrag;
  uint32_t addr[KMAJOR ? 2 : 2 * kFrag];

  // tile0: LDS byte address of this operand's stage-0 slot; w0: the wave
  // strip's first row (K-major) or column (MN-major).
  __device__ __forceinline__ void init(uint32_t tile0, int w0, int lane) {
    const int m = lane & 15, g = lane >> 4;
    if constexpr (KMAJOR && PAIRED) {
      const int r = w0 + m;
#pragma unroll
      for (int h = 0; h < 2; ++h)
        addr[h] = tile0 + static_cast<uint32_t>(r * 128 + (((4 * h + g) ^ (r & 7)) << 4));
    } else if constexpr (KMAJOR) {
      addr[0] = addr[1] = tile0 + static_cast<uint32_t>(kmaj_off(w0 + m, g));
    } else {
      const int col = w0 + 4 * (m & 3);
      const int c = col >> 3;
      const int byte = (m & 1) * 8;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int kr = 8 * g + 4 * h + (m >> 2);
        const uint32_t off = static_cast<uint32_t>(kr * 512 + ((c ^ mnb_swz(kr)) << 4) + byte);
#pragma unroll
        for (int f = 0; f < kFrag; ++f)
          addr[2 * f + h] = tile0 + (off ^ static_cast<uint32_t>(f << 5));
      }
    }
  }
  template <int SLOT>
  __device__ __forceinline__ void read_op(int o, u32x4 (&r)[kFrag]) const {
    if constexpr (KMAJOR && PAIRED) {
      r[o] = *(const lds_u32x4*)(static_cast<uintptr_t>(addr[SLOT & 1] +
                                                        (o * 2048 + (SLOT >> 1) * 2 * kOpBytes)));
    } else if constexpr (KMAJOR) {
      r[o] = *(const lds_u32x4*)(static_cast<uintptr_t>(addr[0] + (o * 1024 + SLOT * kOpBytes)));
    } else {
      const u32x2 w = __builtin_bit_cast(
          u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                     (lds_i16x4*)(static_cast<uintptr_t>(addr[o] + SLOT * kOpBytes))));
      r[o >> 1][2 * (o & 1)] = w[0];
      r[o >> 1][2 * (o & 1) + 1] = w[1];
    }
  }
};

template <int S>
struct SlotC {
  static constexpr int value = S;
};

// One bf16 MFMA with its accumulator pinned to AGPRs (tied in/out). Written
// as inline asm because, once fragment reads are interleaved with the MFMAs,
// the compiler stops tying the builtin's accumulator to its result and keeps
// shuffling the 64 accumulators between VGPRs and AGPRs. The compiler still
// inserts the LDS waits for the operands; the MFMA hazards it cannot see
// (accumulator initialisation before the first MFMA, results read after the
// last one) are covered by explicit s_nop, and the build checks the
// generated code for them.
__device__ __forceinline__ void mfma_bf16(f32x4& acc, const u32x4& a, const u32x4& b) {
  asm("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
// Wait states between the last MFMA and the first read of its result, and
// between an accumulator write by a VALU and the first MFMA reading it.
__device__ __forceinline__ void mfma_drain() { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7"); }
// Copy of an accumulator into VGPRs at this point of the program. Without
// it the compiler moves every accumulator into VGPRs at the start of the
// logits epilogue, which then no longer fits the register file.
__device__ __forceinline__ f32x4 from_acc(const f32x4& a) {
  float x, y, z, w;
  asm volatile(
      "v_accvgpr_read_b32 %0, %4\n\tv_accvgpr_read_b32 %1, %5\n\t"
      "v_accvgpr_read_b32 %2, %6\n\tv_accvgpr_read_b32 %3, %7"
      : "=v"(x), "=v"(y), "=v"(z), "=v"(w)
      : "a"(a[0]), "a"(a[1]), "a"(a[2]), "a"(a[3]));
  return f32x4{x, y, z, w};
}
__device__ __forceinline__ void mfma_prime() { asm volatile("s_nop 7"); }
// max(a, b, c) in one instruction. fmaxf on values that come out of inline
// asm (from_acc) first canonicalises each operand, one more op per value.
__device__ __forceinline__ float max3f(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
// Maximum of a lane's 32 values of one row (all columns valid): 16 v_max3.
__device__ __forceinline__ float row_max32(const f32x4 (&v)[8]) {
  float m = max3f(v[0][0], v[0][1], v[0][2]);
  m = max3f(m, v[0][3], v[1][0]);
#pragma unroll
  for (int k = 5; k < 31; k += 2) m = max3f(m, v[k >> 2][k & 3], v[(k + 1) >> 2][(k + 1) & 3]);
  return max3f(m, v[7][3], v[7][3]);
}

// One stage of MFMAs: acc[i][j] += A-fragment i x B-fragment j. With SWAP the
// operands enter the MFMA the other way round, so acc[i][j] holds the
// transposed 16x16 block: lane (r = lane%16, g = lane/16) then owns row r of
// A-fragment i and the four consecutive columns 4g..4g+3 of B-fragment j,
// instead of four consecutive rows of one column. (The bf16 main loops with
// swapped operands instead keep B-fragment j, then the first source, for 8
// consecutive MFMAs: measured 0.4 % faster on the logits GEMM.)
template <typename T, bool SWAP>
__device__ __forceinline__ void mfma_step(f32x4 (&acc)[kFrag][kFrag], const u32x4 (&a)[kFrag],
                                          const u32x4 (&b)[kFrag]) {
#pragma unroll
  for (int i = 0; i < kFrag; ++i) {
#pragma unroll
    for (int j = 0; j < kFrag; ++j) {
      const u32x4& x = SWAP ? b[j] : a[i];
      const u32x4& y = SWAP ? a[i] : b[j];
      if constexpr (Elem<T>::kSize == 2) {
        mfma_bf16(acc[i][j], x, y);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(x[q]),
                                                           __uint_as_float(y[q]), acc[i][j],
                                                           0, 0, 0);
      }
    }
  }
}

struct TileCoord {
  int p, m0, n0, ntile;
};

__device__ __forceinline__ TileCoord tile_at(int64_t pm, int64_t pn, int64_t Mt) {
  TileCoord c;
  c.p = static_cast<int>(pm / Mt);
  c.m0 = static_cast<int>((pm % Mt) * kTile);
  c.n0 = static_cast<int>(pn * kTile);
  c.ntile = static_cast<int>(pn);
  return c;
}

__device__ __forceinline__ TileCoord map_tile(const GemmArgs& g, int64_t t) {
  const int64_t Mt = (g.M + kTile - 1) / kTile;
  const int64_t Nt = (g.N + kTile - 1) / kTile;
  int64_t Mv = Mt * g.nprob;
  int64_t T = Mv * Nt;
  int64_t mfirst = 0;   // first M-tile of the grouped raster below
  // Shared rounds (few N-tiles, long K: grad_hidden). Each round covers a
  // band of a*xm M-tiles x all Nt N-tiles: xn XCDs side by side in N (b =
  // Nt/xn N-tiles each), xm = 8/xn in M (a M-tiles each), a*b <= 32 tiles
  // per XCD (launch_gemm picks them: at Nt = 16, 8 x 4, the same 12 operand
  // strips per stage in each L2 as the grouped raster). The XCDs of a round
  // read the same strips at the same time, so the MALL serves the repeats
  // and each strip is fetched from HBM once per band (the grouped raster
  // walks an XCD's M-tiles over two passes of N and fetches them twice).
  // The same blocks with b = all N-tiles (xn = 1) walk a large bf16 logits
  // GEMM in M bands (set_band_blocks). Tiles past the last whole band take
  // the grouped raster.
  if (g.sh_a > 0) {
    const int64_t a = g.sh_a, b = g.sh_b, xn = g.sh_xn, bm = a * (8 / xn), per = a * b;
    const int64_t full = Mv / bm * bm * Nt;   // 8 * per tiles per band
    if (t < full) {
      const int64_t x = t % 8, l = t / 8, k = l / per, j = l % per;
      return tile_at(k * bm + (x / xn) * a + j % a, (x % xn) * b + j / a, Mt);
    }
    t -= full;
    T -= full;
    mfirst = Mv / bm * bm;
    Mv -= mfirst;
  }
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
  return tile_at(mfirst + first + r % gsize, r / gsize, Mt);
}

// Two floats as packed bf16 (round to nearest even), low half first.
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const bf16x2 v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}

template <typename T, bool AK, bool BK, GemmEpilogue EPI, typename LT, bool CT>
__device__ __forceinline__ void gemm_body(const GemmArgs& g) {
  // The logits epilogues: the product's own rows (Logits), or student rows
  // beside teacher logits read from memory (LogitsTeacher: fp32,
  // LogitsTeacher16: bf16).
  constexpr bool kTeacherEpi = EPI == GemmEpilogue::LogitsTeacher || EPI == GemmEpilogue::LogitsTeacher16;
  constexpr bool kLogitsEpi = EPI == GemmEpilogue::Logits || kTeacherEpi;
  // Ring layout: A tiles of slots 0-3, then B tiles of slots 0-3 (16 KB
  // each), so every slot offset fits a DS instruction's immediate.
  __shared__ __attribute__((aligned(1024))) unsigned char smem[kRing * kStageBytes + kEpiLds];
  unsigned char* const epi = smem + kRing * kStageBytes;
  auto tileA = [&](int s) -> unsigned char* { return smem + s * kOpBytes; };
  auto tileB = [&](int s) -> unsigned char* { return smem + (kRing + s) * kOpBytes; };
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: M0 of the DMA
  const int wm = wave >> 1, wn = wave & 1;
  // Split K: workgroup s*T + t computes tile t over K range
  // [s*split_len, (s+1)*split_len) into split s's partial buffer.
  const int64_t tiles = ((g.M + kTile - 1) / kTile) * ((g.N + kTile - 1) / kTile) * g.nprob;
  int64_t lin = blockIdx.x, kbeg = 0, Kl = g.K;
  int split = 0;
  if (g.split_k > 1) {
    split = static_cast<int>(lin / tiles);
    lin -= static_cast<int64_t>(split) * tiles;
    kbeg = static_cast<int64_t>(split) * g.split_len;
    Kl = g.K - kbeg < g.split_len ? g.K - kbeg : g.split_len;
  }
  const TileCoord tc = map_tile(g, lin);
  GemmProblem pr = g.prob[tc.p];
  if (g.split_k > 1) {
    constexpr int ES = Elem<T>::kSize;
    pr.a = static_cast<const unsigned char*>(pr.a) + kbeg * (AK ? 1 : g.lda) * ES;
    pr.b = static_cast<const unsigned char*>(pr.b) + kbeg * (BK ? 1 : g.ldb) * ES;
    pr.c = static_cast<float*>(pr.c) + static_cast<int64_t>(split) * g.split_stride;
  }
  // A loader over this workgroup's K range (paired rows read in place for
  // the paired logits GEMM).
  auto init_a = [&](Loader<T, AK>& l) {
    if constexpr (EPI == GemmEpilogue::Logits && AK && Elem<T>::kSize == 2) {
      if (g.lg.pair_rows > 0) {
        l.init_paired(pr.a, g.lg.pair_teacher, g.lda, g.lg.pair_rows, Kl, tc.m0 >> 1, wave, lane);
        return;
      }
    }
    l.init(pr.a, g.lda, g.M, Kl, tc.m0, wave, lane);
  };
  // B loader over this workgroup's K range.
  using LoaderB = Loader<T, BK>;
  auto init_b = [&](LoaderB& l) { l.init(pr.b, g.ldb, g.N, Kl, tc.n0, wave, lane); };

  // Logits: this thread's tile-row label, loaded now so that it has long
  // landed when the epilogue needs it (tile row -> student row as in the
  // epilogue's out_row). A global (not flat) load: a flat load would also
  // count in lgkmcnt and turn the main loop's LDS waits into lgkmcnt(0).
  int64_t lab_pre = 0;
  if constexpr (kLogitsEpi) {
    typedef __attribute__((address_space(1))) const int64_t global_i64;
    const int64_t R = static_cast<int64_t>(tc.m0) + tid;
    const int64_t prs = g.lg.pair_rows;
    const int64_t r = prs > 0 ? ((R >> 5) << 4) + (R & 15) : R;
    const bool ok = prs > 0 ? r < prs : R < g.M;
    lab_pre = ok ? *(global_i64*)(reinterpret_cast<uintptr_t>(g.lg.labels + r)) : g.lg.ignore_index;
  }

  f32x4 acc[kFrag][kFrag];
#pragma unroll
  for (int i = 0; i < kFrag; ++i)
#pragma unroll
    for (int j = 0; j < kFrag; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  constexpr int SK = kSlab / Elem<T>::kSize;
  // The logits epilogue takes swapped MFMA operands, so that each lane owns
  // 4 consecutive columns of a row; the store epilogues (grad_hidden, and
  // grad_W computed transposed) take them unswapped.
  constexpr bool kSwapAB = kLogitsEpi;

  const int nkf = static_cast<int>(Kl / SK);   // full stages
  u32x4 ra[2][kFrag], rb[2][kFrag];
  auto read_stage = [&](int slot_idx, u32x4 (&rA)[kFrag], u32x4 (&rB)[kFrag]) {
#pragma unroll
    for (int i = 0; i < kFrag; ++i) rA[i] = read_frag<T, AK>(tileA(slot_idx), wm * 128 + i * 16, lane);
#pragma unroll
    for (int j = 0; j < kFrag; ++j) rB[j] = read_frag<T, BK>(tileB(slot_idx), wn * 128 + j * 16, lane);
  };
  int st_done = 0;   // stages consumed by the main loop
  if constexpr (Elem<T>::kSize == 2) {
    // Stage pairs (128-byte K-major rows) when both operands are K-major;
    // when only A is, A moves in pairs inside the single-stage loop (the
    // transpose reads of an MN-major operand need the whole iteration);
    // single stages when neither is.
    constexpr bool kPaired = AK && BK;
    constexpr bool kHybrid = AK && !BK;
    // LDS byte address of the ring and of this wave's 1 KB DMA block.
    // The base is hidden from the optimiser: otherwise it folds the B tiles'
    // 64 KB offset into the per-read constant, which then no longer fits the
    // 16-bit immediate and costs a VALU op per read.
    uint32_t lds0 = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(
        static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void*)smem))));
    asm volatile("" : "+s"(lds0));
    const uint32_t m0wave = lds0 + static_cast<uint32_t>(wave) * 1024;
    FragReader<AK, AK> fa;
    FragReader<BK, kPaired> fb;
    fa.init(lds0, wm * 128, lane);
    fb.init(lds0 + kRing * kOpBytes, wn * 128, lane);
    __builtin_amdgcn_sched_barrier(0);
    mfma_prime();
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kPaired) {
      // The ring holds two stage pairs (64 elements of K each): pair p sits in
      // double slot p%2, stage s in half s%2 of double slot (s/2)%2.
      //
      // Iteration s computes stage s from registers and reads stage s+1's
      // fragments into the other register set. An even iteration s reads
      // first, all in its first MFMA pairs; at its barrier (MFMA pair kMid)
      // every wave has finished reading stages s and s+1 (the latter just
      // now, with an LDS wait before the barrier), so their double slot is
      // free and the DMA of pair s/2 + 2 into it follows, spread over the
      // rest of the iteration. An odd iteration s starts by waiting for its
      // own DMAs of pair (s+1)/2 (the newer pair stays in flight) and a
      // barrier, after which every wave's share of that pair has landed. Each
      // pair thus has nearly three iterations to land and up to two pairs are
      // in flight. Past the last pair the DMA re-reads the last pair into a
      // double slot nobody reads again, so the wait counts stay exact.
      //
      // With one wave per SIMD nothing else fills the matrix pipe, so the side
      // operations ride between the MFMAs (64 per stage, issued as 32 pairs).
      PairLoader<AK> pa;
      PairLoader<BK> pb;
      if (EPI == GemmEpilogue::Logits && g.lg.pair_rows > 0)
        pa.init_paired(pr.a, g.lg.pair_teacher, g.lda, g.lg.pair_rows, tc.m0 >> 1, wave, lane);
      else
        pa.init(pr.a, g.lda, g.M, tc.m0, wave, lane);
      pb.init(pr.b, g.ldb, g.N, tc.n0, wave, lane);
      const int np = nkf / 2;
      // Transfer x (0-7 A, 8-15 B) of a pair's DMA into double slot D, from
      // the pair's sources sa, sb.
      auto dma_op = [&](auto d_c, int x, uint64_t sa, uint64_t sb) {
        constexpr int MA = decltype(d_c)::value * 2 * kOpBytes;
        constexpr int MB = MA + kRing * kOpBytes;
        switch (x) {   // 0-7: A transfers, 8-15: B transfers
          case 0: dma16_at<MA + 0 * 4096>(sa, pa.goff[0], m0wave); break;
          case 1: dma16_at<MA + 1 * 4096>(sa, pa.goff[1], m0wave); break;
          case 2: dma16_at<MA + 2 * 4096>(sa, pa.goff[2], m0wave); break;
          case 3: dma16_at<MA + 3 * 4096>(sa, pa.goff[3], m0wave); break;
          case 4: dma16_at<MA + 4 * 4096>(sa, pa.goff[4], m0wave); break;
          case 5: dma16_at<MA + 5 * 4096>(sa, pa.goff[5], m0wave); break;
          case 6: dma16_at<MA + 6 * 4096>(sa, pa.goff[6], m0wave); break;
          case 7: dma16_at<MA + 7 * 4096>(sa, pa.goff[7], m0wave); break;
          case 8: dma16_at<MB + 0 * 4096>(sb, pb.goff[0], m0wave); break;
          case 9: dma16_at<MB + 1 * 4096>(sb, pb.goff[1], m0wave); break;
          case 10: dma16_at<MB + 2 * 4096>(sb, pb.goff[2], m0wave); break;
          case 11: dma16_at<MB + 3 * 4096>(sb, pb.goff[3], m0wave); break;
          case 12: dma16_at<MB + 4 * 4096>(sb, pb.goff[4], m0wave); break;
          case 13: dma16_at<MB + 5 * 4096>(sb, pb.goff[5], m0wave); break;
          case 14: dma16_at<MB + 6 * 4096>(sb, pb.goff[6], m0wave); break;
          default: dma16_at<MB + 7 * 4096>(sb, pb.goff[7], m0wave); break;
        }
      };
      if (np > 0) {
        {
          const uint64_t sa = uniform64(pa.src(0)), sb = uniform64(pb.src(0));
  #pragma unroll
          for (int x = 0; x < 16; ++x) dma_op(SlotC<0>{}, x, sa, sb);
        }
        if (np > 1) {
          const uint64_t sa = uniform64(pa.src(1)), sb = uniform64(pb.src(1));
  #pragma unroll
          for (int x = 0; x < 16; ++x) dma_op(SlotC<1>{}, x, sa, sb);
          __builtin_amdgcn_s_waitcnt(vm_wait(16));   // pair 0 landed
        } else {
          __builtin_amdgcn_s_waitcnt(kWaitAll);
        }
        __builtin_amdgcn_s_barrier();
  #pragma unroll
        for (int o = 0; o < FragReader<AK, AK>::kOps; ++o) fa.template read_op<0>(o, ra[0]);
  #pragma unroll
        for (int o = 0; o < FragReader<BK, kPaired>::kOps; ++o) fb.template read_op<0>(o, rb[0]);
        __builtin_amdgcn_sched_barrier(0);
      }
      constexpr int kOpsA = FragReader<AK, AK>::kOps, kOpsB = FragReader<BK, kPaired>::kOps;
      constexpr int kReads = kOpsA + kOpsB;
      // MFMA pair of an even iteration's barrier. The earlier the barrier,
      // the longer the next pair has to land: measured 13.4 ms at pair 22,
      // 13.1 ms at 16, 12.8 ms at 10, 12.7 ms at 6 and 12.8 ms at 4 (and,
      // with the final epilogue, 0.5 % slower at 5 and at 7 than at 6).
      constexpr int kMid = 6;
      // MFMA pairs the pair's 16 transfers spread over: all the rest of the
      // iteration (over 16 pairs measured 4 % slower, over 8 pairs 8 %).
      constexpr int kSpan = 32 - kMid;
      auto iter = [&](auto slot_c, int st, u32x4 (&rnA)[kFrag], u32x4 (&rnB)[kFrag],
                      const u32x4 (&rcA)[kFrag], const u32x4 (&rcB)[kFrag]) {
        constexpr int S = decltype(slot_c)::value;   // stage s % 4
        constexpr int SN = (S + 1) % kRing;          // stage s+1 % 4
        constexpr bool kOdd = (S & 1) != 0;
        // LDS reads spread over the pairs before the barrier (even) or over
        // the whole iteration (odd); an even iteration's DMAs follow its barrier.
        constexpr int kReadPairs = kOdd ? 32 : kMid - 2;
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (kOdd) {
          __builtin_amdgcn_s_waitcnt(vm_wait(16));   // pair (s+1)/2 landed
          __builtin_amdgcn_s_barrier();
        }
        __builtin_amdgcn_sched_barrier(0);
        uint64_t sa = 0, sb = 0;
  #pragma unroll
        for (int pr = 0; pr < 32; ++pr) {
          if (!kOdd && pr == kMid - 4) {
            // DMA sources of pair s/2 + 2, computed here so the scalar work
            // overlaps MFMAs.
            const int p = (st >> 1) + 2;
            const int nxt = p < np ? p : np - 1;
            sa = uniform64(pa.src(nxt));
            sb = uniform64(pb.src(nxt));
          }
          if (!kOdd && pr == kMid) {
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(kWaitLds);
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
          }
  #pragma unroll
          for (int o = 0; o < kReads; ++o) {
            if ((o * kReadPairs) / kReads != pr) continue;
            if (o < kOpsA)
              fa.template read_op<SN>(o, rnA);
            else
              fb.template read_op<SN>(o - kOpsA, rnB);
          }
          if constexpr (!kOdd) {
            // the pair's 16 transfers, spread over the pairs after the barrier
#pragma unroll
            for (int x = 0; x < 16; ++x)
              if (kMid + (x * kSpan) / 16 == pr) dma_op(SlotC<(S >> 1)>{}, x, sa, sb);
          }
  #pragma unroll
          for (int q = 0; q < 2; ++q) {
            const int mm = 2 * pr + q;
            if constexpr (kSwapAB)
              mfma_bf16(acc[mm & 7][mm >> 3], rcB[mm >> 3], rcA[mm & 7]);
            else
              mfma_bf16(acc[mm >> 3][mm & 7], rcA[mm >> 3], rcB[mm & 7]);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      };
      // Unrolled by the ring depth so each slot is a compile-time immediate;
      // the register sets alternate. 2*np is even, so the remainder is 0 or 2.
      const int ns = 2 * np;
      int s0 = 0;
      for (; s0 + 3 < ns; s0 += 4) {
        iter(SlotC<0>{}, s0, ra[1], rb[1], ra[0], rb[0]);
        iter(SlotC<1>{}, s0 + 1, ra[0], rb[0], ra[1], rb[1]);
        iter(SlotC<2>{}, s0 + 2, ra[1], rb[1], ra[0], rb[0]);
        iter(SlotC<3>{}, s0 + 3, ra[0], rb[0], ra[1], rb[1]);
      }
      if (s0 < ns) {
        iter(SlotC<0>{}, s0, ra[1], rb[1], ra[0], rb[0]);
        iter(SlotC<1>{}, s0 + 1, ra[0], rb[0], ra[1], rb[1]);
      }
      st_done = ns;
    } else if constexpr (kHybrid) {
      // K-major A in stage pairs, MN-major B in single stages, in the
      // single-stage loop: one barrier at the top of every iteration, B's
      // transpose reads spread over the whole iteration. Iteration s DMAs B
      // stage s+4 into B slot s%4 and, when s = 2p+1 is odd, A pair p+2 into
      // A's double slot p%2, whose stages 2p and 2p+1 were read in
      // iterations 2p-1 and 2p. An iteration's transfers go out as B's 4,
      // then A's 8, so at the top of iteration s the newest transfers that
      // must have landed (B stage s+1, and the A pair holding stage s+1) are
      // followed by exactly 16 (s even) or 4 (s odd) younger ones. Past the
      // last pair the DMAs re-read stage 0 (B) or the last pair (A) into
      // slots nobody reads again.
      const int np = nkf / 2;
      const int ns = 2 * np;
      PairLoader<AK> pa;
      pa.init(pr.a, g.lda, g.M, tc.m0, wave, lane);
      LoaderB lb;
      init_b(lb);
      // Transfer x (0-7) of an A pair into double slot D.
      auto dma_a = [&](auto d_c, int x, uint64_t sa) {
        constexpr int MA = decltype(d_c)::value * 2 * kOpBytes;
        switch (x) {
          case 0: dma16_at<MA + 0 * 4096>(sa, pa.goff[0], m0wave); break;
          case 1: dma16_at<MA + 1 * 4096>(sa, pa.goff[1], m0wave); break;
          case 2: dma16_at<MA + 2 * 4096>(sa, pa.goff[2], m0wave); break;
          case 3: dma16_at<MA + 3 * 4096>(sa, pa.goff[3], m0wave); break;
          case 4: dma16_at<MA + 4 * 4096>(sa, pa.goff[4], m0wave); break;
          case 5: dma16_at<MA + 5 * 4096>(sa, pa.goff[5], m0wave); break;
          case 6: dma16_at<MA + 6 * 4096>(sa, pa.goff[6], m0wave); break;
          default: dma16_at<MA + 7 * 4096>(sa, pa.goff[7], m0wave); break;
        }
      };
      // Transfer x (0-3) of a B stage into B slot S.
      auto dma_b = [&](auto s_c, int x, uint64_t sb) {
        constexpr int MB = (kRing + decltype(s_c)::value) * kOpBytes;
        switch (x) {
          case 0: dma16_at<MB + 0 * 4096>(sb, lb.goff[0], m0wave); break;
          case 1: dma16_at<MB + 1 * 4096>(sb, lb.goff[1], m0wave); break;
          case 2: dma16_at<MB + 2 * 4096>(sb, lb.goff[2], m0wave); break;
          default: dma16_at<MB + 3 * 4096>(sb, lb.goff[3], m0wave); break;
        }
      };
      if (np > 0) {
        // A pair 0, B stages 0-3, A pair 1; then stage 0 is followed by 20
        // younger transfers.
        uint64_t sa = uniform64(pa.src(0));
#pragma unroll
        for (int x = 0; x < 8; ++x) dma_a(SlotC<0>{}, x, sa);
        uint64_t sb = uniform64(lb.stage_src(0));
#pragma unroll
        for (int x = 0; x < 4; ++x) dma_b(SlotC<0>{}, x, sb);
        sb = uniform64(lb.stage_src(1 < ns ? 1 : 0));
#pragma unroll
        for (int x = 0; x < 4; ++x) dma_b(SlotC<1>{}, x, sb);
        sb = uniform64(lb.stage_src(2 < ns ? 2 : 0));
#pragma unroll
        for (int x = 0; x < 4; ++x) dma_b(SlotC<2>{}, x, sb);
        sb = uniform64(lb.stage_src(3 < ns ? 3 : 0));
#pragma unroll
        for (int x = 0; x < 4; ++x) dma_b(SlotC<3>{}, x, sb);
        sa = uniform64(pa.src(np > 1 ? 1 : 0));
#pragma unroll
        for (int x = 0; x < 8; ++x) dma_a(SlotC<1>{}, x, sa);
        __builtin_amdgcn_s_waitcnt(vm_wait(20));
        __builtin_amdgcn_s_barrier();
#pragma unroll
        for (int o = 0; o < FragReader<AK, AK>::kOps; ++o) fa.template read_op<0>(o, ra[0]);
#pragma unroll
        for (int o = 0; o < FragReader<BK, kPaired>::kOps; ++o) fb.template read_op<0>(o, rb[0]);
        __builtin_amdgcn_sched_barrier(0);
      }
      constexpr int kOpsA = FragReader<AK, AK>::kOps, kOpsB = FragReader<BK, kPaired>::kOps;
      constexpr int kReads = kOpsA + kOpsB;
      auto iter = [&](auto slot_c, int st, u32x4 (&rnA)[kFrag], u32x4 (&rnB)[kFrag],
                      const u32x4 (&rcA)[kFrag], const u32x4 (&rcB)[kFrag]) {
        constexpr int S = decltype(slot_c)::value;   // stage s % 4
        constexpr int SN = (S + 1) % kRing;          // stage s+1 % 4
        constexpr bool kOdd = (S & 1) != 0;
        constexpr int kDma = kOdd ? 12 : 4;
        constexpr int kSide = kReads + kDma;   // reads keep the slots of a kSide spread
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(kOdd ? vm_wait(4) : vm_wait(16));
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        uint64_t sa = 0, sb = 0;
#pragma unroll
        for (int pr = 0; pr < 32; ++pr) {
          // The slots the DMAs fill were freed by the barrier above. B's
          // transfers go out with MFMA pairs 1-4 and A's with every other
          // pair from 14 to 28 (the order B then A keeps the vmcnt counts
          // above). Measured against the earlier placement after all reads
          // (pairs 21-31): A from pair 14 or 15 runs 3.5-4.5 % faster, and
          // every other pair a further 0.7 %; A from pairs 5-12 runs up to
          // 9 % slower.
          constexpr int kB0 = 1, kA0 = 14;   // first MFMA pair of B's / A's transfers
          constexpr int kAS = 2;             // MFMA pairs between A's transfers
          if (pr >= kB0 && pr < kB0 + 4) dma_b(SlotC<S>{}, pr - kB0, sb);
          if (kOdd && pr >= kA0 && pr < kA0 + 8 * kAS && (pr - kA0) % kAS == 0)
            dma_a(SlotC<(S >> 1)>{}, (pr - kA0) / kAS, sa);
#pragma unroll
          for (int o = 0; o < kReads; ++o) {
            if ((o * 32) / kSide != pr) continue;
            if (o < kOpsA)
              fa.template read_op<SN>(o, rnA);
            else
              fb.template read_op<SN>(o - kOpsA, rnB);
          }
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            const int mm = 2 * pr + q;
            if constexpr (kSwapAB)
              mfma_bf16(acc[mm & 7][mm >> 3], rcB[mm >> 3], rcA[mm & 7]);
            else
              mfma_bf16(acc[mm >> 3][mm & 7], rcA[mm >> 3], rcB[mm & 7]);
          }
          if (pr == 0) {
            // DMA sources (B stage s+4, A pair s/2 + 2), computed behind the
            // first MFMAs.
            const int nb = st + kRing < ns ? st + kRing : 0;
            sb = uniform64(lb.stage_src(nb));
            if constexpr (kOdd) {
              const int p = (st >> 1) + 2;
              sa = uniform64(pa.src(p < np ? p : np - 1));
            }
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      };
      int s0 = 0;
      for (; s0 + 3 < ns; s0 += 4) {
        iter(SlotC<0>{}, s0, ra[1], rb[1], ra[0], rb[0]);
        iter(SlotC<1>{}, s0 + 1, ra[0], rb[0], ra[1], rb[1]);
        iter(SlotC<2>{}, s0 + 2, ra[1], rb[1], ra[0], rb[0]);
        iter(SlotC<3>{}, s0 + 3, ra[0], rb[0], ra[1], rb[1]);
      }
      if (s0 < ns) {
        iter(SlotC<0>{}, s0, ra[1], rb[1], ra[0], rb[0]);
        iter(SlotC<1>{}, s0 + 1, ra[0], rb[0], ra[1], rb[1]);
      }
      st_done = ns;
    } else {
      static_assert(AK, "the bf16 GEMMs take a K-major A");
    }
    __builtin_amdgcn_sched_barrier(0);
    mfma_drain();
    __builtin_amdgcn_sched_barrier(0);
  } else {
    // fp32: an MFMA stage is long (256 v_mfma_f32_16x16x4_f32), so one
    // register set suffices: DMA three stages ahead into the slot read one
    // stage ago, read this stage after the barrier, then compute. Every
    // iteration issues the same number of DMA transfers (past the last full
    // stage, an in-bounds dummy copy of stage 0 into a slot nobody reads
    // again), so one constant vmcnt wait always means "stage s has landed".
    Loader<T, AK> la;
    LoaderB lb;
    init_a(la);
    init_b(lb);
    auto issue_stage = [&](int slot_idx, int st) {
      const int src = st < nkf ? st : 0;
      la.issue(tileA(slot_idx), src, wave, lane);
      lb.issue(tileB(slot_idx), src, wave, lane);
    };
    if (nkf > 0)
      for (int t = 0; t < kRing - 1; ++t) issue_stage(t, t);
    for (int st = 0; st < nkf; ++st) {
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(kWaitTwoStages);
      __builtin_amdgcn_s_barrier();
      read_stage(st % kRing, ra[0], rb[0]);
      __builtin_amdgcn_sched_barrier(0);
      issue_stage((st + kRing - 1) % kRing, st + kRing - 1);
      __builtin_amdgcn_sched_barrier(0);
      mfma_step<T, kSwapAB>(acc, ra[0], rb[0]);
    }
    st_done = nkf;
  }
  if (static_cast<int64_t>(st_done) * SK < Kl) {
    // Stages the main loop left — after the bf16 pairs an odd full stage,
    // and a partial last stage — one at a time through slot 0 in the
    // single-stage layout: DMA the valid part, zero the rest.
    Loader<T, AK> la;
    LoaderB lb;
    init_a(la);
    init_b(lb);
    auto tail_stage = [&](int st) {
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(kWaitAll);
      __builtin_amdgcn_s_barrier();
      la.issue(tileA(0), st, wave, lane);
      lb.issue(tileB(0), st, wave, lane);
      __builtin_amdgcn_s_waitcnt(kWaitAll);
      __builtin_amdgcn_s_barrier();
      read_stage(0, ra[1], rb[1]);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(kWaitAll);
      __builtin_amdgcn_sched_barrier(0);
      mfma_step<T, kSwapAB>(acc, ra[1], rb[1]);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (Elem<T>::kSize == 2) mfma_drain();
    };
    for (int st = st_done; static_cast<int64_t>(st) * SK < Kl; ++st) tail_stage(st);
  }
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(kWaitAll);
  __builtin_amdgcn_s_barrier();

  // ------------------------------------------------------------ epilogue
  const int lrow = lane & 15;
  const int lgrp = lane >> 4;
  if constexpr (EPI == GemmEpilogue::StoreF32 || EPI == GemmEpilogue::AccumF32) {
    float* C = static_cast<float*>(pr.c);
    const float alpha = g.alpha_ptr != nullptr ? g.alpha * *g.alpha_ptr : g.alpha;
    static_assert(!kSwapAB, "the store epilogues take unswapped operands");
    // acc[i][j][e] is row wm*128 + 16i + 4*lgrp + e, column wn*128 + 16j + lrow.
    const int row_w = tc.m0 + wm * 128;
    const int col_l = tc.n0 + wn * 128 + lrow;
    if constexpr (CT) {
      // C[n][m]: each lane holds 4 consecutive m of one n, one 16-byte
      // store where the pitch and base allow (lanes lrow + 16g write 64
      // contiguous bytes of row n).
      const bool vec = (g.ldc % 4) == 0 && (reinterpret_cast<uintptr_t>(C) % 16) == 0;
#pragma unroll
      for (int j = 0; j < kFrag; ++j) {
        const int64_t n = col_l + j * 16;
        if (n >= g.N) continue;
        float* cn = C + n * g.ldc;
#pragma unroll
        for (int i = 0; i < kFrag; ++i) {
          const int64_t m = row_w + i * 16 + lgrp * 4;
          f32x4 v = acc[i][j];
          if (vec && m + 4 <= g.M) {
            f32x4* dst = reinterpret_cast<f32x4*>(cn + m);
            if constexpr (EPI == GemmEpilogue::AccumF32) v = alpha * (*dst + v);
            else v = alpha * v;
            *dst = v;
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if (m + e < g.M) {
                float x = v[e];
                if constexpr (EPI == GemmEpilogue::AccumF32) x = alpha * (cn[m + e] + x);
                else x = alpha * x;
                cn[m + e] = x;
              }
            }
          }
        }
      }
      return;
    }
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
            if constexpr (EPI == GemmEpilogue::AccumF32) v = alpha * (crow[col] + v);
            else v = alpha * v;
            crow[col] = v;
          }
        }
      }
    }
  } else {
    // Logits: per-row partial softmax statistics of this 256-column tile, the
    // label logit, and the logits themselves. The accumulators hold
    // transposed blocks (kSwapAB): acc[i][j][e] is row wm*128 + 16i + lrow,
    // column wn*128 + 16j + 4*lgrp + e, so a lane owns 8 rows x 32 columns
    // and each row's 128 columns of this wave sit in the 4 lanes lrow + 16g.
    // With paired rows (pair_rows > 0) fragments 2q and 2q+1 hold a block of
    // student rows and the same teacher rows, so a lane also holds both
    // logits of every (row, column) it owns and forms the KL cross term.
    LT* C = static_cast<LT*>(pr.c);
    int64_t* lab = reinterpret_cast<int64_t*>(epi);                      // [256]
    float4* part = reinterpret_cast<float4*>(epi + 2048);                // [2][256]
    float2* xpart = reinterpret_cast<float2*>(epi + 10240);              // [2][256]
    const int64_t prs = g.lg.pair_rows;
    // Tile row rl as (output row, teacher?, valid): stats / xy / C row index.
    auto out_row = [&](int rl, bool& teacher, bool& valid) -> int64_t {
      if (prs > 0) {
        const int64_t R = static_cast<int64_t>(tc.m0) + rl;
        const int64_t r = ((R >> 5) << 4) + (R & 15);
        teacher = ((R >> 4) & 1) != 0;
        valid = r < prs;
        return teacher ? prs + r : r;
      }
      teacher = false;
      valid = tc.m0 + rl < g.M;
      return static_cast<int64_t>(tc.p) * g.M + tc.m0 + rl;
    };
    lab[tid] = lab_pre;
    __syncthreads();
    const float it2 = g.lg.inv_t * kLog2e;
    const int64_t colw = static_cast<int64_t>(tc.n0) + wn * 128 + 4 * lgrp;   // (j, e) = (0, 0)
    const int64_t ncol64 = g.N - colw;                    // (j, e) valid iff 16j + e < ncol
    const int ncol = static_cast<int>(ncol64 < 128 ? (ncol64 < 0 ? 0 : ncol64) : 128);
    // This lane's 32 logits of one row, from column colw on.
    auto store_row = [&](auto full_c, LT* crow, const f32x4 (&v)[kFrag]) {
      constexpr bool kFull = decltype(full_c)::value;
#pragma unroll
      for (int j = 0; j < kFrag; ++j) {
        if (kFull || j * 16 + 4 <= ncol) {
          if constexpr (Elem<LT>::kSize == 2) {
            u32x2 w;
            w[0] = pack_bf16(v[j][0], v[j][1]);
            w[1] = pack_bf16(v[j][2], v[j][3]);
            *reinterpret_cast<u32x2*>(crow + j * 16) = w;
          } else {
            *reinterpret_cast<f32x4*>(crow + j * 16) = v[j];
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (j * 16 + e < ncol) crow[j * 16 + e] = static_cast<LT>(v[j][e]);
        }
      }
    };
    // bf16 rows of full tiles leave as 16-byte stores: for each fragment pair
    // (j, j+1), one v_permlane16_swap per dword gives the lanes of 16-lane
    // row g (g = lane/16) eight consecutive columns, 16*(j + g%2) + 8*(g/2)
    // onward, so a store instruction writes 64 contiguous bytes of each of 16
    // rows instead of 32. Done by every lane (the swap pairs lanes 16 apart,
    // which hold the same row); the stores follow under the row's test.
    auto swap_rows = [&](const f32x4 (&v)[kFrag], u32x4 (&w)[kFrag / 2]) {
#pragma unroll
      for (int jp = 0; jp < kFrag; jp += 2) {
        const auto a = __builtin_amdgcn_permlane16_swap(pack_bf16(v[jp][0], v[jp][1]),
                                                        pack_bf16(v[jp + 1][0], v[jp + 1][1]),
                                                        false, false);
        const auto b = __builtin_amdgcn_permlane16_swap(pack_bf16(v[jp][2], v[jp][3]),
                                                        pack_bf16(v[jp + 1][2], v[jp + 1][3]),
                                                        false, false);
        w[jp / 2] = u32x4{a[0], b[0], a[1], b[1]};
      }
    };
    // rowbase: the row's element at column tc.n0 + wn*128. Non-temporal
    // stores: the logits are read again only by the row pass, after gigabytes
    // of other traffic, and as ordinary stores they displace operand strips
    // from L2 (measured 0.04-0.1 ms faster on the logits GEMM; the same for
    // grad_W's fp32 stores measured 0.27 ms slower).
    auto store_swapped = [&](LT* rowbase, const u32x4 (&w)[kFrag / 2]) {
      const int c0 = 16 * (lgrp & 1) + 8 * (lgrp >> 1);
#pragma unroll
      for (int jp = 0; jp < kFrag; jp += 2)
        __builtin_nontemporal_store(w[jp / 2], reinterpret_cast<u32x4*>(rowbase + 16 * jp + c0));
    };
    constexpr bool kSwapStore = Elem<LT>::kSize == 2;
    // bf16 logits are stored as t = (x - m)·log2(e), m the row's maximum over
    // this wave's 128 columns (written to hmax after the merge below): the
    // first exponent's argument, so e^((x-m)/T) = 2^(t/T) costs no more.
    constexpr bool kRel = Elem<LT>::kSize == 2;
    const float inv_t = g.lg.inv_t;
    // The label's logit, if this lane holds its column (16j + e == yl):
    // select e, then j.
    auto pick = [&](const f32x4 (&v)[kFrag], int yl) {
      const int jy = yl >> 4, ey = yl & 3;
      float xy = 0.f;
#pragma unroll
      for (int j = 0; j < kFrag; ++j) {
        float t = v[j][0];
        t = ey == 1 ? v[j][1] : t;
        t = ey == 2 ? v[j][2] : t;
        t = ey == 3 ? v[j][3] : t;
        xy = jy == j ? t : xy;
      }
      return xy;
    };
    auto quad_max = [](float x) {
      x = fmaxf(x, __shfl_xor(x, 16));
      return fmaxf(x, __shfl_xor(x, 32));
    };
    auto quad_sum = [](float x) {
      x += __shfl_xor(x, 16);
      return x + __shfl_xor(x, 32);
    };
    // Full tiles (all but the last column tile when N % 256 != 0) take a
    // path without per-column checks.
    auto rows = [&](auto full_c) {
      constexpr bool kFull = decltype(full_c)::value;
#pragma unroll
      for (int i = 0; i < kFrag; ++i) {
        f32x4 av[kFrag];
#pragma unroll
        for (int j = 0; j < kFrag; ++j) av[j] = from_acc(acc[i][j]);
        const int rl = wm * 128 + i * 16 + lrow;           // row within tile
        const int64_t row = tc.m0 + rl;
        const int64_t yl64 = lab[rl] - colw;
        const int yl = (yl64 >= 0 && yl64 < 128) ? static_cast<int>(yl64) : -1;
        float mx = -INFINITY;
        if constexpr (kFull) {
          mx = row_max32(av);
        } else {
#pragma unroll
          for (int j = 0; j < kFrag; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (j * 16 + e < ncol) mx = fmaxf(mx, av[j][e]);
        }
        mx = quad_max(mx);
        // exp((x - mx)) and exp((x - mx)/T) as exp2 of one fma each.
        const float o1 = -mx * kLog2e, oT = -mx * it2;
        const bool hit = yl >= 0 && (yl & 12) == 0;
        float xyv = 0.f;   // the label's fp32 logit, before av holds t
        if constexpr (kRel) {
          if (hit) xyv = pick(av, yl);
        }
        float d1 = 0.f, dT = 0.f, sx = 0.f;
#pragma unroll
        for (int j = 0; j < kFrag; ++j) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float x = av[j][e];
            float a1, aT;
            if constexpr (kRel) {
              const float t = fmaf(x, kLog2e, o1);
              a1 = __builtin_amdgcn_exp2f(t);
              aT = __builtin_amdgcn_exp2f(t * inv_t);
              av[j][e] = t;
            } else {
              a1 = __builtin_amdgcn_exp2f(fmaf(x, kLog2e, o1));
              aT = __builtin_amdgcn_exp2f(fmaf(x, it2, oT));
            }
            if (kFull || j * 16 + e < ncol) {
              d1 += a1;
              dT += aT;
              sx += x;
            }
          }
        }
        d1 = quad_sum(d1);
        dT = quad_sum(dT);
        sx = quad_sum(sx);
        if (lgrp == 0) part[wn * 256 + rl] = make_float4(mx, d1, dT, sx);
        u32x4 aw[kFrag / 2];
        if constexpr (kSwapStore && kFull) swap_rows(av, aw);
        if (row < g.M) {
          if (hit) g.lg.xy[tc.p * g.M + row] = kRel ? xyv : pick(av, yl);
          if constexpr (kSwapStore && kFull)
            store_swapped(C + row * g.ldc + (colw - 4 * lgrp), aw);
          else
            store_row(full_c, C + row * g.ldc + colw, av);
        }
      }
    };
    auto rows_pair = [&](auto full_c) {
      constexpr bool kFull = decltype(full_c)::value;
#pragma unroll
      for (int q = 0; q < kFrag / 2; ++q) {
        f32x4 as[kFrag], at[kFrag];
#pragma unroll
        for (int j = 0; j < kFrag; ++j) as[j] = from_acc(acc[2 * q][j]);
#pragma unroll
        for (int j = 0; j < kFrag; ++j) at[j] = from_acc(acc[2 * q + 1][j]);
        const int rs = wm * 128 + q * 32 + lrow;                         // tile rows
        const int rt = rs + 16;
        const int64_t row = (tc.m0 >> 1) + wm * 64 + q * 16 + lrow;      // student row
        const int64_t yl64 = lab[rs] - colw;
        const int yl = (yl64 >= 0 && yl64 < 128) ? static_cast<int>(yl64) : -1;
        float ms = -INFINITY, mt = -INFINITY;
        if constexpr (kFull) {
          ms = row_max32(as);
          mt = row_max32(at);
        } else {
#pragma unroll
          for (int j = 0; j < kFrag; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (j * 16 + e < ncol) {
                ms = fmaxf(ms, as[j][e]);
                mt = fmaxf(mt, at[j][e]);
              }
        }
        ms = quad_max(ms);
        mt = quad_max(mt);
        const float o1s = -ms * kLog2e, o1t = -mt * kLog2e;
        const bool hit = yl >= 0 && (yl & 12) == 0;
        float xys = 0.f, xyt = 0.f;   // the label's fp32 logits, before as/at hold t
        if constexpr (kRel) {
          if (hit) {
            xys = pick(as, yl);
            xyt = pick(at, yl);
          }
        }
        // Per element pair, in log2 units relative to the rows' own half
        // maxima: ts, tt (the stored values), e^((x-m)/T) = 2^(t/T). The KL
        // sums take (tt - ts) and (aTs - aTt), so a constant offset between
        // the two rows cancels in each element; Σ aTs = dd + Σ aTt.
        float d1s = 0.f, sxs = 0.f, d1t = 0.f, dTt = 0.f, sxt = 0.f, cx = 0.f, dd = 0.f;
#pragma unroll
        for (int j = 0; j < kFrag; ++j) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float xs = as[j][e], xt = at[j][e];
            const float ts = fmaf(xs, kLog2e, o1s), tt = fmaf(xt, kLog2e, o1t);
            const float a1s = __builtin_amdgcn_exp2f(ts);
            const float aTs = __builtin_amdgcn_exp2f(ts * inv_t);
            const float a1t = __builtin_amdgcn_exp2f(tt);
            const float aTt = __builtin_amdgcn_exp2f(tt * inv_t);
            if constexpr (kRel) {
              as[j][e] = ts;
              at[j][e] = tt;
            }
            if (kFull || j * 16 + e < ncol) {
              d1s += a1s;
              dd += aTs - aTt;
              sxs += xs;
              d1t += a1t;
              dTt += aTt;
              sxt += xt;
              cx = fmaf(aTt, tt - ts, cx);
            }
          }
        }
        d1s = quad_sum(d1s);
        dd = quad_sum(dd);
        sxs = quad_sum(sxs);
        d1t = quad_sum(d1t);
        dTt = quad_sum(dTt);
        sxt = quad_sum(sxt);
        cx = quad_sum(cx);
        const float dTs = dd + dTt;
        if (lgrp == 0) {
          part[wn * 256 + rs] = make_float4(ms, d1s, dTs, sxs);
          part[wn * 256 + rt] = make_float4(mt, d1t, dTt, sxt);
          xpart[wn * 256 + rt] = make_float2(cx, dd);
        }
        u32x4 sw[kFrag / 2], tw[kFrag / 2];
        if constexpr (kSwapStore && kFull) {
          swap_rows(as, sw);
          swap_rows(at, tw);
        }
        if (row < prs) {
          if (hit) {   // one lane of a row at most, for one column tile
            g.lg.xy[row] = kRel ? xys : pick(as, yl);
            g.lg.xy[prs + row] = kRel ? xyt : pick(at, yl);
          }
          if constexpr (kSwapStore && kFull) {
            store_swapped(C + row * g.ldc + (colw - 4 * lgrp), sw);
            store_swapped(C + (prs + row) * g.ldc + (colw - 4 * lgrp), tw);
          } else {
            store_row(full_c, C + row * g.ldc + colw, as);
            store_row(full_c, C + (prs + row) * g.ldc + colw, at);
          }
        }
      }
    };
    // Teacher logits beside the student rows (LogitsTeacher, LogitsTeacher16):
    // per row block the lane's 32 teacher logits of its row are loaded
    // (16-byte vectors of fp32 or 8-byte vectors of bf16, one block ahead,
    // so that they are in flight while the previous block computes) and take
    // the place of the paired GEMM's teacher accumulators: the teacher's
    // half-tile statistics and label logit and the two KL sums come out as
    // with paired rows. Only the student rows are stored. The teacher's half
    // statistics go to partT, in the ring (idle once the main loop has
    // drained). Non-temporal loads: the logits are read again only by the row
    // pass, and the L2 holds the operand strips.
    float4* partT = reinterpret_cast<float4*>(smem);   // [2][256]
    auto load_t = [&](auto full_c, int i, f32x4 (&tv)[kFrag]) {
      constexpr bool kFull = decltype(full_c)::value;
      const int64_t row = static_cast<int64_t>(tc.m0) + wm * 128 + i * 16 + lrow;
      const int64_t off = (row < g.M ? row : g.M - 1) * g.lg.teacher_ld + colw;
      if constexpr (EPI == GemmEpilogue::LogitsTeacher16) {
        const __bf16* trow = static_cast<const __bf16*>(g.lg.teacher_logits) + off;
#pragma unroll
        for (int j = 0; j < kFrag; ++j) {
          if (kFull || j * 16 + 4 <= ncol) {
            const u32x2 w = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(trow + j * 16));
            tv[j][0] = __uint_as_float(w[0] << 16);
            tv[j][1] = __uint_as_float(w[0] & 0xffff0000u);
            tv[j][2] = __uint_as_float(w[1] << 16);
            tv[j][3] = __uint_as_float(w[1] & 0xffff0000u);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              tv[j][e] = j * 16 + e < ncol ? static_cast<float>(trow[j * 16 + e]) : 0.f;
          }
        }
      } else {
        const float* trow = static_cast<const float*>(g.lg.teacher_logits) + off;
#pragma unroll
        for (int j = 0; j < kFrag; ++j) {
          if (kFull || j * 16 + 4 <= ncol) {
            tv[j] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(trow + j * 16));
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) tv[j][e] = j * 16 + e < ncol ? trow[j * 16 + e] : 0.f;
          }
        }
      }
    };
    auto rows_teacher = [&](auto full_c) {
      constexpr bool kFull = decltype(full_c)::value;
      f32x4 tbuf[2][kFrag];
      load_t(full_c, 0, tbuf[0]);
#pragma unroll
      for (int i = 0; i < kFrag; ++i) {
        if (i + 1 < kFrag) load_t(full_c, i + 1, tbuf[(i + 1) & 1]);
        f32x4 as[kFrag];
#pragma unroll
        for (int j = 0; j < kFrag; ++j) as[j] = from_acc(acc[i][j]);
        const f32x4(&at)[kFrag] = tbuf[i & 1];
        const int rl = wm * 128 + i * 16 + lrow;            // row within tile
        const int64_t row = tc.m0 + rl;
        const int64_t yl64 = lab[rl] - colw;
        const int yl = (yl64 >= 0 && yl64 < 128) ? static_cast<int>(yl64) : -1;
        float ms = -INFINITY, mt = -INFINITY;
        if constexpr (kFull) {
          ms = row_max32(as);
          mt = row_max32(at);
        } else {
#pragma unroll
          for (int j = 0; j < kFrag; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (j * 16 + e < ncol) {
                ms = fmaxf(ms, as[j][e]);
                mt = fmaxf(mt, at[j][e]);
              }
        }
        ms = quad_max(ms);
        mt = quad_max(mt);
        const float o1s = -ms * kLog2e, o1t = -mt * kLog2e;
        const bool hit = yl >= 0 && (yl & 12) == 0;
        float xys = 0.f, xyt = 0.f;   // the label's fp32 logits, before as holds t
        if (hit) {
          xys = pick(as, yl);
          xyt = pick(at, yl);
        }
        // as in rows_pair: log2 units relative to the half maxima, the KL sums
        // over (tt - ts) and (aTs - aTt), Σ aTs = dd + Σ aTt
        float d1s = 0.f, sxs = 0.f, d1t = 0.f, dTt = 0.f, sxt = 0.f, cx = 0.f, dd = 0.f;
#pragma unroll
        for (int j = 0; j < kFrag; ++j) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float xs = as[j][e], xt = at[j][e];
            const float ts = fmaf(xs, kLog2e, o1s), tt = fmaf(xt, kLog2e, o1t);
            const float a1s = __builtin_amdgcn_exp2f(ts);
            const float aTs = __builtin_amdgcn_exp2f(ts * inv_t);
            const float a1t = __builtin_amdgcn_exp2f(tt);
            const float aTt = __builtin_amdgcn_exp2f(tt * inv_t);
            if constexpr (kRel) as[j][e] = ts;
            if (kFull || j * 16 + e < ncol) {
              d1s += a1s;
              dd += aTs - aTt;
              sxs += xs;
              d1t += a1t;
              dTt += aTt;
              sxt += xt;
              cx = fmaf(aTt, tt - ts, cx);
            }
          }
        }
        d1s = quad_sum(d1s);
        dd = quad_sum(dd);
        sxs = quad_sum(sxs);
        d1t = quad_sum(d1t);
        dTt = quad_sum(dTt);
        sxt = quad_sum(sxt);
        cx = quad_sum(cx);
        const float dTs = dd + dTt;
        if (lgrp == 0) {
          part[wn * 256 + rl] = make_float4(ms, d1s, dTs, sxs);
          partT[wn * 256 + rl] = make_float4(mt, d1t, dTt, sxt);
          xpart[wn * 256 + rl] = make_float2(cx, dd);
        }
        u32x4 aw[kFrag / 2];
        if constexpr (kSwapStore && kFull) swap_rows(as, aw);
        if (row < g.M) {
          if (hit) {   // one lane of a row at most, for one column tile
            g.lg.xy[row] = xys;
            g.lg.xy[g.M + row] = xyt;
          }
          if constexpr (kSwapStore && kFull)
            store_swapped(C + row * g.ldc + (colw - 4 * lgrp), aw);
          else
            store_row(full_c, C + row * g.ldc + colw, as);
        }
      }
    };
    const bool full = tc.n0 + kTile <= g.N;
    if constexpr (kTeacherEpi) {
      static_assert(kRel, "the student rows beside Precomputed teacher logits are bf16");
      if (full) rows_teacher(SlotC<1>{});
      else rows_teacher(SlotC<0>{});
    } else if (prs > 0) {
      if (full) rows_pair(SlotC<1>{});
      else rows_pair(SlotC<0>{});
    } else {
      if (full) rows(SlotC<1>{});
      else rows(SlotC<0>{});
    }
    __syncthreads();
    {
      bool teacher, ok;
      const int64_t orow = out_row(tid, teacher, ok);
      if (ok) {
        const float4 a = part[tid], b = part[256 + tid];
        const float m = fmaxf(a.x, b.x);
        float4 s;
        s.x = m;
        s.w = a.w + b.w;
        float2 cx = make_float2(0.f, 0.f);
        if (m == -INFINITY) {
          s.y = 0.f;
          s.z = 0.f;
        } else if (teacher) {
          // the KL sums of the two halves relative to the tile's maxima; the
          // student row of this pair is tile row tid - 16
          const float4 sa = part[tid - 16], sb = part[256 + tid - 16];
          const float ms = fmaxf(sa.x, sb.x);
          const float2 xa = kl_rebase(xpart[tid], sa.x, a.x, sa.z, a.z, ms, m, g.lg.inv_t);
          const float2 xb = kl_rebase(xpart[256 + tid], sb.x, b.x, sb.z, b.z, ms, m, g.lg.inv_t);
          cx = make_float2(xa.x + xb.x, xa.y + xb.y);
        }
        if (m != -INFINITY) {
          const float ea = __builtin_amdgcn_exp2f((a.x - m) * kLog2e);
          const float eb = __builtin_amdgcn_exp2f((b.x - m) * kLog2e);
          const float fa = __builtin_amdgcn_exp2f((a.x - m) * it2);
          const float fb = __builtin_amdgcn_exp2f((b.x - m) * it2);
          s.y = a.y * ea + b.y * eb;
          s.z = a.z * fa + b.z * fb;
        }
        g.lg.stats[orow * g.lg.stats_ld + tc.ntile] = s;
        if constexpr (kRel) {   // the two halves' maxima, beside the other block's
          const int64_t hrow = prs > 0 ? (teacher ? orow - prs : orow) : tc.m0 + tid;
          const int side = prs > 0 ? (teacher ? 1 : 0) : tc.p;
          float* hp = g.lg.hmax + hrow * g.lg.hmax_ld + 4 * tc.ntile + side;
          hp[0] = a.x;
          hp[2] = b.x;
        }
        if (teacher) g.lg.cross[(orow - prs) * g.lg.stats_ld + tc.ntile] = cx;
        if constexpr (kTeacherEpi) {
          // the teacher row beside this student row: its tile statistics,
          // and the two KL sums relative to the two rows' tile maxima
          const float4 ta = partT[tid], tb = partT[256 + tid];
          const float mtt = fmaxf(ta.x, tb.x);
          float4 st;
          st.x = mtt;
          st.w = ta.w + tb.w;
          float2 kx = make_float2(0.f, 0.f);
          if (mtt == -INFINITY) {
            st.y = 0.f;
            st.z = 0.f;
          } else {
            st.y = ta.y * __builtin_amdgcn_exp2f((ta.x - mtt) * kLog2e) +
                   tb.y * __builtin_amdgcn_exp2f((tb.x - mtt) * kLog2e);
            st.z = ta.z * __builtin_amdgcn_exp2f((ta.x - mtt) * it2) +
                   tb.z * __builtin_amdgcn_exp2f((tb.x - mtt) * it2);
            const float2 xa = kl_rebase(xpart[tid], a.x, ta.x, a.z, ta.z, m, mtt, g.lg.inv_t);
            const float2 xb = kl_rebase(xpart[256 + tid], b.x, tb.x, b.z, tb.z, m, mtt, g.lg.inv_t);
            kx = make_float2(xa.x + xb.x, xa.y + xb.y);
          }
          const int64_t r = orow - static_cast<int64_t>(tc.p) * g.M;
          g.lg.stats[(g.M + r) * g.lg.stats_ld + tc.ntile] = st;
          g.lg.cross[r * g.lg.stats_ld + tc.ntile] = kx;
        }
      }
    }
  }
}


// One named entry point per variant, so that profiles and the build's ISA
// check can tell them apart: gemm_<A layout><B layout>[t]_<epilogue>_<input>
// [_<logits type>], layout k = K-major, m = N-major, t = C stored
// transposed. The loss uses exactly these products: the logits (kk), the
// hidden-row gradients (km), grad_W computed transposed (kmt), and the fp32
// logits of small problems stored plainly so that K can be split (kk_store).
#define ORDA_GEMM(NAME, T, AK, BK, EPI, LT, CT) \
  __global__ __launch_bounds__(kThreads, 1) void NAME(GemmArgs g) { gemm_body<T, AK, BK, EPI, LT, CT>(g); }
ORDA_GEMM(gemm_kk_logits_bf16_bf16, __bf16, true, true, GemmEpilogue::Logits, __bf16, false)
ORDA_GEMM(gemm_kk_logits_pre_bf16_bf16, __bf16, true, true, GemmEpilogue::LogitsTeacher, __bf16, false)
ORDA_GEMM(gemm_kk_logits_pre16_bf16_bf16, __bf16, true, true, GemmEpilogue::LogitsTeacher16, __bf16, false)
ORDA_GEMM(gemm_kk_logits_bf16_f32, __bf16, true, true, GemmEpilogue::Logits, float, false)
ORDA_GEMM(gemm_km_store_bf16, __bf16, true, false, GemmEpilogue::StoreF32, float, false)
ORDA_GEMM(gemm_km_accum_bf16, __bf16, true, false, GemmEpilogue::AccumF32, float, false)
ORDA_GEMM(gemm_kmt_store_bf16, __bf16, true, false, GemmEpilogue::StoreF32, float, true)
ORDA_GEMM(gemm_kmt_accum_bf16, __bf16, true, false, GemmEpilogue::AccumF32, float, true)
ORDA_GEMM(gemm_kk_logits_f32_bf16, float, true, true, GemmEpilogue::Logits, __bf16, false)
ORDA_GEMM(gemm_kk_logits_f32_f32, float, true, true, GemmEpilogue::Logits, float, false)
ORDA_GEMM(gemm_km_store_f32, float, true, false, GemmEpilogue::StoreF32, float, false)
ORDA_GEMM(gemm_km_accum_f32, float, true, false, GemmEpilogue::AccumF32, float, false)
ORDA_GEMM(gemm_kmt_store_f32, float, true, false, GemmEpilogue::StoreF32, float, true)
ORDA_GEMM(gemm_kmt_accum_f32, float, true, false, GemmEpilogue::AccumF32, float, true)
// fp32 logits of small problems, stored plainly and split over K (the row
// statistics then come from a separate pass over the stored logits).
ORDA_GEMM(gemm_kk_store_f32, float, true, true, GemmEpilogue::StoreF32, float, false)
#undef ORDA_GEMM

typedef void (*GemmKernel)(GemmArgs);

GemmKernel select_kernel(const GemmArgs& g) {
  using E = GemmEpilogue;
  const bool bf = g.in_type == DType::BF16;
  if (g.epi == E::Logits) {
    if (!g.a_kmajor || !g.b_kmajor || g.c_trans) return nullptr;
    if (g.lg.teacher_logits != nullptr) {
      if (!bf || g.logits_type != DType::BF16) return nullptr;
      return g.lg.teacher_type == DType::BF16 ? gemm_kk_logits_pre16_bf16_bf16 : gemm_kk_logits_pre_bf16_bf16;
    }
    if (g.logits_type == DType::BF16) return bf ? gemm_kk_logits_bf16_bf16 : gemm_kk_logits_f32_bf16;
    return bf ? gemm_kk_logits_bf16_f32 : gemm_kk_logits_f32_f32;
  }
  const bool st = g.epi == E::StoreF32;
  if (g.a_kmajor && g.b_kmajor && st && !g.c_trans && !bf) return gemm_kk_store_f32;
  if (!g.a_kmajor || g.b_kmajor) return nullptr;
  if (g.c_trans)
    return bf ? (st ? gemm_kmt_store_bf16 : gemm_kmt_accum_bf16) : (st ? gemm_kmt_store_f32 : gemm_kmt_accum_f32);
  return bf ? (st ? gemm_km_store_bf16 : gemm_km_accum_bf16) : (st ? gemm_km_store_f32 : gemm_km_accum_f32);
}

// Split-K reduction: C = alpha * (Σ_s partial_s) (+ alpha * C when
// accumulating), the partials summed in split order. The partials are laid
// out like C (rows x cols, row pitch ldp, a multiple of 4; transposed
// products store them transposed), so each thread sums 4 consecutive
// columns of one row with 16-byte loads, and stores them with one 16-byte
// store where C's pitch and base allow. The split loop is unrolled so that
// its loads are in flight together; the additions stay in split order.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(
    const float* ws, int64_t stride, int splits, int64_t rows, int64_t cols, int64_t ldp,
    float* c0, float* c1, int64_t ldc, float alpha0, const float* alpha_ptr, bool accum) {
  const float alpha = alpha_ptr != nullptr ? alpha0 * *alpha_ptr : alpha0;
  const int64_t quads = (cols + 3) / 4;
  const int64_t per = rows * quads;
  const int64_t total = per * (c1 ? 2 : 1);
  const bool vec = (ldc % 4) == 0 && (reinterpret_cast<uintptr_t>(c0) % 16) == 0 &&
                   (c1 == nullptr || (reinterpret_cast<uintptr_t>(c1) % 16) == 0);
  for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int p = i >= per ? 1 : 0;
    const int64_t e = i - p * per;
    const int64_t r = e / quads;
    const int64_t q = (e - r * quads) * 4;
    const f32x4* src = reinterpret_cast<const f32x4*>(ws + p * rows * ldp + r * ldp + q);
    const int64_t sq = stride / 4;
    f32x4 v = src[0];
#pragma unroll 8
    for (int s = 1; s < splits; ++s) v += src[s * sq];
    float* dst = (p ? c1 : c0) + r * ldc + q;
    if (vec && q + 4 <= cols) {
      f32x4* d4 = reinterpret_cast<f32x4*>(dst);
      *d4 = accum ? alpha * (*d4 + v) : alpha * v;
    } else {
      for (int k = 0; k < 4 && q + k < cols; ++k) dst[k] = accum ? alpha * (dst[k] + v[k]) : alpha * v[k];
    }
  }
}

// Transposed staging (launch_transpose_rows): a 64 x 64 block of source
// rows r and columns c goes through LDS, read as 16-byte row segments when
// VEC (pitches multiples of 8 elements, bases 16-byte aligned, cols % 8 == 0)
// and written as 16-byte segments of 8 consecutive r of one column.
// Element type E is 2 or 4 bytes wide. Rows krows .. round8(krows) - 1 of
// every column are written as zeros (ldd >= round8(krows) as ldd % 8 == 0).
template <typename E, bool VEC>
__global__ __launch_bounds__(256) void transpose_rows_kernel(const E* a, int64_t lda, const E* b,
                                                             int64_t ldb, int64_t rows,
                                                             int64_t cols, E* dst, int64_t ldd) {
  constexpr int kT = 64;
  __shared__ E tile[kT][kT + 16 / sizeof(E)];
  const int64_t krows = b != nullptr ? 2 * rows : rows;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kT;
  const int64_t c0 = static_cast<int64_t>(blockIdx.y) * kT;
  constexpr int kVec = 16 / sizeof(E);   // elements per 16 bytes
  constexpr int kPerRow = kT / kVec;     // 16-byte segments per tile row
  const int tid = threadIdx.x;
  // Load: rows r0.., columns c0.. of the stacked [a; b] rows.
  for (int q = tid; q < kT * kPerRow; q += 256) {
    const int rl = q / kPerRow, seg = q % kPerRow;
    const int64_t r = r0 + rl, c = c0 + seg * kVec;
    const E* src = nullptr;
    if (r < krows) src = r < rows ? a + r * lda : b + (r - rows) * ldb;
    if constexpr (VEC) {
      typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
      u32x4v w = {0u, 0u, 0u, 0u};
      if (src != nullptr && c < cols) w = *reinterpret_cast<const u32x4v*>(src + c);
      const E* e = reinterpret_cast<const E*>(&w);
#pragma unroll
      for (int k = 0; k < kVec; ++k) tile[rl][seg * kVec + k] = e[k];
    } else {
#pragma unroll
      for (int k = 0; k < kVec; ++k)
        tile[rl][seg * kVec + k] = (src != nullptr && c + k < cols) ? src[c + k] : E(0);
    }
  }
  __syncthreads();
  // Store: column c0 + cl, rows r0 + 8s .. +7 as one 16-byte (2-byte E) or
  // two 16-byte (4-byte E) segments. The segment holding the last row is
  // written whole, with zeros past it: a GEMM reading this as a K-major
  // operand loads the 16-byte chunk that holds its last K element whole,
  // and the other operand is zero there, so the padding must be finite.
  constexpr int kSeg = 8;
  for (int q = tid; q < kT * (kT / kSeg); q += 256) {
    const int cl = q / (kT / kSeg), s = q % (kT / kSeg);
    const int64_t c = c0 + cl, r = r0 + s * kSeg;
    if (c >= cols || r >= krows) continue;
    E* d = dst + c * ldd + r;
    if ((reinterpret_cast<uintptr_t>(d) % 16) == 0) {
      alignas(16) E v[kSeg];
#pragma unroll
      for (int k = 0; k < kSeg; ++k) v[k] = tile[s * kSeg + k][cl];
      typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
#pragma unroll
      for (int h = 0; h < kSeg * static_cast<int>(sizeof(E)) / 16; ++h)
        reinterpret_cast<u32x4v*>(d)[h] = reinterpret_cast<const u32x4v*>(v)[h];
    } else {
      for (int k = 0; k < kSeg; ++k) d[k] = tile[s * kSeg + k][cl];
    }
  }
}

struct SplitPlan {
  int splits;
  int64_t len, ldp, stride, bytes;
};

// Split K when the tiles cannot fill the CUs: about 256 workgroups in all,
// each split at least 128 elements of K (a multiple of 64), at most 64
// splits and 256 MB of partials. (At BT=256, H=512, V=8192 fp32 a 512
// minimum left grad_hidden on 64 workgroups and grad_W unsplit: 0.152 and
// 0.141 ms against 0.072 and 0.070 ms with 128, reductions included; 64
// measured the same as 128.)
// Shared-round blocks (map_tile) for a product with share_rounds set: xn in
// {1, 2, 4, 8} dividing the N-tiles, b = Nt/xn, a = 32/b; the most tiles per
// XCD (at least 24), then the fewest operand strips per stage (a + b), then
// the larger a (8 x 4 measured faster than 4 x 8 at Nt = 16). The band must
// fit in the M-tiles at least once.
void set_share_blocks(GemmArgs& g) {
  g.sh_a = g.sh_b = g.sh_xn = 0;
  if (!g.share_rounds) return;
  const int64_t Nt = (g.N + kTile - 1) / kTile;
  const int64_t Mv = ((g.M + kTile - 1) / kTile) * g.nprob;
  int64_t best_a = 0, best_b = 0, best_xn = 0;
  for (int64_t xn = 1; xn <= 8; xn *= 2) {
    if (Nt % xn != 0) continue;
    const int64_t b = Nt / xn, a = 32 / b;
    if (a < 1 || a * b < 24 || a * (8 / xn) > Mv) continue;
    const bool better = best_a == 0 || a * b > best_a * best_b ||
                        (a * b == best_a * best_b &&
                         (a + b < best_a + best_b || (a + b == best_a + best_b && a > best_a)));
    if (better) {
      best_a = a;
      best_b = b;
      best_xn = xn;
    }
  }
  g.sh_a = static_cast<int>(best_a);
  g.sh_b = static_cast<int>(best_b);
  g.sh_xn = static_cast<int>(best_xn);
}

// M bands for a bf16 logits GEMM whose live rows overflow the MALL. The
// grouped raster gives each XCD its own group_m M-tiles and walks all N with
// every XCD on the same N-tiles, so 8 groups of A's rows (M x K) are live at
// once; past ~192 MB (at K = 8192, 64 M-tiles: 256 MB, the MALL's size) A's
// strips come from HBM again on every round. Then, while a band of 32
// M-tiles fits in 128 MB, the rows are walked in such bands (map_tile's
// block path with b = all N-tiles, xn = 1): each XCD takes 4 of the band's
// M-tiles and all N, 4 M x 8 N tiles a round (the same 12 strips per stage
// as the grouped raster), and B (the weight rows) is read once per band.
// Measured at BT = 8192, V = 128256, H = 8192 (two alternating passes on
// each of two machines): the logits GEMM at 0.545-0.557 of peak against
// 0.49-0.52, the call 73.6-74.7 against 75.0-77.9 ms.
// Not applied where it did not gain: H = 16384 (a 256 MB band, or 128 MB in
// 2 x 16 blocks with 18 strips a stage: 0.50 against 0.51), H = 5120 (A
// 168 MB: 0.51 against 0.52), BT = 16384 at H = 4096 (the grouped raster
// already walks N twice with 128 MB live: equal).
void set_band_blocks(GemmArgs& g) {
  constexpr int64_t kBandLive = int64_t{192} << 20, kBandMax = int64_t{128} << 20;
  if (g.sh_a > 0 || g.epi != GemmEpilogue::Logits || g.in_type != DType::BF16) return;
  const int64_t Mv = ((g.M + kTile - 1) / kTile) * g.nprob;
  const int64_t Nt = (g.N + kTile - 1) / kTile;
  const int64_t strip = int64_t{kTile} * g.K * 2;
  const int64_t gm = g.group_m > 0 ? g.group_m : 1;
  const int64_t live = (Mv < 8 * gm ? Mv : 8 * gm) * strip;
  if (live <= kBandLive || 32 * strip > kBandMax || Mv < 32) return;
  g.sh_a = 4;
  g.sh_b = static_cast<int>(Nt);
  g.sh_xn = 1;
}

SplitPlan plan_split(const GemmArgs& g) {
  SplitPlan sp{1, g.K, 0, 0, 0};
  if (g.epi == GemmEpilogue::Logits || g.M <= 0 || g.N <= 0 || g.K <= 0) return sp;
  const int64_t tiles = ((g.M + kTile - 1) / kTile) * ((g.N + kTile - 1) / kTile) * g.nprob;
  if (tiles >= 192) return sp;
  int64_t s = (256 + tiles - 1) / tiles;
  const int64_t by_k = g.K / 128;
  if (s > by_k) s = by_k;
  if (s > 64) s = 64;
  const int64_t per_split = g.nprob * (g.c_trans ? g.N * ((g.M + 3) / 4 * 4) : g.M * ((g.N + 3) / 4 * 4)) * 4;
  if (s > (int64_t{256} << 20) / per_split) s = (int64_t{256} << 20) / per_split;
  if (s <= 1) return sp;
  const int64_t len = ((g.K + s - 1) / s + 63) / 64 * 64;
  s = (g.K + len - 1) / len;
  if (s <= 1) return sp;
  sp.splits = static_cast<int>(s);
  sp.len = len;
  // partials in C's orientation: rows x ldp, transposed when C is
  sp.ldp = ((g.c_trans ? g.M : g.N) + 3) / 4 * 4;
  sp.stride = g.nprob * (g.c_trans ? g.N : g.M) * sp.ldp;
  sp.bytes = s * sp.stride * 4;
  return sp;
}

// ------------------------------------------------------- small fp32 products
// fp32 Store/Accum products with at most 64 tiles of 256 x 256 (a quarter of
// the CUs) run on 128 x 128 workgroup tiles instead: four times the
// workgroups, so that K is split less finely or not at all. With 256-wide
// tiles such a product splits K into slices of 128 (at BT=256, H=512,
// V=8192: the logits into 4, grad_hidden into 64, grad_W into 4), and each
// workgroup then spends about as long on its 256 KB of partials and on
// filling its operand ring as on its 16.8 MFLOP. A kernel of its own: 4
// waves of 64 x 64 (4 x 4 fragments of v_mfma_f32_16x16x4_f32), operands
// read from global memory into registers one K stage (32) ahead and stored
// to LDS transposed ([k][row], so that the 16 lanes of a fragment read 16
// consecutive floats), two LDS stages (72 KB). A stage's fragments are all
// read from LDS before its MFMAs (64 registers), so that only the first read
// of a stage waits; left to the scheduler, every 4 K rows waited for their
// reads between MFMAs.
constexpr int kSmTile = 128;
constexpr int kSmK = 32;
constexpr int kSmPer = kSmTile * kSmK / 256;   // floats of each operand per thread and stage
constexpr int kSmPitch = kSmTile + 16;   // floats per LDS K row: the 4 K rows of a read in 4 bank groups

int64_t small_tiles(const GemmArgs& g) {
  return ((g.M + kSmTile - 1) / kSmTile) * ((g.N + kSmTile - 1) / kSmTile) * g.nprob;
}

// Whether launch_gemm runs g (a whole product, not a part of a tail split)
// on the small kernel.
bool small_f32(const GemmArgs& g) {
  if (g.in_type != DType::F32 || !g.a_kmajor || g.split_k > 1 || g.M <= 0 || g.N <= 0) return false;
  if (g.epi != GemmEpilogue::StoreF32 && g.epi != GemmEpilogue::AccumF32) return false;
  if (g.b_kmajor && (g.c_trans || g.epi == GemmEpilogue::AccumF32)) return false;
  const int64_t tiles = ((g.M + kTile - 1) / kTile) * ((g.N + kTile - 1) / kTile) * g.nprob;
  return tiles <= 64;
}

// The small kernel's split of K: as plan_split, over its 128 x 128 tiles,
// each split at least 256 elements of K.
SplitPlan plan_split_small(const GemmArgs& g) {
  SplitPlan sp{1, g.K, 0, 0, 0};
  if (g.K <= 0) return sp;
  const int64_t tiles = small_tiles(g);
  if (tiles >= 192) return sp;
  int64_t s = (256 + tiles - 1) / tiles;
  const int64_t by_k = g.K / 256;
  if (s > by_k) s = by_k;
  if (s > 64) s = 64;
  const int64_t per_split = g.nprob * (g.c_trans ? g.N * ((g.M + 3) / 4 * 4) : g.M * ((g.N + 3) / 4 * 4)) * 4;
  if (s > (int64_t{256} << 20) / per_split) s = (int64_t{256} << 20) / per_split;
  if (s <= 1) return sp;
  const int64_t len = ((g.K + s - 1) / s + 63) / 64 * 64;
  s = (g.K + len - 1) / len;
  if (s <= 1) return sp;
  sp.splits = static_cast<int>(s);
  sp.len = len;
  sp.ldp = ((g.c_trans ? g.M : g.N) + 3) / 4 * 4;
  sp.stride = g.nprob * (g.c_trans ? g.N : g.M) * sp.ldp;
  sp.bytes = s * sp.stride * 4;
  return sp;
}

// A is K-major ([M][K], lda); B is K-major ([N][K], BK) or N-major ([K][N]);
// C is [M][ldc], or stored transposed ([N][ldc], CT); ACC adds C's old value
// before the scale, as the big kernel's AccumF32 does. Workgroup w < tiles
// * split_k: split w / tiles over K range [s * split_len, +split_len),
// partials at C + s * split_stride.
template <bool BK, bool CT, bool ACC>
__device__ __forceinline__ void small_body(const GemmArgs& g) {
  __shared__ __attribute__((aligned(16))) float sA[2][kSmK][kSmPitch];
  __shared__ __attribute__((aligned(16))) float sB[2][kSmK][kSmPitch];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t mt = (g.M + kSmTile - 1) / kSmTile, nt = (g.N + kSmTile - 1) / kSmTile;
  const int64_t per = mt * nt;
  int64_t lin = blockIdx.x;
  int64_t kbeg = 0, kend = g.K;
  int split = 0;
  if (g.split_k > 1) {
    split = static_cast<int>(lin / (per * g.nprob));
    lin -= static_cast<int64_t>(split) * per * g.nprob;
    kbeg = static_cast<int64_t>(split) * g.split_len;
    kend = g.K - kbeg < g.split_len ? g.K : kbeg + g.split_len;
  }
  const int p = static_cast<int>(lin / per);
  lin -= static_cast<int64_t>(p) * per;
  const int64_t m0 = (lin % mt) * kSmTile, n0 = (lin / mt) * kSmTile;
  const float* A = static_cast<const float*>(g.prob[p].a);
  const float* B = static_cast<const float*>(g.prob[p].b);
  float* C = static_cast<float*>(g.prob[p].c) + static_cast<int64_t>(split) * g.split_stride;
  const bool avec = (reinterpret_cast<uintptr_t>(A) % 16) == 0 && (g.lda % 4) == 0;
  const bool bvec = (reinterpret_cast<uintptr_t>(B) % 16) == 0 && (g.ldb % 4) == 0;

  // Global loads of one stage: kSmPer consecutive floats of each operand
  // per thread.
  //   K-major operand: tile row tid % 128, K columns kSmPer * (tid / 128) + i;
  //   N-major B: K row tid / kBRow, columns kSmPer * (tid % kBRow) + i, with
  //   kBRow = 128 / kSmPer threads per K row.
  constexpr int kBRow = kSmTile / kSmPer;
  static_assert(2 * kSmPer == kSmK && 256 / kBRow == kSmK, "a stage is 256 threads x kSmPer floats");
  const int kr = tid & 127, kq = (tid >> 7) * kSmPer;
  const int br = tid / kBRow, bq = (tid % kBRow) * kSmPer;
  float ra[kSmPer], rb[kSmPer];
  auto load_run = [&](const float* src, bool whole, int64_t avail, float (&r)[kSmPer]) {
    if (whole) {
#pragma unroll
      for (int v = 0; v < kSmPer / 4; ++v) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(src + 4 * v);
#pragma unroll
        for (int i = 0; i < 4; ++i) r[4 * v + i] = x[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < kSmPer; ++i) r[i] = i < avail ? src[i] : 0.f;
    }
  };
  // A run outside the operand (avail <= 0) loads nothing; its address is
  // formed but never read (clamping it to row 0 made the kernels 10 %
  // slower).
  auto load_kmajor = [&](const float* X, int64_t ld, int64_t rows, int64_t r0, bool vec, int64_t k0,
                         float (&r)[kSmPer]) {
    const int64_t row = r0 + kr, k = k0 + kq;
    const int64_t avail = row < rows ? kend - k : 0;   // elements of the run inside K
    load_run(X + row * ld + k, vec && avail >= kSmPer, avail, r);
  };
  auto load_nmajor = [&](int64_t k0, float (&r)[kSmPer]) {
    const int64_t k = k0 + br, n = n0 + bq;
    const int64_t avail = k < kend ? g.N - n : 0;
    load_run(B + k * g.ldb + n, bvec && avail >= kSmPer, avail, r);
  };
  auto load = [&](int64_t k0) {
    load_kmajor(A, g.lda, g.M, m0, avec, k0, ra);
    if constexpr (BK) load_kmajor(B, g.ldb, g.N, n0, bvec, k0, rb);
    else load_nmajor(k0, rb);
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < kSmPer; ++i) sA[buf][kq + i][kr] = ra[i];
    if constexpr (BK) {
#pragma unroll
      for (int i = 0; i < kSmPer; ++i) sB[buf][kq + i][kr] = rb[i];
    } else {
#pragma unroll
      for (int v = 0; v < kSmPer / 4; ++v) {
        f32x4 x;
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = rb[4 * v + i];
        *reinterpret_cast<f32x4*>(&sB[buf][br][bq + 4 * v]) = x;
      }
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // MFMA ks of a stage takes K row 4 * ks + lane / 16 of the stage: lane
  // (m, q) = (lane % 16, lane / 16) gives A[row m][k] and B[k][column m].
  const int lm = lane & 15, lq = lane >> 4;
  const int64_t nst = kend > kbeg ? (kend - kbeg + kSmK - 1) / kSmK : 0;
  auto compute = [&](int buf) {
    float fa[kSmK / 4][4], fb[kSmK / 4][4];
#pragma unroll
    for (int ks = 0; ks < kSmK / 4; ++ks) {
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        fa[ks][f] = sA[buf][4 * ks + lq][wm * 64 + f * 16 + lm];
        fb[ks][f] = sB[buf][4 * ks + lq][wn * 64 + f * 16 + lm];
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks < kSmK / 4; ++ks)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[ks][i], fb[ks][j], acc[i][j], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  };
  if (nst > 0) {
    load(kbeg);
    store(0);
  }
  __syncthreads();
  for (int64_t st = 0; st < nst; ++st) {
    const int buf = static_cast<int>(st & 1);
    if (st + 1 < nst) load(kbeg + (st + 1) * kSmK);
    compute(buf);
    if (st + 1 < nst) store(buf ^ 1);
    __syncthreads();
  }

  // acc[i][j][e] is row wm*64 + 16i + 4*lq + e, column wn*64 + 16j + lm.
  const float alpha = g.alpha_ptr != nullptr ? g.alpha * *g.alpha_ptr : g.alpha;
  const int64_t row_w = m0 + wm * 64 + 4 * lq;
  const int64_t col_l = n0 + wn * 64 + lm;
  if constexpr (CT) {
    const bool vec = (g.ldc % 4) == 0 && (reinterpret_cast<uintptr_t>(C) % 16) == 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t n = col_l + j * 16;
      if (n >= g.N) continue;
      float* cn = C + n * g.ldc;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t m = row_w + i * 16;
        f32x4 v = acc[i][j];
        if (vec && m + 4 <= g.M) {
          f32x4* dst = reinterpret_cast<f32x4*>(cn + m);
          if constexpr (ACC) v = alpha * (*dst + v);
          else v = alpha * v;
          *dst = v;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (m + e < g.M) {
              float x = v[e];
              if constexpr (ACC) x = alpha * (cn[m + e] + x);
              else x = alpha * x;
              cn[m + e] = x;
            }
          }
        }
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t row = row_w + i * 16 + e;
        if (row >= g.M) continue;
        float* crow = C + row * g.ldc;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t col = col_l + j * 16;
          if (col < g.N) {
            float v = acc[i][j][e];
            if constexpr (ACC) v = alpha * (crow[col] + v);
            else v = alpha * v;
            crow[col] = v;
          }
        }
      }
    }
  }
}

// One named entry point per variant, as for the 256-wide kernels:
// gemm_<A layout><B layout>[t]_small[_accum]_f32.
#define ORDA_SMALL(NAME, BK, CT, ACC) \
  __global__ __launch_bounds__(256) void NAME(GemmArgs g) { small_body<BK, CT, ACC>(g); }
ORDA_SMALL(gemm_kk_small_f32, true, false, false)
ORDA_SMALL(gemm_km_small_f32, false, false, false)
ORDA_SMALL(gemm_km_small_accum_f32, false, false, true)
ORDA_SMALL(gemm_kmt_small_f32, false, true, false)
ORDA_SMALL(gemm_kmt_small_accum_f32, false, true, true)
#undef ORDA_SMALL

// g with small_f32(g): split K over the small tiles where plan_split_small
// splits and the workspace suffices (partials with alpha 1, then the ordered
// reduction applying g's epilogue), else one launch.
hipError_t launch_small(const GemmArgs& g, hipStream_t stream) {
  using K = void (*)(GemmArgs);
  auto pick = [](bool bk, bool ct, bool acc) -> K {
    if (bk) return acc ? nullptr : gemm_kk_small_f32;
    if (ct) return acc ? gemm_kmt_small_accum_f32 : gemm_kmt_small_f32;
    return acc ? gemm_km_small_accum_f32 : gemm_km_small_f32;
  };
  const int64_t tiles = small_tiles(g);
  const SplitPlan sp = plan_split_small(g);
  if (sp.splits > 1 && g.split_ws != nullptr && g.split_ws_bytes >= sp.bytes) {
    GemmArgs s = g;
    s.epi = GemmEpilogue::StoreF32;
    s.alpha = 1.f;
    s.alpha_ptr = nullptr;
    s.ldc = sp.ldp;
    s.split_k = sp.splits;
    s.split_len = sp.len;
    s.split_stride = sp.stride;
    const int64_t rows = g.c_trans ? g.N : g.M, cols = g.c_trans ? g.M : g.N;
    for (int p = 0; p < g.nprob; ++p) s.prob[p].c = g.split_ws + p * rows * sp.ldp;
    const K k = pick(g.b_kmajor, g.c_trans, false);
    if (k == nullptr) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(tiles * sp.splits)), dim3(256), 0, stream, s);
    if (g.partials_only) return hipGetLastError();
    const int64_t total = rows * ((cols + 3) / 4) * g.nprob;
    const unsigned blocks = static_cast<unsigned>((total + 255) / 256 < 8192 ? (total + 255) / 256 : 8192);
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(256), 0, stream, g.split_ws,
                       sp.stride, sp.splits, rows, cols, sp.ldp, static_cast<float*>(g.prob[0].c),
                       g.nprob > 1 ? static_cast<float*>(g.prob[1].c) : nullptr, g.ldc, g.alpha,
                       g.alpha_ptr, g.epi == GemmEpilogue::AccumF32);
    return hipGetLastError();
  }
  if (g.partials_only) return hipErrorInvalidValue;   // not split
  GemmArgs one = g;
  one.split_k = 1;
  const K k = pick(g.b_kmajor, g.c_trans, g.epi == GemmEpilogue::AccumF32);
  if (k == nullptr) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(tiles)), dim3(256), 0, stream, one);
  return hipGetLastError();
}

}  // namespace

int64_t gemm_stat_tiles(int64_t n) { return (n + kTile - 1) / kTile; }

hipError_t launch_transpose_rows(const void* a, int64_t lda, const void* b, int64_t ldb,
                                 int64_t rows, int64_t cols, void* dst, int64_t ldd, DType t,
                                 hipStream_t stream) {
  const int64_t krows = b != nullptr ? 2 * rows : rows;
  if (rows < 0 || cols < 0 || ldd < krows || (ldd % 8) != 0) return hipErrorInvalidValue;
  if (rows == 0 || cols == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((krows + 63) / 64), static_cast<unsigned>((cols + 63) / 64));
  const bool vec = (lda % 8) == 0 && (b == nullptr || (ldb % 8) == 0) && (cols % 8) == 0 &&
                   (reinterpret_cast<uintptr_t>(a) % 16) == 0 &&
                   (reinterpret_cast<uintptr_t>(b) % 16) == 0;
  if (t == DType::BF16) {
    const auto* pa = static_cast<const uint16_t*>(a);
    const auto* pb = static_cast<const uint16_t*>(b);
    auto* pd = static_cast<uint16_t*>(dst);
    if (vec)
      hipLaunchKernelGGL((transpose_rows_kernel<uint16_t, true>), grid, dim3(256), 0, stream, pa,
                         lda, pb, ldb, rows, cols, pd, ldd);
    else
      hipLaunchKernelGGL((transpose_rows_kernel<uint16_t, false>), grid, dim3(256), 0, stream, pa,
                         lda, pb, ldb, rows, cols, pd, ldd);
  } else {
    const auto* pa = static_cast<const uint32_t*>(a);
    const auto* pb = static_cast<const uint32_t*>(b);
    auto* pd = static_cast<uint32_t*>(dst);
    if (vec)
      hipLaunchKernelGGL((transpose_rows_kernel<uint32_t, true>), grid, dim3(256), 0, stream, pa,
                         lda, pb, ldb, rows, cols, pd, ldd);
    else
      hipLaunchKernelGGL((transpose_rows_kernel<uint32_t, false>), grid, dim3(256), 0, stream, pa,
                         lda, pb, ldb, rows, cols, pd, ldd);
  }
  return hipGetLastError();
}

namespace {

// The part of g over columns [c0, c1) and rows [r0, r1) of C (operands and
// C advanced to them).
GemmArgs sub_product(const GemmArgs& g, int64_t r0, int64_t r1, int64_t c0, int64_t c1) {
  GemmArgs t = g;
  t.M = r1 - r0;
  t.N = c1 - c0;
  const int64_t es = g.in_type == DType::BF16 ? 2 : 4;
  for (int p = 0; p < g.nprob; ++p) {
    t.prob[p].a = static_cast<const unsigned char*>(g.prob[p].a) + (g.a_kmajor ? r0 * g.lda : r0) * es;
    t.prob[p].b = static_cast<const unsigned char*>(g.prob[p].b) + (g.b_kmajor ? c0 * g.ldb : c0) * es;
    t.prob[p].c = static_cast<float*>(g.prob[p].c) +
                  (g.c_trans ? c0 * g.ldc + r0 : r0 * g.ldc + c0);
  }
  return t;
}

// Whole rounds and a tail. A Store/Accum product whose tiles leave a last
// round of fewer than 192 workgroups (for 256 CUs) runs its whole rounds as
// one launch and the rest as a second product, which then splits K over the
// CUs (plan_split): the tail costs a fraction of a round instead of a whole
// one. The whole rounds must end on a tile boundary: in the columns (256 x
// rounds divisible by the M-tiles, e.g. grad_W computed transposed with its
// 16 M-tiles at H = 4096), else in the rows of every problem (by the
// N-tiles x problems, e.g. grad_hidden at H = 4096 and BT = 5000); and the
// tail must split. Returns the split point (a multiple of 256) as a column
// (cols = true) or a row, or 0 when the product runs as one launch.
struct TailSplit {
  int64_t at;
  bool cols;
};
TailSplit plan_tail(const GemmArgs& g) {
  const TailSplit none{0, false};
  if (g.epi == GemmEpilogue::Logits || g.split_k > 1 || g.M <= 0 || g.N <= 0) return none;
  const int64_t Mt = (g.M + kTile - 1) / kTile, Nt = (g.N + kTile - 1) / kTile;
  const int64_t Mv = Mt * g.nprob;
  const int64_t T = Mv * Nt, q = T / 256, r = T % 256;
  if (q < 1 || r == 0 || r >= 192) return none;
  if ((256 * q) % Mv == 0) {
    const int64_t n0 = 256 * q / Mv * kTile;
    if (n0 < g.N && plan_split(sub_product(g, 0, g.M, n0, g.N)).splits > 1) return {n0, true};
  }
  if ((256 * q) % (Nt * g.nprob) == 0) {
    const int64_t m0 = 256 * q / (Nt * g.nprob) * kTile;
    if (m0 < g.M && plan_split(sub_product(g, m0, g.M, 0, g.N)).splits > 1) return {m0, false};
  }
  return none;
}

// The two launches of a tail split: whole rounds first, then the tail.
GemmArgs tail_part(const GemmArgs& g, const TailSplit& ts, bool tail) {
  if (ts.cols) return tail ? sub_product(g, 0, g.M, ts.at, g.N) : sub_product(g, 0, g.M, 0, ts.at);
  return tail ? sub_product(g, ts.at, g.M, 0, g.N) : sub_product(g, 0, ts.at, 0, g.N);
}

}  // namespace

GemmSplit gemm_split_plan(const GemmArgs& g) {
  GemmSplit r{0, 0, 0};
  if (g.split_ws == nullptr) return r;
  const bool small = small_f32(g);
  if (!small && plan_tail(g).at > 0) return r;
  const SplitPlan sp = small ? plan_split_small(g) : plan_split(g);
  if (sp.splits > 1 && g.split_ws_bytes >= sp.bytes) r = GemmSplit{sp.splits, sp.stride, sp.ldp};
  return r;
}

int64_t gemm_split_bytes(const GemmArgs& g) {
  if (small_f32(g)) {
    const SplitPlan sp = plan_split_small(g);
    return sp.splits > 1 ? sp.bytes : 0;
  }
  const TailSplit ts = plan_tail(g);
  const SplitPlan sp = plan_split(ts.at > 0 ? tail_part(g, ts, true) : g);
  return sp.splits > 1 ? sp.bytes : 0;
}

bool gemm_small_tiles(const GemmArgs& g) { return small_f32(g); }

namespace {
hipError_t launch_gemm_impl(const GemmArgs& g, hipStream_t stream, bool whole);
}  // namespace

hipError_t launch_gemm(const GemmArgs& g, hipStream_t stream) {
  return launch_gemm_impl(g, stream, true);
}

namespace {
// whole: g is the caller's whole product (not a part of a tail split), which
// may run on the small kernel.
hipError_t launch_gemm_impl(const GemmArgs& g, hipStream_t stream, bool whole) {
  if (g.nprob < 1 || g.nprob > 2) return hipErrorInvalidValue;
  if ((g.lda % 8) || (g.ldb % 8) || (g.ldc % 8 && g.epi == GemmEpilogue::Logits))
    return hipErrorInvalidValue;
  if (g.epi == GemmEpilogue::Logits && g.lg.pair_rows > 0 &&
      (g.nprob != 1 || g.lg.cross == nullptr || g.lg.pair_teacher == nullptr ||
       g.in_type != DType::BF16 || g.M != 2 * ((g.lg.pair_rows + 15) / 16 * 16)))
    return hipErrorInvalidValue;
  if (g.epi == GemmEpilogue::Logits && g.lg.teacher_logits != nullptr &&
      (g.nprob != 1 || g.lg.pair_rows > 0 || g.lg.cross == nullptr || g.lg.teacher_ld % 4 ||
       g.lg.teacher_ld < g.N ||
       reinterpret_cast<uintptr_t>(g.lg.teacher_logits) % (g.lg.teacher_type == DType::BF16 ? 8 : 16)))
    return hipErrorInvalidValue;
  if (g.epi == GemmEpilogue::Logits && g.logits_type == DType::BF16 &&
      (g.lg.hmax == nullptr || g.lg.hmax_ld % 2 || g.lg.hmax_ld < 4 * ((g.N + kTile - 1) / kTile)))
    return hipErrorInvalidValue;
  if (g.M <= 0 || g.N <= 0) return hipSuccess;
  if (whole && small_f32(g)) return launch_small(g, stream);
  if (g.split_ws != nullptr) {
    const TailSplit ts = plan_tail(g);
    if (ts.at > 0 && g.partials_only) return hipErrorInvalidValue;
    if (ts.at > 0) {   // whole rounds, then the tail with K split
      const hipError_t e = launch_gemm_impl(tail_part(g, ts, false), stream, false);
      if (e != hipSuccess) return e;
      return launch_gemm_impl(tail_part(g, ts, true), stream, false);
    }
  }
  const int64_t tiles = ((g.M + kTile - 1) / kTile) * ((g.N + kTile - 1) / kTile) * g.nprob;
  GemmArgs gr = g;
  set_share_blocks(gr);
  set_band_blocks(gr);
  const SplitPlan sp = plan_split(g);
  if (sp.splits > 1 && g.split_ws != nullptr && g.split_ws_bytes >= sp.bytes) {
    // Partials of every split with the Store epilogue (alpha 1), in C's
    // orientation, then one reduction applying the requested epilogue.
    GemmArgs s = gr;
    s.epi = GemmEpilogue::StoreF32;
    s.alpha = 1.f;
    s.alpha_ptr = nullptr;
    s.ldc = sp.ldp;
    s.split_k = sp.splits;
    s.split_len = sp.len;
    s.split_stride = sp.stride;
    const int64_t rows = g.c_trans ? g.N : g.M, cols = g.c_trans ? g.M : g.N;
    for (int p = 0; p < g.nprob; ++p) s.prob[p].c = g.split_ws + p * rows * sp.ldp;
    const GemmKernel k = select_kernel(s);
    if (k == nullptr) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(tiles * sp.splits)), dim3(kThreads), 0,
                       stream, s);
    if (g.partials_only) return hipGetLastError();
    const int64_t total = rows * ((cols + 3) / 4) * g.nprob;
    const unsigned blocks = static_cast<unsigned>((total + 255) / 256 < 8192 ? (total + 255) / 256 : 8192);
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(256), 0, stream, g.split_ws,
                       sp.stride, sp.splits, rows, cols, sp.ldp, static_cast<float*>(g.prob[0].c),
                       g.nprob > 1 ? static_cast<float*>(g.prob[1].c) : nullptr, g.ldc, g.alpha,
                       g.alpha_ptr, g.epi == GemmEpilogue::AccumF32);
    return hipGetLastError();
  }
  if (g.partials_only) return hipErrorInvalidValue;   // not split
  GemmArgs one = gr;
  one.split_k = 1;
  const GemmKernel k = select_kernel(one);
  if (k == nullptr) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k, dim3(static_cast<unsigned>(tiles)), dim3(kThreads), 0, stream, one);
  return hipGetLastError();
}
}  // namespace

}  // namespace orda
