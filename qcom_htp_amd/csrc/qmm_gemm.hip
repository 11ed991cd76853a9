// Quantized GEMM on gfx950 i8 MFMA (v_mfma_i32_32x32x32_i8), bit-exact to the reference's
// float-derived requantisation.
//
// Workgroup: 512 threads = 8 waves (two per SIMD) side by side over a kBM x kBN = 128 x 512 tile
// of the i8 operand space (activation rows x weight-operand columns); each wave owns 4 x 2 MFMA
// 32x32 blocks (all 128 rows x 64 columns).  Two waves per SIMD let one wave's LDS reads and
// conversions run under the other's MFMAs (a lone wave stalls its MFMAs on its own LDS reads).
// The 128-row activation tile is shared by all eight waves, so each k step writes half the LDS
// bytes of a 256 x 256 tile (whose every fragment row is read by four waves either way), and
// each weight fragment is loaded by exactly one wave.  K is consumed 128 deep per pipeline step.
//
// Data movement: activation tiles go global -> LDS with direct-to-LDS loads
// (global_load_lds_dwordx4), bypassing VGPRs, gathered into a swizzled layout by the per-lane
// source addresses; both stages are in flight and one barrier per 128-k tile both publishes the
// landed tile and frees the stage read before.  Weight tiles are int8 (int4 codes and LPBQ
// code * block scale are widened at prepare time) prepared in MFMA fragment order, so each
// wave loads its weight fragments straight into registers (one coalesced 1 KiB load per
// fragment, three 32-k steps ahead) and LDS carries only the activations: per 32-k step a CU
// reads 32 KiB of fragments from LDS and its DMA writes 8 KiB (with the weights through LDS too
// it was 48 + 16 KiB, about the LDS bandwidth during the step's MFMAs).  Activations are
// converted on the MFMA fragments after the LDS read:
//   * 8-bit activations: XOR 0x80 gives the signed a - 128;
//   * 16-bit activations a - 32768 = 256*hi + lo' + 128: the hi and lo' bytes of each u16
//     become two int8 fragments, each multiplied into its own accumulator.
// Epilogue: straight from the accumulator registers.  The exact integer dot product S becomes
// t = S*alpha + beta in float64; rint(t) is certain unless t is within the per-channel margin
// of a rounding boundary, in which case the element is queued in LDS and recomputed after the
// tile by a wave-cooperative float64 dot product that forms each term as the reference oracle
// does (scripts/generate_qnn_matmul_python_cases.py:472-481).  Lanes of a quad exchange their
// 4-row strips with DPP so that every store writes 4 adjacent outputs of one row.

#include <type_traits>
#include <utility>

#include "qmm_internal.h"

namespace qh {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void *lds_void_ptr;
typedef __attribute__((address_space(1))) void *gbl_void_ptr;

// Compile-time loop: f(integral_constant<int, 0>) ... f(integral_constant<int, N-1>).
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F &&f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

struct GemmArgs {
  const uint8_t *act;
  void *out;
  const uint8_t *tiles;
  const double *alpha, *beta, *margin, *absb, *bias_deq;
  const double *alpha_e, *margin_exact;
  const double *margin_lo;  // 16-bit acts: bound of the low-byte residue sum (output LSB)
  const int32_t *scale_exp;
  const int64_t *corr, *mant, *colsum, *colsum_r;
  const float *s32;
  const int8_t *resid;  // 8-bit acts: rounding residues [N][K]
  int M, N, K, KT, TM, TN;
  int act_zp, out_zp, out_qmax, out16;
  double sA, sO;
};

constexpr int kTileA = kBM * kBK;  // A8: kBM rows x 128 B; A16: kBM / 2 rows x 256 B
constexpr int kWM = kBM / 128;     // waves along the tile's rows (each wave: 128 A8 rows x 64 operand columns)
constexpr int kNT = 2;         // 32-column MFMA blocks per wave

struct Cfg {
  static constexpr int kTileB = kBN * kBK;  // kBN operand columns x 128 k, int8
#ifndef QH_GEMM_STAGES
#define QH_GEMM_STAGES 2
#endif
  static constexpr int kStages = QH_GEMM_STAGES;  // activation tiles in LDS (the DMA runs S - 1 tiles ahead)
  static constexpr int kLoadsA = kTileA / (16 * kGemmThreads);  // 16-byte DMA loads per thread per stage
  // Weight fragments: kNT 16-byte loads per lane per 32-k step, into a ring of kBRing step slots,
  // requested kBRing - 1 steps ahead of their MFMAs.
  static constexpr int kBRing = 4;
};

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// s_waitcnt vmcnt(n) with lgkmcnt / expcnt left unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// 16 bytes per lane from global memory (base + off, base uniform) straight into LDS (lane i
// writes lds_wave_base + 16 i).  ASM: issued from inline assembly, invisible to the compiler's
// wait-count bookkeeping.  The builtin form makes the compiler treat every fragment read issued
// while such a load is in flight as needing lgkmcnt(0); the k loop accounts for its own loads
// with explicit vmcnt waits (and a barrier before a stage is rewritten), so it uses the
// assembly form, and the kernel waits for vmcnt(0) itself before the operand stages are reused
// or the waves end.
template <bool ASM>
__device__ __forceinline__ void load_lds16(const uint8_t *base, uint32_t off, void *lds_wave_base) {
  if (ASM) {
    // the LDS address goes in as an m0 operand, so the compiler sets m0 itself and knows it
    // is live (the builtin loads rely on compiler-managed m0 too)
    const uint32_t m0v = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds_wave_base)));
    asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(m0v) : "memory");
  } else {
    __builtin_amdgcn_global_load_lds((gbl_void_ptr)(const_cast<uint8_t *>(base + off)), (lds_void_ptr)(lds_wave_base), 16, 0, 0);
  }
}

__device__ __forceinline__ void store_out(void *out, int out16, size_t idx, int v) {
  if (out16)
    static_cast<uint16_t *>(out)[idx] = static_cast<uint16_t>(v);
  else
    static_cast<uint8_t *>(out)[idx] = static_cast<uint8_t>(v);
}

// 16 consecutive integer weights (k .. k+15, k % 16 == 0) of operand column cb.
__device__ __forceinline__ void load_w16(const GemmArgs g, int cb, int k, int (&w)[16]) {
  const size_t tile = static_cast<size_t>(cb / kBN) * g.KT + k / kBK;
  const uint4 v = *reinterpret_cast<const uint4 *>(g.tiles + tile * (kBN * kBK) + tile_off_i8(cb % kBN, k));
  const int8_t *b = reinterpret_cast<const int8_t *>(&v);
#pragma unroll
  for (int j = 0; j < 16; ++j) w[j] = b[j];
}

typedef unsigned int v2u __attribute__((ext_vector_type(2)));

// Buffer resource over the rows of one tile's output that lie below M.  A store at an offset
// past them is dropped by the hardware range check, so the epilogue tests no row.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t out_rsrc(void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(base, 0, static_cast<int>(bytes), 0x00020000);
}

// R * pitch for a compile-time row step R, as one scalar multiply (left to itself the compiler
// folds the uniform product into a per-lane 64-bit multiply-add).
template <int R>
__device__ __forceinline__ uint32_t row_step(uint32_t pitch) {
  if constexpr (R == 0) {
    return 0u;
  } else {
    uint32_t r;
    asm("s_mul_i32 %0, %1, %2" : "=s"(r) : "s"(pitch), "i"(R));
    return r;
  }
}

// Per-lane constants of the quad exchange in store_strip (lane q of its quad).
struct StripLane {
  uint32_t sel;  // byte (8-bit outputs) or half-word (16-bit outputs) select of row q
  bool upper;    // 16-bit outputs: the lane stores the second pair of rows' words
};
template <bool OUT16>
__device__ __forceinline__ StripLane strip_lane(int q) {
  if (!OUT16) return {static_cast<uint32_t>(q) | (static_cast<uint32_t>(4 + q) << 8) | 0x0C0C0000u, false};
  return {(q & 1) ? 0x07060302u : 0x05040100u, q >= 2};
}

// Lane q of a quad holds outputs o[0..3] of tile rows R..R+3 in its own column; the quad
// exchanges them (DPP quad broadcasts + byte permutes) so that lane q stores tile row R + q,
// tile columns col..col+3 (4 adjacent outputs in one store) at byte offset off of the tile's
// output (an offset at or past the resource's end for a row past M or a column past N).
template <bool OUT16>
__device__ __forceinline__ void store_strip(__amdgpu_buffer_rsrc_t r, uint32_t off, const int (&o)[4], const StripLane &sl) {
  if constexpr (!OUT16) {
    // outputs are clamped to [0, 255]: three byte permutes pack them (the compiler's shift / or
    // form takes four instructions)
    const uint32_t lo = perm(static_cast<uint32_t>(o[1]), static_cast<uint32_t>(o[0]), 0x0C0C0400u);
    const uint32_t hi = perm(static_cast<uint32_t>(o[3]), static_cast<uint32_t>(o[2]), 0x0C0C0400u);
    const uint32_t p = perm(hi, lo, 0x05040100u);
    const uint32_t x0 = __builtin_amdgcn_mov_dpp(p, 0x00, 0xF, 0xF, false);
    const uint32_t x1 = __builtin_amdgcn_mov_dpp(p, 0x55, 0xF, 0xF, false);
    const uint32_t x2 = __builtin_amdgcn_mov_dpp(p, 0xAA, 0xF, 0xF, false);
    const uint32_t x3 = __builtin_amdgcn_mov_dpp(p, 0xFF, 0xF, 0xF, false);
    const uint32_t w = perm(perm(x3, x2, sl.sel), perm(x1, x0, sl.sel), 0x05040100u);
    __builtin_amdgcn_raw_buffer_store_b32(w, r, static_cast<int>(off), 0, 0);
  } else {
    const uint32_t P0 = static_cast<uint32_t>(o[0]) | (static_cast<uint32_t>(o[1]) << 16);
    const uint32_t P1 = static_cast<uint32_t>(o[2]) | (static_cast<uint32_t>(o[3]) << 16);
    // every lane fetches both strips of every quad lane, then keeps the half it stores (a
    // lane-dependent choice between DPP results must come after all DPPs)
    const uint32_t a0 = __builtin_amdgcn_mov_dpp(P0, 0x00, 0xF, 0xF, false);
    const uint32_t a1 = __builtin_amdgcn_mov_dpp(P0, 0x55, 0xF, 0xF, false);
    const uint32_t a2 = __builtin_amdgcn_mov_dpp(P0, 0xAA, 0xF, 0xF, false);
    const uint32_t a3 = __builtin_amdgcn_mov_dpp(P0, 0xFF, 0xF, 0xF, false);
    const uint32_t b0 = __builtin_amdgcn_mov_dpp(P1, 0x00, 0xF, 0xF, false);
    const uint32_t b1 = __builtin_amdgcn_mov_dpp(P1, 0x55, 0xF, 0xF, false);
    const uint32_t b2 = __builtin_amdgcn_mov_dpp(P1, 0xAA, 0xF, 0xF, false);
    const uint32_t b3 = __builtin_amdgcn_mov_dpp(P1, 0xFF, 0xF, 0xF, false);
    const uint32_t lo_w = perm(a1, a0, sl.sel), hi_w = perm(a3, a2, sl.sel);
    const uint32_t lo_w2 = perm(b1, b0, sl.sel), hi_w2 = perm(b3, b2, sl.sel);
    v2u w;
    w.x = sl.upper ? lo_w2 : lo_w;
    w.y = sl.upper ? hi_w2 : hi_w;
    __builtin_amdgcn_raw_buffer_store_b64(w, r, static_cast<int>(off), 0, 0);
  }
}

// Sum over the 64 lanes of a wave: DPP adds within each row of 16 lanes (quad swaps, then the
// half-row and row mirrors), then the four row sums from lanes 0, 16, 32, 48.
__device__ __forceinline__ int wave_sum(int v) {
  v += __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);   // quad_perm [1, 0, 3, 2]
  v += __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);   // quad_perm [2, 3, 0, 1]
  v += __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, false);  // row_half_mirror
  v += __builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, false);  // row_mirror
  return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) + __builtin_amdgcn_readlane(v, 32) +
         __builtin_amdgcn_readlane(v, 48);
}

// min(max(v, 0), qmax) in one instruction: the median of (v, 0, qmax) for qmax >= 0 (the compiler
// forms v_med3_i32 only for compile-time bounds).
__device__ __forceinline__ int clamp_out(int v, int qmax) {
  int r;
  asm("v_med3_i32 %0, %1, 0, %2" : "=v"(r) : "v"(v), "s"(qmax));
  return r;
}

// rint(t) without the float64 round / convert instructions: adding 1.5 * 2^52 leaves the
// rounded integer (ties to even) in the low word, exact for |t| < 2^31.  CLAMP first limits t
// to [-1, qmax + 1] (used when |t| < 2^30 is not proven for every column); rint then lands
// on -1 or qmax + 1 for t outside, whose output is 0 or qmax whichever way t rounds.
// Returns |t - rint(t)|.
template <bool CLAMP>
__device__ __forceinline__ double round_near(double t, double qmax, int *oi) {
  constexpr double kMagic = 6755399441055744.0;  // 1.5 * 2^52
  const double tc = CLAMP ? fmin(fmax(t, -1.0), qmax + 1.0) : t;
  const double y = tc + kMagic;
  *oi = __double2loint(y);
  return fabs(tc - (y - kMagic));
}

// 16 consecutive int8 weights of operand column cb, kept packed.
__device__ __forceinline__ uint4 load_w16_raw(const GemmArgs &g, int cb, int k) {
  const size_t tile = static_cast<size_t>(cb / kBN) * g.KT + k / kBK;
  return *reinterpret_cast<const uint4 *>(g.tiles + tile * (kBN * kBK) + tile_off_i8(cb % kBN, k));
}
__device__ __forceinline__ int w_at(const uint4 &v, int j) { return reinterpret_cast<const int8_t *>(&v)[j]; }


// Exact float64 recomputation of one output, term by term as the oracle forms it:
// sum_k fl64((a_k - zp) * sA) * fl32(w_k * s32), then + bias_deq, / sO, + out_zp, rint, clip.
template <bool A16>
__device__ __forceinline__ void fixup_one(const GemmArgs &g, int m, int n, int lane) {
  const int cb = A16 ? (n / 32) * 64 + (n % 32) : n;
  const float sc = g.s32[n];
  double s = 0.0;
  // Up to 4 chunks of 16 k per lane are loaded before any is used (K <= 4096 in one round).
  constexpr int P = 4;
  for (int kc0 = 0; kc0 < g.K / 16; kc0 += 64 * P) {
    int w[P][16];
    uint4 av[P][A16 ? 2 : 1];
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const int kc = kc0 + lane + 64 * i;
      if (kc < g.K / 16) {
        const int k = kc * 16;
        load_w16(g, cb, k, w[i]);
        if (A16) {
          const uint4 *ap = reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(g.act) + static_cast<size_t>(m) * g.K + k);
          av[i][0] = ap[0];
          av[i][A16 ? 1 : 0] = ap[1];
        } else {
          av[i][0] = *reinterpret_cast<const uint4 *>(g.act + static_cast<size_t>(m) * g.K + k);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < P; ++i) {
      if (kc0 + lane + 64 * i >= g.K / 16) continue;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        int a;
        if (A16)
          a = reinterpret_cast<const uint16_t *>(&av[i][j >> 3])[j & 7];
        else
          a = reinterpret_cast<const uint8_t *>(&av[i][0])[j];
        const float wd = static_cast<float>(w[i][j]) * sc;
        const double xd = static_cast<double>(a - g.act_zp) * g.sA;
        s = fma(xd, static_cast<double>(wd), s);
      }
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
  if (lane == 0) {
    const double qr = s + g.bias_deq[n];
    const double t = qr / g.sO + static_cast<double>(g.out_zp);
    const double o = fmin(fmax(rint(t), 0.0), static_cast<double>(g.out_qmax));
    store_out(g.out, g.out16, static_cast<size_t>(m) * g.N + n, static_cast<int>(o));
  }
}

// Tile coordinates of this workgroup.  Workgroups are dispatched round-robin over the 8 XCDs
// (each with its own L2); consecutive tile indices are given to one XCD and walked in groups
// of 1024 / kBM row tiles, so an XCD's 32 concurrent tiles (8 row tiles x 4 column panels)
// share activation rows and weight columns: 8 x 0.5 + 4 x 2 MB of operands at K = 4096.
__device__ __forceinline__ void tile_of(int w, int TM, int TN, int *tm, int *tn) {
  const int T = TM * TN;
  int lin = w;
  if ((T & 7) == 0) lin = (w & 7) * (T >> 3) + (w >> 3);
  constexpr int GM = 1024 / kBM;
  const int group = GM * TN;
  const int gid = lin / group, first = gid * GM;
  const int gm = TM - first < GM ? TM - first : GM;
  const int in = lin - gid * group;
  *tm = first + in % gm;
  *tn = in / gm;
}

// ---------------------------------------------------------------- main loop pieces
// Everything the k loop needs about the workgroup's tile.
struct MainCtx {
  const uint8_t *act;     // activations [M][K] (u8) or [M][K] (u16)
  const uint8_t *bw;      // weight tiles of this column panel (one per 128-k step), at the wave's quarter
  uint32_t boff;          // this lane's byte offset inside a weight fragment (16 lane)
  int M, K, KT, m0, t, lane, wave, wm, wn;
};

// Issue the direct-to-LDS activation loads of k-tile kt into the stage wa.
template <bool A16, bool ASM>
__device__ __forceinline__ void issue_tile(const MainCtx &c, int kt, uint8_t *__restrict__ wa) {
  using C = Cfg;
  // 32-bit byte offsets from uniform bases: the tile's first activation row, the k-tile of
  // the weight panel (256 rows x K x 2 bytes < 2^32 for K < 2^23)
  const uint8_t *const abase = c.act + static_cast<size_t>(c.m0) * c.K * (A16 ? 2 : 1);
#pragma unroll
  for (int j = 0; j < C::kLoadsA; ++j) {
    const int slot = j * kGemmThreads + c.t;  // 16-byte slot of the tile
    uint32_t off;
    if (!A16) {
      const int row = slot >> 3, phys = slot & 7;
      const int logical = phys ^ swz8(row);
      const int r = c.m0 + row < c.M ? row : c.M - 1 - c.m0;
      const int k = kt * kBK + 16 * logical < c.K ? kt * kBK + 16 * logical : c.K - 16;
      off = static_cast<uint32_t>(r) * static_cast<uint32_t>(c.K) + static_cast<uint32_t>(k);
    } else {
      const int row = slot >> 4, phys = slot & 15;
      const int logical = phys ^ swz16(row);
      const int r = c.m0 + row < c.M ? row : c.M - 1 - c.m0;
      const int k = kt * kBK + 8 * logical < c.K ? kt * kBK + 8 * logical : c.K - 8;
      off = (static_cast<uint32_t>(r) * static_cast<uint32_t>(c.K) + static_cast<uint32_t>(k)) * 2u;
    }
    load_lds16<ASM>(abase, off, wa + (j * kGemmThreads + c.wave * 64) * 16);
  }
}

// The wave's weight fragments of 32-k step kk of k-tile kt (kt clamped to the last tile: past
// the end the loads re-read it, so every step issues the same loads and wait counts stay fixed):
// fragment nt of the wave's column quarter wn is the 1 KiB at 1 KiB * (8 kk + 2 wn + nt).
// Issued from assembly, like the activation DMA, so that the issue order of all of the loop's
// vector-memory requests is the program order and the loop's explicit wait counts are exact (the
// compiler's own counts would not see the DMA and would wait for requests issued later).  The
// registers receive their data only after a covering wait_b().
__device__ __forceinline__ void load_b(const MainCtx &c, int kt, int kk, v4i (&b)[kNT]) {
  const uint8_t *p = c.bw + static_cast<size_t>(min(kt, c.KT - 1)) * Cfg::kTileB + kk * (kBN / 32) * 1024;
  static_assert(kNT == 2, "two fragments per step");
  asm volatile("global_load_dwordx4 %0, %1, %2" : "=v"(b[0]) : "v"(c.boff), "s"(p));
  asm volatile("global_load_dwordx4 %0, %1, %2 offset:1024" : "=v"(b[1]) : "v"(c.boff), "s"(p));
}

// s_waitcnt vmcnt(N) that the weight fragments b pass through: the MFMAs that read them depend
// on this instruction, so they cannot move above it.
template <int N>
__device__ __forceinline__ void wait_b(v4i (&b)[kNT]) {
  static_assert(kNT == 2 && N >= 0 && N < 64, "two fragments per step");
  asm volatile("s_waitcnt vmcnt(%2)" : "+v"(b[0]), "+v"(b[1]) : "n"(N));
}

// Raw LDS words of one 32-k step: the activation fragments.
struct RawStep {
  uint4 a[4];
};

template <bool A16>
__device__ __forceinline__ void read_step(const MainCtx &c, const uint8_t *__restrict__ la, int kk, RawStep &r) {
  const int s16 = 2 * kk + (c.lane >> 5);  // 16-k chunk index inside the 128-k tile
  if (!A16) {
    static_for<4>([&](auto mt) {
      const int row = c.wm * 128 + mt * 32 + (c.lane & 31);
      r.a[mt] = *reinterpret_cast<const uint4 *>(la + row * 128 + 16 * (s16 ^ swz8(row)));
    });
  } else {
    static_for<2>([&](auto mt) {
      const int row = c.wm * 64 + mt * 32 + (c.lane & 31);
      r.a[2 * mt] = *reinterpret_cast<const uint4 *>(la + row * 256 + 16 * ((2 * s16) ^ swz16(row)));
      r.a[2 * mt + 1] = *reinterpret_cast<const uint4 *>(la + row * 256 + 16 * ((2 * s16 + 1) ^ swz16(row)));
    });
  }
}

// Raw words -> MFMA operands: activations to signed bytes (16-bit: hi / lo' byte planes).
template <bool A16>
__device__ __forceinline__ void convert_step(const RawStep &r, v4i (&af)[4]) {
  if (!A16) {
    static_for<4>([&](auto mt) {
      const uint4 v = r.a[mt];
      af[mt] = v4i{static_cast<int>(v.x ^ 0x80808080u), static_cast<int>(v.y ^ 0x80808080u),
                   static_cast<int>(v.z ^ 0x80808080u), static_cast<int>(v.w ^ 0x80808080u)};
    });
  } else {
    static_for<2>([&](auto mt) {
      uint4 v0 = r.a[2 * mt], v1 = r.a[2 * mt + 1];
      v0.x ^= 0x80808080u; v0.y ^= 0x80808080u; v0.z ^= 0x80808080u; v0.w ^= 0x80808080u;
      v1.x ^= 0x80808080u; v1.y ^= 0x80808080u; v1.z ^= 0x80808080u; v1.w ^= 0x80808080u;
      af[2 * mt] = v4i{static_cast<int>(perm(v0.y, v0.x, 0x07050301u)), static_cast<int>(perm(v0.w, v0.z, 0x07050301u)),
                       static_cast<int>(perm(v1.y, v1.x, 0x07050301u)), static_cast<int>(perm(v1.w, v1.z, 0x07050301u))};
      af[2 * mt + 1] = v4i{static_cast<int>(perm(v0.y, v0.x, 0x06040200u)), static_cast<int>(perm(v0.w, v0.z, 0x06040200u)),
                           static_cast<int>(perm(v1.y, v1.x, 0x06040200u)), static_cast<int>(perm(v1.w, v1.z, 0x06040200u))};
    });
  }
}

// The k loop is a software pipeline over 32-k steps sigma = 4 kt + kk (kt: 128-k tile, kk: its
// 32-k step): step sigma runs its MFMAs while the activations of step sigma + 1 are converted
// (VALU), the LDS fragments of step sigma + 2 are read and the weight fragments of step
// sigma + 3 are requested, so the conversions issue in the shadow of the matrix core rather
// than in bursts between MFMA groups.  Tiles: both activation stages are filled up front; in
// step 2 of tile kt each wave has read all of tile kt, waits until tile kt + 1 has landed, and
// one barrier then publishes tile kt + 1 and frees the stage of tile kt, which receives tile
// kt + 2 at once.  The first two steps of tile kt + 1 are read (and the first converted) during
// steps 2 and 3 of tile kt.
struct PipeRegs {
  RawStep raw[2];        // LDS words of the steps sigma + 1 / sigma + 2 (slot sigma & 1)
  v4i af[2][4];          // converted activations of steps sigma / sigma + 1 (slot sigma & 1)
  v4i bq[Cfg::kBRing][kNT];  // weight fragments of steps sigma .. sigma + 3 (slot sigma % 4 = kk)
};


// Workgroup barrier that waits for this wave's LDS reads (not for its loads in flight, which
// the release fence of __syncthreads would also wait for).
__device__ __forceinline__ void lds_read_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// One 128-k tile kt in stage la; the next tile is in na.  On entry af slot 0 holds the converted
// activations of step 0, raw slot 1 the LDS words of step 1, and bq slots 0..2 the weight
// fragments of steps 0..2 (requested).
//
// Memory counter: the activation DMA and the weight loads share this wave's vector-memory
// counter, which retires in issue order, and every request of the loop is issued from assembly
// in program order, so each wait count below is the exact number of requests issued after the
// one waited for.  Step kk issues, in order: [kk == 2: the DMA of tile kt + 2 (kLoadsA)] and the
// weight loads of step sigma + 3 (kNT).  Step kk needs the weights of step sigma, loaded 3 steps
// earlier, followed by the loads of two steps (2 kNT) and, for kk = 3 and 0 (the loads of kk = 0
// and 1 of the tile before), the DMA issued at step 2 in between (kLoadsA more).  At kk = 2 the
// same count also covers the DMA of tile kt + 1, issued before the weights waited for.
template <bool A16>
__device__ __forceinline__ void k_tile(const MainCtx &c, int kt, int KT, uint8_t *__restrict__ la,
                                       const uint8_t *__restrict__ na, PipeRegs &p, v16i (&acc)[4][kNT]) {
  using C = Cfg;
  constexpr int S = C::kStages;
  static_for<4>([&](auto kkc) {
    constexpr int kk = decltype(kkc)::value;
    // each step's loads stay in their step (the scheduler may not hoist or sink them across)
    __builtin_amdgcn_sched_barrier(0);
    // the weights of step sigma have landed (kk = 2: tile kt + 1's DMA too)
    wait_b<(kk == 0 || kk == 3) ? 2 * kNT + C::kLoadsA : 2 * kNT>(p.bq[kk]);
    if (kk == 2) {
      // Every tile slot issues (past the end it reloads tile KT - 1 into a stage nobody reads
      // again): publish tile kt + 1, then refill the stage of tile kt, whose reads are done.
      lds_read_barrier();
      issue_tile<A16, true>(c, min(kt + S, KT - 1), la);
    }
    // weight fragments of step sigma + 3 (tile kt step 3, or tile kt + 1 step kk - 1), into the
    // slot step sigma - 1 used
    if constexpr (kk == 0)
      load_b(c, kt, 3, p.bq[3]);
    else
      load_b(c, kt + 1, kk - 1, p.bq[kk - 1]);
    // LDS words of step sigma + 2 (tile kt step kk + 2, or tile kt + 1 step kk - 2)
    if (kk < 2)
      read_step<A16>(c, la, kk + 2, p.raw[kk & 1]);
    else
      read_step<A16>(c, na, kk - 2, p.raw[kk & 1]);
    // activations of step sigma + 1
    convert_step<A16>(p.raw[(kk + 1) & 1], p.af[(kk + 1) & 1]);
    // MFMAs of step sigma.  16-bit acts: fragments mt = 2 i (high bytes) and 2 i + 1 (low
    // bytes) of row block i; columns nt = 0 (weight codes) and 1 (rounding residues).  The low
    // bytes' residue products are left out: their sum is bounded (|lo'| <= 128) and completed
    // only for listed outputs.
    static_for<4>([&](auto mt) {
      static_for<kNT>([&](auto nt) {
        if constexpr (!(A16 && (decltype(mt)::value & 1) && decltype(nt)::value == 1))
          acc[mt][nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(p.af[kk & 1][mt], p.bq[kk][nt], acc[mt][nt], 0, 0, 0);
      });
    });
    // issue order: the loads and fragment reads early, then one MFMA and a few conversion
    // instructions at a time
    constexpr int kMfmas = A16 ? 6 : 4 * kNT;
    constexpr int kValu = A16 ? 4 : 2;  // conversion work per MFMA
    static_for<kMfmas>([&](auto i) {
      constexpr int ii = decltype(i)::value;
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if constexpr (ii < 4) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      if constexpr (ii < kNT) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      if constexpr (kk == 2) {
        // the stage's tile loads, spread over the step's MFMAs
        constexpr int per = (C::kLoadsA + kMfmas - 1) / kMfmas;
        constexpr int n = C::kLoadsA - ii * per < per ? (C::kLoadsA - ii * per > 0 ? C::kLoadsA - ii * per : 0) : per;
        if constexpr (n > 0) __builtin_amdgcn_sched_group_barrier(0x020, n, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x002, kValu + (kk == 2 ? 4 : 0), 0);
    });
  });
}

// MODE 0: requantised output; MODE 1: exact int64 accumulators sum_k (a - zp) * w_int.
// CLAMP: clamp t before rounding (some column cannot prove |t| < 2^30).  OUT16: 16-bit outputs.
template <bool A16, int MODE, bool CLAMP, bool OUT16>
__global__ __launch_bounds__(kGemmThreads, 1) void qmm_gemm_kernel(const GemmArgs g) {
  using C = Cfg;
  // One LDS object per pipeline stage and operand: the compiler then knows that the
  // direct-to-LDS loads in flight (into other stages) cannot alias the fragment reads, and
  // does not make the reads wait for them.
  constexpr int S = C::kStages;
  static_assert(S == 2 || S == 3, "two or three stages");
  __shared__ __attribute__((aligned(16))) uint8_t sA0[kTileA], sA1[kTileA], sA2[S == 3 ? kTileA : 16];
  __shared__ uint32_t fix_list[kFixCap];  // (row << 16 | column) inside the tile
  // The exact integer sums of each listed output, taken from the accumulators: 8-bit acts
  // S1 = sum (a - 128) w (int32); 16-bit acts X = sum (a - 32896) w and Y = sum (a - 32896) r.
  __shared__ int64_t fix_val[MODE == 0 ? (A16 ? 2 * kFixCap : kFixCap / 2) : 1];
  __shared__ int fix_cnt;
  // Per-column epilogue constants of the tile, filled while the first operand tiles load.
  //   8-bit acts : [alpha | beta' | thr] x kBN columns;
  //   16-bit acts: [alpha | alpha * M | beta' | thr] x kBN / 2 columns.
  constexpr int CB = A16 ? kBN / 2 : kBN;  // real output columns of the tile
  __shared__ double ctab[MODE == 0 ? (A16 ? 4 : 3) * CB : 1];

  const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave % kWM, wn = wave / kWM;  // the wave's 128 rows and 64 operand columns of the tile
  int tm, tn;
  tile_of(blockIdx.x, g.TM, g.TN, &tm, &tn);
  const int rows_real = A16 ? kBM / 2 : kBM;
  const int cols_real = A16 ? kBN / 2 : kBN;
  const int m0 = tm * rows_real;
  const int n0 = tn * cols_real;
  const int M = g.M, K = g.K, KT = g.KT;
  const uint8_t *const act = g.act;
  const uint8_t *const btiles = g.tiles + static_cast<size_t>(tn) * KT * C::kTileB;
  if (t == 0) fix_cnt = 0;

  // stage indices are compile-time constants everywhere (the k loop is unrolled by S)
  auto stage_a = [&](auto st) -> uint8_t * { return st == 0 ? sA0 : (st == 1 ? sA1 : sA2); };

  const MainCtx mc{act, btiles + wn * (2 * kNT * 512), static_cast<uint32_t>(lane * 16), M, K, KT, m0, t, lane, wave, wm, wn};

  v16i acc[4][kNT];
  static_for<4>([&](auto i) { static_for<kNT>([&](auto j) { acc[i][j] = v16i{}; }); });

  // Prologue: the weight fragments of steps 0..2 and both activation stages (assembly, like the
  // loop's requests), then the per-column constants.  Those are ordinary loads issued last, so
  // the compiler's wait for them (before the table writes below) also covers every operand
  // request before them: the loop starts with nothing of the prologue in flight.
  PipeRegs pr;
  load_b(mc, 0, 0, pr.bq[0]);
  load_b(mc, 0, 1, pr.bq[1]);
  load_b(mc, 0, 2, pr.bq[2]);
  static_for<S>([&](auto p) { issue_tile<A16, true>(mc, min(static_cast<int>(p), KT - 1), stage_a(p)); });
  double cv[5] = {0.0, 0.0, 0.0, 0.0, 0.0};
  int64_t ccorr = 0, cmant = 0;
  static_assert(kBN <= kGemmThreads, "one thread per column loads the column constants");
  const int ccol = t & (CB - 1);
  const int cn = n0 + ccol < g.N ? n0 + ccol : 0;
  if (MODE == 0) {
    cv[0] = g.alpha[cn];
    cv[1] = g.beta[cn];
    cv[2] = g.margin[cn] + (A16 ? g.margin_lo[cn] : 0.0);
    cv[3] = g.absb[cn];
    ccorr = g.corr[cn];
    if (A16) cmant = g.mant[cn];
  }
  if (MODE == 0) {
    const double alpha = cv[0];
    // zero-point correction folded into the offset: t = acc * alpha + (beta + corr * alpha)
    const double betap = fma(static_cast<double>(ccorr), alpha, cv[1]);
    const double corr_term = 2.0 * fabs(static_cast<double>(ccorr) * alpha);
    if (!A16 && t < CB) {
      // |t - rint(t)| <= thr certifies the rounding; slack for |t| <= qmax + 2 folded in
      ctab[t] = alpha;
      ctab[CB + t] = betap;
      ctab[2 * CB + t] = 0.5 - cv[2] - 0x1p-48 * (cv[3] + corr_term + static_cast<double>(g.out_qmax) + 2.0);
    } else if (A16 && t < CB) {
      // t = Y * alpha + (X * alpha M + beta'); |X| <= K * 33024 * 127 bounds the float slack
      const double alpha_m = alpha * static_cast<double>(cmant);
      const double umax = fabs(alpha_m) * static_cast<double>(K) * (33024.0 * 127.0);
      ctab[t] = alpha;
      ctab[CB + t] = alpha_m;
      ctab[2 * CB + t] = betap;
      ctab[3 * CB + t] = 0.5 - cv[2] - 0x1p-48 * (cv[3] + corr_term + umax + static_cast<double>(g.out_qmax) + 2.0);
    }
  }

  // k loop, unrolled by the stage count so every stage is a compile-time LDS object
  {
    wait_vmcnt<0>();     // the prologue's requests (MODE 1 has no constants to wait for)
    lds_read_barrier();  // tiles 0 .. S - 1 landed in every wave; also publishes the constants above
    read_step<A16>(mc, sA0, 0, pr.raw[0]);
    read_step<A16>(mc, sA0, 1, pr.raw[1]);
    convert_step<A16>(pr.raw[0], pr.af[0]);
  }
  auto tile = [&](const int kt, auto sc) __attribute__((always_inline)) {
    constexpr int rs = decltype(sc)::value, ns = (rs + 1) % S;
    k_tile<A16>(mc, kt, KT, stage_a(sc), stage_a(std::integral_constant<int, ns>{}), pr, acc);
  };
  // The loop body is S whole tiles (every stage a compile-time object, no branch inside); the
  // last KT mod S tiles run after it.
  int kt0 = 0;
  for (; kt0 + S <= KT; kt0 += S) static_for<S>([&](auto j) { tile(kt0 + decltype(j)::value, j); });
  static_for<S - 1>([&](auto j) {
    if (kt0 + decltype(j)::value < KT) tile(kt0 + decltype(j)::value, j);
  });
  // Every request issued from assembly has landed.  The ring's registers pass through the wait:
  // the weight loads of the steps past the end are never read, and without this use the
  // compiler would hand their registers to other values while the loads can still write them.
  asm volatile("s_waitcnt vmcnt(0)"
               : "+v"(pr.bq[0][0]), "+v"(pr.bq[0][1]), "+v"(pr.bq[1][0]), "+v"(pr.bq[1][1]), "+v"(pr.bq[2][0]),
                 "+v"(pr.bq[2][1]), "+v"(pr.bq[3][0]), "+v"(pr.bq[3][1]));
  static_assert(Cfg::kBRing == 4 && kNT == 2, "every ring slot passes through the final wait");
  // ---------------------------------------------------------------- epilogue
  // Straight from the accumulator registers: each lane requantises the 4-row strips of its
  // MFMA blocks (one column), then the 4 lanes of a quad transpose their strips (DPP quad
  // broadcasts + byte permutes) so every lane stores 4 adjacent outputs of one row.
  // Rounding: t + 1.5 * 2^52 leaves rint(t) in the low word (|t| < 2^30 is proven per
  // column at prepare time, otherwise t is clamped first).  A strip whose largest
  // |t - rint(t)| exceeds the column's certified threshold takes a rare path that lists its
  // uncertain outputs in LDS together with their exact accumulator sums; beyond the list's
  // capacity it marks them instead (in an operand stage every wave has finished reading: one
  // dword per thread and 32x32 block, byte jg = strip jg, bit jj = row jj).  An output is
  // uncertain only if rint(t) lies in [0, qmax] (otherwise both candidate roundings clamp to
  // the same output).
  const int q = lane & 3;
  const double qmaxd = static_cast<double>(g.out_qmax);
  constexpr int kBlocks = A16 ? 2 : 4 * kNT;  // 32-row x 32-column output blocks per lane
  uint32_t *const flagw = reinterpret_cast<uint32_t *>(sA0);  // [kBlocks][kGemmThreads]
  uint8_t *const flagb = sA0;
  if (MODE == 1) {
    // exact int64 accumulators sum_k (a - zp) * w_int
    if (!A16) {
      static_for<kNT>([&](auto nt) {
        const int n = n0 + wn * 64 + nt * 32 + (lane & 31);
        if (n >= g.N) return;
        const int64_t corr = g.corr[n];
        static_for<4>([&](auto mt) {
          static_for<16>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            const int m = m0 + wm * 128 + mt * 32 + 8 * (j / 4) + 4 * (lane >> 5) + (j % 4);
            if (m < M)
              reinterpret_cast<int64_t *>(g.out)[static_cast<size_t>(m) * g.N + n] = static_cast<int64_t>(acc[mt][nt][j]) + corr;
          });
        });
      });
    } else {
      {
        // the wave's 64 operand columns: 32 weight-code columns, then their 32 residue columns
        const int n = n0 + wn * 32 + (lane & 31);
        if (n >= g.N) return;
        const int64_t csum = g.colsum[n] * static_cast<int64_t>(128 + 32768 - g.act_zp);
        static_for<2>([&](auto mt) {
          static_for<16>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            const int m = m0 + wm * 64 + mt * 32 + 8 * (j / 4) + 4 * (lane >> 5) + (j % 4);
            if (m < M)
              reinterpret_cast<int64_t *>(g.out)[static_cast<size_t>(m) * g.N + n] =
                  256 * static_cast<int64_t>(acc[2 * mt][0][j]) + acc[2 * mt + 1][0][j] + csum;
          });
        });
      }
    }
    return;
  }
  __syncthreads();
#pragma unroll
  for (int b = 0; b < kBlocks; ++b) flagw[b * kGemmThreads + t] = 0u;  // this thread's own marks
  // Output addressing: one buffer resource over the tile's rows below M, and per lane the byte
  // offset of its first store (row q of its quad's strip, 4 columns); a strip adds a
  // compile-time row step times the row pitch.  A lane whose 32-column block lies past N (N is
  // a multiple of 32) gets an offset past the resource, so its stores are dropped as well.
  constexpr uint32_t esz = OUT16 ? 2u : 1u;
  const uint32_t pitch = static_cast<uint32_t>(g.N) * esz;  // <= 2^21 bytes
  const auto orsrc = out_rsrc(static_cast<uint8_t *>(g.out) + (static_cast<size_t>(m0) * g.N + n0) * esz,
                              static_cast<uint32_t>(min(M - m0, rows_real)) * pitch);
  const StripLane sl = strip_lane<OUT16>(q);
  constexpr uint32_t kPast = 0x80000000u;  // > 128 rows x 2^21 bytes: past any tile's resource
  if (!A16) {
    static_for<kNT>([&](auto nt) {
      const int cl = wn * 64 + nt * 32 + (lane & 31);  // column inside the tile
      const double alpha = ctab[cl], beta = ctab[CB + cl], thr = ctab[2 * CB + cl];
      const uint32_t off0 = n0 + wn * 64 + nt * 32 < g.N
                                ? static_cast<uint32_t>(wm * 128 + 4 * (lane >> 5) + q) * pitch +
                                      static_cast<uint32_t>(wn * 64 + nt * 32 + (lane & 28)) * esz
                                : kPast;
      static_for<4>([&](auto mt) {
        static_for<4>([&](auto jg) {
          int o[4];
          double dmax = 0.0;
          static_for<4>([&](auto jj) {
            const double tv = fma(static_cast<double>(acc[mt][nt][4 * decltype(jg)::value + decltype(jj)::value]), alpha, beta);
            int oi;
            const double d = round_near<CLAMP>(tv, qmaxd, &oi);
            dmax = decltype(jj)::value == 0 ? d : fmax(dmax, d);
            o[jj] = clamp_out(oi, g.out_qmax);
          });
          if (dmax > thr) {  // rare: list the uncertain outputs of the strip with their sums
            // the strip's first row, formed here: the common path does not need it
            int rb = wm * 128 + 4 * (lane >> 5);
            asm volatile("" : "+v"(rb));
            const int R = rb + mt * 32 + 8 * jg;
            uint32_t keep = 0;
            static_for<4>([&](auto jjc) {
              constexpr int j = 4 * decltype(jg)::value + decltype(jjc)::value;
              const double tv = fma(static_cast<double>(acc[mt][nt][j]), alpha, beta);
              int oi;
              const double d = round_near<CLAMP>(tv, qmaxd, &oi);
              const int r = R + decltype(jjc)::value;
              if ((d > thr) & (static_cast<uint32_t>(oi) <= static_cast<uint32_t>(g.out_qmax)) && m0 + r < M && n0 + cl < g.N) {
                const int slot = atomicAdd(&fix_cnt, 1);
                if (slot < kFixCap) {
                  fix_list[slot] = (static_cast<uint32_t>(r) << 16) | static_cast<uint32_t>(cl);
                  reinterpret_cast<int32_t *>(fix_val)[slot] = acc[mt][nt][j];
                } else {
                  keep |= 1u << decltype(jjc)::value;  // beyond the list: a later pass
                }
              }
            });
            if (keep) flagb[((nt * 4 + mt) * kGemmThreads + t) * 4 + jg] = static_cast<uint8_t>(keep);
          }
          store_strip<OUT16>(orsrc, off0 + row_step<mt * 32 + 8 * jg>(pitch), o, sl);
        });
      });
    });
  } else {
    // 16-bit activations: real row tiles mt (32 rows), real column tiles c (32 columns);
    // acc[2mt + p][2c + s]: p = hi / lo' activation byte, s = weight code / rounding residue.
    // X = sum (a-32768)' q and Y = sum (a-32768)' r are exact in float64.
    {
      constexpr int c = 0;  // one group of 32 real columns per wave
      const int cl = wn * 32 + (lane & 31);
      const double alpha = ctab[cl], alpha_m = ctab[CB + cl], beta = ctab[2 * CB + cl], thr = ctab[3 * CB + cl];
      const uint32_t off0 = n0 + wn * 32 < g.N ? static_cast<uint32_t>(wm * 64 + 4 * (lane >> 5) + q) * pitch +
                                                     static_cast<uint32_t>(wn * 32 + (lane & 28)) * esz
                                               : kPast;
      static_for<2>([&](auto mt) {
        static_for<4>([&](auto jg) {
          auto t_of = [&](auto jj) {
            constexpr int j = 4 * decltype(jg)::value + decltype(jj)::value;
            const double X = fma(static_cast<double>(acc[2 * mt][2 * c][j]), 256.0, static_cast<double>(acc[2 * mt + 1][2 * c][j]));
            const double Y = 256.0 * static_cast<double>(acc[2 * mt][2 * c + 1][j]);  // high-byte residue sum
            return fma(Y, alpha, fma(X, alpha_m, beta));
          };
          int o[4];
          double dmax = 0.0;
          static_for<4>([&](auto jj) {
            int oi;
            const double d = round_near<CLAMP>(t_of(jj), qmaxd, &oi);
            dmax = decltype(jj)::value == 0 ? d : fmax(dmax, d);
            o[jj] = clamp_out(oi, g.out_qmax);
          });
          if (dmax > thr) {  // rare: list the uncertain outputs of the strip with their sums
            // the strip's first row, formed here: the common path does not need it
            int rb = wm * 64 + 4 * (lane >> 5);
            asm volatile("" : "+v"(rb));
            const int R = rb + mt * 32 + 8 * jg;
            uint32_t keep = 0;
            static_for<4>([&](auto jjc) {
              constexpr int j = 4 * decltype(jg)::value + decltype(jjc)::value;
              int oi;
              const double d = round_near<CLAMP>(t_of(jjc), qmaxd, &oi);
              const int r = R + decltype(jjc)::value;
              if ((d > thr) & (static_cast<uint32_t>(oi) <= static_cast<uint32_t>(g.out_qmax)) && m0 + r < M && n0 + cl < g.N) {
                const int slot = atomicAdd(&fix_cnt, 1);
                if (slot < kFixCap) {
                  fix_list[slot] = (static_cast<uint32_t>(r) << 16) | static_cast<uint32_t>(cl);
                  fix_val[2 * slot] = 256 * static_cast<int64_t>(acc[2 * mt][2 * c][j]) + acc[2 * mt + 1][2 * c][j];
                  fix_val[2 * slot + 1] = 256 * static_cast<int64_t>(acc[2 * mt][2 * c + 1][j]);
                } else {
                  keep |= 1u << decltype(jjc)::value;  // beyond the list: a later pass
                }
              }
            });
            if (keep) flagb[((c * 2 + mt) * kGemmThreads + t) * 4 + jg] = static_cast<uint8_t>(keep);
          }
          store_strip<OUT16>(orsrc, off0 + row_step<mt * 32 + 8 * jg>(pitch), o, sl);
        });
      });
    }
  }

  // ---------------------------------------------------------------- exact fixup
  // With s32 = M * 2^E the oracle's weight is fl32(w * s32) = 2^E * W', W' = w * M + r for an
  // integer residue r, so the exact dot product is 2^E * D with
  //   D = sum_k (a_k - zp) W'_k = M * S1 + S2 + (base - zp) * (M * sum_k w_k + sum_k r_k),
  //   S1 = sum_k (a_k - base) w_k,  S2 = sum_k (a_k - base) r_k.
  // Marked outputs were listed by the epilogue with their accumulator sums: 8-bit acts S1
  // (base 128); 16-bit acts S1 and S2 (base 32896, codes and residue columns).  Each wave takes
  // whole outputs, forms S2 for 8-bit acts from the prepared residue plane (dot4 over K), and
  // decides: t = D * sA * 2^E / sO + beta rounds like the oracle unless t is still within the
  // oracle's own float64 noise of a boundary; those outputs get the float64 emulation of the
  // oracle's dot product.  Marks beyond the list's capacity stay in the mark words and are
  // handled in later passes that form S1 and S2 from the operands (base 128 or 32768).
  const int KC = K / 16;
  constexpr int P = A16 ? 2 : 4;  // 16-byte K chunks per lane in flight (16-bit acts: 48 bytes each)
  lds_read_barrier();   // listed outputs and overflow marks complete
  const int listed = fix_cnt;
  if (listed > 0) {
    const int cnt = listed < kFixCap ? listed : kFixCap;
    const int abase_acc = A16 ? 32896 : 128;
    // Operands of one listed output: its column's constants and, per K round of 64 lanes x P
    // chunks of 16 k, the activation row and the residue row (8-bit acts) or the residue column
    // of the tiles (16-bit acts).  Chunks past K read chunk 0 and count as zero.
    struct FixOps {
      int m, n;
      long long mant, csum, csum_r;
      double alpha_e, beta, margin, absb;
      uint4 av[P][A16 ? 2 : 1], rv[P];
    };
    auto fix_rows = [&](FixOps &f, int kc0) __attribute__((always_inline)) {
#pragma unroll
      for (int pp = 0; pp < P; ++pp) {
        const int kc = kc0 + lane + 64 * pp;
        const int kk = kc < KC ? kc : 0;
        if (!A16) {
          f.av[pp][0] = reinterpret_cast<const uint4 *>(act + static_cast<size_t>(f.m) * K)[kk];
          f.rv[pp] = reinterpret_cast<const uint4 *>(g.resid + static_cast<size_t>(f.n) * K)[kk];
        } else {
          const uint16_t *const arow = reinterpret_cast<const uint16_t *>(act) + static_cast<size_t>(f.m) * K;
          f.rv[pp] = load_w16_raw(g, (f.n / 32) * 64 + 32 + (f.n % 32), kk * 16);
          f.av[pp][0] = *reinterpret_cast<const uint4 *>(arow + kk * 16);
          f.av[pp][A16 ? 1 : 0] = *reinterpret_cast<const uint4 *>(arow + kk * 16 + 8);
        }
      }
    };
    auto fix_load = [&](FixOps &f, int e) __attribute__((always_inline)) {
      const uint32_t v = __builtin_amdgcn_readfirstlane(fix_list[e]);  // uniform in the wave
      f.m = m0 + static_cast<int>(v >> 16);
      f.n = n0 + static_cast<int>(v & 0xFFFFu);
      // The index goes through a vector register: as wave-uniform values the compiler would move
      // the constants to scalar registers at once, which waits for their loads before the rows issue.
      int nv = f.n;
      asm volatile("" : "+v"(nv));
      f.mant = g.mant[nv];
      f.csum = g.colsum[nv];
      f.csum_r = g.colsum_r[nv];
      f.alpha_e = g.alpha_e[nv];
      f.beta = g.beta[nv];
      f.margin = g.margin_exact[nv];
      f.absb = g.absb[nv];
      fix_rows(f, 0);
    };
    // This wave's first listed output is requested before the wait for the provisional stores,
    // so the operand latency and the store drain overlap.
    FixOps fo;
    if (wave < cnt) fix_load(fo, wave);
    __syncthreads();  // every provisional output is stored before any is rewritten
    for (int e = wave; e < cnt; e += kGemmThreads / 64) {
      if (e != wave) fix_load(fo, e);
      const int m = fo.m, n = fo.n;
      long long S1, S2;
      int s2 = 0;  // 8-bit acts: sum_k (a_k - 128) r_k; 16-bit: sum_k lo'_k r_k (|.| <= 128 * 64 * K < 2^31)
      for (int kc0 = 0; kc0 < KC; kc0 += 64 * P) {
        if (kc0 > 0) fix_rows(fo, kc0);
#pragma unroll
        for (int pp = 0; pp < P; ++pp) {
          const uint32_t keep = kc0 + lane + 64 * pp < KC ? 0xFFFFFFFFu : 0u;
          const uint4 r = fo.rv[pp];
          if (!A16) {
            const uint4 a = fo.av[pp][0];
            s2 = __builtin_amdgcn_sdot4(static_cast<int>(a.x ^ 0x80808080u), static_cast<int>(r.x & keep), s2, false);
            s2 = __builtin_amdgcn_sdot4(static_cast<int>(a.y ^ 0x80808080u), static_cast<int>(r.y & keep), s2, false);
            s2 = __builtin_amdgcn_sdot4(static_cast<int>(a.z ^ 0x80808080u), static_cast<int>(r.z & keep), s2, false);
            s2 = __builtin_amdgcn_sdot4(static_cast<int>(a.w ^ 0x80808080u), static_cast<int>(r.w & keep), s2, false);
          } else {
            // low activation bytes (a & 255) - 128 times the residue column
            const uint4 a0 = fo.av[pp][0], a1 = fo.av[pp][A16 ? 1 : 0];
            s2 = __builtin_amdgcn_sdot4(static_cast<int>(perm(a0.y, a0.x, 0x06040200u) ^ 0x80808080u), static_cast<int>(r.x & keep), s2, false);
            s2 = __builtin_amdgcn_sdot4(static_cast<int>(perm(a0.w, a0.z, 0x06040200u) ^ 0x80808080u), static_cast<int>(r.y & keep), s2, false);
            s2 = __builtin_amdgcn_sdot4(static_cast<int>(perm(a1.y, a1.x, 0x06040200u) ^ 0x80808080u), static_cast<int>(r.z & keep), s2, false);
            s2 = __builtin_amdgcn_sdot4(static_cast<int>(perm(a1.w, a1.z, 0x06040200u) ^ 0x80808080u), static_cast<int>(r.w & keep), s2, false);
          }
        }
      }
      if (!A16) {
        S1 = __builtin_amdgcn_readfirstlane(reinterpret_cast<const int32_t *>(fix_val)[e]);
        S2 = wave_sum(s2);
      } else {
        const long long x = fix_val[2 * e], y = fix_val[2 * e + 1];
        S1 = static_cast<long long>(static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(x)))) |
             (static_cast<long long>(__builtin_amdgcn_readfirstlane(static_cast<int>(x >> 32))) << 32);
        S2 = static_cast<long long>(static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(y)))) |
             (static_cast<long long>(__builtin_amdgcn_readfirstlane(static_cast<int>(y >> 32))) << 32);
        S2 += wave_sum(s2);
      }
      // |D| < 2^63; partial terms may wrap, so the sum is formed modulo 2^64
      const unsigned long long M64 = static_cast<unsigned long long>(fo.mant);
      const unsigned long long sw = M64 * static_cast<unsigned long long>(fo.csum) + static_cast<unsigned long long>(fo.csum_r);
      const unsigned long long Du = M64 * static_cast<unsigned long long>(S1) + static_cast<unsigned long long>(S2) +
                                    static_cast<unsigned long long>(static_cast<long long>(abase_acc - g.act_zp)) * sw;
      const double u = static_cast<double>(static_cast<long long>(Du)) * fo.alpha_e;
      const double tv = u + fo.beta;
      const double rd = rint(tv);
      const double slack = fo.margin + 0x1p-48 * (fabs(u) + fabs(tv) + fo.absb);
      if (fabs(tv - rd) > 0.5 - slack) {
        fixup_one<A16>(g, m, n, lane);
      } else if (lane == 0) {
        const int oi = static_cast<int>(rd);
        store_out(g.out, OUT16, static_cast<size_t>(m) * g.N + n, oi < 0 ? 0 : (oi > g.out_qmax ? g.out_qmax : oi));
      }
    }
    if (listed > kFixCap) {
      // overflow: the remaining marks, listed and recomputed from the operands pass by pass
      lds_read_barrier();
      if (t == 0) fix_cnt = 0;
      const int abase = A16 ? 32768 : 128;
      constexpr int EW = 1;  // outputs per wave in flight together
      for (;;) {
        lds_read_barrier();  // overflow marks complete
        uint32_t marks[kBlocks];
#pragma unroll
        for (int b = 0; b < kBlocks; ++b) marks[b] = flagw[b * kGemmThreads + t];
#pragma unroll
        for (int b = 0; b < kBlocks; ++b) {
          uint32_t mk = marks[b];
          if (mk == 0) continue;
          uint32_t keep = 0;
          const int rb = A16 ? wm * 64 + (b & 1) * 32 + 4 * (lane >> 5) : wm * 128 + (b & 3) * 32 + 4 * (lane >> 5);
          const int c = A16 ? wn * 32 + (lane & 31) : wn * 64 + (b >> 2) * 32 + (lane & 31);
          while (mk) {
            const int bit = __builtin_ctz(mk);
            mk &= mk - 1;
            const int r = rb + 8 * (bit >> 3) + (bit & 7);
            if (m0 + r >= M || n0 + c >= g.N) continue;  // padding rows / columns of the tile
            const int slot = atomicAdd(&fix_cnt, 1);
            if (slot < kFixCap)
              fix_list[slot] = (static_cast<uint32_t>(r) << 16) | static_cast<uint32_t>(c);
            else
              keep |= 1u << bit;  // listed in a later pass
          }
          flagw[b * kGemmThreads + t] = keep;
        }
        lds_read_barrier();
        const int total = fix_cnt;
        if (total == 0) break;
        const int cnt = total < kFixCap ? total : kFixCap;
        for (int e0 = wave * EW; e0 < cnt; e0 += (kGemmThreads / 64) * EW) {
          // every per-output constant is requested together with the first operand chunks
          int mrow[EW], ncol[EW], mant[EW];
          float mf[EW];
          int64_t csq[EW], csr[EW];
          double ae[EW], bt[EW], mx[EW], ab[EW];
#pragma unroll
          for (int i = 0; i < EW; ++i) {
            const int e = e0 + i < cnt ? e0 + i : cnt - 1;
            const uint32_t v = __builtin_amdgcn_readfirstlane(fix_list[e]);  // uniform in the wave
            mrow[i] = m0 + static_cast<int>(v >> 16);
            const int n = n0 + static_cast<int>(v & 0xFFFFu);
            ncol[i] = n;
            mant[i] = static_cast<int>(g.mant[n]);
            mf[i] = static_cast<float>(mant[i]);  // exact: M < 2^24
            csq[i] = g.colsum[n];
            csr[i] = g.colsum_r[n];
            ae[i] = g.alpha_e[n];
            bt[i] = g.beta[n];
            mx[i] = g.margin_exact[n];
            ab[i] = g.absb[n];
          }
          long long S1[EW], S2[EW];
#pragma unroll
          for (int i = 0; i < EW; ++i) S1[i] = S2[i] = 0;
          for (int kc0 = 0; kc0 < KC; kc0 += 64 * P) {
            uint4 wr[EW][P];
            uint4 av[EW][P][A16 ? 2 : 1];
#pragma unroll
            for (int i = 0; i < EW; ++i) {
#pragma unroll
              for (int pp = 0; pp < P; ++pp) {
                const int kc = kc0 + lane + 64 * pp;
                const int k = kc < KC ? kc * 16 : 0;
                const int n = ncol[i];
                wr[i][pp] = load_w16_raw(g, A16 ? (n / 32) * 64 + (n % 32) : n, k);
                const uint4 *ap = reinterpret_cast<const uint4 *>(act + (static_cast<size_t>(mrow[i]) * K + k) * (A16 ? 2 : 1));
                av[i][pp][0] = ap[0];
                if (A16) av[i][pp][A16 ? 1 : 0] = ap[1];
              }
            }
#pragma unroll
            for (int i = 0; i < EW; ++i) {
              int s1 = 0, s2 = 0;  // |.| < 2^28 for P * 16 terms
#pragma unroll
              for (int pp = 0; pp < P; ++pp) {
                if (kc0 + lane + 64 * pp >= KC) continue;
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                  const int a = (A16 ? static_cast<int>(reinterpret_cast<const uint16_t *>(&av[i][pp][j >> 3])[j & 7])
                                     : static_cast<int>(reinterpret_cast<const uint8_t *>(&av[i][pp][0])[j])) - abase;
                  const int wj = w_at(wr[i][pp], j);
                  // W' = fl32(w * s32) / 2^E = fl32(w * M) (s32 = M * 2^E, no subnormals): the
                  // residue r = W' - w * M is minus the exact rounding error of that product
                  const float wf = static_cast<float>(wj);
                  const float prod = __fmul_rn(wf, mf[i]);
                  const int r = -static_cast<int>(__fmaf_rn(wf, mf[i], -prod));
                  s1 += __mul24(a, wj);
                  s2 += __mul24(a, r);
                }
              }
              S1[i] += s1;
              S2[i] += s2;
            }
          }
#pragma unroll
          for (int i = 0; i < EW; ++i) {
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) {
              S1[i] += __shfl_xor(S1[i], off, 64);
              S2[i] += __shfl_xor(S2[i], off, 64);
            }
            if (e0 + i >= cnt) continue;
            const int m = mrow[i], n = ncol[i];
            // |D| < 2^63; partial terms may wrap, so the sum is formed modulo 2^64
            const unsigned long long M64 = static_cast<unsigned long long>(static_cast<long long>(mant[i]));
            const unsigned long long sw = M64 * static_cast<unsigned long long>(csq[i]) + static_cast<unsigned long long>(csr[i]);
            const unsigned long long Du = M64 * static_cast<unsigned long long>(S1[i]) + static_cast<unsigned long long>(S2[i]) +
                                          static_cast<unsigned long long>(static_cast<long long>(abase - g.act_zp)) * sw;
            const double u = static_cast<double>(static_cast<long long>(Du)) * ae[i];
            const double tv = u + bt[i];
            const double rd = rint(tv);
            const double slack = mx[i] + 0x1p-48 * (fabs(u) + fabs(tv) + ab[i]);
            if (fabs(tv - rd) > 0.5 - slack) {
              fixup_one<A16>(g, m, n, lane);
            } else if (lane == 0) {
              const int oi = static_cast<int>(rd);
              store_out(g.out, OUT16, static_cast<size_t>(m) * g.N + n, oi < 0 ? 0 : (oi > g.out_qmax ? g.out_qmax : oi));
            }
          }
        }
        if (total <= kFixCap) break;
        lds_read_barrier();
        if (t == 0) fix_cnt = 0;
      }
    }
  }
}

template <bool A16, int MODE>
qh_status launch(const GemmArgs &g, bool clamp, hipStream_t stream) {
  dim3 grid(g.TM * g.TN);
  if constexpr (MODE == 0) {
    if (clamp && g.out16)
      hipLaunchKernelGGL((qmm_gemm_kernel<A16, 0, true, true>), grid, dim3(kGemmThreads), 0, stream, g);
    else if (clamp)
      hipLaunchKernelGGL((qmm_gemm_kernel<A16, 0, true, false>), grid, dim3(kGemmThreads), 0, stream, g);
    else if (g.out16)
      hipLaunchKernelGGL((qmm_gemm_kernel<A16, 0, false, true>), grid, dim3(kGemmThreads), 0, stream, g);
    else
      hipLaunchKernelGGL((qmm_gemm_kernel<A16, 0, false, false>), grid, dim3(kGemmThreads), 0, stream, g);
  } else {
    hipLaunchKernelGGL((qmm_gemm_kernel<A16, MODE, false, false>), grid, dim3(kGemmThreads), 0, stream, g);
  }
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return hip_fail(err, "qmm_gemm_kernel launch");
  return QH_STATUS_OK;
}

template <int MODE>
qh_status dispatch(const qh_qmm_prepared *p, int m, const void *act, void *out, hipStream_t stream) {
  const QmmShape &sh = p->shape;
  const QmmDevice &D = p->dev;
  GemmArgs g{};
  g.act = static_cast<const uint8_t *>(act);
  g.out = out;
  g.tiles = D.tiles;
  g.alpha = D.alpha;
  g.beta = D.beta;
  g.margin = D.margin;
  g.absb = D.absb;
  g.bias_deq = D.bias_deq;
  g.corr = D.corr;
  g.mant = D.mant;
  g.colsum = D.colsum;
  g.colsum_r = D.colsum_r;
  g.alpha_e = D.alpha_e;
  g.scale_exp = D.scale_exp;
  g.margin_exact = D.margin_exact;
  g.margin_lo = D.margin_lo;
  g.s32 = D.s32;
  g.resid = D.resid;
  g.M = m;
  g.N = sh.N;
  g.K = sh.K;
  g.KT = sh.Kp / kBK;
  g.act_zp = sh.act_zp;
  g.out_zp = sh.out_zp;
  g.out_qmax = (1 << sh.out_bits) - 1;
  g.out16 = sh.out_bits == 16;
  g.sA = sh.act_scale;
  g.sO = sh.out_scale;
  const bool a16 = sh.act_bits == 16;
  const int rows_real = a16 ? kBM / 2 : kBM;
  g.TN = sh.ncols_op / kBN;
  g.TM = (m + rows_real - 1) / rows_real;
  if (static_cast<long long>(g.TM) * g.TN > 0x7FFFFFFFLL) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "M=%d too large", m);
  const bool clamp = sh.epi_clamp != 0;
  if (!a16) return launch<false, MODE>(g, clamp, stream);
  return launch<true, MODE>(g, clamp, stream);
}

}  // namespace

qh_status launch_qmm_gemm(const qh_qmm_prepared *p, int m, const void *act, void *out, hipStream_t stream) {
  return dispatch<0>(p, m, act, out, stream);
}

qh_status launch_qmm_accumulate(const qh_qmm_prepared *p, int m, const void *act, int64_t *acc, hipStream_t stream) {
  return dispatch<1>(p, m, act, acc, stream);
}

}  // namespace qh
