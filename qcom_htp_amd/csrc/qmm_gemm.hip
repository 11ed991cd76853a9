// Quantized GEMM on gfx950 i8 MFMA (v_mfma_i32_32x32x32_i8), bit-exact to the reference's
// float-derived requantisation.
//
// Workgroup: 256 threads = 4 waves in a 2x2 grid over a 256 x 256 tile of the i8 operand
// space (activation rows x weight-operand columns); each wave owns 4x4 MFMA 32x32 blocks.
// K is consumed 128 deep per pipeline step.
//
// Data movement: every operand tile goes global -> LDS with direct-to-LDS loads
// (global_load_lds_dwordx4), bypassing VGPRs; STAGES tiles are in flight and one barrier per
// step both publishes the landed tile and frees the oldest stage.  Weight tiles are prepared
// as the exact LDS image (pre-swizzled), activation tiles are gathered into the swizzled
// layout by the per-lane source addresses.  Operand conversion happens on the MFMA fragments
// after the LDS read:
//   * 8-bit activations: XOR 0x80 gives the signed a - 128;
//   * 16-bit activations a - 32768 = 256*hi + lo' + 128: the hi and lo' bytes of each u16
//     become two int8 fragments, each multiplied into its own accumulator;
//   * int4 weights (offset-binary nibbles) widen to int8 in registers, LPBQ block scales are
//     applied there too: (u*f + 128 - 8f) ^ 0x80 per byte is the two's complement of
//     (u - 8) * f without carries between bytes.
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
  const uint8_t *lpbq;
  const double *alpha, *beta, *margin, *absb, *bias_deq;
  const double *alpha_e, *inv_pow2e, *margin_exact;
  const int64_t *corr, *mant, *colsum, *colsum_r;
  const float *s32;
  int M, N, K, KT, TM, TN;
  int act_zp, out_zp, out_qmax, out16;
  double sA, sO;
};

constexpr int kTileA = 32768;  // A8: 256 rows x 128 B; A16: 128 rows x 256 B

template <bool A16, int TFMT, bool LPBQ>
struct Cfg {
  static constexpr int kTileB = TFMT == kTileI8 ? 32768 : 16384;
  static constexpr int kTileF = LPBQ ? 1024 : 0;
  static constexpr int kStageBytes = kTileA + kTileB + kTileF;
  static constexpr int kStages = TFMT == kTileI8 ? 2 : 3;
  static constexpr int kLoadsA = kTileA / 4096;   // 16-byte loads per thread per stage
  static constexpr int kLoadsB = kTileB / 4096;
  static constexpr int kLoads = kLoadsA + kLoadsB + (LPBQ ? 1 : 0);  // per wave per stage
  static constexpr int kArena = kStages * kStageBytes;
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

__device__ __forceinline__ void load_lds16(const void *gsrc, void *lds_wave_base) {
  __builtin_amdgcn_global_load_lds((gbl_void_ptr)(const_cast<void *>(gsrc)), (lds_void_ptr)(lds_wave_base), 16, 0, 0);
}

// int4 offset-binary nibbles (already masked to 0x0F per byte) -> int8 (u - 8) * f.
__device__ __forceinline__ uint32_t widen4(uint32_t x, uint32_t f, uint32_t bias) {
  return (x * f + bias) ^ 0x80808080u;
}

__device__ __forceinline__ void store_out(void *out, int out16, size_t idx, int v) {
  if (out16)
    static_cast<uint16_t *>(out)[idx] = static_cast<uint16_t>(v);
  else
    static_cast<uint8_t *>(out)[idx] = static_cast<uint8_t>(v);
}

// 16 consecutive integer weights (k .. k+15, k % 16 == 0) of operand column cb.
template <int TFMT, bool LPBQ>
__device__ __forceinline__ void load_w16(const GemmArgs g, int cb, int k, int (&w)[16]) {
  const size_t tile = static_cast<size_t>(cb / kBN) * g.KT + k / kBK;
  if (TFMT == kTileI8) {
    const uint8_t *p = g.tiles + tile * (kBN * kBK) + tile_off_i8(cb % kBN, k);
    uint4 v = *reinterpret_cast<const uint4 *>(p);
    const int8_t *b = reinterpret_cast<const int8_t *>(&v);
#pragma unroll
    for (int j = 0; j < 16; ++j) w[j] = b[j];
  } else {
    const uint8_t *p = g.tiles + tile * (kBN * kBK / 2) + tile_off_i4(cb % kBN, k);
    uint2 v = *reinterpret_cast<const uint2 *>(p);
    const uint8_t *b = reinterpret_cast<const uint8_t *>(&v);
    int f = 1;
    if (LPBQ) f = g.lpbq[tile * (kBN * 4) + (cb % kBN) * 4 + ((k & 127) >> 5)];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      w[j] = ((b[j] & 15) - 8) * f;
      w[j + 8] = ((b[j] >> 4) - 8) * f;
    }
  }
}

// Exact float64 recomputation of one output, term by term as the oracle forms it:
// sum_k fl64((a_k - zp) * sA) * fl32(w_k * s32), then + bias_deq, / sO, + out_zp, rint, clip.
template <bool A16, int TFMT, bool LPBQ>
__device__ __noinline__ void fixup_one(const GemmArgs g, int m, int n, int lane) {
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
        load_w16<TFMT, LPBQ>(g, cb, k, w[i]);
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
// of 4 row tiles, so an XCD's concurrent tiles share activation rows and weight columns.
__device__ __forceinline__ void tile_of(int w, int TM, int TN, int *tm, int *tn) {
  const int T = TM * TN;
  int lin = w;
  if ((T & 7) == 0) lin = (w & 7) * (T >> 3) + (w >> 3);
  constexpr int GM = 4;
  const int group = GM * TN;
  const int gid = lin / group, first = gid * GM;
  const int gm = TM - first < GM ? TM - first : GM;
  const int in = lin - gid * group;
  *tm = first + in % gm;
  *tn = in / gm;
}

// MODE 0: requantised output; MODE 1: exact int64 accumulators sum_k (a - zp) * w_int.
template <bool A16, int TFMT, bool LPBQ, int MODE>
__global__ __launch_bounds__(kGemmThreads, 1) void qmm_gemm_kernel(const GemmArgs g) {
  using C = Cfg<A16, TFMT, LPBQ>;
  __shared__ __attribute__((aligned(16))) uint8_t arena[C::kArena];
  __shared__ uint32_t fix_list[kFixCap];
  __shared__ int fix_acc[A16 ? 1 : kFixCap];  // 8-bit acts: int32 accumulator of each listed output
  __shared__ int fix_cnt, unc_cnt;

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  int tm, tn;
  tile_of(blockIdx.x, g.TM, g.TN, &tm, &tn);
  const int rows_real = A16 ? kBM / 2 : kBM;
  const int cols_real = A16 ? kBN / 2 : kBN;
  const int m0 = tm * rows_real;
  const int n0 = tn * cols_real;
  const int M = g.M, K = g.K, KT = g.KT;
  const uint8_t *const act = g.act;
  const uint8_t *const btiles = g.tiles + static_cast<size_t>(tn) * KT * C::kTileB;
  const uint8_t *const ftiles = LPBQ ? g.lpbq + static_cast<size_t>(tn) * KT * C::kTileF : nullptr;
  if (t == 0) {
    fix_cnt = 0;
    unc_cnt = 0;
  }

  auto stage_a = [&](int st) { return arena + st * C::kStageBytes; };
  auto stage_b = [&](int st) { return arena + st * C::kStageBytes + kTileA; };
  auto stage_f = [&](int st) { return arena + st * C::kStageBytes + kTileA + C::kTileB; };

  // Issue the direct-to-LDS loads of k-tile kt into stage st (kLoads instructions per wave).
  auto issue = [&](int kt, int st) {
    uint8_t *la = stage_a(st);
#pragma unroll
    for (int j = 0; j < C::kLoadsA; ++j) {
      const int slot = j * 256 + t;  // 16-byte slot of the tile
      const void *src;
      if (!A16) {
        const int row = slot >> 3, phys = slot & 7;
        const int logical = phys ^ swz8(row);
        const int m = m0 + row < M ? m0 + row : M - 1;
        const int k = kt * kBK + 16 * logical < K ? kt * kBK + 16 * logical : K - 16;
        src = act + static_cast<size_t>(m) * K + k;
      } else {
        const int row = slot >> 4, phys = slot & 15;
        const int logical = phys ^ swz16(row);
        const int m = m0 + row < M ? m0 + row : M - 1;
        const int k = kt * kBK + 8 * logical < K ? kt * kBK + 8 * logical : K - 8;
        src = act + (static_cast<size_t>(m) * K + k) * 2;
      }
      load_lds16(src, la + (j * 256 + wave * 64) * 16);
    }
    const uint8_t *bsrc = btiles + static_cast<size_t>(kt) * C::kTileB;
    uint8_t *lb = stage_b(st);
#pragma unroll
    for (int j = 0; j < C::kLoadsB; ++j) load_lds16(bsrc + (j * 256 + t) * 16, lb + (j * 256 + wave * 64) * 16);
    if (LPBQ) {
      const uint8_t *fsrc = ftiles + static_cast<size_t>(kt) * C::kTileF;
      if (lane < 16) load_lds16(fsrc + (wave * 16 + lane) * 16, stage_f(st) + wave * 256);
    }
  };

  v16i acc[4][4];
  static_for<4>([&](auto i) { static_for<4>([&](auto j) { acc[i][j] = v16i{}; }); });

  constexpr int S = C::kStages;
#pragma unroll
  for (int p = 0; p < S - 1; ++p)
    if (p < KT) issue(p, p);

  const int g32 = lane >> 5;  // which 16-k half of a 32-k MFMA step this lane supplies
  for (int kt = 0; kt < KT; ++kt) {
    // tile kt has landed once at most (S-2) later tiles are still in flight
    if (S == 3 && kt + 1 < KT)
      wait_vmcnt<(S - 2) * C::kLoads>();
    else
      wait_vmcnt<0>();
    __syncthreads();
    if (kt + S - 1 < KT) issue(kt + S - 1, (kt + S - 1) % S);
    const int st = kt % S;
    const uint8_t *la = stage_a(st);
    const uint8_t *lb = stage_b(st);
    uint32_t fcol[4];
    if (LPBQ) {
      static_for<4>([&](auto nt) {
        const int col = wn * 128 + nt * 32 + (lane & 31);
        fcol[nt] = *reinterpret_cast<const uint32_t *>(stage_f(st) + col * 4);
      });
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int s16 = 2 * kk + g32;  // 16-k chunk index inside the 128-k tile
      v4i af[4], bf[4];
      if (!A16) {
        static_for<4>([&](auto mt) {
          const int row = wm * 128 + mt * 32 + (lane & 31);
          uint4 v = *reinterpret_cast<const uint4 *>(la + row * 128 + 16 * (s16 ^ swz8(row)));
          af[mt] = v4i{static_cast<int>(v.x ^ 0x80808080u), static_cast<int>(v.y ^ 0x80808080u),
                       static_cast<int>(v.z ^ 0x80808080u), static_cast<int>(v.w ^ 0x80808080u)};
        });
      } else {
        static_for<2>([&](auto mt) {
          const int row = wm * 64 + mt * 32 + (lane & 31);
          uint4 v0 = *reinterpret_cast<const uint4 *>(la + row * 256 + 16 * ((2 * s16) ^ swz16(row)));
          uint4 v1 = *reinterpret_cast<const uint4 *>(la + row * 256 + 16 * ((2 * s16 + 1) ^ swz16(row)));
          v0.x ^= 0x80808080u; v0.y ^= 0x80808080u; v0.z ^= 0x80808080u; v0.w ^= 0x80808080u;
          v1.x ^= 0x80808080u; v1.y ^= 0x80808080u; v1.z ^= 0x80808080u; v1.w ^= 0x80808080u;
          af[2 * mt] = v4i{static_cast<int>(perm(v0.y, v0.x, 0x07050301u)), static_cast<int>(perm(v0.w, v0.z, 0x07050301u)),
                           static_cast<int>(perm(v1.y, v1.x, 0x07050301u)), static_cast<int>(perm(v1.w, v1.z, 0x07050301u))};
          af[2 * mt + 1] = v4i{static_cast<int>(perm(v0.y, v0.x, 0x06040200u)), static_cast<int>(perm(v0.w, v0.z, 0x06040200u)),
                               static_cast<int>(perm(v1.y, v1.x, 0x06040200u)), static_cast<int>(perm(v1.w, v1.z, 0x06040200u))};
        });
      }
      static_for<4>([&](auto nt) {
        const int col = wn * 128 + nt * 32 + (lane & 31);
        if (TFMT == kTileI8) {
          const uint4 v = *reinterpret_cast<const uint4 *>(lb + col * 128 + 16 * (s16 ^ swz8(col)));
          bf[nt] = v4i{static_cast<int>(v.x), static_cast<int>(v.y), static_cast<int>(v.z), static_cast<int>(v.w)};
        } else {
          const uint2 v = *reinterpret_cast<const uint2 *>(lb + col * 64 + 8 * (s16 ^ swz_i4(col)));
          uint32_t f = 1;
          if (LPBQ) f = (fcol[nt] >> (8 * kk)) & 0xFFu;
          const uint32_t bias = (128u - 8u * f) * 0x01010101u;
          const uint32_t m4 = 0x0F0F0F0Fu;
          bf[nt] = v4i{static_cast<int>(widen4(v.x & m4, f, bias)), static_cast<int>(widen4(v.y & m4, f, bias)),
                       static_cast<int>(widen4((v.x >> 4) & m4, f, bias)),
                       static_cast<int>(widen4((v.y >> 4) & m4, f, bias))};
        }
      });
      static_for<4>([&](auto mt) {
        static_for<4>([&](auto nt) {
          acc[mt][nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[mt], bf[nt], acc[mt][nt], 0, 0, 0);
        });
      });
    }
  }
  // ---------------------------------------------------------------- epilogue
  // Straight from the accumulator registers: each lane requantises the 4 rows x 1 column
  // strips of its MFMA blocks, then the 4 lanes of a quad transpose their strips (DPP quad
  // broadcasts + byte permutes) so every lane stores 4 adjacent outputs of one row.
  auto push_fix = [&](int r, int c, int a) {
    const int slot = atomicAdd(&fix_cnt, 1);
    if (slot < kFixCap) {
      fix_list[slot] = (static_cast<uint32_t>(r) << 16) | static_cast<uint32_t>(c);
      if (!A16) fix_acc[slot] = a;
    }
  };
  const int q = lane & 3;
  const double qmaxd = static_cast<double>(g.out_qmax);
  if (!A16) {
    static_for<4>([&](auto nt) {
      const int cl = wn * 128 + nt * 32 + (lane & 31);  // column inside the tile
      const int n = n0 + cl;
      const bool nok = n < g.N;
      const int nn = nok ? n : 0;
      double alpha, beta, thr;
      if (MODE == 0) {
        alpha = g.alpha[nn];
        // zero-point correction folded into the offset: t = acc * alpha + (beta + corr * alpha)
        beta = fma(static_cast<double>(g.corr[nn]), alpha, g.beta[nn]);
        // |t - rint(t)| <= thr certifies the rounding; slack for |t| <= qmax + 2 folded in
        thr = 0.5 - g.margin[nn] - 0x1p-48 * (g.absb[nn] + 2.0 * fabs(g.corr[nn] * alpha) + qmaxd + 2.0);
      }
      static_for<4>([&](auto mt) {
        static_for<4>([&](auto jg) {
          const int R = wm * 128 + mt * 32 + 8 * jg + 4 * (lane >> 5);  // first of 4 rows
          int o[4];
          static_for<4>([&](auto jj) {
            constexpr int j = 4 * decltype(jg)::value + decltype(jj)::value;
            const int a = acc[mt][nt][j];
            if (MODE == 1) {
              if (nok && m0 + R + jj < M)
                reinterpret_cast<int64_t *>(g.out)[static_cast<size_t>(m0 + R + jj) * g.N + n] =
                    static_cast<int64_t>(a) + g.corr[nn];
              return;
            }
            const double tv = fma(static_cast<double>(a), alpha, beta);
            const double rd = rint(tv);
            int oi = static_cast<int>(rd);
            o[jj] = oi < 0 ? 0 : (oi > g.out_qmax ? g.out_qmax : oi);
            if (fabs(tv - rd) > thr && tv > -1.0 && tv < qmaxd + 1.0 && nok && m0 + R + jj < M) push_fix(R + jj, cl, a);
          });
          if (MODE == 1) return;
          if (!g.out16) {
            const uint32_t p = static_cast<uint32_t>(o[0]) | (static_cast<uint32_t>(o[1]) << 8) |
                               (static_cast<uint32_t>(o[2]) << 16) | (static_cast<uint32_t>(o[3]) << 24);
            const uint32_t x0 = __builtin_amdgcn_mov_dpp(p, 0x00, 0xF, 0xF, false);
            const uint32_t x1 = __builtin_amdgcn_mov_dpp(p, 0x55, 0xF, 0xF, false);
            const uint32_t x2 = __builtin_amdgcn_mov_dpp(p, 0xAA, 0xF, 0xF, false);
            const uint32_t x3 = __builtin_amdgcn_mov_dpp(p, 0xFF, 0xF, 0xF, false);
            const uint32_t sel = static_cast<uint32_t>(q) | (static_cast<uint32_t>(4 + q) << 8) | 0x0C0C0000u;
            const uint32_t w = perm(perm(x3, x2, sel), perm(x1, x0, sel), 0x05040100u);
            const int row = m0 + R + q, col = n0 + wn * 128 + nt * 32 + (lane & 28);
            if (row < M && col < g.N) *reinterpret_cast<uint32_t *>(static_cast<uint8_t *>(g.out) + static_cast<size_t>(row) * g.N + col) = w;
          } else {
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
              if (nok && m0 + R + jj < M) store_out(g.out, 1, static_cast<size_t>(m0 + R + jj) * g.N + n, o[jj]);
          }
        });
      });
    });
  } else {
    // 16-bit activations: real row tiles mt (32 rows), real column tiles c (32 columns);
    // acc[2mt + p][2c + s]: p = hi / lo' activation byte, s = weight code / rounding residue.
    static_for<2>([&](auto c) {
      const int cl = wn * 64 + c * 32 + (lane & 31);
      const int n = n0 + cl;
      const bool nok = n < g.N;
      const int nn = nok ? n : 0;
      double alpha = 0, alpha_m = 0, beta = 0, margin = 0, absb = 0;
      const int64_t csum = MODE == 1 ? g.colsum[nn] * static_cast<int64_t>(128 + 32768 - g.act_zp) : 0;
      if (MODE == 0) {
        alpha = g.alpha[nn];
        alpha_m = alpha * static_cast<double>(g.mant[nn]);
        beta = fma(static_cast<double>(g.corr[nn]), alpha, g.beta[nn]);
        margin = g.margin[nn];
        absb = g.absb[nn] + 2.0 * fabs(static_cast<double>(g.corr[nn]) * alpha);
      }
      static_for<2>([&](auto mt) {
        static_for<4>([&](auto jg) {
          const int R = wm * 64 + mt * 32 + 8 * jg + 4 * (lane >> 5);
          int o[4];
          static_for<4>([&](auto jj) {
            constexpr int j = 4 * decltype(jg)::value + decltype(jj)::value;
            const int hq = acc[2 * mt][2 * c][j], lq = acc[2 * mt + 1][2 * c][j];
            const int hr = acc[2 * mt][2 * c + 1][j], lr = acc[2 * mt + 1][2 * c + 1][j];
            if (MODE == 1) {
              if (nok && m0 + R + jj < M)
                reinterpret_cast<int64_t *>(g.out)[static_cast<size_t>(m0 + R + jj) * g.N + n] =
                    256 * static_cast<int64_t>(hq) + lq + csum;
              return;
            }
            // exact: X = sum (a-32768)' q, Y = sum (a-32768)' r as float64 integers
            const double X = fma(static_cast<double>(hq), 256.0, static_cast<double>(lq));
            const double Y = fma(static_cast<double>(hr), 256.0, static_cast<double>(lr));
            const double u = X * alpha_m;
            const double tv = fma(Y, alpha, u + beta);
            const double rd = rint(tv);
            int oi = static_cast<int>(rd);
            o[jj] = oi < 0 ? 0 : (oi > g.out_qmax ? g.out_qmax : oi);
            const double slack = margin + 0x1p-48 * (fabs(u) + fabs(tv) + absb);
            if (fabs(tv - rd) > 0.5 - slack && tv > -1.0 && tv < qmaxd + 1.0 && nok && m0 + R + jj < M) push_fix(R + jj, cl, 0);
          });
          if (MODE == 1) return;
          if (g.out16) {
            const uint32_t P0 = static_cast<uint32_t>(o[0]) | (static_cast<uint32_t>(o[1]) << 16);
            const uint32_t P1 = static_cast<uint32_t>(o[2]) | (static_cast<uint32_t>(o[3]) << 16);
            // every lane fetches both strips of every quad lane, then keeps the half it stores
            const uint32_t a0 = __builtin_amdgcn_mov_dpp(P0, 0x00, 0xF, 0xF, false);
            const uint32_t a1 = __builtin_amdgcn_mov_dpp(P0, 0x55, 0xF, 0xF, false);
            const uint32_t a2 = __builtin_amdgcn_mov_dpp(P0, 0xAA, 0xF, 0xF, false);
            const uint32_t a3 = __builtin_amdgcn_mov_dpp(P0, 0xFF, 0xF, 0xF, false);
            const uint32_t b0 = __builtin_amdgcn_mov_dpp(P1, 0x00, 0xF, 0xF, false);
            const uint32_t b1 = __builtin_amdgcn_mov_dpp(P1, 0x55, 0xF, 0xF, false);
            const uint32_t b2 = __builtin_amdgcn_mov_dpp(P1, 0xAA, 0xF, 0xF, false);
            const uint32_t b3 = __builtin_amdgcn_mov_dpp(P1, 0xFF, 0xF, 0xF, false);
            const uint32_t sel = (q & 1) ? 0x07060302u : 0x05040100u;
            const uint32_t lo_w = perm(a1, a0, sel), hi_w = perm(a3, a2, sel);
            const uint32_t lo_w2 = perm(b1, b0, sel), hi_w2 = perm(b3, b2, sel);
            const uint2 w = q < 2 ? make_uint2(lo_w, hi_w) : make_uint2(lo_w2, hi_w2);
            const int row = m0 + R + q, col = n0 + wn * 64 + c * 32 + (lane & 28);
            if (row < M && col < g.N)
              *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(g.out) + static_cast<size_t>(row) * g.N + col) = w;
          } else {
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
              if (nok && m0 + R + jj < M) store_out(g.out, 0, static_cast<size_t>(m0 + R + jj) * g.N + n, o[jj]);
          }
        });
      });
    });
  }
  if (MODE == 1) return;
  __syncthreads();  // provisional outputs of flagged elements are stored before the fixup rewrites them


  // ---------------------------------------------------------------- exact fixup
  const int cnt = fix_cnt;
  if (cnt == 0) return;
  const bool full = cnt > kFixCap;  // list overflowed: recompute the whole tile exactly
  int total = full ? rows_real * cols_real : cnt;
  if (!A16 && !full) {
    // 8-bit activations, exact in integers.  With s32 = M * 2^E the oracle's weight is
    // fl32(w * s32) = 2^E * (w * M + r) for an integer residue r, so the exact dot product is
    // 2^E * D with D = M * (acc + corr) + sum_k (a_k - 128) r_k + (128 - zp) * sum_k r_k.
    // All 256 threads form the residue sum Y = sum_k (a_k - 128) r_k of a batch of listed
    // outputs at once (one K chunk of 16 per thread per output), reduced with integer LDS
    // atomics (order-independent).  Only outputs whose exact value is still within the oracle's
    // own float64 noise of a rounding boundary are handed to the float64 emulation below.
    int *ysum = reinterpret_cast<int *>(arena);                  // [kFixCap]
    uint32_t *unc = reinterpret_cast<uint32_t *>(arena) + kFixCap;  // [kFixCap]
    for (int e = t; e < cnt; e += kGemmThreads) ysum[e] = 0;
    __syncthreads();
    constexpr int EB = 4;  // listed outputs whose loads are in flight together
    const int KC = K / 16;
    for (int e0 = 0; e0 < cnt; e0 += EB) {
      // the loop bound is uniform so that every lane of a wave takes part in the reduction
      for (int kc0 = 0; kc0 < KC; kc0 += kGemmThreads) {
        const bool kin = kc0 + t < KC;
        const int k = kin ? (kc0 + t) * 16 : 0;
        int w[EB][16];
        uint4 av[EB];
        int nloc[EB];
#pragma unroll
        for (int i = 0; i < EB; ++i) {
          const int e = e0 + i < cnt ? e0 + i : cnt - 1;
          const uint32_t v = fix_list[e];
          const int m = m0 + static_cast<int>(v >> 16), n = n0 + static_cast<int>(v & 0xFFFFu);
          nloc[i] = n;
          load_w16<TFMT, LPBQ>(g, n, k, w[i]);
          av[i] = *reinterpret_cast<const uint4 *>(act + static_cast<size_t>(m) * K + k);
        }
#pragma unroll
        for (int i = 0; i < EB; ++i) {
          const int n = nloc[i];
          const float sc = g.s32[n];
          const double ip = g.inv_pow2e[n];
          const int mant = static_cast<int>(g.mant[n]);
          int y = 0;
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int a = static_cast<int>(reinterpret_cast<const uint8_t *>(&av[i])[j]) - 128;
            const float wd = static_cast<float>(w[i][j]) * sc;
            const int wp = static_cast<int>(static_cast<double>(wd) * ip);  // exact integer
            y += a * (wp - w[i][j] * mant);
          }
          if (!kin) y = 0;
#pragma unroll
          for (int off = 32; off >= 1; off >>= 1) y += __shfl_xor(y, off, 64);
          if (lane == 0 && e0 + i < cnt) atomicAdd(&ysum[e0 + i], y);
        }
      }
    }
    __syncthreads();
    for (int e = t; e < cnt; e += kGemmThreads) {
      const uint32_t v = fix_list[e];
      const int m = m0 + static_cast<int>(v >> 16), n = n0 + static_cast<int>(v & 0xFFFFu);
      const int64_t D = g.mant[n] * (static_cast<int64_t>(fix_acc[e]) + g.corr[n]) + ysum[e] +
                        static_cast<int64_t>(128 - g.act_zp) * g.colsum_r[n];
      const double u = static_cast<double>(D) * g.alpha_e[n];
      const double tv = u + g.beta[n];
      const double rd = rint(tv);
      const double slack = g.margin_exact[n] + 0x1p-48 * (fabs(u) + fabs(tv) + g.absb[n]);
      if (fabs(tv - rd) > 0.5 - slack) {
        unc[atomicAdd(&unc_cnt, 1)] = v;
      } else {
        const int oi = static_cast<int>(rd);
        store_out(g.out, g.out16, static_cast<size_t>(m) * g.N + n, oi < 0 ? 0 : (oi > g.out_qmax ? g.out_qmax : oi));
      }
    }
    __syncthreads();
    total = unc_cnt;
    for (int e = wave; e < total; e += kGemmThreads / 64) {
      const uint32_t v = unc[e];
      fixup_one<A16, TFMT, LPBQ>(g, m0 + static_cast<int>(v >> 16), n0 + static_cast<int>(v & 0xFFFFu), lane);
    }
    return;
  }
  for (int e = wave; e < total; e += kGemmThreads / 64) {
    int r, c;
    if (full) {
      r = e / cols_real;
      c = e % cols_real;
    } else {
      const uint32_t v = fix_list[e];
      r = static_cast<int>(v >> 16);
      c = static_cast<int>(v & 0xFFFFu);
    }
    const int m = m0 + r, n = n0 + c;
    if (m >= M || n >= g.N) continue;
    fixup_one<A16, TFMT, LPBQ>(g, m, n, lane);
  }
}

template <bool A16, int TFMT, bool LPBQ, int MODE>
qh_status launch(const GemmArgs &g, hipStream_t stream) {
  dim3 grid(g.TM * g.TN);
  hipLaunchKernelGGL((qmm_gemm_kernel<A16, TFMT, LPBQ, MODE>), grid, dim3(kGemmThreads), 0, stream, g);
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
  g.lpbq = D.lpbq_tiles;
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
  g.inv_pow2e = D.inv_pow2e;
  g.margin_exact = D.margin_exact;
  g.s32 = D.s32;
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
  const bool lpbq_regs = sh.wfmt == QH_WEIGHT_I4_LPBQ && !a16;
  if (!a16) {
    if (sh.tile_fmt == kTileI8) return launch<false, kTileI8, false, MODE>(g, stream);
    if (lpbq_regs) return launch<false, kTileI4, true, MODE>(g, stream);
    return launch<false, kTileI4, false, MODE>(g, stream);
  }
  if (sh.tile_fmt == kTileI8) return launch<true, kTileI8, false, MODE>(g, stream);
  return launch<true, kTileI4, false, MODE>(g, stream);
}

}  // namespace

qh_status launch_qmm_gemm(const qh_qmm_prepared *p, int m, const void *act, void *out, hipStream_t stream) {
  return dispatch<0>(p, m, act, out, stream);
}

qh_status launch_qmm_accumulate(const qh_qmm_prepared *p, int m, const void *act, int64_t *acc, hipStream_t stream) {
  return dispatch<1>(p, m, act, acc, stream);
}

}  // namespace qh
