// Quantized GEMM on gfx950 i8 MFMA (v_mfma_i32_32x32x32_i8), bit-exact to the reference's
// float-derived requantisation.
//
// Workgroup: 256 threads (4 waves in a 2x2 grid), tile 256 activation-operand rows x 256
// weight-operand columns, K staged 128 bytes at a time through double-buffered LDS
// (2 x 64 KiB).  Each wave owns a 128x128 sub-tile = 4x4 MFMA 32x32 blocks.
//
// Operand preparation happens on the global->LDS path:
//   * 8-bit activations are shifted to signed (a - 128) by an XOR with 0x80;
//   * 16-bit activations a - 32768 = 256*hi + lo' + 128 are split into two int8 planes that
//     occupy adjacent operand rows (hi, lo'), so each MFMA row pair holds one activation row;
//   * int4 weights (offset-binary nibbles) are widened to int8 in registers, and LPBQ
//     block scales are applied there too: (u*f + 128 - 8f) ^ 0x80 per byte is the two's
//     complement of (u - 8) * f with no carry between bytes.
// Epilogue: the accumulators are staged through the (then idle) LDS in two halves, so each
// thread requantises one output channel down a column of rows with coalesced stores.  The
// exact integer dot product S (int32 MFMA accumulators, combined in int64 for 16-bit
// activations) becomes t = S*alpha + beta in float64; rint(t) is certain unless t lies within
// the per-channel margin of a rounding boundary, in which case the element is queued in LDS
// and recomputed after the tile by a wave-cooperative float64 dot product that forms every
// term exactly as the reference oracle does
// (scripts/generate_qnn_matmul_python_cases.py:472-481).

#include <type_traits>
#include <utility>

#include "qmm_internal.h"

namespace qh {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

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
  const int64_t *corr, *mant, *colsum;
  const float *s32;
  int M, N, K, KT, lpbq_nb, lpbq_shift;
  int act_zp, out_zp, out_qmax, out16;
  double sA, sO;
};

// LDS arena: two pipeline stages of (A tile, B tile), 32 KiB each; the epilogue reuses it to
// stage half of the accumulator tile (128 rows x 256 cols int32, row stride padded to 260).
constexpr int kStageU4 = kBM * kBK / 16;      // uint4 per operand tile
constexpr int kEpiStride = 260;               // int32 per staged accumulator row (A8)
constexpr int kArenaU4 = 4 * kStageU4 > 128 * kEpiStride / 4 ? 4 * kStageU4 : 128 * kEpiStride / 4;

// Row-dependent XOR swizzle of the eight 16-byte chunks of a 128-byte LDS row: conflict-free
// for the MFMA fragment reads (32 consecutive rows, same logical chunk) whether the LDS serves
// 8 or 16 lanes per cycle.
__device__ __forceinline__ int swz(int row) { return ((row >> 1) ^ (row << 2)) & 7; }

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
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

// Loads 16 consecutive weight codes (k .. k+15, k % 16 == 0) of operand column cb.
template <int TFMT, bool LPBQ>
__device__ __forceinline__ void load_w16(const GemmArgs g, int cb, int k, int (&w)[16]) {
  const size_t tile = static_cast<size_t>(cb / kBN) * g.KT + k / kBK;
  if (TFMT == kTileI8) {
    const int8_t *p = reinterpret_cast<const int8_t *>(g.tiles) + tile * (kBN * kBK) + (cb % kBN) * kBK + (k % kBK);
    uint4 v = *reinterpret_cast<const uint4 *>(p);
    const int8_t *b = reinterpret_cast<const int8_t *>(&v);
#pragma unroll
    for (int j = 0; j < 16; ++j) w[j] = b[j];
  } else {
    const uint8_t *p = g.tiles + tile * (kBN * kBK / 2) + (cb % kBN) * (kBK / 2) + ((k % kBK) / 16) * 8;
    uint2 v = *reinterpret_cast<const uint2 *>(p);
    const uint8_t *b = reinterpret_cast<const uint8_t *>(&v);
    int f = 1;
    if (LPBQ) f = g.lpbq[static_cast<size_t>(cb) * g.lpbq_nb + (k >> g.lpbq_shift)];
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
  for (int kc = lane; kc < g.K / 16; kc += 64) {
    const int k = kc * 16;
    int w[16];
    load_w16<TFMT, LPBQ>(g, cb, k, w);
    int a[16];
    if (A16) {
      const uint16_t *ap = reinterpret_cast<const uint16_t *>(g.act) + static_cast<size_t>(m) * g.K + k;
      uint4 v0 = reinterpret_cast<const uint4 *>(ap)[0], v1 = reinterpret_cast<const uint4 *>(ap)[1];
      const uint16_t *h0 = reinterpret_cast<const uint16_t *>(&v0), *h1 = reinterpret_cast<const uint16_t *>(&v1);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        a[j] = h0[j];
        a[j + 8] = h1[j];
      }
    } else {
      uint4 v = *reinterpret_cast<const uint4 *>(g.act + static_cast<size_t>(m) * g.K + k);
      const uint8_t *b = reinterpret_cast<const uint8_t *>(&v);
#pragma unroll
      for (int j = 0; j < 16; ++j) a[j] = b[j];
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float wd = static_cast<float>(w[j]) * sc;
      const double xd = static_cast<double>(a[j] - g.act_zp) * g.sA;
      s = fma(xd, static_cast<double>(wd), s);
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

// Requantise one exact integer dot product.  Returns the provisional output and whether the
// rounding could differ from the oracle's (needs the exact fixup).
__device__ __forceinline__ int requant(double S, double alpha, double beta, double margin, double absb, int qmax,
                                       bool *ambiguous) {
  const double t = fma(S, alpha, beta);
  const double fl = floor(t);
  const double slack = margin + 0x1p-48 * (fabs(t) + absb);
  const bool near_tie = fabs((t - fl) - 0.5) <= slack;
  const double lo = fmin(fmax(fl, 0.0), static_cast<double>(qmax));
  const double hi = fmin(fmax(fl + 1.0, 0.0), static_cast<double>(qmax));
  *ambiguous = near_tie && (lo != hi);
  const double o = fmin(fmax(rint(t), 0.0), static_cast<double>(qmax));
  return static_cast<int>(o);
}

// MODE 0: requantised output; MODE 1: exact int64 accumulators sum_k (a - zp) * w_int.
template <bool A16, int TFMT, bool LPBQ, int MODE>
__global__ __launch_bounds__(kGemmThreads, 1) void qmm_gemm_kernel(const GemmArgs g) {
  __shared__ uint4 arena[kArenaU4];
  __shared__ uint32_t fix_list[kFixCap];
  __shared__ int fix_cnt;

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int rows_real = A16 ? kBM / 2 : kBM;
  const int cols_real = A16 ? kBN / 2 : kBN;
  const int m0 = blockIdx.y * rows_real;
  const int c0 = blockIdx.x * kBN;
  const int n0 = blockIdx.x * cols_real;
  const int M = g.M, K = g.K, KT = g.KT;
  const uint8_t *const act = g.act;
  const uint8_t *const tiles_base = g.tiles + static_cast<size_t>(blockIdx.x) * KT * (TFMT == kTileI8 ? kBN * kBK : kBN * kBK / 2);
  if (t == 0) fix_cnt = 0;

  constexpr int NB = TFMT == kTileI8 ? 8 : 4;
  uint4 ra[8];
  uint4 rb[NB];
  uint32_t rf[NB];

  auto lds_a = [&](int st) { return arena + (2 * st) * kStageU4; };
  auto lds_b = [&](int st) { return arena + (2 * st + 1) * kStageU4; };

  auto load_a = [&](int kt) {
    if (!A16) {
      const int c = t & 7, rr = t >> 3;
      const int k = kt * kBK + 16 * c;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int row = m0 + i * 32 + rr;
        if (row < M && k < K)
          ra[i] = *reinterpret_cast<const uint4 *>(act + static_cast<size_t>(row) * K + k);
        else
          ra[i] = make_uint4(0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u);
      }
    } else {
      const int c = t & 15, rr = t >> 4;
      const int k = kt * kBK + 8 * c;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int row = m0 + i * 16 + rr;
        if (row < M && k < K)
          ra[i] = *reinterpret_cast<const uint4 *>(act + (static_cast<size_t>(row) * K + k) * 2);
        else
          ra[i] = make_uint4(0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u);
      }
    }
  };
  auto store_a = [&](int st) {
    uint4 *la = lds_a(st);
    if (!A16) {
      const int c = t & 7, rr = t >> 3;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int row = i * 32 + rr;
        uint4 v = ra[i];
        v.x ^= 0x80808080u;
        v.y ^= 0x80808080u;
        v.z ^= 0x80808080u;
        v.w ^= 0x80808080u;
        la[row * 8 + (c ^ swz(row))] = v;
      }
    } else {
      const int c = t & 15, rr = t >> 4;
      uint2 *l2 = reinterpret_cast<uint2 *>(la);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint4 v = ra[i];
        v.x ^= 0x80808080u;
        v.y ^= 0x80808080u;
        v.z ^= 0x80808080u;
        v.w ^= 0x80808080u;
        const uint2 hi = make_uint2(perm(v.y, v.x, 0x07050301u), perm(v.w, v.z, 0x07050301u));
        const uint2 lo = make_uint2(perm(v.y, v.x, 0x06040200u), perm(v.w, v.z, 0x06040200u));
        const int rh = 2 * (i * 16 + rr), rl = rh + 1;
        const int ch = c >> 1, half = c & 1;
        l2[rh * 16 + 2 * (ch ^ swz(rh)) + half] = hi;
        l2[rl * 16 + 2 * (ch ^ swz(rl)) + half] = lo;
      }
    }
  };
  auto load_b = [&](int kt) {
    if (TFMT == kTileI8) {
      const uint4 *base = reinterpret_cast<const uint4 *>(tiles_base + static_cast<size_t>(kt) * (kBN * kBK));
#pragma unroll
      for (int i = 0; i < 8; ++i) rb[i] = base[i * 256 + t];
    } else {
      const uint4 *base = reinterpret_cast<const uint4 *>(tiles_base + static_cast<size_t>(kt) * (kBN * kBK / 2));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        rb[i] = base[i * 256 + t];
        if (LPBQ) {
          const int col = c0 + i * 64 + (t >> 2);
          const int k = kt * kBK + 32 * (t & 3);
          rf[i] = g.lpbq[static_cast<size_t>(col) * g.lpbq_nb + (k >> g.lpbq_shift)];
        } else {
          rf[i] = 1;
        }
      }
    }
  };
  auto store_b = [&](int st) {
    uint4 *lb = lds_b(st);
    if (TFMT == kTileI8) {
      const int c = t & 7, cc = t >> 3;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int col = i * 32 + cc;
        lb[col * 8 + (c ^ swz(col))] = rb[i];
      }
    } else {
      const int c4 = t & 3, cc = t >> 2;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int col = i * 64 + cc;
        const uint32_t f = rf[i];
        const uint32_t bias = (128u - 8u * f) * 0x01010101u;
        const uint4 v = rb[i];
        const uint32_t m4 = 0x0F0F0F0Fu;
        uint4 g0, g1;
        g0.x = widen4(v.x & m4, f, bias);
        g0.y = widen4(v.y & m4, f, bias);
        g0.z = widen4((v.x >> 4) & m4, f, bias);
        g0.w = widen4((v.y >> 4) & m4, f, bias);
        g1.x = widen4(v.z & m4, f, bias);
        g1.y = widen4(v.w & m4, f, bias);
        g1.z = widen4((v.z >> 4) & m4, f, bias);
        g1.w = widen4((v.w >> 4) & m4, f, bias);
        const int s = swz(col);
        lb[col * 8 + ((2 * c4) ^ s)] = g0;
        lb[col * 8 + ((2 * c4 + 1) ^ s)] = g1;
      }
    }
  };

  v16i acc[4][4];
  static_for<4>([&](auto i) { static_for<4>([&](auto j) { acc[i][j] = v16i{}; }); });

  load_a(0);
  load_b(0);
  store_a(0);
  store_b(0);
  __syncthreads();

  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < KT;
    if (more) {
      load_a(kt + 1);
      load_b(kt + 1);
    }
    const uint4 *la = lds_a(cur);
    const uint4 *lb = lds_b(cur);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int ch = 2 * kk + (lane >> 5);
      v4i af[4], bf[4];
      static_for<4>([&](auto mt) {
        const int row = wm * 128 + mt * 32 + (lane & 31);
        const uint4 v = la[row * 8 + (ch ^ swz(row))];
        af[mt] = v4i{static_cast<int>(v.x), static_cast<int>(v.y), static_cast<int>(v.z), static_cast<int>(v.w)};
      });
      static_for<4>([&](auto nt) {
        const int col = wn * 128 + nt * 32 + (lane & 31);
        const uint4 v = lb[col * 8 + (ch ^ swz(col))];
        bf[nt] = v4i{static_cast<int>(v.x), static_cast<int>(v.y), static_cast<int>(v.z), static_cast<int>(v.w)};
      });
      static_for<4>([&](auto mt) {
        static_for<4>([&](auto nt) {
          acc[mt][nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[mt], bf[nt], acc[mt][nt], 0, 0, 0);
        });
      });
    }
    if (more) {
      store_a(cur ^ 1);
      store_b(cur ^ 1);
    }
    __syncthreads();
  }

  // ---------------------------------------------------------------- epilogue
  int32_t *stage = reinterpret_cast<int32_t *>(arena);
  static_for<2>([&](auto h) {
    // 1) this wave's MFMA blocks mt = 2h, 2h+1 -> LDS
    static_for<2>([&](auto mh) {
      constexpr int mt = 2 * decltype(h)::value + decltype(mh)::value;
      static_for<4>([&](auto nt) {
        static_for<16>([&](auto j) {
          const int qrow = mh * 32 + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);  // 0..63 within the half
          const int col = nt * 32 + (lane & 31);
          const int v = acc[mt][nt][j()];
          if (!A16) {
            stage[(wm * 64 + qrow) * kEpiStride + wn * 128 + col] = v;
          } else {
            // real row wm*32 + qrow/2, real column wn*64 + (nt/2)*32 + lane%32,
            // component (column plane q|r) * 2 + (row plane hi|lo)
            const int rr = wm * 32 + (qrow >> 1);
            const int rc = wn * 64 + (nt >> 1) * 32 + (lane & 31);
            const int comp = (nt & 1) * 2 + (qrow & 1);
            stage[(rr * 128 + rc) * 4 + comp] = v;
          }
        });
      });
    });
    __syncthreads();
    // 2) requantise: one output channel per thread
    if (!A16) {
      const int n = n0 + t;
      if (n < g.N) {
        double alpha = 0, beta = 0, margin = 0, absb = 0;
        if (MODE == 0) {
          alpha = g.alpha[n];
          beta = g.beta[n];
          margin = g.margin[n];
          absb = g.absb[n];
        }
        const int64_t corr = g.corr[n];
        for (int r = 0; r < 128; ++r) {
          const int rl = (r >> 6) * 128 + 64 * h + (r & 63);
          const int m = m0 + rl;
          if (m >= M) continue;
          const int64_t S = static_cast<int64_t>(stage[r * kEpiStride + t]) + corr;
          const size_t idx = static_cast<size_t>(m) * g.N + n;
          if (MODE == 1) {
            reinterpret_cast<int64_t *>(g.out)[idx] = S;
            continue;
          }
          bool amb;
          const int o = requant(static_cast<double>(S), alpha, beta, margin, absb, g.out_qmax, &amb);
          if (amb) {
            const int slot = atomicAdd(&fix_cnt, 1);
            if (slot < kFixCap) fix_list[slot] = (static_cast<uint32_t>(rl) << 16) | static_cast<uint32_t>(t);
          } else {
            store_out(g.out, g.out16, idx, o);
          }
        }
      }
    } else {
      const int rc = t & 127, r0 = t >> 7;
      const int n = n0 + rc;
      if (n < g.N) {
        double alpha = 0, beta = 0, margin = 0, absb = 0;
        if (MODE == 0) {
          alpha = g.alpha[n];
          beta = g.beta[n];
          margin = g.margin[n];
          absb = g.absb[n];
        }
        const int64_t corr = g.corr[n], Mn = g.mant[n];
        const int64_t csum = MODE == 1 ? g.colsum[n] * static_cast<int64_t>(128 + 32768 - g.act_zp) : 0;
        for (int rr = r0; rr < 64; rr += 2) {
          const int rl = (rr >> 5) * 64 + 32 * h + (rr & 31);
          const int m = m0 + rl;
          if (m >= M) continue;
          const int4 v = *reinterpret_cast<const int4 *>(&stage[(rr * 128 + rc) * 4]);
          // v.x = hi*q, v.y = lo*q, v.z = hi*r, v.w = lo*r
          const size_t idx = static_cast<size_t>(m) * g.N + n;
          if (MODE == 1) {
            reinterpret_cast<int64_t *>(g.out)[idx] = 256 * static_cast<int64_t>(v.x) + v.y + csum;
            continue;
          }
          const int64_t S = 256 * (Mn * v.x + v.z) + Mn * v.y + v.w + corr;
          bool amb;
          const int o = requant(static_cast<double>(S), alpha, beta, margin, absb, g.out_qmax, &amb);
          if (amb) {
            const int slot = atomicAdd(&fix_cnt, 1);
            if (slot < kFixCap) fix_list[slot] = (static_cast<uint32_t>(rl) << 16) | static_cast<uint32_t>(rc);
          } else {
            store_out(g.out, g.out16, idx, o);
          }
        }
      }
    }
    __syncthreads();
  });
  if (MODE == 1) return;

  // ---------------------------------------------------------------- exact fixup
  const int cnt = fix_cnt;
  if (cnt == 0) return;
  const bool full = cnt > kFixCap;  // list overflowed: recompute the whole tile exactly
  const int total = full ? rows_real * cols_real : cnt;
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
qh_status launch(const GemmArgs &g, dim3 grid, hipStream_t stream) {
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
  g.s32 = D.s32;
  g.M = m;
  g.N = sh.N;
  g.K = sh.K;
  g.KT = sh.Kp / kBK;
  g.lpbq_nb = sh.lpbq_block ? sh.Kp / sh.lpbq_block : 0;
  g.lpbq_shift = sh.lpbq_block == 64 ? 6 : 5;
  g.act_zp = sh.act_zp;
  g.out_zp = sh.out_zp;
  g.out_qmax = (1 << sh.out_bits) - 1;
  g.out16 = sh.out_bits == 16;
  g.sA = sh.act_scale;
  g.sO = sh.out_scale;
  const bool a16 = sh.act_bits == 16;
  const int rows_real = a16 ? kBM / 2 : kBM;
  dim3 grid(sh.ncols_op / kBN, (m + rows_real - 1) / rows_real);
  if (grid.y > 65535) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "M=%d too large for one launch", m);
  const bool lpbq_regs = sh.wfmt == QH_WEIGHT_I4_LPBQ && !a16;
  if (!a16) {
    if (sh.tile_fmt == kTileI8) return launch<false, kTileI8, false, MODE>(g, grid, stream);
    if (lpbq_regs) return launch<false, kTileI4, true, MODE>(g, grid, stream);
    return launch<false, kTileI4, false, MODE>(g, grid, stream);
  }
  if (sh.tile_fmt == kTileI8) return launch<true, kTileI8, false, MODE>(g, grid, stream);
  return launch<true, kTileI4, false, MODE>(g, grid, stream);
}

}  // namespace

qh_status launch_qmm_gemm(const qh_qmm_prepared *p, int m, const void *act, void *out, hipStream_t stream) {
  return dispatch<0>(p, m, act, out, stream);
}

qh_status launch_qmm_accumulate(const qh_qmm_prepared *p, int m, const void *act, int64_t *acc, hipStream_t stream) {
  return dispatch<1>(p, m, act, acc, stream);
}

}  // namespace qh
