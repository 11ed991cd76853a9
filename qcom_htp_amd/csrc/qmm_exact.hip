// Exact integer GEMM on gfx950 i8 MFMA (v_mfma_i32_32x32x32_i8): int64 sums
//
//     D[m][n] = sum_p sum_g  mult_p[g][n] * sum_{k in g} (a[m][k] - zp) * w_p[n][k]
//             + ones * sum_k (a[m][k] - zp)                               (exact, int64)
//
// over one or two int8 weight planes w_p (stored in the GEMM tile layout) with integer
// multipliers per (plane, 64-k group, channel), and an optional all-ones plane.  It serves the
// weight schemas whose exact dot product is not a single int8 product times one per-channel
// constant, and the reference's integer contracts:
//   * per-group (K64) scales (generate_qnn_matmul_python_cases.py:392-423): with
//     s_g = M_g 2^E_g (M_g a 24-bit integer) the oracle's float32 weight fl32(q s_g) is
//     2^E_g (q M_g + r) for a small integer residue r, so with E_min = min_g E_g and
//     d_g = E_g - E_min the dot product is exactly 2^E_min D for planes q (multiplier
//     M_g 2^d_g) and r (multiplier 2^d_g);
//   * int16 weights as two byte planes (docs/w16a16_is_two_w8a16.md:13-45): q16 = 256 hi +
//     (lo - 128) + 128, planes hi (x 256) and lo - 128 (x 1) plus 128 x the all-ones plane;
//   * the integer contracts (gen_quant_chain.py:963-996, HmxU8I4ToU8MatMulOp.cpp:210-233,
//     HmxU16I4ToU16MatMulOp.cpp:514-568) on the exact accumulator of any prepared weight.
// Activations enter the MFMA shifted to int8: a - 128 (8-bit), or 256 hi + lo' with
// a - 32896 = 256 hi + lo' (16-bit; two MFMAs per product); the shift times the plane column
// sums is a per-channel constant added at the end.  The int32 MFMA sums are moved into the
// int64 accumulators every 64 k (|partial| < 2^30).
//
// Workgroup: 256 threads = 4 waves over a 64 x 64 output tile, one 32 x 32 block per wave;
// fragments come straight from global memory (L2) into registers, one 32-k step ahead.
// Requantisation (per-group): t = D alpha_e + beta in float64 is certain unless t lies within
// the oracle's own float64 noise of a rounding boundary; those outputs are listed and
// recomputed as the oracle forms its dot product (float64 products of fl64((a - zp) sA) and
// fl32(q s_g)).

#include <type_traits>
#include <utility>

#include "qmm_internal.h"

namespace qh {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kExThreads = 256;
constexpr int kExTile = 64;
constexpr int kExFixCap = 512;

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// Operand column of plane p, channel n in the tile layout (planes interleaved by 32 channels).
__device__ __forceinline__ int plane_col(int p, int n, int lp) { return (n >> 5) * (32 * lp) + p * 32 + (n & 31); }

__device__ __forceinline__ uint4 load_w16(const ExactArgs &g, int c, int k) {
  const size_t tile = static_cast<size_t>(c / kBN) * g.KT + k / kBK;
  return *reinterpret_cast<const uint4 *>(g.tiles + tile * (kBN * kBK) + tile_off_i8(c % kBN, k));
}

__device__ __forceinline__ void store_out(const ExactArgs &g, size_t idx, int v) {
  if (g.out16)
    static_cast<uint16_t *>(g.out)[idx] = static_cast<uint16_t>(v);
  else
    static_cast<uint8_t *>(g.out)[idx] = static_cast<uint8_t>(v);
}

// The reference's integer contracts on the exact accumulator D = sum_k (a - zp) w.
// bias: bias_q[n] (0 without a bias operand), read once per column before the k loop.
template <int CT>
__device__ __forceinline__ int contract_ct(const ExactArgs &g, long long D, long long bias) {
  const long long qmax = g.out_qmax;
  if constexpr (CT == QH_CONTRACT_CLIP_I32) {  // int32 arithmetic of the reference (wraps modulo 2^32)
    const int v = static_cast<int>(static_cast<unsigned int>(static_cast<unsigned long long>(D + bias)));
    return v < 0 ? 0 : (v > qmax ? static_cast<int>(qmax) : v);
  } else if constexpr (CT == QH_CONTRACT_CLIP_I64) {
    const long long v = D + bias;
    return static_cast<int>(v < 0 ? 0 : (v > qmax ? qmax : v));
  } else if constexpr (CT == QH_CONTRACT_FLOOR256_DIV_RINT || CT == QH_CONTRACT_DIV_RINT) {
    if (CT == QH_CONTRACT_FLOOR256_DIV_RINT) D = (D >> 8) * 256;  // floor division (shift rounds to -inf)
    const double y = static_cast<double>(D) / static_cast<double>(g.divisor);
    const double o = rint(y + static_cast<double>(g.out_zp));
    return static_cast<int>(fmin(fmax(o, 0.0), static_cast<double>(qmax)));
  } else if constexpr (CT == QH_CONTRACT_ROUND_DIV) {
    const long long d = g.divisor, h = d / 2;
    const long long q = D >= 0 ? (D + h) / d : -((-D + h) / d);
    const long long v = q + g.out_zp;
    return static_cast<int>(v < 0 ? 0 : (v > qmax ? qmax : v));
  } else {  // QH_CONTRACT_U8_DRAIN: (acc + bias) * s / 512 in float64, truncated, + b >> 7
    const uint32_t pk = static_cast<uint32_t>(g.divisor);
    const uint32_t e = (pk >> 10) & 31u, f = pk & 1023u;
    const double mag = e == 0 ? ldexp(static_cast<double>(f), -24) : ldexp(static_cast<double>(1024u + f), static_cast<int>(e) - 25);
    const double s = (pk & 0x8000u) ? -mag : mag;
    const long long drain = D + bias;
    const long long v = static_cast<long long>(trunc(static_cast<double>(drain) * s / 512.0)) + (pk >> 23);
    return static_cast<int>(v < 0 ? 0 : (v > qmax ? qmax : v));
  }
}

__device__ __forceinline__ int apply_contract(const ExactArgs &g, long long D, long long bias) {
  switch (g.contract) {
    case QH_CONTRACT_CLIP_I32: return contract_ct<QH_CONTRACT_CLIP_I32>(g, D, bias);
    case QH_CONTRACT_CLIP_I64: return contract_ct<QH_CONTRACT_CLIP_I64>(g, D, bias);
    case QH_CONTRACT_DIV_RINT: return contract_ct<QH_CONTRACT_DIV_RINT>(g, D, bias);
    case QH_CONTRACT_FLOOR256_DIV_RINT: return contract_ct<QH_CONTRACT_FLOOR256_DIV_RINT>(g, D, bias);
    case QH_CONTRACT_ROUND_DIV: return contract_ct<QH_CONTRACT_ROUND_DIV>(g, D, bias);
    case QH_CONTRACT_U8_DRAIN: return contract_ct<QH_CONTRACT_U8_DRAIN>(g, D, bias);
  }
  return 0;
}

// The oracle's float64 dot product for output (m, n) of a per-group weight, by one wave:
// sum_k fl64((a_k - zp) sA) * fl32(q_k s_g), then + bias, / sO, + zp, rint, clip.
template <bool A16>
__device__ void emulate_one(const ExactArgs &g, int m, int n, int lane) {
  double s = 0.0;
  const int c0 = plane_col(0, n, g.layout_planes);
  for (int kc = lane; kc < g.K / 16; kc += 64) {
    const int k = kc * 16;
    const uint4 wv = load_w16(g, c0, k);
    const float sc = g.s32g[static_cast<size_t>(n) * g.G + (k >> g.gshift)];
    uint4 av[2];
    if (A16) {
      const uint4 *ap = reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(g.act) + static_cast<size_t>(m) * g.K + k);
      av[0] = ap[0];
      av[1] = ap[1];
    } else {
      av[0] = *reinterpret_cast<const uint4 *>(g.act + static_cast<size_t>(m) * g.K + k);
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int a = A16 ? static_cast<int>(reinterpret_cast<const uint16_t *>(av)[j])
                        : static_cast<int>(reinterpret_cast<const uint8_t *>(av)[j]);
      const int w = reinterpret_cast<const int8_t *>(&wv)[j];
      const float wd = static_cast<float>(w) * sc;
      s = fma(static_cast<double>(a - g.act_zp) * g.sA, static_cast<double>(wd), s);
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
  if (lane == 0) {
    const double t = (s + g.bias_deq[n]) / g.sO + static_cast<double>(g.out_zp);
    const double o = fmin(fmax(rint(t), 0.0), static_cast<double>(g.out_qmax));
    store_out(g, static_cast<size_t>(m) * g.N + n, static_cast<int>(o));
  }
}

// Fragments of one 32-k step: activations (A16: two raw words) and the planes' weights.
template <bool A16>
struct Frag {
  uint4 a[A16 ? 2 : 1];
  uint4 b[2];
};

template <bool A16>
__device__ __forceinline__ void load_step(const ExactArgs &g, int mrow, int ncol, int k, Frag<A16> &f) {
  if (A16) {
    const uint4 *ap = reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(g.act) + static_cast<size_t>(mrow) * g.K + k);
    f.a[0] = ap[0];
    f.a[A16 ? 1 : 0] = ap[1];
  } else {
    f.a[0] = *reinterpret_cast<const uint4 *>(g.act + static_cast<size_t>(mrow) * g.K + k);
  }
  f.b[0] = load_w16(g, plane_col(0, ncol, g.layout_planes), k);
  f.b[1] = g.nplanes > 1 ? load_w16(g, plane_col(1, ncol, g.layout_planes), k) : make_uint4(0u, 0u, 0u, 0u);
}

template <bool A16, int MODE>
__global__ __launch_bounds__(kExThreads, 2) void qmm_exact_kernel(const ExactArgs g) {
  constexpr int D = A16 ? 2 : 1;  // activation digits
  __shared__ uint32_t fix_list[MODE == 0 ? kExFixCap : 1];
  __shared__ int fix_cnt;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int m0 = blockIdx.y * kExTile + wm * 32, n0 = blockIdx.x * kExTile + wn * 32;
  const int mrow = min(m0 + (lane & 31), g.M - 1);  // rows past M repeat the last row (never stored)
  const int ncol = n0 + (lane & 31);                // < Np: padding columns hold zero weights
  const int kq = 16 * (lane >> 5);                  // this lane's 16 k of a 32-k step
  if (MODE == 0 && t == 0) fix_cnt = 0;

  v16i acc[2][D], one[D];
  long long acc64[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc64[j] = 0;
#pragma unroll
  for (int d = 0; d < D; ++d) {
    acc[0][d] = v16i{};
    acc[1][d] = v16i{};
    one[d] = v16i{};
  }
  const v4i ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
  // The epilogue's per-column constants are requested before the k loop, so their latency
  // overlaps the operand loads instead of following the products.
  const long long corr = g.corr[ncol];
  const long long bq = MODE == 2 && g.bias_q ? g.bias_q[ncol] : 0;
  double alpha = 0.0, beta = 0.0, mex = 0.0, absb = 0.0;
  if (MODE == 0) {
    alpha = g.alpha_e[ncol];
    beta = g.beta[ncol];
    mex = g.margin_exact[ncol];
    absb = g.absb[ncol];
  }
  const int steps = g.K / 32;
  // Loads go out a batch of NB 32-k steps at a time, one batch ahead of the products: a short K
  // (the reference's 256^3 graphs) then takes a few memory round trips instead of one per step.
  // Slots past the last step reload it (unused), so every batch issues the same loads.
  constexpr int NB = A16 ? 2 : 4;
  const int nbatch = (steps + NB - 1) / NB;
  Frag<A16> cur[NB], nxt[NB];
  auto load_batch = [&](int b, Frag<A16>(&f)[NB]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NB; ++i) load_step<A16>(g, mrow, ncol, 32 * min(b * NB + i, steps - 1) + kq, f[i]);
  };
  load_batch(0, cur);
  for (int bt = 0; bt < nbatch; ++bt) {
    if (bt + 1 < nbatch) load_batch(bt + 1, nxt);
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int s = bt * NB + i;
      if (s >= steps) break;  // wave-uniform
      v4i af[D];
      if (!A16) {
        const uint4 v = cur[i].a[0];
        af[0] = v4i{static_cast<int>(v.x ^ 0x80808080u), static_cast<int>(v.y ^ 0x80808080u),
                    static_cast<int>(v.z ^ 0x80808080u), static_cast<int>(v.w ^ 0x80808080u)};
      } else {
        uint4 v0 = cur[i].a[0], v1 = cur[i].a[D - 1];
        v0.x ^= 0x80808080u; v0.y ^= 0x80808080u; v0.z ^= 0x80808080u; v0.w ^= 0x80808080u;
        v1.x ^= 0x80808080u; v1.y ^= 0x80808080u; v1.z ^= 0x80808080u; v1.w ^= 0x80808080u;
        // a - 32768 = 256 hi + lo' + 128 with hi = high byte ^ 0x80, lo' = low byte ^ 0x80
        af[0] = v4i{static_cast<int>(perm(v0.y, v0.x, 0x07050301u)), static_cast<int>(perm(v0.w, v0.z, 0x07050301u)),
                    static_cast<int>(perm(v1.y, v1.x, 0x07050301u)), static_cast<int>(perm(v1.w, v1.z, 0x07050301u))};
        af[D - 1] = v4i{static_cast<int>(perm(v0.y, v0.x, 0x06040200u)), static_cast<int>(perm(v0.w, v0.z, 0x06040200u)),
                        static_cast<int>(perm(v1.y, v1.x, 0x06040200u)), static_cast<int>(perm(v1.w, v1.z, 0x06040200u))};
      }
#pragma unroll
      for (int d = 0; d < D; ++d) {
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          if (p >= g.nplanes) break;
          const uint4 b = cur[i].b[p];
          acc[p][d] = __builtin_amdgcn_mfma_i32_32x32x32_i8(
              af[d], v4i{static_cast<int>(b.x), static_cast<int>(b.y), static_cast<int>(b.z), static_cast<int>(b.w)},
              acc[p][d], 0, 0, 0);
        }
        if (g.ones) one[d] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[d], ones, one[d], 0, 0, 0);
      }
      // every 64 k (and after the last step): int32 sums into the int64 accumulators
      if ((s & 1) || s + 1 == steps) {
        const int grp = (32 * s) >> g.gshift;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          if (p >= g.nplanes) break;
          const long long mlt = MODE == 0 ? g.mult[(static_cast<size_t>(p) * g.G + grp) * g.Np + ncol] : g.cm[p];
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int v = A16 ? 256 * acc[p][0][j] + acc[p][D - 1][j] : acc[p][0][j];
            acc64[j] += static_cast<long long>(v) * mlt;
          }
#pragma unroll
          for (int d = 0; d < D; ++d) acc[p][d] = v16i{};
        }
        if (g.ones) {
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int v = A16 ? 256 * one[0][j] + one[D - 1][j] : one[0][j];
            acc64[j] += static_cast<long long>(v) * g.ones;
          }
#pragma unroll
          for (int d = 0; d < D; ++d) one[d] = v16i{};
        }
      }
    }
    if (bt + 1 < nbatch) {
#pragma unroll
      for (int i = 0; i < NB; ++i) cur[i] = nxt[i];
    }
  }

  // ---- epilogue: lane holds rows m0 + 8 (j / 4) + 4 (lane / 32) + j % 4 of column ncol
  const bool col_ok = ncol < g.N;
  __syncthreads();  // fix_cnt initialised
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int m = m0 + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
    if (m >= g.M || !col_ok) continue;
    const long long Dv = acc64[j] + corr;
    const size_t idx = static_cast<size_t>(m) * g.N + ncol;
    if (MODE == 1) {
      static_cast<long long *>(g.out)[idx] = Dv;
    } else if (MODE == 2) {
      store_out(g, idx, apply_contract(g, Dv, bq));
    } else {
      const double u = static_cast<double>(Dv) * alpha;
      const double tv = u + beta;
      const double fl = floor(tv);
      const double slack = mex + 0x1p-48 * (fabs(u) + fabs(tv) + absb);
      const double qmaxd = static_cast<double>(g.out_qmax);
      const bool near = fabs((tv - fl) - 0.5) <= slack;
      const bool amb = near && fmin(fmax(fl, 0.0), qmaxd) != fmin(fmax(fl + 1.0, 0.0), qmaxd);
      if (!amb) {
        store_out(g, idx, static_cast<int>(fmin(fmax(rint(tv), 0.0), qmaxd)));
      } else {
        const int slot = atomicAdd(&fix_cnt, 1);
        if (slot < kExFixCap) fix_list[slot] = (static_cast<uint32_t>(m - blockIdx.y * kExTile) << 16) |
                                               static_cast<uint32_t>(ncol - blockIdx.x * kExTile);
      }
    }
  }
  if (MODE == 0) {
    __syncthreads();
    const int cnt = fix_cnt;
    if (cnt == 0) return;
    // listed outputs: one wave each; beyond the list's capacity a second sweep recomputes the
    // tile's ambiguous outputs that were not listed
    for (int e = wave; e < min(cnt, kExFixCap); e += kExThreads / 64) {
      const uint32_t v = __builtin_amdgcn_readfirstlane(fix_list[e]);
      emulate_one<A16>(g, blockIdx.y * kExTile + static_cast<int>(v >> 16),
                       blockIdx.x * kExTile + static_cast<int>(v & 0xFFFFu), lane);
    }
    if (cnt > kExFixCap) {
      __syncthreads();
      // recompute every ambiguous output of this wave's block again, wave-cooperatively
      for (int j = 0; j < 16; ++j) {
        for (int src = 0; src < 64; ++src) {
          const int m = m0 + 8 * (j >> 2) + 4 * (src >> 5) + (j & 3);
          const int n = n0 + (src & 31);
          const long long Dv = __shfl(acc64[j], src, 64) + g.corr[n < g.Np ? n : 0];
          if (m >= g.M || n >= g.N) continue;
          const double u = static_cast<double>(Dv) * g.alpha_e[n];
          const double tv = u + g.beta[n];
          const double fl = floor(tv);
          const double slack = g.margin_exact[n] + 0x1p-48 * (fabs(u) + fabs(tv) + g.absb[n]);
          const double qmaxd = static_cast<double>(g.out_qmax);
          const bool amb = fabs((tv - fl) - 0.5) <= slack &&
                           fmin(fmax(fl, 0.0), qmaxd) != fmin(fmax(fl + 1.0, 0.0), qmaxd);
          if (amb) emulate_one<A16>(g, m, n, lane);
        }
      }
    }
  }
}

// ---- fused integer-contract chains: every step of a CHAIN graph in one launch
//
// Row m of step i+1's activation is row m of step i's output, so a workgroup that owns a block
// of rows runs the whole chain on its own: the block's activation stays in LDS (two buffers,
// the step's input and its output), each wave keeps its 32 weight columns in registers for all
// steps (K == N <= 256: at most 4 x 2 x 2 fragments of 16 bytes per lane), and one barrier per
// step separates a step's writes from the next step's reads.  16-row blocks on
// v_mfma_i32_16x16x64_i8 give twice the workgroups of 32-row blocks (256 rows: 16 compute
// units) and half the work per step.  Every step is the contract kernel's arithmetic (the same
// int32 sums of the shifted operands, per-column correction and contract), so the result is the
// per-step launches' result bit for bit; K <= 256 keeps every int32 MFMA sum below 2^22 in
// magnitude.  The k loop always runs the 4 steps of K = 256: LDS columns K..255 hold the code
// that shifts to 0 (0x80 bytes) and the weight fragments there are zero, so they add nothing.
constexpr int kChRows = 16;                 // activation rows per workgroup
constexpr int kChWaves = 8;                 // wave w owns output columns [32 w, 32 w + 32)
constexpr int kChMaxK = 32 * kChWaves;      // K == N <= 256
constexpr int kChSteps = kChMaxK / 64;      // 64-k MFMA steps
constexpr int kChThreads = 64 * kChWaves;

// The dividing contracts in float64 without a division, on D as an integer-valued double
// (|D| < 2^40: every product and sum below is an exact integer).
//  * rint(double(D) / d + zp): y = D rcp + zp (rcp = fl(1 / d), one fma) is within 2^-34 of
//    X = D / d + zp whenever rint(y) lies in [-1, qmax + 1] (then |D / d| < 2^17 and y < 2^17).
//    If y is also more than 2^-20 from the nearest half-integer, rint(y) = rint(X).  The
//    float64 division rounds the same X for every output that is not clipped: a quotient that
//    is not a tie lies at least 1 / (2 d) >= 2^-31 from a half-integer, and the division's two
//    roundings move it by less.  Outputs outside [-1, qmax + 1] clip the same either way.  The
//    few outputs near a half-integer (exact ties: only for even d) take the exact remainder
//    2 (D - (c - zp) d), which picks the neighbour the exact quotient rounds to (ties to even);
//    a wave enters that branch only when one of its lanes needs it.
//  * floor(n / d) (round_div, n >= 0): floor(n rcp) is within one; the remainder fixes it.
template <int CT>
__device__ __forceinline__ int contract_chain_f64(const ExactArgs &g, double Dd, double rcp) {
  const double dd = static_cast<double>(g.divisor), zp = static_cast<double>(g.out_zp);
  const double qmax = static_cast<double>(g.out_qmax);
  if constexpr (CT == QH_CONTRACT_ROUND_DIV) {
    const double n = fabs(Dd) + static_cast<double>(g.divisor / 2);
    double q = floor(n * rcp);
    const double r = fma(-q, dd, n);
    q = r < 0.0 ? q - 1.0 : (r >= dd ? q + 1.0 : q);
    const double v = (Dd >= 0.0 ? q : -q) + zp;
    return static_cast<int>(fmin(fmax(v, 0.0), qmax));
  } else {
    if (CT == QH_CONTRACT_FLOOR256_DIV_RINT) Dd = floor(Dd * 0x1p-8) * 256.0;  // floor division, exact
    const double y = fma(Dd, rcp, zp);
    double c = rint(y);
    const bool near = fabs(y - c) > 0.5 - 0x1p-20 && c >= -1.0 && c <= qmax + 1.0;
    if (__builtin_amdgcn_ballot_w64(near) != 0) {  // wave-uniform: rare
      // exact for every lane: in range, c is within one of the rounded quotient (and lanes that
      // are not near stay put); out of range, c +- 1 clips like c
      const double r2 = 2.0 * fma(zp - c, dd, Dd);  // 2 (D - q d), q = c - zp
      const double h = c * 0.5;
      const bool odd = h != floor(h);
      c = (r2 > dd || (r2 == dd && odd)) ? c + 1.0 : ((r2 < -dd || (r2 == -dd && odd)) ? c - 1.0 : c);
    }
    return static_cast<int>(fmin(fmax(c, 0.0), qmax));
  }
}

// W16: int16 weights (two planes and the all-ones plane); else one int8 plane.  CT: the contract.
template <bool A16, bool W16, int CT>
__global__ __launch_bounds__(kChThreads, 1) void qmm_chain_kernel(const ExactArgs g, int chain) {
  constexpr int D = A16 ? 2 : 1;       // activation digits
  constexpr int NP = W16 ? 2 : 1;      // weight planes
  constexpr int E = A16 ? 2 : 1;       // bytes per activation / output element
  constexpr int kPitch = E * kChMaxK + 32;  // LDS row pitch: 8 (mod 16) dwords, so 16-byte fragment reads of 16 rows are conflict-free
  // the dividing contracts take the float64 path (bias_q is not part of them)
  constexpr bool kF64 = CT == QH_CONTRACT_DIV_RINT || CT == QH_CONTRACT_FLOOR256_DIV_RINT || CT == QH_CONTRACT_ROUND_DIV;
  __shared__ __align__(16) uint8_t buf[2][kChRows * kPitch];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int m0 = blockIdx.x * kChRows;
  const bool active = 32 * wave < g.N;         // wave-uniform (N % 32 == 0)
  const int kg = 16 * (lane >> 4);             // this lane's 16 k of a 64-k step
  const int rowb = g.K * E;                    // bytes per activation row (a multiple of 32)
  const double rcp = 1.0 / static_cast<double>(g.divisor > 0 ? g.divisor : 1);

  // the block's activation rows into buffer 0 (rows past M repeat the last row; never stored);
  // columns K..255 of both buffers: 0x80 bytes
  for (int i = t; i < kChRows * (kChMaxK * E / 16); i += kChThreads) {
    const int r = i / (kChMaxK * E / 16), c = i - r * (kChMaxK * E / 16);
    const int mr = min(m0 + r, g.M - 1);
    constexpr uint32_t kPad = 0x80808080u;
    const bool in = 16 * c < rowb;
    // a clamped, always valid address and per-word selects (a select of whole uint4 values
    // becomes a select of stack addresses, i.e. scratch memory)
    const uint4 x = *reinterpret_cast<const uint4 *>(g.act + static_cast<size_t>(mr) * rowb + 16 * min(c, rowb / 16 - 1));
    *reinterpret_cast<uint4 *>(&buf[0][r * kPitch + 16 * c]) =
        make_uint4(in ? x.x : kPad, in ? x.y : kPad, in ? x.z : kPad, in ? x.w : kPad);
    if (!in) *reinterpret_cast<uint4 *>(&buf[1][r * kPitch + 16 * c]) = make_uint4(kPad, kPad, kPad, kPad);
  }
  // B fragments: lane holds 16 k (kg..kg+15 of each 64-k step) of column 32 w + 16 ct + lane % 16
  uint4 w[kChSteps][2][NP];
  long long corr[2] = {0, 0}, bq[2] = {0, 0};
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    const int n = 32 * wave + 16 * ct + (lane & 15);
#pragma unroll
    for (int s = 0; s < kChSteps; ++s)
#pragma unroll
      for (int p = 0; p < NP; ++p)
        w[s][ct][p] = active && 64 * s + kg < g.K ? load_w16(g, plane_col(p, n, g.layout_planes), 64 * s + kg)
                                                  : make_uint4(0u, 0u, 0u, 0u);
    if (active) {
      corr[ct] = g.corr[n];
      bq[ct] = g.bias_q ? g.bias_q[n] : 0;
    }
  }
  // quad transpose of the epilogue: lane c = lane % 4 of a quad collects row c of the quad's
  // 4 columns; round t takes the value of quad lane (c + t) % 4 (DPP quad_perm)
  const int qc = lane & 3;
  uint32_t qsel[4];
#pragma unroll
  for (int tt = 1; tt < 4; ++tt) {
    const int k = (qc + tt) & 3;  // byte k of the result <- byte qc of the value from quad lane k
    uint32_t sel = 0;
#pragma unroll
    for (int m = 0; m < 4; ++m) sel |= static_cast<uint32_t>(m == k ? 4 + qc : m) << (8 * m);
    qsel[tt] = sel;
  }
  __syncthreads();

  for (int it = 0; it < chain; ++it) {
    const uint8_t *src = buf[it & 1];
    uint8_t *dst = buf[(it + 1) & 1];
    if (active) {
      v4i acc[2][NP][D];
      int rs = 0;  // W16: partial sum of this lane's activation row (lane % 16) over its k
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
          for (int d = 0; d < D; ++d) acc[ct][p][d] = v4i{0, 0, 0, 0};
#pragma unroll
      for (int s = 0; s < kChSteps; ++s) {
        const uint8_t *ap = src + (lane & 15) * kPitch + E * (64 * s + kg);
        v4i af[D];
        if (!A16) {
          const uint4 v = *reinterpret_cast<const uint4 *>(ap);
          af[0] = v4i{static_cast<int>(v.x ^ 0x80808080u), static_cast<int>(v.y ^ 0x80808080u),
                      static_cast<int>(v.z ^ 0x80808080u), static_cast<int>(v.w ^ 0x80808080u)};
        } else {
          uint4 v0 = reinterpret_cast<const uint4 *>(ap)[0], v1 = reinterpret_cast<const uint4 *>(ap)[1];
          v0.x ^= 0x80808080u; v0.y ^= 0x80808080u; v0.z ^= 0x80808080u; v0.w ^= 0x80808080u;
          v1.x ^= 0x80808080u; v1.y ^= 0x80808080u; v1.z ^= 0x80808080u; v1.w ^= 0x80808080u;
          // a - 32768 = 256 hi + lo' + 128 with hi = high byte ^ 0x80, lo' = low byte ^ 0x80
          af[0] = v4i{static_cast<int>(perm(v0.y, v0.x, 0x07050301u)), static_cast<int>(perm(v0.w, v0.z, 0x07050301u)),
                      static_cast<int>(perm(v1.y, v1.x, 0x07050301u)), static_cast<int>(perm(v1.w, v1.z, 0x07050301u))};
          af[D - 1] = v4i{static_cast<int>(perm(v0.y, v0.x, 0x06040200u)), static_cast<int>(perm(v0.w, v0.z, 0x06040200u)),
                          static_cast<int>(perm(v1.y, v1.x, 0x06040200u)), static_cast<int>(perm(v1.w, v1.z, 0x06040200u))};
        }
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
          for (int p = 0; p < NP; ++p) {
            const uint4 b = w[s][ct][p];
            const v4i bv = v4i{static_cast<int>(b.x), static_cast<int>(b.y), static_cast<int>(b.z), static_cast<int>(b.w)};
#pragma unroll
            for (int d = 0; d < D; ++d)
              acc[ct][p][d] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[d], bv, acc[ct][p][d], 0, 0, 0);
          }
        if (W16) {
          // the all-ones plane's product is the row sum of the shifted activation (byte dot
          // products instead of an MFMA)
          int part[D];
#pragma unroll
          for (int d = 0; d < D; ++d)
            part[d] = __builtin_amdgcn_sdot4(af[d][0], 0x01010101, __builtin_amdgcn_sdot4(af[d][1], 0x01010101,
                      __builtin_amdgcn_sdot4(af[d][2], 0x01010101, __builtin_amdgcn_sdot4(af[d][3], 0x01010101, 0, false),
                                             false), false), false);
          rs += A16 ? 256 * part[0] + part[D - 1] : part[0];
        }
      }
      int rowsum = 0;
      if (W16) {  // lane r < 16: row r over all k (its 4 k-groups sit in lanes r, r + 16, r + 32, r + 48)
        rowsum = rs + __shfl_xor(rs, 16, 64);
        rowsum += __shfl_xor(rowsum, 32, 64);
      }
      // lane holds rows 4 (lane / 16) + i, i < 4, of column 32 w + 16 ct + lane % 16
      const int rbase = 4 * (lane >> 4);
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        int v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if constexpr (kF64) {
            // D as an exact integer-valued double (|D| < 2^40)
            double Dd;
            if constexpr (!A16 && !W16) {
              Dd = static_cast<double>(acc[ct][0][0][i] + static_cast<int>(corr[ct]));
            } else if constexpr (!W16) {
              // one plane with multiplier 1: 256 hi + lo stays below 2^31 in magnitude
              Dd = static_cast<double>(256 * acc[ct][0][0][i] + acc[ct][0][D - 1][i]) + static_cast<double>(corr[ct]);
            } else {
              Dd = static_cast<double>(corr[ct]);
#pragma unroll
              for (int p = 0; p < NP; ++p) {
                const double x = A16 ? fma(256.0, static_cast<double>(acc[ct][p][0][i]), static_cast<double>(acc[ct][p][D - 1][i]))
                                     : static_cast<double>(acc[ct][p][0][i]);
                Dd = fma(x, static_cast<double>(g.cm[p]), Dd);
              }
              if (W16) Dd = fma(static_cast<double>(__shfl(rowsum, rbase + i, 64)), static_cast<double>(g.ones), Dd);
            }
            v[i] = contract_chain_f64<CT>(g, Dd, rcp);
          } else {
            long long Dv;
            if constexpr (!A16 && !W16) {
              // one int8 plane with multiplier 1: |sum| < 2^22 and |corr| < 2^22, so int32 is exact
              Dv = static_cast<long long>(acc[ct][0][0][i] + static_cast<int>(corr[ct]));
            } else {
              Dv = corr[ct];
#pragma unroll
              for (int p = 0; p < NP; ++p) {
                const long long x = A16 ? 256LL * acc[ct][p][0][i] + acc[ct][p][D - 1][i] : static_cast<long long>(acc[ct][p][0][i]);
                Dv += x * g.cm[p];
              }
              if (W16) Dv += static_cast<long long>(__shfl(rowsum, rbase + i, 64)) * g.ones;
            }
            v[i] = contract_ct<CT>(g, Dv, bq[ct]);
          }
        }
        const int col0 = 32 * wave + 16 * ct + (lane & 12);  // the quad's first column
        if (!A16) {
          // rows rbase .. rbase + 3 of this column as bytes, then the quad transpose: lane qc
          // ends with row rbase + qc of columns col0 .. col0 + 3
          const uint32_t P = static_cast<uint32_t>(v[0]) | (static_cast<uint32_t>(v[1]) << 8) |
                             (static_cast<uint32_t>(v[2]) << 16) | (static_cast<uint32_t>(v[3]) << 24);
          uint32_t Q = P;  // round 0: byte qc of its own value is already in place
          Q = perm(static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(P), 0x39, 0xf, 0xf, false)), Q, qsel[1]);
          Q = perm(static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(P), 0x4E, 0xf, 0xf, false)), Q, qsel[2]);
          Q = perm(static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(P), 0x93, 0xf, 0xf, false)), Q, qsel[3]);
          *reinterpret_cast<uint32_t *>(dst + (rbase + qc) * kPitch + col0) = Q;
        } else {
          // pairs of lanes (columns c, c + 1) swap halves: the even lane ends with rows rbase and
          // rbase + 2 of both columns, the odd lane with rows rbase + 1 and rbase + 3
          const bool odd = lane & 1;
          const uint32_t send = odd ? (static_cast<uint32_t>(v[0]) | (static_cast<uint32_t>(v[2]) << 16))
                                    : (static_cast<uint32_t>(v[1]) | (static_cast<uint32_t>(v[3]) << 16));
          const uint32_t got = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(send), 0xB1, 0xf, 0xf, false));
          const int c2 = 32 * wave + 16 * ct + (lane & 14);  // the pair's even column
          const uint32_t lo = odd ? (got & 0xFFFFu) | (static_cast<uint32_t>(v[1]) << 16)
                                  : static_cast<uint32_t>(v[0]) | (got << 16);
          const uint32_t hi = odd ? (got >> 16) | (static_cast<uint32_t>(v[3]) << 16)
                                  : static_cast<uint32_t>(v[2]) | (got & 0xFFFF0000u);
          const int r0 = rbase + (odd ? 1 : 0);
          *reinterpret_cast<uint32_t *>(dst + r0 * kPitch + 2 * c2) = lo;
          *reinterpret_cast<uint32_t *>(dst + (r0 + 2) * kPitch + 2 * c2) = hi;
        }
      }
    }
    __syncthreads();
  }

  // the last step's rows (those below M) to the output, 16 bytes per store
  const uint8_t *res = buf[chain & 1];
  const int outb = g.N * E;
  for (int i = t; i < kChRows * (outb / 16); i += kChThreads) {
    const int r = i / (outb / 16), c = i - r * (outb / 16);
    if (m0 + r < g.M)
      *reinterpret_cast<uint4 *>(static_cast<uint8_t *>(g.out) + static_cast<size_t>(m0 + r) * outb + 16 * c) =
          *reinterpret_cast<const uint4 *>(&res[r * kPitch + 16 * c]);
  }
}

template <bool A16, bool W16>
qh_status launch_chain_ct(const ExactArgs &g, int chain, dim3 grid, hipStream_t stream) {
  switch (g.contract) {
    case QH_CONTRACT_CLIP_I32:
      hipLaunchKernelGGL((qmm_chain_kernel<A16, W16, QH_CONTRACT_CLIP_I32>), grid, dim3(kChThreads), 0, stream, g, chain);
      break;
    case QH_CONTRACT_CLIP_I64:
      hipLaunchKernelGGL((qmm_chain_kernel<A16, W16, QH_CONTRACT_CLIP_I64>), grid, dim3(kChThreads), 0, stream, g, chain);
      break;
    case QH_CONTRACT_DIV_RINT:
      hipLaunchKernelGGL((qmm_chain_kernel<A16, W16, QH_CONTRACT_DIV_RINT>), grid, dim3(kChThreads), 0, stream, g, chain);
      break;
    case QH_CONTRACT_FLOOR256_DIV_RINT:
      hipLaunchKernelGGL((qmm_chain_kernel<A16, W16, QH_CONTRACT_FLOOR256_DIV_RINT>), grid, dim3(kChThreads), 0, stream, g,
                         chain);
      break;
    case QH_CONTRACT_ROUND_DIV:
      hipLaunchKernelGGL((qmm_chain_kernel<A16, W16, QH_CONTRACT_ROUND_DIV>), grid, dim3(kChThreads), 0, stream, g, chain);
      break;
    case QH_CONTRACT_U8_DRAIN:
      hipLaunchKernelGGL((qmm_chain_kernel<A16, W16, QH_CONTRACT_U8_DRAIN>), grid, dim3(kChThreads), 0, stream, g, chain);
      break;
    default:
      return fail(QH_STATUS_UNSUPPORTED, "fused chain: unknown contract %d", g.contract);
  }
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return hip_fail(err, "qmm_chain_kernel launch");
  return QH_STATUS_OK;
}

template <bool A16, int MODE>
qh_status launch(const ExactArgs &g, hipStream_t stream) {
  const dim3 grid((g.N + kExTile - 1) / kExTile, (g.M + kExTile - 1) / kExTile);
  hipLaunchKernelGGL((qmm_exact_kernel<A16, MODE>), grid, dim3(kExThreads), 0, stream, g);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return hip_fail(err, "qmm_exact_kernel launch");
  return QH_STATUS_OK;
}

template <int MODE>
qh_status dispatch(const ExactArgs &g, bool a16, hipStream_t stream) {
  return a16 ? launch<true, MODE>(g, stream) : launch<false, MODE>(g, stream);
}

}  // namespace

namespace {

ExactArgs exact_args(const qh_qmm_prepared *p, int m, const void *act, void *out, int mode, int contract, int divisor) {
  const QmmShape &sh = p->shape;
  const QmmDevice &Dv = p->dev;
  ExactArgs g{};
  g.act = static_cast<const uint8_t *>(act);
  g.out = out;
  g.tiles = Dv.tiles;
  g.KT = sh.Kp / kBK;
  g.layout_planes = sh.layout_planes;
  g.M = m;
  g.N = sh.N;
  g.K = sh.K;
  g.Np = sh.Np;
  g.act_zp = sh.act_zp;
  g.out_zp = sh.out_zp;
  g.out_qmax = (1 << sh.out_bits) - 1;
  g.out16 = sh.out_bits == 16;
  g.sA = sh.act_scale;
  g.sO = sh.out_scale;
  g.contract = contract;
  g.divisor = divisor;
  g.bias_q = Dv.bias_q;
  if (mode == 0) {
    // requantisation of a per-group weight: planes q and r with their group multipliers
    g.nplanes = 2;
    g.ones = 0;
    g.mult = Dv.mult;
    g.G = sh.groups;
    g.gshift = sh.group_shift;
    g.corr = Dv.corr_rq;
    g.alpha_e = Dv.alpha_e;
    g.beta = Dv.beta;
    g.margin_exact = Dv.margin_exact;
    g.absb = Dv.absb;
    g.s32g = Dv.s32g;
    g.bias_deq = Dv.bias_deq;
  } else {
    // the integer dot product sum_k (a - zp) w_int
    g.nplanes = sh.int_planes;
    g.cm[0] = sh.int_mult[0];
    g.cm[1] = sh.int_mult[1];
    g.ones = sh.int_ones;
    g.G = 1;
    g.gshift = 6;
    g.corr = Dv.corr_int;
  }
  return g;
}

}  // namespace

qh_status launch_qmm_exact(const qh_qmm_prepared *p, int m, const void *act, void *out, int mode, int contract,
                           int divisor, hipStream_t stream) {
  if (m > 65535 * kExTile) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "M=%d too large for one launch", m);
  const ExactArgs g = exact_args(p, m, act, out, mode, contract, divisor);
  const bool a16 = p->shape.act_bits == 16;
  if (mode == 0) return dispatch<0>(g, a16, stream);
  if (mode == 1) return dispatch<1>(g, a16, stream);
  return dispatch<2>(g, a16, stream);
}

bool chain_fusable(const qh_qmm_prepared *p) {
  const QmmShape &sh = p->shape;
  // one int8 plane with multiplier 1, or the int16 weight's two planes plus the all-ones plane
  const bool planes = sh.int_planes == 1 ? sh.int_mult[0] == 1 && sh.int_ones == 0 : sh.int_planes == 2 && sh.int_ones != 0;
  return planes && sh.K == sh.N && sh.K <= kChMaxK && sh.K % 32 == 0 && sh.act_bits == sh.out_bits;
}

qh_status launch_qmm_chain(const qh_qmm_prepared *p, int m, int chain, const void *act, void *out, int contract,
                           int divisor, hipStream_t stream) {
  if (!chain_fusable(p)) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "fused chain: K == N <= %d only", kChMaxK);
  const ExactArgs g = exact_args(p, m, act, out, 2, contract, divisor);
  const dim3 grid((m + kChRows - 1) / kChRows);
  const bool a16 = p->shape.act_bits == 16, w16 = g.nplanes == 2;
  if (a16) return w16 ? launch_chain_ct<true, true>(g, chain, grid, stream) : launch_chain_ct<true, false>(g, chain, grid, stream);
  return w16 ? launch_chain_ct<false, true>(g, chain, grid, stream) : launch_chain_ct<false, false>(g, chain, grid, stream);
}

}  // namespace qh
