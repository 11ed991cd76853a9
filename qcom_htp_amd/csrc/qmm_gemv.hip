// Decode-shape (M <= 16) quantized GEMV: HBM streaming of packed weights with dwordx4 loads,
// int8 dot4 MACs (v_dot4_i32_i8) and wavefront reductions -- no MFMA.
//
// Weight stream layout (prepared once): [N/16 column groups][K/32 k-groups][16 columns][bytes],
// 16 B per (column, k-group) for int4 (byte j: low nibble k=j, high nibble k=j+16,
// offset-binary) or 32 B for int8.  One wave instruction therefore reads 4 k-groups x 16 columns
// = 1 KiB (int4) / 2 KiB (int8) of contiguous HBM.  LPBQ block scales are streamed as
// [N/16][K/block][16] bytes and applied to each k-group's integer partial dot product
// (sum_k a*(q*f) = f * sum_k a*q inside a block), which keeps the integer result exact.
//
// Activations (M x K) are staged once per workgroup in LDS as signed int8 planes
// (a - 128 for 8-bit; hi / lo' bytes of a - 32768 for 16-bit).  For 16-bit activations the
// workgroup also forms R1[m] = sum_k |a - zp|, which bounds the float32-rounding residue term
// of the requantisation (the GEMV does not stream the residue plane).  The epilogue and the
// exact fixup follow the GEMM's (qmm_gemm.hip).

#include "qmm_internal.h"

namespace qh {
namespace {

constexpr int kGemvThreads = 256;
constexpr int kGemvMaxLds = 128 * 1024;  // activation planes

struct GemvArgs {
  const uint8_t *act;
  void *out;
  const uint8_t *w;      // GEMV stream
  const uint8_t *lpbq;   // [N/16][K/bs][16]
  const double *alpha, *beta, *margin, *absb, *bias_deq, *mr1;
  const int64_t *corr, *mant, *colsum;
  const float *s32;
  int M, N, K, KG, nblk, bs_shift;
  int act_zp, out_zp, out_qmax, out16;
  double sA, sO;
};

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// Integer weight codes (times the LPBQ block scale) of column n, k-group kg: 32 values.
template <int FMT, bool LPBQ>
__device__ __forceinline__ void load_w32(const GemvArgs &g, int n, int kg, int (&w)[32]) {
  const size_t base = (static_cast<size_t>(n / 16) * g.KG + kg) * 16 + (n % 16);
  if (FMT == kTileI4) {
    uint4 v = *reinterpret_cast<const uint4 *>(g.w + base * 16);
    const uint8_t *b = reinterpret_cast<const uint8_t *>(&v);
    int f = 1;
    if (LPBQ) f = g.lpbq[(static_cast<size_t>(n / 16) * g.nblk + ((kg * 32) >> g.bs_shift)) * 16 + (n % 16)];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      w[j] = ((b[j] & 15) - 8) * f;
      w[j + 16] = ((b[j] >> 4) - 8) * f;
    }
  } else {
    const uint4 *p = reinterpret_cast<const uint4 *>(g.w + base * 32);
    uint4 v0 = p[0], v1 = p[1];
    const int8_t *b0 = reinterpret_cast<const int8_t *>(&v0), *b1 = reinterpret_cast<const int8_t *>(&v1);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      w[j] = b0[j];
      w[j + 16] = b1[j];
    }
  }
}

template <bool A16, int FMT, bool LPBQ>
__device__ void gemv_fixup(const GemvArgs &g, int m, int n, int lane) {
  const float sc = g.s32[n];
  double s = 0.0;
  for (int kg = lane; kg < g.KG; kg += 64) {
    int w[32];
    load_w32<FMT, LPBQ>(g, n, kg, w);
    const int k = kg * 32;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const int a = A16 ? reinterpret_cast<const uint16_t *>(g.act)[static_cast<size_t>(m) * g.K + k + j]
                        : g.act[static_cast<size_t>(m) * g.K + k + j];
      const float wd = static_cast<float>(w[j]) * sc;
      s = fma(static_cast<double>(a - g.act_zp) * g.sA, static_cast<double>(wd), s);
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
  if (lane == 0) {
    const double t = (s + g.bias_deq[n]) / g.sO + static_cast<double>(g.out_zp);
    const double o = fmin(fmax(rint(t), 0.0), static_cast<double>(g.out_qmax));
    const size_t idx = static_cast<size_t>(m) * g.N + n;
    if (g.out16)
      static_cast<uint16_t *>(g.out)[idx] = static_cast<uint16_t>(o);
    else
      static_cast<uint8_t *>(g.out)[idx] = static_cast<uint8_t>(o);
  }
}

template <bool A16, int FMT, bool LPBQ, int MM>
__global__ __launch_bounds__(kGemvThreads) void qmm_gemv_kernel(GemvArgs g) {
  extern __shared__ uint4 smem[];
  uint8_t *act_lds = reinterpret_cast<uint8_t *>(smem);  // [planes][M][K] int8
  __shared__ uint32_t r1[16];

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int M = g.M, K = g.K;
  if (t < 16) r1[t] = 0;
  __syncthreads();

  // ---- stage activations as signed int8 planes ---------------------------------------
  if (!A16) {
    const int chunks = M * K / 16;
    for (int c = t; c < chunks; c += kGemvThreads) {
      uint4 v = reinterpret_cast<const uint4 *>(g.act)[c];
      v.x ^= 0x80808080u;
      v.y ^= 0x80808080u;
      v.z ^= 0x80808080u;
      v.w ^= 0x80808080u;
      reinterpret_cast<uint4 *>(act_lds)[c] = v;
    }
  } else {
    const int chunks = M * K / 8;  // 8 values per 16 B
    uint2 *hi_pl = reinterpret_cast<uint2 *>(act_lds);
    uint2 *lo_pl = reinterpret_cast<uint2 *>(act_lds + static_cast<size_t>(M) * K);
    for (int c = t; c < chunks; c += kGemvThreads) {
      uint4 v = reinterpret_cast<const uint4 *>(g.act)[c];
      const uint16_t *h = reinterpret_cast<const uint16_t *>(&v);
      uint32_t sum = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) sum += static_cast<uint32_t>(abs(static_cast<int>(h[j]) - g.act_zp));
      v.x ^= 0x80808080u;
      v.y ^= 0x80808080u;
      v.z ^= 0x80808080u;
      v.w ^= 0x80808080u;
      hi_pl[c] = make_uint2(perm(v.y, v.x, 0x07050301u), perm(v.w, v.z, 0x07050301u));
      lo_pl[c] = make_uint2(perm(v.y, v.x, 0x06040200u), perm(v.w, v.z, 0x06040200u));
      atomicAdd(&r1[(c * 8) / K], sum);
    }
  }
  __syncthreads();

  const int groups = g.N / 16;
  const int waves_total = gridDim.x * (kGemvThreads / 64);
  const int col = lane & 15, sub = lane >> 4;  // 4 k-groups per wave instruction
  for (int grp = blockIdx.x * (kGemvThreads / 64) + wave; grp < groups; grp += waves_total) {
    const int n = grp * 16 + col;
    int acc[MM], acc2[A16 ? MM : 1];
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      acc[m] = 0;
      if (A16) acc2[m] = 0;
    }
    const uint8_t *wbase = g.w + static_cast<size_t>(grp) * g.KG * 16 * (FMT == kTileI4 ? 16 : 32);
    for (int kg = sub; kg < g.KG; kg += 4) {
      uint32_t w[8];
      if (FMT == kTileI4) {
        const uint4 v = *reinterpret_cast<const uint4 *>(wbase + (static_cast<size_t>(kg) * 16 + col) * 16);
        const uint32_t m4 = 0x0F0F0F0Fu;
        w[0] = ((v.x & m4) + 0x78787878u) ^ 0x80808080u;
        w[1] = ((v.y & m4) + 0x78787878u) ^ 0x80808080u;
        w[2] = ((v.z & m4) + 0x78787878u) ^ 0x80808080u;
        w[3] = ((v.w & m4) + 0x78787878u) ^ 0x80808080u;
        w[4] = (((v.x >> 4) & m4) + 0x78787878u) ^ 0x80808080u;
        w[5] = (((v.y >> 4) & m4) + 0x78787878u) ^ 0x80808080u;
        w[6] = (((v.z >> 4) & m4) + 0x78787878u) ^ 0x80808080u;
        w[7] = (((v.w >> 4) & m4) + 0x78787878u) ^ 0x80808080u;
      } else {
        const uint4 *p = reinterpret_cast<const uint4 *>(wbase + (static_cast<size_t>(kg) * 16 + col) * 32);
        const uint4 v0 = p[0], v1 = p[1];
        w[0] = v0.x; w[1] = v0.y; w[2] = v0.z; w[3] = v0.w;
        w[4] = v1.x; w[5] = v1.y; w[6] = v1.z; w[7] = v1.w;
      }
      int f = 1;
      if (LPBQ) f = g.lpbq[(static_cast<size_t>(grp) * g.nblk + ((kg * 32) >> g.bs_shift)) * 16 + col];
#pragma unroll
      for (int m = 0; m < MM; ++m) {
        if (MM == 1 || m < M) {  // predicated: MM is a compile-time trip count
        const uint4 *ap = reinterpret_cast<const uint4 *>(act_lds + static_cast<size_t>(m) * K + kg * 32);
        const uint4 a0 = ap[0], a1 = ap[1];
        int d = 0;
        d = __builtin_amdgcn_sdot4(static_cast<int>(a0.x), static_cast<int>(w[0]), d, false);
        d = __builtin_amdgcn_sdot4(static_cast<int>(a0.y), static_cast<int>(w[1]), d, false);
        d = __builtin_amdgcn_sdot4(static_cast<int>(a0.z), static_cast<int>(w[2]), d, false);
        d = __builtin_amdgcn_sdot4(static_cast<int>(a0.w), static_cast<int>(w[3]), d, false);
        d = __builtin_amdgcn_sdot4(static_cast<int>(a1.x), static_cast<int>(w[4]), d, false);
        d = __builtin_amdgcn_sdot4(static_cast<int>(a1.y), static_cast<int>(w[5]), d, false);
        d = __builtin_amdgcn_sdot4(static_cast<int>(a1.z), static_cast<int>(w[6]), d, false);
        d = __builtin_amdgcn_sdot4(static_cast<int>(a1.w), static_cast<int>(w[7]), d, false);
        acc[m] += LPBQ ? d * f : d;
        if (A16) {
          const uint4 *lp = reinterpret_cast<const uint4 *>(act_lds + static_cast<size_t>(M + m) * K + kg * 32);
          const uint4 b0 = lp[0], b1 = lp[1];
          int e = 0;
          e = __builtin_amdgcn_sdot4(static_cast<int>(b0.x), static_cast<int>(w[0]), e, false);
          e = __builtin_amdgcn_sdot4(static_cast<int>(b0.y), static_cast<int>(w[1]), e, false);
          e = __builtin_amdgcn_sdot4(static_cast<int>(b0.z), static_cast<int>(w[2]), e, false);
          e = __builtin_amdgcn_sdot4(static_cast<int>(b0.w), static_cast<int>(w[3]), e, false);
          e = __builtin_amdgcn_sdot4(static_cast<int>(b1.x), static_cast<int>(w[4]), e, false);
          e = __builtin_amdgcn_sdot4(static_cast<int>(b1.y), static_cast<int>(w[5]), e, false);
          e = __builtin_amdgcn_sdot4(static_cast<int>(b1.z), static_cast<int>(w[6]), e, false);
          e = __builtin_amdgcn_sdot4(static_cast<int>(b1.w), static_cast<int>(w[7]), e, false);
          acc2[m] += LPBQ ? e * f : e;
        }
        }
      }
    }
    // reduce over the 4 k-group lanes of each column
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      acc[m] += __shfl_xor(acc[m], 16, 64);
      acc[m] += __shfl_xor(acc[m], 32, 64);
      if (A16) {
        acc2[m] += __shfl_xor(acc2[m], 16, 64);
        acc2[m] += __shfl_xor(acc2[m], 32, 64);
      }
    }
    // requantise: lanes 0..15 own one column each
    uint32_t amb_mask = 0;
    if (sub == 0 && n < g.N) {
      double alpha = g.alpha[n];
      const double beta = g.beta[n], margin = g.margin[n], absb = g.absb[n];
      int64_t corr;
      double mr1 = 0.0;
      if (A16) {
        alpha *= static_cast<double>(g.mant[n]);
        corr = g.colsum[n] * static_cast<int64_t>(128 + 32768 - g.act_zp);
        mr1 = g.mr1[n];
      } else {
        corr = g.corr[n];
      }
#pragma unroll
      for (int m = 0; m < MM; ++m) {
        const int64_t S = A16 ? 256 * static_cast<int64_t>(acc[m]) + acc2[m] + corr : static_cast<int64_t>(acc[m]) + corr;
        const double t = fma(static_cast<double>(S), alpha, beta);
        const double fl = floor(t);
        const double slack = margin + (A16 ? mr1 * static_cast<double>(r1[m]) : 0.0) + 0x1p-48 * (fabs(t) + absb);
        const bool near_tie = fabs((t - fl) - 0.5) <= slack;
        const double lo = fmin(fmax(fl, 0.0), static_cast<double>(g.out_qmax));
        const double hi = fmin(fmax(fl + 1.0, 0.0), static_cast<double>(g.out_qmax));
        const bool amb = near_tie && lo != hi;
        if (m < M && amb) amb_mask |= 1u << m;
        if (m < M && !amb) {
          const double o = fmin(fmax(rint(t), 0.0), static_cast<double>(g.out_qmax));
          const size_t idx = static_cast<size_t>(m) * g.N + n;
          if (g.out16)
            static_cast<uint16_t *>(g.out)[idx] = static_cast<uint16_t>(o);
          else
            static_cast<uint8_t *>(g.out)[idx] = static_cast<uint8_t>(o);
        }
      }
    }
    // exact fixup of ambiguous outputs, one wave-cooperative dot product each
    for (int src = 0; src < 16; ++src) {
      uint32_t mask = __shfl(amb_mask, src, 64);
      while (mask) {
        const int m = __ffs(mask) - 1;
        mask &= mask - 1;
        gemv_fixup<A16, FMT, LPBQ>(g, m, grp * 16 + src, lane);
      }
    }
  }
}

template <bool A16, int FMT, bool LPBQ>
qh_status launch_mm(const GemvArgs &g, hipStream_t stream) {
  const int planes = A16 ? 2 : 1;
  const size_t lds = static_cast<size_t>(planes) * g.M * g.K;
  const int groups = g.N / 16;
  int blocks = (groups + 3) / 4;
  if (blocks > 512) blocks = 512;
  dim3 grid(blocks), block(kGemvThreads);
#define QH_GEMV_LAUNCH(MMV)                                                                                  \
  do {                                                                                                       \
    hipError_t e_ = hipFuncSetAttribute(reinterpret_cast<const void *>(&qmm_gemv_kernel<A16, FMT, LPBQ, MMV>), \
                                        hipFuncAttributeMaxDynamicSharedMemorySize, kGemvMaxLds);            \
    if (e_ != hipSuccess) return hip_fail(e_, "hipFuncSetAttribute(qmm_gemv_kernel)");                       \
    hipLaunchKernelGGL((qmm_gemv_kernel<A16, FMT, LPBQ, MMV>), grid, block, lds, stream, g);                 \
  } while (0)
  if (g.M <= 1)
    QH_GEMV_LAUNCH(1);
  else if (g.M <= 4)
    QH_GEMV_LAUNCH(4);
  else
    QH_GEMV_LAUNCH(16);
#undef QH_GEMV_LAUNCH
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return hip_fail(err, "qmm_gemv_kernel launch");
  return QH_STATUS_OK;
}

}  // namespace

qh_status launch_qmm_gemv(const qh_qmm_prepared *p, int m, const void *act, void *out, hipStream_t stream) {
  const QmmShape &sh = p->shape;
  const QmmDevice &D = p->dev;
  const int planes = sh.act_bits == 16 ? 2 : 1;
  if (m > 16) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "GEMV path supports M <= 16 (got %d)", m);
  if (static_cast<size_t>(planes) * m * sh.K > static_cast<size_t>(kGemvMaxLds))
    return fail(QH_STATUS_SHAPE_UNSUPPORTED, "GEMV path: M*K*planes = %zu bytes exceeds LDS staging (%d)",
                static_cast<size_t>(planes) * m * sh.K, kGemvMaxLds);
  GemvArgs g{};
  g.act = static_cast<const uint8_t *>(act);
  g.out = out;
  g.w = D.gemv_tiles;
  g.lpbq = D.gemv_lpbq;
  g.alpha = D.alpha;
  g.beta = D.beta;
  g.margin = D.margin;
  g.absb = D.absb;
  g.bias_deq = D.bias_deq;
  g.mr1 = D.gemv_margin_r1;
  g.corr = D.corr;
  g.mant = D.mant;
  g.colsum = D.colsum;
  g.s32 = D.s32;
  g.M = m;
  g.N = sh.N;
  g.K = sh.K;
  g.KG = sh.K / 32;
  g.nblk = sh.lpbq_block ? sh.K / sh.lpbq_block : 0;
  g.bs_shift = sh.lpbq_block == 64 ? 6 : 5;
  g.act_zp = sh.act_zp;
  g.out_zp = sh.out_zp;
  g.out_qmax = (1 << sh.out_bits) - 1;
  g.out16 = sh.out_bits == 16;
  g.sA = sh.act_scale;
  g.sO = sh.out_scale;
  const bool a16 = sh.act_bits == 16;
  const bool lpbq = sh.wfmt == QH_WEIGHT_I4_LPBQ;
  if (!a16) {
    if (sh.gemv_fmt == kTileI8) return launch_mm<false, kTileI8, false>(g, stream);
    if (lpbq) return launch_mm<false, kTileI4, true>(g, stream);
    return launch_mm<false, kTileI4, false>(g, stream);
  }
  if (sh.gemv_fmt == kTileI8) return launch_mm<true, kTileI8, false>(g, stream);
  if (lpbq) return launch_mm<true, kTileI4, true>(g, stream);
  return launch_mm<true, kTileI4, false>(g, stream);
}

}  // namespace qh
