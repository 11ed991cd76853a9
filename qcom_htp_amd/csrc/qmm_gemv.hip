// Decode-shape (M <= 16) quantized GEMV: HBM streaming of packed weights with dwordx4 loads and
// wavefront reductions; the k-group products are int8 dot4 MACs (v_dot4_i32_i8) for up to 4
// rows and i8 matrix-core products (v_mfma_i32_16x16x32_i8) for 5..16 rows.
//
// Weight stream layout (prepared once): [N/16 column groups][K/32 k-groups][16 columns][bytes],
// 16 B per (column, k-group) for int4 (byte j: low nibble k=j, high nibble k=j+16,
// offset-binary u = code + 8) or 32 B for int8.  One wave instruction reads 4 k-groups x 16
// columns = 1 KiB (int4) / 2 KiB (int8) of contiguous HBM.  LPBQ block scales are streamed as
// [N/16][K/block][16] bytes and read by each lane beside its weight words.
//
// Work split: a workgroup (4 waves) owns one 16-column group at a time and splits its K
// between all 256 lanes: lane (sub, col) of wave w takes the k-groups kg = 4 (w + 4 i) + sub,
// so every wave instruction is one contiguous KiB and a lane issues all of its loads (8 at
// K = 4096) before it uses any.  With one group per workgroup every byte of the matrix is
// requested at once, which is what an HBM-bound stream needs.
//
// Arithmetic: activations are staged once per workgroup in LDS as signed int8 planes
// (a - 128 for 8-bit; hi / lo' bytes of a - 32768 for 16-bit) together with their sums over
// each 32-k group.  Two paths compute the k-group products, both exact in int32:
//   * up to 4 rows (dot4): int4 codes are used as the unsigned nibble u = code + 8 (a mask, no
//     sign extension): sum_k a'_k (u_k - 8) f = f (dot4(a', u) - 8 sum_k a'_k) per k-group
//     (f = the LPBQ block scale, 1 otherwise);
//   * 5..16 rows (matrix core): the weight words of a lane are the B operand of
//     v_mfma_i32_16x16x32_i8 and the staged rows the A operand; int4 codes are widened to int8
//     in registers with the block scale folded in, (u f + 128 - 8 f) ^ 0x80 per byte, which needs
//     u f <= 240 and 8 f <= 128, i.e. f <= 16 (the range prepare accepts).
// The four waves' partial sums meet in LDS; each output is then requantised by one thread
// with the GEMM's rounding rules (t in float64, exact fixup of outputs within the certified
// margin of a rounding boundary).

#include <atomic>

#include "gemv_common.h"

namespace qh {
namespace {

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / 64;
constexpr int kGemvMaxDynLds = 139 * 1024;  // activation planes + k-group sums (+ <= 21 KB static)
constexpr int kU = kGemvKU;                  // k-groups per lane per batch (loads in flight)

struct GemvArgs {
  const uint8_t *act;
  void *out;
  const uint8_t *w;      // GEMV stream
  const uint8_t *lpbq;   // block scales, gemv_scale_index layout
  const double *alpha, *beta, *margin, *absb, *bias_deq, *mr1, *mlo;
  const double *alpha_e, *margin_exact;  // exact integer fixup (8-bit activations)
  const int64_t *corr, *mant, *colsum, *colsum_r;
  const float *s32;
  int M, N, K, KG, nbatch, sub_shift;
  int act_zp, out_zp, out_qmax, out16;
  int ars;       // LDS row stride of the staged activation planes, bytes: K + 16 (the 16 rows
                 // one 16-byte read instruction spans then fall on distinct banks)
  int off_asum;  // byte offset of the k-group sums in dynamic LDS
  int off_fixw;  // byte offset of the fixup columns' weight words (register-held fixup)
  double sA, sO;
};

__device__ __forceinline__ long as_long(uint32_t lo, uint32_t hi) {
  return static_cast<long>((static_cast<unsigned long>(hi) << 32) | lo);
}

// Exact float64 recomputation of output (m, n) by a whole wave, term by term as the reference
// oracle forms it: sum_k fl64((a_k - zp) * sA) * fl32(w_k * s32), + bias_deq, / sO, + out_zp.
// The activations come from the staged LDS planes, or (GA, 8-bit) from the activation matrix.
// Kept lean on purpose: the kernel's register budget is the maximum over all of its code, and
// this rare path must not lower the occupancy of the stream.
template <bool A16, int FMT, bool LPBQ, bool GA = false>
__device__ void gemv_fixup(const GemvArgs &g, const uint8_t *lds, int m, int n, int lane) {
  constexpr int WB = FMT == kTileI4 ? 16 : 32;
  const float sc = g.s32[n];
  const int KG = g.KG;
  const uint8_t *const wcol = g.w + (static_cast<size_t>(n / 16) * KG * 16 + (n % 16)) * WB;
  // a - zp = plane value + off (8-bit: a - 128; 16-bit: 256 hi + lo' with a - 32768 - 128)
  const int off = (A16 ? 32768 + 128 : 128) - g.act_zp;
  double s = 0.0;
  // a lane's k-groups (up to kPre of them: all of them for K <= 8192) are requested before any
  // is used, so the pass costs one memory round trip
  constexpr int kPre = 4;
  for (int kg0 = lane; kg0 < KG; kg0 += 64 * kPre) {
    uint32_t wd[kPre][WB / 4];
    int fs[kPre];
#pragma unroll
    for (int u = 0; u < kPre; ++u) {
      const int kg = min(kg0 + 64 * u, KG - 1);
      const uint4 *p = reinterpret_cast<const uint4 *>(wcol + static_cast<size_t>(kg) * 16 * WB);
#pragma unroll
      for (int q = 0; q < WB / 16; ++q) {
        const uint4 v = p[q];
        wd[u][4 * q] = v.x; wd[u][4 * q + 1] = v.y; wd[u][4 * q + 2] = v.z; wd[u][4 * q + 3] = v.w;
      }
      fs[u] = LPBQ ? g.lpbq[gemv_scale_index_kg(n, kg, g.nbatch, g.sub_shift)] : 1;
    }
#pragma unroll
    for (int u = 0; u < kPre; ++u) {
      const int kg = kg0 + 64 * u;
      if (kg >= KG) break;
      const int f = fs[u];
      const int8_t *hp = reinterpret_cast<const int8_t *>(lds + static_cast<size_t>(m) * g.ars + kg * 32);
      const int8_t *lp = reinterpret_cast<const int8_t *>(lds + static_cast<size_t>(g.M + m) * g.ars + kg * 32);
      const uint8_t *gp = g.act + static_cast<size_t>(m) * g.K + kg * 32;
      const uint16_t *gp16 = reinterpret_cast<const uint16_t *>(g.act) + static_cast<size_t>(m) * g.K + kg * 32;
#pragma unroll 4
      for (int j = 0; j < 32; ++j) {
        int w;
        if (FMT == kTileI4) {
          const uint32_t byte = (wd[u][(j & 15) >> 2] >> (8 * (j & 3))) & 0xFFu;
          w = ((j < 16 ? (byte & 15u) : (byte >> 4)) - 8) * f;
        } else {
          w = static_cast<int8_t>((wd[u][j >> 2] >> (8 * (j & 3))) & 0xFFu);
        }
        const int a = GA ? (A16 ? static_cast<int>(gp16[j]) : static_cast<int>(gp[j])) - g.act_zp
                         : (A16 ? 256 * static_cast<int>(hp[j]) + lp[j] : static_cast<int>(hp[j])) + off;
        const float wf = static_cast<float>(w) * sc;
        s = fma(static_cast<double>(a) * g.sA, static_cast<double>(wf), s);
      }
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
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

// Exact float64 recomputation of up to kFixBatch outputs at once by the whole workgroup, from
// weights that the workgroup already holds: entry e's column weight words and LPBQ scales sit
// in LDS at fixw + e KG WB ([KG][WB bytes]) and fixs + e KG ([KG]), the activations in the
// staged planes.  Thread t takes 16 terms of each of its (k-group, half) pairs for every entry
// (independent accumulation chains); the partial sums meet in LDS.
constexpr int kFixBatch = 8;
template <bool A16, int FMT, bool LPBQ>
__device__ void gemv_fixup_batch(const GemvArgs &g, const uint8_t *lds, const uint8_t *fixw, const uint8_t *fixs,
                                 double *dred, const uint16_t *list, int nb, int grp, int t) {
  constexpr int WB = FMT == kTileI4 ? 16 : 32;
  const int KG = g.KG;
  const int off = (A16 ? 32768 + 128 : 128) - g.act_zp;
  double s[kFixBatch];
  float sc[kFixBatch];
  int mrow[kFixBatch];
#pragma unroll
  for (int e = 0; e < kFixBatch; ++e) {
    s[e] = 0.0;
    const int tt = list[e < nb ? e : 0];
    mrow[e] = tt >> 4;
    sc[e] = g.s32[grp * 16 + (tt & 15)];
  }
  for (int u = t; u < 2 * KG; u += kGemvThreads) {
    const int kg = u >> 1, h = u & 1;  // terms k = 32 kg + 16 h + j, j < 16
#pragma unroll
    for (int e = 0; e < kFixBatch; ++e) {
      if (e >= nb) break;
      const uint4 v = *reinterpret_cast<const uint4 *>(fixw + (static_cast<size_t>(e) * KG + kg) * WB +
                                                       (FMT == kTileI4 ? 0 : 16 * h));
      const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
      const int f = LPBQ ? fixs[e * KG + kg] : 1;
      const int8_t *hp = reinterpret_cast<const int8_t *>(lds + static_cast<size_t>(mrow[e]) * g.ars + kg * 32 + 16 * h);
      const int8_t *lp = reinterpret_cast<const int8_t *>(lds + static_cast<size_t>(g.M + mrow[e]) * g.ars + kg * 32 + 16 * h);
#pragma unroll 4
      for (int j = 0; j < 16; ++j) {
        const uint32_t byte = (wd[j >> 2] >> (8 * (j & 3))) & 0xFFu;
        const int w = FMT == kTileI4 ? ((h ? (byte >> 4) : (byte & 15u)) - 8) * f : static_cast<int8_t>(byte);
        const int a = (A16 ? 256 * static_cast<int>(hp[j]) + lp[j] : static_cast<int>(hp[j])) + off;
        const float wf = static_cast<float>(w) * sc[e];
        s[e] = fma(static_cast<double>(a) * g.sA, static_cast<double>(wf), s[e]);
      }
    }
  }
#pragma unroll
  for (int e = 0; e < kFixBatch; ++e) {
    if (e >= nb) break;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) s[e] += __shfl_xor(s[e], o, 64);
    if ((t & 63) == 0) dred[e * kGemvWaves + (t >> 6)] = s[e];
  }
  lds_barrier();
  if (t < nb) {
    const int tt = list[t];
    const int m = tt >> 4, n = grp * 16 + (tt & 15);
    const double tot = dred[t * kGemvWaves] + dred[t * kGemvWaves + 1] + dred[t * kGemvWaves + 2] + dred[t * kGemvWaves + 3];
    const double tv = (tot + g.bias_deq[n]) / g.sO + static_cast<double>(g.out_zp);
    const double o = fmin(fmax(rint(tv), 0.0), static_cast<double>(g.out_qmax));
    const size_t idx = static_cast<size_t>(m) * g.N + n;
    if (g.out16)
      static_cast<uint16_t *>(g.out)[idx] = static_cast<uint16_t>(o);
    else
      static_cast<uint8_t *>(g.out)[idx] = static_cast<uint8_t>(o);
  }
}

// Exact integer completion of listed outputs, 8-bit activations, by the whole workgroup (one
// output at a time).  With r_k = fl32(w_k M) - w_k M the float32 rounding residue of the
// dequantised weight in units of 2^E (w_k the integer weight, block scale included; M 2^E the
// column scale), D = sum_k (a_k - zp)(w_k M + r_k) = (sum_k a'_k w_k + corr) M + sum_k a'_k r_k
// + (128 - zp) sum_k r_k is an exact integer, so t = D alpha_e + beta carries only the oracle's
// own float64 noise (margin_exact).  Thread t takes the (k-group, half) pairs u = t, t + NT, ..
// (terms k = 32 kg + 16 h + j, j < 16, as gemv_fixup_batch).  Outputs still within that noise of
// a rounding boundary are moved to the front of the list for the term-by-term float64
// recomputation; their count is returned (to every thread).  GA: the activations are read from
// the activation matrix instead of the staged plane.
template <int FMT, bool LPBQ, int NT, bool GA>
__device__ int gemv_fixup_exact(const GemvArgs &g, const uint8_t *lds, uint16_t *list, int nfix, int grp, int t,
                                int (*ired)[NT / 64][2], int *cnt) {
  constexpr int WB = FMT == kTileI4 ? 16 : 32;
  const int KG = g.KG, lane = t & 63, wave = t >> 6;
  int nslow = 0;  // thread 0's count
  for (int e = 0; e < nfix; ++e) {
    const int tt = list[e];
    const int m = tt >> 4, n = grp * 16 + (tt & 15);
    // column constants first (thread 0 uses them after the reduction)
    const int Mi = static_cast<int>(g.mant[n]);
    int64_t corr = 0, csr = 0;
    double ae = 0.0, beta = 0.0, mex = 0.0, absb = 0.0;
    if (t == 0) {
      corr = g.corr[n];
      csr = g.colsum_r[n];
      ae = g.alpha_e[n];
      beta = g.beta[n];
      mex = g.margin_exact[n];
      absb = g.absb[n];
    }
    const uint8_t *const wcol = g.w + (static_cast<size_t>(n / 16) * KG * 16 + (n % 16)) * WB;
    int sw = 0, sr = 0;
    for (int u = t; u < 2 * KG; u += NT) {
      const int kg = u >> 1, h = u & 1;
      const uint4 v = *reinterpret_cast<const uint4 *>(wcol + static_cast<size_t>(kg) * 16 * WB + (FMT == kTileI4 ? 0 : 16 * h));
      const int f = LPBQ ? g.lpbq[gemv_scale_index_kg(n, kg, g.nbatch, g.sub_shift)] : 1;
      uint4 av;
      if constexpr (GA) {
        av = *reinterpret_cast<const uint4 *>(g.act + static_cast<size_t>(m) * g.K + kg * 32 + 16 * h);
        av.x ^= 0x80808080u; av.y ^= 0x80808080u; av.z ^= 0x80808080u; av.w ^= 0x80808080u;
      } else {
        av = *reinterpret_cast<const uint4 *>(lds + static_cast<size_t>(m) * g.ars + kg * 32 + 16 * h);
      }
      const uint32_t wd[4] = {v.x, v.y, v.z, v.w}, ad[4] = {av.x, av.y, av.z, av.w};
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const uint32_t byte = (wd[j >> 2] >> (8 * (j & 3))) & 0xFFu;
        const int w = FMT == kTileI4 ? (static_cast<int>(h ? (byte >> 4) : (byte & 15u)) - 8) * f : static_cast<int8_t>(byte);
        const int a = static_cast<int8_t>((ad[j >> 2] >> (8 * (j & 3))) & 0xFFu);
        const int x = w * Mi;  // |w| <= 127, M < 2^24: no overflow
        sw += a * w;
        sr += a * (static_cast<int>(static_cast<float>(x)) - x);
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      sw += __shfl_xor(sw, o, 64);
      sr += __shfl_xor(sr, o, 64);
    }
    if (lane == 0) {
      ired[e & 1][wave][0] = sw;
      ired[e & 1][wave][1] = sr;
    }
    lds_barrier();  // (double-buffered: iteration e + 2 rewrites this slot after the next barrier)
    if (t == 0) {
      int64_t SW = 0, SR = 0;
#pragma unroll
      for (int w = 0; w < NT / 64; ++w) {
        SW += ired[e & 1][w][0];
        SR += ired[e & 1][w][1];
      }
      const int64_t D = (SW + corr) * static_cast<int64_t>(Mi) + SR + static_cast<int64_t>(128 - g.act_zp) * csr;
      const double tv = fma(static_cast<double>(D), ae, beta);
      const double slack = mex + 0x1p-48 * (fabs(tv) + absb);
      const double fl = floor(tv);
      const double lo = fmin(fmax(fl, 0.0), static_cast<double>(g.out_qmax));
      const double hi = fmin(fmax(fl + 1.0, 0.0), static_cast<double>(g.out_qmax));
      if (fabs((tv - fl) - 0.5) <= slack && lo != hi) {
        list[nslow++] = static_cast<uint16_t>(tt);  // every thread has read entries <= e
      } else {
        const double o = fmin(fmax(rint(tv), 0.0), static_cast<double>(g.out_qmax));
        const size_t idx = static_cast<size_t>(m) * g.N + n;
        if (g.out16)
          static_cast<uint16_t *>(g.out)[idx] = static_cast<uint16_t>(o);
        else
          static_cast<uint8_t *>(g.out)[idx] = static_cast<uint8_t>(o);
      }
    }
  }
  if (t == 0) *cnt = nslow;
  lds_barrier();
  return *cnt;
}

// Staging of the activations, one (row, k-group) unit of 32 values at a time: the signed
// plane bytes and (int4 weights) the plane sums over the unit.  16-bit activations also add
// sum |a - zp| of each row into r1 (the bound of the float32-rounding residue term in the
// margin).  Loading and storing are separate so that the first unit's load can be issued
// ahead of the weight stream.
template <bool A16>
struct ActUnit {
  uint4 v[A16 ? 4 : 2];
};

template <bool A16>
__device__ __forceinline__ void load_unit(const GemvArgs &g, int u, ActUnit<A16> &r) {
  const int m = u / g.KG, kg = u - m * g.KG;
  const uint4 *src = A16 ? reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(g.act) + static_cast<size_t>(m) * g.K + kg * 32)
                         : reinterpret_cast<const uint4 *>(g.act + static_cast<size_t>(m) * g.K + kg * 32);
#pragma unroll
  for (int q = 0; q < (A16 ? 4 : 2); ++q) r.v[q] = src[q];
}

template <bool A16, int FMT>
__device__ __forceinline__ void store_unit(const GemvArgs &g, int u, ActUnit<A16> r, uint8_t *lds, uint32_t *r1) {
  const int M = g.M, KG = g.KG;
  const int m = u / KG, kg = u - m * KG;
  int16_t *asum = reinterpret_cast<int16_t *>(lds + g.off_asum);
  if (!A16) {
    uint4 v0 = r.v[0], v1 = r.v[A16 ? 1 : 1];
    v0.x ^= 0x80808080u; v0.y ^= 0x80808080u; v0.z ^= 0x80808080u; v0.w ^= 0x80808080u;
    v1.x ^= 0x80808080u; v1.y ^= 0x80808080u; v1.z ^= 0x80808080u; v1.w ^= 0x80808080u;
    uint4 *dst = reinterpret_cast<uint4 *>(lds + static_cast<size_t>(m) * g.ars + kg * 32);
    dst[0] = v0;
    dst[1] = v1;
    if (FMT == kTileI4) {
      int s = bsum4(v0.x, 0);
      s = bsum4(v0.y, s); s = bsum4(v0.z, s); s = bsum4(v0.w, s);
      s = bsum4(v1.x, s); s = bsum4(v1.y, s); s = bsum4(v1.z, s); s = bsum4(v1.w, s);
      asum[u] = static_cast<int16_t>(s);
    }
  } else {
    uint32_t hv[8], lv[8];
    uint32_t rs = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint4 v = r.v[q & (A16 ? 3 : 1)];
      const uint16_t *h = reinterpret_cast<const uint16_t *>(&v);
#pragma unroll
      for (int j = 0; j < 8; ++j) rs += static_cast<uint32_t>(abs(static_cast<int>(h[j]) - g.act_zp));
      v.x ^= 0x80808080u; v.y ^= 0x80808080u; v.z ^= 0x80808080u; v.w ^= 0x80808080u;
      hv[2 * q] = perm(v.y, v.x, 0x07050301u);
      hv[2 * q + 1] = perm(v.w, v.z, 0x07050301u);
      lv[2 * q] = perm(v.y, v.x, 0x06040200u);
      lv[2 * q + 1] = perm(v.w, v.z, 0x06040200u);
    }
    uint4 *dh = reinterpret_cast<uint4 *>(lds + static_cast<size_t>(m) * g.ars + kg * 32);
    uint4 *dl = reinterpret_cast<uint4 *>(lds + static_cast<size_t>(M + m) * g.ars + kg * 32);
    dh[0] = make_uint4(hv[0], hv[1], hv[2], hv[3]);
    dh[1] = make_uint4(hv[4], hv[5], hv[6], hv[7]);
    dl[0] = make_uint4(lv[0], lv[1], lv[2], lv[3]);
    dl[1] = make_uint4(lv[4], lv[5], lv[6], lv[7]);
    if (FMT == kTileI4) {
      int sh = 0, sl = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        sh = bsum4(hv[j], sh);
        sl = bsum4(lv[j], sl);
      }
      asum[u] = static_cast<int16_t>(sh);
      asum[M * KG + u] = static_cast<int16_t>(sl);
    }
    if (FMT != kTileI4) atomicAdd(&r1[m], rs);
  }
}

// 16 rows of 16-bit activations stage 128 KiB (one workgroup per compute unit) and need four
// product sets per weight word: their workgroups take 8 waves, waves w and w + 4 splitting the
// slots of one lane pattern, so that two waves per SIMD share the products.
template <bool A16, int MM>
constexpr int gemv_threads() {
  return MM == 16 && A16 ? 2 * kGemvThreads : kGemvThreads;
}

// RA (16 rows, K <= 16 kU k-groups; 16-bit activations with int4 codes): every lane keeps the A
// operands of its slots in registers (16-bit activations: both byte planes), loaded once from the
// activation matrix (the same for every group the workgroup takes), instead of staging the rows
// in LDS.
template <bool A16, int FMT, bool LPBQ, int MM, bool RA = false>
__global__ __launch_bounds__((gemv_threads<A16, MM>()), (MM == 16 ? (A16 ? 1 : 2) : 4)) void qmm_gemv_kernel(const GemvArgs g) {
  static_assert(!RA || (MM == 16 && (!A16 || FMT == kTileI4)), "register-held activations: 16 rows");
  constexpr int NT = gemv_threads<A16, MM>();
  constexpr bool kWide = NT > kGemvThreads;
  constexpr int kUw = kWide ? kU / 2 : kU;  // slots of a batch per wave
  // 16-bit activations with int4 codes also form sum_k hi'_k r_k (the residue products of the
  // high activation byte) exactly, from the residue tables of the group's 16 columns
  constexpr bool HR = A16 && FMT == kTileI4;
  extern __shared__ uint4 smem[];
  uint8_t *const lds = reinterpret_cast<uint8_t *>(smem);
  __shared__ int red[kGemvWaves][MM][16];
  __shared__ int red2[A16 ? kGemvWaves : 1][A16 ? MM : 1][16];
  __shared__ int red3[HR ? kGemvWaves : 1][HR ? MM : 1][16];
  // 16 rows (matrix core) also form sum_k lo'_k r_k, so their dot products are exact
  constexpr bool LR = HR && MM == 16;
  __shared__ int red4[LR ? kGemvWaves : 1][LR ? MM : 1][16];
  __shared__ uint4 rtab[HR ? 16 * kRtabF : 1];  // [column][block scale f = 0 .. 16]
  __shared__ uint32_t r1[16];
  __shared__ uint16_t fix_list[MM * 16];
  __shared__ int fix_cnt;
  __shared__ double dred[kFixBatch * kGemvWaves];
  __shared__ int ired[A16 ? 1 : 2][A16 ? 1 : NT / 64][2];

  const int t = threadIdx.x, lane = t & 63;
  // the wave of the lane pattern (k-groups 4 (wave + 4 i) + sub) and, 8 waves, the half of the
  // batch's slots this wave takes
  const int wave = (t >> 6) & (kGemvWaves - 1), shalf = kWide ? (t >> 8) : 0;
  const int M = g.M, KG = g.KG;
  constexpr int WB = FMT == kTileI4 ? 16 : 32;  // stream bytes per (column, k-group)
  const int16_t *const asum = reinterpret_cast<const int16_t *>(lds + g.off_asum);
  const int col = lane & 15, sub = lane >> 4;
  const int groups = g.N / 16;
  const int iters = (KG + 15) / 16;  // k-group slots per lane (some past KG when KG % 16 != 0)
  // One batch of kU k-groups per lane: the weight words and their LPBQ block scales (one
  // 8-byte load of the lane's kU scales).
  constexpr int WV = FMT == kTileI4 ? 1 : 2;
  uint4 wv[kUw][WV];
  uint2 fsv = make_uint2(0x01010101u, 0x01010101u);
  constexpr bool kLoop = MM == 16;  // 16 rows: workgroups loop over groups
  // Straight-line loads (indices clamped, results of slots past KG discarded) keep every load
  // of a batch in one basic block, so they issue back to back and their waits count down.
  // Buffer loads; a group that does not exist (grp >= groups) gets a resource of 0 bytes, so
  // its loads return zeros without touching memory and every load count stays the same.
  const uint32_t wbytes = static_cast<uint32_t>(KG) * 16 * WB;
  const uint32_t lbytes = LPBQ ? static_cast<uint32_t>(gemv_scale_index(groups, 0, g.nbatch, 0, 0, 4 >> g.sub_shift, 0, 0)) : 0u;
  auto issue_into = [&](int grp, int i0, auto &dst, uint2 &fdst) {
    const bool real = grp < groups;
    const int gi = real ? grp : 0;
    const auto rw = rsrc(g.w + static_cast<size_t>(gi) * wbytes, real ? wbytes : 0u);
    if (LPBQ)  // first: slot 0 needs it, and loads complete in order
      fdst = bload8(rsrc(g.lpbq, real ? lbytes : 0u),
                    static_cast<uint32_t>(gemv_scale_index(gi, i0 / kU, g.nbatch, wave, sub >> g.sub_shift, 4 >> g.sub_shift, col, 0)));
#pragma unroll
    for (int ii = 0; ii < kUw; ++ii) {
      const int kg = min(4 * (wave + 4 * (i0 + ii + shalf * kUw)) + sub, KG - 1);
      const uint32_t off = (static_cast<uint32_t>(kg) * 16 + col) * WB;
      dst[ii][0] = bload16<kNT>(rw, off);
      if (FMT != kTileI4) dst[ii][WV - 1] = bload16<kNT>(rw, off + 16);
    }
  };
  auto issue = [&](int grp, int i0) { issue_into(grp, i0, wv, fsv); };
  // Per-output epilogue constants of thread t's output (row t / 16, column t % 16 of the
  // group), requested together with the group's first batch of weights.
  struct Epi {
    double alpha, beta, margin, absb, mr1;
    int64_t corr, mant, csr;
  } ep{};
  const bool owns_out = t < MM * 16 && (t >> 4) < M;
  auto epi_of = [&](int grp) {  // every thread loads (its column exists), only owners use it
    Epi e{};
    const int n = grp * 16 + (t & 15);
    e.alpha = g.alpha[n];
    e.beta = g.beta[n];
    e.margin = g.margin[n];
    e.absb = g.absb[n];
    if (A16) {
      e.corr = g.colsum[n];
      e.mr1 = HR ? g.mlo[n] : g.mr1[n];
      e.mant = g.mant[n];
      if (HR) e.csr = g.colsum_r[n];
    } else {
      e.corr = g.corr[n];
    }
    return e;
  };
  auto load_epi = [&](int grp) { ep = epi_of(grp); };
  // Residue tables of a group's 16 columns (HR): the column mantissas of the table entries this
  // thread fills, (column, f) = (e / kRtabF, e % kRtabF) for e = t and t + 256
  constexpr int kRtabE = (16 * kRtabF + NT - 1) / NT;
  auto rtab_mant = [&](int grp, int (&mt)[kRtabE]) {
#pragma unroll
    for (int j = 0; j < kRtabE; ++j) {
      const int e = min(t + j * NT, 16 * kRtabF - 1);
      mt[j] = static_cast<int>(g.mant[grp * 16 + e / kRtabF]);
    }
  };
  int rmt[HR ? kRtabE : 1] = {};
  // The first activation unit and the first batch of weights are requested before anything
  // waits: the staging then overlaps the weight stream.
  ActUnit<A16> au;
  const int units = M * KG;
  // further units: for 16 rows a batch of loads is issued before its first LDS store (a
  // load-then-store loop would wait for every load in turn); fewer rows have one or two units
  // per thread and no registers to spare under their occupancy bound
  constexpr int kStageB = MM < 16 ? 1 : (A16 ? 4 : 8);
  int ustart = t + NT;  // the first unit of the staging loop below
  // RA: activation row lane % 16, k-group of the wave's slot ii: 8-bit rows 32 bytes (a - 128);
  // 16-bit rows the high-byte plane hi' = hi - 128 ([0], [1]) and the low-byte plane
  // lo' = lo - 128 ([2], [3]), a - 32896 = 256 hi' + lo'
  uint4 areg[RA ? kUw : 1][A16 ? 4 : 2];
  if constexpr (RA) {
    // the activation fragments first (L2: every workgroup reads the same rows), then the
    // per-group constants and the first group's weights (HBM)
    const int arow = min(lane & 15, M - 1);  // rows past M repeat row M - 1 (never stored)
#pragma unroll
    for (int ii = 0; ii < kUw; ++ii) {
      const int kg = min(4 * (wave + 4 * (ii + shalf * kUw)) + sub, KG - 1);
      if constexpr (A16) {
        const uint4 *p = reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(g.act) +
                                                         static_cast<size_t>(arow) * g.K + kg * 32);
#pragma unroll
        for (int q = 0; q < 4; ++q) areg[ii][q] = p[q];
      } else {
        const uint4 *p = reinterpret_cast<const uint4 *>(g.act + static_cast<size_t>(arow) * g.K + kg * 32);
        areg[ii][0] = p[0];
        areg[ii][1] = p[1];
      }
    }
    if constexpr (HR) rtab_mant(blockIdx.x, rmt);
    load_epi(blockIdx.x);
    issue(blockIdx.x, 0);
    if (t < 16) r1[t] = 0;
    if (t == 0) fix_cnt = 0;
#pragma unroll
    for (int ii = 0; ii < kUw; ++ii) {
      if constexpr (A16) {
        // 8 u16 per uint4: XOR 0x80 on both bytes, then the high and the low bytes of k .. k + 31
        uint32_t hv[8], lv[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          uint4 v = areg[ii][q];
          v.x ^= 0x80808080u; v.y ^= 0x80808080u; v.z ^= 0x80808080u; v.w ^= 0x80808080u;
          hv[2 * q] = perm(v.y, v.x, 0x07050301u);
          hv[2 * q + 1] = perm(v.w, v.z, 0x07050301u);
          lv[2 * q] = perm(v.y, v.x, 0x06040200u);
          lv[2 * q + 1] = perm(v.w, v.z, 0x06040200u);
        }
        areg[ii][0] = make_uint4(hv[0], hv[1], hv[2], hv[3]);
        areg[ii][1] = make_uint4(hv[4], hv[5], hv[6], hv[7]);
        areg[ii][2] = make_uint4(lv[0], lv[1], lv[2], lv[3]);
        areg[ii][3] = make_uint4(lv[4], lv[5], lv[6], lv[7]);
      } else {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          areg[ii][q].x ^= 0x80808080u; areg[ii][q].y ^= 0x80808080u;
          areg[ii][q].z ^= 0x80808080u; areg[ii][q].w ^= 0x80808080u;
        }
      }
    }
    ustart = units;  // nothing to stage
  } else if constexpr (kLoop) {
    // 16 rows: the staged activations (L2) are requested first, then the per-group constants
    // and the first group's weights (HBM): one counter tracks the loads in order, so the staging
    // waits for its own loads only and overlaps the weights' latency.
    ActUnit<A16> s0[kStageB];
#pragma unroll
    for (int j = 0; j < kStageB; ++j) load_unit<A16>(g, min(t + j * NT, units - 1), s0[j]);
    if constexpr (HR) rtab_mant(blockIdx.x, rmt);
    load_epi(blockIdx.x);
    issue(blockIdx.x, 0);
    if (t < 16) r1[t] = 0;
    if (t == 0) fix_cnt = 0;
    lds_barrier();
#pragma unroll
    for (int j = 0; j < kStageB; ++j)
      if (t + j * NT < units) store_unit<A16, FMT>(g, t + j * NT, s0[j], lds, r1);
    ustart = t + kStageB * NT;
  } else {
    load_unit<A16>(g, min(t, units - 1), au);
    issue(blockIdx.x, 0);  // the launch never has more workgroups than groups
    load_epi(blockIdx.x);
    if (t < 16) r1[t] = 0;
    if (t == 0) fix_cnt = 0;
    lds_barrier();
    if (t < units) store_unit<A16, FMT>(g, t, au, lds, r1);
  }
  for (int u0 = ustart; u0 < units; u0 += NT * kStageB) {
    ActUnit<A16> ub[kStageB];
#pragma unroll
    for (int j = 0; j < kStageB; ++j) load_unit<A16>(g, min(u0 + j * NT, units - 1), ub[j]);
#pragma unroll
    for (int j = 0; j < kStageB; ++j)
      if (u0 + j * NT < units) store_unit<A16, FMT>(g, u0 + j * NT, ub[j], lds, r1);
  }
  lds_barrier();

  // Workgroups loop over groups only for 16 rows (whose staging is amortised over several
  // groups); otherwise each workgroup owns exactly one group.
  // 16 rows: the k-group products run on the matrix core (the dot4 path reads every activation
  // row from LDS once per weight word and is LDS bound there)
  constexpr bool kMfma = MM == 16;
  for (int grp = blockIdx.x; grp < groups; grp += gridDim.x) {
    if constexpr (HR) {
      // residue tables of this group's 16 columns, one (column, f) per thread and step
      if constexpr (kLoop) {
        // mantissas requested with the previous group's epilogue constants
#pragma unroll
        for (int j = 0; j < kRtabE; ++j)
          if (t + j * NT < 16 * kRtabF) rtab[t + j * NT] = resid_table(rmt[j], (t + j * NT) % kRtabF);
      } else {
        for (int e = t; e < 16 * kRtabF; e += NT)
          rtab[e] = resid_table(static_cast<int>(g.mant[grp * 16 + e / kRtabF]), e % kRtabF);
      }
      lds_barrier();
    }
    int acc[kMfma ? 1 : MM], acc2[A16 && !kMfma ? MM : 1], acc3[HR && !kMfma ? MM : 1];
#pragma unroll
    for (int m = 0; m < (kMfma ? 1 : MM); ++m) {
      acc[m] = 0;
      if (A16 && !kMfma) acc2[m] = 0;
      if (HR && !kMfma) acc3[m] = 0;
    }
    v4i macc = {0, 0, 0, 0}, macc2 = {0, 0, 0, 0}, macc3 = {0, 0, 0, 0}, macc4 = {0, 0, 0, 0};
    // (RA: the host guarantees one batch, iters <= kU)
    for (int i0 = 0; i0 < (RA ? 1 : iters); i0 += kU) {
      if (i0 > 0) issue(grp, i0);
      if constexpr (kMfma) {
        // 16 rows: v_mfma_i32_16x16x32_i8 over the k-groups of the wave's 4 lane quarters.  In
        // product j, lane quarter sub contributes k = 32 kg + 8 j .. + 7 of its own k-group kg to
        // the B operand (its column) and to the A operand (activation row lane & 15), so the
        // four products j cover each lane quarter's 32 k.
        const int mrow = min(lane & 15, M - 1);  // rows past M repeat row M - 1 (never stored)
#pragma unroll
        for (int ii = 0; ii < kUw; ++ii) {
          const int i = ii + shalf * kUw;  // the slot of the batch
          const int kg_raw = 4 * (wave + 4 * (i0 + i)) + sub;
          const bool valid = kg_raw < KG;
          const int kg = valid ? kg_raw : KG - 1;
          uint32_t b[8];  // B operand dwords of products j = 0..3 (two each)
          uint32_t rr[HR ? 8 : 1];  // residues of the same 32 weights
          if (FMT == kTileI4) {
            const uint32_t f = valid ? (LPBQ ? ((i < 4 ? fsv.x : fsv.y) >> (8 * (i & 3))) & 0xFFu : 1u) : 0u;
            const uint4 v = wv[ii][0];
            if constexpr (HR) {
              const uint4 tab = rtab[col * kRtabF + f];
              rr[0] = resid4(v.x & 0x0F0F0F0Fu, tab); rr[1] = resid4(v.y & 0x0F0F0F0Fu, tab);
              rr[2] = resid4(v.z & 0x0F0F0F0Fu, tab); rr[3] = resid4(v.w & 0x0F0F0F0Fu, tab);
              rr[4] = resid4((v.x >> 4) & 0x0F0F0F0Fu, tab); rr[5] = resid4((v.y >> 4) & 0x0F0F0F0Fu, tab);
              rr[6] = resid4((v.z >> 4) & 0x0F0F0F0Fu, tab); rr[7] = resid4((v.w >> 4) & 0x0F0F0F0Fu, tab);
            }
            // byte j of the 16: k = j (low nibble), k = j + 16 (high nibble)
            b[0] = w4_to_i8(v.x & 0x0F0F0F0Fu, f); b[1] = w4_to_i8(v.y & 0x0F0F0F0Fu, f);
            b[2] = w4_to_i8(v.z & 0x0F0F0F0Fu, f); b[3] = w4_to_i8(v.w & 0x0F0F0F0Fu, f);
            b[4] = w4_to_i8((v.x >> 4) & 0x0F0F0F0Fu, f); b[5] = w4_to_i8((v.y >> 4) & 0x0F0F0F0Fu, f);
            b[6] = w4_to_i8((v.z >> 4) & 0x0F0F0F0Fu, f); b[7] = w4_to_i8((v.w >> 4) & 0x0F0F0F0Fu, f);
          } else {
            const uint4 v0 = wv[ii][0], v1 = wv[ii][FMT == kTileI4 ? 0 : 1];
            const uint32_t mk = valid ? 0xFFFFFFFFu : 0u;
            b[0] = v0.x & mk; b[1] = v0.y & mk; b[2] = v0.z & mk; b[3] = v0.w & mk;
            b[4] = v1.x & mk; b[5] = v1.y & mk; b[6] = v1.z & mk; b[7] = v1.w & mk;
          }
          // 16-byte reads: with the padded row stride the 16 rows of a quarter hit distinct banks
          uint4 ah0, ah1;
          if constexpr (RA) {
            ah0 = areg[ii][0];
            ah1 = areg[ii][1];
          } else {
            const uint4 *ap4 = reinterpret_cast<const uint4 *>(lds + static_cast<size_t>(mrow) * g.ars + kg * 32);
            ah0 = ap4[0];
            ah1 = ap4[1];
          }
          const uint2 ah[4] = {make_uint2(ah0.x, ah0.y), make_uint2(ah0.z, ah0.w), make_uint2(ah1.x, ah1.y), make_uint2(ah1.z, ah1.w)};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint2 a = ah[j];
            macc = __builtin_amdgcn_mfma_i32_16x16x32_i8(as_long(a.x, a.y), as_long(b[2 * j], b[2 * j + 1]), macc, 0, 0, 0);
            if constexpr (HR)
              macc3 = __builtin_amdgcn_mfma_i32_16x16x32_i8(as_long(a.x, a.y), as_long(rr[2 * j], rr[2 * j + 1]), macc3, 0, 0, 0);
          }
          if (A16) {
            uint4 al0, al1;
            if constexpr (RA) {
              al0 = areg[ii][A16 ? 2 : 0];
              al1 = areg[ii][A16 ? 3 : 1];
            } else {
              const uint4 *lp4 = reinterpret_cast<const uint4 *>(lds + static_cast<size_t>(M + mrow) * g.ars + kg * 32);
              al0 = lp4[0];
              al1 = lp4[1];
            }
            const uint2 al[4] = {make_uint2(al0.x, al0.y), make_uint2(al0.z, al0.w), make_uint2(al1.x, al1.y), make_uint2(al1.z, al1.w)};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const uint2 a = al[j];
              macc2 = __builtin_amdgcn_mfma_i32_16x16x32_i8(as_long(a.x, a.y), as_long(b[2 * j], b[2 * j + 1]), macc2, 0, 0, 0);
              if constexpr (LR)
                macc4 = __builtin_amdgcn_mfma_i32_16x16x32_i8(as_long(a.x, a.y), as_long(rr[2 * j], rr[2 * j + 1]), macc4, 0, 0, 0);
            }
          }
        }
        continue;
      }
#pragma unroll
      for (int i = 0; i < kU; ++i) {
        const int kg_raw = 4 * (wave + 4 * (i0 + i)) + sub;
        const bool valid = kg_raw < KG;  // slot past the end of K: zero weights
        const int kg = valid ? kg_raw : KG - 1;
        uint32_t w[8];
        if (FMT == kTileI4) {
          const uint4 v = wv[i][0];
          const uint32_t m4 = valid ? 0x0F0F0F0Fu : 0u;
          w[0] = v.x & m4; w[1] = v.y & m4; w[2] = v.z & m4; w[3] = v.w & m4;
          w[4] = (v.x >> 4) & m4; w[5] = (v.y >> 4) & m4; w[6] = (v.z >> 4) & m4; w[7] = (v.w >> 4) & m4;
        } else {
          const uint4 v0 = wv[i][0], v1 = wv[i][FMT == kTileI4 ? 0 : 1];
          const uint32_t mk = valid ? 0xFFFFFFFFu : 0u;
          w[0] = v0.x & mk; w[1] = v0.y & mk; w[2] = v0.z & mk; w[3] = v0.w & mk;
          w[4] = v1.x & mk; w[5] = v1.y & mk; w[6] = v1.z & mk; w[7] = v1.w & mk;
        }
        const int a8 = valid ? 8 : 0;  // the -8 offset of the unsigned nibble codes
        const int f = LPBQ ? static_cast<int>(((i < 4 ? fsv.x : fsv.y) >> (8 * (i & 3))) & 0xFFu) : 1;
        uint32_t rr[HR ? 8 : 1];  // residues of the 32 weights (zero codes in slots past K: r = 0)
        if constexpr (HR) {
          const uint4 tab = rtab[col * kRtabF + (valid ? f : 0)];
#pragma unroll
          for (int j = 0; j < 8; ++j) rr[j] = resid4(w[j], tab);
        }
#pragma unroll
        for (int m = 0; m < MM; ++m) {
          if (MM > 1 && m >= M) continue;
          const uint4 *ap = reinterpret_cast<const uint4 *>(lds + static_cast<size_t>(m) * g.ars + kg * 32);
          const uint4 a0 = ap[0], a1 = ap[1];
          int d = sdot4(a0.x, w[0], 0);
          d = sdot4(a0.y, w[1], d); d = sdot4(a0.z, w[2], d); d = sdot4(a0.w, w[3], d);
          d = sdot4(a1.x, w[4], d); d = sdot4(a1.y, w[5], d); d = sdot4(a1.z, w[6], d); d = sdot4(a1.w, w[7], d);
          if (FMT == kTileI4) d -= a8 * asum[m * KG + kg];
          acc[m] += LPBQ ? d * f : d;
          if (A16) {
            const uint4 *lp = reinterpret_cast<const uint4 *>(lds + static_cast<size_t>(M + m) * g.ars + kg * 32);
            const uint4 b0 = lp[0], b1 = lp[1];
            int e = sdot4(b0.x, w[0], 0);
            e = sdot4(b0.y, w[1], e); e = sdot4(b0.z, w[2], e); e = sdot4(b0.w, w[3], e);
            e = sdot4(b1.x, w[4], e); e = sdot4(b1.y, w[5], e); e = sdot4(b1.z, w[6], e); e = sdot4(b1.w, w[7], e);
            if (FMT == kTileI4) e -= a8 * asum[(M + m) * KG + kg];
            acc2[m] += LPBQ ? e * f : e;
          }
          if constexpr (HR) {
            int h = sdot4(a0.x, rr[0], acc3[m]);
            h = sdot4(a0.y, rr[1], h); h = sdot4(a0.z, rr[2], h); h = sdot4(a0.w, rr[3], h);
            h = sdot4(a1.x, rr[4], h); h = sdot4(a1.y, rr[5], h); h = sdot4(a1.z, rr[6], h); h = sdot4(a1.w, rr[7], h);
            acc3[m] = h;
          }
        }
      }
    }
    // 16 rows: the next group's constants, then its first batch of weights, are in flight
    // during the reduction and the epilogue (the constants first: the next epilogue's and
    // residue tables' waits then do not include the weights)
    Epi ep_next{};
    if constexpr (kLoop) {
      const int nxt = min(grp + static_cast<int>(gridDim.x), groups - 1);
      ep_next = epi_of(nxt);
      if constexpr (HR) rtab_mant(nxt, rmt);
      issue(grp + static_cast<int>(gridDim.x), 0);
    }
    // reduce over the 4 k-group lanes of each column, then over the waves in LDS
    if constexpr (kMfma) {
      // the product already summed the wave's lanes: lane (quarter q, column c) holds rows 4 q .. + 3
      if (shalf == 0) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          red[wave][4 * sub + q][col] = macc[q];
          if (A16) red2[wave][4 * sub + q][col] = macc2[q];
          if (HR) red3[wave][4 * sub + q][col] = macc3[q];
          if (LR) red4[wave][4 * sub + q][col] = macc4[q];
        }
      }
      if constexpr (kWide) {
        // the second half of the waves adds its sums into the first half's
        lds_barrier();
        if (shalf == 1) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            atomicAdd(&red[wave][4 * sub + q][col], macc[q]);
            if (A16) atomicAdd(&red2[wave][4 * sub + q][col], macc2[q]);
            if (HR) atomicAdd(&red3[wave][4 * sub + q][col], macc3[q]);
            if (LR) atomicAdd(&red4[wave][4 * sub + q][col], macc4[q]);
          }
        }
      }
    }
#pragma unroll
    for (int m = 0; m < (kMfma ? 0 : MM); ++m) {
      acc[m] += __shfl_xor(acc[m], 16, 64);
      acc[m] += __shfl_xor(acc[m], 32, 64);
      if (sub == 0) red[wave][m][col] = acc[m];
      if (A16) {
        acc2[m] += __shfl_xor(acc2[m], 16, 64);
        acc2[m] += __shfl_xor(acc2[m], 32, 64);
        if (sub == 0) red2[wave][m][col] = acc2[m];
      }
      if (HR) {
        acc3[m] += __shfl_xor(acc3[m], 16, 64);
        acc3[m] += __shfl_xor(acc3[m], 32, 64);
        if (sub == 0) red3[wave][m][col] = acc3[m];
      }
    }
    lds_barrier();
    // requantise: thread t owns output (row t / 16, column t % 16) of the group
    const int om = t >> 4, n = grp * 16 + (t & 15);
    bool amb = false;
    if (owns_out) {
      int S1 = 0, S2 = 0, S3 = 0, S4 = 0;
#pragma unroll
      for (int w = 0; w < kGemvWaves; ++w) {
        S1 += red[w][om][t & 15];
        if (A16) S2 += red2[w][om][t & 15];
        if (HR) S3 += red3[w][om][t & 15];
        if (LR) S4 += red4[w][om][t & 15];
      }
      const double beta = ep.beta, margin = ep.margin, absb = ep.absb, mr1 = ep.mr1;
      const int64_t corr = A16 ? ep.corr * static_cast<int64_t>(128 + 32768 - g.act_zp) : ep.corr;
      const int64_t S = A16 ? 256 * static_cast<int64_t>(S1) + S2 + corr : static_cast<int64_t>(S1) + corr;
      double tv, slack;
      if constexpr (HR) {
        // D = sum_k (a - zp) (w M + r) = M S + 256 sum hi' r + sum lo' r + (32896 - zp) sum r.
        // 16 rows form sum lo' r too (D exact: only the oracle's own float noise remains);
        // fewer rows bound it by mr1 (margin_lo).
        const int64_t D = S * ep.mant + 256 * static_cast<int64_t>(S3) + static_cast<int64_t>(S4) +
                          static_cast<int64_t>(128 + 32768 - g.act_zp) * ep.csr;
        tv = fma(static_cast<double>(D), ep.alpha, beta);
        slack = margin + (LR ? 0.0 : mr1) + 0x1p-48 * (fabs(tv) + absb);
      } else {
        const double alpha = A16 ? ep.alpha * static_cast<double>(ep.mant) : ep.alpha;
        tv = fma(static_cast<double>(S), alpha, beta);
        slack = margin + (A16 ? mr1 * static_cast<double>(r1[om]) : 0.0) + 0x1p-48 * (fabs(tv) + absb);
      }
      const double fl = floor(tv);
      const bool near_tie = fabs((tv - fl) - 0.5) <= slack;
      const double lo = fmin(fmax(fl, 0.0), static_cast<double>(g.out_qmax));
      const double hi = fmin(fmax(fl + 1.0, 0.0), static_cast<double>(g.out_qmax));
      amb = near_tie && lo != hi;
      if (!amb) {
        const double o = fmin(fmax(rint(tv), 0.0), static_cast<double>(g.out_qmax));
        const size_t idx = static_cast<size_t>(om) * g.N + n;
        if (g.out16)
          static_cast<uint16_t *>(g.out)[idx] = static_cast<uint16_t>(o);
        else
          static_cast<uint8_t *>(g.out)[idx] = static_cast<uint8_t>(o);
      }
    }
    // exact fixup of the ambiguous outputs: listed in LDS, then shared out over the waves
    if (amb) fix_list[atomicAdd(&fix_cnt, 1)] = static_cast<uint16_t>(t);
    lds_barrier();
    const int nfix = fix_cnt;
    if (kLoop || KG > kGemvBatchKG) {
      // the weight registers hold the next group or only the last batch: re-read the column.
      // 8-bit activations complete the residue term exactly first; what stays ambiguous (within
      // the oracle's own float noise of a rounding boundary) is recomputed term by term.
      int nslow = nfix;
      if constexpr (!A16)
        if (nfix > 0) nslow = gemv_fixup_exact<FMT, LPBQ, NT, RA>(g, lds, fix_list, nfix, grp, t, ired, &fix_cnt);
      for (int e = t >> 6; e < nslow; e += NT / 64) {
        const int tt = fix_list[e];
        gemv_fixup<A16, FMT, LPBQ, RA>(g, lds, tt >> 4, grp * 16 + (tt & 15), lane);
      }
    } else {
      // the column's weights (one batch: K <= 4096) are still in the registers of its 16
      // lanes: they hand them over
      uint8_t *const fixw = lds + g.off_fixw;
      uint8_t *const fixs = fixw + kFixBatch * KG * WB;
      for (int e0 = 0; e0 < nfix; e0 += kFixBatch) {
        const int nb = min(kFixBatch, nfix - e0);
        for (int e = 0; e < nb; ++e) {
          if (col != (fix_list[e0 + e] & 15)) continue;
#pragma unroll
          for (int i = 0; i < kU; ++i) {
            const int kg = 4 * (wave + 4 * i) + sub;
            if (kg < KG) {
              uint8_t *dst = fixw + (static_cast<size_t>(e) * KG + kg) * WB;
              *reinterpret_cast<uint4 *>(dst) = wv[i][0];
              if (FMT != kTileI4) *reinterpret_cast<uint4 *>(dst + 16) = wv[i][FMT == kTileI4 ? 0 : 1];
              if (LPBQ) fixs[e * KG + kg] = static_cast<uint8_t>(((i < 4 ? fsv.x : fsv.y) >> (8 * (i & 3))) & 0xFFu);
            }
          }
        }
        lds_barrier();
        gemv_fixup_batch<A16, FMT, LPBQ>(g, lds, fixw, fixs, dred, fix_list + e0, nb, grp, t);
        lds_barrier();  // fixw / dred are rewritten by the next batch
      }
    }
    lds_barrier();  // red and the fixup list are rewritten by the next group
    if (t == 0) fix_cnt = 0;
    if (!kLoop) break;
    ep = ep_next;
  }
}

// Raises the dynamic LDS limit of one kernel instantiation once per device (the call costs a
// driver round trip, too much for a launch that streams 30 MB in a few microseconds).  The
// cache is keyed by the instantiation's template arguments: every instantiation has the same
// function type, so a cache keyed by that type would be shared by all of them.
template <bool A16, int FMT, bool LPBQ, int MM, bool RA = false>
qh_status allow_dyn_lds() {
  const auto kernel = &qmm_gemv_kernel<A16, FMT, LPBQ, MM, RA>;
  static std::atomic<uint32_t> done{0};  // bit d: set on device d
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  const uint32_t bit = dev < 32 ? 1u << dev : 0u;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return QH_STATUS_OK;
  e = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          kGemvMaxDynLds);
  if (e != hipSuccess) return hip_fail(e, "hipFuncSetAttribute(qmm_gemv_kernel)");
  done.fetch_or(bit, std::memory_order_acq_rel);
  return QH_STATUS_OK;
}

template <bool A16, int FMT, bool LPBQ, int MM, bool RA = false>
qh_status launch_one(const GemvArgs &g, dim3 grid, size_t dyn_lds, hipStream_t stream) {
  const qh_status st = allow_dyn_lds<A16, FMT, LPBQ, MM, RA>();
  if (st != QH_STATUS_OK) return st;
  hipLaunchKernelGGL((qmm_gemv_kernel<A16, FMT, LPBQ, MM, RA>), grid, dim3(gemv_threads<A16, MM>()), dyn_lds, stream, g);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return hip_fail(err, "qmm_gemv_kernel launch");
  return QH_STATUS_OK;
}

// Workgroups of the 16-row kernel that are resident at once with dyn_lds bytes of dynamic LDS
// (occupancy x compute units), or 0 if the runtime cannot say.  Cached for the last query.
template <bool A16, int FMT, bool LPBQ, bool RA>
int resident_workgroups(size_t dyn_lds) {
  static std::atomic<uint64_t> last{0};  // dyn_lds << 24 | device << 16 | workgroups
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev > 255) return 0;
  const uint64_t key = (static_cast<uint64_t>(dyn_lds) << 24) | (static_cast<uint64_t>(dev) << 16);
  const uint64_t hit = last.load(std::memory_order_acquire);
  if ((hit & ~static_cast<uint64_t>(0xFFFF)) == key && (hit & 0xFFFF) != 0) return static_cast<int>(hit & 0xFFFF);
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, reinterpret_cast<const void *>(&qmm_gemv_kernel<A16, FMT, LPBQ, 16, RA>),
                                                   gemv_threads<A16, 16>(), dyn_lds) != hipSuccess)
    return 0;
  const long long wg = static_cast<long long>(occ) * device_cu_count();
  if (wg <= 0 || wg > 0xFFFF) return 0;
  last.store(key | static_cast<uint64_t>(wg), std::memory_order_release);
  return static_cast<int>(wg);
}

// Workgroups of a 16-row launch: one group each while the staged activations are small.  Larger
// staging is amortised over several groups per workgroup: at most 512 workgroups, and no more
// than are resident at once, since a second round would stage the activations again (16 rows of
// 16-bit activations at K = 4096 take 128 KiB, one workgroup per compute unit).  Register-held
// activations follow the same rule: each workgroup reads the rows once.
template <bool A16, int FMT, bool LPBQ, bool RA>
qh_status launch_16(const GemvArgs &g, size_t dyn_lds, hipStream_t stream) {
  const int groups = g.N / 16;
  const int planes = A16 ? 2 : 1;
  int blocks = groups;
  if (static_cast<size_t>(planes) * g.M * g.K > 16384) {
    const qh_status st = allow_dyn_lds<A16, FMT, LPBQ, 16, RA>();  // before the occupancy query
    if (st != QH_STATUS_OK) return st;
    const int cap = resident_workgroups<A16, FMT, LPBQ, RA>(dyn_lds);
    const int lim = cap > 0 && cap < 512 ? cap : 512;
    if (blocks > lim) {
      // the same number of groups per workgroup (rounded up), so the workgroups end together
      const int per = (groups + lim - 1) / lim;
      blocks = (groups + per - 1) / per;
    }
  }
  return launch_one<A16, FMT, LPBQ, 16, RA>(g, dim3(blocks), dyn_lds, stream);
}

template <bool A16, int FMT, bool LPBQ>
qh_status launch_mm(const GemvArgs &g, size_t dyn_lds, hipStream_t stream) {
  const int groups = g.N / 16;
  if (g.M <= 1) return launch_one<A16, FMT, LPBQ, 1>(g, dim3(groups), dyn_lds, stream);
  if (g.M <= 4) return launch_one<A16, FMT, LPBQ, 4>(g, dim3(groups), dyn_lds, stream);
  // rows whose k-groups fit one batch per lane (K <= 16 kU x 32) stay in registers (8-bit
  // activations, and 16-bit activations with int4 codes)
  if constexpr (!A16 || FMT == kTileI4)
    if (g.KG <= 16 * kU) return launch_16<A16, FMT, LPBQ, true>(g, 0, stream);
  return launch_16<A16, FMT, LPBQ, false>(g, dyn_lds, stream);
}

size_t align16(size_t x) { return (x + 15) & ~static_cast<size_t>(15); }

// Dynamic LDS of one launch: activation planes, k-group sums, kFixBatch columns' weight words
// and block scales (register-held fixup).
struct GemvLds {
  size_t off_asum, off_fixw, bytes;
};
GemvLds gemv_lds(const QmmShape &sh, int m) {
  const int planes = sh.act_bits == 16 ? 2 : 1;
  const int KG = sh.K / 32;
  const int WB = sh.gemv_fmt == kTileI4 ? 16 : 32;
  GemvLds L;
  L.off_asum = align16(static_cast<size_t>(planes) * m * (sh.K + 16));
  const size_t asum_bytes = sh.gemv_fmt == kTileI4 ? static_cast<size_t>(planes) * m * KG * 2 : 0;
  L.off_fixw = align16(L.off_asum + asum_bytes);
  // (only single-group launches, M <= 4, with one batch of k-groups hold the weights)
  const bool reg_fix = m <= 4 && KG <= kGemvBatchKG;
  L.bytes = L.off_fixw + (reg_fix ? static_cast<size_t>(kFixBatch) * KG * (WB + 1) : 0);
  return L;
}

}  // namespace

bool gemv_fits(const qh_qmm_prepared *p, int m) {
  return m >= 1 && m <= 16 && gemv_lds(p->shape, m).bytes <= static_cast<size_t>(kGemvMaxDynLds);
}

qh_status launch_qmm_gemv(const qh_qmm_prepared *p, int m, const void *act, void *out, hipStream_t stream) {
  const QmmShape &sh = p->shape;
  const QmmDevice &D = p->dev;
  if (m > 16) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "GEMV path supports M <= 16 (got %d)", m);
  if (m <= 4) {
    // int4 weights: the persistent kernel (one workgroup per compute unit) where its shape
    // limits allow
    const qh_status su = launch_qmm_gemv_unit(p, m, act, out, stream);
    if (su != QH_STATUS_SHAPE_UNSUPPORTED) return su;
  }
  const bool lpbq = sh.wfmt == QH_WEIGHT_I4_LPBQ;
  const int KG = sh.K / 32;
  const GemvLds L = gemv_lds(sh, m);
  const size_t off_asum = L.off_asum, off_fixw = L.off_fixw, dyn = L.bytes;
  if (dyn > static_cast<size_t>(kGemvMaxDynLds))
    return fail(QH_STATUS_SHAPE_UNSUPPORTED, "GEMV path: M=%d, K=%d needs %zu bytes of LDS staging (limit %d)", m,
                sh.K, dyn, kGemvMaxDynLds);
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
  g.mlo = D.margin_lo;
  g.corr = D.corr;
  g.mant = D.mant;
  g.colsum = D.colsum;
  g.colsum_r = D.colsum_r;
  g.alpha_e = D.alpha_e;
  g.margin_exact = D.margin_exact;
  g.s32 = D.s32;
  g.M = m;
  g.N = sh.N;
  g.K = sh.K;
  g.KG = KG;
  g.nbatch = (KG + kGemvBatchKG - 1) / kGemvBatchKG;
  g.sub_shift = sh.lpbq_block == 64 ? 1 : 0;
  g.act_zp = sh.act_zp;
  g.out_zp = sh.out_zp;
  g.out_qmax = (1 << sh.out_bits) - 1;
  g.out16 = sh.out_bits == 16;
  g.ars = sh.K + 16;
  g.off_asum = static_cast<int>(off_asum);
  g.off_fixw = static_cast<int>(off_fixw);
  g.sA = sh.act_scale;
  g.sO = sh.out_scale;
  const bool a16 = sh.act_bits == 16;
  if (!a16) {
    if (sh.gemv_fmt == kTileI8) return launch_mm<false, kTileI8, false>(g, dyn, stream);
    if (lpbq) return launch_mm<false, kTileI4, true>(g, dyn, stream);
    return launch_mm<false, kTileI4, false>(g, dyn, stream);
  }
  if (sh.gemv_fmt == kTileI8) return launch_mm<true, kTileI8, false>(g, dyn, stream);
  if (lpbq) return launch_mm<true, kTileI4, true>(g, dyn, stream);
  return launch_mm<true, kTileI4, false>(g, dyn, stream);
}

}  // namespace qh
