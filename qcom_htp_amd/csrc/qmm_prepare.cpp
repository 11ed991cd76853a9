// Host-side prepare step of the quantized matmul: validates the descriptor, lays the weight
// codes out as MFMA/streaming tiles, and derives the per-channel epilogue constants that make
// the integer-accumulator result bit-exact to the reference's float-derived requantisation.
//
// Reference correspondence: the QHPI precompute of the op packages
// (example/qnn_hmx_matmul_u8i8/src/HmxU8I8ToU8MatMulOp.cpp:196-287) and the const-folded LPBQ
// expansion (example/qnn_hmx_matmul_common/HmxW4LpbqExpandToI8Op.cpp:107-164) both run once
// at graph prepare; this file is that step for the GPU.
//
// Exactness argument (why the epilogue can round like the float64 oracle):
//   The oracle dequantises weights as w_deq = fl32(w_int * s32).  Write s32 = M * 2^E with a
//   24-bit integer mantissa M.  Every w_deq is then an integer multiple W' of 2^E with
//   W' = w_int * M + r, where r is the float32 rounding residue (|r| <= 64 for |w_int| <= 127).
//   The exact dot product is  sum_k (a_k - zp) * w_deq_k = 2^E * (M * acc + sum_k (a_k - zp) r_k)
//   with acc the int32 MFMA accumulator.
//   * 16-bit activations: the kernels accumulate sum (a - zp) * r as well (the residue plane is
//     a second weight operand), so the exact dot product is known in int64.
//   * 8-bit activations: the residue term is bounded by amax * sum_k |r_k| per channel
//     (amax = max |a - zp|); outputs whose rounding could flip within that bound are recomputed
//     exactly by the kernel's fixup pass.

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <vector>

#include "qmm_internal.h"

namespace qh {
namespace {

constexpr double kSafety = 1.0 + 1.0 / 1048576.0;  // 1 + 2^-20 on every bound

inline int round_up(int v, int m) { return (v + m - 1) / m * m; }

// s32 = M * 2^E with M a 24-bit integer (for normal floats M in [2^23, 2^24)).
inline void split_float(float s, int64_t *M, int *E) {
  int e = 0;
  double fr = std::frexp(static_cast<double>(s), &e);  // s = fr * 2^e, fr in [0.5, 1)
  *M = static_cast<int64_t>(std::ldexp(fr, 24));
  *E = e - 24;
}

struct DevAlloc {
  std::vector<void *> ptrs;
  uint64_t bytes = 0;
  template <class T>
  qh_status upload(T **dst, const std::vector<T> &src) {
    *dst = nullptr;
    if (src.empty()) return QH_STATUS_OK;
    size_t nbytes = src.size() * sizeof(T);
    void *p = nullptr;
    hipError_t err = hipMalloc(&p, nbytes);
    if (err != hipSuccess) return hip_fail(err, "hipMalloc(prepared state)");
    ptrs.push_back(p);
    bytes += nbytes;
    err = hipMemcpy(p, src.data(), nbytes, hipMemcpyHostToDevice);
    if (err != hipSuccess) return hip_fail(err, "hipMemcpy(prepared state)");
    *dst = static_cast<T *>(p);
    return QH_STATUS_OK;
  }
  void release() {
    for (void *p : ptrs) (void)hipFree(p);
    ptrs.clear();
  }
};

// Writes value v (int8 range) of operand column c, depth k into the tile image.
// Writes int8 weights into the GEMM tile layout (see qmm_internal.h).
struct TileWriter {
  std::vector<uint8_t> &buf;
  int KT;  // number of 128-deep k tiles
  void put(int c, int k, int v) {
    const size_t tile = static_cast<size_t>(c / kBN) * KT + k / kBK;
    buf[tile * (kBN * kBK) + tile_off_i8(c % kBN, k)] = static_cast<uint8_t>(static_cast<int8_t>(v));
  }
};

// Prepared state of the formats that run on the exact integer GEMM only (qmm_exact.hip):
//   * QH_WEIGHT_I4_GROUP: the oracle's weight fl32(q s_g) = 2^E_g (q M_g + r) (s_g = M_g 2^E_g);
//     with E_min = min_g E_g and d_g = E_g - E_min the dot product is 2^E_min D exactly, where
//     D = sum_g [M_g 2^d_g sum_{k in g} (a - zp) q + 2^d_g sum_{k in g} (a - zp) r].  Plane 0
//     holds q, plane 1 holds r (|r| <= 64), with those multipliers per (group, channel).
//   * QH_WEIGHT_I16: q16 = 256 hi + lo' + 128 (hi = q16 >> 8, lo' = (q16 & 255) - 128): planes hi
//     (x 256) and lo' (x 1) plus 128 times the activation row sum (the all-ones plane).
qh_status prepare_exact(const qh_qmm_desc *d, qh_qmm_prepared **out) {
  const bool group = d->weight_format == QH_WEIGHT_I4_GROUP;
  const int N = static_cast<int>(d->n), K = static_cast<int>(d->k);
  const bool a16 = d->act_bits == 16;
  int gsz = 64, gshift = 6;
  if (group) {
    if (d->weight_nk == nullptr || d->group_scale == nullptr)
      return fail(QH_STATUS_INVALID_ARGUMENT, "per-group weights need weight_nk and group_scale");
    gsz = static_cast<int>(d->group_size);
    if (gsz < 64 || (gsz & (gsz - 1)) || K % gsz)
      return fail(QH_STATUS_SHAPE_UNSUPPORTED, "group_size=%d must be a power of two >= 64 dividing K=%d", gsz, K);
    gshift = 0;
    while ((1 << gshift) < gsz) ++gshift;
  } else if (d->weight16_nk == nullptr) {
    return fail(QH_STATUS_INVALID_ARGUMENT, "QH_WEIGHT_I16 needs weight16_nk");
  }
  const int G = group ? K / gsz : 1;
  QmmShape sh{};
  sh.N = N;
  sh.K = K;
  sh.Kp = round_up(K, kBK);
  sh.act_bits = static_cast<int>(d->act_bits);
  sh.out_bits = static_cast<int>(d->out_bits);
  sh.wfmt = static_cast<int>(d->weight_format);
  sh.act_zp = d->act_zp;
  sh.out_zp = d->out_zp;
  sh.act_scale = d->act_scale;
  sh.out_scale = d->out_scale;
  sh.ncols_op = round_up(2 * N, kBN);
  sh.Np = sh.ncols_op / 2;
  sh.layout_planes = 2;
  sh.exact_only = 1;
  sh.groups = G;
  sh.group_shift = gshift;
  const int Np = sh.Np, KT = sh.Kp / kBK;
  const int64_t c = (a16 ? 32896 : 128) - d->act_zp;  // activation shift of the exact GEMM
  const double amax = static_cast<double>(std::max(d->act_zp, (1 << d->act_bits) - 1 - d->act_zp));

  std::vector<uint8_t> tiles(static_cast<size_t>(sh.ncols_op) * sh.Kp, 0);
  TileWriter tw{tiles, KT};
  std::vector<int64_t> corr_int(Np, 0), corr_rq(Np, 0), mult;
  std::vector<int32_t> biasv(Np, 0);
  std::vector<double> alpha_e(Np, 0.0), beta(Np, 0.0), margin_exact(Np, 0.0), absb(Np, 1.0), bdeq(Np, 0.0);
  std::vector<float> s32g;
  for (int n = 0; n < N; ++n) biasv[n] = d->bias_q ? d->bias_q[n] : 0;
  if (!group) {
    sh.int_planes = 2;
    sh.int_mult[0] = 256;
    sh.int_mult[1] = 1;
    sh.int_ones = 128;
    for (int n = 0; n < N; ++n) {
      const int cq = (n / 32) * 64 + (n % 32);
      int64_t cs = 0;
      for (int k = 0; k < K; ++k) {
        const int q = d->weight16_nk[static_cast<size_t>(n) * K + k];
        tw.put(cq, k, q >> 8);                 // arithmetic: hi in [-128, 127]
        tw.put(cq + 32, k, (q & 255) - 128);   // lo' in [-128, 127]
        cs += q;
      }
      corr_int[n] = c * cs;
    }
  } else {
    sh.int_planes = 1;
    sh.int_mult[0] = 1;
    sh.int_mult[1] = 0;
    sh.int_ones = 0;
    mult.assign(static_cast<size_t>(2) * G * Np, 0);
    s32g.assign(static_cast<size_t>(N) * G, 1.0f);
    const double sA = d->act_scale, sO = d->out_scale;
    std::vector<int64_t> Mg(G);
    std::vector<int> Eg(G);
    std::vector<char> live(G);
    for (int n = 0; n < N; ++n) {
      // the common exponent comes from the groups with a nonzero code: an all-zero group adds
      // exactly nothing whatever its scale (e.g. the epsilon scale of an all-zero weight block)
      int emin = std::numeric_limits<int>::max();
      for (int g = 0; g < G; ++g) {
        const float sg = d->group_scale[static_cast<size_t>(n) * G + g];
        if (!(sg > 0.0f) || !std::isfinite(sg) || sg < std::numeric_limits<float>::min())
          return fail(QH_STATUS_INVALID_ARGUMENT, "group_scale[%d][%d] must be a positive normal float", n, g);
        split_float(sg, &Mg[g], &Eg[g]);
        s32g[static_cast<size_t>(n) * G + g] = sg;
        live[g] = 0;
        for (int k = g * gsz; k < (g + 1) * gsz; ++k) live[g] |= d->weight_nk[static_cast<size_t>(n) * K + k] != 0;
        if (live[g]) emin = std::min(emin, Eg[g]);
      }
      if (emin == std::numeric_limits<int>::max()) emin = Eg[0];
      const int cq = (n / 32) * 64 + (n % 32);
      int64_t csq = 0;
      double sum_abs = 0.0;  // sum_k 2^d_g |q M_g + r|: bounds D and the oracle's float noise
      double corr_d = 0.0;
      int64_t corr_acc = 0;
      for (int g = 0; g < G; ++g) {
        const int dg = live[g] ? Eg[g] - emin : 0;
        if (dg > 30) return fail(QH_STATUS_UNSUPPORTED, "channel %d: group scales span more than 2^30", n);
        const int64_t m0 = live[g] ? Mg[g] << dg : 0, m1 = live[g] ? int64_t{1} << dg : 0;
        mult[(static_cast<size_t>(0) * G + g) * Np + n] = m0;
        mult[(static_cast<size_t>(1) * G + g) * Np + n] = m1;
        int64_t sq = 0, sr = 0;
        const float sg = s32g[static_cast<size_t>(n) * G + g];
        for (int k = g * gsz; k < (g + 1) * gsz; ++k) {
          const int q = d->weight_nk[static_cast<size_t>(n) * K + k];
          if (q < -127 || q > 127)
            return fail(QH_STATUS_INVALID_ARGUMENT, "weight code %d at (n=%d,k=%d) outside [-127,127]", q, n, k);
          const float wd = static_cast<float>(q) * sg;  // the oracle's float32 weight
          const double wp = std::ldexp(static_cast<double>(wd), -Eg[g]);
          const int64_t Wp = static_cast<int64_t>(wp);
          if (static_cast<double>(Wp) != wp) return fail(QH_STATUS_RUNTIME_ERROR, "internal: non-integer weight at n=%d", n);
          const int64_t r = Wp - static_cast<int64_t>(q) * Mg[g];
          if (r < -127 || r > 127) return fail(QH_STATUS_RUNTIME_ERROR, "internal: residue %lld out of int8", (long long)r);
          tw.put(cq, k, q);
          tw.put(cq + 32, k, static_cast<int>(r));
          sq += q;
          sr += r;
          sum_abs += std::ldexp(std::fabs(static_cast<double>(Wp)), dg);
        }
        csq += sq;
        corr_acc += m0 * sq + m1 * sr;
        corr_d += static_cast<double>(m0) * static_cast<double>(sq) + static_cast<double>(m1) * static_cast<double>(sr);
      }
      // D = sum of int64 terms; every partial sum is bounded by amax * sum_abs + |c corr|
      const double bound = amax * sum_abs + std::fabs(static_cast<double>(c) * corr_d);
      if (!(bound < 0x1p62))
        return fail(QH_STATUS_UNSUPPORTED, "channel %d: per-group exact sum exceeds int64 (group scales span too far)", n);
      corr_rq[n] = c * corr_acc;
      corr_int[n] = c * csq;
      const double ae = std::ldexp(sA, emin) / sO;
      alpha_e[n] = ae;
      bdeq[n] = d->bias_float ? static_cast<double>(d->bias_float[n]) : 0.0;
      beta[n] = bdeq[n] / sO + d->out_zp;
      absb[n] = 2.0 * std::fabs(beta[n]) + 2.0 * d->out_zp + 1.0;
      // the oracle's float64 noise: K roundings of terms bounded by amax 2^E_min sum_abs / K
      margin_exact[n] = (K + 8.0) * std::ldexp(1.0, -52) * amax * sum_abs * ae * kSafety;
    }
  }
  auto *p = new qh_qmm_prepared();
  p->shape = sh;
  int dev = 0;
  (void)hipGetDevice(&dev);
  p->device_id = dev;
  DevAlloc al;
  qh_status st = QH_STATUS_OK;
  QmmDevice &D = p->dev;
  std::memset(&D, 0, sizeof(D));
  if (st == QH_STATUS_OK) st = al.upload(&D.tiles, tiles);
  if (st == QH_STATUS_OK) st = al.upload(&D.bias_q, biasv);
  if (st == QH_STATUS_OK) st = al.upload(&D.corr_int, corr_int);
  if (st == QH_STATUS_OK && group) st = al.upload(&D.mult, mult);
  if (st == QH_STATUS_OK && group) st = al.upload(&D.corr_rq, corr_rq);
  if (st == QH_STATUS_OK && group) st = al.upload(&D.s32g, s32g);
  if (st == QH_STATUS_OK && group) st = al.upload(&D.alpha_e, alpha_e);
  if (st == QH_STATUS_OK && group) st = al.upload(&D.beta, beta);
  if (st == QH_STATUS_OK && group) st = al.upload(&D.margin_exact, margin_exact);
  if (st == QH_STATUS_OK && group) st = al.upload(&D.absb, absb);
  if (st == QH_STATUS_OK && group) st = al.upload(&D.bias_deq, bdeq);
  if (st != QH_STATUS_OK) {
    al.release();
    delete p;
    return st;
  }
  p->device_bytes = al.bytes;
  p->gemm_weight_bytes = tiles.size();
  p->gemv_weight_bytes = 0;
  *out = p;
  return QH_STATUS_OK;
}

}  // namespace
}  // namespace qh

using namespace qh;

extern "C" qh_status qh_qmm_prepare(const qh_qmm_desc *d, qh_qmm_prepared **out) {
  if (out == nullptr) return fail(QH_STATUS_INVALID_ARGUMENT, "qh_qmm_prepare: out is NULL");
  *out = nullptr;
  if (d == nullptr) return fail(QH_STATUS_INVALID_ARGUMENT, "qh_qmm_prepare: desc is NULL");
  if (d->act_bits != 8 && d->act_bits != 16)
    return fail(QH_STATUS_UNSUPPORTED, "act_bits must be 8 or 16 (got %u)", d->act_bits);
  if (d->out_bits != 8 && d->out_bits != 16)
    return fail(QH_STATUS_UNSUPPORTED, "out_bits must be 8 or 16 (got %u)", d->out_bits);
  if (d->weight_format > QH_WEIGHT_I16)
    return fail(QH_STATUS_UNSUPPORTED, "unknown weight_format %u", d->weight_format);
  if (d->k == 0 || d->n == 0 || d->k % 32 || d->n % 32)
    return fail(QH_STATUS_SHAPE_UNSUPPORTED, "K and N must be positive multiples of 32 (K=%u N=%u)", d->k, d->n);
  if (d->k > 65536 || d->n > (1u << 20))
    return fail(QH_STATUS_SHAPE_UNSUPPORTED, "K <= 65536 and N <= 2^20 required (K=%u N=%u)", d->k, d->n);
  {
    const int act_qmax = (1 << d->act_bits) - 1, out_qmax = (1 << d->out_bits) - 1;
    if (d->act_zp < 0 || d->act_zp > act_qmax || d->out_zp < 0 || d->out_zp > out_qmax)
      return fail(QH_STATUS_INVALID_ARGUMENT, "zero point out of range (act_zp=%d out_zp=%d)", d->act_zp, d->out_zp);
    if (!(d->act_scale > 0.0) || !(d->out_scale > 0.0) || !std::isfinite(d->act_scale) || !std::isfinite(d->out_scale))
      return fail(QH_STATUS_INVALID_ARGUMENT, "act_scale and out_scale must be finite and > 0");
  }
  if (d->weight_format == QH_WEIGHT_I4_GROUP || d->weight_format == QH_WEIGHT_I16) return prepare_exact(d, out);
  const int act_qmax = (1 << d->act_bits) - 1;
  const bool lpbq = d->weight_format == QH_WEIGHT_I4_LPBQ;
  if (lpbq && d->lpbq_block != 32 && d->lpbq_block != 64)
    return fail(QH_STATUS_UNSUPPORTED, "lpbq_block must be 32 or 64 (got %u)", d->lpbq_block);
  if (lpbq && d->k % d->lpbq_block)
    return fail(QH_STATUS_SHAPE_UNSUPPORTED, "K=%u must be a multiple of lpbq_block=%u", d->k, d->lpbq_block);
  if (d->weight_nk == nullptr || d->weight_scale == nullptr || (lpbq && d->lpbq_block_scale == nullptr))
    return fail(QH_STATUS_INVALID_ARGUMENT, "weight_nk / weight_scale / lpbq_block_scale is NULL");

  const int N = static_cast<int>(d->n), K = static_cast<int>(d->k);
  const int wq_max = d->weight_format == QH_WEIGHT_I8 ? 127 : 7;
  const int bs = lpbq ? static_cast<int>(d->lpbq_block) : 0;
  const int nblk = lpbq ? K / bs : 0;

  // ---- integer weights, scale mantissas, rounding residues --------------------------------
  std::vector<int8_t> wint(static_cast<size_t>(N) * K);
  std::vector<int8_t> resid(static_cast<size_t>(N) * K);
  std::vector<int64_t> mant(N), colsum_q(N), colsum_r(N);
  std::vector<int> expo(N), rmax(N);
  std::vector<double> r1(N), r2(N), wpmax(N);
  for (int n = 0; n < N; ++n) {
    const float s = d->weight_scale[n];
    if (!(s > 0.0f) || !std::isfinite(s) || s < std::numeric_limits<float>::min())
      return fail(QH_STATUS_INVALID_ARGUMENT, "weight_scale[%d] must be a positive normal float", n);
    int64_t M;
    int E;
    split_float(s, &M, &E);
    mant[n] = M;
    expo[n] = E;
    int64_t cq = 0, cr = 0;
    double ra = 0, rs = 0, wm = 0;
    int rm = 0;
    for (int k = 0; k < K; ++k) {
      int q = d->weight_nk[static_cast<size_t>(n) * K + k];
      if (q < -wq_max || q > wq_max)
        return fail(QH_STATUS_INVALID_ARGUMENT, "weight code %d at (n=%d,k=%d) outside [-%d,%d]", q, n, k, wq_max, wq_max);
      int w = q;
      if (lpbq) {
        int f = d->lpbq_block_scale[static_cast<size_t>(n) * nblk + k / bs];
        if (f < 1 || f > 16)
          return fail(QH_STATUS_INVALID_ARGUMENT, "LPBQ block scale %d at (n=%d,block=%d) outside [1,16]", f, n, k / bs);
        w = q * f;  // |w| <= 112: exact, no saturation
      }
      // The oracle's float32 product, then its exact integer multiple of 2^E.
      const float wd = static_cast<float>(w) * s;
      const double wp = std::ldexp(static_cast<double>(wd), -E);
      const int64_t Wp = static_cast<int64_t>(wp);
      if (static_cast<double>(Wp) != wp) return fail(QH_STATUS_RUNTIME_ERROR, "internal: non-integer residue at n=%d", n);
      const int64_t r = Wp - static_cast<int64_t>(w) * M;
      if (r < -127 || r > 127) return fail(QH_STATUS_RUNTIME_ERROR, "internal: residue %lld out of int8", (long long)r);
      // The GEMM's fixup of listed outputs beyond its list capacity recomputes r from w and M on
      // the device as fl32(w M) - w M: the two must agree (they do unless w s32 overflows).
      if (static_cast<int64_t>(static_cast<float>(w) * static_cast<float>(M)) - static_cast<int64_t>(w) * M != r)
        return fail(QH_STATUS_INVALID_ARGUMENT, "weight_scale[%d]: the dequantised weights leave the float32 range", n);
      wint[static_cast<size_t>(n) * K + k] = static_cast<int8_t>(w);
      resid[static_cast<size_t>(n) * K + k] = static_cast<int8_t>(r);
      cq += w;
      cr += r;
      ra += std::fabs(static_cast<double>(r));
      rs += static_cast<double>(r) * static_cast<double>(r);
      rm = std::max(rm, static_cast<int>(std::llabs(r)));
      wm = std::max(wm, std::fabs(wp));
    }
    colsum_q[n] = cq;
    colsum_r[n] = cr;
    r1[n] = ra;
    r2[n] = rs;
    rmax[n] = rm;
    wpmax[n] = wm;
  }

  // ---- shape / format decisions ------------------------------------------------------------
  QmmShape sh{};
  sh.N = N;
  sh.K = K;
  sh.Kp = round_up(K, kBK);
  sh.act_bits = static_cast<int>(d->act_bits);
  sh.out_bits = static_cast<int>(d->out_bits);
  sh.wfmt = static_cast<int>(d->weight_format);
  sh.lpbq_block = bs;
  sh.act_zp = d->act_zp;
  sh.out_zp = d->out_zp;
  sh.act_scale = d->act_scale;
  sh.out_scale = d->out_scale;
  const bool a16 = d->act_bits == 16;
  // The GEMM is bound by the matrix cores, not by its weight bytes: int4 codes (and LPBQ
  // code * block scale, |.| <= 112) are widened to int8 tiles here, once, which keeps every
  // conversion but the activation shift out of its main loop.  The decode GEMV, which is bound
  // by HBM, streams the int4 codes.
  if (!a16) {
    sh.ncols_op = round_up(N, kBN);
    sh.Np = sh.ncols_op;
  } else {
    // codes and residues share one operand
    sh.ncols_op = round_up(2 * N, kBN);
    sh.Np = sh.ncols_op / 2;
  }
  sh.gemv_fmt = d->weight_format == QH_WEIGHT_I8 ? kTileI8 : kTileI4;
  sh.layout_planes = a16 ? 2 : 1;
  sh.int_planes = 1;
  sh.int_mult[0] = 1;
  sh.int_mult[1] = 0;
  sh.int_ones = 0;
  sh.groups = 1;
  sh.group_shift = 6;
  const int KT = sh.Kp / kBK;

  // ---- GEMM operand tiles ------------------------------------------------------------------
  std::vector<uint8_t> tiles(static_cast<size_t>(sh.ncols_op) * sh.Kp, 0);
  TileWriter tw{tiles, KT};
  if (!a16) {
    for (int n = 0; n < N; ++n)
      for (int k = 0; k < K; ++k) tw.put(n, k, wint[static_cast<size_t>(n) * K + k]);
  } else {
    for (int n = 0; n < N; ++n) {
      const int cq = (n / 32) * 64 + (n % 32), cr = cq + 32;
      for (int k = 0; k < K; ++k) {
        tw.put(cq, k, wint[static_cast<size_t>(n) * K + k]);
        tw.put(cr, k, resid[static_cast<size_t>(n) * K + k]);
      }
    }
  }

  // ---- GEMV stream (weights read once per call) --------------------------------------------
  // [N/16 column groups][K/32 k-groups][16 columns][16 B int4 | 32 B int8]; int4 byte j of a
  // (column, k-group) holds k = j in its low nibble and k = j + 16 in its high nibble.
  std::vector<uint8_t> gemv_tiles, gemv_lpbq;
  {
    const int KG = K / 32;
    const int per = sh.gemv_fmt == kTileI8 ? 32 : 16;
    gemv_tiles.assign(static_cast<size_t>(N) * KG * per, 0);
    for (int n = 0; n < N; ++n)
      for (int kg = 0; kg < KG; ++kg) {
        uint8_t *dst = &gemv_tiles[((static_cast<size_t>(n / 16) * KG + kg) * 16 + (n % 16)) * per];
        const int8_t *src = (lpbq ? d->weight_nk : wint.data()) + static_cast<size_t>(n) * K + kg * 32;
        if (sh.gemv_fmt == kTileI8) {
          for (int j = 0; j < 32; ++j) dst[j] = static_cast<uint8_t>(src[j]);
        } else {
          for (int j = 0; j < 16; ++j)
            dst[j] = static_cast<uint8_t>(((src[j] + 8) & 15) | (((src[j + 16] + 8) & 15) << 4));
        }
      }
    if (lpbq) {
      const int nbatch = (KG + kGemvBatchKG - 1) / kGemvBatchKG;
      const int sub_shift = bs == 64 ? 1 : 0;
      gemv_lpbq.assign(static_cast<size_t>(N / 16) * nbatch * 4 * (4 >> sub_shift) * 16 * kGemvKU, 1);
      for (int n = 0; n < N; ++n)
        for (int kg = 0; kg < KG; ++kg)
          gemv_lpbq[gemv_scale_index_kg(n, kg, nbatch, sub_shift)] =
              d->lpbq_block_scale[static_cast<size_t>(n) * nblk + (kg * 32) / bs];
    }
  }

  // ---- epilogue constants ------------------------------------------------------------------
  const double sA = d->act_scale, sO = d->out_scale, inv_sO = 1.0 / sO;
  const double amax = static_cast<double>(std::max(d->act_zp, act_qmax - d->act_zp));
  const int Np = sh.Np;
  std::vector<double> alpha(Np, 0.0), beta(Np, 0.0), margin(Np, 0.0), absb(Np, 1.0), bdeq(Np, 0.0), mr1(Np, 0.0),
      mlo(Np, 0.0);
  std::vector<int64_t> corr(Np, 0), mantv(Np, 0), csum(Np, 0), csum_r(Np, 0);
  std::vector<double> alpha_e(Np, 0.0);
  std::vector<double> margin_exact(Np, 0.0);
  std::vector<int32_t> scale_exp(Np, 0);
  std::vector<float> s32v(Np, 1.0f);
  std::vector<int32_t> biasv(Np, 0);
  std::vector<int64_t> corr_int(Np, 0);
  const double a_base = a16 ? 32768.0 : 128.0;  // the kernels shift activations by this
  for (int n = 0; n < N; ++n) {
    const float s = d->weight_scale[n];
    const double c1 = sA * static_cast<double>(s);  // fl64(sA * s32): the oracle's bias scale
    const double bq = d->bias_q ? static_cast<double>(d->bias_q[n]) : 0.0;
    bdeq[n] = bq * c1;
    const double two_e = std::ldexp(1.0, expo[n]);
    // Float noise of the oracle's own float64 dot product (|sum of terms| bound).
    const double noise = (K + 8.0) * std::ldexp(1.0, -52) * K * amax * wpmax[n];
    if (!a16) {
      alpha[n] = c1 / sO;
      corr[n] = static_cast<int64_t>(a_base - d->act_zp) * colsum_q[n];
      margin[n] = inv_sO * sA * two_e * (amax * r1[n] + noise) * kSafety;
    } else {
      alpha[n] = sA * two_e / sO;
      const int64_t sum_wp = mant[n] * colsum_q[n] + colsum_r[n];
      corr[n] = static_cast<int64_t>(128 + 32768 - d->act_zp) * sum_wp;
      margin[n] = inv_sO * sA * two_e * noise * kSafety;
      // Residue term sum_k (a_k - zp) r_k.  The GEMM and the int4 GEMV form its high-byte part
      // sum_k hi'_k r_k exactly (hi' the high activation byte minus 128); the low-byte part
      // sum_k lo'_k r_k (|lo'| <= 128) is bounded by margin_lo.  The int8 GEMV bounds the whole
      // term, per unit of R1 = sum_k |a_k - zp| (mr1).
      mr1[n] = inv_sO * sA * two_e * rmax[n] * kSafety;
      mlo[n] = inv_sO * sA * two_e * 128.0 * r1[n] * kSafety;
    }
    beta[n] = bdeq[n] / sO + d->out_zp;
    {
      // Largest |t| the GEMM epilogue can see for this column (t = acc * alpha + beta'); the
      // epilogue's rounding shortcut needs |t| < 2^31, otherwise t is clamped first.
      const double betap = std::fabs(beta[n]) + std::fabs(static_cast<double>(corr[n]) * alpha[n]);
      const double tmax = a16 ? (std::fabs(alpha[n]) * static_cast<double>(mant[n]) + std::fabs(alpha[n])) * K * 33024.0 * 127.0 + betap
                              : std::fabs(alpha[n]) * K * 128.0 * 127.0 + betap;
      if (!(tmax < 1073741824.0)) sh.epi_clamp = 1;
    }
    absb[n] = 2.0 * std::fabs(beta[n]) + 2.0 * d->out_zp + 1.0;
    mantv[n] = mant[n];
    csum[n] = colsum_q[n];
    csum_r[n] = colsum_r[n];
    alpha_e[n] = sA * two_e / sO;
    scale_exp[n] = expo[n];
    margin_exact[n] = inv_sO * sA * two_e * noise * kSafety;
    s32v[n] = s;
    biasv[n] = d->bias_q ? d->bias_q[n] : 0;
    // the exact integer GEMM shifts activations by 128 (8-bit) or 32896 (16-bit, 256 hi + lo')
    corr_int[n] = static_cast<int64_t>((a16 ? 32896 : 128) - d->act_zp) * colsum_q[n];
  }

  // ---- int4 decode GEMV: per-column records and the block scales in [N][K / block] order ------
  std::vector<GemvRec> gemv_rec;
  std::vector<uint8_t> lpbq_nk;
  if (sh.gemv_fmt == kTileI4) {
    gemv_rec.resize(N);
    for (int n = 0; n < N; ++n) {
      GemvRec &r = gemv_rec[n];
      r.alpha = alpha[n];
      r.beta = beta[n];
      r.margin = margin[n];
      r.absb = absb[n];
      r.corr = a16 ? colsum_q[n] : corr[n];
      // 16-bit acts: margin_lo.  8-bit acts: the Cauchy-Schwarz bound of the residue term per unit
      // of |a - zp|_2 (|sum_k (a_k - zp) r_k| <= |a - zp|_2 |r|_2), in output LSB.
      r.mlo = a16 ? mlo[n] : inv_sO * sA * std::ldexp(1.0, expo[n]) * std::sqrt(r2[n]) * kSafety;
      r.mant = mant[n];
      r.colsum_r = colsum_r[n];
      r.bias_deq = bdeq[n];
      r.alpha_e = alpha_e[n];
      r.margin_exact = margin_exact[n];
      r.s32 = s32v[n];
      r.pad = 0;
    }
    if (lpbq) lpbq_nk.assign(d->lpbq_block_scale, d->lpbq_block_scale + static_cast<size_t>(N) * nblk);
  }

  // ---- upload -------------------------------------------------------------------------------
  auto *p = new qh_qmm_prepared();
  p->shape = sh;
  int dev = 0;
  (void)hipGetDevice(&dev);
  p->device_id = dev;
  DevAlloc al;
  qh_status st = QH_STATUS_OK;
  QmmDevice &D = p->dev;
  std::memset(&D, 0, sizeof(D));
  if (st == QH_STATUS_OK) st = al.upload(&D.tiles, tiles);
  if (st == QH_STATUS_OK) st = al.upload(&D.gemv_tiles, gemv_tiles);
  if (st == QH_STATUS_OK) st = al.upload(&D.gemv_lpbq, gemv_lpbq);
  if (st == QH_STATUS_OK) st = al.upload(&D.lpbq_nk, lpbq_nk);
  if (st == QH_STATUS_OK) st = al.upload(&D.gemv_rec, gemv_rec);
  if (st == QH_STATUS_OK) st = al.upload(&D.alpha, alpha);
  if (st == QH_STATUS_OK) st = al.upload(&D.beta, beta);
  if (st == QH_STATUS_OK) st = al.upload(&D.corr, corr);
  if (st == QH_STATUS_OK) st = al.upload(&D.margin, margin);
  if (st == QH_STATUS_OK) st = al.upload(&D.absb, absb);
  if (st == QH_STATUS_OK) st = al.upload(&D.bias_deq, bdeq);
  if (st == QH_STATUS_OK) st = al.upload(&D.s32, s32v);
  if (st == QH_STATUS_OK) st = al.upload(&D.mant, mantv);
  if (st == QH_STATUS_OK) st = al.upload(&D.colsum, csum);
  if (st == QH_STATUS_OK) st = al.upload(&D.colsum_r, csum_r);
  if (st == QH_STATUS_OK) st = al.upload(&D.alpha_e, alpha_e);
  if (st == QH_STATUS_OK) st = al.upload(&D.scale_exp, scale_exp);
  if (st == QH_STATUS_OK) st = al.upload(&D.margin_exact, margin_exact);
  if (st == QH_STATUS_OK) st = al.upload(&D.gemv_margin_r1, mr1);
  if (st == QH_STATUS_OK && a16) st = al.upload(&D.margin_lo, mlo);
  if (st == QH_STATUS_OK && !a16) st = al.upload(&D.resid, resid);
  if (st == QH_STATUS_OK) st = al.upload(&D.bias_q, biasv);
  if (st == QH_STATUS_OK) st = al.upload(&D.corr_int, corr_int);
  if (st != QH_STATUS_OK) {
    al.release();
    delete p;
    return st;
  }
  p->device_bytes = al.bytes;
  p->gemm_weight_bytes = tiles.size();
  // Bytes one GEMV call must stream: packed codes (+ block scales) of the logical N x K.
  {
    const uint64_t codes = static_cast<uint64_t>(N) * K / (sh.gemv_fmt == kTileI8 ? 1 : 2);
    p->gemv_weight_bytes = codes + gemv_lpbq.size();
  }
  *out = p;
  return QH_STATUS_OK;
}
