// Decode-shape GEMV (M <= 4) for int4 weights, per-channel and LPBQ: one persistent workgroup
// per compute unit.
//
// Work unit: 8 output columns x the whole K.  The N / 8 units are dealt round-robin to the G
// workgroups (G = compute units), so every CU streams the same number of weight bytes (7 units
// of 16 KiB each at N = 14336, K = 4096).  Workgroup: 512 threads = 8 waves; lane (wave w,
// c = lane / 8, kq = lane % 8) takes column c of each of its units and the k-groups
// kg = 64 s + 8 w + kq (slots s < S = KG / 64, rounded up to a power of two), so one wave
// instruction reads 8 consecutive k-group rows of the GEMV stream, 128 B of each.
//
// Order of requests.  Everything small the workgroup needs (the activations, the LPBQ block
// scales of its units, the per-column epilogue records) is requested and staged in LDS before
// the weight stream starts: a wave that has requested more of the stream than the CU's memory
// pipe holds stalls in issue until it drains, so no barrier may sit behind weight requests.
// The stream is then requested D units ahead of the products (8 slots of 16 B per lane in
// flight): a wave computes unit q and then requests unit q + D.  Slots past the workgroup's
// units or past K are buffer loads with an out-of-range offset, which return zero without a
// memory request, so the request sequence is straight-line and its waits are exact.
//
// Arithmetic is that of the single-group GEMV (qmm_gemv.hip): signed activation planes staged in
// LDS with their 32-value sums (held in registers across the units for one row), v_dot4_i32_i8
// on the offset-binary nibbles, the LPBQ block scale per k-group, and for 16-bit activations the
// exact high-byte residue products from the per-(column, block scale) tables.  Partial sums meet
// over the 8 kq lanes (DPP) and the 8 waves (LDS); one thread per output requantises it.
// Outputs within the certified margin of a rounding boundary are recomputed exactly, 8 at a
// time, from the weight words the lanes still hold (handed over through LDS) and the constants
// already staged: the fixup makes no global memory request.

#include <atomic>
#include <type_traits>
#include <utility>

#include "gemv_common.h"

namespace qh {
namespace {


constexpr int kUT = 512;         // threads per workgroup
constexpr int kUW = kUT / 64;    // waves
constexpr int kUSlots = 16;      // weight slots per lane: U * S <= kUSlots
constexpr int kUMaxUnits = 10;   // units per workgroup (their records: one 16-byte piece per thread)
constexpr int kUFix = 8;         // outputs recomputed together by the float64 fixup
constexpr int kRecPieces = static_cast<int>(sizeof(GemvRec)) / 16;
constexpr uint32_t kOOB = 0x80000000u;  // buffer offset past every buffer: the load returns zero

struct UnitArgs {
  const uint8_t *act;
  void *out;
  const uint8_t *w;       // GEMV stream [N/16][KG][16 columns][16 B]
  const uint8_t *scales;  // LPBQ block scales [N][nblk]
  const GemvRec *rec;     // [N]
  uint32_t act_bytes, w_bytes, sc_bytes, rec_bytes;
  int M, N, K, KG, G, U, units, nblk, blk_shift;
  int act_zp, out_zp, out_qmax, out16;
  double sA, sO;
  int off_asum, off_sc, off_rec, off_rtab, off_red, off_fixw;
};


// Compile-time loop: f(integral_constant<int, 0>) ... f(integral_constant<int, N-1>).
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F &&f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Sum over the 8 lanes of each aligned group of 8 (the kq lanes of one column): DPP within rows.
__device__ __forceinline__ int sum8i(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
  x += __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
  x += __builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, false);  // row_half_mirror
  return x;
}

// Signed activation words of one k-group (32 values) of one row and plane, and their sum.
struct ActKG {
  uint4 a0, a1;
  int sum;
};

template <bool A16, bool LPBQ, int MM, int S>
__global__ __launch_bounds__(kUT, 1) void qmm_gemv_unit_kernel(const UnitArgs g) {
  constexpr bool HR = A16;            // 16-bit acts: exact high-byte residue products
  constexpr int QN = kUSlots / S;     // unit positions per lane
  constexpr int D = 8 / S;            // units in flight ahead of the products (8 slots)
  constexpr int kPre = D / 2;  // units requested before the staging
  constexpr int NSUM = A16 ? 3 : 1;   // partial sums per output: codes x (hi | a), x lo, hi x residues
  constexpr int P = A16 ? 2 : 1;      // activation planes
  constexpr bool AREG = MM == 1;      // one row: the lane's activation words stay in registers
  extern __shared__ uint4 smem[];
  uint8_t *const lds = reinterpret_cast<uint8_t *>(smem);
  __shared__ uint16_t fix_list[kUMaxUnits * MM * 8];   // outputs near a rounding boundary
  __shared__ uint32_t unit_rows[kUSlots];              // rows of each unit with listed outputs
  __shared__ int arow_sq[MM], arow_sum[MM];            // 8-bit acts: sum_k (a - 128)^2, sum_k (a - 128) per row
  __shared__ uint16_t fix_list2[kUMaxUnits * MM * 8];  // ... still undecided by the exact sum (fix_list slots)
  __shared__ int fix_val[kUMaxUnits * MM * 8];         // outputs of the float64 fixup, by fix_list slot
  __shared__ uint8_t fix_done[kUMaxUnits * MM * 8];     // ... set where it ran
  __shared__ int fix_cnt, fix_cnt2;
  __shared__ int xr[MM * 8 * kUW];                     // residue sums of a pass: [row][column][wave]
  __shared__ double dred[kUFix * kUW];

  // lane = 8 c + kq: column c of the unit, k-group offset kq (the 8 kq lanes of a column are an
  // aligned group of 8, summed with DPP)
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, c = lane >> 3, kq = lane & 7;
  const int M = g.M, K = g.K, KG = g.KG, U = g.U, G = g.G, units = g.units, nblk = g.nblk;
  const int b = blockIdx.x;
  int16_t *const asum = reinterpret_cast<int16_t *>(lds + g.off_asum);
  uint8_t *const lsc = lds + g.off_sc;
  GemvRec *const lrec = reinterpret_cast<GemvRec *>(lds + g.off_rec);
  uint4 *const rtab = reinterpret_cast<uint4 *>(lds + g.off_rtab);
  int *const red = reinterpret_cast<int *>(lds + g.off_red);

  // ---- 1. small requests: activations, block scales, records; staged before the stream ------
  // (a wave that has requested its share of the weight stream can stall in issue until the
  // memory pipe drains, so nothing that every wave must reach sits behind the weight requests)
  const bool a_ok = t < M * KG;
  const int am = a_ok ? t / KG : 0, akg = a_ok ? t - am * KG : 0;
  int usq = 0, usum = 0;  // 8-bit acts: this unit's sum of squares and sum of a - 128
  uint4 av[A16 ? 4 : 2];
  {
    const auto r = rsrc(g.act, g.act_bytes);
    const uint32_t off = a_ok ? static_cast<uint32_t>((am * K + akg * 32) * (A16 ? 2 : 1)) : kOOB;
#pragma unroll
    for (int q = 0; q < (A16 ? 4 : 2); ++q) av[q] = bload16(r, off + 16 * q);
  }
  const int sq = t / (LPBQ ? nblk : 1), sj = t - sq * (LPBQ ? nblk : 1);
  const bool s_ok = LPBQ && sq < U && b + G * sq < units;
  uint2 scv = make_uint2(0u, 0u);
  if (LPBQ) {
    const auto r = rsrc(g.scales, g.sc_bytes);
    scv = bload8(r, s_ok ? static_cast<uint32_t>((b + G * sq) * 8 * nblk + 8 * sj) : kOOB);
  }
  const int rq = t / (8 * kRecPieces), rj = t - rq * (8 * kRecPieces);
  const bool r_ok = rq < U && b + G * rq < units;
  uint4 rcv;
  {
    const auto r = rsrc(g.rec, g.rec_bytes);
    rcv = bload16(r, r_ok ? static_cast<uint32_t>((b + G * rq) * 8 * static_cast<int>(sizeof(GemvRec)) + 16 * rj) : kOOB);
  }
  // ---- 2. the weight stream, D units ahead of the products ------------------------------------
  // The first kPre units are requested before the staging waits: they keep the memory system busy
  // during the small requests' latency, and are few enough not to stall any wave's issue.
  uint4 wv[kUSlots];
  const auto rw = rsrc(g.w, g.w_bytes);
  auto issue_unit = [&](auto qc) {
    constexpr int q = decltype(qc)::value;
    const int u = b + G * q;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int kg = 64 * s + 8 * w + kq;
      const bool ok = q < U && u < units && kg < KG;
      const uint32_t off = static_cast<uint32_t>((((u >> 1) * KG + kg) * 16 + 8 * (u & 1) + c) * 16);
      wv[q * S + s] = bload16<kNT>(rw, ok ? off : kOOB);
    }
  };
  static_for<kPre>([&](auto qc) { issue_unit(qc); });

  if (a_ok) {
    if (!A16) {
      uint4 v0 = av[0], v1 = av[1];
      v0.x ^= 0x80808080u; v0.y ^= 0x80808080u; v0.z ^= 0x80808080u; v0.w ^= 0x80808080u;
      v1.x ^= 0x80808080u; v1.y ^= 0x80808080u; v1.z ^= 0x80808080u; v1.w ^= 0x80808080u;
      uint4 *dst = reinterpret_cast<uint4 *>(lds + static_cast<size_t>(am) * K + akg * 32);
      dst[0] = v0;
      dst[1] = v1;
      int sm = bsum4(v0.x, 0);
      sm = bsum4(v0.y, sm); sm = bsum4(v0.z, sm); sm = bsum4(v0.w, sm);
      sm = bsum4(v1.x, sm); sm = bsum4(v1.y, sm); sm = bsum4(v1.z, sm); sm = bsum4(v1.w, sm);
      asum[t] = static_cast<int16_t>(sm);
      int sq = sdot4(v0.x, v0.x, 0);
      sq = sdot4(v0.y, v0.y, sq); sq = sdot4(v0.z, v0.z, sq); sq = sdot4(v0.w, v0.w, sq);
      sq = sdot4(v1.x, v1.x, sq); sq = sdot4(v1.y, v1.y, sq); sq = sdot4(v1.z, v1.z, sq); sq = sdot4(v1.w, v1.w, sq);
      usq = sq;
      usum = sm;
    } else {
      // a - 32768 = 256 hi + lo' + 128: bytes of (a ^ 0x8080) are hi and lo' (signed)
      uint32_t hv[8], lv[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint4 v = av[q];
        v.x ^= 0x80808080u; v.y ^= 0x80808080u; v.z ^= 0x80808080u; v.w ^= 0x80808080u;
        hv[2 * q] = perm(v.y, v.x, 0x07050301u);
        hv[2 * q + 1] = perm(v.w, v.z, 0x07050301u);
        lv[2 * q] = perm(v.y, v.x, 0x06040200u);
        lv[2 * q + 1] = perm(v.w, v.z, 0x06040200u);
      }
      uint4 *dh = reinterpret_cast<uint4 *>(lds + static_cast<size_t>(am) * K + akg * 32);
      uint4 *dl = reinterpret_cast<uint4 *>(lds + static_cast<size_t>(M + am) * K + akg * 32);
      dh[0] = make_uint4(hv[0], hv[1], hv[2], hv[3]);
      dh[1] = make_uint4(hv[4], hv[5], hv[6], hv[7]);
      dl[0] = make_uint4(lv[0], lv[1], lv[2], lv[3]);
      dl[1] = make_uint4(lv[4], lv[5], lv[6], lv[7]);
      int sh = 0, sl = 0;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        sh = bsum4(hv[j], sh);
        sl = bsum4(lv[j], sl);
      }
      asum[t] = static_cast<int16_t>(sh);
      asum[M * KG + t] = static_cast<int16_t>(sl);
    }
  }
  if (s_ok) *reinterpret_cast<uint2 *>(lsc + sq * 8 * nblk + 8 * sj) = scv;
  if (r_ok) *reinterpret_cast<uint4 *>(lds + g.off_rec + (rq * 8 * kRecPieces + rj) * 16) = rcv;
  if (t == 0) {
    fix_cnt = 0;
    fix_cnt2 = 0;
  }
  if (t < kUSlots) unit_rows[t] = 0;
  if (t < MM) {
    arow_sq[t] = 0;
    arow_sum[t] = 0;
  }
  lds_barrier();
  if (!A16 && a_ok) {
    atomicAdd(&arow_sq[am], usq);
    atomicAdd(&arow_sum[am], usum);
  }
  // the rest of the first D units
  static_for<D>([&](auto qc) {
    if constexpr (decltype(qc)::value >= kPre) issue_unit(qc);
  });
  // residue tables of the units' columns, one (column, block scale) entry per thread and step,
  // built while the first units of the stream are in flight (16-bit acts use them in every
  // product, 8-bit acts in the exact fixup)
  for (int e = t; e < U * 8 * kRtabF; e += kUT) {
    const int ci = e / kRtabF;
    rtab[e] = resid_table(static_cast<int>(lrec[ci].mant), e - ci * kRtabF);
  }
  lds_barrier();


  // one row: the lane's activation words and sums for its S k-groups, for every unit
  ActKG ar[AREG ? S : 1][AREG ? P : 1];
  if constexpr (AREG) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int kg = min(64 * s + 8 * w + kq, KG - 1);
#pragma unroll
      for (int pl = 0; pl < P; ++pl) {
        const uint4 *ap = reinterpret_cast<const uint4 *>(lds + static_cast<size_t>(pl) * K + kg * 32);
        ar[s][pl].a0 = ap[0];
        ar[s][pl].a1 = ap[1];
        ar[s][pl].sum = asum[pl * KG + kg];
      }
    }
  }

  // ---- 3. products, unit by unit; the unit D ahead is requested after each ---------------------
  static_for<QN>([&](auto qc) {
    constexpr int q = decltype(qc)::value;
    if (q < U) {  // wave-uniform
      const bool u_ok = b + G * q < units;
      int acc[MM], acc2[MM], acc3[MM];
#pragma unroll
      for (int m = 0; m < MM; ++m) acc[m] = acc2[m] = acc3[m] = 0;
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const int kg_raw = 64 * s + 8 * w + kq;
        const bool valid = u_ok && kg_raw < KG;
        const int kg = valid ? kg_raw : 0;
        const uint4 v = wv[q * S + s];
        const uint32_t m4 = valid ? 0x0F0F0F0Fu : 0u;
        uint32_t wd[8];
        wd[0] = v.x & m4; wd[1] = v.y & m4; wd[2] = v.z & m4; wd[3] = v.w & m4;
        wd[4] = (v.x >> 4) & m4; wd[5] = (v.y >> 4) & m4; wd[6] = (v.z >> 4) & m4; wd[7] = (v.w >> 4) & m4;
        const int a8 = valid ? 8 : 0;  // the -8 offset of the unsigned nibble codes
        const int f = LPBQ ? static_cast<int>(lsc[(q * 8 + c) * nblk + (kg >> g.blk_shift)]) : 1;
        uint32_t rr[HR ? 8 : 1];
        if constexpr (HR) {
          const uint4 tab = rtab[(q * 8 + c) * kRtabF + (valid ? f : 0)];
#pragma unroll
          for (int j = 0; j < 8; ++j) rr[j] = resid4(wd[j], tab);
        }
#pragma unroll
        for (int m = 0; m < MM; ++m) {
          if (MM > 1 && m >= M) continue;
          ActKG ah, al;
          if constexpr (AREG) {
            ah = ar[s][0];
            if constexpr (A16) al = ar[s][P - 1];
          } else {
            const uint4 *ap = reinterpret_cast<const uint4 *>(lds + static_cast<size_t>(m) * K + kg * 32);
            ah.a0 = ap[0];
            ah.a1 = ap[1];
            ah.sum = asum[m * KG + kg];
            if constexpr (A16) {
              const uint4 *lp = reinterpret_cast<const uint4 *>(lds + static_cast<size_t>(M + m) * K + kg * 32);
              al.a0 = lp[0];
              al.a1 = lp[1];
              al.sum = asum[(M + m) * KG + kg];
            }
          }
          int d = sdot4(ah.a0.x, wd[0], 0);
          d = sdot4(ah.a0.y, wd[1], d); d = sdot4(ah.a0.z, wd[2], d); d = sdot4(ah.a0.w, wd[3], d);
          d = sdot4(ah.a1.x, wd[4], d); d = sdot4(ah.a1.y, wd[5], d); d = sdot4(ah.a1.z, wd[6], d); d = sdot4(ah.a1.w, wd[7], d);
          d -= a8 * ah.sum;
          acc[m] += LPBQ ? d * f : d;
          if constexpr (A16) {
            int e = sdot4(al.a0.x, wd[0], 0);
            e = sdot4(al.a0.y, wd[1], e); e = sdot4(al.a0.z, wd[2], e); e = sdot4(al.a0.w, wd[3], e);
            e = sdot4(al.a1.x, wd[4], e); e = sdot4(al.a1.y, wd[5], e); e = sdot4(al.a1.z, wd[6], e); e = sdot4(al.a1.w, wd[7], e);
            e -= a8 * al.sum;
            acc2[m] += LPBQ ? e * f : e;
            int h = sdot4(ah.a0.x, rr[0], acc3[m]);
            h = sdot4(ah.a0.y, rr[1], h); h = sdot4(ah.a0.z, rr[2], h); h = sdot4(ah.a0.w, rr[3], h);
            h = sdot4(ah.a1.x, rr[4], h); h = sdot4(ah.a1.y, rr[5], h); h = sdot4(ah.a1.z, rr[6], h); h = sdot4(ah.a1.w, rr[7], h);
            acc3[m] = h;
          }
        }
      }
      // sums over the 8 kq lanes of each column, then this wave's partials into LDS
#pragma unroll
      for (int m = 0; m < MM; ++m) {
        if (MM > 1 && m >= M) continue;
        int x[NSUM];
        x[0] = sum8i(acc[m]);
        if constexpr (A16) {
          x[1] = sum8i(acc2[m]);
          x[2] = sum8i(acc3[m]);
        }
        if (kq == 0) {
#pragma unroll
          for (int k = 0; k < NSUM; ++k) red[(((k * U + q) * MM + m) * kUW + w) * 8 + c] = x[k];
        }
      }
    }
    if constexpr (q + D < QN) issue_unit(std::integral_constant<int, q + D>{});
  });
  lds_barrier();

  // ---- 4. requantisation: thread t owns output (unit q, row m, column c) ------------------------
  // Every output is stored at the very end: a store in flight counts in vmcnt like a load, and
  // the waits the fixups need would otherwise wait for the stores too.
  const int oq = t / (MM * 8), om = (t / 8) % MM, oc = t & 7;
  const bool owner = oq < U && om < M && b + G * oq < units;
  bool myamb = false;
  int oval = 0, myslot = -1;
  long long Dint = 0;
  if (owner) {
    const GemvRec &rc = lrec[oq * 8 + oc];
    int Sx[NSUM];
#pragma unroll
    for (int k = 0; k < NSUM; ++k) {
      Sx[k] = 0;
#pragma unroll
      for (int ww = 0; ww < kUW; ++ww) Sx[k] += red[(((k * U + oq) * MM + om) * kUW + ww) * 8 + oc];
    }
    double tv, slack;
    if constexpr (A16) {
      // D = sum_k (a - zp) (w M + r) but for sum_k lo'_k r_k, bounded by mlo:
      //   M S + 256 sum hi' r + (32896 - zp) sum r
      const int64_t shift = static_cast<int64_t>(128 + 32768 - g.act_zp);
      const int64_t Sv = 256 * static_cast<int64_t>(Sx[0]) + Sx[1] + rc.corr * shift;
      const int64_t D = Sv * rc.mant + 256 * static_cast<int64_t>(Sx[2]) + shift * rc.colsum_r;
      Dint = D;
      tv = fma(static_cast<double>(D), rc.alpha, rc.beta);
      slack = rc.margin + rc.mlo + 0x1p-48 * (fabs(tv) + rc.absb);
    } else {
      // S = sum_k (a - zp) w; the residue term sum_k (a - zp) r is bounded by the margin
      // (max |a - zp| sum_k |r_k|) or by |a - zp|_2 |r|_2, whichever is smaller
      const int64_t Sv = static_cast<int64_t>(Sx[0]) + rc.corr;
      Dint = Sv;
      tv = fma(static_cast<double>(Sv), rc.alpha, rc.beta);
      const double dz = static_cast<double>(128 - g.act_zp);
      const double a2 = static_cast<double>(arow_sq[om]) + 2.0 * dz * static_cast<double>(arow_sum[om]) + K * dz * dz;
      slack = fmin(rc.margin, rc.margin_exact + rc.mlo * sqrt(a2)) + 0x1p-48 * (fabs(tv) + rc.absb);
    }
    const double fl = floor(tv);
    const bool near_tie = fabs((tv - fl) - 0.5) <= slack;
    const double lo = fmin(fmax(fl, 0.0), static_cast<double>(g.out_qmax));
    const double hi = fmin(fmax(fl + 1.0, 0.0), static_cast<double>(g.out_qmax));
    myamb = near_tie && lo != hi;
    oval = static_cast<int>(fmin(fmax(rint(tv), 0.0), static_cast<double>(g.out_qmax)));
    if (myamb) atomicOr(&unit_rows[oq], 1u << om);
  }
  lds_barrier();

  // ---- 5. exact residue sums of the listed outputs ---------------------------------------------
  // The sum the margin bounded is formed exactly: sum_k (a_k - 128) r_k (8-bit acts) or
  // sum_k lo'_k r_k (16-bit acts), r_k the float32 rounding residue of weight k, from the
  // (column, block scale) residue table.  With it the dot product D = sum_k (a_k - zp) (w_k M +
  // r_k) is exact, and t = D alpha_e + beta is certain unless it lies within the oracle's own
  // float64 noise of a tie; those few go on to the float64 recomputation (section 6).  One pass
  // per (unit, row) with listed outputs: every lane forms the sum of its own column from the
  // weight words in its registers, so the pass serves all 8 columns of the unit at once.
  static_for<QN>([&](auto qc) {
    constexpr int qf = decltype(qc)::value;
    if (qf < U) {
      uint32_t rows = unit_rows[qf];
      while (rows != 0) {
        const int em = __builtin_ctz(rows);
        rows &= rows - 1;
        int part = 0;
#pragma unroll
        for (int s2 = 0; s2 < S; ++s2) {
          const int kg_raw = 64 * s2 + 8 * w + kq;
          const bool valid = kg_raw < KG;
          const int kg = valid ? kg_raw : 0;
          const uint32_t m4 = valid ? 0x0F0F0F0Fu : 0u;
          const uint4 v = wv[qf * S + s2];
          const int f = valid ? (LPBQ ? static_cast<int>(lsc[(qf * 8 + c) * nblk + (kg >> g.blk_shift)]) : 1) : 0;
          const uint4 tab = rtab[(qf * 8 + c) * kRtabF + f];
          uint4 a0, a1;  // 8-bit acts: a - 128; 16-bit acts: the low bytes lo'
          if constexpr (AREG) {
            a0 = ar[s2][P - 1].a0;
            a1 = ar[s2][P - 1].a1;
          } else {
            const uint4 *ap = reinterpret_cast<const uint4 *>(lds + static_cast<size_t>((A16 ? M : 0) + em) * K + kg * 32);
            a0 = ap[0];
            a1 = ap[1];
          }
          part = sdot4(a0.x, resid4(v.x & m4, tab), part);
          part = sdot4(a0.y, resid4(v.y & m4, tab), part);
          part = sdot4(a0.z, resid4(v.z & m4, tab), part);
          part = sdot4(a0.w, resid4(v.w & m4, tab), part);
          part = sdot4(a1.x, resid4((v.x >> 4) & m4, tab), part);
          part = sdot4(a1.y, resid4((v.y >> 4) & m4, tab), part);
          part = sdot4(a1.z, resid4((v.z >> 4) & m4, tab), part);
          part = sdot4(a1.w, resid4((v.w >> 4) & m4, tab), part);
        }
        part = sum8i(part);
        if (kq == 0) xr[(em * 8 + c) * kUW + w] = part;
        lds_barrier();
        // the owners of this (unit, row)'s listed outputs finish them
        if (myamb && oq == qf && om == em) {
          const GemvRec &rc = lrec[oq * 8 + oc];
          long long X = 0;
#pragma unroll
          for (int ww = 0; ww < kUW; ++ww) X += xr[(em * 8 + oc) * kUW + ww];
          long long D;
          if constexpr (A16)
            D = Dint + X;
          else
            D = Dint * rc.mant + X + static_cast<long long>(128 - g.act_zp) * rc.colsum_r;
          const double tv = fma(static_cast<double>(D), rc.alpha_e, rc.beta);
          const double slack = rc.margin_exact + 0x1p-48 * (fabs(tv) + rc.absb);
          const double fl = floor(tv);
          const double lo = fmin(fmax(fl, 0.0), static_cast<double>(g.out_qmax));
          const double hi = fmin(fmax(fl + 1.0, 0.0), static_cast<double>(g.out_qmax));
          if (fabs((tv - fl) - 0.5) <= slack && lo != hi) {
            myslot = atomicAdd(&fix_cnt, 1);
            fix_list[myslot] = static_cast<uint16_t>((oq * MM + om) * 8 + oc);
            fix_done[myslot] = 0;
            fix_list2[atomicAdd(&fix_cnt2, 1)] = static_cast<uint16_t>(myslot);
          } else {
            oval = static_cast<int>(fmin(fmax(rint(tv), 0.0), static_cast<double>(g.out_qmax)));
          }
        }
        lds_barrier();  // xr is rewritten by the next pass
      }
    }
  });
  uint4 *const fixw = reinterpret_cast<uint4 *>(lds + g.off_fixw);  // [kUFix][KG] weight words
  const int nfix = fix_cnt2;

  // ---- 6. float64 fixup of the outputs at the oracle's own noise level, kUFix at a time --------
  const int off = (A16 ? 32768 + 128 : 128) - g.act_zp;  // a - zp = plane value + off
  for (int e0 = 0; e0 < nfix; e0 += kUFix) {
    const int nb = min(kUFix, nfix - e0);
    // the lanes holding an entry's column hand over its weight words
    for (int e = 0; e < nb; ++e) {
      const int tt = fix_list[fix_list2[e0 + e]];
      const int eq = tt / (MM * 8), ec = tt & 7;
      if (c != ec) continue;
#pragma unroll
      for (int i = 0; i < kUSlots; ++i) {
        const int kg = 64 * (i % S) + 8 * w + kq;
        if (i / S == eq && kg < KG) fixw[e * KG + kg] = wv[i];
      }
    }
    lds_barrier();
    // thread t takes 16 terms (k-group kg, half h) of each entry
    double sacc[kUFix];
    int ecol[kUFix], erow[kUFix];
    float esc[kUFix];
#pragma unroll
    for (int e = 0; e < kUFix; ++e) {
      sacc[e] = 0.0;
      const int tt = fix_list[fix_list2[e0 + (e < nb ? e : 0)]];
      ecol[e] = (tt / (MM * 8)) * 8 + (tt & 7);  // unit-local column index q * 8 + c
      erow[e] = (tt / 8) % MM;
      esc[e] = lrec[ecol[e]].s32;
    }
    for (int uu = t; uu < 2 * KG; uu += kUT) {
      const int kg = uu >> 1, h = uu & 1;  // terms k = 32 kg + 16 h + j, j < 16
#pragma unroll
      for (int e = 0; e < kUFix; ++e) {
        if (e >= nb) break;
        const uint4 v = fixw[e * KG + kg];
        const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
        const int f = LPBQ ? lsc[ecol[e] * nblk + (kg >> g.blk_shift)] : 1;
        const int8_t *hp = reinterpret_cast<const int8_t *>(lds + static_cast<size_t>(erow[e]) * K + kg * 32 + 16 * h);
        const int8_t *lp = reinterpret_cast<const int8_t *>(lds + static_cast<size_t>(M + erow[e]) * K + kg * 32 + 16 * h);
#pragma unroll 4
        for (int j = 0; j < 16; ++j) {
          const uint32_t byte = (wd[j >> 2] >> (8 * (j & 3))) & 0xFFu;
          const int wq = ((h ? (byte >> 4) : (byte & 15u)) - 8) * f;
          const int a = (A16 ? 256 * static_cast<int>(hp[j]) + lp[j] : static_cast<int>(hp[j])) + off;
          const float wf = static_cast<float>(wq) * esc[e];
          sacc[e] = fma(static_cast<double>(a) * g.sA, static_cast<double>(wf), sacc[e]);
        }
      }
    }
#pragma unroll
    for (int e = 0; e < kUFix; ++e) {
      if (e >= nb) break;
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) sacc[e] += __shfl_xor(sacc[e], o, 64);
      if (lane == 0) dred[e * kUW + w] = sacc[e];
    }
    lds_barrier();
    if (t < nb) {
      const int slot = fix_list2[e0 + t];
      const int tt = fix_list[slot];
      const GemvRec &rc = lrec[(tt / (MM * 8)) * 8 + (tt & 7)];
      double tot = 0.0;
#pragma unroll
      for (int ww = 0; ww < kUW; ++ww) tot += dred[t * kUW + ww];
      const double tvx = (tot + rc.bias_deq) / g.sO + static_cast<double>(g.out_zp);
      fix_val[slot] = static_cast<int>(fmin(fmax(rint(tvx), 0.0), static_cast<double>(g.out_qmax)));
      fix_done[slot] = 1;
    }
    lds_barrier();  // fixw, dred and the fixed outputs
  }

  // ---- 7. the outputs ------------------------------------------------------------------------------
  if (owner) {
    if (myslot >= 0 && fix_done[myslot]) oval = fix_val[myslot];
    const size_t idx = static_cast<size_t>(om) * g.N + 8 * (b + G * oq) + oc;
    if (g.out16)
      static_cast<uint16_t *>(g.out)[idx] = static_cast<uint16_t>(oval);
    else
      static_cast<uint8_t *>(g.out)[idx] = static_cast<uint8_t>(oval);
  }
}

size_t al16(size_t x) { return (x + 15) & ~static_cast<size_t>(15); }

int cu_count() { return device_cu_count(); }

template <bool A16, bool LPBQ, int MM, int S>
qh_status launch_unit(const UnitArgs &g, size_t dyn, hipStream_t stream) {
  const auto kernel = &qmm_gemv_unit_kernel<A16, LPBQ, MM, S>;
  // bit d: the dynamic-LDS limit is raised on device d (set once per device and instantiation;
  // threads that race here both set the same attribute, which is harmless)
  static std::atomic<uint64_t> attr_set{0};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= 64) return fail(QH_STATUS_UNSUPPORTED, "GEMV: device index %d", dev);
  const uint64_t bit = uint64_t{1} << dev;
  if (!(attr_set.load(std::memory_order_acquire) & bit)) {
    e = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                            150 * 1024);
    if (e != hipSuccess) return hip_fail(e, "hipFuncSetAttribute(qmm_gemv_unit_kernel)");
    attr_set.fetch_or(bit, std::memory_order_release);
  }
  hipLaunchKernelGGL(kernel, dim3(g.G), dim3(kUT), dyn, stream, g);
  e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "qmm_gemv_unit_kernel launch");
  return QH_STATUS_OK;
}

template <bool A16, bool LPBQ, int MM>
qh_status launch_s(const UnitArgs &g, int S, size_t dyn, hipStream_t stream) {
  if (S == 1) return launch_unit<A16, LPBQ, MM, 1>(g, dyn, stream);
  if (S == 2) return launch_unit<A16, LPBQ, MM, 2>(g, dyn, stream);
  return launch_unit<A16, LPBQ, MM, 4>(g, dyn, stream);
}

}  // namespace

int device_cu_count() {
  // per device; 0 = not queried yet (concurrent first queries store the same value)
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

qh_status launch_qmm_gemv_unit(const qh_qmm_prepared *p, int m, const void *act, void *out, hipStream_t stream) {
  const QmmShape &sh = p->shape;
  const QmmDevice &D = p->dev;
  const bool lpbq = sh.wfmt == QH_WEIGHT_I4_LPBQ;
  const bool a16 = sh.act_bits == 16;
  if (sh.gemv_fmt != kTileI4 || D.gemv_rec == nullptr || m < 1 || m > 4) return QH_STATUS_SHAPE_UNSUPPORTED;
  const int N = sh.N, K = sh.K, KG = K / 32;
  const int G0 = cu_count();
  if (G0 <= 0) return QH_STATUS_SHAPE_UNSUPPORTED;
  const int units = N / 8;
  const int G = units < G0 ? units : G0;
  const int U = (units + G - 1) / G;
  const int S = KG <= 64 ? 1 : KG <= 128 ? 2 : KG <= 256 ? 4 : 0;
  const int nblk = lpbq ? K / sh.lpbq_block : 1;
  const int MM = m == 1 ? 1 : 4;
  if (S == 0 || U * S > kUSlots || U > kUMaxUnits || m * KG > kUT || (lpbq && U * nblk > kUT))
    return QH_STATUS_SHAPE_UNSUPPORTED;
  const uint64_t w_bytes = static_cast<uint64_t>(N) * K / 2;
  if (w_bytes >= kOOB) return QH_STATUS_SHAPE_UNSUPPORTED;
  // dynamic LDS: activation planes, k-group sums, block scales, records, residue tables,
  // partial sums, fixup weight words
  const int P = a16 ? 2 : 1;
  const int nsum = a16 ? 3 : 1;
  UnitArgs g{};
  size_t o = al16(static_cast<size_t>(P) * m * K);
  g.off_asum = static_cast<int>(o);
  o = al16(o + static_cast<size_t>(P) * m * KG * 2);
  g.off_sc = static_cast<int>(o);
  o = al16(o + (lpbq ? static_cast<size_t>(U) * 8 * nblk : 0));
  g.off_rec = static_cast<int>(o);
  o = al16(o + static_cast<size_t>(U) * 8 * sizeof(GemvRec));
  g.off_rtab = static_cast<int>(o);
  o = al16(o + static_cast<size_t>(U) * 8 * kRtabF * 16);
  g.off_red = static_cast<int>(o);
  o = al16(o + static_cast<size_t>(nsum) * U * MM * kUW * 8 * 4);
  g.off_fixw = static_cast<int>(o);
  o = al16(o + static_cast<size_t>(kUFix) * KG * 16);
  if (o > 150 * 1024) return QH_STATUS_SHAPE_UNSUPPORTED;
  g.act = static_cast<const uint8_t *>(act);
  g.out = out;
  g.w = D.gemv_tiles;
  g.scales = D.lpbq_nk;
  g.rec = D.gemv_rec;
  g.act_bytes = static_cast<uint32_t>(static_cast<size_t>(m) * K * (a16 ? 2 : 1));
  g.w_bytes = static_cast<uint32_t>(w_bytes);
  g.sc_bytes = lpbq ? static_cast<uint32_t>(static_cast<size_t>(N) * nblk) : 0u;
  g.rec_bytes = static_cast<uint32_t>(static_cast<size_t>(N) * sizeof(GemvRec));
  g.M = m;
  g.N = N;
  g.K = K;
  g.KG = KG;
  g.G = G;
  g.U = U;
  g.units = units;
  g.nblk = nblk;
  g.blk_shift = lpbq && sh.lpbq_block == 64 ? 1 : 0;
  g.act_zp = sh.act_zp;
  g.out_zp = sh.out_zp;
  g.out_qmax = (1 << sh.out_bits) - 1;
  g.out16 = sh.out_bits == 16;
  g.sA = sh.act_scale;
  g.sO = sh.out_scale;
  if (!a16) {
    if (lpbq) return MM == 1 ? launch_s<false, true, 1>(g, S, o, stream) : launch_s<false, true, 4>(g, S, o, stream);
    return MM == 1 ? launch_s<false, false, 1>(g, S, o, stream) : launch_s<false, false, 4>(g, S, o, stream);
  }
  if (lpbq) return MM == 1 ? launch_s<true, true, 1>(g, S, o, stream) : launch_s<true, true, 4>(g, S, o, stream);
  return MM == 1 ? launch_s<true, false, 1>(g, S, o, stream) : launch_s<true, false, 4>(g, S, o, stream);
}

}  // namespace qh
