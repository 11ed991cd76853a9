// GDN chunk recurrence (stage B of the chunked gated delta rule), C = 64, D = 128:
// for every chunk of a (batch, head) sequence, in order, with the state S (D x D) carried,
//     q^ = l2norm(q) / sqrt(D),  k^ = l2norm(k),  g = cumsum(gc) inside the chunk,
//     P     = (q^ k^T) * e^{g_i - g_j}   (j <= i, else 0)
//     v_new = U - W S
//     o     = (q^ * e^g) S + P v_new
//     S     = S e^{g_last} + (k^ * e^{g_last - g})^T v_new
// from the stage-A outputs U = T (beta v) and W = T (beta k^ e^g)
// (scripts/gdn_ref_kernel.py:66-69,91-101; the chunk loop :104-131).
//
// One workgroup (8 waves) per sequence walks its chunks.  S lives in registers for the whole
// sequence: wave w owns S's value columns 16w .. 16w+15 as eight 16 x 16 MFMA result tiles,
// which is also the layout the MFMA reads as a B operand over pairs of key blocks (pair layout,
// bf16_split.h), so W S and q S take S straight from the accumulators.  q and k stay the bf16
// values they arrive as (exact MFMA operands); their l2norm factors scale the products' rows and
// columns instead.  Per chunk:
//   L. q, k rows and W (bf16 hi | lo words) into LDS; the row norms (8-lane DPP
//      sums); g's prefix sum (64-lane DPP scan), e^g and e^{g_last - g} by one wave;
//   M. each wave: W S and q S for its 16 value columns (4 token tiles), v_new = U - W S with U
//      from registers, o's first term e^g q^ S; the 10 lower 16 x 16 tiles of q k^T over the
//      waves, scaled by the norms and decays, into LDS as P;
//   O. o = e^g q^ S + P v_new for the wave's columns (causal tiles only), stored;
//   S. S = e^{g_last} S + k^T ((e^{g_last - g} / |k|) v_new), k^T read from the k rows by LDS
//      transpose reads.
// The next chunk's q, k, W, U and gc are read into registers during M, so their latency
// overlaps this chunk's products; the workgroup issues them before its stores of o.
// Precision: QH_GDN_FP32 carries W, S, P and v_new as bf16 hi/lo splits (hi*hi + hi*lo + lo*hi,
// fp32 accumulation; products with the exact q, k take two terms); QH_GDN_BF16 uses the hi
// parts only.  Norms, decays and the prefix sum are fp32.

#include <type_traits>

#include "bf16_split.h"
#include "lane_ops.h"
#include "qmm_internal.h"

namespace qh {
namespace {

using namespace bf16s;

constexpr int kC = 64;          // chunk (tokens)
constexpr int kD = 128;         // head dimension
constexpr int kThreads = 512;   // 8 waves
constexpr int kQs = kD + 8;     // LDS row stride of the q / k stores, bf16 (16-byte aligned rows)
constexpr int kRs = kD + 4;     // LDS row stride of the W store, words
constexpr int kPs = kC + 4;     // LDS row stride of P, words

struct StateArgs {
  const uint16_t *q, *k;  // bf16 [B][T][H][D]
  const float *g;         // [B][T][H] per-token log decays
  const void *w, *u;      // [B][T][H][D] bf16 or fp32 (stage-A outputs, W in the e^g form)
  const float *s_in;      // [B][H][D][D] or nullptr (zero state)
  float *s_out;           // [B][H][D][D]
  void *o;                // [B][T][H][D] bf16 or fp32
  int B, T, H, nchunks;
};

__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ float bf16f(uint32_t h) { return __uint_as_float(h << 16); }

// One chunk's inputs as read from global memory, per thread: the row segment (token t / 8,
// columns 16 (t % 8) ..) of q, k and W, this wave's U tiles (MFMA result layout) and one gc
// value per lane (every wave reads the same 64; wave 0 uses them).
template <bool WU_F32, int RP>
struct ChunkIn {
  uint4 q[RP][2], k[RP][2];
  uint4 w[RP][WU_F32 ? 4 : 2];
  float u[4][4];
  float gc;
};

// Per-lane element offsets of chunk 0 (a chunk adds 64 H D): the thread's first row segment
// (token t / 8, or t / 8 + 32 r for its r-th), its wave's U / o tile elements (token 4 qd + e of
// tile i is + (16 i + e) H D) and lane's gc.
struct Offsets {
  uint32_t row, tile, g;
  uint32_t tok;  // H D: one token
};

__device__ __forceinline__ Offsets offsets(const StateArgs &a, int b, int h, int t, int wave, int lane) {
  const int row = t >> 3, seg = t & 7, r16 = lane & 15, qd = lane >> 4;
  const uint32_t tok = static_cast<uint32_t>(a.H) * kD;
  const uint32_t seq = (static_cast<uint32_t>(b) * a.T * a.H + h) * kD;  // token 0 of the sequence
  return {seq + row * tok + 16 * seg, seq + 4 * qd * tok + 16 * wave + r16,
          static_cast<uint32_t>(b) * a.T * a.H + lane * a.H + h, tok};
}

template <bool WU_F32, int RP>
__device__ __forceinline__ void load_chunk(const StateArgs &a, const Offsets &of, int n, ChunkIn<WU_F32, RP> &in) {
  const uint32_t c0 = static_cast<uint32_t>(n) * kC * of.tok;
#pragma unroll
  for (int r = 0; r < RP; ++r) {
    const uint32_t ri = of.row + c0 + static_cast<uint32_t>(32 * r) * of.tok;
    const uint4 *qp = reinterpret_cast<const uint4 *>(a.q + ri);
    const uint4 *kp = reinterpret_cast<const uint4 *>(a.k + ri);
    in.q[r][0] = qp[0];
    in.q[r][1] = qp[1];
    in.k[r][0] = kp[0];
    in.k[r][1] = kp[1];
    if constexpr (WU_F32) {
      const uint4 *wp = reinterpret_cast<const uint4 *>(static_cast<const float *>(a.w) + ri);
#pragma unroll
      for (int x = 0; x < 4; ++x) in.w[r][x] = wp[x];
    } else {
      const uint4 *wp = reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(a.w) + ri);
      in.w[r][0] = wp[0];
      in.w[r][1] = wp[1];
    }
  }
  const uint32_t ti = of.tile + c0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t ui = ti + static_cast<uint32_t>(16 * i + e) * of.tok;
      in.u[i][e] = WU_F32 ? static_cast<const float *>(a.u)[ui] : bf16f(static_cast<const uint16_t *>(a.u)[ui]);
    }
  }
  in.gc = a.g[of.g + static_cast<uint32_t>(n) * kC * static_cast<uint32_t>(a.H)];
}

// 8 bf16 values of a uint4 as floats.
__device__ __forceinline__ void unbf16x8(const uint4 v, float *f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    f[2 * x] = bf16f(w[x] & 0xFFFFu);
    f[2 * x + 1] = bf16f(w[x] >> 16);
  }
}

// The 10 lower 16 x 16 tiles of P (token tile i >= j), two for waves 0 and 1.
__device__ __forceinline__ void p_tile(int idx, int &i, int &j) {
  i = idx < 1 ? 0 : idx < 3 ? 1 : idx < 6 ? 2 : 3;
  j = idx - i * (i + 1) / 2;
}

// Four consecutive bf16 of an LDS row (8-byte aligned) as an exact operand half.
__device__ __forceinline__ Half4 bf16x4(const uint16_t *p) {
  const uint2 v = *reinterpret_cast<const uint2 *>(p);
  return exact4(v.x, v.y);
}

// 4 bf16 of one column of a row-major LDS tile, by a transposing LDS read (ds_read_b64_tr_b16):
// in each group of 16 lanes, lane j receives element j % 4 of the 8 bytes addressed by lane
// 4 e + j / 4 as its element e.  So if lane 4 e + a of the group addresses row r0 + e, columns
// c0 + 4 a .. + 3, lane j receives rows r0 .. r0 + 3 of column c0 + j.
__device__ __forceinline__ Half4 bf16x4_tr(const uint16_t *p) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  const v4s r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s *)(p));
  const uint2 v = __builtin_bit_cast(uint2, r);
  return exact4(v.x, v.y);
}
template <bool SPLIT, bool WU_F32, bool OUT_F32>
__global__ __launch_bounds__(kThreads) void gdn_state_kernel(StateArgs a) {
  constexpr int RP = 8 * 64 / kThreads;  // row segments (16 columns of one token) per thread in L
  // q, k rows as given (bf16, exact MFMA operands) with their l2norm factors; W and the lower
  // tiles of P as hi | lo words with SPLIT, as bf16 (hi) without; g, e^g, e^{g_last - g}
  using LW = std::conditional_t<SPLIT, uint32_t, uint16_t>;
  constexpr int kWs = SPLIT ? kRs : kQs;     // W row stride, elements
  constexpr int kPs2 = SPLIT ? kPs : kC + 8;  // P row stride, elements (bf16: 36 words, 8-byte reads conflict-free)
  __shared__ __attribute__((aligned(16))) uint16_t Ql[kC][kQs];
  __shared__ __attribute__((aligned(16))) uint16_t Kl[kC][kQs];
  __shared__ __attribute__((aligned(16))) LW Wl[kC][kWs];
  __shared__ __attribute__((aligned(16))) LW Pl[kC][kPs2];
  __shared__ float invq[kC], invk[kC];  // 1 / |q| / sqrt(D), 1 / |k| (eps 1e-6 inside the root)
  __shared__ float gl[kC], egl[kC], decl[kC];
  __shared__ float eglast;
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int r16 = lane & 15, qd = lane >> 4;
  const int b = blockIdx.x / a.H, h = blockIdx.x % a.H;

  // S: tile kb holds rows (keys) 16 kb + 4 qd + e, column (value) 16 wave + r16
  v4f S[8];
  const size_t sbase = (static_cast<size_t>(b) * a.H + h) * kD * kD;
#pragma unroll
  for (int kb = 0; kb < 8; ++kb) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      S[kb][e] = a.s_in ? a.s_in[sbase + static_cast<size_t>(16 * kb + 4 * qd + e) * kD + 16 * wave + r16] : 0.0f;
  }

  const Offsets of = offsets(a, b, h, t, wave, lane);
  ChunkIn<WU_F32, RP> in;
  load_chunk<WU_F32, RP>(a, of, 0, in);

  auto chunk = [&](const int n) __attribute__((always_inline)) {
    // ---- L: q, k, W into LDS; norms; g, e^g, e^{g_last - g} ------------------------------------
#pragma unroll
    for (int rp = 0; rp < RP; ++rp) {
      const int row = (t >> 3) + 32 * rp, seg = t & 7;
      *reinterpret_cast<uint4 *>(&Ql[row][16 * seg]) = in.q[rp][0];
      *reinterpret_cast<uint4 *>(&Ql[row][16 * seg + 8]) = in.q[rp][1];
      *reinterpret_cast<uint4 *>(&Kl[row][16 * seg]) = in.k[rp][0];
      *reinterpret_cast<uint4 *>(&Kl[row][16 * seg + 8]) = in.k[rp][1];
      float f[16];
      unbf16x8(in.q[rp][0], f);
      unbf16x8(in.q[rp][1], f + 8);
      float ss = 0.0f;
#pragma unroll
      for (int x = 0; x < 16; ++x) ss = fmaf(f[x], f[x], ss);
      ss = sum8(ss);
      if (seg == 0) invq[row] = (1.0f / sqrtf(ss + 1e-6f)) * (1.0f / 11.313708498984761f);  // then 1/sqrt(128)
      unbf16x8(in.k[rp][0], f);
      unbf16x8(in.k[rp][1], f + 8);
      ss = 0.0f;
#pragma unroll
      for (int x = 0; x < 16; ++x) ss = fmaf(f[x], f[x], ss);
      ss = sum8(ss);
      if (seg == 0) invk[row] = 1.0f / sqrtf(ss + 1e-6f);
      if constexpr (SPLIT) {
        if constexpr (WU_F32) {
#pragma unroll
          for (int x = 0; x < 4; ++x)
            *reinterpret_cast<uint4 *>(&Wl[row][16 * seg + 4 * x]) =
                make_uint4(hilo<SPLIT>(__uint_as_float(in.w[rp][x].x)), hilo<SPLIT>(__uint_as_float(in.w[rp][x].y)),
                           hilo<SPLIT>(__uint_as_float(in.w[rp][x].z)), hilo<SPLIT>(__uint_as_float(in.w[rp][x].w)));
        } else {  // bf16 W is exact: the hi part only
#pragma unroll
          for (int x = 0; x < 2; ++x) {
            const uint32_t w4[4] = {in.w[rp][x].x, in.w[rp][x].y, in.w[rp][x].z, in.w[rp][x].w};
            *reinterpret_cast<uint4 *>(&Wl[row][16 * seg + 8 * x]) =
                make_uint4(w4[0] & 0xFFFFu, w4[0] >> 16, w4[1] & 0xFFFFu, w4[1] >> 16);
            *reinterpret_cast<uint4 *>(&Wl[row][16 * seg + 8 * x + 4]) =
                make_uint4(w4[2] & 0xFFFFu, w4[2] >> 16, w4[3] & 0xFFFFu, w4[3] >> 16);
          }
        }
      } else {  // bf16 LDS: W rounded to bf16 (a float32 W) or as given
        if constexpr (WU_F32) {
#pragma unroll
          for (int x = 0; x < 2; ++x) {
            const uint4 lo = in.w[rp][2 * x], hi = in.w[rp][2 * x + 1];
            *reinterpret_cast<uint4 *>(&Wl[row][16 * seg + 8 * x]) =
                make_uint4(pack_bf16(__uint_as_float(lo.x), __uint_as_float(lo.y)), pack_bf16(__uint_as_float(lo.z), __uint_as_float(lo.w)),
                           pack_bf16(__uint_as_float(hi.x), __uint_as_float(hi.y)), pack_bf16(__uint_as_float(hi.z), __uint_as_float(hi.w)));
          }
        } else {
          *reinterpret_cast<uint4 *>(&Wl[row][16 * seg]) = in.w[rp][0];
          *reinterpret_cast<uint4 *>(&Wl[row][16 * seg + 8]) = in.w[rp][1];
        }
      }
    }
    {
      if (wave == 0) {
        const float g = scan64(in.gc);
        const float glast = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(g), 63));
        gl[lane] = g;
        egl[lane] = expf(g);
        decl[lane] = expf(glast - g);
        if (lane == 0) eglast = expf(glast);
      }
    }
    float u[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int e = 0; e < 4; ++e) u[i][e] = in.u[i][e];
    }
    lds_barrier();
    // Unconditional (the last chunk reloads itself, unused): behind a branch the compiler would
    // lose count of the loads in flight and make the next chunk wait for every memory operation,
    // this chunk's o stores included, instead of just these loads.
    load_chunk<WU_F32, RP>(a, of, min(n + 1, a.nchunks - 1), in);

    // ---- M: W S, q^ S, v_new; P tiles ----------------------------------------------------------
    Half4 sB[8];
#pragma unroll
    for (int kb = 0; kb < 8; ++kb) sB[kb] = split4<SPLIT>(S[kb]);
    v4f ws[4], qs[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ws[i] = qs[i] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int p = 0; p < 4; ++p) {  // key blocks 2p, 2p + 1: 8 independent accumulations
      const int c = 32 * p + 4 * qd;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const LW *wrow = Wl[16 * i + r16];
        const uint16_t *qrow = Ql[16 * i + r16];
        Half4 w0, w1;
        if constexpr (SPLIT) {
          w0 = unpack4(*reinterpret_cast<const uint4 *>(wrow + c));
          w1 = unpack4(*reinterpret_cast<const uint4 *>(wrow + c + 16));
        } else {
          w0 = bf16x4(wrow + c);
          w1 = bf16x4(wrow + c + 16);
        }
        ws[i] = WU_F32 ? mma<SPLIT>(w0, w1, sB[2 * p], sB[2 * p + 1], ws[i])
                       : mma_exact_a<SPLIT>(w0, w1, sB[2 * p], sB[2 * p + 1], ws[i]);
        qs[i] = mma_exact_a<SPLIT>(bf16x4(qrow + c), bf16x4(qrow + c + 16), sB[2 * p], sB[2 * p + 1], qs[i]);
      }
    }
    v4f vnew[4], oacc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 16 * i + 4 * qd + e;
        vnew[i][e] = u[i][e] - ws[i][e];
        oacc[i][e] = qs[i][e] * (invq[row] * egl[row]);
      }
    }
    for (int idx = wave; idx < 10; idx += kThreads / 64) {  // wave-uniform
      int ti, tj;
      p_tile(idx, ti, tj);
      v4f acc = {0.f, 0.f, 0.f, 0.f};
      const uint16_t *qrow = Ql[16 * ti + r16];
      const uint16_t *krow = Kl[16 * tj + r16];
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const int c = 32 * p + 4 * qd;
        acc = mma<false>(bf16x4(qrow + c), bf16x4(qrow + c + 16), bf16x4(krow + c), bf16x4(krow + c + 16), acc);
      }
      const int col = 16 * tj + r16;
      const float kf = invk[col];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 16 * ti + 4 * qd + e;
        const float pv = col <= row ? acc[e] * (invq[row] * kf) * expf(gl[row] - gl[col]) : 0.0f;
        Pl[row][col] = static_cast<LW>(hilo<SPLIT>(pv));
      }
    }
    lds_barrier();

    // ---- O: o = e^g q^ S + P v_new (causal pairs of token tiles) -------------------------------
    Half4 vB[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) vB[j] = split4<SPLIT>(vnew[j]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v4f acc = oacc[i];
      const LW *prow = Pl[16 * i + r16];
#pragma unroll
      for (int p = 0; p <= i / 2; ++p) {
        const bool two = 2 * p + 1 <= i;
        const int c = 32 * p + 4 * qd;
        Half4 p0, p1 = kZero4;
        if constexpr (SPLIT) {
          p0 = unpack4(*reinterpret_cast<const uint4 *>(prow + c));
          if (two) p1 = unpack4(*reinterpret_cast<const uint4 *>(prow + c + 16));
        } else {
          p0 = bf16x4(prow + c);
          if (two) p1 = bf16x4(prow + c + 16);
        }
        acc = mma<SPLIT>(p0, p1, vB[2 * p], two ? vB[2 * p + 1] : kZero4, acc);
      }
      if constexpr (OUT_F32) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          static_cast<float *>(a.o)[of.tile + static_cast<uint32_t>(n * kC + 16 * i + e) * of.tok] = acc[e];
      } else {
        // the quad's 4 rows x 4 adjacent columns, transposed with DPP quad broadcasts so that lane
        // q of the quad stores row 4 qd + q, the quad's 4 columns, in one 8-byte store
        const int qq = r16 & 3;
        const uint32_t P0 = pack_bf16(acc[0], acc[1]), P1 = pack_bf16(acc[2], acc[3]);
        const uint32_t a0 = __builtin_amdgcn_mov_dpp(P0, 0x00, 0xF, 0xF, false);
        const uint32_t a1 = __builtin_amdgcn_mov_dpp(P0, 0x55, 0xF, 0xF, false);
        const uint32_t a2 = __builtin_amdgcn_mov_dpp(P0, 0xAA, 0xF, 0xF, false);
        const uint32_t a3 = __builtin_amdgcn_mov_dpp(P0, 0xFF, 0xF, 0xF, false);
        const uint32_t b0 = __builtin_amdgcn_mov_dpp(P1, 0x00, 0xF, 0xF, false);
        const uint32_t b1 = __builtin_amdgcn_mov_dpp(P1, 0x55, 0xF, 0xF, false);
        const uint32_t b2 = __builtin_amdgcn_mov_dpp(P1, 0xAA, 0xF, 0xF, false);
        const uint32_t b3 = __builtin_amdgcn_mov_dpp(P1, 0xFF, 0xF, 0xF, false);
        const uint32_t sel = (qq & 1) ? 0x07060302u : 0x05040100u;
        const uint2 w = qq < 2 ? make_uint2(__builtin_amdgcn_perm(a1, a0, sel), __builtin_amdgcn_perm(a3, a2, sel))
                               : make_uint2(__builtin_amdgcn_perm(b1, b0, sel), __builtin_amdgcn_perm(b3, b2, sel));
        const uint32_t oi = of.tile - static_cast<uint32_t>(qq) + static_cast<uint32_t>(n * kC + 16 * i + qq) * of.tok;
        *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(a.o) + oi) = w;
      }
    }

    // ---- S: S = e^{g_last} S + k^T ((e^{g_last - g} / |k|) v_new) -------------------------------
    Half4 dB[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v4f d;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = 16 * j + 4 * qd + e;
        d[e] = vnew[j][e] * (decl[row] * invk[row]);
      }
      dB[j] = split4<SPLIT>(d);
    }
    const float el = eglast;
#pragma unroll
    for (int kb = 0; kb < 8; ++kb) {
#pragma unroll
      for (int e = 0; e < 4; ++e) S[kb][e] *= el;
    }
    // k^T operand (key 16 kb + r16, tokens c .. c + 3 and c + 16 .. c + 19) read from the
    // row-major k tile by transposing reads: lane 4 e + a of each 16-lane group addresses token
    // c + e, keys 16 kb + 4 a .. + 3
    const int te = r16 >> 2, ka = r16 & 3;
#pragma unroll
    for (int p = 0; p < 2; ++p) {  // token blocks 2p, 2p + 1: 8 independent accumulations
      const int c = 32 * p + 4 * qd;
#pragma unroll
      for (int kb = 0; kb < 8; ++kb) {
        S[kb] = mma_exact_a<SPLIT>(bf16x4_tr(&Kl[c + te][16 * kb + 4 * ka]), bf16x4_tr(&Kl[c + 16 + te][16 * kb + 4 * ka]),
                                   dB[2 * p], dB[2 * p + 1], S[kb]);
      }
    }
    lds_barrier();  // the next chunk overwrites q, k, W, P and the decays
  };
  // Chunk 0 runs on its own: then every path into the loop has the same memory operations in
  // flight (the next chunk's loads, then this chunk's o stores), and the compiler's wait before
  // the first use of the loads counts only them.
  chunk(0);
  for (int n = 1; n < a.nchunks; ++n) chunk(n);

#pragma unroll
  for (int kb = 0; kb < 8; ++kb) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      a.s_out[sbase + static_cast<size_t>(16 * kb + 4 * qd + e) * kD + 16 * wave + r16] = S[kb][e];
  }
}

template <bool SPLIT, bool WU_F32, bool OUT_F32>
qh_status launch3(const StateArgs &a, hipStream_t stream) {
  hipLaunchKernelGGL((gdn_state_kernel<SPLIT, WU_F32, OUT_F32>), dim3(a.B * a.H), dim3(kThreads), 0, stream, a);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return hip_fail(err, "gdn_state_kernel launch");
  return QH_STATUS_OK;
}

template <bool SPLIT>
qh_status launch2(const StateArgs &a, bool wu_f32, bool out_f32, hipStream_t stream) {
  if (wu_f32) return out_f32 ? launch3<SPLIT, true, true>(a, stream) : launch3<SPLIT, true, false>(a, stream);
  return out_f32 ? launch3<SPLIT, false, true>(a, stream) : launch3<SPLIT, false, false>(a, stream);
}

}  // namespace

qh_status launch_gdn_chunk_state(const uint16_t *q, const uint16_t *k, const float *g, const void *w, const void *u,
                                 const float *s_in, float *s_out, void *o, int B, int T, int H, int precision,
                                 bool wu_f32, bool out_f32, hipStream_t stream) {
  StateArgs a{q, k, g, w, u, s_in, s_out, o, B, T, H, T / kC};
  return precision == QH_GDN_BF16 ? launch2<false>(a, wu_f32, out_f32, stream)
                                  : launch2<true>(a, wu_f32, out_f32, stream);
}

}  // namespace qh
