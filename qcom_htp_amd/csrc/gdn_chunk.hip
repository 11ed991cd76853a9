// Fused GDN chunk products: from the keys, values, per-token log decays and betas of one chunk
// of one head, build A, apply T = (I - A)^-1 and write
//     U = T (beta * V),    W = T (beta * K^)   [or T (beta * K^ * e^g)],
// the intra-chunk half of the gated delta rule (scripts/gdn_ref_kernel.py:71-89):
//     K^ = l2norm(K) (eps 1e-6), g = cumsum(gc) inside the chunk,
//     A_ij = -beta_i (K^_i . K^_j) e^{g_i - g_j} for i > j.
//
// Decomposition.  T is never formed.  U and W solve (I - A) X = R with the 256 right-hand-side
// columns R = [beta V | beta K^ (e^g)], by block forward substitution over 16-row blocks:
//     X_I = T_II (R_I + sum_{J<I} A_IJ X_J),   T_II = (I - A_II)^-1 (16 x 16).
// One workgroup per (batch, chunk, head), persistent over items:
//   1. K^ (bf16) into LDS, row-swizzled, with 1 / |k| per row; g cumsum and beta into LDS;
//   2. the lower 16 x 16 blocks of K^ K^T with v_mfma_f32_16x16x32_bf16 (blocks spread over the
//      waves), scaled to A: strictly-lower blocks stored bf16, diagonal blocks fp32;
//   3. T_II for all diagonal blocks by forward substitution (one lane per column), in place;
//   4. all 256 right-hand-side columns (W's 128, then U's 128) as 16-column tiles over the
//      waves: A_IJ X_J with v_mfma_f32_16x16x16_bf16 (X_J kept in registers in the layout that
//      MFMA reads as its B operand, which is the layout the MFMA result comes out in), T_II
//      times the sum with v_mfma_f32_16x16x4_f32, results stored to HBM as they are produced.
//      The right-hand-side rows come from global memory (the keys were just read, so from L2),
//      one block step ahead, scaled on the fly: beta / |k| [e^g] for W, beta for U.
// Precision: bf16 operands, fp32 accumulation; diagonal inverses and T_II products in fp32.

#include <atomic>

#include "lane_ops.h"
#include "qmm_internal.h"

namespace qh {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef unsigned v2u __attribute__((ext_vector_type(2)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

constexpr int kD = 128;  // head dimension
// Floats per diagonal 16 x 16 block in LDS: padded so that the four blocks a wave reads at once in
// the diagonal inverses fall in different banks.
constexpr int kDiagStride = 260;

struct ChunkArgs {
  const uint16_t *k, *v;  // bf16 [B][T][H][D]
  const float *g, *beta;  // [B][T][H]
  void *w, *u;            // [B][T][H][D] bf16 or fp32
  int B, T, H, C, nchunks;
  int decay_w, out_f32;
};

// Workgroup barrier for LDS traffic only (does not wait for outstanding global memory operations).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

// Two floats -> packed bf16 (a in the low half), round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v2f{a, b}, v2bf));
}

// Four floats as bf16 hi (round to nearest even) and lo = bf16(f - hi): the 8-element MFMA
// operand {hi0..hi3, lo0..lo3}; hi + lo carries about 16 significant bits.
__device__ __forceinline__ v8bf split_bf16x4(const float4 f) {
  const uint32_t h01 = pack_bf16(f.x, f.y), h23 = pack_bf16(f.z, f.w);
  const uint32_t l01 = pack_bf16(f.x - __uint_as_float(h01 << 16), f.y - __uint_as_float(h01 & 0xFFFF0000u));
  const uint32_t l23 = pack_bf16(f.z - __uint_as_float(h23 << 16), f.w - __uint_as_float(h23 & 0xFFFF0000u));
  return __builtin_bit_cast(v8bf, make_uint4(h01, h23, l01, l23));
}

// First pair of blocks of block row I in the pair layout: sum over I' < I of ceil(I' / 2).
__host__ __device__ constexpr int pair_base(int I) { return (I / 2) * (I / 2) + (I & 1) * (I / 2); }

// Byte offset of element (row, d) of a [C][128] bf16 matrix in LDS: each 256-byte row holds 16
// chunks of 8 elements, chunk c stored at position c ^ (row & 15) (16 consecutive rows reading
// the same chunk hit distinct banks).
__device__ __forceinline__ int kofs(int row, int d) { return row * 256 + 16 * ((d >> 3) ^ (row & 15)) + 2 * (d & 7); }

// c ? x : y for two kernel-argument pointers, kept in SGPRs, as a global-memory pointer.  Both
// are materialised first so that the choice does not become a dynamically indexed load of the
// argument block.
template <typename T>
using gptr = __attribute__((address_space(1))) T *;
template <typename T>
__device__ __forceinline__ gptr<T> pick_ptr(bool c, const void *x, const void *y) {
  uint64_t xi = reinterpret_cast<uint64_t>(x), yi = reinterpret_cast<uint64_t>(y);
  asm volatile("" : "+s"(xi));
  asm volatile("" : "+s"(yi));
  return (gptr<T>)(reinterpret_cast<T *>(c ? xi : yi));
}

__device__ __forceinline__ size_t tok_index(const ChunkArgs &a, int b, int tok, int h) {
  return (static_cast<size_t>(b) * a.T + tok) * a.H + h;
}

// Workgroup size: 8 waves (two per SIMD) for C >= 128, 4 waves for C = 64.
template <int NB>
constexpr int chunk_threads() { return NB >= 8 ? 512 : 256; }

template <int NB, bool OUT_F32>
__device__ __forceinline__ void chunk_items(const ChunkArgs &a, const int nitems, uint8_t *smat, uint16_t *ablk,
                                            float *adiag, float *gs, float *bs, float *rn, float *wsc, float *wsum) {
  constexpr int C = NB * 16;
  constexpr int kChunkThreads = chunk_threads<NB>();
  constexpr int kWaves = kChunkThreads / 64;
  constexpr int kTiles = 16 / kWaves;  // 16-column tiles of the 256 right-hand sides per wave
  constexpr int kChains = kTiles >= 4 ? 1 : 4 / kTiles;
  static_assert(pair_base(NB) * 1024 <= C * 256, "A' pairs must fit in smat");
  constexpr int kRowPasses = C / (kChunkThreads / 8);   // K rows: 8 lanes per row
  // Right-hand-side loads (memory latency under this load is several microseconds): block rows
  // [0, kEarly) are issued at the start of the item, under the A-build, the rest after it.
  constexpr int kEarly = NB < 8 ? NB : 8;
  // Substitution row at whose start the next item's keys are prefetched (0: before the
  // diagonal inverses), once enough right-hand-side registers have been freed.
  constexpr int kKeyRow = NB >= 16 ? 12 : 0;
  constexpr int kWords = kTiles / 2;  // 32-bit words per MFMA-layout row of a lane (16 kWords bytes row-major)
  // Per-wave staging of right-hand-side and result rows (16 rows): in smat after the A' pairs
  // when it fits, else in the A_IJ blocks (both free during the substitution).
  constexpr int kStageRow = kWords == 1 ? 80 : 144;
  constexpr bool kStageInSmat = pair_base(NB) * 1024 + kWaves * 16 * kStageRow <= C * 256;
  static_assert(kStageInSmat || kWaves * 16 * kStageRow <= NB * (NB - 1) / 2 * 512, "staging must fit");
  static_assert(kRowPasses >= 1, "chunk too small for the workgroup");
  static_assert(kTiles == 2 || kTiles == 4, "tile pairing");

  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int q = lane >> 4, l16 = lane & 15;

  // Work item -> (batch, chunk, head).
  struct Item {
    int b, c, h;
    bool valid;
  };
  // An index past the end yields the last item, marked invalid (its loads stay in bounds).
  auto item_of = [&](int it) __attribute__((always_inline)) {
    Item r;
    const int ic = it < nitems ? it : nitems - 1;
    r.h = ic % a.H;
    const int rest = ic / a.H;
    r.c = rest % a.nchunks;
    r.b = rest / a.nchunks;
    r.valid = it < nitems;
    return r;
  };
  // Key rows, g and beta of an item into registers (all loads in flight together).  Issued for
  // an invalid item too (the last item again): branch-free, so the compiler counts the
  // outstanding loads exactly.
  uint4 kr[kRowPasses][2];
  float gpre = 0.0f, bpre = 0.0f;
  auto prefetch = [&](const Item &it) __attribute__((always_inline)) {
#pragma unroll
    for (int p = 0; p < kRowPasses; ++p) {
      const int row = p * (kChunkThreads / 8) + (t >> 3), part = t & 7;
      const uint4 *src = reinterpret_cast<const uint4 *>(a.k + tok_index(a, it.b, it.c * C + row, it.h) * kD + part * 16);
      kr[p][0] = src[0];
      kr[p][1] = src[1];
    }
    {  // every lane loads (rows clamped), so that the count of outstanding loads is uniform
      const size_t ix = tok_index(a, it.b, it.c * C + (t < C ? t : C - 1), it.h);
      gpre = a.g[ix];
      bpre = a.beta[ix];
    }
  };

  // ---- 1. g cumsum, beta, K^ (from the prefetched registers) ---------------------------------
  auto phase1 = [&]() __attribute__((always_inline)) {
    float gv = t < C ? gpre : 0.0f;
    if (t < C) bs[t] = bpre;
    gv = scan64(gv);  // DPP: no LDS round trips
    if (lane == 63 && wave < 4) wsum[wave] = gv;
#pragma unroll
    for (int p = 0; p < kRowPasses; ++p) {
      const int row = p * (kChunkThreads / 8) + (t >> 3), part = t & 7;
      const uint32_t w[8] = {kr[p][0].x, kr[p][0].y, kr[p][0].z, kr[p][0].w,
                             kr[p][1].x, kr[p][1].y, kr[p][1].z, kr[p][1].w};
      float f[16];
      float ss = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        f[2 * i] = bf16_to_f32(w[i] & 0xFFFFu);
        f[2 * i + 1] = bf16_to_f32(w[i] >> 16);
        ss = fmaf(f[2 * i], f[2 * i], ss);
        ss = fmaf(f[2 * i + 1], f[2 * i + 1], ss);
      }
      ss = sum8(ss);
      const float inv = rsqrtf(ss + 1e-6f);
      if (part == 0) rn[row] = inv;
      uint32_t o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = pack_bf16(f[2 * i] * inv, f[2 * i + 1] * inv);
      *reinterpret_cast<uint4 *>(smat + kofs(row, part * 16)) = make_uint4(o[0], o[1], o[2], o[3]);
      *reinterpret_cast<uint4 *>(smat + kofs(row, part * 16 + 8)) = make_uint4(o[4], o[5], o[6], o[7]);
    }
    lds_barrier();
    if (t < C) {
      float pre = 0.0f;
      for (int w = 0; w < (t >> 6); ++w) pre += wsum[w];
      const float gt = gv + pre;
      gs[t] = gt;
      // scale of row t of W's right-hand side: beta / |k| [e^g]
      wsc[t] = bpre * rn[t] * (a.decay_w ? __expf(gt) : 1.0f);
    }
    lds_barrier();
  };

  // Phase 1 of the next item runs at the end of the current one, in straight-line code after the
  // substitution's loads and stores, so that waiting for the prefetched keys does not wait for
  // those (the outstanding-load count is in issue order).
  int it = blockIdx.x;
  Item cur = item_of(it);
  prefetch(cur);
  phase1();
  while (cur.valid) {
    const int b = cur.b, h = cur.h, tok0 = cur.c * C;
    // Right-hand sides.  A wave owns kTiles 16-column tiles, all of W (keys) or all of U
    // (values): the 16 * kTiles adjacent columns from cb = ((wave * kTiles) % 8) * 16, column
    // cb + kTiles * l16 + tl in tile tl; in the MFMA layout lane (q, l16) holds rows 4q .. 4q+3
    // of its kTiles columns.  Global memory is accessed row-major instead, 16 rows x 32 kTiles
    // bytes per block row and wave, 16 kWords bytes per lane (lane L: row L / 4, part L % 4),
    // and transposed through a per-wave LDS staging area (rows kStageRow bytes apart: the four
    // row groups of the MFMA layout fall in different banks).  Block rows [0, kEarly) load at
    // the start of the item, under the A-build, the others after it.  Byte offsets fit in 32 bits (B * T * H * 128 <= 2^31
    // elements is checked at the boundary) and are added to base pointers held in SGPRs.
    const bool is_w = wave * kTiles < 8;
    const gptr<const uint8_t> rsrc = pick_ptr<const uint8_t>(is_w, a.k, a.v);
    const uint32_t tstride = static_cast<uint32_t>(a.H) * kD;  // elements per token
    const uint32_t tsb = 2 * tstride;                          // bytes per token
    const int cb = ((wave * kTiles) & 7) * 16;
    const uint32_t rm_base =
        2 * ((static_cast<uint32_t>(b * a.T + tok0 + (lane >> 2)) * static_cast<uint32_t>(a.H) + h) * kD + cb) +
        (lane & 3) * 16 * kWords;
    uint8_t *const stg = (kStageInSmat ? smat + pair_base(NB) * 1024 : reinterpret_cast<uint8_t *>(ablk)) +
                         wave * 16 * kStageRow;
    uint8_t *const stg_rm = stg + (lane >> 2) * kStageRow + (lane & 3) * 16 * kWords;  // row-major slot
    uint8_t *const stg_mf = stg + 4 * q * kStageRow + 4 * kWords * l16;               // MFMA-layout slot
    // The running offset advances one block row at a time, opaque to the compiler, so that it
    // does not precompute (and keep live) the offsets of every row.
    uint32_t ld_off = rm_base;
    v4u rring[NB][kWords];
    auto rhs_load = [&](v4u (&r)[kWords]) __attribute__((always_inline)) {
#pragma unroll
      for (int w = 0; w < kWords; ++w) r[w] = *(gptr<const v4u>)(rsrc + (ld_off + 16 * w));
      ld_off += 16 * tsb;
      asm volatile("" : "+v"(ld_off));
    };
#pragma unroll
    for (int I = 0; I < kEarly; ++I) rhs_load(rring[I]);

    // ---- 2. A = -beta_i (K^ K^T)_ij e^{g_i - g_j}, lower blocks -----------------------------
    // Wave w < NB/2 takes the block rows I0 = w and I1 = NB-1-w (NB+1 blocks, balanced): the
    // key fragments of block row J (the MFMA B operand) are read once for both rows and
    // prefetched one J ahead.  For block (I, J) the MFMA computes D = K^_I K^_J^T = G_IJ, so each
    // lane holds rows 4q .. 4q+3 of column l16; blocks are stored column-major (element (r, c)
    // at c * 16 + r).
    auto a_store = [&](int I, int J, float gj, const float4 &b4, const float4 &g4, const v4f &acc)
                       __attribute__((always_inline)) {
      const float bi[4] = {b4.x, b4.y, b4.z, b4.w}, gi[4] = {g4.x, g4.y, g4.z, g4.w};
      float av[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bool low = I > J || 4 * q + s > l16;  // i > j
        av[s] = low ? -bi[s] * acc[s] * __expf(gi[s] - gj) : 0.0f;
      }
      if (I > J) {
        *reinterpret_cast<uint2 *>(ablk + (I * (I - 1) / 2 + J) * 256 + l16 * 16 + 4 * q) =
            make_uint2(pack_bf16(av[0], av[1]), pack_bf16(av[2], av[3]));
      } else {
        *reinterpret_cast<float4 *>(adiag + I * kDiagStride + l16 * 16 + 4 * q) = make_float4(av[0], av[1], av[2], av[3]);
      }
    };
    auto frag = [&](int row_blk, int kk) __attribute__((always_inline)) {
      const int r = row_blk * 16 + l16, ch = kk * 4 + q;
      return __builtin_bit_cast(v8bf, *reinterpret_cast<const uint4 *>(smat + r * 256 + 16 * (ch ^ (r & 15))));
    };
    if (wave < NB / 2) {
      const int I0 = wave, I1 = NB - 1 - wave;
      v8bf f0[kD / 32], f1[kD / 32], fa[kD / 32], fb[kD / 32];
#pragma unroll
      for (int kk = 0; kk < kD / 32; ++kk) {
        f0[kk] = frag(I0, kk);
        f1[kk] = frag(I1, kk);
        fa[kk] = frag(0, kk);
      }
      const float4 b0 = *reinterpret_cast<const float4 *>(bs + I0 * 16 + 4 * q);
      const float4 g0 = *reinterpret_cast<const float4 *>(gs + I0 * 16 + 4 * q);
      const float4 b1 = *reinterpret_cast<const float4 *>(bs + I1 * 16 + 4 * q);
      const float4 g1 = *reinterpret_cast<const float4 *>(gs + I1 * 16 + 4 * q);
      float gja = gs[l16], gjb = 0.0f;
      auto step = [&](int J, const v8bf (&cur)[kD / 32], float gjc, v8bf (&nxt)[kD / 32], float &gjn)
                      __attribute__((always_inline)) {
        const int Jn = J + 1 <= I1 ? J + 1 : I1;  // clamped: the loads stay branch-free
#pragma unroll
        for (int kk = 0; kk < kD / 32; ++kk) nxt[kk] = frag(Jn, kk);
        gjn = gs[Jn * 16 + l16];
        v4f acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kk = 0; kk < kD / 32; ++kk) acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f1[kk], cur[kk], acc1, 0, 0, 0);
        if (J <= I0) {
          v4f acc0 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int kk = 0; kk < kD / 32; ++kk) acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f0[kk], cur[kk], acc0, 0, 0, 0);
          a_store(I0, J, gjc, b0, g0, acc0);
        }
        a_store(I1, J, gjc, b1, g1, acc1);
      };
      for (int J = 0; J <= I1; J += 2) {
        step(J, fa, gja, fb, gjb);
        if (J + 1 <= I1) step(J + 1, fb, gjb, fa, gja);
      }
    }
    lds_barrier();

#pragma unroll
    for (int J = kEarly; J < NB; ++J) rhs_load(rring[J]);  // the A-build's registers are free now
    it += gridDim.x;
    const Item nxt = item_of(it);
    if (kKeyRow == 0) prefetch(nxt);

    // ---- 3. T_II = (I - A_II)^-1, one lane per column, in place ----------------------------
    if (t < NB * 16) {
      const int I = t >> 4, col = t & 15;  // the 16 lanes of a block are in one wave
      const float *Ad = adiag + I * kDiagStride;
      float x[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float sacc = r == col ? 1.0f : 0.0f;
#pragma unroll
        for (int kx = 0; kx < r; ++kx) sacc = fmaf(Ad[kx * 16 + r], x[kx], sacc);
        x[r] = sacc;
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) adiag[I * kDiagStride + r * 16 + col] = x[r];  // T_II row-major
    }
    lds_barrier();

    // ---- 3b. A'_IJ = T_II A_IJ (I > J) in bf16, into smat (free after the A-build) ----------
    // Computed transposed, D = A_IJ^T T_II^T, so that lane (q, l16) holds row l16 of A'_IJ,
    // columns 4q .. 4q+3: the A-operand fragment of the substitution.  T_II is split into
    // bf16 hi + lo along K (16 x 16 x 32 MFMA, K = the 16 inner indices twice).  Pair layout: the
    // blocks (I, 2p) and (I, 2p + 1) form pair pair_base(I) + p, 1 KiB, lane-major, 16 bytes per
    // lane (8 bytes per block); the second half of a row's last pair is zero when I is odd.
    // Wave w < NB/2 folds the block rows w and NB-1-w: NB-1 blocks, block n of the wave is
    // (w, n) for n < w, else (NB-1-w, n-w); all A loads are issued first.
    if (wave < NB / 2) {
      const int I0 = wave, I1 = NB - 1 - wave;
      const v8bf t0 = split_bf16x4(*reinterpret_cast<const float4 *>(adiag + I0 * kDiagStride + l16 * 16 + 4 * q));
      const v8bf t1 = split_bf16x4(*reinterpret_cast<const float4 *>(adiag + I1 * kDiagStride + l16 * 16 + 4 * q));
      uint2 ac[NB - 1];
      // block n of row I0 is ablk block I0(I0-1)/2 + n, of row I1 block I1(I1-1)/2 + n - I0
      const uint16_t *const ab0 = ablk + (I0 * (I0 - 1) / 2) * 256 + l16 * 16 + 4 * q;
      const uint16_t *const ab1 = ablk + (I1 * (I1 - 1) / 2 - I0) * 256 + l16 * 16 + 4 * q;
#pragma unroll
      for (int n = 0; n < NB - 1; ++n) ac[n] = *reinterpret_cast<const uint2 *>((n < I0 ? ab0 : ab1) + n * 256);
#pragma unroll
      for (int n = 0; n < NB - 1; ++n) {
        const int I = n < I0 ? I0 : I1, J = n < I0 ? n : n - I0;
        const v4f d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(v8bf, make_uint4(ac[n].x, ac[n].y, ac[n].x, ac[n].y)), n < I0 ? t0 : t1,
            v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
        uint8_t *const dst = smat + (pair_base(I) + (J >> 1)) * 1024 + lane * 16 + (J & 1) * 8;
        *reinterpret_cast<uint2 *>(dst) =
            make_uint2(pack_bf16(d[0], d[1]), pack_bf16(d[2], d[3]));
        if ((I & 1) && J == I - 1) *reinterpret_cast<uint2 *>(dst + 8) = make_uint2(0u, 0u);
      }
    }
    lds_barrier();

    // ---- 4. X_I = T'_I R_I + sum_{J<I} A'_IJ X_J,  T'_I = T_II diag(row scales) ------------
    // One 16 x 16 x 32 MFMA per tile for T'_I R_I (T' split hi + lo, R_I raw bf16 twice) and one
    // per pair of blocks J for the sum; only the last pair depends on X_{I-1}.
    const float *const rsc = bs + (is_w ? C : 0);  // wsc = bs + C: one LDS object
    const gptr<float> of = pick_ptr<float>(is_w, a.w, a.u);
    const gptr<uint8_t> oh = pick_ptr<uint8_t>(is_w, a.w, a.u);
    // fp32 outputs are stored from the MFMA layout (element offsets); bf16 through the staging
    uint32_t st_off = OUT_F32 ? (static_cast<uint32_t>(b * a.T + tok0 + 4 * q) * static_cast<uint32_t>(a.H) + h) * kD +
                                    cb + kTiles * l16
                              : rm_base;
    v4s xb[NB][kTiles];  // X_J in bf16, the MFMA B-operand layout (= result layout)
#pragma unroll
    for (int I = 0; I < NB; ++I) {
      if (kKeyRow > 0 && I == kKeyRow) prefetch(nxt);
      // this row's A' pairs, all reads issued before the T' operand is formed
      uint4 apr[(NB + 1) / 2];
#pragma unroll
      for (int pj = 0; pj < (I + 1) / 2; ++pj)
        apr[pj] = *reinterpret_cast<const uint4 *>(smat + (pair_base(I) + pj) * 1024 + lane * 16);
      // right-hand side rows of block row I into the MFMA layout
      uint32_t r[4][kWords];
#pragma unroll
      for (int w = 0; w < kWords; ++w)
        *reinterpret_cast<v4u *>(stg_rm + 16 * w) = rring[I][w];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        if constexpr (kWords == 1) {
          r[s][0] = *reinterpret_cast<const uint32_t *>(stg_mf + s * kStageRow);
        } else {
          const uint2 v = *reinterpret_cast<const uint2 *>(stg_mf + s * kStageRow);
          r[s][0] = v.x;
          r[s][1] = v.y;
        }
      }
      v4f acc[kTiles][kChains];
      {
        const float4 tr = *reinterpret_cast<const float4 *>(adiag + I * kDiagStride + l16 * 16 + 4 * q);
        const float4 sc = *reinterpret_cast<const float4 *>(rsc + I * 16 + 4 * q);
        const v8bf tp = split_bf16x4(make_float4(tr.x * sc.x, tr.y * sc.y, tr.z * sc.z, tr.w * sc.w));
#pragma unroll
        for (int tl = 0; tl < kTiles; ++tl) {
          const int w = tl >> 1;
          // rows 0..3 of tile tl: the low or high halves of the row words
          const uint32_t sel = tl & 1 ? 0x07060302u : 0x05040100u;
          const uint32_t r01 = __builtin_amdgcn_perm(r[1][w], r[0][w], sel);
          const uint32_t r23 = __builtin_amdgcn_perm(r[3][w], r[2][w], sel);
          acc[tl][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(tp, __builtin_bit_cast(v8bf, make_uint4(r01, r23, r01, r23)),
                                                               v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
          for (int c = 1; c < kChains; ++c) acc[tl][c] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
        }
      }
#pragma unroll
      for (int pj = 0; pj < (I + 1) / 2; ++pj) {
        const v8bf ap = __builtin_bit_cast(v8bf, apr[pj]);
#pragma unroll
        for (int tl = 0; tl < kTiles; ++tl) {
          const uint2 x0 = __builtin_bit_cast(uint2, xb[2 * pj][tl]);
          const uint2 x1 = 2 * pj + 1 < I ? __builtin_bit_cast(uint2, xb[2 * pj + 1][tl]) : make_uint2(0u, 0u);
          const int c = (pj + 1) % kChains;
          acc[tl][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ap, __builtin_bit_cast(v8bf, make_uint4(x0.x, x0.y, x1.x, x1.y)),
                                                               acc[tl][c], 0, 0, 0);
        }
      }
      v4f xt[kTiles];
#pragma unroll
      for (int tl = 0; tl < kTiles; ++tl) {
        v4f x = acc[tl][0];
#pragma unroll
        for (int c = 1; c < kChains; ++c) x += acc[tl][c];
        xt[tl] = x;
        xb[I][tl] = __builtin_bit_cast(v4s, make_uint2(pack_bf16(x[0], x[1]), pack_bf16(x[2], x[3])));
      }
      if constexpr (OUT_F32) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const uint32_t o = st_off + s * tstride;
          if constexpr (kTiles == 2)
            *(gptr<v2f>)(of + o) = v2f{xt[0][s], xt[1][s]};
          else
            *(gptr<v4f>)(of + o) = v4f{xt[0][s], xt[1][s], xt[2][s], xt[3][s]};
        }
        st_off += 16 * tstride;
      } else {
        // X rows into the staging (MFMA layout), read back row-major, one wide store per lane
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          uint32_t wv[kWords];
#pragma unroll
          for (int j = 0; j < kWords; ++j) {
            const v2u lo = __builtin_bit_cast(v2u, xb[I][2 * j]), hi = __builtin_bit_cast(v2u, xb[I][2 * j + 1]);
            wv[j] = __builtin_amdgcn_perm(s < 2 ? hi[0] : hi[1], s < 2 ? lo[0] : lo[1], s & 1 ? 0x07060302u : 0x05040100u);
          }
          if constexpr (kWords == 1)
            *reinterpret_cast<uint32_t *>(stg_mf + s * kStageRow) = wv[0];
          else
            *reinterpret_cast<uint2 *>(stg_mf + s * kStageRow) = make_uint2(wv[0], wv[1]);
        }
#pragma unroll
        for (int w = 0; w < kWords; ++w)
          *(gptr<v4u>)(oh + (st_off + 16 * w)) = *reinterpret_cast<const v4u *>(stg_rm + 16 * w);
        st_off += 16 * tsb;
      }
      asm volatile("" : "+v"(st_off));
    }
    lds_barrier();  // every wave is done with this item's LDS contents
    phase1();       // next item (an invalid one ends the loop; its phase 1 is harmless)
    cur = nxt;
  }
}

template <int NB, bool OUT_F32>
__global__ __launch_bounds__(chunk_threads<NB>(), 1) void gdn_chunk_kernel(const ChunkArgs a, const int nitems) {
  constexpr int C = NB * 16;
  constexpr int kLowBlocks = NB * (NB - 1) / 2;
  __shared__ __attribute__((aligned(16))) uint8_t smat[C * 256];             // K^
  __shared__ __attribute__((aligned(16))) uint16_t ablk[(kLowBlocks > 0 ? kLowBlocks : 1) * 256];  // A_IJ, I > J
  __shared__ __attribute__((aligned(16))) float adiag[NB * kDiagStride];     // A_II, then T_II
  __shared__ float gs[C], bsw[2 * C], rn[C], wsum[8];  // bsw: beta, then W's row scales
  chunk_items<NB, OUT_F32>(a, nitems, smat, ablk, adiag, gs, bsw, rn, bsw + C, wsum);
}

template <int NB, bool OUT_F32>
qh_status launch_nb(const ChunkArgs &a, int max_wg, hipStream_t stream) {
  const long long items = static_cast<long long>(a.B) * a.nchunks * a.H;  // (batch, chunk, head)
  if (items > 0x7FFFFFFFLL) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_gdn_chunk_uw: too many chunks");
  if (items == 0) return QH_STATUS_OK;
  // Persistent grid: as many workgroups as fit on the device at once (per device, cached).
  constexpr int kMaxDevices = 64;
  static std::atomic<int> slots[kMaxDevices];
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return hip_fail(err, "hipGetDevice");
  int grid_slots = dev >= 0 && dev < kMaxDevices ? slots[dev].load(std::memory_order_relaxed) : 0;
  if (grid_slots == 0) {
    int per_cu = 0, cus = 0;
    err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gdn_chunk_kernel<NB, OUT_F32>, chunk_threads<NB>(), 0);
    if (err != hipSuccess) return hip_fail(err, "hipOccupancyMaxActiveBlocksPerMultiprocessor");
    err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (err != hipSuccess) return hip_fail(err, "hipDeviceGetAttribute");
    grid_slots = (per_cu < 1 ? 1 : per_cu) * cus;
    if (dev >= 0 && dev < kMaxDevices) slots[dev].store(grid_slots, std::memory_order_relaxed);
  }
  if (max_wg > 0 && max_wg < grid_slots) grid_slots = max_wg;  // caller's cap on the persistent grid
  const long long grid = grid_slots < items ? grid_slots : items;
  hipLaunchKernelGGL((gdn_chunk_kernel<NB, OUT_F32>), dim3(static_cast<unsigned>(grid)), dim3(chunk_threads<NB>()), 0,
                     stream, a, static_cast<int>(items));
  err = hipGetLastError();
  if (err != hipSuccess) return hip_fail(err, "gdn_chunk_kernel launch");
  return QH_STATUS_OK;
}

template <int NB>
qh_status launch_nb(const ChunkArgs &a, int max_wg, hipStream_t stream) {
  return a.out_f32 ? launch_nb<NB, true>(a, max_wg, stream) : launch_nb<NB, false>(a, max_wg, stream);
}

}  // namespace

qh_status launch_gdn_chunk_uw(const uint16_t *k, const uint16_t *v, const float *g, const float *beta, void *w,
                              void *u, int B, int T, int H, int C, int flags, int max_wg, hipStream_t stream) {
  ChunkArgs a{};
  a.k = k;
  a.v = v;
  a.g = g;
  a.beta = beta;
  a.w = w;
  a.u = u;
  a.B = B;
  a.T = T;
  a.H = H;
  a.C = C;
  a.nchunks = T / C;
  a.decay_w = (flags & QH_GDN_W_DECAY) != 0;
  a.out_f32 = (flags & QH_GDN_OUT_F32) != 0;
  switch (C) {
    case 64:
      return launch_nb<4>(a, max_wg, stream);
    case 128:
      return launch_nb<8>(a, max_wg, stream);
    case 256:
      return launch_nb<16>(a, max_wg, stream);
    default:
      return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_gdn_chunk_uw: chunk %d (need 64, 128 or 256)", C);
  }
}

}  // namespace qh
