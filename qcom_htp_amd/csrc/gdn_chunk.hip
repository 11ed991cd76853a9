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

#include "qmm_internal.h"

namespace qh {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

constexpr int kD = 128;  // head dimension

struct ChunkArgs {
  const uint16_t *k, *v;  // bf16 [B][T][H][D]
  const float *g, *beta;  // [B][T][H]
  void *w, *u;            // [B][T][H][D] bf16 or fp32
  int B, T, H, C, nchunks;
  int decay_w, out_f32;
};

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// float -> bf16 bits, round to nearest even (inputs are finite)
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

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

template <int NB>
__device__ __forceinline__ void chunk_items(const ChunkArgs &a, const int nitems, uint8_t *smat, uint16_t *ablk,
                                            float *adiag, float *gs, float *bs, float *rn, float *wsc, float *wsum) {
  constexpr int C = NB * 16;
  constexpr int kChunkThreads = chunk_threads<NB>();
  constexpr int kWaves = kChunkThreads / 64;
  constexpr int kTiles = 16 / kWaves;  // 16-column tiles of the 256 right-hand sides per wave
  constexpr int kChains = kTiles >= 4 ? 1 : 4 / kTiles;
  constexpr int kRowPasses = C / (kChunkThreads / 8);   // K rows: 8 lanes per row
  static_assert(kRowPasses >= 1, "chunk too small for the workgroup");

  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int q = lane >> 4, l16 = lane & 15;

  // Work item -> (batch, chunk, head).
  struct Item {
    int b, c, h;
    bool valid;
  };
  auto item_of = [&](int it) __attribute__((always_inline)) {
    Item r;
    r.h = it % a.H;
    const int rest = it / a.H;
    r.c = rest % a.nchunks;
    r.b = rest / a.nchunks;
    r.valid = it < nitems;
    return r;
  };
  // Key rows, g and beta of an item into registers (all loads in flight together).
  uint4 kr[kRowPasses][2];
  float gpre = 0.0f, bpre = 0.0f;
  auto prefetch = [&](const Item &it) __attribute__((always_inline)) {
    if (!it.valid) return;
#pragma unroll
    for (int p = 0; p < kRowPasses; ++p) {
      const int row = p * (kChunkThreads / 8) + (t >> 3), part = t & 7;
      const uint4 *src = reinterpret_cast<const uint4 *>(a.k + tok_index(a, it.b, it.c * C + row, it.h) * kD + part * 16);
      kr[p][0] = src[0];
      kr[p][1] = src[1];
    }
    if (t < C) {
      const size_t ix = tok_index(a, it.b, it.c * C + t, it.h);
      gpre = a.g[ix];
      bpre = a.beta[ix];
    }
  };

  int it = blockIdx.x;
  Item cur = item_of(it);
  prefetch(cur);
  while (cur.valid) {
    const int b = cur.b, h = cur.h, tok0 = cur.c * C;
    // ---- 1. g cumsum, beta, K^ -------------------------------------------------------------
    float gv = t < C ? gpre : 0.0f;
    if (t < C) bs[t] = bpre;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float y = __shfl_up(gv, off, 64);
      if (lane >= off) gv += y;
    }
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
      ss += __shfl_xor(ss, 1, 64);
      ss += __shfl_xor(ss, 2, 64);
      ss += __shfl_xor(ss, 4, 64);
      const float inv = 1.0f / sqrtf(ss + 1e-6f);
      if (part == 0) rn[row] = inv;
      uint32_t o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = f32_to_bf16(f[2 * i] * inv) | (f32_to_bf16(f[2 * i + 1] * inv) << 16);
      *reinterpret_cast<uint4 *>(smat + kofs(row, part * 16)) = make_uint4(o[0], o[1], o[2], o[3]);
      *reinterpret_cast<uint4 *>(smat + kofs(row, part * 16 + 8)) = make_uint4(o[4], o[5], o[6], o[7]);
    }
    __syncthreads();
    if (t < C) {
      float pre = 0.0f;
      for (int w = 0; w < (t >> 6); ++w) pre += wsum[w];
      const float gt = gv + pre;
      gs[t] = gt;
      // scale of row t of W's right-hand side: beta / |k| [e^g]
      wsc[t] = bpre * rn[t] * (a.decay_w ? __expf(gt) : 1.0f);
    }
    __syncthreads();

    // ---- 2. A = -beta_i (K^ K^T)_ij e^{g_i - g_j}, lower blocks -----------------------------
    // Wave w takes the block rows w and NB-1-w (NB+1 blocks, balanced).  For block (I, J) the
    // MFMA computes D = K^_J K^_I^T = G_IJ^T, so each lane holds row l16 of G_IJ, columns
    // 4q .. 4q+3; the fragments of K^_I are read once per row, two J chains run together.
    auto a_store = [&](int I, int J, const v4f &acc) __attribute__((always_inline)) {
      const int i = I * 16 + l16;
      const float bi = bs[i], gi = gs[i];
      float av[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int j = J * 16 + 4 * q + s;
        av[s] = i > j ? -bi * acc[s] * __expf(gi - gs[j]) : 0.0f;
      }
      if (I > J) {
        const uint32_t p0 = f32_to_bf16(av[0]) | (f32_to_bf16(av[1]) << 16);
        const uint32_t p1 = f32_to_bf16(av[2]) | (f32_to_bf16(av[3]) << 16);
        *reinterpret_cast<uint2 *>(ablk + (I * (I - 1) / 2 + J) * 256 + l16 * 16 + 4 * q) = make_uint2(p0, p1);
      } else {
        *reinterpret_cast<float4 *>(adiag + I * 256 + l16 * 16 + 4 * q) = make_float4(av[0], av[1], av[2], av[3]);
      }
    };
    auto frag = [&](int row_blk, int kk) __attribute__((always_inline)) {
      const int r = row_blk * 16 + l16, ch = kk * 4 + q;
      return __builtin_bit_cast(v8bf, *reinterpret_cast<const uint4 *>(smat + r * 256 + 16 * (ch ^ (r & 15))));
    };
    if (wave < (NB + 1) / 2) {
#pragma unroll
      for (int side = 0; side < 2; ++side) {
        const int I = side == 0 ? wave : NB - 1 - wave;
        if (side == 1 && I == wave) break;  // NB odd: the middle row once
        v8bf bi[kD / 32];
#pragma unroll
        for (int kk = 0; kk < kD / 32; ++kk) bi[kk] = frag(I, kk);
        for (int J = 0; J <= I; J += 2) {
          const bool two = J + 1 <= I;
          v4f acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int kk = 0; kk < kD / 32; ++kk) {
            acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(frag(J, kk), bi[kk], acc0, 0, 0, 0);
            if (two) acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(frag(J + 1, kk), bi[kk], acc1, 0, 0, 0);
          }
          a_store(I, J, acc0);
          if (two) a_store(I, J + 1, acc1);
        }
      }
    }
    __syncthreads();

    // The first block row of right-hand sides and the next item's keys load under the diagonal
    // inverses.  Tile tg of the 256 right-hand-side columns: tg < 8 are W's (keys), the rest
    // U's (values); lane column d = (tg % 8) * 16 + l16, rows 4q .. 4q + 3 of the block row.
    // The columns of a wave all belong to W or all to U.  Element offsets fit in 32 bits
    // (B * T * H * 128 <= 2^31 is checked at the boundary).
    const bool is_w = wave * kTiles < 8;
    const gptr<const uint16_t> rsrc = pick_ptr<const uint16_t>(is_w, a.k, a.v);
    const uint32_t tstride = static_cast<uint32_t>(a.H) * kD;  // elements per token
    const uint32_t lbase =
        (static_cast<uint32_t>(b * a.T + tok0 + 4 * q) * static_cast<uint32_t>(a.H) + h) * kD + l16;
    uint32_t rraw[2][kTiles][4];
    auto rhs_load = [&](int I, uint32_t (&r)[kTiles][4]) __attribute__((always_inline)) {
#pragma unroll
      for (int tl = 0; tl < kTiles; ++tl) {
        const uint32_t dcol = ((wave * kTiles + tl) & 7) * 16;
#pragma unroll
        for (int s = 0; s < 4; ++s) r[tl][s] = rsrc[lbase + dcol + (I * 16 + s) * tstride];
      }
    };
    rhs_load(0, rraw[0]);
    it += gridDim.x;
    const Item nxt = item_of(it);
    prefetch(nxt);

    // ---- 3. T_II = (I - A_II)^-1, one lane per column, in place ----------------------------
    if (t < NB * 16) {
      const int I = t >> 4, col = t & 15;  // the 16 lanes of a block are in one wave
      const float *Ad = adiag + I * 256;
      float x[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float sacc = r == col ? 1.0f : 0.0f;
#pragma unroll
        for (int kx = 0; kx < r; ++kx) sacc = fmaf(Ad[r * 16 + kx], x[kx], sacc);
        x[r] = sacc;
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) adiag[I * 256 + r * 16 + col] = x[r];
    }
    __syncthreads();

    // ---- 4. X_I = T_II (R_I + sum_{J<I} A_IJ X_J), 16 * kTiles columns per wave ------------
    const float *const rsc = is_w ? wsc : bs;
    const gptr<float> of = pick_ptr<float>(is_w, a.w, a.u);
    const gptr<uint16_t> oh = pick_ptr<uint16_t>(is_w, a.w, a.u);
    v4s xb[NB][kTiles];  // X_J in bf16, the MFMA B-operand layout (= result layout)
#pragma unroll
    for (int I = 0; I < NB; ++I) {
      if (I + 1 < NB) rhs_load(I + 1, rraw[(I + 1) & 1]);
      v4f acc[kTiles][kChains];  // kTiles * kChains = 4 independent accumulation chains
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const float sc = rsc[I * 16 + 4 * q + s];
#pragma unroll
        for (int tl = 0; tl < kTiles; ++tl) {
          acc[tl][0][s] = sc * bf16_to_f32(rraw[I & 1][tl][s]);
#pragma unroll
          for (int c = 1; c < kChains; ++c) acc[tl][c][s] = 0.0f;
        }
      }
#pragma unroll
      for (int J = 0; J < I; ++J) {
        const uint2 ap = *reinterpret_cast<const uint2 *>(ablk + (I * (I - 1) / 2 + J) * 256 + l16 * 16 + 4 * q);
#pragma unroll
        for (int tl = 0; tl < kTiles; ++tl)
          acc[tl][J % kChains] =
              __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(v4s, ap), xb[J][tl], acc[tl][J % kChains], 0, 0, 0);
      }
      const float4 tr = *reinterpret_cast<const float4 *>(adiag + I * 256 + l16 * 16 + 4 * q);
      const float trv[4] = {tr.x, tr.y, tr.z, tr.w};
#pragma unroll
      for (int tl = 0; tl < kTiles; ++tl) {
        v4f sum = acc[tl][0];
#pragma unroll
        for (int c = 1; c < kChains; ++c) sum += acc[tl][c];
        v4f x = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 4; ++s) x = __builtin_amdgcn_mfma_f32_16x16x4f32(trv[s], sum[s], x, 0, 0, 0);
        const uint32_t p0 = f32_to_bf16(x[0]) | (f32_to_bf16(x[1]) << 16);
        const uint32_t p1 = f32_to_bf16(x[2]) | (f32_to_bf16(x[3]) << 16);
        xb[I][tl] = __builtin_bit_cast(v4s, make_uint2(p0, p1));
        const uint32_t dcol = ((wave * kTiles + tl) & 7) * 16;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const uint32_t o = lbase + dcol + (I * 16 + s) * tstride;
          if (a.out_f32)
            of[o] = x[s];
          else
            oh[o] = static_cast<uint16_t>(s < 2 ? (s == 0 ? p0 & 0xFFFFu : p0 >> 16) : (s == 2 ? p1 & 0xFFFFu : p1 >> 16));
        }
      }
    }
    __syncthreads();  // LDS is rewritten by the next item
    cur = nxt;
  }
}

template <int NB>
__global__ __launch_bounds__(chunk_threads<NB>(), 1) void gdn_chunk_kernel(const ChunkArgs a, const int nitems) {
  constexpr int C = NB * 16;
  constexpr int kLowBlocks = NB * (NB - 1) / 2;
  __shared__ __attribute__((aligned(16))) uint8_t smat[C * 256];             // K^
  __shared__ __attribute__((aligned(16))) uint16_t ablk[(kLowBlocks > 0 ? kLowBlocks : 1) * 256];  // A_IJ, I > J
  __shared__ __attribute__((aligned(16))) float adiag[NB * 256];             // A_II, then T_II
  __shared__ float gs[C], bs[C], rn[C], wsc[C], wsum[8];
  chunk_items<NB>(a, nitems, smat, ablk, adiag, gs, bs, rn, wsc, wsum);
}

template <int NB>
qh_status launch_nb(const ChunkArgs &a, hipStream_t stream) {
  const long long items = static_cast<long long>(a.B) * a.nchunks * a.H;  // (batch, chunk, head)
  if (items > 0x7FFFFFFFLL) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_gdn_chunk_uw: too many chunks");
  if (items == 0) return QH_STATUS_OK;
  // Persistent grid: as many workgroups as fit on the device at once.
  static int slots[17] = {0};
  int dev = 0;
  (void)hipGetDevice(&dev);
  if (slots[NB] == 0) {
    int per_cu = 0, cus = 0;
    hipError_t err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gdn_chunk_kernel<NB>, chunk_threads<NB>(), 0);
    if (err != hipSuccess) return hip_fail(err, "hipOccupancyMaxActiveBlocksPerMultiprocessor");
    err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (err != hipSuccess) return hip_fail(err, "hipDeviceGetAttribute");
    slots[NB] = (per_cu < 1 ? 1 : per_cu) * cus;
  }
  long long grid = slots[NB];
  if (grid > items) grid = items;
  hipLaunchKernelGGL(gdn_chunk_kernel<NB>, dim3(static_cast<unsigned>(grid)), dim3(chunk_threads<NB>()), 0, stream, a,
                     static_cast<int>(items));
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return hip_fail(err, "gdn_chunk_kernel launch");
  return QH_STATUS_OK;
}

}  // namespace

qh_status launch_gdn_chunk_uw(const uint16_t *k, const uint16_t *v, const float *g, const float *beta, void *w,
                              void *u, int B, int T, int H, int C, int flags, hipStream_t stream) {
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
      return launch_nb<4>(a, stream);
    case 128:
      return launch_nb<8>(a, stream);
    case 256:
      return launch_nb<16>(a, stream);
    default:
      return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_gdn_chunk_uw: chunk %d (need 64, 128 or 256)", C);
  }
}

}  // namespace qh
