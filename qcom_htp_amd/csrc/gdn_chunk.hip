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
// Two workgroups per (batch, chunk, head): one solves the U columns, one the W columns; each
// builds A itself (the A-build is a sixth of the work, and the split halves the LDS and
// register footprint).  Inside a workgroup:
//   1. K^ (bf16) into LDS, row-swizzled; g cumsum and beta into LDS;
//   2. the lower 16 x 16 blocks of K^ K^T with v_mfma_f32_16x16x32_bf16 (blocks spread over the
//      4 waves), scaled to A: strictly-lower blocks stored bf16, diagonal blocks fp32;
//   3. T_II for all diagonal blocks by forward substitution (one lane per column), in place;
//   4. the U workgroup replaces K^ in LDS by V; then each wave solves 32 of the 128 columns:
//      A_IJ X_J with v_mfma_f32_16x16x16_bf16 (X_J kept in registers in the layout that MFMA
//      reads as its B operand, which is the layout the MFMA result comes out in), T_II times
//      the sum with v_mfma_f32_16x16x4_f32, results stored to HBM as they are produced.
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

__device__ __forceinline__ size_t tok_index(const ChunkArgs &a, int b, int tok, int h) {
  return (static_cast<size_t>(b) * a.T + tok) * a.H + h;
}

// The role of a workgroup is fixed: items blockIdx.x + k * gridDim.x with gridDim.x a multiple
// of 16 all have bit 3 of the item index equal to bit 3 of blockIdx.x.
// Workgroup size: 8 waves (two per SIMD) for C >= 128, 4 waves for C = 64.
template <int NB>
constexpr int chunk_threads() { return NB >= 8 ? 512 : 256; }

template <int NB, int ROLE>
__device__ __forceinline__ void chunk_items(const ChunkArgs &a, const int nitems, uint8_t *smat, uint16_t *ablk,
                                            float *adiag, float *gs, float *bs, float *wsum) {
  constexpr int C = NB * 16;
  constexpr int kChunkThreads = chunk_threads<NB>();
  constexpr int kWaves = kChunkThreads / 64;
  constexpr int kTiles = 8 / kWaves;  // 16-column tiles of the 128 right-hand sides per wave
  constexpr int kRowPasses = C / (kChunkThreads / 8);   // K rows: 8 lanes per row
  constexpr int kVPasses = C / (kChunkThreads / 16);    // V rows: 16 lanes per row
  static_assert(kRowPasses >= 1 && kVPasses >= 1, "chunk too small for the workgroup");

  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int q = lane >> 4, l16 = lane & 15;

  // Work item -> (batch, chunk, head).  The two roles of one (batch, chunk, head) differ by 8
  // in the item index, so workgroups w and w + 8 of the persistent grid (one XCD) run them
  // together and share the key rows in L2.
  struct Item {
    int b, c, h;
    bool valid;
  };
  auto item_of = [&](int it) __attribute__((always_inline)) {
    Item r;
    const int ch_idx = ((it >> 4) << 3) | (it & 7);
    r.h = ch_idx % a.H;
    const int rest = ch_idx / a.H;
    r.c = rest % a.nchunks;
    r.b = rest / a.nchunks;
    r.valid = it < nitems && r.b < a.B;
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
      gs[t] = gv + pre;
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

    // The U role reads its values into registers now; the next item's keys are prefetched;
    // both sets of loads run under the diagonal inverses.
    uint4 vr[ROLE == 0 ? kVPasses : 1];
    if (ROLE == 0) {
#pragma unroll
      for (int p = 0; p < kVPasses; ++p) {
        const int row = p * (kChunkThreads / 16) + (t >> 4), part = t & 15;
        vr[p] = *reinterpret_cast<const uint4 *>(a.v + tok_index(a, b, tok0 + row, h) * kD + part * 8);
      }
    }
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
    if (ROLE == 0) {
#pragma unroll
      for (int p = 0; p < kVPasses; ++p) {
        const int row = p * (kChunkThreads / 16) + (t >> 4), part = t & 15;
        *reinterpret_cast<uint4 *>(smat + kofs(row, part * 8)) = vr[p];
      }
    }
    __syncthreads();

    // ---- 4. X_I = T_II (R_I + sum_{J<I} A_IJ X_J), 16 * kTiles columns per wave ------------
    const bool decay = ROLE == 1 && a.decay_w;
    v4s xb[NB][kTiles];  // X_J in bf16, the MFMA B-operand layout (= result layout)
    float *const wf = static_cast<float *>(ROLE ? a.w : a.u);
    uint16_t *const wh = static_cast<uint16_t *>(ROLE ? a.w : a.u);
#pragma unroll
    for (int I = 0; I < NB; ++I) {
      v4f acc[kTiles][4];  // four independent accumulation chains per tile (J mod 4)
#pragma unroll
      for (int tl = 0; tl < kTiles; ++tl) {
        const int d = (wave * kTiles + tl) * 16 + l16;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int i = I * 16 + 4 * q + s;
          float r = bs[i] * bf16_to_f32(*reinterpret_cast<const uint16_t *>(smat + kofs(i, d)));
          if (decay) r *= __expf(gs[i]);
          acc[tl][0][s] = r;
          acc[tl][1][s] = 0.0f;
          acc[tl][2][s] = 0.0f;
          acc[tl][3][s] = 0.0f;
        }
      }
#pragma unroll
      for (int J = 0; J < I; ++J) {
        const uint2 ap = *reinterpret_cast<const uint2 *>(ablk + (I * (I - 1) / 2 + J) * 256 + l16 * 16 + 4 * q);
#pragma unroll
        for (int tl = 0; tl < kTiles; ++tl)
          acc[tl][J & 3] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(v4s, ap), xb[J][tl], acc[tl][J & 3], 0, 0, 0);
      }
      const float4 tr = *reinterpret_cast<const float4 *>(adiag + I * 256 + l16 * 16 + 4 * q);
      const float trv[4] = {tr.x, tr.y, tr.z, tr.w};
#pragma unroll
      for (int tl = 0; tl < kTiles; ++tl) {
        const v4f sum = (acc[tl][0] + acc[tl][1]) + (acc[tl][2] + acc[tl][3]);
        v4f x = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 4; ++s) x = __builtin_amdgcn_mfma_f32_16x16x4f32(trv[s], sum[s], x, 0, 0, 0);
        const uint32_t p0 = f32_to_bf16(x[0]) | (f32_to_bf16(x[1]) << 16);
        const uint32_t p1 = f32_to_bf16(x[2]) | (f32_to_bf16(x[3]) << 16);
        xb[I][tl] = __builtin_bit_cast(v4s, make_uint2(p0, p1));
        const int d = (wave * kTiles + tl) * 16 + l16;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const size_t o = tok_index(a, b, tok0 + I * 16 + 4 * q + s, h) * kD + d;
          if (a.out_f32)
            wf[o] = x[s];
          else
            wh[o] = static_cast<uint16_t>(s < 2 ? (s == 0 ? p0 & 0xFFFFu : p0 >> 16) : (s == 2 ? p1 & 0xFFFFu : p1 >> 16));
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
  __shared__ __attribute__((aligned(16))) uint8_t smat[C * 256];             // K^, then V (U role)
  __shared__ __attribute__((aligned(16))) uint16_t ablk[(kLowBlocks > 0 ? kLowBlocks : 1) * 256];  // A_IJ, I > J
  __shared__ __attribute__((aligned(16))) float adiag[NB * 256];             // A_II, then T_II
  __shared__ float gs[C], bs[C], wsum[8];
  if ((blockIdx.x >> 3) & 1)
    chunk_items<NB, 1>(a, nitems, smat, ablk, adiag, gs, bs, wsum);
  else
    chunk_items<NB, 0>(a, nitems, smat, ablk, adiag, gs, bs, wsum);
}

template <int NB>
qh_status launch_nb(const ChunkArgs &a, hipStream_t stream) {
  const long long pairs = static_cast<long long>(a.B) * a.nchunks * a.H;
  const long long items = (pairs + 7) / 8 * 16;  // groups of 8 (batch, chunk, head) x 2 roles
  if (items > 0x7FFFFFFFLL) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_gdn_chunk_uw: too many chunks");
  // Persistent grid: as many workgroups as fit on the device at once, a multiple of 16.
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
  long long grid = slots[NB] / 16 * 16;
  if (grid < 16) grid = 16;
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
