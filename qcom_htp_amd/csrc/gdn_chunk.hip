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

constexpr int kChunkThreads = 256;
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

template <int NB>
__global__ __launch_bounds__(kChunkThreads, 1) void gdn_chunk_kernel(const ChunkArgs a) {
  constexpr int C = NB * 16;
  constexpr int kLowBlocks = NB * (NB - 1) / 2;
  __shared__ __attribute__((aligned(16))) uint8_t smat[C * 256];             // K^, then V (U role)
  __shared__ __attribute__((aligned(16))) uint16_t ablk[(kLowBlocks > 0 ? kLowBlocks : 1) * 256];  // A_IJ, I > J
  __shared__ __attribute__((aligned(16))) float adiag[NB * 256];             // A_II, then T_II
  __shared__ float gs[C], bs[C], wsum[4];

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  // blockIdx: the two roles of one (batch, chunk, head) differ by 8, so they land on one XCD
  const int bid = blockIdx.x;
  const int role = (bid >> 3) & 1;  // 0: U, 1: W
  const int ch_idx = ((bid >> 4) << 3) | (bid & 7);
  const int h = ch_idx % a.H;
  const int rest = ch_idx / a.H;
  const int c = rest % a.nchunks, b = rest / a.nchunks;
  if (b >= a.B) return;  // padding of the last group of 8
  const int tok0 = c * C;

  // ---- 1. g cumsum, beta, K^ ---------------------------------------------------------------
  float gv = 0.0f;
  if (t < C) {
    const size_t ix = tok_index(a, b, tok0 + t, h);
    gv = a.g[ix];
    bs[t] = a.beta[ix];
  }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float y = __shfl_up(gv, off, 64);
    if (lane >= off) gv += y;
  }
  if (lane == 63) wsum[wave] = gv;
  // K rows: 8 lanes per row, 16 elements per lane
  for (int r0 = 0; r0 < C; r0 += kChunkThreads / 8) {
    const int row = r0 + (t >> 3), part = t & 7;
    const uint4 *src = reinterpret_cast<const uint4 *>(a.k + tok_index(a, b, tok0 + row, h) * kD + part * 16);
    const uint4 x0 = src[0], x1 = src[1];
    const uint32_t w[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
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
    for (int w = 0; w < wave; ++w) pre += wsum[w];
    gs[t] = gv + pre;
  }
  __syncthreads();

  // ---- 2. A = -beta_i (K^ K^T)_ij e^{g_i - g_j}, lower blocks -------------------------------
  const int q = lane >> 4, l16 = lane & 15;
  for (int e = wave; e < NB * (NB + 1) / 2; e += 4) {
    int I = 0;
    while ((I + 1) * (I + 2) / 2 <= e) ++I;
    const int J = e - I * (I + 1) / 2;
    // D = K^_J K^_I^T = G_IJ^T: lane holds G_IJ[l16][4q .. 4q+3]
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kk = 0; kk < kD / 32; ++kk) {
      const int ch = kk * 4 + q;
      const int rj = J * 16 + l16, ri = I * 16 + l16;
      const uint4 va = *reinterpret_cast<const uint4 *>(smat + rj * 256 + 16 * (ch ^ (rj & 15)));
      const uint4 vb = *reinterpret_cast<const uint4 *>(smat + ri * 256 + 16 * (ch ^ (ri & 15)));
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, va), __builtin_bit_cast(v8bf, vb), acc, 0, 0, 0);
    }
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
  }
  __syncthreads();

  // ---- 3. T_II = (I - A_II)^-1, one lane per column, in place ------------------------------
  if (t < NB * 16) {
    const int I = t >> 4, col = t & 15;  // the 16 lanes of a block are in one wave
    const float *Ad = adiag + I * 256;
    float x[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float s = r == col ? 1.0f : 0.0f;
#pragma unroll
      for (int kx = 0; kx < r; ++kx) s = fmaf(Ad[r * 16 + kx], x[kx], s);
      x[r] = s;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) adiag[I * 256 + r * 16 + col] = x[r];
  }
  if (role == 0) {
    __syncthreads();  // every wave is done with K^
    for (int r0 = 0; r0 < C; r0 += kChunkThreads / 16) {
      const int row = r0 + (t >> 4), part = t & 15;
      const uint4 x = *reinterpret_cast<const uint4 *>(a.v + tok_index(a, b, tok0 + row, h) * kD + part * 8);
      *reinterpret_cast<uint4 *>(smat + kofs(row, part * 8)) = x;
    }
  }
  __syncthreads();

  // ---- 4. X_I = T_II (R_I + sum_{J<I} A_IJ X_J), 32 columns per wave -------------------------
  const int d0 = wave * 32;
  const bool decay = role == 1 && a.decay_w;
  v4s xb[NB][2];  // X_J in bf16, the MFMA B-operand layout (= result layout)
  float *const wf = static_cast<float *>(role ? a.w : a.u);
  uint16_t *const wh = static_cast<uint16_t *>(role ? a.w : a.u);
#pragma unroll
  for (int I = 0; I < NB; ++I) {
    v4f acc[2];
#pragma unroll
    for (int tl = 0; tl < 2; ++tl) {
      const int d = d0 + tl * 16 + l16;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int i = I * 16 + 4 * q + s;
        float r = bs[i] * bf16_to_f32(*reinterpret_cast<const uint16_t *>(smat + kofs(i, d)));
        if (decay) r *= __expf(gs[i]);
        acc[tl][s] = r;
      }
    }
#pragma unroll
    for (int J = 0; J < I; ++J) {
      const uint2 ap = *reinterpret_cast<const uint2 *>(ablk + (I * (I - 1) / 2 + J) * 256 + l16 * 16 + 4 * q);
      const v4s av = __builtin_bit_cast(v4s, ap);
#pragma unroll
      for (int tl = 0; tl < 2; ++tl) acc[tl] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av, xb[J][tl], acc[tl], 0, 0, 0);
    }
    const float4 tr = *reinterpret_cast<const float4 *>(adiag + I * 256 + l16 * 16 + 4 * q);
    const float trv[4] = {tr.x, tr.y, tr.z, tr.w};
#pragma unroll
    for (int tl = 0; tl < 2; ++tl) {
      v4f x = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < 4; ++s) x = __builtin_amdgcn_mfma_f32_16x16x4f32(trv[s], acc[tl][s], x, 0, 0, 0);
      const uint32_t p0 = f32_to_bf16(x[0]) | (f32_to_bf16(x[1]) << 16);
      const uint32_t p1 = f32_to_bf16(x[2]) | (f32_to_bf16(x[3]) << 16);
      xb[I][tl] = __builtin_bit_cast(v4s, make_uint2(p0, p1));
      const int d = d0 + tl * 16 + l16;
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
}

template <int NB>
qh_status launch_nb(const ChunkArgs &a, hipStream_t stream) {
  const long long pairs = static_cast<long long>(a.B) * a.nchunks * a.H;
  const long long groups = (pairs + 7) / 8;
  if (groups * 16 > 0x7FFFFFFFLL) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_gdn_chunk_uw: too many chunks");
  hipLaunchKernelGGL(gdn_chunk_kernel<NB>, dim3(static_cast<unsigned>(groups * 16)), dim3(kChunkThreads), 0, stream, a);
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
