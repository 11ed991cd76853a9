// The GdnSolve op's own scalar model on the GPU, code for code
// (example/gdn_native/solve_op/src/gdn_solve_core.h:28-83 as GdnSolveOp.cpp:201-208 drives it):
//   A_int16 = code - zpA (scale sA);  C % 16 == 0, C <= 64;  internal scale sTi = 2/32767:
//   1. each 16 x 16 diagonal block by forward substitution on int16 codes: the int32 sum
//      sum_k A_ik T_kj (two's complement, as the op's int32 accumulator), then
//      T_ij = clip(lroundf(e_ij / sTi + (float) acc * sA), +-32767), and Tf = T_ij * sTi;
//   2. block merges for j = 0 .., i = j+1 ..: acc = sum_{k=j}^{i-1} (sum_m ((float) A * sA) * Tf),
//      Tf_ij = sum_m Tf_ii[r][m] acc[m][c], every float32 operation rounded on its own in the
//      op's order;
//   3. T_code = clip(lroundf(Tf / sT), +-32767) + zpT, zpT above the diagonal.
// The products and sums are kept as separate roundings (fp contract off for this file: the op's
// host build fuses nothing), so the codes equal the op's bit for bit.  One workgroup of 256 threads per
// head; the work is small (C <= 64) and the order of operations, not throughput, is the contract.
// lroundf: round half away from zero; values beyond +-32767 clip (the op's lroundf is undefined
// beyond the long range, which valid inputs never reach).

#pragma clang fp contract(off)

#include "qmm_internal.h"

namespace qh {
namespace {

constexpr int kOpThreads = 256;
constexpr int kOpMaxC = 64;

struct OpArgs {
  const uint16_t *A;
  uint16_t *T;
  int C, heads, zpA, zpT;
  float sA, sT;
};

__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// lroundf, then clip to +-32767 (as a float).
__device__ __forceinline__ float round_clip(float v) {
  float r = truncf(v);
  if (fabsf(v - r) >= 0.5f) r = r + copysignf(1.0f, v);
  return fminf(fmaxf(r, -32767.0f), 32767.0f);
}

__global__ __launch_bounds__(kOpThreads) void gdn_op_model_kernel(OpArgs g) {
  __shared__ int16_t As[kOpMaxC][kOpMaxC + 2];
  __shared__ float Tf[kOpMaxC][kOpMaxC + 1];
  __shared__ float accb[16][17];
  const int t = threadIdx.x, C = g.C, nb = C / 16;
  const size_t base = static_cast<size_t>(blockIdx.x) * C * C;
  const float sA = g.sA;
  const float sTi = 2.0f / 32767.0f;
  const float inv_sTi = 1.0f / sTi;
  const float inv_sT = 1.0f / g.sT;

  for (int e = t; e < C * C; e += kOpThreads) {
    const int r = e / C, c = e - r * C;
    As[r][c] = static_cast<int16_t>(static_cast<int32_t>(g.A[base + e]) - g.zpA);
  }
  lds_barrier();

  // 1. diagonal blocks: thread (block b, column j) walks the rows
  if (t < nb * 16) {
    const int b = t >> 4, j = t & 15, o = 16 * b;
    int32_t col[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      uint32_t acc = 0;  // int32 with wrap-around
#pragma unroll
      for (int k = 0; k < i; ++k)
        acc += static_cast<uint32_t>(static_cast<int32_t>(As[o + i][o + k]) * col[k]);
      const float ei = (j == i) ? inv_sTi : 0.0f;
      const float v = ei + static_cast<float>(static_cast<int32_t>(acc)) * sA;
      col[i] = static_cast<int32_t>(round_clip(v));
      Tf[o + i][o + j] = static_cast<float>(col[i]) * sTi;
    }
  }
  lds_barrier();

  // 2. block merges in the op's order
  const int r = t >> 4, c = t & 15;
  for (int j = 0; j < nb; ++j) {
    for (int i = j + 1; i < nb; ++i) {
      float acc = 0.0f;
      for (int k = j; k < i; ++k) {
        float s = 0.0f;
#pragma unroll
        for (int m = 0; m < 16; ++m)
          s = s + static_cast<float>(As[16 * i + r][16 * k + m]) * sA * Tf[16 * k + m][16 * j + c];
        acc = acc + s;
      }
      accb[r][c] = acc;
      lds_barrier();
      float s = 0.0f;
#pragma unroll
      for (int m = 0; m < 16; ++m) s = s + Tf[16 * i + r][16 * i + m] * accb[m][c];
      Tf[16 * i + r][16 * j + c] = s;
      lds_barrier();
    }
  }

  // 3. output codes
  for (int e = t; e < C * C; e += kOpThreads) {
    const int rr = e / C, cc = e - rr * C;
    const int q = cc > rr ? 0 : static_cast<int>(round_clip(Tf[rr][cc] * inv_sT));
    g.T[base + e] = static_cast<uint16_t>(q + g.zpT);
  }
}

}  // namespace

qh_status launch_gdn_solve_op_model(const uint16_t *A, uint16_t *T, int heads, int C, int zpA, int zpT, float sA,
                                    float sT, hipStream_t stream) {
  if (C > kOpMaxC) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "gdn op model: C=%d (the op supports C <= 64)", C);
  OpArgs g{A, T, C, heads, zpA, zpT, sA, sT};
  hipLaunchKernelGGL(gdn_op_model_kernel, dim3(heads), dim3(kOpThreads), 0, stream, g);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return hip_fail(err, "gdn_op_model_kernel launch");
  return QH_STATUS_OK;
}

}  // namespace qh
