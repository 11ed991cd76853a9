// GDN / KDA per-head triangular solve T = (I - A)^-1, A strictly lower triangular, C <= 256.
//
// Parallel decomposition: the 16-column panels of T are independent (column J of T only
// depends on A's rows and columns >= J), so one workgroup solves one (head, panel J) pair:
//   1. the 16x16 diagonal blocks T_II = (I - A_II)^-1 for I >= J, by forward substitution with
//      one lane per column (16 lanes per block, 16 blocks per round across the 4 waves);
//   2. X_J = T_JJ, then for I = J+1 .. C/16-1 (block forward substitution)
//         G   = sum_{K=J}^{I-1} A_IK X_K      (MFMA; wave w takes the blocks K - J = w, w+4, ...)
//         X_I = T_II G                         (MFMA, by the wave that owns block I - J)
//      -- the block merge T_ij = T_ii * sum_{k=j}^{i-1} A_ik T_kj of the reference core
//      (example/gdn_native/solve_op/src/gdn_solve_core.h:55-75), evaluated column-panel-wise.
// The chain of dependent block steps is the critical path, so a step has one barrier: the A
// operands come straight from global memory into registers (two row blocks ahead), each wave
// keeps the X blocks it owns in LDS in the MFMA lane layout (written and read by that wave
// only), only the partial sums of G cross waves (double-buffered by step parity), and T is
// written out after the chain.
// Precision: QH_GDN_FP32 uses v_mfma_f32_16x16x4_f32; QH_GDN_BF16 feeds the G products through
// v_mfma_f32_16x16x32_bf16 (fp32 accumulation) and keeps the diagonal solves and T_II G in fp32.
// The u16 variant applies the GdnSolve op's code contract on load / store
// (A = (code - zpA) * sA; T_code = clip(rint(T / sT) + zpT, 0, 65535)).

#include "qmm_internal.h"

namespace qh {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

constexpr int kGdnThreads = 256;

// Workgroup barrier for data exchanged through LDS: waits for this wave's LDS operations only.
// __syncthreads() would also wait for the row-block prefetches in flight (its release fence).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
constexpr int kMaxNb = 16;  // C <= 256

struct GdnArgs {
  const void *A;
  void *T;
  int C, nb;
  int zpA, zpT;
  float sA, sT, inv_sT;
};

template <bool U16>
__device__ __forceinline__ void store_t(const GdnArgs &g, size_t idx, float v) {
  if (U16) {
    float q = rintf(v * g.inv_sT) + static_cast<float>(g.zpT);
    q = fminf(fmaxf(q, 0.0f), 65535.0f);
    static_cast<uint16_t *>(g.T)[idx] = static_cast<uint16_t>(q);
  } else {
    static_cast<float *>(g.T)[idx] = v;
  }
}

// Loads 4 consecutive A values (row r, columns c..c+3, c % 4 == 0) of the head's matrix.
template <bool U16>
__device__ __forceinline__ float4 load_a4(const GdnArgs &g, size_t idx) {
  if (U16) {
    const uint2 v = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(g.A) + idx);
    float4 f;
    f.x = static_cast<float>(static_cast<int>(v.x & 0xFFFFu) - g.zpA) * g.sA;
    f.y = static_cast<float>(static_cast<int>(v.x >> 16) - g.zpA) * g.sA;
    f.z = static_cast<float>(static_cast<int>(v.y & 0xFFFFu) - g.zpA) * g.sA;
    f.w = static_cast<float>(static_cast<int>(v.y >> 16) - g.zpA) * g.sA;
    return f;
  }
  return *reinterpret_cast<const float4 *>(static_cast<const float *>(g.A) + idx);
}

template <bool U16, bool BF16>
__global__ __launch_bounds__(kGdnThreads) void gdn_panel_kernel(GdnArgs g) {
  // LDS: diagonal inverses of blocks J..nb-1 (rows padded to 20 floats so a lane reads 4
  // adjacent columns with one 16-byte load), one staged A row block for the diagonal solves,
  // the solved panel blocks in the MFMA lane layout, and double-buffered per-wave partial sums.
  __shared__ __attribute__((aligned(16))) float tdiag[kMaxNb][16][20];
  __shared__ float abuf[16][kMaxNb * 16 + 4];
  __shared__ float4 xs[kMaxNb][64];
  __shared__ float4 gpart[2][4][64];

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int J = blockIdx.x, head = blockIdx.y;
  const int C = g.C, nb = g.nb;
  const size_t hbase = static_cast<size_t>(head) * C * C;
  const int c0 = J * 16;
  // MFMA lane roles: r = row of the A operand / column of B and of the result, kq = k quarter.
  // The k index of product step s is 4 kq + s, so a lane's result rows 4 kq .. 4 kq + 3 (one
  // float4) are exactly its B operand for the next product.
  const int r = lane & 15, kq = lane >> 4;
  // Panel blocks are handed to the waves in units of UB blocks (one 16x16x4 f32 MFMA per k step,
  // or two blocks per 16x16x32 bf16 MFMA): wave w owns units w, w + 4, ...
  constexpr int UB = BF16 ? 2 : 1;

  // A values of row block I that this wave multiplies: for each of its units i (kb0 = UB (wave
  // + 4 i)), row 16 I + r, columns 16 (J + kb) + 4 kq .. + 3 of the unit's UB blocks.
  float4 pre0[4][UB], pre1[4][UB];
  auto prefetch = [&](int I, float4 (&pre)[4][UB]) {
    const int n = I - J;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int h = 0; h < UB; ++h) {
        const int kb = UB * (wave + 4 * i) + h;
        if (kb < n)
          pre[i][h] = load_a4<U16>(g, hbase + static_cast<size_t>(I * 16 + r) * C + (J + kb) * 16 + 4 * kq);
        else
          pre[i][h] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
  };
  // ---- diagonal inverses T_II, I = J .. nb-1 ----------------------------------------------
  for (int base = J; base < nb; base += 16) {
    // stage the 16x16 diagonal blocks of this round: every load is issued before the first LDS
    // write (a load-then-store loop would wait for each load in turn)
    float4 dv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int e = t + u * kGdnThreads;  // float4 slot: block e / 64, row (e / 4) % 16, quarter e % 4
      const int b = e >> 6, i = (e >> 2) & 15, k4 = e & 3;
      const int I = base + b;
      if (I < nb) dv[u] = load_a4<U16>(g, hbase + static_cast<size_t>(I * 16 + i) * C + I * 16 + 4 * k4);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int e = t + u * kGdnThreads;
      const int b = e >> 6, i = (e >> 2) & 15, k4 = e & 3;
      if (base + b < nb) {
        float *dst = &abuf[i][b * 16 + 4 * k4];
        dst[0] = dv[u].x;
        dst[1] = dv[u].y;
        dst[2] = dv[u].z;
        dst[3] = dv[u].w;
      }
    }
    if (base == J) {  // the first two row blocks of the chain load under the diagonal solves
      if (J + 1 < nb) prefetch(J + 1, pre0);
      if (J + 2 < nb) prefetch(J + 2, pre1);
    }
    lds_barrier();
    const int b = wave * 4 + (lane >> 4), j = lane & 15;
    const int I = base + b;
    if (I < nb) {
      float x[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float sacc = (i == j) ? 1.0f : 0.0f;
#pragma unroll
        for (int k = 0; k < i; ++k) sacc = fmaf(abuf[i][b * 16 + k], x[k], sacc);
        x[i] = sacc;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) tdiag[I - J][i][j] = x[i];
    }
    lds_barrier();
  }

  // ---- X_J = T_JJ (kept by wave 0, the owner of block 0, in the lane layout) -----------------
  if (wave == 0)
    xs[0][lane] = make_float4(tdiag[0][4 * kq][r], tdiag[0][4 * kq + 1][r], tdiag[0][4 * kq + 2][r],
                              tdiag[0][4 * kq + 3][r]);

  // ---- block forward substitution down the panel -------------------------------------------
  //   G_I = sum_{K=J}^{I-1} A_IK X_K   (each wave over its own blocks, A from registers, X_K from
  //                                     the wave's own LDS blocks)
  //   X_I = T_II G_I                   (only the wave that owns block I - J, after one barrier)
  // Each block X_K is written and later read by the same wave, so one barrier per row block
  // (for the partial sums) is the only synchronisation of the chain.
  auto step = [&](const int I, float4 (&pre)[4][UB]) __attribute__((always_inline)) {
    const int n = I - J;
    v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int kb0 = UB * (wave + 4 * i);
      if (kb0 >= n) break;
      if (!BF16) {
        const float4 a = pre[i][0], x = xs[kb0][lane];
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, x.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, x.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, x.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, x.w, acc, 0, 0, 0);
      } else {
        // k = 8 kq + jj: jj < 4 from block kb0, jj >= 4 from block kb0 + 1 (zero past the panel)
        const float4 x0 = xs[kb0][lane];
        const float4 x1 = kb0 + 1 < n ? xs[kb0 + 1][lane] : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 a0 = pre[i][0], a1 = pre[i][UB - 1];
        v8bf av, bv;
        av[0] = static_cast<__bf16>(a0.x); av[1] = static_cast<__bf16>(a0.y);
        av[2] = static_cast<__bf16>(a0.z); av[3] = static_cast<__bf16>(a0.w);
        av[4] = static_cast<__bf16>(a1.x); av[5] = static_cast<__bf16>(a1.y);
        av[6] = static_cast<__bf16>(a1.z); av[7] = static_cast<__bf16>(a1.w);
        bv[0] = static_cast<__bf16>(x0.x); bv[1] = static_cast<__bf16>(x0.y);
        bv[2] = static_cast<__bf16>(x0.z); bv[3] = static_cast<__bf16>(x0.w);
        bv[4] = static_cast<__bf16>(x1.x); bv[5] = static_cast<__bf16>(x1.y);
        bv[6] = static_cast<__bf16>(x1.z); bv[7] = static_cast<__bf16>(x1.w);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc, 0, 0, 0);
      }
    }
    if (I + 2 < nb) prefetch(I + 2, pre);  // this slot's registers take row block I + 2
    gpart[I & 1][wave][lane] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    lds_barrier();
    if (wave == (n / UB) % 4) {
      // G_I rows 4 kq .. 4 kq + 3 of column r, summed over the waves, as the B operand
      const float4 p0 = gpart[I & 1][0][lane], p1 = gpart[I & 1][1][lane], p2 = gpart[I & 1][2][lane],
                   p3 = gpart[I & 1][3][lane];
      const float4 tr = *reinterpret_cast<const float4 *>(&tdiag[n][r][4 * kq]);
      v4f x = {0.f, 0.f, 0.f, 0.f};
      x = __builtin_amdgcn_mfma_f32_16x16x4f32(tr.x, (p0.x + p1.x) + (p2.x + p3.x), x, 0, 0, 0);
      x = __builtin_amdgcn_mfma_f32_16x16x4f32(tr.y, (p0.y + p1.y) + (p2.y + p3.y), x, 0, 0, 0);
      x = __builtin_amdgcn_mfma_f32_16x16x4f32(tr.z, (p0.z + p1.z) + (p2.z + p3.z), x, 0, 0, 0);
      x = __builtin_amdgcn_mfma_f32_16x16x4f32(tr.w, (p0.w + p1.w) + (p2.w + p3.w), x, 0, 0, 0);
      xs[n][lane] = make_float4(x[0], x[1], x[2], x[3]);
    }
  };
  for (int I = J + 1; I < nb; I += 2) {
    step(I, pre0);
    if (I + 1 < nb) step(I + 1, pre1);
  }

  // ---- write the panel: every global store comes after the chain ---------------------------
  // (stores count in the same in-order counter as the loads, so a store issued inside the chain
  // would make the wait for the next row block's A operands wait for it too)
  for (int kb = 0; kb < nb - J; ++kb) {
    if ((kb / UB) % 4 != wave) continue;  // each wave writes the blocks it owns
    const float4 x = xs[kb][lane];
    const size_t row0 = static_cast<size_t>((J + kb) * 16 + 4 * kq) * C + c0 + r;
    store_t<U16>(g, hbase + row0, x.x);
    store_t<U16>(g, hbase + row0 + C, x.y);
    store_t<U16>(g, hbase + row0 + 2 * static_cast<size_t>(C), x.z);
    store_t<U16>(g, hbase + row0 + 3 * static_cast<size_t>(C), x.w);
  }
  for (int e = t; e < c0 * 16; e += kGdnThreads) {  // zeros above the diagonal block
    const int rr = e >> 4, c = e & 15;
    store_t<U16>(g, hbase + static_cast<size_t>(rr) * C + c0 + c, 0.0f);
  }
}

template <bool U16, bool BF16>
qh_status launch(const GdnArgs &g, int heads, hipStream_t stream) {
  dim3 grid(g.nb, heads);
  hipLaunchKernelGGL((gdn_panel_kernel<U16, BF16>), grid, dim3(kGdnThreads), 0, stream, g);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return hip_fail(err, "gdn_panel_kernel launch");
  return QH_STATUS_OK;
}

}  // namespace

qh_status launch_gdn_solve_f32(const float *A, float *T, int heads, int C, int precision, hipStream_t stream) {
  if (heads > 65535) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "gdn: heads=%d exceeds one launch (65535)", heads);
  GdnArgs g{A, T, C, C / 16, 0, 0, 1.0f, 1.0f, 1.0f};
  return precision == QH_GDN_BF16 ? launch<false, true>(g, heads, stream) : launch<false, false>(g, heads, stream);
}

qh_status launch_gdn_solve_u16(const uint16_t *A, uint16_t *T, int heads, int C, int zpA, int zpT, float sA, float sT,
                               int precision, hipStream_t stream) {
  if (heads > 65535) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "gdn: heads=%d exceeds one launch (65535)", heads);
  GdnArgs g{A, T, C, C / 16, zpA, zpT, sA, sT, 1.0f / sT};
  return precision == QH_GDN_BF16 ? launch<true, true>(g, heads, stream) : launch<true, false>(g, heads, stream);
}

}  // namespace qh
