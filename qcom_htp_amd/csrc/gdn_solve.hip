// GDN / KDA per-head triangular solve T = (I - A)^-1, A strictly lower triangular, C <= 256.
//
// Parallel decomposition: the 16-column panels of T are independent (column J of T only
// depends on A's rows and columns >= J), so one workgroup solves one (head, panel J) pair:
//   1. the 16x16 diagonal blocks T_II = (I - A_II)^-1 for I >= J, by forward substitution with
//      one lane per column (16 lanes per block, 16 blocks per round across the 4 waves);
//   2. X_J = T_JJ, then for I = J+1 .. C/16-1 (block forward substitution)
//         G   = sum_{K=J}^{I-1} A_IK X_K      (MFMA, the K range split across the 4 waves)
//         X_I = T_II G                         (MFMA)
//      -- the block merge T_ij = T_ii * sum_{k=j}^{i-1} A_ik T_kj of the reference core
//      (example/gdn_native/solve_op/src/gdn_solve_core.h:55-75), evaluated column-panel-wise.
// The next two row blocks of A are prefetched into registers while the current block is
// multiplied, and the barriers wait for LDS traffic only, so the chain of dependent block steps
// is not paced by global-memory latency.
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
__device__ __forceinline__ float load_a(const GdnArgs &g, size_t idx) {
  if (U16) return static_cast<float>(static_cast<int>(static_cast<const uint16_t *>(g.A)[idx]) - g.zpA) * g.sA;
  return static_cast<const float *>(g.A)[idx];
}

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
  // LDS: diagonal inverses of blocks J..nb-1, the solved panel rows, one staged A row block
  // (16 rows x up to 240 columns), and per-wave partial products.
  __shared__ float tdiag[kMaxNb][16][17];
  __shared__ float xs[kMaxNb * 16][16];
  __shared__ float abuf[16][kMaxNb * 16 + 4];
  __shared__ float gpart[4][16][17];

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int J = blockIdx.x, head = blockIdx.y;
  const int C = g.C, nb = g.nb;
  const size_t hbase = static_cast<size_t>(head) * C * C;
  const int c0 = J * 16;

  // ---- zero the panel above its diagonal block ------------------------------------------
  for (int e = t; e < c0 * 16; e += kGdnThreads) {
    const int r = e >> 4, c = e & 15;
    store_t<U16>(g, hbase + static_cast<size_t>(r) * C + c0 + c, 0.0f);
  }

  float4 pre0[4], pre1[4];
  auto prefetch = [&](int I, float4 (&pre)[4]) {
    const int L = 16 * (I - J), q = L / 4;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int e = t + u * kGdnThreads;
      if (e < 16 * q) {
        const int r = e / q, c4 = e % q;
        pre[u] = load_a4<U16>(g, hbase + static_cast<size_t>(I * 16 + r) * C + c0 + 4 * c4);
      }
    }
  };
  auto commit = [&](int I, const float4 (&pre)[4]) {
    const int L = 16 * (I - J), q = L / 4;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int e = t + u * kGdnThreads;
      if (e < 16 * q) {
        const int r = e / q, c4 = e % q;
        abuf[r][4 * c4 + 0] = pre[u].x;
        abuf[r][4 * c4 + 1] = pre[u].y;
        abuf[r][4 * c4 + 2] = pre[u].z;
        abuf[r][4 * c4 + 3] = pre[u].w;
      }
    }
  };
  // ---- diagonal inverses T_II, I = J .. nb-1 ----------------------------------------------
  for (int base = J; base < nb; base += 16) {
    // stage the 16x16 diagonal blocks of this round
    for (int e = t; e < 16 * 256; e += kGdnThreads) {
      const int b = e >> 8, i = (e >> 4) & 15, k = e & 15;
      const int I = base + b;
      if (I < nb) abuf[i][b * 16 + k] = load_a<U16>(g, hbase + static_cast<size_t>(I * 16 + i) * C + I * 16 + k);
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
        float s = (i == j) ? 1.0f : 0.0f;
#pragma unroll
        for (int k = 0; k < i; ++k) s = fmaf(abuf[i][b * 16 + k], x[k], s);
        x[i] = s;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) tdiag[I - J][i][j] = x[i];
    }
    lds_barrier();
  }

  // ---- X_J = T_JJ ----------------------------------------------------------------------------
  {
    const int i = t >> 4, j = t & 15;
    const float v = tdiag[0][i][j];
    xs[i][j] = v;
    store_t<U16>(g, hbase + static_cast<size_t>(c0 + i) * C + c0 + j, v);
  }

  // ---- block forward substitution down the panel -------------------------------------------
  // Row block I needs A[16I .. 16I+15][c0 .. 16I-1]: 16 rows x L columns, L = 16 (I - J).
  // Each thread holds up to 4 float4 of a block (16 * 240 / 4 / 256 < 4); two blocks are in
  // flight ahead of the one being multiplied.
  // Row blocks alternate between the two prefetch slots (a register copy between slots would
  // wait for the load in flight).
  auto step = [&](const int I, float4 (&pre)[4]) __attribute__((always_inline)) {
    lds_barrier();  // xs rows of the previous block visible; abuf free
    commit(I, pre);
    lds_barrier();
    if (I + 2 < nb) prefetch(I + 2, pre);  // the slot just committed takes block I + 2
    const int L = 16 * (I - J);
    // partial G over this wave's 16-wide K blocks
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    const int r = lane & 15, kq = lane >> 4;
    if (!BF16) {
      for (int kb = wave; kb < I - J; kb += 4) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int k = kb * 16 + 4 * s + kq;
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(abuf[r][k], xs[k][r], acc, 0, 0, 0);
        }
      }
    } else {
      // 32-deep bf16 steps: wave w takes steps w, w+4, ...; the last half step is zero-padded.
      const int steps = (L + 31) / 32;
      for (int st = wave; st < steps; st += 4) {
        v8bf a, b;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
          const int k = st * 32 + 8 * kq + jj;
          const bool ok = k < L;
          a[jj] = static_cast<__bf16>(ok ? abuf[r][k] : 0.0f);
          b[jj] = static_cast<__bf16>(ok ? xs[k][r] : 0.0f);
        }
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) gpart[wave][4 * kq + q][r] = acc[q];
    lds_barrier();
    if (wave == 0) {
      // G (summed over waves) as the B operand of X_I = T_II G
      v4f x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int k = 4 * s + kq;
        const float gk = gpart[0][k][r] + gpart[1][k][r] + gpart[2][k][r] + gpart[3][k][r];
        x = __builtin_amdgcn_mfma_f32_16x16x4f32(tdiag[I - J][r][k], gk, x, 0, 0, 0);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int row = 4 * kq + q;
        xs[L + row][r] = x[q];
        store_t<U16>(g, hbase + static_cast<size_t>(I * 16 + row) * C + c0 + r, x[q]);
      }
    }
  };
  for (int I = J + 1; I < nb; I += 2) {
    step(I, pre0);
    if (I + 1 < nb) step(I + 1, pre1);
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
