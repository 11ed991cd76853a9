// GDN / KDA per-head triangular solve T = (I - A)^-1, A strictly lower triangular, C <= 256, by
// recursive doubling with matrix-core merges.
//
// C is padded to P = 2^p >= C (zero A there, so the padding's T is the identity and never
// couples to the rest):
//   level 0: the 16 x 16 diagonal blocks T_bb = (I - A_bb)^-1 by forward substitution in fp32,
//            one lane per column;
//   level s = 16, 32, .., P/2: pairs of diagonal blocks of size s merge into blocks of size 2s,
//            [T11 0; A21 T22] -> [T11 0; T21 T22] with T21 = T22 (A21 T11)
//            -- the block-recursive merge of GdnSolveBR (M = A21 T11, T21 = T22 M,
//            example/gdn_native/solve_br_op/src/gdn_solve_br_core.h:1-8) applied at every
//            level, which equals the block merges T_ij = T_ii sum_k A_ik T_kj of
//            example/gdn_native/solve_op/src/gdn_solve_core.h:50-72: log2(P / 16) dependent
//            levels instead of P / 16 - 1 block steps.
// Work split: G = P / 32 workgroups (8 waves each) per head.  Every workgroup of a head computes
// the two block-diagonal halves (levels 0 .. P/4) itself -- short, latency-bound levels whose
// redundancy costs less than a cross-workgroup exchange -- then one 16-column strip of the last
// merge (T21 rows P/2 .. P-1).  The G workgroups of a head get block indexes of one residue mod
// 8, which places them on one XCD and one L2.
// Inside the halves a level gives each wave one 16-row tile of one merge's T21:
//   Y[i][:] = A21[i][:] T11, written to LDS transposed in the merge's upper-right block (the
//            zero block T12, which no product ever reads), then
//   X[i][:] = sum_{l <= i} T22[i][l] Y[l][:]  (registers; into the T21 region at once).
// The products run on v_mfma_f32_16x16x32_bf16: a 32-deep k step takes rows 4q .. 4q+3 of two
// 16-row blocks, the k order in which the MFMA result layout (lane: rows 4q .. 4q+3 of one
// column) is read back as the next B operand.
// LDS holds T's block-diagonal halves (row r holds the columns of its half) as packed bf16
// hi | lo words (lo = bf16(x - hi)), the form the MFMA operands take; each level's fp32 results
// go to global memory from registers, so T is exact fp32 accumulation output.
// Memory order: one counter tracks vector loads and stores together, so a wait for a load also
// waits for every store issued before it.  All of a workgroup's A reads are therefore issued at
// the start, straight-line (a skipped read becomes a discarded read), level 0's first; stores
// only follow.
// Precision: QH_GDN_FP32 multiplies hi/lo splits (hi*hi + hi*lo + lo*hi, fp32 accumulation:
// about 16 significant bits per product); QH_GDN_BF16 multiplies the hi parts only.  The
// diagonal blocks are fp32 in both.
// The u16 variant applies the GdnSolve op's code contract on load / store
// (A = (code - zpA) * sA; T_code = clip(rint(T / sT) + zpT, 0, 65535)).

#include "bf16_split.h"
#include "qmm_internal.h"

namespace qh {
namespace {

using namespace bf16s;

constexpr int kRdThreads = 512;
constexpr int kTs = 132;   // LDS row stride of the T store, words (conflict-free column reads)
constexpr int kAtRow = 20;  // staged diagonal block A^T: row stride (16-byte aligned rows) ..
constexpr int kAtBlk = 336;  // .. and block stride (= 16 mod 64 banks: the 4 blocks of a wave differ)

struct GdnArgs {
  const void *A;
  void *T;
  int C, P, half, groups, heads;
  int zpA, zpT;
  float sA, sT, inv_sT;
};

__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// 4 consecutive A values of the head (row r, columns c .. c + 3, c % 4 == 0), in bounds.
template <bool U16>
__device__ __forceinline__ float4 load_a4(const GdnArgs &g, size_t hbase, int r, int c) {
  const size_t idx = hbase + static_cast<size_t>(r) * g.C + c;
  if (U16) {
    const uint2 v = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(g.A) + idx);
    return make_float4(static_cast<float>(static_cast<int>(v.x & 0xFFFFu) - g.zpA) * g.sA,
                       static_cast<float>(static_cast<int>(v.x >> 16) - g.zpA) * g.sA,
                       static_cast<float>(static_cast<int>(v.y & 0xFFFFu) - g.zpA) * g.sA,
                       static_cast<float>(static_cast<int>(v.y >> 16) - g.zpA) * g.sA);
  }
  return *reinterpret_cast<const float4 *>(static_cast<const float *>(g.A) + idx);
}

// load_a4 when ok, else zeros -- without a branch: a skipped read is a read of the head's first
// values, discarded.  The reads before level 0 stay straight-line code, so the compiler counts
// exactly which of them each wait needs (after a branch it waits for all of them).
template <bool U16>
__device__ __forceinline__ float4 load_a4_or0(const GdnArgs &g, size_t hbase, int r, int c, bool ok) {
  const float4 v = load_a4<U16>(g, hbase, ok ? r : 0, ok ? c : 0);
  return ok ? v : make_float4(0.f, 0.f, 0.f, 0.f);
}

template <bool U16>
__device__ __forceinline__ uint16_t t_code(const GdnArgs &g, float v) {
  float q = rintf(v * g.inv_sT) + static_cast<float>(g.zpT);
  q = fminf(fmaxf(q, 0.0f), 65535.0f);
  return static_cast<uint16_t>(q);
}

template <bool U16>
__device__ __forceinline__ void store_t(const GdnArgs &g, size_t idx, float v) {
  if (U16) {
    static_cast<uint16_t *>(g.T)[idx] = t_code<U16>(g, v);
  } else {
    static_cast<float *>(g.T)[idx] = v;
  }
}

// The MFMA result tile acc (rows row0 + 4q + e, column col) to T.
template <bool U16>
__device__ __forceinline__ void store_tile(const GdnArgs &g, size_t hbase, int row0, int col, int q, const v4f &acc) {
#pragma unroll
  for (int e = 0; e < 4; ++e) store_t<U16>(g, hbase + static_cast<size_t>(row0 + 4 * q + e) * g.C + col, acc[e]);
}

// Wave -> (merge at row b, tile i) of a level inside the halves (NB tiles per block): P / 32
// tasks, one per wave.  Waves w and w + 4 share a SIMD; the T22 product of tile i costs i + 1 k
// blocks, so the second half of the waves takes the tiles of its merge in reverse order.
template <int NB>
__device__ __forceinline__ void tile_task(int wave, int &b, int &i) {
  const int m = wave / NB, ii = wave % NB;
  i = wave >= 4 ? NB - 1 - ii : ii;
  b = 32 * NB * m;
}

// A21 row blocks of tile i of the merge at row b (NB = s / 16): block l holds row b + s + 16 i +
// r16, columns b + 16 l + 4q .. + 3 (zero past C or when !ok).
template <bool U16, int NB>
__device__ __forceinline__ void load_tile(const GdnArgs &g, size_t hbase, int b, int i, bool ok, int lane,
                                          float4 (&av)[NB]) {
  constexpr int s = 16 * NB;
  const int r16 = lane & 15, q = lane >> 4;
#pragma unroll
  for (int l = 0; l < NB; ++l)
    av[l] = load_a4_or0<U16>(g, hbase, b + s + 16 * i + r16, b + 16 * l + 4 * q,
                             ok && b + s + 16 * i < g.C && b + 16 * l < g.C);
}

// One merge level inside the halves (NB tiles per block), tile i of the merge at row b per task
// wave; `owner` marks the workgroup that stores this task's T21 tile.  Two barriers: Y complete
// (in the upper-right block, rows b .. b + s, columns b + s .. b + 2 s), then X complete (in the
// T21 region, which no wave reads during the X products).
template <bool U16, bool SPLIT, int NB>
__device__ __forceinline__ void merge_level(const GdnArgs &g, size_t hbase, uint32_t (*Tl)[kTs], bool task, bool owner,
                                            int b, int i, const float4 (&av)[NB], int lane) {
  constexpr int s = 16 * NB;
  const int r16 = lane & 15, q = lane >> 4;
  const int shift = b >= g.half ? g.half : 0;  // Tl column offset of this merge's rows
  const int rt = b + s + 16 * i;                // first row of this wave's tile
  if (task) {
    Half4 as[NB];
#pragma unroll
    for (int l = 0; l < NB; ++l) as[l] = split4<SPLIT>(av[l]);
#pragma unroll
    for (int j = 0; j < NB; ++j) {  // strip j: T11 is zero above block j, so k blocks l = j ..
      const int c = b - shift + 16 * j + r16;
      v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int l = j; l < NB; l += 2) {
        const bool two = l + 1 < NB;
        const int r0 = b + 16 * l + 4 * q;
        const Half4 t0 = unpack4(Tl[r0][c], Tl[r0 + 1][c], Tl[r0 + 2][c], Tl[r0 + 3][c]);
        const Half4 t1 = two ? unpack4(Tl[r0 + 16][c], Tl[r0 + 17][c], Tl[r0 + 18][c], Tl[r0 + 19][c]) : kZero4;
        acc = mma<SPLIT>(as[l], two ? as[l + 1] : kZero4, t0, t1, acc);
      }
      // Y tile (i, j) transposed at tile (i, j) of the upper-right block: row b + 16 i + column,
      // column b + s + 16 j + row (half-local)
      *reinterpret_cast<uint4 *>(&Tl[b + 16 * i + r16][b - shift + s + 16 * j + 4 * q]) =
          make_uint4(hilo<SPLIT>(acc[0]), hilo<SPLIT>(acc[1]), hilo<SPLIT>(acc[2]), hilo<SPLIT>(acc[3]));
    }
  }
  lds_barrier();
  v4f X[NB];
#pragma unroll
  for (int j = 0; j < NB; ++j) X[j] = v4f{0.f, 0.f, 0.f, 0.f};
  if (task) {
    const uint32_t *trow = Tl[rt + r16];
    for (int l = 0; l <= i; l += 2) {  // wave-uniform bounds
      const bool two = l + 1 <= i;
      const int cA = b + s - shift + 16 * l + 4 * q;  // Tl column of T22's block l, this lane's k
      const Half4 w0 = unpack4(*reinterpret_cast<const uint4 *>(trow + cA));
      const Half4 w1 = two ? unpack4(*reinterpret_cast<const uint4 *>(trow + cA + 16)) : kZero4;
      const uint32_t *yrow = Tl[b + 16 * l + r16];  // transposed Y tile (l, j): column r16 of it
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const int c = b - shift + s + 16 * j + 4 * q;
        const Half4 y0 = unpack4(*reinterpret_cast<const uint4 *>(yrow + c));
        const Half4 y1 = two ? unpack4(*reinterpret_cast<const uint4 *>(yrow + 16 * kTs + c)) : kZero4;
        X[j] = mma<SPLIT>(w0, w1, y0, y1, X[j]);
      }
    }
    if (owner && rt < g.C) {
#pragma unroll
      for (int j = 0; j < NB; ++j)
        if (b + 16 * j < g.C) store_tile<U16>(g, hbase, rt, b + 16 * j + r16, q, X[j]);
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
#pragma unroll
      for (int e = 0; e < 4; ++e) Tl[rt + 4 * q + e][b - shift + 16 * j + r16] = hilo<SPLIT>(X[j][e]);
    }
  }
  lds_barrier();
}

// Level 0 from the staged, transposed diagonal blocks (At[k][r] = A[r][k]): block t / 16, column
// jc = t % 16 per thread, by a column sweep -- at step i, x_i is final and every later row takes
// A[r][i] x_i -- which keeps each x_r's sum in the order k = 0, 1, .. of plain forward
// substitution while the dependent chain is one FMA per step.  Results into LDS; the workgroup
// `part` stores blocks 2 part and 2 part + 1.
template <bool U16, bool SPLIT>
__device__ __forceinline__ void level0(const GdnArgs &g, size_t hbase, uint32_t (*Tl)[kTs], const float *dstage,
                                       int nblocks, int part, int t) {
  const int bb = t >> 4, jc = t & 15;
  if (bb < nblocks) {
    // column i of A (rows 0 .. 15) = row i of At: 4 aligned float4, two columns read ahead
    const float4 *At = static_cast<const float4 *>(__builtin_assume_aligned(dstage + bb * kAtBlk, 16));
    float x[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) x[r] = (r == jc) ? 1.0f : 0.0f;
    float4 col[3][4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int m = 0; m < 4; ++m) col[i][m] = At[i * (kAtRow / 4) + m];
    }
#pragma unroll
    for (int i = 0; i < 15; ++i) {
      if (i + 2 < 15) {
#pragma unroll
        for (int m = (i + 3) / 4; m < 4; ++m) col[(i + 2) % 3][m] = At[(i + 2) * (kAtRow / 4) + m];
      }
      __builtin_amdgcn_sched_barrier(0);  // the reads ahead stay ahead
      const float xi = x[i];
#pragma unroll
      for (int m = (i + 1) / 4; m < 4; ++m) {
        const float4 v = col[i % 3][m];
        const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (4 * m + e > i) x[4 * m + e] = fmaf(vv[e], xi, x[4 * m + e]);
      }
    }
    const int col0 = 16 * bb + jc;
    const int lcol = col0 - (16 * bb >= g.half ? g.half : 0);
#pragma unroll
    for (int i = 0; i < 16; ++i) Tl[16 * bb + i][lcol] = hilo<SPLIT>(x[i]);
    if ((bb >> 1) == part && 16 * bb < g.C) {
#pragma unroll
      for (int i = 0; i < 16; ++i) store_t<U16>(g, hbase + static_cast<size_t>(16 * bb + i) * g.C + col0, x[i]);
    }
  }
}

// Stages a diagonal-block row quarter (row i, columns 4 k4 .. + 3 of block bb) transposed.
__device__ __forceinline__ void stage_at(float *dstage, int bb, int i, int k4, const float4 v) {
  float *d = dstage + bb * kAtBlk + (4 * k4) * kAtRow + i;
  d[0] = v.x;
  d[kAtRow] = v.y;
  d[2 * kAtRow] = v.z;
  d[3 * kAtRow] = v.w;
}

// Zeros above the block diagonal: workgroup `part` of `groups` takes rows part, part + groups, ..,
// one row per wave at a time, one float4 per lane (C / 4 <= 64).
template <bool U16>
__device__ __forceinline__ void store_zeros(const GdnArgs &g, size_t hbase, int part, int wave, int lane) {
  const int C = g.C;
  for (int row = part + wave * g.groups; row < C; row += 8 * g.groups) {
    const int c = 4 * lane;
    if (c < C && c >= 16 * (row / 16) + 16) {
      const size_t idx = hbase + static_cast<size_t>(row) * C + c;
      if (U16) {
        const uint32_t z = static_cast<uint32_t>(g.zpT) * 0x10001u;  // code of 0.0: clip(zpT)
        *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(g.T) + idx) = make_uint2(z, z);
      } else {
        *reinterpret_cast<float4 *>(static_cast<float *>(g.T) + idx) = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
  }
}

// The solve for padded size P = 2^LOGP (32 <= P <= 256) by workgroup `part` of G = P / 32.
template <bool U16, bool SPLIT, int LOGP>
__device__ __forceinline__ void solve_head(const GdnArgs &g, uint32_t (*Tl)[kTs], float *dstage, int part,
                                           size_t hbase, int t, int wave, int lane) {
  constexpr int P = 1 << LOGP;
  constexpr int NBF = P / 32;  // 16-row tiles per block of the last merge
  const int C = g.C;
  const int r16 = lane & 15, q = lane >> 4;
  // ---- A reads: level 0's, then each level's, straight-line ---------------------------------------
  float4 dv[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {  // float4 slot t + 512 u: block wave + 8 u, row (t / 4) % 16, quarter t % 4
    const int bb = wave + 8 * u, i = (lane >> 2) & 15, k4 = lane & 3;
    dv[u] = load_a4_or0<U16>(g, hbase, 16 * bb + i, 16 * bb + 4 * k4, bb < P / 16 && 16 * bb < C);
  }
  __builtin_amdgcn_sched_barrier(0);  // keep level 0's reads first: its wait then covers only them
  const bool task = wave < P / 32;
  const bool owner = wave == part;  // this workgroup stores task `part` of every level
  int b1 = 0, i1 = 0, b2 = 0, i2 = 0, b4 = 0, i4 = 0;
  float4 a1[1], a2[2], a4[4];
  if (P > 32) {
    tile_task<1>(wave, b1, i1);
    load_tile<U16, 1>(g, hbase, b1, i1, task, lane, a1);
  }
  if (P > 64) tile_task<2>(wave, b2, i2);
  if (P > 128) tile_task<4>(wave, b4, i4);
  // last merge, strip `part`, tile `wave`: k blocks l = part + 2 p + h
  constexpr int kPF = (NBF + 1) / 2;
  float4 af[kPF][2];
  auto load_last = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int p = 0; p < kPF; ++p) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int l = part + 2 * p + h;
        af[p][h] = load_a4_or0<U16>(g, hbase, P / 2 + 16 * wave + r16, 16 * l + 4 * q,
                                    wave < NBF && l < NBF && P / 2 + 16 * wave < C && 16 * l < C);
      }
    }
  };
  __builtin_amdgcn_sched_barrier(0);

  // ---- level 0 ------------------------------------------------------------------------------------
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int bb = wave + 8 * u, i = (lane >> 2) & 15, k4 = lane & 3;
    if (bb < P / 16) stage_at(dstage, bb, i, k4, dv[u]);
  }
  lds_barrier();
  level0<U16, SPLIT>(g, hbase, Tl, dstage, P / 16, part, t);
  lds_barrier();
  store_zeros<U16>(g, hbase, part, wave, lane);

  // ---- merges inside the halves -------------------------------------------------------------------
  // Each level's A tiles are requested one level ahead (the last merge's strip two ahead), so the
  // requests are issued a few at a time; the stores issued before them are a level old by the
  // time the wait for them (which counts those stores too) comes.
  if (P > 64) load_tile<U16, 2>(g, hbase, b2, i2, task, lane, a2);
  if (P <= 128) load_last();
  if (P > 32) merge_level<U16, SPLIT, 1>(g, hbase, Tl, task, owner, b1, i1, a1, lane);
  if (P > 128) load_tile<U16, 4>(g, hbase, b4, i4, task, lane, a4);
  if (P > 64) merge_level<U16, SPLIT, 2>(g, hbase, Tl, task, owner, b2, i2, a2, lane);
  if (P > 128) load_last();
  if (P > 128) merge_level<U16, SPLIT, 4>(g, hbase, Tl, task, owner, b4, i4, a4, lane);

  // ---- last merge, strip `part`: Y tiles (one per wave) through LDS, then T21 = T22 Y -----------
  // Y tiles, transposed (ybuf[tile][column][row]): level 0 is done with the staging area
  uint32_t(*ybuf)[16][16] = reinterpret_cast<uint32_t(*)[16][16]>(dstage);
  if (wave < NBF) {
    v4f y = {0.f, 0.f, 0.f, 0.f};
    const int c = 16 * part + r16;  // T11 is in the first half: Tl column = T column
#pragma unroll
    for (int p = 0; p < kPF; ++p) {
      const int l = part + 2 * p;
      if (l >= NBF) break;  // part is uniform: a scalar branch
      const bool two = l + 1 < NBF;
      const int r0 = 16 * l + 4 * q;
      const Half4 t0 = unpack4(Tl[r0][c], Tl[r0 + 1][c], Tl[r0 + 2][c], Tl[r0 + 3][c]);
      const Half4 t1 = two ? unpack4(Tl[r0 + 16][c], Tl[r0 + 17][c], Tl[r0 + 18][c], Tl[r0 + 19][c]) : kZero4;
      y = mma<SPLIT>(split4<SPLIT>(af[p][0]), two ? split4<SPLIT>(af[p][1]) : kZero4, t0, t1, y);
    }
    *reinterpret_cast<uint4 *>(&ybuf[wave][r16][4 * q]) =
        make_uint4(hilo<SPLIT>(y[0]), hilo<SPLIT>(y[1]), hilo<SPLIT>(y[2]), hilo<SPLIT>(y[3]));
  }
  lds_barrier();
  if (wave < NBF) {
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    const uint32_t *trow = Tl[P / 2 + 16 * wave + r16];  // T22 row; its Tl columns start at 0
    for (int l = 0; l <= wave; l += 2) {  // wave-uniform bounds
      const bool two = l + 1 <= wave;
      const Half4 w0 = unpack4(*reinterpret_cast<const uint4 *>(trow + 16 * l + 4 * q));
      const Half4 w1 = two ? unpack4(*reinterpret_cast<const uint4 *>(trow + 16 * l + 16 + 4 * q)) : kZero4;
      const Half4 y0 = unpack4(*reinterpret_cast<const uint4 *>(&ybuf[l][r16][4 * q]));
      const Half4 y1 = two ? unpack4(*reinterpret_cast<const uint4 *>(&ybuf[l + 1][r16][4 * q])) : kZero4;
      acc = mma<SPLIT>(w0, w1, y0, y1, acc);
    }
    if (P / 2 + 16 * wave < C && 16 * part < C) store_tile<U16>(g, hbase, P / 2 + 16 * wave, 16 * part + r16, q, acc);
  }
}

template <bool U16, bool SPLIT>
__global__ __launch_bounds__(kRdThreads) void gdn_rd_kernel(GdnArgs g) {
  __shared__ __attribute__((aligned(16))) uint32_t Tl[256][kTs];     // block-diagonal halves of T, hi | lo
  __shared__ __attribute__((aligned(16))) float dstage[16 * kAtBlk];  // A's diagonal blocks (A^T); then Y tiles
  const int t = threadIdx.x, lane = t & 63;
  // The wave index (and the task indexes derived from it) must be scalar: the merge loops branch
  // on it, and a branch on a vector value becomes an exec-masked region, in which the MFMA still
  // runs while the conversions that build its operands do not.
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  // Workgroups go to the 8 XCDs round-robin (block b on XCD b % 8), each XCD with its own L2: the
  // `groups` workgroups of one head all read that head's A, so they are given block indexes of
  // one residue mod 8.  Block b: XCD x = b % 8, k = b / 8, part = k % groups, head = x + 8 (k /
  // groups); the grid is rounded up to whole sets of 8 heads.
  const int k8 = blockIdx.x >> 3;
  const int head = (blockIdx.x & 7) + 8 * (k8 / g.groups), part = k8 % g.groups;
  if (head >= g.heads) return;  // uniform: the whole workgroup leaves before any barrier
  const size_t hbase = static_cast<size_t>(head) * g.C * g.C;
  switch (g.P) {
    case 16: {  // one diagonal block
      if (t < 64) {
        const int i = (lane >> 2) & 15, k4 = lane & 3;
        stage_at(dstage, 0, i, k4, load_a4<U16>(g, hbase, i, 4 * k4));
      }
      lds_barrier();
      level0<U16, SPLIT>(g, hbase, Tl, dstage, 1, 0, t);
      store_zeros<U16>(g, hbase, 0, wave, lane);
      break;
    }
    case 32: solve_head<U16, SPLIT, 5>(g, Tl, dstage, part, hbase, t, wave, lane); break;
    case 64: solve_head<U16, SPLIT, 6>(g, Tl, dstage, part, hbase, t, wave, lane); break;
    case 128: solve_head<U16, SPLIT, 7>(g, Tl, dstage, part, hbase, t, wave, lane); break;
    default: solve_head<U16, SPLIT, 8>(g, Tl, dstage, part, hbase, t, wave, lane); break;
  }
}

template <bool U16, bool SPLIT>
qh_status launch(const GdnArgs &g, int heads, hipStream_t stream) {
  const long long blocks = static_cast<long long>((heads + 7) / 8) * 8 * g.groups;
  if (blocks > 0x7FFFFFFFLL) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "gdn: %d heads exceed one launch", heads);
  hipLaunchKernelGGL((gdn_rd_kernel<U16, SPLIT>), dim3(static_cast<unsigned>(blocks)), dim3(kRdThreads), 0, stream, g);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return hip_fail(err, "gdn_rd_kernel launch");
  return QH_STATUS_OK;
}

GdnArgs make_args(const void *A, void *T, int heads, int C, int zpA, int zpT, float sA, float sT) {
  int P = 16;
  while (P < C) P *= 2;
  return GdnArgs{A, T, C, P, P >= 32 ? P / 2 : 16, P >= 32 ? P / 32 : 1, heads, zpA, zpT, sA, sT, 1.0f / sT};
}

}  // namespace

qh_status launch_gdn_solve_f32(const float *A, float *T, int heads, int C, int precision, hipStream_t stream) {
  const GdnArgs g = make_args(A, T, heads, C, 0, 0, 1.0f, 1.0f);
  return precision == QH_GDN_BF16 ? launch<false, false>(g, heads, stream) : launch<false, true>(g, heads, stream);
}

qh_status launch_gdn_solve_u16(const uint16_t *A, uint16_t *T, int heads, int C, int zpA, int zpT, float sA, float sT,
                               int precision, hipStream_t stream) {
  const GdnArgs g = make_args(A, T, heads, C, zpA, zpT, sA, sT);
  return precision == QH_GDN_BF16 ? launch<true, false>(g, heads, stream) : launch<true, true>(g, heads, stream);
}

}  // namespace qh
