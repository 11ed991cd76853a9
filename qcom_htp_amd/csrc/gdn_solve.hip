// GDN / KDA per-head triangular solve T = (I - A)^-1, A strictly lower triangular, C <= 256
// (C % 16 == 0, NB = C / 16 diagonal blocks), by block forward substitution over 16-column
// strips on the matrix cores.
//
//   level 0: the 16 x 16 diagonal blocks T_bb = (I - A_bb)^-1 by forward substitution in fp32,
//            one lane per column;
//   strip j: X = T[:, 16 j .. 16 j + 15] solves (I - A) X = E_j, block by block:
//            X_j = T_jj,  X_b = T_bb sum_{j <= c < b} A_bc X_c  (b = j + 1 .. NB - 1),
//            the block merges T_ij = T_ii sum_k A_ik T_kj of
//            example/gdn_native/solve_op/src/gdn_solve_core.h:50-72 taken one column strip at
//            a time.
// One wave runs one strip.  Its X_c stay in registers in the MFMA result layout, which is also
// the B operand layout of the next products (bf16_split.h), so the NB - 1 - j steps of a strip
// need no barrier and no LDS round trip for X; the A blocks and T_bb are LDS reads, issued one
// step ahead.  Every strip reads A's strictly lower blocks, so a workgroup stages them in LDS
// once, as ready operand records.
// Work split: G = 2 workgroups (8 waves) per head for NB > 8, one otherwise.  Strips k and
// NB - 1 - k share a SIMD (waves w and w + 4), so the longest strip (k = 0) has its SIMD's matrix
// core nearly to itself.  The G workgroups of a head get block indexes of one residue mod 8,
// which places them on one XCD and one L2.
// The products run on v_mfma_f32_16x16x32_bf16: a 32-deep k step takes rows 4q .. 4q+3 of two
// 16-row blocks, the k order in which the MFMA result layout (lane: rows 4q .. 4q+3 of one
// column) is read back as the next B operand.
// Precision: QH_GDN_FP32 multiplies hi/lo splits (hi*hi + hi*lo + lo*hi, fp32 accumulation:
// about 16 significant bits per product); QH_GDN_BF16 multiplies the hi parts only.  The
// diagonal blocks are fp32 in both, and T is stored from the fp32 accumulators.
// The u16 variant applies the GdnSolve op's code contract on load / store
// (A = (code - zpA) * sA; T_code = clip(rint(T / sT) + zpT, 0, 65535)).

#include "bf16_split.h"
#include "qmm_internal.h"

namespace qh {
namespace {

using namespace bf16s;

typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef unsigned int v2u __attribute__((ext_vector_type(2)));

constexpr int kRdThreads = 512;
constexpr int kAtRow = 20;  // staged diagonal block A^T: row stride (16-byte aligned rows) ..
constexpr int kAtBlk = 336;  // .. and block stride (= 16 mod 64 banks: the 4 blocks of a wave differ)

struct GdnArgs {
  const void *A;
  void *T;
  int C, groups, heads;
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

// Stages a diagonal-block row quarter (row i, columns 4 k4 .. + 3 of block bb) transposed.
__device__ __forceinline__ void stage_at(float *dstage, int bb, int i, int k4, const float4 v) {
  float *d = dstage + bb * kAtBlk + (4 * k4) * kAtRow + i;
  d[0] = v.x;
  d[kAtRow] = v.y;
  d[2 * kAtRow] = v.z;
  d[3 * kAtRow] = v.w;
}

constexpr int kFsMaxNB = 16;
constexpr int kFsLowBlocks = kFsMaxNB * (kFsMaxNB - 1) / 2;  // strictly lower 16 x 16 blocks
constexpr int kFsTd = 16;  // Td row stride, words

// Word column of column c in row r of a 16 x 16 LDS block: the 4-word quarters of row r are
// XOR-swizzled by r / 4.  An A operand read (lane: row r16, quarter q, 16 bytes) then puts the 16
// lanes of a quarter on 16 distinct 16-byte bank groups; unswizzled, rows 64 bytes apart shared 4
// groups (4-way bank conflicts on every read).
__device__ __forceinline__ int fs_col(int r, int c) { return ((((c >> 2) ^ (r >> 2)) & 3) << 2) | (c & 3); }

// Strip of wave `wave` in workgroup `part`: pair k = 4 part + wave % 4, strip k for waves 0..3 and
// NB - 1 - k for waves 4..7 (none when that would repeat strip k or lie past NB).
__device__ __forceinline__ int fs_strip(int NB, int part, int wave) {
  const int k = 4 * part + (wave & 3);
  const int j = wave < 4 ? k : NB - 1 - k;
  return (j < NB && (wave < 4 || j > k)) ? j : -1;
}

// Level 0 into Td (T_bb as hi | lo words, row-major with fs_col quarters) from the staged
// transposed diagonal blocks (At[k][r] = A[r][k]): block t / 16, column jc = t % 16 per thread, by
// a column sweep -- at step i, x_i is final and every later row takes A[r][i] x_i -- which keeps
// each x_r's sum in the order k = 0, 1, .. of plain forward substitution while the dependent
// chain is one FMA per step.  T_bb also goes, in fp32 and row-major, over its own staged block
// in dstage (read only by this wave, and fully read by the time the sweep ends), for the wave of
// strip bb to store: stores issued here kept the strips waiting (their data registers are reused
// by the strips, and the compiler then waits for the stores).
template <bool SPLIT>
__device__ __forceinline__ void fs_level0(uint32_t (*Td)[16][kFsTd], float *dstage, int NB, int t) {
  const int bb = t >> 4, jc = t & 15;
  if (bb < NB) {
    const float4 *At = static_cast<const float4 *>(__builtin_assume_aligned(dstage + bb * kAtBlk, 16));  // A_bb^T
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
#pragma unroll
    for (int i = 0; i < 16; ++i) Td[bb][i][fs_col(i, jc)] = hilo<SPLIT>(x[i]);
    float *const tf = dstage + bb * kAtBlk;
#pragma unroll
    for (int i = 0; i < 16; ++i) tf[16 * i + jc] = x[i];
  }
}

// The MFMA result tile acc (lane: rows row0 + 4q + e of column col0 + r16) to T by rows: the 4
// lanes of a quad transpose their 4 x 4 values in two DPP butterfly stages (partner lane p ^ 1,
// then p ^ 2), after which lane 4a + p holds row row0 + 4q + p, columns col0 + 4a .. + 3 and
// stores them at once (one 16-byte store where the column layout took four 4-byte ones).  The
// store is a buffer store: the tile's offset (row0 C + col0 elements) is a scalar and the lane's
// part (lane_off) one register for the whole strip, so no per-store address register is
// rewritten while earlier stores may still read theirs.
template <bool U16>
__device__ __forceinline__ void store_tile_rows(const GdnArgs &g, __amdgpu_buffer_rsrc_t tr, uint32_t lane_off,
                                                int row0, int col0, int lane, const v4f &acc, float (&w)[4]) {
  const int p = lane & 3;
  float u[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float o = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(acc[e ^ 1]), 0xB1, 0xF, 0xF, false));
    u[e] = ((e ^ p) & 1) ? o : acc[e];
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float o = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(u[e ^ 2]), 0x4E, 0xF, 0xF, false));
    w[e] = ((e ^ p) & 2) ? o : u[e];
  }
  const int soff = __builtin_amdgcn_readfirstlane((row0 * g.C + col0) * (U16 ? 2 : 4));
  if (U16) {
    const uint32_t c01 = t_code<U16>(g, w[0]) | (static_cast<uint32_t>(t_code<U16>(g, w[1])) << 16);
    const uint32_t c23 = t_code<U16>(g, w[2]) | (static_cast<uint32_t>(t_code<U16>(g, w[3])) << 16);
    __builtin_amdgcn_raw_buffer_store_b64(v2u{c01, c23}, tr, static_cast<int>(lane_off), soff, 0);
  } else {
    __builtin_amdgcn_raw_buffer_store_b128(v4u{__float_as_uint(w[0]), __float_as_uint(w[1]), __float_as_uint(w[2]), __float_as_uint(w[3])},
                                           tr, static_cast<int>(lane_off), soff, 0);
  }
}

// One wave's strip j (after level 0, with Al, Td and the fp32 T_bb in dstage staged): T_jj, then
// the strip's steps, each tile stored as it is computed.
template <bool U16, bool SPLIT>
__device__ __forceinline__ void fs_strip_solve(const GdnArgs &g, size_t hbase, const uint32_t (*Al)[16][16],
                                               const uint32_t (*Td)[16][kFsTd], const float *dstage, int NB, int j,
                                               int lane) {
  const int r16 = lane & 15, q = lane >> 4;
  // Blocks are indexed relative to the strip (u = c - j, v = b - j), so every step's loops have
  // compile-time bounds: a step is one basic block whose LDS reads all issue before its products
  // (guards per block pair made each pair wait for its own reads).
  Half4 xs[kFsMaxNB];  // X_{j+u} as B operands (rows 4q .. 4q + 3 of column r16)
  // The stored values of every step stay allocated until the strip ends: when a later step's LDS
  // reads reused a store's data registers, the compiler made them wait for the whole store.
  float wk[kFsMaxNB][4];
  // T of this head as a buffer (C x C elements) and this lane's offset in a stored tile: row
  // 4q + p, columns 4a .. 4a + 3 (lane 16 q + 4 a + p)
  const size_t esz = U16 ? 2 : 4;
  const __amdgpu_buffer_rsrc_t tr = __builtin_amdgcn_make_buffer_rsrc(
      static_cast<uint8_t *>(g.T) + hbase * esz, 0, static_cast<int>(static_cast<size_t>(g.C) * g.C * esz), 0x00020000);
  const uint32_t lane_off = static_cast<uint32_t>(((4 * q + (lane & 3)) * g.C + (r16 & 12)) * esz);
  {
    const float *tf = dstage + j * kAtBlk;  // T_jj in fp32, row-major
    const v4f xj = {tf[16 * (4 * q) + r16], tf[16 * (4 * q + 1) + r16], tf[16 * (4 * q + 2) + r16], tf[16 * (4 * q + 3) + r16]};
    store_tile_rows<U16>(g, tr, lane_off, 16 * j, 16 * j, lane, xj, wk[0]);
  }
  xs[0] = unpack4(Td[j][4 * q][fs_col(4 * q, r16)], Td[j][4 * q + 1][fs_col(4 * q + 1, r16)],
                  Td[j][4 * q + 2][fs_col(4 * q + 2, r16)], Td[j][4 * q + 3][fs_col(4 * q + 3, r16)]);
  const int steps = NB - 1 - j;
  const int qs = fs_col(r16, 4 * q);  // this lane's quarter in its row of a block
  // A step's operands (the operand records of its A blocks and its T_bb) are read during the step
  // before: the reads of a step issued at its start left one LDS round trip per few products on
  // the strip's critical path.  Reads for a step past the last one fetch block 0 (never used).
  uint4 rc[kFsMaxNB];
  uint4 tc;
  {
    const bool any = steps > 0;
    rc[0] = *reinterpret_cast<const uint4 *>(&Al[any ? (j + 1) * j / 2 + j : 0][r16][qs]);
    tc = *reinterpret_cast<const uint4 *>(&Td[any ? j + 1 : 0][r16][qs]);
  }
#pragma unroll
  for (int v = 1; v < kFsMaxNB; ++v) {
    if (v > steps) continue;  // uniform (a break would stop the unrolling)
    const int b = j + v;
    const bool more = v < steps;
    const int nbase = more ? (b + 1) * b / 2 + j : 0;  // the next step's row of A blocks
    const int nstep = more ? 1 : 0;
    uint4 rn[kFsMaxNB];
    // Y = sum_{u < v} A_{b, j+u} X_{j+u} over pairs (u, u + 1); products go to kAcc accumulators
    // in turn (with SPLIT one per product kind), so consecutive products do not wait for each other
    constexpr int kAcc = SPLIT ? 3 : 2;
    v4f acc[kAcc];
#pragma unroll
    for (int i = 0; i < kAcc; ++i) acc[i] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < v; u += 2) {
      const Half4 a0 = {rc[u].x, rc[u].y, rc[u].z, rc[u].w};
      const Half4 a1 = u + 1 < v ? Half4{rc[u + 1].x, rc[u + 1].y, rc[u + 1].z, rc[u + 1].w} : kZero4;
      rn[u] = *reinterpret_cast<const uint4 *>(&Al[nbase + nstep * u][r16][qs]);
      rn[u + 1] = *reinterpret_cast<const uint4 *>(&Al[nbase + nstep * (u + 1)][r16][qs]);
      const Half4 &b0 = xs[u], &b1 = u + 1 < v ? xs[u + 1] : kZero4;
      constexpr int kPer = SPLIT ? 3 : 1;
      const int s0 = (u / 2) * kPer;  // compile-time: the loop is unrolled
      acc[s0 % kAcc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(op_hi(a0, a1), op_hi(b0, b1), acc[s0 % kAcc], 0, 0, 0);
      if (SPLIT) {
        acc[(s0 + 1) % kAcc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(op_hi(a0, a1), op_lo(b0, b1), acc[(s0 + 1) % kAcc], 0, 0, 0);
        acc[(s0 + 2) % kAcc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(op_lo(a0, a1), op_hi(b0, b1), acc[(s0 + 2) % kAcc], 0, 0, 0);
      }
    }
    if ((v & 1) == 0) rn[v] = *reinterpret_cast<const uint4 *>(&Al[nbase + nstep * v][r16][qs]);
    v4f y = acc[0];
#pragma unroll
    for (int i = 1; i < kAcc; ++i) y += acc[i];
    // X_b = T_bb Y: T_bb as the A operand (row r16, columns 4q .. 4q + 3), Y as the B operand;
    // the split products into separate accumulators as well
    const Half4 tb = unpack4(tc);
    tc = *reinterpret_cast<const uint4 *>(&Td[more ? b + 1 : 0][r16][qs]);
    const Half4 ys = split4<SPLIT>(y);
    const v4f z = {0.f, 0.f, 0.f, 0.f};
    v4f x = __builtin_amdgcn_mfma_f32_16x16x32_bf16(op_hi(tb, kZero4), op_hi(ys, kZero4), z, 0, 0, 0);
    if (SPLIT) {
      const v4f x1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(op_hi(tb, kZero4), op_lo(ys, kZero4), z, 0, 0, 0);
      const v4f x2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(op_lo(tb, kZero4), op_hi(ys, kZero4), z, 0, 0, 0);
      x += x1 + x2;
    }
    store_tile_rows<U16>(g, tr, lane_off, 16 * b, 16 * j, lane, x, wk[v]);
    xs[v] = split4<SPLIT>(x);
#pragma unroll
    for (int u = 0; u <= v; ++u) rc[u] = rn[u];
  }
#pragma unroll
  for (int v = 0; v < kFsMaxNB; ++v)
    if (v <= steps) asm volatile("" ::"v"(wk[v][0]), "v"(wk[v][1]), "v"(wk[v][2]), "v"(wk[v][3]));
}

template <bool U16, bool SPLIT>
__global__ __launch_bounds__(kRdThreads) void gdn_fs_kernel(GdnArgs g) {
  // A's strictly lower blocks (b, c), block index b (b - 1) / 2 + c.  Row r16 of a block is 16
  // words: per 4-column quarter, the operand record of the lane that reads it (bf16 hi parts of
  // the 4 values as two pairs, then the lo parts), so an A operand is one 16-byte read with no
  // unpacking, and a block's reads are one contiguous KiB
  __shared__ __attribute__((aligned(16))) uint32_t Al[kFsLowBlocks][16][16];
  __shared__ __attribute__((aligned(16))) uint32_t Td[kFsMaxNB][16][kFsTd];  // T_bb, hi | lo
  __shared__ __attribute__((aligned(16))) float dstage[kFsMaxNB * kAtBlk];   // A_bb^T for level 0
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);  // scalar: strip choices branch on it
  const int k8 = blockIdx.x >> 3;
  const int head = (blockIdx.x & 7) + 8 * (k8 / g.groups), part = k8 % g.groups;
  if (head >= g.heads) return;  // uniform: the whole workgroup leaves before any barrier
  const size_t hbase = static_cast<size_t>(head) * g.C * g.C;
  const int C = g.C, NB = C / 16;

  // ---- A reads: the diagonal blocks (level 0) first, then the strictly lower blocks -------------
  float4 dv[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {  // block wave + 8 u, row (t / 4) % 16, quarter t % 4
    const int bb = wave + 8 * u, i = (lane >> 2) & 15, k4 = lane & 3;
    dv[u] = load_a4_or0<U16>(g, hbase, 16 * bb + i, 16 * bb + 4 * k4, bb < NB);
  }
  __builtin_amdgcn_sched_barrier(0);  // level 0's reads first: its wait then covers only them
  // lower block slot s = t + 512 u (u < 15): block s / 64 in row-major (b, c) order, row
  // (s / 4) % 16, quarter s % 4
  constexpr int kLowLoads = kFsLowBlocks * 64 / kRdThreads;
  static_assert(kFsLowBlocks * 64 % kRdThreads == 0, "whole lower-block loads per thread");
  const int nlow = NB * (NB - 1) / 2;
  float4 lv[kLowLoads];
#pragma unroll
  for (int u = 0; u < kLowLoads; ++u) {
    const int s = t + kRdThreads * u, blk = s >> 6;
    // block index -> (b, c): b is the largest with b (b - 1) / 2 <= blk
    int b = 1;
#pragma unroll
    for (int bb = 2; bb < kFsMaxNB; ++bb) b = (bb * (bb - 1) / 2 <= blk) ? bb : b;
    const int c = blk - b * (b - 1) / 2;
    lv[u] = load_a4_or0<U16>(g, hbase, 16 * b + ((s >> 2) & 15), 16 * c + 4 * (s & 3), blk < nlow);
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- level 0 --------------------------------------------------------------------------------
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int bb = wave + 8 * u, i = (lane >> 2) & 15, k4 = lane & 3;
    if (bb < NB) stage_at(dstage, bb, i, k4, dv[u]);
  }
  lds_barrier();
  fs_level0<SPLIT>(Td, dstage, NB, t);
#pragma unroll
  for (int u = 0; u < kLowLoads; ++u) {
    const int s = t + kRdThreads * u, blk = s >> 6;
    if (blk < nlow) {
      // the operand record of lane (row, quarter): hi pairs then lo pairs, read as one Half4
      const Half4 h = split4<SPLIT>(lv[u]);
      *reinterpret_cast<uint4 *>(&Al[blk][(s >> 2) & 15][fs_col((s >> 2) & 15, 4 * (s & 3))]) =
          make_uint4(h.h01, h.h23, h.l01, h.l23);
    }
  }
  lds_barrier();

  // ---- the wave's strip ---------------------------------------------------------------------------
  const int j = __builtin_amdgcn_readfirstlane(fs_strip(NB, part, wave));
  if (j >= 0) fs_strip_solve<U16, SPLIT>(g, hbase, Al, Td, dstage, NB, j, lane);
  // Zeros above the diagonal blocks, after the strips and by waves 4..7 (the shorter strips):
  // issued before the strips they held the longest strip back by about a microsecond
  if (wave >= 4) {
    for (int row = part + (wave - 4) * g.groups; row < C; row += 4 * g.groups) {
      const int c = 4 * lane;
      if (c < C && c >= 16 * (row / 16) + 16) {
        const size_t idx = hbase + static_cast<size_t>(row) * C + c;
        if (U16) {
          const uint32_t zc = static_cast<uint32_t>(g.zpT) * 0x10001u;  // code of 0.0: clip(zpT)
          *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(g.T) + idx) = make_uint2(zc, zc);
        } else {
          *reinterpret_cast<float4 *>(static_cast<float *>(g.T) + idx) = make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
    }
  }
}

// G = 2 workgroups per head for more than 8 strips, one otherwise.
GdnArgs make_args(const void *A, void *T, int heads, int C, int zpA, int zpT, float sA, float sT) {
  return GdnArgs{A, T, C, C / 16 > 8 ? 2 : 1, heads, zpA, zpT, sA, sT, 1.0f / sT};
}

template <bool U16, bool SPLIT>
qh_status launch_fs(const GdnArgs &g, int heads, hipStream_t stream) {
  const long long blocks = static_cast<long long>((heads + 7) / 8) * 8 * g.groups;
  if (blocks > 0x7FFFFFFFLL) return fail(QH_STATUS_SHAPE_UNSUPPORTED, "gdn: %d heads exceed one launch", heads);
  hipLaunchKernelGGL((gdn_fs_kernel<U16, SPLIT>), dim3(static_cast<unsigned>(blocks)), dim3(kRdThreads), 0, stream, g);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return hip_fail(err, "gdn_fs_kernel launch");
  return QH_STATUS_OK;
}

}  // namespace

qh_status launch_gdn_solve_f32(const float *A, float *T, int heads, int C, int precision, hipStream_t stream) {
  const GdnArgs g = make_args(A, T, heads, C, 0, 0, 1.0f, 1.0f);
  return precision == QH_GDN_BF16 ? launch_fs<false, false>(g, heads, stream) : launch_fs<false, true>(g, heads, stream);
}

qh_status launch_gdn_solve_u16(const uint16_t *A, uint16_t *T, int heads, int C, int zpA, int zpT, float sA, float sT,
                               int precision, hipStream_t stream) {
  const GdnArgs g = make_args(A, T, heads, C, zpA, zpT, sA, sT);
  return precision == QH_GDN_BF16 ? launch_fs<true, false>(g, heads, stream) : launch_fs<true, true>(g, heads, stream);
}

}  // namespace qh
