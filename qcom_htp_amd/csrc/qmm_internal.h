// Internal definitions shared by the quantized-matmul kernels and the host-side prepare.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qhtp.h"

namespace qh {

// GEMM workgroup tile in the i8 operand space: BM rows of the activation operand,
// BN columns of the weight operand, BK bytes of K per pipeline stage.
constexpr int kBM = 128;
constexpr int kBN = 512;
constexpr int kBK = 128;
constexpr int kGemmThreads = 512;
// Capacity of the per-workgroup list of outputs that need the exact fp64 fixup.
constexpr int kFixCap = 1024;

// Tile storage of the GEMM weight operand (the "B" operand of the MFMA): int8 integer weights
// (int4 codes and LPBQ code * block scale widened at prepare time).  A tile (nt, kt) covers 256
// operand columns x 128 k (32 KiB) in MFMA fragment order: the 16 bytes of column c, depth
// k .. k + 15 (k % 16 == 0) are lane 32 h + (c & 31) of the v_mfma_i32_32x32x32_i8 B fragment of
// 32-k step s and 32-column block cb, with s = (k & 127) >> 5, h = (k >> 4) & 1, cb = c >> 5, and
// the 64 lanes of one fragment are 1 KiB in a row, fragment (s, cb) at 1 KiB * (kBN / 32 * s + cb).
// A wave loads a whole fragment with one coalesced 16-byte-per-lane load straight into registers.
// Element format of the decode GEMV stream: int8 codes, or int4 codes (two per byte).
enum TileFormat : int { kTileI8 = 0, kTileI4 = 1 };

// XOR swizzles that make the activation fragment reads from LDS bank-conflict free (32
// consecutive rows reading the same logical chunk hit distinct banks for 8- or 16-lane LDS phases).
__host__ __device__ inline int swz8(int row) { return ((row >> 1) ^ (row << 2)) & 7; }
__host__ __device__ inline int swz16(int row) { return row & 15; }

// Byte offset of (operand column c, depth k) inside its tile (fragment order, see above).
__host__ __device__ inline int tile_off_i8(int c, int k) {
  return (((((k & 127) >> 5) * (kBN / 32) + (c >> 5)) * 64 + ((k >> 4) & 1) * 32 + (c & 31)) << 4) + (k & 15);
}

// GEMV k-split: the 4 waves x 4 lanes of a workgroup that share a column take its 32-k groups
// in batches of kGemvKU per lane; lane (wave w, sub s) takes kg = 16 i + 4 w + s in slot i of
// the batch, so one batch covers kGemvBatchKG k-groups.
constexpr int kGemvKU = 8;
constexpr int kGemvBatchKG = 16 * kGemvKU;

// LPBQ block scales of the GEMV stream, laid out so that a lane reads the kGemvKU scales of
// its batch slots with one 8-byte load:
//   [N/16 groups][batches][4 waves][4 >> sub_shift][16 columns][kGemvKU slots],
// sub_shift = log2(block / 32): the lanes whose k-groups fall in one block share its scales.
__host__ __device__ inline size_t gemv_scale_index(int grp, int batch, int nbatch, int wave, int subq, int nsubq,
                                                   int col, int slot) {
  return ((((static_cast<size_t>(grp) * nbatch + batch) * 4 + wave) * nsubq + subq) * 16 + col) * kGemvKU + slot;
}
__host__ __device__ inline size_t gemv_scale_index_kg(int n, int kg, int nbatch, int sub_shift) {
  const int j = kg % kGemvBatchKG;
  return gemv_scale_index(n / 16, kg / kGemvBatchKG, nbatch, (j >> 2) & 3, (j & 3) >> sub_shift, 4 >> sub_shift,
                          n % 16, j >> 4);
}

// Per-output-channel epilogue record of the int4 decode GEMV (qmm_gemv_unit.hip): everything its
// requantisation and exact fixup read about a column, 96 bytes (six 16-byte pieces).
struct GemvRec {
  double alpha, beta, margin, absb;  // as QmmDevice
  int64_t corr;                      // 8-bit acts: corr; 16-bit acts: colsum (sum_k w_int)
  double mlo;                        // 16-bit acts: margin_lo; 8-bit acts: residue bound per unit of |a - zp|_2
  int64_t mant, colsum_r;            // M of s32 = M 2^E; sum_k r_k
  double bias_deq;
  double alpha_e, margin_exact;      // as QmmDevice
  float s32;
  int32_t pad;
};
static_assert(sizeof(GemvRec) == 96, "GemvRec is six 16-byte pieces");

// Everything the GEMM / GEMV kernels read, resident on the device.
struct QmmDevice {
  // Weight operand tiles (GEMM).  For 16-bit activations the operand has 2N columns:
  // inside each 64-column group, columns [0,32) carry the weight codes of 32 output
  // channels and columns [32,64) the fl32 rounding residues of the same channels.
  uint8_t *tiles;
  // GEMV stream: [N/16 column groups][K/32 k-groups][16 columns][16 B int4 | 32 B int8]
  // (int4 byte j: k = j in the low nibble, k = j + 16 in the high nibble, offset-binary).
  uint8_t *gemv_tiles;
  uint8_t *gemv_lpbq;   // LPBQ block scales for the GEMV stream (gemv_scale_index layout)
  uint8_t *lpbq_nk;     // LPBQ block scales in the descriptor's [N][K / block] order (int4 GEMV)
  GemvRec *gemv_rec;    // [N] (int4 weights)
  // Per output channel epilogue constants.
  double *alpha;    // t = fma(S, alpha, beta): S is the exact integer dot product
  double *beta;     //   (alpha = sA * s32 / sO for 8-bit acts, sA * 2^E / sO for 16-bit)
  int64_t *corr;    // 8-bit acts: (128 - act_zp) * sum_k w_int ; 16-bit: exact constant term
  double *margin;   // rounding-decision margin in output LSB (excluding the |t| term)
  double *absb;     // |beta| + out_zp + 1 (scale of the float slack term)
  double *bias_deq; // bias_q * fl64(sA * s32) exactly as the oracle forms it
  float *s32;       // per-channel weight scale
  int64_t *mant;    // 16-bit acts: 24-bit mantissa M of s32 (s32 = M * 2^E)
  int64_t *colsum;  // sum_k w_int[n][k]
  int64_t *colsum_r; // sum_k r[n][k] (float32 rounding residues of the dequantised weights)
  double *alpha_e;  // sA * 2^E / sO: output LSB per unit of the exact integer dot product in 2^E units
  int32_t *scale_exp; // E of s32 = M * 2^E
  double *margin_exact; // 8-bit acts: float64 noise bound of the oracle's dot product, output LSB
  double *gemv_margin_r1; // 16-bit acts, int8-code GEMV: coefficient of R1[m] = sum |a - zp| in the margin
  double *margin_lo;      // 16-bit acts: bound of sum_k lo'_k r_k in output LSB (the GEMM and the int4-code
                          // GEMV form the high-byte residue sum exactly)
  int8_t *resid;    // 8-bit acts: rounding residues r[n][k] (fl32(w s32) = 2^E (w M + r)), [N][K],
                    // read by the GEMM's exact fixup (|r| <= 64): one contiguous row per listed
                    // output, where the same weights in the fragment-ordered tiles are 256
                    // scattered 16-byte pieces
  int32_t *bias_q;  // [Np] the descriptor's int32 bias (integer contracts)
  int64_t *corr_int; // [Np] activation-shift term of the exact integer dot product sum (a - zp) w_int
  // Per-group weights (exact integer GEMM): multipliers of the code and residue planes per
  // (plane, group, channel) [2][G][Np], the shift term of that sum, and the float32 group scales
  int64_t *mult;
  int64_t *corr_rq;
  float *s32g;      // [N][G]
};

struct QmmShape {
  int N, K;           // logical
  int Np;             // N padded to the GEMM column tile (in output channels)
  int Kp;             // K padded to kBK
  int ncols_op;       // columns of the weight operand (N or 2N), padded to kBN
  int act_bits, out_bits;
  int wfmt;           // qh_weight_format
  int gemv_fmt;       // TileFormat of the GEMV stream
  int lpbq_block;     // 0 unless LPBQ
  int act_zp, out_zp;
  double act_scale, out_scale;
  int epi_clamp;      // GEMM epilogue must clamp t before rounding (|t| < 2^30 not proven)
  // Exact integer GEMM (qmm_exact.hip): weight planes per 32 channels in the tile layout (1, or 2
  // for 16-bit acts and the exact-only formats), the planes / multipliers / all-ones multiplier
  // of the integer dot product, and the per-group scale groups.
  int layout_planes;
  int exact_only;     // per-group / int16 weights: no GEMM / GEMV state
  int int_planes;
  long long int_mult[2];
  int int_ones;
  int groups, group_shift;
};

// Arguments of the exact integer GEMM (qmm_exact.hip).
struct ExactArgs {
  const uint8_t *act;
  void *out;
  const uint8_t *tiles;
  int KT, layout_planes;
  int M, N, K, Np;
  int nplanes, ones;
  long long cm[2];
  const int64_t *mult;
  int G, gshift;
  const int64_t *corr;
  const double *alpha_e, *beta, *margin_exact, *absb, *bias_deq;
  const float *s32g;
  double sA, sO;
  int act_zp, out_zp, out_qmax, out16;
  int contract, divisor;
  const int32_t *bias_q;
};

}  // namespace qh

struct qh_qmm_prepared {
  qh::QmmShape shape;
  qh::QmmDevice dev;
  uint64_t device_bytes;
  uint64_t gemm_weight_bytes;
  uint64_t gemv_weight_bytes;
  int device_id;
};

// Error plumbing (defined in qhtp_abi.cpp).
namespace qh {
qh_status fail(qh_status st, const char *fmt, ...);
qh_status hip_fail(hipError_t err, const char *what);

// Kernel launchers (defined in the .hip files).
qh_status launch_qmm_gemm(const qh_qmm_prepared *p, int m, const void *act, void *out, hipStream_t stream);
qh_status launch_qmm_gemv(const qh_qmm_prepared *p, int m, const void *act, void *out, hipStream_t stream);
// The persistent int4 decode GEMV for M <= 4; returns QH_STATUS_SHAPE_UNSUPPORTED (without
// launching or recording an error) for the shapes it does not take.
// Compute units of the current device (cached per device; 0 if the query fails).
int device_cu_count();
qh_status launch_qmm_gemv_unit(const qh_qmm_prepared *p, int m, const void *act, void *out, hipStream_t stream);
bool gemv_fits(const qh_qmm_prepared *p, int m);  // the GEMV's LDS staging holds M x K
qh_status launch_qmm_accumulate(const qh_qmm_prepared *p, int m, const void *act, int64_t *acc,
                                hipStream_t stream);
// mode 0: requantised output (per-group weights), 1: int64 accumulators, 2: integer contract
qh_status launch_qmm_exact(const qh_qmm_prepared *p, int m, const void *act, void *out, int mode, int contract,
                           int divisor, hipStream_t stream);
// Every step of an integer-contract chain in one launch, for K == N <= 256 (chain_fusable).
bool chain_fusable(const qh_qmm_prepared *p);
qh_status launch_qmm_chain(const qh_qmm_prepared *p, int m, int chain, const void *act, void *out, int contract,
                           int divisor, hipStream_t stream);
qh_status launch_gdn_solve_f32(const float *A, float *T, int heads, int C, int precision, hipStream_t stream);
qh_status launch_gdn_solve_u16(const uint16_t *A, uint16_t *T, int heads, int C, int zpA, int zpT, float sA,
                               float sT, int precision, hipStream_t stream);
qh_status launch_gdn_solve_op_model(const uint16_t *A, uint16_t *T, int heads, int C, int zpA, int zpT, float sA,
                                    float sT, hipStream_t stream);
qh_status launch_lpbq_expand(const uint8_t *codes, const uint8_t *scales, uint8_t *out, uint32_t K, uint32_t N,
                             hipStream_t stream);
qh_status launch_gdn_chunk_uw(const uint16_t *k, const uint16_t *v, const float *g, const float *beta, void *w,
                              void *u, int B, int T, int H, int C, int flags, int max_wg, hipStream_t stream);
qh_status launch_gdn_chunk_state(const uint16_t *q, const uint16_t *k, const float *g, const void *w, const void *u,
                                 const float *s_in, float *s_out, void *o, int B, int T, int H, int precision,
                                 bool wu_f32, bool out_f32, hipStream_t stream);
}  // namespace qh
