// Internal definitions shared by the quantized-matmul kernels and the host-side prepare.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qhtp.h"

namespace qh {

// GEMM workgroup tile in the i8 operand space: BM rows of the activation operand,
// BN columns of the weight operand, BK bytes of K per pipeline stage.
constexpr int kBM = 256;
constexpr int kBN = 256;
constexpr int kBK = 128;
constexpr int kGemmThreads = 256;
// Capacity of the per-workgroup list of outputs that need the exact fp64 fixup.
constexpr int kFixCap = 1024;

// Tile storage of the weight operand (the "B" operand of the MFMA):
//   kTileI8 : int8 bytes, tile (nt, kt) = [256 cols][128 k] contiguous (32 KiB)
//   kTileI4 : two int4 codes per byte, offset-binary (code + 8); tile = [256 cols][64 B]
//             (16 KiB); inside a column's 64 B, each 16-k group is 8 bytes whose low nibble
//             j holds k = j and high nibble holds k = j + 8.
enum TileFormat : int { kTileI8 = 0, kTileI4 = 1 };

// Everything the GEMM / GEMV kernels read, resident on the device.
struct QmmDevice {
  // Weight operand tiles (GEMM).  For 16-bit activations the operand has 2N columns:
  // inside each 64-column group, columns [0,32) carry the weight codes of 32 output
  // channels and columns [32,64) the fl32 rounding residues of the same channels.
  uint8_t *tiles;
  uint8_t *lpbq_tiles;  // [Ncols_padded][Kp / lpbq_block] uint8 block scales (I4 LPBQ GEMM)
  // GEMV stream: per 256-column panel and 128-k tile, [256][64 B] nibbles (I4 / LPBQ) or
  // [256][128 B] int8 -- the same tile layout as the GEMM for 8-bit activations.
  uint8_t *gemv_tiles;
  uint8_t *gemv_lpbq;   // [Np][Kp / lpbq_block] uint8 block scales for the GEMV stream
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
  double *gemv_margin_r1; // 16-bit acts GEMV: per-channel coefficient of R1[m] in the margin
};

struct QmmShape {
  int N, K;           // logical
  int Np;             // N padded to the GEMM column tile (in output channels)
  int Kp;             // K padded to kBK
  int ncols_op;       // columns of the weight operand (N or 2N), padded to kBN
  int act_bits, out_bits;
  int wfmt;           // qh_weight_format
  int tile_fmt;       // TileFormat of the GEMM tiles
  int gemv_fmt;       // TileFormat of the GEMV stream
  int lpbq_block;     // 0 unless LPBQ
  int act_zp, out_zp;
  double act_scale, out_scale;
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
qh_status launch_qmm_accumulate(const qh_qmm_prepared *p, int m, const void *act, int64_t *acc,
                                hipStream_t stream);
qh_status launch_gdn_solve_f32(const float *A, float *T, int heads, int C, int precision, hipStream_t stream);
qh_status launch_gdn_solve_u16(const uint16_t *A, uint16_t *T, int heads, int C, int zpA, int zpT, float sA,
                               float sT, int precision, hipStream_t stream);
}  // namespace qh
