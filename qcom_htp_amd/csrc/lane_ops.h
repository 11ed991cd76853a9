// Cross-lane sums on DPP (data moved between lanes by the VALU, no LDS round trip), shared by the
// GDN kernels.

#ifndef QHTP_LANE_OPS_H_
#define QHTP_LANE_OPS_H_

#include "qmm_internal.h"

namespace qh {
namespace {

// Lane move within a wave by DPP (CTRL: quad_perm 0x00-0xFF, row_shr:n 0x110+n, row_half_mirror
// 0x141, row_bcast:15 0x142, row_bcast:31 0x143); lanes without a source, and rows outside
// ROW_MASK, read 0.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xF, false));
}

// Sum over the 8 lanes 8r .. 8r+7: xor 1, xor 2 inside quads, then the mirrored quad (the same
// additions, in the same order, as a butterfly over xor 1, 2, 4).
__device__ __forceinline__ float sum8(float x) {
  x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp<0x141>(x);  // row_half_mirror
  return x;
}

// Inclusive prefix sum over the 64 lanes: within rows of 16 by shifts 1, 2, 4, 8, then row 0's
// total into row 1 and row 2's into row 3, then the first 32 lanes' total into rows 2 and 3.
__device__ __forceinline__ float scan64(float x) {
  x += dpp<0x111>(x);
  x += dpp<0x112>(x);
  x += dpp<0x114>(x);
  x += dpp<0x118>(x);
  x += dpp<0x142, 0xA>(x);
  x += dpp<0x143, 0xC>(x);
  return x;
}

}  // namespace
}  // namespace qh

#endif  // QHTP_LANE_OPS_H_
