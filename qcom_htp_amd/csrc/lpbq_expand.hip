// LPBQ expand on the device: int4 K-pair codes x per-(channel, 32-k block) integer scale ->
// saturated int8 in the 32x32 K-major tile stream (the reference op HmxW4LpbqExpandToI8,
// example/qnn_hmx_matmul_common/HmxW4LpbqExpandToI8Op.cpp:47-104).
//
// Byte work, HBM bound: K*N/2 bytes of codes and N*K/32 bytes of scales in, K*N bytes out.
// One thread writes 16 output bytes: in tile (kt, nt), the 4 k of row quad rq and the
// 4 channels of column quad cq, i.e. bytes rq*128 + cq*16 .. +15 (channel-major, 4 k each).
// Those 16 codes come from two 4-byte loads (input rows k/2 and k/2+1, 4 adjacent channels).
// 64 consecutive threads write one 1024-byte tile contiguously.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qmm_internal.h"

namespace qh {
namespace {

__device__ __forceinline__ int int4_twos(uint32_t nib) { return static_cast<int>(nib & 15u) - ((nib & 8u) << 1); }

__device__ __forceinline__ uint32_t sat_i8_byte(int v) {
  v = v < -128 ? -128 : (v > 127 ? 127 : v);
  return static_cast<uint32_t>(v) & 0xffu;
}

__global__ __launch_bounds__(256) void lpbq_expand_kernel(const uint8_t *__restrict__ codes,
                                                          const uint8_t *__restrict__ scales,
                                                          uint8_t *__restrict__ out, uint32_t K, uint32_t N,
                                                          uint64_t total) {
  const uint64_t t = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= total) return;
  const uint32_t NT = N / 32, KT = K / 32;
  const uint32_t cq = static_cast<uint32_t>(t & 7), rq = static_cast<uint32_t>((t >> 3) & 7);
  const uint64_t tile = t >> 6;
  const uint32_t nt = static_cast<uint32_t>(tile % NT), kt = static_cast<uint32_t>(tile / NT);
  const uint32_t n0 = nt * 32 + cq * 4;
  const uint64_t row = static_cast<uint64_t>(kt) * 16 + rq * 2;  // input row of k = 32 kt + 4 rq (and +1)
  const uint32_t a = *reinterpret_cast<const uint32_t *>(codes + row * N + n0);        // k, k+1
  const uint32_t b = *reinterpret_cast<const uint32_t *>(codes + (row + 1) * N + n0);  // k+2, k+3
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int s = scales[static_cast<uint64_t>(n0 + i) * KT + kt];
    const uint32_t ba = (a >> (8 * i)) & 0xffu, bb = (b >> (8 * i)) & 0xffu;
    w[i] = sat_i8_byte(int4_twos(ba) * s) | (sat_i8_byte(int4_twos(ba >> 4) * s) << 8) |
           (sat_i8_byte(int4_twos(bb) * s) << 16) | (sat_i8_byte(int4_twos(bb >> 4) * s) << 24);
  }
  uint4 v;
  v.x = w[0];
  v.y = w[1];
  v.z = w[2];
  v.w = w[3];
  *reinterpret_cast<uint4 *>(out + tile * 1024 + rq * 128 + cq * 16) = v;
}

}  // namespace

qh_status launch_lpbq_expand(const uint8_t *codes, const uint8_t *scales, uint8_t *out, uint32_t K, uint32_t N,
                             hipStream_t stream) {
  const uint64_t total = static_cast<uint64_t>(K) * N / 16;
  const uint64_t blocks = (total + 255) / 256;
  hipLaunchKernelGGL(lpbq_expand_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, stream, codes, scales, out,
                     K, N, total);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return hip_fail(err, "qh_w4_lpbq_expand_to_i8 launch");
  return QH_STATUS_OK;
}

}  // namespace qh
