// Device helpers shared by the decode GEMV kernels (qmm_gemv.hip, qmm_gemv_unit.hip): int4 code
// widening, the per-(column, block scale) float32 rounding-residue tables of 16-bit
// activations, dot products and LDS-only barriers.

#ifndef QHTP_GEMV_COMMON_H_
#define QHTP_GEMV_COMMON_H_

#include "qmm_internal.h"

namespace qh {
namespace {

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef unsigned int v2u __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));

typedef unsigned short us2 __attribute__((ext_vector_type(2)));

// int8 weight bytes of 4 int4 codes: nibbles u (offset-binary, code = u - 8) times the LPBQ block
// scale f, as (u * f + 128 - 8 f) ^ 0x80 per byte.  u * f <= 240 and 128 - 8 f >= 0 keep every
// byte of the product and the sum below 256 (no carries between bytes); f = 0 gives zero weights.
// The multiply-add runs on the two 16-bit halves (one packed v_pk_mad_u16 at the full rate; a
// 32-bit integer multiply issues at a quarter of it): each half holds two bytes, and no byte
// carries, so no half overflows.
__device__ __forceinline__ uint32_t w4_to_i8(uint32_t u4, uint32_t f) {
  const unsigned short fs = static_cast<unsigned short>(f);
  const unsigned short cs = static_cast<unsigned short>((128u - 8u * f) * 0x0101u);
  const us2 r = __builtin_bit_cast(us2, u4) * us2{fs, fs} + us2{cs, cs};
  return __builtin_bit_cast(uint32_t, r) ^ 0x80808080u;
}

// 16-bit activations, int4 codes: the float32 rounding residue r = fl32(w s32) / 2^E - w M of a
// weight w = (u - 8) f depends only on the code u and the block scale f (s32 = M 2^E).  A table
// per (column, f) holds R(j f) for j = 0..7 (bytes 0-7, codes u >= 8: index u - 8) and
// R((u - 8) f) for u = 0..7 (bytes 8-15, codes u < 8: index u); four codes are looked up with
// two byte permutes and a per-byte select on the code's bit 3.
__device__ __forceinline__ uint32_t resid4(uint32_t nb, const uint4 &tab) {
  const uint32_t sel = nb & 0x07070707u;
  const uint32_t pos = perm(tab.y, tab.x, sel);
  const uint32_t neg = perm(tab.w, tab.z, sel);
  // 0xFF in the bytes whose code has bit 3 set: with y = nb << 4 that bit is each byte's sign
  // bit, and permute selectors 8..11 replicate the sign bits of bytes 1 and 3 of either source
  // (bytes of y << 8 and of y), in the byte order 0, 1, 2, 3
  const uint32_t y = nb << 4;
  const uint32_t m = perm(y, y << 8, 0x0B090A08u);
  return (pos & m) | (neg & ~m);
}

// Residue tables per column: one for each block scale f = 0 .. 16 (the LPBQ factor range; f = 0
// serves the slots past K, whose codes are zero).
constexpr int kRtabF = 17;

// The residue table of (column n, block scale f): R(x) = fl32(x) - x for x = w M, computed as
// the float32 conversion of the exact integer product (|x| < 2^31: |w| <= 112, M < 2^24), which
// rounds like the float32 product w * s32 of the oracle.
__device__ __forceinline__ uint4 resid_table(int Mn, int f) {
  uint32_t b[16];
  const int F = f * Mn;
  b[0] = 0u;
  b[8] = 0u;  // code 0 (q = -8) never occurs
#pragma unroll
  for (int j = 1; j < 8; ++j) {
    const int x = j * F;
    const int r = static_cast<int>(static_cast<float>(x)) - x;  // |r| <= 64
    b[j] = static_cast<uint32_t>(r) & 0xFFu;
    b[16 - j] = static_cast<uint32_t>(-r) & 0xFFu;  // R(-j f) = -R(j f), code u = 8 - j
  }
  return make_uint4(b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24), b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24),
                    b[8] | (b[9] << 8) | (b[10] << 16) | (b[11] << 24),
                    b[12] | (b[13] << 8) | (b[14] << 16) | (b[15] << 24));
}

// Workgroup barrier for data exchanged through LDS: waits for this wave's LDS operations
// only.  __syncthreads() would also wait for every global load in flight (its release fence),
// which would hold the staging and the reductions behind the weight stream.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Streaming load that bypasses cache retention (the weights are read once per call).
__device__ __forceinline__ uint4 load_stream(const uint8_t *p) {
  const v4u x = __builtin_nontemporal_load(reinterpret_cast<const v4u *>(p));
  return make_uint4(x.x, x.y, x.z, x.w);
}

// Buffer loads: an offset at or past `bytes` returns zero without a memory access (and a
// resource of 0 bytes turns every load of it into such a load, still counted like the others).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, static_cast<int>(bytes), 0x00020000);
}
template <int AUX = 0>
__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const v4u v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 bload8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const v2u v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
  return make_uint2(v.x, v.y);
}
constexpr int kNT = 2;  // buffer-load cache policy: nontemporal (the weights are read once per call)

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}

// sum of the four signed bytes of x
__device__ __forceinline__ int bsum4(uint32_t x, int c) { return sdot4(x, 0x01010101u, c); }

}  // namespace
}  // namespace qh

#endif  // QHTP_GEMV_COMMON_H_
