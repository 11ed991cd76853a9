// bf16 hi / lo operand splitting for fp32-accurate products on v_mfma_f32_16x16x32_bf16.
//
// A float x is carried as hi = bf16(x) (round to nearest even) and lo = bf16(x - hi); hi + lo
// holds about 16 significant bits, and a product a * b is taken as hi*hi + hi*lo + lo*hi with
// fp32 accumulation (the lo*lo term is below fp32 resolution of the sum).
//
// Pair layout of a 32-deep k step: k indices 8q + e (e < 4) of the MFMA come from block 0,
// rows 4q + e, and 8q + 4 + e from block 1, rows 4q + e (q = lane / 16).  The MFMA result
// layout (lane: rows 4q .. 4q+3 of column lane % 16) is therefore read back directly as a B
// operand over two 16-row blocks.

#ifndef QHTP_BF16_SPLIT_H_
#define QHTP_BF16_SPLIT_H_

#include <hip/hip_runtime.h>
#include <cstdint>

namespace qh {
namespace bf16s {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

// Two floats -> packed bf16 (a in the low half), round to nearest even.
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v2f{a, b}, v2bf));
}

// x as one LDS word: bf16 hi in the low half, bf16(x - hi) in the high half (0 without SPLIT).
template <bool SPLIT>
__device__ __forceinline__ uint32_t hilo(float x) {
  const uint32_t h = pack_bf16(x, 0.0f) & 0xFFFFu;
  if (!SPLIT) return h;
  return h | (pack_bf16(x - __uint_as_float(h << 16), 0.0f) << 16);
}

// 4 operand values (4 k of one MFMA row / column): bf16 hi parts and lo parts, two per dword.
struct Half4 {
  uint32_t h01, h23, l01, l23;
};
constexpr Half4 kZero4 = {0u, 0u, 0u, 0u};

// ... from 4 hilo words
__device__ __forceinline__ Half4 unpack4(uint32_t d0, uint32_t d1, uint32_t d2, uint32_t d3) {
  return {__builtin_amdgcn_perm(d1, d0, 0x05040100u), __builtin_amdgcn_perm(d3, d2, 0x05040100u),
          __builtin_amdgcn_perm(d1, d0, 0x07060302u), __builtin_amdgcn_perm(d3, d2, 0x07060302u)};
}
__device__ __forceinline__ Half4 unpack4(const uint4 w) { return unpack4(w.x, w.y, w.z, w.w); }

// ... from 4 floats
template <bool SPLIT>
__device__ __forceinline__ Half4 split4(float x, float y, float z, float w) {
  const uint32_t h01 = pack_bf16(x, y), h23 = pack_bf16(z, w);
  if (!SPLIT) return {h01, h23, 0u, 0u};
  const uint32_t l01 = pack_bf16(x - __uint_as_float(h01 << 16), y - __uint_as_float(h01 & 0xFFFF0000u));
  const uint32_t l23 = pack_bf16(z - __uint_as_float(h23 << 16), w - __uint_as_float(h23 & 0xFFFF0000u));
  return {h01, h23, l01, l23};
}
template <bool SPLIT>
__device__ __forceinline__ Half4 split4(const float4 f) {
  return split4<SPLIT>(f.x, f.y, f.z, f.w);
}
template <bool SPLIT>
__device__ __forceinline__ Half4 split4(const v4f f) {
  return split4<SPLIT>(f[0], f[1], f[2], f[3]);
}

__device__ __forceinline__ v8bf op_hi(const Half4 &a, const Half4 &b) {
  return __builtin_bit_cast(v8bf, make_uint4(a.h01, a.h23, b.h01, b.h23));
}
__device__ __forceinline__ v8bf op_lo(const Half4 &a, const Half4 &b) {
  return __builtin_bit_cast(v8bf, make_uint4(a.l01, a.l23, b.l01, b.l23));
}

// acc += A B for one 32-deep pair step (k blocks a0/b0, then a1/b1); with SPLIT the hi*lo and
// lo*hi products are added.
template <bool SPLIT>
__device__ __forceinline__ v4f mma(const Half4 &a0, const Half4 &a1, const Half4 &b0, const Half4 &b1, v4f acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(op_hi(a0, a1), op_hi(b0, b1), acc, 0, 0, 0);
  if (SPLIT) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(op_hi(a0, a1), op_lo(b0, b1), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(op_lo(a0, a1), op_hi(b0, b1), acc, 0, 0, 0);
  }
  return acc;
}

// acc += A B when A is exact in bf16 (lo parts zero): hi*hi, and with SPLIT hi*lo of B.
template <bool SPLIT>
__device__ __forceinline__ v4f mma_exact_a(const Half4 &a0, const Half4 &a1, const Half4 &b0, const Half4 &b1,
                                           v4f acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(op_hi(a0, a1), op_hi(b0, b1), acc, 0, 0, 0);
  if (SPLIT) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(op_hi(a0, a1), op_lo(b0, b1), acc, 0, 0, 0);
  return acc;
}

// Four bf16 bit patterns as the hi half of an operand (lo zero).
__device__ __forceinline__ Half4 exact4(uint32_t h01, uint32_t h23) { return {h01, h23, 0u, 0u}; }

}  // namespace bf16s
}  // namespace qh

#endif  // QHTP_BF16_SPLIT_H_
