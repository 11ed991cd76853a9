// Host-side decoding of the reference's packed weight carriers into logical int8 codes.
//
// Each carrier is a permutation of the logical [K, N] codes (W8: one byte per code; W4: two
// codes per byte).  `locate` gives, for one logical (k, n), the byte that holds it and whether
// it is the first element of that byte's pair; the loop then decodes it.  The layouts are
// those the reference's generator writes (example/qnn_hmx_matmul_common/gen_quant_chain.py)
// and its op packages read; each case below names its lines.
#include <stdint.h>
#include <string.h>

#include "qmm_internal.h"

namespace {

struct Where {
  size_t byte;
  bool first;  // W4: first element of the byte's pair (low nibble in the "lohi" orders)
};

struct Carrier {
  uint32_t id;
  uint64_t K, N;

  Where locate(uint64_t k, uint64_t n) const {
    switch (id) {
      case QH_CARRIER_I8_KN:  // gen_quant_chain.py:729-738
      case QH_CARRIER_W4_FULL_CODES:  // :619-627
        return {k * N + n, true};
      case QH_CARRIER_W8_KMAJOR:  // :285-303; HmxW4LpbqExpandToI8Op.cpp:84-101
        return {((k / 32) * (N / 32) + n / 32) * 1024 + ((k & 31) / 4) * 128 + (n & 31) * 4 + (k & 3), true};
      case QH_CARRIER_W8_KMAJOR_SPLIT128: {  // :306-314, a W8_KMAJOR stream of N = 128 per slice
        const uint64_t g = n / 128, c = n & 127;
        return {g * K * 128 + ((k / 32) * 4 + c / 32) * 1024 + ((k & 31) / 4) * 128 + (c & 31) * 4 + (k & 3), true};
      }
      case QH_CARRIER_W4_KMAJOR_N64:  // :680-714; HmxU8I4ToU8MatMulOp.cpp:184-201
        return {((k / 32) * (N / 64) + n / 64) * 1024 + ((k & 31) / 4) * 128 + (n & 31) * 4 + (k & 3), (n & 63) < 32};
      case QH_CARRIER_W4_KPAIR:  // :369-382; HmxW4LpbqExpandToI8Op.cpp:35-41
        return {(k / 2) * N + n, (k & 1) == 0};
      case QH_CARRIER_W4_NMAJOR_KPAIR:  // :385-398
        return {n * (K / 2) + k / 2, (k & 1) == 0};
      case QH_CARRIER_W4_NMAJOR_K4:  // :401-422
        return {(((n / 32) * (K / 8) + k / 8) * 32 + (n & 31)) * 4 + (k & 3), (k & 7) < 4};
      case QH_CARRIER_W4_KBLOCK32_NMAJOR_K4:  // :425-452; HmxU16I4ToU16MatMulOp.cpp:526-543
        return {((((k / 32) * (N / 32) + n / 32) * 4 + (k & 31) / 8) * 32 + (n & 31)) * 4 + (k & 3), (k & 7) < 4};
      case QH_CARRIER_W4_NPAIR_NMAJOR:  // :455-468
        return {(n / 2) * K + k, (n & 1) == 0};
      case QH_CARRIER_W4_NPAIR_TILE32_NMAJOR:  // :471-489
        return {((n / 64) * 32 + (n & 31)) * K + k, (n & 63) < 32};
    }
    return {0, true};
  }
};

bool is_w4(uint32_t c) { return c >= QH_CARRIER_W4_KMAJOR_N64; }

// Shape rules of the generator's packers; returns nullptr when the shape is accepted.
const char *shape_rule(uint32_t c, uint64_t K, uint64_t N) {
  switch (c) {
    case QH_CARRIER_I8_KN:
    case QH_CARRIER_W4_FULL_CODES:
      return nullptr;
    case QH_CARRIER_W8_KMAJOR:
    case QH_CARRIER_W4_KBLOCK32_NMAJOR_K4:
      return (K % 32 || N % 32) ? "K and N multiples of 32" : nullptr;
    case QH_CARRIER_W8_KMAJOR_SPLIT128:
      return (K % 32 || N % 128) ? "K multiple of 32, N multiple of 128" : nullptr;
    case QH_CARRIER_W4_KMAJOR_N64:
      return (K % 32 || N % 64) ? "K multiple of 32, N multiple of 64" : nullptr;
    case QH_CARRIER_W4_KPAIR:
    case QH_CARRIER_W4_NMAJOR_KPAIR:
      return (K % 2) ? "even K" : nullptr;
    case QH_CARRIER_W4_NMAJOR_K4:
      return (K % 8 || N % 32) ? "K multiple of 8, N multiple of 32" : nullptr;
    case QH_CARRIER_W4_NPAIR_NMAJOR:
      return (N % 2) ? "even N" : nullptr;
    case QH_CARRIER_W4_NPAIR_TILE32_NMAJOR:
      return (N % 64) ? "N multiple of 64" : nullptr;
  }
  return "a known carrier";
}

}  // namespace

extern "C" qh_status qh_weight_unpack(uint32_t carrier, uint32_t flags, const uint8_t *packed, size_t packed_bytes,
                                      uint32_t k, uint32_t n, int8_t *weight_nk) {
  using qh::fail;
  if (packed == nullptr || weight_nk == nullptr) return fail(QH_STATUS_INVALID_ARGUMENT, "qh_weight_unpack: NULL buffer");
  if (carrier > QH_CARRIER_W4_FULL_CODES) return fail(QH_STATUS_UNSUPPORTED, "qh_weight_unpack: unknown carrier %u", carrier);
  const uint32_t known = QH_CARRIER_XOR80 | QH_CARRIER_HILO | QH_CARRIER_BIASED;
  if (flags & ~known) return fail(QH_STATUS_UNSUPPORTED, "qh_weight_unpack: unknown flags 0x%x", flags);
  const bool w4 = is_w4(carrier);
  if (!w4 && (flags & (QH_CARRIER_HILO | QH_CARRIER_BIASED)))
    return fail(QH_STATUS_INVALID_ARGUMENT, "qh_weight_unpack: nibble flags given for an 8-bit carrier");
  if (carrier == QH_CARRIER_W4_FULL_CODES && (flags & QH_CARRIER_HILO))
    return fail(QH_STATUS_INVALID_ARGUMENT, "qh_weight_unpack: full-code carrier has no nibble pairs");
  if (k == 0 || n == 0 || k > (1u << 20) || n > (1u << 20))
    return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_weight_unpack: K=%u N=%u out of range", k, n);
  const uint64_t K = k, N = n;
  if (const char *rule = shape_rule(carrier, K, N))
    return fail(QH_STATUS_SHAPE_UNSUPPORTED, "qh_weight_unpack: carrier %u needs %s (K=%u N=%u)", carrier, rule, k, n);
  const bool one_per_byte = !w4 || carrier == QH_CARRIER_W4_FULL_CODES;
  const uint64_t want = one_per_byte ? K * N : K * N / 2;
  if (packed_bytes != want)
    return fail(QH_STATUS_INVALID_ARGUMENT, "qh_weight_unpack: carrier is %zu bytes, K=%u N=%u needs %llu", packed_bytes,
                k, n, static_cast<unsigned long long>(want));

  const Carrier c{carrier, K, N};
  const uint8_t x = (flags & QH_CARRIER_XOR80) ? 0x80 : 0x00;
  const bool hilo = (flags & QH_CARRIER_HILO) != 0;
  const int bias = (flags & QH_CARRIER_BIASED) ? 8 : 0;
  for (uint64_t col = 0; col < N; ++col) {
    int8_t *dst = weight_nk + col * K;
    for (uint64_t kk = 0; kk < K; ++kk) {
      const Where w = c.locate(kk, col);
      const uint8_t b = packed[w.byte] ^ x;
      if (!w4) {
        dst[kk] = static_cast<int8_t>(b);
        continue;
      }
      int nib;
      if (carrier == QH_CARRIER_W4_FULL_CODES) {
        if (b > 15)
          return fail(QH_STATUS_INVALID_ARGUMENT, "qh_weight_unpack: full-code byte 0x%02x at (k=%llu, n=%llu) is not a 4-bit code",
                      b, static_cast<unsigned long long>(kk), static_cast<unsigned long long>(col));
        nib = b;
      } else {
        nib = (w.first != hilo) ? (b & 15) : (b >> 4);
      }
      dst[kk] = static_cast<int8_t>(bias ? nib - 8 : (nib < 8 ? nib : nib - 16));
    }
  }
  return QH_STATUS_OK;
}
