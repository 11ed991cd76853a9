// qh_qmm_run_chain without a scratch operand: the intermediate results of the chain live in a
// file-scope device array, so the call allocates nothing (for callers that cannot allocate:
// code under HIP graph capture, tight serving loops).
//
// The array is one per device (each device that loads the library holds its own copy for the
// life of the process).  Host code never passes the array's name to a kernel -- in host code it
// is a stand-in, not a device address -- but the address hipGetSymbolAddress returns for it on
// the current device, looked up once per device on the first call there.  Every call on one
// device uses the same array: calls that overlap on one device (different streams, threads)
// race on it.  Nothing in it must start at zero: each chain step writes every output element
// before the next step reads it.

#include <atomic>
#include <mutex>

#include "qmm_internal.h"

namespace qh {
namespace {

constexpr size_t kChainScratchBytes = size_t{8} << 20;  // 8 MiB: M x N outputs of one step
static __device__ __align__(256) uint8_t scratch[kChainScratchBytes];

constexpr int kMaxDevices = 64;
std::atomic<void *> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of this device's array (looked up once per device, with that device current).
qh_status scratch_for_current_device(void **out) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return hip_fail(err, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(QH_STATUS_UNSUPPORTED, "device %d beyond %d devices", dev, kMaxDevices);
  void *p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (err != hipSuccess) return hip_fail(err, "hipGetSymbolAddress(chain scratch)");
      if (p == nullptr) return fail(QH_STATUS_RUNTIME_ERROR, "hipGetSymbolAddress(chain scratch) returned NULL");
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return QH_STATUS_OK;
}

}  // namespace
}  // namespace qh

using namespace qh;

extern "C" qh_status qh_qmm_run_chain_noalloc(const qh_qmm_prepared *prep, uint32_t m, uint32_t chain,
                                              const void *act_dev, void *out_dev, uint32_t contract, uint32_t divisor,
                                              void *stream) {
  if (prep == nullptr) return fail(QH_STATUS_INVALID_ARGUMENT, "qh_qmm_run_chain_noalloc: prepared handle is NULL");
  if (chain <= 1) return qh_qmm_run_chain(prep, m, chain, act_dev, out_dev, nullptr, contract, divisor, stream);
  const size_t elem = prep->shape.out_bits == 16 ? 2 : 1;
  const size_t need = static_cast<size_t>(m) * static_cast<size_t>(prep->shape.N) * elem;
  if (need > kChainScratchBytes)
    return fail(QH_STATUS_SHAPE_UNSUPPORTED,
                "qh_qmm_run_chain_noalloc: M x N outputs take %zu bytes, beyond the %zu-byte static scratch "
                "(use qh_qmm_run_chain with a scratch buffer)",
                need, kChainScratchBytes);
  void *ptr = nullptr;
  const qh_status st = scratch_for_current_device(&ptr);
  if (st != QH_STATUS_OK) return st;
  return qh_qmm_run_chain(prep, m, chain, act_dev, out_dev, ptr, contract, divisor, stream);
}
