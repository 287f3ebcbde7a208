// kq_linear_int4_noalloc: kq_linear_int4 without a caller workspace and
// without any allocation, for callers that cannot allocate device memory
// (code under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc).
//
// Scratch: one file-scope device array per GPU, resident from module load to
// process end.  Host code never passes the array's name to a kernel (on the
// host it only names the symbol); its device address is looked up once per
// device with hipGetSymbolAddress, on that device, and that address is what
// the kernels receive.  The kernels write every scratch byte they later read
// (staged activations, row exponents, split-K partials), so nothing is
// cleared between calls.  Calls that overlap on one GPU (different streams,
// or host threads without ordering) share the array and race; order them.
#include <atomic>
#include <mutex>

#include "kq_common.hpp"

static __device__ __align__(256) unsigned char scratch[KQ_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of `scratch` on the current device, looked up on the first
// call made with that device current.
int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return kq_set_error(KQ_ERR_HIP, std::string("kq_linear_int4_noalloc: hipGetDevice: ") + hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return kq_set_error(KQ_ERR_ARG, "kq_linear_int4_noalloc: device index beyond 64");
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || p == nullptr)
        return kq_set_error(KQ_ERR_HIP, std::string("kq_linear_int4_noalloc: hipGetSymbolAddress: ") +
                                            hipGetErrorString(e));
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return KQ_OK;
}

}  // namespace

extern "C" int kq_linear_int4_noalloc(const float* x, int64_t m, int64_t ldx, const uint8_t* payload,
                                      const uint16_t* scales, int64_t group_size, int64_t k_padded,
                                      const float* bias, float* y, int64_t ldy, int64_t n, int64_t k,
                                      kq_stream_t stream) {
  const size_t need = kq_linear_workspace_bytes(4, m, n, k, group_size);
  if (need > (size_t)KQ_NOALLOC_SCRATCH_BYTES)
    return kq_set_error(KQ_ERR_WORKSPACE,
                        "kq_linear_int4_noalloc: this shape needs " + std::to_string(need) +
                            " bytes of scratch, more than the " +
                            std::to_string((size_t)KQ_NOALLOC_SCRATCH_BYTES) +
                            " bytes it holds; use kq_linear_int4 with a workspace");
  void* p = nullptr;
  if (int s = scratch_address(&p)) return s;
  return kq_linear_int4(x, m, ldx, payload, scales, group_size, k_padded, bias, y, ldy, n, k, p,
                        (size_t)KQ_NOALLOC_SCRATCH_BYTES, stream);
}
