// Static device scratch of the allocation-free decode step
// (krill_decode_append_attention_noalloc).
//
// The array below is the split-K workspace of that entry point: partial
// outputs and (max, sum) pairs of the attention waves, read back by the
// merge launch of the same call.  Every device the library runs on holds its
// own copy from module load until the process ends.  In host code the name
// `scratch` is only a stand-in for the device symbol; the device address of
// each GPU's copy comes from hipGetSymbolAddress with that GPU current, once,
// and is the only value host code hands to kernels.
#include <hip/hip_runtime.h>

#include <mutex>

#include "scratch.hpp"

namespace krill {

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {
std::mutex g_scratch_mu;
void *g_scratch_ptr[kScratchMaxDevices] = {};
}  // namespace

hipError_t scratch_init(int device) {
  if (device < 0 || device >= kScratchMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (g_scratch_ptr[device]) return hipSuccess;
  int cur = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return e;
  if (cur != device) return hipErrorInvalidDevice;  // the caller makes `device` current
  void *p = nullptr;
  e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return e;
  if (!p) return hipErrorInvalidSymbol;
  g_scratch_ptr[device] = p;
  return hipSuccess;
}

void *scratch_ptr(int device) {
  if (device < 0 || device >= kScratchMaxDevices) return nullptr;
  std::lock_guard<std::mutex> g(g_scratch_mu);
  return g_scratch_ptr[device];
}

}  // namespace krill
