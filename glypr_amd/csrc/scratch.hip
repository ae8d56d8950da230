// scratch.hip — the activation scratch of glypr_hip_q8_0_matmul_noalloc.
//
// A file-scope device array of GLYPR_NOALLOC_SCRATCH_BYTES: each device the
// library runs on holds its own copy (loaded with the code object) until the
// process ends, so the no-allocation matmul needs no hipMalloc.  In host code
// `scratch` names a host-side stand-in, not device memory: it is never passed
// to a kernel.  resolve_scratch, called by glypr_hip_ctx_create with the
// context's device current, returns that device's address of the array, and
// kernels take that pointer.  All calls on one device share the array; the
// device's ScratchGuard rejects a call that would overlap a pending one on
// another stream.
#include <map>
#include <mutex>

#include "internal.hpp"

namespace glypr {

static __device__ __align__(256) uint8_t scratch[GLYPR_NOALLOC_SCRATCH_BYTES];

// One guard per device, made by the first context on the device and kept
// until the process ends (like the array it guards).
static std::mutex g_guards_mu;
static std::map<int, ScratchGuard*> g_guards;

hipError_t scratch_guard_init(int device) {
  std::lock_guard<std::mutex> lk(g_guards_mu);
  if (g_guards.count(device)) return hipSuccess;
  ScratchGuard* g = new (std::nothrow) ScratchGuard();
  if (!g) return hipErrorOutOfMemory;
  const hipError_t e = hipEventCreateWithFlags(&g->done, hipEventDisableTiming);
  if (e != hipSuccess) {
    delete g;
    return e;
  }
  g_guards[device] = g;
  return hipSuccess;
}

ScratchGuard* scratch_guard(int device) {
  std::lock_guard<std::mutex> lk(g_guards_mu);
  auto it = g_guards.find(device);
  return it == g_guards.end() ? nullptr : it->second;
}

hipError_t resolve_scratch(void** ptr) {
  *ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess) {
    *ptr = nullptr;
    (void)hipGetLastError();   // clear the sticky error of the failed lookup
  }
  return e;
}

}  // namespace glypr
