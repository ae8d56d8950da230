// scratch.hip — the activation scratch of glypr_hip_q8_0_matmul_noalloc.
//
// A file-scope device array of GLYPR_NOALLOC_SCRATCH_BYTES: each device the
// library runs on holds its own copy (loaded with the code object) until the
// process ends, so the no-allocation matmul needs no hipMalloc.  In host code
// `scratch` names a host-side stand-in, not device memory: it is never passed
// to a kernel.  resolve_scratch, called by glypr_hip_ctx_create with the
// context's device current, returns that device's address of the array, and
// kernels take that pointer.  All calls on one device share the array.
#include "internal.hpp"

namespace glypr {

static __device__ __align__(256) uint8_t scratch[GLYPR_NOALLOC_SCRATCH_BYTES];

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
