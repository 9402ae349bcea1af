// C-ABI entry points: add/sub, mul, div (true, trunc, floor).
#include "ew_factories.h"

using namespace sa;

extern "C" {

int supa_amd_add(const supa_amd_ew_desc* d, double alpha, int64_t ialpha, void* stream) {
  return run_ew(AddFactory{alpha, ialpha}, d, stream, 3);
}

int supa_amd_mul(const supa_amd_ew_desc* d, void* stream) { return run_ew(SimpleFactory<MulOp>{}, d, stream, 3); }

int supa_amd_div(const supa_amd_ew_desc* d, int mode, void* stream) {
  switch (mode) {
    case SUPA_AMD_DIV_TRUE: return run_ew(SimpleFactory<DivTrueOp, true>{}, d, stream, 3);
    case SUPA_AMD_DIV_TRUNC: {
      // a 16-bit quotient is rounded to its storage type before the trunc,
      // except for an immediate (CPU-scalar) divisor: the reference's
      // is_cpu_scalar branch (BinaryDivTruncKernel.cu:30-41) and upstream CPU
      // truncate the float quotient there
      const int rt = (d->noperands > 2 && d->op[2].is_scalar) ? 0 : half_code(d);
      return run_ew(DivTruncFactory{rt}, d, stream, 3);
    }
    case SUPA_AMD_DIV_FLOOR: return run_ew(SimpleFactory<DivFloorOp>{}, d, stream, 3);
    default: return SUPA_AMD_EINVAL;
  }
}

}  // extern "C"
