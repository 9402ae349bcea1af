// C-ABI entry points: maximum / minimum (also clamp_min / clamp_max) and the
// ternary pointwise ops addcmul / addcdiv / lerp.
#include "ew_factories.h"

using namespace sa;

extern "C" {

int supa_amd_minmax(const supa_amd_ew_desc* d, int is_max, void* stream) {
  if (is_max) return run_ew(SimpleFactory<MaxOp>{}, d, stream, 3);
  return run_ew(SimpleFactory<MinOp>{}, d, stream, 3);
}

int supa_amd_pointwise(const supa_amd_ew_desc* d, int op, double value, int64_t ivalue, void* stream) {
  if (!d || d->noperands != 4) return SUPA_AMD_EINVAL;
  switch (op) {
    case SUPA_AMD_ADDCMUL: return run_ew(ValueFactory<AddcmulOp>{value, ivalue}, d, stream, 4);
    case SUPA_AMD_ADDCDIV:
      if (d->common_dtype != SUPA_AMD_F32 && d->common_dtype != SUPA_AMD_BF16 && d->common_dtype != SUPA_AMD_F16 &&
          d->common_dtype != SUPA_AMD_F64)
        return SUPA_AMD_EDTYPE;
      return run_ew(ValueFactory<AddcdivOp, true>{value, ivalue}, d, stream, 4);
    case SUPA_AMD_LERP:
      if (d->common_dtype != SUPA_AMD_F32 && d->common_dtype != SUPA_AMD_BF16 && d->common_dtype != SUPA_AMD_F16 &&
          d->common_dtype != SUPA_AMD_F64)
        return SUPA_AMD_EDTYPE;
      return run_ew(SimpleFactory<LerpOp, true>{}, d, stream, 4);
    default: return SUPA_AMD_EINVAL;
  }
}

}  // extern "C"
