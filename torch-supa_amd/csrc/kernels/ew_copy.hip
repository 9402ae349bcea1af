// C-ABI entry points: copy/cast, fill, status strings.
#include "ew_factories.h"

namespace sa {

// Copy: out = cast(in).  The compute type follows the source's class so no
// value passes through a narrower type than both ends: integers (and bool)
// travel as int64, floating values as double when either end is float64,
// else as float.
int run_copy(const supa_amd_ew_desc* d, void* stream) {
  int rc = check_desc(d, 2, 2);
  if (rc) return rc;
  if (d->op[1].is_scalar) return SUPA_AMD_EINVAL;
  if (desc_numel(d) == 0) return SUPA_AMD_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int so = d->op[0].dtype, si = d->op[1].dtype;
  const int tin[1] = {1};
  supa_amd_ew_desc e = *d;
  e.common_dtype = si;
  if (so == si) {
    return with_storage(si, [&](auto* tag) -> int {
      using T = std::remove_pointer_t<decltype(tag)>;
      using C = opmath_t<T>;
      return launch_static<IdentityOp<C>, C, T, T, T>(IdentityOp<C>{}, e, tin, st);
    });
  }
  auto ffam = [](int dt) { return dt == SUPA_AMD_F32 || dt == SUPA_AMD_BF16 || dt == SUPA_AMD_F16 || dt == SUPA_AMD_F64; };
  if (ffam(so) && ffam(si)) {
    auto w = [](int dt, auto&& f) -> int {
      switch (dt) {
        case SUPA_AMD_F32: return f((float*)nullptr);
        case SUPA_AMD_BF16: return f((bf16*)nullptr);
        case SUPA_AMD_F16: return f((f16*)nullptr);
        default: return f((double*)nullptr);
      }
    };
    return w(so, [&](auto* to) -> int {
      return w(si, [&](auto* ti) -> int {
        using TO = std::remove_pointer_t<decltype(to)>;
        using TI = std::remove_pointer_t<decltype(ti)>;
        if constexpr (std::is_same<TO, TI>::value) {
          return SUPA_AMD_EINVAL;
        } else {
          using C = typename std::conditional<std::is_same<TO, double>::value || std::is_same<TI, double>::value,
                                              double, float>::type;
          return launch_static<IdentityOp<C>, C, TI, TO, TI>(IdentityOp<C>{}, e, tin, st);
        }
      });
    });
  }
  if (dtype_is_floating(si)) return launch_dynamic<2, IdentityOp<double>, double>(IdentityOp<double>{}, e, tin, si, st);
  return launch_dynamic<2, IdentityOp<int64_t>, int64_t>(IdentityOp<int64_t>{}, e, tin, si, st);
}

// Fill: the value is an immediate scalar converted to the output's dtype.
int run_fill(const supa_amd_ew_desc* d, void* stream) {
  int rc = check_desc(d, 2, 2);
  if (rc) return rc;
  if (!d->op[1].is_scalar) return SUPA_AMD_EINVAL;
  supa_amd_ew_desc e = *d;
  e.common_dtype = d->op[0].dtype;
  return run_ew(SimpleFactory<IdentityOp>{}, &e, stream, 2);
}

}  // namespace sa


using namespace sa;

extern "C" {

const char* supa_amd_status_string(int status) {
  switch (status) {
    case SUPA_AMD_OK: return "success";
    case SUPA_AMD_EINVAL: return "invalid argument or descriptor";
    case SUPA_AMD_EDTYPE: return "unsupported dtype combination";
    case SUPA_AMD_ELAYOUT: return "unsupported layout";
    case SUPA_AMD_EWORKSPACE: return "workspace missing or too small";
    default: return status > 0 ? hipGetErrorString((hipError_t)status) : "unknown error";
  }
}

int supa_amd_abi_version(void) { return SUPA_AMD_ABI_VERSION; }

int supa_amd_copy(const supa_amd_ew_desc* d, void* stream) { return run_copy(d, stream); }

int supa_amd_fill(const supa_amd_ew_desc* d, void* stream) { return run_fill(d, stream); }

}  // extern "C"
