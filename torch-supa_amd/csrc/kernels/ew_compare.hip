// C-ABI entry points: comparisons, isnan, where (masked_fill), and the
// dropout gradient's mask-and-scale.
#include "ew_factories.h"

using namespace sa;

namespace {

template <int K> struct CmpFactory {
  template <typename C> static constexpr bool ok() { return true; }
  template <typename C> CmpOp<K, C> make() const { return CmpOp<K, C>{}; }
};

struct MaskScaleFactory {
  double s;
  template <typename C> static constexpr bool ok() { return std::is_floating_point<C>::value; }
  template <typename C> MaskScaleOp<C> make() const { return MaskScaleOp<C>{static_cast<C>(s)}; }
};

}  // namespace

extern "C" {

int supa_amd_compare(const supa_amd_ew_desc* d, int kind, void* stream) {
  switch (kind) {
    case SUPA_AMD_CMP_EQ: return run_ew(CmpFactory<CMP_EQ>{}, d, stream, 3);
    case SUPA_AMD_CMP_NE: return run_ew(CmpFactory<CMP_NE>{}, d, stream, 3);
    case SUPA_AMD_CMP_LT: return run_ew(CmpFactory<CMP_LT>{}, d, stream, 3);
    case SUPA_AMD_CMP_LE: return run_ew(CmpFactory<CMP_LE>{}, d, stream, 3);
    case SUPA_AMD_CMP_GT: return run_ew(CmpFactory<CMP_GT>{}, d, stream, 3);
    case SUPA_AMD_CMP_GE: return run_ew(CmpFactory<CMP_GE>{}, d, stream, 3);
    default: return SUPA_AMD_EINVAL;
  }
}

int supa_amd_isnan(const supa_amd_ew_desc* d, void* stream) { return run_ew(SimpleFactory<IsNanOp>{}, d, stream, 2); }

int supa_amd_where(const supa_amd_ew_desc* d, void* stream) { return run_ew(SimpleFactory<WhereOp>{}, d, stream, 4); }

int supa_amd_mask_scale(const supa_amd_ew_desc* d, double scale, void* stream) {
  return run_ew(MaskScaleFactory{scale}, d, stream, 3);
}

}  // extern "C"
