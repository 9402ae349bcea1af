// C-ABI entry points: parameterised activations (leaky_relu, elu, softplus,
// hardswish, hardsigmoid, mish, log_sigmoid, threshold, hardshrink,
// softshrink) and their backwards (plus hardtanh's, whose forward is clamp);
// glu and prelu with theirs.
#include "ew_factories.h"

using namespace sa;

namespace {

template <int K, bool Bwd>
int run_act(const supa_amd_ew_desc* d, double p0, double p1, double p2, int flag, void* stream) {
  return run_ew(ActFactory<K, Bwd>{p0, p1, p2, flag}, d, stream, Bwd ? 3 : 2);
}

template <bool Bwd>
int act_dispatch(int act, const supa_amd_ew_desc* d, double p0, double p1, double p2, int flag, void* stream) {
  switch (act) {
    case SUPA_AMD_ACT_LEAKY_RELU: return run_act<A_LEAKY_RELU, Bwd>(d, p0, p1, p2, flag, stream);
    case SUPA_AMD_ACT_HARDTANH:
      if constexpr (Bwd) return run_act<A_HARDTANH, true>(d, p0, p1, p2, flag, stream);
      else return SUPA_AMD_EINVAL;  // the forward is clamp
    case SUPA_AMD_ACT_ELU: return run_act<A_ELU, Bwd>(d, p0, p1, p2, flag, stream);
    case SUPA_AMD_ACT_SOFTPLUS: return run_act<A_SOFTPLUS, Bwd>(d, p0, p1, p2, flag, stream);
    case SUPA_AMD_ACT_HARDSWISH: return run_act<A_HARDSWISH, Bwd>(d, p0, p1, p2, flag, stream);
    case SUPA_AMD_ACT_HARDSIGMOID: return run_act<A_HARDSIGMOID, Bwd>(d, p0, p1, p2, flag, stream);
    case SUPA_AMD_ACT_MISH: return run_act<A_MISH, Bwd>(d, p0, p1, p2, flag, stream);
    case SUPA_AMD_ACT_LOG_SIGMOID: return run_act<A_LOG_SIGMOID, Bwd>(d, p0, p1, p2, flag, stream);
    case SUPA_AMD_ACT_THRESHOLD: return run_act<A_THRESHOLD, Bwd>(d, p0, p1, p2, flag, stream);
    // lambda in scalar_t: rounded to a 16-bit common dtype
    case SUPA_AMD_ACT_HARDSHRINK:
      return run_act<A_HARDSHRINK, Bwd>(d, storage_param<double>(p0, half_code(d)), p1, p2, flag, stream);
    case SUPA_AMD_ACT_SOFTSHRINK:
      return run_act<A_SOFTSHRINK, Bwd>(d, storage_param<double>(p0, half_code(d)), p1, p2, flag, stream);
    default: return SUPA_AMD_EINVAL;
  }
}

}  // namespace

extern "C" {

int supa_amd_activation(const supa_amd_ew_desc* d, int act, double p0, double p1, double p2, void* stream) {
  return act_dispatch<false>(act, d, p0, p1, p2, 0, stream);
}

int supa_amd_activation_backward(const supa_amd_ew_desc* d, int act, double p0, double p1, double p2, int flag,
                                 void* stream) {
  return act_dispatch<true>(act, d, p0, p1, p2, flag, stream);
}

int supa_amd_glu(const supa_amd_ew_desc* d, void* stream) {
  return run_ew(SimpleFactory<GluOp, true>{}, d, stream, 3);
}

int supa_amd_glu_backward(const supa_amd_ew_desc* d, int half, void* stream) {
  if (half == 0) return run_ew(SimpleFactory<GluBwdFirstOp, true>{}, d, stream, 3);
  if (half == 1) return run_ew(SimpleFactory<GluBwdSecondOp, true>{}, d, stream, 4);
  return SUPA_AMD_EINVAL;
}

int supa_amd_prelu(const supa_amd_ew_desc* d, void* stream) {
  return run_ew(SimpleFactory<PreluOp, true>{}, d, stream, 3);
}

int supa_amd_prelu_backward(const supa_amd_ew_desc* d, int which, void* stream) {
  if (which == 0) return run_ew(SimpleFactory<PreluBwdInputOp, true>{}, d, stream, 4);
  if (which == 1) return run_ew(SimpleFactory<PreluBwdWeightOp, true>{}, d, stream, 3);
  return SUPA_AMD_EINVAL;
}

}  // extern "C"
