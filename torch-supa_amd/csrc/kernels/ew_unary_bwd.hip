// C-ABI entry points: activation gradients and pointwise loss gradients.
#include "ew_factories.h"

using namespace sa;

extern "C" {

int supa_amd_unary_backward(const supa_amd_ew_desc* d, int op, void* stream) {
  switch (op) {
    case SUPA_AMD_GELU: return run_unary<U_GELU, true>(d, stream);
    case SUPA_AMD_GELU_TANH: return run_unary<U_GELU_TANH, true>(d, stream);
    case SUPA_AMD_SILU: return run_unary<U_SILU, true>(d, stream);
    case SUPA_AMD_SIGMOID: return run_unary<U_SIGMOID, true>(d, stream);
    case SUPA_AMD_TANH: return run_unary<U_TANH, true>(d, stream);
    default: return SUPA_AMD_EINVAL;
  }
}

int supa_amd_loss_backward(const supa_amd_ew_desc* d, int loss, double norm, double beta, void* stream) {
  switch (loss) {
    case SUPA_AMD_LOSS_MSE: return run_ew(MseBwdFactory{norm}, d, stream, 4);
    case SUPA_AMD_LOSS_SMOOTH_L1: return run_ew(SmoothL1BwdFactory{norm, beta}, d, stream, 4);
    default: return SUPA_AMD_EINVAL;
  }
}

}  // extern "C"
