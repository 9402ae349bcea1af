// C-ABI entry point: activation functions (forward).
#include "ew_factories.h"

using namespace sa;

extern "C" {

int supa_amd_unary(const supa_amd_ew_desc* d, int op, void* stream) {
  switch (op) {
    case SUPA_AMD_GELU: return run_unary<U_GELU, false>(d, stream);
    case SUPA_AMD_GELU_TANH: return run_unary<U_GELU_TANH, false>(d, stream);
    case SUPA_AMD_SILU: return run_unary<U_SILU, false>(d, stream);
    case SUPA_AMD_SIGMOID: return run_unary<U_SIGMOID, false>(d, stream);
    case SUPA_AMD_TANH: return run_unary<U_TANH, false>(d, stream);
    case SUPA_AMD_EXP: return run_unary<U_EXP, false>(d, stream);
    case SUPA_AMD_LOG: return run_unary<U_LOG, false>(d, stream);
    case SUPA_AMD_ERF: return run_unary<U_ERF, false>(d, stream);
    case SUPA_AMD_RELU: return run_unary<U_RELU, false>(d, stream);
    case SUPA_AMD_NEG: return run_unary<U_NEG, false>(d, stream);
    case SUPA_AMD_RECIPROCAL: return run_unary<U_RECIPROCAL, false>(d, stream);
    case SUPA_AMD_ABS: return run_unary<U_ABS, false>(d, stream);
    case SUPA_AMD_SQRT: return run_unary<U_SQRT, false>(d, stream);
    case SUPA_AMD_EXPM1: return run_unary<U_EXPM1, false>(d, stream);
    case SUPA_AMD_LOG1P: return run_unary<U_LOG1P, false>(d, stream);
    default: return SUPA_AMD_EINVAL;
  }
}

}  // extern "C"
