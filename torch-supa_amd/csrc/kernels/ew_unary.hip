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
    case SUPA_AMD_SIGN: return run_unary<U_SIGN, false>(d, stream);
    case SUPA_AMD_FLOOR: return run_unary<U_FLOOR, false>(d, stream);
    case SUPA_AMD_CEIL: return run_unary<U_CEIL, false>(d, stream);
    case SUPA_AMD_ROUND: return run_unary<U_ROUND, false>(d, stream);
    case SUPA_AMD_TRUNC: return run_unary<U_TRUNC, false>(d, stream);
    case SUPA_AMD_RSQRT: return run_unary<U_RSQRT, false>(d, stream);
    case SUPA_AMD_BITWISE_NOT: return run_unary<U_BITNOT, false>(d, stream);
    case SUPA_AMD_GELU_LOGERFC: return run_unary<U_GELU_LOGERFC, false>(d, stream);
    case SUPA_AMD_GELU_TANH_LOGISTIC: return run_unary<U_GELU_TANH_LOGISTIC, false>(d, stream);
    default: return SUPA_AMD_EINVAL;
  }
}

int supa_amd_bitwise(const supa_amd_ew_desc* d, int op, void* stream) {
  switch (op) {
    case SUPA_AMD_BIT_AND: return run_ew(BitFactory<BIT_AND>{}, d, stream, 3);
    case SUPA_AMD_BIT_OR: return run_ew(BitFactory<BIT_OR>{}, d, stream, 3);
    case SUPA_AMD_BIT_XOR: return run_ew(BitFactory<BIT_XOR>{}, d, stream, 3);
    default: return SUPA_AMD_EINVAL;
  }
}

int supa_amd_logical(const supa_amd_ew_desc* d, int op, void* stream) {
  switch (op) {
    case SUPA_AMD_LOGICAL_AND: return run_ew(LogicalFactory<LOG_AND>{}, d, stream, 3);
    case SUPA_AMD_LOGICAL_OR: return run_ew(LogicalFactory<LOG_OR>{}, d, stream, 3);
    case SUPA_AMD_LOGICAL_XOR: return run_ew(LogicalFactory<LOG_XOR>{}, d, stream, 3);
    case SUPA_AMD_LOGICAL_NOT: return run_ew(LogicalFactory<LOG_NOT>{}, d, stream, 2);
    default: return SUPA_AMD_EINVAL;
  }
}

int supa_amd_pow_scalar(const supa_amd_ew_desc* d, double exponent, void* stream) {
  if (!d) return SUPA_AMD_EINVAL;
  // the exponent in the tensor's dtype, as upstream's exp_scalar.to<scalar_t>()
  if (d->common_dtype == SUPA_AMD_F32) exponent = (double)(float)exponent;
  else if (d->common_dtype == SUPA_AMD_BF16) exponent = (double)host_round_bf16((float)exponent);
  else if (d->common_dtype == SUPA_AMD_F16) exponent = (double)(float)(_Float16)(float)exponent;
  const int mode = exponent == 2.0 ? POW_SQUARE
                   : exponent == 3.0 ? POW_CUBE
                   : exponent == -2.0 ? POW_INV_SQUARE
                                      : POW_GENERAL;
  const int half = half_code(d);
  return run_ew(PowScalarFactory{mode, half, exponent}, d, stream, 2);
}

int supa_amd_xlogy(const supa_amd_ew_desc* d, void* stream) {
  return run_ew(SimpleFactory<XlogyOp, true>{}, d, stream, 3);
}

int supa_amd_xlog1py(const supa_amd_ew_desc* d, void* stream) {
  return run_ew(SimpleFactory<Xlog1pyOp, true>{}, d, stream, 3);
}

int supa_amd_pow(const supa_amd_ew_desc* d, void* stream) {
  return run_ew(SimpleFactory<PowOp, true>{}, d, stream, 3);
}

}  // extern "C"
