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
    case SUPA_AMD_GELU_LOGERFC: return run_unary<U_GELU_LOGERFC, true>(d, stream);
    case SUPA_AMD_GELU_TANH_LOGISTIC: return run_unary<U_GELU_TANH_LOGISTIC, true>(d, stream);
    default: return SUPA_AMD_EINVAL;
  }
}

int supa_amd_loss_backward(const supa_amd_ew_desc* d, int loss, double norm, double beta, void* stream) {
  switch (loss) {
    case SUPA_AMD_LOSS_MSE: return d ? run_ew(MseBwdFactory{norm, half_code(d)}, d, stream, 4) : SUPA_AMD_EINVAL;
    case SUPA_AMD_LOSS_SMOOTH_L1:
      return d ? run_ew(SmoothL1BwdFactory{norm, beta, half_code(d)}, d, stream, 4) : SUPA_AMD_EINVAL;
    case SUPA_AMD_LOSS_HUBER:
      return d ? run_ew(HuberBwdFactory{norm, beta, half_code(d)}, d, stream, 4) : SUPA_AMD_EINVAL;
    case SUPA_AMD_LOSS_BCE:
      if (!d) return SUPA_AMD_EINVAL;
      {
        const int half = half_code(d);
        return d->noperands == 5 ? run_ew(BceProbBwdFactory<true>{norm, half}, d, stream, 5)
                                 : run_ew(BceProbBwdFactory<false>{norm, half}, d, stream, 4);
      }
    default: return SUPA_AMD_EINVAL;
  }
}

int supa_amd_bce_logits_backward(const supa_amd_ew_desc* d, int has_pos_weight, int has_weight, int mean,
                                 double numel, void* stream) {
  if (!d) return SUPA_AMD_EINVAL;
  const int want = 4 + (has_pos_weight ? 1 : 0) + (has_weight ? 1 : 0);
  if (d->noperands != want) return SUPA_AMD_EINVAL;
  for (int k = 0; k < d->noperands; ++k)
    if (!d->op[k].is_scalar && d->op[k].dtype != d->common_dtype) return SUPA_AMD_EDTYPE;
  const int rt = half_code(d);
  const int m = mean ? 1 : 0;
  if (has_pos_weight && has_weight) return run_ew(BceBwdFactory<true, true>{numel, m, rt}, d, stream, want);
  if (has_pos_weight) return run_ew(BceBwdFactory<true, false>{numel, m, rt}, d, stream, want);
  if (has_weight) return run_ew(BceBwdFactory<false, true>{numel, m, rt}, d, stream, want);
  return run_ew(BceBwdFactory<false, false>{numel, m, rt}, d, stream, want);
}

}  // extern "C"
