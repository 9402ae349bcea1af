/*
 * supa_amd.h -- C ABI of the MI355X (gfx950) kernels behind the PrivateUse1
 * elementwise + loss operator path.
 *
 * Every entry point enqueues work on `stream` (a hipStream_t passed as void*;
 * NULL is the legacy default stream) and returns without waiting.  Entry points
 * never allocate device memory and never throw; outputs, and any workspace an
 * entry point asks for, come pre-allocated from the caller.  All tensors are
 * borrowed raw device pointers for the duration of the enqueue.
 *
 * Return value: SUPA_AMD_OK (0), a negative SUPA_AMD_E* argument error, or a
 * positive hipError_t from the launch.  supa_amd_status_string() names both.
 *
 * Each declaration names the reference interface it replaces.  Paths are in
 * BIRENSUPA/torch-supa; "NF:<line>" is the schema line in upstream
 * torchgen/packaged/ATen/native/native_functions.yaml (torch 2.10.0), for ops
 * whose device kernel the reference takes from its upstream-ATen operator
 * library (third-party/torch-supa-op, registered by the generated
 * RegisterSUPANative_0.cpp, script/codegen_native/gen.py:537-612).
 */
#ifndef SUPA_AMD_H
#define SUPA_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SUPA_AMD_ABI_VERSION 2

/* ------------------------------------------------------------ status codes */
#define SUPA_AMD_OK 0
#define SUPA_AMD_EINVAL (-1)   /* malformed descriptor or argument */
#define SUPA_AMD_EDTYPE (-2)   /* dtype combination without a kernel */
#define SUPA_AMD_ELAYOUT (-3)  /* layout the entry point does not take */
#define SUPA_AMD_EWORKSPACE (-4) /* workspace missing or too small */

/* ------------------------------------------------------------ dtype codes
 * Equal to c10::ScalarType so the host layer passes them through. */
#define SUPA_AMD_U8 0
#define SUPA_AMD_I8 1
#define SUPA_AMD_I16 2
#define SUPA_AMD_I32 3
#define SUPA_AMD_I64 4
#define SUPA_AMD_F16 5
#define SUPA_AMD_F32 6
#define SUPA_AMD_F64 7
#define SUPA_AMD_BOOL 11
#define SUPA_AMD_BF16 15

/* ------------------------------------------------- elementwise descriptor
 * An already broadcast, dimension-coalesced iteration space (the planner's
 * output, the role TensorIteratorBase plays for the reference's gpu_kernel,
 * torch_supa/csrc/aten/ops/kernels/elementwise/Loops.cuh:110-134).
 * Dimension 0 is the fastest-moving one.  op[0] is the output, op[1..] are
 * the inputs in the order each entry point documents. */
#define SUPA_AMD_MAX_DIMS 8
#define SUPA_AMD_MAX_OPERANDS 6

typedef struct supa_amd_operand {
  void* data;                          /* element (0,...,0) of the view */
  int64_t strides[SUPA_AMD_MAX_DIMS];  /* in elements; 0 = broadcast dim */
  int32_t dtype;                       /* storage dtype code */
  int32_t is_scalar;                   /* 1: an immediate host scalar; data and strides unused */
  double scalar;                       /* immediate value for floating/bool ops */
  int64_t iscalar;                     /* immediate value for integer ops */
} supa_amd_operand;

typedef struct supa_amd_ew_desc {
  int64_t sizes[SUPA_AMD_MAX_DIMS];
  int32_t ndim;          /* 0 means one element */
  int32_t noperands;     /* outputs + inputs */
  int32_t common_dtype;  /* inputs are converted to this dtype, then computed in its opmath type */
  int32_t reserved;
  supa_amd_operand op[SUPA_AMD_MAX_OPERANDS];
} supa_amd_ew_desc;

const char* supa_amd_status_string(int status);
int supa_amd_abi_version(void);

/* ------------------------------------------------------ elementwise binary */

/* out = a + alpha * b in the opmath type of common_dtype (sub is alpha = -alpha).
 * op = {out, a, b}.  Replaces add_stub: add_kernel,
 * torch_supa/csrc/aten/ops/kernels/elementwise/UfuncCUDA_add.cu:77-340,
 * registered at :341-345. */
int supa_amd_add(const supa_amd_ew_desc* d, double alpha, int64_t ialpha, void* stream);

/* out = a * b (bool: a && b).  op = {out, a, b}.  Replaces mul_stub:
 * mul_kernel_cuda, .../elementwise/BinaryMulKernel.cu:25-43. */
int supa_amd_mul(const supa_amd_ew_desc* d, void* stream);

/* Division.  mode 0 = true division (IEEE a / b, also for a CPU-scalar
 * divisor), 1 = trunc, 2 = floor.  op = {out, a, b}.  Trunc of bf16 / f16
 * tensors truncates the quotient rounded to the 16-bit type; with an
 * immediate divisor (op[2].is_scalar) it truncates the float quotient.
 * Replaces
 * div_true_stub / div_trunc_stub / div_floor_stub:
 * .../elementwise/BinaryDivTrueKernel.cu:22-65, BinaryDivTruncKernel.cu:22-55,
 * BinaryDivFloorKernel.cu:22-82. */
#define SUPA_AMD_DIV_TRUE 0
#define SUPA_AMD_DIV_TRUNC 1
#define SUPA_AMD_DIV_FLOOR 2
int supa_amd_div(const supa_amd_ew_desc* d, int mode, void* stream);

/* out = maximum(a, b) (is_max) or minimum(a, b); a NaN operand is the
 * result.  op = {out, a, b}.  Replaces maximum.out / minimum.out (upstream
 * MaxMinElementwiseKernel.cu) and, with a bound operand, clamp_min /
 * clamp_max. */
int supa_amd_minmax(const supa_amd_ew_desc* d, int is_max, void* stream);

/* Ternary pointwise ops, op = {out, self, t1, t2}:
 *   ADDCMUL  out = self + value * (t1 * t2)
 *   ADDCDIV  out = self + value * (t1 / t2)        (floating dtypes)
 *   LERP     out = lerp(self, end = t1, weight = t2): |w| < 0.5 ?
 *            self + w (end - self) : end - (end - self)(1 - w)  (floating)
 * value / ivalue: the bound value for floating / integer results (unused by
 * LERP, whose weight may be an immediate scalar operand).  Each `a + v * x`
 * is one fused multiply-add.  Replaces addcmul.out / addcdiv.out (upstream
 * PointwiseOpsKernel.cu) and lerp.Scalar_out / lerp.Tensor_out (upstream
 * Lerp.cu), which the reference takes from its operator library. */
#define SUPA_AMD_ADDCMUL 0
#define SUPA_AMD_ADDCDIV 1
#define SUPA_AMD_LERP 2
int supa_amd_pointwise(const supa_amd_ew_desc* d, int op, double value, int64_t ivalue, void* stream);

/* ------------------------------------------------ activations (unary) */
#define SUPA_AMD_GELU 0
#define SUPA_AMD_GELU_TANH 1
#define SUPA_AMD_SILU 2
#define SUPA_AMD_SIGMOID 3
#define SUPA_AMD_TANH 4
#define SUPA_AMD_EXP 5
#define SUPA_AMD_LOG 6
#define SUPA_AMD_ERF 7
#define SUPA_AMD_RELU 8
#define SUPA_AMD_NEG 9
#define SUPA_AMD_RECIPROCAL 10
#define SUPA_AMD_ABS 11
#define SUPA_AMD_SQRT 12
#define SUPA_AMD_EXPM1 13
#define SUPA_AMD_LOG1P 14
#define SUPA_AMD_SIGN 15
#define SUPA_AMD_FLOOR 16
#define SUPA_AMD_CEIL 17
#define SUPA_AMD_ROUND 18
#define SUPA_AMD_TRUNC 19
#define SUPA_AMD_RSQRT 20
#define SUPA_AMD_BITWISE_NOT 21
/* Opt-in gelu forms free of the cancellation of 1 + erf / 1 + tanh for
 * x << 0 (not the reference's arithmetic; the host selects them only when
 * torch.supa.set_accurate_gelu_enabled(True) or SUPA_AMD_ACCURATE_GELU=1):
 * GELU_LOGERFC = x - (x/2) erfc(|x|/sqrt2) (x >= 0) / (x/2) erfc(|x|/sqrt2)
 * (x < 0); GELU_TANH_LOGISTIC = x / (1 + exp(-2u)), u = b (x + k x^3).
 * Both are accepted by supa_amd_unary and supa_amd_unary_backward (whose
 * GELU_TANH_LOGISTIC gradient is GELU_TANH's). */
#define SUPA_AMD_GELU_LOGERFC 22
#define SUPA_AMD_GELU_TANH_LOGISTIC 23

/* out = f(x), floating dtypes (RELU, NEG and ABS also integer).  op = {out, x}.
 * Replaces the reference's upstream-ATen activation kernels: gelu.out NF:5216,
 * silu.out NF:5374, sigmoid.out NF:5441, tanh.out, exp.out, log.out, erf.out,
 * relu, neg.out, expm1.out NF:2650, log1p.out NF:3585, and the pointwise
 * helpers reciprocal.out (x.__rtruediv__), abs.out, sqrt.out (IEEE 1/x, |x|,
 * correctly rounded sqrt). */
int supa_amd_unary(const supa_amd_ew_desc* d, int op, void* stream);
/* The rounding / sign family and friends on the same entry: SIGN (also sgn
 * for real dtypes; (0 < x) - (x < 0), NaN -> 0) sign.out NF:9892 / sgn.out NF:445; FLOOR,
 * CEIL, TRUNC, ROUND (halves to even; integers copy) floor.out NF:2768,
 * ceil.out NF:1490, trunc.out NF:6505, round.out NF:5123; RSQRT (IEEE 1 /
 * correctly rounded sqrt, as upstream CPU) rsqrt.out NF:5303; BITWISE_NOT
 * (bool: not; integers: ~) bitwise_not.out NF:1231. */

/* Bitwise and / or / xor on bool and integer dtypes.  op = {out, a, b}.
 * Replaces bitwise_and.Tensor_out NF:8549, bitwise_or.Tensor_out NF:8616,
 * bitwise_xor.Tensor_out NF:8683 (upstream BinaryBitwiseOpsKernels.cu). */
#define SUPA_AMD_BIT_AND 0
#define SUPA_AMD_BIT_OR 1
#define SUPA_AMD_BIT_XOR 2
int supa_amd_bitwise(const supa_amd_ew_desc* d, int op, void* stream);

/* Logical and / or / xor (op = {out, a, b}) and not (op = {out, x}): every
 * operand tested against zero, the output bool (or any dtype: 1 / 0).
 * Replaces logical_and.out NF:1339, logical_or.out NF:1360, logical_xor.out
 * NF:1318, logical_not.out NF:1297 (upstream LogicalOpsKernels.cu). */
#define SUPA_AMD_LOGICAL_AND 0
#define SUPA_AMD_LOGICAL_OR 1
#define SUPA_AMD_LOGICAL_XOR 2
#define SUPA_AMD_LOGICAL_NOT 3
int supa_amd_logical(const supa_amd_ew_desc* d, int op, void* stream);

/* out = x ** exponent, floating dtypes, op = {out, x}.  The exponent is first
 * rounded to the tensor's dtype; 2 -> x*x, 3 -> x*x*x, -2 -> 1/(x*x) (products
 * rounded to a 16-bit storage type between factors), otherwise pow evaluated
 * in double and rounded once.  (0, 1, 0.5, -0.5 and -1 are the caller's
 * fill / copy / sqrt / rsqrt / reciprocal.)  Replaces pow.Tensor_Scalar_out
 * NF:10494 (upstream PowKernel.cu pow_tensor_scalar_kernel). */
int supa_amd_pow_scalar(const supa_amd_ew_desc* d, double exponent, void* stream);
/* out = base ** exponent elementwise, floating dtypes, pow in double rounded
 * once; op = {out, base, exponent}, either may be an immediate scalar.
 * Replaces pow.Tensor_Tensor_out NF:10466 and pow.Scalar_out NF:10481. */
int supa_amd_pow(const supa_amd_ew_desc* d, void* stream);
/* out = x * log(y), 0 where x == 0, NaN where y is NaN; floating dtypes,
 * op = {out, x, y}, either may be an immediate scalar.  Replaces
 * xlogy.OutTensor NF:3673, xlogy.OutScalar_Self NF:3683,
 * xlogy.OutScalar_Other NF:3690 (upstream xlogy_kernel_cuda). */
int supa_amd_xlogy(const supa_amd_ew_desc* d, void* stream);
/* out = x * log1p(y), 0 where x == 0, NaN where y is NaN; as supa_amd_xlogy.
 * Replaces special_xlog1py.out NF:13652, .self_scalar_out NF:13662 and
 * .other_scalar_out NF:13670 (upstream xlog1py_kernel_cuda). */
int supa_amd_xlog1py(const supa_amd_ew_desc* d, void* stream);

/* scatter_(dim, index, value), the assign form: for every element of index
 * (ndim dims of index_sizes, index_strides in elements, int64 values), the
 * element of out at the same coordinates but with coordinate `dim` replaced
 * by the index value becomes value (ivalue for integer and bool dtypes).
 * out_strides in elements; an index outside [0, out_dim_size) writes nothing
 * and sets *error_flag (when given) to 2.  Replaces scatter_.value NF:8458
 * and scatter.value_out NF:8462 (upstream scatter_fill_kernel), which one_hot
 * runs. */
int supa_amd_scatter_fill(void* out, int32_t dtype, const int64_t* out_strides, int64_t out_dim_size,
                          const int64_t* index, const int64_t* index_sizes, const int64_t* index_strides, int32_t ndim,
                          int32_t dim, double value, int64_t ivalue, int32_t* error_flag, void* stream);

/* grad_in = f'(...) * dy.  op = {grad_in, dy, x} where x is the forward input
 * for GELU, GELU_TANH, SILU and the forward output for SIGMOID, TANH.
 * Replaces gelu_backward.grad_input NF:5245, silu_backward.grad_input NF:5383,
 * sigmoid_backward.grad_input NF:13229, tanh_backward.grad_input. */
int supa_amd_unary_backward(const supa_amd_ew_desc* d, int op, void* stream);

/* Parameterised activations, floating dtypes (THRESHOLD: every non-bool
 * dtype).  Forward op = {out, x}; backward op = {grad_in, grad, x}.
 *   LEAKY_RELU   p0 negative_slope           leaky_relu.out NF:12217, _backward NF:12234
 *   HARDTANH     p0 min, p1 max (backward; the forward is clamp)  hardtanh_backward NF:12174
 *   ELU          p0 alpha, p1 scale, p2 input_scale; backward flag = is_result
 *                (x is then the forward output)  elu.out NF:12057, elu_backward NF:12071
 *   SOFTPLUS     p0 beta, p1 threshold        softplus.out NF:12318, _backward NF:12333
 *   HARDSWISH    -                            hardswish.out NF:12193, _backward NF:12211
 *   HARDSIGMOID  -                            hardsigmoid.out NF:12126, _backward NF:12148
 *   MISH         -                            mish.out NF:5409, mish_backward NF:5417
 *   LOG_SIGMOID  -                            log_sigmoid_forward NF:12260, _backward NF:12276
 *   THRESHOLD    p0 threshold, p1 value (forward); backward: x <= p0 ? 0 : grad
 *                                             threshold.out NF:6244, threshold_backward NF:6252
 *   HARDSHRINK   p0 lambda                    hardshrink.out NF:5268, hardshrink_backward NF:5281
 *   SOFTSHRINK   p0 lambda                    softshrink.out NF:12345, softshrink_backward NF:12359
 *                (both backwards: |x| <= lambda ? 0 : grad; lambda is rounded
 *                to a 16-bit common dtype, upstream's scalar_t lambda)
 * The formulas are upstream's CUDA activation functors, evaluated in float
 * (double for f64) with the parameters rounded to it. */
#define SUPA_AMD_ACT_LEAKY_RELU 0
#define SUPA_AMD_ACT_HARDTANH 1
#define SUPA_AMD_ACT_ELU 2
#define SUPA_AMD_ACT_SOFTPLUS 3
#define SUPA_AMD_ACT_HARDSWISH 4
#define SUPA_AMD_ACT_HARDSIGMOID 5
#define SUPA_AMD_ACT_MISH 6
#define SUPA_AMD_ACT_LOG_SIGMOID 7
#define SUPA_AMD_ACT_THRESHOLD 8
#define SUPA_AMD_ACT_HARDSHRINK 9
#define SUPA_AMD_ACT_SOFTSHRINK 10
int supa_amd_activation(const supa_amd_ew_desc* d, int act, double p0, double p1, double p2, void* stream);
int supa_amd_activation_backward(const supa_amd_ew_desc* d, int act, double p0, double p1, double p2, int flag,
                                 void* stream);

/* glu: out = a * sigmoid(b), a and b the two halves of the input along the
 * gated dim (strided views; sigmoid = 1 / (1 + exp(-b)) in float).  op = {out,
 * a, b}.  Replaces glu.out NF:12087 (upstream ActivationGluKernel.cu
 * glu_kernel).
 * glu_backward, one half per call: half 0 writes the first half's gradient
 * sigmoid(b) g, op = {grad_a, b, g}; half 1 the second half's
 * ((1 - s) s) g a, op = {grad_b, a, b, g}.  Replaces
 * glu_backward.grad_input NF:12100 (upstream glu_backward_kernel, which writes
 * both halves from one launch). */
int supa_amd_glu(const supa_amd_ew_desc* d, void* stream);
int supa_amd_glu_backward(const supa_amd_ew_desc* d, int half, void* stream);

/* prelu: out = x > 0 ? x : w x, w broadcast to x.  op = {out, x, w}.
 * Replaces _prelu_kernel NF:5203 (upstream prelu_kernel).
 * prelu backward, one output per call: which 0 the input gradient
 * x > 0 ? g : w g, op = {grad_x, x, w, g}; which 1 the elementwise weight
 * gradient x > 0 ? 0 : x g, op = {grad_w, x, g} (full shape; autograd sums
 * it to the weight's).  Replaces _prelu_kernel_backward NF:5210 (upstream
 * prelu_backward_kernel, one launch with two outputs). */
int supa_amd_prelu(const supa_amd_ew_desc* d, void* stream);
int supa_amd_prelu_backward(const supa_amd_ew_desc* d, int which, void* stream);

/* ------------------------------------------ comparisons and selects */

/* out = (a OP b) as 1 / 0, compared in common_dtype (NaN unequal to
 * everything); out is usually bool.  op = {out, a, b}.  Replaces
 * ne.Scalar_out / ne.Tensor_out NF:9089 / 9107, eq NF:9152 / 9171, ge NF:9190 /
 * 9209, le NF:9254 / 9272, gt NF:9317 / 9336, lt NF:9381 / 9399 (upstream
 * CompareEQKernel.cu, CompareKernels.cu). */
#define SUPA_AMD_CMP_EQ 0
#define SUPA_AMD_CMP_NE 1
#define SUPA_AMD_CMP_LT 2
#define SUPA_AMD_CMP_LE 3
#define SUPA_AMD_CMP_GT 4
#define SUPA_AMD_CMP_GE 5
int supa_amd_compare(const supa_amd_ew_desc* d, int kind, void* stream);

/* out = (x != x).  op = {out, x}.  Replaces isnan NF:3219 (upstream: self != self). */
int supa_amd_isnan(const supa_amd_ew_desc* d, void* stream);

/* out = cond ? a : b, cond bool; a or b may be immediate scalars.
 * op = {out, cond, a, b}.  Replaces where.self_out NF:6701 (upstream
 * TensorCompare.cu where_kernel) and, with a = value and b = out = self,
 * masked_fill_.Scalar NF:8254 (upstream masked_fill_kernel). */
int supa_amd_where(const supa_amd_ew_desc* d, void* stream);

/* out = (mask * grad) * scale, mask bool.  op = {out, mask, grad}.
 * Replaces native_dropout_backward NF:296 (upstream masked_scale_kernel). */
int supa_amd_mask_scale(const supa_amd_ew_desc* d, double scale, void* stream);

/* ------------------------------------------------------ random numbers */

/* Counter-based Philox4x32-10 draws: element i of a call with (seed, offset)
 * is word i % 4 of philox(counter = (i / 4, offset), key = seed), u =
 * (word >> 8) * 2^-24 in [0, 1).  out is a contiguous f32 / bf16 / f16
 * buffer of n elements.  The caller's generator supplies (seed, offset) and
 * advances offset by one per call.
 *   uniform:   out = fma(u, hi - lo, lo)        uniform_ NF:8983
 *   bernoulli: out = u < p ? 1 : 0              bernoulli_.float NF:1146
 *   dropout:   mask = u < keep, out = (x * mask) * (1 / keep)
 *                                               native_dropout NF:286
 *   normal:    Box-Muller in double on word pairs (0,1) and (2,3) of each
 *              Philox call: r = sqrt(-2 log u1), u1 = (hi24 + 1) 2^-24,
 *              t = 2 pi u2; elements r cos t, r sin t; out = mean + std z
 *                                               normal_ NF:10552
 * (The reference draws through curand's Philox; the streams differ.) */
int supa_amd_uniform(void* out, int32_t dtype, int64_t n, double lo, double hi, uint64_t seed, uint64_t offset,
                     void* stream);
int supa_amd_bernoulli(void* out, int32_t dtype, int64_t n, double p, uint64_t seed, uint64_t offset, void* stream);
int supa_amd_normal(void* out, int32_t dtype, int64_t n, double mean, double stdv, uint64_t seed, uint64_t offset,
                    void* stream);
int supa_amd_dropout(const void* x, int32_t dtype, void* out, uint8_t* mask, int64_t n, double keep, uint64_t seed,
                     uint64_t offset, void* stream);

/* ------------------------------------------------------ copy / fill */

/* out = cast(in), any strides and dtypes.  op = {out, in}.  Replaces the
 * device-to-device part of SUPANativeFunctions::copy_,
 * torch_supa/csrc/aten/common/Copy.cpp:154-245, and direct_copy_kernel_cuda,
 * .../elementwise/copy.cu:791-859. */
int supa_amd_copy(const supa_amd_ew_desc* d, void* stream);

/* out = value (op[1] is an immediate scalar).  op = {out, value}.  Replaces
 * fill_.Scalar NF:2727 (upstream FillKernel) and zero_ NF:7079. */
int supa_amd_fill(const supa_amd_ew_desc* d, void* stream);

/* ------------------------------------------------------ pointwise losses */
#define SUPA_AMD_LOSS_MSE 0
#define SUPA_AMD_LOSS_SMOOTH_L1 1
#define SUPA_AMD_LOSS_BCE_LOGITS 2
#define SUPA_AMD_LOSS_HUBER 3 /* beta = delta */
#define SUPA_AMD_LOSS_BCE 4   /* on probabilities; optional weight (has_weight) */

#define SUPA_AMD_REDUCTION_NONE 0
#define SUPA_AMD_REDUCTION_MEAN 1
#define SUPA_AMD_REDUCTION_SUM 2

/* Loss terms per element.  op = {out, input, target[, pos_weight][, weight]}
 * (pos_weight only for BCE, flagged by has_pos_weight; weight only for BCE,
 * flagged by has_weight).
 * reduction NONE: op[0] is the [n] loss tensor.
 * reduction MEAN/SUM: op[0] describes the iteration space only (its data is
 * unused) and the single f32/f64-rounded-to-out_dtype result is written to
 * `out_scalar` (a one-element device buffer of dtype op[0].dtype); the sum is
 * accumulated in float32 (float64 for f64), deterministically, in two stages
 * through `workspace` (see supa_amd_loss_workspace_bytes).
 * Replaces mse_loss.out NF:11832, smooth_l1_loss.out NF:11988 (upstream
 * structured kernels + at::sum/at::mean, sum_kernel_cuda
 * .../kernels/reduce/ReduceSumKernel.cu:102-113, mean_kernel_cuda
 * ReduceMomentKernel.cu:37-55), and
 * SUPANativeFunctions::binary_cross_entropy_with_logits,
 * torch_supa/csrc/aten/ops/BinaryCrossEntropyWithLogits.cpp:23-73 with its
 * kernel .../elementwise/BinaryCrossEntropyWithLogitsKernel.cu:17-113.
 * HUBER replaces huber_loss.out NF:12014 (upstream huber_kernel_cuda), BCE
 * binary_cross_entropy.out NF:1178 ((t - 1) max(log1p(-x), -100) -
 * t max(log x, -100), times the weight). */
int supa_amd_loss_forward(const supa_amd_ew_desc* d, int loss, int reduction, double beta,
                          int has_pos_weight, int has_weight, void* out_scalar,
                          void* workspace, int64_t workspace_bytes, void* stream);
int64_t supa_amd_loss_workspace_bytes(int64_t numel);

/* Loss gradients.  op = {grad_in, grad_out, input, target}; grad_out is
 * broadcast (0-dim) for MEAN/SUM.  norm is the reduction factor the reference
 * applies (2/n or 2 for MSE, 1/n or 1 for SMOOTH_L1 and HUBER); for BCE
 * op = {grad_in, grad_out, input, target[, weight]} and norm is the divisor
 * (n for MEAN, else 1): g (x - t) / max((1 - x) x, 1e-12), times the weight,
 * / norm.  Replaces mse_loss_backward.grad_input NF:11846,
 * smooth_l1_loss_backward.grad_input NF:12002, huber_loss_backward.out
 * NF:12026 and binary_cross_entropy_backward.grad_input NF:1195. */
int supa_amd_loss_backward(const supa_amd_ew_desc* d, int loss, double norm, double beta,
                           void* stream);

/* Gradient of binary_cross_entropy_with_logits w.r.t. its input in one pass.
 * op = {grad_in, grad_out, input, target[, pos_weight][, weight]} (pos_weight
 * flagged by has_pos_weight, weight by has_weight; grad_out broadcast 0-dim
 * for MEAN/SUM).  Evaluates the autograd formula's op sequence in its order
 * -- u = pos_weight * target; ((u + 1) - target) * sigmoid(input) - u
 * (sigmoid(input) - target without pos_weight); * grad_out; * weight;
 * / numel for MEAN (mean != 0) -- rounding every intermediate to the
 * tensors' dtype, so the result is bit-identical to running those ops one by
 * one.  Every tensor operand has the descriptor's common dtype.  Replaces the
 * 7-8 elementwise kernels the reference runs for this gradient
 * (binary_cross_entropy_with_logits_backward of upstream's autograd,
 * torchgen/packaged/autograd/derivatives.yaml:2017-2019; the reference
 * registers only the forward, BinaryCrossEntropyWithLogits.cpp:23-73). */
int supa_amd_bce_logits_backward(const supa_amd_ew_desc* d, int has_pos_weight, int has_weight, int mean,
                                 double numel, void* stream);

/* ---------------------------------------------------------- reductions */

/* out[0] = scale * sum(in) over every element of the described input
 * (op = {out, in}; op[0] describes the input's iteration space, its data is
 * the one-element output).  Accumulates in float32 (float64 for f64 input;
 * int64 for bool and integer input, whose output must be int64 and scale 1),
 * deterministic two-stage tree through `workspace`.  scale = 1 for sum,
 * 1/n for mean (the reference's mean factor, ReduceMomentKernel.cu:20).
 * Replaces sum_stub / mean_stub for full reductions:
 * .../kernels/reduce/ReduceSumKernel.cu:102-113, ReduceMomentKernel.cu:37-55. */
int supa_amd_sum(const supa_amd_ew_desc* d, double scale, void* workspace,
                 int64_t workspace_bytes, void* stream);
int64_t supa_amd_sum_workspace_bytes(int64_t numel);

/* supa_amd_sum without a workspace argument and without any allocation.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The workspace is a file-scope device array of the
 * library, 8448 bytes on each GPU it runs on, held until the process ends and
 * set up on the first call on a device; a reduction needing more than
 * supa_amd_sum_noalloc_max_workspace_bytes() is refused with
 * SUPA_AMD_EWORKSPACE (supa_amd_sum's need is that size for every numel).
 * The array needs no initial contents.  Every call on one GPU shares it:
 * calls that overlap in time on that GPU (different streams, or threads
 * without ordering) race and must not be issued; calls in one stream's order
 * are safe.  Same arguments, results and errors as supa_amd_sum otherwise. */
int supa_amd_sum_noalloc(const supa_amd_ew_desc* d, double scale, void* stream);
int64_t supa_amd_sum_noalloc_max_workspace_bytes(void);

/* Reduction of the innermost `inner` elements of each of `outer` rows of a
 * contiguous input: out[r] = scale * sum(in[r*inner .. r*inner+inner)).
 * Bool / integer input sums into an int64 output (scale 1).
 * Replaces sum_stub / mean_stub for dim reductions over trailing dims. */
int supa_amd_sum_rows(const void* in, int32_t in_dtype, void* out, int32_t out_dtype,
                      int64_t outer, int64_t inner, double scale, void* stream);

/* ------------------------------------------------------ row softmax ops */

/* out[r, :] = x[r, :] - max_r - log(sum exp(x[r, :] - max_r)) over rows of a
 * contiguous [rows, cols] input.  in/out dtypes: f32 -> f32, bf16 -> bf16,
 * f16 -> f16, bf16/f16 -> f32 (half_to_float).  Replaces _log_softmax.out
 * NF:3752 (upstream SoftMax.cu, torch/include/ATen/native/cuda/PersistentSoftmax.cuh). */
int supa_amd_log_softmax_forward(const void* in, int32_t in_dtype, void* out, int32_t out_dtype,
                                 int64_t rows, int64_t cols, void* stream);

/* grad_in[r, :] = g[r, :] - exp(y[r, :]) * sum(g[r, :]).  g and y share
 * dtype gy_dtype; grad_in has gin_dtype.  Replaces
 * _log_softmax_backward_data.out NF:3763. */
int supa_amd_log_softmax_backward(const void* grad, const void* output, int32_t gy_dtype,
                                  void* grad_in, int32_t gin_dtype, int64_t rows, int64_t cols,
                                  void* stream);

/* out[r, :] = exp(x[r, :] - max_r) / sum(exp(x[r, :] - max_r)), dtypes as
 * for log_softmax; a row holding NaN or +inf, or only -inf, is NaN.
 * Replaces _softmax.out NF:5697 (upstream SoftMax.cu, PersistentSoftmax.cuh). */
int supa_amd_softmax_forward(const void* in, int32_t in_dtype, void* out, int32_t out_dtype,
                             int64_t rows, int64_t cols, void* stream);

/* grad_in[r, :] = y[r, :] * (g[r, :] - sum(g[r, :] * y[r, :])), dtypes as
 * for the log_softmax backward.  Replaces _softmax_backward_data.out NF:5709. */
int supa_amd_softmax_backward(const void* grad, const void* output, int32_t gy_dtype,
                              void* grad_in, int32_t gin_dtype, int64_t rows, int64_t cols,
                              void* stream);

/* ------------------------------------------------------------ nll_loss */

/* nll_loss over logp [n, c] (contiguous, dtype f32/bf16/f16/f64), int64
 * target [n], optional weight [c] (same dtype, or NULL).
 * reduction NONE: out [n]; MEAN/SUM: out and total_weight are one-element
 * buffers of the logp dtype.  Rows whose target equals ignore_index
 * contribute nothing and are not counted (mean of no rows is NaN).
 * *error_flag (device int32, may be NULL) is set to 1 when a target is out of
 * range; the caller reads it lazily.  Replaces nll_loss_forward.output
 * NF:11928; ignore semantics as CrossEntropyLossKernel.cu:71-119. */
int supa_amd_nll_loss_forward(const void* logp, int32_t dtype, const int64_t* target,
                              const void* weight, int64_t n, int64_t c, int reduction,
                              int64_t ignore_index, void* out, void* total_weight,
                              int32_t* error_flag, void* stream);

/* grad_in [n, c] (fully written: zero except grad_in[i, t_i] = -w[t_i] * g_i,
 * or -w[t_i] * g / total_weight for MEAN, -w[t_i] * g for SUM).  grad_out is
 * [n] for NONE, one element otherwise; total_weight is the forward's
 * one-element buffer.  Replaces nll_loss_backward.grad_input NF:11940. */
int supa_amd_nll_loss_backward(const void* grad_out, int32_t dtype, const int64_t* target,
                               const void* weight, const void* total_weight, int64_t n, int64_t c,
                               int reduction, int64_t ignore_index, void* grad_in,
                               int32_t* error_flag, void* stream);

/* nll_loss2d over logp [n, c, s] (contiguous; s = H * W), int64 target
 * [n, s]: out [n, s] for `none`, else the weighted sum or mean and
 * total_weight as for nll_loss.  The mean/sum forward reduces in two stages
 * through `workspace` (supa_amd_nll_loss2d_workspace_bytes(), no content
 * requirement).  Replaces nll_loss2d_forward.output NF:11960 (upstream
 * LossNLL2d.cu). */
int64_t supa_amd_nll_loss2d_workspace_bytes(void);
int supa_amd_nll_loss2d_forward(const void* logp, int32_t dtype, const int64_t* target,
                                const void* weight, int64_t n, int64_t c, int64_t s, int reduction,
                                int64_t ignore_index, void* out, void* total_weight, void* workspace,
                                int64_t ws_bytes, int32_t* error_flag, void* stream);

/* grad_in [n, c, s]: every element written once, -w[t] g at (i, t[i, p], p)
 * and zero elsewhere (g per position for `none`, g / total_weight for
 * mean).  Replaces nll_loss2d_backward.grad_input NF:11974. */
int supa_amd_nll_loss2d_backward(const void* grad_out, int32_t dtype, const int64_t* target,
                                 const void* weight, const void* total_weight, int64_t n, int64_t c,
                                 int64_t s, int reduction, int64_t ignore_index, void* grad_in,
                                 int32_t* error_flag, void* stream);

/* ------------------------------------------------- fused cross-entropy
 * cross_entropy over contiguous logits [n, c] (f32 / bf16 / f16) with int64
 * targets [n], no class weight, no label smoothing: the forward reads the
 * logits once and saves lse[i] = log(sum_j exp(x[i, j])) in float32; the
 * backward reads them once more and writes
 * grad[i, j] = (exp(x[i, j] - lse[i]) - [j == t_i]) * g_i.  Rows whose target
 * is ignore_index have loss 0 and gradient 0 and are not counted; a mean over
 * no rows is NaN.  This generalises the reference's fp32-only fast path to
 * bf16 / f16 and ignore_index, with a fused backward:
 * SUPANativeFunctions::cross_entropy_loss and CrossEntropyLossFastPathFunction,
 * torch_supa/csrc/aten/ops/CrossEntropyLoss.cpp:23-151, and
 * cross_entropy_loss_2d_kernel_supa,
 * .../kernels/elementwise/CrossEntropyLossKernel.cu:71-195. */

/* Bytes of workspace the forward needs (float32 per-row losses). */
int64_t supa_amd_cross_entropy_workspace_bytes(int64_t n);

/* reduction NONE: out is [n] in the logits dtype.  MEAN / SUM: out is one
 * element in the logits dtype (sum over rows in a fixed order, float32), and
 * count (one float32, may be NULL for SUM) receives the kept-row count.
 * lse: [n] float32, written for the backward (0 for ignored rows). */
int supa_amd_cross_entropy_forward(const void* logits, int32_t dtype, const int64_t* target, int64_t n,
                                   int64_t c, int64_t ignore_index, int reduction, void* out, float* lse,
                                   float* count, void* workspace, int64_t workspace_bytes,
                                   int32_t* error_flag, void* stream);

/* grad_out: [n] for NONE, one element otherwise (logits dtype); lse and count
 * as written by the forward.  grad_logits: [n, c], every element written. */
int supa_amd_cross_entropy_backward(const void* grad_out, const void* logits, int32_t dtype,
                                    const int64_t* target, const float* lse, const float* count, int64_t n,
                                    int64_t c, int64_t ignore_index, int reduction, void* grad_logits,
                                    int32_t* error_flag, void* stream);

/* Probability (soft-label) targets: target is [n, c] in the logits' dtype
 * (both contiguous); loss_i = sum_j t_ij (lse_i - x_ij), reduced over rows
 * as none / sum / mean (mean divides by n; NaN for n = 0).  The forward reads
 * logits and target once each and saves lse [n] and tsum [n] = sum_j t_ij
 * (float32); the backward writes
 * grad[i, j] = g_i (exp(x_ij - lse_i) tsum_i - t_ij), g_i = grad_out[i]
 * (NONE), grad_out[0] (SUM) or grad_out[0] / n (MEAN).  workspace: as
 * supa_amd_cross_entropy_workspace_bytes(n).  Replaces the reference's
 * fp32 probability-target fast path: cross_entropy_prob_kernel,
 * .../kernels/elementwise/CrossEntropyLossKernel.cu:532-576 (forward), and
 * CrossEntropyLossFastPathFunction::backward's prob_target branch,
 * torch_supa/csrc/aten/ops/CrossEntropyLoss.cpp:94-131 (backward through
 * -target * grad_factor and _log_softmax_backward_data), for f32 / bf16 /
 * f16. */
int supa_amd_cross_entropy_prob_forward(const void* logits, const void* target, int32_t dtype, int64_t n,
                                        int64_t c, int reduction, void* out, float* lse, float* tsum,
                                        void* workspace, int64_t workspace_bytes, void* stream);
int supa_amd_cross_entropy_prob_backward(const void* grad_out, const void* logits, const void* target,
                                         int32_t dtype, const float* lse, const float* tsum, int64_t n,
                                         int64_t c, int reduction, void* grad_logits, void* stream);

/* ------------------------------------------------- multi-tensor apply */
#define SUPA_AMD_FOREACH_ADD 0      /* out = a + alpha * y                    */
#define SUPA_AMD_FOREACH_MUL 1      /* out = a * y                            */
#define SUPA_AMD_FOREACH_DIV 2      /* out = a / y                            */
#define SUPA_AMD_FOREACH_MAXIMUM 3  /* out = max(a, y), a NaN in either wins  */
#define SUPA_AMD_FOREACH_MINIMUM 4  /* out = min(a, y), a NaN in either wins  */
#define SUPA_AMD_FOREACH_ADDCMUL 5  /* out = a + s * (b * c)                  */
#define SUPA_AMD_FOREACH_ADDCDIV 6  /* out = a + s * (b / c)                  */
#define SUPA_AMD_FOREACH_LERP 7     /* out = lerp(a, b, w)                    */
#define SUPA_AMD_FOREACH_ZERO 8     /* out = 0                                */
#define SUPA_AMD_FOREACH_POW 9      /* out = a ** y (LIST or SCALARS; a SCALARS
                                       exponent must be exact in `dtype`)     */
#define SUPA_AMD_FOREACH_RPOW 10    /* out = scalars[k] ** a (SCALARS only)   */
#define SUPA_AMD_FOREACH_COPY 11    /* out = a                                */
#define SUPA_AMD_FOREACH_UNARY 32   /* + SUPA_AMD_SIGMOID, _TANH, _EXP, _LOG, _ERF,
                                       _NEG, _RECIPROCAL, _ABS, _SQRT, _EXPM1,
                                       _LOG1P, _SIGN, _FLOOR, _CEIL, _ROUND,
                                       _TRUNC, _RSQRT: out = f(a) */
/* Where y (lerp: the weight w) comes from: */
#define SUPA_AMD_FOREACH_LIST 0       /* y = b[k][i]; lerp w = c[k][i]            */
#define SUPA_AMD_FOREACH_SCALARS 1    /* y = scalars[k] (a Scalar repeats)        */
#define SUPA_AMD_FOREACH_DEVSCALAR 2  /* y = *scalar_ptr, one device element of `dtype` */

/* In-place or out-of-place list arithmetic over `ntensors` contiguous tensors
 * of one dtype (f32 / bf16 / f16 / f64), computed in float (double for f64)
 * exactly as the elementwise entry points do, so every output equals the
 * per-tensor op bit for bit.  out may equal a (the in-place overloads).
 * addcmul / addcdiv take their value from scalars[k] whatever `form` says;
 * the unary ops and ZERO ignore `form`.  One launch covers up to 40 tensors.
 * Replaces the fast paths of upstream ForeachBinaryOpList.cu,
 * ForeachBinaryOpScalar.cu, ForeachBinaryOpScalarList.cu,
 * ForeachBinaryOpScalarTensor.cu, ForeachPointwiseOp.cu, ForeachTernaryOp.cu
 * and ForeachUnaryOp.cu that the reference registers through its codegen
 * (script/codegen_supa/gen.py:1708-1734): _foreach_add_.Tensor NF:10716,
 * _foreach_sub_ NF:10732-10762, _foreach_mul_.Tensor NF:10826, _foreach_div_
 * NF:10842-10890, _foreach_clamp_max_ / _clamp_min_ NF:10906-10981,
 * _foreach_maximum_ / _minimum_ NF:10997-11075, _foreach_addcdiv_
 * NF:11104-11120, _foreach_addcmul_ NF:11150-11167, _foreach_lerp_
 * NF:11380-11412, _foreach_sqrt_ NF:11691, _foreach_zero_ NF:11745, the
 * other unary ops listed above (_foreach_ceil_ NF:11244, _foreach_floor_
 * NF:11349, _foreach_round_ NF:11601, _foreach_rsqrt_ NF:11616,
 * _foreach_sign_ NF:11646, _foreach_trunc_ NF:11737), _foreach_pow in its
 * List / Scalar / ScalarList / ScalarAndTensor forms NF:11527-11571
 * (upstream ForeachBinaryOp*.cu over pow), _foreach_copy_ NF:11753, and the
 * out-of-place forms.  POW with SCALARS evaluates each exponent as the
 * per-tensor pow(Tensor, Scalar) does: 0 gives 1, 1 a copy, 0.5 / -0.5 / -1
 * sqrt / rsqrt / reciprocal, 2 / 3 / -2 products, else pow in double. */
int supa_amd_foreach(int op, int form, int32_t ntensors, void* const* out, const void* const* a,
                     const void* const* b, const void* const* c, const int64_t* numel, int32_t dtype,
                     const double* scalars, double alpha, const void* scalar_ptr, void* stream);

/* The add / mul subset with one scalar for every tensor; b == NULL selects
 * the scalar overload (value `scalar`).  Replaces _foreach_add_.List
 * NF:10685, _foreach_add_.Scalar NF:10668, _foreach_mul_.List NF:10794,
 * _foreach_mul_.Scalar NF:10777 and their out-of-place forms. */
int supa_amd_foreach_binary(int op, int32_t ntensors, void* const* out, void* const* a,
                            void* const* b, const int64_t* numel, int32_t dtype, double scalar,
                            double alpha, void* stream);

/* Per-tensor vector norms: out[k] = ||x[k]||_ord for ord 1, 2 or +inf
 * (HUGE_VAL), accumulated in float (double for f64 inputs) per chunk and
 * combined per tensor in a second kernel; an empty tensor gives 0, a NaN
 * anywhere gives NaN.  out: `ntensors` contiguous elements of out_dtype
 * (the input dtype, f32 or f64).  The workspace holds one partial per chunk:
 * supa_amd_foreach_norm_workspace_bytes, no content requirement.  Replaces
 * _foreach_norm.Scalar NF:11518 (upstream ForeachReduceOp.cu). */
int64_t supa_amd_foreach_norm_workspace_bytes(int32_t ntensors, const int64_t* numel, int32_t dtype);
int supa_amd_foreach_norm(int32_t ntensors, const void* const* x, const int64_t* numel, int32_t dtype,
                          double ord, void* out, int32_t out_dtype, void* workspace, int64_t ws_bytes,
                          void* stream);

/* Vector norm of each row of a contiguous [outer, inner] input (f32 / bf16 /
 * f16 / f64; inner >= 1) into out[outer] (the input dtype, or f32), for
 * every order: 0 (count of non-zeros), 1, 2, +inf / -inf (largest /
 * smallest |x|, NaN propagating), any other finite p (sum |x|^p, then
 * ^(1/p)); accumulated in f32 (f64 for f64).  Long rows with few of them
 * reduce in two launches through a workspace of
 * supa_amd_norm_rows_workspace_bytes (0: none needed).  The caller moves
 * the reduced dims last.  Replaces linalg_vector_norm.out NF:14470 over
 * dims (upstream ReduceNormKernel.cu: NormZeroOps / NormOneOps /
 * NormTwoOps / AbsMaxOps / AbsMinOps / NormOps). */
int64_t supa_amd_norm_rows_workspace_bytes(int64_t outer, int64_t inner, int32_t dtype);
int supa_amd_norm_rows(const void* in, int32_t dtype, void* out, int32_t out_dtype, int64_t outer, int64_t inner,
                       double ord, void* workspace, int64_t ws_bytes, void* stream);

/* Variance (take_sqrt 0) or standard deviation (1) of each row of a
 * contiguous [outer, inner] input (f32 / bf16 / f16 / f64; inner >= 1) into
 * out_var[outer], and the row mean into out_mean[outer] when it is not NULL,
 * both in the input dtype: Welford's (count, mean, M2) accumulated in f32
 * (f64 for f64), var = M2 / max(0, count - correction).  Long rows with few
 * of them reduce in two launches through a workspace of
 * supa_amd_moments_rows_workspace_bytes (0: none needed).  The caller moves
 * the reduced dims last.  Replaces var.correction_out NF:6629,
 * std.correction_out NF:6088, var_mean.correction NF:6668,
 * std_mean.correction NF:6063 (upstream ReduceMomentKernel.cu over
 * WelfordOps). */
int64_t supa_amd_moments_rows_workspace_bytes(int64_t outer, int64_t inner, int32_t dtype);
int supa_amd_moments_rows(const void* in, int32_t dtype, int64_t outer, int64_t inner, double correction,
                          int take_sqrt, void* out_var, void* out_mean, void* workspace, int64_t ws_bytes,
                          void* stream);

/* Mixed-precision gradient unscale: every element of the `ntensors`
 * contiguous tensors (f32 / bf16 / f16 / f64) is multiplied in place by
 * *inv_scale (left as is when that is exactly 1), and *found_inf (device
 * float) is set to 1.0 if any element is inf or NaN.  Replaces
 * _amp_foreach_non_finite_check_and_unscale_ NF:10632 (upstream
 * AmpKernels.cu over MultiTensorApply.cuh). */
int supa_amd_amp_unscale(int32_t ntensors, void* const* tensors, const int64_t* numel, int32_t dtype,
                         float* found_inf, const float* inv_scale, void* stream);

/* Dynamic loss-scale update, one device thread: after an overflow
 * (*found_inf != 0) scale *= backoff and growth_tracker = 0; otherwise the
 * tracker counts successful steps and, on reaching growth_interval, the scale
 * grows by growth_factor (unless that overflows float32) and the tracker
 * resets.  scale and found_inf are one device float each, growth_tracker one
 * device int32.  Replaces _amp_update_scale_ NF:10640. */
int supa_amd_amp_update_scale(float* scale, int32_t* growth_tracker, const float* found_inf,
                              double growth_factor, double backoff_factor, int64_t growth_interval,
                              void* stream);

/* One fused AdamW step over `ntensors` tensors (params, grads, exp_avgs,
 * exp_avg_sqs [, max_exp_avg_sqs when amsgrad]) of one dtype (f32, bf16, f16,
 * f64), each with a one-element f32 state_step on the device.  lr_ptr (device
 * f32, may be NULL) overrides lr; grad_scale / found_inf (device f32, may be
 * NULL) follow the AMP contract.  Replaces _fused_adamw_ NF:16041 and
 * _fused_adamw_.tensor_lr NF:16050 (upstream fused_adamw_impl.cu,
 * torch/include/ATen/native/cuda/fused_adam_utils.cuh:27-93, :130-137). */
int supa_amd_fused_adamw(int32_t ntensors, void* const* params, void* const* grads,
                         void* const* exp_avgs, void* const* exp_avg_sqs,
                         void* const* max_exp_avg_sqs, void* const* state_steps,
                         const int64_t* numel, int32_t dtype, double lr, const float* lr_ptr,
                         double beta1, double beta2, double weight_decay, double eps,
                         int amsgrad, int maximize, const float* grad_scale,
                         const float* found_inf, void* stream);

/* ----------------------------------------------- max / min with index */
/* For each of `outer` rows of a contiguous input with `inner` elements, and
 * each chunk of `chunk` elements of the row (chunk = inner: one per row), the
 * extremal element: a NaN beats every number, equal values (and NaNs) go to
 * the smaller index, otherwise the larger (is_min = 0) or smaller value.
 * Writes the value (out_val, the input dtype; may be NULL) and its index
 * (out_idx, int64; may be NULL) at [row * nchunks + chunk].  The index is the
 * position in the row, or in_idx[row * inner + j] when in_idx is given (the
 * second launch over chunk winners).  Any dtype but complex.  Replaces
 * amax.out NF:3926, amin.out NF:4115, max.dim_max NF:3894, min.dim_min
 * NF:4091, argmax.out NF:839, argmin.out NF:852, max.unary_out NF:10274,
 * min.unary_out NF:10204. */
int supa_amd_argext_rows(const void* in, int32_t dtype, const int64_t* in_idx, int64_t outer,
                         int64_t inner, int64_t chunk, int is_min, void* out_val,
                         int64_t* out_idx, void* stream);

/* Fused Adam (weight decay added to the gradient, upstream adam_math's
 * ADAM_MODE::ORIGINAL: grad += param * weight_decay after the maximize
 * negation); otherwise as supa_amd_fused_adamw.  Replaces _fused_adam_
 * NF:16021 and _fused_adam_.tensor_lr NF:16030 (upstream fused_adam_impl.cu). */
int supa_amd_fused_adam(int32_t ntensors, void* const* params, void* const* grads,
                        void* const* exp_avgs, void* const* exp_avg_sqs,
                        void* const* max_exp_avg_sqs, void* const* state_steps,
                        const int64_t* numel, int32_t dtype, double lr, const float* lr_ptr,
                        double beta1, double beta2, double weight_decay, double eps,
                        int amsgrad, int maximize, const float* grad_scale,
                        const float* found_inf, void* stream);

/* _fused_sgd_ over a tensor list, in place: one multi-tensor launch per
 * table of tensors, as supa_amd_fused_adamw.  params, grads and (with momentum) momentum_buffers are
 * device pointers to contiguous tensors of `dtype` (f32, bf16, f16, f64) with
 * numel[i] elements each.  momentum_buffers is NULL exactly when momentum is
 * 0; with is_first_step each buffer is written with the gradient instead of
 * read.  lr_ptr (a device float, may be NULL) overrides lr; grad_scale divides
 * the gradients first (and they are stored back unscaled); a found_inf of 1
 * makes the step a no-op.  Per element, as upstream sgd_math
 * (FusedSgdKernel.cu) with double hyper-parameters:
 *   g /= grad_scale; g = -g if maximize; g += weight_decay p;
 *   buf = first ? g : momentum buf + (1 - dampening) g;
 *   g = nesterov ? g + momentum buf : buf;  p -= lr g
 * Replaces _fused_sgd_ NF:16061 and _fused_sgd_.tensor_lr NF:16070. */
int supa_amd_fused_sgd(int32_t ntensors, void* const* params, void* const* grads, void* const* momentum_buffers,
                       const int64_t* numel, int32_t dtype, double weight_decay, double momentum, double lr,
                       const float* lr_ptr, double dampening, int nesterov, int maximize, int is_first_step,
                       const float* grad_scale, const float* found_inf, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SUPA_AMD_H */
