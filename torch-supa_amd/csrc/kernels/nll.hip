// nll_loss forward / backward for a [n, c] log-probability matrix with int64
// targets, an optional class weight and ignore_index.
//
// Forward (mean/sum): one 1024-thread workgroup gathers the n selected
// log-probabilities, accumulates -w*logp and the weight total in float32
// (float64 for float64 data) with a fixed-order tree, and writes the loss and
// total_weight in the data dtype; mean divides by the float32 total.  A mean
// over no rows is 0/0 = NaN, as in the reference
// (CrossEntropyLossKernel.cu:67, :191-193).  Forward (none): one thread per row.
//
// Backward: writes every element of grad_input once -- 16-byte vectors of
// zeros, with the row's target element replaced by its gradient -- so the
// [n, c] tensor costs one HBM write and no separate zero fill.
//
// Spatial form (nll_loss2d: logp [n, c, s], target [n, s], s = H * W): the
// forward gathers with a multi-workgroup two-stage reduction (a fixed number
// of partials, so the order is deterministic); the backward writes every
// element of grad_input once in 16-byte vectors along s, each vector's
// (image, class) found by two magic-number divisions.
//
// Out-of-range targets set *error_flag (when given) and contribute nothing;
// the host reads the flag lazily.
#include "ew_launch.h"
#include "divmod.h"

namespace sa {

constexpr int kNllBlock = 1024;
constexpr int kNllUnroll = 1;  // 16-byte vectors per thread in the backward writer (1: 80 % of peak, 4: 66 %)

template <typename T, typename ACC>
__global__ void __launch_bounds__(kNllBlock)
k_nll_fwd_reduce(const T* __restrict__ logp, const int64_t* __restrict__ target, const T* __restrict__ weight,
                 int64_t n, int64_t c, int64_t ignore_index, int mean, T* __restrict__ out, T* __restrict__ total_weight,
                 int32_t* error_flag) {
  __shared__ ACC lds_v[kNllBlock / 64];
  __shared__ ACC lds_w[kNllBlock / 64];
  ACC v = ACC(0), w = ACC(0);
  bool bad = false;
  constexpr int U = 8;  // rows in flight per step (targets, then their gathers); sums keep the row order
  for (int64_t i0 = threadIdx.x; i0 < n; i0 += (int64_t)U * kNllBlock) {
    int64_t tg[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = i0 + (int64_t)u * kNllBlock;
      tg[u] = i < n ? target[i] : ignore_index;
    }
    ACC lp[U], wt[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = i0 + (int64_t)u * kNllBlock, t = tg[u];
      const bool use = i < n && t != ignore_index && t >= 0 && t < c;
      lp[u] = use ? (ACC)to_arith(logp[i * c + t]) : ACC(0);
      wt[u] = use ? (weight ? (ACC)to_arith(weight[t]) : ACC(1)) : ACC(0);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t t = tg[u];
      if (i0 + (int64_t)u * kNllBlock >= n || t == ignore_index) continue;
      if (t < 0 || t >= c) {
        bad = true;
        continue;
      }
      v += -wt[u] * lp[u];
      w += wt[u];
    }
  }
  if (bad && error_flag) *error_flag = 1;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    v += __shfl_xor(v, off, 64);
    w += __shfl_xor(w, off, 64);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    lds_v[wave] = v;
    lds_w[wave] = w;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    ACC sv = ACC(0), sw = ACC(0);
#pragma unroll
    for (int k = 0; k < kNllBlock / 64; ++k) {
      sv += lds_v[k];
      sw += lds_w[k];
    }
    total_weight[0] = from_arith<T>(sw);
    out[0] = from_arith<T>(mean ? sv / sw : sv);
  }
}

template <typename T>
__global__ void __launch_bounds__(kBlock)
k_nll_fwd_none(const T* __restrict__ logp, const int64_t* __restrict__ target, const T* __restrict__ weight, int64_t n,
               int64_t c, int64_t ignore_index, T* __restrict__ out, int32_t* error_flag) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  const int64_t t = target[i];
  if (t == ignore_index) {
    out[i] = from_arith<T>(0.0f);
    return;
  }
  if (t < 0 || t >= c) {
    if (error_flag) *error_flag = 1;
    out[i] = from_arith<T>(0.0f);
    return;
  }
  using C = opmath_t<T>;
  const C wt = weight ? (C)to_arith(weight[t]) : C(1);
  out[i] = from_arith<T>(-wt * (C)to_arith(logp[i * c + t]));
}

// The writer keeps four wavefronts per workgroup: c3's [8192, 128256] bf16
// gradient took 0.315 ms with 256 threads against 0.446 ms with 64.
constexpr int kNllBwdBlock = 256;

// grad_in[i, :] over a 2-D grid: blockIdx.y = row, x = column chunks of
// kNllBwdBlock * VEC elements.  g_row is the row's gradient before the weight:
// -(g_i) for none, -(g / total_weight) for mean, -g for sum, formed in the data
// dtype as upstream does.
template <typename T, int VEC>
__global__ void __launch_bounds__(kNllBwdBlock)
k_nll_bwd(const T* __restrict__ grad_out, const int64_t* __restrict__ target, const T* __restrict__ weight,
          const T* __restrict__ total_weight, int64_t c, int reduction, int64_t ignore_index, T* __restrict__ gin,
          int32_t* error_flag) {
  using C = opmath_t<T>;
  const int64_t row = blockIdx.y;
  const int64_t t = target[row];
  const bool active = t != ignore_index && t >= 0 && t < c;
  if (threadIdx.x == 0 && blockIdx.x == 0 && t != ignore_index && (t < 0 || t >= c) && error_flag) *error_flag = 1;
  T gval = from_arith<T>(C(0));
  if (active) {
    C g;
    if (reduction == SUPA_AMD_REDUCTION_NONE) g = (C)to_arith(grad_out[row]);
    else if (reduction == SUPA_AMD_REDUCTION_MEAN) g = (C)to_arith(grad_out[0]) / (C)to_arith(total_weight[0]);
    else g = (C)to_arith(grad_out[0]);
    const T gs = from_arith<T>(-g);  // rounded to the storage type, as upstream forms it
    gval = weight ? from_arith<T>((C)to_arith(weight[t]) * (C)to_arith(gs)) : gs;
  }
  T* dst = gin + row * c;
  const T zero = from_arith<T>(C(0));
#pragma unroll
  for (int u = 0; u < kNllUnroll; ++u) {
    const int64_t col0 = (((int64_t)blockIdx.x * kNllUnroll + u) * kNllBwdBlock + threadIdx.x) * VEC;
    if (col0 >= c) break;
    if (VEC > 1 && col0 + VEC <= c) {
      Vec<T, VEC> w;
#pragma unroll
      for (int k = 0; k < VEC; ++k) w.v[k] = zero;
      if (active && t >= col0 && t < col0 + VEC) w.v[t - col0] = gval;
      st_stream(reinterpret_cast<Vec<T, VEC>*>(dst + col0), w);
    } else {
      for (int k = 0; k < VEC && col0 + k < c; ++k) dst[col0 + k] = (active && col0 + k == t) ? gval : zero;
    }
  }
}

// ------------------------------------------------------- spatial (2d)
constexpr int kNll2dParts = 512;  // partial (value, weight) pairs of the forward

// Row i of the [n * s] target is image i / s, position i % s; its selected
// log-probability is logp[(i / s) * c * s + t * s + i % s].
template <typename T, typename ACC>
__global__ void __launch_bounds__(kBlock)
k_nll2d_fwd_partial(const T* __restrict__ logp, const int64_t* __restrict__ target, const T* __restrict__ weight,
                    int64_t rows, int64_t c, int64_t s, int64_t ignore_index, int none, T* __restrict__ out,
                    ACC* __restrict__ ws, int32_t* error_flag) {
  __shared__ ACC lds_v[kBlock / 64];
  __shared__ ACC lds_w[kBlock / 64];
  ACC v = ACC(0), w = ACC(0);
  bool bad = false;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < rows; i += (int64_t)gridDim.x * kBlock) {
    const int64_t t = target[i];
    if (t == ignore_index || t < 0 || t >= c) {
      bad = bad || t != ignore_index;
      if (none) out[i] = from_arith<T>(ACC(0));
      continue;
    }
    const int64_t img = i / s, pos = i - img * s;
    const ACC wt = weight ? (ACC)to_arith(weight[t]) : ACC(1);
    const ACC term = -wt * (ACC)to_arith(logp[(img * c + t) * s + pos]);
    if (none) {
      out[i] = from_arith<T>(term);
    } else {
      v += term;
      w += wt;
    }
  }
  if (bad && error_flag) *error_flag = 1;
  if (none) return;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    v += __shfl_xor(v, off, 64);
    w += __shfl_xor(w, off, 64);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    lds_v[wave] = v;
    lds_w[wave] = w;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    ACC sv = ACC(0), sw = ACC(0);
#pragma unroll
    for (int k = 0; k < kBlock / 64; ++k) {
      sv += lds_v[k];
      sw += lds_w[k];
    }
    ws[2 * blockIdx.x] = sv;
    ws[2 * blockIdx.x + 1] = sw;
  }
}

// Stage 2: one wavefront adds the partials in a fixed order.
template <typename T, typename ACC>
__global__ void __launch_bounds__(64)
k_nll2d_fwd_final(const ACC* __restrict__ ws, int nparts, int mean, T* __restrict__ out, T* __restrict__ total_weight) {
  ACC v = ACC(0), w = ACC(0);
  constexpr int U = kNll2dParts / 64;  // every partial's load in flight at once
  ACC pv[U], pw[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int k = threadIdx.x + 64 * u;
    pv[u] = k < nparts ? ws[2 * k] : ACC(0);
    pw[u] = k < nparts ? ws[2 * k + 1] : ACC(0);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (threadIdx.x + 64 * u < nparts) {
      v += pv[u];
      w += pw[u];
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    v += __shfl_xor(v, off, 64);
    w += __shfl_xor(w, off, 64);
  }
  if (threadIdx.x == 0) {
    total_weight[0] = from_arith<T>(w);
    out[0] = from_arith<T>(mean ? v / w : v);
  }
}

// grad_in [n, c, s], one VEC-wide vector along s per thread (s % VEC == 0;
// VEC = 1 otherwise).  The element (img, k, pos) is the gradient when
// target[img, pos] == k, else zero.
template <typename T, int VEC>
__global__ void __launch_bounds__(kBlock)
k_nll2d_bwd(const T* __restrict__ grad_out, const int64_t* __restrict__ target, const T* __restrict__ weight,
            const T* __restrict__ total_weight, uint32_t nvec, FastDiv vps, FastDiv cdiv, int64_t s,
            int reduction, int64_t ignore_index, T* __restrict__ gin, int32_t* error_flag) {
  using C = opmath_t<T>;
  const uint32_t v = blockIdx.x * kBlock + threadIdx.x;
  if (v >= nvec) return;
  uint32_t nc, sv, img, k;
  vps.divmod(v, nc, sv);
  cdiv.divmod(nc, img, k);
  const int64_t c = cdiv.d;
  const int64_t pos0 = (int64_t)sv * VEC;
  C gsc = C(0);
  if (reduction == SUPA_AMD_REDUCTION_MEAN) gsc = (C)to_arith(grad_out[0]) / (C)to_arith(total_weight[0]);
  else if (reduction == SUPA_AMD_REDUCTION_SUM) gsc = (C)to_arith(grad_out[0]);
  const C wk = weight ? (C)to_arith(weight[k]) : C(1);
  Vec<T, VEC> o;
  bool bad = false;
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    const int64_t r = (int64_t)img * s + pos0 + j;
    const int64_t t = target[r];
    bad = bad || (t != ignore_index && (t < 0 || t >= c));
    C val = C(0);
    if (t == (int64_t)k && t != ignore_index) {
      const C g = reduction == SUPA_AMD_REDUCTION_NONE ? (C)to_arith(grad_out[r]) : gsc;
      const T gs = from_arith<T>(-g);  // rounded to the storage type, as upstream forms it
      val = weight ? wk * (C)to_arith(gs) : (C)to_arith(gs);
    }
    o.v[j] = from_arith<T>(val);
  }
  if (bad && k == 0 && error_flag) *error_flag = 1;
  T* dst = gin + ((int64_t)nc * s + pos0);
  if constexpr (VEC > 1) st_stream(reinterpret_cast<Vec<T, VEC>*>(dst), o);
  else dst[0] = o.v[0];
}

template <typename F>
int with_nll_storage(int dtype, F&& f) {
  switch (dtype) {
    case SUPA_AMD_F32: return f((float*)nullptr);
    case SUPA_AMD_BF16: return f((bf16*)nullptr);
    case SUPA_AMD_F16: return f((f16*)nullptr);
    case SUPA_AMD_F64: return f((double*)nullptr);
    default: return SUPA_AMD_EDTYPE;
  }
}

}  // namespace sa

using namespace sa;

extern "C" {

int supa_amd_nll_loss_forward(const void* logp, int32_t dtype, const int64_t* target, const void* weight, int64_t n,
                              int64_t c, int reduction, int64_t ignore_index, void* out, void* total_weight,
                              int32_t* error_flag, void* stream) {
  if ((!logp && n > 0) || (!target && n > 0) || !out || n < 0 || c < 0) return SUPA_AMD_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_nll_storage(dtype, [&](auto* tag) -> int {
    using T = std::remove_pointer_t<decltype(tag)>;
    using ACC = typename std::conditional<std::is_same<T, double>::value, double, float>::type;
    const T* lp = static_cast<const T*>(logp);
    const T* w = static_cast<const T*>(weight);
    if (reduction == SUPA_AMD_REDUCTION_NONE) {
      if (n == 0) return SUPA_AMD_OK;
      k_nll_fwd_none<T><<<(unsigned)((n + kBlock - 1) / kBlock), kBlock, 0, st>>>(lp, target, w, n, c, ignore_index,
                                                                                   static_cast<T*>(out), error_flag);
      return launch_status();
    }
    if (reduction != SUPA_AMD_REDUCTION_MEAN && reduction != SUPA_AMD_REDUCTION_SUM) return SUPA_AMD_EINVAL;
    if (!total_weight) return SUPA_AMD_EINVAL;
    k_nll_fwd_reduce<T, ACC><<<1, kNllBlock, 0, st>>>(lp, target, w, n, c, ignore_index,
                                                      reduction == SUPA_AMD_REDUCTION_MEAN ? 1 : 0, static_cast<T*>(out),
                                                      static_cast<T*>(total_weight), error_flag);
    return launch_status();
  });
}

int supa_amd_nll_loss_backward(const void* grad_out, int32_t dtype, const int64_t* target, const void* weight,
                               const void* total_weight, int64_t n, int64_t c, int reduction, int64_t ignore_index,
                               void* grad_in, int32_t* error_flag, void* stream) {
  if (n < 0 || c < 0 || n >= 65536ll * 65536ll) return SUPA_AMD_EINVAL;
  if (n == 0 || c == 0) return SUPA_AMD_OK;
  if (!grad_out || !target || !grad_in) return SUPA_AMD_EINVAL;
  if (reduction == SUPA_AMD_REDUCTION_MEAN && !total_weight) return SUPA_AMD_EINVAL;
  if (n > 2147483647ll) return SUPA_AMD_ELAYOUT;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_nll_storage(dtype, [&](auto* tag) -> int {
    using T = std::remove_pointer_t<decltype(tag)>;
    constexpr int VEC = 16 / sizeof(T);
    const bool vec_ok = (c % VEC) == 0 && aligned(grad_in, 16);
    const T* g = static_cast<const T*>(grad_out);
    const T* w = static_cast<const T*>(weight);
    const T* tw = static_cast<const T*>(total_weight);
    T* gi = static_cast<T*>(grad_in);
    if (n > 65535) {
      // grid.y is limited; launch in row slabs
      for (int64_t r0 = 0; r0 < n; r0 += 65535) {
        const int64_t rows = std::min<int64_t>(65535, n - r0);
        const T* gslab = reduction == SUPA_AMD_REDUCTION_NONE ? g + r0 : g;
        if (vec_ok) {
          dim3 grid((unsigned)((c / VEC + kNllBwdBlock * kNllUnroll - 1) / (kNllBwdBlock * kNllUnroll)), (unsigned)rows);
          k_nll_bwd<T, VEC><<<grid, kNllBwdBlock, 0, st>>>(gslab, target + r0, w, tw, c, reduction, ignore_index,
                                                      gi + r0 * c, error_flag);
        } else {
          dim3 grid((unsigned)((c + kNllBwdBlock * kNllUnroll - 1) / (kNllBwdBlock * kNllUnroll)), (unsigned)rows);
          k_nll_bwd<T, 1><<<grid, kNllBwdBlock, 0, st>>>(gslab, target + r0, w, tw, c, reduction, ignore_index,
                                                    gi + r0 * c, error_flag);
        }
        const int rc = launch_status();
        if (rc) return rc;
      }
      return SUPA_AMD_OK;
    }
    if (vec_ok) {
      dim3 grid((unsigned)((c / VEC + kNllBwdBlock * kNllUnroll - 1) / (kNllBwdBlock * kNllUnroll)), (unsigned)n);
      k_nll_bwd<T, VEC><<<grid, kNllBwdBlock, 0, st>>>(g, target, w, tw, c, reduction, ignore_index, gi, error_flag);
    } else {
      dim3 grid((unsigned)((c + kNllBwdBlock * kNllUnroll - 1) / (kNllBwdBlock * kNllUnroll)), (unsigned)n);
      k_nll_bwd<T, 1><<<grid, kNllBwdBlock, 0, st>>>(g, target, w, tw, c, reduction, ignore_index, gi, error_flag);
    }
    return launch_status();
  });
}

int64_t supa_amd_nll_loss2d_workspace_bytes(void) { return 2 * kNll2dParts * (int64_t)sizeof(double); }

int supa_amd_nll_loss2d_forward(const void* logp, int32_t dtype, const int64_t* target, const void* weight,
                                int64_t n, int64_t c, int64_t s, int reduction, int64_t ignore_index, void* out,
                                void* total_weight, void* workspace, int64_t ws_bytes, int32_t* error_flag,
                                void* stream) {
  if (n < 0 || c < 0 || s < 0 || !out) return SUPA_AMD_EINVAL;
  const int64_t rows = n * s;
  if (rows > 0 && (!logp || !target)) return SUPA_AMD_EINVAL;
  const bool none = reduction == SUPA_AMD_REDUCTION_NONE;
  if (!none && reduction != SUPA_AMD_REDUCTION_MEAN && reduction != SUPA_AMD_REDUCTION_SUM) return SUPA_AMD_EINVAL;
  if (!none && !total_weight) return SUPA_AMD_EINVAL;
  if (!none && (!workspace || ws_bytes < supa_amd_nll_loss2d_workspace_bytes())) return SUPA_AMD_EWORKSPACE;
  if (none && rows == 0) return SUPA_AMD_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_nll_storage(dtype, [&](auto* tag) -> int {
    using T = std::remove_pointer_t<decltype(tag)>;
    using ACC = typename std::conditional<std::is_same<T, double>::value, double, float>::type;
    const int parts = (int)std::max<int64_t>(1, std::min<int64_t>(kNll2dParts, (rows + kBlock - 1) / kBlock));
    ACC* ws = static_cast<ACC*>(workspace);
    k_nll2d_fwd_partial<T, ACC><<<parts, kBlock, 0, st>>>(static_cast<const T*>(logp), target,
                                                          static_cast<const T*>(weight), rows, c, s, ignore_index,
                                                          none ? 1 : 0, static_cast<T*>(out), ws, error_flag);
    int rc = launch_status();
    if (rc || none) return rc;
    k_nll2d_fwd_final<T, ACC><<<1, 64, 0, st>>>(ws, parts, reduction == SUPA_AMD_REDUCTION_MEAN ? 1 : 0,
                                                static_cast<T*>(out), static_cast<T*>(total_weight));
    return launch_status();
  });
}

int supa_amd_nll_loss2d_backward(const void* grad_out, int32_t dtype, const int64_t* target, const void* weight,
                                 const void* total_weight, int64_t n, int64_t c, int64_t s, int reduction,
                                 int64_t ignore_index, void* grad_in, int32_t* error_flag, void* stream) {
  if (n < 0 || c < 0 || s < 0) return SUPA_AMD_EINVAL;
  if (n == 0 || c == 0 || s == 0) return SUPA_AMD_OK;
  if (!grad_out || !target || !grad_in) return SUPA_AMD_EINVAL;
  if (reduction != SUPA_AMD_REDUCTION_NONE && reduction != SUPA_AMD_REDUCTION_MEAN &&
      reduction != SUPA_AMD_REDUCTION_SUM)
    return SUPA_AMD_EINVAL;
  if (reduction == SUPA_AMD_REDUCTION_MEAN && !total_weight) return SUPA_AMD_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_nll_storage(dtype, [&](auto* tag) -> int {
    using T = std::remove_pointer_t<decltype(tag)>;
    constexpr int VEC = 16 / sizeof(T);
    const bool vec_ok = (s % VEC) == 0 && aligned(grad_in, 16);
    const int64_t per = vec_ok ? s / VEC : s;  // vectors per (image, class) row
    const int64_t nvec = n * c * per;
    // 32-bit magic division: every quotient and dividend below 2^31
    if (nvec >= (int64_t(1) << 31) || per >= (int64_t(1) << 31) || c >= (int64_t(1) << 31)) return SUPA_AMD_ELAYOUT;
    const T* g = static_cast<const T*>(grad_out);
    const T* w = static_cast<const T*>(weight);
    const T* tw = static_cast<const T*>(total_weight);
    T* gi = static_cast<T*>(grad_in);
    const unsigned grid = (unsigned)((nvec + kBlock - 1) / kBlock);
    if (vec_ok)
      k_nll2d_bwd<T, VEC><<<grid, kBlock, 0, st>>>(g, target, w, tw, (uint32_t)nvec, FastDiv((uint32_t)per),
                                                    FastDiv((uint32_t)c), s, reduction, ignore_index, gi, error_flag);
    else
      k_nll2d_bwd<T, 1><<<grid, kBlock, 0, st>>>(g, target, w, tw, (uint32_t)nvec, FastDiv((uint32_t)per),
                                                  FastDiv((uint32_t)c), s, reduction, ignore_index, gi, error_flag);
    return launch_status();
  });
}

}  // extern "C"
