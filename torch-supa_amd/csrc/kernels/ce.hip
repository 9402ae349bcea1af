// Fused cross-entropy over a contiguous [n, c] logit matrix with int64
// targets and ignore_index: the forward reads the logits once and keeps one
// float32 log-sum-exp per row; the backward reads the logits once more and
// writes grad = (softmax - onehot) * g in one pass.  12 N C bytes of the
// log_softmax + nll_loss decomposition (bf16) become 6 N C.
//
// Forward, per row (one 256-thread workgroup; rows in a grid of n):
//   each thread folds its 16-byte vectors into an online (max, sum exp) pair,
//   pairs combine across the wavefront and the workgroup, lse = m + log(s),
//   loss = lse - x[t] in float32.  Rows whose target is ignore_index get
//   loss 0 and are not counted.  Stage 2 (one workgroup): the sum over rows
//   in a fixed order, and for mean the division by the kept-row count (NaN
//   for none, as CrossEntropyLossKernel.cu:67 / :191-193 of the reference).
// Backward, per (row, 16-byte vector) thread: g_i * (exp(x - lse_i) - [j == t_i]).
//
// Out-of-range targets set *error_flag (when given); their rows count as
// ignored.
//
// Probability targets (a float [n, c] target of the logits' dtype, the
// reference's other fp32 fast-path case): the forward reads logits and
// target once each, folds per thread an online (max m, sum of exp(x - m) s,
// sum of t T, sum of t (x - m) B) state, combines it across the workgroup and
// writes loss = T log(s) - B = sum_j t_j (lse - x_j) with lse and T saved per
// row; the backward writes g_i (exp(x - lse_i) T_i - t) in one pass.
#include "devmath.h"
#include "ew_launch.h"

namespace sa {

constexpr int kCeBlock = 256;
// The backward is a pure stream (one vector in, one out per thread): one
// wavefront per workgroup, as the elementwise kernels.
constexpr int kCeBwdBlock = 64;
constexpr int kCeUnroll = 4;  // 16-byte vectors in flight per thread in the forward
constexpr float kCeLog2e = 1.44269504088896340736f;

template <typename T> struct CeVec {
  static constexpr int V = 16 / sizeof(T);
};

template <typename T>
__device__ __forceinline__ float ce_elem(const uint4& w, int k) {
  if constexpr (std::is_same<T, float>::value) {
    return __uint_as_float(k == 0 ? w.x : (k == 1 ? w.y : (k == 2 ? w.z : w.w)));
  } else {
    const int wi = k >> 1;
    const uint32_t u = wi == 0 ? w.x : (wi == 1 ? w.y : (wi == 2 ? w.z : w.w));
    const uint32_t h = (k & 1) ? (u >> 16) : (u & 0xffffu);
    if constexpr (std::is_same<T, bf16>::value) return __uint_as_float(h << 16);
    else return (float)__builtin_bit_cast(f16, (uint16_t)h);
  }
}

// (m, s) (+) (m2, s2) with s relative to m; a pair with m = -inf has s = 0.
__device__ __forceinline__ void ce_combine(float& m, float& s, float m2, float s2) {
  const float M = fmaxf(m, m2);
  if (M != -__builtin_inff())
    s = s * __builtin_amdgcn_exp2f((m - M) * kCeLog2e) + s2 * __builtin_amdgcn_exp2f((m2 - M) * kCeLog2e);
  m = M;
}

__device__ __forceinline__ bool ce_kept(int64_t t, int64_t c, int64_t ignore_index) {
  return t != ignore_index && t >= 0 && t < c;
}

// loss_rows[i] (float32): the row's loss, 0 for an ignored row.  lse[i]: the
// row's log-sum-exp (0 for an ignored row).  out_none (may be null): the loss
// in the logits dtype, for reduction 'none'.
// VECOK: rows are 16-byte aligned and c % V == 0, so rows stream as 16-byte
// vectors; otherwise every element takes the scalar path.
template <typename T, bool VECOK>
__global__ void __launch_bounds__(kCeBlock)
k_ce_fwd(const T* __restrict__ x, const int64_t* __restrict__ target, int64_t c, int64_t ignore_index,
         float* __restrict__ loss_rows, float* __restrict__ lse, T* __restrict__ out_none, int32_t* error_flag) {
  constexpr int V = CeVec<T>::V;
  constexpr int NW = kCeBlock / 64;
  __shared__ float lds_m[NW];
  __shared__ float lds_s[NW];
  const int64_t row = blockIdx.x;
  const int64_t t = target[row];
  if (!ce_kept(t, c, ignore_index)) {
    if (threadIdx.x == 0) {
      if (t != ignore_index && error_flag) *error_flag = 1;
      loss_rows[row] = 0.0f;
      lse[row] = 0.0f;
      if (out_none) out_none[row] = from_arith<T>(0.0f);
    }
    return;
  }
  const T* xr = x + row * c;
  const uint4* src = reinterpret_cast<const uint4*>(xr);
  const int64_t nvec = VECOK ? c / V : 0;
  float m = -__builtin_inff(), s = 0.0f;
  for (int64_t v0 = threadIdx.x; v0 < nvec; v0 += (int64_t)kCeBlock * kCeUnroll) {
    uint4 w[kCeUnroll];
#pragma unroll
    for (int u = 0; u < kCeUnroll; ++u) {
      const int64_t v = v0 + (int64_t)u * kCeBlock;
      if (v < nvec) w[u] = ld_stream(src + v);
    }
    float mb = -__builtin_inff();
#pragma unroll
    for (int u = 0; u < kCeUnroll; ++u) {
      if (v0 + (int64_t)u * kCeBlock < nvec) {
#pragma unroll
        for (int k = 0; k < V; ++k) mb = fmaxf(mb, ce_elem<T>(w[u], k));
      }
    }
    const float M = fmaxf(m, mb);
    if (M != -__builtin_inff()) {
      float sb = 0.0f;
#pragma unroll
      for (int u = 0; u < kCeUnroll; ++u) {
        if (v0 + (int64_t)u * kCeBlock < nvec) {
#pragma unroll
          for (int k = 0; k < V; ++k) sb += __builtin_amdgcn_exp2f((ce_elem<T>(w[u], k) - M) * kCeLog2e);
        }
      }
      s = s * __builtin_amdgcn_exp2f((m - M) * kCeLog2e) + sb;
      m = M;
    }
  }
  // elements not covered by whole vectors (all of them when !VECOK)
  for (int64_t j = nvec * V + threadIdx.x; j < c; j += kCeBlock) {
    const float xv = (float)to_arith(xr[j]);
    ce_combine(m, s, xv, 1.0f);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ce_combine(m, s, __shfl_xor(m, off, 64), __shfl_xor(s, off, 64));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    lds_m[wave] = m;
    lds_s[wave] = s;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float M = lds_m[0], S = lds_s[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) ce_combine(M, S, lds_m[w], lds_s[w]);
    const float l = M + sa_logf(S);
    const float loss = l - (float)to_arith(xr[t]);
    loss_rows[row] = loss;
    lse[row] = l;
    if (out_none) out_none[row] = from_arith<T>(loss);
  }
}

// Stage 2: sum of the row losses and the kept-row count, fixed order
// (target null: every row counts, the probability-target form).
template <typename T>
__global__ void __launch_bounds__(kCeBlock)
k_ce_final(const float* __restrict__ loss_rows, const int64_t* __restrict__ target, int64_t n, int64_t c,
           int64_t ignore_index, int mean, T* __restrict__ out, float* __restrict__ count) {
  constexpr int NW = kCeBlock / 64;
  __shared__ float lds_v[NW];
  __shared__ float lds_c[NW];
  float v = 0.0f, k = 0.0f;
  constexpr int U = 8;  // loads in flight per step; the sums keep the row order
  for (int64_t i0 = threadIdx.x; i0 < n; i0 += (int64_t)U * kCeBlock) {
    float lv[U];
    int64_t tg[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = i0 + (int64_t)u * kCeBlock;
      lv[u] = i < n ? loss_rows[i] : 0.0f;
      tg[u] = i < n && target ? target[i] : ignore_index;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (i0 + (int64_t)u * kCeBlock < n) {
        v += lv[u];
        k += (!target || ce_kept(tg[u], c, ignore_index)) ? 1.0f : 0.0f;
      }
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    v += __shfl_xor(v, off, 64);
    k += __shfl_xor(k, off, 64);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    lds_v[wave] = v;
    lds_c[wave] = k;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float sv = 0.0f, sk = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      sv += lds_v[w];
      sk += lds_c[w];
    }
    out[0] = from_arith<T>(mean ? sv / sk : sv);  // 0/0 = NaN for a mean over no rows
    if (count) count[0] = sk;
  }
}

// grad[i, :] over a 2-d grid: blockIdx.y = row in the slab, x = column blocks
// of kCeBwdBlock vectors.  VECOK (c % V == 0, aligned rows: every vector is
// whole): the logits load goes out unconditionally, before the row's target,
// and the scale and lse that depend on it, have arrived (an ignored row then
// reads logits it does not need); waiting for the target first held the
// kernel at 75 % of the HBM roofline on c3's bf16 rows, against 85 % with the
// load first.
template <typename T, bool VECOK>
__global__ void __launch_bounds__(kCeBwdBlock)
k_ce_bwd(const T* __restrict__ grad_out, const T* __restrict__ x, const int64_t* __restrict__ target,
         const float* __restrict__ lse, const float* __restrict__ count, int64_t c, int64_t ignore_index,
         int reduction, T* __restrict__ gx) {
  constexpr int V = CeVec<T>::V;
  const int64_t row = blockIdx.y;
  const T* xr = x + row * c;
  T* dst = gx + row * c;
  const int64_t col0 = ((int64_t)blockIdx.x * kCeBwdBlock + threadIdx.x) * V;
  if (col0 >= c) return;
  Vec<T, V> w;
  if constexpr (VECOK) w = ld_stream(reinterpret_cast<const Vec<T, V>*>(xr + col0));
  const int64_t t = target[row];
  const bool kept = ce_kept(t, c, ignore_index);
  float g = 0.0f;
  if (kept) {
    if (reduction == SUPA_AMD_REDUCTION_NONE) g = (float)to_arith(grad_out[row]);
    else if (reduction == SUPA_AMD_REDUCTION_MEAN) g = (float)to_arith(grad_out[0]) / count[0];
    else g = (float)to_arith(grad_out[0]);
  }
  const float l = kept ? lse[row] : 0.0f;
  if constexpr (VECOK) {
    // p g everywhere, (p - 1) g at the target: the one thread of the row that
    // holds the target patches its element in a branch, so the other threads
    // spend no compare or select per element (the same values as
    // (p - [j == t]) g; ignored rows, uniform in the workgroup, store zeros)
    Vec<T, V> o;
    if (kept) {
      float p[V];
#pragma unroll
      for (int k = 0; k < V; ++k) p[k] = __builtin_amdgcn_exp2f(((float)to_arith(w.v[k]) - l) * kCeLog2e);
      float r[V];
#pragma unroll
      for (int k = 0; k < V; ++k) r[k] = p[k] * g;
      if ((uint64_t)(t - col0) < (uint64_t)V) {
#pragma unroll
        for (int k = 0; k < V; ++k)
          if (col0 + k == t) r[k] = (p[k] - 1.0f) * g;
      }
#pragma unroll
      for (int k = 0; k < V; ++k) o.v[k] = from_arith<T>(r[k]);
    } else {
#pragma unroll
      for (int k = 0; k < V; ++k) o.v[k] = from_arith<T>(0.0f);
    }
    st_stream(reinterpret_cast<Vec<T, V>*>(dst + col0), o);
  } else {
    for (int k = 0; k < V && col0 + k < c; ++k) {
      float r = 0.0f;
      if (kept) {
        const float p = __builtin_amdgcn_exp2f(((float)to_arith(xr[col0 + k]) - l) * kCeLog2e);
        r = (p - (col0 + k == t ? 1.0f : 0.0f)) * g;
      }
      dst[col0 + k] = from_arith<T>(r);
    }
  }
}

// ------------------------------------------------- probability targets
// Online state of a row: max m, s = sum exp(x - m), T = sum t,
// B = sum t (x - m).  (+) of two states rebases both to M = max(m, m2):
// s -> s e^{m - M}, B -> B + T (m - M).  A state whose elements are all -inf
// keeps m = -inf, s = 0 and B = sum t x (-inf, or NaN where a t is 0), which
// no rebase changes: its elements add t (lse - x) = +inf (or NaN for t = 0)
// to the loss, as -t log_softmax(x) does in the decomposition.
struct CeProbState {
  float m, s, T, B;
};
__device__ __forceinline__ CeProbState ce_prob_elem(float x, float t) {
  if (x == -__builtin_inff()) return CeProbState{x, 0.0f, t, t * x};
  return CeProbState{x, 1.0f, t, 0.0f};
}
__device__ __forceinline__ void ce_prob_combine(CeProbState& a, const CeProbState& b) {
  const float M = fmaxf(a.m, b.m);
  const bool fa = a.m != -__builtin_inff(), fb = b.m != -__builtin_inff();
  const float ea = fa ? __builtin_amdgcn_exp2f((a.m - M) * kCeLog2e) : 0.0f;
  const float eb = fb ? __builtin_amdgcn_exp2f((b.m - M) * kCeLog2e) : 0.0f;
  const float Ba = fa ? fmaf(a.T, a.m - M, a.B) : a.B;
  const float Bb = fb ? fmaf(b.T, b.m - M, b.B) : b.B;
  a.s = a.s * ea + b.s * eb;
  a.B = Ba + Bb;
  a.T = a.T + b.T;
  a.m = M;
}

// loss_rows[i] = T log(s) - B (float32); lse[i] = m + log(s); tsum[i] = T;
// out_none (may be null): the loss in the logits dtype.
template <typename T, bool VECOK>
__global__ void __launch_bounds__(kCeBlock)
k_ce_prob_fwd(const T* __restrict__ x, const T* __restrict__ tgt, int64_t c, float* __restrict__ loss_rows,
              float* __restrict__ lse, float* __restrict__ tsum, T* __restrict__ out_none) {
  constexpr int V = CeVec<T>::V;
  constexpr int NW = kCeBlock / 64;
  constexpr int U = 2;  // vectors of each stream in flight per thread
  __shared__ CeProbState lds[NW];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * c;
  const T* tr = tgt + row * c;
  const uint4* xs = reinterpret_cast<const uint4*>(xr);
  const uint4* ts = reinterpret_cast<const uint4*>(tr);
  const int64_t nvec = VECOK ? c / V : 0;
  CeProbState st{-__builtin_inff(), 0.0f, 0.0f, 0.0f};
  for (int64_t v0 = threadIdx.x; v0 < nvec; v0 += (int64_t)kCeBlock * U) {
    uint4 wx[U], wt[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t v = v0 + (int64_t)u * kCeBlock;
      if (v < nvec) {
        wx[u] = ld_stream(xs + v);
        wt[u] = ld_stream(ts + v);
      }
    }
    float mb = -__builtin_inff();
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (v0 + (int64_t)u * kCeBlock < nvec) {
#pragma unroll
        for (int k = 0; k < V; ++k) mb = fmaxf(mb, ce_elem<T>(wx[u], k));
      }
    const float M = fmaxf(st.m, mb);
    if (M != -__builtin_inff()) {
      if (st.m != -__builtin_inff()) {
        st.s *= __builtin_amdgcn_exp2f((st.m - M) * kCeLog2e);
        st.B = fmaf(st.T, st.m - M, st.B);
      }
      st.m = M;
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (v0 + (int64_t)u * kCeBlock < nvec) {
#pragma unroll
          for (int k = 0; k < V; ++k) {
            const float xv = ce_elem<T>(wx[u], k), tv = ce_elem<T>(wt[u], k);
            st.s += __builtin_amdgcn_exp2f((xv - M) * kCeLog2e);
            st.T += tv;
            st.B = fmaf(tv, xv - M, st.B);
          }
        }
    } else {  // every value so far -inf: s stays 0, B = sum t x
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (v0 + (int64_t)u * kCeBlock < nvec) {
#pragma unroll
          for (int k = 0; k < V; ++k) {
            const float xv = ce_elem<T>(wx[u], k), tv = ce_elem<T>(wt[u], k);
            st.T += tv;
            st.B = fmaf(tv, xv, st.B);
          }
        }
    }
  }
  // elements not covered by whole vectors (all of them when !VECOK)
  for (int64_t j = nvec * V + threadIdx.x; j < c; j += kCeBlock)
    ce_prob_combine(st, ce_prob_elem((float)to_arith(xr[j]), (float)to_arith(tr[j])));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const CeProbState o{__shfl_xor(st.m, off, 64), __shfl_xor(st.s, off, 64), __shfl_xor(st.T, off, 64),
                        __shfl_xor(st.B, off, 64)};
    ce_prob_combine(st, o);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) lds[wave] = st;
  __syncthreads();
  if (threadIdx.x == 0) {
    CeProbState a = lds[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) ce_prob_combine(a, lds[w]);
    const float L = sa_logf(a.s);
    const float loss = fmaf(a.T, L, -a.B);
    loss_rows[row] = loss;
    lse[row] = a.m + L;
    tsum[row] = a.T;
    if (out_none) out_none[row] = from_arith<T>(loss);
  }
}

// grad[i, j] = g_i (exp(x - lse_i) T_i - t_ij); g_i = grad_out[i] (none),
// grad_out[0] (sum) or grad_out[0] / n (mean).
template <typename T, bool VECOK>
__global__ void __launch_bounds__(kCeBwdBlock)
k_ce_prob_bwd(const T* __restrict__ grad_out, const T* __restrict__ x, const T* __restrict__ tgt,
              const float* __restrict__ lse, const float* __restrict__ tsum, int64_t c, int reduction, float inv_n,
              T* __restrict__ gx) {
  constexpr int V = CeVec<T>::V;
  const int64_t row = blockIdx.y;
  float g;
  if (reduction == SUPA_AMD_REDUCTION_NONE) g = (float)to_arith(grad_out[row]);
  else if (reduction == SUPA_AMD_REDUCTION_MEAN) g = (float)to_arith(grad_out[0]) * inv_n;
  else g = (float)to_arith(grad_out[0]);
  const float l = lse[row];
  const float Tr = tsum[row];
  const T* xr = x + row * c;
  const T* tr = tgt + row * c;
  T* dst = gx + row * c;
  const int64_t col0 = ((int64_t)blockIdx.x * kCeBwdBlock + threadIdx.x) * V;
  if (col0 >= c) return;
  if (VECOK && col0 + V <= c) {
    const Vec<T, V> w = ld_stream(reinterpret_cast<const Vec<T, V>*>(xr + col0));
    const Vec<T, V> wt = ld_stream(reinterpret_cast<const Vec<T, V>*>(tr + col0));
    Vec<T, V> o;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const float p = __builtin_amdgcn_exp2f(((float)to_arith(w.v[k]) - l) * kCeLog2e);
      o.v[k] = from_arith<T>(fmaf(p, Tr, -(float)to_arith(wt.v[k])) * g);
    }
    st_stream(reinterpret_cast<Vec<T, V>*>(dst + col0), o);
  } else {
    for (int k = 0; k < V && col0 + k < c; ++k) {
      const float p = __builtin_amdgcn_exp2f(((float)to_arith(xr[col0 + k]) - l) * kCeLog2e);
      dst[col0 + k] = from_arith<T>(fmaf(p, Tr, -(float)to_arith(tr[col0 + k])) * g);
    }
  }
}

template <typename F>
int with_ce_storage(int dtype, F&& f) {
  switch (dtype) {
    case SUPA_AMD_F32: return f((float*)nullptr);
    case SUPA_AMD_BF16: return f((bf16*)nullptr);
    case SUPA_AMD_F16: return f((f16*)nullptr);
    default: return SUPA_AMD_EDTYPE;
  }
}

}  // namespace sa

using namespace sa;

extern "C" {

int64_t supa_amd_cross_entropy_workspace_bytes(int64_t n) { return n > 0 ? 4 * n : 0; }

int supa_amd_cross_entropy_forward(const void* logits, int32_t dtype, const int64_t* target, int64_t n, int64_t c,
                                   int64_t ignore_index, int reduction, void* out, float* lse, float* count,
                                   void* workspace, int64_t workspace_bytes, int32_t* error_flag, void* stream) {
  if (n < 0 || c <= 0 || n >= (int64_t(1) << 31)) return SUPA_AMD_EINVAL;
  if (reduction != SUPA_AMD_REDUCTION_NONE && reduction != SUPA_AMD_REDUCTION_MEAN &&
      reduction != SUPA_AMD_REDUCTION_SUM)
    return SUPA_AMD_EINVAL;
  if (!out || (n > 0 && (!logits || !target || !lse))) return SUPA_AMD_EINVAL;
  if (n > 0 && (!workspace || workspace_bytes < supa_amd_cross_entropy_workspace_bytes(n))) return SUPA_AMD_EWORKSPACE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_ce_storage(dtype, [&](auto* tag) -> int {
    using T = std::remove_pointer_t<decltype(tag)>;
    constexpr int V = CeVec<T>::V;
    float* rows = static_cast<float*>(workspace);
    T* o = static_cast<T*>(out);
    if (n > 0) {
      const T* x = static_cast<const T*>(logits);
      T* on = reduction == SUPA_AMD_REDUCTION_NONE ? o : nullptr;
      if (aligned(logits, 16) && (c % V) == 0)
        k_ce_fwd<T, true><<<(unsigned)n, kCeBlock, 0, st>>>(x, target, c, ignore_index, rows, lse, on, error_flag);
      else
        k_ce_fwd<T, false><<<(unsigned)n, kCeBlock, 0, st>>>(x, target, c, ignore_index, rows, lse, on, error_flag);
      const int rc = launch_status();
      if (rc) return rc;
    }
    if (reduction == SUPA_AMD_REDUCTION_NONE) return SUPA_AMD_OK;
    k_ce_final<T><<<1, kCeBlock, 0, st>>>(rows, target, n, c, ignore_index, reduction == SUPA_AMD_REDUCTION_MEAN ? 1 : 0,
                                          o, count);
    return launch_status();
  });
}

int supa_amd_cross_entropy_backward(const void* grad_out, const void* logits, int32_t dtype, const int64_t* target,
                                    const float* lse, const float* count, int64_t n, int64_t c, int64_t ignore_index,
                                    int reduction, void* grad_logits, int32_t* error_flag, void* stream) {
  (void)error_flag;  // out-of-range targets were flagged by the forward
  if (n < 0 || c <= 0 || n >= (int64_t(1) << 31)) return SUPA_AMD_EINVAL;
  if (n == 0) return SUPA_AMD_OK;
  if (!grad_out || !logits || !target || !lse || !grad_logits) return SUPA_AMD_EINVAL;
  if (reduction == SUPA_AMD_REDUCTION_MEAN && !count) return SUPA_AMD_EINVAL;
  if (reduction != SUPA_AMD_REDUCTION_NONE && reduction != SUPA_AMD_REDUCTION_MEAN &&
      reduction != SUPA_AMD_REDUCTION_SUM)
    return SUPA_AMD_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_ce_storage(dtype, [&](auto* tag) -> int {
    using T = std::remove_pointer_t<decltype(tag)>;
    constexpr int V = CeVec<T>::V;
    const bool vecok = aligned(logits, 16) && aligned(grad_logits, 16) && (c % V) == 0;
    const T* g = static_cast<const T*>(grad_out);
    const T* x = static_cast<const T*>(logits);
    T* gx = static_cast<T*>(grad_logits);
    const unsigned gx_blocks = (unsigned)((c + (int64_t)kCeBwdBlock * V - 1) / ((int64_t)kCeBwdBlock * V));
    for (int64_t r0 = 0; r0 < n; r0 += 65535) {
      const int64_t rows = std::min<int64_t>(65535, n - r0);
      const T* gs = reduction == SUPA_AMD_REDUCTION_NONE ? g + r0 : g;
      const dim3 grid(gx_blocks, (unsigned)rows);
      if (vecok)
        k_ce_bwd<T, true><<<grid, kCeBwdBlock, 0, st>>>(gs, x + r0 * c, target + r0, lse + r0, count, c, ignore_index,
                                                     reduction, gx + r0 * c);
      else
        k_ce_bwd<T, false><<<grid, kCeBwdBlock, 0, st>>>(gs, x + r0 * c, target + r0, lse + r0, count, c, ignore_index,
                                                      reduction, gx + r0 * c);
      const int rc = launch_status();
      if (rc) return rc;
    }
    return SUPA_AMD_OK;
  });
}

int supa_amd_cross_entropy_prob_forward(const void* logits, const void* target, int32_t dtype, int64_t n, int64_t c,
                                        int reduction, void* out, float* lse, float* tsum, void* workspace,
                                        int64_t workspace_bytes, void* stream) {
  if (n < 0 || c <= 0 || n >= (int64_t(1) << 31)) return SUPA_AMD_EINVAL;
  if (reduction != SUPA_AMD_REDUCTION_NONE && reduction != SUPA_AMD_REDUCTION_MEAN &&
      reduction != SUPA_AMD_REDUCTION_SUM)
    return SUPA_AMD_EINVAL;
  if (!out || (n > 0 && (!logits || !target || !lse || !tsum))) return SUPA_AMD_EINVAL;
  if (n > 0 && (!workspace || workspace_bytes < supa_amd_cross_entropy_workspace_bytes(n))) return SUPA_AMD_EWORKSPACE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_ce_storage(dtype, [&](auto* tag) -> int {
    using T = std::remove_pointer_t<decltype(tag)>;
    constexpr int V = CeVec<T>::V;
    float* rows = static_cast<float*>(workspace);
    T* o = static_cast<T*>(out);
    if (n > 0) {
      const T* x = static_cast<const T*>(logits);
      const T* t = static_cast<const T*>(target);
      T* on = reduction == SUPA_AMD_REDUCTION_NONE ? o : nullptr;
      if (aligned(logits, 16) && aligned(target, 16) && (c % V) == 0)
        k_ce_prob_fwd<T, true><<<(unsigned)n, kCeBlock, 0, st>>>(x, t, c, rows, lse, tsum, on);
      else
        k_ce_prob_fwd<T, false><<<(unsigned)n, kCeBlock, 0, st>>>(x, t, c, rows, lse, tsum, on);
      const int rc = launch_status();
      if (rc) return rc;
    }
    if (reduction == SUPA_AMD_REDUCTION_NONE) return SUPA_AMD_OK;
    k_ce_final<T><<<1, kCeBlock, 0, st>>>(rows, nullptr, n, c, 0, reduction == SUPA_AMD_REDUCTION_MEAN ? 1 : 0, o,
                                          nullptr);
    return launch_status();
  });
}

int supa_amd_cross_entropy_prob_backward(const void* grad_out, const void* logits, const void* target, int32_t dtype,
                                         const float* lse, const float* tsum, int64_t n, int64_t c, int reduction,
                                         void* grad_logits, void* stream) {
  if (n < 0 || c <= 0 || n >= (int64_t(1) << 31)) return SUPA_AMD_EINVAL;
  if (n == 0) return SUPA_AMD_OK;
  if (!grad_out || !logits || !target || !lse || !tsum || !grad_logits) return SUPA_AMD_EINVAL;
  if (reduction != SUPA_AMD_REDUCTION_NONE && reduction != SUPA_AMD_REDUCTION_MEAN &&
      reduction != SUPA_AMD_REDUCTION_SUM)
    return SUPA_AMD_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_ce_storage(dtype, [&](auto* tag) -> int {
    using T = std::remove_pointer_t<decltype(tag)>;
    constexpr int V = CeVec<T>::V;
    const bool vecok = aligned(logits, 16) && aligned(target, 16) && aligned(grad_logits, 16) && (c % V) == 0;
    const T* g = static_cast<const T*>(grad_out);
    const T* x = static_cast<const T*>(logits);
    const T* t = static_cast<const T*>(target);
    T* gx = static_cast<T*>(grad_logits);
    const float inv_n = 1.0f / (float)n;
    const unsigned gx_blocks = (unsigned)((c + (int64_t)kCeBwdBlock * V - 1) / ((int64_t)kCeBwdBlock * V));
    for (int64_t r0 = 0; r0 < n; r0 += 65535) {
      const int64_t rows = std::min<int64_t>(65535, n - r0);
      const T* gs = reduction == SUPA_AMD_REDUCTION_NONE ? g + r0 : g;
      const dim3 grid(gx_blocks, (unsigned)rows);
      if (vecok)
        k_ce_prob_bwd<T, true><<<grid, kCeBwdBlock, 0, st>>>(gs, x + r0 * c, t + r0 * c, lse + r0, tsum + r0, c,
                                                          reduction, inv_n, gx + r0 * c);
      else
        k_ce_prob_bwd<T, false><<<grid, kCeBwdBlock, 0, st>>>(gs, x + r0 * c, t + r0 * c, lse + r0, tsum + r0, c,
                                                           reduction, inv_n, gx + r0 * c);
      const int rc = launch_status();
      if (rc) return rc;
    }
    return SUPA_AMD_OK;
  });
}

}  // extern "C"
