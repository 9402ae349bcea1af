// Multi-tensor apply kernels of the optimizer step: the fused AdamW update and
// the mixed-precision unscale / loss-scale update beside it.  Each workgroup
// owns one chunk of one tensor (mta.h) -- one 16-byte vector of each operand
// per thread, all loads of a vector issued before the math.  Tensors whose
// base is not 16-byte aligned, and the last partial vector of a tensor, take
// a scalar path.  The reference's counterpart is the adam_math functor of
// upstream fused_adam_utils.cuh and AmpKernels.cu over MultiTensorApply.cuh.
#include "mta.h"
#include "ops.h"

namespace sa {

// ----------------------------------------------------------- fused AdamW
struct AdamTable {
  void* p[kMtaTensors];
  void* g[kMtaTensors];
  void* m[kMtaTensors];
  void* v[kMtaTensors];
  void* vmax[kMtaTensors];
  const float* step[kMtaTensors];
  int64_t numel[kMtaTensors];
  uint32_t chunk_start[kMtaTensors + 1];
  int32_t ntensors;
  uint32_t bucket_shift;
  MtaBucket bucket[kMtaBuckets];
};

struct AdamHyper {
  double lr, beta1, beta2, weight_decay, eps;
  const float* lr_ptr;
  const float* grad_scale;
  const float* found_inf;
  int amsgrad, maximize;
  int l2;  // 1: Adam (weight decay added to the gradient), 0: AdamW (decoupled)
};

// beta^step for integral step counts by square-and-multiply in double (the
// state_steps tensors hold 1, 2, 3, ... as float); pow() otherwise.
__device__ __forceinline__ double pow_steps(double beta, float step) {
  const uint64_t k = (uint64_t)step;
  if ((float)k != step) return pow(beta, (double)step);
  double r = 1.0, b = beta;
  uint64_t e = k;
  while (e) {
    if (e & 1u) r *= b;
    b *= b;
    e >>= 1;
  }
  return r;
}

// One element of upstream adam_math in ADAMW mode (ORIGINAL mode with h.l2)
// (torch/include/ATen/native/cuda/fused_adam_utils.cuh:27-93): hyper-parameters
// in double, state in the storage type's opmath (float), each mixed
// expression evaluated in double and rounded once.
template <typename T>
__device__ __forceinline__ void adamw_elem(T& pr, T& gr, T& mr, T& vr, T* vmx, const AdamHyper& h, double lr,
                                           double lr_wd, float bc1, float bc2_sqrt, float step_size) {
  using C = opmath_t<T>;
  C param = (C)to_arith(pr);
  C grad = (C)to_arith(gr);
  if (h.grad_scale) grad = (C)((double)grad / (double)(*h.grad_scale));
  const C grad_to_store = grad;
  if (h.maximize) grad = -grad;
  C ea = (C)to_arith(mr);
  C eas = (C)to_arith(vr);
  if (h.weight_decay != 0.0) {
    if (h.l2) grad = (C)((double)grad + (double)param * h.weight_decay);  // ADAM_MODE::ORIGINAL
    else param = (C)fma(-lr_wd, (double)param, (double)param);
  }
  ea = (C)fma(h.beta1, (double)ea, (1.0 - h.beta1) * (double)grad);
  eas = (C)fma(h.beta2, (double)eas, ((1.0 - h.beta2) * (double)grad) * (double)grad);
  C denom;
  if (h.amsgrad) {
    C mx = (C)to_arith(*vmx);
    mx = mx > eas ? mx : eas;
    *vmx = from_arith<T>(mx);
    denom = (C)((double)(sqrt(mx) / (C)bc2_sqrt) + h.eps);
  } else {
    denom = (C)((double)(sqrt(eas) / (C)bc2_sqrt) + h.eps);
  }
  param = param - ((C)step_size * ea) / denom;
  pr = from_arith<T>(param);
  if (h.grad_scale) gr = from_arith<T>(grad_to_store);
  mr = from_arith<T>(ea);
  vr = from_arith<T>(eas);
}

template <typename T, int64_t CHUNK, int UNR>
__global__ void __launch_bounds__(kMtaBlock)
k_adamw(AdamTable tab, AdamHyper h) {
  if (h.found_inf && *h.found_inf == 1.0f) return;
  constexpr int V = 16 / sizeof(T);
  const MtaRange r = mta_range<CHUNK>(tab);
  const int k = r.k;
  const int64_t lo = r.lo, hi = r.hi;
  const double lr = h.lr_ptr ? (double)(*h.lr_ptr) : h.lr;
  const float step = *tab.step[k];
  const float bc1 = (float)(1.0 - pow_steps(h.beta1, step));
  const float bc2_sqrt = (float)sqrt(1.0 - pow_steps(h.beta2, step));
  const float step_size = (float)(lr / (double)bc1);
  const double lr_wd = lr * h.weight_decay;
  T* p = static_cast<T*>(tab.p[k]);
  T* g = static_cast<T*>(tab.g[k]);
  T* m = static_cast<T*>(tab.m[k]);
  T* v = static_cast<T*>(tab.v[k]);
  T* vm = static_cast<T*>(tab.vmax[k]);
  const bool vec = !h.amsgrad && aligned(p, 16) && aligned(g, 16) && aligned(m, 16) && aligned(v, 16);
  int64_t start = lo;
  if (vec) {
    const int64_t nv = (hi - lo) / V;
    for (int64_t i0 = threadIdx.x; i0 < nv; i0 += kMtaBlock * UNR) {
      Vec<T, V> P[UNR], G[UNR], M[UNR], W[UNR];
#pragma unroll
      for (int u = 0; u < UNR; ++u) {
        const int64_t i = i0 + u * kMtaBlock;
        if (i < nv) {
          const int64_t e = lo + i * V;
          P[u] = ld_stream(reinterpret_cast<const Vec<T, V>*>(p + e));
          G[u] = ld_stream(reinterpret_cast<const Vec<T, V>*>(g + e));
          M[u] = ld_stream(reinterpret_cast<const Vec<T, V>*>(m + e));
          W[u] = ld_stream(reinterpret_cast<const Vec<T, V>*>(v + e));
        }
      }
#pragma unroll
      for (int u = 0; u < UNR; ++u) {
        const int64_t i = i0 + u * kMtaBlock;
        if (i < nv) {
          const int64_t e = lo + i * V;
#pragma unroll
          for (int j = 0; j < V; ++j)
            adamw_elem<T>(P[u].v[j], G[u].v[j], M[u].v[j], W[u].v[j], nullptr, h, lr, lr_wd, bc1, bc2_sqrt, step_size);
          st_stream(reinterpret_cast<Vec<T, V>*>(p + e), P[u]);
          if (h.grad_scale) st_stream(reinterpret_cast<Vec<T, V>*>(g + e), G[u]);
          st_stream(reinterpret_cast<Vec<T, V>*>(m + e), M[u]);
          st_stream(reinterpret_cast<Vec<T, V>*>(v + e), W[u]);
        }
      }
    }
    start = lo + nv * V;
  }
  for (int64_t e = start + threadIdx.x; e < hi; e += kMtaBlock)
    adamw_elem<T>(p[e], g[e], m[e], v[e], h.amsgrad ? vm + e : nullptr, h, lr, lr_wd, bc1, bc2_sqrt, step_size);
}

// AdamW / Adam (what torch.optim.AdamW(fused=True) runs, also with amsgrad,
// maximize, a device lr and under GradScaler; Adam's weight decay under
// maximize takes k_adamw): the same arithmetic
// as adamw_elem with the configuration fixed at compile time (MODE 0: AdamW
// with weight decay, 1: Adam with weight decay, 2: no weight decay; GS, AMS
// below), so the four elements of a vector are straight-line code, and one
// division fewer per element: sqrt(v) / bc2_sqrt, a float32 quotient by a
// per-tensor constant c, is rounded from the binary64 product
// sqrt(v) * RN64(1 / c).  That product is within 2^-52 (relative) of the
// exact quotient, and a quotient of two binary32 numbers that is not a
// binary32 midpoint lies at least 2^-49 (relative) from every midpoint, so
// the rounding to binary32 is the IEEE quotient's, for every c in
// [2^-60, 1] (a normal-range quotient; other c take the division).  The
// wave runs at raised priority while it issues its loads (as k_contig's
// heavy functors).
// One vector of each stream per thread: two (with the loads of both issued
// first) measured 60 % of the HBM roofline against 74-75 % at c5.
constexpr int kAdamPlainUnroll = 1;

// GS: grad_scale and found_inf given (GradScaler's AMP step): the gradient is
// divided by the scale (the binary64 quotient rounded once: the IEEE float32
// quotient) and stored back, and a step with found_inf set changes nothing.
// AMS: amsgrad, the running maximum of exp_avg_sq in max_exp_avg_sq.  As
// adamw_elem's arithmetic for those switches.
template <int MODE, bool GS, bool AMS>
__device__ __forceinline__ void adamw_plain_elem(float& param, float& grad, float& ea, float& eas, float& mx,
                                                 double lr_wd, double wd, double beta1, double omb1, double beta2,
                                                 double omb2, double eps, float c, double rc, bool exact_rc,
                                                 float step_size, float scale) {
  if constexpr (GS) grad = (float)((double)grad / (double)scale);
  float gr = grad;  // `grad` is what GS stores back; the update uses gr
  if constexpr (MODE == 0) param = (float)fma(-lr_wd, (double)param, (double)param);
  if constexpr (MODE == 1) gr = (float)((double)gr + (double)param * wd);
  ea = (float)fma(beta1, (double)ea, omb1 * (double)gr);
  eas = (float)fma(beta2, (double)eas, (omb2 * (double)gr) * (double)gr);
  float vv = eas;
  if constexpr (AMS) {
    mx = mx > eas ? mx : eas;
    vv = mx;
  }
  const float sq = sqrtf(vv);
  const float q = exact_rc ? (float)((double)sq * rc) : sq / c;
  const float denom = (float)((double)q + eps);
  param = param - (step_size * ea) / denom;
}

// The per-tensor constants of a step (from the tensor's device step count).
struct AdamStepConst {
  float bc2_sqrt, step_size;
  double lr_wd, omb1, omb2, rc;
  bool exact_rc;
};
// maximize negates the gradient the update uses; outside Adam's weight decay
// (which adds to that gradient first) the gradient enters the step only
// through (1 - beta1) g and the sign-free g g, and (-(1 - beta1)) g rounds
// to exactly -((1 - beta1) g), so maximize is the sign of omb1.
__device__ __forceinline__ AdamStepConst adam_step_const(const AdamHyper& h, float step) {
  AdamStepConst c;
  const double lr = h.lr_ptr ? (double)(*h.lr_ptr) : h.lr;
  const float bc1 = (float)(1.0 - pow_steps(h.beta1, step));
  c.bc2_sqrt = (float)sqrt(1.0 - pow_steps(h.beta2, step));
  c.step_size = (float)(lr / (double)bc1);
  c.lr_wd = lr * h.weight_decay;
  c.omb1 = h.maximize ? -(1.0 - h.beta1) : 1.0 - h.beta1;
  c.omb2 = 1.0 - h.beta2;
  c.exact_rc = c.bc2_sqrt >= 0x1p-60f && c.bc2_sqrt <= 1.0f;
  c.rc = 1.0 / (double)c.bc2_sqrt;
  return c;
}

template <int MODE, bool GS, bool AMS, typename T>
__device__ __forceinline__ void adamw_plain_one(T& p, T& g, T& m, T& v, T& x, const AdamHyper& h,
                                                const AdamStepConst& c, float scale) {
  float pp = (float)to_arith(p), gg = (float)to_arith(g), ea = (float)to_arith(m), eas = (float)to_arith(v);
  float mx = AMS ? (float)to_arith(x) : 0.0f;
  adamw_plain_elem<MODE, GS, AMS>(pp, gg, ea, eas, mx, c.lr_wd, h.weight_decay, h.beta1, c.omb1, h.beta2, c.omb2,
                                  h.eps, c.bc2_sqrt, c.rc, c.exact_rc, c.step_size, scale);
  p = from_arith<T>(pp);
  if constexpr (GS) g = from_arith<T>(gg);
  m = from_arith<T>(ea);
  v = from_arith<T>(eas);
  if constexpr (AMS) x = from_arith<T>(mx);
}

// A full, aligned chunk issues its loads before it reads the step count (and
// found_inf / grad_scale) and computes the bias corrections (a chain of
// dependent scalar loads and binary64 arithmetic), so the loads are in flight
// meanwhile; a step with found_inf set then returns before any store.
template <typename T, int64_t CHUNK, int MODE, int UNR, bool GS, bool AMS>
__global__ void __launch_bounds__(kMtaBlock)
k_adamw_plain(AdamTable tab, AdamHyper h) {
  constexpr int V = 16 / sizeof(T);
  const MtaRange r = mta_range<CHUNK>(tab);
  const int k = r.k;
  const int64_t lo = r.lo, hi = r.hi;
  T* p = static_cast<T*>(tab.p[k]);
  T* g = static_cast<T*>(tab.g[k]);
  T* m = static_cast<T*>(tab.m[k]);
  T* v = static_cast<T*>(tab.v[k]);
  T* x = static_cast<T*>(tab.vmax[k]);
  const bool vec = aligned(p, 16) && aligned(g, 16) && aligned(m, 16) && aligned(v, 16) && (!AMS || aligned(x, 16));
  const int64_t nv = (hi - lo) / V;  // at most UNR * kMtaBlock vectors
  if (vec && nv == (int64_t)UNR * kMtaBlock) {  // a full chunk: no guards
    Vec<T, V> P[UNR], G[UNR], M[UNR], W[UNR], X[AMS ? UNR : 1];
    __builtin_amdgcn_s_setprio(3);
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int64_t e = lo + (threadIdx.x + (int64_t)u * kMtaBlock) * V;
      P[u] = ld_stream(reinterpret_cast<const Vec<T, V>*>(p + e));
      G[u] = ld_stream(reinterpret_cast<const Vec<T, V>*>(g + e));
      M[u] = ld_stream(reinterpret_cast<const Vec<T, V>*>(m + e));
      W[u] = ld_stream(reinterpret_cast<const Vec<T, V>*>(v + e));
      if constexpr (AMS) X[u] = ld_stream(reinterpret_cast<const Vec<T, V>*>(x + e));
    }
    __builtin_amdgcn_s_setprio(0);
    if constexpr (GS) {
      if (*h.found_inf == 1.0f) return;
    }
    const float scale = GS ? *h.grad_scale : 1.0f;
    const AdamStepConst c = adam_step_const(h, *tab.step[k]);
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int64_t e = lo + (threadIdx.x + (int64_t)u * kMtaBlock) * V;
#pragma unroll
      for (int j = 0; j < V; ++j)
        adamw_plain_one<MODE, GS, AMS, T>(P[u].v[j], G[u].v[j], M[u].v[j], W[u].v[j], X[AMS ? u : 0].v[j], h, c,
                                          scale);
      st_stream(reinterpret_cast<Vec<T, V>*>(p + e), P[u]);
      if constexpr (GS) st_stream(reinterpret_cast<Vec<T, V>*>(g + e), G[u]);
      st_stream(reinterpret_cast<Vec<T, V>*>(m + e), M[u]);
      st_stream(reinterpret_cast<Vec<T, V>*>(v + e), W[u]);
      if constexpr (AMS) st_stream(reinterpret_cast<Vec<T, V>*>(x + e), X[u]);
    }
    return;
  }
  if constexpr (GS) {
    if (*h.found_inf == 1.0f) return;
  }
  const float scale = GS ? *h.grad_scale : 1.0f;
  const AdamStepConst c = adam_step_const(h, *tab.step[k]);
  int64_t start = lo;
  if (vec) {
    for (int64_t i = threadIdx.x; i < nv; i += kMtaBlock) {
      const int64_t e = lo + i * V;
      Vec<T, V> P = ld_stream(reinterpret_cast<const Vec<T, V>*>(p + e));
      Vec<T, V> G = ld_stream(reinterpret_cast<const Vec<T, V>*>(g + e));
      Vec<T, V> M = ld_stream(reinterpret_cast<const Vec<T, V>*>(m + e));
      Vec<T, V> W = ld_stream(reinterpret_cast<const Vec<T, V>*>(v + e));
      Vec<T, V> X;
      if constexpr (AMS) X = ld_stream(reinterpret_cast<const Vec<T, V>*>(x + e));
#pragma unroll
      for (int j = 0; j < V; ++j)
        adamw_plain_one<MODE, GS, AMS, T>(P.v[j], G.v[j], M.v[j], W.v[j], X.v[j], h, c, scale);
      st_stream(reinterpret_cast<Vec<T, V>*>(p + e), P);
      if constexpr (GS) st_stream(reinterpret_cast<Vec<T, V>*>(g + e), G);
      st_stream(reinterpret_cast<Vec<T, V>*>(m + e), M);
      st_stream(reinterpret_cast<Vec<T, V>*>(v + e), W);
      if constexpr (AMS) st_stream(reinterpret_cast<Vec<T, V>*>(x + e), X);
    }
    start = lo + nv * V;
  }
  for (int64_t e = start + threadIdx.x; e < hi; e += kMtaBlock) {
    if constexpr (AMS) {
      adamw_plain_one<MODE, GS, AMS, T>(p[e], g[e], m[e], v[e], x[e], h, c, scale);
    } else {
      T unused = T{};
      adamw_plain_one<MODE, GS, AMS, T>(p[e], g[e], m[e], v[e], unused, h, c, scale);
    }
  }
}

// ------------------------------------------------------------- fused SGD
struct SgdTable {
  void* p[kMtaTensors];
  void* g[kMtaTensors];
  void* b[kMtaTensors];
  int64_t numel[kMtaTensors];
  uint32_t chunk_start[kMtaTensors + 1];
  int32_t ntensors;
  uint32_t bucket_shift;
  MtaBucket bucket[kMtaBuckets];
};

struct SgdHyper {
  double weight_decay, momentum, lr, dampening;
  const float* lr_ptr;
  const float* grad_scale;
  const float* found_inf;
  int nesterov, maximize, first;
};

// One element of upstream sgd_math (FusedSgdKernel.cu): the state in the
// storage type's opmath, the hyper-parameters in double, so every mixed
// expression is evaluated in double (a + b c contracted into one fma, as that
// compiler does) and rounded once.  MOM: a momentum buffer (depth 3).
//   g = g / grad_scale (stored back); -g if maximize; g += wd p;
//   buf = first ? g : momentum buf + (1 - dampening) g;
//   g = nesterov ? g + momentum buf : buf;  p -= lr g
// The double buf feeds the nesterov step before it is rounded for storage.
template <typename T, bool MOM>
__device__ __forceinline__ void sgd_elem(T& pr, T& gr, T* br, const SgdHyper& h, double lr) {
  using C = opmath_t<T>;
  C p = (C)to_arith(pr);
  C g = (C)to_arith(gr);
  if (h.grad_scale) {
    g = (C)((double)g / (double)(*h.grad_scale));
    gr = from_arith<T>(g);
  }
  if (h.maximize) g = -g;
  if (h.weight_decay != 0.0) g = (C)fma(h.weight_decay, (double)p, (double)g);
  if constexpr (MOM) {
    const double buf =
        h.first ? (double)g : fma(h.momentum, (double)(C)to_arith(*br), (1.0 - h.dampening) * (double)g);
    *br = from_arith<T>((C)buf);
    g = h.nesterov ? (C)fma(h.momentum, buf, (double)g) : (C)buf;
  }
  p = (C)fma(-lr, (double)g, (double)p);
  pr = from_arith<T>(p);
}

template <typename T, bool MOM, int64_t CHUNK>
__global__ void __launch_bounds__(kMtaBlock)
k_sgd(SgdTable tab, SgdHyper h) {
  if (h.found_inf && *h.found_inf == 1.0f) return;
  constexpr int V = 16 / sizeof(T);
  const MtaRange r = mta_range<CHUNK>(tab);
  const int k = r.k;
  const int64_t lo = r.lo, hi = r.hi;
  const double lr = h.lr_ptr ? (double)(*h.lr_ptr) : h.lr;
  T* p = static_cast<T*>(tab.p[k]);
  T* g = static_cast<T*>(tab.g[k]);
  T* b = static_cast<T*>(tab.b[k]);
  const bool vec = aligned(p, 16) && aligned(g, 16) && (!MOM || aligned(b, 16));
  int64_t start = lo;
  if (vec) {
    const int64_t nv = (hi - lo) / V;
    for (int64_t i = threadIdx.x; i < nv; i += kMtaBlock) {
      const int64_t e = lo + i * V;
      Vec<T, V> P = ld_stream(reinterpret_cast<const Vec<T, V>*>(p + e));
      Vec<T, V> G = ld_stream(reinterpret_cast<const Vec<T, V>*>(g + e));
      Vec<T, V> B;
      if constexpr (MOM) {
        if (!h.first) B = ld_stream(reinterpret_cast<const Vec<T, V>*>(b + e));
      }
#pragma unroll
      for (int j = 0; j < V; ++j) sgd_elem<T, MOM>(P.v[j], G.v[j], &B.v[j], h, lr);
      st_stream(reinterpret_cast<Vec<T, V>*>(p + e), P);
      if (h.grad_scale) st_stream(reinterpret_cast<Vec<T, V>*>(g + e), G);
      if constexpr (MOM) st_stream(reinterpret_cast<Vec<T, V>*>(b + e), B);
    }
    start = lo + nv * V;
  }
  for (int64_t e = start + threadIdx.x; e < hi; e += kMtaBlock) sgd_elem<T, MOM>(p[e], g[e], b + e, h, lr);
}

// ------------------------------------------------------------ AMP
// In-place unscale of a gradient list with the non-finite check of upstream
// _amp_foreach_non_finite_check_and_unscale_ (AmpKernels.cu): each element is
// widened to opmath, *found_inf becomes 1 if it is inf or NaN, and it is
// multiplied by *inv_scale unless that is exactly 1.  Every writer of
// *found_inf stores the same 1.0f.
struct UnscaleTable {
  void* x[kMtaTensors];
  int64_t numel[kMtaTensors];
  uint32_t chunk_start[kMtaTensors + 1];
  int32_t ntensors;
  uint32_t bucket_shift;
  MtaBucket bucket[kMtaBuckets];
};

template <typename T, int64_t CHUNK>
__global__ void __launch_bounds__(kMtaBlock)
k_amp_unscale(UnscaleTable tab, float* __restrict__ found_inf, const float* __restrict__ inv_scale) {
  using C = opmath_t<T>;
  constexpr int V = 16 / sizeof(T);
  const MtaRange r = mta_range<CHUNK>(tab);
  const int64_t lo = r.lo, hi = r.hi;
  T* x = static_cast<T*>(tab.x[r.k]);
  const C inv = (C)*inv_scale;
  bool bad = false;
  auto f = [&](C v) -> C {
    bad = bad || !isfinite(v);
    return inv == C(1) ? v : v * inv;
  };
  int64_t start = lo;
  if (aligned(x, 16)) {
    const int64_t nv = (hi - lo) / V;
    for (int64_t i = threadIdx.x; i < nv; i += kMtaBlock) {
      Vec<T, V> w = ld_stream(reinterpret_cast<const Vec<T, V>*>(x + lo + i * V));
#pragma unroll
      for (int j = 0; j < V; ++j) w.v[j] = from_arith<T>(f((C)to_arith(w.v[j])));
      st_stream(reinterpret_cast<Vec<T, V>*>(x + lo + i * V), w);
    }
    start = lo + nv * V;
  }
  for (int64_t e = start + threadIdx.x; e < hi; e += kMtaBlock) x[e] = from_arith<T>(f((C)to_arith(x[e])));
  if (bad) *found_inf = 1.0f;
}

// Loss-scale update of upstream _amp_update_scale_ (AmpKernels.cu): one thread.
__global__ void k_amp_update_scale(float* scale, int32_t* growth_tracker, const float* found_inf, double growth,
                                   double backoff, int64_t interval) {
  // products in double, rounded once to float, as upstream's float * double
  if (*found_inf) {
    *scale = (float)((double)(*scale) * backoff);
    *growth_tracker = 0;
  } else {
    const int64_t successful = (int64_t)(*growth_tracker) + 1;
    if (successful == interval) {
      const float grown = (float)((double)(*scale) * growth);
      if (isfinite(grown)) *scale = grown;
      *growth_tracker = 0;
    } else {
      *growth_tracker = (int32_t)successful;
    }
  }
}

template <typename T, int64_t CHUNK, int UNR>
int launch_adamw(int32_t ntensors, void* const* params, void* const* grads, void* const* exp_avgs,
                 void* const* exp_avg_sqs, void* const* max_exp_avg_sqs, void* const* state_steps,
                 const int64_t* numel, const AdamHyper& h, hipStream_t st) {
  return mta_for_tables<CHUNK, AdamTable>(
      ntensors, numel,
      [&](AdamTable& tab, int slot, int i) -> int {
        if (!state_steps[i]) return SUPA_AMD_EINVAL;
        tab.p[slot] = params[i];
        tab.g[slot] = grads[i];
        tab.m[slot] = exp_avgs[i];
        tab.v[slot] = exp_avg_sqs[i];
        tab.vmax[slot] = h.amsgrad ? max_exp_avg_sqs[i] : nullptr;
        tab.step[slot] = static_cast<const float*>(state_steps[i]);
        return SUPA_AMD_OK;
      },
      [&](const AdamTable& tab, uint32_t chunks) { k_adamw<T, CHUNK, UNR><<<chunks, kMtaBlock, 0, st>>>(tab, h); });
}

// Dynamic LDS (unused by the kernel) that caps a long plain-AdamW launch at
// 16 resident one-wave workgroups per CU: with all 32 the seven streams'
// requests contend in HBM (c5: 74.8 % of the roofline at 32, 77.5 % at 16
// with the bias corrections first, 80.3 % with the loads first; 13 or fewer
// lose again).  Short launches keep the full occupancy.
constexpr unsigned kAdamCapLds = 9728;
inline unsigned adam_occupancy_lds(uint32_t chunks) { return chunks >= (1u << 16) ? kAdamCapLds : 0u; }

// The plain configurations (k_adamw_plain): PU vectors per thread, chunks of
// PU * kMtaBlock vectors.
template <typename T, int PU>
int launch_adamw_plain(int32_t ntensors, void* const* params, void* const* grads, void* const* exp_avgs,
                       void* const* exp_avg_sqs, void* const* max_exp_avg_sqs, void* const* state_steps,
                       const int64_t* numel, const AdamHyper& h, hipStream_t st) {
  constexpr int64_t CHUNK = chunk_one<T>() * PU;
  return mta_for_tables<CHUNK, AdamTable>(
      ntensors, numel,
      [&](AdamTable& tab, int slot, int i) -> int {
        if (!state_steps[i]) return SUPA_AMD_EINVAL;
        tab.p[slot] = params[i];
        tab.g[slot] = grads[i];
        tab.m[slot] = exp_avgs[i];
        tab.v[slot] = exp_avg_sqs[i];
        tab.vmax[slot] = h.amsgrad ? max_exp_avg_sqs[i] : nullptr;
        tab.step[slot] = static_cast<const float*>(state_steps[i]);
        return SUPA_AMD_OK;
      },
      [&](const AdamTable& tab, uint32_t chunks) {
        const unsigned lds = adam_occupancy_lds(chunks);
        const int mode = h.weight_decay == 0.0 ? 2 : (h.l2 ? 1 : 0);
        const bool gs = h.grad_scale != nullptr, ams = h.amsgrad != 0;
        auto go = [&](auto mode_c, auto gs_c, auto ams_c) {
          k_adamw_plain<T, CHUNK, decltype(mode_c)::value, PU, decltype(gs_c)::value, decltype(ams_c)::value>
              <<<chunks, kMtaBlock, lds, st>>>(tab, h);
        };
        auto by_flags = [&](auto mode_c) {
          if (gs && ams) go(mode_c, std::true_type{}, std::true_type{});
          else if (gs) go(mode_c, std::true_type{}, std::false_type{});
          else if (ams) go(mode_c, std::false_type{}, std::true_type{});
          else go(mode_c, std::false_type{}, std::false_type{});
        };
        if (mode == 2) by_flags(std::integral_constant<int, 2>{});
        else if (mode == 1) by_flags(std::integral_constant<int, 1>{});
        else by_flags(std::integral_constant<int, 0>{});
      });
}

template <typename T, bool MOM>
int launch_sgd(int32_t ntensors, void* const* params, void* const* grads, void* const* bufs, const int64_t* numel,
               const SgdHyper& h, hipStream_t st) {
  constexpr int64_t CHUNK = chunk_one<T>();
  return mta_for_tables<CHUNK, SgdTable>(
      ntensors, numel,
      [&](SgdTable& tab, int slot, int i) -> int {
        if (MOM && !bufs[i]) return SUPA_AMD_EINVAL;
        tab.p[slot] = params[i];
        tab.g[slot] = grads[i];
        tab.b[slot] = MOM ? bufs[i] : nullptr;
        return SUPA_AMD_OK;
      },
      [&](const SgdTable& tab, uint32_t chunks) {
        // with a momentum buffer (three address streams, five accesses) long
        // launches run at 20 workgroups per CU (c5's tensors: 79.5 -> 81 %)
        const unsigned lds = MOM && chunks >= (1u << 16) ? 8192u : 0u;
        k_sgd<T, MOM, CHUNK><<<chunks, kMtaBlock, lds, st>>>(tab, h);
      });
}

}  // namespace sa

using namespace sa;

extern "C" {

int supa_amd_fused_sgd(int32_t ntensors, void* const* params, void* const* grads, void* const* momentum_buffers,
                       const int64_t* numel, int32_t dtype, double weight_decay, double momentum, double lr,
                       const float* lr_ptr, double dampening, int nesterov, int maximize, int is_first_step,
                       const float* grad_scale, const float* found_inf, void* stream) {
  if (ntensors < 0) return SUPA_AMD_EINVAL;
  if (ntensors > 0 && (!params || !grads || !numel)) return SUPA_AMD_EINVAL;
  const bool mom = momentum_buffers != nullptr;
  // upstream: a momentum buffer list exactly when momentum > 0
  if (mom ? !(momentum > 0.0) : momentum != 0.0) return SUPA_AMD_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const SgdHyper h{weight_decay, momentum, lr, dampening, lr_ptr, grad_scale, found_inf,
                   nesterov ? 1 : 0, maximize ? 1 : 0, is_first_step ? 1 : 0};
  return with_mta_storage(dtype, [&](auto* tag) -> int {
    using T = std::remove_pointer_t<decltype(tag)>;
    return mom ? launch_sgd<T, true>(ntensors, params, grads, momentum_buffers, numel, h, st)
               : launch_sgd<T, false>(ntensors, params, grads, nullptr, numel, h, st);
  });
}

int supa_amd_amp_unscale(int32_t ntensors, void* const* tensors, const int64_t* numel, int32_t dtype,
                         float* found_inf, const float* inv_scale, void* stream) {
  if (ntensors < 0 || (ntensors > 0 && (!tensors || !numel || !found_inf || !inv_scale))) return SUPA_AMD_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_mta_storage(dtype, [&](auto* tag) -> int {
    using T = std::remove_pointer_t<decltype(tag)>;
    constexpr int64_t CHUNK = chunk_one<T>();
    return mta_for_tables<CHUNK, UnscaleTable>(
        ntensors, numel,
        [&](UnscaleTable& tab, int slot, int i) -> int {
          tab.x[slot] = tensors[i];
          return SUPA_AMD_OK;
        },
        [&](const UnscaleTable& tab, uint32_t chunks) {
          k_amp_unscale<T, CHUNK><<<chunks, kMtaBlock, 0, st>>>(tab, found_inf, inv_scale);
        });
  });
}

int supa_amd_amp_update_scale(float* scale, int32_t* growth_tracker, const float* found_inf, double growth_factor,
                              double backoff_factor, int64_t growth_interval, void* stream) {
  if (!scale || !growth_tracker || !found_inf) return SUPA_AMD_EINVAL;
  k_amp_update_scale<<<1, 1, 0, static_cast<hipStream_t>(stream)>>>(scale, growth_tracker, found_inf, growth_factor,
                                                                     backoff_factor, growth_interval);
  return launch_status();
}

}  // extern "C"

namespace {
int fused_adam_any(int l2, int32_t ntensors, void* const* params, void* const* grads, void* const* exp_avgs,
                   void* const* exp_avg_sqs, void* const* max_exp_avg_sqs, void* const* state_steps,
                   const int64_t* numel, int32_t dtype, double lr, const float* lr_ptr, double beta1, double beta2,
                   double weight_decay, double eps, int amsgrad, int maximize, const float* grad_scale,
                   const float* found_inf, void* stream) {
  if (ntensors < 0) return SUPA_AMD_EINVAL;
  if (ntensors > 0 && (!params || !grads || !exp_avgs || !exp_avg_sqs || !state_steps || !numel)) return SUPA_AMD_EINVAL;
  if (amsgrad && ntensors > 0 && !max_exp_avg_sqs) return SUPA_AMD_EINVAL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const AdamHyper h{lr,        beta1,      beta2,     weight_decay,          eps, lr_ptr,
                    grad_scale, found_inf, amsgrad ? 1 : 0, maximize ? 1 : 0, l2};
  // the plain kernel: grad_scale and found_inf together or neither
  // (GradScaler passes both), and not maximize with Adam's weight decay
  // (the plain kernel folds maximize into the sign of 1 - beta1)
  const bool plain = !(maximize && l2 && weight_decay != 0.0) && (grad_scale == nullptr) == (found_inf == nullptr);
  return with_mta_storage(dtype, [&](auto* tag) -> int {
    using T = std::remove_pointer_t<decltype(tag)>;
    if constexpr (!std::is_same<T, double>::value) {
      if (plain)
        return launch_adamw_plain<T, kAdamPlainUnroll>(ntensors, params, grads, exp_avgs, exp_avg_sqs,
                                                       max_exp_avg_sqs, state_steps, numel, h, st);
    }
    return launch_adamw<T, chunk_one<T>(), 1>(ntensors, params, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, state_steps, numel,
                                   h, st);
  });
}
}  // namespace

extern "C" {

int supa_amd_fused_adamw(int32_t ntensors, void* const* params, void* const* grads, void* const* exp_avgs,
                         void* const* exp_avg_sqs, void* const* max_exp_avg_sqs, void* const* state_steps,
                         const int64_t* numel, int32_t dtype, double lr, const float* lr_ptr, double beta1,
                         double beta2, double weight_decay, double eps, int amsgrad, int maximize,
                         const float* grad_scale, const float* found_inf, void* stream) {
  return fused_adam_any(0, ntensors, params, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, state_steps, numel,
                        dtype, lr, lr_ptr, beta1, beta2, weight_decay, eps, amsgrad, maximize, grad_scale, found_inf,
                        stream);
}

int supa_amd_fused_adam(int32_t ntensors, void* const* params, void* const* grads, void* const* exp_avgs,
                        void* const* exp_avg_sqs, void* const* max_exp_avg_sqs, void* const* state_steps,
                        const int64_t* numel, int32_t dtype, double lr, const float* lr_ptr, double beta1,
                        double beta2, double weight_decay, double eps, int amsgrad, int maximize,
                        const float* grad_scale, const float* found_inf, void* stream) {
  return fused_adam_any(1, ntensors, params, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs, state_steps, numel,
                        dtype, lr, lr_ptr, beta1, beta2, weight_decay, eps, amsgrad, maximize, grad_scale, found_inf,
                        stream);
}

}  // extern "C"
