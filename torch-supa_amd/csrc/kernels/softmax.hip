// log_softmax and softmax, forward and backward, over the last dim of a
// contiguous [rows, cols] tensor.
//
// Main path (16-byte aligned rows of up to 1024 threads x VPT vectors): one
// 1024-thread workgroup per row holds the whole row in registers, so the
// forward reads the row once and writes it once, and the backward reads grad
// and output once each and writes once -- the HBM minimum for these aten ops.
// Row statistics: per-thread partials, a 64-lane butterfly inside each
// wavefront, then the 16 wavefront results through LDS (the forward combines
// (max, sum) pairs in one exchange and walks rows with a persistent grid).  exp() of the row
// statistics uses the hardware base-2 exponential on a pre-scaled argument;
// the row results are rounded to bf16/f16 (or kept in f32) exactly once.
//
// Fallback (any cols, any alignment): one 256-thread workgroup per row,
// online max/sum in a first pass over memory, the output in a second pass.
//
// Replaces _log_softmax.out (NF:3752), _log_softmax_backward_data.out
// (NF:3763), _softmax.out and _softmax_backward_data.out, upstream SoftMax.cu /
// PersistentSoftmax.cuh in the reference's operator library.  softmax's
// epilogue is exp(x - max) * (1 / sum) and its gradient y (g - sum(g y)).
#include "devmath.h"
#include "ew_launch.h"

namespace sa {

constexpr int kRowBlock = 1024;
constexpr float kLog2e = 1.44269504088896340736f;

__device__ __forceinline__ float fast_exp(float x) {
  // e^x = 2^(x * log2 e); v_exp_f32 for the power of two
  return __builtin_amdgcn_exp2f(x * kLog2e);
}

// NaN-propagating max (a NaN anywhere in the row makes the row NaN, as the
// upstream kernels' results are).
__device__ __forceinline__ float nmax(float a, float b) { return (a != a || b != b) ? __builtin_nanf("") : fmaxf(a, b); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = nmax(v, __shfl_xor(v, off, 64));
  return v;
}
template <typename ACC>
__device__ __forceinline__ ACC wave_sum(ACC v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Block-wide reductions returning the result to every thread.  `lds` holds
// one slot per wavefront; NW = blockDim / 64.
template <int NW>
__device__ __forceinline__ float block_max_all(float v, float* lds) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) lds[wave] = v;
  __syncthreads();
  float r = lds[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) r = nmax(r, lds[w]);
  return r;
}
template <int NW>
__device__ __forceinline__ float block_sum_all(float v, float* lds) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) lds[wave] = v;
  __syncthreads();
  float r = lds[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) r += lds[w];
  return r;
}

template <typename T> struct VecOf {
  static constexpr int V = 16 / sizeof(T);
  using type = Vec<T, V>;
};

// The register-resident kernels keep each 16-byte vector as four raw 32-bit
// words and widen an element to float only where it is used; an empty asm
// statement between phases tells the compiler the words may have changed, so
// it never keeps a second, unpacked copy of the row alive (which would spill).
__device__ __forceinline__ uint32_t word_of(const uint4& w, int i) {
  return i == 0 ? w.x : (i == 1 ? w.y : (i == 2 ? w.z : w.w));
}

template <typename T>
__device__ __forceinline__ float elem_f(const uint4& w, int k) {
  if constexpr (std::is_same<T, float>::value) {
    return __uint_as_float(word_of(w, k));
  } else {
    const uint32_t word = word_of(w, k >> 1);
    const uint32_t h = (k & 1) ? (word >> 16) : (word & 0xffffu);
    if constexpr (std::is_same<T, bf16>::value) {
      return __uint_as_float(h << 16);
    } else {
      return (float)__builtin_bit_cast(f16, (uint16_t)h);
    }
  }
}

template <int VPT>
__device__ __forceinline__ void opaque(uint4 (&x)[VPT]) {
#pragma unroll
  for (int j = 0; j < VPT; ++j) asm volatile("" : "+v"(x[j].x), "+v"(x[j].y), "+v"(x[j].z), "+v"(x[j].w));
}

// Row results: 16-byte vectors of TO built from V floats.  bf16 pairs go
// through the gfx950 packed convert (round to nearest even; a NaN keeps its
// NaN-ness, its payload may differ from c10's canonical 0x7FC0).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));

template <typename TO, int V>
__device__ __forceinline__ void store_row_vec(Vec<TO, V>* dst, int v, const float (&f)[V]) {
  if constexpr (std::is_same<TO, bf16>::value) {
    uint32_t w[V / 2];
#pragma unroll
    for (int k = 0; k < V / 2; ++k) {
      const float2_t p = {f[2 * k], f[2 * k + 1]};
      w[k] = __builtin_bit_cast(uint32_t, __builtin_convertvector(p, bf16x2_t));
    }
    st_stream(reinterpret_cast<Vec<uint32_t, V / 2>*>(dst + v), *reinterpret_cast<const Vec<uint32_t, V / 2>*>(w));
  } else {
    Vec<TO, V> o;
#pragma unroll
    for (int k = 0; k < V; ++k) o.v[k] = from_arith<TO>(f[k]);
    st_stream(dst + v, o);
  }
}

// ------------------------------------------------------------- forward
// Persistent: a fixed grid of kLsmGrid workgroups walks the rows, so the next
// row's loads issue right behind the current row's stores.  Row statistics
// in one pass ("online" softmax): each thread reduces its own elements to
// (m, s) = (max, sum of exp(x - m)), and the pairs are combined across the
// wavefront and the workgroup by (m, s) (+) (m', s') = (M, s e^(m-M) + s' e^(m'-M)),
// M = max(m, m'), which needs one workgroup exchange instead of two.  A NaN
// anywhere in a row turns the row's sum, hence every output of the row, into
// NaN, as in the upstream kernels.
constexpr int kLsmGrid = 512;  // 2 workgroups per CU on MI355X's 256 CUs

// (m, s) (+) (m2, s2); a pair with m = -inf has s = 0 and drops out.
__device__ __forceinline__ void lse_combine(float& m, float& s, float m2, float s2) {
  const float M = fmaxf(m, m2);
  if (M != -__builtin_inff())
    s = s * __builtin_amdgcn_exp2f((m - M) * kLog2e) + s2 * __builtin_amdgcn_exp2f((m2 - M) * kLog2e);
  m = M;
}

template <typename TI, typename TO, int VPT, bool LOG>
__global__ void __launch_bounds__(kRowBlock)
k_lsm_fwd_reg(const TI* __restrict__ in, TO* __restrict__ out, int64_t rows, int64_t cols) {
  constexpr int V = VecOf<TI>::V;
  constexpr int NW = kRowBlock / 64;
  __shared__ float lds_m[NW];
  __shared__ float lds_s[NW];
  const int nvec = (int)(cols / V);
  const int full = nvec / kRowBlock;  // vectors every thread has (uniform)
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const uint4* src = reinterpret_cast<const uint4*>(in + row * cols);
    uint4 x[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      if (j < full) x[j] = ld_stream(src + tid + j * kRowBlock);
      else if (tid + j * kRowBlock < nvec) x[j] = ld_stream(src + tid + j * kRowBlock);
    }
    float m = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      if (j < full || tid + j * kRowBlock < nvec) {
#pragma unroll
        for (int k = 0; k < V; ++k) m = fmaxf(m, elem_f<TI>(x[j], k));
      }
    }
    const float mbl = (m == -__builtin_inff() ? 0.0f : m) * kLog2e;  // all -inf: keep exp args finite
    opaque<VPT>(x);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      if (j < full || tid + j * kRowBlock < nvec) {
#pragma unroll
        for (int k = 0; k < V; ++k) s += __builtin_amdgcn_exp2f(fmaf(elem_f<TI>(x[j], k), kLog2e, -mbl));
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) lse_combine(m, s, __shfl_xor(m, off, 64), __shfl_xor(s, off, 64));
    __syncthreads();  // the previous row's readers are done with the slots
    if (lane == 0) {
      lds_m[wave] = m;
      lds_s[wave] = s;
    }
    __syncthreads();
    float M = lds_m[0], S = lds_s[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) lse_combine(M, S, lds_m[w], lds_s[w]);
    // log: (x - M) - log S;  softmax: 2^(x log2e - M log2e) / S with the
    // scaled max of the sum (an all -inf row gives 0 * inf = NaN, as upstream)
    const float logsum = LOG ? sa_logf(S) : 0.0f;
    const float inv = LOG ? 0.0f : 1.0f / S;
    const float Mb = (M == -__builtin_inff() ? 0.0f : M) * kLog2e;
    opaque<VPT>(x);
    Vec<TO, V>* dst = reinterpret_cast<Vec<TO, V>*>(out + row * cols);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      if (j < full || tid + j * kRowBlock < nvec) {
        float f[V];
#pragma unroll
        for (int k = 0; k < V; ++k) {
          if constexpr (LOG) f[k] = (elem_f<TI>(x[j], k) - M) - logsum;
          else f[k] = __builtin_amdgcn_exp2f(fmaf(elem_f<TI>(x[j], k), kLog2e, -Mb)) * inv;
        }
        store_row_vec<TO, V>(dst, tid + j * kRowBlock, f);
      }
    }
  }
}

// Streaming fallback: any cols.
template <typename TI, typename TO, bool LOG>
__global__ void __launch_bounds__(kBlock)
k_lsm_fwd_stream(const TI* __restrict__ in, TO* __restrict__ out, int64_t cols) {
  __shared__ float lds[kBlock / 64];
  const TI* x = in + (int64_t)blockIdx.x * cols;
  float m = -__builtin_inff();
  for (int64_t c = threadIdx.x; c < cols; c += kBlock) m = nmax(m, (float)to_arith(x[c]));
  m = block_max_all<kBlock / 64>(m, lds);
  const float mb = (m == -__builtin_inff()) ? 0.0f : m;
  float s = 0.0f;
  for (int64_t c = threadIdx.x; c < cols; c += kBlock) s += fast_exp((float)to_arith(x[c]) - mb);
  s = block_sum_all<kBlock / 64>(s, lds);
  TO* o = out + (int64_t)blockIdx.x * cols;
  if constexpr (LOG) {
    const float logsum = sa_logf(s);
    for (int64_t c = threadIdx.x; c < cols; c += kBlock) o[c] = from_arith<TO>(((float)to_arith(x[c]) - m) - logsum);
  } else {
    const float inv = 1.0f / s;
    for (int64_t c = threadIdx.x; c < cols; c += kBlock) o[c] = from_arith<TO>(fast_exp((float)to_arith(x[c]) - mb) * inv);
  }
}

// ------------------------------------------------------------ backward
// grad's row stays in registers (raw words) for the row sum; the output row
// streams through in chunks of CH = 4 vectors with the next chunk's loads
// issued before the current chunk's math (8 vectors in flight per thread; two
// measured 3 % slower).
template <typename TG, typename TO, int VPT>
__global__ void __launch_bounds__(kRowBlock)
k_lsm_bwd_reg(const TG* __restrict__ grad, const TG* __restrict__ outp, TO* __restrict__ gin, int64_t cols) {
  constexpr int V = VecOf<TG>::V;
  constexpr int CH = VPT < 4 ? VPT : 4;
  __shared__ float lds[kRowBlock / 64];
  const int64_t row = blockIdx.x;
  const uint4* g = reinterpret_cast<const uint4*>(grad + row * cols);
  const uint4* y = reinterpret_cast<const uint4*>(outp + row * cols);
  const int nvec = (int)(cols / V);
  const int full = nvec / kRowBlock;
  const int tid = threadIdx.x;
  uint4 gv[VPT];
#pragma unroll
  for (int j = 0; j < VPT; ++j)
    if (j < full || tid + j * kRowBlock < nvec) gv[j] = ld_stream(g + tid + j * kRowBlock);
  uint4 yv[CH];
#pragma unroll
  for (int j = 0; j < CH; ++j)
    if (j < full || tid + j * kRowBlock < nvec) yv[j] = ld_stream(y + tid + j * kRowBlock);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    if (j < full || tid + j * kRowBlock < nvec) {
#pragma unroll
      for (int k = 0; k < V; ++k) s += elem_f<TG>(gv[j], k);
    }
  }
  s = block_sum_all<kRowBlock / 64>(s, lds);
  opaque<VPT>(gv);
  Vec<TO, V>* dst = reinterpret_cast<Vec<TO, V>*>(gin + row * cols);
#pragma unroll
  for (int c = 0; c < VPT; c += CH) {
    uint4 yn[CH];
    if (c + CH < VPT) {
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        const int jj = c + CH + j;
        if (jj < full || tid + jj * kRowBlock < nvec) yn[j] = ld_stream(y + tid + jj * kRowBlock);
      }
    }
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int jj = c + j;
      if (jj < full || tid + jj * kRowBlock < nvec) {
        float f[V];
#pragma unroll
        for (int k = 0; k < V; ++k)
          f[k] = fmaf(-__builtin_amdgcn_exp2f(elem_f<TG>(yv[j], k) * kLog2e), s, elem_f<TG>(gv[jj], k));
        store_row_vec<TO, V>(dst, tid + jj * kRowBlock, f);
      }
    }
    if (c + CH < VPT) {
#pragma unroll
      for (int j = 0; j < CH; ++j) yv[j] = yn[j];
    }
  }
}

template <typename TG, typename TO>
__global__ void __launch_bounds__(kBlock)
k_lsm_bwd_stream(const TG* __restrict__ grad, const TG* __restrict__ outp, TO* __restrict__ gin, int64_t cols) {
  __shared__ float lds[kBlock / 64];
  const int64_t base = (int64_t)blockIdx.x * cols;
  float s = 0.0f;
  for (int64_t c = threadIdx.x; c < cols; c += kBlock) s += (float)to_arith(grad[base + c]);
  s = block_sum_all<kBlock / 64>(s, lds);
  for (int64_t c = threadIdx.x; c < cols; c += kBlock)
    gin[base + c] = from_arith<TO>(fmaf(-fast_exp((float)to_arith(outp[base + c])), s, (float)to_arith(grad[base + c])));
}

// softmax backward: gi = y (g - sum(g y)).  Both rows stay in registers
// (up to 8 vectors each per thread); longer rows take the streaming kernel.
template <typename TG, typename TO, int VPT>
__global__ void __launch_bounds__(kRowBlock)
k_sm_bwd_reg(const TG* __restrict__ grad, const TG* __restrict__ outp, TO* __restrict__ gin, int64_t cols) {
  constexpr int V = VecOf<TG>::V;
  __shared__ float lds[kRowBlock / 64];
  const int64_t row = blockIdx.x;
  const uint4* g = reinterpret_cast<const uint4*>(grad + row * cols);
  const uint4* y = reinterpret_cast<const uint4*>(outp + row * cols);
  const int nvec = (int)(cols / V);
  const int full = nvec / kRowBlock;
  const int tid = threadIdx.x;
  uint4 gv[VPT], yv[VPT];
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    if (j < full || tid + j * kRowBlock < nvec) {
      gv[j] = ld_stream(g + tid + j * kRowBlock);
      yv[j] = ld_stream(y + tid + j * kRowBlock);
    }
  }
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    if (j < full || tid + j * kRowBlock < nvec) {
#pragma unroll
      for (int k = 0; k < V; ++k) s = fmaf(elem_f<TG>(gv[j], k), elem_f<TG>(yv[j], k), s);
    }
  }
  s = block_sum_all<kRowBlock / 64>(s, lds);
  opaque<VPT>(gv);
  opaque<VPT>(yv);
  Vec<TO, V>* dst = reinterpret_cast<Vec<TO, V>*>(gin + row * cols);
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    if (j < full || tid + j * kRowBlock < nvec) {
      float f[V];
#pragma unroll
      for (int k = 0; k < V; ++k) f[k] = elem_f<TG>(yv[j], k) * (elem_f<TG>(gv[j], k) - s);
      store_row_vec<TO, V>(dst, tid + j * kRowBlock, f);
    }
  }
}

template <typename TG, typename TO>
__global__ void __launch_bounds__(kBlock)
k_sm_bwd_stream(const TG* __restrict__ grad, const TG* __restrict__ outp, TO* __restrict__ gin, int64_t cols) {
  __shared__ float lds[kBlock / 64];
  const int64_t base = (int64_t)blockIdx.x * cols;
  float s = 0.0f;
  for (int64_t c = threadIdx.x; c < cols; c += kBlock)
    s = fmaf((float)to_arith(grad[base + c]), (float)to_arith(outp[base + c]), s);
  s = block_sum_all<kBlock / 64>(s, lds);
  for (int64_t c = threadIdx.x; c < cols; c += kBlock)
    gin[base + c] = from_arith<TO>((float)to_arith(outp[base + c]) * ((float)to_arith(grad[base + c]) - s));
}

template <typename F>
int with_float_storage(int dtype, F&& f) {
  switch (dtype) {
    case SUPA_AMD_F32: return f((float*)nullptr);
    case SUPA_AMD_BF16: return f((bf16*)nullptr);
    case SUPA_AMD_F16: return f((f16*)nullptr);
    default: return SUPA_AMD_EDTYPE;
  }
}

template <bool LOG>
int softmax_forward(const void* in, int32_t in_dtype, void* out, int32_t out_dtype, int64_t rows, int64_t cols,
                    void* stream) {
  if (!in || !out || rows < 0 || cols < 0 || rows >= (int64_t(1) << 31)) return SUPA_AMD_EINVAL;
  if (rows == 0 || cols == 0) return SUPA_AMD_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_float_storage(in_dtype, [&](auto* ti) -> int {
    return with_float_storage(out_dtype, [&](auto* to) -> int {
      using TI = std::remove_pointer_t<decltype(ti)>;
      using TO = std::remove_pointer_t<decltype(to)>;
      if (in_dtype != out_dtype && out_dtype != SUPA_AMD_F32) return SUPA_AMD_EDTYPE;
      constexpr int V = VecOf<TI>::V;
      const bool reg_ok = (cols % V) == 0 && aligned(in, 16) && aligned(out, V * sizeof(TO)) && (cols / V) <= 16 * kRowBlock;
      if (reg_ok) {
        const int64_t nvec = cols / V;
        const int vpt = (int)((nvec + kRowBlock - 1) / kRowBlock);
        const TI* pi = static_cast<const TI*>(in);
        TO* po = static_cast<TO*>(out);
        const unsigned grid = (unsigned)std::min<int64_t>(rows, kLsmGrid);
        if (vpt <= 1) k_lsm_fwd_reg<TI, TO, 1, LOG><<<grid, kRowBlock, 0, st>>>(pi, po, rows, cols);
        else if (vpt <= 2) k_lsm_fwd_reg<TI, TO, 2, LOG><<<grid, kRowBlock, 0, st>>>(pi, po, rows, cols);
        else if (vpt <= 4) k_lsm_fwd_reg<TI, TO, 4, LOG><<<grid, kRowBlock, 0, st>>>(pi, po, rows, cols);
        else if (vpt <= 8) k_lsm_fwd_reg<TI, TO, 8, LOG><<<grid, kRowBlock, 0, st>>>(pi, po, rows, cols);
        else k_lsm_fwd_reg<TI, TO, 16, LOG><<<grid, kRowBlock, 0, st>>>(pi, po, rows, cols);
        return launch_status();
      }
      k_lsm_fwd_stream<TI, TO, LOG><<<(unsigned)rows, kBlock, 0, st>>>(static_cast<const TI*>(in),
                                                                       static_cast<TO*>(out), cols);
      return launch_status();
    });
  });
}

}  // namespace sa

using namespace sa;

extern "C" {

int supa_amd_log_softmax_forward(const void* in, int32_t in_dtype, void* out, int32_t out_dtype, int64_t rows,
                                 int64_t cols, void* stream) {
  return softmax_forward<true>(in, in_dtype, out, out_dtype, rows, cols, stream);
}

int supa_amd_softmax_forward(const void* in, int32_t in_dtype, void* out, int32_t out_dtype, int64_t rows,
                             int64_t cols, void* stream) {
  return softmax_forward<false>(in, in_dtype, out, out_dtype, rows, cols, stream);
}

int supa_amd_log_softmax_backward(const void* grad, const void* output, int32_t gy_dtype, void* grad_in,
                                  int32_t gin_dtype, int64_t rows, int64_t cols, void* stream) {
  if (!grad || !output || !grad_in || rows < 0 || cols < 0 || rows >= (int64_t(1) << 31)) return SUPA_AMD_EINVAL;
  if (rows == 0 || cols == 0) return SUPA_AMD_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_float_storage(gy_dtype, [&](auto* tg) -> int {
    return with_float_storage(gin_dtype, [&](auto* to) -> int {
      using TG = std::remove_pointer_t<decltype(tg)>;
      using TO = std::remove_pointer_t<decltype(to)>;
      if (gy_dtype != gin_dtype && gin_dtype != SUPA_AMD_F32) return SUPA_AMD_EDTYPE;
      constexpr int V = VecOf<TG>::V;
      const bool reg_ok = (cols % V) == 0 && aligned(grad, 16) && aligned(output, 16) && aligned(grad_in, V * sizeof(TO)) &&
                          (cols / V) <= 16 * kRowBlock;
      const TG* pg = static_cast<const TG*>(grad);
      const TG* py = static_cast<const TG*>(output);
      TO* po = static_cast<TO*>(grad_in);
      if (reg_ok) {
        const int64_t nvec = cols / V;
        const int vpt = (int)((nvec + kRowBlock - 1) / kRowBlock);
        if (vpt <= 1) k_lsm_bwd_reg<TG, TO, 1><<<(unsigned)rows, kRowBlock, 0, st>>>(pg, py, po, cols);
        else if (vpt <= 2) k_lsm_bwd_reg<TG, TO, 2><<<(unsigned)rows, kRowBlock, 0, st>>>(pg, py, po, cols);
        else if (vpt <= 4) k_lsm_bwd_reg<TG, TO, 4><<<(unsigned)rows, kRowBlock, 0, st>>>(pg, py, po, cols);
        else if (vpt <= 8) k_lsm_bwd_reg<TG, TO, 8><<<(unsigned)rows, kRowBlock, 0, st>>>(pg, py, po, cols);
        else k_lsm_bwd_reg<TG, TO, 16><<<(unsigned)rows, kRowBlock, 0, st>>>(pg, py, po, cols);
        return launch_status();
      }
      k_lsm_bwd_stream<TG, TO><<<(unsigned)rows, kBlock, 0, st>>>(pg, py, po, cols);
      return launch_status();
    });
  });
}

int supa_amd_softmax_backward(const void* grad, const void* output, int32_t gy_dtype, void* grad_in,
                              int32_t gin_dtype, int64_t rows, int64_t cols, void* stream) {
  if (!grad || !output || !grad_in || rows < 0 || cols < 0 || rows >= (int64_t(1) << 31)) return SUPA_AMD_EINVAL;
  if (rows == 0 || cols == 0) return SUPA_AMD_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_float_storage(gy_dtype, [&](auto* tg) -> int {
    return with_float_storage(gin_dtype, [&](auto* to) -> int {
      using TG = std::remove_pointer_t<decltype(tg)>;
      using TO = std::remove_pointer_t<decltype(to)>;
      if (gy_dtype != gin_dtype && gin_dtype != SUPA_AMD_F32) return SUPA_AMD_EDTYPE;
      constexpr int V = VecOf<TG>::V;
      const bool reg_ok = (cols % V) == 0 && aligned(grad, 16) && aligned(output, 16) && aligned(grad_in, V * sizeof(TO)) &&
                          (cols / V) <= 8 * kRowBlock;
      const TG* pg = static_cast<const TG*>(grad);
      const TG* py = static_cast<const TG*>(output);
      TO* po = static_cast<TO*>(grad_in);
      if (reg_ok) {
        const int64_t nvec = cols / V;
        const int vpt = (int)((nvec + kRowBlock - 1) / kRowBlock);
        if (vpt <= 1) k_sm_bwd_reg<TG, TO, 1><<<(unsigned)rows, kRowBlock, 0, st>>>(pg, py, po, cols);
        else if (vpt <= 2) k_sm_bwd_reg<TG, TO, 2><<<(unsigned)rows, kRowBlock, 0, st>>>(pg, py, po, cols);
        else if (vpt <= 4) k_sm_bwd_reg<TG, TO, 4><<<(unsigned)rows, kRowBlock, 0, st>>>(pg, py, po, cols);
        else k_sm_bwd_reg<TG, TO, 8><<<(unsigned)rows, kRowBlock, 0, st>>>(pg, py, po, cols);
        return launch_status();
      }
      k_sm_bwd_stream<TG, TO><<<(unsigned)rows, kBlock, 0, st>>>(pg, py, po, cols);
      return launch_status();
    });
  });
}

}  // extern "C"
