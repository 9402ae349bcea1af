// max / min (with their index) along the last dim of a contiguous [outer,
// inner] input: amax / amin, max.dim / min.dim, argmax / argmin and the full
// max() / min().
//
// Selection order (a total order on (value, index) pairs, so the result does
// not depend on the reduction tree): a NaN beats every number (upstream's
// max / min propagate NaN, and argmax / argmin point at a NaN); between two
// NaNs or two equal values the smaller index wins (upstream returns the first
// extremal index); otherwise the larger (max) or smaller (min) value wins.
//
// One 256-thread workgroup per (row, chunk of `chunk` elements): each thread
// keeps its best pair over a strided walk with 8 loads in flight, the pairs
// meet through wavefront shuffles and LDS.  Long rows take two launches: the
// first writes one pair per chunk, the second reduces each row's chunk pairs
// (reading their indices from `in_idx`).
//
// Replaces amax.out NF:3926, amin.out NF:4115, max.dim_max NF:3894,
// min.dim_min NF:4091, argmax.out NF:839, argmin.out NF:852, max.unary_out
// NF:10274, min.unary_out NF:10204 (upstream ReduceMinMaxKernel.cu /
// ReduceArgMaxKernel.cu / ReduceArgMinKernel.cu).
#include "ew_launch.h"

namespace sa {

constexpr int kExtBlock = 256;

template <typename A> __device__ __forceinline__ bool is_nan_v(A a) {
  if constexpr (std::is_floating_point<A>::value) return a != a;
  else return false;
}

// true when (a, ai) comes before (b, bi)
template <bool MIN, typename A>
__device__ __forceinline__ bool ext_better(A a, int64_t ai, A b, int64_t bi) {
  const bool na = is_nan_v(a), nb = is_nan_v(b);
  if (na != nb) return na;
  if (na || a == b) return ai < bi;
  return MIN ? a < b : a > b;
}

template <bool MIN, typename A>
__device__ __forceinline__ void ext_take(A& v, int64_t& i, A b, int64_t bi) {
  if (ext_better<MIN>(b, bi, v, i)) {
    v = b;
    i = bi;
  }
}

// A = the comparison type (float for the float family, double, int64 for
// integers and bool); T = storage.
template <bool MIN, typename T, typename A>
__global__ void __launch_bounds__(kExtBlock)
k_argext(const T* __restrict__ in, const int64_t* __restrict__ in_idx, int64_t inner, int64_t chunk,
         uint32_t nchunks, T* __restrict__ out_val, int64_t* __restrict__ out_idx) {
  __shared__ A lds_v[kExtBlock / 64];
  __shared__ int64_t lds_i[kExtBlock / 64];
  const uint32_t row = blockIdx.x / nchunks, c = blockIdx.x % nchunks;
  const int64_t lo = (int64_t)c * chunk;
  const int64_t hi = lo + chunk < inner ? lo + chunk : inner;
  const T* src = in + (int64_t)row * inner;
  const int64_t* isrc = in_idx ? in_idx + (int64_t)row * inner : nullptr;
  // start from the first element of the segment (always present)
  A bv = (A)to_arith(src[lo]);
  int64_t bi = isrc ? isrc[lo] : lo;
  constexpr int U = 8;
  for (int64_t j0 = lo + threadIdx.x; j0 < hi; j0 += (int64_t)U * kExtBlock) {
    A v[U];
    int64_t ix[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = j0 + (int64_t)u * kExtBlock;
      const bool in_r = j < hi;
      v[u] = in_r ? (A)to_arith(src[j]) : bv;
      ix[u] = in_r ? (isrc ? isrc[j] : j) : bi;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) ext_take<MIN>(bv, bi, v[u], ix[u]);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const A ov = __shfl_xor(bv, off, 64);
    const int64_t oi = __shfl_xor(bi, off, 64);
    ext_take<MIN>(bv, bi, ov, oi);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    lds_v[wave] = bv;
    lds_i[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 1; w < kExtBlock / 64; ++w) ext_take<MIN>(bv, bi, lds_v[w], lds_i[w]);
    if (out_val) out_val[blockIdx.x] = from_arith<T>(bv);
    if (out_idx) out_idx[blockIdx.x] = bi;
  }
}

template <typename T> struct ExtCmp {
  using type = typename std::conditional<std::is_same<T, double>::value, double,
                                         typename std::conditional<std::is_integral<T>::value ||
                                                                       std::is_same<T, b8>::value,
                                                                   int64_t, float>::type>::type;
};

template <typename F>
int with_ext_storage(int dtype, F&& f) {
  switch (dtype) {
    case SUPA_AMD_F32: return f((float*)nullptr);
    case SUPA_AMD_BF16: return f((bf16*)nullptr);
    case SUPA_AMD_F16: return f((f16*)nullptr);
    case SUPA_AMD_F64: return f((double*)nullptr);
    case SUPA_AMD_U8: return f((uint8_t*)nullptr);
    case SUPA_AMD_I8: return f((int8_t*)nullptr);
    case SUPA_AMD_I16: return f((int16_t*)nullptr);
    case SUPA_AMD_I32: return f((int32_t*)nullptr);
    case SUPA_AMD_I64: return f((int64_t*)nullptr);
    case SUPA_AMD_BOOL: return f((b8*)nullptr);
    default: return SUPA_AMD_EDTYPE;
  }
}

}  // namespace sa

using namespace sa;

extern "C" {

int supa_amd_argext_rows(const void* in, int32_t dtype, const int64_t* in_idx, int64_t outer, int64_t inner,
                         int64_t chunk, int is_min, void* out_val, int64_t* out_idx, void* stream) {
  if (!in || outer < 0 || inner <= 0 || chunk <= 0 || (!out_val && !out_idx)) return SUPA_AMD_EINVAL;
  if (outer == 0) return SUPA_AMD_OK;
  const int64_t nchunks = (inner + chunk - 1) / chunk;
  if (outer * nchunks >= (int64_t(1) << 31)) return SUPA_AMD_ELAYOUT;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_ext_storage(dtype, [&](auto* tag) -> int {
    using T = std::remove_pointer_t<decltype(tag)>;
    using A = typename ExtCmp<T>::type;
    const unsigned blocks = (unsigned)(outer * nchunks);
    if (is_min)
      k_argext<true, T, A><<<blocks, kExtBlock, 0, st>>>(static_cast<const T*>(in), in_idx, inner, chunk,
                                                         (uint32_t)nchunks, static_cast<T*>(out_val), out_idx);
    else
      k_argext<false, T, A><<<blocks, kExtBlock, 0, st>>>(static_cast<const T*>(in), in_idx, inner, chunk,
                                                          (uint32_t)nchunks, static_cast<T*>(out_val), out_idx);
    return launch_status();
  });
}

}  // extern "C"
