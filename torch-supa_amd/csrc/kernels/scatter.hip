// C-ABI entry point: scatter_ with a scalar value (the assign form of
// upstream scatter_fill_kernel, ScatterGatherKernel.cu), which one_hot runs.
// One thread per index element: its coordinates come from the linear id by
// division over the index shape; the output offset takes those coordinates
// with the one along `dim` replaced by the index value.  An index outside
// [0, out_dim_size) writes nothing and sets the error flag the host reads at
// its next synchronisation (upstream stops at a device assert instead).
#include "ew_launch.h"

namespace sa {

struct ScatterGeom {
  int64_t size[SUPA_AMD_MAX_DIMS];        // index shape
  int64_t out_stride[SUPA_AMD_MAX_DIMS];  // elements
  int64_t idx_stride[SUPA_AMD_MAX_DIMS];  // elements
  int32_t ndim, dim;
  int64_t out_dim_size;
};

template <typename T>
__global__ void __launch_bounds__(256)
k_scatter_fill(T* __restrict__ out, const int64_t* __restrict__ idx, ScatterGeom g, int64_t n, double value,
               int64_t ivalue, int32_t* error_flag) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  // integer outputs take the exact integer value, the others the double
  T v;
  if constexpr (std::is_integral<T>::value) v = static_cast<T>(ivalue);
  else v = from_arith<T>(static_cast<opmath_t<T>>(value));
  int64_t rem = i, o = 0, ix = 0;
  for (int d = g.ndim - 1; d >= 0; --d) {
    const int64_t c = rem % g.size[d];
    rem /= g.size[d];
    ix += c * g.idx_stride[d];
    if (d != g.dim) o += c * g.out_stride[d];
  }
  const int64_t k = idx[ix];
  if (k < 0 || k >= g.out_dim_size) {
    if (error_flag) *error_flag = 2;
    return;
  }
  out[o + k * g.out_stride[g.dim]] = v;
}

}  // namespace sa

using namespace sa;

extern "C" {

int supa_amd_scatter_fill(void* out, int32_t dtype, const int64_t* out_strides, int64_t out_dim_size,
                          const int64_t* index, const int64_t* index_sizes, const int64_t* index_strides, int32_t ndim,
                          int32_t dim, double value, int64_t ivalue, int32_t* error_flag, void* stream) {
  if (!out || !index || !out_strides || !index_sizes || !index_strides) return SUPA_AMD_EINVAL;
  if (ndim < 1 || ndim > SUPA_AMD_MAX_DIMS || dim < 0 || dim >= ndim || out_dim_size < 0) return SUPA_AMD_EINVAL;
  ScatterGeom g{};
  g.ndim = ndim;
  g.dim = dim;
  g.out_dim_size = out_dim_size;
  int64_t n = 1;
  for (int d = 0; d < ndim; ++d) {
    if (index_sizes[d] < 0) return SUPA_AMD_EINVAL;
    g.size[d] = index_sizes[d];
    g.out_stride[d] = out_strides[d];
    g.idx_stride[d] = index_strides[d];
    n *= index_sizes[d];
  }
  if (n == 0) return SUPA_AMD_OK;
  const int64_t blocks = (n + 255) / 256;
  if (blocks > (int64_t)0x7fffffff) return SUPA_AMD_ELAYOUT;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_storage(dtype, [&](auto* tag) -> int {
    using T = std::remove_pointer_t<decltype(tag)>;
    k_scatter_fill<T><<<(unsigned)blocks, 256, 0, st>>>(static_cast<T*>(out), index, g, n, value, ivalue,
                                                        error_flag);
    return launch_status();
  });
}

}  // extern "C"
