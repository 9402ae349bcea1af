// Variance / standard deviation (and the mean beside them) along the last
// dim of a contiguous [outer, inner] input: var / std / var_mean / std_mean
// with a correction, which LayerNorm and BatchNorm written by hand, and
// normalisation statistics, call next to the loss path.
//
// Welford's running (count, mean, M2) per thread over a strided walk, merged
// pairwise by Chan et al.'s update (wavefront shuffles, then LDS); the
// result is M2 / max(0, count - correction), its square root for std.
// Upstream's device reduction (WelfordOps in SharedReduceOps.h) accumulates
// the same triple, so a NaN propagates and a row with count <= correction
// divides by zero (inf or NaN) as it does there.  Every value is first
// shifted by its row's first element K (the shifted-data algorithm): the
// triple then tracks mean - K, which keeps its precision when the mean is
// large against the spread (float Welford on unshifted data loses about
// (ulp(mean) / sigma)^2 of the variance); the mean written out adds K back.
//
// Each thread takes its values eight at a time: the batch's own triple
// (its mean, and the squared deviations from it, in registers) merges into
// the running one, one division per batch instead of one per value.
//
// One workgroup per (row, chunk of `chunk` elements): a single wavefront for
// rows up to kMomWaveRow elements (no LDS stage; more rows in flight per CU),
// four for longer ones.  Long rows with few of them take two launches: the
// first writes one triple per chunk into the workspace, the second merges
// each row's triples.
//
// Replaces var.correction_out NF:6629, std.correction_out NF:6088,
// var_mean.correction NF:6668, std_mean.correction NF:6063 (upstream
// ReduceMomentKernel.cu: std_var_kernel_cuda over WelfordOps).
#include "ew_launch.h"

namespace sa {

constexpr int kMomBlock = 256;
constexpr int64_t kMomWaveRow = 4096;  // rows up to this length take one-wavefront workgroups
constexpr int64_t kMomChunk = 16384;    // elements per workgroup in the first of two launches
constexpr int64_t kMomTwoPass = 65536;  // rows longer than this (with few rows) take two launches

template <typename A> struct Welford {
  A n, mean, m2;
};

template <typename A> __device__ __forceinline__ Welford<A> wf_merge(Welford<A> a, Welford<A> b) {
  if (a.n == A(0)) return b;
  if (b.n == A(0)) return a;
  const A n = a.n + b.n;
  const A d = b.mean - a.mean;
  const A nb_n = b.n / n;
  return {n, a.mean + d * nb_n, a.m2 + b.m2 + d * d * a.n * nb_n};
}

template <typename A> __device__ __forceinline__ Welford<A> wf_shfl(Welford<A> w, int off) {
  return {__shfl_xor(w.n, off, 64), __shfl_xor(w.mean, off, 64), __shfl_xor(w.m2, off, 64)};
}

inline int64_t mom_chunks(int64_t outer, int64_t inner) {
  return inner > kMomTwoPass && outer < 2048 ? (inner + kMomChunk - 1) / kMomChunk : 1;
}

// TERM: `in` holds elements of T (else the triples of an earlier launch, as
// three A per chunk).  FINAL: write var-or-std (and the mean) in OT (else the
// chunk's triple into `part`).
// K of a row is kin[row * kstride] (the row's first input element, in both
// launches).
template <int BS, typename T, typename KT, typename OT, typename A, bool TERM, bool FINAL>
__global__ void __launch_bounds__(BS)
k_moments(const void* __restrict__ in, const KT* __restrict__ kin, int64_t kstride, int64_t inner, int64_t chunk,
          uint32_t nchunks, A correction, int take_sqrt, OT* __restrict__ out_var, OT* __restrict__ out_mean,
          A* __restrict__ part) {
  __shared__ Welford<A> lds[BS / 64];
  const uint32_t row = blockIdx.x / nchunks, c = blockIdx.x % nchunks;
  const A K = (A)to_arith(kin[(int64_t)row * kstride]);
  const int64_t lo = (int64_t)c * chunk;
  const int64_t n = lo + chunk < inner ? chunk : inner - lo;
  Welford<A> w{A(0), A(0), A(0)};
  if constexpr (TERM) {
    const T* src = static_cast<const T*>(in) + (int64_t)row * inner + lo;
    constexpr int U = 8;
    for (int64_t i0 = threadIdx.x; i0 < n; i0 += (int64_t)U * BS) {
      A x[U];
      int cnt = 0;
      A sum = A(0);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t i = i0 + (int64_t)u * BS;
        x[u] = i < n ? (A)to_arith(src[i]) - K : A(0);
        cnt += i < n ? 1 : 0;
        sum += x[u];
      }
      const A bn = (A)cnt;
      const A bmean = sum / bn;
      A bm2 = A(0);
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const A d = x[u] - bmean;
        if (u < cnt) bm2 += d * d;
      }
      w = wf_merge(w, Welford<A>{bn, bmean, bm2});
    }
  } else {
    const A* src = static_cast<const A*>(in) + ((int64_t)row * inner + lo) * 3;
    for (int64_t i = threadIdx.x; i < n; i += BS)
      w = wf_merge(w, Welford<A>{src[3 * i], src[3 * i + 1], src[3 * i + 2]});
  }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) w = wf_merge(w, wf_shfl(w, off));
  if constexpr (BS > 64) {
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = w;
    __syncthreads();
  }
  if (threadIdx.x == 0) {
#pragma unroll
    for (int k = 1; k < BS / 64; ++k) w = wf_merge(w, lds[k]);
    if constexpr (FINAL) {
      const A div = w.n > correction ? w.n - correction : A(0);
      const A var = w.m2 / div;
      out_var[blockIdx.x] = from_arith<OT>(take_sqrt ? sqrt(var) : var);
      if (out_mean) out_mean[blockIdx.x] = from_arith<OT>(w.mean + K);
    } else {
      part[3 * (int64_t)blockIdx.x] = w.n;
      part[3 * (int64_t)blockIdx.x + 1] = w.mean;
      part[3 * (int64_t)blockIdx.x + 2] = w.m2;
    }
  }
}

template <typename T>
int moments_launch(const T* in, T* out_var, T* out_mean, int64_t outer, int64_t inner, double correction,
                   int take_sqrt, void* ws, hipStream_t st) {
  using A = opmath_t<T>;
  const int64_t nch = mom_chunks(outer, inner);
  if (nch == 1 && inner <= kMomWaveRow) {
    k_moments<64, T, T, T, A, true, true><<<(unsigned)outer, 64, 0, st>>>(
        in, in, inner, inner, inner, 1u, (A)correction, take_sqrt, out_var, out_mean, nullptr);
    return launch_status();
  }
  if (nch == 1) {
    k_moments<kMomBlock, T, T, T, A, true, true><<<(unsigned)outer, kMomBlock, 0, st>>>(
        in, in, inner, inner, inner, 1u, (A)correction, take_sqrt, out_var, out_mean, nullptr);
    return launch_status();
  }
  A* part = static_cast<A*>(ws);
  k_moments<kMomBlock, T, T, T, A, true, false><<<(unsigned)(outer * nch), kMomBlock, 0, st>>>(
      in, in, inner, inner, kMomChunk, (uint32_t)nch, (A)correction, take_sqrt, nullptr, nullptr, part);
  const int rc = launch_status();
  if (rc) return rc;
  k_moments<kMomBlock, A, T, T, A, false, true><<<(unsigned)outer, kMomBlock, 0, st>>>(
      part, in, inner, nch, nch, 1u, (A)correction, take_sqrt, out_var, out_mean, nullptr);
  return launch_status();
}

}  // namespace sa

using namespace sa;

extern "C" {

int64_t supa_amd_moments_rows_workspace_bytes(int64_t outer, int64_t inner, int32_t dtype) {
  if (outer < 0 || inner <= 0) return SUPA_AMD_EINVAL;
  if (dtype != SUPA_AMD_F32 && dtype != SUPA_AMD_BF16 && dtype != SUPA_AMD_F16 && dtype != SUPA_AMD_F64)
    return SUPA_AMD_EDTYPE;
  const int64_t nch = mom_chunks(outer, inner);
  return nch == 1 ? 0 : outer * nch * 3 * (dtype == SUPA_AMD_F64 ? 8 : 4);
}

int supa_amd_moments_rows(const void* in, int32_t dtype, int64_t outer, int64_t inner, double correction,
                          int take_sqrt, void* out_var, void* out_mean, void* workspace, int64_t ws_bytes,
                          void* stream) {
  if (!in || !out_var || outer < 0 || inner <= 0 || correction != correction) return SUPA_AMD_EINVAL;
  if (outer == 0) return SUPA_AMD_OK;
  if (outer * mom_chunks(outer, inner) >= (int64_t(1) << 31)) return SUPA_AMD_ELAYOUT;
  const int64_t need = supa_amd_moments_rows_workspace_bytes(outer, inner, dtype);
  if (need < 0) return (int)need;
  if (need > 0 && (!workspace || ws_bytes < need)) return SUPA_AMD_EWORKSPACE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto go = [&](auto* tag) -> int {
    using T = std::remove_pointer_t<decltype(tag)>;
    return moments_launch<T>(static_cast<const T*>(in), static_cast<T*>(out_var), static_cast<T*>(out_mean), outer,
                             inner, correction, take_sqrt ? 1 : 0, workspace, st);
  };
  switch (dtype) {
    case SUPA_AMD_F32: return go((float*)nullptr);
    case SUPA_AMD_BF16: return go((bf16*)nullptr);
    case SUPA_AMD_F16: return go((f16*)nullptr);
    case SUPA_AMD_F64: return go((double*)nullptr);
    default: return SUPA_AMD_EDTYPE;
  }
}

}  // extern "C"
