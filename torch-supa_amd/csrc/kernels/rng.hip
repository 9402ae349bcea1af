// Counter-based random numbers: uniform_, normal_, bernoulli_ and the fused
// dropout forward (native_dropout) on Philox4x32-10 (Salmon et al., SC 2011).
//
// Element i draws word i % 4 of philox(counter = (i / 4, offset), key =
// seed), so every element's value depends only on (seed, offset, i): the
// result is the same for any launch shape, and a generator hands each call a
// fresh offset.  One thread produces four consecutive elements from one
// Philox call.  The reference draws through curand's Philox (CUDA
// DistributionTemplates.h, Dropout.cu); the streams differ, the
// distributions do not.
#include "ew_launch.h"

namespace sa {

__device__ __forceinline__ uint4 philox4x32_10(uint4 c, uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint32_t hi0 = __umulhi(0xD2511F53u, c.x), lo0 = 0xD2511F53u * c.x;
    const uint32_t hi1 = __umulhi(0xCD9E8D57u, c.z), lo1 = 0xCD9E8D57u * c.z;
    c = make_uint4(hi1 ^ c.y ^ k0, lo1, hi0 ^ c.w ^ k1, lo0);
  }
  return c;
}

__device__ __forceinline__ uint4 draw4(uint64_t q, uint64_t seed, uint64_t offset) {
  return philox4x32_10(make_uint4((uint32_t)q, (uint32_t)(q >> 32), (uint32_t)offset, (uint32_t)(offset >> 32)),
                       (uint32_t)seed, (uint32_t)(seed >> 32));
}

// [0, 1) from the top 24 bits
__device__ __forceinline__ float u01(uint32_t r) { return (float)(r >> 8) * 5.9604644775390625e-08f; }

__device__ __forceinline__ uint32_t word(const uint4& r, int j) {
  return j == 0 ? r.x : (j == 1 ? r.y : (j == 2 ? r.z : r.w));
}

// MODE 0: uniform (a = lo, b = hi - lo, c = hi): a value that rounds to hi
// in T is replaced by lo, keeping [lo, hi) for 16-bit types (upstream
// uniform_kernel's bound reversal, DistributionTemplates.h); 1: bernoulli
// (a = p).
template <typename T, int MODE>
__global__ void __launch_bounds__(kBlock)
k_rng_fill(T* __restrict__ out, int64_t n, uint64_t seed, uint64_t offset, float a, float b, float c) {
  const uint64_t q = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t e0 = (int64_t)q * 4;
  if (e0 >= n) return;
  const uint4 r = draw4(q, seed, offset);
  float v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float u = u01(word(r, j));
    v[j] = MODE == 0 ? fmaf(u, b, a) : (u < a ? 1.0f : 0.0f);
  }
  T w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    w[j] = from_arith<T>(v[j]);
    if constexpr (MODE == 0) {
      if (to_arith(w[j]) == to_arith(from_arith<T>(c))) w[j] = from_arith<T>(a);
    }
  }
  if (e0 + 4 <= n && aligned(out + e0, 4 * sizeof(T))) {
    Vec<T, 4> wv;
#pragma unroll
    for (int j = 0; j < 4; ++j) wv.v[j] = w[j];
    *reinterpret_cast<Vec<T, 4>*>(out + e0) = wv;
  } else {
    for (int j = 0; j < 4 && e0 + j < n; ++j) out[e0 + j] = w[j];
  }
}

// normal(mean, std): Box-Muller on two words per pair of outputs, in double
// (u1 = (hi24(w) + 1) 2^-24 in (0, 1], u2 = hi24(w') 2^-24): elements 4q + 0,1
// are r cos(t), r sin(t) of words 0, 1, elements 4q + 2,3 of words 2, 3, with
// r = sqrt(-2 log u1), t = 2 pi u2; out = mean + std z in double, rounded to
// float (and for a 16-bit storage type, from float to that type).
__device__ __forceinline__ void box_muller(uint32_t w1, uint32_t w2, double& z0, double& z1) {
  const double u1 = ((double)(w1 >> 8) + 1.0) * 5.9604644775390625e-08;
  const double u2 = (double)(w2 >> 8) * 5.9604644775390625e-08;
  const double r = sqrt(-2.0 * log(u1));
  double sn, cs;
  sincospi(2.0 * u2, &sn, &cs);
  z0 = r * cs;
  z1 = r * sn;
}

template <typename T>
__global__ void __launch_bounds__(kBlock)
k_rng_normal(T* __restrict__ out, int64_t n, uint64_t seed, uint64_t offset, double mean, double stdv) {
  const uint64_t q = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t e0 = (int64_t)q * 4;
  if (e0 >= n) return;
  const uint4 r = draw4(q, seed, offset);
  double z[4];
  box_muller(r.x, r.y, z[0], z[1]);
  box_muller(r.z, r.w, z[2], z[3]);
  for (int j = 0; j < 4 && e0 + j < n; ++j) out[e0 + j] = from_arith<T>((float)(mean + stdv * z[j]));
}

// dropout with keep probability q: mask = u < q, out = (x * mask) * scale.
template <typename T>
__global__ void __launch_bounds__(kBlock)
k_dropout(const T* __restrict__ x, T* __restrict__ out, b8* __restrict__ mask, int64_t n, uint64_t seed,
          uint64_t offset, float keep, float scale) {
  using C = opmath_t<T>;
  const uint64_t q = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t e0 = (int64_t)q * 4;
  if (e0 >= n) return;
  const uint4 r = draw4(q, seed, offset);
  const bool full = e0 + 4 <= n && aligned(x + e0, 4 * sizeof(T)) && aligned(out + e0, 4 * sizeof(T)) &&
                    aligned(mask + e0, 4);
  if (full) {
    const Vec<T, 4> xv = ld_stream(reinterpret_cast<const Vec<T, 4>*>(x + e0));
    Vec<T, 4> o;
    Vec<b8, 4> m;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool k = u01(word(r, j)) < keep;
      m.v[j].x = k ? 1 : 0;
      o.v[j] = from_arith<T>(((C)to_arith(xv.v[j]) * (k ? C(1) : C(0))) * (C)scale);
    }
    st_stream(reinterpret_cast<Vec<T, 4>*>(out + e0), o);
    *reinterpret_cast<Vec<b8, 4>*>(mask + e0) = m;
  } else {
    for (int j = 0; j < 4 && e0 + j < n; ++j) {
      const bool k = u01(word(r, j)) < keep;
      mask[e0 + j].x = k ? 1 : 0;
      out[e0 + j] = from_arith<T>(((C)to_arith(x[e0 + j]) * (k ? C(1) : C(0))) * (C)scale);
    }
  }
}

template <typename F>
int with_rng_storage(int dtype, F&& f) {
  switch (dtype) {
    case SUPA_AMD_F32: return f((float*)nullptr);
    case SUPA_AMD_BF16: return f((bf16*)nullptr);
    case SUPA_AMD_F16: return f((f16*)nullptr);
    default: return SUPA_AMD_EDTYPE;
  }
}

inline unsigned rng_blocks(int64_t n) { return (unsigned)(((n + 3) / 4 + kBlock - 1) / kBlock); }

}  // namespace sa

using namespace sa;

extern "C" {

int supa_amd_uniform(void* out, int32_t dtype, int64_t n, double lo, double hi, uint64_t seed, uint64_t offset,
                     void* stream) {
  if (n < 0 || (n > 0 && !out)) return SUPA_AMD_EINVAL;
  if ((n + 3) / 4 > (int64_t)kBlock * 0x7fffffffll) return SUPA_AMD_ELAYOUT;
  if (n == 0) return SUPA_AMD_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const float a = (float)lo, b = (float)hi - (float)lo;
  return with_rng_storage(dtype, [&](auto* tag) -> int {
    using T = std::remove_pointer_t<decltype(tag)>;
    k_rng_fill<T, 0><<<rng_blocks(n), kBlock, 0, st>>>(static_cast<T*>(out), n, seed, offset, a, b, (float)hi);
    return launch_status();
  });
}

int supa_amd_bernoulli(void* out, int32_t dtype, int64_t n, double p, uint64_t seed, uint64_t offset, void* stream) {
  if (n < 0 || (n > 0 && !out) || !(p >= 0.0 && p <= 1.0)) return SUPA_AMD_EINVAL;
  if ((n + 3) / 4 > (int64_t)kBlock * 0x7fffffffll) return SUPA_AMD_ELAYOUT;
  if (n == 0) return SUPA_AMD_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_rng_storage(dtype, [&](auto* tag) -> int {
    using T = std::remove_pointer_t<decltype(tag)>;
    k_rng_fill<T, 1><<<rng_blocks(n), kBlock, 0, st>>>(static_cast<T*>(out), n, seed, offset, (float)p, 0.0f,
                                                        0.0f);
    return launch_status();
  });
}

int supa_amd_normal(void* out, int32_t dtype, int64_t n, double mean, double stdv, uint64_t seed, uint64_t offset,
                    void* stream) {
  if (n < 0 || (n > 0 && !out) || !(stdv >= 0.0)) return SUPA_AMD_EINVAL;
  if ((n + 3) / 4 > (int64_t)kBlock * 0x7fffffffll) return SUPA_AMD_ELAYOUT;
  if (n == 0) return SUPA_AMD_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_rng_storage(dtype, [&](auto* tag) -> int {
    using T = std::remove_pointer_t<decltype(tag)>;
    k_rng_normal<T><<<rng_blocks(n), kBlock, 0, st>>>(static_cast<T*>(out), n, seed, offset, mean, stdv);
    return launch_status();
  });
}

int supa_amd_dropout(const void* x, int32_t dtype, void* out, uint8_t* mask, int64_t n, double keep, uint64_t seed,
                     uint64_t offset, void* stream) {
  if (n < 0 || (n > 0 && (!x || !out || !mask)) || !(keep > 0.0 && keep <= 1.0)) return SUPA_AMD_EINVAL;
  if ((n + 3) / 4 > (int64_t)kBlock * 0x7fffffffll) return SUPA_AMD_ELAYOUT;
  if (n == 0) return SUPA_AMD_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const float keepf = (float)keep;
  // upstream fused_dropout_kernel: scale = 1.0 / p with p the float keep
  // probability, the quotient taken in double and stored as float
  const float scale = (float)(1.0 / (double)keepf);
  return with_rng_storage(dtype, [&](auto* tag) -> int {
    using T = std::remove_pointer_t<decltype(tag)>;
    k_dropout<T><<<rng_blocks(n), kBlock, 0, st>>>(static_cast<const T*>(x), static_cast<T*>(out),
                                                    reinterpret_cast<b8*>(mask), n, seed, offset, keepf, scale);
    return launch_status();
  });
}

}  // extern "C"
