// Storage types, conversions and vector IO for the gfx950 kernels.
//
// bfloat16 and bool are carried as plain 16-/8-bit structs so every
// conversion is spelled out here: float -> bfloat16 is round to nearest even
// with NaN -> 0x7FC0, the rule of c10::BFloat16 (c10/util/BFloat16.h), so a
// bf16 result is bit-identical to the one the upstream CPU kernels store.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "supa_amd.h"

namespace sa {

struct bf16 {
  uint16_t x;
};
struct b8 {
  uint8_t x;
};
typedef _Float16 f16;

__device__ __forceinline__ float bf16_to_f32(bf16 h) { return __uint_as_float((uint32_t)h.x << 16); }
// Round to nearest even through the gfx950 convert instruction; NaN becomes
// the canonical 0x7FC0 that c10::BFloat16 produces.
__device__ __forceinline__ bf16 f32_to_bf16(float f) {
  const __bf16 hw = (__bf16)f;
  bf16 h;
  h.x = (f != f) ? (uint16_t)0x7FC0u : __builtin_bit_cast(uint16_t, hw);
  return h;
}
// Round a float result to f16.  The empty asm pins the value as a float32
// first: without it the compiler folds a producing fma into v_fma_mixlo_f16,
// which rounds the exact product-sum once to f16, while the upstream kernels
// round it to float and then to half (about 1 result in 10^4 differs).
__device__ __forceinline__ f16 f32_to_f16(float f) {
  __asm__("" : "+v"(f));
  return static_cast<f16>(f);
}

// opmath: the type an op computes in for a given storage type.
template <typename T> struct opmath { using type = T; };
template <> struct opmath<bf16> { using type = float; };
template <> struct opmath<f16> { using type = float; };
template <> struct opmath<b8> { using type = bool; };
template <typename T> using opmath_t = typename opmath<T>::type;

template <typename T> struct is_floating_st : std::is_floating_point<T> {};
template <> struct is_floating_st<bf16> : std::true_type {};
template <> struct is_floating_st<f16> : std::true_type {};

// to_arith: storage value -> an arithmetic value (float for the 16-bit floats).
__device__ __forceinline__ float to_arith(bf16 v) { return bf16_to_f32(v); }
__device__ __forceinline__ float to_arith(f16 v) { return (float)v; }
__device__ __forceinline__ bool to_arith(b8 v) { return v.x != 0; }
template <typename T>
__device__ __forceinline__ typename std::enable_if<std::is_arithmetic<T>::value, T>::type to_arith(T v) {
  return v;
}

// from_arith<S>(v): arithmetic value -> storage type S, with torch's cast rules
// (16-bit floats are formed from float; bool is v != 0).
template <typename S> struct FromArith {
  template <typename A> __device__ __forceinline__ static S f(A v) { return static_cast<S>(v); }
};
template <> struct FromArith<bf16> {
  template <typename A> __device__ __forceinline__ static bf16 f(A v) { return f32_to_bf16(static_cast<float>(v)); }
};
template <> struct FromArith<f16> {
  template <typename A> __device__ __forceinline__ static f16 f(A v) { return f32_to_f16(static_cast<float>(v)); }
};
template <> struct FromArith<b8> {
  template <typename A> __device__ __forceinline__ static b8 f(A v) {
    b8 r;
    r.x = (v != A(0)) ? 1 : 0;
    return r;
  }
};
template <typename S, typename A> __device__ __forceinline__ S from_arith(A v) { return FromArith<S>::f(v); }

// Load conversion of one input: storage S -> common dtype CT -> compute type C.
// When S == CT this is a single widening; otherwise the value is first rounded
// to CT, as TensorIterator's cast to the common dtype does.
template <typename C, typename CT, typename S>
__device__ __forceinline__ C load_cvt(S s) {
  if constexpr (std::is_same<S, CT>::value) {
    return static_cast<C>(to_arith(s));
  } else {
    return static_cast<C>(to_arith(from_arith<CT>(to_arith(s))));
  }
}

// Fixed-size vector for 16-byte global loads/stores.
template <typename T, int V> struct alignas(sizeof(T) * V) Vec {
  T v[V];
};

// Streaming (nontemporal) vector load/store: data read or written once per
// kernel bypasses cache residency, which measured faster for HBM-bound
// streams on MI355X.  Operands that are re-read (broadcast rows) keep plain
// loads.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
template <typename VT>
__device__ __forceinline__ VT ld_stream(const VT* p) {
  if constexpr (sizeof(VT) % 16 != 0) {
    return *p;  // sub-vector accesses (scalar paths) stay plain
  } else {
    VT r;
#pragma unroll
    for (int w = 0; w < (int)(sizeof(VT) / 16); ++w)
      reinterpret_cast<u32x4_t*>(&r)[w] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p) + w);
    return r;
  }
}
template <typename VT>
__device__ __forceinline__ void st_stream(VT* p, const VT& v) {
  if constexpr (sizeof(VT) % 16 != 0) {
    *p = v;
  } else {
#pragma unroll
    for (int w = 0; w < (int)(sizeof(VT) / 16); ++w)
      __builtin_nontemporal_store(reinterpret_cast<const u32x4_t*>(&v)[w], reinterpret_cast<u32x4_t*>(p) + w);
  }
}

// ----------------------------------------------------------------- runtime
// Dynamic-dtype load/store for the generic kernels.
template <typename C>
__device__ __forceinline__ C load_dyn(const void* p, int64_t off, int dtype) {
  switch (dtype) {
    case SUPA_AMD_F32: return static_cast<C>(static_cast<const float*>(p)[off]);
    case SUPA_AMD_BF16: return static_cast<C>(bf16_to_f32(static_cast<const bf16*>(p)[off]));
    case SUPA_AMD_F16: return static_cast<C>(static_cast<float>(static_cast<const f16*>(p)[off]));
    case SUPA_AMD_F64: return static_cast<C>(static_cast<const double*>(p)[off]);
    case SUPA_AMD_I64: return static_cast<C>(static_cast<const int64_t*>(p)[off]);
    case SUPA_AMD_I32: return static_cast<C>(static_cast<const int32_t*>(p)[off]);
    case SUPA_AMD_I16: return static_cast<C>(static_cast<const int16_t*>(p)[off]);
    case SUPA_AMD_I8: return static_cast<C>(static_cast<const int8_t*>(p)[off]);
    case SUPA_AMD_U8: return static_cast<C>(static_cast<const uint8_t*>(p)[off]);
    default: return static_cast<C>(static_cast<const uint8_t*>(p)[off] != 0);
  }
}

// Round an arithmetic value to what dtype can hold, returned in type C
// (the "cast to common dtype" step of the dynamic path).
template <typename C>
__device__ __forceinline__ C round_to_dtype(C v, int dtype) {
  switch (dtype) {
    case SUPA_AMD_F32: return static_cast<C>(static_cast<float>(v));
    case SUPA_AMD_BF16: return static_cast<C>(bf16_to_f32(f32_to_bf16(static_cast<float>(v))));
    case SUPA_AMD_F16: return static_cast<C>(static_cast<float>(f32_to_f16(static_cast<float>(v))));
    case SUPA_AMD_F64: return static_cast<C>(static_cast<double>(v));
    case SUPA_AMD_I64: return static_cast<C>(static_cast<int64_t>(v));
    case SUPA_AMD_I32: return static_cast<C>(static_cast<int32_t>(v));
    case SUPA_AMD_I16: return static_cast<C>(static_cast<int16_t>(v));
    case SUPA_AMD_I8: return static_cast<C>(static_cast<int8_t>(v));
    case SUPA_AMD_U8: return static_cast<C>(static_cast<uint8_t>(v));
    default: return static_cast<C>(v != C(0));
  }
}

template <typename C>
__device__ __forceinline__ void store_dyn(void* p, int64_t off, int dtype, C v) {
  switch (dtype) {
    case SUPA_AMD_F32: static_cast<float*>(p)[off] = static_cast<float>(v); break;
    case SUPA_AMD_BF16: static_cast<bf16*>(p)[off] = f32_to_bf16(static_cast<float>(v)); break;
    case SUPA_AMD_F16: static_cast<f16*>(p)[off] = f32_to_f16(static_cast<float>(v)); break;
    case SUPA_AMD_F64: static_cast<double*>(p)[off] = static_cast<double>(v); break;
    case SUPA_AMD_I64: static_cast<int64_t*>(p)[off] = static_cast<int64_t>(v); break;
    case SUPA_AMD_I32: static_cast<int32_t*>(p)[off] = static_cast<int32_t>(v); break;
    case SUPA_AMD_I16: static_cast<int16_t*>(p)[off] = static_cast<int16_t>(v); break;
    case SUPA_AMD_I8: static_cast<int8_t*>(p)[off] = static_cast<int8_t>(v); break;
    case SUPA_AMD_U8: static_cast<uint8_t*>(p)[off] = static_cast<uint8_t>(v); break;
    default: static_cast<uint8_t*>(p)[off] = (v != C(0)) ? 1 : 0; break;
  }
}

__host__ __device__ inline int dtype_size(int dtype) {
  switch (dtype) {
    case SUPA_AMD_F64:
    case SUPA_AMD_I64: return 8;
    case SUPA_AMD_F32:
    case SUPA_AMD_I32: return 4;
    case SUPA_AMD_BF16:
    case SUPA_AMD_F16:
    case SUPA_AMD_I16: return 2;
    default: return 1;
  }
}

inline bool dtype_is_floating(int dtype) {
  return dtype == SUPA_AMD_F32 || dtype == SUPA_AMD_BF16 || dtype == SUPA_AMD_F16 || dtype == SUPA_AMD_F64;
}
inline bool dtype_is_known(int dtype) {
  switch (dtype) {
    case SUPA_AMD_U8: case SUPA_AMD_I8: case SUPA_AMD_I16: case SUPA_AMD_I32: case SUPA_AMD_I64:
    case SUPA_AMD_F16: case SUPA_AMD_F32: case SUPA_AMD_F64: case SUPA_AMD_BOOL: case SUPA_AMD_BF16:
      return true;
    default:
      return false;
  }
}

}  // namespace sa
