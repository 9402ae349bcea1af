// Host side of the elementwise engine: validates a descriptor, binds
// immediate scalars, picks the dtype and layout class and launches.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>

#include "ew_engine.h"
#include "split32.h"

namespace sa {

__host__ __device__ inline bool aligned(const void* p, int bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

// 1 / 2 when the common dtype is bf16 / f16, else 0: the ops that follow
// upstream's scalar_t arithmetic round their intermediates to that type.
inline int half_code(const supa_amd_ew_desc* d) {
  return d->common_dtype == SUPA_AMD_BF16 ? 1 : (d->common_dtype == SUPA_AMD_F16 ? 2 : 0);
}

// Host-side rounding of a float to bf16 / f16 precision (round to nearest
// even; NaN kept NaN), for parameters a kernel takes already rounded.
inline float host_round_bf16(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return f;
  u += 0x7fffu + ((u >> 16) & 1u);
  u &= 0xffff0000u;
  float r;
  __builtin_memcpy(&r, &u, 4);
  return r;
}
inline float host_round_f16(float f) {
  const float a = std::fabs(f);
  if (a != a) return f;
  if (!(a < 65520.0f)) return std::copysign(HUGE_VALF, f);  // rounds past the largest finite f16
  if (a < 6.103515625e-05f) return std::nearbyint(f * 16777216.0f) / 16777216.0f;  // subnormal: 2^-24 steps
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  u += 0xfffu + ((u >> 13) & 1u);
  u &= ~0x1fffu;
  float r;
  __builtin_memcpy(&r, &u, 4);
  return r;
}
// A kernel parameter in the compute type C: v rounded to the 16-bit storage
// type for `half` 1 / 2 (upstream's scalar_t parameters), else C(v).
template <typename C> inline C storage_param(double v, int half) {
  if (half == 1) return static_cast<C>(host_round_bf16(static_cast<float>(v)));
  if (half == 2) return static_cast<C>(host_round_f16(static_cast<float>(v)));
  return static_cast<C>(v);
}

inline int64_t desc_numel(const supa_amd_ew_desc* d) {
  int64_t n = 1;
  for (int i = 0; i < d->ndim; ++i) n *= d->sizes[i];
  return n;
}

inline int check_desc(const supa_amd_ew_desc* d, int min_ops, int max_ops) {
  if (!d) return SUPA_AMD_EINVAL;
  if (d->ndim < 0 || d->ndim > SUPA_AMD_MAX_DIMS) return SUPA_AMD_EINVAL;
  if (d->noperands < min_ops || d->noperands > max_ops || d->noperands > SUPA_AMD_MAX_OPERANDS)
    return SUPA_AMD_EINVAL;
  for (int i = 0; i < d->ndim; ++i)
    if (d->sizes[i] < 0) return SUPA_AMD_EINVAL;
  if (!dtype_is_known(d->common_dtype)) return SUPA_AMD_EDTYPE;
  for (int k = 0; k < d->noperands; ++k) {
    const supa_amd_operand& o = d->op[k];
    if (!dtype_is_known(o.dtype)) return SUPA_AMD_EDTYPE;
    if (!o.is_scalar && !o.data && desc_numel(d) > 0) return SUPA_AMD_EINVAL;
  }
  if (d->op[0].is_scalar) return SUPA_AMD_EINVAL;
  return SUPA_AMD_OK;
}

// Calls fn(sub_desc) on pieces whose element count is below 2^31, so the
// 32-bit coordinate arithmetic of the N-d kernels is exact (split32.h).
template <typename Fn>
int for_each_32bit_piece(const supa_amd_ew_desc& d, Fn&& fn) {
  return split_32bit(d, fn, [](int dtype) { return (int64_t)dtype_size(dtype); });
}

inline NdGeom make_geom(const supa_amd_ew_desc& d) {
  NdGeom g;
  g.ndim = d.ndim;
  for (int i = 0; i < SUPA_AMD_MAX_DIMS; ++i) {
    g.size[i] = i < d.ndim ? (uint32_t)d.sizes[i] : 1u;
    g.div[i] = FastDiv(i < d.ndim ? (uint32_t)std::max<int64_t>(d.sizes[i], 1) : 1u);
  }
  return g;
}

inline int launch_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SUPA_AMD_OK : (int)e;
}

template <typename T> inline T scalar_as(const supa_amd_operand& o) {
  if constexpr (std::is_same<T, bool>::value) return o.iscalar != 0 || o.scalar != 0.0;
  else if constexpr (std::is_floating_point<T>::value) return static_cast<T>(o.scalar);
  else return static_cast<T>(o.iscalar);
}

// Storage type for a dtype code, as a template callback.
template <typename F>
inline int with_storage(int dtype, F&& f) {
  switch (dtype) {
    case SUPA_AMD_F32: return f((float*)nullptr);
    case SUPA_AMD_BF16: return f((bf16*)nullptr);
    case SUPA_AMD_F16: return f((f16*)nullptr);
    case SUPA_AMD_F64: return f((double*)nullptr);
    case SUPA_AMD_I64: return f((int64_t*)nullptr);
    case SUPA_AMD_I32: return f((int32_t*)nullptr);
    case SUPA_AMD_I16: return f((int16_t*)nullptr);
    case SUPA_AMD_I8: return f((int8_t*)nullptr);
    case SUPA_AMD_U8: return f((uint8_t*)nullptr);
    case SUPA_AMD_BOOL: return f((b8*)nullptr);
    default: return SUPA_AMD_EDTYPE;
  }
}

template <typename T> constexpr int cmin(T a, T b) { return a < b ? a : b; }
template <typename T> constexpr int cmax(T a, T b) { return a < b ? b : a; }
template <typename... S> constexpr int min_size() {
  int m = 16;
  ((m = cmin<int>(m, (int)sizeof(S))), ...);
  return m;
}
template <typename... S> constexpr int max_size() {
  int m = 1;
  ((m = cmax<int>(m, (int)sizeof(S))), ...);
  return m;
}

// Static-dtype launch: output OT, inputs S..., common CT, compute C.
template <typename Op, typename C, typename CT, typename OT, typename... S>
int launch_static(const Op& op, const supa_amd_ew_desc& d, const int* tin, hipStream_t st) {
  constexpr int N = sizeof...(S);
  // one storage type per tensor input of the (scalar-bound) op
  static_assert(N == Op::arity, "launch_static: the input storage types must match the op's tensor inputs");
  // one 16-byte access for the widest operand: a bf16 -> f32 widening moves
  // 8-byte input and 16-byte output vectors (66 % faster than 16 / 32 bytes)
  constexpr int VEC0 = 16 / max_size<OT, S...>();
  constexpr int VEC = VEC0 < 1 ? 1 : VEC0;
  const int64_t n = desc_numel(&d);
  if (n == 0) return SUPA_AMD_OK;
  TArgs<1 + N> a;
  a.p[0] = d.op[0].data;
  for (int j = 0; j < SUPA_AMD_MAX_DIMS; ++j) a.st[0][j] = j < d.ndim ? d.op[0].strides[j] : 0;
  a.mode[0] = 0;
  for (int i = 0; i < N; ++i) {
    const supa_amd_operand& o = d.op[tin[i]];
    a.p[1 + i] = o.data;
    for (int j = 0; j < SUPA_AMD_MAX_DIMS; ++j) a.st[1 + i][j] = j < d.ndim ? o.strides[j] : 0;
    a.mode[1 + i] = 0;
  }
  const int sizes_of[1 + N > 0 ? 1 + N : 1] = {(int)sizeof(OT), (int)sizeof(S)...};

  // CONTIG?
  bool contig = d.ndim <= 1;
  if (contig && d.ndim == 1 && n > 1) {
    if (a.st[0][0] != 1) contig = false;
    for (int i = 0; i < N && contig; ++i) {
      if (a.st[1 + i][0] == 0) a.mode[1 + i] = 1;
      else if (a.st[1 + i][0] != 1) contig = false;
    }
  } else if (contig) {
    for (int i = 0; i < N; ++i) a.mode[1 + i] = 1;  // one element: read element 0
  }
  if (contig) {
    bool al = true;
    for (int k = 0; k <= N; ++k)
      if (!(k > 0 && a.mode[k]) && !aligned(a.p[k], VEC * sizes_of[k])) al = false;
    if (al && n / VEC < (int64_t(1) << 31)) {  // grid of at most 2^31 threads
      // write-only streams (fills) keep four wavefronts per workgroup: 83-85 %
      // of peak against 47-60 % with one
      constexpr int BS = N == 0 ? kBlock : kStreamBlock;
      constexpr int U = contig_unroll<Op>();
      int64_t blocks, nfull = 0;
      if (U == 1) {  // one guarded vector per thread
        blocks = std::max<int64_t>(1, (n / VEC + BS - 1) / BS);
      } else {  // full tiles of BS * U vectors, plus one workgroup for the rest
        nfull = n / VEC / (BS * U);
        blocks = nfull + (nfull * BS * U * VEC < n ? 1 : 0);
      }
      int dense = 0;  // tensor inputs (not one-element broadcasts)
      for (int k = 1; k <= N; ++k) dense += a.mode[k] == 0 ? 1 : 0;
      const unsigned lds = CapsOccupancy<Op>::value && dense >= 3 && blocks >= (1 << 17) ? kStreamCapLds : 0u;
      k_contig<BS, VEC, Op, C, CT, OT, S...><<<dim3((unsigned)blocks), dim3(BS), lds, st>>>(op, a, n,
                                                                                            (uint32_t)nfull);
      return launch_status();
    }
  }
  return for_each_32bit_piece(d, [&](const supa_amd_ew_desc& p) -> int {
    const int64_t pn = desc_numel(&p);
    if (pn == 0) return SUPA_AMD_OK;
    TArgs<1 + N> b = a;
    b.p[0] = p.op[0].data;
    for (int i = 0; i < N; ++i) b.p[1 + i] = p.op[tin[i]].data;
    // TRANSPOSE?  One input, dense output, the input contiguous along dim 1 or 2.
    if constexpr (N == 1) {
      if ((p.ndim == 2 || p.ndim == 3) && b.st[0][0] == 1 && b.st[0][1] == p.sizes[0] &&
          (p.ndim == 2 || b.st[0][2] == p.sizes[0] * p.sizes[1]) && b.st[1][0] != 1 && b.st[1][0] != 0 &&
          p.sizes[0] >= 16) {
        int k = -1;
        for (int j = 1; j < p.ndim; ++j)
          if (b.st[1][j] == 1 && p.sizes[j] >= 16) k = j;
        if (k > 0) {
          const int bd = p.ndim == 3 ? 3 - k : -1;  // the batch dim
          TransposeGeom tg;
          tg.d0 = (uint32_t)p.sizes[0];
          tg.dk = (uint32_t)p.sizes[k];
          tg.db = bd > 0 ? (uint32_t)p.sizes[bd] : 1u;
          tg.in_s0 = b.st[1][0];
          tg.in_sb = bd > 0 ? b.st[1][bd] : 0;
          tg.out_sk = b.st[0][k];
          tg.out_sb = bd > 0 ? b.st[0][bd] : 0;
          using S0 = typename NthT<0, S...>::type;
          constexpr int VI = 16 / (int)sizeof(S0), VO = 16 / (int)sizeof(OT);
          const bool vec = VI > 1 && VO > 1 && tg.d0 % VO == 0 && tg.dk % VI == 0 && tg.in_s0 % VI == 0 &&
                           tg.in_sb % VI == 0 && tg.out_sk % VO == 0 && tg.out_sb % VO == 0 && aligned(b.p[1], 16) &&
                           aligned(b.p[0], 16);
          const uint32_t tile_k = vec ? (uint32_t)tile_k_vec<S0>() : (uint32_t)kTile;  // the kernel's tile width
          const uint32_t t0 = (tg.d0 + kTile - 1) / kTile, tk = (tg.dk + tile_k - 1) / tile_k;
          tg.t0 = FastDiv(t0);
          tg.tk = FastDiv(tk);
          const uint64_t blocks = (uint64_t)t0 * tk * tg.db;
          if (blocks < (1ull << 31)) {
            if (vec)
              k_transpose_vec<Op, C, CT, OT, S0><<<(unsigned)blocks, kTileVecBlock, 0, st>>>(
                  op, static_cast<const S0*>(b.p[1]), static_cast<OT*>(b.p[0]), tg);
            else
              k_transpose<Op, C, CT, OT, S0><<<(unsigned)blocks, kBlock, 0, st>>>(
                  op, static_cast<const S0*>(b.p[1]), static_cast<OT*>(b.p[0]), tg);
            return launch_status();
          }
        }
      }
    }
    // ROW2D?  Two dims, or three with the outer two flattened into rows.
    if ((p.ndim == 2 || p.ndim == 3) && VEC > 1 && (p.sizes[0] % VEC) == 0 && b.st[0][0] == 1 &&
        b.st[0][1] == p.sizes[0] && (p.ndim == 2 || b.st[0][2] == p.sizes[0] * p.sizes[1]) &&
        aligned(b.p[0], VEC * sizes_of[0]) && (uint64_t)pn / VEC < (1ull << 32)) {
      const int64_t d0 = p.sizes[0], d1 = p.sizes[1];
      bool ok = true;
      TArgs<1 + N> c = b;
      c.mode[0] = R2_DENSE;
      for (int k = 1; k <= N && ok; ++k) {
        const int64_t s0 = b.st[k][0], s1 = b.st[k][1], s2 = p.ndim == 3 ? b.st[k][2] : -1;
        const bool two = p.ndim == 2;
        if (s0 == 1 && s1 == d0 && (two || s2 == d0 * d1)) c.mode[k] = R2_DENSE;
        else if (s0 == 1 && s1 == 0 && (two || s2 == 0)) c.mode[k] = R2_ROW;
        else if (s0 == 0 && s1 == 1 && (two || s2 == d1)) c.mode[k] = R2_COL;
        else if (s0 == 0 && s1 == 0 && (two || s2 == 0)) c.mode[k] = R2_ONE;
        else if (!two && s0 == 0 && s1 == 1 && s2 == 0) c.mode[k] = R2_MID;
        else ok = false;
        if (ok && s0 == 1 && !aligned(b.p[k], VEC * sizes_of[k])) ok = false;
      }
      if (ok) {
        const uint32_t inner = (uint32_t)d0;
        const uint32_t rows = (uint32_t)(pn / d0);
        const uint32_t bpr = (inner / VEC + kStreamBlock - 1) / kStreamBlock;
        const uint32_t K = row2d_pair(inner * (uint32_t)sizeof(OT), rows);
        if constexpr (IsRowB<Op>::value) {
          // long rows: one vector per thread (k_rowb), the functor's rounding
          // and mean switches fixed at compile time (kRowB functors carry
          // rt, mean and fixed<RT, MEAN>())
          constexpr int kRt = std::is_same<OT, bf16>::value ? 1 : (std::is_same<OT, f16>::value ? 2 : 0);
          bool rb = K == 1 && (uint64_t)inner * sizeof(OT) > kPairBytes / 2 && op.rt == kRt;
          for (int k = 1; k <= N && rb; ++k)
            if (c.mode[k] == R2_MID) rb = false;
          if (rb) {
            const uint32_t nvec = (uint32_t)(pn / VEC);
            const unsigned nb = (nvec + kStreamBlock - 1) / kStreamBlock;
            const FastDiv ivec(inner / VEC);
            if (op.mean) {
              const auto fop = op.template fixed<kRt, 1>();
              k_rowb<VEC, decltype(fop), C, CT, OT, S...><<<nb, kStreamBlock, 0, st>>>(fop, c, nvec, ivec);
            } else {
              const auto fop = op.template fixed<kRt, 0>();
              k_rowb<VEC, decltype(fop), C, CT, OT, S...><<<nb, kStreamBlock, 0, st>>>(fop, c, nvec, ivec);
            }
            return launch_status();
          }
        }
        const uint64_t blocks = (uint64_t)bpr * K * ((rows + kRow2dRows * K - 1) / (kRow2dRows * K));
        if (blocks < (1ull << 31)) {
          // long launches: dynamic LDS the kernel does not use caps residency
          // at 26 one-wave workgroups per CU (c2's bias add 81.7-82.3 ->
          // 83.3-83.7 % of the HBM roofline; short launches lose from it)
          const unsigned lds = blocks >= (1u << 19) ? 6144u : 0u;
          k_row2d<kStreamBlock, VEC, Op, C, CT, OT, S...><<<(unsigned)blocks, kStreamBlock, lds, st>>>(
              op, c, inner, rows, FastDiv(bpr), FastDiv((uint32_t)d1), FastDiv(K));
          return launch_status();
        }
      }
    }
    const NdGeom g = make_geom(p);
    // every operand's largest element offset below 2^31: 32-bit offset math
    bool off32 = true;
    for (int k = 0; k <= N; ++k) {
      int64_t mx = 0;
      for (int j = 0; j < p.ndim; ++j) mx += (p.sizes[j] - 1) * (b.st[k][j] < 0 ? -b.st[k][j] : b.st[k][j]);
      if (mx >= (int64_t(1) << 31)) off32 = false;
    }
    // VECND?
    bool vnd = p.ndim >= 1 && (p.sizes[0] % VEC) == 0 && b.st[0][0] == 1 && VEC > 1;
    for (int k = 0; k <= N && vnd; ++k) {
      const int64_t s0 = b.st[k][0];
      if (s0 != 0 && s0 != 1) { vnd = false; break; }
      if (s0 == 1) {
        if (!aligned(b.p[k], VEC * sizes_of[k])) vnd = false;
        for (int j = 1; j < p.ndim; ++j)
          if (b.st[k][j] % VEC) vnd = false;
      }
    }
    if (vnd) {
      // operands broadcast along some outer dim are re-read: keep them cached
      for (int k = 1; k <= N; ++k) {
        b.mode[k] = 0;
        for (int j = 1; j < p.ndim; ++j)
          if (b.st[k][j] == 0 && p.sizes[j] > 1) b.mode[k] = 1;
      }
      const uint32_t nvec = (uint32_t)(pn / VEC);
      const unsigned blocks = (nvec + kStreamBlock - 1) / kStreamBlock;
      if (off32) k_vecnd<VEC, int32_t, Op, C, CT, OT, S...><<<blocks, kStreamBlock, 0, st>>>(op, b, g, nvec);
      else k_vecnd<VEC, int64_t, Op, C, CT, OT, S...><<<blocks, kStreamBlock, 0, st>>>(op, b, g, nvec);
      return launch_status();
    }
    const unsigned blocks = (unsigned)((pn + kStreamBlock - 1) / kStreamBlock);
    if (off32) k_strided<int32_t, Op, C, CT, OT, S...><<<blocks, kStreamBlock, 0, st>>>(op, b, g, (uint32_t)pn);
    else k_strided<int64_t, Op, C, CT, OT, S...><<<blocks, kStreamBlock, 0, st>>>(op, b, g, (uint32_t)pn);
    return launch_status();
  });
}

template <int NT, typename Op, typename C>
int launch_dynamic(const Op& op, const supa_amd_ew_desc& d, const int* tin, int common, hipStream_t st) {
  return for_each_32bit_piece(d, [&](const supa_amd_ew_desc& p) -> int {
    const int64_t pn = desc_numel(&p);
    if (pn == 0) return SUPA_AMD_OK;
    TArgs<NT> a;
    DynTypes<NT> t;
    t.common = common;
    for (int k = 0; k < NT; ++k) {
      const supa_amd_operand& o = p.op[k == 0 ? 0 : tin[k - 1]];
      a.p[k] = o.data;
      a.mode[k] = 0;
      t.dtype[k] = o.dtype;
      for (int j = 0; j < SUPA_AMD_MAX_DIMS; ++j) a.st[k][j] = j < p.ndim ? o.strides[j] : 0;
    }
    const NdGeom g = make_geom(p);
    const unsigned blocks = (unsigned)((pn + kBlock - 1) / kBlock);
    k_dynamic<NT, Op, C><<<blocks, kBlock, 0, st>>>(op, a, t, g, (uint32_t)pn);
    return launch_status();
  });
}

// Compute type used for a storage type: float for the float32/16-bit floats,
// double for float64, bool for bool, int64 for every integer type (wrapping
// add/sub/mul are exact modulo 2^bits, so the narrow result is the same).
template <typename T, typename C> constexpr bool compute_compatible() {
  if constexpr (std::is_same<C, float>::value)
    return std::is_same<T, float>::value || std::is_same<T, bf16>::value || std::is_same<T, f16>::value;
  else if constexpr (std::is_same<C, double>::value) return std::is_same<T, double>::value;
  else if constexpr (std::is_same<C, bool>::value) return std::is_same<T, b8>::value;
  else return std::is_integral<T>::value;
}

// Dispatch over storage types once the op (with scalars bound) is fixed.
// N = number of tensor inputs.
template <int N, typename Op, typename C>
int dispatch_types(const Op& op, const supa_amd_ew_desc& d, const int* tin, hipStream_t st) {
  const int common = d.common_dtype;
  bool same = d.op[0].dtype == common;
  for (int i = 0; i < N; ++i) same = same && d.op[tin[i]].dtype == common;
  if (same) {
    return with_storage(common, [&](auto* tag) -> int {
      using T = std::remove_pointer_t<decltype(tag)>;
      if constexpr (!compute_compatible<T, C>()) {
        return SUPA_AMD_EDTYPE;
      } else if constexpr (N == 0) {
        return launch_static<Op, C, T, T>(op, d, tin, st);
      } else if constexpr (N == 1) {
        return launch_static<Op, C, T, T, T>(op, d, tin, st);
      } else if constexpr (N == 2) {
        return launch_static<Op, C, T, T, T, T>(op, d, tin, st);
      } else if constexpr (N == 3) {
        return launch_static<Op, C, T, T, T, T, T>(op, d, tin, st);
      } else if constexpr (N == 4) {
        return launch_static<Op, C, T, T, T, T, T, T>(op, d, tin, st);
      } else {
        return launch_static<Op, C, T, T, T, T, T, T, T>(op, d, tin, st);
      }
    });
  }
  constexpr int mode = DtypeModeOf<Op>::value;
  if constexpr (mode == 1 && N >= 1 && N <= 2) {  // bool output, common-dtype inputs
    bool ok = d.op[0].dtype == SUPA_AMD_BOOL && common != SUPA_AMD_BOOL;
    for (int i = 0; i < N; ++i) ok = ok && d.op[tin[i]].dtype == common;
    if (ok) {
      return with_storage(common, [&](auto* tag) -> int {
        using T = std::remove_pointer_t<decltype(tag)>;
        if constexpr (!compute_compatible<T, C>()) return SUPA_AMD_EDTYPE;
        else if constexpr (N == 1) return launch_static<Op, C, T, b8, T>(op, d, tin, st);
        else return launch_static<Op, C, T, b8, T, T>(op, d, tin, st);
      });
    }
  }
  if constexpr (mode == 2 && N >= 1 && N <= 3) {  // bool first input, the rest common
    bool ok = d.op[0].dtype == common && d.op[tin[0]].dtype == SUPA_AMD_BOOL && common != SUPA_AMD_BOOL;
    for (int i = 1; i < N; ++i) ok = ok && d.op[tin[i]].dtype == common;
    if (ok) {
      return with_storage(common, [&](auto* tag) -> int {
        using T = std::remove_pointer_t<decltype(tag)>;
        if constexpr (!compute_compatible<T, C>()) return SUPA_AMD_EDTYPE;
        else if constexpr (N == 1) return launch_static<Op, C, T, T, b8>(op, d, tin, st);
        else if constexpr (N == 2) return launch_static<Op, C, T, T, b8, T>(op, d, tin, st);
        else return launch_static<Op, C, T, T, b8, T, T>(op, d, tin, st);
      });
    }
  }
  if constexpr (std::is_same<C, float>::value && N == 2 && LowpMixOf<Op>::value) {
    // bf16 / f16 common dtype and output, one input a 0-dim float32 tensor
    const int d0 = d.op[tin[0]].dtype, d1 = d.op[tin[1]].dtype;
    if ((common == SUPA_AMD_BF16 || common == SUPA_AMD_F16) && d.op[0].dtype == common &&
        ((d0 == common && d1 == SUPA_AMD_F32) || (d0 == SUPA_AMD_F32 && d1 == common))) {
      const int fpos = d1 == SUPA_AMD_F32 ? 1 : 0;
      const supa_amd_operand& fo = d.op[tin[fpos]];
      bool one = true;
      for (int j = 0; j < d.ndim; ++j) one = one && fo.strides[j] == 0;
      if (one) {
        const int rest[1] = {tin[1 - fpos]};
        auto go = [&](auto* tag) -> int {
          using T = std::remove_pointer_t<decltype(tag)>;
          using B = BindDev1<Op, float, T, float>;
          const B b{op, fpos, static_cast<const float*>(fo.data)};
          return launch_static<B, float, T, T, T>(b, d, rest, st);
        };
        return common == SUPA_AMD_BF16 ? go((bf16*)nullptr) : go((f16*)nullptr);
      }
    }
  }
  if constexpr (std::is_same<C, float>::value && N >= 1 && N <= 2) {
    auto fam = [](int dt) { return dt == SUPA_AMD_F32 || dt == SUPA_AMD_BF16 || dt == SUPA_AMD_F16; };
    bool mixed = common == SUPA_AMD_F32 && d.op[0].dtype == SUPA_AMD_F32;
    for (int i = 0; i < N; ++i) mixed = mixed && fam(d.op[tin[i]].dtype);
    if (mixed) {
      auto w16 = [](int dt, auto&& f) -> int {
        if (dt == SUPA_AMD_F32) return f((float*)nullptr);
        if (dt == SUPA_AMD_BF16) return f((bf16*)nullptr);
        return f((f16*)nullptr);
      };
      if constexpr (N == 1) {
        return w16(d.op[tin[0]].dtype, [&](auto* t0) -> int {
          using S0 = std::remove_pointer_t<decltype(t0)>;
          return launch_static<Op, float, float, float, S0>(op, d, tin, st);
        });
      } else {
        return w16(d.op[tin[0]].dtype, [&](auto* t0) -> int {
          return w16(d.op[tin[1]].dtype, [&](auto* t1) -> int {
            using S0 = std::remove_pointer_t<decltype(t0)>;
            using S1 = std::remove_pointer_t<decltype(t1)>;
            return launch_static<Op, float, float, float, S0, S1>(op, d, tin, st);
          });
        });
      }
    }
  }
  return launch_dynamic<N + 1, Op, C>(op, d, tin, common, st);
}

// Entry: Factory::make<C>() builds the op for compute type C;
// Factory::ok<C>() says whether the op exists for C.  Immediate scalar inputs
// (at most two) are bound into the functor.
template <typename C, typename Factory>
int run_with_compute(const Factory& f, const supa_amd_ew_desc& d, hipStream_t st) {
  if constexpr (!Factory::template ok<C>()) {
    return SUPA_AMD_EDTYPE;
  } else {
    using Op = decltype(f.template make<C>());
    constexpr int A = Op::arity;
    if (d.noperands != A + 1) return SUPA_AMD_EINVAL;
    int tin[kMaxIn];
    int sc[kMaxIn];
    int nt = 0, ns = 0;
    for (int k = 1; k < d.noperands; ++k) {
      if (d.op[k].is_scalar) sc[ns++] = k;
      else tin[nt++] = k;
    }
    const Op op = f.template make<C>();
    if (ns == 0) {
      return dispatch_types<A, Op, C>(op, d, tin, st);
    }
    if constexpr (A >= 1) {
      if (ns == 1) {
        Bind1<Op, C> b{op, sc[0] - 1, scalar_as<C>(d.op[sc[0]])};
        return dispatch_types<A - 1, Bind1<Op, C>, C>(b, d, tin, st);
      }
    }
    if constexpr (A >= 3) {
      if (ns == 2) {
        // bind the later position first so the earlier index stays valid
        Bind1<Op, C> b1{op, sc[1] - 1, scalar_as<C>(d.op[sc[1]])};
        Bind1<Bind1<Op, C>, C> b2{b1, sc[0] - 1, scalar_as<C>(d.op[sc[0]])};
        return dispatch_types<A - 2, Bind1<Bind1<Op, C>, C>, C>(b2, d, tin, st);
      }
    }
    return SUPA_AMD_EINVAL;
  }
}

template <typename Factory>
int run_ew(const Factory& f, const supa_amd_ew_desc* d, void* stream, int min_ops = 1) {
  const int rc = check_desc(d, min_ops, SUPA_AMD_MAX_OPERANDS);
  if (rc) return rc;
  if (desc_numel(d) == 0) return SUPA_AMD_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (d->common_dtype) {
    case SUPA_AMD_F32:
    case SUPA_AMD_BF16:
    case SUPA_AMD_F16: return run_with_compute<float>(f, *d, st);
    case SUPA_AMD_F64: return run_with_compute<double>(f, *d, st);
    case SUPA_AMD_BOOL: return run_with_compute<bool>(f, *d, st);
    default: return run_with_compute<int64_t>(f, *d, st);
  }
}

}  // namespace sa
