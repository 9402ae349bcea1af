// Generic multi-tensor apply for the _foreach_* family: one kernel template
// covers the unary, binary (List / ScalarList / device-scalar Tensor forms)
// and pointwise ternary ops (addcmul, addcdiv, lerp), pow in its three forms,
// _foreach_copy_ and _foreach_zero_; and a two-kernel _foreach_norm.
//
// Arithmetic per element is the one the elementwise kernels use (ops.h), in
// the storage type's opmath, so _foreach_op(xs, ys)[k] equals op(xs[k], ys[k])
// bit for bit.  The reference's counterparts are upstream ForeachBinaryOp*.cu,
// ForeachPointwiseOp.cu, ForeachTernaryOp.cu, ForeachUnaryOp.cu and
// ForeachReduceOp.cu, all over MultiTensorApply.cuh.
#include "mta.h"
#include "ops.h"

namespace sa {

struct MtaTable {
  void* out[kMtaTensors];
  const void* in[3][kMtaTensors];
  double s[kMtaTensors];  // per-tensor scalar (ScalarList; a Scalar repeats)
  int64_t numel[kMtaTensors];
  uint32_t chunk_start[kMtaTensors + 1];
  int32_t ntensors;
  uint32_t bucket_shift;
  MtaBucket bucket[kMtaBuckets];
};

constexpr int kFeList = SUPA_AMD_FOREACH_LIST;
constexpr int kFeScalars = SUPA_AMD_FOREACH_SCALARS;
constexpr int kFeDev = SUPA_AMD_FOREACH_DEVSCALAR;
constexpr int kFeUnary = SUPA_AMD_FOREACH_UNARY;

// Tensor operands an op reads (the output is not counted).
constexpr int fe_inputs(int op, int form) {
  return op == SUPA_AMD_FOREACH_ZERO                                         ? 0
         : op >= kFeUnary                                                    ? 1
         : (op == SUPA_AMD_FOREACH_ADDCMUL || op == SUPA_AMD_FOREACH_ADDCDIV) ? 3
         : op == SUPA_AMD_FOREACH_LERP                                       ? (form == kFeList ? 3 : 2)
                                                                             : (form == kFeList ? 2 : 1);
}

// base ** e for a per-tensor exponent e that is exact in the storage type T,
// evaluated as the per-tensor pow(Tensor, Scalar) evaluates it: upstream
// pow_out's fill / copy for 0 and 1, its sqrt / rsqrt / reciprocal routes for
// 0.5 / -0.5 / -1, then pow_tensor_scalar_kernel's 2 / 3 / -2 special cases
// (PowScalarOp) and pow in double rounded once.
template <typename T, typename C>
__device__ __forceinline__ C fe_pow_scalar(C b, C e) {
  if (e == C(0)) return C(1);
  if (e == C(1)) return b;
  if (e == C(0.5)) return sqrt(b);
  if (e == C(-0.5)) return C(1) / sqrt(b);
  if (e == C(-1)) return C(1) / b;
  constexpr int half = std::is_same<T, bf16>::value ? 1 : (std::is_same<T, f16>::value ? 2 : 0);
  const int mode = e == C(2) ? POW_SQUARE : e == C(3) ? POW_CUBE : e == C(-2) ? POW_INV_SQUARE : POW_GENERAL;
  const C xb[1] = {b};
  return PowScalarOp<C>{mode, half, (double)e}(xb);
}

// One element.  x[0..NIN) are the loaded operands, s the tensor's scalar
// (or the device scalar), al the add/sub alpha.
template <typename T, int OP, int FORM, typename C>
__device__ __forceinline__ C fe_apply(const C* x, C s, C al) {
  if constexpr (OP == SUPA_AMD_FOREACH_ZERO) {
    return C(0);
  } else if constexpr (OP == SUPA_AMD_FOREACH_COPY) {
    return x[0];
  } else if constexpr (OP == SUPA_AMD_FOREACH_POW) {
    if constexpr (FORM == kFeList) return PowOp<C>{}(x);
    else return fe_pow_scalar<T, C>(x[0], s);
  } else if constexpr (OP == SUPA_AMD_FOREACH_RPOW) {
    const C sx[2] = {s, x[0]};
    return PowOp<C>{}(sx);
  } else if constexpr (OP >= kFeUnary) {
    return UnaryOp<OP - kFeUnary, C>{}(x);
  } else if constexpr (OP == SUPA_AMD_FOREACH_ADDCMUL) {
    return AddcmulOp<C>{s}(x);
  } else if constexpr (OP == SUPA_AMD_FOREACH_ADDCDIV) {
    return AddcdivOp<C>{s}(x);
  } else if constexpr (OP == SUPA_AMD_FOREACH_LERP) {
    const C w[3] = {x[0], x[1], FORM == kFeList ? x[2] : s};
    return LerpOp<C>{}(w);
  } else {
    const C y = FORM == kFeList ? x[1] : s;
    const C xy[2] = {x[0], y};
    if constexpr (OP == SUPA_AMD_FOREACH_ADD) return muladd<C>(al, y, x[0]);
    else if constexpr (OP == SUPA_AMD_FOREACH_MUL) return x[0] * y;
    else if constexpr (OP == SUPA_AMD_FOREACH_DIV) return x[0] / y;
    else if constexpr (OP == SUPA_AMD_FOREACH_MAXIMUM) return MaxOp<C>{}(xy);
    else return MinOp<C>{}(xy);
  }
}

// One chunk per workgroup: one 16-byte vector per operand per thread (two
// for _foreach_zero_, which only writes), all loads issued before the math;
// bases not 16-byte aligned and the last partial vector take the scalar
// path.  With the 32-bit chunk index one vector per thread is the fastest
// for the one-input forms too: _foreach_mul_.Scalar over c5's 72 tensors
// 86.7 % of the HBM roofline against 80.5 % with two and 78.7 % with four.
template <typename T, int OP, int FORM, int64_t CHUNK>
__global__ void __launch_bounds__(kMtaBlock)
k_foreach(MtaTable tab, double alpha, const void* sp) {
  using C = opmath_t<T>;
  constexpr int NIN = fe_inputs(OP, FORM);
  constexpr int NL = NIN > 0 ? NIN : 1;
  constexpr int V = 16 / sizeof(T);
  const MtaRange r = mta_range<CHUNK>(tab);
  T* out = static_cast<T*>(tab.out[r.k]);
  const T* in[NL];
  bool vec = aligned(out, 16);
#pragma unroll
  for (int j = 0; j < NIN; ++j) {
    in[j] = static_cast<const T*>(tab.in[j][r.k]);
    vec = vec && aligned(in[j], 16);
  }
  C s;
  if constexpr (FORM == kFeDev) s = (C)to_arith(*static_cast<const T*>(sp));
  else s = (C)tab.s[r.k];
  const C al = (C)alpha;
  int64_t start = r.lo;
  if (vec) {
    const int64_t nv = (r.hi - r.lo) / V;
    for (int64_t v = threadIdx.x; v < nv; v += kMtaBlock) {
      const int64_t e = r.lo + v * V;
      Vec<T, V> xv[NL];
#pragma unroll
      for (int j = 0; j < NIN; ++j) xv[j] = ld_stream(reinterpret_cast<const Vec<T, V>*>(in[j] + e));
      Vec<T, V> res;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        C xi[NL];
#pragma unroll
        for (int j = 0; j < NIN; ++j) xi[j] = (C)to_arith(xv[j].v[i]);
        res.v[i] = from_arith<T>(fe_apply<T, OP, FORM, C>(xi, s, al));
      }
      st_stream(reinterpret_cast<Vec<T, V>*>(out + e), res);
    }
    start = r.lo + nv * V;
  }
  for (int64_t e = start + threadIdx.x; e < r.hi; e += kMtaBlock) {
    C xi[NL];
#pragma unroll
    for (int j = 0; j < NIN; ++j) xi[j] = (C)to_arith(in[j][e]);
    out[e] = from_arith<T>(fe_apply<T, OP, FORM, C>(xi, s, al));
  }
}

struct FeArgs {
  int32_t n;
  void* const* out;
  const void* const* in[3];
  const int64_t* numel;
  const double* scalars;
  double alpha;
  const void* sp;
};

template <typename T, int OP, int FORM>
int fe_launch(const FeArgs& a, hipStream_t st) {
  constexpr int NIN = fe_inputs(OP, FORM);
  constexpr int64_t CHUNK = NIN >= 1 ? chunk_one<T>() : 2 * chunk_one<T>();
  for (int j = 0; j < NIN; ++j)
    if (!a.in[j]) return SUPA_AMD_EINVAL;
  return mta_for_tables<CHUNK, MtaTable>(
      a.n, a.numel,
      [&](MtaTable& tab, int slot, int i) -> int {
        if (!a.out[i]) return SUPA_AMD_EINVAL;
        tab.out[slot] = a.out[i];
        for (int j = 0; j < NIN; ++j) {
          if (!a.in[j][i]) return SUPA_AMD_EINVAL;
          tab.in[j][slot] = a.in[j][i];
        }
        tab.s[slot] = a.scalars ? a.scalars[i] : 0.0;
        return SUPA_AMD_OK;
      },
      [&](const MtaTable& tab, uint32_t chunks) {
        k_foreach<T, OP, FORM, CHUNK><<<chunks, kMtaBlock, 0, st>>>(tab, a.alpha, a.sp);
      });
}

template <typename T>
int fe_dispatch(int op, int form, const FeArgs& a, hipStream_t st) {
#define SA_FE_BINARY(OPC)                                          \
  case OPC:                                                        \
    if (form == kFeList) return fe_launch<T, OPC, kFeList>(a, st); \
    if (form == kFeScalars) return fe_launch<T, OPC, kFeScalars>(a, st); \
    return fe_launch<T, OPC, kFeDev>(a, st);
#define SA_FE_UNARY(U) \
  case kFeUnary + U: return fe_launch<T, kFeUnary + U, kFeScalars>(a, st);
  switch (op) {
    SA_FE_BINARY(SUPA_AMD_FOREACH_ADD)
    SA_FE_BINARY(SUPA_AMD_FOREACH_MUL)
    SA_FE_BINARY(SUPA_AMD_FOREACH_DIV)
    SA_FE_BINARY(SUPA_AMD_FOREACH_MAXIMUM)
    SA_FE_BINARY(SUPA_AMD_FOREACH_MINIMUM)
    case SUPA_AMD_FOREACH_ADDCMUL: return fe_launch<T, SUPA_AMD_FOREACH_ADDCMUL, kFeScalars>(a, st);
    case SUPA_AMD_FOREACH_ADDCDIV: return fe_launch<T, SUPA_AMD_FOREACH_ADDCDIV, kFeScalars>(a, st);
    case SUPA_AMD_FOREACH_LERP:
      if (form == kFeList) return fe_launch<T, SUPA_AMD_FOREACH_LERP, kFeList>(a, st);
      return fe_launch<T, SUPA_AMD_FOREACH_LERP, kFeScalars>(a, st);
    case SUPA_AMD_FOREACH_ZERO: return fe_launch<T, SUPA_AMD_FOREACH_ZERO, kFeScalars>(a, st);
    case SUPA_AMD_FOREACH_COPY: return fe_launch<T, SUPA_AMD_FOREACH_COPY, kFeScalars>(a, st);
    case SUPA_AMD_FOREACH_POW:
      if (form == kFeList) return fe_launch<T, SUPA_AMD_FOREACH_POW, kFeList>(a, st);
      if (form == kFeScalars) return fe_launch<T, SUPA_AMD_FOREACH_POW, kFeScalars>(a, st);
      return SUPA_AMD_EINVAL;
    case SUPA_AMD_FOREACH_RPOW:
      if (form == kFeScalars) return fe_launch<T, SUPA_AMD_FOREACH_RPOW, kFeScalars>(a, st);
      return SUPA_AMD_EINVAL;
    SA_FE_UNARY(SUPA_AMD_SIGMOID)
    SA_FE_UNARY(SUPA_AMD_TANH)
    SA_FE_UNARY(SUPA_AMD_EXP)
    SA_FE_UNARY(SUPA_AMD_LOG)
    SA_FE_UNARY(SUPA_AMD_ERF)
    SA_FE_UNARY(SUPA_AMD_NEG)
    SA_FE_UNARY(SUPA_AMD_RECIPROCAL)
    SA_FE_UNARY(SUPA_AMD_ABS)
    SA_FE_UNARY(SUPA_AMD_SQRT)
    SA_FE_UNARY(SUPA_AMD_EXPM1)
    SA_FE_UNARY(SUPA_AMD_LOG1P)
    SA_FE_UNARY(SUPA_AMD_SIGN)
    SA_FE_UNARY(SUPA_AMD_FLOOR)
    SA_FE_UNARY(SUPA_AMD_CEIL)
    SA_FE_UNARY(SUPA_AMD_ROUND)
    SA_FE_UNARY(SUPA_AMD_TRUNC)
    SA_FE_UNARY(SUPA_AMD_RSQRT)
    default: return SUPA_AMD_EINVAL;
  }
#undef SA_FE_BINARY
#undef SA_FE_UNARY
}

// ------------------------------------------------------------- norm
constexpr int kOrdInf = 0;
// The norm kernels keep four wavefronts per workgroup: stage 2 walks every
// chunk partial of a tensor with one workgroup.
constexpr int kNormBlock = 256;

template <int ORD, typename A> __device__ __forceinline__ A norm_term(A x) {
  if constexpr (ORD == 2) return x * x;
  else return fabs(x);
}
// inf-norm: max with NaN propagation; 1- and 2-norm: sum (NaN propagates).
template <int ORD, typename A> __device__ __forceinline__ A norm_combine(A a, A b) {
  if constexpr (ORD == kOrdInf) return (a != a || a > b) ? a : b;
  else return a + b;
}
// Reduce over the workgroup; the result is valid in thread 0.
template <int ORD, typename A> __device__ __forceinline__ A norm_block(A v) {
  __shared__ A part[kNormBlock / 64];
  for (int off = 32; off > 0; off >>= 1) v = norm_combine<ORD>(v, __shfl_xor(v, off, 64));
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 1; w < kNormBlock / 64; ++w) v = norm_combine<ORD>(v, part[w]);
  }
  return v;
}

// Stage 1: ws[table base + block] = the combine of |x|^ord over one chunk.
template <typename T, int ORD, int64_t CHUNK>
__global__ void __launch_bounds__(kNormBlock)
k_norm_partial(MtaTable tab, opmath_t<T>* __restrict__ ws) {
  using A = opmath_t<T>;
  constexpr int V = 16 / sizeof(T);
  const MtaRange r = mta_range<CHUNK>(tab);
  const T* x = static_cast<const T*>(tab.in[0][r.k]);
  A acc = A(0);
  int64_t start = r.lo;
  if (aligned(x, 16)) {
    const int64_t nv = (r.hi - r.lo) / V;
    for (int64_t v = threadIdx.x; v < nv; v += kNormBlock) {
      const Vec<T, V> w = ld_stream(reinterpret_cast<const Vec<T, V>*>(x + r.lo + v * V));
#pragma unroll
      for (int i = 0; i < V; ++i) acc = norm_combine<ORD>(acc, norm_term<ORD>((A)to_arith(w.v[i])));
    }
    start = r.lo + nv * V;
  }
  for (int64_t e = start + threadIdx.x; e < r.hi; e += kNormBlock)
    acc = norm_combine<ORD>(acc, norm_term<ORD>((A)to_arith(x[e])));
  acc = norm_block<ORD>(acc);
  if (threadIdx.x == 0) ws[blockIdx.x] = acc;
}

// Stage 2: one workgroup per tensor combines its chunks' partials (none for
// an empty tensor: norm 0) and writes the norm.
template <typename A, typename OT, int ORD>
__global__ void __launch_bounds__(kNormBlock)
k_norm_final(MtaTable tab, const A* __restrict__ ws) {
  const int k = blockIdx.x;
  A acc = fold_strided<8>(
      A(0), (int64_t)tab.chunk_start[k] + threadIdx.x, kNormBlock, (int64_t)tab.chunk_start[k + 1],
      [&](int64_t c) { return ws[c]; }, [](A a, A b) { return norm_combine<ORD>(a, b); });
  acc = norm_block<ORD>(acc);
  if (threadIdx.x == 0) *static_cast<OT*>(tab.out[k]) = from_arith<OT>(ORD == 2 ? sqrt(acc) : acc);
}

// Chunks per table: tensors are packed kMtaTensors at a time, empty ones
// included (they own no chunk; the lookup still finds the non-empty tensor
// that owns a block because it takes the last equal start).
template <int64_t CHUNK, typename F>
int norm_tables(int32_t n, const int64_t* numel, F&& per_table) {
  int i = 0;
  while (i < n) {
    MtaTable tab{};
    uint32_t chunks = 0;
    int nt = 0;
    const int first = i;
    while (i < n && nt < kMtaTensors) {
      if (numel[i] < 0) return SUPA_AMD_EINVAL;
      const int64_t c = (numel[i] + CHUNK - 1) / CHUNK;
      if (c > (int64_t)0x7fffffff) return SUPA_AMD_ELAYOUT;
      if ((int64_t)chunks + c > (int64_t)0x7fffffff) break;
      tab.numel[nt] = numel[i];
      tab.chunk_start[nt] = chunks;
      chunks += (uint32_t)c;
      ++nt;
      ++i;
    }
    tab.chunk_start[nt] = chunks;
    tab.ntensors = nt;
    mta_index(tab, chunks);
    const int rc = per_table(tab, chunks, first);
    if (rc) return rc;
  }
  return SUPA_AMD_OK;
}

template <typename T> constexpr int64_t norm_chunk() { return 2 * kNormBlock * (16 / (int64_t)sizeof(T)); }

template <typename T>
int64_t norm_ws_bytes(int32_t n, const int64_t* numel) {
  int64_t total = 0;
  const int rc = norm_tables<norm_chunk<T>()>(n, numel, [&](const MtaTable&, uint32_t chunks, int) {
    total += chunks;
    return SUPA_AMD_OK;
  });
  return rc ? -1 : total * (int64_t)sizeof(opmath_t<T>);
}

template <typename T, typename OT, int ORD>
int norm_launch(int32_t n, const void* const* x, const int64_t* numel, void* out, void* ws, hipStream_t st) {
  using A = opmath_t<T>;
  constexpr int64_t CHUNK = norm_chunk<T>();
  A* base = static_cast<A*>(ws);
  return norm_tables<CHUNK>(n, numel, [&](MtaTable& tab, uint32_t chunks, int first) -> int {
    for (int s = 0; s < tab.ntensors; ++s) {
      if (tab.numel[s] > 0 && !x[first + s]) return SUPA_AMD_EINVAL;
      tab.in[0][s] = x[first + s];
      tab.out[s] = static_cast<OT*>(out) + first + s;
    }
    if (chunks > 0) {
      // the partial kernel only sees non-empty tensors' blocks
      k_norm_partial<T, ORD, CHUNK><<<chunks, kNormBlock, 0, st>>>(tab, base);
      const int rc = launch_status();
      if (rc) return rc;
    }
    k_norm_final<A, OT, ORD><<<tab.ntensors, kNormBlock, 0, st>>>(tab, base);
    base += chunks;
    return launch_status();
  });
}


// ------------------------------------------------------ norm over rows
// linalg_vector_norm over the last dim of a contiguous [outer, inner] input,
// every order upstream's norm kernel knows: 0 (count of non-zeros), 1, 2,
// inf / -inf (largest / smallest |x|, NaN propagating) and any other p
// (sum of |x|^p, then ^(1/p)), accumulated in opmath.
constexpr int kRowOrdZero = 3, kRowOrdNegInf = 4, kRowOrdP = 5;

template <int ORD, typename A> __device__ __forceinline__ A row_norm_term(A x, A p) {
  if constexpr (ORD == kRowOrdZero) return x != A(0) ? A(1) : A(0);
  else if constexpr (ORD == kRowOrdP) return pow(fabs(x), p);
  else return norm_term<ORD>(x);
}
template <int ORD, typename A> __device__ __forceinline__ A row_norm_combine(A a, A b) {
  if constexpr (ORD == kRowOrdNegInf) return (a != a || a < b) ? a : b;
  else if constexpr (ORD == kOrdInf) return norm_combine<kOrdInf>(a, b);
  else return a + b;
}
template <int ORD, typename A> __device__ __forceinline__ A row_norm_init() {
  if constexpr (ORD == kRowOrdNegInf) return A(INFINITY);
  else return A(0);
}

// One workgroup per (row, chunk of `chunk` elements): a single wavefront for
// rows up to kNormWaveRow elements (no LDS stage), four for longer ones.
// TERM: the input holds elements (else partials of an earlier launch); PROJ:
// write the norm (else the chunk's partial, in A).
constexpr int64_t kNormWaveRow = 4096;

template <int BS, typename T, typename OT, typename A, int ORD, bool TERM, bool PROJ>
__global__ void __launch_bounds__(BS)
k_norm_rows(const T* __restrict__ in, OT* __restrict__ out, int64_t inner, int64_t chunk, uint32_t nchunks, A p) {
  __shared__ A part[BS / 64];
  const uint32_t row = blockIdx.x / nchunks, c = blockIdx.x % nchunks;
  const int64_t lo = (int64_t)c * chunk;
  const int64_t n = lo + chunk < inner ? chunk : inner - lo;
  const T* src = in + (int64_t)row * inner + lo;
  auto comb = [](A a, A b) { return row_norm_combine<ORD>(a, b); };
  A acc = fold_strided<8>(
      row_norm_init<ORD, A>(), threadIdx.x, BS, n,
      [&](int64_t i) {
        const A x = (A)to_arith(src[i]);
        if constexpr (TERM) return row_norm_term<ORD>(x, p);
        else return x;
      },
      comb);
  for (int off = 32; off > 0; off >>= 1) acc = comb(acc, __shfl_xor(acc, off, 64));
  if constexpr (BS > 64) {
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
  }
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 1; w < BS / 64; ++w) acc = comb(acc, part[w]);
    if constexpr (PROJ) {
      if constexpr (ORD == 2) acc = sqrt(acc);
      else if constexpr (ORD == kRowOrdP) acc = pow(acc, A(1) / p);
    }
    out[blockIdx.x] = from_arith<OT>(acc);
  }
}

constexpr int64_t kNormRowChunk = 16384;       // elements per workgroup in the first of two launches
constexpr int64_t kNormRowTwoPass = 65536;     // rows longer than this (with few rows) take two launches

inline int64_t norm_row_chunks(int64_t outer, int64_t inner) {
  return inner > kNormRowTwoPass && outer < 2048 ? (inner + kNormRowChunk - 1) / kNormRowChunk : 1;
}

template <typename T, typename OT, int ORD>
int norm_rows_launch(const T* in, OT* out, int64_t outer, int64_t inner, double p, void* ws, hipStream_t st) {
  using A = opmath_t<T>;
  const int64_t nch = norm_row_chunks(outer, inner);
  if (nch == 1 && inner <= kNormWaveRow) {
    k_norm_rows<64, T, OT, A, ORD, true, true><<<(unsigned)outer, 64, 0, st>>>(in, out, inner, inner, 1u, (A)p);
    return launch_status();
  }
  if (nch == 1) {
    k_norm_rows<kNormBlock, T, OT, A, ORD, true, true><<<(unsigned)outer, kNormBlock, 0, st>>>(in, out, inner, inner,
                                                                                             1u, (A)p);
    return launch_status();
  }
  A* part = static_cast<A*>(ws);
  k_norm_rows<kNormBlock, T, A, A, ORD, true, false><<<(unsigned)(outer * nch), kNormBlock, 0, st>>>(
      in, part, inner, kNormRowChunk, (uint32_t)nch, (A)p);
  const int rc = launch_status();
  if (rc) return rc;
  k_norm_rows<kNormBlock, A, OT, A, ORD, false, true><<<(unsigned)outer, kNormBlock, 0, st>>>(part, out, nch, nch, 1u, (A)p);
  return launch_status();
}

}  // namespace sa

using namespace sa;

extern "C" {

int supa_amd_foreach(int op, int form, int32_t ntensors, void* const* out, const void* const* a,
                     const void* const* b, const void* const* c, const int64_t* numel, int32_t dtype,
                     const double* scalars, double alpha, const void* scalar_ptr, void* stream) {
  if (ntensors < 0 || (ntensors > 0 && (!out || !numel))) return SUPA_AMD_EINVAL;
  if (form != kFeList && form != kFeScalars && form != kFeDev) return SUPA_AMD_EINVAL;
  const bool binary = op >= SUPA_AMD_FOREACH_ADD && op <= SUPA_AMD_FOREACH_MINIMUM;
  if (binary || op == SUPA_AMD_FOREACH_LERP) {
    if (form == kFeScalars && !scalars) return SUPA_AMD_EINVAL;
    if (form == kFeDev && (!scalar_ptr || op == SUPA_AMD_FOREACH_LERP)) return SUPA_AMD_EINVAL;
  }
  if ((op == SUPA_AMD_FOREACH_ADDCMUL || op == SUPA_AMD_FOREACH_ADDCDIV) && !scalars) return SUPA_AMD_EINVAL;
  if (ntensors == 0) return SUPA_AMD_OK;
  const FeArgs args{ntensors, out, {a, b, c}, numel, scalars, alpha, scalar_ptr};
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_mta_storage(dtype, [&](auto* tag) -> int {
    using T = std::remove_pointer_t<decltype(tag)>;
    return fe_dispatch<T>(op, form, args, st);
  });
}

int supa_amd_foreach_binary(int op, int32_t ntensors, void* const* out, void* const* a, void* const* b,
                            const int64_t* numel, int32_t dtype, double scalar, double alpha, void* stream) {
  if (ntensors < 0 || (ntensors > 0 && (!out || !a || !numel))) return SUPA_AMD_EINVAL;
  if (op != SUPA_AMD_FOREACH_ADD && op != SUPA_AMD_FOREACH_MUL) return SUPA_AMD_EINVAL;
  if (b) return supa_amd_foreach(op, kFeList, ntensors, out, a, b, nullptr, numel, dtype, nullptr, alpha, nullptr, stream);
  std::vector<double> s((size_t)ntensors, scalar);
  return supa_amd_foreach(op, kFeScalars, ntensors, out, a, nullptr, nullptr, numel, dtype, s.data(), 1.0, nullptr,
                          stream);
}

int64_t supa_amd_foreach_norm_workspace_bytes(int32_t ntensors, const int64_t* numel, int32_t dtype) {
  if (ntensors < 0 || (ntensors > 0 && !numel)) return -1;
  return with_mta_storage(dtype, [&](auto* tag) -> int64_t {
    using T = std::remove_pointer_t<decltype(tag)>;
    return norm_ws_bytes<T>(ntensors, numel);
  });
}

int supa_amd_foreach_norm(int32_t ntensors, const void* const* x, const int64_t* numel, int32_t dtype, double ord,
                          void* out, int32_t out_dtype, void* workspace, int64_t ws_bytes, void* stream) {
  if (ntensors < 0 || (ntensors > 0 && (!x || !numel || !out))) return SUPA_AMD_EINVAL;
  int o;
  if (ord == 1.0) o = 1;
  else if (ord == 2.0) o = 2;
  else if (ord == HUGE_VAL) o = kOrdInf;
  else return SUPA_AMD_EINVAL;
  if (ntensors == 0) return SUPA_AMD_OK;
  const int64_t need = supa_amd_foreach_norm_workspace_bytes(ntensors, numel, dtype);
  if (need < 0) return need == -1 ? SUPA_AMD_EINVAL : (int)need;
  if (need > 0 && (!workspace || ws_bytes < need)) return SUPA_AMD_EWORKSPACE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_mta_storage(dtype, [&](auto* tag) -> int {
    using T = std::remove_pointer_t<decltype(tag)>;
    auto go = [&](auto* otag) -> int {
      using OT = std::remove_pointer_t<decltype(otag)>;
      if (o == 1) return norm_launch<T, OT, 1>(ntensors, x, numel, out, workspace, st);
      if (o == 2) return norm_launch<T, OT, 2>(ntensors, x, numel, out, workspace, st);
      return norm_launch<T, OT, kOrdInf>(ntensors, x, numel, out, workspace, st);
    };
    if (out_dtype == dtype) return go((T*)nullptr);
    if (out_dtype == SUPA_AMD_F32) return go((float*)nullptr);
    if (out_dtype == SUPA_AMD_F64) return go((double*)nullptr);
    return SUPA_AMD_EDTYPE;
  });
}


int64_t supa_amd_norm_rows_workspace_bytes(int64_t outer, int64_t inner, int32_t dtype) {
  if (outer < 0 || inner <= 0) return -1;
  const int64_t nch = norm_row_chunks(outer, inner);
  if (nch == 1) return 0;
  if (dtype != SUPA_AMD_F32 && dtype != SUPA_AMD_BF16 && dtype != SUPA_AMD_F16 && dtype != SUPA_AMD_F64)
    return SUPA_AMD_EDTYPE;
  return outer * nch * (dtype == SUPA_AMD_F64 ? 8 : 4);  // opmath partials
}

int supa_amd_norm_rows(const void* in, int32_t dtype, void* out, int32_t out_dtype, int64_t outer, int64_t inner,
                       double ord, void* workspace, int64_t ws_bytes, void* stream) {
  if (!in || !out || outer < 0 || inner <= 0) return SUPA_AMD_EINVAL;
  if (ord != ord) return SUPA_AMD_EINVAL;
  if (outer == 0) return SUPA_AMD_OK;
  if (outer * norm_row_chunks(outer, inner) >= (int64_t(1) << 31)) return SUPA_AMD_ELAYOUT;
  const int64_t need = supa_amd_norm_rows_workspace_bytes(outer, inner, dtype);
  if (need < 0) return need == -1 ? SUPA_AMD_EINVAL : (int)need;
  if (need > 0 && (!workspace || ws_bytes < need)) return SUPA_AMD_EWORKSPACE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return with_mta_storage(dtype, [&](auto* tag) -> int {
    using T = std::remove_pointer_t<decltype(tag)>;
    auto go = [&](auto* otag) -> int {
      using OT = std::remove_pointer_t<decltype(otag)>;
      const T* x = static_cast<const T*>(in);
      OT* o = static_cast<OT*>(out);
      if (ord == 0.0) return norm_rows_launch<T, OT, kRowOrdZero>(x, o, outer, inner, ord, workspace, st);
      if (ord == 1.0) return norm_rows_launch<T, OT, 1>(x, o, outer, inner, ord, workspace, st);
      if (ord == 2.0) return norm_rows_launch<T, OT, 2>(x, o, outer, inner, ord, workspace, st);
      if (ord == HUGE_VAL) return norm_rows_launch<T, OT, kOrdInf>(x, o, outer, inner, ord, workspace, st);
      if (ord == -HUGE_VAL) return norm_rows_launch<T, OT, kRowOrdNegInf>(x, o, outer, inner, ord, workspace, st);
      return norm_rows_launch<T, OT, kRowOrdP>(x, o, outer, inner, ord, workspace, st);
    };
    if (out_dtype == dtype) return go((T*)nullptr);
    if (out_dtype == SUPA_AMD_F32) return go((float*)nullptr);
    return SUPA_AMD_EDTYPE;
  });
}

}  // extern "C"
