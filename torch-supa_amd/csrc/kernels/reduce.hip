// Full reductions: sum/mean of a tensor, and the sum/mean reductions of the
// pointwise losses fused with the loss term (one read of the inputs, no
// materialised loss tensor).
//
// Two kernels, deterministic.  Stage 1: a fixed grid of G blocks; each thread
// accumulates a strided subset of 16-byte vectors in float32 (float64 for
// float64 data), the block combines its 256 partials in a fixed tree and
// writes one partial to the workspace.  Stage 2: one block combines the G
// partials in a fixed tree, applies the scale (1 for sum, 1/n for mean) and
// stores the result.  The order of every addition depends only on n and G, so
// reruns are bit-identical.  The kernel boundary orders the two stages: a
// last-block-done counter would need a device-scope release per block, which
// on gfx950 writes back and invalidates the XCD's L2 each time and halved the
// stream rate when measured.
//
// Workspace contract: supa_amd_*_workspace_bytes() bytes of device memory
// with no required contents; calls that overlap in time on different streams
// need separate buffers.
#include <mutex>

#include "ew_launch.h"
#include "ops.h"

namespace sa {

constexpr int kRedBlocks = 1024;   // stage-1 grid (capped by the work)
constexpr int kRedBlock = 256;     // stage-1 workgroup
constexpr int kCounterBytes = 256; // reserved head of the workspace (keeps partials 256-byte aligned)

enum RedLayout { R_CONTIG = 0, R_VECND = 1, R_STRIDED = 2 };

template <int BS, typename ACC>
__device__ __forceinline__ ACC block_sum(ACC v, ACC* lds) {
  // wavefront (64 lanes) tree, then the 4 wave results in a fixed order
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) lds[wave] = v;
  __syncthreads();
  ACC r = ACC(0);
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 0; w < BS / 64; ++w) r += lds[w];
  }
  return r;  // valid in thread 0
}

// Accumulates op(...) over this thread's share of the iteration space.  BC:
// some input is broadcast (a one-element input, or stride 0 / re-read rows in
// the N-d layout); without it the loop carries no per-operand branches.
template <int BS, int LAYOUT, int VEC, bool BC, typename Op, typename C, typename CT, typename ACC, typename... S>
__device__ __forceinline__ ACC accumulate(const Op& op, const TArgs<1 + sizeof...(S)>& a, const NdGeom& g, int64_t n) {
  constexpr int N = sizeof...(S);
  ACC acc = ACC(0);
  const int64_t tid = (int64_t)blockIdx.x * BS + threadIdx.x;
  const int64_t nthreads = (int64_t)gridDim.x * BS;
  if constexpr (LAYOUT == R_CONTIG) {
    const int64_t nvec = n / VEC;
    for (int64_t v = tid; v < nvec; v += nthreads) {
      C x[VEC][N > 0 ? N : 1];
      [&]<int... I>(std::integer_sequence<int, I...>) {
        (([&] {
           using St = typename NthT<I, S...>::type;
           const St* p = static_cast<const St*>(a.p[1 + I]);
           if (BC && a.mode[1 + I]) {
             const C s = load_cvt<C, CT>(p[0]);
#pragma unroll
             for (int k = 0; k < VEC; ++k) x[k][I] = s;
           } else {
             const Vec<St, VEC> w = ld_stream(reinterpret_cast<const Vec<St, VEC>*>(p + v * VEC));
#pragma unroll
             for (int k = 0; k < VEC; ++k) x[k][I] = load_cvt<C, CT>(w.v[k]);
           }
         }()),
         ...);
      }(std::make_integer_sequence<int, N>{});
#pragma unroll
      for (int k = 0; k < VEC; ++k) acc += (ACC)op(x[k]);
    }
    const int64_t t = nvec * VEC + tid;
    if (t < n) {
      C y[N > 0 ? N : 1];
      [&]<int... I>(std::integer_sequence<int, I...>) {
        (([&] {
           using St = typename NthT<I, S...>::type;
           const St* p = static_cast<const St*>(a.p[1 + I]);
           y[I] = load_cvt<C, CT>((BC && a.mode[1 + I]) ? p[0] : p[t]);
         }()),
         ...);
      }(std::make_integer_sequence<int, N>{});
      acc += (ACC)op(y);
    }
  } else if constexpr (LAYOUT == R_VECND) {
    const uint32_t nvec = (uint32_t)(n / VEC);
    for (uint32_t v = (uint32_t)tid; v < nvec; v += (uint32_t)nthreads) {
      uint32_t q, r;
      g.div[0].divmod(v * VEC, q, r);
      int64_t off[1 + N];
#pragma unroll
      for (int k = 0; k <= N; ++k) off[k] = (int64_t)r * a.st[k][0];
      for (int d = 1; d < g.ndim; ++d) {
        uint32_t qq, rr;
        g.div[d].divmod(q, qq, rr);
        q = qq;
#pragma unroll
        for (int k = 0; k <= N; ++k) off[k] += (int64_t)rr * a.st[k][d];
      }
      C x[VEC][N > 0 ? N : 1];
      [&]<int... I>(std::integer_sequence<int, I...>) {
        (([&] {
           using St = typename NthT<I, S...>::type;
           const St* p = static_cast<const St*>(a.p[1 + I]) + off[1 + I];
           if (BC && a.st[1 + I][0] == 0) {
             const C s = load_cvt<C, CT>(p[0]);
#pragma unroll
             for (int k = 0; k < VEC; ++k) x[k][I] = s;
           } else {
             const Vec<St, VEC> w = (BC && a.mode[1 + I]) ? *reinterpret_cast<const Vec<St, VEC>*>(p)
                                                          : ld_stream(reinterpret_cast<const Vec<St, VEC>*>(p));
#pragma unroll
             for (int k = 0; k < VEC; ++k) x[k][I] = load_cvt<C, CT>(w.v[k]);
           }
         }()),
         ...);
      }(std::make_integer_sequence<int, N>{});
#pragma unroll
      for (int k = 0; k < VEC; ++k) acc += (ACC)op(x[k]);
    }
  } else {
    for (uint32_t i = (uint32_t)tid; i < (uint32_t)n; i += (uint32_t)nthreads) {
      int64_t off[1 + N];
#pragma unroll
      for (int k = 0; k <= N; ++k) off[k] = 0;
      uint32_t q = i;
      for (int d = 0; d < g.ndim; ++d) {
        uint32_t qq, rr;
        g.div[d].divmod(q, qq, rr);
        q = qq;
#pragma unroll
        for (int k = 0; k <= N; ++k) off[k] += (int64_t)rr * a.st[k][d];
      }
      C y[N > 0 ? N : 1];
      [&]<int... I>(std::integer_sequence<int, I...>) {
        (([&] {
           using St = typename NthT<I, S...>::type;
           y[I] = load_cvt<C, CT>(static_cast<const St*>(a.p[1 + I])[off[1 + I]]);
         }()),
         ...);
      }(std::make_integer_sequence<int, N>{});
      acc += (ACC)op(y);
    }
  }
  return acc;
}

template <int BS, int LAYOUT, int VEC, bool BC, typename Op, typename C, typename CT, typename ACC, typename... S>
__global__ void __launch_bounds__(BS)
k_reduce_partial(Op op, TArgs<1 + sizeof...(S)> a, NdGeom g, int64_t n, ACC* __restrict__ partial) {
  __shared__ ACC lds[BS / 64];
  ACC acc = accumulate<BS, LAYOUT, VEC, BC, Op, C, CT, ACC, S...>(op, a, g, n);
  acc = block_sum<BS, ACC>(acc, lds);
  if (threadIdx.x == 0) partial[blockIdx.x] = acc;
}

// Stage 2: partials 0..nparts-1 in a fixed order, then the fixed block tree.
template <typename ACC, typename OT>
__global__ void __launch_bounds__(kBlock)
k_reduce_final(const ACC* __restrict__ partial, int nparts, ACC scale, OT* __restrict__ out) {
  __shared__ ACC lds[kBlock / 64];
  ACC v = fold_strided<kRedBlocks / kBlock>(
      ACC(0), threadIdx.x, kBlock, nparts, [&](int64_t i) { return partial[i]; },
      [](ACC a, ACC b) { return a + b; });
  v = block_sum<kBlock, ACC>(v, lds);
  if (threadIdx.x == 0) out[0] = from_arith<OT>(v * scale);
}

template <typename Op, typename C, typename CT, typename OT, typename... S>
int launch_reduce(const Op& op, const supa_amd_ew_desc& d, const int* tin, double scale, void* ws,
                  int64_t ws_bytes, hipStream_t st) {
  constexpr int N = sizeof...(S);
  // float32 partials for the float family, float64 for double, int64 for
  // the integer sums (exact and order-free: wrapping adds modulo 2^64)
  using ACC = typename std::conditional<std::is_same<C, double>::value, double,
                                        typename std::conditional<std::is_integral<C>::value, int64_t,
                                                                  float>::type>::type;
  constexpr int VEC0 = 16 / min_size<S...>();
  constexpr int VEC = VEC0 < 1 ? 1 : VEC0;
  const int64_t n = desc_numel(&d);
  if (!ws || ws_bytes < kCounterBytes + (int64_t)kRedBlocks * (int64_t)sizeof(double)) return SUPA_AMD_EWORKSPACE;
  TArgs<1 + N> a;
  a.p[0] = d.op[0].data;
  a.mode[0] = 0;
  for (int j = 0; j < SUPA_AMD_MAX_DIMS; ++j) a.st[0][j] = 0;
  for (int i = 0; i < N; ++i) {
    const supa_amd_operand& o = d.op[tin[i]];
    a.p[1 + i] = o.data;
    a.mode[1 + i] = 0;
    for (int j = 0; j < SUPA_AMD_MAX_DIMS; ++j) a.st[1 + i][j] = j < d.ndim ? o.strides[j] : 0;
  }
  const int sizes_of[N > 0 ? N : 1] = {(int)sizeof(S)...};
  int layout = R_STRIDED;
  bool contig = d.ndim <= 1;
  if (contig && d.ndim == 1 && n > 1) {
    for (int i = 0; i < N && contig; ++i) {
      if (a.st[1 + i][0] == 0) a.mode[1 + i] = 1;
      else if (a.st[1 + i][0] != 1) contig = false;
      if (!a.mode[1 + i] && !aligned(a.p[1 + i], VEC * sizes_of[i])) contig = false;
    }
  } else if (contig) {
    for (int i = 0; i < N; ++i) a.mode[1 + i] = 1;
  }
  if (contig) layout = R_CONTIG;
  if (layout != R_CONTIG) {
    if (n >= (int64_t(1) << 31)) return SUPA_AMD_ELAYOUT;
    bool vnd = VEC > 1 && d.ndim >= 1 && (d.sizes[0] % VEC) == 0;
    for (int i = 0; i < N && vnd; ++i) {
      const int64_t s0 = a.st[1 + i][0];
      if (s0 != 0 && s0 != 1) vnd = false;
      if (s0 == 1) {
        if (!aligned(a.p[1 + i], VEC * sizes_of[i])) vnd = false;
        for (int j = 1; j < d.ndim; ++j)
          if (a.st[1 + i][j] % VEC) vnd = false;
      }
    }
    layout = vnd ? R_VECND : R_STRIDED;
    if (vnd) {
      // operands broadcast along an outer dim are re-read: keep them cached
      for (int i = 0; i < N; ++i) {
        a.mode[1 + i] = 0;
        for (int j = 1; j < d.ndim; ++j)
          if (a.st[1 + i][j] == 0 && d.sizes[j] > 1) a.mode[1 + i] = 1;
      }
    }
  }
  const NdGeom g = make_geom(d);
  const int64_t units = layout == R_STRIDED ? n : std::max<int64_t>(n / VEC, 1);
  const int64_t want = (units + 4 * kRedBlock - 1) / (4 * kRedBlock);
  const unsigned blocks = (unsigned)std::max<int64_t>(1, std::min<int64_t>(want, kRedBlocks));
  bool bc = false;
  for (int i = 0; i < N; ++i) bc = bc || a.mode[1 + i] != 0 || a.st[1 + i][0] == 0;
  ACC* partial = reinterpret_cast<ACC*>(static_cast<char*>(ws) + kCounterBytes);
  switch (layout) {
    case R_CONTIG:
      if (bc) k_reduce_partial<kRedBlock, R_CONTIG, VEC, true, Op, C, CT, ACC, S...><<<blocks, kRedBlock, 0, st>>>(op, a, g, n, partial);
      else k_reduce_partial<kRedBlock, R_CONTIG, VEC, false, Op, C, CT, ACC, S...><<<blocks, kRedBlock, 0, st>>>(op, a, g, n, partial);
      break;
    case R_VECND:
      if (bc) k_reduce_partial<kRedBlock, R_VECND, VEC, true, Op, C, CT, ACC, S...><<<blocks, kRedBlock, 0, st>>>(op, a, g, n, partial);
      else k_reduce_partial<kRedBlock, R_VECND, VEC, false, Op, C, CT, ACC, S...><<<blocks, kRedBlock, 0, st>>>(op, a, g, n, partial);
      break;
    default:
      k_reduce_partial<kRedBlock, R_STRIDED, 1, false, Op, C, CT, ACC, S...><<<blocks, kRedBlock, 0, st>>>(op, a, g, n, partial);
      break;
  }
  const int rc = launch_status();
  if (rc) return rc;
  k_reduce_final<ACC, OT><<<1, kBlock, 0, st>>>(partial, (int)blocks, static_cast<ACC>(scale),
                                                  static_cast<OT*>(a.p[0]));
  return launch_status();
}

// Same-dtype reduction dispatch (every tensor input has the common dtype; the
// output has the common dtype or, for sum/mean with a dtype argument, float32
// / float64 -- handled by the caller converting first).
template <int N, typename Op, typename C, typename T>
int reduce_same(const Op& op, const supa_amd_ew_desc& d, const int* tin, double scale, void* ws, int64_t wsb,
                hipStream_t st) {
  auto with_out = [&](auto* o) -> int {
    using OT = std::remove_pointer_t<decltype(o)>;
    if constexpr (N == 1) return launch_reduce<Op, C, T, OT, T>(op, d, tin, scale, ws, wsb, st);
    else if constexpr (N == 2) return launch_reduce<Op, C, T, OT, T, T>(op, d, tin, scale, ws, wsb, st);
    else if constexpr (N == 3) return launch_reduce<Op, C, T, OT, T, T, T>(op, d, tin, scale, ws, wsb, st);
    else return launch_reduce<Op, C, T, OT, T, T, T, T>(op, d, tin, scale, ws, wsb, st);
  };
  const int od = d.op[0].dtype;
  if constexpr (std::is_integral<C>::value) {
    // integer and bool sums are int64 (upstream's sum of integral tensors)
    return od == SUPA_AMD_I64 ? with_out((int64_t*)nullptr) : SUPA_AMD_EDTYPE;
  } else {
    if (od == d.common_dtype) return with_out((T*)nullptr);
    if (od == SUPA_AMD_F32) return with_out((float*)nullptr);
    if (od == SUPA_AMD_F64) return with_out((double*)nullptr);
    return SUPA_AMD_EDTYPE;
  }
}

template <typename Factory>
int run_reduce(const Factory& f, const supa_amd_ew_desc* d, double scale, void* ws, int64_t wsb, void* stream) {
  int rc = check_desc(d, 2, SUPA_AMD_MAX_OPERANDS);
  if (rc) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  int tin[kMaxIn];
  int nt = 0;
  for (int k = 1; k < d->noperands; ++k) {
    if (d->op[k].is_scalar) return SUPA_AMD_EINVAL;
    if (d->op[k].dtype != d->common_dtype) return SUPA_AMD_EDTYPE;
    tin[nt++] = k;
  }
  auto go = [&](auto* ctag, auto* ttag) -> int {
    using C = std::remove_pointer_t<decltype(ctag)>;
    using T = std::remove_pointer_t<decltype(ttag)>;
    // a storage-aware factory builds its op for the storage type as well,
    // so that 16-bit rounding is fixed at compile time
    auto make_op = [&]() {
      if constexpr (Factory::kStorageAware) return f.template make<C, T>();
      else return f.template make<C>();
    };
    using Op = decltype(make_op());
    const Op op = make_op();
    constexpr int A = Op::arity;
    if (nt != A) return SUPA_AMD_EINVAL;
    return reduce_same<A, Op, C, T>(op, *d, tin, scale, ws, wsb, st);
  };
  switch (d->common_dtype) {
    case SUPA_AMD_F32: return go((float*)nullptr, (float*)nullptr);
    case SUPA_AMD_BF16: return go((float*)nullptr, (bf16*)nullptr);
    case SUPA_AMD_F16: return go((float*)nullptr, (f16*)nullptr);
    case SUPA_AMD_F64: return go((double*)nullptr, (double*)nullptr);
    default: break;
  }
  if constexpr (Factory::kIntegers) {
    switch (d->common_dtype) {
      case SUPA_AMD_BOOL: return go((int64_t*)nullptr, (b8*)nullptr);
      case SUPA_AMD_U8: return go((int64_t*)nullptr, (uint8_t*)nullptr);
      case SUPA_AMD_I8: return go((int64_t*)nullptr, (int8_t*)nullptr);
      case SUPA_AMD_I16: return go((int64_t*)nullptr, (int16_t*)nullptr);
      case SUPA_AMD_I32: return go((int64_t*)nullptr, (int32_t*)nullptr);
      case SUPA_AMD_I64: return go((int64_t*)nullptr, (int64_t*)nullptr);
      default: break;
    }
  }
  return SUPA_AMD_EDTYPE;
}

// Reduction factories.  kStorageAware ones have make<C, T>() (T the storage
// type) beside the elementwise engine's make<C>() (T = void: the 16-bit
// rounding of the term is then chosen at run time from `half`).
template <typename T> constexpr int storage_half() {
  if constexpr (std::is_void<T>::value) return -1;
  else return half_of<T>();
}
struct IdentityFactory {
  static constexpr bool kIntegers = true;  // sum has integer / bool forms
  static constexpr bool kStorageAware = false;
  template <typename C> IdentityOp<C> make() const { return IdentityOp<C>{}; }
};
struct MseTermFactory {
  static constexpr bool kIntegers = false;
  static constexpr bool kStorageAware = true;
  int half;
  template <typename C, typename T = void> auto make() const { return MseTermOp<C, storage_half<T>()>{half}; }
};
struct SmoothL1TermFactory {
  static constexpr bool kIntegers = false;
  static constexpr bool kStorageAware = true;
  double beta;
  int half;
  template <typename C, typename T = void> auto make() const {
    const C b = storage_param<C>(beta, half);
    return SmoothL1TermOp<C, storage_half<T>()>{b, storage_param<C>(0.5 * static_cast<double>(b), half), half};
  }
};
template <bool PW, bool W, bool HW = false>
struct BceTermFactory {
  static constexpr bool kIntegers = false;
  static constexpr bool kStorageAware = false;
  template <typename C> BceTermOp<PW, W, C, HW> make() const { return BceTermOp<PW, W, C, HW>{}; }
  template <typename C> static constexpr bool ok() { return std::is_floating_point<C>::value; }
};
struct HuberTermFactory {
  static constexpr bool kIntegers = false;
  static constexpr bool kStorageAware = true;
  double delta;
  int half;
  template <typename C> static constexpr bool ok() { return std::is_floating_point<C>::value; }
  template <typename C, typename T = void> auto make() const {
    const C dl = storage_param<C>(delta, half);
    return HuberTermOp<C, storage_half<T>()>{dl, storage_param<C>(0.5 * static_cast<double>(dl), half), half};
  }
};
template <bool W>
struct BceProbTermFactory {
  static constexpr bool kIntegers = false;
  static constexpr bool kStorageAware = false;
  int half;
  template <typename C> static constexpr bool ok() { return std::is_floating_point<C>::value; }
  template <typename C> BceProbTermOp<W, C> make() const { return BceProbTermOp<W, C>{half}; }
};
struct MseTermEwFactory {
  static constexpr bool kIntegers = false;
  int half;
  template <typename C> static constexpr bool ok() { return std::is_floating_point<C>::value; }
  template <typename C> MseTermOp<C> make() const { return MseTermOp<C>{half}; }
};
struct SmoothL1TermEwFactory {
  static constexpr bool kIntegers = false;
  double beta;
  int half;
  template <typename C> static constexpr bool ok() { return std::is_floating_point<C>::value; }
  template <typename C> SmoothL1TermOp<C> make() const {
    const C b = storage_param<C>(beta, half);
    return SmoothL1TermOp<C>{b, storage_param<C>(0.5 * static_cast<double>(b), half), half};
  }
};

// ---------------------------------------------------------------- rows
template <typename T, typename OT, typename ACC>
__global__ void __launch_bounds__(kBlock)
k_sum_rows(const T* __restrict__ in, OT* __restrict__ out, int64_t inner, ACC scale) {
  __shared__ ACC lds[kBlock / 64];
  const T* row = in + (int64_t)blockIdx.x * inner;
  ACC acc = fold_strided<8>(
      ACC(0), threadIdx.x, kBlock, inner, [&](int64_t i) { return (ACC)to_arith(row[i]); },
      [](ACC a, ACC b) { return a + b; });
  acc = block_sum<kBlock, ACC>(acc, lds);
  if (threadIdx.x == 0) out[blockIdx.x] = from_arith<OT>(acc * scale);
}

}  // namespace sa

using namespace sa;

// ------------------------------------------------ no-allocation variant
// supa_amd_sum_noalloc's workspace: a file-scope device array of exactly the
// two-stage reduction's workspace (256 reserved bytes + one partial per
// stage-1 block), which each GPU the library runs on holds until the process
// ends.  Host code never passes `scratch` itself (on the host it is only a
// stand-in symbol): its device address comes from hipGetSymbolAddress, once
// per device with that device current, and is kept per device.
namespace {
constexpr int64_t kNoAllocScratchBytes = sa::kCounterBytes + (int64_t)sa::kRedBlocks * 8;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kNoAllocDevices = 64;
std::mutex g_noalloc_mu;
void* g_noalloc_ptr[kNoAllocDevices] = {};

// The current device's scratch address (set up on the first call on a
// device), or a hipError_t.
int noalloc_scratch(void** out) {
  int dev = 0;
  hipError_t rc = hipGetDevice(&dev);
  if (rc != hipSuccess) return (int)rc;
  if (dev < 0 || dev >= kNoAllocDevices) return SUPA_AMD_EINVAL;
  std::lock_guard<std::mutex> g(g_noalloc_mu);
  if (!g_noalloc_ptr[dev]) {
    void* ptr = nullptr;
    rc = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (rc != hipSuccess || !ptr) return rc != hipSuccess ? (int)rc : (int)hipErrorInvalidSymbol;
    g_noalloc_ptr[dev] = ptr;
  }
  *out = g_noalloc_ptr[dev];
  return SUPA_AMD_OK;
}
}  // namespace

extern "C" {

int64_t supa_amd_sum_workspace_bytes(int64_t /*numel*/) { return kCounterBytes + (int64_t)kRedBlocks * 8; }
int64_t supa_amd_loss_workspace_bytes(int64_t /*numel*/) { return kCounterBytes + (int64_t)kRedBlocks * 8; }

int supa_amd_sum(const supa_amd_ew_desc* d, double scale, void* workspace, int64_t workspace_bytes, void* stream) {
  if (!d || d->noperands != 2) return SUPA_AMD_EINVAL;
  if (desc_numel(d) == 0) return SUPA_AMD_EINVAL;  // the caller writes the empty-sum value
  return run_reduce(IdentityFactory{}, d, scale, workspace, workspace_bytes, stream);
}

int64_t supa_amd_sum_noalloc_max_workspace_bytes(void) { return kNoAllocScratchBytes; }

int supa_amd_sum_noalloc(const supa_amd_ew_desc* d, double scale, void* stream) {
  if (!d || d->noperands != 2) return SUPA_AMD_EINVAL;
  if (desc_numel(d) == 0) return SUPA_AMD_EINVAL;
  // the reduction's workspace is a fixed size; refuse anything needing more
  // than the scratch array holds
  if (supa_amd_sum_workspace_bytes(desc_numel(d)) > kNoAllocScratchBytes) return SUPA_AMD_EWORKSPACE;
  void* ws = nullptr;
  const int rc = noalloc_scratch(&ws);
  if (rc != SUPA_AMD_OK) return rc;
  return run_reduce(IdentityFactory{}, d, scale, ws, kNoAllocScratchBytes, stream);
}

int supa_amd_sum_rows(const void* in, int32_t in_dtype, void* out, int32_t out_dtype, int64_t outer, int64_t inner,
                      double scale, void* stream) {
  if (!in || !out || outer < 0 || inner <= 0 || outer >= (int64_t(1) << 31)) return SUPA_AMD_EINVAL;
  if (outer == 0) return SUPA_AMD_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto go = [&](auto* ti, auto* to) -> int {
    using T = std::remove_pointer_t<decltype(ti)>;
    using OT = std::remove_pointer_t<decltype(to)>;
    using ACC = typename std::conditional<
        std::is_integral<OT>::value, int64_t,
        typename std::conditional<std::is_same<T, double>::value || std::is_same<OT, double>::value, double,
                                  float>::type>::type;
    k_sum_rows<T, OT, ACC><<<(unsigned)outer, kBlock, 0, st>>>(static_cast<const T*>(in), static_cast<OT*>(out), inner,
                                                              (ACC)scale);
    return launch_status();
  };
  auto outsel = [&](auto* ti) -> int {
    switch (out_dtype) {
      case SUPA_AMD_F32: return go(ti, (float*)nullptr);
      case SUPA_AMD_BF16: return go(ti, (bf16*)nullptr);
      case SUPA_AMD_F16: return go(ti, (f16*)nullptr);
      case SUPA_AMD_F64: return go(ti, (double*)nullptr);
      default: return SUPA_AMD_EDTYPE;
    }
  };
  auto intsel = [&](auto* ti) -> int {
    return out_dtype == SUPA_AMD_I64 ? go(ti, (int64_t*)nullptr) : SUPA_AMD_EDTYPE;
  };
  switch (in_dtype) {
    case SUPA_AMD_F32: return outsel((float*)nullptr);
    case SUPA_AMD_BF16: return outsel((bf16*)nullptr);
    case SUPA_AMD_F16: return outsel((f16*)nullptr);
    case SUPA_AMD_F64: return outsel((double*)nullptr);
    case SUPA_AMD_BOOL: return intsel((b8*)nullptr);
    case SUPA_AMD_U8: return intsel((uint8_t*)nullptr);
    case SUPA_AMD_I8: return intsel((int8_t*)nullptr);
    case SUPA_AMD_I16: return intsel((int16_t*)nullptr);
    case SUPA_AMD_I32: return intsel((int32_t*)nullptr);
    case SUPA_AMD_I64: return intsel((int64_t*)nullptr);
    default: return SUPA_AMD_EDTYPE;
  }
}

int supa_amd_loss_forward(const supa_amd_ew_desc* d, int loss, int reduction, double beta, int has_pos_weight,
                          int has_weight, void* out_scalar, void* workspace, int64_t workspace_bytes, void* stream) {
  if (!d) return SUPA_AMD_EINVAL;
  if (loss != SUPA_AMD_LOSS_BCE_LOGITS && has_pos_weight) return SUPA_AMD_EINVAL;
  if (loss != SUPA_AMD_LOSS_BCE_LOGITS && loss != SUPA_AMD_LOSS_BCE && has_weight) return SUPA_AMD_EINVAL;
  if (reduction == SUPA_AMD_REDUCTION_NONE) {
    switch (loss) {
      case SUPA_AMD_LOSS_HUBER: return run_ew(HuberTermFactory{beta, half_code(d)}, d, stream, 3);
      case SUPA_AMD_LOSS_BCE:
        return has_weight ? run_ew(BceProbTermFactory<true>{half_code(d)}, d, stream, 4)
                          : run_ew(BceProbTermFactory<false>{half_code(d)}, d, stream, 3);
      case SUPA_AMD_LOSS_MSE: return run_ew(MseTermEwFactory{half_code(d)}, d, stream, 3);
      case SUPA_AMD_LOSS_SMOOTH_L1: return run_ew(SmoothL1TermEwFactory{beta, half_code(d)}, d, stream, 3);
      case SUPA_AMD_LOSS_BCE_LOGITS:
        if (has_pos_weight && has_weight) return run_ew(BceTermFactory<true, true>{}, d, stream, 5);
        if (has_pos_weight) return run_ew(BceTermFactory<true, false>{}, d, stream, 4);
        if (has_weight) return run_ew(BceTermFactory<false, true>{}, d, stream, 4);
        return run_ew(BceTermFactory<false, false>{}, d, stream, 3);
      default: return SUPA_AMD_EINVAL;
    }
  }
  if (reduction != SUPA_AMD_REDUCTION_MEAN && reduction != SUPA_AMD_REDUCTION_SUM) return SUPA_AMD_EINVAL;
  if (!out_scalar) return SUPA_AMD_EINVAL;
  const int64_t n = desc_numel(d);
  if (n == 0) return SUPA_AMD_EINVAL;  // the caller writes the empty-reduction value
  const double scale = reduction == SUPA_AMD_REDUCTION_MEAN ? 1.0 / (double)n : 1.0;
  supa_amd_ew_desc e = *d;
  e.op[0].data = out_scalar;
  switch (loss) {
    case SUPA_AMD_LOSS_HUBER:
      return run_reduce(HuberTermFactory{beta, half_code(d)}, &e, scale, workspace, workspace_bytes, stream);
    case SUPA_AMD_LOSS_BCE:
      return has_weight
                 ? run_reduce(BceProbTermFactory<true>{half_code(d)}, &e, scale, workspace, workspace_bytes, stream)
                 : run_reduce(BceProbTermFactory<false>{half_code(d)}, &e, scale, workspace, workspace_bytes, stream);
    case SUPA_AMD_LOSS_MSE:
      return run_reduce(MseTermFactory{half_code(d)}, &e, scale, workspace, workspace_bytes, stream);
    case SUPA_AMD_LOSS_SMOOTH_L1:
      return run_reduce(SmoothL1TermFactory{beta, half_code(d)}, &e, scale, workspace, workspace_bytes, stream);
    case SUPA_AMD_LOSS_BCE_LOGITS:
      if (has_pos_weight && has_weight)
        return run_reduce(BceTermFactory<true, true, true>{}, &e, scale, workspace, workspace_bytes, stream);
      if (has_pos_weight)
        return run_reduce(BceTermFactory<true, false, true>{}, &e, scale, workspace, workspace_bytes, stream);
      if (has_weight)
        return run_reduce(BceTermFactory<false, true, true>{}, &e, scale, workspace, workspace_bytes, stream);
      return run_reduce(BceTermFactory<false, false, true>{}, &e, scale, workspace, workspace_bytes, stream);
    default: return SUPA_AMD_EINVAL;
  }
}

}  // extern "C"
