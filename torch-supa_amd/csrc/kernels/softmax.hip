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
// statistics is the hardware base-2 exponential of (x - max) * log2 e: the
// row maximum's term is exactly 1, as upstream's exp(x - max) makes it (a
// pre-scaled x * log2 e - max * log2 e leaves max's term 1 +- 2^-18 at
// |max| near 60, and a row with one dominant logit then gets a log-probability
// of -1.7e-6 where upstream gives 0); the row results are rounded to bf16/f16
// (or kept in f32) exactly once.
//
// Split rows (rows of 2 to 32 parts of 2048 or 2560 vectors): K workgroups
// of 512 threads share a row, exchanging row partials through a small
// per-stream buffer, so the same single pass runs with four parts per CU
// (the section below).
//
// Fallback (any cols, any alignment): one 256-thread workgroup per row,
// online max/sum in a first pass over memory, the output in a second pass.
//
// Replaces _log_softmax.out (NF:3752), _log_softmax_backward_data.out
// (NF:3763), _softmax.out and _softmax_backward_data.out, upstream SoftMax.cu /
// PersistentSoftmax.cuh in the reference's operator library.  softmax's
// epilogue is exp(x - max) * (1 / sum) and its gradient y (g - sum(g y)).
#include <cstdlib>
#include <map>
#include <mutex>

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

// s = sum of exp(x - m) rescaled to a maximum M >= m: s e^(m - M) (an all
// -inf M leaves s, which is then 0; a NaN s stays NaN).
__device__ __forceinline__ float lse_rescale(float s, float m, float M) {
  return M != -__builtin_inff() ? s * __builtin_amdgcn_exp2f((m - M) * kLog2e) : s;
}

// (max, sum of exp) pairs of `width` lanes (a power of two; lanes w apart in
// the XOR pattern hold the other pairs) combined: a max butterfly, one
// rescale per lane to that max, and a sum butterfly -- one exponential per
// lane where pairwise (m, s) combining takes two per step.  Every butterfly
// step is symmetric in its operands, so every lane ends with the same value.
template <int WIDTH>
__device__ __forceinline__ void lanes_lse(float& m, float& s) {
  float M = m;
#pragma unroll
  for (int off = WIDTH / 2; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
  s = lse_rescale(s, m, M);
#pragma unroll
  for (int off = WIDTH / 2; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
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
    const float mb = m == -__builtin_inff() ? 0.0f : m;  // all -inf: keep exp args finite
    opaque<VPT>(x);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      if (j < full || tid + j * kRowBlock < nvec) {
#pragma unroll
        for (int k = 0; k < V; ++k) s += __builtin_amdgcn_exp2f((elem_f<TI>(x[j], k) - mb) * kLog2e);
      }
    }
    lanes_lse<64>(m, s);
    __syncthreads();  // the previous row's readers are done with the slots
    if (lane == 0) {
      lds_m[wave] = m;
      lds_s[wave] = s;
    }
    __syncthreads();
    float M = lds_m[lane & 15], S = lds_s[lane & 15];
    lanes_lse<NW>(M, S);
    // log: (x - M) - log S;  softmax: 2^(x log2e - M log2e) / S with the
    // scaled max of the sum (an all -inf row gives 0 * inf = NaN, as upstream)
    const float logsum = LOG ? sa_logf(S) : 0.0f;
    const float inv = LOG ? 0.0f : 1.0f / S;
    const float Mb = M == -__builtin_inff() ? 0.0f : M;
    opaque<VPT>(x);
    Vec<TO, V>* dst = reinterpret_cast<Vec<TO, V>*>(out + row * cols);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      if (j < full || tid + j * kRowBlock < nvec) {
        float f[V];
#pragma unroll
        for (int k = 0; k < V; ++k) {
          if constexpr (LOG) f[k] = (elem_f<TI>(x[j], k) - M) - logsum;
          else f[k] = __builtin_amdgcn_exp2f((elem_f<TI>(x[j], k) - Mb) * kLog2e) * inv;
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

// ------------------------------------------------------- split rows
// Rows of 2 to 32 parts (split_parts below says which) are split over K
// workgroups of 512 threads, one part each: the backward's parts are at most
// 2048 16-byte vectors (4 per thread, 32 KiB of grad and of output), the
// forward's 2560 (5 per thread, 40 KiB), and a row is spread evenly over its
// K parts (split_part_len below).  Four such workgroups share a CU, so one part's statistics and
// stores overlap other parts' loads; a whole row per 1024-thread workgroup
// leaves a CU with one row, whose stores never overlap the next row's loads.
// On c3's rows (bf16 [8192, 128256]) the backward ran 79.9-80.0 % of the HBM
// roofline against 75.5-76.3 % with 1024-thread parts of 4096 vectors and
// 73.2-73.6 % with a whole row per workgroup, the forward 75.3-75.6 %
// against 69.3-69.7 % and 71.0-71.3 % (parts of 2048 / 2304 / 2688 vectors,
// 256-768 threads: 59-76 %).  Workgroup b takes part b % K of row b / K.  Each
// part publishes its row partial -- (max, sum of exp) forward, sum of grad
// backward -- to slots[row * K + part] with a device-scope atomic store, then
// waits for the row's other parts by polling their slots (device-scope loads,
// a short s_sleep between polls), and every part folds the K partials in slot
// order, so the K parts of a row use one bit-identical total.
//
// A part that is still missing after spin_limit polls (a peer not yet
// resident) is computed by the waiting workgroup itself: it loads that part
// with the same thread layout and reduces it in the same order, so the value
// is bit-identical to the one the peer publishes, and no wait depends on
// another workgroup being scheduled.  The inputs must not overlap the output
// for this (the host checks it).
//
// Slots are 64-bit; 0 marks an empty slot (kSlotTag below).  done[row]
// counts the parts that have read the row's slots; the last one resets the
// row's slots and done[row] to 0, so a buffer is clean after every launch.
// A buffer belongs to one (device, stream) until the process ends; launches
// on one stream are ordered, so they never share it (a stream destroyed with
// split work still queued, whose handle a new stream then receives, would
// share it with that work).
constexpr int kSplitBlock = 512;
constexpr int kSplitNW = kSplitBlock / 64;
constexpr int kFwdNV = 5, kBwdNV = 4;  // vectors per thread of a forward / backward part
constexpr int kSplitMaxK = 32;
constexpr int64_t kSplitSlots = int64_t(1) << 16;  // row parts per launch (c3's 8192 rows x 8 parts: one)
// An empty slot holds 0; a partial v is published as v ^ kSlotTag, whose high
// word is never 0 (a forward partial's high word is its sum, a non-negative
// float or the canonical NaN, below 0x80000000; a backward partial's is 0).
constexpr uint64_t kSlotTag = 0xFFFFFFFF00000000ull;
constexpr uint32_t kSplitSpinDefault = 1u << 16;
// Slot buffers per device (in the library's own device memory, 6 MiB a
// device): streams past the 8th of a device that reach a split call take the
// one-row or streaming kernels instead.
constexpr int kSplitBuffers = 8;

__device__ __forceinline__ void slot_store(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void slot_publish(uint64_t* p, uint64_t v) { slot_store(p, v ^ kSlotTag); }
__device__ __forceinline__ uint64_t slot_load(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Polls the row's K slots (wave 0; lane q < K reads slot q) for at most
// spin_limit rounds; stores every published partial to part_w[q] and returns
// the bit mask of parts still missing (same value in every thread).
__device__ __forceinline__ uint32_t split_wait(const uint64_t* rs, int K, uint32_t spin_limit, uint64_t* part_w,
                                               uint32_t* lds_missing) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (wave == 0) {
    uint64_t v = 0;
    if (lane < K) {
      v = slot_load(rs + lane);
      for (uint32_t n = 0; v == 0 && n < spin_limit; ++n) {
        __builtin_amdgcn_s_sleep(8);
        v = slot_load(rs + lane);
      }
      part_w[lane] = v ^ kSlotTag;
    }
    const uint64_t miss = __ballot(lane < K && v == 0);
    if (lane == 0) *lds_missing = (uint32_t)miss;  // K <= 32
  }
  __syncthreads();
  return *lds_missing;
}

// After every part of the row has read the slots, the last one clears them.
// A part's own publish is complete before its increment: thread 0 stores it
// and then waits on its own slot loads in split_wait, and on gfx9 the vector
// memory counter that wait drains covers stores too, so no slot is published
// after the last part's clear.
__device__ __forceinline__ void split_release(uint64_t* rs, uint32_t* done_row, int K) {
  if (threadIdx.x == 0) {
    const uint32_t d = __hip_atomic_fetch_add(done_row, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (d == (uint32_t)K - 1) {
      for (int q = 0; q < K; ++q) slot_store(rs + q, 0);
      __hip_atomic_store(done_row, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// A whole part loads without per-vector guards (a uniform branch), so its
// loads are not split by divergent ones; a part that fills all but its
// threads' last vector guards only that one.  `end` is one past the part's
// last vector.
template <int NV>
__device__ __forceinline__ void split_load(uint4 (&x)[NV], const uint4* src, int base, int end) {
  const int tid = threadIdx.x;
  const int nvec = end;
  if (base + kSplitBlock * NV <= nvec) {
#pragma unroll
    for (int j = 0; j < NV; ++j) x[j] = ld_stream(src + base + tid + j * kSplitBlock);
  } else if (base + kSplitBlock * (NV - 1) <= nvec) {
#pragma unroll
    for (int j = 0; j < NV - 1; ++j) x[j] = ld_stream(src + base + tid + j * kSplitBlock);
    if (base + tid + (NV - 1) * kSplitBlock < nvec) x[NV - 1] = ld_stream(src + base + tid + (NV - 1) * kSplitBlock);
  } else {
#pragma unroll
    for (int j = 0; j < NV; ++j)
      if (base + tid + j * kSplitBlock < nvec) x[j] = ld_stream(src + base + tid + j * kSplitBlock);
  }
}

// The kSplitNW wavefront values of a workgroup, combined over 16 lanes (lane
// l reads wavefront l % 16, or the identity past kSplitNW).
__device__ __forceinline__ void block_lse(float& M, float& S, const float* lds_m, const float* lds_s) {
  const int i = threadIdx.x & 15;
  M = i < kSplitNW ? lds_m[i] : -__builtin_inff();
  S = i < kSplitNW ? lds_s[i] : 0.0f;
  lanes_lse<16>(M, S);
}
__device__ __forceinline__ float block_sum(const float* lds) {
  const int i = threadIdx.x & 15;
  float S = i < kSplitNW ? lds[i] : 0.0f;
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) S += __shfl_xor(S, off, 64);
  return S;
}

// Per-thread (max, sum of exp(x - max)) over the thread's vectors of a part.
// The forward keeps its per-vector guards on whole parts too: a specialization
// without them took 62 VGPRs against 57 and ran at 71.1-71.9 % of the HBM
// roofline against 73.2-74.7 % on c3's rows.
template <typename TI, int NV>
__device__ __forceinline__ void thread_lse(uint4 (&x)[NV], int base, int nvec, float& m, float& s) {
  constexpr int V = VecOf<TI>::V;
  const int tid = threadIdx.x;
  m = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < NV; ++j)
    if (base + tid + j * kSplitBlock < nvec) {
#pragma unroll
      for (int k = 0; k < V; ++k) m = fmaxf(m, elem_f<TI>(x[j], k));
    }
  const float mb = m == -__builtin_inff() ? 0.0f : m;
  opaque<NV>(x);
  s = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j)
    if (base + tid + j * kSplitBlock < nvec) {
#pragma unroll
      for (int k = 0; k < V; ++k) s += __builtin_amdgcn_exp2f((elem_f<TI>(x[j], k) - mb) * kLog2e);
    }
}

// (max, sum of exp(x - max)) of one part, the same in every thread; the
// sum's NaN is canonical.
template <typename TI, int NV>
__device__ __forceinline__ uint64_t part_lse(uint4 (&x)[NV], int base, int nvec, float* lds_m, float* lds_s) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float m, s;
  thread_lse<TI, NV>(x, base, nvec, m, s);
  lanes_lse<64>(m, s);
  __syncthreads();
  if (lane == 0) {
    lds_m[wave] = m;
    lds_s[wave] = s;
  }
  __syncthreads();
  float M, S;
  block_lse(M, S, lds_m, lds_s);
  const uint32_t sb = S != S ? 0x7fc00000u : __float_as_uint(S);
  return ((uint64_t)sb << 32) | __float_as_uint(M);
}

template <typename TI, typename TO, bool LOG>
__device__ __forceinline__ void fwd_split_out(const uint4 (&x)[kFwdNV], Vec<TO, VecOf<TI>::V>* dst, int base,
                                              int nvec, float M, float logsum, float Mb, float inv) {
  constexpr int V = VecOf<TI>::V;
#pragma unroll
  for (int j = 0; j < kFwdNV; ++j) {
    const int v = base + (int)threadIdx.x + j * kSplitBlock;
    if (v < nvec) {
      float f[V];
#pragma unroll
      for (int k = 0; k < V; ++k) {
        if constexpr (LOG) f[k] = (elem_f<TI>(x[j], k) - M) - logsum;
        else f[k] = __builtin_amdgcn_exp2f((elem_f<TI>(x[j], k) - Mb) * kLog2e) * inv;
      }
      store_row_vec<TO, V>(dst, v, f);
    }
  }
}

template <typename TI, typename TO, bool LOG>
__global__ void __launch_bounds__(kSplitBlock, 8)
k_lsm_fwd_split(const TI* __restrict__ in, TO* __restrict__ out, int64_t cols, int K, int plen,
                uint64_t* __restrict__ slots, uint32_t* __restrict__ done, uint32_t spin_limit) {
  constexpr int V = VecOf<TI>::V;
  __shared__ float lds_m[kSplitNW];
  __shared__ float lds_s[kSplitNW];
  __shared__ uint64_t part_w[kSplitMaxK];
  __shared__ uint32_t lds_missing;
  const int row = (int)(blockIdx.x / (unsigned)K);
  const int part = (int)(blockIdx.x - (unsigned)row * (unsigned)K);
  const int nvec = (int)(cols / V);
  const int base = part * plen;
  const int end = min(base + plen, nvec);
  const uint4* src = reinterpret_cast<const uint4*>(in + (int64_t)row * cols);
  uint4 x[kFwdNV];
  split_load<kFwdNV>(x, src, base, end);
  const uint64_t mine = part_lse<TI, kFwdNV>(x, base, end, lds_m, lds_s);
  opaque<kFwdNV>(x);
  uint64_t* rs = slots + (int64_t)row * K;
  if (threadIdx.x == 0) slot_publish(rs + part, mine);
  uint32_t miss = split_wait(rs, K, spin_limit, part_w, &lds_missing);
  split_release(rs, done + row, K);
  if (miss) {  // uniform; the own part is loaded again afterwards, so the fallback reuses its registers
    do {
      const int q = __builtin_ctz(miss);
      miss &= miss - 1;
      const int qb = q * plen, qe = min(qb + plen, nvec);
      split_load<kFwdNV>(x, src, qb, qe);
      const uint64_t w = part_lse<TI, kFwdNV>(x, qb, qe, lds_m, lds_s);
      if (threadIdx.x == 0) part_w[q] = w;
    } while (miss);
    split_load<kFwdNV>(x, src, base, end);
  }
  __syncthreads();
  // the row's (max, sum) from the K part pairs, in part order: the max, then
  // each part's sum rescaled to it (K exponentials)
  float M = __uint_as_float((uint32_t)part_w[0]);
  for (int q = 1; q < K; ++q) M = fmaxf(M, __uint_as_float((uint32_t)part_w[q]));
  float S = 0.0f;
  for (int q = 0; q < K; ++q)
    S += lse_rescale(__uint_as_float((uint32_t)(part_w[q] >> 32)), __uint_as_float((uint32_t)part_w[q]), M);
  const float logsum = LOG ? sa_logf(S) : 0.0f;
  const float inv = LOG ? 0.0f : 1.0f / S;
  const float Mb = M == -__builtin_inff() ? 0.0f : M;
  opaque<kFwdNV>(x);
  Vec<TO, V>* dst = reinterpret_cast<Vec<TO, V>*>(out + (int64_t)row * cols);
  fwd_split_out<TI, TO, LOG>(x, dst, base, end, M, logsum, Mb, inv);
}

template <typename TG, bool WHOLE>
__device__ __forceinline__ float thread_sum(const uint4 (&g)[kBwdNV], int base, int nvec) {
  constexpr int V = VecOf<TG>::V;
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < kBwdNV; ++j)
    if (WHOLE || base + (int)threadIdx.x + j * kSplitBlock < nvec) {
#pragma unroll
      for (int k = 0; k < V; ++k) s += elem_f<TG>(g[j], k);
    }
  return s;
}

// Sum of one part of grad, the same in every thread.
template <typename TG>
__device__ __forceinline__ uint64_t part_sum(uint4 (&g)[kBwdNV], int base, int nvec, float* lds) {
  float s = base + kSplitBlock * kBwdNV <= nvec ? thread_sum<TG, true>(g, base, nvec)
                                                : thread_sum<TG, false>(g, base, nvec);
  s = wave_sum(s);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = s;
  __syncthreads();
  return (uint64_t)__float_as_uint(block_sum(lds));
}

template <typename TG, typename TO, bool WHOLE>
__device__ __forceinline__ void bwd_split_out(const uint4 (&gv)[kBwdNV], const uint4 (&yv)[kBwdNV],
                                              Vec<TO, VecOf<TG>::V>* dst, int base, int nvec, float S) {
  constexpr int V = VecOf<TG>::V;
#pragma unroll
  for (int j = 0; j < kBwdNV; ++j) {
    const int v = base + (int)threadIdx.x + j * kSplitBlock;
    if (WHOLE || v < nvec) {
      float f[V];
#pragma unroll
      for (int k = 0; k < V; ++k)
        f[k] = fmaf(-__builtin_amdgcn_exp2f(elem_f<TG>(yv[j], k) * kLog2e), S, elem_f<TG>(gv[j], k));
      store_row_vec<TO, V>(dst, v, f);
    }
  }
}

template <typename TG, typename TO>
__global__ void __launch_bounds__(kSplitBlock, 8)
k_lsm_bwd_split(const TG* __restrict__ grad, const TG* __restrict__ outp, TO* __restrict__ gin, int64_t cols, int K,
                int plen, uint64_t* __restrict__ slots, uint32_t* __restrict__ done, uint32_t spin_limit) {
  constexpr int V = VecOf<TG>::V;
  __shared__ float lds[kSplitNW];
  __shared__ uint64_t part_w[kSplitMaxK];
  __shared__ uint32_t lds_missing;
  const int row = (int)(blockIdx.x / (unsigned)K);
  const int part = (int)(blockIdx.x - (unsigned)row * (unsigned)K);
  const int nvec = (int)(cols / V);
  const int base = part * plen;
  const int end = min(base + plen, nvec);
  const uint4* g = reinterpret_cast<const uint4*>(grad + (int64_t)row * cols);
  const uint4* y = reinterpret_cast<const uint4*>(outp + (int64_t)row * cols);
  uint4 gv[kBwdNV], yv[kBwdNV];
  split_load<kBwdNV>(gv, g, base, end);
  split_load<kBwdNV>(yv, y, base, end);
  // every load of the part in flight before the sum: float32 parts, whose
  // sum is short, otherwise had it scheduled between the loads (75.2 ->
  // 76.3 % on [8192, 64128], 72.8 -> 75.3 % on [16384, 28672]; bf16 rows
  // unchanged)
  opaque<kBwdNV>(gv);
  opaque<kBwdNV>(yv);
  const uint64_t mine = part_sum<TG>(gv, base, end, lds);
  opaque<kBwdNV>(gv);
  uint64_t* rs = slots + (int64_t)row * K;
  if (threadIdx.x == 0) slot_publish(rs + part, mine);
  uint32_t miss = split_wait(rs, K, spin_limit, part_w, &lds_missing);
  split_release(rs, done + row, K);
  if (miss) {  // uniform; the own part is loaded again afterwards, so the fallback reuses its registers
    do {
      const int q = __builtin_ctz(miss);
      miss &= miss - 1;
      const int qb = q * plen, qe = min(qb + plen, nvec);
      split_load<kBwdNV>(gv, g, qb, qe);
      const uint64_t w = part_sum<TG>(gv, qb, qe, lds);
      if (threadIdx.x == 0) part_w[q] = w;
    } while (miss);
    split_load<kBwdNV>(gv, g, base, end);
  }
  __syncthreads();
  float S = __uint_as_float((uint32_t)part_w[0]);
  for (int q = 1; q < K; ++q) S += __uint_as_float((uint32_t)part_w[q]);
  opaque<kBwdNV>(gv);
  opaque<kBwdNV>(yv);
  Vec<TO, V>* dst = reinterpret_cast<Vec<TO, V>*>(gin + (int64_t)row * cols);
  if (base + kSplitBlock * kBwdNV <= end) bwd_split_out<TG, TO, true>(gv, yv, dst, base, end, S);
  else bwd_split_out<TG, TO, false>(gv, yv, dst, base, end, S);
}

__global__ void __launch_bounds__(kBlock) k_split_init(uint64_t* slots, uint32_t* done, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i < n) {
    slots[i] = 0;
    done[i] = 0u;
  }
}

// The slot buffers live in the library's own device memory (a copy on every
// device), so the entry points allocate nothing.  Host code reaches them only
// through the addresses hipGetSymbolAddress gives on each device.
static __device__ __align__(256) uint64_t g_split_slots[kSplitBuffers * kSplitSlots];
static __device__ __align__(256) uint32_t g_split_done[kSplitBuffers * kSplitSlots];

struct SplitScratch {
  uint64_t* slots = nullptr;
  uint32_t* done = nullptr;
};

// The split kernels' buffer for (current device, st): one of the device's
// kSplitBuffers, given to the stream on its first split call (and cleared on
// it then) and kept; false when the split path is switched off
// (SUPA_AMD_ROW_SPLIT=0), the stream is capturing a graph, or the device has
// given out every buffer -- the caller then takes the one-row kernels.
inline bool split_scratch(hipStream_t st, SplitScratch& out, uint32_t& spin_limit) {
  const char* e = std::getenv("SUPA_AMD_ROW_SPLIT");
  if (e && e[0] == '0') return false;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return false;
  const char* sp = std::getenv("SUPA_AMD_ROW_SPLIT_SPIN");
  spin_limit = sp ? (uint32_t)std::strtoul(sp, nullptr, 10) : kSplitSpinDefault;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return false;
  static std::mutex mu;
  static std::map<std::pair<int, hipStream_t>, SplitScratch> bufs;
  static std::map<int, std::pair<SplitScratch, int>> base;  // device -> (symbol addresses, buffers given out)
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_pair(dev, st);
  auto it = bufs.find(key);
  if (it != bufs.end()) {
    out = it->second;
    return true;
  }
  auto bt = base.find(dev);
  if (bt == base.end()) {
    SplitScratch a;
    void* ps = nullptr;
    void* pd = nullptr;
    if (hipGetSymbolAddress(&ps, HIP_SYMBOL(g_split_slots)) != hipSuccess ||
        hipGetSymbolAddress(&pd, HIP_SYMBOL(g_split_done)) != hipSuccess) {
      (void)hipGetLastError();
      return false;
    }
    a.slots = static_cast<uint64_t*>(ps);
    a.done = static_cast<uint32_t*>(pd);
    bt = base.emplace(dev, std::make_pair(a, 0)).first;
  }
  if (bt->second.second >= kSplitBuffers) return false;
  const int idx = bt->second.second;
  SplitScratch b;
  b.slots = bt->second.first.slots + (int64_t)idx * kSplitSlots;
  b.done = bt->second.first.done + (int64_t)idx * kSplitSlots;
  k_split_init<<<(unsigned)(kSplitSlots / kBlock), kBlock, 0, st>>>(b.slots, b.done, kSplitSlots);
  if (hipGetLastError() != hipSuccess) return false;
  ++bt->second.second;
  bufs.emplace(key, b);
  out = b;
  return true;
}

// Parts per row for the split kernels (at most `part` vectors each), 0 when
// the row takes another kernel: 2 to kSplitMaxK parts, inputs that do not
// overlap the output.
inline int split_parts(int64_t nvec, int part, const void* a, const void* b, int64_t a_bytes, const void* o,
                       int64_t o_bytes) {
  const int64_t K = (nvec + part - 1) / part;
  if (K < 2 || K > kSplitMaxK) return 0;
  auto overlap = [](const void* x, int64_t xb, const void* y, int64_t yb) {
    const uintptr_t x0 = reinterpret_cast<uintptr_t>(x), y0 = reinterpret_cast<uintptr_t>(y);
    return x0 < y0 + (uintptr_t)yb && y0 < x0 + (uintptr_t)xb;
  };
  if (overlap(a, a_bytes, o, o_bytes) || (b && overlap(b, a_bytes, o, o_bytes))) return 0;
  return (int)K;
}

// Vectors per part when a row of nvec vectors is split in K parts of at most
// `part`: the row spread evenly, rounded up to whole wavefronts (a part's
// guards are then uniform in every wavefront but the last part's), or, from
// `whole_from` parts on, full parts and a short last one (the backward's
// whole parts run unguarded loops).  Measured on MI355X, % of the HBM
// roofline, even parts / full parts and a short last / one-row kernel:
// forward bf16 [8192, 128256] (7 parts) 77.6 / 76.7 / 71.8, [16384, 65536]
// (4) 79.0 / 73.5 / 73.1, [16384, 50304] (3) 78.8 / 77.9 / 70.2; backward
// bf16 [16384, 50304] (4) 79.8 / 74.9 / 75.3, [2048, 57344] (4) 78.3 /
// 76.3 / 73.6, float32 [5120, 50304] (7) 68.4 / 71.2 / 72.5 (bf16 rows of
// those 12576 vectors 74.6 / 76.0 / 74.0).
inline int split_part_len(int64_t nvec, int K, int part, int whole_from) {
  if (K >= whole_from) return part;
  return (int)(((nvec + K - 1) / K + 63) / 64 * 64);
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
      const bool vec_ok = (cols % V) == 0 && aligned(in, 16) && aligned(out, V * sizeof(TO));
      const int K = vec_ok ? split_parts(cols / V, kSplitBlock * kFwdNV, in, nullptr,
                                         rows * cols * (int64_t)sizeof(TI), out, rows * cols * (int64_t)sizeof(TO))
                           : 0;
      SplitScratch sb;
      uint32_t spin = 0;
      if (K > 0 && split_scratch(st, sb, spin)) {
        const int plen = split_part_len(cols / V, K, kSplitBlock * kFwdNV, kSplitMaxK + 1);
        const int64_t chunk = kSplitSlots / K;
        for (int64_t r0 = 0; r0 < rows; r0 += chunk) {
          const int64_t nr = std::min(chunk, rows - r0);
          k_lsm_fwd_split<TI, TO, LOG><<<(unsigned)(nr * K), kSplitBlock, 0, st>>>(
              static_cast<const TI*>(in) + r0 * cols, static_cast<TO*>(out) + r0 * cols, cols, K, plen, sb.slots,
              sb.done, spin);
        }
        return launch_status();
      }
      const bool reg_ok = vec_ok && (cols / V) <= 16 * kRowBlock;
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
      const bool vec_ok = (cols % V) == 0 && aligned(grad, 16) && aligned(output, 16) && aligned(grad_in, V * sizeof(TO));
      const TG* pg = static_cast<const TG*>(grad);
      const TG* py = static_cast<const TG*>(output);
      TO* po = static_cast<TO*>(grad_in);
      const int K = vec_ok ? split_parts(cols / V, kSplitBlock * kBwdNV, grad, output,
                                         rows * cols * (int64_t)sizeof(TG), grad_in, rows * cols * (int64_t)sizeof(TO))
                           : 0;
      SplitScratch sb;
      uint32_t spin = 0;
      if (K > 0 && split_scratch(st, sb, spin)) {
        const int plen = split_part_len(cols / V, K, kSplitBlock * kBwdNV, 6);
        const int64_t chunk = kSplitSlots / K;
        for (int64_t r0 = 0; r0 < rows; r0 += chunk) {
          const int64_t nr = std::min(chunk, rows - r0);
          k_lsm_bwd_split<TG, TO><<<(unsigned)(nr * K), kSplitBlock, 0, st>>>(pg + r0 * cols, py + r0 * cols,
                                                                           po + r0 * cols, cols, K, plen, sb.slots,
                                                                           sb.done, spin);
        }
        return launch_status();
      }
      const bool reg_ok = vec_ok && (cols / V) <= 16 * kRowBlock;
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
