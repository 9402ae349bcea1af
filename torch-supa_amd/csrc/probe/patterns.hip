// Access-pattern ceilings of one MI355X for the shapes this library's
// kernels use: trivial kernels (copy, add, fill, a register-resident row copy,
// a 4-read / 3-write stream) with the same launch shapes and the same
// nontemporal 16-byte accesses, timed with HIP events, plus the binary32 and
// binary64 FMA issue rates.  The measured kernels' fractions of the 8 TB/s
// roofline are read against these.  Built by build.py as
// torch_supa/supa_patterns; `python3 bench.py --patterns` runs it.
//
// Prints one markdown table row per case.  Every access is in bounds of its
// allocation and no kernel waits on another workgroup.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <vector>

#include "dtypes.h"

using sa::ld_stream;
using sa::st_stream;

#define CHECK(x)                                                                             \
  do {                                                                                       \
    hipError_t e_ = (x);                                                                     \
    if (e_ != hipSuccess) {                                                                  \
      fprintf(stderr, "patterns: %s failed: %s (line %d)\n", #x, hipGetErrorString(e_), __LINE__); \
      exit(1);                                                                               \
    }                                                                                        \
  } while (0)

constexpr double kPeakGBs = 8000.0;

// ------------------------------------------------------------- kernels
// U vectors per thread, vector v = b * BS + t + u * gridDim.x * BS: the
// library's contiguous kernel (k_contig) layout.  CASE only tells the cases
// apart in a profiler's per-kernel summary.
template <int BS, int U, int CASE = 0>
__global__ void __launch_bounds__(BS) p_copy(const uint4* __restrict__ in, uint4* __restrict__ out, int64_t nvec) {
  const int64_t v0 = (int64_t)blockIdx.x * BS + threadIdx.x;
  const int64_t step = (int64_t)gridDim.x * BS;
  uint4 x[U];
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (v0 + u * step < nvec) x[u] = ld_stream(in + v0 + u * step);
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (v0 + u * step < nvec) st_stream(out + v0 + u * step, x[u]);
}

template <int BS>
__global__ void __launch_bounds__(BS) p_add(const float4* __restrict__ a, const float4* __restrict__ b,
                                             float4* __restrict__ c, int64_t nvec) {
  const int64_t v = (int64_t)blockIdx.x * BS + threadIdx.x;
  if (v >= nvec) return;
  const float4 x = ld_stream(a + v), y = ld_stream(b + v);
  st_stream(c + v, make_float4(x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w));
}

template <int BS>
__global__ void __launch_bounds__(BS) p_fill(uint4* __restrict__ out, int64_t nvec, uint32_t value) {
  const int64_t v = (int64_t)blockIdx.x * BS + threadIdx.x;
  if (v < nvec) st_stream(out + v, make_uint4(value, value, value, value));
}

// 4 streams read, 3 written (AdamW's p, g, m, v -> p, m, v).
template <int BS>
__global__ void __launch_bounds__(BS) p_rw43(const float4* __restrict__ g, float4* __restrict__ p,
                                              float4* __restrict__ m, float4* __restrict__ s, int64_t nvec) {
  const int64_t v = (int64_t)blockIdx.x * BS + threadIdx.x;
  if (v >= nvec) return;
  const float4 gv = ld_stream(g + v), pv = ld_stream(p + v), mv = ld_stream(m + v), sv = ld_stream(s + v);
  st_stream(p + v, make_float4(pv.x + gv.x, pv.y + gv.y, pv.z + gv.z, pv.w + gv.w));
  st_stream(m + v, make_float4(mv.x + gv.x, mv.y + gv.y, mv.z + gv.z, mv.w + gv.w));
  st_stream(s + v, make_float4(sv.x + gv.x, sv.y + gv.y, sv.z + gv.z, sv.w + gv.w));
}

// The row kernels' pattern (log_softmax at c3's shape): one 1024-thread
// workgroup per row, the whole row in registers (VPT vectors per thread,
// vector tid + j * 1024), then (BARRIER) a workgroup-wide sum through LDS
// as the row statistics take, then the row written back.  Rows are walked
// with a stride of gridDim.x (grid = rows: one row per workgroup).  GRID
// names the launch's grid for a profiler's per-kernel summary.
template <int VPT, bool BARRIER, int GRID>
__global__ void __launch_bounds__(1024) p_rows(const uint4* __restrict__ in, uint4* __restrict__ out, int64_t rows,
                                                int rowvec) {
  __shared__ float red[16];
  const int tid = threadIdx.x;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const uint4* src = in + row * rowvec;
    uint4* dst = out + row * rowvec;
    uint4 x[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j)
      if (tid + j * 1024 < rowvec) x[j] = ld_stream(src + tid + j * 1024);
    if (BARRIER) {
      float s = 0.0f;
#pragma unroll
      for (int j = 0; j < VPT; ++j)
        if (tid + j * 1024 < rowvec) s += __uint_as_float(x[j].x & 0xffff0000u);
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
      __syncthreads();
      if ((tid & 63) == 0) red[tid >> 6] = s;
      __syncthreads();
      float t = 0.0f;
#pragma unroll
      for (int w = 0; w < 16; ++w) t += red[w];
      if (t == 1234.5f) x[0].y ^= 1u;  // keeps the sum live; never true for the zero-filled input
    }
#pragma unroll
    for (int j = 0; j < VPT; ++j)
      if (tid + j * 1024 < rowvec) st_stream(dst + tid + j * 1024, x[j]);
  }
}

// The backward row pattern (_log_softmax_backward_data at c3's shape): a
// 1024-thread workgroup per row holds the gradient row in registers, sums it
// through LDS, then streams the second input row and writes the result row
// (2 reads + 1 write per element).
template <int VPT>
__global__ void __launch_bounds__(1024) p_rows_bwd(const uint4* __restrict__ g, const uint4* __restrict__ y,
                                                    uint4* __restrict__ out, int rowvec) {
  __shared__ float red[16];
  const int tid = threadIdx.x;
  const int64_t base = (int64_t)blockIdx.x * rowvec;
  uint4 x[VPT];
#pragma unroll
  for (int j = 0; j < VPT; ++j)
    if (tid + j * 1024 < rowvec) x[j] = ld_stream(g + base + tid + j * 1024);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < VPT; ++j)
    if (tid + j * 1024 < rowvec) s += __uint_as_float(x[j].x & 0xffff0000u);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  if ((tid & 63) == 0) red[tid >> 6] = s;
  __syncthreads();
  float t = 0.0f;
#pragma unroll
  for (int w = 0; w < 16; ++w) t += red[w];
  const uint32_t flip = (t == 1234.5f) ? 1u : 0u;  // never set for the zero-filled input
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    if (tid + j * 1024 < rowvec) {
      const uint4 yv = ld_stream(y + base + tid + j * 1024);
      st_stream(out + base + tid + j * 1024,
                make_uint4(x[j].x ^ yv.x ^ flip, x[j].y ^ yv.y, x[j].z ^ yv.z, x[j].w ^ yv.w));
    }
  }
}

// FMA issue rate: 8 independent chains per lane, ITERS steps each.
template <typename T, int ITERS>
__global__ void __launch_bounds__(256) p_fma(T* __restrict__ out, T a, T b) {
  T c[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) c[k] = (T)(threadIdx.x + k);
  for (int i = 0; i < ITERS; ++i) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if constexpr (sizeof(T) == 4) c[k] = __builtin_fmaf(c[k], a, b);
      else c[k] = __builtin_fma(c[k], a, b);
    }
  }
  T s = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) s += c[k];
  out[(int64_t)blockIdx.x * 256 + threadIdx.x] = s;
}

// ------------------------------------------------------------- harness
template <typename F>
static double time_us(F&& launch, int reps = 20) {
  for (int i = 0; i < 3; ++i) launch(i);
  CHECK(hipDeviceSynchronize());
  hipEvent_t a, b;
  CHECK(hipEventCreate(&a));
  CHECK(hipEventCreate(&b));
  CHECK(hipEventRecord(a, 0));
  for (int i = 0; i < reps; ++i) launch(i);
  CHECK(hipEventRecord(b, 0));
  CHECK(hipEventSynchronize(b));
  CHECK(hipGetLastError());
  float ms = 0.0f;
  CHECK(hipEventElapsedTime(&ms, a, b));
  CHECK(hipEventDestroy(a));
  CHECK(hipEventDestroy(b));
  return 1e3 * ms / reps;
}

static void row(const char* name, double bytes, double us) {
  const double gbs = bytes / (us * 1e-6) / 1e9;
  printf("| %s | %.0f | %.1f | %.0f | %.1f |\n", name, bytes, us, gbs, 100.0 * gbs / kPeakGBs);
  fflush(stdout);
}

static void* dmalloc(size_t bytes) {
  void* p = nullptr;
  CHECK(hipMalloc(&p, bytes));
  CHECK(hipMemset(p, 0, bytes));
  return p;
}

static unsigned blocks(int64_t nvec, int bs, int u = 1) { return (unsigned)((nvec + (int64_t)bs * u - 1) / ((int64_t)bs * u)); }

int main() {
  int dev = 0;
  CHECK(hipSetDevice(dev));
  hipDeviceProp_t prop;
  CHECK(hipGetDeviceProperties(&prop, dev));
  printf("device: %s (%s), %d CUs\n\n", prop.name, prop.gcnArchName, prop.multiProcessorCount);
  printf("| case | bytes per launch | avg us | GB/s | %% of 8 TB/s |\n|---|---:|---:|---:|---:|\n");

  {  // 1 read + 1 write, 1 GiB each way
    const int64_t n = int64_t(1) << 28, nvec = n / 4;
    auto* in = (uint4*)dmalloc(n * 4);
    auto* out = (uint4*)dmalloc(n * 4);
    const double by = 8.0 * n;
    row("copy f32 2^28: 64 threads, 1 vector per thread", by,
        time_us([&](int) { p_copy<64, 1><<<blocks(nvec, 64), 64>>>(in, out, nvec); }));
    row("copy f32 2^28: 256 threads, 1 vector per thread", by,
        time_us([&](int) { p_copy<256, 1><<<blocks(nvec, 256), 256>>>(in, out, nvec); }));
    row("copy f32 2^28: 64 threads, 2 vectors per thread", by,
        time_us([&](int) { p_copy<64, 2><<<blocks(nvec, 64, 2), 64>>>(in, out, nvec); }));
    row("copy f32 2^28: 64 threads, 4 vectors per thread", by,
        time_us([&](int) { p_copy<64, 4><<<blocks(nvec, 64, 4), 64>>>(in, out, nvec); }));
    row("copy f32 2^28: 256 threads, 4 vectors per thread", by,
        time_us([&](int) { p_copy<256, 4><<<blocks(nvec, 256, 4), 256>>>(in, out, nvec); }));
    row("fill (write only) f32 2^28: 256 threads", 4.0 * n,
        time_us([&](int) { p_fill<256><<<blocks(nvec, 256), 256>>>(out, nvec, 0x3f800000u); }));
    row("fill (write only) f32 2^28: 64 threads", 4.0 * n,
        time_us([&](int) { p_fill<64><<<blocks(nvec, 64), 64>>>(out, nvec, 0x3f800000u); }));
    CHECK(hipFree(in));
    CHECK(hipFree(out));
  }
  {  // c1's shape: [4096, 4096] f32, six rotating sets (1.2 GB > the 256 MB MALL)
    const int64_t n = 4096 * 4096, nvec = n / 4;
    std::vector<float4*> a(6), b(6), c(6);
    for (int i = 0; i < 6; ++i) {
      a[i] = (float4*)dmalloc(n * 4);
      b[i] = (float4*)dmalloc(n * 4);
      c[i] = (float4*)dmalloc(n * 4);
    }
    row("copy f32 [4096,4096], 6 rotating sets: 64 threads, 1 vector", 8.0 * n, time_us([&](int i) {
          p_copy<64, 1, 1><<<blocks(nvec, 64), 64>>>((const uint4*)a[i % 6], (uint4*)c[i % 6], nvec);
        }, 60));
    row("add f32 [4096,4096] (c1), 6 rotating sets: 64 threads", 12.0 * n, time_us([&](int i) {
          p_add<64><<<blocks(nvec, 64), 64>>>(a[i % 6], b[i % 6], c[i % 6], nvec);
        }, 60));
    for (int i = 0; i < 6; ++i) {
      CHECK(hipFree(a[i]));
      CHECK(hipFree(b[i]));
      CHECK(hipFree(c[i]));
    }
  }
  {  // 4 reads + 3 writes (AdamW's streams), 2^27 f32 per stream
    const int64_t n = int64_t(1) << 27, nvec = n / 4;
    auto* g = (float4*)dmalloc(n * 4);
    auto* p = (float4*)dmalloc(n * 4);
    auto* m = (float4*)dmalloc(n * 4);
    auto* s = (float4*)dmalloc(n * 4);
    row("4 reads + 3 writes f32 2^27 per stream: 64 threads", 28.0 * n,
        time_us([&](int) { p_rw43<64><<<blocks(nvec, 64), 64>>>(g, p, m, s, nvec); }));
    CHECK(hipFree(g));
    CHECK(hipFree(p));
    CHECK(hipFree(m));
    CHECK(hipFree(s));
  }
  {  // c3's row pattern: [8192, 128256] bf16 rows of 16032 16-byte vectors
    const int64_t rows = 8192;
    const int rowvec = 128256 * 2 / 16;
    auto* in = (uint4*)dmalloc(rows * rowvec * 16);
    auto* out = (uint4*)dmalloc(rows * rowvec * 16);
    const double by = 2.0 * rows * rowvec * 16;
    const int cus = prop.multiProcessorCount;
    row("rows bf16 [8192,128256], row in registers: grid = rows", by,
        time_us([&](int) { p_rows<16, false, 0><<<(unsigned)rows, 1024>>>(in, out, rows, rowvec); }, 10));
    row("rows, row in registers + LDS row sum: grid = rows", by,
        time_us([&](int) { p_rows<16, true, 0><<<(unsigned)rows, 1024>>>(in, out, rows, rowvec); }, 10));
    row("rows, row in registers + LDS row sum: grid = 2 x CUs (persistent)", by,
        time_us([&](int) { p_rows<16, true, 2><<<(unsigned)(2 * cus), 1024>>>(in, out, rows, rowvec); }, 10));
    row("rows, row in registers + LDS row sum: grid = CUs (persistent)", by,
        time_us([&](int) { p_rows<16, true, 1><<<(unsigned)cus, 1024>>>(in, out, rows, rowvec); }, 10));
    auto* y = (uint4*)dmalloc(rows * rowvec * 16);
    row("backward rows (gradient row in registers + LDS sum, second row streamed): grid = rows", 1.5 * by,
        time_us([&](int) { p_rows_bwd<16><<<(unsigned)rows, 1024>>>(in, y, out, rowvec); }, 10));
    CHECK(hipFree(y));
    CHECK(hipFree(in));
    CHECK(hipFree(out));
  }
  {  // FMA issue rate
    constexpr int kIters = 4096;
    const unsigned grid = 256u * 64u;
    auto* o32 = (float*)dmalloc((size_t)grid * 256 * 4);
    auto* o64 = (double*)dmalloc((size_t)grid * 256 * 8);
    const double lane_fmas = (double)grid * 256 * 8 * kIters;
    const double t32 = time_us([&](int) { p_fma<float, kIters><<<grid, 256>>>(o32, 0.999f, 0.001f); }, 5);
    const double t64 = time_us([&](int) { p_fma<double, kIters><<<grid, 256>>>(o64, 0.999, 0.001); }, 5);
    printf("\n| FMA issue rate | lane FMAs per launch | avg us | T lane-FMA/s |\n|---|---:|---:|---:|\n");
    printf("| v_fma_f32 (no packed math) | %.0f | %.1f | %.1f |\n", lane_fmas, t32, lane_fmas / (t32 * 1e-6) / 1e12);
    printf("| v_fma_f64 | %.0f | %.1f | %.1f |\n", lane_fmas, t64, lane_fmas / (t64 * 1e-6) / 1e12);
    CHECK(hipFree(o32));
    CHECK(hipFree(o64));
  }
  return 0;
}
