// Issue-rate probe for the flash attention's per-tile instruction mix (a
// measurement aid, no counterpart in the reference).
//
// Per 16-query x 64-key tile a wave of flash_pipe_kernel_bf16 issues 10
// v_mfma_f32_16x16x32_bf16 (4 scores, 4 probability-value products, 2 row
// sums), 16 v_exp_f32 and about 24 other VALU instructions (16 bias
// widenings, 8 bf16 packs). This kernel issues exactly such a mix in a loop,
// with independent operands (no memory, no LDS, no barriers), on every SIMD
// of the GPU at a chosen number of waves per SIMD, so its time per iteration
// is the rate at which one SIMD can issue one tile's instructions: the floor
// the flash kernel's tile loop is measured against.
//
// Mixes: 0 = the kernel's (10 MFMA + 16 exp + 24 VALU), 1 = without the bias
// widenings (10 MFMA + 16 exp + 8 VALU), 2 = the 10 MFMAs alone, 3 = the 16
// exponentials alone, 4 = the 24 VALU alone; 5 = the same tile's scores and
// products on v_mfma_f32_32x32x16_bf16 (4 of them carry the matrix-pipe work
// of the 8 16x16x32 ones; the 2 row-sum MFMAs stay 16x16x32) with the same
// 16 exp + 24 VALU, 6 = those 6 MFMAs alone: whether the issue floor depends
// on the number of MFMA instructions or only on their matrix-pipe cycles.
//
// A second probe streams 16-byte accesses through HBM (copy, nontemporal
// copy, read only, write only) at a chosen number of workgroups per CU: the
// rate a plain streaming kernel reaches on this part, the practical ceiling
// the HBM-bound row kernels are measured against beside the 8 TB/s figure.
#include <hip/hip_runtime.h>

#include "fjx_common.hpp"
#include "fjx_kernels.hpp"

namespace fjx {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));  // a 32x32 MFMA accumulator

#define FJX_M(i) "v_mfma_f32_16x16x32_bf16 %" #i ", %34, %35, %" #i "\n"
#define FJX_E(j) "v_exp_f32 %" #j ", %36\n"
#define FJX_V(j) "v_fma_f32 %" #j ", %" #j ", 0.5, 1.0\n"
// operands: %0..%9 accumulators (f32x4), %10..%25 exponential results,
// %26..%33 VALU chains, %34 / %35 the MFMA's A and B fragments, %36 the
// exponentials' argument (a fixed normal value: the scores the kernel
// exponentiates are normal numbers, never infinities)
#define FJX_OPS                                                                                           \
  "+v"(c[0]), "+v"(c[1]), "+v"(c[2]), "+v"(c[3]), "+v"(c[4]), "+v"(c[5]), "+v"(c[6]), "+v"(c[7]),         \
      "+v"(c[8]), "+v"(c[9]), "+v"(e[0]), "+v"(e[1]), "+v"(e[2]), "+v"(e[3]), "+v"(e[4]), "+v"(e[5]),     \
      "+v"(e[6]), "+v"(e[7]), "+v"(e[8]), "+v"(e[9]), "+v"(e[10]), "+v"(e[11]), "+v"(e[12]), "+v"(e[13]), \
      "+v"(e[14]), "+v"(e[15]), "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]),   \
      "+v"(x[6]), "+v"(x[7])                                                                              \
  : "v"(fa), "v"(fb), "v"(xe)

template <int MIX>
__global__ __launch_bounds__(256) void issue_mix_kernel(float* sink, int iters) {
  f32x4 c[10];
  float e[16], x[8];
  bf16x8 fa, fb;
  const float t = 1e-3f * (float)threadIdx.x;
  const float xe = -0.75f - t;
#pragma unroll
  for (int i = 0; i < 10; ++i) c[i] = f32x4{t, t, t, t};
#pragma unroll
  for (int j = 0; j < 16; ++j) e[j] = -0.01f * (float)j;
#pragma unroll
  for (int j = 0; j < 8; ++j) x[j] = t + (float)j;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    fa[k] = static_cast<bf16>(0.001f * (float)k);
    fb[k] = static_cast<bf16>(t);
  }
  for (int it = 0; it < iters; ++it) {
    if constexpr (MIX == 0) {
      // 10 MFMA, each followed by its share of 16 exp and 24 VALU (8 VALU
      // chains, each used three times)
      asm volatile(FJX_M(0) FJX_E(10) FJX_E(11) FJX_V(26) FJX_V(27) FJX_V(28)
                   FJX_M(1) FJX_E(12) FJX_E(13) FJX_V(29) FJX_V(30) FJX_V(31)
                   FJX_M(2) FJX_E(14) FJX_E(15) FJX_V(32) FJX_V(33)
                   FJX_M(3) FJX_E(16) FJX_E(17) FJX_V(26) FJX_V(27) FJX_V(28)
                   FJX_M(4) FJX_E(18) FJX_E(19) FJX_V(29) FJX_V(30)
                   FJX_M(5) FJX_E(20) FJX_E(21) FJX_V(31) FJX_V(32) FJX_V(33)
                   FJX_M(6) FJX_E(22) FJX_E(23) FJX_V(26) FJX_V(27)
                   FJX_M(7) FJX_E(24) FJX_E(25) FJX_V(28) FJX_V(29) FJX_V(30)
                   FJX_M(8) FJX_V(31) FJX_V(32)
                   FJX_M(9) FJX_V(33)
                   : FJX_OPS);
    } else if constexpr (MIX == 1) {
      asm volatile(FJX_M(0) FJX_E(10) FJX_E(11) FJX_V(26)
                   FJX_M(1) FJX_E(12) FJX_E(13) FJX_V(27)
                   FJX_M(2) FJX_E(14) FJX_E(15) FJX_V(28)
                   FJX_M(3) FJX_E(16) FJX_E(17) FJX_V(29)
                   FJX_M(4) FJX_E(18) FJX_E(19) FJX_V(30)
                   FJX_M(5) FJX_E(20) FJX_E(21) FJX_V(31)
                   FJX_M(6) FJX_E(22) FJX_E(23) FJX_V(32)
                   FJX_M(7) FJX_E(24) FJX_E(25) FJX_V(33)
                   FJX_M(8) FJX_M(9)
                   : FJX_OPS);
    } else if constexpr (MIX == 2) {
      asm volatile(FJX_M(0) FJX_M(1) FJX_M(2) FJX_M(3) FJX_M(4) FJX_M(5) FJX_M(6) FJX_M(7) FJX_M(8) FJX_M(9)
                   : FJX_OPS);
    } else if constexpr (MIX == 3) {
      asm volatile(FJX_E(10) FJX_E(11) FJX_E(12) FJX_E(13) FJX_E(14) FJX_E(15) FJX_E(16) FJX_E(17)
                   FJX_E(18) FJX_E(19) FJX_E(20) FJX_E(21) FJX_E(22) FJX_E(23) FJX_E(24) FJX_E(25)
                   : FJX_OPS);
    } else {
      asm volatile(FJX_V(26) FJX_V(27) FJX_V(28) FJX_V(29) FJX_V(30) FJX_V(31) FJX_V(32) FJX_V(33)
                   FJX_V(26) FJX_V(27) FJX_V(28) FJX_V(29) FJX_V(30) FJX_V(31) FJX_V(32) FJX_V(33)
                   FJX_V(26) FJX_V(27) FJX_V(28) FJX_V(29) FJX_V(30) FJX_V(31) FJX_V(32) FJX_V(33)
                   : FJX_OPS);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 10; ++i) s += c[i][0] + c[i][3];
#pragma unroll
  for (int j = 0; j < 16; ++j) s += e[j];
#pragma unroll
  for (int j = 0; j < 8; ++j) s += x[j];
  sink[(int64_t)blockIdx.x * 256 + threadIdx.x] = s;
}
#undef FJX_M
#undef FJX_E
#undef FJX_V
#undef FJX_OPS

// mixes 5 and 6: %0, %1 the 16x16x32 accumulators, %2..%5 the 32x32x16 ones
// (f32x16), %6..%21 exponential results, %22..%29 VALU chains, %30 / %31 the
// MFMA fragments, %32 the exponentials' argument
#define FJX_M16(i) "v_mfma_f32_16x16x32_bf16 %" #i ", %30, %31, %" #i "\n"
#define FJX_M32(i) "v_mfma_f32_32x32x16_bf16 %" #i ", %30, %31, %" #i "\n"
#define FJX_E(j) "v_exp_f32 %" #j ", %32\n"
#define FJX_V(j) "v_fma_f32 %" #j ", %" #j ", 0.5, 1.0\n"
#define FJX_OPS32                                                                                         \
  "+v"(c[0]), "+v"(c[1]), "+v"(d[0]), "+v"(d[1]), "+v"(d[2]), "+v"(d[3]), "+v"(e[0]), "+v"(e[1]),         \
      "+v"(e[2]), "+v"(e[3]), "+v"(e[4]), "+v"(e[5]), "+v"(e[6]), "+v"(e[7]), "+v"(e[8]), "+v"(e[9]),     \
      "+v"(e[10]), "+v"(e[11]), "+v"(e[12]), "+v"(e[13]), "+v"(e[14]), "+v"(e[15]), "+v"(x[0]), "+v"(x[1]), \
      "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]), "+v"(x[6]), "+v"(x[7])                              \
  : "v"(fa), "v"(fb), "v"(xe)

template <int MIX>
__global__ __launch_bounds__(256) void issue_mix32_kernel(float* sink, int iters) {
  f32x4 c[2];
  f32x16 d[4];
  float e[16], x[8];
  bf16x8 fa, fb;
  const float t = 1e-3f * (float)threadIdx.x;
  const float xe = -0.75f - t;
#pragma unroll
  for (int i = 0; i < 2; ++i) c[i] = f32x4{t, t, t, t};
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int k = 0; k < 16; ++k) d[i][k] = t;
#pragma unroll
  for (int j = 0; j < 16; ++j) e[j] = -0.01f * (float)j;
#pragma unroll
  for (int j = 0; j < 8; ++j) x[j] = t + (float)j;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    fa[k] = static_cast<bf16>(0.001f * (float)k);
    fb[k] = static_cast<bf16>(t);
  }
  for (int it = 0; it < iters; ++it) {
    if constexpr (MIX == 5) {
      // each 32x32x16 MFMA (32 cycles) followed by the VALU work two 16x16x32
      // ones (16 cycles each) carry in mix 0
      asm volatile(FJX_M32(2) FJX_E(6) FJX_E(7) FJX_V(22) FJX_V(23) FJX_V(24) FJX_E(8) FJX_E(9) FJX_V(25) FJX_V(26) FJX_V(27)
                   FJX_M32(3) FJX_E(10) FJX_E(11) FJX_V(28) FJX_V(29) FJX_E(12) FJX_E(13) FJX_V(22) FJX_V(23) FJX_V(24)
                   FJX_M16(0) FJX_E(14) FJX_E(15) FJX_V(25) FJX_V(26)
                   FJX_M32(4) FJX_E(16) FJX_E(17) FJX_V(27) FJX_V(28) FJX_V(29) FJX_E(18) FJX_E(19) FJX_V(22) FJX_V(23)
                   FJX_M32(5) FJX_E(20) FJX_E(21) FJX_V(24) FJX_V(25) FJX_V(26)
                   FJX_M16(1) FJX_V(27) FJX_V(28) FJX_V(29)
                   : FJX_OPS32);
    } else {
      asm volatile(FJX_M32(2) FJX_M32(3) FJX_M16(0) FJX_M32(4) FJX_M32(5) FJX_M16(1) : FJX_OPS32);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 2; ++i) s += c[i][0] + c[i][3];
#pragma unroll
  for (int i = 0; i < 4; ++i) s += d[i][0] + d[i][15];
#pragma unroll
  for (int j = 0; j < 16; ++j) s += e[j];
#pragma unroll
  for (int j = 0; j < 8; ++j) s += x[j];
  sink[(int64_t)blockIdx.x * 256 + threadIdx.x] = s;
}
#undef FJX_M16
#undef FJX_M32
#undef FJX_E
#undef FJX_V
#undef FJX_OPS32

// HBM streaming probe: 16-byte accesses over two device buffers, a
// grid-stride loop of gridDim.x 256-thread workgroups, four accesses in
// flight per lane. Mode 0 copies a -> b, mode 1 copies with nontemporal
// loads and stores, mode 2 only reads a (folded into one value per lane
// that is stored only if it matches a constant), mode 3 only writes b.
template <int MODE>
__global__ __launch_bounds__(256) void hbm_stream_kernel(const u32x4* __restrict__ a, u32x4* __restrict__ b,
                                                         int64_t n, unsigned* sink) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  unsigned acc = 0;
  for (; i + 3 * stride < n; i += 4 * stride) {
    u32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if constexpr (MODE == 1) v[u] = __builtin_nontemporal_load(a + i + u * stride);
      else if constexpr (MODE == 3) v[u] = u32x4{(unsigned)i, 1u, 2u, (unsigned)u};
      else v[u] = a[i + u * stride];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if constexpr (MODE == 1) __builtin_nontemporal_store(v[u], b + i + u * stride);
      else if constexpr (MODE == 2) acc ^= v[u][u];
      else b[i + u * stride] = v[u];
    }
  }
  if (MODE == 2 && acc == 0x9E3779B9u) sink[0] = acc;
}

}  // namespace

// waves_per_simd waves on each SIMD of the device's CUs (256-thread
// workgroups: one wave per SIMD each), every wave `iters` iterations; the
// kernel time in ms (HIP events on `st`, synchronised)
int probe_issue_mix(int mix, int waves_per_simd, int iters, float* ms, hipStream_t st) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                               hipSuccess)
    return -1;
  const int blocks = cus * waves_per_simd;
  float* sink = nullptr;
  if (hipMallocAsync(reinterpret_cast<void**>(&sink), (size_t)blocks * 256 * sizeof(float), st) != hipSuccess)
    return -1;
  hipEvent_t a, b;
  if (hipEventCreate(&a) != hipSuccess) return -1;
  if (hipEventCreate(&b) != hipSuccess) return -1;
  auto launch = [&]() {
    switch (mix) {
      case 0: hipLaunchKernelGGL(issue_mix_kernel<0>, dim3(blocks), dim3(256), 0, st, sink, iters); break;
      case 1: hipLaunchKernelGGL(issue_mix_kernel<1>, dim3(blocks), dim3(256), 0, st, sink, iters); break;
      case 2: hipLaunchKernelGGL(issue_mix_kernel<2>, dim3(blocks), dim3(256), 0, st, sink, iters); break;
      case 3: hipLaunchKernelGGL(issue_mix_kernel<3>, dim3(blocks), dim3(256), 0, st, sink, iters); break;
      case 4: hipLaunchKernelGGL(issue_mix_kernel<4>, dim3(blocks), dim3(256), 0, st, sink, iters); break;
      case 5: hipLaunchKernelGGL(issue_mix32_kernel<5>, dim3(blocks), dim3(256), 0, st, sink, iters); break;
      default: hipLaunchKernelGGL(issue_mix32_kernel<6>, dim3(blocks), dim3(256), 0, st, sink, iters); break;
    }
  };
  launch();  // warm-up: the clock settles under load
  (void)hipEventRecord(a, st);
  launch();
  (void)hipEventRecord(b, st);
  int rc = hipEventSynchronize(b) == hipSuccess && hipEventElapsedTime(ms, a, b) == hipSuccess ? 0 : -1;
  (void)hipFreeAsync(sink, st);
  (void)hipStreamSynchronize(st);
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  return rc;
}

// mode (0-3, hbm_stream_kernel) over `bytes` (a multiple of 4 KiB) with
// wgs_per_cu workgroups per CU: one warm-up launch, then one timed launch;
// its time in ms (HIP events on `st`, synchronised). The two buffers are
// allocated and freed on `st`.
int probe_hbm_stream(int mode, int wgs_per_cu, int64_t bytes, float* ms, hipStream_t st) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                               hipSuccess)
    return -1;
  u32x4 *a = nullptr, *b = nullptr;
  unsigned* sink = nullptr;
  if (hipMallocAsync(reinterpret_cast<void**>(&a), (size_t)bytes, st) != hipSuccess) return -1;
  if (hipMallocAsync(reinterpret_cast<void**>(&b), (size_t)bytes, st) != hipSuccess) return -1;
  if (hipMallocAsync(reinterpret_cast<void**>(&sink), 64, st) != hipSuccess) return -1;
  if (hipMemsetAsync(a, 1, (size_t)bytes, st) != hipSuccess) return -1;
  const int64_t n = bytes / 16;
  const dim3 grid((unsigned)(cus * wgs_per_cu));
  auto launch = [&]() {
    switch (mode) {
      case 0: hipLaunchKernelGGL(hbm_stream_kernel<0>, grid, dim3(256), 0, st, a, b, n, sink); break;
      case 1: hipLaunchKernelGGL(hbm_stream_kernel<1>, grid, dim3(256), 0, st, a, b, n, sink); break;
      case 2: hipLaunchKernelGGL(hbm_stream_kernel<2>, grid, dim3(256), 0, st, a, b, n, sink); break;
      default: hipLaunchKernelGGL(hbm_stream_kernel<3>, grid, dim3(256), 0, st, a, b, n, sink); break;
    }
  };
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess) return -1;
  if (hipEventCreate(&e1) != hipSuccess) return -1;
  launch();
  (void)hipEventRecord(e0, st);
  launch();
  (void)hipEventRecord(e1, st);
  int rc = hipEventSynchronize(e1) == hipSuccess && hipEventElapsedTime(ms, e0, e1) == hipSuccess ? 0 : -1;
  (void)hipFreeAsync(a, st);
  (void)hipFreeAsync(b, st);
  (void)hipFreeAsync(sink, st);
  (void)hipStreamSynchronize(st);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return rc;
}

}  // namespace fjx
