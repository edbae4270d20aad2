// Shared device helpers for the gfx950 triangle kernels: element types, MFMA
// fragments, vector loads and the launch-error plumbing.
//
// MFMA convention used by every kernel (64-lane wavefront, lane l, g = l/16):
//   one 16x16 output tile D[16][16] per `mma()` call, fp32 accumulators;
//   A fragment: the 8 elements A[row = l%16][k = kbase + 8g + e], e = 0..7
//   B fragment: the 8 elements B[k = kbase + 8g + e][col = l%16]
//   D: lane l holds D[4g + r][l%16], r = 0..3
// The k-slot of element e of lane group g only has to be the same in A and B,
// so a kernel may assign any 8 distinct k values to (g, e) as long as it loads
// both operands with that same assignment. bf16 uses one
// v_mfma_f32_16x16x32_bf16; fp32 uses eight v_mfma_f32_16x16x4_f32, step e
// taking element e of every lane.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fjx {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;

// 8-element operand fragment per element type
template <typename T> struct Frag;
template <> struct Frag<bf16> { typedef bf16x8 type; };
template <> struct Frag<float> { typedef f32x8 type; };

__device__ __forceinline__ void mma(f32x4& acc, const bf16x8& a, const bf16x8& b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
}

__device__ __forceinline__ void mma(f32x4& acc, const f32x8& a, const f32x8& b) {
#pragma unroll
  for (int e = 0; e < 8; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], b[e], acc, 0, 0, 0);
}

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) { return static_cast<float>(x); }

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float x) { return static_cast<bf16>(x); }

// 8 contiguous elements <-> fragment (16 B for bf16, 32 B for fp32)
__device__ __forceinline__ bf16x8 load8(const bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }
__device__ __forceinline__ f32x8 load8(const float* p) {
  f32x4 lo = *reinterpret_cast<const f32x4*>(p);
  f32x4 hi = *reinterpret_cast<const f32x4*>(p + 4);
  return f32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}
__device__ __forceinline__ void store8(bf16* p, const bf16x8& v) { *reinterpret_cast<bf16x8*>(p) = v; }
__device__ __forceinline__ void store8(float* p, const f32x8& v) {
  *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
  *reinterpret_cast<f32x4*>(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
}

// 4 contiguous elements <-> fp32 (8 B for bf16, 16 B for fp32)
__device__ __forceinline__ void load4f(const bf16* p, float* o) {
  const bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = static_cast<float>(v[e]);
}
__device__ __forceinline__ void load4f(const float* p, float* o) {
  const f32x4 v = *reinterpret_cast<const f32x4*>(p);
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = v[e];
}
__device__ __forceinline__ void store4f(bf16* p, const float* f) {
  bf16x4 v;
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = static_cast<bf16>(f[e]);
  *reinterpret_cast<bf16x4*>(p) = v;
}
__device__ __forceinline__ void store4f(float* p, const float* f) {
  *reinterpret_cast<f32x4*>(p) = f32x4{f[0], f[1], f[2], f[3]};
}

// round an fp32 value through the element type T
template <typename T> __device__ __forceinline__ float round_to(float x) { return static_cast<float>(static_cast<T>(x)); }

// 8 elements -> fp32 and back
__device__ __forceinline__ void to_f32x8(const bf16x8& v, float* o) {
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = static_cast<float>(v[e]);
}
__device__ __forceinline__ void to_f32x8(const f32x8& v, float* o) {
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = v[e];
}
template <typename T> __device__ __forceinline__ typename Frag<T>::type pack8(const float* f);
template <> __device__ __forceinline__ bf16x8 pack8<bf16>(const float* f) {
  bf16x8 v;
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = static_cast<bf16>(f[e]);
  return v;
}
template <> __device__ __forceinline__ f32x8 pack8<float>(const float* f) {
  f32x8 v;
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = f[e];
  return v;
}

__device__ __forceinline__ float fast_sigmoid(float x) {
  // 1 / (1 + 2^(-x log2 e)) on the hardware v_exp_f32 / v_rcp_f32 (about 1 ulp
  // each); saturates cleanly to 0 (2^big = inf, rcp(inf) = 0) and to 1
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * kLog2e));
}
// the same sigmoid of x given y = -x log2 e, for a gate whose projection
// weights were scaled by -log2 e in advance (scale_wslab): no multiply per
// element
__device__ __forceinline__ float sigmoid_nl2e(float y) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(y));
}

// pair-grid row r = b n^2 + i n + j -> b n^2 + j n + i when t is set
__device__ __forceinline__ int64_t grid_row(int64_t r, int64_t n, int t) {
  if (!t) return r;
  const int64_t nn = n * n;
  const int64_t b = r / nn;
  const int64_t v = r - b * nn;
  const int64_t i = v / n;
  return b * nn + (v - i * n) * n + i;
}

// wave-wide xor shuffle of a float (64 lanes)
__device__ __forceinline__ float shfl_xor(float v, int mask) { return __shfl_xor(v, mask, 64); }

// v + v[lane ^ 1], then + [lane ^ 2]: the sum over each quad of lanes, the
// same additions in the same order as two shfl_xor steps, on DPP quad
// permutes (VALU operand modifiers) instead of ds_bpermute round trips
__device__ __forceinline__ float quad_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  return v;
}

// LayerNorm of one row of c <= 512 channels by one wave, lane l holding
// channels 8 l .. 8 l + 7
template <typename T>
__device__ __forceinline__ void ln_row8(const T* __restrict__ xr, const T* __restrict__ w, const T* __restrict__ b,
                                        T* __restrict__ yr, int c, float eps, int lane) {
  const int c0 = 8 * lane;
  const bool on = c0 < c;
  float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (on) to_f32x8(load8(xr + c0), v);
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) s += v[e];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) s += shfl_xor(s, o);
  const float mean = s / c;
  float q2 = 0.f;
  if (on) {
#pragma unroll
    for (int e = 0; e < 8; ++e) q2 += (v[e] - mean) * (v[e] - mean);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) q2 += shfl_xor(q2, o);
  const float rstd = __builtin_amdgcn_rsqf(q2 / c + eps);
  if (on) {
    float wv[8], bv[8], o[8];
    to_f32x8(load8(w + c0), wv);
    to_f32x8(load8(b + c0), bv);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (v[e] - mean) * rstd * wv[e] + bv[e];
    store8(yr + c0, pack8<T>(o));
  }
}

}  // namespace fjx
