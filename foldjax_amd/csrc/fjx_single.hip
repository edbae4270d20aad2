// Single-track helpers for the attention with pair bias of a Pairformer block
// (Boltz-2 attention_pair_bias_forward): row LayerNorm, head split into the
// padded flash layout, the pair-bias projection LN(z) W_z^T, the key mask
// bias and the gate-and-unpad step before the output projection.
#include "fjx_common.hpp"
#include "fjx_kernels.hpp"

namespace fjx {

namespace {

// one wave per row, C <= 1024, C % 64 == 0 or handled by the stride loop
template <typename T>
__global__ __launch_bounds__(256) void layernorm_rows_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                             const T* __restrict__ b, T* __restrict__ y,
                                                             int64_t rows, int c, float eps) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const T* xr = x + row * c;
  float v[16];
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const int ch = lane + 64 * u;
    v[u] = ch < c ? to_f32(xr[ch]) : 0.f;
    s += v[u];
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) s += shfl_xor(s, o);
  const float mean = s / c;
  float q2 = 0.f;
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const int ch = lane + 64 * u;
    if (ch < c) q2 += (v[u] - mean) * (v[u] - mean);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) q2 += shfl_xor(q2, o);
  const float rstd = __builtin_amdgcn_rsqf(q2 / c + eps);
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const int ch = lane + 64 * u;
    if (ch < c) y[row * c + ch] = from_f32<T>((v[u] - mean) * rstd * to_f32(w[ch]) + to_f32(b[ch]));
  }
}

// qkv rows [B*N][ld] holding q | k | v (each heads*dh wide) ->
//   q, k: [B][H][Np][32] (q times q_mul), vt: [B][H*32][Np]; zero padding in d and keys
template <typename T>
__global__ void split_heads_kernel(const T* __restrict__ qkv, int64_t ld, int64_t batch, int64_t n, int64_t np,
                                   int heads, int dh, float q_mul, T* __restrict__ q, T* __restrict__ k,
                                   T* __restrict__ vt) {
  const int64_t total = batch * heads * np * 32;
  const int64_t hd = (int64_t)heads * dh;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int d = idx % 32;
    const int64_t s = (idx / 32) % np;
    const int64_t h = (idx / (32 * np)) % heads;
    const int64_t b = idx / (32 * np * heads);
    float qv = 0.f, kv = 0.f, vv = 0.f;
    if (s < n && d < dh) {
      const T* r = qkv + (b * n + s) * ld + h * dh + d;
      qv = to_f32(r[0]) * q_mul;
      kv = to_f32(r[hd]);
      vv = to_f32(r[2 * hd]);
    }
    q[idx] = from_f32<T>(qv);
    k[idx] = from_f32<T>(kv);
    vt[((b * heads + h) * 32 + d) * np + s] = from_f32<T>(vv);
  }
}

// bias[b][h][q][k] = log2(e) * LN(z[b,q,k,:]) . w[h,:], 128 channels, 4 threads per
// position of the padded [np, np] grid; padded entries are written as zeros so
// that the attention never reads uninitialised memory next to a -inf key mask
template <typename T>
__global__ __launch_bounds__(256) void pair_bias_kernel(const T* __restrict__ z, const T* __restrict__ ln_w,
                                                        const T* __restrict__ ln_b, const T* __restrict__ w,
                                                        T* __restrict__ bias, int64_t batch, int64_t n,
                                                        int64_t np, int heads, float eps) {
  constexpr int C = 128;
  const int64_t ppos = (int64_t)blockIdx.x * 64 + (threadIdx.x >> 2);  // padded position
  const int part = threadIdx.x & 3;
  const int64_t total = batch * np * np;
  const bool in_grid = ppos < total;
  const int64_t b = in_grid ? ppos / (np * np) : 0;
  const int64_t qi = in_grid ? (ppos / np) % np : 0;
  const int64_t ki = in_grid ? ppos % np : 0;
  const bool ok = in_grid && qi < n && ki < n;
  const int64_t pos = (b * n + qi) * n + ki;
  float v[32];
  const int c0 = part * 32;
  if (ok) {
#pragma unroll
    for (int q = 0; q < 4; ++q) to_f32x8(load8(z + pos * C + c0 + 8 * q), v + 8 * q);
  } else {
#pragma unroll
    for (int e = 0; e < 32; ++e) v[e] = 0.f;
  }
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 32; ++e) s += v[e];
  s += shfl_xor(s, 1);
  s += shfl_xor(s, 2);
  const float mean = s * (1.0f / C);
  float q2 = 0.f;
#pragma unroll
  for (int e = 0; e < 32; ++e) q2 += (v[e] - mean) * (v[e] - mean);
  q2 += shfl_xor(q2, 1);
  q2 += shfl_xor(q2, 2);
  const float rstd = __builtin_amdgcn_rsqf(q2 * (1.0f / C) + eps);
#pragma unroll
  for (int e = 0; e < 32; ++e) v[e] = (v[e] - mean) * rstd * to_f32(ln_w[c0 + e]) + to_f32(ln_b[c0 + e]);
  for (int h = 0; h < heads; ++h) {
    float acc = 0.f;
#pragma unroll
    for (int e = 0; e < 32; ++e) acc += v[e] * to_f32(w[h * C + c0 + e]);
    acc += shfl_xor(acc, 1);
    acc += shfl_xor(acc, 2);
    if (in_grid && part == 0) bias[((b * heads + h) * np + qi) * np + ki] = from_f32<T>(ok ? acc * kLog2e : 0.f);
  }
}

// mb[b][k] = log2(e) * (1 - mask[b,k]) * (-inf_const), -inf for padded keys
template <typename T>
__global__ void key_mask_kernel(const T* __restrict__ mask, float* __restrict__ mb, int64_t batch, int64_t n,
                                int64_t np, float inf) {
  const int64_t total = batch * np;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t k = idx % np;
    const int64_t b = idx / np;
    float v = -INFINITY;
    if (k < n) v = mask ? (1.0f - to_f32(mask[b * n + k])) * (-inf) * kLog2e : 0.f;
    mb[idx] = v;
  }
}

// out[r][h*dh + d] = g[r*ldg + h*dh + d] * o[r][h][d] (o rows padded to 32 per head)
template <typename T>
__global__ void gate_unpad_kernel(const T* __restrict__ o, const T* __restrict__ g, int64_t ldg, T* __restrict__ out,
                                  int64_t rows, int heads, int dh) {
  const int64_t hd = (int64_t)heads * dh;
  const int64_t total = rows * hd;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = idx / hd;
    const int64_t c = idx % hd;
    const int64_t h = c / dh;
    const int64_t d = c % dh;
    out[idx] = from_f32<T>(to_f32(g[r * ldg + c]) * to_f32(o[(r * heads + h) * 32 + d]));
  }
}

dim3 grid_stride(int64_t total) {
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  return dim3((unsigned)blocks);
}

}  // namespace

template <typename T>
void launch_layernorm_rows(const T* x, const T* w, const T* b, T* y, int64_t rows, int c, float eps, hipStream_t st) {
  hipLaunchKernelGGL(layernorm_rows_kernel<T>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, x, w, b, y, rows, c,
                     eps);
}
template <typename T>
void launch_split_heads(const T* qkv, int64_t ld, int64_t batch, int64_t n, int64_t np, int heads, int dh,
                        float q_mul, T* q, T* k, T* vt, hipStream_t st) {
  hipLaunchKernelGGL(split_heads_kernel<T>, grid_stride(batch * heads * np * 32), dim3(256), 0, st, qkv, ld, batch, n,
                     np, heads, dh, q_mul, q, k, vt);
}
template <typename T>
void launch_pair_bias(const T* z, const T* ln_w, const T* ln_b, const T* w, T* bias, int64_t batch, int64_t n,
                      int64_t np, int heads, float eps, hipStream_t st) {
  const int64_t total = batch * np * np;
  hipLaunchKernelGGL(pair_bias_kernel<T>, dim3((unsigned)((total + 63) / 64)), dim3(256), 0, st, z, ln_w, ln_b, w,
                     bias, batch, n, np, heads, eps);
}
template <typename T>
void launch_key_mask(const T* mask, float* mb, int64_t batch, int64_t n, int64_t np, float inf, hipStream_t st) {
  hipLaunchKernelGGL(key_mask_kernel<T>, grid_stride(batch * np), dim3(256), 0, st, mask, mb, batch, n, np, inf);
}
template <typename T>
void launch_gate_unpad(const T* o, const T* g, int64_t ldg, T* out, int64_t rows, int heads, int dh,
                       hipStream_t st) {
  hipLaunchKernelGGL(gate_unpad_kernel<T>, grid_stride(rows * heads * dh), dim3(256), 0, st, o, g, ldg, out, rows,
                     heads, dh);
}

#define FJX_INST(T)                                                                                              \
  template void launch_layernorm_rows<T>(const T*, const T*, const T*, T*, int64_t, int, float, hipStream_t);   \
  template void launch_split_heads<T>(const T*, int64_t, int64_t, int64_t, int64_t, int, int, float, T*, T*, T*, \
                                      hipStream_t);                                                              \
  template void launch_pair_bias<T>(const T*, const T*, const T*, const T*, T*, int64_t, int64_t, int64_t, int,  \
                                    float, hipStream_t);                                                         \
  template void launch_key_mask<T>(const T*, float*, int64_t, int64_t, int64_t, float, hipStream_t);             \
  template void launch_gate_unpad<T>(const T*, const T*, int64_t, T*, int64_t, int, int, hipStream_t);
FJX_INST(bf16)
FJX_INST(float)
#undef FJX_INST

}  // namespace fjx
