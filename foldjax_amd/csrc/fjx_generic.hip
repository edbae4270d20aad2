// Layout and elementwise kernels of the general-width paths: the triangle
// ops and the transition for channel widths the fused kernels do not take
// (the fused ones are built for c_z = c_h = 128, H*D = 128). The C ABI layer
// composes these with the row LayerNorm, the generic GEMM, the contraction
// and the flash attention core into the same computation:
//
//   tri-mul:  xn = LN_in(x) -> G = sigmoid(xn g_in^T), P = (xn p_in^T) * G
//             -> a, b = mask * P, channel-major in the virtual grid
//             -> o[c] = a[c] b[c]^T -> LN_out(o) -> (.. p_out^T) * sigmoid(xn g_out^T)
//   tri-attn: xn = LN(x) in the virtual grid -> q|k|v|g and the bias by GEMM
//             -> padded head layouts -> flash core -> o * sigmoid(g) -> o w_o^T
//   transition: LN -> silu(xn a^T) * (xn b^T) -> (..) o^T [* row mask]
//
// Positions of the virtual grid are v = r*n + s; for the incoming direction
// and the ending node they read the original grid at s*n + r.
#include "fjx_common.hpp"
#include "fjx_kernels.hpp"

namespace fjx {

namespace {

__device__ __forceinline__ int64_t orig_pos(int64_t v, int64_t n, int t) {
  if (!t) return v;
  const int64_t r = v / n;
  return (v - r * n) * n + r;
}

dim3 stride_grid(int64_t total) {
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  return dim3((unsigned)blocks);
}

// one wave per position: y[b][v][:] = LN(x[b][orig(v)][:]), c <= 1024
template <typename T>
__global__ __launch_bounds__(256) void ln_grid_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                      const T* __restrict__ b, T* __restrict__ y, int64_t rows,
                                                      int64_t n, int c, float eps, int t) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const int64_t nn = n * n;
  const int64_t bb = row / nn;
  const T* xr = x + (bb * nn + orig_pos(row - bb * nn, n, t)) * c;
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

// dst[b][c][v] = src[b][orig(v)][c0 + c] * mask[b][orig(v)] (c < C), through
// 64 x 64 LDS tiles so that both sides move whole rows
template <typename T>
__global__ __launch_bounds__(256) void to_channel_major_kernel(const T* __restrict__ src, int64_t ld, int c0, int C,
                                                               const T* __restrict__ mask, T* __restrict__ dst,
                                                               int64_t n, int t) {
  __shared__ float tile[64][65];
  const int64_t nn = n * n;
  const int64_t vtiles = (nn + 63) / 64;
  const int ctiles = (C + 63) / 64;
  int64_t id = blockIdx.x;
  const int ct = (int)(id % ctiles);
  id /= ctiles;
  const int64_t vt = id % vtiles;
  const int64_t bb = id / vtiles;
  const int64_t v0 = vt * 64;
  const int cb = ct * 64;
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int pv = e >> 6, pc = e & 63;
    const int64_t v = v0 + pv;
    const int c = cb + pc;
    float val = 0.f;
    if (v < nn && c < C) {
      const int64_t o = bb * nn + orig_pos(v, n, t);
      val = to_f32(src[o * ld + c0 + c]);
      if (mask) val *= to_f32(mask[o]);
    }
    tile[pv][pc] = val;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int pc = e >> 6, pv = e & 63;
    const int64_t v = v0 + pv;
    const int c = cb + pc;
    if (v < nn && c < C) dst[(bb * C + c) * nn + v] = from_f32<T>(tile[pv][pc]);
  }
}

// dst[b][v][c] = src[b][c][v]
template <typename T>
__global__ __launch_bounds__(256) void to_position_major_kernel(const T* __restrict__ src, int C, T* __restrict__ dst,
                                                                int64_t nn) {
  __shared__ float tile[64][65];
  const int64_t vtiles = (nn + 63) / 64;
  const int ctiles = (C + 63) / 64;
  int64_t id = blockIdx.x;
  const int ct = (int)(id % ctiles);
  id /= ctiles;
  const int64_t vt = id % vtiles;
  const int64_t bb = id / vtiles;
  const int64_t v0 = vt * 64;
  const int cb = ct * 64;
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int pc = e >> 6, pv = e & 63;
    const int64_t v = v0 + pv;
    const int c = cb + pc;
    tile[pc][pv] = (v < nn && c < C) ? to_f32(src[(bb * C + c) * nn + v]) : 0.f;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int pv = e >> 6, pc = e & 63;
    const int64_t v = v0 + pv;
    const int c = cb + pc;
    if (v < nn && c < C) dst[(bb * nn + v) * C + c] = from_f32<T>(tile[pc][pv]);
  }
}

// q/k of the flash core: dst[br][h][s][d] (s < np) = src[br*n + s][c0 + 32h + d] * mul, zero padded keys
template <typename T>
__global__ void split_qk_kernel(const T* __restrict__ src, int64_t ld, int64_t c0, T* __restrict__ dst, int64_t rows,
                                int64_t n, int64_t np, int heads, float mul) {
  const int64_t total = rows * heads * np * 32;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int d = (int)(idx % 32);
    const int64_t s = (idx / 32) % np;
    const int h = (int)((idx / (32 * np)) % heads);
    const int64_t br = idx / (32 * np * heads);
    dst[idx] = s < n ? from_f32<T>(to_f32(src[(br * n + s) * ld + c0 + 32 * h + d]) * mul) : from_f32<T>(0.f);
  }
}

// triangle bias planes: dst[b][h][q][k] (np x np) = src[b][q*n + k][c0 + h] * log2 e, zeros outside
template <typename T>
__global__ void bias_planes_kernel(const T* __restrict__ src, int64_t ld, int64_t c0, T* __restrict__ dst,
                                   int64_t batch, int64_t n, int64_t np, int heads) {
  const int64_t total = batch * heads * np * np;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t k = idx % np;
    const int64_t q = (idx / np) % np;
    const int h = (int)((idx / (np * np)) % heads);
    const int64_t bb = idx / (np * np * heads);
    dst[idx] = (q < n && k < n) ? from_f32<T>(to_f32(src[(bb * n * n + q * n + k) * ld + c0 + h]) * kLog2e)
                                : from_f32<T>(0.f);
  }
}

// mask bias of row r: mb[b][r][k] = inf * (mask[b][orig(r*n + k)] - 1) * log2 e (0 without a mask),
// -inf for the padded keys
template <typename T>
__global__ void grid_mask_bias_kernel(const T* __restrict__ mask, float* __restrict__ mb, int64_t batch, int64_t n,
                                      int64_t np, float inf, int t) {
  const int64_t total = batch * n * np;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t k = idx % np;
    const int64_t r = (idx / np) % n;
    const int64_t bb = idx / (np * n);
    float v = -INFINITY;
    if (k < n) v = mask ? inf * (to_f32(mask[bb * n * n + orig_pos(r * n + k, n, t)]) - 1.0f) * kLog2e : 0.f;
    mb[idx] = v;
  }
}

// o[i][j] *= g[i*ldg + c0 + j] for rows x width
template <typename T>
__global__ void gate_rows_kernel(T* __restrict__ o, const T* __restrict__ g, int64_t ldg, int64_t c0, int64_t rows,
                                 int width) {
  const int64_t total = rows * width;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = idx / width;
    const int j = (int)(idx - i * width);
    o[idx] = from_f32<T>(to_f32(o[idx]) * to_f32(g[i * ldg + c0 + j]));
  }
}


// ---- vectorized forms (8 contiguous elements, 16-byte accesses for bf16),
// used when the widths and offsets are multiples of 8

template <typename T>
__global__ __launch_bounds__(256) void ln_grid8_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                       const T* __restrict__ b, T* __restrict__ y, int64_t rows,
                                                       int64_t n, int c, float eps, int t) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t nn = n * n;
  const int64_t bb = row / nn;
  ln_row8<T>(x + (bb * nn + orig_pos(row - bb * nn, n, t)) * c, w, b, y + row * c, c, eps, threadIdx.x & 63);
}

// split_qk_kernel, 8 head dims per thread
template <typename T>
__global__ void split_qk8_kernel(const T* __restrict__ src, int64_t ld, int64_t c0, T* __restrict__ dst, int64_t rows,
                                 int64_t n, int64_t np, int heads, float mul) {
  const int64_t total = rows * heads * np * 4;
  for (int64_t i8 = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i8 < total;
       i8 += (int64_t)gridDim.x * blockDim.x) {
    const int d0 = (int)(i8 & 3) * 8;
    int64_t r = i8 >> 2;
    const int64_t s = r % np;
    r /= np;
    const int h = (int)(r % heads);
    const int64_t br = r / heads;
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (s < n) {
      to_f32x8(load8(src + (br * n + s) * ld + c0 + 32 * h + d0), v);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] *= mul;
    }
    store8(dst + i8 * 8, pack8<T>(v));
  }
}

// v of the flash core, keys innermost: dst[br][hd][s] = src[br*n + s][c0 + hd] (zero for
// s >= n), through 64 x 64 LDS tiles so that both sides move whole rows
template <typename T>
__global__ __launch_bounds__(256) void split_vt_tiled_kernel(const T* __restrict__ src, int64_t ld, int64_t c0,
                                                             T* __restrict__ dst, int64_t n, int64_t np,
                                                             int hd_total) {
  __shared__ T tile[64][66];
  const int htiles = (hd_total + 63) / 64;
  const int64_t stiles = (np + 63) / 64;
  int64_t id = blockIdx.x;
  const int ht = (int)(id % htiles);
  id /= htiles;
  const int64_t st = id % stiles;
  const int64_t br = id / stiles;
  const int64_t s0 = st * 64;
  const int h0 = ht * 64;
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int sl = e >> 6, hl = e & 63;
    const int64_t s = s0 + sl;
    const int hd = h0 + hl;
    tile[sl][hl] = (s < n && hd < hd_total) ? src[(br * n + s) * ld + c0 + hd] : from_f32<T>(0.f);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 64 * 64; e += 256) {
    const int hl = e >> 6, sl = e & 63;
    const int64_t s = s0 + sl;
    const int hd = h0 + hl;
    if (s < np && hd < hd_total) dst[(br * hd_total + hd) * np + s] = tile[sl][hl];
  }
}

// gate_rows_kernel, 8 columns per thread
template <typename T>
__global__ void gate_rows8_kernel(T* __restrict__ o, const T* __restrict__ g, int64_t ldg, int64_t c0, int64_t rows,
                                  int width) {
  const int w8 = width / 8;
  const int64_t total = rows * w8;
  for (int64_t i8 = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i8 < total;
       i8 += (int64_t)gridDim.x * blockDim.x) {
    const int64_t i = i8 / w8;
    const int j = (int)(i8 - i * w8) * 8;
    float ov[8], gv[8];
    to_f32x8(load8(o + i * width + j), ov);
    to_f32x8(load8(g + i * ldg + c0 + j), gv);
#pragma unroll
    for (int e = 0; e < 8; ++e) ov[e] *= gv[e];
    store8(o + i * width + j, pack8<T>(ov));
  }
}

// to_channel_major_kernel and to_position_major_kernel with 16-byte global
// accesses (8 channels of a position, 8 positions of a channel per thread);
// the float tile's 65-float rows keep both LDS phases conflict-free
template <typename T>
__global__ __launch_bounds__(256) void to_channel_major8_kernel(const T* __restrict__ src, int64_t ld, int c0, int C,
                                                                const T* __restrict__ mask, T* __restrict__ dst,
                                                                int64_t n, int t) {
  __shared__ float tile[64][65];
  const int64_t nn = n * n;
  const int64_t vtiles = (nn + 63) / 64;
  const int ctiles = (C + 63) / 64;
  int64_t id = blockIdx.x;
  const int ct = (int)(id % ctiles);
  id /= ctiles;
  const int64_t vt = id % vtiles;
  const int64_t bb = id / vtiles;
  const int64_t v0 = vt * 64;
  const int cb = ct * 64;
  for (int e = threadIdx.x; e < 512; e += 256) {
    const int pv = e >> 3, cc = (e & 7) * 8;
    const int64_t v = v0 + pv;
    const int c = cb + cc;
    float val[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (v < nn && c < C) {
      const int64_t o = bb * nn + orig_pos(v, n, t);
      to_f32x8(load8(src + o * ld + c0 + c), val);
      if (mask) {
        const float m = to_f32(mask[o]);
#pragma unroll
        for (int k = 0; k < 8; ++k) val[k] *= m;
      }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) tile[pv][cc + k] = val[k];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 512; e += 256) {
    const int pc = e >> 3, vv = (e & 7) * 8;
    const int64_t v = v0 + vv;
    const int c = cb + pc;
    if (v < nn && c < C) {
      float o8[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) o8[k] = tile[vv + k][pc];
      store8(dst + (bb * C + c) * nn + v, pack8<T>(o8));
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void to_position_major8_kernel(const T* __restrict__ src, int C, T* __restrict__ dst,
                                                                 int64_t nn) {
  __shared__ float tile[64][65];
  const int64_t vtiles = (nn + 63) / 64;
  const int ctiles = (C + 63) / 64;
  int64_t id = blockIdx.x;
  const int ct = (int)(id % ctiles);
  id /= ctiles;
  const int64_t vt = id % vtiles;
  const int64_t bb = id / vtiles;
  const int64_t v0 = vt * 64;
  const int cb = ct * 64;
  for (int e = threadIdx.x; e < 512; e += 256) {
    const int pc = e >> 3, vv = (e & 7) * 8;
    const int64_t v = v0 + vv;
    const int c = cb + pc;
    float val[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (v < nn && c < C) to_f32x8(load8(src + (bb * C + c) * nn + v), val);
#pragma unroll
    for (int k = 0; k < 8; ++k) tile[pc][vv + k] = val[k];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < 512; e += 256) {
    const int pv = e >> 3, cc = (e & 7) * 8;
    const int64_t v = v0 + pv;
    const int c = cb + cc;
    if (v < nn && c < C) {
      float o8[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) o8[k] = tile[cc + k][pv];
      store8(dst + (bb * nn + v) * C + c, pack8<T>(o8));
    }
  }
}

// out[b][orig(v)][c] = (T(y[b][v][c] * m) + residual[b][orig(v)][c]) * (g != 0),
// with m the row mask and g the output mask at the output position (1 without);
// y the sum of `splits` partial products ss elements apart
template <typename T>
__global__ void scatter_add_kernel(const T* __restrict__ y, const T* __restrict__ row_mask,
                                   const T* __restrict__ residual, const T* __restrict__ out_mask,
                                   T* __restrict__ out, int64_t rows, int64_t n, int c, int t, int splits, int64_t ss) {
  const int64_t total = rows * c;
  const int64_t nn = n * n;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = idx / c;
    const int ch = (int)(idx - row * c);
    const int64_t bb = row / nn;
    const int64_t o = bb * nn + orig_pos(row - bb * nn, n, t);
    float v = to_f32(y[idx]);
    for (int s = 1; s < splits; ++s) v += to_f32(y[s * ss + idx]);
    if (row_mask) v *= to_f32(row_mask[o]);
    v = round_to<T>(v);
    if (residual) v += to_f32(residual[o * c + ch]);
    if (out_mask && to_f32(out_mask[o]) == 0.f) v *= 0.f;
    out[o * c + ch] = from_f32<T>(v);
  }
}

// scatter_add_kernel, 8 channels per thread
template <typename T>
__global__ void scatter_add8_kernel(const T* __restrict__ y, const T* __restrict__ row_mask,
                                    const T* __restrict__ residual, const T* __restrict__ out_mask,
                                    T* __restrict__ out, int64_t rows, int64_t n, int c, int t, int splits,
                                    int64_t ss) {
  const int c8 = c / 8;
  const int64_t total = rows * c8;
  const int64_t nn = n * n;
  for (int64_t i8 = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i8 < total;
       i8 += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = i8 / c8;
    const int ch = (int)(i8 - row * c8) * 8;
    const int64_t bb = row / nn;
    const int64_t o = bb * nn + orig_pos(row - bb * nn, n, t);
    float v[8];
    to_f32x8(load8(y + row * c + ch), v);
    for (int s = 1; s < splits; ++s) {
      float w[8];
      to_f32x8(load8(y + s * ss + row * c + ch), w);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] += w[e];
    }
    const float m = row_mask ? to_f32(row_mask[o]) : 1.f;
    const float g = out_mask && to_f32(out_mask[o]) == 0.f ? 0.f : 1.f;
    float r[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (residual) to_f32x8(load8(residual + o * c + ch), r);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (round_to<T>(v[e] * m) + r[e]) * g;
    store8(out + o * c + ch, pack8<T>(v));
  }
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

template <typename T>
void launch_ln_grid(const T* x, const T* w, const T* b, T* y, int64_t batch, int64_t n, int c, float eps, int t,
                    hipStream_t st) {
  const int64_t rows = batch * n * n;
  if (c % 8 == 0 && c <= 512 && al16(x) && al16(w) && al16(b) && al16(y))
    hipLaunchKernelGGL(ln_grid8_kernel<T>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, x, w, b, y, rows, n, c,
                       eps, t);
  else
    hipLaunchKernelGGL(ln_grid_kernel<T>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, x, w, b, y, rows, n, c,
                       eps, t);
}
template <typename T>
void launch_to_channel_major(const T* src, int64_t ld, int c0, int C, const T* mask, T* dst, int64_t batch, int64_t n,
                             int t, hipStream_t st) {
  const int64_t blocks = batch * ((n * n + 63) / 64) * ((C + 63) / 64);
  if (C % 8 == 0 && ld % 8 == 0 && c0 % 8 == 0 && (n * n) % 8 == 0 && al16(src) && al16(dst))
    hipLaunchKernelGGL(to_channel_major8_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, st, src, ld, c0, C, mask,
                       dst, n, t);
  else
    hipLaunchKernelGGL(to_channel_major_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, st, src, ld, c0, C, mask, dst,
                       n, t);
}
template <typename T>
void launch_to_position_major(const T* src, int C, T* dst, int64_t batch, int64_t nn, hipStream_t st) {
  const int64_t blocks = batch * ((nn + 63) / 64) * ((C + 63) / 64);
  if (C % 8 == 0 && nn % 8 == 0 && al16(src) && al16(dst))
    hipLaunchKernelGGL(to_position_major8_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, st, src, C, dst, nn);
  else
    hipLaunchKernelGGL(to_position_major_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, st, src, C, dst, nn);
}
template <typename T>
void launch_split_qk(const T* src, int64_t ld, int64_t c0, T* dst, int64_t rows, int64_t n, int64_t np, int heads,
                     float mul, hipStream_t st) {
  if (ld % 8 == 0 && c0 % 8 == 0 && al16(src) && al16(dst))
    hipLaunchKernelGGL(split_qk8_kernel<T>, stride_grid(rows * heads * np * 4), dim3(256), 0, st, src, ld, c0, dst,
                       rows, n, np, heads, mul);
  else
    hipLaunchKernelGGL(split_qk_kernel<T>, stride_grid(rows * heads * np * 32), dim3(256), 0, st, src, ld, c0, dst,
                       rows, n, np, heads, mul);
}
template <typename T>
void launch_split_vt(const T* src, int64_t ld, int64_t c0, T* dst, int64_t rows, int64_t n, int64_t np, int hd_total,
                     hipStream_t st) {
  const int64_t blocks = rows * ((np + 63) / 64) * ((hd_total + 63) / 64);
  hipLaunchKernelGGL(split_vt_tiled_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, st, src, ld, c0, dst, n, np,
                     hd_total);
}
template <typename T>
void launch_bias_planes(const T* src, int64_t ld, int64_t c0, T* dst, int64_t batch, int64_t n, int64_t np, int heads,
                        hipStream_t st) {
  hipLaunchKernelGGL(bias_planes_kernel<T>, stride_grid(batch * heads * np * np), dim3(256), 0, st, src, ld, c0, dst,
                     batch, n, np, heads);
}
template <typename T>
void launch_grid_mask_bias(const T* mask, float* mb, int64_t batch, int64_t n, int64_t np, float inf, int t,
                           hipStream_t st) {
  hipLaunchKernelGGL(grid_mask_bias_kernel<T>, stride_grid(batch * n * np), dim3(256), 0, st, mask, mb, batch, n, np,
                     inf, t);
}
template <typename T>
void launch_gate_rows(T* o, const T* g, int64_t ldg, int64_t c0, int64_t rows, int width, hipStream_t st) {
  if (width % 8 == 0 && ldg % 8 == 0 && c0 % 8 == 0 && al16(o) && al16(g))
    hipLaunchKernelGGL(gate_rows8_kernel<T>, stride_grid(rows * width / 8), dim3(256), 0, st, o, g, ldg, c0, rows,
                       width);
  else
    hipLaunchKernelGGL(gate_rows_kernel<T>, stride_grid(rows * width), dim3(256), 0, st, o, g, ldg, c0, rows, width);
}
template <typename T>
void launch_scatter_add(const T* y, const T* row_mask, const T* residual, const T* out_mask, T* out, int64_t rows,
                        int64_t n, int c, int t, hipStream_t st, int splits, int64_t split_stride) {
  if (c % 8 == 0 && split_stride % 8 == 0 && al16(y) && al16(out) && (!residual || al16(residual)))
    hipLaunchKernelGGL(scatter_add8_kernel<T>, stride_grid(rows * c / 8), dim3(256), 0, st, y, row_mask, residual,
                       out_mask, out, rows, n, c, t, splits, split_stride);
  else
    hipLaunchKernelGGL(scatter_add_kernel<T>, stride_grid(rows * c), dim3(256), 0, st, y, row_mask, residual, out_mask,
                       out, rows, n, c, t, splits, split_stride);
}

#define FJX_INST(T)                                                                                                \
  template void launch_ln_grid<T>(const T*, const T*, const T*, T*, int64_t, int64_t, int, float, int, hipStream_t); \
  template void launch_to_channel_major<T>(const T*, int64_t, int, int, const T*, T*, int64_t, int64_t, int,        \
                                           hipStream_t);                                                           \
  template void launch_to_position_major<T>(const T*, int, T*, int64_t, int64_t, hipStream_t);                    \
  template void launch_split_qk<T>(const T*, int64_t, int64_t, T*, int64_t, int64_t, int64_t, int, float,           \
                                   hipStream_t);                                                                   \
  template void launch_split_vt<T>(const T*, int64_t, int64_t, T*, int64_t, int64_t, int64_t, int, hipStream_t);   \
  template void launch_bias_planes<T>(const T*, int64_t, int64_t, T*, int64_t, int64_t, int64_t, int, hipStream_t); \
  template void launch_grid_mask_bias<T>(const T*, float*, int64_t, int64_t, int64_t, float, int, hipStream_t);     \
  template void launch_gate_rows<T>(T*, const T*, int64_t, int64_t, int64_t, int, hipStream_t);                      \
  template void launch_scatter_add<T>(const T*, const T*, const T*, const T*, T*, int64_t, int64_t, int, int,     \
                                      hipStream_t, int, int64_t);
FJX_INST(float)
FJX_INST(bf16)
#undef FJX_INST

}  // namespace fjx
