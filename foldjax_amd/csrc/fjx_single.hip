// Single-track helpers for the attention with pair bias of a Pairformer block
// (Boltz-2 attention_pair_bias_forward): row LayerNorm, head split into the
// padded flash layout, the pair-bias projection LN(z) W_z^T, the key mask
// bias and the gate-and-unpad step before the output projection.
#include "fjx_common.hpp"
#include "fjx_kernels.hpp"
#include "fjx_tile.hpp"

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

// the same for c <= 512 channels, a multiple of 8 (ln_row8)
template <typename T>
__global__ __launch_bounds__(256) void layernorm_rows8_kernel(const T* __restrict__ x, const T* __restrict__ w,
                                                              const T* __restrict__ b, T* __restrict__ y,
                                                              int64_t rows, int c, float eps) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  ln_row8<T>(x + row * c, w, b, y + row * c, c, eps, threadIdx.x & 63);
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

// bias[b][h][q][k] = log2(e) * LN(z[b,q,k,:]) . w[h,:] over the padded
// [np, np] grid, zeros outside [n, n] (the attention never reads
// uninitialised memory next to a -inf key mask). Persistent 512-thread
// workgroups over tiles of 128 keys of one query row: the LayerNormed tile
// goes to LDS, wave w multiplies row tile w (16 keys) by the [heads][128]
// weight, 16 heads per MFMA column tile, and each lane stores 4 consecutive
// keys of one head. The next tile's z rows are loaded before the current one
// is multiplied; the weight is held in registers when heads <= 16.
// z may be narrower than the bias (TZ = bf16, T = float: the fp32 single
// track of Boltz-2 over a bf16 pair tensor); the LayerNorm runs in fp32 and
// its output is stored in T, so the projection then runs at T's precision.
template <typename TZ, typename T>
__global__ __launch_bounds__(512) void pair_bias_kernel(const TZ* __restrict__ z, const T* __restrict__ ln_w,
                                                        const T* __restrict__ ln_b, const T* __restrict__ w,
                                                        T* __restrict__ bias, int64_t n, int64_t np, int heads,
                                                        float eps, int64_t ntiles) {
  using namespace tile;
  __shared__ __attribute__((aligned(16))) T xs[kTP][kLd];
  __shared__ __attribute__((aligned(16))) LnAffine ln;

  const int64_t ntx = (np + kTP - 1) / kTP;
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int p = t >> 2;
  const int nht = (heads + 15) / 16;

  auto load_heads = [&](int ht, typename Frag<T>::type (&wf)[4]) {
    const float zero[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const int h = 16 * ht + li;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) wf[ks] = h < heads ? load8(w + (int64_t)h * kC + 32 * ks + 8 * lg) : pack8<T>(zero);
  };
  typename Frag<T>::type w0[4];
  load_heads(0, w0);
  stage_ln<T>(ln_w, ln_b, ln);

  RowPart<TZ> xr;
  auto fetch = [&](int64_t tile) {
    const TileRS tl = tile_at(tile, ntx, np);
    const int64_t kk = tl.s0 + p;
    const bool valid = tl.r < n && kk < n;
    load_row_part<TZ>(valid ? z + (((int64_t)tl.b * n + tl.r) * n + kk) * kC : nullptr, xr);
  };

  int64_t tile = blockIdx.x;
  if (tile < ntiles) fetch(tile);
  __syncthreads();
  for (; tile < ntiles; tile += gridDim.x) {
    const TileRS tl = tile_at(tile, ntx, np);
    const int nstore = (int)min<int64_t>(kTP, np - tl.s0);  // a multiple of 64
    const int nreal = tl.r < n ? (int)max<int64_t>(0, min<int64_t>(kTP, n - tl.s0)) : 0;
    ln_quad<TZ>(xr, ln, eps, &xs[p][0]);
    __syncthreads();
    if (tile + gridDim.x < ntiles) fetch(tile + gridDim.x);

    const int p0 = 16 * wave + 4 * lg;  // this lane's 4 keys within the tile
#pragma unroll 1
    for (int ht = 0; ht < nht; ++ht) {
      typename Frag<T>::type wf[4];
      if (ht == 0) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) wf[ks] = w0[ks];
      } else {
        load_heads(ht, wf);
      }
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) mma(acc, load8(&xs[16 * wave + li][32 * ks + 8 * lg]), wf[ks]);
      const int h = 16 * ht + li;
      if (h < heads && p0 < nstore) {
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = p0 + q < nreal ? acc[q] * kLog2e : 0.f;
        store4f(bias + (((int64_t)tl.b * heads + h) * np + tl.r) * np + tl.s0 + p0, v);
      }
    }
    __syncthreads();  // xs is free for the next tile
  }
}

// zeros of a prepared pair bias outside the [n, n] block of each padded
// [np, np] plane: rows r < n, columns n .. np-1, then rows n .. np-1 whole
// (the transition's fused epilogue writes only the real positions)
template <typename T>
__global__ void pair_bias_border_kernel(T* __restrict__ bias, int64_t planes, int64_t n, int64_t np) {
  const int64_t w = np - n;
  const int64_t per = n * w + w * np;
  const int64_t total = planes * per;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t plane = idx / per;
    int64_t j = idx - plane * per;
    int64_t r, c;
    if (j < n * w) {
      r = j / w;
      c = n + (j - r * w);
    } else {
      j -= n * w;
      r = n + j / np;
      c = j - (r - n) * np;
    }
    bias[(plane * np + r) * np + c] = from_f32<T>(0.f);
  }
}

// an additive attention bias given by the caller (Protenix's extra_attn_bias),
// broadcast over batch (sb = 0) and heads (sh = 0), added in fp32 to the
// projected bias: bias = src + log2(e) * extra over the real [n, n] block.
// src is a prepared bias (read-only) or bias itself.
template <typename T>
__global__ void add_extra_bias_kernel(const T* __restrict__ src, T* __restrict__ bias, const T* __restrict__ extra,
                                      int64_t sb, int64_t sh, int64_t batch, int heads, int64_t n, int64_t np) {
  const int64_t total = batch * heads * n * n;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t k = idx % n;
    const int64_t q = (idx / n) % n;
    const int64_t h = (idx / (n * n)) % heads;
    const int64_t b = idx / (n * n * heads);
    const int64_t at = ((b * heads + h) * np + q) * np + k;
    const float e = to_f32(extra[b * sb + h * sh + q * n + k]);
    bias[at] = from_f32<T>(to_f32(src[at]) + e * kLog2e);
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
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (c % 8 == 0 && c <= 512 && al16(x) && al16(w) && al16(b) && al16(y))
    hipLaunchKernelGGL(layernorm_rows8_kernel<T>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, x, w, b, y, rows,
                       c, eps);
  else
    hipLaunchKernelGGL(layernorm_rows_kernel<T>, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, x, w, b, y, rows,
                       c, eps);
}
template <typename T>
void launch_split_heads(const T* qkv, int64_t ld, int64_t batch, int64_t n, int64_t np, int heads, int dh,
                        float q_mul, T* q, T* k, T* vt, hipStream_t st) {
  hipLaunchKernelGGL(split_heads_kernel<T>, grid_stride(batch * heads * np * 32), dim3(256), 0, st, qkv, ld, batch, n,
                     np, heads, dh, q_mul, q, k, vt);
}
template <typename TZ, typename T>
void launch_pair_bias(const TZ* z, const T* ln_w, const T* ln_b, const T* w, T* bias, int64_t batch, int64_t n,
                      int64_t np, int heads, float eps, hipStream_t st) {
  const int64_t ntiles = (np + tile::kTP - 1) / tile::kTP * np * batch;
  const unsigned grid =
      tile::persistent_grid(reinterpret_cast<const void*>(&pair_bias_kernel<TZ, T>), 512, ntiles);
  hipLaunchKernelGGL((pair_bias_kernel<TZ, T>), dim3(grid), dim3(512), 0, st, z, ln_w, ln_b, w, bias, n, np, heads,
                     eps, ntiles);
}
template <typename T>
void launch_add_extra_bias(const T* src, T* bias, const T* extra, int64_t sb, int64_t sh, int64_t batch, int heads,
                           int64_t n, int64_t np, hipStream_t st) {
  hipLaunchKernelGGL(add_extra_bias_kernel<T>, grid_stride(batch * heads * n * n), dim3(256), 0, st, src ? src : bias,
                     bias, extra, sb, sh, batch, heads, n, np);
}
template <typename T>
void launch_pair_bias_border(T* bias, int64_t planes, int64_t n, int64_t np, hipStream_t st) {
  if (np == n) return;
  hipLaunchKernelGGL(pair_bias_border_kernel<T>, grid_stride(planes * (n * (np - n) + (np - n) * np)), dim3(256), 0,
                     st, bias, planes, n, np);
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
  template void launch_pair_bias<T, T>(const T*, const T*, const T*, const T*, T*, int64_t, int64_t, int64_t, int, \
                                       float, hipStream_t);                                                      \
  template void launch_add_extra_bias<T>(const T*, T*, const T*, int64_t, int64_t, int64_t, int, int64_t, int64_t,  \
                                         hipStream_t);                                                           \
  template void launch_pair_bias_border<T>(T*, int64_t, int64_t, int64_t, hipStream_t);                        \
  template void launch_key_mask<T>(const T*, float*, int64_t, int64_t, int64_t, float, hipStream_t);             \
  template void launch_gate_unpad<T>(const T*, const T*, int64_t, T*, int64_t, int, int, hipStream_t);
FJX_INST(bf16)
FJX_INST(float)
#undef FJX_INST
template void launch_pair_bias<bf16, float>(const bf16*, const float*, const float*, const float*, float*, int64_t,
                                            int64_t, int64_t, int, float, hipStream_t);
template void launch_pair_bias<float, bf16>(const float*, const bf16*, const bf16*, const bf16*, bf16*, int64_t,
                                            int64_t, int64_t, int, float, hipStream_t);

}  // namespace fjx
