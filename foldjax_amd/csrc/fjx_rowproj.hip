// LayerNorm + projection prologues and the projection epilogue of the
// triangle ops, on MFMA.
//
// All three kernels work on tiles of 64 pair positions (one "row" r of the
// pair grid, 64 consecutive columns s0..s0+63) with 256 threads (4 waves).
// Prologues address the pair tensor through a *virtual* grid: virtual (r, s)
// reads x[b, r, s] or, when transposed, x[b, s, r]. The incoming tri-mul and
// the ending-node tri-attn run entirely in that transposed virtual grid, so
// no transposed copy of x is ever written.
//
// Weights are PyTorch [out][in] row-major: output channel o is the contiguous
// row W[o][0..127], which is exactly the MFMA B fragment (8 contiguous k for
// one output column) and is read straight from L2.
#include "fjx_common.hpp"
#include "fjx_kernels.hpp"

namespace fjx {

constexpr int kTile = 64;        // positions per workgroup
constexpr int kC = 128;          // channels handled by these kernels
constexpr int kXPad = 8;         // LDS row padding (elements) for the [pos][ch] tile
constexpr int kYPad = 8;         // LDS padding for the [ch][pos] staging tile

// ---------------------------------------------------------------------------
// Stage 1 shared by the prologues: load 64 positions x 128 channels, LayerNorm
// in fp32, write the normalised (and affine-transformed) rows to LDS as T.
// Thread t owns position t/4 and channels [32*(t%4), +32).
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void ln_tile_to_lds(const T* __restrict__ x, int64_t row_off,
                                               bool valid, const T* __restrict__ ln_w,
                                               const T* __restrict__ ln_b, float eps,
                                               T (*xs)[kC + kXPad]) {
  const int t = threadIdx.x;
  const int p = t >> 2;
  const int c0 = (t & 3) * 32;
  float v[32];
  if (valid) {
    const T* src = x + row_off + c0;
#pragma unroll
    for (int q = 0; q < 4; ++q) to_f32x8(load8(src + 8 * q), v + 8 * q);
  } else {
#pragma unroll
    for (int e = 0; e < 32; ++e) v[e] = 0.f;
  }
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 32; ++e) s += v[e];
  s += shfl_xor(s, 1);
  s += shfl_xor(s, 2);
  const float mean = s * (1.0f / kC);
  float q2 = 0.f;
#pragma unroll
  for (int e = 0; e < 32; ++e) {
    const float d = v[e] - mean;
    q2 += d * d;
  }
  q2 += shfl_xor(q2, 1);
  q2 += shfl_xor(q2, 2);
  const float rstd = __builtin_amdgcn_rsqf(q2 * (1.0f / kC) + eps);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float w[8], b[8], o[8];
    to_f32x8(load8(ln_w + c0 + 8 * q), w);
    to_f32x8(load8(ln_b + c0 + 8 * q), b);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (v[8 * q + e] - mean) * rstd * w[e] + b[e];
    store8(&xs[p][c0 + 8 * q], pack8<T>(o));
  }
}

// One wave: acc[rt][ct] += X[16rt.., :] * W[col0 + 16ct.., :]^T over K = 128.
template <typename T>
__device__ __forceinline__ void wave_gemm_64x32(const T (*xs)[kC + kXPad], const T* __restrict__ w,
                                                int col0, f32x4 (&acc)[4][2]) {
  const int lane = threadIdx.x & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) acc[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < kC / 32; ++ks) {
    typename Frag<T>::type bf[2];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
      bf[ct] = load8(w + (int64_t)(col0 + 16 * ct + li) * kC + 32 * ks + 8 * lg);
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const typename Frag<T>::type af = load8(&xs[16 * rt + li][32 * ks + 8 * lg]);
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) mma(acc[rt][ct], af, bf[ct]);
    }
  }
}

// Copy a channel-major LDS tile ys[ch][pos] (64 positions) to dst[ch * ch_stride + pos],
// positions [0, nvalid) of the tile; when `pad_to` > nvalid, positions
// [nvalid, pad_to) are written with `fill`.
template <typename T>
__device__ __forceinline__ void store_cm_tile(const T (*ys)[kTile + kYPad], T* __restrict__ dst,
                                              int64_t ch_stride, int nvalid, int pad_to, bool aligned,
                                              float fill) {
  const int t = threadIdx.x;
  const int limit = pad_to > nvalid ? pad_to : nvalid;
  // 128 channels x 8 chunks of 8 positions = 1024 chunks, 4 per thread
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int idx = t + 256 * it;
    const int ch = idx >> 3;
    const int p0 = (idx & 7) * 8;
    T* d = dst + (int64_t)ch * ch_stride + p0;
    if (aligned && p0 + 8 <= nvalid) {
      store8(d, load8(&ys[ch][p0]));
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int p = p0 + e;
        if (p < nvalid) d[e] = ys[ch][p];
        else if (p < limit) d[e] = from_f32<T>(fill);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Triangle multiplication prologue.
//   a_cm/b_cm: [B][c_h][N*N] channel-major in the virtual grid (contraction
//   operands with the contracted axis contiguous); g: [B][N*N][c_z]
//   position-major in the original grid, holding sigmoid(x_ln g_out^T).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void trimul_prologue_kernel(TriMulPrologueParams<T> P) {
  __shared__ __attribute__((aligned(16))) T xs[kTile][kC + kXPad];
  __shared__ __attribute__((aligned(16))) T ys[kC][kTile + kYPad];
  __shared__ float mrow[kTile];

  const int64_t n = P.n;
  const int r = blockIdx.y;
  const int s0 = blockIdx.x * kTile;
  const int b = blockIdx.z;
  const int t = threadIdx.x;
  const int nvalid = (int)min<int64_t>(kTile, n - s0);
  const int64_t nn = n * n;

  {
    const int p = t >> 2;
    const int s = s0 + p;
    const bool valid = s < n;
    const int64_t orig = P.transpose ? (int64_t)s * n + r : (int64_t)r * n + s;
    const int64_t off = ((int64_t)b * nn + (valid ? orig : 0)) * kC;
    ln_tile_to_lds<T>(P.x, off, valid, P.ln_w, P.ln_b, P.eps, xs);
    if ((t & 3) == 0) {
      float m = 0.f;
      if (valid) m = P.mask ? to_f32(P.mask[(int64_t)b * nn + orig]) : 1.0f;
      mrow[p] = m;
    }
  }
  __syncthreads();

  const int wave = t >> 6;
  const int lane = t & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int col0 = 32 * wave;
  const bool aligned = (n % 8) == 0;

  // a then b: gated projections, channel-major stores
#pragma unroll 1
  for (int half = 0; half < 2; ++half) {
    f32x4 accp[4][2], accg[4][2];
    wave_gemm_64x32<T>(xs, P.w_p + (int64_t)half * kC * kC, col0, accp);
    wave_gemm_64x32<T>(xs, P.w_g + (int64_t)half * kC * kC, col0, accg);
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int row = 16 * rt + 4 * lg + q;
          const int col = col0 + 16 * ct + li;
          const float val = mrow[row] * fast_sigmoid(accg[rt][ct][q]) * accp[rt][ct][q];
          ys[col][row] = from_f32<T>(val);
        }
    __syncthreads();
    T* dst = (half == 0 ? P.a_cm : P.b_cm) + (int64_t)b * kC * nn + (int64_t)r * n + s0;
    store_cm_tile<T>(ys, dst, nn, nvalid, nvalid, aligned, 0.f);
    __syncthreads();
  }

  // output gate sigmoid(x_ln g_out^T), position-major in the original grid
  {
    f32x4 acc[4][2];
    wave_gemm_64x32<T>(xs, P.w_gout, col0, acc);
    // reuse ys as a [pos][ch] tile: 64 x 128 fits in 128 x 72
    T(*yp)[kC + kXPad] = reinterpret_cast<T(*)[kC + kXPad]>(&ys[0][0]);
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          yp[16 * rt + 4 * lg + q][col0 + 16 * ct + li] = from_f32<T>(fast_sigmoid(acc[rt][ct][q]));
    __syncthreads();
    // 64 positions x 16 chunks of 8 channels = 1024 chunks, 4 per thread
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int idx = t + 256 * it;
      const int p = idx >> 4;
      const int c8 = (idx & 15) * 8;
      const int s = s0 + p;
      if (s < n) {
        const int64_t orig = P.transpose ? (int64_t)s * n + r : (int64_t)r * n + s;
        store8(P.g + ((int64_t)b * nn + orig) * kC + c8, load8(&yp[p][c8]));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Triangle attention prologue (virtual grid, transposed for the ending node).
//   q  [B][N][H][Np][D]  q_ln * (scale*log2 e)
//   k  [B][N][H][Np][D]
//   vt [B][N][H*D][Np]   v transposed so that keys are contiguous
//   g  [B][N][N][H*D]    sigmoid(x_ln w_g^T), or absent
//   bias [B][H][Np][Np]  x_ln w_bias^T times log2 e (in T)
//   mb [B][N][Np] fp32   inf*(mask-1)*log2 e, -inf for keys >= N
// Np = N rounded up to 64; padded key slots of q/k/vt are written as zeros.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void triattn_prologue_kernel(TriAttnPrologueParams<T> P) {
  __shared__ __attribute__((aligned(16))) T xs[kTile][kC + kXPad];
  __shared__ __attribute__((aligned(16))) T ys[kC][kTile + kYPad];

  const int64_t n = P.n;
  const int64_t np = P.np;
  const int r = blockIdx.y;
  const int s0 = blockIdx.x * kTile;
  const int b = blockIdx.z;
  const int t = threadIdx.x;
  const int nvalid = (int)max<int64_t>(0, min<int64_t>(kTile, n - s0));
  const int64_t nn = n * n;
  constexpr int D = 32;
  constexpr int H = 4;

  {
    const int p = t >> 2;
    const int s = s0 + p;
    const bool valid = s < n;
    const int64_t orig = P.transpose ? (int64_t)s * n + r : (int64_t)r * n + s;
    const int64_t off = ((int64_t)b * nn + (valid ? orig : 0)) * kC;
    ln_tile_to_lds<T>(P.x, off, valid, P.ln_w, P.ln_b, P.eps, xs);
    if ((t & 3) == 0) {
      float mbv = -INFINITY;
      if (valid) {
        const float m = P.mask ? to_f32(P.mask[(int64_t)b * nn + orig]) : 1.0f;
        mbv = P.inf * (m - 1.0f) * kLog2e;
      }
      P.mb[((int64_t)b * n + r) * np + s] = mbv;
    }
  }
  __syncthreads();

  // triangle bias: 64 positions x 4 heads, one dot product of length 128 per thread
  {
    const int p = t >> 2;
    const int h = t & 3;
    const int s = s0 + p;
    if (s < np) {
      float acc = 0.f;
      if (s < n) {
        const T* wrow = P.w_bias + h * kC;
#pragma unroll 4
        for (int c = 0; c < kC; c += 8) {
          float xv[8], wv[8];
          to_f32x8(load8(&xs[p][c]), xv);
          to_f32x8(load8(wrow + c), wv);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc += xv[e] * wv[e];
        }
      }
      P.bias[(((int64_t)b * H + h) * np + r) * np + s] = from_f32<T>(acc * kLog2e);
    }
  }

  const int wave = t >> 6;
  const int lane = t & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int col0 = 32 * wave;
  const int nstore = (int)min<int64_t>(kTile, np - s0);  // positions incl. zero padding
  T(*yp)[kC + kXPad] = reinterpret_cast<T(*)[kC + kXPad]>(&ys[0][0]);

  // q and k: [pos][ch] staging, per-head contiguous blocks of 64 x 32
#pragma unroll 1
  for (int which = 0; which < 2; ++which) {
    f32x4 acc[4][2];
    wave_gemm_64x32<T>(xs, which == 0 ? P.w_q : P.w_k, col0, acc);
    const float sc = which == 0 ? P.q_scale : 1.0f;
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int row = 16 * rt + 4 * lg + q;
          const float val = (s0 + row < n) ? acc[rt][ct][q] * sc : 0.f;
          yp[row][col0 + 16 * ct + li] = from_f32<T>(val);
        }
    __syncthreads();
    T* base = (which == 0 ? P.q : P.k) + ((int64_t)b * n + r) * H * np * D;
    // 64 positions x 4 heads x 4 chunks of 8 = 1024 chunks
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int idx = t + 256 * it;
      const int p = idx >> 4;
      const int h = (idx >> 2) & 3;
      const int d8 = (idx & 3) * 8;
      if (p < nstore) store8(base + ((int64_t)h * np + s0 + p) * D + d8, load8(&yp[p][h * D + d8]));
    }
    __syncthreads();
  }

  // v: channel-major staging -> vt[b][r][ch][s]
  {
    f32x4 acc[4][2];
    wave_gemm_64x32<T>(xs, P.w_v, col0, acc);
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int row = 16 * rt + 4 * lg + q;
          ys[col0 + 16 * ct + li][row] = from_f32<T>(s0 + row < n ? acc[rt][ct][q] : 0.f);
        }
    __syncthreads();
    T* dst = P.vt + ((int64_t)b * n + r) * kC * np + s0;
    store_cm_tile<T>(ys, dst, np, nstore, nstore, true, 0.f);
    __syncthreads();
  }

  // gate: sigmoid, position-major in the virtual grid
  if (P.w_g) {
    f32x4 acc[4][2];
    wave_gemm_64x32<T>(xs, P.w_g, col0, acc);
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          yp[16 * rt + 4 * lg + q][col0 + 16 * ct + li] = from_f32<T>(fast_sigmoid(acc[rt][ct][q]));
    __syncthreads();
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int idx = t + 256 * it;
      const int p = idx >> 4;
      const int c8 = (idx & 15) * 8;
      if (p < nvalid) store8(P.g + (((int64_t)b * n + r) * n + s0 + p) * kC + c8, load8(&yp[p][c8]));
    }
  }
}

// ---------------------------------------------------------------------------
// Epilogue: y = [LN](X) W^T [* gate] [+ residual], 128 -> 128 channels.
//   X is channel-major ([B][128][N*N], tri-mul contraction output) or
//   position-major ([B][N*N][128], gated attention output) in the virtual grid
//   rows r, columns s; the result goes to out[b, r, s] or, transposed,
//   out[b, s, r]. gate and residual are read at the output position.
// ---------------------------------------------------------------------------
template <typename T, bool kChannelMajor, bool kLN>
__global__ __launch_bounds__(256) void rowgemm_epilogue_kernel(EpilogueParams<T> P) {
  __shared__ __attribute__((aligned(16))) T xs[kTile][kC + kXPad];
  __shared__ __attribute__((aligned(16))) float yf[kTile][kC + 4];

  const int64_t n = P.n;
  const int r = blockIdx.y;
  const int s0 = blockIdx.x * kTile;
  const int b = blockIdx.z;
  const int t = threadIdx.x;
  const int nvalid = (int)min<int64_t>(kTile, n - s0);
  const int64_t nn = n * n;
  const int64_t vrow = (int64_t)r * n + s0;  // flat virtual index of the tile's first position

  if (kChannelMajor) {
    const T* src = P.x + (int64_t)b * kC * nn + vrow;
    const bool aligned = (n % 8) == 0;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int idx = t + 256 * it;
      const int ch = idx >> 3;
      const int p0 = (idx & 7) * 8;
      float v[8];
      if (aligned && p0 + 8 <= nvalid) {
        to_f32x8(load8(src + (int64_t)ch * nn + p0), v);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (p0 + e < nvalid) ? to_f32(src[(int64_t)ch * nn + p0 + e]) : 0.f;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) xs[p0 + e][ch] = from_f32<T>(v[e]);
    }
  } else {
    const T* src = P.x + ((int64_t)b * nn + vrow) * kC;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int idx = t + 256 * it;
      const int p = idx >> 4;
      const int c8 = (idx & 15) * 8;
      if (p < nvalid) store8(&xs[p][c8], load8(src + (int64_t)p * kC + c8));
      else {
        const float zero[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        store8(&xs[p][c8], pack8<T>(zero));
      }
    }
  }
  __syncthreads();

  if (kLN) {
    const int p = t >> 2;
    const int c0 = (t & 3) * 32;
    float v[32];
#pragma unroll
    for (int q = 0; q < 4; ++q) to_f32x8(load8(&xs[p][c0 + 8 * q]), v + 8 * q);
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 32; ++e) s += v[e];
    s += shfl_xor(s, 1);
    s += shfl_xor(s, 2);
    const float mean = s * (1.0f / kC);
    float q2 = 0.f;
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      const float d = v[e] - mean;
      q2 += d * d;
    }
    q2 += shfl_xor(q2, 1);
    q2 += shfl_xor(q2, 2);
    const float rstd = __builtin_amdgcn_rsqf(q2 * (1.0f / kC) + P.eps);
    // every thread of the quad has read its row before anyone rewrites it
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float w[8], bb[8], o[8];
      to_f32x8(load8(P.ln_w + c0 + 8 * q), w);
      to_f32x8(load8(P.ln_b + c0 + 8 * q), bb);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (v[8 * q + e] - mean) * rstd * w[e] + bb[e];
      store8(&xs[p][c0 + 8 * q], pack8<T>(o));
    }
    __syncthreads();
  }

  const int wave = t >> 6;
  const int lane = t & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int col0 = 32 * wave;
  f32x4 acc[4][2];
  wave_gemm_64x32<T>(xs, P.w, col0, acc);
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
      for (int q = 0; q < 4; ++q) yf[16 * rt + 4 * lg + q][col0 + 16 * ct + li] = acc[rt][ct][q];
  __syncthreads();

#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int idx = t + 256 * it;
    const int p = idx >> 4;
    const int c8 = (idx & 15) * 8;
    const int s = s0 + p;
    if (s < n) {
      const int64_t orig = P.transpose ? (int64_t)s * n + r : (int64_t)r * n + s;
      const int64_t off = ((int64_t)b * nn + orig) * kC + c8;
      float y[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = yf[p][c8 + e];
      if (P.gate) {
        float g[8];
        to_f32x8(load8(P.gate + off), g);
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] *= g[e];
      }
      if (P.residual) {
        float rv[8];
        to_f32x8(load8(P.residual + off), rv);
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] += rv[e];
      }
      store8(P.out + off, pack8<T>(y));
    }
  }
}

// ---------------------------------------------------------------------------
// host-side launchers
// ---------------------------------------------------------------------------
template <typename T>
void launch_trimul_prologue(const TriMulPrologueParams<T>& p, int64_t batch, hipStream_t st) {
  dim3 grid((unsigned)((p.n + kTile - 1) / kTile), (unsigned)p.n, (unsigned)batch);
  hipLaunchKernelGGL(trimul_prologue_kernel<T>, grid, dim3(256), 0, st, p);
}
template <typename T>
void launch_triattn_prologue(const TriAttnPrologueParams<T>& p, int64_t batch, hipStream_t st) {
  dim3 grid((unsigned)(p.np / kTile), (unsigned)p.n, (unsigned)batch);
  hipLaunchKernelGGL(triattn_prologue_kernel<T>, grid, dim3(256), 0, st, p);
}
template <typename T>
void launch_epilogue(const EpilogueParams<T>& p, bool channel_major, bool ln, int64_t batch, hipStream_t st) {
  dim3 grid((unsigned)((p.n + kTile - 1) / kTile), (unsigned)p.n, (unsigned)batch);
  if (channel_major && ln)
    hipLaunchKernelGGL((rowgemm_epilogue_kernel<T, true, true>), grid, dim3(256), 0, st, p);
  else if (!channel_major && !ln)
    hipLaunchKernelGGL((rowgemm_epilogue_kernel<T, false, false>), grid, dim3(256), 0, st, p);
  else if (channel_major)
    hipLaunchKernelGGL((rowgemm_epilogue_kernel<T, true, false>), grid, dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((rowgemm_epilogue_kernel<T, false, true>), grid, dim3(256), 0, st, p);
}

template void launch_trimul_prologue<float>(const TriMulPrologueParams<float>&, int64_t, hipStream_t);
template void launch_trimul_prologue<bf16>(const TriMulPrologueParams<bf16>&, int64_t, hipStream_t);
template void launch_triattn_prologue<float>(const TriAttnPrologueParams<float>&, int64_t, hipStream_t);
template void launch_triattn_prologue<bf16>(const TriAttnPrologueParams<bf16>&, int64_t, hipStream_t);
template void launch_epilogue<float>(const EpilogueParams<float>&, bool, bool, int64_t, hipStream_t);
template void launch_epilogue<bf16>(const EpilogueParams<bf16>&, bool, bool, int64_t, hipStream_t);

}  // namespace fjx
