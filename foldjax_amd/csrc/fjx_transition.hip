// Fused transition: y = (silu(LN(x) Wa^T) * (LN(x) Wb^T)) Wo^T [* row_mask] [+ residual]
// for rows of C channels with a 4C hidden width (Boltz-2 transition_forward,
// Protenix transition, OpenFold3 swiglu_transition).
//
// A workgroup owns a tile of rows. The LayerNormed rows stay in LDS; the
// hidden width is walked in chunks of 128: each wave forms 16 hidden columns
// of a and b for the tile's rows on MFMA, writes silu(a)*b to an LDS chunk,
// and after a barrier every wave accumulates that chunk into its share of the
// output channels. The [rows, 4C] hidden tensor never reaches HBM.
#include "fjx_common.hpp"
#include "fjx_kernels.hpp"
#include "fjx_tile.hpp"

namespace fjx {

namespace {

__device__ __forceinline__ float silu(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * kLog2e)); }

}  // namespace

// ---------------------------------------------------------------------------
// Pair-track transition (C = 128, hidden 512): 128-row tiles, 512 threads.
// Wave w owns hidden columns 16w .. 16w+15 of every 128-wide hidden chunk and
// output channels 16w .. 16w+15, so per chunk it holds just three 16-column
// weight tiles (W_a, W_b rows of its hidden columns, W_o rows of its output
// channels) in registers while the 8 row tiles of 16 stream past. Both
// products use the transposed accumulator form (a lane holds 4 consecutive
// columns of one row), so silu(a)*b and the output go out 8 bytes per lane.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(512) void transition128_kernel(TransitionParams<T> P) {
  using namespace tile;
  __shared__ __attribute__((aligned(16))) T xs[kTP][kLd];  // LN(x)
  __shared__ __attribute__((aligned(16))) T hs[kTP][kLd];  // silu(a) * b, one hidden chunk
  __shared__ __attribute__((aligned(16))) LnAffine ln;

  const int64_t m0 = (int64_t)blockIdx.x * kTP;
  const int nvalid = (int)min<int64_t>(kTP, P.rows - m0);
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const int p = t >> 2;
  const int col = 16 * wave;

  {
    RowPart<T> xr;
    load_row_part<T>(p < nvalid ? P.x + (m0 + p) * kC : nullptr, xr);
    stage_ln<T>(P.ln_w, P.ln_b, ln);
    __syncthreads();
    ln_quad<T>(xr, ln, P.eps, &xs[p][0]);
  }
  __syncthreads();

  f32x4 out[8];
#pragma unroll
  for (int rt = 0; rt < 8; ++rt) out[rt] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll 1
  for (int ch = 0; ch < 4; ++ch) {
    WCol<T> wa, wb, wo;
    load_wcol<T>(P.w_a, kC, ch * kC + col, 0, wa);
    load_wcol<T>(P.w_b, kC, ch * kC + col, 0, wb);
    load_wcol<T>(P.w_o, 4 * kC, col, ch * kC, wo);
#pragma unroll 2
    for (int rt = 0; rt < 8; ++rt) {
      f32x4 a = f32x4{0.f, 0.f, 0.f, 0.f}, b = f32x4{0.f, 0.f, 0.f, 0.f};
      tile_mma1_acc<T>(xs, rt, wa, a);
      tile_mma1_acc<T>(xs, rt, wb, b);
      float h[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) h[q] = silu(a[q]) * b[q];
      store4f(&hs[16 * rt + (lane & 15)][col + 4 * (lane >> 4)], h);
    }
    __syncthreads();
#pragma unroll
    for (int rt = 0; rt < 8; ++rt) tile_mma1_acc<T>(hs, rt, wo, out[rt]);
    __syncthreads();  // hs is rewritten by the next chunk
  }

  // the update is rounded to T (the reference's projection output is), then
  // the residual is added
#pragma unroll
  for (int rt = 0; rt < 8; ++rt) {
    const int row = 16 * rt + (lane & 15);
    if (row < nvalid) {
      const float m = P.row_mask ? to_f32(P.row_mask[m0 + row]) : 1.0f;
      const int64_t off = (m0 + row) * kC + col + 4 * (lane >> 4);
      float y[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) y[q] = round_to<T>(out[rt][q] * m);
      if (P.residual) {
        float r[4];
        load4f(P.residual + off, r);
#pragma unroll
        for (int q = 0; q < 4; ++q) y[q] += r[q];
      }
      store4f(P.out + off, y);
    }
  }
}

// ---------------------------------------------------------------------------
// Single-track transition (C = 384, hidden 1536) over few rows (one per
// token): 16-row tiles so that even 1024 rows spread over 64 workgroups.
// 512 threads; per 128-wide hidden chunk, wave w forms hidden columns
// 16w .. 16w+15 (K = 384) and then adds the chunk's contribution to output
// channels 48w .. 48w+47. All weight fragments of a chunk are requested at
// its start, so each chunk costs about one L2 round trip.
// ---------------------------------------------------------------------------
constexpr int kC3 = 384;
constexpr int kR3 = 16;
constexpr int kLd3 = kC3 + 8;

template <typename T>
__global__ __launch_bounds__(512) void transition384_kernel(TransitionParams<T> P) {
  using tile::kLd;
  __shared__ __attribute__((aligned(16))) T xs[kR3][kLd3];  // LN(x)
  __shared__ __attribute__((aligned(16))) T hs[kR3][kLd];   // silu(a) * b, one hidden chunk

  const int64_t m0 = (int64_t)blockIdx.x * kR3;
  const int nvalid = (int)min<int64_t>(kR3, P.rows - m0);
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;

  // LayerNorm: wave w normalises rows 2w and 2w+1, 6 channels per lane
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int r = 2 * wave + k;
    float v[6];
#pragma unroll
    for (int u = 0; u < 6; ++u) v[u] = r < nvalid ? to_f32(P.x[(m0 + r) * kC3 + lane + 64 * u]) : 0.f;
    float s = 0.f;
#pragma unroll
    for (int u = 0; u < 6; ++u) s += v[u];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) s += shfl_xor(s, o);
    const float mean = s * (1.0f / kC3);
    float q2 = 0.f;
#pragma unroll
    for (int u = 0; u < 6; ++u) q2 += (v[u] - mean) * (v[u] - mean);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) q2 += shfl_xor(q2, o);
    const float rstd = __builtin_amdgcn_rsqf(q2 * (1.0f / kC3) + P.eps);
#pragma unroll
    for (int u = 0; u < 6; ++u) {
      const int c = lane + 64 * u;
      xs[r][c] = from_f32<T>((v[u] - mean) * rstd * to_f32(P.ln_w[c]) + to_f32(P.ln_b[c]));
    }
  }
  __syncthreads();

  f32x4 out[3];
#pragma unroll
  for (int ct = 0; ct < 3; ++ct) out[ct] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll 1
  for (int ch = 0; ch < 12; ++ch) {
    const int hc = ch * 128 + 16 * wave;  // this wave's hidden columns
    typename Frag<T>::type wa[12], wb[12], wo[4][3];
#pragma unroll
    for (int ks = 0; ks < 12; ++ks) {
      wa[ks] = load8(P.w_a + (int64_t)(hc + li) * kC3 + 32 * ks + 8 * lg);
      wb[ks] = load8(P.w_b + (int64_t)(hc + li) * kC3 + 32 * ks + 8 * lg);
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int ct = 0; ct < 3; ++ct)
        wo[ks][ct] = load8(P.w_o + (int64_t)(48 * wave + 16 * ct + li) * (4 * kC3) + ch * 128 + 32 * ks + 8 * lg);
    // transposed form: lane holds row l%16, hidden columns hc + 4g .. +3
    f32x4 a = f32x4{0.f, 0.f, 0.f, 0.f}, b = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 12; ++ks) {
      const typename Frag<T>::type xf = load8(&xs[li][32 * ks + 8 * lg]);
      mma(a, wa[ks], xf);
      mma(b, wb[ks], xf);
    }
    float h[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) h[q] = silu(a[q]) * b[q];
    store4f(&hs[li][16 * wave + 4 * lg], h);
    __syncthreads();
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const typename Frag<T>::type hf = load8(&hs[li][32 * ks + 8 * lg]);
#pragma unroll
      for (int ct = 0; ct < 3; ++ct) mma(out[ct], wo[ks][ct], hf);
    }
    __syncthreads();  // hs is rewritten by the next chunk
  }

  const int row = li;
  if (row < nvalid) {
    const float m = P.row_mask ? to_f32(P.row_mask[m0 + row]) : 1.0f;
#pragma unroll
    for (int ct = 0; ct < 3; ++ct) {
      const int64_t off = (m0 + row) * kC3 + 48 * wave + 16 * ct + 4 * lg;
      float y[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) y[q] = round_to<T>(out[ct][q] * m);
      if (P.residual) {
        float r[4];
        load4f(P.residual + off, r);
#pragma unroll
        for (int q = 0; q < 4; ++q) y[q] += r[q];
      }
      store4f(P.out + off, y);
    }
  }
}

template <typename T>
void launch_transition(const TransitionParams<T>& p, int c, hipStream_t st) {
  if (c == 128) {
    const dim3 grid((unsigned)((p.rows + tile::kTP - 1) / tile::kTP));
    hipLaunchKernelGGL(transition128_kernel<T>, grid, dim3(512), 0, st, p);
  } else {
    const dim3 grid((unsigned)((p.rows + kR3 - 1) / kR3));
    hipLaunchKernelGGL(transition384_kernel<T>, grid, dim3(512), 0, st, p);
  }
}

template void launch_transition<bf16>(const TransitionParams<bf16>&, int, hipStream_t);
template void launch_transition<float>(const TransitionParams<float>&, int, hipStream_t);

}  // namespace fjx
