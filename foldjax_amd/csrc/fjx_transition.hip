// Fused transition: y = (silu(LN(x) Wa^T) * (LN(x) Wb^T)) Wo^T [* row_mask] [+ residual]
// for rows of C channels with a 4C hidden width (Boltz-2 transition_forward,
// Protenix transition, OpenFold3 swiglu_transition).
//
// One 256-thread workgroup owns 64 rows. The LayerNormed rows stay in LDS; the
// hidden width is walked in chunks of 128: each wave forms 32 hidden columns
// of a and b for all 64 rows on MFMA, writes silu(a)*b to an LDS chunk, and
// after a barrier every wave accumulates that chunk into its C/4 output
// columns. The [rows, 4C] hidden tensor never reaches HBM.
#include "fjx_common.hpp"
#include "fjx_kernels.hpp"
#include "fjx_tile.hpp"

namespace fjx {

namespace {

constexpr int kRowsT = 64;
constexpr int kHC = 128;  // hidden chunk

// acc[rt][ct] += A[16rt.., k] * W[col0 + 16ct.., k]^T, k over [0, K)
template <typename T, int K, int CT, int LDA>
__device__ __forceinline__ void wave_gemm(const T (*a)[LDA], const T* __restrict__ w, int64_t ldw, int col0,
                                          f32x4 (&acc)[4][CT]) {
  const int lane = threadIdx.x & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;
#pragma unroll 2
  for (int ks = 0; ks < K / 32; ++ks) {
    typename Frag<T>::type bf[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) bf[ct] = load8(w + (int64_t)(col0 + 16 * ct + li) * ldw + 32 * ks + 8 * lg);
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const typename Frag<T>::type af = load8(&a[16 * rt + li][32 * ks + 8 * lg]);
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) mma(acc[rt][ct], af, bf[ct]);
    }
  }
}

__device__ __forceinline__ float silu(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * kLog2e)); }

}  // namespace

template <typename T, int C>
__global__ __launch_bounds__(256) void transition_kernel(TransitionParams<T> P) {
  constexpr int XLD = C + 8;
  constexpr int HLD = kHC + 8;
  constexpr int CT = C / 64;  // 16-column output tiles per wave (C/4 columns)
  __shared__ __attribute__((aligned(16))) T xs[kRowsT][XLD];
  __shared__ __attribute__((aligned(16))) T hs[kRowsT][HLD];

  const int64_t m0 = (int64_t)blockIdx.x * kRowsT;
  const int nvalid = (int)min<int64_t>(kRowsT, P.rows - m0);
  const int t = threadIdx.x;

  // LayerNorm: 4 threads per row, C/4 channels each
  {
    constexpr int PER = C / 4;
    const int p = t >> 2;
    const int c0 = (t & 3) * PER;
    float v[PER];
    if (p < nvalid) {
      const T* src = P.x + (m0 + p) * C + c0;
#pragma unroll
      for (int q = 0; q < PER / 8; ++q) to_f32x8(load8(src + 8 * q), v + 8 * q);
    } else {
#pragma unroll
      for (int e = 0; e < PER; ++e) v[e] = 0.f;
    }
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < PER; ++e) s += v[e];
    s += shfl_xor(s, 1);
    s += shfl_xor(s, 2);
    const float mean = s * (1.0f / C);
    float q2 = 0.f;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const float d = v[e] - mean;
      q2 += d * d;
    }
    q2 += shfl_xor(q2, 1);
    q2 += shfl_xor(q2, 2);
    const float rstd = __builtin_amdgcn_rsqf(q2 * (1.0f / C) + P.eps);
#pragma unroll
    for (int q = 0; q < PER / 8; ++q) {
      float w[8], b[8], o[8];
      to_f32x8(load8(P.ln_w + c0 + 8 * q), w);
      to_f32x8(load8(P.ln_b + c0 + 8 * q), b);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (v[8 * q + e] - mean) * rstd * w[e] + b[e];
      store8(&xs[p][c0 + 8 * q], pack8<T>(o));
    }
  }
  __syncthreads();

  const int wave = t >> 6;
  const int lane = t & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;

  f32x4 out[4][CT];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) out[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};

  constexpr int NCHUNK = 4 * C / kHC;
#pragma unroll 1
  for (int ch = 0; ch < NCHUNK; ++ch) {
    const int hcol0 = ch * kHC + 32 * wave;  // this wave's 32 hidden columns
    f32x4 a[4][2], b[4][2];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        a[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
        b[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    wave_gemm<T, C, 2, XLD>(xs, P.w_a, C, hcol0, a);
    wave_gemm<T, C, 2, XLD>(xs, P.w_b, C, hcol0, b);
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          hs[16 * rt + 4 * lg + q][32 * wave + 16 * ct + li] = from_f32<T>(silu(a[rt][ct][q]) * b[rt][ct][q]);
    __syncthreads();
    wave_gemm<T, kHC, CT, HLD>(hs, P.w_o + ch * kHC, 4 * C, wave * (C / 4), out);
    __syncthreads();
  }

  // stage the update (rounded to T, as the reference's projection output is)
  // in xs, then add the residual row by row with coalesced accesses
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int row = 16 * rt + 4 * lg + q;
        float y = out[rt][ct][q];
        if (P.row_mask && row < nvalid) y *= to_f32(P.row_mask[m0 + row]);
        xs[row][wave * (C / 4) + 16 * ct + li] = from_f32<T>(y);
      }
  __syncthreads();
  constexpr int CH8 = C / 8;
  for (int idx = t; idx < kRowsT * CH8; idx += 256) {
    const int p = idx / CH8;
    const int c8 = (idx % CH8) * 8;
    if (p < nvalid) {
      float y[8];
      to_f32x8(load8(&xs[p][c8]), y);
      if (P.residual) {
        float r[8];
        to_f32x8(load8(P.residual + (m0 + p) * C + c8), r);
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] += r[e];
      }
      store8(P.out + (m0 + p) * C + c8, pack8<T>(y));
    }
  }
}

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

template <typename T>
void launch_transition(const TransitionParams<T>& p, int c, hipStream_t st) {
  if (c == 128) {
    const dim3 grid((unsigned)((p.rows + tile::kTP - 1) / tile::kTP));
    hipLaunchKernelGGL(transition128_kernel<T>, grid, dim3(512), 0, st, p);
  } else {
    const dim3 grid((unsigned)((p.rows + kRowsT - 1) / kRowsT));
    hipLaunchKernelGGL((transition_kernel<T, 384>), grid, dim3(256), 0, st, p);
  }
}

template void launch_transition<bf16>(const TransitionParams<bf16>&, int, hipStream_t);
template void launch_transition<float>(const TransitionParams<float>&, int, hipStream_t);

}  // namespace fjx
