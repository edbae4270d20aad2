// Fused transition: y = ((silu(LN(x) Wa^T) * (LN(x) Wb^T)) Wo^T [* row_mask] [+ residual]) [* (out_mask != 0)]
// for rows of C = 128 channels with a 4C hidden width (Boltz-2 transition_forward,
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

// The attention-with-pair-bias projection of the transition's output rows,
// fused so that the pair tensor is not read again: the rows (as stored, in
// T) are in xs; they are LayerNormed in place with the attention's pair norm
// and multiplied by its [heads][128] weight. Wave w owns rows 16w .. 16w+15
// of the tile, and a lane holds 4 consecutive rows (positions) of head
// l % 16, stored as bias[b][h][r][s] * log2(e).
template <typename T>
__device__ __forceinline__ void pair_bias_epilogue(const TransitionParams<T>& P, T (*xs)[tile::kLd],
                                                   const tile::LnAffine& ln, const tile::WCol<T>& wf,
                                                   int64_t m0, int nvalid) {
  using namespace tile;
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int p = t >> 2;
  __syncthreads();
  {
    RowPart<T> yr;
#pragma unroll
    for (int q = 0; q < 4; ++q) yr.f[q] = load8(&xs[p][row_chunk(q)]);
    ln_quad<T>(yr, ln, P.pb_eps, &xs[p][0]);  // each thread rewrites only the chunks it read
  }
  __syncthreads();
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) mma(acc, load8(&xs[16 * wave + li][32 * ks + 8 * lg]), wf[ks]);
  const int pos0 = 16 * wave + 4 * lg;
  if (li >= P.pb_heads || pos0 >= nvalid) return;
  const int64_t n = P.pb_n, nn = n * n, np = P.pb_np;
  float v[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) v[q] = acc[q] * kLog2e;
  if ((n & 3) == 0) {
    // rows = B n^2 is then a multiple of 16, so nvalid is too, and the 4
    // positions share (b, r) with s a multiple of 4 (aligned stores)
    const int64_t m = m0 + pos0;
    const int64_t b = m / nn, rem = m - b * nn, r = rem / n, c = rem - r * n;
    store4f(P.pb_out + ((b * P.pb_heads + li) * np + r) * np + c, v);
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (pos0 + q >= nvalid) break;
      const int64_t m = m0 + pos0 + q;
      const int64_t b = m / nn, rem = m - b * nn, r = rem / n, c = rem - r * n;
      P.pb_out[((b * P.pb_heads + li) * np + r) * np + c] = from_f32<T>(v[q]);
    }
  }
}

// The fp32 pair-bias weight split into bf16 high and low parts (16 heads x
// 128) lives in the padding columns of the two tiles, which no tile access
// touches: the high part in xs, the low part in hs. Without it in a buffer
// of its own the kernel's LDS stays within two workgroups per CU. The 16
// 8-element chunks c = k / 8 of head h sit in row 16 (c / 2) + h, padding
// half (c % 2) ^ (h / 8): with 288-byte rows the 16-byte bank group of that
// half is 2 h + ((c % 2) ^ (h / 8)) mod 16, so the 16 heads a fragment read
// gathers (one per lane row) hit 16 distinct groups (rows 8h + k/16 would
// put all 16 on one group).
static_assert(tile::kLd - tile::kC == 16 && 16 * tile::kC == 16 * tile::kTP, "the split weight fills the padding");
__device__ __forceinline__ bf16* wz_at(bf16 (*tl)[tile::kLd], int h, int k) {
  const int c = k >> 3;
  return &tl[16 * (c >> 1) + h][tile::kC + 8 * ((c & 1) ^ (h >> 3)) + (k & 7)];
}

// The same projection in fp32 for a bf16 transition (the attention runs in
// fp32 over the bf16 pair tensor): the LayerNormed rows and the fp32 weight
// are split into bf16 high and low parts, hi = bf16(v), lo = bf16(v - hi),
// and the product is taken as hi.hi + hi.lo + lo.hi on the bf16 MFMA (the
// dropped lo.lo term is below 2^-16 of the product). The high parts go to
// xs, the low parts to hs (free after the last chunk).
__device__ __forceinline__ void pair_bias_epilogue_f32(const TransitionParams<bf16>& P, bf16 (*xs)[tile::kLd],
                                                       bf16 (*hs)[tile::kLd], const tile::LnAffine& ln, int64_t m0,
                                                       int nvalid) {
  using namespace tile;
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int p = t >> 2;
  // the weight rows of head l % 16, split hi + lo at the kernel's start
  // (stage_wz_split; zero past pb_heads)
  WCol<bf16> whi, wlo;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    whi[ks] = load8(wz_at(xs, li, 32 * ks + 8 * lg));
    wlo[ks] = load8(wz_at(hs, li, 32 * ks + 8 * lg));
  }
  __syncthreads();
  {
    RowPart<bf16> yr;
#pragma unroll
    for (int q = 0; q < 4; ++q) yr.f[q] = load8(&xs[p][row_chunk(q)]);
    ln_quad_put(yr, ln, P.pb_eps, [&](int c, const float* o) {  // each thread rewrites only the chunks it read
      float hi[8], lo[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        hi[e] = round_to<bf16>(o[e]);
        lo[e] = o[e] - hi[e];
      }
      store8(&xs[p][c], pack8<bf16>(hi));
      store8(&hs[p][c], pack8<bf16>(lo));
    });
  }
  __syncthreads();
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const bf16x8 xh = load8(&xs[16 * wave + li][32 * ks + 8 * lg]);
    const bf16x8 xl = load8(&hs[16 * wave + li][32 * ks + 8 * lg]);
    mma(acc, xh, whi[ks]);
    mma(acc, xh, wlo[ks]);
    mma(acc, xl, whi[ks]);
  }
  const int pos0 = 16 * wave + 4 * lg;
  if (li >= P.pb_heads || pos0 >= nvalid) return;
  const int64_t n = P.pb_n, nn = n * n, np = P.pb_np;
  float v[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) v[q] = acc[q] * kLog2e;
  if ((n & 3) == 0) {
    const int64_t m = m0 + pos0;
    const int64_t b = m / nn, rem = m - b * nn, r = rem / n, c = rem - r * n;
    store4f(P.pbf_out + ((b * P.pb_heads + li) * np + r) * np + c, v);
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (pos0 + q >= nvalid) break;
      const int64_t m = m0 + pos0 + q;
      const int64_t b = m / nn, rem = m - b * nn, r = rem / n, c = rem - r * n;
      P.pbf_out[((b * P.pb_heads + li) * np + r) * np + c] = v[q];
    }
  }
}

// The fp32 pair-bias weight [heads][128], split once per workgroup into
// bf16 high and low parts (hi = bf16(w), lo = bf16(w - hi)) in LDS, rows past
// pb_heads zero (wz_at: the padding columns of xs and hs): the epilogue then
// reads its fragments from LDS instead of waiting, at the end of the tile,
// for global loads and the split. In two halves like ln_fetch / ln_put: one
// unconditional load per thread (512 threads x 4 weights = 16 x 128; heads
// past pb_heads read the last one), then the split and the LDS writes.
__device__ __forceinline__ f32x4 wz_fetch(const TransitionParams<bf16>& P) {
  const int t = threadIdx.x;
  const int h = min(t >> 5, P.pb_heads - 1);
  return *reinterpret_cast<const f32x4*>(P.pbf_w + (int64_t)h * tile::kC + 4 * (t & 31));
}
__device__ __forceinline__ void wz_put(const TransitionParams<bf16>& P, f32x4 w, bf16 (*xs)[tile::kLd],
                                       bf16 (*hs)[tile::kLd]) {
  const int t = threadIdx.x;
  const int h = t >> 5;
  const int k0 = 4 * (t & 31);
  float hi[4], lo[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float v = h < P.pb_heads ? w[e] : 0.f;
    hi[e] = round_to<bf16>(v);
    lo[e] = v - hi[e];
  }
  store4f(wz_at(xs, h, k0), hi);
  store4f(wz_at(hs, h, k0), lo);
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
// kPbF32: the fp32 pair-bias epilogue of a bf16 transition (a kernel of its
// own, so the other paths compile exactly as without it)
// kNarrow: x and out have cw = P.cw < 128 channels (a multiple of 32) and
// the hidden width is 4 cw; the tile works at 128 channels with the ones past
// cw at zero (zero affine, zero weight rows and columns), in cw / 32 hidden
// chunks, and stores only the first cw channels
template <typename T, bool kPbF32, bool kNarrow = false, int NB = 4>
__device__ __forceinline__ void transition128_body(const TransitionParams<T>& P) {
  using namespace tile;
  __shared__ __attribute__((aligned(16))) T xs[kTP][kLd];  // LN(x)
  __shared__ __attribute__((aligned(16))) T hs[kTP][kLd];  // silu(a) * b, one hidden chunk
  __shared__ __attribute__((aligned(16))) LnAffine ln;
  __shared__ __attribute__((aligned(16))) LnAffine pb_ln;  // the pair-bias epilogue's norm
  // (the fp32-bias form's split weight: the padding columns of xs and hs, wz_at)

  const int64_t m0 = (int64_t)blockIdx.x * kTP;
  const int nvalid = (int)min<int64_t>(kTP, P.rows - m0);
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const int p = t >> 2;
  const int col = 16 * wave;
  const int cw = kNarrow ? P.cw : kC;  // channels of x and out
  const int nch = kNarrow ? cw / 32 : 4;  // 128-wide hidden chunks (hidden = 4 cw)

  {
    // every workgroup stages its affines (one tile each): their loads go out
    // before the tile's rows, so that the LDS writes wait for them alone
    // (ln_fetch)
    const T lnv = ln_fetch<T>(P.ln_w, P.ln_b, cw);
    const bool pb = !kNarrow && !kPbF32 && P.pb_out;
    const T pbv = pb ? ln_fetch<T>(P.pb_ln_w, P.pb_ln_b) : lnv;
    float pbfv = 0.f;
    f32x4 wz = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (kPbF32) {
      pbfv = ln_fetch<float>(P.pbf_ln_w, P.pbf_ln_b);
      wz = wz_fetch(P);
    }
    RowPart<T> xr;
    if constexpr (kNarrow) load_row_part_w<T, NB>(p < nvalid ? P.x + (m0 + p) * cw : nullptr, xr, cw);
    else load_row_part<T>(p < nvalid ? P.x + (m0 + p) * kC : nullptr, xr);
    ln_put<T>(ln, lnv, cw);
    if (pb) ln_put<T>(pb_ln, pbv);
    if constexpr (kPbF32) {
      ln_put<float>(pb_ln, pbfv);
      wz_put(P, wz, xs, hs);
    }
    __syncthreads();
    ln_quad<T, T, NB>(xr, ln, P.eps, &xs[p][0], cw);
  }
  __syncthreads();

  f32x4 out[8];
#pragma unroll
  for (int rt = 0; rt < 8; ++rt) out[rt] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll 1
  for (int ch = 0; ch < nch; ++ch) {
    WCol<T> wa, wb, wo;
    if constexpr (kNarrow) {
      load_wcol_w<T, NB>(P.w_a, cw, ch * kC + col, 0, wa, 4 * cw, cw);
      load_wcol_w<T, NB>(P.w_b, cw, ch * kC + col, 0, wb, 4 * cw, cw);
      load_wcol_w<T>(P.w_o, 4 * cw, col, ch * kC, wo, cw, 4 * cw);
    } else {
      load_wcol<T>(P.w_a, kC, ch * kC + col, 0, wa);
      load_wcol<T>(P.w_b, kC, ch * kC + col, 0, wb);
      load_wcol<T>(P.w_o, 4 * kC, col, ch * kC, wo);
    }
#pragma unroll 2
    for (int rt = 0; rt < 8; ++rt) {
      f32x4 a = f32x4{0.f, 0.f, 0.f, 0.f}, b = f32x4{0.f, 0.f, 0.f, 0.f};
      tile_mma1_acc<T, NB>(xs, rt, wa, a);
      tile_mma1_acc<T, NB>(xs, rt, wb, b);
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

  // the pair-bias weight (rows = heads, zero past pb_heads) is fetched ahead
  // of the output stores so that its latency is not exposed after them
  WCol<T> pb_wf;
  if (!kPbF32 && !kNarrow && P.pb_out) {
    const float zero[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const int h = lane & 15;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      pb_wf[ks] = h < P.pb_heads ? load8(P.pb_w + (int64_t)h * kC + 32 * ks + 8 * (lane >> 4)) : pack8<T>(zero);
  }
  // every row tile's row mask and residual are loaded before the first
  // store: a store counts against the same memory counter a load's use
  // waits on, so loads between stores would each wait for the stores
  // before (rows past the tile's end read the last valid row, unused), with
  // no per-lane branch around them
  float res[8][4], msk[8];
#pragma unroll
  for (int rt = 0; rt < 8; ++rt) {
    msk[rt] = 1.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) res[rt][q] = 0.f;
  }
  // a narrow form's waves past cw hold only zero channels: nothing to store
  if (kNarrow && col >= cw) return;
  if (P.residual) {
#pragma unroll
    for (int rt = 0; rt < 8; ++rt) {
      const int row = min(16 * rt + (lane & 15), nvalid - 1);
      load4f(P.residual + (m0 + row) * cw + col + 4 * (lane >> 4), res[rt]);
    }
  }
  if (P.row_mask) {
#pragma unroll
    for (int rt = 0; rt < 8; ++rt) msk[rt] = to_f32(P.row_mask[m0 + min(16 * rt + (lane & 15), nvalid - 1)]);
  }
  float gate[8];
#pragma unroll
  for (int rt = 0; rt < 8; ++rt) gate[rt] = 1.0f;
  if (P.out_mask) {
#pragma unroll
    for (int rt = 0; rt < 8; ++rt)
      gate[rt] = to_f32(P.out_mask[m0 + min(16 * rt + (lane & 15), nvalid - 1)]) != 0.f ? 1.f : 0.f;
  }

  // the update is rounded to T (the reference's projection output is), then
  // the residual is added
#pragma unroll
  for (int rt = 0; rt < 8; ++rt) {
    const int row = 16 * rt + (lane & 15);
    if (row < nvalid) {
      const int64_t off = (m0 + row) * cw + col + 4 * (lane >> 4);
      float y[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) y[q] = round_to<T>(out[rt][q] * msk[rt]);
      if (P.residual) {
#pragma unroll
        for (int q = 0; q < 4; ++q) y[q] += res[rt][q];
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) y[q] *= gate[rt];
      store4f(P.out + off, y);
      if (kPbF32 || (!kNarrow && P.pb_out)) store4f(&xs[row][col + 4 * (lane >> 4)], y);  // xs is free after the last chunk
    }
  }
  if constexpr (kPbF32) {
    pair_bias_epilogue_f32(P, xs, hs, pb_ln, m0, nvalid);
  } else if constexpr (!kNarrow) {
    if (P.pb_out) pair_bias_epilogue<T>(P, xs, pb_ln, pb_wf, m0, nvalid);
  }
}

template <typename T>
__global__ __launch_bounds__(512) void transition128_kernel(TransitionParams<T> P) {
  transition128_body<T, false>(P);
}
template <typename T, int NB>
__global__ __launch_bounds__(512) void transition_narrow_kernel(TransitionParams<T> P) {
  transition128_body<T, false, true, NB>(P);
}
// two 512-thread workgroups (70 KB of LDS each) share a CU only at 4 waves
// per SIMD, so this variant is held to 128 VGPRs as the plain one fits
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 4)))
void transition128_pbf32_kernel(TransitionParams<bf16> P) {
  transition128_body<bf16, true>(P);
}

// C = 128, or a narrow C (32, 64, 96: p.cw) with a 4C hidden width; other
// widths take the general path of the C ABI layer (row LayerNorm and three
// GEMMs), which also measured faster than a fused kernel for the single
// track's C = 384 at every row count tried (1 K to 1 M rows).
template <typename T>
void launch_transition(const TransitionParams<T>& p, int c, hipStream_t st) {
  const dim3 grid((unsigned)((p.rows + tile::kTP - 1) / tile::kTP));
  if (c < tile::kC) {
    // c = 64 (the template stack): the x side compiled for its 2 blocks of 32
    if (c == 64) hipLaunchKernelGGL((transition_narrow_kernel<T, 2>), grid, dim3(512), 0, st, p);
    else hipLaunchKernelGGL((transition_narrow_kernel<T, 4>), grid, dim3(512), 0, st, p);
    return;
  }
  if constexpr (std::is_same<T, bf16>::value) {
    if (p.pbf_out) {
      hipLaunchKernelGGL(transition128_pbf32_kernel, grid, dim3(512), 0, st, p);
      return;
    }
  }
  hipLaunchKernelGGL(transition128_kernel<T>, grid, dim3(512), 0, st, p);
}

template void launch_transition<bf16>(const TransitionParams<bf16>&, int, hipStream_t);
template void launch_transition<float>(const TransitionParams<float>&, int, hipStream_t);

}  // namespace fjx
