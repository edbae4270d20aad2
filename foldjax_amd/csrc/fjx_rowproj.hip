// LayerNorm + projection prologues and the projection epilogues of the
// triangle ops, on MFMA.
//
// Work unit: a tile of 128 pair positions -- one row r of the (virtual) pair
// grid, 128 consecutive columns s0..s0+127. The LayerNormed tile sits in LDS
// as [position][channel]; each wave computes all 128 positions for 32 output
// channels of one weight, streaming the 8 row tiles of 16 positions past a
// weight slab held in registers.
//
// The kernels are persistent: a grid sized to the resident capacity of the
// device loops over tiles, keeps its weight slabs in registers for the whole
// launch and, once a tile's inputs are in LDS, issues the global loads of its
// next tile before computing the current one. Vector-memory loads complete in
// issue order, so after that prefetch an iteration issues no other global load
// it has to wait for: the residual, when it is the op's own input, is read
// back from a raw copy of the input tile in LDS.
//
// Results are stored straight from the MFMA accumulators, 4 contiguous
// elements per lane:
//   channel-major outputs use D[pos][ch] = X W^T (a lane holds 4 consecutive
//   positions of one channel),
//   position-major outputs use D'[ch][pos] = W X^T (a lane holds 4 consecutive
//   channels of one position); the two differ only in the MFMA operand order.
//
// Prologues address the pair tensor through a *virtual* grid: virtual (r, s)
// reads x[b, r, s] or, when transposed, x[b, s, r]. The incoming tri-mul and
// the ending-node tri-attn run entirely in that transposed virtual grid, so no
// transposed copy of x is ever written.
//
// The output gates -- tri-mul's sigmoid(LN_in(x) g_out^T) and tri-attn's
// sigmoid(LN(x) w_g^T) -- are computed in the epilogues, which read x anyway
// at the output positions; no gate tensor makes an HBM round trip.
//
// Weights are PyTorch [out][in] row-major: output channel o is the contiguous
// row W[o][0..127], which is exactly an MFMA fragment (8 contiguous k for one
// output channel).
#include "fjx_common.hpp"
#include "fjx_kernels.hpp"
#include "fjx_tile.hpp"

namespace fjx {

using namespace tile;

namespace {


}  // namespace

// ---------------------------------------------------------------------------
// Triangle multiplication prologue, 512 threads: waves 0-3 produce a, waves 4-7
// produce b, each wave 32 channels, holding the p_in and g_in slabs of those
// channels for the whole launch.
//   a_cm/b_cm: [B][128][N*N] channel-major in the virtual grid (contraction
//   operands with the contracted axis contiguous), each
//   mask * sigmoid(x_ln g_in^T) * (x_ln p_in^T).
// kNarrow: x has P.cw < 128 channels (a multiple of 32); the tile's channels
// past cw are held at zero (zero LayerNorm affine, zero weight columns). NB:
// the 32-channel blocks of x worked on (cw / 32 when it is known at compile
// time, else all 4, the ones past cw being zero).
// Pipeline: two LDS tiles. Halfway through a tile's MFMAs and sigmoids the
// workgroup LayerNorms the next tile into the other buffer (its rows were
// fetched a tile earlier) and fetches the one after: the two waves of a SIMD
// belong to this one workgroup and would otherwise run the VALU-only
// LayerNorm and the MFMA phase in lockstep, one after the other.
// ---------------------------------------------------------------------------
template <typename T, bool kNarrow, int NB = 4>
__global__ __launch_bounds__(512) void trimul_prologue_kernel(TriMulPrologueParams<T> P, int64_t ntiles) {
  __shared__ __attribute__((aligned(16))) T xs[2][kTP][kLd];
  __shared__ __attribute__((aligned(16))) float mrow[2][kTP];
  __shared__ __attribute__((aligned(16))) LnAffine ln;

  const int64_t n = P.n;
  const int64_t nn = n * n;
  const int64_t ntx = (n + kTP - 1) / kTP;
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const int half = wave >> 2;
  const int col0 = 32 * (wave & 3);
  const int p = t >> 2;  // LayerNorm position of this thread
  const bool vec4 = (n % 4) == 0;
  const bool vec8 = (n % 8) == 0;
  const int cw = kNarrow ? P.cw : kC;

  WSlab<T> wp, wg;
  if constexpr (kNarrow) {
    load_wslab_w<T, NB>(P.w_p + (int64_t)half * kC * cw, cw, col0, wp, kC, cw);
    load_wslab_w<T, NB>(P.w_g + (int64_t)half * kC * cw, cw, col0, wg, kC, cw);
    stage_ln_w<T>(P.ln_w, P.ln_b, ln, cw);
  } else {
    load_wslab<T>(P.w_p + (int64_t)half * kC * kC, col0, wp);
    load_wslab<T>(P.w_g + (int64_t)half * kC * kC, col0, wg);
    stage_ln<T>(P.ln_w, P.ln_b, ln);
  }
  scale_wslab<T>(wg, -kLog2e);  // gates from sigmoid_nl2e

  // the fetched position's mask value stays raw until it is used: a
  // conversion in the fetch would wait there for every load in flight,
  // the row prefetch included
  RowPart<T> xr;
  T mraw = from_f32<T>(0.f);
  bool mvalid = false;
  auto fetch = [&](int64_t tile) {
    const TileRS tl = tile_at(tile, ntx, n);
    const int s = tl.s0 + p;
    const bool valid = s < n;
    auto pos_of = [&](int ss) {
      return (int64_t)tl.b * nn + (P.transpose ? (int64_t)ss * n + tl.r : (int64_t)tl.r * n + ss);
    };
    if constexpr (kNarrow) load_row_part_w<T, NB>(valid ? P.x + pos_of(s) * cw : nullptr, xr, cw);
    else load_row_part<T>(valid ? P.x + pos_of(s) * kC : nullptr, xr);
    mvalid = valid;
    if (P.mask) mraw = P.mask[pos_of(valid ? s : tl.s0)];
  };

  int64_t tile = blockIdx.x;
  if (tile < ntiles) fetch(tile);
  __syncthreads();  // LayerNorm affine staged
  auto ln_tile = [&](int buf) {
    // two-pass statistics: the dot2 form measured 8 % slower here, where
    // this LayerNorm runs between the current tile's MFMA phases
    ln_quad<T, T, NB, false>(xr, ln, P.eps, &xs[buf][p][0], cw);
    if ((t & 3) == 0) mrow[buf][p] = mvalid ? (P.mask ? to_f32(mraw) : 1.0f) : 0.f;
  };
  if (tile < ntiles) {
    ln_tile(0);
    if (tile + gridDim.x < ntiles) fetch(tile + gridDim.x);
  }
  __syncthreads();
  for (int cur = 0; tile < ntiles; tile += gridDim.x, cur ^= 1) {
    const TileRS tl = tile_at(tile, ntx, n);
    const int nvalid = (int)min<int64_t>(kTP, n - tl.s0);
    T* dst = (half == 0 ? P.a_cm : P.b_cm) + (int64_t)tl.b * kC * nn + (int64_t)tl.r * n + tl.s0;
    auto pair = [&](int j) {
      f32x4 ap[2][2], ag[2][2];
#pragma unroll
      for (int h = 0; h < 2; ++h)
        tile_mma2_row<T, false, NB>(xs[cur], paired_row(j, h, lane & 15), wp, wg, ap[h], ag[h]);
      const int p0 = 32 * j + 8 * (lane >> 4);
      const f32x4 m0 = *reinterpret_cast<const f32x4*>(&mrow[cur][p0]);
      const f32x4 m1 = *reinterpret_cast<const f32x4*>(&mrow[cur][p0 + 4]);
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        float v[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          v[q] = m0[q] * sigmoid_nl2e(ag[0][ct][q]) * ap[0][ct][q];
          v[4 + q] = m1[q] * sigmoid_nl2e(ag[1][ct][q]) * ap[1][ct][q];
        }
        store8_masked<T>(dst + (int64_t)(col0 + 16 * ct + (lane & 15)) * nn + p0, v, nvalid - p0, vec8, vec4);
      }
    };
    pair(0);
    pair(1);
    if (tile + gridDim.x < ntiles) {
      ln_tile(cur ^ 1);  // the next tile's LayerNorm, under this tile's MFMAs
      if (tile + 2 * gridDim.x < ntiles) fetch(tile + 2 * gridDim.x);
    }
    pair(2);
    pair(3);
    __syncthreads();  // the next tile's rows are in LDS; this tile's buffer is free
  }
}

// ---------------------------------------------------------------------------
// Triangle attention prologue (virtual grid, transposed for the ending node),
// 512 threads: waves 0-3 produce q and k of head w, waves 4-7 produce v
// channels 32(w-4).. and rows 2(w-4), 2(w-4)+1 of the triangle-bias tile.
//   q  [B][N][H][Np][D]  q_ln * (scale*log2 e)
//   k  [B][N][H][Np][D]
//   vt [B][N][H*D][Np]   v transposed so that keys are contiguous
//   bias [B][H][Np][Np]  x_ln w_bias^T times log2 e (in T)
//   mb [B][N][Np] fp32   inf*(mask-1)*log2 e, -inf for keys >= N
// Np = N rounded up to 64; key slots in [N, Np) are written as zeros.
// kNarrow and NB: x has P.cw < 128 channels, as for the tri-mul prologue.
// ---------------------------------------------------------------------------
template <typename T, bool kNarrow, int NB = 4>
__global__ __launch_bounds__(512) void triattn_prologue_kernel(TriAttnPrologueParams<T> P, int64_t ntiles) {
  __shared__ __attribute__((aligned(16))) T xs[kTP][kLd];
  __shared__ __attribute__((aligned(16))) LnAffine ln;
  constexpr int D = 32;
  constexpr int H = 4;

  const int64_t n = P.n;
  const int64_t np = P.np;
  const int64_t nn = n * n;
  const int64_t ntx = (np + kTP - 1) / kTP;
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const int role = wave >> 2;  // 0: q and k; 1: v and bias
  const int col0 = 32 * (wave & 3);
  const int p = t >> 2;
  const int cw = kNarrow ? P.cw : kC;

  // role 0: w1 = q slab, w2 = k slab of head (wave & 3)
  // role 1: w1 = v slab; w2[ks][0] = bias weights as one 16-column tile
  //         (columns 0..3 = heads, the rest zero)
  WSlab<T> w1, w2;
  if (role == 0) {
    // paired: lane group g holds head dims 8g .. +7, a quarter of a q/k row
    if constexpr (kNarrow) {
      load_wslab_paired_w<T, NB>(P.w_q, cw, col0, w1, kC, cw);
      load_wslab_paired_w<T, NB>(P.w_k, cw, col0, w2, kC, cw);
    } else {
      load_wslab_paired<T>(P.w_q, col0, w1);
      load_wslab_paired<T>(P.w_k, col0, w2);
    }
  } else {
    if constexpr (kNarrow) load_wslab_w<T, NB>(P.w_v, cw, col0, w1, kC, cw);
    else load_wslab<T>(P.w_v, col0, w1);
    const int li = lane & 15;
    const float z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int k = 32 * ks + 8 * (lane >> 4);
      w2[ks][0] = li < H && k < cw ? load8(P.w_bias + li * cw + k) : pack8<T>(z);
      w2[ks][1] = pack8<T>(z);
    }
  }
  if constexpr (kNarrow) stage_ln_w<T>(P.ln_w, P.ln_b, ln, cw);
  else stage_ln<T>(P.ln_w, P.ln_b, ln);

  // the mask value stays raw until it is used (as in the tri-mul prologue)
  RowPart<T> xr;
  T mraw = from_f32<T>(0.f);
  bool mvalid = false;
  auto fetch = [&](int64_t tile) {
    const TileRS tl = tile_at(tile, ntx, n);
    const int s = tl.s0 + p;
    const bool valid = s < n;
    auto pos_of = [&](int ss) {
      return (int64_t)tl.b * nn + (P.transpose ? (int64_t)ss * n + tl.r : (int64_t)tl.r * n + ss);
    };
    if constexpr (kNarrow) load_row_part_w<T, NB>(valid ? P.x + pos_of(s) * cw : nullptr, xr, cw);
    else load_row_part<T>(valid ? P.x + pos_of(s) * kC : nullptr, xr);
    mvalid = valid;
    if (P.mask) mraw = P.mask[pos_of(valid ? s : tl.s0)];
  };

  int64_t tile = blockIdx.x;
  if (tile < ntiles) fetch(tile);
  __syncthreads();
  for (; tile < ntiles; tile += gridDim.x) {
    const TileRS tl = tile_at(tile, ntx, n);
    const int nstore = (int)min<int64_t>(kTP, np - tl.s0);  // incl. zero padding; a multiple of 64
    const int nreal = (int)max<int64_t>(0, min<int64_t>(kTP, n - tl.s0));
    ln_quad<T, T, NB>(xr, ln, P.eps, &xs[p][0], cw);
    if ((t & 3) == 0 && p < nstore) {
      const float mv = P.mask ? to_f32(mraw) : 1.0f;
      P.mb[((int64_t)tl.b * n + tl.r) * np + tl.s0 + p] = mvalid ? P.inf * (mv - 1.0f) * kLog2e : -INFINITY;
    }
    __syncthreads();
    if (tile + gridDim.x < ntiles) fetch(tile + gridDim.x);

    if (role == 0) {
      // transposed accumulators, paired slabs: lane (rt) holds position
      // 16rt + l%16, head dims 8g .. +7 of head (wave & 3) -- 16 lanes cover
      // 16 whole 64-byte q (k) rows
      const int64_t head_off = (((int64_t)tl.b * n + tl.r) * H + (wave & 3)) * np * D;
      T* qb = P.q + head_off;
      T* kb = P.k + head_off;
#pragma unroll 2
      for (int rt = 0; rt < 8; ++rt) {
        const int pp = 16 * rt + (lane & 15);
        f32x4 aq[2], ak[2];
        tile_mma2<T, true, NB>(xs, rt, w1, w2, aq, ak);
        if (pp < nstore) {
          const bool real = pp < nreal;
          float vq[8], vk[8];
#pragma unroll
          for (int ct = 0; ct < 2; ++ct)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              vq[4 * ct + q] = real ? aq[ct][q] * P.q_scale : 0.f;
              vk[4 * ct + q] = real ? ak[ct][q] : 0.f;
            }
          const int64_t off = (int64_t)(tl.s0 + pp) * D + 8 * (lane >> 4);
          store8(qb + off, pack8<T>(vq));
          store8(kb + off, pack8<T>(vk));
        }
      }
    } else {
      // v, channel-major: vt[b][r][ch][s]; row tiles in pairs with paired
      // rows, so lane group g holds positions 32j + 8g .. +7 of its channel
      T* vdst = P.vt + ((int64_t)tl.b * n + tl.r) * kC * np + tl.s0;
#pragma unroll 1
      for (int j = 0; j < kTP / 32; ++j) {
        const int p0 = 32 * j + 8 * (lane >> 4);
        f32x4 av[2][2];
#pragma unroll
        for (int h = 0; h < 2; ++h) tile_mma_row<T, false, NB>(xs, paired_row(j, h, lane & 15), w1, av[h]);
        if (p0 < nstore) {  // nstore is a multiple of 64: all 8 positions are stored
#pragma unroll
          for (int ct = 0; ct < 2; ++ct) {
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = p0 + e < nreal ? av[e >> 2][ct][e & 3] : 0.f;
            store8(vdst + (int64_t)(col0 + 16 * ct + (lane & 15)) * np + p0, pack8<T>(v));
          }
        }
      }
      // triangle bias, pair j = wave & 3: lane holds positions 32j + 8g .. +7
      // of head l%16
      {
        const int j = wave & 3;
        const int p0 = 32 * j + 8 * (lane >> 4);
        f32x4 ab[2][2];
#pragma unroll
        for (int h = 0; h < 2; ++h) tile_mma_row<T, false, NB>(xs, paired_row(j, h, lane & 15), w2, ab[h]);
        const int hd = lane & 15;
        if (hd < H && p0 < nstore) {
          float v[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = p0 + e < nreal ? ab[e >> 2][0][e & 3] * kLog2e : 0.f;
          const int64_t boff = (((int64_t)tl.b * H + hd) * np + tl.r) * np + tl.s0 + p0;
          T* brow = P.bias + boff;
          store8(brow, pack8<T>(v));
          // the bias rows of the padded queries n .. np-1 (whose outputs are
          // dropped) are zeroed too, so the attention never reads stale
          // workspace memory
          const float zero[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
          for (int64_t rz = n + tl.r; rz < np; rz += n) {
            store8(brow + (rz - tl.r) * np, pack8<T>(zero));
          }
        }
      }
    }
    __syncthreads();  // xs is free for the next tile
  }
}

// Epilogue tiles are 64 positions wide (256 threads, 38-57 KB of LDS in
// bf16), so two workgroups share a CU (their 230-256 VGPRs allow no more)
// and their phases interleave.
constexpr int kTE = 64;

// ---------------------------------------------------------------------------
// Triangle multiplication epilogue, original grid (i, j):
//   out[i,j] = LN_out(o[:, i, j]) p_out^T * T(sigmoid(LN_in(x[i,j]) g_out^T)) (+ residual)
// with o channel-major [B][128][N*N]. 256 threads: wave w owns output channels
// 32w .. 32w+31 of both products for the 64 positions, holding the g_out and
// p_out slabs of those channels; the two LayerNormed tiles sit side by side
// in LDS so the gate and the projection of a row tile combine at once.
// kResX: the residual is x itself (read back from the tile's raw copy in
// LDS). A compile-time choice: one pointer that may address LDS or global
// memory compiles to a generic load, which waits for every global access in
// flight -- the previous row tile's store and the next tile's prefetch.
// kNarrow: x, the residual and out have P.cw < 128 channels (a multiple of
// 32); o keeps 128. The waves whose output channels start at or past cw
// only help fill the LDS tiles. NB as for the prologues (the x side only: o
// and its LayerNorm keep 128 channels).
// ---------------------------------------------------------------------------
template <typename T, bool kResX, bool kNarrow, int NB = 4>
__global__ __launch_bounds__(256) void trimul_epilogue_kernel(TriMulEpilogueParams<T> P, int64_t ntiles) {
  __shared__ __attribute__((aligned(16))) T xg[kTE][kLd];    // LN_in(x)
  __shared__ __attribute__((aligned(16))) T xp[kTE][kLd];    // LN_out(o)
  __shared__ __attribute__((aligned(16))) T xraw[kTE][kLd];  // x, when it is also the residual
  __shared__ __attribute__((aligned(16))) LnAffine ln_in, ln_out;

  const int64_t n = P.n;
  const int64_t nn = n * n;
  const int64_t ntx = (n + kTE - 1) / kTE;
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const int col0 = 32 * wave;
  const int p = t >> 2;  // LayerNorm position of this thread
  constexpr bool res_x = kResX;
  const bool vec8 = (n % 8) == 0;
  const int cw = kNarrow ? P.cw : kC;
  const bool active = !kNarrow || col0 < cw;

  WSlab<T> wg, wp;
  if constexpr (kNarrow) {
    load_wslab_paired_w<T, NB>(P.w_gout, cw, col0, wg, cw, cw);
    load_wslab_paired_w<T>(P.w_pout, kC, col0, wp, cw, kC);
    stage_ln_w<T>(P.ln_in_w, P.ln_in_b, ln_in, cw);
  } else {
    load_wslab_paired<T>(P.w_gout, col0, wg);
    load_wslab_paired<T>(P.w_pout, col0, wp);
    stage_ln<T>(P.ln_in_w, P.ln_in_b, ln_in);
  }
  scale_wslab<T>(wg, -kLog2e);  // gates from sigmoid_nl2e
  stage_ln<T>(P.ln_out_w, P.ln_out_b, ln_out);

  // per-tile inputs: the x row of position t/4 and 4 chunks of the
  // channel-major o tile (chunk it: 16 channels x 4 runs of 8 positions per
  // wave; measured faster than 8 lanes per channel reading whole lines,
  // whose transposing LDS writes collide more)
  RowPart<T> xr;
  typename Frag<T>::type ot[4];
  T om[kTE / 16];  // the output mask of this lane's output positions, fetched with the tile
  auto o_chunk = [&](int it, int& ch, int& p0) {
    const int grp = 4 * it + wave;  // 0..15
    ch = 16 * (grp & 7) + (lane & 15);
    p0 = 8 * (4 * (grp >> 3) + (lane >> 4));
  };
  auto fetch = [&](int64_t tile) {
    const TileRS tl = tile_at(tile, ntx, n, kTE);
    const int nvalid = (int)min<int64_t>(kTE, n - tl.s0);
    const int64_t pos0 = (int64_t)tl.b * nn + (int64_t)tl.r * n + tl.s0;
    if constexpr (kNarrow) load_row_part_w<T, NB>(p < nvalid ? P.x + (pos0 + p) * cw : nullptr, xr, cw);
    else load_row_part<T>(p < nvalid ? P.x + (pos0 + p) * kC : nullptr, xr);
    // channel-major: channel ch of the tile at src + ch * nn; tile-blocked:
    // the whole tile is one contiguous [128][64] block
    const int64_t cstride = P.o_blocked ? 256 : nn;
    const int64_t ipos = (int64_t)tl.r * n + tl.s0;  // within the batch item
    const T* src = P.o_blocked ? P.o + ((int64_t)tl.b * nn + (ipos & ~(int64_t)255)) * kC + (ipos & 255)
                               : P.o + (int64_t)tl.b * kC * nn + ipos;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      int ch, p0;
      o_chunk(it, ch, p0);
      if (vec8 && p0 + 8 <= nvalid) {
        ot[it] = load8(src + (int64_t)ch * cstride + p0);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) ot[it][e] = (p0 + e < nvalid) ? src[(int64_t)ch * cstride + p0 + e] : from_f32<T>(0.f);
      }
    }
    if (P.out_mask) {
#pragma unroll
      for (int rt = 0; rt < kTE / 16; ++rt) om[rt] = P.out_mask[pos0 + min(16 * rt + (lane & 15), nvalid - 1)];
    }
  };

  int64_t tile = blockIdx.x;
  if (tile < ntiles) fetch(tile);
  __syncthreads();  // LayerNorm affines staged
  for (; tile < ntiles; tile += gridDim.x) {
    const TileRS tl = tile_at(tile, ntx, n, kTE);
    const int nvalid = (int)min<int64_t>(kTE, n - tl.s0);
    const int64_t pos0 = (int64_t)tl.b * nn + (int64_t)tl.r * n + tl.s0;

    if (res_x) store_row_part<T, NB>(xr, &xraw[p][0]);
    // the output gate of this tile (bit rt: row tile rt is kept), taken
    // before the next fetch replaces om
    uint32_t keep = (1u << (kTE / 16)) - 1;
    if (P.out_mask) {
      keep = 0;
#pragma unroll
      for (int rt = 0; rt < kTE / 16; ++rt) keep |= to_f32(om[rt]) != 0.f ? 1u << rt : 0u;
    }
    ln_quad<T, T, NB>(xr, ln_in, P.eps, &xg[p][0], cw);
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      int ch, p0;
      o_chunk(it, ch, p0);
#pragma unroll
      for (int e = 0; e < 8; ++e) xp[p0 + e][ch] = ot[it][e];
    }
    // the tile's x and o are in LDS: the next tile's loads go out now, ahead
    // of LN_out and its two barriers
    if (tile + gridDim.x < ntiles) fetch(tile + gridDim.x);
    __syncthreads();
    {
      // LN_out in place: each thread rewrites exactly the 32 channels it reads
      RowPart<T> rp;
      load_row_part<T>(&xp[p][0], rp);
      ln_quad<T>(rp, ln_out, P.eps, &xp[p][0]);
    }
    __syncthreads();

#pragma unroll 2
    for (int rt = 0; rt < (active ? kTE / 16 : 0); ++rt) {
      f32x4 ag[2], ap[2];
      tile_mma<T, true, NB>(xg, rt, wg, ag);
      tile_mma<T, true>(xp, rt, wp, ap);
      // paired slabs: this lane holds channels col0 + 8g .. +7 of position pp
      const int pp = 16 * rt + (lane & 15);
      if (pp < nvalid) {
        const int c = col0 + 8 * (lane >> 4);
        const int64_t off = (pos0 + pp) * cw + c;
        float y[8];
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
          for (int q = 0; q < 4; ++q) y[4 * ct + q] = ap[ct][q] * round_to<T>(sigmoid_nl2e(ag[ct][q]));
        if (P.residual) {
          float rv[8];
          if constexpr (res_x) to_f32x8(load8(&xraw[pp][c]), rv);
          else to_f32x8(load8(P.residual + off), rv);
#pragma unroll
          for (int e = 0; e < 8; ++e) y[e] += rv[e];
        }
        if (P.out_mask) {
          const float g = (keep >> rt) & 1u ? 1.f : 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) y[e] *= g;
        }
        store8(P.out + off, pack8<T>(y));
      }
    }
    __syncthreads();  // the LDS tiles are free for the next tile
  }
}

// ---------------------------------------------------------------------------
// Triangle attention epilogue, virtual grid rows r, columns s:
//   out[orig] = T(o[r,s] * sigmoid(LN(x[orig]) w_g^T)) w_o^T (+ residual[orig])
// with o position-major [B][N*N][128] and orig = (r, s) or (s, r). 256
// threads: wave w owns output channels 32w .. 32w+31 of both products for the
// 64 positions, holding the w_g and w_o slabs. kResX, kNarrow and NB as for
// the tri-mul epilogue (o and the gate keep 128 channels).
// ---------------------------------------------------------------------------
template <typename T, bool kResX, bool kNarrow, int NB = 4>
__global__ __launch_bounds__(256) void triattn_epilogue_kernel(TriAttnEpilogueParams<T> P, int64_t ntiles) {
  __shared__ __attribute__((aligned(16))) T xs[kTE][kLd];    // LN(x)
  __shared__ __attribute__((aligned(16))) T xo[kTE][kLd];    // gated o
  __shared__ __attribute__((aligned(16))) T xraw[kTE][kLd];  // x, when it is also the residual
  __shared__ __attribute__((aligned(16))) LnAffine ln;

  const int64_t n = P.n;
  const int64_t nn = n * n;
  const int64_t ntx = (n + kTE - 1) / kTE;
  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const int col0 = 32 * wave;
  const int p = t >> 2;
  const bool gated = P.w_g != nullptr;
  constexpr bool res_x = kResX;
  const bool need_x = gated || res_x;
  const int cw = kNarrow ? P.cw : kC;
  const bool active = !kNarrow || col0 < cw;

  // paired slabs: lane group g works on the 8 consecutive channels
  // col0 + 8g .. +7, so o, the residual and the output move 16 bytes a lane
  WSlab<T> wg, wo;
  if constexpr (kNarrow) {
    if (gated) load_wslab_paired_w<T, NB>(P.w_g, cw, col0, wg, kC, cw);
    load_wslab_paired_w<T>(P.w_o, kC, col0, wo, cw, kC);
    if (gated) stage_ln_w<T>(P.ln_w, P.ln_b, ln, cw);
  } else {
    if (gated) load_wslab_paired<T>(P.w_g, col0, wg);
    load_wslab_paired<T>(P.w_o, col0, wo);
    if (gated) stage_ln<T>(P.ln_w, P.ln_b, ln);
  }
  if (gated) scale_wslab<T>(wg, -kLog2e);  // gates from sigmoid_nl2e

  auto orig_of = [&](const TileRS& tl, int pp) -> int64_t {
    const int64_t s = tl.s0 + pp;
    return (int64_t)tl.b * nn + (P.transpose ? s * n + tl.r : (int64_t)tl.r * n + s);
  };

  // per-tile inputs: the x row of position t/4 (at its output position) and o
  // for this wave's accumulator slots (position 16rt + l%16, channels
  // col0 + 8g .. +7)
  RowPart<T> xr;
  typename Frag<T>::type ov[kTE / 16];
  T om[kTE / 16];  // the output mask of this lane's output positions, fetched with the tile
  auto fetch = [&](int64_t tile) {
    const TileRS tl = tile_at(tile, ntx, n, kTE);
    const int nvalid = (int)min<int64_t>(kTE, n - tl.s0);
    if constexpr (kNarrow) {
      if (need_x) load_row_part_w<T, NB>(p < nvalid ? P.x + orig_of(tl, p) * cw : nullptr, xr, cw);
    } else {
      if (need_x) load_row_part<T>(p < nvalid ? P.x + orig_of(tl, p) * kC : nullptr, xr);
    }
    // head-major o: this wave's head (channels col0 .. col0+31) of the tile's
    // 64 positions is one contiguous 4 KB block
    const T* osrc = P.o + ((((int64_t)tl.b * n + tl.r) * 4 + wave) * n + tl.s0) * 32;
#pragma unroll
    for (int rt = 0; rt < kTE / 16; ++rt) {
      const int pp = 16 * rt + (lane & 15);
      if (pp < nvalid) {
        ov[rt] = load8(osrc + (int64_t)pp * 32 + 8 * (lane >> 4));
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) ov[rt][e] = from_f32<T>(0.f);
      }
    }
    if (P.out_mask) {
#pragma unroll
      for (int rt = 0; rt < kTE / 16; ++rt) om[rt] = P.out_mask[orig_of(tl, min(16 * rt + (lane & 15), nvalid - 1))];
    }
  };

  int64_t tile = blockIdx.x;
  if (tile < ntiles) fetch(tile);
  __syncthreads();
  for (; tile < ntiles; tile += gridDim.x) {
    const TileRS tl = tile_at(tile, ntx, n, kTE);
    const int nvalid = (int)min<int64_t>(kTE, n - tl.s0);

    if (res_x) store_row_part<T, NB>(xr, &xraw[p][0]);
    // the output gate of this tile (bit rt: row tile rt is kept), taken
    // before the next fetch replaces om
    uint32_t keep = (1u << (kTE / 16)) - 1;
    if (P.out_mask) {
      keep = 0;
#pragma unroll
      for (int rt = 0; rt < kTE / 16; ++rt) keep |= to_f32(om[rt]) != 0.f ? 1u << rt : 0u;
    }
    if (gated) {
      ln_quad<T, T, NB>(xr, ln, P.eps, &xs[p][0], cw);
      __syncthreads();
#pragma unroll
      for (int rt = 0; rt < kTE / 16; ++rt) {
        f32x4 ag[2];
        tile_mma<T, true, NB>(xs, rt, wg, ag);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            ov[rt][4 * ct + q] = from_f32<T>(to_f32(ov[rt][4 * ct + q]) * sigmoid_nl2e(ag[ct][q]));
      }
    }
    // gated (or raw) o -> xo; the four waves fill its 128 channels
#pragma unroll
    for (int rt = 0; rt < kTE / 16; ++rt) store8(&xo[16 * rt + (lane & 15)][col0 + 8 * (lane >> 4)], ov[rt]);
    __syncthreads();
    if (tile + gridDim.x < ntiles) fetch(tile + gridDim.x);

#pragma unroll
    for (int rt = 0; rt < (active ? kTE / 16 : 0); ++rt) {
      f32x4 acc[2];
      tile_mma<T, true>(xo, rt, wo, acc);
      const int pp = 16 * rt + (lane & 15);
      if (pp < nvalid) {
        const int c = col0 + 8 * (lane >> 4);
        const int64_t off = orig_of(tl, pp) * cw + c;
        float y[8];
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
          for (int q = 0; q < 4; ++q) y[4 * ct + q] = acc[ct][q];
        if (P.residual) {
          float rv[8];
          if constexpr (res_x) to_f32x8(load8(&xraw[pp][c]), rv);
          else to_f32x8(load8(P.residual + off), rv);
#pragma unroll
          for (int e = 0; e < 8; ++e) y[e] += rv[e];
        }
        if (P.out_mask) {
          const float g = (keep >> rt) & 1u ? 1.f : 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) y[e] *= g;
        }
        store8(P.out + off, pack8<T>(y));
      }
    }
    __syncthreads();  // the LDS tiles are free for the next tile
  }
}

// ---------------------------------------------------------------------------
// host-side launchers
// ---------------------------------------------------------------------------
// a persistent launch of one kernel instance over ntiles tiles
template <typename P>
void launch_persistent(void (*kern)(P, int64_t), const P& p, int threads, int64_t ntiles, hipStream_t st) {
  const void* k = reinterpret_cast<const void*>(kern);
  hipLaunchKernelGGL(kern, dim3(persistent_grid(k, threads, ntiles)), dim3(threads), 0, st, p, ntiles);
}

template <typename T>
void launch_trimul_prologue(const TriMulPrologueParams<T>& p, int64_t batch, hipStream_t st) {
  const int64_t ntiles = (p.n + kTP - 1) / kTP * p.n * batch;
  launch_persistent(p.cw == 64 ? trimul_prologue_kernel<T, true, 2>
                    : p.cw ? trimul_prologue_kernel<T, true> : trimul_prologue_kernel<T, false>,
                    p, 512, ntiles, st);
}
template <typename T>
void launch_triattn_prologue(const TriAttnPrologueParams<T>& p, int64_t batch, hipStream_t st) {
  const int64_t ntiles = (p.np + kTP - 1) / kTP * p.n * batch;
  launch_persistent(p.cw == 64 ? triattn_prologue_kernel<T, true, 2>
                    : p.cw ? triattn_prologue_kernel<T, true> : triattn_prologue_kernel<T, false>,
                    p, 512, ntiles, st);
}
template <typename T>
void launch_trimul_epilogue(const TriMulEpilogueParams<T>& p, int64_t batch, hipStream_t st) {
  const int64_t ntiles = (p.n + kTE - 1) / kTE * p.n * batch;
  const bool res_x = p.residual && p.residual == p.x;
  auto kern = p.cw == 64 ? (res_x ? trimul_epilogue_kernel<T, true, true, 2> : trimul_epilogue_kernel<T, false, true, 2>)
              : res_x ? (p.cw ? trimul_epilogue_kernel<T, true, true> : trimul_epilogue_kernel<T, true, false>)
                      : (p.cw ? trimul_epilogue_kernel<T, false, true> : trimul_epilogue_kernel<T, false, false>);
  launch_persistent(kern, p, 256, ntiles, st);
}
template <typename T>
void launch_triattn_epilogue(const TriAttnEpilogueParams<T>& p, int64_t batch, hipStream_t st) {
  const int64_t ntiles = (p.n + kTE - 1) / kTE * p.n * batch;
  const bool res_x = p.residual && p.residual == p.x;
  auto kern = p.cw == 64 ? (res_x ? triattn_epilogue_kernel<T, true, true, 2> : triattn_epilogue_kernel<T, false, true, 2>)
              : res_x ? (p.cw ? triattn_epilogue_kernel<T, true, true> : triattn_epilogue_kernel<T, true, false>)
                      : (p.cw ? triattn_epilogue_kernel<T, false, true> : triattn_epilogue_kernel<T, false, false>);
  launch_persistent(kern, p, 256, ntiles, st);
}

#define FJX_INST(T)                                                                                 \
  template void launch_trimul_prologue<T>(const TriMulPrologueParams<T>&, int64_t, hipStream_t);   \
  template void launch_triattn_prologue<T>(const TriAttnPrologueParams<T>&, int64_t, hipStream_t); \
  template void launch_trimul_epilogue<T>(const TriMulEpilogueParams<T>&, int64_t, hipStream_t);   \
  template void launch_triattn_epilogue<T>(const TriAttnEpilogueParams<T>&, int64_t, hipStream_t);
FJX_INST(float)
FJX_INST(bf16)
#undef FJX_INST

}  // namespace fjx
