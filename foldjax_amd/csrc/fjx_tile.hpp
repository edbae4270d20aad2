// Tile building blocks shared by the 128-channel row kernels (triangle
// prologues/epilogues, pair transition): LayerNorm of a tile held as
// [position][channel] in LDS by quads of threads, and MFMA row tiles against
// weight slabs held in registers.
#pragma once

#include <map>
#include <mutex>
#include <type_traits>
#include <utility>

#include "fjx_common.hpp"

namespace fjx {
namespace tile {

constexpr int kTP = 128;     // positions per tile
constexpr int kC = 128;      // channels
// Padded LDS row (elements): 288-byte rows. An MFMA fragment read (16 rows,
// four 16-byte chunks a row, one ds_read_b128 per lane) runs at the
// conflict-free rate on them, where 272-byte rows take twice the LDS cycles
// (timed on gfx950 for every stride from 256 to 384 bytes: 288 and 352 are
// the conflict-free ones). The 16 padding elements of a row are free space
// (the fp32 pair-bias transition keeps its split weight there).
constexpr int kLd = kC + 16;

// fp32 copy of a LayerNorm affine (gamma, beta) in LDS, staged once per
// workgroup so the per-element normalisation does no bf16 unpacking
struct LnAffine {
  float w[kC];
  float b[kC];
};

template <typename T>
__device__ __forceinline__ void stage_ln(const T* __restrict__ ln_w, const T* __restrict__ ln_b, LnAffine& l) {
  const int t = threadIdx.x;  // >= 256 threads: 0..127 gamma, 128..255 beta
  if (t < kC) l.w[t] = to_f32(ln_w[t]);
  else if (t < 2 * kC) l.b[t - kC] = to_f32(ln_b[t - kC]);
}
// A narrow width cw < 128 (a multiple of 32) runs the 128-channel kernels
// with the channels past cw held at zero: the affine is zero there, so the
// LayerNorm writes zeros into them and they add nothing to any product.
template <typename T>
__device__ __forceinline__ void stage_ln_w(const T* __restrict__ ln_w, const T* __restrict__ ln_b, LnAffine& l,
                                           int cw) {
  const int t = threadIdx.x;
  if (t < kC) l.w[t] = t < cw ? to_f32(ln_w[t]) : 0.f;
  else if (t < 2 * kC) l.b[t - kC] = t - kC < cw ? to_f32(ln_b[t - kC]) : 0.f;
}
// The same staging in two halves, for a kernel that stages an affine per
// tile: the fetch is one unconditional load per thread (threads 0..127 gamma,
// 128..255 beta, the others a clamped duplicate; channels at or past cw read
// the last valid one), issued before the tile's row loads, and the put writes
// it to LDS after them. A branch per thread, as in stage_ln, puts a wait for
// every load issued so far (the row loads included) in front of each LDS
// write.
template <typename T>
__device__ __forceinline__ T ln_fetch(const T* __restrict__ ln_w, const T* __restrict__ ln_b, int cw = kC) {
  const int ti = min((int)threadIdx.x, 2 * kC - 1);
  const int c = min(ti < kC ? ti : ti - kC, cw - 1);
  return *((ti < kC ? ln_w : ln_b) + c);
}
template <typename T>
__device__ __forceinline__ void ln_put(LnAffine& l, T v, int cw = kC) {
  const int t = threadIdx.x;
  if (t < 2 * kC) {
    const int c = t < kC ? t : t - kC;
    (t < kC ? l.w : l.b)[c] = c < cw ? to_f32(v) : 0.f;
  }
}

// The 32 channels [32*part, +32) of one pair-tensor row (part = threadIdx.x % 4),
// raw, or zeros when src is null (a position outside the grid)
template <typename T>
struct RowPart {
  typename Frag<T>::type f[4];
};
// The 4 threads of a position hold interleaved 8-channel chunks: part j has
// chunks j, 4+j, 8+j, 12+j (f[q] = channels 32q + 8j .. +7), so each of the
// four 16-byte loads of the quad reads 64 contiguous bytes of the row.
__device__ __forceinline__ int row_chunk(int q) { return 32 * q + 8 * (threadIdx.x & 3); }

template <typename T>
__device__ __forceinline__ void load_row_part(const T* __restrict__ src, RowPart<T>& r) {
  if (src) {
#pragma unroll
    for (int q = 0; q < 4; ++q) r.f[q] = load8(src + row_chunk(q));
  } else {
    const float z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < 4; ++q) r.f[q] = pack8<T>(z);
  }
}
// the same for a row of cw channels (a multiple of 32): the chunks past cw
// are zero
// NB (the compile-time number of 32-channel blocks, cw / 32 when known):
// only the first NB chunks of a row part are loaded, normalised or stored
template <typename T, int NB = 4>
__device__ __forceinline__ void load_row_part_w(const T* __restrict__ src, RowPart<T>& r, int cw) {
  const float z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < NB; ++q) r.f[q] = src && 32 * q < cw ? load8(src + row_chunk(q)) : pack8<T>(z);
}
template <typename T, int NB = 4>
__device__ __forceinline__ void store_row_part(const RowPart<T>& r, T* __restrict__ dst_row) {
#pragma unroll
  for (int q = 0; q < NB; ++q) store8(dst_row + row_chunk(q), r.f[q]);
}

// LayerNorm of 128 channels held by 4 consecutive threads (the chunks of
// load_row_part); put(c, o) receives the 8 outputs of channels c .. c+7.
// cw < 128: the statistics are those of the first cw channels (the chunks
// past cw hold zeros and are left out of the variance). kDot: bf16 rows
// take their statistics on v_dot2_f32_bf16 (below) and the quad sums on
// DPP; otherwise, and for fp32 rows, two passes over the unpacked values
template <typename T, typename Put, int NB = 4, bool kDot = true>
__device__ __forceinline__ void ln_quad_put(const RowPart<T>& r, const LnAffine& l, float eps, Put put, int cw = kC) {
  float v[8 * NB];
#pragma unroll
  for (int q = 0; q < NB; ++q) to_f32x8(r.f[q], v + 8 * q);
  const float inv_c = cw == kC ? 1.0f / kC : 1.0f / (float)cw;
  float mean, var;
  if constexpr (kDot && std::is_same<T, bf16>::value) {
    // bf16 rows: the sum and the sum of squares straight from the packed
    // pairs on v_dot2_f32_bf16 (a bf16 product is exact in fp32), one
    // instruction per two channels instead of an unpack, an add and a
    // square per channel; var = E[x^2] - mean^2 in fp32 (chunks past cw
    // hold zeros and add nothing to either sum)
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const bf16x2 one = {static_cast<bf16>(1.0f), static_cast<bf16>(1.0f)};
    float s[2] = {0.f, 0.f}, q2[2] = {0.f, 0.f};
#pragma unroll
    for (int q = 0; q < NB; ++q) {
      const u32x4 u = __builtin_bit_cast(u32x4, r.f[q]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // through a scalar: a bit_cast of the vector element itself compiles
        // to a read of element 0 whatever e is
        const uint32_t w = u[e];
        const bf16x2 pr = __builtin_bit_cast(bf16x2, w);
        s[e & 1] = __builtin_amdgcn_fdot2_f32_bf16(pr, one, s[e & 1], false);
        q2[e & 1] = __builtin_amdgcn_fdot2_f32_bf16(pr, pr, q2[e & 1], false);
      }
    }
    const float st = quad_sum(s[0] + s[1]), qt = quad_sum(q2[0] + q2[1]);
    mean = st * inv_c;
    var = fmaxf(fmaf(-mean, mean, qt * inv_c), 0.f);
    // E[x^2] - mean^2 cancels when the mean dwarfs the spread; past a
    // ratio of 64 (6 bits of the fp32 sums) the row takes the two-pass
    // variance instead (quad-uniform: the 4 lanes hold the same sums)
    if (mean * mean > 64.0f * var) {
      float q2b = 0.f;
#pragma unroll
      for (int e = 0; e < 8 * NB; ++e) {
        const float d = v[e] - mean;
        if (cw == kC || 32 * (e / 8) < cw) q2b += d * d;
      }
      var = quad_sum(q2b) * inv_c;
    }
  } else {
    // the same sums whichever way the quad's lanes are combined (DPP or
    // ds_bpermute); the tri-mul prologue measured faster with the latter
    auto qsum = [](float x) {
      if constexpr (kDot) return quad_sum(x);
      x += shfl_xor(x, 1);
      return x + shfl_xor(x, 2);
    };
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8 * NB; ++e) s += v[e];
    mean = qsum(s) * inv_c;
    float q2 = 0.f;
#pragma unroll
    for (int e = 0; e < 8 * NB; ++e) {
      const float d = v[e] - mean;
      if (cw == kC || 32 * (e / 8) < cw) q2 += d * d;
    }
    var = qsum(q2) * inv_c;
  }
  const float rstd = __builtin_amdgcn_rsqf(var + eps);
  const float shift = -mean * rstd;
#pragma unroll
  for (int q = 0; q < NB; ++q) {
    // one 8-channel chunk at a time: keeps the scheduler from hoisting all 16
    // affine reads (64 VGPRs) ahead of the arithmetic
    __builtin_amdgcn_sched_barrier(0);
    const int c = row_chunk(q);
    const f32x4 w0 = *reinterpret_cast<const f32x4*>(&l.w[c]);
    const f32x4 w1 = *reinterpret_cast<const f32x4*>(&l.w[c + 4]);
    const f32x4 b0 = *reinterpret_cast<const f32x4*>(&l.b[c]);
    const f32x4 b1 = *reinterpret_cast<const f32x4*>(&l.b[c + 4]);
    float o[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o[e] = fmaf(fmaf(v[8 * q + e], rstd, shift), w0[e], b0[e]);
      o[4 + e] = fmaf(fmaf(v[8 * q + 4 + e], rstd, shift), w1[e], b1[e]);
    }
    put(c, o);
  }
}

// ... written to the same channels of dst_row as TO
template <typename T, typename TO, int NB = 4, bool kDot = true>
__device__ __forceinline__ void ln_quad(const RowPart<T>& r, const LnAffine& l, float eps, TO* __restrict__ dst_row,
                                        int cw = kC) {
  auto put = [&](int c, const float* o) { store8(dst_row + c, pack8<TO>(o)); };
  ln_quad_put<T, decltype(put), NB, kDot>(r, l, eps, put, cw);
}

// One wave's 32 output channels col0..col0+31 of a [128][128] weight as MFMA
// fragments: wf[ks][ct] holds W[col0 + 16ct + l%16][32ks + 8g .. +7].
template <typename T>
using WSlab = typename Frag<T>::type[4][2];

template <typename T>
__device__ __forceinline__ void load_wslab(const T* __restrict__ w, int col0, WSlab<T>& wf) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
      wf[ks][ct] = load8(w + (int64_t)(col0 + 16 * ct + (lane & 15)) * kC + 32 * ks + 8 * (lane >> 4));
}

// A slab times s, each weight rounded back to T: the persistent row kernels
// hold their gate slabs as -log2(e) W once per launch, so that a gate is
// sigmoid_nl2e of the accumulator (one multiply per element less; in bf16
// each weight moves by at most half an ulp of the scaled value)
template <typename T>
__device__ __forceinline__ void scale_wslab(WSlab<T>& wf, float s) {
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
      for (int e = 0; e < 8; ++e) wf[ks][ct][e] = from_f32<T>(to_f32(wf[ks][ct][e]) * s);
}

// The same slab with its output channels paired: row i of column tile ct is
// channel col0 + 8 (i/4) + 4 ct + i%4, so in the transposed form lane group g
// holds the 8 consecutive channels col0 + 8g .. +7 (acc[0] the first four,
// acc[1] the next four) and a row goes out in one 16-byte store per lane.
template <typename T>
__device__ __forceinline__ void load_wslab_paired(const T* __restrict__ w, int col0, WSlab<T>& wf) {
  const int lane = threadIdx.x & 63;
  const int li = lane & 15;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
      wf[ks][ct] = load8(w + (int64_t)(col0 + 8 * (li >> 2) + 4 * ct + (li & 3)) * kC + 32 * ks + 8 * (lane >> 4));
}

// the same two loaders for a weight with rows ld elements apart, rows >=
// nrows and columns >= kmax read as zero (a narrow width's padding)
template <typename T, int NB = 4>
__device__ __forceinline__ void load_wslab_w(const T* __restrict__ w, int64_t ld, int col0, WSlab<T>& wf, int nrows,
                                             int kmax) {
  const int lane = threadIdx.x & 63;
  const float z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < NB; ++ks)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      const int row = col0 + 16 * ct + (lane & 15), k = 32 * ks + 8 * (lane >> 4);
      wf[ks][ct] = row < nrows && k < kmax ? load8(w + (int64_t)row * ld + k) : pack8<T>(z);
    }
}
template <typename T, int NB = 4>
__device__ __forceinline__ void load_wslab_paired_w(const T* __restrict__ w, int64_t ld, int col0, WSlab<T>& wf,
                                                    int nrows, int kmax) {
  const int lane = threadIdx.x & 63;
  const int li = lane & 15;
  const float z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < NB; ++ks)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      const int row = col0 + 8 * (li >> 2) + 4 * ct + (li & 3), k = 32 * ks + 8 * (lane >> 4);
      wf[ks][ct] = row < nrows && k < kmax ? load8(w + (int64_t)row * ld + k) : pack8<T>(z);
    }
}

// One 16-row tile against one slab, K = 128; `row` is the tile row this lane
// feeds (16rt + l%16 for row tile rt):
//   kTrans = false: acc[ct][q] = D[row of lane 4g + q][ch col0 + 16ct + l%16]
//   kTrans = true:  acc[ct][q] = D[row of lane l%16][ch col0 + 16ct + 4g + q]
template <typename T, bool kTrans, int NB = 4>
__device__ __forceinline__ void tile_mma_row(const T (*xs)[kLd], int row, const WSlab<T>& wf, f32x4 (&acc)[2]) {
  const int lane = threadIdx.x & 63;
  acc[0] = acc[1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < NB; ++ks) {
    const typename Frag<T>::type xf = load8(&xs[row][32 * ks + 8 * (lane >> 4)]);
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      if (kTrans) mma(acc[ct], wf[ks][ct], xf);
      else mma(acc[ct], xf, wf[ks][ct]);
    }
  }
}
template <typename T, bool kTrans, int NB = 4>
__device__ __forceinline__ void tile_mma(const T (*xs)[kLd], int rt, const WSlab<T>& wf, f32x4 (&acc)[2]) {
  tile_mma_row<T, kTrans, NB>(xs, 16 * rt + (threadIdx.x & 15), wf, acc);
}

// Rows of the tile pair j (rows 32j .. 32j+31) in paired order: half h of
// the pair feeds row 32j + 8 (l%16 / 4) + 4h + l%4 from lane l, so in the
// plain form lane group g holds rows 32j + 8g .. +7 (half 0 the first four,
// half 1 the next four): a channel-major output goes out 16 bytes a lane.
__device__ __forceinline__ int paired_row(int j, int h, int li) { return 32 * j + 8 * (li >> 2) + 4 * h + (li & 3); }

// the same for two slabs sharing the row fragments
template <typename T, bool kTrans, int NB = 4>
__device__ __forceinline__ void tile_mma2_row(const T (*xs)[kLd], int row, const WSlab<T>& w1, const WSlab<T>& w2,
                                              f32x4 (&a1)[2], f32x4 (&a2)[2]) {
  const int lane = threadIdx.x & 63;
  a1[0] = a1[1] = a2[0] = a2[1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < NB; ++ks) {
    const typename Frag<T>::type xf = load8(&xs[row][32 * ks + 8 * (lane >> 4)]);
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      if (kTrans) {
        mma(a1[ct], w1[ks][ct], xf);
        mma(a2[ct], w2[ks][ct], xf);
      } else {
        mma(a1[ct], xf, w1[ks][ct]);
        mma(a2[ct], xf, w2[ks][ct]);
      }
    }
  }
}
template <typename T, bool kTrans, int NB = 4>
__device__ __forceinline__ void tile_mma2(const T (*xs)[kLd], int rt, const WSlab<T>& w1, const WSlab<T>& w2,
                                          f32x4 (&a1)[2], f32x4 (&a2)[2]) {
  tile_mma2_row<T, kTrans, NB>(xs, 16 * rt + (threadIdx.x & 15), w1, w2, a1, a2);
}

// 4 elements of T packed in registers (two VGPRs for bf16)
template <typename T> struct Vec4;
template <> struct Vec4<bf16> { typedef bf16x4 type; };
template <> struct Vec4<float> { typedef f32x4 type; };

template <typename T>
__device__ __forceinline__ typename Vec4<T>::type load4raw(const T* p) {
  return *reinterpret_cast<const typename Vec4<T>::type*>(p);
}
template <typename T>
__device__ __forceinline__ void store4raw(T* p, const typename Vec4<T>::type& v) {
  *reinterpret_cast<typename Vec4<T>::type*>(p) = v;
}

// Store 4 consecutive elements v[0..3] at dst[0..3], of which the first `cnt`
// exist; vectorised when all 4 exist and `vec` says the address is aligned.
// 8 consecutive elements: one 16-byte store when `vec8` and all are in
// range, else two store4_masked halves (8-byte stores when `vec4`)
template <typename T>
__device__ __forceinline__ void store4_masked(T* dst, const float* v, int cnt, bool vec);
template <typename T>
__device__ __forceinline__ void store8_masked(T* dst, const float* v, int cnt, bool vec8, bool vec4) {
  if (cnt >= 8 && vec8) {
    store8(dst, pack8<T>(v));
  } else {
    store4_masked<T>(dst, v, cnt, vec4);
    if (cnt > 4) store4_masked<T>(dst + 4, v + 4, cnt - 4, vec4);
  }
}

template <typename T>
__device__ __forceinline__ void store4_masked(T* dst, const float* v, int cnt, bool vec) {
  if (cnt >= 4 && vec) {
    store4f(dst, v);
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (q < cnt) dst[q] = from_f32<T>(v[q]);
  }
}

// One 16-column tile of a weight over K = 128: wf[ks] holds
// W[row0 + l%16][k0 + 32ks + 8g .. +7] with rows ldw elements apart.
template <typename T>
using WCol = typename Frag<T>::type[4];

template <typename T>
__device__ __forceinline__ void load_wcol(const T* __restrict__ w, int64_t ldw, int row0, int64_t k0, WCol<T>& wf) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) wf[ks] = load8(w + (int64_t)(row0 + (lane & 15)) * ldw + k0 + 32 * ks + 8 * (lane >> 4));
}

// the same with rows >= nrows and columns k >= kmax (multiples of 8) read as zero
template <typename T, int NB = 4>
__device__ __forceinline__ void load_wcol_w(const T* __restrict__ w, int64_t ldw, int row0, int64_t k0, WCol<T>& wf,
                                            int nrows, int64_t kmax) {
  const int lane = threadIdx.x & 63;
  const float z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const int row = row0 + (lane & 15);
#pragma unroll
  for (int ks = 0; ks < NB; ++ks) {
    const int64_t k = k0 + 32 * ks + 8 * (lane >> 4);
    wf[ks] = row < nrows && k < kmax ? load8(w + (int64_t)row * ldw + k) : pack8<T>(z);
  }
}

// acc += rows 16rt.. of the tile against one 16-column tile, transposed form:
// acc[q] = D[pos 16rt + l%16][col 4g + q]
template <typename T, int NB = 4>
__device__ __forceinline__ void tile_mma1_acc(const T (*xs)[kLd], int rt, const WCol<T>& wf, f32x4& acc) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int ks = 0; ks < NB; ++ks)
    mma(acc, wf[ks], load8(&xs[16 * rt + (lane & 15)][32 * ks + 8 * (lane >> 4)]));
}

// tile index -> (batch, row, first column); columns fastest, then rows
struct TileRS {
  int b;
  int r;
  int s0;
};
__device__ __forceinline__ TileRS tile_at(int64_t tile, int64_t ntx, int64_t nrows, int width = kTP) {
  TileRS t;
  t.s0 = (int)(tile % ntx) * width;
  const int64_t q = tile / ntx;
  t.r = (int)(q % nrows);
  t.b = (int)(q / nrows);
  return t;
}


// Workgroups that fit on the current device at once for `kernel` (resident
// capacity: CUs x blocks per CU), cached per (kernel, device). Persistent
// kernels size their grid with it.
inline int resident_blocks(const void* kernel, int threads) {
  static std::mutex mu;
  static std::map<std::pair<const void*, int>, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_pair(kernel, dev);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess || per_cu < 1) per_cu = 1;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 1;
  cache[key] = per_cu * cus;
  return per_cu * cus;
}

// grid for a persistent kernel over ntiles tiles
inline unsigned persistent_grid(const void* kernel, int threads, int64_t ntiles) {
  const int64_t cap = resident_blocks(kernel, threads);
  const int64_t g = ntiles < cap ? ntiles : cap;
  return (unsigned)(g < 1 ? 1 : g);
}

}  // namespace tile
}  // namespace fjx
