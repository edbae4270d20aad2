// Flash triangle attention on MFMA.
//
// One wave owns one attention row i of the pair grid and 64 or 128 queries of
// one head; the ROWS waves of a workgroup own ROWS consecutive rows with the same
// head and query tile, so the [queries x 64] tile of the triangle bias -- shared by
// every row -- is staged once in LDS per key block (double-buffered, the next
// tile prefetched into registers while the current one is consumed) and read
// by all of them. Each row's mask bias for the block travels the same way.
//
// Memory pipeline per key block: at its top the wave issues the loads of the
// next block's V (into a second register set), bias tile and mask bias; after
// the last query tile has used K it issues the next block's K. Every prefetch
// is unconditional (the last block re-reads itself), so no path through the
// loop leaves a load outstanding at its top, and the in-order memory counter
// never makes a product wait for a prefetch issued after its own operands. Q
// lives in LDS (fragment order, conflict-free) to leave registers for V.
//
// Everything is computed transposed so that each lane keeps one query:
//   S^T[key][q] = K[key][:] . Q[q][:]   (A = K fragment, B = Q fragment)
//   lane l holds S^T[key_of(kt, 4g + r)][16qt + l%16], g = l/16
// with the accumulator initialised to the bias tile (plus the mask bias when
// the block holds masked keys). The K rows of a block are loaded in a
// permuted order (key_of below) so that lane group g ends up holding the 8
// consecutive keys 32c + 8g .. +7 of each 32-key chunk c: the probabilities
// then feed the second product directly as the B operand,
//   O^T[d][q] += V^T[d][keys] . P^T[keys][q]
// and each V^T fragment is one contiguous 16-byte load (an unpermuted order
// needs two 8-byte pieces per lane, twice the load instructions and cache-line
// touches, and the memory pipeline bounds this kernel). The
// online-softmax max lives in the lane of its query. The softmax
// denominator is a third product with an all-ones A operand, so the running
// sums cost MFMA cycles instead of VALU adds. The softmax offset of each query
// is lazy: it moves (rescaling O and the sums, behind a wave-uniform test)
// only when some score of the block exceeds it by more than 2^8 in
// probability.
// Scores are in log2 units: q carries scale*log2(e), and the bias and mask
// bias arrive multiplied by log2(e).
#include <type_traits>

#include "fjx_common.hpp"
#include "fjx_kernels.hpp"
#include "fjx_tile.hpp"

namespace fjx {

constexpr int kQT = 64;   // queries per wave
constexpr int kKB = 64;   // keys per block
constexpr int kD = 32;    // head dim
constexpr int kNumXcdF = 8;
constexpr int kBiasLd = kKB + 4;  // padded LDS row (floats)
constexpr float kLazy = 8.0f;     // running-max slack before a rescale (log2 units)

__device__ __forceinline__ int64_t xcd_remap_f(int64_t w, int64_t total) {
  const int64_t per = total / kNumXcdF;
  if (w >= per * kNumXcdF) return w;
  return (w % kNumXcdF) * per + w / kNumXcdF;
}

// Key order inside a 64-key block. Row i of the K tile kt holds key
//   key_of(kt, i) = 32 (kt/2) + 8 (i/4) + 4 (kt%2) + i%4,
// so accumulator row 4g + r of tile kt is key 32 (kt/2) + 8g + 4 (kt%2) + r:
// lane group g holds, for the 32-key chunk c = kt/2, the 8 consecutive keys
// 32c + 8g .. +7 -- one contiguous 16-byte V^T fragment per lane -- and its
// 4 bias / mask values of tile kt are 4 consecutive columns.
__device__ __forceinline__ int key_of(int kt, int i) { return 32 * (kt >> 1) + 8 * (i >> 2) + 4 * (kt & 1) + (i & 3); }
__device__ __forceinline__ int col_of(int kt, int g) { return 32 * (kt >> 1) + 8 * g + 4 * (kt & 1); }

// max over the 4 lanes {l%16 + 16g}
__device__ __forceinline__ float max_over_groups(float x) {
  const unsigned u = __float_as_uint(x);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const float y = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const unsigned v = __float_as_uint(y);
  const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// all eight elements 1 when `on`, else 0
template <typename T> __device__ __forceinline__ typename Frag<T>::type ones8(bool on);
template <> __device__ __forceinline__ bf16x8 ones8<bf16>(bool on) {
  const bf16 o = static_cast<bf16>(on ? 1.0f : 0.0f);
  return bf16x8{o, o, o, o, o, o, o, o};
}
template <> __device__ __forceinline__ f32x8 ones8<float>(bool on) {
  const float o = on ? 1.f : 0.f;
  return f32x8{o, o, o, o, o, o, o, o};
}

// NQT query tiles of 16 per wave: 4 (64 queries; Q fragments in LDS, one
// softmax-sum accumulator per tile) or 8 (128 queries: every K and V load
// serves twice the queries; Q in registers, and the sums of 4 tiles share an
// accumulator whose A operand is 1 only in rows 4(qt%4) .. +3, so lane group
// g holds the sums of tile 4(qt/4) + g -- padded queries have zero scores,
// so the zero-weighted rows add nothing)
// vb: the workgroup's index in the launch grid of `total` workgroups (its
// fallback flag and, through xcd_remap_f, its tile)
template <typename T, int ROWS, int NQT, bool FAST = false>
__device__ __forceinline__ void flash_tri_body(const FlashParams<T>& P, int64_t vb, int64_t total) {
  typedef typename Frag<T>::type FragT;
  constexpr int QTL = 16 * NQT;
  constexpr bool kQLds = NQT == 4;
  constexpr int NLS = kQLds ? 4 : NQT / 4;
  __shared__ __attribute__((aligned(16))) float bias_s[2][QTL][kBiasLd];
  __shared__ __attribute__((aligned(16))) FragT q_s[kQLds ? ROWS : 1][4][64];  // [wave][qt][lane]: B fragments of Q
  __shared__ __attribute__((aligned(16))) float mb_s[2][ROWS][kKB];  // each row's mask bias, one key block

  // the offset path after a FAST launch: only the workgroups it flagged
  if constexpr (!FAST) {
    if (P.fallback && P.fallback[vb] == 0u) return;
  }

  const int64_t n = P.n;
  const int64_t np = P.np;
  const int64_t H = P.heads;
  const int64_t QT = np / QTL;
  const int64_t RG = (P.rows + ROWS - 1) / ROWS;
  int64_t lid = xcd_remap_f(vb, total);
  const int64_t qtile = lid % QT;
  lid /= QT;
  const int64_t rg = lid % RG;
  lid /= RG;
  const int64_t h = lid % H;
  const int64_t b = lid / H;

  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int64_t row = rg * ROWS + wave;
  const bool row_ok = row < P.rows;
  const int64_t i = row_ok ? row : P.rows - 1;
  const int64_t q0 = qtile * QTL;

  const int64_t head_off = ((b * P.rows + i) * H + h) * np;  // in rows of length kD
  const T* Q = P.q + head_off * kD;
  const T* K = P.k + head_off * kD;
  const T* VT = P.vt + ((b * P.rows + i) * H * kD + h * kD) * np;
  const float* MB = P.mb + (b * P.rows + i) * np;
  const T* BIAS = P.bias + b * P.bias_stride_b + h * np * np;

  const int64_t nblk = np / kKB;

  // offset-free pass: a row with every key masked (no mask bias above -1e8)
  // would sum to 0. Its softmax is that of the unmasked scores (the mask is
  // the same constant on every key and cancels), so such a row drops the
  // masked keys' bias and keeps only the -inf of the padded keys.
  bool full_row = false;
  if constexpr (FAST) {
    // 16-byte loads over the whole padded row (np is a multiple of 128; the
    // padded keys hold -inf), four in flight per lane
    bool any_valid = false;
#pragma unroll 4
    for (int64_t k0 = 4 * lane; k0 < np; k0 += 256) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(MB + k0);
      any_valid |= (v[0] > -1.0e8f) | (v[1] > -1.0e8f) | (v[2] > -1.0e8f) | (v[3] > -1.0e8f);
    }
    full_row = __builtin_amdgcn_ballot_w64(any_valid) == 0;
  }

  // Q stays in LDS (in fragment order: conflict-free 16-byte reads) and is
  // re-read per key block, which leaves registers for a second V buffer
  FragT qreg[kQLds ? 1 : NQT];
  if constexpr (kQLds) {
#pragma unroll
    for (int qt = 0; qt < 4; ++qt) q_s[wave][qt][lane] = load8(Q + (q0 + 16 * qt + li) * kD + 8 * lg);
  } else {
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) qreg[qt] = load8(Q + (q0 + 16 * qt + li) * kD + 8 * lg);
  }

  float m[NQT];
  f32x4 o[2][NQT], lsum[NLS];
#pragma unroll
  for (int qt = 0; qt < NQT; ++qt) {
    m[qt] = -1.0e30f;
    o[0][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
    o[1][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int u = 0; u < NLS; ++u) lsum[u] = f32x4{0.f, 0.f, 0.f, 0.f};

  // bias tile fill: 8 threads cover one 64-key row (a whole cache line in
  // bf16), 64*ROWS/8 rows per pass
  constexpr int NT = 64 * ROWS;
  constexpr int RPP = NT / 8;             // rows per pass
  constexpr int PASSES = QTL / RPP;
  static_assert(PASSES * RPP == QTL, "bias tile fill");
  const int br = t >> 3;
  const int bc = 8 * (t & 7);
  const T* bsrc = BIAS + (q0 + br) * np + bc;
  // the next key block's bias tile and mask bias travel in registers and are
  // written to the other LDS buffer at the end of the current block; the
  // mask flag (any non-zero mask bias in this row's block) is wave-uniform
  typename Frag<T>::type breg[PASSES];
  float mbn;
  auto fetch_tile = [&](int64_t k0) {
#pragma unroll
    for (int c = 0; c < PASSES; ++c) breg[c] = load8(bsrc + (int64_t)RPP * c * np + k0);
    mbn = MB[k0 + lane];
  };
  auto put_tile = [&](int buf) {
#pragma unroll
    for (int c = 0; c < PASSES; ++c) {
      float f[8];
      to_f32x8(breg[c], f);
      *reinterpret_cast<f32x4*>(&bias_s[buf][br + RPP * c][bc]) = f32x4{f[0], f[1], f[2], f[3]};
      *reinterpret_cast<f32x4*>(&bias_s[buf][br + RPP * c][bc + 4]) = f32x4{f[4], f[5], f[6], f[7]};
    }
    mb_s[buf][wave][lane] = mbn;
    return __builtin_amdgcn_ballot_w64(mbn != 0.f) != 0;
  };
  fetch_tile(0);
  bool masked_blk = put_tile(0);

  FragT kf[4];
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) kf[kt] = load8(K + key_of(kt, li) * kD + 8 * lg);
  // V of the current block in vf, the next block's arriving in vn
  FragT vf[2][2], vn[2][2];  // [dt][c]
  auto load_v = [&](FragT (&v)[2][2], int64_t k0) {
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        v[dt][c] = load8(VT + (int64_t)(16 * dt + li) * np + k0 + 32 * c + 8 * lg);
      }
  };
  load_v(vf, 0);
  // drain every counter once here: the loop's own waits then see nothing
  // pending from before it (an outstanding pre-loop load would be waited on,
  // in issue order, behind the next block's prefetch)
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // one key block; V of this block in vc, the next block's loaded into vx
  auto key_block = [&](int64_t blk, FragT (&vc)[2][2], FragT (&vx)[2][2]) {
    const int buf = blk & 1;
    const int64_t k0 = blk * kKB;
    // prefetches run unconditionally (the last block re-reads itself), so
    // that no path through the loop leaves a load outstanding at its top
    const int64_t kn = blk + 1 < nblk ? k0 + kKB : k0;
    load_v(vx, kn);
    fetch_tile(kn);

#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
      FragT qf;
      if constexpr (kQLds) qf = q_s[wave][qt][lane];
      else qf = qreg[qt];
      f32x4 s[4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) s[kt] = *reinterpret_cast<const f32x4*>(&bias_s[buf][16 * qt + li][col_of(kt, lg)]);
      // blocks holding masked or padded keys add the mask bias (re-read per
      // query tile, a cache hit, so that it is not live across the block);
      // the test is wave-uniform, a scalar branch
      if (masked_blk) {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
          f32x4 mv = *reinterpret_cast<const f32x4*>(&mb_s[buf][wave][col_of(kt, lg)]);
          if (FAST && full_row) {
#pragma unroll
            for (int r = 0; r < 4; ++r) mv[r] = mv[r] < -1.0e30f ? mv[r] : 0.f;
          }
          s[kt] += mv;
        }
      }
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) mma(s[kt], kf[kt], qf);
      if (qt == NQT - 1) {
        // K of this block is consumed: fetch the next block's into the same registers
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) kf[kt] = load8(K + (kn + key_of(kt, li)) * kD + 8 * lg);
      }
      float pv[4][4];
      if constexpr (FAST) {
        // no offset: exp2 of the raw log2-unit score; overflow or underflow
        // of a whole row is caught after the last block
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) pv[kt][r] = __builtin_amdgcn_exp2f(s[kt][r]);
      } else {
      // this lane's 16 scores: a max3 tree (5 + 2 + 1)
      const float t0 = fmaxf(fmaxf(s[0][0], s[0][1]), s[0][2]);
      const float t1 = fmaxf(fmaxf(s[0][3], s[1][0]), s[1][1]);
      const float t2 = fmaxf(fmaxf(s[1][2], s[1][3]), s[2][0]);
      const float t3 = fmaxf(fmaxf(s[2][1], s[2][2]), s[2][3]);
      const float t4 = fmaxf(fmaxf(s[3][0], s[3][1]), s[3][2]);
      const float u0 = fmaxf(fmaxf(t0, t1), t2);
      const float u1 = fmaxf(fmaxf(t3, t4), s[3][3]);
      const float lmx = fmaxf(u0, u1);
      // lazy offset: m moves only when some score of the block exceeds it by
      // more than kLazy (log2 units), so exp2(s - m) <= 2^kLazy; the test
      // needs no cross-lane reduction, and the rescale (a wave-uniform
      // branch, rare after the first block) takes the exact block max of
      // each query over its 4 lane groups
      if (__builtin_amdgcn_ballot_w64(lmx > m[qt] + kLazy) != 0) {
        const float mnew = fmaxf(m[qt], max_over_groups(lmx));
        const float alpha = __builtin_amdgcn_exp2f(m[qt] - mnew);
        o[0][qt] *= alpha;
        o[1][qt] *= alpha;
        if constexpr (kQLds) lsum[qt] *= alpha;
        else lsum[qt >> 2] *= lg == (qt & 3) ? alpha : 1.0f;
        m[qt] = mnew;
      }
      const float mnew = m[qt];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) pv[kt][r] = __builtin_amdgcn_exp2f(s[kt][r] - mnew);
      }
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const float f[8] = {pv[2 * c][0], pv[2 * c][1], pv[2 * c][2], pv[2 * c][3],
                            pv[2 * c + 1][0], pv[2 * c + 1][1], pv[2 * c + 1][2], pv[2 * c + 1][3]};
        const FragT pf = pack8<T>(f);
        mma(o[0][qt], vc[0][c], pf);
        mma(o[1][qt], vc[1][c], pf);
        if constexpr (kQLds) mma(lsum[qt], ones8<T>(true), pf);
        else mma(lsum[qt >> 2], ones8<T>((li >> 2) == (qt & 3)), pf);
      }
    }

    masked_blk = put_tile(buf ^ 1);
    __syncthreads();
  };
  // unrolled by two so that the V register sets alternate instead of being copied
  for (int64_t blk = 0;;) {
    key_block(blk, vf, vn);
    if (++blk >= nblk) break;
    key_block(blk, vn, vf);
    if (++blk >= nblk) break;
  }

  if (!row_ok) return;
  if constexpr (FAST) {
    // every softmax sum in [2^-100, inf) and every output finite, checked on
    // the bit patterns (this file is compiled without NaN semantics);
    // otherwise the workgroup is left to the offset path
    bool bad = false;
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
      float ls;
      if constexpr (kQLds) ls = lsum[qt][0];
      else ls = __shfl(lsum[qt >> 2][0], 16 * (qt & 3) + li, 64);
      const unsigned u = __float_as_uint(ls);
      bad |= !(u >= 0x0D800000u && u < 0x7F800000u);
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) bad |= (__float_as_uint(o[dt][qt][r]) & 0x7F800000u) == 0x7F800000u;
    }
    if (__builtin_amdgcn_ballot_w64(bad) != 0) {
      if (lane == 0) P.fallback[vb] = 1u;
      return;
    }
  }
  T* OUT = P.out + b * P.o_stride_b + i * P.o_stride_row + h * P.o_stride_head;
#pragma unroll
  for (int qt = 0; qt < NQT; ++qt) {
    float ls;
    if constexpr (kQLds) ls = lsum[qt][0];
    else ls = __shfl(lsum[qt >> 2][0], 16 * (qt & 3) + li, 64);
    const float inv = 1.0f / ls;
    const int64_t q = q0 + 16 * qt + li;
    if (q >= n) continue;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = o[dt][qt][r] * inv;
      // 4 consecutive head dims; every o_stride_* is a multiple of 4
      store4f(OUT + q * P.o_stride_q + 16 * dt + 4 * lg, v);
    }
  }
}

constexpr int kRows = 4;

// 128 queries per wave (bf16, np a multiple of 128): 256 VGPRs, 2 waves per
// SIMD, 72 KB of LDS (two workgroups per CU); measured a few percent faster
// than 64 queries at 3 waves per SIMD, as each K and V load serves twice the
// queries
__global__ __launch_bounds__(64 * kRows) __attribute__((amdgpu_waves_per_eu(2, 2))) void flash_tri8_kernel_bf16(FlashParams<bf16> P) {
  flash_tri_body<bf16, kRows, 8>(P, blockIdx.x, gridDim.x);
}

// The same kernel as the fallback of the pipelined pass, over that pass's
// grid of `total` workgroups: workgroup w reads the flags of `per`
// consecutive ones (64 a load) and recomputes the flagged ones. Launched with
// no more workgroups than the GPU holds at once, it costs few short
// workgroups when nothing is flagged and, when everything is, as many rounds
// of resident workgroups as the full grid would.
__global__ __launch_bounds__(64 * kRows) __attribute__((amdgpu_waves_per_eu(2, 2)))
void flash_tri8_redo_kernel_bf16(FlashParams<bf16> P, int64_t total, int64_t per) {
  const int64_t base = (int64_t)blockIdx.x * per;
  const int lane = threadIdx.x & 63;
  for (int64_t c0 = 0; c0 < per; c0 += 64) {
    const int64_t vb = base + c0 + lane;
    const bool f = c0 + lane < per && vb < total && P.fallback[vb] != 0u;
    uint64_t m = __builtin_amdgcn_ballot_w64(f);  // the same in every wave
    while (m != 0) {
      const int k = __builtin_ctzll(m);
      m &= m - 1;
      flash_tri_body<bf16, kRows, 8>(P, base + c0 + k, total);
      __syncthreads();  // LDS is reused by the next flagged workgroup
    }
  }
}

// The same 128-query kernel without a softmax offset: p = exp2(s) straight
// from the log2-unit scores, so no running max, no subtraction and no rescale
// branch per query tile. Softmax is invariant to the offset, and exp2 of any
// score in [-126, 127] is a normal float whose bf16 rounding is the same
// relative error as with an offset; a row whose scores leave that range (or a
// row with every key masked, whose sums underflow to 0) shows up as a sum
// below 2^-100 or a non-finite value after its last block, and its workgroup
// is then recomputed by the offset kernel above.
__global__ __launch_bounds__(64 * kRows) __attribute__((amdgpu_waves_per_eu(2, 2))) void flash_tri8_fast_kernel_bf16(FlashParams<bf16> P) {
  flash_tri_body<bf16, kRows, 8, true>(P, blockIdx.x, gridDim.x);
}

__global__ void zero_flags_kernel(unsigned* __restrict__ f, int64_t count) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x)
    f[i] = 0u;
}

// bf16: 3 waves per SIMD (168 VGPRs) measured faster than 2 without spills;
// the fp32 variant would spill heavily under that cap and keeps 2.
__global__ __launch_bounds__(64 * kRows) __attribute__((amdgpu_waves_per_eu(3, 3)))
void flash_tri_kernel_bf16(FlashParams<bf16> P) {
  flash_tri_body<bf16, kRows, 4>(P, blockIdx.x, gridDim.x);
}
// its offset-free pass (as flash_tri8_fast_kernel_bf16)
__global__ __launch_bounds__(64 * kRows) __attribute__((amdgpu_waves_per_eu(3, 3)))
void flash_tri_fast_kernel_bf16(FlashParams<bf16> P) {
  flash_tri_body<bf16, kRows, 4, true>(P, blockIdx.x, gridDim.x);
}
__global__ __launch_bounds__(64 * kRows) void flash_tri_kernel_f32(FlashParams<float> P) {
  flash_tri_body<float, kRows, 4>(P, blockIdx.x, gridDim.x);
}

template <typename T>
void launch_flash(const FlashParams<T>& p_in, int64_t batch, hipStream_t st) {
  const int64_t rg = (p_in.rows + kRows - 1) / kRows;
  const dim3 grid((unsigned)(batch * p_in.heads * rg * (p_in.np / kQT)));
  // one row (the single-track attention, a bias per head): the keys are split
  // over the waves of a workgroup instead (fjx_single_flash.hip)
  if (p_in.rows == 1) {
    launch_flash_single<T>(p_in, batch, st);
    return;
  }
  // the offset kernels skip unflagged workgroups whenever `fallback` is set,
  // so it stays set only where an offset-free pass fills the flags first
  FlashParams<T> plain = p_in;
  plain.fallback = nullptr;
  if constexpr (std::is_same<T, bf16>::value) {
    const FlashParams<T>& p = p_in;
    const bool q128 = p.np % 128 == 0;
    const dim3 g = q128 ? dim3((unsigned)(batch * p.heads * rg * (p.np / 128))) : grid;
    if (p.fallback) {
      // the pipelined pass writes every flag in the 128-query grid of the
      // offset kernel; the offset kernel then redoes the flagged workgroups
      if (q128 && launch_flash_pipe(p, batch, st)) {
        const int64_t total = g.x;
        const int64_t cap = tile::resident_blocks(reinterpret_cast<const void*>(&flash_tri8_redo_kernel_bf16), 64 * kRows);
        const int64_t per = (total + cap - 1) / cap;
        hipLaunchKernelGGL(flash_tri8_redo_kernel_bf16, dim3((unsigned)((total + per - 1) / per)), dim3(64 * kRows), 0,
                           st, p, total, per);
        return;
      }
      // offset-free pass, then the offset kernel for the workgroups it flagged
      const int64_t nb = ((int64_t)g.x + 255) / 256;
      hipLaunchKernelGGL(zero_flags_kernel, dim3((unsigned)(nb < 4096 ? nb : 4096)), dim3(256), 0, st, p.fallback,
                         (int64_t)g.x);
      hipLaunchKernelGGL(q128 ? flash_tri8_fast_kernel_bf16 : flash_tri_fast_kernel_bf16, g, dim3(64 * kRows), 0, st,
                         p);
    }
    hipLaunchKernelGGL(q128 ? flash_tri8_kernel_bf16 : flash_tri_kernel_bf16, g, dim3(64 * kRows), 0, st, p);
  } else
    hipLaunchKernelGGL(flash_tri_kernel_f32, grid, dim3(64 * kRows), 0, st, plain);
}

template void launch_flash<bf16>(const FlashParams<bf16>&, int64_t, hipStream_t);
template void launch_flash<float>(const FlashParams<float>&, int64_t, hipStream_t);

}  // namespace fjx
