// Flash triangle attention on MFMA.
//
// One wave owns one attention row i of the pair grid and 64 queries of one
// head; the ROWS waves of a workgroup own ROWS consecutive rows with the same
// head and query tile, so the [64 x 64] tile of the triangle bias -- shared by
// every row -- is staged once in LDS per key block and read by all of them.
//
// Everything is computed transposed so that each lane keeps one query:
//   S^T[key][q] = K[key][:] . Q[q][:]   (A = K fragment, B = Q fragment)
//   lane l holds S^T[16kt + 4g + r][16qt + l%16], g = l/16
// The online-softmax state (running max m, partial sum l) therefore lives in
// the lane of its query; only the block max needs a 4-lane reduction. The
// probabilities then feed the second product directly as the B operand,
//   O^T[d][q] += V^T[d][keys] . P^T[keys][q]
// with the 8 keys of lane group g in a 32-key chunk c taken as
// {32c + 4g + 0..3, 32c + 16 + 4g + 0..3} -- the keys that lane already holds
// -- and the V^T fragment loaded with the same key assignment.
// Scores are in log2 units: q carries scale*log2(e), the bias and mask bias
// are multiplied by log2(e), and exp2 is used.
#include "fjx_common.hpp"
#include "fjx_kernels.hpp"

namespace fjx {

constexpr int kQT = 64;   // queries per wave
constexpr int kKB = 64;   // keys per block
constexpr int kD = 32;    // head dim
constexpr int kNumXcdF = 8;

__device__ __forceinline__ int64_t xcd_remap_f(int64_t w, int64_t total) {
  const int64_t per = total / kNumXcdF;
  if (w >= per * kNumXcdF) return w;
  return (w % kNumXcdF) * per + w / kNumXcdF;
}

// 4 contiguous elements -> 4 fp32 / half of an 8-element fragment
__device__ __forceinline__ void load4_into(const bf16* p, bf16x8& f, int half) {
  const bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
#pragma unroll
  for (int e = 0; e < 4; ++e) f[4 * half + e] = v[e];
}
__device__ __forceinline__ void load4_into(const float* p, f32x8& f, int half) {
  const f32x4 v = *reinterpret_cast<const f32x4*>(p);
#pragma unroll
  for (int e = 0; e < 4; ++e) f[4 * half + e] = v[e];
}

template <typename T, int ROWS>
__global__ __launch_bounds__(64 * ROWS) void flash_tri_kernel(FlashParams<T> P) {
  __shared__ __attribute__((aligned(16))) float bias_s[kQT][kKB + 4];

  const int64_t n = P.n;
  const int64_t np = P.np;
  const int64_t H = P.heads;
  const int64_t QT = np / kQT;
  const int64_t RG = (P.rows + ROWS - 1) / ROWS;
  const int64_t total = (int64_t)gridDim.x;
  int64_t lid = xcd_remap_f(blockIdx.x, total);
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
  const int64_t q0 = qtile * kQT;

  const int64_t head_off = ((b * P.rows + i) * H + h) * np;  // in rows of length kD
  const T* Q = P.q + head_off * kD;
  const T* K = P.k + head_off * kD;
  const T* VT = P.vt + ((b * P.rows + i) * H * kD + h * kD) * np;
  const float* MB = P.mb + (b * P.rows + i) * np;
  const T* BIAS = P.bias + b * P.bias_stride_b + h * np * np;

  typedef typename Frag<T>::type FragT;
  FragT qf[4];
#pragma unroll
  for (int qt = 0; qt < 4; ++qt) qf[qt] = load8(Q + (q0 + 16 * qt + li) * kD + 8 * lg);

  float m[4], l[4];
  f32x4 o[2][4];
#pragma unroll
  for (int qt = 0; qt < 4; ++qt) {
    m[qt] = -1.0e30f;
    l[qt] = 0.f;
    o[0][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
    o[1][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  constexpr int NT = 64 * ROWS;
  constexpr int PER = kQT * kKB / NT;  // bias elements per thread per block

  for (int64_t k0 = 0; k0 < np; k0 += kKB) {
    __syncthreads();
    {
      const int e0 = t * PER;
      const int br = e0 / kKB;
      const int bc = e0 % kKB;
      const T* src = BIAS + (q0 + br) * np + k0 + bc;
#pragma unroll
      for (int c = 0; c < PER; c += 8) {
        float f[8];
        to_f32x8(load8(src + c), f);
        f32x4 lo = {f[0] * kLog2e, f[1] * kLog2e, f[2] * kLog2e, f[3] * kLog2e};
        f32x4 hi = {f[4] * kLog2e, f[5] * kLog2e, f[6] * kLog2e, f[7] * kLog2e};
        *reinterpret_cast<f32x4*>(&bias_s[br][bc + c]) = lo;
        *reinterpret_cast<f32x4*>(&bias_s[br][bc + c + 4]) = hi;
      }
    }
    __syncthreads();

    f32x4 s[4][4];  // [kt][qt]
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      const FragT kf = load8(K + (k0 + 16 * kt + li) * kD + 8 * lg);
      const f32x4 mbv = *reinterpret_cast<const f32x4*>(MB + k0 + 16 * kt + 4 * lg);
#pragma unroll
      for (int qt = 0; qt < 4; ++qt) {
        f32x4 init = *reinterpret_cast<const f32x4*>(&bias_s[16 * qt + li][16 * kt + 4 * lg]);
        init += mbv;
        mma(init, kf, qf[qt]);
        s[kt][qt] = init;
      }
    }

    // online softmax per query (one query per lane per qt)
#pragma unroll
    for (int qt = 0; qt < 4; ++qt) {
      float mx = s[0][qt][0];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[kt][qt][r]);
      mx = fmaxf(mx, shfl_xor(mx, 16));
      mx = fmaxf(mx, shfl_xor(mx, 32));
      const float mnew = fmaxf(m[qt], mx);
      const float alpha = __builtin_amdgcn_exp2f(m[qt] - mnew);
      m[qt] = mnew;
      float ls = 0.f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = __builtin_amdgcn_exp2f(s[kt][qt][r] - mnew);
          s[kt][qt][r] = p;
          ls += p;
        }
      l[qt] = l[qt] * alpha + ls;
      o[0][qt] *= alpha;
      o[1][qt] *= alpha;
    }

    // O^T += V^T P^T over two 32-key chunks
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      FragT vf[2];
#pragma unroll
      for (int dt = 0; dt < 2; ++dt) {
        const T* vrow = VT + (int64_t)(16 * dt + li) * np + k0 + 32 * c + 4 * lg;
        load4_into(vrow, vf[dt], 0);
        load4_into(vrow + 16, vf[dt], 1);
      }
#pragma unroll
      for (int qt = 0; qt < 4; ++qt) {
        float pv[8];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          pv[r] = s[2 * c][qt][r];
          pv[4 + r] = s[2 * c + 1][qt][r];
        }
        const FragT pf = pack8<T>(pv);
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) mma(o[dt][qt], vf[dt], pf);
      }
    }
  }

  if (!row_ok) return;
  T* OUT = P.out + b * P.o_stride_b + i * P.o_stride_row + h * P.o_stride_head;
  const T* G = P.gate ? P.gate + b * P.o_stride_b + i * P.o_stride_row + h * P.o_stride_head : nullptr;
#pragma unroll
  for (int qt = 0; qt < 4; ++qt) {
    float lt = l[qt];
    lt += shfl_xor(lt, 16);
    lt += shfl_xor(lt, 32);
    const float inv = 1.0f / lt;
    const int64_t q = q0 + 16 * qt + li;
    if (q >= n) continue;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
      const int64_t off = q * P.o_stride_q + 16 * dt + 4 * lg;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v = o[dt][qt][r] * inv;
        if (G) v *= to_f32(G[off + r]);
        OUT[off + r] = from_f32<T>(v);
      }
    }
  }
}

template <typename T>
void launch_flash(const FlashParams<T>& p, int64_t batch, hipStream_t st) {
  constexpr int ROWS = 4;
  const int64_t rg = (p.rows + ROWS - 1) / ROWS;
  const int64_t total = batch * p.heads * rg * (p.np / kQT);
  hipLaunchKernelGGL((flash_tri_kernel<T, ROWS>), dim3((unsigned)total), dim3(64 * ROWS), 0, st, p);
}

template void launch_flash<bf16>(const FlashParams<bf16>&, int64_t, hipStream_t);
template void launch_flash<float>(const FlashParams<float>&, int64_t, hipStream_t);

}  // namespace fjx
