// Flash attention for the single-track attention with pair bias (one row:
// FlashParams::rows == 1), the bias per head. The triangle kernels give each
// wave a row of the pair grid; here there is one row, so the waves of a
// workgroup split the keys instead: a workgroup owns 32 queries of one
// (batch, head), each of its 4 waves runs the online softmax over a quarter
// of the 64-key blocks, and the four partial (max, sum, output) triples are
// merged through LDS. At N = 1024 and 16 heads that is 2048 waves, where one
// wave per row and 64 queries would give 256.
//
// Layouts as for the triangle kernels (fjx_kernels.hpp FlashParams): q, k
// [B][1][H][Np][32] (q pre-scaled by D^-1/2 log2 e), vt [B][1][H*32][Np],
// bias [B][H][Np][Np] times log2 e, mb [B][1][Np] fp32 times log2 e (-inf on
// padded keys). K rows are loaded in the permuted key order of the triangle
// kernels, so each lane's score accumulators hold 8 consecutive keys of one
// query, exactly the P fragment of the P V product.
#include "fjx_common.hpp"
#include "fjx_kernels.hpp"

namespace fjx {

namespace {

constexpr int kSD = 32;      // head dim (padded)
constexpr int kSKB = 64;     // keys per block
constexpr int kSQT = 2;      // query tiles of 16 per wave
constexpr int kSQ = 16 * kSQT;
constexpr int kSWaves = 4;

// key of accumulator row i of key tile kt: lane group g holds the keys
// 32 (kt/2) + 8g + 4 (kt%2) + 0..3
__device__ __forceinline__ int skey(int kt, int i) { return 32 * (kt >> 1) + 8 * (i >> 2) + 4 * (kt & 1) + (i & 3); }

template <typename T>
__device__ __forceinline__ void flash_single_body(const FlashParams<T>& P) {
  __shared__ float m_s[kSWaves][kSQ];
  __shared__ float l_s[kSWaves][kSQ];
  __shared__ float o_s[kSWaves][kSQ][kSD + 1];

  const int64_t np = P.np;
  const int64_t H = P.heads;
  const int64_t QB = np / kSQ;
  int64_t lid = blockIdx.x;
  const int64_t qb = lid % QB;
  lid /= QB;
  const int64_t h = lid % H;
  const int64_t b = lid / H;
  const int64_t q0 = qb * kSQ;

  const int t = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int lane = t & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;

  const T* Q = P.q + ((b * H + h) * np) * kSD;
  const T* K = P.k + ((b * H + h) * np) * kSD;
  const T* VT = P.vt + (b * H * kSD + h * kSD) * np;
  const float* MB = P.mb + b * np;
  const T* BIAS = P.bias + b * P.bias_stride_b + h * np * np;

  typename Frag<T>::type qf[kSQT];
#pragma unroll
  for (int qt = 0; qt < kSQT; ++qt) qf[qt] = load8(Q + (q0 + 16 * qt + li) * kSD + 8 * lg);

  float m[kSQT], l[kSQT];
  f32x4 o[2][kSQT];
#pragma unroll
  for (int qt = 0; qt < kSQT; ++qt) {
    m[qt] = -INFINITY;
    l[qt] = 0.f;
    o[0][qt] = o[1][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const int64_t nblk = np / kSKB;
  for (int64_t kb = wave; kb < nblk; kb += kSWaves) {
    const int64_t k0 = kb * kSKB;
    typename Frag<T>::type kf[4], vf[2][2];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) kf[kt] = load8(K + (k0 + skey(kt, li)) * kSD + 8 * lg);
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int c = 0; c < 2; ++c) vf[dt][c] = load8(VT + (16 * dt + li) * np + k0 + 32 * c + 8 * lg);
    float mb[4][4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(MB + k0 + skey(kt, 4 * lg));
#pragma unroll
      for (int r = 0; r < 4; ++r) mb[kt][r] = v[r];
    }
#pragma unroll
    for (int qt = 0; qt < kSQT; ++qt) {
      const int64_t q = q0 + 16 * qt + li;
      f32x4 s[4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        s[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
        mma(s[kt], kf[kt], qf[qt]);
        float bv[4];
        load4f(BIAS + q * np + k0 + skey(kt, 4 * lg), bv);
#pragma unroll
        for (int r = 0; r < 4; ++r) s[kt][r] += bv[r] + mb[kt][r];
      }
      float bm = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) bm = fmaxf(bm, s[kt][r]);
      bm = fmaxf(bm, shfl_xor(bm, 16));
      bm = fmaxf(bm, shfl_xor(bm, 32));
      const float mn = fmaxf(m[qt], bm);
      const float base = mn == -INFINITY ? 0.f : mn;  // every key so far masked out: all weights 0
      const float alpha = __builtin_amdgcn_exp2f(m[qt] - base);
      m[qt] = mn;
      float p[4][4];
      float ps = 0.f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          p[kt][r] = __builtin_amdgcn_exp2f(s[kt][r] - base);
          ps += p[kt][r];
        }
      l[qt] = l[qt] * alpha + ps;
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) o[dt][qt][r] *= alpha;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        float pf8[8];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          pf8[r] = p[2 * c][r];
          pf8[4 + r] = p[2 * c + 1][r];
        }
        const typename Frag<T>::type pf = pack8<T>(pf8);
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) mma(o[dt][qt], vf[dt][c], pf);
      }
    }
  }

  // per-lane partial sums -> the query's sum over this wave's keys
#pragma unroll
  for (int qt = 0; qt < kSQT; ++qt) {
    l[qt] += shfl_xor(l[qt], 16);
    l[qt] += shfl_xor(l[qt], 32);
    if (lg == 0) {
      m_s[wave][16 * qt + li] = m[qt];
      l_s[wave][16 * qt + li] = l[qt];
    }
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) o_s[wave][16 * qt + li][16 * dt + 4 * lg + r] = o[dt][qt][r];
  }
  __syncthreads();

  // merge: thread t owns query t/8 and head dims 4 (t%8) .. +3
  const int qq = t >> 3;
  const int d0 = 4 * (t & 7);
  float mx = -INFINITY;
#pragma unroll
  for (int w = 0; w < kSWaves; ++w) mx = fmaxf(mx, m_s[w][qq]);
  float L = 0.f, O[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int w = 0; w < kSWaves; ++w) {
    const float sc = m_s[w][qq] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_s[w][qq] - mx);
    L += sc * l_s[w][qq];
#pragma unroll
    for (int e = 0; e < 4; ++e) O[e] += sc * o_s[w][qq][d0 + e];
  }
  const int64_t q = q0 + qq;
  if (q >= P.n) return;
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  float y[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) y[e] = O[e] * inv;
  store4f(P.out + b * P.o_stride_b + q * P.o_stride_q + h * P.o_stride_head + d0, y);
}

}  // namespace

__global__ __launch_bounds__(64 * kSWaves) void flash_single_kernel_bf16(FlashParams<bf16> P) {
  flash_single_body<bf16>(P);
}
__global__ __launch_bounds__(64 * kSWaves) void flash_single_kernel_f32(FlashParams<float> P) {
  flash_single_body<float>(P);
}

template <typename T>
void launch_flash_single(const FlashParams<T>& p, int64_t batch, hipStream_t st) {
  const dim3 grid((unsigned)(batch * p.heads * (p.np / kSQ)));
  if constexpr (std::is_same<T, bf16>::value)
    hipLaunchKernelGGL(flash_single_kernel_bf16, grid, dim3(64 * kSWaves), 0, st, p);
  else
    hipLaunchKernelGGL(flash_single_kernel_f32, grid, dim3(64 * kSWaves), 0, st, p);
}

template void launch_flash_single<bf16>(const FlashParams<bf16>&, int64_t, hipStream_t);
template void launch_flash_single<float>(const FlashParams<float>&, int64_t, hipStream_t);

}  // namespace fjx
