// Triangle contraction: for every (batch, channel) an independent N x N x N
// product with both operands k-contiguous,
//     out[i][j] = sum_k a[i][k] * b[j][k]
// The prologue lays a and b out channel-major with the contracted index
// innermost (the incoming direction is prepared in the transposed grid), so
// one "NT" kernel serves both directions.
//
// Tiling: 128 x 128 output tile per 256-thread workgroup, 2 x 2 waves of
// 64 x 64 (4 x 4 MFMA tiles of 16 x 16), k-tiles of BK staged through LDS with
// a register prefetch of the next k-tile. Blocks are numbered so that all
// tiles of one channel land on one XCD (workgroups are dealt round-robin over
// the 8 XCDs), keeping that channel's a and b in the XCD's L2.
#include "fjx_common.hpp"
#include "fjx_kernels.hpp"

namespace fjx {

constexpr int kBM = 128;
constexpr int kNumXcd = 8;

template <typename T> struct ContractCfg;
template <> struct ContractCfg<bf16> { static constexpr int BK = 64; };
template <> struct ContractCfg<float> { static constexpr int BK = 32; };

// Map hardware block id -> logical tile id so that consecutive logical ids run
// on the same XCD. Bijective on [0, total).
__device__ __forceinline__ int64_t xcd_remap(int64_t w, int64_t total) {
  const int64_t per = total / kNumXcd;
  if (w >= per * kNumXcd) return w;
  return (w % kNumXcd) * per + w / kNumXcd;
}

template <typename T, typename TO>
__global__ __launch_bounds__(256) void contract_nt_kernel(ContractParams<T, TO> P) {
  constexpr int BK = ContractCfg<T>::BK;
  constexpr int LD = BK + 8;                  // padded LDS row (elements)
  constexpr int CHUNKS = kBM * BK / 8;        // 8-element chunks per operand tile
  constexpr int PER_T = CHUNKS / 256;         // chunks per thread per operand
  __shared__ __attribute__((aligned(16))) T As[2][kBM][LD];
  __shared__ __attribute__((aligned(16))) T Bs[2][kBM][LD];

  const int64_t n = P.n;
  const int64_t tiles = (n + kBM - 1) / kBM;
  const int64_t total = P.batches * tiles * tiles;
  const int64_t lid = xcd_remap(blockIdx.x, total);
  const int64_t bc = lid / (tiles * tiles);
  const int64_t tile = lid % (tiles * tiles);
  const int64_t m0 = (tile / tiles) * kBM;
  const int64_t n0 = (tile % tiles) * kBM;

  const T* A = P.a + bc * n * n;
  const T* B = P.b + bc * n * n;
  const int t = threadIdx.x;
  const bool aligned = (n % 8) == 0;

  typename Frag<T>::type ra[PER_T], rb[PER_T];

  auto load_tile = [&](int64_t k0) {
#pragma unroll
    for (int it = 0; it < PER_T; ++it) {
      const int c = t + 256 * it;
      const int row = c / (BK / 8);
      const int kc = (c % (BK / 8)) * 8;
      const int64_t gk = k0 + kc;
      const int64_t ga = m0 + row;
      const int64_t gb = n0 + row;
      if (aligned && gk + 8 <= n) {
        if (ga < n) ra[it] = load8(A + ga * n + gk);
        else ra[it] = typename Frag<T>::type{};
        if (gb < n) rb[it] = load8(B + gb * n + gk);
        else rb[it] = typename Frag<T>::type{};
      } else {
        float fa[8], fb[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const bool kin = gk + e < n;
          fa[e] = (kin && ga < n) ? to_f32(A[ga * n + gk + e]) : 0.f;
          fb[e] = (kin && gb < n) ? to_f32(B[gb * n + gk + e]) : 0.f;
        }
        ra[it] = pack8<T>(fa);
        rb[it] = pack8<T>(fb);
      }
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int it = 0; it < PER_T; ++it) {
      const int c = t + 256 * it;
      const int row = c / (BK / 8);
      const int kc = (c % (BK / 8)) * 8;
      store8(&As[buf][row][kc], ra[it]);
      store8(&Bs[buf][row][kc], rb[it]);
    }
  };

  const int wave = t >> 6;
  const int lane = t & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int wm = (wave >> 1) * 64;
  const int wn = (wave & 1) * 64;

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int64_t ktiles = (n + BK - 1) / BK;
  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (int64_t kt = 0; kt < ktiles; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < ktiles) load_tile((kt + 1) * BK);
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      typename Frag<T>::type af[4], bf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) af[i] = load8(&As[buf][wm + 16 * i + li][32 * ks + 8 * lg]);
#pragma unroll
      for (int j = 0; j < 4; ++j) bf[j] = load8(&Bs[buf][wn + 16 * j + li][32 * ks + 8 * lg]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) mma(acc[i][j], af[i], bf[j]);
    }
    if (kt + 1 < ktiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  TO* O = P.out + bc * n * n;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t col = n0 + wn + 16 * j + li;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t row = m0 + wm + 16 * i + 4 * lg + q;
        if (row < n && col < n) O[row * n + col] = from_f32<TO>(acc[i][j][q]);
      }
    }
}

template <typename T, typename TO>
void launch_contract(const ContractParams<T, TO>& p, hipStream_t st) {
  const int64_t tiles = (p.n + kBM - 1) / kBM;
  const int64_t total = p.batches * tiles * tiles;
  hipLaunchKernelGGL((contract_nt_kernel<T, TO>), dim3((unsigned)total), dim3(256), 0, st, p);
}

template void launch_contract<bf16, bf16>(const ContractParams<bf16, bf16>&, hipStream_t);
template void launch_contract<float, float>(const ContractParams<float, float>&, hipStream_t);

}  // namespace fjx
