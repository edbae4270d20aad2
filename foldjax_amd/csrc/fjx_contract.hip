// Batched "NT" GEMM on MFMA: for every batch b
//     C[i][j] = epilogue( sum_k A[i][k] * B[j][k] )
// with both operands k-contiguous. It is the triangle contraction (one batch
// per (batch, channel), M = N = K = N_tok, a and b laid out channel-major with
// the contracted index innermost; the incoming direction is prepared in the
// transposed grid, so one kernel serves both directions) and the plain
// x W^T projections of the single track (B = a PyTorch [out, in] weight).
//
// Epilogue, in order: + bias[j], sigmoid, * gate[i][j], + residual[i][j].
//
// Tiling: 128 x 128 output tile per 256-thread workgroup, 2 x 2 waves of
// 64 x 64 (4 x 4 MFMA tiles of 16 x 16) -- 64 x 64 tiles when the problem has
// too few 128-tiles to occupy the GPU -- k-tiles of BK staged through LDS with
// a register prefetch of the next k-tile. Blocks are numbered so that all
// tiles of one batch land on one XCD (workgroups are dealt round-robin over
// the 8 XCDs), keeping that batch's operands in the XCD's L2.
#include <algorithm>

#include "fjx_common.hpp"
#include "fjx_kernels.hpp"
#include "fjx_tile.hpp"

namespace fjx {

constexpr int kNumXcd = 8;
constexpr int64_t kOBlk = 256;  // positions per block of the tile-blocked output

template <typename T> struct GemmCfg;
template <> struct GemmCfg<bf16> { static constexpr int BK = 64; };
template <> struct GemmCfg<float> { static constexpr int BK = 32; };

// Map hardware block id -> logical tile id so that consecutive logical ids run
// on the same XCD. Bijective on [0, total).
__device__ __forceinline__ int64_t xcd_remap(int64_t w, int64_t total) {
  const int64_t per = total / kNumXcd;
  if (w >= per * kNumXcd) return w;
  return (w % kNumXcd) * per + w / kNumXcd;
}

// BM x BM output tile per 256-thread workgroup (BM = 128, or 64 for small
// problems that would otherwise leave most CUs idle, or 32 for small fp32
// problems), 2 x 2 waves of (BM/2) x (BM/2). The 32-wide tile stages k-tiles
// of 64 so that each of the 256 threads still fills one 8-element chunk per
// operand; the k order of every accumulation is the same for all three tile
// sizes, so they give bit-identical results.
template <typename T, typename TO, int kBM>
__global__ __launch_bounds__(256) void gemm_nt_kernel(GemmParams<T, TO> P) {
  constexpr int BK = kBM == 32 ? 64 : GemmCfg<T>::BK;
  constexpr int LD = BK + 8;                  // padded LDS row (elements)
  constexpr int CHUNKS = kBM * BK / 8;        // 8-element chunks per operand tile
  constexpr int PER_T = CHUNKS / 256;         // chunks per thread per operand
  constexpr int WT = kBM / 32;                // 16 x 16 MFMA tiles per wave and dimension
  static_assert(PER_T >= 1 && PER_T * 256 == CHUNKS, "tile fill");
  __shared__ __attribute__((aligned(16))) T As[2][kBM][LD];
  __shared__ __attribute__((aligned(16))) T Bs[2][kBM][LD];

  const int64_t M = P.m, N = P.n, K = P.k;
  const int64_t tm = (M + kBM - 1) / kBM;
  const int64_t tn = (N + kBM - 1) / kBM;
  const int64_t total = P.batches * tm * tn;
  const int64_t lid = xcd_remap(blockIdx.x, total);
  const int64_t bat = lid / (tm * tn);
  const int64_t tile = lid % (tm * tn);
  const int64_t m0 = (tile / tn) * kBM;
  const int64_t n0 = (tile % tn) * kBM;

  const T* A = P.a + bat * P.sa;
  const T* B = P.b + bat * P.sb;
  const int t = threadIdx.x;
  const bool aligned = (K % 8) == 0 && (P.lda % 8) == 0 && (P.ldb % 8) == 0;

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
      if (aligned && gk + 8 <= K) {
        if (ga < M) ra[it] = load8(A + ga * P.lda + gk);
        else ra[it] = typename Frag<T>::type{};
        if (gb < N) rb[it] = load8(B + gb * P.ldb + gk);
        else rb[it] = typename Frag<T>::type{};
      } else {
        float fa[8], fb[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const bool kin = gk + e < K;
          fa[e] = (kin && ga < M) ? to_f32(A[ga * P.lda + gk + e]) : 0.f;
          fb[e] = (kin && gb < N) ? to_f32(B[gb * P.ldb + gk + e]) : 0.f;
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
  const int wm = (wave >> 1) * (kBM / 2);
  const int wn = (wave & 1) * (kBM / 2);

  f32x4 acc[WT][WT];
#pragma unroll
  for (int i = 0; i < WT; ++i)
#pragma unroll
    for (int j = 0; j < WT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int64_t ktiles = (K + BK - 1) / BK;
  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (int64_t kt = 0; kt < ktiles; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < ktiles) load_tile((kt + 1) * BK);
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      typename Frag<T>::type af[WT], bf[WT];
#pragma unroll
      for (int i = 0; i < WT; ++i) af[i] = load8(&As[buf][wm + 16 * i + li][32 * ks + 8 * lg]);
#pragma unroll
      for (int j = 0; j < WT; ++j) bf[j] = load8(&Bs[buf][wn + 16 * j + li][32 * ks + 8 * lg]);
#pragma unroll
      for (int i = 0; i < WT; ++i)
#pragma unroll
        for (int j = 0; j < WT; ++j) mma(acc[i][j], af[i], bf[j]);
    }
    if (kt + 1 < ktiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  TO* O = P.c + bat * P.sc;
  const TO* G = P.gate ? P.gate + bat * P.sc : nullptr;
  const TO* R = P.residual ? P.residual + bat * P.sc : nullptr;
#pragma unroll
  for (int i = 0; i < WT; ++i)
#pragma unroll
    for (int j = 0; j < WT; ++j) {
      const int64_t col = n0 + wn + 16 * j + li;
      if (col >= N) continue;
      const float bias = P.bias && (P.bias_n == 0 || col < P.bias_n) ? to_f32(P.bias[col]) : 0.f;
      const int act = col >= P.act_col0 ? P.act : 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t row0 = m0 + wm + 16 * i + 4 * lg + q;
        if (row0 >= M) continue;
        const int64_t row = grid_row(row0, P.map_n, P.map_t);
        float v = acc[i][j][q] + bias;
        if (act == 1) v = fast_sigmoid(v);
        else if (act == 2) v *= fast_sigmoid(v);  // silu
        const int64_t off = row * P.ldc + col;
        if (G) v *= to_f32(G[off]);
        if (P.proj_round) {
          v = round_to<TO>(v);
          if (P.row_scale) v = round_to<TO>(v * to_f32(P.row_scale[row]));
        }
        if (R) v += to_f32(R[off]);
        if (P.row_gate && to_f32(P.row_gate[row]) == 0.f) v *= 0.f;
        O[off] = from_f32<TO>(v);
      }
    }
}

// ---------------------------------------------------------------------------
// Triangle contraction, bf16: for every batch c, O[c] = A[c] B[c]^T with all
// three n x n and k-contiguous (channel-major a and b of the tri-mul).
// 256 x 256 output tile per 512-thread workgroup, 2 x 4 waves of 128 x 64;
// k-tiles of 64 double-buffered in LDS with a register prefetch of the next
// one. The accumulators are computed transposed (A operand = B rows) so each
// lane ends up holding 4 consecutive output columns of one row.
// ---------------------------------------------------------------------------
constexpr int kCT = 256;
constexpr int kCK = 64;
constexpr int kCLd = kCK + 8;

__global__ __launch_bounds__(512) void contract_kernel(const bf16* __restrict__ A, const bf16* __restrict__ B,
                                                       bf16* __restrict__ O, int64_t n, int64_t batches) {
  __shared__ __attribute__((aligned(16))) bf16 As[2][kCT][kCLd];
  __shared__ __attribute__((aligned(16))) bf16 Bs[2][kCT][kCLd];

  const int64_t tpd = (n + kCT - 1) / kCT;
  const int64_t total = batches * tpd * tpd;
  const int64_t lid = xcd_remap(blockIdx.x, total);
  const int64_t bat = lid / (tpd * tpd);
  const int64_t tile = lid % (tpd * tpd);
  const int64_t m0 = (tile / tpd) * kCT;
  const int64_t n0 = (tile % tpd) * kCT;
  const bf16* Ab = A + bat * n * n;
  const bf16* Bb = B + bat * n * n;

  const int t = threadIdx.x;
  const int wave = t >> 6;
  const int lane = t & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int wm = (wave >> 2) * 128;
  const int wn = (wave & 3) * 64;
  const bool vec = (n % 8) == 0;

  // global -> registers -> LDS: 256 rows x 8 chunks of 8 per operand, 4 chunks per thread
  bf16x8 ra[4], rb[4];
  auto load_stage = [&](int64_t k0) {
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int c = t + 512 * it;
      const int row = c >> 3;
      const int64_t gk = k0 + (c & 7) * 8;
      const int64_t ga = m0 + row;
      const int64_t gb = n0 + row;
      if (vec && gk + 8 <= n) {
        ra[it] = ga < n ? load8(Ab + ga * n + gk) : bf16x8{};
        rb[it] = gb < n ? load8(Bb + gb * n + gk) : bf16x8{};
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const bool kin = gk + e < n;
          ra[it][e] = (kin && ga < n) ? Ab[ga * n + gk + e] : static_cast<bf16>(0.f);
          rb[it][e] = (kin && gb < n) ? Bb[gb * n + gk + e] : static_cast<bf16>(0.f);
        }
      }
    }
  };
  auto store_stage = [&](int buf) {
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int c = t + 512 * it;
      store8(&As[buf][c >> 3][(c & 7) * 8], ra[it]);
      store8(&Bs[buf][c >> 3][(c & 7) * 8], rb[it]);
    }
  };

  f32x4 acc[4][8];  // [j: 16-column tile][i: 16-row tile], transposed: lane holds C[row 16i + l%16][col 16j + 4g + q]
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[j][i] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int64_t ktiles = (n + kCK - 1) / kCK;
  load_stage(0);
  store_stage(0);
  __syncthreads();
  for (int64_t kt = 0; kt < ktiles; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < ktiles) load_stage((kt + 1) * kCK);
#pragma unroll
    for (int ks = 0; ks < kCK / 32; ++ks) {
      bf16x8 af[8], bfr[4];
#pragma unroll
      for (int i = 0; i < 8; ++i) af[i] = load8(&As[buf][wm + 16 * i + li][32 * ks + 8 * lg]);
#pragma unroll
      for (int j = 0; j < 4; ++j) bfr[j] = load8(&Bs[buf][wn + 16 * j + li][32 * ks + 8 * lg]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) mma(acc[j][i], bfr[j], af[i]);
    }
    if (kt + 1 < ktiles) store_stage(buf ^ 1);
    __syncthreads();
  }

  bf16* Ob = O + bat * n * n;
  const bool vec4 = (n % 4) == 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t row = m0 + wm + 16 * i + li;
    if (row >= n) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t col = n0 + wn + 16 * j + 4 * lg;
      float v[4] = {acc[j][i][0], acc[j][i][1], acc[j][i][2], acc[j][i][3]};
      bf16* dst = Ob + row * n + col;
      if (vec4 && col + 4 <= n) {
        store4f(dst, v);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (col + q < n) dst[q] = static_cast<bf16>(v[q]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// The same contraction for n a multiple of 256, fed by LDS DMA
// (global_load_lds_dwordx4): the operands go global -> LDS without passing
// through registers or LDS write instructions. DS stages of DK k each; the
// configuration used (2 x 64, 128 KB) measured faster than deeper pipelines
// of 32-wide stages (3 or 4 x 32), which pay a barrier per 32 k. Stage layout
// per operand: 256 rows of 8 16-byte chunks (DK = 64), chunk c of row r in
// slot 8r + (c ^ swz(r)) -- each wave's DMA instruction writes whole rows
// (1 KB, lane-ordered), and the swizzle, applied through the lanes' source
// addresses, keeps the 16-byte fragment reads on 16 distinct bank groups:
// with 128-byte rows the bank group of a chunk is 8 (r % 2) + (c ^ swz(r)).
//
// Output columns: the B fragment of column tile j holds B rows in the
// permuted order pcol(j, r) (the same permutation the flash attention uses
// for its keys), so that a lane's accumulators of tiles 2s and 2s+1 are 8
// consecutive columns: one 16-byte store per lane, each row's four lanes
// writing 64 contiguous bytes, half the store instructions of 4-column
// pieces. An A fragment covers 16 consecutive rows, so A keeps the swizzle
// of row bits 1-3; a B fragment covers rows {0..3, 8..11, 16..19, 24..27}
// + 4 (j % 2) + 32 (j / 2), so B's swizzle takes row bits 1, 3 and 4. Each
// is a bijection on its rows and ignores the bits that differ between its
// fragments, so every fragment of a k-step is a constant offset from the
// first (no address registers per fragment). B's DMA offsets are A's XOR
// 16 (swz_a ^ swz_b)(r), which for the rows of DMA instruction j is
// 32 (lane bit 5) XOR a constant.
//
// Synchronisation: each wave waits for its own DMA with an explicit vmcnt,
// then a bare s_barrier (a fenced __syncthreads would wait for every DMA
// still in flight).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int swz_a(int r) { return (r >> 1) & 7; }
__device__ __forceinline__ int swz_b(int r) { return ((r >> 1) & 1) | (((r >> 3) & 3) << 1); }
__device__ __forceinline__ int slot_a(int r, int c) { return 8 * r + (c ^ swz_a(r)); }
__device__ __forceinline__ int slot_b(int r, int c) { return 8 * r + (c ^ swz_b(r)); }
// B row (within the wave's 64) behind accumulator row r of column tile j
__device__ __forceinline__ int pcol(int j, int r) { return 32 * (j >> 1) + 8 * (r >> 2) + 4 * (j & 1) + (r & 3); }
// a lane's 8 consecutive output columns 32s + 8 (lane / 16) .. +7 of row tile
// i: accumulator rows 4 (lane / 16) .. +3 of column tiles 2s and 2s + 1
__device__ __forceinline__ bf16x8 cols8(const f32x4 (&acc)[4][8], int i, int s) {
  const float v[8] = {acc[2 * s][i][0],     acc[2 * s][i][1],     acc[2 * s][i][2],     acc[2 * s][i][3],
                      acc[2 * s + 1][i][0], acc[2 * s + 1][i][1], acc[2 * s + 1][i][2], acc[2 * s + 1][i][3]};
  return pack8<bf16>(v);
}

// Persistent: one workgroup per CU walks its XCD's contiguous share of the
// tiles (workgroup w runs on XCD w % 8), so all tiles of a channel stay on
// one XCD and reuse its L2. During the last k-step of a tile the first stage
// of the next tile is already in flight (its LDS buffer is free), and the
// tile's output stores go out after it: the next tile's first wait then
// covers that DMA only (vmcnt counts loads and stores in issue order, so it
// waits for vmcnt(kStores)), and the stores drain under the next k-loop
// instead of holding the workgroup at its exit.
template <int DS, int DK>
__global__ __launch_bounds__(512) void contract_dma_kernel(const bf16* __restrict__ A, const bf16* __restrict__ B,
                                                           bf16* __restrict__ O, int64_t n, int64_t batches,
                                                           bool blocked) {
  static_assert(DS == 2, "the persistent hand-over assumes two stages");
  static_assert(DK == 64, "the swizzle is built for 8 chunks per row");
  constexpr int CH = DK / 8;       // 16-byte chunks per row
  constexpr int RPI = 64 / CH;     // rows per DMA instruction (1 KB)
  constexpr int NI = CH / 2;       // DMA instructions per wave per operand per stage
  constexpr int kStores = 16;      // output stores per lane per tile (8 rows x 2 of 8 elements)
  __shared__ __attribute__((aligned(16))) bf16 S[DS][2][kCT * DK];  // [stage][A, B][256 rows x DK]

  const int64_t tpd = n / kCT;
  const int64_t total = batches * tpd * tpd;
  const int64_t per_xcd = gridDim.x / kNumXcd;  // workgroups per XCD (the grid is a multiple of 8)
  const int64_t xcd = blockIdx.x % kNumXcd;
  const int64_t hi = (xcd + 1) * total / kNumXcd;  // this XCD's tiles: [xcd * total / 8, hi)

  const int t = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);  // uniform: wave offsets in SGPRs
  const int lane = t & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int wm = (wave >> 2) * 128;
  const int wn = (wave & 3) * 64;

  // DMA sources: a uniform base per operand plus a 32-bit per-lane byte
  // offset that is the same for both operands (row r of the tile, swizzled
  // chunk c); 64-bit per-lane pointers would cost 32 VGPRs at a point where
  // the accumulators leave none to spare
  uint32_t voff[NI];
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int r = 32 * wave + RPI * j + lane / CH;
    const int c = (lane % CH) ^ swz_a(r);
    voff[j] = (uint32_t)(r * n * 2 + 16 * c);
  }
  // B's offsets: voff[j] ^ xb ^ kBx[j] (r * n * 2 is a multiple of 512, so
  // the XOR touches only the chunk bits)
  static_assert(NI == 4, "kBx lists the four DMA instructions of a stage");
  constexpr uint32_t kBx[4] = {0u, 32u | 64u, 64u, 32u};  // 16 (2 (j % 2) + 4 ((j ^ (j >> 1)) % 2))
  const uint32_t xb = (uint32_t)(32 * ((lane >> 5) & 1));
  struct Tile {
    int64_t bat, m0, n0;
    const char* base[2];
  };
  // tile (bat, ti, tj) = lid as bat * tpd^2 + ti * tpd + tj; a workgroup's
  // tiles are lid, lid + per_xcd, ..., so the next one's coordinates come
  // from fixed carries instead of 64-bit divisions in the tile loop (whose
  // reciprocal estimates the compiler keeps in spilled registers, with a
  // vmcnt(0) reload that would wait for the previous tile's stores)
  auto tile_at = [&](int64_t bat, int64_t ti, int64_t tj) {
    Tile tl;
    tl.bat = bat;
    tl.m0 = ti * kCT;
    tl.n0 = tj * kCT;
    tl.base[0] = reinterpret_cast<const char*>(A + (tl.bat * n + tl.m0) * n);
    tl.base[1] = reinterpret_cast<const char*>(B + (tl.bat * n + tl.n0) * n);
    return tl;
  };
  const int64_t tt = tpd * tpd;
  const int64_t step_b = per_xcd / tt, step_i = (per_xcd % tt) / tpd, step_j = per_xcd % tpd;
  // k-tile kt goes to stage kt % DS; the stage is always a compile-time
  // constant (a run-time stage index makes the compiler wait for every DMA in
  // flight before each LDS read)
  auto issue = [&](const Tile& tl, int64_t kt, int st) {
    const int64_t k0 = kt * DK;
#pragma unroll
    for (int op = 0; op < 2; ++op)
#pragma unroll
      for (int j = 0; j < NI; ++j)
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(tl.base[op] + 2 * k0 +
                                                                       (op ? voff[j] ^ (xb ^ kBx[j]) : voff[j])),
                                         reinterpret_cast<void*>(&S[st][op][(32 * wave + RPI * j) * DK]), 16, 0, 0);
  };

  const int64_t ktiles = n / DK;  // a multiple of DS (checked by the launcher)
  int64_t lid = xcd * total / kNumXcd + blockIdx.x / kNumXcd;
  if (lid >= hi) return;
  int64_t cb = lid / tt, ci = (lid % tt) / tpd, cj = lid % tpd;
  Tile cur = tile_at(cb, ci, cj);
  issue(cur, 0, 0);
  bool first = true;
  for (;;) {
    const int64_t next_lid = lid + per_xcd;
    const bool has_next = next_lid < hi;
    int64_t nb = cb + step_b, ni = ci + step_i, nj = cj + step_j;
    if (nj >= tpd) {
      nj -= tpd;
      ++ni;
    }
    if (ni >= tpd) {
      ni -= tpd;
      ++nb;
    }
    const Tile nxt = has_next ? tile_at(nb, ni, nj) : cur;

    f32x4 acc[4][8];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[j][i] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int64_t kb = 0; kb < ktiles; kb += DS) {
#pragma unroll
      for (int st = 0; st < DS; ++st) {
        const int64_t kt = kb + st;
        // opaque per iteration: keeps the compiler from hoisting base + voff
        // into eight loop-invariant 64-bit pointers (it then spills them)
#pragma unroll
        for (int j = 0; j < NI; ++j) asm volatile("" : "+v"(voff[j]));
        // this wave's DMA of stage st is complete; on a tile's first k-step
        // the previous tile's stores, issued after that DMA, may still run
        if (st == 0 && kt == 0 && !first) __builtin_amdgcn_s_waitcnt(0x0F70 | ((kStores >> 4) << 14) | (kStores & 15));
        else __builtin_amdgcn_s_waitcnt(0xF70);
        __builtin_amdgcn_s_barrier();
        if (kt + 1 < ktiles) issue(cur, kt + 1, st ^ 1);
        else if (has_next) issue(nxt, 0, st ^ 1);  // stage 0 of the next tile (ktiles is even: buffer 0)
        const bf16* As_ = &S[st][0][0];
        const bf16* Bs_ = &S[st][1][0];
#pragma unroll
        for (int ks = 0; ks < DK / 32; ++ks) {
          bf16x8 af[8], bfr[4];
#pragma unroll
          for (int i = 0; i < 8; ++i)
            af[i] = *reinterpret_cast<const bf16x8*>(As_ + 8 * slot_a(wm + 16 * i + li, 4 * ks + lg));
#pragma unroll
          for (int j = 0; j < 4; ++j)
            bfr[j] = *reinterpret_cast<const bf16x8*>(Bs_ + 8 * slot_b(wn + pcol(j, li), 4 * ks + lg));
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 8; ++i) mma(acc[j][i], bfr[j], af[i]);
        }
      }
    }

    // the lane's row and column offsets, opaque here: the store addresses are
    // then formed after the k-loop instead of being hoisted above it (eight
    // 64-bit addresses the accumulators leave no room for: spilled, and the
    // reload's vmcnt(0) would wait for the next tile's DMA)
    int lrow = li, lcol = 8 * lg;
    asm volatile("" : "+v"(lrow), "+v"(lcol));
    if (blocked) {
      // [item][position / 64][channel][position % 64]; cur.bat = item * 128 + channel
      // the tile's 256 columns are one 256-position block of each row (n and
      // n0 are multiples of 256): block row * n/256 + n0/256
      bf16* Ob = O + ((cur.bat >> 7) * (n * n) * tile::kC) + (cur.bat & 127) * kOBlk +
                 (cur.n0 / kOBlk) * (tile::kC * kOBlk) + wn + lcol;
      const int64_t bpr = (n / kOBlk) * (tile::kC * kOBlk);  // elements per row of blocks
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        bf16* dst = Ob + (cur.m0 + wm + 16 * i + lrow) * bpr;
#pragma unroll
        for (int s = 0; s < 2; ++s) store8(dst + 32 * s, cols8(acc, i, s));
      }
    } else {
      bf16* Ob = O + cur.bat * n * n + cur.n0 + wn + lcol;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        bf16* dst = Ob + (cur.m0 + wm + 16 * i + lrow) * n;
#pragma unroll
        for (int s = 0; s < 2; ++s) store8(dst + 32 * s, cols8(acc, i, s));
      }
    }
    if (!has_next) break;
    lid = next_lid;
    cb = nb;
    ci = ni;
    cj = nj;
    cur = nxt;
    first = false;
  }
}

bool launch_contract(const bf16* a, const bf16* b, bf16* o, int64_t n, int64_t batches, hipStream_t st,
                     bool blocked) {
  const int64_t tpd = (n + kCT - 1) / kCT;
  if (n % kCT == 0) {
    blocked = blocked && batches % tile::kC == 0;
    // persistent: the device's resident capacity, a multiple of the 8 XCDs,
    // and no more workgroups than tiles need (rounded up to 8)
    const void* k = reinterpret_cast<const void*>(&contract_dma_kernel<2, 64>);
    const int64_t total = batches * tpd * tpd;
    const int64_t cap = std::max<int64_t>(kNumXcd, tile::resident_blocks(k, 512) / kNumXcd * kNumXcd);
    const int64_t grid = std::min<int64_t>(cap, (total + kNumXcd - 1) / kNumXcd * kNumXcd);
    hipLaunchKernelGGL((contract_dma_kernel<2, 64>), dim3((unsigned)grid), dim3(512), 0, st, a, b, o, n, batches,
                       blocked);
    return blocked;
  }
  hipLaunchKernelGGL(contract_kernel, dim3((unsigned)(batches * tpd * tpd)), dim3(512), 0, st, a, b, o, n, batches);
  return false;
}

template <typename T, typename TO>
void launch_gemm(const GemmParams<T, TO>& p, hipStream_t st) {
  if constexpr (std::is_same<T, bf16>::value && std::is_same<TO, bf16>::value) {
    if (launch_gemm_dma(p, st)) return;
  }
  auto tiles = [&](int64_t bm) { return p.batches * ((p.m + bm - 1) / bm) * ((p.n + bm - 1) / bm); };
  // 128-wide tiles unless they would leave most of the 256 CUs idle. fp32
  // problems of fewer than four 64-wide tiles per CU (the single track's
  // projections: 384 tiles at 1024 tokens, so half the SIMDs would run two
  // waves and half one) take 32-wide tiles, which spread them evenly at
  // several waves per SIMD; fp32 MFMAs are slow enough that the smaller
  // tile's extra LDS reads stay far below the LDS rate.
  if (tiles(128) >= 512)
    hipLaunchKernelGGL((gemm_nt_kernel<T, TO, 128>), dim3((unsigned)tiles(128)), dim3(256), 0, st, p);
  else if (std::is_same<T, float>::value && tiles(64) < 1024)
    hipLaunchKernelGGL((gemm_nt_kernel<T, TO, 32>), dim3((unsigned)tiles(32)), dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((gemm_nt_kernel<T, TO, 64>), dim3((unsigned)tiles(64)), dim3(256), 0, st, p);
}

template void launch_gemm<bf16, bf16>(const GemmParams<bf16, bf16>&, hipStream_t);
template void launch_gemm<float, float>(const GemmParams<float, float>&, hipStream_t);

}  // namespace fjx
