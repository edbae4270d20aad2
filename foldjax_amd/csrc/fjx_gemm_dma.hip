// General bf16 "NT" GEMM on the LDS-DMA pipeline of the triangle contraction:
// for every batch b
//     C[i][j] = epilogue( sum_k A[i][k] * B[j][k] )
// with both operands k-contiguous (B a PyTorch [out, in] weight), the epilogue
// of gemm_nt_kernel (fjx_contract.hip): + bias[j], sigmoid or SiLU on the
// columns from act_col0, * gate[i][j], + residual[i][j], rows whose row_gate
// is 0 written as 0. It serves the projections of the general-width paths,
// whose row counts are the pair grid's (B N^2) and whose K is a layer width.
//
// Tiling as contract_dma_kernel: a 256 x 256 output tile per 512-thread
// workgroup (8 waves of 128 x 64), k in stages of 64 copied global -> LDS by
// DMA (buffer_load ... lds: no registers, no LDS write instructions), two
// stages in 128 KB of LDS, chunk c of row r in slot 8 r + (c ^ ((r / 2) % 8))
// so the fragment reads of 16 consecutive rows hit 16 bank groups. The DMA
// goes through buffer resources sized to the operands, and a lane whose chunk
// lies past K gets an offset past the resource's end: rows past M or N and
// the k tail read as zero, so any M, N and K (K a multiple of 8) work. A
// lane's whole row offset is in its vector offset: the raw-buffer range check
// covers the vector and instruction offsets, not the scalar one, which
// carries only the k offset.
//
// Persistent: one workgroup per CU walks its XCD's contiguous share of the
// tiles, n-tiles fastest, so an A row block is reused from that XCD's L2 by
// its consecutive n-tiles; the next tile's first stage goes out during the
// last k-step. Accumulators are transposed (A operand = B rows), and the
// B rows of a wave's 64 columns sit in LDS in a permuted order (the DMA of B
// writes LDS row 16 j + r of a 64-row block from B row pcol(j, r) =
// 32 (j / 2) + 8 (r / 4) + 4 (j % 2) + r % 4), so that a lane's accumulators
// of column tiles 2s and 2s+1 are 8 consecutive output columns: 16-byte
// epilogue accesses, half the store instructions of 4-column pieces. The
// fragment reads and their swizzle are those of consecutive LDS rows.
#include <algorithm>

#include "fjx_common.hpp"
#include "fjx_kernels.hpp"
#include "fjx_tile.hpp"

namespace fjx {
namespace {

constexpr int kGT = 256;         // output tile rows and columns
constexpr int kGDK = 64;         // k per stage
constexpr int kGCH = kGDK / 8;   // 16-byte chunks per tile row in a stage
constexpr int kGRPI = 64 / kGCH; // tile rows per DMA instruction (1 KB)
constexpr int kGNI = kGCH / 2;   // DMA instructions per wave per operand per stage (32 rows)
constexpr int kGXcd = 8;
constexpr uint32_t kGOob = 0x80000000u;  // a lane offset past every resource's end
// fewer 256 x 256 tiles than this go to gemm_nt_kernel's 128- or 64-wide tiles
constexpr int64_t kMinTiles = 64;

__device__ __forceinline__ int gswz(int r) { return (r / (16 / kGCH)) % kGCH; }
__device__ __forceinline__ int gslot(int r, int c) { return kGCH * r + (c ^ gswz(r)); }

// raw buffer resource over `bytes` bytes from `base` (at most 2^31 - 1: the
// tiles address their operands from a per-tile base)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t grsrc(const void* base, int64_t bytes) {
  const int64_t b = bytes < 0 ? 0 : (bytes > 0x7FFFFFFF ? 0x7FFFFFFF : bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)b, 0x00020000);
}

__global__ __launch_bounds__(512) void gemm_dma_kernel(GemmParams<bf16, bf16> P) {
  __shared__ __attribute__((aligned(16))) bf16 S[2][2][kGT * kGDK];  // [stage][A, B][256 rows x 64]

  const int64_t M = P.m, N = P.n, K = P.k;
  const int64_t tm = (M + kGT - 1) / kGT;
  const int64_t tn = (N + kGT - 1) / kGT;
  const int64_t total = P.batches * tm * tn;
  const int64_t per_xcd = gridDim.x / kGXcd;  // the grid is a multiple of 8
  const int64_t xcd = blockIdx.x % kGXcd;
  const int64_t hi = (xcd + 1) * total / kGXcd;

  const int t = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);  // uniform: wave offsets in SGPRs
  const int lane = t & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int wm = (wave >> 2) * 128;
  const int wn = (wave & 3) * 64;

  // this lane's DMA rows and chunks: instruction j writes LDS row
  // r = 32 wave + 8 j + lane / 8, chunk c (k = 8 c), from A row r and from B
  // row 32 wave + 16 (j % 2) + 4 (j / 2) + 8 (lane bit 5) + (lane / 8) % 4
  // (the permuted order above). The swizzle of r depends on j only through
  // j % 2, so two per-lane offsets per operand serve all four instructions,
  // plus a uniform step (16 A rows or 4 B rows per two instructions) added
  // to the lane's offset
  uint32_t aoff[2], boff[2];
  int kc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int r = 32 * wave + kGRPI * j + lane / kGCH;
    const int c = (lane % kGCH) ^ gswz(r);
    kc[j] = 8 * c;
    aoff[j] = (uint32_t)(r * P.lda * 2 + 16 * c);
    const int rb = 32 * wave + 16 * j + 8 * ((lane >> 5) & 1) + ((lane >> 3) & 3);
    boff[j] = (uint32_t)(rb * P.ldb * 2 + 16 * c);
  }
  const uint32_t astep = (uint32_t)(2 * kGRPI * P.lda * 2), bstep = (uint32_t)(4 * P.ldb * 2);

  struct Tile {
    int64_t bat, m0, n0;
    __amdgpu_buffer_rsrc_t ra, rb;
  };
  auto tile_of = [&](int64_t lid) {
    Tile tl;
    tl.bat = lid / (tm * tn);
    const int64_t r = lid % (tm * tn);
    tl.m0 = (r / tn) * kGT;
    tl.n0 = (r % tn) * kGT;
    tl.ra = grsrc(P.a + tl.bat * P.sa + tl.m0 * P.lda, (M - tl.m0) * P.lda * 2);
    tl.rb = grsrc(P.b + tl.bat * P.sb + tl.n0 * P.ldb, (N - tl.n0) * P.ldb * 2);
    return tl;
  };
  // stage st <- k-tile kt of tile tl (st a compile-time constant at every call)
  auto issue = [&](const Tile& tl, int64_t kt, int st) {
    const int64_t k0 = kt * kGDK;
    // opaque here, so the sums and compares below are formed per call rather
    // than hoisted into loop-invariant registers, which spilled: the reload of
    // a spilled 64-bit k offset waited (vmcnt counts in issue order) for the
    // next stage's DMA issued just before it, in every k-step
#pragma unroll
    for (int j = 0; j < 2; ++j) asm volatile("" : "+v"(aoff[j]), "+v"(boff[j]), "+v"(kc[j]));
    // the k offset and the uniform row offset go in the scalar offset; a
    // lane whose chunk lies past K reads from past the resource's end. The
    // tail test in 32 bits against the uniform remaining depth (at least 1;
    // clamped, a chunk offset is below 64)
    const int krem = (int)min<int64_t>(K - k0, (int64_t)1 << 30);
    const bool in0 = kc[0] < krem, in1 = kc[1] < krem;
#pragma unroll
    for (int j = 0; j < kGNI; ++j) {
      const bool kin = (j & 1) ? in1 : in0;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          tl.ra, (__attribute__((address_space(3))) void*)(&S[st][0][(32 * wave + kGRPI * j) * kGDK]), 16,
          kin ? aoff[j & 1] + (uint32_t)(j >> 1) * astep : kGOob, (uint32_t)(2 * k0), 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          tl.rb, (__attribute__((address_space(3))) void*)(&S[st][1][(32 * wave + kGRPI * j) * kGDK]), 16,
          kin ? boff[j & 1] + (uint32_t)(j >> 1) * bstep : kGOob, (uint32_t)(2 * k0), 0, 0);
    }
  };

  const int64_t ktiles = (K + kGDK - 1) / kGDK;
  int64_t lid = xcd * total / kGXcd + blockIdx.x / kGXcd;
  if (lid >= hi) return;
  Tile cur = tile_of(lid);
  issue(cur, 0, 0);
  for (;;) {
    const int64_t next_lid = lid + per_xcd;
    const bool has_next = next_lid < hi;
    const Tile nxt = tile_of(has_next ? next_lid : lid);

    f32x4 acc[4][8];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[j][i] = f32x4{0.f, 0.f, 0.f, 0.f};

    // k-tile kt uses stage kt % 2; every tile starts in stage 0, so the
    // next tile's first stage goes to the stage after the last k-tile's
    auto kstep = [&](int64_t kt, auto stc) {
      constexpr int st = decltype(stc)::value;
      // this wave's DMA of stage st (and everything before it) is complete
      __builtin_amdgcn_s_waitcnt(0xF70);
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");  // no LDS read moves above the barrier
      if (kt + 1 < ktiles) issue(cur, kt + 1, st ^ 1);
      else if (has_next && st == 1) issue(nxt, 0, 0);
      const bf16* As_ = &S[st][0][0];
      const bf16* Bs_ = &S[st][1][0];
#pragma unroll
      for (int ks = 0; ks < kGDK / 32; ++ks) {
        bf16x8 af[8], bfr[4];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          af[i] = *reinterpret_cast<const bf16x8*>(As_ + 8 * gslot(wm + 16 * i + li, 4 * ks + lg));
#pragma unroll
        for (int j = 0; j < 4; ++j)
          bfr[j] = *reinterpret_cast<const bf16x8*>(Bs_ + 8 * gslot(wn + 16 * j + li, 4 * ks + lg));
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int i = 0; i < 8; ++i) mma(acc[j][i], bfr[j], af[i]);
      }
    };
    int64_t kt = 0;
    for (; kt + 1 < ktiles; kt += 2) {
      kstep(kt, std::integral_constant<int, 0>());
      kstep(kt + 1, std::integral_constant<int, 1>());
    }
    if (kt < ktiles) {
      // an odd number of k-tiles: the last one is in stage 0, and the next
      // tile's first stage (stage 0 again) is issued once every wave is past
      // its reads (below)
      kstep(kt, std::integral_constant<int, 0>());
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if (has_next) issue(nxt, 0, 0);
    }

    if (P.swiglu) {
      // the tile's columns 0..127 are a, 128..255 b of the same 128 output
      // units: the b waves hand their values (rounded to bf16) to the a
      // waves of the same rows through stage 1 of LDS -- free: the next
      // tile's first stage goes to stage 0 -- once every wave is past its
      // last k-step's reads
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      bf16* X = &S[1][0][0];  // 64 KB: 4 b waves x 32 groups x 64 lanes x 4 values
      const bool bwave = (wave & 3) >= 2;
      const int pair = (wave >> 2) * 2 + (wave & 3) - (bwave ? 2 : 0);
      if (bwave) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            bf16x4 v;
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = static_cast<bf16>(acc[j][i][q]);
            *reinterpret_cast<bf16x4*>(X + 4 * ((pair * 32 + j * 8 + i) * 64 + lane)) = v;
          }
      }
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      if (!bwave) {
        bf16* O = P.c + cur.bat * P.sc;
        const int64_t hid = N / 2;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const int64_t col = cur.n0 / 2 + wn + 32 * s + 8 * lg;
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const bf16x4 b0 = *reinterpret_cast<const bf16x4*>(X + 4 * ((pair * 32 + 2 * s * 8 + i) * 64 + lane));
            const bf16x4 b1 = *reinterpret_cast<const bf16x4*>(X + 4 * ((pair * 32 + (2 * s + 1) * 8 + i) * 64 + lane));
            const int64_t row = cur.m0 + wm + 16 * i + li;
            if (row >= M || col >= hid) continue;
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const float a = round_to<bf16>(e < 4 ? acc[2 * s][i][e] : acc[2 * s + 1][i][e - 4]);
              const float bb = static_cast<float>(e < 4 ? b0[e] : b1[e - 4]);
              v[e] = P.swiglu == 1 ? a * fast_sigmoid(a) * bb : a * round_to<bf16>(fast_sigmoid(bb));
            }
            store8(O + row * P.ldc + col, pack8<bf16>(v));
          }
        }
      }
      if (!has_next) break;
      lid = next_lid;
      cur = nxt;
      continue;
    }

    // epilogue: this lane holds row m0 + wm + 16 i + li, columns
    // n0 + wn + 32 s + 8 lg .. +7 in acc[2s][i] (the first 4) and acc[2s+1][i]
    bf16* O = P.c + cur.bat * P.sc;
    const bf16* G = P.gate ? P.gate + cur.bat * P.sc : nullptr;
    const bf16* R = P.residual ? P.residual + cur.bat * P.sc : nullptr;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int64_t col = cur.n0 + wn + 32 * s + 8 * lg;
      if (col >= N) continue;  // N is a multiple of 8 (checked by the launcher)
      float bias[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        bias[e] = P.bias && (P.bias_n == 0 || col + e < P.bias_n) ? to_f32(P.bias[col + e]) : 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int64_t row0 = cur.m0 + wm + 16 * i + li;
        if (row0 >= M) continue;
        const int64_t row = grid_row(row0, P.map_n, P.map_t);
        const bool zero_row = P.row_gate && to_f32(P.row_gate[row]) == 0.f;
        const int64_t off = row * P.ldc + col;
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float x = (e < 4 ? acc[2 * s][i][e] : acc[2 * s + 1][i][e - 4]) + bias[e];
          const int act = col + e >= P.act_col0 ? P.act : 0;
          if (act == 1) x = fast_sigmoid(x);
          else if (act == 2) x *= fast_sigmoid(x);  // silu
          v[e] = x;
        }
        if (G) {
          float g[8];
          to_f32x8(load8(G + off), g);
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] *= g[e];
        }
        if (P.proj_round) {
          const float rs = P.row_scale ? to_f32(P.row_scale[row]) : 1.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = round_to<bf16>(round_to<bf16>(v[e]) * rs);
        }
        if (R) {
          float r[8];
          to_f32x8(load8(R + off), r);
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] += r[e];
        }
        if (zero_row) {
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] *= 0.f;
        }
        store8(O + off, pack8<bf16>(v));
      }
    }
    if (!has_next) break;
    lid = next_lid;
    cur = nxt;
  }
  // the last tile's clamped prefetch is not issued (has_next is false), so
  // no DMA is in flight here
}

}  // namespace

bool gemm_dma_ok(const GemmParams<bf16, bf16>& p) {
  // 16-byte rows for the DMA, 16-byte output groups, and enough rows to fill
  // the device with 256 x 256 tiles
  const bool ok = p.k % 8 == 0 && p.lda % 8 == 0 && p.ldb % 8 == 0 && p.n % 8 == 0 && p.ldc % 8 == 0 &&
                  (reinterpret_cast<uintptr_t>(p.a) & 15) == 0 && (reinterpret_cast<uintptr_t>(p.b) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(p.c) & 15) == 0 && (!p.gate || (reinterpret_cast<uintptr_t>(p.gate) & 15) == 0) &&
                  (!p.residual || (reinterpret_cast<uintptr_t>(p.residual) & 15) == 0) &&
                  (p.batches == 1 || (p.sa % 8 == 0 && p.sb % 8 == 0 && p.sc % 8 == 0)) &&
                  p.lda * 2 * (int64_t)kGT < (int64_t)kGOob && p.ldb * 2 * (int64_t)kGT < (int64_t)kGOob &&
                  p.ldc * 2 * (int64_t)kGT < (int64_t)kGOob;
  const int64_t total = p.batches * ((p.m + kGT - 1) / kGT) * ((p.n + kGT - 1) / kGT);
  // at least half a tile of columns: narrower products (a triangle bias of a
  // few heads) would waste most of every tile
  return ok && total >= kMinTiles && p.n >= kGT / 2 &&
         (!p.swiglu || (p.n % kGT == 0 && !p.gate && !p.residual && !p.proj_round && !p.map_t));
}

bool launch_gemm_dma(const GemmParams<bf16, bf16>& p, hipStream_t st) {
  if (!gemm_dma_ok(p)) return false;
  const int64_t total = p.batches * ((p.m + kGT - 1) / kGT) * ((p.n + kGT - 1) / kGT);
  const void* k = reinterpret_cast<const void*>(&gemm_dma_kernel);
  const int64_t cap = std::max<int64_t>(kGXcd, tile::resident_blocks(k, 512) / kGXcd * kGXcd);
  const int64_t grid = std::min<int64_t>(cap, (total + kGXcd - 1) / kGXcd * kGXcd);
  hipLaunchKernelGGL(gemm_dma_kernel, dim3((unsigned)grid), dim3(512), 0, st, p);
  return true;
}

}  // namespace fjx
