// Flash triangle attention, bf16, software-pipelined over query tiles.
//
// The same mathematics and register layouts as fjx_flash.hip (transposed
// scores S^T = K Q^T with the triangle bias as the accumulator input, the
// permuted key order that lets the probabilities feed O^T = V^T P^T directly,
// softmax sums on MFMA), for the offset-free pass only: p = exp2(s) straight
// from the log2-unit score. A workgroup whose sums or outputs leave the safe
// range is flagged for the offset kernel of fjx_flash.hip, which recomputes
// it (flash_tri8_redo_kernel_bf16 walks the flags); the flags are indexed in
// that kernel's grid, which this kernel runs exactly (4 rows x 128 queries of
// one head per workgroup).
//
// Layout: 4 waves per workgroup, each owning one row of the group and its
// 128 queries (NQT = 8 tiles of 16); two workgroups per CU, so two waves per
// SIMD (a wave cannot overlap its own exponentials with its own MFMAs; the
// other wave of the SIMD fills in, also while one workgroup waits at its
// per-block barrier).
//
// Schedule: for every 64-key block, tile t goes through
//   bias load (LDS) -> S = K Q_t^T + bias (4 MFMA) -> p = exp2(S) (16 v_exp)
//   -> pack to bf16 -> O_t += V^T P_t^T, sums (6 MFMA)
// and step t of a wave reads the bias of tile t+1, issues the products of
// tile t-1 interleaved with the exponentials of tile t, then the score MFMAs
// of tile t+1; the pipeline runs across key blocks without draining.
//
// Memory: the triangle bias (bf16, times log2 e) is copied global -> LDS by
// DMA (global_load_lds_dwordx4: no registers), double-buffered, one block
// ahead; the 16-byte chunk c (8 keys) of bias row r sits in LDS slot
// 8 r + (c ^ ((r >> 1) & 7)), so the 16-byte reads of 16 rows by 16 lanes hit
// 16 distinct bank groups. A lane widens its 8 bf16 to the fp32 score
// accumulators with one shift or mask each. K and V are loaded straight into
// registers one block ahead (two register sets). Masked keys: see block_mask
// below.
#include <type_traits>

#include "fjx_common.hpp"
#include "fjx_kernels.hpp"

namespace fjx {
namespace {

constexpr int kPKB = 64;    // keys per block
constexpr int kPD = 32;     // head dim
constexpr int kPRows = 4;   // rows per workgroup
constexpr int kPHalves = 1; // query groups per row (waves per row)
constexpr int kPNqt = 8;    // query tiles of 16 per wave
constexpr int kPQwg = 16 * kPNqt * kPHalves;  // queries per workgroup: 128, the fallback kernel's tile
constexpr int kPWaves = kPRows * kPHalves;
static_assert(kPWaves <= 4, "one byte of a workgroup's 32-bit fallback flag per wave");
constexpr int kPXcd = 8;

// blockIdx -> logical workgroup id, all tiles of a row group on one XCD (as
// fjx_flash.hip's launch of the same grid)
__device__ __forceinline__ int64_t pipe_remap(int64_t w, int64_t total) {
  const int64_t per = total / kPXcd;
  if (w >= per * kPXcd) return w;
  return (w % kPXcd) * per + w / kPXcd;
}

// permuted key order of a 64-key block (fjx_flash.hip, key_of / col_of):
// accumulator row 4g + r of key tile kt is key pkey(kt, 4g + r); lane group g
// holds the 4 consecutive keys 32 (kt/2) + 8g + 4 (kt%2) .. +3 of tile kt
__device__ __forceinline__ int pkey(int kt, int i) { return 32 * (kt >> 1) + 8 * (i >> 2) + 4 * (kt & 1) + (i & 3); }

template <int V>
using IC = std::integral_constant<int, V>;

// raw buffer resource over `bytes` bytes at `base` (gfx9 descriptor word 3):
// a load addresses it with a 32-bit lane offset and a scalar offset, so no
// 64-bit address per load lives in VGPRs; reads past the end return 0
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ bf16x8 buf_load8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

}  // namespace

__global__ __launch_bounds__(64 * kPWaves) __attribute__((amdgpu_waves_per_eu(2, 2)))
void flash_pipe_kernel_bf16(FlashParams<bf16> P) {
  constexpr int NQT = kPNqt;
  constexpr int NDMA = kPQwg / kPWaves / 8;  // DMA instructions per wave per block (8 bias rows of 128 B each)
  __shared__ __attribute__((aligned(16))) u32x4 bias_s[2][kPQwg * 8];

  const int64_t n = P.n;
  const int64_t np = P.np;
  const int64_t H = P.heads;
  const int64_t QT = np / kPQwg;
  const int64_t RG = (P.rows + kPRows - 1) / kPRows;
  int64_t lid = pipe_remap(blockIdx.x, (int64_t)gridDim.x);
  const int64_t qtile = lid % QT;
  lid /= QT;
  const int64_t rg = lid % RG;
  lid /= RG;
  const int64_t h = lid % H;
  const int64_t b = lid / H;

  const int t = threadIdx.x;
  // wave-uniform: readfirstlane tells the compiler, so that the row's
  // pointers and buffer descriptors live in SGPRs
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int lane = t & 63;
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int half = wave / kPRows;
  const int64_t row = rg * kPRows + wave % kPRows;
  const bool row_ok = row < P.rows;
  const int64_t i = row_ok ? row : P.rows - 1;
  const int64_t q0 = qtile * kPQwg;
  const int qw = 16 * NQT * half;  // this wave's first query in the workgroup's tile

  const int64_t head_off = ((b * P.rows + i) * H + h) * np;  // in rows of kPD
  const bf16* Q = P.q + head_off * kPD;
  const bf16* K = P.k + head_off * kPD;
  const bf16* VT = P.vt + ((b * P.rows + i) * H * kPD + h * kPD) * np;
  const float* MB = P.mb + (b * P.rows + i) * np;
  const bf16* BIAS = P.bias + b * P.bias_stride_b + (h * np + q0) * np;
  const __amdgpu_buffer_rsrc_t rk = buf_rsrc(K, (uint32_t)(np * kPD * 2));
  const __amdgpu_buffer_rsrc_t rv = buf_rsrc(VT, (uint32_t)(kPD * np * 2));
  const __amdgpu_buffer_rsrc_t rm = buf_rsrc(MB, (uint32_t)(np * 4));
  const __amdgpu_buffer_rsrc_t rb = buf_rsrc(BIAS, (uint32_t)(kPQwg * np * 2));
  const int64_t nblk = np / kPKB;  // even: np is a multiple of 128

  // a row with every key masked would sum to 0; its softmax is that of the
  // unmasked scores (the mask is one constant on every key), so such a row
  // drops the masked keys' bias and keeps the -inf of the padded keys. The
  // scan stops at the first valid key (the first load, for every normal row).
  bool any_valid = false;
  for (int64_t k0 = 0; k0 < np; k0 += 256) {
    bool v = false;
    if (k0 + 4 * lane < np) {
      const f32x4 m4 = *reinterpret_cast<const f32x4*>(MB + k0 + 4 * lane);
      v = (m4[0] > -1.0e8f) | (m4[1] > -1.0e8f) | (m4[2] > -1.0e8f) | (m4[3] > -1.0e8f);
    }
    if (__builtin_amdgcn_ballot_w64(v) != 0) {
      any_valid = true;
      break;
    }
  }
  const bool full_row = !any_valid;

  // DMA of a block's bias tile: wave w copies RPW bias rows of the
  // workgroup's 128; instruction j covers rows RPW w + 8j + lane/8, and lane
  // fetches the chunk that belongs in slot lane%8: (lane%8) ^ ((row >> 1) & 7)
  constexpr int RPW = kPQwg / kPWaves;  // bias rows each wave copies
  // (row >> 1) & 7 of instruction j depends on j only through j % 2 (RPW is
  // a multiple of 16): two per-lane offsets, the rest uniform
  uint32_t dma_off[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int r = RPW * wave + 8 * j + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    dma_off[j] = (uint32_t)(r * np * 2 + 16 * c);
  }
  auto dma_bias = [&](int64_t blk, auto buf) {
#pragma unroll
    for (int j = 0; j < NDMA; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rb, (__attribute__((address_space(3))) void*)(&bias_s[decltype(buf)::value][(RPW * wave + 8 * j) * 8]),
          16, dma_off[j & 1], (uint32_t)(blk * kPKB * 2 + (j >> 1) * 16 * np * 2), 0, 0);
  };

  // Q of the wave's tiles, in registers for the whole row; loaded through a
  // buffer descriptor at the workgroup's first query with 32-bit lane
  // offsets, so that no 64-bit query index is formed here and kept (spilled
  // to scratch, whose stores and reloads reached HBM) until the output
  // stores after the key loop
  const __amdgpu_buffer_rsrc_t rq = buf_rsrc(Q + q0 * kPD, (uint32_t)(kPQwg * kPD * 2));
  bf16x8 qreg[NQT];
#pragma unroll
  for (int qt = 0; qt < NQT; ++qt)
    qreg[qt] = buf_load8(rq, (uint32_t)((qw + 16 * qt + li) * kPD * 2 + 16 * lg), 0);

  bf16x8 kf[2][4];     // K of two blocks
  bf16x8 vf[2][2][2];  // V^T of two blocks: [set][dt][32-key chunk]
  // K rows of a block in the permuted order: key pkey(kt, li) is
  // 8 (li/4) + li%4 plus 32 (kt/2) + 4 (kt%2), the latter a constant offset
  const uint32_t koff = (uint32_t)((8 * (li >> 2) + (li & 3)) * kPD * 2 + 16 * lg);
  auto load_k = [&](int64_t blk, auto set) {
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
      kf[decltype(set)::value][kt] =
          buf_load8(rk, koff + (uint32_t)((32 * (kt >> 1) + 4 * (kt & 1)) * kPD * 2), (uint32_t)(blk * kPKB * kPD * 2));
  };
  const uint32_t voff = (uint32_t)(li * np * 2 + 16 * lg);  // V^T row li, keys 8 lg .. +7
  auto load_v = [&](int64_t blk, auto set) {
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int c = 0; c < 2; ++c)
        vf[decltype(set)::value][dt][c] =
            buf_load8(rv, voff + (uint32_t)(64 * c), (uint32_t)(blk * kPKB * 2 + dt * 16 * np * 2));
  };
  // the row's mask bias, one key per lane, one block ahead
  float mbn[2];
  auto load_mb = [&](int64_t blk, auto set) {
    mbn[decltype(set)::value] =
        __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rm, (uint32_t)(4 * lane), (uint32_t)(blk * kPKB * 4), 0));
  };
  auto eff_mb = [&](float v) { return full_row ? (v < -1.0e30f ? v : 0.f) : v; };

  f32x4 o[NQT][2];
  f32x4 lsum[NQT / 4];  // the sums of 4 tiles share one accumulator (see ones_sel)
#pragma unroll
  for (int qt = 0; qt < NQT; ++qt) o[qt][0] = o[qt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < NQT / 4; ++u) lsum[u] = f32x4{0.f, 0.f, 0.f, 0.f};

  // prologue: blocks 0 and 1 staged, their K, V and mask bias
  dma_bias(0, IC<0>());
  dma_bias(1, IC<1>());
  load_k(0, IC<0>());
  load_k(1, IC<1>());
  load_v(0, IC<0>());
  load_v(1, IC<1>());
  load_mb(0, IC<0>());
  load_mb(1, IC<1>());
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // Masking. In this pass a key is either kept (mask bias 0 after the
  // full-row rule) or dropped (a mask bias <= -1e8: exp2 of it is 0 at any
  // score), so a block's mask is a 64-bit keep set, one ballot of the
  // prefetched values; the probabilities of dropped keys are cleared with a
  // bitwise AND on the packed bf16 values (inf & 0 = 0 too). Any other mask
  // value (an additive bias of moderate size, possible through the
  // attention-core entry) sends the workgroup to the exact offset kernel.
  bool unusual = false;
  uint64_t keep = ~0ull;  // the current block's keep set (wave-uniform)
  auto block_mask = [&](float v) {
    unusual |= __builtin_amdgcn_ballot_w64(!(v == 0.f || v <= -1.0e8f)) != 0;
    keep = __builtin_amdgcn_ballot_w64(eff_mb(v) == 0.f);
    return keep != ~0ull;
  };
  bool masked = block_mask(mbn[0]);

  // bias tile of this wave's query tile qt from LDS buffer buf, as the score
  // accumulators: chunk lg (keys 8 lg .. +7) holds key tiles 0 and 1, chunk
  // 4 + lg key tiles 2 and 3; bf16 -> fp32 is the 16-bit word moved to the
  // high half
  auto read_bias = [&](f32x4 (&s)[4], auto buf, int qt) {
    const int r = qw + 16 * qt + li;
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const u32x4 w = bias_s[decltype(buf)::value][8 * r + ((4 * h2 + lg) ^ ((r >> 1) & 7))];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        s[2 * h2 + j][0] = __uint_as_float(w[2 * j] << 16);
        s[2 * h2 + j][1] = __uint_as_float(w[2 * j] & 0xFFFF0000u);
        s[2 * h2 + j][2] = __uint_as_float(w[2 * j + 1] << 16);
        s[2 * h2 + j][3] = __uint_as_float(w[2 * j + 1] & 0xFFFF0000u);
      }
    }
  };
  auto scores = [&](f32x4 (&s)[4], auto set, int qt) {
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) mma(s[kt], kf[decltype(set)::value][kt], qreg[qt]);
  };
  auto probs = [&](const f32x4 (&s)[4], bf16x8 (&p)[2]) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      float f[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f[e] = __builtin_amdgcn_exp2f(s[2 * c][e]);
        f[4 + e] = __builtin_amdgcn_exp2f(s[2 * c + 1][e]);
      }
      p[c] = pack8<bf16>(f);
    }
  };
  // element e of p[c] is key 32c + 8g + e: two bf16 per word
  auto mask_probs = [&](bf16x8 (&p)[2]) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const uint32_t byte = (uint32_t)(keep >> (32 * c + 8 * lg)) & 0xFFu;
      u32x4 w = __builtin_bit_cast(u32x4, p[c]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        w[j] &= ((byte >> (2 * j)) & 1u ? 0x0000FFFFu : 0u) | ((byte >> (2 * j + 1)) & 1u ? 0xFFFF0000u : 0u);
      p[c] = __builtin_bit_cast(bf16x8, w);
    }
  };
  // the all-ones operand of the sums: 1 in rows 4(qt%4) .. +3 only, so 4
  // tiles share one accumulator and lane group g holds the sums of tile
  // 4(qt/4) + g
  auto ones_sel = [&](int qt) {
    const bf16 v = static_cast<bf16>((li >> 2) == (qt & 3) ? 1.0f : 0.0f);
    return bf16x8{v, v, v, v, v, v, v, v};
  };
  auto accumulate = [&](const bf16x8 (&p)[2], auto set, int qt) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      mma(o[qt][0], vf[decltype(set)::value][0][c], p[c]);
      mma(o[qt][1], vf[decltype(set)::value][1][c], p[c]);
      mma(lsum[qt >> 2], ones_sel(qt), p[c]);
    }
  };
  // Instruction order of one step: the bias reads of the next tile first;
  // then the 6 product MFMAs of the previous tile, each followed by VALU
  // instructions of this tile's exponentials and packs; then, behind a
  // barrier only VALU may cross, the 4 score MFMAs of the next tile (its bias
  // has arrived by then). The next step's exponentials read those scores
  // only after its own product MFMAs.
  auto products_phase = [&](bool with_reads) {
    if (with_reads) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS read
#pragma unroll
    for (int m = 0; m < 6; ++m) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // VALU
    }
    __builtin_amdgcn_sched_barrier(0x0002 | 0x0400);  // only VALU (incl. transcendental) crosses
  };
  auto scores_phase = [&]() {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 1);  // VALU
    }
  };

  // The pipeline. Step t of a block reads the bias of tile t+1, issues the
  // products of tile t-1, the exponentials of tile t and the score MFMAs of
  // tile t+1. S[u % 2] holds tile u from its bias read to its exponentials;
  // Pp the (masked) probabilities of the tile before the current one (zero
  // before the first tile, so its product adds nothing). Tiles past the
  // block's end are the next block's first ones.
  f32x4 S[2][4];
  const bf16 zb = static_cast<bf16>(0.0f);
  bf16x8 Pp[2] = {bf16x8{zb, zb, zb, zb, zb, zb, zb, zb}, bf16x8{zb, zb, zb, zb, zb, zb, zb, zb}};
  read_bias(S[0], IC<0>(), 0);
  scores(S[0], IC<0>(), 0);

  // one 64-key block in register set / LDS buffer SET (= blk % 2). Every
  // prefetch is unconditional, clamped to the last block (a re-read nobody
  // uses), so a step's work is one branch-free region; the only branch is
  // the mask of the rare blocks that hold masked keys, after it.
  auto run_block = [&](int64_t blk, auto set, auto has_next) {
    constexpr int SET = decltype(set)::value;
    constexpr bool NEXT = decltype(has_next)::value != 0;
    const int64_t b1 = blk + 1 < nblk ? blk + 1 : nblk - 1;
    const int64_t b2 = blk + 2 < nblk ? blk + 2 : nblk - 1;
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
      f32x4 (&cur)[4] = S[qt & 1];
      f32x4 (&nxt)[4] = S[(qt + 1) & 1];
      if (qt == NQT - 1 && NEXT) {
        // the next block's bias tile, K and mask bias are complete after this
        // wait and barrier; this block's LDS buffer (every wave read its last
        // tile in the previous step) is free for block blk + 2. The wait
        // leaves the next block's 4 V loads (the youngest, issued in step 1)
        // in flight: their first reader waits for them itself.
        __builtin_amdgcn_s_waitcnt(0xF70 | 4);  // vmcnt(4)
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");  // no LDS read moves above the barrier
        dma_bias(b2, IC<SET>());
        load_mb(b2, IC<SET>());
      }
      if (qt < NQT - 1) read_bias(nxt, IC<SET>(), qt + 1);
      else if (NEXT) read_bias(nxt, IC<SET ^ 1>(), 0);
      if (qt == 1) load_v(b1, IC<SET ^ 1>());  // that set's last reader was tile 0's product
      // product of the previous tile (tile 0: the previous block's last
      // tile, with that block's V)
      if (qt > 0) accumulate(Pp, IC<SET>(), qt - 1);
      else accumulate(Pp, IC<SET ^ 1>(), NQT - 1);
      probs(cur, Pp);
      products_phase(qt < NQT - 1 || NEXT);
      if (qt < NQT - 1) scores(nxt, IC<SET>(), qt + 1);
      else if (NEXT) scores(nxt, IC<SET ^ 1>(), 0);
      scores_phase();
      if (qt == NQT - 1 && NEXT) load_k(b2, IC<SET>());  // this set's last reader was the previous step
      if (masked) mask_probs(Pp);
      if (qt == NQT - 1 && NEXT) masked = block_mask(mbn[SET ^ 1]);
    }
  };
  for (int64_t blk = 0; blk + 2 < nblk; blk += 2) {
    run_block(blk, IC<0>(), IC<1>());
    run_block(blk + 1, IC<1>(), IC<1>());
  }
  run_block(nblk - 2, IC<0>(), IC<1>());
  run_block(nblk - 1, IC<1>(), IC<0>());
  accumulate(Pp, IC<1>(), NQT - 1);  // nblk is even: the last block used set 1
  // the clamped prefetches may still be writing LDS: drain before leaving
  __builtin_amdgcn_s_waitcnt(0);

  // every softmax sum in [2^-100, inf) and every output finite, checked on
  // the bit patterns; otherwise the fallback kernel recomputes the workgroup.
  // Each wave writes its own byte of the workgroup's flag word, 1 or 0 (0 for
  // rows past the end), so the flags need no clearing before this pass.
  bool bad = unusual;
#pragma unroll
  for (int qt = 0; qt < NQT; ++qt) {
    const float ls = __shfl(lsum[qt >> 2][0], 16 * (qt & 3) + li, 64);
    const unsigned u = __float_as_uint(ls);
    bad |= !(u >= 0x0D800000u && u < 0x7F800000u);
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) bad |= (__float_as_uint(o[qt][dt][r]) & 0x7F800000u) == 0x7F800000u;
  }
  const bool redo = row_ok && __builtin_amdgcn_ballot_w64(bad) != 0;
  if (lane == 0) reinterpret_cast<unsigned char*>(P.fallback + blockIdx.x)[wave] = redo ? 1 : 0;
  if (!row_ok || redo) return;
  // Output: lane (li, g) holds dims 4g .. 4g+3 and 16 + 4g .. +3 of query
  // li. Two lane swaps (lanes 32 apart, then 16 apart; the query stays) give
  // it dims 8g .. 8g+7 instead, so each query's 64 bytes leave as four
  // 16-byte stores of one instruction: whole cache lines, not 8-byte pieces
  // written by two instructions.
  bf16* OUT = P.out + b * P.o_stride_b + i * P.o_stride_row + h * P.o_stride_head + q0 * P.o_stride_q;
  auto pack2 = [](float x, float y) {
    return (uint32_t)__builtin_bit_cast(uint16_t, static_cast<bf16>(x)) |
           ((uint32_t)__builtin_bit_cast(uint16_t, static_cast<bf16>(y)) << 16);
  };
#pragma unroll
  for (int qt = 0; qt < NQT; ++qt) {
    const float ls = __shfl(lsum[qt >> 2][0], 16 * (qt & 3) + li, 64);
    const float inv = 1.0f / ls;
    const int ql = qw + 16 * qt + li;  // query q0 + ql
    uint32_t a[2], c[2];  // a: dims 4g .., c: dims 16 + 4g ..
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      a[e] = pack2(o[qt][0][2 * e] * inv, o[qt][0][2 * e + 1] * inv);
      c[e] = pack2(o[qt][1][2 * e] * inv, o[qt][1][2 * e + 1] * inv);
    }
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      // lanes 0-31 keep a and take c of lanes 0-31; lanes 32-63 the a and c of lanes 32-63
      const auto s32 = __builtin_amdgcn_permlane32_swap(a[e], c[e], false, false);
      // then rows of 16: row 0 keeps its own and takes row 1's, and so on
      const auto s16 = __builtin_amdgcn_permlane16_swap(s32[0], s32[1], false, false);
      a[e] = s16[0];  // dims 8g .. 8g+3
      c[e] = s16[1];  // dims 8g+4 .. 8g+7
    }
    if (q0 + ql < n) *reinterpret_cast<u32x4*>(OUT + ql * P.o_stride_q + 8 * lg) = u32x4{a[0], a[1], c[0], c[1]};
  }
}

bool launch_flash_pipe(const FlashParams<bf16>& p, int64_t batch, hipStream_t st) {
  // needs the fallback flags (the offset kernel recomputes what this pass
  // flags; every flag is written, none needs clearing first) and a padded
  // length that is a multiple of 128; launches the grid of the fallback
  // kernel
  if (!p.fallback || p.rows < 2 || p.np % kPQwg != 0) return false;
  const int64_t rg = (p.rows + kPRows - 1) / kPRows;
  const dim3 grid((unsigned)(batch * p.heads * rg * (p.np / kPQwg)));
  hipLaunchKernelGGL(flash_pipe_kernel_bf16, grid, dim3(64 * kPWaves), 0, st, p);
  return true;
}

}  // namespace fjx
