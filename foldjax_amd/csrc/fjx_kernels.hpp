// Kernel parameter blocks and launchers shared between the HIP translation
// units and the C ABI layer (fjx_capi.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fjx {

template <typename T>
struct TriMulPrologueParams {
  const T* x;     // [B][N][N][128]
  const T* mask;  // [B][N][N] or null
  const T* ln_w;
  const T* ln_b;
  const T* w_p;     // [256][128]: rows 0..127 -> a, 128..255 -> b
  const T* w_g;     // [256][128]
  T* a_cm;          // [B][128][N*N] virtual grid
  T* b_cm;
  int64_t n;
  float eps;
  int transpose;    // 1 for the incoming direction
  int cw;           // channels of x (and rows of w_p/w_g) when below 128 (a multiple of 32); 0: 128
};

template <typename T>
struct TriAttnPrologueParams {
  const T* x;
  const T* mask;
  const T* ln_w;
  const T* ln_b;
  const T* w_bias;  // [4][128]
  const T* w_q;     // [128][128]
  const T* w_k;
  const T* w_v;
  T* q;             // [B][N][4][Np][32]
  T* k;
  T* vt;            // [B][N][128][Np]
  T* bias;          // [B][4][Np][Np]
  float* mb;        // [B][N][Np]
  int64_t n;
  int64_t np;
  float eps;
  float inf;
  float q_scale;    // head_dim^-0.5 * log2(e)
  int transpose;    // 1 for the ending node
  int cw;           // channels of x (the k of every weight) when below 128 (a multiple of 32); 0: 128
};

template <typename T>
struct TriMulEpilogueParams {
  const T* o;         // contraction output, channel-major [B][128][N*N], or tile-blocked (o_blocked)
  const T* x;         // the op's input [B][N][N][128] (for the output gate)
  const T* ln_in_w;   // LN_in, recomputed for the gate
  const T* ln_in_b;
  const T* ln_out_w;  // LN over the contraction output
  const T* ln_out_b;
  const T* w_pout;    // [128][128]
  const T* w_gout;    // [128][128]
  const T* residual;  // [B][N][N][128] or null (may alias out)
  const T* out_mask;  // [B][N][N] or null: positions where it is 0 are written as 0
  T* out;
  int64_t n;
  float eps;
  // o tile-blocked: [B][N*N/256][128][256], the 128 channels of 256
  // consecutive positions in one 64 KB block (the LDS-DMA contraction's
  // blocked output)
  bool o_blocked;
  int cw;             // channels of x / out (k of w_gout, rows of both weights) when below 128; 0: 128
};

template <typename T>
struct TriAttnEpilogueParams {
  const T* o;         // attention output, head-major [B][N rows][4 heads][N][32] in the virtual grid
  const T* x;         // the op's input [B][N][N][128] (for the gate)
  const T* ln_w;
  const T* ln_b;
  const T* w_g;       // [128][128] or null (ungated)
  const T* w_o;       // [128][128]
  const T* residual;  // original grid, or null (may alias out)
  const T* out_mask;  // original grid [B][N][N], or null: positions where it is 0 are written as 0
  T* out;             // original grid
  int64_t n;
  float eps;
  int transpose;      // 1 for the ending node
  int cw;             // channels of x / out (k of w_g, rows of w_o) when below 128; 0: 128
};

template <typename T, typename TO>
struct GemmParams {
  const T* a;       // [batches][m][lda], k-contiguous rows
  const T* b;       // [batches][n][ldb], k-contiguous rows (a PyTorch [out, in] weight)
  TO* c;            // [batches][m][ldc]
  int64_t m, n, k;
  int64_t lda, ldb, ldc;
  int64_t sa, sb, sc;  // batch strides in elements (0 = shared)
  int64_t batches;
  const T* bias;       // [n] or null
  int64_t bias_n;      // the bias covers columns < bias_n (0: all n)
  int act;             // 0 none, 1 sigmoid, 2 silu
  int64_t act_col0;    // the activation applies to columns >= act_col0
  const TO* gate;      // indexed like c, or null
  const TO* residual;  // indexed like c, or null (may alias c)
  const TO* row_gate;  // [m] per output row, or null: rows where it is 0 are written as 0 (after the residual)
  // proj_round: the product is a projection output -- rounded to TO, times
  // row_scale[row] when set, rounded again -- before the residual is added
  // (the order of a transition's row mask and residual)
  int proj_round;
  const TO* row_scale;  // [m] or null (with proj_round)
  // map_t: row r of the product is stored at, and reads its residual and
  // row gate from, the transposed pair-grid position: with N = map_n,
  // r = b N^2 + i N + j goes to b N^2 + j N + i (the ending node's grid)
  int map_t;
  int64_t map_n;
  // pair mode (launch_gemm_dma only): B holds two weights interleaved in
  // blocks of 128 rows (a block of the first, then the block of the second
  // for the same 128 output units), n = 2 units, and C[i][u] combines a and b
  // (both rounded to TO first): 1 = silu(a) * b (SwiGLU), 2 = a * sigmoid(b)
  // (a gated projection); C has `units` columns
  int swiglu;
};

template <typename T>
struct TransitionParams {
  const T* x;         // [rows][C]
  const T* ln_w;
  const T* ln_b;
  const T* w_a;       // [4C][C] (silu branch)
  const T* w_b;       // [4C][C]
  const T* w_o;       // [C][4C]
  const T* row_mask;  // [rows] or null
  const T* residual;  // [rows][C] or null (may alias out)
  const T* out_mask;  // [rows] or null: rows where it is 0 are written as 0 (after the residual)
  T* out;             // [rows][C]
  int64_t rows;
  float eps;
  // optional pair-bias epilogue (pb_out null: off): rows are the positions
  // (b, r, s) of [B, pb_n, pb_n]; pb_out[b][h][r][s] = log2(e) *
  // LN_pb(out row) . pb_w[h] in the padded [B, pb_heads, pb_np, pb_np]
  // layout the flash kernel reads; pb_heads <= 16
  const T* pb_ln_w;
  const T* pb_ln_b;
  const T* pb_w;      // [pb_heads][C]
  T* pb_out;
  int64_t pb_n;
  int64_t pb_np;
  int pb_heads;
  float pb_eps;
  // the same epilogue with the norm, weight and bias in fp32 over a bf16
  // transition (the Boltz-2 single track's precision); pbf_out null: off
  const float* pbf_ln_w;
  const float* pbf_ln_b;
  const float* pbf_w;  // [pb_heads][C]
  float* pbf_out;
  // channels of x / out when below 128 (a multiple of 32, hidden 4 cw): the
  // narrow form of the kernel; 0 or 128: the full form
  int cw;
};

template <typename T>
struct FlashParams {
  const T* q;        // [B][N][H][Np][32], pre-scaled by scale*log2 e
  const T* k;        // [B][N][H][Np][32]
  const T* vt;       // [B][N][H*32][Np]
  const T* bias;     // [B][H][Np][Np], already times log2 e
  const float* mb;   // [B][N][Np], already times log2 e; -inf for padded keys
  T* out;            // out[b][i][q][h*32+d] via the strides below
  int64_t n;
  int64_t np;
  int64_t heads;
  int64_t rows;      // number of attention rows i (== n for the fused module)
  int64_t o_stride_b;
  int64_t o_stride_row;
  int64_t o_stride_head;
  int64_t o_stride_q;
  int64_t bias_stride_b;  // 0 when one bias is shared by all batches
  // the bf16 pair-track path without a softmax offset (see fjx_flash.hip):
  // one flag per workgroup of that launch, or null for the offset path only
  unsigned* fallback;
};

template <typename T>
void launch_trimul_prologue(const TriMulPrologueParams<T>& p, int64_t batch, hipStream_t st);
template <typename T>
void launch_triattn_prologue(const TriAttnPrologueParams<T>& p, int64_t batch, hipStream_t st);
template <typename T>
void launch_trimul_epilogue(const TriMulEpilogueParams<T>& p, int64_t batch, hipStream_t st);
template <typename T>
void launch_triattn_epilogue(const TriAttnEpilogueParams<T>& p, int64_t batch, hipStream_t st);
template <typename T, typename TO>
void launch_gemm(const GemmParams<T, TO>& p, hipStream_t st);
// the bf16 GEMM on the LDS-DMA pipeline (fjx_gemm_dma.hip); false when the
// shape or alignment does not suit it (the caller then runs gemm_nt_kernel)
bool launch_gemm_dma(const GemmParams<bf16, bf16>& p, hipStream_t st);
// whether launch_gemm_dma takes p (shape, alignment and size)
bool gemm_dma_ok(const GemmParams<bf16, bf16>& p);
// triangle contraction, bf16: o[c] = a[c] b[c]^T for c < batches, each n x n
// blocked: write o tile-blocked, [batches / 128][N*N/256][128][256] (needs
// batches a multiple of 128 and n a multiple of 256), else [batches][N*N];
// returns whether it wrote the blocked layout
bool launch_contract(const bf16* a, const bf16* b, bf16* o, int64_t n, int64_t batches, hipStream_t st,
                     bool blocked = false);
template <typename T>
void launch_transition(const TransitionParams<T>& p, int c, hipStream_t st);

// single-track helpers (fjx_single.hip)
template <typename T>
void launch_layernorm_rows(const T* x, const T* w, const T* b, T* y, int64_t rows, int c, float eps, hipStream_t st);
template <typename T>
void launch_split_heads(const T* qkv, int64_t ld, int64_t batch, int64_t n, int64_t np, int heads, int dh,
                        float q_mul, T* q, T* k, T* vt, hipStream_t st);
// z (and its norm and weight) in TZ, the bias in T: the Boltz-2 single track
// runs in fp32 over a bf16 pair tensor
template <typename TZ, typename T>
void launch_pair_bias(const TZ* z, const T* ln_w, const T* ln_b, const T* w, T* bias, int64_t batch, int64_t n,
                      int64_t np, int heads, float eps, hipStream_t st);
// bias[b][h][q][k] (+)= log2(e) * extra[b * sb + h * sh + q * n + k] for q, k < n;
// src (a prepared bias of the same layout) is read when given, else bias itself
template <typename T>
void launch_add_extra_bias(const T* src, T* bias, const T* extra, int64_t sb, int64_t sh, int64_t batch, int heads,
                           int64_t n, int64_t np, hipStream_t st);
template <typename T>
void launch_pair_bias_border(T* bias, int64_t planes, int64_t n, int64_t np, hipStream_t st);
template <typename T>
void launch_key_mask(const T* mask, float* mb, int64_t batch, int64_t n, int64_t np, float inf, hipStream_t st);
template <typename T>
void launch_gate_unpad(const T* o, const T* g, int64_t ldg, T* out, int64_t rows, int heads, int dh,
                       hipStream_t st);
template <typename T>
void launch_flash(const FlashParams<T>& p, int64_t batch, hipStream_t st);
// rows == 1, a bias per head: keys split over the waves of a workgroup
// (fjx_single_flash.hip); launch_flash routes such calls here
template <typename T>
void launch_flash_single(const FlashParams<T>& p, int64_t batch, hipStream_t st);
// the pipelined offset-free pass (fjx_flash_pipe.hip); false when the shape
// or the parameters do not suit it (then nothing is launched)
bool launch_flash_pipe(const FlashParams<bf16>& p, int64_t batch, hipStream_t st);
// the flash tile's instruction mix alone (fjx_probe.hip): kernel ms, or -1 on a HIP error
int probe_issue_mix(int mix, int waves_per_simd, int iters, float* ms, hipStream_t st);
int probe_hbm_stream(int mode, int wgs_per_cu, int64_t bytes, float* ms, hipStream_t st);

// general-width paths (fjx_generic.hip); positions v = r*n + s of the virtual
// grid read the original grid at s*n + r when t = 1
template <typename T>
void launch_ln_grid(const T* x, const T* w, const T* b, T* y, int64_t batch, int64_t n, int c, float eps, int t,
                    hipStream_t st);
template <typename T>
void launch_to_channel_major(const T* src, int64_t ld, int c0, int C, const T* mask, T* dst, int64_t batch, int64_t n,
                             int t, hipStream_t st);
template <typename T>
void launch_to_position_major(const T* src, int C, T* dst, int64_t batch, int64_t nn, hipStream_t st);
template <typename T>
void launch_split_qk(const T* src, int64_t ld, int64_t c0, T* dst, int64_t rows, int64_t n, int64_t np, int heads,
                     float mul, hipStream_t st);
template <typename T>
void launch_split_vt(const T* src, int64_t ld, int64_t c0, T* dst, int64_t rows, int64_t n, int64_t np, int hd_total,
                     hipStream_t st);
template <typename T>
void launch_bias_planes(const T* src, int64_t ld, int64_t c0, T* dst, int64_t batch, int64_t n, int64_t np, int heads,
                        hipStream_t st);
template <typename T>
void launch_grid_mask_bias(const T* mask, float* mb, int64_t batch, int64_t n, int64_t np, float inf, int t,
                           hipStream_t st);
template <typename T>
void launch_gate_rows(T* o, const T* g, int64_t ldg, int64_t c0, int64_t rows, int width, hipStream_t st);
// out[orig(v)] = (T(y[v] * row_mask) + residual[orig(v)]) * (out_mask != 0),
// for a product the DMA GEMM does not take (its epilogue does this itself);
// y may be `splits` partial products (split K), `split_stride` elements
// apart, summed here
template <typename T>
void launch_scatter_add(const T* y, const T* row_mask, const T* residual, const T* out_mask, T* out, int64_t rows,
                        int64_t n, int c, int t, hipStream_t st, int splits = 1, int64_t split_stride = 0);

}  // namespace fjx
