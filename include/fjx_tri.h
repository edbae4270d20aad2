/*
 * fjx_tri.h -- C ABI of the MI355X (gfx950) Pairformer triangle kernels.
 *
 * Plain C: device pointers, sizes, enums and a hipStream_t. No C++ or torch
 * types cross this boundary. Every entry point enqueues its kernels on the
 * given stream and returns without synchronising; buffers are owned by the
 * caller (inputs, weights, outputs and the workspace). Nothing is retained
 * between calls except read-only launch configuration and, when enabled, the
 * per-kernel timing events of fjx_prof_*.
 *
 * Errors: every int-returning call returns FJX_OK (0) or an FJX_ERR_* code;
 * fjx_last_error() then gives a message for the calling thread.
 *
 * Alignment: every activation, weight, output and residual pointer must be
 * 16-byte aligned (the kernels move rows in 16-byte pieces); masks need only
 * element alignment. A misaligned pointer is rejected with FJX_ERR_INVALID.
 *
 * Output masks: every pair- and single-track entry point takes an optional
 * out_mask (same element type as the activations, one element per output
 * position or row). Where it is 0 the written value, residual included, is
 * multiplied by 0; elsewhere it is left alone. This is Protenix's re-masking
 * z = z * pair_gate after every sublayer and s = s * single_gate after each
 * single-track sublayer (pair_gate = bool(pair_mask)),
 * src/foldjax/models/protenix/models/trunk_blocks/pairformer.py:99-149,
 * fused into the kernel that writes the output.
 *
 * Reference interfaces replaced (paths relative to the eightmm/FoldJAX tree):
 *   fjx_trimul_fwd     cuex.triangle_multiplicative_update as called from
 *                      src/foldjax/models/boltz2/models/triangle/triangle_cueq.py:88-102
 *                      and src/foldjax/models/protenix/models/triangle/triangle_cueq.py:28-47;
 *                      numerically the XLA path of
 *                      src/foldjax/models/boltz2/models/triangle/triangle.py:78-129.
 *   fjx_triattn_fwd    the fused XLA module of
 *                      src/foldjax/models/boltz2/models/triangle/triangle_attention.py:125-162
 *                      (LN, mask bias, triangle bias, q/k/v/g projections,
 *                      attention, gate, output projection; ending node by
 *                      transposed addressing).
 *   fjx_triattn_core   cueq_attention_core, src/foldjax/models/_cueq.py:66-121
 *                      (cuex.triangle_attention with an additive mask).
 */
#ifndef FJX_TRI_H
#define FJX_TRI_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FJX_ABI_VERSION 6

/* element types of activations, masks and weights */
enum { FJX_DTYPE_F32 = 0, FJX_DTYPE_BF16 = 1 };

/* triangle multiplication direction (AF3 Algorithms 12 / 13) */
enum { FJX_OUTGOING = 0, FJX_INCOMING = 1 };

/* return codes */
enum {
  FJX_OK = 0,
  FJX_ERR_INVALID = 1,     /* null pointer, bad enum, negative size */
  FJX_ERR_UNSUPPORTED = 2, /* a shape this build has no kernel for */
  FJX_ERR_WORKSPACE = 3,   /* workspace missing or smaller than required */
  FJX_ERR_HIP = 4          /* a HIP runtime call failed */
};

/*
 * Triangle multiplicative update, returning the update (or residual+update).
 *
 *   x_ln = LN_in(x)
 *   a    = mask * sigmoid(x_ln g_in[:c_h]^T)  * (x_ln p_in[:c_h]^T)
 *   b    = mask * sigmoid(x_ln g_in[c_h:]^T) * (x_ln p_in[c_h:]^T)
 *   o    = outgoing: o[i,j,c] = sum_k a[i,k,c] b[j,k,c]
 *          incoming: o[i,j,c] = sum_k a[k,i,c] b[k,j,c]
 *   out  = (LN_out(o) p_out^T) * sigmoid(x_ln g_out^T)   (+ residual)
 *
 * Weights use the PyTorch [out, in] layout of the cuEquivariance call:
 * p_in/g_in are [2*c_h, c_z] with the a rows first. In BF16 mode the
 * contraction runs on bf16 MFMA with fp32 accumulation (the reference's
 * fp32-upcast contraction of bf16 values, B2T/triangle.py:95-97) and o is
 * rounded to bf16 before LN_out (B2T/triangle.py:124). Fused kernels serve
 * c_h == 128 with c_z of 128 or 32, 64, 96 (the Protenix template stack's
 * c_z = 64, c_h = 128, protenix/models/triangle/triangle.py:131-137); other
 * widths (c_z, c_h multiples of 8 up to 1024) run a general path of row
 * LayerNorms, GEMMs and the same contraction, with a larger workspace.
 */
typedef struct fjx_trimul_args {
  int64_t batch;
  int64_t n;
  int64_t c_z;
  int64_t c_h;
  int32_t direction; /* FJX_OUTGOING or FJX_INCOMING */
  int32_t dtype;     /* of x, mask, weights, residual and out */
  float eps;         /* LayerNorm epsilon, 1e-5 in every port */
  const void* x;     /* [batch, n, n, c_z] */
  const void* mask;  /* [batch, n, n], or NULL for all ones */
  const void* norm_in_weight;  /* [c_z] */
  const void* norm_in_bias;    /* [c_z] */
  const void* p_in_weight;     /* [2*c_h, c_z] */
  const void* g_in_weight;     /* [2*c_h, c_z] */
  const void* norm_out_weight; /* [c_h] */
  const void* norm_out_bias;   /* [c_h] */
  const void* p_out_weight;    /* [c_z, c_h] */
  const void* g_out_weight;    /* [c_z, c_z] */
  const void* residual;        /* NULL, or [batch, n, n, c_z] added to the update; x, residual and out
                                  may be one buffer (in place: every position's inputs are read before
                                  it is written, by the workgroup that writes it) */
  void* out;                   /* [batch, n, n, c_z] */
  void* workspace;
  size_t workspace_bytes;
  const void* out_mask;        /* NULL, or [batch, n, n]: see "Output masks" */
} fjx_trimul_args;

size_t fjx_trimul_workspace_size(int64_t batch, int64_t n, int64_t c_z, int64_t c_h, int32_t dtype);
int fjx_trimul_fwd(const fjx_trimul_args* args, hipStream_t stream);

/*
 * fjx_trimul_fwd without any device allocation. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 *
 * Same arguments, checks, kernels and results as fjx_trimul_fwd, except that
 * args->workspace and args->workspace_bytes are ignored: the workspace is a
 * static device array of the library, FJX_NOALLOC_SCRATCH_BYTES per GPU,
 * reserved when the library's code is loaded on a GPU and held until the
 * process ends. A shape whose fjx_trimul_workspace_size exceeds it is
 * refused with FJX_ERR_WORKSPACE (bf16 with c_z == c_h == 128: batch * n^2
 * up to 349525, i.e. n <= 591 at batch 1; fp32: n <= 418). The stream must
 * belong to the current device (FJX_ERR_INVALID otherwise).
 *
 * Every call on one GPU uses that GPU's single array: calls that overlap on
 * one GPU (other streams, other threads) race and must be serialised by the
 * caller. No part of the array needs clearing between calls: each call writes
 * every byte it reads before reading it.
 */
#define FJX_NOALLOC_SCRATCH_BYTES ((size_t)256 << 20)
int fjx_trimul_fwd_noalloc(const fjx_trimul_args* args, hipStream_t stream);

/*
 * Triangle attention around the starting (Algorithm 14) or ending
 * (Algorithm 15) node, returning the update (or residual+update).
 *
 *   ending node: x and mask are read with their two pair axes swapped and the
 *   result is written back swapped, without materialising a transpose.
 *   x_ln      = LN(x)
 *   mask_bias = inf * (mask[b,i,k] - 1)                 (fp32)
 *   tri_bias  = x_ln w_bias^T, as [b, h, q, k]
 *   q,k,v,g   = x_ln w_{q,k,v,g}^T, heads of width d
 *   o[b,i,q]  = softmax_k( q.k / sqrt(d) + mask_bias[b,i,k] + tri_bias[b,h,q,k] ) v
 *   out       = (sigmoid(g) * o) w_o^T                 (+ residual)
 *
 * Weights are PyTorch [out, in]. The softmax runs in fp32 with exp2 and the
 * log2(e) factor folded into q and the biases. Fused kernels serve c_z of 128
 * or 32, 64, 96 with heads * head_dim == 128, head_dim == 32; other widths
 * (c_z a multiple of 8 up to 1024, any heads, head_dim == 32) run a general
 * path of row LayerNorms, GEMMs and the same flash core, with a larger
 * workspace.
 */
typedef struct fjx_triattn_args {
  int64_t batch;
  int64_t n;
  int64_t c_z;
  int64_t heads;
  int64_t head_dim;
  int32_t starting; /* 1 = starting node, 0 = ending node */
  int32_t dtype;
  float eps;
  float inf;        /* masking constant, 1e9 in every port */
  const void* x;    /* [batch, n, n, c_z] */
  const void* mask; /* [batch, n, n], or NULL for all ones */
  const void* norm_weight;  /* [c_z] */
  const void* norm_bias;    /* [c_z] */
  const void* bias_weight;  /* [heads, c_z]   (Boltz-2 `linear`, OpenFold3 `linear_z`) */
  const void* q_weight;     /* [heads*head_dim, c_z] */
  const void* k_weight;     /* [heads*head_dim, c_z] */
  const void* v_weight;     /* [heads*head_dim, c_z] */
  const void* g_weight;     /* [heads*head_dim, c_z], or NULL for an ungated module */
  const void* o_weight;     /* [c_z, heads*head_dim] */
  const void* residual;     /* NULL, or [batch, n, n, c_z]; x, residual and out may be one buffer */
  void* out;                /* [batch, n, n, c_z] */
  void* workspace;
  size_t workspace_bytes;
  const void* out_mask;     /* NULL, or [batch, n, n] indexed like out (never swapped) */
} fjx_triattn_args;

size_t fjx_triattn_workspace_size(int64_t batch, int64_t n, int64_t c_z, int64_t heads,
                                  int64_t head_dim, int32_t dtype);
int fjx_triattn_fwd(const fjx_triattn_args* args, hipStream_t stream);

/*
 * Attention core with the cuEquivariance layouts (src/foldjax/models/_cueq.py:77-87):
 *   q, k, v   [batch, rows, heads, n, head_dim]
 *   tri_bias  [batch, heads, n, n]      (the row axis of [B,1,H,N,N] dropped)
 *   mask_bias [batch, rows, n] fp32 additive, or NULL for zeros
 *   out       [batch, rows, heads, n, head_dim]
 * out = softmax(scale * q k^T + mask_bias + tri_bias) v per (batch, row, head).
 * q/k/v/tri_bias/out share `dtype`. Supported here: head_dim == 32.
 */
typedef struct fjx_triattn_core_args {
  int64_t batch;
  int64_t rows;
  int64_t heads;
  int64_t n;
  int64_t head_dim;
  int32_t dtype;
  float scale;
  const void* q;
  const void* k;
  const void* v;
  const void* tri_bias;
  const float* mask_bias;
  void* out;
  void* workspace;
  size_t workspace_bytes;
} fjx_triattn_core_args;

size_t fjx_triattn_core_workspace_size(int64_t batch, int64_t rows, int64_t heads, int64_t n,
                                       int64_t head_dim, int32_t dtype);
int fjx_triattn_core(const fjx_triattn_core_args* args, hipStream_t stream);

/*
 * Transition (pair or single track): for every row of c channels
 *   out = ((silu(LN(x) w_a^T) * (LN(x) w_b^T)) w_o^T  [* row_mask]  [+ residual])  [* (out_mask != 0)]
 * Replaces src/foldjax/models/boltz2/models/primitives/transition.py:39-122
 * (fc1 = w_a, fc2 = w_b, fc3 = w_o), protenix/models/primitives/primitives.py:117-146
 * and openfold3/models/primitives.py:133-150 (row_mask = the OpenFold3 mask).
 * Weights PyTorch [out, in]: w_a, w_b [hidden, c]; w_o [c, hidden]; hidden = 0
 * means 4c. A fused kernel (the hidden activations never leave the chip)
 * serves c of 128 or 32, 64, 96 with hidden == 4c and needs no workspace;
 * every other width
 * (c and hidden multiples of 8, c <= 1024; the single track's c = 384
 * included) runs a general path of GEMMs through the workspace of
 * fjx_transition_workspace_size.
 *
 * Optional pair-bias output (pb_out non-NULL; c == 128): the pair block's
 * transition is followed by the single attention with pair bias, whose bias
 * LN_z(z) w_z^T reads the whole pair tensor again
 * (src/foldjax/models/boltz2/models/trunk_blocks/pairformer.py:173-201).
 * With pb_out set, the rows are taken as the positions (b, i, j) of
 * [rows / pb_n^2, pb_n, pb_n] and the transition also writes that bias of its
 * own output (pb_norm_*, pb_weight [pb_heads, c], pb_eps: the attention's
 * z_norm_*, z_weight and eps) into pb_out, fjx_pair_bias_size bytes in a
 * library-internal layout that fjx_single_attention_fwd takes as pair_bias.
 * Fused into the transition's epilogue when c == 128, hidden == 4c and
 * pb_heads <= 16; computed from out by a separate pass otherwise.
 */
typedef struct fjx_transition_args {
  int64_t rows;
  int64_t c;
  int32_t dtype;
  float eps;
  const void* x;         /* [rows, c] */
  const void* norm_weight;
  const void* norm_bias;
  const void* w_a;
  const void* w_b;
  const void* w_o;
  const void* row_mask;  /* [rows] or NULL */
  const void* residual;  /* [rows, c] or NULL; x, residual and out may be one buffer */
  void* out;             /* [rows, c] */
  int64_t hidden;        /* 0 for 4c */
  void* workspace;       /* general path only; may be NULL when the size is 0 */
  size_t workspace_bytes;
  int64_t pb_n;          /* pair-bias output, see above; ignored when pb_out is NULL */
  int64_t pb_heads;
  float pb_eps;
  const void* pb_norm_weight;  /* [c] */
  const void* pb_norm_bias;
  const void* pb_weight;       /* [pb_heads, c] */
  void* pb_out;                /* fjx_pair_bias_size(rows / pb_n^2, pb_n, pb_heads, dtype) bytes, or NULL */
  const void* out_mask;        /* NULL, or [rows]: see "Output masks"; the pair bias is taken of the masked rows */
  int32_t pb_f32;              /* 1: pb_norm_*, pb_weight and pb_out are fp32 over a bf16 transition (an fp32
                                  single track over the bf16 pair track); the bias is computed to fp32 accuracy
                                  (bf16 high + low parts, three MFMA products); pb_out holds
                                  fjx_pair_bias_size(..., FJX_DTYPE_F32) bytes. 0: they are `dtype` */
} fjx_transition_args;

size_t fjx_transition_workspace_size(int64_t rows, int64_t c, int64_t hidden, int32_t dtype);
/* Bytes of a prepared pair bias (the pb_out / pair_bias buffer). */
size_t fjx_pair_bias_size(int64_t batch, int64_t n, int64_t heads, int32_t dtype);
int fjx_transition_fwd(const fjx_transition_args* args, hipStream_t stream);

/*
 * Single-track attention with pair bias of a Pairformer block, in the form
 * all three ports share:
 *   Boltz-2   src/foldjax/models/boltz2/models/primitives/attention.py:19-115,
 *             called from trunk_blocks/pairformer.py:182-201 (inf = 1e6; fp32
 *             s and weights over the bf16 pair tensor: dtype F32, z_dtype BF16);
 *   Protenix  src/foldjax/models/protenix/models/primitives/attention.py:108-169
 *             (layernorm_a = pre_norm; extra_attn_bias = extra_bias);
 *   OpenFold3 src/foldjax/models/openfold3/models/attention_pair_bias.py:40-75
 *             (layer_norm_a = pre_norm; inf = 1e9).
 *   s_ln = LN_pre(s)            (s itself when pre_norm_weight is NULL)
 *   q = s_ln w_q^T + b_q, k = s_ln w_k^T, v = s_ln w_v^T, g = sigmoid(s_ln w_g^T)
 *   bias[b,h,i,j] = LN_z(z[b,i,j]) w_z[h]^T  (+ extra_bias[b,h,i,j])
 *   o = softmax(q k^T / sqrt(d) + bias + (1 - mask[b,j]) * (-inf)) v
 *   out = ((g * o) w_o^T  (+ residual))  (* (out_mask[b,i] != 0))
 * Weights PyTorch [out, in]. Supported: c_z == 128, heads * head_dim == c_s,
 * head_dim <= 32. s, the weights, extra_bias, residual, out and a prepared
 * pair_bias are `dtype`; z is `z_dtype` (either may be narrower: the bias is
 * computed at `dtype`'s precision from z's values).
 */
typedef struct fjx_single_attention_args {
  int64_t batch;
  int64_t n;
  int64_t c_s;
  int64_t c_z;
  int64_t heads;
  int32_t dtype;
  float eps;
  float inf;            /* 1e6 in Boltz-2 */
  const void* s;        /* [batch, n, c_s] */
  const void* z;        /* [batch, n, n, c_z] */
  const void* mask;     /* [batch, n] token mask, or NULL */
  const void* pre_norm_weight;  /* [c_s], or NULL: s is already normalised */
  const void* pre_norm_bias;
  const void* z_norm_weight;    /* [c_z] */
  const void* z_norm_bias;
  const void* z_weight;         /* [heads, c_z] */
  const void* q_weight;         /* [c_s, c_s] */
  const void* q_bias;           /* [c_s] or NULL */
  const void* k_weight;
  const void* v_weight;
  const void* g_weight;
  const void* o_weight;
  const void* residual; /* [batch, n, c_s] or NULL; may equal out */
  void* out;            /* [batch, n, c_s]; may equal s when residual == s */
  void* workspace;
  size_t workspace_bytes;
  const void* pair_bias; /* a bias prepared by fjx_transition_fwd's pb_out for this z, or NULL;
                            when given, z, z_norm_* and z_weight are not read and may be NULL */
  int32_t z_dtype;       /* element type of z; set it even when it equals dtype (FJX_DTYPE_F32 is 0) */
  const void* out_mask;  /* NULL, or [batch, n]: see "Output masks" */
  const void* extra_bias;        /* NULL, or [n, n] planes added to the bias, element (b, h, i, j) at */
  int64_t extra_bias_stride_b;   /* extra_bias[b * stride_b + h * stride_h + i * n + j]; a stride of 0 */
  int64_t extra_bias_stride_h;   /* broadcasts that axis */
} fjx_single_attention_args;

size_t fjx_single_attention_workspace_size(int64_t batch, int64_t n, int64_t c_s, int64_t heads, int32_t dtype);
int fjx_single_attention_fwd(const fjx_single_attention_args* args, hipStream_t stream);

/* Message for the last error on the calling thread ("" if none). */
const char* fjx_last_error(void);

/* FJX_ABI_VERSION of the loaded library. */
int fjx_abi_version(void);

/*
 * Per-kernel timing with HIP events recorded on the launch stream around
 * every kernel the library enqueues. Off by default. fjx_prof_collect waits
 * for the recorded events, adds each kernel's elapsed time to its running
 * total and count, and recycles the events; fjx_prof_read copies the totals.
 */
int fjx_prof_enable(int on);
int fjx_prof_reset(void);
int fjx_prof_collect(void);
int fjx_prof_num_kernels(void);
const char* fjx_prof_kernel_name(int id);
int fjx_prof_read(int id, double* total_ms, int64_t* launches);

/*
 * Measurement aid, no counterpart in the reference: the issue rate of the
 * flash attention's per-tile instruction mix on its own. Runs a kernel that
 * issues the mix (0: 10 v_mfma_f32_16x16x32_bf16 + 16 v_exp_f32 + 24 other
 * VALU, the pipelined flash pass's instructions per 16 x 64 tile and wave;
 * 1: the same without the 16 bias widenings; 2: the MFMAs alone; 3: the
 * exponentials alone; 4: the 24 VALU alone; 5: mix 0 with its 8 score and
 * product MFMAs as 4 v_mfma_f32_32x32x16_bf16 (the same matrix-pipe cycles
 * in half the instructions); 6: those 6 MFMAs alone) `iters` times in every wave,
 * waves_per_simd (1-4) waves on each SIMD of the device, no memory traffic,
 * and returns its time in *ms (HIP events on `stream`; the call waits for
 * them). One SIMD issues one tile's mix in ms / (iters * waves_per_simd).
 */
int fjx_probe_issue_mix(int mix, int waves_per_simd, int iters, float* ms, hipStream_t stream);

/*
 * Measurement aid, no counterpart in the reference: the rate of a plain HBM
 * streaming kernel, the practical ceiling beside the 8 TB/s figure for the
 * HBM-bound row kernels. Streams 16-byte accesses over two device buffers of
 * `bytes` each (a multiple of 4096, at most 16 GiB; allocated and freed on
 * `stream`): mode 0 copies, 1 copies with nontemporal loads and stores, 2
 * only reads, 3 only writes; wgs_per_cu (1-32) 256-thread workgroups per CU.
 * Returns the time of one launch after a warm-up launch in *ms (the call
 * waits for it).
 */
int fjx_probe_hbm_stream(int mode, int wgs_per_cu, int64_t bytes, float* ms, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FJX_TRI_H */
