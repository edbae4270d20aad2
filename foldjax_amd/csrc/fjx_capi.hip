// C ABI of the triangle kernels: argument checks, workspace layout, launch
// sequence, thread-local error strings and optional per-kernel event timing.
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>
#include <initializer_list>
#include <type_traits>
#include <vector>

#include "fjx_tri.h"
#include "fjx_common.hpp"
#include "fjx_kernels.hpp"

using namespace fjx;

namespace {

thread_local std::string g_err;
// set while an allocation-free entry point runs: no timing events are taken
// (creating one is a driver allocation)
thread_local bool g_no_events = false;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(FJX_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return FJX_OK;
}

constexpr size_t kAlign = 256;
size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }
int64_t round64(int64_t v) { return (v + 63) / 64 * 64; }
size_t esize(int32_t dt) { return dt == FJX_DTYPE_BF16 ? 2 : 4; }

// ------------------------------------------------------------ event timing
enum KernelId {
  K_TRIMUL_PROLOGUE = 0,
  K_TRIMUL_CONTRACT,
  K_TRIMUL_EPILOGUE,
  K_TRIATTN_PROLOGUE,
  K_TRIATTN_FLASH,
  K_TRIATTN_EPILOGUE,
  K_TRIATTN_CORE_PREP,
  K_TRANSITION,
  K_SINGLE_PROJ,
  K_SINGLE_PAIR_BIAS,
  K_SINGLE_FLASH,
  K_SINGLE_OUT,
  K_SINGLE_TRANSITION,
  K_COUNT
};
const char* kKernelNames[K_COUNT] = {"trimul_prologue", "trimul_contract", "trimul_epilogue",
                                     "triattn_prologue", "triattn_flash", "triattn_epilogue",
                                     "triattn_core_prep", "transition",     "single_proj",
                                     "single_pair_bias", "single_flash",   "single_out",
                                     "single_transition"};

struct Prof {
  std::mutex mu;
  bool on = false;
  std::vector<hipEvent_t> pool;
  struct Rec {
    int id;
    hipEvent_t a, b;
  };
  std::vector<Rec> pending;
  double total_ms[K_COUNT] = {};
  int64_t count[K_COUNT] = {};
};
Prof& prof() {
  static Prof p;
  return p;
}

hipEvent_t take_event(Prof& p) {
  if (!p.pool.empty()) {
    hipEvent_t e = p.pool.back();
    p.pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

template <class F>
int timed(int id, hipStream_t st, const char* what, F&& launch) {
  Prof& p = prof();
  hipEvent_t a = nullptr, b = nullptr;
  {
    std::lock_guard<std::mutex> lk(p.mu);
    if (p.on && !g_no_events) {
      a = take_event(p);
      b = take_event(p);
    }
  }
  if (a && b) (void)hipEventRecord(a, st);
  launch();
  const int rc = check_launch(what);
  if (a && b) {
    (void)hipEventRecord(b, st);
    std::lock_guard<std::mutex> lk(p.mu);
    p.pending.push_back({id, a, b});
  }
  return rc;
}

// --------------------------------------------------- attention-core prep
// q/k: [B][R][H][n][32] -> [B][R][H][np][32] (q times qscale), zero padded keys
template <typename T>
__global__ void pad_qk_kernel(const T* __restrict__ src, T* __restrict__ dst, int64_t n, int64_t np,
                              int64_t heads_rows, float mul) {
  const int64_t total = heads_rows * np * 32;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t d = idx % 32;
    const int64_t s = (idx / 32) % np;
    const int64_t hr = idx / (32 * np);
    dst[idx] = s < n ? from_f32<T>(to_f32(src[(hr * n + s) * 32 + d]) * mul) : from_f32<T>(0.f);
  }
}
// v: [B][R][H][n][32] -> vt [B][R][H*32][np]
template <typename T>
__global__ void transpose_v_kernel(const T* __restrict__ src, T* __restrict__ dst, int64_t n, int64_t np,
                                   int64_t heads_rows) {
  const int64_t total = heads_rows * 32 * np;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t s = idx % np;
    const int64_t d = (idx / np) % 32;
    const int64_t hr = idx / (32 * np);
    dst[idx] = s < n ? src[(hr * n + s) * 32 + d] : from_f32<T>(0.f);
  }
}
// bias [B][H][n][n] -> [B][H][np][np] times log2 e, zeros outside
template <typename T>
__global__ void pad_bias_kernel(const T* __restrict__ src, T* __restrict__ dst, int64_t n, int64_t np,
                                int64_t planes) {
  const int64_t total = planes * np * np;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t k = idx % np;
    const int64_t q = (idx / np) % np;
    const int64_t pl = idx / (np * np);
    const float v = (q < n && k < n) ? to_f32(src[(pl * n + q) * n + k]) * kLog2e : 0.f;
    dst[idx] = from_f32<T>(v);
  }
}
// mask bias [B][R][n] fp32 -> [B][R][np] times log2 e, -inf for padded keys
__global__ void pad_mb_kernel(const float* __restrict__ src, float* __restrict__ dst, int64_t n, int64_t np,
                              int64_t rows) {
  const int64_t total = rows * np;
  for (int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t k = idx % np;
    const int64_t r = idx / np;
    dst[idx] = k < n ? (src ? src[r * n + k] * kLog2e : 0.f) : -INFINITY;
  }
}

dim3 grid_for(int64_t total) {
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  return dim3((unsigned)blocks);
}

// --------------------------------------------------------------- layouts
struct TriMulWs {
  size_t a, b, o, total;
};
TriMulWs trimul_ws(int64_t batch, int64_t n, int32_t dtype) {
  const size_t per = align_up((size_t)batch * n * n * 128 * esize(dtype));
  TriMulWs w;
  w.a = 0;
  w.b = per;
  w.o = 2 * per;
  w.total = 3 * per;
  return w;
}

struct TriAttnWs {
  size_t q, k, vt, bias, mb, o, flags, total;
};
// one flag per workgroup of the flash launch (4 rows x 64 or 128 queries)
size_t flash_flags_bytes(int64_t batch, int64_t rows, int64_t heads, int64_t np) {
  return align_up((size_t)batch * heads * ((rows + 3) / 4) * ((np + 63) / 64) * sizeof(unsigned));
}
TriAttnWs triattn_ws(int64_t batch, int64_t rows, int64_t n, int64_t heads, int32_t dtype, bool with_o) {
  const int64_t np = round64(n);
  const size_t es = esize(dtype);
  const size_t qk = align_up((size_t)batch * rows * heads * np * 32 * es);
  TriAttnWs w;
  size_t off = 0;
  w.q = off;
  off += qk;
  w.k = off;
  off += qk;
  w.vt = off;
  off += qk;
  w.bias = off;
  off += align_up((size_t)batch * heads * np * np * es);
  w.mb = off;
  off += align_up((size_t)batch * rows * np * sizeof(float));
  w.o = off;
  if (with_o) off += align_up((size_t)batch * rows * n * heads * 32 * es);
  w.flags = off;
  off += flash_flags_bytes(batch, rows, heads, np);
  w.total = off;
  return w;
}

template <typename T>
T* at(void* base, size_t off) {
  return reinterpret_cast<T*>(static_cast<char*>(base) + off);
}

// ----------------------------------------------------------- tri-mul body
template <typename T>
int trimul_run(const fjx_trimul_args* a, hipStream_t st) {
  const TriMulWs ws = trimul_ws(a->batch, a->n, a->dtype);
  T* abuf = at<T>(a->workspace, ws.a);
  T* bbuf = at<T>(a->workspace, ws.b);
  T* obuf = at<T>(a->workspace, ws.o);

  // c_z below 128 (the template stack's 64): the narrow forms of the kernels
  const int cw = a->c_z < 128 ? (int)a->c_z : 0;
  TriMulPrologueParams<T> pp = {};
  pp.x = static_cast<const T*>(a->x);
  pp.mask = static_cast<const T*>(a->mask);
  pp.ln_w = static_cast<const T*>(a->norm_in_weight);
  pp.ln_b = static_cast<const T*>(a->norm_in_bias);
  pp.w_p = static_cast<const T*>(a->p_in_weight);
  pp.w_g = static_cast<const T*>(a->g_in_weight);
  pp.a_cm = abuf;
  pp.b_cm = bbuf;
  pp.n = a->n;
  pp.eps = a->eps;
  pp.transpose = a->direction == FJX_INCOMING;
  pp.cw = cw;
  int rc = timed(K_TRIMUL_PROLOGUE, st, "trimul_prologue", [&] { launch_trimul_prologue<T>(pp, a->batch, st); });
  if (rc) return rc;

  bool o_blocked = false;  // the LDS-DMA contraction writes o tile-blocked for the epilogue
  rc = timed(K_TRIMUL_CONTRACT, st, "trimul_contract", [&] {
    if constexpr (std::is_same<T, bf16>::value) {
      o_blocked = launch_contract(abuf, bbuf, obuf, a->n, a->batch * 128, st, true);
    } else {
      GemmParams<T, T> cp = {};
      cp.a = abuf;
      cp.b = bbuf;
      cp.c = obuf;
      cp.m = cp.n = cp.k = a->n;
      cp.lda = cp.ldb = cp.ldc = a->n;
      cp.sa = cp.sb = cp.sc = a->n * a->n;
      cp.batches = a->batch * 128;
      launch_gemm<T, T>(cp, st);
    }
  });
  if (rc) return rc;

  TriMulEpilogueParams<T> ep = {};
  ep.o = obuf;
  ep.o_blocked = o_blocked;
  ep.x = static_cast<const T*>(a->x);
  ep.ln_in_w = pp.ln_w;
  ep.ln_in_b = pp.ln_b;
  ep.ln_out_w = static_cast<const T*>(a->norm_out_weight);
  ep.ln_out_b = static_cast<const T*>(a->norm_out_bias);
  ep.w_pout = static_cast<const T*>(a->p_out_weight);
  ep.w_gout = static_cast<const T*>(a->g_out_weight);
  ep.residual = static_cast<const T*>(a->residual);
  ep.out_mask = static_cast<const T*>(a->out_mask);
  ep.out = static_cast<T*>(a->out);
  ep.n = a->n;
  ep.eps = a->eps;
  ep.cw = cw;
  return timed(K_TRIMUL_EPILOGUE, st, "trimul_epilogue", [&] { launch_trimul_epilogue<T>(ep, a->batch, st); });
}

// ---------------------------------------------------------- tri-attn body
template <typename T>
int triattn_run(const fjx_triattn_args* a, hipStream_t st) {
  const int64_t n = a->n;
  const int64_t np = round64(n);
  const TriAttnWs ws = triattn_ws(a->batch, n, n, a->heads, a->dtype, true);
  void* W = a->workspace;

  const int cw = a->c_z < 128 ? (int)a->c_z : 0;
  TriAttnPrologueParams<T> pp = {};
  pp.x = static_cast<const T*>(a->x);
  pp.mask = static_cast<const T*>(a->mask);
  pp.ln_w = static_cast<const T*>(a->norm_weight);
  pp.ln_b = static_cast<const T*>(a->norm_bias);
  pp.w_bias = static_cast<const T*>(a->bias_weight);
  pp.w_q = static_cast<const T*>(a->q_weight);
  pp.w_k = static_cast<const T*>(a->k_weight);
  pp.w_v = static_cast<const T*>(a->v_weight);
  pp.q = at<T>(W, ws.q);
  pp.k = at<T>(W, ws.k);
  pp.vt = at<T>(W, ws.vt);
  pp.bias = at<T>(W, ws.bias);
  pp.mb = at<float>(W, ws.mb);
  pp.n = n;
  pp.np = np;
  pp.eps = a->eps;
  pp.inf = a->inf;
  pp.q_scale = (1.0f / sqrtf((float)a->head_dim)) * kLog2e;
  pp.transpose = a->starting ? 0 : 1;
  pp.cw = cw;
  int rc = timed(K_TRIATTN_PROLOGUE, st, "triattn_prologue", [&] { launch_triattn_prologue<T>(pp, a->batch, st); });
  if (rc) return rc;

  FlashParams<T> fp = {};
  fp.q = pp.q;
  fp.k = pp.k;
  fp.vt = pp.vt;
  fp.bias = pp.bias;
  fp.mb = pp.mb;
  fp.out = at<T>(W, ws.o);
  fp.n = n;
  fp.np = np;
  fp.heads = a->heads;
  fp.rows = n;
  // o head-major, [B][N rows][4 heads][N][32]: a workgroup's 128 queries of
  // one head are 8 KB in one piece, and the epilogue's wave for head h reads
  // one 4 KB block per 64-position tile
  fp.o_stride_b = n * n * 128;
  fp.o_stride_row = n * 128;
  fp.o_stride_head = n * 32;
  fp.o_stride_q = 32;
  fp.bias_stride_b = a->heads * np * np;
  fp.fallback = at<unsigned>(W, ws.flags);
  rc = timed(K_TRIATTN_FLASH, st, "triattn_flash", [&] { launch_flash<T>(fp, a->batch, st); });
  if (rc) return rc;

  TriAttnEpilogueParams<T> ep = {};
  ep.o = fp.out;
  ep.x = pp.x;
  ep.ln_w = pp.ln_w;
  ep.ln_b = pp.ln_b;
  ep.w_g = static_cast<const T*>(a->g_weight);
  ep.w_o = static_cast<const T*>(a->o_weight);
  ep.residual = static_cast<const T*>(a->residual);
  ep.out_mask = static_cast<const T*>(a->out_mask);
  ep.out = static_cast<T*>(a->out);
  ep.n = n;
  ep.eps = a->eps;
  ep.transpose = pp.transpose;
  ep.cw = cw;
  return timed(K_TRIATTN_EPILOGUE, st, "triattn_epilogue", [&] { launch_triattn_epilogue<T>(ep, a->batch, st); });
}

template <typename T>
int core_run(const fjx_triattn_core_args* a, hipStream_t st) {
  const int64_t n = a->n;
  const int64_t np = round64(n);
  const int64_t hr = a->batch * a->rows * a->heads;
  const TriAttnWs ws = triattn_ws(a->batch, a->rows, n, a->heads, a->dtype, false);
  void* W = a->workspace;
  T* q = at<T>(W, ws.q);
  T* k = at<T>(W, ws.k);
  T* vt = at<T>(W, ws.vt);
  T* bias = at<T>(W, ws.bias);
  float* mb = at<float>(W, ws.mb);
  int rc = timed(K_TRIATTN_CORE_PREP, st, "triattn_core_prep", [&] {
    hipLaunchKernelGGL(pad_qk_kernel<T>, grid_for(hr * np * 32), dim3(256), 0, st,
                       static_cast<const T*>(a->q), q, n, np, hr, a->scale * kLog2e);
    hipLaunchKernelGGL(pad_qk_kernel<T>, grid_for(hr * np * 32), dim3(256), 0, st,
                       static_cast<const T*>(a->k), k, n, np, hr, 1.0f);
    hipLaunchKernelGGL(transpose_v_kernel<T>, grid_for(hr * np * 32), dim3(256), 0, st,
                       static_cast<const T*>(a->v), vt, n, np, hr);
    hipLaunchKernelGGL(pad_bias_kernel<T>, grid_for(a->batch * a->heads * np * np), dim3(256), 0, st,
                       static_cast<const T*>(a->tri_bias), bias, n, np, a->batch * a->heads);
    hipLaunchKernelGGL(pad_mb_kernel, grid_for(a->batch * a->rows * np), dim3(256), 0, st, a->mask_bias, mb, n,
                       np, a->batch * a->rows);
  });
  if (rc) return rc;

  FlashParams<T> fp = {};
  fp.q = q;
  fp.k = k;
  fp.vt = vt;
  fp.bias = bias;
  fp.mb = mb;
  fp.out = static_cast<T*>(a->out);
  fp.n = n;
  fp.np = np;
  fp.heads = a->heads;
  fp.rows = a->rows;
  fp.o_stride_b = a->rows * a->heads * n * 32;
  fp.o_stride_row = a->heads * n * 32;
  fp.o_stride_head = n * 32;
  fp.o_stride_q = 32;
  fp.bias_stride_b = a->heads * np * np;
  fp.fallback = at<unsigned>(W, ws.flags);
  return timed(K_TRIATTN_FLASH, st, "triattn_flash", [&] { launch_flash<T>(fp, a->batch, st); });
}

// -------------------------------------------------------- transition body
template <typename T>
int transition_run(const fjx_transition_args* a, bool pb_fused, hipStream_t st) {
  TransitionParams<T> p = {};
  p.x = static_cast<const T*>(a->x);
  p.ln_w = static_cast<const T*>(a->norm_weight);
  p.ln_b = static_cast<const T*>(a->norm_bias);
  p.w_a = static_cast<const T*>(a->w_a);
  p.w_b = static_cast<const T*>(a->w_b);
  p.w_o = static_cast<const T*>(a->w_o);
  p.row_mask = static_cast<const T*>(a->row_mask);
  p.residual = static_cast<const T*>(a->residual);
  p.out_mask = static_cast<const T*>(a->out_mask);
  p.out = static_cast<T*>(a->out);
  p.rows = a->rows;
  p.eps = a->eps;
  p.cw = a->c < 128 ? (int)a->c : 0;
  const bool pb_f32 = pb_fused && a->pb_f32 && std::is_same<T, bf16>::value;
  if (pb_fused) {
    if (pb_f32) {
      p.pbf_ln_w = static_cast<const float*>(a->pb_norm_weight);
      p.pbf_ln_b = static_cast<const float*>(a->pb_norm_bias);
      p.pbf_w = static_cast<const float*>(a->pb_weight);
      p.pbf_out = static_cast<float*>(a->pb_out);
    } else {
      p.pb_ln_w = static_cast<const T*>(a->pb_norm_weight);
      p.pb_ln_b = static_cast<const T*>(a->pb_norm_bias);
      p.pb_w = static_cast<const T*>(a->pb_weight);
      p.pb_out = static_cast<T*>(a->pb_out);
    }
    p.pb_n = a->pb_n;
    p.pb_np = round64(a->pb_n);
    p.pb_heads = (int)a->pb_heads;
    p.pb_eps = a->pb_eps;
  }
  return timed(K_TRANSITION, st, "transition", [&] {
    const int64_t planes = pb_fused ? a->rows / (a->pb_n * a->pb_n) * a->pb_heads : 0;
    if (pb_f32)
      launch_pair_bias_border<float>(p.pbf_out, planes, a->pb_n, p.pb_np, st);
    else if (pb_fused)
      launch_pair_bias_border<T>(p.pb_out, planes, a->pb_n, p.pb_np, st);
    launch_transition<T>(p, (int)a->c, st);
  });
}

// the pair-bias output of a transition that could not fuse it: the same
// projection as the single attention's own, over the transition's output
template <typename T>
int transition_pair_bias_pass(const fjx_transition_args* a, hipStream_t st) {
  const int64_t batch = a->rows / (a->pb_n * a->pb_n);
  if (a->pb_f32 && std::is_same<T, bf16>::value)
    return timed(K_SINGLE_PAIR_BIAS, st, "single_pair_bias", [&] {
      launch_pair_bias<bf16, float>(static_cast<const bf16*>(a->out), static_cast<const float*>(a->pb_norm_weight),
                                    static_cast<const float*>(a->pb_norm_bias), static_cast<const float*>(a->pb_weight),
                                    static_cast<float*>(a->pb_out), batch, a->pb_n, round64(a->pb_n),
                                    (int)a->pb_heads, a->pb_eps, st);
    });
  return timed(K_SINGLE_PAIR_BIAS, st, "single_pair_bias", [&] {
    launch_pair_bias<T, T>(static_cast<const T*>(a->out), static_cast<const T*>(a->pb_norm_weight),
                        static_cast<const T*>(a->pb_norm_bias), static_cast<const T*>(a->pb_weight),
                        static_cast<T*>(a->pb_out), batch, a->pb_n, round64(a->pb_n), (int)a->pb_heads, a->pb_eps,
                        st);
  });
}

// ------------------------------------------------- general-width paths
// Widths the fused kernels are not built for (wider tracks such as 384,
// hidden widths other than 128): row LayerNorms, GEMMs and layout passes
// around the same contraction and flash kernels (fjx_generic.hip).
// The fused kernels also take a narrow pair width c_z of 32, 64 or 96 (the
// Protenix template stack's 64 among them), with the channels past c_z held
// at zero.
bool fused_width(int64_t c) { return c == 128 || (c >= 32 && c < 128 && c % 32 == 0); }
bool fused_trimul(int64_t c_z, int64_t c_h) { return fused_width(c_z) && c_h == 128; }
bool fused_triattn(int64_t c_z, int64_t heads, int64_t head_dim) {
  return fused_width(c_z) && head_dim == 32 && heads * head_dim == 128;
}
bool fused_transition(int64_t c, int64_t hidden) { return fused_width(c) && hidden == 4 * c; }
int64_t transition_hidden(const fjx_transition_args* a) { return a->hidden > 0 ? a->hidden : 4 * a->c; }

template <typename T>
GemmParams<T, T> rows_gemm(const T* x, int64_t rows, int64_t k, const void* w, int64_t n_out, T* out, int64_t ldc) {
  GemmParams<T, T> g = {};
  g.a = x;
  g.b = static_cast<const T*>(w);
  g.c = out;
  g.m = rows;
  g.n = n_out;
  g.k = k;
  g.lda = k;
  g.ldb = k;
  g.ldc = ldc;
  g.batches = 1;
  return g;
}

struct GenTriMulWs {
  size_t xn, pg, acm, bcm, ocm, g2, wcat, total;
};
GenTriMulWs gen_trimul_ws(int64_t batch, int64_t n, int64_t c_z, int64_t c_h, int32_t dtype) {
  const size_t pos = (size_t)batch * n * n * esize(dtype);
  GenTriMulWs w;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += align_up(bytes);
    return at;
  };
  w.xn = take(pos * c_z);
  w.pg = take(pos * 2 * c_h);  // G, then P = (x p_in^T) * G, then o position-major
  w.acm = take(pos * c_h);     // a, then LN_out(o)
  w.bcm = take(pos * c_h);
  w.ocm = take(pos * c_h);
  w.g2 = take(pos * c_z);
  w.wcat = take((size_t)4 * c_h * c_z * esize(dtype));  // p_in and g_in interleaved by 128 rows (the pair GEMM)
  w.total = off;
  return w;
}

template <typename T>
int trimul_generic_run(const fjx_trimul_args* a, hipStream_t st) {
  const int64_t B = a->batch, n = a->n, nn = n * n, cz = a->c_z, ch = a->c_h, rows = B * nn;
  const GenTriMulWs ws = gen_trimul_ws(B, n, cz, ch, a->dtype);
  void* W = a->workspace;
  T* xn = at<T>(W, ws.xn);
  T* pg = at<T>(W, ws.pg);
  T* acm = at<T>(W, ws.acm);
  T* bcm = at<T>(W, ws.bcm);
  T* ocm = at<T>(W, ws.ocm);
  T* g2 = at<T>(W, ws.g2);
  const int t = a->direction == FJX_INCOMING;
  const T* mask = static_cast<const T*>(a->mask);

  int rc = timed(K_TRIMUL_PROLOGUE, st, "trimul_prologue", [&] {
    launch_ln_grid<T>(static_cast<const T*>(a->x), static_cast<const T*>(a->norm_in_weight),
                      static_cast<const T*>(a->norm_in_bias), xn, B, n, (int)cz, a->eps, 0, st);
    bool fused = false;
    if constexpr (std::is_same<T, bf16>::value) {
      // (x p_in^T) * sigmoid(x g_in^T) as one GEMM over the interleaved weights
      T* wcat = at<T>(W, ws.wcat);
      GemmParams<T, T> g = rows_gemm<T>(xn, rows, cz, wcat, 4 * ch, pg, 2 * ch);
      g.swiglu = 2;
      if ((2 * ch) % 128 == 0 && gemm_dma_ok(g)) {
        const size_t blk = (size_t)128 * cz * sizeof(T);
        fused = hipMemcpy2DAsync(wcat, 2 * blk, a->p_in_weight, blk, blk, 2 * ch / 128, hipMemcpyDeviceToDevice,
                                 st) == hipSuccess &&
                hipMemcpy2DAsync(reinterpret_cast<char*>(wcat) + blk, 2 * blk, a->g_in_weight, blk, blk,
                                 2 * ch / 128, hipMemcpyDeviceToDevice, st) == hipSuccess &&
                launch_gemm_dma(g, st);
      }
    }
    if (!fused) {
      GemmParams<T, T> g = rows_gemm<T>(xn, rows, cz, a->g_in_weight, 2 * ch, pg, 2 * ch);
      g.act = 1;
      launch_gemm<T, T>(g, st);
      g = rows_gemm<T>(xn, rows, cz, a->p_in_weight, 2 * ch, pg, 2 * ch);
      g.gate = pg;  // in place: each element reads its gate, then is overwritten
      launch_gemm<T, T>(g, st);
    }
    launch_to_channel_major<T>(pg, 2 * ch, 0, (int)ch, mask, acm, B, n, t, st);
    launch_to_channel_major<T>(pg, 2 * ch, (int)ch, (int)ch, mask, bcm, B, n, t, st);
  });
  if (rc) return rc;

  rc = timed(K_TRIMUL_CONTRACT, st, "trimul_contract", [&] {
    if constexpr (std::is_same<T, bf16>::value) {
      launch_contract(acm, bcm, ocm, n, B * ch, st);
    } else {
      GemmParams<T, T> cp = {};
      cp.a = acm;
      cp.b = bcm;
      cp.c = ocm;
      cp.m = cp.n = cp.k = n;
      cp.lda = cp.ldb = cp.ldc = n;
      cp.sa = cp.sb = cp.sc = nn;
      cp.batches = B * ch;
      launch_gemm<T, T>(cp, st);
    }
  });
  if (rc) return rc;

  return timed(K_TRIMUL_EPILOGUE, st, "trimul_epilogue", [&] {
    launch_to_position_major<T>(ocm, (int)ch, pg, B, nn, st);
    launch_layernorm_rows<T>(pg, static_cast<const T*>(a->norm_out_weight), static_cast<const T*>(a->norm_out_bias),
                             acm, rows, (int)ch, a->eps, st);
    GemmParams<T, T> g = rows_gemm<T>(xn, rows, cz, a->g_out_weight, cz, g2, cz);
    g.act = 1;
    launch_gemm<T, T>(g, st);
    g = rows_gemm<T>(acm, rows, ch, a->p_out_weight, cz, static_cast<T*>(a->out), cz);
    g.gate = g2;
    g.residual = static_cast<const T*>(a->residual);
    g.row_gate = static_cast<const T*>(a->out_mask);
    bool direct = false;
    if constexpr (std::is_same<T, bf16>::value) direct = gemm_dma_ok(g);
    if (direct) {
      launch_gemm<T, T>(g, st);
    } else {
      // the gated product into xn (no longer read), then a vectorized pass
      // adds the residual and applies the output mask
      g.c = xn;
      g.residual = nullptr;
      g.row_gate = nullptr;
      launch_gemm<T, T>(g, st);
      launch_scatter_add<T>(xn, nullptr, static_cast<const T*>(a->residual), static_cast<const T*>(a->out_mask),
                            static_cast<T*>(a->out), rows, n, (int)cz, 0, st);
    }
  });
}

struct GenTriAttnWs {
  size_t xn, proj, bias_pm, q, k, vt, bias, mb, o, wcat, flags, total;
};
GenTriAttnWs gen_triattn_ws(int64_t batch, int64_t n, int64_t c_z, int64_t heads, int32_t dtype) {
  const int64_t np = round64(n), hd = 32 * heads;
  const size_t es = esize(dtype), pos = (size_t)batch * n * n * es;
  GenTriAttnWs w;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += align_up(bytes);
    return at;
  };
  w.xn = take(pos * c_z);
  w.proj = take(pos * 4 * hd);  // q | k | v | sigmoid(g)
  w.bias_pm = take(pos * heads);
  w.q = take((size_t)batch * n * heads * np * 32 * es);
  w.k = take((size_t)batch * n * heads * np * 32 * es);
  w.vt = take((size_t)batch * n * heads * np * 32 * es);
  w.bias = take((size_t)batch * heads * np * np * es);
  w.mb = take((size_t)batch * n * np * sizeof(float));
  w.o = take(pos * hd);
  w.wcat = take((size_t)4 * hd * c_z * es);  // w_q | w_k | w_v | w_g back to back (one projection GEMM)
  w.flags = take(flash_flags_bytes(batch, n, heads, np));
  w.total = off;
  return w;
}

template <typename T>
int triattn_generic_run(const fjx_triattn_args* a, hipStream_t st) {
  const int64_t B = a->batch, n = a->n, nn = n * n, cz = a->c_z, H = a->heads, hd = 32 * H, rows = B * nn;
  const int64_t np = round64(n);
  const GenTriAttnWs ws = gen_triattn_ws(B, n, cz, H, a->dtype);
  void* W = a->workspace;
  T* xn = at<T>(W, ws.xn);
  T* proj = at<T>(W, ws.proj);
  T* bpm = at<T>(W, ws.bias_pm);
  const int t = a->starting ? 0 : 1;

  int rc = timed(K_TRIATTN_PROLOGUE, st, "triattn_prologue", [&] {
    launch_ln_grid<T>(static_cast<const T*>(a->x), static_cast<const T*>(a->norm_weight),
                      static_cast<const T*>(a->norm_bias), xn, B, n, (int)cz, a->eps, t, st);
    // q | k | v | sigmoid(g) as one GEMM over the weights back to back (the
    // caller's, when they already are; else a copy in the workspace)
    const void* wq[4] = {a->q_weight, a->k_weight, a->v_weight, a->g_weight};
    const int nw = a->g_weight ? 4 : 3;
    const size_t wbytes = (size_t)hd * cz * sizeof(T);
    bool contiguous = true;
    for (int j = 1; j < nw; ++j)
      contiguous = contiguous && static_cast<const char*>(wq[j]) == static_cast<const char*>(wq[0]) + j * wbytes;
    const T* wcat = static_cast<const T*>(a->q_weight);
    bool ok = true;
    if (!contiguous) {
      T* dst = at<T>(W, ws.wcat);
      for (int j = 0; j < nw && ok; ++j)
        ok = hipMemcpyAsync(reinterpret_cast<char*>(dst) + j * wbytes, wq[j], wbytes, hipMemcpyDeviceToDevice, st) ==
             hipSuccess;
      wcat = dst;
    }
    if (ok) {
      GemmParams<T, T> g = rows_gemm<T>(xn, rows, cz, wcat, nw * hd, proj, 4 * hd);
      g.act = 1;  // sigmoid on the gate columns only
      g.act_col0 = 3 * hd;
      launch_gemm<T, T>(g, st);
    } else {
      for (int j = 0; j < nw; ++j) {
        GemmParams<T, T> g = rows_gemm<T>(xn, rows, cz, wq[j], hd, proj + j * hd, 4 * hd);
        g.act = j == 3 ? 1 : 0;
        launch_gemm<T, T>(g, st);
      }
    }
    launch_gemm<T, T>(rows_gemm<T>(xn, rows, cz, a->bias_weight, H, bpm, H), st);
    launch_split_qk<T>(proj, 4 * hd, 0, at<T>(W, ws.q), B * n, n, np, (int)H,
                       (1.0f / sqrtf((float)a->head_dim)) * kLog2e, st);
    launch_split_qk<T>(proj, 4 * hd, hd, at<T>(W, ws.k), B * n, n, np, (int)H, 1.0f, st);
    launch_split_vt<T>(proj, 4 * hd, 2 * hd, at<T>(W, ws.vt), B * n, n, np, (int)hd, st);
    launch_bias_planes<T>(bpm, H, 0, at<T>(W, ws.bias), B, n, np, (int)H, st);
    launch_grid_mask_bias<T>(static_cast<const T*>(a->mask), at<float>(W, ws.mb), B, n, np, a->inf, t, st);
  });
  if (rc) return rc;

  FlashParams<T> fp = {};
  fp.q = at<T>(W, ws.q);
  fp.k = at<T>(W, ws.k);
  fp.vt = at<T>(W, ws.vt);
  fp.bias = at<T>(W, ws.bias);
  fp.mb = at<float>(W, ws.mb);
  fp.out = at<T>(W, ws.o);
  fp.n = n;
  fp.np = np;
  fp.heads = H;
  fp.rows = n;
  fp.o_stride_b = nn * hd;
  fp.o_stride_row = n * hd;
  fp.o_stride_head = 32;
  fp.o_stride_q = hd;
  fp.bias_stride_b = H * np * np;
  fp.fallback = at<unsigned>(W, ws.flags);
  rc = timed(K_TRIATTN_FLASH, st, "triattn_flash", [&] { launch_flash<T>(fp, B, st); });
  if (rc) return rc;

  return timed(K_TRIATTN_EPILOGUE, st, "triattn_epilogue", [&] {
    if (a->g_weight) launch_gate_rows<T>(fp.out, proj, 4 * hd, 3 * hd, rows, (int)hd, st);
    // the output projection stores straight into the original grid (the
    // ending node's rows transposed) with the residual and the output mask
    GemmParams<T, T> g = rows_gemm<T>(fp.out, rows, hd, a->o_weight, cz, static_cast<T*>(a->out), cz);
    g.proj_round = 1;
    g.residual = static_cast<const T*>(a->residual);
    g.row_gate = static_cast<const T*>(a->out_mask);
    g.map_t = t;
    g.map_n = n;
    bool direct = false;
    if constexpr (std::is_same<T, bf16>::value) direct = gemm_dma_ok(g);
    if (direct) {
      launch_gemm<T, T>(g, st);
    } else {
      // the product into xn (read only by the prologue), then a vectorized
      // pass scatters it to the original grid with the residual and mask
      launch_gemm<T, T>(rows_gemm<T>(fp.out, rows, hd, a->o_weight, cz, xn, cz), st);
      launch_scatter_add<T>(xn, nullptr, static_cast<const T*>(a->residual), static_cast<const T*>(a->out_mask),
                            static_cast<T*>(a->out), rows, n, (int)cz, t, st);
    }
  });
}

// K splits of the fp32 output projection of the general transition: its
// [rows, c] output is a grid of few 64 x 64 tiles (the 384-wide single track:
// 96 at 1024 rows) whose k loop runs the whole hidden width; split, the
// partial products go to the workspace and the scatter pass sums them. bf16
// keeps one product (its projection rounds the whole sum once).
int transition_out_splits(int64_t rows, int64_t c, int64_t hidden, int32_t dtype) {
  if (dtype != FJX_DTYPE_F32) return 1;
  const int64_t tiles = ((rows + 63) / 64) * ((c + 63) / 64);
  int s = 1;
  while (s < 8 && tiles * s < 256 && hidden % (16 * s) == 0 && hidden / (2 * s) >= 128) s *= 2;
  return s;
}

struct GenTransitionWs {
  size_t xn, h, wcat, y, total;
};
GenTransitionWs gen_transition_ws(int64_t rows, int64_t c, int64_t hidden, int32_t dtype) {
  const size_t es = esize(dtype);
  GenTransitionWs w;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += align_up(bytes);
    return at;
  };
  w.xn = take((size_t)rows * c * es);
  w.h = take((size_t)rows * hidden * es);
  w.wcat = take((size_t)2 * hidden * c * es);  // W_a and W_b interleaved by 128 rows (the fused SwiGLU GEMM)
  // the output projection (each of its K splits), when its GEMM cannot apply the epilogue
  w.y = take((size_t)transition_out_splits(rows, c, hidden, dtype) * rows * c * es);
  w.total = off;
  return w;
}

template <typename T>
int transition_generic_run(const fjx_transition_args* a, hipStream_t st) {
  const int64_t rows = a->rows, c = a->c, hid = transition_hidden(a);
  const GenTransitionWs ws = gen_transition_ws(rows, c, hid, a->dtype);
  void* W = a->workspace;
  T* xn = at<T>(W, ws.xn);
  T* h = at<T>(W, ws.h);
  // the 384-channel single track is timed apart from the pair track
  const int id = c == 384 ? K_SINGLE_TRANSITION : K_TRANSITION;
  return timed(id, st, "transition", [&] {
    launch_layernorm_rows<T>(static_cast<const T*>(a->x), static_cast<const T*>(a->norm_weight),
                             static_cast<const T*>(a->norm_bias), xn, rows, (int)c, a->eps, st);
    bool fused = false;
    if constexpr (std::is_same<T, bf16>::value) {
      // silu(x W_a^T) * (x W_b^T) as one GEMM over the interleaved weights
      T* wcat = at<T>(W, ws.wcat);
      GemmParams<T, T> g = rows_gemm<T>(xn, rows, c, wcat, 2 * hid, h, hid);
      g.swiglu = 1;
      if (hid % 128 == 0 && gemm_dma_ok(g)) {
        const size_t blk = (size_t)128 * c * sizeof(T);  // one block of 128 weight rows
        fused = hipMemcpy2DAsync(wcat, 2 * blk, a->w_a, blk, blk, hid / 128, hipMemcpyDeviceToDevice, st) ==
                    hipSuccess &&
                hipMemcpy2DAsync(reinterpret_cast<char*>(wcat) + blk, 2 * blk, a->w_b, blk, blk, hid / 128,
                                 hipMemcpyDeviceToDevice, st) == hipSuccess &&
                launch_gemm_dma(g, st);
      }
    }
    if (!fused) {
      GemmParams<T, T> g = rows_gemm<T>(xn, rows, c, a->w_a, hid, h, hid);
      g.act = 2;
      launch_gemm<T, T>(g, st);
      g = rows_gemm<T>(xn, rows, c, a->w_b, hid, h, hid);
      g.gate = h;  // in place
      launch_gemm<T, T>(g, st);
    }
    // the output projection with the row mask, the residual and the output
    // mask in the DMA GEMM's epilogue (rows map to themselves); a product it
    // does not take goes to a buffer and a vectorized pass adds them
    GemmParams<T, T> g = rows_gemm<T>(h, rows, hid, a->w_o, c, static_cast<T*>(a->out), c);
    g.proj_round = 1;
    g.row_scale = static_cast<const T*>(a->row_mask);
    g.residual = static_cast<const T*>(a->residual);
    g.row_gate = static_cast<const T*>(a->out_mask);
    bool direct = false;
    if constexpr (std::is_same<T, bf16>::value) direct = gemm_dma_ok(g);
    if (direct) {
      launch_gemm<T, T>(g, st);
    } else {
      T* y = at<T>(W, ws.y);
      const int splits = transition_out_splits(rows, c, hid, a->dtype);
      // split s: hidden columns s kc .. (s + 1) kc - 1 into y + s rows c
      GemmParams<T, T> gy = rows_gemm<T>(h, rows, hid / splits, a->w_o, c, y, c);
      gy.lda = gy.ldb = hid;
      gy.batches = splits;
      gy.sa = gy.sb = hid / splits;
      gy.sc = rows * c;
      launch_gemm<T, T>(gy, st);
      launch_scatter_add<T>(y, static_cast<const T*>(a->row_mask), static_cast<const T*>(a->residual),
                            static_cast<const T*>(a->out_mask), static_cast<T*>(a->out), rows, 1, (int)c, 0, st,
                            splits, rows * c);
    }
  });
}

// ------------------------------------------------ single-track attention
struct SingleWs {
  size_t s_ln, qkvg, q, k, vt, bias, mb, o, go, total;
};
SingleWs single_ws(int64_t batch, int64_t n, int64_t c_s, int64_t heads, int32_t dtype) {
  const int64_t np = round64(n);
  const size_t es = esize(dtype);
  SingleWs w;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off += align_up(bytes);
    return at;
  };
  w.s_ln = take((size_t)batch * n * c_s * es);
  w.qkvg = take((size_t)batch * n * 4 * c_s * es);
  w.q = take((size_t)batch * heads * np * 32 * es);
  w.k = take((size_t)batch * heads * np * 32 * es);
  w.vt = take((size_t)batch * heads * np * 32 * es);
  w.bias = take((size_t)batch * heads * np * np * es);
  w.mb = take((size_t)batch * np * sizeof(float));
  w.o = take((size_t)batch * n * heads * 32 * es);
  w.go = take((size_t)batch * n * c_s * es);
  w.total = off;
  return w;
}

// T: s, the weights and the attention; TZ: the pair tensor z
template <typename T, typename TZ>
int single_run(const fjx_single_attention_args* a, hipStream_t st) {
  const int64_t B = a->batch, n = a->n, cs = a->c_s, H = a->heads;
  const int64_t np = round64(n);
  const int dh = (int)(cs / H);
  const SingleWs ws = single_ws(B, n, cs, H, a->dtype);
  void* W = a->workspace;
  T* s_ln = at<T>(W, ws.s_ln);
  T* qkvg = at<T>(W, ws.qkvg);
  const T* s_in = static_cast<const T*>(a->s);

  int rc = timed(K_SINGLE_PROJ, st, "single_proj", [&] {
    if (a->pre_norm_weight)
      launch_layernorm_rows<T>(s_in, static_cast<const T*>(a->pre_norm_weight),
                               static_cast<const T*>(a->pre_norm_bias), s_ln, B * n, (int)cs, a->eps, st);
    const T* ws_[4] = {static_cast<const T*>(a->q_weight), static_cast<const T*>(a->k_weight),
                       static_cast<const T*>(a->v_weight), static_cast<const T*>(a->g_weight)};
    // weights stored back to back ([4 c_s, c_s], as the package packs them)
    // run as one GEMM of four times the width: four times the tiles in flight
    const bool stacked = ws_[1] == ws_[0] + cs * cs && ws_[2] == ws_[1] + cs * cs && ws_[3] == ws_[2] + cs * cs;
    for (int j = 0; j < (stacked ? 1 : 4); ++j) {
      GemmParams<T, T> g = {};
      g.a = a->pre_norm_weight ? s_ln : s_in;
      g.b = ws_[j];
      g.c = qkvg + j * cs;
      g.m = B * n;
      g.n = stacked ? 4 * cs : cs;
      g.k = cs;
      g.lda = cs;
      g.ldb = cs;
      g.ldc = 4 * cs;
      g.batches = 1;
      g.bias = j == 0 ? static_cast<const T*>(a->q_bias) : nullptr;
      g.bias_n = cs;
      g.act = stacked || j == 3 ? 1 : 0;
      g.act_col0 = stacked ? 3 * cs : 0;  // the gate's columns
      launch_gemm<T, T>(g, st);
    }
    launch_split_heads<T>(qkvg, 4 * cs, B, n, np, (int)H, dh, (1.0f / sqrtf((float)dh)) * kLog2e,
                          at<T>(W, ws.q), at<T>(W, ws.k), at<T>(W, ws.vt), st);
    launch_key_mask<T>(static_cast<const T*>(a->mask), at<float>(W, ws.mb), B, n, np, a->inf, st);
  });
  if (rc) return rc;
  if (!a->pair_bias || a->extra_bias) {
    rc = timed(K_SINGLE_PAIR_BIAS, st, "single_pair_bias", [&] {
      if (!a->pair_bias)
        launch_pair_bias<TZ, T>(static_cast<const TZ*>(a->z), static_cast<const T*>(a->z_norm_weight),
                                static_cast<const T*>(a->z_norm_bias), static_cast<const T*>(a->z_weight),
                                at<T>(W, ws.bias), B, n, np, (int)H, a->eps, st);
      if (a->extra_bias)
        launch_add_extra_bias<T>(static_cast<const T*>(a->pair_bias), at<T>(W, ws.bias),
                                 static_cast<const T*>(a->extra_bias), a->extra_bias_stride_b, a->extra_bias_stride_h,
                                 B, (int)H, n, np, st);
    });
    if (rc) return rc;
  }

  FlashParams<T> fp = {};
  fp.q = at<T>(W, ws.q);
  fp.k = at<T>(W, ws.k);
  fp.vt = at<T>(W, ws.vt);
  fp.bias = a->pair_bias && !a->extra_bias ? static_cast<const T*>(a->pair_bias) : at<T>(W, ws.bias);
  fp.mb = at<float>(W, ws.mb);
  fp.out = at<T>(W, ws.o);
  fp.n = n;
  fp.np = np;
  fp.heads = H;
  fp.rows = 1;
  fp.o_stride_b = n * H * 32;
  fp.o_stride_row = 0;
  fp.o_stride_head = 32;
  fp.o_stride_q = H * 32;
  fp.bias_stride_b = H * np * np;
  rc = timed(K_SINGLE_FLASH, st, "single_flash", [&] { launch_flash<T>(fp, B, st); });
  if (rc) return rc;

  return timed(K_SINGLE_OUT, st, "single_out", [&] {
    T* go = at<T>(W, ws.go);
    launch_gate_unpad<T>(fp.out, qkvg + 3 * cs, 4 * cs, go, B * n, (int)H, dh, st);
    GemmParams<T, T> g = {};
    g.a = go;
    g.b = static_cast<const T*>(a->o_weight);
    g.c = static_cast<T*>(a->out);
    g.m = B * n;
    g.n = cs;
    g.k = cs;
    g.lda = cs;
    g.ldb = cs;
    g.ldc = cs;
    g.batches = 1;
    g.residual = static_cast<const T*>(a->residual);
    g.row_gate = static_cast<const T*>(a->out_mask);
    launch_gemm<T, T>(g, st);
  });
}

bool dtype_ok(int32_t dt) { return dt == FJX_DTYPE_F32 || dt == FJX_DTYPE_BF16; }

// grid dimensions are 32-bit; y/z additionally capped at 65535
bool grid_ok(int64_t n, int64_t batch) { return n <= 65535 && batch <= 65535; }

// every kernel moves rows in 16-byte pieces; NULL (an absent optional) passes
bool aligned16(std::initializer_list<const void*> ps) {
  for (const void* q : ps)
    if (reinterpret_cast<uintptr_t>(q) & 15u) return false;
  return true;
}

// every check of fjx_trimul_fwd except the workspace's; `fn` names the entry point in messages
int trimul_check(const fjx_trimul_args* a, const char* fn) {
  if (!a) return fail(FJX_ERR_INVALID, "%s: args is NULL", fn);
  if (a->batch < 1 || a->n < 1) return fail(FJX_ERR_INVALID, "%s: batch and n must be >= 1", fn);
  if (!dtype_ok(a->dtype)) return fail(FJX_ERR_INVALID, "%s: unknown dtype %d", fn, a->dtype);
  if (a->direction != FJX_OUTGOING && a->direction != FJX_INCOMING)
    return fail(FJX_ERR_INVALID, "Unsupported triangle multiplication direction: %d", a->direction);
  if (a->c_z < 8 || a->c_h < 8 || a->c_z % 8 || a->c_h % 8 || a->c_z > 1024 || a->c_h > 1024)
    return fail(FJX_ERR_UNSUPPORTED, "%s: c_z and c_h must be multiples of 8 in [8, 1024], got c_z=%lld c_h=%lld",
                fn, (long long)a->c_z, (long long)a->c_h);
  if (!grid_ok(a->n, a->batch)) return fail(FJX_ERR_UNSUPPORTED, "%s: n or batch too large", fn);
  if (!a->x || !a->out || !a->norm_in_weight || !a->norm_in_bias || !a->p_in_weight || !a->g_in_weight ||
      !a->norm_out_weight || !a->norm_out_bias || !a->p_out_weight || !a->g_out_weight)
    return fail(FJX_ERR_INVALID, "%s: a required pointer is NULL", fn);
  if (!aligned16({a->x, a->out, a->residual, a->norm_in_weight, a->norm_in_bias, a->p_in_weight, a->g_in_weight,
                  a->norm_out_weight, a->norm_out_bias, a->p_out_weight, a->g_out_weight}))
    return fail(FJX_ERR_INVALID, "%s: tensors must be 16-byte aligned", fn);
  return FJX_OK;
}

int trimul_dispatch(const fjx_trimul_args* a, hipStream_t st) {
  if (!fused_trimul(a->c_z, a->c_h))
    return a->dtype == FJX_DTYPE_BF16 ? trimul_generic_run<bf16>(a, st) : trimul_generic_run<float>(a, st);
  return a->dtype == FJX_DTYPE_BF16 ? trimul_run<bf16>(a, st) : trimul_run<float>(a, st);
}

}  // namespace

extern "C" {

const char* fjx_last_error(void) { return g_err.c_str(); }
int fjx_abi_version(void) { return FJX_ABI_VERSION; }

size_t fjx_trimul_workspace_size(int64_t batch, int64_t n, int64_t c_z, int64_t c_h, int32_t dtype) {
  if (batch < 1 || n < 1 || c_z < 1 || c_h < 1 || !dtype_ok(dtype)) return 0;
  return fused_trimul(c_z, c_h) ? trimul_ws(batch, n, dtype).total : gen_trimul_ws(batch, n, c_z, c_h, dtype).total;
}


int fjx_trimul_fwd(const fjx_trimul_args* a, hipStream_t st) {
  g_err.clear();
  if (int rc = trimul_check(a, "fjx_trimul_fwd")) return rc;
  const size_t need = fjx_trimul_workspace_size(a->batch, a->n, a->c_z, a->c_h, a->dtype);
  if (!a->workspace || a->workspace_bytes < need)
    return fail(FJX_ERR_WORKSPACE, "fjx_trimul_fwd: workspace of %zu bytes needed, %zu given", need,
                a->workspace_bytes);
  return trimul_dispatch(a, st);
}


size_t fjx_triattn_workspace_size(int64_t batch, int64_t n, int64_t c_z, int64_t heads, int64_t head_dim,
                                  int32_t dtype) {
  if (batch < 1 || n < 1 || c_z < 1 || heads < 1 || !dtype_ok(dtype)) return 0;
  return fused_triattn(c_z, heads, head_dim) ? triattn_ws(batch, n, n, heads, dtype, true).total
                                             : gen_triattn_ws(batch, n, c_z, heads, dtype).total;
}

int fjx_triattn_fwd(const fjx_triattn_args* a, hipStream_t st) {
  g_err.clear();
  if (!a) return fail(FJX_ERR_INVALID, "fjx_triattn_fwd: args is NULL");
  if (a->batch < 1 || a->n < 1) return fail(FJX_ERR_INVALID, "fjx_triattn_fwd: batch and n must be >= 1");
  if (!dtype_ok(a->dtype)) return fail(FJX_ERR_INVALID, "fjx_triattn_fwd: unknown dtype %d", a->dtype);
  if (a->heads < 1 || a->head_dim != 32 || a->c_z < 8 || a->c_z % 8 || a->c_z > 1024 || a->heads > 32)
    return fail(FJX_ERR_UNSUPPORTED,
                "fjx_triattn_fwd: this build supports head_dim == 32, 1 <= heads <= 32 and c_z a multiple of 8 in "
                "[8, 1024]; got c_z=%lld heads=%lld head_dim=%lld",
                (long long)a->c_z, (long long)a->heads, (long long)a->head_dim);
  if (!grid_ok(a->n, a->batch)) return fail(FJX_ERR_UNSUPPORTED, "fjx_triattn_fwd: n or batch too large");
  if (!a->x || !a->out || !a->norm_weight || !a->norm_bias || !a->bias_weight || !a->q_weight ||
      !a->k_weight || !a->v_weight || !a->o_weight)
    return fail(FJX_ERR_INVALID, "fjx_triattn_fwd: a required pointer is NULL");
  if (!aligned16({a->x, a->out, a->residual, a->norm_weight, a->norm_bias, a->bias_weight, a->q_weight, a->k_weight,
                  a->v_weight, a->g_weight, a->o_weight}))
    return fail(FJX_ERR_INVALID, "fjx_triattn_fwd: tensors must be 16-byte aligned");
  const bool fused = fused_triattn(a->c_z, a->heads, a->head_dim);
  const size_t need = fjx_triattn_workspace_size(a->batch, a->n, a->c_z, a->heads, a->head_dim, a->dtype);
  if (!a->workspace || a->workspace_bytes < need)
    return fail(FJX_ERR_WORKSPACE, "fjx_triattn_fwd: workspace of %zu bytes needed, %zu given", need,
                a->workspace_bytes);
  if (!fused)
    return a->dtype == FJX_DTYPE_BF16 ? triattn_generic_run<bf16>(a, st) : triattn_generic_run<float>(a, st);
  return a->dtype == FJX_DTYPE_BF16 ? triattn_run<bf16>(a, st) : triattn_run<float>(a, st);
}

size_t fjx_triattn_core_workspace_size(int64_t batch, int64_t rows, int64_t heads, int64_t n, int64_t head_dim,
                                       int32_t dtype) {
  (void)head_dim;
  if (batch < 1 || rows < 1 || heads < 1 || n < 1 || !dtype_ok(dtype)) return 0;
  return triattn_ws(batch, rows, n, heads, dtype, false).total;
}

int fjx_triattn_core(const fjx_triattn_core_args* a, hipStream_t st) {
  g_err.clear();
  if (!a) return fail(FJX_ERR_INVALID, "fjx_triattn_core: args is NULL");
  if (a->batch < 1 || a->rows < 1 || a->heads < 1 || a->n < 1)
    return fail(FJX_ERR_INVALID, "fjx_triattn_core: batch, rows, heads and n must be >= 1");
  if (!dtype_ok(a->dtype)) return fail(FJX_ERR_INVALID, "fjx_triattn_core: unknown dtype %d", a->dtype);
  if (a->head_dim != 32)
    return fail(FJX_ERR_UNSUPPORTED, "fjx_triattn_core: this build supports head_dim == 32, got %lld",
                (long long)a->head_dim);
  if (!a->q || !a->k || !a->v || !a->tri_bias || !a->out)
    return fail(FJX_ERR_INVALID, "fjx_triattn_core: a required pointer is NULL");
  if (!aligned16({a->q, a->k, a->v, a->tri_bias, a->out}))
    return fail(FJX_ERR_INVALID, "fjx_triattn_core: tensors must be 16-byte aligned");
  const size_t need = triattn_ws(a->batch, a->rows, a->n, a->heads, a->dtype, false).total;
  if (!a->workspace || a->workspace_bytes < need)
    return fail(FJX_ERR_WORKSPACE, "fjx_triattn_core: workspace of %zu bytes needed, %zu given", need,
                a->workspace_bytes);
  return a->dtype == FJX_DTYPE_BF16 ? core_run<bf16>(a, st) : core_run<float>(a, st);
}

size_t fjx_transition_workspace_size(int64_t rows, int64_t c, int64_t hidden, int32_t dtype) {
  if (rows < 1 || c < 1 || hidden < 0 || !dtype_ok(dtype)) return 0;
  const int64_t hid = hidden > 0 ? hidden : 4 * c;
  return fused_transition(c, hid) ? 0 : gen_transition_ws(rows, c, hid, dtype).total;
}

int fjx_transition_fwd(const fjx_transition_args* a, hipStream_t st) {
  g_err.clear();
  if (!a) return fail(FJX_ERR_INVALID, "fjx_transition_fwd: args is NULL");
  if (a->rows < 1) return fail(FJX_ERR_INVALID, "fjx_transition_fwd: rows must be >= 1");
  if (!dtype_ok(a->dtype)) return fail(FJX_ERR_INVALID, "fjx_transition_fwd: unknown dtype %d", a->dtype);
  if (a->hidden < 0) return fail(FJX_ERR_INVALID, "fjx_transition_fwd: hidden must be >= 0");
  const int64_t hid = transition_hidden(a);
  if (a->c < 8 || a->c % 8 || a->c > 1024 || hid % 8)
    return fail(FJX_ERR_UNSUPPORTED,
                "fjx_transition_fwd: c must be a multiple of 8 in [8, 1024] and hidden a multiple of 8; got c=%lld "
                "hidden=%lld",
                (long long)a->c, (long long)hid);
  if ((a->rows + 15) / 16 > 0x7fffffffLL) return fail(FJX_ERR_UNSUPPORTED, "fjx_transition_fwd: too many rows");
  if (!a->x || !a->out || !a->norm_weight || !a->norm_bias || !a->w_a || !a->w_b || !a->w_o)
    return fail(FJX_ERR_INVALID, "fjx_transition_fwd: a required pointer is NULL");
  if (!aligned16({a->x, a->out, a->residual, a->norm_weight, a->norm_bias, a->w_a, a->w_b, a->w_o}))
    return fail(FJX_ERR_INVALID, "fjx_transition_fwd: tensors must be 16-byte aligned");
  if (a->pb_out) {
    if (a->c != 128)
      return fail(FJX_ERR_UNSUPPORTED, "fjx_transition_fwd: the pair-bias output needs c == 128; got c=%lld",
                  (long long)a->c);
    if (a->pb_n < 1 || a->pb_n > 65535 || a->pb_heads < 1 || a->pb_heads > 1024 || a->rows % (a->pb_n * a->pb_n))
      return fail(FJX_ERR_INVALID,
                  "fjx_transition_fwd: the pair-bias output needs 1 <= pb_n <= 65535, 1 <= pb_heads <= 1024 and "
                  "rows a multiple of pb_n^2; got rows=%lld pb_n=%lld pb_heads=%lld",
                  (long long)a->rows, (long long)a->pb_n, (long long)a->pb_heads);
    if (!grid_ok(a->pb_n, a->rows / (a->pb_n * a->pb_n)))
      return fail(FJX_ERR_UNSUPPORTED, "fjx_transition_fwd: the pair-bias batch is too large");
    if (!a->pb_norm_weight || !a->pb_norm_bias || !a->pb_weight)
      return fail(FJX_ERR_INVALID, "fjx_transition_fwd: a pair-bias weight pointer is NULL");
    if (a->pb_f32 && a->dtype != FJX_DTYPE_BF16)
      return fail(FJX_ERR_INVALID, "fjx_transition_fwd: pb_f32 is for a bf16 transition (an fp32 one has fp32 pair-bias "
                                   "weights already)");
    if (!aligned16({a->pb_norm_weight, a->pb_norm_bias, a->pb_weight, a->pb_out}))
      return fail(FJX_ERR_INVALID, "fjx_transition_fwd: tensors must be 16-byte aligned");
  }
  const bool bf = a->dtype == FJX_DTYPE_BF16;
  int rc;
  bool pb_fused = false;
  if (fused_transition(a->c, hid)) {
    pb_fused = a->pb_out && a->pb_heads <= 16 && a->c == 128;
    rc = bf ? transition_run<bf16>(a, pb_fused, st) : transition_run<float>(a, pb_fused, st);
  } else {
    const size_t need = fjx_transition_workspace_size(a->rows, a->c, hid, a->dtype);
    if (!a->workspace || a->workspace_bytes < need)
      return fail(FJX_ERR_WORKSPACE, "fjx_transition_fwd: workspace of %zu bytes needed, %zu given", need,
                  a->workspace_bytes);
    rc = bf ? transition_generic_run<bf16>(a, st) : transition_generic_run<float>(a, st);
  }
  if (rc || !a->pb_out || pb_fused) return rc;
  return bf ? transition_pair_bias_pass<bf16>(a, st) : transition_pair_bias_pass<float>(a, st);
}

size_t fjx_pair_bias_size(int64_t batch, int64_t n, int64_t heads, int32_t dtype) {
  if (batch < 1 || n < 1 || heads < 1 || !dtype_ok(dtype)) return 0;
  const int64_t np = round64(n);
  return (size_t)batch * heads * np * np * esize(dtype);
}

size_t fjx_single_attention_workspace_size(int64_t batch, int64_t n, int64_t c_s, int64_t heads, int32_t dtype) {
  if (batch < 1 || n < 1 || c_s < 1 || heads < 1 || !dtype_ok(dtype)) return 0;
  return single_ws(batch, n, c_s, heads, dtype).total;
}

int fjx_single_attention_fwd(const fjx_single_attention_args* a, hipStream_t st) {
  g_err.clear();
  if (!a) return fail(FJX_ERR_INVALID, "fjx_single_attention_fwd: args is NULL");
  if (a->batch < 1 || a->n < 1 || a->heads < 1)
    return fail(FJX_ERR_INVALID, "fjx_single_attention_fwd: batch, n and heads must be >= 1");
  if (!dtype_ok(a->dtype)) return fail(FJX_ERR_INVALID, "fjx_single_attention_fwd: unknown dtype %d", a->dtype);
  if (!dtype_ok(a->z_dtype)) return fail(FJX_ERR_INVALID, "fjx_single_attention_fwd: unknown z_dtype %d", a->z_dtype);
  if (a->extra_bias && (a->extra_bias_stride_b < 0 || a->extra_bias_stride_h < 0))
    return fail(FJX_ERR_INVALID, "fjx_single_attention_fwd: extra_bias strides must be >= 0");
  if ((!a->pair_bias && a->c_z != 128) || a->c_s % a->heads != 0 || a->c_s / a->heads > 32 || a->c_s > 1024)
    return fail(FJX_ERR_UNSUPPORTED,
                "fjx_single_attention_fwd: this build supports c_z == 128, heads dividing c_s <= 1024 with "
                "head_dim <= 32; got c_s=%lld c_z=%lld heads=%lld",
                (long long)a->c_s, (long long)a->c_z, (long long)a->heads);
  if (!grid_ok(a->n, a->batch)) return fail(FJX_ERR_UNSUPPORTED, "fjx_single_attention_fwd: n or batch too large");
  if ((a->pre_norm_weight == nullptr) != (a->pre_norm_bias == nullptr))
    return fail(FJX_ERR_INVALID, "fjx_single_attention_fwd: pre_norm weight and bias must both be given or both NULL");
  if (!a->s || !a->out || !a->q_weight || !a->k_weight || !a->v_weight || !a->g_weight || !a->o_weight ||
      (!a->pair_bias && (!a->z || !a->z_norm_weight || !a->z_norm_bias || !a->z_weight)))
    return fail(FJX_ERR_INVALID, "fjx_single_attention_fwd: a required pointer is NULL");
  if (!aligned16({a->s, a->z, a->out, a->residual, a->pre_norm_weight, a->pre_norm_bias, a->z_norm_weight,
                  a->z_norm_bias, a->z_weight, a->q_weight, a->q_bias, a->k_weight, a->v_weight, a->g_weight,
                  a->o_weight, a->pair_bias}))
    return fail(FJX_ERR_INVALID, "fjx_single_attention_fwd: tensors must be 16-byte aligned");
  const size_t need = single_ws(a->batch, a->n, a->c_s, a->heads, a->dtype).total;
  if (!a->workspace || a->workspace_bytes < need)
    return fail(FJX_ERR_WORKSPACE, "fjx_single_attention_fwd: workspace of %zu bytes needed, %zu given", need,
                a->workspace_bytes);
  const bool bf = a->dtype == FJX_DTYPE_BF16, zbf = a->z_dtype == FJX_DTYPE_BF16;
  if (bf) return zbf ? single_run<bf16, bf16>(a, st) : single_run<bf16, float>(a, st);
  return zbf ? single_run<float, bf16>(a, st) : single_run<float, float>(a, st);
}

int fjx_prof_enable(int on) {
  std::lock_guard<std::mutex> lk(prof().mu);
  prof().on = on != 0;
  return FJX_OK;
}

int fjx_prof_reset(void) {
  Prof& p = prof();
  std::lock_guard<std::mutex> lk(p.mu);
  for (auto& r : p.pending) {
    (void)hipEventSynchronize(r.b);
    p.pool.push_back(r.a);
    p.pool.push_back(r.b);
  }
  p.pending.clear();
  for (int i = 0; i < K_COUNT; ++i) {
    p.total_ms[i] = 0.0;
    p.count[i] = 0;
  }
  return FJX_OK;
}

int fjx_prof_collect(void) {
  Prof& p = prof();
  std::lock_guard<std::mutex> lk(p.mu);
  for (auto& r : p.pending) {
    if (hipEventSynchronize(r.b) != hipSuccess) return fail(FJX_ERR_HIP, "fjx_prof_collect: event sync failed");
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, r.a, r.b) != hipSuccess)
      return fail(FJX_ERR_HIP, "fjx_prof_collect: elapsed time failed");
    p.total_ms[r.id] += ms;
    p.count[r.id] += 1;
    p.pool.push_back(r.a);
    p.pool.push_back(r.b);
  }
  p.pending.clear();
  return FJX_OK;
}

int fjx_probe_issue_mix(int mix, int waves_per_simd, int iters, float* ms, hipStream_t st) {
  g_err.clear();
  if (mix < 0 || mix > 6 || waves_per_simd < 1 || waves_per_simd > 4 || iters < 1 || !ms)
    return fail(FJX_ERR_INVALID, "fjx_probe_issue_mix: mix 0..6, 1..4 waves per SIMD, iters >= 1, ms non-NULL");
  if (fjx::probe_issue_mix(mix, waves_per_simd, iters, ms, st) != 0)
    return fail(FJX_ERR_HIP, "fjx_probe_issue_mix: a HIP call failed");
  return FJX_OK;
}

int fjx_probe_hbm_stream(int mode, int wgs_per_cu, int64_t bytes, float* ms, hipStream_t st) {
  g_err.clear();
  if (mode < 0 || mode > 3 || wgs_per_cu < 1 || wgs_per_cu > 32 || bytes < 4096 || bytes % 4096 != 0 ||
      bytes > ((int64_t)1 << 34) || !ms)
    return fail(FJX_ERR_INVALID,
                "fjx_probe_hbm_stream: mode 0..3, 1..32 workgroups per CU, bytes a multiple of 4096 in [4 KiB, "
                "16 GiB], ms non-NULL");
  if (fjx::probe_hbm_stream(mode, wgs_per_cu, bytes, ms, st) != 0)
    return fail(FJX_ERR_HIP, "fjx_probe_hbm_stream: a HIP call failed");
  return FJX_OK;
}

int fjx_prof_num_kernels(void) { return K_COUNT; }

const char* fjx_prof_kernel_name(int id) { return (id >= 0 && id < K_COUNT) ? kKernelNames[id] : ""; }

int fjx_prof_read(int id, double* total_ms, int64_t* launches) {
  if (id < 0 || id >= K_COUNT) return fail(FJX_ERR_INVALID, "fjx_prof_read: bad kernel id %d", id);
  Prof& p = prof();
  std::lock_guard<std::mutex> lk(p.mu);
  if (total_ms) *total_ms = p.total_ms[id];
  if (launches) *launches = p.count[id];
  return FJX_OK;
}

}  // extern "C"

namespace fjx {
// fjx_trimul_fwd on a caller-supplied device scratch (fjx_noalloc.hip): the
// same checks and kernels, the workspace fields of `a` ignored, no timing
// events, nothing allocated
__attribute__((visibility("hidden"))) int trimul_fwd_on_scratch(const fjx_trimul_args* a, hipStream_t st,
                                                               void* scratch, size_t scratch_bytes, const char* fn) {
  g_err.clear();
  if (int rc = trimul_check(a, fn)) return rc;
  const size_t need = fjx_trimul_workspace_size(a->batch, a->n, a->c_z, a->c_h, a->dtype);
  if (need > scratch_bytes)
    return fail(FJX_ERR_WORKSPACE,
                "%s: this shape needs %zu bytes of scratch, the library's static scratch holds %zu "
                "(use fjx_trimul_fwd with a workspace)",
                fn, need, scratch_bytes);
  fjx_trimul_args b = *a;
  b.workspace = scratch;
  b.workspace_bytes = scratch_bytes;
  g_no_events = true;
  const int rc = trimul_dispatch(&b, st);
  g_no_events = false;
  return rc;
}

__attribute__((visibility("hidden"))) int set_error(int code, const char* msg) { return fail(code, "%s", msg); }
}  // namespace fjx
