// C ABI entry points of libalgebraic_hip.so (declared in include/algebraic_hip.h).
//
// Host-side validation mirrors the reference's ValueErrors where the reference raises
// (src/algebraic/kernels/flash.py:740-743, 796-797; fused_head.py:163-164, 269-272);
// everything else is shape/pointer checking before any launch, so a bad call returns an
// error instead of launching a kernel whose grid does not match its operands.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <initializer_list>
#include <mutex>
#include <string>

#include "algebraic_hip.h"
#include "launchers.h"

// Scratch of alg_attn_bwd_noalloc: the sink-gradient and guard partials and, for f32 inputs,
// the dQ accumulator (the layout of attn_ws below), for callers that cannot allocate. Each GPU
// the library runs on holds its own copy of this array until the process ends. Host code never
// uses its name as an address: the device address comes from hipGetSymbolAddress, once per
// device (noalloc_scratch below).
constexpr size_t NOALLOC_SCRATCH_BYTES = ALG_ATTN_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_status(hipError_t e, const char* where) {
  if (e == hipSuccess) return ALG_OK;
  return fail(ALG_ERR_HIP, "%s: %s", where, hipGetErrorString(e));
}

int log2_pow2(int n) {
  if (n < 1 || (n & (n - 1))) return -1;
  int k = 0;
  while ((1 << k) < n) ++k;
  return k;
}

double root_pow2(double v, int n) {
  while (n > 1) { v = std::sqrt(v); n /= 2; }
  return v;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

int check_attn_shape(int dtype, int B, int H, int T, int D) {
  if (dtype != ALG_DTYPE_BF16 && dtype != ALG_DTYPE_F32) return fail(ALG_ERR_INVALID, "dtype must be bf16 or f32");
  if (B <= 0 || H <= 0 || T <= 0) return fail(ALG_ERR_INVALID, "B, H, T must be positive (got %d, %d, %d)", B, H, T);
  if (D != 64 && D != 128) return fail(ALG_ERR_UNSUPPORTED, "head_dim %d: gfx950 kernels are built for D in {64, 128}", D);
  if ((double)B * H * T * D > 4.0e9) return fail(ALG_ERR_INVALID, "tensor too large");
  // One (b, h) slice of q/k/v/dO is addressed with 32-bit byte offsets (buffer descriptors).
  if ((double)(T + 64) * D * 4 >= 2147483648.0)
    return fail(ALG_ERR_UNSUPPORTED, "T = %d: at most %d positions per head", T, (int)(2147483648.0 / (D * 4)) - 64);
  return ALG_OK;
}

// Layout check: with (B, T, H, D) storage a head's rows are H*D elements apart, and one head's
// rows are addressed with 32-bit byte offsets.
int check_layout(int layout, int H, int T, int D) {
  if (layout != ALG_LAYOUT_BHTD && layout != ALG_LAYOUT_BTHD) return fail(ALG_ERR_INVALID, "unknown layout %d", layout);
  const double ld = layout == ALG_LAYOUT_BTHD ? (double)H * D : (double)D;
  if ((T + 64.0) * ld * 4 >= 2147483648.0)
    return fail(ALG_ERR_UNSUPPORTED, "T = %d with H = %d: one head's rows exceed 32-bit offsets in this layout", T, H);
  return ALG_OK;
}

// The reference takes any power of two (flash.py:740-741, fused_head.py:269-270); the kernels
// form powers by repeated squaring with the exponent's log2 as a loop count, so the C ABI
// takes exponents up to 2^20 (beyond that every weight but the largest underflows in f32).
constexpr int MAX_LOG2N = 20;

int check_n(int n) {
  const int k = log2_pow2(n);
  if (k < 1 || k > MAX_LOG2N)
    return fail(ALG_ERR_INVALID, "asinh kernel needs n to be a power of two in [2, 2^%d] (got %d)", MAX_LOG2N, n);
  return ALG_OK;
}

// Workspace layout for attention: [sink partials f32 B*H*nblk][guard partials f32 3*max(1024,
// B*H*ceil(T/128)): the prep kernel's (at most 1024 workgroups) or the guarded bf16 forward's
// (one per 128-query workgroup)], and for f32 inputs then [dq accumulator f32 B*H*T*D] (the
// bf16 dQ kernel needs none).
size_t attn_fwd_workgroups(int B, int H, int T) { return (size_t)B * H * ((T + alg::FWD_BQ - 1) / alg::FWD_BQ); }
size_t attn_fwd_f32_workgroups(int B, int H, int T) {
  const int bq = alg::attn_fwd_f32_query_block(B, H, T);
  return (size_t)B * H * ((T + bq - 1) / bq);
}
struct AttnWs {
  size_t sink_part, prep_part, dq_acc, total;
};
AttnWs attn_ws(int dtype, int B, int H, int T, int D) {
  AttnWs w;
  w.sink_part = 0;
  w.prep_part = align256((size_t)B * H * alg::attn_bwd_sink_blocks(T) * sizeof(float));
  // Guard maxima: one triple per forward workgroup (alg_attn_fwd_guarded) or prep workgroup.
  size_t nwg = std::max<size_t>(1024, attn_fwd_workgroups(B, H, T));
  if (dtype == ALG_DTYPE_F32 && D == 64) nwg = std::max(nwg, attn_fwd_f32_workgroups(B, H, T));
  w.dq_acc = w.prep_part + align256(3 * nwg * sizeof(float));
  w.total = w.dq_acc + (dtype == ALG_DTYPE_F32 ? align256((size_t)B * H * T * D * sizeof(float)) : 0);
  return w;
}

// Head buffers. Workspace: [partials f32 nvt*N][obj parts] (+ bwd: dZ bf16 Npad*Vp for the
// recompute schedule, or s*h/l bf16 N*d for the residual schedule; then, when the dh product
// is split over the vocabulary, its f32 partials split*N*d; then, when the last round of dE
// tiles is split over the tokens, their f32 tiles (head_de_plan)). Residual (optional,
// forward -> backward): [U bf16 Npad*Vp][l f32 N]. dZ and U are token-major with rows of
// Vp = V rounded up to 8 (16-byte aligned rows).
struct HeadWs {
  size_t partial, obj_part, bwd, dh_part, de_part, total;
  size_t res_ut, res_l, res_total;
  int Npad, Vp, dh_split;
  alg::HeadDePlan de;
};
HeadWs head_ws(int N, int d, int V, int pass, bool residual) {
  HeadWs w;
  w.Npad = alg::head_token_pad(N);
  w.Vp = alg::head_vocab_pitch(V);
  w.partial = 0;
  w.obj_part = align256((size_t)alg::head_vocab_tiles(V) * N * sizeof(float));
  w.bwd = w.obj_part + align256((size_t)alg::head_stat_blocks(N) * sizeof(float));
  const size_t bwd_bytes = residual ? (size_t)N * d * 2 : (size_t)w.Npad * w.Vp * 2;
  w.dh_split = alg::head_dh_split(N, d, V);
  w.dh_part = w.bwd + align256(bwd_bytes);
  const size_t part_bytes = w.dh_split > 1 ? (size_t)w.dh_split * N * d * sizeof(float) : 0;
  w.de = alg::head_de_plan(N, d, V);
  w.de_part = w.dh_part + align256(part_bytes);
  const size_t de_bytes =
      w.de.split > 1 ? (size_t)(w.de.tiles - w.de.full) * w.de.split * alg::HT_M * alg::HT_N * sizeof(float) : 0;
  w.total = pass == 0 ? w.bwd : w.de_part + align256(de_bytes);
  w.res_ut = 0;
  w.res_l = align256((size_t)w.Npad * w.Vp * 2);
  w.res_total = w.res_l + align256((size_t)N * sizeof(float));
  return w;
}

// f32 hidden states (head_f32.hip, the reference's recompute schedule in f32): [partials f32
// nvt*N over 128-entry vocabulary tiles][obj parts] (+ bwd: dZ f32 N*Vp, then the f32 partials
// split*N*d of a vocabulary-split dh product). No residual.
HeadWs head_ws_f32(int N, int d, int V, int pass) {
  HeadWs w;
  w.Npad = N;
  w.Vp = alg::head_vocab_pitch(V);
  w.partial = 0;
  w.obj_part = align256((size_t)alg::head_f32_vocab_tiles(V) * N * sizeof(float));
  w.bwd = w.obj_part + align256((size_t)alg::head_stat_blocks(N) * sizeof(float));
  w.dh_split = alg::head_f32_dh_split(N, d, V);
  w.dh_part = w.bwd + align256((size_t)N * w.Vp * sizeof(float));
  const size_t part_bytes = w.dh_split > 1 ? (size_t)w.dh_split * N * d * sizeof(float) : 0;
  w.de = alg::HeadDePlan{0, 0, 1, 0};
  w.de_part = 0;
  w.total = pass == 0 ? w.bwd : w.dh_part + align256(part_bytes);
  w.res_ut = w.res_l = w.res_total = 0;
  return w;
}

// Eval workspace: [row-sum partials f32 nvt*N][tile maxima f32 nvt*N][their indices i32 nvt*N].
struct HeadEvalWs {
  size_t partial, pmax, pidx, total;
};
HeadEvalWs head_eval_ws(int N, int V, bool f32) {
  const size_t cells = (size_t)(f32 ? alg::head_f32_vocab_tiles(V) : alg::head_vocab_tiles(V)) * N;
  HeadEvalWs w;
  w.partial = 0;
  w.pmax = align256(cells * sizeof(float));
  w.pidx = w.pmax + align256(cells * sizeof(float));
  w.total = w.pidx + align256(cells * sizeof(int));
  return w;
}

int check_head(int N, int d, int V, int n, float c) {
  if (N <= 0 || d <= 0 || V <= 0) return fail(ALG_ERR_INVALID, "N, d, V must be positive (got %d, %d, %d)", N, d, V);
  if (d % 8) return fail(ALG_ERR_UNSUPPORTED, "d_model %d: head rows must be 16-byte aligned (d %% 8 == 0)", d);
  if (alg::head_token_pad(N) > (1 << 23))  // residual rows are addressed with 32-bit buffer offsets
    return fail(ALG_ERR_UNSUPPORTED, "N = %d tokens: at most %d per call", N, 1 << 23);
  if ((double)N * d > 2.0e9 || (double)V * d > 2.0e9 ||
      (double)alg::head_vocab_pitch(V) * alg::head_token_pad(N) > 4.0e9)
    return fail(ALG_ERR_INVALID, "head too large");
  const int k = log2_pow2(n);
  if (k < 0 || k > MAX_LOG2N) return fail(ALG_ERR_INVALID, "n must be a power of two in [1, 2^%d] (got %d)", MAX_LOG2N, n);
  if (!(c > 0.0f) || !std::isfinite(c)) return fail(ALG_ERR_INVALID, "c must be positive and finite");
  return ALG_OK;
}

// The training head's statistic is l^(-1/n), formed as the reference's _inv_root does
// (fused_head.py:59-65: rsqrt, then y * rsqrt(y) while k = n/2 > 1). For n = 1 that loop gives
// rsqrt(l) rather than 1/l, and the reference's fused head then computes p = rho * rsqrt(l)
// and its gradient from it; the kernels here form the same quantities (stat = inv_root(l, n),
// p = (rho stat)^n), so n = 1 returns what the reference returns. The residual schedule
// alone cannot take it: its U' = (l / s) dz rests on stat^n = 1 / l.
int check_train_head_n(int n, const void* residual) {
  if (n == 1 && residual)
    return fail(ALG_ERR_UNSUPPORTED,
                "n = 1: the residual schedule needs stat^n = 1/l, which the reference's l^(-1/n) "
                "(rsqrt(l) at n = 1) does not give; pass no residual (recompute schedule)");
  return ALG_OK;
}

// Guard bounds (flash.py:747-748, 840-849), evaluated in double then rounded like the
// reference's weakly typed Python-float constants.
alg::GuardParams guard_params(int H, int T, int n, float c, const float* sink_logit, int sink_count, float* sink_scaled,
                              int* guard_flag, int range_guard) {
  const double t = root_pow2(1e37 / (T + 1.0), n);
  const double clamp = 0.5 * (t - 1.0 / t);
  const double bound = std::fmin(16.0, clamp / 2.0);
  const int has_sink = sink_logit ? 1 : 0;
  alg::GuardParams g;
  g.part = nullptr; g.nblocks = 0;
  g.sink_logit = sink_logit; g.sink_count = sink_count;
  g.sink_out = sink_scaled; g.H = H; g.c = c;
  g.flag = guard_flag;
  g.q2k2_bound = (float)((bound / 1.01) * (bound / 1.01));
  g.sink_bound = (float)(bound / 1.01);
  g.v_bound = (float)std::fmin(1e8, 1e37 / ((T + has_sink) * std::pow(2.0 * bound + 1.0, n)));
  g.want_guard = range_guard && n <= 32 ? 1 : 0;
  return g;
}

// Prologue workspace: [guard maxima f32 3*nb][gain-gradient partials f32 2*D*nb], nb the
// prologue's workgroup count (the f32 count, the larger of the two dtypes).
struct PrologueWs {
  size_t guard_part, gain_part, total;
};
PrologueWs prologue_ws(int B, int H, int T, int D) {
  const size_t nb = (size_t)alg::attn_qk_prologue_blocks(B, H, T, D, false);
  PrologueWs w;
  w.guard_part = 0;
  w.gain_part = align256(3 * nb * sizeof(float));
  w.total = w.gain_part + align256(nb * 2 * D * sizeof(float));
  return w;
}

int check_prologue(int dtype, int layout, int B, int H, int T, int D, const float* cos_t, const float* sin_t,
                   float eps) {
  int rc = check_attn_shape(dtype, B, H, T, D);
  if (rc) return rc;
  if ((rc = check_layout(layout, H, T, D))) return rc;
  if ((cos_t == nullptr) != (sin_t == nullptr)) return fail(ALG_ERR_INVALID, "cos and sin are given together");
  if (!(eps > 0.0f) || !std::isfinite(eps)) return fail(ALG_ERR_INVALID, "eps must be positive and finite");
  return ALG_OK;
}

// Every matrix (and workspace) is read or written 16 bytes per lane: its base must sit on a
// 16-byte boundary (rows stay aligned because row lengths are multiples of 8 elements).
// Null pointers (optional arguments) pass.
bool aligned16(std::initializer_list<const void*> ptrs) {
  for (const void* q : ptrs)
    if (reinterpret_cast<uintptr_t>(q) & 15) return false;
  return true;
}

// Device address of `scratch` on the current device, looked up with that device current on the
// first call that runs there and kept per device.
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[MAX_DEVICES];

int noalloc_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, "alg_attn_bwd_noalloc: hipGetDevice");
  if (dev < 0 || dev >= MAX_DEVICES) return fail(ALG_ERR_UNSUPPORTED, "device %d: at most %d devices", dev, MAX_DEVICES);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_status(e, "alg_attn_bwd_noalloc: hipGetSymbolAddress");
    if (!ptr) return fail(ALG_ERR_HIP, "alg_attn_bwd_noalloc: no device address for the scratch array");
    g_scratch_dev[dev] = ptr;
  }
  *out = g_scratch_dev[dev];
  return ALG_OK;
}

}  // namespace

extern "C" {

const char* alg_last_error(void) { return g_err.c_str(); }
const char* alg_version(void) { return "algebraic_hip 0.2 gfx950 (ABI 2)"; }
int alg_abi_version(void) { return ALG_ABI_VERSION; }

size_t alg_attn_workspace_size(int dtype, int B, int H, int T, int D) {
  if (B <= 0 || H <= 0 || T <= 0 || D <= 0) return 0;
  if (dtype != ALG_DTYPE_BF16 && dtype != ALG_DTYPE_F32) return 0;
  return attn_ws(dtype, B, H, T, D).total;
}

int alg_attn_prepare(alg_stream_t stream, int dtype, int B, int H, int T, int D, const void* q, const void* k,
                     const void* v, const float* sink_logit, int sink_count, float c, int n, int range_guard,
                     void* q_s, float* sink_scaled, int* guard_flag, void* workspace, size_t workspace_bytes) {
  int rc = check_attn_shape(dtype, B, H, T, D);
  if (rc) return rc;
  if ((rc = check_n(n))) return rc;
  if (!(c > 0.0f) || !std::isfinite(c)) return fail(ALG_ERR_INVALID, "asinh scale c must be positive and finite");
  if (!q || !q_s || !guard_flag) return fail(ALG_ERR_INVALID, "q, q_s and guard_flag are required");
  if (!aligned16({q, k, v, q_s, workspace})) return fail(ALG_ERR_INVALID, "matrices must be 16-byte aligned");
  if (range_guard && (!k || !v)) return fail(ALG_ERR_INVALID, "range_guard needs k and v");
  if (sink_logit && sink_count != 1 && sink_count != H) return fail(ALG_ERR_INVALID, "sink_count must be 1 or H");
  if (sink_logit && !sink_scaled) return fail(ALG_ERR_INVALID, "sink_scaled output required with a sink");
  const AttnWs ws = attn_ws(dtype, B, H, T, D);
  if (!workspace || workspace_bytes < ws.total)
    return fail(ALG_ERR_INVALID, "workspace too small: need %zu bytes", ws.total);
  alg::PrepParams pp;
  pp.q = q; pp.k = k; pp.v = v; pp.q_s = q_s;
  pp.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + ws.prep_part);
  pp.rows = (size_t)B * H * T;
  pp.D = D;
  pp.alpha = (float)(1.0 / (std::sqrt((double)D) * (double)c));
  pp.want_guard = range_guard ? 1 : 0;
  const alg::GuardParams g = guard_params(H, T, n, c, sink_logit, sink_count, sink_scaled, guard_flag, range_guard);
  return hip_status(alg::launch_attn_prep(pp, dtype == ALG_DTYPE_BF16, g, (hipStream_t)stream), "alg_attn_prepare");
}

size_t alg_attn_prologue_workspace_size(int B, int H, int T, int D) {
  if (B <= 0 || H <= 0 || T <= 0 || D <= 0) return 0;
  return prologue_ws(B, H, T, D).total;
}

int alg_cayley_tables(alg_stream_t stream, const float* w, int half, int seq_len, float* cos_out, float* sin_out) {
  if (!w || !cos_out || !sin_out) return fail(ALG_ERR_INVALID, "w, cos and sin are required");
  if (half <= 0 || seq_len <= 0) return fail(ALG_ERR_INVALID, "half and seq_len must be positive");
  if ((double)half * seq_len > 2.0e9) return fail(ALG_ERR_INVALID, "table too large");
  return hip_status(alg::launch_cayley_tables(w, half, seq_len, cos_out, sin_out, (hipStream_t)stream),
                    "alg_cayley_tables");
}

int alg_attn_qk_prologue(alg_stream_t stream, int dtype, int layout, int B, int H, int T, int D, const void* q,
                         const void* k, const void* v, const float* q_gain, const float* k_gain, const float* cos_t,
                         const float* sin_t, float eps, const float* sink_logit, int sink_count, float c, int n,
                         int range_guard, void* q_s, void* k_r, float* tau_q, float* tau_k, float* sink_scaled,
                         int* guard_flag, void* workspace, size_t workspace_bytes) {
  int rc = check_prologue(dtype, layout, B, H, T, D, cos_t, sin_t, eps);
  if (rc) return rc;
  if ((rc = check_n(n))) return rc;
  if (!(c > 0.0f) || !std::isfinite(c)) return fail(ALG_ERR_INVALID, "asinh scale c must be positive and finite");
  if (!q || !k || !q_s || !k_r || !tau_q || !tau_k || !guard_flag)
    return fail(ALG_ERR_INVALID, "q, k, q_s, k_r, tau_q, tau_k and guard_flag are required");
  if (!aligned16({q, k, v, q_s, k_r, workspace})) return fail(ALG_ERR_INVALID, "matrices must be 16-byte aligned");
  if (range_guard && !v) return fail(ALG_ERR_INVALID, "range_guard needs v");
  if (sink_logit && sink_count != 1 && sink_count != H) return fail(ALG_ERR_INVALID, "sink_count must be 1 or H");
  if (sink_logit && !sink_scaled) return fail(ALG_ERR_INVALID, "sink_scaled output required with a sink");
  const PrologueWs ws = prologue_ws(B, H, T, D);
  if (!workspace || workspace_bytes < ws.total)
    return fail(ALG_ERR_INVALID, "workspace too small: need %zu bytes", ws.total);
  alg::QkPrologueParams p;
  p.q = q; p.k = k; p.v = v;
  p.q_gain = q_gain; p.k_gain = k_gain; p.cos = cos_t; p.sin = sin_t;
  p.q_s = q_s; p.k_r = k_r; p.tau_q = tau_q; p.tau_k = tau_k;
  p.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + ws.guard_part);
  p.B = B; p.H = H; p.T = T; p.D = D; p.layout = layout;
  p.eps = eps;
  p.alpha = (float)(1.0 / (std::sqrt((double)D) * (double)c));
  p.want_guard = range_guard ? 1 : 0;
  const alg::GuardParams g = guard_params(H, T, n, c, sink_logit, sink_count, sink_scaled, guard_flag, range_guard);
  return hip_status(alg::launch_attn_qk_prologue(p, dtype == ALG_DTYPE_BF16, g, (hipStream_t)stream),
                    "alg_attn_qk_prologue");
}

int alg_attn_qk_prologue_bwd(alg_stream_t stream, int dtype, int layout, int B, int H, int T, int D, const void* q,
                             const void* k, const float* q_gain, const float* k_gain, const float* cos_t,
                             const float* sin_t, const float* tau_q, const float* tau_k, const void* dq_r,
                             const void* dk_r, void* dq, void* dk, float* dq_gain, float* dk_gain, void* workspace,
                             size_t workspace_bytes) {
  int rc = check_prologue(dtype, layout, B, H, T, D, cos_t, sin_t, 1.0f);
  if (rc) return rc;
  if (!q || !k || !tau_q || !tau_k || !dq_r || !dk_r || !dq || !dk)
    return fail(ALG_ERR_INVALID, "q, k, tau_q, tau_k, dq_r, dk_r, dq and dk are required");
  if (!aligned16({q, k, dq_r, dk_r, dq, dk, workspace}))
    return fail(ALG_ERR_INVALID, "matrices must be 16-byte aligned");
  if ((dq_gain && !q_gain) || (dk_gain && !k_gain))
    return fail(ALG_ERR_INVALID, "a gain gradient needs the gain it differentiates");
  const PrologueWs ws = prologue_ws(B, H, T, D);
  if (!workspace || workspace_bytes < ws.total)
    return fail(ALG_ERR_INVALID, "workspace too small: need %zu bytes", ws.total);
  alg::QkPrologueBwdParams p;
  p.q = q; p.k = k; p.q_gain = q_gain; p.k_gain = k_gain; p.cos = cos_t; p.sin = sin_t;
  p.tau_q = tau_q; p.tau_k = tau_k; p.dq_r = dq_r; p.dk_r = dk_r; p.dq = dq; p.dk = dk;
  p.gpart = reinterpret_cast<float*>(static_cast<char*>(workspace) + ws.gain_part);
  p.B = B; p.H = H; p.T = T; p.D = D; p.layout = layout;
  return hip_status(alg::launch_attn_qk_prologue_bwd(p, dtype == ALG_DTYPE_BF16, dq_gain, dk_gain, (hipStream_t)stream),
                    "alg_attn_qk_prologue_bwd");
}

int alg_attn_fwd(alg_stream_t stream, int dtype, int layout, int B, int H, int T, int D, const void* q_s,
                 const void* k, const void* v, const float* sink_scaled, int n, int variant, const int* guard_flag,
                 float clamp, int fast_rho, int inv_stat, void* o, float* o_precise, float* stat) {
  int rc = check_attn_shape(dtype, B, H, T, D);
  if (rc) return rc;
  if ((rc = check_layout(layout, H, T, D))) return rc;
  if ((rc = check_n(n))) return rc;
  if (!q_s || !k || !v || !o || !stat) return fail(ALG_ERR_INVALID, "q_s, k, v, o and stat are required");
  if (!aligned16({q_s, k, v, o, o_precise})) return fail(ALG_ERR_INVALID, "matrices must be 16-byte aligned");
  if (variant < ALG_ATTN_INRANGE || variant > ALG_ATTN_GUARDED) return fail(ALG_ERR_INVALID, "unknown variant %d", variant);
  if (variant == ALG_ATTN_GUARDED && !guard_flag) return fail(ALG_ERR_INVALID, "GUARDED needs guard_flag");
  alg::AttnFwdParams p;
  p.q = q_s; p.k = k; p.v = v; p.sink = sink_scaled;
  p.flag = variant == ALG_ATTN_GUARDED ? guard_flag : nullptr;
  p.o = o; p.o_precise = o_precise; p.stat = stat;
  p.B = B; p.H = H; p.T = T;
  p.log2n = log2_pow2(n);
  p.clamp = clamp; p.fast_rho = fast_rho; p.inv_stat = inv_stat;
  p.layout = layout;
  const bool bf = dtype == ALG_DTYPE_BF16;
  hipStream_t st = (hipStream_t)stream;
  if (variant == ALG_ATTN_GUARDED) {
    alg::AttnFwdParams ps = p;
    ps.fast_rho = 0;  // the guard's fallback uses stable rho (flash.py:851)
    rc = hip_status(alg::launch_attn_fwd(p, D, bf, alg::MODE_INRANGE, st), "alg_attn_fwd");
    if (rc) return rc;
    return hip_status(alg::launch_attn_fwd(ps, D, bf, alg::MODE_SHIFTED, st), "alg_attn_fwd");
  }
  return hip_status(alg::launch_attn_fwd(p, D, bf, variant, st), "alg_attn_fwd");
}

int alg_attn_fwd_guarded(alg_stream_t stream, int dtype, int layout, int B, int H, int T, int D, const void* q,
                         const void* k, const void* v, const float* sink_logit, int sink_count, float c, int n,
                         void* q_s, float* sink_scaled, int* guard_flag, void* o, float* o_precise, float* stat,
                         void* workspace, size_t workspace_bytes) {
  int rc = check_attn_shape(dtype, B, H, T, D);
  if (rc) return rc;
  if ((rc = check_layout(layout, H, T, D))) return rc;
  if ((rc = check_n(n))) return rc;
  if (n > 32) return fail(ALG_ERR_INVALID, "the range guard applies for n <= 32 (got %d)", n);
  if (!(c > 0.0f) || !std::isfinite(c)) return fail(ALG_ERR_INVALID, "asinh scale c must be positive and finite");
  if (!q || !k || !v || !q_s || !guard_flag || !o || !stat)
    return fail(ALG_ERR_INVALID, "q, k, v, q_s, guard_flag, o and stat are required");
  if (!aligned16({q, k, v, q_s, o, o_precise, workspace})) return fail(ALG_ERR_INVALID, "matrices must be 16-byte aligned");
  if (sink_logit && sink_count != 1 && sink_count != H) return fail(ALG_ERR_INVALID, "sink_count must be 1 or H");
  if (sink_logit && !sink_scaled) return fail(ALG_ERR_INVALID, "sink_scaled output required with a sink");
  const AttnWs ws = attn_ws(dtype, B, H, T, D);
  if (!workspace || workspace_bytes < ws.total)
    return fail(ALG_ERR_INVALID, "workspace too small: need %zu bytes", ws.total);
  // The guard's clamp (flash.py:747-748); the in-range and shifted kernels do not read it.
  const double t = root_pow2(1e37 / (T + 1.0), n);
  const float clamp = (float)(0.5 * (t - 1.0 / t));
  const bool bf = dtype == ALG_DTYPE_BF16;
  if (!bf && D != 64) {  // the f32 D = 128 forward has no FROM_Q form: prepare, then forward
    rc = alg_attn_prepare(stream, dtype, B, H, T, D, q, k, v, sink_logit, sink_count, c, n, 1, q_s, sink_scaled,
                          guard_flag, workspace, workspace_bytes);
    if (rc) return rc;
    // sink/c exists only with a sink: a sink_scaled buffer passed without one is not read.
    return alg_attn_fwd(stream, dtype, layout, B, H, T, D, q_s, k, v, sink_logit ? sink_scaled : nullptr, n,
                        ALG_ATTN_GUARDED, guard_flag,
                        clamp, 1, 1, o, o_precise, stat);
  }
  hipStream_t st = (hipStream_t)stream;
  float* part = reinterpret_cast<float*>(static_cast<char*>(workspace) + ws.prep_part);
  alg::AttnFwdParams p;
  p.q = q; p.k = k; p.v = v; p.sink = nullptr; p.flag = nullptr;
  p.o = o; p.o_precise = nullptr; p.stat = stat;
  p.B = B; p.H = H; p.T = T;
  p.log2n = log2_pow2(n);
  p.clamp = clamp; p.fast_rho = 1; p.inv_stat = 1;
  p.layout = layout;
  p.q_s_out = q_s;
  p.alpha = (float)(1.0 / (std::sqrt((double)D) * (double)c));  // as alg_attn_prepare
  p.guard_part = part;
  p.sink_logit = sink_logit; p.sink_count = sink_count; p.sink_c = c;
  rc = hip_status(alg::launch_attn_fwd(p, D, bf, alg::MODE_INRANGE, st), "alg_attn_fwd_guarded");
  if (rc) return rc;
  alg::GuardParams g = guard_params(H, T, n, c, sink_logit, sink_count, sink_scaled, guard_flag, 1);
  g.part = part;
  g.nblocks = (int)(bf ? attn_fwd_workgroups(B, H, T) : attn_fwd_f32_workgroups(B, H, T));
  rc = hip_status(alg::launch_attn_guard(g, st), "alg_attn_fwd_guarded");
  if (rc) return rc;
  alg::AttnFwdParams ps;
  ps.q = q_s; ps.k = k; ps.v = v; ps.flag = guard_flag;
  ps.sink = sink_logit ? sink_scaled : nullptr;  // written by the guard kernel only with a sink
  ps.o = o; ps.o_precise = o_precise; ps.stat = stat;
  ps.B = B; ps.H = H; ps.T = T;
  ps.log2n = p.log2n;
  ps.clamp = clamp; ps.fast_rho = 0; ps.inv_stat = 1;  // the fallback uses stable rho (flash.py:851)
  ps.layout = layout;
  return hip_status(alg::launch_attn_fwd(ps, D, bf, alg::MODE_SHIFTED, st), "alg_attn_fwd_guarded");
}

int alg_attn_bwd(alg_stream_t stream, int dtype, int layout, int B, int H, int T, int D, const void* q_s,
                 const void* k, const void* v, const float* sink_scaled, const void* o, const float* stat,
                 const void* dO, int n, int variant, const int* guard_flag, float clamp, int fast_rho, int inv_stat,
                 float dq_scale, void* dq, void* dk, void* dv, float* di, float* dsink_scaled, void* workspace,
                 size_t workspace_bytes) {
  int rc = check_attn_shape(dtype, B, H, T, D);
  if (rc) return rc;
  if ((rc = check_layout(layout, H, T, D))) return rc;
  if ((rc = check_n(n))) return rc;
  if (!q_s || !k || !v || !o || !stat || !dO || !dq || !dk || !dv || !di)
    return fail(ALG_ERR_INVALID, "q_s, k, v, o, stat, dO, dq, dk, dv and di are required");
  if (!aligned16({q_s, k, v, o, dO, dq, dk, dv, workspace}))
    return fail(ALG_ERR_INVALID, "matrices must be 16-byte aligned");
  if (variant < ALG_ATTN_INRANGE || variant > ALG_ATTN_GUARDED) return fail(ALG_ERR_INVALID, "unknown variant %d", variant);
  if (variant == ALG_ATTN_GUARDED && !guard_flag) return fail(ALG_ERR_INVALID, "GUARDED needs guard_flag");
  const AttnWs ws = attn_ws(dtype, B, H, T, D);
  if (!workspace || workspace_bytes < ws.total)
    return fail(ALG_ERR_INVALID, "workspace too small: need %zu bytes", ws.total);
  alg::AttnBwdParams p;
  p.q = q_s; p.k = k; p.v = v; p.o = o; p.dO = dO; p.stat = stat;
  p.sink = sink_scaled;
  p.flag = variant == ALG_ATTN_GUARDED ? guard_flag : nullptr;
  p.di = di;
  p.dq_acc = dtype == ALG_DTYPE_F32 ? reinterpret_cast<float*>(static_cast<char*>(workspace) + ws.dq_acc) : nullptr;
  p.sink_part = reinterpret_cast<float*>(static_cast<char*>(workspace) + ws.sink_part);
  p.dq = dq; p.dk = dk; p.dv = dv; p.dbeta = dsink_scaled;
  p.B = B; p.H = H; p.T = T;
  p.log2n = log2_pow2(n);
  p.clamp = clamp; p.fast_rho = fast_rho; p.inv_stat = inv_stat;
  p.mode = variant == ALG_ATTN_GUARDED ? alg::MODE_INRANGE : variant;
  p.dq_scale = dq_scale;
  p.layout = layout;
  const bool bf = dtype == ALG_DTYPE_BF16;
  hipStream_t st = (hipStream_t)stream;
  if (variant == ALG_ATTN_GUARDED) {
    // Both branches are launched; each exits unless the device flag selects it. The
    // fallback uses stable rho (flash.py:851); the in-range kernels do not read fast_rho.
    const int modes[2] = {alg::MODE_INRANGE, alg::MODE_SHIFTED};
    p.fast_rho = 0;
    return hip_status(alg::launch_attn_bwd(p, D, bf, modes, 2, st), "alg_attn_bwd");
  }
  const int modes[1] = {variant};
  return hip_status(alg::launch_attn_bwd(p, D, bf, modes, 1, st), "alg_attn_bwd");
}

int alg_attn_bwd_noalloc(alg_stream_t stream, int dtype, int layout, int B, int H, int T, int D, const void* q_s,
                         const void* k, const void* v, const float* sink_scaled, const void* o, const float* stat,
                         const void* dO, int n, int variant, const int* guard_flag, float clamp, int fast_rho,
                         int inv_stat, float dq_scale, void* dq, void* dk, void* dv, float* di, float* dsink_scaled) {
  int rc = check_attn_shape(dtype, B, H, T, D);
  if (rc) return rc;
  const size_t need = attn_ws(dtype, B, H, T, D).total;
  if (need > NOALLOC_SCRATCH_BYTES)
    return fail(ALG_ERR_UNSUPPORTED,
                "alg_attn_bwd_noalloc: this call needs %zu bytes of scratch, above the %zu bytes the library "
                "holds per GPU; use alg_attn_bwd with a workspace",
                need, NOALLOC_SCRATCH_BYTES);
  void* ptr = nullptr;
  if ((rc = noalloc_scratch(&ptr))) return rc;
  return alg_attn_bwd(stream, dtype, layout, B, H, T, D, q_s, k, v, sink_scaled, o, stat, dO, n, variant, guard_flag,
                      clamp, fast_rho, inv_stat, dq_scale, dq, dk, dv, di, dsink_scaled, ptr, NOALLOC_SCRATCH_BYTES);
}

size_t alg_head_workspace_size(int dtype, int N, int d, int V, int pass) {
  if (N <= 0 || d <= 0 || V <= 0) return 0;
  if (dtype != ALG_DTYPE_BF16 && dtype != ALG_DTYPE_F32) return 0;
  const bool f32 = dtype == ALG_DTYPE_F32;
  // pass 0: forward; 1: backward without a residual; 2: backward with a residual; 3: eval
  if (pass == 3) return head_eval_ws(N, V, f32).total;
  if (f32) return pass == 2 ? 0 : head_ws_f32(N, d, V, pass ? 1 : 0).total;  // no residual in f32
  return head_ws(N, d, V, pass ? 1 : 0, pass == 2).total;
}

// Streamed backward (alg_head_bwd_streamed): the vocabulary in chunks of `chunk` rows. The
// default chunk gives one chunk's dE product at least 256 tiles of 256 x 256 (one per CU).
// Workspace: [logit gradient of one chunk: bf16 Npad x pitch(chunk), or f32 N x pitch(chunk)]
// (+ bf16, several chunks: [dh accumulator f32 N*d]) (+ bf16: [f32 tiles of the token-split
// dE tail, sized for the larger of the two chunk plans]).
struct HeadStreamWs {
  size_t dz, acc, de_part, total;
  int chunk, nchunks;
  bool has_de_part;  // some chunk's dE tail is token-split
};
static int head_stream_chunk(int d, int V, int vocab_chunk) {
  int chunk = vocab_chunk;
  if (chunk == 0) {
    const int dtiles = (d + alg::HT_N - 1) / alg::HT_N;
    chunk = alg::HT_M * ((256 + dtiles - 1) / dtiles);
  }
  return std::min(chunk, V);
}
static HeadStreamWs head_stream_ws(int dtype, int N, int d, int V, int vocab_chunk) {
  HeadStreamWs w;
  w.chunk = head_stream_chunk(d, V, vocab_chunk);
  const int nchunks = (V + w.chunk - 1) / w.chunk;
  w.nchunks = nchunks;
  w.has_de_part = false;
  const size_t pitch = (size_t)alg::head_vocab_pitch(w.chunk);
  w.dz = 0;
  if (dtype == ALG_DTYPE_F32) {  // dh accumulates in place in the f32 output; no dE split
    w.acc = w.de_part = w.total = align256((size_t)N * pitch * sizeof(float));
    return w;
  }
  w.acc = align256((size_t)alg::head_token_pad(N) * pitch * 2);
  w.de_part = w.acc + (nchunks > 1 ? align256((size_t)N * d * sizeof(float)) : 0);
  size_t de_bytes = 0;
  for (int vc : {w.chunk, V - (nchunks - 1) * w.chunk}) {
    const alg::HeadDePlan pl = alg::head_de_plan(N, d, vc);
    if (pl.split > 1)
      de_bytes = std::max(de_bytes, (size_t)(pl.tiles - pl.full) * pl.split * alg::HT_M * alg::HT_N * sizeof(float));
  }
  w.has_de_part = de_bytes > 0;
  w.total = w.de_part + align256(de_bytes);
  return w;
}

size_t alg_head_streamed_workspace_size(int dtype, int N, int d, int V, int vocab_chunk) {
  if (N <= 0 || d <= 0 || V <= 0 || vocab_chunk < 0 || vocab_chunk % alg::HT_M) return 0;
  if (dtype != ALG_DTYPE_BF16 && dtype != ALG_DTYPE_F32) return 0;
  return head_stream_ws(dtype, N, d, V, vocab_chunk).total;
}

size_t alg_head_residual_size(int N, int d, int V) {
  if (N <= 0 || d <= 0 || V <= 0) return 0;
  return head_ws(N, d, V, 0, true).res_total;
}

// Head dtype check: bf16 (the tuned kernels, both schedules) or f32 (the reference's recompute
// schedule in f32; no residual).
static int check_head_dtype(int dtype, const void* residual) {
  if (dtype != ALG_DTYPE_BF16 && dtype != ALG_DTYPE_F32) return fail(ALG_ERR_INVALID, "dtype must be bf16 or f32");
  if (dtype == ALG_DTYPE_F32 && residual)
    return fail(ALG_ERR_UNSUPPORTED, "the residual schedule is built for bf16 hidden states only; pass NULL");
  return ALG_OK;
}

static alg::HeadParams head_params(int dtype, int N, int d, int V, const void* h, const void* E,
                                   const int32_t* targets, int n, float c, void* workspace, const HeadWs& ws) {
  alg::HeadParams p;
  std::memset(&p, 0, sizeof p);
  if (dtype == ALG_DTYPE_F32) {
    p.h32 = static_cast<const float*>(h);
    p.E32 = static_cast<const float*>(E);
  } else {
    p.h = static_cast<const bf16*>(h);
    p.E = static_cast<const bf16*>(E);
  }
  p.targets = targets;
  p.N = N; p.d = d; p.V = V; p.Npad = ws.Npad; p.Vp = ws.Vp;
  p.log2n = log2_pow2(n);
  p.c = c;
  p.inv_c = (float)(1.0 / (double)c);
  p.clamp = (float)(0.25 * root_pow2(1e38 / (double)V, n));  // fused_head.py:273
  char* w = static_cast<char*>(workspace);
  p.partial = reinterpret_cast<float*>(w + ws.partial);
  p.obj_part = reinterpret_cast<float*>(w + ws.obj_part);
  return p;
}

int alg_head_fwd(alg_stream_t stream, int dtype, int N, int d, int V, const void* h, const void* E,
                 const int32_t* targets, int n, float c, float* stat, float* zt, float* pt, float* obj,
                 void* residual, void* workspace, size_t workspace_bytes) {
  int rc = check_head(N, d, V, n, c);
  if (!rc) rc = check_train_head_n(n, residual);
  if (!rc) rc = check_head_dtype(dtype, residual);
  if (rc) return rc;
  const bool f32 = dtype == ALG_DTYPE_F32;
  if (!h || !E || !targets || !stat || !zt || !pt || !obj) return fail(ALG_ERR_INVALID, "null argument");
  if (!aligned16({h, E, residual, workspace})) return fail(ALG_ERR_INVALID, "matrices must be 16-byte aligned");
  const HeadWs ws = f32 ? head_ws_f32(N, d, V, 0) : head_ws(N, d, V, 0, residual != nullptr);
  if (!workspace || workspace_bytes < ws.total)
    return fail(ALG_ERR_INVALID, "workspace too small: need %zu bytes", ws.total);
  alg::HeadParams p = head_params(dtype, N, d, V, h, E, targets, n, c, workspace, ws);
  p.stat = stat; p.zt = zt; p.pt = pt; p.obj = obj;
  if (f32) return hip_status(alg::launch_head_fwd_f32(p, (hipStream_t)stream), "alg_head_fwd");
  if (residual) {
    p.ut = reinterpret_cast<bf16*>(static_cast<char*>(residual) + ws.res_ut);
    p.lsum = reinterpret_cast<float*>(static_cast<char*>(residual) + ws.res_l);
  }
  return hip_status(alg::launch_head_fwd(p, (hipStream_t)stream), "alg_head_fwd");
}

size_t alg_rms_norm_workspace_size(int rows, int d) {
  if (rows <= 0 || d <= 0) return 0;
  // Per-workgroup gain partials (blocks x d), then their group sums (groups x d).
  return align256((size_t)d * alg::rms_norm_blocks(rows) * sizeof(float)) +
         align256((size_t)d * alg::rms_norm_gain_groups(rows) * sizeof(float));
}

static int check_rms_norm(int rows, int d, float eps) {
  if (rows <= 0 || d <= 0) return fail(ALG_ERR_INVALID, "rows and d must be positive (got %d, %d)", rows, d);
  if (d % 8) return fail(ALG_ERR_UNSUPPORTED, "d = %d: rows must be 16-byte aligned (d %% 8 == 0)", d);
  if (d > alg::rms_norm_max_d()) return fail(ALG_ERR_UNSUPPORTED, "d = %d: at most %d", d, alg::rms_norm_max_d());
  if (!(eps > 0.0f) || !std::isfinite(eps)) return fail(ALG_ERR_INVALID, "eps must be positive and finite");
  return ALG_OK;
}

int alg_rms_norm_fwd(alg_stream_t stream, int rows, int d, const void* x, const float* gain, float eps, void* y,
                     float* tau) {
  int rc = check_rms_norm(rows, d, eps);
  if (rc) return rc;
  if (!x || !y || !tau) return fail(ALG_ERR_INVALID, "x, y and tau are required");
  if (!aligned16({x, y})) return fail(ALG_ERR_INVALID, "x and y must be 16-byte aligned");
  alg::RmsNormParams p;
  std::memset(&p, 0, sizeof p);
  p.x = static_cast<const bf16*>(x); p.gain = gain; p.y = static_cast<bf16*>(y); p.tau = tau;
  p.rows = rows; p.d = d; p.eps = eps;
  return hip_status(alg::launch_rms_norm_fwd(p, (hipStream_t)stream), "alg_rms_norm_fwd");
}

int alg_rms_norm_bwd(alg_stream_t stream, int rows, int d, const void* x, const float* gain, const float* tau,
                     const void* dy, void* dx, float* dgain, void* workspace, size_t workspace_bytes) {
  int rc = check_rms_norm(rows, d, 1.0f);
  if (rc) return rc;
  if (!x || !tau || !dy || !dx) return fail(ALG_ERR_INVALID, "x, tau, dy and dx are required");
  if (!aligned16({x, dy, dx})) return fail(ALG_ERR_INVALID, "x, dy and dx must be 16-byte aligned");
  if (dgain && !gain) return fail(ALG_ERR_INVALID, "a gain gradient needs the gain it differentiates");
  const size_t need = alg_rms_norm_workspace_size(rows, d);
  if (dgain && (!workspace || workspace_bytes < need))
    return fail(ALG_ERR_INVALID, "workspace too small: need %zu bytes", need);
  alg::RmsNormParams p;
  std::memset(&p, 0, sizeof p);
  p.x = static_cast<const bf16*>(x); p.gain = gain; p.tau = const_cast<float*>(tau);
  p.dy = static_cast<const bf16*>(dy); p.dx = static_cast<bf16*>(dx);
  p.gpart = dgain ? static_cast<float*>(workspace) : nullptr;
  p.rows = rows; p.d = d;
  return hip_status(alg::launch_rms_norm_bwd(p, dgain, (hipStream_t)stream), "alg_rms_norm_bwd");
}

static int check_ffn(int N, int d, int F) {
  if (N <= 0 || d <= 0 || F <= 0) return fail(ALG_ERR_INVALID, "N, d, F must be positive (got %d, %d, %d)", N, d, F);
  if (d % 8) return fail(ALG_ERR_UNSUPPORTED, "width %d: rows must be 16-byte aligned (%% 8 == 0)", d);
  if (F % 128) return fail(ALG_ERR_UNSUPPORTED, "d_ff = %d: the fused gate/up product needs d_ff %% 128 == 0", F);
  if ((double)N * 2 * F > 2.0e9 || (double)d * 2 * F > 2.0e9 || (double)N * d > 2.0e9)
    return fail(ALG_ERR_INVALID, "feed-forward too large");
  return ALG_OK;
}

int alg_ffn_alu_glu_fwd(alg_stream_t stream, int N, int d, int F, const void* h2, const void* w_gu, float beta,
                        void* y, void* gate, void* up) {
  int rc = check_ffn(N, d, F);
  if (rc) return rc;
  if (!h2 || !w_gu || !y || !gate || !up) return fail(ALG_ERR_INVALID, "null argument");
  if (!aligned16({h2, w_gu, y, gate, up})) return fail(ALG_ERR_INVALID, "matrices must be 16-byte aligned");
  if (!std::isfinite(beta)) return fail(ALG_ERR_INVALID, "beta must be finite");
  alg::FfnParams p;
  std::memset(&p, 0, sizeof p);
  p.h2 = static_cast<const bf16*>(h2); p.w_gu = static_cast<const bf16*>(w_gu);
  p.y = static_cast<bf16*>(y); p.gate = static_cast<bf16*>(gate); p.up = static_cast<bf16*>(up);
  p.N = N; p.d = d; p.F = F; p.beta = beta;
  return hip_status(alg::launch_ffn_fwd(p, (hipStream_t)stream), "alg_ffn_alu_glu_fwd");
}

int alg_ffn_alu_glu_dy(alg_stream_t stream, int N, int dm, int F, const void* dout, const void* w_d, const void* gate,
                       const void* up, float beta, void* d_gu) {
  int rc = check_ffn(N, dm, F);
  if (rc) return rc;
  if (!dout || !w_d || !gate || !up || !d_gu) return fail(ALG_ERR_INVALID, "null argument");
  if (!aligned16({dout, w_d, gate, up, d_gu})) return fail(ALG_ERR_INVALID, "matrices must be 16-byte aligned");
  if (!std::isfinite(beta)) return fail(ALG_ERR_INVALID, "beta must be finite");
  alg::FfnParams p;
  std::memset(&p, 0, sizeof p);
  p.dout = static_cast<const bf16*>(dout); p.w_d = static_cast<const bf16*>(w_d);
  p.gate = const_cast<bf16*>(static_cast<const bf16*>(gate)); p.up = const_cast<bf16*>(static_cast<const bf16*>(up));
  p.d_gu = static_cast<bf16*>(d_gu);
  p.N = N; p.dm = dm; p.F = F; p.beta = beta;
  return hip_status(alg::launch_ffn_dy(p, (hipStream_t)stream), "alg_ffn_alu_glu_dy");
}

size_t alg_ffn_gemm_workspace_size(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return alg::ffn_gemm_workspace_bytes(alg::ffn_gemm_plan(M, N, K));
}

int alg_ffn_gemm(alg_stream_t stream, int M, int N, int K, const void* A, long lda, int a_trans, const void* B,
                 long ldb, int b_trans, void* C, long ldc, void* workspace, size_t workspace_bytes) {
  if (M <= 0 || N <= 0 || K <= 0) return fail(ALG_ERR_INVALID, "M, N, K must be positive (got %d, %d, %d)", M, N, K);
  if (!A || !B || !C) return fail(ALG_ERR_INVALID, "null argument");
  if (!aligned16({A, B, C})) return fail(ALG_ERR_INVALID, "A, B and C must be 16-byte aligned");
  // Stored row lengths: A (M, K) or (K, M); B (K, N) or (N, K).
  const int a_cols = a_trans ? M : K, a_rows = a_trans ? K : M;
  const int b_cols = b_trans ? K : N, b_rows = b_trans ? N : K;
  if (a_cols % 8 || b_cols % 8 || N % 8)
    return fail(ALG_ERR_INVALID, "stored row lengths (%d, %d) and N = %d must be multiples of 8", a_cols, b_cols, N);
  if (lda < a_cols || ldb < b_cols || ldc < N || lda % 8 || ldb % 8 || ldc % 8)
    return fail(ALG_ERR_INVALID, "leading dimensions (%ld, %ld, %ld) must cover the rows and be multiples of 8", lda,
                ldb, ldc);
  if ((double)(a_rows - 1) * lda + a_cols > 2.0e9 || (double)(b_rows - 1) * ldb + b_cols > 2.0e9 ||
      (double)(M - 1) * ldc + N > 2.0e9)
    return fail(ALG_ERR_INVALID, "matrices too large");
  const alg::FfnGemmPlan pl = alg::ffn_gemm_plan(M, N, K);
  const size_t need = alg::ffn_gemm_workspace_bytes(pl);
  if (need && (!workspace || workspace_bytes < need))
    return fail(ALG_ERR_INVALID, "workspace too small: need %zu bytes", need);
  if (need && !aligned16({workspace})) return fail(ALG_ERR_INVALID, "workspace must be 16-byte aligned");
  alg::FfnGemmParams g;
  std::memset(&g, 0, sizeof g);
  g.A = alg::GemmOperand{static_cast<const bf16*>(A), lda, a_rows, a_cols, (long)(a_rows - 1) * lda + a_cols};
  g.B = alg::GemmOperand{static_cast<const bf16*>(B), ldb, b_rows, b_cols, (long)(b_rows - 1) * ldb + b_cols};
  g.C = static_cast<bf16*>(C);
  g.ldc = ldc;
  g.M = M; g.N = N; g.K = K;
  g.full = pl.full; g.split = pl.split; g.kchunk = pl.kchunk;
  g.part = need ? static_cast<float*>(workspace) : nullptr;
  // A stored (M, K) is k-contiguous; B stored (N, K) is k-contiguous.
  return hip_status(alg::launch_ffn_gemm(g, a_trans ? alg::MNMAJOR : alg::KMAJOR, b_trans ? alg::KMAJOR : alg::MNMAJOR,
                                         (hipStream_t)stream),
                    "alg_ffn_gemm");
}

int alg_head_eval(alg_stream_t stream, int dtype, int N, int d, int V, const void* h, const void* E,
                  const int32_t* targets, int n, float c, float* logprob, int32_t* argmax, void* workspace,
                  size_t workspace_bytes) {
  int rc = check_head(N, d, V, n, c);
  if (!rc) rc = check_head_dtype(dtype, nullptr);
  if (rc) return rc;
  const bool f32 = dtype == ALG_DTYPE_F32;
  if (!h || !E || !targets || !logprob) return fail(ALG_ERR_INVALID, "null argument");
  if (!aligned16({h, E, workspace})) return fail(ALG_ERR_INVALID, "matrices must be 16-byte aligned");
  const HeadEvalWs ws = head_eval_ws(N, V, f32);
  if (!workspace || workspace_bytes < ws.total)
    return fail(ALG_ERR_INVALID, "workspace too small: need %zu bytes", ws.total);
  const HeadWs hw = f32 ? head_ws_f32(N, d, V, 0) : head_ws(N, d, V, 0, false);
  alg::HeadParams p = head_params(dtype, N, d, V, h, E, targets, n, c, workspace, hw);
  char* w = static_cast<char*>(workspace);
  p.partial = reinterpret_cast<float*>(w + ws.partial);
  p.pmax = reinterpret_cast<float*>(w + ws.pmax);
  p.pidx = reinterpret_cast<int*>(w + ws.pidx);
  p.obj_part = nullptr;
  p.zt = reinterpret_cast<float*>(logprob);  // the target logit is staged in the output
  p.logprob = logprob;
  p.argmax = argmax;
  if (f32) return hip_status(alg::launch_head_eval_f32(p, (hipStream_t)stream), "alg_head_eval");
  return hip_status(alg::launch_head_eval(p, (hipStream_t)stream), "alg_head_eval");
}

int alg_head_bwd(alg_stream_t stream, int dtype, int N, int d, int V, const void* h, const void* E,
                 const int32_t* targets, const float* stat, const float* g, int n, float c, const void* residual,
                 void* dh, void* dE, int dE_dtype, void* workspace, size_t workspace_bytes) {
  int rc = check_head(N, d, V, n, c);
  if (!rc) rc = check_train_head_n(n, residual);
  if (!rc) rc = check_head_dtype(dtype, residual);
  if (rc) return rc;
  const bool f32 = dtype == ALG_DTYPE_F32;
  if (!h || !E || !targets || !stat || !g || !dh || !dE) return fail(ALG_ERR_INVALID, "null argument");
  if (!aligned16({h, E, residual, dh, dE, workspace})) return fail(ALG_ERR_INVALID, "matrices must be 16-byte aligned");
  if (dE_dtype != ALG_DTYPE_BF16 && dE_dtype != ALG_DTYPE_F32) return fail(ALG_ERR_INVALID, "dE dtype must be bf16 or f32");
  const HeadWs ws = f32 ? head_ws_f32(N, d, V, 1) : head_ws(N, d, V, 1, residual != nullptr);
  if (!workspace || workspace_bytes < ws.total)
    return fail(ALG_ERR_INVALID, "workspace too small: need %zu bytes", ws.total);
  alg::HeadParams p = head_params(dtype, N, d, V, h, E, targets, n, c, workspace, ws);
  p.stat = const_cast<float*>(stat);
  p.g = g;
  char* w = static_cast<char*>(workspace);
  p.dE = dE;
  p.dE_f32 = dE_dtype == ALG_DTYPE_F32;
  if (f32) {
    p.dz32 = reinterpret_cast<float*>(w + ws.bwd);
    p.dh32 = static_cast<float*>(dh);
    p.dh_split = ws.dh_split;
    p.dh_kchunk = alg::head_f32_dh_kchunk(V, ws.dh_split);
    p.dh_part = ws.dh_split > 1 ? reinterpret_cast<float*>(w + ws.dh_part) : nullptr;
    return hip_status(alg::launch_head_bwd_f32(p, (hipStream_t)stream), "alg_head_bwd");
  }
  if (residual) {
    p.ut = reinterpret_cast<bf16*>(static_cast<char*>(const_cast<void*>(residual)) + ws.res_ut);
    p.lsum = reinterpret_cast<float*>(static_cast<char*>(const_cast<void*>(residual)) + ws.res_l);
    p.hs = reinterpret_cast<bf16*>(w + ws.bwd);
  } else {
    p.dzt = reinterpret_cast<bf16*>(w + ws.bwd);
  }
  p.dh = static_cast<bf16*>(dh);
  p.dh_split = ws.dh_split;
  p.dh_kchunk = alg::head_dh_kchunk(V, ws.dh_split);
  p.dh_part = ws.dh_split > 1 ? reinterpret_cast<float*>(w + ws.dh_part) : nullptr;
  p.de_full = ws.de.full;
  p.de_split = ws.de.split;
  p.de_kchunk = ws.de.kchunk;
  p.de_part = ws.de.split > 1 ? reinterpret_cast<float*>(w + ws.de_part) : nullptr;
  return hip_status(alg::launch_head_bwd(p, (hipStream_t)stream), "alg_head_bwd");
}

int alg_head_bwd_streamed(alg_stream_t stream, int dtype, int N, int d, int V, const void* h, const void* E,
                          const int32_t* targets, const float* stat, const float* g, int n, float c, int vocab_chunk,
                          void* dh, void* dE, int dE_dtype, void* workspace, size_t workspace_bytes) {
  int rc = check_head(N, d, V, n, c);
  if (!rc) rc = check_head_dtype(dtype, nullptr);
  if (rc) return rc;
  if (vocab_chunk < 0 || vocab_chunk % alg::HT_M)
    return fail(ALG_ERR_INVALID, "vocab_chunk %d: 0 (the default) or a positive multiple of %d", vocab_chunk,
                alg::HT_M);
  const bool f32 = dtype == ALG_DTYPE_F32;
  if (!h || !E || !targets || !stat || !g || !dh || !dE) return fail(ALG_ERR_INVALID, "null argument");
  if (!aligned16({h, E, dh, dE, workspace})) return fail(ALG_ERR_INVALID, "matrices must be 16-byte aligned");
  if (dE_dtype != ALG_DTYPE_BF16 && dE_dtype != ALG_DTYPE_F32) return fail(ALG_ERR_INVALID, "dE dtype must be bf16 or f32");
  const HeadStreamWs ws = head_stream_ws(dtype, N, d, V, vocab_chunk);
  if (!workspace || workspace_bytes < ws.total)
    return fail(ALG_ERR_INVALID, "workspace too small: need %zu bytes", ws.total);
  HeadWs hw;
  std::memset(&hw, 0, sizeof hw);
  hw.Npad = f32 ? N : alg::head_token_pad(N);
  hw.Vp = alg::head_vocab_pitch(V);
  alg::HeadParams p = head_params(dtype, N, d, V, h, E, targets, n, c, workspace, hw);
  p.partial = p.obj_part = nullptr;  // forward buffers
  p.stat = const_cast<float*>(stat);
  p.g = g;
  p.dE = dE;
  p.dE_f32 = dE_dtype == ALG_DTYPE_F32;
  char* w = static_cast<char*>(workspace);
  if (f32) {
    p.dz32 = reinterpret_cast<float*>(w + ws.dz);
    p.dh32 = static_cast<float*>(dh);
    return hip_status(alg::launch_head_bwd_f32_streamed(p, ws.chunk, (hipStream_t)stream), "alg_head_bwd_streamed");
  }
  p.dzt = reinterpret_cast<bf16*>(w + ws.dz);
  p.dh = static_cast<bf16*>(dh);
  p.dh_part = ws.nchunks > 1 ? reinterpret_cast<float*>(w + ws.acc) : nullptr;
  p.de_part = ws.has_de_part ? reinterpret_cast<float*>(w + ws.de_part) : nullptr;
  return hip_status(alg::launch_head_bwd_streamed(p, ws.chunk, (hipStream_t)stream), "alg_head_bwd_streamed");
}

}  // extern "C"
