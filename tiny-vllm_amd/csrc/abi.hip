// C ABI of libtinyvllm_quant.so: argument validation, the M-bucketed path
// selection and the launches. Declared in include/tvq.h.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>

#include "../../include/tvq.h"
#include "tvq_internal.h"

namespace tvq {
namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return TVQ_OK;
}

constexpr int64_t kMaxDim = 0x7fffffff;

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int check_dims(int64_t M, int64_t N, int64_t K) {
  if (M < 0 || N <= 0 || K <= 0) return fail(TVQ_E_INVALID, "invalid shape M=%lld N=%lld K=%lld", (long long)M,
                                             (long long)N, (long long)K);
  if (M > kMaxDim || N > kMaxDim || K > kMaxDim)
    return fail(TVQ_E_UNSUPPORTED, "dimension exceeds 2^31-1: M=%lld N=%lld K=%lld", (long long)M, (long long)N,
                (long long)K);
  return TVQ_OK;
}

int check_dtype(int dtype) {
  if (dtype != TVQ_DTYPE_F16 && dtype != TVQ_DTYPE_BF16)
    return fail(TVQ_E_INVALID, "dtype must be TVQ_DTYPE_F16 (0) or TVQ_DTYPE_BF16 (1), got %d", dtype);
  return TVQ_OK;
}

bool shape_vec_ok(int64_t K) { return K % 16 == 0; }

// Recommended split-K workspace: the counter block plus the largest set of
// partial tiles the split policies produce on a 256-CU device (stream-K with
// 64x256 fp32 tiles: two 64 KiB images for each of 256 workgroups).
constexpr int64_t kGemmWorkspaceBytes = (32 << 20) + (64 << 10);

int check_workspace(const void* ws, int64_t bytes) {
  if (ws == nullptr) return TVQ_OK;
  if (((uintptr_t)ws & 255u) != 0) return fail(TVQ_E_INVALID, "workspace must be 256-byte aligned");
  if (bytes < 0) return fail(TVQ_E_INVALID, "negative workspace size %lld", (long long)bytes);
  return TVQ_OK;
}

int run_gemm(const GemmArgs& a, void* stream) {
  if (a.M == 0) return ok();
  hipError_t e;
  switch (select_gemm_path(a)) {
    case Path::kSkinny: e = launch_skinny(a, (hipStream_t)stream); break;
    case Path::kTiled: e = launch_tiled(a, (hipStream_t)stream); break;
    case Path::kDma: e = launch_dma_gemm(a, (hipStream_t)stream); break;
    case Path::kStream: e = launch_stream(a, (hipStream_t)stream); break;
    case Path::kGemv: e = launch_gemv(a, (hipStream_t)stream); break;
    default: e = launch_generic(a, (hipStream_t)stream); break;
  }
  if (e != hipSuccess) return fail(TVQ_E_HIP, "kernel launch failed: %s", hipGetErrorString(e));
  return ok();
}

}  // namespace

int report_error(int code, const char* msg) { return fail(code, "%s", msg); }

namespace {

// TVQ_GEMM_PATH=<gemv|skinny|stream|dma> forces that kernel family for
// the shapes it supports (others keep the automatic choice). A diagnostic for
// benchmarks and for tests that compare the families on the same inputs.
bool forced_path(const GemmArgs& a, Path* out) {
  const int f = switches().gemm_path;
  if (f < 0) return false;
  const Path p = (Path)f;
  bool ok;
  if (p == Path::kGemv) ok = gemv_shape_ok(a.M, a.K);
  else if (p == Path::kSkinny) ok = a.M <= kSkinnyMaxM;
  else if (p == Path::kStream) ok = stream_shape_ok(a.M, a.N, a.K);
  else ok = dma_shape_ok(a.K);
  if (!ok) return false;
  *out = p;
  return true;
}

thread_local const Switches* t_switches = nullptr;

}  // namespace

Switches read_switches() {
  Switches w{-1, false, 8, false};
  if (const char* e = getenv("TVQ_GEMM_PATH")) {
    if (!strcmp(e, "gemv")) w.gemm_path = (int)Path::kGemv;
    else if (!strcmp(e, "skinny")) w.gemm_path = (int)Path::kSkinny;
    else if (!strcmp(e, "stream")) w.gemm_path = (int)Path::kStream;
    else if (!strcmp(e, "dma")) w.gemm_path = (int)Path::kDma;
  }
  const char* sk = getenv("TVQ_STREAMK");
  w.streamk = sk != nullptr && sk[0] == '1';
  if (const char* e = getenv("TVQ_STREAMK_MIN")) {
    const int v = atoi(e);
    if (v >= 1 && v <= 64) w.streamk_min = v;
  }
  const char* w4 = getenv("TVQ_PREFILL_W4");
  w.prefill_w4 = w4 != nullptr && w4[0] == '1';
  return w;
}

const Switches& switches() {
  if (t_switches != nullptr) return *t_switches;
  thread_local Switches fresh;
  fresh = read_switches();
  return fresh;
}

SwitchScope::SwitchScope() : snap_(), owner_(t_switches == nullptr) {
  if (owner_) {
    snap_ = read_switches();
    t_switches = &snap_;
  }
}

SwitchScope::~SwitchScope() {
  if (owner_) t_switches = nullptr;
}

Path select_gemm_path(const GemmArgs& a) {
  const bool aligned = aligned16(a.x) && aligned16(a.qweight) && aligned16(a.y) && shape_vec_ok(a.K);
  if (!aligned) return Path::kGeneric;
  Path forced;
  if (forced_path(a, &forced)) return forced;
  if (gemv_shape_ok(a.M, a.K)) return Path::kGemv;
  if (a.M > kGemvMaxM && dma_shape_ok(a.K) && dma_streamk_on(a.M)) return Path::kDma;
  if (a.M <= kSkinnyMaxM) {
    if (dma_shape_ok(a.K) && (a.M > kDmaMinM || (a.M > 8 && a.N * a.K >= kDmaMidWeights))) return Path::kDma;
    return stream_shape_ok(a.M, a.N, a.K) ? Path::kStream : Path::kSkinny;
  }
  return dma_shape_ok(a.K) ? Path::kDma : Path::kTiled;
}

const char* gemm_path_name(bool w8a8, int64_t M, int64_t N, int64_t K, bool aligned) {
  if (!aligned || !shape_vec_ok(K)) return "generic_simt";
  if (gemv_shape_ok(M, K)) return w8a8 ? "gemv_dot4_i8" : "gemv_dot2_f16x";
  if (M > kGemvMaxM && dma_shape_ok(K) && dma_streamk_on(M)) return dma_path_name(w8a8, M, N, K, kGemmWorkspaceBytes);
  if (M <= kSkinnyMaxM && dma_shape_ok(K) && (M > kDmaMinM || (M > 8 && N * K >= kDmaMidWeights)))
    return dma_path_name(w8a8, M, N, K, kGemmWorkspaceBytes);
  if (M <= kSkinnyMaxM && stream_shape_ok(M, N, K)) {
    static const char* s8[4] = {"stream_mfma_i8_m16", "stream_mfma_i8_m32", "stream_mfma_i8_m48", "stream_mfma_i8_m64"};
    static const char* s16[4] = {"stream_mfma_f16x_m16", "stream_mfma_f16x_m32", "stream_mfma_f16x_m48",
                                 "stream_mfma_f16x_m64"};
    const int mg = (int)((M + 15) / 16) - 1;
    return w8a8 ? s8[mg] : s16[mg];
  }
  if (M <= kSkinnyMaxM) {
    static const char* names8[4] = {"skinny_mfma_i8_m16", "skinny_mfma_i8_m32", "skinny_mfma_i8_m48",
                                    "skinny_mfma_i8_m64"};
    static const char* names16[4] = {"skinny_mfma_f16x_m16", "skinny_mfma_f16x_m32", "skinny_mfma_f16x_m48",
                                     "skinny_mfma_f16x_m64"};
    const int mg = M <= 0 ? 0 : (int)((M + 15) / 16) - 1;
    return w8a8 ? names8[mg] : names16[mg];
  }
  if (dma_shape_ok(K)) return dma_path_name(w8a8, M, N, K, kGemmWorkspaceBytes);
  return w8a8 ? "tiled_mfma_i8_128x128x128" : "tiled_mfma_f16x_128x128x64";
}

}  // namespace tvq

using namespace tvq;

extern "C" {

int tvq_abi_version(void) { return TVQ_ABI_VERSION; }

const char* tvq_last_error(void) { return g_last_error.c_str(); }

const char* tvq_select_path(int op, int64_t M, int64_t N, int64_t K, int dtype) {
  SwitchScope switch_scope;
  (void)dtype;
  switch (op) {
    case TVQ_OP_ACT_QUANT: return (K % 8 == 0) ? "act_quant_vec" : "act_quant_scalar";
    case TVQ_OP_W8A16: return gemm_path_name(false, M, N, K, true);
    case TVQ_OP_W8A8: return gemm_path_name(true, M, N, K, true);
    default: return nullptr;
  }
}

int tvq_act_quant(const void* x, int dtype, int64_t M, int64_t K, float eps, int8_t* xq, float* a_scales,
                  void* stream) {
  if (int rc = check_dtype(dtype)) return rc;
  if (int rc = check_dims(M, 1, K)) return rc;
  if (M == 0) return ok();
  if (!x || !xq || !a_scales) return fail(TVQ_E_INVALID, "null pointer argument");
  if (!(eps >= 0.0f)) return fail(TVQ_E_INVALID, "eps must be >= 0");
  hipError_t e = launch_act_quant(x, dtype == TVQ_DTYPE_BF16, M, K, eps, xq, a_scales, (hipStream_t)stream);
  if (e != hipSuccess) return fail(TVQ_E_HIP, "act_quant launch failed: %s", hipGetErrorString(e));
  return ok();
}

int64_t tvq_gemm_workspace_bytes(void) { return kGemmWorkspaceBytes; }

int tvq_w8a16_gemm(const void* x, int dtype, const int8_t* qweight, const float* scales, const void* bias, void* y,
                   int64_t M, int64_t N, int64_t K, void* workspace, int64_t workspace_bytes, void* stream) {
  SwitchScope switch_scope;
  if (int rc = check_dtype(dtype)) return rc;
  if (int rc = check_dims(M, N, K)) return rc;
  if (int rc = check_workspace(workspace, workspace_bytes)) return rc;
  if (M == 0) return ok();
  if (!x || !qweight || !scales || !y) return fail(TVQ_E_INVALID, "null pointer argument");
  GemmArgs a{x, nullptr, qweight, scales, bias, y, M, N, K, false, dtype == TVQ_DTYPE_BF16, false, workspace,
             workspace_bytes};
  return run_gemm(a, stream);
}

int tvq_w8a8_gemm(const int8_t* xq, const float* a_scales, const int8_t* qweight, const float* w_scales,
                  const void* bias, void* y, int out_dtype, int64_t M, int64_t N, int64_t K, void* workspace,
                  int64_t workspace_bytes, void* stream) {
  SwitchScope switch_scope;
  if (int rc = check_dtype(out_dtype)) return rc;
  if (int rc = check_dims(M, N, K)) return rc;
  if (int rc = check_workspace(workspace, workspace_bytes)) return rc;
  if (M == 0) return ok();
  if (!xq || !a_scales || !qweight || !w_scales || !y) return fail(TVQ_E_INVALID, "null pointer argument");
  GemmArgs a{xq, a_scales, qweight, w_scales, bias, y, M, N, K, true, out_dtype == TVQ_DTYPE_BF16, false, workspace,
             workspace_bytes};
  return run_gemm(a, stream);
}

int tvq_w8a16_gemm_rounded(const void* x, int dtype, const int8_t* qweight, const float* scales, const void* bias,
                           void* y, int64_t M, int64_t N, int64_t K, void* stream) {
  SwitchScope switch_scope;
  if (int rc = check_dtype(dtype)) return rc;
  if (int rc = check_dims(M, N, K)) return rc;
  if (M == 0) return ok();
  if (!x || !qweight || !scales || !y) return fail(TVQ_E_INVALID, "null pointer argument");
  GemmArgs a{x, nullptr, qweight, scales, bias, y, M, N, K, false, dtype == TVQ_DTYPE_BF16, false};
  const bool aligned = aligned16(x) && aligned16(qweight) && aligned16(y);
  hipError_t e = (aligned && dma_shape_ok(K)) ? launch_dma_dq(a, (hipStream_t)stream)
                                              : launch_generic_dq(a, (hipStream_t)stream);
  if (e != hipSuccess) return fail(TVQ_E_HIP, "kernel launch failed: %s", hipGetErrorString(e));
  return ok();
}

int tvq_gemm_operand_floor(int op, const void* x, const int8_t* qweight, int64_t M, int64_t N, int64_t K,
                           void* stream) {
  SwitchScope switch_scope;
  if (op != TVQ_OP_W8A16 && op != TVQ_OP_W8A8) return fail(TVQ_E_INVALID, "op must be TVQ_OP_W8A16 or TVQ_OP_W8A8");
  if (int rc = check_dims(M, N, K)) return rc;
  if (M == 0) return ok();
  if (!x || !qweight) return fail(TVQ_E_INVALID, "null pointer argument");
  if (!dma_shape_ok(K) || !aligned16(x) || !aligned16(qweight))
    return fail(TVQ_E_UNSUPPORTED, "operand floor: the DMA tiles need K %% 128 == 0 and 16-byte aligned operands");
  GemmArgs a{x, nullptr, qweight, nullptr, nullptr, nullptr, M, N, K, op == TVQ_OP_W8A8, true, false};
  hipError_t e = launch_dma_floor(a, (hipStream_t)stream);
  if (e != hipSuccess) return fail(TVQ_E_HIP, "kernel launch failed: %s", hipGetErrorString(e));
  return ok();
}

int tvq_w8a8_gemm_i32(const int8_t* xq, const int8_t* qweight, int32_t* y_i32, int64_t M, int64_t N, int64_t K,
                      void* workspace, int64_t workspace_bytes, void* stream) {
  SwitchScope switch_scope;
  if (int rc = check_dims(M, N, K)) return rc;
  if (int rc = check_workspace(workspace, workspace_bytes)) return rc;
  if (M == 0) return ok();
  if (!xq || !qweight || !y_i32) return fail(TVQ_E_INVALID, "null pointer argument");
  GemmArgs a{xq, nullptr, qweight, nullptr, nullptr, y_i32, M, N, K, true, true, true, workspace, workspace_bytes};
  return run_gemm(a, stream);
}

int tvq_w8a8_linear(const void* x, int dtype, const int8_t* qweight, const float* w_scales, const void* bias,
                    void* y, int64_t M, int64_t N, int64_t K, int8_t* xq_buf, float* a_scales_buf, void* workspace,
                    int64_t workspace_bytes, void* stream) {
  SwitchScope switch_scope;
  if (int rc = check_dtype(dtype)) return rc;
  if (int rc = check_dims(M, N, K)) return rc;
  if (int rc = check_workspace(workspace, workspace_bytes)) return rc;
  if (M == 0) return ok();
  if (!x || !qweight || !w_scales || !y || !xq_buf || !a_scales_buf)
    return fail(TVQ_E_INVALID, "null pointer argument");
  if (int rc = tvq_act_quant(x, dtype, M, K, 1e-8f, xq_buf, a_scales_buf, stream)) return rc;
  return tvq_w8a8_gemm(xq_buf, a_scales_buf, qweight, w_scales, bias, y, dtype, M, N, K, workspace, workspace_bytes,
                       stream);
}

int tvq_rmsnorm(const void* x, void* residual, const void* weight, float eps, void* y, int8_t* xq, float* a_scales,
                int dtype, int64_t M, int64_t K, void* stream) {
  if (int rc = check_dtype(dtype)) return rc;
  if (int rc = check_dims(M, 1, K)) return rc;
  if (M == 0) return ok();
  if (!x || !weight) return fail(TVQ_E_INVALID, "null pointer argument");
  if (!y && !xq) return fail(TVQ_E_INVALID, "rmsnorm needs an output: y and/or xq");
  if (xq && !a_scales) return fail(TVQ_E_INVALID, "xq given without a_scales");
  if (!(eps >= 0.0f)) return fail(TVQ_E_INVALID, "eps must be >= 0");
  hipError_t e = launch_rmsnorm(x, residual, weight, eps, y, xq, a_scales, dtype == TVQ_DTYPE_BF16, M, K,
                                (hipStream_t)stream);
  if (e != hipSuccess) return fail(TVQ_E_HIP, "rmsnorm launch failed: %s", hipGetErrorString(e));
  return ok();
}

int tvq_w8a8_gemm_glu(const int8_t* xq, const float* a_scales, const int8_t* qweight_glu, const float* w_scales_glu,
                      void* y, int out_dtype, int64_t M, int64_t N2, int64_t K, void* stream) {
  SwitchScope switch_scope;
  if (int rc = check_dtype(out_dtype)) return rc;
  if (int rc = check_dims(M, N2, K)) return rc;
  if (M == 0) return ok();
  if (!xq || !a_scales || !qweight_glu || !w_scales_glu || !y) return fail(TVQ_E_INVALID, "null pointer argument");
  if (N2 % 64 != 0 || !dma_shape_ok(K))
    return fail(TVQ_E_UNSUPPORTED, "gemm_glu needs N2 %% 64 == 0 and K %% 128 == 0 (K <= 2^22)");
  if (!aligned16(xq) || !aligned16(qweight_glu) || !aligned16(y) || !aligned16(w_scales_glu))
    return fail(TVQ_E_UNSUPPORTED, "gemm_glu needs 16-byte aligned pointers");
  GemmArgs a{xq, a_scales, qweight_glu, w_scales_glu, nullptr, y, M, N2, K, true, out_dtype == TVQ_DTYPE_BF16, false};
  hipError_t e = launch_dma_glu(a, (hipStream_t)stream);
  if (e != hipSuccess) return fail(TVQ_E_HIP, "gemm_glu launch failed: %s", hipGetErrorString(e));
  return ok();
}

int tvq_silu_mul(const void* gate_up, void* y, int8_t* xq, float* a_scales, int dtype, int64_t M, int64_t I,
                 void* stream) {
  if (int rc = check_dtype(dtype)) return rc;
  if (int rc = check_dims(M, 1, 2 * I)) return rc;
  if (M == 0) return ok();
  if (!gate_up) return fail(TVQ_E_INVALID, "null pointer argument");
  if (!y && !xq) return fail(TVQ_E_INVALID, "silu_mul needs an output: y and/or xq");
  if (xq && !a_scales) return fail(TVQ_E_INVALID, "xq given without a_scales");
  hipError_t e = launch_silu_mul(gate_up, y, xq, a_scales, dtype == TVQ_DTYPE_BF16, M, I, (hipStream_t)stream);
  if (e != hipSuccess) return fail(TVQ_E_HIP, "silu_mul launch failed: %s", hipGetErrorString(e));
  return ok();
}

int tvq_decode_attention(const void* q, int64_t q_stride, const void* k_new, int64_t k_stride, const void* v_new,
                         int64_t v_stride, void* k_cache, void* v_cache, const int32_t* slots, const int32_t* lens,
                         int64_t B, int Hq, int Hkv, int head_dim, int64_t num_slots, int64_t max_len, float scale,
                         void* out, int dtype, void* stream) {
  if (int rc = check_dtype(dtype)) return rc;
  if (B < 0 || B > kMaxDim || max_len <= 0 || max_len > kMaxDim || num_slots <= 0 || num_slots > kMaxDim)
    return fail(TVQ_E_INVALID, "invalid B / num_slots / max_len");
  if (B == 0) return ok();
  if (!q || !k_new || !v_new || !k_cache || !v_cache || !slots || !lens || !out)
    return fail(TVQ_E_INVALID, "null pointer argument");
  if (head_dim != 128) return fail(TVQ_E_UNSUPPORTED, "head_dim must be 128, got %d", head_dim);
  if (Hkv <= 0 || Hq <= 0 || Hq % Hkv != 0 || (Hq / Hkv != 1 && Hq / Hkv != 2 && Hq / Hkv != 4))
    return fail(TVQ_E_UNSUPPORTED, "Hq/Hkv must be 1, 2 or 4 (Hq=%d, Hkv=%d)", Hq, Hkv);
  if (!aligned16(q) || !aligned16(k_new) || !aligned16(v_new) || !aligned16(k_cache) || !aligned16(v_cache) ||
      !aligned16(out) || q_stride % 8 || k_stride % 8 || v_stride % 8)
    return fail(TVQ_E_UNSUPPORTED, "decode attention needs 16-byte aligned pointers and strides");
  hipError_t e = launch_decode_attention(q, q_stride, k_new, k_stride, v_new, v_stride, k_cache, v_cache, slots, lens,
                                         (int)B, Hq, Hkv, (int)max_len, (int)num_slots, scale, out, dtype == TVQ_DTYPE_BF16,
                                         (hipStream_t)stream);
  if (e != hipSuccess) return fail(TVQ_E_HIP, "decode attention launch failed: %s", hipGetErrorString(e));
  return ok();
}

int tvq_qk_norm_rope(const void* qkv, int64_t row_stride, const int64_t* positions, const float* cos_t,
                     const float* sin_t, const void* q_weight, const void* k_weight, float eps, int64_t T, int Hq,
                     int Hkv, int head_dim, int64_t max_pos, void* q_out, void* k_out, void* k_cache, void* v_cache,
                     const int64_t* slots, int64_t num_slots, int64_t max_len, int dtype, void* stream) {
  if (int rc = check_dtype(dtype)) return rc;
  if (T < 0 || T > kMaxDim || Hq <= 0 || Hkv <= 0 || max_pos <= 0 || max_pos > kMaxDim)
    return fail(TVQ_E_INVALID, "invalid T / heads / max_pos");
  if (T == 0) return ok();
  if (head_dim != 128) return fail(TVQ_E_UNSUPPORTED, "head_dim must be 128, got %d", head_dim);
  if (!qkv || !positions || !cos_t || !sin_t || !q_out || !k_out) return fail(TVQ_E_INVALID, "null pointer argument");
  if ((q_weight == nullptr) != (k_weight == nullptr)) return fail(TVQ_E_INVALID, "give both norm weights or neither");
  const bool store = k_cache != nullptr;
  if (store != (v_cache != nullptr) || store != (slots != nullptr))
    return fail(TVQ_E_INVALID, "give k_cache, v_cache and slots together or none");
  if (store && (num_slots <= 0 || num_slots > kMaxDim || max_len <= 0 || max_len > kMaxDim))
    return fail(TVQ_E_INVALID, "invalid num_slots / max_len");
  if (row_stride < (int64_t)(Hq + (store ? 2 : 1) * Hkv) * head_dim)
    return fail(TVQ_E_INVALID, "row_stride shorter than the heads read");
  if (T * (Hq + 2 * Hkv) / 32 + 1 > kMaxDim) return fail(TVQ_E_UNSUPPORTED, "too many (token, head) pairs");
  // 16-byte accesses throughout
  if (!aligned16(qkv) || row_stride % 8 || !aligned16(q_out) || !aligned16(k_out) || !aligned16(q_weight) ||
      !aligned16(k_weight) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(cos_t) || !aligned16(sin_t))
    return fail(TVQ_E_UNSUPPORTED, "qk_norm_rope needs 16-byte aligned rows (row_stride %% 8 == 0), outputs, "
                                   "weights, caches and cos/sin tables");
  hipError_t e = launch_qk_norm_rope(qkv, row_stride, positions, cos_t, sin_t, q_weight, k_weight, eps, T, Hq, Hkv,
                                     (int)max_pos, q_out, k_out, k_cache, v_cache, slots, (int)num_slots,
                                     (int)max_len, dtype == TVQ_DTYPE_BF16, (hipStream_t)stream);
  if (e != hipSuccess) return fail(TVQ_E_HIP, "qk_norm_rope launch failed: %s", hipGetErrorString(e));
  return ok();
}

int tvq_prefill_attention(const void* q, const void* k, const void* v, int64_t v_stride, const int32_t* blocks,
                          int64_t nblocks, int Hq, int Hkv, int head_dim, float scale, void* out, int dtype,
                          void* stream) {
  if (int rc = check_dtype(dtype)) return rc;
  if (nblocks < 0 || nblocks > kMaxDim) return fail(TVQ_E_INVALID, "invalid nblocks");
  if (nblocks == 0) return ok();
  if (!q || !k || !v || !blocks || !out) return fail(TVQ_E_INVALID, "null pointer argument");
  if (head_dim != 128) return fail(TVQ_E_UNSUPPORTED, "head_dim must be 128, got %d", head_dim);
  if (Hkv <= 0 || Hq <= 0 || Hq % Hkv != 0 || Hq > 65535) return fail(TVQ_E_INVALID, "invalid Hq / Hkv");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out) || v_stride % 8)
    return fail(TVQ_E_UNSUPPORTED, "prefill attention needs 16-byte aligned pointers and strides");
  hipError_t e = launch_prefill_attention(q, k, v, v_stride, blocks, (int)nblocks, Hq, Hkv, scale, out,
                                          dtype == TVQ_DTYPE_BF16, (hipStream_t)stream);
  if (e != hipSuccess) return fail(TVQ_E_HIP, "prefill attention launch failed: %s", hipGetErrorString(e));
  return ok();
}

namespace {

// Checks of the quantized-output arguments of the attention entry points.
int check_attn_quant(int8_t* xq, float* a_scales, int32_t* counters, int64_t counters_len, int64_t needed,
                     float eps) {
  if (!xq || !a_scales || !counters) return fail(TVQ_E_INVALID, "null xq / a_scales / counters");
  if (counters_len < needed)
    return fail(TVQ_E_INVALID, "counters hold %lld entries, %lld needed", (long long)counters_len, (long long)needed);
  if (((uintptr_t)xq & 3u) != 0 || ((uintptr_t)counters & 3u) != 0)
    return fail(TVQ_E_UNSUPPORTED, "xq and counters must be 4-byte aligned");
  if (!(eps > 0.0f)) return fail(TVQ_E_INVALID, "eps must be positive");
  return TVQ_OK;
}

}  // namespace

int tvq_decode_attention_quant(const void* q, int64_t q_stride, const void* k_new, int64_t k_stride,
                               const void* v_new, int64_t v_stride, void* k_cache, void* v_cache,
                               const int32_t* slots, const int32_t* lens, int64_t B, int Hq, int Hkv, int head_dim,
                               int64_t num_slots, int64_t max_len, float scale, void* out, int dtype, int8_t* xq,
                               float* a_scales, float eps, int32_t* counters, int64_t counters_len, void* stream) {
  if (B > 0)
    if (int rc = check_attn_quant(xq, a_scales, counters, counters_len, B, eps)) return rc;
  if (int rc = check_dtype(dtype)) return rc;
  if (B < 0 || B > kMaxDim || max_len <= 0 || max_len > kMaxDim || num_slots <= 0 || num_slots > kMaxDim)
    return fail(TVQ_E_INVALID, "invalid B / num_slots / max_len");
  if (B == 0) return ok();
  if (!q || !k_new || !v_new || !k_cache || !v_cache || !slots || !lens || !out)
    return fail(TVQ_E_INVALID, "null pointer argument");
  if (head_dim != 128) return fail(TVQ_E_UNSUPPORTED, "head_dim must be 128, got %d", head_dim);
  if (Hkv <= 0 || Hq <= 0 || Hq % Hkv != 0 || (Hq / Hkv != 1 && Hq / Hkv != 2 && Hq / Hkv != 4))
    return fail(TVQ_E_UNSUPPORTED, "Hq/Hkv must be 1, 2 or 4 (Hq=%d, Hkv=%d)", Hq, Hkv);
  if (!aligned16(q) || !aligned16(k_new) || !aligned16(v_new) || !aligned16(k_cache) || !aligned16(v_cache) ||
      !aligned16(out) || q_stride % 8 || k_stride % 8 || v_stride % 8)
    return fail(TVQ_E_UNSUPPORTED, "decode attention needs 16-byte aligned pointers and strides");
  const AttnQuant qo{xq, a_scales, counters, eps};
  hipError_t e = launch_decode_attention(q, q_stride, k_new, k_stride, v_new, v_stride, k_cache, v_cache, slots, lens,
                                         (int)B, Hq, Hkv, (int)max_len, (int)num_slots, scale, out,
                                         dtype == TVQ_DTYPE_BF16, (hipStream_t)stream, &qo);
  if (e != hipSuccess) return fail(TVQ_E_HIP, "decode attention launch failed: %s", hipGetErrorString(e));
  return ok();
}

int tvq_prefill_attention_quant(const void* q, const void* k, const void* v, int64_t v_stride, const int32_t* blocks,
                                int64_t nblocks, int Hq, int Hkv, int head_dim, float scale, void* out, int dtype,
                                int8_t* xq, float* a_scales, float eps, int32_t* counters, int64_t counters_len,
                                void* stream) {
  if (nblocks > 0)
    if (int rc = check_attn_quant(xq, a_scales, counters, counters_len, nblocks, eps)) return rc;
  if (int rc = check_dtype(dtype)) return rc;
  if (nblocks < 0 || nblocks > kMaxDim) return fail(TVQ_E_INVALID, "invalid nblocks");
  if (nblocks == 0) return ok();
  if (!q || !k || !v || !blocks || !out) return fail(TVQ_E_INVALID, "null pointer argument");
  if (head_dim != 128) return fail(TVQ_E_UNSUPPORTED, "head_dim must be 128, got %d", head_dim);
  if (Hkv <= 0 || Hq <= 0 || Hq % Hkv != 0 || Hq > 65535) return fail(TVQ_E_INVALID, "invalid Hq / Hkv");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out) || v_stride % 8)
    return fail(TVQ_E_UNSUPPORTED, "prefill attention needs 16-byte aligned pointers and strides");
  const AttnQuant qo{xq, a_scales, counters, eps};
  hipError_t e = launch_prefill_attention(q, k, v, v_stride, blocks, (int)nblocks, Hq, Hkv, scale, out,
                                          dtype == TVQ_DTYPE_BF16, (hipStream_t)stream, &qo);
  if (e != hipSuccess) return fail(TVQ_E_HIP, "prefill attention launch failed: %s", hipGetErrorString(e));
  return ok();
}

}  // extern "C"
