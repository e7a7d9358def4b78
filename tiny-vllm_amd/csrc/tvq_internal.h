// Host-side launch helpers shared between the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tvq {

// Kernel families chosen by the M-bucketed dispatcher.
enum class Path : int {
  kGeneric = 0,  // scalar reference-order kernel: any K, any alignment
  kSkinny = 1,   // M <= 64: weight-streaming MFMA GEMV / skinny GEMM
  kTiled = 2,    // M > 64, K % 128 != 0: register-staged double-buffered MFMA tiles
  kDma = 3,      // M > 64, K % 128 == 0: LDS-DMA multi-stage MFMA tiles
  kStream = 4,   // 8 < M <= 64, N >= 16384, K % 256 == 0: weight streaming, LDS-shared activations
  kGemv = 5,     // M <= 2, K % 1024 == 0: row-contiguous vector-ALU GEMV
};

struct GemmArgs {
  const void* x;         // W8A16: [M,K] 16-bit; W8A8: [M,K] int8
  const float* a_scales; // W8A8 only
  const int8_t* qweight; // [N,K]
  const float* scales;   // [N]
  const void* bias;      // [N] 16-bit or nullptr
  void* y;               // [M,N] 16-bit, or int32 when raw_i32
  int64_t M, N, K;
  bool w8a8;
  bool bf16;     // activation (W8A16) / output (W8A8) element type
  bool raw_i32;  // W8A8 only: write the int32 accumulator instead of y
  void* workspace = nullptr;    // split-K workspace (counters zero on entry), or nullptr
  int64_t workspace_bytes = 0;
};

bool act_quant_vec_ok(const void* x, const void* xq, int64_t K);

// Environment switches of the GEMM dispatch (diagnostic / opt-in):
//   TVQ_GEMM_PATH=gemv|skinny|stream|dma  force a kernel family where valid
//   TVQ_STREAMK=1      stream-K for decode-size DMA shapes
//   TVQ_STREAMK_MIN=n  stream-K: at least n k-stages per workgroup (default 8)
//   TVQ_PREFILL_W4=1   the 4-wave prefill tiles
// Read once per C-ABI call (SwitchScope at each GEMM entry point), so every
// decision inside one call (path name, tile, split, launch) sees the same
// values; outside a scope they are read afresh.
struct Switches {
  int gemm_path;  // -1 none, else a Path value
  bool streamk;
  int streamk_min;
  bool prefill_w4;
};
Switches read_switches();
const Switches& switches();  // the current call's snapshot
class SwitchScope {
 public:
  SwitchScope();
  ~SwitchScope();
  SwitchScope(const SwitchScope&) = delete;
  SwitchScope& operator=(const SwitchScope&) = delete;

 private:
  Switches snap_;
  bool owner_;
};

// Attention output quantized for the W8A8 o_proj in the same launch: per-token
// int8 codes [T, Hq*128] and fp32 scales [T], and the row-block counters of
// the last-arrival handoff (zero on entry, left zero).
struct AttnQuant {
  int8_t* xq;
  float* a_scales;
  int32_t* counters;
  float eps;
};
hipError_t launch_rmsnorm(const void* x, void* residual, const void* weight, float eps, void* y, int8_t* xq,
                          float* a_scales, bool bf16, int64_t M, int64_t K, hipStream_t stream);
hipError_t launch_decode_attention(const void* q, int64_t q_stride, const void* k_new, int64_t k_stride,
                                   const void* v_new, int64_t v_stride, void* k_cache, void* v_cache,
                                   const int32_t* slots, const int32_t* lens, int B, int Hq, int Hkv, int max_len,
                                   int num_slots, float scale, void* out, bool bf16, hipStream_t stream,
                                   const AttnQuant* quant = nullptr);
hipError_t launch_qk_norm_rope(const void* qkv, int64_t row_stride, const int64_t* positions, const float* cos_t,
                               const float* sin_t, const void* q_weight, const void* k_weight, float eps, int64_t T_,
                               int Hq, int Hkv, int max_pos, void* q_out, void* k_out, void* k_cache, void* v_cache,
                               const int64_t* slots, int num_slots, int max_len, bool bf16, hipStream_t stream);
hipError_t launch_prefill_attention(const void* q, const void* k, const void* v, int64_t v_stride,
                                    const int32_t* blocks, int nblocks, int Hq, int Hkv, float scale, void* out,
                                    bool bf16, hipStream_t stream, const AttnQuant* quant = nullptr);
hipError_t launch_silu_mul(const void* gate_up, void* y, int8_t* xq, float* a_scales, bool bf16, int64_t M,
                           int64_t I, hipStream_t stream);
hipError_t launch_act_quant(const void* x, bool bf16, int64_t M, int64_t K, float eps, int8_t* xq, float* a_scales,
                            hipStream_t stream);

// Records `msg` as this thread's tvq_last_error() and returns `code`.
int report_error(int code, const char* msg);

// Path selection (pure function of shape and pointer alignment).
Path select_gemm_path(const GemmArgs& a);
const char* gemm_path_name(bool w8a8, int64_t M, int64_t N, int64_t K, bool aligned);

hipError_t launch_skinny(const GemmArgs& a, hipStream_t stream);
hipError_t launch_tiled(const GemmArgs& a, hipStream_t stream);
hipError_t launch_generic(const GemmArgs& a, hipStream_t stream);
hipError_t launch_dma_gemm(const GemmArgs& a, hipStream_t stream);
hipError_t launch_dma_glu(const GemmArgs& a, hipStream_t stream);
// The DMA tiling's operand stream alone (no arithmetic, no output): the
// measurement floor of launch_dma_gemm for the same shape.
hipError_t launch_dma_floor(const GemmArgs& a, hipStream_t stream);
// W8A16 with each weight dequantized to T(T(q) * T(s)) before the dot product
// (the reference kernel's rounding): DMA tiles when K % 128 == 0, else the
// generic kernel.
hipError_t launch_dma_dq(const GemmArgs& a, hipStream_t stream);
hipError_t launch_generic_dq(const GemmArgs& a, hipStream_t stream);
bool dma_shape_ok(int64_t K);
// TVQ_STREAMK=1 and M <= 64: decode-size DMA launches use stream-K, and the
// dispatcher sends every such M above the GEMV range (M > 2) to the DMA tiles.
bool dma_streamk_on(int64_t M);
// Path name, with a "_splitk" suffix when a workspace of the given size makes
// the launch split K (which needs the device: without one it never splits).
const char* dma_path_name(bool w8a8, int64_t M, int64_t N, int64_t K, int64_t workspace_bytes);
int dma_splits(bool w8a8, int64_t M, int64_t N, int64_t K, int64_t workspace_bytes);

hipError_t launch_stream(const GemmArgs& a, hipStream_t stream);
hipError_t launch_gemv(const GemmArgs& a, hipStream_t stream);
bool gemv_shape_ok(int64_t M, int64_t K);
bool stream_shape_ok(int64_t M, int64_t N, int64_t K);

// Largest M served by the skinny / stream families; above kDmaMinM they are
// used only when K % 128 != 0 (the DMA tiles need whole 128-k stages).
constexpr int64_t kSkinnyMaxM = 64;
constexpr int64_t kDmaMinM = 16;
// 8 < M <= 16 also takes the DMA tiles (with split-K) when the weights are at
// least this large: 1.2-1.3x faster than the skinny / stream kernels on the
// 8B qkv, gate_up and down shapes at M = 16, slower on smaller ones.
constexpr int64_t kDmaMidWeights = 24ll << 20;
constexpr int64_t kGemvMaxM = 2;  // M = 4 measured 20-35 % slower than the skinny MFMA kernel

}  // namespace tvq
