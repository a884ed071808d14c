// Shared definitions for the gfx950 MoE kernels and their C-ABI shim.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <type_traits>

#include "nt_moe.h"

namespace ntmoe {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x8 __attribute__((ext_vector_type(8)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kRouteBlock = NT_MOE_ROUTE_BLOCK;  // tokens per router / histogram block
constexpr int kRouterChunk = 128;               // features per fixed-order partial sum

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __builtin_bit_cast(float, bits16 << 16);
}

// Round-to-nearest-even fp32 -> bf16 (gfx950 v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return (uint32_t)f32_to_bf16_bits(lo) | ((uint32_t)f32_to_bf16_bits(hi) << 16);
}

// (va, ia) ranks before (vb, ib): larger logit, or equal logit and lower expert index.
__device__ __forceinline__ bool rank_before(float va, int ia, float vb, int ib) {
  return va > vb || (va == vb && ia < ib);
}

__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// f(integral_constant<int, i>) for i = 0 .. N-1, each index a constant expression.
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>());
    static_for<I + 1, N>(f);
  }
}

inline int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

// Kernel launchers (one per translation unit). They assume validated arguments and return
// a hipError_t from the launch.
hipError_t launch_router(const uint16_t* x, int64_t ld_x, const float* wt, const float* bias,
                         int64_t T, int d, int E, int k, int score_fn, float* logits,
                         int32_t* topk_ids, float* topk_w, float* prob_partial,
                         float* z_partial, float* workspace, size_t workspace_bytes,
                         hipStream_t stream, int32_t* block_counts = nullptr);
hipError_t launch_topk_from_logits(const float* logits, int64_t T, int E, int k,
                                   int score_fn, int32_t* topk_ids, float* topk_w,
                                   float* prob_partial, float* z_partial, hipStream_t stream);
size_t router_workspace_need(int64_t T, int d, int E);

hipError_t launch_histogram_scan(const int32_t* topk_ids, int64_t T, int k, int E,
                                 int32_t* counts, int32_t* offsets, int32_t* ranks,
                                 int32_t* block_counts, hipStream_t stream);
// The router's route-plan outputs (launch_router's block_counts): the per-64-token-block expert
// counts [ceil(T/64)][E], then, from this offset (ints), each assignment's rank within its block
// among the tokens that chose its expert [T * k].
__host__ __device__ inline int64_t route_ranks_offset(int64_t T, int E) {
  return ((T + kRouteBlock - 1) / kRouteBlock * E + 63) / 64 * 64;
}
// The route plan from the router's per-64-token-block expert counts (ceil(T/64) x E, written by
// launch_router's block_counts): plan_kernel without the histogram launch. E <= 256.
hipError_t launch_plan_from_counts(const int32_t* topk_ids, const float* topk_w, int64_t T, int k,
                                   int E, const int32_t* block_counts64, int32_t* counts,
                                   int32_t* offsets, int32_t* src_row, float* perm_w,
                                   int32_t* combine_dest, float* combine_w, hipStream_t stream);
hipError_t launch_permute(const uint16_t* x, int64_t ld_x, const int32_t* topk_ids,
                          const float* topk_w, int64_t T, int d, int k, int E,
                          const int32_t* ranks, const int32_t* block_base,
                          int32_t* src_row, float* perm_w, int32_t* combine_dest,
                          float* combine_w, uint16_t* x_perm, hipStream_t stream);
hipError_t launch_grouped_gemm_bf16_packed_keep(const uint16_t* a, int64_t ld_a, int64_t a_rows,
                                                const int32_t* src_row,
                                                const int32_t* seg_offsets, int num_segments,
                                                int64_t total_rows, const uint16_t* wp, int K,
                                                int n_out, int epilogue, uint16_t* c,
                                                uint16_t* pre, hipStream_t stream);
hipError_t launch_grouped_wgrad(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                                int64_t b_rows, const int32_t* b_src_row,
                                const int32_t* seg_offsets, int num_segments, int64_t total_rows,
                                int N, int M, int splits, float* partial, bool c_f32, void* c,
                                hipStream_t stream);
// Two products over the same segments without split K: one launch of the 256 x 256 kernel
// when both take it, else one launch_grouped_wgrad after the other.
hipError_t launch_grouped_wgrad_pair(const uint16_t* a0, int64_t lda0, const uint16_t* b0,
                                     int64_t ldb0, int64_t b_rows0, const int32_t* b_src_row0,
                                     int N0, int M0, void* c0, const uint16_t* a1, int64_t lda1,
                                     const uint16_t* b1, int64_t ldb1, int64_t b_rows1,
                                     const int32_t* b_src_row1, int N1, int M1, void* c1,
                                     const int32_t* seg_offsets, int num_segments,
                                     int64_t total_rows, bool c_f32, hipStream_t stream);
hipError_t launch_combine_bwd(const uint16_t* g, int64_t ld_g, const uint16_t* y,
                              const int32_t* topk_ids, const int32_t* combine_dest,
                              const float* combine_w, int64_t T, int d, int k, uint16_t* dy,
                              float* dw, hipStream_t stream);
hipError_t launch_act_bwd(const uint16_t* fc1, const uint16_t* dh, int64_t rows, int H,
                          int activation, uint16_t* dfc1, hipStream_t stream);
hipError_t launch_first_operand(const float* grad_logits, int E, const uint16_t* dfc1s, int Fs,
                                int64_t T, int Ep, int Kc, uint16_t* out, hipStream_t stream);
hipError_t launch_router_bwd(const float* logits, const int32_t* topk_ids, const float* topk_w,
                             const float* dw, const int32_t* counts, int64_t T, int E, int k,
                             int score_fn, const float* grad_aux, float aux_coeff, float z_coeff,
                             float* dlogits, hipStream_t stream);
hipError_t launch_route_plan(const uint16_t* x, int64_t ld_x, const int32_t* topk_ids,
                             const float* topk_w, int64_t T, int d, int k, int E, int32_t* counts,
                             int32_t* offsets, int32_t* ranks, int32_t* block_counts,
                             int32_t* src_row, float* perm_w, int32_t* combine_dest,
                             float* combine_w, uint16_t* x_perm, hipStream_t stream);

hipError_t launch_grouped_ffn_bf16(const uint16_t* a, int64_t ld_a, int64_t a_rows,
                                   const int32_t* src_row,
                                   const int32_t* seg_offsets, int num_segments,
                                   int64_t total_rows, const uint16_t* w1, const uint16_t* w2,
                                   int d, int H, int activation, uint16_t* h, uint16_t* y,
                                   int* counters, hipStream_t stream);

hipError_t launch_grouped_gemm_bf16(const uint16_t* a, int64_t ld_a, int64_t a_rows,
                                    const int32_t* src_row, const int32_t* seg_offsets,
                                    int num_segments, int64_t total_rows, const uint16_t* w,
                                    int K, int n_out, int epilogue, uint16_t* c, int* counters,
                                    hipStream_t stream);

hipError_t launch_combine_aux(const uint16_t* y, const int32_t* combine_dest,
                              const float* combine_w, int64_t T, int d, int k,
                              const uint16_t* shared_y, int64_t ld_shared, uint16_t* out,
                              int64_t ld_out, const float* prob_partial, const float* z_partial,
                              const int32_t* counts, int E, float aux_coeff, float z_coeff,
                              float* aux_out, hipStream_t stream);

hipError_t launch_quantize_fp8_rowwise(const uint16_t* x, int64_t ld_x, int64_t rows, int d,
                                       uint8_t* q, int64_t ld_q, float* scale, hipStream_t stream);
hipError_t launch_quantize_fp8_blockwise(const float* w, int64_t S, int R, int C, uint8_t* q,
                                         float* scale, hipStream_t stream);
hipError_t launch_grouped_gemm_fp8(const uint8_t* a, int64_t ld_a, int64_t a_rows,
                                   const float* a_scale, const int32_t* src_row,
                                   const int32_t* seg_offsets, int num_segments,
                                   int64_t total_rows, const uint8_t* w, const float* w_scale,
                                   int K, int n_out, int epilogue, bool packed, uint16_t* c,
                                   hipStream_t stream);
hipError_t launch_pack_weights_fp8(const uint8_t* w, int64_t S, int R, int K, int epilogue,
                                   uint8_t* packed, hipStream_t stream);

hipError_t launch_pack_weights_bf16(const uint16_t* w, int64_t S, int R, int K, int epilogue,
                                    uint16_t* packed, hipStream_t stream);
hipError_t launch_grouped_gemm_bf16_packed(const uint16_t* a, int64_t ld_a, int64_t a_rows,
                                           const int32_t* src_row, const int32_t* seg_offsets,
                                           int num_segments, int64_t total_rows,
                                           const uint16_t* wp, int K, int n_out, int epilogue,
                                           uint16_t* c, hipStream_t stream);
int packed_gemm_min_k();
// The ping-pong packed GEMM (grouped_gemm_pp.hip): same operands and results as the packed
// kernel; pre (the fc1 pre-activations, SWIGLU / RELU2 only) may be null.
bool pp_gemm_supported(int K, int num_segments);
hipError_t launch_grouped_gemm_bf16_pp(const uint16_t* a, int64_t ld_a, int64_t a_rows,
                                       const int32_t* src_row, const int32_t* seg_offsets,
                                       int num_segments, int64_t total_rows, const uint16_t* wp,
                                       int K, int n_out, int epilogue, uint16_t* c, uint16_t* pre,
                                       hipStream_t stream);
hipError_t launch_convert_weights(const float* w, int64_t S, int R, int K, uint16_t* out,
                                  uint16_t* out_t, hipStream_t stream, uint16_t* pk = nullptr,
                                  int pk_swiglu_n = 0, uint16_t* pk_t = nullptr);
hipError_t launch_router_operands(const float* w, int64_t ldw, int E, int d, int dp,
                                  const uint16_t* sw, int64_t lds, int Fs, float* router_t,
                                  uint16_t* first, int Ep, int Kc, hipStream_t stream);
hipError_t launch_grouped_gemm_bf16_t256(const uint16_t* a, int64_t ld_a, int64_t a_rows,
                                         const int32_t* src_row, const int32_t* seg_offsets,
                                         int num_segments, int64_t total_rows, const uint16_t* w,
                                         int K, int n_out, int epilogue, uint16_t* c,
                                         hipStream_t stream);
// The same with the SWIGLU / RELU2 epilogue storing the fc1 pre-activations to pre as well.
hipError_t launch_grouped_gemm_bf16_t256_keep(const uint16_t* a, int64_t ld_a, int64_t a_rows,
                                              const int32_t* src_row, const int32_t* seg_offsets,
                                              int num_segments, int64_t total_rows,
                                              const uint16_t* w, int K, int n_out, int epilogue,
                                              uint16_t* c, uint16_t* pre, hipStream_t stream);

int num_cus();

// Workspace of the grouped GEMM entry points: per-XCD tile claim counters.
constexpr size_t kGemmWorkspaceBytes = 256;

// Lets `kernel` take `bytes` of dynamic LDS (gfx950: up to 160 KB per workgroup).
hipError_t allow_dynamic_lds(const void* kernel, size_t bytes);

}  // namespace ntmoe
