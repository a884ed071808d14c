// C-ABI shim: argument validation, workspace layout and status codes around the kernel
// launchers. Declarations and contracts: include/nt_moe.h.
//
// Error model (mirrors the reference's ValueError / RuntimeError split,
// nexttransformer/scaling/moe_recipe.py:54-72, megatron_moe.py:97-98): invalid arguments give
// NT_MOE_EINVAL, a short workspace NT_MOE_ENOSPC, a failed launch NT_MOE_EDEVICE; the message
// is kept per thread for nt_moe_last_error(). Nothing here allocates device memory or
// synchronises.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>
#include <mutex>
#include <unordered_map>

#include "common.h"

namespace ntmoe {
namespace {

thread_local char g_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof g_error, fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_error[0] = '\0';
  return NT_MOE_OK;
}

int launched(hipError_t err, const char* what) {
  if (err != hipSuccess)
    return fail(NT_MOE_EDEVICE, "%s: launch failed: %s", what, hipGetErrorString(err));
  return ok();
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool aligned_to(const void* p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }

size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

constexpr int kHistBlock = 256;  // tokens per histogram block (route.hip)

struct RouteWorkspace {
  int32_t* ranks;
  int32_t* block_counts;
};

size_t route_ws_bytes(int64_t T, int k, int E) {
  int64_t nblk = (T + kHistBlock - 1) / kHistBlock;
  return align256((size_t)T * k * 4) + align256((size_t)nblk * E * 4);
}

RouteWorkspace route_ws(void* ws, int64_t T, int k) {
  RouteWorkspace r;
  r.ranks = reinterpret_cast<int32_t*>(ws);
  r.block_counts = reinterpret_cast<int32_t*>(reinterpret_cast<char*>(ws) + align256((size_t)T * k * 4));
  return r;
}

#define NT_REQUIRE(cond, ...) \
  do {                        \
    if (!(cond)) return fail(NT_MOE_EINVAL, __VA_ARGS__); \
  } while (0)

int check_route_shape(int64_t T, int k, int E) {
  NT_REQUIRE(T >= 0 && T <= (int64_t)1 << 26, "T must be in [0, 2^26], got %lld", (long long)T);
  NT_REQUIRE(E >= 1 && E <= NT_MOE_MAX_EXPERTS, "E must be in [1, %d], got %d", NT_MOE_MAX_EXPERTS, E);
  NT_REQUIRE(k >= 1 && k <= NT_MOE_MAX_TOPK && k <= E, "top-k must be in [1, min(%d, E)], got %d",
             NT_MOE_MAX_TOPK, k);
  NT_REQUIRE(T * k < ((int64_t)1 << 31), "T * k must fit int32");
  return NT_MOE_OK;
}

// The grouped GEMM addresses its operands with 32-bit byte offsets per lane.
int check_gemm_extent(int64_t a_rows, int64_t ld_a, int64_t w_rows_per_segment, int64_t K) {
  NT_REQUIRE(a_rows * ld_a * 2 <= ((int64_t)1 << 32),
             "grouped GEMM: a spans %lld bytes, more than the 4 GiB the loader addresses",
             (long long)(a_rows * ld_a * 2));
  NT_REQUIRE(w_rows_per_segment * K * 2 <= ((int64_t)1 << 32),
             "grouped GEMM: one segment's weights exceed 4 GiB");
  return NT_MOE_OK;
}

}  // namespace

int num_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v > 0) return v;
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    n = 256;
  cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

// Raises a kernel's dynamic-LDS limit once per (device, kernel) to the largest size asked for so
// far: hipFuncSetAttribute on every launch stalled the stream for about 6 us before each
// large-LDS kernel.
hipError_t allow_dynamic_lds(const void* kernel, size_t bytes) {
  if (bytes <= 65536) return hipSuccess;
  static std::mutex mu;
  static std::unordered_map<const void*, size_t> granted[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  std::lock_guard<std::mutex> lock(mu);
  auto it = granted[dev].find(kernel);
  if (it != granted[dev].end() && it->second >= bytes) return hipSuccess;
  hipError_t err =
      hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (err == hipSuccess) granted[dev][kernel] = bytes;
  return err;
}

}  // namespace ntmoe

using namespace ntmoe;

extern "C" {

int nt_moe_abi_version(void) { return NT_MOE_ABI_VERSION; }

const char* nt_moe_last_error(void) { return g_error; }

size_t nt_moe_router_workspace_bytes(int64_t T, int32_t d, int32_t E, int32_t k) {
  (void)k;
  if (T <= 0 || d <= 0 || E <= 0) return 0;
  return router_workspace_need(T, d, E);
}

int nt_moe_router_fwd(const uint16_t* x, int64_t ld_x, const float* w_router_t,
                      const float* logit_bias, int64_t T, int32_t d, int32_t E, int32_t k,
                      int32_t score_fn, float* logits, int32_t* topk_ids, float* topk_w,
                      float* prob_partial, float* z_partial, void* workspace,
                      size_t workspace_bytes, nt_moe_stream_t stream) {
  int rc = check_route_shape(T, k, E);
  if (rc) return rc;
  NT_REQUIRE(d > 0 && d % 8 == 0, "router: d must be a positive multiple of 8, got %d", d);
  NT_REQUIRE(ld_x >= d && ld_x % 8 == 0, "router: ld_x must be >= d and a multiple of 8");
  NT_REQUIRE(score_fn == NT_MOE_SCORE_SOFTMAX || score_fn == NT_MOE_SCORE_SIGMOID,
             "router: unknown score_fn %d", score_fn);
  if (T == 0) return ok();
  NT_REQUIRE(x && w_router_t && topk_ids && topk_w && prob_partial && z_partial,
             "router: null buffer");
  NT_REQUIRE(aligned16(x), "router: x must be 16-byte aligned");
  NT_REQUIRE(E <= 256 || (workspace && workspace_bytes >= router_workspace_need(T, d, E)) ||
                 (logits && d <= 16 * 128),
             "router: more than 256 experts need the workspace");
  hipError_t err = launch_router(x, ld_x, w_router_t, logit_bias, T, d, E, k, score_fn, logits,
                                 topk_ids, topk_w, prob_partial, z_partial,
                                 reinterpret_cast<float*>(workspace), workspace_bytes,
                                 reinterpret_cast<hipStream_t>(stream));
  return launched(err, "router");
}

int nt_moe_topk_from_logits(const float* logits, int64_t T, int32_t E, int32_t k,
                            int32_t score_fn, int32_t* topk_ids, float* topk_w,
                            float* prob_partial, float* z_partial, nt_moe_stream_t stream) {
  int rc = check_route_shape(T, k, E);
  if (rc) return rc;
  NT_REQUIRE(score_fn == NT_MOE_SCORE_SOFTMAX || score_fn == NT_MOE_SCORE_SIGMOID,
             "topk: unknown score_fn %d", score_fn);
  if (T == 0) return ok();
  NT_REQUIRE(logits && topk_ids && topk_w && prob_partial && z_partial, "topk: null buffer");
  hipError_t err = launch_topk_from_logits(logits, T, E, k, score_fn, topk_ids, topk_w,
                                           prob_partial, z_partial,
                                           reinterpret_cast<hipStream_t>(stream));
  return launched(err, "topk");
}

size_t nt_moe_route_workspace_bytes(int64_t T, int32_t k, int32_t E) {
  if (T < 0 || k <= 0 || E <= 0) return 0;
  return route_ws_bytes(T, k, E);
}

int nt_moe_histogram_scan(const int32_t* topk_ids, int64_t T, int32_t k, int32_t E,
                          int32_t* counts, int32_t* offsets, void* workspace,
                          size_t workspace_bytes, nt_moe_stream_t stream) {
  int rc = check_route_shape(T, k, E);
  if (rc) return rc;
  NT_REQUIRE(counts && offsets && workspace, "histogram: null buffer");
  NT_REQUIRE(T == 0 || topk_ids, "histogram: null topk_ids");
  if (workspace_bytes < route_ws_bytes(T, k, E))
    return fail(NT_MOE_ENOSPC, "histogram: workspace %zu < %zu bytes", workspace_bytes,
                route_ws_bytes(T, k, E));
  RouteWorkspace ws = route_ws(workspace, T, k);
  hipError_t err = launch_histogram_scan(topk_ids, T, k, E, counts, offsets, ws.ranks,
                                         ws.block_counts, reinterpret_cast<hipStream_t>(stream));
  return launched(err, "histogram_scan");
}

int nt_moe_permute(const uint16_t* x, int64_t ld_x, const int32_t* topk_ids,
                   const float* topk_w, int64_t T, int32_t d, int32_t k, int32_t E,
                   const void* workspace, size_t workspace_bytes, int32_t* src_row,
                   float* perm_w, int32_t* combine_dest, float* combine_w, uint16_t* x_perm,
                   nt_moe_stream_t stream) {
  int rc = check_route_shape(T, k, E);
  if (rc) return rc;
  if (T == 0) return ok();
  NT_REQUIRE(topk_ids && topk_w && workspace && src_row && combine_dest && combine_w,
             "permute: null buffer");
  if (workspace_bytes < route_ws_bytes(T, k, E))
    return fail(NT_MOE_ENOSPC, "permute: workspace %zu < %zu bytes", workspace_bytes,
                route_ws_bytes(T, k, E));
  if (x_perm) {
    NT_REQUIRE(x, "permute: x_perm requested without x");
    NT_REQUIRE(d > 0 && d % 8 == 0, "permute: d must be a positive multiple of 8, got %d", d);
    NT_REQUIRE(ld_x >= d && ld_x % 8 == 0, "permute: ld_x must be >= d and a multiple of 8");
    NT_REQUIRE(aligned16(x) && aligned16(x_perm), "permute: x and x_perm must be 16-byte aligned");
  }
  RouteWorkspace ws = route_ws(const_cast<void*>(workspace), T, k);
  hipError_t err = launch_permute(x, ld_x, topk_ids, topk_w, T, d, k, E, ws.ranks,
                                  ws.block_counts, src_row, perm_w, combine_dest, combine_w,
                                  x_perm, reinterpret_cast<hipStream_t>(stream));
  return launched(err, "permute");
}

int nt_moe_combine_bwd(const uint16_t* grad_out, int64_t ld_grad, const uint16_t* y,
                       const int32_t* topk_ids, const int32_t* combine_dest,
                       const float* combine_w, int64_t T, int32_t d, int32_t k,
                       uint16_t* grad_y, float* grad_w, nt_moe_stream_t stream) {
  NT_REQUIRE(T >= 0 && T * (int64_t)k < ((int64_t)1 << 31), "combine_bwd: T * k must fit int32");
  NT_REQUIRE(k >= 1 && k <= NT_MOE_MAX_TOPK, "combine_bwd: top-k must be in [1, %d], got %d",
             NT_MOE_MAX_TOPK, k);
  NT_REQUIRE(d > 0 && d % 8 == 0, "combine_bwd: d must be a positive multiple of 8, got %d", d);
  NT_REQUIRE(ld_grad >= d && ld_grad % 8 == 0, "combine_bwd: ld_grad must be >= d and a multiple of 8");
  if (T == 0) return ok();
  NT_REQUIRE(grad_out && y && topk_ids && combine_dest && combine_w && grad_y && grad_w,
             "combine_bwd: null buffer");
  NT_REQUIRE(aligned16(grad_out) && aligned16(y) && aligned16(grad_y),
             "combine_bwd: grad_out, y and grad_y must be 16-byte aligned");
  return launched(launch_combine_bwd(grad_out, ld_grad, y, topk_ids, combine_dest, combine_w, T,
                                     d, k, grad_y, grad_w, reinterpret_cast<hipStream_t>(stream)),
                  "combine_bwd");
}

int nt_moe_act_bwd(const uint16_t* fc1, const uint16_t* grad_h, int64_t rows, int32_t H,
                   int32_t activation, uint16_t* grad_fc1, nt_moe_stream_t stream) {
  NT_REQUIRE(rows >= 0, "act_bwd: rows must be >= 0");
  NT_REQUIRE(H > 0 && H % 8 == 0, "act_bwd: H must be a positive multiple of 8, got %d", H);
  NT_REQUIRE(activation == NT_MOE_ACT_SWIGLU || activation == NT_MOE_ACT_RELU2,
             "act_bwd: unknown activation %d", activation);
  if (rows == 0) return ok();
  NT_REQUIRE(fc1 && grad_h && grad_fc1, "act_bwd: null buffer");
  NT_REQUIRE(aligned16(fc1) && aligned16(grad_h) && aligned16(grad_fc1),
             "act_bwd: buffers must be 16-byte aligned");
  return launched(launch_act_bwd(fc1, grad_h, rows, H, activation, grad_fc1,
                                 reinterpret_cast<hipStream_t>(stream)),
                  "act_bwd");
}

int nt_moe_backward_first_operand(const float* grad_logits, int32_t E, const uint16_t* dfc1s,
                                  int32_t Fs, int64_t T, int32_t Ep, int32_t Kc, uint16_t* out,
                                  nt_moe_stream_t stream) {
  NT_REQUIRE(T >= 0 && E > 0 && Ep >= E && Ep % 8 == 0 && Fs >= 0 && Fs % 8 == 0 && Kc % 8 == 0 &&
                 Kc >= Fs + 3 * Ep,
             "backward_first_operand: need E <= Ep, Kc >= Fs + 3 Ep, Fs, Ep, Kc multiples of 8");
  if (T == 0) return ok();
  NT_REQUIRE(grad_logits && out && (Fs == 0 || dfc1s),
             "backward_first_operand: null buffer");
  NT_REQUIRE(aligned16(out) && (Fs == 0 || aligned16(dfc1s)),
             "backward_first_operand: buffers must be 16-byte aligned");
  return launched(launch_first_operand(grad_logits, E, dfc1s, Fs, T, Ep, Kc, out,
                                       reinterpret_cast<hipStream_t>(stream)),
                  "backward_first_operand");
}

namespace {

int check_wgrad(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb, int64_t b_rows,
                const int32_t* b_src_row, const int32_t* seg_offsets, int32_t num_segments,
                int64_t total_rows, int32_t N, int32_t M, const void* c) {
  NT_REQUIRE(N > 0 && N % 64 == 0 && M > 0 && M % 64 == 0,
             "grouped_wgrad: N and M must be positive multiples of 64, got %d, %d", N, M);
  NT_REQUIRE(num_segments >= 1 && num_segments <= NT_MOE_MAX_SEGMENTS,
             "grouped_wgrad: num_segments must be in [1, %d]", NT_MOE_MAX_SEGMENTS);
  NT_REQUIRE(total_rows >= 0 && total_rows < ((int64_t)1 << 31), "grouped_wgrad: bad total_rows");
  NT_REQUIRE(lda >= N && lda % 8 == 0 && ldb >= M && ldb % 8 == 0,
             "grouped_wgrad: lda >= N, ldb >= M, both multiples of 8");
  NT_REQUIRE(b_src_row ? b_rows >= 1 : b_rows >= total_rows,
             "grouped_wgrad: b needs total_rows rows without b_src_row");
  NT_REQUIRE(a && b && seg_offsets && c, "grouped_wgrad: null buffer");
  NT_REQUIRE(aligned16(a) && aligned16(b) && aligned16(c),
             "grouped_wgrad: buffers must be 16-byte aligned");
  return NT_MOE_OK;
}

}  // namespace

int nt_moe_grouped_wgrad_bf16(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                              int64_t b_rows, const int32_t* b_src_row,
                              const int32_t* seg_offsets, int32_t num_segments,
                              int64_t total_rows, int32_t N, int32_t M, uint16_t* c,
                              nt_moe_stream_t stream) {
  int rc = check_wgrad(a, lda, b, ldb, b_rows, b_src_row, seg_offsets, num_segments, total_rows,
                       N, M, c);
  if (rc) return rc;
  return launched(launch_grouped_wgrad(a, lda, b, ldb, b_rows, b_src_row, seg_offsets,
                                       num_segments, total_rows, N, M, 1, nullptr, false, c,
                                       reinterpret_cast<hipStream_t>(stream)),
                  "grouped_wgrad");
}

int nt_moe_grouped_wgrad_splitk(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                                int64_t b_rows, const int32_t* b_src_row,
                                const int32_t* seg_offsets, int32_t num_segments,
                                int64_t total_rows, int32_t N, int32_t M, int32_t splits,
                                float* partial, size_t partial_bytes, int32_t c_fp32, void* c,
                                nt_moe_stream_t stream) {
  int rc = check_wgrad(a, lda, b, ldb, b_rows, b_src_row, seg_offsets, num_segments, total_rows,
                       N, M, c);
  if (rc) return rc;
  NT_REQUIRE(splits >= 1 && splits <= 256, "grouped_wgrad_splitk: splits must be in [1, 256]");
  const size_t need = splits > 1 ? (size_t)splits * num_segments * N * M * sizeof(float) : 0;
  if (splits > 1) {
    NT_REQUIRE(partial && aligned16(partial), "grouped_wgrad_splitk: null or unaligned partial");
    if (partial_bytes < need)
      return fail(NT_MOE_ENOSPC, "grouped_wgrad_splitk: partial %zu < %zu bytes", partial_bytes,
                  need);
  }
  return launched(launch_grouped_wgrad(a, lda, b, ldb, b_rows, b_src_row, seg_offsets,
                                       num_segments, total_rows, N, M, splits, partial,
                                       c_fp32 != 0, c, reinterpret_cast<hipStream_t>(stream)),
                  "grouped_wgrad_splitk");
}

int nt_moe_grouped_wgrad_pair(const uint16_t* a0, int64_t lda0, const uint16_t* b0, int64_t ldb0,
                              int64_t b_rows0, const int32_t* b_src_row0, int32_t N0, int32_t M0,
                              void* c0, const uint16_t* a1, int64_t lda1, const uint16_t* b1,
                              int64_t ldb1, int64_t b_rows1, const int32_t* b_src_row1,
                              int32_t N1, int32_t M1, void* c1, const int32_t* seg_offsets,
                              int32_t num_segments, int64_t total_rows, int32_t c_fp32,
                              nt_moe_stream_t stream) {
  int rc = check_wgrad(a0, lda0, b0, ldb0, b_rows0, b_src_row0, seg_offsets, num_segments,
                       total_rows, N0, M0, c0);
  if (rc) return rc;
  rc = check_wgrad(a1, lda1, b1, ldb1, b_rows1, b_src_row1, seg_offsets, num_segments, total_rows,
                   N1, M1, c1);
  if (rc) return rc;
  return launched(launch_grouped_wgrad_pair(a0, lda0, b0, ldb0, b_rows0, b_src_row0, N0, M0, c0,
                                            a1, lda1, b1, ldb1, b_rows1, b_src_row1, N1, M1, c1,
                                            seg_offsets, num_segments, total_rows, c_fp32 != 0,
                                            reinterpret_cast<hipStream_t>(stream)),
                  "grouped_wgrad_pair");
}

int nt_moe_router_bwd(const float* logits, const int32_t* topk_ids, const float* topk_w,
                      const float* grad_w, const int32_t* counts, int64_t T, int32_t E,
                      int32_t k, int32_t score_fn, const float* grad_aux, float aux_coeff,
                      float z_coeff, float* grad_logits, nt_moe_stream_t stream) {
  int rc = check_route_shape(T, k, E);
  if (rc) return rc;
  NT_REQUIRE(score_fn == NT_MOE_SCORE_SOFTMAX || score_fn == NT_MOE_SCORE_SIGMOID,
             "router_bwd: unknown score_fn %d", score_fn);
  if (T == 0) return ok();
  NT_REQUIRE(logits && topk_ids && topk_w && grad_w && counts && grad_logits,
             "router_bwd: null buffer");
  return launched(launch_router_bwd(logits, topk_ids, topk_w, grad_w, counts, T, E, k, score_fn,
                                    grad_aux, aux_coeff, z_coeff, grad_logits,
                                    reinterpret_cast<hipStream_t>(stream)),
                  "router_bwd");
}

namespace {

// Argument checks shared by the route-plan entry points (everything but the scratch memory).
int check_route_plan(const uint16_t* x, int64_t ld_x, const int32_t* topk_ids,
                     const float* topk_w, int64_t T, int32_t d, int32_t k, int32_t E,
                     const int32_t* counts, const int32_t* offsets, const int32_t* src_row,
                     const int32_t* combine_dest, const float* combine_w, const uint16_t* x_perm) {
  int rc = check_route_shape(T, k, E);
  if (rc) return rc;
  NT_REQUIRE(counts && offsets, "route_plan: null buffer");
  NT_REQUIRE(T == 0 || (topk_ids && topk_w && src_row && combine_dest && combine_w),
             "route_plan: null buffer");
  if (x_perm && T > 0) {
    NT_REQUIRE(x, "route_plan: x_perm requested without x");
    NT_REQUIRE(d > 0 && d % 8 == 0, "route_plan: d must be a positive multiple of 8, got %d", d);
    NT_REQUIRE(ld_x >= d && ld_x % 8 == 0, "route_plan: ld_x must be >= d and a multiple of 8");
    NT_REQUIRE(aligned16(x) && aligned16(x_perm),
               "route_plan: x and x_perm must be 16-byte aligned");
  }
  return NT_MOE_OK;
}

}  // namespace

int nt_moe_route_plan(const uint16_t* x, int64_t ld_x, const int32_t* topk_ids,
                      const float* topk_w, int64_t T, int32_t d, int32_t k, int32_t E,
                      int32_t* counts, int32_t* offsets, void* workspace, size_t workspace_bytes,
                      int32_t* src_row, float* perm_w, int32_t* combine_dest, float* combine_w,
                      uint16_t* x_perm, nt_moe_stream_t stream) {
  int rc = check_route_plan(x, ld_x, topk_ids, topk_w, T, d, k, E, counts, offsets, src_row,
                            combine_dest, combine_w, x_perm);
  if (rc) return rc;
  NT_REQUIRE(workspace, "route_plan: null buffer");
  if (workspace_bytes < route_ws_bytes(T, k, E))
    return fail(NT_MOE_ENOSPC, "route_plan: workspace %zu < %zu bytes", workspace_bytes,
                route_ws_bytes(T, k, E));
  RouteWorkspace ws = route_ws(workspace, T, k);
  hipError_t err = launch_route_plan(x, ld_x, topk_ids, topk_w, T, d, k, E, counts, offsets,
                                     ws.ranks, ws.block_counts, src_row, perm_w, combine_dest,
                                     combine_w, x_perm, reinterpret_cast<hipStream_t>(stream));
  return launched(err, "route_plan");
}

namespace {

// The one-launch plan reads the whole per-64-token-block counts table in every workgroup; past
// this many entries the histogram + plan kernels (a table four times smaller) are faster
// (measured at T = 16384, E = 256 and T = 32768, E = 64).
constexpr int64_t kCountsPlanMax = 16384;

bool plan_from_counts(int64_t T, int E) {
  return ((T + NT_MOE_ROUTE_BLOCK - 1) / NT_MOE_ROUTE_BLOCK) * E <= kCountsPlanMax;
}

}  // namespace

size_t nt_moe_router_plan_workspace_bytes(int64_t T, int32_t d, int32_t E, int32_t k) {
  if (T <= 0 || d <= 0 || E <= 0 || k <= 0) return 0;
  // the router's counts table and ranks (route_ranks_offset), or the route plan's workspace
  const size_t plan = plan_from_counts(T, E)
                          ? align256((size_t)(route_ranks_offset(T, E) + T * (int64_t)k) * 4)
                          : route_ws_bytes(T, k, E);
  return align256(router_workspace_need(T, d, E)) + plan;
}

int nt_moe_router_plan(const uint16_t* x, int64_t ld_x, const float* w_router_t,
                       const float* logit_bias, int64_t T, int32_t d, int32_t E, int32_t k,
                       int32_t score_fn, float* logits, int32_t* topk_ids, float* topk_w,
                       float* prob_partial, float* z_partial, int32_t* counts, int32_t* offsets,
                       int32_t* src_row, float* perm_w, int32_t* combine_dest,
                       float* combine_w, void* workspace, size_t workspace_bytes,
                       nt_moe_stream_t stream) {
  int rc = check_route_shape(T, k, E);
  if (rc) return rc;
  NT_REQUIRE(d > 0 && d % 8 == 0, "router_plan: d must be a positive multiple of 8, got %d", d);
  NT_REQUIRE(ld_x >= d && ld_x % 8 == 0, "router_plan: ld_x must be >= d and a multiple of 8");
  NT_REQUIRE(score_fn == NT_MOE_SCORE_SOFTMAX || score_fn == NT_MOE_SCORE_SIGMOID,
             "router_plan: unknown score_fn %d", score_fn);
  NT_REQUIRE(counts && offsets, "router_plan: null buffer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (T == 0)  // counts and offsets are zero: the scan over no blocks
    return launched(launch_histogram_scan(nullptr, 0, k, E, counts, offsets, nullptr, nullptr, st),
                    "router_plan");
  NT_REQUIRE(x && w_router_t && topk_ids && topk_w && prob_partial && z_partial && src_row &&
                 combine_dest && combine_w && workspace,
             "router_plan: null buffer");
  NT_REQUIRE(aligned16(x), "router_plan: x must be 16-byte aligned");
  const size_t need = nt_moe_router_plan_workspace_bytes(T, d, E, k);
  if (workspace_bytes < need)
    return fail(NT_MOE_ENOSPC, "router_plan: workspace %zu < %zu bytes", workspace_bytes, need);
  const size_t router_part = align256(router_workspace_need(T, d, E));
  void* plan_ws = reinterpret_cast<char*>(workspace) + router_part;
  const bool from_counts = plan_from_counts(T, E);
  hipError_t err = launch_router(x, ld_x, w_router_t, logit_bias, T, d, E, k, score_fn, logits,
                                 topk_ids, topk_w, prob_partial, z_partial,
                                 router_part ? reinterpret_cast<float*>(workspace) : nullptr,
                                 router_part, st,
                                 from_counts ? reinterpret_cast<int32_t*>(plan_ws) : nullptr);
  if (err != hipSuccess) return launched(err, "router_plan (router)");
  if (from_counts)
    return launched(launch_plan_from_counts(topk_ids, topk_w, T, k, E,
                                            reinterpret_cast<int32_t*>(plan_ws), counts, offsets,
                                            src_row, perm_w, combine_dest, combine_w, st),
                    "router_plan (plan)");
  RouteWorkspace ws = route_ws(plan_ws, T, k);
  return launched(launch_route_plan(nullptr, 0, topk_ids, topk_w, T, d, k, E, counts, offsets,
                                    ws.ranks, ws.block_counts, src_row, perm_w, combine_dest,
                                    combine_w, nullptr, st),
                  "router_plan (plan)");
}

namespace {

// The route plan's scratch for nt_moe_route_plan_noalloc: NT_MOE_NOALLOC_MAX_ASSIGNMENTS ranks,
// then NT_MOE_NOALLOC_MAX_BLOCK_COUNTS per-block expert counts (2 MiB). Each GPU holds its own
// copy at its own address until the process ends. Host code never passes the array's name to a
// kernel (on the host it is only a stand-in): it uses the device address that
// hipGetSymbolAddress returns, looked up once per device with that device current.
constexpr int64_t kNoAllocRanks = NT_MOE_NOALLOC_MAX_ASSIGNMENTS;
constexpr int64_t kNoAllocBlockCounts = NT_MOE_NOALLOC_MAX_BLOCK_COUNTS;
static __device__ __align__(256) int32_t scratch[kNoAllocRanks + kNoAllocBlockCounts];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
int32_t* g_scratch_ptr[kMaxDevices];  // device address of `scratch` on each device, or null

// The current device's scratch address (looked up on the device's first call); the stream must
// belong to that device, since the address is only valid there.
int scratch_address(hipStream_t stream, int32_t** out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(NT_MOE_EDEVICE, "route_plan_noalloc: no usable current device (%s)",
                hipGetErrorString(err));
  if (stream) {
    int stream_dev = -1;
    err = hipStreamGetDevice(stream, &stream_dev);
    if (err != hipSuccess)
      return fail(NT_MOE_EDEVICE, "route_plan_noalloc: hipStreamGetDevice: %s",
                  hipGetErrorString(err));
    NT_REQUIRE(stream_dev == dev,
               "route_plan_noalloc: the stream belongs to device %d but device %d is current",
               stream_dev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !p)
      return fail(NT_MOE_EDEVICE, "route_plan_noalloc: hipGetSymbolAddress: %s",
                  hipGetErrorString(err));
    g_scratch_ptr[dev] = static_cast<int32_t*>(p);
  }
  *out = g_scratch_ptr[dev];
  return NT_MOE_OK;
}

}  // namespace

int nt_moe_route_plan_noalloc(const uint16_t* x, int64_t ld_x, const int32_t* topk_ids,
                              const float* topk_w, int64_t T, int32_t d, int32_t k, int32_t E,
                              int32_t* counts, int32_t* offsets, int32_t* src_row, float* perm_w,
                              int32_t* combine_dest, float* combine_w, uint16_t* x_perm,
                              nt_moe_stream_t stream) {
  int rc = check_route_plan(x, ld_x, topk_ids, topk_w, T, d, k, E, counts, offsets, src_row,
                            combine_dest, combine_w, x_perm);
  if (rc) return rc;
  const int64_t nblk = (T + kHistBlock - 1) / kHistBlock;
  NT_REQUIRE(T * k <= kNoAllocRanks,
             "route_plan_noalloc: T * k = %lld exceeds the static scratch's %lld assignments",
             (long long)(T * k), (long long)kNoAllocRanks);
  NT_REQUIRE(nblk * E <= kNoAllocBlockCounts,
             "route_plan_noalloc: ceil(T / %d) * E = %lld exceeds the static scratch's %lld "
             "block counts", kHistBlock, (long long)(nblk * E), (long long)kNoAllocBlockCounts);
  int32_t* base = nullptr;
  rc = scratch_address(reinterpret_cast<hipStream_t>(stream), &base);
  if (rc) return rc;
  // Every scratch value the kernels read is written earlier in the same call (ranks of every
  // assignment, counts of every block and expert), so nothing needs clearing between calls.
  hipError_t err = launch_route_plan(x, ld_x, topk_ids, topk_w, T, d, k, E, counts, offsets,
                                     base, base + kNoAllocRanks, src_row, perm_w, combine_dest,
                                     combine_w, x_perm, reinterpret_cast<hipStream_t>(stream));
  return launched(err, "route_plan_noalloc");
}

size_t nt_moe_grouped_gemm_workspace_bytes(void) { return kGemmWorkspaceBytes; }

int nt_moe_grouped_ffn_bf16(const uint16_t* a, int64_t ld_a, int64_t a_rows, const int32_t* src_row,
                            const int32_t* seg_offsets, int32_t num_segments,
                            int64_t total_rows, const uint16_t* w1, const uint16_t* w2,
                            int32_t d, int32_t H, int32_t activation, uint16_t* h,
                            uint16_t* y, void* workspace, size_t workspace_bytes,
                            nt_moe_stream_t stream) {
  NT_REQUIRE(d > 0 && d % 64 == 0, "grouped_ffn: d must be a positive multiple of 64, got %d", d);
  NT_REQUIRE(H > 0 && H % 64 == 0, "grouped_ffn: H must be a positive multiple of 64, got %d", H);
  NT_REQUIRE(num_segments >= 1 && num_segments <= NT_MOE_MAX_SEGMENTS,
             "grouped_ffn: num_segments must be in [1, %d]", NT_MOE_MAX_SEGMENTS);
  NT_REQUIRE(total_rows >= 0 && total_rows < ((int64_t)1 << 31), "grouped_ffn: bad total_rows");
  NT_REQUIRE(activation == NT_MOE_ACT_SWIGLU || activation == NT_MOE_ACT_RELU2,
             "grouped_ffn: unknown activation %d", activation);
  NT_REQUIRE(ld_a >= d && ld_a % 8 == 0, "grouped_ffn: ld_a must be >= d and a multiple of 8");
  NT_REQUIRE(a_rows >= 1, "grouped_ffn: a_rows must be positive");
  NT_REQUIRE(src_row || a_rows >= total_rows, "grouped_ffn: a needs total_rows rows without src_row");
  NT_REQUIRE(a && seg_offsets && w1 && w2 && h && y, "grouped_ffn: null buffer");
  NT_REQUIRE(aligned16(a) && aligned16(w1) && aligned16(w2) && aligned16(h) && aligned16(y),
             "grouped_ffn: buffers must be 16-byte aligned");
  int rc = check_gemm_extent(a_rows, ld_a, (int64_t)2 * H, d);
  if (rc) return rc;
  rc = check_gemm_extent(total_rows, H, d, H);
  if (rc) return rc;
  if (!workspace || workspace_bytes < kGemmWorkspaceBytes)
    return fail(NT_MOE_ENOSPC, "grouped_ffn: workspace %zu < %zu bytes", workspace_bytes,
                kGemmWorkspaceBytes);
  if (total_rows == 0) return ok();
  hipError_t err = launch_grouped_ffn_bf16(a, ld_a, a_rows, src_row, seg_offsets, num_segments,
                                           total_rows, w1, w2, d, H, activation, h, y,
                                           reinterpret_cast<int*>(workspace),
                                           reinterpret_cast<hipStream_t>(stream));
  return launched(err, "grouped_ffn_bf16");
}

static int check_plain(const uint16_t* a, int64_t ld_a, int64_t a_rows, const int32_t* src_row,
                       const int32_t* seg_offsets, int32_t num_segments, int64_t total_rows,
                       const uint16_t* w, int32_t K, int32_t n_out, int32_t epilogue,
                       uint16_t* c) {
  NT_REQUIRE(K > 0 && K % 64 == 0, "grouped_gemm: K must be a positive multiple of 64, got %d", K);
  NT_REQUIRE(epilogue == NT_MOE_EPI_SWIGLU || epilogue == NT_MOE_EPI_RELU2 ||
                 epilogue == NT_MOE_EPI_NONE, "grouped_gemm: unknown epilogue %d", epilogue);
  NT_REQUIRE(n_out > 0 && n_out % (epilogue == NT_MOE_EPI_SWIGLU ? 64 : 4) == 0,
             "grouped_gemm: n_out must be a positive multiple of %d, got %d",
             epilogue == NT_MOE_EPI_SWIGLU ? 64 : 4, n_out);
  NT_REQUIRE(num_segments >= 1 && num_segments <= NT_MOE_MAX_SEGMENTS,
             "grouped_gemm: num_segments must be in [1, %d]", NT_MOE_MAX_SEGMENTS);
  NT_REQUIRE(total_rows >= 0 && total_rows < ((int64_t)1 << 31), "grouped_gemm: bad total_rows");
  NT_REQUIRE(ld_a >= K && ld_a % 8 == 0, "grouped_gemm: ld_a must be >= K and a multiple of 8");
  NT_REQUIRE(a_rows >= 1, "grouped_gemm: a_rows must be positive");
  NT_REQUIRE(src_row || a_rows >= total_rows, "grouped_gemm: a needs total_rows rows without src_row");
  NT_REQUIRE(a && seg_offsets && w && c, "grouped_gemm: null buffer");
  NT_REQUIRE(aligned16(a) && aligned16(w) && aligned16(c), "grouped_gemm: buffers must be 16-byte aligned");
  int rc = check_gemm_extent(a_rows, ld_a,
                             epilogue == NT_MOE_EPI_SWIGLU ? (int64_t)2 * n_out : n_out, K);
  if (rc) return rc;
  NT_REQUIRE(total_rows * n_out * 2 < ((int64_t)1 << 31),
             "grouped_gemm: the output must stay below 2 GiB");
  return 0;
}

int nt_moe_grouped_gemm_bf16(const uint16_t* a, int64_t ld_a, int64_t a_rows,
                             const int32_t* src_row, const int32_t* seg_offsets,
                             int32_t num_segments, int64_t total_rows, const uint16_t* w,
                             int32_t K, int32_t n_out, int32_t epilogue, uint16_t* c,
                             void* workspace, size_t workspace_bytes, nt_moe_stream_t stream) {
  int rc = check_plain(a, ld_a, a_rows, src_row, seg_offsets, num_segments, total_rows, w, K,
                       n_out, epilogue, c);
  if (rc) return rc;
  if (!workspace || workspace_bytes < kGemmWorkspaceBytes)
    return fail(NT_MOE_ENOSPC, "grouped_gemm: workspace %zu < %zu bytes", workspace_bytes,
                kGemmWorkspaceBytes);
  if (total_rows == 0) return ok();
  // 256 x 256 tiles with both operands staged through LDS when K spans two steps of 64 and
  // output rows are whole 16-byte stores; otherwise the 2 x 4-wave macro-tile kernel
  hipError_t err =
      K >= 128 && n_out % 8 == 0
          ? launch_grouped_gemm_bf16_t256(a, ld_a, a_rows, src_row, seg_offsets, num_segments,
                                          total_rows, w, K, n_out, epilogue, c,
                                          reinterpret_cast<hipStream_t>(stream))
          : launch_grouped_gemm_bf16(a, ld_a, a_rows, src_row, seg_offsets, num_segments,
                                     total_rows, w, K, n_out, epilogue, c,
                                     reinterpret_cast<int*>(workspace),
                                     reinterpret_cast<hipStream_t>(stream));
  return launched(err, "grouped_gemm_bf16");
}

int nt_moe_grouped_gemm_bf16_keep(const uint16_t* a, int64_t ld_a, int64_t a_rows,
                                  const int32_t* src_row, const int32_t* seg_offsets,
                                  int32_t num_segments, int64_t total_rows, const uint16_t* w,
                                  int32_t K, int32_t n_out, int32_t epilogue, uint16_t* c,
                                  uint16_t* pre, nt_moe_stream_t stream) {
  NT_REQUIRE(epilogue == NT_MOE_EPI_SWIGLU || epilogue == NT_MOE_EPI_RELU2,
             "grouped_gemm_keep: the epilogue must be SWIGLU or RELU2, got %d", epilogue);
  int rc = check_plain(a, ld_a, a_rows, src_row, seg_offsets, num_segments, total_rows, w, K,
                       n_out, epilogue, c);
  if (rc) return rc;
  NT_REQUIRE(K >= 128 && n_out % 8 == 0,
             "grouped_gemm_keep: K must be >= 128 and n_out a multiple of 8, got K %d n_out %d",
             K, n_out);
  const int64_t pw = epilogue == NT_MOE_EPI_SWIGLU ? 2 * (int64_t)n_out : n_out;
  NT_REQUIRE(total_rows * pw * 2 < ((int64_t)1 << 31),
             "grouped_gemm_keep: the pre-activations must stay below 2 GiB");
  NT_REQUIRE(pre && aligned16(pre), "grouped_gemm_keep: pre must be a 16-byte aligned buffer");
  if (total_rows == 0) return ok();
  return launched(launch_grouped_gemm_bf16_t256_keep(a, ld_a, a_rows, src_row, seg_offsets,
                                                     num_segments, total_rows, w, K, n_out,
                                                     epilogue, c, pre,
                                                     reinterpret_cast<hipStream_t>(stream)),
                  "grouped_gemm_keep");
}

int nt_moe_convert_expert_weights(const float* w, int64_t num_matrices, int32_t rows,
                                  int32_t cols, uint16_t* out, uint16_t* out_t,
                                  nt_moe_stream_t stream) {
  NT_REQUIRE(num_matrices >= 0 && rows > 0 && rows % 64 == 0 && cols > 0 && cols % 64 == 0,
             "convert_expert_weights: rows and cols must be positive multiples of 64, got %d x %d",
             rows, cols);
  if (num_matrices == 0 || (!out && !out_t)) return ok();
  NT_REQUIRE(w && aligned16(w) && (!out || aligned16(out)) && (!out_t || aligned16(out_t)),
             "convert_expert_weights: null or unaligned buffer");
  return launched(launch_convert_weights(w, num_matrices, rows, cols, out, out_t,
                                         reinterpret_cast<hipStream_t>(stream)),
                  "convert_expert_weights");
}

int nt_moe_convert_expert_weights_packed(const float* w, int64_t num_matrices, int32_t rows,
                                         int32_t cols, uint16_t* out, uint16_t* out_t,
                                         uint16_t* packed, int32_t epilogue, uint16_t* packed_t,
                                         nt_moe_stream_t stream) {
  NT_REQUIRE(num_matrices >= 0 && rows > 0 && rows % 64 == 0 && cols > 0 && cols % 64 == 0,
             "convert_expert_weights_packed: rows and cols must be positive multiples of 64, "
             "got %d x %d", rows, cols);
  NT_REQUIRE(epilogue == NT_MOE_EPI_SWIGLU || epilogue == NT_MOE_EPI_RELU2 ||
                 epilogue == NT_MOE_EPI_NONE,
             "convert_expert_weights_packed: unknown epilogue %d", epilogue);
  if (num_matrices == 0 || (!out && !out_t && !packed && !packed_t)) return ok();
  NT_REQUIRE(w && aligned16(w) && (!out || aligned16(out)) && (!out_t || aligned16(out_t)) &&
                 (!packed || aligned16(packed)) && (!packed_t || aligned16(packed_t)),
             "convert_expert_weights_packed: null or unaligned buffer");
  return launched(launch_convert_weights(w, num_matrices, rows, cols, out, out_t,
                                         reinterpret_cast<hipStream_t>(stream), packed,
                                         epilogue == NT_MOE_EPI_SWIGLU ? rows / 2 : 0, packed_t),
                  "convert_expert_weights_packed");
}

int nt_moe_router_operands(const float* w, int64_t ld_w, int32_t num_experts, int32_t d,
                           int32_t dp, const uint16_t* shared_w1, int64_t ld_s, int32_t Fs,
                           float* w_router_t, uint16_t* first, int32_t Ep, int32_t Kc,
                           nt_moe_stream_t stream) {
  NT_REQUIRE(num_experts > 0 && d > 0 && dp >= d && ld_w >= d,
             "router_operands: need num_experts > 0, 0 < d <= dp and ld_w >= d, got E=%d d=%d "
             "dp=%d ld_w=%lld", num_experts, d, dp, (long long)ld_w);
  NT_REQUIRE(w && w_router_t, "router_operands: null weight or w_router_t");
  if (first) {
    NT_REQUIRE(Ep >= num_experts && Fs >= 0 && (int64_t)Kc >= (int64_t)Fs + 3 * (int64_t)Ep &&
                   (int64_t)dp * Kc < (int64_t)1 << 31,
               "router_operands: need Ep >= E, Fs >= 0 and Fs + 3 Ep <= Kc, got E=%d Ep=%d "
               "Fs=%d Kc=%d", num_experts, Ep, Fs, Kc);
    NT_REQUIRE(Fs == 0 || (shared_w1 && ld_s >= dp),
               "router_operands: Fs > 0 needs shared_w1 with row stride >= dp");
  }
  return launched(launch_router_operands(w, ld_w, num_experts, d, dp, shared_w1, ld_s,
                                         first ? Fs : 0, w_router_t, first, first ? Ep : num_experts,
                                         first ? Kc : 0, reinterpret_cast<hipStream_t>(stream)),
                  "router_operands");
}

int nt_moe_pack_expert_weights_bf16(const uint16_t* w, int64_t num_segments, int32_t rows,
                                    int32_t K, int32_t epilogue, uint16_t* packed,
                                    nt_moe_stream_t stream) {
  NT_REQUIRE(epilogue == NT_MOE_EPI_SWIGLU || epilogue == NT_MOE_EPI_RELU2 ||
                 epilogue == NT_MOE_EPI_NONE, "pack_expert_weights: unknown epilogue %d", epilogue);
  NT_REQUIRE(num_segments >= 0 && rows > 0 && rows % 32 == 0 && K > 0 && K % 64 == 0,
             "pack_expert_weights: rows must be a multiple of 32 and K of 64, got %d x %d", rows, K);
  NT_REQUIRE(epilogue != NT_MOE_EPI_SWIGLU || rows % 64 == 0,
             "pack_expert_weights: SwiGLU rows (2 n_out) must be a multiple of 64");
  if (num_segments == 0) return ok();
  NT_REQUIRE(w && packed && aligned16(w) && aligned16(packed),
             "pack_expert_weights: null or unaligned buffer");
  hipError_t err = launch_pack_weights_bf16(w, num_segments, rows, K, epilogue, packed,
                                            reinterpret_cast<hipStream_t>(stream));
  return launched(err, "pack_expert_weights_bf16");
}

static int check_packed(const uint16_t* a, int64_t ld_a, int64_t a_rows, const int32_t* src_row,
                        const int32_t* seg_offsets, int32_t num_segments, int64_t total_rows,
                        const uint16_t* w_packed, int32_t K, int32_t n_out, int32_t epilogue,
                        uint16_t* c) {
  NT_REQUIRE(K >= packed_gemm_min_k() && K % 64 == 0,
             "grouped_gemm_packed: K must be a multiple of 64 and >= %d, got %d",
             packed_gemm_min_k(), K);
  NT_REQUIRE(epilogue == NT_MOE_EPI_SWIGLU || epilogue == NT_MOE_EPI_RELU2 ||
                 epilogue == NT_MOE_EPI_NONE, "grouped_gemm_packed: unknown epilogue %d", epilogue);
  NT_REQUIRE(n_out > 0 && n_out % (epilogue == NT_MOE_EPI_SWIGLU ? 16 : 32) == 0,
             "grouped_gemm_packed: n_out must be a positive multiple of %d, got %d",
             epilogue == NT_MOE_EPI_SWIGLU ? 16 : 32, n_out);
  NT_REQUIRE(num_segments >= 1 && num_segments <= NT_MOE_MAX_SEGMENTS,
             "grouped_gemm_packed: num_segments must be in [1, %d]", NT_MOE_MAX_SEGMENTS);
  NT_REQUIRE(total_rows >= 0 && total_rows * n_out * 2 < ((int64_t)1 << 31),
             "grouped_gemm_packed: the output must stay below 2 GiB");
  NT_REQUIRE(ld_a >= K && ld_a % 8 == 0, "grouped_gemm_packed: ld_a must be >= K and a multiple of 8");
  NT_REQUIRE(a_rows >= 1, "grouped_gemm_packed: a_rows must be positive");
  NT_REQUIRE(src_row || a_rows >= total_rows,
             "grouped_gemm_packed: a needs total_rows rows without src_row");
  NT_REQUIRE(a && seg_offsets && w_packed && c, "grouped_gemm_packed: null buffer");
  NT_REQUIRE(aligned16(a) && aligned16(w_packed) && aligned16(c),
             "grouped_gemm_packed: a, w_packed and c must be 16-byte aligned");
  int rc = check_gemm_extent(a_rows, ld_a, 0, 0);
  if (rc) return rc;
  return 0;
}

int nt_moe_grouped_gemm_bf16_packed(const uint16_t* a, int64_t ld_a, int64_t a_rows,
                                    const int32_t* src_row, const int32_t* seg_offsets,
                                    int32_t num_segments, int64_t total_rows,
                                    const uint16_t* w_packed, int32_t K, int32_t n_out,
                                    int32_t epilogue, uint16_t* c, nt_moe_stream_t stream) {
  int rc = check_packed(a, ld_a, a_rows, src_row, seg_offsets, num_segments, total_rows,
                        w_packed, K, n_out, epilogue, c);
  if (rc) return rc;
  if (total_rows == 0) return ok();
  hipError_t err = launch_grouped_gemm_bf16_packed(a, ld_a, a_rows, src_row, seg_offsets,
                                                   num_segments, total_rows, w_packed, K, n_out,
                                                   epilogue, c,
                                                   reinterpret_cast<hipStream_t>(stream));
  return launched(err, "grouped_gemm_bf16_packed");
}

int nt_moe_grouped_gemm_bf16_packed_keep(const uint16_t* a, int64_t ld_a, int64_t a_rows,
                                         const int32_t* src_row, const int32_t* seg_offsets,
                                         int32_t num_segments, int64_t total_rows,
                                         const uint16_t* w_packed, int32_t K, int32_t n_out,
                                         int32_t epilogue, uint16_t* c, uint16_t* pre,
                                         nt_moe_stream_t stream) {
  NT_REQUIRE(epilogue == NT_MOE_EPI_SWIGLU || epilogue == NT_MOE_EPI_RELU2,
             "grouped_gemm_packed_keep: the epilogue must be SWIGLU or RELU2, got %d", epilogue);
  int rc = check_packed(a, ld_a, a_rows, src_row, seg_offsets, num_segments, total_rows,
                        w_packed, K, n_out, epilogue, c);
  if (rc) return rc;
  const int64_t pw = epilogue == NT_MOE_EPI_SWIGLU ? 2 * (int64_t)n_out : n_out;
  NT_REQUIRE(total_rows * pw * 2 < ((int64_t)1 << 31),
             "grouped_gemm_packed_keep: the pre-activations must stay below 2 GiB");
  NT_REQUIRE(pre && aligned16(pre), "grouped_gemm_packed_keep: pre must be a 16-byte aligned buffer");
  if (total_rows == 0) return ok();
  return launched(launch_grouped_gemm_bf16_packed_keep(a, ld_a, a_rows, src_row, seg_offsets,
                                                       num_segments, total_rows, w_packed, K,
                                                       n_out, epilogue, c, pre,
                                                       reinterpret_cast<hipStream_t>(stream)),
                  "grouped_gemm_packed_keep");
}

int nt_moe_quantize_fp8_rowwise(const uint16_t* x, int64_t ld_x, int64_t rows, int32_t d,
                                uint8_t* q, int64_t ld_q, float* scale, nt_moe_stream_t stream) {
  NT_REQUIRE(rows >= 0 && rows < ((int64_t)1 << 31), "quantize_fp8_rowwise: bad row count");
  NT_REQUIRE(d > 0 && d % 8 == 0, "quantize_fp8_rowwise: d must be a positive multiple of 8, got %d", d);
  NT_REQUIRE(ld_x >= d && ld_x % 8 == 0 && ld_q >= d && ld_q % 8 == 0,
             "quantize_fp8_rowwise: ld_x and ld_q must be >= d and multiples of 8");
  if (rows == 0) return ok();
  NT_REQUIRE(x && q && scale, "quantize_fp8_rowwise: null buffer");
  NT_REQUIRE(aligned16(x) && aligned_to(q, 8), "quantize_fp8_rowwise: x must be 16-byte and q 8-byte aligned");
  hipError_t err = launch_quantize_fp8_rowwise(x, ld_x, rows, d, q, ld_q, scale,
                                               reinterpret_cast<hipStream_t>(stream));
  return launched(err, "quantize_fp8_rowwise");
}

int nt_moe_quantize_fp8_blockwise(const float* w, int64_t num_matrices, int32_t rows,
                                  int32_t cols, uint8_t* q, float* scale, nt_moe_stream_t stream) {
  NT_REQUIRE(num_matrices >= 0, "quantize_fp8_blockwise: negative matrix count");
  NT_REQUIRE(rows > 0 && rows % 128 == 0 && cols > 0 && cols % 128 == 0,
             "quantize_fp8_blockwise: rows and cols must be positive multiples of 128, got %d x %d",
             rows, cols);
  NT_REQUIRE(num_matrices * (rows / 128) * (cols / 128) < ((int64_t)1 << 31),
             "quantize_fp8_blockwise: too many blocks");
  if (num_matrices == 0) return ok();
  NT_REQUIRE(w && q && scale, "quantize_fp8_blockwise: null buffer");
  NT_REQUIRE(aligned16(w) && aligned_to(q, 4), "quantize_fp8_blockwise: w must be 16-byte and q 4-byte aligned");
  hipError_t err = launch_quantize_fp8_blockwise(w, num_matrices, rows, cols, q, scale,
                                                 reinterpret_cast<hipStream_t>(stream));
  return launched(err, "quantize_fp8_blockwise");
}

int nt_moe_grouped_gemm_fp8(const uint8_t* a, int64_t ld_a, int64_t a_rows, const float* a_scale,
                            const int32_t* src_row, const int32_t* seg_offsets,
                            int32_t num_segments, int64_t total_rows, const uint8_t* w,
                            const float* w_scale, int32_t K, int32_t n_out, int32_t epilogue,
                            uint16_t* c, nt_moe_stream_t stream) {
  NT_REQUIRE(K > 0 && K % 128 == 0, "grouped_gemm_fp8: K must be a positive multiple of 128, got %d", K);
  NT_REQUIRE(epilogue == NT_MOE_EPI_SWIGLU || epilogue == NT_MOE_EPI_RELU2 ||
                 epilogue == NT_MOE_EPI_NONE, "grouped_gemm_fp8: unknown epilogue %d", epilogue);
  NT_REQUIRE(n_out > 0 && n_out % (epilogue == NT_MOE_EPI_SWIGLU ? 64 : 128) == 0,
             "grouped_gemm_fp8: n_out must be a positive multiple of %d, got %d",
             epilogue == NT_MOE_EPI_SWIGLU ? 64 : 128, n_out);
  NT_REQUIRE(num_segments >= 1 && num_segments <= NT_MOE_MAX_SEGMENTS,
             "grouped_gemm_fp8: num_segments must be in [1, %d]", NT_MOE_MAX_SEGMENTS);
  NT_REQUIRE(total_rows >= 0 && total_rows < ((int64_t)1 << 31), "grouped_gemm_fp8: bad total_rows");
  NT_REQUIRE(ld_a >= K && ld_a % 32 == 0, "grouped_gemm_fp8: ld_a must be >= K and a multiple of 32");
  NT_REQUIRE(a_rows >= 1, "grouped_gemm_fp8: a_rows must be positive");
  NT_REQUIRE(src_row || a_rows >= total_rows, "grouped_gemm_fp8: a needs total_rows rows without src_row");
  NT_REQUIRE(a && a_scale && seg_offsets && w && w_scale && c, "grouped_gemm_fp8: null buffer");
  NT_REQUIRE(aligned_to(a, 32) && aligned_to(w, 32) && aligned_to(c, 8),
             "grouped_gemm_fp8: a and w must be 32-byte aligned, c 8-byte aligned");
  if (total_rows == 0) return ok();
  hipError_t err = launch_grouped_gemm_fp8(a, ld_a, a_rows, a_scale, src_row, seg_offsets,
                                           num_segments, total_rows, w, w_scale, K, n_out,
                                           epilogue, false, c,
                                           reinterpret_cast<hipStream_t>(stream));
  return launched(err, "grouped_gemm_fp8");
}

int nt_moe_pack_expert_weights_fp8(const uint8_t* w, int64_t num_segments, int32_t rows,
                                   int32_t K, int32_t epilogue, uint8_t* packed,
                                   nt_moe_stream_t stream) {
  NT_REQUIRE(epilogue == NT_MOE_EPI_SWIGLU || epilogue == NT_MOE_EPI_RELU2 ||
                 epilogue == NT_MOE_EPI_NONE, "pack_expert_weights_fp8: unknown epilogue %d", epilogue);
  NT_REQUIRE(num_segments >= 0 && rows > 0 && rows % 128 == 0 && K > 0 && K % 128 == 0,
             "pack_expert_weights_fp8: rows and K must be multiples of 128, got %d x %d", rows, K);
  if (num_segments == 0) return ok();
  NT_REQUIRE(w && packed && aligned16(w) && aligned16(packed),
             "pack_expert_weights_fp8: null or unaligned buffer");
  hipError_t err = launch_pack_weights_fp8(w, num_segments, rows, K, epilogue, packed,
                                           reinterpret_cast<hipStream_t>(stream));
  return launched(err, "pack_expert_weights_fp8");
}

int nt_moe_grouped_gemm_fp8_packed(const uint8_t* a, int64_t ld_a, int64_t a_rows,
                                   const float* a_scale, const int32_t* src_row,
                                   const int32_t* seg_offsets, int32_t num_segments,
                                   int64_t total_rows, const uint8_t* w_packed,
                                   const float* w_scale, int32_t K, int32_t n_out,
                                   int32_t epilogue, uint16_t* c, nt_moe_stream_t stream) {
  NT_REQUIRE(K > 0 && K % 128 == 0, "grouped_gemm_fp8_packed: K must be a positive multiple of 128, got %d", K);
  NT_REQUIRE(epilogue == NT_MOE_EPI_SWIGLU || epilogue == NT_MOE_EPI_RELU2 ||
                 epilogue == NT_MOE_EPI_NONE, "grouped_gemm_fp8_packed: unknown epilogue %d", epilogue);
  NT_REQUIRE(n_out > 0 && n_out % (epilogue == NT_MOE_EPI_SWIGLU ? 64 : 128) == 0,
             "grouped_gemm_fp8_packed: n_out must be a positive multiple of %d, got %d",
             epilogue == NT_MOE_EPI_SWIGLU ? 64 : 128, n_out);
  NT_REQUIRE(num_segments >= 1 && num_segments <= NT_MOE_MAX_SEGMENTS,
             "grouped_gemm_fp8_packed: num_segments must be in [1, %d]", NT_MOE_MAX_SEGMENTS);
  NT_REQUIRE(total_rows >= 0 && total_rows < ((int64_t)1 << 31), "grouped_gemm_fp8_packed: bad total_rows");
  NT_REQUIRE(ld_a >= K && ld_a % 32 == 0, "grouped_gemm_fp8_packed: ld_a must be >= K and a multiple of 32");
  NT_REQUIRE(a_rows >= 1, "grouped_gemm_fp8_packed: a_rows must be positive");
  NT_REQUIRE(src_row || a_rows >= total_rows,
             "grouped_gemm_fp8_packed: a needs total_rows rows without src_row");
  NT_REQUIRE(a && a_scale && seg_offsets && w_packed && w_scale && c,
             "grouped_gemm_fp8_packed: null buffer");
  NT_REQUIRE(aligned_to(a, 32) && aligned16(w_packed) && aligned_to(c, 8),
             "grouped_gemm_fp8_packed: a 32-byte, w_packed 16-byte and c 8-byte aligned");
  if (total_rows == 0) return ok();
  hipError_t err = launch_grouped_gemm_fp8(a, ld_a, a_rows, a_scale, src_row, seg_offsets,
                                           num_segments, total_rows, w_packed, w_scale, K, n_out,
                                           epilogue, true, c,
                                           reinterpret_cast<hipStream_t>(stream));
  return launched(err, "grouped_gemm_fp8_packed");
}

int nt_moe_combine_aux(const uint16_t* y, const int32_t* combine_dest, const float* combine_w,
                       int64_t T, int32_t d, int32_t k, const uint16_t* shared_y,
                       int64_t ld_shared, uint16_t* out, int64_t ld_out,
                       const float* prob_partial, const float* z_partial,
                       const int32_t* counts, int32_t E, float aux_coeff, float z_coeff,
                       float* aux_out, nt_moe_stream_t stream) {
  int rc = check_route_shape(T, k, E);
  if (rc) return rc;
  NT_REQUIRE(d > 0 && d % 8 == 0, "combine: d must be a positive multiple of 8, got %d", d);
  NT_REQUIRE(ld_out >= d && ld_out % 8 == 0, "combine: ld_out must be >= d and a multiple of 8");
  NT_REQUIRE(!shared_y || (ld_shared >= d && ld_shared % 8 == 0 && aligned16(shared_y)),
             "combine: shared_y needs ld_shared >= d, a multiple of 8, 16-byte alignment");
  if (T > 0) {
    NT_REQUIRE(y && combine_dest && combine_w && out, "combine: null buffer");
    NT_REQUIRE(aligned16(y) && aligned16(out), "combine: y and out must be 16-byte aligned");
  }
  if (aux_out) NT_REQUIRE(counts && (T == 0 || (prob_partial && z_partial)), "combine: null aux input");
  hipError_t err = launch_combine_aux(y, combine_dest, combine_w, T, d, k, shared_y, ld_shared,
                                      out, ld_out, prob_partial, z_partial, counts, E, aux_coeff,
                                      z_coeff, aux_out, reinterpret_cast<hipStream_t>(stream));
  return launched(err, "combine_aux");
}

}  // extern "C"
