// Router: fp32 gating GEMM in a fixed reduction order, softmax / sigmoid scoring and
// a wavefront-shuffle top-k, with per-block auxiliary-loss partials.
//
// Replaces NativeRouter.gating -> F.linear(x.float(), W.float())
// (nexttransformer/scaling/megatron_moe.py:95-99) and TopKRouter's top-k followed by softmax
// over the selected logits (megatron_moe.py:43; reference_blocks.py:37-38).
//
// Fixed order (bit-exact contract shared with oracle/router_ref.c):
//   c_j   = fma chain over features [128 j, 128 j + 128) in ascending order, from 0.0f
//   logit = ((c_0 + c_1) + c_2) + ...   then  + bias[e]
// Ties in top-k: equal logits rank the lower expert index first.
//
// Work mapping. A block of 256 threads (4 waves) owns 64 tokens; lane = token. Wave w owns a
// window of EPW consecutive experts, so its router weights are wave-uniform and come in
// through scalar loads (w_router_t is [d, E], E contiguous); each lane keeps EPW fp32
// accumulators. x is staged through LDS one 128-feature chunk at a time (coalesced global
// loads, padded rows so per-lane row reads are conflict-free).
// Unless T is very large the fused grid has too few waves per CU: the split variant gives every
// (token block, chunk, expert group) its own block and writes the chunk sums c_j to a
// workspace (expert-major planes); a plane-sum kernel adds them in ascending j -- the same
// order -- and a top-k kernel ranks.
//
// Top-k: logits go to an LDS tile [64][E+1]; LPT lanes share a token (4 in the fused kernel,
// 16 in the top-k kernel), each scans every LPT-th expert into a sorted register list, then k
// rounds of an xor-shuffle butterfly over the LPT lanes emit the global order.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "common.h"

namespace ntmoe {
namespace {

constexpr int kXStride = kRouterChunk + 8;  // bf16 per padded LDS row (272 bytes)
constexpr int kXTileBytes = kRouteBlock * kXStride * 2;

__host__ __device__ inline int lg_tile_bytes(int E) { return kRouteBlock * (E + 1) * 4; }
__host__ __device__ inline int zt_offset(int E) {
  int lg = lg_tile_bytes(E);
  return lg > kXTileBytes ? lg : kXTileBytes;
}
inline size_t router_lds_bytes(int E) { return zt_offset(E) + kRouteBlock * sizeof(float); }

// acc[e] = fma chain over the clen features of the staged chunk (row of this lane's token).
template <int EPW>
__device__ __forceinline__ void chunk_fma(const uint16_t* xs_row, const float* __restrict__ wt,
                                          int E, int ws, int c0, int clen, float* acc) {
  for (int kk = 0; kk < clen; kk += 8) {
    u32x4 raw = *reinterpret_cast<const u32x4*>(xs_row + kk);
    float xf[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      xf[2 * i] = __builtin_bit_cast(float, raw[i] << 16);
      xf[2 * i + 1] = __builtin_bit_cast(float, raw[i] & 0xffff0000u);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float* wrow = wt + (size_t)(c0 + kk + i) * E + ws;
#pragma unroll
      for (int e = 0; e < EPW; ++e) acc[e] = __builtin_fmaf(xf[i], wrow[e], acc[e]);
    }
  }
}

// Stage x[t0 .. t0+63][c0 .. c0+clen) into LDS (zeros beyond T).
__device__ __forceinline__ void stage_x(const uint16_t* __restrict__ x, int64_t ld_x, int64_t T,
                                        int64_t t0, int c0, int clen, uint16_t* xs) {
  const int groups = clen >> 3;  // 16-byte groups per row
  for (int g = threadIdx.x; g < kRouteBlock * 16; g += blockDim.x) {
    int row = g >> 4, col = g & 15;
    if (col >= groups) continue;
    u32x4 v = {0u, 0u, 0u, 0u};
    int64_t t = t0 + row;
    if (t < T) v = *reinterpret_cast<const u32x4*>(x + t * ld_x + c0 + col * 8);
    *reinterpret_cast<u32x4*>(xs + row * kXStride + col * 8) = v;
  }
}

template <int KMAX>
__device__ __forceinline__ void list_insert(float v, int e, float* lv, int* li) {
  if (!rank_before(v, e, lv[KMAX - 1], li[KMAX - 1])) return;
  lv[KMAX - 1] = v;
  li[KMAX - 1] = e;
#pragma unroll
  for (int j = KMAX - 1; j > 0; --j) {
    if (rank_before(lv[j], li[j], lv[j - 1], li[j - 1])) {
      float tv = lv[j]; lv[j] = lv[j - 1]; lv[j - 1] = tv;
      int ti = li[j]; li[j] = li[j - 1]; li[j - 1] = ti;
    }
  }
}

// Top-k, weights, full scores and aux partials for the 64 tokens whose logits sit in the
// LDS tile lg[64][E+1]; overwrites lg with the full scores s_te. Called by all 64 * LPT threads
// of the block: LPT lanes per token, each scanning every LPT-th expert.
template <int KMAX, int LPT = 4>
__device__ void topk_and_scores(float* lg, float* zt, int64_t t0, int64_t T, int E, int k,
                                int score_fn, int32_t* __restrict__ topk_ids,
                                float* __restrict__ topk_w, float* __restrict__ prob_partial,
                                float* __restrict__ z_partial) {
  static_assert(LPT == 4 || LPT == 8 || LPT == 16, "lanes per token");
  const int ldl = E + 1;
  const int tt = threadIdx.x / LPT;   // token within the block
  const int sub = threadIdx.x % LPT;  // which of the LPT expert strides this lane scans
  const int64_t t = t0 + tt;
  float* row = lg + tt * ldl;

  float lv[KMAX];
  int li[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) { lv[j] = -INFINITY; li[j] = 0x7fffffff; }
  for (int e = sub; e < E; e += LPT) list_insert<KMAX>(row[e], e, lv, li);

  // k rounds: best head of the LPT lists (xor butterfly), the owner pops it.
  float ov[KMAX];
  int oi[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    float bv = lv[0];
    int bi = li[0];
#pragma unroll
    for (int m = 1; m < LPT; m <<= 1) {
      float v2 = __shfl_xor(bv, m);
      int i2 = __shfl_xor(bi, m);
      if (rank_before(v2, i2, bv, bi)) { bv = v2; bi = i2; }
    }
    ov[j] = bv;
    oi[j] = bi;
    if (li[0] == bi) {
#pragma unroll
      for (int q = 0; q < KMAX - 1; ++q) { lv[q] = lv[q + 1]; li[q] = li[q + 1]; }
      lv[KMAX - 1] = -INFINITY;
      li[KMAX - 1] = 0x7fffffff;
    }
  }

  // Routing weights over the k selected: softmax, or sigmoid normalised over the selected.
  const float top = ov[0];
  float wsum = 0.f, wv[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    float s = score_fn == NT_MOE_SCORE_SOFTMAX ? expf(ov[j] - top) : 1.f / (1.f + expf(-ov[j]));
    wv[j] = j < k ? s : 0.f;
    wsum += wv[j];
  }
  const float winv = 1.f / wsum;
  if (t < T) {
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      if (j < k && j % LPT == sub) {
        topk_ids[t * k + j] = oi[j];
        topk_w[t * k + j] = wv[j] * winv;
      }
    }
  }

  // Full scores s_te for the load-balance loss, logsumexp for the z-loss.
  float part = 0.f, spart = 0.f;
  for (int e = sub; e < E; e += LPT) {
    part += expf(row[e] - top);
    if (score_fn == NT_MOE_SCORE_SIGMOID) spart += 1.f / (1.f + expf(-row[e]));
  }
#pragma unroll
  for (int m = 1; m < LPT; m <<= 1) {
    part += __shfl_xor(part, m);
    spart += __shfl_xor(spart, m);
  }
  const float lse = top + logf(part);
  if (score_fn == NT_MOE_SCORE_SOFTMAX) {
    const float inv = 1.f / part;
    for (int e = sub; e < E; e += LPT) row[e] = expf(row[e] - top) * inv;
  } else {
    const float inv = 1.f / spart;
    for (int e = sub; e < E; e += LPT) row[e] = inv / (1.f + expf(-row[e]));
  }
  if (sub == 0) zt[tt] = lse * lse;
  __syncthreads();

  // Per-block column sums in a fixed order (deterministic): P consecutive lanes per expert,
  // lane p summing tokens p, p + P, ..., then a butterfly over the P lanes; P is the largest
  // power of two <= 64 with E P <= the block's threads. The z sum likewise over one wave.
  const int nvalid = (int)((T - t0) < kRouteBlock ? (T - t0) : kRouteBlock);
  const int64_t blk = t0 / kRouteBlock;
  int P = 64;
  while (P > 1 && E * P > (int)blockDim.x) P >>= 1;
  for (int base = 0; base < E * P; base += blockDim.x) {
    const int idx = base + threadIdx.x;
    const int e = idx / P, p = idx % P;
    float s = 0.f;
    if (e < E)
      for (int r = p; r < nvalid; r += P) s += lg[r * ldl + e];
    for (int m = P >> 1; m >= 1; m >>= 1) s += __shfl_xor(s, m);
    if (e < E && p == 0) prob_partial[blk * E + e] = s;
  }
  if (threadIdx.x < 64) {
    float s = threadIdx.x < nvalid ? zt[threadIdx.x] : 0.f;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m);
    if (threadIdx.x == 0) z_partial[blk] = s;
  }
}

__device__ __forceinline__ void write_logits_out(const float* lg, int64_t t0, int64_t T, int E,
                                                 float* __restrict__ logits) {
  for (int idx = threadIdx.x; idx < kRouteBlock * E; idx += blockDim.x) {
    int r = idx / E, e = idx - r * E;
    if (t0 + r < T) logits[(t0 + r) * E + e] = lg[r * (E + 1) + e];
  }
}

// Fused: all chunks and all experts for 64 tokens, then top-k in the same block.
template <int EPW, int KMAX>
__global__ __launch_bounds__(256) void router_fused_kernel(
    const uint16_t* __restrict__ x, int64_t ld_x, const float* __restrict__ wt,
    const float* __restrict__ bias, int64_t T, int d, int E, int k, int score_fn,
    float* __restrict__ logits, int32_t* __restrict__ topk_ids, float* __restrict__ topk_w,
    float* __restrict__ prob_partial, float* __restrict__ z_partial) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
  float* lg = reinterpret_cast<float*>(smem);
  float* zt = reinterpret_cast<float*>(smem + zt_offset(E));
  const int64_t t0 = (int64_t)blockIdx.x * kRouteBlock;
  const int lane = lane_id();
  const int e0 = wave_id() * EPW;
  const int ws = e0 < E - EPW ? e0 : E - EPW;  // window start kept inside [0, E)

  float total[EPW];
#pragma unroll
  for (int e = 0; e < EPW; ++e) total[e] = 0.f;
  for (int c0 = 0; c0 < d; c0 += kRouterChunk) {
    const int clen = d - c0 < kRouterChunk ? d - c0 : kRouterChunk;
    __syncthreads();
    stage_x(x, ld_x, T, t0, c0, clen, xs);
    __syncthreads();
    float acc[EPW];
#pragma unroll
    for (int e = 0; e < EPW; ++e) acc[e] = 0.f;
    chunk_fma<EPW>(xs + lane * kXStride, wt, E, ws, c0, clen, acc);
#pragma unroll
    for (int e = 0; e < EPW; ++e) total[e] = c0 == 0 ? acc[e] : total[e] + acc[e];
  }
  if (bias) {
#pragma unroll
    for (int e = 0; e < EPW; ++e) total[e] = total[e] + bias[ws + e];
  }
  __syncthreads();  // the x tile is dead; lg aliases it
#pragma unroll
  for (int i = 0; i < EPW; ++i) {
    int e = ws + i;
    if (e >= e0 && e < E) lg[lane * (E + 1) + e] = total[i];
  }
  __syncthreads();
  if (logits) write_logits_out(lg, t0, T, E, logits);
  topk_and_scores<KMAX>(lg, zt, t0, T, E, k, score_fn, topk_ids, topk_w, prob_partial,
                        z_partial);
}

// Split: one chunk of one expert group for 64 tokens -> partials[chunk][e][t]. Expert-major
// planes make every store of a wave 64 consecutive floats (token-major rows of E floats would
// scatter each store over 64 rows, which cost more than the FMAs).
template <int EPW>
__global__ __launch_bounds__(256) void router_partial_kernel(
    const uint16_t* __restrict__ x, int64_t ld_x, const float* __restrict__ wt, int64_t T, int d,
    int E, float* __restrict__ partials) {
  __shared__ __align__(16) uint16_t xs[kRouteBlock * kXStride];
  const int64_t t0 = (int64_t)blockIdx.x * kRouteBlock;
  const int c0 = blockIdx.y * kRouterChunk;
  const int clen = d - c0 < kRouterChunk ? d - c0 : kRouterChunk;
  const int lane = lane_id();
  const int e0 = (blockIdx.z * 4 + wave_id()) * EPW;
  const int ws = e0 < E - EPW ? e0 : E - EPW;
  stage_x(x, ld_x, T, t0, c0, clen, xs);
  __syncthreads();
  float acc[EPW];
#pragma unroll
  for (int e = 0; e < EPW; ++e) acc[e] = 0.f;
  chunk_fma<EPW>(xs + lane * kXStride, wt, E, ws, c0, clen, acc);
  const int64_t t = t0 + lane;
  if (t < T) {
    float* out = partials + (int64_t)blockIdx.y * E * T + t;
#pragma unroll
    for (int i = 0; i < EPW; ++i) {
      int e = ws + i;
      if (e >= e0 && e < E) out[(int64_t)e * T] = acc[i];
    }
  }
}

// Sums the nchunk partial planes ([e][t]) of the split router into plane 0, in place, in the
// fixed order ((p0 + p1) + p2) + ... then + bias[e]: four consecutive values per thread, the
// planes' loads issued together. This keeps the plane reduction off the top-k kernel, whose grid
// has one block per 64 tokens and so cannot hide the loads' latency when T is small.
__global__ __launch_bounds__(256) void router_sum_planes_kernel(float* __restrict__ partials,
                                                                 int nchunk,
                                                                 const float* __restrict__ bias,
                                                                 int64_t n4, int64_t T) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  const int64_t plane4 = n4;  // plane size in float4 units
  floatx4* p = reinterpret_cast<floatx4*>(partials) + i;
  floatx4 v = p[0];
  for (int c0 = 1; c0 < nchunk; c0 += 8) {
    floatx4 part[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (c0 + j < nchunk) part[j] = p[(int64_t)(c0 + j) * plane4];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (c0 + j < nchunk) {
        v[0] = v[0] + part[j][0];
        v[1] = v[1] + part[j][1];
        v[2] = v[2] + part[j][2];
        v[3] = v[3] + part[j][3];
      }
  }
  if (bias) {
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = v[j] + bias[(i * 4 + j) / T];
  }
  p[0] = v;
}

// Sum nchunk partial planes in ascending order (+ bias), then top-k. Element (t, e) of a plane
// sits at t + e T (expert-major, the split router's planes) or t E + e (token-major: caller-
// supplied logits, with nchunk = 1 and no bias); the tile loads walk the contiguous index.
template <int KMAX>
__global__ __launch_bounds__(1024) void router_topk_kernel(
    const float* __restrict__ partials, int nchunk, bool expert_major,
    const float* __restrict__ bias, int64_t T, int E, int k, int score_fn,
    float* __restrict__ logits, int32_t* __restrict__ topk_ids, float* __restrict__ topk_w,
    float* __restrict__ prob_partial, float* __restrict__ z_partial) {
  extern __shared__ __align__(16) unsigned char smem[];
  float* lg = reinterpret_cast<float*>(smem);
  float* zt = reinterpret_cast<float*>(smem + zt_offset(E));
  const int64_t t0 = (int64_t)blockIdx.x * kRouteBlock;
  // Chunk planes are summed in ascending order; loads go out 8 planes at a time so the sum is
  // not a chain of dependent memory round trips.
  const int64_t plane = T * E;
  // Tile index idx -> (token row r, expert e), contiguous in memory along idx.
  // (Plain selects, not assignments through references: the latter made the compiler keep r
  // and e in scratch memory with a dynamic index.)
  auto row_of = [&](int idx) { return expert_major ? idx % kRouteBlock : idx / E; };
  auto col_of = [&](int idx) { return expert_major ? idx / kRouteBlock : idx % E; };
  auto at = [&](int64_t t, int e) { return expert_major ? t + e * T : t * E + e; };
  if (nchunk == 1) {
    // One plane (the split router's planes are summed by router_sum_planes_kernel): eight loads
    // per thread go out together, so a block does not wait on one round trip per element.
    for (int base = threadIdx.x; base < kRouteBlock * E; base += 8 * blockDim.x) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int idx = base + j * blockDim.x;
        const int r = row_of(idx), e = col_of(idx);
        const int64_t t = t0 + r;
        v[j] = (idx < kRouteBlock * E && t < T) ? partials[at(t, e)] : 0.f;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int idx = base + j * blockDim.x;
        if (idx >= kRouteBlock * E) break;
        const int r = row_of(idx), e = col_of(idx);
        const int64_t t = t0 + r;
        float val = v[j];
        if (t < T) {
          if (bias) val = val + bias[e];
          if (logits) logits[t * E + e] = val;
        }
        lg[r * (E + 1) + e] = val;
      }
    }
  }
  for (int idx = nchunk == 1 ? kRouteBlock * E : threadIdx.x; idx < kRouteBlock * E;
       idx += blockDim.x) {
    const int r = row_of(idx), e = col_of(idx);
    int64_t t = t0 + r;
    float v = 0.f;
    if (t < T) {
      const float* p = partials + at(t, e);
      v = p[0];
      for (int c0 = 1; c0 < nchunk; c0 += 8) {
        float part[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) part[j] = c0 + j < nchunk ? p[(int64_t)(c0 + j) * plane] : 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (c0 + j < nchunk) v = v + part[j];
      }
      if (bias) v = v + bias[e];
      if (logits) logits[t * E + e] = v;
    }
    lg[r * (E + 1) + e] = v;
  }
  __syncthreads();
  topk_and_scores<KMAX, 16>(lg, zt, t0, T, E, k, score_fn, topk_ids, topk_w, prob_partial,
                        z_partial);
}

int experts_per_wave(int E) {
  int need = (E + 3) / 4, epw = 1;
  while (epw < need) epw <<= 1;
  return epw;
}

int kmax_for(int k) { return k <= 2 ? 2 : (k <= 4 ? 4 : 8); }

// NT_MOE_ROUTER_MODE=fused|split overrides the size heuristic (for tuning runs).
int router_mode_override() {
  static int mode = [] {
    const char* s = getenv("NT_MOE_ROUTER_MODE");
    if (!s) return 0;
    if (!strcmp(s, "fused")) return 1;
    if (!strcmp(s, "split")) return 2;
    return 0;
  }();
  return mode;
}

template <int KMAX>
hipError_t launch_topk_k(const float* partials, int nchunk, bool expert_major, const float* bias,
                         int64_t T, int E, int k, int score_fn, float* logits, int32_t* ids,
                         float* w, float* pp, float* zp, hipStream_t stream) {
  dim3 grid(ceil_div(T, kRouteBlock));
  hipError_t err = allow_dynamic_lds(reinterpret_cast<const void*>(router_topk_kernel<KMAX>),
                                     router_lds_bytes(E));
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL((router_topk_kernel<KMAX>), grid, dim3(1024), router_lds_bytes(E), stream,
                     partials, nchunk, expert_major, bias, T, E, k, score_fn, logits, ids, w, pp,
                     zp);
  return hipGetLastError();
}

hipError_t launch_topk_any(const float* partials, int nchunk, bool expert_major,
                           const float* bias, int64_t T, int E, int k, int score_fn,
                           float* logits, int32_t* ids, float* w, float* pp, float* zp,
                           hipStream_t stream) {
  switch (kmax_for(k)) {
    case 2: return launch_topk_k<2>(partials, nchunk, expert_major, bias, T, E, k, score_fn, logits, ids, w, pp, zp, stream);
    case 4: return launch_topk_k<4>(partials, nchunk, expert_major, bias, T, E, k, score_fn, logits, ids, w, pp, zp, stream);
    default: return launch_topk_k<8>(partials, nchunk, expert_major, bias, T, E, k, score_fn, logits, ids, w, pp, zp, stream);
  }
}

template <int EPW, int KMAX>
hipError_t launch_fused_k(const uint16_t* x, int64_t ld_x, const float* wt, const float* bias,
                          int64_t T, int d, int E, int k, int score_fn, float* logits,
                          int32_t* ids, float* w, float* pp, float* zp, hipStream_t stream) {
  dim3 grid(ceil_div(T, kRouteBlock));
  hipError_t err = allow_dynamic_lds(
      reinterpret_cast<const void*>(router_fused_kernel<EPW, KMAX>), router_lds_bytes(E));
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL((router_fused_kernel<EPW, KMAX>), grid, dim3(256), router_lds_bytes(E),
                     stream, x, ld_x, wt, bias, T, d, E, k, score_fn, logits, ids, w, pp, zp);
  return hipGetLastError();
}

template <int EPW>
hipError_t launch_fused_e(const uint16_t* x, int64_t ld_x, const float* wt, const float* bias,
                          int64_t T, int d, int E, int k, int score_fn, float* logits,
                          int32_t* ids, float* w, float* pp, float* zp, hipStream_t stream) {
  switch (kmax_for(k)) {
    case 2: return launch_fused_k<EPW, 2>(x, ld_x, wt, bias, T, d, E, k, score_fn, logits, ids, w, pp, zp, stream);
    case 4: return launch_fused_k<EPW, 4>(x, ld_x, wt, bias, T, d, E, k, score_fn, logits, ids, w, pp, zp, stream);
    default: return launch_fused_k<EPW, 8>(x, ld_x, wt, bias, T, d, E, k, score_fn, logits, ids, w, pp, zp, stream);
  }
}

template <int EPW>
hipError_t launch_partial_e(const uint16_t* x, int64_t ld_x, const float* wt, int64_t T, int d,
                            int E, float* partials, hipStream_t stream) {
  dim3 grid(ceil_div(T, kRouteBlock), ceil_div(d, kRouterChunk), ceil_div(E, 4 * EPW));
  hipLaunchKernelGGL((router_partial_kernel<EPW>), grid, dim3(256), 0, stream, x, ld_x, wt, T,
                     d, E, partials);
  return hipGetLastError();
}

}  // namespace

// Chunks of the split variant when it is used for this shape, else 0 (fused). The fused kernel
// has one 4-wave block per 64 tokens, too few waves per CU to hide its scalar weight loads until
// there are several blocks per CU (measured: at T = 32768, d = 2048, E = 64 the split variant is
// 24 % faster); the split variant's partial planes are capped at 512 MB of workspace.
int router_split_chunks(int64_t T, int d, int E) {
  int mode = router_mode_override();
  if (mode == 1) return 0;
  const int nchunk = ceil_div(d, kRouterChunk);
  const int64_t blocks = ceil_div(T, kRouteBlock);
  const int64_t plane_bytes = (int64_t)nchunk * T * E * (int64_t)sizeof(float);
  if (mode == 2 || (blocks < 8LL * num_cus() && plane_bytes <= (512LL << 20))) return nchunk;
  return 0;
}

hipError_t launch_router(const uint16_t* x, int64_t ld_x, const float* wt, const float* bias,
                         int64_t T, int d, int E, int k, int score_fn, float* logits,
                         int32_t* topk_ids, float* topk_w, float* prob_partial,
                         float* z_partial, float* partials, bool split, hipStream_t stream) {
  int epw = experts_per_wave(E);
  if (!split) {
    switch (epw) {
#define NT_FUSED(N) case N: return launch_fused_e<N>(x, ld_x, wt, bias, T, d, E, k, score_fn, logits, topk_ids, topk_w, prob_partial, z_partial, stream);
      NT_FUSED(1) NT_FUSED(2) NT_FUSED(4) NT_FUSED(8) NT_FUSED(16) NT_FUSED(32) NT_FUSED(64)
#undef NT_FUSED
      default: return hipErrorInvalidValue;
    }
  }
  // Split: smaller expert groups give more blocks when T is small (aim for >= 4 per CU: each
  // block is a single wave whose weight loads nothing else on the CU would hide).
  int epw_split = epw < 16 ? epw : 16;
  const int64_t row_chunks = (int64_t)ceil_div(T, kRouteBlock) * ceil_div(d, kRouterChunk);
  while (epw_split > 1 && row_chunks * ceil_div(E, 4 * epw_split) < 4LL * num_cus()) epw_split /= 2;
  hipError_t err;
  switch (epw_split) {
    case 1: err = launch_partial_e<1>(x, ld_x, wt, T, d, E, partials, stream); break;
    case 2: err = launch_partial_e<2>(x, ld_x, wt, T, d, E, partials, stream); break;
    case 4: err = launch_partial_e<4>(x, ld_x, wt, T, d, E, partials, stream); break;
    case 8: err = launch_partial_e<8>(x, ld_x, wt, T, d, E, partials, stream); break;
    default: err = launch_partial_e<16>(x, ld_x, wt, T, d, E, partials, stream); break;
  }
  if (err != hipSuccess) return err;
  const int nchunk = ceil_div(d, kRouterChunk);
  if (E % 4 == 0) {
    const int64_t n4 = T * E / 4;
    router_sum_planes_kernel<<<dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, stream>>>(
        partials, nchunk, bias, n4, T);
    err = hipGetLastError();
    if (err != hipSuccess) return err;
    return launch_topk_any(partials, 1, true, nullptr, T, E, k, score_fn, logits, topk_ids,
                           topk_w, prob_partial, z_partial, stream);
  }
  return launch_topk_any(partials, nchunk, true, bias, T, E, k, score_fn, logits, topk_ids,
                         topk_w, prob_partial, z_partial, stream);
}

hipError_t launch_topk_from_logits(const float* logits, int64_t T, int E, int k,
                                   int score_fn, int32_t* topk_ids, float* topk_w,
                                   float* prob_partial, float* z_partial, hipStream_t stream) {
  return launch_topk_any(logits, 1, false, nullptr, T, E, k, score_fn, nullptr, topk_ids,
                         topk_w, prob_partial, z_partial, stream);
}

}  // namespace ntmoe
