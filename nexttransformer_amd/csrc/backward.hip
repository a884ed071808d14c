// Backward of the MoE layer: the kernels that are not grouped GEMMs.
//
// The layer (forward, nexttransformer/scaling/megatron_moe.py:137-150, reference_blocks.py:35-45):
//   logits = x Wr^T + bias;  (ids, w) = top-k of logits, w = scores normalised over the k selected
//   y_r = act(a_r W1_s^T) W2_s^T for each assignment row r (expert s, token t = src_row[r])
//   out_t = shared_t + sum_j w_tj y_{dest_tj};  aux = lb + z from the full scores and counts
// Given g = d loss / d out and the aux loss's gradient, this file provides
//   combine_bwd:  dy_r = w_tj g_t (bf16, expert-major rows) and dw_tj = <g_t, y_r> (fp32)
//   act_bwd:      d fc1 from d h and the fc1 pre-activations (SwiGLU or ReLU^2)
//   router_bwd:   d logits from dw (the k-selected normalisation) plus the load-balance and
//                 z-loss terms (MCore TopKRouter, megatron_moe.py:43-45)
// The dgrad GEMMs run on the packed grouped GEMM with transposed packed weights, and the
// token-side scatter (dx_t = sum_j dx_perm_{dest_tj}) on the forward's combine kernel.
// Every reduction has a fixed shape, so results do not depend on timing.
#include "common.h"

namespace ntmoe {
namespace {

// One wave per token. The k rows are visited in ascending expert order (combine_dest's order);
// dw comes out in the caller's top-k slot order (slot j of token t is combine slot
// #{i : ids[t, i] < ids[t, j]}).
__global__ __launch_bounds__(256) void combine_bwd_kernel(
    const uint16_t* __restrict__ g, int64_t ld_g, const uint16_t* __restrict__ y,
    const int32_t* __restrict__ topk_ids, const int32_t* __restrict__ combine_dest,
    const float* __restrict__ combine_w, int64_t T, int d, int k, uint16_t* __restrict__ dy,
    float* __restrict__ dw) {
  const int lane = lane_id();
  const int vecs = d >> 3;
  const int64_t A = T * k;
  const int64_t waves = (int64_t)gridDim.x * 4;
  for (int64_t t = (int64_t)blockIdx.x * 4 + wave_id(); t < T; t += waves) {
    int dest = 0, e = 0x7fffffff;
    float w = 0.f;
    if (lane < k) {
      dest = combine_dest[t * k + lane];
      dest = dest < 0 ? 0 : (dest >= A ? (int)(A - 1) : dest);
      w = combine_w[t * k + lane];
      e = topk_ids[t * k + lane];
    }
    const u32x4* grow = reinterpret_cast<const u32x4*>(g + t * ld_g);
    float dots[NT_MOE_MAX_TOPK];
#pragma unroll
    for (int j = 0; j < NT_MOE_MAX_TOPK; ++j) dots[j] = 0.f;
    for (int v = lane; v < vecs; v += 64) {
      const u32x4 gv = grow[v];
      float gf[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        gf[2 * i] = bf16_bits_to_f32(gv[i] & 0xffffu);
        gf[2 * i + 1] = __builtin_bit_cast(float, gv[i] & 0xffff0000u);
      }
#pragma unroll
      for (int j = 0; j < NT_MOE_MAX_TOPK; ++j) {
        if (j < k) {
          const int64_t r = __shfl(dest, j);
          const float wj = __shfl(w, j);
          const u32x4 yv = reinterpret_cast<const u32x4*>(y + r * d)[v];
          u32x4 o;
          float s = 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            s = __builtin_fmaf(gf[2 * i], bf16_bits_to_f32(yv[i] & 0xffffu), s);
            s = __builtin_fmaf(gf[2 * i + 1], __builtin_bit_cast(float, yv[i] & 0xffff0000u), s);
            o[i] = pack_bf16x2(wj * gf[2 * i], wj * gf[2 * i + 1]);
          }
          dots[j] += s;
          reinterpret_cast<u32x4*>(dy + r * d)[v] = o;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < NT_MOE_MAX_TOPK; ++j)
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) dots[j] += __shfl_xor(dots[j], m);
    // lane i < k: its slot's combine position among the token's ids (all lanes read e_j)
    int pos = 0;
    for (int j = 0; j < k; ++j) pos += __shfl(e, j) < e ? 1 : 0;
    float mine = 0.f;
#pragma unroll
    for (int j = 0; j < NT_MOE_MAX_TOPK; ++j) mine = pos == j ? dots[j] : mine;
    if (lane < k) dw[t * k + lane] = mine;
  }
}

__device__ __forceinline__ float sigmoidf_(float v) { return 1.f / (1.f + expf(-v)); }

// d fc1 for rows x H hidden units, 8 units per thread (H % 8 == 0). SwiGLU: fc1 row = [gate |
// value] (2H wide), h = silu(gate) value; ReLU^2: fc1 row H wide, h = relu(f)^2.
template <int ACT>
__global__ __launch_bounds__(256) void act_bwd_kernel(const uint16_t* __restrict__ fc1,
                                                      const uint16_t* __restrict__ dh, int64_t rows,
                                                      int H, uint16_t* __restrict__ dfc1) {
  const int per_row = H >> 3;
  const int64_t n = rows * per_row;
  const int F = ACT == NT_MOE_ACT_SWIGLU ? 2 * H : H;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / per_row;
    const int c = (int)(i - r * per_row) * 8;
    const u32x4 dv = *reinterpret_cast<const u32x4*>(dh + r * H + c);
    const u32x4 fv = *reinterpret_cast<const u32x4*>(fc1 + r * F + c);
    if (ACT == NT_MOE_ACT_SWIGLU) {
      const u32x4 uv = *reinterpret_cast<const u32x4*>(fc1 + r * F + H + c);
      u32x4 dg, du;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float gg[2], uu[2], dd[2], og[2], ou[2];
        gg[0] = bf16_bits_to_f32(fv[q] & 0xffffu);
        gg[1] = __builtin_bit_cast(float, fv[q] & 0xffff0000u);
        uu[0] = bf16_bits_to_f32(uv[q] & 0xffffu);
        uu[1] = __builtin_bit_cast(float, uv[q] & 0xffff0000u);
        dd[0] = bf16_bits_to_f32(dv[q] & 0xffffu);
        dd[1] = __builtin_bit_cast(float, dv[q] & 0xffff0000u);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float s = sigmoidf_(gg[h]);
          const float silu = gg[h] * s;
          og[h] = dd[h] * uu[h] * s * (1.f + gg[h] * (1.f - s));
          ou[h] = dd[h] * silu;
        }
        dg[q] = pack_bf16x2(og[0], og[1]);
        du[q] = pack_bf16x2(ou[0], ou[1]);
      }
      *reinterpret_cast<u32x4*>(dfc1 + r * F + c) = dg;
      *reinterpret_cast<u32x4*>(dfc1 + r * F + H + c) = du;
    } else {
      u32x4 o;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float f0 = bf16_bits_to_f32(fv[q] & 0xffffu);
        const float f1 = __builtin_bit_cast(float, fv[q] & 0xffff0000u);
        const float d0 = bf16_bits_to_f32(dv[q] & 0xffffu);
        const float d1 = __builtin_bit_cast(float, dv[q] & 0xffff0000u);
        o[q] = pack_bf16x2(d0 * 2.f * (f0 > 0.f ? f0 : 0.f), d1 * 2.f * (f1 > 0.f ? f1 : 0.f));
      }
      *reinterpret_cast<u32x4*>(dfc1 + r * F + c) = o;
    }
  }
}

// One wave per token; lane l holds experts l, l + 64, ... (E <= 256).
//   selected (softmax over the k):     dl_j = w_j (dw_j - sum_i w_i dw_i)
//   selected (sigmoid, normalised):    dl_j = s_j (1 - s_j) / S (dw_j - sum_i w_i dw_i)
//   load balance, lb = c_lb sum_e S_e counts_e with S_e = sum_t p_te (p = full scores):
//     dl_e += g_lb c_lb q_e (counts_e - sum_e' p_e' counts_e'),  q = p (softmax) or
//     s (1 - s) / sum s (sigmoid normalised over all experts)
//   z-loss, z = c_z / T sum_t lse_t^2:  dl_e += g_z c_z 2 lse_t / T softmax_e
// with c_lb = aux_coeff E / (k T^2), c_z = z_coeff, and g_lb, g_z read from grad_aux (the
// gradient of the forward's aux = {lb + z, lb, z}; NULL = no aux gradient).
// PER = experts per lane (E <= 64 PER): the per-token work is sized by E, not by the largest E.
template <int PER>
__global__ __launch_bounds__(256) void router_bwd_kernel(
    const float* __restrict__ logits, const int32_t* __restrict__ topk_ids,
    const float* __restrict__ topk_w, const float* __restrict__ dw,
    const int32_t* __restrict__ counts, int64_t T, int E, int k, int score_fn,
    const float* __restrict__ grad_aux, float aux_coeff, float z_coeff,
    float* __restrict__ dlogits) {
  const bool sigmoid = score_fn != NT_MOE_SCORE_SOFTMAX;
  const int lane = lane_id();
  // aux = {lb + z, lb, z}: gradients reach lb through entries 0 and 1, z through 0 and 2
  float g_lb = 0.f, g_z = 0.f;
  if (grad_aux) {
    g_lb = grad_aux[0] + grad_aux[1];
    g_z = grad_aux[0] + grad_aux[2];
  }
  const float lb_scale = g_lb * aux_coeff * (float)E / ((float)k * (float)T * (float)T);
  const float z_scale = g_z * z_coeff / (float)T;
  const int64_t waves = (int64_t)gridDim.x * 4;
  for (int64_t t = (int64_t)blockIdx.x * 4 + wave_id(); t < T; t += waves) {
    const float* row = logits + t * E;
    float l[PER], c[PER];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = lane + 64 * i;
      l[i] = e < E ? row[e] : -INFINITY;
      c[i] = e < E ? (float)counts[e] : 0.f;
      m = fmaxf(m, l[i]);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    float ex[PER], sg[PER], sum_ex = 0.f, sum_sg = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const bool in = lane + 64 * i < E;
      ex[i] = in ? expf(l[i] - m) : 0.f;
      sg[i] = in && sigmoid ? sigmoidf_(l[i]) : 0.f;  // (the softmax path needs none)
      sum_ex += ex[i];
      sum_sg += sg[i];
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      sum_ex += __shfl_xor(sum_ex, o);
      sum_sg += __shfl_xor(sum_sg, o);
    }
    const float lse = m + logf(sum_ex);
    // full scores and their counts-weighted mean
    float pc = 0.f;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const float p = score_fn == NT_MOE_SCORE_SOFTMAX ? ex[i] / sum_ex : sg[i] / sum_sg;
      pc += p * c[i];
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) pc += __shfl_xor(pc, o);
    float out[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const float q = score_fn == NT_MOE_SCORE_SOFTMAX ? ex[i] / sum_ex
                                                       : sg[i] * (1.f - sg[i]) / sum_sg;
      out[i] = lb_scale * q * (c[i] - pc) + z_scale * 2.f * lse * (ex[i] / sum_ex);
    }
    // the k selected: lane j < k holds slot j
    int e = -1;
    float wj = 0.f, dwj = 0.f, lj = 0.f;
    if (lane < k) {
      e = topk_ids[t * k + lane];
      if ((unsigned)e >= (unsigned)E) e = -1;
      wj = topk_w[t * k + lane];
      dwj = dw[t * k + lane];
      lj = e >= 0 ? row[e] : 0.f;
    }
    float wdw = wj * dwj, ssel = lane < k && e >= 0 ? sigmoidf_(lj) : 0.f;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      wdw += __shfl_xor(wdw, o);
      ssel += __shfl_xor(ssel, o);
    }
    float dsel = 0.f;
    if (lane < k && e >= 0) {
      dsel = score_fn == NT_MOE_SCORE_SOFTMAX
                 ? wj * (dwj - wdw)
                 : sigmoidf_(lj) * (1.f - sigmoidf_(lj)) / ssel * (dwj - wdw);
    }
    // add each slot's term to its expert's lane (slots hold distinct experts)
    for (int j = 0; j < k; ++j) {
      const int ej = __shfl(e, j);
      const float dj = __shfl(dsel, j);
#pragma unroll
      for (int i = 0; i < PER; ++i)
        if (ej == lane + 64 * i) out[i] += dj;
    }
    float* drow = dlogits + t * E;
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (lane + 64 * i < E) drow[lane + 64 * i] = out[i];
  }
}

// The backward's first-row operand: a [T, Kc] bf16 row is
//   [dfc1_shared (Fs) | g_hi (Ep) | g_hi (Ep) | g_lo (Ep) | 0 ...]
// with g = grad_logits (fp32 [T, E], columns past E zero in each Ep block), g_hi = g rounded to
// bf16 and g_lo = (g - g_hi) rounded to bf16 (the remainder is exact in fp32). One thread per 8
// columns (Fs, Ep and Kc are multiples of 8, so 8 columns never straddle two parts).
__global__ __launch_bounds__(256) void first_operand_kernel(
    const float* __restrict__ g, int E, const uint16_t* __restrict__ dfc1s, int Fs, int64_t T,
    int Ep, int Kc, uint16_t* __restrict__ out) {
  const int per_row = Kc / 8;
  const int64_t n = T * per_row;
  const bool narrow = n < ((int64_t)1 << 31);  // 32-bit index arithmetic
  // 8 columns of g lie wholly inside or wholly past E, 16-byte aligned: two loads
  const bool vec = E % 8 == 0 && (reinterpret_cast<uintptr_t>(g) & 15) == 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    int64_t t;
    int j0;
    if (narrow) {
      const int tt = (int)i / per_row;
      t = tt;
      j0 = ((int)i - tt * per_row) * 8;
    } else {
      t = i / per_row;
      j0 = (int)(i - t * per_row) * 8;
    }
    u32x4 v = {0u, 0u, 0u, 0u};
    if (j0 < Fs) {
      v = *reinterpret_cast<const u32x4*>(dfc1s + t * Fs + j0);
    } else if (j0 < Fs + 3 * Ep) {
      const int part = (j0 - Fs) / Ep, e0 = (j0 - Fs) - part * Ep;
      const float* row = g + t * E;
      float x[8];
      if (vec) {
        floatx4 x0 = {0.f, 0.f, 0.f, 0.f}, x1 = x0;
        if (e0 < E) {
          x0 = *reinterpret_cast<const floatx4*>(row + e0);
          x1 = *reinterpret_cast<const floatx4*>(row + e0 + 4);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          x[q] = x0[q];
          x[4 + q] = x1[q];
        }
      } else {
#pragma unroll
        for (int q = 0; q < 8; ++q) x[q] = e0 + q < E ? row[e0 + q] : 0.f;
      }
      uint16_t h[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const uint16_t hi = f32_to_bf16_bits(x[q]);
        h[q] = part < 2 ? hi
                        : f32_to_bf16_bits(x[q] - __builtin_bit_cast(float, (uint32_t)hi << 16));
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = (uint32_t)h[2 * q] | ((uint32_t)h[2 * q + 1] << 16);
    }
    *reinterpret_cast<u32x4*>(out + t * Kc + j0) = v;
  }
}

}  // namespace

hipError_t launch_combine_bwd(const uint16_t* g, int64_t ld_g, const uint16_t* y,
                              const int32_t* topk_ids, const int32_t* combine_dest,
                              const float* combine_w, int64_t T, int d, int k, uint16_t* dy,
                              float* dw, hipStream_t stream) {
  if (T == 0) return hipSuccess;
  int64_t blocks = (T + 3) / 4;
  const int64_t cap = (int64_t)num_cus() * 32;
  if (blocks > cap) blocks = cap;
  hipLaunchKernelGGL(combine_bwd_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, g, ld_g, y,
                     topk_ids, combine_dest, combine_w, T, d, k, dy, dw);
  return hipGetLastError();
}

hipError_t launch_act_bwd(const uint16_t* fc1, const uint16_t* dh, int64_t rows, int H,
                          int activation, uint16_t* dfc1, hipStream_t stream) {
  const int64_t n = rows * (H / 8);
  if (n == 0) return hipSuccess;
  int64_t blocks = (n + 255) / 256;
  const int64_t cap = (int64_t)num_cus() * 16;
  if (blocks > cap) blocks = cap;
  if (activation == NT_MOE_ACT_SWIGLU)
    hipLaunchKernelGGL(act_bwd_kernel<NT_MOE_ACT_SWIGLU>, dim3((unsigned)blocks), dim3(256), 0,
                       stream, fc1, dh, rows, H, dfc1);
  else
    hipLaunchKernelGGL(act_bwd_kernel<NT_MOE_ACT_RELU2>, dim3((unsigned)blocks), dim3(256), 0,
                       stream, fc1, dh, rows, H, dfc1);
  return hipGetLastError();
}

hipError_t launch_router_bwd(const float* logits, const int32_t* topk_ids, const float* topk_w,
                             const float* dw, const int32_t* counts, int64_t T, int E, int k,
                             int score_fn, const float* grad_aux, float aux_coeff, float z_coeff,
                             float* dlogits, hipStream_t stream) {
  if (T == 0) return hipSuccess;
  int64_t blocks = (T + 3) / 4;
  const int64_t cap = (int64_t)num_cus() * 32;
  if (blocks > cap) blocks = cap;
  auto kern = E <= 64 ? router_bwd_kernel<1>
                      : (E <= 128 ? router_bwd_kernel<2> : router_bwd_kernel<NT_MOE_MAX_EXPERTS / 64>);
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), 0, stream, logits, topk_ids, topk_w,
                     dw, counts, T, E, k, score_fn, grad_aux, aux_coeff, z_coeff, dlogits);
  return hipGetLastError();
}

hipError_t launch_first_operand(const float* grad_logits, int E, const uint16_t* dfc1s, int Fs,
                                int64_t T, int Ep, int Kc, uint16_t* out, hipStream_t stream) {
  const int64_t n = T * (Kc / 8);
  if (n == 0) return hipSuccess;
  int64_t blocks = (n + 255) / 256;
  const int64_t cap = (int64_t)num_cus() * 16;
  if (blocks > cap) blocks = cap;
  hipLaunchKernelGGL(first_operand_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     grad_logits, E, dfc1s, Fs, T, Ep, Kc, out);
  return hipGetLastError();
}

}  // namespace ntmoe
