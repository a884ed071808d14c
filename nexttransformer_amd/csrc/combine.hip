// Deterministic weighted combine (unpermute) and the auxiliary losses.
//
// Replaces result = zeros_like(rows).index_add(0, ids, output) + shared_experts(hidden)
// (nexttransformer/scaling/megatron_moe.py:148-150) and RoutedFFN's shared-then-index_add
// loop (reference_blocks.py:39-44). No atomics: one wave owns one output row and adds its k
// expert rows in ascending expert order (combine_dest is stored in that order) into fp32,
// starting from the shared expert row when there is one, and rounds to bf16 once.
// All k source rows are loaded before the first add so k row reads are in flight at once.
//
// Aux losses (MCore TopKRouter "aux_loss" type and z-loss, megatron_moe.py:44-45) from the
// router's per-block partials, reduced in block order in double precision:
//   lb = aux_coeff * E / (k T^2) * sum_e S_e * counts[e],  S_e = sum_t s_te
//   z  = z_coeff * (sum_t lse_t^2) / T
#include "common.h"

namespace ntmoe {
namespace {

// One wave per output row at a time; the row is walked in column chunks of 64 lanes x VPC
// 16-byte vectors (VPC = 2: 1024 bf16 per chunk, when the row is whole chunks of that; else
// VPC = 1, so a row of 1280 bf16 is chunks of 64, 64 and 32 vectors rather than 128 and 32:
// 85 against 96 us for the T3 cell's combine). Waves are persistent over tokens (t, t + the
// grid's waves, ...) and walk the items (token, chunk) in order, issuing the next item's k row
// loads (and its shared-expert chunk) before summing the current one, so 2 (k + 1) VPC vectors
// per lane are in flight. KMAX bounds k (registers are sized by it).
template <int KMAX, int VPC>
__device__ __forceinline__ void combine_rows(
    const uint16_t* __restrict__ y, const int32_t* __restrict__ combine_dest,
    const float* __restrict__ combine_w, int64_t T, int d, int k,
    const uint16_t* __restrict__ shared_y, int64_t ld_shared, uint16_t* __restrict__ out,
    int64_t ld_out, int blocks) {
  const int lane = lane_id();
  const int vecs = d >> 3;
  const int chunk = 64 * VPC;
  const int64_t waves = (int64_t)blocks * 4;
  const int64_t A = T * k;  // rows of y; out-of-range rows are clamped
  // The token's k destination rows and weights, lane j holding slot j.
  auto plan = [&](int64_t t, int& dest, float& w) {
    dest = 0;
    w = 0.f;
    if (lane < k && t < T) {
      dest = combine_dest[t * k + lane];
      w = combine_w[t * k + lane];
      dest = dest < 0 ? 0 : (dest >= A ? (int)(A - 1) : dest);
    }
  };
  // Chunk v0 of token t: its k expert rows and its shared-expert row (zeros without one).
  auto load_rows = [&](int64_t t, int dest, int v0, u32x4 (&rows)[KMAX][VPC], u32x4 (&sh)[VPC]) {
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      if (j < k) {
        const u32x4* src = reinterpret_cast<const u32x4*>(y + (int64_t)__shfl(dest, j) * d);
#pragma unroll
        for (int q = 0; q < VPC; ++q) {
          const int v = v0 + q * 64 + lane;
          rows[j][q] = v < vecs ? src[v] : u32x4{0u, 0u, 0u, 0u};
        }
      }
    }
    const u32x4* srow = reinterpret_cast<const u32x4*>(shared_y + t * ld_shared);
#pragma unroll
    for (int q = 0; q < VPC; ++q) {
      const int v = v0 + q * 64 + lane;
      sh[q] = shared_y && v < vecs ? srow[v] : u32x4{0u, 0u, 0u, 0u};
    }
  };
  // Sum of the shared row and the k weighted rows of chunk v0 of token t, stored.
  auto finish = [&](int64_t t, int v0, float w, const u32x4 (&rows)[KMAX][VPC],
                    const u32x4 (&sh)[VPC]) {
    float acc[VPC][8];
#pragma unroll
    for (int q = 0; q < VPC; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[q][2 * i] = __builtin_bit_cast(float, sh[q][i] << 16);
        acc[q][2 * i + 1] = __builtin_bit_cast(float, sh[q][i] & 0xffff0000u);
      }
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      if (j < k) {
        const float wj = __shfl(w, j);
#pragma unroll
        for (int q = 0; q < VPC; ++q)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            acc[q][2 * i] = __builtin_fmaf(
                wj, __builtin_bit_cast(float, rows[j][q][i] << 16), acc[q][2 * i]);
            acc[q][2 * i + 1] = __builtin_fmaf(
                wj, __builtin_bit_cast(float, rows[j][q][i] & 0xffff0000u), acc[q][2 * i + 1]);
          }
      }
    }
    u32x4* orow = reinterpret_cast<u32x4*>(out + t * ld_out);
#pragma unroll
    for (int q = 0; q < VPC; ++q) {
      const int v = v0 + q * 64 + lane;
      if (v < vecs) {
        u32x4 r;
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = pack_bf16x2(acc[q][2 * i], acc[q][2 * i + 1]);
        orow[v] = r;
      }
    }
  };

  int64_t t = (int64_t)blockIdx.x * 4 + wave_id();
  if (t >= T) return;
  int v0 = 0, dest;
  float w;
  u32x4 rows[KMAX][VPC], sh[VPC], nrows[KMAX][VPC], nsh[VPC];
  plan(t, dest, w);
  load_rows(t, dest, 0, rows, sh);
  while (t < T) {
    // the next item: the row's next chunk, or the first chunk of the wave's next token
    int64_t tn = t;
    int vn = v0 + chunk, ndest = dest;
    float nw = w;
    if (vn >= vecs) {
      tn = t + waves;
      vn = 0;
      plan(tn, ndest, nw);
    }
    if (tn < T) load_rows(tn, ndest, vn, nrows, nsh);
    finish(t, v0, w, rows, sh);
#pragma unroll
    for (int j = 0; j < KMAX; ++j)
#pragma unroll
      for (int q = 0; q < VPC; ++q) rows[j][q] = nrows[j][q];
#pragma unroll
    for (int q = 0; q < VPC; ++q) sh[q] = nsh[q];
    t = tn;
    v0 = vn;
    dest = ndest;
    w = nw;
  }
}

// The auxiliary losses, by one 256-thread workgroup. Thread (e, p), p < P = 256 / E rounded
// down to a power of two, sums block partials b = p, p + P, ... of expert e in order; fixed-shape
// trees then combine the P values and the E experts, so the result does not depend on timing.
constexpr int kAuxThreads = 256;

__device__ void aux_block(const float* __restrict__ prob_partial,
                          const float* __restrict__ z_partial, int nblk,
                          const int32_t* __restrict__ counts, int E, int P, int k, int64_t T,
                          float aux_coeff, float z_coeff, float* __restrict__ aux_out) {
  __shared__ double red[kAuxThreads];
  __shared__ double zred[kAuxThreads];
  const int tid = threadIdx.x;
  const int e = tid / P, p = tid - (tid / P) * P;
  double s = 0.0;
  if (e < E) {
#pragma unroll 8
    for (int b = p; b < nblk; b += P) s += (double)prob_partial[(int64_t)b * E + e];
  }
  double z = 0.0;
#pragma unroll 8
  for (int b = tid; b < nblk; b += kAuxThreads) z += (double)z_partial[b];
  red[tid] = s;
  zred[tid] = z;
  __syncthreads();
  for (int w = P >> 1; w > 0; w >>= 1) {  // tree over p inside each expert's group
    if (e < E && p < w) red[tid] += red[tid + w];
    __syncthreads();
  }
  if (e < E && p == 0) red[tid] *= (double)counts[e];  // S_e * count_e at red[e * P]
  __syncthreads();
  // Sum the E products (stride P) and the z partials with fixed trees.
  for (int w = kAuxThreads >> 1; w > 0; w >>= 1) {
    if (tid < w) {
      zred[tid] += zred[tid + w];
      int a = tid, bidx = tid + w;
      if (bidx < E) red[a * P] += red[bidx * P];
    }
    __syncthreads();
  }
  if (tid == 0) {
    double Td = (double)T;
    double lb = T > 0 ? (double)aux_coeff * E / ((double)k * Td * Td) * red[0] : 0.0;
    double zz = T > 0 ? (double)z_coeff * zred[0] / Td : 0.0;
    aux_out[0] = (float)(lb + zz);
    aux_out[1] = (float)lb;
    aux_out[2] = (float)zz;
  }
}

struct AuxArgs {
  const float* prob_partial;
  const float* z_partial;
  const int32_t* counts;
  int nblk, E, P;
  float aux_coeff, z_coeff;
  float* aux_out;  // null: no aux workgroup
};

// The combine grid plus, when aux.aux_out is set, one last workgroup that computes the losses
// (they depend only on the router's partials and the counts, so they run beside the combine).
template <int KMAX, int VPC>
__global__ __launch_bounds__(256) void combine_aux_kernel(
    const uint16_t* __restrict__ y, const int32_t* __restrict__ combine_dest,
    const float* __restrict__ combine_w, int64_t T, int d, int k,
    const uint16_t* __restrict__ shared_y, int64_t ld_shared, uint16_t* __restrict__ out,
    int64_t ld_out, AuxArgs aux) {
  const int combine_blocks = (int)gridDim.x - (aux.aux_out ? 1 : 0);
  if ((int)blockIdx.x == combine_blocks) {
    aux_block(aux.prob_partial, aux.z_partial, aux.nblk, aux.counts, aux.E, aux.P, k, T,
              aux.aux_coeff, aux.z_coeff, aux.aux_out);
    return;
  }
  combine_rows<KMAX, VPC>(y, combine_dest, combine_w, T, d, k, shared_y, ld_shared, out, ld_out,
                          combine_blocks);
}

}  // namespace

hipError_t launch_combine_aux(const uint16_t* y, const int32_t* combine_dest,
                              const float* combine_w, int64_t T, int d, int k,
                              const uint16_t* shared_y, int64_t ld_shared, uint16_t* out,
                              int64_t ld_out, const float* prob_partial, const float* z_partial,
                              const int32_t* counts, int E, float aux_coeff, float z_coeff,
                              float* aux_out, hipStream_t stream) {
  AuxArgs aux{prob_partial, z_partial, counts, ceil_div(T, kRouteBlock), E, 1, aux_coeff,
              z_coeff, aux_out};
  while (aux.P * 2 * E <= kAuxThreads) aux.P *= 2;
  // persistent waves, as many as stay resident at the variant's register use (each then takes
  // several tokens), or one per token
  int64_t blocks = (T + 3) / 4;
  const int per_cu = k <= 2 ? 7 : (k <= 4 ? 4 : 3);
  const int64_t cap = (int64_t)num_cus() * per_cu;
  if (blocks > cap) blocks = cap;
  if (aux_out) ++blocks;
  if (blocks == 0) return hipSuccess;
  const bool two = (d / 8) % 128 == 0;  // rows of whole 2-vector chunks
  auto kern = two ? (k <= 2 ? combine_aux_kernel<2, 2>
                            : (k <= 4 ? combine_aux_kernel<4, 2>
                                      : combine_aux_kernel<NT_MOE_MAX_TOPK, 2>))
                  : (k <= 2 ? combine_aux_kernel<2, 1>
                            : (k <= 4 ? combine_aux_kernel<4, 1>
                                      : combine_aux_kernel<NT_MOE_MAX_TOPK, 1>));
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), 0, stream, y, combine_dest,
                     combine_w, T, d, k, shared_y, ld_shared, out, ld_out, aux);
  hipError_t err = hipGetLastError();
  return err;
}

}  // namespace ntmoe
