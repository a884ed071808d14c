// Route plan: per-expert histogram with stable in-block ranks, an LDS prefix scan that turns
// block counts into permutation offsets, and the permute kernel that writes the expert-major,
// token-ascending order (and optionally moves the token rows).
//
// Replaces (nexttransformer/scaling/megatron_moe.py:142-145):
//   ids = mapping.T.nonzero()[:, 1]   counts = mapping.sum(0)
//   selected_probs = probs.T[mapping.T]   rows[ids]
// Destination row of assignment (t, j) with expert e = topk_ids[t, j]:
//   offsets[e] + #{t' < t : e in topk_ids[t']}    (a token never picks an expert twice)
//
// Everything is integer and order-independent (bit ORs, integer adds), so results are
// deterministic with no sorting: a 64-token wave ORs lane bits into one 64-bit mask per
// expert in LDS; a lane's rank inside its wave is popcount(mask & lanes-below).
#include "common.h"

namespace ntmoe {
namespace {

constexpr int kHistBlock = 256;  // tokens per histogram block (4 waves x 64 lanes)

__global__ __launch_bounds__(256) void histogram_kernel(const int32_t* __restrict__ topk_ids,
                                                        int64_t T, int k, int E,
                                                        int32_t* __restrict__ ranks,
                                                        int32_t* __restrict__ block_counts) {
  extern __shared__ __align__(16) unsigned char smem[];
  uint64_t* mask = reinterpret_cast<uint64_t*>(smem);              // [4][E]
  int32_t* wave_prefix = reinterpret_cast<int32_t*>(mask + 4 * E);  // [4][E]
  const int w = wave_id(), lane = lane_id();
  const int64_t t = (int64_t)blockIdx.x * kHistBlock + threadIdx.x;
  for (int i = threadIdx.x; i < 4 * E; i += blockDim.x) mask[i] = 0ull;
  __syncthreads();
  int ids[NT_MOE_MAX_TOPK];
#pragma unroll
  for (int j = 0; j < NT_MOE_MAX_TOPK; ++j) {
    ids[j] = -1;
    if (j < k && t < T) {
      int e = topk_ids[t * k + j];
      if ((unsigned)e < (unsigned)E) {  // ids outside [0, E) are ignored
        ids[j] = e;
        atomicOr(reinterpret_cast<unsigned long long*>(&mask[w * E + e]), 1ull << lane);
      }
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int run = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      wave_prefix[q * E + e] = run;
      run += __popcll(mask[q * E + e]);
    }
    block_counts[(int64_t)blockIdx.x * E + e] = run;
  }
  __syncthreads();
  const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
  for (int j = 0; j < NT_MOE_MAX_TOPK; ++j) {
    if (ids[j] >= 0) {
      int e = ids[j];
      ranks[t * k + j] = wave_prefix[w * E + e] + __popcll(mask[w * E + e] & below);
    }
  }
}

// One workgroup: counts, offsets and block_base[b][e] = offsets[e] + sum_{b' < b} counts_b'[e].
// P = 1024 / E threads cooperate on each expert's column of block counts.
__global__ __launch_bounds__(1024) void scan_kernel(int32_t* __restrict__ block_counts, int nblk,
                                                    int E, int32_t* __restrict__ counts,
                                                    int32_t* __restrict__ offsets) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int P = blockDim.x / E;
  int32_t* part = reinterpret_cast<int32_t*>(smem);  // [E][P]
  int32_t* off = part + E * P;                       // [E+1]
  const int e = threadIdx.x / P, p = threadIdx.x - (threadIdx.x / P) * P;
  const bool active = e < E;
  const int per = (nblk + P - 1) / P;
  const int b0 = p * per, b1 = (b0 + per < nblk) ? b0 + per : nblk;
  int local = 0;
  if (active)
    for (int b = b0; b < b1; ++b) local += block_counts[(int64_t)b * E + e];
  if (active) part[e * P + p] = local;
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int q = 0; q < E; ++q) {
      int c = 0;
      for (int r = 0; r < P; ++r) c += part[q * P + r];
      off[q] = run;
      counts[q] = c;
      offsets[q] = run;
      run += c;
    }
    off[E] = run;
    offsets[E] = run;
  }
  __syncthreads();
  if (active) {
    int run = off[e];
    for (int r = 0; r < p; ++r) run += part[e * P + r];
    for (int b = b0; b < b1; ++b) {
      int c = block_counts[(int64_t)b * E + e];
      block_counts[(int64_t)b * E + e] = run;  // becomes block_base in place
      run += c;
    }
  }
}

// One wave per token: destinations, metadata in expert-ascending order, optional row move.
__global__ __launch_bounds__(256) void permute_kernel(
    const uint16_t* __restrict__ x, int64_t ld_x, const int32_t* __restrict__ topk_ids,
    const float* __restrict__ topk_w, int64_t T, int d, int k, int E,
    const int32_t* __restrict__ ranks, const int32_t* __restrict__ block_base,
    int32_t* __restrict__ src_row, float* __restrict__ perm_w, int32_t* __restrict__ combine_dest,
    float* __restrict__ combine_w, uint16_t* __restrict__ x_perm) {
  const int lane = lane_id();
  const int64_t waves = (int64_t)gridDim.x * 4;
  for (int64_t t = (int64_t)blockIdx.x * 4 + wave_id(); t < T; t += waves) {
    int e = 0x7fffffff, dest = 0;
    float w = 0.f;
    const int64_t A = T * k;
    if (lane < k) {
      e = topk_ids[t * k + lane];
      w = topk_w[t * k + lane];
      if ((unsigned)e < (unsigned)E) {
        dest = block_base[(t / kHistBlock) * E + e] + ranks[t * k + lane];
        dest = dest < 0 ? 0 : (dest >= A ? (int)(A - 1) : dest);
        src_row[dest] = (int32_t)t;
        if (perm_w) perm_w[dest] = w;
      } else {
        e = 0x7ffffffe;  // ignored id: sorts last, row 0 as a harmless target
      }
    }
    int pos = 0;
    for (int j = 0; j < k; ++j) pos += __shfl(e, j) < e;
    if (lane < k) {
      combine_dest[t * k + pos] = dest;
      combine_w[t * k + pos] = w;
    }
    if (x_perm) {
      const u32x4* srow = reinterpret_cast<const u32x4*>(x + t * ld_x);
      const int vecs = d >> 3;  // 16-byte vectors per row
      for (int v0 = 0; v0 < vecs; v0 += 64 * 4) {
        u32x4 buf[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          int v = v0 + q * 64 + lane;
          if (v < vecs) buf[q] = srow[v];
        }
        for (int j = 0; j < k; ++j) {
          int dj = __shfl(dest, j);
          u32x4* drow = reinterpret_cast<u32x4*>(x_perm + (int64_t)dj * d);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            int v = v0 + q * 64 + lane;
            if (v < vecs) drow[v] = buf[q];
          }
        }
      }
    }
  }
}

}  // namespace

hipError_t launch_histogram_scan(const int32_t* topk_ids, int64_t T, int k, int E,
                                 int32_t* counts, int32_t* offsets, int32_t* ranks,
                                 int32_t* block_counts, hipStream_t stream) {
  const int nblk = ceil_div(T, kHistBlock);
  if (nblk > 0) {
    size_t lds = (size_t)4 * E * (sizeof(uint64_t) + sizeof(int32_t));
    hipLaunchKernelGGL(histogram_kernel, dim3(nblk), dim3(256), lds, stream, topk_ids, T, k, E,
                       ranks, block_counts);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  const int P = 1024 / E;
  size_t lds = (size_t)(E * P + E + 1) * sizeof(int32_t);
  hipLaunchKernelGGL(scan_kernel, dim3(1), dim3(1024), lds, stream, block_counts, nblk, E, counts,
                     offsets);
  return hipGetLastError();
}

hipError_t launch_permute(const uint16_t* x, int64_t ld_x, const int32_t* topk_ids,
                          const float* topk_w, int64_t T, int d, int k, int E,
                          const int32_t* ranks, const int32_t* block_base,
                          int32_t* src_row, float* perm_w, int32_t* combine_dest,
                          float* combine_w, uint16_t* x_perm, hipStream_t stream) {
  if (T == 0) return hipSuccess;
  int64_t blocks = (T + 3) / 4;
  int cap = num_cus() * 16;
  if (blocks > cap) blocks = cap;
  hipLaunchKernelGGL(permute_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, x, ld_x,
                     topk_ids, topk_w, T, d, k, E, ranks, block_base, src_row, perm_w,
                     combine_dest, combine_w, x_perm);
  return hipGetLastError();
}

}  // namespace ntmoe
