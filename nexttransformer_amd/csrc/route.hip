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

// Inclusive scan of v over groups of `width` consecutive lanes (width a power of two <= 64).
__device__ __forceinline__ int group_inclusive_scan(int v, int width) {
  const int lane = lane_id();
  for (int o = 1; o < width; o <<= 1) {
    int u = __shfl_up(v, o, width);
    if ((lane & (width - 1)) >= o) v += u;
  }
  return v;
}

// One workgroup of 1024 threads: counts, offsets and
//   block_base[b][e] = offsets[e] + sum_{b' < b} block_counts[b'][e]   (written in place).
// P = min(64, 1024 / E) threads (a power of two, inside one wave) own expert e's column, each a
// contiguous run of blocks; shuffle scans combine runs and then experts.
__global__ __launch_bounds__(1024) void scan_kernel(int32_t* __restrict__ block_counts, int nblk,
                                                    int E, int P, int32_t* __restrict__ counts,
                                                    int32_t* __restrict__ offsets) {
  __shared__ int32_t cnt[NT_MOE_MAX_EXPERTS];
  __shared__ int32_t off[NT_MOE_MAX_EXPERTS + 1];
  const int tid = threadIdx.x;
  const int e = tid / P, p = tid - (tid / P) * P;
  const bool active = e < E;
  const int per = (nblk + P - 1) / P;
  const int b0 = p * per < nblk ? p * per : nblk;
  const int b1 = b0 + per < nblk ? b0 + per : nblk;
  int local = 0;
  if (active) {
#pragma unroll 4
    for (int b = b0; b < b1; ++b) local += block_counts[(int64_t)b * E + e];
  }
  const int incl = group_inclusive_scan(local, P);
  if (active && p == P - 1) cnt[e] = incl;
  __syncthreads();
  // Exclusive scan over experts by wave 0, 64 experts per pass.
  if (tid < 64) {
    int carry = 0;
    for (int base = 0; base < E; base += 64) {
      int v = base + tid < E ? cnt[base + tid] : 0;
      int inc = group_inclusive_scan(v, 64);
      if (base + tid < E) {
        off[base + tid] = carry + inc - v;
        counts[base + tid] = v;
        offsets[base + tid] = carry + inc - v;
      }
      carry += __shfl(inc, 63);
    }
    if (tid == 0) {
      off[E] = carry;
      offsets[E] = carry;
    }
  }
  __syncthreads();
  if (active) {
    int run = off[e] + incl - local;
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
  int P = 1;
  while (P < 64 && P * 2 * E <= 1024) P *= 2;
  hipLaunchKernelGGL(scan_kernel, dim3(1), dim3(1024), 0, stream, block_counts, nblk, E, P,
                     counts, offsets);
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
