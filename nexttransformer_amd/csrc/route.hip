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

// Largest counts table (blocks x experts) that plan_kernel reads in every workgroup; larger
// shapes take scan_kernel + permute_kernel.
constexpr int64_t kPlanTableMax = 16384;

// scan_kernel and permute_kernel (without the row move) in one launch, one workgroup per
// histogram block: the block's expert bases from the counts table -- each column summed over
// the earlier blocks, plus the exclusive scan over experts of the column totals -- then the
// permutation of its 256 tokens, one thread per token. Workgroup 0 writes counts and offsets.
// Every workgroup sums the table in the same fixed shape; all integer, so the bases equal
// scan_kernel's block_base exactly.
__global__ __launch_bounds__(256) void plan_kernel(
    const int32_t* __restrict__ topk_ids, const float* __restrict__ topk_w, int64_t T, int k,
    int E, int nblk, const int32_t* __restrict__ ranks, const int32_t* __restrict__ block_counts,
    int32_t* __restrict__ counts, int32_t* __restrict__ offsets, int32_t* __restrict__ src_row,
    float* __restrict__ perm_w, int32_t* __restrict__ combine_dest,
    float* __restrict__ combine_w) {
  __shared__ int32_t pre_s[256], tot_s[256];  // [G][E] partial column sums, G * E <= 256
  __shared__ int32_t base_s[NT_MOE_MAX_EXPERTS];
  __shared__ int32_t wave_tot[4];
  const int tid = threadIdx.x, lane = lane_id(), w = wave_id();
  const int blk = blockIdx.x;
  // The token's ids, weights and ranks are loaded first; their latency overlaps the table's.
  const int64_t t = (int64_t)blk * kHistBlock + tid;
  const bool live = t < T;
  int ev[NT_MOE_MAX_TOPK], rv[NT_MOE_MAX_TOPK];
  float wv[NT_MOE_MAX_TOPK];
#pragma unroll
  for (int j = 0; j < NT_MOE_MAX_TOPK; ++j) {
    ev[j] = 0x7fffffff;
    rv[j] = 0;
    wv[j] = 0.f;
    if (live && j < k) {
      ev[j] = topk_ids[t * k + j];
      wv[j] = topk_w[t * k + j];
      rv[j] = ranks[t * k + j];  // in bounds; used only for valid ids
    }
  }
  const int G = 256 / E;  // groups of E threads; group g sums blocks g, g + G, ...
  const int g = tid / E, e = tid - g * E;
  if (g < G) {
    int pre = 0, tot = 0;
#pragma unroll 8
    for (int b = g; b < nblk; b += G) {
      const int c = block_counts[(int64_t)b * E + e];
      tot += c;
      pre += b < blk ? c : 0;
    }
    pre_s[tid] = pre;
    tot_s[tid] = tot;
  }
  __syncthreads();
  int before = 0, total = 0;  // thread tid owns expert tid
  if (tid < E) {
    for (int q = 0; q < G; ++q) {
      before += pre_s[q * E + tid];
      total += tot_s[q * E + tid];
    }
  }
  const int incl = group_inclusive_scan(total, 64);
  if (lane == 63) wave_tot[w] = incl;
  __syncthreads();
  int carry = 0;
  for (int q = 0; q < w; ++q) carry += wave_tot[q];
  const int excl = carry + incl - total;  // offsets[tid]
  if (tid < E) {
    base_s[tid] = excl + before;
    if (blk == 0) {
      counts[tid] = total;
      offsets[tid] = excl;
    }
  }
  if (blk == 0 && tid == 0) offsets[E] = wave_tot[0] + wave_tot[1] + wave_tot[2] + wave_tot[3];
  __syncthreads();

  if (!live) return;
  const int64_t A = T * k;
  int dv[NT_MOE_MAX_TOPK];
#pragma unroll
  for (int j = 0; j < NT_MOE_MAX_TOPK; ++j) {
    dv[j] = 0;
    if (j < k) {
      if ((unsigned)ev[j] < (unsigned)E) {
        int dest = base_s[ev[j]] + rv[j];
        dest = dest < 0 ? 0 : (dest >= A ? (int)(A - 1) : dest);
        src_row[dest] = (int32_t)t;
        if (perm_w) perm_w[dest] = wv[j];
        dv[j] = dest;
      } else {
        ev[j] = 0x7ffffffe;  // ignored id: sorts last, row 0 as a harmless target
      }
    }
  }
  // Ascending expert order; equal keys (only ignored ids) keep their slot order.
#pragma unroll
  for (int j = 0; j < NT_MOE_MAX_TOPK; ++j) {
    if (j < k) {
      int pos = 0;
#pragma unroll
      for (int i = 0; i < NT_MOE_MAX_TOPK; ++i)
        pos += (ev[i] < ev[j] || (ev[i] == ev[j] && i < j)) ? 1 : 0;
      combine_dest[t * k + pos] = dv[j];
      combine_w[t * k + pos] = wv[j];
    }
  }
}

// plan_kernel from the router's outputs at its 64-token granularity: block_counts64[b][e]
// (assignments of tokens [64 b, 64 b + 64) to expert e) and each assignment's rank within its
// 64-token block (route_ranks_offset), both written by the router's top-k, so the histogram
// launch is not needed. One workgroup per 256 tokens (its four 64-token blocks, one per wave):
// every column of the table summed over the whole table and over the blocks before its own, in
// the same fixed shape in every workgroup, plus the counts of its own earlier 64-token blocks.
// All integer: the same destinations as histogram_kernel + plan_kernel.
__global__ __launch_bounds__(256) void plan_c64_kernel(
    const int32_t* __restrict__ topk_ids, const float* __restrict__ topk_w, int64_t T, int k,
    int E, int nblk64, const int32_t* __restrict__ block_counts64, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ src_row, float* __restrict__ perm_w,
    int32_t* __restrict__ combine_dest, float* __restrict__ combine_w) {
  __shared__ int32_t pre_s[1024], tot_s[1024];  // [G][E] partial column sums, G * E <= 1024
  __shared__ int32_t base_s[NT_MOE_MAX_EXPERTS];
  __shared__ int32_t sub_s[4][NT_MOE_MAX_EXPERTS];  // earlier 64-token blocks of this workgroup
  __shared__ int32_t wave_tot[4];
  const int tid = threadIdx.x, lane = lane_id(), w = wave_id();
  const int blk = blockIdx.x;
  const int64_t t = (int64_t)blk * kHistBlock + tid;
  const bool live = t < T;
  const int32_t* __restrict__ ranks64 = block_counts64 + route_ranks_offset(T, E);
  int ev[NT_MOE_MAX_TOPK], rv[NT_MOE_MAX_TOPK];
  float wv[NT_MOE_MAX_TOPK];
#pragma unroll
  for (int j = 0; j < NT_MOE_MAX_TOPK; ++j) {
    ev[j] = 0x7fffffff;
    rv[j] = 0;
    wv[j] = 0.f;
    if (live && j < k) {
      ev[j] = topk_ids[t * k + j];
      wv[j] = topk_w[t * k + j];
      rv[j] = ranks64[t * k + j];  // in bounds; used only for valid ids
    }
  }
  // Column sums of the table: groups of E / 4 threads, each thread four consecutive experts
  // (16-byte loads; E % 4 == 0, else one expert per thread); group g sums blocks g, g + G, ...
  // When E / 4 divides 64 the groups of a wave are combined by shuffles first, so the LDS
  // partials are one per wave.
  const int pre_end = 4 * blk;  // 64-token blocks before this workgroup's first token
  int G;
  const bool shfl = E % 4 == 0 && 64 % (E / 4) == 0;
  if (shfl) {
    const int E4 = E / 4;  // a power of two <= 64
    const int GT = 256 / E4;
    const int g = tid / E4, e4 = tid - g * E4;
    i32x4 pre = {0, 0, 0, 0}, tot = {0, 0, 0, 0};
#pragma unroll 16
    for (int b = g; b < nblk64; b += GT) {
      const i32x4 c = *reinterpret_cast<const i32x4*>(block_counts64 + (int64_t)b * E + 4 * e4);
      tot += c;
      if (b < pre_end) pre += c;
    }
    for (int m = E4; m < 64; m <<= 1) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        pre[q] += __shfl_xor(pre[q], m);
        tot[q] += __shfl_xor(tot[q], m);
      }
    }
    G = 4;  // one partial per wave
    if (lane < E4) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        pre_s[w * E + 4 * lane + q] = pre[q];
        tot_s[w * E + 4 * lane + q] = tot[q];
      }
    }
  } else if (E % 4 == 0) {
    const int E4 = E / 4;
    G = 256 / E4;
    const int g = tid / E4, e4 = tid - g * E4;
    if (g < G) {
      i32x4 pre = {0, 0, 0, 0}, tot = {0, 0, 0, 0};
#pragma unroll 16
      for (int b = g; b < nblk64; b += G) {
        const i32x4 c = *reinterpret_cast<const i32x4*>(block_counts64 + (int64_t)b * E + 4 * e4);
        tot += c;
        if (b < pre_end) pre += c;
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        pre_s[g * E + 4 * e4 + q] = pre[q];
        tot_s[g * E + 4 * e4 + q] = tot[q];
      }
    }
  } else {
    G = 256 / E;
    const int g = tid / E, e = tid - g * E;
    if (g < G) {
      int pre = 0, tot = 0;
#pragma unroll 8
      for (int b = g; b < nblk64; b += G) {
        const int c = block_counts64[(int64_t)b * E + e];
        tot += c;
        pre += b < pre_end ? c : 0;
      }
      pre_s[tid] = pre;
      tot_s[tid] = tot;
    }
  }
  // this workgroup's own 64-token blocks, exclusive prefix over them per expert
  if (tid < E) {
    int run = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int b = pre_end + q;
      const int c = b < nblk64 ? block_counts64[(int64_t)b * E + tid] : 0;
      sub_s[q][tid] = run;
      run += c;
    }
  }
  __syncthreads();
  int before = 0, total = 0;  // thread tid owns expert tid
  if (tid < E) {
    for (int q = 0; q < G; ++q) {
      before += pre_s[q * E + tid];
      total += tot_s[q * E + tid];
    }
  }
  const int incl = group_inclusive_scan(total, 64);
  if (lane == 63) wave_tot[w] = incl;
  __syncthreads();
  int carry = 0;
  for (int q = 0; q < w; ++q) carry += wave_tot[q];
  const int excl = carry + incl - total;  // offsets[tid]
  if (tid < E) {
    base_s[tid] = excl + before;
    if (blk == 0) {
      counts[tid] = total;
      offsets[tid] = excl;
    }
  }
  if (blk == 0 && tid == 0) offsets[E] = wave_tot[0] + wave_tot[1] + wave_tot[2] + wave_tot[3];
  __syncthreads();

  if (!live) return;
  const int64_t A = T * k;
  int dv[NT_MOE_MAX_TOPK];
#pragma unroll
  for (int j = 0; j < NT_MOE_MAX_TOPK; ++j) {
    dv[j] = 0;
    if (j < k) {
      if ((unsigned)ev[j] < (unsigned)E) {
        const int ej = ev[j];
        int dest = base_s[ej] + sub_s[w][ej] + rv[j];
        dest = dest < 0 ? 0 : (dest >= A ? (int)(A - 1) : dest);
        src_row[dest] = (int32_t)t;
        if (perm_w) perm_w[dest] = wv[j];
        dv[j] = dest;
      } else {
        ev[j] = 0x7ffffffe;  // ignored id: sorts last, row 0 as a harmless target
      }
    }
  }
  // Ascending expert order; equal keys (only ignored ids) keep their slot order.
#pragma unroll
  for (int j = 0; j < NT_MOE_MAX_TOPK; ++j) {
    if (j < k) {
      int pos = 0;
#pragma unroll
      for (int i = 0; i < NT_MOE_MAX_TOPK; ++i)
        pos += (ev[i] < ev[j] || (ev[i] == ev[j] && i < j)) ? 1 : 0;
      combine_dest[t * k + pos] = dv[j];
      combine_w[t * k + pos] = wv[j];
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

hipError_t launch_route_plan(const uint16_t* x, int64_t ld_x, const int32_t* topk_ids,
                             const float* topk_w, int64_t T, int d, int k, int E, int32_t* counts,
                             int32_t* offsets, int32_t* ranks, int32_t* block_counts,
                             int32_t* src_row, float* perm_w, int32_t* combine_dest,
                             float* combine_w, uint16_t* x_perm, hipStream_t stream) {
  const int64_t nblk = ceil_div(T, kHistBlock);
  if (T == 0 || x_perm || nblk * E > kPlanTableMax) {
    hipError_t err = launch_histogram_scan(topk_ids, T, k, E, counts, offsets, ranks,
                                           block_counts, stream);
    if (err != hipSuccess) return err;
    return launch_permute(x, ld_x, topk_ids, topk_w, T, d, k, E, ranks, block_counts, src_row,
                          perm_w, combine_dest, combine_w, x_perm, stream);
  }
  size_t lds = (size_t)4 * E * (sizeof(uint64_t) + sizeof(int32_t));
  hipLaunchKernelGGL(histogram_kernel, dim3((unsigned)nblk), dim3(256), lds, stream, topk_ids, T,
                     k, E, ranks, block_counts);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(plan_kernel, dim3((unsigned)nblk), dim3(256), 0, stream, topk_ids, topk_w, T,
                     k, E, (int)nblk, ranks, block_counts, counts, offsets, src_row, perm_w,
                     combine_dest, combine_w);
  return hipGetLastError();
}

// The route plan from the router's per-64-token-block counts (one launch); E <= 256.
hipError_t launch_plan_from_counts(const int32_t* topk_ids, const float* topk_w, int64_t T, int k,
                                   int E, const int32_t* block_counts64, int32_t* counts,
                                   int32_t* offsets, int32_t* src_row, float* perm_w,
                                   int32_t* combine_dest, float* combine_w, hipStream_t stream) {
  if (T == 0 || E > 256) return hipErrorInvalidValue;
  const int64_t nblk = ceil_div(T, kHistBlock);
  const int nblk64 = ceil_div(T, kRouteBlock);
  hipLaunchKernelGGL(plan_c64_kernel, dim3((unsigned)nblk), dim3(256), 0, stream, topk_ids,
                     topk_w, T, k, E, nblk64, block_counts64, counts, offsets, src_row, perm_w,
                     combine_dest, combine_w);
  return hipGetLastError();
}

}  // namespace ntmoe
