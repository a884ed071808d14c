// Grouped weight gradient on bf16 MFMA (gfx950 v_mfma_f32_32x32x16_bf16), fp32 accumulation:
//   C_s[n, m] = sum_{r in [seg_offsets[s], seg_offsets[s+1])} A[r, n] * B[row(r), m]
// with row(r) = b_src_row[r] when given (the token rows the up projection gathered) else r.
// This is the expert weight gradient of the grouped FFN (autograd of megatron_moe.py:145's
// per-expert MasterLinear products, megatron_moe.py:58-78): dW2_s = dy_s^T h_s and
// dW1_s = dfc1_s^T x_s, each over the expert's own rows (ragged K).
//
// Both operands are row-major in r (the reduction index), but the matrix core wants each
// lane's 8 operand values consecutive in K. So every K step moves a 64-row slab of A and B
// through LDS transposed: a thread loads an 8-row x 8-column block (eight 16-byte row pieces),
// interleaves it in registers with v_perm_b32 into eight 8-row column pieces and writes them
// as 16-byte LDS stores into a [column][row] layout (row pitch 72 bf16 = 144 bytes); the
// fragment reads are then 16-byte ds_read_b128 of 8 consecutive rows. Workgroup = 128 (n) x
// 128 (m) tile of one segment, 4 waves of 64 x 64 (2 x 2 MFMA blocks), LDS double-buffered
// (72 KB, two workgroups per CU), the next slab's global loads in flight during the current
// slab's MFMAs. An empty segment's tiles are written as zeros. N and M are multiples of 64: a
// last tile 64 wide reads clamped columns and stores only the columns that exist.
// Split K: with `splits` > 1 each segment's rows are cut into `splits` consecutive chunks of
// whole 64-row slabs, each chunk's tile a workgroup of its own writing fp32 partial sums
// partial[i][s]; sum_splits_kernel then adds the chunks in ascending i (a fixed order, so the
// result does not depend on scheduling) -- for long segments (a shared expert's single segment
// of every token, the router's weight gradient) that would otherwise leave most CUs idle.
#include "common.h"

namespace ntmoe {
namespace {

constexpr int kWT = 128;     // tile edge (n and m)
constexpr int kWK = 64;      // rows per K step
constexpr int kWPitch = 72;  // LDS row pitch of the transposed slabs, bf16 elements
constexpr int kWSlab = kWT * kWPitch;  // one operand's slab, bf16 elements

__device__ __forceinline__ uint32_t lo_pair(uint32_t a, uint32_t b) {
  // low halves of a and b -> (a.lo, b.lo)
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t hi_pair(uint32_t a, uint32_t b) {
  // high halves of a and b -> (a.hi, b.hi)
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// OUT_F32: store fp32 (the split-K partials) instead of bf16.
template <bool OUT_F32>
__global__ __launch_bounds__(256) void grouped_wgrad_kernel(
    const uint16_t* __restrict__ a, int64_t lda, const uint16_t* __restrict__ b, int64_t ldb,
    int64_t b_rows, const int32_t* __restrict__ b_src_row, const int32_t* __restrict__ seg_offsets,
    int num_segments, int64_t total_rows, int N, int M, int splits, void* __restrict__ c) {
  __shared__ __align__(16) uint16_t lds[2][2][kWSlab];  // [buffer][operand A, B][col][row]
  const int ntn = (N + kWT - 1) / kWT, ntm = (M + kWT - 1) / kWT;
  const int per_seg = ntn * ntm;
  const int split = blockIdx.x / (num_segments * per_seg);
  const int rest = blockIdx.x - split * num_segments * per_seg;
  const int s = rest / per_seg;
  const int tile = rest - s * per_seg;
  const int n0 = (tile / ntm) * kWT, m0 = (tile % ntm) * kWT;
  int64_t lo = seg_offsets[s], hi = seg_offsets[s + 1];
  lo = lo < 0 ? 0 : (lo > total_rows ? total_rows : lo);
  hi = hi < lo ? lo : (hi > total_rows ? total_rows : hi);
  if (splits > 1) {  // this chunk: whole 64-row slabs, the last chunk ending at hi
    const int64_t slabs = (hi - lo + kWK - 1) / kWK;
    const int64_t per = (slabs + splits - 1) / splits;
    const int64_t c_lo = lo + split * per * kWK, c_hi = c_lo + per * kWK;
    lo = c_lo < hi ? c_lo : hi;
    hi = c_hi < hi ? c_hi : hi;
  }
  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int wn = wave >> 1, wm = wave & 1;  // the wave's 64 x 64 quarter
  const int64_t c_base = ((int64_t)split * num_segments + s) * N * M;

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.f;

  if (hi > lo) {
    // Loader: threads 0-127 move A, 128-255 move B; thread -> (8-row group rg, 8-column group cg)
    const int op = tid >> 7;
    const int lt = tid & 127;
    // rg varies fastest so a wave's eight 16-byte LDS stores per column land in eight different
    // 16-byte bank groups (columns 8 apart map to the same group)
    const int rg = lt & 7;         // 0..7: rows 8 rg .. 8 rg + 7 of the slab
    const int cg = lt >> 3;        // 0..15: columns 8 cg .. 8 cg + 7 of the tile
    // columns past N (or M) in a 64-wide last tile re-read the last 8 columns; their products
    // land in outputs that are not stored
    const int col = (op == 0 ? n0 : m0) + 8 * cg, width = op == 0 ? N : M;
    const uint16_t* base = (op == 0 ? a : b) + (col < width ? col : width - 8);
    const int64_t ld = op == 0 ? lda : ldb;
    // Gathered B rows: the row indices of a slab are loaded one slab ahead of its data (idx), so
    // the data loads do not wait on an index load.
    const bool gather = op == 1 && b_src_row != nullptr;
    int32_t idx[8];
    auto load_idx = [&](int64_t r0) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int64_t r = r0 + 8 * rg + i;
        idx[i] = b_src_row[r < hi ? r : lo];
      }
    };
    auto load = [&](int64_t r0, u32x4 (&v)[8]) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int64_t r = r0 + 8 * rg + i;
        int64_t row = r < hi ? r : lo;
        if (gather) row = idx[i] < 0 ? 0 : (idx[i] >= b_rows ? b_rows - 1 : idx[i]);
        v[i] = *reinterpret_cast<const u32x4*>(base + row * ld);
        if (r >= hi) v[i] = u32x4{0u, 0u, 0u, 0u};
      }
    };
    auto store = [&](int buf, const u32x4 (&v)[8]) {
      uint16_t* slab = lds[buf][op];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // columns 8 cg + 2 j (low halves) and 8 cg + 2 j + 1 (high halves), rows 8 rg .. + 7
        u32x4 even, odd;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          even[q] = lo_pair(v[2 * q][j], v[2 * q + 1][j]);
          odd[q] = hi_pair(v[2 * q][j], v[2 * q + 1][j]);
        }
        *reinterpret_cast<u32x4*>(slab + (8 * cg + 2 * j) * kWPitch + 8 * rg) = even;
        *reinterpret_cast<u32x4*>(slab + (8 * cg + 2 * j + 1) * kWPitch + 8 * rg) = odd;
      }
    };

    u32x4 v[8];
    if (gather) load_idx(lo);
    load(lo, v);
    if (gather && lo + kWK < hi) load_idx(lo + kWK);
    store(0, v);
    __syncthreads();
    int buf = 0;
    for (int64_t r0 = lo; r0 < hi; r0 += kWK) {
      const bool more = r0 + kWK < hi;
      if (more) load(r0 + kWK, v);
      if (gather && r0 + 2 * kWK < hi) load_idx(r0 + 2 * kWK);
      const uint16_t* sa = lds[buf][0];
      const uint16_t* sb = lds[buf][1];
#pragma unroll
      for (int kk = 0; kk < kWK / 16; ++kk) {
        const int koff = kk * 16 + (lane >> 5) * 8;
        bf16x8 fa[2], fb[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          fa[i] = *reinterpret_cast<const bf16x8*>(sa + (64 * wn + 32 * i + (lane & 31)) * kWPitch + koff);
          fb[i] = *reinterpret_cast<const bf16x8*>(sb + (64 * wm + 32 * i + (lane & 31)) * kWPitch + koff);
        }
        // D[m][n] += B-side (m x k) . A-side (k x n): lane holds column n, runs of 4 rows m
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[j], fa[i], acc[i][j], 0, 0, 0);
      }
      if (more) store(buf ^ 1, v);
      __syncthreads();
      buf ^= 1;
    }
  }
  // acc[i][j]: n = n0 + 64 wn + 32 i + lane % 32, m = m0 + 64 wm + 32 j + 8 (q / 4) + 4 (lane / 32) + q % 4
  // (a 64-wide last tile: the quarter past N or M is not stored)
  if (n0 + 64 * wn >= N || m0 + 64 * wm >= M) return;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int n = n0 + 64 * wn + 32 * i + (lane & 31);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int m = m0 + 64 * wm + 32 * j + 8 * g + 4 * (lane >> 5);
        const int64_t off = c_base + (int64_t)n * M + m;
        if constexpr (OUT_F32) {
          const floatx4 o = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                             acc[i][j][4 * g + 3]};
          *reinterpret_cast<floatx4*>(reinterpret_cast<float*>(c) + off) = o;
        } else {
          u32x2 o;
          o[0] = pack_bf16x2(acc[i][j][4 * g], acc[i][j][4 * g + 1]);
          o[1] = pack_bf16x2(acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]);
          *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(c) + off) = o;
        }
      }
    }
  }
}

// out[j] = sum over i = 0, 1, ..., splits - 1 (in that order) of partial[i][j], fp32, stored as
// fp32 or rounded once to bf16; 4 consecutive elements per thread.
template <bool OUT_F32>
__global__ __launch_bounds__(256) void sum_splits_kernel(const float* __restrict__ partial,
                                                         int splits, int64_t count,
                                                         void* __restrict__ out) {
  const int64_t j = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (j >= count) return;
  floatx4 v = *reinterpret_cast<const floatx4*>(partial + j);
  for (int i = 1; i < splits; ++i) v = v + *reinterpret_cast<const floatx4*>(partial + i * count + j);
  if constexpr (OUT_F32) {
    *reinterpret_cast<floatx4*>(reinterpret_cast<float*>(out) + j) = v;
  } else {
    const u32x2 o = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(out) + j) = o;
  }
}

}  // namespace

hipError_t launch_grouped_wgrad(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                                int64_t b_rows, const int32_t* b_src_row,
                                const int32_t* seg_offsets, int num_segments, int64_t total_rows,
                                int N, int M, int splits, float* partial, bool c_f32, void* c,
                                hipStream_t stream) {
  const int64_t tiles = (int64_t)num_segments * ((N + kWT - 1) / kWT) * ((M + kWT - 1) / kWT);
  if (tiles == 0) return hipSuccess;
  if (splits <= 1) {
    auto kern = c_f32 ? grouped_wgrad_kernel<true> : grouped_wgrad_kernel<false>;
    hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(256), 0, stream, a, lda, b, ldb, b_rows,
                       b_src_row, seg_offsets, num_segments, total_rows, N, M, 1, c);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(grouped_wgrad_kernel<true>, dim3((unsigned)(tiles * splits)), dim3(256), 0,
                     stream, a, lda, b, ldb, b_rows, b_src_row, seg_offsets, num_segments,
                     total_rows, N, M, splits, static_cast<void*>(partial));
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  const int64_t count = (int64_t)num_segments * N * M;  // a multiple of 4096
  auto sum = c_f32 ? sum_splits_kernel<true> : sum_splits_kernel<false>;
  hipLaunchKernelGGL(sum, dim3((unsigned)((count / 4 + 255) / 256)), dim3(256), 0, stream,
                     partial, splits, count, c);
  return hipGetLastError();
}

}  // namespace ntmoe
