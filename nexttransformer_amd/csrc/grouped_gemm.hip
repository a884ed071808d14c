// Grouped expert FFN on bf16 MFMA (gfx950 v_mfma_f32_32x32x16_bf16), fp32 accumulation.
//
// Replaces SequentialMLP's per-expert loop (nexttransformer/scaling/megatron_moe.py:145) over
// MasterLinear fc1 -> activation -> fc2 (megatron_moe.py:58-78, :23-24; lm.py:29-35). Two
// launches of one kernel template:
//   up   : h[r, :] = act(a[src(r)] . W1_s^T)   gather fused into the A loads, SwiGLU/ReLU^2
//          fused into the epilogue (W1_s rows [0,H) gate, [H,2H) value)
//   down : y[r, :] = h[r] . W2_s^T
// over ragged segments s (experts) with rows [seg_offsets[s], seg_offsets[s+1]).
//
// Scheduling. The kernel is persistent: every workgroup reads seg_offsets, builds the tile
// prefix in LDS, and walks a static share of the tile list (segment-major, then m, then n).
// The tile list is cut into 8 contiguous ranges, one per XCD (workgroup b runs on XCD b % 8),
// so the tiles of one expert -- which share its weights -- stay in one L2.
//
// Tile. BM x BN x BK with WM x WN waves. The MFMA is issued with the weight fragment as the
// "A" operand and the activation fragment as "B", so a lane's 16 accumulators are 4 runs of 4
// consecutive output columns of one row: stores are 8-byte packed bf16. Both tiles are staged
// through LDS, double buffered, as 16-byte chunks XOR-swizzled by (row & 7) so the 32-row
// fragment reads are bank-conflict free.
//
// SwiGLU pairing: the BN weight rows of a tile are laid out per wave as [gate half | value
// half] of the same BN/(2 WN) hidden columns, so gate and value of one output element land in
// the same lane and the epilogue needs no exchange.
#include <math.h>

#include "common.h"

namespace ntmoe {
namespace {

enum Epilogue { kEpiSwiglu = 0, kEpiRelu2 = 1, kEpiPlain = 2 };

template <int BM, int BN, int BK, int WM, int WN, int EPI, bool GATHER>
struct Gemm {
  static constexpr int kThreads = WM * WN * 64;
  static constexpr int kWaveM = BM / WM, kWaveN = BN / WN;
  static constexpr int TM = kWaveM / 32, TN = kWaveN / 32;
  static constexpr int kChunks = BK / 8;  // 16-byte chunks per tile row
  static constexpr int kAPer = BM * kChunks / kThreads;
  static constexpr int kBPer = BN * kChunks / kThreads;
  static constexpr int kBNOut = EPI == kEpiSwiglu ? BN / 2 : BN;  // output columns per tile
  static constexpr int kStageBytes = (BM + BN) * BK * 2;
  static_assert(BK == 64, "swizzle assumes 8 chunks per row");
  static_assert(kAPer * kThreads == BM * kChunks && kBPer * kThreads == BN * kChunks, "tiling");
  static_assert(EPI != kEpiSwiglu || TN % 2 == 0, "SwiGLU needs gate and value tiles per wave");
};

__device__ __forceinline__ int swz(int row, int chunk) { return row * 8 + (chunk ^ (row & 7)); }

template <int BM, int BN, int BK, int WM, int WN, int EPI, bool GATHER>
__global__ __launch_bounds__(WM * WN * 64) void grouped_gemm_kernel(
    const uint16_t* __restrict__ A, int64_t ld_a, const int32_t* __restrict__ src_row,
    const int32_t* __restrict__ seg_offsets, int S, int total_rows, int64_t a_rows,
    const uint16_t* __restrict__ W, int64_t w_seg_stride, int K, int n_out, int H,
    uint16_t* __restrict__ C) {
  using G = Gemm<BM, BN, BK, WM, WN, EPI, GATHER>;
  extern __shared__ __align__(16) unsigned char smem[];
  u32x4* stage_base = reinterpret_cast<u32x4*>(smem);
  int* tile_prefix = reinterpret_cast<int*>(smem + 2 * G::kStageBytes);  // [S+1]

  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int wm = wave / WN, wn = wave % WN;
  const int n_tiles = (n_out + G::kBNOut - 1) / G::kBNOut;

  // Segment bounds are clamped to [0, total_rows] and made non-decreasing, so malformed
  // offsets can only produce wrong rows, never out-of-bounds accesses.
  int* seg_lo = tile_prefix + (S + 1);
  if (tid == 0) {
    int run = 0, prev = 0;
    tile_prefix[0] = 0;
    for (int s = 0; s <= S; ++s) {
      int o = seg_offsets[s];
      o = o < prev ? prev : (o > total_rows ? total_rows : o);
      seg_lo[s] = o;
      if (s > 0) {
        run += ((o - prev + BM - 1) / BM) * n_tiles;
        tile_prefix[s] = run;
      }
      prev = o;
    }
  }
  __syncthreads();
  const int total = tile_prefix[S];
  const int G8 = gridDim.x / 8;
  const int xcd = blockIdx.x % 8, local = blockIdx.x / 8;
  const int t_begin = (int)((int64_t)total * xcd / 8);
  const int t_end = (int)((int64_t)total * (xcd + 1) / 8);
  const int nk = K / BK;

  for (int tile = t_begin + local; tile < t_end; tile += G8) {
    // Segment by binary search over the tile prefix.
    int lo = 0, hi = S;
    while (hi - lo > 1) {
      int mid = (lo + hi) >> 1;
      if (tile_prefix[mid] <= tile) lo = mid; else hi = mid;
    }
    const int s = lo;
    const int ltile = tile - tile_prefix[s];
    const int mt = ltile / n_tiles, nt = ltile - mt * n_tiles;
    const int seg_begin = seg_lo[s], seg_end = seg_lo[s + 1];
    const int m0 = seg_begin + mt * BM;
    const uint16_t* Ws = W + (int64_t)s * w_seg_stride;

    // Per-thread global row pointers for the A and B tile loads.
    const uint16_t* a_ptr[G::kAPer];
    const uint16_t* b_ptr[G::kBPer];
    int a_lds[G::kAPer], b_lds[G::kBPer];
#pragma unroll
    for (int q = 0; q < G::kAPer; ++q) {
      int id = q * G::kThreads + tid, row = id / G::kChunks, c = id % G::kChunks;
      int gr = m0 + row;
      gr = gr < seg_end ? gr : seg_end - 1;
      int64_t src = GATHER ? (int64_t)src_row[gr] : (int64_t)gr;
      src = src < 0 ? 0 : (src >= a_rows ? a_rows - 1 : src);
      a_ptr[q] = A + src * ld_a + c * 8;
      a_lds[q] = swz(row, c);
    }
#pragma unroll
    for (int q = 0; q < G::kBPer; ++q) {
      int id = q * G::kThreads + tid, row = id / G::kChunks, c = id % G::kChunks;
      int wrow;
      if (EPI == kEpiSwiglu) {
        int slot = row / G::kWaveN, qq = row % G::kWaveN, half = G::kWaveN / 2;
        int hcol = nt * G::kBNOut + slot * half + (qq % half);
        hcol = hcol < H ? hcol : H - 1;  // partial N tile: clamp, results are not stored
        wrow = qq < half ? hcol : H + hcol;
      } else {
        wrow = nt * BN + row;
        wrow = wrow < n_out ? wrow : n_out - 1;
      }
      b_ptr[q] = Ws + (int64_t)wrow * K + c * 8;
      b_lds[q] = BM * 8 + swz(row, c);
    }

    floatx16 acc[G::TN][G::TM];
#pragma unroll
    for (int i = 0; i < G::TN; ++i)
#pragma unroll
      for (int j = 0; j < G::TM; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    u32x4 ra[G::kAPer], rb[G::kBPer];
#pragma unroll
    for (int q = 0; q < G::kAPer; ++q) ra[q] = *reinterpret_cast<const u32x4*>(a_ptr[q]);
#pragma unroll
    for (int q = 0; q < G::kBPer; ++q) rb[q] = *reinterpret_cast<const u32x4*>(b_ptr[q]);
#pragma unroll
    for (int q = 0; q < G::kAPer; ++q) stage_base[a_lds[q]] = ra[q];
#pragma unroll
    for (int q = 0; q < G::kBPer; ++q) stage_base[b_lds[q]] = rb[q];
    __syncthreads();

    for (int kt = 0; kt < nk; ++kt) {
      const int cur = kt & 1;
      const bool more = kt + 1 < nk;
      if (more) {
        const int koff = (kt + 1) * BK;
#pragma unroll
        for (int q = 0; q < G::kAPer; ++q) ra[q] = *reinterpret_cast<const u32x4*>(a_ptr[q] + koff);
#pragma unroll
        for (int q = 0; q < G::kBPer; ++q) rb[q] = *reinterpret_cast<const u32x4*>(b_ptr[q] + koff);
      }
      const u32x4* st = stage_base + cur * (G::kStageBytes / 16);
#pragma unroll
      for (int ks = 0; ks < BK / 16; ++ks) {
        const int chunk = 2 * ks + (lane >> 5);
        bf16x8 fa[G::TM], fb[G::TN];
#pragma unroll
        for (int j = 0; j < G::TM; ++j) {
          int row = wm * G::kWaveM + j * 32 + (lane & 31);
          fa[j] = __builtin_bit_cast(bf16x8, st[swz(row, chunk)]);
        }
#pragma unroll
        for (int i = 0; i < G::TN; ++i) {
          int row = wn * G::kWaveN + i * 32 + (lane & 31);
          fb[i] = __builtin_bit_cast(bf16x8, st[BM * 8 + swz(row, chunk)]);
        }
#pragma unroll
        for (int i = 0; i < G::TN; ++i)
#pragma unroll
          for (int j = 0; j < G::TM; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[i], fa[j], acc[i][j], 0, 0, 0);
      }
      if (more) {
        u32x4* nx = stage_base + (cur ^ 1) * (G::kStageBytes / 16);
#pragma unroll
        for (int q = 0; q < G::kAPer; ++q) nx[a_lds[q]] = ra[q];
#pragma unroll
        for (int q = 0; q < G::kBPer; ++q) nx[b_lds[q]] = rb[q];
      }
      __syncthreads();
    }

    // Epilogue: lane holds rows m = ... + (lane & 31), columns n = 8 (e/4) + 4 (lane/32) + e%4.
    constexpr int kOutTN = EPI == kEpiSwiglu ? G::TN / 2 : G::TN;
    const int col_base = EPI == kEpiSwiglu ? nt * G::kBNOut + wn * (G::kWaveN / 2)
                                           : nt * BN + wn * G::kWaveN;
#pragma unroll
    for (int j = 0; j < G::TM; ++j) {
      const int m = m0 + wm * G::kWaveM + j * 32 + (lane & 31);
      if (m >= seg_end) continue;
      uint16_t* crow = C + (int64_t)m * n_out;
#pragma unroll
      for (int i = 0; i < kOutTN; ++i) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float a = acc[i][j][g * 4 + e];
            if (EPI == kEpiSwiglu) {
              float u = acc[i + kOutTN][j][g * 4 + e];
              v[e] = a / (1.f + expf(-a)) * u;
            } else if (EPI == kEpiRelu2) {
              float r = a > 0.f ? a : 0.f;
              v[e] = r * r;
            } else {
              v[e] = a;
            }
          }
          const int n = col_base + i * 32 + g * 8 + (lane >> 5) * 4;
          if (n >= n_out) continue;
          uint2 packed;
          packed.x = pack_bf16x2(v[0], v[1]);
          packed.y = pack_bf16x2(v[2], v[3]);
          *reinterpret_cast<uint2*>(crow + n) = packed;
        }
      }
    }
  }
}

template <int BM, int BN, int BK, int WM, int WN, int EPI, bool GATHER>
hipError_t launch_gemm(const uint16_t* A, int64_t ld_a, int64_t a_rows, const int32_t* src_row,
                       const int32_t* seg_offsets, int S, int64_t total_rows, const uint16_t* W,
                       int64_t w_seg_stride, int K, int n_out, int H, uint16_t* C,
                       hipStream_t stream) {
  using G = Gemm<BM, BN, BK, WM, WN, EPI, GATHER>;
  const int64_t n_tiles = (n_out + G::kBNOut - 1) / G::kBNOut;
  const int64_t upper = ((total_rows + BM - 1) / BM + S) * n_tiles;
  int64_t grid = (int64_t)num_cus() * 2;
  if (upper < grid) grid = upper;
  grid = ((grid + 7) / 8) * 8;
  if (grid == 0) return hipSuccess;
  size_t lds = 2 * G::kStageBytes + (size_t)(2 * S + 2) * sizeof(int);
  auto kern = grouped_gemm_kernel<BM, BN, BK, WM, WN, EPI, GATHER>;
  hipError_t err = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds);
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(G::kThreads), lds, stream, A, ld_a,
                     src_row, seg_offsets, S, (int)total_rows, a_rows, W, w_seg_stride, K,
                     n_out, H, C);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_grouped_ffn_bf16(const uint16_t* a, int64_t ld_a, int64_t a_rows,
                                   const int32_t* src_row,
                                   const int32_t* seg_offsets, int num_segments,
                                   int64_t total_rows, const uint16_t* w1, const uint16_t* w2,
                                   int d, int H, int activation, uint16_t* h, uint16_t* y,
                                   hipStream_t stream) {
  constexpr int BM = 128, BN = 128, BK = 64, WM = 2, WN = 2;
  hipError_t err;
  if (activation == NT_MOE_ACT_SWIGLU) {
    const int64_t stride = (int64_t)2 * H * d;
    err = src_row ? launch_gemm<BM, BN, BK, WM, WN, kEpiSwiglu, true>(
                        a, ld_a, a_rows, src_row, seg_offsets, num_segments, total_rows, w1, stride, d,
                        H, H, h, stream)
                  : launch_gemm<BM, BN, BK, WM, WN, kEpiSwiglu, false>(
                        a, ld_a, a_rows, src_row, seg_offsets, num_segments, total_rows, w1, stride, d,
                        H, H, h, stream);
  } else {
    const int64_t stride = (int64_t)H * d;
    err = src_row ? launch_gemm<BM, BN, BK, WM, WN, kEpiRelu2, true>(
                        a, ld_a, a_rows, src_row, seg_offsets, num_segments, total_rows, w1, stride, d,
                        H, H, h, stream)
                  : launch_gemm<BM, BN, BK, WM, WN, kEpiRelu2, false>(
                        a, ld_a, a_rows, src_row, seg_offsets, num_segments, total_rows, w1, stride, d,
                        H, H, h, stream);
  }
  if (err != hipSuccess) return err;
  return launch_gemm<BM, BN, BK, WM, WN, kEpiPlain, false>(
      h, H, total_rows, nullptr, seg_offsets, num_segments, total_rows, w2, (int64_t)d * H, H, d, H, y,
      stream);
}

}  // namespace ntmoe
