// FP8 (OCP E4M3FN) path of the MoE layer on gfx950: quantisation kernels and a block-scaled
// grouped expert GEMM for the small-batch, weight-streaming regime.
//
// Numerics (the fp8 variant of SequentialMLP's expert loop, megatron_moe.py:145, with weights
// stored as e4m3 and one fp32 scale per 128 x 128 block, activations quantised per row):
//   row scale      s = amax(|row|) / 448 (1 for an all-zero row); q = e4m3_rne(v / s)
//   block scale    the same per 128 x 128 block of a weight matrix
//   GEMM           c[r, j] = epi( a_scale[row(r)] * sum_kb w_scale[s, j/128, kb] *
//                                  sum_{k in block kb} e4m3(a[row(r), k]) * e4m3(w[s, j, k]) )
// The inner 128-wide block sums run on v_mfma_scale_f32_32x32x64_f8f6f4 (both formats e4m3,
// E8M0 scales fixed at 2^0) into a zeroed fp32 fragment, which is then scaled and added to the
// fp32 accumulator: the block scales are arbitrary fp32 values, not powers of two, so they are
// applied outside the matrix core.
//
// GEMM shape. The regime this kernel is for (a few rows per expert, e.g. T = 64 tokens over
// 128 experts) is bound by streaming the weights from HBM once, so the kernel streams: a
// workgroup owns one (segment, column tile) pair, each of its 4 waves a 32-row slice of the
// weight matrix, and every weight byte is loaded exactly once per 32 rows of the segment. The
// segment's activation rows (gathered through src_row) are the MFMA's B operand, read from L2.
// A lane holds 32 consecutive K bytes of its weight row for a 64-wide K step (bytes
// [32 * (lane / 32), +32)); the activation operand uses the same byte mapping, so whatever
// order the matrix core assigns those bytes to, both operands agree and the dot product is
// exact up to fp32 accumulation order. The next 128-wide K block is loaded while the current
// one is multiplied.
// SwiGLU tiles pair 16 gate rows with the 16 value rows of the same output columns in one MFMA
// (A rows 0-15 gate, 16-31 value), so both land in the same lane of the accumulator layout
// (row i of a 32 x 32 fragment sits in lane (i / 4) % 2 * 32 + column, element (i / 8) * 4 + i % 4).
#include <math.h>
#include <stdlib.h>

#include "common.h"

namespace ntmoe {
namespace {

constexpr float kE4m3Max = 448.0f;
constexpr int kScaleBlock = 128;
constexpr int kScaleOne = 127;  // E8M0 encoding of 2^0

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

// Four fp32 values -> four e4m3 bytes (round to nearest even), little-endian in one word.
__device__ __forceinline__ uint32_t to_e4m3x4(float a, float b, float c, float d) {
  int packed = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  packed = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, packed, true);
  return (uint32_t)packed;
}

__device__ __forceinline__ float row_scale(float amax) {
  return amax > 0.f ? amax / kE4m3Max : 1.f;
}

// One wave per row: amax over the row, then q = e4m3(v / s). d % 8 == 0.
__global__ __launch_bounds__(256) void quantize_rowwise_kernel(
    const uint16_t* __restrict__ x, int64_t ld_x, int64_t rows, int d, uint8_t* __restrict__ q,
    int64_t ld_q, float* __restrict__ scale) {
  const int64_t row = (int64_t)blockIdx.x * 4 + wave_id();
  if (row >= rows) return;
  const int lane = lane_id();
  const uint16_t* xr = x + row * ld_x;
  float amax = 0.f;
  for (int c = lane * 8; c < d; c += 512) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(xr + c);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      amax = fmaxf(amax, fabsf(bf16_bits_to_f32(v[i] & 0xffffu)));
      amax = fmaxf(amax, fabsf(bf16_bits_to_f32(v[i] >> 16)));
    }
  }
  const float s = row_scale(wave_max(amax));
  uint8_t* qr = q + row * ld_q;
  for (int c = lane * 8; c < d; c += 512) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(xr + c);
    float f[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = bf16_bits_to_f32(v[i] & 0xffffu) / s;
      f[2 * i + 1] = bf16_bits_to_f32(v[i] >> 16) / s;
    }
    u32x2 out;
    out[0] = to_e4m3x4(f[0], f[1], f[2], f[3]);
    out[1] = to_e4m3x4(f[4], f[5], f[6], f[7]);
    *reinterpret_cast<u32x2*>(qr + c) = out;
  }
  if (lane == 0) scale[row] = s;
}

// One 256-thread workgroup per 128 x 128 block of w [S, R, C] (fp32 masters).
__global__ __launch_bounds__(256) void quantize_blockwise_kernel(
    const float* __restrict__ w, int R, int C, uint8_t* __restrict__ q, float* __restrict__ scale) {
  __shared__ float part[4];
  const int cb_count = C / kScaleBlock, rb_count = R / kScaleBlock;
  const int64_t blk = blockIdx.x;
  const int cb = (int)(blk % cb_count);
  const int rb = (int)((blk / cb_count) % rb_count);
  const int64_t s = blk / ((int64_t)cb_count * rb_count);
  const int t = threadIdx.x;
  const int col = cb * kScaleBlock + (t & 31) * 4;  // 32 threads x 4 columns per row
  const int64_t base = (s * R + (int64_t)rb * kScaleBlock) * C + col;
  float amax = 0.f;
  for (int r = t >> 5; r < kScaleBlock; r += 8) {
    const floatx4 v = *reinterpret_cast<const floatx4*>(w + base + (int64_t)r * C);
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
  }
  amax = wave_max(amax);
  if (lane_id() == 0) part[wave_id()] = amax;
  __syncthreads();
  const float sc = row_scale(fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3])));
  for (int r = t >> 5; r < kScaleBlock; r += 8) {
    const floatx4 v = *reinterpret_cast<const floatx4*>(w + base + (int64_t)r * C);
    *reinterpret_cast<uint32_t*>(q + base + (int64_t)r * C) =
        to_e4m3x4(v[0] / sc, v[1] / sc, v[2] / sc, v[3] / sc);
  }
  if (t == 0) scale[blk] = sc;
}

template <int EPI>
struct Fp8Tile {
  // output columns per wave / per workgroup
  static constexpr int kColsPerWave = EPI == NT_MOE_EPI_SWIGLU ? 16 : 32;
  static constexpr int kColsPerBlock = 4 * kColsPerWave;
};

__device__ __forceinline__ float silu_mul(float g, float u) {
  return g * u * __builtin_amdgcn_rcpf(1.f + __expf(-g));
}

// D: K blocks of weights in flight per wave beyond the one being multiplied (a register ring of
// D + 1 blocks). The kernel streams weights, so bytes in flight per CU set its bandwidth.
template <int EPI, bool PACKED, int D>
__global__ __launch_bounds__(256) void fp8_grouped_gemm_kernel(
    const uint8_t* __restrict__ a, int64_t ld_a, int64_t a_rows, const float* __restrict__ a_scale,
    const int32_t* __restrict__ src_row, const int32_t* __restrict__ seg_offsets,
    int64_t total_rows, const uint8_t* __restrict__ w, const float* __restrict__ w_scale, int K,
    int n_out, int n_tiles, uint16_t* __restrict__ c) {
  using Tile = Fp8Tile<EPI>;
  const int seg = blockIdx.x / n_tiles;
  const int tile = blockIdx.x - seg * n_tiles;
  int64_t lo = seg_offsets[seg], hi = seg_offsets[seg + 1];
  lo = lo < 0 ? 0 : (lo > total_rows ? total_rows : lo);
  hi = hi < lo ? lo : (hi > total_rows ? total_rows : hi);
  if (hi <= lo) return;
  const int wave = wave_id(), lane = lane_id();
  const int li = lane & 31, half = lane >> 5;
  const int col0 = tile * Tile::kColsPerBlock + wave * Tile::kColsPerWave;
  if (col0 >= n_out) return;  // no barriers below: a wave past the last column just leaves

  const int w_rows = EPI == NT_MOE_EPI_SWIGLU ? 2 * n_out : n_out;
  const int scale_rows = (w_rows + kScaleBlock - 1) / kScaleBlock;
  const int kblocks = K / kScaleBlock;
  int wrow;
  if (EPI == NT_MOE_EPI_SWIGLU)
    wrow = li < 16 ? col0 + li : n_out + col0 + (li - 16);
  else
    wrow = col0 + li;
  const bool wvalid = EPI == NT_MOE_EPI_SWIGLU ? (col0 + (li & 15) < n_out) : (wrow < n_out);
  // Unpacked: row wrow of the segment's [R, K] matrix, this lane's 32 bytes of each 64-wide step.
  // Packed: the wave's 32-row group nb is a run of 4 KB blocks (one per 128-wide K block) in
  // which the two 16-byte chunks of lane l for step st sit at ((2 st + h) * 64 + l) * 16.
  const uint8_t* wp;
  int64_t w_step;  // bytes from one 128-wide K block to the next
  if (PACKED) {
    const int nb = col0 / Tile::kColsPerWave;
    wp = w + (((int64_t)seg * (w_rows / 32) + nb) * kblocks) * 4096 + lane * 16;
    w_step = 4096;
  } else {
    wp = w + ((int64_t)seg * w_rows + (wvalid ? wrow : col0)) * K + half * 32;
    w_step = kScaleBlock;
  }
  // One K block = four 16-byte loads of weights and four of activations per lane, issued from
  // inline assembly: the compiler neither counts them nor adds its own (conservative, loop-
  // merged) waits; the explicit wait before a block is used names that block's registers, so
  // no use of them, and no copy, can be scheduled above it. Weights: packed, bytes
  // {0, 1024, 2048, 3072} of the block's 4 KB run; plain, bytes {0, 16, 64, 80} of the lane's
  // row at K offset 128 kb. Activations: bytes {0, 16, 64, 80} of the token row at 128 kb.
  auto load4 = [&](const uint8_t* p, bool wide, u32x4 (&r)[4]) {
    if (wide) {
      asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r[0]) : "v"(p) : "memory");
      asm volatile("global_load_dwordx4 %0, %1, off offset:1024" : "=v"(r[1]) : "v"(p) : "memory");
      asm volatile("global_load_dwordx4 %0, %1, off offset:2048" : "=v"(r[2]) : "v"(p) : "memory");
      asm volatile("global_load_dwordx4 %0, %1, off offset:3072" : "=v"(r[3]) : "v"(p) : "memory");
    } else {
      asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r[0]) : "v"(p) : "memory");
      asm volatile("global_load_dwordx4 %0, %1, off offset:16" : "=v"(r[1]) : "v"(p) : "memory");
      asm volatile("global_load_dwordx4 %0, %1, off offset:64" : "=v"(r[2]) : "v"(p) : "memory");
      asm volatile("global_load_dwordx4 %0, %1, off offset:80" : "=v"(r[3]) : "v"(p) : "memory");
    }
  };
  // scale rows of the gate (or only) half and of the value half
  const float* ws_lo = w_scale + ((int64_t)seg * scale_rows + col0 / kScaleBlock) * kblocks;
  const float* ws_hi =
      EPI == NT_MOE_EPI_SWIGLU
          ? w_scale + ((int64_t)seg * scale_rows + (n_out + col0) / kScaleBlock) * kblocks
          : ws_lo;

  for (int64_t t0 = lo; t0 < hi; t0 += 32) {
    const int64_t tok = t0 + li;
    const bool tvalid = tok < hi;
    int64_t arow = tok;
    if (src_row) arow = tvalid ? (int64_t)src_row[tok] : 0;
    arow = arow < 0 ? 0 : (arow >= a_rows ? a_rows - 1 : arow);
    const uint8_t* ap = a + arow * ld_a + half * 32;

    // Ring of D + 1 K blocks: slot kb % (D + 1) holds block kb's weights (wq) and activations
    // (xq). Every step issues one block (past the last one it re-reads the last; a token past
    // the segment reads a valid row whose results are not stored), so the number of loads
    // issued after block kb is always 8 D when block kb is needed.
    u32x4 wq[D + 1][4], xq[D + 1][4];
    auto issue = [&](int kb, int slot_unused, u32x4 (&w4)[4], u32x4 (&x4)[4]) {
      (void)slot_unused;
      const int kc = kb < kblocks ? kb : kblocks - 1;
      load4(wp + (int64_t)kc * w_step, PACKED, w4);
      load4(ap + (int64_t)kc * kScaleBlock, false, x4);
    };
#pragma unroll
    for (int j = 0; j < D; ++j) issue(j, j, wq[j], xq[j]);
    floatx16 acc = {};
    for (int kb0 = 0; kb0 < kblocks; kb0 += D + 1) {
#pragma unroll
      for (int u = 0; u <= D; ++u) {
        const int kb = kb0 + u;
        issue(kb + D, (u + D) % (D + 1), wq[(u + D) % (D + 1)], xq[(u + D) % (D + 1)]);
        asm volatile("s_waitcnt vmcnt(%8)"
                     : "+v"(wq[u][0]), "+v"(wq[u][1]), "+v"(wq[u][2]), "+v"(wq[u][3]),
                       "+v"(xq[u][0]), "+v"(xq[u][1]), "+v"(xq[u][2]), "+v"(xq[u][3])
                     : "n"(8 * D)
                     : "memory");
        if (kb >= kblocks) continue;  // the ring's trailing re-reads (uniform)
        const i32x8 w0 = {(int)wq[u][0][0], (int)wq[u][0][1], (int)wq[u][0][2], (int)wq[u][0][3],
                          (int)wq[u][1][0], (int)wq[u][1][1], (int)wq[u][1][2], (int)wq[u][1][3]};
        const i32x8 w1 = {(int)wq[u][2][0], (int)wq[u][2][1], (int)wq[u][2][2], (int)wq[u][2][3],
                          (int)wq[u][3][0], (int)wq[u][3][1], (int)wq[u][3][2], (int)wq[u][3][3]};
        const i32x8 x0 = {(int)xq[u][0][0], (int)xq[u][0][1], (int)xq[u][0][2], (int)xq[u][0][3],
                          (int)xq[u][1][0], (int)xq[u][1][1], (int)xq[u][1][2], (int)xq[u][1][3]};
        const i32x8 x1 = {(int)xq[u][2][0], (int)xq[u][2][1], (int)xq[u][2][2], (int)xq[u][2][3],
                          (int)xq[u][3][0], (int)xq[u][3][1], (int)xq[u][3][2], (int)xq[u][3][3]};
        floatx16 part = {};
        part = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(w0, x0, part, 0, 0, 0, kScaleOne,
                                                               0, kScaleOne);
        part = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(w1, x1, part, 0, 0, 0, kScaleOne,
                                                               0, kScaleOne);
        const float s_lo = ws_lo[kb], s_hi = ws_hi[kb];
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = fmaf(part[i], i < 8 ? s_lo : s_hi, acc[i]);
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the ring's last re-reads
    if (!tvalid) continue;
    const float as = a_scale[arow];
    uint16_t* crow = c + tok * n_out;
    if (EPI == NT_MOE_EPI_SWIGLU) {
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const int col = col0 + 8 * g + 4 * half;
        if (col >= n_out) continue;
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = silu_mul(as * acc[4 * g + r], as * acc[4 * (g + 2) + r]);
        u32x2 v;
        v[0] = pack_bf16x2(o[0], o[1]);
        v[1] = pack_bf16x2(o[2], o[3]);
        *reinterpret_cast<u32x2*>(crow + col) = v;
      }
    } else {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int col = col0 + 8 * g + 4 * half;
        if (col >= n_out) continue;
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float v = as * acc[4 * g + r];
          if (EPI == NT_MOE_EPI_RELU2) v = v > 0.f ? v * v : 0.f;
          o[r] = v;
        }
        u32x2 v;
        v[0] = pack_bf16x2(o[0], o[1]);
        v[1] = pack_bf16x2(o[2], o[3]);
        *reinterpret_cast<u32x2*>(crow + col) = v;
      }
    }
  }
}

}  // namespace

hipError_t launch_quantize_fp8_rowwise(const uint16_t* x, int64_t ld_x, int64_t rows, int d,
                                       uint8_t* q, int64_t ld_q, float* scale, hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  quantize_rowwise_kernel<<<dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream>>>(
      x, ld_x, rows, d, q, ld_q, scale);
  return hipGetLastError();
}

hipError_t launch_quantize_fp8_blockwise(const float* w, int64_t S, int R, int C, uint8_t* q,
                                         float* scale, hipStream_t stream) {
  const int64_t blocks = S * (R / kScaleBlock) * (C / kScaleBlock);
  if (blocks == 0) return hipSuccess;
  quantize_blockwise_kernel<<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(w, R, C, q, scale);
  return hipGetLastError();
}

// Weight blocks in flight per wave (NT_MOE_FP8_DEPTH overrides, for tuning runs).
int fp8_weight_depth() {
  static int n = [] {
    const char* s = getenv("NT_MOE_FP8_DEPTH");
    int v = s ? atoi(s) : 0;
    return v >= 1 && v <= 3 ? v : 2;
  }();
  return n;
}

template <int EPI, bool P>
hipError_t launch_fp8(dim3 grid, hipStream_t stream, const uint8_t* a, int64_t ld_a,
                      int64_t a_rows, const float* a_scale, const int32_t* src_row,
                      const int32_t* seg_offsets, int64_t total_rows, const uint8_t* w,
                      const float* w_scale, int K, int n_out, int n_tiles, uint16_t* c) {
  const dim3 block(256);
  switch (fp8_weight_depth()) {
    case 1:
      fp8_grouped_gemm_kernel<EPI, P, 1><<<grid, block, 0, stream>>>(
          a, ld_a, a_rows, a_scale, src_row, seg_offsets, total_rows, w, w_scale, K, n_out,
          n_tiles, c);
      break;
    case 2:
      fp8_grouped_gemm_kernel<EPI, P, 2><<<grid, block, 0, stream>>>(
          a, ld_a, a_rows, a_scale, src_row, seg_offsets, total_rows, w, w_scale, K, n_out,
          n_tiles, c);
      break;
    default:
      fp8_grouped_gemm_kernel<EPI, P, 3><<<grid, block, 0, stream>>>(
          a, ld_a, a_rows, a_scale, src_row, seg_offsets, total_rows, w, w_scale, K, n_out,
          n_tiles, c);
      break;
  }
  return hipGetLastError();
}

hipError_t launch_grouped_gemm_fp8(const uint8_t* a, int64_t ld_a, int64_t a_rows,
                                   const float* a_scale, const int32_t* src_row,
                                   const int32_t* seg_offsets, int num_segments,
                                   int64_t total_rows, const uint8_t* w, const float* w_scale,
                                   int K, int n_out, int epilogue, bool packed, uint16_t* c,
                                   hipStream_t stream) {
  const int per_block = epilogue == NT_MOE_EPI_SWIGLU ? Fp8Tile<NT_MOE_EPI_SWIGLU>::kColsPerBlock
                                                      : Fp8Tile<NT_MOE_EPI_NONE>::kColsPerBlock;
  const int n_tiles = ceil_div(n_out, per_block);
  const dim3 grid((unsigned)((int64_t)num_segments * n_tiles));
  if (total_rows == 0) return hipSuccess;
#define NT_F8_ARGS grid, stream, a, ld_a, a_rows, a_scale, src_row, seg_offsets, total_rows, w, \
                   w_scale, K, n_out, n_tiles, c
  switch (epilogue) {
    case NT_MOE_EPI_SWIGLU:
      return packed ? launch_fp8<NT_MOE_EPI_SWIGLU, true>(NT_F8_ARGS)
                    : launch_fp8<NT_MOE_EPI_SWIGLU, false>(NT_F8_ARGS);
    case NT_MOE_EPI_RELU2:
      return packed ? launch_fp8<NT_MOE_EPI_RELU2, true>(NT_F8_ARGS)
                    : launch_fp8<NT_MOE_EPI_RELU2, false>(NT_F8_ARGS);
    default:
      return packed ? launch_fp8<NT_MOE_EPI_NONE, true>(NT_F8_ARGS)
                    : launch_fp8<NT_MOE_EPI_NONE, false>(NT_F8_ARGS);
  }
#undef NT_F8_ARGS
}

// Packs e4m3 weights w [S, R, K] for the packed fp8 GEMM: 32-row groups (for SwiGLU 16 gate
// rows then the 16 value rows of the same columns), each a run of 4 KB blocks per 128-wide K
// block, chunk ((2 st + h) * 64 + l) of a block holding row l % 32 and K bytes
// 128 kb + 64 st + 32 (l / 32) + 16 h .. + 16.
__global__ __launch_bounds__(256) void pack_fp8_kernel(const uint8_t* __restrict__ w,
                                                        int64_t chunks, int R, int K, int n_out,
                                                        int swiglu, uint8_t* __restrict__ out) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= chunks) return;
  const int KB = K / 128, NB = R / 32;
  const int l = (int)(c % 64), sh = (int)((c / 64) % 4), st = sh / 2, h = sh % 2;
  const int kb = (int)((c / 256) % KB);
  const int64_t rest = c / (256 * (int64_t)KB);
  const int nb = (int)(rest % NB);
  const int64_t s = rest / NB;
  const int i = l % 32;
  const int row = swiglu ? (i < 16 ? 16 * nb + i : n_out + 16 * nb + (i - 16)) : 32 * nb + i;
  const int k0 = kb * 128 + st * 64 + 32 * (l / 32) + 16 * h;
  *reinterpret_cast<u32x4*>(out + c * 16) =
      *reinterpret_cast<const u32x4*>(w + (s * R + row) * (int64_t)K + k0);
}

hipError_t launch_pack_weights_fp8(const uint8_t* w, int64_t S, int R, int K, int epilogue,
                                   uint8_t* packed, hipStream_t stream) {
  const int n_out = epilogue == NT_MOE_EPI_SWIGLU ? R / 2 : R;
  const int64_t chunks = S * (int64_t)R * K / 16;
  if (chunks == 0) return hipSuccess;
  pack_fp8_kernel<<<dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, stream>>>(
      w, chunks, R, K, n_out, epilogue == NT_MOE_EPI_SWIGLU ? 1 : 0, packed);
  return hipGetLastError();
}

}  // namespace ntmoe
