// Weight preparation: fp32 master weights -> the bf16 operands the expert GEMMs read, in one pass.
//
// MasterLinear keeps fp32 masters and casts them to the activation dtype for every product
// (megatron_moe.py:58-78, backbone.py:45-50); the backward's dgrad products need the transposes
// (autograd of F.linear). After every optimizer update all of them are stale at once, so one
// kernel reads each master exactly once and writes any of the bf16 copy w [S, R, K], the bf16
// transpose w^T [S, K, R], and both in the packed GEMM's fragment order (w with its epilogue's
// row pairing, w^T as a plain projection), so no separate pack pass follows: a workgroup moves a 64 x 64 tile, the
// transpose through LDS (row pitch 65 floats, so the column reads hit 64 different banks), every
// global read and write a run of consecutive 16-byte (read) or 8-byte (write) pieces per row.
#include "common.h"

namespace ntmoe {
namespace {

constexpr int kCT = 64;  // tile edge

// Packed (fragment-order) position of the 16-byte chunk holding K elements [kc, kc + 8) of row
// `row` of a [S, R, K] weight stack, as the packed GEMM reads it: block (s, nb, kb) of 32 rows x
// 64 K, chunk q * 64 + l with l = 32 h + block_row(i) for logical row i of the block and
// K = kb * 64 + 32 h + 8 q. Logical row i of block nb is row 32 nb + i, or for SwiGLU
// (swiglu_n = n_out > 0) gate row 16 nb + i (i < 16) and value row n_out + 16 nb + i - 16.
__device__ __forceinline__ int64_t packed_chunk(int64_t s, int row, int kc, int R, int K,
                                                int swiglu_n) {
  int nb, i;
  if (swiglu_n > 0) {
    const bool val = row >= swiglu_n;
    const int rr = val ? row - swiglu_n : row;
    nb = rr >> 4;
    i = (rr & 15) + (val ? 16 : 0);
  } else {
    nb = row >> 5;
    i = row & 31;
  }
  const int kb = kc >> 6, kk = kc & 63, h = kk >> 5, q = (kk & 31) >> 3;
  const int l = 32 * h + (i ^ (((i >> 2) ^ (i >> 3)) & 1) * 12);  // block_row(i), an involution
  return ((s * (R / 32) + nb) * (int64_t)(K / 64) + kb) * 256 + q * 64 + l;
}

// STREAM: the fp32 reads and the packed stores carry non-temporal hints, for stacks much larger
// than the last-level cache (the T3 cell's 419 MB pools: 155 -> 144 and 148 -> 132 us); smaller
// stacks keep the default policy (config 2's 134 and 67 MB pools took 17 % longer with the hints).
template <bool STREAM>
__global__ __launch_bounds__(256) void convert_weights_kernel(const float* __restrict__ w,
                                                              int64_t S, int R, int K,
                                                              uint16_t* __restrict__ out,
                                                              uint16_t* __restrict__ out_t,
                                                              uint16_t* __restrict__ pk,
                                                              int pk_swiglu_n,
                                                              uint16_t* __restrict__ pk_t) {
  __shared__ float tile[kCT][kCT + 1];
  const int tiles_k = K / kCT, tiles_r = R / kCT;
  const int64_t b = blockIdx.x;
  const int64_t s = b / ((int64_t)tiles_r * tiles_k);
  const int rest = (int)(b - s * tiles_r * tiles_k);
  const int r0 = (rest / tiles_k) * kCT, k0 = (rest % tiles_k) * kCT;
  const int ty = threadIdx.x >> 4, tx = threadIdx.x & 15;  // 16 rows x 16 four-element pieces
  const float* src = w + s * R * (int64_t)K;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = r0 + ty + 16 * i;
    const floatx4* vp = reinterpret_cast<const floatx4*>(src + (int64_t)r * K + k0 + 4 * tx);
    floatx4 v;
    if constexpr (STREAM) v = __builtin_nontemporal_load(vp);
    else v = *vp;
    if (out) {
      const u32x2 o = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
      *reinterpret_cast<u32x2*>(out + s * R * (int64_t)K + (int64_t)r * K + k0 + 4 * tx) = o;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) tile[ty + 16 * i][4 * tx + j] = v[j];
  }
  if (!out_t && !pk && !pk_t) return;
  __syncthreads();
  if (out_t) {
    uint16_t* dst = out_t + s * R * (int64_t)K;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int kk = ty + 16 * i;  // row of w^T within the tile
      const u32x2 o = {pack_bf16x2(tile[4 * tx][kk], tile[4 * tx + 1][kk]),
                       pack_bf16x2(tile[4 * tx + 2][kk], tile[4 * tx + 3][kk])};
      *reinterpret_cast<u32x2*>(dst + (int64_t)(k0 + kk) * R + r0 + 4 * tx) = o;
    }
  }
  // Packed w and packed w^T: the tile's 64 x 8 chunks of each, one 16-byte chunk per thread
  // and pass, consecutive threads on consecutive rows (runs of consecutive packed chunks).
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int p = threadIdx.x + 256 * it, a = p & 63, c = p >> 6;
    if (pk) {  // row r0 + a, K [k0 + 8 c, + 8)
      const u32x4 o = {pack_bf16x2(tile[a][8 * c], tile[a][8 * c + 1]),
                       pack_bf16x2(tile[a][8 * c + 2], tile[a][8 * c + 3]),
                       pack_bf16x2(tile[a][8 * c + 4], tile[a][8 * c + 5]),
                       pack_bf16x2(tile[a][8 * c + 6], tile[a][8 * c + 7])};
      u32x4* dst = reinterpret_cast<u32x4*>(pk + packed_chunk(s, r0 + a, k0 + 8 * c, R, K,
                                                              pk_swiglu_n) * 8);
      if constexpr (STREAM) __builtin_nontemporal_store(o, dst);
      else *dst = o;
    }
    if (pk_t) {  // w^T [S, K, R]: row k0 + a, K [r0 + 8 c, + 8)
      const u32x4 o = {pack_bf16x2(tile[8 * c][a], tile[8 * c + 1][a]),
                       pack_bf16x2(tile[8 * c + 2][a], tile[8 * c + 3][a]),
                       pack_bf16x2(tile[8 * c + 4][a], tile[8 * c + 5][a]),
                       pack_bf16x2(tile[8 * c + 6][a], tile[8 * c + 7][a])};
      u32x4* dst =
          reinterpret_cast<u32x4*>(pk_t + packed_chunk(s, k0 + a, r0 + 8 * c, K, R, 0) * 8);
      if constexpr (STREAM) __builtin_nontemporal_store(o, dst);
      else *dst = o;
    }
  }
}

// The router's operands from its fp32 weight W [E, d] (row stride ldw), one 64 x 64 tile per
// workgroup through LDS: router_t = W^T fp32 [dp, E] (rows d .. dp - 1 zero) and, when `first`
// is given, the backward's concatenated operand first bf16 [dp, Kc]: columns [0, Fs) = S^T for
// the shared expert's W1 S bf16 [Fs, dp] (row stride lds), hi = bf16(W^T) at [Fs, Fs + E),
// lo = bf16(W^T - hi) at [Fs + Ep, Fs + Ep + E) (the difference is exact in fp32), hi again at
// [Fs + 2 Ep, Fs + 2 Ep + E), every other column zero. blockIdx.y < ceil(Ep / 64) picks a tile
// of router columns (those past E read zeros), the rest tiles of S's rows.
__global__ __launch_bounds__(256) void router_operands_kernel(
    const float* __restrict__ w, int64_t ldw, int E, int d, int dp,
    const uint16_t* __restrict__ sw, int64_t lds, int Fs, float* __restrict__ router_t,
    uint16_t* __restrict__ first, int Ep, int Kc) {
  __shared__ float tile[kCT][kCT + 1];  // [source row][j - j0]
  const int tiles_r = (Ep + kCT - 1) / kCT;
  const bool router = (int)blockIdx.y < tiles_r;
  const int j0 = (int)blockIdx.x * kCT;
  const int c0 = ((int)blockIdx.y - (router ? 0 : tiles_r)) * kCT;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll 4
  for (int i = 0; i < kCT / 4; ++i) {  // coalesced along j
    const int c = c0 + ty + 4 * i, j = j0 + tx;
    float v = 0.f;
    if (router) {
      if (c < E && j < d) v = w[(int64_t)c * ldw + j];
    } else if (c < Fs && j < dp) {
      v = bf16_bits_to_f32(sw[(int64_t)c * lds + j]);
    }
    tile[ty + 4 * i][tx] = v;
  }
  __syncthreads();
#pragma unroll 4
  for (int i = 0; i < kCT / 4; ++i) {  // coalesced along the output column c
    const int j = j0 + ty + 4 * i, c = c0 + tx;
    if (j >= dp) continue;
    const float v = tile[tx][ty + 4 * i];
    if (router) {
      if (c < E) router_t[(int64_t)j * E + c] = v;
      if (first && c < Ep) {
        const uint16_t hi = f32_to_bf16_bits(v);
        const uint16_t lo = f32_to_bf16_bits(v - bf16_bits_to_f32(hi));
        uint16_t* row = first + (int64_t)j * Kc + Fs;
        row[c] = hi;
        row[Ep + c] = lo;
        row[2 * Ep + c] = hi;
      }
    } else if (c < Fs) {
      first[(int64_t)j * Kc + c] = f32_to_bf16_bits(v);
    }
  }
  if (first && blockIdx.y == 0) {  // columns [Fs + 3 Ep, Kc): zeros
    const int z0 = Fs + 3 * Ep, nz = Kc - z0;
    for (int p = (int)threadIdx.x; p < kCT * nz; p += 256) {
      const int j = j0 + p / nz;
      if (j < dp) first[(int64_t)j * Kc + z0 + p % nz] = 0;
    }
  }
}

}  // namespace

hipError_t launch_convert_weights(const float* w, int64_t S, int R, int K, uint16_t* out,
                                  uint16_t* out_t, hipStream_t stream, uint16_t* pk,
                                  int pk_swiglu_n, uint16_t* pk_t) {
  const int64_t blocks = S * (int64_t)(R / kCT) * (K / kCT);
  if (blocks == 0 || (!out && !out_t && !pk && !pk_t)) return hipSuccess;
  const bool stream_hints = S * (int64_t)R * K * (int64_t)sizeof(float) >= (int64_t(256) << 20);
  hipLaunchKernelGGL(stream_hints ? convert_weights_kernel<true> : convert_weights_kernel<false>,
                     dim3((unsigned)blocks), dim3(256), 0, stream, w, S, R, K, out, out_t, pk,
                     pk_swiglu_n, pk_t);
  return hipGetLastError();
}

hipError_t launch_router_operands(const float* w, int64_t ldw, int E, int d, int dp,
                                  const uint16_t* sw, int64_t lds, int Fs, float* router_t,
                                  uint16_t* first, int Ep, int Kc, hipStream_t stream) {
  const int ty = (Ep + kCT - 1) / kCT + (first ? (Fs + kCT - 1) / kCT : 0);
  hipLaunchKernelGGL(router_operands_kernel, dim3((unsigned)((dp + kCT - 1) / kCT), (unsigned)ty),
                     dim3(256), 0, stream, w, ldw, E, d, dp, sw, lds, first ? Fs : 0, router_t,
                     first, Ep, Kc);
  return hipGetLastError();
}

}  // namespace ntmoe
