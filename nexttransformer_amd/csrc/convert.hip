// Weight preparation: fp32 master weights -> the bf16 operands the expert GEMMs read, in one pass.
//
// MasterLinear keeps fp32 masters and casts them to the activation dtype for every product
// (megatron_moe.py:58-78, backbone.py:45-50); the backward's dgrad products need the transposes
// (autograd of F.linear). After every optimizer update all of them are stale at once, so one
// kernel reads each master exactly once and writes both the bf16 copy w [S, R, K] and the bf16
// transpose w^T [S, K, R] (either may be skipped): a workgroup moves a 64 x 64 tile, the
// transpose through LDS (row pitch 65 floats, so the column reads hit 64 different banks), every
// global read and write a run of consecutive 16-byte (read) or 8-byte (write) pieces per row.
#include "common.h"

namespace ntmoe {
namespace {

constexpr int kCT = 64;  // tile edge

__global__ __launch_bounds__(256) void convert_weights_kernel(const float* __restrict__ w,
                                                              int64_t S, int R, int K,
                                                              uint16_t* __restrict__ out,
                                                              uint16_t* __restrict__ out_t) {
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
    const floatx4 v = *reinterpret_cast<const floatx4*>(src + (int64_t)r * K + k0 + 4 * tx);
    if (out) {
      const u32x2 o = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
      *reinterpret_cast<u32x2*>(out + s * R * (int64_t)K + (int64_t)r * K + k0 + 4 * tx) = o;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) tile[ty + 16 * i][4 * tx + j] = v[j];
  }
  if (!out_t) return;
  __syncthreads();
  uint16_t* dst = out_t + s * R * (int64_t)K;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int kk = ty + 16 * i;  // row of w^T within the tile
    const u32x2 o = {pack_bf16x2(tile[4 * tx][kk], tile[4 * tx + 1][kk]),
                     pack_bf16x2(tile[4 * tx + 2][kk], tile[4 * tx + 3][kk])};
    *reinterpret_cast<u32x2*>(dst + (int64_t)(k0 + kk) * R + r0 + 4 * tx) = o;
  }
}

}  // namespace

hipError_t launch_convert_weights(const float* w, int64_t S, int R, int K, uint16_t* out,
                                  uint16_t* out_t, hipStream_t stream) {
  const int64_t blocks = S * (int64_t)(R / kCT) * (K / kCT);
  if (blocks == 0 || (!out && !out_t)) return hipSuccess;
  hipLaunchKernelGGL(convert_weights_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, w, S,
                     R, K, out, out_t);
  return hipGetLastError();
}

}  // namespace ntmoe
