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
#include <stdlib.h>
#include <string.h>
#include <type_traits>

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

// ---- Transposing-read kernel ---------------------------------------------------------------
// The same product with the operands staged as they lie in memory: every K step copies a
// 32-row slab of A (TN columns) and of B (TM columns) straight into LDS with 16-byte direct-to-LDS
// buffer loads, row-major, in a ring of three slabs, and the matrix-core operands are read out of
// the slabs with gfx950's transposing LDS read ds_read_b64_tr_b16. That instruction works on
// groups of 16 lanes: if lane p of a group addresses four consecutive 16-bit elements, lane
// 4 a + b receives, as its element e, element b of the four addressed by lane 4 e + a. So when
// lane p addresses row r0 + p / 4 at columns c + 4 (p % 4), lane j receives rows r0 .. r0 + 3 of
// column c + j: two such reads give a lane the 8 consecutive K values (rows) of one column that
// a v_mfma_f32_32x32x16_bf16 operand holds, without the register transposes of the kernel above.
// LDS rows are TN or TM bf16 wide; the 16-byte chunk c of row r sits at chunk c ^ 4 (r % 4), so
// the 16 lanes of a group (4 rows x 2 chunks) and the 32 of a half wave (4 rows x 4 chunks) each
// hit distinct bank groups. Rows past the segment read zeros (the buffer range check of A's
// per-tile resource, an out-of-range offset for B), columns past N or M repeat the last 8
// columns (their outputs are not stored). With gathered B rows, the rows' indices go into an LDS
// ring (direct-to-LDS, one instruction per wave) four slabs ahead of the data copies that read
// them, so one count of outstanding vector memory operations covers indices and data.
// Tile TN x TM (128 x 256 or 256 x 128) of one segment, 4 waves of TN/2 x TM/2, two workgroups
// per CU; otherwise as the kernel above (split K, zero tiles for empty segments, fp32 or bf16).
constexpr int kTK = 32;     // rows per slab
constexpr int kTRing = 3;   // slabs in the ring
constexpr int kTIdx = 5;    // index slots (four slabs ahead, plus the one being read)

typedef __attribute__((address_space(1))) void gvoid_t;
typedef __attribute__((address_space(3))) void lvoid_t;
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
constexpr int kBufWord3 = 0x00020000;

// 4 or 16 bytes per lane from a buffer at byte offset voff into LDS at dst + lane * (4 or 16)
// (dst uniform). A __device__ function of its own: called from a kernel's lambda, the builtin
// makes the host pass drop the kernel's launch stub.
__device__ __forceinline__ void buffer_to_lds4(__amdgpu_buffer_rsrc_t rsrc, void* dst, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lvoid_t*)dst, 4, voff, 0, 0, 0);
}
__device__ __forceinline__ void buffer_to_lds16(__amdgpu_buffer_rsrc_t rsrc, void* dst, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lvoid_t*)dst, 16, voff, 0, 0, 0);
}

template <int TN, int TM>
struct TrGeo {
  static constexpr int kSlabA = kTK * TN * 2;             // bytes
  static constexpr int kSlabB = kTK * TM * 2;
  static constexpr int kStage = kSlabA + kSlabB;
  static constexpr int kCopiesA = kSlabA / 1024 / 4;      // per wave per slab
  static constexpr int kCopiesB = kSlabB / 1024 / 4;
  static constexpr int kBN = TN / 64, kBM = TM / 64;      // 32-wide blocks per wave
  static constexpr size_t lds() { return (size_t)kTRing * kStage + kTIdx * kTK * 4; }
  static_assert(kCopiesA >= 1 && kCopiesB >= 1, "copies per wave");
};

template <int TN, int TM, bool GATHER, bool OUT_F32>
__global__ __launch_bounds__(256, 2) void grouped_wgrad_tr_kernel(
    const uint16_t* __restrict__ a, int64_t lda, const uint16_t* __restrict__ b, int64_t ldb,
    int64_t b_rows, const int32_t* __restrict__ b_src_row, const int32_t* __restrict__ seg_offsets,
    int num_segments, int64_t total_rows, int N, int M, int splits, void* __restrict__ c) {
  using G = TrGeo<TN, TM>;
  extern __shared__ __align__(16) unsigned char smem[];
  int* idx_ring = reinterpret_cast<int*>(smem + kTRing * G::kStage);  // [kTIdx][kTK]
  const int ntn = (N + TN - 1) / TN, ntm = (M + TM - 1) / TM;
  const int per_seg = ntn * ntm;
  // Workgroup b runs on XCD b % 8: give each XCD a contiguous range of the tile list, so the
  // tiles that share a segment's slabs (all of a segment's tiles, which read the same rows) run
  // at about the same time behind one L2 and each slab comes from HBM once.
  int blk;
  {
    const int nb = (int)gridDim.x, q = nb / 8, r = nb % 8;
    const int xcd = (int)blockIdx.x % 8, slot = (int)blockIdx.x / 8;
    blk = xcd * q + (xcd < r ? xcd : r) + slot;
  }
  const int split = blk / (num_segments * per_seg);
  const int rest = blk - split * num_segments * per_seg;
  const int s = rest / per_seg;
  const int tile = rest - s * per_seg;
  const int n0 = (tile / ntm) * TN, m0 = (tile % ntm) * TM;
  int64_t lo = seg_offsets[s], hi = seg_offsets[s + 1];
  lo = lo < 0 ? 0 : (lo > total_rows ? total_rows : lo);
  hi = hi < lo ? lo : (hi > total_rows ? total_rows : hi);
  if (splits > 1) {  // this chunk: whole 64-row slabs, the last chunk ending at hi
    const int64_t slabs = (hi - lo + 63) / 64;
    const int64_t per = (slabs + splits - 1) / splits;
    const int64_t c_lo = lo + split * per * 64, c_hi = c_lo + per * 64;
    lo = c_lo < hi ? c_lo : hi;
    hi = c_hi < hi ? c_hi : hi;
  }
  const int lane = lane_id(), wave = wave_id();
  const int wn = wave >> 1, wm = wave & 1;  // the wave's TN/2 x TM/2 quarter
  const int64_t c_base = ((int64_t)split * num_segments + s) * N * M;

  floatx16 acc[G::kBN][G::kBM];
#pragma unroll
  for (int i = 0; i < G::kBN; ++i)
#pragma unroll
    for (int j = 0; j < G::kBM; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.f;

  const int rows = (int)(hi - lo);
  const int n_slabs = (rows + kTK - 1) / kTK;
  if (n_slabs > 0) {
    // A: this tile's rows of the segment (a row past hi is out of range: zeros)
    const __amdgpu_buffer_rsrc_t ar = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a + lo * lda), 0, (int)((int64_t)rows * lda * 2), kBufWord3);
    // B: the whole matrix (gathered rows) or this tile's rows; an explicit out-of-range offset
    // for rows past hi
    const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(GATHER ? b : b + lo * ldb), 0,
        (int)(GATHER ? b_rows * ldb * 2 : (int64_t)rows * ldb * 2), kBufWord3);
    const __amdgpu_buffer_rsrc_t ir = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(GATHER ? b_src_row + lo : seg_offsets), 0, GATHER ? rows * 4 : 0, kBufWord3);

    // Copy instruction i of this wave for an operand W columns wide covers rows
    // (wave * copies + i) * rpi + lane / cpr of the slab, cpr = W / 8 chunks per row, rpi =
    // 64 / cpr rows per instruction; the lane writes chunk position lane % cpr, i.e. global chunk
    // (lane % cpr) ^ 4 (row % 4).
    auto chunk_col = [&](int row, int cpr, int col0, int width) {
      const int cg = (lane % cpr) ^ (4 * (row & 3));
      const int col = col0 + 8 * cg;
      return col < width ? col : width - 8;
    };
    int a_voff[G::kCopiesA], b_coloff[G::kCopiesB], b_row[G::kCopiesB];
#pragma unroll
    for (int i = 0; i < G::kCopiesA; ++i) {
      constexpr int cpr = TN / 8, rpi = 64 / cpr;
      const int row = (wave * G::kCopiesA + i) * rpi + lane / cpr;
      a_voff[i] = row * (int)lda * 2 + chunk_col(row, cpr, n0, N) * 2;
    }
#pragma unroll
    for (int i = 0; i < G::kCopiesB; ++i) {
      constexpr int cpr = TM / 8, rpi = 64 / cpr;
      b_row[i] = (wave * G::kCopiesB + i) * rpi + lane / cpr;
      b_coloff[i] = chunk_col(b_row[i], cpr, m0, M) * 2;
    }
    // Index loads of slab t (GATHER): wave w copies indices of rows 8 w .. 8 w + 7 with lanes
    // 0-7 (the other lanes are masked off: lane l would write dst + 4 l).
    auto issue_idx = [&](int t) __attribute__((always_inline)) {
      if constexpr (GATHER) {
        int* dst = idx_ring + (t % kTIdx) * kTK + 8 * wave;
        const int r = t * kTK + 8 * wave + lane;
        if (lane < 8) buffer_to_lds4(ir, dst, r * 4);
      }
    };
    auto issue_copies = [&](int t) __attribute__((always_inline)) {
      unsigned char* st = smem + (t % kTRing) * G::kStage;
      const int r0 = t * kTK;
#pragma unroll
      for (int i = 0; i < G::kCopiesA; ++i)
        buffer_to_lds16(ar, st + (wave * G::kCopiesA + i) * 1024,
                          a_voff[i] + r0 * (int)lda * 2);
#pragma unroll
      for (int i = 0; i < G::kCopiesB; ++i) {
        const int r = r0 + b_row[i];
        int voff;
        if (GATHER) {
          int g = idx_ring[(t % kTIdx) * kTK + b_row[i]];
          g = g < 0 ? 0 : (g >= b_rows ? (int)b_rows - 1 : g);
          voff = r < rows ? g * (int)ldb * 2 + b_coloff[i] : 0x7fffffff;
        } else {
          voff = r < rows ? r * (int)ldb * 2 + b_coloff[i] : 0x7fffffff;
        }
        buffer_to_lds16(br, st + G::kSlabA + (wave * G::kCopiesB + i) * 1024, voff);
      }
    };
    // Vector memory operations per slab and wave after its copies: the next slab's index load
    // and copies.
    constexpr int kPer = G::kCopiesA + G::kCopiesB + (GATHER ? 1 : 0);

    // Fragment reads: lane l = 16 g + p of a 32 x 32 x 16 operand block at column cb (tile
    // relative) and K rows k0 .. k0 + 15: provider row k0 + 8 (l / 32) + 4 t + p / 4, columns
    // cb + 16 (g % 2) + 4 (p % 4); lane l gets column cb + l % 32, rows k0 + 8 (l / 32) + 4 t ..
    // + 3. Per-lane byte offsets inside a slab for k0 = 0 and t = 0; t and the K step add whole
    // rows (4 and 16), multiples of 4, so the chunk swizzle 4 (row % 4) is unchanged and they
    // go into the instruction's offset field.
    const int pg = (lane >> 4) & 1, pp = lane & 15, ph = lane >> 5;
    auto tr_off = [&](int width, int cb) {
      const int row = 8 * ph + (pp >> 2);
      const int col = cb + 16 * pg + 4 * (pp & 3);
      const int chunk = (col >> 3) ^ (4 * (row & 3));
      return (uint32_t)(row * width * 2 + chunk * 16 + (col & 7) * 2);
    };
    const uint32_t smem_base = (uint32_t)(uintptr_t)smem;
    uint32_t offa[G::kBN], offb[G::kBM];
#pragma unroll
    for (int i = 0; i < G::kBN; ++i) offa[i] = smem_base + tr_off(TN, (TN / 2) * wn + 32 * i);
#pragma unroll
    for (int j = 0; j < G::kBM; ++j)
      offb[j] = smem_base + G::kSlabA + tr_off(TM, (TM / 2) * wm + 32 * j);
    // Inline assembly keeps the reads where they are written and out of the compiler's wait
    // analysis (which would wait for every outstanding direct-to-LDS copy before any LDS read);
    // frag_wait completes them with a wait that names their registers.
    struct Frags {
      u32x2 a[G::kBN][2], b[G::kBM][2];
    };
    auto read_frags = [](uint32_t stage_off, auto kk_c, const uint32_t (&oa)[G::kBN],
                         const uint32_t (&ob)[G::kBM], Frags& f) __attribute__((always_inline)) {
      constexpr int kk = decltype(kk_c)::value;
#pragma unroll
      for (int i = 0; i < G::kBN; ++i) {
        asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2"
                     : "=v"(f.a[i][0]) : "v"(oa[i] + stage_off), "n"(16 * kk * TN * 2));
        asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2"
                     : "=v"(f.a[i][1]) : "v"(oa[i] + stage_off), "n"((16 * kk + 4) * TN * 2));
      }
#pragma unroll
      for (int j = 0; j < G::kBM; ++j) {
        asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2"
                     : "=v"(f.b[j][0]) : "v"(ob[j] + stage_off), "n"(16 * kk * TM * 2));
        asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2"
                     : "=v"(f.b[j][1]) : "v"(ob[j] + stage_off), "n"((16 * kk + 4) * TM * 2));
      }
    };
    auto frag_wait = [](Frags& f) __attribute__((always_inline)) {
      static_assert(G::kBN + G::kBM == 6, "operand count of the wait");
      if constexpr (G::kBN == 2) {
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(f.a[0][0]), "+v"(f.a[0][1]), "+v"(f.a[1][0]), "+v"(f.a[1][1]),
                       "+v"(f.b[0][0]), "+v"(f.b[0][1]), "+v"(f.b[1][0]), "+v"(f.b[1][1]),
                       "+v"(f.b[2][0]), "+v"(f.b[2][1]), "+v"(f.b[3][0]), "+v"(f.b[3][1])
                     :
                     : "memory");
      } else {
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(f.a[0][0]), "+v"(f.a[0][1]), "+v"(f.a[1][0]), "+v"(f.a[1][1]),
                       "+v"(f.a[2][0]), "+v"(f.a[2][1]), "+v"(f.a[3][0]), "+v"(f.a[3][1]),
                       "+v"(f.b[0][0]), "+v"(f.b[0][1]), "+v"(f.b[1][0]), "+v"(f.b[1][1])
                     :
                     : "memory");
      }
    };
    auto mfmas = [&](const Frags& f) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < G::kBN; ++i) {
        const bf16x8 fa = __builtin_bit_cast(
            bf16x8, u32x4{f.a[i][0][0], f.a[i][0][1], f.a[i][1][0], f.a[i][1][1]});
#pragma unroll
        for (int j = 0; j < G::kBM; ++j) {
          const bf16x8 fb = __builtin_bit_cast(
              bf16x8, u32x4{f.b[j][0][0], f.b[j][0][1], f.b[j][1][0], f.b[j][1][1]});
          // D[m][n] += B-side (m x k) . A-side (k x n): lane holds column n, runs of 4 rows m
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb, fa, acc[i][j], 0, 0, 0);
        }
      }
    };
    // Workgroup barrier without a memory fence (a fence would wait for the copies in flight).
    auto barrier = []() __attribute__((always_inline)) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    };

    if (GATHER) {
      issue_idx(0);
      issue_idx(1);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      barrier();
      issue_idx(2);
      issue_copies(0);
      issue_idx(3);
      issue_copies(1);
    } else {
      issue_copies(0);
      issue_copies(1);
    }
    // A wave whose quarter lies wholly past N or M (the second half of a 64-wide last tile)
    // only copies and waits: its products would all be dropped.
    const bool live = n0 + (TN / 2) * wn < N && m0 + (TM / 2) * wm < M;
    Frags f0, f1;
    for (int t = 0; t < n_slabs; ++t) {
      // slab t's copies (and every index load issued before them) have landed once at most the
      // next slab's operations are outstanding
      if (t + 1 < n_slabs) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kPer) : "memory");
      else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      barrier();
      if (t + 2 < n_slabs) {
        issue_idx(t + 4);
        issue_copies(t + 2);
      }
      if (!live) continue;
      const uint32_t st = (t % kTRing) * G::kStage;
      __builtin_amdgcn_sched_barrier(0);
      read_frags(st, std::integral_constant<int, 0>(), offa, offb, f0);
      frag_wait(f0);
      read_frags(st, std::integral_constant<int, 1>(), offa, offb, f1);
      __builtin_amdgcn_sched_barrier(0);
      mfmas(f0);
      __builtin_amdgcn_sched_barrier(0);
      frag_wait(f1);
      mfmas(f1);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // acc[i][j]: n = n0 + TN/2 wn + 32 i + lane % 32,
  //            m = m0 + TM/2 wm + 32 j + 8 (q / 4) + 4 (lane / 32) + q % 4
#pragma unroll
  for (int i = 0; i < G::kBN; ++i) {
    const int n = n0 + (TN / 2) * wn + 32 * i + (lane & 31);
    if (n0 + (TN / 2) * wn + 32 * i >= N) continue;
#pragma unroll
    for (int j = 0; j < G::kBM; ++j) {
      if (m0 + (TM / 2) * wm + 32 * j >= M) continue;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int m = m0 + (TM / 2) * wm + 32 * j + 8 * g + 4 * (lane >> 5);
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

// ---- 256 x 256 transposing-read kernel ----------------------------------------------------
// The same product and slab layout as the kernel above, with a 256 x 256 tile per workgroup and
// one workgroup per CU: 4 waves of 128 x 128 (16 accumulator blocks each, 256 registers, which
// the compiler places in the accumulation registers). Per 32-row slab the workgroup copies 32 KB
// for 2^22 multiply-adds where the 128 x 256 tile copies 24 KB for 2^21, and each wave reads 16
// fragments per 16 MFMAs where a 64 x 128 wave reads 12 per 8: a third less copied and read per
// product. Slabs go through a ring of four (128 KB of LDS) with the copies three slabs ahead of
// the slab being published. The wait and barrier that publish slab t + 1 sit between slab t's
// two 16-MFMA halves, so slab t + 1's first fragments are read while slab t's second half runs
// (one wave per SIMD: nothing else would cover their latency). With gathered B rows the index
// loads run four slabs ahead of the copies that read them, in a ring of eight.
constexpr int kT2Ring = 4;  // slabs in the ring
constexpr int kT2Idx = 8;   // index slots
constexpr int kT2Lead = 3;  // copies: slabs ahead of the slab being published
static_assert(kT2Lead == kT2Ring - 1, "a group refills the slot the previous slab left");
constexpr int kT2ILead = 7; // index loads: slabs ahead of the slab being published

struct T2Geo {
  static constexpr int kSlab = kTK * 256 * 2;       // bytes per operand and slab
  static constexpr int kStage = 2 * kSlab;
  static constexpr int kCopies = kSlab / 1024 / 4;  // per wave, operand and slab
  static constexpr size_t lds() { return (size_t)kT2Ring * kStage + kT2Idx * kTK * 4; }
};

// One product of the kernel below (its workgroups: tiles x splits) and the launch's products,
// which share the segments: up to two, their tile lists one after the other.
struct T2Product {
  const uint16_t* a;
  const uint16_t* b;
  const int32_t* b_src_row;  // NULL: no gather
  void* c;
  int64_t lda, ldb, b_rows;
  int N, M, blocks;
};
struct T2Args {
  T2Product p[2];
  const int32_t* seg_offsets;
  int64_t total_rows;
  int num_segments, splits, count;
};

template <bool OUT_F32>
__global__ __launch_bounds__(256, 1) void grouped_wgrad_t256_kernel(T2Args args) {
  using G = T2Geo;
  constexpr int TN = 256, TM = 256, kB = 4;  // kB: 32-wide blocks per wave and dimension
  extern __shared__ __align__(16) unsigned char smem[];
  int* idx_ring = reinterpret_cast<int*>(smem + kT2Ring * G::kStage);  // [kT2Idx][kTK]
  int blk;  // XCD-contiguous ranges of the tile list, as above
  {
    const int nb = (int)gridDim.x, q = nb / 8, r = nb % 8;
    const int xcd = (int)blockIdx.x % 8, slot = (int)blockIdx.x / 8;
    blk = xcd * q + (xcd < r ? xcd : r) + slot;
  }
  // this workgroup's product (fields selected one by one: no indexing of the argument block)
  const bool second = args.count > 1 && blk >= args.p[0].blocks;
  if (second) blk -= args.p[0].blocks;
  const uint16_t* __restrict__ a = second ? args.p[1].a : args.p[0].a;
  const uint16_t* __restrict__ b = second ? args.p[1].b : args.p[0].b;
  const int32_t* __restrict__ b_src_row = second ? args.p[1].b_src_row : args.p[0].b_src_row;
  void* __restrict__ c = second ? args.p[1].c : args.p[0].c;
  const int64_t lda = second ? args.p[1].lda : args.p[0].lda;
  const int64_t ldb = second ? args.p[1].ldb : args.p[0].ldb;
  const int64_t b_rows = second ? args.p[1].b_rows : args.p[0].b_rows;
  const int N = second ? args.p[1].N : args.p[0].N, M = second ? args.p[1].M : args.p[0].M;
  const int32_t* __restrict__ seg_offsets = args.seg_offsets;
  const int num_segments = args.num_segments, splits = args.splits;
  const int64_t total_rows = args.total_rows;
  const bool gather = b_src_row != nullptr;
  const int ntn = (N + TN - 1) / TN, ntm = (M + TM - 1) / TM;
  const int per_seg = ntn * ntm;
  const int split = blk / (num_segments * per_seg);
  const int rest = blk - split * num_segments * per_seg;
  const int s = rest / per_seg;
  const int tile = rest - s * per_seg;
  const int n0 = (tile / ntm) * TN, m0 = (tile % ntm) * TM;
  int64_t lo = seg_offsets[s], hi = seg_offsets[s + 1];
  lo = lo < 0 ? 0 : (lo > total_rows ? total_rows : lo);
  hi = hi < lo ? lo : (hi > total_rows ? total_rows : hi);
  if (splits > 1) {  // this chunk: whole 64-row slabs, the last chunk ending at hi
    const int64_t slabs = (hi - lo + 63) / 64;
    const int64_t per = (slabs + splits - 1) / splits;
    const int64_t c_lo = lo + split * per * 64, c_hi = c_lo + per * 64;
    lo = c_lo < hi ? c_lo : hi;
    hi = c_hi < hi ? c_hi : hi;
  }
  const int lane = lane_id(), wave = wave_id();
  const int wn = wave >> 1, wm = wave & 1;  // the wave's 128 x 128 quarter
  const int64_t c_base = ((int64_t)split * num_segments + s) * N * M;

  floatx16 acc[kB][kB];
#pragma unroll
  for (int i = 0; i < kB; ++i)
#pragma unroll
    for (int j = 0; j < kB; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.f;

  const int rows = (int)(hi - lo);
  const int n_slabs = (rows + kTK - 1) / kTK;
  if (n_slabs > 0) {
    const __amdgpu_buffer_rsrc_t ar = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a + lo * lda), 0, (int)((int64_t)rows * lda * 2), kBufWord3);
    const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(gather ? b : b + lo * ldb), 0,
        (int)(gather ? b_rows * ldb * 2 : (int64_t)rows * ldb * 2), kBufWord3);
    const __amdgpu_buffer_rsrc_t ir = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(gather ? b_src_row + lo : seg_offsets), 0, gather ? rows * 4 : 0, kBufWord3);

    // The slab loop, compiled once per gather kind (gather: one product's rows gathered through
    // b_src_row, with the index loads and reads; a launch may hold one product of each kind).
    auto run = [&](auto gather_c) __attribute__((always_inline)) {
      constexpr bool GATHER = decltype(gather_c)::value;
      // Copy instruction i of this wave covers slab row (wave * kCopies + i) * 2 + lane / 32, chunk
      // position lane % 32, i.e. global chunk (lane % 32) ^ 4 (row % 4) (columns past N or M
      // repeat the last 8).
      auto chunk_col = [&](int row, int col0, int width) {
        const int cg = (lane % 32) ^ (4 * (row & 3));
        const int col = col0 + 8 * cg;
        return col < width ? col : width - 8;
      };
      int a_voff[G::kCopies], b_coloff[G::kCopies], b_row[G::kCopies];
  #pragma unroll
      for (int i = 0; i < G::kCopies; ++i) {
        const int row = (wave * G::kCopies + i) * 2 + lane / 32;
        a_voff[i] = row * (int)lda * 2 + chunk_col(row, n0, N) * 2;
        b_row[i] = row;
        b_coloff[i] = chunk_col(row, m0, M) * 2;
      }
      // Index loads of slab t (GATHER): wave w loads rows 8 w .. 8 w + 7 with lanes 0-7.
      auto issue_idx = [&](int t) __attribute__((always_inline)) {
        if constexpr (GATHER) {
          int* dst = idx_ring + (t % kT2Idx) * kTK + 8 * wave;
          const int r = t * kTK + 8 * wave + lane;
          if (lane < 8) buffer_to_lds4(ir, dst, r * 4);
        }
      };
      // Slab t's gathered row indices for this wave's B copies, read from the index ring without a
      // wait (the caller's next wait for every LDS read covers them), and B's source offsets for
      // slab t's copies from them (or from the row itself without the gather); rows past the chunk
      // get an out-of-range offset.
      const uint32_t idx_lds = (uint32_t)(uintptr_t)idx_ring;
      auto idx_read = [&](int t, int (&gi)[G::kCopies]) __attribute__((always_inline)) {
        if constexpr (GATHER) {
          const uint32_t slot = idx_lds + (uint32_t)((t % kT2Idx) * kTK * 4);
  #pragma unroll
          for (int i = 0; i < G::kCopies; ++i)
            asm volatile("ds_read_b32 %0, %1" : "=v"(gi[i]) : "v"(slot + b_row[i] * 4));
        }
      };
      auto idx_fence = [](int (&gi)[G::kCopies]) __attribute__((always_inline)) {
        if constexpr (GATHER) asm volatile("" : "+v"(gi[0]), "+v"(gi[1]), "+v"(gi[2]), "+v"(gi[3]));
      };
      auto b_offsets = [&](int t, const int (&gi)[G::kCopies], int (&bv)[G::kCopies])
                           __attribute__((always_inline)) {
  #pragma unroll
        for (int i = 0; i < G::kCopies; ++i) {
          const int r = t * kTK + b_row[i];
          int src = r;
          if constexpr (GATHER) {
            const int g = gi[i];
            src = g < 0 ? 0 : (g >= b_rows ? (int)b_rows - 1 : g);
          }
          bv[i] = r < rows ? src * (int)ldb * 2 + b_coloff[i] : 0x7fffffff;
        }
      };
      // Item k of the group published with slab p: A copies, B copies, the index load of slab
      // p + kT2ILead. The copies of slab t = p + kT2Lead go into the slot slab p - 1 left; every
      // group is issued, those past the last slab reading only out-of-range offsets (zeros, no
      // memory traffic), so each wait below counts a fixed number of operations.
      constexpr int kPer = 2 * G::kCopies + (GATHER ? 1 : 0);  // vector memory operations per group
      auto group_item = [&](int p, auto k_c, const int (&bv)[G::kCopies])
                            __attribute__((always_inline)) {
        constexpr int k = decltype(k_c)::value;
        const int t = p + kT2Lead;
        unsigned char* st = smem + (t % kT2Ring) * G::kStage;
        if constexpr (k < G::kCopies) {
          buffer_to_lds16(ar, st + (wave * G::kCopies + k) * 1024,
                          a_voff[k] + t * kTK * (int)lda * 2);
        } else if constexpr (k < 2 * G::kCopies) {
          constexpr int i = k - G::kCopies;
          buffer_to_lds16(br, st + G::kSlab + (wave * G::kCopies + i) * 1024, bv[i]);
        } else {
          issue_idx(p + kT2ILead);
        }
      };
      auto group = [&](int p, const int (&bv)[G::kCopies]) __attribute__((always_inline)) {
        static_for<0, kPer>([&](auto k_c) __attribute__((always_inline)) {
          group_item(p, k_c, bv);
        });
      };
      // Slab p's copies (group p - kT2Lead) have landed once at most the two groups issued after it
      // are outstanding.
      auto wait_slab = []() __attribute__((always_inline)) {
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * kPer) : "memory");
      };

      const int pg = (lane >> 4) & 1, pp = lane & 15, ph = lane >> 5;
      auto tr_off = [&](int cb) {
        const int row = 8 * ph + (pp >> 2);
        const int col = cb + 16 * pg + 4 * (pp & 3);
        const int chunk = (col >> 3) ^ (4 * (row & 3));
        return (uint32_t)(row * 256 * 2 + chunk * 16 + (col & 7) * 2);
      };
      const uint32_t smem_base = (uint32_t)(uintptr_t)smem;
      uint32_t offa[kB], offb[kB];
  #pragma unroll
      for (int i = 0; i < kB; ++i) {
        offa[i] = smem_base + tr_off(128 * wn + 32 * i);
        offb[i] = smem_base + G::kSlab + tr_off(128 * wm + 32 * i);
      }
      struct Frags {
        u32x2 a[kB][2], b[kB][2];
      };
      // Read r (0-15) of the fragments for K rows 16 kk .. 16 kk + 15 of the slab at stage_off:
      // A blocks for r < 8, B blocks after.
      auto read_one = [](uint32_t stage_off, auto kk_c, auto r_c, const uint32_t (&oa)[kB],
                         const uint32_t (&ob)[kB], Frags& f) __attribute__((always_inline)) {
        constexpr int kk = decltype(kk_c)::value, r = decltype(r_c)::value;
        constexpr int blk = (r % 8) / 2, hf = r % 2;
        constexpr int off = (16 * kk + 4 * hf) * 512;
        if constexpr (r < 8)
          asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2"
                       : "=v"(f.a[blk][hf]) : "v"(oa[blk] + stage_off), "n"(off));
        else
          asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2"
                       : "=v"(f.b[blk][hf]) : "v"(ob[blk] + stage_off), "n"(off));
      };
      // Waits for every LDS read in flight, naming the fragment registers.
      auto frag_wait = [](Frags& f) __attribute__((always_inline)) {
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(f.a[0][0]), "+v"(f.a[0][1]), "+v"(f.a[1][0]), "+v"(f.a[1][1]),
                       "+v"(f.a[2][0]), "+v"(f.a[2][1]), "+v"(f.a[3][0]), "+v"(f.a[3][1]),
                       "+v"(f.b[0][0]), "+v"(f.b[0][1]), "+v"(f.b[1][0]), "+v"(f.b[1][1]),
                       "+v"(f.b[2][0]), "+v"(f.b[2][1]), "+v"(f.b[3][0]), "+v"(f.b[3][1])
                     :
                     : "memory");
      };
      // The 16 MFMAs of fragments fc (one wave per SIMD, so nothing else would fill the matrix
      // core while this wave issued a burst of reads or copies: they go out between the MFMAs).
      // READ: the 16 reads of fn (stage sn, K half KKN), two after each of the first four MFMAs and
      // one after each of the next eight, so they land while the last four run. COPY: the items
      // of group p, one after each of the first kPer MFMAs. IDX: the index reads of slab ti after
      // the fifth MFMA.
      auto half = [&](const Frags& fc, Frags& fn, uint32_t sn, auto kkn_c, auto read_c, auto copy_c,
                      auto idx_c, int p, const int (&bv)[G::kCopies], int ti,
                      int (&gi)[G::kCopies]) __attribute__((always_inline)) {
        constexpr bool READ = decltype(read_c)::value, COPY = decltype(copy_c)::value;
        constexpr bool IDX = decltype(idx_c)::value;
        static_for<0, 16>([&](auto k_c) __attribute__((always_inline)) {
          constexpr int k = decltype(k_c)::value;
          constexpr int i = k / kB, j = k % kB;
          const bf16x8 fa = __builtin_bit_cast(
              bf16x8, u32x4{fc.a[i][0][0], fc.a[i][0][1], fc.a[i][1][0], fc.a[i][1][1]});
          const bf16x8 fb = __builtin_bit_cast(
              bf16x8, u32x4{fc.b[j][0][0], fc.b[j][0][1], fc.b[j][1][0], fc.b[j][1][1]});
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb, fa, acc[i][j], 0, 0, 0);
          if constexpr (READ) {
            constexpr int r0 = k < 4 ? 2 * k : (k < 12 ? k + 4 : 16);
            constexpr int r1 = k < 4 ? 2 * k + 2 : (k < 12 ? k + 5 : 16);
            static_for<r0, r1>([&](auto r_c) __attribute__((always_inline)) {
              read_one(sn, kkn_c, r_c, offa, offb, fn);
            });
          }
          if constexpr (COPY && k < kPer) group_item(p, k_c, bv);
          if constexpr (IDX && k == 4) idx_read(ti, gi);
          __builtin_amdgcn_sched_barrier(0);
        });
      };
      auto barrier = []() __attribute__((always_inline)) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
      };
      using I0 = std::integral_constant<int, 0>;
      using I1 = std::integral_constant<int, 1>;

      // Prologue: the index loads of slabs 0 .. 3 published; groups -3, -2, -1 (the copies of
      // slabs 0, 1, 2); slab 0 published; group 0; slab 0's first fragments.
      int bv[G::kCopies], gi[G::kCopies] = {0, 0, 0, 0};
      if (GATHER) {
        issue_idx(0);
        issue_idx(1);
        issue_idx(2);
        issue_idx(3);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        barrier();
      }
  #pragma unroll
      for (int p = -kT2Lead; p < 0; ++p) {
        idx_read(p + kT2Lead, gi);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        idx_fence(gi);
        b_offsets(p + kT2Lead, gi, bv);
        group(p, bv);
      }
      wait_slab();
      barrier();
      idx_read(kT2Lead, gi);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      idx_fence(gi);
      b_offsets(kT2Lead, gi, bv);
      group(0, bv);
      Frags f0, f1;
      static_for<0, 16>([&](auto r_c) __attribute__((always_inline)) {
        read_one(0, I0(), r_c, offa, offb, f0);
      });
      // Slab t: its first K half, with the second half's reads and the index reads of group t + 1;
      // slab t + 1 published (its copies landed, every wave past its reads of slab t, whose slot
      // the next group then refills; the indices of group t + 1 were published with slab t); the
      // second half, with slab t + 1's first reads and group t + 1.
      for (int t = 0; t + 1 < n_slabs; ++t) {
        const uint32_t st = (t % kT2Ring) * G::kStage;
        frag_wait(f0);
        __builtin_amdgcn_sched_barrier(0);
        half(f0, f1, st, I1(), std::true_type(), std::false_type(), std::true_type(), 0, bv,
             t + 1 + kT2Lead, gi);
        wait_slab();
        barrier();
        frag_wait(f1);
        idx_fence(gi);
        b_offsets(t + 1 + kT2Lead, gi, bv);
        __builtin_amdgcn_sched_barrier(0);
        half(f1, f0, ((t + 1) % kT2Ring) * G::kStage, I0(), std::true_type(), std::true_type(),
             std::false_type(), t + 1, bv, 0, gi);
      }
      {  // the last slab
        const uint32_t st = ((n_slabs - 1) % kT2Ring) * G::kStage;
        frag_wait(f0);
        __builtin_amdgcn_sched_barrier(0);
        half(f0, f1, st, I1(), std::true_type(), std::false_type(), std::false_type(), 0, bv, 0,
             gi);
        frag_wait(f1);
        __builtin_amdgcn_sched_barrier(0);
        half(f1, f0, 0, I0(), std::false_type(), std::false_type(), std::false_type(), 0, bv, 0,
             gi);
      }
    };
    if (gather) run(std::true_type());
    else run(std::false_type());
    // the trailing groups' copies land before the workgroup's LDS is released
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  // acc[i][j]: n = n0 + 128 wn + 32 i + lane % 32, m = m0 + 128 wm + 32 j + 8 (q / 4) +
  // 4 (lane / 32) + q % 4
#pragma unroll
  for (int i = 0; i < kB; ++i) {
    const int n = n0 + 128 * wn + 32 * i + (lane & 31);
    if (n0 + 128 * wn + 32 * i >= N) continue;
#pragma unroll
    for (int j = 0; j < kB; ++j) {
      if (m0 + 128 * wm + 32 * j >= M) continue;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int m = m0 + 128 * wm + 32 * j + 8 * g + 4 * (lane >> 5);
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

namespace {

// NT_MOE_WGRAD=regs selects the register-transpose kernel (for comparisons).
bool wgrad_regs_override() {
  static const bool v = [] {
    const char* e = getenv("NT_MOE_WGRAD");
    return e && !strcmp(e, "regs");
  }();
  return v;
}

template <int TN, int TM, bool GATHER, bool OUT_F32>
hipError_t launch_tr(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                     int64_t b_rows, const int32_t* b_src_row, const int32_t* seg_offsets,
                     int num_segments, int64_t total_rows, int N, int M, int splits, void* c,
                     hipStream_t stream) {
  auto kern = grouped_wgrad_tr_kernel<TN, TM, GATHER, OUT_F32>;
  const size_t lds = TrGeo<TN, TM>::lds();
  hipError_t err = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds);
  if (err != hipSuccess) return err;
  const int64_t tiles = (int64_t)num_segments * ((N + TN - 1) / TN) * ((M + TM - 1) / TM);
  hipLaunchKernelGGL(kern, dim3((unsigned)(tiles * splits)), dim3(256), lds, stream, a, lda, b,
                     ldb, b_rows, b_src_row, seg_offsets, num_segments, total_rows, N, M, splits,
                     c);
  return hipGetLastError();
}

template <bool OUT_F32>
hipError_t launch_t256(const T2Args& args, hipStream_t stream) {
  auto kern = grouped_wgrad_t256_kernel<OUT_F32>;
  const size_t lds = T2Geo::lds();
  hipError_t err = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds);
  if (err != hipSuccess) return err;
  const int64_t blocks = (int64_t)args.p[0].blocks + (args.count > 1 ? args.p[1].blocks : 0);
  if (blocks == 0) return hipSuccess;
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), lds, stream, args);
  return hipGetLastError();
}

T2Product t256_product(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                       int64_t b_rows, const int32_t* b_src_row, int num_segments, int N, int M,
                       int splits, void* c) {
  T2Product p;
  p.a = a;
  p.b = b;
  p.b_src_row = b_src_row;
  p.c = c;
  p.lda = lda;
  p.ldb = ldb;
  p.b_rows = b_rows;
  p.N = N;
  p.M = M;
  p.blocks = num_segments * ((N + 255) / 256) * ((M + 255) / 256) * splits;
  return p;
}

// Whether the 256 x 256 kernel takes a product: both widths whole 256-wide tiles, and no split
// K (a split product has too few tiles to fill the chip with one workgroup per CU at the split
// count sized for the two-per-CU kernels: the T3 cell's router gradient ran 39 -> 45 us on it).
bool wgrad_t256(int N, int M, int splits) { return N % 256 == 0 && M % 256 == 0 && splits == 1; }

// The transposing-read kernels: 256 x 256 tiles when both widths are multiples of 256 and K is
// not split, else 128 x 256 when N <= M, else 256 x 128.
template <bool OUT_F32>
hipError_t launch_tr_any(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                         int64_t b_rows, const int32_t* b_src_row, const int32_t* seg_offsets,
                         int num_segments, int64_t total_rows, int N, int M, int splits, void* c,
                         hipStream_t stream) {
  const bool g = b_src_row != nullptr;
  if (wgrad_t256(N, M, splits)) {
    T2Args args;
    args.p[0] = t256_product(a, lda, b, ldb, b_rows, b_src_row, num_segments, N, M, splits, c);
    args.p[1] = args.p[0];
    args.seg_offsets = seg_offsets;
    args.total_rows = total_rows;
    args.num_segments = num_segments;
    args.splits = splits;
    args.count = 1;
    return launch_t256<OUT_F32>(args, stream);
  }
#define NT_TR(TN, TM, GG)                                                                      \
  return launch_tr<TN, TM, GG, OUT_F32>(a, lda, b, ldb, b_rows, b_src_row, seg_offsets,         \
                                        num_segments, total_rows, N, M, splits, c, stream);
  if (N <= M) {
    if (g) { NT_TR(128, 256, true) } else { NT_TR(128, 256, false) }
  } else {
    if (g) { NT_TR(256, 128, true) } else { NT_TR(256, 128, false) }
  }
#undef NT_TR
}

}  // namespace

hipError_t launch_grouped_wgrad(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                                int64_t b_rows, const int32_t* b_src_row,
                                const int32_t* seg_offsets, int num_segments, int64_t total_rows,
                                int N, int M, int splits, float* partial, bool c_f32, void* c,
                                hipStream_t stream) {
  const int64_t tiles = (int64_t)num_segments * ((N + kWT - 1) / kWT) * ((M + kWT - 1) / kWT);
  if (tiles == 0) return hipSuccess;
  // The transposing-read kernel addresses its operands through 32-bit buffer offsets.
  const int64_t lim = (int64_t)1 << 31;
  if (!wgrad_regs_override() && total_rows * lda * 2 < lim &&
      (b_src_row ? b_rows : total_rows) * ldb * 2 < lim) {
    hipError_t err;
    if (splits <= 1)
      return c_f32 ? launch_tr_any<true>(a, lda, b, ldb, b_rows, b_src_row, seg_offsets,
                                         num_segments, total_rows, N, M, 1, c, stream)
                   : launch_tr_any<false>(a, lda, b, ldb, b_rows, b_src_row, seg_offsets,
                                          num_segments, total_rows, N, M, 1, c, stream);
    err = launch_tr_any<true>(a, lda, b, ldb, b_rows, b_src_row, seg_offsets, num_segments,
                              total_rows, N, M, splits, static_cast<void*>(partial), stream);
    if (err != hipSuccess) return err;
    const int64_t count = (int64_t)num_segments * N * M;
    auto sum = c_f32 ? sum_splits_kernel<true> : sum_splits_kernel<false>;
    hipLaunchKernelGGL(sum, dim3((unsigned)((count / 4 + 255) / 256)), dim3(256), 0, stream,
                       partial, splits, count, c);
    return hipGetLastError();
  }
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

hipError_t launch_grouped_wgrad_pair(const uint16_t* a0, int64_t lda0, const uint16_t* b0,
                                     int64_t ldb0, int64_t b_rows0, const int32_t* b_src_row0,
                                     int N0, int M0, void* c0, const uint16_t* a1, int64_t lda1,
                                     const uint16_t* b1, int64_t ldb1, int64_t b_rows1,
                                     const int32_t* b_src_row1, int N1, int M1, void* c1,
                                     const int32_t* seg_offsets, int num_segments,
                                     int64_t total_rows, bool c_f32, hipStream_t stream) {
  if (num_segments == 0) return hipSuccess;
  const int64_t lim = (int64_t)1 << 31;
  auto fits = [&](int64_t lda, int64_t ldb, int64_t b_rows, const int32_t* src, int N, int M) {
    return wgrad_t256(N, M, 1) && total_rows * lda * 2 < lim &&
           (src ? b_rows : total_rows) * ldb * 2 < lim;
  };
  if (!wgrad_regs_override() && fits(lda0, ldb0, b_rows0, b_src_row0, N0, M0) &&
      fits(lda1, ldb1, b_rows1, b_src_row1, N1, M1)) {
    // one launch over both tile lists: the second product's tiles start as CUs free up from the
    // first's, and the launch has one tail instead of two
    T2Args args;
    args.p[0] = t256_product(a0, lda0, b0, ldb0, b_rows0, b_src_row0, num_segments, N0, M0, 1, c0);
    args.p[1] = t256_product(a1, lda1, b1, ldb1, b_rows1, b_src_row1, num_segments, N1, M1, 1, c1);
    args.seg_offsets = seg_offsets;
    args.total_rows = total_rows;
    args.num_segments = num_segments;
    args.splits = 1;
    args.count = 2;
    return c_f32 ? launch_t256<true>(args, stream) : launch_t256<false>(args, stream);
  }
  hipError_t err = launch_grouped_wgrad(a0, lda0, b0, ldb0, b_rows0, b_src_row0, seg_offsets,
                                        num_segments, total_rows, N0, M0, 1, nullptr, c_f32, c0,
                                        stream);
  if (err != hipSuccess) return err;
  return launch_grouped_wgrad(a1, lda1, b1, ldb1, b_rows1, b_src_row1, seg_offsets, num_segments,
                              total_rows, N1, M1, 1, nullptr, c_f32, c1, stream);
}

}  // namespace ntmoe
