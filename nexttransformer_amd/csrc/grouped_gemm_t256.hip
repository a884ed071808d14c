// Grouped expert GEMM with 256 x 256 tiles, both operands staged through LDS.
//
// Same computation as the other grouped GEMMs (SequentialMLP's per-expert fc1 / fc2,
// megatron_moe.py:145, over MasterLinear, :58-78, with the SwiGLU / ReLU^2 epilogue fused):
//   c[r, j] = epilogue(a_src(r) . w_s[j, :])   for every row r of segment s,
// with plain weights w [S, R, K] (R = 2 n_out for SwiGLU: gate rows, then value rows).
//
// Shape: one persistent 8-wave workgroup per CU. A tile is 256 token rows x 256 weight rows;
// per 64-wide K step both operands (32 KB each) are copied from global memory straight into LDS
// (gfx950 global_load_lds_dwordx4), so every weight byte fetched by the CU feeds 256 token rows
// and every token byte 256 weight rows: 64 KB of global reads per 8.4 MFLOP. Each wave owns 128
// tokens x 64 weight rows of the tile (8 32x32 accumulators), two waves per SIMD. Two LDS stages
// (128 KB); one workgroup barrier per K step, after the wait for the next stage's copies, frees
// the slot just read. A stage's copies go out in two halves spread between MFMAs (issued
// together ahead of them they held back the first products): its token rows right after the
// barrier two steps before it, its weight rows during the step before it. With four waves of
// 128 x 128 (one per SIMD) the kernel measured 96-107 vs 86-93 us at config 2's down projection.
//
// LDS rows are 128 bytes (64 bf16 of K) with the 16-byte chunks of row r XOR-swizzled by
// (r / 2) % 8, which keeps the 16-lane fragment reads free of bank conflicts; each copy
// instruction writes 1 KB of consecutive LDS bytes (8 rows), every lane choosing which global
// chunk lands in its 16 bytes. Weight rows are placed in fragment order on the way in: position
// p of a 32-row block holds logical row block_row(p) (the middle 4-row groups of each 16-row half
// swapped), and for SwiGLU a block's logical rows are 16 gate rows and the 16 value rows of the
// same output columns, so a lane's accumulators hold gate and value of 8 consecutive columns
// (one 16-byte store) -- the same arrangement the packed-weight kernel gets from its pre-packed
// weights, here made by the copy addresses, so the weights need no packing.
// MFMA operand order: A = weight rows, B = token rows; lane l holds token l % 32 of a block.
// K order: lane half h holds K elements [32 h + 8 q, +8) for slice q on both operands.
//
// Scheduling: the (segment, m, n) tile list is split into 8 contiguous shares, one per XCD, and
// each XCD's workgroups take its tiles round-robin. A partial m tile (the last of a segment)
// multiplies only the 32-token blocks that hold rows and skips copies of rows past the segment.
#include <stdlib.h>
#include <type_traits>

#include "common.h"

namespace ntmoe {
namespace {

typedef __attribute__((address_space(1))) void gvoid;
typedef __attribute__((address_space(3))) void lvoid;

constexpr int kBufferWord3 = 0x00020000;
constexpr int kTM = 256;                       // token rows per tile
constexpr int kTN = 256;                       // weight rows per tile
constexpr int kTK = 64;                        // K per step
constexpr int kRowBytes = kTK * 2;             // 128
constexpr int kOperBytes = kTM * kRowBytes;    // 32 KB per operand per stage
constexpr int kStageBytes = 2 * kOperBytes;    // 64 KB
constexpr int kStages = 2;
constexpr int kBlocksPerTile = kTN / 32;                // weight blocks of 32 rows per tile (8)
static_assert(kTM == kTN, "one copy pattern serves both operands");

__host__ __device__ constexpr int block_row(int p) { return p ^ (((p >> 2) ^ (p >> 3)) & 1) * 12; }
__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }

__device__ __forceinline__ void barrier_nofence() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

struct Tile {
  int s, nt, m0, seg_end;
};

template <int EPI>
__device__ __forceinline__ int weight_row(int nt, int p_tile, int n_out, int R) {
  // LDS weight row p_tile (0..255) of n tile nt -> global weight row of the segment.
  const int b = p_tile >> 5, i = block_row(p_tile & 31);
  const int nb = nt * kBlocksPerTile + b;
  int row;
  if (EPI == NT_MOE_EPI_SWIGLU) row = i < 16 ? 16 * nb + i : n_out + 16 * nb + (i - 16);
  else row = 32 * nb + i;
  return row < R ? row : R - 1;
}

// KEEP: also store the epilogue's input, the fc1 pre-activations, to Pre: bf16 [rows, R]
// (SwiGLU: gate columns then value columns; ReLU^2: the output's columns), rounded from the same
// fp32 accumulators, for the backward.
template <int EPI, bool GATHER, bool KEEP = false>
__global__ __launch_bounds__(512, 1) void grouped_gemm_t256_kernel(
    const uint16_t* __restrict__ A, int64_t ld_a, int64_t a_rows,
    const int32_t* __restrict__ src_row, const int32_t* __restrict__ seg_offsets, int S,
    int total_rows, const uint16_t* __restrict__ W, int K, int n_out,
    uint16_t* __restrict__ Cout, uint16_t* __restrict__ Pre) {
  extern __shared__ __align__(16) unsigned char smem[];
  int* tile_prefix = reinterpret_cast<int*>(smem + kStages * kStageBytes);  // [S+1]
  int* seg_lo = tile_prefix + (S + 1);                                      // [S+1]

  constexpr int NW = 8;                                 // waves
  constexpr int kCopies = kOperBytes / (64 * NW * 16);  // copy instructions per operand per lane
  constexpr int kCRows = 8 * kCopies;                   // LDS rows each wave copies per operand
  constexpr int kWB = 16 / NW;                          // weight blocks per wave
  const int lane = lane_id(), wave = wave_id();
  const int R = EPI == NT_MOE_EPI_SWIGLU ? 2 * n_out : n_out;  // weight rows per segment
  // weight blocks: SwiGLU blocks pair 16 gate with 16 value rows (n_out % 16 == 0); other
  // epilogues take 32 rows per block, the last one clamped when R is not a multiple of 32
  const int NB = EPI == NT_MOE_EPI_SWIGLU ? n_out / 16 : (R + 31) / 32;
  const int n_tiles = (NB + kBlocksPerTile - 1) / kBlocksPerTile;
  const int nk = K / kTK;
  __builtin_assume(nk >= 2);

  // Segment table (clamped, non-decreasing) and the tile prefix over segments.
  for (int i = threadIdx.x; i <= S; i += blockDim.x) {
    int o = seg_offsets[i];
    seg_lo[i] = o < 0 ? 0 : (o > total_rows ? total_rows : o);
  }
  __syncthreads();
  if (wave == 0) {
    int run_max = 0, run_tiles = 0;
    for (int base = 0; base <= S; base += 64) {
      const int i = base + lane;
      int o = i <= S ? seg_lo[i] : total_rows;
      for (int w = 1; w < 64; w <<= 1) {
        int u = __shfl_up(o, w);
        if (lane >= w) o = o > u ? o : u;
      }
      o = o > run_max ? o : run_max;
      int prev = __shfl_up(o, 1);
      if (lane == 0) prev = run_max;
      int t = i >= 1 && i <= S ? ((o - prev + kTM - 1) / kTM) * n_tiles : 0;
      for (int w = 1; w < 64; w <<= 1) {
        int u = __shfl_up(t, w);
        if (lane >= w) t += u;
      }
      if (i <= S) {
        seg_lo[i] = o;
        tile_prefix[i] = run_tiles + t;
      }
      run_max = __shfl(o, 63);
      run_tiles += __shfl(t, 63);
    }
  }
  __syncthreads();

  const int total = __builtin_amdgcn_readfirstlane(tile_prefix[S]);
  const int xcd = blockIdx.x % 8, local = blockIdx.x / 8, per_xcd = gridDim.x / 8;
  const int t_begin = (int)((int64_t)total * xcd / 8);
  const int t_end = (int)((int64_t)total * (xcd + 1) / 8);
  const int n_my = (t_end - t_begin - local + per_xcd - 1) / per_xcd;
  if (n_my <= 0) return;

  auto locate = [&](int idx, Tile& t) {
    const int tl = t_begin + local + idx * per_xcd;
    int cnt = 0;
    for (int base = 0; base < S; base += 64) {
      const int i = base + lane;
      cnt += __popcll(__ballot(i < S && tile_prefix[i] <= tl));
    }
    t.s = __builtin_amdgcn_readfirstlane(cnt - 1);
    const int lt = tl - __builtin_amdgcn_readfirstlane(tile_prefix[t.s]);
    const int mt = lt / n_tiles;
    t.nt = lt - mt * n_tiles;
    t.seg_end = __builtin_amdgcn_readfirstlane(seg_lo[t.s + 1]);
    t.m0 = __builtin_amdgcn_readfirstlane(seg_lo[t.s]) + mt * kTM;
  };

  // ---- copies --------------------------------------------------------------------------
  // Copy instruction i of this wave covers LDS rows kCRows wave + 8 i + [0, 8) of each operand;
  // lane l writes row kCRows wave + 8 i + l / 8, physical chunk l % 8, i.e. logical chunk
  // (l % 8) ^ ((row / 2) % 8) (kCRows is a multiple of 16, so the row parity is that of 8 i).
  const int crow = lane >> 3;
  const uint32_t cchunk[2] = {(uint32_t)(((lane & 7) ^ ((crow >> 1) & 7)) << 4),
                              (uint32_t)(((lane & 7) ^ (((8 + crow) >> 1) & 7)) << 4)};
  // per-lane byte offsets of the A and B rows of the current tile (K step 0)
  uint32_t aoff[kCopies], boff[kCopies];
  const char* wseg = nullptr;  // this tile's segment weights
  int nidx[kCopies];            // the next tile's gathered row indices

  auto set_b = [&](const Tile& t) {
    wseg = reinterpret_cast<const char*>(W) + (int64_t)t.s * R * (int64_t)K * 2;
#pragma unroll
    for (int i = 0; i < kCopies; ++i) {
      const int p = kCRows * wave + 8 * i + crow;
      boff[i] = (uint32_t)weight_row<EPI>(t.nt, p, n_out, R) * (uint32_t)K * 2u + cchunk[i & 1];
    }
  };
  // Loads the gathered indices of tile t's rows this lane copies (into nidx).
  auto load_idx = [&](const Tile& t) {
#pragma unroll
    for (int i = 0; i < kCopies; ++i) {
      const int r = t.m0 + kCRows * wave + 8 * i + crow;
      const int rr = r < t.seg_end ? r : t.seg_end - 1;
      nidx[i] = GATHER ? src_row[rr] : rr;
    }
  };
  auto set_a = [&](const Tile& t) {
#pragma unroll
    for (int i = 0; i < kCopies; ++i) {
      int64_t r = nidx[i];
      r = r < 0 ? 0 : (r >= a_rows ? a_rows - 1 : r);
      aoff[i] = (uint32_t)(r * ld_a * 2) + cchunk[i & 1];
    }
  };
  // Copy c (of 2 kCopies) of stage kt: the weight rows first, then the token rows.
  auto copy = [&](int kt, int slot, int c) __attribute__((always_inline)) {
    unsigned char* sa = smem + slot * kStageBytes + wave * kCRows * kRowBytes;
    unsigned char* sb = sa + kOperBytes;
    if (c < kCopies)
      __builtin_amdgcn_global_load_lds((gvoid*)(wseg + kt * kRowBytes + boff[c]),
                                       (lvoid*)(sb + c * 1024), 16, 0, 0);
    else
      __builtin_amdgcn_global_load_lds(
          (gvoid*)(reinterpret_cast<const char*>(A) + kt * kRowBytes + aoff[c - kCopies]),
          (lvoid*)(sa + (c - kCopies) * 1024), 16, 0, 0);
  };
  auto issue = [&](int kt, int slot) {
#pragma unroll
    for (int c = 0; c < 2 * kCopies; ++c) copy(kt, slot, c);
  };

  // ---- fragments -----------------------------------------------------------------------
  const int wm = wave / (NW / 2), wn = wave % (NW / 2);  // token half, weight part of the tile
  int frag_off[4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
    frag_off[q] = (lane & 31) * kRowBytes + (swz(lane & 31, 4 * (lane >> 5) + q) << 4);

  const __amdgpu_buffer_rsrc_t out_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      Cout, 0, (int)((int64_t)total_rows * n_out * 2), kBufferWord3);
  const __amdgpu_buffer_rsrc_t pre_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      KEEP ? Pre : Cout, 0, KEEP ? (int)((int64_t)total_rows * R * 2) : 0, kBufferWord3);

  // Fragment reads of slice q of stage `slot`: the wave's kWB weight blocks and 4 token blocks
  // (all 4 even in a partial tile: reading rows nobody copied is harmless, their products are
  // dropped). Issued as inline assembly so they stay where they are written (ahead of the MFMAs
  // of the previous slice) and land in registers of their own; frag_wait() then waits for them
  // with a count that names those registers.
  auto read_frags = [&](int slot, int q, bf16x8 (&wf)[kWB], bf16x8 (&tf)[4]) {
    const uint32_t a_addr = (uint32_t)(uintptr_t)(smem + slot * kStageBytes) +
                            wm * 128 * kRowBytes + frag_off[q];
    const uint32_t b_addr =
        a_addr - wm * 128 * kRowBytes + kOperBytes + wn * (32 * kWB) * kRowBytes;
    static_assert(kWB == 2, "two weight blocks per wave");
    asm volatile("ds_read_b128 %0, %1" : "=v"(wf[0]) : "v"(b_addr));
    asm volatile("ds_read_b128 %0, %1 offset:4096" : "=v"(wf[1]) : "v"(b_addr));
    asm volatile("ds_read_b128 %0, %1" : "=v"(tf[0]) : "v"(a_addr));
    asm volatile("ds_read_b128 %0, %1 offset:4096" : "=v"(tf[1]) : "v"(a_addr));
    asm volatile("ds_read_b128 %0, %1 offset:8192" : "=v"(tf[2]) : "v"(a_addr));
    asm volatile("ds_read_b128 %0, %1 offset:12288" : "=v"(tf[3]) : "v"(a_addr));
  };
  auto frag_wait = [](bf16x8 (&wf)[kWB], bf16x8 (&tf)[4]) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(wf[0]), "+v"(wf[1]), "+v"(tf[0]), "+v"(tf[1]), "+v"(tf[2]), "+v"(tf[3])
                 :
                 : "memory");
  };

  // ---- prologue ------------------------------------------------------------------------
  Tile ct;
  locate(0, ct);
  load_idx(ct);
  set_a(ct);
  set_b(ct);
  issue(0, 0);
#pragma unroll
  for (int c = kCopies; c < 2 * kCopies; ++c) copy(1, 1, c);  // stage 1's token rows
  Tile nt_tile = ct;
  bool has_next = n_my > 1;
  if (has_next) locate(1, nt_tile);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  barrier_nofence();

  // Per K step: slices 0-2 are multiplied between the step's start and its barrier, slice 3
  // after it, overlapping the next step's first fragment reads (slice 3's fragments are read
  // before the barrier, so the slot may be refilled meanwhile). fr0 holds slices 0 and 2, fr1
  // slices 1 and 3. The next stage's copies go out at the start of the step.
  bf16x8 wf0[kWB], tf0[4], wf1[kWB], tf1[4];
  read_frags(0, 0, wf0, tf0);
  frag_wait(wf0, tf0);
  int g = 0;
  for (int ti = 0;; ++ti) {
    const int live_m = ct.seg_end - ct.m0 - 128 * wm;  // rows of this wave's token half
    if (has_next) load_idx(nt_tile);  // used by the tile's last step; lands by the first wait

    // K loop and epilogue of one tile for NJ live 32-token blocks in this wave's half (the
    // accumulators are local to each variant).
    auto tile_pass = [&](auto nj_c) {
      constexpr int NJ = decltype(nj_c)::value;
      floatx16 acc[kWB][NJ > 0 ? NJ : 1];
#pragma unroll
      for (int b = 0; b < kWB; ++b)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[b][j] = floatx16{};
      auto mfmas = [&](const bf16x8 (&wf)[kWB], const bf16x8 (&tf)[4]) {
#pragma unroll
        for (int b = 0; b < kWB; ++b)
#pragma unroll
          for (int j = 0; j < NJ; ++j)
            acc[b][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[b], tf[j], acc[b][j], 0, 0, 0);
      };
      // The same, with copies c0, c0 + 1, ... of the next stage spread evenly between the MFMAs
      // (issued together ahead of them they held back the first products).
      auto mfmas_copies = [&](const bf16x8 (&wf)[kWB], const bf16x8 (&tf)[4], int kt_next,
                              int slot_next, int c0) __attribute__((always_inline)) {
        constexpr int kPer = kCopies;         // copies per slice (two slices carry them)
        constexpr int kGap = 4 * kWB / kPer;  // MFMA positions per copy
#pragma unroll
        for (int b = 0; b < kWB; ++b)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if (j < NJ)
              acc[b][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[b], tf[j], acc[b][j], 0, 0, 0);
            const int n = b * 4 + j;
            if (kt_next >= 0 && n % kGap == kGap - 1) {
              __builtin_amdgcn_sched_barrier(0);
              copy(kt_next, slot_next, c0 + n / kGap);
              __builtin_amdgcn_sched_barrier(0);
            }
          }
      };
      // K step kt from slot g & 1. Stage s's copies go out in two halves, each spread over one
      // slice: its token rows (gathered: the longer latency) during slice 3 of step s - 2, right
      // after the barrier that frees the slot, its weight rows during slice 0 of step s - 1; the
      // wait before step s - 1's barrier completes both. Past the tile's last stages the halves
      // are the next tile's stages 0 and 1, whose row offsets are set after step nk - 2's
      // barrier (every copy of this tile has gone out by then).
      auto body = [&](int kt, bool read_next, auto set_c) {
        constexpr bool kSet = decltype(set_c)::value;  // step nk - 2: take the next tile's rows
        const int slot = g & 1;
        const int kt_w = kt + 1 < nk ? kt + 1 : (has_next ? kt + 1 - nk : -1);
        __builtin_amdgcn_sched_barrier(0);
        read_frags(slot, 1, wf1, tf1);
        __builtin_amdgcn_sched_barrier(0);
        mfmas_copies(wf0, tf0, kt_w, slot ^ 1, 0);  // stage kt + 1: weight rows
        __builtin_amdgcn_sched_barrier(0);
        frag_wait(wf1, tf1);
        read_frags(slot, 2, wf0, tf0);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(wf1, tf1);
        __builtin_amdgcn_sched_barrier(0);
        frag_wait(wf0, tf0);
        read_frags(slot, 3, wf1, tf1);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(wf0, tf0);
        __builtin_amdgcn_sched_barrier(0);
        frag_wait(wf1, tf1);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        barrier_nofence();
        ++g;
        if constexpr (kSet) {
          if (has_next) {  // the next tile's rows (its indices landed above)
            set_a(nt_tile);
            set_b(nt_tile);
          }
        }
        const int kt_t = kt + 2 < nk ? kt + 2 : (has_next ? kt + 2 - nk : -1);
        if (read_next) read_frags(g & 1, 0, wf0, tf0);
        __builtin_amdgcn_sched_barrier(0);
        mfmas_copies(wf1, tf1, kt_t, slot, kCopies);  // stage kt + 2: token rows
        __builtin_amdgcn_sched_barrier(0);
        if (read_next) frag_wait(wf0, tf0);
      };
      for (int kt = 0; kt + 2 < nk; ++kt) body(kt, true, std::false_type());
      body(nk - 2, true, std::true_type());
      body(nk - 1, has_next, std::false_type());

      // Epilogue: lane (token j, half h) holds logical block rows 8 h + [0, 8) in elements 0-7
      // and 16 + 8 h + [0, 8) in 8-15: for SwiGLU gate and value of output columns
      // 16 nb + 8 h + [0, 8), otherwise columns 32 nb + 8 h + [0, 8) and 32 nb + 16 + 8 h + [0, 8).
      // Rows past the segment and columns past n_out are dropped by the buffer range check.
      const int hbit = lane >> 5;
#pragma unroll
      for (int b = 0; b < kWB; ++b) {
        const int nb = ct.nt * kBlocksPerTile + wn * kWB + b;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const int m = ct.m0 + wm * 128 + j * 32 + (lane & 31);
          const bool row_ok = m < ct.seg_end;
#pragma unroll
          for (int st = 0; st < (EPI == NT_MOE_EPI_SWIGLU ? 1 : 2); ++st) {
            int col;
            float v[8];
            if (EPI == NT_MOE_EPI_SWIGLU) {
              col = nb * 16 + 8 * hbit;
#pragma unroll
              for (int r = 0; r < 8; ++r) {
                const float a = acc[b][j][r], u = acc[b][j][8 + r];
                v[r] = a * u * __builtin_amdgcn_rcpf(1.f + __expf(-a));
              }
            } else {
              col = nb * 32 + 16 * st + 8 * hbit;
#pragma unroll
              for (int r = 0; r < 8; ++r) {
                const float a = acc[b][j][8 * st + r];
                v[r] = EPI == NT_MOE_EPI_RELU2 ? (a > 0.f ? a * a : 0.f) : a;
              }
            }
            const u32x4 packed = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                  pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7])};
            const bool ok = row_ok && nb < NB && col < n_out;
            const uint32_t voff = ok ? (uint32_t)(((int64_t)m * n_out + col) * 2) : 0x80000000u;
            __builtin_amdgcn_raw_buffer_store_b128(packed, out_rsrc, voff, 0, 0);
            if constexpr (KEEP) {
              // the accumulators behind these columns: SwiGLU gate (elements 0-7) at col and
              // value (8-15) at n_out + col of a [rows, 2 n_out] row; otherwise elements
              // 8 st .. 8 st + 7 at col of a [rows, n_out] row
              const int e0 = EPI == NT_MOE_EPI_SWIGLU ? 0 : 8 * st;
#pragma unroll
              for (int part = 0; part < (EPI == NT_MOE_EPI_SWIGLU ? 2 : 1); ++part) {
                const int eb = e0 + 8 * part;
                const floatx16& av = acc[b][j];
                const u32x4 pk = {pack_bf16x2(av[eb], av[eb + 1]), pack_bf16x2(av[eb + 2], av[eb + 3]),
                                  pack_bf16x2(av[eb + 4], av[eb + 5]),
                                  pack_bf16x2(av[eb + 6], av[eb + 7])};
                const uint32_t poff =
                    ok ? (uint32_t)(((int64_t)m * R + col + part * n_out) * 2) : 0x80000000u;
                __builtin_amdgcn_raw_buffer_store_b128(pk, pre_rsrc, poff, 0, 0);
              }
            }
          }
        }
      }
    };
    if (live_m > 64) tile_pass(std::integral_constant<int, 4>());
    else if (live_m > 32) tile_pass(std::integral_constant<int, 2>());
    else if (live_m > 0) tile_pass(std::integral_constant<int, 1>());
    else tile_pass(std::integral_constant<int, 0>());

    if (!has_next) break;
    ct = nt_tile;
    has_next = ti + 2 < n_my;
    if (has_next) locate(ti + 2, nt_tile);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

template <int EPI, bool GATHER, bool KEEP = false>
hipError_t launch_t256(const uint16_t* a, int64_t ld_a, int64_t a_rows, const int32_t* src_row,
                       const int32_t* seg_offsets, int S, int64_t total_rows, const uint16_t* w,
                       int K, int n_out, uint16_t* c, hipStream_t stream,
                       uint16_t* pre = nullptr) {
  const int R = EPI == NT_MOE_EPI_SWIGLU ? 2 * n_out : n_out;
  const int64_t n_tiles = ((R + 31) / 32 + kBlocksPerTile - 1) / kBlocksPerTile;
  const int64_t upper = ((total_rows + kTM - 1) / kTM + S) * n_tiles;
  int64_t grid = num_cus();
  if (upper < grid) grid = upper;
  grid = ((grid + 7) / 8) * 8;
  const size_t lds = (size_t)kStages * kStageBytes + (size_t)(2 * S + 2) * sizeof(int);
  auto kern = grouped_gemm_t256_kernel<EPI, GATHER, KEEP>;
  hipError_t err = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds);
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(512), lds, stream, a, ld_a, a_rows,
                     src_row, seg_offsets, S, (int)total_rows, w, K, n_out, c, pre);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_grouped_gemm_bf16_t256(const uint16_t* a, int64_t ld_a, int64_t a_rows,
                                         const int32_t* src_row, const int32_t* seg_offsets,
                                         int num_segments, int64_t total_rows, const uint16_t* w,
                                         int K, int n_out, int epilogue, uint16_t* c,
                                         hipStream_t stream) {
  if (total_rows == 0) return hipSuccess;
#define NT_T(EPI)                                                                          \
  return src_row ? launch_t256<EPI, true>(a, ld_a, a_rows, src_row, seg_offsets,           \
                                          num_segments, total_rows, w, K, n_out, c, stream) \
                 : launch_t256<EPI, false>(a, ld_a, a_rows, src_row, seg_offsets,          \
                                           num_segments, total_rows, w, K, n_out, c, stream)
  switch (epilogue) {
    case NT_MOE_EPI_SWIGLU: NT_T(NT_MOE_EPI_SWIGLU);
    case NT_MOE_EPI_RELU2: NT_T(NT_MOE_EPI_RELU2);
    default: NT_T(NT_MOE_EPI_NONE);
  }
#undef NT_T
}

hipError_t launch_grouped_gemm_bf16_t256_keep(const uint16_t* a, int64_t ld_a, int64_t a_rows,
                                              const int32_t* src_row, const int32_t* seg_offsets,
                                              int num_segments, int64_t total_rows,
                                              const uint16_t* w, int K, int n_out, int epilogue,
                                              uint16_t* c, uint16_t* pre, hipStream_t stream) {
  if (total_rows == 0) return hipSuccess;
#define NT_TK(EPI)                                                                            \
  return src_row ? launch_t256<EPI, true, true>(a, ld_a, a_rows, src_row, seg_offsets,        \
                                                num_segments, total_rows, w, K, n_out, c,     \
                                                stream, pre)                                  \
                 : launch_t256<EPI, false, true>(a, ld_a, a_rows, src_row, seg_offsets,       \
                                                 num_segments, total_rows, w, K, n_out, c,    \
                                                 stream, pre)
  switch (epilogue) {
    case NT_MOE_EPI_SWIGLU: NT_TK(NT_MOE_EPI_SWIGLU);
    default: NT_TK(NT_MOE_EPI_RELU2);
  }
#undef NT_TK
}

}  // namespace ntmoe
