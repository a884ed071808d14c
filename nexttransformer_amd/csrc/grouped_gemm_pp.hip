// Grouped expert GEMM on bf16 MFMA, packed weights, two wave groups in a ping-pong schedule.
//
// Same computation and the same packed weight layout as grouped_gemm_packed.hip (SequentialMLP's
// per-expert fc1/fc2, megatron_moe.py:145, over MasterLinear, :58-78, with the SwiGLU / ReLU^2
// epilogue fused):  c[r, j] = epilogue(a_src(r) . w_s[j, :])  for every row r of segment s.
// Each output element accumulates the same MFMA slices in the same order, so the two kernels
// give identical bits.
//
// What differs is how the matrix cores are fed. One workgroup of 8 waves per CU owns a tile of
// 256 tokens x 256 weight rows. Both operands of a 64-wide K step are staged in LDS (64 KB per
// stage, two stages): the token rows (gathered through src_row for the up projection) and the 8
// packed 32-row weight blocks. Wave w = 4 g + s (g: group, s: SIMD) computes the 128 tokens of
// half g against weight blocks 2 s and 2 s + 1, i.e. 8 accumulators of 32 x 32 -- the same
// per-wave shape as the 4-wave packed kernel -- but the weights are read from LDS, once per
// workgroup, instead of by every wave from L2: per K step and 256 x 256 tile the CU takes 64 KB
// from L2 instead of 96 KB.
//
// The two waves of a SIMD (one per group) alternate phases: while group 0 runs the 32 MFMAs of
// K step j from registers, group 1 reads its fragments of step j from LDS; then group 1
// multiplies while group 0 reads step j + 1. One workgroup barrier separates two phases, group 1
// having passed one extra barrier first, so a wave never waits for its own operands while its
// SIMD's matrix core could run the other wave's products. Group 1 also streams the stages:
// during its compute phase of step j (after the barrier by which every wave has read step j)
// it issues the direct-to-LDS loads of step j + 2 into that stage, and at the end of its next
// memory phase it waits for them, before the barrier that lets group 0 read them: about two
// phases of load latency. A tile's epilogue (activation, bf16, transposed 16-byte stores,
// optional fc1 pre-activations) runs in the wave's next memory phase.
#include <stdlib.h>

#include <type_traits>

#include "common.h"

namespace ntmoe {
namespace {

typedef __attribute__((address_space(1))) void gvoid;
typedef __attribute__((address_space(3))) void lvoid;

constexpr int kBufferWord3 = 0x00020000;

constexpr int kBK = 64;                         // K per step
constexpr int kRB = kBK * 2;                    // bytes of one staged token row (one K step)
constexpr int kCH = kRB / 16;                   // 16-byte chunks per token row (8)
constexpr int kWIN = 256 / kRB;                 // token rows per 256-byte bank window (2)
constexpr int kRPI = 64 / kCH;                  // token rows per load instruction (8)
constexpr int kBM = 256;                        // tokens per tile
constexpr int kHalf = kBM / 2;                  // tokens per wave group
constexpr int kTB = 8;                          // packed 32-row weight blocks per tile
constexpr int kBlockBytes = 32 * kRB;           // one packed block, one K step (4 KB)
constexpr int kBlockElems = kBlockBytes / 2;
constexpr int kTokBytes = kBM * kRB;            // token part of a stage (32 KB)
constexpr int kStage = kTokBytes + kTB * kBlockBytes;  // 64 KB
constexpr int kXposeBytes = 2048;               // per-wave scratch of the epilogue's transpose
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kMinSteps = 4;                    // the gather table needs four K steps of lead
constexpr int kTokLoads = kBM / kRPI / 4;       // token-row load instructions per loader wave (8)
constexpr int kWLoads = 2 * (kBlockBytes / 1024);  // weight load instructions per loader wave (8)

__host__ __device__ size_t pp_lds_bytes(int S) {
  return 2 * (size_t)kStage + (size_t)kWaves * kXposeBytes + 2 * kBM * sizeof(int) +
         (size_t)(2 * S + 2) * sizeof(int);
}

// Row order inside a packed 32-row block (the packed kernel's): position p holds logical row
// block_row(p), so each lane's accumulator holds 8 consecutive output columns.
template <int EPI>
struct Ep {
  static constexpr int kStores = EPI == NT_MOE_EPI_SWIGLU ? 1 : 2;  // 16-byte stores per lane
};                                                                   // per 32-token block

__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row / kWIN) % kCH); }

// The lane id computed afresh: inside the main loop every register is taken by accumulators and
// operand fragments, so lane-derived values are recomputed where they are needed instead of
// being kept live (a value the compiler hoists out of the loop gets spilled, and its reload's
// wait would also wait for the direct-to-LDS loads in flight).
__device__ __forceinline__ int fresh_lane() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

__device__ __forceinline__ void barrier_all() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

struct Tile {
  int s, nt, m0, seg_end;
};

template <int EPI, bool GATHER, bool KEEP>
__global__ __launch_bounds__(kThreads, 1) void grouped_gemm_pp_kernel(
    const uint16_t* __restrict__ A, int64_t ld_a, const int32_t* __restrict__ src_row,
    const int32_t* __restrict__ seg_offsets, int S, int total_rows, int64_t a_rows,
    const uint16_t* __restrict__ Wp, int K, int n_out, uint16_t* __restrict__ Cout,
    uint16_t* __restrict__ Pre) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int lane = lane_id(), wave = wave_id();
  const int grp = wave >> 2, sub = wave & 3;
  unsigned char* xpose = smem + 2 * kStage + wave * kXposeBytes;
  int* src_tab = reinterpret_cast<int*>(smem + 2 * kStage + kWaves * kXposeBytes);  // [2][kBM]
  int* tile_prefix = src_tab + 2 * kBM;                                            // [S+1]
  int* seg_lo = tile_prefix + (S + 1);                                             // [S+1]

  const int NB = (EPI == NT_MOE_EPI_SWIGLU ? 2 * n_out : n_out) / 32;  // packed 32-row blocks
  const int n_tiles = (NB + kTB - 1) / kTB;
  const int nk = K / kBK;
  __builtin_assume(nk >= kMinSteps);

  // Segment table (clamped, non-decreasing) and tile prefix: the packed kernel's construction.
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
      int t = i >= 1 && i <= S ? ((o - prev + kBM - 1) / kBM) * n_tiles : 0;
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

  // Tiles: an XCD-contiguous share of the list, round-robin over the XCD's workgroups.
  const int total = __builtin_amdgcn_readfirstlane(tile_prefix[S]);
  const int xcd = blockIdx.x % 8, local = blockIdx.x / 8, per_xcd = gridDim.x / 8;
  const int t_begin = (int)((int64_t)total * xcd / 8);
  const int t_end = (int)((int64_t)total * (xcd + 1) / 8);
  const int n_x = t_end - t_begin;
  const int n_my = n_x > local ? (n_x - local + per_xcd - 1) / per_xcd : 0;
  if (n_my == 0) return;  // uniform over the workgroup

  // The idx-th tile of this workgroup -> segment and position (one ballot per 64 segments).
  auto locate = [&](int idx) {
    const int tl = t_begin + local + idx * per_xcd;
    const int lane = fresh_lane();
    int cnt = 0;
    for (int base = 0; base < S; base += 64) {
      const int i = base + lane;
      cnt += __popcll(__ballot(i < S && tile_prefix[i] <= tl));
    }
    Tile t;
    t.s = __builtin_amdgcn_readfirstlane(cnt - 1);
    const int lt = tl - __builtin_amdgcn_readfirstlane(tile_prefix[t.s]);
    const int mt = lt / n_tiles;
    t.nt = lt - mt * n_tiles;
    t.seg_end = __builtin_amdgcn_readfirstlane(seg_lo[t.s + 1]);
    t.m0 = __builtin_amdgcn_readfirstlane(seg_lo[t.s]) + mt * kBM;
    return t;
  };

  // ---- loaders ---------------------------------------------------------------------------------
  // Loads are issued only in memory phases (a load that waits for room in the CU's memory queue
  // would otherwise hold up the MFMAs behind it). Group 0, in its memory phase of step j, loads
  // the 8 weight blocks of step j + 1 (wave sub: blocks 2 sub, 2 sub + 1). Group 1, in its
  // memory phase of step j, loads the token rows: rows 128 .. 255 of step j + 1 (its own half,
  // which it read from that stage two phases ago) and rows 0 .. 127 of step j + 2 (group 0's
  // half, read by group 0 one phase ago); wave sub takes rows sub * 32 .. + 32 of each half.
  // Each phase thus carries 32 KB of loads.
  const char* abase = reinterpret_cast<const char*>(A);
  static_assert(2 * kRPI == kWIN * kCH, "swizzle period of two load instructions");
  constexpr int kTL = 32 / kRPI;  // token-row load instructions per half and step (4)
  // The direct-to-LDS loads are issued from inline assembly, so the compiler does not see LDS
  // writes in flight: it would otherwise wait for every outstanding load before any LDS read.
  // Their completion is ordered by hand (vmcnt waits before the workgroup barriers).
  // LDS destination m0 (wave-uniform), global address = 64-bit scalar base + 32-bit lane offset.
  auto dma16 = [](const void* base, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :: "s"(lds), "v"(voff), "s"(base) : "memory", "m0");
  };
  auto dma4 = [](const void* base, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2"
                 :: "s"(lds), "v"(voff), "s"(base) : "memory", "m0");
  };
  const uint32_t lds_base = (uint32_t)reinterpret_cast<uintptr_t>((lvoid*)smem);
  const uint32_t tab_base = lds_base + 2 * kStage + kWaves * kXposeBytes;  // src_tab
  // A loader cursor: the tile and K step it loads next.
  struct Cursor {
    int idx, kt;
    Tile t;
  };
  // Gather table slot layout: group-1 wave sub's 64 entries at sub * 64: lanes 0-31 rows
  // sub * 32 + l (half 0), lanes 32-63 rows 128 + sub * 32 + l - 32 (half 1).
  auto load_indices = [&](const Tile& t, int slot) {
    const int lane = fresh_lane();
    const int r = (lane < 32 ? 0 : kHalf - 32) + sub * 32 + lane;
    const int gr = t.m0 + r < t.seg_end ? t.m0 + r : t.seg_end - 1;
    dma4(src_row, (uint32_t)gr * 4, tab_base + (slot * kBM + sub * 64) * 4);
  };
  // per-lane offsets of group-1 wave sub's token rows of half h in tile t
  auto token_tile = [&](const Tile& t, int slot, int h, uint32_t (&off)[kTL]) {
    const int lane = fresh_lane();
    const int lrow = lane / kCH, lphys = lane % kCH;
    const uint32_t aswz[2] = {(uint32_t)swz(lrow, lphys) * 16,
                              (uint32_t)swz(kRPI + lrow, lphys) * 16};
#pragma unroll
    for (int q = 0; q < kTL; ++q) {
      const int rl = q * kRPI + lrow;  // row within the wave's 32
      int64_t r;
      if (GATHER) r = src_tab[slot * kBM + sub * 64 + h * 32 + rl];
      else {
        const int row = h * kHalf + sub * 32 + rl;
        r = t.m0 + row < t.seg_end ? t.m0 + row : t.seg_end - 1;
      }
      r = r < 0 ? 0 : (r >= a_rows ? a_rows - 1 : r);
      off[q] = (uint32_t)(r * ld_a * 2) + aswz[q % 2];
    }
  };
  // group 1: token-row load instruction q of half h, K step kt, into stage `slot`
  auto load_tokens = [&](const uint32_t (&off)[kTL], int h, int kt, int slot, int q) {
    dma16(abase + kt * kRB, off[q],
          lds_base + slot * kStage + (h * kHalf + sub * 32 + q * kRPI) * kRB);
  };
  const char* wblk[2];  // group 0: its weight blocks in the weight cursor's tile
  auto weight_tile = [&](const Tile& t) {
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      int nb = t.nt * kTB + 2 * sub + rb;
      nb = nb < NB ? nb : NB - 1;
      wblk[rb] = reinterpret_cast<const char*>(Wp + ((int64_t)t.s * NB + nb) * (int64_t)nk * kBlockElems);
    }
  };
  auto load_weights = [&](int kt, int slot) {
    const uint32_t st = lds_base + slot * kStage + kTokBytes + 2 * sub * kBlockBytes;
    const uint32_t lane16 = fresh_lane() * 16;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int q = 0; q < kBlockBytes / 1024; ++q)
        dma16(wblk[rb] + (int64_t)kt * kBlockBytes + q * 1024, lane16,
              st + rb * kBlockBytes + q * 1024);
  };

  const int J = n_my * nk;  // K steps of this workgroup, over all its tiles
  // Cursors (steps 0 and 1 go out in the prologue): group 0's weight cursor wc and group 1's
  // token cursors c0 (half 0) and c1 (half 1) all start at step 2.
  Cursor wc, c0, c1;
  wc.idx = c0.idx = c1.idx = 0;
  wc.kt = c0.kt = c1.kt = 2;
  wc.t = c0.t = c1.t = locate(0);
  uint32_t off0[kTL], off1[kTL];
  if (grp == 0) {
    weight_tile(wc.t);
    load_weights(0, 0);
    load_weights(1, 1);
  } else {
    if (GATHER) {
      load_indices(c0.t, 0);
      if (n_my > 1) load_indices(locate(1), 1);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    token_tile(c0.t, 0, 0, off0);
    token_tile(c1.t, 0, 1, off1);
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int q = 0; q < kTL; ++q) {
        load_tokens(off0, 0, kt, kt, q);
        load_tokens(off1, 1, kt, kt, q);
      }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  barrier_all();
  // Advances a cursor to its next step; false past the last step. Entering a new tile, the
  // weight cursor takes its block addresses, a token cursor its row offsets from the gather
  // table; cursor c1 also sends out the gather indices of the tile after it (counted in
  // *idx_loads), which cursor c0 reaches nk - 1 steps later.
  auto weight_next = [&]() {
    if (wc.idx * nk + wc.kt >= J) return false;
    if (wc.kt == nk) {
      ++wc.idx;
      wc.kt = 0;
      wc.t = locate(wc.idx);
      weight_tile(wc.t);
    }
    return true;
  };
  auto token_next = [&](Cursor& c, int h, uint32_t (&off)[kTL], int& idx_loads) {
    if (c.idx * nk + c.kt >= J) return false;
    if (c.kt == nk) {
      ++c.idx;
      c.kt = 0;
      c.t = locate(c.idx);
      token_tile(c.t, c.idx & 1, h, off);
      if (GATHER && h == 1 && c.idx + 1 < n_my) {
        load_indices(locate(c.idx + 1), (c.idx + 1) & 1);
        ++idx_loads;
      }
    }
    return true;
  };

  // ---- fragment reads ------------------------------------------------------------------------

  const __amdgpu_buffer_rsrc_t out_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      Cout, 0, (int)((int64_t)total_rows * n_out * 2), kBufferWord3);
  constexpr int kPreW = EPI == NT_MOE_EPI_SWIGLU ? 2 : 1;
  __amdgpu_buffer_rsrc_t pre_rsrc = out_rsrc;
  if constexpr (KEEP)
    pre_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        Pre, 0, (int)((int64_t)total_rows * kPreW * n_out * 2), kBufferWord3);

  floatx16 acc[2][4];
  bf16x8 tf[4][4];  // token fragments [block][slice]
  bf16x8 wf[2][4];  // weight fragments [block][slice]
  Tile ct = wc.t;   // the tile being multiplied
  bool live = true;

  // Epilogue of tile ct (the packed kernel's, for this wave's 64 weight rows x 128 tokens).
  auto epilogue = [&]() __attribute__((always_inline)) {
    constexpr bool SW = EPI == NT_MOE_EPI_SWIGLU;
    constexpr int CPR = 2 * (SW ? 2 : 4);  // 16-byte chunks per row of the wave's columns
    constexpr int RPH = kXposeBytes / (CPR * 16) < 32 ? kXposeBytes / (CPR * 16) : 32;
    constexpr int RPS = 64 / CPR;
    static_assert(RPH * CPR * 16 <= kXposeBytes && 32 % RPH == 0 && RPH % RPS == 0, "passes");
    auto xoff = [](int r, int c) { return r * CPR * 16 + ((c ^ ((r / (8 / CPR)) % CPR)) << 4); };
    const int lane = fresh_lane();
    const int hbit = lane >> 5, t = lane & 31;
    const int col0 = (ct.nt * kTB + 2 * sub) * (SW ? 16 : 32);
    const int mrow0 = ct.m0 + grp * kHalf;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u32x4 pk[2][Ep<EPI>::kStores];
      const int m_lane = mrow0 + j * 32 + t;
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int st = 0; st < Ep<EPI>::kStores; ++st) {
          float v[8];
          if (SW) {
#pragma unroll
            for (int r = 0; r < 8; ++r) {
              const float a = acc[rb][j][r], u = acc[rb][j][8 + r];
              v[r] = a * u * __builtin_amdgcn_rcpf(1.f + __expf(-a));
            }
          } else {
#pragma unroll
            for (int r = 0; r < 8; ++r) {
              const float a = acc[rb][j][8 * st + r];
              v[r] = EPI == NT_MOE_EPI_RELU2 ? (a > 0.f ? a * a : 0.f) : a;
            }
          }
          pk[rb][st] = u32x4{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                             pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7])};
          if constexpr (KEEP) {  // the fc1 pre-activations, straight from the accumulator layout
            const int nb = ct.nt * kTB + 2 * sub + rb;
            const int col = SW ? nb * 16 + 8 * hbit : nb * 32 + 16 * st + 8 * hbit;
            const bool ok = m_lane < ct.seg_end && nb < NB && col < n_out;
            const int64_t prow = (int64_t)m_lane * kPreW * n_out;
#pragma unroll
            for (int h = 0; h < (SW ? 2 : 1); ++h) {
              const int e0 = SW ? 8 * h : 8 * st;
              const u32x4 pv = {pack_bf16x2(acc[rb][j][e0], acc[rb][j][e0 + 1]),
                                pack_bf16x2(acc[rb][j][e0 + 2], acc[rb][j][e0 + 3]),
                                pack_bf16x2(acc[rb][j][e0 + 4], acc[rb][j][e0 + 5]),
                                pack_bf16x2(acc[rb][j][e0 + 6], acc[rb][j][e0 + 7])};
              const uint32_t poff = ok ? (uint32_t)((prow + h * n_out + col) * 2) : 0x80000000u;
              __builtin_amdgcn_raw_buffer_store_b128(pv, pre_rsrc, poff, 0, 0);
            }
          }
        }
#pragma unroll
      for (int pass = 0; pass < 32 / RPH; ++pass) {
        if (t / RPH == pass) {
#pragma unroll
          for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int st = 0; st < Ep<EPI>::kStores; ++st)
              *reinterpret_cast<u32x4*>(
                  xpose + xoff(t - pass * RPH, SW ? rb * 2 + hbit : rb * 4 + st * 2 + hbit)) =
                  pk[rb][st];
        }
        asm volatile("" ::: "memory");  // the wave's LDS operations run in order
#pragma unroll
        for (int sidx = 0; sidx < RPH / RPS; ++sidx) {
          const int r = sidx * RPS + lane / CPR, q = lane % CPR;
          const u32x4 val = *reinterpret_cast<const u32x4*>(xpose + xoff(r, q));
          const int m = mrow0 + j * 32 + pass * RPH + r;
          const int col = col0 + q * 8;
          const uint32_t voff = (m < ct.seg_end && col < n_out)
                                    ? (uint32_t)(((int64_t)m * n_out + col) * 2)
                                    : 0x80000000u;
          __builtin_amdgcn_raw_buffer_store_b128(val, out_rsrc, voff, 0, 0);
        }
        asm volatile("" ::: "memory");
      }
    }
  };

  // Stores of one epilogue (fixed per shape). A wait lets the newest n vector memory operations
  // stay in flight (they retire in order): the loads and stores issued after the ones the
  // barrier must cover.
  constexpr int kEpiStores = 4 * (EPI == NT_MOE_EPI_SWIGLU ? 2 : 4) + (KEEP ? 16 : 0);
  auto vm_wait = [&](int n) {
#define NT_VM(N) \
  if (n == (N)) { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); return; }
    NT_VM(0) NT_VM(1) NT_VM(kTL) NT_VM(kTL + 1) NT_VM(2 * kTL) NT_VM(2 * kTL + 1)
    NT_VM(kEpiStores) NT_VM(kEpiStores + kTL) NT_VM(kEpiStores + kTL + 1)
    NT_VM(kEpiStores + 2 * kTL) NT_VM(kEpiStores + 2 * kTL + 1)
#undef NT_VM
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  };

  if (grp == 1) barrier_all();  // group 1 runs one phase behind group 0
  for (int j = 0; j < J; ++j) {
    // ---- memory phase of step j: finish the previous tile, read this step's fragments, load ----
    const int kt = j % nk;
    int pending = 0;  // memory operations of this phase that its wait leaves in flight
    if (kt == 0) {
      if (j > 0 && live) {
        epilogue();
        pending += kEpiStores;
      }
      ct = locate(j / nk);
      live = ct.m0 + grp * kHalf < ct.seg_end && ct.nt * kTB + 2 * sub < NB;
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[rb][b] = floatx16{};
    }
    // Loads of this phase: group 0 the weights of step j + 1 (their stage was read by group 0
    // two phases ago and by group 1 one phase ago); group 1 its own token rows of step j + 1
    // and group 0's of step j + 2 (see above). They go out between the fragment reads, one per
    // three reads, so the LDS reads and the memory queue work at the same time.
    int loaded_last = 0;  // group 1: loads issued after its rows of step j + 1
    bool ld_w = false, ld_1 = false, ld_0 = false;
    int kt_w = 0, kt_1 = 0, kt_0 = 0;
    if (grp == 0) {
      if (j >= 1 && weight_next()) {
        ld_w = true;
        kt_w = wc.kt++;
      }
    } else {
      int idx_loads = 0;
      if (j >= 1 && token_next(c1, 1, off1, idx_loads)) {  // own half, step j + 1
        ld_1 = true;
        kt_1 = c1.kt++;
      }
      if (token_next(c0, 0, off0, idx_loads)) {  // group 0's half, step j + 2
        ld_0 = true;
        kt_0 = c0.kt++;
      }
      const int n1 = ld_1 ? kTL : 0, n0 = ld_0 ? kTL : 0;
      pending += n1 + n0 + idx_loads;
      loaded_last = n0;  // (a gather-index load goes out before the rows of step j + 1)
    }
    const uint32_t w_lds = lds_base + ((j + 1) & 1) * kStage + kTokBytes + 2 * sub * kBlockBytes;
    const unsigned char* st = smem + (j & 1) * kStage;
    // token row (lane & 31) of a 32-token block, K chunk 4 (lane >> 5) + q; weight chunk
    // q * 64 + lane of the wave's blocks
    const int lane = fresh_lane();
    const int w_off = kTokBytes + 2 * sub * kBlockBytes + lane * 16;
    int tok_off[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      tok_off[q] = (lane & 31) * kRB + (swz(lane & 31, 4 * (lane >> 5) + q) << 4);
    auto read = [&](int r) __attribute__((always_inline)) {  // read r of 24: slice r / 6, then
      const int q = r / 6, i = r % 6;                         // 4 token and 2 weight fragments
      if (i < 4)
        tf[i][q] = *reinterpret_cast<const bf16x8*>(st + (grp * kHalf + i * 32) * kRB + tok_off[q]);
      else
        wf[i - 4][q] = *reinterpret_cast<const bf16x8*>(st + w_off + (i - 4) * kBlockBytes + q * 1024);
    };
    // load instruction g of 8 of this wave's loads (no branch inside an interleaved sequence)
    auto load_w = [&](int g) __attribute__((always_inline)) {
      dma16(wblk[g / 4] + (int64_t)kt_w * kBlockBytes + (g % 4) * 1024, lane * 16,
            w_lds + (g / 4) * kBlockBytes + (g % 4) * 1024);
    };
    auto load_t = [&](int g) __attribute__((always_inline)) {
      if (g < kTL) load_tokens(off1, 1, kt_1, (j + 1) & 1, g);
      else load_tokens(off0, 0, kt_0, j & 1, g - kTL);
    };
    const bool all_loads = grp == 0 ? ld_w : (ld_1 && ld_0);
    if (live && all_loads) {
      if (grp == 0) {
#pragma unroll
        for (int g = 0; g < 8; ++g) {
          read(3 * g); read(3 * g + 1); read(3 * g + 2);
          load_w(g);
        }
      } else {
#pragma unroll
        for (int g = 0; g < 8; ++g) {
          read(3 * g); read(3 * g + 1); read(3 * g + 2);
          load_t(g);
        }
      }
    } else {
      if (live) {
#pragma unroll
        for (int r = 0; r < 24; ++r) read(r);
      }
      if (grp == 0) {
        if (ld_w) {
#pragma unroll
          for (int g = 0; g < 8; ++g) load_w(g);
        }
      } else {
        if (ld_1) {
#pragma unroll
          for (int g = 0; g < kTL; ++g) load_t(g);
        }
        if (ld_0) {
#pragma unroll
          for (int g = kTL; g < 2 * kTL; ++g) load_t(g);
        }
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    // group 1: group 0's token rows of step j + 1 (issued in its previous memory phase) have
    // landed before the barrier after which group 0 reads them
    if (grp == 1) vm_wait(pending);
    barrier_all();
    // ---- compute phase of step j ----
    __builtin_amdgcn_s_setprio(1);
    if (live) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
          for (int rb = 0; rb < 2; ++rb)
            acc[rb][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[rb][q], tf[b][q], acc[rb][b],
                                                                 0, 0, 0);
    }
    __builtin_amdgcn_s_setprio(0);
    // group 0: the weights of step j + 1 have landed; group 1: its own token rows of step j + 1
    // (group 0's rows of step j + 2 and gather indices may stay in flight)
    vm_wait(grp == 0 ? 0 : loaded_last);
    barrier_all();
  }
  if (live) epilogue();
  if (grp == 0) barrier_all();
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the trailing loads land before LDS is freed
}

template <int EPI, bool GATHER, bool KEEP>
hipError_t launch_pp(const uint16_t* a, int64_t ld_a, int64_t a_rows, const int32_t* src_row,
                     const int32_t* seg_offsets, int S, int64_t total_rows, const uint16_t* wp,
                     int K, int n_out, uint16_t* c, uint16_t* pre, hipStream_t stream) {
  const int NB = (EPI == NT_MOE_EPI_SWIGLU ? 2 * n_out : n_out) / 32;
  const int64_t n_tiles = (NB + kTB - 1) / kTB;
  const int64_t upper = ((total_rows + kBM - 1) / kBM + S) * n_tiles;
  int64_t grid = num_cus();
  if (upper < grid) grid = upper;
  grid = ((grid + 7) / 8) * 8;
  const size_t lds = pp_lds_bytes(S);
  auto kern = grouped_gemm_pp_kernel<EPI, GATHER, KEEP>;
  hipError_t err = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds);
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(kThreads), lds, stream, a, ld_a, src_row,
                     seg_offsets, S, (int)total_rows, a_rows, wp, K, n_out, c, pre);
  return hipGetLastError();
}

}  // namespace

bool pp_gemm_supported(int K, int S) {
  return K % kBK == 0 && K / kBK >= kMinSteps && pp_lds_bytes(S) <= 160 * 1024;
}

hipError_t launch_grouped_gemm_bf16_pp(const uint16_t* a, int64_t ld_a, int64_t a_rows,
                                       const int32_t* src_row, const int32_t* seg_offsets,
                                       int num_segments, int64_t total_rows, const uint16_t* wp,
                                       int K, int n_out, int epilogue, uint16_t* c, uint16_t* pre,
                                       hipStream_t stream) {
  if (total_rows == 0) return hipSuccess;
#define NT_PP(EPI, KEEP)                                                                      \
  return src_row ? launch_pp<EPI, true, KEEP>(a, ld_a, a_rows, src_row, seg_offsets,          \
                                              num_segments, total_rows, wp, K, n_out, c, pre, \
                                              stream)                                         \
                 : launch_pp<EPI, false, KEEP>(a, ld_a, a_rows, src_row, seg_offsets,         \
                                               num_segments, total_rows, wp, K, n_out, c,     \
                                               pre, stream)
  if (pre) {
    if (epilogue == NT_MOE_EPI_SWIGLU) NT_PP(NT_MOE_EPI_SWIGLU, true);
    NT_PP(NT_MOE_EPI_RELU2, true);
  }
  switch (epilogue) {
    case NT_MOE_EPI_SWIGLU: NT_PP(NT_MOE_EPI_SWIGLU, false);
    case NT_MOE_EPI_RELU2: NT_PP(NT_MOE_EPI_RELU2, false);
    default: NT_PP(NT_MOE_EPI_NONE, false);
  }
#undef NT_PP
}

}  // namespace ntmoe
