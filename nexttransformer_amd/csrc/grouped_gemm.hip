// Grouped expert GEMM on bf16 MFMA (gfx950 v_mfma_f32_32x32x16_bf16), fp32 accumulation.
//
// Replaces SequentialMLP's per-expert loop (nexttransformer/scaling/megatron_moe.py:145) over
// MasterLinear fc1 -> activation -> fc2 (megatron_moe.py:58-78, :23-24; lm.py:29-35).
// One launch computes, for every ragged segment s (expert) with rows
// [seg_offsets[s], seg_offsets[s+1]):
//   c[r, j] = epilogue(a_src(r) . w_s[j, :])
// up   : a = x gathered through src_row (the permutation is fused into the tile loads),
//        epilogue SwiGLU (w_s rows [0,H) gate, [H,2H) value) or ReLU^2
// down : a = h, plain epilogue.
//
// Scheduling. Persistent: each workgroup reads seg_offsets, builds the tile prefix in LDS and
// walks a static share of the tile list (segment-major, then m, then n). The list is cut into
// 8 contiguous ranges, one per XCD (workgroup b runs on XCD b % 8), so the tiles of one
// expert -- which share its weights -- stay in one L2.
//
// Tile. BM x BN macro tile, BK-deep stages, WM x WN waves (default 256 x 256 x 64 with 2 x 4
// waves: a 128 x 64 sub-tile per wave). Global -> LDS movement uses gfx950's direct-to-LDS loads
// (global_load_lds_dwordx4): lane i of a load instruction lands in the i-th 16-byte slot of a
// 1 KB LDS block, so the row gather and the bank swizzle are both expressed by which global
// chunk each lane fetches.
//
// LDS banks. gfx950 serves a ds_read_b128 16 lanes at a time from 64 four-byte banks (256 B).
// A fragment read has 16 lanes on 16 consecutive rows at one logical chunk c; a row of RB bytes
// sits in bank window (r * RB) mod 256, so rows r and r + 256/RB share a window. Storing chunk c
// of row r in slot c ^ ((r / (256/RB)) % CH) (CH = chunks per row) spreads the 16 lanes over 16
// distinct slots: conflict free.
//
// Pipeline. The STAGES LDS stages form one ring across all tiles of a workgroup: the loads of
// a tile's first stages are issued before the previous tile's epilogue, and the gather indices
// of the next tile are fetched during the last K step, so tile changes do not drain the
// pipeline. Waits count outstanding vector-memory operations (on gfx9-class hardware they
// retire in issue order, loads and stores alike); barriers carry no memory fence. The epilogue
// uses range-checked buffer stores: every wave issues the same number of stores (rows and
// columns outside the tile's segment are sent out of range and dropped), so a wait can count
// past them.
//
// The MFMA takes the weight fragment as its "A" operand and the activation fragment as "B",
// so a lane's accumulators are runs of 4 consecutive output columns of one row (8-byte packed
// bf16 stores). For SwiGLU the BN weight rows of a tile are laid out per wave as
// [gate half | value half] of the same hidden columns, so gate and value of an output element
// sit in the same lane.
#include <math.h>
#include <stdlib.h>

#include <type_traits>

#include "common.h"

namespace ntmoe {
namespace {

enum Epilogue { kEpiSwiglu = NT_MOE_EPI_SWIGLU, kEpiRelu2 = NT_MOE_EPI_RELU2, kEpiPlain = NT_MOE_EPI_NONE };

typedef __attribute__((address_space(1))) void gvoid;
typedef __attribute__((address_space(3))) void lvoid;

// Buffer resource word 3 for raw (untyped) buffer access on gfx9-class GPUs.
constexpr int kBufferWord3 = 0x00020000;

template <int BM_, int BN_, int BK_, int STAGES_, int WM_, int WN_, int EPI_>
struct Cfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, STAGES = STAGES_, WM = WM_, WN = WN_;
  static constexpr int EPI = EPI_;
  static constexpr int kWaves = WM * WN, kThreads = kWaves * 64;
  static constexpr int kWaveM = BM / WM, kWaveN = BN / WN;
  static constexpr int TM = kWaveM / 32, TN = kWaveN / 32;
  static constexpr int CH = BK / 8;             // 16-byte chunks per tile row
  static constexpr int RB = BK * 2;             // bytes per tile row
  static constexpr int RPI = 64 / CH;           // tile rows per load instruction
  static constexpr int WIN = 256 / RB;          // rows sharing one 256-byte bank window
  static constexpr int kAQ = BM / RPI / kWaves;  // A load instructions per wave per stage
  static constexpr int kBQ = BN / RPI / kWaves;
  static constexpr int kQ = kAQ + kBQ;
  static constexpr int kStage = (BM + BN) * RB;  // bytes
  // Workgroups resident per CU: two when both fit in LDS (stages + segment tables <= 80 KB).
  static constexpr int kPerCU = STAGES * kStage + 4096 <= 80 * 1024 ? 2 : 1;
  static constexpr int kBNOut = EPI == kEpiSwiglu ? BN / 2 : BN;  // output columns per tile
  static constexpr int kOutTN = EPI == kEpiSwiglu ? TN / 2 : TN;
  static constexpr int kStores = TM * kOutTN * 4;  // buffer stores per wave per tile
  static_assert(kAQ * kWaves * RPI == BM && kBQ * kWaves * RPI == BN, "load tiling");
  static_assert(EPI != kEpiSwiglu || TN % 2 == 0, "SwiGLU needs gate and value tiles per wave");
  static_assert(BK == 32 || BK == 64, "BK");
  // Stores can be counted past only while the wait immediate (6 bits) covers them.
  static constexpr bool kCountStores = (STAGES - 2) * kQ + kStores <= 63;
  static_assert((STAGES - 2) * kQ <= 63, "vmcnt range");
};

__device__ __forceinline__ int swizzle_slot(int row, int chunk, int win, int ch) {
  return chunk ^ ((row / win) % ch);
}

// Waits until at most `ahead` stages of loads (kQ each) plus, when `stores`, one epilogue's
// buffer stores remain outstanding: everything older -- the stage being consumed -- is done.
template <class C>
__device__ __forceinline__ void wait_stage(int ahead, bool stores) {
  constexpr int Q = C::kQ, M = C::kCountStores ? C::kStores : 0;
  if (stores && !C::kCountStores) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  } else if (stores) {
    if (ahead <= 0) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(M) : "memory");
    else if (ahead == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(Q + M) : "memory");
    else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * Q + M) : "memory");
  } else {
    if (ahead <= 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    else if (ahead == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(Q) : "memory");
    else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * Q) : "memory");
  }
}

// Workgroup barrier without a memory fence (a fence would wait for every outstanding load).
__device__ __forceinline__ void barrier_nofence() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// One tile of the workgroup's list and the per-lane load offsets that stream it.
template <class C>
struct TileWork {
  int s, nt, m0, seg_end;
  const char* wseg;
  uint32_t aoff[C::kAQ], boff[C::kBQ];
};

template <class C>
__device__ __forceinline__ void issue_stage(unsigned char* smem, int slot, int kt, const char* abase,
                                            const TileWork<C>& w, int wave) {
  unsigned char* sb = smem + slot * C::kStage;
  const char* ak = abase + kt * C::RB;
  const char* bk = w.wseg + kt * C::RB;
#pragma unroll
  for (int q = 0; q < C::kAQ; ++q)
    __builtin_amdgcn_global_load_lds((gvoid*)(ak + w.aoff[q]),
                                     (lvoid*)(sb + (wave * C::kAQ + q) * 1024), 16, 0, 0);
#pragma unroll
  for (int q = 0; q < C::kBQ; ++q)
    __builtin_amdgcn_global_load_lds((gvoid*)(bk + w.boff[q]),
                                     (lvoid*)(sb + C::BM * C::RB + (wave * C::kBQ + q) * 1024),
                                     16, 0, 0);
}

template <class C>
__device__ __forceinline__ void load_frags(const unsigned char* st, int wm, int wn, int off,
                                           bf16x8* fa, bf16x8* fb) {
#pragma unroll
  for (int j = 0; j < C::TM; ++j)
    fa[j] = *reinterpret_cast<const bf16x8*>(st + (wm * C::kWaveM + j * 32) * C::RB + off);
#pragma unroll
  for (int i = 0; i < C::TN; ++i)
    fb[i] = *reinterpret_cast<const bf16x8*>(st + (C::BM + wn * C::kWaveN + i * 32) * C::RB + off);
}

// MFMAs of one staged K step; fragments double buffered so the LDS reads of sub-step ks + 1 are
// in flight during the MFMAs of ks. CHECK skips 32-row sub-tiles at or past live_m rows.
template <class C, bool CHECK>
__device__ __forceinline__ void compute_stage(const unsigned char* st, int wm, int wn,
                                              const int* frag_off, int live_m,
                                              floatx16 (&acc)[C::TN][C::TM]) {
  constexpr int KS = C::BK / 16;
  bf16x8 fa[2][C::TM], fb[2][C::TN];
  load_frags<C>(st, wm, wn, frag_off[0], fa[0], fb[0]);
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    if (ks + 1 < KS) load_frags<C>(st, wm, wn, frag_off[ks + 1], fa[(ks + 1) & 1], fb[(ks + 1) & 1]);
#pragma unroll
    for (int j = 0; j < C::TM; ++j) {
      if (!CHECK || j * 32 < live_m) {
#pragma unroll
        for (int i = 0; i < C::TN; ++i)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[ks & 1][i], fa[ks & 1][j],
                                                              acc[i][j], 0, 0, 0);
      }
    }
  }
}

template <class C, bool GATHER>
__global__ __launch_bounds__(C::kThreads, C::kPerCU) void grouped_gemm_kernel(
    const uint16_t* __restrict__ A, int64_t ld_a, const int32_t* __restrict__ src_row,
    const int32_t* __restrict__ seg_offsets, int S, int total_rows, int64_t a_rows,
    const uint16_t* __restrict__ W, int64_t w_seg_stride, int64_t ld_w, int K, int n_out,
    uint16_t* __restrict__ Cout) {
  extern __shared__ __align__(16) unsigned char smem[];
  int* tile_prefix = reinterpret_cast<int*>(smem + C::STAGES * C::kStage);  // [S+1]
  int* seg_lo = tile_prefix + (S + 1);                                      // [S+1]

  const int lane = lane_id(), wave = wave_id();
  const int wm = wave / C::WN, wn = wave % C::WN;
  const int n_tiles = (n_out + C::kBNOut - 1) / C::kBNOut;
  // Segment bounds clamped to [0, total_rows] and made non-decreasing (a running max), so
  // malformed offsets can only give wrong rows, never out-of-bounds accesses. All threads load
  // the offsets in parallel; wave 0 turns them into the tile prefix with shuffle scans.
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
      for (int w = 1; w < 64; w <<= 1) {  // inclusive running max
        int u = __shfl_up(o, w);
        if (lane >= w) o = o > u ? o : u;
      }
      o = o > run_max ? o : run_max;
      int prev = __shfl_up(o, 1);
      if (lane == 0) prev = run_max;
      int t = i >= 1 && i <= S ? ((o - prev + C::BM - 1) / C::BM) * n_tiles : 0;
      for (int w = 1; w < 64; w <<= 1) {  // inclusive sum
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
  // Each XCD owns a contiguous range of the tile list (workgroup b runs on XCD b % 8); its
  // workgroups take the range's tiles round robin.
  const int total = __builtin_amdgcn_readfirstlane(tile_prefix[S]);
  const int xcd = blockIdx.x % 8, local = blockIdx.x / 8, per_xcd = gridDim.x / 8;
  const int t_begin = (int)((int64_t)total * xcd / 8);
  const int t_end = (int)((int64_t)total * (xcd + 1) / 8);
  const int nk = K / C::BK;
  int tile = t_begin + local;
  if (tile >= t_end) return;

  // Loader: in instruction q lane i fills slot (row = inst*RPI + i/CH, phys = i%CH) with
  // logical chunk phys ^ ((row / WIN) % CH) of that row.
  const int lrow = lane / C::CH, lphys = lane % C::CH;
  // Fragment reads: row base + (lane & 31) (base a multiple of 32), chunk 2 ks + (lane >> 5).
  int frag_off[C::BK / 16];
#pragma unroll
  for (int ks = 0; ks < C::BK / 16; ++ks)
    frag_off[ks] = (lane & 31) * C::RB +
                   (swizzle_slot(lane & 31, 2 * ks + (lane >> 5), C::WIN, C::CH) << 4);
  const char* abase = reinterpret_cast<const char*>(A);
  const __amdgpu_buffer_rsrc_t out_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      Cout, 0, (int)((int64_t)total_rows * n_out * 2), kBufferWord3);

  // Tile metadata (wave-uniform) and the gather indices of its A rows (one per load q).
  auto locate = [&](int t, TileWork<C>& w, int* src) {
    int lo = 0, hi = S;
    while (hi - lo > 1) {
      int mid = (lo + hi) >> 1;
      if (tile_prefix[mid] <= t) lo = mid; else hi = mid;
    }
    w.s = __builtin_amdgcn_readfirstlane(lo);
    const int ltile = t - __builtin_amdgcn_readfirstlane(tile_prefix[w.s]);
    const int mt = ltile / n_tiles;
    w.nt = ltile - mt * n_tiles;
    w.seg_end = __builtin_amdgcn_readfirstlane(seg_lo[w.s + 1]);
    w.m0 = __builtin_amdgcn_readfirstlane(seg_lo[w.s]) + mt * C::BM;
    w.wseg = reinterpret_cast<const char*>(W + (int64_t)w.s * w_seg_stride);
#pragma unroll
    for (int q = 0; q < C::kAQ; ++q) {
      const int row = (wave * C::kAQ + q) * C::RPI + lrow;
      const int gr = w.m0 + row < w.seg_end ? w.m0 + row : w.seg_end - 1;
      src[q] = GATHER ? src_row[gr] : gr;
    }
  };
  auto offsets = [&](TileWork<C>& w, const int* src) {
#pragma unroll
    for (int q = 0; q < C::kAQ; ++q) {
      const int row = (wave * C::kAQ + q) * C::RPI + lrow;
      const int chunk = swizzle_slot(row, lphys, C::WIN, C::CH);
      int64_t r = src[q] < 0 ? 0 : (src[q] >= a_rows ? a_rows - 1 : (int64_t)src[q]);
      w.aoff[q] = (uint32_t)(r * ld_a * 2) + chunk * 16;
    }
#pragma unroll
    for (int q = 0; q < C::kBQ; ++q) {
      const int row = (wave * C::kBQ + q) * C::RPI + lrow;
      const int chunk = swizzle_slot(row, lphys, C::WIN, C::CH);
      int wrow;
      if (C::EPI == kEpiSwiglu) {
        int slot = row / C::kWaveN, qq = row % C::kWaveN, half = C::kWaveN / 2;
        int hcol = w.nt * C::kBNOut + slot * half + (qq % half);
        hcol = hcol < n_out ? hcol : n_out - 1;  // partial N tile: clamp, results dropped
        wrow = qq < half ? hcol : n_out + hcol;
      } else {
        wrow = w.nt * C::BN + row;
        wrow = wrow < n_out ? wrow : n_out - 1;
      }
      w.boff[q] = (uint32_t)(wrow * ld_w * 2) + chunk * 16;
    }
  };

  TileWork<C> cur;
  int src[C::kAQ];
  locate(tile, cur, src);
  offsets(cur, src);
  int ring = 0;  // stage slot of the current tile's K step 0
#pragma unroll
  for (int p = 0; p < C::STAGES - 1; ++p)
    if (p < nk) issue_stage<C>(smem, (ring + p) % C::STAGES, p, abase, cur, wave);
  bool stores_pending = false;

  while (true) {
    const int next = tile + per_xcd;
    const bool has_next = next < t_end;
    floatx16 acc[C::TN][C::TM];
#pragma unroll
    for (int i = 0; i < C::TN; ++i)
#pragma unroll
      for (int j = 0; j < C::TM; ++j) acc[i][j] = floatx16{};
    // 32-row sub-tiles of this wave that hold segment rows (wave-uniform).
    const int live_m = cur.seg_end - (cur.m0 + wm * C::kWaveM);
    // The epilogue's view of this tile: `cur` is overwritten with the next tile during the
    // last K step.
    int ep_m0 = cur.m0, ep_seg_end = cur.seg_end, ep_nt = cur.nt;
    // One K loop per sub-tile policy, chosen once per tile (a branch inside the loop would make
    // the compiler keep two copies of the accumulators).
    auto k_loop = [&](auto check) {
      constexpr bool CHECK = decltype(check)::value;
      for (int kt = 0; kt < nk; ++kt) {
        const int ahead = (nk - 1 - kt) < (C::STAGES - 2) ? (nk - 1 - kt) : (C::STAGES - 2);
        wait_stage<C>(ahead, stores_pending && kt <= C::STAGES - 2);
        barrier_nofence();
        if (kt + C::STAGES - 1 < nk)
          issue_stage<C>(smem, (ring + kt + C::STAGES - 1) % C::STAGES, kt + C::STAGES - 1,
                         abase, cur, wave);
        if (kt == nk - 1 && has_next) {  // next tile's metadata; its gather indices in flight
          ep_m0 = cur.m0;
          ep_seg_end = cur.seg_end;
          ep_nt = cur.nt;
          locate(next, cur, src);
        }
        compute_stage<C, CHECK>(smem + ((ring + kt) % C::STAGES) * C::kStage, wm, wn, frag_off,
                                live_m, acc);
      }
    };
    if (live_m >= C::kWaveM)
      k_loop(std::integral_constant<bool, false>());
    else
      k_loop(std::integral_constant<bool, true>());
    // Next tile's first stages go out before this tile's epilogue. Their slots held K steps
    // nk - STAGES .. nk - 2 of this tile, which every wave finished before the last barrier.
    if (has_next) {
      offsets(cur, src);
      const int nring = (ring + nk) % C::STAGES;
#pragma unroll
      for (int p = 0; p < C::STAGES - 1; ++p)
        if (p < nk) issue_stage<C>(smem, (nring + p) % C::STAGES, p, abase, cur, wave);
    }

    // Epilogue: lane holds row m = ... + (lane & 31) and columns 8 (e/4) + 4 (lane/32) + e%4.
    // Exactly kStores buffer stores per wave; out-of-tile rows/columns get an out-of-range
    // offset and are dropped by the buffer range check.
    const int col_base = C::EPI == kEpiSwiglu ? ep_nt * C::kBNOut + wn * (C::kWaveN / 2)
                                              : ep_nt * C::BN + wn * C::kWaveN;
#pragma unroll
    for (int j = 0; j < C::TM; ++j) {
      const int m = ep_m0 + wm * C::kWaveM + j * 32 + (lane & 31);
      const bool row_ok = m < ep_seg_end;
#pragma unroll
      for (int i = 0; i < C::kOutTN; ++i) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = col_base + i * 32 + g * 8 + (lane >> 5) * 4;
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float a = acc[i][j][g * 4 + e];
            if (C::EPI == kEpiSwiglu) {
              float u = acc[i + C::kOutTN][j][g * 4 + e];
              // silu(a) * u with the hardware reciprocal (1 ulp): the result is rounded to bf16.
              v[e] = a * u * __builtin_amdgcn_rcpf(1.f + __expf(-a));
            } else if (C::EPI == kEpiRelu2) {
              float r = a > 0.f ? a : 0.f;
              v[e] = r * r;
            } else {
              v[e] = a;
            }
          }
          uint2 packed;
          packed.x = pack_bf16x2(v[0], v[1]);
          packed.y = pack_bf16x2(v[2], v[3]);
          const uint32_t voff =
              (row_ok && n < n_out) ? (uint32_t)(((int64_t)m * n_out + n) * 2) : 0x80000000u;
          __builtin_amdgcn_raw_buffer_store_b64(u32x2{packed.x, packed.y}, out_rsrc, voff, 0, 0);
        }
      }
    }
    if (!has_next) break;
    tile = next;
    ring = (ring + nk) % C::STAGES;
    stores_pending = true;
  }
}

template <class C, bool GATHER>
hipError_t launch_gemm(const uint16_t* A, int64_t ld_a, int64_t a_rows, const int32_t* src_row,
                       const int32_t* seg_offsets, int S, int64_t total_rows, const uint16_t* W,
                       int64_t w_seg_stride, int64_t ld_w, int K, int n_out, uint16_t* Cout,
                       int* counters, hipStream_t stream) {
  if (K % C::BK) return hipErrorInvalidValue;
  const int64_t n_tiles = (n_out + C::kBNOut - 1) / C::kBNOut;
  const int64_t upper = ((total_rows + C::BM - 1) / C::BM + S) * n_tiles;
  int64_t grid = (int64_t)num_cus() * C::kPerCU;
  if (upper < grid) grid = upper;
  grid = ((grid + 7) / 8) * 8;
  size_t lds = (size_t)C::STAGES * C::kStage + (size_t)(2 * S + 2) * sizeof(int);
  auto kern = grouped_gemm_kernel<C, GATHER>;
  hipError_t err = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds);
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(C::kThreads), lds, stream, A, ld_a,
                     src_row, seg_offsets, S, (int)total_rows, a_rows, W, w_seg_stride, ld_w, K,
                     n_out, Cout);
  return hipGetLastError();
}

// Tile shapes, selected by NT_MOE_GEMM_VARIANT (for tuning runs); index 0 is the default.
//   0: 256x256, BK 64, 2 stages, 2x4 waves (wave tile 128x64)
//   1: 256x256, BK 64, 2 stages, 2x2 waves (wave tile 128x128)
//   2: 256x256, BK 32, 3 stages, 2x4 waves
//   3: 256x256, BK 32, 4 stages, 2x4 waves
//   4: 256x128, BK 32, 3 stages, 2x2 waves, two workgroups per CU
int gemm_variant() {
  static int v = [] {
    const char* s = getenv("NT_MOE_GEMM_VARIANT");
    int x = s ? atoi(s) : 0;
    return (x >= 0 && x <= 4) ? x : 0;
  }();
  return v;
}

template <int EPI, bool GATHER>
hipError_t launch_variant(int variant, const uint16_t* a, int64_t ld_a, int64_t a_rows,
                          const int32_t* src_row, const int32_t* seg_offsets, int S,
                          int64_t total_rows, const uint16_t* w, int64_t stride, int64_t ld_w,
                          int K, int n_out, uint16_t* c, int* counters, hipStream_t stream) {
#define NT_V(BM, BN, BK, ST, WM, WN)                                                     \
  launch_gemm<Cfg<BM, BN, BK, ST, WM, WN, EPI>, GATHER>(a, ld_a, a_rows, src_row,        \
                                                        seg_offsets, S, total_rows, w,   \
                                                        stride, ld_w, K, n_out, c,       \
                                                        counters, stream)
  switch (variant) {
    case 1: return NT_V(256, 256, 64, 2, 2, 2);
    case 2: return NT_V(256, 256, 32, 3, 2, 4);
    case 3: return NT_V(256, 256, 32, 4, 2, 4);
    case 4: return NT_V(256, 128, 32, 3, 2, 2);
    default: return NT_V(256, 256, 64, 2, 2, 4);
  }
#undef NT_V
}

}  // namespace

hipError_t launch_grouped_gemm_bf16(const uint16_t* a, int64_t ld_a, int64_t a_rows,
                                    const int32_t* src_row, const int32_t* seg_offsets,
                                    int num_segments, int64_t total_rows, const uint16_t* w,
                                    int K, int n_out, int epilogue, uint16_t* c, int* counters,
                                    hipStream_t stream) {
  const int64_t rows_per_seg = epilogue == NT_MOE_EPI_SWIGLU ? 2 * n_out : n_out;
  const int64_t ld_w = K;
  const int64_t stride = rows_per_seg * ld_w;
  const int v = gemm_variant();
#define NT_GEMM(EPI, GATHER)                                                                   \
  launch_variant<EPI, GATHER>(v, a, ld_a, a_rows, src_row, seg_offsets, num_segments,          \
                              total_rows, w, stride, ld_w, K, n_out, c, counters, stream)
  switch (epilogue) {
    case NT_MOE_EPI_SWIGLU: return src_row ? NT_GEMM(kEpiSwiglu, true) : NT_GEMM(kEpiSwiglu, false);
    case NT_MOE_EPI_RELU2: return src_row ? NT_GEMM(kEpiRelu2, true) : NT_GEMM(kEpiRelu2, false);
    default: return src_row ? NT_GEMM(kEpiPlain, true) : NT_GEMM(kEpiPlain, false);
  }
#undef NT_GEMM
}

hipError_t launch_grouped_ffn_bf16(const uint16_t* a, int64_t ld_a, int64_t a_rows,
                                   const int32_t* src_row, const int32_t* seg_offsets,
                                   int num_segments, int64_t total_rows, const uint16_t* w1,
                                   const uint16_t* w2, int d, int H, int activation, uint16_t* h,
                                   uint16_t* y, int* counters, hipStream_t stream) {
  const int epi = activation == NT_MOE_ACT_SWIGLU ? NT_MOE_EPI_SWIGLU : NT_MOE_EPI_RELU2;
  hipError_t err = launch_grouped_gemm_bf16(a, ld_a, a_rows, src_row, seg_offsets, num_segments,
                                            total_rows, w1, d, H, epi, h, counters, stream);
  if (err != hipSuccess) return err;
  return launch_grouped_gemm_bf16(h, H, total_rows, nullptr, seg_offsets, num_segments,
                                  total_rows, w2, H, d, NT_MOE_EPI_NONE, y, counters, stream);
}

}  // namespace ntmoe
