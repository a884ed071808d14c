// Grouped expert GEMM on bf16 MFMA with the expert weights pre-packed in fragment order.
//
// Same computation as grouped_gemm.hip (SequentialMLP's per-expert fc1/fc2, megatron_moe.py:145,
// over MasterLinear, :58-78, with the SwiGLU / ReLU^2 epilogue fused):
//   c[r, j] = epilogue(a_src(r) . w_s[j, :])   for every row r of segment s.
// What changes is how the two operands reach the matrix cores:
//   * token rows (A, gathered through src_row for the up projection) are shared by all waves
//     of a workgroup, so they go through LDS, in a ring of 4 stages: while one pair of K steps
//     is computed from two stages, the next pair's two are loaded (direct-to-LDS loads,
//     XOR-swizzled so fragment reads are conflict-free);
//   * expert weights are not shared between waves (each wave owns 32 or 64 of the tile's 256
//     weight rows), so they skip LDS: each wave streams its own 4 KB blocks per K step into
//     registers, one K step ahead. The weights are packed once (pack kernel below) so that the
//     16-byte fragment chunk of lane l for K slice q sits at offset (q * 64 + l) * 16 of a 4 KB
//     block: every weight load instruction reads 1 KB of consecutive bytes.
// K order. Inside a 64-wide K step, lane half h of both operands holds K elements
// [32 h + 8 q, +8) for MFMA slice q (instead of [16 q + 8 h, +8)): the same permutation on both
// operands, so each product still pairs equal K indices and the 4 slices cover the step.
// Tile: 128 tokens x 256 weight rows x 64 K, 4 waves, two workgroups per CU (the default); or
// 256 tokens x 256 rows with 8 waves, one workgroup per CU. A wave computes 8 32 x 32
// accumulators: its 64 weight rows against 128 tokens (each token fragment read from LDS
// feeds two MFMAs), or 32 rows against 256 tokens. For SwiGLU a 32-row block is 16 gate rows
// and the 16 value rows of the same output columns (packed together), so gate and value of an
// output land in the same lane (elements 4 g + r and 4 (g + 2) + r).
// Two workgroups per CU: while one waits at its barrier or in its epilogue, the other keeps
// the matrix cores busy, and LDS fragment reads are halved; the weights are then streamed once
// per 128 tokens instead of 256.
// Scheduling: persistent workgroups walk an XCD-contiguous share of the (segment, m, n) tile
// list, as the unpacked kernel does. The load pipeline runs across tile boundaries; the gather
// indices of the next tile go into an LDS table four K steps before they are needed, so the
// in-order completion of vector memory operations already guarantees them when they are read.
// The producer locates that next tile (one ballot over the segment table), and the consumer
// takes it from there.
// K steps go in pairs (g even, g + 1) with one workgroup barrier per pair: a barrier per K step
// idles the matrix cores far more than its own latency (the waves of a SIMD, released together,
// finish together and leave the pipe empty while the workgroup gathers). Waits count
// outstanding vector memory operations (loads and stores retire in order on this GPU family):
// the even step issues B(g + 1) (weights, registers), then A(g + 2) and A(g + 3) (token rows,
// LDS, each with one gather-index load); the odd step issues B(g + 2); at the end of a tile the
// epilogue's fixed number of stores follow. An odd K-step count (K = 320: 5 steps) runs one
// more odd step per tile that re-reads the last stage and weights but multiplies nothing, so
// tiles stay whole pairs at the cost of a sixth of the loads.
#include <math.h>
#include <stdlib.h>
#include <type_traits>

#include "common.h"

namespace ntmoe {
namespace {


typedef __attribute__((address_space(1))) void gvoid;
typedef __attribute__((address_space(3))) void lvoid;

constexpr int kBufferWord3 = 0x00020000;

constexpr int kBK = 64;            // K per step
constexpr int kSA = 4;             // LDS stages of token rows
constexpr int kRB = kBK * 2;       // bytes per staged token row
constexpr int kCH = kRB / 16;      // 16-byte chunks per row (8)
constexpr int kWIN = 256 / kRB;    // rows per 256-byte bank window (2)
constexpr int kRPI = 64 / kCH;     // rows per load instruction (8)
constexpr int kBlockElems = 32 * kBK;  // packed weight block (32 rows x 64 K) = 2048 bf16
constexpr int kMinK = 4 * kBK;     // the gather table needs four K steps of lead
constexpr int kTileBlocks = 8;     // packed 32-row weight blocks per N tile (256 weight rows)
constexpr int kXposeBytes = 2048;  // per-wave LDS scratch of the epilogue's output transpose

// Two workgroup shapes share the kernel. WAVES = 8: 256 tokens per tile, one weight block per
// wave, one workgroup per CU. WAVES = 4: 128 tokens per tile, two weight blocks per wave (each
// token fragment read from LDS feeds two MFMAs), two workgroups per CU, so one workgroup's
// barrier waits and epilogue run while the other's waves keep the matrix cores busy.
template <int WAVES>
struct Geo {
  static constexpr int kWaves = WAVES;
  static constexpr int kThreads = WAVES * 64;
  static constexpr int kWB = kTileBlocks / WAVES;   // weight blocks per wave
  static constexpr int kBM = WAVES * 32;            // tokens per tile
  static constexpr int kNJ = kBM / 32;              // 32-token blocks per tile
  static constexpr int kAQ = kBM / kRPI / WAVES;    // A load instructions per wave per stage (4)
  static constexpr int kStage = kBM * kRB;          // bytes per LDS stage
  static constexpr int kIdxWaves = kBM / 64;        // waves that load a tile's gather indices
  static constexpr int kPerCU = 8 / WAVES;          // workgroups per CU
  static constexpr size_t lds(int S) {  // (two 4-wave workgroups fit a CU up to 512 segments)
    return (size_t)kSA * kStage + (size_t)kWaves * kXposeBytes +
           (2 * kBM + kWaves * 64) * sizeof(int) + (size_t)(2 * S + 2) * sizeof(int);
  }
};

// Row order inside a packed 32-row block. A 32 x 32 accumulator holds, in element i of lane
// half h, block position 8 (i / 4) + 4 h + i % 4; the pack kernel puts logical row
// 8 (2 (i / 8) + h) + i % 8 there, so elements 0-7 and 8-15 of a lane are each 8 consecutive
// logical rows (one 16-byte store of bf16 outputs). Position p holds logical row
// block_row(p): the middle two 4-row groups of each 16-row half are swapped.
__host__ __device__ constexpr int block_row(int p) { return p ^ (((p >> 2) ^ (p >> 3)) & 1) * 12; }
static_assert(block_row(4) == 8 && block_row(8) == 4 && block_row(20) == 24 && block_row(3) == 3,
              "middle groups swapped");

template <int EPI>
struct Ep {
  static constexpr int kStores = EPI == NT_MOE_EPI_SWIGLU ? 1 : 2;  // 16-byte stores per lane
};                                                                   // per 32-token block

__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ ((row / kWIN) % kCH); }

// Workgroup barrier without a memory fence (a fence would wait for every outstanding load). The
// LDS reads of the previous K step are complete first (their results are already consumed), so
// the slot they read may be refilled once every wave is past the barrier.
__device__ __forceinline__ void barrier_nofence() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int N>
__device__ __forceinline__ void vm_wait() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

struct Tile {
  int s, nt, m0, seg_end;
};

// KEEP: also store the epilogue's input (the fc1 pre-activations: SwiGLU gate then value, 2 n_out
// wide, or the ReLU^2 input, n_out wide) to Pre, for a backward pass.
// EDGE: shapes with an odd K-step count or a partial last N tile (the extra step, waves that
// multiply nothing). Without it the kernel holds neither, so the common shapes' code stays small
// enough for the instruction cache (both together double it).
template <int EPI, bool GATHER, int WAVES, bool KEEP = false, bool EDGE = false>
__global__ __launch_bounds__(WAVES * 64, 2) void grouped_gemm_packed_kernel(
    const uint16_t* __restrict__ A, int64_t ld_a, const int32_t* __restrict__ src_row,
    const int32_t* __restrict__ seg_offsets, int S, int total_rows, int64_t a_rows,
    const uint16_t* __restrict__ Wp, int K, int n_out, uint16_t* __restrict__ Cout,
    uint16_t* __restrict__ Pre) {
  using Gm = Geo<WAVES>;
  constexpr int kBM = Gm::kBM, kWaves = Gm::kWaves, kAQ = Gm::kAQ, kStage = Gm::kStage;
  constexpr int kWB = Gm::kWB, kNJ = Gm::kNJ, kIdxWaves = Gm::kIdxWaves;
  constexpr int G = GATHER ? 1 : 0;
  extern __shared__ __align__(16) unsigned char smem[];
  unsigned char* xpose = smem + kSA * kStage + wave_id() * kXposeBytes;  // this wave's scratch
  int* src_tab = reinterpret_cast<int*>(smem + kSA * kStage + kWaves * kXposeBytes);  // [2][kBM]
  int* src_dummy = src_tab + 2 * kBM;                           // [kWaves][64] sink
  int* tile_prefix = src_dummy + kWaves * 64;                   // [S+1]
  int* seg_lo = tile_prefix + (S + 1);                          // [S+1]

  const int lane = lane_id(), wave = wave_id();
  const int NB = (EPI == NT_MOE_EPI_SWIGLU ? 2 * n_out : n_out) / 32;  // packed 32-row blocks
  const int n_tiles = (NB + kTileBlocks - 1) / kTileBlocks;
  const int nk = K / kBK;
  __builtin_assume(nk >= kMinK / kBK);  // the launcher guarantees it (and an even nk unless EDGE)
  if constexpr (!EDGE) __builtin_assume(nk % 2 == 0);
  // K steps per tile in the pipeline: an odd count gets one more step that loads and waits like
  // the others but multiplies nothing, so every tile keeps whole pairs.
  const int nks = EDGE ? nk + (nk & 1) : nk;
  constexpr bool kSplit = EDGE && GATHER;  // partial N tiles may be split (below)

  // Segment table and tile prefix (as in the unpacked kernel): clamped, non-decreasing.
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

  const int total = __builtin_amdgcn_readfirstlane(tile_prefix[S]);
  const int xcd = blockIdx.x % 8, local = blockIdx.x / 8, per_xcd = gridDim.x / 8;
  const int t_begin = (int)((int64_t)total * xcd / 8);
  const int t_end = (int)((int64_t)total * (xcd + 1) / 8);
  const int n_x = t_end - t_begin;
  // Round-robin over the XCD's workgroups. When the last round would leave more than half of
  // them idle, its tiles are split into two kBM/2-row halves, so twice as many workgroups share
  // it (a half still streams the tile's weights, so it costs more than half a tile: worth it
  // only when the workgroups would idle anyway). With two workgroups per CU, the first
  // dispatched (lower local index) wins instruction arbitration, so the leftover tiles, which
  // go to the lowest local indices, land on the faster ones.
  const int full_rounds = n_x / per_xcd, rem = n_x - full_rounds * per_xcd;
  const bool split_tail = rem > 0 && 2 * rem <= per_xcd;
  const int n_my = full_rounds + (local < (split_tail ? 2 * rem : rem) ? 1 : 0);
  if (n_my == 0) return;

  // Tile number tl (half: -1 whole, 0 or 1 for the lower or upper kBM/2 rows) -> segment and
  // position. The segment is the last one whose tile prefix is <= tl: one ballot per 64 segments.
  auto locate_tl = [&](int tl, int half, Tile& t) {
    int cnt = 0;
    for (int base = 0; base < S; base += 64) {
      const int i = base + lane;
      const bool le = i < S && tile_prefix[i] <= tl;
      cnt += __popcll(__ballot(le));
    }
    t.s = __builtin_amdgcn_readfirstlane(cnt - 1);
    const int lt = tl - __builtin_amdgcn_readfirstlane(tile_prefix[t.s]);
    const int mt = lt / n_tiles;
    t.nt = lt - mt * n_tiles;
    t.seg_end = __builtin_amdgcn_readfirstlane(seg_lo[t.s + 1]);
    t.m0 = __builtin_amdgcn_readfirstlane(seg_lo[t.s]) + mt * kBM;
    if (half >= 0) {  // rows [m0, m0 + kBM/2) or [m0 + kBM/2, m0 + kBM) of the tile
      const int tile_end = t.seg_end < t.m0 + kBM ? t.seg_end : t.m0 + kBM;
      if (half) t.m0 += kBM / 2;
      t.seg_end = half ? tile_end : (tile_end < t.m0 + kBM / 2 ? tile_end : t.m0 + kBM / 2);
    }
  };
  // The idx-th tile of this workgroup. In each round the two workgroups that share a CU
  // (local l and l + per_xcd / 2) take neighbouring tiles, 2 l' and 2 l' + 1 (l' = l mod
  // per_xcd / 2), and each workgroup alternates between the even and the odd one from round to
  // round, when the N tiles include a partial one: where a row tile's N tiles alternate full and
  // partial (the T3 cell's 320-wide outputs), every CU then runs one of each at a time instead
  // of two of a kind (T3 up projection 166 -> 155 us with the split partial tiles below).
  auto locate_static = [&](int idx, Tile& t) {
    if (split_tail && idx == full_rounds) {
      locate_tl(t_begin + full_rounds * per_xcd + (local >> 1), local & 1, t);
    } else {
      // (full rounds only: the last, partial round takes the first tiles of its range in order;
      // and only with partial N tiles: at config 2 the plain order measured 1.5 % faster)
      const int h = per_xcd / 2;
      const bool pair = EDGE && NB % kTileBlocks != 0 && !(per_xcd & 1) && idx < full_rounds;
      const int pos = !pair ? local
                            : (local < h ? 2 * local + (idx & 1) : 2 * (local - h) + 1 - (idx & 1));
      locate_tl(t_begin + pos + idx * per_xcd, -1, t);
    }
  };

  // Gather indices of tile t into table slot `slot`: the first kBM / 64 waves load 64 rows each,
  // straight to LDS; rows past the segment end repeat its last row (their results are dropped).
  const char* abase = reinterpret_cast<const char*>(A);
  // Byte offsets of this lane's four A chunks (one per load instruction) for tile t.
  // Instruction q covers rows (wave kAQ + q) kRPI + [0, kRPI); a row's swizzle depends only on
  // q % 2 and the lane, so two per-lane values serve every instruction.
  static_assert(2 * kRPI == kWIN * kCH, "swizzle period of two load instructions");
  const int lrow = lane / kCH, lphys = lane % kCH;
  const uint32_t aswz[2] = {(uint32_t)swz(lrow, lphys) * 16,
                            (uint32_t)swz(kRPI + lrow, lphys) * 16};
  auto a_offsets = [&](const Tile& t, int slot, uint32_t (&aoff)[kAQ]) {
#pragma unroll
    for (int q = 0; q < kAQ; ++q) {
      const int row = (wave * kAQ + q) * kRPI + lrow;
      int64_t r;
      if (GATHER) r = src_tab[slot * kBM + row];
      else r = t.m0 + row < t.seg_end ? t.m0 + row : t.seg_end - 1;
      r = r < 0 ? 0 : (r >= a_rows ? a_rows - 1 : r);
      aoff[q] = (uint32_t)(r * ld_a * 2) + aswz[q % 2];
    }
  };
  // This wave's packed weight blocks for tile t (clamped in a partial N tile): wave-uniform
  // addresses, to which each lane adds lane * 16 bytes.
  auto w_base = [&](const Tile& t, const uint16_t* (&wb)[kWB]) {
    // a split partial N tile (below): every wave streams the tile's first kWB blocks
    const int wv = kSplit && NB - t.nt * kTileBlocks <= kWB ? 0 : wave;
#pragma unroll
    for (int rb = 0; rb < kWB; ++rb) {
      int nb = t.nt * kTileBlocks + wv * kWB + rb;
      nb = nb < NB ? nb : NB - 1;
      wb[rb] = Wp + ((int64_t)t.s * NB + nb) * (int64_t)nk * kBlockElems;
    }
  };
  const uint32_t b_lane = lane * 16;
  // Weight loads are issued from inline assembly: the compiler then neither counts them nor
  // inserts its own (conservative, loop-merged) waits for their registers; the explicit wait
  // before their use names the registers, so no use can be scheduled above it. The block address
  // is a scalar operand, the lane offset the only vector one.
  auto load_blk = [&](const uint16_t* blk, u32x4 (&b)[4]) {
    asm volatile("global_load_dwordx4 %0, %1, %2" : "=v"(b[0]) : "v"(b_lane), "s"(blk) : "memory");
    asm volatile("global_load_dwordx4 %0, %1, %2 offset:1024"
                 : "=v"(b[1]) : "v"(b_lane), "s"(blk) : "memory");
    asm volatile("global_load_dwordx4 %0, %1, %2 offset:2048"
                 : "=v"(b[2]) : "v"(b_lane), "s"(blk) : "memory");
    asm volatile("global_load_dwordx4 %0, %1, %2 offset:3072"
                 : "=v"(b[3]) : "v"(b_lane), "s"(blk) : "memory");
  };
  // K step kt of this wave's blocks (kt = nks: the first step of the blocks in wn; the extra
  // step of an odd count, kt = nk < nks, re-reads the last).
  auto load_b = [&](const uint16_t* const (&wc)[kWB], const uint16_t* const (&wn)[kWB], int kt,
                    u32x4 (&b)[kWB][4]) {
#pragma unroll
    for (int rb = 0; rb < kWB; ++rb)
      load_blk(kt >= nks ? wn[rb] : wc[rb] + (int64_t)(kt < nk ? kt : nk - 1) * kBlockElems,
               b[rb]);
  };
  // Waits until at most N vector memory operations are outstanding, naming the registers of
  // the weight blocks b: no read of them can be scheduled above the wait.
  auto wait_b = [&](auto n_c, u32x4 (&b)[kWB][4]) {
    constexpr int N = decltype(n_c)::value;
    if constexpr (kWB == 1) {
      asm volatile("s_waitcnt vmcnt(%4)"
                   : "+v"(b[0][0]), "+v"(b[0][1]), "+v"(b[0][2]), "+v"(b[0][3])
                   : "n"(N)
                   : "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(%8)"
                   : "+v"(b[0][0]), "+v"(b[0][1]), "+v"(b[0][2]), "+v"(b[0][3]),
                     "+v"(b[1][0]), "+v"(b[1][1]), "+v"(b[1][2]), "+v"(b[1][3])
                   : "n"(N)
                   : "memory");
    }
  };

  // ---- producer: one A stage (+ one gather-index load) per call, two calls per pair ----------
  // Every call issues the same vector memory operations -- 4 token-row loads and, with GATHER,
  // one gather-index load -- whether or not they are needed (past the end they re-read valid

  // ---- producer: one A stage (+ one gather-index load) per call, two calls per pair ----------
  // Every call issues the same vector memory operations -- 4 token-row loads and, with GATHER,
  // one gather-index load -- whether or not they are needed (past the end they re-read valid
  // addresses into slots nobody reads), so the wait counts are the same in every pair.
  // The producer also finds the workgroup's next tile, four K steps before its first stage:
  // tile i goes to tq[i % 2] (tile_ok[i % 2] says whether it exists), which is where the
  // consumer takes it from.
  Tile pt, tq0, tq1;
  bool ok0 = true, ok1 = false;
  int p_idx = 0, p_kt = 0, p_slot = 0, produced = 0;
  int total_steps = 0x7fffffff;  // known once the producer finds there is no next tile
  uint32_t aoff[kAQ];
  const int src_lead_kt = nks - 4;  // K step of a tile at which the next tile's indices go out
  // Selects between the values (not between the two variables' addresses, which would put
  // them in scratch memory).
  auto pick = [](bool o, int x1, int x0) {
    const int a1 = __builtin_amdgcn_readfirstlane(x1), a0 = __builtin_amdgcn_readfirstlane(x0);
    return o ? a1 : a0;
  };
  auto tile_at = [&](int i) {
    Tile r;
    const bool o = i & 1;
    r.s = pick(o, tq1.s, tq0.s);
    r.nt = pick(o, tq1.nt, tq0.nt);
    r.m0 = pick(o, tq1.m0, tq0.m0);
    r.seg_end = pick(o, tq1.seg_end, tq0.seg_end);
    return r;
  };
  auto tile_ok = [&](int i) { return pick(i & 1, ok1, ok0) != 0; };

  locate_static(0, pt);
  tq0 = pt;
  if (GATHER && wave < kIdxWaves) {  // the first tile's gather indices, before anything else
    const int r = wave * 64 + lane;
    const int gr = pt.m0 + r < pt.seg_end ? pt.m0 + r : pt.seg_end - 1;
    __builtin_amdgcn_global_load_lds((gvoid*)(src_row + gr), (lvoid*)(src_tab + wave * 64), 4,
                                     0, 0);
  }
  vm_wait<0>();
  barrier_nofence();
  a_offsets(pt, 0, aoff);

  auto produce = [&]() {
    const bool live = produced < total_steps;
    if (live && p_kt == nks) {  // next tile: its gather indices went out four stages ago
      pt = tile_at(p_idx + 1);
      ++p_idx;
      p_kt = 0;
      p_slot ^= 1;
      a_offsets(pt, p_slot, aoff);
    }
    const int kt_load = live && p_kt < nk ? p_kt : nk - 1;  // the extra step re-reads the last
    unsigned char* sb = smem + (produced % kSA) * kStage;
#pragma unroll
    for (int q = 0; q < kAQ; ++q)
      __builtin_amdgcn_global_load_lds((gvoid*)(abase + kt_load * kRB + aoff[q]),
                                       (lvoid*)(sb + (wave * kAQ + q) * 1024), 16, 0, 0);
    bool real = false;
    Tile nx;
    if (live && p_kt == src_lead_kt) {  // find tile p_idx + 1
      real = p_idx + 1 < n_my;
      if (real) locate_static(p_idx + 1, nx);
      if ((p_idx + 1) & 1) {
        tq1 = nx;
        ok1 = real;
      } else {
        tq0 = nx;
        ok0 = real;
      }
      if (!real) total_steps = (p_idx + 1) * nks;
    }
    if (GATHER) {
      const bool load_idx = real && wave < kIdxWaves;
      const int r = (wave % kIdxWaves) * 64 + lane;
      const int gr = load_idx ? (nx.m0 + r < nx.seg_end ? nx.m0 + r : nx.seg_end - 1) : 0;
      int* dst = load_idx ? src_tab + (p_slot ^ 1) * kBM + wave * 64 : src_dummy + wave * 64;
      __builtin_amdgcn_global_load_lds((gvoid*)(src_row + gr), (lvoid*)dst, 4, 0, 0);
    }
    if (live) ++p_kt;
    ++produced;
  };

  // Fragment read offsets inside a stage: token row 32 j + (lane & 31), K chunk 4 h + q.
  int frag_off[4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
    frag_off[q] = (lane & 31) * kRB + (swz(lane & 31, 4 * (lane >> 5) + q) << 4);

  const __amdgpu_buffer_rsrc_t out_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      Cout, 0, (int)((int64_t)total_rows * n_out * 2), kBufferWord3);
  constexpr int kPreW = EPI == NT_MOE_EPI_SWIGLU ? 2 : 1;  // pre-activation width / n_out
  __amdgpu_buffer_rsrc_t pre_rsrc = out_rsrc;
  if constexpr (KEEP)
    pre_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        Pre, 0, (int)((int64_t)total_rows * kPreW * n_out * 2), kBufferWord3);

  // ---- consumer ---------------------------------------------------------------------------
  Tile ct = pt;
  const uint16_t* wb[kWB];
  w_base(ct, wb);
  u32x4 b0[kWB][4], b1[kWB][4];
  // Prologue: A(0), A(1), B(0), all landed before the first pair's barrier.
  produce();
  asm volatile("" ::: "memory");
  produce();
  asm volatile("" ::: "memory");
  load_b(wb, wb, 0, b0);
  wait_b(std::integral_constant<int, 0>(), b0);

  int g = 0;   // global K step of this workgroup
  int ti = 0;  // this workgroup's tile number
  for (;;) {
    const int live_m = ct.seg_end - ct.m0;  // token rows of this tile that exist (uniform)
    // A split partial N tile (EDGE with the gather; without it the kernel's registers are at the
    // limit and the split spills): when the tile's blocks fit one wave's kWB, every wave takes
    // those blocks with one 32-token block of its own (wave w: rows 32 w .. 32 w + 31) instead of
    // one wave taking them with all kNJ token blocks while the others idle (the T3 cell's 320-wide
    // outputs: the second N tile of each row tile holds 2 of 8 blocks).
    const bool split = kSplit && NB - ct.nt * kTileBlocks <= kWB;
    const int jb = split ? wave : 0;    // the wave's first token block
    const int wv = split ? 0 : wave;    // the wave whose weight blocks this wave takes
    const uint16_t* wb_next[kWB];
#pragma unroll
    for (int rb = 0; rb < kWB; ++rb) wb_next[rb] = wb[rb];
    floatx16 acc[kWB][kNJ];
#pragma unroll
    for (int rb = 0; rb < kWB; ++rb)
#pragma unroll
      for (int j = 0; j < kNJ; ++j) acc[rb][j] = floatx16{};

    // K steps go in pairs (g even, g + 1) with one workgroup barrier per pair. The even step
    // issues B(g + 1) and both token-row stages of the next pair, A(g + 2) and A(g + 3) (each
    // with its index load), into the two slots the previous pair read; the odd step issues
    // B(g + 2). Each step computes with B(g) and ends by waiting for the weights of the next
    // step, which names their registers so no copy of them can happen before they are valid;
    // the odd step's wait (vmcnt 0) also lands this wave's part of the next pair's stages,
    // which the next barrier then publishes to every wave.
    auto step = [&](auto nj_c, auto odd_c, int kt, u32x4 (&bc)[kWB][4], u32x4 (&bn)[kWB][4])
                    __attribute__((always_inline)) {  // (an outlined step spills in-flight loads)
      constexpr int NJ = decltype(nj_c)::value;  // 32-token blocks that hold segment rows (0:
                                                 // loads and waits only, no products)
      constexpr bool ODD = decltype(odd_c)::value;
      constexpr int NM = 4 * NJ;                 // token fragments per step (kWB MFMAs each)
      constexpr int PF = NM < 4 ? NM : 4;        // fragment reads kept in flight
      constexpr int NJd = NJ > 0 ? NJ : 1;        // (divisor; no fragment exists when NJ = 0)
      constexpr int PFd = PF > 0 ? PF : 1;
      if (!ODD) {
        // Two workgroups share each CU (b and b + gridDim.x / 2) and the one dispatched first
        // would win instruction arbitration throughout, leaving its partner to finish alone.
        // Instead the two take turns at the higher wave priority, switching every 2^11 ticks
        // (about 20 us) of the 100 MHz real-time counter, so both progress alike. The counter is
        // read before the barrier, in the same statement as the wait for it, so its latency
        // overlaps the barrier wait (the barrier's own wait for the LDS reads is the same one).
        if (kWaves == 4) {
          uint64_t now;
          asm volatile("s_memrealtime %0\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier"
                       : "=s"(now)::"memory");
          const bool high = (((now >> 11) & 1) != 0) != (blockIdx.x >= gridDim.x / 2);
          if (high) __builtin_amdgcn_s_setprio(1);
          else __builtin_amdgcn_s_setprio(0);
        } else {
          barrier_nofence();
        }
      }
      // The first PF token fragments go out first, so their latency overlaps the issue of this
      // step's loads instead of idling the matrix core.
      // (a split tile's wave reads its own token block jb)
      const unsigned char* st = smem + (g % kSA) * kStage + jb * 32 * kRB;
      // NM token fragments (slice q = n / NJ, token block j = n % NJ), read PF ahead.
      auto frag = [&](int n) {
        return *reinterpret_cast<const bf16x8*>(st + (n % NJd) * 32 * kRB + frag_off[n / NJd]);
      };
      bf16x8 fr[PF > 0 ? PF : 1];
#pragma unroll
      for (int n = 0; n < PF; ++n) fr[n] = frag(n);
      asm volatile("" ::: "memory");
      if (kt + 1 == nks && tile_ok(ti + 1)) w_base(tile_at(ti + 1), wb_next);
      // The step's vector memory operations -- B(g + 1) as kWB x 4 loads of 1 KB, then on even
      // steps the two token-row stages (produce) -- go out spread between the MFMA groups, in
      // that order: issued together ahead of the MFMAs they filled the wave's memory queue and
      // held back its first products (config 2 up projection 139 -> 132 us, down 85 -> 78 us).
      // EDGE: the two stages follow the last group; EDGE without the gather, whose registers
      // are at the limit, keeps the loads ahead of the MFMAs.
      constexpr bool kSpread = GATHER || !EDGE;
      if constexpr (kSpread) {
        const uint16_t* bsrc[kWB];
#pragma unroll
        for (int rb = 0; rb < kWB; ++rb)  // past the last tile: re-reads of its first step
          bsrc[rb] = kt + 1 >= nks
                         ? wb_next[rb]
                         : wb[rb] + (int64_t)(kt + 1 < nk ? kt + 1 : nk - 1) * kBlockElems;
        constexpr int kItems = kWB * 4 + (ODD || EDGE ? 0 : 2);
        auto item = [&](auto i_c) __attribute__((always_inline)) {
          constexpr int i = decltype(i_c)::value;
          if constexpr (i < kWB * 4) {
            asm volatile("global_load_dwordx4 %0, %1, %2 offset:%3"
                         : "=v"(bn[i / 4][i % 4])
                         : "v"(b_lane), "s"(bsrc[i / 4]), "n"((i % 4) * 1024)
                         : "memory");
          } else {
            produce();
            asm volatile("" ::: "memory");
          }
        };
        if constexpr (NM == 0) static_for<0, kItems>(item);
        static_for<0, NM>([&](auto n_c) __attribute__((always_inline)) {
          constexpr int n = decltype(n_c)::value;
#pragma unroll
          for (int rb = 0; rb < kWB; ++rb)
            acc[rb][n % NJd] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                __builtin_bit_cast(bf16x8, bc[rb][n / NJd]), fr[n % PFd], acc[rb][n % NJd], 0,
                0, 0);
          if constexpr (n + PF < NM) fr[n % PFd] = frag(n + PF);
          // this group's share of the memory operations, after its MFMAs and fragment read:
          // the weight loads over the first half of the groups, the stages at 1/2 and 3/4
          __builtin_amdgcn_sched_barrier(0);
          static_for<0, kItems>([&](auto i_c) __attribute__((always_inline)) {
            constexpr int i = decltype(i_c)::value;
            constexpr int at = i < kWB * 4 ? i * (NM / 2) / (kWB * 4) : NM / 2 + (i - kWB * 4) * (NM / 4);
            if constexpr (at == n) item(i_c);
          });
          __builtin_amdgcn_sched_barrier(0);
        });
        if constexpr (EDGE && !ODD) {
          produce();
          asm volatile("" ::: "memory");
          produce();
          asm volatile("" ::: "memory");
        }
      } else {
        load_b(wb, wb_next, kt + 1, bn);  // past the last tile: re-reads of its first step
        asm volatile("" ::: "memory");
        if (!ODD) {
          produce();
          asm volatile("" ::: "memory");
          produce();
          asm volatile("" ::: "memory");
        }
#pragma unroll
        for (int n = 0; n < NM; ++n) {
#pragma unroll
          for (int rb = 0; rb < kWB; ++rb)
            acc[rb][n % NJd] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                __builtin_bit_cast(bf16x8, bc[rb][n / NJd]), fr[n % PFd], acc[rb][n % NJd], 0,
                0, 0);
          if (n + PF < NM) fr[n % PFd] = frag(n + PF);
        }
        // Keep PF fragment reads in flight: (kWB MFMAs, 1 read) groups, then the last PF
        // groups' MFMAs. Without this the scheduler pulls each read next to its MFMA and waits
        // on it.
#pragma unroll
        for (int n = 0; n < NM - PF; ++n) {
          __builtin_amdgcn_sched_group_barrier(0x008, kWB, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        if constexpr (PF > 0) __builtin_amdgcn_sched_group_barrier(0x008, kWB * PF, 0);
      }
      // Even step: the two stages and index loads issued after B(g + 1) may stay in flight.
      wait_b(std::integral_constant<int, ODD ? 0 : 2 * (kAQ + G)>(), bn);
      ++g;
    };
    auto k_loop = [&](auto nj_c) __attribute__((always_inline)) {
      for (int kt = 0; kt < nk; kt += 2) {
        step(nj_c, std::false_type(), kt, b0, b1);
        // The extra step of an odd count multiplies nothing. No register load is in flight at
        // this branch (the even step waited for its weights) or after it (both sides end with
        // vmcnt(0)).
        if (!EDGE || kt + 1 < nk) step(nj_c, std::true_type(), kt + 1, b1, b0);
        else step(std::integral_constant<int, 0>(), std::true_type(), kt + 1, b1, b0);
      }
    };
    // A partial tile (the last of a segment) multiplies only the 32-token blocks that hold
    // rows; in a partial N tile a wave whose weight blocks all lie past the last one multiplies
    // nothing (its SIMD's matrix core goes to the other workgroup's wave). The loads are the
    // same in every variant.
    const bool wave_live = !EDGE || split || ct.nt * kTileBlocks + wave * kWB < NB;
    // (a split tile's wave multiplies one token block, or none past the segment's rows)
    const bool mul_none = EDGE && (!wave_live || (split && live_m <= 32 * wave));
    const bool mul_one = kSplit && split;
    if (mul_none) k_loop(std::integral_constant<int, 0>());
    else if (!mul_one && live_m > kBM / 2) k_loop(std::integral_constant<int, kNJ>());
    else if (!mul_one && live_m > kBM / 4) k_loop(std::integral_constant<int, kNJ / 2>());
    else if (!mul_one && kNJ >= 8 && live_m > kBM / 8)
      k_loop(std::integral_constant<int, kNJ / 4 ? kNJ / 4 : 1>());
    else k_loop(std::integral_constant<int, 1>());

    // Epilogue. Lane (token j, half h) holds logical block rows 8 h + [0, 8) in elements 0-7 and
    // 16 + 8 h + [0, 8) in 8-15: for SwiGLU gate and value of output columns 16 nb + 8 h + [0, 8),
    // otherwise columns 32 nb + 8 h + [0, 8) and 32 nb + 16 + 8 h + [0, 8). Stored straight from
    // that layout, one instruction would write 32 B of each of 32 rows; instead each wave
    // transposes its outputs through its LDS scratch (row-major, 16-byte chunks XOR-swizzled by
    // row so writes and reads are conflict-free), 16 rows (or 32 for SwiGLU) at a time, and every
    // store instruction writes whole 128-byte (SwiGLU: 64-byte) row segments of the wave's
    // columns. The store count per wave is fixed (none from a wave past the last block: no later
    // wait counts stores, as they are older than every load a wait names); rows past the segment
    // or columns past n_out get an out-of-range offset and are dropped by the buffer range check.
    const int hbit = lane >> 5;
    if (wave_live) {
      constexpr bool SW = EPI == NT_MOE_EPI_SWIGLU;
      constexpr int CPR = kWB * (SW ? 2 : 4);  // 16-byte chunks per row of the wave's columns
      constexpr int RPH = kXposeBytes / (CPR * 16) < 32 ? kXposeBytes / (CPR * 16) : 32;  // rows
      constexpr int RPS = 64 / CPR;            // per pass through the scratch; per store
      static_assert(RPH * CPR * 16 <= kXposeBytes && 32 % RPH == 0 && RPH % RPS == 0, "passes");
      // chunk c of row r: the 8 rows that share a 128-byte LDS line pattern get distinct chunks
      auto xoff = [](int r, int c) { return r * CPR * 16 + ((c ^ ((r / (8 / CPR)) % CPR)) << 4); };
      const int col0 = (ct.nt * kTileBlocks + wv * kWB) * (SW ? 16 : 32);
      const int t = lane & 31;
#pragma unroll
      for (int j = 0; j < kNJ; ++j) {
        // block j's outputs packed first (and its pre-activations stored), so its accumulators
        // are free before the transpose
        u32x4 pk[kWB][Ep<EPI>::kStores];
        const int m_lane = ct.m0 + (jb + j) * 32 + t;
        // a split tile's wave holds one token block: its other blocks store nothing
        const bool j_ok = !(kSplit && split) || j == 0;
#pragma unroll
        for (int rb = 0; rb < kWB; ++rb)
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
              const int nb = ct.nt * kTileBlocks + wv * kWB + rb;
              const int col = SW ? nb * 16 + 8 * hbit : nb * 32 + 16 * st + 8 * hbit;
              const bool ok = j_ok && m_lane < ct.seg_end && nb < NB && col < n_out;
              const int64_t prow = (int64_t)m_lane * kPreW * n_out;
#pragma unroll
              for (int h = 0; h < (SW ? 2 : 1); ++h) {
                const int e0 = SW ? 8 * h : 8 * st;
                const u32x4 pv = {pack_bf16x2(acc[rb][j][e0], acc[rb][j][e0 + 1]),
                                  pack_bf16x2(acc[rb][j][e0 + 2], acc[rb][j][e0 + 3]),
                                  pack_bf16x2(acc[rb][j][e0 + 4], acc[rb][j][e0 + 5]),
                                  pack_bf16x2(acc[rb][j][e0 + 6], acc[rb][j][e0 + 7])};
                const uint32_t poff =
                    ok ? (uint32_t)((prow + h * n_out + col) * 2) : 0x80000000u;
                __builtin_amdgcn_raw_buffer_store_b128(pv, pre_rsrc, poff, 0, 0);
              }
            }
          }
#pragma unroll
        for (int pass = 0; pass < 32 / RPH; ++pass) {
          if (t / RPH == pass) {
#pragma unroll
            for (int rb = 0; rb < kWB; ++rb)
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
            const int m = ct.m0 + (jb + j) * 32 + pass * RPH + r;
            const int col = col0 + q * 8;
            const uint32_t voff = (j_ok && m < ct.seg_end && col < n_out)
                                      ? (uint32_t)(((int64_t)m * n_out + col) * 2)
                                      : 0x80000000u;
            __builtin_amdgcn_raw_buffer_store_b128(val, out_rsrc, voff, 0, 0);
          }
          asm volatile("" ::: "memory");
        }
      }
    }
    if (!tile_ok(ti + 1)) break;
    ++ti;
    ct = tile_at(ti);
#pragma unroll
    for (int rb = 0; rb < kWB; ++rb) wb[rb] = wb_next[rb];
  }
  vm_wait<0>();  // the trailing re-reads land in LDS before the workgroup's LDS is released
}

// Packs w [S, R, K] (bf16) into 32-row x 64-K blocks of fragment order: block (s, nb, kb) holds,
// at 16-byte chunk q * 64 + l, logical row i = block_row(l % 32) of the block and K elements
// kb * 64 + 32 (l / 32) + 8 q .. + 8. Logical row i of block nb is w row 32 nb + i, or for
// SwiGLU (R = 2 n_out) gate row 16 nb + i (i < 16) and value row n_out + 16 nb + i - 16.
__global__ __launch_bounds__(256) void pack_weights_kernel(const uint16_t* __restrict__ w,
                                                            int64_t chunks, int R, int K,
                                                            int n_out, int swiglu,
                                                            uint16_t* __restrict__ out) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= chunks) return;
  const int KB = K / kBK, NB = R / 32;
  const int l = (int)(c % 64), q = (int)((c / 64) % 4);
  const int kb = (int)((c / 256) % KB);
  const int64_t rest = c / (256 * (int64_t)KB);
  const int nb = (int)(rest % NB);
  const int64_t s = rest / NB;
  const int i = block_row(l % 32);
  const int row = swiglu ? (i < 16 ? 16 * nb + i : n_out + 16 * nb + (i - 16)) : 32 * nb + i;
  const int k0 = kb * kBK + 32 * (l / 32) + 8 * q;
  *reinterpret_cast<u32x4*>(out + c * 8) =
      *reinterpret_cast<const u32x4*>(w + (s * R + row) * (int64_t)K + k0);
}

template <int EPI, bool GATHER, int WAVES, bool KEEP = false, bool EDGE = false>
hipError_t launch_packed(const uint16_t* a, int64_t ld_a, int64_t a_rows, const int32_t* src_row,
                         const int32_t* seg_offsets, int S, int64_t total_rows,
                         const uint16_t* wp, int K, int n_out, uint16_t* c, hipStream_t stream,
                         uint16_t* pre = nullptr) {
  using Gm = Geo<WAVES>;
  const int NB = (EPI == NT_MOE_EPI_SWIGLU ? 2 * n_out : n_out) / 32;
  const int64_t n_tiles = (NB + kTileBlocks - 1) / kTileBlocks;
  const int64_t upper = ((total_rows + Gm::kBM - 1) / Gm::kBM + S) * n_tiles;
  int64_t grid = (int64_t)num_cus() * Gm::kPerCU;
  if (upper < grid) grid = upper;
  grid = ((grid + 7) / 8) * 8;
  const size_t lds = Gm::lds(S);
  auto kern = grouped_gemm_packed_kernel<EPI, GATHER, WAVES, KEEP, EDGE>;
  hipError_t err = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds);
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(Gm::kThreads), lds, stream, a, ld_a,
                     src_row, seg_offsets, S, (int)total_rows, a_rows, wp, K, n_out, c, pre);
  return hipGetLastError();
}

// Whether the ping-pong kernel serves the packed entry points (NT_MOE_GEMM_PP=1).
bool use_pp() {
  static const bool v = [] {
    const char* s = getenv("NT_MOE_GEMM_PP");
    return s && atoi(s) == 1;
  }();
  return v;
}

// Workgroup shape of the packed kernel: 4 (two workgroups per CU) unless NT_MOE_PACKED_WAVES=8.
int packed_waves() {
  static const int w = [] {
    const char* s = getenv("NT_MOE_PACKED_WAVES");
    return s && atoi(s) == 8 ? 8 : 4;
  }();
  return w;
}

}  // namespace

int packed_gemm_min_k() { return kMinK; }

hipError_t launch_pack_weights_bf16(const uint16_t* w, int64_t S, int R, int K, int epilogue,
                                    uint16_t* packed, hipStream_t stream) {
  const int n_out = epilogue == NT_MOE_EPI_SWIGLU ? R / 2 : R;
  const int64_t chunks = S * (int64_t)R * K / 8;
  if (chunks == 0) return hipSuccess;
  pack_weights_kernel<<<dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, stream>>>(
      w, chunks, R, K, n_out, epilogue == NT_MOE_EPI_SWIGLU ? 1 : 0, packed);
  return hipGetLastError();
}

// Whether a shape needs the EDGE kernel: an odd count of 64-wide K steps, or a last N tile with
// fewer than 8 packed blocks.
static bool packed_edge(int K, int n_out, int epilogue) {
  const int NB = (epilogue == NT_MOE_EPI_SWIGLU ? 2 * n_out : n_out) / 32;
  return (K / kBK) % 2 != 0 || NB % kTileBlocks != 0;
}

hipError_t launch_grouped_gemm_bf16_packed(const uint16_t* a, int64_t ld_a, int64_t a_rows,
                                           const int32_t* src_row, const int32_t* seg_offsets,
                                           int num_segments, int64_t total_rows,
                                           const uint16_t* wp, int K, int n_out, int epilogue,
                                           uint16_t* c, hipStream_t stream) {
  if (total_rows == 0) return hipSuccess;
  if (use_pp() && pp_gemm_supported(K, num_segments))
    return launch_grouped_gemm_bf16_pp(a, ld_a, a_rows, src_row, seg_offsets, num_segments,
                                       total_rows, wp, K, n_out, epilogue, c, nullptr, stream);
  const bool edge = packed_edge(K, n_out, epilogue);
#define NT_PW(EPI, W, EDGE)                                                                   \
  return src_row ? launch_packed<EPI, true, W, false, EDGE>(a, ld_a, a_rows, src_row,         \
                                                            seg_offsets, num_segments,        \
                                                            total_rows, wp, K, n_out, c,      \
                                                            stream)                           \
                 : launch_packed<EPI, false, W, false, EDGE>(a, ld_a, a_rows, src_row,        \
                                                             seg_offsets, num_segments,       \
                                                             total_rows, wp, K, n_out, c,     \
                                                             stream)
#define NT_P(EPI)                        \
  if (edge) {                            \
    NT_PW(EPI, 4, true);                 \
  } else if (packed_waves() == 8) {      \
    NT_PW(EPI, 8, false);                \
  } else {                               \
    NT_PW(EPI, 4, false);                \
  }
  switch (epilogue) {
    case NT_MOE_EPI_SWIGLU: NT_P(NT_MOE_EPI_SWIGLU);
    case NT_MOE_EPI_RELU2: NT_P(NT_MOE_EPI_RELU2);
    default: NT_P(NT_MOE_EPI_NONE);
  }
#undef NT_P
#undef NT_PW
}

hipError_t launch_grouped_gemm_bf16_packed_keep(const uint16_t* a, int64_t ld_a, int64_t a_rows,
                                                const int32_t* src_row,
                                                const int32_t* seg_offsets, int num_segments,
                                                int64_t total_rows, const uint16_t* wp, int K,
                                                int n_out, int epilogue, uint16_t* c,
                                                uint16_t* pre, hipStream_t stream) {
  if (total_rows == 0) return hipSuccess;
  if (use_pp() && pp_gemm_supported(K, num_segments))
    return launch_grouped_gemm_bf16_pp(a, ld_a, a_rows, src_row, seg_offsets, num_segments,
                                       total_rows, wp, K, n_out, epilogue, c, pre, stream);
  const bool edge = packed_edge(K, n_out, epilogue);
#define NT_PKE(EPI, EDGE)                                                                    \
  return src_row ? launch_packed<EPI, true, 4, true, EDGE>(a, ld_a, a_rows, src_row,         \
                                                           seg_offsets, num_segments,        \
                                                           total_rows, wp, K, n_out, c,      \
                                                           stream, pre)                      \
                 : launch_packed<EPI, false, 4, true, EDGE>(a, ld_a, a_rows, src_row,        \
                                                            seg_offsets, num_segments,       \
                                                            total_rows, wp, K, n_out, c,     \
                                                            stream, pre)
#define NT_PK(EPI)        \
  if (edge) {             \
    NT_PKE(EPI, true);    \
  } else {                \
    NT_PKE(EPI, false);   \
  }
  if (epilogue == NT_MOE_EPI_SWIGLU) {
    NT_PK(NT_MOE_EPI_SWIGLU);
  }
  NT_PK(NT_MOE_EPI_RELU2);
#undef NT_PK
#undef NT_PKE
}

}  // namespace ntmoe
