// Router: fp32 gating GEMM in a fixed reduction order, softmax / sigmoid scoring and
// a wavefront-shuffle top-k, with per-block auxiliary-loss partials.
//
// Replaces NativeRouter.gating -> F.linear(x.float(), W.float())
// (nexttransformer/scaling/megatron_moe.py:95-99) and TopKRouter's top-k followed by softmax
// over the selected logits (megatron_moe.py:43; reference_blocks.py:37-38).
//
// Fixed order (bit-exact contract shared with oracle/router_ref.c):
//   c_j   = fma chain over features [128 j, 128 j + 128) in ascending order, from 0.0f
//   logit = ((c_0 + c_1) + c_2) + ...   then  + bias[e]
// Ties in top-k: equal logits rank the lower expert index first.
//
// Work mapping. The chains run on the matrix cores: v_mfma_f32_32x32x2_f32 computes, for a
// 32 x 32 output block, acc = fma(a1, b1, fma(a0, b0, acc)) -- two steps of the same sequential
// fp32 fma chain (features 2n, then 2n + 1), bit for bit -- so 64 of them in ascending feature
// order are exactly c_j for 32 tokens x 32 experts. Lane l supplies token/expert l % 32 and
// feature parity l / 32. A block owns 64 tokens; one wave per (32-token half, 32-expert block,
// feature range). x comes straight from global memory (16 bytes = 8 features per lane, the
// lane's parity picked out with one byte permute), router weights from w_router_t [d, E] (for a
// feature pair, the two lane halves read two 128-byte rows); both are prefetched half a chunk
// ahead. With one expert block the features are split over two waves per output block: the
// first keeps the running sum of its chunks, the second its chunk sums, added to that running
// sum in chunk order after a barrier.
// For small T (too few waves for the chip) the split variant gives every (token block, chunk,
// expert block) its own waves and writes the chunk sums c_j to a workspace (token-major planes);
// a plane-sum kernel adds them in ascending j -- the same order -- and a top-k kernel ranks.
// For 129-256 experts the streamed kernel (below) keeps one workgroup per 64 tokens for all
// experts: token rows staged once in LDS, router weights loaded by each wave into registers.
//
// Top-k: logits go to an LDS tile [64][E+1]; LPT lanes share a token (4 in the fused kernel,
// 16 in the top-k kernel), each scans every LPT-th expert into a sorted register list, then k
// rounds of an xor-shuffle butterfly over the LPT lanes emit the global order.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "common.h"

namespace ntmoe {
namespace {

typedef __attribute__((address_space(1))) void gvoid;
typedef __attribute__((address_space(3))) void lvoid;

constexpr int kBufferWord3 = 0x00020000;

__host__ __device__ inline int lg_tile_bytes(int E) { return kRouteBlock * (E + 1) * 4; }
__host__ __device__ inline int zt_offset(int E) { return (lg_tile_bytes(E) + 15) & ~15; }
// After the logits tile: zt (64 floats), then the block's per-expert assignment masks (E
// 64-bit words, bit tt set when token tt of the block chose the expert).
__host__ __device__ inline int cnt_offset(int E) { return zt_offset(E) + kRouteBlock * 4; }
__host__ __device__ inline size_t router_lds_bytes(int E) { return cnt_offset(E) + (size_t)E * 8; }

// LDS stages of the fused kernel: for each feature range, 64 features of x (64 tokens, rows
// padded to kXPitch bf16) and of the router weights for all expert blocks, stored so that a
// lane's 4 weights for MFMAs 4q .. 4q + 3 (features 8q + 2j + h, expert e) are one 16-byte
// word: float index ((q * 2 + h) * Ew + e) * 4 + j, Ew = 32 EB. Lane (t, h) reads x[t][8q ..
// 8q + 8) and those weights with one ds_read_b128 each; both reads are conflict-free.
constexpr int kStageF = 64;                       // features per stage
constexpr int kXPitch = kStageF + 8;              // bf16 per staged x row
constexpr int kXStageBytes = kRouteBlock * kXPitch * 2;
__host__ __device__ inline int w_stage_bytes(int EB) { return kStageF * 32 * EB * 4; }
__host__ __device__ inline int range_stage_bytes(int EB) { return kXStageBytes + w_stage_bytes(EB); }

// Element i of a lane's 32 x 32 accumulator is token row 8 (i / 4) + 4 (lane / 32) + i % 4 and
// expert column lane % 32 of the block.
__device__ __forceinline__ int acc_row(int i, int lane) { return 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3); }

template <int KMAX>
__device__ __forceinline__ void list_insert(float v, int e, float* lv, int* li) {
  // Branch-free: the new entry moves down the list, each slot keeps the better of it and the
  // carried entry.
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    const bool c = rank_before(v, e, lv[j], li[j]);
    const float tv = lv[j];
    const int ti = li[j];
    lv[j] = c ? v : tv;
    li[j] = c ? e : ti;
    v = c ? tv : v;
    e = c ? ti : e;
  }
}

// Top-k, weights, full scores and aux partials for the 64 tokens whose logits sit in the
// LDS tile lg[64][E+1]; overwrites lg with the full scores s_te. Called by all 64 * LPT threads
// of the block: LPT lanes per token, each scanning every LPT-th expert.
template <int KMAX, int LPT = 4>
__device__ __forceinline__ void topk_and_scores(float* lg, float* zt, int64_t t0, int64_t T, int E, int k,
                                int score_fn, int32_t* __restrict__ topk_ids,
                                float* __restrict__ topk_w, float* __restrict__ prob_partial,
                                float* __restrict__ z_partial, int32_t* __restrict__ block_counts) {
  static_assert(LPT == 1 || LPT == 2 || LPT == 4 || LPT == 8 || LPT == 16, "lanes per token");
  // The block's assignments per expert, for the route plan: a 64-bit mask per expert (bit tt
  // for token tt; LDS ORs, so the result does not depend on their order) gives the counts
  // (popcount) and each assignment's rank among the block's tokens that chose its expert
  // (popcount of the lower bits) -- block_counts[blk][e] and, after the table,
  // ranks[t k + j] (route_ranks_offset).
  unsigned long long* msk =
      reinterpret_cast<unsigned long long*>(reinterpret_cast<unsigned char*>(zt) + kRouteBlock * 4);
  if (block_counts)
    for (int e = threadIdx.x; e < E; e += blockDim.x) msk[e] = 0ull;
  const int ldl = E + 1;
  const int tt = threadIdx.x / LPT;   // token within the block
  const int sub = threadIdx.x % LPT;  // which of the LPT expert strides this lane scans
  const int64_t t = t0 + tt;
  float* row = lg + tt * ldl;

  float lv[KMAX];
  int li[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) { lv[j] = -INFINITY; li[j] = 0x7fffffff; }
  if (LPT >= k && E >= 16 * LPT && E <= 64 * LPT) {
    // (Worth it from 16 logits per lane on: 256 experts over 8 lanes, 137 -> 132 us for the
    // streamed router at T = 16384; with 4 or 8 per lane it gained nothing.)
    // The LPT lane maxima are LPT distinct logits of the token, so with LPT >= k its k-th largest
    // logit is at least the smallest of them, tau: a logit below tau is in no top k, and each lane
    // inserts only its logits >= tau (in the same ascending order). The lists then hold each
    // lane's best candidates, which contain every logit the merge below picks, so the selection
    // is the one the full insertion gives (NaNs, which the insertion never takes, fail >= too).
    float lmax = -INFINITY;
    for (int e = sub; e < E; e += LPT) lmax = fmaxf(lmax, row[e]);
    float tau = lmax;
#pragma unroll
    for (int m = 1; m < LPT; m <<= 1) tau = fminf(tau, __shfl_xor(tau, m));
    unsigned long long cand = 0ull;
    for (int e = sub, i = 0; e < E; e += LPT, ++i)
      if (row[e] >= tau) cand |= 1ull << i;
    while (cand) {
      const int e = sub + LPT * __builtin_ctzll(cand);
      cand &= cand - 1ull;
      list_insert<KMAX>(row[e], e, lv, li);
    }
  } else {
    for (int e = sub; e < E; e += LPT) list_insert<KMAX>(row[e], e, lv, li);
  }

  // k rounds: best head of the LPT lists (xor butterfly), the owner pops it.
  float ov[KMAX];
  int oi[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    float bv = lv[0];
    int bi = li[0];
#pragma unroll
    for (int m = 1; m < LPT; m <<= 1) {
      float v2 = __shfl_xor(bv, m);
      int i2 = __shfl_xor(bi, m);
      if (rank_before(v2, i2, bv, bi)) { bv = v2; bi = i2; }
    }
    ov[j] = bv;
    oi[j] = bi;
    if (li[0] == bi) {
#pragma unroll
      for (int q = 0; q < KMAX - 1; ++q) { lv[q] = lv[q + 1]; li[q] = li[q + 1]; }
      lv[KMAX - 1] = -INFINITY;
      li[KMAX - 1] = 0x7fffffff;
    }
  }

  // Routing weights over the k selected: softmax, or sigmoid normalised over the selected.
  const float top = ov[0];
  float wsum = 0.f, wv[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    float s = score_fn == NT_MOE_SCORE_SOFTMAX ? expf(ov[j] - top) : 1.f / (1.f + expf(-ov[j]));
    wv[j] = j < k ? s : 0.f;
    wsum += wv[j];
  }
  const float winv = 1.f / wsum;
  if (t < T) {
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      if (j < k && j % LPT == sub) {
        topk_ids[t * k + j] = oi[j];
        topk_w[t * k + j] = wv[j] * winv;
      }
    }
  }

  // Full scores s_te for the load-balance loss, logsumexp for the z-loss.
  // The first pass leaves expf(l - top) (softmax) or 1 + expf(-l) (sigmoid) in row, so the
  // second only scales.
  float part = 0.f, spart = 0.f;
  for (int e = sub; e < E; e += LPT) {
    const float l = row[e];
    const float ex = expf(l - top);
    part += ex;
    if (score_fn == NT_MOE_SCORE_SIGMOID) {
      const float den = 1.f + expf(-l);
      spart += 1.f / den;
      row[e] = den;
    } else {
      row[e] = ex;
    }
  }
#pragma unroll
  for (int m = 1; m < LPT; m <<= 1) {
    part += __shfl_xor(part, m);
    spart += __shfl_xor(spart, m);
  }
  const float lse = top + logf(part);
  if (score_fn == NT_MOE_SCORE_SOFTMAX) {
    const float inv = 1.f / part;
    for (int e = sub; e < E; e += LPT) row[e] = row[e] * inv;
  } else {
    const float inv = 1.f / spart;
    for (int e = sub; e < E; e += LPT) row[e] = inv / row[e];
  }
  if (sub == 0) zt[tt] = lse * lse;
  __syncthreads();
  if (block_counts && t < T) {
#pragma unroll
    for (int j = 0; j < KMAX; ++j)
      if (j < k && j % LPT == sub) atomicOr(&msk[oi[j]], 1ull << tt);
  }

  // Per-block column sums in a fixed order (deterministic): P consecutive lanes per expert,
  // lane p summing tokens p, p + P, ..., then a butterfly over the P lanes; P is the largest
  // power of two <= 64 with E P <= the block's threads. The z sum likewise over one wave.
  const int nvalid = (int)((T - t0) < kRouteBlock ? (T - t0) : kRouteBlock);
  const int64_t blk = t0 / kRouteBlock;
  int P = 64;
  while (P > 1 && E * P > (int)blockDim.x) P >>= 1;
  for (int base = 0; base < E * P; base += blockDim.x) {
    const int idx = base + threadIdx.x;
    const int e = idx / P, p = idx % P;
    float s = 0.f;
    if (e < E)
      for (int r = p; r < nvalid; r += P) s += lg[r * ldl + e];
    for (int m = P >> 1; m >= 1; m >>= 1) s += __shfl_xor(s, m);
    if (e < E && p == 0) prob_partial[blk * E + e] = s;
  }
  if (threadIdx.x < 64) {
    float s = threadIdx.x < nvalid ? zt[threadIdx.x] : 0.f;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, m);
    if (threadIdx.x == 0) z_partial[blk] = s;
  }
  if (block_counts) {
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x) block_counts[blk * E + e] = __popcll(msk[e]);
    if (t < T) {
      int32_t* ranks = block_counts + route_ranks_offset(T, E);
      const unsigned long long below = (1ull << tt) - 1ull;
#pragma unroll
      for (int j = 0; j < KMAX; ++j)
        if (j < k && j % LPT == sub) ranks[t * k + j] = __popcll(msk[oi[j]] & below);
    }
  }
}

__device__ __forceinline__ void write_logits_out(const float* lg, int64_t t0, int64_t T, int E,
                                                 float* __restrict__ logits) {
  for (int idx = threadIdx.x; idx < kRouteBlock * E; idx += blockDim.x) {
    int r = idx / E, e = idx - r * E;
    if (t0 + r < T) logits[(t0 + r) * E + e] = lg[r * (E + 1) + e];
  }
}

// One workgroup's chunk sums on the matrix cores: tokens [t0, t0 + 64), experts
// [e0, e0 + 32 EBW), chunks [c_lo, c_hi) split into R ranges of whole chunks. Wave = (range r,
// 32-token half sub, expert block ebl), 128 EBW R threads. Every step stages 64 features of each
// range (x and router weights, double-buffered in smem: router_stage_bytes) and runs 32 MFMAs
// per wave from LDS. Range 0 keeps the running sum of its chunk sums, ranges r > 0 their chunk
// sums (at most 4); then, in range order, each adds its chunk sums to the running sum left in
// xch (LDS, row pitch xp floats, block (sub, ebl) at rows 32 sub, columns 32 ebl). Returns the
// complete sum ((c_lo + c_lo+1) + ...) to the waves of range R - 1 (others: partial values),
// every element also left in xch, which may alias the stage buffers (smem): it is touched only
// after the last step's barrier.
template <int EBW, int R>
struct RouterBlock {
  static constexpr int NT = 128 * EBW * R;
  static constexpr int Ew = 32 * EBW;
  static constexpr int XP = 4 / EBW;  // x pieces (16 bytes) per thread per step: 512 R / NT
  static constexpr int WP = 16;       // weights per thread per step: 64 Ew R / NT
  static constexpr int kRS = kXStageBytes + 64 * Ew * 4;  // one range's stage
  static constexpr int PMAX = 4;
  static_assert(XP >= 1 && XP * NT == 512 * R && WP * NT == 64 * Ew * R, "stage split");
  static constexpr size_t stage_bytes() { return (size_t)2 * R * kRS; }

  __device__ __forceinline__ static floatx16 run(const uint16_t* __restrict__ x, int64_t ld_x,
                                 const float* __restrict__ wt, int64_t T, int d, int E,
                                 int64_t t0, int e0, int c_lo, int c_hi, unsigned char* smem,
                                 float* xch, int xp) {
    const int lane = lane_id(), wave = wave_id(), h = lane >> 5;
    const int r = wave % R, ob = wave / R, sub = ob & 1, ebl = ob >> 1;
    const int nch = c_hi - c_lo;
    auto F = [&](int rr) { return (c_lo + rr * nch / R) * kRouterChunk; };
    auto FE = [&](int rr) {
      const int e = (c_lo + (rr + 1) * nch / R) * kRouterChunk;
      return e < d ? e : d;
    };
    // Every wave steps through the stages of the longest range (the split rounds down, so the
    // ranges differ by up to one chunk and the longest is not always range 0); a shorter
    // range's surplus stages hold no groups and their chains are dropped.
    int n_stages = 0;
#pragma unroll
    for (int rr = 0; rr < R; ++rr) {
      const int s = (FE(rr) - F(rr) + kStageF - 1) / kStageF;
      n_stages = s > n_stages ? s : n_stages;
    }
    struct Regs {
      u32x4 x[XP];
      float w[WP];
    };
    // Stage st (clamped to the last stage: a load past the end re-reads it, unused) -> regs.
    auto load_stage = [&](int st, Regs& g) {
      st = st < n_stages ? st : n_stages - 1;
#pragma unroll
      for (int i = 0; i < XP; ++i) {
        const int p = i * NT + threadIdx.x;  // [range][row][col]
        const int rr = p / 512, row = (p / 8) % 64, col = p % 8;
        const int64_t t = t0 + row < T ? t0 + row : T - 1;
        int f = F(rr) + st * kStageF + 8 * col;
        f = f < FE(rr) ? f : FE(rr) - 8;
        g.x[i] = *reinterpret_cast<const u32x4*>(x + t * ld_x + f);
      }
#pragma unroll
      for (int i = 0; i < WP; ++i) {
        const int p = i * NT + threadIdx.x;  // [range][feature][expert]
        const int rr = p / (64 * Ew), rem = p % (64 * Ew);
        int f = F(rr) + st * kStageF + rem / Ew;
        f = f < FE(rr) ? f : FE(rr) - 1;
        const int e = e0 + rem % Ew < E ? e0 + rem % Ew : E - 1;
        g.w[i] = wt[(int64_t)f * E + e];
      }
    };
    auto store_stage = [&](int buf, const Regs& g) {
#pragma unroll
      for (int i = 0; i < XP; ++i) {
        const int p = i * NT + threadIdx.x;
        const int rr = p / 512, row = (p / 8) % 64, col = p % 8;
        *reinterpret_cast<u32x4*>(smem + (buf * R + rr) * kRS + (row * kXPitch + col * 8) * 2) =
            g.x[i];
      }
#pragma unroll
      for (int i = 0; i < WP; ++i) {
        const int p = i * NT + threadIdx.x;
        const int rr = p / (64 * Ew), rem = p % (64 * Ew), f = rem / Ew, e = rem % Ew;
        float* ws = reinterpret_cast<float*>(smem + (buf * R + rr) * kRS + kXStageBytes);
        ws[(((f >> 3) * 2 + (f & 1)) * Ew + e) * 4 + ((f & 7) >> 1)] = g.w[i];
      }
    };
    const uint32_t sel = h ? 0x07060C0Cu : 0x05040C0Cu;
    auto compute = [&](int buf, int nq, floatx16 chain) {
      const unsigned char* base = smem + (buf * R + r) * kRS;
      const unsigned char* xs = base + ((sub * 32 + (lane & 31)) * kXPitch) * 2;
      const float* ws =
          reinterpret_cast<const float*>(base + kXStageBytes) + (ebl * 32 + (lane & 31)) * 4;
      auto group = [&](int q, floatx16 c) {
        const u32x4 xv = *reinterpret_cast<const u32x4*>(xs + q * 16);
        const floatx4 wv = *reinterpret_cast<const floatx4*>(ws + (q * 2 + h) * Ew * 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float a = __builtin_bit_cast(float, __builtin_amdgcn_perm(xv[j], 0u, sel));
          c = __builtin_amdgcn_mfma_f32_32x32x2f32(a, wv[j], c, 0, 0, 0);
        }
        return c;
      };
      if (nq == 8) {
#pragma unroll
        for (int q = 0; q < 8; ++q) chain = group(q, chain);
      } else {
        for (int q = 0; q < nq; ++q) chain = group(q, chain);
      }
      return chain;
    };
    auto groups_at = [&](int st) {  // real 8-feature groups of this wave's range in stage st
      const int left = FE(r) - (F(r) + st * kStageF);
      return left <= 0 ? 0 : (left >= kStageF ? 8 : left / 8);
    };

    // Two stages of loads in flight: stage st + 1 lands while stage st is computed, stage st + 2
    // is issued meanwhile. One loop iteration is one chunk (stages 2 i, 2 i + 1).
    floatx16 sum = {};
    floatx16 part[PMAX];
    Regs ga, gb;
    load_stage(0, ga);
    load_stage(1, gb);
    store_stage(0, ga);
    __syncthreads();
    auto chunk = [&](int i) {  // stages 2 i (buffer 0) and 2 i + 1 (buffer 1)
      const int st = 2 * i;
      load_stage(st + 2, ga);
      floatx16 chain = compute(0, groups_at(st), floatx16{});
      store_stage(1, gb);  // stage st + 1 (a re-read of stage st past the end: unused)
      __syncthreads();
      load_stage(st + 3, gb);
      chain = compute(1, groups_at(st + 1), chain);
      store_stage(0, ga);  // stage st + 2
      __syncthreads();
      return chain;
    };
    const int n_iter = (n_stages + 1) / 2;
    if (R == 1) {
      for (int i = 0; i < n_iter; ++i) {
        const floatx16 chain = chunk(i);
        sum = i == 0 ? chain : sum + chain;
      }
    } else {
#pragma unroll
      for (int i = 0; i < PMAX; ++i) {
        if (i < n_iter) {
          const floatx16 chain = chunk(i);
          if (groups_at(2 * i) > 0) {  // this range has chunk i
            if (r == 0) sum = i == 0 ? chain : sum + chain;
            else part[i] = chain;
          }
        }
      }
    }
    // In range order: range 0 leaves its running sum in xch, range r adds its chunk sums.
    float* xb = xch + (sub * 32) * xp + ebl * 32 + (lane & 31);
    const int r_chunks = (FE(r) - F(r) + kRouterChunk - 1) / kRouterChunk;
#pragma unroll
    for (int step_r = 0; step_r < R; ++step_r) {
      if (r == step_r) {
        if (step_r > 0) {
#pragma unroll
          for (int i = 0; i < 16; ++i) sum[i] = xb[acc_row(i, lane) * xp];
#pragma unroll
          for (int p = 0; p < PMAX; ++p)
            if (p < r_chunks) sum = sum + part[p];
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) xb[acc_row(i, lane) * xp] = sum[i];
      }
      __syncthreads();
    }
    return sum;
  }
};

// Fused (no workspace): 64 tokens x all E experts per block, 2 EB R waves; the logits (+ bias) go
// to the LDS tile lg[64][E+1], then top-k in the same block, 2 EB R lanes per token.
template <int EB, int R, int KMAX>
__global__ __launch_bounds__(128 * EB * R) void router_mfma_kernel(
    const uint16_t* __restrict__ x, int64_t ld_x, const float* __restrict__ wt,
    const float* __restrict__ bias, int64_t T, int d, int E, int k, int score_fn,
    float* __restrict__ logits, int32_t* __restrict__ topk_ids, float* __restrict__ topk_w,
    float* __restrict__ prob_partial, float* __restrict__ z_partial,
    int32_t* __restrict__ block_counts) {
  using RB = RouterBlock<EB, R>;
  extern __shared__ __align__(16) unsigned char smem[];
  float* lg = reinterpret_cast<float*>(smem + RB::stage_bytes());
  float* zt = reinterpret_cast<float*>(smem + RB::stage_bytes() + zt_offset(E));
  const int64_t t0 = (int64_t)blockIdx.x * kRouteBlock;
  const int nchunk = (d + kRouterChunk - 1) / kRouterChunk;
  constexpr int xp = 32 * EB + 1;
  const float* xch = reinterpret_cast<const float*>(smem);  // [64][32 EB + 1] over the stages
  RB::run(x, ld_x, wt, T, d, E, t0, 0, 0, nchunk, smem, reinterpret_cast<float*>(smem), xp);
  for (int idx = threadIdx.x; idx < kRouteBlock * E; idx += blockDim.x) {
    const int row = idx / E, e = idx - row * E;
    float v = xch[row * xp + e];
    if (bias) v = v + bias[e];
    lg[row * (E + 1) + e] = v;
  }
  __syncthreads();
  if (logits) write_logits_out(lg, t0, T, E, logits);
  topk_and_scores<KMAX, 2 * EB * R>(lg, zt, t0, T, E, k, score_fn, topk_ids, topk_w,
                                    prob_partial, z_partial, block_counts);
}

inline size_t router_mfma_lds_bytes(int EB, int R, int E) {
  return (size_t)2 * R * (kXStageBytes + 64 * 32 * EB * 4) + router_lds_bytes(E);
}

// Logits: one 64-token block x one 32-expert block (blockIdx.y) per workgroup, 2 R waves; the
// complete logits (+ bias) go to out[t][e] (token-major), for the top-k kernel.
template <int R>
__global__ __launch_bounds__(128 * R) void router_logits_kernel(
    const uint16_t* __restrict__ x, int64_t ld_x, const float* __restrict__ wt,
    const float* __restrict__ bias, int64_t T, int d, int E, float* __restrict__ out) {
  using RB = RouterBlock<1, R>;
  extern __shared__ __align__(16) unsigned char smem[];
  float* xch = reinterpret_cast<float*>(smem);  // [64][33] over the stages
  const int64_t t0 = (int64_t)blockIdx.x * kRouteBlock;
  const int e0 = blockIdx.y * 32;
  const int nchunk = (d + kRouterChunk - 1) / kRouterChunk;
  const floatx16 sum = RB::run(x, ld_x, wt, T, d, E, t0, e0, 0, nchunk, smem, xch, 33);
  const int lane = lane_id(), wave = wave_id();
  const int e = e0 + (lane & 31);
  if (wave % R == R - 1 && e < E) {
    const int sub = wave / R;
    const float bv = bias ? bias[e] : 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t t = t0 + sub * 32 + acc_row(i, lane);
      if (t < T) out[t * E + e] = bias ? sum[i] + bv : sum[i];
    }
  }
}

inline size_t router_logits_lds_bytes(int R) { return (size_t)2 * R * (kXStageBytes + 64 * 32 * 4); }

// ---- Streamed router ----------------------------------------------------------------------
// For more than 128 experts. One workgroup per 64-token block computes the block's logits for
// every expert (E <= 32 EBW) and ranks them. Wave w owns expert block w: two fixed-order chains,
// the block's two 32-token halves against its 32 experts, over all chunks; a router weight
// operand feeds both.
// Token rows are staged in LDS once per block: per 64-feature stage a [64 rows][128 B] tile,
// written by 16-byte direct-to-LDS buffer loads (chunk c of row j at slot c ^ ((j >> 1) & 7),
// so a fragment read of 32 rows at one chunk is conflict-free), in a ring of four stages filled
// two stages ahead. Router weights are not shared between waves: each lane loads its B operands
// straight from w_router_t [d, E] into registers, one stage ahead (per stage 32 values, features
// 8 q + 2 j + (lane / 32) of its expert). One barrier per stage.
// Measured against the one-workgroup-per-expert-block logits kernel (which re-reads x once per
// expert block and stages the weights through LDS) at T = 16384, d = 1280, E = 256: 142 us for
// logits and top-k against 230 us.
constexpr int kSRing = 4;                    // LDS stages in the ring
constexpr int kSRow = 128;                   // bytes per staged row (64 bf16 features)
constexpr int kSTile = kRouteBlock * kSRow;  // one stage: 8 KB

// 16 bytes per lane from a buffer at byte offset voff into LDS at dst + 16 lane (dst uniform).
__device__ __forceinline__ void buffer_copy_lds16(__amdgpu_buffer_rsrc_t rsrc, unsigned char* dst,
                                                  int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lvoid*)dst, 16, voff, 0, 0, 0);
}

// One fp32 per lane from the buffer rsrc at byte offset voff + soff (soff wave-uniform), as
// inline assembly: the compiler neither moves it next to its first use nor adds waits of its own
// for it (its wait analysis is conservative across loop back-edges and would wait for the next
// stage's loads); the caller waits with stage_wait() before the result is read.
__device__ __forceinline__ float load_w_asm(__amdgpu_buffer_rsrc_t rsrc, int voff, int soff) {
  float v;
  asm volatile("buffer_load_dword %0, %1, %2, %3 offen"
               : "=v"(v)
               : "v"(voff), "s"(rsrc), "s"(soff)
               : "memory");
  return v;
}

// s_waitcnt vmcnt(N) that also stands as the producer of the 32 weight registers loaded by
// load_w_asm, so no read of them is scheduled before the wait.
template <int N>
__device__ __forceinline__ void stage_wait(float (&w)[32]) {
  asm volatile("s_waitcnt vmcnt(%16)"
               : "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]), "+v"(w[4]), "+v"(w[5]),
                 "+v"(w[6]), "+v"(w[7]), "+v"(w[8]), "+v"(w[9]), "+v"(w[10]), "+v"(w[11]),
                 "+v"(w[12]), "+v"(w[13]), "+v"(w[14]), "+v"(w[15])
               : "n"(N)
               : "memory");
  asm volatile(""
               : "+v"(w[16]), "+v"(w[17]), "+v"(w[18]), "+v"(w[19]), "+v"(w[20]), "+v"(w[21]),
                 "+v"(w[22]), "+v"(w[23]), "+v"(w[24]), "+v"(w[25]), "+v"(w[26]), "+v"(w[27]),
                 "+v"(w[28]), "+v"(w[29]), "+v"(w[30]), "+v"(w[31])
               :
               : "memory");
}

template <int EBW>
struct StreamGeo {
  static constexpr int kThreads = 64 * EBW;
  static constexpr int kXCopies = 8 / EBW;  // 1 KB copies per wave per stage (8 in total)
  static_assert(kXCopies * EBW == 8, "x copies per stage");
  static constexpr size_t ring_bytes() { return (size_t)kSRing * kSTile; }
  static constexpr size_t lds_bytes(int E) {
    return ring_bytes() + router_lds_bytes(E);
  }
};

template <int EBW, int KMAX>
__global__ __launch_bounds__(64 * EBW) void router_stream_kernel(
    const uint16_t* __restrict__ x, int64_t ld_x, const float* __restrict__ wt,
    const float* __restrict__ bias, int64_t T, int d, int E, int k, int score_fn,
    float* __restrict__ logits, int32_t* __restrict__ topk_ids, float* __restrict__ topk_w,
    float* __restrict__ prob_partial, float* __restrict__ z_partial,
    int32_t* __restrict__ block_counts) {
  using G = StreamGeo<EBW>;
  extern __shared__ __align__(16) unsigned char smem[];
  float* lg = reinterpret_cast<float*>(smem + G::ring_bytes());
  float* zt = reinterpret_cast<float*>(smem + G::ring_bytes() + zt_offset(E));
  const int lane = lane_id(), wave = wave_id();
  const int64_t t0 = (int64_t)blockIdx.x * kRouteBlock;
  const int n_stages = (d + 63) / 64;

  // x copies of this wave: copy i is block b = wave + i EBW of the stage (rows 8 b + lane / 8,
  // slot lane % 8 holding chunk slot ^ ((row >> 1) & 7)). Buffer loads against this block's
  // rows: a row past T or a feature past the last row's end reads 0, and features past d are
  // never multiplied, so no clamping is needed.
  const int rows = T - t0 < kRouteBlock ? (int)(T - t0) : kRouteBlock;
  const __amdgpu_buffer_rsrc_t xrsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(x + t0 * ld_x), 0, (int)(((int64_t)(rows - 1) * ld_x + d) * 2), kBufferWord3);
  int xoff[G::kXCopies];
#pragma unroll
  for (int i = 0; i < G::kXCopies; ++i) {
    const int row = 8 * (wave + i * EBW) + (lane >> 3);
    xoff[i] = (int)(row * ld_x * 2) + (((lane & 7) ^ ((row >> 1) & 7)) << 4);
  }
  auto issue_x = [&](int st, int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < G::kXCopies; ++i)
      buffer_copy_lds16(xrsrc, smem + (size_t)slot * kSTile + (wave + i * EBW) * 1024,
                        xoff[i] + st * 128);
  };
  const int ec = wave * 32 + (lane & 31);
  const int ecl = ec < E ? ec : E - 1;
  const int hk = lane >> 5;  // feature parity this lane supplies
  const __amdgpu_buffer_rsrc_t wrsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)wt, 0, (int)((int64_t)d * E * 4), kBufferWord3);
  // Router weights of stage st for this wave, without branches (a join of two load paths could
  // make the compiler copy registers whose loads are still in flight): the row of each feature
  // pair, clamped to the last pair, is the scalar operand, the lane's parity and expert the
  // vector one. Pairs past a partial last stage read valid, unused weights.
  const int voff_w = (hk * E + ecl) * 4;
  auto issue_w = [&](int st, float (&wr)[32]) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < 8; ++q)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int f = st * 64 + 8 * q + 2 * j;
        wr[4 * q + j] = load_w_asm(wrsrc, voff_w, (f < d - 2 ? f : d - 2) * E * 4);
      }
  };
  const uint32_t sel = hk ? 0x07060C0Cu : 0x05040C0Cu;
  const int row0 = lane & 31, row1 = 32 + (lane & 31);
  const int sw0 = (row0 >> 1) & 7, sw1 = (row1 >> 1) & 7;
  // The stage's chains, with the next stage's weight loads (wn) issued four at a time after each
  // group of eight MFMAs: issued together at the stage's start they filled the wave's memory
  // queue and held back its first MFMAs.
  auto compute = [&](int st, const float (&wr)[32], float (&wn)[32], floatx16& c0, floatx16& c1)
                     __attribute__((always_inline)) {
    const int left = d - st * 64;
    const int ng = left >= 64 ? 8 : left / 8;
    const unsigned char* tile = smem + (size_t)(st % kSRing) * kSTile;
    // All of the stage's token fragments are read first (in order, so the MFMAs of group q wait
    // only for its own reads): with two waves per SIMD in step with each other, a read issued
    // just ahead of its MFMAs would leave the matrix pipe idle for the LDS latency in every group.
    u32x4 x0[8], x1[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      x0[q] = *reinterpret_cast<const u32x4*>(tile + row0 * kSRow + ((q ^ sw0) << 4));
      x1[q] = *reinterpret_cast<const u32x4*>(tile + row1 * kSRow + ((q ^ sw1) << 4));
    }
    auto group = [&](int q) __attribute__((always_inline)) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float a0 = __builtin_bit_cast(float, __builtin_amdgcn_perm(x0[q][j], 0u, sel));
        const float a1 = __builtin_bit_cast(float, __builtin_amdgcn_perm(x1[q][j], 0u, sel));
        c0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, wr[4 * q + j], c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, wr[4 * q + j], c1, 0, 0, 0);
      }
    };
    auto next_w = [&](int q) __attribute__((always_inline)) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int f = (st + 1) * 64 + 8 * q + 2 * j;
        wn[4 * q + j] = load_w_asm(wrsrc, voff_w, (f < d - 2 ? f : d - 2) * E * 4);
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    if (ng == 8) {
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        group(q);
        next_w(q);
      }
    } else {
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        if (q < ng) group(q);
        next_w(q);
      }
    }
  };
  // Stage st: issue the x copies of st + 2, wait until x(st) and W(st) are complete (at most the
  // operations issued after W(st) outstanding: x(st + 1) and x(st + 2) for stage 0, whose
  // weights were loaded before the loop, and x(st + 2) later, W(st) having been issued during
  // stage st - 1's chains after x(st + 1); vector memory operations retire in order), then the
  // chains, which issue W(st + 1). Past the last stage these loads read in-bounds data nobody
  // uses.
  auto stage = [&](int st, float (&wcur)[32], float (&wnext)[32], floatx16& c0, floatx16& c1)
                   __attribute__((always_inline)) {
    issue_x(st + 2, (st + 2) % kSRing);
    if (st == 0) stage_wait<2 * G::kXCopies>(wcur);
    else stage_wait<G::kXCopies>(wcur);
    // Barrier without a memory fence (a fence would wait for the prefetches too): every wave's
    // copies of stage st have landed (its own vmcnt wait above), and every wave's reads of the
    // slot refilled next stage are complete (lgkmcnt).
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    compute(st, wcur, wnext, c0, c1);
  };

  float wa[32], wb[32];
  issue_x(0, 0);
  issue_w(0, wa);
  issue_x(1, 1);
  // One chunk (128 features, the fixed order's chain) = stages 2 i (weights in wa) and 2 i + 1
  // (wb); the last chunk may have one stage.
  floatx16 s0 = {}, s1 = {};
  const int n_chunks = (n_stages + 1) / 2;
  for (int i = 0; i < n_chunks; ++i) {
    floatx16 c0 = {}, c1 = {};
    stage(2 * i, wa, wb, c0, c1);
    if (2 * i + 1 < n_stages) stage(2 * i + 1, wb, wa, c0, c1);
    s0 = i == 0 ? c0 : s0 + c0;
    s1 = i == 0 ? c1 : s1 + c1;
  }
  // Every copy and weight load (including those past the end) has landed before the ring is
  // reused and before their registers can be: the waits hold both weight buffers.
  stage_wait<0>(wa);
  stage_wait<0>(wb);
  __syncthreads();
  // Logits (+ bias) into the tile lg[64][E+1].
  if (ec < E) {
    const float bv = bias ? bias[ec] : 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      lg[acc_row(i, lane) * (E + 1) + ec] = bias ? s0[i] + bv : s0[i];
      lg[(32 + acc_row(i, lane)) * (E + 1) + ec] = bias ? s1[i] + bv : s1[i];
    }
  }
  __syncthreads();
  if (logits) write_logits_out(lg, t0, T, E, logits);
  topk_and_scores<KMAX, EBW>(lg, zt, t0, T, E, k, score_fn, topk_ids, topk_w, prob_partial,
                             z_partial, block_counts);
}

// ---- Chunk-per-wave router -----------------------------------------------------------------
// For up to 32 experts and up to 8 chunks (d <= 1024), one workgroup per 64-token block: wave j
// computes chunk sum c_j of all 64 tokens (two chains, one per 32-token half, sharing each
// router weight operand) from token rows it stages itself, so no wave waits for another until
// every chunk sum is done. Per wave: the block's rows of its 128 features (two [64 rows][128 B]
// tiles, 16 KB, the streamed kernel's swizzled layout, written by its own 16-byte direct-to-LDS
// buffer loads) and its 64 router weight operands per lane (straight into registers); the chains
// run as soon as the wave's own first tile and weights have landed. The chunk sums then go to
// LDS over the wave's own tiles and the fixed-order sum ((c_0 + c_1) + c_2) + ... (+ bias) fills
// the logits tile, ranked as in the other fused kernels.
template <int NW>
struct ChunkGeo {
  static constexpr int kWaveBytes = 2 * kSTile;  // two [64 rows][128 B] tiles per wave
  static constexpr int kCsPitch = 33;            // floats per row of a wave's chunk-sum tile
  static_assert(kRouteBlock * kCsPitch * 4 <= kWaveBytes, "chunk sums fit the wave's tiles");
  static constexpr size_t lds_bytes(int E) { return (size_t)NW * kWaveBytes + router_lds_bytes(E); }
};

template <int NW, int KMAX>
__global__ __launch_bounds__(64 * NW) void router_chunk_kernel(
    const uint16_t* __restrict__ x, int64_t ld_x, const float* __restrict__ wt,
    const float* __restrict__ bias, int64_t T, int d, int E, int k, int score_fn,
    float* __restrict__ logits, int32_t* __restrict__ topk_ids, float* __restrict__ topk_w,
    float* __restrict__ prob_partial, float* __restrict__ z_partial,
    int32_t* __restrict__ block_counts) {
  using G = ChunkGeo<NW>;
  extern __shared__ __align__(16) unsigned char smem[];
  float* lg = reinterpret_cast<float*>(smem + NW * G::kWaveBytes);
  float* zt = reinterpret_cast<float*>(smem + NW * G::kWaveBytes + zt_offset(E));
  const int lane = lane_id(), wave = wave_id();
  const int64_t t0 = (int64_t)blockIdx.x * kRouteBlock;
  const int nchunk = (d + kRouterChunk - 1) / kRouterChunk;
  unsigned char* xs = smem + wave * G::kWaveBytes;
  const int ec = lane & 31;
  if (wave < nchunk) {
    const int f0 = wave * kRouterChunk;
    const int fe = f0 + kRouterChunk < d ? f0 + kRouterChunk : d;
    // Token rows [t0, t0 + rows): a row past T or a feature past the last row's end reads 0
    // (buffer range check); features past fe are never multiplied.
    const int rows = T - t0 < kRouteBlock ? (int)(T - t0) : kRouteBlock;
    const __amdgpu_buffer_rsrc_t xrsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(x + t0 * ld_x), 0, (int)(((int64_t)(rows - 1) * ld_x + d) * 2), kBufferWord3);
    // Copy i of tile h: rows 8 i + lane / 8, LDS slot lane % 8 holding chunk slot ^ ((row >> 1) & 7)
    // of features [f0 + 64 h, +64).
    auto issue_tile = [&](int h) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int row = 8 * i + (lane >> 3);
        const int voff = (int)(row * ld_x * 2) + (((lane & 7) ^ ((row >> 1) & 7)) << 4) +
                         (f0 + 64 * h) * 2;
        buffer_copy_lds16(xrsrc, xs + h * kSTile + i * 1024, voff);
      }
    };
    const int ecl = ec < E ? ec : E - 1;
    const int hk = lane >> 5;  // feature parity this lane supplies
    const __amdgpu_buffer_rsrc_t wrsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)wt, 0, (int)((int64_t)d * E * 4), kBufferWord3);
    const int voff_w = (hk * E + ecl) * 4;
    // Operands of tile h: pair 4 q + j is features f0 + 64 h + 8 q + 2 j + hk (pairs past d read
    // the last pair, unused).
    auto issue_w = [&](int h, float (&wr)[32]) __attribute__((always_inline)) {
#pragma unroll
      for (int q = 0; q < 8; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int f = f0 + 64 * h + 8 * q + 2 * j;
          wr[4 * q + j] = load_w_asm(wrsrc, voff_w, (f < d - 2 ? f : d - 2) * E * 4);
        }
    };
    const uint32_t sel = hk ? 0x07060C0Cu : 0x05040C0Cu;
    const int row0 = lane & 31, row1 = 32 + (lane & 31);
    const int sw0 = (row0 >> 1) & 7, sw1 = (row1 >> 1) & 7;
    floatx16 c0 = {}, c1 = {};
    // Tile h's chains; with issue, tile 1's weight loads (into wn) go out four at a time after
    // each group of eight MFMAs (issued together ahead of them they held back the products).
    auto compute = [&](int h, const float (&wr)[32], float (&wn)[32], bool issue)
                       __attribute__((always_inline)) {
      const int left = fe - (f0 + 64 * h);
      const int ng = left >= 64 ? 8 : (left > 0 ? left / 8 : 0);
      const unsigned char* tile = xs + h * kSTile;
      u32x4 x0[8], x1[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        x0[q] = *reinterpret_cast<const u32x4*>(tile + row0 * kSRow + ((q ^ sw0) << 4));
        x1[q] = *reinterpret_cast<const u32x4*>(tile + row1 * kSRow + ((q ^ sw1) << 4));
      }
      auto group = [&](int q) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float a0 = __builtin_bit_cast(float, __builtin_amdgcn_perm(x0[q][j], 0u, sel));
          const float a1 = __builtin_bit_cast(float, __builtin_amdgcn_perm(x1[q][j], 0u, sel));
          c0 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, wr[4 * q + j], c0, 0, 0, 0);
          c1 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, wr[4 * q + j], c1, 0, 0, 0);
        }
      };
      auto next_w = [&](int q) __attribute__((always_inline)) {
        if (issue) {
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int f = f0 + 64 + 8 * q + 2 * j;
            wn[4 * q + j] = load_w_asm(wrsrc, voff_w, (f < d - 2 ? f : d - 2) * E * 4);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      };
      if (ng == 8) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          group(q);
          next_w(q);
        }
      } else {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          if (q < ng) group(q);
          next_w(q);
        }
      }
    };
    float wlo[32], whi[32];
    issue_tile(0);
    issue_w(0, wlo);
    issue_tile(1);
    // Tile 0 and its weights are the first 40 operations: at most tile 1's 8 copies after them
    // outstanding. Tile 1's weights go out during tile 0's chains.
    stage_wait<8>(wlo);
    compute(0, wlo, whi, true);
    stage_wait<0>(whi);
    compute(1, whi, whi, false);
    // Chunk sums over this wave's own tiles (its LDS reads of them are complete: a wave's LDS
    // operations run in order).
    float* cs = reinterpret_cast<float*>(xs);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      cs[acc_row(i, lane) * G::kCsPitch + ec] = c0[i];
      cs[(32 + acc_row(i, lane)) * G::kCsPitch + ec] = c1[i];
    }
  }
  __syncthreads();
  // logit = ((c_0 + c_1) + c_2) + ... (+ bias) into the tile lg[64][E+1].
  for (int idx = threadIdx.x; idx < kRouteBlock * E; idx += blockDim.x) {
    const int r = idx / E, e = idx - r * E;
    float v = reinterpret_cast<const float*>(smem)[r * G::kCsPitch + e];
    for (int c = 1; c < nchunk; ++c)
      v = v + reinterpret_cast<const float*>(smem + c * G::kWaveBytes)[r * G::kCsPitch + e];
    if (bias) v = v + bias[e];
    lg[r * (E + 1) + e] = v;
  }
  __syncthreads();
  if (logits) write_logits_out(lg, t0, T, E, logits);
  topk_and_scores<KMAX, NW>(lg, zt, t0, T, E, k, score_fn, topk_ids, topk_w, prob_partial,
                            z_partial, block_counts);
}

// Split: the chunk sum c_j (blockIdx.y = j) of a 64-token x 32-expert block (blockIdx.z) ->
// partials[j][t][e], token-major (a wave's store covers 32 consecutive experts of a token).
__global__ __launch_bounds__(128) void router_mfma_partial_kernel(
    const uint16_t* __restrict__ x, int64_t ld_x, const float* __restrict__ wt, int64_t T, int d,
    int E, float* __restrict__ partials) {
  using RB = RouterBlock<1, 1>;
  __shared__ __align__(16) unsigned char smem[RB::stage_bytes()];
  float* xch = reinterpret_cast<float*>(smem);
  const int64_t t0 = (int64_t)blockIdx.x * kRouteBlock;
  const int c = blockIdx.y, e0 = blockIdx.z * 32;
  const floatx16 sum = RB::run(x, ld_x, wt, T, d, E, t0, e0, c, c + 1, smem, xch, 33);
  const int lane = lane_id(), sub = wave_id();
  const int e = e0 + (lane & 31);
  if (e < E) {
    float* out = partials + (int64_t)c * T * E + e;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t t = t0 + sub * 32 + acc_row(i, lane);
      if (t < T) out[t * E] = sum[i];
    }
  }
}

// Sums the nchunk partial planes ([t][e]) of the split router into plane 0, in place, in the
// fixed order ((p0 + p1) + p2) + ... then + bias[e]: four consecutive values per thread, the
// planes' loads issued together. This keeps the plane reduction off the top-k kernel, whose grid
// has one block per 64 tokens and so cannot hide the loads' latency when T is small.
__global__ __launch_bounds__(256) void router_sum_planes_kernel(float* __restrict__ partials,
                                                                 int nchunk,
                                                                 const float* __restrict__ bias,
                                                                 int64_t n4, int E) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  const int64_t plane4 = n4;  // plane size in float4 units
  floatx4* p = reinterpret_cast<floatx4*>(partials) + i;
  floatx4 v = p[0];
  for (int c0 = 1; c0 < nchunk; c0 += 8) {
    floatx4 part[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (c0 + j < nchunk) part[j] = p[(int64_t)(c0 + j) * plane4];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (c0 + j < nchunk) {
        v[0] = v[0] + part[j][0];
        v[1] = v[1] + part[j][1];
        v[2] = v[2] + part[j][2];
        v[3] = v[3] + part[j][3];
      }
  }
  if (bias) {
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = v[j] + bias[(i * 4 + j) % E];
  }
  p[0] = v;
}

// Sum nchunk partial planes ([t][e], token-major) in ascending order (+ bias), then top-k; with
// nchunk = 1 and no bias the plane is caller-supplied logits. The tile loads walk the contiguous
// index.
template <int KMAX>
__global__ __launch_bounds__(1024) void router_topk_kernel(
    const float* __restrict__ partials, int nchunk, const float* __restrict__ bias, int64_t T,
    int E, int k, int score_fn,
    float* __restrict__ logits, int32_t* __restrict__ topk_ids, float* __restrict__ topk_w,
    float* __restrict__ prob_partial, float* __restrict__ z_partial,
    int32_t* __restrict__ block_counts) {
  extern __shared__ __align__(16) unsigned char smem[];
  float* lg = reinterpret_cast<float*>(smem);
  float* zt = reinterpret_cast<float*>(smem + zt_offset(E));
  const int64_t t0 = (int64_t)blockIdx.x * kRouteBlock;
  // Chunk planes are summed in ascending order; loads go out 8 planes at a time so the sum is
  // not a chain of dependent memory round trips.
  const int64_t plane = T * E;
  // Tile index idx -> (token row r, expert e), contiguous in memory along idx.
  auto row_of = [&](int idx) { return idx / E; };
  auto col_of = [&](int idx) { return idx % E; };
  auto at = [&](int64_t t, int e) { return t * E + e; };
  if (nchunk == 1) {
    // One plane (the split router's planes are summed by router_sum_planes_kernel): eight loads
    // per thread go out together, so a block does not wait on one round trip per element.
    for (int base = threadIdx.x; base < kRouteBlock * E; base += 8 * blockDim.x) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int idx = base + j * blockDim.x;
        const int r = row_of(idx), e = col_of(idx);
        const int64_t t = t0 + r;
        v[j] = (idx < kRouteBlock * E && t < T) ? partials[at(t, e)] : 0.f;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int idx = base + j * blockDim.x;
        if (idx >= kRouteBlock * E) break;
        const int r = row_of(idx), e = col_of(idx);
        const int64_t t = t0 + r;
        float val = v[j];
        if (t < T) {
          if (bias) val = val + bias[e];
          if (logits) logits[t * E + e] = val;
        }
        lg[r * (E + 1) + e] = val;
      }
    }
  }
  for (int idx = nchunk == 1 ? kRouteBlock * E : threadIdx.x; idx < kRouteBlock * E;
       idx += blockDim.x) {
    const int r = row_of(idx), e = col_of(idx);
    int64_t t = t0 + r;
    float v = 0.f;
    if (t < T) {
      const float* p = partials + at(t, e);
      v = p[0];
      for (int c0 = 1; c0 < nchunk; c0 += 8) {
        float part[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) part[j] = c0 + j < nchunk ? p[(int64_t)(c0 + j) * plane] : 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (c0 + j < nchunk) v = v + part[j];
      }
      if (bias) v = v + bias[e];
      if (logits) logits[t * E + e] = v;
    }
    lg[r * (E + 1) + e] = v;
  }
  __syncthreads();
  topk_and_scores<KMAX, 16>(lg, zt, t0, T, E, k, score_fn, topk_ids, topk_w, prob_partial,
                            z_partial, block_counts);
}

int kmax_for(int k) { return k <= 2 ? 2 : (k <= 4 ? 4 : 8); }

// Expert blocks of 32 (a power of two: the fused kernel's waves per token row set the top-k's
// lanes per token).
int expert_blocks(int E) {
  int eb = 1;
  while (eb * 32 < E) eb <<= 1;
  return eb;
}

// Feature ranges per output block of the fused kernel: two when there is one expert block and
// at most 8 chunks (the second range keeps up to 4 chunk sums in registers), else one.
int router_ranges(int d, int E) {
  const int nchunk = ceil_div(d, kRouterChunk);
  if (expert_blocks(E) != 1 || nchunk < 2) return 1;
  return nchunk >= 4 && nchunk <= 16 ? 4 : (nchunk <= 8 ? 2 : 1);
}

// NT_MOE_ROUTER_MODE=fused|split|stream overrides the size heuristic (for tuning runs): fused =
// the fused range kernel (up to 128 experts, never the chunk-per-wave one), split = chunk
// planes, stream = the streamed kernel
// (129-256 experts).
int router_mode_override() {
  static int mode = [] {
    const char* s = getenv("NT_MOE_ROUTER_MODE");
    if (!s) return 0;
    if (!strcmp(s, "fused")) return 1;
    if (!strcmp(s, "split")) return 2;
    if (!strcmp(s, "stream")) return 3;
    return 0;
  }();
  return mode;
}

template <int KMAX>
hipError_t launch_topk_k(const float* partials, int nchunk, const float* bias, int64_t T, int E,
                         int k, int score_fn, float* logits, int32_t* ids, float* w, float* pp,
                         float* zp, int32_t* bc, hipStream_t stream) {
  dim3 grid(ceil_div(T, kRouteBlock));
  hipError_t err = allow_dynamic_lds(reinterpret_cast<const void*>(router_topk_kernel<KMAX>),
                                     router_lds_bytes(E));
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL((router_topk_kernel<KMAX>), grid, dim3(1024), router_lds_bytes(E), stream,
                     partials, nchunk, bias, T, E, k, score_fn, logits, ids, w, pp, zp, bc);
  return hipGetLastError();
}

hipError_t launch_topk_any(const float* partials, int nchunk, const float* bias, int64_t T,
                           int E, int k, int score_fn, float* logits, int32_t* ids, float* w,
                           float* pp, float* zp, int32_t* bc, hipStream_t stream) {
  switch (kmax_for(k)) {
    case 2: return launch_topk_k<2>(partials, nchunk, bias, T, E, k, score_fn, logits, ids, w, pp, zp, bc, stream);
    case 4: return launch_topk_k<4>(partials, nchunk, bias, T, E, k, score_fn, logits, ids, w, pp, zp, bc, stream);
    default: return launch_topk_k<8>(partials, nchunk, bias, T, E, k, score_fn, logits, ids, w, pp, zp, bc, stream);
  }
}

template <int EB, int R, int KMAX>
hipError_t launch_mfma_k(const uint16_t* x, int64_t ld_x, const float* wt, const float* bias,
                         int64_t T, int d, int E, int k, int score_fn, float* logits,
                         int32_t* ids, float* w, float* pp, float* zp, int32_t* bc, hipStream_t stream) {
  auto kern = router_mfma_kernel<EB, R, KMAX>;
  const size_t lds = router_mfma_lds_bytes(EB, R, E);
  hipError_t err = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds);
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(kern, dim3(ceil_div(T, kRouteBlock)), dim3(128 * EB * R), lds, stream, x,
                     ld_x, wt, bias, T, d, E, k, score_fn, logits, ids, w, pp, zp, bc);
  return hipGetLastError();
}

template <int EB, int R>
hipError_t launch_mfma_r(const uint16_t* x, int64_t ld_x, const float* wt, const float* bias,
                         int64_t T, int d, int E, int k, int score_fn, float* logits,
                         int32_t* ids, float* w, float* pp, float* zp, int32_t* bc, hipStream_t stream) {
  switch (kmax_for(k)) {
    case 2: return launch_mfma_k<EB, R, 2>(x, ld_x, wt, bias, T, d, E, k, score_fn, logits, ids, w, pp, zp, bc, stream);
    case 4: return launch_mfma_k<EB, R, 4>(x, ld_x, wt, bias, T, d, E, k, score_fn, logits, ids, w, pp, zp, bc, stream);
    default: return launch_mfma_k<EB, R, 8>(x, ld_x, wt, bias, T, d, E, k, score_fn, logits, ids, w, pp, zp, bc, stream);
  }
}

// Feature ranges of the logits kernel: up to 4, each at most 4 chunks (so d <= 2048).
int logit_ranges(int d) {
  const int nchunk = ceil_div(d, kRouterChunk);
  return nchunk >= 4 ? 4 : (nchunk >= 2 ? 2 : 1);
}

enum RouterPath { kFused = 0, kLogits = 1, kPlanes = 2, kStream = 3 };

// Path for this shape. Up to 128 experts: the fused kernel (top-k in the block, no workspace)
// when every CU gets a 64-token block, else the logits kernel (one workgroup per 64 tokens x 32
// experts, up to 16 chunks) when that gives two waves per CU, else chunk planes (small T, planes
// capped at 512 MB). 129-256 experts: the streamed kernel (top-k in the block, no workspace)
// when it gives every other SIMD a wave. Measured on MI355X, router alone: T = 16384, d = 1280,
// E = 256 streamed 142 us (logits + top-k 230); T = 32768, d = 2048, E = 64 fused 122 us
// (streamed 133); T = 8192, d = 2048, E = 128 logits + top-k 121 us (streamed 131).
int router_path(int64_t T, int d, int E) {
  const int mode = router_mode_override();
  const int nchunk = ceil_div(d, kRouterChunk);
  const int64_t blocks = ceil_div(T, kRouteBlock);
  const int64_t logit_waves = blocks * (int64_t)ceil_div(E, 32) * 2 * logit_ranges(d);
  const int64_t plane_bytes = (int64_t)nchunk * T * E * (int64_t)sizeof(float);
  if (mode == 2) return kPlanes;
  if (mode == 1) return E <= 128 ? kFused : kLogits;
  if (mode == 3) return E > 128 && E <= 256 ? kStream : kLogits;
  if (E <= 128 && blocks >= num_cus()) return kFused;
  if (E > 128 && E <= 256 && blocks * 8 >= 2LL * num_cus()) return kStream;
  if (nchunk <= 16 && logit_waves >= 2LL * num_cus()) return kLogits;
  if (plane_bytes <= (512LL << 20)) return kPlanes;
  return nchunk <= 16 ? kLogits : (E <= 128 ? kFused : kStream);
}

template <int KMAX>
hipError_t launch_stream_k(const uint16_t* x, int64_t ld_x, const float* wt, const float* bias,
                           int64_t T, int d, int E, int k, int score_fn, float* logits,
                           int32_t* ids, float* w, float* pp, float* zp, int32_t* bc, hipStream_t stream) {
  auto kern = router_stream_kernel<8, KMAX>;
  const size_t lds = StreamGeo<8>::lds_bytes(E);
  hipError_t err = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds);
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(kern, dim3(ceil_div(T, kRouteBlock)), dim3(StreamGeo<8>::kThreads), lds,
                     stream, x, ld_x, wt, bias, T, d, E, k, score_fn, logits, ids, w, pp, zp, bc);
  return hipGetLastError();
}

template <int NW, int KMAX>
hipError_t launch_chunk_k(const uint16_t* x, int64_t ld_x, const float* wt, const float* bias,
                          int64_t T, int d, int E, int k, int score_fn, float* logits,
                          int32_t* ids, float* w, float* pp, float* zp, int32_t* bc, hipStream_t stream) {
  auto kern = router_chunk_kernel<NW, KMAX>;
  const size_t lds = ChunkGeo<NW>::lds_bytes(E);
  hipError_t err = allow_dynamic_lds(reinterpret_cast<const void*>(kern), lds);
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(kern, dim3(ceil_div(T, kRouteBlock)), dim3(64 * NW), lds, stream, x, ld_x,
                     wt, bias, T, d, E, k, score_fn, logits, ids, w, pp, zp, bc);
  return hipGetLastError();
}

template <int NW>
hipError_t launch_chunk_w(const uint16_t* x, int64_t ld_x, const float* wt, const float* bias,
                          int64_t T, int d, int E, int k, int score_fn, float* logits,
                          int32_t* ids, float* w, float* pp, float* zp, int32_t* bc, hipStream_t stream) {
  switch (kmax_for(k)) {
    case 2: return launch_chunk_k<NW, 2>(x, ld_x, wt, bias, T, d, E, k, score_fn, logits, ids, w, pp, zp, bc, stream);
    case 4: return launch_chunk_k<NW, 4>(x, ld_x, wt, bias, T, d, E, k, score_fn, logits, ids, w, pp, zp, bc, stream);
    default: return launch_chunk_k<NW, 8>(x, ld_x, wt, bias, T, d, E, k, score_fn, logits, ids, w, pp, zp, bc, stream);
  }
}

// The chunk-per-wave kernel: up to 32 experts and 8 chunks, one wave per chunk (2, 4 or 8).
bool chunk_router_fits(int d, int E) { return E <= 32 && ceil_div(d, kRouterChunk) <= 8; }

hipError_t launch_chunk(const uint16_t* x, int64_t ld_x, const float* wt, const float* bias,
                        int64_t T, int d, int E, int k, int score_fn, float* logits,
                        int32_t* ids, float* w, float* pp, float* zp, int32_t* bc, hipStream_t stream) {
  const int nchunk = ceil_div(d, kRouterChunk);
  if (nchunk <= 2) return launch_chunk_w<2>(x, ld_x, wt, bias, T, d, E, k, score_fn, logits, ids, w, pp, zp, bc, stream);
  if (nchunk <= 4) return launch_chunk_w<4>(x, ld_x, wt, bias, T, d, E, k, score_fn, logits, ids, w, pp, zp, bc, stream);
  return launch_chunk_w<8>(x, ld_x, wt, bias, T, d, E, k, score_fn, logits, ids, w, pp, zp, bc, stream);
}

// The streamed kernel for 129-256 experts (eight 32-expert blocks).
hipError_t launch_stream(const uint16_t* x, int64_t ld_x, const float* wt, const float* bias,
                         int64_t T, int d, int E, int k, int score_fn, float* logits,
                         int32_t* ids, float* w, float* pp, float* zp, int32_t* bc, hipStream_t stream) {
  if (E > 256) return hipErrorInvalidValue;
  switch (kmax_for(k)) {
    case 2: return launch_stream_k<2>(x, ld_x, wt, bias, T, d, E, k, score_fn, logits, ids, w, pp, zp, bc, stream);
    case 4: return launch_stream_k<4>(x, ld_x, wt, bias, T, d, E, k, score_fn, logits, ids, w, pp, zp, bc, stream);
    default: return launch_stream_k<8>(x, ld_x, wt, bias, T, d, E, k, score_fn, logits, ids, w, pp, zp, bc, stream);
  }
}

}  // namespace

// Workspace the router uses for this shape: the chunk planes, one T x E logits plane, or none.
size_t router_workspace_need(int64_t T, int d, int E) {
  const int path = router_path(T, d, E);
  const size_t plane = (size_t)T * (size_t)E * sizeof(float);
  return path == kPlanes ? plane * ceil_div(d, kRouterChunk) : (path == kLogits ? plane : 0);
}

// Runs the path for the shape when its buffers are there; without enough workspace the fused
// kernel (up to 128 experts).
hipError_t launch_router(const uint16_t* x, int64_t ld_x, const float* wt, const float* bias,
                         int64_t T, int d, int E, int k, int score_fn, float* logits,
                         int32_t* topk_ids, float* topk_w, float* prob_partial,
                         float* z_partial, float* workspace, size_t workspace_bytes,
                         hipStream_t stream, int32_t* block_counts) {
  const int nchunk = ceil_div(d, kRouterChunk);
  const int path = router_path(T, d, E);
  const size_t plane = (size_t)T * (size_t)E * sizeof(float);
  hipError_t err;
  if (path == kPlanes && workspace && workspace_bytes >= plane * nchunk) {
    hipLaunchKernelGGL(router_mfma_partial_kernel,
                       dim3((unsigned)ceil_div(T, kRouteBlock), (unsigned)nchunk,
                            (unsigned)ceil_div(E, 32)),
                       dim3(128), 0, stream, x, ld_x, wt, T, d, E, workspace);
    err = hipGetLastError();
    if (err != hipSuccess) return err;
    if (E % 4 == 0) {
      const int64_t n4 = T * E / 4;
      router_sum_planes_kernel<<<dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, stream>>>(
          workspace, nchunk, bias, n4, E);
      err = hipGetLastError();
      if (err != hipSuccess) return err;
      return launch_topk_any(workspace, 1, nullptr, T, E, k, score_fn, logits, topk_ids, topk_w,
                             prob_partial, z_partial, block_counts, stream);
    }
    return launch_topk_any(workspace, nchunk, bias, T, E, k, score_fn, logits, topk_ids, topk_w,
                           prob_partial, z_partial, block_counts, stream);
  }
  if (path == kStream || (path == kPlanes && E > 128 && E <= 256))
    return launch_stream(x, ld_x, wt, bias, T, d, E, k, score_fn, logits, topk_ids, topk_w,
                         prob_partial, z_partial, block_counts, stream);
  float* lbuf = logits ? logits : (workspace && workspace_bytes >= plane ? workspace : nullptr);
  if ((path != kFused || E > 128) && lbuf && nchunk <= 16) {
    const int ranges = logit_ranges(d);
    const dim3 grid((unsigned)ceil_div(T, kRouteBlock), (unsigned)ceil_div(E, 32));
#define NT_LOGITS(R)                                                                       \
  if (ranges == R) {                                                                       \
    auto kern = router_logits_kernel<R>;                                                   \
    err = allow_dynamic_lds(reinterpret_cast<const void*>(kern), router_logits_lds_bytes(R)); \
    if (err != hipSuccess) return err;                                                     \
    hipLaunchKernelGGL(kern, grid, dim3(128 * R), router_logits_lds_bytes(R), stream, x, ld_x, \
                       wt, bias, T, d, E, lbuf);                                           \
  }
    NT_LOGITS(1) NT_LOGITS(2) NT_LOGITS(4)
#undef NT_LOGITS
    err = hipGetLastError();
    if (err != hipSuccess) return err;
    return launch_topk_any(lbuf, 1, nullptr, T, E, k, score_fn, nullptr, topk_ids, topk_w,
                           prob_partial, z_partial, block_counts, stream);
  }
  if (E <= 128) {  // the fused kernel: its path, or planes / logits without their buffers
    // (the chunk-per-wave kernel where it fits, unless NT_MOE_ROUTER_MODE=fused)
    if (chunk_router_fits(d, E) && router_mode_override() != 1)
      return launch_chunk(x, ld_x, wt, bias, T, d, E, k, score_fn, logits, topk_ids, topk_w,
                          prob_partial, z_partial, block_counts, stream);
    const int eb = expert_blocks(E), ranges = router_ranges(d, E);
#define NT_MFMA(EB, R) \
  if (eb == EB && ranges == R) return launch_mfma_r<EB, R>(x, ld_x, wt, bias, T, d, E, k, score_fn, logits, topk_ids, topk_w, prob_partial, z_partial, block_counts, stream);
    NT_MFMA(1, 1) NT_MFMA(1, 2) NT_MFMA(1, 4) NT_MFMA(2, 1) NT_MFMA(4, 1)
#undef NT_MFMA
  }
  if (E <= 256)
    return launch_stream(x, ld_x, wt, bias, T, d, E, k, score_fn, logits, topk_ids, topk_w,
                         prob_partial, z_partial, block_counts, stream);
  return hipErrorInvalidValue;  // more than 256 experts need the workspace or a logits buffer
}

hipError_t launch_topk_from_logits(const float* logits, int64_t T, int E, int k,
                                   int score_fn, int32_t* topk_ids, float* topk_w,
                                   float* prob_partial, float* z_partial, hipStream_t stream) {
  return launch_topk_any(logits, 1, nullptr, T, E, k, score_fn, nullptr, topk_ids, topk_w,
                         prob_partial, z_partial, nullptr, stream);
}

}  // namespace ntmoe
