// Routed-expert path kernels (EschaSparseMoeBlock._expert_path,
// escha_mlx/models/qwen3_5_moe.py:207-253).  Rows are token-major: slot s of
// token t is row t*top_k + s (models/qwen3_5_moe.py:97-101), so a token's
// contributions are rows [t*k, t*k+k) and combine in fixed slot order.
#pragma once

#include "fast.hpp"

namespace esc {

// xh[row] = f16(H128(f32(x[row / k]) * rin[ids[row]]) * RS), 128-block blk
// of one row, by one wave.
__device__ __forceinline__ void moe_input_wave(const uint16_t* __restrict__ x,
                                               const int* __restrict__ ids, int top_k,
                                               const float* __restrict__ rin, int H, float rs,
                                               uint16_t* __restrict__ xh, int blk, int row) {
  const int lane = threadIdx.x & 63;
  const int tok = row / top_k, e = ids[row];
  const int c = blk * 128 + 2 * lane;
  const uint16_t* xr = x + (size_t)tok * H + c;
  const float* r = rin + (size_t)e * H + c;
  float v0 = (float)__builtin_bit_cast(half_t, xr[0]) * r[0];
  float v1 = (float)__builtin_bit_cast(half_t, xr[1]) * r[1];
  h128_wave(v0, v1);
  uint16_t* o = xh + (size_t)row * H + c;
  o[0] = __builtin_bit_cast(uint16_t, to_f16(v0 * rs));
  o[1] = __builtin_bit_cast(uint16_t, to_f16(v1 * rs));
}

// grid (H/128, T*k), block 64.
__global__ __launch_bounds__(64) void k_moe_input(const uint16_t* __restrict__ x,
                                                  const int* __restrict__ ids, int top_k,
                                                  const float* __restrict__ rin, int H, float rs,
                                                  uint16_t* __restrict__ xh) {
  moe_input_wave(x, ids, top_k, rin, H, rs, xh, blockIdx.x, blockIdx.y);
}

// The chain's two independent first steps in one launch: block 0 groups the
// routed rows by expert (build_groups_block); every other block runs 16 of
// the (128-block, row) input transforms, one per wave.  grid
// 1 + ceil(H/128 * m / 16), block 1024.
__global__ __launch_bounds__(1024) void k_moe_prep(const uint16_t* __restrict__ x,
                                                   const int* __restrict__ ids, int top_k,
                                                   const float* __restrict__ rin, int H, float rs,
                                                   uint16_t* __restrict__ xh, int m, int E, int R,
                                                   int n_groups, int* __restrict__ rows_idx,
                                                   int* __restrict__ group_expert,
                                                   int* __restrict__ n_active) {
  if (blockIdx.x == 0) {
    build_groups_block(ids, m, E, R, n_groups, rows_idx, group_expert, n_active);
    return;
  }
  const int nhb = H / 128, w = (blockIdx.x - 1) * 16 + (threadIdx.x >> 6);
  if (w < nhb * m) moe_input_wave(x, ids, top_k, rin, H, rs, xh, w % nhb, w / nhb);
}

// The grouped split-K GEMM of k_gemv_fast_rows with the table decode, as a
// persistent launch: one workgroup of 16 waves per CU requests the
// 65,536-entry table into LDS once (LDS DMA; a short-lived workgroup that
// stages 128 KiB for one wave-step range of a few rows costs more than the
// table saves), then each wave walks a contiguous range of wave-items.  A
// wave-item is one wave's share of k_gemv_fast_rows -- TPS tiles (tw) of
// group g over the KS kt of split z -- and writes the same partial slice
// part[z][row][16 TPS tw ..], so the consumers are unchanged.  Items run
// (g, z, tw) with tw fastest, over the n_active groups build_groups filled
// (groups past them belong to no expert).  The wave walks its items' steps
// as one sequence: each step requests the next step's code and inputs, the
// next item's first step included, and each item's group and rows are
// loaded one item ahead.  Table pairs are the table's image of the hash and
// the MFMAs run in mma_tile's order: the partials are bit-identical to
// k_gemv_fast_rows'.  grid: one workgroup per CU, block 1024, dynamic LDS
// 128 KiB.
// One wave-item's loaded values (both per lane: the expert is read with a
// vector load so that nothing waits for it until the item's first code is
// requested, one item later) and its place.
struct RowsItem {
  int e, row;  // the group's expert, the lane's row (M: padding)
  int z, tw;   // split, wave tile
};

template <int K, int R>
__global__ __launch_bounds__(1024) void k_gemv_rows_table(const uint16_t* __restrict__ xh,
                                                          const uint32_t* __restrict__ code,
                                                          const int* __restrict__ rows_idx,
                                                          const int* __restrict__ group_expert,
                                                          const int* __restrict__ n_active, int M,
                                                          int TK, int TN, int KS, int S,
                                                          float* __restrict__ part) {
  static_assert(R >= 1 && R <= 16, "");
  using G = Geo<K>;
  constexpr int TPS = 16 / G::LPT;
  extern __shared__ uint16_t s_tab[];
  table_dma(s_tab);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int NTW = TN / TPS;  // wave tiles per group row
  const long n = (long)*n_active * S * NTW;
  if (n <= 0) {
    // no filled group (the items below would read group 0, an expert of -1)
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    return;
  }
  const long W = (long)gridDim.x * 16, gw = (long)blockIdx.x * 16 + wave;
  const int i0 = (int)(n * gw / W), i1 = (int)(n * (gw + 1) / W);
  const int gk = lane >> 4, c = lane & 15, tc = c / G::LPT, q = lane % G::LPT;
  const int src = (lane & ~(G::LPT - 1)) | ((lane + G::LPT - 1) & (G::LPT - 1));
  const int rc = c < R ? c : R - 1;  // the lane's B column: row min(c, R-1) of the group
  const size_t kstride = (size_t)TN * (8 * K);
  const size_t estride = (size_t)TK * TN * (8 * K);
  const int last_i = (int)(n - 1);
  auto item = [&](int i) {
    RowsItem it;
    it.tw = i % NTW;
    const int gz = i / NTW, g = gz / S;
    it.z = gz % S;
    // g as a per-lane value (an identity DPP move): the expert is loaded
    // with a vector load, not a scalar one that the next LDS wait would
    // also wait for
    const int gv = __builtin_amdgcn_update_dpp(0, g, 0xE4, 0xF, 0xF, false);
    it.e = group_expert[gv];
    it.row = rows_idx[g * R + rc];
    return it;
  };
  // the lane's code words at kt 0 and its input row
  auto code_of = [&](const RowsItem& it) {
    return code + (size_t)it.e * estride + (size_t)(TPS * it.tw + tc) * (8 * K) + q * G::WPL;
  };
  auto x_of = [&](const RowsItem& it) {
    return reinterpret_cast<const uint4*>(xh + (size_t)(it.row < M ? it.row : 0) * TK * 16);
  };
  // this wave's first item, the next and the one after (each item's values
  // are loaded three items ahead: the compiler computes an item's pointers
  // where the item before it starts)
  RowsItem cur = item(min(i0, last_i)), nxt = item(min(i0 + 1, last_i));
  RowsItem pend = item(min(i0 + 2, last_i));
  const int nsteps = KS / 4;
  const uint32_t* lp = code_of(cur);
  const uint4* xq = x_of(cur);
  int kt = cur.z * KS + gk;
  LaneWords<K> w = load_lane_words_nt<K>(lp + (size_t)kt * kstride);
  uint4 xa = xq[2 * kt], xb = xq[2 * kt + 1];
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's table pieces
  __syncthreads();
  const uint32_t tb = (uint32_t)(size_t)s_tab;
  if (i0 >= i1) return;
  f32x4_t acc[G::NCOL];
#pragma unroll
  for (int j = 0; j < G::NCOL; ++j) acc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int i = i0; i < i1; ++i) {
    const uint32_t* lp_next = code_of(nxt);
    const uint4* xq_next = x_of(nxt);
    const int kt_next = nxt.z * KS + gk;
    RowsItem p3;
    // one wave-step: the next step's code and inputs requested (this item's
    // k + 1, or the next item's first; the last item's re-reads its own: in
    // bounds, unused), then the decode and the MFMAs.  The first step also
    // requests item i + 3's values, just before its own loads: the wait for
    // those covers them, where a load of their own at the item's start would
    // be waited for at the first step
    auto step = [&](int k, bool first) {
      if (first) p3 = item(min(i + 3, i1 - 1));
      const bool last = k + 1 == nsteps;
      const uint32_t* lpn = last ? lp_next : lp;
      const uint4* xqn = last ? xq_next : xq;
      const int ktn = last ? kt_next : kt + 4;
      const LaneWords<K> wn = load_lane_words_nt<K>(lpn + (size_t)ktn * kstride);
      const uint4 na = xqn[2 * ktn], nb = xqn[2 * ktn + 1];
      const uint32_t wprev = __shfl(w.w[G::WPL - 1], src);
      mma_tile_mix<K>(w, wprev, __builtin_bit_cast(u32x4_t, xa), __builtin_bit_cast(u32x4_t, xb),
                      acc, tb);
      w = wn;
      xa = na;
      xb = nb;
      lp = lpn;
      xq = xqn;
      kt = ktn;
    };
    step(0, true);
#pragma unroll 1
    for (int k = 1; k < nsteps; ++k) step(k, false);
    if (c < R && cur.row < M)
      mma_store<K>(acc, gk, part + ((size_t)cur.z * M + cur.row) * TN * 16 + 16 * TPS * cur.tw);
#pragma unroll
    for (int j = 0; j < G::NCOL; ++j) acc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    cur = nxt;
    nxt = pend;
    pend = p3;
  }
}

// h = f16(f16(silu(g)) * u) with silu(g) = g / (1 + exp(-g)) in float32
// (escha_mlx/ref.py:296-301).
__device__ __forceinline__ half_t swiglu1(half_t g, half_t u) {
  const float gf = (float)g;
  const half_t s16 = to_f16(gf / (1.0f + expf(-gf)));
  return to_f16((float)s16 * (float)u);
}

// Split-K sums, in z order, of the partials of several (row, column pair)
// points at once.  SC > 0: S == SC splits, every load in one straight run
// (no branch between them, so they issue back to back and their latencies
// overlap); SC == 0: any S, in chunks of 4 whose loads are unconditional (the
// split index clamped to S - 1) and whose adds take the splits below S.  v
// starts at +0 and a sum of floats from +0 is never -0, so adding +0 for a
// clamped split is exact.  (Loads under a condition each got a full wait for
// the loads before them: one memory latency per load.)  rows[j] must be rows
// of part (0 <= rows[j] < M).
template <int NP, int SC>
__device__ __forceinline__ void sum_splits(const float* __restrict__ part, int S, int M, int OC,
                                           const int* rows, const int* cols, float2* v) {
  auto ld = [&](int z, int j) {
    return *reinterpret_cast<const float2*>(part + ((size_t)z * M + rows[j]) * OC + cols[j]);
  };
#pragma unroll
  for (int j = 0; j < NP; ++j) v[j] = make_float2(0.f, 0.f);
  if constexpr (SC > 0) {
    float2 pv[NP][SC];
#pragma unroll
    for (int j = 0; j < NP; ++j)
#pragma unroll
      for (int z = 0; z < SC; ++z) pv[j][z] = ld(z, j);
#pragma unroll
    for (int j = 0; j < NP; ++j)
#pragma unroll
      for (int z = 0; z < SC; ++z) {
        v[j].x = v[j].x + pv[j][z].x;
        v[j].y = v[j].y + pv[j][z].y;
      }
  } else {
    for (int z0 = 0; z0 < S; z0 += 4) {
      float2 pv[NP][4];
#pragma unroll
      for (int j = 0; j < NP; ++j)
#pragma unroll
        for (int zz = 0; zz < 4; ++zz) pv[j][zz] = ld(min(z0 + zz, S - 1), j);
#pragma unroll
      for (int j = 0; j < NP; ++j)
#pragma unroll
        for (int zz = 0; zz < 4; ++zz) {
          const bool in = z0 + zz < S;
          v[j].x = v[j].x + (in ? pv[j][zz].x : 0.f);
          v[j].y = v[j].y + (in ? pv[j][zz].y : 0.f);
        }
    }
  }
}

// the split counts with a straight-line sum_splits; others take SC = 0
__host__ __device__ constexpr int splits_class(int S) { return S == 1 || S == 2 || S == 4 ? S : 0; }

// gate_up epilogue -> swiglu -> down input transform, one wave per
// (row, 128-block of the intermediate): grid (I/128, M), block 64;
// SC = splits_class(S).
template <int SC>
__global__ __launch_bounds__(64) void k_moe_mid(const float* __restrict__ part, int S, int M,
                                                int I, const int* __restrict__ ids,
                                                const float* __restrict__ gu_rout,
                                                const float* __restrict__ dn_rin, float rs,
                                                uint16_t* __restrict__ xh2) {
  const int b = blockIdx.x, row = blockIdx.y, lane = threadIdx.x;
  const int e = ids[row];
  const int OC = 2 * I;
  const int c = b * 128 + 2 * lane;
  // the expert's scales of the lane's columns, requested before the partial
  // sums so that their latency overlaps the partials'
  const float2 rg = *reinterpret_cast<const float2*>(gu_rout + (size_t)e * OC + c);
  const float2 ru = *reinterpret_cast<const float2*>(gu_rout + (size_t)e * OC + I + c);
  const float2 ri = *reinterpret_cast<const float2*>(dn_rin + (size_t)e * I + c);
  // the gate and up partials of the lane's two columns, summed in z order
  const int rows2[2] = {row, row}, cols2[2] = {c, I + c};
  float2 gu[2];
  sum_splits<2, SC>(part, S, M, OC, rows2, cols2, gu);
  h128_wave(gu[0].x, gu[0].y);
  h128_wave(gu[1].x, gu[1].y);
  const half_t g0 = to_f16((gu[0].x * rs) * rg.x), g1 = to_f16((gu[0].y * rs) * rg.y);
  const half_t u0 = to_f16((gu[1].x * rs) * ru.x), u1 = to_f16((gu[1].y * rs) * ru.y);
  const half_t h0 = swiglu1(g0, u0), h1 = swiglu1(g1, u1);
  float v0 = (float)h0 * ri.x;
  float v1 = (float)h1 * ri.y;
  h128_wave(v0, v1);
  uint16_t* o = xh2 + (size_t)row * I + c;
  o[0] = __builtin_bit_cast(uint16_t, to_f16(v0 * rs));
  o[1] = __builtin_bit_cast(uint16_t, to_f16(v1 * rs));
}

// down epilogue + weighted combine: y[t] = f16(sum_s f32(d16[t*k+s]) * f32(f16(score)))
// summed in slot order in float32 (models/qwen3_5_moe.py:227-253).  The
// partials of 8 slots are requested together, then transformed and summed
// in slot order.  grid (H/128, T), block 64; SC = splits_class(S).
template <int SC>
__global__ __launch_bounds__(64) void k_moe_combine(const float* __restrict__ part, int S,
                                                    int M, int H, const int* __restrict__ ids,
                                                    const float* __restrict__ scores, int top_k,
                                                    const float* __restrict__ dn_rout, float rs,
                                                    uint16_t* __restrict__ y) {
  const int blk = blockIdx.x, tok = blockIdx.y, lane = threadIdx.x;
  const int c = blk * 128 + 2 * lane;
  float a0 = 0.f, a1 = 0.f;
  for (int s0 = 0; s0 < top_k; s0 += 8) {
    // slots past the token's last one re-read its last slot (every load
    // unconditional) and are not summed
    const int n = min(8, top_k - s0);
    int rows[8], cols[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      rows[j] = tok * top_k + s0 + min(j, n - 1);
      cols[j] = c;
    }
    // slot j's expert and weight by lane j (one vector load for the 8
    // slots, not a scalar round trip per slot), then every slot's output
    // scales, requested before the partial sums so that the loads overlap
    const int rl = tok * top_k + s0 + min(lane & 7, n - 1);
    const int e_l = ids[rl];
    const float w_l = (float)(half_t)scores[rl];
    float2 ro[8];
    float w[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int e = __builtin_amdgcn_readlane(e_l, j);
      ro[j] = *reinterpret_cast<const float2*>(dn_rout + (size_t)e * H + c);
      w[j] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w_l), j));
    }
      float2 d[8];
    sum_splits<8, SC>(part, S, M, H, rows, cols, d);
    // no branch between the loads and their use (the compiler would sink
    // each slot's loads into its branch, one latency per slot): the slots
    // past n add +0 (a0, a1 start at +0 and are never -0, so this is exact)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      h128_wave(d[j].x, d[j].y);
      const half_t d0 = to_f16((d[j].x * rs) * ro[j].x);
      const half_t d1 = to_f16((d[j].y * rs) * ro[j].y);
      a0 = a0 + (j < n ? (float)d0 * w[j] : 0.f);
      a1 = a1 + (j < n ? (float)d1 * w[j] : 0.f);
    }
  }
  y[(size_t)tok * H + c] = __builtin_bit_cast(uint16_t, (half_t)a0);
  y[(size_t)tok * H + c + 1] = __builtin_bit_cast(uint16_t, (half_t)a1);
}

// Standalone swiglu over f16 rows: gu [m][2I] -> h [m][I].  grid (ceil(I/256), m), block 256.
__global__ __launch_bounds__(256) void k_swiglu(const uint16_t* __restrict__ gu, int I,
                                                uint16_t* __restrict__ h) {
  const int i = blockIdx.x * 256 + threadIdx.x, row = blockIdx.y;
  if (i >= I) return;
  const uint16_t* g = gu + (size_t)row * 2 * I;
  h[(size_t)row * I + i] = __builtin_bit_cast(
      uint16_t, swiglu1(__builtin_bit_cast(half_t, g[i]), __builtin_bit_cast(half_t, g[I + i])));
}

// Weighted slot-order combine of already-transformed down outputs:
// y[t] = f16(sum_s f32(d16[t*k+s]) * f32(f16(score[t*k+s]))).  grid (ceil(H/256), T), block 256.
__global__ __launch_bounds__(256) void k_combine(const uint16_t* __restrict__ d16,
                                                 const float* __restrict__ scores, int top_k,
                                                 int H, uint16_t* __restrict__ y) {
  const int c = blockIdx.x * 256 + threadIdx.x, tok = blockIdx.y;
  if (c >= H) return;
  float a = 0.f;
  for (int s = 0; s < top_k; ++s) {
    const int row = tok * top_k + s;
    const float w = (float)(half_t)scores[row];
    a = a + (float)__builtin_bit_cast(half_t, d16[(size_t)row * H + c]) * w;
  }
  y[(size_t)tok * H + c] = __builtin_bit_cast(uint16_t, (half_t)a);
}

}  // namespace esc
