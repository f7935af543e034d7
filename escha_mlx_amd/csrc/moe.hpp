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
                                                   int* __restrict__ group_expert) {
  if (blockIdx.x == 0) {
    build_groups_block(ids, m, E, R, n_groups, rows_idx, group_expert);
    return;
  }
  const int nhb = H / 128, w = (blockIdx.x - 1) * 16 + (threadIdx.x >> 6);
  if (w < nhb * m) moe_input_wave(x, ids, top_k, rin, H, rs, xh, w % nhb, w / nhb);
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
