// Routed-expert path kernels (EschaSparseMoeBlock._expert_path,
// escha_mlx/models/qwen3_5_moe.py:207-253).  Rows are token-major: slot s of
// token t is row t*top_k + s (models/qwen3_5_moe.py:97-101), so a token's
// contributions are rows [t*k, t*k+k) and combine in fixed slot order.
#pragma once

#include "fast.hpp"

namespace esc {

// xh[row] = f16(H128(f32(x[row / k]) * rin[ids[row]]) * RS).  grid (H/128, T*k), block 64.
__global__ __launch_bounds__(64) void k_moe_input(const uint16_t* __restrict__ x,
                                                  const int* __restrict__ ids, int top_k,
                                                  const float* __restrict__ rin, int H, float rs,
                                                  uint16_t* __restrict__ xh) {
  const int blk = blockIdx.x, row = blockIdx.y, lane = threadIdx.x;
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

// h = f16(f16(silu(g)) * u) with silu(g) = g / (1 + exp(-g)) in float32
// (escha_mlx/ref.py:296-301).
__device__ __forceinline__ half_t swiglu1(half_t g, half_t u) {
  const float gf = (float)g;
  const half_t s16 = to_f16(gf / (1.0f + expf(-gf)));
  return to_f16((float)s16 * (float)u);
}

// One 128-block of the gate_up output of one row, from split-K partials:
// f16((H128(sum_z part) * RS) * rout[e]) for the lane's two elements.
__device__ __forceinline__ void gu_block(const float* __restrict__ part, int S, int M, int OC,
                                         int row, int blk, const float* __restrict__ rout_e,
                                         float rs, half_t& y0, half_t& y1) {
  const int lane = threadIdx.x & 63;
  const int c = blk * 128 + 2 * lane;
  float v0 = 0.f, v1 = 0.f;
  // loads issued 8 at a time so their latencies overlap; summed in z order
  for (int z0 = 0; z0 < S; z0 += 8) {
    float2 pv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (z0 + j < S)
        pv[j] = *reinterpret_cast<const float2*>(part + ((size_t)(z0 + j) * M + row) * OC + c);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (z0 + j < S) {
        v0 = v0 + pv[j].x;
        v1 = v1 + pv[j].y;
      }
  }
  h128_wave(v0, v1);
  y0 = to_f16((v0 * rs) * rout_e[c]);
  y1 = to_f16((v1 * rs) * rout_e[c + 1]);
}

// gate_up epilogue -> swiglu -> down input transform, one wave per
// (row, 128-block of the intermediate): grid (I/128, M), block 64.
__global__ __launch_bounds__(64) void k_moe_mid(const float* __restrict__ part, int S, int M,
                                                int I, const int* __restrict__ ids,
                                                const float* __restrict__ gu_rout,
                                                const float* __restrict__ dn_rin, float rs,
                                                uint16_t* __restrict__ xh2) {
  const int b = blockIdx.x, row = blockIdx.y, lane = threadIdx.x;
  const int e = ids[row];
  const int OC = 2 * I;
  const float* ro = gu_rout + (size_t)e * OC;
  half_t g0, g1, u0, u1;
  gu_block(part, S, M, OC, row, b, ro, rs, g0, g1);
  gu_block(part, S, M, OC, row, b + I / 128, ro, rs, u0, u1);
  const half_t h0 = swiglu1(g0, u0), h1 = swiglu1(g1, u1);
  const int c = b * 128 + 2 * lane;
  const float* ri = dn_rin + (size_t)e * I + c;
  float v0 = (float)h0 * ri[0];
  float v1 = (float)h1 * ri[1];
  h128_wave(v0, v1);
  uint16_t* o = xh2 + (size_t)row * I + c;
  o[0] = __builtin_bit_cast(uint16_t, to_f16(v0 * rs));
  o[1] = __builtin_bit_cast(uint16_t, to_f16(v1 * rs));
}

// down epilogue + weighted combine: y[t] = f16(sum_s f32(d16[t*k+s]) * f32(f16(score)))
// summed in slot order in float32 (models/qwen3_5_moe.py:227-253).
// grid (H/128, T), block 64.
__global__ __launch_bounds__(64) void k_moe_combine(const float* __restrict__ part, int S,
                                                    int M, int H, const int* __restrict__ ids,
                                                    const float* __restrict__ scores, int top_k,
                                                    const float* __restrict__ dn_rout, float rs,
                                                    uint16_t* __restrict__ y) {
  const int blk = blockIdx.x, tok = blockIdx.y, lane = threadIdx.x;
  const int c = blk * 128 + 2 * lane;
  float a0 = 0.f, a1 = 0.f;
  for (int s = 0; s < top_k; ++s) {
    const int row = tok * top_k + s, e = ids[row];
    half_t d0, d1;
    gu_block(part, S, M, H, row, blk, dn_rout + (size_t)e * H, rs, d0, d1);
    const float w = (float)(half_t)scores[row];
    a0 = a0 + (float)d0 * w;
    a1 = a1 + (float)d1 * w;
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
