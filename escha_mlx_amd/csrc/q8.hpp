// Dense int8 / f16 GEMV around the routed experts: the w8a16 linears of the
// shared expert and the vocabulary head (escha_mlx/quant.py:1-30, contract
// wf = f16(f32(w8) * f32(scale)), y = f16(f32-accumulated x @ wf^T); CPU
// statement ref.w8a16, escha_mlx/ref.py:308-311), and the f16 router /
// shared-expert gates (y = f16(x @ w^T), escha_mlx/models/qwen3_5_moe.py:257-273).
//
// Weights are [O][K] row-major (one output channel per row), read once from
// HBM with 16-byte loads: LPR lanes share a row (the chunk count rounded up to
// a power of two, at most 64), each owning up to CPL 16-byte chunks of it, so
// a wave-step covers 64/LPR rows.  The
// lane's inputs for its chunks (NR rows of x) stay in VGPRs for the whole
// launch; the rows' partial sums meet through lane exchanges (DPP / permlane).
// Each weight is rounded exactly as the contract says (int8 -> f32, one fma
// with the row scale, RNE to f16) before the f16 x f16 products, which
// v_dot2c_f32_f16 sums in float32 (tolerance contract: reassociated sum).
#pragma once

#include "basic.hpp"
#include "fast.hpp"

namespace esc {

// partial sum of the lanes of one row group (LPR lanes, LPR a power of two)
template <int LPR>
__device__ __forceinline__ float row_sum(float v) {
  if constexpr (LPR >= 2) v = v + lane_xor<1>(v);
  if constexpr (LPR >= 4) v = v + lane_xor<2>(v);
  if constexpr (LPR >= 8) v = v + lane_xor<4>(v);
  if constexpr (LPR >= 16) v = v + lane_xor<8>(v);
  if constexpr (LPR >= 32) {
    const unsigned x = __builtin_bit_cast(unsigned, v);
    const auto p = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    const unsigned lo = p[0], hi = p[1];
    v = __builtin_bit_cast(float, lo) + __builtin_bit_cast(float, hi);
  }
  if constexpr (LPR >= 64) {
    const unsigned x = __builtin_bit_cast(unsigned, v);
    const auto p = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    const unsigned lo = p[0], hi = p[1];
    v = __builtin_bit_cast(float, lo) + __builtin_bit_cast(float, hi);
  }
  return v;
}

// 4 int8 weights (one word) -> two packed f16 pairs per the w8a16 contract:
// f32(w8) * f32(scale), RNE to f16.  q = w8 ^ 0x80 is the unsigned byte w8 + 128,
// and fma(q, s, -128 s) rounds the exact (q - 128) * s once, as the product does.
__device__ __forceinline__ void w8_to_f16x4(uint32_t w, float s, float ms, uint32_t& p0,
                                            uint32_t& p1) {
  const uint32_t q = w ^ 0x80808080u;
  const float f0 = __builtin_fmaf((float)(q & 0xFFu), s, ms);
  const float f1 = __builtin_fmaf((float)((q >> 8) & 0xFFu), s, ms);
  const float f2 = __builtin_fmaf((float)((q >> 16) & 0xFFu), s, ms);
  const float f3 = __builtin_fmaf((float)(q >> 24), s, ms);
  p0 = pack2(to_f16(f0), to_f16(f1));
  p1 = pack2(to_f16(f2), to_f16(f3));
}

// y[m][o] (ldy between rows) for m < M <= NR.  Q8: w is int8 [O][K] with
// scale [O]; otherwise w is f16 [O][K] and scale unused.  The row's `chunks`
// 16-byte pieces are spread over LPR lanes x CPL pieces each.  A lane's piece
// sub + LPR*j beyond the row (chunks not a multiple of LPR) has zero inputs
// and reads the row's last piece instead, so every weight load stays
// unconditional; int8 weights convert to finite values, whose products with
// the zero inputs add +0, while f16 weights (which may hold Inf) are replaced
// by zeros.  grid: any; block 256.
template <bool Q8, int NR, int LPR, int CPL>
__global__ __launch_bounds__(256) void k_rows_gemv(const uint16_t* __restrict__ x,
                                                   const void* __restrict__ wv,
                                                   const float* __restrict__ scale, int M, int K,
                                                   int O, uint16_t* __restrict__ y, int ldy) {
  constexpr int RPS = 64 / LPR;                  // rows per wave-step
  constexpr int WB = Q8 ? 1 : 2;                 // bytes per weight
  constexpr int CW = 16 / WB;                    // weights per 16-byte chunk
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int sub = lane % LPR, rsel = lane / LPR;
  const int chunks = K / CW;
  bool has[CPL];
  int coff[CPL];  // byte offset of the lane's piece j within a weight row
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    has[j] = sub + LPR * j < chunks;
    coff[j] = min(sub + LPR * j, chunks - 1) * 16;
  }
  // the lane's inputs: NR rows x CPL chunks x CW halves, as f16 pairs
  uint32_t xr[NR][CPL][CW / 2];
#pragma unroll
  for (int m = 0; m < NR; ++m)
#pragma unroll
    for (int j = 0; j < CPL; ++j)
#pragma unroll
      for (int i = 0; i < CW / 2; ++i) xr[m][j][i] = 0u;
#pragma unroll
  for (int m = 0; m < NR; ++m) {
    if (m >= M) break;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      if (!has[j]) continue;
      const uint16_t* xp = x + (size_t)m * K + (size_t)(sub + LPR * j) * CW;
#pragma unroll
      for (int i = 0; i < CW / 8; ++i) {
        const uint4 v = *reinterpret_cast<const uint4*>(xp + 8 * i);
        xr[m][j][4 * i] = v.x;
        xr[m][j][4 * i + 1] = v.y;
        xr[m][j][4 * i + 2] = v.z;
        xr[m][j][4 * i + 3] = v.w;
      }
    }
  }
  const uint8_t* w8 = reinterpret_cast<const uint8_t*>(wv);
  const int nwaves = gridDim.x * 4;
  const int steps = (O + RPS - 1) / RPS;
  // the weights (and scale) of the wave's next step are requested before the
  // current step is converted and multiplied
  auto load_step = [&](int st, uint4* wc, float& s) {
    const int oc = min(st * RPS + rsel, O - 1);  // in-bounds reads for a partial last step
    const uint8_t* row = w8 + (size_t)oc * K * WB;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      wc[j] = *reinterpret_cast<const uint4*>(row + coff[j]);
      if constexpr (!Q8)
        if (!has[j]) wc[j] = make_uint4(0u, 0u, 0u, 0u);
    }
    if constexpr (Q8) s = scale[oc];
  };
  int st = blockIdx.x * 4 + wave;
  uint4 wn[CPL];
  float sn = 0.f;
  if (st < steps) load_step(st, wn, sn);
  for (; st < steps; st += nwaves) {
    const int o = st * RPS + rsel;
    const bool ok = o < O;
    uint4 wc[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) wc[j] = wn[j];
    const float s = sn, ms = -128.f * sn;
    if (st + nwaves < steps) load_step(st + nwaves, wn, sn);
    float acc[NR];
#pragma unroll
    for (int m = 0; m < NR; ++m) acc[m] = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const uint32_t ww[4] = {wc[j].x, wc[j].y, wc[j].z, wc[j].w};
      uint32_t wp[CW / 2];
      if constexpr (Q8) {
#pragma unroll
        for (int i = 0; i < 4; ++i) w8_to_f16x4(ww[i], s, ms, wp[2 * i], wp[2 * i + 1]);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) wp[i] = ww[i];
      }
#pragma unroll
      for (int m = 0; m < NR; ++m)
#pragma unroll
        for (int i = 0; i < CW / 2; ++i) acc[m] = dot2(xr[m][j][i], wp[i], acc[m]);
    }
#pragma unroll
    for (int m = 0; m < NR; ++m) acc[m] = row_sum<LPR>(acc[m]);
    if (ok && sub == 0) {
#pragma unroll
      for (int m = 0; m < NR; ++m)
        if (m < M) y[(size_t)m * ldy + o] = __builtin_bit_cast(uint16_t, to_f16(acc[m]));
    }
  }
}

// w8a16 GEMV for 2..16 rows of x on the matrix core: y[m][o] = f16(sum_k
// x[m][k] * wf[o][k]), wf = f16(f32(w8) * scale[o]) (the contract rounding, as
// k_rows_gemv).  A wave owns 16 output channels at a time and walks all of K in
// steps of 64: lane l reads 16 int8 of channel o0 + l % 16 at k0 + 16 (l / 16),
// converts them, and the two halves are the A operands of two
// v_mfma_f32_16x16x32_f16 (A slot 8g + t <-> k0 + 16g + t, second half +8);
// the B operands are the same k of token l % 16 from x staged in LDS (rows at a
// 16-byte-padded pitch, so the 16 tokens of a lane group hit different banks).
// Every product of a channel lands in one accumulator: no lane reduction.  D
// lane l: token l % 16, channels o0 + 4 (l / 16) + r.  K a multiple of 64;
// dynamic LDS = M x (2K + 16) bytes; grid: any; block 256.
__global__ __launch_bounds__(256) void k_rows_w8_mma(const uint16_t* __restrict__ x,
                                                     const int8_t* __restrict__ w8,
                                                     const float* __restrict__ scale, int M,
                                                     int K, int O, uint16_t* __restrict__ y,
                                                     int ldy) {
  extern __shared__ uint4 s_xm[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int pitch = K / 8 + 1;  // 16-byte units per staged row
  for (int i = threadIdx.x; i < M * (K / 8); i += 256) {
    const int r = i / (K / 8), c = i % (K / 8);
    s_xm[r * pitch + c] = *reinterpret_cast<const uint4*>(x + (size_t)r * K + 8 * c);
  }
  __syncthreads();
  const int j = lane & 15, g = lane >> 4;
  const uint4* xb = s_xm + (size_t)min(j, M - 1) * pitch + 2 * g;  // token j, k0 + 16g
  const int ngroups = (O + 15) / 16, nwaves = gridDim.x * 4;
  for (int grp = blockIdx.x * 4 + wave; grp < ngroups; grp += nwaves) {
    const int oc = min(grp * 16 + j, O - 1);  // in-bounds reads for a partial last group
    const float s = scale[oc], ms = -128.f * s;
    const uint4* wr = reinterpret_cast<const uint4*>(w8 + (size_t)oc * K + 16 * g);
    f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
    auto step = [&](const uint4 wc, int k0) {
      u32x4_t a0, a1;
      uint32_t p0, p1;
      w8_to_f16x4(wc.x, s, ms, p0, p1);
      a0[0] = p0;
      a0[1] = p1;
      w8_to_f16x4(wc.y, s, ms, p0, p1);
      a0[2] = p0;
      a0[3] = p1;
      w8_to_f16x4(wc.z, s, ms, p0, p1);
      a1[0] = p0;
      a1[1] = p1;
      w8_to_f16x4(wc.w, s, ms, p0, p1);
      a1[2] = p0;
      a1[3] = p1;
      const uint4 b0 = xb[k0 / 8], b1 = xb[k0 / 8 + 1];
      acc = mma16(a0, __builtin_bit_cast(u32x4_t, b0), acc);
      acc = mma16(a1, __builtin_bit_cast(u32x4_t, b1), acc);
    };
    // two 64-k steps per iteration, the next two requested before these are used
    uint4 n0 = wr[0], n1 = wr[K > 64 ? 4 : 0];
    for (int k0 = 0; k0 < K; k0 += 128) {
      const uint4 c0 = n0, c1 = n1;
      if (k0 + 128 < K) {
        n0 = wr[(k0 + 128) / 16];
        n1 = wr[(k0 + 192 < K ? k0 + 192 : k0 + 128) / 16];
      }
      step(c0, k0);
      if (k0 + 64 < K) step(c1, k0 + 64);
    }
    if (j < M) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int o = grp * 16 + 4 * g + r;
        if (o < O) y[(size_t)j * ldy + o] = __builtin_bit_cast(uint16_t, to_f16(acc[r]));
      }
    }
  }
}

// Embedding rows of an int8 table (escha_mlx/quant.py:253-266 under the w8a16
// contract): out[t][k] = f16(f32(w8[ids[t]][k]) * f32(scale[ids[t]])), the
// same rounding as the GEMV's weights.  An id outside [0, N) yields a row of
// f16 NaN (0x7E00) instead of a read outside the table.  K a multiple of 16;
// grid (T), block 256, each thread converting 16-byte chunks of the row.
__global__ __launch_bounds__(256) void k_q8_embed(const int32_t* __restrict__ ids,
                                                  const int8_t* __restrict__ w8,
                                                  const float* __restrict__ scale, int N, int K,
                                                  uint16_t* __restrict__ out) {
  const int t = blockIdx.x;
  const int id = ids[t];
  const bool ok = id >= 0 && id < N;
  const float s = ok ? scale[id] : 0.f, ms = -128.f * s;
  uint4* dst = reinterpret_cast<uint4*>(out + (size_t)t * K);
  const uint4* src = reinterpret_cast<const uint4*>(w8 + (size_t)(ok ? id : 0) * K);
  for (int c = threadIdx.x; c < K / 16; c += 256) {
    uint32_t p[8];
    if (ok) {
      const uint4 v = src[c];
      w8_to_f16x4(v.x, s, ms, p[0], p[1]);
      w8_to_f16x4(v.y, s, ms, p[2], p[3]);
      w8_to_f16x4(v.z, s, ms, p[4], p[5]);
      w8_to_f16x4(v.w, s, ms, p[6], p[7]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) p[i] = 0x7E007E00u;
    }
    dst[2 * c] = make_uint4(p[0], p[1], p[2], p[3]);
    dst[2 * c + 1] = make_uint4(p[4], p[5], p[6], p[7]);
  }
}

// Shared-expert activation (escha_mlx/ref.py:345): hh = f16((g / (1 + exp(-g))) * u)
// in float32, g and u f16 [m][I].  grid (ceil(I/256), m), block 256.
__global__ __launch_bounds__(256) void k_shared_act(const uint16_t* __restrict__ g,
                                                    const uint16_t* __restrict__ u, int I,
                                                    uint16_t* __restrict__ hh) {
  const int i = blockIdx.x * 256 + threadIdx.x, row = blockIdx.y;
  if (i >= I) return;
  const size_t o = (size_t)row * I + i;
  const float gf = (float)__builtin_bit_cast(half_t, g[o]);
  const float uf = (float)__builtin_bit_cast(half_t, u[o]);
  hh[o] = __builtin_bit_cast(uint16_t, to_f16((gf / (1.0f + expf(-gf))) * uf));
}

// Block output (escha_mlx/ref.py:346-349, models/qwen3_5_moe.py:270-272):
// out = f16(f32(y) + f32(sh) * sigmoid(f32(shg))), y the f16 routed sum, sh
// the shared expert's f16 output, shg [m] the f16 shared gate logit.
// grid (ceil(H/256), m), block 256.
__global__ __launch_bounds__(256) void k_block_out(const uint16_t* __restrict__ yr,
                                                   const uint16_t* __restrict__ sh,
                                                   const uint16_t* __restrict__ shg, int H,
                                                   uint16_t* __restrict__ out) {
  const int c = blockIdx.x * 256 + threadIdx.x, row = blockIdx.y;
  if (c >= H) return;
  const size_t o = (size_t)row * H + c;
  const float sg = 1.0f / (1.0f + expf(-(float)__builtin_bit_cast(half_t, shg[row])));
  const float v = (float)__builtin_bit_cast(half_t, yr[o]) +
                  (float)__builtin_bit_cast(half_t, sh[o]) * sg;
  out[o] = __builtin_bit_cast(uint16_t, to_f16(v));
}

}  // namespace esc
