// One-launch coded linear for a few rows (M < 16): the whole of
// EschaLinear.__call__ (escha_mlx/dense.py:337-362) -- input transform, coded
// GEMV and output transform (+ optional bias) -- in a single kernel.
//
// grid (ceil(TN/TPW), ceil(M/R), S); block = 4 waves; block z owns kt range
// [z*KS, (z+1)*KS) with KS a multiple of 8, i.e. whole 128-input blocks:
//   1. the block input-transforms its own KS/8 blocks of x for its R rows
//      (one wave per (row, block)) into LDS, so no xh tensor is written;
//   2. decode + multiply as k_gemv_fast_rows (R rows share each decoded
//      weight), reduce the 4 waves in LDS, publish float32 partials
//      [S][M][OC] with device-coherent stores;
//   3. the last of the S blocks of a (row group, column group) -- found with
//      a device-scope counter that it resets to zero -- sums the S partials
//      in z order (one thread per column, 32 loads in flight at a time),
//      output-transforms each 128-column block and writes y.
// Deterministic (fixed summation order, no float atomics); tolerance
// contract like k_gemv_fast (reassociated float32 sum).
#pragma once

#include "fused.hpp"

namespace esc {

template <int K, bool LUT, int R>
__global__ __launch_bounds__(256) void k_linear_small(
    const uint16_t* __restrict__ x, const float* __restrict__ rin,
    const uint32_t* __restrict__ code, const float* __restrict__ rout,
    const uint16_t* __restrict__ bias, int M, int TK, int TN, int KS, float rs,
    float* __restrict__ part, int* __restrict__ cnt, uint16_t* __restrict__ y) {
  using G = Geo<K>;
  __shared__ uint16_t s_lut[LUT ? 65536 : 1];
  __shared__ float s_red[4][64][G::NCOL];
  __shared__ uint32_t s_x[R][8 * 64];  // up to 64 kt of inputs per row
  __shared__ int s_last;
  stage_lut<LUT>(s_lut);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int ntg = blockIdx.x, row0 = blockIdx.y * R, z = blockIdx.z, S = gridDim.z;
  const int IC = TK * 16, OC = TN * 16;
  const int nb = KS / 8;  // 128-input blocks of the block's kt range
  // the first kt step's code is requested before anything else, so its
  // latency overlaps the input transform
  const int q = lane % G::LPT, tile = lane / G::LPT;
  const int src = tile * G::LPT + (q + G::LPT - 1) % G::LPT;
  const bool valid = ntg * G::TPW + tile < TN;
  const int KW = KS / 4;
  const int kl0 = wave * KW, kt0 = z * KS + kl0;
  const size_t lane_off = (size_t)ntg * G::TPW * (8 * K) + (size_t)lane * G::WPL;
  LaneWords<K> zero{};
  LaneWords<K> cur = valid ? load_lane_words<K>(code + (size_t)kt0 * TN * (8 * K) + lane_off) : zero;
  // 1. input transform: xh = f16(H128(f32(x) * rin) * RS) per (row, block)
  for (int it = wave; it < R * nb; it += 4) {
    const int r = it / nb, b = it % nb;
    const int row = min(row0 + r, M - 1);
    const int c = 16 * KS * z + 128 * b + 2 * lane;
    float v0 = (float)__builtin_bit_cast(half_t, x[(size_t)row * IC + c]) * rin[c];
    float v1 = (float)__builtin_bit_cast(half_t, x[(size_t)row * IC + c + 1]) * rin[c + 1];
    h128_wave(v0, v1);
    s_x[r][64 * b + lane] = pack2(to_f16(v0 * rs), to_f16(v1 * rs));
  }
  __syncthreads();
  // 2. decode + multiply the block's tiles over its kt range
  float acc[R][G::NCOL];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int i = 0; i < G::NCOL; ++i) acc[r][i] = 0.f;
  for (int k = 0; k < KW; ++k) {
    LaneWords<K> nxt = cur;
    if (valid && k + 1 < KW)
      nxt = load_lane_words<K>(code + (size_t)(kt0 + k + 1) * TN * (8 * K) + lane_off);
    uint32_t xp[R][8];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      uint32_t xw[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) xw[i] = s_x[r][8 * (kl0 + k) + i];
      x_pairs(xw, xp[r]);
    }
    const uint32_t wprev = __shfl(cur.w[G::WPL - 1], src);
    fast_tile_rows<K, LUT, R>(cur, wprev, xp, s_lut, acc);
    cur = nxt;
  }
  // reduce the 4 waves (fixed order) and publish the partials
#pragma unroll
  for (int r = 0; r < R; ++r) {
#pragma unroll
    for (int i = 0; i < G::NCOL; ++i) s_red[wave][lane][i] = acc[r][i];
    __syncthreads();
    if (wave == 0 && valid && row0 + r < M) {
      float* pr = part + ((size_t)z * M + row0 + r) * OC + (size_t)(ntg * G::TPW + tile) * 16;
#pragma unroll
      for (int i = 0; i < G::NCOL; ++i) {
        float v = s_red[0][lane][i];
        v = v + s_red[1][lane][i];
        v = v + s_red[2][lane][i];
        v = v + s_red[3][lane][i];
        st_coherent(pr + G::col(q, i), v);
      }
    }
    __syncthreads();
  }
  wait_vm();
  __syncthreads();
  // 3. the last split of (row group, column group) finishes the columns
  if (threadIdx.x == 0) {
    int* c = &cnt[(size_t)blockIdx.y * gridDim.x + ntg];
    const bool last = add_relaxed(c, 1) == S - 1;
    if (last) __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last;
  }
  __syncthreads();
  if (!s_last) return;
  // one thread per column: the splits' partials are requested 32 at a time,
  // summed in z order, and staged in LDS for the output transform
  constexpr int kCols = G::TPW * 16;          // columns per column group
  constexpr int kBlocks = kCols / 128;        // 128-column blocks per group
  float* s_sum = &s_red[0][0][0];             // [R][kCols] floats (<= 8 KiB needed)
  static_assert(sizeof(s_red) >= 2 * kCols * sizeof(float), "");
  const int col0 = ntg * kCols;
  for (int r0 = 0; r0 < R; r0 += 2) {         // two rows per pass fit s_red
    for (int rr = 0; rr < 2 && r0 + rr < R; ++rr) {
      const int row = min(row0 + r0 + rr, M - 1);
      const int j = threadIdx.x;
      if (j < kCols && col0 + j < OC) {
        const float* pb = part + (size_t)row * OC + col0 + j;
        float v = 0.f;
        for (int z0 = 0; z0 < S; z0 += 32) {
          float pv[32];
#pragma unroll
          for (int zz = 0; zz < 32; ++zz)
            if (z0 + zz < S)
              pv[zz] = __builtin_bit_cast(
                  float, __hip_atomic_load(
                             reinterpret_cast<const uint32_t*>(pb + (size_t)(z0 + zz) * M * OC),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
#pragma unroll
          for (int zz = 0; zz < 32; ++zz)
            if (z0 + zz < S) v = v + pv[zz];
        }
        s_sum[rr * kCols + j] = v;
      }
    }
    __syncthreads();
    for (int it = wave; it < 2 * kBlocks; it += 4) {
      const int rr = it / kBlocks, b = it % kBlocks, r = r0 + rr;
      const int col = col0 + 128 * b + 2 * lane;
      if (r >= R || row0 + r >= M || col >= OC) continue;
      float v0 = s_sum[rr * kCols + 128 * b + 2 * lane];
      float v1 = s_sum[rr * kCols + 128 * b + 2 * lane + 1];
      h128_wave(v0, v1);
      half_t y0 = to_f16((v0 * rs) * rout[col]);
      half_t y1 = to_f16((v1 * rs) * rout[col + 1]);
      if (bias) {
        y0 = to_f16((float)y0 + (float)__builtin_bit_cast(half_t, bias[col]));
        y1 = to_f16((float)y1 + (float)__builtin_bit_cast(half_t, bias[col + 1]));
      }
      uint16_t* yr = y + (size_t)(row0 + r) * OC + col;
      yr[0] = __builtin_bit_cast(uint16_t, y0);
      yr[1] = __builtin_bit_cast(uint16_t, y1);
    }
    __syncthreads();
  }
}

}  // namespace esc
