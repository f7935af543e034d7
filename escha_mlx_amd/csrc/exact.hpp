// Order-exact coded GEMV / row-blocked GEMM: the reference GPU kernels'
// float32 accumulation order reproduced bit-for-bit on wave64.
//
// Order (escha_mlx/msl.py:205-308; identical in the staged, row-blocked,
// direct-rows and fused-out kernels msl.py:389-435, 438-597, 688-872): for
// output column c of a tile and quarter p, the partial a_p walks kt ascending
// and adds x[16kt+r] * w[16kt+r][c] for r = 2p, 2p+1, 2p+8, 2p+9; the column
// is (a0 + a1) + (a2 + a3).  f16 x f16 products are exact in float32, so an
// fma and a multiply-then-add give the same bits; only the order matters.
//
// Wave64 mapping: one wave per 16-column tile, lane = 4c + p, so the xor-1
// then xor-2 shuffle reduction is exactly (a0 + a1) + (a2 + a3).  A block of
// 8 waves covers 128 output channels (one H128 block), which lets the fused
// output epilogue transform in-block as the reference's direct_out kernel does
// (msl.py:509-597).
#pragma once

#include "basic.hpp"

namespace esc {

enum RowMode { kDenseRows = 0, kMoeGroups = 1, kPerRow = 2 };

template <int K>
struct LaneWindow {
  int a0, a1, off0;
  __device__ __forceinline__ LaneWindow(int lane) {
    const int c = lane >> 2, p = lane & 3;
    const int L = 8 * ((c >> 1) & 3) + 4 * (c & 1) + p;  // reference 32-lane index
    const int t0 = 8 * L + ((c >= 8) ? 4 : 0);          // first of the lane's 4 steps
    const int start0 = (K * (t0 + 1) - 16 + 256 * K) % (256 * K);
    a0 = start0 >> 5;
    a1 = (a0 + 1) % (8 * K);
    off0 = start0 & 31;  // 4 windows span 3K+16 <= 25 bits: all inside {a0, a1}
  }
};

template <bool LUT>
__device__ __forceinline__ float dec_f32(uint32_t s, const uint16_t* lut) {
  if constexpr (LUT) return (float)__builtin_bit_cast(half_t, lut[s]);
  return (float)decode_hash(s);
}

template <bool LUT>
__device__ __forceinline__ void stage_lut(uint16_t* s_lut) {
  if constexpr (LUT) {
    copy_table(s_lut);
    __syncthreads();
  }
}

// Accumulate the block's R rows over all kt for one 16-column tile per wave.
// rows[r] < 0 marks a row that contributes nothing (its accumulator stays 0).
template <int K, bool LUT, int R>
__device__ __forceinline__ void exact_tile_chain(const uint32_t* __restrict__ base,
                                                 const uint16_t* __restrict__ xh, int IC,
                                                 int TK, int TN, int nt, const int* rows,
                                                 const uint16_t* lut, float* acc) {
  const int lane = threadIdx.x & 63;
  const int p = lane & 3;
  LaneWindow<K> lw(lane);
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  for (int kt = 0; kt < TK; ++kt) {
    const uint32_t* wp = base + ((size_t)kt * TN + nt) * (8 * K);
    const uint32_t hi = wp[lw.a0], lo = wp[lw.a1];
    float d[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) d[i] = dec_f32<LUT>(window16(hi, lo, lw.off0 + K * i), lut);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint16_t* xr = xh + (size_t)rows[r] * IC + 16 * kt + 2 * p;
      const float x0 = (float)__builtin_bit_cast(half_t, xr[0]);
      const float x1 = (float)__builtin_bit_cast(half_t, xr[1]);
      const float x8 = (float)__builtin_bit_cast(half_t, xr[8]);
      const float x9 = (float)__builtin_bit_cast(half_t, xr[9]);
      float a = acc[r];
      a = __builtin_fmaf(x0, d[0], a);
      a = __builtin_fmaf(x1, d[1], a);
      a = __builtin_fmaf(x8, d[2], a);
      a = __builtin_fmaf(x9, d[3], a);
      acc[r] = a;
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float a = acc[r];
    a = a + __shfl_xor(a, 1);
    a = a + __shfl_xor(a, 2);
    acc[r] = a;
  }
}

// Resolve the block's expert and its R source / destination rows.
template <int MODE, int R>
__device__ __forceinline__ bool exact_rows(int grp, int M, const int* __restrict__ idx_a,
                                           const int* __restrict__ idx_b, int* src, int* dst,
                                           int* expert) {
  if constexpr (MODE == kPerRow) {
    *expert = idx_a ? idx_a[grp] : 0;
    src[0] = dst[0] = grp;
    return true;
  } else if constexpr (MODE == kMoeGroups) {
    // idx_a = rows_idx [n_groups*R] (padding = M, the zero sink row),
    // idx_b = group_expert [n_groups] (-1 past the end): msl.py:688-872.
    const int e = idx_b[grp];
    if (e < 0) return false;
    *expert = e;
#pragma unroll
    for (int r = 0; r < R; ++r) src[r] = dst[r] = idx_a[grp * R + r];
    return true;
  } else {
    // dense: group grp owns rows [grp*R, grp*R+R); tail rows re-read row M-1
    // and are not stored (msl.py:780-799).
    if (grp * R >= M) return false;
    *expert = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = grp * R + r;
      src[r] = row < M ? row : M - 1;
      dst[r] = row < M ? row : -1;
    }
    return true;
  }
}

// mid[row][OC] f32.  grid (TN/8, n_groups), block 512 (8 waves = 128 columns).
template <int K, bool LUT, int R, int MODE>
__global__ __launch_bounds__(512) void k_gemm_exact(const uint16_t* __restrict__ xh,
                                                    const uint32_t* __restrict__ code,
                                                    const int* __restrict__ idx_a,
                                                    const int* __restrict__ idx_b, int M,
                                                    int TK, int TN, float* __restrict__ mid) {
  __shared__ uint16_t s_lut[LUT ? 65536 : 1];
  stage_lut<LUT>(s_lut);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nt = blockIdx.x * 8 + wave;
  const int IC = TK * 16, OC = TN * 16;
  int src[R], dst[R], e;
  if (!exact_rows<MODE, R>(blockIdx.y, M, idx_a, idx_b, src, dst, &e)) return;
  const uint32_t* base = code + (size_t)e * TK * TN * (8 * K);
  float acc[R];
  exact_tile_chain<K, LUT, R>(base, xh, IC, TK, TN, nt, src, s_lut, acc);
  if ((lane & 3) == 0) {
    const int col = 16 * nt + (lane >> 2);
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (dst[r] >= 0) mid[(size_t)dst[r] * OC + col] = acc[r];
  }
}

// Dense rows with the output transform fused in the epilogue:
// out = f16((H128(mid) * RS) * rout) for the block's 128 channels
// (escha_mlx/msl.py:509-597).  grid (TN/8, ceil(M/R)), block 512.
template <int K, bool LUT, int R>
__global__ __launch_bounds__(512) void k_gemm_exact_out(const uint16_t* __restrict__ xh,
                                                        const uint32_t* __restrict__ code,
                                                        const float* __restrict__ rout, int M,
                                                        int TK, int TN, float rs,
                                                        uint16_t* __restrict__ out) {
  __shared__ uint16_t s_lut[LUT ? 65536 : 1];
  __shared__ float s_mid[R][128];
  stage_lut<LUT>(s_lut);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nt = blockIdx.x * 8 + wave;
  const int IC = TK * 16, OC = TN * 16;
  int src[R], dst[R], e;
  if (!exact_rows<kDenseRows, R>(blockIdx.y, M, nullptr, nullptr, src, dst, &e)) return;
  float acc[R];
  exact_tile_chain<K, LUT, R>(code, xh, IC, TK, TN, nt, src, s_lut, acc);
  if ((lane & 3) == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) s_mid[r][16 * wave + (lane >> 2)] = acc[r];
  }
  __syncthreads();
  for (int r = wave; r < R; r += 8) {
    if (dst[r] < 0) continue;
    float v0 = s_mid[r][2 * lane], v1 = s_mid[r][2 * lane + 1];
    h128_wave(v0, v1);
    const int c = blockIdx.x * 128 + 2 * lane;
    const size_t o = (size_t)dst[r] * OC + c;
    out[o] = __builtin_bit_cast(uint16_t, to_f16((v0 * rs) * rout[c]));
    out[o + 1] = __builtin_bit_cast(uint16_t, to_f16((v1 * rs) * rout[c + 1]));
  }
}

}  // namespace esc
