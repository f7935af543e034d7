// Decode-rate probe (measurement only; no counterpart in the reference): the
// K=2 decode + dot2 loop of the expert GEMVs streamed over a large code buffer
// by persistent workgroups, with NT of every 8 step pairs decoded from the
// 65,536-entry table in LDS and the rest by hash.  It bounds what any
// kernel built on this decode can reach: weights per CU-clock for the hash
// alone, the table alone and their mixes, at a given number of waves per CU.
//
// The decode is fast_tile_mix (fast.hpp).
#pragma once

#include "fast.hpp"

namespace esc {

// grid: CUs x (WPC / 16) workgroups of 1024 threads; each wave streams
// `steps` consecutive wave-steps (1 KiB of code each) of its own code range,
// PF steps ahead (PF loads in flight per wave; steps a multiple of 4).
template <int NT, int PF>
__global__ __launch_bounds__(1024) void k_decode_probe(const uint32_t* __restrict__ code,
                                                       int steps, float* __restrict__ out) {
  static_assert(PF >= 1 && PF <= 3, "prefetch depth");
  extern __shared__ uint16_t s_tab[];
  if constexpr (NT > 0) {
    const uint4* src = reinterpret_cast<const uint4*>(g_lut);
    uint4* dst = reinterpret_cast<uint4*>(s_tab);
    for (int i = threadIdx.x; i < 65536 / 8; i += blockDim.x) dst[i] = src[i];
    __syncthreads();
  }
  const uint32_t tb = (uint32_t)(size_t)s_tab;  // LDS byte address of the table
  const int lane = threadIdx.x & 63;
  const size_t gw = (size_t)blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6);
  const uint32_t* lp = code + (gw * steps * 64 + lane) * 4;
  uint32_t xp[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) xp[j] = 0x3C003C00u ^ (j * 0x00100010u);
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  // ring of 4 steps: step k sits in w[k % 4]; step k + PF is requested
  // before step k is decoded
  LaneWords<2> w[4];
#pragma unroll
  for (int j = 0; j < PF; ++j) w[j] = load_lane_words<2>(lp + (size_t)j * 256);
  for (int k0 = 0; k0 < steps; k0 += 4) {
    // issue priority from the quarter of the range left, as in the item
    // kernels (otherwise the oldest wave of a SIMD runs ahead and the last
    // ones finish alone)
    {
      const int q4 = 4 * (steps - k0) / steps;
      if (q4 >= 3) __builtin_amdgcn_s_setprio(3);
      else if (q4 == 2) __builtin_amdgcn_s_setprio(2);
      else if (q4 == 1) __builtin_amdgcn_s_setprio(1);
      else __builtin_amdgcn_s_setprio(0);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = k0 + j;
      // past the end: the last step again (in bounds, unused)
      const int kn = k + PF < steps ? k + PF : steps - 1;
      w[(j + PF) & 3] = load_lane_words<2>(lp + (size_t)kn * 256);
      fast_tile_mix<NT>(w[j], quad_prev_word(w[j].w[3]), xp, acc, tb);
      __builtin_amdgcn_sched_barrier(0);  // one step at a time (register pressure)
    }
  }
  out[gw * 64 + lane] = acc[0] + acc[1] + acc[2] + acc[3];
}

}  // namespace esc
