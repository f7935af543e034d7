// Coded projections at batch 1 (M = 1): one to four EschaLinear.__call__
// (escha_mlx/dense.py:337-362) of one input row each -- input transform,
// coded GEMV, output transform (+ bias) -- in one launch of persistent
// workgroups (16 waves, one per CU when the decode table is staged).
//
// Work unit: one kt (16 inputs) of one column group (16 tiles = 256 output
// columns) of one projection: 1 KiB of K=2 code (one wave-step) or 1.5 KiB of
// K=3 code (two wave-steps of 8 tiles).  A projection's units are ordered
// (column group, kt); its G workgroups split them evenly (workgroup k:
// [k n / G, (k + 1) n / G), rounded down) and each splits its range evenly
// over its 16 waves, so every wave runs one run of consecutive units -- the
// code of consecutive kt of one column group, one unit's load in flight while
// the previous one decodes.  With at most 8 units per wave a range touches at
// most two 128-input blocks and at most two column groups, so the wave
// input-transforms both blocks once at its start and keeps at most two
// partial sums in registers.  Each projection has its own workgroups and
// partials; a single launch chooses G from the projection's own shape, so its
// outputs do not depend on what else shares the launch.
//
// With the table (NT > 0; staged in LDS once per workgroup) NT of every 8
// step pairs are decoded from it and the rest by hash (fast_tile_mix for K=2,
// fast_tile_mix3 for K=3); NT = 0 decodes by hash.  Reduction, in a fixed
// order (deterministic, no float atomics):
//   1. every wave's partial of each group it touched goes to LDS; the
//      workgroup sums them in wave order, one wave per group, and publishes
//      one float32 partial per (workgroup, group) with agent-scope stores;
//   2. the last workgroup to publish for a group (device-scope counter, which
//      it resets) sums the group's partials in workgroup order,
//      output-transforms its two 128-column blocks and writes y.
#pragma once

#include "layers.hpp"

namespace esc {

constexpr int kProjWaves = 16;  // waves per workgroup
constexpr int kProjMaxP = 8;    // units per wave
constexpr int kProjMax = 4;     // projections per launch
constexpr int kProjGroupCols = 256;
// units each wave decodes by hash before the table barrier (measured on
// MI355X, config 2 at batch 1: 1 beats 2 and 3)
constexpr int kProjHashUnits = 1;

// One projection of the launch.
struct ProjOne {
  const uint16_t* x;     // [IC] f16 input row
  const float* rin;      // [IC]
  const uint32_t* code;  // [TK][TN][8K]
  const float* rout;     // [OC]
  const uint16_t* bias;  // [OC] f16 or null
  uint16_t* y;           // [OC] f16
  float* part;           // [TN/16][maxc][256] float32 partials, lane-major
  int* cnt;              // [TN/16] workgroups published per group (zero between calls)
  int TK, TN;            // IC / 16, OC / 16 (TN a multiple of 16)
  int n;                 // units: (TN / 16) TK
  int G;                 // workgroups (at most kProjMaxP units per wave)
  int maxc;              // partial slots per group (>= the workgroups a group spans)
  int wg0;               // first workgroup of this projection in the launch
};

struct ProjArgs {
  ProjOne pr[kProjMax];
  int np;    // projections
  float rs;  // the transforms' scale
};

// LDS of the kernel beyond the table: each wave's partials of its two
// groups (phase 1 -> 2) and the finishers' column sums; both live in the
// table's space once every wave has finished decoding.
constexpr int kProjLdsWork = (kProjWaves * 2 * 256 + kProjWaves * 256) * 4;

// unit -> (column group, kt)
struct ProjUnit {
  int g, kt;
};
__device__ __forceinline__ ProjUnit proj_unit(const ProjOne& q, int u) {
  return ProjUnit{u / q.TK, u % q.TK};
}
// first unit of workgroup k, and the workgroup that holds unit u
__device__ __forceinline__ int proj_wg_start(const ProjOne& q, int k) {
  return (int)((long)k * q.n / q.G);
}
__device__ __forceinline__ int proj_wg_of(const ProjOne& q, int u) {
  return (int)(((long)(u + 1) * q.G - 1) / q.n);
}

// the first wave-step's words of unit (g, kt)
template <int K>
__device__ __forceinline__ const uint32_t* proj_code(const ProjOne& q, const ProjUnit& c) {
  return q.code + ((size_t)c.kt * q.TN + 16 * c.g) * (8 * K);
}

// the lane's two inputs of block kb and their input scales
struct ProjIn {
  uint32_t xw;
  float2 ri;
};
__device__ __forceinline__ ProjIn proj_fetch(const ProjOne& q, int kb) {
  const int lane = threadIdx.x & 63;
  return ProjIn{*reinterpret_cast<const uint32_t*>(q.x + 128 * kb + 2 * lane),
                *reinterpret_cast<const float2*>(q.rin + 128 * kb + 2 * lane)};
}
// the block's 128 inputs, f16(H128(x * rin) * rs), as the decode's paired
// words (lane j: word j)
__device__ __forceinline__ uint32_t proj_inputs(const ProjIn& in, float rs) {
  float v0 = (float)__builtin_bit_cast(half_t, (uint16_t)in.xw) * in.ri.x;
  float v1 = (float)__builtin_bit_cast(half_t, (uint16_t)(in.xw >> 16)) * in.ri.y;
  h128_wave(v0, v1);
  return paired_word(pack2(to_f16(v0 * rs), to_f16(v1 * rs)));
}

// One unit: decode + multiply, inputs lanes j0 .. j0+7 of xv.  acc: 4 floats
// per lane (K=2: Geo<2> slots; K=3: slots 0-1 first 8 tiles, 2-3 last 8).
// The table (NT > 0) is at LDS byte address tb, also as the pointer lut.
template <int K, int NT>
__device__ __forceinline__ void proj_step(const LaneWords<K>* w, uint32_t xv, int j0, uint32_t tb,
                                          const uint16_t* lut, float* acc) {
  uint32_t xp[1][8];
#pragma unroll
  for (int j = 0; j < 8; ++j) xp[0][j] = __builtin_amdgcn_readlane(xv, j0 + j);
  if constexpr (K == 2) {
    fast_tile_mix<NT>(w[0], quad_prev_word(w[0].w[3]), xp[0], acc, tb);
  } else {
    const int lane = threadIdx.x & 63;
    const int src = (lane & ~7) | ((lane + 7) & 7);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t wprev = __shfl(w[h].w[2], src);
      if constexpr (NT > 0)
        fast_tile_mix3<NT>(w[h], wprev, xp[0], acc + 2 * h, tb);
      else
        fast_tile_rows<3, false, 1>(w[h], wprev, xp, nullptr,
                                    reinterpret_cast<float(*)[2]>(acc + 2 * h));
    }
  }
}

template <int K>
__device__ __forceinline__ void proj_load(const uint32_t* base, size_t half_off, uint32_t off,
                                          LaneWords<K>* w) {
  w[0] = load_lane_words_nt<K>(base + off);
  if constexpr (K == 3) w[1] = load_lane_words_nt<K>(base + half_off + off);
}

// output column (0..255 of the group) of the lane's accumulator slot ci
template <int K>
__device__ __forceinline__ int proj_col(int lane, int ci) {
  if constexpr (K == 2) return 16 * (lane >> 2) + Geo<2>::col(lane & 3, ci);
  return 128 * (ci >> 1) + 16 * (lane >> 3) + Geo<3>::col(lane & 7, ci & 1);
}

// grid: the projections' workgroups one after the other (projection j's
// from pr[j].wg0), 16 waves each; dynamic LDS: the table (NT > 0) or
// kProjLdsWork bytes.
template <int K, int NT>
__global__ __launch_bounds__(64 * kProjWaves) void k_proj_rows1(ProjArgs p) {
  extern __shared__ uint16_t s_dyn[];
  __shared__ int s_grp[kProjWaves][2];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  ProjOne q = p.pr[0];
#pragma unroll
  for (int i = 1; i < kProjMax; ++i)
    if (i < p.np && (int)blockIdx.x >= p.pr[i].wg0) q = p.pr[i];
  const int wg = blockIdx.x - q.wg0;
  const int wa = proj_wg_start(q, wg), wlen = proj_wg_start(q, wg + 1) - wa;
  const int a = wa + wave * wlen / kProjWaves, b = wa + (wave + 1) * wlen / kProjWaves;
  const bool busy = a < b;
  // per lane: K=2 16 consecutive tiles x 4 words; K=3 8 tiles x 3 words, twice
  const uint32_t off = (uint32_t)(lane * Geo<K>::WPL);
  const size_t half_off = (size_t)8 * 8 * K;  // K=3: the next 8 tiles

  // this wave's first unit and its inputs, then the table's pieces (LDS DMA),
  // are requested before anything waits
  ProjUnit c = proj_unit(q, busy ? a : 0);
  const ProjUnit cl = proj_unit(q, busy ? b - 1 : 0);
  LaneWords<K> w[K == 3 ? 2 : 1];
  proj_load<K>(proj_code<K>(q, c), half_off, off, w);
  const bool two_blocks = cl.g != c.g || (cl.kt >> 3) != (c.kt >> 3);
  const ProjIn ina = proj_fetch(q, c.kt >> 3), inb = proj_fetch(q, cl.kt >> 3);
  // units [a, ub) use block A, [ub, b) block B; [a, ug) group c.g, [ug, b) cl.g
  const int ub = two_blocks ? b - 1 - (cl.kt & 7) : b;
  const int ug = cl.g != c.g ? b - 1 - cl.kt : b;
  if (lane == 0) {
    s_grp[wave][0] = busy ? c.g : -1;
    s_grp[wave][1] = busy && ug < b ? cl.g : -1;
  }

  const uint32_t xa = proj_inputs(ina, p.rs);
  const uint32_t xb = two_blocks ? proj_inputs(inb, p.rs) : xa;
  if constexpr (NT > 0) {
    // The table's pieces are requested once the first unit's code and the
    // inputs are in registers (the compiler waits for every outstanding load
    // after a DMA into LDS, so a wait placed later would also wait for the
    // table), and land while the first unit decodes.
#pragma unroll
    for (int h = 0; h < (K == 3 ? 2 : 1); ++h)
#pragma unroll
      for (int j = 0; j < Geo<K>::WPL; ++j) __asm__ volatile("" : : "v"(w[h].w[j]));
    table_dma(s_dyn);
  }

  float acc[4] = {0.f, 0.f, 0.f, 0.f}, accA[4] = {0.f, 0.f, 0.f, 0.f};
  // unit u: the next unit's code requested (this one again at the end: in
  // bounds, unused), decode + multiply (table pairs from LDS when TAB), and
  // the partial of group c.g set aside when that group ends inside the range
  auto unit = [&](int u, auto tab, uint32_t tbu) {
    ProjUnit cn = c;
    if (u + 1 < b && ++cn.kt == q.TK) {
      cn.kt = 0;
      ++cn.g;
    }
    LaneWords<K> wn[K == 3 ? 2 : 1];
    proj_load<K>(proj_code<K>(q, cn), half_off, off, wn);
    proj_step<K, decltype(tab)::value>(w, u < ub ? xa : xb, 8 * (c.kt & 7), tbu, s_dyn, acc);
    if (u + 1 == ug && ug < b) {  // group c.g ends inside the range
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        accA[i] = acc[i];
        acc[i] = 0.f;
      }
    }
#pragma unroll
    for (int h = 0; h < (K == 3 ? 2 : 1); ++h) w[h] = wn[h];
    c = cn;
  };
  // the first units are decoded by hash before the table is in LDS, so their
  // decode runs while the table's pieces are still arriving (the table is
  // the hash's image and the step order is the same: bit-identical)
  const int uh = NT > 0 ? min(b, a + kProjHashUnits) : a;
#pragma unroll 1
  for (int u = a; u < uh; ++u) {
    prio_left(b - u);
    unit(u, std::integral_constant<int, 0>{}, 0u);
  }
  uint32_t tb = 0;
  if constexpr (NT > 0) {
    wait_vm();  // this wave's table pieces are in LDS
    tb = (uint32_t)(size_t)s_dyn;
  }
  __syncthreads();

  if (busy) {
#pragma unroll 1
    for (int u = uh; u < b; ++u) {
      prio_left(b - u);
      unit(u, std::integral_constant<int, NT>{}, tb);
    }
  }
  // every wave has finished decoding: the table's space holds the partials
  __syncthreads();
  float* s_wp = reinterpret_cast<float*>(s_dyn);             // [16][2][64][4]
  float* s_fin = s_wp + kProjWaves * 2 * 256 + wave * 256;  // [256] this wave's
  if (busy) {
    const bool split = ug < b;
    float* d0 = s_wp + (wave * 2) * 256 + 4 * lane;
    const float* first = split ? accA : acc;
    *reinterpret_cast<float4*>(d0) = make_float4(first[0], first[1], first[2], first[3]);
    if (split) *reinterpret_cast<float4*>(d0 + 256) = make_float4(acc[0], acc[1], acc[2], acc[3]);
  }
  __syncthreads();

  // 2. one wave per group of this workgroup: the waves' partials in wave order
  if (wlen == 0) return;
  const int gfirst = wa / q.TK, glast = (wa + wlen - 1) / q.TK;
  for (int g = gfirst + wave; g <= glast; g += kProjWaves) {
    // the group's output scales and bias, requested before the hand-off so
    // that the finisher does not wait on them
    const int col0 = kProjGroupCols * g;
    float2 ro[2];
    uint32_t bw[2] = {0u, 0u};
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      ro[blk] = *reinterpret_cast<const float2*>(q.rout + col0 + 128 * blk + 2 * lane);
      if (q.bias) bw[blk] = *reinterpret_cast<const uint32_t*>(q.bias + col0 + 128 * blk + 2 * lane);
    }
    // which waves' partials hold group g (lane v reads wave v's slots), then
    // every wave's partial requested at once and summed in wave order,
    // skipping the waves without the group (one LDS round trip, not two per
    // wave)
    int slot_l = -1;
    if (lane < kProjWaves) slot_l = s_grp[lane][0] == g ? 0 : (s_grp[lane][1] == g ? 1 : -1);
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int v0 = 0; v0 < kProjWaves; v0 += 8) {
      float4 tv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int slot = __builtin_amdgcn_readlane(slot_l, v0 + j);
        tv[j] = *reinterpret_cast<const float4*>(s_wp + ((v0 + j) * 2 + (slot > 0 ? 1 : 0)) * 256 +
                                                 4 * lane);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (__builtin_amdgcn_readlane(slot_l, v0 + j) < 0) continue;
        s.x = s.x + tv[j].x;
        s.y = s.y + tv[j].y;
        s.z = s.z + tv[j].z;
        s.w = s.w + tv[j].w;
      }
    }
    // the workgroups that publish for group g (its units [g TK, (g+1) TK));
    // a group inside one workgroup needs no hand-off
    const int wfirst = proj_wg_of(q, g * q.TK),
              count = proj_wg_of(q, (g + 1) * q.TK - 1) - wfirst + 1;
    float4 t = s;
    if (count > 1) {
      float* part = q.part + (size_t)g * q.maxc * 256;
      float* dst = part + (size_t)(wg - wfirst) * 256 + 4 * lane;
      st_coherent2(dst, s.x, s.y);
      st_coherent2(dst + 2, s.z, s.w);
      wait_vm();
      int last = 0;
      if (lane == 0) {
        int* cn = q.cnt + g;
        last = add_publish(cn, 1) == count - 1;
        if (last) {
          after_count();
          __hip_atomic_store(cn, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      if (!__builtin_amdgcn_readfirstlane(last)) continue;
      // 3. the group's last publisher: partials in workgroup order, 16 in flight
      t = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int k0 = 0; k0 < count; k0 += 16) {
        float2 lo[16], hi[16];
#pragma unroll
        for (int k = 0; k < 16; ++k)
          if (k0 + k < count) {
            lo[k] = ld_coherent2(part + (size_t)(k0 + k) * 256 + 4 * lane);
            hi[k] = ld_coherent2(part + (size_t)(k0 + k) * 256 + 4 * lane + 2);
          }
#pragma unroll
        for (int k = 0; k < 16; ++k)
          if (k0 + k < count) {
            t.x = t.x + lo[k].x;
            t.y = t.y + lo[k].y;
            t.z = t.z + hi[k].x;
            t.w = t.w + hi[k].y;
          }
      }
    }
    // lane-major sums -> columns, then the two 128-column blocks
    s_fin[proj_col<K>(lane, 0)] = t.x;
    s_fin[proj_col<K>(lane, 1)] = t.y;
    s_fin[proj_col<K>(lane, 2)] = t.z;
    s_fin[proj_col<K>(lane, 3)] = t.w;
    lds_wave_sync();
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      const int cc = 128 * blk + 2 * lane;
      float v0 = s_fin[cc], v1 = s_fin[cc + 1];
      h128_wave(v0, v1);
      half_t y0 = to_f16((v0 * p.rs) * ro[blk].x);
      half_t y1 = to_f16((v1 * p.rs) * ro[blk].y);
      if (q.bias) {
        y0 = to_f16((float)y0 + (float)__builtin_bit_cast(half_t, (uint16_t)bw[blk]));
        y1 = to_f16((float)y1 + (float)__builtin_bit_cast(half_t, (uint16_t)(bw[blk] >> 16)));
      }
      *reinterpret_cast<uint32_t*>(q.y + col0 + cc) = pack2(y0, y1);
    }
    lds_wave_sync();
  }
}

}  // namespace esc
