// Many independent token-layers of routed experts with the decode shared
// between the VALU and the LDS pipe: the throughput mode of
// esc_moe_expert_path_layers (the steady-state form of
// EschaSparseMoeBlock._expert_path, escha_mlx/models/qwen3_5_moe.py:207-253)
// for 2-bit (K=2) gate_up and down.
//
// Launches: gate_up items, then down items with the slot combine.  The item kernels run
// one workgroup of 16 waves per CU: it stages the 65,536-entry decode table
// (128 KiB) in LDS once, and its waves decode kTablePairsLayers of every 8
// step pairs from it and the rest by hash (fast_tile_mix).  Every wave works
// on its own contiguous range of P items, streaming their code one wave-step
// (1 KiB) at a time with the next step's load in flight; the last step of an
// item requests the first step (and the small inputs) of the next.  Both
// kernels load their code non-temporally (it is read once per call), so the
// x, scales and partials that are read again stay in the L2 (config 3: 307.1
// -> 299.7 MB of HBM traffic per call, 1947-1952 -> 1962-1971 GB/s on one box).  The
// workgroup stages its items' pointers in LDS at the start, so no item waits
// on a chain of dependent global loads.
//
//   gate_up item (l, r, b, kc): layer l, routed row r, the 8 gate and the 8
//     up tiles of h-block b over kt [8kc, 8kc+8): 8 wave-steps of 16 tiles.
//     The wave input-transforms the item's 128 inputs of x (one H128) and
//     decodes.  A group (l, r, b) is H/128 consecutive items, so a wave's
//     range covers one or two groups: it sums its items of a group in
//     registers and publishes one partial per group; the group's last
//     contributor sums the partials in wave order and derives the h-block's
//     128 down inputs (gate_up output transform, SwiGLU, down input
//     transform) into xh2.
//   down item (l, r, cp, e8): row r's 256 output columns [256cp, 256cp+256)
//     -- two blocks of the output transform -- over the eighth e8 of the I
//     inputs: I/128 wave-steps of 16 tiles.  Groups (l, r, cp) of 8 items
//     are published and finished as above: the output transform of both
//     blocks into the f16 rows.
//   combine (l, t, cp): the last of a token's top_k finishers of column pair
//     cp (a device-scope counter per (l, t, cp), reset by it) sums the f16
//     rows of the token in slot order (f16(score) weights, float32 sum, one
//     f16 rounding) into y.
//
// Hand-offs use agent-scope atomics (add_publish, fused.hpp), with a wave's
// partial stores completed (s_waitcnt) before its increment of the group
// counter; the finisher reads the partials with agent-scope atomic loads
// after the count and resets the counter, so the integer workspace is zero
// again after every call (it must be zero before the first).  No float atomics: every sum has a fixed
// order (items in kc order within a wave, partials in wave order) and the
// result is deterministic.
#pragma once

#include "fused.hpp"

namespace esc {

constexpr int kLayersWaves = 16;      // waves per workgroup (one workgroup per CU)
constexpr int kTablePairsLayers = 4;  // table pairs of every 8 in the layer kernels
constexpr int kDownEighths = 8;       // down items split the I inputs in eighths
constexpr int kLayersMaxI = 2048;     // the down kernel keeps I/16 input words per wave (2 VGPRs)
constexpr int kLayersMaxRange = 8;    // items per wave (the host sizes the grid)

struct LayersMoe {
  const MoeLayer* layers;  // [L]
  char* ws;                // workspace; byte offsets:
  size_t off_part;         //   [groups][maxc][2][128] f32 partials of this launch's groups
  size_t off_cnt;          //   [groups] int: partials published per group
  size_t off_cnt_cb;       //   [L][T][H/256] int: down rows finished per (token, column pair)
  size_t off_xh2;          //   [L][M][I/2] u32 down inputs (paired f16 words)
  size_t off_rows;         //   [L][M][H/2] u32 down output rows (f16 pairs)
  int L, T, top_k, H, I;
  int M;     // T * top_k
  int NB;    // I / 128   h-blocks
  int NKC;   // H / 128   gate_up items per (row, h-block)
  int NHB;   // H / 128   down column blocks
  int P;     // items per wave of the launch (<= kLayersMaxRange)
  int maxc;  // partial slots per group (waves a group's items can span)
};


__device__ __forceinline__ void st_coherent_u32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_coherent_u32(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Issue priority from the work a wave has left: a SIMD issues from its
// oldest ready wave first, so with equal ranges the oldest wave runs ahead
// and the youngest is left alone at the end with nothing to hide its
// latencies; a wave with more items left gets the higher priority instead,
// and the waves of a SIMD finish together.
__device__ __forceinline__ void prio_left(int left) {
  if (left >= 4)
    __builtin_amdgcn_s_setprio(3);
  else if (left == 3)
    __builtin_amdgcn_s_setprio(2);
  else if (left == 2)
    __builtin_amdgcn_s_setprio(1);
  else
    __builtin_amdgcn_s_setprio(0);
}

__device__ __forceinline__ void lds_wave_sync() {
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

template <typename T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
  const uint64_t v = (uint64_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (T*)(((uint64_t)hi << 32) | lo);
}

// One wave-step: decode + multiply the words in w.  The step's 8 input
// words are lanes j0 .. j0+7 of xv (uniform: read into scalar registers).
__device__ __forceinline__ void mix_step(const LaneWords<2>& w, uint32_t xv, int j0, uint32_t tb,
                                         float* acc) {
  uint32_t xp[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) xp[j] = __builtin_amdgcn_readlane(xv, j0 + j);
  fast_tile_mix<kTablePairsLayers>(w, quad_prev_word(w.w[3]), xp, acc, tb);
}

// Steps 0 .. nsteps-2 of an item at base + k * stride + off (words), the
// first step's words already in w; each step requests the following one
// (one load per step, never conditional: a conditional load costs the
// decode registers and its schedule).  Step k's inputs are lanes 8k .. 8k+7
// of xv.  The caller runs the last step.
__device__ __forceinline__ void walk_head(const uint32_t* base, uint32_t off, int nsteps,
                                          uint32_t stride, uint32_t xv, uint32_t tb,
                                          LaneWords<2>& w, float* acc) {
#pragma unroll 1
  for (int k = 0; k + 1 < nsteps; ++k) {
    const LaneWords<2> wn = load_lane_words_nt(base + ((size_t)(k + 1) * stride + off));
    mix_step(w, xv, 8 * k, tb, acc);
    w = wn;
  }
}

// The waves of [first, last] that a group of `size` consecutive items spans
// when every wave runs P consecutive items.
__device__ __forceinline__ void group_waves(int g, int size, int P, int& first, int& count) {
  first = g * size / P;
  count = ((g + 1) * size - 1) / P - first + 1;
}

// Publish this wave's partial of group g (acc, 4 per lane, stored as
// [slot pair][lane][2] so each store covers 512 contiguous bytes); true when
// this wave is the group's last contributor (which then resets the counter
// and finishes the group).
__device__ __forceinline__ bool publish(const LayersMoe& p, int g, int size, const float* acc) {
  const int lane = threadIdx.x & 63;
  const int gw = blockIdx.x * kLayersWaves + (threadIdx.x >> 6);
  int first, count;
  group_waves(g, size, p.P, first, count);
  float* dst = reinterpret_cast<float*>(p.ws + p.off_part) +
               ((size_t)g * p.maxc + (gw - first)) * 256 + 2 * lane;
  st_coherent2(dst, acc[0], acc[1]);
  st_coherent2(dst + 128, acc[2], acc[3]);
  wait_vm();
  int last = 0;
  if (lane == 0) {
    int* c = reinterpret_cast<int*>(p.ws + p.off_cnt) + g;
    last = add_publish(c, 1) == count - 1;
    if (last) {
      after_count();
      __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  return __builtin_amdgcn_readfirstlane(last);
}

// The finisher's view of group g: lane's floats 2 lane, +1 of the 16-tile
// columns' first 8 tiles (a) and last 8 tiles (b), summed over the group's
// partials in wave order.  Tile t of the lane's pair is lane / 8; column
// cc = 2 (lane % 8) sits in tile-lane il = 4 t + (cc & 7) / 2 at slot pair
// cc >> 3; tiles 8-15 are 32 tile-lanes (64 floats) further.
__device__ __forceinline__ void group_sum(const LayersMoe& p, int g, int size, float& a0, float& a1,
                                          float& b0, float& b1) {
  const int lane = threadIdx.x & 63, cc = 2 * (lane & 7);
  const int off = 128 * (cc >> 3) + 2 * (4 * (lane >> 3) + ((cc & 7) >> 1));
  int first, count;
  group_waves(g, size, p.P, first, count);
  const float* src = reinterpret_cast<const float*>(p.ws + p.off_part) + (size_t)g * p.maxc * 256 + off;
  a0 = a1 = b0 = b1 = 0.f;
  for (int j0 = 0; j0 < count; j0 += 4) {
    float2 av[4], bv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (j0 + j < count) {
        av[j] = ld_coherent2(src + (j0 + j) * 256);
        bv[j] = ld_coherent2(src + (j0 + j) * 256 + 64);
      }
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (j0 + j < count) {
        a0 = a0 + av[j].x;
        a1 = a1 + av[j].y;
        b0 = b0 + bv[j].x;
        b1 = b1 + bv[j].y;
      }
  }
}

// ---------------------------------------------------------------- gate_up

struct GuItem {
  int l, r, b, kc;
};
__device__ __forceinline__ GuItem gu_item(const LayersMoe& p, int i) {
  const int per_row = p.NB * p.NKC, per_layer = p.M * per_row;
  GuItem it;
  it.l = i / per_layer;
  const int j = i - it.l * per_layer;
  it.r = j / per_row;
  const int rem = j - it.r * per_row;
  it.b = rem / p.NKC;
  it.kc = rem - it.b * p.NKC;
  return it;
}

struct GuMeta {
  const uint32_t* code;  // the item's first wave-step, lane 0
  const uint16_t* x;     // the token's x at input 128 kc
  const float* rin;      // the expert's gate_up rin at input 128 kc
  const float* rout;     // the expert's gate_up rout at gate column 128 b (up: + I)
  const float* drin;     // the expert's down rin at input 128 b
};

__device__ __forceinline__ GuMeta gu_meta(const LayersMoe& p, const MoeLayer& L, const GuItem& it) {
  const int e = as_global(L.ids)[it.r];
  const size_t tn = 2 * p.I / 16;
  GuMeta m;
  m.code = L.gu_code + (size_t)e * (p.H / 16) * tn * 16 + (size_t)(8 * it.kc) * tn * 16 +
           8 * it.b * 16;
  m.x = L.x + (size_t)(it.r / p.top_k) * p.H + 128 * it.kc;
  m.rin = L.gu_rin + (size_t)e * p.H + 128 * it.kc;
  m.rout = L.gu_rout + (size_t)e * 2 * p.I + 128 * it.b;
  m.drin = L.dn_rin + (size_t)e * p.I + 128 * it.b;
  return m;
}

__device__ __forceinline__ GuMeta gu_meta_uniform(const GuMeta& s) {
  GuMeta m;
  m.code = uniform_ptr(s.code);
  m.x = uniform_ptr(s.x);
  m.rin = uniform_ptr(s.rin);
  m.rout = uniform_ptr(s.rout);
  m.drin = uniform_ptr(s.drin);
  return m;
}

// the item's 128 inputs times rin, H128, * RS, f16, as the decode's input
// pairs: lane j holds word j (kt j / 8)
__device__ __forceinline__ uint32_t gu_inputs(uint32_t xw, float2 ri) {
  float v0 = (float)__builtin_bit_cast(half_t, (uint16_t)xw) * ri.x;
  float v1 = (float)__builtin_bit_cast(half_t, (uint16_t)(xw >> 16)) * ri.y;
  h128_wave(v0, v1);
  return paired_word(pack2(to_f16(v0 * kRS), to_f16(v1 * kRS)));
}

// gate and up sums of the lane's two columns -> the lane's word of xh2
// the lane's gate and up output scales and down input scales of the item's
// h-block (requested before the group's hand-off, so the finisher does not
// wait on them)
struct GuScales {
  float2 rg, ru, ri;
};
__device__ __forceinline__ GuScales gu_scales(const LayersMoe& p, const GuMeta& m) {
  const int lane = threadIdx.x & 63;
  return GuScales{ld_global_f2(m.rout + 2 * lane),
                  ld_global_f2(m.rout + p.I + 2 * lane),
                  ld_global_f2(m.drin + 2 * lane)};
}

__device__ __forceinline__ void gu_epilogue(const LayersMoe& p, int l, int r, int b,
                                            const GuScales& sc, float g0, float g1, float u0,
                                            float u1) {
  const int lane = threadIdx.x & 63;
  h128_wave(g0, g1);
  h128_wave(u0, u1);
  const float2 rg = sc.rg, ru = sc.ru, ri = sc.ri;
  const half_t h0 = swiglu1(to_f16((g0 * kRS) * rg.x), to_f16((u0 * kRS) * ru.x));
  const half_t h1 = swiglu1(to_f16((g1 * kRS) * rg.y), to_f16((u1 * kRS) * ru.y));
  float v0 = (float)h0 * ri.x;
  float v1 = (float)h1 * ri.y;
  h128_wave(v0, v1);
  reinterpret_cast<uint32_t*>(p.ws + p.off_xh2)[(size_t)(l * p.M + r) * (p.I / 2) + 64 * b +
                                                lane] =
      paired_word(pack2(to_f16(v0 * kRS), to_f16(v1 * kRS)));
}

// grid: G workgroups of 16 waves, each wave P consecutive items
// (P = ceil(items / 16 G) <= 8); dynamic LDS 128 KiB (the table).
__global__ __launch_bounds__(64 * kLayersWaves) void k_moe_layers_gu(LayersMoe p) {
  extern __shared__ uint16_t s_tab[];
  __shared__ GuMeta s_meta[kLayersMaxRange * kLayersWaves];
  const int n = p.L * p.M * p.NB * p.NKC;
  {
    // the item's layer record, then the table's pieces, then the item's
    // routed pointers: the table copy overlaps the dependent loads
    const int t = threadIdx.x, i = blockIdx.x * kLayersWaves * p.P + t;
    const bool has = t < p.P * kLayersWaves && i < n;
    const GuItem it = gu_item(p, has ? i : 0);
    const MoeLayer L = p.layers[it.l];
    TablePieces tp;
    table_fetch(tp);
    const GuMeta m = gu_meta(p, L, it);
    table_put(tp, s_tab);
    if (has) s_meta[t] = m;
  }
  const uint32_t tb = (uint32_t)(size_t)s_tab;
  __syncthreads();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int i0 = (blockIdx.x * kLayersWaves + wave) * p.P;
  const int iend = min(i0 + p.P, n);
  if (i0 >= n) return;
  const int il = lane >> 2, q = lane & 3;
  const uint32_t off = (uint32_t)((il < 8 ? il : p.I / 16 + (il - 8)) * 16 + q * 4);
  const uint32_t stride = (2 * p.I / 16) * 16;
  const GuMeta* meta = s_meta + wave * p.P - i0;  // meta[i]: item i of this wave
  GuMeta m = gu_meta_uniform(meta[i0]);
  LaneWords<2> w = load_lane_words_nt(m.code + off);
  uint32_t xw = *as_global(reinterpret_cast<const uint32_t*>(m.x + 2 * lane));
  float2 ri = ld_global_f2(m.rin + 2 * lane);
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int i = i0; i < iend; ++i) {
    prio_left(iend - i);
    const bool more = i + 1 < iend;
    const GuMeta m1 = more ? gu_meta_uniform(meta[i + 1]) : m;
    const uint32_t xv = gu_inputs(xw, ri);
    walk_head(m.code, off, 8, stride, xv, tb, w, acc);
    // the next item's inputs and first step (the current item's again when
    // there is none: in bounds, unused)
    xw = *as_global(reinterpret_cast<const uint32_t*>(m1.x + 2 * lane));
    ri = ld_global_f2(m1.rin + 2 * lane);
    {
      const LaneWords<2> wn = load_lane_words_nt(m1.code + off);
      mix_step(w, xv, 56, tb, acc);
      w = wn;
    }
    const int g = i / p.NKC;  // group (l, r, b)
    if (!more || (i + 1) / p.NKC != g) {
      const GuScales sc = gu_scales(p, m);
      if (publish(p, g, p.NKC, acc)) {
        float g0, g1, u0, u1;
        group_sum(p, g, p.NKC, g0, g1, u0, u1);
        const GuItem it = gu_item(p, i);
        gu_epilogue(p, it.l, it.r, it.b, sc, g0, g1, u0, u1);
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c] = 0.f;
    }
    m = m1;
  }
}

// ---------------------------------------------------------------- down

// y of (l, t) at the column pair cp (blocks 2 cp and 2 cp + 1): the token's
// top_k rows in slot order (f16(score) weights, float32 sum, one f16
// rounding), read with device-coherent loads (other waves wrote them).
__device__ __forceinline__ void combine_pair(const LayersMoe& p, int l, int t, int cp) {
  const int lane = threadIdx.x & 63;
  const MoeLayer& L = p.layers[l];
  const uint32_t* rws = reinterpret_cast<const uint32_t*>(p.ws + p.off_rows) +
                        ((size_t)l * p.M + t * p.top_k) * (p.H / 2) + 128 * cp + lane;
  float s[2][2] = {{0.f, 0.f}, {0.f, 0.f}};
  for (int k0 = 0; k0 < p.top_k; k0 += 8) {
    // slots past top_k re-read the last slot and add +0 (s starts at +0 and
    // is never -0, so this is exact): every load unconditional and issued
    // together (a load under a branch waits for all the loads before it)
    const int n = min(8, p.top_k - k0);
    uint32_t d8[2][8];
    float w8[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int k = k0 + min(j, n - 1);
      d8[0][j] = ld_coherent_u32(rws + (size_t)k * (p.H / 2));
      d8[1][j] = ld_coherent_u32(rws + (size_t)k * (p.H / 2) + 64);
      w8[j] = (float)(half_t)as_global(L.scores)[t * p.top_k + k];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
      for (int blk = 0; blk < 2; ++blk) {
        const float v0 = (float)__builtin_bit_cast(half_t, (uint16_t)d8[blk][j]) * w8[j];
        const float v1 = (float)__builtin_bit_cast(half_t, (uint16_t)(d8[blk][j] >> 16)) * w8[j];
        s[blk][0] = s[blk][0] + (j < n ? v0 : 0.f);
        s[blk][1] = s[blk][1] + (j < n ? v1 : 0.f);
      }
    }
  }
#pragma unroll
  for (int blk = 0; blk < 2; ++blk)
    as_global_w(reinterpret_cast<uint32_t*>(L.y + (size_t)t * p.H + 256 * cp + 128 * blk))[lane] =
        pack2((half_t)s[blk][0], (half_t)s[blk][1]);
}


struct DnItem {
  int l, r, cp, e8;
};
__device__ __forceinline__ DnItem dn_item(const LayersMoe& p, int i) {
  const int per_row = (p.NHB / 2) * kDownEighths, per_layer = p.M * per_row;
  DnItem it;
  it.l = i / per_layer;
  const int j = i - it.l * per_layer;
  it.r = j / per_row;
  const int rem = j - it.r * per_row;
  it.cp = rem / kDownEighths;
  it.e8 = rem - it.cp * kDownEighths;
  return it;
}

struct DnMeta {
  const uint32_t* code;  // the item's first wave-step, lane 0
  const float* rout;     // the expert's down rout at column 256 cp
};

__device__ __forceinline__ DnMeta dn_meta(const LayersMoe& p, const MoeLayer& L, const DnItem& it) {
  const int e = as_global(L.ids)[it.r];
  const size_t tn = p.H / 16;
  DnMeta m;
  m.code = L.dn_code + (size_t)e * (p.I / 16) * tn * 16 + (size_t)(it.e8 * (p.I / 128)) * tn * 16 +
           16 * it.cp * 16;
  m.rout = L.dn_rout + (size_t)e * p.H + 256 * it.cp;
  return m;
}

// the eighth's I/16 input words of item i: word j in lane j % 64 of xq[j / 64]
template <int QV>
__device__ __forceinline__ void dn_load_inputs(const LayersMoe& p, int i, uint32_t* xq) {
  const int lane = threadIdx.x & 63;
  const int per_row = (p.NHB / 2) * kDownEighths;
  const int row = i / per_row, e8 = i % kDownEighths;  // row = l M + r
  const int nw = p.I / 16;
  const uint32_t* src = reinterpret_cast<const uint32_t*>(p.ws + p.off_xh2) +
                        (size_t)row * (p.I / 2) + nw * e8;
#pragma unroll
  for (int j = 0; j < QV; ++j) xq[j] = src[min(64 * j + lane, nw - 1)];
}

// QV = ceil(I / 1024): input registers per lane (I/16 words per item).
// grid: G workgroups of 16 waves, each wave P consecutive items (P <= 8);
// dynamic LDS 128 KiB.
template <int QV>
__global__ __launch_bounds__(64 * kLayersWaves) void k_moe_layers_dn(LayersMoe p) {
  extern __shared__ uint16_t s_tab[];
  __shared__ DnMeta s_meta[kLayersMaxRange * kLayersWaves];
  const int n = p.L * p.M * (p.NHB / 2) * kDownEighths;
  const int NS = p.I / 128;  // wave-steps per item
  {
    // as in the gate_up kernel: the table copy overlaps the item's loads
    const int t = threadIdx.x, i = blockIdx.x * kLayersWaves * p.P + t;
    const bool has = t < p.P * kLayersWaves && i < n;
    const DnItem it = dn_item(p, has ? i : 0);
    const MoeLayer L = p.layers[it.l];
    TablePieces tp;
    table_fetch(tp);
    const DnMeta m = dn_meta(p, L, it);
    table_put(tp, s_tab);
    if (has) s_meta[t] = m;
  }
  const uint32_t tb = (uint32_t)(size_t)s_tab;
  __syncthreads();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int i0 = (blockIdx.x * kLayersWaves + wave) * p.P;
  const int iend = min(i0 + p.P, n);
  if (i0 >= n) return;
  const uint32_t off = (uint32_t)(lane * 4);  // 16 consecutive tiles of one kt
  const uint32_t stride = (p.H / 16) * 16;
  const DnMeta* meta = s_meta + wave * p.P - i0;  // meta[i]: item i of this wave
  DnMeta m{uniform_ptr(meta[i0].code), uniform_ptr(meta[i0].rout)};
  LaneWords<2> w = load_lane_words_nt(m.code + off);
  uint32_t xq[QV];
  dn_load_inputs<QV>(p, i0, xq);
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int i = i0; i < iend; ++i) {
    prio_left(iend - i);
    const bool more = i + 1 < iend;
    const int in = more ? i + 1 : i;
    const DnMeta m1 = {uniform_ptr(meta[in].code), uniform_ptr(meta[in].rout)};
    uint32_t xv[QV];
#pragma unroll
    for (int j = 0; j < QV; ++j) xv[j] = xq[j];
    // step k: kt e8 NS + k, input words 8k .. 8k+7 (register k / 8)
#pragma unroll 1
    for (int k = 0; k + 1 < NS; ++k) {
      const LaneWords<2> wn = load_lane_words_nt(m.code + ((size_t)(k + 1) * stride + off));
      mix_step(w, QV == 1 || k < 8 ? xv[0] : xv[QV - 1], 8 * (k & 7), tb, acc);
      w = wn;
    }
    dn_load_inputs<QV>(p, in, xq);
    {
      const LaneWords<2> wn = load_lane_words_nt(m1.code + off);
      mix_step(w, QV == 1 || NS <= 8 ? xv[0] : xv[QV - 1], 8 * ((NS - 1) & 7), tb, acc);
      w = wn;
    }
    const int g = i / kDownEighths;  // group (l, r, cp)
    if (!more || (i + 1) / kDownEighths != g) {
      // the output scales, requested before the hand-off
      const float2 ra = ld_global_f2(m.rout + 2 * lane);
      const float2 rb = ld_global_f2(m.rout + 128 + 2 * lane);
      if (publish(p, g, kDownEighths, acc)) {
        // columns 2 lane, +1 of block 2 cp (tiles 0-7, a) and 2 cp + 1 (b)
        float a0, a1, b0, b1;
        group_sum(p, g, kDownEighths, a0, a1, b0, b1);
        const DnItem it = dn_item(p, i);
        h128_wave(a0, a1);
        h128_wave(b0, b1);
        uint32_t* row = reinterpret_cast<uint32_t*>(p.ws + p.off_rows) +
                        (size_t)(it.l * p.M + it.r) * (p.H / 2) + 128 * it.cp + lane;
        st_coherent_u32(row, pack2(to_f16((a0 * kRS) * ra.x), to_f16((a1 * kRS) * ra.y)));
        st_coherent_u32(row + 64, pack2(to_f16((b0 * kRS) * rb.x), to_f16((b1 * kRS) * rb.y)));
        wait_vm();
        // the last of the token's top_k rows of this column pair combines them
        const int t = it.r / p.top_k;
        int last = 0;
        if (lane == 0) {
          int* c = reinterpret_cast<int*>(p.ws + p.off_cnt_cb) +
                   ((size_t)it.l * p.T + t) * (p.NHB / 2) + it.cp;
          last = add_publish(c, 1) == p.top_k - 1;
          if (last) {
            after_count();
            __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        }
        if (__builtin_amdgcn_readfirstlane(last)) combine_pair(p, it.l, t, it.cp);
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c] = 0.f;
    }
    m = m1;
  }
}

}  // namespace esc
