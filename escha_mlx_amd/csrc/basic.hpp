// Table build, tile decode, 128-point transforms, router top-k, row grouping.
#pragma once

#include "codec.hpp"

namespace esc {

// ---------------------------------------------------------------- table
__global__ __launch_bounds__(256) void k_lut_init() {
  uint32_t s = blockIdx.x * 256u + threadIdx.x;
  g_lut[s] = decode_hash_bits(s);
}

// ---------------------------------------------------------------- decode
// code [TK][TN][8K] -> w [IC][OC] f16 (escha_mlx/msl.py:183-202, ref.py:126-134).
// One 256-thread block per tile, one thread per trellis step.
template <int K, bool LUT>
__global__ __launch_bounds__(256) void k_decode_tiles(const uint32_t* __restrict__ code, int TN,
                                                      int OC, uint16_t* __restrict__ w) {
  const int tile = blockIdx.x;
  const int kt = tile / TN, nt = tile - kt * TN;
  const int t = threadIdx.x;
  const uint32_t* wp = code + (size_t)tile * (8 * K);
  uint32_t s = step_state<K>([&](int i) { return wp[i]; }, t);
  uint16_t v = LUT ? g_lut[s] : decode_hash_bits(s);
  w[(size_t)(16 * kt + step_row(t)) * OC + 16 * nt + step_col(t)] = v;
}

// ---------------------------------------------------------------- H128
// One wave owns one 128-block of one row; lane l holds elements 2l and 2l+1.
// Stage s pairs i with i ^ (1 << s), bit 0 first, (a + b, a - b) in float32
// (escha_mlx/ref.py:204-218, msl.py:905-913).  Built with -ffp-contract=off.
// The lane exchanges stay on the VALU: DPP quad permutes for lane ^ 1 and
// ^ 2, two bank-masked DPP row shifts for ^ 4 and ^ 8, and the gfx950 row /
// half-wave swaps (v_permlane16_swap, v_permlane32_swap) for ^ 16 and ^ 32.

// value of lane ^ M (M in {1, 2, 4, 8}: within a row of 16 lanes)
template <int M>
__device__ __forceinline__ float lane_xor(float v) {
  const int x = __builtin_bit_cast(int, v);
  int r;
  if constexpr (M == 1) {
    r = __builtin_amdgcn_update_dpp(x, x, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
  } else if constexpr (M == 2) {
    r = __builtin_amdgcn_update_dpp(x, x, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
  } else {
    // lanes with bit M clear read lane + M (row_shl), the others lane - M
    // (row_shr); each shift writes only its banks of 4 lanes
    constexpr int lo_banks = M == 4 ? 0x5 : 0x3, hi_banks = M == 4 ? 0xA : 0xC;
    r = __builtin_amdgcn_update_dpp(x, x, 0x100 + M, 0xF, lo_banks, false);
    r = __builtin_amdgcn_update_dpp(r, x, 0x110 + M, 0xF, hi_banks, false);
  }
  return __builtin_bit_cast(float, r);
}

__device__ __forceinline__ void h128_wave(float& v0, float& v1) {
  const int lane = threadIdx.x & 63;
  {
    float a = v0, b = v1;
    v0 = a + b;
    v1 = a - b;
  }
  auto stage = [&](float o0, float o1, bool upper) {
    if (upper) {
      v0 = o0 - v0;
      v1 = o1 - v1;
    } else {
      v0 = v0 + o0;
      v1 = v1 + o1;
    }
  };
  stage(lane_xor<1>(v0), lane_xor<1>(v1), lane & 1);
  stage(lane_xor<2>(v0), lane_xor<2>(v1), lane & 2);
  stage(lane_xor<4>(v0), lane_xor<4>(v1), lane & 4);
  stage(lane_xor<8>(v0), lane_xor<8>(v1), lane & 8);
  // ^ 16 and ^ 32: the swap returns the lower partner's value (lo) and the
  // upper partner's (hi) in every lane: a + b below, a - b above
  auto swap_stage = [&](auto swp, bool upper) {
    const auto p0 = swp(__builtin_bit_cast(unsigned, v0));
    const auto p1 = swp(__builtin_bit_cast(unsigned, v1));
    // elements copied out first: __builtin_bit_cast of a vector element
    // reads element 0 with this compiler
    const unsigned l0 = p0[0], h0 = p0[1], l1 = p1[0], h1 = p1[1];
    const float lo0 = __builtin_bit_cast(float, l0), hi0 = __builtin_bit_cast(float, h0);
    const float lo1 = __builtin_bit_cast(float, l1), hi1 = __builtin_bit_cast(float, h1);
    v0 = upper ? lo0 - hi0 : lo0 + hi0;
    v1 = upper ? lo1 - hi1 : lo1 + hi1;
  };
  swap_stage([](unsigned x) { return __builtin_amdgcn_permlane16_swap(x, x, false, false); },
             lane & 16);
  swap_stage([](unsigned x) { return __builtin_amdgcn_permlane32_swap(x, x, false, false); },
             lane & 32);
}

// Transform kernels: one wave per (row, 128-block); a 256-thread workgroup
// covers kTransformRows rows of one 128-block (kTransformRows / 4 per wave,
// their loads issued together).  grid (dim/128, ceil(m / kTransformRows)).
constexpr int kTransformRows = 16;

// Element types of the rows an input transform reads (esc_input_transform_typed).
enum { kRowsF16 = 0, kRowsBF16 = 1, kRowsF32 = 2 };

// Elements c, c + 1 of a row as float32 (exact for every type).
template <int DT>
__device__ __forceinline__ float2 row_pair(const void* rows, size_t i) {
  if constexpr (DT == kRowsF32) {
    return *reinterpret_cast<const float2*>(static_cast<const float*>(rows) + i);
  } else {
    const uint32_t xv = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(rows) + i);
    if constexpr (DT == kRowsBF16)
      return make_float2(__builtin_bit_cast(float, xv << 16),
                         __builtin_bit_cast(float, xv & 0xFFFF0000u));
    else
      return make_float2((float)__builtin_bit_cast(half_t, (uint16_t)xv),
                         (float)__builtin_bit_cast(half_t, (uint16_t)(xv >> 16)));
  }
}

// xh = f16(H128(f32(rows) * rin) * RS); rin is [E][IC] gathered by row_expert,
// or [IC] when row_expert is null (escha_mlx/msl.py:875-916, 1029-1047).
// DT: the rows' element type; f16 rows are the fused kernel's input, bf16 and
// f32 rows the reference's unfused branch (escha_mlx/dense.py:290-292,
// models/qwen3_5_moe.py:108-110), converted exactly to float32 here with no
// f16 rounding before the transform.
template <int DT>
__global__ __launch_bounds__(256) void k_input_transform(const void* __restrict__ rows,
                                                         const float* __restrict__ rin,
                                                         const int* __restrict__ row_expert,
                                                         int m, int IC, float rs,
                                                         uint16_t* __restrict__ out) {
  constexpr int RPW = kTransformRows / 4;
  const int blk = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c = blk * 128 + 2 * lane;
  const int row0 = blockIdx.y * kTransformRows + RPW * wave;
  float v[RPW][2];
#pragma unroll
  for (int j = 0; j < RPW; ++j) {
    const int row = min(row0 + j, m - 1);
    const float2 xv = row_pair<DT>(rows, (size_t)row * IC + c);
    const float* r = rin + (row_expert ? (size_t)row_expert[row] * IC : 0) + c;
    v[j][0] = xv.x * r[0];
    v[j][1] = xv.y * r[1];
  }
#pragma unroll
  for (int j = 0; j < RPW; ++j) {
    h128_wave(v[j][0], v[j][1]);
    if (row0 + j < m)
      *reinterpret_cast<uint32_t*>(out + (size_t)(row0 + j) * IC + c) =
          (uint32_t)__builtin_bit_cast(uint16_t, to_f16(v[j][0] * rs)) |
          ((uint32_t)__builtin_bit_cast(uint16_t, to_f16(v[j][1] * rs)) << 16);
  }
}

// y = f16((H128(mid) * RS) * rout) [+ bias, added in f32 after the f16 round]
// (escha_mlx/msl.py:919-949, 1050-1067; bias per dense.py:358-361).
// EXP: row_expert is given (rout per row's expert).
template <bool EXP>
__global__ __launch_bounds__(256) void k_output_transform(const float* __restrict__ mid,
                                                          const float* __restrict__ rout,
                                                          const int* __restrict__ row_expert,
                                                          const uint16_t* __restrict__ bias,
                                                          int m, int OC, float rs,
                                                          uint16_t* __restrict__ out) {
  constexpr int RPW = kTransformRows / 4;
  const int blk = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c = blk * 128 + 2 * lane;
  const int row0 = blockIdx.y * kTransformRows + RPW * wave;
  // every load unconditional (rows past m re-read row m - 1 and are not
  // stored), the bias (under its branch) first: a load under a branch waits
  // for all the loads before it
  const uint32_t bw = bias ? *reinterpret_cast<const uint32_t*>(bias + c) : 0u;
  float2 v[RPW], r[RPW];
#pragma unroll
  for (int j = 0; j < RPW; ++j) {
    const int row = min(row0 + j, m - 1);
    v[j] = *reinterpret_cast<const float2*>(mid + (size_t)row * OC + c);
    r[j] = *reinterpret_cast<const float2*>(rout + (EXP ? (size_t)row_expert[row] * OC : 0) + c);
  }
#pragma unroll
  for (int j = 0; j < RPW; ++j) {
    const int row = row0 + j;
    float v0 = v[j].x, v1 = v[j].y;
    h128_wave(v0, v1);
    half_t y0 = to_f16((v0 * rs) * r[j].x);
    half_t y1 = to_f16((v1 * rs) * r[j].y);
    if (bias) {
      y0 = to_f16((float)y0 + (float)__builtin_bit_cast(half_t, (uint16_t)(bw & 0xFFFFu)));
      y1 = to_f16((float)y1 + (float)__builtin_bit_cast(half_t, (uint16_t)(bw >> 16)));
    }
    if (row < m)
      *reinterpret_cast<uint32_t*>(out + (size_t)row * OC + c) =
          (uint32_t)__builtin_bit_cast(uint16_t, y0) | ((uint32_t)__builtin_bit_cast(uint16_t, y1) << 16);
  }
}

// ---------------------------------------------------------------- router
// logits [T][E] f32 -> ids [T][k] (descending, ties -> lower id), scores [T][k]
// = softmax over the k selected logits (escha_mlx/ref.py:326-331).
// One wave per token; E <= 1024 held as 16 values per lane.
__global__ __launch_bounds__(64) void k_route_topk(const float* __restrict__ logits, int E,
                                                   int top_k, int* __restrict__ ids,
                                                   float* __restrict__ scores) {
  const int tok = blockIdx.x, lane = threadIdx.x;
  const float* lg = logits + (size_t)tok * E;
  constexpr int kPer = 16;
  float v[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    int e = lane + 64 * i;
    v[i] = e < E ? lg[e] : -__builtin_inff();
  }
  float top0 = 0.f, sel[32];
  int selid[32];
  for (int k = 0; k < top_k; ++k) {
    // lane-local best (value desc, id asc)
    float bv = -__builtin_inff();
    int bi = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      int e = lane + 64 * i;
      if (e < E && (v[i] > bv || (v[i] == bv && e < bi))) {
        bv = v[i];
        bi = e;
      }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      float ov = __shfl_xor(bv, m);
      int oi = __shfl_xor(bi, m);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    sel[k] = bv;
    selid[k] = bi;
    if (k == 0) top0 = bv;
#pragma unroll
    for (int i = 0; i < kPer; ++i)
      if (lane + 64 * i == bi) v[i] = -__builtin_inff();
  }
  if (lane == 0) {
    float den = 0.f;
    float ex[32];
    for (int k = 0; k < top_k; ++k) {
      ex[k] = expf(sel[k] - top0);
      den += ex[k];
    }
    for (int k = 0; k < top_k; ++k) {
      ids[(size_t)tok * top_k + k] = selid[k];
      scores[(size_t)tok * top_k + k] = ex[k] / den;
    }
  }
}

// ---------------------------------------------------------------- groups
// Device build_groups (escha_mlx/moe.py:30-78): rows sorted stably by expert,
// each expert padded to a multiple of R, padding slots = m (zero sink row),
// groups past the end = expert -1.  Integer only, one block, deterministic.
// Shared memory holds per-expert counts; E <= 4096.
// The body runs in one block of 1024 threads (k_build_groups, or block 0 of
// k_moe_prep).
// Fast form when E * ceil(m / 64) <= kGroupMaskWords: a bit per (expert,
// row) in LDS.  A row's rank within its expert is the popcount of its
// expert's bits below it, an expert's count the popcount of all of them, so
// every slot is written once (no clearing pass, no ordering between writers)
// and the only serial step is the prefix over the experts' padded counts.
constexpr int kGroupMaskWords = 4096;

// exclusive prefix over the block (1024 threads) of one int per thread; the
// block's total in *total
__device__ __forceinline__ int block_exclusive_scan(int v, int* s_wsum, int* total) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int inc = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(inc, o);
    if (lane >= o) inc += t;
  }
  if (lane == 63) s_wsum[wave] = inc;
  __syncthreads();
  int before = 0, all = 0;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) {
    before += w < wave ? s_wsum[w] : 0;
    all += s_wsum[w];
  }
  *total = all;
  return before + inc - v;
}

__device__ void build_groups_mask(const int* __restrict__ row_expert, int m, int E, int R,
                                  int n_groups, int* __restrict__ rows_idx,
                                  int* __restrict__ group_expert, int* s_start,
                                  int* __restrict__ n_active) {
  __shared__ unsigned long long s_mask[kGroupMaskWords];  // [E][nw]
  __shared__ int s_wsum[16];
  const int tid = threadIdx.x, nt = blockDim.x;
  const int nw = (m + 63) >> 6;
  for (int i = tid; i < E * nw; i += nt) s_mask[i] = 0ull;
  __syncthreads();
  for (int r = tid; r < m; r += nt)
    atomicOr(&s_mask[row_expert[r] * nw + (r >> 6)], 1ull << (r & 63));
  __syncthreads();
  // experts 4 tid .. 4 tid + 3: counts, padded counts, first slots
  int cnt[4], pad[4], sum = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = 4 * tid + j;
    cnt[j] = 0;
    if (e < E)
      for (int w = 0; w < nw; ++w) cnt[j] += __popcll(s_mask[e * nw + w]);
    pad[j] = (cnt[j] + R - 1) / R * R;
    sum += pad[j];
  }
  int total;
  int start = block_exclusive_scan(sum, s_wsum, &total);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = 4 * tid + j;
    if (e < E) {
      s_start[e] = start;
      // the expert's groups and its padding slots (= m)
      for (int g = start / R; g < (start + pad[j]) / R; ++g) group_expert[g] = e;
      for (int i = cnt[j]; i < pad[j]; ++i) rows_idx[start + i] = m;
    }
    start += pad[j];
  }
  // past the last expert: padding slots and groups of expert -1
  if (n_active && tid == 0) *n_active = total / R;
  for (int i = total + tid; i < n_groups * R; i += nt) rows_idx[i] = m;
  for (int g = total / R + tid; g < n_groups; g += nt) group_expert[g] = -1;
  __syncthreads();
  // each row at its expert's first slot + the rows of its expert before it
  for (int r = tid; r < m; r += nt) {
    const int e = row_expert[r], w0 = r >> 6;
    const unsigned long long* me = s_mask + e * nw;
    int rank = __popcll(me[w0] & ((1ull << (r & 63)) - 1ull));
    for (int w = 0; w < w0; ++w) rank += __popcll(me[w]);
    rows_idx[s_start[e] + rank] = r;
  }
}

// n_active (when not null): the number of groups that hold rows.
__device__ void build_groups_block(const int* __restrict__ row_expert, int m, int E, int R,
                                   int n_groups, int* __restrict__ rows_idx,
                                   int* __restrict__ group_expert,
                                   int* __restrict__ n_active = nullptr) {
  __shared__ int s_start[4096];  // first padded slot of each expert
  if ((long)E * ((m + 63) >> 6) <= kGroupMaskWords) {
    build_groups_mask(row_expert, m, E, R, n_groups, rows_idx, group_expert, s_start, n_active);
    return;
  }
  __shared__ int s_cnt[4096];    // rows per expert, then rows placed so far
  __shared__ int s_e[1024];      // one chunk of row_expert
  const int tid = threadIdx.x, nt = blockDim.x;
  for (int e = tid; e < E; e += nt) s_cnt[e] = 0;
  for (int i = tid; i < n_groups * R; i += nt) rows_idx[i] = m;
  for (int g = tid; g < n_groups; g += nt) group_expert[g] = -1;
  __syncthreads();
  for (int r = tid; r < m; r += nt) atomicAdd(&s_cnt[row_expert[r]], 1);
  __syncthreads();
  // exclusive prefix of the padded counts: each thread sums 4 experts, then a
  // block-wide scan of the 1024 partial sums (Hillis-Steele in LDS)
  {
    int loc[4], sum = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = 4 * tid + j;
      loc[j] = e < E ? (s_cnt[e] + R - 1) / R * R : 0;
      sum += loc[j];
    }
    s_e[tid] = sum;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
      const int v = tid >= off ? s_e[tid - off] : 0;
      __syncthreads();
      s_e[tid] += v;
      __syncthreads();
    }
    int acc = s_e[tid] - sum;  // exclusive
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = 4 * tid + j;
      if (e < E) s_start[e] = acc;
      acc += loc[j];
    }
  }
  __syncthreads();
  // group_expert: every padded group of expert e
  for (int e = tid; e < E; e += nt) {
    const int ng = (s_cnt[e] + R - 1) / R;
    for (int g = 0; g < ng; ++g) group_expert[s_start[e] / R + g] = e;
    if (n_active && e == E - 1) *n_active = s_start[e] / R + ng;
    s_cnt[e] = 0;
  }
  __syncthreads();
  // stable placement, one chunk of nt rows at a time: a row's rank is the
  // number of earlier rows of its expert (earlier chunks counted in s_cnt)
  for (int c0 = 0; c0 < m; c0 += nt) {
    const int r = c0 + tid;
    const int e = r < m ? row_expert[r] : -1;
    s_e[tid] = e;
    __syncthreads();
    if (r < m) {
      int rank = s_cnt[e];
      for (int q = 0; q < tid; ++q) rank += (s_e[q] == e);
      rows_idx[s_start[e] + rank] = r;
    }
    __syncthreads();
    if (r < m) atomicAdd(&s_cnt[e], 1);
    __syncthreads();
  }
}

__global__ __launch_bounds__(1024) void k_build_groups(const int* __restrict__ row_expert, int m,
                                                       int E, int R, int n_groups,
                                                       int* __restrict__ rows_idx,
                                                       int* __restrict__ group_expert) {
  build_groups_block(row_expert, m, E, R, n_groups, rows_idx, group_expert);
}

}  // namespace esc
