// One-launch routed-expert path (replaces the ~10 launches of
// EschaSparseMoeBlock._expert_path, escha_mlx/models/qwen3_5_moe.py:207-253).
//
// Work is split into two kinds of items, each one block of 4 waves:
//   gate_up item (r, b, kc): row r, output columns gate[128b, 128b+128) and
//     up[I+128b, I+128b+128), input rows [256kc, 256kc+256).  The block
//     input-transforms its own 256 inputs of x (no global hand-off), decodes
//     and multiplies 16 tiles x 16 kt, and writes 256 float32 partials.
//   down item (r, p, kb): row r, output columns [256p, 256p+256), input rows
//     [128kb, 128kb+128) = one 128-block of h.  It waits until all gate_up
//     items of (r, b=kb) are published, sums their partials in fixed kc order,
//     applies the gate_up output transform, swiglu and the down input
//     transform to get its 128 inputs, then decodes and multiplies 16 tiles x
//     8 kt and writes 256 float32 partials.  The last down item to finish a
//     (token, 256-column) tile sums every slot's partials in fixed order,
//     transforms them and combines the slots in slot order (f16(score)
//     weights, float32 sum, one f16 rounding): no float atomics anywhere, the
//     result is deterministic.
//
// Forward progress: blocks never wait on a block that has not started.  Every
// gate_up item is claimed (integer CAS) by the block that runs it; a down item
// whose inputs are not ready claims and runs the missing gate_up items itself,
// and otherwise waits only on items already claimed by running blocks, which
// never wait.  A bounded spin (err flag) is a last safety net.  The last block
// to finish resets every counter, so the integer workspace is zero again for
// the next call (it must be zero before the first).
#pragma once

#include "moe.hpp"

namespace esc {

__device__ __forceinline__ int ld_relaxed(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int add_acq_rel(int* p, int v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool claim(int* p) {
  int expected = 0;
  return __hip_atomic_compare_exchange_strong(p, &expected, 1, __ATOMIC_ACQ_REL,
                                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void fence_release() { __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent"); }
__device__ __forceinline__ void fence_acquire() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent"); }

struct FusedMoe {
  const uint16_t* x;
  const int* ids;
  const float* scores;
  const uint32_t* gu_code;
  const float* gu_rin;
  const float* gu_rout;
  const uint32_t* dn_code;
  const float* dn_rin;
  const float* dn_rout;
  uint16_t* y;
  float* partA;  // [nA][256]
  float* partB;  // [nB][256]
  int* cntA;     // [M*NB]  published gate_up items per (row, h-block)
  int* claimA;   // [nA]
  int* cntB;     // [T*NCP] finished down items per (token, column pair)
  int* done;     // [1]
  int* err;      // [1] sticky: a spin bound was hit
  int T, top_k, H, I;
  int NB;   // I / 128
  int NKC;  // H / 256
  int NCP;  // H / 256
  int nA, nB;
};

constexpr int kFusedThreads = 256;
constexpr int kSpinLimit = 1 << 11;  // outer polls of 64 (x s_sleep) before giving up
enum { kReady = -1, kWait = -2, kTimeout = -3 };

// Inverse of Geo<K>::col: tile column c -> (lane within tile, column slot).
template <int K>
__device__ __forceinline__ void col_owner(int c, int& q, int& ci) {
  if constexpr (K == 2) {
    q = (c & 7) >> 1;
    ci = (c & 1) + 2 * (c >> 3);
  } else {
    q = c & 7;
    ci = c >> 3;
  }
}

// 16 tiles x nkt kt of one stream: float32 partial of the item's 256 columns
// (item column j = 16 * item_tile + tile_col) written to dst.  nt_of(it) maps
// the item's tile 0..15 to the stream's tile column.
template <int K, typename NtFn>
__device__ __forceinline__ void item_gemv(const uint32_t* __restrict__ code_e, int TN, int kt_base,
                                          int nkt, NtFn nt_of, const uint32_t* s_x,
                                          float (*s_red)[64][4], float* __restrict__ dst) {
  using G = Geo<K>;
  constexpr int NG = 16 / G::TPW;  // tile groups per item
  constexpr int WPG = 4 / NG;      // waves per group
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int g = wave / WPG, wi = wave % WPG;
  const int q = lane % G::LPT, i = lane / G::LPT;
  const int nt = nt_of(g * G::TPW + i);
  const int src = i * G::LPT + (q + G::LPT - 1) % G::LPT;
  const int kper = nkt / WPG, k0 = wi * kper;
  const size_t kstride = (size_t)TN * (8 * K);
  const uint32_t* lp = code_e + (size_t)nt * (8 * K) + q * G::WPL + (size_t)(kt_base + k0) * kstride;
  float acc[G::NCOL];
#pragma unroll
  for (int c = 0; c < G::NCOL; ++c) acc[c] = 0.f;
  LaneWords<K> cur = load_lane_words<K>(lp);
  for (int k = 0; k < kper; ++k) {
    LaneWords<K> nxt = cur;
    if (k + 1 < kper) nxt = load_lane_words<K>(lp + (size_t)(k + 1) * kstride);
    uint32_t xw[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) xw[j] = s_x[8 * (k0 + k) + j];
    const uint32_t wprev = __shfl(cur.w[G::WPL - 1], src);
    fast_tile<K, false>(cur, wprev, xw, nullptr, acc);
    cur = nxt;
  }
#pragma unroll
  for (int c = 0; c < G::NCOL; ++c) s_red[wave][lane][c] = acc[c];
  __syncthreads();
  {
    const int j = threadIdx.x, it = j >> 4, c = j & 15;
    const int gg = it / G::TPW, ii = it % G::TPW;
    int qq, ci;
    col_owner<K>(c, qq, ci);
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < WPG; ++w) v = v + s_red[gg * WPG + w][ii * G::LPT + qq][ci];
    dst[j] = v;
  }
}

__device__ __forceinline__ uint32_t pack2(half_t a, half_t b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

template <int K>
__device__ void run_gate_up(const FusedMoe& p, int a, uint32_t* s_x, float (*s_red)[64][4]) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int kc = a % p.NKC, rb = a / p.NKC, b = rb % p.NB, r = rb / p.NB;
  const int t = r / p.top_k, e = p.ids[r];
  const int TK = p.H / 16, TN = 2 * p.I / 16;
  if (wave < 2) {
    const int c = 256 * kc + 128 * wave + 2 * lane;
    const uint16_t* xr = p.x + (size_t)t * p.H + c;
    const float* ri = p.gu_rin + (size_t)e * p.H + c;
    float v0 = (float)__builtin_bit_cast(half_t, xr[0]) * ri[0];
    float v1 = (float)__builtin_bit_cast(half_t, xr[1]) * ri[1];
    h128_wave(v0, v1);
    s_x[64 * wave + lane] = pack2(to_f16(v0 * kRS), to_f16(v1 * kRS));
  }
  __syncthreads();
  const int half_tn = p.I / 16;
  item_gemv<K>(p.gu_code + (size_t)e * TK * TN * (8 * K), TN, 16 * kc, 16,
               [&](int it) { return it < 8 ? 8 * b + it : half_tn + 8 * b + (it - 8); }, s_x, s_red,
               p.partA + (size_t)a * 256);
  fence_release();
  __syncthreads();
  if (threadIdx.x == 0) add_acq_rel(&p.cntA[r * p.NB + b], 1);
}

// h-block kb of row r -> the 128 down inputs (f16 pairs) in s_x[0..63].
__device__ void down_inputs(const FusedMoe& p, int r, int kb, uint32_t* s_x) {
  const int lane = threadIdx.x & 63;
  const int e = p.ids[r];
  const float* base = p.partA + (size_t)(r * p.NB + kb) * p.NKC * 256;
  float g0 = 0.f, g1 = 0.f, u0 = 0.f, u1 = 0.f;
  for (int kc = 0; kc < p.NKC; ++kc) {
    const float2 gv = *reinterpret_cast<const float2*>(base + (size_t)kc * 256 + 2 * lane);
    const float2 uv = *reinterpret_cast<const float2*>(base + (size_t)kc * 256 + 128 + 2 * lane);
    g0 = g0 + gv.x;
    g1 = g1 + gv.y;
    u0 = u0 + uv.x;
    u1 = u1 + uv.y;
  }
  h128_wave(g0, g1);
  h128_wave(u0, u1);
  const int cg = 128 * kb + 2 * lane, cu = p.I + cg;
  const float* ro = p.gu_rout + (size_t)e * 2 * p.I;
  const half_t h0 = swiglu1(to_f16((g0 * kRS) * ro[cg]), to_f16((u0 * kRS) * ro[cu]));
  const half_t h1 = swiglu1(to_f16((g1 * kRS) * ro[cg + 1]), to_f16((u1 * kRS) * ro[cu + 1]));
  const float* ri = p.dn_rin + (size_t)e * p.I + cg;
  float v0 = (float)h0 * ri[0];
  float v1 = (float)h1 * ri[1];
  h128_wave(v0, v1);
  s_x[lane] = pack2(to_f16(v0 * kRS), to_f16(v1 * kRS));
}

// Last down item of (token t, column pair cp): transform every slot and combine.
__device__ void combine_tile(const FusedMoe& p, int t, int cp) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (wave >= 2) return;
  const int col = 256 * cp + 128 * wave + 2 * lane;
  float a0 = 0.f, a1 = 0.f;
  for (int s = 0; s < p.top_k; ++s) {
    const int row = t * p.top_k + s, e = p.ids[row];
    const float* pb = p.partB + (size_t)(row * p.NCP + cp) * p.NB * 256 + 128 * wave + 2 * lane;
    float v0 = 0.f, v1 = 0.f;
    for (int kb = 0; kb < p.NB; ++kb) {
      const float2 pv = *reinterpret_cast<const float2*>(pb + (size_t)kb * 256);
      v0 = v0 + pv.x;
      v1 = v1 + pv.y;
    }
    h128_wave(v0, v1);
    const float* ro = p.dn_rout + (size_t)e * p.H + col;
    const half_t d0 = to_f16((v0 * kRS) * ro[0]);
    const half_t d1 = to_f16((v1 * kRS) * ro[1]);
    const float w = (float)(half_t)p.scores[row];
    a0 = a0 + (float)d0 * w;
    a1 = a1 + (float)d1 * w;
  }
  p.y[(size_t)t * p.H + col] = __builtin_bit_cast(uint16_t, (half_t)a0);
  p.y[(size_t)t * p.H + col + 1] = __builtin_bit_cast(uint16_t, (half_t)a1);
}

template <int K_GU, int K_DN>
__device__ void run_down(const FusedMoe& p, int bi, uint32_t* s_x, float (*s_red)[64][4],
                         int* s_flag) {
  const int tid = threadIdx.x;
  const int kb = bi % p.NB, rc = bi / p.NB, cp = rc % p.NCP, r = rc / p.NCP;
  const int t = r / p.top_k, e = p.ids[r];
  // wait for the gate_up items of (r, kb); run unclaimed ones ourselves
  int* cnt = &p.cntA[r * p.NB + kb];
  int spins = 0;
  for (;;) {
    if (tid == 0) {
      int st = kWait;
      for (int poll = 0; poll < 64 && st == kWait; ++poll) {
        if (ld_relaxed(cnt) >= p.NKC) {
          st = kReady;
          break;
        }
        for (int kc = 0; kc < p.NKC; ++kc) {
          const int a = (r * p.NB + kb) * p.NKC + kc;
          if (ld_relaxed(&p.claimA[a]) == 0 && claim(&p.claimA[a])) {
            st = a;
            break;
          }
        }
        if (st == kWait) __builtin_amdgcn_s_sleep(2);
      }
      if (st == kWait && (++spins > kSpinLimit || ld_relaxed(p.err) != 0)) st = kTimeout;
      *s_flag = st;
    }
    __syncthreads();
    const int st = *s_flag;
    __syncthreads();
    if (st == kReady) break;
    if (st >= 0) {
      run_gate_up<K_GU>(p, st, s_x, s_red);
      __syncthreads();
      continue;
    }
    if (st == kTimeout) {
      if (tid == 0) atomicOr(p.err, 1);
      break;
    }
  }
  fence_acquire();
  if ((tid >> 6) == 0) down_inputs(p, r, kb, s_x);
  __syncthreads();
  const int TK = p.I / 16, TN = p.H / 16;
  item_gemv<K_DN>(p.dn_code + (size_t)e * TK * TN * (8 * K_DN), TN, 8 * kb, 8,
                  [&](int it) { return 16 * cp + it; }, s_x, s_red, p.partB + (size_t)bi * 256);
  fence_release();
  __syncthreads();
  if (tid == 0) *s_flag = (add_acq_rel(&p.cntB[t * p.NCP + cp], 1) == p.top_k * p.NB - 1);
  __syncthreads();
  const int last = *s_flag;
  __syncthreads();
  if (last) {
    fence_acquire();
    combine_tile(p, t, cp);
  }
}

template <int K_GU, int K_DN>
__global__ __launch_bounds__(kFusedThreads) void k_moe_fused(FusedMoe p) {
  __shared__ float s_red[4][64][4];
  __shared__ uint32_t s_x[128];
  __shared__ int s_flag;
  const int tid = threadIdx.x;
  for (int a = blockIdx.x; a < p.nA; a += gridDim.x) {
    if (tid == 0) s_flag = claim(&p.claimA[a]);
    __syncthreads();
    const int mine = s_flag;
    __syncthreads();
    if (mine) {
      run_gate_up<K_GU>(p, a, s_x, s_red);
      __syncthreads();
    }
  }
  for (int bi = blockIdx.x; bi < p.nB; bi += gridDim.x) {
    run_down<K_GU, K_DN>(p, bi, s_x, s_red, &s_flag);
    __syncthreads();
  }
  // teardown: the last block resets the integer workspace for the next call
  fence_release();
  __syncthreads();
  if (tid == 0) s_flag = (add_acq_rel(p.done, 1) == (int)gridDim.x - 1);
  __syncthreads();
  if (s_flag) {
    fence_acquire();
    const int M = p.T * p.top_k;
    for (int i = tid; i < M * p.NB; i += kFusedThreads) p.cntA[i] = 0;
    for (int i = tid; i < p.nA; i += kFusedThreads) p.claimA[i] = 0;
    for (int i = tid; i < p.T * p.NCP; i += kFusedThreads) p.cntB[i] = 0;
    __syncthreads();
    if (tid == 0) *p.done = 0;
  }
}

}  // namespace esc
