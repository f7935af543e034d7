// One-launch coded linear for a few rows (M < 16): the whole of
// EschaLinear.__call__ (escha_mlx/dense.py:337-362) -- input transform, coded
// GEMV and output transform (+ optional bias) -- in a single kernel.
//
// grid (ceil(TN/TPW), ceil(M/R), S); block = 4 waves; block z owns kt range
// [z*KS, (z+1)*KS) with KS a multiple of 8, i.e. whole 128-input blocks:
//   1. the block input-transforms its own KS/8 blocks of x for its R rows
//      (one wave per (row, block)) into LDS, so no xh tensor is written;
//   2. one row (RMAX == 1, the GEMV): the 4 waves split the kt range, decode
//      TPW tiles per kt step and multiply-add with packed dot2 on the VALU,
//      then reduce in LDS.  Several rows (RMAX > 1, the row-blocked GEMM):
//      wave w decodes its 16/LPT tiles over the block's kt and multiplies them
//      on the matrix core (mma_tile), B column c =
//      row c of the group, so R <= RMAX rows share every decoded weight.  The
//      block publishes float32 partials [S][M][OC] with device-coherent stores;
//   3. the last of the S blocks of a (row group, column group) -- found with
//      a device-scope counter that it resets to zero -- sums the S partials
//      of each (row, column pair) in z order (each thread walks its pairs'
//      partials 32 loads at a time, so all rows' loads overlap),
//      output-transforms each (row, 128-column block) and writes y.
// Deterministic (fixed summation order, no float atomics); tolerance
// contract like k_gemv_fast (reassociated float32 sum).
#pragma once

#include "fused.hpp"

namespace esc {

// Arguments of one projection's one-launch linear: the launch covers
// groups x row_groups x S workgroups (column group, row group, kt split).
struct LinearSmallArgs {
  const uint16_t* x;
  const float* rin;
  const uint32_t* code;
  const float* rout;
  const uint16_t* bias;
  int M, TK, TN, KS, R, S, groups, row_groups;
  float rs;
  float* part;
  int* cnt;
  uint16_t* y;
};

// The workgroup's LDS: decode table (table decode only), the transformed
// inputs of its rows (after the decode loop: the finishing sums, [R][TPW*16]
// floats), the VALU path's wave partials.
template <int K, bool LUT, int RMAX>
struct LinearSmallSmem {
  uint16_t lut[LUT ? 65536 : 1];
  alignas(16) uint32_t x[RMAX][8 * 64];  // up to 64 kt per row
  float red[RMAX > 1 ? 1 : 4][64][Geo<K>::NCOL];
  int last;
  static_assert(Geo<K>::TPW * 16 <= 8 * 64, "finishing sums fit in the input stage");
};

template <int K, bool LUT, int RMAX>
__device__ __forceinline__ void linear_small_body(const LinearSmallArgs& a, int ntg, int rg, int z,
                                                  LinearSmallSmem<K, LUT, RMAX>& sm) {
  const uint16_t* __restrict__ x = a.x;
  const float* __restrict__ rin = a.rin;
  const uint32_t* __restrict__ code = a.code;
  const float* __restrict__ rout = a.rout;
  const uint16_t* __restrict__ bias = a.bias;
  const int M = a.M, TK = a.TK, TN = a.TN, KS = a.KS, R = a.R, S = a.S;
  const float rs = a.rs;
  float* __restrict__ part = a.part;
  int* __restrict__ cnt = a.cnt;
  uint16_t* __restrict__ y = a.y;
  using G = Geo<K>;
  constexpr int TPS = 16 / G::LPT;
  constexpr int kCols = G::TPW * 16;  // columns per column group
  constexpr int kBlocks = kCols / 128;  // 128-column blocks per group
  constexpr bool kMma = RMAX > 1;
  uint16_t* s_lut = sm.lut;
  auto& s_x = sm.x;
  auto& s_red = sm.red;
  int& s_last = sm.last;
  stage_lut<LUT>(s_lut);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row0 = rg * R;
  const int IC = TK * 16, OC = TN * 16;
  const int nb = KS / 8;  // 128-input blocks of the block's kt range
  const size_t kstride = (size_t)TN * (8 * K);
  const int src = (lane & ~(G::LPT - 1)) | ((lane + G::LPT - 1) & (G::LPT - 1));
  // matrix-core geometry: wave w owns tiles [tile0, tile0 + 16/LPT), lane
  // kt offset gk, tile-lane c = LPT*tc + q, B column c
  const int tile0 = ntg * G::TPW + TPS * wave;
  const int gk = lane >> 4, c = lane & 15, tc = c / G::LPT, q = lane % G::LPT;
  // VALU geometry: all waves on the group's TPW tiles, kt split 4 ways
  const int vtile = lane / G::LPT, kl0 = wave * (KS / 4);
  const bool valid = kMma ? tile0 < TN : ntg * G::TPW + vtile < TN;  // kMma: wave-uniform
  const uint32_t* lp = kMma ? code + (size_t)(tile0 + tc) * (8 * K) + q * G::WPL
                            : code + (size_t)(ntg * G::TPW) * (8 * K) + lane * G::WPL;
  const int kt0 = kMma ? z * KS + gk : z * KS + kl0;
  const int nsteps = KS / 4, kstep = kMma ? 4 : 1;
  // the first step's code is requested before anything else, so its latency
  // overlaps the input transform; lanes past the last tile read the code's
  // first words instead (in bounds, never stored) -- a load under a branch
  // would be waited for where the branch ends, before the inputs are
  // requested
  const uint32_t* lp0 = valid ? lp + (size_t)kt0 * kstride : code;
  LaneWords<K> cur = load_lane_words_nt<K>(lp0);
  // 1. input transform: xh = f16(H128(f32(x) * rin) * RS) per (row, block);
  // wave w takes items w, w + 4, ...; with several rows it requests up to 8
  // items' inputs before transforming them, so one memory round trip serves
  // 8 items
  constexpr int kXB = RMAX > 1 ? 8 : 1;
  for (int base = wave; base < R * nb; base += 4 * kXB) {
    uint16_t xa[kXB], xb[kXB];
    float ra[kXB], rb[kXB];
    int r = base / nb, b = base - (base / nb) * nb;
#pragma unroll
    for (int j = 0; j < kXB; ++j) {
      if (base + 4 * j < R * nb) {
        const int row = min(row0 + r, M - 1);
        const int cc = 16 * KS * z + 128 * b + 2 * lane;
        xa[j] = x[(size_t)row * IC + cc];
        xb[j] = x[(size_t)row * IC + cc + 1];
        ra[j] = rin[cc];
        rb[j] = rin[cc + 1];
      }
      for (b += 4; b >= nb; b -= nb) ++r;
    }
    r = base / nb, b = base - (base / nb) * nb;
#pragma unroll
    for (int j = 0; j < kXB; ++j) {
      if (base + 4 * j < R * nb) {
        float v0 = (float)__builtin_bit_cast(half_t, xa[j]) * ra[j];
        float v1 = (float)__builtin_bit_cast(half_t, xb[j]) * rb[j];
        h128_wave(v0, v1);
        s_x[r][64 * b + lane] = pack2(to_f16(v0 * rs), to_f16(v1 * rs));
      }
      for (b += 4; b >= nb; b -= nb) ++r;
    }
  }
  __syncthreads();
  // 2. decode + multiply over the block's kt range
  if constexpr (kMma) {
    if (valid) {
      f32x4_t acc[G::NCOL];
#pragma unroll
      for (int i = 0; i < G::NCOL; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      const uint32_t* xs = s_x[c < R ? c : R - 1];
      for (int k = 0; k < nsteps; ++k) {
        LaneWords<K> nxt = cur;
        if (k + 1 < nsteps) nxt = load_lane_words_nt<K>(lp + (size_t)(kt0 + kstep * (k + 1)) * kstride);
        const u32x4_t* xb = reinterpret_cast<const u32x4_t*>(xs + 8 * (4 * k + gk));
        const uint32_t wprev = __shfl(cur.w[G::WPL - 1], src);
        mma_tile<K, LUT>(cur, wprev, xb[0], xb[1], acc, s_lut);
        cur = nxt;
      }
      if (c < R && row0 + c < M)
        mma_store<K, true>(acc, gk, part + ((size_t)z * M + row0 + c) * OC + 16 * tile0);
    }
  } else {
    float acc[1][G::NCOL];
#pragma unroll
    for (int i = 0; i < G::NCOL; ++i) acc[0][i] = 0.f;
    for (int k = 0; k < nsteps; ++k) {
      LaneWords<K> nxt = cur;
      if (valid && k + 1 < nsteps) nxt = load_lane_words_nt<K>(lp + (size_t)(kt0 + k + 1) * kstride);
      uint32_t xw[8], xp[1][8];
#pragma unroll
      for (int i = 0; i < 8; ++i) xw[i] = s_x[0][8 * (kl0 + k) + i];
      x_pairs(xw, xp[0]);
      const uint32_t wprev = __shfl(cur.w[G::WPL - 1], src);
      fast_tile_rows<K, LUT, 1>(cur, wprev, xp, s_lut, acc);
      cur = nxt;
    }
    // reduce the 4 waves (fixed order) and publish the partials
#pragma unroll
    for (int i = 0; i < G::NCOL; ++i) s_red[wave][lane][i] = acc[0][i];
    __syncthreads();
    if (wave == 0 && valid) {
      float* pr = part + ((size_t)z * M + row0) * OC + (size_t)(ntg * G::TPW + vtile) * 16;
#pragma unroll
      for (int i = 0; i < G::NCOL; ++i) {
        float v = s_red[0][lane][i];
        v = v + s_red[1][lane][i];
        v = v + s_red[2][lane][i];
        v = v + s_red[3][lane][i];
        st_coherent(pr + G::col(q, i), v);
      }
    }
  }
  // this wave's output scales and bias for the finishing passes (every pass
  // of a wave transforms the same 128-column block, wave % kBlocks), requested
  // now so that the last split does not wait on them after the counter
  const int colw = ntg * kCols + 128 * (wave % kBlocks) + 2 * lane;
  float ro0 = 0.f, ro1 = 0.f, bs0 = 0.f, bs1 = 0.f;
  if (colw < OC) {
    ro0 = rout[colw];
    ro1 = rout[colw + 1];
    if (bias) {
      bs0 = (float)__builtin_bit_cast(half_t, bias[colw]);
      bs1 = (float)__builtin_bit_cast(half_t, bias[colw + 1]);
    }
  }
  wait_vm();
  __syncthreads();
  // 3. the last split of (row group, column group) finishes the columns
  if (threadIdx.x == 0) {
    int* cn = &cnt[(size_t)rg * a.groups + ntg];
    const bool last = add_publish(cn, 1) == S - 1;
    if (last) {
      after_count();
      __hip_atomic_store(cn, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    s_last = last;
  }
  __syncthreads();
  if (!s_last) return;
  // The sums go to LDS over the inputs' stage (unused since the decode loop).
  // Several rows: the group's (row, column pair) items, thread t summing
  // items t, t + 256, ..., each item's S partials in z order, 32 loads in
  // flight across its items.
  const int col0 = ntg * kCols;
  constexpr int kPairs = kCols / 2;
  const int n_rows = min(R, M - row0);
  float* s_fin = reinterpret_cast<float*>(&s_x[0][0]);  // [n_rows][kCols]
  if constexpr (RMAX == 1) {
    // one row: one thread per column, its partials 32 at a time
    const int j = threadIdx.x;
    if (j < kCols && col0 + j < OC) {
      const float* pb = part + (size_t)row0 * OC + col0 + j;
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
      s_fin[j] = v;
    }
  } else {
    const int t = threadIdx.x, n_items = n_rows * kPairs;
    const int T = t < n_items ? ((n_items - 1 - t) / 256 + 1) * S : 0;
    const size_t zstride = (size_t)M * OC;
    auto item_ptr = [&](int jj) {
      const int item = t + 256 * jj, r = item / kPairs, cp = item % kPairs;
      return part + (size_t)(row0 + r) * OC + col0 + 2 * cp;
    };
    auto item_ok = [&](int jj) { return col0 + 2 * ((t + 256 * jj) % kPairs) < OC; };
    int jl = 0, zl = 0;  // the next load's item and split
    const float* pl = item_ptr(0);
    bool okl = item_ok(0);
    int js = 0, zs = 0;  // the next sum's item and split
    float sx = 0.f, sy = 0.f;
    for (int p0 = 0; p0 < T; p0 += 32) {
      float2 pv[32];
#pragma unroll
      for (int q = 0; q < 32; ++q) {
        pv[q] = make_float2(0.f, 0.f);
        if (p0 + q < T) {
          if (okl) pv[q] = ld_coherent2(pl);
          pl += zstride;
          if (++zl == S) {
            zl = 0;
            ++jl;
            pl = item_ptr(jl);
            okl = item_ok(jl);
          }
        }
      }
#pragma unroll
      for (int q = 0; q < 32; ++q) {
        if (p0 + q < T) {
          sx = sx + pv[q].x;
          sy = sy + pv[q].y;
          if (++zs == S) {
            const int item = t + 256 * js, r = item / kPairs, cp = item % kPairs;
            s_fin[r * kCols + 2 * cp] = sx;
            s_fin[r * kCols + 2 * cp + 1] = sy;
            sx = 0.f;
            sy = 0.f;
            zs = 0;
            ++js;
          }
        }
      }
    }
  }
  __syncthreads();
  // one wave per (row, 128-column block); a wave's blocks are all block
  // wave % kBlocks, whose output scales it requested above
  for (int it = wave; it < n_rows * kBlocks; it += 4) {
    const int r = it / kBlocks, b = it % kBlocks;
    const int col = col0 + 128 * b + 2 * lane;
    if (col >= OC) continue;
    float v0 = s_fin[r * kCols + 128 * b + 2 * lane];
    float v1 = s_fin[r * kCols + 128 * b + 2 * lane + 1];
    h128_wave(v0, v1);
    half_t y0 = to_f16((v0 * rs) * ro0);  // col == colw
    half_t y1 = to_f16((v1 * rs) * ro1);
    if (bias) {
      y0 = to_f16((float)y0 + bs0);
      y1 = to_f16((float)y1 + bs1);
    }
    uint16_t* yr = y + (size_t)(row0 + r) * OC + col;
    yr[0] = __builtin_bit_cast(uint16_t, y0);
    yr[1] = __builtin_bit_cast(uint16_t, y1);
  }
}


template <int K, bool LUT, int RMAX>
__global__ __launch_bounds__(256) void k_linear_small(LinearSmallArgs a) {
  __shared__ LinearSmallSmem<K, LUT, RMAX> sm;
  linear_small_body<K, LUT, RMAX>(a, blockIdx.x, blockIdx.y, blockIdx.z, sm);
}

// 1 to 4 projections of the same input rows and K in one launch (an attention
// block's q, k and v): the flat grid holds projection 0's workgroups, then
// projection 1's, ..., each running exactly its own single-projection plan
// (column groups, splits, partials and counters), so each output is
// bit-identical to its own k_linear_small launch.
constexpr int kLinearMultiMax = 4;
struct LinearMultiArgs {
  LinearSmallArgs p[kLinearMultiMax];
  int n;
};

template <int K, int RMAX>
__global__ __launch_bounds__(256) void k_linear_multi(LinearMultiArgs m) {
  __shared__ LinearSmallSmem<K, false, RMAX> sm;
  int b = blockIdx.x, i = 0;
  for (; i + 1 < m.n; ++i) {
    const int nw = m.p[i].groups * m.p[i].row_groups * m.p[i].S;
    if (b < nw) break;
    b -= nw;
  }
  // one body, its arguments chosen per workgroup (as k_linear_pair)
  const LinearSmallArgs& a = m.p[i];
  const int gr = a.groups * a.row_groups;
  linear_small_body<K, false, RMAX>(a, b % a.groups, (b % gr) / a.groups, b / gr, sm);
}

// Two projections of the same input rows in one launch (the projection-pair
// dispatch of escha_mlx/dense.py:365-437): the flat grid holds projection
// 0's workgroups, then projection 1's, each running exactly the single
// projection's plan (its own column groups, splits, partials and counters),
// so each output is bit-identical to its own k_linear_small launch.  The two
// projections' LDS layouts share one allocation.
template <int K0, int K1, bool LUT, int RMAX>
__global__ __launch_bounds__(256) void k_linear_pair(LinearSmallArgs a0, LinearSmallArgs a1) {
  __shared__ union {
    LinearSmallSmem<K0, LUT, RMAX> p0;
    LinearSmallSmem<K1, LUT, RMAX> p1;
  } sm;
  const int n0 = a0.groups * a0.row_groups * a0.S;
  const bool first = (int)blockIdx.x < n0;
  const int b = first ? (int)blockIdx.x : (int)blockIdx.x - n0;
  if constexpr (K0 == K1) {
    // one body, its arguments chosen per workgroup (two inlined copies of the
    // same body would spill)
    const LinearSmallArgs& a = first ? a0 : a1;
    const int gr = a.groups * a.row_groups;
    linear_small_body<K0, LUT, RMAX>(a, b % a.groups, (b % gr) / a.groups, b / gr, sm.p0);
  } else if (first) {
    const int gr = a0.groups * a0.row_groups;
    linear_small_body<K0, LUT, RMAX>(a0, b % a0.groups, (b % gr) / a0.groups, b / gr, sm.p0);
  } else {
    const int gr = a1.groups * a1.row_groups;
    linear_small_body<K1, LUT, RMAX>(a1, b % a1.groups, (b % gr) / a1.groups, b / gr, sm.p1);
  }
}

}  // namespace esc
