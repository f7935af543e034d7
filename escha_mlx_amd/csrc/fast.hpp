// Split-K coded GEMV for gfx950 (tolerance contract: the float32 sum is
// reassociated, every decoded weight is still the bit-exact f16 of the format).
//
// Wave-step = one kt row of TPW consecutive tiles, which are contiguous in
// memory (code [kt][nt][8K]), so one coalesced vector load per lane pulls a
// wave's whole step: K=2 -> 16 B per lane (dwordx4, 4 lanes per 64 B tile,
// 16 tiles = 1 KiB); K=3 -> 12 B per lane (dwordx3, 8 lanes per 96 B tile,
// 8 tiles = 768 B).  Lane q of a tile owns the stream bits [q*32*WPL,
// (q+1)*32*WPL) and therefore the trellis steps whose window ENDS there; the
// 13-14 bits of history before its first word come from the previous lane of
// the same tile (circularly) through one cross-lane move.  Every window offset,
// tile row and output column is then a compile-time function of the step
// index, so decode + multiply-add fully unroll with the window in VGPRs.
//
// Reduction: the 4 waves of a block split the block's kt range; their column
// sums meet in LDS in a fixed order, and blocks along kt write float32
// partials [S][M][OC] that the epilogue kernels sum in fixed order: the
// result is deterministic run to run (no float atomics anywhere).
#pragma once

#include "exact.hpp"

namespace esc {

template <int K>
struct Geo;
template <>
struct Geo<2> {
  static constexpr int LPT = 4;   // lanes per tile
  static constexpr int WPL = 4;   // words per lane
  static constexpr int SPL = 64;  // trellis steps per lane
  static constexpr int TPW = 16;  // tiles per wave-step
  static constexpr int NCOL = 4;  // output columns per lane
  __device__ static constexpr int col_slot(int u) { return 2 * ((u & 7) >= 4) + ((u >> 5) & 1); }
  __device__ static int col(int q, int ci) { return 2 * q + (ci & 1) + 8 * (ci >> 1); }
};
template <>
struct Geo<3> {
  static constexpr int LPT = 8;
  static constexpr int WPL = 3;
  static constexpr int SPL = 32;
  static constexpr int TPW = 8;
  static constexpr int NCOL = 2;
  __device__ static constexpr int col_slot(int u) { return (u & 7) >= 4; }
  __device__ static int col(int q, int ci) { return q + 8 * ci; }
};

// Input-channel row (0..15) of the lane's step u (same for K=2 and K=3).
__device__ constexpr int fast_row(int u) {
  return 2 * ((u >> 3) & 3) + (u & 1) + 8 * ((u >> 1) & 1);
}

template <int K>
struct LaneWords {
  uint32_t w[Geo<K>::WPL];
};

// Global-memory view of a device pointer.  A pointer that arrives through
// memory (a layer record, an item pointer staged in LDS) is generic to the
// compiler, and its loads become FLAT instructions, which count against the
// LDS counter as well: every wait for LDS results (the table reads, the
// reductions) would then also wait for them, so a prefetch of the next
// step's code could not stay in flight across the decode.  Every device
// allocation this library reads is global memory.
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* as_global(const T* p) {
  return (const __attribute__((address_space(1))) T*)p;
}
template <typename T>
__device__ __forceinline__ __attribute__((address_space(1))) T* as_global_w(T* p) {
  return (__attribute__((address_space(1))) T*)p;
}
// float2 through the global view (HIP's float2 is a class that cannot be
// copied from an address-space-qualified reference; the native vector can)
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float2 ld_global_f2(const float* p) {
  const f32x2_t v = *as_global(reinterpret_cast<const f32x2_t*>(p));
  return make_float2(v.x, v.y);
}

template <int K>
__device__ __forceinline__ LaneWords<K> load_lane_words(const uint32_t* p) {
  LaneWords<K> r;
  if constexpr (K == 2) {
    typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
    const u32x4_t v = *as_global(reinterpret_cast<const u32x4_t*>(p));
    r.w[0] = v.x;
    r.w[1] = v.y;
    r.w[2] = v.z;
    r.w[3] = v.w;
  } else {
    const auto* g = as_global(p);
    r.w[0] = g[0];
    r.w[1] = g[1];
    r.w[2] = g[2];
  }
  return r;
}

// The same words through the streaming (non-temporal) path: for code that a
// call reads once, so it does not push the inputs, scales and partials that
// the call reads again out of the L2.
typedef uint32_t nt_u32x4_t __attribute__((ext_vector_type(4)));
template <int K = 2>
__device__ __forceinline__ LaneWords<K> load_lane_words_nt(const uint32_t* p) {
  LaneWords<K> r;
  if constexpr (K == 2) {
    const nt_u32x4_t v =
        __builtin_nontemporal_load(as_global(reinterpret_cast<const nt_u32x4_t*>(p)));
    r.w[0] = v.x;
    r.w[1] = v.y;
    r.w[2] = v.z;
    r.w[3] = v.w;
  } else {
    const auto* g = as_global(p);
    r.w[0] = __builtin_nontemporal_load(g);
    r.w[1] = __builtin_nontemporal_load(g + 1);
    r.w[2] = __builtin_nontemporal_load(g + 2);
  }
  return r;
}

// Decode the lane's SPL steps of one tile and accumulate x * w into acc[NCOL].
// xw: the 16 f16 inputs of this kt packed two per word (row r in half r&1 of
// word r>>1).  wprev: the previous lane's last word.
template <int K, bool LUT>
__device__ __forceinline__ void fast_tile(const LaneWords<K>& lw, uint32_t wprev,
                                          const uint32_t* xw, const uint16_t* lut, float* acc) {
  using G = Geo<K>;
#pragma unroll
  for (int u = 0; u < G::SPL; ++u) {
    const int rel = K * (u + 1) - 16;             // window start, bits from the lane's first bit
    const int a = (rel + 32) / 32 - 1;            // word holding the first bit (-1: previous lane)
    const int off = rel - 32 * a;
    const uint32_t hi = a < 0 ? wprev : lw.w[a];
    const uint32_t lo = (a + 1 < G::WPL) ? lw.w[a + 1] : 0u;
    const uint32_t s = window16(hi, lo, off);
    half_t wv;
    if constexpr (LUT)
      wv = __builtin_bit_cast(half_t, lut[s]);
    else
      wv = decode_hash(s);
    const int r = fast_row(u);
    const half_t xv = __builtin_bit_cast(half_t, (uint16_t)(xw[r >> 1] >> (16 * (r & 1))));
    const int ci = G::col_slot(u);
    acc[ci] = __builtin_fmaf((float)xv, (float)wv, acc[ci]);
  }
}

// ---------------------------------------------------------------- packed decode
// Hash decode of two states at a time, written against the gfx950 VALU:
//   x = s * 0xCBAC1FED mod 2^32 = s*0x1FED + (lo16(s*0xCBAC) << 16) for a
//   16-bit s: v_mul_lo_u16 with an SDWA destination in the high half, then
//   v_mad_u32_u16 (2 full-rate ops instead of one quarter-rate v_mul_lo_u32);
//   r = (x & 0x8FFF8FFF) ^ 0x3B603B60 (one v_bitop3_b32);
//   w = f16(lo16 r) + f16(hi16 r), RNE, written by an SDWA add straight into
//   one half of a packed pair, so two weights feed one v_dot2_f32_f16.
// The weights are bit-identical to decode_hash(); only the multiply-add is
// pairwise (tolerance contract).
constexpr uint32_t kClo = 0x1FEDu, kChi = 0xCBACu;

// x of the state in the low (HI=false) or high (HI=true) half of p.
template <bool HI>
__device__ __forceinline__ uint32_t hash_x(uint32_t p, uint32_t clo, uint32_t chi) {
  uint32_t y, x;
  if constexpr (HI) {
    __asm__("v_mul_lo_u16_sdwa %0, %1, %2 dst_sel:WORD_1 dst_unused:UNUSED_PAD src0_sel:WORD_1 src1_sel:WORD_0"
            : "=v"(y) : "v"(p), "v"(chi));
    __asm__("v_mad_u32_u16 %0, %1, %2, %3 op_sel:[1,0,0,0]" : "=v"(x) : "v"(p), "v"(clo), "v"(y));
  } else {
    __asm__("v_mul_lo_u16_sdwa %0, %1, %2 dst_sel:WORD_1 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_0"
            : "=v"(y) : "v"(p), "v"(chi));
    __asm__("v_mad_u32_u16 %0, %1, %2, %3" : "=v"(x) : "v"(p), "v"(clo), "v"(y));
  }
  return x;
}

// packed [w(r_lo), w(r_hi)] from two hash words
__device__ __forceinline__ uint32_t halves_sum2(uint32_t r_lo, uint32_t r_hi) {
  uint32_t w;
  __asm__("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1"
          : "=v"(w) : "v"(r_lo));
  __asm__("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1"
          : "+v"(w) : "v"(r_hi));
  return w;
}

__device__ __forceinline__ uint32_t mask_xor(uint32_t x) { return (x & kHashMask) ^ kHashXor; }

__device__ __forceinline__ float dot2(uint32_t xp, uint32_t wp, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, xp), __builtin_bit_cast(half2_t, wp),
                                acc, false);
}

// The 8 input pairs [x(r+2), x(r)] (r = 0,1,4,5,8,9,12,13 -> index
// 2(r>>2) | (r&1)) one kt's pairs of trellis steps (u, u+8) multiply.
__device__ __forceinline__ void x_pairs(const uint32_t* xw, uint32_t* xp) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 4 * (i >> 1) + (i & 1);
    const uint32_t sel = (r & 1) ? 0x07060302u : 0x05040100u;
    xp[i] = __builtin_amdgcn_perm(xw[r >> 1], xw[(r >> 1) + 1], sel);
  }
}
__device__ constexpr int xpair_index(int r) { return 2 * (r >> 2) | (r & 1); }

// Packed hash decode of the lane's steps u and u+8 (u>>3 even): they share a
// tile column and sit 2 rows apart, so they form one dot2 pair.  K=2: their
// 16-bit windows are adjacent, one v_alignbit gives both.
template <int K>
__device__ __forceinline__ uint32_t decode_pair(const LaneWords<K>& lw, uint32_t wprev, int u) {
  using G = Geo<K>;
  const uint32_t clo = kClo, chi = kChi;
  if constexpr (K == 2) {
    // 32-bit window starting at step u's first bit: [s_u | s_{u+8}]
    const int rel = 2 * (u + 1) - 16;
    const int a = (rel + 32) / 32 - 1, off = rel - 32 * a;
    const uint32_t hi = a < 0 ? wprev : lw.w[a];
    uint32_t p;
    if (off == 0)
      p = hi;
    else
      p = __builtin_amdgcn_alignbit(hi, lw.w[a + 1], 32 - off);
    return halves_sum2(mask_xor(hash_x<false>(p, clo, chi)), mask_xor(hash_x<true>(p, clo, chi)));
  } else {
    static_assert(G::WPL == 3, "");
    uint32_t s2[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int uu = u + 8 * (1 - h);  // low half: step u+8, high half: step u
      const int rel = 3 * (uu + 1) - 16;
      const int a = (rel + 32) / 32 - 1, off = rel - 32 * a;
      const uint32_t hi = a < 0 ? wprev : lw.w[a];
      // the state in the low 16 bits (bits above are ignored by the u16 ops)
      s2[h] = off <= 16 ? hi >> (16 - off) : __builtin_amdgcn_alignbit(hi, lw.w[a + 1], 48 - off);
    }
    return halves_sum2(mask_xor(hash_x<false>(s2[0], clo, chi)),
                       mask_xor(hash_x<false>(s2[1], clo, chi)));
  }
}

// Packed-decode variant of fast_tile (hash only), each pair multiplied as soon
// as it is decoded (the form the streaming kernels use).
template <int K>
__device__ __forceinline__ void fast_tile_packed(const LaneWords<K>& lw, uint32_t wprev,
                                                 const uint32_t* xp, float* acc) {
  using G = Geo<K>;
#pragma unroll
  for (int u = 0; u < G::SPL; ++u) {
    if ((u >> 3) & 1) continue;  // u+8 handled with u
    const int ci = G::col_slot(u);
    acc[ci] = dot2(xp[xpair_index(fast_row(u))], decode_pair<K>(lw, wprev, u), acc[ci]);
  }
}

// The same in two phases, so that a caller can decode while its inputs are
// still on their way: decode_pairs_packed keeps the lane's SPL/2 weight pairs
// in registers (step order), dot_pairs_packed multiplies them into acc in the
// same order, so the two are bit-identical to fast_tile_packed.
template <int K>
struct TilePairs {
  uint32_t w[Geo<K>::SPL / 2];
};

// The pairs are pinned where the decode is written (empty volatile asm with
// each pair as an operand): left alone, the compiler sinks each decode next to
// its multiply, past the barrier that waits for the inputs.
template <int K>
__device__ __forceinline__ TilePairs<K> decode_pairs_packed(const LaneWords<K>& lw,
                                                           uint32_t wprev) {
  TilePairs<K> t;
  int n = 0;
#pragma unroll
  for (int u = 0; u < Geo<K>::SPL; ++u)
    if (!((u >> 3) & 1)) t.w[n++] = decode_pair<K>(lw, wprev, u);
#pragma unroll
  for (int i = 0; i < Geo<K>::SPL / 2; ++i) __asm__ volatile("" : "+v"(t.w[i]));
  return t;
}

template <int K>
__device__ __forceinline__ void dot_pairs_packed(const TilePairs<K>& t, const uint32_t* xp,
                                                 float* acc) {
  using G = Geo<K>;
  int n = 0;
#pragma unroll
  for (int u = 0; u < G::SPL; ++u) {
    if ((u >> 3) & 1) continue;
    const int ci = G::col_slot(u);
    acc[ci] = dot2(xp[xpair_index(fast_row(u))], t.w[n++], acc[ci]);
  }
}

// R-row variant of fast_tile_packed: every state pair is decoded once (hash,
// or two table reads from LDS into the two halves) and multiplied into R
// rows' accumulators.  xp[r] are row r's input pairs (x_pairs).
// Step pairs of every 8 that the table-decode GEMV reads from the table in
// LDS; the others are hashed (the table is the hash's image, so the weights
// are the same either way).  Measured on MI355X (config 2, 5120^2 K=2 at
// batch 1): 4 of 8 beats 2, 6 and all 8.
constexpr int kTablePairs = 4;

template <int K, bool LUT, int R>
__device__ __forceinline__ void fast_tile_rows(const LaneWords<K>& lw, uint32_t wprev,
                                               const uint32_t (*xp)[8], const uint16_t* lut,
                                               float (*acc)[Geo<K>::NCOL]) {
  using G = Geo<K>;
  const uint32_t clo = kClo, chi = kChi;
  int pair = 0;
#pragma unroll
  for (int u = 0; u < G::SPL; ++u) {
    if ((u >> 3) & 1) continue;  // u+8 handled with u
    // table path: kTablePairs of every 8 pairs from the table, the rest by
    // hash (bit-identical), so the LDS and the VALU share the decode
    const bool from_lut = LUT && (pair++ & 7) < kTablePairs;
    uint32_t w2;
    if constexpr (K == 2) {
      const int rel = 2 * (u + 1) - 16;
      const int a = (rel + 32) / 32 - 1, off = rel - 32 * a;
      const uint32_t hi = a < 0 ? wprev : lw.w[a];
      const uint32_t p = off == 0 ? hi : __builtin_amdgcn_alignbit(hi, lw.w[a + 1], 32 - off);
      if (from_lut)
        w2 = (uint32_t)lut[p & 0xFFFFu] | ((uint32_t)lut[p >> 16] << 16);
      else
        w2 = halves_sum2(mask_xor(hash_x<false>(p, clo, chi)), mask_xor(hash_x<true>(p, clo, chi)));
    } else {
      uint32_t s2[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int uu = u + 8 * (1 - h);  // low half: step u+8, high half: step u
        const int rel = 3 * (uu + 1) - 16;
        const int a = (rel + 32) / 32 - 1, off = rel - 32 * a;
        const uint32_t hi = a < 0 ? wprev : lw.w[a];
        s2[h] = off <= 16 ? hi >> (16 - off)
                          : __builtin_amdgcn_alignbit(hi, lw.w[a + 1], 48 - off);
      }
      if (from_lut)
        w2 = (uint32_t)lut[s2[0] & 0xFFFFu] | ((uint32_t)lut[s2[1] & 0xFFFFu] << 16);
      else
        w2 = halves_sum2(mask_xor(hash_x<false>(s2[0], clo, chi)),
                         mask_xor(hash_x<false>(s2[1], clo, chi)));
    }
    const int ci = G::col_slot(u), xi = xpair_index(fast_row(u));
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r][ci] = dot2(xp[r][xi], w2, acc[r][ci]);
  }
}

// ---------------------------------------------------------------- MFMA accumulate
// The multiply-add of decoded tiles on the matrix core:
// v_mfma_f32_16x16x32_f16 with the decoded weights as the A operand and the
// inputs as B, one input row (token) per B column.
//
// Wave-step geometry: lane l works on kt offset g = l / 16 and on tile-lane
// i = l % 16 = LPT * tc + q (tile tc of the step's 16 / LPT tiles, lane q of
// the tile), so a wave-step covers 16 / LPT tiles x 4 kt.  A row i is one
// output column (tile tc, column Geo::col(q, ci)) for every k of an operand,
// and k = 8g + j runs over 8 inputs of kt g: one MFMA sums four kt.
//
// The lane's steps of column slot ci are u = (m, v): tile row 2m + (v & 1) +
// 8(v >> 1), m, v = 0..3.  A operand (ci, P) holds the 8 steps v in
// {2P, 2P+1}: register m = [w(m, 2P) | w(m, 2P+1) << 16], tile rows 8P + 2m
// and +1.  So the matching B operand is input words 4P..4P+3 of the kt in
// plain row order (word k = inputs 2k, 2k+1): one 16-byte piece.
//
// D (16x16 f32, 4 registers): lane l holds rows 4(l / 16) + r, i.e. the
// output columns of tile-lanes i = 4(l / 16) + r, for token l % 16.
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// the lane's step index of (m, v) in column slot ci
template <int K>
__device__ constexpr int mma_step(int m, int v, int ci) {
  return K == 2 ? 32 * (ci & 1) + 8 * m + 4 * (ci >> 1) + v : 8 * m + 4 * ci + v;
}

// 16-bit state of step u in the low half (K = 3; bits above ignored by the
// u16 ops and masked for the table)
__device__ __forceinline__ uint32_t state3(const LaneWords<3>& lw, uint32_t wprev, int u) {
  const int rel = 3 * (u + 1) - 16;
  const int a = (rel + 32) / 32 - 1, off = rel - 32 * a;
  const uint32_t hi = a < 0 ? wprev : lw.w[a];
  return off <= 16 ? hi >> (16 - off) : __builtin_amdgcn_alignbit(hi, lw.w[a + 1], 48 - off);
}
// 32-bit window [s_u | s_{u+8}] (K = 2: the two states are 16 bits apart)
__device__ __forceinline__ uint32_t window2(const LaneWords<2>& lw, uint32_t wprev, int u) {
  const int rel = 2 * (u + 1) - 16;
  const int a = (rel + 32) / 32 - 1, off = rel - 32 * a;
  const uint32_t hi = a < 0 ? wprev : lw.w[a];
  return off == 0 ? hi : __builtin_amdgcn_alignbit(hi, lw.w[a + 1], 32 - off);
}

// A operand (ci, P) of the lane's tile: hash decode, or reads of the
// 65,536-entry table (LUT) into the two halves of each register.
template <int K, bool LUT = false>
__device__ __forceinline__ u32x4_t mma_a_operand(const LaneWords<K>& lw, uint32_t wprev, int ci,
                                                 int P, const uint16_t* lut = nullptr) {
  const uint32_t clo = kClo, chi = kChi;
  u32x4_t a;
#pragma unroll
  for (int m = 0; m < 4; m += 2) {
    const int ua = mma_step<K>(m, 2 * P, ci), ub = mma_step<K>(m, 2 * P + 1, ci);
    // table path: half the words from the table, half by hash (as kTablePairs)
    const bool from_lut = LUT && m == 0;
    if constexpr (K == 2) {
      // one window per v gives the steps of m (high half) and m + 1 (low half)
      const uint32_t pa = window2(lw, wprev, ua), pb = window2(lw, wprev, ub);
      if (from_lut) {
        a[m] = (uint32_t)lut[pa >> 16] | ((uint32_t)lut[pb >> 16] << 16);
        a[m + 1] = (uint32_t)lut[pa & 0xFFFFu] | ((uint32_t)lut[pb & 0xFFFFu] << 16);
      } else {
        a[m] = halves_sum2(mask_xor(hash_x<true>(pa, clo, chi)), mask_xor(hash_x<true>(pb, clo, chi)));
        a[m + 1] =
            halves_sum2(mask_xor(hash_x<false>(pa, clo, chi)), mask_xor(hash_x<false>(pb, clo, chi)));
      }
    } else {
      const uint32_t sa0 = state3(lw, wprev, ua), sb0 = state3(lw, wprev, ub);
      const uint32_t sa1 = state3(lw, wprev, ua + 8), sb1 = state3(lw, wprev, ub + 8);
      if (from_lut) {
        a[m] = (uint32_t)lut[sa0 & 0xFFFFu] | ((uint32_t)lut[sb0 & 0xFFFFu] << 16);
        a[m + 1] = (uint32_t)lut[sa1 & 0xFFFFu] | ((uint32_t)lut[sb1 & 0xFFFFu] << 16);
      } else {
        a[m] = halves_sum2(mask_xor(hash_x<false>(sa0, clo, chi)),
                           mask_xor(hash_x<false>(sb0, clo, chi)));
        a[m + 1] = halves_sum2(mask_xor(hash_x<false>(sa1, clo, chi)),
                               mask_xor(hash_x<false>(sb1, clo, chi)));
      }
    }
  }
  return a;
}

__device__ __forceinline__ f32x4_t mma16(u32x4_t a, u32x4_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a),
                                                __builtin_bit_cast(half8_t, b), c, 0, 0, 0);
}

// Decode the lane's tile of one wave-step and accumulate it into acc[ci]
// (NCOL accumulators) with 2 * NCOL MFMAs; b0 / b1: the lane's B operands
// (input words 0..3 and 4..7 of its kt).
template <int K, bool LUT = false>
__device__ __forceinline__ void mma_tile(const LaneWords<K>& lw, uint32_t wprev, u32x4_t b0,
                                         u32x4_t b1, f32x4_t* acc, const uint16_t* lut = nullptr) {
  using G = Geo<K>;
#pragma unroll
  for (int ci = 0; ci < G::NCOL; ++ci) {
    acc[ci] = mma16(mma_a_operand<K, LUT>(lw, wprev, ci, 0, lut), b0, acc[ci]);
    acc[ci] = mma16(mma_a_operand<K, LUT>(lw, wprev, ci, 1, lut), b1, acc[ci]);
  }
}

__device__ __forceinline__ uint32_t pack2(half_t a, half_t b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}
__device__ __forceinline__ void st_coherent(float* p, float v) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __builtin_bit_cast(uint32_t, v),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coherent2(float* p, float a, float b) {
  const uint64_t v = (uint64_t)__builtin_bit_cast(uint32_t, a) |
                     ((uint64_t)__builtin_bit_cast(uint32_t, b) << 32);
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// two consecutive floats; COH: device-coherent (for a consumer in the same launch)
template <bool COH>
__device__ __forceinline__ void st_pair(float* p, float a, float b) {
  if constexpr (COH)
    st_coherent2(p, a, b);
  else
    *reinterpret_cast<float2*>(p) = make_float2(a, b);
}

// Store one token's D values of a wave-step's tile-lane group: lane 16g + c
// holds tile-lanes i = 4g + r (r = 0..3).  dst: column 0 of the step's first
// tile in the token's output row.
template <int K, bool COH = false>
__device__ __forceinline__ void mma_store(const f32x4_t* acc, int g, float* dst) {
  if constexpr (K == 2) {
    // tile g, lane q = r: columns 2r + {0,1} (slots 0,1), 8 + 2r + {0,1} (slots 2,3)
    float* d = dst + 16 * g;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      st_pair<COH>(d + 2 * r, acc[0][r], acc[1][r]);
      st_pair<COH>(d + 8 + 2 * r, acc[2][r], acc[3][r]);
    }
  } else {
    // tile g/2, lanes q = 4(g&1) + r: columns q (slot 0) and q + 8 (slot 1)
    float* d = dst + 16 * (g >> 1) + 4 * (g & 1);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      st_pair<COH>(d + 8 * h, acc[h][0], acc[h][1]);
      st_pair<COH>(d + 8 * h + 2, acc[h][2], acc[h][3]);
    }
  }
}

// The previous lane's word within each quad of lanes (a tile's 4 lanes).
__device__ __forceinline__ uint32_t quad_prev_word(uint32_t w) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)w, (int)w, 0x93, 0xF, 0xF, false);  // [3,0,1,2]
}

// One f16 of the decode table in LDS at byte address addr (zero-extended).
typedef __attribute__((address_space(3))) const uint16_t lds_u16_t;
__device__ __forceinline__ uint32_t lds_u16(uint32_t addr) { return *(lds_u16_t*)(size_t)addr; }

// K=2 tile decode with NT of every 8 step pairs from the 65,536-entry table
// in LDS (at byte address tb) and the rest by hash (as fast_tile_packed).
// Table pair: the two states' byte addresses come from v_mad_u32_u16 (the
// state's half selected by op_sel, times 2, plus the table base), two
// ds_read_u16 fetch the f16 values and one v_lshl_or_b32 packs them: 3 VALU
// per pair against 8 for the hash, so the LDS pipe takes part of the decode.
// (A d16 read into each half of one register would save the pack, but with
// SRAM ECC on -- as on MI355X -- d16 loads zero the other half.)  The table
// is the hash's image and the pairs are accumulated in step order, as in
// fast_tile_packed: the result is bit-identical to it for every NT.  The
// table pairs are the last NT of each 8 and their reads are issued first, so
// their latency overlaps the group's hash pairs.
template <int NT>
__device__ __forceinline__ void fast_tile_mix(const LaneWords<2>& lw, uint32_t wprev,
                                              const uint32_t* xp, float* acc, uint32_t tb) {
  const uint32_t clo = kClo, chi = kChi;
  // pair k (0..31) is step u = 16 (k / 8) + k % 8 with step u + 8; pairs
  // k % 8 >= 8 - NT come from the table
  auto step_of = [](int k) { return 16 * (k >> 3) + (k & 7); };
  uint32_t tlo[32], thi[32];
#pragma unroll
  for (int k = 0; k < 32; ++k) {
    if ((k & 7) < 8 - NT) continue;
    const uint32_t p = window2(lw, wprev, step_of(k));
    uint32_t a_lo, a_hi;
    __asm__("v_mad_u32_u16 %0, %1, 2, %2" : "=v"(a_lo) : "v"(p), "v"(tb));
    __asm__("v_mad_u32_u16 %0, %1, 2, %2 op_sel:[1,0,0,0]" : "=v"(a_hi) : "v"(p), "v"(tb));
    tlo[k] = lds_u16(a_lo);  // step u + 8 (low half)
    thi[k] = lds_u16(a_hi);  // step u (high half)
  }
  // every table read issued here, before the hash work: the hash reads its
  // code words through this barrier (the compiler would otherwise hoist the
  // hash above the reads, sink each read next to its use and wait on it at
  // once)
  LaneWords<2> lh = lw;
  uint32_t wph = wprev;
  if constexpr (NT > 0)
    __asm__ volatile("" : "+v"(lh.w[0]), "+v"(lh.w[1]), "+v"(lh.w[2]), "+v"(lh.w[3]), "+v"(wph)
                     :
                     : "memory");
  // every hash pair first (into registers), then the table values: their
  // wait lands after all the hash work; the products are then accumulated
  // in step order, as in fast_tile_packed
  uint32_t hw[32];
#pragma unroll
  for (int k = 0; k < 32; ++k) {
    if ((k & 7) >= 8 - NT) continue;
    const uint32_t p = window2(lh, wph, step_of(k));
    hw[k] = halves_sum2(mask_xor(hash_x<false>(p, clo, chi)), mask_xor(hash_x<true>(p, clo, chi)));
    if constexpr (NT > 0) __asm__ volatile("" : "+v"(hw[k]));
  }
#pragma unroll
  for (int k = 0; k < 32; ++k) {
    const int u = step_of(k);
    uint32_t w2;
    if ((k & 7) < 8 - NT) {
      w2 = hw[k];
    } else {
      __asm__ volatile("" : "+v"(tlo[k]), "+v"(thi[k]));
      w2 = (thi[k] << 16) | tlo[k];
    }
    acc[Geo<2>::col_slot(u)] = dot2(xp[xpair_index(fast_row(u))], w2, acc[Geo<2>::col_slot(u)]);
  }
}

// K=3 tile decode with NT of every 8 step pairs from the table in LDS (at
// byte address tb) and the rest by hash (as fast_tile_rows<3, false, 1>).
// The two states of a pair (steps u + 8 and u) are 24 bits apart, so each
// is extracted on its own (state3); a table pair then costs the two
// extractions, two v_mad_u32_u16 for the byte addresses (the u16 operand
// ignores the bits above the state), two ds_read_u16 and one v_lshl_or_b32,
// against the extractions and 8 VALU by hash.  Same order of the reads, the
// hash work and the products as fast_tile_mix: bit-identical to the hash
// decode for every NT.
template <int NT>
__device__ __forceinline__ void fast_tile_mix3(const LaneWords<3>& lw, uint32_t wprev,
                                               const uint32_t* xp, float* acc, uint32_t tb) {
  const uint32_t clo = kClo, chi = kChi;
  // pair k (0..15) is step u = 16 (k / 8) + k % 8 with step u + 8
  auto step_of = [](int k) { return 16 * (k >> 3) + (k & 7); };
  uint32_t tlo[16], thi[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    if ((k & 7) < 8 - NT) continue;
    const int u = step_of(k);
    const uint32_t s_lo = state3(lw, wprev, u + 8), s_hi = state3(lw, wprev, u);
    uint32_t a_lo, a_hi;
    __asm__("v_mad_u32_u16 %0, %1, 2, %2" : "=v"(a_lo) : "v"(s_lo), "v"(tb));
    __asm__("v_mad_u32_u16 %0, %1, 2, %2" : "=v"(a_hi) : "v"(s_hi), "v"(tb));
    tlo[k] = lds_u16(a_lo);
    thi[k] = lds_u16(a_hi);
  }
  LaneWords<3> lh = lw;
  uint32_t wph = wprev;
  if constexpr (NT > 0)
    __asm__ volatile("" : "+v"(lh.w[0]), "+v"(lh.w[1]), "+v"(lh.w[2]), "+v"(wph) : : "memory");
  uint32_t hw[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    if ((k & 7) >= 8 - NT) continue;
    const int u = step_of(k);
    const uint32_t s_lo = state3(lh, wph, u + 8), s_hi = state3(lh, wph, u);
    hw[k] = halves_sum2(mask_xor(hash_x<false>(s_lo, clo, chi)),
                        mask_xor(hash_x<false>(s_hi, clo, chi)));
    if constexpr (NT > 0) __asm__ volatile("" : "+v"(hw[k]));
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int u = step_of(k);
    uint32_t w2;
    if ((k & 7) < 8 - NT) {
      w2 = hw[k];
    } else {
      __asm__ volatile("" : "+v"(tlo[k]), "+v"(thi[k]));
      w2 = (thi[k] << 16) | tlo[k];
    }
    acc[Geo<3>::col_slot(u)] = dot2(xp[xpair_index(fast_row(u))], w2, acc[Geo<3>::col_slot(u)]);
  }
}

// mma_tile with the table decode from the 65,536-entry table in LDS (at byte
// address tb): the first register pair of every A operand (m = 0, as in
// mma_a_operand<K, true>) from the table, the second by hash.  In chunks of
// CH operands: every table read of the chunk is issued first (byte
// addresses by v_mad_u32_u16: the state's half selected by op_sel, times 2,
// plus the base), then the chunk's hash work, so the reads' latency is spent
// on the hash; then the operands are packed and multiplied in mma_tile's
// order.  The table is the hash's image: bit-identical to mma_tile.
template <int K, int CH = 4>
__device__ __forceinline__ void mma_tile_mix(const LaneWords<K>& lw, uint32_t wprev, u32x4_t b0,
                                             u32x4_t b1, f32x4_t* acc, uint32_t tb) {
  using G = Geo<K>;
  const uint32_t clo = kClo, chi = kChi;
  constexpr int NO = 2 * G::NCOL;  // operands (ci, P), ci major
  static_assert(NO % CH == 0, "");
#pragma unroll
  for (int o0 = 0; o0 < NO; o0 += CH) {
    uint32_t t[CH][4];  // [a[0] lo, a[0] hi, a[1] lo, a[1] hi] f16 values
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int o = o0 + j, ci = o >> 1, P = o & 1;
      const int ua = mma_step<K>(0, 2 * P, ci), ub = mma_step<K>(0, 2 * P + 1, ci);
      uint32_t ad[4];
      if constexpr (K == 2) {
        // a[0] = [w of ua | w of ub] from the windows' high halves, a[1] from the low
        const uint32_t pa = window2(lw, wprev, ua), pb = window2(lw, wprev, ub);
        __asm__("v_mad_u32_u16 %0, %1, 2, %2 op_sel:[1,0,0,0]" : "=v"(ad[0]) : "v"(pa), "v"(tb));
        __asm__("v_mad_u32_u16 %0, %1, 2, %2 op_sel:[1,0,0,0]" : "=v"(ad[1]) : "v"(pb), "v"(tb));
        __asm__("v_mad_u32_u16 %0, %1, 2, %2" : "=v"(ad[2]) : "v"(pa), "v"(tb));
        __asm__("v_mad_u32_u16 %0, %1, 2, %2" : "=v"(ad[3]) : "v"(pb), "v"(tb));
      } else {
        const uint32_t sa0 = state3(lw, wprev, ua), sb0 = state3(lw, wprev, ub);
        const uint32_t sa1 = state3(lw, wprev, ua + 8), sb1 = state3(lw, wprev, ub + 8);
        __asm__("v_mad_u32_u16 %0, %1, 2, %2" : "=v"(ad[0]) : "v"(sa0), "v"(tb));
        __asm__("v_mad_u32_u16 %0, %1, 2, %2" : "=v"(ad[1]) : "v"(sb0), "v"(tb));
        __asm__("v_mad_u32_u16 %0, %1, 2, %2" : "=v"(ad[2]) : "v"(sa1), "v"(tb));
        __asm__("v_mad_u32_u16 %0, %1, 2, %2" : "=v"(ad[3]) : "v"(sb1), "v"(tb));
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) t[j][r] = lds_u16(ad[r]);
    }
    // the hash reads its code words through this barrier (left alone, the
    // compiler hoists the hash above the reads and waits on each read at once)
    LaneWords<K> lh = lw;
    uint32_t wph = wprev;
#pragma unroll
    for (int r = 0; r < G::WPL; ++r) __asm__ volatile("" : "+v"(lh.w[r]) : : "memory");
    __asm__ volatile("" : "+v"(wph) : : "memory");
    uint32_t h[CH][2];
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int o = o0 + j, ci = o >> 1, P = o & 1;
      const int ua = mma_step<K>(2, 2 * P, ci), ub = mma_step<K>(2, 2 * P + 1, ci);
      if constexpr (K == 2) {
        const uint32_t pa = window2(lh, wph, ua), pb = window2(lh, wph, ub);
        h[j][0] = halves_sum2(mask_xor(hash_x<true>(pa, clo, chi)), mask_xor(hash_x<true>(pb, clo, chi)));
        h[j][1] = halves_sum2(mask_xor(hash_x<false>(pa, clo, chi)), mask_xor(hash_x<false>(pb, clo, chi)));
      } else {
        const uint32_t sa0 = state3(lh, wph, ua), sb0 = state3(lh, wph, ub);
        const uint32_t sa1 = state3(lh, wph, ua + 8), sb1 = state3(lh, wph, ub + 8);
        h[j][0] = halves_sum2(mask_xor(hash_x<false>(sa0, clo, chi)), mask_xor(hash_x<false>(sb0, clo, chi)));
        h[j][1] = halves_sum2(mask_xor(hash_x<false>(sa1, clo, chi)), mask_xor(hash_x<false>(sb1, clo, chi)));
      }
      __asm__ volatile("" : "+v"(h[j][0]), "+v"(h[j][1]));
    }
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int o = o0 + j, ci = o >> 1, P = o & 1;
      __asm__ volatile("" : "+v"(t[j][0]), "+v"(t[j][1]), "+v"(t[j][2]), "+v"(t[j][3]));
      u32x4_t a;
      a[0] = t[j][0] | (t[j][1] << 16);
      a[1] = t[j][2] | (t[j][3] << 16);
      a[2] = h[j][0];
      a[3] = h[j][1];
      acc[ci] = mma16(a, P ? b1 : b0, acc[ci]);
    }
  }
}

// One wave's share of the split-K row-group GEMM on the matrix core: tiles
// [tile0, tile0 + 16/LPT) of the stream at code_e over kt [z*KS, (z+1)*KS),
// B column c = input row xr_c (the lane's row, xr), accumulated into acc.
template <int K, bool LUT>
__device__ __forceinline__ void rows_mma_accum(const uint16_t* __restrict__ xh,
                                               const uint32_t* __restrict__ code_e, int xr,
                                               int TK, int TN, int KS, int z, int tile0,
                                               const uint16_t* s_lut, f32x4_t* acc) {
  using G = Geo<K>;
  const int lane = threadIdx.x & 63;
  const int gk = lane >> 4, tc = (lane & 15) / G::LPT, q = lane % G::LPT;
  const int src = (lane & ~(G::LPT - 1)) | ((lane + G::LPT - 1) & (G::LPT - 1));
  const uint4* xq = reinterpret_cast<const uint4*>(xh + (size_t)xr * TK * 16);
  const size_t kstride = (size_t)TN * (8 * K);
  const uint32_t* lp = code_e + (size_t)(tile0 + tc) * (8 * K) + q * G::WPL;
  const int kt0 = z * KS + gk, nsteps = KS / 4;
#pragma unroll
  for (int i = 0; i < G::NCOL; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  LaneWords<K> cur = load_lane_words_nt<K>(lp + (size_t)kt0 * kstride);
  uint4 xa = xq[2 * kt0], xb = xq[2 * kt0 + 1];
  for (int k = 0; k < nsteps; ++k) {
    LaneWords<K> nxt = cur;
    uint4 na = xa, nb = xb;
    if (k + 1 < nsteps) {
      const int kt = kt0 + 4 * (k + 1);
      nxt = load_lane_words_nt<K>(lp + (size_t)kt * kstride);
      na = xq[2 * kt];
      nb = xq[2 * kt + 1];
    }
    const uint32_t wprev = __shfl(cur.w[G::WPL - 1], src);
    mma_tile<K, LUT>(cur, wprev, __builtin_bit_cast(u32x4_t, xa), __builtin_bit_cast(u32x4_t, xb),
                     acc, s_lut);
    cur = nxt;
    xa = na;
    xb = nb;
  }
}

// Split-K GEMM for up to 16 rows sharing every decoded weight, on the matrix
// core (rows_mma_accum; B column c = row c of the group): part[z][row][OC] as
// k_gemv_fast.  grid (ceil(TN/TPW), n_groups, S), block 256; wave w owns tiles
// [TPW*x + (16/LPT)*w, +16/LPT) over the block's KS kt (KS % 4 == 0), so no
// cross-wave reduction.  Dense (rows_idx null): group g is rows gR..gR+R-1 of
// one stream; rows past M read row M-1 and are not stored.  Grouped
// (moe.build_groups layout, escha_mlx/moe.py:30-78): group g holds rows
// rows_idx[gR..gR+R) of expert group_expert[g] (code stacked [E][TK][TN][8K]);
// padding rows (== M) compute on row 0 and are not stored, groups of expert -1
// do nothing.
template <int K, bool LUT, int R>
__global__ __launch_bounds__(256) void k_gemv_fast_rows(const uint16_t* __restrict__ xh,
                                                        const uint32_t* __restrict__ code,
                                                        const int* __restrict__ rows_idx,
                                                        const int* __restrict__ group_expert,
                                                        int M, int TK, int TN, int KS,
                                                        float* __restrict__ part) {
  static_assert(R >= 1 && R <= 16, "");
  using G = Geo<K>;
  constexpr int TPS = 16 / G::LPT;
  const int grp = blockIdx.y;
  const int e = group_expert ? group_expert[grp] : 0;
  if (e < 0) return;  // whole block: no barrier reached
  __shared__ uint16_t s_lut[LUT ? 65536 : 1];
  stage_lut<LUT>(s_lut);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int tile0 = blockIdx.x * G::TPW + TPS * wave;
  if (tile0 >= TN) return;  // whole wave (TN is a multiple of TPS)
  const int gk = lane >> 4, c = lane & 15;
  // the lane's B column: row min(c, R-1) of the group
  const int rc = c < R ? c : R - 1;
  const int row = rows_idx ? rows_idx[grp * R + rc] : min(grp * R + rc, M);
  const int xr = row < M ? row : (rows_idx ? 0 : M - 1);
  f32x4_t acc[G::NCOL];
  rows_mma_accum<K, LUT>(xh, code + (size_t)e * TK * TN * (8 * K), xr, TK, TN, KS, blockIdx.z,
                         tile0, s_lut, acc);
  if (c < R && row < M)
    mma_store<K>(acc, gk, part + ((size_t)blockIdx.z * M + row) * TN * 16 + 16 * tile0);
}

// Partial GEMV: part[z][row][OC] = sum over the block's kt range.
// grid (TN/TPW, M, S), block 256; KS = TK/S kt per block, KS % 4 == 0.
// row_expert null -> dense (single stream).
template <int K, bool LUT>
__global__ __launch_bounds__(256) void k_gemv_fast(const uint16_t* __restrict__ xh,
                                                   const uint32_t* __restrict__ code,
                                                   const int* __restrict__ row_expert, int M,
                                                   int TK, int TN, int KS,
                                                   float* __restrict__ part) {
  using G = Geo<K>;
  __shared__ uint16_t s_lut[LUT ? 65536 : 1];
  __shared__ float s_red[4][64][G::NCOL];
  stage_lut<LUT>(s_lut);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int ntg = blockIdx.x, row = blockIdx.y, z = blockIdx.z;
  const int IC = TK * 16, OC = TN * 16;
  const int e = row_expert ? row_expert[row] : 0;
  const uint32_t* base = code + (size_t)e * TK * TN * (8 * K);
  const int q = lane % G::LPT, tile = lane / G::LPT;
  const int src = tile * G::LPT + (q + G::LPT - 1) % G::LPT;
  // a partial last tile group (TN not a multiple of TPW): those lanes neither
  // load nor store
  const bool valid = ntg * G::TPW + tile < TN;
  const int KW = KS / 4;
  const int kt0 = z * KS + wave * KW;
  const uint32_t* xrow = reinterpret_cast<const uint32_t*>(xh + (size_t)row * IC);
  float acc[G::NCOL];
#pragma unroll
  for (int i = 0; i < G::NCOL; ++i) acc[i] = 0.f;
  const size_t lane_off = (size_t)ntg * G::TPW * (8 * K) + (size_t)lane * G::WPL;
  LaneWords<K> zero{};
  LaneWords<K> cur = valid ? load_lane_words_nt<K>(base + (size_t)kt0 * TN * (8 * K) + lane_off) : zero;
  for (int k = 0; k < KW; ++k) {
    const int kt = kt0 + k;
    LaneWords<K> nxt = cur;
    if (valid && k + 1 < KW)
      nxt = load_lane_words_nt<K>(base + (size_t)(kt + 1) * TN * (8 * K) + lane_off);
    uint32_t xw[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) xw[i] = xrow[8 * kt + i];
    const uint32_t wprev = __shfl(cur.w[G::WPL - 1], src);
    if constexpr (LUT) {
      fast_tile<K, true>(cur, wprev, xw, s_lut, acc);
    } else {
      uint32_t xp[8];
      x_pairs(xw, xp);
      fast_tile_packed<K>(cur, wprev, xp, acc);
    }
    cur = nxt;
  }
#pragma unroll
  for (int i = 0; i < G::NCOL; ++i) s_red[wave][lane][i] = acc[i];
  __syncthreads();
  if (wave == 0 && valid) {
    float* pr = part + ((size_t)z * M + row) * OC + (size_t)(ntg * G::TPW + tile) * 16;
#pragma unroll
    for (int i = 0; i < G::NCOL; ++i) {
      float v = s_red[0][lane][i];
      v = v + s_red[1][lane][i];
      v = v + s_red[2][lane][i];
      v = v + s_red[3][lane][i];
      pr[G::col(q, i)] = v;
    }
  }
}

// out[row] = f16((H128(sum_z part[z][row]) * RS) * rout[e]); grid (OC/128, M), block 64.
__global__ __launch_bounds__(64) void k_splitk_out(const float* __restrict__ part, int S, int M,
                                                   int OC, const float* __restrict__ rout,
                                                   const int* __restrict__ row_expert, float rs,
                                                   uint16_t* __restrict__ out) {
  const int blk = blockIdx.x, row = blockIdx.y, lane = threadIdx.x;
  const int c = blk * 128 + 2 * lane;
  float v0 = 0.f, v1 = 0.f;
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
  const float* r = rout + (row_expert ? (size_t)row_expert[row] * OC : 0) + c;
  out[(size_t)row * OC + c] = __builtin_bit_cast(uint16_t, to_f16((v0 * rs) * r[0]));
  out[(size_t)row * OC + c + 1] = __builtin_bit_cast(uint16_t, to_f16((v1 * rs) * r[1]));
}

}  // namespace esc
