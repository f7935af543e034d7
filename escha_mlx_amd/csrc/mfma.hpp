// Coded dense GEMM on the matrix cores (prefill / many rows):
//   mid[M][OC] f32 = xh[M][IC] f16 @ decode(code[IC/16][OC/16][8K]).
// Replaces msl.dense_gemm_mat (escha_mlx/msl.py:1608-1782), the reference's
// R=16 simdgroup-matrix GEMM.  Tolerance contract, as there: every decoded
// weight is the bit-exact f16 of the format, f16 x f16 products are exact in
// the f32 accumulator, and only the order of the f32 sum differs from the
// scalar kernels.  The result is deterministic run to run.
//
// Block = 256 threads (4 waves), tile 256 rows x 128 columns (8 code tiles),
// K walked in stages of 2 kt (32 inputs), double-buffered through LDS:
//   * decode: per kt each thread decodes 8 weights, rows 8h..8h+7 of one
//     column, straight into the f16 B operand layout in LDS (wave w decodes
//     half h = w & 1 of the columns with jhi = w >> 1).
//   * X: the block's 256 rows x 32 inputs are staged to LDS once per stage.
//   * MFMA: wave (wm, wn) owns rows 128wm.. and columns 64wn..; per kt it runs
//     4 x 2 v_mfma_f32_32x32x16_f16 (A: lane l holds row l%32, inputs
//     8(l/32)..+7; B: inputs 8(l/32)..+7 of column l%32; D register r of lane
//     l is row 8(r/4) + 4(l/32) + r%4, column l%32).
// The decode of stage s+1 is issued between the MFMAs of stage s, so the
// VALU (decode) and the matrix pipe overlap.  LDS rows are padded to 80 B so
// the 16-byte fragment reads of 16 consecutive rows hit distinct banks.
#pragma once

#include "fast.hpp"

namespace esc {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr int kMmaRows = 256;           // rows per block
constexpr int kMmaCols = 128;           // columns per block (8 tiles)
constexpr int kMmaPitch = 40;           // halves per LDS row: 2 kt x 16 + 8 pad
constexpr int kMmaThreads = 256;

// Code words one decode lane reads per kt: K=2 -> 3 (a 66-bit span),
// K=3 -> 4 (a 91-bit span).
template <int K>
struct MmaWords {
  static constexpr int N = K == 2 ? 3 : 4;
};

// The 8 weights of (column, half h) of one tile -> 4 words of f16 pairs in
// row order 8h+0..7.  Steps t0 + 8i + e (i = 0..3, e = 0..1) sit at row
// 8h + 2i + e; w[] holds the stream words from the one containing step t0's
// first window bit, o = that bit's offset in it.
template <int K>
__device__ __forceinline__ uint4 mma_decode8(const uint32_t (&w)[MmaWords<K>::N], uint32_t o);

template <>
__device__ __forceinline__ uint4 mma_decode8<2>(const uint32_t (&w)[3], uint32_t o) {
  // steps t and t+8 have adjacent 16-bit windows: one 32-bit funnel shift
  // gives [s_t | s_t+8] (rows r and r+2); the window of step t0+16i starts 32i
  // bits later, that of t0+e 2e bits later
  const uint32_t clo = kClo, chi = kChi;
  uint32_t p[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int i2 = q >> 1, e = q & 1;  // i = 2 * i2
    const uint32_t f = __builtin_amdgcn_alignbit(w[i2], w[i2 + 1], 32u - (o + 2u * e));
    p[q] = halves_sum2(mask_xor(hash_x<false>(f, clo, chi)), mask_xor(hash_x<true>(f, clo, chi)));
  }
  // p[q] = [w(row 4i2 + e) | w(row 4i2 + e + 2)]: regroup into row pairs
  uint4 r;
  r.x = __builtin_amdgcn_perm(p[1], p[0], 0x07060302u);  // rows 1 | 0
  r.y = __builtin_amdgcn_perm(p[1], p[0], 0x05040100u);  // rows 3 | 2
  r.z = __builtin_amdgcn_perm(p[3], p[2], 0x07060302u);  // rows 5 | 4
  r.w = __builtin_amdgcn_perm(p[3], p[2], 0x05040100u);  // rows 7 | 6
  return r;
}

// K=3: windows 3 bits apart.  The lane's words are first re-aligned so the
// stream starts at step t0's first bit (three funnel shifts by the lane's
// offset o); every state is then one shift or funnel shift at a compile-time
// position into the low half (the u16 hash ignores the bits above), so the
// decode has no branches.
template <>
__device__ __forceinline__ uint4 mma_decode8<3>(const uint32_t (&w)[4], uint32_t o) {
  const uint32_t clo = kClo, chi = kChi;
  uint32_t a3w[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) a3w[k] = __builtin_amdgcn_alignbit(w[k], w[k + 1], 32u - o);
  uint32_t r[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int i = q >> 1, e = q & 1;
    const int pos = 3 * (8 * i + e);
    const int a = pos >> 5, off = pos & 31;
    const uint32_t st = off <= 16 ? a3w[a] >> (16 - off)
                                  : __builtin_amdgcn_alignbit(a3w[a], a3w[a + 1], 48 - off);
    r[q] = mask_xor(hash_x<false>(st, clo, chi));
  }
  uint4 v;
  v.x = halves_sum2(r[0], r[1]);
  v.y = halves_sum2(r[2], r[3]);
  v.z = halves_sum2(r[4], r[5]);
  v.w = halves_sum2(r[6], r[7]);
  return v;
}

template <int K>
__global__ __launch_bounds__(kMmaThreads, 2) void k_gemm_mfma(const uint16_t* __restrict__ xh,
                                                              const uint32_t* __restrict__ code,
                                                              int M, int TK, int TN,
                                                              float* __restrict__ mid) {
  constexpr int NW = MmaWords<K>::N;
  constexpr int WPT = 8 * K;  // words per tile
  __shared__ __attribute__((aligned(16))) uint16_t s_x[2][kMmaRows * kMmaPitch];
  __shared__ __attribute__((aligned(16))) uint16_t s_b[2][kMmaCols * kMmaPitch];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int OC = TN * 16, IC = TK * 16;
  // block -> (row block, column block): all XCDs walk the same row block at
  // once, each on its own eighth of the columns, so a row block's inputs are
  // shared through each XCD's L2
  const int ncb = TN / 8;
  int rb, cb;
  if (ncb % 8 == 0) {
    const int per = ncb / 8, q = blockIdx.x / 8, x = blockIdx.x % 8;
    rb = q / per;
    cb = 8 * (q % per) + x;
  } else {
    rb = blockIdx.x / ncb;
    cb = blockIdx.x % ncb;
  }
  const int row0 = rb * kMmaRows;

  // ---- decode role: (column n, half h) of each kt
  const int jhi = wave >> 1, h = wave & 1;
  const int ti = lane >> 3, a3 = (lane >> 1) & 3, bq = lane & 1;
  const int n = 16 * ti + 2 * (a3 + 4 * jhi) + bq;
  int st0 = K * (64 * a3 + 32 * bq + 4 * jhi + 2 * h) - (16 - K);
  if (st0 < 0) st0 += 256 * K;
  const uint32_t o = (uint32_t)(st0 & 31);  // 1..31: never 0 (K=2: 18..30, K=3: 5..31)
  int woff[NW];
#pragma unroll
  for (int k = 0; k < NW; ++k) woff[k] = ((st0 >> 5) + k) % WPT;
  const uint32_t* ctile = code + (size_t)(8 * cb + ti) * WPT;  // kt = 0
  const size_t kstride = (size_t)TN * WPT;

  // ---- X role: rows 64i + tid/4, 16-byte chunk tid%4 of the stage's 64 bytes
  const int xchunk = tid & 3;
  const uint16_t* xrow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = min(row0 + 64 * i + (tid >> 2), M - 1);
    xrow[i] = xh + (size_t)r * IC + 8 * xchunk;
  }

  // global -> register staging of one stage, two sets in flight: the loads
  // of stage s+2 are issued two MFMA phases before their data is needed
  struct Regs {
    uint32_t cw[2][NW];
    uint4 xv[4];
  };
  auto load_stage = [&](Regs& r, int s) {
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      const uint32_t* tp = ctile + (size_t)(2 * s + k2) * kstride;
#pragma unroll
      for (int k = 0; k < NW; ++k) r.cw[k2][k] = tp[woff[k]];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) r.xv[i] = *reinterpret_cast<const uint4*>(xrow[i] + 32 * s);
  };
  auto store_stage = [&](const Regs& r, int buf) {
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      const uint4 v = mma_decode8<K>(r.cw[k2], o);
      *reinterpret_cast<uint4*>(&s_b[buf][n * kMmaPitch + 16 * k2 + 8 * h]) = v;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<uint4*>(&s_x[buf][(64 * i + (tid >> 2)) * kMmaPitch + 8 * xchunk]) =
          r.xv[i];
  };

  // ---- MFMA role
  const int wm = wave >> 1, wn = wave & 1;
  float16_t acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  auto mma_stage = [&](int buf) {
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      half8_t a[4], b[2];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        a[i] = *reinterpret_cast<const half8_t*>(
            &s_x[buf][(128 * wm + 32 * i + (lane & 31)) * kMmaPitch + 16 * k2 + 8 * (lane >> 5)]);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        b[j] = *reinterpret_cast<const half8_t*>(
            &s_b[buf][(64 * wn + 32 * j + (lane & 31)) * kMmaPitch + 16 * k2 + 8 * (lane >> 5)]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  };

  // Interleave one stage's 16 MFMAs with the decode of the next stage (VALU)
  // and its LDS traffic: each 32-cycle MFMA hides about six VALU issues.
  auto interleave = [] {
    __builtin_amdgcn_sched_group_barrier(0x020, 16, 0);  // global loads first
    __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);   // k2 = 0 fragments
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);   // k2 = 1 fragments
#pragma unroll
    for (int i = 0; i < 12; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
    }
  };

  // stage s lives in LDS buffer s & 1; register set r_even carries the even
  // stages, r_odd the odd ones (NS = TK / 2 is a multiple of 4).  Loads past
  // the last stage re-read the last stage (in bounds, never stored to a
  // buffer that is read again), which keeps each half straight-line code.
  const int NS = TK / 2;
  Regs r_even, r_odd;
  load_stage(r_even, 0);
  load_stage(r_odd, 1);
  store_stage(r_even, 0);
  load_stage(r_even, 2);
  lds_barrier();
  for (int s = 0; s < NS; s += 2) {
    mma_stage(0);  // stage s
    store_stage(r_odd, 1);
    load_stage(r_odd, min(s + 3, NS - 1));
    interleave();
    lds_barrier();
    mma_stage(1);  // stage s + 1
    store_stage(r_even, 0);
    load_stage(r_even, min(s + 4, NS - 1));
    interleave();
    lds_barrier();
  }

  // ---- epilogue: D register r of lane l -> row 8(r/4) + 4(l/32) + r%4, col l%32
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = row0 + 128 * wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      if (row < M) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
          mid[(size_t)row * OC + kMmaCols * cb + 64 * wn + 32 * j + (lane & 31)] = acc[i][j][r];
      }
    }
}

}  // namespace esc
