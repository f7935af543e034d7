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
//     column, straight into the f16 B operand layout in LDS.
//   * X: the block's 256 rows x 32 inputs are staged to LDS once per stage.
//   * MFMA: wave (wm, wn) owns rows 128wm.. and columns 64wn..; per kt it runs
//     4 x 2 v_mfma_f32_32x32x16_f16 (A: lane l holds row l%32, inputs
//     8(l/32)..+7; B: inputs 8(l/32)..+7 of column l%32; D register r of lane
//     l is row 8(r/4) + 4(l/32) + r%4, column l%32).
// The decode of stage s+1 is issued between the MFMAs of stage s, so the
// VALU (decode) and the matrix pipe overlap.  LDS chunks are XOR-swizzled so
// the 16-byte fragment reads and writes hit distinct banks.
#pragma once

#include "fast.hpp"

namespace esc {

typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr int kMmaRows = 256;           // rows per block
constexpr int kMmaCols = 128;           // columns per block (8 tiles)
constexpr int kMmaPitch = 32;           // halves per LDS row: 2 kt x 16 inputs

// LDS row r holds one stage (2 kt) of one input row (s_x) or one column
// (s_b) as four 16-byte chunks c = 2*kt + half; chunk c is stored at
// position c ^ swz(r).  Every access pattern of the kernel (16 consecutive
// rows at one chunk; 4 rows x 4 chunks) then touches distinct bank groups,
// for 8- and 16-lane phases alike.
__device__ __forceinline__ int swz(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }
__device__ __forceinline__ int lds_off(int r, int c) { return r * kMmaPitch + 8 * (c ^ swz(r)); }
constexpr int kMmaThreads = 256;

// Raw buffer resource over [p, p + bytes) (gfx9 descriptor word 3); loads
// through it take a scalar base and a 32-bit lane offset, and read zero past
// the end instead of faulting.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* p, size_t bytes) {
  const int n = bytes > 0xFFFFFFF0u ? (int)0xFFFFFFF0u : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, n, 0x00020000);
}

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

  // ---- decode role: (column n, half h) of each kt; wave w decodes half
  // h = w & 1 of tiles 4(w >> 1)..+3, 16 consecutive columns per 16 lanes
  const int h = wave & 1;
  const int ti = 4 * (wave >> 1) + (lane >> 4), c16 = lane & 15;
  const int n = 16 * ti + c16;
  const int jhi = c16 >> 3, a3 = (c16 >> 1) & 3, bq = c16 & 1;  // c16 = 2(a3 + 4jhi) + bq
  int st0 = K * (64 * a3 + 32 * bq + 4 * jhi + 2 * h) - (16 - K);
  if (st0 < 0) st0 += 256 * K;
  const uint32_t o = (uint32_t)(st0 & 31);  // 1..31: never 0 (K=2: 18..30, K=3: 5..31)
  // loads go through buffer resources: a scalar base, a scalar per-stage
  // offset and a constant 32-bit lane offset, so the loop spends no VALU on
  // addresses
  uint32_t loff[NW];  // byte offsets of the lane's words within a kt row of the block
#pragma unroll
  for (int k = 0; k < NW; ++k) loff[k] = 4u * (ti * WPT + ((st0 >> 5) + k) % WPT);
  const uint32_t kstride = 4u * TN * WPT;  // bytes per kt row
  const __amdgpu_buffer_rsrc_t crs =
      buf_rsrc(code + (size_t)(8 * cb) * WPT, (size_t)TK * kstride - (size_t)(8 * cb) * WPT * 4);

  // ---- X role: rows 64i + tid/4, 16-byte chunk tid%4 of the stage's 64 bytes
  const int xchunk = tid & 3;
  uint32_t xoff[4];  // byte offsets (M * IC * 2 < 2^32)
#pragma unroll
  for (int i = 0; i < 4; ++i)
    xoff[i] = 2u * ((uint32_t)min(row0 + 64 * i + (tid >> 2), M - 1) * IC + 8 * xchunk);
  const __amdgpu_buffer_rsrc_t xrs = buf_rsrc(xh, (size_t)M * IC * 2);

  // global -> register staging of one stage, two sets in flight: the loads
  // of stage s+2 are issued two MFMA phases before their data is needed
  struct Regs {
    uint32_t cw[2][NW];
    uint4 xv[4];
  };
  auto load_stage = [&](Regs& r, int s) {
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      const uint32_t so = (uint32_t)(2 * s + k2) * kstride;
#pragma unroll
      for (int k = 0; k < NW; ++k)
        r.cw[k2][k] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(crs, loff[k], so, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(xrs, xoff[i], 64u * s, 0);
      r.xv[i] = make_uint4(v[0], v[1], v[2], v[3]);
    }
  };
  auto store_stage = [&](const Regs& r, int buf) {
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      const uint4 v = mma_decode8<K>(r.cw[k2], o);
      *reinterpret_cast<uint4*>(&s_b[buf][lds_off(n, 2 * k2 + h)]) = v;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<uint4*>(&s_x[buf][lds_off(64 * i + (tid >> 2), xchunk)]) =
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
            &s_x[buf][lds_off(128 * wm + 32 * i + (lane & 31), 2 * k2 + (lane >> 5))]);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        b[j] = *reinterpret_cast<const half8_t*>(
            &s_b[buf][lds_off(64 * wn + 32 * j + (lane & 31), 2 * k2 + (lane >> 5))]);
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

// Coded GEMM with the weights decoded straight into MFMA A operands (no LDS
// for weights): mid[M][OC] f32 = xh[M][IC] f16 @ decode(code), for OC a
// multiple of 256.  Same tolerance contract as k_gemm_mfma.
//
// Block = 4 waves, tile 16*NRB rows x 256 columns (16 code tiles); wave w owns
// tiles 4w..4w+3 (64 columns).  K is walked in steps of 4 kt (64 inputs):
//   * each lane decodes its tile-lane of the wave-step (mma_a_operand: 4
//     column groups x 2 input halves = 8 A operands, v_mfma_f32_16x16x32_f16
//     layout, one kt per 16 lanes), so each weight is decoded once per block;
//   * X: the block's rows x 64 inputs are staged through LDS (double
//     buffered, 16-byte chunks XOR-swizzled by row); a B operand is one
//     16-byte read (16 rows x 8 inputs of one kt per 16 lanes) and feeds the
//     4 A operands of its input half;
//   * each A operand meets NRB row blocks: 8 * NRB MFMAs per wave-step, in
//     one straight-line body with the decode of the next wave-step, so the
//     matrix pipe and the VALU overlap (two workgroups per CU).
// The kernel is decode-bound: the host picks NRB for the shape.
// D register r of lane l: output column of tile-lane 4(l/16) + r, row l%16 of
// the row block.
// OUT: the output transform is fused into the epilogue (y f16 = (bias +)
// f16((H128(row) * rs) * rout), the formula of k_output_transform): per 16-row
// block the two waves of each 128-column block exchange their 64 columns
// through LDS and each transforms 8 rows; mid is not written.
template <int K, int NRB, bool OUT = false>
__global__ __launch_bounds__(256, 2) void k_gemm_mma2(
    const uint16_t* __restrict__ xh, const uint32_t* __restrict__ code, int M, int TK, int TN,
    float* __restrict__ mid, const float* __restrict__ rout = nullptr,
    const uint16_t* __restrict__ bias = nullptr, float rs = 0.f, uint16_t* __restrict__ y = nullptr) {
  using G = Geo<K>;
  constexpr int TPS = 16 / G::LPT, GPW = 4 / TPS, NA = GPW * G::NCOL;
  static_assert(NA == 4, "four 16-column groups per wave");
  static_assert(NRB % 2 == 0 && NRB >= 2 && NRB <= 8, "whole x chunks per thread, 2 waves/SIMD");
  constexpr int BR = 16 * NRB;            // rows per block
  constexpr int XCH = BR * 8 / 256;       // 16-byte x chunks per thread per stage
  __shared__ uint4 s_x[2][BR * 8];        // [stage][row][chunk ^ (row & 7)]

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int IC = TK * 16, OC = TN * 16;
  const int ncb = TN / 16;
  int rb, cb;
  if (ncb % 8 == 0) {
    const int per = ncb / 8, qq = blockIdx.x / 8, x = blockIdx.x % 8;
    rb = qq / per;
    cb = 8 * (qq % per) + x;
  } else {
    rb = blockIdx.x / ncb;
    cb = blockIdx.x % ncb;
  }
  const int row0 = rb * BR;
  const int tile0 = cb * 16 + 4 * wave;
  const int gk = lane >> 4, c = lane & 15, tc = c / G::LPT, q = lane % G::LPT;
  const int src = (lane & ~(G::LPT - 1)) | ((lane + G::LPT - 1) & (G::LPT - 1));

  // code: tile group tg of the wave, lane's kt = 4s + gk
  const size_t kstride = (size_t)TN * (8 * K);
  const uint32_t* cbase = code + (size_t)(tile0 + tc) * (8 * K) + q * G::WPL + gk * kstride;
  auto load_code = [&](LaneWords<K>* cw, int s) {
#pragma unroll
    for (int tg = 0; tg < GPW; ++tg)
      cw[tg] = load_lane_words<K>(cbase + (size_t)tg * TPS * (8 * K) + (size_t)(4 * s) * kstride);
  };
  // x: chunk e = tid + 256j of a stage is row e/8, logical chunk (e%8)^(row&7)
  // = kt (lc/2) half (lc%2), 128 bytes per row per stage
  uint32_t xoff[XCH];
#pragma unroll
  for (int j = 0; j < XCH; ++j) {
    const int e = tid + 256 * j, r = e >> 3, lc = (e & 7) ^ (r & 7);
    xoff[j] = 2u * ((uint32_t)min(row0 + r, M - 1) * IC) + 16u * lc;
  }
  const __amdgpu_buffer_rsrc_t xrs = buf_rsrc(xh, (size_t)M * IC * 2);
  auto load_x = [&](uint4* xr, int s) {
#pragma unroll
    for (int j = 0; j < XCH; ++j) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(xrs, xoff[j], 128u * s, 0);
      xr[j] = make_uint4(v[0], v[1], v[2], v[3]);
    }
  };
  auto store_x = [&](const uint4* xr, int buf) {
#pragma unroll
    for (int j = 0; j < XCH; ++j) s_x[buf][tid + 256 * j] = xr[j];
  };

  f32x4_t acc[NA][NRB];
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int r = 0; r < NRB; ++r) acc[a][r] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // software pipeline: the MFMAs of step s and the decode of step s+1 sit in
  // one straight-line body (the matrix pipe and the VALU overlap); loads past
  // the last step re-read it (in bounds, never used)
  const int NS = TK / 4;
  auto decode_step = [&](const LaneWords<K>* w, u32x4_t (*Ad)[2]) {
#pragma unroll
    for (int tg = 0; tg < GPW; ++tg) {
      const uint32_t wprev = __shfl(w[tg].w[G::WPL - 1], src);
#pragma unroll
      for (int ci = 0; ci < G::NCOL; ++ci)
#pragma unroll
        for (int P = 0; P < 2; ++P) Ad[tg * G::NCOL + ci][P] = mma_a_operand<K>(w[tg], wprev, ci, P);
    }
  };
  LaneWords<K> cw[GPW];
  uint4 xr[XCH];
  u32x4_t A[NA][2];
  load_code(cw, 0);
  load_x(xr, 0);
  store_x(xr, 0);
  decode_step(cw, A);
  load_code(cw, min(1, NS - 1));
  lds_barrier();
  for (int s = 0; s < NS; ++s) {
    const int buf = s & 1;
    load_x(xr, min(s + 1, NS - 1));
    LaneWords<K> cn[GPW];
    load_code(cn, min(s + 2, NS - 1));
    u32x4_t An[NA][2];
#pragma unroll
    for (int P = 0; P < 2; ++P)
#pragma unroll
      for (int r = 0; r < NRB; ++r) {
        const uint4 bv = s_x[buf][(16 * r + c) * 8 + ((2 * gk + P) ^ (c & 7))];
        const u32x4_t b = __builtin_bit_cast(u32x4_t, bv);
#pragma unroll
        for (int a = 0; a < NA; ++a) acc[a][r] = mma16(A[a][P], b, acc[a][r]);
      }
    decode_step(cw, An);
    store_x(xr, buf ^ 1);
#pragma unroll
    for (int a = 0; a < NA; ++a) {
      A[a][0] = An[a][0];
      A[a][1] = An[a][1];
    }
#pragma unroll
    for (int tg = 0; tg < GPW; ++tg) cw[tg] = cn[tg];
    lds_barrier();
  }

  if constexpr (!OUT) {
#pragma unroll
    for (int r = 0; r < NRB; ++r) {
      const int row = row0 + 16 * r + c;
      if (row < M) {
#pragma unroll
        for (int tg = 0; tg < GPW; ++tg) {
          f32x4_t t[G::NCOL];
#pragma unroll
          for (int ci = 0; ci < G::NCOL; ++ci) t[ci] = acc[tg * G::NCOL + ci][r];
          mma_store<K>(t, gk, mid + (size_t)row * OC + 16 * (tile0 + TPS * tg));
        }
      }
    }
  } else {
    constexpr int kPitch = 128 + 4;  // floats per staged row
    static_assert(sizeof(s_x) >= 2 * 16 * kPitch * sizeof(float) || NRB < 6, "");
    __shared__ float s_o[NRB < 6 ? 2 * 16 * kPitch : 1];
    float* so = NRB < 6 ? s_o : reinterpret_cast<float*>(&s_x[0][0]);
    const int pair = wave >> 1, hw = wave & 1;
    float* sp = so + pair * 16 * kPitch;
    const int col0 = 256 * cb + 128 * pair;  // the pair's 128-column block
#pragma unroll
    for (int r = 0; r < NRB; ++r) {
      // this wave's 64 columns of rows 16r..16r+15 into the pair's LDS block
#pragma unroll
      for (int tg = 0; tg < GPW; ++tg)
#pragma unroll
        for (int ci = 0; ci < G::NCOL; ++ci)
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            const int i = 4 * gk + rr, tc = i / G::LPT, q = i % G::LPT;
            sp[c * kPitch + 64 * hw + 16 * (TPS * tg + tc) + G::col(q, ci)] =
                acc[tg * G::NCOL + ci][r][rr];
          }
      __syncthreads();
#pragma unroll 2
      for (int j = 0; j < 8; ++j) {
        const int rl = 8 * hw + j, row = row0 + 16 * r + rl;
        float v0 = sp[rl * kPitch + 2 * lane], v1 = sp[rl * kPitch + 2 * lane + 1];
        h128_wave(v0, v1);
        const int col = col0 + 2 * lane;
        half_t y0 = to_f16((v0 * rs) * rout[col]);
        half_t y1 = to_f16((v1 * rs) * rout[col + 1]);
        if (bias) {
          y0 = to_f16((float)y0 + (float)__builtin_bit_cast(half_t, bias[col]));
          y1 = to_f16((float)y1 + (float)__builtin_bit_cast(half_t, bias[col + 1]));
        }
        if (row < M)
          *reinterpret_cast<uint32_t*>(y + (size_t)row * OC + col) = pack2(y0, y1);
      }
      __syncthreads();
    }
  }
}

}  // namespace esc
