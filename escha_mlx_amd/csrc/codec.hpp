// escha trellis codec for gfx950: format constants, state windows, lane map,
// hash / table decode.  Shared by every kernel of libescha_hip.
//
// Format (escha_mlx/ref.py:10-11, 37-48, 58-134):
//   * a projection with IC inputs / OC outputs is code[IC/16][OC/16][8K] uint32
//     (the int16 export viewed little-endian; MoE stacks prepend E);
//   * tile (kt, nt) holds W[16kt:16kt+16, 16nt:16nt+16] of W [IC, OC], y = x @ W;
//   * a tile's 8K words form one circular bitstream of 256K bits, word 0 bit 31
//     first; trellis step t's 16-bit state is the window of bits
//     [K(t+1)-16, K(t+1)) mod 256K read MSB-first;
//   * step t = 8L + j sits at row 2(L&3) + (j&1) + 8((j>>1)&1),
//     col 2((L>>3) + 4[j>=4]) + ((L>>2)&1) of the tile (ref.py:96-111);
//   * decode(s): r = ((s * 0xCBAC1FED) & 0x8FFF8FFF) ^ 0x3B603B60,
//     value = f16(lo16 r) + f16(hi16 r), round-to-nearest-even.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace esc {

constexpr uint32_t kHashMul = 0xCBAC1FEDu;
constexpr uint32_t kHashMask = 0x8FFF8FFFu;
constexpr uint32_t kHashXor = 0x3B603B60u;
// 1/sqrt(128) as the float32 the format pins (escha_mlx/ref.py:30).
constexpr float kRS = 0.088388347648f;

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// float32 -> f16 with the float32 value materialised first.  Without the
// barrier the backend folds fptrunc(fmul(a, b)) into v_fma_mixlo_f16, which
// rounds the exact product once to f16 instead of to f32 and then f16 — a
// different rounding point from the reference's (escha_mlx/ref.py:221-228).
__device__ __forceinline__ half_t to_f16(float x) {
  __asm__ volatile("" : "+v"(x));
  return (half_t)x;
}

// Workgroup barrier for LDS hand-offs only.  __syncthreads() also waits for
// every outstanding global load of the wave (one vmcnt counter on gfx9),
// which would stall on register prefetches issued just before it; this waits
// for the wave's LDS operations only.
__device__ __forceinline__ void lds_barrier() {
  __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  __asm__ volatile("" ::: "memory");
}

// ---------------------------------------------------------------- lane map
// Row / column of trellis step t inside its 16x16 tile.
__host__ __device__ constexpr int step_row(int t) {
  return 2 * ((t >> 3) & 3) + ((t & 7) & 1) + 8 * (((t & 7) >> 1) & 1);
}
__host__ __device__ constexpr int step_col(int t) {
  return 2 * (((t >> 3) >> 3) + 4 * ((t & 7) >= 4)) + (((t >> 3) >> 2) & 1);
}

// ---------------------------------------------------------------- decode
// The 32-bit hash word whose two f16 halves sum to the decoded weight.
__device__ __forceinline__ uint32_t hash_word(uint32_t s) {
  uint32_t x = s * kHashMul;
  return (x & kHashMask) ^ kHashXor;
}

__device__ __forceinline__ half_t halves_sum(uint32_t r) {
  half_t lo = __builtin_bit_cast(half_t, (uint16_t)(r & 0xFFFFu));
  half_t hi = __builtin_bit_cast(half_t, (uint16_t)(r >> 16));
  return lo + hi;  // f16 add, RNE (default rounding mode)
}

__device__ __forceinline__ half_t decode_hash(uint32_t s) {
  return halves_sum(hash_word(s));
}

__device__ __forceinline__ uint16_t decode_hash_bits(uint32_t s) {
  return __builtin_bit_cast(uint16_t, decode_hash(s));
}

// 16-bit state whose window starts `start` bits into the 64-bit MSB-first
// funnel {hi, lo}; any 0 <= start <= 48 keeps the window inside the pair.
__device__ __forceinline__ uint32_t window16(uint32_t hi, uint32_t lo, int start) {
  uint64_t m = ((uint64_t)hi << 32) | lo;
  return (uint32_t)(m >> (48 - start)) & 0xFFFFu;
}

// State of trellis step t of a tile whose words are reachable through `w(i)`.
template <int K, typename WordFn>
__device__ __forceinline__ uint32_t step_state(WordFn w, int t) {
  constexpr int kBits = 256 * K;
  constexpr int kWords = 8 * K;
  int start = (K * (t + 1) - 16 + kBits) % kBits;
  int a = start >> 5;
  return window16(w(a), w((a + 1) % kWords), start & 31);
}

// Table decode: 65,536 f16 values, built on the device by the hash itself
// (bit-identical by construction) and staged through LDS by the kernels that
// use it.  One copy per device, filled once by esc_init().
__device__ uint16_t g_lut[65536];

// Copying the table into LDS: 8,192 pieces of 16 bytes.  A load-then-store
// loop waits one round trip to L2 per piece a thread copies; these issue
// eight loads before the first store, so a workgroup of B threads (B dividing
// 1024) waits 1024 / B round trips.
constexpr int kTablePieces = 65536 / 8;
__device__ __forceinline__ void copy_table(uint16_t* s_dst) {
  const uint4* src = reinterpret_cast<const uint4*>(g_lut);
  uint4* dst = reinterpret_cast<uint4*>(s_dst);
  const int nt = blockDim.x;
  for (int i0 = threadIdx.x; i0 < kTablePieces; i0 += 8 * nt) {
    uint4 v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = src[i0 + k * nt];
#pragma unroll
    for (int k = 0; k < 8; ++k) dst[i0 + k * nt] = v[k];
  }
}
// The same for a workgroup of exactly 1024 threads, in two halves, so that
// other loads can be issued between them: table_fetch (the thread's eight
// pieces into registers) and table_put (into LDS).
struct TablePieces {
  uint4 v[8];
};
__device__ __forceinline__ void table_fetch(TablePieces& t) {
  const uint4* src = reinterpret_cast<const uint4*>(g_lut);
#pragma unroll
  for (int k = 0; k < 8; ++k) t.v[k] = src[threadIdx.x + 1024 * k];
}
__device__ __forceinline__ void table_put(const TablePieces& t, uint16_t* s_dst) {
  uint4* dst = reinterpret_cast<uint4*>(s_dst);
#pragma unroll
  for (int k = 0; k < 8; ++k) dst[threadIdx.x + 1024 * k] = t.v[k];
}
// The same copy for a workgroup of 16 waves through the LDS DMA path
// (global_load_lds_dwordx4): each wave's eight loads write their 1 KiB pieces
// straight into LDS (lane i's 16 bytes at the wave's base + 16 i), so no
// register holds the table and the wave can decode meanwhile.  The loads
// count against vmcnt: the caller waits for them (s_waitcnt vmcnt(0)) before
// the barrier after which the table is read.
__device__ __forceinline__ void table_dma(uint16_t* s_dst) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const char* src = reinterpret_cast<const char*>(g_lut);
  char* dst = reinterpret_cast<char*>(s_dst);
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int piece = (16 * k + wave) * 1024;  // bytes
    __builtin_amdgcn_global_load_lds(
        (const __attribute__((address_space(1))) void*)(src + piece + 16 * lane),
        (__attribute__((address_space(3))) void*)(dst + piece), 16, 0, 0);
  }
}

}  // namespace esc
