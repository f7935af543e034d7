// One-launch routed-expert path (replaces the ~10 launches of
// EschaSparseMoeBlock._expert_path, escha_mlx/models/qwen3_5_moe.py:207-253),
// for one token-layer or for a list of independent token-layers.
//
// Work is split into two kinds of items, each one block (4 waves; 16 in the
// two-launch path for one token-layer, where latency rules):
//   gate_up item (l, r, b, kc): layer l, row r, output columns
//     gate[128b, 128b+128) and up[I+128b, I+128b+128), input rows
//     [16*KTA*kc, 16*KTA*(kc+1)).  The block input-transforms its own inputs of
//     x (no global hand-off), decodes and multiplies 16 tiles x KTA kt, and
//     publishes 256 float32 partials.
//   down item (l, r, p, kb): row r, output columns [256p, 256p+256), input rows
//     [16*KTB*kb, 16*KTB*(kb+1)) of h.  It waits until every gate_up item of
//     the h-blocks it reads is published, sums their partials in fixed kc
//     order, applies the gate_up output transform, swiglu and the down input
//     transform to get its inputs, decodes and multiplies 16 tiles x KTB kt and
//     publishes 256 partials.  The last down item to finish a (token,
//     256-column) tile sums every slot's partials in fixed order, transforms
//     them and combines the slots in slot order (f16(score) weights, float32
//     sum, one f16 rounding).  No float atomics: the result is deterministic.
//   With I == 512 the two-launch path uses block down items instead
//   (k_moe_down_blocks): one per (row, 128-column block) over all 512 inputs,
//   each finishing its own output transform, so only f16 rows are combined.
//
// Two item sizes: small items (KTA=8, KTB=4) spread one token-layer over the
// whole GPU for latency; large items (KTA=16, KTB=16) cut the partial traffic
// when many token-layers share a launch (throughput).  In the single-layer
// mode each block requests its first down item's code before doing anything
// else, so that code is in registers by the time the item's inputs are ready.
//
// Hand-off across the GPU's XCDs (each has its own L2): partials are written
// and read with agent-scope monotonic atomics, which gfx950 performs at the
// device's coherence point; a producer waits for its stores to complete
// (s_waitcnt vmcnt(0)) before the counter increment that publishes them, and
// a consumer reads them only after observing the counter (see add_publish).
//
// Forward progress: blocks never wait on a block that has not started.  Every
// gate_up item is claimed (integer CAS) by the block that runs it; a down item
// whose inputs are not ready claims and runs the missing gate_up items itself,
// and otherwise waits only on items already claimed by running blocks, which
// never wait.  A bounded spin is a last safety net: a down item that gives up
// computes on NaN inputs (so its outputs are NaN, never stale values), raises
// the call's err flag (every other waiting block then gives up too) and the
// status flag that esc_moe_status reports, and sets a device-wide flag in
// pinned host memory that the next expert-path call on the device returns as
// ESC_ETIMEOUT (without a synchronisation).  The last block to finish resets
// every counter and the call's err flag, so the integer workspace is zero
// again for the next call (it must be zero before the first).
#pragma once

#include "moe.hpp"

namespace esc {

__device__ __forceinline__ int ld_relaxed(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Hand-off counters.  What a producer hands over (partials, f16 rows) it
// writes with agent-scope atomic stores, which gfx950 performs as
// write-through stores to the device's coherence point (sc1); the producer
// waits for them to complete (s_waitcnt vmcnt(0), wait_vm) before the
// relaxed agent-scope increment that publishes them, which is performed at
// the same point.  A consumer that sees the count it waits for reads the
// data with agent-scope atomic loads (sc1, from the coherence point, never a
// stale L2 line), issued after the count returned; the workgroup-scope
// acquire fence keeps the compiler from moving them above it (it emits no
// instruction).  The memory model's release / acquire at agent scope would
// add an L2 write-back of the XCD (buffer_wbl2 sc1) before every increment
// and an invalidate (buffer_inv sc1) after every count, for plain stores
// that these hand-offs do not use: measured on MI355X, 491 against 129 us
// per many-layer expert call at config 3, so the hand-offs do not take it.
__device__ __forceinline__ int add_publish(int* p, int v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void after_count() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup"); }
__device__ __forceinline__ bool claim(int* p) {
  int expected = 0;
  return __hip_atomic_compare_exchange_strong(p, &expected, 1, __ATOMIC_RELAXED,
                                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 ld_coherent2(const float* p) {
  const uint64_t v = __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
  return make_float2(__builtin_bit_cast(float, (uint32_t)v),
                     __builtin_bit_cast(float, (uint32_t)(v >> 32)));
}
// this wave's global stores (and loads) have completed
__device__ __forceinline__ void wait_vm() { __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// One token-layer of routed experts (all device pointers).
struct MoeLayer {
  const uint16_t* x;      // [T][H] f16
  const int* ids;         // [T*k]
  const float* scores;    // [T*k]
  const uint32_t* gu_code;
  const float* gu_rin;
  const float* gu_rout;
  const uint32_t* dn_code;
  const float* dn_rin;
  const float* dn_rout;
  uint16_t* y;            // [T][H] f16
};

struct FusedMoe {
  MoeLayer l0;              // the layer when `layers` is null
  const MoeLayer* layers;   // [L] device array for multi-layer launches
  float* partA;  // [L][nA][256]
  float* partB;  // [L][nB][256]
  uint16_t* xh2; // [L][M][I]   down inputs (two-launch path)
  int* cntA;     // [L][M*NB]  published gate_up items per (row, h-block)
  int* claimA;   // [L][nA]
  int* cntB;     // [L][T*NCP] finished down items per (token, column pair or block)
  int* done;     // [1]
  int* err;      // [1] a spin bound was hit in this call (reset by the last block)
  int* status;   // [1] a spin bound was hit since the host last read it
  int* host_err; // device-wide flag in pinned host memory: a spin bound was hit
                 // (the next expert-path call on the device reports it)
  int spin_limit;  // polls before a wait gives up (kSpinLimit; the host may lower it)
  int L, T, top_k, H, I;
  int NB;   // I / 128        h-blocks
  int NKC;  // H / (16*KTA)   gate_up items per (row, h-block), <= 62
  int NKB;  // I / (16*KTB)   down items per (row, column pair)
  int NCP;  // H / 256        column pairs (H / 128 column blocks: k_moe_down_blocks)
  int nA, nB;  // items per layer
  __device__ __forceinline__ const MoeLayer& layer(int l) const { return layers ? layers[l] : l0; }
};

constexpr int kFusedThreads = 256;
constexpr int kSpinLimit = 1 << 18;  // polls (one round trip + s_sleep each) before giving up
enum { kReady = -1, kTimeout = -3 };

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

// One item = 16 tiles x NKT kt of one stream, run by NW waves.  Waves split
// the tiles into 16/TPW groups and the kt range among the WPG waves of a
// group; each lane holds its NSTEP kt-steps of code in VGPRs.
template <int K, int NKT, int NW = 4>
struct ItemGeo {
  static constexpr int NG = 16 / Geo<K>::TPW;
  static constexpr int WPG = NW / NG;
  static constexpr int NSTEP = NKT / WPG;
  static_assert(NW % NG == 0 && NKT % WPG == 0, "item does not split over its waves");
};

template <int K, int NKT, int NW = 4>
struct ItemCode {
  LaneWords<K> w[ItemGeo<K, NKT, NW>::NSTEP];
};

template <int K, int NKT, int NW = 4, typename NtFn>
__device__ __forceinline__ ItemCode<K, NKT, NW> load_item(const uint32_t* __restrict__ code_e,
                                                          int TN, int kt_base, NtFn nt_of) {
  using G = Geo<K>;
  using IG = ItemGeo<K, NKT, NW>;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int g = wave / IG::WPG, wi = wave % IG::WPG;
  const int q = lane % G::LPT, i = lane / G::LPT;
  const size_t kstride = (size_t)TN * (8 * K);
  const uint32_t* lp = code_e + (size_t)nt_of(g * G::TPW + i) * (8 * K) + q * G::WPL +
                       (size_t)(kt_base + wi * IG::NSTEP) * kstride;
  ItemCode<K, NKT, NW> c;
#pragma unroll
  for (int k = 0; k < IG::NSTEP; ++k) c.w[k] = load_lane_words_nt<K>(lp + (size_t)k * kstride);
  return c;
}

// The item kernels keep their inputs in LDS as the decode's input pairs:
// per kt, word i (= xpair_index(r), r in {0,1,4,5,8,9,12,13}) holds
// [x(r+2) | x(r)], so the decode reads them as they are (no per-step
// permutes).  A lane holding the natural word [x(2j) | x(2j+1)] of kt-local
// position j = lane % 8 writes the paired word of the same position: even j
// [x(2j+2) | x(2j)], odd j [x(2j+1) | x(2j-1)], from its neighbour's word.
__device__ __forceinline__ uint32_t paired_word(uint32_t w) {
  const uint32_t nb = __builtin_bit_cast(uint32_t, lane_xor<1>(__builtin_bit_cast(float, w)));
  return (threadIdx.x & 1) ? __builtin_amdgcn_perm(nb, w, 0x07060302u)
                           : __builtin_amdgcn_perm(w, nb, 0x05040100u);
}

// Decode + multiply the item (inputs: 8 f16-pair words per kt in s_x); each
// wave leaves its lanes' column partials in s_red[wave].
template <int K, int NKT, int NW = 4>
__device__ __forceinline__ void item_to_lds(const ItemCode<K, NKT, NW>& code, const uint32_t* s_x,
                                            float (*s_red)[64][4]) {
  using G = Geo<K>;
  using IG = ItemGeo<K, NKT, NW>;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wi = wave % IG::WPG;
  const int q = lane % G::LPT, i = lane / G::LPT;
  const int src = i * G::LPT + (q + G::LPT - 1) % G::LPT;
  float acc[G::NCOL];
#pragma unroll
  for (int c = 0; c < G::NCOL; ++c) acc[c] = 0.f;
#pragma unroll
  for (int k = 0; k < IG::NSTEP; ++k) {
    const int kl = wi * IG::NSTEP + k;
    uint32_t xp[8];  // the kt's input pairs, stored paired (paired_word)
#pragma unroll
    for (int j = 0; j < 8; ++j) xp[j] = s_x[8 * kl + j];
    const uint32_t wprev = __shfl(code.w[k].w[G::WPL - 1], src);
    fast_tile_packed<K>(code.w[k], wprev, xp, acc);
  }
#pragma unroll
  for (int c = 0; c < G::NCOL; ++c) s_red[wave][lane][c] = acc[c];
}

// The item's weights decoded ahead of its inputs (items of one token-layer,
// whose code arrives before the inputs are transformed): the lane's packed
// pairs per kt-step, multiplied later by the overload below in the same
// order, so the item's partials are bit-identical to the one-pass form.
template <int K, int NKT, int NW>
struct ItemPairs {
  TilePairs<K> t[ItemGeo<K, NKT, NW>::NSTEP];
};

template <int K, int NKT, int NW>
__device__ __forceinline__ ItemPairs<K, NKT, NW> decode_item(const ItemCode<K, NKT, NW>& code) {
  using G = Geo<K>;
  const int lane = threadIdx.x & 63;
  const int q = lane % G::LPT, i = lane / G::LPT;
  const int src = i * G::LPT + (q + G::LPT - 1) % G::LPT;
  ItemPairs<K, NKT, NW> w;
#pragma unroll
  for (int k = 0; k < ItemGeo<K, NKT, NW>::NSTEP; ++k)
    w.t[k] = decode_pairs_packed<K>(code.w[k], __shfl(code.w[k].w[G::WPL - 1], src));
  return w;
}

template <int K, int NKT, int NW>
__device__ __forceinline__ void item_to_lds(const ItemPairs<K, NKT, NW>& w, const uint32_t* s_x,
                                            float (*s_red)[64][4]) {
  using G = Geo<K>;
  using IG = ItemGeo<K, NKT, NW>;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wi = wave % IG::WPG;
  float acc[G::NCOL];
#pragma unroll
  for (int c = 0; c < G::NCOL; ++c) acc[c] = 0.f;
#pragma unroll
  for (int k = 0; k < IG::NSTEP; ++k) {
    const int kl = wi * IG::NSTEP + k;
    uint32_t xp[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) xp[j] = s_x[8 * kl + j];
    dot_pairs_packed<K>(w.t[k], xp, acc);
  }
#pragma unroll
  for (int c = 0; c < G::NCOL; ++c) s_red[wave][lane][c] = acc[c];
}

// Column c (0..255) of an item after item_to_lds and a barrier: its wave
// partials summed in wave order.
template <int K, int NW = 4>
__device__ __forceinline__ float item_col(const float (*s_red)[64][4], int c) {
  using G = Geo<K>;
  constexpr int WPG = NW / (16 / G::TPW);
  const int it = c >> 4, gg = it / G::TPW, ii = it % G::TPW;
  int qq, ci;
  col_owner<K>(c & 15, qq, ci);
  float v = 0.f;
#pragma unroll
  for (int w = 0; w < WPG; ++w) v = v + s_red[gg * WPG + w][ii * G::LPT + qq][ci];
  return v;
}

// Decode + multiply an item and publish its 256 float32 column partials to
// dst (device-coherent stores when COH, for a consumer in the same launch;
// plain stores when the only consumer runs in a later launch).  Thread j < 256
// returns column j.
template <int K, int NKT, bool WAIT = true, bool COH = true, bool STORE = true, int NW = 4,
          typename Code = ItemCode<K, NKT, NW>>
__device__ __forceinline__ float compute_item(const Code& code, const uint32_t* s_x,
                                              float (*s_red)[64][4], float* __restrict__ dst) {
  item_to_lds<K, NKT, NW>(code, s_x, s_red);
  __syncthreads();
  const int j = threadIdx.x;
  float v = 0.f;
  if (NW == 4 || j < 256) {
    v = item_col<K, NW>(s_red, j);
    if constexpr (STORE) {
      if constexpr (COH)
        st_coherent(dst + j, v);
      else
        dst[j] = v;
    }
  }
  if constexpr (WAIT) {
    wait_vm();
    __syncthreads();
  }
  return v;
}

template <int K, int KTA, int NW = 4>
__device__ __forceinline__ ItemCode<K, KTA, NW> load_gate_up(const FusedMoe& p, const MoeLayer& L,
                                                             int a) {
  const int kc = a % p.NKC, rb = a / p.NKC, b = rb % p.NB, r = rb / p.NB;
  const int TK = p.H / 16, TN = 2 * p.I / 16, half_tn = p.I / 16;
  return load_item<K, KTA, NW>(L.gu_code + (size_t)as_global(L.ids)[r] * TK * TN * (8 * K), TN, KTA * kc,
                           [&](int it) { return it < 8 ? 8 * b + it : half_tn + 8 * b + (it - 8); });
}

template <int K, int KTA, int NW = 4>
__device__ __forceinline__ ItemCode<K, KTA, NW> load_gate_up(const FusedMoe& p, int l, int a) {
  return load_gate_up<K, KTA, NW>(p, p.layer(l), a);
}

template <int K, int KTB>
__device__ __forceinline__ ItemCode<K, KTB> load_down(const FusedMoe& p, int l, int bi) {
  const MoeLayer& L = p.layer(l);
  const int kb = bi % p.NKB, cp = (bi / p.NKB) % p.NCP, r = bi / p.NKB / p.NCP;
  const int TK = p.I / 16, TN = p.H / 16;
  return load_item<K, KTB>(L.dn_code + (size_t)as_global(L.ids)[r] * TK * TN * (8 * K), TN, KTB * kb,
                           [&](int it) { return 16 * cp + it; });
}

// count gate_up item a of layer l as published (its partials are complete)
__device__ __forceinline__ void publish_gate_up(const FusedMoe& p, int l, int a) {
  const int rb = a / p.NKC, b = rb % p.NB, r = rb / p.NB;
  add_publish(&p.cntA[(size_t)l * p.T * p.top_k * p.NB + r * p.NB + b], 1);
}

// gate_up item a of layer l with its code already in flight: transform the
// item's 16*KTA inputs (one wave per 128-block), decode + multiply, publish.
// The inputs of gate_up item a that wave `wave` < KTA/8 transforms: its two
// values of x and their two input scales.
struct GateUpIn {
  half_t x0, x1;
  float r0, r1;
};

template <int KTA>
__device__ __forceinline__ GateUpIn gate_up_in(const FusedMoe& p, const MoeLayer& L, int a) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  GateUpIn in{};
  if (wave < KTA / 8) {
    const int kc = a % p.NKC, r = a / p.NKC / p.NB;
    const int t = r / p.top_k, e = as_global(L.ids)[r];
    const int c = 16 * KTA * kc + 128 * wave + 2 * lane;
    const auto* xr = as_global(L.x + (size_t)t * p.H + c);
    const auto* ri = as_global(L.gu_rin + (size_t)e * p.H + c);
    in.x0 = __builtin_bit_cast(half_t, xr[0]);
    in.x1 = __builtin_bit_cast(half_t, xr[1]);
    in.r0 = ri[0];
    in.r1 = ri[1];
  }
  return in;
}

// Input transform of the item's 16*KTA inputs (one wave per 128-block) into
// s_x as decode input pairs.
template <int KTA>
__device__ __forceinline__ void gate_up_transform(const GateUpIn& in, uint32_t* s_x) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (wave < KTA / 8) {
    float v0 = (float)in.x0 * in.r0;
    float v1 = (float)in.x1 * in.r1;
    h128_wave(v0, v1);
    s_x[64 * wave + lane] = paired_word(pack2(to_f16(v0 * kRS), to_f16(v1 * kRS)));
  }
}

template <int K, int KTA, bool PUBLISH = true, bool COH = true, int NW = 4>
__device__ void run_gate_up(const FusedMoe& p, int l, int a, const ItemCode<K, KTA, NW>& code,
                            uint32_t* s_x, float (*s_red)[64][4]) {
  gate_up_transform<KTA>(gate_up_in<KTA>(p, p.layer(l), a), s_x);
  __syncthreads();
  compute_item<K, KTA, PUBLISH, COH, true, NW>(code, s_x, s_red,
                                              p.partA + ((size_t)l * p.nA + a) * 256);
  if (PUBLISH && threadIdx.x == 0) publish_gate_up(p, l, a);
}

// h-block kb of row r (layer l) -> this lane's word of its 128 down inputs
// (columns 128kb + 2lane, +1, stored as paired_word): the gate_up partials summed in fixed
// kc order, the gate_up output transform, SwiGLU and the down input transform.
// COH: the partials were published in this launch (device-coherent loads);
// otherwise by an earlier launch (plain loads, which may hit L2).
// One batch of CH kc partials of the h-block (gate and up values of the
// lane's two columns), loaded together.
template <int CH>
struct HBatch {
  float2 g[CH], u[CH];
};

template <bool COH, int CH>
__device__ __forceinline__ HBatch<CH> h_batch(const FusedMoe& p, const float* base, int kc0) {
  HBatch<CH> b;
#pragma unroll
  for (int j = 0; j < CH; ++j)
    if (kc0 + j < p.NKC) {
      if constexpr (COH) {
        b.g[j] = ld_coherent2(base + (size_t)(kc0 + j) * 256);
        b.u[j] = ld_coherent2(base + (size_t)(kc0 + j) * 256 + 128);
      } else {
        b.g[j] = *reinterpret_cast<const float2*>(base + (size_t)(kc0 + j) * 256);
        b.u[j] = *reinterpret_cast<const float2*>(base + (size_t)(kc0 + j) * 256 + 128);
      }
    }
  return b;
}

__device__ __forceinline__ const float* h_base(const FusedMoe& p, int l, int r, int kb) {
  return p.partA + ((size_t)l * p.nA + (size_t)(r * p.NB + kb) * p.NKC) * 256 +
         2 * (threadIdx.x & 63);
}

// The scales h-block kb of row r needs after its sums: the gate_up output
// scales of the lane's two gate and two up columns and the down input scales
// of its two inputs (expert e).
struct HScales {
  float2 g, u, ri;
};

__device__ __forceinline__ HScales h_scales(const FusedMoe& p, const MoeLayer& L, int e, int kb) {
  const int cg = 128 * kb + 2 * (threadIdx.x & 63);
  const float* ro = L.gu_rout + (size_t)e * 2 * p.I;
  return HScales{ld_global_f2(ro + cg), ld_global_f2(ro + p.I + cg),
                 ld_global_f2(L.dn_rin + (size_t)e * p.I + cg)};
}

// h_pair with its first batch of partials and its scales already requested
// (h_batch at kc0 = 0, h_scales), so that a caller can issue those loads
// before other work.
template <bool COH = true, int CH = 8>
__device__ uint32_t h_pair_from(const FusedMoe& p, int l, int r, int kb, const HBatch<CH>& first,
                                const HScales& sc) {
  const float* base = h_base(p, l, r, kb);
  float g0 = 0.f, g1 = 0.f, u0 = 0.f, u1 = 0.f;
  for (int kc0 = 0; kc0 < p.NKC; kc0 += CH) {
    const HBatch<CH> b = kc0 == 0 ? first : h_batch<COH, CH>(p, base, kc0);
#pragma unroll
    for (int j = 0; j < CH; ++j)
      if (kc0 + j < p.NKC) {
        g0 = g0 + b.g[j].x;
        g1 = g1 + b.g[j].y;
        u0 = u0 + b.u[j].x;
        u1 = u1 + b.u[j].y;
      }
  }
  h128_wave(g0, g1);
  h128_wave(u0, u1);
  const half_t h0 = swiglu1(to_f16((g0 * kRS) * sc.g.x), to_f16((u0 * kRS) * sc.u.x));
  const half_t h1 = swiglu1(to_f16((g1 * kRS) * sc.g.y), to_f16((u1 * kRS) * sc.u.y));
  float v0 = (float)h0 * sc.ri.x;
  float v1 = (float)h1 * sc.ri.y;
  h128_wave(v0, v1);
  return paired_word(pack2(to_f16(v0 * kRS), to_f16(v1 * kRS)));
}

template <bool COH = true, int CH = 8>
__device__ uint32_t h_pair(const FusedMoe& p, int l, int r, int kb) {
  const MoeLayer& L = p.layer(l);
  return h_pair_from<COH, CH>(p, l, r, kb, h_batch<COH, CH>(p, h_base(p, l, r, kb), 0),
                              h_scales(p, L, as_global(L.ids)[r], kb));
}

// h-block kb of row r (layer l) -> its 128 down inputs (paired words) in s_x[0..63].
template <bool COH = true>
__device__ void down_inputs(const FusedMoe& p, int l, int r, int kb, uint32_t* s_x) {
  s_x[threadIdx.x & 63] = h_pair<COH>(p, l, r, kb);
}

// Last down item of (layer l, token t, column pair cp): every slot's 256
// columns are summed (fixed kb order) and transformed to d16 in LDS by the 4
// waves (slot s on wave s % 4, two slots' loads issued together), then each
// thread combines one column over the slots in slot order.
__device__ void combine_tile(const FusedMoe& p, int l, int t, int cp, uint16_t (*s_d)[256]) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const MoeLayer& L = p.layer(l);
  for (int s0 = wave; s0 < p.top_k; s0 += 8) {
    float v[2][2][2] = {};
    for (int kb0 = 0; kb0 < p.NKB; kb0 += 4) {
      float2 pv[2][2][4];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int s = s0 + 4 * u;
        if (s >= p.top_k) continue;
        const float* pb = p.partB +
                          ((size_t)l * p.nB + (size_t)((t * p.top_k + s) * p.NCP + cp) * p.NKB) * 256 +
                          2 * lane;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (kb0 + j < p.NKB) {
            pv[u][0][j] = ld_coherent2(pb + (size_t)(kb0 + j) * 256);
            pv[u][1][j] = ld_coherent2(pb + (size_t)(kb0 + j) * 256 + 128);
          }
      }
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (s0 + 4 * u < p.top_k && kb0 + j < p.NKB) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              v[u][h][0] = v[u][h][0] + pv[u][h][j].x;
              v[u][h][1] = v[u][h][1] + pv[u][h][j].y;
            }
          }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int s = s0 + 4 * u;
      if (s >= p.top_k) continue;
      const int e = as_global(L.ids)[t * p.top_k + s];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        h128_wave(v[u][h][0], v[u][h][1]);
        const int col = 256 * cp + 128 * h + 2 * lane;
        const auto* ro = as_global(L.dn_rout + (size_t)e * p.H + col);
        s_d[s][128 * h + 2 * lane] = __builtin_bit_cast(uint16_t, to_f16((v[u][h][0] * kRS) * ro[0]));
        s_d[s][128 * h + 2 * lane + 1] =
            __builtin_bit_cast(uint16_t, to_f16((v[u][h][1] * kRS) * ro[1]));
      }
    }
  }
  __syncthreads();
  const int j = threadIdx.x;
  float a = 0.f;
  for (int s = 0; s < p.top_k; ++s) {
    const float w = (float)(half_t)as_global(L.scores)[t * p.top_k + s];
    a = a + (float)__builtin_bit_cast(half_t, s_d[s][j]) * w;
  }
  as_global_w(L.y)[(size_t)t * p.H + 256 * cp + j] = __builtin_bit_cast(uint16_t, (half_t)a);
}

// Block-uniform wait for the gate_up items of (layer l, row r, h-block kb):
// one wave polls; an unclaimed item is claimed and returned (>= 0, the item
// index within the layer) for the block to run.
__device__ int wait_gate_up(const FusedMoe& p, int l, int r, int kb, int* s_flag) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (wave == 0) {
    const int abase = (r * p.NB + kb) * p.NKC;
    const int* cnt = &p.cntA[(size_t)l * p.T * p.top_k * p.NB + r * p.NB + kb];
    int* claims = p.claimA + (size_t)l * p.nA + abase;
    int st = kTimeout;
    for (int spin = 0; spin < p.spin_limit; ++spin) {
      // the counter every poll; the claim flags and the error flag only on
      // every 32nd (they change rarely, and each is a device-coherent load)
      const bool full = (spin & 31) == 0;
      int v = full ? 0 : 1;
      if (lane == 0)
        v = ld_relaxed(cnt);
      else if (full && lane <= p.NKC)
        v = ld_relaxed(&claims[lane - 1]);
      else if (full && lane == 63)
        v = ld_relaxed(p.err);
      else if (lane == 63)
        v = 0;
      if (__shfl(v, 0) >= p.NKC) {
        after_count();
        st = kReady;
        break;
      }
      if (__shfl(v, 63) != 0) break;  // another block timed out: give up too
      uint64_t free_mask = __ballot(lane >= 1 && lane <= p.NKC && v == 0);
      int got = -1;
      if (lane == 0) {
        while (free_mask) {
          const int i = __builtin_ctzll(free_mask);
          free_mask &= free_mask - 1;
          if (claim(&claims[i - 1])) {
            got = abase + i - 1;
            break;
          }
        }
      }
      got = __shfl(got, 0);
      if (got >= 0) {
        st = got;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    if (lane == 0) *s_flag = st;
  }
  __syncthreads();
  const int st = *s_flag;
  __syncthreads();
  return st;
}

// ---------------------------------------------------------------- two launches
// Every gate_up item of every layer in one launch, then every down item (plus
// the last-arriver combine) in a second, one item per block.  The launch
// boundary is the gate_up -> down hand-off, so nothing waits, the partials go
// through plain stores and loads, and the hardware dispatcher balances the
// items over the CUs.

// The dispatcher places consecutive workgroups on the 8 XCDs in turn.  Block
// b runs logical item xcd_item(b, n), so each XCD gets one contiguous item
// range: the gate_up items of a row, and later the down items that re-read
// that row's partials (8 column pairs x the same h-blocks), share an L2.
constexpr int kXcds = 8;
__device__ __forceinline__ int xcd_item(int b, int n) {
  return n % kXcds ? b : (b % kXcds) * (n / kXcds) + b / kXcds;
}

// gate_up item a of layer l.  PREH (many token-layers per launch): the last
// of the NKC items of its (row, h-block) to finish turns the h-block's
// partials into the 128 down inputs (xh2), so every down item reads them
// ready-made instead of redoing the transforms.  Without PREH (one
// token-layer, latency-bound) the partials go out with plain stores and each
// down item derives its own inputs, which keeps the counter round trip off
// the critical path.
template <int KG, int KTA, bool PREH, int NW = 4>
__global__ __launch_bounds__(64 * NW) void k_moe_gate_up_items(FusedMoe p) {
  __shared__ float s_red[NW][64][4];
  __shared__ uint32_t s_x[256];
  __shared__ int s_last;
  const int tid = threadIdx.x;
  const int g = xcd_item(blockIdx.x, gridDim.x);
  const int l = g / p.nA, a = g % p.nA;
  if constexpr (NW == 16) {
    // one token-layer (the record in the kernel arguments, read once): one
    // kt-step per wave, whose weights are decoded as soon as the code arrives,
    // while the inputs' loads and transform are still pending
    static_assert(!PREH, "16-wave items run one token-layer");
    const MoeLayer L = p.l0;
    const auto code = load_gate_up<KG, KTA, NW>(p, L, a);
    const GateUpIn in = gate_up_in<KTA>(p, L, a);
    const auto w = decode_item<KG, KTA, NW>(code);
    gate_up_transform<KTA>(in, s_x);
    __syncthreads();
    compute_item<KG, KTA, false, false, true, NW>(w, s_x, s_red, p.partA + (size_t)a * 256);
  } else {
    const auto code = load_gate_up<KG, KTA, NW>(p, l, a);
    run_gate_up<KG, KTA, false, PREH, NW>(p, l, a, code, s_x, s_red);
  }
  if constexpr (PREH) {
    wait_vm();  // this wave's partial stores have completed
    __syncthreads();
    const int rb = a / p.NKC, b = rb % p.NB, r = rb / p.NB;
    const int M = p.T * p.top_k;
    if (tid == 0) {
      int* c = &p.cntA[((size_t)l * M + r) * p.NB + b];
      const bool last = add_publish(c, 1) == p.NKC - 1;
      if (last) {
        after_count();
        __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      s_last = last;
    }
    __syncthreads();
    if (s_last && tid < 64) {
      const uint32_t v = h_pair<true>(p, l, r, b);
      reinterpret_cast<uint32_t*>(p.xh2 + ((size_t)l * M + r) * p.I + 128 * b)[tid] = v;
    }
  }
}

template <int KG, int KD, int KTB, bool PREH>
__global__ __launch_bounds__(kFusedThreads, 4) void k_moe_down_items(FusedMoe p) {
  __shared__ float s_red[4][64][4];
  __shared__ uint32_t s_x[256];
  __shared__ uint16_t s_d[32][256];
  __shared__ int s_flag;
  constexpr int kHB = KTB >= 8 ? KTB / 8 : 1;
  const int tid = threadIdx.x;
  const int g = xcd_item(blockIdx.x, gridDim.x);
  const int l = g / p.nB, bi = g % p.nB;
  const int kb = bi % p.NKB, rc = bi / p.NKB, cp = rc % p.NCP, r = rc / p.NCP;
  const int t = r / p.top_k, hb0 = (KTB * kb) / 8;
  const auto code = load_down<KD, KTB>(p, l, bi);
  if ((tid >> 6) < kHB) {
    const int w = tid >> 6;
    if constexpr (PREH)
      s_x[64 * w + (tid & 63)] = reinterpret_cast<const uint32_t*>(
          p.xh2 + ((size_t)l * p.T * p.top_k + r) * p.I + 128 * (hb0 + w))[tid & 63];
    else
      down_inputs<false>(p, l, r, hb0 + w, s_x + 64 * w);
  }
  __syncthreads();
  compute_item<KD, KTB>(code, s_x + ((KTB * kb) % 8) * 8, s_red,
                        p.partB + ((size_t)l * p.nB + bi) * 256);
  if (tid == 0) {
    int* c = &p.cntB[(size_t)l * p.T * p.NCP + t * p.NCP + cp];
    const bool last = add_publish(c, 1) == p.top_k * p.NKB - 1;
    if (last) {
      after_count();
      __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    s_flag = last;
  }
  __syncthreads();
  if (s_flag) combine_tile(p, l, t, cp, s_d);
}

// Down items of one token-layer with I == 512 (k_moe_down_blocks): item
// (row r, column block hb) covers output columns [128hb, 128hb+128) -- 8
// tiles, one block of the output transform -- over all 32 kt, so no split-K
// sum crosses blocks.  A K=2 wave-step spans 16 tile slots: slot i takes tile
// i % 8 at kt 2s + i / 8 (two kt per step); a K=3 step spans the 8 tiles at one
// kt.  NW waves split the steps.
template <int K, int NW>
struct BlockItem {
  static constexpr int KPS = Geo<K>::TPW / 8;  // kt per wave-step
  static constexpr int NSTEP = 32 / (KPS * NW);
  static_assert(NSTEP * KPS * NW == 32, "32 kt do not split over the waves");
};

template <int K, int NW>
struct BlockCode {
  LaneWords<K> w[BlockItem<K, NW>::NSTEP];
};

template <int K, int NW>
__device__ __forceinline__ BlockCode<K, NW> load_block_item(const uint32_t* __restrict__ code_e,
                                                            int TN, int hb) {
  using G = Geo<K>;
  using BI = BlockItem<K, NW>;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int q = lane % G::LPT, i = lane / G::LPT;
  const size_t kstride = (size_t)TN * (8 * K);
  const int kt0 = BI::KPS * wave * BI::NSTEP + i / 8;
  const uint32_t* lp = code_e + (size_t)(8 * hb + i % 8) * (8 * K) + q * G::WPL + kt0 * kstride;
  BlockCode<K, NW> c;
#pragma unroll
  for (int k = 0; k < BI::NSTEP; ++k)
    c.w[k] = load_lane_words_nt<K>(lp + (size_t)(k * BI::KPS) * kstride);
  return c;
}

// Decode + multiply the block item (inputs: all 32 kt of paired words in
// s_x); each wave leaves its lanes' column partials in s_red[wave].
template <int K, int NW>
__device__ __forceinline__ void block_item_to_lds(const BlockCode<K, NW>& code,
                                                  const uint32_t* s_x, float (*s_red)[64][4]) {
  using G = Geo<K>;
  using BI = BlockItem<K, NW>;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int q = lane % G::LPT, i = lane / G::LPT;
  const int src = i * G::LPT + (q + G::LPT - 1) % G::LPT;
  float acc[G::NCOL];
#pragma unroll
  for (int c = 0; c < G::NCOL; ++c) acc[c] = 0.f;
#pragma unroll
  for (int k = 0; k < BI::NSTEP; ++k) {
    const int kl = BI::KPS * (wave * BI::NSTEP + k) + i / 8;
    uint32_t xp[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) xp[j] = s_x[8 * kl + j];
    const uint32_t wprev = __shfl(code.w[k].w[G::WPL - 1], src);
    fast_tile_packed<K>(code.w[k], wprev, xp, acc);
  }
#pragma unroll
  for (int c = 0; c < G::NCOL; ++c) s_red[wave][lane][c] = acc[c];
}

// A block item's weights decoded ahead of its inputs (as ItemPairs).
template <int K, int NW>
struct BlockPairs {
  TilePairs<K> t[BlockItem<K, NW>::NSTEP];
};

template <int K, int NW>
__device__ __forceinline__ BlockPairs<K, NW> decode_block_item(const BlockCode<K, NW>& code) {
  using G = Geo<K>;
  const int lane = threadIdx.x & 63;
  const int q = lane % G::LPT, i = lane / G::LPT;
  const int src = i * G::LPT + (q + G::LPT - 1) % G::LPT;
  BlockPairs<K, NW> w;
#pragma unroll
  for (int k = 0; k < BlockItem<K, NW>::NSTEP; ++k)
    w.t[k] = decode_pairs_packed<K>(code.w[k], __shfl(code.w[k].w[G::WPL - 1], src));
  return w;
}

template <int K, int NW>
__device__ __forceinline__ void block_item_to_lds(const BlockPairs<K, NW>& w, const uint32_t* s_x,
                                                  float (*s_red)[64][4]) {
  using G = Geo<K>;
  using BI = BlockItem<K, NW>;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int i = (lane & 63) / G::LPT;
  float acc[G::NCOL];
#pragma unroll
  for (int c = 0; c < G::NCOL; ++c) acc[c] = 0.f;
#pragma unroll
  for (int k = 0; k < BI::NSTEP; ++k) {
    const int kl = BI::KPS * (wave * BI::NSTEP + k) + i / 8;
    uint32_t xp[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) xp[j] = s_x[8 * kl + j];
    dot_pairs_packed<K>(w.t[k], xp, acc);
  }
#pragma unroll
  for (int c = 0; c < G::NCOL; ++c) s_red[wave][lane][c] = acc[c];
}

// Column c (0..127) of a block item after block_item_to_lds and a barrier:
// summed over the waves in order, each wave's kt slots in order.
template <int K, int NW>
__device__ __forceinline__ float block_item_col(const float (*s_red)[64][4], int c) {
  using G = Geo<K>;
  int qq, ci;
  col_owner<K>(c & 15, qq, ci);
  const int tile = c >> 4;
  float v = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w)
#pragma unroll
    for (int h = 0; h < BlockItem<K, NW>::KPS; ++h)
      v = v + s_red[w][(tile + 8 * h) * G::LPT + qq][ci];
  return v;
}

// What wave 0 of a block down item needs after the decode, requested when the
// item starts so that no load waits behind its barriers: the two output
// scales of column pair `lane` and the f16-rounded score of slot `lane`.
struct DownTail {
  float ro0 = 0.f, ro1 = 0.f, score = 0.f;
};

__device__ __forceinline__ DownTail down_tail(const FusedMoe& p, const MoeLayer& L, int e, int t,
                                              int hb) {
  const int lane = threadIdx.x & 63;
  DownTail d;
  if ((threadIdx.x >> 6) == 0) {
    const auto* ro = as_global(L.dn_rout + (size_t)e * p.H + 128 * hb + 2 * lane);
    d.ro0 = ro[0];
    d.ro1 = ro[1];
    if (lane < p.top_k) d.score = (float)(half_t)as_global(L.scores)[t * p.top_k + lane];
  }
  return d;
}

// Block down item bi of layer l after block_item_to_lds and a barrier: wave 0
// sums the waves, applies the down output transform, rounds the 128 columns
// to f16 and publishes them (256 bytes of partB at float offset 64 bi); the
// last of the (token, hb)'s top_k items to publish gathers their f16 rows and
// combines them in slot order (f16(score) weights, float32 sum, one f16
// rounding) into y.
template <int KD, int NW>
__device__ __forceinline__ void down_block_finish(const FusedMoe& p, const MoeLayer& L, int l,
                                                  int bi, const DownTail& d,
                                                  const float (*s_red)[64][4]) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (wave != 0) return;
  const int hb = bi % p.NCP, t = bi / p.NCP / p.top_k;
  uint32_t* rows = reinterpret_cast<uint32_t*>(p.partB + (size_t)l * p.nB * 256);
  float v0 = block_item_col<KD, NW>(s_red, 2 * lane);
  float v1 = block_item_col<KD, NW>(s_red, 2 * lane + 1);
  h128_wave(v0, v1);
  const uint32_t w = pack2(to_f16((v0 * kRS) * d.ro0), to_f16((v1 * kRS) * d.ro1));
  __hip_atomic_store(rows + (size_t)bi * 64 + lane, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  wait_vm();
  int last = 0;
  if (lane == 0) {
    int* c = &p.cntB[(size_t)l * p.T * p.NCP + t * p.NCP + hb];
    last = add_publish(c, 1) == p.top_k - 1;
    if (last) {
      after_count();
      __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (!__shfl(last, 0)) return;
  float a0 = 0.f, a1 = 0.f;
  for (int s0 = 0; s0 < p.top_k; s0 += 8) {
    uint32_t d8[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (s0 + j < p.top_k)
        d8[j] = __hip_atomic_load(rows + (size_t)((t * p.top_k + s0 + j) * p.NCP + hb) * 64 + lane,
                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (s0 + j < p.top_k) {
        const float sw = __shfl(d.score, s0 + j);
        a0 = a0 + (float)__builtin_bit_cast(half_t, (uint16_t)d8[j]) * sw;
        a1 = a1 + (float)__builtin_bit_cast(half_t, (uint16_t)(d8[j] >> 16)) * sw;
      }
  }
  as_global_w(reinterpret_cast<uint32_t*>(L.y + (size_t)t * p.H + 128 * hb))[lane] =
      pack2((half_t)a0, (half_t)a1);
}

// One item per block (plan: NCP = H / 128 column blocks, NKB = 1).  The item
// takes the row's 512 down inputs (4 waves, one h-block each: derived from the
// gate_up partials, or read ready-made from xh2 when PREH), decodes and
// multiplies, and finishes as down_block_finish.
template <int KG, int KD, bool PREH, int NW>
__global__ __launch_bounds__(64 * NW) void k_moe_down_blocks(FusedMoe p) {
  static_assert(NW >= 4, "one wave per h-block");
  __shared__ float s_red[NW][64][4];
  __shared__ uint32_t s_x[256];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = xcd_item(blockIdx.x, gridDim.x);
  const int l = g / p.nB, bi = g % p.nB;
  const int hb = bi % p.NCP, r = bi / p.NCP, t = r / p.top_k;
  const int TN = p.H / 16;
  if constexpr (NW == 16) {
    // one token-layer (the record in the kernel arguments, read once): the
    // gate_up partials are requested first (their address needs no expert
    // id), then the expert's code and every scale the item needs, and the
    // weights are decoded while the partials are still on their way
    static_assert(!PREH, "16-wave block items run one token-layer");
    const MoeLayer L = p.l0;
    const HBatch<8> first = wave < 4 ? h_batch<false, 8>(p, h_base(p, 0, r, wave), 0) : HBatch<8>{};
    const int e = as_global(L.ids)[r];
    const auto code =
        load_block_item<KD, NW>(L.dn_code + (size_t)e * (p.I / 16) * TN * (8 * KD), TN, hb);
    const DownTail d = down_tail(p, L, e, t, hb);
    const HScales sc = wave < 4 ? h_scales(p, L, e, wave) : HScales{};
    const auto w = decode_block_item<KD, NW>(code);
    if (wave < 4) s_x[64 * wave + lane] = h_pair_from<false, 8>(p, 0, r, wave, first, sc);
    __syncthreads();
    block_item_to_lds<KD, NW>(w, s_x, s_red);
    __syncthreads();
    down_block_finish<KD, NW>(p, L, 0, bi, d, s_red);
  } else {
    const MoeLayer& L = p.layer(l);
    const int e = as_global(L.ids)[r];
    const auto code =
        load_block_item<KD, NW>(L.dn_code + (size_t)e * (p.I / 16) * TN * (8 * KD), TN, hb);
    const DownTail d = down_tail(p, L, e, t, hb);
    if (wave < 4) {
      if constexpr (PREH)
        s_x[64 * wave + lane] = reinterpret_cast<const uint32_t*>(
            p.xh2 + ((size_t)l * p.T * p.top_k + r) * p.I + 128 * wave)[lane];
      else
        s_x[64 * wave + lane] = h_pair<false>(p, l, r, wave);
    }
    __syncthreads();
    block_item_to_lds<KD, NW>(code, s_x, s_red);
    __syncthreads();
    down_block_finish<KD, NW>(p, L, l, bi, d, s_red);
  }
}

template <int KG, int KD, int KTA, int KTB, bool PRE>
__global__ __launch_bounds__(kFusedThreads, 4) void k_moe_fused(FusedMoe p) {
  static_assert(KTA % 8 == 0 && KTA <= 32 && (KTB == 4 || (KTB % 8 == 0 && KTB <= 32)), "");
  __shared__ float s_red[4][64][4];
  __shared__ uint32_t s_x[256];
  __shared__ uint16_t s_d[32][256];
  __shared__ int s_flag;
  const int tid = threadIdx.x;
  const int nA_all = p.L * p.nA, nB_all = p.L * p.nB;
  const int M = p.T * p.top_k;

  // single-layer latency mode: the block's first down item's code is
  // requested now and used after its inputs are ready
  const int g0 = blockIdx.x;
  ItemCode<KD, KTB> code0{};
  if (PRE && g0 < nB_all) code0 = load_down<KD, KTB>(p, g0 / p.nB, g0 % p.nB);

  // gate_up items, software-pipelined: the next item's code loads and claim
  // are issued before waiting for this item's partial stores to complete
  {
    int ga = blockIdx.x;
    ItemCode<KG, KTA> code{};
    if (ga < nA_all) {
      code = load_gate_up<KG, KTA>(p, ga / p.nA, ga % p.nA);
      if (tid == 0) s_flag = claim(&p.claimA[ga]);
    }
    while (ga < nA_all) {
      __syncthreads();
      const int mine = s_flag;
      __syncthreads();
      const int l = ga / p.nA, a = ga % p.nA, gn = ga + gridDim.x;
      if (mine) run_gate_up<KG, KTA, false>(p, l, a, code, s_x, s_red);
      if (gn < nA_all) {
        code = load_gate_up<KG, KTA>(p, gn / p.nA, gn % p.nA);
        if (tid == 0) s_flag = claim(&p.claimA[gn]);
      }
      wait_vm();
      __syncthreads();
      if (mine && tid == 0) publish_gate_up(p, l, a);
      ga = gn;
    }
  }

  constexpr int kHB = KTB >= 8 ? KTB / 8 : 1;  // h-blocks read by one down item
  for (int gb = blockIdx.x; gb < nB_all; gb += gridDim.x) {
    const int l = gb / p.nB, bi = gb % p.nB;
    const int kb = bi % p.NKB, rc = bi / p.NKB, cp = rc % p.NCP, r = rc / p.NCP;
    const int t = r / p.top_k, hb0 = (KTB * kb) / 8;
    const auto code = (PRE && gb == g0) ? code0 : load_down<KD, KTB>(p, l, bi);
    bool ok = true;
    for (int h = 0; h < kHB; ++h) {
      int st;
      while ((st = wait_gate_up(p, l, r, hb0 + h, &s_flag)) >= 0)
        run_gate_up<KG, KTA>(p, l, st, load_gate_up<KG, KTA>(p, l, st), s_x, s_red);
      ok = ok && st != kTimeout;
    }
    if (!ok) {
      // inputs never became ready: NaN inputs make this item's outputs NaN
      if ((tid >> 6) < kHB) s_x[tid] = 0x7E007E00u;
      if (tid == 0) {
        atomicOr(p.err, 1);
        atomicOr(p.status, 1);
        if (p.host_err) __hip_atomic_store(p.host_err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      }
    } else if ((tid >> 6) < kHB) {
      down_inputs(p, l, r, hb0 + (tid >> 6), s_x + 64 * (tid >> 6));
    }
    __syncthreads();
    // a 4-kt item reads the first or second half of its 128-block
    compute_item<KD, KTB>(code, s_x + ((KTB * kb) % 8) * 8, s_red,
                          p.partB + ((size_t)l * p.nB + bi) * 256);
    if (tid == 0) {
      s_flag = (add_publish(&p.cntB[(size_t)l * p.T * p.NCP + t * p.NCP + cp], 1) ==
                p.top_k * p.NKB - 1);
      if (s_flag) after_count();
    }
    __syncthreads();
    const int last = s_flag;
    __syncthreads();
    if (last) combine_tile(p, l, t, cp, s_d);
    __syncthreads();
  }

  // teardown: the last block resets the integer workspace for the next call
  wait_vm();
  __syncthreads();
  if (tid == 0) {
    s_flag = (add_publish(p.done, 1) == (int)gridDim.x - 1);
    if (s_flag) after_count();
  }
  __syncthreads();
  if (s_flag) {
    for (int i = tid; i < p.L * M * p.NB; i += kFusedThreads) p.cntA[i] = 0;
    for (int i = tid; i < nA_all; i += kFusedThreads) p.claimA[i] = 0;
    for (int i = tid; i < p.L * p.T * p.NCP; i += kFusedThreads) p.cntB[i] = 0;
    __syncthreads();
    if (tid == 0) {
      *p.err = 0;
      *p.done = 0;
    }
  }
}

}  // namespace esc
