// libescha_hip: the C ABI declared in include/escha_hip.h.
// One translation unit so the device decode table is a single symbol.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <atomic>
#include <mutex>
#include <string>

#include "../../include/escha_hip.h"
#include "fused.hpp"
#include "mfma.hpp"
#include "linear.hpp"
#include "q8.hpp"
#include "probe.hpp"
#include "layers.hpp"
#include "proj.hpp"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

#define ESC_REQUIRE(cond, ...) \
  do {                         \
    if (!(cond)) return fail(ESC_EINVAL, __VA_ARGS__); \
  } while (0)

int hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(ESC_EHIP, "%s: %s", what, hipGetErrorString(e));
  return ESC_OK;
}

int launched(const char* what) { return hip_check(hipGetLastError(), what); }

inline hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

constexpr int kMaxDevices = 64;
std::mutex g_init_mu;
bool g_lut_ready[kMaxDevices];

int ensure_lut() {
  int dev = 0;
  if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
  if (dev < 0 || dev >= kMaxDevices) return fail(ESC_EINVAL, "device index %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_init_mu);
  if (g_lut_ready[dev]) return ESC_OK;
  hipLaunchKernelGGL(esc::k_lut_init, dim3(256), dim3(256), 0, 0);
  if (int rc = launched("k_lut_init")) return rc;
  if (int rc = hip_check(hipDeviceSynchronize(), "esc_init sync")) return rc;
  g_lut_ready[dev] = true;
  return ESC_OK;
}

bool lut_ready() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
  std::lock_guard<std::mutex> lk(g_init_mu);
  return g_lut_ready[dev];
}

int ensure_scratch(void** out);
// Device-wide bounded-wait flag of the single persistent expert launch
// (k_moe_fused): one int per device in pinned, coherent host memory, set by a
// workgroup that gave up a wait and read by the host with no synchronisation,
// so a later call can report the failure.  Allocated at set-up (esc_init, or
// the first esc_moe_expert_path call on the device); the allocation-free entry
// point only uses it once it exists.
int* g_wait_flag[kMaxDevices];
int* g_wait_flag_dev[kMaxDevices];
std::atomic<int> g_spin_limit{esc::kSpinLimit};

int ensure_wait_flag() {
  int dev = 0;
  if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
  if (dev < 0 || dev >= kMaxDevices) return fail(ESC_EINVAL, "device index %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_init_mu);
  if (g_wait_flag[dev]) return ESC_OK;
  void* h = nullptr;
  if (int rc = hip_check(hipHostMalloc(&h, 64, hipHostMallocMapped | hipHostMallocCoherent),
                         "hipHostMalloc"))
    return rc;
  void* d = nullptr;
  if (int rc = hip_check(hipHostGetDevicePointer(&d, h, 0), "hipHostGetDevicePointer")) {
    (void)hipHostFree(h);
    return rc;
  }
  *static_cast<volatile int*>(h) = 0;
  g_wait_flag_dev[dev] = static_cast<int*>(d);
  g_wait_flag[dev] = static_cast<int*>(h);
  return ESC_OK;
}

// Takes the device's flag: ESC_ETIMEOUT (flag cleared) if a single persistent
// launch on this device gave up a wait since the last take; *dev_flag is the
// flag's device address for the next launch (null before set-up).
int take_wait_error(int** dev_flag) {
  *dev_flag = nullptr;
  int dev = 0;
  if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
  if (dev < 0 || dev >= kMaxDevices) return fail(ESC_EINVAL, "device index %d out of range", dev);
  int* h = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_init_mu);
    h = g_wait_flag[dev];
    *dev_flag = g_wait_flag_dev[dev];
  }
  if (h && __atomic_exchange_n(h, 0, __ATOMIC_ACQ_REL) != 0)
    return fail(ESC_ETIMEOUT,
                "an earlier single-launch expert-path call on device %d gave up a bounded wait: "
                "its outputs are NaN (this call did not run)",
                dev);
  return ESC_OK;
}

int check_proj(int K, int IC, int OC) {
  ESC_REQUIRE(K == 2 || K == 3, "escha code implies K=%d; this runtime implements K in [2, 3]", K);
  ESC_REQUIRE(IC > 0 && OC > 0 && IC % 128 == 0 && OC % 128 == 0,
              "escha linear dimensions must be positive multiples of 128, got %dx%d", IC, OC);
  return ESC_OK;
}

// ---- dispatch helpers over compile-time parameters
template <template <int, bool> class F, typename... A>
int by_k_lut(int K, int lut, A... a) {
  if (K == 2) return lut ? F<2, true>::run(a...) : F<2, false>::run(a...);
  return lut ? F<3, true>::run(a...) : F<3, false>::run(a...);
}

template <int K, bool LUT>
struct DecodeF {
  static int run(const uint32_t* code, int IC, int OC, uint16_t* w, hipStream_t s) {
    const int TK = IC / 16, TN = OC / 16;
    hipLaunchKernelGGL((esc::k_decode_tiles<K, LUT>), dim3(TK * TN), dim3(256), 0, s, code, TN,
                       OC, w);
    return launched("k_decode_tiles");
  }
};

template <int K, bool LUT, int MODE>
struct ExactF {
  template <int R>
  static int go(const uint16_t* xh, const uint32_t* code, const int* a, const int* b, int M,
                int n_groups, int TK, int TN, float* mid, hipStream_t s) {
    hipLaunchKernelGGL((esc::k_gemm_exact<K, LUT, R, MODE>), dim3(TN / 8, n_groups), dim3(512),
                       0, s, xh, code, a, b, M, TK, TN, mid);
    return launched("k_gemm_exact");
  }
  static int run(int R, const uint16_t* xh, const uint32_t* code, const int* a, const int* b,
                 int M, int n_groups, int TK, int TN, float* mid, hipStream_t s) {
    switch (R) {
      case 1: return go<1>(xh, code, a, b, M, n_groups, TK, TN, mid, s);
      case 2: return go<2>(xh, code, a, b, M, n_groups, TK, TN, mid, s);
      case 3: return go<3>(xh, code, a, b, M, n_groups, TK, TN, mid, s);
      case 4: return go<4>(xh, code, a, b, M, n_groups, TK, TN, mid, s);
      case 8: return go<8>(xh, code, a, b, M, n_groups, TK, TN, mid, s);
      case 12: return go<12>(xh, code, a, b, M, n_groups, TK, TN, mid, s);
      case 16: return go<16>(xh, code, a, b, M, n_groups, TK, TN, mid, s);
    }
    return fail(ESC_EINVAL, "rows per group R=%d not in {1,2,3,4,8,12,16}", R);
  }
};

template <int MODE>
int exact_dispatch(int K, int lut, int R, const uint16_t* xh, const uint32_t* code,
                   const int* a, const int* b, int M, int n_groups, int TK, int TN, float* mid,
                   hipStream_t s) {
  if (K == 2)
    return lut ? ExactF<2, true, MODE>::run(R, xh, code, a, b, M, n_groups, TK, TN, mid, s)
               : ExactF<2, false, MODE>::run(R, xh, code, a, b, M, n_groups, TK, TN, mid, s);
  return lut ? ExactF<3, true, MODE>::run(R, xh, code, a, b, M, n_groups, TK, TN, mid, s)
             : ExactF<3, false, MODE>::run(R, xh, code, a, b, M, n_groups, TK, TN, mid, s);
}

template <int K, bool LUT>
struct ExactOutF {
  template <int R>
  static int go(const uint16_t* xh, const uint32_t* code, const float* rout, int M, int TK,
                int TN, float rs, uint16_t* out, hipStream_t s) {
    hipLaunchKernelGGL((esc::k_gemm_exact_out<K, LUT, R>), dim3(TN / 8, (M + R - 1) / R),
                       dim3(512), 0, s, xh, code, rout, M, TK, TN, rs, out);
    return launched("k_gemm_exact_out");
  }
  static int run(int R, const uint16_t* xh, const uint32_t* code, const float* rout, int M,
                 int TK, int TN, float rs, uint16_t* out, hipStream_t s) {
    switch (R) {
      case 1: return go<1>(xh, code, rout, M, TK, TN, rs, out, s);
      case 2: return go<2>(xh, code, rout, M, TK, TN, rs, out, s);
      case 4: return go<4>(xh, code, rout, M, TK, TN, rs, out, s);
      case 8: return go<8>(xh, code, rout, M, TK, TN, rs, out, s);
    }
    return fail(ESC_EINVAL, "rows per group R=%d not in {1,2,4,8}", R);
  }
};

// ---- split-K GEMV geometry: KS kt per block (multiple of 4, divides TK)
int fast_splits(int K, int M, int TK, int TN, int target = 1024) {
  const int tpw = K == 2 ? 16 : 8;
  const int per_split = ((TN + tpw - 1) / tpw) * M;  // blocks per kt split
  int S = 1;
  // aim for >= target blocks of 4 waves while keeping >= 4 kt per block
  while (per_split * S < target && TK % (S * 2 * 4) == 0 && TK / (S * 2) >= 4) S *= 2;
  return S;
}

template <int K, bool LUT>
struct FastF {
  static int run(const uint16_t* xh, const uint32_t* code, const int* row_expert, int M, int TK,
                 int TN, int S, float* part, hipStream_t s) {
    const int tpw = K == 2 ? 16 : 8;
    hipLaunchKernelGGL((esc::k_gemv_fast<K, LUT>), dim3((TN + tpw - 1) / tpw, M, S), dim3(256), 0, s, xh,
                       code, row_expert, M, TK, TN, TK / S, part);
    return launched("k_gemv_fast");
  }
};

template <int K, bool LUT>
struct FastRowsF {
  template <int R>
  static int go(const uint16_t* xh, const uint32_t* code, int M, int TK, int TN, int S,
                float* part, hipStream_t s) {
    const int tpw = K == 2 ? 16 : 8;
    hipLaunchKernelGGL((esc::k_gemv_fast_rows<K, LUT, R>), dim3((TN + tpw - 1) / tpw, (M + R - 1) / R, S),
                       dim3(256), 0, s, xh, code, nullptr, nullptr, M, TK, TN, TK / S, part);
    return launched("k_gemv_fast_rows");
  }
  static int run(int R, const uint16_t* xh, const uint32_t* code, int M, int TK, int TN, int S,
                 float* part, hipStream_t s) {
    switch (R) {
      case 2: return go<2>(xh, code, M, TK, TN, S, part, s);
      case 4: return go<4>(xh, code, M, TK, TN, S, part, s);
      case 8: return go<8>(xh, code, M, TK, TN, S, part, s);
    }
    return fail(ESC_EINVAL, "rows per block R=%d not in {2,4,8}", R);
  }
};

// ---- one-launch linear for M < 16 (linear.hpp)
constexpr int kLinearSmallRows = 16;
constexpr int kLinearSmallRowsLut = 8;

// k_proj_rows1: partial slots per 256-column group, at least the workgroups
// a group of TK units can span: every workgroup holds at least 8 units when
// there are several (at most ceil(n / 16) workgroups for n units)
int rows1_maxc(int TK) { return TK / 8 + 2; }
// K=3 step pairs of every 8 that k_proj_rows1 decodes from the table
constexpr int kTablePairs3 = 4;

// One row (M = 1): the persistent table-mix kernel (k_proj_rows1) for the
// table decode of a projection of at least kRows1MinUnits units (kt x
// 256-column groups); the one-launch split-K kernel (k_linear_small) by hash
// otherwise, also when the table decode was asked for (the two decodes give
// the same weights; by hash the split-K kernel is ahead of its table form at
// every size).  Measured on MI355X with HIP-graph replay: K=2 5120 x 5120
// (6,400 units) 12.35 us by hash split-K against 14.8 us in the persistent
// kernel; K=3 5120 -> 17408 (21,760 units) 20.0 against 22.6 us, and
// 17408 -> 5120 level (23.2 against 23.1 us).
constexpr long kRows1MinUnits = 16384;
bool rows1_single(int M, int IC, int OC, bool lut) {
  return M == 1 && lut && OC % 256 == 0 && (long)(IC / 16) * (OC / 256) >= kRows1MinUnits;
}
// The decode a one-launch linear runs: the table only where the persistent
// kernel takes it (one row); 2..15 rows run the row-blocked split-K kernel by
// hash (the table form stages 128 KiB of LDS per workgroup and holds 8 rows:
// measured on MI355X at 4 rows, K=2 5120 x 5120 21.3 us by hash against
// 23.7 us, K=3 5120 -> 17408 30.9 against 48.9 us).
bool linear_uses_lut(int M, int IC, int OC, bool lut) { return rows1_single(M, IC, OC, lut); }
size_t rows1_part_bytes(int TK, int TN) { return (size_t)(TN / 16) * rows1_maxc(TK) * 256 * 4; }

struct LinearPlan {
  int R, S, KS, groups, row_groups;
  size_t off_part, off_cnt, off_xh, off_mid, total;
};

// Fewest splits that reach the workgroup target: more splits mean more
// float32 partials through the device-coherent path and a longer last-arriver
// sum; the table path also stages 128 KiB of LDS per workgroup.
LinearPlan linear_plan(int M, int K, int IC, int OC, bool lut) {
  LinearPlan p{};
  const int TK = IC / 16, TN = OC / 16, tpw = K == 2 ? 16 : 8;
  auto al = [](size_t v) { return (v + 255) & ~size_t(255); };
  if (M < kLinearSmallRows) {
    // every row of the group shares each decoded weight (one B column of
    // the matrix-core multiply each); the table path's LDS holds 8 rows
    p.R = std::min(M, lut ? kLinearSmallRowsLut : kLinearSmallRows - 1);
    p.groups = (TN + tpw - 1) / tpw;
    const int nb = TK / 8;  // 128-input blocks
    // fewest splits (largest KS <= 64) that reach `target` workgroups
    auto splits = [&](int row_groups, int target) {
      int best = nb;
      for (int S = 1; S <= std::min(nb, 64); ++S) {
        if (nb % S || 8 * (nb / S) > 64) continue;
        best = S;
        if (p.groups * row_groups * S >= target) break;
      }
      return best;
    };
    // Several rows by hash: each split's float32 partials (written and summed
    // back through the device-coherent level) grow with the rows, so fewer
    // splits than one row wants; and two row groups when one group at its
    // fewest splits leaves the GPU short of workgroups (each group decodes
    // the weights once, the partials halve again).  Measured on MI355X, K=2
    // 5120 x 5120: 4 rows 21.3 us at 200 workgroups against 23.9 us at 400;
    // 15 rows 30.9 us as 8 + 7 rows against 36.0 us as one group.
    if (!lut && M > 1 && p.R > kLinearSmallRowsLut && p.groups * splits(1, 0) < 256)
      p.R = (M + 1) / 2;
    p.row_groups = (M + p.R - 1) / p.R;
    // measured best on MI355X for 2048..17408 shapes
    const int target = lut ? 128 : M > 1 ? 200 : 256;
    p.S = splits(p.row_groups, target);
    p.KS = 8 * (nb / p.S);
    // counters first, sized for the most row groups either plan of this M
    // has (the table plan's 8-row groups), so that neither plan's partials
    // start inside the other's counters: one zero-filled workspace serves the
    // table and the hash plan alike
    const int rg_max = (M + kLinearSmallRowsLut - 1) / kLinearSmallRowsLut;
    p.off_cnt = 0;
    p.off_part = al((size_t)p.groups * std::max(p.row_groups, rg_max) * 4);
    p.total = p.off_part + al((size_t)p.S * M * OC * 4);
    // one row, OC a multiple of 256: room for the persistent kernel
    // (k_proj_rows1, also esc_linear_multi's), whose counters (one per 256
    // columns) fit in the ones above and whose partials start at off_part
    if (M == 1 && TN % 16 == 0)
      p.total = std::max(p.total, p.off_part + al(rows1_part_bytes(TK, TN)));
  } else {
    p.off_xh = 0;
    p.off_mid = al((size_t)M * IC * 2);
    p.total = p.off_mid + al((size_t)M * OC * 4);
  }
  return p;
}

esc::LinearSmallArgs small_args(const uint16_t* x, const float* rin, const uint32_t* code,
                                const float* rout, const uint16_t* bias, int M, int TK, int TN,
                                const LinearPlan& lp, float rs, float* part, int* cnt,
                                uint16_t* y) {
  return {x, rin, code, rout, bias, M, TK, TN, lp.KS, lp.R, lp.S, lp.groups, lp.row_groups, rs,
          part, cnt, y};
}

template <int K, bool LUT>
struct LinearSmallF {
  static int run(const esc::LinearSmallArgs& a, hipStream_t s) {
    // one row: VALU GEMV; several rows: matrix-core row-blocked GEMM
    constexpr int RMAX = LUT ? kLinearSmallRowsLut : kLinearSmallRows;
    if (a.R < 1 || a.R > RMAX) return fail(ESC_EINVAL, "rows per group %d > %d", a.R, RMAX);
    const dim3 grid(a.groups, a.row_groups, a.S);
    if (a.R == 1)
      hipLaunchKernelGGL((esc::k_linear_small<K, LUT, 1>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((esc::k_linear_small<K, LUT, RMAX>), grid, dim3(256), 0, s, a);
    return launched("k_linear_small");
  }
};

template <int K0, int K1, bool LUT>
int linear_pair_launch(const esc::LinearSmallArgs& a0, const esc::LinearSmallArgs& a1,
                       hipStream_t s) {
  constexpr int RMAX = LUT ? kLinearSmallRowsLut : kLinearSmallRows;
  if (a0.R != a1.R || a0.R < 1 || a0.R > RMAX)
    return fail(ESC_EINVAL, "rows per group %d / %d (max %d)", a0.R, a1.R, RMAX);
  const long n = (long)a0.groups * a0.row_groups * a0.S + (long)a1.groups * a1.row_groups * a1.S;
  if (a0.R == 1)
    hipLaunchKernelGGL((esc::k_linear_pair<K0, K1, LUT, 1>), dim3(n), dim3(256), 0, s, a0, a1);
  else
    hipLaunchKernelGGL((esc::k_linear_pair<K0, K1, LUT, RMAX>), dim3(n), dim3(256), 0, s, a0, a1);
  return launched("k_linear_pair");
}

template <bool LUT>
int linear_pair_k(int K0, int K1, const esc::LinearSmallArgs& a0, const esc::LinearSmallArgs& a1,
                  hipStream_t s) {
  if (K0 == 2) return K1 == 2 ? linear_pair_launch<2, 2, LUT>(a0, a1, s)
                              : linear_pair_launch<2, 3, LUT>(a0, a1, s);
  return K1 == 2 ? linear_pair_launch<3, 2, LUT>(a0, a1, s) : linear_pair_launch<3, 3, LUT>(a0, a1, s);
}

// Compute units of the current device (queried once per device).
int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cus[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

// k_proj_rows1 over a.np projections whose x .. TK, TN are filled: each
// projection's plan from its own shape (one workgroup per CU, or more when a
// wave would run more than kProjMaxP units), its workgroups after the
// previous projection's.  K=2 with the table decodes kTablePairsLayers of 8
// pairs from it, K=3 4 of 8.
template <int K, int NT>
int launch_rows1_k(const esc::ProjArgs& a, int grid, hipStream_t s) {
  static std::once_flag once;
  static hipError_t err = hipSuccess;
  if constexpr (NT > 0)
    std::call_once(once, [] {
      err = hipFuncSetAttribute((const void*)esc::k_proj_rows1<K, NT>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, 65536 * 2);
    });
  if (int rc = hip_check(err, "hipFuncSetAttribute")) return rc;
  const size_t lds = NT > 0 ? 65536 * 2 : esc::kProjLdsWork;
  hipLaunchKernelGGL((esc::k_proj_rows1<K, NT>), dim3(grid), dim3(64 * esc::kProjWaves), lds, s, a);
  return launched("k_proj_rows1");
}

// workgroups for n units: wgs, fewer when a wave would get fewer than two
// units, more when it would get more than kProjMaxP.  (Measured on MI355X:
// spreading 6,400 units over 256 workgroups, one or two per wave, is 5 %
// slower than 200 workgroups of two per wave -- more partials per group; 5 to
// 6 units per wave over 256 workgroups beat 6 over 227 by 2 %.)
int rows1_workgroups(long n, long wgs) {
  const long w = esc::kProjWaves;
  return (int)std::max(std::min(wgs, (n + 2 * w - 1) / (2 * w)),
                       (n + w * esc::kProjMaxP - 1) / (w * esc::kProjMaxP));
}

// merged: the workgroups shared out over the projections by their units
// (one round of workgroups for several small projections); otherwise each
// projection's from its own size alone, so that its outputs are those of
// its own launch.
int launch_rows1(esc::ProjArgs& a, int K, bool lut, hipStream_t s, bool merged = false) {
  // one workgroup per CU (two per CU without the table measured slower:
  // fewer units per wave, more partials per group)
  const int cus = device_cus();
  long total = 0;
  for (int i = 0; i < a.np; ++i) {
    ESC_REQUIRE((long)(a.pr[i].TN / 16) * a.pr[i].TK < (1L << 28), "projection too large");
    total += (long)(a.pr[i].TN / 16) * a.pr[i].TK;
  }
  long grid = 0;
  for (int i = 0; i < a.np; ++i) {
    esc::ProjOne& q = a.pr[i];
    q.n = (q.TN / 16) * q.TK;
    q.G = rows1_workgroups(q.n, merged ? std::max(1L, (cus * (long)q.n + total / 2) / total) : cus);
    q.maxc = rows1_maxc(q.TK);
    q.wg0 = (int)grid;
    grid += q.G;
  }
  if (lut)
    if (int rc = ensure_lut()) return rc;
  if (K == 2)
    return lut ? launch_rows1_k<2, esc::kTablePairsLayers>(a, (int)grid, s)
               : launch_rows1_k<2, 0>(a, (int)grid, s);
  return lut ? launch_rows1_k<3, kTablePairs3>(a, (int)grid, s) : launch_rows1_k<3, 0>(a, (int)grid, s);
}

// Row blocks of 16 per k_gemm_mma2 workgroup (NRB in {2,4,6,8}).  The kernel
// is decode-bound, so a tile's time grows slowly with its rows (measured on
// MI355X: 0.76 + 0.03 NRB, relative to NRB = 8), and a launch takes as many
// tile-times as the busiest CU holds tiles: pick the NRB that minimises
// ceil(tiles / CUs) * tile time.
int mma2_row_blocks(int M, int TN) {
  const int cus = device_cus();
  int best = 8;
  double best_cost = 1e30;
  for (int nrb = 8; nrb >= 2; nrb -= 2) {
    const long tiles = (long)((M + 16 * nrb - 1) / (16 * nrb)) * (TN / 16);
    const double cost = (double)((tiles + cus - 1) / cus) * (0.76 + 0.03 * nrb);
    if (cost < best_cost * 0.999) {
      best_cost = cost;
      best = nrb;
    }
  }
  return best;
}

// k_gemm_mma2 launch (TN % 16 == 0); OUT: output transform fused, y written.
template <bool OUT>
int gemm_mma2(int K, const uint16_t* xh, const uint32_t* code, int M, int TK, int TN, float* mid,
              const float* rout, const uint16_t* bias, float rs, uint16_t* y, hipStream_t s) {
  const int nrb = mma2_row_blocks(M, TN);
  const int blocks = ((M + 16 * nrb - 1) / (16 * nrb)) * (TN / 16);
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), 0, s, xh, code, M, TK, TN, mid, rout, bias,
                       rs, y);
  };
  if (K == 2) {
    if (nrb == 2) go(esc::k_gemm_mma2<2, 2, OUT>);
    else if (nrb == 4) go(esc::k_gemm_mma2<2, 4, OUT>);
    else if (nrb == 6) go(esc::k_gemm_mma2<2, 6, OUT>);
    else go(esc::k_gemm_mma2<2, 8, OUT>);
  } else {
    if (nrb == 2) go(esc::k_gemm_mma2<3, 2, OUT>);
    else if (nrb == 4) go(esc::k_gemm_mma2<3, 4, OUT>);
    else if (nrb == 6) go(esc::k_gemm_mma2<3, 6, OUT>);
    else go(esc::k_gemm_mma2<3, 8, OUT>);
  }
  return launched("k_gemm_mma2");
}

}  // namespace

extern "C" {

int esc_version(void) { return 100; }

const char* esc_last_error(void) { return g_err.c_str(); }

int esc_init(void) {
  if (int rc = ensure_lut()) return rc;
  if (int rc = ensure_wait_flag()) return rc;
  void* ptr = nullptr;
  return ensure_scratch(&ptr);
}

int esc_decode_tiles(const uint32_t* code, int K, int IC, int OC, int use_lut, uint16_t* w,
                     void* stream) {
  if (int rc = check_proj(K, IC, OC)) return rc;
  ESC_REQUIRE(code && w, "null pointer");
  if (use_lut)
    if (int rc = ensure_lut()) return rc;
  return by_k_lut<DecodeF>(K, use_lut, code, IC, OC, w, S(stream));
}

int esc_input_transform_typed(const void* rows, int dtype, const float* rin,
                              const int32_t* row_expert, int m, int IC, float rs, uint16_t* out,
                              void* stream) {
  ESC_REQUIRE(rows && rin && out, "null pointer");
  ESC_REQUIRE(IC > 0 && IC % 128 == 0, "Hadamard dimension must be divisible by 128, got %d", IC);
  ESC_REQUIRE(m >= 0, "negative row count");
  ESC_REQUIRE(dtype == ESC_ROWS_F16 || dtype == ESC_ROWS_BF16 || dtype == ESC_ROWS_F32,
              "row element type must be ESC_ROWS_F16, ESC_ROWS_BF16 or ESC_ROWS_F32, got %d",
              dtype);
  if (m == 0) return ESC_OK;
  const int ry = (m + esc::kTransformRows - 1) / esc::kTransformRows;
  const dim3 grid(IC / 128, ry), blk(256);
  if (dtype == ESC_ROWS_F16)
    hipLaunchKernelGGL(esc::k_input_transform<esc::kRowsF16>, grid, blk, 0, S(stream), rows, rin,
                       row_expert, m, IC, rs, out);
  else if (dtype == ESC_ROWS_BF16)
    hipLaunchKernelGGL(esc::k_input_transform<esc::kRowsBF16>, grid, blk, 0, S(stream), rows,
                       rin, row_expert, m, IC, rs, out);
  else
    hipLaunchKernelGGL(esc::k_input_transform<esc::kRowsF32>, grid, blk, 0, S(stream), rows, rin,
                       row_expert, m, IC, rs, out);
  return launched("k_input_transform");
}

int esc_input_transform(const uint16_t* rows, const float* rin, const int32_t* row_expert, int m,
                        int IC, float rs, uint16_t* out, void* stream) {
  return esc_input_transform_typed(rows, ESC_ROWS_F16, rin, row_expert, m, IC, rs, out, stream);
}

int esc_output_transform(const float* mid, const float* rout, const int32_t* row_expert,
                         const uint16_t* bias, int m, int OC, float rs, uint16_t* out,
                         void* stream) {
  ESC_REQUIRE(mid && rout && out, "null pointer");
  ESC_REQUIRE(OC > 0 && OC % 128 == 0, "Hadamard dimension must be divisible by 128, got %d", OC);
  ESC_REQUIRE(m >= 0, "negative row count");
  if (m == 0) return ESC_OK;
  const int ry = (m + esc::kTransformRows - 1) / esc::kTransformRows;
  if (row_expert)
    hipLaunchKernelGGL(esc::k_output_transform<true>, dim3(OC / 128, ry), dim3(256), 0, S(stream),
                       mid, rout, row_expert, bias, m, OC, rs, out);
  else
    hipLaunchKernelGGL(esc::k_output_transform<false>, dim3(OC / 128, ry), dim3(256), 0, S(stream),
                       mid, rout, row_expert, bias, m, OC, rs, out);
  return launched("k_output_transform");
}

int esc_gemv(const uint16_t* xh, const uint32_t* code, const int32_t* row_expert, int M, int K,
             int IC, int OC, int use_lut, float* mid, void* stream) {
  if (int rc = check_proj(K, IC, OC)) return rc;
  ESC_REQUIRE(xh && code && mid, "null pointer");
  ESC_REQUIRE(M >= 0, "negative row count");
  if (M == 0) return ESC_OK;
  if (use_lut)
    if (int rc = ensure_lut()) return rc;
  return exact_dispatch<esc::kPerRow>(K, use_lut, 1, xh, code, row_expert, nullptr, M, M,
                                      IC / 16, OC / 16, mid, S(stream));
}

size_t esc_gemv_fast_workspace(int M, int K, int IC, int OC) {
  if (check_proj(K, IC, OC) || M <= 0) return 0;
  return (size_t)fast_splits(K, M, IC / 16, OC / 16) * M * OC * sizeof(float);
}

int esc_gemv_fast_out(const uint16_t* xh, const uint32_t* code, const int32_t* row_expert,
                      const float* rout, int M, int K, int IC, int OC, int use_lut, float rs,
                      uint16_t* out, void* ws, size_t ws_bytes, void* stream) {
  if (int rc = check_proj(K, IC, OC)) return rc;
  ESC_REQUIRE(xh && code && rout && out, "null pointer");
  ESC_REQUIRE(M >= 0, "negative row count");
  if (M == 0) return ESC_OK;
  const int TK = IC / 16, TN = OC / 16;
  const int Sp = fast_splits(K, M, TK, TN);
  const size_t need = (size_t)Sp * M * OC * sizeof(float);
  if (!ws || ws_bytes < need)
    return fail(ESC_ENOSPACE, "workspace %zu bytes < required %zu", ws_bytes, need);
  if (use_lut)
    if (int rc = ensure_lut()) return rc;
  float* part = static_cast<float*>(ws);
  if (int rc = by_k_lut<FastF>(K, use_lut, xh, code, row_expert, M, TK, TN, Sp, part, S(stream)))
    return rc;
  hipLaunchKernelGGL(esc::k_splitk_out, dim3(OC / 128, M), dim3(64), 0, S(stream), part, Sp, M,
                     OC, rout, row_expert, rs, out);
  return launched("k_splitk_out");
}

size_t esc_linear_workspace(int M, int K, int IC, int OC) {
  if (check_proj(K, IC, OC) || M <= 0) return 0;
  return std::max(linear_plan(M, K, IC, OC, false).total, linear_plan(M, K, IC, OC, true).total);
}

int esc_linear(const uint16_t* x, const float* rin, const uint32_t* code, const float* rout,
               const uint16_t* bias, int M, int K, int IC, int OC, int use_lut, float rs,
               uint16_t* y, void* ws, size_t ws_bytes, void* stream) {
  if (int rc = check_proj(K, IC, OC)) return rc;
  ESC_REQUIRE(x && rin && code && rout && y, "null pointer");
  ESC_REQUIRE(M >= 0, "negative row count");
  if (M == 0) return ESC_OK;
  use_lut = linear_uses_lut(M, IC, OC, use_lut != 0);
  const LinearPlan lp = linear_plan(M, K, IC, OC, use_lut != 0);
  if (!ws || ws_bytes < lp.total)
    return fail(ESC_ENOSPACE, "workspace %zu bytes < required %zu", ws_bytes, lp.total);
  const int TK = IC / 16, TN = OC / 16;
  hipStream_t s = S(stream);
  char* w = static_cast<char*>(ws);
  if (rows1_single(M, IC, OC, use_lut != 0)) {
    // one row: the persistent kernel, its counters at off_cnt and its
    // partials at off_part (linear_plan sizes both)
    esc::ProjArgs a{};
    a.np = 1;
    a.rs = rs;
    a.pr[0] = esc::ProjOne{x, rin, code, rout, bias, y, reinterpret_cast<float*>(w + lp.off_part),
                           reinterpret_cast<int*>(w + lp.off_cnt), TK, TN};
    return launch_rows1(a, K, use_lut != 0, s);
  }
  if (M < kLinearSmallRows) {
    // the split-K kernel, by hash (linear_uses_lut)
    float* part = reinterpret_cast<float*>(w + lp.off_part);
    int* cnt = reinterpret_cast<int*>(w + lp.off_cnt);
    const esc::LinearSmallArgs a = small_args(x, rin, code, rout, bias, M, TK, TN, lp, rs, part, cnt, y);
    return K == 2 ? LinearSmallF<2, false>::run(a, s) : LinearSmallF<3, false>::run(a, s);
  }
  // many rows: input transform, then the matrix-core GEMM with the output
  // transform in its epilogue (or GEMM + output transform for OC % 256 != 0)
  uint16_t* xh = reinterpret_cast<uint16_t*>(w + lp.off_xh);
  if (int rc = esc_input_transform(x, rin, nullptr, M, IC, rs, xh, stream)) return rc;
  return esc_gemm_mfma_out(xh, code, rout, bias, M, K, IC, OC, rs, y, w + lp.off_mid,
                           lp.total - lp.off_mid, stream);
}

size_t esc_gemm_mfma_out_workspace(int M, int K, int IC, int OC) {
  if (check_proj(K, IC, OC) || M <= 0) return 0;
  return OC % 256 ? (size_t)M * OC * sizeof(float) : 0;
}

int esc_gemm_mfma_out(const uint16_t* xh, const uint32_t* code, const float* rout,
                      const uint16_t* bias, int M, int K, int IC, int OC, float rs, uint16_t* y,
                      void* ws, size_t ws_bytes, void* stream) {
  if (int rc = check_proj(K, IC, OC)) return rc;
  ESC_REQUIRE(xh && code && rout && y, "null pointer");
  ESC_REQUIRE(M >= 0, "negative row count");
  if (M == 0) return ESC_OK;
  const int TK = IC / 16, TN = OC / 16;
  hipStream_t s = S(stream);
  // OC a multiple of 256: the output transform in the GEMM's epilogue
  if (TN % 16 == 0) return gemm_mma2<true>(K, xh, code, M, TK, TN, nullptr, rout, bias, rs, y, s);
  const size_t need = esc_gemm_mfma_out_workspace(M, K, IC, OC);
  if (!ws || ws_bytes < need)
    return fail(ESC_ENOSPACE, "workspace %zu bytes < required %zu", ws_bytes, need);
  float* mid = static_cast<float*>(ws);
  if (int rc = esc_gemm_mfma(xh, code, M, K, IC, OC, 0, mid, stream)) return rc;
  return esc_output_transform(mid, rout, nullptr, bias, M, OC, rs, y, stream);
}

size_t esc_linear_pair_workspace(int M, int K0, int K1, int IC, int OC0, int OC1) {
  const size_t a = esc_linear_workspace(M, K0, IC, OC0), b = esc_linear_workspace(M, K1, IC, OC1);
  if (!a || !b) return 0;
  return ((a + 255) & ~size_t(255)) + b;
}

int esc_linear_pair(const uint16_t* x, int M, int IC, const float* rin0, const uint32_t* code0,
                    const float* rout0, const uint16_t* bias0, int K0, int OC0, const float* rin1,
                    const uint32_t* code1, const float* rout1, const uint16_t* bias1, int K1,
                    int OC1, int use_lut, float rs, uint16_t* y0, uint16_t* y1, void* ws,
                    size_t ws_bytes, void* stream) {
  if (int rc = check_proj(K0, IC, OC0)) return rc;
  if (int rc = check_proj(K1, IC, OC1)) return rc;
  ESC_REQUIRE(x && rin0 && code0 && rout0 && y0 && rin1 && code1 && rout1 && y1, "null pointer");
  ESC_REQUIRE(M >= 0, "negative row count");
  if (M == 0) return ESC_OK;
  const size_t need = esc_linear_pair_workspace(M, K0, K1, IC, OC0, OC1);
  if (!ws || ws_bytes < need)
    return fail(ESC_ENOSPACE, "workspace %zu bytes < required %zu", ws_bytes, need);
  // projection 1's workspace follows projection 0's (each as esc_linear's)
  const size_t ws0 = esc_linear_workspace(M, K0, IC, OC0);
  const size_t off1 = (ws0 + 255) & ~size_t(255);
  char* w = static_cast<char*>(ws);
  if (M >= kLinearSmallRows) {
    // many rows: each projection's GEMM fills the GPU on its own
    if (int rc = esc_linear(x, rin0, code0, rout0, bias0, M, K0, IC, OC0, use_lut, rs, y0, w, ws0,
                            stream))
      return rc;
    return esc_linear(x, rin1, code1, rout1, bias1, M, K1, IC, OC1, use_lut, rs, y1, w + off1,
                      ws_bytes - off1, stream);
  }
  const bool r0 = rows1_single(M, IC, OC0, use_lut != 0), r1 = rows1_single(M, IC, OC1, use_lut != 0);
  // the pair kernel runs the decode each projection's own call would
  if (!r0 && !r1) use_lut = 0;
  if (use_lut)
    if (int rc = ensure_lut()) return rc;
  const int TK = IC / 16;
  const LinearPlan p0 = linear_plan(M, K0, IC, OC0, use_lut != 0);
  const LinearPlan p1 = linear_plan(M, K1, IC, OC1, use_lut != 0);
  char* w1 = w + off1;
  if (r0 && r1 && K0 == K1) {
    // one row: both projections in one persistent launch, each with its own
    // plan and workspace, so each output is its own esc_linear call's
    esc::ProjArgs a{};
    a.np = 2;
    a.rs = rs;
    a.pr[0] = esc::ProjOne{x, rin0, code0, rout0, bias0, y0,
                           reinterpret_cast<float*>(w + p0.off_part),
                           reinterpret_cast<int*>(w + p0.off_cnt), TK, OC0 / 16};
    a.pr[1] = esc::ProjOne{x, rin1, code1, rout1, bias1, y1,
                           reinterpret_cast<float*>(w1 + p1.off_part),
                           reinterpret_cast<int*>(w1 + p1.off_cnt), TK, OC1 / 16};
    return launch_rows1(a, K0, use_lut != 0, S(stream));
  }
  if (r0 || r1 || p0.R != p1.R) {
    // one row with the projections on different kernels (or K), or row
    // groups of different sizes: each as its own call
    if (int rc = esc_linear(x, rin0, code0, rout0, bias0, M, K0, IC, OC0, use_lut, rs, y0, w, ws0,
                            stream))
      return rc;
    return esc_linear(x, rin1, code1, rout1, bias1, M, K1, IC, OC1, use_lut, rs, y1, w + off1,
                      ws_bytes - off1, stream);
  }
  const esc::LinearSmallArgs a0 =
      small_args(x, rin0, code0, rout0, bias0, M, TK, OC0 / 16, p0, rs,
                 reinterpret_cast<float*>(w + p0.off_part), reinterpret_cast<int*>(w + p0.off_cnt), y0);
  const esc::LinearSmallArgs a1 =
      small_args(x, rin1, code1, rout1, bias1, M, TK, OC1 / 16, p1, rs,
                 reinterpret_cast<float*>(w1 + p1.off_part), reinterpret_cast<int*>(w1 + p1.off_cnt), y1);
  // the split-K pair kernel, by hash (linear_uses_lut)
  return linear_pair_k<false>(K0, K1, a0, a1, S(stream));
}

size_t esc_linear_multi_workspace(int M, int n, int K, int IC, const int* OC) {
  if (M <= 0 || n < 1 || n > esc::kProjMax || !OC) return 0;
  size_t total = 0;
  for (int i = 0; i < n; ++i) {
    if (check_proj(K, IC, OC[i])) return 0;
    if (M == 1) {
      if (OC[i] % 256) return 0;
      // this projection's counters, then its partials
      total += ((size_t)(OC[i] / 256) * 4 + 255) / 256 * 256 + rows1_part_bytes(IC / 16, OC[i] / 16);
    } else {
      // this projection's esc_linear workspace
      total += (esc_linear_workspace(M, K, IC, OC[i]) + 255) & ~size_t(255);
    }
  }
  return total;
}

int esc_linear_multi(const uint16_t* x, int M, int IC, int K, int n, const uint32_t* const* code,
                     const float* const* rin, const float* const* rout,
                     const uint16_t* const* bias, const int* OC, int use_lut, float rs,
                     uint16_t* const* y, void* ws, size_t ws_bytes, void* stream) {
  ESC_REQUIRE(x && code && rin && rout && OC && y, "null pointer");
  ESC_REQUIRE(M >= 0, "negative row count");
  ESC_REQUIRE(n >= 1 && n <= esc::kProjMax, "%d projections (1 to %d)", n, esc::kProjMax);
  static_assert(esc::kLinearMultiMax == esc::kProjMax, "projections per launch");
  for (int i = 0; i < n; ++i) {
    if (int rc = check_proj(K, IC, OC[i])) return rc;
    ESC_REQUIRE(code[i] && rin[i] && rout[i] && y[i], "null pointer (projection %d)", i);
    ESC_REQUIRE(M != 1 || OC[i] % 256 == 0, "OC=%d of projection %d is not a multiple of 256",
                OC[i], i);
  }
  if (M == 0) return ESC_OK;
  const size_t need = esc_linear_multi_workspace(M, n, K, IC, OC);
  if (!ws || ws_bytes < need)
    return fail(ESC_ENOSPACE, "workspace %zu bytes < required %zu", ws_bytes, need);
  char* w = static_cast<char*>(ws);
  if (M == 1) {
    // one row: one persistent k_proj_rows1 launch, the units of all
    // projections split over its waves
    esc::ProjArgs a{};
    a.np = n;
    a.rs = rs;
    for (int i = 0; i < n; ++i) {
      int* cnt = reinterpret_cast<int*>(w);
      w += ((size_t)(OC[i] / 256) * 4 + 255) / 256 * 256;
      float* part = reinterpret_cast<float*>(w);
      w += rows1_part_bytes(IC / 16, OC[i] / 16);
      a.pr[i] = esc::ProjOne{x, rin[i], code[i], rout[i], bias ? bias[i] : nullptr, y[i], part,
                             cnt, IC / 16, OC[i] / 16};
    }
    return launch_rows1(a, K, use_lut != 0, S(stream), true);
  }
  // several rows: each projection's esc_linear plan and workspace, as one
  // k_linear_multi launch when all run the split-K kernel with one row group
  // size, else one call each
  size_t off[esc::kProjMax];
  LinearPlan pl[esc::kProjMax];
  bool one = M < kLinearSmallRows;
  size_t o = 0;
  for (int i = 0; i < n; ++i) {
    off[i] = o;
    o += (esc_linear_workspace(M, K, IC, OC[i]) + 255) & ~size_t(255);
    pl[i] = linear_plan(M, K, IC, OC[i], false);
    one = one && pl[i].R == pl[0].R;
  }
  if (!one) {
    for (int i = 0; i < n; ++i)
      if (int rc = esc_linear(x, rin[i], code[i], rout[i], bias ? bias[i] : nullptr, M, K, IC,
                              OC[i], use_lut, rs, y[i], w + off[i], ws_bytes - off[i], stream))
        return rc;
    return ESC_OK;
  }
  esc::LinearMultiArgs m{};
  m.n = n;
  long nw = 0;
  for (int i = 0; i < n; ++i) {
    char* wi = w + off[i];
    m.p[i] = small_args(x, rin[i], code[i], rout[i], bias ? bias[i] : nullptr, M, IC / 16, OC[i] / 16,
                        pl[i], rs, reinterpret_cast<float*>(wi + pl[i].off_part),
                        reinterpret_cast<int*>(wi + pl[i].off_cnt), y[i]);
    nw += (long)pl[i].groups * pl[i].row_groups * pl[i].S;
  }
  ESC_REQUIRE(pl[0].R >= 2 && pl[0].R <= kLinearSmallRows, "rows per group %d", pl[0].R);
  if (K == 2)
    hipLaunchKernelGGL((esc::k_linear_multi<2, kLinearSmallRows>), dim3(nw), dim3(256), 0, S(stream), m);
  else
    hipLaunchKernelGGL((esc::k_linear_multi<3, kLinearSmallRows>), dim3(nw), dim3(256), 0, S(stream), m);
  return launched("k_linear_multi");
}

size_t esc_gemm_rows_fast_workspace(int M, int R, int K, int IC, int OC) {
  if (check_proj(K, IC, OC) || M <= 0 || R <= 0) return 0;
  return (size_t)fast_splits(K, (M + R - 1) / R, IC / 16, OC / 16) * M * OC * sizeof(float);
}

int esc_gemm_rows_fast_out(const uint16_t* xh, const uint32_t* code, const float* rout, int M,
                           int R, int K, int IC, int OC, int use_lut, float rs, uint16_t* out,
                           void* ws, size_t ws_bytes, void* stream) {
  if (int rc = check_proj(K, IC, OC)) return rc;
  ESC_REQUIRE(xh && code && rout && out, "null pointer");
  ESC_REQUIRE(M >= 0, "negative row count");
  ESC_REQUIRE(R == 2 || R == 4 || R == 8, "rows per block R=%d not in {2,4,8}", R);
  if (M == 0) return ESC_OK;
  const int TK = IC / 16, TN = OC / 16;
  const int Sp = fast_splits(K, (M + R - 1) / R, TK, TN);
  const size_t need = (size_t)Sp * M * OC * sizeof(float);
  if (!ws || ws_bytes < need)
    return fail(ESC_ENOSPACE, "workspace %zu bytes < required %zu", ws_bytes, need);
  if (use_lut)
    if (int rc = ensure_lut()) return rc;
  float* part = static_cast<float*>(ws);
  hipStream_t s = S(stream);
  int rc;
  if (K == 2)
    rc = use_lut ? FastRowsF<2, true>::run(R, xh, code, M, TK, TN, Sp, part, s)
                 : FastRowsF<2, false>::run(R, xh, code, M, TK, TN, Sp, part, s);
  else
    rc = use_lut ? FastRowsF<3, true>::run(R, xh, code, M, TK, TN, Sp, part, s)
                 : FastRowsF<3, false>::run(R, xh, code, M, TK, TN, Sp, part, s);
  if (rc) return rc;
  hipLaunchKernelGGL(esc::k_splitk_out, dim3(OC / 128, M), dim3(64), 0, s, part, Sp, M, OC, rout,
                     nullptr, rs, out);
  return launched("k_splitk_out");
}

int esc_gemm_rows(const uint16_t* xh, const uint32_t* code, const int32_t* rows_idx,
                  const int32_t* group_expert, int n_groups, int R, int n_rows, int K, int IC,
                  int OC, int use_lut, float* mid, void* stream) {
  if (int rc = check_proj(K, IC, OC)) return rc;
  ESC_REQUIRE(xh && code && rows_idx && group_expert && mid, "null pointer");
  ESC_REQUIRE(n_groups >= 0 && n_rows >= 0, "negative size");
  if (n_groups == 0) return ESC_OK;
  if (use_lut)
    if (int rc = ensure_lut()) return rc;
  return exact_dispatch<esc::kMoeGroups>(K, use_lut, R, xh, code, rows_idx, group_expert, n_rows,
                                         n_groups, IC / 16, OC / 16, mid, S(stream));
}

int esc_dense_gemm_rows(const uint16_t* xh, const uint32_t* code, int M, int R, int K, int IC,
                        int OC, int use_lut, float* mid, void* stream) {
  if (int rc = check_proj(K, IC, OC)) return rc;
  ESC_REQUIRE(xh && code && mid, "null pointer");
  ESC_REQUIRE(M >= 0, "negative row count");
  ESC_REQUIRE(R == 1 || R == 2 || R == 4 || R == 8 || R == 16, "dense R=%d not in {1,2,4,8,16}", R);
  if (M == 0) return ESC_OK;
  if (use_lut)
    if (int rc = ensure_lut()) return rc;
  return exact_dispatch<esc::kDenseRows>(K, use_lut, R, xh, code, nullptr, nullptr, M,
                                         (M + R - 1) / R, IC / 16, OC / 16, mid, S(stream));
}

int esc_dense_gemm_rows_out(const uint16_t* xh, const uint32_t* code, const float* rout, int M,
                            int R, int K, int IC, int OC, int use_lut, float rs, uint16_t* out,
                            void* stream) {
  if (int rc = check_proj(K, IC, OC)) return rc;
  ESC_REQUIRE(xh && code && rout && out, "null pointer");
  ESC_REQUIRE(M >= 0, "negative row count");
  if (M == 0) return ESC_OK;
  if (use_lut)
    if (int rc = ensure_lut()) return rc;
  const int TK = IC / 16, TN = OC / 16;
  hipStream_t s = S(stream);
  if (K == 2)
    return use_lut ? ExactOutF<2, true>::run(R, xh, code, rout, M, TK, TN, rs, out, s)
                   : ExactOutF<2, false>::run(R, xh, code, rout, M, TK, TN, rs, out, s);
  return use_lut ? ExactOutF<3, true>::run(R, xh, code, rout, M, TK, TN, rs, out, s)
                 : ExactOutF<3, false>::run(R, xh, code, rout, M, TK, TN, rs, out, s);
}

int esc_gemm_mfma(const uint16_t* xh, const uint32_t* code, int M, int K, int IC, int OC,
                  int use_lut, float* mid, void* stream) {
  if (int rc = check_proj(K, IC, OC)) return rc;
  ESC_REQUIRE(xh && code && mid, "null pointer");
  ESC_REQUIRE(M >= 0, "negative row count");
  (void)use_lut;  // the table holds the hash's own values: both decodes give the same bits
  if (M == 0) return ESC_OK;
  const int TK = IC / 16, TN = OC / 16;
  hipStream_t s = S(stream);
  if (TN % 16 == 0)
    return gemm_mma2<false>(K, xh, code, M, TK, TN, mid, nullptr, nullptr, 0.f, nullptr, s);
  const int blocks = ((M + esc::kMmaRows - 1) / esc::kMmaRows) * (TN / 8);
  if (K == 2)
    hipLaunchKernelGGL(esc::k_gemm_mfma<2>, dim3(blocks), dim3(esc::kMmaThreads), 0, s, xh, code,
                       M, TK, TN, mid);
  else
    hipLaunchKernelGGL(esc::k_gemm_mfma<3>, dim3(blocks), dim3(esc::kMmaThreads), 0, s, xh, code,
                       M, TK, TN, mid);
  return launched("k_gemm_mfma");
}

int esc_build_groups(const int32_t* row_expert, int m, int E, int R, int n_groups,
                     int32_t* rows_idx, int32_t* group_expert, void* stream) {
  ESC_REQUIRE(row_expert && rows_idx && group_expert, "null pointer");
  ESC_REQUIRE(E > 0 && E <= 4096, "expert count %d not in [1, 4096]", E);
  ESC_REQUIRE(R >= 1 && m >= 0, "bad R=%d / m=%d", R, m);
  const long bound = ((long)m + (long)E * (R - 1) + R - 1) / R;
  ESC_REQUIRE(n_groups >= bound, "n_groups %d below the bound %ld", n_groups, bound);
  hipLaunchKernelGGL(esc::k_build_groups, dim3(1), dim3(1024), 0, S(stream), row_expert, m, E, R,
                     n_groups, rows_idx, group_expert);
  return launched("k_build_groups");
}

int esc_route_topk(const float* logits, int T, int E, int top_k, int32_t* ids, float* scores,
                   void* stream) {
  ESC_REQUIRE(logits && ids && scores, "null pointer");
  ESC_REQUIRE(E > 0 && E <= 1024, "expert count %d not in [1, 1024]", E);
  ESC_REQUIRE(top_k >= 1 && top_k <= 32 && top_k <= E, "top_k %d not in [1, min(32, E)]", top_k);
  ESC_REQUIRE(T >= 0, "negative token count");
  if (T == 0) return ESC_OK;
  hipLaunchKernelGGL(esc::k_route_topk, dim3(T), dim3(64), 0, S(stream), logits, E, top_k, ids,
                     scores);
  return launched("k_route_topk");
}

int esc_swiglu(const uint16_t* gu, int m, int I, uint16_t* h, void* stream) {
  ESC_REQUIRE(gu && h, "null pointer");
  ESC_REQUIRE(m >= 0 && I > 0, "bad m=%d / I=%d", m, I);
  if (m == 0) return ESC_OK;
  hipLaunchKernelGGL(esc::k_swiglu, dim3((I + 255) / 256, m), dim3(256), 0, S(stream), gu, I, h);
  return launched("k_swiglu");
}

int esc_moe_combine(const uint16_t* d16, const float* scores, int T, int top_k, int H,
                    uint16_t* y, void* stream) {
  ESC_REQUIRE(d16 && scores && y, "null pointer");
  ESC_REQUIRE(T >= 0 && top_k >= 1 && H > 0, "bad T=%d / top_k=%d / H=%d", T, top_k, H);
  if (T == 0) return ESC_OK;
  hipLaunchKernelGGL(esc::k_combine, dim3((H + 255) / 256, T), dim3(256), 0, S(stream), d16,
                     scores, top_k, H, y);
  return launched("k_combine");
}

// ---- dense int8 / f16 GEMV (q8.hpp): shared expert, gates, vocabulary head

}  // extern "C"

namespace {
// k_rows_gemv geometry: LPR lanes per output row (the row's 16-byte chunk
// count rounded up to a power of two, 8..64), CPL chunks per lane (1..8).
// The lanes keep NR rows of x in registers, NR * CPL * XW words (XW = 8 f16
// pairs per int8 chunk, 4 per f16 chunk): rows per launch are capped at 128
// such words.
constexpr int kRowsXWords = 128;
constexpr int kRowsMaxCpl = 8;

struct RowsGeo {
  int lpr, cpl;
};
RowsGeo rows_geo(int chunks) {
  int lpr = 8;
  while (lpr < chunks && lpr < 64) lpr *= 2;
  return {lpr, (chunks + lpr - 1) / lpr};
}
constexpr int rows_x_words(bool q8) { return q8 ? 8 : 4; }
int rows_nr_max(bool q8, int cpl) {
  int nr = 8;
  while (nr > 1 && nr * cpl * rows_x_words(q8) > kRowsXWords) nr /= 2;
  return nr;
}

template <bool Q8, int NR, int LPR, int CPL>
int rows_launch(const uint16_t* x, const void* w, const float* scale, int M, int K, int O,
                uint16_t* y, hipStream_t s) {
  if constexpr (NR * CPL * rows_x_words(Q8) > kRowsXWords) {
    return fail(ESC_EINVAL, "internal: %d rows x %d chunks exceed the register budget", NR, CPL);
  } else {
    const long steps = ((long)O + 64 / LPR - 1) / (64 / LPR);
    // eight workgroups per CU, each wave striding over the row steps (measured
    // on MI355X with the 248320 x 2048 head: 103 us at 8 per CU, 107 us at 4,
    // 16 no better than 8)
    const int blocks = (int)std::min<long>((steps + 3) / 4, 8L * device_cus());
    hipLaunchKernelGGL((esc::k_rows_gemv<Q8, NR, LPR, CPL>), dim3(blocks), dim3(256), 0, s, x, w,
                       scale, M, K, O, y, O);
    return launched("k_rows_gemv");
  }
}

template <bool Q8, int NR>
int rows_by_geo(RowsGeo g, const uint16_t* x, const void* w, const float* scale, int M, int K,
                int O, uint16_t* y, hipStream_t s) {
  switch (g.lpr) {
    case 8: return rows_launch<Q8, NR, 8, 1>(x, w, scale, M, K, O, y, s);
    case 16: return rows_launch<Q8, NR, 16, 1>(x, w, scale, M, K, O, y, s);
    case 32: return rows_launch<Q8, NR, 32, 1>(x, w, scale, M, K, O, y, s);
  }
  switch (g.cpl) {
    case 1: return rows_launch<Q8, NR, 64, 1>(x, w, scale, M, K, O, y, s);
    case 2: return rows_launch<Q8, NR, 64, 2>(x, w, scale, M, K, O, y, s);
    case 3: return rows_launch<Q8, NR, 64, 3>(x, w, scale, M, K, O, y, s);
    case 4: return rows_launch<Q8, NR, 64, 4>(x, w, scale, M, K, O, y, s);
    case 5: return rows_launch<Q8, NR, 64, 5>(x, w, scale, M, K, O, y, s);
    case 6: return rows_launch<Q8, NR, 64, 6>(x, w, scale, M, K, O, y, s);
    case 7: return rows_launch<Q8, NR, 64, 7>(x, w, scale, M, K, O, y, s);
    default: return rows_launch<Q8, NR, 64, 8>(x, w, scale, M, K, O, y, s);
  }
}

// int8 weights and 2..16 rows per launch: k_rows_w8_mma, the rows' products on
// the matrix core (x staged in LDS, at most kW8MmaLds bytes per workgroup)
constexpr int kW8MmaLds = 64 * 1024;
int w8_mma_rows(int M, int K) {
  if (M < 2 || K % 64) return 0;
  return std::min(16, kW8MmaLds / (2 * K + 16));
}

int rows_w8_mma(const uint16_t* x, const void* w, const float* scale, int M, int K, int O,
                uint16_t* y, int nr, hipStream_t s) {
  const int groups = (O + 15) / 16;
  for (int m0 = 0; m0 < M; m0 += nr) {
    const int mr = std::min(nr, M - m0);
    const size_t lds = (size_t)mr * (2 * K + 16);
    const int per_cu = (int)std::max<size_t>(1, std::min<size_t>(8, 160 * 1024 / lds));
    const int blocks = std::min((groups + 3) / 4, per_cu * device_cus());
    hipLaunchKernelGGL(esc::k_rows_w8_mma, dim3(blocks), dim3(256), lds, s, x + (size_t)m0 * K,
                       static_cast<const int8_t*>(w), scale, mr, K, O, y + (size_t)m0 * O, O);
    if (int rc = launched("k_rows_w8_mma")) return rc;
  }
  return ESC_OK;
}

template <bool Q8>
int rows_gemv(const uint16_t* x, const void* w, const float* scale, int M, int K, int O,
              uint16_t* y, hipStream_t s) {
  const int cw = Q8 ? 16 : 8;  // weights per 16-byte chunk
  const int chunks = K / cw;
  ESC_REQUIRE(K > 0 && K % cw == 0 && chunks >= 8 && chunks <= 64 * kRowsMaxCpl,
              "K=%d: need a multiple of %d in [%d, %d]", K, cw, 8 * cw, 64 * kRowsMaxCpl * cw);
  if constexpr (Q8) {
    if (const int nr = w8_mma_rows(M, K); nr >= 2) return rows_w8_mma(x, w, scale, M, K, O, y, nr, s);
  }
  const RowsGeo g = rows_geo(chunks);
  const int nr_max = rows_nr_max(Q8, g.cpl);
  for (int m0 = 0; m0 < M; m0 += nr_max) {
    const int mr = std::min(nr_max, M - m0);
    const uint16_t* xm = x + (size_t)m0 * K;
    uint16_t* ym = y + (size_t)m0 * O;
    int rc;
    if (mr == 1) rc = rows_by_geo<Q8, 1>(g, xm, w, scale, mr, K, O, ym, s);
    else if (mr == 2) rc = rows_by_geo<Q8, 2>(g, xm, w, scale, mr, K, O, ym, s);
    else if (mr <= 4) rc = rows_by_geo<Q8, 4>(g, xm, w, scale, mr, K, O, ym, s);
    else rc = rows_by_geo<Q8, 8>(g, xm, w, scale, mr, K, O, ym, s);
    if (rc) return rc;
  }
  return ESC_OK;
}
}  // namespace

extern "C" {

int esc_w8a16(const uint16_t* x, const int8_t* w8, const float* scale, int M, int K, int O,
              uint16_t* y, void* stream) {
  ESC_REQUIRE(x && w8 && scale && y, "null pointer");
  ESC_REQUIRE(M >= 0 && O > 0, "bad M=%d / O=%d", M, O);
  if (M == 0) return ESC_OK;
  return rows_gemv<true>(x, w8, scale, M, K, O, y, S(stream));
}

int esc_gemv_f16w(const uint16_t* x, const uint16_t* w, int M, int K, int O, uint16_t* y,
                  void* stream) {
  ESC_REQUIRE(x && w && y, "null pointer");
  ESC_REQUIRE(M >= 0 && O > 0, "bad M=%d / O=%d", M, O);
  if (M == 0) return ESC_OK;
  return rows_gemv<false>(x, w, nullptr, M, K, O, y, S(stream));
}

int esc_moe_shared_act(const uint16_t* g, const uint16_t* u, int m, int I, uint16_t* hh,
                       void* stream) {
  ESC_REQUIRE(g && u && hh, "null pointer");
  ESC_REQUIRE(m >= 0 && I > 0, "bad m=%d / I=%d", m, I);
  if (m == 0) return ESC_OK;
  hipLaunchKernelGGL(esc::k_shared_act, dim3((I + 255) / 256, m), dim3(256), 0, S(stream), g, u,
                     I, hh);
  return launched("k_shared_act");
}

int esc_moe_block_out(const uint16_t* y, const uint16_t* sh, const uint16_t* shg, int m, int H,
                      uint16_t* out, void* stream) {
  ESC_REQUIRE(y && sh && shg && out, "null pointer");
  ESC_REQUIRE(m >= 0 && H > 0, "bad m=%d / H=%d", m, H);
  if (m == 0) return ESC_OK;
  hipLaunchKernelGGL(esc::k_block_out, dim3((H + 255) / 256, m), dim3(256), 0, S(stream), y, sh,
                     shg, H, out);
  return launched("k_block_out");
}

int esc_q8_embed(const int32_t* ids, int T, const int8_t* w8, const float* scale, int N, int K,
                 uint16_t* out, void* stream) {
  ESC_REQUIRE(ids && w8 && scale && out, "null pointer");
  ESC_REQUIRE(T >= 0 && N > 0 && K > 0 && K % 16 == 0, "bad T=%d / N=%d / K=%d (K a multiple of 16)",
              T, N, K);
  if (T == 0) return ESC_OK;
  hipLaunchKernelGGL(esc::k_q8_embed, dim3(T), dim3(256), 0, S(stream), ids, w8, scale, N, K, out);
  return launched("k_q8_embed");
}

}  // extern "C"

// ---- routed experts: input transform -> gate_up -> swiglu/transform -> down -> combine
namespace {
// Rows per expert group of the split-K chain: once there are as many routed
// rows as experts, rows of one expert share each decoded weight (groups laid
// out by moe.build_groups, one row per B column of the matrix-core multiply,
// so a group costs one decode whatever its row count); below that almost
// every expert has one row.
constexpr int kMoeGroupRows = 8;
int moe_group_rows(int M, int E) { return M >= E ? kMoeGroupRows : 0; }

int moe_input(const uint16_t* x, const int32_t* ids, int top_k, const float* rin, int H, float rs,
              uint16_t* xh, int M, hipStream_t s) {
  hipLaunchKernelGGL(esc::k_moe_input, dim3(H / 128, M), dim3(64), 0, s, x, ids, top_k, rin, H, rs,
                     xh);
  return launched("k_moe_input");
}

struct MoePlan {
  int M, S1, S2, R, n_groups;
  size_t off_xh, off_p1, off_xh2, off_p2, off_rows, off_gexp, off_nact, total;
};
// base: bytes at the start of the workspace left to the caller (the
// no-allocation variant keeps its counters there).
MoePlan moe_plan(int T, int top_k, int E, int H, int I, int K_gu, int K_dn, size_t base = 0) {
  MoePlan p;
  p.M = T * top_k;
  p.R = E <= 4096 ? moe_group_rows(p.M, E) : 0;
  p.n_groups = p.R ? (p.M + E * (p.R - 1) + p.R - 1) / p.R : 0;
  // non-empty groups, about: the experts a uniform routing touches, or M/R
  const int eff = p.R ? std::max((p.M + p.R - 1) / p.R,
                                 (int)(E * (1.0 - std::pow(1.0 - 1.0 / E, (double)p.M))))
                      : p.M;
  // the grouped GEMVs aim for 2048 blocks: at 32 tokens (E = 256, H = 2048,
  // I = 512, top-8) 1,201 GB/s against 1,171 at 1024, 1,147 at 512 and
  // 1,161 at 4096 on MI355X; below about 16 tokens the kt bound sets S first
  p.S1 = fast_splits(K_gu, eff, H / 16, 2 * I / 16, 2048);
  p.S2 = fast_splits(K_dn, eff, I / 16, H / 16, 2048);
  auto al = [](size_t v) { return (v + 255) & ~size_t(255); };
  p.off_xh = al(base);
  p.off_p1 = al(p.off_xh + (size_t)p.M * H * 2);
  p.off_xh2 = al(p.off_p1 + (size_t)p.S1 * p.M * 2 * I * 4);
  p.off_p2 = al(p.off_xh2 + (size_t)p.M * I * 2);
  p.off_rows = al(p.off_p2 + (size_t)p.S2 * p.M * H * 4);
  p.off_gexp = al(p.off_rows + (size_t)p.n_groups * p.R * 4);
  p.off_nact = al(p.off_gexp + (size_t)p.n_groups * 4);
  p.total = al(p.off_nact + 4);
  return p;
}

template <int K, bool LUT>
struct GroupRowsF {
  template <int R>
  static int go(const uint16_t* xh, const uint32_t* code, const int* rows, const int* gexp,
                int n_groups, int M, int TK, int TN, int S, float* part, hipStream_t s) {
    const int tpw = K == 2 ? 16 : 8;
    hipLaunchKernelGGL((esc::k_gemv_fast_rows<K, LUT, R>), dim3((TN + tpw - 1) / tpw, n_groups, S),
                       dim3(256), 0, s, xh, code, rows, gexp, M, TK, TN, TK / S, part);
    return launched("k_gemv_fast_rows");
  }
  static int run(int R, const uint16_t* xh, const uint32_t* code, const int* rows, const int* gexp,
                 int n_groups, int M, int TK, int TN, int S, float* part, hipStream_t s) {
    if (R != kMoeGroupRows) return fail(ESC_EINVAL, "rows per expert group %d", R);
    return go<kMoeGroupRows>(xh, code, rows, gexp, n_groups, M, TK, TN, S, part, s);
  }
};

// The grouped GEMM with the table decode: the persistent k_gemv_rows_table
// (one workgroup per CU, the table staged once), its item count from the
// groups build_groups filled (nact, on the device).
template <int K>
int launch_rows_table(const uint16_t* xh, const uint32_t* code, const int* rows, const int* gexp,
                      const int* nact, int M, int TK, int TN, int S, float* part, hipStream_t s) {
  static std::once_flag once;
  static hipError_t err = hipSuccess;
  std::call_once(once, [] {
    err = hipFuncSetAttribute((const void*)esc::k_gemv_rows_table<K, kMoeGroupRows>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, 65536 * 2);
  });
  if (int rc = hip_check(err, "hipFuncSetAttribute")) return rc;
  hipLaunchKernelGGL((esc::k_gemv_rows_table<K, kMoeGroupRows>), dim3(device_cus()), dim3(1024),
                     65536 * 2, s, xh, code, rows, gexp, nact, M, TK, TN, TK / S, S, part);
  return launched("k_gemv_rows_table");
}

int group_rows(int K, int lut, int R, const uint16_t* xh, const uint32_t* code, const int* rows,
               const int* gexp, const int* nact, int n_groups, int M, int TK, int TN, int S,
               float* part, hipStream_t s) {
  if (lut) {
    if (R != kMoeGroupRows) return fail(ESC_EINVAL, "rows per expert group %d", R);
    return K == 2 ? launch_rows_table<2>(xh, code, rows, gexp, nact, M, TK, TN, S, part, s)
                  : launch_rows_table<3>(xh, code, rows, gexp, nact, M, TK, TN, S, part, s);
  }
  return K == 2 ? GroupRowsF<2, false>::run(R, xh, code, rows, gexp, n_groups, M, TK, TN, S, part, s)
                : GroupRowsF<3, false>::run(R, xh, code, rows, gexp, n_groups, M, TK, TN, S, part, s);
}

// One-launch path (fused.hpp).  Latency mode: small items over the whole GPU
// for one token-layer; throughput mode: large items for many token-layers.
constexpr int kFusedMaxRows = 64;

struct FusedPlan {
  int L, M, NB, NKC, NKB, NCP, nA, nB, grid;
  size_t off_pa, off_pb, off_xh2, off_int, total;
  int n_int;
};

// H/(16*KTA) <= 62: one polling wave reads the counter and every claim flag
// at once; top_k <= 32: the combine stages one row of d16 per slot in LDS.
bool fused_eligible(int T, int top_k, int H, int I) {
  return T * top_k <= kFusedMaxRows && top_k <= 32 && H % 256 == 0 && H / 128 <= 62 &&
         I % 128 == 0;
}

// kt per item of the many-layer two-launch path (gate_up, down)
// (measured on MI355X: 32 kt per item for either kernel is no faster)
constexpr int kKtaLayers = 16, kKtbLayers = 16;
// kt per item of one token-layer (latency-bound); with I == 512 the down
// items are 128-column blocks over all 32 kt (k_moe_down_blocks)
constexpr int kKtaSingle = 16, kKtbSingle = 16;
constexpr int kKtbBlocks = 32;
// kt per gate_up / down item of the single persistent launch: small items
// where it is esc_moe_expert_path's own choice (H or I not a multiple of 512);
// at the shapes that call runs as two launches (H and I multiples of 512),
// esc_moe_expert_path_one_launch takes larger ones (config 3: 22.3 us per
// token-layer against 32.9 us with the small items, 22.7-22.9 us with 16 and
// 8 kt, 24.5-28.0 us with 32 kt gate_up items)
constexpr int kKtaOne = 8, kKtbOne = 4;
constexpr int kKtaOneLarge = 16, kKtbOneLarge = 16;
// waves per gate_up / block down item of one token-layer, and per block
// down item of many token-layers
constexpr int kGateUpWavesSingle = 16, kDownBlockWavesSingle = 16;
constexpr int kDownBlockWavesLayers = 4;

// int_region > 0: the integer counters sit at offset 0 in a region of that
// many bytes and the float data after it, so calls of different shapes on one
// workspace never find another call's floats where their counters are (the
// no-allocation variant; the caller checks n_int * 4 <= int_region).
bool throughput_ok(int H, int I);

FusedPlan fused_plan(int L, int T, int top_k, int H, int I, bool throughput,
                     size_t int_region = 0) {
  // the two-launch path (throughput) uses the large items; the one-launch
  // path the small ones (KTA = 8, KTB = 4), which spread one token-layer wide,
  // or at two-launch shapes the middle ones (KTA = KTB = 16)
  const bool large = throughput;
  const bool layers = large && L > 1;
  const bool one_large = !large && throughput_ok(H, I);
  const int kta = layers ? kKtaLayers : large ? kKtaSingle : one_large ? kKtaOneLarge : kKtaOne;
  const bool blocks = large && I == 16 * kKtbBlocks;
  const int ktb = blocks ? kKtbBlocks
                  : layers ? kKtbLayers
                  : large  ? kKtbSingle
                  : one_large ? kKtbOneLarge : kKtbOne;
  FusedPlan f;
  f.L = L;
  f.M = T * top_k;
  f.NB = I / 128;
  f.NKC = std::max(1, H / (16 * kta));
  f.NKB = std::max(1, I / (16 * ktb));
  // 128-column blocks for the block kernels, 256-column pairs for every
  // other down item (k_moe_down_items, k_moe_fused): keyed on the kernel the
  // plan is for, not on the item's kt count
  f.NCP = blocks ? H / 128 : H / 256;
  f.nA = f.M * f.NB * f.NKC;
  f.nB = f.M * f.NCP * f.NKB;
  f.grid = throughput ? std::min(L * std::max(f.nA, f.nB), 1024)
                      : std::min(std::max(f.nA, f.nB), 2048);
  auto al = [](size_t v) { return (v + 255) & ~size_t(255); };
  f.n_int = L * (f.M * f.NB + f.nA + T * f.NCP) + 3;
  f.off_pa = al(int_region);
  f.off_pb = f.off_pa + al((size_t)L * f.nA * 256 * 4);
  f.off_xh2 = f.off_pb + al((size_t)L * f.nB * 256 * 4);
  const size_t end = f.off_xh2 + al((size_t)L * f.M * I * 2);
  f.off_int = int_region ? 0 : end;
  f.total = int_region ? end : end + al((size_t)f.n_int * 4);
  return f;
}

// Throughput mode needs the item sizes to divide the shapes.
bool throughput_ok(int H, int I) { return H % 512 == 0 && I % 512 == 0; }

esc::FusedMoe fused_args(const FusedPlan& f, void* ws, int T, int top_k, int H, int I) {
  char* w = static_cast<char*>(ws);
  int* ints = reinterpret_cast<int*>(w + f.off_int);
  esc::FusedMoe p{};
  p.partA = reinterpret_cast<float*>(w + f.off_pa);
  p.partB = reinterpret_cast<float*>(w + f.off_pb);
  p.xh2 = reinterpret_cast<uint16_t*>(w + f.off_xh2);
  p.cntA = ints;
  p.claimA = p.cntA + (size_t)f.L * f.M * f.NB;
  p.cntB = p.claimA + (size_t)f.L * f.nA;
  p.done = p.cntB + (size_t)f.L * T * f.NCP;
  p.err = p.done + 1;
  p.status = p.done + 2;
  p.host_err = nullptr;
  p.spin_limit = g_spin_limit.load(std::memory_order_relaxed);
  p.L = f.L;
  p.T = T;
  p.top_k = top_k;
  p.H = H;
  p.I = I;
  p.NB = f.NB;
  p.NKC = f.NKC;
  p.NKB = f.NKB;
  p.NCP = f.NCP;
  p.nA = f.nA;
  p.nB = f.nB;
  return p;
}

template <int KG, int KD, bool TP>
int launch_fused_k(const esc::FusedMoe& p, int grid, hipStream_t s) {
  if constexpr (TP) {
    // two launches: every gate_up item, then every down item (grid unused);
    // the down inputs are precomputed once per (row, h-block) for
    // multi-layer calls
    (void)grid;
    const dim3 ga(p.L * p.nA), gb(p.L * p.nB), blk(esc::kFusedThreads);
    // the plan's down item size: whole-input blocks (I == 512) or split-K
    const int ktb = p.I / (16 * p.NKB);
    // records in a device table (esc_moe_expert_path_layers, any L): the
    // many-layer items; one record in the arguments: the single-layer ones
    if (p.layers) {
      hipLaunchKernelGGL((esc::k_moe_gate_up_items<KG, kKtaLayers, true>), ga, blk, 0, s, p);
      if (int rc = launched("k_moe_gate_up_items")) return rc;
      if (ktb == kKtbBlocks) {
        hipLaunchKernelGGL((esc::k_moe_down_blocks<KG, KD, true, kDownBlockWavesLayers>), gb,
                           dim3(64 * kDownBlockWavesLayers), 0, s, p);
        return launched("k_moe_down_blocks");
      }
      hipLaunchKernelGGL((esc::k_moe_down_items<KG, KD, kKtbLayers, true>), gb, blk, 0, s, p);
      return launched("k_moe_down_items");
    }
    hipLaunchKernelGGL((esc::k_moe_gate_up_items<KG, kKtaSingle, false, kGateUpWavesSingle>), ga,
                       dim3(64 * kGateUpWavesSingle), 0, s, p);
    if (int rc = launched("k_moe_gate_up_items")) return rc;
    if (ktb == kKtbBlocks) {
      hipLaunchKernelGGL((esc::k_moe_down_blocks<KG, KD, false, kDownBlockWavesSingle>), gb,
                         dim3(64 * kDownBlockWavesSingle), 0, s, p);
      return launched("k_moe_down_blocks");
    }
    hipLaunchKernelGGL((esc::k_moe_down_items<KG, KD, kKtbSingle, false>), gb, blk, 0, s, p);
    return launched("k_moe_down_items");
  } else {
    // k_moe_fused's down items are 256-column pairs (16 tiles each)
    ESC_REQUIRE(p.NCP * 256 == p.H, "one-launch plan with %d column groups for H=%d", p.NCP, p.H);
    // the plan's item size (fused_plan: large items at two-launch shapes)
    if (p.H == 16 * kKtaOneLarge * p.NKC)
      hipLaunchKernelGGL((esc::k_moe_fused<KG, KD, kKtaOneLarge, kKtbOneLarge, true>), dim3(grid),
                         dim3(esc::kFusedThreads), 0, s, p);
    else
      hipLaunchKernelGGL((esc::k_moe_fused<KG, KD, kKtaOne, kKtbOne, true>), dim3(grid),
                         dim3(esc::kFusedThreads), 0, s, p);
    return launched("k_moe_fused");
  }
}

template <bool TP>
int launch_fused(const esc::FusedMoe& p, int K_gu, int K_dn, int grid, hipStream_t s) {
  if (K_gu == 2)
    return K_dn == 2 ? launch_fused_k<2, 2, TP>(p, grid, s) : launch_fused_k<2, 3, TP>(p, grid, s);
  return K_dn == 2 ? launch_fused_k<3, 2, TP>(p, grid, s) : launch_fused_k<3, 3, TP>(p, grid, s);
}

// ---- many-layer calls: the table-assisted kernels (K=2 gate_up and down,
// layers.hpp) or the item kernels above (any other K).  One workspace serves
// both: the item kernels' counters at offset 0, the table-assisted kernels'
// group counters after them, and each path's float data after both counter
// regions, so calls of either path on one workspace never find the other's
// floats where their counters are.
struct LayersWs {
  FusedPlan f;  // the item kernels' plan
  size_t off_cnt_gu, off_cnt_dn, off_cnt_cb, off_part, off_xh2, off_rows, total;
};

LayersWs layers_ws(int L, int T, int top_k, int H, int I) {
  auto al = [](size_t v) { return (v + 255) & ~size_t(255); };
  LayersWs w;
  const size_t M = (size_t)T * top_k, NB = I / 128, NKC = H / 128, NCP = H / 256;
  w.off_cnt_gu = al((size_t)fused_plan(L, T, top_k, H, I, true).n_int * 4);
  w.off_cnt_dn = w.off_cnt_gu + al(L * M * NB * 4);
  w.off_cnt_cb = w.off_cnt_dn + al(L * M * NCP * 4);
  const size_t ireg = w.off_cnt_cb + al((size_t)L * T * NCP * 4);
  w.f = fused_plan(L, T, top_k, H, I, true, ireg);
  // partials: at most one slot per item of a group (one item per wave)
  w.off_part = ireg;
  const size_t part = std::max(L * M * NB * NKC, L * M * NCP * esc::kDownEighths) * 1024;
  w.off_xh2 = w.off_part + al(part);
  w.off_rows = w.off_xh2 + al(L * M * I * 2);
  w.total = std::max(w.f.total, w.off_rows + al(L * M * H * 2));
  return w;
}

bool layers_table_ok(int K_gu, int K_dn, int I) {
  return K_gu == 2 && K_dn == 2 && I <= esc::kLayersMaxI;
}

int launch_layers_table(const esc::MoeLayer* layers, const LayersWs& w, void* ws, int L, int T,
                        int top_k, int H, int I, hipStream_t s) {
  if (int rc = ensure_lut()) return rc;
  static std::once_flag attr_once;
  static hipError_t attr_err = hipSuccess;
  std::call_once(attr_once, [] {
    const void* kerns[] = {(const void*)esc::k_moe_layers_gu, (const void*)esc::k_moe_layers_dn<1>,
                           (const void*)esc::k_moe_layers_dn<2>};
    for (const void* k : kerns) {
      const hipError_t e =
          hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, 65536 * 2);
      if (e != hipSuccess) attr_err = e;
    }
  });
  if (int rc = hip_check(attr_err, "hipFuncSetAttribute")) return rc;
  esc::LayersMoe p{};
  p.layers = layers;
  p.ws = static_cast<char*>(ws);
  p.off_part = w.off_part;
  p.off_xh2 = w.off_xh2;
  p.off_rows = w.off_rows;
  p.off_cnt_cb = w.off_cnt_cb;
  p.L = L;
  p.T = T;
  p.top_k = top_k;
  p.H = H;
  p.I = I;
  p.M = T * top_k;
  p.NB = I / 128;
  p.NKC = H / 128;
  p.NHB = H / 128;
  const int cus = device_cus();
  const long na = (long)L * p.M * p.NB * p.NKC, nd = (long)L * p.M * (p.NHB / 2) * esc::kDownEighths;
  ESC_REQUIRE(na < (1L << 30) && nd < (1L << 30), "too many items (%ld, %ld)", na, nd);
  // one workgroup per CU, more when a wave would otherwise run more than
  // kLayersMaxRange items (its items' pointers are staged in LDS); each
  // wave runs P consecutive items, so a group of `size` items spans at most
  // (size + P - 2) / P + 1 waves
  auto plan = [&](long n, int size, int& grid) {
    const long wg = esc::kLayersWaves;
    grid = (int)std::max(std::min<long>(cus, (n + wg - 1) / wg),
                         (n + wg * esc::kLayersMaxRange - 1) / (wg * esc::kLayersMaxRange));
    p.P = (int)((n + wg * grid - 1) / (wg * grid));
    p.maxc = std::min(size, (size + p.P - 2) / p.P + 1);
  };
  const dim3 blk(64 * esc::kLayersWaves);
  const size_t lds = 65536 * 2;
  int grid = 0;
  plan(na, p.NKC, grid);
  p.off_cnt = w.off_cnt_gu;
  hipLaunchKernelGGL(esc::k_moe_layers_gu, dim3(grid), blk, lds, s, p);
  if (int rc = launched("k_moe_layers_gu")) return rc;
  plan(nd, esc::kDownEighths, grid);
  p.off_cnt = w.off_cnt_dn;
  // the down items' inputs: I/16 words, one or two registers per lane
  if (I <= 1024)
    hipLaunchKernelGGL(esc::k_moe_layers_dn<1>, dim3(grid), blk, lds, s, p);
  else
    hipLaunchKernelGGL(esc::k_moe_layers_dn<2>, dim3(grid), blk, lds, s, p);
  return launched("k_moe_layers_dn");
}
}  // namespace

extern "C" {
size_t esc_moe_expert_path_workspace(int T, int top_k, int E, int H, int I) {
  if (T <= 0 || top_k <= 0 || H <= 0 || I <= 0) return 0;
  // the plan's sizes depend on K only through the split counts; take the max
  size_t a = moe_plan(T, top_k, E, H, I, 2, 2).total, b = moe_plan(T, top_k, E, H, I, 3, 3).total;
  size_t c = moe_plan(T, top_k, E, H, I, 2, 3).total, d = moe_plan(T, top_k, E, H, I, 3, 2).total;
  size_t m = std::max(std::max(a, b), std::max(c, d));
  if (fused_eligible(T, top_k, H, I)) {
    m = std::max(m, fused_plan(1, T, top_k, H, I, false).total);
    if (throughput_ok(H, I)) m = std::max(m, fused_plan(1, T, top_k, H, I, true).total);
  }
  return m;
}

int esc_moe_status(const void* ws, size_t ws_bytes, int T, int top_k, int H, int I,
                   int32_t* host_flag, void* stream) {
  ESC_REQUIRE(ws && host_flag, "null pointer");
  *host_flag = 0;
  // only the single persistent launch has a bounded wait
  if (!fused_eligible(T, top_k, H, I)) return ESC_OK;
  if (throughput_ok(H, I)) {
    // esc_moe_expert_path runs two launches at this shape; a call through
    // esc_moe_expert_path_one_launch reports a give-up through the
    // device-wide flag (its workspace slot is not read: the same workspace
    // may have served the two-launch plan, whose layout differs)
    int* unused = nullptr;
    if (take_wait_error(&unused) == ESC_ETIMEOUT) *host_flag = 1;
    return ESC_OK;
  }
  const FusedPlan f = fused_plan(1, T, top_k, H, I, false);
  ESC_REQUIRE(ws_bytes >= f.total, "workspace smaller than the plan");
  // the status slot (the last integer): read, then cleared for the next read
  int32_t* st = reinterpret_cast<int32_t*>(static_cast<char*>(const_cast<void*>(ws)) + f.off_int) +
                (f.n_int - 1);
  if (int rc = hip_check(hipMemcpyAsync(host_flag, st, 4, hipMemcpyDeviceToHost, S(stream)),
                         "hipMemcpyAsync"))
    return rc;
  if (int rc = hip_check(hipMemsetAsync(st, 0, 4, S(stream)), "hipMemsetAsync")) return rc;
  if (int rc = hip_check(hipStreamSynchronize(S(stream)), "hipStreamSynchronize")) return rc;
  // the device-wide flag records the same event: taken here too, so a later
  // call does not report it again
  int* unused = nullptr;
  if (take_wait_error(&unused) == ESC_ETIMEOUT) *host_flag = 1;
  return ESC_OK;
}

int esc_moe_set_spin_limit(int polls) {
  g_spin_limit.store(polls < 0 ? esc::kSpinLimit : polls, std::memory_order_relaxed);
  return ESC_OK;
}

}  // extern "C"

namespace {
// The expert path on a given workspace; int_region > 0 puts every counter in
// a fixed region at its start (see fused_plan).
int moe_expert_path(const uint16_t* x, const int32_t* ids, const float* scores, int T, int top_k,
                    int E, int H, int I, const uint32_t* gu_code, const float* gu_rin,
                    const float* gu_rout, int K_gu, const uint32_t* dn_code, const float* dn_rin,
                    const float* dn_rout, int K_dn, int use_lut, uint16_t* y, void* ws,
                    size_t ws_bytes, size_t int_region, void* stream, bool one_launch = false) {
  ESC_REQUIRE(x && ids && scores && gu_code && gu_rin && gu_rout && dn_code && dn_rin && dn_rout &&
                  y,
              "null pointer");
  ESC_REQUIRE(E > 0 && top_k >= 1 && top_k <= E, "bad E=%d / top_k=%d", E, top_k);
  if (int rc = check_proj(K_gu, H, 2 * I)) return rc;
  if (int rc = check_proj(K_dn, I, H)) return rc;
  ESC_REQUIRE(T >= 0, "negative token count");
  if (T == 0) return ESC_OK;
  if (fused_eligible(T, top_k, H, I)) {
    // throughput_ok: two launches (gate_up items, down items + combine),
    // measured faster than the single persistent launch for one token-layer
    // on gfx950; otherwise (or when the caller asks for it) the single
    // persistent launch
    const bool two = throughput_ok(H, I) && !one_launch;
    const FusedPlan f = fused_plan(1, T, top_k, H, I, two, int_region);
    // a fixed counter region keeps its last word for the status flag
    if (int_region && (size_t)f.n_int * 4 > int_region - 4)
      return fail(ESC_ENOSPACE, "%d counters exceed the %zu-byte counter region", f.n_int,
                  int_region - 4);
    if (!ws || ws_bytes < f.total)
      return fail(ESC_ENOSPACE, "workspace %zu bytes < required %zu", ws_bytes, f.total);
    esc::FusedMoe p = fused_args(f, ws, T, top_k, H, I);
    // Nothing clears the status flag of a fixed counter region (no caller
    // workspace is read by esc_moe_status): it lives in the region's last
    // word, outside every shape's counters, so a give-up of one call never
    // lands in the counters of a later call of another shape.
    if (int_region) p.status = reinterpret_cast<int*>(static_cast<char*>(ws) + int_region) - 1;
    p.l0 = esc::MoeLayer{x, ids, scores, gu_code, gu_rin, gu_rout, dn_code, dn_rin, dn_rout, y};
    p.layers = nullptr;
    if (two) return launch_fused<true>(p, K_gu, K_dn, f.grid, S(stream));
    // only the single persistent launch waits across workgroups
    if (int rc = take_wait_error(&p.host_err)) return rc;
    return launch_fused<false>(p, K_gu, K_dn, f.grid, S(stream));
  }
  const MoePlan p = moe_plan(T, top_k, E, H, I, K_gu, K_dn, int_region);
  if (!ws || ws_bytes < p.total)
    return fail(ESC_ENOSPACE, "workspace %zu bytes < required %zu", ws_bytes, p.total);
  if (use_lut)
    if (int rc = ensure_lut()) return rc;
  char* w = static_cast<char*>(ws);
  uint16_t* xh = reinterpret_cast<uint16_t*>(w + p.off_xh);
  float* p1 = reinterpret_cast<float*>(w + p.off_p1);
  uint16_t* xh2 = reinterpret_cast<uint16_t*>(w + p.off_xh2);
  float* p2 = reinterpret_cast<float*>(w + p.off_p2);
  hipStream_t s = S(stream);
  const float rs = esc::kRS;
  int* rows = reinterpret_cast<int*>(w + p.off_rows);
  int* gexp = reinterpret_cast<int*>(w + p.off_gexp);
  int* nact = reinterpret_cast<int*>(w + p.off_nact);
  if (p.R) {
    // input transform and expert grouping in one launch
    const int waves = H / 128 * p.M;
    hipLaunchKernelGGL(esc::k_moe_prep, dim3(1 + (waves + 15) / 16), dim3(1024), 0, s, x, ids,
                       top_k, gu_rin, H, rs, xh, p.M, E, p.R, p.n_groups, rows, gexp, nact);
    if (int rc = launched("k_moe_prep")) return rc;
    if (int rc = group_rows(K_gu, use_lut, p.R, xh, gu_code, rows, gexp, nact, p.n_groups, p.M,
                            H / 16, 2 * I / 16, p.S1, p1, s))
      return rc;
  } else if (int rc = moe_input(x, ids, top_k, gu_rin, H, rs, xh, p.M, s)) {
    return rc;
  } else if (int rc = by_k_lut<FastF>(K_gu, use_lut, xh, gu_code, ids, p.M, H / 16, 2 * I / 16,
                                      p.S1, p1, s)) {
    return rc;
  }
  auto mid = [&](auto sc) {
    hipLaunchKernelGGL((esc::k_moe_mid<decltype(sc)::value>), dim3(I / 128, p.M), dim3(64), 0, s,
                       p1, p.S1, p.M, I, ids, gu_rout, dn_rin, rs, xh2);
  };
  switch (esc::splits_class(p.S1)) {
    case 1: mid(std::integral_constant<int, 1>{}); break;
    case 2: mid(std::integral_constant<int, 2>{}); break;
    case 4: mid(std::integral_constant<int, 4>{}); break;
    default: mid(std::integral_constant<int, 0>{});
  }
  if (int rc = launched("k_moe_mid")) return rc;
  if (p.R) {
    if (int rc = group_rows(K_dn, use_lut, p.R, xh2, dn_code, rows, gexp, nact, p.n_groups, p.M,
                            I / 16, H / 16, p.S2, p2, s))
      return rc;
  } else if (int rc = by_k_lut<FastF>(K_dn, use_lut, xh2, dn_code, ids, p.M, I / 16, H / 16, p.S2,
                                      p2, s)) {
    return rc;
  }
  auto combine = [&](auto sc) {
    hipLaunchKernelGGL((esc::k_moe_combine<decltype(sc)::value>), dim3(H / 128, T), dim3(64), 0, s,
                       p2, p.S2, p.M, H, ids, scores, top_k, dn_rout, rs, y);
  };
  switch (esc::splits_class(p.S2)) {
    case 1: combine(std::integral_constant<int, 1>{}); break;
    case 2: combine(std::integral_constant<int, 2>{}); break;
    case 4: combine(std::integral_constant<int, 4>{}); break;
    default: combine(std::integral_constant<int, 0>{});
  }
  return launched("k_moe_combine");
}

// ---- the expert path without allocation: a file-scope device scratch array
// Its counters sit in the first kStaticIntBytes (zeroed once per device at
// set-up, left zero by every call), the float data after them.
constexpr size_t kStaticScratchBytes = size_t(4) << 20;
constexpr size_t kStaticIntBytes = size_t(128) << 10;
}  // namespace

__device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace {
// Device address of `scratch` per device (the symbol's host-side name is not
// a device address): looked up once per device, with that device current,
// and its counter region zeroed by a fill kernel.
void* g_scratch_ptr[kMaxDevices];

__global__ void k_zero_words(uint32_t* p, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

int ensure_scratch(void** out) {
  int dev = 0;
  if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
  if (dev < 0 || dev >= kMaxDevices) return fail(ESC_EINVAL, "device index %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_init_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    if (int rc = hip_check(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress"))
      return rc;
    if (!ptr) return fail(ESC_EHIP, "hipGetSymbolAddress returned a null scratch address");
    hipLaunchKernelGGL(k_zero_words, dim3(64), dim3(256), 0, 0, static_cast<uint32_t*>(ptr),
                       kStaticIntBytes / 4);
    if (int rc = launched("k_zero_words")) return rc;
    if (int rc = hip_check(hipDeviceSynchronize(), "scratch set-up sync")) return rc;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return ESC_OK;
}

bool scratch_ready() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
  std::lock_guard<std::mutex> lk(g_init_mu);
  return g_scratch_ptr[dev] != nullptr;
}
}  // namespace

extern "C" {
int esc_moe_expert_path(const uint16_t* x, const int32_t* ids, const float* scores, int T,
                        int top_k, int E, int H, int I, const uint32_t* gu_code,
                        const float* gu_rin, const float* gu_rout, int K_gu,
                        const uint32_t* dn_code, const float* dn_rin, const float* dn_rout,
                        int K_dn, int use_lut, uint16_t* y, void* ws, size_t ws_bytes,
                        void* stream) {
  if (int rc = ensure_wait_flag()) return rc;
  return moe_expert_path(x, ids, scores, T, top_k, E, H, I, gu_code, gu_rin, gu_rout, K_gu,
                         dn_code, dn_rin, dn_rout, K_dn, use_lut, y, ws, ws_bytes, 0, stream);
}

int esc_moe_expert_path_one_launch(const uint16_t* x, const int32_t* ids, const float* scores,
                                   int T, int top_k, int E, int H, int I,
                                   const uint32_t* gu_code, const float* gu_rin,
                                   const float* gu_rout, int K_gu, const uint32_t* dn_code,
                                   const float* dn_rin, const float* dn_rout, int K_dn,
                                   int use_lut, uint16_t* y, void* ws, size_t ws_bytes,
                                   void* stream) {
  ESC_REQUIRE(T >= 0 && top_k >= 1 && H > 0 && I > 0, "bad sizes T=%d top_k=%d H=%d I=%d", T,
              top_k, H, I);
  ESC_REQUIRE(fused_eligible(T, top_k, H, I),
              "one-launch expert path needs T*top_k <= %d, top_k <= 32, H a multiple of 256 "
              "up to 7936 and I a multiple of 128 (got T=%d top_k=%d H=%d I=%d)",
              kFusedMaxRows, T, top_k, H, I);
  if (int rc = ensure_wait_flag()) return rc;
  return moe_expert_path(x, ids, scores, T, top_k, E, H, I, gu_code, gu_rin, gu_rout, K_gu,
                         dn_code, dn_rin, dn_rout, K_dn, use_lut, y, ws, ws_bytes, 0, stream,
                         true);
}

size_t esc_moe_expert_path_static_max(void) { return kStaticScratchBytes; }

int esc_moe_expert_path_static(const uint16_t* x, const int32_t* ids, const float* scores, int T,
                               int top_k, int E, int H, int I, const uint32_t* gu_code,
                               const float* gu_rin, const float* gu_rout, int K_gu,
                               const uint32_t* dn_code, const float* dn_rin,
                               const float* dn_rout, int K_dn, int use_lut, uint16_t* y,
                               void* stream) {
  ESC_REQUIRE(T >= 0 && top_k >= 1 && H > 0 && I > 0, "bad sizes T=%d top_k=%d H=%d I=%d", T,
              top_k, H, I);
  if (T == 0) return ESC_OK;
  // the table, when asked for, is built by esc_init (a kernel, no allocation)
  ESC_REQUIRE(!use_lut || lut_ready(), "use_lut needs esc_init() on this device first");
  // the scratch set-up launches a fill kernel and synchronises, which a
  // stream under graph capture cannot do: such callers run esc_init first
  if (!scratch_ready()) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (int rc = hip_check(hipStreamIsCapturing(S(stream), &cs), "hipStreamIsCapturing"))
      return rc;
    ESC_REQUIRE(cs == hipStreamCaptureStatusNone,
                "the static scratch is not set up on this device: call esc_init() before "
                "capturing esc_moe_expert_path_static");
  }
  void* ptr = nullptr;
  if (int rc = ensure_scratch(&ptr)) return rc;
  return moe_expert_path(x, ids, scores, T, top_k, E, H, I, gu_code, gu_rin, gu_rout, K_gu,
                         dn_code, dn_rin, dn_rout, K_dn, use_lut, y, ptr, kStaticScratchBytes,
                         kStaticIntBytes, stream);
}

size_t esc_moe_layers_workspace(int L, int T, int top_k, int H, int I) {
  if (L <= 0 || T <= 0 || top_k <= 0 || !fused_eligible(T, top_k, H, I) || !throughput_ok(H, I))
    return 0;
  return layers_ws(L, T, top_k, H, I).total;
}

int esc_moe_expert_path_layers(const esc_moe_layer* layers, int L, int T, int top_k, int E, int H,
                               int I, int K_gu, int K_dn, void* ws, size_t ws_bytes,
                               void* stream) {
  static_assert(sizeof(esc_moe_layer) == sizeof(esc::MoeLayer), "layer record layout");
  ESC_REQUIRE(layers, "null pointer");
  ESC_REQUIRE(L >= 0 && T >= 0, "negative size");
  ESC_REQUIRE(E > 0 && top_k >= 1 && top_k <= E, "bad E=%d / top_k=%d", E, top_k);
  if (int rc = check_proj(K_gu, H, 2 * I)) return rc;
  if (int rc = check_proj(K_dn, I, H)) return rc;
  ESC_REQUIRE(fused_eligible(T, top_k, H, I) && throughput_ok(H, I),
              "multi-layer expert path needs T*top_k <= %d, top_k <= 32, H and I multiples of "
              "512, H <= 7936 (got T=%d top_k=%d H=%d I=%d)",
              kFusedMaxRows, T, top_k, H, I);
  if (L == 0 || T == 0) return ESC_OK;
  const LayersWs w = layers_ws(L, T, top_k, H, I);
  if (!ws || ws_bytes < w.total)
    return fail(ESC_ENOSPACE, "workspace %zu bytes < required %zu", ws_bytes, w.total);
  const auto* lr = reinterpret_cast<const esc::MoeLayer*>(layers);
  if (layers_table_ok(K_gu, K_dn, I))
    return launch_layers_table(lr, w, ws, L, T, top_k, H, I, S(stream));
  esc::FusedMoe p = fused_args(w.f, ws, T, top_k, H, I);
  p.layers = lr;
  return launch_fused<true>(p, K_gu, K_dn, w.f.grid, S(stream));
}


// ---- decode-rate probe (measurement only)
size_t esc_decode_probe_words(int steps, int waves_per_cu) {
  if (steps <= 0 || steps % 4 || (waves_per_cu != 16 && waves_per_cu != 32)) return 0;
  return (size_t)device_cus() * waves_per_cu * steps * 64 * 4;
}

int esc_decode_probe(const uint32_t* code, int steps, int nt, int waves_per_cu, int prefetch,
                     float* out, void* stream) {
  ESC_REQUIRE(code && out, "null pointer");
  ESC_REQUIRE(steps > 0 && steps % 4 == 0, "steps must be a positive multiple of 4");
  ESC_REQUIRE(waves_per_cu == 16 || waves_per_cu == 32, "waves per CU must be 16 or 32");
  ESC_REQUIRE(nt == 0 || waves_per_cu == 16, "the table (nt > 0) fits one workgroup per CU");
  ESC_REQUIRE(prefetch >= 1 && prefetch <= 3, "prefetch depth must be 1, 2 or 3");
  if (nt > 0)
    if (int rc = ensure_lut()) return rc;
  const dim3 grid(device_cus() * (waves_per_cu / 16)), blk(1024);
  const size_t lds = nt > 0 ? 131072 : 0;
  auto go = [&](auto kern) -> int {
    if (lds)
      if (int rc = hip_check(hipFuncSetAttribute((const void*)kern,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)lds),
                             "hipFuncSetAttribute"))
        return rc;
    hipLaunchKernelGGL(kern, grid, blk, lds, S(stream), code, steps, out);
    return launched("k_decode_probe");
  };
  auto by_pf = [&](auto k1, auto k2, auto k3) -> int {
    return prefetch == 1 ? go(k1) : prefetch == 2 ? go(k2) : go(k3);
  };
#define ESC_PROBE(NT) \
  by_pf(esc::k_decode_probe<NT, 1>, esc::k_decode_probe<NT, 2>, esc::k_decode_probe<NT, 3>)
  switch (nt) {
    case 0: return ESC_PROBE(0);
    case 2: return ESC_PROBE(2);
    case 3: return ESC_PROBE(3);
    case 4: return ESC_PROBE(4);
    case 5: return ESC_PROBE(5);
    case 6: return ESC_PROBE(6);
    case 8: return ESC_PROBE(8);
  }
#undef ESC_PROBE
  return fail(ESC_EINVAL, "table pairs per 8 must be one of 0, 2, 3, 4, 5, 6, 8 (got %d)", nt);
}

}  // extern "C"
