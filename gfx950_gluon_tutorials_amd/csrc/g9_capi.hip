// extern "C" entry points of the gfx950 GEMM library (declared in
// include/gfx950_gemm.h).  Each validates shapes, strides and alignment,
// fills a GemmParams and launches one named kernel on the caller's stream
// (split-K: the segment kernel, then its reduction, on that stream).
#include <atomic>
#include <cstring>
#include <mutex>

#include "../../include/gfx950_gemm.h"
#include "g9_gemm.hpp"

using namespace g9;

// ---------------------------------------------------------------------------
// Named kernels: one symbol per (operand type, output type, schedule, waves) so
// profilers can filter on a stable substring.
// ---------------------------------------------------------------------------
#define G9_ATTRS(G) \
  __launch_bounds__(G::kThreads) __attribute__((amdgpu_waves_per_eu(G::kWavesPerSimd, G::kWavesPerSimd)))

#define G9_DEFINE(NAME, OP, OUT)                                                                    \
  using NAME##_g4 = Geo4<kMfmaDim<OP>>;                                                             \
  using NAME##_g8 = Geo8<kMfmaDim8<OP>>;                                                            \
  extern "C" __global__ G9_ATTRS(NAME##_g4) void NAME##_dp_4w(GemmParams p) {                       \
    gemm_dp<OP, OUT, NAME##_g4>(p);                                                                 \
  }                                                                                                 \
  extern "C" __global__ G9_ATTRS(NAME##_g4) void NAME##_sk_4w(GemmParams p) {                       \
    gemm_sk<OP, OUT, NAME##_g4>(p);                                                                 \
  }                                                                                                 \
  extern "C" __global__ G9_ATTRS(NAME##_g8) void NAME##_dp_8w(GemmParams p) {                       \
    gemm_dp<OP, OUT, NAME##_g8>(p);                                                                 \
  }                                                                                                 \
  extern "C" __global__ G9_ATTRS(NAME##_g8) void NAME##_sk_8w(GemmParams p) { gemm_sk<OP, OUT, NAME##_g8>(p); }

G9_DEFINE(g9_a16w16_f16, Op::F16, OUT_F16)
G9_DEFINE(g9_a16w16_bf16, Op::BF16, OUT_BF16)
G9_DEFINE(g9_a8w8_f16out, Op::BF8, OUT_F16)
G9_DEFINE(g9_a8w8_bf16out, Op::BF8, OUT_BF16)
G9_DEFINE(g9_a4w4_bf16out, Op::FP4, OUT_BF16)
G9_DEFINE(g9_a4w4_f16out, Op::FP4, OUT_F16)

// Stream-K over 256x128 tiles (FP16/BF16, 4-wave).
using G9Half4 = Geo4<16>;
extern "C" __global__ G9_ATTRS(G9Half4) void g9_a16w16_f16_skh_4w(GemmParams p) {
  gemm_sk_h<Op::F16, OUT_F16, G9Half4>(p);
}
extern "C" __global__ G9_ATTRS(G9Half4) void g9_a16w16_bf16_skh_4w(GemmParams p) {
  gemm_sk_h<Op::BF16, OUT_BF16, G9Half4>(p);
}

// MXFP4 with preshuffled scales: data-parallel, 4-wave.
using G9Fp4p4 = Geo4<kMfmaDim<Op::FP4P>>;
extern "C" __global__ G9_ATTRS(G9Fp4p4) void g9_a4w4ps_bf16out_dp_4w(GemmParams p) {
  gemm_dp<Op::FP4P, OUT_BF16, G9Fp4p4>(p);
}
extern "C" __global__ G9_ATTRS(G9Fp4p4) void g9_a4w4ps_f16out_dp_4w(GemmParams p) {
  gemm_dp<Op::FP4P, OUT_F16, G9Fp4p4>(p);
}

// MXFP4 with K-major scales (the reference bench's transposed scale views):
// 4-wave, data-parallel, stream-K and split-K.
using G9Fp4k4 = Geo4<kMfmaDim<Op::FP4K>>;
extern "C" __global__ G9_ATTRS(G9Fp4k4) void g9_a4w4km_bf16out_dp_4w(GemmParams p) {
  gemm_dp<Op::FP4K, OUT_BF16, G9Fp4k4>(p);
}
extern "C" __global__ G9_ATTRS(G9Fp4k4) void g9_a4w4km_f16out_dp_4w(GemmParams p) {
  gemm_dp<Op::FP4K, OUT_F16, G9Fp4k4>(p);
}
extern "C" __global__ G9_ATTRS(G9Fp4k4) void g9_a4w4km_bf16out_sk_4w(GemmParams p) {
  gemm_sk<Op::FP4K, OUT_BF16, G9Fp4k4>(p);
}
extern "C" __global__ G9_ATTRS(G9Fp4k4) void g9_a4w4km_f16out_sk_4w(GemmParams p) {
  gemm_sk<Op::FP4K, OUT_F16, G9Fp4k4>(p);
}
extern "C" __global__ G9_ATTRS(G9Fp4k4) void g9_a4w4km_splitk_4w(GemmParams p) { gemm_splitk<Op::FP4K, G9Fp4k4>(p); }

// Grouped (MoE) kernels, 4-wave.
#define G9_DEFINE_MOE(NAME, OP, OUT)                                                                \
  extern "C" __global__ G9_ATTRS(NAME##_g4) void NAME##_moe_4w(GemmParams p) {                      \
    gemm_moe<OP, OUT, NAME##_g4>(p);                                                                \
  }

G9_DEFINE_MOE(g9_a16w16_f16, Op::F16, OUT_F16)
G9_DEFINE_MOE(g9_a16w16_bf16, Op::BF16, OUT_BF16)
G9_DEFINE_MOE(g9_a8w8_bf16out, Op::BF8, OUT_BF16)
G9_DEFINE_MOE(g9_a8w8_f16out, Op::BF8, OUT_F16)
G9_DEFINE_MOE(g9_a4w4_bf16out, Op::FP4, OUT_BF16)
G9_DEFINE_MOE(g9_a4w4_f16out, Op::FP4, OUT_F16)

// Split-K kernels: the segment kernel depends only on the operand type (its
// output is fp32 partials), the reduction only on the output type.
#define G9_DEFINE_SPLITK(NAME, OP)                                                                 \
  extern "C" __global__ G9_ATTRS(Geo4<kMfmaDim<OP>>) void NAME##_splitk_4w(GemmParams p) {       \
    gemm_splitk<OP, Geo4<kMfmaDim<OP>>>(p);                                                        \
  }                                                                                                \
  extern "C" __global__ G9_ATTRS(Geo8<kMfmaDim8<OP>>) void NAME##_splitk_8w(GemmParams p) {      \
    gemm_splitk<OP, Geo8<kMfmaDim8<OP>>>(p);                                                       \
  }

G9_DEFINE_SPLITK(g9_a16w16_f16, Op::F16)
G9_DEFINE_SPLITK(g9_a16w16_bf16, Op::BF16)
G9_DEFINE_SPLITK(g9_a8w8, Op::BF8)
G9_DEFINE_SPLITK(g9_a4w4, Op::FP4)

extern "C" __global__ __launch_bounds__(256) void g9_splitk_reduce_f16(GemmParams p) { splitk_reduce<OUT_F16>(p); }
extern "C" __global__ __launch_bounds__(256) void g9_splitk_reduce_bf16(GemmParams p) { splitk_reduce<OUT_BF16>(p); }

typedef void (*KernelFn)(GemmParams);

namespace {

struct KernelEntry {
  int dtype, out, sched, waves;
  KernelFn fn;
  const char* name;
};

#define G9_ENTRY(DT, OUT, NAME)                                                                   \
  {DT, OUT, G9_SCHED_DP, 4, NAME##_dp_4w, #NAME "_dp_4w"}, {DT, OUT, G9_SCHED_SK, 4, NAME##_sk_4w, #NAME "_sk_4w"}, \
      {DT, OUT, G9_SCHED_DP, 8, NAME##_dp_8w, #NAME "_dp_8w"},                                               \
  {                                                                                               \
    DT, OUT, G9_SCHED_SK, 8, NAME##_sk_8w, #NAME "_sk_8w"                                       \
  }

const KernelEntry kKernels[] = {
    G9_ENTRY(G9_F16, G9_F16, g9_a16w16_f16),     G9_ENTRY(G9_BF16, G9_BF16, g9_a16w16_bf16),
    G9_ENTRY(G9_BF8, G9_F16, g9_a8w8_f16out),    G9_ENTRY(G9_BF8, G9_BF16, g9_a8w8_bf16out),
    G9_ENTRY(G9_FP4, G9_BF16, g9_a4w4_bf16out),  G9_ENTRY(G9_FP4, G9_F16, g9_a4w4_f16out),
    {G9_FP4P, G9_BF16, G9_SCHED_DP, 4, g9_a4w4ps_bf16out_dp_4w, "g9_a4w4ps_bf16out_dp_4w"},
    {G9_FP4P, G9_F16, G9_SCHED_DP, 4, g9_a4w4ps_f16out_dp_4w, "g9_a4w4ps_f16out_dp_4w"},
    {G9_FP4K, G9_BF16, G9_SCHED_DP, 4, g9_a4w4km_bf16out_dp_4w, "g9_a4w4km_bf16out_dp_4w"},
    {G9_FP4K, G9_F16, G9_SCHED_DP, 4, g9_a4w4km_f16out_dp_4w, "g9_a4w4km_f16out_dp_4w"},
    {G9_FP4K, G9_BF16, G9_SCHED_SK, 4, g9_a4w4km_bf16out_sk_4w, "g9_a4w4km_bf16out_sk_4w"},
    {G9_FP4K, G9_F16, G9_SCHED_SK, 4, g9_a4w4km_f16out_sk_4w, "g9_a4w4km_f16out_sk_4w"},
    {G9_F16, G9_F16, G9_SCHED_SK_HALF, 4, g9_a16w16_f16_skh_4w, "g9_a16w16_f16_skh_4w"},
    {G9_BF16, G9_BF16, G9_SCHED_SK_HALF, 4, g9_a16w16_bf16_skh_4w, "g9_a16w16_bf16_skh_4w"},
};

#define G9_SPLITK_ENTRY(DT, OUT, NAME)                                                              \
  {DT, OUT, G9_SCHED_SPLITK, 4, NAME##_splitk_4w, #NAME "_splitk_4w"}, {                           \
    DT, OUT, G9_SCHED_SPLITK, 8, NAME##_splitk_8w, #NAME "_splitk_8w"                              \
  }

const KernelEntry kSplitKernels[] = {
    G9_SPLITK_ENTRY(G9_F16, G9_F16, g9_a16w16_f16),  G9_SPLITK_ENTRY(G9_BF16, G9_BF16, g9_a16w16_bf16),
    G9_SPLITK_ENTRY(G9_BF8, G9_F16, g9_a8w8),        G9_SPLITK_ENTRY(G9_BF8, G9_BF16, g9_a8w8),
    G9_SPLITK_ENTRY(G9_FP4, G9_BF16, g9_a4w4),       G9_SPLITK_ENTRY(G9_FP4, G9_F16, g9_a4w4),
    {G9_FP4K, G9_BF16, G9_SCHED_SPLITK, 4, g9_a4w4km_splitk_4w, "g9_a4w4km_splitk_4w"},
    {G9_FP4K, G9_F16, G9_SCHED_SPLITK, 4, g9_a4w4km_splitk_4w, "g9_a4w4km_splitk_4w"},
};

const KernelEntry kMoeKernels[] = {
    {G9_F16, G9_F16, G9_SCHED_DP, 4, g9_a16w16_f16_moe_4w, "g9_a16w16_f16_moe_4w"},
    {G9_BF16, G9_BF16, G9_SCHED_DP, 4, g9_a16w16_bf16_moe_4w, "g9_a16w16_bf16_moe_4w"},
    {G9_BF8, G9_BF16, G9_SCHED_DP, 4, g9_a8w8_bf16out_moe_4w, "g9_a8w8_bf16out_moe_4w"},
    {G9_BF8, G9_F16, G9_SCHED_DP, 4, g9_a8w8_f16out_moe_4w, "g9_a8w8_f16out_moe_4w"},
    {G9_FP4, G9_BF16, G9_SCHED_DP, 4, g9_a4w4_bf16out_moe_4w, "g9_a4w4_bf16out_moe_4w"},
    {G9_FP4, G9_F16, G9_SCHED_DP, 4, g9_a4w4_f16out_moe_4w, "g9_a4w4_f16out_moe_4w"},
};

const KernelEntry* find_moe_kernel(int dtype, int out) {
  for (const KernelEntry& k : kMoeKernels)
    if (k.dtype == dtype && k.out == out) return &k;
  return nullptr;
}

const KernelEntry* find_kernel(int dtype, int out, int sched, int waves) {
  for (const KernelEntry& k : kKernels)
    if (k.dtype == dtype && k.out == out && k.sched == sched && k.waves == waves) return &k;
  for (const KernelEntry& k : kSplitKernels)
    if (k.dtype == dtype && k.out == out && k.sched == sched && k.waves == waves) return &k;
  return nullptr;
}

// K values per 128-byte stage row.
int stage_k(int dtype) {
  switch (dtype) {
    case G9_F16:
    case G9_BF16:
      return 64;
    case G9_BF8:
      return 128;
    case G9_FP4:
    case G9_FP4P:
    case G9_FP4K:
      return 256;
  }
  return 0;
}

constexpr int kNumXcds = 8;
constexpr int kGroupM = 4;
constexpr size_t kWsHeader = 256;          // error word + padding
constexpr size_t kWsTileBytes = 256 * 256 * 4;
// Workspaces are accounted in units of a 256x128 tile's fp32 partial: a
// 256x256 partial is two, and the flag region holds one flag per unit.
constexpr size_t kWsUnit = kWsTileBytes / 2;

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

size_t flags_bytes(long long tiles) { return align256((size_t)tiles * 4); }

std::atomic<unsigned> g_epoch{0};

// Polls of a stream-K flag wait before it gives up and sets the workspace
// error word (g9_set_streamk_spin_limit changes it, for tests of that path).
constexpr uint32_t kDefaultSpinLimit = 1u << 26;
std::atomic<uint32_t> g_spin_limit{kDefaultSpinLimit};

// CUs of the current device (cached per device; 0 if it cannot be queried).
int cu_count() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cache[kMaxDevices];
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < kMaxDevices && (n = cache[dev].load(std::memory_order_relaxed)) > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 0;
  if (dev < kMaxDevices) cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// Workspace layout (both schedules): the header, then a flag region as large
// as the one g9_workspace_init clears for a workspace of this size (the flags
// of any stream-K launch that fits it), then the partials.  Split-K never
// writes the header or the flags, so one workspace serves both schedules.
size_t splitk_base(size_t ws_bytes) {
  return kWsHeader + flags_bytes((long long)((ws_bytes - kWsHeader) / kWsUnit + 1));
}
// Smallest workspace whose partials (behind its own flag region) hold
// `units` partial units.  Stream-K needs one partial (and one flag) per tile.
size_t units_bytes(long long units) {
  size_t s = kWsHeader + flags_bytes(units + 1) + (size_t)units * kWsUnit;
  while (splitk_base(s) + (size_t)units * kWsUnit > s) s += 256;
  return s;
}
size_t splitk_bytes(long long partials) { return units_bytes(2 * partials); }
size_t streamk_bytes(long long tiles) { return units_bytes(2 * tiles); }
size_t streamk_half_bytes(long long tiles) { return units_bytes(tiles); }

// A resolved launch: the kernel (and split-K's reduction), the grid and the
// parameter block, i.e. everything an entry point works out before it
// enqueues.  g9_plan_* keep it in the caller's g9_plan; run_plan only
// enqueues it (a stream-K plan takes a new flag epoch and the current spin
// limit at each launch).
constexpr uint32_t kPlanMagic = 0x6c703967u;
struct Plan {
  uint32_t magic;
  int device;     // the device current when the plan was made
  int grid, block;
  int red_grid;   // split-K reduction grid (0: no reduction)
  int streamk;
  const void* fn;
  const void* red;
  GemmParams p;
};
static_assert(sizeof(Plan) <= G9_PLAN_BYTES && alignof(Plan) <= alignof(g9_plan), "g9_plan cannot hold a Plan");

// Shared launch path.  Sizes/strides were validated by the caller except the
// generic checks done here.
int make_plan(int dtype, int out, int schedule, int waves, GemmParams& p, void* ws, size_t ws_bytes, Plan& pl) {
  if (waves != 4 && waves != 8) return G9_ERR_SCHEDULE;
  if (schedule != G9_SCHED_DP && schedule != G9_SCHED_SK && schedule != G9_SCHED_SPLITK &&
      schedule != G9_SCHED_SK_HALF)
    return G9_ERR_SCHEDULE;
  // 256x128 stream-K tiles exist for FP16/BF16 with 4 waves only.
  if (schedule == G9_SCHED_SK_HALF && (waves != 4 || (dtype != G9_F16 && dtype != G9_BF16)))
    return G9_ERR_SCHEDULE;
  const KernelEntry* k = find_kernel(dtype, out, schedule, waves);
  if (!k) return G9_ERR_DTYPE;
  pl = Plan{};
  pl.block = 64 * waves;
  const bool half = schedule == G9_SCHED_SK_HALF;
  p.tiles_m = (p.M + kTile - 1) / kTile;
  p.tiles_n = half ? (p.N + 127) / 128 : (p.N + kTile - 1) / kTile;
  p.num_xcds = kNumXcds;
  p.group_m = kGroupM;
  const long long tiles = (long long)p.tiles_m * p.tiles_n;
  int grid;
  if (schedule == G9_SCHED_SPLITK) {
    const int cus = cu_count();
    if (cus <= 0) return G9_ERR_HIP;
    const int S = g9_splitk_factor(tiles, p.ns, cus);
    if (S <= 1) {
      // The grid fills the chip (or K is one stage): run the data-parallel kernel.
      k = find_kernel(dtype, out, G9_SCHED_DP, waves);
      grid = (int)tiles;
    } else {
      if (!ws || ws_bytes < splitk_bytes(tiles * S) || !aligned(ws, 256)) return G9_ERR_WORKSPACE;
      const size_t base = splitk_base(ws_bytes);
      if (base + (size_t)(tiles * S) * kWsTileBytes > ws_bytes) return G9_ERR_WORKSPACE;
      p.ws = reinterpret_cast<float*>(static_cast<char*>(ws) + base);
      p.split = S;
      grid = (int)(tiles * S);
      const long long threads = (long long)p.M * p.tiles_n * (kTile / 8);
      pl.red = reinterpret_cast<const void*>(out == G9_BF16 ? g9_splitk_reduce_bf16 : g9_splitk_reduce_f16);
      pl.red_grid = (int)((threads + 255) / 256);
    }
  } else if (schedule == G9_SCHED_DP) {
    grid = (int)tiles;
  } else {
    // The partials go behind the whole flag region g9_workspace_init clears
    // for this workspace size (as split-K's do), so a launch with fewer tiles
    // never writes partials over flag words a later, larger launch polls.
    const size_t tile_bytes = half ? kWsUnit : kWsTileBytes;
    if (!ws || ws_bytes < (half ? streamk_half_bytes(tiles) : streamk_bytes(tiles)) || !aligned(ws, 256))
      return G9_ERR_WORKSPACE;
    const size_t base = splitk_base(ws_bytes);
    if (base + (size_t)tiles * tile_bytes > ws_bytes) return G9_ERR_WORKSPACE;
    char* w = static_cast<char*>(ws);
    p.err = reinterpret_cast<int*>(w);
    p.flags = reinterpret_cast<u32*>(w + kWsHeader);
    p.ws = reinterpret_cast<float*>(w + base);
    const long long units = tiles * p.ns;
    int cus = cu_count();
    if (cus <= 0) return G9_ERR_HIP;
    grid = (int)(units < cus ? units : cus);
    p.sk_ctas = grid;
    pl.streamk = 1;
  }
  // Last, after every argument check, so bad arguments are reported
  // without touching the HIP runtime.
  if (hipGetDevice(&pl.device) != hipSuccess) return G9_ERR_HIP;
  pl.fn = reinterpret_cast<const void*>(k->fn);
  pl.grid = grid;
  pl.p = p;
  pl.magic = kPlanMagic;
  return G9_OK;
}

int run_plan(const Plan& pl, hipStream_t s) {
  GemmParams p = pl.p;
  if (pl.streamk) {
    p.epoch = (g_epoch.fetch_add(1) % 65535u) + 1u;
    p.spin_limit = g_spin_limit.load(std::memory_order_relaxed);
  }
  // hipLaunchKernel reports this launch's own status (hipGetLastError would
  // also return an earlier, unrelated error of the calling thread).
  void* args[] = {&p};
  if (hipLaunchKernel(pl.fn, dim3(pl.grid), dim3(pl.block), args, 0, s) != hipSuccess) return G9_ERR_HIP;
  if (pl.red && hipLaunchKernel(pl.red, dim3(pl.red_grid), dim3(256), args, 0, s) != hipSuccess) return G9_ERR_HIP;
  return G9_OK;
}

int launch(int dtype, int out, int schedule, int waves, GemmParams& p, void* ws, size_t ws_bytes,
           void* stream) {
  Plan pl;
  const int st = make_plan(dtype, out, schedule, waves, p, ws, ws_bytes, pl);
  return st ? st : run_plan(pl, reinterpret_cast<hipStream_t>(stream));
}

int check_common(int64_t M, int64_t N, int64_t K, int dtype, int64_t stride_cm, int64_t stride_cn,
                 const void* c, bool allow_tail = false);

// Shared launch path of the grouped kernels: T token rows, E experts.
int launch_moe(int dtype, int out, GemmParams& p, int64_t E, void* stream) {
  const KernelEntry* k = find_moe_kernel(dtype, out);
  if (!k) return G9_ERR_DTYPE;
  if (p.M == 0) return G9_OK;  // no tokens: nothing to write
  // Upper bound of the experts' m-tiles: sum ceil(M_e / 256) <= ceil(T / 256) + E.
  const long long tiles_m = (p.M + kTile - 1) / kTile + E;
  p.tiles_n = (p.N + kTile - 1) / kTile;
  if (tiles_m * p.tiles_n > INT32_MAX) return G9_ERR_SHAPE;
  p.tiles_m = (int)tiles_m;
  p.num_xcds = kNumXcds;
  p.group_m = kGroupM;
  p.moe_experts = (int)E;
  void* args[] = {&p};
  return hipLaunchKernel(reinterpret_cast<const void*>(k->fn), dim3((unsigned)(tiles_m * p.tiles_n)), dim3(256),
                         args, 0, reinterpret_cast<hipStream_t>(stream)) == hipSuccess
             ? G9_OK
             : G9_ERR_HIP;
}

int check_moe(int64_t T, int64_t N, int64_t K, int64_t E, int dtype, int64_t stride_cm, const void* c,
              const int32_t* offsets, int64_t stride_be) {
  if (T < 0 || T > (1 << 30) || E <= 0 || E > (1 << 20)) return G9_ERR_SHAPE;
  if (!offsets || !aligned(offsets, 4)) return G9_ERR_LAYOUT;
  if (stride_be < 0 || stride_be % 16 != 0) return G9_ERR_LAYOUT;
  if (T == 0) {  // only the remaining arguments' own validity matters
    if (N <= 0 || K <= 0 || K % stage_k(dtype) != 0) return G9_ERR_SHAPE;
    return G9_OK;
  }
  return check_common(T, N, K, dtype, stride_cm, 1, c);
}

int check_common(int64_t M, int64_t N, int64_t K, int dtype, int64_t stride_cm, int64_t stride_cn,
                 const void* c, bool allow_tail) {
  if (M <= 0 || N <= 0 || K <= 0) return G9_ERR_SHAPE;
  if (M > (1 << 30) || N > (1 << 30)) return G9_ERR_SHAPE;
  // Tile ids and the data-parallel grid are 32-bit.
  if (((M + kTile - 1) / kTile) * ((N + kTile - 1) / kTile) > INT32_MAX) return G9_ERR_SHAPE;
  const int sk = stage_k(dtype);
  // K tails (FP16/BF16/BF8 dense GEMMs): a partial first stage, whole 16-byte
  // chunks (K a multiple of 8 for 16-bit types, 16 for BF8).
  const int64_t chunk_k = sk / 8;  // elements per 16 bytes: 8 (16-bit), 16 (8-bit)
  if (allow_tail ? K % chunk_k != 0 : K % sk != 0) return G9_ERR_SHAPE;
  if ((K + sk - 1) / sk >= 65536) return G9_ERR_SHAPE;
  if (stride_cn != 1 || stride_cm < N || !aligned(c, 2)) return G9_ERR_LAYOUT;
  return G9_OK;
}

int check_operand(const void* p, int64_t row_stride_bytes, int64_t k_stride, int64_t k_bytes, bool k_tail = false) {
  if (k_stride != 1) return G9_ERR_LAYOUT;
  if (!aligned(p, 16) || row_stride_bytes % 16 != 0 || row_stride_bytes < k_bytes) return G9_ERR_LAYOUT;
  // 128 rows x stride must fit 31-bit offsets (dead offsets start at 2^31);
  // a K tail adds up to 112 bytes to a resource, so the stride stays below 2^24.
  if (row_stride_bytes > (1 << 24) || (k_tail && row_stride_bytes >= (1 << 24))) return G9_ERR_LAYOUT;
  return G9_OK;
}

}  // namespace

namespace {
// Validates the a16w16 arguments and fills p (shared by the two a16w16 entry points).
int prep_a16w16(GemmParams& p, const void* a, const void* b, void* c, int64_t M, int64_t N, int64_t K,
                int64_t stride_am, int64_t stride_ak, int64_t stride_bk, int64_t stride_bn, int64_t stride_cm,
                int64_t stride_cn, int dtype) {
  if (dtype != G9_F16 && dtype != G9_BF16) return G9_ERR_DTYPE;
  int st = check_common(M, N, K, dtype, stride_cm, stride_cn, c, /*allow_tail=*/true);
  if (st) return st;
  if ((st = check_operand(a, stride_am * 2, stride_ak, K * 2, K % 64 != 0))) return st;
  if ((st = check_operand(b, stride_bn * 2, stride_bk, K * 2, K % 64 != 0))) return st;
  p = GemmParams{};
  p.a = static_cast<const char*>(a);
  p.b = static_cast<const char*>(b);
  p.c = static_cast<char*>(c);
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  p.lda = (u32)(stride_am * 2);
  p.ldb = (u32)(stride_bn * 2);
  p.ldc = stride_cm;
  p.ns = (int)((K + 63) / 64);
  p.kshift = (u32)(p.ns * 128 - K * 2);
  return G9_OK;
}
}  // namespace

namespace {

int plan_a16w16(Plan& pl, const void* a, const void* b, void* c, int64_t M, int64_t N, int64_t K,
                int64_t stride_am, int64_t stride_ak, int64_t stride_bk, int64_t stride_bn,
                int64_t stride_cm, int64_t stride_cn, int dtype, int schedule, int waves,
                void* workspace, size_t workspace_bytes) {
  GemmParams p;
  const int st = prep_a16w16(p, a, b, c, M, N, K, stride_am, stride_ak, stride_bk, stride_bn, stride_cm, stride_cn,
                             dtype);
  if (st) return st;
  return make_plan(dtype, dtype, schedule, waves, p, workspace, workspace_bytes, pl);
}

int plan_a8w8(Plan& pl, const void* a, const void* b, void* c, int64_t M, int64_t N, int64_t K,
              int64_t stride_am, int64_t stride_ak, int64_t stride_bk, int64_t stride_bn,
              int64_t stride_cm, int64_t stride_cn, const float* a_scale, const float* b_scale,
              int out_dtype, int schedule, int waves, void* workspace, size_t workspace_bytes) {
  if (out_dtype != G9_F16 && out_dtype != G9_BF16) return G9_ERR_DTYPE;
  int st = check_common(M, N, K, G9_BF8, stride_cm, stride_cn, c, /*allow_tail=*/true);
  if (st) return st;
  if ((st = check_operand(a, stride_am, stride_ak, K, K % 128 != 0))) return st;
  if ((st = check_operand(b, stride_bn, stride_bk, K, K % 128 != 0))) return st;
  if ((a_scale && !aligned(a_scale, 4)) || (b_scale && !aligned(b_scale, 4))) return G9_ERR_LAYOUT;
  GemmParams p{};
  p.a = static_cast<const char*>(a);
  p.b = static_cast<const char*>(b);
  p.c = static_cast<char*>(c);
  p.a_scale = a_scale;
  p.b_scale = b_scale;
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  p.lda = (u32)stride_am;
  p.ldb = (u32)stride_bn;
  p.ldc = stride_cm;
  p.ns = (int)((K + 127) / 128);
  p.kshift = (u32)(p.ns * 128 - K);
  return make_plan(G9_BF8, out_dtype, schedule, waves, p, workspace, workspace_bytes, pl);
}

int plan_a4w4(Plan& pl, const void* a, const void* b, void* c, const void* a_scales, const void* b_scales,
              int64_t M, int64_t N, int64_t K, int64_t stride_am, int64_t stride_ak,
              int64_t stride_bn, int64_t stride_bk, int64_t stride_cm, int64_t stride_cn,
              int64_t stride_asm, int64_t stride_ask, int64_t stride_bsn, int64_t stride_bsk,
              int out_dtype, int schedule, int waves, void* workspace, size_t workspace_bytes) {
  if (out_dtype != G9_F16 && out_dtype != G9_BF16) return G9_ERR_DTYPE;
  int st = check_common(M, N, K, G9_FP4, stride_cm, stride_cn, c);
  if (st) return st;
  if ((st = check_operand(a, stride_am, stride_ak, K / 2))) return st;
  if ((st = check_operand(b, stride_bn, stride_bk, K / 2))) return st;
  if (!a_scales || !b_scales) return G9_ERR_LAYOUT;
  if (!aligned(a_scales, 4) || !aligned(b_scales, 4)) return G9_ERR_LAYOUT;
  // Row-major scales (K/32 contiguous groups per row), or K-major for both
  // operands (rows contiguous, groups stride_ask / stride_bsk bytes apart:
  // the transposed views the reference bench passes), which the 4-wave
  // kernels read without a re-layout.
  const bool kmajor = stride_asm == 1 && stride_bsn == 1 && stride_ask != 1 && stride_bsk != 1;
  int dtype = G9_FP4;
  if (kmajor) {
    if (waves != 4) return G9_ERR_SCHEDULE;
    if (stride_ask % 4 || stride_bsk % 4 || stride_ask < M || stride_bsk < N) return G9_ERR_LAYOUT;
    // Group offsets stay below the kernels' 2^31 dead offset.
    if ((K / 32) * stride_ask + 4096 >= (int64_t(1) << 31) || (K / 32) * stride_bsk + 4096 >= (int64_t(1) << 31))
      return G9_ERR_SHAPE;
    dtype = G9_FP4K;
    stride_asm = stride_ask;
    stride_bsn = stride_bsk;
  } else {
    if (stride_ask != 1 || stride_bsk != 1) return G9_ERR_LAYOUT;
    if (stride_asm % 4 || stride_bsn % 4 || stride_asm < K / 32 || stride_bsn < K / 32) return G9_ERR_LAYOUT;
    if (stride_asm > (1 << 24) || stride_bsn > (1 << 24)) return G9_ERR_LAYOUT;
  }
  GemmParams p{};
  p.a = static_cast<const char*>(a);
  p.b = static_cast<const char*>(b);
  p.c = static_cast<char*>(c);
  p.a_sc = static_cast<const unsigned char*>(a_scales);
  p.b_sc = static_cast<const unsigned char*>(b_scales);
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  p.lda = (u32)stride_am;
  p.ldb = (u32)stride_bn;
  p.ldsa = (u32)stride_asm;  // K-major: bytes between scale groups
  p.ldsb = (u32)stride_bsn;
  p.ldc = stride_cm;
  p.ns = (int)(K / stage_k(G9_FP4));
  return make_plan(dtype, out_dtype, schedule, waves, p, workspace, workspace_bytes, pl);
}

int plan_a4w4_preshuffled(Plan& pl, const void* a, const void* b, void* c, const void* a_scales, const void* b_scales,
                          int64_t M, int64_t N, int64_t K, int64_t stride_am, int64_t stride_ak,
                          int64_t stride_bn, int64_t stride_bk, int64_t stride_cm, int64_t stride_cn,
                          int64_t stride_asc, int64_t stride_bsc, int out_dtype, int schedule, int waves,
                          void* workspace, size_t workspace_bytes) {
  if (out_dtype != G9_F16 && out_dtype != G9_BF16) return G9_ERR_DTYPE;
  int st = check_common(M, N, K, G9_FP4P, stride_cm, stride_cn, c);
  if (st) return st;
  if ((st = check_operand(a, stride_am, stride_ak, K / 2))) return st;
  if ((st = check_operand(b, stride_bn, stride_bk, K / 2))) return st;
  if (schedule != G9_SCHED_DP || waves != 4) return G9_ERR_SCHEDULE;
  // Chunks of 32 bytes per row; every chunk part is a 16-byte aligned KiB.
  if (!a_scales || !b_scales || !aligned(a_scales, 16) || !aligned(b_scales, 16)) return G9_ERR_LAYOUT;
  const int64_t chunks = (K / 256 + 3) / 4;
  if (chunks == 1) {  // the stride of a single chunk is never used (and reads as anything in a size-1 dimension)
    stride_asc = 32 * M;
    stride_bsc = 32 * N;
  }
  if (stride_asc < 32 * M || stride_bsc < 32 * N || stride_asc % 16 || stride_bsc % 16) return G9_ERR_LAYOUT;
  // The kernel addresses each scale array with 32-bit offsets below 2^31.
  if ((chunks - 1) * stride_asc + 32 * M + 4096 >= (int64_t(1) << 31) ||
      (chunks - 1) * stride_bsc + 32 * N + 4096 >= (int64_t(1) << 31))
    return G9_ERR_SHAPE;
  GemmParams p{};
  p.a = static_cast<const char*>(a);
  p.b = static_cast<const char*>(b);
  p.c = static_cast<char*>(c);
  p.a_sc = static_cast<const unsigned char*>(a_scales);
  p.b_sc = static_cast<const unsigned char*>(b_scales);
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  p.lda = (u32)stride_am;
  p.ldb = (u32)stride_bn;
  p.ldsa = (u32)stride_asc;
  p.ldsb = (u32)stride_bsc;
  p.ldc = stride_cm;
  p.ns = (int)(K / stage_k(G9_FP4P));
  return make_plan(G9_FP4P, out_dtype, schedule, waves, p, workspace, workspace_bytes, pl);
}

}  // namespace

extern "C" {

int g9_gemm_a16w16(const void* a, const void* b, void* c, int64_t M, int64_t N, int64_t K,
                   int64_t stride_am, int64_t stride_ak, int64_t stride_bk, int64_t stride_bn,
                   int64_t stride_cm, int64_t stride_cn, int dtype, int schedule, int waves,
                   void* workspace, size_t workspace_bytes, void* stream) {
  Plan pl;
  const int st = plan_a16w16(pl, a, b, c, M, N, K, stride_am, stride_ak, stride_bk, stride_bn, stride_cm, stride_cn,
                             dtype, schedule, waves, workspace, workspace_bytes);
  return st ? st : run_plan(pl, reinterpret_cast<hipStream_t>(stream));
}

int g9_gemm_a8w8(const void* a, const void* b, void* c, int64_t M, int64_t N, int64_t K,
                 int64_t stride_am, int64_t stride_ak, int64_t stride_bk, int64_t stride_bn,
                 int64_t stride_cm, int64_t stride_cn, const float* a_scale, const float* b_scale,
                 int out_dtype, int schedule, int waves, void* workspace, size_t workspace_bytes,
                 void* stream) {
  Plan pl;
  const int st = plan_a8w8(pl, a, b, c, M, N, K, stride_am, stride_ak, stride_bk, stride_bn, stride_cm, stride_cn,
                           a_scale, b_scale, out_dtype, schedule, waves, workspace, workspace_bytes);
  return st ? st : run_plan(pl, reinterpret_cast<hipStream_t>(stream));
}

int g9_gemm_a4w4(const void* a, const void* b, void* c, const void* a_scales, const void* b_scales,
                 int64_t M, int64_t N, int64_t K, int64_t stride_am, int64_t stride_ak,
                 int64_t stride_bn, int64_t stride_bk, int64_t stride_cm, int64_t stride_cn,
                 int64_t stride_asm, int64_t stride_ask, int64_t stride_bsn, int64_t stride_bsk,
                 int out_dtype, int schedule, int waves, void* workspace, size_t workspace_bytes,
                 void* stream) {
  Plan pl;
  const int st = plan_a4w4(pl, a, b, c, a_scales, b_scales, M, N, K, stride_am, stride_ak, stride_bn, stride_bk,
                           stride_cm, stride_cn, stride_asm, stride_ask, stride_bsn, stride_bsk, out_dtype, schedule,
                           waves, workspace, workspace_bytes);
  return st ? st : run_plan(pl, reinterpret_cast<hipStream_t>(stream));
}

int g9_gemm_a4w4_preshuffled(const void* a, const void* b, void* c, const void* a_scales, const void* b_scales,
                             int64_t M, int64_t N, int64_t K, int64_t stride_am, int64_t stride_ak,
                             int64_t stride_bn, int64_t stride_bk, int64_t stride_cm, int64_t stride_cn,
                             int64_t stride_asc, int64_t stride_bsc, int out_dtype, int schedule, int waves,
                             void* workspace, size_t workspace_bytes, void* stream) {
  Plan pl;
  const int st = plan_a4w4_preshuffled(pl, a, b, c, a_scales, b_scales, M, N, K, stride_am, stride_ak, stride_bn,
                                       stride_bk, stride_cm, stride_cn, stride_asc, stride_bsc, out_dtype, schedule,
                                       waves, workspace, workspace_bytes);
  return st ? st : run_plan(pl, reinterpret_cast<hipStream_t>(stream));
}

// Prepared launches: the same validation and plan as the entry points above,
// kept in the caller's g9_plan instead of being enqueued.
namespace {
int store_plan(g9_plan* out, const Plan& pl, int st) {
  if (st) return st;
  memcpy(out, &pl, sizeof pl);
  return G9_OK;
}
}  // namespace

int g9_plan_a16w16(g9_plan* plan, const void* a, const void* b, void* c, int64_t M, int64_t N, int64_t K,
                   int64_t stride_am, int64_t stride_ak, int64_t stride_bk, int64_t stride_bn,
                   int64_t stride_cm, int64_t stride_cn, int dtype, int schedule, int waves,
                   void* workspace, size_t workspace_bytes) {
  if (!plan) return G9_ERR_PLAN;
  Plan pl;
  return store_plan(plan, pl,
                    plan_a16w16(pl, a, b, c, M, N, K, stride_am, stride_ak, stride_bk, stride_bn, stride_cm,
                                stride_cn, dtype, schedule, waves, workspace, workspace_bytes));
}

int g9_plan_a8w8(g9_plan* plan, const void* a, const void* b, void* c, int64_t M, int64_t N, int64_t K,
                 int64_t stride_am, int64_t stride_ak, int64_t stride_bk, int64_t stride_bn,
                 int64_t stride_cm, int64_t stride_cn, const float* a_scale, const float* b_scale,
                 int out_dtype, int schedule, int waves, void* workspace, size_t workspace_bytes) {
  if (!plan) return G9_ERR_PLAN;
  Plan pl;
  return store_plan(plan, pl,
                    plan_a8w8(pl, a, b, c, M, N, K, stride_am, stride_ak, stride_bk, stride_bn, stride_cm,
                              stride_cn, a_scale, b_scale, out_dtype, schedule, waves, workspace, workspace_bytes));
}

int g9_plan_a4w4(g9_plan* plan, const void* a, const void* b, void* c, const void* a_scales, const void* b_scales,
                 int64_t M, int64_t N, int64_t K, int64_t stride_am, int64_t stride_ak,
                 int64_t stride_bn, int64_t stride_bk, int64_t stride_cm, int64_t stride_cn,
                 int64_t stride_asm, int64_t stride_ask, int64_t stride_bsn, int64_t stride_bsk,
                 int out_dtype, int schedule, int waves, void* workspace, size_t workspace_bytes) {
  if (!plan) return G9_ERR_PLAN;
  Plan pl;
  return store_plan(plan, pl,
                    plan_a4w4(pl, a, b, c, a_scales, b_scales, M, N, K, stride_am, stride_ak, stride_bn, stride_bk,
                              stride_cm, stride_cn, stride_asm, stride_ask, stride_bsn, stride_bsk, out_dtype,
                              schedule, waves, workspace, workspace_bytes));
}

int g9_plan_a4w4_preshuffled(g9_plan* plan, const void* a, const void* b, void* c, const void* a_scales,
                             const void* b_scales, int64_t M, int64_t N, int64_t K, int64_t stride_am,
                             int64_t stride_ak, int64_t stride_bn, int64_t stride_bk, int64_t stride_cm,
                             int64_t stride_cn, int64_t stride_asc, int64_t stride_bsc, int out_dtype,
                             int schedule, int waves, void* workspace, size_t workspace_bytes) {
  if (!plan) return G9_ERR_PLAN;
  Plan pl;
  return store_plan(plan, pl,
                    plan_a4w4_preshuffled(pl, a, b, c, a_scales, b_scales, M, N, K, stride_am, stride_ak, stride_bn,
                                          stride_bk, stride_cm, stride_cn, stride_asc, stride_bsc, out_dtype,
                                          schedule, waves, workspace, workspace_bytes));
}

int g9_plan_launch(const g9_plan* plan, void* stream) {
  if (!plan) return G9_ERR_PLAN;
  Plan pl;
  memcpy(&pl, plan, sizeof pl);
  if (pl.magic != kPlanMagic) return G9_ERR_PLAN;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int dev = -1;
  if ((s ? hipStreamGetDevice(s, &dev) : hipGetDevice(&dev)) != hipSuccess) return G9_ERR_HIP;
  if (dev != pl.device) return G9_ERR_PLAN;
  return run_plan(pl, s);
}

int g9_moe_a16w16(const void* a, const void* b, void* c, const int32_t* expert_offsets, int64_t T,
                  int64_t N, int64_t K, int64_t E, int64_t stride_am, int64_t stride_bn, int64_t stride_be,
                  int64_t stride_cm, int dtype, void* stream) {
  if (dtype != G9_F16 && dtype != G9_BF16) return G9_ERR_DTYPE;
  int st = check_moe(T, N, K, E, dtype, stride_cm, c, expert_offsets, stride_be);
  if (st || T == 0) return st;
  if ((st = check_operand(a, stride_am * 2, 1, K * 2))) return st;
  if ((st = check_operand(b, stride_bn * 2, 1, K * 2))) return st;
  GemmParams p{};
  p.a = static_cast<const char*>(a);
  p.b = static_cast<const char*>(b);
  p.c = static_cast<char*>(c);
  p.M = (int)T;
  p.N = (int)N;
  p.K = (int)K;
  p.lda = (u32)(stride_am * 2);
  p.ldb = (u32)(stride_bn * 2);
  p.ldc = stride_cm;
  p.ns = (int)(K / stage_k(dtype));
  p.moe_off = expert_offsets;
  p.moe_b_stride = stride_be;
  return launch_moe(dtype, dtype, p, E, stream);
}

int g9_moe_a8w8(const void* a, const void* b, void* c, const int32_t* expert_offsets, const float* a_scale,
                const float* b_scales, int64_t T, int64_t N, int64_t K, int64_t E, int64_t stride_am,
                int64_t stride_bn, int64_t stride_be, int64_t stride_cm, int out_dtype, void* stream) {
  if (out_dtype != G9_F16 && out_dtype != G9_BF16) return G9_ERR_DTYPE;
  int st = check_moe(T, N, K, E, G9_BF8, stride_cm, c, expert_offsets, stride_be);
  if (st || T == 0) return st;
  if ((st = check_operand(a, stride_am, 1, K))) return st;
  if ((st = check_operand(b, stride_bn, 1, K))) return st;
  if ((a_scale && !aligned(a_scale, 4)) || (b_scales && !aligned(b_scales, 4))) return G9_ERR_LAYOUT;
  GemmParams p{};
  p.a = static_cast<const char*>(a);
  p.b = static_cast<const char*>(b);
  p.c = static_cast<char*>(c);
  p.a_scale = a_scale;
  p.b_scale = b_scales;
  p.M = (int)T;
  p.N = (int)N;
  p.K = (int)K;
  p.lda = (u32)stride_am;
  p.ldb = (u32)stride_bn;
  p.ldc = stride_cm;
  p.ns = (int)(K / stage_k(G9_BF8));
  p.moe_off = expert_offsets;
  p.moe_b_stride = stride_be;
  return launch_moe(G9_BF8, out_dtype, p, E, stream);
}

int g9_moe_a4w4(const void* a, const void* b, void* c, const void* a_scales, const void* b_scales,
                const int32_t* expert_offsets, int64_t T, int64_t N, int64_t K, int64_t E, int64_t stride_am,
                int64_t stride_bn, int64_t stride_be, int64_t stride_asm, int64_t stride_bsn,
                int64_t stride_bse, int64_t stride_cm, int out_dtype, void* stream) {
  if (out_dtype != G9_F16 && out_dtype != G9_BF16) return G9_ERR_DTYPE;
  int st = check_moe(T, N, K, E, G9_FP4, stride_cm, c, expert_offsets, stride_be);
  if (st || T == 0) return st;
  if ((st = check_operand(a, stride_am, 1, K / 2))) return st;
  if ((st = check_operand(b, stride_bn, 1, K / 2))) return st;
  if (!a_scales || !b_scales || !aligned(a_scales, 4) || !aligned(b_scales, 4)) return G9_ERR_LAYOUT;
  if (stride_asm % 4 || stride_bsn % 4 || stride_asm < K / 32 || stride_bsn < K / 32) return G9_ERR_LAYOUT;
  if (stride_asm > (1 << 24) || stride_bsn > (1 << 24)) return G9_ERR_LAYOUT;
  if (stride_bse < 0 || stride_bse % 4) return G9_ERR_LAYOUT;
  GemmParams p{};
  p.a = static_cast<const char*>(a);
  p.b = static_cast<const char*>(b);
  p.c = static_cast<char*>(c);
  p.a_sc = static_cast<const unsigned char*>(a_scales);
  p.b_sc = static_cast<const unsigned char*>(b_scales);
  p.M = (int)T;
  p.N = (int)N;
  p.K = (int)K;
  p.lda = (u32)stride_am;
  p.ldb = (u32)stride_bn;
  p.ldsa = (u32)stride_asm;
  p.ldsb = (u32)stride_bsn;
  p.ldc = stride_cm;
  p.ns = (int)(K / stage_k(G9_FP4));
  p.moe_off = expert_offsets;
  p.moe_b_stride = stride_be;
  p.moe_bsc_stride = stride_bse;
  return launch_moe(G9_FP4, out_dtype, p, E, stream);
}

const char* g9_moe_kernel_name(int dtype, int out_dtype) {
  const KernelEntry* k = find_moe_kernel(dtype, out_dtype);
  return k ? k->name : nullptr;
}

size_t g9_workspace_size(int dtype, int64_t M, int64_t N, int64_t K, int schedule, int waves) {
  if (M <= 0 || N <= 0 || K <= 0 || stage_k(dtype) == 0) return 0;
  const long long tiles = ((M + kTile - 1) / kTile) * ((N + kTile - 1) / kTile);
  if (schedule == G9_SCHED_SPLITK) {
    const int cus = cu_count();
    const int S = cus > 0 ? g9_splitk_factor(tiles, (int)((K + stage_k(dtype) - 1) / stage_k(dtype)), cus) : 1;
    return S > 1 ? splitk_bytes(tiles * S) : 0;
  }
  if (schedule == G9_SCHED_SK_HALF) {
    // Only FP16/BF16 with 4 waves run this schedule (the launch rejects the rest).
    if ((dtype != G9_F16 && dtype != G9_BF16) || waves != 4) return 0;
    return streamk_half_bytes(((M + kTile - 1) / kTile) * ((N + 127) / 128));
  }
  if (schedule != G9_SCHED_SK) return 0;
  return streamk_bytes(tiles);
}

// Split factor from a cost model in units of one K stage (~2048 MFMA cycles):
// data-parallel costs its one tile chain plus the epilogue (~4); split-K with
// S segments costs one segment (one wave of tiles * S <= cus workgroups) plus
// ~7 for its prologue and partial store, plus ~0.04 per 256 KiB partial the
// reduction reads at full-chip bandwidth.  Grids that fill half the chip, and
// factors past 16, are not split.
int g9_splitk_factor(int64_t tiles, int stages, int cus) {
  if (tiles <= 0 || stages < 2 || cus <= 0 || tiles * 2 > cus) return 1;
  int best = 1;
  long long best_cost = 100LL * stages + 400;
  for (int S = 2; S <= 16 && S <= stages && tiles * S <= cus; ++S) {
    const long long cost = 100LL * ((stages + S - 1) / S) + 700 + 4LL * S * tiles;
    if (cost < best_cost) {
      best = S;
      best_cost = cost;
    }
  }
  return best;
}

}  // extern "C"

namespace {
__global__ void zero_words(u32* p, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}
__global__ void set_words2(u32* p, u32 lo, u32 hi) {
  if (threadIdx.x == 0) {
    p[0] = lo;
    p[1] = hi;
  }
}
// dst (cols x rows, row stride dst_ld) = transpose of src (rows x cols, row
// stride src_ld), bytes, through a 64 x 64 LDS tile per workgroup.  Full
// tiles with 4-byte aligned rows move dwords: 16 lanes read a source row's 64
// bytes, and each lane then packs 4 source rows' bytes of one column into a
// dword of the destination row; edge tiles and unaligned operands go byte by
// byte.
__global__ __launch_bounds__(256) void transpose_u8(const unsigned char* src, long long rows, long long cols,
                                                    long long src_ld, unsigned char* dst, long long dst_ld,
                                                    int words) {
  __shared__ __attribute__((aligned(4))) unsigned char tile[64][68];
  const long long r0 = (long long)blockIdx.y * 64, c0 = (long long)blockIdx.x * 64;
  const bool full = words && r0 + 64 <= rows && c0 + 64 <= cols;
  if (full) {
    for (int i = threadIdx.x; i < 64 * 16; i += 256) {
      const int r = i >> 4, w = i & 15;
      *reinterpret_cast<u32*>(&tile[r][4 * w]) = *reinterpret_cast<const u32*>(src + (r0 + r) * src_ld + c0 + 4 * w);
    }
  } else {
    for (int i = threadIdx.x; i < 64 * 64; i += 256) {
      const int r = i >> 6, c = i & 63;
      if (r0 + r < rows && c0 + c < cols) tile[r][c] = src[(r0 + r) * src_ld + c0 + c];
    }
  }
  __syncthreads();
  if (full) {
    for (int i = threadIdx.x; i < 64 * 16; i += 256) {
      const int c = i >> 4, w = i & 15;
      const u32 v = (u32)tile[4 * w][c] | ((u32)tile[4 * w + 1][c] << 8) | ((u32)tile[4 * w + 2][c] << 16) |
                    ((u32)tile[4 * w + 3][c] << 24);
      *reinterpret_cast<u32*>(dst + (c0 + c) * dst_ld + r0 + 4 * w) = v;
    }
  } else {
    for (int i = threadIdx.x; i < 64 * 64; i += 256) {
      const int c = i >> 6, r = i & 63;
      if (r0 + r < rows && c0 + c < cols) dst[(c0 + c) * dst_ld + r0 + r] = tile[r][c];
    }
  }
}
}  // namespace

extern "C" {

int g9_workspace_init(void* workspace, size_t workspace_bytes, void* stream) {
  if (!workspace || workspace_bytes < kWsHeader || !aligned(workspace, 256)) return G9_ERR_WORKSPACE;
  // Header and flags precede the partial tiles.  Clear the flags of the
  // largest tile count whose partials fit this workspace, so every launch the
  // workspace is large enough for finds its flags cleared.
  const size_t max_tiles = (workspace_bytes - kWsHeader) / kWsUnit + 1;
  size_t words = (kWsHeader + flags_bytes((long long)max_tiles)) / 4;
  if (words > workspace_bytes / 4) words = workspace_bytes / 4;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int threads = 256;
  const int blocks = (int)((words + threads - 1) / threads);
  u32* w = static_cast<u32*>(workspace);
  void* args[] = {&w, &words};
  return hipLaunchKernel(reinterpret_cast<const void*>(zero_words), dim3(blocks), dim3(threads), args, 0, s) ==
                 hipSuccess
             ? G9_OK
             : G9_ERR_HIP;
}

int g9_workspace_watch(void* workspace, size_t workspace_bytes, int* host_flag, void* stream) {
  if (!workspace || workspace_bytes < kWsHeader || !aligned(workspace, 256)) return G9_ERR_WORKSPACE;
  if (host_flag && !aligned(host_flag, 4)) return G9_ERR_LAYOUT;
  // Header bytes 8-15 hold the flag's address; written by a kernel on the
  // stream (no memset or copy, so the call can be captured in a graph).
  u32* w = reinterpret_cast<u32*>(static_cast<char*>(workspace) + 8);
  const uint64_t a = reinterpret_cast<uintptr_t>(host_flag);
  u32 lo = (u32)a, hi = (u32)(a >> 32);
  void* args[] = {&w, &lo, &hi};
  return hipLaunchKernel(reinterpret_cast<const void*>(set_words2), dim3(1), dim3(64), args, 0,
                         reinterpret_cast<hipStream_t>(stream)) == hipSuccess
             ? G9_OK
             : G9_ERR_HIP;
}

int g9_transpose_u8(const void* src, int64_t rows, int64_t cols, int64_t src_ld, void* dst, int64_t dst_ld,
                    void* stream) {
  if (rows < 0 || cols < 0) return G9_ERR_SHAPE;
  if (rows == 0 || cols == 0) return G9_OK;
  if (!src || !dst || src_ld < cols || dst_ld < rows) return G9_ERR_LAYOUT;
  if ((rows + 63) / 64 > 65535 || (cols + 63) / 64 > INT32_MAX) return G9_ERR_SHAPE;
  const unsigned char* s = static_cast<const unsigned char*>(src);
  unsigned char* d = static_cast<unsigned char*>(dst);
  long long r = rows, c = cols, sl = src_ld, dl = dst_ld;
  int words = aligned(src, 4) && aligned(dst, 4) && src_ld % 4 == 0 && dst_ld % 4 == 0;
  void* args[] = {&s, &r, &c, &sl, &d, &dl, &words};
  return hipLaunchKernel(reinterpret_cast<const void*>(transpose_u8), dim3((unsigned)((cols + 63) / 64),
                                                                           (unsigned)((rows + 63) / 64)),
                         dim3(256), args, 0, reinterpret_cast<hipStream_t>(stream)) == hipSuccess
             ? G9_OK
             : G9_ERR_HIP;
}

uint32_t g9_set_streamk_spin_limit(uint32_t polls) {
  return g_spin_limit.exchange(polls ? polls : kDefaultSpinLimit);
}

int g9_workspace_error(const void* workspace, size_t workspace_bytes, void* stream, int* error) {
  if (!workspace || workspace_bytes < kWsHeader || !error) return G9_ERR_WORKSPACE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int v = 0;
  if (hipMemcpyAsync(&v, workspace, sizeof(int), hipMemcpyDeviceToHost, s) != hipSuccess) return G9_ERR_HIP;
  if (hipStreamSynchronize(s) != hipSuccess) return G9_ERR_HIP;
  *error = v;
  return G9_OK;
}

const char* g9_kernel_name(int dtype, int out_dtype, int schedule, int waves) {
  const KernelEntry* k = find_kernel(dtype, out_dtype, schedule, waves);
  return k ? k->name : nullptr;
}

const char* g9_status_string(int status) {
  switch (status) {
    case G9_OK:
      return "ok";
    case G9_ERR_SHAPE:
      return "unsupported shape";
    case G9_ERR_LAYOUT:
      return "unsupported layout, stride or alignment";
    case G9_ERR_DTYPE:
      return "unsupported dtype";
    case G9_ERR_SCHEDULE:
      return "unsupported schedule or wave count";
    case G9_ERR_WORKSPACE:
      return "stream-K / split-K workspace missing or too small";
    case G9_ERR_HIP:
      return "HIP launch failed";
    case G9_ERR_SCRATCH:
      return "the call needs more workspace than the static scratch buffer of g9_gemm_a16w16_noalloc holds";
    case G9_ERR_PLAN:
      return "plan not prepared by g9_plan_*, or launched on a device other than the one it was prepared on";
  }
  return "unknown status";
}

int g9_streamk_workgroups(void) { return cu_count(); }

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free a16w16 (g9_gemm_a16w16_noalloc): the stream-K / split-K
// workspace is this static device array instead of a caller buffer.  It holds
// kScratchTiles 256x256 partial tiles, or twice as many 256x128 ones (64 MiB
// plus the header and one flag word per 256x128 unit), and
// lives, on every GPU the library runs on, until the process ends.  Host code
// never passes `scratch` itself to a kernel (in host code the name is a
// stand-in, not a device address): the device address comes from
// hipGetSymbolAddress, once per device, with that device current.
// ---------------------------------------------------------------------------
constexpr long long kScratchTiles = G9_NOALLOC_MAX_TILES;
constexpr size_t kScratchBytes =
    kWsHeader + ((size_t)(2 * kScratchTiles + 1) * 4 + 255) / 256 * 256 + (size_t)kScratchTiles * kWsTileBytes;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices];

// Device address of `scratch` on the current device `dev` (looked up on the
// first call for that device).
int scratch_ptr(int dev, void** out) {
  if (dev < 0 || dev >= kMaxScratchDevices) return G9_ERR_HIP;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return G9_ERR_HIP;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return G9_OK;
}

// Makes `dev` current for the lifetime of the object, restoring the previous
// device afterwards.
struct DeviceGuard {
  int prev = -1;
  bool ok = false;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) return;
    ok = prev == dev || hipSetDevice(dev) == hipSuccess;
  }
  ~DeviceGuard() {
    if (ok && prev >= 0) (void)hipSetDevice(prev);
  }
};
}  // namespace

extern "C" {

int g9_gemm_a16w16_noalloc(const void* a, const void* b, void* c, int64_t M, int64_t N, int64_t K,
                           int64_t stride_am, int64_t stride_ak, int64_t stride_bk, int64_t stride_bn,
                           int64_t stride_cm, int64_t stride_cn, int dtype, int schedule, int waves,
                           void* stream) {
  GemmParams p;
  int st = prep_a16w16(p, a, b, c, M, N, K, stride_am, stride_ak, stride_bk, stride_bn, stride_cm, stride_cn, dtype);
  if (st) return st;
  if (waves != 4 && waves != 8) return G9_ERR_SCHEDULE;
  if (schedule != G9_SCHED_DP && schedule != G9_SCHED_SK && schedule != G9_SCHED_SPLITK &&
      schedule != G9_SCHED_SK_HALF)
    return G9_ERR_SCHEDULE;
  if (schedule == G9_SCHED_SK_HALF && waves != 4) return G9_ERR_SCHEDULE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int dev = 0;
  if (hipStreamGetDevice(s, &dev) != hipSuccess) return G9_ERR_HIP;
  DeviceGuard guard(dev);
  if (!guard.ok) return G9_ERR_HIP;
  const size_t need = g9_workspace_size(dtype, M, N, K, schedule, waves);
  if (need == 0) return launch(dtype, dtype, schedule, waves, p, nullptr, 0, stream);
  if (need > kScratchBytes) return G9_ERR_SCRATCH;
  void* ws = nullptr;
  if ((st = scratch_ptr(dev, &ws))) return st;
  // Stream-K needs its error word and flags at zero: clear them with a fill
  // kernel (no hipMemsetAsync, so the call can be captured in a graph).
  // Split-K writes every partial it reads, so it needs no clearing.
  if ((schedule == G9_SCHED_SK || schedule == G9_SCHED_SK_HALF) && (st = g9_workspace_init(ws, kScratchBytes, stream)))
    return st;
  return launch(dtype, dtype, schedule, waves, p, ws, kScratchBytes, stream);
}

int g9_noalloc_error(void* stream, int* error) {
  if (!error) return G9_ERR_LAYOUT;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int dev = 0;
  if (hipStreamGetDevice(s, &dev) != hipSuccess) return G9_ERR_HIP;
  DeviceGuard guard(dev);
  if (!guard.ok) return G9_ERR_HIP;
  void* ws = nullptr;
  const int st = scratch_ptr(dev, &ws);
  if (st) return st;
  return g9_workspace_error(ws, kScratchBytes, stream, error);
}

int g9_version(void) { return 100; }

}  // extern "C"

#ifdef G9_TIMING
#include "../../include/gfx950_gemm_timing.h"
extern "C" int g9_timing_read(void* host, size_t bytes) {
  if (bytes > sizeof(g9::g9_timing_buf)) return G9_ERR_SHAPE;
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(g9::g9_timing_buf), bytes, 0, hipMemcpyDeviceToHost) == hipSuccess
             ? G9_OK
             : G9_ERR_HIP;
}
extern "C" int g9_timing_capacity(void) { return g9::kTimingTiles; }
#endif
