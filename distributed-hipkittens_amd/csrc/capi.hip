// C ABI of the gfx950 FP8 MoE path (declarations: include/hkmoe.h).
//
// Host code: argument validation (before any launch), launch configuration,
// workspace carving and stream-ordered enqueueing.  No host synchronisation and
// no allocation happens in any entry point: callers own every buffer, as with
// the reference's dispatch functions (include/pyutils/pyutils.cuh:54-71,
// kernels/cdna3/.../256_256_64_32.cpp:202-206).
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>

#include "../../include/hkmoe.h"
#include "gemm_fp8.hpp"
#include "gemm_narrow.hpp"
#include "gemm_small.hpp"
#include "moe_kernels.hpp"

#include <atomic>
#include <cstdlib>
#include <mutex>
#include <vector>

using namespace hkmoe;

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(HKMOE_ERR_HIP, "%s: %s", what, hipGetErrorString(err));
  return HKMOE_OK;
}

// ---------------------------------------------------------------------------
// Kernel timing of the layer entry points (hkmoe_kernel_timing).  While it is
// on, each kernel a layer call enqueues is launched by hipExtLaunchKernelGGL
// with a pair of library-owned events that take that dispatch's own start and
// end timestamps: no marker packet goes between the kernels, so the timed
// calls keep the untimed schedule.  One set of events per call, in a ring of
// `calls` sets; t_slot is the set of the call being enqueued (-1: untimed) and
// t_role the kernel role about to be launched.
// ---------------------------------------------------------------------------
struct KernelTiming {
  int calls = 0;                 // ring size, 0: off
  int next = 0;                  // next call's set
  int device = -1;
  std::vector<hipEvent_t> ev;    // [calls][HKMOE_TIMING_ROLES][2]
  std::vector<uint8_t> used;     // [calls][HKMOE_TIMING_ROLES]
  std::vector<int> first, last;  // [calls]: roles of the call's first and last launch
};
KernelTiming g_timing;
std::mutex g_timing_mu;
thread_local int t_slot = -1;
thread_local int t_role = -1;

// The events of the launch about to be made (false: launch untimed).
bool timing_events(hipEvent_t* start, hipEvent_t* stop) {
  if (t_slot < 0 || t_role < 0 || t_role >= HKMOE_TIMING_ROLES) return false;
  const size_t i = static_cast<size_t>(t_slot) * HKMOE_TIMING_ROLES + t_role;
  *start = g_timing.ev[2 * i];
  *stop = g_timing.ev[2 * i + 1];
  g_timing.used[i] = 1;
  if (g_timing.first[t_slot] < 0) g_timing.first[t_slot] = t_role;
  g_timing.last[t_slot] = t_role;
  return true;
}

// Every kernel of the layer entry points goes through here.
template <typename... Kargs, typename... Args>
void hk_launch(void (*kern)(Kargs...), dim3 grid, dim3 block, uint32_t lds, hipStream_t stream, Args... args) {
  hipEvent_t a, b;
  if (timing_events(&a, &b))
    hipExtLaunchKernelGGL(kern, grid, block, lds, stream, a, b, 0u, static_cast<Kargs>(args)...);
  else
    hipLaunchKernelGGL(kern, grid, block, lds, stream, static_cast<Kargs>(args)...);
}

// Marks the launches of one layer call as timed (a set of the ring) for its
// lifetime; does nothing while timing is off or on another device.  A timed
// call holds the timing mutex until it has enqueued its last launch, so
// timing_events never sees the ring replaced by a concurrent
// hkmoe_kernel_timing, and timed calls from several host threads take their
// sets one after the other.
struct TimedCall {
  bool on = false;
  std::unique_lock<std::mutex> lk;
  TimedCall() : lk(g_timing_mu) {
    int dev = -1;
    if (g_timing.calls <= 0 || hipGetDevice(&dev) != hipSuccess || dev != g_timing.device) {
      lk.unlock();
      return;
    }
    t_slot = g_timing.next;
    g_timing.next = (g_timing.next + 1) % g_timing.calls;
    std::fill_n(g_timing.used.begin() + static_cast<size_t>(t_slot) * HKMOE_TIMING_ROLES, HKMOE_TIMING_ROLES, 0);
    g_timing.first[t_slot] = g_timing.last[t_slot] = -1;
    on = true;
  }
  ~TimedCall() {
    if (on) t_slot = -1;
    t_role = -1;
  }
};

#define HK_REQUIRE(cond, ...)                                 \
  do {                                                        \
    if (!(cond)) return fail(HKMOE_ERR_INVALID_ARGUMENT, __VA_ARGS__); \
  } while (0)

#define HK_TRY(expr)               \
  do {                             \
    const int _rc = (expr);        \
    if (_rc != HKMOE_OK) return _rc; \
  } while (0)

constexpr int kMaxDevices = 64;

int device_cus() {
  static int cus[kMaxDevices] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

int route_blocks(int64_t t) { return static_cast<int>((t + kRouteTok - 1) / kRouteTok); }

template <Epi EPI, Scale SC>
int launch_gemm(GemmParams p, hipStream_t stream, int grid_override = 0) {
  p.a_bytes = static_cast<uint32_t>(std::min<int64_t>(p.a_rows * p.K, 0xffffffffll));
  static bool attr_set[kMaxDevices] = {false};
  int dev = 0;
  (void)hipGetDevice(&dev);
  auto kern = gemm_fp8_persistent<EPI, SC>;
  if (dev >= 0 && dev < kMaxDevices && !attr_set[dev]) {
    const hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    if (err != hipSuccess) return fail(HKMOE_ERR_HIP, "hipFuncSetAttribute: %s", hipGetErrorString(err));
    attr_set[dev] = true;
  }
  const int grid = grid_override > 0 ? grid_override : device_cus();
  hk_launch(kern, dim3(grid), dim3(kThreads), kLdsBytes, stream, p);
  return check_launch("gemm_fp8_persistent");
}

// MFMA shape of the 128x128-tile dense kernel (hkmoe_set_dense_mfma): 16 or 32.
// 32x32x64 is the default: 2048^3 runs in 14.0 vs 15.1 us, 1024x4096x4096 in
// 23.2 vs 24.7 us, 4096x2048x1024 in 16.8 vs 17.1 us (graph-replayed launches,
// rotating operand copies, best of three interleaved rounds on one box).
std::atomic<int> g_dense_mfma{32};

// The dense GEMM on 128x128 tiles (gemm_small.hpp): one workgroup per tile,
// the grid a whole number of 4x8 tile blocks.
template <bool F32OUT, bool M32>
int launch_gemm_small(const SmallGemmParams& p, hipStream_t stream) {
  static bool attr_set[kMaxDevices] = {false};
  int dev = 0;
  (void)hipGetDevice(&dev);
  auto kern = gemm_fp8_small<F32OUT, M32>;
  if (dev >= 0 && dev < kMaxDevices && !attr_set[dev]) {
    const hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, kSmLdsBytes);
    if (err != hipSuccess) return fail(HKMOE_ERR_HIP, "hipFuncSetAttribute: %s", hipGetErrorString(err));
    attr_set[dev] = true;
  }
  const int grid = ((p.m_tiles + 3) / 4) * p.nbn * 32;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kSmThreads), kSmLdsBytes, stream, p);
  return check_launch("gemm_fp8_small");
}

// Prefetch depth of the narrow kernel for K / 128 steps: the largest of 8, 4,
// 2 that divides the step count (0: the narrow path cannot run this K: an odd
// step count, or more than 64 steps).
int narrow_depth(int k_steps) {
  if (k_steps > kNarrowMaxSteps) return 0;  // an item's scales must fit one LDS buffer
  return k_steps % 8 == 0 ? 8 : k_steps % 4 == 0 ? 4 : k_steps % 2 == 0 ? 2 : 0;
}

template <Epi EPI, int P>
int launch_narrow_p(const GemmParams& p, hipStream_t stream, int grid) {
  static bool attr_set[kMaxDevices] = {false};
  int dev = 0;
  (void)hipGetDevice(&dev);
  auto kern = gemm_fp8_narrow<EPI, P>;
  constexpr int lds = narrow_lds_bytes(P);
  if (dev >= 0 && dev < kMaxDevices && !attr_set[dev]) {
    const hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (err != hipSuccess) return fail(HKMOE_ERR_HIP, "hipFuncSetAttribute: %s", hipGetErrorString(err));
    attr_set[dev] = true;
  }
  hk_launch(kern, dim3(grid), dim3(kThreads), lds, stream, p);
  return check_launch("gemm_fp8_narrow");
}

template <Epi EPI>
int launch_narrow(GemmParams p, hipStream_t stream, int grid) {
  p.a_bytes = static_cast<uint32_t>(std::min<int64_t>(p.a_rows * p.K, 0xffffffffll));
  switch (narrow_depth(p.K / kBK)) {
    case 8: return launch_narrow_p<EPI, 8>(p, stream, grid);
    case 4: return launch_narrow_p<EPI, 4>(p, stream, grid);
    case 2: return launch_narrow_p<EPI, 2>(p, stream, grid);
    default: return fail(HKMOE_ERR_INVALID_ARGUMENT, "narrow GEMM: K=%d has an odd number of 128 steps", p.K);
  }
}

// Narrow path settings, read once from the environment:
//   HKMOE_NARROW_CUS   workgroups (CUs) of the narrow kernels, 0 = off (default 64)
//   HKMOE_NARROW_MAX   largest expert (rows) the narrow kernel takes, <= 64 (default 64)
//   HKMOE_NARROW_SHARE 1: the first wide GEMM leaves those CUs to the narrow
//                      kernel while it has work; 0: it keeps them (default 1).  A
//                      wide GEMM that keeps every CU takes them first, and the
//                      narrow kernel then mostly runs after it.
// hkmoe_set_narrow overrides them.
struct NarrowConfig {
  int cus, max_rows, share;
};
int env_int(const char* name, int dflt) {
  const char* v = std::getenv(name);
  return (v && *v) ? std::atoi(v) : dflt;
}
std::mutex g_narrow_mu;
NarrowConfig& narrow_config_ref() {
  static NarrowConfig cfg = [] {
    NarrowConfig c;
    c.cus = std::max(0, env_int("HKMOE_NARROW_CUS", 64));
    c.max_rows = std::min(kNarrowRows, std::max(0, env_int("HKMOE_NARROW_MAX", kNarrowRows)));
    c.share = std::min(2, std::max(0, env_int("HKMOE_NARROW_SHARE", 1)));
    return c;
  }();
  return cfg;
}
NarrowConfig narrow_config() {
  std::lock_guard<std::mutex> g(g_narrow_mu);
  return narrow_config_ref();
}

// Tile blocks of the grouped GEMMs: 2^b M tiles x 32 / 2^b N tiles share an
// XCD's L2.  2^b = HKMOE_BLOCK_M1 (GEMM 1) / HKMOE_BLOCK_M2 (GEMM 2) from the
// environment (1, 2, 4, 8, 16 or 32; read once; other values give the
// default), default 2 M tiles x 16 N tiles: a block then spans one or two
// experts, whose N tiles share the A rows.  A measurement knob for the L2-miss
// traffic of other block shapes.
int block_m_log2(int gemm) {
  static const int b1 = [] {
    const int m = env_int("HKMOE_BLOCK_M1", 2);
    for (int t = 0; t <= 5; ++t)
      if (m == (1 << t)) return t;
    return 1;
  }();
  static const int b2 = [] {
    const int m = env_int("HKMOE_BLOCK_M2", 2);
    for (int t = 0; t <= 5; ++t)
      if (m == (1 << t)) return t;
    return 1;
  }();
  return gemm == 1 ? b1 : b2;
}

// Per-device auxiliary stream (default priority, non-blocking) and fork/join
// events of the one-call layer.  Created on the first call that is not being
// captured into a graph; the mutex keeps fork/join sequences of concurrent
// host threads from interleaving on the shared events.
struct AuxStreams {
  hipStream_t aux = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
  bool ok = false;
};
std::mutex g_aux_mu;
AuxStreams g_aux[kMaxDevices];

int get_aux(hipStream_t main_stream, AuxStreams** out) {
  *out = nullptr;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return HKMOE_OK;
  AuxStreams& a = g_aux[dev];
  if (!a.ok) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(main_stream, &st) != hipSuccess || st != hipStreamCaptureStatusNone)
      return HKMOE_OK;  // no set-up under capture: this call runs without the narrow path
    if (hipStreamCreateWithFlags(&a.aux, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&a.fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&a.join, hipEventDisableTiming) != hipSuccess)
      return fail(HKMOE_ERR_HIP, "moe_forward: cannot create the auxiliary stream / events");
    a.ok = true;
  }
  *out = &a;
  return HKMOE_OK;
}

// The allocation-free layer's workspace: one array per device, created with
// the code object, held until the process ends.  In host code `scratch` names
// a host-side stand-in: its device address (different on every GPU) comes from
// hipGetSymbolAddress, looked up once per device on the first call with that
// device current, and only that address is passed to kernels.
constexpr size_t kScratchBytes = HKMOE_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_ptr(void** out) {
  *out = nullptr;
  int dev = 0;
  const hipError_t gerr = hipGetDevice(&dev);
  if (gerr != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(HKMOE_ERR_HIP, "moe_forward_noalloc: no usable current device (%s)", hipGetErrorString(gerr));
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || p == nullptr)
      return fail(HKMOE_ERR_HIP, "moe_forward_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                  hipGetErrorString(err));
    if ((reinterpret_cast<uintptr_t>(p) & 255) != 0)
      return fail(HKMOE_ERR_HIP, "moe_forward_noalloc: scratch of device %d is not 256-byte aligned", dev);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return HKMOE_OK;
}

// Workgroups the narrow kernels may take while 256x256 tiles exist: at most
// three quarters of the CUs, so the first 256x256 GEMM keeps at least a quarter
// of them whatever hkmoe_set_narrow asked for.
int narrow_cus_limit(int cus) { return std::min(cus, device_cus() - device_cus() / 4); }

// Joins the auxiliary stream back into the caller's stream when it goes out of
// scope, unless disarmed: every exit path after the fork (errors included)
// leaves the caller's stream ordered after the narrow kernels, which read and
// write the workspace, and a capture with the auxiliary stream joined.
struct AuxJoin {
  AuxStreams* a;
  hipStream_t s;
  bool armed = true;
  ~AuxJoin() {
    if (armed) {
      (void)hipEventRecord(a->join, a->aux);
      (void)hipStreamWaitEvent(s, a->join, 0);
    }
  }
};

int launch_expert_offsets(const int32_t* block_counts, int64_t num_tokens, int32_t num_experts,
                          int32_t* counts, int32_t* offsets, int32_t* block_base,
                          int32_t* mtile_offsets, int32_t* mtile_list, float* amax_reset,
                          int32_t* tile_counters, int narrow_max, int32_t* narrow_info,
                          hipStream_t stream) {
  const int nblk = route_blocks(num_tokens);
  // few routing blocks: expert_offsets_kernel also does the block scan (one
  // launch instead of two; ~6 us less on a decode step's critical path)
  const bool fuse = nblk <= kOffFuseBlocks;
  if (!fuse) {
    const bool timed = t_role == HKMOE_TIMING_OFFSETS;
    if (timed) t_role = HKMOE_TIMING_BLOCK_SCAN;
    hk_launch(expert_block_scan_kernel, dim3((num_experts + kOffExperts - 1) / kOffExperts),
              dim3(kScanThreads), 0, stream, block_counts, nblk, num_experts, counts, block_base);
    HK_TRY(check_launch("expert_block_scan_kernel"));
    if (timed) t_role = HKMOE_TIMING_OFFSETS;
  }
  hk_launch(expert_offsets_kernel, dim3(1), dim3(kScanThreads), 0, stream, num_experts, counts, offsets,
            mtile_offsets, mtile_list, kBM, amax_reset, tile_counters, narrow_max, narrow_info,
            block_counts, fuse ? nblk : -1, block_base);
  return check_launch("expert_offsets_kernel");
}


}  // namespace

extern "C" {

int hkmoe_version(void) { return 200; }

int hkmoe_set_narrow(int32_t cus, int32_t max_rows, int32_t wide_share) {
  HK_REQUIRE(cus >= 0 && cus <= 4096, "set_narrow: cus=%d outside [0, 4096]", cus);
  HK_REQUIRE(max_rows >= 0 && max_rows <= kNarrowRows, "set_narrow: max_rows=%d outside [0, %d]", max_rows,
             kNarrowRows);
  HK_REQUIRE(wide_share >= 0 && wide_share <= 2, "set_narrow: wide_share=%d outside [0, 2]", wide_share);
  std::lock_guard<std::mutex> g(g_narrow_mu);
  NarrowConfig& c = narrow_config_ref();
  c.cus = cus;
  c.max_rows = max_rows;
  c.share = wide_share;
  return HKMOE_OK;
}

int hkmoe_get_narrow(int32_t* cus, int32_t* max_rows, int32_t* wide_share) {
  HK_REQUIRE(cus && max_rows && wide_share, "get_narrow: null pointer");
  const NarrowConfig c = narrow_config();
  *cus = c.cus;
  *max_rows = c.max_rows;
  *wide_share = c.share;
  return HKMOE_OK;
}

const char* hkmoe_last_error(void) { return g_last_error.c_str(); }

int hkmoe_set_dense_mfma(int32_t shape) {
  HK_REQUIRE(shape == 16 || shape == 32, "set_dense_mfma: shape=%d must be 16 or 32", shape);
  g_dense_mfma.store(shape);
  return HKMOE_OK;
}

int hkmoe_get_dense_mfma(void) { return g_dense_mfma.load(); }

int hkmoe_gemm_fp8(const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t k,
                   const float* scale_a, const float* scale_b, int out_dtype, hkmoe_stream_t stream) {
  HK_REQUIRE(b && (m == 0 || (a && c)), "gemm_fp8: null tensor pointer");
  HK_REQUIRE(m >= 0 && n > 0 && k > 0, "gemm_fp8: bad shape M=%lld N=%lld K=%lld", (long long)m,
             (long long)n, (long long)k);
  HK_REQUIRE(k % 128 == 0, "gemm_fp8: K=%lld must be a multiple of 128", (long long)k);
  HK_REQUIRE(n % kBN == 0, "gemm_fp8: N=%lld must be a multiple of 256", (long long)n);
  HK_REQUIRE(k <= (1 << 20) && n * k < (1ll << 32) && m * k < (1ll << 32) && m < (1ll << 31),
             "gemm_fp8: operand too large for 32-bit buffer offsets (M*K and N*K must be < 2^32)");
  HK_REQUIRE(out_dtype == HKMOE_BF16 || out_dtype == HKMOE_F32, "gemm_fp8: bad out_dtype %d", out_dtype);
  if (m == 0) return HKMOE_OK;
  auto s = static_cast<hipStream_t>(stream);
  // Fewer 256x256 tiles than two per CU: 128x128 tiles, one workgroup each.
  if (((m + kBM - 1) / kBM) * (n / kBN) < 2ll * device_cus()) {
    SmallGemmParams q{};
    q.a = static_cast<const uint8_t*>(a);
    q.b = static_cast<const uint8_t*>(b);
    q.c = c;
    q.a_scale = scale_a;
    q.b_scale = scale_b;
    q.m = static_cast<int32_t>(m);
    q.n = static_cast<int32_t>(n);
    q.k = static_cast<int32_t>(k);
    q.a_bytes = static_cast<uint32_t>(std::min<int64_t>(m * k, 0xffffffffll));
    q.b_bytes = static_cast<uint32_t>(std::min<int64_t>(n * k, 0xffffffffll));
    q.m_tiles = static_cast<int32_t>((m + kSmTile - 1) / kSmTile);
    q.n_tiles = static_cast<int32_t>(n / kSmTile);
    q.nbn = (q.n_tiles + 7) / 8;
    if (g_dense_mfma.load() == 32)
      return out_dtype == HKMOE_BF16 ? launch_gemm_small<false, true>(q, s) : launch_gemm_small<true, true>(q, s);
    return out_dtype == HKMOE_BF16 ? launch_gemm_small<false, false>(q, s) : launch_gemm_small<true, false>(q, s);
  }
  GemmParams p{};
  p.a = static_cast<const uint8_t*>(a);
  p.b = static_cast<const uint8_t*>(b);
  p.c = c;
  p.a_scale = scale_a;
  p.b_scale = scale_b;
  p.rows = m;
  p.a_rows = m;
  p.num_experts = 1;
  p.K = static_cast<int32_t>(k);
  p.nb = static_cast<int32_t>(n);
  p.n_out = static_cast<int32_t>(n);
  p.n_tiles = static_cast<int32_t>(n / kBN);
  p.blk_m_log2 = 2;  // 4 x 8 tile blocks
  return out_dtype == HKMOE_BF16 ? launch_gemm<Epi::kStoreBf16, Scale::kTensor>(p, s)
                                 : launch_gemm<Epi::kStoreF32, Scale::kTensor>(p, s);
}

int hkmoe_route_blocks(int64_t num_tokens) { return route_blocks(num_tokens); }

int hkmoe_route_topk(const float* logits, int64_t num_tokens, int32_t num_experts, int32_t top_k,
                     int32_t* topk_idx, float* topk_w, int32_t* block_counts, hkmoe_stream_t stream) {
  HK_REQUIRE(num_tokens == 0 || (logits && topk_idx && topk_w && block_counts), "route_topk: null pointer");
  HK_REQUIRE(num_tokens >= 0 && num_tokens < (1ll << 31) / kMaxTopK, "route_topk: bad T=%lld",
             (long long)num_tokens);
  HK_REQUIRE(num_experts >= 1 && num_experts <= kMaxExperts, "route_topk: E=%d outside [1, %d]",
             num_experts, kMaxExperts);
  HK_REQUIRE(top_k >= 1 && top_k <= num_experts && top_k <= kMaxTopK,
             "route_topk: top_k=%d outside [1, min(E, %d)]", top_k, kMaxTopK);
  if (num_tokens == 0) return HKMOE_OK;
  const int per_lane = (num_experts + 15) / 16;  // experts per lane of a token's 16-lane row
  auto kern = per_lane <= 1 ? route_topk_kernel<1> : per_lane <= 2 ? route_topk_kernel<2>
            : per_lane <= 4 ? route_topk_kernel<4> : per_lane <= 8 ? route_topk_kernel<8>
            : per_lane <= 16 ? route_topk_kernel<16> : per_lane <= 32 ? route_topk_kernel<32>
                             : route_topk_kernel<64>;
  hk_launch(kern, dim3(route_blocks(num_tokens)), dim3(kTopkThreads), 0, static_cast<hipStream_t>(stream), logits,
            static_cast<int>(num_tokens), num_experts, top_k, topk_idx, topk_w, block_counts);
  return check_launch("route_topk_kernel");
}

int hkmoe_expert_offsets(const int32_t* block_counts, int64_t num_tokens, int32_t num_experts,
                         int32_t* counts, int32_t* offsets, int32_t* block_base,
                         int32_t* mtile_offsets, int32_t* mtile_list, float* amax_reset,
                         int32_t* tile_counters, hkmoe_stream_t stream) {
  HK_REQUIRE(counts && offsets && mtile_offsets && (num_tokens == 0 || block_base), "expert_offsets: null pointer");
  HK_REQUIRE(num_experts >= 1 && num_experts <= kMaxExperts, "expert_offsets: E=%d outside [1, %d]",
             num_experts, kMaxExperts);
  HK_REQUIRE(num_tokens >= 0, "expert_offsets: bad T");
  HK_REQUIRE(num_tokens == 0 || block_counts, "expert_offsets: null block_counts");
  return launch_expert_offsets(block_counts, num_tokens, num_experts, counts, offsets, block_base,
                               mtile_offsets, mtile_list, amax_reset, tile_counters, 0, nullptr,
                               static_cast<hipStream_t>(stream));
}

int hkmoe_expert_offsets_narrow(const int32_t* block_counts, int64_t num_tokens, int32_t num_experts,
                                int32_t* counts, int32_t* offsets, int32_t* block_base,
                                int32_t* mtile_offsets, int32_t* mtile_list, float* amax_reset,
                                int32_t* tile_counters, int32_t narrow_max, int32_t* narrow_info,
                                hkmoe_stream_t stream) {
  HK_REQUIRE(counts && offsets && mtile_offsets && mtile_list && narrow_info && (num_tokens == 0 || block_base),
             "expert_offsets_narrow: null pointer");
  HK_REQUIRE(num_experts >= 1 && num_experts <= kMaxExperts, "expert_offsets_narrow: E=%d outside [1, %d]",
             num_experts, kMaxExperts);
  HK_REQUIRE(num_tokens >= 0, "expert_offsets_narrow: bad T");
  HK_REQUIRE(num_tokens == 0 || block_counts, "expert_offsets_narrow: null block_counts");
  HK_REQUIRE(narrow_max >= 0 && narrow_max <= kNarrowRows, "expert_offsets_narrow: narrow_max=%d outside [0, %d]",
             narrow_max, kNarrowRows);
  return launch_expert_offsets(block_counts, num_tokens, num_experts, counts, offsets, block_base,
                               mtile_offsets, mtile_list, amax_reset, tile_counters, narrow_max, narrow_info,
                               static_cast<hipStream_t>(stream));
}

int hkmoe_scatter(const int32_t* topk_idx, int64_t num_tokens, int32_t num_experts, int32_t top_k,
                  const int32_t* offsets, const int32_t* block_base, int32_t* perm, int32_t* inv_perm,
                  const void* x_q, const float* x_scale, int64_t hidden, int scale_mode, void* xp,
                  float* xp_scale_t, hkmoe_stream_t stream) {
  HK_REQUIRE(num_tokens == 0 || (topk_idx && offsets && block_base && perm && inv_perm), "scatter: null pointer");
  HK_REQUIRE(num_experts >= 1 && num_experts <= kMaxExperts, "scatter: E=%d outside [1, %d]",
             num_experts, kMaxExperts);
  HK_REQUIRE(top_k >= 1 && top_k <= num_experts && top_k <= kMaxTopK, "scatter: bad top_k=%d", top_k);
  HK_REQUIRE(num_tokens >= 0, "scatter: bad T");
  HK_REQUIRE(scale_mode == HKMOE_SCALE_TENSOR || scale_mode == HKMOE_SCALE_BLOCK,
             "scatter: bad scale_mode %d", scale_mode);
  if (x_q != nullptr) {
    HK_REQUIRE(xp != nullptr, "scatter: x_q given without xp");
    HK_REQUIRE(hidden > 0 && hidden % 16 == 0, "scatter: hidden=%lld must be a multiple of 16",
               (long long)hidden);
    if (scale_mode == HKMOE_SCALE_BLOCK) {
      HK_REQUIRE(hidden % kGroup == 0, "scatter: hidden must be a multiple of 128 for block scales");
      HK_REQUIRE(x_scale && xp_scale_t, "scatter: block scales need x_scale and xp_scale_t");
    }
  }
  if (num_tokens == 0) return HKMOE_OK;
  hk_launch(scatter_kernel, dim3(route_blocks(num_tokens)), dim3(kRouteThreads), 0,
                     static_cast<hipStream_t>(stream), topk_idx, static_cast<int>(num_tokens),
                     num_experts, top_k, offsets, block_base, perm, inv_perm,
                     static_cast<const uint8_t*>(x_q), x_scale, hidden,
                     scale_mode == HKMOE_SCALE_BLOCK ? 1 : 0, static_cast<uint8_t*>(xp), xp_scale_t,
                     num_tokens * top_k);
  return check_launch("scatter_kernel");
}

// narrow_cnt: skip (wide kernel) the list's last *narrow_cnt M tiles, and with
// yield_from > 0 leave CUs >= yield_from to the narrow kernel when it has work;
// narrow_active > 0: run the narrow kernel on exactly those tiles instead (one
// workgroup per CU; narrow_active of them while 256x256 tiles exist).
static int grouped_gemm1_impl(const void* x, const float* x_scale, const int32_t* gather,
                              int32_t gather_div, int64_t x_rows, const void* w13, const float* w13_scale,
                              const int32_t* offsets, const int32_t* mtile_offsets,
                              const int32_t* mtile_list, int64_t rows,
                              int32_t num_experts, int32_t hidden, int32_t inter, int scale_mode,
                              int w_layout, int out_format, void* h, float* h_aux,
                              int32_t* tile_counters, hkmoe_stream_t stream,
                              const int32_t* narrow_cnt, int yield_from, int narrow_active,
                              int narrow_grid = 0) {
  HK_REQUIRE(w13 && w13_scale && offsets && mtile_offsets, "grouped_gemm1: null pointer");
  HK_REQUIRE(rows == 0 || (x && x_scale && h), "grouped_gemm1: null pointer");
  HK_REQUIRE(num_experts >= 1 && num_experts <= kMaxExperts, "grouped_gemm1: bad E=%d", num_experts);
  HK_REQUIRE(hidden > 0 && hidden % kGroup == 0 && hidden <= kGroup * kMaxKBlocks,
             "grouped_gemm1: hidden=%d must be a multiple of 128 and <= %d", hidden, kGroup * kMaxKBlocks);
  HK_REQUIRE(inter > 0 && inter % 128 == 0, "grouped_gemm1: inter=%d must be a multiple of 128", inter);
  HK_REQUIRE(rows >= 0 && rows < (1ll << 31), "grouped_gemm1: bad rows");
  HK_REQUIRE(x_rows >= (rows > 0 ? 1 : 0) && x_rows * hidden < (1ll << 32), "grouped_gemm1: x_rows=%lld out of range",
             (long long)x_rows);
  HK_REQUIRE(gather == nullptr || gather_div >= 1, "grouped_gemm1: gather_div must be >= 1");
  HK_REQUIRE(gather != nullptr || x_rows >= rows, "grouped_gemm1: x has fewer rows than rows");
  HK_REQUIRE(2ll * inter * hidden < (1ll << 32), "grouped_gemm1: expert weight too large");
  HK_REQUIRE(scale_mode == HKMOE_SCALE_TENSOR || scale_mode == HKMOE_SCALE_BLOCK,
             "grouped_gemm1: bad scale_mode %d", scale_mode);
  HK_REQUIRE(w_layout == HKMOE_W_ROWS || w_layout == HKMOE_W_PACKED, "grouped_gemm1: bad w_layout %d",
             w_layout);
  HK_REQUIRE(out_format == HKMOE_BF16 || (out_format == HKMOE_E4M3 && scale_mode == HKMOE_SCALE_BLOCK),
             "grouped_gemm1: out_format %d not supported with scale_mode %d", out_format, scale_mode);
  HK_REQUIRE(out_format != HKMOE_E4M3 || rows == 0 || h_aux != nullptr, "grouped_gemm1: e4m3 output needs h_aux scales");
  if (rows == 0) return HKMOE_OK;
  GemmParams p{};
  p.a = static_cast<const uint8_t*>(x);
  p.a_gather = gather;
  p.gather_div = gather ? gather_div : 1;
  p.b = static_cast<const uint8_t*>(w13);
  p.c = h;
  p.a_scale = x_scale;
  p.b_scale = w13_scale;
  p.offsets = offsets;
  p.mtile_offsets = mtile_offsets;
  p.rows = rows;
  p.a_rows = x_rows;
  p.as_rs = hidden / kGroup;  // x_scale is row-major [x_rows, H/128]
  p.as_ks = 1;
  p.num_experts = num_experts;
  p.K = hidden;
  p.nb = 2 * inter;
  p.n_out = inter;
  p.n_tiles = inter / 128;
  p.b_packed = w_layout == HKMOE_W_PACKED;
  p.mtile_list = mtile_list;
  p.blk_m_log2 = block_m_log2(1);  // 2 x 16 tile blocks by default
  p.tile_ctr = tile_counters;
  p.narrow_cnt = narrow_cnt;
  p.yield_from = yield_from;
  p.narrow_active = narrow_active;
  auto s = static_cast<hipStream_t>(stream);
  if (narrow_active > 0) {
    if (scale_mode != HKMOE_SCALE_BLOCK || out_format != HKMOE_E4M3 || narrow_cnt == nullptr ||
        mtile_list == nullptr || tile_counters == nullptr)
      return fail(HKMOE_ERR_INVALID_ARGUMENT, "grouped_gemm1: the narrow kernel needs block scales, "
                                              "e4m3 output, the M-tile list and an item counter");
    p.c_scale = h_aux;
    return launch_narrow<Epi::kSiluQuant>(p, s, narrow_grid > 0 ? narrow_grid : narrow_active);
  }
  if (scale_mode == HKMOE_SCALE_TENSOR) {
    p.amax = h_aux;
    return launch_gemm<Epi::kSiluBf16, Scale::kTensor>(p, s);
  }
  if (out_format == HKMOE_E4M3) {
    p.c_scale = h_aux;
    return launch_gemm<Epi::kSiluQuant, Scale::kBlock>(p, s, yield_from < 0 ? narrow_grid : 0);
  }
  return launch_gemm<Epi::kSiluBf16, Scale::kBlock>(p, s);
}

int hkmoe_grouped_gemm1(const void* x, const float* x_scale, const int32_t* gather,
                        int32_t gather_div, int64_t x_rows, const void* w13, const float* w13_scale,
                        const int32_t* offsets, const int32_t* mtile_offsets,
                        const int32_t* mtile_list, int64_t rows,
                        int32_t num_experts, int32_t hidden, int32_t inter, int scale_mode,
                        int w_layout, int out_format, void* h, float* h_aux,
                        int32_t* tile_counters, hkmoe_stream_t stream) {
  return grouped_gemm1_impl(x, x_scale, gather, gather_div, x_rows, w13, w13_scale, offsets,
                            mtile_offsets, mtile_list, rows, num_experts, hidden, inter, scale_mode,
                            w_layout, out_format, h, h_aux, tile_counters, stream, nullptr, 0, 0);
}

int hkmoe_requant(const void* h, int64_t rows, int32_t inter, int scale_mode, const float* amax,
                  void* hq, float* hs, hkmoe_stream_t stream) {
  HK_REQUIRE(inter > 0 && inter % 128 == 0, "requant: inter=%d must be a multiple of 128", inter);
  HK_REQUIRE(rows >= 0, "requant: bad rows");
  // rows == 0: h and hq are empty; block scales hs too, a tensor scale is still written
  HK_REQUIRE(rows == 0 || (h && hq), "requant: null pointer");
  HK_REQUIRE(hs || (rows == 0 && scale_mode == HKMOE_SCALE_BLOCK), "requant: null pointer");
  auto s = static_cast<hipStream_t>(stream);
  if (scale_mode == HKMOE_SCALE_BLOCK) {
    if (rows == 0) return HKMOE_OK;
    HK_REQUIRE(rows < (1ll << 31), "requant: too many rows");
    hk_launch(requant_group_kernel, dim3(static_cast<unsigned>(rows)), dim3(256), 0, s,
                       static_cast<const uint16_t*>(h), rows, inter, static_cast<uint8_t*>(hq), hs);
    return check_launch("requant_group_kernel");
  }
  HK_REQUIRE(scale_mode == HKMOE_SCALE_TENSOR, "requant: bad scale_mode %d", scale_mode);
  HK_REQUIRE(amax != nullptr, "requant: per-tensor mode needs amax");
  const int64_t n8 = rows * inter / 8;
  const int grid = static_cast<int>(std::min<int64_t>(std::max<int64_t>(1, (n8 + 255) / 256), 4 * 1024));
  hk_launch(requant_tensor_kernel, dim3(grid), dim3(256), 0, s,
                     static_cast<const uint16_t*>(h), n8, amax, static_cast<uint8_t*>(hq), hs);
  return check_launch("requant_tensor_kernel");
}

static int grouped_gemm2_impl(const void* hq, const float* hs, const void* w2, const float* w2_scale,
                              const int32_t* offsets, const int32_t* mtile_offsets,
                              const int32_t* mtile_list, int64_t rows,
                              int32_t num_experts, int32_t hidden, int32_t inter, int scale_mode,
                              int w_layout, void* y, int32_t* tile_counters, hkmoe_stream_t stream,
                              const int32_t* narrow_cnt, int yield_from, int narrow_active,
                              int narrow_grid = 0) {
  HK_REQUIRE(w2 && w2_scale && offsets && mtile_offsets, "grouped_gemm2: null pointer");
  HK_REQUIRE(rows == 0 || (hq && hs && y), "grouped_gemm2: null pointer");
  HK_REQUIRE(num_experts >= 1 && num_experts <= kMaxExperts, "grouped_gemm2: bad E=%d", num_experts);
  HK_REQUIRE(hidden > 0 && hidden % kBN == 0, "grouped_gemm2: hidden=%d must be a multiple of 256", hidden);
  HK_REQUIRE(inter > 0 && inter % kGroup == 0 && inter <= kGroup * kMaxKBlocks,
             "grouped_gemm2: inter=%d must be a multiple of 128 and <= %d", inter, kGroup * kMaxKBlocks);
  HK_REQUIRE(rows >= 0 && rows < (1ll << 31), "grouped_gemm2: bad rows");
  HK_REQUIRE(rows * inter < (1ll << 32), "grouped_gemm2: rows*inter must be < 2^32 (32-bit buffer offsets into hq)");
  HK_REQUIRE(static_cast<int64_t>(hidden) * inter < (1ll << 32), "grouped_gemm2: expert weight too large");
  HK_REQUIRE(scale_mode == HKMOE_SCALE_TENSOR || scale_mode == HKMOE_SCALE_BLOCK,
             "grouped_gemm2: bad scale_mode %d", scale_mode);
  HK_REQUIRE(w_layout == HKMOE_W_ROWS || w_layout == HKMOE_W_PACKED, "grouped_gemm2: bad w_layout %d",
             w_layout);
  if (rows == 0) return HKMOE_OK;
  GemmParams p{};
  p.a = static_cast<const uint8_t*>(hq);
  p.b = static_cast<const uint8_t*>(w2);
  p.c = y;
  p.a_scale = hs;
  p.b_scale = w2_scale;
  p.offsets = offsets;
  p.mtile_offsets = mtile_offsets;
  p.rows = rows;
  p.a_rows = rows;
  p.as_rs = 1;  // group scales are transposed [I/128, rows]
  p.as_ks = rows;
  p.num_experts = num_experts;
  p.K = inter;
  p.nb = hidden;
  p.n_out = hidden;
  p.n_tiles = hidden / kBN;
  p.b_packed = w_layout == HKMOE_W_PACKED;
  p.mtile_list = mtile_list;
  p.blk_m_log2 = block_m_log2(2);  // 2 x 16 tile blocks by default
  p.tile_ctr = tile_counters;
  p.narrow_cnt = narrow_cnt;
  p.yield_from = yield_from;
  p.narrow_active = narrow_active;
  auto s = static_cast<hipStream_t>(stream);
  if (narrow_active > 0) {
    if (scale_mode != HKMOE_SCALE_BLOCK || narrow_cnt == nullptr || mtile_list == nullptr ||
        tile_counters == nullptr)
      return fail(HKMOE_ERR_INVALID_ARGUMENT, "grouped_gemm2: the narrow kernel needs block scales, "
                                              "the M-tile list and an item counter");
    return launch_narrow<Epi::kStoreBf16>(p, s, narrow_grid > 0 ? narrow_grid : narrow_active);
  }
  return scale_mode == HKMOE_SCALE_BLOCK ? launch_gemm<Epi::kStoreBf16, Scale::kBlock>(p, s)
                                         : launch_gemm<Epi::kStoreBf16, Scale::kTensor>(p, s);
}

int hkmoe_grouped_gemm2(const void* hq, const float* hs, const void* w2, const float* w2_scale,
                        const int32_t* offsets, const int32_t* mtile_offsets,
                        const int32_t* mtile_list, int64_t rows,
                        int32_t num_experts, int32_t hidden, int32_t inter, int scale_mode,
                        int w_layout, void* y, int32_t* tile_counters, hkmoe_stream_t stream) {
  return grouped_gemm2_impl(hq, hs, w2, w2_scale, offsets, mtile_offsets, mtile_list, rows, num_experts,
                            hidden, inter, scale_mode, w_layout, y, tile_counters, stream, nullptr, 0, 0);
}

int hkmoe_grouped_gemm1_part(const void* x, const float* x_scale, const int32_t* gather,
                             int32_t gather_div, int64_t x_rows, const void* w13, const float* w13_scale,
                             const int32_t* offsets, const int32_t* mtile_offsets,
                             const int32_t* mtile_list, int64_t rows, int32_t num_experts, int32_t hidden,
                             int32_t inter, int w_layout, void* hq, float* hs, int32_t* tile_counters,
                             const int32_t* narrow_info, int32_t part, int32_t grid, hkmoe_stream_t stream) {
  HK_REQUIRE(narrow_info && mtile_list, "grouped_gemm1_part: needs narrow_info and mtile_list");
  HK_REQUIRE(part == 0 || part == 1, "grouped_gemm1_part: part=%d must be 0 (wide) or 1 (narrow)", part);
  HK_REQUIRE(grid >= 0 && grid <= 65536, "grouped_gemm1_part: bad grid %d", grid);
  HK_REQUIRE(part == 0 || narrow_depth(hidden / kBK) > 0,
             "grouped_gemm1_part: the narrow kernel needs an even number of at most 64 128-wide K steps (H=%d)", hidden);
  if (part == 1) {
    // the narrow kernel's item counter: narrow_info[1], zeroed by hkmoe_expert_offsets_narrow
    return grouped_gemm1_impl(x, x_scale, gather, gather_div, x_rows, w13, w13_scale, offsets, mtile_offsets,
                              mtile_list, rows, num_experts, hidden, inter, HKMOE_SCALE_BLOCK, w_layout,
                              HKMOE_E4M3, hq, hs, const_cast<int32_t*>(narrow_info) + 1, stream, narrow_info, 0,
                              grid > 0 ? grid : device_cus(), device_cus());
  }
  return grouped_gemm1_impl(x, x_scale, gather, gather_div, x_rows, w13, w13_scale, offsets, mtile_offsets,
                            mtile_list, rows, num_experts, hidden, inter, HKMOE_SCALE_BLOCK, w_layout, HKMOE_E4M3,
                            hq, hs, tile_counters, stream, narrow_info, grid, 0);
}

int hkmoe_grouped_gemm2_part(const void* hq, const float* hs, const void* w2, const float* w2_scale,
                             const int32_t* offsets, const int32_t* mtile_offsets, const int32_t* mtile_list,
                             int64_t rows, int32_t num_experts, int32_t hidden, int32_t inter, int w_layout,
                             void* y, int32_t* tile_counters, const int32_t* narrow_info, int32_t part,
                             int32_t grid, hkmoe_stream_t stream) {
  HK_REQUIRE(narrow_info && mtile_list, "grouped_gemm2_part: needs narrow_info and mtile_list");
  HK_REQUIRE(part == 0 || part == 1, "grouped_gemm2_part: part=%d must be 0 (wide) or 1 (narrow)", part);
  HK_REQUIRE(grid >= 0 && grid <= 65536, "grouped_gemm2_part: bad grid %d", grid);
  HK_REQUIRE(part == 0 || narrow_depth(inter / kBK) > 0,
             "grouped_gemm2_part: the narrow kernel needs an even number of at most 64 128-wide K steps (I=%d)", inter);
  // the narrow kernel's item counter: narrow_info[2], zeroed by hkmoe_expert_offsets_narrow
  return grouped_gemm2_impl(hq, hs, w2, w2_scale, offsets, mtile_offsets, mtile_list, rows, num_experts, hidden,
                            inter, HKMOE_SCALE_BLOCK, w_layout, y,
                            part == 1 ? const_cast<int32_t*>(narrow_info) + 2 : tile_counters, stream,
                            narrow_info, part == 0 ? grid : 0, part == 1 ? (grid > 0 ? grid : device_cus()) : 0,
                            part == 1 ? device_cus() : 0);
}

int hkmoe_pack_weights(const void* w, int64_t num_experts, int64_t n, int64_t k, int32_t gate_up,
                       void* packed, hkmoe_stream_t stream) {
  HK_REQUIRE(w && packed, "pack_weights: null pointer");
  HK_REQUIRE(w != packed, "pack_weights: in-place packing is not supported");
  HK_REQUIRE(num_experts >= 0 && n > 0 && n % kBN == 0 && k > 0 && k % kBK == 0,
             "pack_weights: N=%lld must be a multiple of 256 and K=%lld of 128", (long long)n,
             (long long)k);
  HK_REQUIRE(n * k < (1ll << 32) && k <= kBK * kMaxKBlocks, "pack_weights: expert weight too large");
  HK_REQUIRE(gate_up == 0 || (gate_up > 0 && n == 2ll * gate_up),
             "pack_weights: gate_up=%d must be 0 or N/2", gate_up);
  const int64_t chunks = num_experts * n * k / 16;
  if (chunks == 0) return HKMOE_OK;
  const int grid = static_cast<int>(std::min<int64_t>((chunks + 255) / 256, 8 * 1024));
  hipLaunchKernelGGL(pack_weights_kernel, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint8_t*>(w), n, static_cast<int>(k), gate_up,
                     static_cast<uint8_t*>(packed), chunks);
  return check_launch("pack_weights_kernel");
}

int hkmoe_requant_quotient_check(int32_t* counts, hkmoe_stream_t stream) {
  HK_REQUIRE(counts, "requant_quotient_check: null pointer");
  hipLaunchKernelGGL(requant_quotient_check_kernel, dim3(128, 37 + 27 + 1), dim3(128), 0,
                     static_cast<hipStream_t>(stream), counts);
  return check_launch("requant_quotient_check_kernel");
}

int hkmoe_combine(const void* y, const float* topk_w, const int32_t* inv_perm, int64_t num_tokens,
                  int32_t top_k, int32_t hidden, void* out, hkmoe_stream_t stream) {
  HK_REQUIRE(num_tokens == 0 || (y && topk_w && inv_perm && out), "combine: null pointer");
  HK_REQUIRE(top_k >= 1 && top_k <= kMaxTopK, "combine: bad top_k=%d", top_k);
  HK_REQUIRE(hidden > 0 && hidden % 8 == 0, "combine: hidden=%d must be a multiple of 8", hidden);
  HK_REQUIRE(num_tokens >= 0 && num_tokens < (1ll << 31), "combine: bad T");
  if (num_tokens == 0) return HKMOE_OK;
  // the largest multiple of 64 threads (<= 512) that divides the row's 16-byte
  // chunks, so no workgroup ends on a partly idle pass (H = 7168: 448 threads
  // and two passes instead of 256 and a half-empty fourth); 256 otherwise
  const int chunks = hidden / 8;
  int threads = 256;
  for (int t = 512; t >= 64; t -= 64)
    if (chunks % t == 0) {
      threads = t;
      break;
    }
  hk_launch(combine_kernel, dim3(static_cast<unsigned>(num_tokens)), dim3(threads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(y), topk_w,
                     inv_perm, top_k, hidden, static_cast<uint16_t*>(out));
  return check_launch("combine_kernel");
}

// ---------------------------------------------------------------------------
// whole layer
// ---------------------------------------------------------------------------
namespace {
struct MoeWorkspace {
  int32_t* topk_idx;
  float* topk_w;
  int32_t* block_counts;
  int32_t* block_base;
  int32_t* counts;
  int32_t* offsets;
  int32_t* mtile_offsets;
  int32_t* mtile_list;  // [M tiles][2], at most ceil(T*k/256) + E tiles
  float* amax;
  int32_t* tile_ctr;  // HKMOE_TILE_COUNTERS
  int32_t* narrow_info;  // [0] narrow M tiles, [1] / [2] narrow item counters of GEMM 1 / 2,
                         // [3] / [4] their active-slot counters
  int32_t* perm;
  int32_t* inv_perm;
  uint16_t* h;   // per-tensor mode only: bf16 intermediate before requantisation
  uint8_t* hq;
  float* hs;     // block: group scales; MX: packed e8m0 words of hq [I/128][ws]
  uint32_t* xw;  // MX only: packed e8m0 words of the gathered x rows [H/128][ws]
  uint16_t* y;
  size_t bytes;
};

// Words per K step of the tile-aligned MX exponent layouts: every M tile
// (at most ceil(rows/256) + E of them) owns 256 words.
int64_t mx_words_per_step(int64_t rows, int32_t e) { return ((rows + kBM - 1) / kBM + e) * kBM; }

MoeWorkspace carve(uint8_t* base, int64_t t, int32_t e, int32_t k, int32_t hidden, int32_t inter,
                   int mode) {
  const bool block = mode == HKMOE_SCALE_BLOCK, mx = mode == HKMOE_SCALE_MX;
  MoeWorkspace w{};
  size_t off = 0;
  const int64_t r = t * k;
  const int64_t nblk = route_blocks(t);
  auto take = [&](size_t bytes) -> uint8_t* {
    uint8_t* p = base ? base + off : nullptr;
    off += align256(bytes);
    return p;
  };
  w.topk_idx = reinterpret_cast<int32_t*>(take(r * 4));
  w.topk_w = reinterpret_cast<float*>(take(r * 4));
  w.block_counts = reinterpret_cast<int32_t*>(take(nblk * e * 4));
  w.block_base = reinterpret_cast<int32_t*>(take(nblk * e * 4));
  w.counts = reinterpret_cast<int32_t*>(take(e * 4));
  w.offsets = reinterpret_cast<int32_t*>(take((e + 1) * 4));
  w.mtile_offsets = reinterpret_cast<int32_t*>(take((e + 1) * 4));
  w.mtile_list = reinterpret_cast<int32_t*>(take(((r + kBM - 1) / kBM + e) * 8));
  w.amax = reinterpret_cast<float*>(take(4));
  w.tile_ctr = reinterpret_cast<int32_t*>(take(HKMOE_TILE_COUNTERS * 4));
  w.narrow_info = reinterpret_cast<int32_t*>(take((1 + kNarrowCounters) * 4));  // HKMOE_NARROW_INFO ints
  w.perm = reinterpret_cast<int32_t*>(take(r * 4));
  w.inv_perm = reinterpret_cast<int32_t*>(take(r * 4));
  const int64_t ws = mx_words_per_step(r, e);
  w.h = (block || mx) ? nullptr : reinterpret_cast<uint16_t*>(take(r * inter * 2));
  w.hq = take(r * inter);
  w.hs = reinterpret_cast<float*>(take(block ? r * (inter / kGroup) * 4 : mx ? (inter / kGroup) * ws * 4 : 4));
  w.xw = mx ? reinterpret_cast<uint32_t*>(take((hidden / kGroup) * ws * 4)) : nullptr;
  w.y = reinterpret_cast<uint16_t*>(take(r * hidden * 2));
  w.bytes = off;
  return w;
}
}  // namespace

size_t hkmoe_moe_workspace_size(int64_t num_tokens, int32_t num_experts, int32_t top_k,
                                int32_t hidden, int32_t inter, int scale_mode) {
  if (num_tokens < 0 || num_experts < 1 || top_k < 1 || hidden < 1 || inter < 1) return 0;
  if (scale_mode != HKMOE_SCALE_TENSOR && scale_mode != HKMOE_SCALE_BLOCK && scale_mode != HKMOE_SCALE_MX)
    return 0;
  return carve(nullptr, num_tokens, num_experts, top_k, hidden, inter, scale_mode).bytes;
}

// The layer; aux_ok: the narrow path may fork to the library's auxiliary
// stream (else every kernel runs on `stream`: the one-stream narrow schedule
// where it applies, otherwise the 256x256 kernels alone).
static int moe_forward_impl(const void* x_q, const float* x_scale, const float* logits, const void* w13,
                            const float* w13_scale, const void* w2, const float* w2_scale,
                            int64_t num_tokens, int32_t num_experts, int32_t top_k, int32_t hidden,
                            int32_t inter, int scale_mode, int w_layout, void* out, void* workspace,
                            size_t workspace_bytes, hkmoe_stream_t stream, bool aux_ok) {
  // with no tokens the activations, the output and the workspace may be empty
  // (null); the weights and shapes are checked either way
  HK_REQUIRE(w13 && w13_scale && w2 && w2_scale, "moe_forward: null pointer");
  HK_REQUIRE(num_tokens == 0 || (x_q && x_scale && logits && out), "moe_forward: null pointer");
  HK_REQUIRE(scale_mode == HKMOE_SCALE_TENSOR || scale_mode == HKMOE_SCALE_BLOCK,
             "moe_forward: bad scale_mode %d", scale_mode);
  HK_REQUIRE(w_layout == HKMOE_W_ROWS || w_layout == HKMOE_W_PACKED, "moe_forward: bad w_layout %d",
             w_layout);
  HK_REQUIRE(num_tokens >= 0 && num_tokens * top_k < (1ll << 31), "moe_forward: bad T");
  HK_REQUIRE(num_experts >= 1 && num_experts <= kMaxExperts, "moe_forward: E=%d outside [1, %d]",
             num_experts, kMaxExperts);
  HK_REQUIRE(top_k >= 1 && top_k <= num_experts && top_k <= kMaxTopK, "moe_forward: bad top_k=%d", top_k);
  HK_REQUIRE(hidden > 0 && hidden % kBN == 0 && hidden <= kGroup * kMaxKBlocks,
             "moe_forward: hidden=%d must be a multiple of 256 and <= %d", hidden, kGroup * kMaxKBlocks);
  HK_REQUIRE(inter > 0 && inter % 128 == 0 && inter <= kGroup * kMaxKBlocks,
             "moe_forward: inter=%d must be a multiple of 128 and <= %d", inter, kGroup * kMaxKBlocks);
  // every operand of the grouped GEMMs is addressed by 32-bit buffer offsets:
  // checked here, before any kernel of the layer is launched
  HK_REQUIRE(2ll * inter * hidden < (1ll << 32), "moe_forward: expert weight too large (2*I*H must be < 2^32)");
  HK_REQUIRE(num_tokens * hidden < (1ll << 32) && num_tokens * top_k * inter < (1ll << 32),
             "moe_forward: T*H and T*k*I must be < 2^32 (32-bit buffer offsets)");
  if (num_tokens == 0) return HKMOE_OK;
  const bool block = scale_mode == HKMOE_SCALE_BLOCK;
  const MoeWorkspace need = carve(nullptr, num_tokens, num_experts, top_k, hidden, inter, scale_mode);
  if (workspace == nullptr || workspace_bytes < need.bytes)
    return fail(HKMOE_ERR_WORKSPACE, "moe_forward: workspace of %zu bytes needed, %zu given", need.bytes,
                workspace_bytes);
  HK_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255) == 0, "moe_forward: workspace must be 256-byte aligned");
  const MoeWorkspace w = carve(static_cast<uint8_t*>(workspace), num_tokens, num_experts, top_k,
                               hidden, inter, scale_mode);
  const int64_t rows = num_tokens * top_k;
  auto s = static_cast<hipStream_t>(stream);
  // Narrow path (block scales): experts of at most HKMOE_NARROW_MAX rows go to
  // the weight-streaming narrow kernels on an auxiliary stream, which run
  // beside the 256x256 kernels of the larger experts on the main stream.
  const NarrowConfig nc = narrow_config();
  const bool narrow_ok = block && nc.cus > 0 && nc.max_rows > 0 && narrow_depth(hidden / kBK) > 0 &&
                         narrow_depth(inter / kBK) > 0;
  // Up to 2*max_rows rows per expert on average (T*k <= 2*E*max_rows) the small
  // experts' weight stream dominates: the narrow kernels then run on `stream`
  // after the 256x256 ones, each on every CU, instead of on max. 3/4 of them
  // beside the 256x256 kernels, and without the fork to the auxiliary stream and
  // the join back (≈20 µs of cross-stream latency).  Measured on the config-3
  // shape (H=7168, I=2048, E=256, k=8): T=512 / 1024 / 2048 / 4096 run 26 / 21 /
  // 13 / 4% faster on one stream, T=6144 / 8192 10 / 8% slower.
  const bool narrow_seq = narrow_ok && rows <= 2 * static_cast<int64_t>(num_experts) * nc.max_rows;
  // the two-stream schedule needs the auxiliary stream; without it (aux_ok
  // false) such layers run the 256x256 kernels alone
  AuxStreams* aux = nullptr;
  if (aux_ok && narrow_ok && !narrow_seq) HK_TRY(get_aux(s, &aux));
  std::unique_lock<std::mutex> aux_lock(g_aux_mu, std::defer_lock);
  if (aux) aux_lock.lock();
  TimedCall timed_call;
  t_role = HKMOE_TIMING_ROUTE;
  HK_TRY(hkmoe_route_topk(logits, num_tokens, num_experts, top_k, w.topk_idx, w.topk_w,
                          w.block_counts, stream));
  t_role = HKMOE_TIMING_OFFSETS;
  HK_TRY(launch_expert_offsets(w.block_counts, num_tokens, num_experts, w.counts, w.offsets,
                               w.block_base, w.mtile_offsets, w.mtile_list, w.amax, w.tile_ctr,
                               (aux || narrow_seq) ? nc.max_rows : 0,
                               (aux || narrow_seq) ? w.narrow_info : nullptr, s));
  t_role = HKMOE_TIMING_SCATTER;
  HK_TRY(hkmoe_scatter(w.topk_idx, num_tokens, num_experts, top_k, w.offsets, w.block_base, w.perm,
                       w.inv_perm, nullptr, nullptr, hidden, scale_mode, nullptr, nullptr, stream));
  if (narrow_seq) {
    // one stream: each 256x256 GEMM keeps every CU (yield_from 0) and skips the
    // narrow experts' tiles; each narrow GEMM then runs its items on every CU.
    // A token's k experts are distinct, so no expert has more than T rows: with
    // T <= max_rows every expert is narrow, and the 256x256 GEMMs, which would
    // find no tile, are not launched.
    const int ngrid = device_cus();
    const bool wide = num_tokens > nc.max_rows;
    t_role = HKMOE_TIMING_GEMM1;
    if (wide)
      HK_TRY(grouped_gemm1_impl(x_q, x_scale, w.perm, top_k, num_tokens, w13, w13_scale, w.offsets,
                                w.mtile_offsets, w.mtile_list, rows, num_experts, hidden, inter, scale_mode,
                                w_layout, HKMOE_E4M3, w.hq, w.hs, w.tile_ctr, stream, w.narrow_info, 0, 0));
    t_role = HKMOE_TIMING_GEMM1_NARROW;
    HK_TRY(grouped_gemm1_impl(x_q, x_scale, w.perm, top_k, num_tokens, w13, w13_scale, w.offsets,
                              w.mtile_offsets, w.mtile_list, rows, num_experts, hidden, inter, scale_mode,
                              w_layout, HKMOE_E4M3, w.hq, w.hs, w.narrow_info + 1, stream, w.narrow_info, 0,
                              ngrid, ngrid));
    t_role = HKMOE_TIMING_GEMM2;
    if (wide)
      HK_TRY(grouped_gemm2_impl(w.hq, w.hs, w2, w2_scale, w.offsets, w.mtile_offsets, w.mtile_list, rows,
                                num_experts, hidden, inter, scale_mode, w_layout, w.y, w.tile_ctr + 8, stream,
                                w.narrow_info, 0, 0));
    t_role = HKMOE_TIMING_GEMM2_NARROW;
    HK_TRY(grouped_gemm2_impl(w.hq, w.hs, w2, w2_scale, w.offsets, w.mtile_offsets, w.mtile_list, rows,
                              num_experts, hidden, inter, scale_mode, w_layout, w.y, w.narrow_info + 2, stream,
                              w.narrow_info, 0, ngrid, ngrid));
    t_role = HKMOE_TIMING_COMBINE;
    HK_TRY(hkmoe_combine(w.y, w.topk_w, w.inv_perm, num_tokens, top_k, hidden, out, stream));
    return HKMOE_OK;
  }
  if (aux) {
    // fork: both GEMMs of the narrow experts on the auxiliary stream, enqueued
    // first so that their workgroups find free CUs; join before the combine
    const int ncus = narrow_cus_limit(nc.cus);
    // Which workgroups work is decided on the device from narrow_info: with
    // experts of both kinds the narrow kernels use ncus workgroups and (share)
    // the first 256x256 GEMM leaves them those CUs; with one kind only, that
    // kind gets every CU it was launched on.
    if (hipEventRecord(aux->fork, s) != hipSuccess)
      return fail(HKMOE_ERR_HIP, "moe_forward: fork event failed");
    const int yield_from = nc.share ? device_cus() - ncus : 0;  // >= device_cus() / 4
    if (hipStreamWaitEvent(aux->aux, aux->fork, 0) != hipSuccess)
      return fail(HKMOE_ERR_HIP, "moe_forward: fork to the auxiliary stream failed");
    AuxJoin guard{aux, s};
    // the narrow kernels launch one workgroup per CU: beside 256x256 tiles the
    // first ncus to start take items, else all of them (decode-like shapes)
    const int ngrid = device_cus();
    t_role = HKMOE_TIMING_GEMM1_NARROW;
    HK_TRY(grouped_gemm1_impl(x_q, x_scale, w.perm, top_k, num_tokens, w13, w13_scale, w.offsets,
                              w.mtile_offsets, w.mtile_list, rows, num_experts, hidden, inter, scale_mode,
                              w_layout, HKMOE_E4M3, w.hq, w.hs, w.narrow_info + 1, aux->aux,
                              w.narrow_info, 0, ncus, ngrid));
    t_role = HKMOE_TIMING_GEMM2_NARROW;
    HK_TRY(grouped_gemm2_impl(w.hq, w.hs, w2, w2_scale, w.offsets, w.mtile_offsets, w.mtile_list, rows,
                              num_experts, hidden, inter, scale_mode, w_layout, w.y, w.narrow_info + 2,
                              aux->aux, w.narrow_info, 0, ncus, ngrid));
    // share == 2: once the narrow GEMMs are done, their CUs join the first 256x256
    // GEMM's tile queues (a second launch of it on the auxiliary stream, which
    // takes whatever tiles are left); the second 256x256 GEMM then waits for both.
    // (Shapes with rows <= 2 * E * max_rows took the one-stream path above.)
    const bool late_join = nc.share == 2;
    t_role = HKMOE_TIMING_GEMM1_JOIN;
    if (late_join)
      HK_TRY(grouped_gemm1_impl(x_q, x_scale, w.perm, top_k, num_tokens, w13, w13_scale, w.offsets,
                                w.mtile_offsets, w.mtile_list, rows, num_experts, hidden, inter, scale_mode,
                                w_layout, HKMOE_E4M3, w.hq, w.hs, w.tile_ctr, aux->aux, w.narrow_info,
                                -1, 0, ncus));
    if (hipEventRecord(aux->join, aux->aux) != hipSuccess)
      return fail(HKMOE_ERR_HIP, "moe_forward: join event failed");
    t_role = HKMOE_TIMING_GEMM1;
    HK_TRY(grouped_gemm1_impl(x_q, x_scale, w.perm, top_k, num_tokens, w13, w13_scale, w.offsets,
                              w.mtile_offsets, w.mtile_list, rows, num_experts, hidden, inter, scale_mode,
                              w_layout, HKMOE_E4M3, w.hq, w.hs, w.tile_ctr, stream, w.narrow_info,
                              yield_from, 0));
    if (late_join && hipStreamWaitEvent(s, aux->join, 0) != hipSuccess)
      return fail(HKMOE_ERR_HIP, "moe_forward: join of the auxiliary stream failed");
    t_role = HKMOE_TIMING_GEMM2;
    HK_TRY(grouped_gemm2_impl(w.hq, w.hs, w2, w2_scale, w.offsets, w.mtile_offsets, w.mtile_list, rows,
                              num_experts, hidden, inter, scale_mode, w_layout, w.y, w.tile_ctr + 8,
                              stream, w.narrow_info, 0, 0));
    if (!late_join && hipStreamWaitEvent(s, aux->join, 0) != hipSuccess)
      return fail(HKMOE_ERR_HIP, "moe_forward: join of the auxiliary stream failed");
    guard.armed = false;  // joined above
    aux_lock.unlock();
    t_role = HKMOE_TIMING_COMBINE;
    HK_TRY(hkmoe_combine(w.y, w.topk_w, w.inv_perm, num_tokens, top_k, hidden, out, stream));
    return HKMOE_OK;
  }
  if (block) {
    // GEMM 1 reads token rows through perm and writes the requantised e4m3
    // intermediate and its 1x128 group scales directly.
    t_role = HKMOE_TIMING_GEMM1;
    HK_TRY(hkmoe_grouped_gemm1(x_q, x_scale, w.perm, top_k, num_tokens, w13, w13_scale, w.offsets,
                               w.mtile_offsets, w.mtile_list, rows, num_experts, hidden, inter,
                               scale_mode, w_layout, HKMOE_E4M3, w.hq, w.hs, w.tile_ctr, stream));
  } else {
    t_role = HKMOE_TIMING_GEMM1;
    HK_TRY(hkmoe_grouped_gemm1(x_q, x_scale, w.perm, top_k, num_tokens, w13, w13_scale, w.offsets,
                               w.mtile_offsets, w.mtile_list, rows, num_experts, hidden, inter,
                               scale_mode, w_layout, HKMOE_BF16, w.h, w.amax, w.tile_ctr, stream));
    t_role = HKMOE_TIMING_REQUANT;
    HK_TRY(hkmoe_requant(w.h, rows, inter, scale_mode, w.amax, w.hq, w.hs, stream));
  }
  t_role = HKMOE_TIMING_GEMM2;
  HK_TRY(hkmoe_grouped_gemm2(w.hq, w.hs, w2, w2_scale, w.offsets, w.mtile_offsets, w.mtile_list,
                             rows, num_experts, hidden, inter, scale_mode, w_layout, w.y,
                             w.tile_ctr + 8, stream));
  t_role = HKMOE_TIMING_COMBINE;
  HK_TRY(hkmoe_combine(w.y, w.topk_w, w.inv_perm, num_tokens, top_k, hidden, out, stream));
  return HKMOE_OK;
}

int hkmoe_moe_forward(const void* x_q, const float* x_scale, const float* logits, const void* w13,
                      const float* w13_scale, const void* w2, const float* w2_scale,
                      int64_t num_tokens, int32_t num_experts, int32_t top_k, int32_t hidden,
                      int32_t inter, int scale_mode, int w_layout, void* out, void* workspace,
                      size_t workspace_bytes, hkmoe_stream_t stream) {
  return moe_forward_impl(x_q, x_scale, logits, w13, w13_scale, w2, w2_scale, num_tokens, num_experts, top_k,
                          hidden, inter, scale_mode, w_layout, out, workspace, workspace_bytes, stream, true);
}

// ---------------------------------------------------------------------------
// quantisers
// ---------------------------------------------------------------------------
int hkmoe_quant_group(const float* x, int64_t rows, int64_t cols, void* q, float* s,
                      hkmoe_stream_t stream) {
  HK_REQUIRE(rows == 0 || (x && q && s), "quant_group: null pointer");
  HK_REQUIRE(rows >= 0 && cols > 0 && cols % kGroup == 0, "quant_group: cols must be a multiple of 128");
  const int64_t waves = rows * (cols / kGroup);
  if (waves == 0) return HKMOE_OK;
  HK_REQUIRE((waves + 3) / 4 < (1ll << 31), "quant_group: too large");
  hipLaunchKernelGGL(quant_group_kernel, dim3(static_cast<unsigned>((waves + 3) / 4)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, rows, cols, static_cast<uint8_t*>(q), s);
  return check_launch("quant_group_kernel");
}

int hkmoe_quant_block(const float* x, int64_t batch, int64_t rows, int64_t cols, void* q, float* s,
                      hkmoe_stream_t stream) {
  HK_REQUIRE(batch == 0 || (x && q && s), "quant_block: null pointer");
  HK_REQUIRE(batch >= 0 && rows > 0 && cols > 0 && rows % kGroup == 0 && cols % kGroup == 0,
             "quant_block: rows and cols must be multiples of 128");
  const int64_t blocks = batch * (rows / kGroup) * (cols / kGroup);
  if (blocks == 0) return HKMOE_OK;
  HK_REQUIRE(blocks < (1ll << 31), "quant_block: too large");
  hipLaunchKernelGGL(quant_block_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), x, rows, cols, static_cast<uint8_t*>(q), s);
  return check_launch("quant_block_kernel");
}

int hkmoe_quant_tensor(const float* x, int64_t rows, int64_t cols, void* q, float* s, float* amax_ws,
                       hkmoe_stream_t stream) {
  HK_REQUIRE(s && amax_ws && (rows == 0 || cols == 0 || (x && q)), "quant_tensor: null pointer");
  HK_REQUIRE(rows >= 0 && cols >= 0, "quant_tensor: bad shape");
  const int64_t n = rows * cols;
  auto st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(fill_f32_kernel, dim3(1), dim3(1), 0, st, amax_ws, 0.0f);
  HK_TRY(check_launch("fill_f32_kernel"));
  const int grid = static_cast<int>(std::min<int64_t>(std::max<int64_t>(1, (n + 255) / 256), 4096));
  if (n > 0) {
    hipLaunchKernelGGL(amax_kernel, dim3(grid), dim3(256), 0, st, x, n, amax_ws);
    HK_TRY(check_launch("amax_kernel"));
  }
  hipLaunchKernelGGL(quant_tensor_kernel, dim3(grid), dim3(256), 0, st, x, n, amax_ws,
                     static_cast<uint8_t*>(q), s);
  return check_launch("quant_tensor_kernel");
}

// ---------------------------------------------------------------------------
// MX (e8m0 1x32) operands and GEMM
// ---------------------------------------------------------------------------
int hkmoe_quant_mx(const float* x, int64_t rows, int64_t cols, void* q, void* s, hkmoe_stream_t stream) {
  HK_REQUIRE(rows == 0 || (x && q && s), "quant_mx: null pointer");
  HK_REQUIRE(rows >= 0 && cols > 0 && cols % 32 == 0, "quant_mx: cols=%lld must be a positive multiple of 32",
             (long long)cols);
  const int64_t blocks = rows * (cols / 32);
  if (blocks == 0) return HKMOE_OK;
  const int grid = static_cast<int>(std::min<int64_t>((blocks * 8 + 255) / 256, 8192));
  hipLaunchKernelGGL(quant_mx_kernel, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream), x, blocks,
                     static_cast<uint8_t*>(q), static_cast<uint8_t*>(s));
  return check_launch("quant_mx_kernel");
}

int hkmoe_mx_pack_scales(const void* s, int64_t rows, int64_t cols, void* packed, hkmoe_stream_t stream) {
  HK_REQUIRE(rows == 0 || (s && packed), "mx_pack_scales: null pointer");
  HK_REQUIRE(rows >= 0 && cols > 0 && cols % kBK == 0,
             "mx_pack_scales: cols=%lld must be a positive multiple of 128", (long long)cols);
  const int64_t rows64 = (rows + 63) / 64 * 64;
  const int64_t words = (cols / kBK) * rows64;
  if (words == 0) return HKMOE_OK;
  const int grid = static_cast<int>(std::min<int64_t>((words + 255) / 256, 8192));
  hipLaunchKernelGGL(mx_pack_scales_kernel, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint8_t*>(s), rows, cols / 32, rows64, static_cast<uint32_t*>(packed),
                     words);
  return check_launch("mx_pack_scales_kernel");
}

int hkmoe_gemm_mx(const void* a, const void* a_scale, const void* b, const void* b_scale, void* c, int64_t m,
                  int64_t n, int64_t k, int out_dtype, hkmoe_stream_t stream) {
  HK_REQUIRE(b && b_scale && (m == 0 || (a && a_scale && c)), "gemm_mx: null pointer");
  HK_REQUIRE(m >= 0 && n > 0 && k > 0, "gemm_mx: bad shape M=%lld N=%lld K=%lld", (long long)m, (long long)n,
             (long long)k);
  HK_REQUIRE(k % kBK == 0, "gemm_mx: K=%lld must be a multiple of 128", (long long)k);
  HK_REQUIRE(n % kBN == 0, "gemm_mx: N=%lld must be a multiple of 256", (long long)n);
  const int64_t m64 = (m + 63) / 64 * 64;
  HK_REQUIRE(k <= (1 << 20) && n * k < (1ll << 32) && m * k < (1ll << 32) && m < (1ll << 31) &&
                 m64 * (k / 32) < (1ll << 32) && n * (k / 32) < (1ll << 32),
             "gemm_mx: operand too large for 32-bit buffer offsets (M*K and N*K must be < 2^32)");
  HK_REQUIRE(out_dtype == HKMOE_BF16 || out_dtype == HKMOE_F32, "gemm_mx: bad out_dtype %d", out_dtype);
  if (m == 0) return HKMOE_OK;
  GemmParams p{};
  p.a = static_cast<const uint8_t*>(a);
  p.b = static_cast<const uint8_t*>(b);
  p.c = c;
  p.a_scale = static_cast<const float*>(a_scale);
  p.b_scale = static_cast<const float*>(b_scale);
  p.rows = m;
  p.a_rows = m;
  p.as_rs = m64;
  p.num_experts = 1;
  p.K = static_cast<int32_t>(k);
  p.nb = static_cast<int32_t>(n);
  p.n_out = static_cast<int32_t>(n);
  p.n_tiles = static_cast<int32_t>(n / kBN);
  p.blk_m_log2 = 2;  // 4 x 8 tile blocks
  auto st = static_cast<hipStream_t>(stream);
  return out_dtype == HKMOE_BF16 ? launch_gemm<Epi::kStoreBf16, Scale::kMX>(p, st)
                                 : launch_gemm<Epi::kStoreF32, Scale::kMX>(p, st);
}


int64_t hkmoe_mx_words_per_step(int64_t rows, int32_t num_experts) {
  return rows < 0 || num_experts < 1 ? 0 : mx_words_per_step(rows, num_experts);
}

int hkmoe_mx_pack_weight_scales(const void* s, int64_t num_experts, int64_t n, int64_t k, int32_t gate_up,
                                void* words, hkmoe_stream_t stream) {
  HK_REQUIRE(s && words, "mx_pack_weight_scales: null pointer");
  HK_REQUIRE(num_experts >= 0 && n > 0 && k > 0 && n % kBN == 0 && k % kBK == 0,
             "mx_pack_weight_scales: N=%lld must be a multiple of 256 and K=%lld of 128", (long long)n,
             (long long)k);
  HK_REQUIRE(gate_up == 0 || (gate_up > 0 && 2ll * gate_up == n && gate_up % 128 == 0),
             "mx_pack_weight_scales: gate_up=%d must be 0 or N/2 (a multiple of 128)", gate_up);
  HK_REQUIRE(k <= (1 << 20), "mx_pack_weight_scales: K too large");
  const int64_t n_words = num_experts * n * (k / 128);
  if (n_words == 0) return HKMOE_OK;
  const int grid = static_cast<int>(std::min<int64_t>((n_words + 255) / 256, 8192));
  hipLaunchKernelGGL(mx_pack_weight_words_kernel, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint8_t*>(s), n, static_cast<int>(k), gate_up,
                     static_cast<uint32_t*>(words), n_words);
  return check_launch("mx_pack_weight_words_kernel");
}

int hkmoe_mx_gather_scales(const void* s, int64_t x_rows, int32_t k, const int32_t* gather, int32_t gather_div,
                           const int32_t* offsets, const int32_t* mtile_offsets, int32_t num_experts,
                           int64_t rows, void* words, hkmoe_stream_t stream) {
  HK_REQUIRE(offsets && mtile_offsets, "mx_gather_scales: null pointer");
  HK_REQUIRE(rows == 0 || (s && words), "mx_gather_scales: null pointer");
  HK_REQUIRE(k > 0 && k % kBK == 0 && k / 32 <= kMxGatherMaxKb,
             "mx_gather_scales: K=%d must be a multiple of 128 and <= %d", k, 32 * kMxGatherMaxKb);
  HK_REQUIRE(num_experts >= 1 && num_experts <= kMaxExperts, "mx_gather_scales: bad E=%d", num_experts);
  HK_REQUIRE(rows >= 0 && rows < (1ll << 31) && x_rows >= 0, "mx_gather_scales: bad rows");
  HK_REQUIRE(gather != nullptr ? gather_div >= 1 : x_rows >= rows, "mx_gather_scales: bad gather");
  HK_REQUIRE((reinterpret_cast<uintptr_t>(s) & 3) == 0, "mx_gather_scales: exponents must be 4-byte aligned");
  if (rows == 0) return HKMOE_OK;
  const int64_t ws = mx_words_per_step(rows, num_experts);
  // one workgroup per M tile (ws / 256 bounds their number), the tile's exponent
  // rows in LDS
  static bool attr_set[kMaxDevices] = {false};
  int dev = 0;
  (void)hipGetDevice(&dev);
  if (dev >= 0 && dev < kMaxDevices && !attr_set[dev]) {
    const hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(mx_gather_words_kernel),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, 256 * kMxGatherMaxKb);
    if (err != hipSuccess) return fail(HKMOE_ERR_HIP, "hipFuncSetAttribute: %s", hipGetErrorString(err));
    attr_set[dev] = true;
  }
  const int grid = static_cast<int>(std::min<int64_t>(ws / 256, 4096));
  hk_launch(mx_gather_words_kernel, dim3(grid), dim3(256), static_cast<uint32_t>(256 * (k / 32)),
            static_cast<hipStream_t>(stream),
                     static_cast<const uint8_t*>(s), k, gather, gather ? gather_div : 1, offsets, mtile_offsets,
                     num_experts, ws, static_cast<uint32_t*>(words));
  return check_launch("mx_gather_words_kernel");
}

int hkmoe_grouped_gemm1_mx(const void* x, const void* x_words, const int32_t* gather, int32_t gather_div,
                           int64_t x_rows, const void* w13, const void* w13_words, const int32_t* offsets,
                           const int32_t* mtile_offsets, const int32_t* mtile_list, int64_t rows,
                           int32_t num_experts, int32_t hidden, int32_t inter, int w_layout, int out_format,
                           void* h, void* h_words, int32_t* tile_counters, hkmoe_stream_t stream) {
  HK_REQUIRE(w13 && w13_words && offsets && mtile_offsets, "grouped_gemm1_mx: null pointer");
  HK_REQUIRE(rows == 0 || (x && x_words && h), "grouped_gemm1_mx: null pointer");
  HK_REQUIRE(num_experts >= 1 && num_experts <= kMaxExperts, "grouped_gemm1_mx: bad E=%d", num_experts);
  HK_REQUIRE(hidden > 0 && hidden % kGroup == 0 && hidden <= kGroup * kMaxKBlocks,
             "grouped_gemm1_mx: hidden=%d must be a multiple of 128 and <= %d", hidden, kGroup * kMaxKBlocks);
  HK_REQUIRE(inter > 0 && inter % 128 == 0, "grouped_gemm1_mx: inter=%d must be a multiple of 128", inter);
  HK_REQUIRE(rows >= 0 && rows < (1ll << 31), "grouped_gemm1_mx: bad rows");
  HK_REQUIRE(x_rows >= (rows > 0 ? 1 : 0) && x_rows * hidden < (1ll << 32), "grouped_gemm1_mx: x_rows=%lld out of range",
             (long long)x_rows);
  HK_REQUIRE(gather == nullptr || gather_div >= 1, "grouped_gemm1_mx: gather_div must be >= 1");
  HK_REQUIRE(gather != nullptr || x_rows >= rows, "grouped_gemm1_mx: x has fewer rows than rows");
  HK_REQUIRE(2ll * inter * hidden < (1ll << 32), "grouped_gemm1_mx: expert weight too large");
  HK_REQUIRE(w_layout == HKMOE_W_ROWS || w_layout == HKMOE_W_PACKED, "grouped_gemm1_mx: bad w_layout %d",
             w_layout);
  HK_REQUIRE(out_format == HKMOE_BF16 || out_format == HKMOE_E4M3, "grouped_gemm1_mx: bad out_format %d",
             out_format);
  HK_REQUIRE(out_format != HKMOE_E4M3 || h_words != nullptr, "grouped_gemm1_mx: e4m3 output needs h_words");
  if (rows == 0) return HKMOE_OK;
  const int64_t ws = mx_words_per_step(rows, num_experts);
  HK_REQUIRE(ws * (std::max(hidden, inter) / kBK) * 4 < (1ll << 32), "grouped_gemm1_mx: too many rows");
  GemmParams p{};
  p.a = static_cast<const uint8_t*>(x);
  p.a_gather = gather;
  p.gather_div = gather ? gather_div : 1;
  p.b = static_cast<const uint8_t*>(w13);
  p.c = h;
  p.a_scale = static_cast<const float*>(x_words);
  p.b_scale = static_cast<const float*>(w13_words);
  p.c_scale = static_cast<float*>(h_words);
  p.offsets = offsets;
  p.mtile_offsets = mtile_offsets;
  p.rows = rows;
  p.a_rows = x_rows;
  p.as_rs = ws;
  p.cs_rs = ws;
  p.num_experts = num_experts;
  p.K = hidden;
  p.nb = 2 * inter;
  p.n_out = inter;
  p.n_tiles = inter / 128;
  p.b_packed = w_layout == HKMOE_W_PACKED;
  p.mtile_list = mtile_list;
  p.blk_m_log2 = block_m_log2(1);  // 2 x 16 tile blocks by default
  p.tile_ctr = tile_counters;
  auto st = static_cast<hipStream_t>(stream);
  return out_format == HKMOE_E4M3 ? launch_gemm<Epi::kSiluMx, Scale::kMX>(p, st)
                                  : launch_gemm<Epi::kSiluBf16, Scale::kMX>(p, st);
}

int hkmoe_grouped_gemm2_mx(const void* hq, const void* hq_words, const void* w2, const void* w2_words,
                           const int32_t* offsets, const int32_t* mtile_offsets, const int32_t* mtile_list,
                           int64_t rows, int32_t num_experts, int32_t hidden, int32_t inter, int w_layout,
                           void* y, int32_t* tile_counters, hkmoe_stream_t stream) {
  HK_REQUIRE(w2 && w2_words && offsets && mtile_offsets, "grouped_gemm2_mx: null pointer");
  HK_REQUIRE(rows == 0 || (hq && hq_words && y), "grouped_gemm2_mx: null pointer");
  HK_REQUIRE(num_experts >= 1 && num_experts <= kMaxExperts, "grouped_gemm2_mx: bad E=%d", num_experts);
  HK_REQUIRE(hidden > 0 && hidden % kBN == 0, "grouped_gemm2_mx: hidden=%d must be a multiple of 256", hidden);
  HK_REQUIRE(inter > 0 && inter % kGroup == 0 && inter <= kGroup * kMaxKBlocks,
             "grouped_gemm2_mx: inter=%d must be a multiple of 128 and <= %d", inter, kGroup * kMaxKBlocks);
  HK_REQUIRE(rows >= 0 && rows < (1ll << 31), "grouped_gemm2_mx: bad rows");
  HK_REQUIRE(rows * inter < (1ll << 32), "grouped_gemm2_mx: rows*inter must be < 2^32 (32-bit buffer offsets into hq)");
  HK_REQUIRE(static_cast<int64_t>(hidden) * inter < (1ll << 32), "grouped_gemm2_mx: expert weight too large");
  HK_REQUIRE(w_layout == HKMOE_W_ROWS || w_layout == HKMOE_W_PACKED, "grouped_gemm2_mx: bad w_layout %d",
             w_layout);
  if (rows == 0) return HKMOE_OK;
  const int64_t ws = mx_words_per_step(rows, num_experts);
  HK_REQUIRE(ws * (inter / kBK) * 4 < (1ll << 32), "grouped_gemm2_mx: too many rows");
  GemmParams p{};
  p.a = static_cast<const uint8_t*>(hq);
  p.b = static_cast<const uint8_t*>(w2);
  p.c = y;
  p.a_scale = static_cast<const float*>(hq_words);
  p.b_scale = static_cast<const float*>(w2_words);
  p.offsets = offsets;
  p.mtile_offsets = mtile_offsets;
  p.rows = rows;
  p.a_rows = rows;
  p.as_rs = ws;
  p.num_experts = num_experts;
  p.K = inter;
  p.nb = hidden;
  p.n_out = hidden;
  p.n_tiles = hidden / kBN;
  p.b_packed = w_layout == HKMOE_W_PACKED;
  p.mtile_list = mtile_list;
  p.blk_m_log2 = block_m_log2(2);
  p.tile_ctr = tile_counters;
  return launch_gemm<Epi::kStoreBf16, Scale::kMX>(p, static_cast<hipStream_t>(stream));
}

int hkmoe_moe_forward_mx(const void* x_q, const void* x_e8m0, const float* logits, const void* w13,
                         const void* w13_words, const void* w2, const void* w2_words, int64_t num_tokens,
                         int32_t num_experts, int32_t top_k, int32_t hidden, int32_t inter, int w_layout,
                         void* out, void* workspace, size_t workspace_bytes, hkmoe_stream_t stream) {
  // with no tokens the activations, the output and the workspace may be empty (null)
  HK_REQUIRE(w13 && w13_words && w2 && w2_words, "moe_forward_mx: null pointer");
  HK_REQUIRE(num_tokens == 0 || (x_q && x_e8m0 && logits && out), "moe_forward_mx: null pointer");
  HK_REQUIRE(w_layout == HKMOE_W_ROWS || w_layout == HKMOE_W_PACKED, "moe_forward_mx: bad w_layout %d",
             w_layout);
  HK_REQUIRE(num_tokens >= 0 && num_tokens * top_k < (1ll << 31), "moe_forward_mx: bad T");
  HK_REQUIRE(num_experts >= 1 && num_experts <= kMaxExperts, "moe_forward_mx: E=%d outside [1, %d]",
             num_experts, kMaxExperts);
  HK_REQUIRE(top_k >= 1 && top_k <= num_experts && top_k <= kMaxTopK, "moe_forward_mx: bad top_k=%d", top_k);
  HK_REQUIRE(hidden > 0 && hidden % kBN == 0 && hidden <= kGroup * kMaxKBlocks,
             "moe_forward_mx: hidden=%d must be a multiple of 256 and <= %d", hidden, kGroup * kMaxKBlocks);
  HK_REQUIRE(inter > 0 && inter % 128 == 0 && inter <= kGroup * kMaxKBlocks,
             "moe_forward_mx: inter=%d must be a multiple of 128 and <= %d", inter, kGroup * kMaxKBlocks);
  HK_REQUIRE(2ll * inter * hidden < (1ll << 32), "moe_forward_mx: expert weight too large (2*I*H must be < 2^32)");
  HK_REQUIRE(num_tokens * hidden < (1ll << 32) && num_tokens * top_k * inter < (1ll << 32),
             "moe_forward_mx: T*H and T*k*I must be < 2^32 (32-bit buffer offsets)");
  if (num_tokens == 0) return HKMOE_OK;
  const MoeWorkspace need = carve(nullptr, num_tokens, num_experts, top_k, hidden, inter, HKMOE_SCALE_MX);
  if (workspace == nullptr || workspace_bytes < need.bytes)
    return fail(HKMOE_ERR_WORKSPACE, "moe_forward_mx: workspace of %zu bytes needed, %zu given", need.bytes,
                workspace_bytes);
  HK_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255) == 0, "moe_forward_mx: workspace must be 256-byte aligned");
  const MoeWorkspace w = carve(static_cast<uint8_t*>(workspace), num_tokens, num_experts, top_k, hidden,
                               inter, HKMOE_SCALE_MX);
  const int64_t rows = num_tokens * top_k;
  TimedCall timed_call;
  t_role = HKMOE_TIMING_ROUTE;
  HK_TRY(hkmoe_route_topk(logits, num_tokens, num_experts, top_k, w.topk_idx, w.topk_w, w.block_counts, stream));
  t_role = HKMOE_TIMING_OFFSETS;
  HK_TRY(hkmoe_expert_offsets(w.block_counts, num_tokens, num_experts, w.counts, w.offsets, w.block_base,
                              w.mtile_offsets, w.mtile_list, w.amax, w.tile_ctr, stream));
  t_role = HKMOE_TIMING_SCATTER;
  HK_TRY(hkmoe_scatter(w.topk_idx, num_tokens, num_experts, top_k, w.offsets, w.block_base, w.perm, w.inv_perm,
                       nullptr, nullptr, hidden, HKMOE_SCALE_TENSOR, nullptr, nullptr, stream));
  // token exponents -> tile-aligned words in expert order (x rows stay in place)
  t_role = HKMOE_TIMING_MX_WORDS;
  HK_TRY(hkmoe_mx_gather_scales(x_e8m0, num_tokens, hidden, w.perm, top_k, w.offsets, w.mtile_offsets,
                                num_experts, rows, w.xw, stream));
  t_role = HKMOE_TIMING_GEMM1;
  HK_TRY(hkmoe_grouped_gemm1_mx(x_q, w.xw, w.perm, top_k, num_tokens, w13, w13_words, w.offsets, w.mtile_offsets,
                                w.mtile_list, rows, num_experts, hidden, inter, w_layout, HKMOE_E4M3, w.hq, w.hs,
                                w.tile_ctr, stream));
  t_role = HKMOE_TIMING_GEMM2;
  HK_TRY(hkmoe_grouped_gemm2_mx(w.hq, w.hs, w2, w2_words, w.offsets, w.mtile_offsets, w.mtile_list, rows,
                                num_experts, hidden, inter, w_layout, w.y, w.tile_ctr + 8, stream));
  t_role = HKMOE_TIMING_COMBINE;
  HK_TRY(hkmoe_combine(w.y, w.topk_w, w.inv_perm, num_tokens, top_k, hidden, out, stream));
  return HKMOE_OK;
}

// ---------------------------------------------------------------------------
// kernel timing of the layer entry points
// ---------------------------------------------------------------------------
int hkmoe_kernel_timing(int32_t calls) {
  HK_REQUIRE(calls >= 0 && calls <= 4096, "kernel_timing: calls=%d outside [0, 4096]", calls);
  std::lock_guard<std::mutex> g(g_timing_mu);
  for (hipEvent_t e : g_timing.ev) (void)hipEventDestroy(e);
  g_timing = KernelTiming{};
  if (calls == 0) return HKMOE_OK;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return fail(HKMOE_ERR_HIP, "kernel_timing: no device");
  const size_t n = static_cast<size_t>(calls) * HKMOE_TIMING_ROLES * 2;
  g_timing.ev.reserve(n);
  for (size_t i = 0; i < n; ++i) {
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) {
      for (hipEvent_t x : g_timing.ev) (void)hipEventDestroy(x);
      g_timing = KernelTiming{};
      return fail(HKMOE_ERR_HIP, "kernel_timing: hipEventCreate failed");
    }
    g_timing.ev.push_back(e);
  }
  g_timing.used.assign(static_cast<size_t>(calls) * HKMOE_TIMING_ROLES, 0);
  g_timing.first.assign(calls, -1);
  g_timing.last.assign(calls, -1);
  g_timing.device = dev;
  g_timing.calls = calls;
  return HKMOE_OK;
}

int hkmoe_kernel_timing_read(int32_t set, float* begin_ms, float* end_ms, int32_t n) {
  HK_REQUIRE(begin_ms && end_ms && n >= HKMOE_TIMING_ROLES, "kernel_timing_read: need %d floats per array",
             HKMOE_TIMING_ROLES);
  std::lock_guard<std::mutex> g(g_timing_mu);
  HK_REQUIRE(set >= 0 && set < g_timing.calls, "kernel_timing_read: set=%d outside [0, %d)", set,
             g_timing.calls);
  const size_t base = static_cast<size_t>(set) * HKMOE_TIMING_ROLES;
  const int f = g_timing.first[set];
  for (int r = 0; r < HKMOE_TIMING_ROLES; ++r) {
    begin_ms[r] = end_ms[r] = -1.0f;
    if (f < 0 || !g_timing.used[base + r]) continue;
    const hipEvent_t t0 = g_timing.ev[2 * (base + f)];
    if (hipEventElapsedTime(&begin_ms[r], t0, g_timing.ev[2 * (base + r)]) != hipSuccess ||
        hipEventElapsedTime(&end_ms[r], t0, g_timing.ev[2 * (base + r) + 1]) != hipSuccess)
      return fail(HKMOE_ERR_HIP, "kernel_timing_read: events of set %d not complete", set);
  }
  return HKMOE_OK;
}

// ---------------------------------------------------------------------------
// allocation-free layer (hkmoe_moe_forward_noalloc)
// ---------------------------------------------------------------------------
int hkmoe_moe_forward_noalloc(const void* x_q, const float* x_scale, const float* logits, const void* w13,
                              const float* w13_scale, const void* w2, const float* w2_scale,
                              int64_t num_tokens, int32_t num_experts, int32_t top_k, int32_t hidden,
                              int32_t inter, int scale_mode, int w_layout, void* out, hkmoe_stream_t stream) {
  HK_REQUIRE(num_tokens >= 0 && num_experts >= 1 && top_k >= 1 && hidden > 0 && inter > 0,
             "moe_forward_noalloc: bad shape");
  HK_REQUIRE(scale_mode == HKMOE_SCALE_TENSOR || scale_mode == HKMOE_SCALE_BLOCK,
             "moe_forward_noalloc: bad scale_mode %d", scale_mode);
  const size_t need = carve(nullptr, num_tokens, num_experts, top_k, hidden, inter, scale_mode).bytes;
  if (need > kScratchBytes)
    return fail(HKMOE_ERR_WORKSPACE,
                "moe_forward_noalloc: the layer needs %zu bytes of workspace, the library's per-device scratch "
                "holds %zu (HKMOE_NOALLOC_SCRATCH_BYTES); pass a workspace to hkmoe_moe_forward instead",
                need, kScratchBytes);
  if (num_tokens == 0) return moe_forward_impl(x_q, x_scale, logits, w13, w13_scale, w2, w2_scale, num_tokens,
                                               num_experts, top_k, hidden, inter, scale_mode, w_layout, out,
                                               nullptr, 0, stream, false);
  void* ws = nullptr;
  HK_TRY(scratch_ptr(&ws));
  return moe_forward_impl(x_q, x_scale, logits, w13, w13_scale, w2, w2_scale, num_tokens, num_experts, top_k,
                          hidden, inter, scale_mode, w_layout, out, ws, kScratchBytes, stream, false);
}
}  // extern "C"
