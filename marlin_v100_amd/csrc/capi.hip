// capi.hip -- extern "C" entry points of libmarlin_mi355x.so (declared in
// include/marlin_mi355x.h): argument validation, tile selection, split-K workspace and
// kernel dispatch.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <map>
#include <mutex>
#include <sstream>
#include <string>
#include <tuple>
#include <unordered_map>
#include <utility>

#include "../../include/marlin_mi355x.h"
#include "host_common.h"

using namespace mmi;

namespace {

thread_local std::string g_last_error;

struct CheckFailed {
  marlin_status_t status;
};

// Builds the message from the streamed pieces, like TORCH_CHECK(cond, a, b, ...).
template <typename... Args>
void check(bool cond, Args&&... args) {
  if (cond) return;
  std::ostringstream os;
  (os << ... << args);
  g_last_error = os.str();
  throw CheckFailed{MARLIN_STATUS_INVALID_ARGUMENT};
}
template <typename... Args>
void check_supported(bool cond, Args&&... args) {
  if (cond) return;
  std::ostringstream os;
  (os << ... << args);
  g_last_error = os.str();
  throw CheckFailed{MARLIN_STATUS_NOT_SUPPORTED};
}
void check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return;
  g_last_error = std::string(what) + ": " + hipGetErrorString(e);
  throw CheckFailed{MARLIN_STATUS_HIP_ERROR};
}

template <typename F>
marlin_status_t guarded(F&& f) {
  try {
    f();
    g_last_error.clear();
    return MARLIN_STATUS_OK;
  } catch (const CheckFailed& c) {
    return c.status;
  } catch (const std::exception& e) {
    g_last_error = e.what();
    return MARLIN_STATUS_HIP_ERROR;
  }
}

// vllm ScalarType ids (vllm/scalar_type.py:25-43).
constexpr int64_t kU4 = 1125899906843648LL;
constexpr int64_t kU4B8 = 1125899907892224LL;
constexpr int64_t kU8 = 1125899906844672LL;
constexpr int64_t kU8B128 = 1125899923621888LL;
constexpr int64_t kFE2M1f = 562949953487106LL;
constexpr int64_t kFE4M3fn = 2814749767172868LL;

int fmt_from_type(int64_t b_type_id, marlin_dtype_t scales_dtype) {
  if (b_type_id == kU4B8) return FMT_U4B8;
  if (b_type_id == kU4) return FMT_U4;
  if (b_type_id == kU8B128) return FMT_U8B128;
  if (b_type_id == kU8) return FMT_U8;
  if (b_type_id == kFE4M3fn) return FMT_FP8;
  if (b_type_id == kFE2M1f) {
    if (scales_dtype == MARLIN_DTYPE_FLOAT8_E4M3FN) return FMT_NVFP4;
    if (scales_dtype == MARLIN_DTYPE_FLOAT8_E8M0FNU) return FMT_MXFP4;
    check(false,
          "When b_type = float4_e2m1f, b_scales must be float8_e4m3fn for NVFP4 or "
          "float8_e8m0fnu for MXFP4 scales.");
  }
  check_supported(false,
                  "marlin_gemm implements only uint4, uint4b8, uint8, uint8b128, fp8_e4m3fn, "
                  "nvfp4, and mxfp4 weights. Got b_type_id = ",
                  b_type_id);
  return -1;
}

bool is_half_type(marlin_dtype_t d) {
  return d == MARLIN_DTYPE_FLOAT16 || d == MARLIN_DTYPE_BFLOAT16;
}

int ilog2_exact(int64_t v) {
  int s = 0;
  while ((int64_t(1) << s) < v) ++s;
  return (int64_t(1) << s) == v ? s : -1;
}

// ---- device properties and split-K workspace ------------------------------------------
int device_cu_count(int dev) {
  static std::mutex mu;
  static std::map<int, int> cache;
  std::lock_guard<std::mutex> lk(mu);
  auto it = cache.find(dev);
  if (it != cache.end()) return it->second;
  int cus = 0;
  check_hip(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev),
            "hipDeviceGetAttribute");
  cache[dev] = cus;
  return cus;
}

struct Workspace {
  float* ws = nullptr;
  size_t ws_elems = 0;
  int* counters = nullptr;
  size_t n_counters = 0;
};

// One zero-initialised workspace per (device, stream).  Kernels leave it zeroed, so it is
// cleared only when allocated.  Growing it synchronises the stream (first calls only); a
// stream that is capturing a graph cannot allocate, so growth there is an error that names
// the remedy instead of an allocation and a memset recorded into the graph.
Workspace& get_workspace(int dev, hipStream_t stream, size_t need_elems, size_t need_counters) {
  static std::mutex mu;
  static std::map<std::pair<int, hipStream_t>, Workspace> spaces;
  std::lock_guard<std::mutex> lk(mu);
  Workspace& w = spaces[{dev, stream}];
  if (need_elems > w.ws_elems || need_counters > w.n_counters) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    check_hip(hipStreamIsCapturing(stream, &cs), "hipStreamIsCapturing");
    check_supported(cs == hipStreamCaptureStatusNone,
                    "split-K workspace for this shape is not yet allocated on the capturing "
                    "stream: run the same shape once on that stream before capturing, or use "
                    "marlin_gemm_no_alloc");
  }
  if (need_elems > w.ws_elems) {
    size_t n = std::max<size_t>(need_elems, std::max<size_t>(2 * w.ws_elems, size_t(1) << 20));
    if (w.ws) {
      check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
      check_hip(hipFree(w.ws), "hipFree");
      w.ws = nullptr;
      w.ws_elems = 0;
    }
    check_hip(hipMalloc(&w.ws, n * sizeof(float)), "hipMalloc(split-K workspace)");
    check_hip(hipMemsetAsync(w.ws, 0, n * sizeof(float), stream), "hipMemsetAsync");
    w.ws_elems = n;
  }
  if (need_counters > w.n_counters) {
    size_t n = std::max<size_t>(need_counters, std::max<size_t>(2 * w.n_counters, 4096));
    if (w.counters) {
      check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
      check_hip(hipFree(w.counters), "hipFree");
      w.counters = nullptr;
      w.n_counters = 0;
    }
    check_hip(hipMalloc(&w.counters, n * sizeof(int)), "hipMalloc(split-K counters)");
    check_hip(hipMemsetAsync(w.counters, 0, n * sizeof(int), stream), "hipMemsetAsync");
    w.n_counters = n;
  }
  return w;
}

// Staging buffers, one per (purpose, device, stream), grown like the workspace (refused
// while the stream captures a graph): the act-order copy of A[:, perm] and the 16-bit codes
// of packed integer zero points.  Each call rewrites what it uses in full, so they need no
// clearing.
enum StagingSlot { kStageActOrder = 0, kStageZeros = 1 };
void* get_staging(int slot, int dev, hipStream_t stream, size_t bytes) {
  static std::mutex mu;
  static std::map<std::tuple<int, int, hipStream_t>, std::pair<void*, size_t>> bufs;
  std::lock_guard<std::mutex> lk(mu);
  auto& b = bufs[{slot, dev, stream}];
  if (bytes > b.second) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    check_hip(hipStreamIsCapturing(stream, &cs), "hipStreamIsCapturing");
    check_supported(cs == hipStreamCaptureStatusNone,
                    slot == kStageActOrder
                        ? "act_order staging buffer for this shape is not yet allocated on the "
                          "capturing stream: run the same shape once on that stream before "
                          "capturing"
                        : "zero-point staging buffer for this shape is not yet allocated on the "
                          "capturing stream: run the same shape once on that stream before "
                          "capturing");
    const size_t n = std::max<size_t>(bytes, std::max<size_t>(2 * b.second, size_t(1) << 21));
    if (b.first) {
      check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
      check_hip(hipFree(b.first), "hipFree");
      b = {nullptr, 0};
    }
    check_hip(hipMalloc(&b.first, n), "hipMalloc(staging)");
    b.second = n;
  }
  return b.first;
}

// Packed integer zero points -> 16-bit codes in a staging buffer; returns the codes.
const void* stage_int_zeros(int dev, hipStream_t stream, const void* words, int bits,
                            int64_t n_codes) {
  void* codes = get_staging(kStageZeros, dev, stream, (size_t)n_codes * sizeof(uint16_t));
  check_hip(launch_expand_zeros(words, bits, n_codes, codes, stream), "zero-point expand launch");
  return codes;
}

// ---- static split-K scratch of marlin_gemm_no_alloc -------------------------------------
// One array per GPU, held until the process ends: kScratchPartials fp32 partial sums, then
// kScratchCounters arrival counters.  A static __device__ array starts zeroed when the code
// object loads, and the kernels' split-K protocol leaves every entry it used zeroed again
// (the last arriver reads the sums back with atomic exchanges against 0 and resets its
// counter), so each call finds it zeroed.  Calls that overlap on one GPU share the array
// and race.
constexpr size_t kScratchPartials = size_t(1) << 21;  // 8 MiB of fp32 partial sums
constexpr size_t kScratchCounters = size_t(1) << 16;  // 256 KiB of arrival counters
static_assert(kScratchPartials == MARLIN_NO_ALLOC_MAX_PARTIALS, "header limit");
static_assert(kScratchCounters == MARLIN_NO_ALLOC_MAX_COUNTERS, "header limit");
static __device__ __align__(256) uint32_t scratch[kScratchPartials + kScratchCounters];

__global__ void clear_words(uint32_t* p, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

// Device address of this GPU's scratch (the host-side name of the array is not one).  The
// first call on a device, with that device current, looks the address up and clears the
// array once with a fill kernel on the caller's stream (no allocation, no memset node).
uint32_t* scratch_on_device(int dev, hipStream_t stream) {
  static std::mutex mu;
  static std::map<int, uint32_t*> ptrs;
  std::lock_guard<std::mutex> lk(mu);
  auto it = ptrs.find(dev);
  if (it != ptrs.end()) return it->second;
  void* ptr = nullptr;
  check_hip(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
  hipLaunchKernelGGL(clear_words, dim3(1024), dim3(256), 0, stream,
                     reinterpret_cast<uint32_t*>(ptr), kScratchPartials + kScratchCounters);
  check_hip(hipGetLastError(), "scratch clear launch");
  ptrs[dev] = reinterpret_cast<uint32_t*>(ptr);
  return ptrs[dev];
}

// ---- tile selection -------------------------------------------------------------------
struct Plan {
  int bm, nt, ch, depth, wpb, ksplit, occ, stream, splits, steps_per_split, main_blocks, n_blocks,
      m_blocks, xcd_group_m;
  int64_t grid;
};

hipError_t dispatch_gemm(const GemmLaunch& l, const GemmParams& p, hipStream_t s);

// Workgroups of one kernel instance that fit on a CU at once, and whether its registers
// spill to scratch (cached per instance).
struct Fit {
  int blocks_per_cu;
  bool spills;
};
Fit kernel_fit(const GemmLaunch& l) {
  static std::mutex mu;
  static std::map<std::tuple<int, int, int, int, int, int, int, int, int, int, int, int>, Fit> cache;
  const auto key = std::make_tuple(l.fmt, (int)l.bf16, l.gsm, l.bm, l.nt, l.ch, l.depth, l.wpb,
                                   (int)l.ksplit, l.occ, (int)l.stream, (int)l.moe);
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  GemmLaunch q = l;
  int occ = 0, scratch = 0;
  q.occupancy = &occ;
  q.scratch = &scratch;
  GemmParams dummy{};
  Fit f{1, false};
  if (dispatch_gemm(q, dummy, nullptr) == hipSuccess) f = Fit{std::max(occ, 1), scratch > 0};
  cache.emplace(key, f);
  return f;
}
int blocks_per_cu(const GemmLaunch& l) { return kernel_fit(l).blocks_per_cu; }

// Whether the library holds an instance for a launch configuration (occupancy query only).
bool instantiated(const GemmLaunch& l) {
  GemmLaunch q = l;
  int occ = 0;
  q.occupancy = &occ;
  q.scratch = nullptr;
  GemmParams dummy{};
  return dispatch_gemm(q, dummy, nullptr) == hipSuccess;
}

// Tuning overrides (MARLIN_MI355X_*), read once per process: the hot path reads no
// environment.  -1 / unset means "the selector decides".
struct Overrides {
  bool decode_set = false;
  int decode[5] = {0, 0, 0, 0, 0};  // nt, depth, wpb, ksplit, occ
  bool tile_set = false;
  int tile[3] = {0, 0, 1};          // bm, nt, ch
  int split_k = -1;
  int stream = 1;
  int stream_max_m = 1 << 30;
  int small_group_max_m = -1;  // -1: 2048 rows for fp4 weights, 1024 for integer small groups
  int stream_nt = -1;
  int stream_bm = -1;
  int xcd_group_m = -1;
  int moe_split_k = -1;
  int moe_group_m = 4;
  int moe_decode = 1;
  int moe_depth = 2;
  int moe_wpb = 1;
  int moe_nt = -1;
  bool any = false;  // some override is set (plans are then checked for an instance)
};

const Overrides& overrides() {
  static const Overrides o = [] {
    Overrides r;
    auto env = [&](const char* name) -> const char* {
      const char* v = getenv(name);
      if (v && *v) {
        r.any = true;
        return v;
      }
      return nullptr;
    };
    auto env_int = [&](const char* name, int& dst) {
      if (const char* v = env(name)) dst = atoi(v);
    };
    if (const char* t = env("MARLIN_MI355X_DECODE")) {
      r.decode_set = sscanf(t, "%d,%d,%d,%d,%d", &r.decode[0], &r.decode[1], &r.decode[2],
                            &r.decode[3], &r.decode[4]) == 5;
    }
    if (const char* t = env("MARLIN_MI355X_TILE")) {
      r.tile_set = sscanf(t, "%d,%d,%d", &r.tile[0], &r.tile[1], &r.tile[2]) >= 2;
    }
    env_int("MARLIN_MI355X_SPLIT_K", r.split_k);
    env_int("MARLIN_MI355X_STREAM", r.stream);
    env_int("MARLIN_MI355X_STREAM_MAX_M", r.stream_max_m);
    env_int("MARLIN_MI355X_SMALL_GROUP_MAX_M", r.small_group_max_m);
    env_int("MARLIN_MI355X_STREAM_NT", r.stream_nt);
    env_int("MARLIN_MI355X_STREAM_BM", r.stream_bm);
    env_int("MARLIN_MI355X_XCD_GROUP_M", r.xcd_group_m);
    env_int("MARLIN_MI355X_MOE_SPLIT_K", r.moe_split_k);
    env_int("MARLIN_MI355X_MOE_GROUP_M", r.moe_group_m);
    env_int("MARLIN_MI355X_MOE_DECODE", r.moe_decode);
    env_int("MARLIN_MI355X_MOE_DEPTH", r.moe_depth);
    env_int("MARLIN_MI355X_MOE_WPB", r.moe_wpb);
    env_int("MARLIN_MI355X_MOE_NT", r.moe_nt);
    return r;
  }();
  return o;
}

// Dense selector.
//  * M <= 16 (decode) is weight-bandwidth bound: the decode kernel, each wave NT n16 tiles,
//    DEPTH-1 K steps in flight, the WPB waves of a workgroup splitting K.  The grid must be
//    resident in one round -- a second, partial round would stream its weights alone at the
//    end -- and spread evenly over the CUs: each CU takes the same number of whole column
//    groups and the groups left over are split along K into about one small block per CU.
//    With at most half as many 64-column groups as CUs the groups are 32 columns wide, and
//    16 columns wide when that many 16-column groups still fit one per CU; K is split across
//    blocks only when under a quarter of the CUs would have a group, within an atomics budget.
//  * 16 < M <= 32 is still weight bound: 32-row blocks with split-K until the grid holds
//    about 4 workgroups per CU.
//  * Larger M is MFMA bound: 64x256 or 128x256 blocks (each wave 64/128 x 64) visited in the
//    XCD-aware grouped order; split-K only when the grid cannot cover the CUs once.
// MARLIN_MI355X_DECODE="nt,depth,wpb,ksplit,occ" (nt 0 disables the decode kernel),
// MARLIN_MI355X_TILE="bm,nt,ch" (tiled kernel), MARLIN_MI355X_STREAM_BM / _STREAM_NT
// (multistage kernel) and MARLIN_MI355X_SPLIT_K override the choice (tuning).
Plan select_dense(int64_t M, int64_t N, int64_t K, int cus, const GemmLaunch& kinds) {
  const Overrides& ov = overrides();
  Plan p{};
  // Integer and fp8 weights with channelwise or >= 128-deep groups multiply raw codes
  // (integer-operand path): 64-column groups, three steps in flight.  fp4 weights and small
  // groups dequantize every weight (more VALU per byte): 32-column groups and four steps in
  // flight keep more waves streaming (measured on cfg4: 8.3 vs 11.4 us at M=1).
  const bool int_operand = kinds.fmt != FMT_MXFP4 && kinds.fmt != FMT_NVFP4 && kinds.gsm != GSM_SMALL;
  if (M <= 16) {
    int nt = int_operand ? 4 : 2, depth = int_operand ? 3 : 4, wpb = 4, ksplit = 1,
        occ = int_operand ? 3 : 1;
    // at most half as many 64-column groups as CUs: 32-column groups instead (twice the
    // workgroups, no cross-workgroup split; cfg1 4096x4096: 6.9 us against 12.7 us with
    // split K; N = 14336, 224 groups, stays at 64 columns: 9.5 against 11.9 us)
    if (int_operand && N / 64 <= cus / 2) nt = 2, depth = 4, occ = 1;
    // with no more 16-column groups than CUs, 16-column groups keep every CU streaming
    // (cfg1 4096x4096: 6.1 us against 6.8 us with 32-column groups on half the CUs), each
    // by a 16-wave workgroup that splits K into two steps per wave, all in flight at once
    // (cfg1 M = 16 / 1: 5.75 / 4.97 us against 6.27 / 5.91 us with four waves of eight
    // steps; the same form on fp4 weights or wider N was slower, so it stays here)
    if (int_operand && N % 16 == 0 && N / 16 <= cus) nt = 1, depth = 3, wpb = 16, occ = 1;
    // MXFP4 from four rows on: 64-column groups (cfg4 shape, M = 4 / 8 / 16: 9.1 / 9.0 / 9.6
    // against 9.9 / 10.0 / 10.4 us with 32-column groups; NVFP4 keeps 32 columns at every M)
    if (kinds.fmt == FMT_MXFP4 && M >= 4) nt = 4;
    if (ov.decode_set) {
      nt = ov.decode[0], depth = ov.decode[1], wpb = ov.decode[2], ksplit = ov.decode[3],
      occ = ov.decode[4];
    } else if (occ == 3) {
      // three waves per SIMD where the instance's registers fit that budget without
      // spilling (checked once per instance); the compiler's choice otherwise.  Up to eight
      // rows, two steps in flight at three waves per SIMD stream a little faster (cfg2
      // shape, M = 1 / 2 / 4 / 8: 18.9 / 19.1 / 19.4 / 19.9 against 19.3 / 19.5 / 19.9 /
      // 20.5 us with three; level at M = 16).  A spilling depth-2 instance falls back to
      // depth 3, whose one-wave-per-SIMD instance always exists.
      auto spills = [&](int d) {
        GemmLaunch q = kinds;
        q.bm = 16, q.nt = nt, q.ch = 1, q.depth = d, q.wpb = wpb, q.ksplit = true, q.occ = 3;
        return kernel_fit(q).spills;
      };
      if (M <= 8 && nt == 4 && depth == 3 && !spills(2)) depth = 2;
      else if (spills(depth)) occ = 1;
    }
    if (nt > 0 && N % (16 * nt) == 0) {
      const int64_t groups = N / (16 * nt);
      while (!ksplit && wpb > 1 && groups % wpb != 0) wpb /= 2;
      p.bm = 16;
      p.nt = nt;
      p.ch = 1;
      p.depth = depth;
      p.wpb = wpb;
      p.ksplit = ksplit;
      p.occ = occ;
      p.m_blocks = 1;
      p.n_blocks = (int)groups;  // split-K counters are per column group
      p.xcd_group_m = 0;
      GemmLaunch q = kinds;
      q.bm = p.bm;
      q.nt = nt;
      q.ch = 1;
      q.depth = depth;
      q.wpb = wpb;
      q.ksplit = ksplit != 0;
      q.occ = occ;
      const int64_t resident = (int64_t)blocks_per_cu(q) * cus;
      const int64_t blocks_n = ksplit ? groups : groups / wpb;
      const int steps = (int)(K / 128);
      int splits = 1;
      int64_t main_blocks = 0;
      if (blocks_n >= cus && blocks_n < resident) {
        // Every CU gets the same number of whole column groups; the groups left over are
        // split along K into about one small block per CU, so that no CU carries a whole
        // extra group (an extra group on a few CUs sets the span of the launch).
        main_blocks = blocks_n - blocks_n % cus;
        const int64_t left = blocks_n - main_blocks;
        if (left > 0) {
          const int min_steps = ksplit ? wpb : 1;
          splits = (int)std::min<int64_t>(std::min<int64_t>(cus / left, (resident - main_blocks) / left),
                                          steps / std::max(min_steps, 1));
          splits = std::max(splits, 1);
        }
        if (splits == 1) main_blocks = 0;
      } else if (blocks_n * 4 <= cus) {
        // far fewer groups than CUs: split K across blocks, as far as the device-scope
        // atomics of the partial sums stay cheap (about 64K per call; measured: splitting
        // cost more than it gained whenever a quarter of the CUs or more had a group)
        const int min_steps = 2 * (ksplit ? wpb : 1);  // per split
        if (steps >= 2 * min_steps)
          splits = (int)std::min<int64_t>(resident / blocks_n, steps / min_steps);
        const int64_t budget = std::max<int64_t>(1, (int64_t(1) << 16) / std::max<int64_t>(M * N, 1));
        splits = (int)std::min<int64_t>(splits, budget);
        splits = std::max(splits, 1);
      }
      if (ov.split_k >= 0) {
        splits = ov.split_k;
        main_blocks = 0;
      }
      splits = std::max(1, std::min(splits, std::max(steps, 1)));
      p.steps_per_split = steps == 0 ? 0 : (steps + splits - 1) / splits;
      p.splits = steps == 0 ? 1 : (steps + p.steps_per_split - 1) / p.steps_per_split;
      p.main_blocks = (int)main_blocks;
      p.grid = main_blocks + (blocks_n - main_blocks) * p.splits;
      return p;
    }
  }
  // The multistage kernel (all of K's operands three steps ahead): 16..64-row blocks up to
  // M = 128, 128-row blocks (one wave per SIMD, accumulators in AGPRs) beyond.
  if (ov.stream != 0 && M <= ov.stream_max_m) {
    int bm = M <= 16 ? 16 : (M <= 32 ? 32 : (M <= 128 ? 64 : 128));
    // per-32/16 group metadata for 48+ rows does not fit the register budget: 32-row blocks
    // up to M = 2048 for fp4 weights and 1024 for integer ones, the tiled kernel beyond
    // (measured on cfg4 MXFP4: 35 / 75 at M = 64 / 512 against 47 / 184 us tiled; M = 1536 /
    // 2048 / 4096: 154 / 204 / 417 against 201 / 203 / 400 us tiled)
    const bool fp4_fmt = kinds.fmt == FMT_MXFP4 || kinds.fmt == FMT_NVFP4;
    const int64_t small_group_max_m =
        ov.small_group_max_m >= 0 ? ov.small_group_max_m : (fp4_fmt ? 2048 : 1024);
    if (kinds.gsm == GSM_SMALL && bm >= 48 && M <= small_group_max_m)
      bm = 32;
    int nt = N % 256 == 0 ? 4 : (N % 128 == 0 ? 2 : 1);
    // 65..128 rows with at least one 256-column block per two CUs: one 128-row block (each
    // weight dequantized once, 32x32 MFMAs) instead of two 64-row blocks (cfg2 N = 34816,
    // M = 80 / 128: 79 / 82 against 90 / 93 us; N = 4096 / 8192 have too few blocks: 58 /
    // 89 against 41 / 71 us at M = 128)
    if (bm == 64 && M > 64 && nt == 4 && N / 256 >= cus / 2) bm = 128;
    // NVFP4 weights beyond 128 rows: 64-row x 128-column blocks, so each weight (whose
    // dequantization costs four times MXFP4's VALU) is dequantized for twice the rows (cfg4
    // shape, M = 192 / 256 / 320 / 512: 42.2 / 42.7 / 44.2 / 63.7 against 49.7 / 51.3 / 53.1 /
    // 67.1 us with 32 x 256 blocks).  MXFP4 stays on 32-row blocks: with its scale bytes kept
    // opaque until use (device_common.h) 32 x 256 blocks are level or ahead (M = 384 / 512 /
    // 768: 56.6 / 60.0 / 81.2 against 58.0 / 60.4 / 85.8 us with 64 x 128; M = 1024, K = N =
    // 4096: 47.2 against 50.8 us).
    const bool fp4_wide = kinds.fmt == FMT_NVFP4 && bm == 32 && M > 128 && N % 128 == 0;
    if (fp4_wide) bm = 64;
    // fp4 weights at 17..128 rows: 16-row blocks, 64 columns wide while that gives at most
    // three blocks per CU, else 128, with at most two K splits (cfg4 shape, MXFP4 M = 32 / 64
    // / 128: 17.3 / 25.1 / 32.7 against 24.5 / 28.0 / 44.5 us with 32-row blocks; NVFP4 M =
    // 64 / 128: 28.3 / 40.5 against 29.5 / 51.3 us; MXFP4 M = 64, K = N = 4096: 16.4 against
    // 26.1 us.  64 against 128 columns, one K split: M = 64 MXFP4 / NVFP4 18.6 / 22.9 against
    // 19.7 / 25.5 us; M = 96 / 128 MXFP4 31.7 / 37.4 against 26.8 / 27.4 us).  More rows per
    // block would dequantize each weight fewer times, but at these sizes the grid's width,
    // not the dequantization, sets the time.  (Integer weights with small groups are not
    // measured here and keep the general rule.)
    const bool small_group_narrow = (kinds.fmt == FMT_MXFP4 || kinds.fmt == FMT_NVFP4) &&
                                    M > 16 && M <= 128;
    if (small_group_narrow) {
      bm = 16;
      nt = (N % 128 == 0 && ((M + 15) / 16) * (N / 64) > 3 * (int64_t)cus) ? 2 : 1;
    }
    if (fp4_wide) nt = 2;
    if ((bm > 16 && nt == 1) || (bm == 128 && nt != 4)) nt = 0;  // not instantiated: tiled kernel
    if (ov.stream_nt >= 0) nt = ov.stream_nt;
    if (ov.stream_bm > 0) bm = ov.stream_bm;
    const bool small_meta_fits = !(kinds.gsm == GSM_SMALL && bm >= 48 && nt >= 4);
    if (nt > 0 && N % (64 * nt) == 0 && small_meta_fits) {
      p.bm = bm;
      p.nt = nt;
      p.ch = 1;
      p.stream = 1;
      p.m_blocks = (int)((M + bm - 1) / bm);
      p.n_blocks = (int)(N / (64 * nt));
      // (cfg3: groups of 8 block rows 588 against 605-615 us with 4; 16: 590-597 us)
      p.xcd_group_m = ov.xcd_group_m >= 0 ? ov.xcd_group_m : (bm >= 64 ? 8 : 0);
      GemmLaunch q = kinds;
      q.bm = bm;
      q.nt = nt;
      q.ch = 1;
      q.stream = true;
      const int64_t resident = (int64_t)blocks_per_cu(q) * cus;
      const int64_t base = (int64_t)p.m_blocks * p.n_blocks;
      const int steps = (int)(K / 128);
      int splits = 1;
      // Split K only while the partial sums stay few: each split adds M x N device-scope
      // atomics, which cost more than the idle CUs they fill from about half a million
      // outputs on (split 1 against the split choice: cfg4 MXFP4 M = 64 20.0 / 22.2 us, uint4
      // M = 128 N = 32768 85 / 111 us, uint8b128 M = 256 K = N = 4096 61 / 86 us; below the
      // limit splitting still wins: uint4 M = 64 K = N = 4096 40 / 43 us, M = 48 K = 8192
      // N = 2048 30 / 80 us, MXFP4 M = 64 K = N = 4096 14.0 / 16.3 us)
      if (base < resident && steps >= 8 && M * N <= (int64_t(1) << 19))
        splits = (int)std::min<int64_t>(resident / base, steps / 4);
      if (small_group_narrow) splits = std::min(splits, 2);
      if (ov.split_k >= 0) splits = ov.split_k;
      splits = std::max(1, std::min(splits, std::max(steps, 1)));
      p.steps_per_split = steps == 0 ? 0 : (steps + splits - 1) / splits;
      p.splits = steps == 0 ? 1 : (steps + p.steps_per_split - 1) / p.steps_per_split;
      p.grid = base * p.splits;
      return p;
    }
  }
  if (M <= 16) {
    p.bm = 16;
    p.nt = 1;
    p.ch = 2;
  } else if (M <= 32 && N % 128 == 0) {
    p.bm = 32;
    p.nt = 2;
    p.ch = 2;
  } else if (M <= 64 && N % 256 == 0) {
    p.bm = 64;
    p.nt = 4;
    p.ch = 1;
  } else if (N % 256 == 0) {
    p.bm = 128;
    p.nt = 4;
    p.ch = 1;
  } else {
    p.bm = 16;  // narrowest tile that divides N (N % 64 == 0 is guaranteed)
    p.nt = 1;
    p.ch = 2;
  }
  if (ov.tile_set) {
    p.bm = ov.tile[0];
    p.nt = ov.tile[1];
    p.ch = ov.tile[2];
  }
  p.m_blocks = (int)((M + p.bm - 1) / p.bm);
  p.n_blocks = (int)(N / (64 * p.nt));
  p.xcd_group_m = p.bm >= 64 ? 4 : 0;
  if (ov.xcd_group_m >= 0) p.xcd_group_m = ov.xcd_group_m;
  const int steps = (int)(K / (128 * p.ch));
  const int64_t base = (int64_t)p.m_blocks * p.n_blocks;
  const int64_t target = (p.bm <= 32) ? (int64_t)cus * 4 : (int64_t)cus;
  int splits = 1;
  if (base < target && steps > 1) {
    splits = (int)std::min<int64_t>((target + base - 1) / base, steps);
    const int min_steps = (p.bm <= 32) ? 2 : 4;
    splits = std::max(1, std::min(splits, std::max(1, steps / min_steps)));
  }
  if (ov.split_k >= 0) splits = ov.split_k;
  if (steps == 0) splits = 1;
  splits = std::max(1, std::min(splits, std::max(steps, 1)));
  p.steps_per_split = steps == 0 ? 0 : (steps + splits - 1) / splits;
  p.splits = steps == 0 ? 1 : (steps + p.steps_per_split - 1) / p.steps_per_split;
  p.grid = (int64_t)p.m_blocks * p.n_blocks * p.splits;
  return p;
}

hipError_t dispatch_gemm(const GemmLaunch& l, const GemmParams& p, hipStream_t s) {
#define MMI_CASE_FMT(E, F) \
  case E: return l.bf16 ? launch_gemm_##F##_bf16(l, p, s) : launch_gemm_##F##_f16(l, p, s);
  switch (l.fmt) {
    MMI_CASE_FMT(FMT_U4B8, u4b8)
    MMI_CASE_FMT(FMT_U4, u4)
    MMI_CASE_FMT(FMT_U8B128, u8b128)
    MMI_CASE_FMT(FMT_U8, u8)
    MMI_CASE_FMT(FMT_U4Z, u4z)
    MMI_CASE_FMT(FMT_U8Z, u8z)
    MMI_CASE_FMT(FMT_FP8, fp8)
    MMI_CASE_FMT(FMT_MXFP4, mxfp4)
    MMI_CASE_FMT(FMT_NVFP4, nvfp4)
  }
#undef MMI_CASE_FMT
  return hipErrorInvalidValue;
}

// Validation shared by marlin_gemm, moe_wna16_marlin_gemm and marlin_dequantize for the
// weight metadata (reference marlin.cu:107-383, ops.cu:134-402).  Returns the format.
struct MetaCheck {
  int fmt;
  int group_size;  // -1 channelwise
  int gsm;
  int group_shift;
  int zp_packed;  // uint4/uint8 zero points are integer codes packed along N
};

MetaCheck check_weight_meta(int64_t b_type_id, marlin_dtype_t a_dtype,
                            marlin_dtype_t scales_dtype, int64_t scales_numel,
                            int64_t num_groups, int64_t per_expert, const float* global_scale,
                            int64_t global_scale_numel, int64_t expected_global,
                            const void* b_zeros, marlin_dtype_t zeros_dtype,
                            int64_t zeros_numel, int is_zp_float, int64_t size_n,
                            int64_t size_k) {
  MetaCheck mc{};
  mc.fmt = fmt_from_type(b_type_id, scales_dtype);
  const bool fp4 = mc.fmt == FMT_MXFP4 || mc.fmt == FMT_NVFP4;
  if (!fp4) {
    check(scales_dtype == a_dtype,
          "b_scales must have the activation dtype (float16 or bfloat16), except FP4 uses "
          "float8_e4m3fn scales for NVFP4 or float8_e8m0fnu scales for MXFP4.");
  }
  check(num_groups >= 1, "b_scales has no groups");
  check(scales_numel == per_expert * num_groups * size_n, "b_scales numel = ", scales_numel,
        " does not match num_groups * size_n = ", num_groups * size_n);
  int group_size = -1;
  if (num_groups > 1) {
    check(size_k % num_groups == 0, "size_k = ", size_k,
          ", is not divisible by b_scales.size(0) = ", num_groups);
    group_size = (int)(size_k / num_groups);
  }
  mc.group_size = group_size;

  const bool has_global = global_scale_numel > 0;
  if (has_global) {
    check(mc.fmt == FMT_NVFP4, "global_scale is supported only for nvfp4 format.");
    check(global_scale != nullptr, "global_scale pointer is null");
    check(global_scale_numel == expected_global, "nvfp4 expects global_scale numel = ",
          expected_global, ". Got global_scale.numel() = ", global_scale_numel);
  } else {
    check(mc.fmt != FMT_NVFP4, "the global_scale parameter must be passed for nvfp4 format.");
  }

  const bool has_zp = zeros_numel > 0;
  check(!has_zp || mc.fmt == FMT_U4 || mc.fmt == FMT_U8,
        "zero-point metadata is supported only for uint4 and uint8 weights.");
  if (has_zp) {
    check(b_zeros != nullptr, "b_zeros pointer is null");
    if (is_zp_float) {
      check(zeros_dtype == a_dtype,
            "uint4/uint8 float zero points must have the activation dtype (float16 or "
            "bfloat16).");
      check(zeros_numel == scales_numel, "b_zeros numel = ", zeros_numel,
            " is not num_groups * size_n = ", scales_numel / per_expert);
    } else {
      // integer zero points packed along N, 32/bits per int32 word (upstream marlin's
      // is_zp_float=false mode; the SM70 reference rejects it, marlin.cu:336-339)
      const int64_t zpack = 32 / fmt_bits(mc.fmt);
      check(zeros_dtype == MARLIN_DTYPE_INT32,
            "packed integer zero points (is_zp_float=false) must be int32.");
      check(size_n % zpack == 0, "size_n must be divisible by the zero-point pack factor");
      check(zeros_numel * zpack == scales_numel, "b_zeros numel = ", zeros_numel,
            " is not num_groups * size_n / pack_factor = ", scales_numel / zpack / per_expert);
      mc.zp_packed = 1;
    }
  } else {
    check(!is_zp_float, "is_zp_float is true but b_zeros was not provided.");
  }
  if (mc.fmt == FMT_U4 || mc.fmt == FMT_U8) {
    check(has_zp, mc.fmt == FMT_U4 ? "uint4" : "uint8",
          " path requires zero points (float with is_zp_float=true, or packed int32).");
  }

  // group-size support per format (reference marlin.cu:434-493, sm70_marlin_gemm.cuh:98-141)
  if (mc.fmt == FMT_NVFP4) {
    check(group_size == 16, "nvfp4 supports only group_size 16. Got ", group_size);
  } else if (mc.fmt == FMT_MXFP4) {
    check(group_size == 32, "mxfp4 supports only group_size 32 when global_scale is not "
                            "provided. Got ", group_size);
  } else if (mc.fmt == FMT_FP8) {
    check(group_size == -1 || group_size == 128,
          "fp8_e4m3 supports only group_size -1 or 128. Got ", group_size);
  } else {
    check(group_size == -1 || (group_size >= 32 && ilog2_exact(group_size) >= 0),
          "unsupported group_size = ", group_size,
          " (supported: -1 or a power of two >= 32)");
  }
  if (group_size == -1) {
    mc.gsm = GSM_CHANNEL;
    mc.group_shift = 0;
  } else {
    mc.group_shift = ilog2_exact(group_size);
    mc.gsm = group_size >= 128 ? GSM_BIG : GSM_SMALL;
  }
  // integer zero points run the integer-zero instances (the codes are staged as 16 bits)
  if (mc.zp_packed) mc.fmt = mc.fmt == FMT_U4 ? FMT_U4Z : FMT_U8Z;
  return mc;
}

// ---- dense plan cache ---------------------------------------------------------------------
// The selector's choice for one (device, format, dtype, group mode, M, N, K): the plan and
// the kernel instance it launches.  Computed once per key (the selector queries occupancy
// and register spills on first use), so a repeated shape costs one hash lookup.
struct DensePlan {
  Plan plan;
  GemmLaunch launch;
};

struct PlanKey {
  int dev, fmt, bf16, gsm;
  int64_t m, n, k;
  bool operator==(const PlanKey& o) const {
    return dev == o.dev && fmt == o.fmt && bf16 == o.bf16 && gsm == o.gsm && m == o.m &&
           n == o.n && k == o.k;
  }
};
struct PlanKeyHash {
  size_t operator()(const PlanKey& x) const {
    uint64_t h = 1469598103934665603ull;
    for (int64_t v : {(int64_t)x.dev, (int64_t)x.fmt, (int64_t)x.bf16, (int64_t)x.gsm, x.m, x.n, x.k})
      h = (h ^ (uint64_t)v) * 1099511628211ull;
    return (size_t)h;
  }
};

const char* fmt_name(int fmt) {
  static const char* names[] = {"uint4b8", "uint4", "uint8b128", "uint8", "fp8_e4m3", "mxfp4", "nvfp4"};
  return (fmt >= 0 && fmt < 7) ? names[fmt] : "?";
}

DensePlan dense_plan(int dev, int fmt, bool bf16, int gsm, int64_t M, int64_t N, int64_t K) {
  static std::mutex mu;
  static std::unordered_map<PlanKey, DensePlan, PlanKeyHash> cache;
  const PlanKey key{dev, fmt, (int)bf16, gsm, M, N, K};
  {
    std::lock_guard<std::mutex> lk(mu);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
  }
  GemmLaunch l{};
  l.fmt = fmt;
  l.bf16 = bf16;
  l.gsm = gsm;
  DensePlan d{};
  d.plan = select_dense(M, N, K, device_cu_count(dev), l);
  l.bm = d.plan.bm;
  l.nt = d.plan.nt;
  l.ch = d.plan.ch;
  l.depth = d.plan.depth;
  l.wpb = d.plan.wpb;
  l.ksplit = d.plan.ksplit != 0;
  l.occ = d.plan.occ;
  l.stream = d.plan.stream != 0;
  l.moe = false;
  l.grid = (unsigned)d.plan.grid;
  d.launch = l;
  if (!instantiated(l)) {
    std::ostringstream os;
    os << "no " << fmt_name(fmt) << (bf16 ? "/bf16" : "/fp16") << " kernel instance for the "
       << "selected configuration (bm " << l.bm << ", nt " << l.nt << ", ch " << l.ch
       << ", depth " << l.depth << ", wpb " << l.wpb << ", ksplit " << l.ksplit << ", occ "
       << l.occ << ", stream " << l.stream << ")";
    if (overrides().any) os << "; a MARLIN_MI355X_* tuning override selects a configuration "
                               "this build does not instantiate";
    check_supported(false, os.str());
  }
  std::lock_guard<std::mutex> lk(mu);
  if (cache.size() >= (1u << 16)) cache.clear();  // bound the cache for callers with many shapes
  cache.emplace(key, d);
  return d;
}

// A validated dense call: its plan, the kernel parameters (all but the split-K scratch)
// and the scratch it needs.
struct DenseCall {
  bool empty;  // nothing to compute (M = 0 or N = 0)
  int dev;
  DensePlan plan;
  GemmParams params;
  size_t ws_elems;     // fp32 partial sums (splits > 1)
  size_t ws_counters;  // arrival counters (splits > 1)
  // act-order: A's columns are gathered by perm into a staging buffer first
  bool act_order;
  const int* perm;
  const int* g_idx;
  int act_group_shift;  // log2(group size), -1 channelwise
};

// Validation of marlin_gemm (reference marlin.cu:83-506) and everything the launch needs
// except the split-K scratch.
DenseCall check_dense(const void* a, marlin_dtype_t a_dtype, int64_t a_row_stride, void* c,
                      const int32_t* b_q_weight, int64_t b_q_weight_numel, const void* b_bias,
                      int64_t b_bias_numel, const void* b_scales, marlin_dtype_t b_scales_dtype,
                      int64_t b_scales_numel, int64_t num_groups, int64_t a_scales_numel,
                      const float* global_scale, int64_t global_scale_numel, const void* b_zeros,
                      marlin_dtype_t b_zeros_dtype, int64_t b_zeros_numel, const int32_t* g_idx,
                      int64_t g_idx_numel, const int32_t* perm, int64_t perm_numel,
                      int64_t b_type_id, int64_t size_m, int64_t size_n, int64_t size_k,
                      int is_zp_float, int is_k_full) {
  const bool act_order = g_idx_numel > 0 || perm_numel > 0;
  if (act_order) {
    // act-order (upstream gptq_marlin; the SM70 reference rejects it, marlin.cu:95-102):
    // weights repacked with perm = argsort(g_idx), A gathered by perm before the GEMM
    check(g_idx_numel == size_k && perm_numel == size_k, "act_order needs g_idx and perm with "
          "size_k = ", size_k, " entries each (got ", g_idx_numel, " and ", perm_numel, ")");
    check(g_idx != nullptr && perm != nullptr, "null g_idx / perm pointer");
    check_supported(is_k_full, "act_order with is_k_full=false (a row-parallel K shard) is not "
                               "supported on this build");
  }
  check_supported(is_half_type(a_dtype),
                  "only float16 and bfloat16 activations are supported (8-bit activations are "
                  "not implemented).");
  check(a_scales_numel == 0, "a_scales can only be used for 8bit activation.");
  const MetaCheck mc = check_weight_meta(b_type_id, a_dtype, b_scales_dtype, b_scales_numel,
                                         num_groups, 1, global_scale, global_scale_numel, 1,
                                         b_zeros, b_zeros_dtype, b_zeros_numel, is_zp_float,
                                         size_n, size_k);
  if (act_order)
    check_supported(mc.fmt == FMT_U4B8 || mc.fmt == FMT_U4 || mc.fmt == FMT_U8B128 ||
                        mc.fmt == FMT_U8 || fmt_int_zero(mc.fmt),
                    "act_order is supported for integer weight types only");
  const int bits = fmt_bits(mc.fmt);
  const int64_t pack = 32 / bits;
  check(size_k % 16 == 0, "size_k = ", size_k, " is not divisible by tile_size = ", 16);
  check(b_q_weight_numel == size_k * size_n / pack, "Shape mismatch: b_q_weight numel = ",
        b_q_weight_numel, ", size_k * size_n / pack_factor = ", size_k * size_n / pack);
  check(size_k % 32 == 0, "marlin_gemm requires size_k % 32 == 0.");
  check(size_n % 64 == 0, "marlin_gemm requires size_n % 64 == 0. size_n = ", size_n,
        ", min_thread_n = ", 64);
  check(a_row_stride % 8 == 0, "A.stride(0) must divisible by 8");
  check(((uintptr_t)a) % 16 == 0, "A must aligned to 16 bytes");
  check(b_bias_numel == 0 || b_bias_numel == size_n, "b_bias.size(0) != size_n");
  check(size_m >= 0 && size_m <= INT32_MAX, "size_m out of range");
  DenseCall d{};
  d.empty = size_m == 0 || size_n == 0;
  d.act_order = act_order;
  d.perm = perm;
  d.g_idx = g_idx;
  d.act_group_shift = mc.group_size > 0 ? mc.group_shift : -1;
  if (d.empty) return d;
  check(size_k > 0, "size_k must be positive");
  check(a && c && b_q_weight && b_scales, "null tensor pointer");

  check_hip(hipGetDevice(&d.dev), "hipGetDevice");
  d.plan = dense_plan(d.dev, mc.fmt, a_dtype == MARLIN_DTYPE_BFLOAT16, mc.gsm, size_m, size_n,
                      size_k);
  const Plan& plan = d.plan.plan;
  GemmParams& p = d.params;
  p.a = a;
  p.a_stride = a_row_stride;
  p.c = c;
  p.b = reinterpret_cast<const uint32_t*>(b_q_weight);
  p.b_expert_stride = 0;
  p.scales = b_scales;
  p.zeros = b_zeros_numel ? b_zeros : nullptr;
  p.meta_expert_stride = 0;
  p.bias = b_bias_numel ? b_bias : nullptr;
  p.global_scale = global_scale;
  p.alpha_exp = 7 - (a_dtype == MARLIN_DTYPE_FLOAT16 ? 14 : 126);
  p.M = (int)size_m;
  p.N = (int)size_n;
  p.K = (int)size_k;
  p.group_shift = mc.group_shift;
  p.splits = plan.splits;
  p.steps_per_split = plan.steps_per_split;
  p.main_blocks = plan.main_blocks;
  p.num_n_blocks = plan.n_blocks;
  p.num_m_blocks = plan.m_blocks;
  p.xcd_group_m = plan.xcd_group_m;
  if (plan.splits > 1) {
    d.ws_elems = (size_t)size_m * size_n;
    d.ws_counters = (size_t)plan.m_blocks * plan.n_blocks;
  }
  return d;
}

}  // namespace

extern "C" {

const char* marlin_get_last_error(void) { return g_last_error.c_str(); }

int marlin_abi_version(void) { return MARLIN_MI355X_ABI_VERSION; }

marlin_status_t marlin_gptq_marlin_repack(const int32_t* b_q_weight, int64_t b_q_weight_numel,
                                          const int32_t* perm, int64_t perm_numel,
                                          int64_t size_k, int64_t size_n, int64_t num_bits,
                                          int is_a_8bit, int32_t* out, int64_t out_numel,
                                          marlin_stream_t stream) {
  return guarded([&] {
    check(size_k % 16 == 0, "size_k = ", size_k, " is not divisible by tile_k_size = ", 16);
    check(size_n % 64 == 0, "size_n = ", size_n, " is not divisible by tile_n_size = ", 64);
    check(num_bits == 4 || num_bits == 8, "num_bits must be 4 or 8. Got = ", num_bits);
    // (the reference has no act-order form of the 8-bit-activation layout,
    // gptq_marlin_repack.cu:250, 377-396)
    check(!(is_a_8bit && perm_numel != 0), "Unsupported repack config: num_bits = ", num_bits,
          ", has_perm = 1, is_a_8bit = 1");
    check(size_k % 32 == 0, "size_k = ", size_k,
          " is not divisible by 32 (the gfx950 layout packs 32-deep MFMA blocks)");
    const int64_t pack = 32 / num_bits;
    check(b_q_weight_numel == size_k / pack * size_n, "Shape mismatch: b_q_weight numel = ",
          b_q_weight_numel, ", expected size_k / pack_factor * size_n = ", size_k / pack * size_n);
    check(out_numel == size_k * size_n / pack, "out numel = ", out_numel, ", expected ",
          size_k * size_n / pack);
    check(perm_numel == 0 || perm_numel == size_k, "perm numel = ", perm_numel,
          " must be 0 or size_k = ", size_k);
    if (size_k == 0 || size_n == 0) return;
    check(b_q_weight != nullptr && out != nullptr, "null tensor pointer");
    if (is_a_8bit) {
      check_hip(launch_a8_repack(reinterpret_cast<const uint32_t*>(b_q_weight), false,
                                 reinterpret_cast<uint32_t*>(out), size_k, size_n, (int)num_bits,
                                 (hipStream_t)stream),
                "gptq_marlin_repack launch");
      return;
    }
    check_hip(launch_gptq_repack(reinterpret_cast<const uint32_t*>(b_q_weight),
                                 perm_numel ? perm : nullptr, reinterpret_cast<uint32_t*>(out),
                                 size_k, size_n, (int)num_bits, (hipStream_t)stream),
              "gptq_marlin_repack launch");
  });
}

marlin_status_t marlin_awq_marlin_repack(const int32_t* b_q_weight, int64_t b_q_weight_numel,
                                         int64_t size_k, int64_t size_n, int64_t num_bits,
                                         int is_a_8bit, int32_t* out, int64_t out_numel,
                                         marlin_stream_t stream) {
  return guarded([&] {
    check(size_k % 16 == 0, "size_k = ", size_k, " is not divisible by tile_k_size = ", 16);
    check(size_n % 64 == 0, "size_n = ", size_n, " is not divisible by tile_n_size = ", 64);
    check(num_bits == 4 || num_bits == 8, "num_bits must be 4 or 8. Got = ", num_bits);
    check(size_k % 32 == 0, "size_k = ", size_k,
          " is not divisible by 32 (the gfx950 layout packs 32-deep MFMA blocks)");
    const int64_t pack = 32 / num_bits;
    check(b_q_weight_numel == size_k * (size_n / pack), "Shape mismatch: b_q_weight numel = ",
          b_q_weight_numel, ", expected size_k * size_n / pack_factor = ", size_k * (size_n / pack));
    check(out_numel == size_k * size_n / pack, "out numel = ", out_numel, ", expected ",
          size_k * size_n / pack);
    if (size_k == 0 || size_n == 0) return;
    check(b_q_weight != nullptr && out != nullptr, "null tensor pointer");
    if (is_a_8bit) {
      check_hip(launch_a8_repack(reinterpret_cast<const uint32_t*>(b_q_weight), true,
                                 reinterpret_cast<uint32_t*>(out), size_k, size_n, (int)num_bits,
                                 (hipStream_t)stream),
                "awq_marlin_repack launch");
      return;
    }
    check_hip(launch_awq_repack(reinterpret_cast<const uint32_t*>(b_q_weight),
                                reinterpret_cast<uint32_t*>(out), size_k, size_n, (int)num_bits,
                                (hipStream_t)stream),
              "awq_marlin_repack launch");
  });
}

marlin_status_t marlin_int4_fp8_preprocess(const int32_t* qweight, int64_t qweight_rows,
                                           int64_t qweight_cols, const int32_t* qzeros,
                                           int64_t qzeros_rows, int64_t qzeros_cols, int32_t* out,
                                           marlin_stream_t stream) {
  return guarded([&] {
    const int64_t numel = qweight_rows * qweight_cols;
    check(qweight_rows >= 0 && qweight_cols >= 0, "qweight shape must be non-negative");
    int group_size = 1;
    if (qzeros == nullptr) {
      check(numel * 8 % 256 == 0, "qweight.numel() * 8 % 256 != 0");
    } else {
      // AWQ weights [size_k, size_n / 8] with zero points [size_k / group_size, size_n / 8]
      check(qweight_rows % 32 == 0, "size_k % 32 != 0");
      check(qzeros_rows > 0, "qzeros has no rows");
      check(qweight_cols == qzeros_cols, "qweight.size(1) != qzeros.size(1)");
      check(qweight_rows % qzeros_rows == 0, "qweight.size(0) % qzeros.size(0) != 0");
      group_size = (int)(qweight_rows / qzeros_rows);
      check(group_size % 8 == 0, "group_size % 8 != 0");
    }
    if (numel == 0) return;
    check(qweight != nullptr && out != nullptr, "null tensor pointer");
    check_hip(launch_int4_fp8_preprocess(reinterpret_cast<const uint32_t*>(qweight),
                                         reinterpret_cast<uint32_t*>(out),
                                         reinterpret_cast<const uint32_t*>(qzeros), numel,
                                         qzeros ? qweight_cols : 1, group_size,
                                         (hipStream_t)stream),
              "marlin_int4_fp8_preprocess launch");
  });
}

marlin_status_t marlin_gemm(const void* a, marlin_dtype_t a_dtype, int64_t a_row_stride,
                            void* c, const int32_t* b_q_weight, int64_t b_q_weight_numel,
                            const void* b_bias, int64_t b_bias_numel,
                            const void* b_scales, marlin_dtype_t b_scales_dtype,
                            int64_t b_scales_numel, int64_t num_groups,
                            int64_t a_scales_numel,
                            const float* global_scale, int64_t global_scale_numel,
                            const void* b_zeros, marlin_dtype_t b_zeros_dtype,
                            int64_t b_zeros_numel, const int32_t* g_idx, int64_t g_idx_numel,
                            const int32_t* perm, int64_t perm_numel, void* workspace,
                            int64_t workspace_bytes, int64_t b_type_id, int64_t size_m,
                            int64_t size_n, int64_t size_k, int is_k_full, int use_atomic_add,
                            int use_fp32_reduce, int is_zp_float, marlin_stream_t stream) {
  (void)workspace;
  (void)workspace_bytes;
  (void)use_atomic_add;
  (void)use_fp32_reduce;
  return guarded([&] {
    const DenseCall d = check_dense(a, a_dtype, a_row_stride, c, b_q_weight, b_q_weight_numel,
                                    b_bias, b_bias_numel, b_scales, b_scales_dtype,
                                    b_scales_numel, num_groups, a_scales_numel, global_scale,
                                    global_scale_numel, b_zeros, b_zeros_dtype, b_zeros_numel,
                                    g_idx, g_idx_numel, perm, perm_numel, b_type_id, size_m,
                                    size_n, size_k, is_zp_float, is_k_full);
    if (d.empty) return;
    hipStream_t s = (hipStream_t)stream;
    GemmParams p = d.params;
    if (fmt_int_zero(d.plan.launch.fmt))
      p.zeros = stage_int_zeros(d.dev, s, p.zeros, fmt_bits(d.plan.launch.fmt),
                                (int64_t)num_groups * size_n);
    if (d.act_order) {
      // A[:, perm] into a staging buffer (rows of size_k), then the plain grouped GEMM: the
      // repacked weights' row j is source row perm[j], whose group is j / group_size
      void* staged = get_staging(kStageActOrder, d.dev, s, (size_t)size_m * size_k * 2);
      check_hip(launch_permute_cols(a, a_dtype == MARLIN_DTYPE_BFLOAT16, a_row_stride, d.perm,
                                    d.g_idx, d.act_group_shift, size_k, size_m, staged, s),
                "act_order permute launch");
      p.a = staged;
      p.a_stride = size_k;
    }
    if (d.plan.plan.splits > 1) {
      Workspace& w = get_workspace(d.dev, s, d.ws_elems, d.ws_counters);
      p.ws = w.ws;
      p.counters = w.counters;
    }
    check_hip(dispatch_gemm(d.plan.launch, p, s), "marlin_gemm launch");
  });
}

marlin_status_t marlin_gemm_no_alloc(const void* a, marlin_dtype_t a_dtype, int64_t a_row_stride,
                                     void* c, const int32_t* b_q_weight, int64_t b_q_weight_numel,
                                     const void* b_bias, int64_t b_bias_numel,
                                     const void* b_scales, marlin_dtype_t b_scales_dtype,
                                     int64_t b_scales_numel, int64_t num_groups,
                                     int64_t a_scales_numel, const float* global_scale,
                                     int64_t global_scale_numel, const void* b_zeros,
                                     marlin_dtype_t b_zeros_dtype, int64_t b_zeros_numel,
                                     int64_t g_idx_numel, int64_t perm_numel, int64_t b_type_id,
                                     int64_t size_m, int64_t size_n, int64_t size_k,
                                     int is_zp_float, marlin_stream_t stream) {
  return guarded([&] {
    check_supported(g_idx_numel == 0 && perm_numel == 0,
                    "marlin_gemm_no_alloc does not support act_order (its A staging buffer "
                    "would need an allocation); use marlin_gemm");
    const DenseCall d = check_dense(a, a_dtype, a_row_stride, c, b_q_weight, b_q_weight_numel,
                                    b_bias, b_bias_numel, b_scales, b_scales_dtype,
                                    b_scales_numel, num_groups, a_scales_numel, global_scale,
                                    global_scale_numel, b_zeros, b_zeros_dtype, b_zeros_numel,
                                    nullptr, 0, nullptr, 0, b_type_id, size_m, size_n, size_k,
                                    is_zp_float, 1);
    if (d.empty) return;
    check_supported(!fmt_int_zero(d.plan.launch.fmt),
                    "marlin_gemm_no_alloc does not support packed integer zero points (their "
                    "16-bit staging would need an allocation); use marlin_gemm");
    hipStream_t s = (hipStream_t)stream;
    uint32_t* base = scratch_on_device(d.dev, s);
    GemmParams p = d.params;
    if (d.plan.plan.splits > 1) {
      check(d.ws_elems <= kScratchPartials && d.ws_counters <= kScratchCounters,
            "marlin_gemm_no_alloc: this shape splits K and needs ", d.ws_elems,
            " fp32 partial sums (size_m * size_n) and ", d.ws_counters,
            " counters; the static scratch holds ", kScratchPartials, " and ",
            kScratchCounters);
      p.ws = reinterpret_cast<float*>(base);
      p.counters = reinterpret_cast<int*>(base + kScratchPartials);
    }
    check_hip(dispatch_gemm(d.plan.launch, p, s), "marlin_gemm_no_alloc launch");
  });
}

marlin_status_t marlin_moe_align_block_size(const void* topk_ids, marlin_dtype_t topk_ids_dtype,
                                            int64_t numel, int64_t num_experts,
                                            int64_t block_size, int32_t* sorted_token_ids,
                                            int64_t sorted_numel, int32_t* expert_ids,
                                            int64_t expert_ids_numel,
                                            int32_t* num_tokens_post_pad,
                                            const int32_t* expert_map, int64_t expert_map_numel,
                                            marlin_stream_t stream) {
  return guarded([&] {
    check(topk_ids_dtype == MARLIN_DTYPE_INT32 || topk_ids_dtype == MARLIN_DTYPE_INT64,
          "topk_ids must be int32 or int64");
    check(num_experts >= 1, "num_experts must be positive");
    const int64_t padded_num_experts = (num_experts + 63) / 64 * 64;
    check(padded_num_experts <= 1024, "padded_num_experts must be at most 1024");
    check(block_size >= 1, "block_size must be positive");
    check(numel >= 0 && numel < INT32_MAX, "topk_ids numel out of range");
    // the padded total reaches numel + E * (block_size - 1) in the worst case; a shorter
    // buffer would drop routes (the reference sizes it so: moe_align_block_size.py:15)
    const int64_t max_padded = numel + num_experts * (block_size - 1);
    check(sorted_numel >= max_padded, "sorted_token_ids must hold numel + num_experts * "
          "(block_size - 1) = ", max_padded, " entries, got ", sorted_numel);
    check(expert_ids_numel >= (max_padded + block_size - 1) / block_size,
          "experts_ids must hold ceil(max_num_tokens_padded / block_size) = ",
          (max_padded + block_size - 1) / block_size, " entries, got ", expert_ids_numel);
    check(expert_map_numel == 0 || expert_map_numel >= num_experts,
          "expert_map must cover num_experts entries");
    check(sorted_token_ids && expert_ids && num_tokens_post_pad, "null output pointer");
    check(numel == 0 || topk_ids, "null topk_ids pointer");
    check_hip(launch_moe_align(topk_ids, topk_ids_dtype == MARLIN_DTYPE_INT64, numel,
                               (int)num_experts, (int)block_size, sorted_token_ids, sorted_numel,
                               expert_ids, expert_ids_numel, num_tokens_post_pad,
                               expert_map_numel ? expert_map : nullptr, (hipStream_t)stream),
              "moe_align_block_size launch");
  });
}

static marlin_status_t moe_gemm(bool gated,
    
    const void* a, marlin_dtype_t a_dtype, void* c, const int32_t* b_q_weight,
    int64_t b_q_weight_numel, int64_t num_experts, const void* b_bias, int64_t b_bias_numel,
    const void* b_scales, marlin_dtype_t b_scales_dtype, int64_t b_scales_numel,
    int64_t num_groups, int64_t a_scales_numel, const float* global_scale,
    int64_t global_scale_numel, const void* b_zeros, marlin_dtype_t b_zeros_dtype,
    int64_t b_zeros_numel, int64_t g_idx_numel, int64_t perm_numel, void* workspace,
    int64_t workspace_bytes, const int32_t* sorted_token_ids, int64_t sorted_numel,
    const int32_t* expert_ids, int64_t expert_ids_numel,
    const int32_t* num_tokens_past_padded, const float* topk_weights,
    int64_t topk_weights_numel, int64_t moe_block_size, int64_t top_k, int mul_topk_weights,
    int64_t b_type_id, int64_t size_m, int64_t size_n, int64_t size_k, int is_k_full,
    int use_atomic_add, int use_fp32_reduce, int is_zp_float, int64_t thread_k,
    int64_t thread_n, int64_t blocks_per_sm, marlin_stream_t stream) {
  (void)workspace;
  (void)workspace_bytes;
  (void)is_k_full;
  (void)use_atomic_add;
  (void)use_fp32_reduce;
  (void)thread_k;
  (void)thread_n;
  (void)blocks_per_sm;
  return guarded([&] {
    check(g_idx_numel == 0, "moe_wna16_marlin_gemm does not support act_order g_idx.");
    check(perm_numel == 0, "moe_wna16_marlin_gemm does not support act_order perm.");
    check_supported(is_half_type(a_dtype),
                    "only float16 and bfloat16 activations are supported (8-bit activations are "
                    "not implemented).");
    check(a_scales_numel == 0, "a_scales can only be used for 8bit activation.");
    if (moe_block_size != 8) {
      check(moe_block_size % 16 == 0, "unsupported moe_block_size=", moe_block_size);
      check(moe_block_size >= 16 && moe_block_size <= 64, "unsupported moe_block_size=",
            moe_block_size);
    }
    check(num_experts >= 1, "num_experts must be positive");
    const MetaCheck mc = check_weight_meta(b_type_id, a_dtype, b_scales_dtype, b_scales_numel,
                                           num_groups, num_experts, global_scale,
                                           global_scale_numel, num_experts, b_zeros,
                                           b_zeros_dtype, b_zeros_numel, is_zp_float, size_n,
                                           size_k);
    const int bits = fmt_bits(mc.fmt);
    const int64_t pack = 32 / bits;
    check(size_k % 16 == 0, "size_k = ", size_k, " is not divisible by tile_size = ", 16);
    check(b_q_weight_numel == num_experts * size_k * size_n / pack,
          "Shape mismatch: b_q_weight numel = ", b_q_weight_numel,
          ", expected num_experts * size_k * size_n / pack_factor = ",
          num_experts * size_k * size_n / pack);
    check(size_k % 32 == 0, "moe_wna16_marlin_gemm requires size_k % 32 == 0.");
    check(size_n % 64 == 0, "size_n = ", size_n, ", is not divisible by min_thread_n = ", 64);
    check(b_bias_numel == 0 || b_bias_numel == num_experts * size_n,
          "b_bias must be [num_experts, size_n]");
    check(top_k >= 1, "top_k must be positive");
    check(!mul_topk_weights || topk_weights_numel >= size_m * top_k,
          "topk_weights must hold size_m * top_k values");
    check(((uintptr_t)a) % 16 == 0, "A must aligned to 16 bytes");
    check(size_k % 8 == 0, "A row stride must be divisible by 8");
    check((int64_t)size_m * top_k <= INT32_MAX, "size_m * top_k out of range");
    check(expert_ids_numel >= 1, "expert_ids is empty");
    if (size_m == 0 || size_n == 0 || sorted_numel == 0) return;
    check(a && c && b_q_weight && b_scales && sorted_token_ids && expert_ids &&
              num_tokens_past_padded,
          "null tensor pointer");

    hipStream_t s = (hipStream_t)stream;
    int dev = 0;
    check_hip(hipGetDevice(&dev), "hipGetDevice");
    const int cus = device_cu_count(dev);

    const Overrides& ov = overrides();
    const int bm = moe_block_size <= 16 ? 16 : (int)moe_block_size;  // 8 -> 16 rows
    // column blocks of the multistage kernel: 4 waves x nt n16 tiles; the widest that divides
    // size_n (the reference requires size_n % 64, ops.cu:390-392)
    int nt = size_n % 256 == 0 ? 4 : (size_n % 128 == 0 ? 2 : 1);
    if (ov.moe_nt > 0 && size_n % (64 * ov.moe_nt) == 0) nt = ov.moe_nt;
    // Moe blocks that can hold routes: every expert with routes has at least one route, so
    // there are at most (routes + min(routes, E) (bs - 1)) / bs of them (expert ids index the
    // num_experts weight slabs).  sorted_token_ids is sized for E (bs - 1) padding slots; with
    // fewer routes than experts the blocks past this bound could only launch workgroups that
    // read the padded total and exit (T = 16, E = 256, bs = 64: 128 instead of 254 blocks).
    const int64_t routes = size_m * top_k;
    const int64_t live_bound =
        (routes + std::min<int64_t>(routes, num_experts) * (moe_block_size - 1)) / moe_block_size;
    const int m_blocks = (int)std::min<int64_t>((sorted_numel + moe_block_size - 1) / moe_block_size,
                                                live_bound);
    const int n_blocks = (int)(size_n / (64 * nt));
    const int steps = (int)(size_k / 128);
    // Only a fraction of the moe blocks are live; estimate them from the route count.
    const int64_t live = std::min<int64_t>(m_blocks, (size_m * top_k + moe_block_size - 1) /
                                                         moe_block_size + num_experts);
    int splits = 1;
    const int64_t base = live * n_blocks;
    if (base < (int64_t)cus * 2 && steps >= 4) {
      splits = (int)std::min<int64_t>(((int64_t)cus * 2 + base - 1) / base, steps / 2);
    }
    if (ov.moe_split_k >= 0) splits = ov.moe_split_k;
    splits = std::max(1, std::min(splits, std::max(steps, 1)));
    const int sps = steps == 0 ? 0 : (steps + splits - 1) / splits;
    splits = steps == 0 ? 1 : (steps + sps - 1) / sps;

    GemmParams p{};
    p.a = a;
    p.a_stride = size_k;
    p.c = c;
    p.b = reinterpret_cast<const uint32_t*>(b_q_weight);
    p.b_expert_stride = size_k * size_n / pack;
    p.scales = b_scales;
    p.zeros = b_zeros_numel ? b_zeros : nullptr;
    p.meta_expert_stride = num_groups * size_n;
    p.bias = b_bias_numel ? b_bias : nullptr;
    p.global_scale = global_scale;
    p.alpha_exp = 7 - (a_dtype == MARLIN_DTYPE_FLOAT16 ? 14 : 126);
    p.M = (int)size_m;
    p.N = (int)size_n;
    p.K = (int)size_k;
    p.group_shift = mc.group_shift;
    p.splits = splits;
    p.steps_per_split = sps;
    p.num_n_blocks = n_blocks;
    p.num_m_blocks = m_blocks;
    p.xcd_group_m = 0;
    if (splits == 1) {
      // moe blocks of one expert (and their activation rows) in one L2: groups of
      // consecutive moe blocks x all column blocks dealt to the XCDs in turn
      p.xcd_group_m = ov.moe_group_m;
      p.xcd_interleave = p.xcd_group_m > 0 ? 1 : 0;
    }
    p.sorted_ids = sorted_token_ids;
    p.sorted_numel = (int)sorted_numel;
    p.expert_ids = expert_ids;
    p.expert_ids_numel = (int)std::min<int64_t>(expert_ids_numel, INT32_MAX);
    p.num_post_pad = num_tokens_past_padded;
    p.topk_w = topk_weights;
    p.top_k = (int)top_k;
    p.moe_bs = (int)moe_block_size;
    p.mul_topk = mul_topk_weights ? 1 : 0;
    p.valid_ids = (int)(size_m * top_k);
    if (splits > 1) {
      Workspace& w = get_workspace(dev, s, (size_t)size_m * top_k * size_n,
                                   (size_t)m_blocks * n_blocks);
      p.ws = w.ws;
      p.counters = w.counters;
    }
    GemmLaunch l{};
    l.fmt = mc.fmt;
    l.bf16 = a_dtype == MARLIN_DTYPE_BFLOAT16;
    l.gsm = mc.gsm;
    l.bm = bm;
    l.nt = nt;
    l.ch = 1;
    l.moe = true;
    // (small-group metadata of 48/64-row blocks over 256 columns does not fit the multistage
    // kernel's registers: those blocks take the tiled kernel)
    l.stream = !(mc.gsm == GSM_SMALL && bm >= 48 && nt == 4) && ov.stream != 0;
    l.grid = (unsigned)((int64_t)m_blocks * n_blocks * splits);
    // Few routes per expert (decode-sized batches): the K-split decode kernel, one moe block
    // and 64 columns per workgroup, multiplying only the block's 16-row parts that hold
    // routes.  Its integer-operand path needs integer or fp8 weights with >= 128-deep groups.
    const bool int_operand = mc.fmt != FMT_MXFP4 && mc.fmt != FMT_NVFP4 && mc.gsm != GSM_SMALL;
    if (int_operand && size_m * top_k <= 16 * num_experts && ov.moe_decode != 0) {
      const int groups = (int)(size_n / 64);
      p.splits = 1;
      p.steps_per_split = steps;
      p.num_n_blocks = groups;
      p.num_m_blocks = m_blocks;
      l.stream = false;
      l.depth = ov.moe_depth;
      l.nt = 4;
      // one wave per workgroup, all of K: thousands of short workgroups that the dispatcher
      // load-balances across CUs as they finish
      l.wpb = ov.moe_wpb;
      l.ksplit = true;
      // two waves per SIMD (tiles scaled in pairs: no spills) rather than one wave with the
      // compiler's full register choice, and a ring two steps deep: cfg5 layer at T = 16 /
      // 64 / 300: 138 / 296 / 430 us, against 141 / 302 / 439 with three steps and 157 /
      // 340 / 470 with one wave per SIMD
      l.occ = (l.depth <= 3 && l.wpb == 1) ? 2 : 1;
      l.grid = (unsigned)((int64_t)m_blocks * groups);
    }
    if (gated) {
      // the fused activation runs in the epilogue of the multistage kernel (256-column
      // blocks, no split K) or of the few-routes decode kernel (one wave per block, its
      // tiles 32 gate and the matching 32 up columns); any other plan (a split K, narrower
      // column blocks, the tiled kernel) is reported as NOT_SUPPORTED before anything
      // launches, and the caller runs the two passes instead
      const bool stream_ok = l.stream && l.depth == 0 && nt == 4 && splits == 1 && size_n % 256 == 0;
      const bool decode_ok = l.depth == 2 && l.wpb == 1 && size_n % 64 == 0;
      check_supported((stream_ok || decode_ok) && !ov.any,
                      "the fused SiLU stage-1 epilogue does not cover this shape or batch");
      l.gated = true;
      check_supported(instantiated(l), "no gated moe kernel instance for this configuration");
    }
    if (ov.any && !instantiated(l))
      check_supported(false, "no moe kernel instance for the selected configuration; a "
                             "MARLIN_MI355X_* tuning override selects a configuration this "
                             "build does not instantiate");
    if (fmt_int_zero(mc.fmt))
      p.zeros = stage_int_zeros(dev, s, b_zeros, fmt_bits(mc.fmt),
                                num_experts * num_groups * size_n);
    check_hip(dispatch_gemm(l, p, s), "moe_wna16_marlin_gemm launch");
  });
}

#define MMI_MOE_ARGS_DECL                                                                        \
    const void* a, marlin_dtype_t a_dtype, void* c, const int32_t* b_q_weight,                  \
    int64_t b_q_weight_numel, int64_t num_experts, const void* b_bias, int64_t b_bias_numel,    \
    const void* b_scales, marlin_dtype_t b_scales_dtype, int64_t b_scales_numel,                \
    int64_t num_groups, int64_t a_scales_numel, const float* global_scale,                      \
    int64_t global_scale_numel, const void* b_zeros, marlin_dtype_t b_zeros_dtype,              \
    int64_t b_zeros_numel, int64_t g_idx_numel, int64_t perm_numel, void* workspace,            \
    int64_t workspace_bytes, const int32_t* sorted_token_ids, int64_t sorted_numel,             \
    const int32_t* expert_ids, int64_t expert_ids_numel,                                        \
    const int32_t* num_tokens_past_padded, const float* topk_weights,                           \
    int64_t topk_weights_numel, int64_t moe_block_size, int64_t top_k, int mul_topk_weights,    \
    int64_t b_type_id, int64_t size_m, int64_t size_n, int64_t size_k, int is_k_full,           \
    int use_atomic_add, int use_fp32_reduce, int is_zp_float, int64_t thread_k,                 \
    int64_t thread_n, int64_t blocks_per_sm, marlin_stream_t stream
#define MMI_MOE_ARGS                                                                             \
    a, a_dtype, c, b_q_weight, b_q_weight_numel, num_experts, b_bias, b_bias_numel, b_scales,     \
    b_scales_dtype, b_scales_numel, num_groups, a_scales_numel, global_scale, global_scale_numel, \
    b_zeros, b_zeros_dtype, b_zeros_numel, g_idx_numel, perm_numel, workspace, workspace_bytes,   \
    sorted_token_ids, sorted_numel, expert_ids, expert_ids_numel, num_tokens_past_padded,         \
    topk_weights, topk_weights_numel, moe_block_size, top_k, mul_topk_weights, b_type_id, size_m, \
    size_n, size_k, is_k_full, use_atomic_add, use_fp32_reduce, is_zp_float, thread_k, thread_n,  \
    blocks_per_sm, stream

marlin_status_t marlin_moe_wna16_marlin_gemm(MMI_MOE_ARGS_DECL) {
  return moe_gemm(false, MMI_MOE_ARGS);
}

marlin_status_t marlin_moe_wna16_marlin_gemm_silu(MMI_MOE_ARGS_DECL) {
  return moe_gemm(true, MMI_MOE_ARGS);
}
#undef MMI_MOE_ARGS_DECL
#undef MMI_MOE_ARGS

marlin_status_t marlin_dequantize(const int32_t* b_q_weight, int64_t b_q_weight_numel,
                                  const void* b_scales, marlin_dtype_t b_scales_dtype,
                                  int64_t b_scales_numel, int64_t num_groups,
                                  const void* b_zeros, marlin_dtype_t b_zeros_dtype,
                                  int64_t b_zeros_numel, const float* global_scale,
                                  int64_t global_scale_numel, int64_t b_type_id,
                                  int64_t size_k, int64_t size_n, marlin_dtype_t out_dtype,
                                  void* out, marlin_stream_t stream) {
  return guarded([&] {
    check(is_half_type(out_dtype), "out_dtype must be float16 or bfloat16");
    const MetaCheck mc = check_weight_meta(b_type_id, out_dtype, b_scales_dtype, b_scales_numel,
                                           num_groups, 1, global_scale, global_scale_numel, 1,
                                           b_zeros, b_zeros_dtype, b_zeros_numel,
                                           b_zeros_numel > 0 && b_zeros_dtype != MARLIN_DTYPE_INT32,
                                           size_n, size_k);
    const int64_t pack = 32 / fmt_bits(mc.fmt);
    check(size_k % 32 == 0, "size_k must be divisible by 32");
    check(size_n % 16 == 0, "size_n must be divisible by 16");
    check(b_q_weight_numel == size_k * size_n / pack, "b_q_weight numel mismatch");
    if (size_k == 0 || size_n == 0) return;
    GemmParams p{};
    p.b = reinterpret_cast<const uint32_t*>(b_q_weight);
    p.scales = b_scales;
    p.zeros = b_zeros_numel ? b_zeros : nullptr;
    p.global_scale = global_scale;
    p.alpha_exp = 7 - (out_dtype == MARLIN_DTYPE_FLOAT16 ? 14 : 126);
    p.N = (int)size_n;
    p.K = (int)size_k;
    p.group_shift = mc.group_shift;
    if (fmt_int_zero(mc.fmt)) {
      int dev = 0;
      check_hip(hipGetDevice(&dev), "hipGetDevice");
      p.zeros = stage_int_zeros(dev, (hipStream_t)stream, b_zeros, fmt_bits(mc.fmt),
                                num_groups * size_n);
    }
    check_hip(launch_dequant(mc.fmt, p, out_dtype == MARLIN_DTYPE_BFLOAT16, out, mc.gsm,
                             (hipStream_t)stream),
              "marlin_dequantize launch");
  });
}

marlin_status_t marlin_moe_sum(const void* input, marlin_dtype_t dtype, int64_t num_tokens,
                               int64_t top_k, int64_t hidden, void* out,
                               marlin_stream_t stream) {
  return guarded([&] {
    check(is_half_type(dtype) || dtype == MARLIN_DTYPE_FLOAT32,
          "moe_sum supports float16, bfloat16 and float32");
    check(num_tokens >= 0 && top_k >= 1 && top_k <= INT32_MAX && hidden >= 0,
          "invalid moe_sum shape");
    if (num_tokens == 0 || hidden == 0) return;
    check(input && out, "null tensor pointer");
    const int kind = dtype == MARLIN_DTYPE_FLOAT32 ? 2 : (dtype == MARLIN_DTYPE_BFLOAT16 ? 1 : 0);
    check_hip(launch_moe_sum(input, kind, num_tokens, (int)top_k, hidden, out,
                             (hipStream_t)stream),
              "moe_sum launch");
  });
}

marlin_status_t marlin_silu_and_mul(const void* input, marlin_dtype_t dtype, int64_t rows,
                                    int64_t d, void* out, marlin_stream_t stream) {
  return guarded([&] {
    check(is_half_type(dtype), "silu_and_mul supports float16 and bfloat16");
    check(rows >= 0 && d >= 0, "invalid silu_and_mul shape");
    if (rows == 0 || d == 0) return;
    check(input && out, "null tensor pointer");
    check_hip(launch_silu_and_mul(input, dtype == MARLIN_DTYPE_BFLOAT16, rows, d, out,
                                  (hipStream_t)stream),
              "silu_and_mul launch");
  });
}

}  // extern "C"

namespace {

marlin_status_t topk_gating(bool sigmoid, float* topk_weights, void* topk_indices,
                            marlin_dtype_t ids_dtype, int32_t* token_expert_indices,
                            int64_t top_k, const void* gating, marlin_dtype_t gating_dtype,
                            int64_t num_tokens, int64_t num_experts, int renormalize,
                            const float* bias, int64_t bias_numel, marlin_stream_t stream) {
  return guarded([&] {
    check(gating_dtype == MARLIN_DTYPE_FLOAT32 || gating_dtype == MARLIN_DTYPE_FLOAT16 ||
              gating_dtype == MARLIN_DTYPE_BFLOAT16,
          "Unsupported gating_output data type: ", (int)gating_dtype);
    check(ids_dtype == MARLIN_DTYPE_INT32 || ids_dtype == MARLIN_DTYPE_UINT32 ||
              ids_dtype == MARLIN_DTYPE_INT64,
          "topk_indices must be int32, uint32 or int64");
    check(num_experts > 0, "num_experts must be positive");
    check(num_tokens >= 0, "invalid num_tokens");
    check(top_k >= 1 && top_k <= num_experts, "topk must be in [1, num_experts]");
    if (bias) check(bias_numel == num_experts, "bias size mismatch, expected: ", num_experts);
    check_supported(num_experts <= kRouterMaxExperts, "this build supports at most ",
                    kRouterMaxExperts, " experts per router row");
    check_supported(top_k <= kMaxK, "this build supports topk <= ", kMaxK);
    if (num_tokens == 0) return;
    check(topk_weights && topk_indices && token_expert_indices && gating, "null tensor pointer");
    const int in_kind = gating_dtype == MARLIN_DTYPE_FLOAT16 ? 0
                        : gating_dtype == MARLIN_DTYPE_BFLOAT16 ? 1 : 2;
    const int ids_kind = ids_dtype == MARLIN_DTYPE_INT32 ? 0 : ids_dtype == MARLIN_DTYPE_UINT32 ? 1 : 2;
    check_hip(launch_topk_gating(sigmoid, in_kind, gating, bias, topk_weights, topk_indices,
                                 ids_kind, token_expert_indices, num_tokens, (int)num_experts,
                                 (int)top_k, renormalize != 0, (hipStream_t)stream),
              sigmoid ? "topk_sigmoid launch" : "topk_softmax launch");
  });
}

}  // namespace

extern "C" {

marlin_status_t marlin_topk_softmax(float* topk_weights, void* topk_indices,
                                    marlin_dtype_t topk_indices_dtype,
                                    int32_t* token_expert_indices, int64_t top_k,
                                    const void* gating_output, marlin_dtype_t gating_dtype,
                                    int64_t num_tokens, int64_t num_experts, int renormalize,
                                    const float* bias, int64_t bias_numel,
                                    marlin_stream_t stream) {
  return topk_gating(false, topk_weights, topk_indices, topk_indices_dtype, token_expert_indices,
                     top_k, gating_output, gating_dtype, num_tokens, num_experts, renormalize,
                     bias, bias_numel, stream);
}

marlin_status_t marlin_topk_sigmoid(float* topk_weights, void* topk_indices,
                                    marlin_dtype_t topk_indices_dtype,
                                    int32_t* token_expert_indices, int64_t top_k,
                                    const void* gating_output, marlin_dtype_t gating_dtype,
                                    int64_t num_tokens, int64_t num_experts, int renormalize,
                                    const float* bias, int64_t bias_numel,
                                    marlin_stream_t stream) {
  return topk_gating(true, topk_weights, topk_indices, topk_indices_dtype, token_expert_indices,
                     top_k, gating_output, gating_dtype, num_tokens, num_experts, renormalize,
                     bias, bias_numel, stream);
}

marlin_status_t marlin_grouped_topk(const void* scores, marlin_dtype_t scores_dtype,
                                    int64_t num_tokens, int64_t num_experts, int64_t n_group,
                                    int64_t topk_group, int64_t topk, int renormalize,
                                    double routed_scaling_factor, const void* bias,
                                    marlin_dtype_t bias_dtype, int64_t bias_numel,
                                    int64_t scoring_func, float* topk_values,
                                    int32_t* topk_indices, marlin_stream_t stream) {
  return guarded([&] {
    const auto half_or_f32 = [](marlin_dtype_t d) {
      return d == MARLIN_DTYPE_FLOAT16 || d == MARLIN_DTYPE_BFLOAT16 || d == MARLIN_DTYPE_FLOAT32;
    };
    check(half_or_f32(scores_dtype), "Invalid dtype, only supports float16, float32, and bfloat16");
    check(half_or_f32(bias_dtype),
          "Invalid bias dtype, only supports float16, float32, and bfloat16");
    check(num_tokens >= 0 && num_experts > 0, "invalid scores shape");
    check(n_group > 0, "n_group must be positive");
    check(topk > 0, "topk must be positive");
    check(topk_group > 0, "topk_group must be positive");
    check(topk_group <= n_group, "topk_group must be <= n_group");
    check(num_experts % n_group == 0, "num_experts should be divisible by n_group");
    check(n_group <= 32, "n_group should be smaller than or equal to 32 for now");
    check(topk <= 32, "topk should be smaller than or equal to 32 for now");
    check(topk <= topk_group * (num_experts / n_group),
          "topk must be <= topk_group * (num_experts / n_group)");
    check(scoring_func == 0 || scoring_func == 1,
          "scoring_func must be SCORING_NONE (0) or SCORING_SIGMOID (1)");
    check(bias_numel == num_experts, "bias size mismatch, expected: ", num_experts);
    check_supported(num_experts <= kGroupedMaxExperts, "this build supports at most ",
                    kGroupedMaxExperts, " experts for grouped_topk");
    if (num_tokens == 0) return;
    check(scores && bias && topk_values && topk_indices, "null tensor pointer");
    const auto kind = [](marlin_dtype_t d) {
      return d == MARLIN_DTYPE_FLOAT16 ? 0 : d == MARLIN_DTYPE_BFLOAT16 ? 1 : 2;
    };
    check_hip(launch_grouped_topk((int)scoring_func, kind(scores_dtype), kind(bias_dtype), scores,
                                  bias, topk_values, topk_indices, num_tokens, (int)num_experts,
                                  (int)n_group, (int)topk_group, (int)topk, renormalize != 0,
                                  (float)routed_scaling_factor, (hipStream_t)stream),
              "grouped_topk launch");
  });
}

}  // extern "C"
