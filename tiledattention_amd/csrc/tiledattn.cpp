// Host side of the C ABI declared in include/tiledattn.h.
//
// Replaces the reference's launch boundary (src/tiledattention/kernels/flash_fwd.py:786-818,
// torch-ext/torch_binding.cpp:6-19, tiledattention_cuda/tiledattention.cu:13-33) and its
// kernel cache (src/tiledattention/kernels/compile_cache.py:10-37):
//   * kernels are precompiled into gfx950 code objects: attn_fwd_m<TM>_n<TN>.hsaco per tile
//     shape, and attn_fwd_pp.hsaco with the eight-wave kernels that serve the (128, 64)
//     and (128, 128) shapes with fp32 accumulation; one module per (device, file) is loaded on first use
//     and kept, and resolved hipFunction_t handles are cached per (device, kernel name);
//   * the cache is guarded by a mutex (the reference's dict is unguarded);
//   * launches go to the caller's stream under a device guard, like the reference's torch op
//     (OptionalCUDAGuard + current stream, tiledattention.cu:29-31).
#include <dlfcn.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <functional>
#include <map>
#include <mutex>
#include <queue>
#include <unordered_map>
#include <string>
#include <tuple>
#include <vector>

#include "../../include/tiledattn.h"
#include "attn_fwd_params.h"
#include "attn_fwd_split.h"

namespace {

thread_local std::string g_last_error;

// Records the error text for ta_last_error().  A failed HIP call also leaves its code in
// the runtime's per-thread last-error slot, where the caller's next error check (torch
// checks after every kernel launch) would pick it up as its own; the status returned here
// reports it instead, so the slot is cleared.
ta_status fail(ta_status st, const char* fmt, ...) {
  if (st == TA_EHIP || st == TA_ENOKERNEL) (void)hipGetLastError();
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return st;
}

std::mutex g_mu;
std::string g_dir;   // code object directory; empty = next to this library
std::map<std::pair<int, std::string>, hipModule_t> g_modules;  // (device, code object file)
std::map<std::pair<int, std::string>, hipFunction_t> g_funcs;  // (device, kernel name)
std::map<int, bool> g_arch_ok;                                 // device -> gfx950?
// In-kernel merge: the device address of attn_fwd_pp.hsaco's ta_merge_counters per device
// (zeroed when the module loads), and the counter region each (device, stream) launches
// with, so that split launches that may overlap (other streams) never share counters.
std::map<int, unsigned*> g_counters;
std::map<std::pair<int, void*>, int> g_regions;
std::map<int, int> g_regions_used;
const char kPPObject[] = "attn_fwd_pp.hsaco";
const char kWideObject[] = "attn_fwd_wide.hsaco";

std::string default_dir() {
  Dl_info info;
  if (dladdr(reinterpret_cast<void*>(&default_dir), &info) && info.dli_fname) {
    std::string p(info.dli_fname);
    size_t cut = p.find_last_of('/');
    if (cut != std::string::npos) return p.substr(0, cut);
  }
  return ".";
}

// Restores the caller's current device on scope exit (the reference's torch op does the
// same with OptionalCUDAGuard, tiledattention.cu:29).
struct DeviceGuard {
  int prev = -1;
  bool changed = false;
  hipError_t err = hipSuccess;
  explicit DeviceGuard(int dev) {
    err = hipGetDevice(&prev);
    if (err == hipSuccess && prev != dev) {
      err = hipSetDevice(dev);
      changed = (err == hipSuccess);
    }
  }
  ~DeviceGuard() {
    if (changed) (void)hipSetDevice(prev);
  }
};

// Which kernel serves a launch: code object file, symbol and workgroup size.
struct KernelId {
  std::string file;
  std::string name;
  unsigned block;
};

// The eight-wave kernel (attn_fwd_pp.hip) serves 128-row tiles with fp32 accumulation at
// D = 64, 96, 128 and 160: its workgroup step is 128 rows x 128 keys, 64 keys per wave group,
// so it stands for both TILE_N = 64 and TILE_N = 128 (the latter only up to D = 128,
// check_shape).
bool eight_wave(int64_t tm, int64_t tn, int64_t accum, int64_t d) {
  return tm == 128 && (tn == 64 || tn == 128) && accum == TA_ACC_FP32 && d <= 160;
}

// Its 64-row form (ta_fwd_pp64_*) serves the 64-row tiles with fp32 accumulation at D = 64,
// 96, 128 and 160: the same 128-key steps, each group's 64 keys split between two waves per
// row block, and no split key ranges or causal pairs.
bool eight_wave64(int64_t tm, int64_t tn, int64_t accum, int64_t d) {
  return tm == 64 && (tn == 64 || tn == 128) && accum == TA_ACC_FP32 &&
         (d == 64 || d == 96 || d == 128 || d == 160);
}

// Input-dtype accumulation on the eight-wave kernels (ta_fwd_ppl_* for 128-row tiles,
// ta_fwd_ppl64_* for 64-row ones) at D = 64 and 128: whole rows, no split or pairs.
bool eight_wave_lowp(int64_t tm, int64_t tn, int64_t accum, int64_t d) {
  return accum == TA_ACC_INPUT && (tm == 64 || tm == 128) && (tn == 64 || tn == 128) &&
         (d == 64 || d == 128);
}

// Any of them: direct-to-LDS staging of Q, K and V (in-place padding of narrower head dims
// through d_real; 128-key steps).
bool eight_wave_family(int64_t tm, int64_t tn, int64_t accum, int64_t d) {
  return eight_wave(tm, tn, accum, d) || eight_wave64(tm, tn, accum, d) ||
         eight_wave_lowp(tm, tn, accum, d);
}

KernelId kernel_id(int dtype, int d, int tm, int tn, int causal, int tail, int accum) {
  const char* dt = dtype == TA_BF16 ? "bf16" : "f16";
  char buf[96];
  if (eight_wave(tm, tn, accum, d)) {
    // Eight waves: two per SIMD sharing the rows of a 32-row block, splitting every
    // 128-key step between them.
    snprintf(buf, sizeof(buf), "ta_fwd_pp_%s_d%d_c%d_t%d", dt, d, causal ? 1 : 0, tail ? 1 : 0);
    return {"attn_fwd_pp.hsaco", buf, 512u};
  }
  if (eight_wave64(tm, tn, accum, d)) {
    snprintf(buf, sizeof(buf), "ta_fwd_pp64_%s_d%d_c%d_t%d", dt, d, causal ? 1 : 0, tail ? 1 : 0);
    return {"attn_fwd_pp.hsaco", buf, 512u};
  }
  if (eight_wave_lowp(tm, tn, accum, d)) {
    // one kernel per tile_n: the keys of a wave's slice between roundings of O
    snprintf(buf, sizeof(buf), "ta_fwd_%s_n%d_%s_d%d_c%d_t%d", tm == 128 ? "ppl" : "ppl64", tn, dt, d,
             causal ? 1 : 0, tail ? 1 : 0);
    return {"attn_fwd_pp.hsaco", buf, 512u};
  }
  snprintf(buf, sizeof(buf), "ta_fwd_%s_d%d_m%d_n%d_c%d_t%d_a%d", dt, d, tm, tn, causal ? 1 : 0,
           tail ? 1 : 0, accum ? 1 : 0);
  char file[64];
  snprintf(file, sizeof(file), "attn_fwd_m%d_n%d.hsaco", tm, tn);
  return {file, buf, static_cast<unsigned>(tm * 2)};  // tm / 32 waves of 64
}

// The causal query-block pair kernel of the eight-wave family (use_pairs).
KernelId pair_kernel_id(int dtype, int d, int tail) {
  char buf[96];
  snprintf(buf, sizeof(buf), "ta_fwd_pp_pair_%s_d%d_c1_t%d", dtype == TA_BF16 ? "bf16" : "f16", d,
           tail ? 1 : 0);
  return {"attn_fwd_pp.hsaco", buf, 512u};
}

bool valid_tile(int t) { return t == 64 || t == 128; }

bool valid_head_dim(int64_t d) { return d == 64 || d == 96 || d == 128 || d == 160 || d == 256; }

// Head dims above 128 exist only with 64-key tiles (two stages of wider rows fill the LDS);
// D = 96 only on the eight-wave kernels with fp32 accumulation.
ta_status check_shape(int64_t d, int tile_m, int tile_n, int accum) {
  if (!valid_head_dim(d))
    return fail(TA_EUNSUPPORTED, "head_dim %lld (kernels exist for 64, 96, 128, 160 and 256)",
                (long long)d);
  if (!valid_tile(tile_m) || !valid_tile(tile_n))
    return fail(TA_EUNSUPPORTED, "tile (%d, %d) (supported: 64 or 128 each)", tile_m, tile_n);
  if (d == 96 && accum != TA_ACC_FP32)
    return fail(TA_EUNSUPPORTED,
                "head_dim 96 with tile (%d, %d) and accum %d (D = 96 kernels: fp32 accumulation)",
                tile_m, tile_n, accum);
  if (d > 128 && tile_n != 64)
    return fail(TA_EUNSUPPORTED, "tile_n %d with head_dim %lld (head dims above 128 need tile_n 64)",
                tile_n, (long long)d);
  return TA_OK;
}

// Caller holds g_mu and has made `device` current.
ta_status check_arch_locked(int device) {
  auto it = g_arch_ok.find(device);
  if (it != g_arch_ok.end()) {
    if (!it->second) return fail(TA_EUNSUPPORTED, "device %d is not gfx950", device);
    return TA_OK;
  }
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess)
    return fail(TA_EHIP, "hipGetDeviceProperties(%d): %s", device, hipGetErrorString(e));
  bool ok = strncmp(prop.gcnArchName, "gfx950", 6) == 0;
  g_arch_ok[device] = ok;
  if (!ok)
    return fail(TA_EUNSUPPORTED, "device %d is %s; kernels are built for gfx950", device,
                prop.gcnArchName);
  return TA_OK;
}

// Caller holds g_mu and has made `device` current.
ta_status get_function_locked(int device, const KernelId& id, hipFunction_t* out) {
  auto fk = std::make_pair(device, id.name);
  auto fit = g_funcs.find(fk);
  if (fit != g_funcs.end()) {
    *out = fit->second;
    return TA_OK;
  }
  ta_status st = check_arch_locked(device);
  if (st != TA_OK) return st;
  auto mk = std::make_pair(device, id.file);
  hipModule_t mod = nullptr;
  auto mit = g_modules.find(mk);
  if (mit == g_modules.end()) {
    std::string path = (g_dir.empty() ? default_dir() : g_dir) + "/" + id.file;
    hipError_t e = hipModuleLoad(&mod, path.c_str());
    if (e != hipSuccess)
      return fail(TA_ENOKERNEL, "hipModuleLoad(%s): %s", path.c_str(), hipGetErrorString(e));
    if (id.file == kPPObject) {
      // The merge counters start at zero; every launch leaves them zero.  Zeroed here
      // once per load, synchronously, before any kernel of the module can run.
      hipDeviceptr_t cnt = nullptr;
      size_t bytes = 0;
      e = hipModuleGetGlobal(&cnt, &bytes, mod, "ta_merge_counters");
      if (e == hipSuccess && bytes == sizeof(unsigned) * ta::kMergeRegions * ta::kMergeRegionCounters) {
        e = hipMemsetAsync(cnt, 0, bytes, nullptr);
        if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
      } else if (e == hipSuccess) {
        e = hipErrorInvalidValue;
      }
      if (e != hipSuccess) {
        (void)hipModuleUnload(mod);
        return fail(TA_ENOKERNEL, "merge counters of %s: %s", path.c_str(), hipGetErrorString(e));
      }
      g_counters[device] = static_cast<unsigned*>(cnt);
      for (auto it = g_regions.begin(); it != g_regions.end();)
        it = it->first.first == device ? g_regions.erase(it) : std::next(it);
      g_regions_used[device] = 0;
    }
    g_modules[mk] = mod;
  } else {
    mod = mit->second;
  }
  hipFunction_t fn = nullptr;
  hipError_t e = hipModuleGetFunction(&fn, mod, id.name.c_str());
  if (e != hipSuccess)
    return fail(TA_ENOKERNEL, "hipModuleGetFunction(%s): %s", id.name.c_str(),
                hipGetErrorString(e));
  g_funcs[fk] = fn;
  *out = fn;
  return TA_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The dispatch packet counts work-items in 32 bits: grid * block must fit.
ta_status check_grid(int64_t blocks, unsigned block, const char* what) {
  if (blocks * static_cast<int64_t>(block) > 0xffffffffLL)
    return fail(TA_EINVAL, "%s grid of %lld workgroups x %u threads exceeds 2^32 work-items", what,
                (long long)blocks, block);
  return TA_OK;
}

void clear_resolved_plans();  // below: the resolved launch plans hold functions of the modules

// Caller holds g_mu.  Unloads every module; the launch paths resolve and launch under the
// same lock, so no launch can use a function of a module unloaded here.
ta_status cache_reset_locked() {
  ta_status st = TA_OK;
  for (auto& kv : g_modules) {
    DeviceGuard guard(std::get<0>(kv.first));
    hipError_t e = hipModuleUnload(kv.second);
    if (e != hipSuccess && st == TA_OK)
      st = fail(TA_EHIP, "hipModuleUnload: %s", hipGetErrorString(e));
  }
  g_modules.clear();
  g_funcs.clear();
  clear_resolved_plans();
  g_counters.clear();
  g_regions.clear();
  g_regions_used.clear();
  return st;
}

// Caller holds g_mu and has loaded attn_fwd_pp.hsaco on `device`.  The counter region of
// (device, stream): the stream's own, or a new one while any is left; null when every
// region belongs to other streams (the launch then runs the merge kernel).
unsigned* merge_counters_locked(int device, void* stream) {
  auto cit = g_counters.find(device);
  if (cit == g_counters.end()) return nullptr;
  const auto key = std::make_pair(device, stream);
  auto rit = g_regions.find(key);
  int region;
  if (rit != g_regions.end()) {
    region = rit->second;
  } else {
    int& used = g_regions_used[device];
    if (used >= ta::kMergeRegions) return nullptr;
    region = used++;
    g_regions[key] = region;
  }
  return cit->second + static_cast<int64_t>(region) * ta::kMergeRegionCounters;
}

// ---- split key ranges ------------------------------------------------------------------
// The eight-wave kernel (128 query rows, steps of 128 keys) can cut each query block's key
// range into chunks of C steps counted back from its last step; every chunk is one
// workgroup, and blocks of more than one chunk are combined by the merge kernel from
// fp32 partials in a caller-provided workspace.  The numbering below is the one the
// kernels derive from their block id (attn_fwd_pp.hip).
using ta::SplitLayout;
using ta::split_layout;
constexpr int kSplitRows = ta::kPPRows;

// Cut offset f of the paired split (attn_fwd_split.h psplit_items): the fixed cost of a
// workgroup's second block, in key steps, moved to the workgroup that runs one block.
constexpr int kPairCut = 4;
static_assert(TA_SPLIT_PAIRS == ta::kSplitPairs, "header and numbering agree");

// Layout of chunk length c (kSplitPairs: the paired split with offset kPairCut).
bool layout_for(int64_t S, bool causal, int64_t c, SplitLayout* l) {
  return split_layout(S, causal, c, l, kPairCut);
}

// Workspace: fp32 partial outputs [slots][128][D], then the log-sum-exps [slots][128].
int64_t split_ws_bytes(int64_t n_bh, int64_t d, const SplitLayout& l) {
  const int64_t rows = n_bh * l.slots * kSplitRows;
  const int64_t o_bytes = (rows * d * 4 + 255) / 256 * 256;
  return o_bytes + rows * 4;
}

// Finish time of the slowest CU when the grid (split with chunks of c steps, or the
// whole-row grid for c = 0) is dispatched onto `ncu` CUs holding one workgroup each, in
// units of one key step of a lightly loaded chip.  The hardware hands block ids to the 8
// XCDs round-robin and each XCD starts its blocks in id order on whichever CU frees first.
// An item costs its steps, slower the more CUs the grid keeps busy (clock and memory
// contention), plus a fixed cost (launch, Q and first K/V loads, pipeline fill and drain,
// merge of the two key halves, output stores); a split grid adds the merge kernel, whose
// cost grows with the partial slots it reads.  Constants fitted to MI355X timings of the
// eight-wave kernel (B*H 1-16, S 1024-16384, causal and not).
double simulate_split(int64_t S, int64_t n_bh, bool causal, int64_t c, int ncu) {
  const double kItem = 10.0, kLoad = 0.5, kMerge = 6.0, kMergeSlot = 1.0;
  const int nq = (int)((S + ta::kPPRows - 1) / ta::kPPRows);
  const int len = (int)((S + ta::kPPKeys - 1) / ta::kPPKeys);
  SplitLayout l;
  const bool split = c > 0 && layout_for(S, causal, c, &l);
  const int64_t total = split ? n_bh * l.items : n_bh * nq;
  const int xcds = 8;
  const int per_xcd = std::max(1, ncu / xcds);
  const double step = 1.0 + kLoad * (double)std::min<int64_t>(total, ncu) / ncu;
  std::vector<std::priority_queue<double, std::vector<double>, std::greater<double>>> cu(xcds);
  for (auto& q : cu)
    for (int i = 0; i < per_xcd; ++i) q.push(0.0);
  for (int64_t blk = 0; blk < total; ++blk) {
    const ta::WorkItem w =
        split ? ta::split_item((int)blk, (int)n_bh, (int)l.items, 1, causal, (int)c, (int)l.ns,
                               (int)l.slots, (int)S)
              : ta::whole_item((int)blk, (int)n_bh, nq, 1, causal);
    const int t_end = w.t_end >= 0 ? w.t_end : (causal ? w.qt + 1 : len);
    auto& q = cu[blk % xcds];
    const double t = q.top();
    q.pop();
    q.push(t + (t_end - w.t_beg) * step + kItem);
  }
  double worst = 0.0;
  for (auto& q : cu) {
    while (q.size() > 1) q.pop();
    worst = std::max(worst, q.top());
  }
  return worst + (split ? kMerge + kMergeSlot * (double)(n_bh * l.slots) / ncu : 0.0);
}

std::map<int, int> g_cu_count;  // device -> compute units
std::map<std::tuple<int64_t, int64_t, int, int>, int32_t> g_plans;

// Caller holds g_mu and has made `device` current.
ta_status cu_count_locked(int device, int* out) {
  auto it = g_cu_count.find(device);
  if (it != g_cu_count.end()) {
    *out = it->second;
    return TA_OK;
  }
  int n = 0;
  hipError_t e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device);
  if (e != hipSuccess)
    return fail(TA_EHIP, "hipDeviceGetAttribute(%d): %s", device, hipGetErrorString(e));
  g_cu_count[device] = n;
  *out = n;
  return TA_OK;
}

// Chunk length (key steps) with the earliest simulated finish, or 0 when no split beats
// the whole-row grid by 20 % (the model's error on the fitted timings stays below that).
// Grids of several waves of workgroups balance by themselves and are not split.  Causal
// grids of more than half and at most one workgroup per CU, with 32 or more query blocks
// a head, take the paired split instead, the fastest of the three there on the MI355X
// (per call, bf16 unless noted, B1 H8 S4096: D = 128 45.0 us whole rows / 45.1 best
// chunk / 44.0 paired, fp16 D = 64 33.0 / 33.0 / 30.2, D = 96 38.0 / 38.0 / 36.5, D = 160
// 55.0 / 54.8 / 51.7; B1 H4 S8192 84.3 / 70.8 / 70.6).  With fewer workgroups chunks win
// (B1 H2 S8192 47.2 against 51.0 paired, B1 H4 S4096 30.9 against 33.9), and with
// shorter rows the second block's fixed cost outweighs the balance (B1 H16 S2048 24.5
// whole rows, 28.5 paired).
int32_t plan_split(int64_t S, int64_t n_bh, bool causal, int ncu) {
  const int64_t nq = (S + kSplitRows - 1) / kSplitRows;
  const int64_t len = (S + ta::kPPKeys - 1) / ta::kPPKeys;
  if (ncu < 8 || n_bh * nq > 4 * (int64_t)ncu) return 0;
  if (causal && nq >= 32 && 2 * n_bh * nq > (int64_t)ncu && n_bh * nq <= (int64_t)ncu) {
    SplitLayout l;
    if (layout_for(S, causal, ta::kSplitPairs, &l)) return ta::kSplitPairs;
  }
  const double base = simulate_split(S, n_bh, causal, 0, ncu);
  double best = base * 0.8;
  int32_t best_c = 0;
  for (int64_t c = 1; c < len; ++c) {
    SplitLayout l;
    if (!layout_for(S, causal, c, &l)) continue;
    if (l.items * n_bh > 8 * (int64_t)ncu) continue;  // more items than waves help
    const double t = simulate_split(S, n_bh, causal, c, ncu);
    if (t < best) {
      best = t;
      best_c = (int32_t)c;
    }
  }
  return best_c;
}

// Whether a whole-row launch of a 64-row tile runs the wide kernel (attn_fwd_wide.hip,
// ta_fwd_wide_*: 32 query rows a workgroup, its eight waves splitting the keys of every
// pass of 512 keys at D = 128, 1024 at D = 64; fp32 accumulation): D = 64 or 128, a grid of
// 32-row blocks that fits one round of one workgroup per CU, and either at most two passes
// for the longest block or at most four on more than half the CUs.  There the eight-wave kernel's
// chain of 128-key steps is the latency (back to back, B1 H8 bf16 D = 128 causal, 64-row
// kernel -> wide: S = 512 8.1 -> 6.6 us, S = 1024 11.0 -> 9.0; fp16 D = 64 non-causal
// S = 1024 7.9 -> 6.4; B1 H4 S2048 causal against the 64-row split 15.9 -> 13.4).  With
// fewer blocks and more passes the split spreads the keys over more CUs (B1 H1 S2048 D = 128
// causal: split 12.6, wide 13.2), and a second round of workgroups loses to the 64-row
// kernel (B1 H8 S2048: 17.6 against 19.2; B1 H32 S512: 8.6 against 11.2).
bool use_wide(int64_t S, int64_t n_bh, int64_t D, int ncu) {
  if ((D != 64 && D != 128) || S <= 0 || n_bh <= 0 || ncu <= 0) return false;
  const int64_t grid = n_bh * ((S + 31) / 32);
  if (grid > ncu) return false;
  const int64_t pass_keys = D == 128 ? 512 : 1024;
  const int64_t passes = (S + pass_keys - 1) / pass_keys;
  return passes <= 2 || (passes <= 4 && 2 * grid > ncu);
}

// Split plan for the 64-row kernel (ta_fwd_pp64_split_*): 0 (whole rows) or the chunk
// length with the shortest modelled time, for grids whose 64-row blocks fill at most half
// of the CUs (larger grids keep whole rows, or the 128-row kernel's plan).  Time model in
// microseconds, least-squares fitted (4.9 % rms) to 241 MI355X timings of whole rows and
// forced chunks at D = 64-160, B*H = 1-8, S = 1024-8192, causal and not: a workgroup's
// fixed cost F (launch, prologue, fill and drain, the four-way merge of key slices,
// stores), t_D per 128-key step of the longest workgroup, slower the more CUs the grid
// keeps busy, and for a split the merge kernel's M, m per chunk of the longest block and a
// cost per partial slot written and read back (n_bh * slots 128-row partials of D floats,
// spread over the CUs).  A split must beat whole rows by 2 % and keep every workgroup
// resident at once (one 64-row workgroup per CU).
int32_t plan_split64(int64_t S, int64_t n_bh, bool causal, int64_t d, int ncu) {
  const double kF = 6.08, kM = 3.96, kChunk = 0.30, kLoad = 0.25, kSlot = 3.67;
  const double t = d <= 64 ? 0.40 : d <= 96 ? 0.50 : d <= 128 ? 0.65 : 0.81;
  const int64_t nq64 = (S + 63) / 64;
  const int64_t len = (S + ta::kPPKeys - 1) / ta::kPPKeys;
  if (ncu < 8 || S <= 0 || n_bh <= 0 || 2 * n_bh * nq64 > ncu || len < 2) return 0;
  if (use_wide(S, n_bh, d, ncu)) return 0;  // whole rows on the wide kernel
  auto step = [&](int64_t wgs) { return t * (1.0 + kLoad * (double)wgs / ncu); };
  const double whole = kF + (double)len * step(n_bh * nq64);
  double best = whole * 0.98;
  int32_t best_c = 0;
  for (int64_t c = 1; c < len; ++c) {
    SplitLayout l;
    if (!layout_for(S, causal, c, &l)) continue;
    const int64_t wgs = 2 * n_bh * l.items;  // two 64-row halves per item
    if (wgs > ncu) continue;                 // one wave of workgroups
    const int64_t ns = (len + c - 1) / c;    // chunks of the longest block
    const double slots = (double)(n_bh * l.slots) * (double)d / 128.0 / ncu;
    const double tc = kF + kM + (double)c * step(wgs) + kChunk * (double)ns + kSlot * slots;
    if (tc < best) {
      best = tc;
      best_c = (int32_t)c;
    }
  }
  return best_c;
}

// plan_split memoised per (S, B*H, causal, CUs): the dispatch model runs once per shape.
int32_t cached_split_plan(int64_t S, int64_t n_bh, bool causal, int ncu) {
  {
    std::lock_guard<std::mutex> lock(g_mu);
    auto it = g_plans.find(std::make_tuple(S, n_bh, (int)causal, ncu));
    if (it != g_plans.end()) return it->second;
  }
  // The model runs without the lock; two threads planning one shape compute the same value.
  const int32_t c = plan_split(S, n_bh, causal, ncu);
  std::lock_guard<std::mutex> lock(g_mu);
  g_plans.emplace(std::make_tuple(S, n_bh, (int)causal, ncu), c);
  return c;
}

// Checks shared by every entry point that takes ta_fwd_args.  Fills the grid size.  The
// planning queries (launch = false) need only the shape fields, not tensors or strides.
ta_status validate_args(const ta_fwd_args* a, int64_t* n_bh_out, int64_t* n_qblk_out,
                        bool launch = true) {
  if (a == nullptr) return fail(TA_EINVAL, "args is NULL");
  if (a->dtype != TA_FP16 && a->dtype != TA_BF16) return fail(TA_EINVAL, "dtype %d", a->dtype);
  if (a->accum != TA_ACC_FP32 && a->accum != TA_ACC_INPUT)
    return fail(TA_EINVAL, "accum %d", a->accum);
  if (a->causal != 0 && a->causal != 1) return fail(TA_EINVAL, "causal %d", a->causal);
  if (a->sched < 0 || a->sched > 3) return fail(TA_EINVAL, "sched %d", a->sched);
  if (a->d_real != 0) {
    if (a->d_real < 8 || a->d_real > a->D || (a->d_real & 7) != 0)
      return fail(TA_EINVAL, "d_real %d (0, or a multiple of 8 in [8, D])", a->d_real);
    if (!eight_wave_family(a->tile_m, a->tile_n, a->accum, a->D))
      return fail(TA_EUNSUPPORTED,
                  "d_real needs an eight-wave kernel: fp32 accumulation with D <= 160 (tile "
                  "(128, 64) or (128, 128), or (64, 64) / (64, 128) up to D = 128 and (64, 64) "
                  "at D = 160), or D = 64 or 128 with any tile and input-dtype accumulation");
  }
  if (a->B < 0 || a->H < 0 || a->S < 0) return fail(TA_EINVAL, "negative shape");
  ta_status shape_st = check_shape(a->D, a->tile_m, a->tile_n, a->accum);
  if (shape_st != TA_OK) return shape_st;
  *n_bh_out = a->B * a->H;
  *n_qblk_out = 0;
  if (a->B == 0 || a->H == 0 || a->S == 0) return TA_OK;
  if (a->S > 0x7fffffffLL || a->H > 0x7fffffffLL) return fail(TA_EINVAL, "S or H too large");
  const int64_t n_bh = a->B * a->H;
  const int64_t n_qblk = (a->S + a->tile_m - 1) / a->tile_m;
  if (n_bh > 0x7fffffffLL || n_bh * n_qblk > 0x7fffffffLL)
    return fail(TA_EINVAL, "grid too large (B*H*ceil(S/TM) must fit in int32)");
  if (!launch) {
    *n_qblk_out = n_qblk;
    return TA_OK;
  }
  if (!a->q || !a->k || !a->v || !a->o) return fail(TA_EINVAL, "null tensor pointer");
  if (!aligned16(a->q) || !aligned16(a->k) || !aligned16(a->v) || !aligned16(a->o))
    return fail(TA_EINVAL, "q/k/v/o must be 16-byte aligned");
  const int64_t* st[4] = {a->q_stride, a->k_stride, a->v_stride, a->o_stride};
  const char* nm[4] = {"q", "k", "v", "o"};
  // Rows are read (and o written) as whole rows of the head dim actually present; a row
  // stride below that width makes rows overlap, and a zero one (a tensor expanded along S)
  // would give every buffer resource below a size of zero, so its loads would read zeros.
  const int64_t width = a->d_real ? a->d_real : a->D;
  for (int i = 0; i < 4; ++i) {
    if (st[i][3] != 1) return fail(TA_EINVAL, "%s: last-dim stride must be 1", nm[i]);
    for (int j = 0; j < 3; ++j)
      if (st[i][j] < 0 || (st[i][j] & 7) != 0)
        return fail(TA_EINVAL, "%s: stride[%d]=%lld must be a non-negative multiple of 8", nm[i], j,
                    (long long)st[i][j]);
    if (st[i][2] < width)
      return fail(TA_EINVAL, "%s: row stride %lld is below the row width %lld (rows overlap)",
                  nm[i], (long long)st[i][2], (long long)width);
    // Bounded first, so that the products below cannot overflow (S < 2^31).
    if (st[i][2] >= (1LL << 23))
      return fail(TA_EINVAL, "%s: row stride %lld must stay below 2^23 elements", nm[i],
                  (long long)st[i][2]);
  }
  // K and V are read with buffer instructions whose byte range is 32-bit: a (b, h) slice,
  // and the 128 rows one tile step addresses (below 2^31 by the bound above), must stay
  // below 2^31 bytes.
  if (a->S * a->k_stride[2] * 2 > 0x7fffffffLL || a->S * a->v_stride[2] * 2 > 0x7fffffffLL)
    return fail(TA_EINVAL, "k/v: S * row stride must stay below 2^31 bytes per (b, h) slice");
  // The eight-wave kernels stage Q the same way (one buffer resource per query block).
  if (eight_wave_family(a->tile_m, a->tile_n, a->accum, a->D) &&
      a->S * a->q_stride[2] * 2 > 0x7fffffffLL)
    return fail(TA_EINVAL, "q: S * row stride must stay below 2^31 bytes per (b, h) slice");
  if (a->aligned != 0 && a->aligned != 1) return fail(TA_EINVAL, "aligned %d", a->aligned);
  *n_qblk_out = n_qblk;
  return TA_OK;
}

void fill_params(const ta_fwd_args* a, int64_t n_bh, int64_t n_qblk, ta::FwdParams* p) {
  memset(p, 0, sizeof(*p));
  p->q = static_cast<const uint16_t*>(a->q);
  p->k = static_cast<const uint16_t*>(a->k);
  p->v = static_cast<const uint16_t*>(a->v);
  p->o = static_cast<uint16_t*>(a->o);
  p->q_sb = a->q_stride[0]; p->q_sh = a->q_stride[1]; p->q_ss = a->q_stride[2];
  p->k_sb = a->k_stride[0]; p->k_sh = a->k_stride[1]; p->k_ss = a->k_stride[2];
  p->v_sb = a->v_stride[0]; p->v_sh = a->v_stride[1]; p->v_ss = a->v_stride[2];
  p->o_sb = a->o_stride[0]; p->o_sh = a->o_stride[1]; p->o_ss = a->o_stride[2];
  p->H = static_cast<int32_t>(a->H);
  p->S = static_cast<int32_t>(a->S);
  p->n_qblk = static_cast<int32_t>(n_qblk);
  p->n_bh = static_cast<int32_t>(n_bh);
  p->scale_log2 = static_cast<float>(static_cast<double>(a->scale) * 1.4426950408889634);
  p->sched = a->sched;
  p->d_real = a->d_real ? a->d_real : static_cast<int32_t>(a->D);
}

// Whether a launch runs the kernel variant without tail masking: the caller allows it
// (args->aligned, the aligned fast-path decision, flash_fwd.py:199-238) and every tile is
// whole (S a multiple of both tile sizes, and of the 128-key step for the eight-wave
// kernels).
bool unmasked_tail(const ta_fwd_args* a) {
  const bool steps = !eight_wave_family(a->tile_m, a->tile_n, a->accum, a->D) || a->S % ta::kPPKeys == 0;
  return a->aligned == 1 && a->S % a->tile_m == 0 && a->S % a->tile_n == 0 && steps;
}

// Whether a whole-row launch runs causal query blocks in pairs (nq - 1 - j, then j; one
// workgroup each pair, attn_fwd_split.h pair_items): the eight-wave kernel at D <= 128,
// causal, at least two blocks a head, and either forced (sched 3) or, with XCD grouping
// (sched 1), a grid of two or more workgroups per CU.  Below that every block runs at once and pairing would
// only lengthen the longest workgroup.  With two waves of workgroups or more, the hardware
// hands block ids to the XCDs in a fixed round-robin, so an XCD whose CUs finish early
// waits for the others before it gets its next block; pairs give every workgroup the same
// work (nq + 1 key steps) instead of relying on that order.
bool use_pairs(const ta_fwd_args* a, int64_t n_bh, int64_t n_qblk, int ncu) {
  // (D = 160 pairs measured slower: B1 H8 S8192 bf16 147.6 -> 153.9 us)
  if (!a->causal || n_qblk < 2 || a->D > 128 || !eight_wave(a->tile_m, a->tile_n, a->accum, a->D))
    return false;
  if (a->sched == 3) return true;
  return a->sched == 1 && n_bh * n_qblk >= 2 * (int64_t)ncu;
}

// Whether a whole-row launch runs 256-row blocks (ta_fwd_pp256_*: the two wave groups own
// different rows and each takes every key of a step, 64 MFMAs a cluster): non-causal, the
// eight-wave kernel at D = 64 or 128 with fp32 accumulation, when the grid takes no more
// rounds of one workgroup per CU than half the 128-row grid's (a 256-row block is two
// 128-row blocks of work at ≈4 % less time: B1 H8 S8192 D = 128, 256 blocks on 256 CUs,
// 222 -> 214 µs bf16; a round more, e.g. 384 blocks against 768, loses).
bool use_rows256(const ta_fwd_args* a, int64_t n_bh, int ncu) {
  if (a->causal || !eight_wave(a->tile_m, a->tile_n, a->accum, a->D) || (a->D != 64 && a->D != 128) ||
      ncu <= 0)
    return false;
  const int64_t rounds256 = (n_bh * ((a->S + 255) / 256) + ncu - 1) / ncu;
  const int64_t rounds128 = (n_bh * ((a->S + 127) / 128) + ncu - 1) / ncu;
  return 2 * rounds256 <= rounds128;
}

// Whether split key ranges exist for this configuration: the eight-wave kernels with fp32
// accumulation, 128-row blocks (chunks and the paired split) or 64-row blocks (chunks, each
// 128-row item of the numbering run as two 64-row halves).
bool split_capable(const ta_fwd_args* a) {
  return eight_wave(a->tile_m, a->tile_n, a->accum, a->D) || eight_wave64(a->tile_m, a->tile_n, a->accum, a->D);
}

// Whether a chunk length can run on this configuration: the paired split needs 128-row
// blocks.
bool split_runs(const ta_fwd_args* a, int32_t chunk_steps) {
  if (!split_capable(a)) return false;
  return chunk_steps != TA_SPLIT_PAIRS || a->tile_m == 128;
}

// Everything one forward launches, decided in one place: ta_sdpa_fwd, ta_sdpa_fwd_split
// and ta_describe_launch all read it from plan_launch, so the launch and its description
// cannot disagree.
struct LaunchPlan {
  KernelId main;         // the attention kernel
  int64_t grid = 0;      // its workgroups
  int32_t rows = 0;      // query rows per query block it processes
  bool tail = false;     // tail-masked variant
  int32_t layout = TA_LAYOUT_WHOLE_ROWS;
  int32_t chunk = 0;     // split actually run (0 = whole rows)
  bool merge = false;    // a merge kernel follows (split layouts)
  bool merge_in_kernel = false;  // ... unless the split kernel merges (counters fit)
  KernelId merge_id;
  int64_t merge_grid = 0;
  SplitLayout split;     // valid when merge
  int64_t ws_bytes = 0;  // split workspace
};

// The plan for shape-validated arguments with n_bh * n_qblk > 0, on a device of `ncu`
// compute units.  chunk_steps = 0, or a chunk length that splits nothing, plans the
// whole-row launch (pairs or 256-row blocks where their rules pick them); a chunk length
// that splits something on a configuration without split kernels is TA_EUNSUPPORTED.
ta_status plan_launch(const ta_fwd_args* a, int64_t n_bh, int64_t n_qblk, int32_t chunk_steps,
                      int ncu, LaunchPlan* pl) {
  *pl = LaunchPlan();
  const bool aligned = unmasked_tail(a);
  pl->tail = !aligned;
  const char* dt = a->dtype == TA_BF16 ? "bf16" : "f16";
  SplitLayout l;
  if (chunk_steps != 0 && layout_for(a->S, a->causal != 0, chunk_steps, &l)) {
    if (!split_runs(a, chunk_steps))
      return fail(TA_EUNSUPPORTED,
                  "split key ranges need fp32 accumulation on tile (128, 64) or (128, 128) with D <= 160, "
                  "or chunks on tile (64, 64) or (64, 128) with D = 64, 96, 128 or 160 (the paired split: "
                  "128-row tiles)");
    if (n_bh * l.items > 0x7fffffffLL || n_bh * l.slots * kSplitRows > 0x7fffffffLL ||
        n_bh * l.merge * kSplitRows > 0x7fffffffLL)
      return fail(TA_EINVAL, "split grid too large");
    const bool paired = chunk_steps == TA_SPLIT_PAIRS;
    const bool rows64 = a->tile_m == 64;
    char name[96];
    snprintf(name, sizeof(name), "ta_fwd_%s_%s_d%d_c%d_t%d",
             rows64 ? "pp64_split" : paired ? "pp_psplit" : "pp_split", dt, (int)a->D, a->causal ? 1 : 0,
             aligned ? 0 : 1);
    pl->main = KernelId{"attn_fwd_pp.hsaco", name, 512u};
    pl->grid = (rows64 ? 2 : 1) * n_bh * l.items;  // 64-row: two halves per item
    pl->rows = rows64 ? 64 : kSplitRows;
    pl->layout = paired ? TA_LAYOUT_PAIRED_SPLIT : TA_LAYOUT_SPLIT;
    pl->chunk = chunk_steps;
    // merge: one thread per (row, 16-byte output chunk), merge_rows_per_wg(D) rows a workgroup
    const int d8 = static_cast<int>(a->D);
    snprintf(name, sizeof(name), "ta_fwd_merge_%s_d%d_c%d", dt, d8, a->causal ? 1 : 0);
    pl->merge = true;
    pl->merge_id = KernelId{"attn_fwd_pp.hsaco", name, static_cast<unsigned>(ta::merge_threads(d8))};
    pl->merge_grid = n_bh * l.merge * (kSplitRows / ta::merge_rows_per_wg(d8));
    pl->split = l;
    pl->ws_bytes = split_ws_bytes(n_bh, a->D, l);
    // The split kernel merges its blocks itself (the last workgroup to finish a block) when
    // a counter per block fits a region (a block's counter is its chunk-0 slot, below
    // n_bh * slots) and either no block has more than two chunks or the merges are many
    // (3/8 of the CUs or more) and so spread over the chip.  A block of many chunks merged
    // by one workgroup at the end of a small grid costs more than the merge kernel, which
    // spreads each block over 8-16 workgroups (B1 H1 S4096 causal, 7 chunks: 17.8 -> 22.2
    // µs in the kernel; the paired split at C3 S = 4096: 44.4 -> 43.6 µs, D = 64
    // 30.6 -> 28.9).
    const int64_t nq128 = (a->S + kSplitRows - 1) / kSplitRows;
    const int64_t max_ns = chunk_steps == TA_SPLIT_PAIRS ? 2
                           : a->causal                  ? (nq128 + chunk_steps - 1) / chunk_steps
                                                        : l.ns;
    pl->merge_in_kernel = n_bh * l.slots <= ta::kMergeRegionCounters &&
                          (max_ns <= 2 || 8 * n_bh * l.merge >= 3 * (int64_t)ncu);
    ta_status gst = check_grid(pl->grid, 512u, "split kernel");
    if (gst == TA_OK) gst = check_grid(pl->merge_grid, pl->merge_id.block, "merge kernel");
    return gst;
  }
  pl->main = kernel_id(a->dtype, (int)a->D, a->tile_m, a->tile_n, a->causal, !aligned, a->accum);
  pl->grid = n_bh * n_qblk;
  pl->rows = a->tile_m;
  if (eight_wave(a->tile_m, a->tile_n, a->accum, a->D)) {
    if (a->causal && use_pairs(a, n_bh, n_qblk, ncu)) {
      pl->main = pair_kernel_id(a->dtype, (int)a->D, !aligned);
      pl->grid = n_bh * ((n_qblk + 1) / 2);
      pl->layout = TA_LAYOUT_PAIRS;
    } else if (use_rows256(a, n_bh, ncu)) {
      const int64_t nq256 = (a->S + 255) / 256;
      const bool t256 = !(aligned && a->S % 256 == 0);
      char name[64];
      snprintf(name, sizeof(name), "ta_fwd_pp256_%s_d%d_c0_t%d", dt, (int)a->D, t256 ? 1 : 0);
      pl->main = KernelId{"attn_fwd_pp.hsaco", name, 512u};
      pl->grid = n_bh * nq256;
      pl->rows = 256;
      pl->tail = t256;
      pl->layout = TA_LAYOUT_ROWS256;
    }
  } else if (eight_wave64(a->tile_m, a->tile_n, a->accum, a->D) && use_wide(a->S, n_bh, a->D, ncu)) {
    // The aligned variant's S (a multiple of 128) is whole 32-row blocks and whole passes of
    // a wave's keys, as its t0 form needs.
    char name[64];
    snprintf(name, sizeof(name), "ta_fwd_wide_%s_d%d_c%d_t%d", dt, (int)a->D, a->causal ? 1 : 0, aligned ? 0 : 1);
    pl->main = KernelId{kWideObject, name, 512u};
    pl->grid = n_bh * ((a->S + 31) / 32);
    pl->rows = 32;
    pl->layout = TA_LAYOUT_WIDE;
  }
  return check_grid(pl->grid, pl->main.block, "kernel");
}

void fill_desc(const ta_fwd_args* a, const LaunchPlan& pl, int ncu, ta_launch_desc* d) {
  memset(d, 0, sizeof(*d));
  snprintf(d->code_object, sizeof(d->code_object), "%s", pl.main.file.c_str());
  snprintf(d->kernel, sizeof(d->kernel), "%s", pl.main.name.c_str());
  d->grid = pl.grid;
  d->block = static_cast<int32_t>(pl.main.block);
  d->rows = pl.rows;
  d->tail = pl.tail ? 1 : 0;
  d->layout = pl.layout;
  d->chunk_steps = pl.chunk;
  d->compute_units = ncu;
  if (pl.merge) {
    snprintf(d->merge_kernel, sizeof(d->merge_kernel), "%s", pl.merge_id.name.c_str());
    d->merge_grid = pl.merge_grid;
    d->merge_in_kernel = pl.merge_in_kernel ? 1 : 0;
    d->merge_block = static_cast<int32_t>(pl.merge_id.block);
  }
  d->workspace_bytes = pl.ws_bytes;
  d->in_place_pad = eight_wave_family(a->tile_m, a->tile_n, a->accum, a->D) ? 1 : 0;
  d->split_capable = split_capable(a) ? 1 : 0;
}

// Shape checks, then the plan and its description (no device, no tensors).
ta_status describe_model(const ta_fwd_args* a, int32_t chunk_steps, int ncu, ta_launch_desc* out) {
  if (out == nullptr) return fail(TA_EINVAL, "out is NULL");
  memset(out, 0, sizeof(*out));
  if (chunk_steps < 0 && chunk_steps != TA_SPLIT_PAIRS) return fail(TA_EINVAL, "chunk_steps %d", chunk_steps);
  if (ncu <= 0) return fail(TA_EINVAL, "compute_units %d", ncu);
  int64_t n_bh = 0, n_qblk = 0;
  ta_status vst = validate_args(a, &n_bh, &n_qblk, false);
  if (vst != TA_OK) return vst;
  out->compute_units = ncu;
  out->in_place_pad = eight_wave_family(a->tile_m, a->tile_n, a->accum, a->D) ? 1 : 0;
  out->split_capable = split_capable(a) ? 1 : 0;
  if (n_qblk == 0) return TA_OK;  // zero-size: nothing is launched
  LaunchPlan pl;
  ta_status st = plan_launch(a, n_bh, n_qblk, chunk_steps, ncu, &pl);
  if (st != TA_OK) return st;
  fill_desc(a, pl, ncu, out);
  return TA_OK;
}

// A plan with its kernels resolved on the device.
struct ResolvedPlan {
  LaunchPlan pl;
  hipFunction_t fn = nullptr;   // the attention kernel
  hipFunction_t mfn = nullptr;  // the merge kernel (split layouts)
};

// Resolved plans of recent launches, keyed by every argument the plan depends on (the
// tensors and strides are not among them) and the device's CU count: a call of a known
// configuration skips the planning (kernel names, rules) and the function lookup.  Cleared
// with the module cache (cache_reset_locked), so a plan never outlives its functions.
struct PlanKey {
  int64_t B, H, S, D;
  int32_t causal, dtype, tile_m, tile_n, accum, device, sched, d_real, aligned, ncu, chunk, pad;
  bool operator==(const PlanKey& o) const {
    return B == o.B && H == o.H && S == o.S && D == o.D && causal == o.causal && dtype == o.dtype &&
           tile_m == o.tile_m && tile_n == o.tile_n && accum == o.accum && device == o.device &&
           sched == o.sched && d_real == o.d_real && aligned == o.aligned && ncu == o.ncu && chunk == o.chunk;
  }
};
struct PlanKeyHash {
  size_t operator()(const PlanKey& k) const {
    uint64_t h = 1469598103934665603ull;
    auto mix = [&](uint64_t v) { h = (h ^ v) * 1099511628211ull; };
    mix((uint64_t)k.B); mix((uint64_t)k.H); mix((uint64_t)k.S); mix((uint64_t)k.D);
    mix(((uint64_t)(uint32_t)k.causal << 32) | (uint32_t)k.dtype);
    mix(((uint64_t)(uint32_t)k.tile_m << 32) | (uint32_t)k.tile_n);
    mix(((uint64_t)(uint32_t)k.accum << 32) | (uint32_t)k.device);
    mix(((uint64_t)(uint32_t)k.sched << 32) | (uint32_t)k.d_real);
    mix(((uint64_t)(uint32_t)k.aligned << 32) | (uint32_t)k.ncu);
    mix((uint64_t)(uint32_t)k.chunk);
    return (size_t)h;
  }
};
std::unordered_map<PlanKey, ResolvedPlan, PlanKeyHash> g_resolved;
constexpr size_t kResolvedMax = 4096;
void clear_resolved_plans() { g_resolved.clear(); }

// Caller holds g_mu and has made the device current.  The resolved plan of a launch (from
// the cache, or planned and resolved now); the pointer stays valid until the cache lock is
// released.
ta_status resolved_plan_locked(const ta_fwd_args* a, int64_t n_bh, int64_t n_qblk, int32_t chunk_steps,
                               int ncu, const ResolvedPlan** out) {
  const PlanKey key{a->B,      a->H,     a->S,      a->D,     a->causal, a->dtype,  a->tile_m, a->tile_n,
                    a->accum,  a->device, a->sched, a->d_real, a->aligned, ncu,      chunk_steps, 0};
  auto it = g_resolved.find(key);
  if (it != g_resolved.end()) {
    *out = &it->second;
    return TA_OK;
  }
  ResolvedPlan r;
  ta_status st = plan_launch(a, n_bh, n_qblk, chunk_steps, ncu, &r.pl);
  if (st == TA_OK) st = get_function_locked(a->device, r.pl.main, &r.fn);
  if (st == TA_OK && r.pl.merge) st = get_function_locked(a->device, r.pl.merge_id, &r.mfn);
  if (st != TA_OK) return st;
  if (g_resolved.size() >= kResolvedMax) g_resolved.clear();
  *out = &g_resolved.emplace(key, std::move(r)).first->second;
  return TA_OK;
}

// Enqueues a resolved plan.  Caller holds g_mu and has made the device current; p carries
// the tensors (and, for a split, the workspace).
ta_status launch_plan_locked(const ta_fwd_args* a, const ResolvedPlan& r, ta::FwdParams* p, void* stream) {
  const LaunchPlan& pl = r.pl;
  if (pl.layout == TA_LAYOUT_ROWS256) p->n_qblk = static_cast<int32_t>((a->S + 255) / 256);
  if (pl.layout == TA_LAYOUT_WIDE) p->n_qblk = static_cast<int32_t>((a->S + 31) / 32);
  // the split numbering and the merge count 128-row blocks, whatever rows a workgroup takes
  if (pl.merge) p->n_qblk = static_cast<int32_t>((a->S + kSplitRows - 1) / kSplitRows);
  p->merge_cnt = nullptr;
  if (pl.merge && pl.merge_in_kernel) p->merge_cnt = merge_counters_locked(a->device, stream);
  void* params[] = {p};
  hipStream_t hs = static_cast<hipStream_t>(stream);
  hipError_t e = hipModuleLaunchKernel(r.fn, static_cast<unsigned>(pl.grid), 1, 1, pl.main.block, 1, 1,
                                       0, hs, params, nullptr);
  if (e != hipSuccess) return fail(TA_EHIP, "hipModuleLaunchKernel: %s", hipGetErrorString(e));
  if (pl.merge && p->merge_cnt == nullptr) {
    e = hipModuleLaunchKernel(r.mfn, static_cast<unsigned>(pl.merge_grid), 1, 1, pl.merge_id.block, 1,
                              1, 0, hs, params, nullptr);
    if (e != hipSuccess) return fail(TA_EHIP, "hipModuleLaunchKernel: %s", hipGetErrorString(e));
  }
  return TA_OK;
}

// ---- call policy ------------------------------------------------------------------
// What a call with given knobs runs: tile, accumulation, kernel head dim and padding, the
// aligned fast path, workgroup order and split.  The rules restate the host policy of the
// reference (flash_fwd.py:47-259, 851-921) with this build's gfx950 choices, and are the
// same rules tiledattention/kernels/flash_fwd.py applies (a CPU test compares the two over
// a grid of shapes and knob values).

// Head dim of the kernel that runs `d`, and its zero padding: kernels exist for 64, 128,
// 160 and 256, and 96 with fp32 accumulation on tiles of 64 or 128 keys (native_96); other
// head dims pad up to the next (flash_fwd.py:149-163 pads to a power of two).
bool kernel_head_dim(int64_t d, bool native_96, int* kd, int* pad) {
  if (d <= 0) return false;
  if (native_96 && d > 64 && d <= 96) {
    *kd = 96;
    *pad = (int)(96 - d);
    return true;
  }
  for (int k : {64, 128, 160, 256}) {
    if (d <= k) {
      *kd = k;
      *pad = (int)(k - d);
      return true;
    }
  }
  return false;
}

// Default tile when no tile is given: 128 query rows, or 64 when the 64-row blocks of every
// head fit the compute units once (head dims up to 128, up to 160 with fp32 accumulation);
// TILE_N 128 for non-causal D = 128 at S >= 2048, else 64 (the reference's rule,
// flash_fwd.py:254-259).
void default_tile(int64_t S, int64_t d, bool causal, int64_t n_bh, bool fp32, int ncu, int* tm, int* tn) {
  *tn = (!causal && d == 128 && S >= 2048) ? 128 : 64;
  const int64_t max_d64 = fp32 ? 160 : 128;
  *tm = (d > 0 && d <= max_d64 && n_bh > 0 && S > 0 && n_bh * ((S + 63) / 64) <= ncu) ? 64 : 128;
}

// Workgroups of one launch resident on a CU: two for the non-causal eight-wave kernels at
// D = 64 with fp32 accumulation, one for the other eight-wave kernels; for the four-wave
// kernels two at (128, 64) with input-dtype accumulation, two at (64, 128) up to D = 128,
// four at (64, 64) up to D = 128 and two above, one otherwise.
int workgroups_per_cu(int tm, int tn, int accum, int d, bool causal) {
  if (eight_wave_family(tm, tn, accum, d)) return (accum == TA_ACC_FP32 && d <= 64 && !causal) ? 2 : 1;
  if (tm == 128 && tn == 64 && accum == TA_ACC_INPUT) return 2;
  if (tm == 64 && tn == 128 && d <= 128) return 2;
  if (tm == 64 && tn == 64) return d <= 128 ? 4 : 2;
  return 1;
}

// Default workgroup order: XCD grouping when the grid splits evenly over the 8 XCDs; for
// causal grids that are resident all at once, the heavy/light complementary order.
int default_sched(int64_t n_blocks, bool causal, int tm, int tn, int accum, int d, int ncu) {
  if (n_blocks % 8 != 0) return 0;
  const int64_t resident = (int64_t)ncu * workgroups_per_cu(tm, tn, accum, d, causal);
  return (causal && n_blocks <= resident) ? 2 : 1;
}

ta_status plan_call(int64_t B, int64_t H, int64_t S, int64_t D, int32_t dtype, int32_t causal,
                    int32_t device, int ncu, const ta_call_knobs* k, ta_call_plan* out) {
  if (dtype != TA_FP16 && dtype != TA_BF16) return fail(TA_EINVAL, "dtype %d", dtype);
  if (causal != 0 && causal != 1) return fail(TA_EINVAL, "causal %d", causal);
  if (B < 0 || H < 0 || S < 0) return fail(TA_EINVAL, "negative shape");
  if ((k->tile_m == 0) != (k->tile_n == 0))
    return fail(TA_EINVAL, "tile_m and tile_n must both be 0 (default) or both be given");
  if (k->accum != -1 && k->accum != TA_ACC_FP32 && k->accum != TA_ACC_INPUT)
    return fail(TA_EINVAL, "accum %d", k->accum);
  if (k->sched < -1 || k->sched > 3) return fail(TA_EINVAL, "sched %d", k->sched);
  if (k->split < 0 && k->split != TA_SPLIT_AUTO && k->split != TA_SPLIT_PAIRS)
    return fail(TA_EINVAL, "split %d", k->split);
  if (D <= 0) return fail(TA_EINVAL, "head dimension D must be positive");
  const int64_t n_bh = B * H;
  const bool cz = causal != 0;
  const int accum = k->accum == TA_ACC_INPUT ? TA_ACC_INPUT : TA_ACC_FP32;  // auto: fp32 on gfx950
  const bool explicit_tile = k->tile_m != 0;
  int tm = k->tile_m, tn = k->tile_n;
  if (explicit_tile) {
    if (!valid_tile(tm) || !valid_tile(tn))
      return fail(TA_EUNSUPPORTED, "tile (%d, %d) (supported: 64 or 128 each)", tm, tn);
  } else {
    default_tile(S, D, cz, n_bh, accum == TA_ACC_FP32, ncu, &tm, &tn);
    // Keep 128 rows where the 128-row kernel would split key ranges (split kernels exist
    // for fp32 accumulation only), unless the 64-row grid fills at most half the CUs: there
    // the 64-row kernel, whole or split by its own plan, is faster.
    const bool small64 = 2 * n_bh * ((S + 63) / 64) <= ncu;
    if (tm == 64 && accum == TA_ACC_FP32 && k->split != 0 && !(small64 && k->split == TA_SPLIT_AUTO)) {
      if (k->split != TA_SPLIT_AUTO) {
        tm = 128;
      } else {
        int kd = 0, pad = 0;
        if (kernel_head_dim(D, true, &kd, &pad) && cached_split_plan(S, n_bh, cz, ncu) != 0) tm = 128;
      }
    }
  }
  int kd = 0, pad = 0;
  if (!kernel_head_dim(D, (tn == 64 || tn == 128) && accum == TA_ACC_FP32, &kd, &pad))
    return fail(TA_EUNSUPPORTED, "head dimension D=%lld is not supported: the gfx950 kernels cover D <= 256",
                (long long)D);
  if (kd > 128 && tn != 64) {
    if (explicit_tile)
      return fail(TA_EUNSUPPORTED, "TILE_N=%d is not supported for head dimension D=%lld: head dims above 128 run with TILE_N=64",
                  tn, (long long)D);
    tn = 64;
  }
  ta_status st = check_shape(kd, tm, tn, accum);
  if (st != TA_OK) return st;
  const bool in_place = pad > 0 && D % 8 == 0 && eight_wave_family(tm, tn, accum, kd);
  memset(out, 0, sizeof(*out));
  ta_fwd_args& a = out->args;
  a.B = B;
  a.H = H;
  a.S = S;
  a.D = kd;
  a.causal = causal;
  a.dtype = dtype;
  a.tile_m = tm;
  a.tile_n = tn;
  a.accum = accum;
  a.device = device;
  a.d_real = in_place ? (int32_t)D : 0;
  a.aligned = (k->aligned && S % tm == 0 && S % tn == 0) ? 1 : 0;
  const int64_t n_qblk = (S + tm - 1) / tm;
  a.sched = k->sched >= 0 ? k->sched : default_sched(n_bh * n_qblk, cz, tm, tn, accum, kd, ncu);
  out->host_pad = in_place ? 0 : pad;
  out->out_width = in_place ? (int32_t)D : kd;
  if (n_bh == 0 || S == 0) return TA_OK;
  // Split: the dispatch model (auto), a forced chunk length or the paired split.
  int32_t chunk = 0;
  if (k->split == TA_SPLIT_AUTO) {
    chunk = eight_wave(tm, tn, accum, kd) ? cached_split_plan(S, n_bh, cz, ncu)
            : eight_wave64(tm, tn, accum, kd) ? plan_split64(S, n_bh, cz, kd, ncu) : 0;
  } else if (k->split != 0) {
    if (!split_runs(&a, k->split))
      return fail(TA_EUNSUPPORTED,
                  "split key ranges need fp32 accumulation on tile (128, 64) or (128, 128) with D <= 160, "
                  "or chunks on tile (64, 64) or (64, 128) with D = 64, 96, 128 or 160 (the paired split: "
                  "128-row tiles)");
    chunk = k->split;
  }
  out->chunk_steps = chunk;
  if (chunk != 0) {
    SplitLayout l;
    if (layout_for(S, cz, chunk, &l)) {
      out->workspace_bytes = split_ws_bytes(n_bh, kd, l);
      if (k->sched < 0) a.sched = 1;  // the split grid regroups per XCD whenever it divides evenly
    }
  }
  return TA_OK;
}

}  // namespace

extern "C" {

// Error channel for the library's other translation unit (tiledattn_static.hip): records
// `msg` for ta_last_error() on this thread and returns `st`.
__attribute__((visibility("hidden"))) ta_status ta_internal_fail(ta_status st, const char* msg) {
  return fail(st, "%s", msg);
}

int ta_abi_version(void) { return TA_ABI_VERSION; }

const char* ta_last_error(void) { return g_last_error.c_str(); }

const char* ta_status_string(int32_t status) {
  switch (status) {
    case TA_OK: return "TA_OK";
    case TA_EINVAL: return "TA_EINVAL";
    case TA_EUNSUPPORTED: return "TA_EUNSUPPORTED";
    case TA_ENOKERNEL: return "TA_ENOKERNEL";
    case TA_EHIP: return "TA_EHIP";
    default: return "TA_UNKNOWN";
  }
}

ta_status ta_cache_reset(void) {
  std::lock_guard<std::mutex> lock(g_mu);
  return cache_reset_locked();
}

int32_t ta_cache_size(void) {
  std::lock_guard<std::mutex> lock(g_mu);
  return static_cast<int32_t>(g_funcs.size());
}

ta_status ta_set_code_object_dir(const char* dir) {
  if (dir == nullptr) return fail(TA_EINVAL, "code object dir is NULL");
  std::lock_guard<std::mutex> lock(g_mu);
  ta_status st = cache_reset_locked();
  g_dir = dir;
  return st;
}

ta_status ta_prepare(int32_t device, int32_t dtype, int32_t head_dim, int32_t tile_m,
                     int32_t tile_n, int32_t causal, int32_t accum, int32_t aligned) {
  if (dtype != TA_FP16 && dtype != TA_BF16) return fail(TA_EINVAL, "dtype %d", dtype);
  if (accum != TA_ACC_FP32 && accum != TA_ACC_INPUT) return fail(TA_EINVAL, "accum %d", accum);
  ta_status shape_st = check_shape(head_dim, tile_m, tile_n, accum);
  if (shape_st != TA_OK) return shape_st;
  std::lock_guard<std::mutex> lock(g_mu);
  DeviceGuard guard(device);
  if (guard.err != hipSuccess)
    return fail(TA_EHIP, "set device %d: %s", device, hipGetErrorString(guard.err));
  hipFunction_t fn;
  return get_function_locked(
      device, kernel_id(dtype, head_dim, tile_m, tile_n, causal != 0, aligned == 0, accum), &fn);
}

ta_status ta_sdpa_fwd(const ta_fwd_args* a, void* stream) {
  int64_t n_bh = 0, n_qblk = 0;
  ta_status vst = validate_args(a, &n_bh, &n_qblk);
  if (vst != TA_OK || n_qblk == 0) return vst;
  // The whole-row grid bounds every layout's (pairs and 256-row blocks only shrink it; the
  // wide kernel's runs only within one round of the CUs), so an oversized request is
  // rejected before any device call.
  const unsigned base_block = eight_wave_family(a->tile_m, a->tile_n, a->accum, a->D)
                                  ? 512u
                                  : static_cast<unsigned>(a->tile_m * 2);  // kernel_id's block
  ta_status gst = check_grid(n_bh * n_qblk, base_block, "kernel");
  if (gst != TA_OK) return gst;
  ta::FwdParams p;
  fill_params(a, n_bh, n_qblk, &p);

  // Plan, resolve and launch under the cache lock (a concurrent ta_cache_reset cannot unload
  // the module in between); the launch only enqueues.
  std::lock_guard<std::mutex> lock(g_mu);
  DeviceGuard guard(a->device);
  if (guard.err != hipSuccess)
    return fail(TA_EHIP, "set device %d: %s", a->device, hipGetErrorString(guard.err));
  int ncu = 0;
  ta_status cst = cu_count_locked(a->device, &ncu);
  if (cst != TA_OK) return cst;
  const ResolvedPlan* rp = nullptr;
  ta_status st = resolved_plan_locked(a, n_bh, n_qblk, 0, ncu, &rp);
  if (st != TA_OK) return st;
  return launch_plan_locked(a, *rp, &p, stream);
}

ta_status ta_plan_call(int64_t B, int64_t H, int64_t S, int64_t D, int32_t dtype, int32_t causal,
                       int32_t device, int32_t compute_units, const ta_call_knobs* knobs,
                       ta_call_plan* out) {
  if (knobs == nullptr || out == nullptr) return fail(TA_EINVAL, "knobs or out is NULL");
  int ncu = compute_units;
  if (ncu == 0) {
    std::lock_guard<std::mutex> lock(g_mu);
    DeviceGuard guard(device);
    if (guard.err != hipSuccess)
      return fail(TA_EHIP, "set device %d: %s", device, hipGetErrorString(guard.err));
    ta_status cst = cu_count_locked(device, &ncu);
    if (cst != TA_OK) return cst;
  }
  if (ncu <= 0) return fail(TA_EINVAL, "compute_units %d", ncu);
  return plan_call(B, H, S, D, dtype, causal, device, ncu, knobs, out);
}

ta_status ta_describe_launch_model(const ta_fwd_args* args, int32_t chunk_steps,
                                   int32_t compute_units, ta_launch_desc* out) {
  return describe_model(args, chunk_steps, compute_units, out);
}

ta_status ta_describe_launch(const ta_fwd_args* args, int32_t chunk_steps, ta_launch_desc* out) {
  if (args == nullptr) return fail(TA_EINVAL, "args is NULL");
  int ncu = 0;
  {
    std::lock_guard<std::mutex> lock(g_mu);
    DeviceGuard guard(args->device);
    if (guard.err != hipSuccess)
      return fail(TA_EHIP, "set device %d: %s", args->device, hipGetErrorString(guard.err));
    ta_status cst = cu_count_locked(args->device, &ncu);
    if (cst != TA_OK) return cst;
  }
  return describe_model(args, chunk_steps, ncu, out);
}

ta_status ta_split_plan(const ta_fwd_args* a, int32_t* chunk_steps) {
  if (chunk_steps == nullptr) return fail(TA_EINVAL, "chunk_steps is NULL");
  *chunk_steps = 0;
  int64_t n_bh = 0, n_qblk = 0;
  ta_status vst = validate_args(a, &n_bh, &n_qblk, false);
  if (vst != TA_OK || n_qblk == 0 || !split_capable(a)) return vst;
  int ncu = 0;
  {
    std::lock_guard<std::mutex> lock(g_mu);
    DeviceGuard guard(a->device);
    if (guard.err != hipSuccess)
      return fail(TA_EHIP, "set device %d: %s", a->device, hipGetErrorString(guard.err));
    ta_status cst = cu_count_locked(a->device, &ncu);
    if (cst != TA_OK) return cst;
  }
  *chunk_steps = a->tile_m == 64 ? plan_split64(a->S, n_bh, a->causal != 0, a->D, ncu)
                                 : cached_split_plan(a->S, n_bh, a->causal != 0, ncu);
  return TA_OK;
}

int32_t ta_split_plan_model_rows(int64_t S, int64_t n_bh, int32_t causal, int32_t head_dim, int32_t rows,
                                 int32_t compute_units) {
  if (S <= 0 || n_bh <= 0 || compute_units <= 0 || S > 0x7fffffffLL || n_bh > 0x7fffffffLL) return 0;
  if (rows == 64) return plan_split64(S, n_bh, causal != 0, head_dim, compute_units);
  return rows == 128 ? plan_split(S, n_bh, causal != 0, compute_units) : 0;
}

int32_t ta_split_plan_model(int64_t S, int64_t n_bh, int32_t causal, int32_t compute_units) {
  if (S <= 0 || n_bh <= 0 || compute_units <= 0 || S > 0x7fffffffLL || n_bh > 0x7fffffffLL)
    return 0;
  return plan_split(S, n_bh, causal != 0, compute_units);
}

ta_status ta_split_workspace_size(const ta_fwd_args* a, int32_t chunk_steps, int64_t* bytes) {
  if (bytes == nullptr) return fail(TA_EINVAL, "bytes is NULL");
  *bytes = 0;
  if (chunk_steps < 0 && chunk_steps != TA_SPLIT_PAIRS) return fail(TA_EINVAL, "chunk_steps %d", chunk_steps);
  int64_t n_bh = 0, n_qblk = 0;
  ta_status vst = validate_args(a, &n_bh, &n_qblk, false);
  if (vst != TA_OK || n_qblk == 0 || chunk_steps == 0) return vst;
  // A chunk length that splits nothing runs whole rows (as ta_sdpa_fwd_split does): no
  // workspace, on any kernel.
  SplitLayout l;
  if (!layout_for(a->S, a->causal != 0, chunk_steps, &l)) return TA_OK;
  if (!split_runs(a, chunk_steps))
    return fail(TA_EUNSUPPORTED,
                "split key ranges need fp32 accumulation on tile (128, 64) or (128, 128) with D <= 160, "
                "or chunks on tile (64, 64) or (64, 128) with D = 64, 96, 128 or 160 (the paired split: "
                "128-row tiles)");
  *bytes = split_ws_bytes(n_bh, a->D, l);
  return TA_OK;
}

ta_status ta_sdpa_fwd_split(const ta_fwd_args* a, int32_t chunk_steps, void* workspace,
                            int64_t workspace_bytes, void* stream) {
  if (chunk_steps < 0 && chunk_steps != TA_SPLIT_PAIRS) return fail(TA_EINVAL, "chunk_steps %d", chunk_steps);
  int64_t n_bh = 0, n_qblk = 0;
  ta_status vst = validate_args(a, &n_bh, &n_qblk);
  if (vst != TA_OK || n_qblk == 0) return vst;
  SplitLayout l;
  if (chunk_steps == 0 || !layout_for(a->S, a->causal != 0, chunk_steps, &l))
    return ta_sdpa_fwd(a, stream);
  // Planned once before any device call (grids and the workspace are checked there), and
  // again under the lock with the device's compute-unit count, which decides whether the
  // split kernel merges its blocks itself.
  LaunchPlan pl;
  ta_status st = plan_launch(a, n_bh, n_qblk, chunk_steps, 1, &pl);
  if (st != TA_OK) return st;
  if (workspace == nullptr || workspace_bytes < pl.ws_bytes)
    return fail(TA_EINVAL, "workspace of %lld bytes needed, %lld given", (long long)pl.ws_bytes,
                (long long)(workspace == nullptr ? 0 : workspace_bytes));
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
    return fail(TA_EINVAL, "workspace must be 256-byte aligned");
  ta::FwdParams p;
  fill_params(a, n_bh, n_qblk, &p);
  const int64_t rows = n_bh * l.slots * kSplitRows;
  p.part_o = static_cast<float*>(workspace);
  p.part_lse = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                        (rows * a->D * 4 + 255) / 256 * 256);
  p.split_c = chunk_steps;
  p.split_items = static_cast<int32_t>(l.items);
  p.split_ns = chunk_steps == TA_SPLIT_PAIRS ? kPairCut : static_cast<int32_t>(l.ns);
  p.split_slots = static_cast<int32_t>(l.slots);

  // Resolve and launch under the cache lock, as ta_sdpa_fwd does.
  std::lock_guard<std::mutex> lock(g_mu);
  DeviceGuard guard(a->device);
  if (guard.err != hipSuccess)
    return fail(TA_EHIP, "set device %d: %s", a->device, hipGetErrorString(guard.err));
  int ncu = 0;
  st = cu_count_locked(a->device, &ncu);
  const ResolvedPlan* rp = nullptr;
  if (st == TA_OK) st = resolved_plan_locked(a, n_bh, n_qblk, chunk_steps, ncu, &rp);
  if (st != TA_OK) return st;
  return launch_plan_locked(a, *rp, &p, stream);
}

}  // extern "C"
