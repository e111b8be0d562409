// torch.ops.tiledattention.sdpa_fwd as a C++ operator, for callers without Python
// (libtorch, TorchScript) and without the Python layer's per-call overhead.
//
// Replaces the reference's torch extension registration (torch-ext/torch_binding.cpp:6-19,
// whose only op is an add-one placeholder, tiledattention_cuda/tiledattention.cu:13-33):
// the schema is defined here (TORCH_LIBRARY) and the implementation registered on the
// GPU dispatch key (CUDA, which HIP tensors carry on ROCm builds of torch).  The Python
// package registers the fake kernel for tracers (tiledattention/torch_op.py).
//
// A call does what tiledattention.sdpa does, in C++:
//   * the operator's tile / accum arguments, then scale, then the input checks, in the
//     order and with the messages of src/tiledattention/utils/checks.py:10-55 and
//     sdpa.py:37-47 (raised as c10::Error, a RuntimeError in Python);
//   * the TILEDATTN_* knobs read from the environment on every call and parsed as the
//     Python layer parses them (flash_fwd.py:47-146, 166-196, 225-226, 805-818), with the
//     operator's arguments taking the place of the tile and accumulation knobs;
//   * the call policy from the library (ta_plan_call: tile, accumulation, kernel head dim and
//     padding, aligned fast path, workgroup order, split), the same rules the Python layer
//     applies;
//   * inputs the kernels cannot read in place (host padding, strides, alignment) copied,
//     the output and any split workspace allocated through torch's caching allocator, and
//     the launch on torch's current stream of the inputs' device (ta_sdpa_fwd /
//     ta_sdpa_fwd_split).
#include <ATen/ATen.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <hip/hip_runtime.h>

#include <cctype>
#include <cerrno>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <optional>
#include <string>

#include "../../include/tiledattn.h"

namespace {

std::string trim(const char* s) {
  std::string t = s ? s : "";
  size_t a = 0, b = t.size();
  while (a < b && std::isspace((unsigned char)t[a])) ++a;
  while (b > a && std::isspace((unsigned char)t[b - 1])) --b;
  return t.substr(a, b - a);
}

std::string lower(std::string s) {
  for (auto& c : s) c = (char)std::tolower((unsigned char)c);
  return s;
}

// Integer env knob: unset or blank -> nullopt; else a base-10 integer (surrounding spaces
// allowed) or ValueError, as flash_fwd.py:47-65.
std::optional<long> env_int(const char* name) {
  const char* raw = std::getenv(name);
  std::string t = trim(raw);
  if (raw == nullptr || t.empty()) return std::nullopt;
  errno = 0;
  char* end = nullptr;
  const long v = std::strtol(t.c_str(), &end, 10);
  TORCH_CHECK_VALUE(errno == 0 && end && *end == '\0', "Environment variable ", name, " must be an integer.");
  return v;
}

void check_tile(long tm, long tn) {
  TORCH_CHECK_VALUE((tm == 64 || tm == 128) && (tn == 64 || tn == 128), "Unsupported tile (", tm, ", ", tn,
                    "): the gfx950 kernels are built for TILEDATTN_TILE_M and TILEDATTN_TILE_N in {64, 128}.");
}

struct CallKnobs {
  ta_call_knobs k{};
  std::string sync = "async";
};

// The knobs of one call (the operator's tile_m / tile_n / accum arguments, when given,
// take the place of TILEDATTN_TILE_M / _N and TILEDATTN_ACCUM_MODE).
CallKnobs read_knobs(int64_t tile_m, int64_t tile_n, int64_t accum) {
  CallKnobs c;
  // kernel options: parsed (integers) and otherwise without effect on precompiled kernels
  (void)env_int("TILEDATTN_KERNEL_OPT_LEVEL");
  (void)env_int("TILEDATTN_KERNEL_OCCUPANCY");
  (void)env_int("TILEDATTN_KERNEL_NUM_CTAS");
  const std::string sync = lower(trim(std::getenv("TILEDATTN_SYNC_MODE") ? std::getenv("TILEDATTN_SYNC_MODE") : "async"));
  TORCH_CHECK_VALUE(sync == "async" || sync == "post" || sync == "strict", "Unsupported TILEDATTN_SYNC_MODE='",
                    sync, "'. Use one of: strict, post, async.");
  c.sync = sync;
  if (tile_m != 0) {
    c.k.tile_m = (int32_t)tile_m;
    c.k.tile_n = (int32_t)tile_n;
  } else {
    const auto tm = env_int("TILEDATTN_TILE_M");
    const auto tn = env_int("TILEDATTN_TILE_N");
    if (tm || tn) {
      const long m = tm.value_or(64), n = tn.value_or(64);
      TORCH_CHECK_VALUE(m > 0 && n > 0, "TILEDATTN_TILE_M and TILEDATTN_TILE_N must be positive.");
      check_tile(m, n);
      c.k.tile_m = (int32_t)m;
      c.k.tile_n = (int32_t)n;
    }
  }
  if (accum != -1) {
    c.k.accum = (int32_t)accum;
  } else {
    const char* raw = std::getenv("TILEDATTN_ACCUM_MODE");
    const std::string mode = lower(trim(raw));
    if (raw == nullptr || mode.empty() || mode == "auto") {
      c.k.accum = -1;
    } else {
      TORCH_CHECK_VALUE(mode == "fp32" || mode == "fp16", "Unsupported TILEDATTN_ACCUM_MODE='", mode,
                        "'. Use one of: auto, fp32, fp16.");
      c.k.accum = mode == "fp16" ? TA_ACC_INPUT : TA_ACC_FP32;
    }
  }
  const std::string dis = trim(std::getenv("TILEDATTN_DISABLE_ALIGNED_FASTPATH"));
  c.k.aligned = (dis.empty() || dis == "0" || dis == "false" || dis == "False") ? 1 : 0;
  const std::string sched = trim(std::getenv("TILEDATTN_SCHED"));
  if (sched.empty()) {
    c.k.sched = -1;
  } else {
    TORCH_CHECK_VALUE(sched == "0" || sched == "1" || sched == "2" || sched == "3", "Unsupported TILEDATTN_SCHED='",
                      sched, "'. Use 0, 1, 2 or 3.");
    c.k.sched = sched[0] - '0';
  }
  const std::string split = lower(trim(std::getenv("TILEDATTN_SPLIT")));
  if (split.empty() || split == "auto") {
    c.k.split = TA_SPLIT_AUTO;
  } else if (split == "0" || split == "off") {
    c.k.split = 0;
  } else if (split == "pairs") {
    c.k.split = TA_SPLIT_PAIRS;
  } else {
    errno = 0;
    char* end = nullptr;
    const long v = std::strtol(split.c_str(), &end, 10);
    TORCH_CHECK_VALUE(errno == 0 && end && *end == '\0',
                      "TILEDATTN_SPLIT must be 'auto', 'off', 'pairs' or an integer, got '", split, "'.");
    TORCH_CHECK_VALUE(v >= 0, "TILEDATTN_SPLIT must be >= 0, got ", v, ".");
    c.k.split = (int32_t)v;
  }
  // TILEDATTN_CHUNKED_HEAD_DIMS: a chunked plan runs the same kernels; only its syntax is checked
  const std::string chunked = trim(std::getenv("TILEDATTN_CHUNKED_HEAD_DIMS"));
  if (!chunked.empty()) {
    size_t pos = 0;
    while (pos <= chunked.size()) {
      size_t comma = chunked.find(',', pos);
      if (comma == std::string::npos) comma = chunked.size();
      const std::string item = trim(chunked.substr(pos, comma - pos).c_str());
      if (!item.empty()) {
        char* end = nullptr;
        (void)std::strtol(item.c_str(), &end, 10);
        TORCH_CHECK_VALUE(end && *end == '\0',
                          "Environment variable TILEDATTN_CHUNKED_HEAD_DIMS must be a comma-separated list of integers.");
      }
      pos = comma + 1;
    }
  }
  return c;
}

// Whether the kernels read a [B, H, S, D] view in place: unit last stride, 16-byte rows, rows
// that do not overlap, 32-bit buffer ranges, 16-byte aligned base.
bool readable_in_place(const at::Tensor& t, int64_t width) {
  const auto st = t.strides();
  const int64_t row = st[2];
  for (int i = 0; i < 3; ++i)
    if (st[i] < 0 || st[i] % 8 != 0) return false;
  return st[3] == 1 && t.size(3) == width && row >= width && row < (int64_t(1) << 23) &&
         t.size(2) * row * 2 < (int64_t(1) << 31) && reinterpret_cast<uintptr_t>(t.data_ptr()) % 16 == 0;
}

void check_status(ta_status st) {
  if (st == TA_OK) return;
  TORCH_CHECK(false, ta_status_string(st), ": ", ta_last_error());
}

at::Tensor sdpa_fwd_hip(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, bool causal,
                        std::optional<double> scale, int64_t tile_m, int64_t tile_n, int64_t accum) {
  // the operator's own arguments first (tiledattention/torch_op.py _overrides)
  TORCH_CHECK_VALUE((tile_m == 0) == (tile_n == 0),
                    "tile_m and tile_n must both be 0 (use the knobs) or both be given.");
  if (tile_m != 0)
    TORCH_CHECK_VALUE((tile_m == 64 || tile_m == 128) && (tile_n == 64 || tile_n == 128), "Unsupported tile (",
                      tile_m, ", ", tile_n, "): tiles are 64 or 128.");
  TORCH_CHECK_VALUE(accum == -1 || accum == 0 || accum == 1,
                    "accum must be -1 (knob), 0 (fp32) or 1 (input dtype), got ", accum, ".");
  // sdpa.py:39-40 (NaN and inf pass, as there)
  TORCH_CHECK(!(scale.has_value() && *scale <= 0.0), "scale must be a positive number when provided.");
  // utils/checks.py:34-55
  const at::Tensor* qkv[3] = {&q, &k, &v};
  const char* nm[3] = {"q", "k", "v"};
  for (int i = 0; i < 3; ++i) {
    TORCH_CHECK(qkv[i]->dim() == 4, nm[i], " must have shape [B, H, S, D].");
    TORCH_CHECK(qkv[i]->is_cuda(), nm[i], " must be a CUDA tensor.");
  }
  TORCH_CHECK(q.sizes() == k.sizes() && q.sizes() == v.sizes(), "q, k, and v must have matching shape [B, H, S, D].");
  TORCH_CHECK(q.device() == k.device() && q.device() == v.device(), "q, k, and v must be on the same CUDA device.");
  const auto dt = q.scalar_type();
  TORCH_CHECK(dt == at::kHalf || dt == at::kBFloat16, "q dtype must be torch.float16 or torch.bfloat16.");
  TORCH_CHECK(k.scalar_type() == dt && v.scalar_type() == dt, "q, k, and v must have identical dtype.");
  const int64_t B = q.size(0), H = q.size(1), S = q.size(2), D = q.size(3);
  TORCH_CHECK(D != 0, "head dimension D must be positive.");
  const double sc = scale.has_value() ? *scale : 1.0 / std::sqrt((double)D);

  const CallKnobs kn = read_knobs(tile_m, tile_n, accum);
  const int device = q.device().index();
  ta_call_plan plan;
  check_status(ta_plan_call(B, H, S, D, dt == at::kBFloat16 ? TA_BF16 : TA_FP16, causal ? 1 : 0, device, 0,
                            &kn.k, &plan));
  at::Tensor out = at::empty({B, H, S, plan.out_width}, q.options().memory_format(at::MemoryFormat::Contiguous));
  if (B * H == 0 || S == 0) return plan.host_pad ? out.narrow(3, 0, D).contiguous() : out;

  const int64_t width = plan.out_width;
  auto ready = [&](const at::Tensor& t) {
    if (plan.host_pad > 0) return at::constant_pad_nd(t, {0, plan.host_pad}).contiguous();
    if (readable_in_place(t, width)) return t;
    return t.clone(at::MemoryFormat::Contiguous);
  };
  const at::Tensor qr = ready(q), kr = ready(k), vr = ready(v);
  ta_fwd_args a = plan.args;
  a.q = qr.data_ptr();
  a.k = kr.data_ptr();
  a.v = vr.data_ptr();
  a.o = out.data_ptr();
  const at::Tensor* rs[4] = {&qr, &kr, &vr, &out};
  int64_t* dst[4] = {a.q_stride, a.k_stride, a.v_stride, a.o_stride};
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 4; ++j) dst[i][j] = rs[i]->stride(j);
  a.scale = (float)sc;
  auto stream = c10::hip::getCurrentHIPStream(device);
  if (kn.sync == "strict") stream.synchronize();
  if (plan.chunk_steps == 0) {
    check_status(ta_sdpa_fwd(&a, stream.stream()));
  } else {
    // 256-byte aligned blocks from torch's caching allocator, stream-ordered
    at::Tensor ws = at::empty({plan.workspace_bytes}, q.options().dtype(at::kByte));
    check_status(ta_sdpa_fwd_split(&a, plan.chunk_steps, ws.data_ptr(), plan.workspace_bytes, stream.stream()));
  }
  if (kn.sync == "strict" || kn.sync == "post") stream.synchronize();
  return plan.host_pad ? out.narrow(3, 0, D).contiguous() : out;
}

}  // namespace

TORCH_LIBRARY(tiledattention, m) {
  m.def(
      "sdpa_fwd(Tensor q, Tensor k, Tensor v, bool causal=False, float? scale=None, int tile_m=0, "
      "int tile_n=0, int accum=-1) -> Tensor");
}

TORCH_LIBRARY_IMPL(tiledattention, CUDA, m) { m.impl("sdpa_fwd", &sdpa_fwd_hip); }
