// C-ABI of librepresentax_amd: validation, workspace planning and launch
// sequencing for the quantized-linear path. No entry point allocates device
// memory or synchronizes; every launch goes to the caller's stream.
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <string>
#include <utility>

#include "../../include/representax_amd.h"
#include "common.h"
#include "act.h"
#include "kernels.h"
#include "tuning.h"

namespace rpx {

namespace {
thread_local std::string g_last_error;

// Bump allocator over a caller-provided workspace.
struct Arena {
  uint8_t* base;
  size_t cap;
  size_t used = 0;
  bool overflow = false;
  Arena(void* p, size_t c) : base(static_cast<uint8_t*>(p)), cap(c) {}
  template <typename T>
  T* take(int64_t count) {
    const size_t bytes = (static_cast<size_t>(count) * sizeof(T) + 255) & ~static_cast<size_t>(255);
    if (used + bytes > cap) {
      overflow = true;
      return nullptr;
    }
    T* p = reinterpret_cast<T*>(base + used);
    used += bytes;
    return p;
  }
};

// Size-only twin of Arena.
struct Sizer {
  size_t used = 0;
  template <typename T>
  void take(int64_t count) {
    used += (static_cast<size_t>(count) * sizeof(T) + 255) & ~static_cast<size_t>(255);
  }
};

size_t elem_size(int dtype) { return dtype == kBF16 ? 2 : 4; }
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
// Every non-null pointer 16-byte aligned.
bool aligned16_all(std::initializer_list<const void*> ps) {
  for (const void* p : ps)
    if (p != nullptr && !aligned16(p)) return false;
  return true;
}
bool pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

float round_to_dtype(float v, int dtype) {
  if (dtype != kBF16) return v;
  uint32_t u;
  std::memcpy(&u, &v, 4);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return v;
  u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
  float r;
  std::memcpy(&r, &u, 4);
  return r;
}

int check_int4_shape(int64_t n, int64_t k, int64_t group_size, int64_t* n_groups, int64_t* group) {
  if (n < 0 || k <= 0) return fail_invalid("INT4 weight needs n >= 0 and k > 0");
  if (group_size <= 0 || group_size == k) {
    *n_groups = 1;
    *group = k;
    return kOk;
  }
  if (k % group_size != 0) return fail_invalid("group_size must divide the input size");
  if (group_size % 2 != 0) return fail_invalid("group_size must be even");
  *n_groups = k / group_size;
  *group = group_size;
  return kOk;
}

int check_dtype(int dtype) {
  if (dtype != kF32 && dtype != kBF16) return fail_invalid("dtype must be RPX_DTYPE_F32 or RPX_DTYPE_BF16");
  return kOk;
}

int check_fmt(int fmt) {
  if (fmt != kE4M3FN && fmt != kE5M2) return fail_invalid("fp8 format must be RPX_FP8_E4M3FN or RPX_FP8_E5M2");
  return kOk;
}

#define RPX_TRY(expr)            \
  do {                           \
    const int _rc = (expr);      \
    if (_rc != kOk) return _rc;  \
  } while (0)

#define RPX_HIP(expr, what) RPX_TRY(check_hip((expr), (what)))

// --- INT4 + LoRA path selection -------------------------------------------
bool lora_fast_shape(int dtype, int64_t k, int64_t n_groups, int64_t group, int64_t rank) {
  if (dtype != kBF16) return false;
  if (k % 64 != 0) return false;
  if (rank < 1 || rank > 64) return false;
  if (n_groups > 1 && !(pow2(group) && group >= 32)) return false;
  return true;
}

bool lora_skinny(int dtype, int64_t m, int64_t n, int64_t k, int64_t n_groups, int64_t group,
                 int64_t rank) {
  return dtype == kBF16 && skinny_ok(m, n, k, rank, n_groups, group);
}

template <typename A>
void plan_forward(A& a, bool fast, bool skinny, int64_t m, int64_t n, int64_t k, int64_t rank) {
  if (skinny) {
    a.template take<float>(skinny_workspace_floats(m, n, k, rank));
    return;
  }
  if (fast) return;
  a.template take<float>(m * n);  // base product
  a.template take<float>(m * n);  // adapter product
  a.template take<float>(m * rank);
}

template <typename A>
void plan_backward(A& a, bool fast, int64_t m, int64_t n, int64_t k, int64_t rank, int dtype) {
  if (fast) {
    a.template take<uint16_t>(rank * n);  // B^T
    a.template take<uint16_t>(k * rank);  // A^T
    a.template take<uint16_t>(m * rank);  // dh
    a.template take<uint16_t>(k * n);     // W_b^T
    a.template take<float>(rank_tn_workspace_floats(m, n, rank));  // dB partials
    a.template take<float>(rank_tn_workspace_floats(m, rank, k));  // dA partials
    return;
  }
  a.template take<uint8_t>(m * n * static_cast<int64_t>(elem_size(dtype)));  // g_a
  a.template take<uint8_t>(m * rank * static_cast<int64_t>(elem_size(dtype)));  // dh
  a.template take<float>(m * rank);  // dh (f32 product)
  a.template take<float>(m * k);     // g W
  a.template take<float>(m * k);     // dh A
}

__global__ void __launch_bounds__(256)
    k_lora_combine(const float* __restrict__ base, const float* __restrict__ lowrank,
                   int64_t rows, int64_t cols, float scale, const uint16_t* __restrict__ bias,
                   int dtype, void* __restrict__ out) {
  const int64_t total = rows * cols;
  for (int64_t e = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; e < total;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    float y;
    if (dtype == kBF16) {
      y = round_bf16(round_bf16(base[e]) + round_bf16(round_bf16(lowrank[e]) * scale));
      if (bias != nullptr) y = round_bf16(y + bf16_to_f32(bias[e % cols]));
      static_cast<uint16_t*>(out)[e] = f32_to_bf16(y);
    } else {
      y = base[e] + lowrank[e] * scale;
      if (bias != nullptr) y = y + bf16_to_f32(bias[e % cols]);
      static_cast<float*>(out)[e] = y;
    }
  }
}

__global__ void __launch_bounds__(256)
    k_scale_round(const void* __restrict__ in, int64_t n, float scale, int dtype,
                  void* __restrict__ out) {
  for (int64_t e = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; e < n;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    if (dtype == kBF16) {
      const float v = bf16_to_f32(static_cast<const uint16_t*>(in)[e]) * scale;
      static_cast<uint16_t*>(out)[e] = f32_to_bf16(v);
    } else {
      static_cast<float*>(out)[e] = static_cast<const float*>(in)[e] * scale;
    }
  }
}

__global__ void __launch_bounds__(256)
    k_round_inplace_f32(float* __restrict__ buf, int64_t n, int dtype) {
  for (int64_t e = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; e < n;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x)
    if (dtype == kBF16) buf[e] = round_bf16(buf[e]);
}

int grid1d(int64_t work) {
  int64_t g = ceil_div(work, 256);
  if (g > 8192) g = 8192;
  if (g < 1) g = 1;
  return static_cast<int>(g);
}

}  // namespace

// --- tuning knobs --------------------------------------------------------------
namespace {

bool knob_value_ok(int knob, int v) {
  switch (knob) {
    case kTuneInt4Tile:
      return v == kTileAuto || v == kTileI4_256x128 || v == kTileI4_128x128 ||
             v == kTileI4_64x128 || v == kTileI4_256x256 || v == kTileI4_128x128s2 ||
             v == kTileI4_128x128s3 || v == kTileI4_256x128s2 || v == kTileI4L_256x192;
    case kTuneBf16Tile:
      return v == kTileAuto || v == kTileBf_256x128 || v == kTileBf_128x128 ||
             v == kTileBf_64x128 || v == kTileBf_256x256 || v == kTileBf_128x96 ||
             v == kTileBf_256x128s3 || v == kTileT4_256x128 || v == kTileT4_128x128 ||
             v == kTileT4_64x128;
    case kTuneFp8Tile: return v >= 0 && v < fp8_tile_count();
    case kTuneSkinnyTile: return v >= 0 && v <= skinny_tile_count();
    case kTuneSkinny2: return v >= -1 && v <= 1;
    case kTuneSkinny2One: return v >= -1 && v <= 1;
    case kTuneSpinLimit: return v >= 0;
    case kTuneBand: return v >= 0 && v <= 64;
    case kTuneDxPacked: return v >= -1 && v <= 1;
    case kTuneRankBlocks: return v == 0 || (v >= 16 && v <= 8192);
    case kTuneRankNtU: return v == 0 || v == 4 || v == 8 || v == 16;
    case kTuneFp8Splits: return v >= 0 && v <= 32;
    case kTuneFp8Pair: return v == -1 || v == 0;
    default: return false;
  }
}

int env_int(const char* name, int fallback) {
  const char* v = std::getenv(name);
  return v != nullptr && *v != '\0' ? std::atoi(v) : fallback;
}

struct Knobs {
  std::atomic<int> v[kTuneCount];
  Knobs() {
    const int defaults[kTuneCount] = {0, 0, 0, 0, -1, -1, 0, 0, -1, 0, 0, 0, -1};
    for (int i = 0; i < kTuneCount; ++i) v[i].store(defaults[i], std::memory_order_relaxed);
    // RPX_GEMM_TILE names a tile of either GEMM (the id sets are disjoint)
    const int gemm = env_int("RPX_GEMM_TILE", 0);
    if (knob_value_ok(kTuneInt4Tile, gemm)) v[kTuneInt4Tile].store(gemm);
    if (knob_value_ok(kTuneBf16Tile, gemm)) v[kTuneBf16Tile].store(gemm);
    const std::pair<int, const char*> envs[] = {{kTuneFp8Tile, "RPX_FP8_TILE"},
                                                {kTuneSkinnyTile, "RPX_SKINNY_TILE"},
                                                {kTuneSkinny2, "RPX_SKINNY2"},
                                                {kTuneSkinny2One, "RPX_SKINNY2_ONE"},
                                                {kTuneBand, "RPX_GEMM_BAND"},
                                                {kTuneDxPacked, "RPX_DX_PACKED"},
                                                {kTuneFp8Pair, "RPX_FP8_PAIR"}};
    for (const auto& e : envs) {
      const int val = env_int(e.second, v[e.first].load());
      if (knob_value_ok(e.first, val)) v[e.first].store(val);
    }
  }
};

Knobs& knobs() {
  static Knobs k;  // thread-safe one-time initialization
  return k;
}

}  // namespace

int tune(int knob) {
  if (knob < 0 || knob >= kTuneCount) return 0;
  return knobs().v[knob].load(std::memory_order_relaxed);
}

bool tune_set(int knob, int value) {
  if (!knob_value_ok(knob, value)) return false;
  knobs().v[knob].store(value, std::memory_order_relaxed);
  return true;
}

// --- device error word -----------------------------------------------------------
namespace {
// [0]: bits kDevErr*, per device; [1]: the bits the last check took
__device__ unsigned int g_device_error[2];
constexpr int kMaxDevices = 64;
std::atomic<unsigned int*> g_error_ptr[kMaxDevices];

// Takes the error bits in one atomic exchange, so a bit that another
// stream's kernel raises after it stays in the word for the next check.
__global__ void k_take_device_errors(unsigned int* word) {
  if (threadIdx.x == 0)
    word[1] = __hip_atomic_exchange(word, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
}  // namespace

unsigned int* device_error_word() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  unsigned int* p = g_error_ptr[dev].load(std::memory_order_acquire);
  if (p != nullptr) return p;
  void* addr = nullptr;
  if (hipGetSymbolAddress(&addr, HIP_SYMBOL(g_device_error)) != hipSuccess) return nullptr;
  p = static_cast<unsigned int*>(addr);
  g_error_ptr[dev].store(p, std::memory_order_release);
  return p;
}

hipError_t ensure_lds_limit(const void* kernel, int bytes, std::atomic<unsigned>& done_devices) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const unsigned bit = 1u << (dev & 31);
  if (done_devices.load(std::memory_order_acquire) & bit) return hipSuccess;
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e != hipSuccess) return e;
  done_devices.fetch_or(bit, std::memory_order_acq_rel);
  return hipSuccess;
}

void set_error(const std::string& msg) { g_last_error = msg; }

int fail_invalid(const std::string& msg) {
  g_last_error = msg;
  return kErrInvalid;
}

int check_hip(hipError_t err, const char* what) {
  if (err == hipSuccess) return kOk;
  g_last_error = std::string(what) + ": " + hipGetErrorString(err);
  return kErrHip;
}

}  // namespace rpx

using namespace rpx;

extern "C" {

const char* rpx_last_error(void) { return g_last_error.c_str(); }

int rpx_abi_version(void) { return RPX_ABI_VERSION; }

int rpx_set_tuning(int knob, int value) {
  if (!tune_set(knob, value)) return fail_invalid("rpx_set_tuning: unknown knob or value");
  return kOk;
}

int rpx_get_tuning(int knob) { return tune(knob); }

int rpx_check_device_errors(void* stream, uint32_t* flags_out) {
  if (flags_out != nullptr) *flags_out = 0;
  unsigned int* word = device_error_word();
  if (word == nullptr) return check_hip(hipErrorInvalidSymbol, "rpx_check_device_errors");
  // the exchange runs after the work already queued on `stream`
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_take_device_errors, dim3(1), dim3(64), 0, s, word);
  RPX_HIP(hipGetLastError(), "rpx_check_device_errors: take");
  unsigned int bits = 0;
  RPX_HIP(hipMemcpyAsync(&bits, word + 1, sizeof(bits), hipMemcpyDeviceToHost, s),
          "rpx_check_device_errors: read");
  RPX_HIP(hipStreamSynchronize(s), "rpx_check_device_errors: sync");
  if (bits == 0) return kOk;
  if (flags_out != nullptr) *flags_out = bits;
  std::string msg = "a kernel's bounded wait expired (its outputs hold NaN):";
  if (bits & kDevErrSkinnyWait) msg += " skinny-M forward (one launch, M <= 64): adapter arrivals;";
  if (bits & kDevErrSkinnyOneWait) msg += " skinny-M forward (one launch, M <= 4): adapter partials;";
  set_error(msg);
  return kErrDevice;
}

// ---------------------------------------------------------------------------
// INT4 codec
// ---------------------------------------------------------------------------
int rpx_int4_pack(const void* weight, int dtype, int64_t n, int64_t k, int64_t group_size,
                  uint8_t* packed, uint16_t* scale_bits, void* stream) {
  RPX_TRY(check_dtype(dtype));
  int64_t ng, g;
  RPX_TRY(check_int4_shape(n, k, group_size, &ng, &g));
  if (n > 0 && (weight == nullptr || packed == nullptr || scale_bits == nullptr))
    return fail_invalid("rpx_int4_pack: null pointer");
  RPX_HIP(launch_int4_pack(weight, dtype, packed, scale_bits, n, k, (k + 1) / 2, ng, g,
                           static_cast<hipStream_t>(stream)),
          "rpx_int4_pack");
  return kOk;
}

int rpx_int4_dequant(const uint8_t* packed, const uint16_t* scale_bits, int64_t n, int64_t k,
                     int64_t group_size, uint16_t* out, void* stream) {
  int64_t ng, g;
  RPX_TRY(check_int4_shape(n, k, group_size, &ng, &g));
  if (n > 0 && (packed == nullptr || scale_bits == nullptr || out == nullptr))
    return fail_invalid("rpx_int4_dequant: null pointer");
  RPX_HIP(launch_int4_dequant(packed, scale_bits, out, n, k, (k + 1) / 2, ng, g,
                              static_cast<hipStream_t>(stream)),
          "rpx_int4_dequant");
  return kOk;
}

int rpx_int4_merge(const uint8_t* packed, const uint16_t* scale_bits, const float* lora_a,
                   const float* lora_b, int64_t n, int64_t k, int64_t group_size, int64_t rank,
                   float scaling, float* out, void* stream) {
  int64_t ng, g;
  RPX_TRY(check_int4_shape(n, k, group_size, &ng, &g));
  if (rank < 0) return fail_invalid("rank must be non-negative");
  if (n > 0 && (packed == nullptr || scale_bits == nullptr || out == nullptr ||
                (rank > 0 && (lora_a == nullptr || lora_b == nullptr))))
    return fail_invalid("rpx_int4_merge: null pointer");
  RPX_HIP(launch_int4_merge(packed, scale_bits, lora_a, lora_b, out, n, k, (k + 1) / 2, ng, g,
                            rank, scaling, static_cast<hipStream_t>(stream)),
          "rpx_int4_merge");
  return kOk;
}

// ---------------------------------------------------------------------------
// INT4 + LoRA linear
// ---------------------------------------------------------------------------
size_t rpx_int4lora_forward_workspace(int64_t m, int64_t n, int64_t k, int64_t group_size,
                                      int64_t rank, int dtype) {
  int64_t ng = 1, g = k;
  if (group_size > 0 && group_size != k && k % group_size == 0) {
    ng = k / group_size;
    g = group_size;
  }
  Sizer s;
  plan_forward(s, lora_fast_shape(dtype, k, ng, g, rank), lora_skinny(dtype, m, n, k, ng, g, rank), m,
               n, k, rank);
  return s.used;
}

namespace {

// Activation applied to a linear's output (ActMode) and its [M, N] operands.
struct ActIO {
  int mode = kActNone;
  const uint16_t* aux = nullptr;
  const uint16_t* aux2 = nullptr;
  uint16_t* pre_out = nullptr;  // forward modes: the linear's own output
  uint16_t* out2 = nullptr;     // SiLU-mul backward: d gate
  bool h_given = false;         // forward: h = x A^T is already in h (MFMA path only)
};

int int4lora_forward_impl(const void* x, int dtype, int64_t m, int64_t k, const uint8_t* packed,
                          const uint16_t* scale_bits, int64_t n, int64_t group_size,
                          const uint16_t* bias_bits, const void* lora_a, const void* lora_b,
                          int64_t rank, float scaling, void* y, void* h, void* workspace,
                          size_t workspace_bytes, void* stream, const ActIO& act) {
  RPX_TRY(check_dtype(dtype));
  int64_t ng, g;
  RPX_TRY(check_int4_shape(n, k, group_size, &ng, &g));
  if (m < 0) return fail_invalid("m must be non-negative");
  if (rank < 1 || rank > n || rank > k) return fail_invalid("adapter rank must fit both linear dimensions");
  if (m == 0 || n == 0) return kOk;
  if (x == nullptr || packed == nullptr || scale_bits == nullptr || lora_a == nullptr ||
      lora_b == nullptr || y == nullptr || h == nullptr)
    return fail_invalid("rpx_int4lora_forward: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const float c = round_to_dtype(scaling, dtype);
  const int64_t pc = (k + 1) / 2;
  Int4Operand w;
  w.packed = packed;
  w.packed_cols = pc;
  w.scales = scale_bits;
  w.n_groups = ng;
  w.group = g;
  // the workspace query sizes the MFMA and skinny paths from the shape alone;
  // those paths load every operand in 16-byte vectors
  const bool fast = lora_fast_shape(dtype, k, ng, g, rank);
  if ((fast || lora_skinny(dtype, m, n, k, ng, g, rank)) &&
      !aligned16_all({x, packed, scale_bits, lora_a, y}))
    return fail_invalid(
        "rpx_int4lora_forward: this shape takes the vectorized kernels, which need x, packed, "
        "scale_bits, lora_a and y 16-byte aligned");
  Arena arena(workspace, workspace_bytes);
  // where the paths without the activation epilogue put the linear's output;
  // the activation then runs elementwise from there into y
  void* lin = act.mode != kActNone ? static_cast<void*>(act.pre_out) : y;
  auto finish_act = [&]() -> int {
    if (act.mode != kActNone)
      RPX_HIP(launch_act(act.mode, act.pre_out, act.aux, nullptr, m * n, static_cast<uint16_t*>(y),
                         nullptr, st),
              "int4lora_forward: activation");
    return kOk;
  };
  if (lora_skinny(dtype, m, n, k, ng, g, rank)) {
    float* ws = arena.take<float>(skinny_workspace_floats(m, n, k, rank));
    if (arena.overflow) return fail_invalid("rpx_int4lora_forward: workspace too small");
    if (skinny2_selected(m, n, k, rank, ng, g)) {
      RPX_HIP(launch_skinny2_forward(static_cast<const uint16_t*>(x), m, k, w, n,
                                     static_cast<const uint16_t*>(lora_a),
                                     static_cast<const uint16_t*>(lora_b), rank, c, bias_bits,
                                     static_cast<uint16_t*>(lin), static_cast<uint16_t*>(h), ws,
                                     st),
              "int4lora_forward: skinny-M row-block kernels");
      return finish_act();
    }
    RPX_HIP(launch_skinny_forward(static_cast<const uint16_t*>(x), m, k, w, n,
                                  static_cast<const uint16_t*>(lora_a),
                                  static_cast<const uint16_t*>(lora_b), rank, c, bias_bits,
                                  static_cast<uint16_t*>(lin), static_cast<uint16_t*>(h), ws, st),
            "int4lora_forward: skinny-M kernels");
    return finish_act();
  }
  if (act.h_given && !fast) return fail_invalid("int4lora_forward: a given h needs the MFMA path");
  if (fast) {
    const uint16_t* xb = static_cast<const uint16_t*>(x);
    uint16_t* hb = static_cast<uint16_t*>(h);
    if (!act.h_given)
      RPX_HIP(launch_rank_nt(xb, k, static_cast<const uint16_t*>(lora_a), k, m, rank, k, false,
                             1.0f, hb, rank, st),
              "int4lora_forward: adapter down-projection");
    LowRankEpilogue epi;
    epi.rows = static_cast<const uint16_t*>(lora_b);
    epi.rows_sn = rank;
    epi.rows_sj = 1;
    epi.cols = hb;
    epi.cols_sm = rank;
    epi.cols_sj = 1;
    epi.rank = rank;
    epi.scale = c;
    epi.bias = bias_bits;
    epi.act = act.mode;
    epi.aux = act.aux;
    epi.pre_out = act.pre_out;
    RPX_HIP(launch_gemm_int4(xb, k, w, m, n, k, static_cast<uint16_t*>(y), n, epi, st),
            "int4lora_forward: fused dequant GEMM");
    return kOk;
  }
  float* base = arena.take<float>(m * n);
  float* low = arena.take<float>(m * n);
  float* hf = arena.take<float>(m * rank);
  if (arena.overflow) return fail_invalid("rpx_int4lora_forward: workspace too small");
  RPX_HIP(launch_generic_gemm(x, dtype, k, 1, nullptr, dtype, 0, 0, &w, false, m, n, k, base, st),
          "int4lora_forward: base product");
  RPX_HIP(launch_generic_gemm(x, dtype, k, 1, lora_a, dtype, k, 1, nullptr, false, m, rank, k, hf,
                              st),
          "int4lora_forward: adapter down-projection");
  RPX_HIP(launch_round_store(hf, m * rank, dtype, h, st), "int4lora_forward: round h");
  RPX_HIP(launch_generic_gemm(h, dtype, rank, 1, lora_b, dtype, rank, 1, nullptr, false, m, n,
                              rank, low, st),
          "int4lora_forward: adapter up-projection");
  hipLaunchKernelGGL(k_lora_combine, dim3(grid1d(m * n)), dim3(256), 0, st, base, low, m, n, c,
                     bias_bits, dtype, lin);
  RPX_HIP(hipGetLastError(), "int4lora_forward: combine");
  return finish_act();
}

}  // namespace

int rpx_int4lora_forward(const void* x, int dtype, int64_t m, int64_t k, const uint8_t* packed,
                         const uint16_t* scale_bits, int64_t n, int64_t group_size,
                         const uint16_t* bias_bits, const void* lora_a, const void* lora_b,
                         int64_t rank, float scaling, void* y, void* h, void* workspace,
                         size_t workspace_bytes, void* stream) {
  return int4lora_forward_impl(x, dtype, m, k, packed, scale_bits, n, group_size, bias_bits, lora_a,
                               lora_b, rank, scaling, y, h, workspace, workspace_bytes, stream,
                               ActIO{});
}

}  // extern "C"

namespace {

// The fused form of rpx_int4lora_forward_multi: bf16, every projection on
// the two-launch skinny path (M <= 4 by default), one rank, at most 4
// projections, 16-byte aligned operands. Fills `out` when it applies.
bool multi_fused_shape(int dtype, int64_t m, int64_t k, int count,
                       const rpx_int4lora_projection* proj, Skinny2Projection* out) {
  if (dtype != kBF16 || count < 2 || count > 4 || m < 1) return false;
  for (int i = 0; i < count; ++i) {
    const rpx_int4lora_projection& q = proj[i];
    int64_t ng = 1, g = k;
    if (q.group_size > 0 && q.group_size != k) {
      if (k % q.group_size != 0) return false;
      ng = k / q.group_size;
      g = q.group_size;
    }
    if (q.rank != proj[0].rank || q.n < 1 || q.rank < 1 || q.rank > q.n || q.rank > k)
      return false;
    if (!lora_skinny(dtype, m, q.n, k, ng, g, q.rank) ||
        !skinny2_selected(m, q.n, k, q.rank, ng, g))
      return false;
    Skinny2Projection& o = out[i];
    o.w.packed = q.packed;
    o.w.packed_cols = (k + 1) / 2;
    o.w.scales = q.scale_bits;
    o.w.n_groups = ng;
    o.w.group = g;
    o.n = q.n;
    o.lora_a = static_cast<const uint16_t*>(q.lora_a);
    o.lora_b = static_cast<const uint16_t*>(q.lora_b);
    o.rank = q.rank;
    o.scale = round_to_dtype(q.scaling, dtype);
    o.bias = q.bias_bits;
    o.y = static_cast<uint16_t*>(q.y);
    o.h = static_cast<uint16_t*>(q.h);
  }
  return skinny2_multi_ok(m, k, count, out);
}

// The MFMA form of rpx_int4lora_forward_multi above the small-M sizes: every
// projection on the fused dequant GEMM path (bf16, not skinny, the usual
// alignment), their adapters together at most eight 16-rank blocks. The h of
// every projection then comes from one pass over x, and each GEMM takes its
// h as given.
bool multi_shared_h(const void* x, int dtype, int64_t m, int64_t k, int count,
                    const rpx_int4lora_projection* proj) {
  if (x == nullptr || dtype != kBF16 || count < 2 || m < 1) return false;
  int blocks = 0;
  for (int i = 0; i < count; ++i) {
    const rpx_int4lora_projection& q = proj[i];
    int64_t ng = 1, g = k;
    if (q.group_size > 0 && q.group_size != k) {
      if (k % q.group_size != 0) return false;
      ng = k / q.group_size;
      g = q.group_size;
    }
    if (q.n < 1 || q.rank < 1 || q.rank > q.n || q.rank > k) return false;
    if (!lora_fast_shape(dtype, k, ng, g, q.rank) || lora_skinny(dtype, m, q.n, k, ng, g, q.rank))
      return false;
    if (q.packed == nullptr || q.scale_bits == nullptr || q.lora_a == nullptr ||
        q.lora_b == nullptr || q.y == nullptr || q.h == nullptr ||
        !aligned16_all({x, q.packed, q.scale_bits, q.lora_a, q.y}))
      return false;
    blocks += rank_nt_blocks_of(q.rank);
    if (blocks > rank_nt_max_blocks()) return false;
  }
  return true;
}

bool multi_fused(const void* x, int dtype, int64_t m, int64_t k, int count,
                 const rpx_int4lora_projection* proj, Skinny2Projection* out) {
  if (x == nullptr || !multi_fused_shape(dtype, m, k, count, proj, out)) return false;
  for (int i = 0; i < count; ++i) {
    const rpx_int4lora_projection& q = proj[i];
    if (q.packed == nullptr || q.scale_bits == nullptr || q.lora_a == nullptr ||
        q.lora_b == nullptr || q.y == nullptr || q.h == nullptr ||
        !aligned16_all({x, q.packed, q.scale_bits, q.lora_a, q.y}))
      return false;
  }
  return true;
}

}  // namespace

extern "C" {

size_t rpx_int4lora_forward_multi_workspace(int64_t m, int64_t k, int count,
                                            const rpx_int4lora_projection* projections,
                                            int dtype) {
  if (count < 1 || projections == nullptr) return 0;
  // sized from the shapes alone (pointers may be unset at query time): the
  // larger of the fused form and of one projection at a time
  Skinny2Projection fused[4];
  size_t most = 0;
  if (multi_fused_shape(dtype, m, k, count, projections, fused)) {
    Sizer s;
    s.take<float>(skinny2_multi_workspace_floats(m, k, count, fused));
    most = s.used;
  }
  for (int i = 0; i < count; ++i) {
    const size_t b = rpx_int4lora_forward_workspace(m, projections[i].n, k,
                                                    projections[i].group_size,
                                                    projections[i].rank, dtype);
    if (b > most) most = b;
  }
  return most;
}

int rpx_int4lora_forward_multi(const void* x, int dtype, int64_t m, int64_t k, int count,
                               const rpx_int4lora_projection* projections, void* workspace,
                               size_t workspace_bytes, void* stream) {
  if (count < 1 || count > 64 || projections == nullptr)
    return fail_invalid("rpx_int4lora_forward_multi: need 1..64 projections");
  Skinny2Projection fused[4];
  if (multi_fused(x, dtype, m, k, count, projections, fused)) {
    Arena arena(workspace, workspace_bytes);
    float* ws = arena.take<float>(skinny2_multi_workspace_floats(m, k, count, fused));
    if (arena.overflow) return fail_invalid("rpx_int4lora_forward_multi: workspace too small");
    RPX_HIP(launch_skinny2_forward_multi(static_cast<const uint16_t*>(x), m, k, count, fused, ws,
                                         static_cast<hipStream_t>(stream)),
            "rpx_int4lora_forward_multi: skinny-M kernels");
    return kOk;
  }
  ActIO io;
  if (multi_shared_h(x, dtype, m, k, count, projections)) {
    // multi_shared_h admits at most rank_nt_max_blocks() projections (one
    // 16-rank block each at least)
    const uint16_t* r_mats[rank_nt_max_blocks()];
    int64_t ranks[rank_nt_max_blocks()];
    uint16_t* outs[rank_nt_max_blocks()];
    for (int i = 0; i < count; ++i) {
      r_mats[i] = static_cast<const uint16_t*>(projections[i].lora_a);
      ranks[i] = projections[i].rank;
      outs[i] = static_cast<uint16_t*>(projections[i].h);
    }
    RPX_HIP(launch_rank_nt_multi(static_cast<const uint16_t*>(x), k, m, k, count, r_mats, ranks,
                                 outs, static_cast<hipStream_t>(stream)),
            "rpx_int4lora_forward_multi: adapter down-projections");
    io.h_given = true;
  }
  for (int i = 0; i < count; ++i) {
    const rpx_int4lora_projection& q = projections[i];
    RPX_TRY(int4lora_forward_impl(x, dtype, m, k, q.packed, q.scale_bits, q.n, q.group_size,
                                  q.bias_bits, q.lora_a, q.lora_b, q.rank, q.scaling, q.y, q.h,
                                  workspace, workspace_bytes, stream, io));
  }
  return kOk;
}

}  // extern "C"

// --- static scratch for the entry point that allocates nothing ----------------
namespace rpx {
namespace {
// Scratch of rpx_int4lora_forward_static: a file-scope device array, one copy
// per GPU, kept until the process ends. Host code must not pass the array's
// name to a kernel (on the host it is only a stand-in for the symbol); the
// device address of this GPU's copy comes from hipGetSymbolAddress, once per
// device, on the device's first call.
constexpr size_t kStaticScratchBytes = RPX_STATIC_SCRATCH_BYTES;
__device__ __align__(256) uint8_t scratch[kStaticScratchBytes];
std::atomic<void*> g_scratch_ptr[kMaxDevices];

int static_scratch(void** out) {
  int dev = 0;
  RPX_HIP(hipGetDevice(&dev), "static scratch: current device");
  if (dev < 0 || dev >= kMaxDevices) return fail_invalid("static scratch: device index out of range");
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    RPX_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "static scratch: symbol address");
    g_scratch_ptr[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return kOk;
}
}  // namespace
}  // namespace rpx

extern "C" {

int rpx_int4lora_forward_static(const void* x, int dtype, int64_t m, int64_t k,
                                const uint8_t* packed, const uint16_t* scale_bits, int64_t n,
                                int64_t group_size, const uint16_t* bias_bits, const void* lora_a,
                                const void* lora_b, int64_t rank, float scaling, void* y, void* h,
                                void* stream) {
  const size_t need = rpx_int4lora_forward_workspace(m, n, k, group_size, rank, dtype);
  if (need > kStaticScratchBytes)
    return fail_invalid("rpx_int4lora_forward_static: the call needs " + std::to_string(need) +
                        " bytes of scratch, more than the " +
                        std::to_string(kStaticScratchBytes) +
                        " of the static buffer; use rpx_int4lora_forward with a workspace");
  void* ws = nullptr;
  if (m > 0 && n > 0) RPX_TRY(static_scratch(&ws));
  return int4lora_forward_impl(x, dtype, m, k, packed, scale_bits, n, group_size, bias_bits, lora_a,
                               lora_b, rank, scaling, y, h, ws, kStaticScratchBytes, stream,
                               ActIO{});
}

int rpx_int4lora_forward_act(const void* x, int dtype, int64_t m, int64_t k, const uint8_t* packed,
                             const uint16_t* scale_bits, int64_t n, int64_t group_size,
                             const uint16_t* bias_bits, const void* lora_a, const void* lora_b,
                             int64_t rank, float scaling, int act, const void* gate, void* y,
                             void* z, void* h, void* workspace, size_t workspace_bytes,
                             void* stream) {
  if (act != RPX_ACT_GELU && act != RPX_ACT_SILU_MUL)
    return fail_invalid("rpx_int4lora_forward_act: unknown activation");
  if (dtype != kBF16) return fail_invalid("rpx_int4lora_forward_act: activations need bf16 compute");
  if (m > 0 && n > 0 && (z == nullptr || (act == RPX_ACT_SILU_MUL && gate == nullptr)))
    return fail_invalid("rpx_int4lora_forward_act: null pointer");
  ActIO io;
  io.mode = act == RPX_ACT_GELU ? kActGeluFwd : kActSiluMulFwd;
  io.aux = static_cast<const uint16_t*>(gate);
  io.pre_out = static_cast<uint16_t*>(z);
  return int4lora_forward_impl(x, dtype, m, k, packed, scale_bits, n, group_size, bias_bits, lora_a,
                               lora_b, rank, scaling, y, h, workspace, workspace_bytes, stream, io);
}

size_t rpx_int4lora_backward_workspace(int64_t m, int64_t n, int64_t k, int64_t group_size,
                                       int64_t rank, int dtype) {
  int64_t ng = 1, g = k;
  if (group_size > 0 && group_size != k && k % group_size == 0) {
    ng = k / group_size;
    g = group_size;
  }
  Sizer s;
  plan_backward(s, lora_fast_shape(dtype, k, ng, g, rank) && n % 64 == 0, m, n, k, rank, dtype);
  return s.used;
}

namespace {

int int4lora_backward_impl(const void* grad, const void* x, int dtype, int64_t m, int64_t k,
                           const uint8_t* packed, const uint16_t* scale_bits, int64_t n,
                           int64_t group_size, const void* lora_a, const void* lora_b,
                           int64_t rank, float scaling, const void* h, void* dx, float* d_lora_a,
                           float* d_lora_b, void* workspace, size_t workspace_bytes, void* stream,
                           const ActIO& act) {
  RPX_TRY(check_dtype(dtype));
  int64_t ng, g;
  RPX_TRY(check_int4_shape(n, k, group_size, &ng, &g));
  if (m < 0) return fail_invalid("m must be non-negative");
  if (rank < 1 || rank > n || rank > k) return fail_invalid("adapter rank must fit both linear dimensions");
  if (grad == nullptr && m > 0) return fail_invalid("rpx_int4lora_backward: null gradient");
  // an empty batch has no rows to point at: x, dx and h may be null then
  if (packed == nullptr || scale_bits == nullptr || lora_a == nullptr || lora_b == nullptr ||
      d_lora_a == nullptr || d_lora_b == nullptr ||
      (m > 0 && (x == nullptr || dx == nullptr || h == nullptr)))
    return fail_invalid("rpx_int4lora_backward: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (m == 0) {
    RPX_HIP(launch_fill_f32(d_lora_a, rank * k, 0.0f, st), "int4lora_backward: zero dA");
    RPX_HIP(launch_fill_f32(d_lora_b, n * rank, 0.0f, st), "int4lora_backward: zero dB");
    return kOk;
  }
  const float c = round_to_dtype(scaling, dtype);
  const int64_t pc = (k + 1) / 2;
  Int4Operand w;
  w.packed = packed;
  w.packed_cols = pc;
  w.scales = scale_bits;
  w.n_groups = ng;
  w.group = g;
  // the workspace query sizes the MFMA path from the shape alone; it loads
  // every operand in 16-byte vectors
  const bool fast = lora_fast_shape(dtype, k, ng, g, rank) && n % 64 == 0;
  if (fast && !aligned16_all({grad, x, packed, scale_bits, lora_a, lora_b, dx}))
    return fail_invalid(
        "rpx_int4lora_backward: this shape takes the vectorized kernels, which need grad, x, "
        "packed, scale_bits, lora_a, lora_b and dx 16-byte aligned");
  Arena arena(workspace, workspace_bytes);
  if (fast) {
    const uint16_t* gb = static_cast<const uint16_t*>(grad);
    const uint16_t* xb = static_cast<const uint16_t*>(x);
    const uint16_t* ab = static_cast<const uint16_t*>(lora_a);
    const uint16_t* bb = static_cast<const uint16_t*>(lora_b);
    uint16_t* bt = arena.take<uint16_t>(rank * n);
    uint16_t* at = arena.take<uint16_t>(k * rank);
    uint16_t* dh = arena.take<uint16_t>(m * rank);
    uint16_t* wt = arena.take<uint16_t>(k * n);
    float* part_b = arena.take<float>(rank_tn_workspace_floats(m, n, rank));
    float* part_a = arena.take<float>(rank_tn_workspace_floats(m, rank, k));
    if (arena.overflow) return fail_invalid("rpx_int4lora_backward: workspace too small");
    // B^T [r, N] so that dh = g_a . B is an NT product; A^T [K, r] for the
    // dx epilogue's contiguous fragment loads; W_b^T [K, N] for dx unless dx
    // reads the packed weight itself (its own GEMM operand form, on request:
    // the planner keeps W_b^T, which measured faster on every train-step
    // shape)
    const bool dx_packed = tune(kTuneDxPacked) == 1 && int4t_gemm_ok(m, k, n, n, gb, w);
    const bool prep_fused = g % 32 == 0 || dx_packed;
    if (prep_fused) {
      RPX_HIP(launch_int4lora_bwd_prep(bb, bt, ab, at, packed, scale_bits, dx_packed ? nullptr : wt,
                                       n, k, rank, pc, ng, g, st),
              "int4lora_backward: B^T, A^T, W_b^T");
    } else {
      RPX_HIP(launch_transpose_bf16(bb, n, rank, rank, bt, n, st), "int4lora_backward: B^T");
      RPX_HIP(launch_transpose_bf16(ab, rank, k, k, at, rank, st), "int4lora_backward: A^T");
    }
    // dh = bf16(bf16(g * c) . B)
    RPX_HIP(launch_rank_nt(gb, n, bt, n, m, rank, n, true, c, dh, rank, st),
            "int4lora_backward: dh");
    // dB = f32(bf16(g_a^T . h)) and dA = f32(bf16(dh^T . x)), one launch
    RPX_HIP(launch_rank_tn2(gb, n, static_cast<const uint16_t*>(h), rank, m, n, rank, true, c,
                            part_b, d_lora_b, dh, rank, xb, k, m, rank, k, false, 1.0f, part_a,
                            d_lora_a, st),
            "int4lora_backward: dB, dA");
    if (!prep_fused)
      RPX_HIP(launch_int4_dequant_t(packed, scale_bits, wt, n, k, pc, ng, g, n, st),
              "int4lora_backward: dequantized transpose");
    // dx = bf16(bf16(g . W_b) + bf16(dh . A))
    LowRankEpilogue epi;
    epi.rows = at;  // R(k, j) = A[j, k] = A^T[k, j]
    epi.rows_sn = rank;
    epi.rows_sj = 1;
    epi.cols = dh;
    epi.cols_sm = rank;
    epi.cols_sj = 1;
    epi.rank = rank;
    epi.scale = 1.0f;
    epi.act = act.mode;
    epi.aux = act.aux;
    epi.aux2 = act.aux2;
    epi.out2 = act.out2;
    if (dx_packed)
      RPX_HIP(launch_gemm_int4t(gb, n, w, m, k, n, static_cast<uint16_t*>(dx), k, epi, st),
              "int4lora_backward: dx from the packed weight");
    else
      RPX_HIP(launch_gemm_bf16(gb, n, wt, n, m, k, n, static_cast<uint16_t*>(dx), k, epi, st),
              "int4lora_backward: dx");
    return kOk;
  }
  const size_t es = elem_size(dtype);
  void* ga = arena.take<uint8_t>(m * n * static_cast<int64_t>(es));
  void* dh = arena.take<uint8_t>(m * rank * static_cast<int64_t>(es));
  float* dhf = arena.take<float>(m * rank);
  float* p1 = arena.take<float>(m * k);
  float* p2 = arena.take<float>(m * k);
  if (arena.overflow) return fail_invalid("rpx_int4lora_backward: workspace too small");
  hipLaunchKernelGGL(k_scale_round, dim3(grid1d(m * n)), dim3(256), 0, st, grad, m * n, c, dtype,
                     ga);
  RPX_HIP(hipGetLastError(), "int4lora_backward: g_a");
  // dh[m, j] = sum_n g_a[m, n] B[n, j]
  RPX_HIP(launch_generic_gemm(ga, dtype, n, 1, lora_b, dtype, 1, rank, nullptr, false, m, rank, n,
                              dhf, st),
          "int4lora_backward: dh");
  RPX_HIP(launch_round_store(dhf, m * rank, dtype, dh, st), "int4lora_backward: round dh");
  // dB[n, j] = sum_m g_a[m, n] h[m, j]
  RPX_HIP(launch_generic_gemm(ga, dtype, 1, n, h, dtype, 1, rank, nullptr, false, n, rank, m,
                              d_lora_b, st),
          "int4lora_backward: dB");
  hipLaunchKernelGGL(k_round_inplace_f32, dim3(grid1d(n * rank)), dim3(256), 0, st, d_lora_b,
                     n * rank, dtype);
  RPX_HIP(hipGetLastError(), "int4lora_backward: round dB");
  // g . W_b : B(k, n) = W_b[n, k]
  RPX_HIP(launch_generic_gemm(grad, dtype, n, 1, nullptr, dtype, 0, 0, &w, true, m, k, n, p1, st),
          "int4lora_backward: g W");
  // dh . A : B(k, j) = A[j, k]
  RPX_HIP(launch_generic_gemm(dh, dtype, rank, 1, lora_a, dtype, 1, k, nullptr, false, m, k, rank,
                              p2, st),
          "int4lora_backward: dh A");
  hipLaunchKernelGGL(k_lora_combine, dim3(grid1d(m * k)), dim3(256), 0, st, p1, p2, m, k, 1.0f,
                     nullptr, dtype, dx);
  RPX_HIP(hipGetLastError(), "int4lora_backward: combine dx");
  // dA[j, k] = sum_m dh[m, j] x[m, k]
  RPX_HIP(launch_generic_gemm(dh, dtype, 1, rank, x, dtype, 1, k, nullptr, false, rank, k, m,
                              d_lora_a, st),
          "int4lora_backward: dA");
  hipLaunchKernelGGL(k_round_inplace_f32, dim3(grid1d(rank * k)), dim3(256), 0, st, d_lora_a,
                     rank * k, dtype);
  RPX_HIP(hipGetLastError(), "int4lora_backward: round dA");
  if (act.mode != kActNone)
    RPX_HIP(launch_act(act.mode, static_cast<const uint16_t*>(dx), act.aux, act.aux2, m * k,
                       static_cast<uint16_t*>(dx), act.out2, st),
            "int4lora_backward: activation");
  return kOk;
}

}  // namespace

int rpx_int4lora_backward(const void* grad, const void* x, int dtype, int64_t m, int64_t k,
                          const uint8_t* packed, const uint16_t* scale_bits, int64_t n,
                          int64_t group_size, const void* lora_a, const void* lora_b,
                          int64_t rank, float scaling, const void* h, void* dx, float* d_lora_a,
                          float* d_lora_b, void* workspace, size_t workspace_bytes,
                          void* stream) {
  return int4lora_backward_impl(grad, x, dtype, m, k, packed, scale_bits, n, group_size, lora_a,
                                lora_b, rank, scaling, h, dx, d_lora_a, d_lora_b, workspace,
                                workspace_bytes, stream, ActIO{});
}

int rpx_int4lora_backward_act(const void* grad, const void* x, int dtype, int64_t m, int64_t k,
                              const uint8_t* packed, const uint16_t* scale_bits, int64_t n,
                              int64_t group_size, const void* lora_a, const void* lora_b,
                              int64_t rank, float scaling, const void* h, int act, const void* z,
                              const void* gate, void* dz, void* dgate, float* d_lora_a,
                              float* d_lora_b, void* workspace, size_t workspace_bytes,
                              void* stream) {
  if (act != RPX_ACT_GELU && act != RPX_ACT_SILU_MUL && act != RPX_ACT_ADD)
    return fail_invalid("rpx_int4lora_backward_act: unknown activation");
  if (act == RPX_ACT_ADD && z == dz && z != nullptr)
    return fail_invalid("rpx_int4lora_backward_act: dz must not alias z");
  if (dtype != kBF16) return fail_invalid("rpx_int4lora_backward_act: activations need bf16 compute");
  if (m > 0 && (z == nullptr || (act == RPX_ACT_SILU_MUL && (gate == nullptr || dgate == nullptr))))
    return fail_invalid("rpx_int4lora_backward_act: null pointer");
  ActIO io;
  if (act == RPX_ACT_GELU || act == RPX_ACT_ADD) {
    io.mode = act == RPX_ACT_GELU ? kActGeluBwd : kActAddBwd;
    io.aux = static_cast<const uint16_t*>(z);
  } else {
    io.mode = kActSiluMulBwd;
    io.aux = static_cast<const uint16_t*>(gate);
    io.aux2 = static_cast<const uint16_t*>(z);
    io.out2 = static_cast<uint16_t*>(dgate);
  }
  return int4lora_backward_impl(grad, x, dtype, m, k, packed, scale_bits, n, group_size, lora_a,
                                lora_b, rank, scaling, h, dz, d_lora_a, d_lora_b, workspace,
                                workspace_bytes, stream, io);
}

// ---------------------------------------------------------------------------
// INT4 + LoRA linear without a precision policy: bf16 activations, float32
// adapter masters (jnp.matmul promotes the adapter products to float32)
// ---------------------------------------------------------------------------
}  // extern "C"

namespace rpx {
namespace {

// y = f32(base_b) + low * c (+ f32(bias)): base_b the bf16-rounded base
// product (bf16 bits when base_bf16, else f32 values rounded here).
__global__ void __launch_bounds__(256)
    k_promoted_combine(const void* __restrict__ base, int base_bf16,
                       const float* __restrict__ low, int64_t rows, int64_t cols, float c,
                       const uint16_t* __restrict__ bias, float* __restrict__ out) {
  const int64_t total = rows * cols;
  for (int64_t e = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; e < total;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const float b = base_bf16 ? bf16_to_f32(static_cast<const uint16_t*>(base)[e])
                              : round_bf16(static_cast<const float*>(base)[e]);
    float y = b + low[e] * c;
    if (bias != nullptr) y = y + bf16_to_f32(bias[e % cols]);
    out[e] = y;
  }
}

bool promoted_fast_base(int64_t k, int64_t n_groups, int64_t group, const void* x,
                        const void* packed, const void* scales) {
  return lora_fast_shape(kBF16, k, n_groups, group, 1) && aligned16_all({x, packed, scales});
}

template <typename A>
void plan_forward_promoted(A& a, int64_t m, int64_t n) {
  a.template take<float>(m * n);  // base product (f32, or bf16 bits from the MFMA GEMM)
  a.template take<float>(m * n);  // adapter product
}

template <typename A>
void plan_backward_promoted(A& a, int64_t m, int64_t n, int64_t k, int64_t rank) {
  a.template take<uint16_t>(m * n);  // bf16(g)
  a.template take<float>(m * n);     // g * c
  a.template take<float>(m * rank);  // dh
  a.template take<float>(m * k);     // bf16(g) W_b
  a.template take<float>(m * k);     // dh A
}

}  // namespace
}  // namespace rpx

extern "C" {

size_t rpx_int4lora_forward_promoted_workspace(int64_t m, int64_t n, int64_t k,
                                               int64_t group_size, int64_t rank) {
  (void)k;
  (void)group_size;
  (void)rank;
  Sizer s;
  plan_forward_promoted(s, m, n);
  return s.used;
}

int rpx_int4lora_forward_promoted(const uint16_t* x, int64_t m, int64_t k, const uint8_t* packed,
                                  const uint16_t* scale_bits, int64_t n, int64_t group_size,
                                  const uint16_t* bias_bits, const float* lora_a,
                                  const float* lora_b, int64_t rank, float scaling, float* y,
                                  float* h, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  int64_t ng, g;
  RPX_TRY(check_int4_shape(n, k, group_size, &ng, &g));
  if (m < 0) return fail_invalid("m must be non-negative");
  if (rank < 1 || rank > n || rank > k) return fail_invalid("adapter rank must fit both linear dimensions");
  if (m == 0 || n == 0) return kOk;
  if (x == nullptr || packed == nullptr || scale_bits == nullptr || lora_a == nullptr ||
      lora_b == nullptr || y == nullptr || h == nullptr)
    return fail_invalid("rpx_int4lora_forward_promoted: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  Int4Operand w;
  w.packed = packed;
  w.packed_cols = (k + 1) / 2;
  w.scales = scale_bits;
  w.n_groups = ng;
  w.group = g;
  Arena arena(workspace, workspace_bytes);
  float* base = arena.take<float>(m * n);
  float* low = arena.take<float>(m * n);
  if (arena.overflow) return fail_invalid("rpx_int4lora_forward_promoted: workspace too small");
  // base = bf16(x W_b^T): the MFMA GEMM with no epilogue term where it applies
  const bool fast = promoted_fast_base(k, ng, g, x, packed, scale_bits);
  if (fast) {
    RPX_HIP(launch_gemm_int4(x, k, w, m, n, k, reinterpret_cast<uint16_t*>(base), n,
                             LowRankEpilogue{}, st),
            "int4lora_forward_promoted: base product");
  } else {
    RPX_HIP(launch_generic_gemm(x, kBF16, k, 1, nullptr, kBF16, 0, 0, &w, false, m, n, k, base,
                                st),
            "int4lora_forward_promoted: base product");
  }
  // h = f32(x A^T), a = f32(h B^T), on the float32 masters
  RPX_HIP(launch_generic_gemm(x, kBF16, k, 1, lora_a, kF32, k, 1, nullptr, false, m, rank, k, h,
                              st),
          "int4lora_forward_promoted: adapter down-projection");
  RPX_HIP(launch_generic_gemm(h, kF32, rank, 1, lora_b, kF32, rank, 1, nullptr, false, m, n, rank,
                              low, st),
          "int4lora_forward_promoted: adapter up-projection");
  hipLaunchKernelGGL(k_promoted_combine, dim3(grid1d(m * n)), dim3(256), 0, st, base,
                     fast ? 1 : 0, low, m, n, scaling, bias_bits, y);
  RPX_HIP(hipGetLastError(), "int4lora_forward_promoted: combine");
  return kOk;
}

size_t rpx_int4lora_backward_promoted_workspace(int64_t m, int64_t n, int64_t k,
                                                int64_t group_size, int64_t rank) {
  (void)group_size;
  Sizer s;
  plan_backward_promoted(s, m, n, k, rank);
  return s.used;
}

int rpx_int4lora_backward_promoted(const float* grad, const uint16_t* x, int64_t m, int64_t k,
                                   const uint8_t* packed, const uint16_t* scale_bits, int64_t n,
                                   int64_t group_size, const float* lora_a, const float* lora_b,
                                   int64_t rank, float scaling, const float* h, uint16_t* dx,
                                   float* d_lora_a, float* d_lora_b, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  int64_t ng, g;
  RPX_TRY(check_int4_shape(n, k, group_size, &ng, &g));
  if (m < 0) return fail_invalid("m must be non-negative");
  if (rank < 1 || rank > n || rank > k) return fail_invalid("adapter rank must fit both linear dimensions");
  if (packed == nullptr || scale_bits == nullptr || lora_a == nullptr || lora_b == nullptr ||
      d_lora_a == nullptr || d_lora_b == nullptr ||
      (m > 0 && (grad == nullptr || x == nullptr || dx == nullptr || h == nullptr)))
    return fail_invalid("rpx_int4lora_backward_promoted: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (m == 0) {
    RPX_HIP(launch_fill_f32(d_lora_a, rank * k, 0.0f, st), "int4lora_backward_promoted: zero dA");
    RPX_HIP(launch_fill_f32(d_lora_b, n * rank, 0.0f, st), "int4lora_backward_promoted: zero dB");
    return kOk;
  }
  Int4Operand w;
  w.packed = packed;
  w.packed_cols = (k + 1) / 2;
  w.scales = scale_bits;
  w.n_groups = ng;
  w.group = g;
  Arena arena(workspace, workspace_bytes);
  uint16_t* gb = arena.take<uint16_t>(m * n);
  float* ga = arena.take<float>(m * n);
  float* dh = arena.take<float>(m * rank);
  float* p1 = arena.take<float>(m * k);
  float* p2 = arena.take<float>(m * k);
  if (arena.overflow) return fail_invalid("rpx_int4lora_backward_promoted: workspace too small");
  // the base product's cotangent is bf16(g); dx_base = bf16(bf16(g) W_b)
  RPX_HIP(launch_round_store(grad, m * n, kBF16, gb, st), "int4lora_backward_promoted: bf16(g)");
  RPX_HIP(launch_generic_gemm(gb, kBF16, n, 1, nullptr, kBF16, 0, 0, &w, true, m, k, n, p1, st),
          "int4lora_backward_promoted: g W");
  // g_a = f32(g c), dh = f32(g_a B), dB = f32(g_a^T h)
  hipLaunchKernelGGL(k_scale_round, dim3(grid1d(m * n)), dim3(256), 0, st, grad, m * n, scaling,
                     kF32, ga);
  RPX_HIP(hipGetLastError(), "int4lora_backward_promoted: g_a");
  RPX_HIP(launch_generic_gemm(ga, kF32, n, 1, lora_b, kF32, 1, rank, nullptr, false, m, rank, n,
                              dh, st),
          "int4lora_backward_promoted: dh");
  RPX_HIP(launch_generic_gemm(ga, kF32, 1, n, h, kF32, 1, rank, nullptr, false, n, rank, m,
                              d_lora_b, st),
          "int4lora_backward_promoted: dB");
  // dx = bf16(bf16(g W_b) + bf16(f32(dh A))), summed in bf16
  RPX_HIP(launch_generic_gemm(dh, kF32, rank, 1, lora_a, kF32, 1, k, nullptr, false, m, k, rank,
                              p2, st),
          "int4lora_backward_promoted: dh A");
  hipLaunchKernelGGL(k_lora_combine, dim3(grid1d(m * k)), dim3(256), 0, st, p1, p2, m, k, 1.0f,
                     nullptr, kBF16, dx);
  RPX_HIP(hipGetLastError(), "int4lora_backward_promoted: combine dx");
  // dA = f32(dh^T x)
  RPX_HIP(launch_generic_gemm(dh, kF32, 1, rank, x, kBF16, 1, k, nullptr, false, rank, k, m,
                              d_lora_a, st),
          "int4lora_backward_promoted: dA");
  return kOk;
}

// ---------------------------------------------------------------------------
// FP8
// ---------------------------------------------------------------------------
size_t rpx_fp8_scale_workspace(int64_t numel) {
  return static_cast<size_t>(fp8_amax_partials(numel)) * sizeof(uint32_t);
}

int rpx_fp8_scale(const void* t, int dtype, int64_t numel, int fmt, float* scale_out,
                  void* workspace, size_t workspace_bytes, void* stream) {
  RPX_TRY(check_dtype(dtype));
  RPX_TRY(check_fmt(fmt));
  if (numel < 0) return fail_invalid("numel must be non-negative");
  if (scale_out == nullptr || (numel > 0 && t == nullptr)) return fail_invalid("rpx_fp8_scale: null pointer");
  const int64_t np = fp8_amax_partials(numel);
  if (workspace == nullptr || workspace_bytes < static_cast<size_t>(np) * sizeof(uint32_t))
    return fail_invalid("rpx_fp8_scale: workspace too small");
  RPX_HIP(launch_fp8_amax(t, dtype, numel, static_cast<uint32_t*>(workspace), np, fmt, scale_out,
                          static_cast<hipStream_t>(stream)),
          "rpx_fp8_scale");
  return kOk;
}

int rpx_fp8_cast(const void* t, int dtype, int64_t rows, int64_t cols, int64_t row_stride,
                 int64_t col_stride, const float* scale, int fmt, uint8_t* out, uint8_t* out_t,
                 void* stream) {
  RPX_TRY(check_dtype(dtype));
  RPX_TRY(check_fmt(fmt));
  if (rows < 0 || cols < 0) return fail_invalid("rows and cols must be non-negative");
  if (scale == nullptr || (rows * cols > 0 && t == nullptr)) return fail_invalid("rpx_fp8_cast: null pointer");
  if (out == nullptr && out_t == nullptr) return fail_invalid("rpx_fp8_cast: no output requested");
  RPX_HIP(launch_fp8_cast(t, dtype, rows, cols, row_stride, col_stride, scale, nullptr, 0, nullptr,
                          fmt, out, out_t, static_cast<hipStream_t>(stream)),
          "rpx_fp8_cast");
  return kOk;
}

size_t rpx_fp8_gemm_workspace(int64_t m, int64_t n, int64_t k) {
  if (k % 128 != 0) return static_cast<size_t>(m * n) * sizeof(float);
  return static_cast<size_t>(fp8_gemm_workspace_floats(m, n, k)) * sizeof(float);
}

}  // extern "C"

namespace rpx {
namespace {
// OCP fp8 decode tables (e4m3fn, e5m2), built at compile time.
constexpr float pow2_constexpr(int e) {
  float v = 1.0f;
  for (; e > 0; --e) v *= 2.0f;
  for (; e < 0; ++e) v *= 0.5f;
  return v;
}

constexpr float decode_fp8_constexpr(uint32_t code, int fmt) {
  const int eb = fmt == kE4M3FN ? 4 : 5;
  const int mb = fmt == kE4M3FN ? 3 : 2;
  const int bias = fmt == kE4M3FN ? 7 : 15;
  const float sign = (code & 0x80u) ? -1.0f : 1.0f;
  const uint32_t e = (code >> mb) & ((1u << eb) - 1u);
  const uint32_t mnt = code & ((1u << mb) - 1u);
  const uint32_t all = (1u << eb) - 1u;
  if (fmt == kE5M2 && e == all) return mnt == 0 ? sign * __builtin_inff() : __builtin_nanf("");
  if (fmt == kE4M3FN && e == all && mnt == (1u << mb) - 1u) return __builtin_nanf("");
  if (e == 0) return sign * static_cast<float>(mnt) * pow2_constexpr(1 - bias - mb);
  return sign * (1.0f + static_cast<float>(mnt) / static_cast<float>(1u << mb)) *
         pow2_constexpr(static_cast<int>(e) - bias);
}

struct Fp8Table {
  float v[2][256];
};

constexpr Fp8Table make_fp8_table() {
  Fp8Table t{};
  for (int f = 0; f < 2; ++f)
    for (int c = 0; c < 256; ++c) t.v[f][c] = decode_fp8_constexpr(static_cast<uint32_t>(c), f);
  return t;
}

__constant__ Fp8Table c_fp8_table = make_fp8_table();

// a(m, kk) = a[m * a_sm + kk * a_sk], b(n, kk) = b[n * b_sn + kk * b_sk]:
// row-major [M, K] / [N, K] codes, or K-row [K, M] / [K, N] ones.
__global__ void __launch_bounds__(256)
    k_fp8_gemm_generic(const uint8_t* __restrict__ a, int fmt_a, const uint8_t* __restrict__ b,
                       int fmt_b, int64_t M, int64_t N, int64_t K, int64_t a_sm, int64_t a_sk,
                       int64_t b_sn, int64_t b_sk, const float* __restrict__ s_a,
                       const float* __restrict__ s_b, void* __restrict__ out, int out_dtype) {
  const int64_t total = M * N;
  for (int64_t e = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; e < total;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t m = e / N;
    const int64_t n = e % N;
    float acc = 0.0f;
    for (int64_t kk = 0; kk < K; ++kk)
      acc = __builtin_fmaf(c_fp8_table.v[fmt_a][a[m * a_sm + kk * a_sk]],
                           c_fp8_table.v[fmt_b][b[n * b_sn + kk * b_sk]], acc);
    const float y = (acc * s_a[0]) * s_b[0];
    if (out_dtype == kBF16)
      static_cast<uint16_t*>(out)[e] = f32_to_bf16(y);
    else
      static_cast<float*>(out)[e] = y;
  }
}

}  // namespace
}  // namespace rpx

extern "C" {

int rpx_fp8_gemm(const uint8_t* a, int fmt_a, const float* scale_a, const uint8_t* b, int fmt_b,
                 const float* scale_b, int64_t m, int64_t n, int64_t k, void* out, int out_dtype,
                 void* workspace, size_t workspace_bytes, void* stream) {
  RPX_TRY(check_fmt(fmt_a));
  RPX_TRY(check_fmt(fmt_b));
  RPX_TRY(check_dtype(out_dtype));
  if (m < 0 || n < 0 || k < 0) return fail_invalid("m, n, k must be non-negative");
  if (m == 0 || n == 0) return kOk;
  if (a == nullptr || b == nullptr || scale_a == nullptr || scale_b == nullptr || out == nullptr)
    return fail_invalid("rpx_fp8_gemm: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool fast = k > 0 && k % 128 == 0 && aligned16(a) && aligned16(b);
  if (fast) {
    const int64_t need = fp8_gemm_workspace_floats(m, n, k);
    if (static_cast<size_t>(need) * sizeof(float) > workspace_bytes || (need > 0 && workspace == nullptr))
      return fail_invalid("rpx_fp8_gemm: workspace too small");
    RPX_HIP(launch_fp8_gemm(a, fmt_a, scale_a, b, fmt_b, scale_b, m, n, k, out, out_dtype, n,
                            static_cast<float*>(workspace), need, st),
            "rpx_fp8_gemm");
    return kOk;
  }
  hipLaunchKernelGGL(k_fp8_gemm_generic, dim3(grid1d(m * n)), dim3(256), 0, st, a, fmt_a, b, fmt_b,
                     m, n, k, k, int64_t{1}, k, int64_t{1}, scale_a, scale_b, out, out_dtype);
  RPX_HIP(hipGetLastError(), "rpx_fp8_gemm (generic)");
  return kOk;
}

}  // extern "C"

namespace {
// out [m, n] = ((a^T . b) * s_a) * s_b from K-row codes a [k, m] and b [k, n]:
// the pipelined K-row GEMM where the shapes and alignment allow it, else the
// generic kernel. Workspace: fp8_krows_bytes(m, n, k).
size_t fp8_krows_bytes(int64_t m, int64_t n, int64_t k) {
  if (k % 128 != 0 || m % 16 != 0 || n % 16 != 0) return 0;
  return static_cast<size_t>(fp8_gemm_krows_workspace_floats(m, n, k)) * sizeof(float);
}

int fp8_gemm_krows(const uint8_t* a, int fmt_a, const float* s_a, const uint8_t* b, int fmt_b,
                   const float* s_b, int64_t m, int64_t n, int64_t k, void* out, int out_dtype,
                   void* workspace, size_t workspace_bytes, hipStream_t st) {
  if (k % 128 == 0 && m % 16 == 0 && n % 16 == 0 && aligned16(a) && aligned16(b)) {
    const size_t need = fp8_krows_bytes(m, n, k);
    if (need > workspace_bytes || (need > 0 && workspace == nullptr))
      return fail_invalid("fp8 K-row GEMM: workspace too small");
    RPX_HIP(launch_fp8_gemm_krows(a, fmt_a, s_a, b, fmt_b, s_b, m, n, k, out, out_dtype, n,
                                  static_cast<float*>(workspace),
                                  static_cast<int64_t>(need / sizeof(float)), st),
            "fp8 K-row GEMM");
    return kOk;
  }
  hipLaunchKernelGGL(k_fp8_gemm_generic, dim3(grid1d(m * n)), dim3(256), 0, st, a, fmt_a, b, fmt_b,
                     m, n, k, int64_t{1}, m, int64_t{1}, n, s_a, s_b, out, out_dtype);
  RPX_HIP(hipGetLastError(), "fp8 K-row GEMM (generic)");
  return kOk;
}

template <typename A>
void plan_fp8_forward(A& a, int64_t m, int64_t n, int64_t k) {
  a.template take<uint32_t>(fp8_quant_partials(m, k));
  a.template take<uint32_t>(fp8_quant_partials(k, n));
  a.template take<uint8_t>(m * k);
  a.template take<uint8_t>(n * k);
  a.template take<uint8_t>(rpx_fp8_gemm_workspace(m, n, k));
}
template <typename A>
void plan_fp8_backward(A& a, int64_t m, int64_t n, int64_t k) {
  a.template take<uint32_t>(fp8_quant_partials(m, n));
  a.template take<float>(1);
  a.template take<uint8_t>(m * n);  // g codes [M, N]
  a.template take<uint8_t>(k * n);  // right codes [K, N]
  a.template take<uint8_t>(m * k);  // left codes [M, K]
  a.template take<uint8_t>(static_cast<int64_t>(rpx_fp8_linear_backward_gemms_workspace(m, n, k)));
}
}  // namespace

extern "C" {

size_t rpx_fp8_linear_forward_workspace(int64_t m, int64_t n, int64_t k) {
  Sizer s;
  plan_fp8_forward(s, m, n, k);
  return s.used;
}

int rpx_fp8_linear_forward(const void* left, int left_dtype, int64_t m, int64_t k,
                           const void* right, int right_dtype, int64_t n, int64_t right_row_stride,
                           int64_t right_col_stride, void* out, int out_dtype, float* scales_out,
                           uint8_t* left_codes, uint8_t* right_codes, void* workspace,
                           size_t workspace_bytes, void* stream) {
  RPX_TRY(check_dtype(left_dtype));
  RPX_TRY(check_dtype(right_dtype));
  RPX_TRY(check_dtype(out_dtype));
  if (m < 0 || n < 0 || k < 0) return fail_invalid("m, n, k must be non-negative");
  if (scales_out == nullptr) return fail_invalid("rpx_fp8_linear_forward: null scales_out");
  // the dynamic scale of an empty operand is undefined: the reference's
  // amax (a max reduction with no identity) raises on it too
  if (m == 0 || n == 0 || k == 0)
    return fail_invalid("rpx_fp8_linear_forward: empty operand (no amax to scale by)");
  if (left == nullptr || right == nullptr || out == nullptr)
    return fail_invalid("rpx_fp8_linear_forward: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  Arena ar(workspace, workspace_bytes);
  uint32_t* pl = ar.take<uint32_t>(fp8_quant_partials(m, k));
  uint32_t* pr = ar.take<uint32_t>(fp8_quant_partials(k, n));
  uint8_t* ql_ws = ar.take<uint8_t>(m * k);
  uint8_t* qr = ar.take<uint8_t>(n * k);
  const size_t gws = rpx_fp8_gemm_workspace(m, n, k);
  uint8_t* gw = ar.take<uint8_t>(static_cast<int64_t>(gws));
  if (ar.overflow) return fail_invalid("rpx_fp8_linear_forward: workspace too small");
  // both tensors' amaxes in one launch, then both casts in one launch:
  // left [M, K] -> codes [M, K] (this product's, and the weight gradient's
  // K-row operand); right [K, N] -> codes [N, K] for this product (+ [K, N]
  // for the input gradient)
  uint8_t* ql = left_codes != nullptr ? left_codes : ql_ws;
  RPX_HIP(launch_fp8_quantize2(left, left_dtype, m, k, k, 1, pl, scales_out, ql, nullptr, right,
                               right_dtype, k, n, right_row_stride, right_col_stride, pr,
                               scales_out + 1, right_codes, qr, kE4M3FN, st),
          "fp8_linear_forward: quantize");
  return rpx_fp8_gemm(ql, kE4M3FN, scales_out, qr, kE4M3FN, scales_out + 1, m, n, k, out,
                      out_dtype, gw, gws, stream);
}

size_t rpx_fp8_linear_backward_workspace(int64_t m, int64_t n, int64_t k) {
  Sizer s;
  plan_fp8_backward(s, m, n, k);
  return s.used;
}

int rpx_fp8_linear_backward_codes(const uint8_t* left_codes, const uint8_t* right_codes,
                                  const float* scales, int64_t m, int64_t k, int64_t n,
                                  const void* grad, int grad_dtype, void* d_left, void* d_right,
                                  int d_right_transposed, int out_dtype, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  RPX_TRY(check_dtype(grad_dtype));
  RPX_TRY(check_dtype(out_dtype));
  if (m <= 0 || n <= 0 || k <= 0)
    return fail_invalid("rpx_fp8_linear_backward: m, n, k must be positive");
  if (grad == nullptr || scales == nullptr || (d_left != nullptr && right_codes == nullptr) ||
      (d_right != nullptr && left_codes == nullptr))
    return fail_invalid("rpx_fp8_linear_backward: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  Arena ar(workspace, workspace_bytes);
  uint32_t* pg = ar.take<uint32_t>(fp8_quant_partials(m, n));
  float* sg = ar.take<float>(1);
  uint8_t* qg = ar.take<uint8_t>(m * n);
  ar.take<uint8_t>(k * n);
  ar.take<uint8_t>(m * k);
  const size_t gws = rpx_fp8_linear_backward_gemms_workspace(m, n, k);
  uint8_t* gw = ar.take<uint8_t>(static_cast<int64_t>(gws));
  if (ar.overflow) return fail_invalid("rpx_fp8_linear_backward: workspace too small");
  // s_g (e5m2) and the gradient's codes [M, N], the operand of both products
  RPX_HIP(launch_fp8_quantize2(grad, grad_dtype, m, n, n, 1, pg, sg, qg, nullptr, nullptr,
                               grad_dtype, 0, 0, 0, 1, nullptr, nullptr, nullptr, nullptr, kE5M2,
                               st),
          "fp8_linear_backward: quantize(grad)");
  return rpx_fp8_linear_backward_gemms(qg, sg, left_codes, scales, right_codes, scales + 1, m, k,
                                       n, d_left, d_right, d_right_transposed, out_dtype, gw, gws,
                                       stream);
}

size_t rpx_fp8_linear_backward_gemms_workspace(int64_t m, int64_t n, int64_t k) {
  size_t g1 = rpx_fp8_gemm_workspace(m, k, n);
  size_t g2 = fp8_krows_bytes(k, n, m);
  const size_t g3 = fp8_krows_bytes(n, k, m);
  if (g2 < g3) g2 = g3;
  return g1 > g2 ? g1 : g2;
}

int rpx_fp8_linear_backward_gemms(const uint8_t* g_codes, const float* s_grad,
                                  const uint8_t* left_codes, const float* s_left,
                                  const uint8_t* right_codes, const float* s_right, int64_t m,
                                  int64_t k, int64_t n, void* d_left, void* d_right,
                                  int d_right_transposed, int out_dtype, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  RPX_TRY(check_dtype(out_dtype));
  if (m <= 0 || n <= 0 || k <= 0)
    return fail_invalid("rpx_fp8_linear_backward_gemms: m, n, k must be positive");
  if (g_codes == nullptr || s_grad == nullptr ||
      (d_left != nullptr && (right_codes == nullptr || s_right == nullptr)) ||
      (d_right != nullptr && (left_codes == nullptr || s_left == nullptr)))
    return fail_invalid("rpx_fp8_linear_backward_gemms: null pointer");
  const size_t gws = rpx_fp8_linear_backward_gemms_workspace(m, n, k);
  if (workspace_bytes < gws || (gws > 0 && workspace == nullptr))
    return fail_invalid("rpx_fp8_linear_backward_gemms: workspace too small");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (d_left != nullptr && d_right != nullptr && d_right_transposed &&
      aligned16_all({g_codes, right_codes, left_codes})) {
    // both products in one launch where their plans allow it
    bool paired = false;
    RPX_HIP(launch_fp8_backward_pair(g_codes, right_codes, left_codes, s_grad, s_right, s_left, m,
                                     k, n, d_left, d_right, out_dtype,
                                     static_cast<float*>(workspace),
                                     static_cast<int64_t>(gws / sizeof(float)), st, &paired),
            "fp8_linear_backward: paired products");
    if (paired) return kOk;
  }
  // d_left [M, K] = ((g . right^T) * s_g) * s_r
  if (d_left != nullptr)
    RPX_TRY(rpx_fp8_gemm(g_codes, kE5M2, s_grad, right_codes, kE4M3FN, s_right, m, k, n, d_left,
                         out_dtype, workspace, gws, stream));
  if (d_right == nullptr) return kOk;
  // d_right = ((left^T . g) * s_l) * s_g over the tokens, from the K-row
  // (tokens-major) codes of both operands, as [K, N] or transposed [N, K]
  if (d_right_transposed)
    return fp8_gemm_krows(g_codes, kE5M2, s_left, left_codes, kE4M3FN, s_grad, n, k, m, d_right,
                          out_dtype, workspace, gws, st);
  return fp8_gemm_krows(left_codes, kE4M3FN, s_left, g_codes, kE5M2, s_grad, k, n, m, d_right,
                        out_dtype, workspace, gws, st);
}

int rpx_fp8_linear_backward(const void* left, int left_dtype, const void* right, int right_dtype,
                            int64_t m, int64_t k, int64_t n, int64_t right_row_stride,
                            int64_t right_col_stride, const void* grad, int grad_dtype,
                            const float* scales, void* d_left, void* d_right,
                            int d_right_transposed, int out_dtype, void* workspace,
                            size_t workspace_bytes, void* stream) {
  RPX_TRY(check_dtype(left_dtype));
  RPX_TRY(check_dtype(right_dtype));
  if (left == nullptr || right == nullptr || grad == nullptr || scales == nullptr)
    return fail_invalid("rpx_fp8_linear_backward: null pointer");
  if (m <= 0 || n <= 0 || k <= 0)
    return fail_invalid("rpx_fp8_linear_backward: m, n, k must be positive");
  hipStream_t st = static_cast<hipStream_t>(stream);
  // re-quantize the operands with the forward scales (same values, same
  // amax), into the tail of the workspace that the code path reserves
  Arena ar(workspace, workspace_bytes);
  ar.take<uint32_t>(fp8_quant_partials(m, n));
  ar.take<float>(1);
  ar.take<uint8_t>(m * n);
  uint8_t* qr = ar.take<uint8_t>(k * n);
  uint8_t* ql = ar.take<uint8_t>(m * k);
  if (ar.overflow) return fail_invalid("rpx_fp8_linear_backward: workspace too small");
  if (d_left != nullptr)
    RPX_HIP(launch_fp8_cast(right, right_dtype, k, n, right_row_stride, right_col_stride,
                            scales + 1, nullptr, 0, nullptr, kE4M3FN, qr, nullptr, st),
            "fp8_linear_backward: cast(right)");
  if (d_right != nullptr)
    RPX_HIP(launch_fp8_cast(left, left_dtype, m, k, k, 1, scales, nullptr, 0, nullptr, kE4M3FN,
                            ql, nullptr, st),
            "fp8_linear_backward: cast(left)");
  return rpx_fp8_linear_backward_codes(ql, qr, scales, m, k, n, grad, grad_dtype, d_left, d_right,
                                       d_right_transposed, out_dtype, workspace, workspace_bytes,
                                       stream);
}

size_t rpx_fp8_delayed_pending_words(void) { return static_cast<size_t>(fp8_rec_words()); }

namespace {
int delayed_args(const char* who, int64_t rows, int64_t cols, int64_t n_slots, int64_t slot,
                 const void* t, const uint8_t* out, const uint8_t* out_t) {
  if (rows < 0 || cols < 0) return fail_invalid(std::string(who) + ": negative shape");
  if (n_slots < 1 || slot < 0 || slot >= n_slots)
    return fail_invalid(std::string(who) + ": slot outside the scale state");
  if (rows > 0 && cols > 0 && (t == nullptr || (out == nullptr && out_t == nullptr)))
    return fail_invalid(std::string(who) + ": null pointer");
  return kOk;
}
}  // namespace

int rpx_fp8_cast_delayed(const void* t, int dtype, int64_t rows, int64_t cols, int64_t row_stride,
                         int64_t col_stride, int fmt, const float* scales,
                         uint32_t* amax_pending, int64_t n_slots, int64_t slot, uint8_t* out,
                         uint8_t* out_t, void* stream) {
  RPX_TRY(check_dtype(dtype));
  RPX_TRY(check_fmt(fmt));
  if (scales == nullptr || amax_pending == nullptr)
    return fail_invalid("rpx_fp8_cast_delayed: null scale state");
  RPX_TRY(delayed_args("rpx_fp8_cast_delayed", rows, cols, n_slots, slot, t, out, out_t));
  const DelayedCast c{t, dtype, rows, cols, row_stride, col_stride, scales + slot,
                      amax_pending + slot * fp8_rec_words(), out, out_t};
  RPX_HIP(launch_fp8_cast_delayed(c, nullptr, fmt, static_cast<hipStream_t>(stream)),
          "rpx_fp8_cast_delayed");
  return kOk;
}

int rpx_fp8_cast_delayed2(const void* t0, int64_t rows0, int64_t cols0, int64_t row_stride0,
                          int64_t col_stride0, int64_t slot0, uint8_t* out0, uint8_t* out_t0,
                          const void* t1, int64_t rows1, int64_t cols1, int64_t row_stride1,
                          int64_t col_stride1, int64_t slot1, uint8_t* out1, uint8_t* out_t1,
                          int dtype, int fmt, const float* scales, uint32_t* amax_pending,
                          int64_t n_slots, void* stream) {
  RPX_TRY(check_dtype(dtype));
  RPX_TRY(check_fmt(fmt));
  if (scales == nullptr || amax_pending == nullptr)
    return fail_invalid("rpx_fp8_cast_delayed2: null scale state");
  RPX_TRY(delayed_args("rpx_fp8_cast_delayed2", rows0, cols0, n_slots, slot0, t0, out0, out_t0));
  RPX_TRY(delayed_args("rpx_fp8_cast_delayed2", rows1, cols1, n_slots, slot1, t1, out1, out_t1));
  const DelayedCast c0{t0, dtype, rows0, cols0, row_stride0, col_stride0, scales + slot0,
                       amax_pending + slot0 * fp8_rec_words(), out0, out_t0};
  const DelayedCast c1{t1, dtype, rows1, cols1, row_stride1, col_stride1, scales + slot1,
                       amax_pending + slot1 * fp8_rec_words(), out1, out_t1};
  RPX_HIP(launch_fp8_cast_delayed(c0, &c1, fmt, static_cast<hipStream_t>(stream)),
          "rpx_fp8_cast_delayed2");
  return kOk;
}

int rpx_fp8_scale_update(float* scales, const float* fmax, uint32_t* amax_pending,
                         uint32_t* amax_history, int32_t* cursor, int64_t n_slots,
                         int64_t history_len, void* stream) {
  if (n_slots < 1 || history_len < 1)
    return fail_invalid("rpx_fp8_scale_update: need at least one slot and one history row");
  if (scales == nullptr || fmax == nullptr || amax_pending == nullptr || amax_history == nullptr ||
      cursor == nullptr)
    return fail_invalid("rpx_fp8_scale_update: null scale state");
  RPX_HIP(launch_fp8_scale_update(scales, fmax, amax_pending, amax_history, cursor, n_slots,
                                  history_len, static_cast<hipStream_t>(stream)),
          "rpx_fp8_scale_update");
  return kOk;
}

int rpx_fp8_encode_selfcheck(int fmt, uint64_t first, uint64_t count, uint32_t* block_counts,
                             uint32_t* block_first, int64_t blocks, void* stream) {
  RPX_TRY(check_fmt(fmt));
  if (blocks < 1 || block_counts == nullptr || block_first == nullptr)
    return fail_invalid("rpx_fp8_encode_selfcheck: bad output slots");
  if (count == 0 || first + count - 1 > 0xFFFFFFFFull)
    return fail_invalid("rpx_fp8_encode_selfcheck: range must lie within 32-bit patterns");
  RPX_HIP(launch_fp8_encode_selfcheck(fmt, first, count, block_counts, block_first, blocks,
                                      static_cast<hipStream_t>(stream)),
          "rpx_fp8_encode_selfcheck");
  return kOk;
}

// ---------------------------------------------------------------------------
// Host-side codec hook: runs the exact device quantizer (divide + fp8
// rounding) on the CPU so that it can be checked exhaustively without a GPU.
// ---------------------------------------------------------------------------
int rpx_host_fp8_quantize(const float* in, int64_t n, float scale, int fmt, uint8_t* out) {
  RPX_TRY(check_fmt(fmt));
  if (n > 0 && (in == nullptr || out == nullptr)) return fail_invalid("null pointer");
  const float r = 1.0f / scale;
  for (int64_t i = 0; i < n; ++i) {
    const float q = div_rn(in[i], scale, r);
    out[i] = static_cast<uint8_t>(fmt == kE4M3FN ? f32_to_e4m3fn(q) : f32_to_e5m2(q));
  }
  return kOk;
}

// ---------------------------------------------------------------------------
// Fused in-batch MNR loss (the train-step objective)
// ---------------------------------------------------------------------------
size_t rpx_mnr_saved_bytes(int64_t n_queries, int64_t n_documents, int64_t dim) {
  if (!mnr_shape_ok(n_queries, n_documents, dim)) return 0;
  return static_cast<size_t>(mnr_saved_floats(n_queries, n_documents, dim)) * sizeof(float);
}

static int check_mnr(int64_t nq, int64_t nd, int64_t dim, float scale, size_t saved_bytes,
                     const char* who) {
  if (!mnr_shape_ok(nq, nd, dim))
    return fail_invalid(std::string(who) +
                        ": need 1 <= n_queries <= n_documents <= 8192 and 1 <= dim <= 4096 "
                        "(query i's positive is document i)");
  if (!(scale > 0.0f) || !std::isfinite(scale))
    return fail_invalid(std::string(who) + ": scale must be finite and positive");
  if (saved_bytes < static_cast<size_t>(mnr_saved_floats(nq, nd, dim)) * sizeof(float))
    return fail_invalid(std::string(who) + ": saved buffer too small");
  return kOk;
}

int rpx_mnr_forward(const void* queries, const void* documents, int dtype, int64_t n_queries,
                    int64_t n_documents, int64_t dim, float scale, float* loss, void* saved,
                    size_t saved_bytes, void* stream) {
  RPX_TRY(check_dtype(dtype));
  RPX_TRY(check_mnr(n_queries, n_documents, dim, scale, saved_bytes, "rpx_mnr_forward"));
  if (queries == nullptr || documents == nullptr || loss == nullptr || saved == nullptr)
    return fail_invalid("rpx_mnr_forward: null pointer");
  RPX_HIP(launch_mnr_forward(queries, documents, dtype, n_queries, n_documents, dim, scale, loss,
                             static_cast<float*>(saved), static_cast<hipStream_t>(stream)),
          "rpx_mnr_forward");
  return kOk;
}

int rpx_mnr_backward(const float* grad_loss, const void* saved, size_t saved_bytes,
                     int64_t n_queries, int64_t n_documents, int64_t dim, float scale,
                     void* d_queries, void* d_documents, int dtype, void* stream) {
  RPX_TRY(check_dtype(dtype));
  RPX_TRY(check_mnr(n_queries, n_documents, dim, scale, saved_bytes, "rpx_mnr_backward"));
  if (grad_loss == nullptr || saved == nullptr || d_queries == nullptr || d_documents == nullptr)
    return fail_invalid("rpx_mnr_backward: null pointer");
  RPX_HIP(launch_mnr_backward(grad_loss, static_cast<const float*>(saved), n_queries, n_documents,
                              dim, scale, d_queries, d_documents, dtype,
                              static_cast<hipStream_t>(stream)),
          "rpx_mnr_backward");
  return kOk;
}

}  // extern "C"
