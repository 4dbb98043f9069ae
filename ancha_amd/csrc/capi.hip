// C ABI entry points (include/ancha_hip.h): argument checks, the sticky failure state and
// dispatch to the gfx950 kernels.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/ancha_hip.h"
#include "kernels.hpp"
#include "status.hpp"

namespace {

std::atomic<int> g_sticky{0};
// Text of the failure that set g_sticky (written once, by the call that set it).
std::mutex g_first_mu;
std::string g_first;
thread_local std::string g_last;

// Records the first failure of the process: `code` becomes the sticky state and `text` the
// description every later call reports (device::record keeps the first panic message,
// src/device.rs:11-28).
int record_failure(int code, const std::string& text) {
  std::lock_guard<std::mutex> lock(g_first_mu);
  int expected = 0;
  if (g_sticky.compare_exchange_strong(expected, code)) g_first = text;
  return code;
}

// Failure injection for the tests of the sticky contract: ANCHA_HIP_INJECT_FAILURE=<positive
// hipError_t code> in the environment when the library loads starts the process in the failed
// state that HIP error would have left (tests/device_guard.rs of the reference drives its guard
// the same way, from the host). Nothing else reads the variable.
[[maybe_unused]] const int g_injected = [] {
  const char* v = std::getenv("ANCHA_HIP_INJECT_FAILURE");
  const int code = v ? std::atoi(v) : 0;
  if (code > 0)
    record_failure(-code, "injected failure (ANCHA_HIP_INJECT_FAILURE=" + std::to_string(code) +
                              ")");
  return code;
}();

}  // namespace

namespace ancha {

int fail(int code, const std::string& msg) {
  g_last = msg;
  return code;
}

int hip_fail(hipError_t e, const std::string& where) {
  const std::string text = where + ": " + hipGetErrorString(e);
  record_failure(-static_cast<int>(e), text);
  g_last = text;
  return -static_cast<int>(e);
}

int sticky() {
  const int s = g_sticky.load();
  if (s) {
    std::lock_guard<std::mutex> lock(g_first_mu);
    g_last = "an earlier HIP call failed (sticky device failure " + std::to_string(s) +
             "): " + g_first;
  }
  return s;
}

}  // namespace ancha

namespace {

using ancha::fail;
using ancha::hip_fail;
using ancha::sticky;

// Per-device cache: 1 = gfx950, 0 = other, -1 = unknown.
constexpr int kMaxDevices = 64;
std::atomic<int> g_arch[kMaxDevices];
std::atomic<bool> g_arch_init{false};

bool device_is_gfx950() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
  if (!g_arch_init.exchange(true))
    for (auto& a : g_arch) a.store(-1);
  int known = g_arch[dev].load();
  if (known < 0) {
    hipDeviceProp_t prop;
    known = hipGetDeviceProperties(&prop, dev) == hipSuccess &&
                    std::strncmp(prop.gcnArchName, "gfx950", 6) == 0
                ? 1
                : 0;
    g_arch[dev].store(known);
  }
  return known == 1;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

constexpr size_t kHeadDim = ANCHA_ATTENTION_HEAD_DIM;
constexpr size_t kIntMax = 0x7fffffff;

int run_attention(ancha::AttnParams& p, size_t groups, size_t tokens, size_t heads,
                  hipStream_t stream, const char* name) {
  if (groups == 0 || tokens == 0 || heads == 0) return ANCHA_HIP_OK;
  if (tokens > kIntMax || groups > kIntMax || heads > kIntMax ||
      !ancha::attention_grid_fits(groups, tokens, heads))
    return fail(ANCHA_HIP_UNSUPPORTED, std::string(name) + ": problem count exceeds the grid");
  // The kernels address one (group, head) sequence through 32-bit buffer ranges of
  // (tokens - 1) rows of stride plus one row, in bytes.
  const size_t ld = std::max({static_cast<size_t>(p.ldq), static_cast<size_t>(p.ldk),
                              static_cast<size_t>(p.ldv), static_cast<size_t>(p.ldg),
                              heads * kHeadDim});
  if (tokens > 1 && ld > (0xffffffffull - kHeadDim * 4) / 4 / (tokens - 1))
    return fail(ANCHA_HIP_UNSUPPORTED, std::string(name) + ": rows exceed the 32-bit buffer range");
  if (!device_is_gfx950()) return fail(ANCHA_HIP_UNSUPPORTED, std::string(name) + ": not a gfx950 device");
  p.groups = static_cast<int>(groups);
  p.tokens = static_cast<int>(tokens);
  p.heads = static_cast<int>(heads);
  const bool aligned = aligned16(p.q) && aligned16(p.k) && aligned16(p.v) && aligned16(p.out) &&
                       (!p.rope || aligned16(p.rope)) && p.ldq % 4 == 0 && p.ldk % 4 == 0 &&
                       p.ldv % 4 == 0;
  const hipError_t e = ancha::launch_attention(p, aligned, stream);
  if (e != hipSuccess) return hip_fail(e, name);
  return ANCHA_HIP_OK;
}

// fused::linear's shape contract (fused/mod.rs:100-127) plus the limits of 32-bit buffer
// offsets inside one 128-row tile.
int run_linear(const float* x, size_t n, size_t k, size_t ldx, const float* w, size_t m,
               const float* bias, int gelu, const float* rope, size_t tokens, size_t width,
               const float* residual, float* out, bool norm, hipStream_t stream,
               const char* name) {
  if (const int s = sticky()) return s;
  const std::string who(name);
  if (k == 0 || k % 8 != 0 || m == 0) return fail(ANCHA_HIP_UNSUPPORTED, who + ": k % 8 != 0 or empty");
  const bool epilogue = bias || gelu || rope || residual;
  if (epilogue && m % 128 != 0)
    return fail(ANCHA_HIP_UNSUPPORTED, who + ": an epilogue needs m % 128 == 0");
  if (rope && (tokens == 0 || n % tokens != 0 || width % 64 != 0 || 2 * width > m))
    return fail(ANCHA_HIP_UNSUPPORTED, who + ": rotary shape (tokens, width) does not fit");
  if (ldx < k) return fail(ANCHA_HIP_INVALID, who + ": ldx < k");
  if (n == 0) return ANCHA_HIP_OK;
  if (!x || !w || !out) return fail(ANCHA_HIP_INVALID, who + ": null tensor");
  const size_t kLimit = size_t(1) << 31;
  const size_t tiles = ((n + 127) / 128) * ((m + 127) / 128);
  if (n > kIntMax || tiles > kIntMax || (k + 64) * m * 4 >= kLimit * 2 || 128 * ldx * 4 >= kLimit ||
      128 * m * 4 >= kLimit || (rope && (tokens > kIntMax || tokens * 1024 >= kLimit * 2)))
    return fail(ANCHA_HIP_UNSUPPORTED, who + ": operand exceeds the 32-bit buffer range");
  if (!device_is_gfx950()) return fail(ANCHA_HIP_UNSUPPORTED, who + ": not a gfx950 device");
  ancha::LinearParams p{};
  p.x = x;
  p.w = w;
  p.bias = bias;
  p.rope = rope;
  p.residual = residual;
  p.out = out;
  p.ldx = static_cast<long>(ldx);
  p.n = static_cast<int>(n);
  p.k = static_cast<int>(k);
  p.m = static_cast<int>(m);
  p.tokens = rope ? static_cast<int>(tokens) : 1;
  p.width = rope ? static_cast<int>(width) : 0;
  p.gelu = gelu ? 1 : 0;
  p.norm = norm ? 1 : 0;
  const bool aligned = aligned16(x) && aligned16(w) && aligned16(out) &&
                       (!bias || aligned16(bias)) && (!residual || aligned16(residual)) &&
                       (!rope || aligned16(rope)) && ldx % 4 == 0 && m % 4 == 0;
  const hipError_t e = ancha::launch_linear(p, aligned, stream);
  if (e != hipSuccess) return hip_fail(e, name);
  return ANCHA_HIP_OK;
}

}  // namespace

extern "C" {

int ancha_hip_linear_supported(size_t k, size_t m) {
  return k > 0 && k % 8 == 0 && m > 0 && m % 128 == 0 ? 1 : 0;
}

int ancha_hip_linear(const float* x, size_t n, size_t k, size_t ldx, const float* w, size_t m,
                     const float* bias, int gelu, const float* rope, size_t tokens, size_t width,
                     const float* residual, float* out, hipStream_t stream) {
  return run_linear(x, n, k, ldx, w, m, bias, gelu, rope, tokens, width, residual, out, false,
                    stream, "ancha_hip_linear");
}

int ancha_hip_norm_linear(const float* x, size_t n, size_t k, size_t ldx, const float* w,
                          size_t m, const float* bias, int gelu, const float* rope,
                          size_t tokens, size_t width, const float* residual, float* out,
                          hipStream_t stream) {
  return run_linear(x, n, k, ldx, w, m, bias, gelu, rope, tokens, width, residual, out, true,
                    stream, "ancha_hip_norm_linear");
}

int ancha_hip_swap_axes(const float* x, size_t batch, size_t a, size_t b, size_t dim, float* out,
                        hipStream_t stream) {
  if (const int s = sticky()) return s;
  if (batch == 0 || a == 0 || b == 0 || dim == 0) return ANCHA_HIP_OK;
  if (!x || !out) return fail(ANCHA_HIP_INVALID, "ancha_hip_swap_axes: null tensor");
  if (x == out && a != 1 && b != 1)
    return fail(ANCHA_HIP_INVALID, "ancha_hip_swap_axes: out must not alias x");
  if (batch * a * b > kIntMax * size_t(4) || batch > kIntMax || a > kIntMax || b > kIntMax ||
      dim * 4 >= (size_t(1) << 31))
    return fail(ANCHA_HIP_UNSUPPORTED, "ancha_hip_swap_axes: too many rows");
  if (!device_is_gfx950()) return fail(ANCHA_HIP_UNSUPPORTED, "ancha_hip_swap_axes: not a gfx950 device");
  ancha::SwapParams p{};
  p.x = x;
  p.out = out;
  p.batch = static_cast<int>(batch);
  p.a = static_cast<int>(a);
  p.b = static_cast<int>(b);
  p.dim = static_cast<int>(dim);
  const hipError_t e = ancha::launch_swap_axes(p, aligned16(x) && aligned16(out) && dim % 4 == 0,
                                               stream);
  if (e != hipSuccess) return hip_fail(e, "ancha_hip_swap_axes");
  return ANCHA_HIP_OK;
}

int ancha_hip_unit_norm(const float* x, size_t rows, size_t dim, size_t ldx, const float* scale,
                        float* out, hipStream_t stream) {
  if (const int s = sticky()) return s;
  if (ldx < dim) return fail(ANCHA_HIP_INVALID, "ancha_hip_unit_norm: ldx < dim");
  if (rows == 0 || dim == 0) return ANCHA_HIP_OK;
  if (!x || !out) return fail(ANCHA_HIP_INVALID, "ancha_hip_unit_norm: null tensor");
  if (rows > kIntMax || dim * 4 >= (size_t(1) << 31))
    return fail(ANCHA_HIP_UNSUPPORTED, "ancha_hip_unit_norm: too many rows or columns");
  if (!device_is_gfx950()) return fail(ANCHA_HIP_UNSUPPORTED, "ancha_hip_unit_norm: not a gfx950 device");
  ancha::NormParams p{};
  p.x = x;
  p.scale = scale;
  p.out = out;
  p.ldx = static_cast<long>(ldx);
  p.rows = static_cast<int>(rows);
  p.dim = static_cast<int>(dim);
  const bool aligned = aligned16(x) && aligned16(out) && (!scale || aligned16(scale)) &&
                       dim % 4 == 0 && ldx % 4 == 0;
  const hipError_t e = ancha::launch_unit_norm(p, aligned, stream);
  if (e != hipSuccess) return hip_fail(e, "ancha_hip_unit_norm");
  return ANCHA_HIP_OK;
}

int ancha_hip_available(void) {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) return 0;
  return device_is_gfx950() ? 1 : 0;
}

int ancha_hip_attention(const float* q, const float* k, const float* v, size_t groups,
                        size_t tokens, size_t heads, size_t ldq, size_t ldk, size_t ldv,
                        const float* rope, float* out, hipStream_t stream) {
  if (const int s = sticky()) return s;
  const size_t span = heads * kHeadDim;
  if (groups && tokens && heads && (!q || !k || !v || !out))
    return fail(ANCHA_HIP_INVALID, "ancha_hip_attention: null tensor");
  if (ldq < span || ldk < span || ldv < span)
    return fail(ANCHA_HIP_INVALID,
                "ancha_hip_attention: q / k / v column ranges do not fit the row stride");
  ancha::AttnParams p{};
  p.q = q;
  p.k = k;
  p.v = v;
  p.gate = nullptr;
  p.rope = rope;
  p.out = out;
  p.ldq = static_cast<long>(ldq);
  p.ldk = static_cast<long>(ldk);
  p.ldv = static_cast<long>(ldv);
  p.ldg = 0;
  return run_attention(p, groups, tokens, heads, stream, "ancha_hip_attention");
}

int ancha_hip_gated_attention(const float* packed, size_t groups, size_t tokens, size_t columns,
                              size_t heads, const float* rope, float* out, hipStream_t stream) {
  if (const int s = sticky()) return s;
  if (columns < heads * (3 * kHeadDim + 1))
    return fail(ANCHA_HIP_UNSUPPORTED,
                "ancha_hip_gated_attention: columns < heads*(3*64+1)");
  if (groups && tokens && heads && (!packed || !out))
    return fail(ANCHA_HIP_INVALID, "ancha_hip_gated_attention: null tensor");
  const size_t inner = heads * kHeadDim;
  ancha::AttnParams p{};
  p.q = packed;
  p.k = packed + inner;
  p.v = packed + 2 * inner;
  p.gate = packed + 3 * inner;
  p.rope = rope;
  p.out = out;
  p.ldq = p.ldk = p.ldv = p.ldg = static_cast<long>(columns);
  return run_attention(p, groups, tokens, heads, stream, "ancha_hip_gated_attention");
}

int ancha_hip_check(void) { return g_sticky.load(); }

const char* ancha_hip_last_error(void) { return g_last.c_str(); }

}  // extern "C"
