// The exactmm::linear op without any allocation, for callers that cannot allocate device
// memory (code under HIP graph capture, fixed serving loops, harnesses that forbid it).
//
// It runs what vxa_digitize_packed followed by vxa_exact_linear_packed run, with the two
// intermediates those leave to the caller -- the packed activation digits with their row sums
// and shifts, and the split-K int64 partials -- placed in one file-scope device array of
// VXA_NOALLOC_SCRATCH_BYTES. Each GPU holds its own copy of the array until the process ends;
// its device address is looked up once per device (hipGetSymbolAddress) at the first call on
// that device and kept. Calls that overlap on one GPU share the array and race: a caller
// serialises them (one stream, or events). Arguments are checked on the host before anything is
// launched, so a refused call leaves the array alone. Every byte the kernels read from the array is
// written earlier in the same call (the digitize kernel writes every packed byte, padding
// included; each split writes its whole partial tile), so nothing needs clearing between
// calls.

#include <mutex>

#include "common.h"

namespace {

constexpr size_t kScratchBytes = VXA_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` on each device, once looked up

// Device address of this device's scratch array (the caller's current device).
int scratch_base(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return VXA_ERR_LAUNCH;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return VXA_ERR_LAUNCH;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return VXA_OK;
}

constexpr size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

}  // namespace

extern "C" int vxa_exact_linear_op_noalloc(const void* x, int x_dtype, int64_t ldx, const int8_t* wp,
                                           const int32_t* cw, const int32_t* sw, void* out, int out_dtype,
                                           int64_t ldo, int64_t m, int64_t n, int64_t k, int f, int trunc,
                                           const int32_t* cfg, int cfg_len, vxa_stream_t stream) {
  if (m < 0 || n < 0 || k < 0 || f < 1 || f > 15) return VXA_ERR_ARG;
  int32_t sk = 0;
  int64_t kch = 0;
  size_t ws_bytes = 0;
  // the same plan vxa_exact_linear_packed makes: K rounded up to whole 64-column tiles
  int rc = vxa_exact_linear_plan(m, n, cdiv<int64_t>(k, 64) * 64, cfg, cfg_len, &sk, &kch, &ws_bytes);
  if (rc != VXA_OK) return rc;
  if (m == 0 || n == 0) return VXA_OK;
  if (k == 0) return VXA_ERR_UNSUPPORTED;  // K = 0 has no packed form
  // Every argument both launches check, checked here first: a call refused with VXA_ERR_ARG
  // launches nothing, so it cannot overwrite the scratch of a call still running on this GPU.
  if (!x || ldx < k || (x_dtype != VXA_F32 && x_dtype != VXA_BF16 && x_dtype != VXA_F16)) return VXA_ERR_ARG;
  if (!wp || !sw || !out || ldo < n || (out_dtype != VXA_F32 && out_dtype != VXA_BF16 && out_dtype != VXA_F16))
    return VXA_ERR_ARG;
  if ((uintptr_t)wp % 16 || (f == 15 && !cw)) return VXA_ERR_ARG;
  if (cdiv<int64_t>(m, 16) * 16 > 0x7FFFFFFFLL) return VXA_ERR_UNSUPPORTED;
  const size_t xp_bytes = align256(vxa_packed_bytes(m, k));
  const size_t sum_bytes = align256((size_t)m * sizeof(int32_t));
  if (xp_bytes > kScratchBytes || ws_bytes > kScratchBytes || xp_bytes + 2 * sum_bytes + ws_bytes > kScratchBytes)
    return VXA_ERR_TOO_LARGE;
  void* base = nullptr;
  rc = scratch_base(&base);
  if (rc != VXA_OK) return rc;
  int8_t* xp = static_cast<int8_t*>(base);
  int32_t* cx = reinterpret_cast<int32_t*>(xp + xp_bytes);
  int32_t* sx = reinterpret_cast<int32_t*>(reinterpret_cast<uint8_t*>(cx) + sum_bytes);
  void* ws = ws_bytes ? static_cast<void*>(reinterpret_cast<uint8_t*>(sx) + sum_bytes) : nullptr;
  rc = vxa_digitize_packed(x, x_dtype, m, k, ldx, xp, cx, sx, f, stream);
  if (rc != VXA_OK) return rc;
  return vxa_exact_linear_packed(xp, cx, sx, wp, cw, sw, out, out_dtype, ldo, m, n, k, f, trunc, cfg, cfg_len, ws,
                                 ws_bytes, stream);
}
