// Shared device helpers for the gfx950 exact linear path.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/vllm_exact_amd.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef unsigned short v8u16 __attribute__((ext_vector_type(8)));
typedef unsigned int v2u32 __attribute__((ext_vector_type(2)));
typedef unsigned int v4u32 __attribute__((ext_vector_type(4)));

template <typename T>
__host__ __device__ inline constexpr T cdiv(T a, T b) {
  return (a + b - 1) / b;
}

// bf16 bit pattern -> fp32 (exact).
__device__ inline float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// fp32 -> bf16 with round-to-nearest-even; NaN -> 0x7FC0 (the canonical quiet NaN torch
// produces). Infinities and overflow follow IEEE (the rounding bias carries into the
// exponent and saturates at the Inf pattern).
__device__ inline uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)0x7FC0u;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Store one fp32 value to an output of runtime dtype (uniform branch across the wave).
__device__ inline void store_f32_as(void* out, int dtype, int64_t idx, float v) {
  if (dtype == VXA_F32) {
    reinterpret_cast<float*>(out)[idx] = v;
  } else if (dtype == VXA_BF16) {
    reinterpret_cast<uint16_t*>(out)[idx] = f32_to_bf16_rne(v);
  } else {
    reinterpret_cast<_Float16*>(out)[idx] = (_Float16)v;  // v_cvt_f16_f32: RNE
  }
}

// Wave-wide lane shuffles built on ds_bpermute (byte-addressed lane index).
__device__ inline float shfl_f32(float v, int src_lane) {
  return __int_as_float(__builtin_amdgcn_ds_bpermute(src_lane << 2, __float_as_int(v)));
}
__device__ inline float shfl_xor_f32(float v, int mask) {
  const int lane = threadIdx.x & 63;
  return shfl_f32(v, lane ^ mask);
}

// Row scale of the digitization (kernels.py:25-29): e = frexp exponent of the row absmax
// (0 for a zero row), sh = F - e, scale = 2^sh built from its exponent bits.
__device__ inline float digit_scale(float absmax, int F, int& sh) {
  const int e = (absmax > 0.0f) ? __builtin_amdgcn_frexp_expf(absmax) : 0;
  sh = F - e;
  return __uint_as_float((uint32_t)(sh + 127) << 23);
}

// The packed digit words of four values q_j = trunc(v_j * scale), as the MFMA operands take
// them: byte j of h4 / l4 is the low byte of q_j's high / low digit.
//   Balanced digits (F < 15, kernels.py:35-38): q = 256 h + l, l in [-128, 127], so
//   l = ((q + 128) & 255) - 128 and h = (q - l) >> 8: h's byte is byte 1 of q + 128 and l's
//   byte 0 of q + 128 with its top bit flipped.
//   Offset digits (F == 15, kernels.py:31-34): q = 256 h + l + 128 in 32-bit wrap-around
//   arithmetic, so l = (q & 255) - 128 and h = (q - l - 128) >> 8: h's byte is byte 1 of q and
//   l's byte 0 of q with its top bit flipped; 256 h + l = q - 128, and q = 128 gives zero
//   digits.
// Four byte permutes and one xor.
template <bool OFFSET>
__device__ inline void pack_digit_bytes(const int32_t (&q)[4], uint32_t& h4, uint32_t& l4) {
  uint32_t y[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) y[j] = OFFSET ? (uint32_t)q[j] : (uint32_t)q[j] + 128u;
  const uint32_t p01 = __builtin_amdgcn_perm(y[1], y[0], 0x05040100u);  // y0.b0 y0.b1 y1.b0 y1.b1
  const uint32_t p23 = __builtin_amdgcn_perm(y[3], y[2], 0x05040100u);  // y2.b0 y2.b1 y3.b0 y3.b1
  l4 = __builtin_amdgcn_perm(p23, p01, 0x06040200u) ^ 0x80808080u;
  h4 = __builtin_amdgcn_perm(p23, p01, 0x07050301u);
}

// Workgroups are handed to the 8 XCDs round-robin (linear id % 8), and each XCD has its own
// L2. This bijection gives XCD x the logical ids [x*base + min(x, rem), ...) in dispatch
// order, so neighbouring logical tiles (which share an operand tile) run on one XCD at about
// the same time and meet in its L2.
__device__ inline int64_t xcd_swizzle(int64_t lin, int64_t total) {
  constexpr int64_t kXcd = 8;
  const int64_t xcd = lin % kXcd, j = lin / kXcd;
  const int64_t base = total / kXcd, rem = total % kXcd;
  return xcd * base + (xcd < rem ? xcd : rem) + j;
}

// Single-pass digitize (digitize_fast.hip) into row-major planes (h, l, ldd) or, when
// `packed`, the fragment-major layout at h. hipErrorInvalidValue: K needs the multi-pass path.
hipError_t launch_digitize_fast(const void* x, int x_dtype, int64_t R, int64_t K, int64_t ldx, int vec, int8_t* h,
                                int8_t* l, int64_t ldd, bool packed, int32_t* cs, int32_t* sh, int F,
                                hipStream_t st);

#define VXA_CHECK_LAUNCH()                         \
  do {                                             \
    if (hipGetLastError() != hipSuccess) return VXA_ERR_LAUNCH; \
  } while (0)
