// Per-row F-bit fixed-point digitization on gfx950.
//
// Spec (kernels.py:3-9, CPU statement kernels.py:22-39, device kernel kernels.py:47-71):
//   a  = max_k |x[k]|,  e = frexp exponent of a (0 when a == 0),  sh = F - e
//   q  = trunc_toward_zero(x * 2^sh)            (2^sh built from its fp32 bit pattern)
//   F == 15: l = (q & 255) - 128,          h = (q - l - 128) >> 8,  cs = sum(256h + l)
//   F <  15: l = ((q + 128) & 255) - 128,  h = (q - l) >> 8,        cs = 0
// Integer steps use 32-bit unsigned wrap-around so no step is undefined even for rows
// outside the scheme's domain (absmax < 2^(F-128), Inf or NaN), where the bits are
// whatever the formula gives.
//
// This file holds the multi-pass kernel for rows longer than the single-pass kernel takes
// (digitize_fast.hip, up to 32768 columns), and the C-ABI entry point. One workgroup of
// 256 lanes per row; pass 1 reduces the row absmax, pass 2 re-reads the row (now in L2)
// and writes both digit planes with vector stores.

#include "common.h"

namespace {

constexpr int kThreads = 256;

template <int DT>
struct Elem;
template <>
struct Elem<VXA_F32> {
  static constexpr int kSize = 4;
  __device__ static float get(const void* p, int64_t i) { return reinterpret_cast<const float*>(p)[i]; }
};
template <>
struct Elem<VXA_BF16> {
  static constexpr int kSize = 2;
  __device__ static float get(const void* p, int64_t i) {
    return bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
  }
};
template <>
struct Elem<VXA_F16> {
  static constexpr int kSize = 2;
  __device__ static float get(const void* p, int64_t i) {
    return (float)reinterpret_cast<const _Float16*>(p)[i];
  }
};

// Load VEC consecutive elements starting at element i (16-byte aligned when VEC > 1).
template <int DT, int VEC>
__device__ inline void load_vec(const void* p, int64_t i, float (&v)[VEC]) {
  if constexpr (VEC == 1) {
    v[0] = Elem<DT>::get(p, i);
  } else {
    static_assert(VEC * Elem<DT>::kSize == 16, "vector path loads 16 bytes");
    const uint4 raw = *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(p) + i * Elem<DT>::kSize);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
    if constexpr (DT == VXA_F32) {
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = __uint_as_float(w[j]);
    } else if constexpr (DT == VXA_BF16) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[2 * j] = __uint_as_float(w[j] << 16);
        v[2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint16_t lo = (uint16_t)(w[j] & 0xFFFFu), hi = (uint16_t)(w[j] >> 16);
        v[2 * j] = (float)__builtin_bit_cast(_Float16, lo);
        v[2 * j + 1] = (float)__builtin_bit_cast(_Float16, hi);
      }
    }
  }
}

__device__ inline float block_max(float v, float* red) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, shfl_xor_f32(v, m));
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < kThreads / 64; ++w) r = fmaxf(r, red[w]);
  return r;
}

__device__ inline int block_sum_i32(int v, int* red) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __builtin_amdgcn_ds_bpermute(((threadIdx.x & 63) ^ m) << 2, v);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  int r = 0;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) r += red[w];
  return r;
}

template <bool OFFSET>
__device__ inline void split_digits(int32_t q, int32_t& h, int32_t& l) {
  const uint32_t uq = (uint32_t)q;
  if constexpr (OFFSET) {
    l = (int32_t)(uq & 255u) - 128;
    h = (int32_t)(uq - (uint32_t)l - 128u) >> 8;
  } else {
    l = (int32_t)((uq + 128u) & 255u) - 128;
    h = (int32_t)(uq - (uint32_t)l) >> 8;
  }
}

template <int DT, int VEC, bool OFFSET>
__global__ __launch_bounds__(kThreads) void digitize_kernel(const void* __restrict__ x, int64_t K, int64_t ldx,
                                                            int8_t* __restrict__ h, int8_t* __restrict__ l,
                                                            int64_t ldd, int32_t* __restrict__ cs,
                                                            int32_t* __restrict__ sh, int F) {
  __shared__ float redf[kThreads / 64];
  __shared__ int redi[kThreads / 64];
  const int64_t row = blockIdx.x;
  const char* xr = reinterpret_cast<const char*>(x) + row * ldx * Elem<DT>::kSize;
  const int64_t step = (int64_t)kThreads * VEC;

  // pass 1: row absmax
  float a = 0.0f;
  for (int64_t i = (int64_t)threadIdx.x * VEC; i < K; i += step) {
    float v[VEC];
    load_vec<DT, VEC>(xr, i, v);
#pragma unroll
    for (int j = 0; j < VEC; ++j) a = fmaxf(a, fabsf(v[j]));
  }
  a = block_max(a, redf);

  // exponent and power-of-two scale from bits (kernels.py:25-29)
  const int e = (a > 0.0f) ? __builtin_amdgcn_frexp_expf(a) : 0;
  const int s = F - e;
  const float scale = __uint_as_float((uint32_t)(s + 127) << 23);

  // pass 2: quantize and split
  int8_t* hr = h + row * ldd;
  int8_t* lr = l + row * ldd;
  uint32_t csum = 0;
  for (int64_t i = (int64_t)threadIdx.x * VEC; i < K; i += step) {
    float v[VEC];
    load_vec<DT, VEC>(xr, i, v);
    int8_t hv[VEC], lv[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const int32_t q = (int32_t)(v[j] * scale);  // v_cvt_i32_f32: truncation toward zero
      int32_t hd, ld;
      split_digits<OFFSET>(q, hd, ld);
      hv[j] = (int8_t)hd;
      lv[j] = (int8_t)ld;
      if constexpr (OFFSET) csum += (uint32_t)(256 * hd + ld);
    }
    if constexpr (VEC == 8) {
      *reinterpret_cast<uint2*>(hr + i) = *reinterpret_cast<const uint2*>(hv);
      *reinterpret_cast<uint2*>(lr + i) = *reinterpret_cast<const uint2*>(lv);
    } else if constexpr (VEC == 4) {
      *reinterpret_cast<uint32_t*>(hr + i) = *reinterpret_cast<const uint32_t*>(hv);
      *reinterpret_cast<uint32_t*>(lr + i) = *reinterpret_cast<const uint32_t*>(lv);
    } else {
      hr[i] = hv[0];
      lr[i] = lv[0];
    }
  }
  int total = 0;
  if constexpr (OFFSET) total = block_sum_i32((int)csum, redi);
  if (threadIdx.x == 0) {
    cs[row] = total;
    sh[row] = s;
  }
}

template <int DT, int VEC>
hipError_t launch_digitize(const void* x, int64_t rows, int64_t K, int64_t ldx, int8_t* h, int8_t* l,
                           int64_t ldd, int32_t* cs, int32_t* sh, int F, hipStream_t st) {
  dim3 grid((unsigned)rows), block(kThreads);
  if (F == 15)
    hipLaunchKernelGGL((digitize_kernel<DT, VEC, true>), grid, block, 0, st, x, K, ldx, h, l, ldd, cs, sh, F);
  else
    hipLaunchKernelGGL((digitize_kernel<DT, VEC, false>), grid, block, 0, st, x, K, ldx, h, l, ldd, cs, sh, F);
  return hipGetLastError();
}

template <int DT>
hipError_t dispatch_vec(const void* x, int64_t rows, int64_t K, int64_t ldx, int8_t* h, int8_t* l, int64_t ldd,
                        int32_t* cs, int32_t* sh, int F, hipStream_t st) {
  constexpr int VEC = 16 / Elem<DT>::kSize;
  const bool aligned = ((uintptr_t)x % 16 == 0) && ((ldx * Elem<DT>::kSize) % 16 == 0) && (K % VEC == 0) &&
                       ((uintptr_t)h % VEC == 0) && ((uintptr_t)l % VEC == 0) && (ldd % VEC == 0);
  if (aligned) return launch_digitize<DT, VEC>(x, rows, K, ldx, h, l, ldd, cs, sh, F, st);
  return launch_digitize<DT, 1>(x, rows, K, ldx, h, l, ldd, cs, sh, F, st);
}

}  // namespace

extern "C" int vxa_digitize(const void* x, int x_dtype, int64_t rows, int64_t k, int64_t ldx, int8_t* h,
                            int8_t* l, int64_t ldd, int32_t* cs, int32_t* sh, int f, vxa_stream_t stream) {
  if (rows < 0 || k < 0 || f < 1 || f > 15) return VXA_ERR_ARG;
  if (rows == 0) return VXA_OK;
  if (rows > 0x7FFFFFFFLL) return VXA_ERR_UNSUPPORTED;
  if (!x || !h || !l || !cs || !sh || ldx < k || ldd < k) return VXA_ERR_ARG;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (x_dtype != VXA_F32 && x_dtype != VXA_BF16 && x_dtype != VXA_F16) return VXA_ERR_ARG;
  const int esize = x_dtype == VXA_F32 ? 4 : 2;
  const int vec = ((uintptr_t)x % 16 == 0) && ((ldx * esize) % 16 == 0) && ((uintptr_t)h % 16 == 0) &&
                  ((uintptr_t)l % 16 == 0) && (ldd % 16 == 0);
  hipError_t err = k > 0 ? launch_digitize_fast(x, x_dtype, rows, k, ldx, vec, h, l, ldd, false, cs, sh, f, st)
                         : hipErrorInvalidValue;
  if (err != hipErrorInvalidValue) return err == hipSuccess ? VXA_OK : VXA_ERR_LAUNCH;
  switch (x_dtype) {
    case VXA_F32: err = dispatch_vec<VXA_F32>(x, rows, k, ldx, h, l, ldd, cs, sh, f, st); break;
    case VXA_BF16: err = dispatch_vec<VXA_BF16>(x, rows, k, ldx, h, l, ldd, cs, sh, f, st); break;
    case VXA_F16: err = dispatch_vec<VXA_F16>(x, rows, k, ldx, h, l, ldd, cs, sh, f, st); break;
    default: return VXA_ERR_ARG;
  }
  return err == hipSuccess ? VXA_OK : VXA_ERR_LAUNCH;
}
