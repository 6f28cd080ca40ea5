// Fragment-major packed digit layout, and digitization straight into it.
//
// Layout of a [R, K] matrix of two int8 digit planes (h, l):
//   fragment (rt, kt, plane) is 1 KiB at byte offset ((rt * KT + kt) * 2 + plane) * 1024,
//   rt = row tile of 16 rows (RT = cdiv(R, 16)), kt = K tile of 64 bytes (KT = cdiv(K, 64));
//   inside a fragment, lane l's 16 bytes sit at 16 * l and hold row rt*16 + (l & 15),
//   columns kt*64 + 16*(l >> 4) .. +16.
// This is the MFMA operand order of v_mfma_i32_16x16x64_i8, so one wave loads one operand
// as 1 KiB of contiguous memory (the row-major layout needs 16 rows x 64 bytes per load,
// which the memory pipeline serves at a third of the rate). Rows >= R and columns >= K are
// zero digits, which add nothing to any dot product.

#include "common.h"

namespace {

constexpr int kThreads = 256;

// One thread per 16-byte lane slot of a fragment pair (h and l).
__global__ __launch_bounds__(kThreads) void pack_kernel(const int8_t* __restrict__ h, const int8_t* __restrict__ l,
                                                        int64_t R, int64_t K, int64_t ldd, int8_t* __restrict__ out,
                                                        int64_t KT, int64_t total_slots, int aligned) {
  const int64_t slot = (int64_t)blockIdx.x * kThreads + threadIdx.x;  // (rt, kt, lane)
  if (slot >= total_slots) return;
  const int lane = (int)(slot & 63);
  const int64_t frag = slot >> 6;  // rt * KT + kt
  const int64_t rt = frag / KT, kt = frag % KT;
  const int64_t row = rt * 16 + (lane & 15);
  const int64_t col = kt * 64 + (lane >> 4) * 16;
  uint4 vh = {0u, 0u, 0u, 0u}, vl = {0u, 0u, 0u, 0u};
  if (row < R) {
    if (aligned && col + 16 <= K) {
      vh = *reinterpret_cast<const uint4*>(h + row * ldd + col);
      vl = *reinterpret_cast<const uint4*>(l + row * ldd + col);
    } else {
      uint8_t bh[16], bl[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const bool in = col + j < K;
        bh[j] = in ? (uint8_t)h[row * ldd + col + j] : 0;
        bl[j] = in ? (uint8_t)l[row * ldd + col + j] : 0;
      }
      vh = *reinterpret_cast<const uint4*>(bh);
      vl = *reinterpret_cast<const uint4*>(bl);
    }
  }
  int8_t* dst = out + frag * 2048 + lane * 16;
  *reinterpret_cast<uint4*>(dst) = vh;
  *reinterpret_cast<uint4*>(dst + 1024) = vl;
}

template <int DT>
__device__ inline float load_in(const void* p, int64_t i) {
  if constexpr (DT == VXA_F32) return reinterpret_cast<const float*>(p)[i];
  else if constexpr (DT == VXA_BF16) return bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
  else return (float)reinterpret_cast<const _Float16*>(p)[i];
}

__device__ inline float block_max(float v, float* red) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, shfl_xor_f32(v, m));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < kThreads / 64; ++w) r = fmaxf(r, red[w]);
  return r;
}

__device__ inline int block_sum(int v, int* red) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __builtin_amdgcn_ds_bpermute(((threadIdx.x & 63) ^ m) << 2, v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  int r = 0;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) r += red[w];
  return r;
}

// Multi-pass digitization writing the packed layout, for rows longer than the single-pass
// kernel (digitize_fast.hip) takes; same arithmetic as digitize.hip (kernels.py:22-39). One
// workgroup per row (grid = 16 * RT rows); rows >= R write zero digits. Each thread handles
// 16-column chunks of its row.
template <int DT, bool OFFSET>
__global__ __launch_bounds__(kThreads) void digitize_packed_kernel(const void* __restrict__ x, int64_t R, int64_t K,
                                                                   int64_t ldx, int8_t* __restrict__ out, int64_t KT,
                                                                   int32_t* __restrict__ cs, int32_t* __restrict__ sh,
                                                                   int F) {
  __shared__ float redf[kThreads / 64];
  __shared__ int redi[kThreads / 64];
  const int64_t row = blockIdx.x;
  const int64_t rt = row >> 4;
  const int r16 = (int)(row & 15);
  const int64_t nchunk = KT * 4;  // 16-column chunks, padded columns included
  if (row >= R) {
    for (int64_t c = threadIdx.x; c < nchunk; c += kThreads) {
      int8_t* dst = out + (rt * KT + (c >> 2)) * 2048 + ((int)(c & 3) * 16 + r16) * 16;
      *reinterpret_cast<uint4*>(dst) = uint4{0u, 0u, 0u, 0u};
      *reinterpret_cast<uint4*>(dst + 1024) = uint4{0u, 0u, 0u, 0u};
    }
    return;
  }
  const char* xr = reinterpret_cast<const char*>(x) + row * ldx * (DT == VXA_F32 ? 4 : 2);
  float a = 0.0f;
  for (int64_t i = threadIdx.x; i < K; i += kThreads) a = fmaxf(a, fabsf(load_in<DT>(xr, i)));
  a = block_max(a, redf);
  const int e = (a > 0.0f) ? __builtin_amdgcn_frexp_expf(a) : 0;
  const int s = F - e;
  const float scale = __uint_as_float((uint32_t)(s + 127) << 23);
  uint32_t csum = 0;
  for (int64_t c = threadIdx.x; c < nchunk; c += kThreads) {
    uint8_t hb[16], lb[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int64_t col = c * 16 + j;
      int32_t hd = 0, ld = 0;
      if (col < K) {
        const int32_t q = (int32_t)(load_in<DT>(xr, col) * scale);
        const uint32_t uq = (uint32_t)q;
        if constexpr (OFFSET) {
          ld = (int32_t)(uq & 255u) - 128;
          hd = (int32_t)(uq - (uint32_t)ld - 128u) >> 8;
          csum += (uint32_t)(256 * hd + ld);
        } else {
          ld = (int32_t)((uq + 128u) & 255u) - 128;
          hd = (int32_t)(uq - (uint32_t)ld) >> 8;
        }
      }
      hb[j] = (uint8_t)hd;
      lb[j] = (uint8_t)ld;
    }
    int8_t* dst = out + (rt * KT + (c >> 2)) * 2048 + ((int)(c & 3) * 16 + r16) * 16;
    *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(hb);
    *reinterpret_cast<uint4*>(dst + 1024) = *reinterpret_cast<const uint4*>(lb);
  }
  int total = 0;
  if constexpr (OFFSET) total = block_sum((int)csum, redi);
  if (threadIdx.x == 0) {
    cs[row] = total;
    sh[row] = s;
  }
}

template <int DT>
hipError_t launch_dp(const void* x, int64_t R, int64_t K, int64_t ldx, int8_t* out, int64_t KT, int32_t* cs,
                     int32_t* sh, int F, hipStream_t st) {
  const int64_t rows = cdiv<int64_t>(R, 16) * 16;
  if (F == 15)
    hipLaunchKernelGGL((digitize_packed_kernel<DT, true>), dim3((unsigned)rows), dim3(kThreads), 0, st, x, R, K, ldx,
                       out, KT, cs, sh, F);
  else
    hipLaunchKernelGGL((digitize_packed_kernel<DT, false>), dim3((unsigned)rows), dim3(kThreads), 0, st, x, R, K,
                       ldx, out, KT, cs, sh, F);
  return hipGetLastError();
}

}  // namespace

extern "C" size_t vxa_packed_bytes(int64_t rows, int64_t k) {
  if (rows <= 0 || k <= 0) return 0;
  return (size_t)cdiv<int64_t>(rows, 16) * (size_t)cdiv<int64_t>(k, 64) * 2048;
}

extern "C" int vxa_pack_digits(const int8_t* h, const int8_t* l, int64_t rows, int64_t k, int64_t ldd, int8_t* packed,
                               vxa_stream_t stream) {
  if (rows < 0 || k < 0 || ldd < k) return VXA_ERR_ARG;
  if (rows == 0 || k == 0) return VXA_OK;
  if (!h || !l || !packed) return VXA_ERR_ARG;
  const int64_t KT = cdiv<int64_t>(k, 64);
  const int64_t slots = cdiv<int64_t>(rows, 16) * KT * 64;
  const int64_t blocks = cdiv<int64_t>(slots, kThreads);
  if (blocks > 0x7FFFFFFFLL) return VXA_ERR_UNSUPPORTED;
  const int aligned = ((uintptr_t)h % 16 == 0) && ((uintptr_t)l % 16 == 0) && (ldd % 16 == 0);
  hipLaunchKernelGGL(pack_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, reinterpret_cast<hipStream_t>(stream), h,
                     l, rows, k, ldd, packed, KT, slots, aligned);
  return hipGetLastError() == hipSuccess ? VXA_OK : VXA_ERR_LAUNCH;
}

extern "C" int vxa_digitize_packed(const void* x, int x_dtype, int64_t rows, int64_t k, int64_t ldx, int8_t* packed,
                                   int32_t* cs, int32_t* sh, int f, vxa_stream_t stream) {
  if (rows < 0 || k < 0 || f < 1 || f > 15 || ldx < k) return VXA_ERR_ARG;
  if (rows == 0) return VXA_OK;
  if (!x || !packed || !cs || !sh) return VXA_ERR_ARG;
  if (k == 0 || cdiv<int64_t>(rows, 16) * 16 > 0x7FFFFFFFLL) return VXA_ERR_UNSUPPORTED;
  const int64_t KT = cdiv<int64_t>(k, 64);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (x_dtype != VXA_F32 && x_dtype != VXA_BF16 && x_dtype != VXA_F16) return VXA_ERR_ARG;
  if ((uintptr_t)packed % 16) return VXA_ERR_ARG;
  const int esize = x_dtype == VXA_F32 ? 4 : 2;
  const int vec = ((uintptr_t)x % 16 == 0) && ((ldx * esize) % 16 == 0);
  hipError_t err = launch_digitize_fast(x, x_dtype, rows, k, ldx, vec, packed, nullptr, 0, true, cs, sh, f, st);
  if (err != hipErrorInvalidValue) return err == hipSuccess ? VXA_OK : VXA_ERR_LAUNCH;
  switch (x_dtype) {
    case VXA_F32: err = launch_dp<VXA_F32>(x, rows, k, ldx, packed, KT, cs, sh, f, st); break;
    case VXA_BF16: err = launch_dp<VXA_BF16>(x, rows, k, ldx, packed, KT, cs, sh, f, st); break;
    case VXA_F16: err = launch_dp<VXA_F16>(x, rows, k, ldx, packed, KT, cs, sh, f, st); break;
    default: return VXA_ERR_ARG;
  }
  return err == hipSuccess ? VXA_OK : VXA_ERR_LAUNCH;
}
