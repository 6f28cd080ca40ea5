// Single-pass digitization (the common case: rows up to 32768 columns).
//
// Same arithmetic as digitize.hip (kernels.py:22-39): row absmax, frexp exponent,
// sh = F - e, q = trunc(x * 2^sh), balanced (F < 15) or offset (F == 15) digit split.
// One workgroup per row, as many lanes as the row has 16-column chunks (64 to 1024, a
// multiple of 64); a lane owns CPT chunks of 16 columns, issues every
// load of its chunks at once (one memory latency per row instead of one per loop trip),
// keeps the values in registers through the absmax reduction, and writes the digits from
// registers: 16-byte stores into the row-major planes, or into the fragment-major packed
// layout (pack.hip). Packed rows past R (the padding of the last 16-row tile) are written
// as zero digits by their own workgroups.

#include "common.h"

namespace {

constexpr int kMaxThreads = 1024;
constexpr int kMaxWaves = kMaxThreads / 64;

template <int DT>
struct In {
  static constexpr int kBytes = DT == VXA_F32 ? 4 : 2;
};

// 16 consecutive elements starting at column c0 (zeros past K).
template <int DT>
__device__ inline void load16(const char* row, int64_t c0, int64_t K, bool vec, float (&v)[16]) {
  if (vec && c0 + 16 <= K) {
    const uint4* p = reinterpret_cast<const uint4*>(row + c0 * In<DT>::kBytes);
    if constexpr (DT == VXA_F32) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint4 w = p[q];
        v[4 * q] = __uint_as_float(w.x);
        v[4 * q + 1] = __uint_as_float(w.y);
        v[4 * q + 2] = __uint_as_float(w.z);
        v[4 * q + 3] = __uint_as_float(w.w);
      }
    } else {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint4 w = p[q];
        const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (DT == VXA_BF16) {
            v[8 * q + 2 * e] = __uint_as_float(u[e] << 16);
            v[8 * q + 2 * e + 1] = __uint_as_float(u[e] & 0xFFFF0000u);
          } else {
            v[8 * q + 2 * e] = (float)__builtin_bit_cast(_Float16, (uint16_t)(u[e] & 0xFFFFu));
            v[8 * q + 2 * e + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(u[e] >> 16));
          }
        }
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int64_t c = c0 + j;
      float f = 0.0f;
      if (c < K) {
        if constexpr (DT == VXA_F32) f = reinterpret_cast<const float*>(row)[c];
        else if constexpr (DT == VXA_BF16) f = bf16_to_f32(reinterpret_cast<const uint16_t*>(row)[c]);
        else f = (float)reinterpret_cast<const _Float16*>(row)[c];
      }
      v[j] = f;
    }
  }
}

// Workgroup max / sum: wave reductions, then the wave results in wave order from LDS (max
// is order-free; the int32 sum wraps like the other digitize paths).
__device__ inline float block_max(float v, float* red) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, shfl_xor_f32(v, m));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w) r = fmaxf(r, red[w]);
  return r;
}

__device__ inline int block_sum(int v, int* red) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __builtin_amdgcn_ds_bpermute(((threadIdx.x & 63) ^ m) << 2, v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  int r = 0;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) r += red[w];
  return r;
}

// h/l row-major planes (ldd) or packed (KT) output; PACKED selects.
template <int DT, int CPT, bool OFFSET, bool PACKED>
__global__ __launch_bounds__(kMaxThreads) void digitize_fast_kernel(const void* __restrict__ x, int64_t R, int64_t K,
                                                                 int64_t ldx, int vec, int8_t* __restrict__ h,
                                                                 int8_t* __restrict__ l, int64_t ldd, int64_t KT,
                                                                 int32_t* __restrict__ cs, int32_t* __restrict__ sh,
                                                                 int F) {
  __shared__ float redf[kMaxWaves];
  __shared__ int redi[kMaxWaves];
  const int nthr = (int)blockDim.x;
  // Packed digits interleave the 16 rows of a tile at 16-byte granularity: the workgroups of
  // one tile go to one XCD (xcd_swizzle), so their partial cache lines meet in that XCD's L2.
  const int64_t row = PACKED ? xcd_swizzle(blockIdx.x, gridDim.x) : (int64_t)blockIdx.x;
  const int64_t nchunk = PACKED ? KT * 4 : (K + 15) / 16;
  if (PACKED && row >= R) {  // padding rows of the last tile: zero digits
    const int64_t rt = row >> 4;
    const int r16 = (int)(row & 15);
    for (int64_t c = threadIdx.x; c < nchunk; c += nthr) {
      int8_t* dst = h + (rt * KT + (c >> 2)) * 2048 + ((int)(c & 3) * 16 + r16) * 16;
      *reinterpret_cast<uint4*>(dst) = uint4{0u, 0u, 0u, 0u};
      *reinterpret_cast<uint4*>(dst + 1024) = uint4{0u, 0u, 0u, 0u};
    }
    return;
  }
  const char* xr = reinterpret_cast<const char*>(x) + row * ldx * In<DT>::kBytes;

  float v[CPT][16];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int64_t c = threadIdx.x + (int64_t)i * nthr;
    if (c < nchunk) {
      load16<DT>(xr, c * 16, K, vec != 0, v[i]);
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) v[i][j] = 0.0f;
    }
  }
  float a = 0.0f;
#pragma unroll
  for (int i = 0; i < CPT; ++i)
#pragma unroll
    for (int j = 0; j < 16; ++j) a = fmaxf(a, fabsf(v[i][j]));
  a = block_max(a, redf);
  int s;
  const float scale = digit_scale(a, F, s);

  uint32_t csum = 0;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int64_t c = threadIdx.x + (int64_t)i * nthr;
    if (c >= nchunk) continue;
    // Digit bytes straight from q = trunc(v * scale) (pack_digit_bytes). Columns past K: v is
    // zero, so balanced digits are zero; offset digits take q = 128 (zero digits, and nothing
    // added to the sum, which adds 256 h + l = q - 128 per column).
    const int lim = (int)max<int64_t>(min<int64_t>(K - c * 16, 16), 0);
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      int32_t qv[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        qv[b] = (int32_t)(v[i][4 * g + b] * scale);  // truncation toward zero
        if constexpr (OFFSET) {
          qv[b] = 4 * g + b < lim ? qv[b] : 128;
          csum += (uint32_t)qv[b] - 128u;
        }
      }
      pack_digit_bytes<OFFSET>(qv, hw[g], lw[g]);
    }
    const uint4 hv = uint4{hw[0], hw[1], hw[2], hw[3]}, lv = uint4{lw[0], lw[1], lw[2], lw[3]};
    if constexpr (PACKED) {
      int8_t* dst = h + ((row >> 4) * KT + (c >> 2)) * 2048 + ((int)(c & 3) * 16 + (int)(row & 15)) * 16;
      *reinterpret_cast<uint4*>(dst) = hv;
      *reinterpret_cast<uint4*>(dst + 1024) = lv;
    } else {
      int8_t* hr = h + row * ldd + c * 16;
      int8_t* lr = l + row * ldd + c * 16;
      if (vec && c * 16 + 16 <= K) {
        *reinterpret_cast<uint4*>(hr) = hv;
        *reinterpret_cast<uint4*>(lr) = lv;
      } else {
        for (int j = 0; j < lim; ++j) {
          hr[j] = (int8_t)(hw[j >> 2] >> (8 * (j & 3)));
          lr[j] = (int8_t)(lw[j >> 2] >> (8 * (j & 3)));
        }
      }
    }
  }
  int total = 0;
  if constexpr (OFFSET) total = block_sum((int)csum, redi);
  if (threadIdx.x == 0) {
    cs[row] = total;
    sh[row] = s;
  }
}

template <int DT, bool PACKED>
hipError_t launch_cpt(int cpt, int nthr, int64_t grid_rows, const void* x, int64_t R, int64_t K, int64_t ldx,
                      int vec, int8_t* h, int8_t* l, int64_t ldd, int64_t KT, int32_t* cs, int32_t* sh, int F,
                      hipStream_t st) {
#define VXA_DF(C)                                                                                           \
  if (cpt == C) {                                                                                           \
    if (F == 15)                                                                                            \
      hipLaunchKernelGGL((digitize_fast_kernel<DT, C, true, PACKED>), dim3((unsigned)grid_rows), dim3(nthr), \
                         0, st, x, R, K, ldx, vec, h, l, ldd, KT, cs, sh, F);                                \
    else                                                                                                    \
      hipLaunchKernelGGL((digitize_fast_kernel<DT, C, false, PACKED>), dim3((unsigned)grid_rows),            \
                         dim3(nthr), 0, st, x, R, K, ldx, vec, h, l, ldd, KT, cs, sh, F);                   \
    return hipGetLastError();                                                                               \
  }
  VXA_DF(1) VXA_DF(2)
#undef VXA_DF
  return hipErrorInvalidValue;
}

}  // namespace

// Lanes per row and 16-column chunks per lane for K columns: one chunk per lane up to
// 16384 columns (64..1024 lanes), two up to 32768; 0 chunks when K needs the multi-pass
// kernel. The lane count is a multiple of 64 and depends only on K.
int digitize_fast_shape(int64_t K, int* nthr) {
  const int64_t nchunk = cdiv<int64_t>(K, 16);
  const int cpt = nchunk <= kMaxThreads ? 1 : (nchunk <= 2 * kMaxThreads ? 2 : 0);
  if (cpt == 0) return 0;
  *nthr = (int)(cdiv<int64_t>(cdiv<int64_t>(nchunk, cpt), 64) * 64);
  return cpt;
}

// Single-pass digitize into row-major planes or the packed layout. `vec` enables 16-byte
// loads and stores (caller checked alignment). Returns hipErrorInvalidValue when K needs
// the multi-pass kernels.
hipError_t launch_digitize_fast(const void* x, int x_dtype, int64_t R, int64_t K, int64_t ldx, int vec, int8_t* h,
                                int8_t* l, int64_t ldd, bool packed, int32_t* cs, int32_t* sh, int F,
                                hipStream_t st) {
  int nthr = 0;
  const int cpt = digitize_fast_shape(K, &nthr);
  if (cpt == 0) return hipErrorInvalidValue;
  const int64_t KT = cdiv<int64_t>(K, 64);
  const int64_t grid_rows = packed ? cdiv<int64_t>(R, 16) * 16 : R;
  if (grid_rows > 0x7FFFFFFFLL) return hipErrorInvalidConfiguration;
#define VXA_DT(DT)                                                                                            \
  return packed ? launch_cpt<DT, true>(cpt, nthr, grid_rows, x, R, K, ldx, vec, h, l, ldd, KT, cs, sh, F, st)        \
                : launch_cpt<DT, false>(cpt, nthr, grid_rows, x, R, K, ldx, vec, h, l, ldd, KT, cs, sh, F, st);
  switch (x_dtype) {
    case VXA_F32: VXA_DT(VXA_F32)
    case VXA_BF16: VXA_DT(VXA_BF16)
    case VXA_F16: VXA_DT(VXA_F16)
    default: return hipErrorInvalidValue;
  }
#undef VXA_DT
}
