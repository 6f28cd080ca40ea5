// Shared pieces of the exact two-digit INT8 GEMM (exact_gemm*.hip).
//
// out[m, n] = fp32(fp64(tot) * 2^-(sx[m] + sw[n])) with
//   tot = 2^16 * sum(xh*wh) + 2^8 * sum(xh*wl + xl*wh) [+ sum(xl*wl)]  [+ F=15 offset terms]
// (kernels.py:89-100 integer closed form; device kernels kernels.py:104-177).
// Products are int8 x int8 MFMA (v_mfma_i32_16x16x64_i8) into int32; the digit sums combine
// in int64. Integer addition is exact and associative: no tiling or K partition changes a bit.
#pragma once

#include "common.h"

struct ExactParams {
  const int8_t* xh;
  const int8_t* xl;
  const int32_t* cx;
  const int32_t* sx;
  int64_t ldx;
  const int8_t* wh;
  const int8_t* wl;
  const int32_t* cw;
  const int32_t* sw;
  int64_t ldw;
  void* out;
  int64_t ldo;
  int32_t out_dtype;
  int32_t offset;  // 1 when F == 15 (offset digits)
  int64_t M, N, K;
  int64_t kch;  // K extent of one split (multiple of 64)
  int32_t sk;   // number of splits (gridDim.y)
  int64_t* ws;  // int64 [sk][M][N] partial sums when sk > 1
  // Packed operands (fragment-major layout, pack.hip): xh / wh point at the packed
  // buffers, xl / wl are unused; KT = cdiv(K, 64) K tiles, kpad = 64 * KT.
  int64_t KT;
  int64_t kpad;
};

// Kernel family and shape picked from a cfg tuple.
enum ExactFamily { kFamilySmall = 0, kFamilyLds = 1, kFamilyScalar = 2, kFamilyXw = 3, kFamilyXk = 4 };

struct ExactPlan {
  int family;
  // small-M register-streaming kernel: MT x NT MFMA tiles per wave, NWK waves along K,
  // C 64-wide K steps whose loads are issued together
  int mt, nt, nwk, chunk;
  // LDS pipeline kernel: BM x BN workgroup tile, S ring stages; x-through-LDS kernel:
  // BM x BN workgroup tile, `stages` = R weight register sets, `nwk` = 3, 4, 6 or 8 waves
  int bm, bn, stages;
  // K-split kernel: KG K groups of nwk / KG waves (bm, bn, stages as for the x-through-LDS kernel)
  int kg;
  int64_t kch;
  int32_t sk;
};

// int64 -> fp64 (exact: |tot| < 2^53) -> * 2^e (a power of two built from its bits,
// kernels.py:152-155) -> fp32 (round to nearest even).
__device__ inline float exact_epilogue(int64_t tot, int32_t sxm, int32_t swn) {
  const int64_t e = -(int64_t)(sxm + swn);
  const double scale = __longlong_as_double((e + 1023) << 52);
  return (float)((double)tot * scale);
}

// The same value from the digit sums, tot = (hh 2^8 + md) 2^8 [+ ll]: every step below is exact
// in fp64 (|tot| < 2^53, and scaling by a power of two in range is exact), so the conversion to
// fp32 is the one rounding, as above.
template <bool TRUNC>
__device__ inline float exact_epilogue_digits(int32_t hh, int32_t md, int32_t ll, int32_t e) {
  const double hm = __builtin_fma((double)hh, 256.0, (double)md);
  if constexpr (TRUNC) return (float)__builtin_ldexp(hm, 8 - e);
  return (float)__builtin_ldexp(__builtin_fma(hm, 256.0, (double)ll), -e);
}

// fp32 -> bf16 with round-to-nearest-even for finite values (the exact GEMM's outputs are finite).
__device__ inline uint16_t f32_to_bf16_rne_finite(float f) {
  const uint32_t u = __float_as_uint(f);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// F == 15: 128*(cx + cw) + 128*128*K (kernels.py:96-97, 148-151)
__device__ inline int64_t offset_terms(const ExactParams& p, int64_t m, int64_t n) {
  return 128 * ((int64_t)p.cx[m] + (int64_t)p.cw[n]) + 128 * 128 * p.K;
}

// Final value of one output element (or its int64 partial for split-K).
__device__ inline void exact_store(const ExactParams& p, int split, int64_t m, int64_t n, int64_t tot) {
  if (p.sk > 1) {
    p.ws[((int64_t)split * p.M + m) * p.N + n] = tot;
  } else {
    if (p.offset) tot += offset_terms(p, m, n);
    store_f32_as(p.out, p.out_dtype, m * p.ldo + n, exact_epilogue(tot, p.sx[m], p.sw[n]));
  }
}

__device__ inline v4i mfma_i8(v4i a, v4i b, v4i c) { return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0); }

// Host-side launchers implemented per family (exact_gemm_sm.hip, exact_gemm_lds.hip).
// Return hipErrorInvalidValue for a shape no instantiation covers.
hipError_t launch_exact_small(const ExactPlan& pl, const ExactParams& ep, bool trunc, bool packed, hipStream_t st);
hipError_t launch_exact_lds(const ExactPlan& pl, const ExactParams& ep, bool trunc, bool packed, hipStream_t st);
// True when the small-M kernel has an instantiation for (MT, NT, C, NWK).
bool exact_small_supported(int mt, int nt, int chunk, int nwk);
// Digitize + small-M GEMM in one launch (exact_gemm_fused.hip): bf16 x [m, k] with row stride
// ldx, packed weights (cw used for F = 15), a small-M plan with MT = 1 and one split.
// hipErrorInvalidValue for a plan it has no instantiation for, and for F = 15 where the
// x-in-registers kernel does not apply.
hipError_t launch_exact_fused(const ExactPlan& pl, const void* x, int64_t ldx, const int8_t* wp, const int32_t* cw,
                              const int32_t* sw, void* out, int out_dtype, int64_t ldo, int64_t m, int64_t n,
                              int64_t k, int f, bool trunc, hipStream_t st);
// Packed operands only (exact_gemm_xw.hip).
hipError_t launch_exact_xw(const ExactPlan& pl, const ExactParams& ep, bool trunc, hipStream_t st);
bool exact_xw_supported(int bm, int bn, int r, int waves, bool trunc);
// K steps split over the waves of a workgroup (exact_gemm_xk.hip), packed operands only.
hipError_t launch_exact_xk(const ExactPlan& pl, const ExactParams& ep, bool trunc, hipStream_t st);
bool exact_xk_supported(int bm, int bn, int kg, int r, int waves, bool trunc);
// The K-split kernel takes K splits that are whole rounds (2 * KG steps of 64).
bool exact_xk_whole_rounds(int kg, int64_t kch, int64_t kpad);
