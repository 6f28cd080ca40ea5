// Digitize + exact GEMM in one launch for decode at batch 1-4 (M <= 4 rows of bf16 x, packed
// weights, F <= 14).
//
// The two-launch path runs the digitize kernel (one workgroup per row) and then the small-M
// GEMM; at M = 1 the second launch and the wait between them are a quarter of the op. Here
// every GEMM workgroup digitizes the x it needs itself:
//   1. the row absmax of the M rows over all of K (a few KiB of L2-resident bf16 per
//      workgroup), reduced across the workgroup, gives each row's scale (digit_scale, the
//      digitize kernels' own helper);
//   2. in the K loop, a lane reads its 16 bf16 columns of its row straight from x and splits
//      them into the two MFMA digit operands (digits_balanced) in registers;
//   3. MFMAs, wave partials and the epilogue are the small-M kernel's (exact_gemm_sm.hip).
// The digits are the ones the digitize kernel writes, so every output bit is the two-launch
// path's. Lanes of rows past M take zero operands; their results are never stored.

#include "exact_gemm_common.h"

namespace {

constexpr int kFusedMaxRows = 4;

struct FusedParams {
  const uint16_t* x;  // bf16 [M, K], row stride ldx elements
  int64_t ldx;
  const int8_t* wp;  // packed weight digits
  const int32_t* sw;
  void* out;
  int64_t ldo;
  int32_t out_dtype;
  int32_t F;
  int64_t M, N, K, KT;
};

template <int NT, int NWK, int C, bool TRUNC>
__global__ __launch_bounds__(64 * NWK) void exact_fused_kernel(FusedParams p) {
  constexpr int BN = 16 * NT;
  __shared__ unsigned long long red[16 * BN];
  __shared__ float s_max[NWK][kFusedMaxRows];
  __shared__ float s_scale[kFusedMaxRows];
  __shared__ int32_t s_sh[kFusedMaxRows];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r16 = lane & 15;
  const int kq = lane >> 4;
  const int nthr = 64 * NWK;
  const int64_t n0 = (int64_t)blockIdx.x * BN;
  const int M = (int)p.M;

  for (int i = threadIdx.x; i < 16 * BN; i += nthr) red[i] = 0ull;

  // Operand addressing.
  const bool row_ok = r16 < M;
  float scale = 0.0f;  // this lane's row scale, set after the row-absmax pass
  const uint16_t* xrow = p.x + (int64_t)(row_ok ? r16 : 0) * p.ldx + kq * 16;
  const int8_t* whp[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int64_t tile = min((int64_t)blockIdx.x * NT + nt, cdiv<int64_t>(p.N, 16) - 1);
    whp[nt] = p.wp + tile * p.KT * 2048 + lane * 16;
  }
  // x of this lane's 16 columns of K step s; zero past K and for rows past M. The last step
  // of a K that is not a multiple of 64 reads its tail per element.
  auto x_load = [&](int64_t s, uint4 (&r)[2]) {
    if (row_ok && s * 64 + kq * 16 + 16 <= p.K) {
      r[0] = *reinterpret_cast<const uint4*>(xrow + s * 64);
      r[1] = *reinterpret_cast<const uint4*>(xrow + s * 64 + 8);
    } else {
      r[0] = uint4{0u, 0u, 0u, 0u};
      r[1] = uint4{0u, 0u, 0u, 0u};
    }
  };
  auto x_digits = [&](int64_t s, const uint4 (&r)[2], v4i& ah, v4i& al) {
    float v[16];
    const int64_t c0 = s * 64 + kq * 16;
    if (!row_ok || c0 + 16 <= p.K) {
      const uint32_t w[8] = {r[0].x, r[0].y, r[0].z, r[0].w, r[1].x, r[1].y, r[1].z, r[1].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[2 * e] = __uint_as_float(w[e] << 16);
        v[2 * e + 1] = __uint_as_float(w[e] & 0xFFFF0000u);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = c0 + j < p.K ? bf16_to_f32(xrow[s * 64 + j]) : 0.0f;
    }
    uint32_t hw[4], lw[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t h4 = 0, l4 = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        int32_t hd, ld;
        digits_balanced(v[4 * q + b], scale, hd, ld);
        h4 |= ((uint32_t)hd & 255u) << (8 * b);
        l4 |= ((uint32_t)ld & 255u) << (8 * b);
      }
      hw[q] = h4;
      lw[q] = l4;
    }
    ah = v4i{(int)hw[0], (int)hw[1], (int)hw[2], (int)hw[3]};
    al = v4i{(int)lw[0], (int)lw[1], (int)lw[2], (int)lw[3]};
  };

  constexpr bool kSplitMd = NT <= 2;
  v4i hh[NT], md[NT], mx[NT], ll[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    hh[nt] = v4i{0, 0, 0, 0};
    md[nt] = v4i{0, 0, 0, 0};
    mx[nt] = v4i{0, 0, 0, 0};
    ll[nt] = v4i{0, 0, 0, 0};
  }
  // 1. Row absmax of the M rows: each thread takes 8-column chunks (one 16-byte load each).
  float amax[kFusedMaxRows];
#pragma unroll
  for (int r = 0; r < kFusedMaxRows; ++r) {
    amax[r] = 0.0f;
    if (r < M) {
      const uint16_t* row = p.x + (int64_t)r * p.ldx;
      for (int64_t c = threadIdx.x; c * 8 < p.K; c += nthr) {
        if (c * 8 + 8 <= p.K) {
          const uint4 u = *reinterpret_cast<const uint4*>(row + c * 8);
          const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            amax[r] = fmaxf(amax[r], fabsf(__uint_as_float(w[e] << 16)));
            amax[r] = fmaxf(amax[r], fabsf(__uint_as_float(w[e] & 0xFFFF0000u)));
          }
        } else {
          for (int64_t k = c * 8; k < p.K; ++k) amax[r] = fmaxf(amax[r], fabsf(bf16_to_f32(row[k])));
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kFusedMaxRows; ++r) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) amax[r] = fmaxf(amax[r], shfl_xor_f32(amax[r], m));
    if (lane == 0) s_max[wave][r] = amax[r];
  }
  __syncthreads();
  if (threadIdx.x < kFusedMaxRows) {
    float a = 0.0f;
    for (int w = 0; w < NWK; ++w) a = fmaxf(a, s_max[w][threadIdx.x]);
    int sh;
    s_scale[threadIdx.x] = digit_scale(a, p.F, sh);
    s_sh[threadIdx.x] = sh;
  }
  __syncthreads();
  scale = s_scale[row_ok ? r16 : 0];

  // 2. K loop: wave w takes the 64-wide K steps w, w + NWK, ..., C steps per round. A round
  // issues its x loads first, then its weight loads (loads retire in issue order, so the x
  // conversion waits for x alone while the weights are in flight).
  const int64_t nsteps = p.KT;
  for (int64_t s0 = wave; s0 < nsteps; s0 += (int64_t)NWK * C) {
    v4i bh[C][NT], bl[C][NT];
    uint4 xr[C][2];
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int64_t s = s0 + (int64_t)c * NWK;
      if (s < nsteps) x_load(s, xr[c]);
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int64_t s = s0 + (int64_t)c * NWK;
      if (s < nsteps) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          bh[c][nt] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(whp[nt] + s * 2048));
          bl[c][nt] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(whp[nt] + s * 2048 + 1024));
        }
      }
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int64_t s = s0 + (int64_t)c * NWK;
      if (s < nsteps) {
        // digits of step s just before its MFMAs: one step's digits live at a time
        v4i ah, al;
        x_digits(s, xr[c], ah, al);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) hh[nt] = mfma_i8(ah, bh[c][nt], hh[nt]);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) md[nt] = mfma_i8(ah, bl[c][nt], md[nt]);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          if constexpr (kSplitMd) mx[nt] = mfma_i8(al, bh[c][nt], mx[nt]);
          else md[nt] = mfma_i8(al, bh[c][nt], md[nt]);
        }
        if constexpr (!TRUNC) {
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) ll[nt] = mfma_i8(al, bl[c][nt], ll[nt]);
        }
      }
    }
  }

  // 3. Wave partials meet in LDS (exact int64 adds), then the epilogue.
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      int64_t cross = (int64_t)md[nt][r];
      if constexpr (kSplitMd) cross += (int64_t)mx[nt][r];
      int64_t tot = ((int64_t)hh[nt][r] << 16) + (cross << 8);
      if constexpr (!TRUNC) tot += (int64_t)ll[nt][r];
      const int m = kq * 4 + r;
      if (m < M) atomicAdd(&red[m * BN + nt * 16 + r16], (unsigned long long)tot);
    }
  __syncthreads();
  for (int i = threadIdx.x; i < M * BN; i += nthr) {
    const int m = i / BN;
    const int64_t n = n0 + i % BN;
    if (n < p.N)
      store_f32_as(p.out, p.out_dtype, m * p.ldo + n, exact_epilogue((int64_t)red[i], s_sh[m], p.sw[n]));
  }
}

template <int NT, int NWK, int C, bool TRUNC>
hipError_t launch(const FusedParams& fp, hipStream_t st) {
  const int64_t blocks = cdiv<int64_t>(fp.N, 16 * NT);
  if (blocks > 0x7FFFFFFFLL) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((exact_fused_kernel<NT, NWK, C, TRUNC>), dim3((unsigned)blocks), dim3(64 * NWK), 0, st, fp);
  return hipGetLastError();
}

// (NT, C, NWK): the small-M kernel's one-row-tile shapes.
#define VXA_FUSED_TABLE(X)                                                                       \
  X(1, 1, 4) X(1, 1, 8) X(1, 1, 16) X(1, 2, 4) X(1, 2, 8) X(1, 2, 16) X(1, 4, 4) X(1, 4, 8)      \
  X(1, 4, 16) X(2, 1, 4) X(2, 1, 8) X(2, 1, 16) X(2, 2, 4) X(2, 2, 8) X(2, 2, 16) X(2, 4, 4)     \
  X(2, 4, 8) X(4, 1, 4) X(4, 1, 8) X(4, 1, 16) X(4, 2, 4) X(4, 2, 8)

template <bool TRUNC>
hipError_t dispatch(const ExactPlan& pl, const FusedParams& fp, hipStream_t st) {
#define VXA_FUSED(NT_, C_, NWK_) \
  if (pl.nt == NT_ && pl.chunk == C_ && pl.nwk == NWK_) return launch<NT_, NWK_, C_, TRUNC>(fp, st);
  VXA_FUSED_TABLE(VXA_FUSED)
#undef VXA_FUSED
  return hipErrorInvalidValue;
}

}  // namespace

int exact_fused_max_rows() { return kFusedMaxRows; }

hipError_t launch_exact_fused(const ExactPlan& pl, const void* x, int64_t ldx, const int8_t* wp, const int32_t* sw,
                              void* out, int out_dtype, int64_t ldo, int64_t m, int64_t n, int64_t k, int f,
                              bool trunc, hipStream_t st) {
  if (pl.family != kFamilySmall || pl.mt != 1 || pl.sk != 1) return hipErrorInvalidValue;
  FusedParams fp;
  fp.x = reinterpret_cast<const uint16_t*>(x);
  fp.ldx = ldx;
  fp.wp = wp;
  fp.sw = sw;
  fp.out = out;
  fp.ldo = ldo;
  fp.out_dtype = out_dtype;
  fp.F = f;
  fp.M = m;
  fp.N = n;
  fp.K = k;
  fp.KT = cdiv<int64_t>(k, 64);
  return trunc ? dispatch<true>(pl, fp, st) : dispatch<false>(pl, fp, st);
}
