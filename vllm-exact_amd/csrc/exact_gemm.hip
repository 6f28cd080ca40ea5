// Exact two-digit INT8 GEMM on gfx950 (CDNA4) matrix cores.
//
// out[m, n] = fp32(fp64(tot) * 2^-(sx[m] + sw[n])) with
//   tot = 2^16 * sum(xh*wh) + 2^8 * sum(xh*wl + xl*wh) [+ sum(xl*wl)]  [+ F=15 offset terms]
// (kernels.py:89-100 integer closed form; device kernels kernels.py:104-177).
//
// Every product is an int8 x int8 MFMA (v_mfma_i32_16x16x64_i8) into int32 accumulators;
// the three (or, truncated, two) digit sums are combined in int64. Integer addition is exact
// and associative, so neither the tile shape, the split of K between waves, nor the split
// of K between workgroups changes a bit of the result.
//
// Layout: x digits [M, K] and w digits [N, K] are both K-contiguous (NT GEMM). One wave
// lane (r16 = lane & 15, kq = lane >> 4) loads 32 contiguous bytes of one row per 128-wide
// K step: the four lanes of a row cover 128 contiguous bytes (one full cache line). Each
// 16-byte half feeds one MFMA; A (x) and B (w) fragments use the same K assignment, so the
// MFMA's internal K order is irrelevant to the integer dot product.

#include "common.h"

namespace {

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
  int64_t kch;  // K extent of one split
  int32_t sk;   // number of splits (gridDim.y)
  int64_t* ws;  // int64 [sk][M][N] partial sums when sk > 1
};

// int64 -> fp64 (exact: |tot| < 2^53) -> * 2^e (exact power of two built from bits,
// kernels.py:152-155) -> fp32 (RNE).
__device__ inline float exact_epilogue(int64_t tot, int32_t sxm, int32_t swn) {
  const int64_t e = -(int64_t)(sxm + swn);
  const double scale = __longlong_as_double((e + 1023) << 52);
  return (float)((double)tot * scale);
}

__device__ inline int64_t offset_terms(const ExactParams& p, int64_t m, int64_t n) {
  // F == 15: 128*(cx + cw) + 128*128*K (kernels.py:96-97, 148-151)
  return 128 * ((int64_t)p.cx[m] + (int64_t)p.cw[n]) + 128 * 128 * p.K;
}

__device__ inline v4i mfma_i8(v4i a, v4i b, v4i c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// Register-blocked kernel: the workgroup owns an output block of (16*MT) x (64*NWN) and a
// K range [kb, ke) (one split). Waves are arranged NWN (along N) x NWK (along K); each wave
// computes MT x 4 MFMA tiles of 16x16 over every NWK-th 128-wide K step of the range. Wave
// partial sums meet in an LDS int64 tile through ds_add_u64 (exact, order-free), then the
// whole workgroup applies the epilogue with coalesced stores (or writes the int64 partial
// for split-K).
template <int MT, int NWN, int NWK, bool TRUNC>
__global__ __launch_bounds__(64 * NWN * NWK) void exact_rb_kernel(ExactParams p) {
  constexpr int NT = 4;
  constexpr int BM = 16 * MT;
  constexpr int BN = 16 * NT * NWN;
  __shared__ unsigned long long red[BM * BN];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wn = wave % NWN;
  const int wk = wave / NWN;
  const int r16 = lane & 15;
  const int kq = lane >> 4;

  const int64_t nbn = cdiv<int64_t>(p.N, BN);
  const int64_t bn = blockIdx.x % nbn;
  const int64_t bm = blockIdx.x / nbn;
  const int64_t m0 = bm * BM;
  const int64_t n0 = bn * BN + wn * (16 * NT);
  const int64_t kb = (int64_t)blockIdx.y * p.kch;
  const int64_t ke = min(kb + p.kch, p.K);

  for (int i = threadIdx.x; i < BM * BN; i += blockDim.x) red[i] = 0ull;

  // Row pointers, clamped into the matrix: out-of-range rows read valid memory and their
  // results are never stored.
  const int8_t* xhp[MT];
  const int8_t* xlp[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int64_t m = min(m0 + mt * 16 + r16, p.M - 1);
    xhp[mt] = p.xh + m * p.ldx;
    xlp[mt] = p.xl + m * p.ldx;
  }
  const int8_t* whp[NT];
  const int8_t* wlp[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int64_t n = min(n0 + nt * 16 + r16, p.N - 1);
    whp[nt] = p.wh + n * p.ldw;
    wlp[nt] = p.wl + n * p.ldw;
  }

  v4i hh[MT][NT], md[MT][NT], ll[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      hh[mt][nt] = v4i{0, 0, 0, 0};
      md[mt][nt] = v4i{0, 0, 0, 0};
      ll[mt][nt] = v4i{0, 0, 0, 0};
    }

  // Full 128-wide steps: this wave takes steps wk, wk + NWK, ...
  const int64_t nfull = (ke - kb) / 128;
  for (int64_t st = wk; st < nfull; st += NWK) {
    const int64_t ko = kb + st * 128 + kq * 32;
    v4i ah[MT][2], al[MT][2], bh[NT][2], bl[NT][2];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      bh[nt][0] = *reinterpret_cast<const v4i*>(whp[nt] + ko);
      bh[nt][1] = *reinterpret_cast<const v4i*>(whp[nt] + ko + 16);
      bl[nt][0] = *reinterpret_cast<const v4i*>(wlp[nt] + ko);
      bl[nt][1] = *reinterpret_cast<const v4i*>(wlp[nt] + ko + 16);
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      ah[mt][0] = *reinterpret_cast<const v4i*>(xhp[mt] + ko);
      ah[mt][1] = *reinterpret_cast<const v4i*>(xhp[mt] + ko + 16);
      al[mt][0] = *reinterpret_cast<const v4i*>(xlp[mt] + ko);
      al[mt][1] = *reinterpret_cast<const v4i*>(xlp[mt] + ko + 16);
    }
#pragma unroll
    for (int hlf = 0; hlf < 2; ++hlf)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          hh[mt][nt] = mfma_i8(ah[mt][hlf], bh[nt][hlf], hh[mt][nt]);
          md[mt][nt] = mfma_i8(ah[mt][hlf], bl[nt][hlf], md[mt][nt]);
          md[mt][nt] = mfma_i8(al[mt][hlf], bh[nt][hlf], md[mt][nt]);
          if constexpr (!TRUNC) ll[mt][nt] = mfma_i8(al[mt][hlf], bl[nt][hlf], ll[mt][nt]);
        }
  }
  // A trailing 64-wide step (ranges are multiples of 64) goes to the next wave in turn.
  if ((ke - kb) - nfull * 128 >= 64 && wk == (int)(nfull % NWK)) {
    const int64_t ko = kb + nfull * 128 + kq * 16;
    v4i ah[MT], al[MT], bh[NT], bl[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      bh[nt] = *reinterpret_cast<const v4i*>(whp[nt] + ko);
      bl[nt] = *reinterpret_cast<const v4i*>(wlp[nt] + ko);
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      ah[mt] = *reinterpret_cast<const v4i*>(xhp[mt] + ko);
      al[mt] = *reinterpret_cast<const v4i*>(xlp[mt] + ko);
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        hh[mt][nt] = mfma_i8(ah[mt], bh[nt], hh[mt][nt]);
        md[mt][nt] = mfma_i8(ah[mt], bl[nt], md[mt][nt]);
        md[mt][nt] = mfma_i8(al[mt], bh[nt], md[mt][nt]);
        if constexpr (!TRUNC) ll[mt][nt] = mfma_i8(al[mt], bl[nt], ll[mt][nt]);
      }
  }

  __syncthreads();  // LDS tile zeroed
  // MFMA 16x16 output layout: register r of lane holds C[4*(lane>>4) + r][lane & 15].
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        int64_t tot = ((int64_t)hh[mt][nt][r] << 16) + ((int64_t)md[mt][nt][r] << 8);
        if constexpr (!TRUNC) tot += (int64_t)ll[mt][nt][r];
        const int row = mt * 16 + kq * 4 + r;
        const int col = wn * (16 * NT) + nt * 16 + r16;
        atomicAdd(&red[row * BN + col], (unsigned long long)tot);
      }
  __syncthreads();

  const int64_t nb0 = bn * BN;
  for (int i = threadIdx.x; i < BM * BN; i += blockDim.x) {
    const int row = i / BN, col = i % BN;
    const int64_t m = m0 + row, n = nb0 + col;
    if (m >= p.M || n >= p.N) continue;
    int64_t tot = (int64_t)red[i];
    if (p.sk > 1) {
      p.ws[((int64_t)blockIdx.y * p.M + m) * p.N + n] = tot;
    } else {
      if (p.offset) tot += offset_terms(p, m, n);
      store_f32_as(p.out, p.out_dtype, m * p.ldo + n, exact_epilogue(tot, p.sx[m], p.sw[n]));
    }
  }
}

// Split-K finalize: sum the int64 partials of every split in a fixed order (any order gives
// the same integer), add the offset terms once, apply the epilogue (kernels.py:159-177).
__global__ __launch_bounds__(256) void exact_finalize_kernel(ExactParams p) {
  const int64_t mn = p.M * p.N;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < mn;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = idx / p.N, n = idx % p.N;
    int64_t tot = 0;
    for (int s = 0; s < p.sk; ++s) tot += p.ws[s * mn + idx];
    if (p.offset) tot += offset_terms(p, m, n);
    store_f32_as(p.out, p.out_dtype, m * p.ldo + n, exact_epilogue(tot, p.sx[m], p.sw[n]));
  }
}

// Slow path for shapes the vector kernels do not take (K not a multiple of 64, rows not
// 16-byte aligned): one lane per output element, scalar int32 sums per digit pair. Same
// integer result, hence the same bits.
__global__ __launch_bounds__(256) void exact_scalar_kernel(ExactParams p, int trunc) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t m = blockIdx.y;
  const int64_t kb = (int64_t)blockIdx.z * p.kch;
  const int64_t ke = min(kb + p.kch, p.K);
  if (n >= p.N) return;
  const int8_t* xh = p.xh + m * p.ldx;
  const int8_t* xl = p.xl + m * p.ldx;
  const int8_t* wh = p.wh + n * p.ldw;
  const int8_t* wl = p.wl + n * p.ldw;
  int32_t hh = 0, md = 0, ll = 0;
  for (int64_t k = kb; k < ke; ++k) {
    const int32_t a = xh[k], b = xl[k], c = wh[k], d = wl[k];
    hh += a * c;
    md += a * d + b * c;
    ll += b * d;
  }
  int64_t tot = ((int64_t)hh << 16) + ((int64_t)md << 8) + (trunc ? 0 : (int64_t)ll);
  if (p.sk > 1) {
    p.ws[((int64_t)blockIdx.z * p.M + m) * p.N + n] = tot;
  } else {
    if (p.offset) tot += offset_terms(p, m, n);
    store_f32_as(p.out, p.out_dtype, m * p.ldo + n, exact_epilogue(tot, p.sx[m], p.sw[n]));
  }
}

// ---------------------------------------------------------------------------------------
// Host side: cfg decoding, split-K plan, dispatch.

// Largest K extent one int32 accumulator may cover: |md| <= K * 2 * 128 * 128 < 2^31.
constexpr int64_t kMaxKch = 32768;

struct Plan {
  int mt, nwn, nwk;  // register-blocked kernel shape
  int64_t kch;
  int32_t sk;
};

int make_plan(int64_t M, int64_t N, int64_t K, const int32_t* cfg, int cfg_len, Plan* out) {
  (void)M;
  (void)N;
  if (cfg_len < 6 || cfg_len > 8 || !cfg) return VXA_ERR_ARG;
  const int32_t BM = cfg[0], BN = cfg[1], BK = cfg[2], warps = cfg[3];
  const int32_t SKr = cfg_len > 6 ? cfg[6] : 1;
  if (BM <= 0 || BN <= 0 || BK <= 0 || warps <= 0 || SKr <= 0) return VXA_ERR_ARG;
  Plan p;
  p.mt = BM <= 16 ? 1 : (BM <= 32 ? 2 : 4);
  const int nwn_req = BN <= 64 ? 1 : (BN <= 128 ? 2 : 4);
  p.nwn = nwn_req;
  while (p.mt * p.nwn > 4) p.nwn >>= 1;  // LDS int64 tile stays <= 32 KiB
  // 64-row blocks hold 192 int32 accumulators per lane: one wave per SIMD, 4 waves.
  const int waves = (warps <= 4 || p.mt == 4) ? 4 : 8;
  p.nwk = waves / p.nwn;
  if (p.nwk < 1) p.nwk = 1;
  // kernels.py:271-272: KCH = cdiv(cdiv(K, SK), BK) * BK, SK = cdiv(K, KCH); K ranges are
  // kept in multiples of 64 (one MFMA K step), which changes the split count, never bits.
  const int64_t bk = cdiv<int64_t>(BK, 64) * 64;
  int64_t kch = K > 0 ? cdiv<int64_t>(cdiv<int64_t>(K, SKr), bk) * bk : bk;
  if (kch > kMaxKch) kch = kMaxKch;
  p.kch = kch;
  p.sk = K > 0 ? (int32_t)cdiv<int64_t>(K, kch) : 1;
  *out = p;
  return VXA_OK;
}

template <int MT, int NWN, int NWK, bool TRUNC>
hipError_t launch_rb(const ExactParams& ep, hipStream_t st) {
  constexpr int BM = 16 * MT, BN = 64 * NWN;
  const int64_t blocks = cdiv<int64_t>(ep.M, BM) * cdiv<int64_t>(ep.N, BN);
  if (blocks > 0x7FFFFFFFLL || ep.sk > 65535) return hipErrorInvalidConfiguration;
  dim3 grid((unsigned)blocks, (unsigned)ep.sk), block(64 * NWN * NWK);
  hipLaunchKernelGGL((exact_rb_kernel<MT, NWN, NWK, TRUNC>), grid, block, 0, st, ep);
  return hipGetLastError();
}

template <bool TRUNC>
hipError_t dispatch_rb(const Plan& pl, const ExactParams& ep, hipStream_t st) {
#define VXA_RB_CASE(MT_, NWN_, NWK_) \
  if (pl.mt == MT_ && pl.nwn == NWN_ && pl.nwk == NWK_) return launch_rb<MT_, NWN_, NWK_, TRUNC>(ep, st);
  VXA_RB_CASE(1, 1, 4)
  VXA_RB_CASE(1, 1, 8)
  VXA_RB_CASE(1, 2, 2)
  VXA_RB_CASE(1, 2, 4)
  VXA_RB_CASE(1, 4, 1)
  VXA_RB_CASE(1, 4, 2)
  VXA_RB_CASE(2, 1, 4)
  VXA_RB_CASE(2, 1, 8)
  VXA_RB_CASE(2, 2, 2)
  VXA_RB_CASE(2, 2, 4)
  VXA_RB_CASE(4, 1, 4)
#undef VXA_RB_CASE
  return hipErrorInvalidValue;
}

}  // namespace

extern "C" int vxa_exact_linear_plan(int64_t m, int64_t n, int64_t k, const int32_t* cfg, int cfg_len,
                                     int32_t* sk_out, int64_t* kch_out, size_t* ws_bytes) {
  if (m < 0 || n < 0 || k < 0) return VXA_ERR_ARG;
  Plan pl;
  const int rc = make_plan(m, n, k, cfg, cfg_len, &pl);
  if (rc != VXA_OK) return rc;
  if (sk_out) *sk_out = pl.sk;
  if (kch_out) *kch_out = pl.kch;
  if (ws_bytes) *ws_bytes = pl.sk > 1 ? (size_t)pl.sk * (size_t)m * (size_t)n * sizeof(int64_t) : 0;
  return VXA_OK;
}

extern "C" int vxa_exact_linear(const int8_t* xh, const int8_t* xl, const int32_t* cx, const int32_t* sx,
                                int64_t ldx, const int8_t* wh, const int8_t* wl, const int32_t* cw,
                                const int32_t* sw, int64_t ldw, void* out, int out_dtype, int64_t ldo, int64_t m,
                                int64_t n, int64_t k, int f, int trunc, const int32_t* cfg, int cfg_len, void* ws,
                                size_t ws_bytes, vxa_stream_t stream) {
  if (m < 0 || n < 0 || k < 0 || f < 1 || f > 15) return VXA_ERR_ARG;
  if (out_dtype != VXA_F32 && out_dtype != VXA_BF16 && out_dtype != VXA_F16) return VXA_ERR_ARG;
  Plan pl;
  int rc = make_plan(m, n, k, cfg, cfg_len, &pl);
  if (rc != VXA_OK) return rc;
  if (m == 0 || n == 0) return VXA_OK;
  if (!xh || !xl || !sx || !wh || !wl || !sw || !out || ldx < k || ldw < k || ldo < n) return VXA_ERR_ARG;
  if (f == 15 && (!cx || !cw)) return VXA_ERR_ARG;
  const size_t need = pl.sk > 1 ? (size_t)pl.sk * (size_t)m * (size_t)n * sizeof(int64_t) : 0;
  if (need > 0 && (!ws || ws_bytes < need)) return VXA_ERR_WORKSPACE;

  ExactParams ep;
  ep.xh = xh; ep.xl = xl; ep.cx = cx; ep.sx = sx; ep.ldx = ldx;
  ep.wh = wh; ep.wl = wl; ep.cw = cw; ep.sw = sw; ep.ldw = ldw;
  ep.out = out; ep.ldo = ldo; ep.out_dtype = out_dtype; ep.offset = (f == 15);
  ep.M = m; ep.N = n; ep.K = k; ep.kch = pl.kch; ep.sk = pl.sk;
  ep.ws = reinterpret_cast<int64_t*>(ws);

  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const bool vec_ok = (k % 64 == 0) && (ldx % 16 == 0) && (ldw % 16 == 0) && ((uintptr_t)xh % 16 == 0) &&
                      ((uintptr_t)xl % 16 == 0) && ((uintptr_t)wh % 16 == 0) && ((uintptr_t)wl % 16 == 0);
  hipError_t err;
  if (vec_ok && k > 0) {
    err = trunc ? dispatch_rb<true>(pl, ep, st) : dispatch_rb<false>(pl, ep, st);
  } else {
    if (m > 65535 || pl.sk > 65535) return VXA_ERR_UNSUPPORTED;
    dim3 grid((unsigned)cdiv<int64_t>(n, 256), (unsigned)m, (unsigned)pl.sk);
    hipLaunchKernelGGL(exact_scalar_kernel, grid, dim3(256), 0, st, ep, trunc);
    err = hipGetLastError();
  }
  if (err == hipErrorInvalidValue) return VXA_ERR_UNSUPPORTED;
  if (err != hipSuccess) return VXA_ERR_LAUNCH;
  if (pl.sk > 1) {
    const int64_t fb = cdiv<int64_t>(m * n, 256);
    const int64_t blocks = fb < 65536 ? fb : 65536;
    hipLaunchKernelGGL(exact_finalize_kernel, dim3((unsigned)blocks), dim3(256), 0, st, ep);
    if (hipGetLastError() != hipSuccess) return VXA_ERR_LAUNCH;
  }
  return VXA_OK;
}
