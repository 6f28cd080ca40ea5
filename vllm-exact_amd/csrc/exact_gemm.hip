// Exact two-digit INT8 GEMM: C-ABI entry points, the split-K plan, the split-K finalize and
// the scalar fallback. The vector kernels are in exact_gemm_sm.hip (decode-sized M,
// HBM-bound) and exact_gemm_lds.hip (large M, MFMA-bound).

#include "exact_gemm_common.h"

namespace {

// Split-K finalize: sum the int64 partials of every split in a fixed order (any order gives
// the same integer), add the offset terms once, apply the epilogue (kernels.py:159-177).
// Grid: x over column pairs (two outputs a lane, one 16-byte load a split when N is even),
// y over rows (grid-stride past 65535 rows).
constexpr int kFinThreads = 256;
__global__ __launch_bounds__(kFinThreads) void exact_finalize_kernel(ExactParams p) {
  const int64_t mn = p.M * p.N;
  const int64_t n0 = ((int64_t)blockIdx.x * kFinThreads + threadIdx.x) * 2;
  if (n0 >= p.N) return;
  const bool two = n0 + 1 < p.N;
  const bool vec = (p.N & 1) == 0 && ((uintptr_t)p.ws & 15) == 0;  // every pair 16-byte aligned
  for (int64_t m = blockIdx.y; m < p.M; m += gridDim.y) {
    const int64_t idx = m * p.N + n0;
    int64_t t0 = 0, t1 = 0;
    if (vec) {
      for (int s = 0; s < p.sk; ++s) {
        const longlong2 v = *reinterpret_cast<const longlong2*>(p.ws + s * mn + idx);
        t0 += v.x;
        t1 += v.y;
      }
    } else {
      for (int s = 0; s < p.sk; ++s) {
        t0 += p.ws[s * mn + idx];
        if (two) t1 += p.ws[s * mn + idx + 1];
      }
    }
    if (p.offset) t0 += offset_terms(p, m, n0);
    store_f32_as(p.out, p.out_dtype, m * p.ldo + n0, exact_epilogue(t0, p.sx[m], p.sw[n0]));
    if (two) {
      if (p.offset) t1 += offset_terms(p, m, n0 + 1);
      store_f32_as(p.out, p.out_dtype, m * p.ldo + n0 + 1, exact_epilogue(t1, p.sx[m], p.sw[n0 + 1]));
    }
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
  const int64_t tot = ((int64_t)hh << 16) + ((int64_t)md << 8) + (trunc ? 0 : (int64_t)ll);
  exact_store(p, blockIdx.z, m, n, tot);
}

// Largest K extent one int32 accumulator may cover: |md| <= K * 2 * 128 * 128 < 2^31.
constexpr int64_t kMaxKch = 32768;

// Deepest instantiated LDS ring for a tile, at most `want`.
int lds_stages(int bm, int bn, int want) {
  static const int s64x64[] = {2, 4, 8}, s_mixed[] = {2, 4, 6}, s128[] = {2, 3, 4};
  const int* set = (bm == 128 && bn == 128) ? s128 : (bm == 64 && bn == 64) ? s64x64 : s_mixed;
  int s = set[0];
  for (int i = 0; i < 3; ++i)
    if (set[i] <= want) s = set[i];
  return s;
}

// cfg tuple (BM, BN, BK, warps, stages, GM[, SK[, mma]]) -> kernel family and shape:
//   BM >= 64, BK == 128 or 256, warps == 8, stages >= 2: on packed operands, the K-split kernel
//     with tile BM x BN, KG = BK / 64 K groups of 8 / KG waves and R = stages weight register
//     sets when instantiated (exact_xk_supported); otherwise the LDS-ring kernel below;
//   BK == 64, warps 3, 4, 6 or 8: on packed operands, the x-through-LDS kernel with tile BM x BN,
//     R = stages weight register sets and `warps` waves when instantiated (exact_xw_supported); otherwise, and
//     on row-major digits, the LDS-ring kernel below with BM and BN clamped to 64..128;
//   BM >= 64, BN >= 64, warps == 4, stages >= 2: LDS-ring kernel with tile
//     min(BM,128) x min(BN,128) and `stages` ring stages (clamped to instantiated depths);
//   otherwise the small-M kernel: MT = BM/16 and NT = BN/16 (each clamped to 1, 2, 4),
//     NWK = warps (4, 8, 16), C = stages (1, 2, 4), reduced to the nearest instantiated
//     combination (fewer waves first, then a shorter chunk).
// SK and BK give the split-K chunk as in kernels.py:271-272, kept a multiple of 64 (one
// MFMA K step). GM and mma are accepted and do not change the schedule: INT8 MFMA gives the
// bits of both of the reference's tensor-core paths.
int make_plan(int64_t K, const int32_t* cfg, int cfg_len, ExactPlan* out) {
  if (cfg_len < 6 || cfg_len > 8 || !cfg) return VXA_ERR_ARG;
  const int32_t BM = cfg[0], BN = cfg[1], BK = cfg[2], warps = cfg[3], stages = cfg[4];
  const int32_t SKr = cfg_len > 6 ? cfg[6] : 1;
  if (BM <= 0 || BN <= 0 || BK <= 0 || warps <= 0 || stages <= 0 || SKr <= 0) return VXA_ERR_ARG;
  ExactPlan p = {};
  if (BM >= 64 && (BK == 128 || BK == 256) && warps == 8 && stages >= 2) {
    p.family = kFamilyXk;
    p.bm = BM;
    p.bn = BN;
    p.kg = BK / 64;
    p.stages = stages;
    p.nwk = warps;
  } else if (BK == 64 && (warps == 3 || warps == 4 || warps == 6 || warps == 8)) {
    p.family = kFamilyXw;
    p.bm = BM;
    p.bn = BN;
    p.stages = stages;
    p.nwk = warps;
  } else if (BM >= 64 && BN >= 64 && warps == 4 && stages >= 2) {
    p.family = kFamilyLds;
    p.bm = BM >= 128 ? 128 : 64;
    p.bn = BN >= 128 ? 128 : 64;
    p.stages = lds_stages(p.bm, p.bn, stages);
  } else {
    p.family = kFamilySmall;
    p.mt = BM <= 16 ? 1 : (BM <= 32 ? 2 : 4);
    p.nt = BN <= 16 ? 1 : (BN <= 32 ? 2 : 4);
    int nwk = warps <= 4 ? 4 : (warps <= 8 ? 8 : 16);
    int chunk = stages <= 1 ? 1 : (stages <= 3 ? 2 : 4);
    bool found = false;
    for (int c = chunk; c >= 1 && !found; c >>= 1)
      for (int w = nwk; w >= 4 && !found; w >>= 1)
        if (exact_small_supported(p.mt, p.nt, c, w)) {
          p.chunk = c;
          p.nwk = w;
          found = true;
        }
    if (!found) return VXA_ERR_UNSUPPORTED;
  }
  const int64_t bk = cdiv<int64_t>(BK, 64) * 64;
  int64_t kch = K > 0 ? cdiv<int64_t>(cdiv<int64_t>(K, SKr), bk) * bk : bk;
  if (kch > kMaxKch) kch = kMaxKch;
  p.kch = kch;
  p.sk = K > 0 ? (int32_t)cdiv<int64_t>(K, kch) : 1;
  *out = p;
  return VXA_OK;
}

}  // namespace

extern "C" int vxa_exact_linear_plan(int64_t m, int64_t n, int64_t k, const int32_t* cfg, int cfg_len,
                                     int32_t* sk_out, int64_t* kch_out, size_t* ws_bytes) {
  if (m < 0 || n < 0 || k < 0) return VXA_ERR_ARG;
  ExactPlan pl;
  const int rc = make_plan(k, cfg, cfg_len, &pl);
  if (rc != VXA_OK) return rc;
  if (sk_out) *sk_out = pl.sk;
  if (kch_out) *kch_out = pl.kch;
  if (ws_bytes) *ws_bytes = pl.sk > 1 ? (size_t)pl.sk * (size_t)m * (size_t)n * sizeof(int64_t) : 0;
  return VXA_OK;
}

namespace {

// Launch the GEMM kernels (and the split-K finalize) for a filled-in ExactParams.
int run_exact(const ExactPlan& pl, ExactParams& ep, int trunc, bool packed, bool vec_ok, hipStream_t st) {
  hipError_t err;
  const int64_t fin_bx = cdiv<int64_t>(ep.N, 2 * kFinThreads);  // finalize grid: column pairs x rows
  const int64_t fin_by = ep.M < 65535 ? ep.M : 65535;
  if (pl.sk > 1 && fin_bx > 0x7FFFFFFFLL) return VXA_ERR_UNSUPPORTED;
  if (!vec_ok) {
    if (ep.M > 65535 || pl.sk > 65535) return VXA_ERR_UNSUPPORTED;
    dim3 grid((unsigned)cdiv<int64_t>(ep.N, 256), (unsigned)ep.M, (unsigned)pl.sk);
    hipLaunchKernelGGL(exact_scalar_kernel, grid, dim3(256), 0, st, ep, trunc);
    err = hipGetLastError();
  } else if (pl.family == kFamilyXw && packed && exact_xw_supported(pl.bm, pl.bn, pl.stages, pl.nwk, trunc != 0)) {
    err = launch_exact_xw(pl, ep, trunc != 0, st);
  } else if (pl.family == kFamilyXk && packed && exact_xk_supported(pl.bm, pl.bn, pl.kg, pl.stages, pl.nwk, trunc != 0) &&
             exact_xk_whole_rounds(pl.kg, ep.kch, ep.kpad)) {
    err = launch_exact_xk(pl, ep, trunc != 0, st);
  } else if (pl.family == kFamilyXw || pl.family == kFamilyXk || pl.family == kFamilyLds) {
    ExactPlan lp = pl;
    if (pl.family != kFamilyLds) {  // no instantiation of its own family for it: nearest LDS-ring tile
      lp.bm = pl.bm >= 128 ? 128 : 64;
      lp.bn = pl.bn >= 128 ? 128 : 64;
      lp.stages = lds_stages(lp.bm, lp.bn, 4);
    }
    err = launch_exact_lds(lp, ep, trunc != 0, packed, st);
  } else {
    err = launch_exact_small(pl, ep, trunc != 0, packed, st);
  }
  if (err == hipErrorInvalidValue) return VXA_ERR_UNSUPPORTED;
  if (err != hipSuccess) return VXA_ERR_LAUNCH;
  if (pl.sk > 1) {
    hipLaunchKernelGGL(exact_finalize_kernel, dim3((unsigned)fin_bx, (unsigned)fin_by), dim3(kFinThreads), 0, st,
                       ep);
    if (hipGetLastError() != hipSuccess) return VXA_ERR_LAUNCH;
  }
  return VXA_OK;
}

}  // namespace

extern "C" int vxa_exact_linear(const int8_t* xh, const int8_t* xl, const int32_t* cx, const int32_t* sx,
                                int64_t ldx, const int8_t* wh, const int8_t* wl, const int32_t* cw,
                                const int32_t* sw, int64_t ldw, void* out, int out_dtype, int64_t ldo, int64_t m,
                                int64_t n, int64_t k, int f, int trunc, const int32_t* cfg, int cfg_len, void* ws,
                                size_t ws_bytes, vxa_stream_t stream) {
  if (m < 0 || n < 0 || k < 0 || f < 1 || f > 15) return VXA_ERR_ARG;
  if (out_dtype != VXA_F32 && out_dtype != VXA_BF16 && out_dtype != VXA_F16) return VXA_ERR_ARG;
  ExactPlan pl;
  int rc = make_plan(k, cfg, cfg_len, &pl);
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
  ep.KT = cdiv<int64_t>(k, 64);
  ep.kpad = ep.KT * 64;
  const bool vec_ok = k > 0 && (k % 64 == 0) && (ldx % 16 == 0) && (ldw % 16 == 0) && ((uintptr_t)xh % 16 == 0) &&
                      ((uintptr_t)xl % 16 == 0) && ((uintptr_t)wh % 16 == 0) && ((uintptr_t)wl % 16 == 0);
  return run_exact(pl, ep, trunc, false, vec_ok, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int vxa_exact_linear_packed(const int8_t* xp, const int32_t* cx, const int32_t* sx, const int8_t* wp,
                                       const int32_t* cw, const int32_t* sw, void* out, int out_dtype, int64_t ldo,
                                       int64_t m, int64_t n, int64_t k, int f, int trunc, const int32_t* cfg,
                                       int cfg_len, void* ws, size_t ws_bytes, vxa_stream_t stream) {
  if (m < 0 || n < 0 || k < 0 || f < 1 || f > 15) return VXA_ERR_ARG;
  if (out_dtype != VXA_F32 && out_dtype != VXA_BF16 && out_dtype != VXA_F16) return VXA_ERR_ARG;
  ExactPlan pl;
  // the packed kernels step over whole 64-wide K tiles (zero-padded past K)
  int rc = make_plan(cdiv<int64_t>(k, 64) * 64, cfg, cfg_len, &pl);
  if (rc != VXA_OK) return rc;
  if (m == 0 || n == 0 || k == 0) {
    if (m > 0 && n > 0) return VXA_ERR_UNSUPPORTED;  // K = 0 has no packed form
    return VXA_OK;
  }
  if (!xp || !sx || !wp || !sw || !out || ldo < n) return VXA_ERR_ARG;
  if (f == 15 && (!cx || !cw)) return VXA_ERR_ARG;
  if ((uintptr_t)xp % 16 || (uintptr_t)wp % 16) return VXA_ERR_ARG;
  const size_t need = pl.sk > 1 ? (size_t)pl.sk * (size_t)m * (size_t)n * sizeof(int64_t) : 0;
  if (need > 0 && (!ws || ws_bytes < need)) return VXA_ERR_WORKSPACE;

  ExactParams ep;
  ep.xh = xp; ep.xl = nullptr; ep.cx = cx; ep.sx = sx; ep.ldx = 0;
  ep.wh = wp; ep.wl = nullptr; ep.cw = cw; ep.sw = sw; ep.ldw = 0;
  ep.out = out; ep.ldo = ldo; ep.out_dtype = out_dtype; ep.offset = (f == 15);
  ep.M = m; ep.N = n; ep.K = k; ep.kch = pl.kch; ep.sk = pl.sk;
  ep.ws = reinterpret_cast<int64_t*>(ws);
  ep.KT = cdiv<int64_t>(k, 64);
  ep.kpad = ep.KT * 64;
  return run_exact(pl, ep, trunc, true, true, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int vxa_exact_linear_bf16x(const void* x, int64_t ldx, const int8_t* wp, const int32_t* cw,
                                      const int32_t* sw, void* out, int out_dtype, int64_t ldo, int64_t m, int64_t n,
                                      int64_t k, int f, int trunc, const int32_t* cfg, int cfg_len,
                                      vxa_stream_t stream) {
  if (m < 0 || n < 0 || k < 0 || f < 1 || f > 15) return VXA_ERR_ARG;
  if (out_dtype != VXA_F32 && out_dtype != VXA_BF16 && out_dtype != VXA_F16) return VXA_ERR_ARG;
  ExactPlan pl;
  const int rc = make_plan(cdiv<int64_t>(k, 64) * 64, cfg, cfg_len, &pl);
  if (rc != VXA_OK) return rc;
  if (pl.family != kFamilySmall || pl.mt != 1 || pl.sk != 1) return VXA_ERR_UNSUPPORTED;
  if (m == 0 || n == 0) return VXA_OK;
  if (k == 0) return VXA_ERR_UNSUPPORTED;  // K = 0 has no packed form
  if (!x || !wp || !sw || !out || ldo < n || ldx < k || (f == 15 && !cw)) return VXA_ERR_ARG;
  if ((uintptr_t)wp % 16) return VXA_ERR_ARG;
  // x rows are read 16 bytes at a time
  if ((uintptr_t)x % 16 || ldx % 8) return VXA_ERR_UNSUPPORTED;
  const hipError_t err = launch_exact_fused(pl, x, ldx, wp, cw, sw, out, out_dtype, ldo, m, n, k, f, trunc != 0,
                                            reinterpret_cast<hipStream_t>(stream));
  if (err == hipErrorInvalidValue) return VXA_ERR_UNSUPPORTED;
  return err == hipSuccess ? VXA_OK : VXA_ERR_LAUNCH;
}
