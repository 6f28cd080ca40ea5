// Large-M exact GEMM on packed digits: the x tile through an LDS ring, the weight fragments
// straight into registers.
//
// Workgroup tile BM x (NWN * WN): NWN waves side by side along N, each computing all BM rows
// of its WN columns (times WMS waves along M, each on BM / WMS rows). The x fragments of a K
// step (BM/16 tiles x 2 digit planes, 1 KiB each in MFMA lane order) are shared by the waves,
// so they go through a ring of S = R + 1 LDS stages filled by global_load_lds_dwordx4 (gfx950
// direct-to-LDS loads, split over the waves; when the count does not divide evenly, some
// waves copy one fragment a second time, the same bytes to the same place). The weight fragments of a wave are its own: each is one contiguous
// 1 KiB global_load_dwordx4 per wave straight into a ring of R register sets, so the weight
// stream (the HBM-bound operand) keeps R steps in flight per wave without using LDS.
//
// K step j:  s_waitcnt for the loads of step j (x stage and weight set) and for this wave's
// LDS reads -> s_barrier (every wave's quarter of stage j landed, and every wave has finished
// reading stage j-1) -> issue
// the x loads of step j+R into the stage of step j-1 -> read stage j into registers ->
// MFMAs -> issue the weight loads of step j+R into the register set of step j.
// Every step issues the same loads (past the last step they repeat step nk-1 into a stage or
// set no live step reads), so the wait count is one constant and the loop has no branch.
//
// Epilogue: for 2-byte outputs without a K split or offset terms (the STAGED instantiations)
// the workgroup converts its accumulators, assembles the BM x BN tile in the free x ring and
// stores it as 16-byte pieces of whole rows; otherwise every lane stores its own values.
//
// Products and sums are the same int32 MFMA dot products as the other kernels; only the
// order of integer additions differs, which changes no bit.

#include "exact_gemm_common.h"

// The direct-to-LDS copies set M0 from inline asm and name it as clobbered; clang warns that
// M0 is a reserved register. The build checks the generated code of these kernels
// (check_async_loads.py): no compiler-generated instruction uses M0 in them.
#pragma clang diagnostic ignored "-Winline-asm"

namespace {

typedef __attribute__((address_space(3))) void lds_void_t;

// Bytes of one row of the output tile as the epilogue stages it in LDS: BN 2-byte values plus
// 16 bytes of padding, so the four row groups of one LDS store land on different banks
// (BN is a multiple of 32).
constexpr int staged_row_bytes(int bn) { return bn * 2 + 16; }
// The staged tile fits in the x ring.
constexpr bool staged_fits(int bm, int bn, int r) { return bm * staged_row_bytes(bn) <= (r + 1) * 2 * (bm / 16) * 1024; }

// STAGED: 2-byte output, one K split, no F = 15 offset terms; the epilogue goes through LDS.
template <int BM, int NWN, int WN, int R, int WMS, bool TRUNC, bool STAGED>
__global__ __launch_bounds__(64 * NWN * WMS) void exact_xw_kernel(ExactParams p) {
  constexpr int NWAVE = NWN * WMS;  // waves: NWN along N times WMS along M
  constexpr int TMA = BM / 16;      // 16-row tiles of the x tile
  constexpr int TM = TMA / WMS;     // ... of one wave
  constexpr int TN = WN / 16;       // 16-column tiles of one wave
  constexpr int BN = NWN * WN;      // workgroup tile width
  constexpr int S = R + 1;          // x ring stages
  constexpr int NFX = 2 * TMA;      // x fragments per stage (h and l planes)
  constexpr int LX = (NFX + NWAVE - 1) / NWAVE;  // x fragments each wave copies per stage
  constexpr int LW = 2 * TN;        // weight fragments each wave loads per step
  constexpr int kWait = (R - 1) * (LX + LW);
  static_assert(TMA % WMS == 0, "row tiles split evenly over the waves along M");
  static_assert(kWait <= 63, "vmcnt limit");
  static_assert(!STAGED || staged_fits(BM, BN, R), "staged tile fits the ring");
  __shared__ __attribute__((aligned(1024))) int8_t ring[S * NFX * 1024];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wn = wave % NWN;  // column block of this wave
  const int wm = wave / NWN;  // row block of this wave (WMS > 1)

  // Logical tile order: M tiles fastest, then N tiles, then K splits; the workgroups that
  // share one weight tile are neighbours and, through xcd_swizzle, on one XCD.
  const int64_t nbm = cdiv<int64_t>(p.M, BM);
  const int64_t nbn = cdiv<int64_t>(p.N, BN);
  const int64_t t = xcd_swizzle((int64_t)blockIdx.y * gridDim.x + blockIdx.x, (int64_t)gridDim.x * gridDim.y);
  const int64_t bm = t % nbm;
  const int64_t bn = (t / nbm) % nbn;
  const int split = (int)(t / (nbm * nbn));
  const int64_t m0 = bm * BM + wm * (BM / WMS);
  const int64_t n0 = bn * BN + wn * WN;
  const int64_t kb = (int64_t)split * p.kch;
  const int64_t ke = min(kb + p.kch, p.kpad);
  const int64_t nk = (ke - kb) >> 6;
  const int64_t kt0 = kb >> 6;

  // x fragments this wave copies into each stage (tiles past M clamped: rows >= M are never stored)
  const int8_t* xsrc[LX];
  int xdst[LX];
#pragma unroll
  for (int i = 0; i < LX; ++i) {
    const int f = (wave + NWAVE * i) % NFX;  // fragment f: plane f / TMA, tile f % TMA
    const int64_t tile = min(bm * TMA + f % TMA, cdiv<int64_t>(p.M, 16) - 1);
    xsrc[i] = p.xh + (tile * p.KT + kt0) * 2048 + (f / TMA) * 1024 + lane * 16;
    xdst[i] = f * 1024;
  }
  // weight fragments of this wave (tiles past N clamped: columns >= N are never stored)
  const int8_t* wsrc[TN];
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) {
    const int64_t tile = min((n0 >> 4) + tn, cdiv<int64_t>(p.N, 16) - 1);
    wsrc[tn] = p.wh + (tile * p.KT + kt0) * 2048 + lane * 16;
  }

  // The x copies are issued from inline asm: the compiler's wait-count pass cannot tell which
  // stage a direct-to-LDS load writes, and with the builtin it drains every load in flight
  // (weights included) once per unrolled loop trip. Only this code reads the ring, after the
  // explicit s_waitcnt + s_barrier of each step. The asm has no register outputs; M0 (the
  // LDS destination, wave-uniform) needs one wait state before the load that uses it.
  auto issue_x = [&](int64_t step, int slot) {
#pragma unroll
    for (int i = 0; i < LX; ++i) {
      const uint32_t lds = __builtin_amdgcn_readfirstlane(
          (uint32_t)(uintptr_t)(lds_void_t*)(ring + slot * NFX * 1024 + xdst[i]));
      asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(xsrc[i] + step * 2048),
                   "s"(lds)
                   : "memory", "m0");
    }
  };
  // When one M tile covers all rows, each weight fragment is read by this workgroup alone:
  // stream it with non-temporal loads. Otherwise the workgroups of the other M tiles read the
  // same fragments at about the same time (xcd_swizzle) and should find them in L2.
  const bool stream_w = nbm == 1;
  auto load_w = [&](int64_t step, v4i (&wb)[LW]) {
    if (stream_w) {
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        wb[2 * tn] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wsrc[tn] + step * 2048));
        wb[2 * tn + 1] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wsrc[tn] + step * 2048 + 1024));
      }
    } else {
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        wb[2 * tn] = *reinterpret_cast<const v4i*>(wsrc[tn] + step * 2048);
        wb[2 * tn + 1] = *reinterpret_cast<const v4i*>(wsrc[tn] + step * 2048 + 1024);
      }
    }
  };

  v4i hh[TM][TN], md[TM][TN], ll[TM][TN];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      hh[tm][tn] = v4i{0, 0, 0, 0};
      md[tm][tn] = v4i{0, 0, 0, 0};
      ll[tm][tn] = v4i{0, 0, 0, 0};
    }

  // Row and column scales of this wave's outputs, loaded before the K loop so the staged
  // epilogue does not wait for them, where the registers allow: accumulators, weight ring and
  // x fragments (VGPRs of one wave) plus the scales stay 32 below the budget of a wave, 256
  // registers when two or more waves share a SIMD and 512 (with the accumulation registers)
  // when one does.
  const int r16 = lane & 15, kq = lane >> 4;
  constexpr int kLiveRegs = 4 * (TM * TN * (TRUNC ? 2 : 3) + R * LW + 2 * TM) + 4 * TM + TN;
  constexpr bool kPrefetch = STAGED && kLiveRegs <= (NWAVE > 4 ? 224 : 480);
  int32_t swp[TN], sxp[TM][4];
  if constexpr (kPrefetch) {
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) swp[tn] = p.sw[min(n0 + tn * 16 + r16, p.N - 1)];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int r = 0; r < 4; ++r) sxp[tm][r] = p.sx[min(m0 + tm * 16 + kq * 4 + r, p.M - 1)];
  }

  const int8_t* lds_lane = ring + lane * 16;
  auto step = [&](int64_t j, v4i (&wb)[LW]) {
    // lgkmcnt(0): this wave's reads of stage j-1 are complete before any wave refills it
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(kWait) : "memory");
    const int64_t nxt = j + R < nk ? j + R : nk - 1;
    issue_x(nxt, (int)((j + R) % S));
    const int8_t* stage = lds_lane + (int)(j % S) * NFX * 1024;
    v4i xh[TM], xl[TM];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      xh[tm] = *reinterpret_cast<const v4i*>(stage + (wm * TM + tm) * 1024);
      xl[tm] = *reinterpret_cast<const v4i*>(stage + (TMA + wm * TM + tm) * 1024);
    }
    // One pass per digit product over all tiles: the two updates of an `md` accumulator are
    // TM * TN MFMAs apart, so no MFMA waits for the result of the one before it.
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) hh[tm][tn] = mfma_i8(xh[tm], wb[2 * tn], hh[tm][tn]);
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) md[tm][tn] = mfma_i8(xh[tm], wb[2 * tn + 1], md[tm][tn]);
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) md[tm][tn] = mfma_i8(xl[tm], wb[2 * tn], md[tm][tn]);
    if constexpr (!TRUNC) {
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) ll[tm][tn] = mfma_i8(xl[tm], wb[2 * tn + 1], ll[tm][tn]);
    }
    load_w(nxt, wb);
  };

  if (nk > 0) {
    v4i w[R][LW];
#pragma unroll
    for (int s = 0; s < R; ++s) {
      const int64_t st = s < nk ? s : nk - 1;
      issue_x(st, s);
      load_w(st, w[s]);
    }
    int64_t j = 0;
    for (; j + R <= nk; j += R) {
#pragma unroll
      for (int r = 0; r < R; ++r) step(j + r, w[r]);
    }
#pragma unroll
    for (int r = 0; r < R - 1; ++r)
      if (j + r < nk) step(j + r, w[r]);
    // the repeated loads of the tail still target this workgroup's LDS and registers: drain them
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }

  // Register r of lane holds C[4*(lane>>4) + r][lane & 15] of each 16 x 16 tile: a store
  // straight from registers writes 2-byte values 16 to a row. The staged epilogue first
  // assembles the workgroup's BM x BN tile in LDS (the x ring is free now), then writes it
  // out in 16-byte pieces, whole rows at a time.
  if constexpr (STAGED) {
    constexpr int kRowBytes = staged_row_bytes(BN);
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = min(m0 + tm * 16 + kq * 4 + r, p.M - 1);
        const int32_t sxm = kPrefetch ? sxp[tm][r] : p.sx[m];
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
          const int64_t n = min(n0 + tn * 16 + r16, p.N - 1);
          int64_t tot = ((int64_t)hh[tm][tn][r] << 16) + ((int64_t)md[tm][tn][r] << 8);
          if constexpr (!TRUNC) tot += (int64_t)ll[tm][tn][r];
          const float v = exact_epilogue(tot, sxm, kPrefetch ? swp[tn] : p.sw[n]);
          const uint16_t bits = p.out_dtype == VXA_BF16 ? f32_to_bf16_rne(v) : __builtin_bit_cast(uint16_t, (_Float16)v);
          const int row = wm * (BM / WMS) + tm * 16 + kq * 4 + r;
          const int col = wn * WN + tn * 16 + r16;
          *reinterpret_cast<uint16_t*>(ring + row * kRowBytes + col * 2) = bits;
        }
      }
    __syncthreads();
    constexpr int kPieces = BN / 8;  // 16-byte pieces per row
    const bool whole = reinterpret_cast<uintptr_t>(p.out) % 16 == 0 && p.ldo % 8 == 0;
    for (int i = threadIdx.x; i < BM * kPieces; i += 64 * NWAVE) {
      const int row = i / kPieces, c = i % kPieces;
      const int64_t m = bm * BM + row, n = bn * BN + c * 8;
      if (m >= p.M || n >= p.N) continue;
      const int8_t* src = ring + row * kRowBytes + c * 16;
      uint16_t* dst = reinterpret_cast<uint16_t*>(p.out) + m * p.ldo + n;
      if (whole && n + 8 <= p.N) {
        *reinterpret_cast<v4i*>(dst) = *reinterpret_cast<const v4i*>(src);
      } else {
        for (int e = 0; e < 8 && n + e < p.N; ++e) dst[e] = reinterpret_cast<const uint16_t*>(src)[e];
      }
    }
    return;
  }
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = m0 + tm * 16 + kq * 4 + r;
        const int64_t n = n0 + tn * 16 + r16;
        if (m < p.M && n < p.N) {
          int64_t tot = ((int64_t)hh[tm][tn][r] << 16) + ((int64_t)md[tm][tn][r] << 8);
          if constexpr (!TRUNC) tot += (int64_t)ll[tm][tn][r];
          exact_store(p, split, m, n, tot);
        }
      }
}

template <int BM, int NWN, int WN, int R, int WMS, bool TRUNC>
hipError_t launch(const ExactParams& ep, hipStream_t st) {
  constexpr bool kCanStage = staged_fits(BM, NWN * WN, R);
  const int64_t blocks = cdiv<int64_t>(ep.M, BM) * cdiv<int64_t>(ep.N, NWN * WN);
  if (blocks > 0x7FFFFFFFLL || ep.sk > 65535) return hipErrorInvalidConfiguration;
  const dim3 grid((unsigned)blocks, (unsigned)ep.sk), block(64 * NWN * WMS);
  if constexpr (kCanStage) {
    if (ep.sk == 1 && ep.out_dtype != VXA_F32 && !ep.offset) {
      hipLaunchKernelGGL((exact_xw_kernel<BM, NWN, WN, R, WMS, TRUNC, true>), grid, block, 0, st, ep);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((exact_xw_kernel<BM, NWN, WN, R, WMS, TRUNC, false>), grid, block, 0, st, ep);
  return hipGetLastError();
}

// Instantiated (BM, NWN, WN, R, WMS); the 4-dot (F = 15) variants only where three
// accumulator sets fit. WMS = 2 runs two waves per SIMD, each on half of the BM rows. The
// 96-column tiles (NWN = 3 or 6) put a 24576-column product on 256 workgroups.
#define VXA_XW_TABLE(X)                                                                                   \
  X(32, 4, 32, 4, 1, 1) X(32, 4, 64, 4, 1, 1) X(64, 4, 16, 4, 1, 1) X(64, 4, 32, 4, 1, 1)                 \
  X(64, 4, 48, 4, 1, 1) X(64, 4, 64, 3, 1, 1) X(64, 4, 64, 4, 1, 0) X(128, 4, 16, 4, 1, 1)                \
  X(128, 4, 32, 3, 1, 1) X(128, 4, 32, 4, 1, 0) X(128, 4, 48, 3, 1, 0) X(128, 4, 48, 4, 1, 0)             \
  X(64, 4, 32, 4, 2, 1) X(64, 4, 48, 4, 2, 1) X(64, 4, 64, 4, 2, 0) X(128, 4, 32, 4, 2, 1)                \
  X(128, 4, 48, 3, 2, 0) X(128, 4, 48, 4, 2, 0) X(128, 4, 64, 2, 2, 0) X(64, 6, 16, 4, 1, 1)              \
  X(64, 6, 16, 6, 1, 1) X(64, 6, 16, 8, 1, 1) X(64, 3, 32, 4, 1, 1) X(64, 3, 32, 6, 1, 1)

template <bool TRUNC>
hipError_t dispatch(const ExactPlan& pl, const ExactParams& ep, hipStream_t st) {
#define VXA_XW(BM_, NWN_, WN_, R_, WMS_, FOUR_)                                             \
  if constexpr (TRUNC || FOUR_) {                                                           \
    if (pl.bm == BM_ && pl.bn == NWN_ * WN_ && pl.stages == R_ && pl.nwk == NWN_ * WMS_)    \
      return launch<BM_, NWN_, WN_, R_, WMS_, TRUNC>(ep, st);                               \
  }
  VXA_XW_TABLE(VXA_XW)
#undef VXA_XW
  return hipErrorInvalidValue;
}

}  // namespace

bool exact_xw_supported(int bm, int bn, int r, int waves, bool trunc) {
#define VXA_XW_HAS(BM_, NWN_, WN_, R_, WMS_, FOUR_) \
  if (bm == BM_ && bn == NWN_ * WN_ && r == R_ && waves == NWN_ * WMS_ && (trunc || FOUR_)) return true;
  VXA_XW_TABLE(VXA_XW_HAS)
#undef VXA_XW_HAS
  return false;
}

hipError_t launch_exact_xw(const ExactPlan& pl, const ExactParams& ep, bool trunc, hipStream_t st) {
  return trunc ? dispatch<true>(pl, ep, st) : dispatch<false>(pl, ep, st);
}
