// Large-M exact GEMM on packed digits with the K steps split over the waves of a workgroup.
//
// Workgroup tile BM x (NWN * WN), NWN * KG waves (8: two per SIMD). Wave (wn, kg) computes all
// BM rows of its WN columns over its K group's share of the K steps; the KG partial sums of a
// column block meet in LDS after the K loop. Every weight fragment of the workgroup is loaded
// once, by one wave, straight into registers: a 128 x 192 tile loads 40 KiB per K step, where
// waves split along M (each loading the whole weight column block) load 64 KiB.
//
// Round r covers KG * 2 K steps: K group g takes steps (r * KG + g) * 2 + {0, 1} (the launcher
// takes only K splits of whole rounds). The x fragments of a round (KG * 2 steps x BM/16 row
// tiles x 2 digit planes, 1 KiB each in MFMA lane order) go through a two-slot LDS ring filled
// by global_load_lds_dwordx4 (gfx950 direct-to-LDS loads) split over all waves; a wave whose
// share does not divide evenly copies some fragment twice (the same bytes to the same place).
// A wave's weight fragments of its two steps go to two register sets (loaded nontemporal when the
// grid has a single M tile, NTW: then no other workgroup reads them). Every load is issued from
// inline asm and every wait is explicit, in one fixed order per round:
//
//   wait x(r) -> s_barrier -> wait W0(r) -> step 0, the x copies of round r + 1 (into the slot
//   read in round r - 1) issued between its row tiles -> wait W1(r) -> step 1, the W0 loads of
//   round r + 1 issued between its row tiles -> the W1 loads of round r + 1
//
// Each load has most of a round to arrive and no wait covers a younger load. A CU's texture
// path takes about one KiB-wide wave load per 16-18 clocks, so loads issued between MFMAs keep
// every wave issuing MFMAs, where a burst of them stalls the waves behind it. Past the last
// round the loads repeat the last step (into a slot or set no live step reads), so the wait
// counts are constants. The build checks the generated code (check_async_loads.py): no asm
// load's destination registers are touched before a wait covers the load, and
// compiler-generated code never uses M0.
//
// Group g walks the row tiles rotated by g * TM / KG, so that its accumulators 0 .. TM/KG - 1
// hold the row tiles it owns after the K loop, [g * TM / KG, (g + 1) * TM / KG): one copy of
// the reduction and epilogue code serves every group. The K groups reduce in LDS, then the
// owner applies the epilogue to its rows: for 2-byte outputs without a K split or offset terms
// (STAGED) through an LDS tile stored in 16-byte pieces of whole rows, otherwise lane by lane.
// The row and column scales were copied into LDS at the start. Integer addition is exact and
// associative, so the bits are those of every other kernel.

#include "exact_gemm_common.h"

#pragma clang diagnostic ignored "-Winline-asm"

namespace {

typedef __attribute__((address_space(3))) void lds_void_t;

constexpr int staged_row_bytes(int bn) { return bn * 2 + 16; }
constexpr int cmax(int a, int b) { return a > b ? a : b; }
constexpr int kSteps = 2;  // K steps of one K group in a round
// LDS bytes of a tile, one array reused in turn by: the x ring (two rounds), the K-group
// reduction (one owner group's tiles when KG == 2, else every owner), the staged output tile.
constexpr int xk_lds_bytes(int bm, int bn, int kg, int nacc) {
  return cmax(cmax(2 * kg * kSteps * 2 * (bm / 16) * 1024, (kg == 2 ? 1 : kg) * (bm / 16 / kg) * (bn / 16) * nacc * 1024),
              bm * staged_row_bytes(bn));
}

// Epilogue variants: bf16 or fp16 tile staged in LDS (2-byte output, one K split, no offset
// terms), or lane-by-lane stores of any output (fp32, split-K partials, F = 15).
enum XkOut { kOutBf16 = 0, kOutF16 = 1, kOutWide = 2 };

template <int BM, int NWN, int WN, int KG, bool TRUNC, int OUT, bool NTW>
__global__ __launch_bounds__(64 * NWN * KG) void exact_xk_kernel(ExactParams p) {
  constexpr int NWAVE = NWN * KG;
  constexpr int TM = BM / 16;          // 16-row tiles (every wave covers all of them)
  constexpr int TN = WN / 16;          // 16-column tiles of one wave
  constexpr int BN = NWN * WN;         // workgroup tile width
  constexpr int NACC = TRUNC ? 2 : 3;  // accumulators per tile: hh, md (+ ll)
  constexpr int NFX = 2 * TM;          // x fragments of one K step (h and l planes)
  constexpr int NCOPY = KG * kSteps * NFX;  // x fragments of one round
  constexpr int LX = (NCOPY + NWAVE - 1) / NWAVE;
  constexpr int LW = 2 * TN;           // weight fragments of one step of one wave
  constexpr int kSlot = NCOPY * 1024;  // bytes of one round in the ring
  constexpr int TMO = TM / KG;         // row tiles each K group owns after the reduction
  constexpr int kLds = xk_lds_bytes(BM, BN, KG, NACC);
  static_assert(TM % KG == 0, "row tiles split evenly over the K groups");
  static_assert(2 * LW + LX <= 63, "vmcnt limit");
  static_assert((TM & (TM - 1)) == 0, "row tiles rotate by masking");
  static_assert(kLds + (cdiv(BM, 64) + cdiv(BN, 64)) * 256 <= 160 * 1024, "LDS of one CU");
  static_assert(TMO * 16 % 4 == 0, "owned rows");
  __shared__ __attribute__((aligned(1024))) int8_t lds[kLds];
  constexpr int kScaleX = cdiv(BM, 64) * 64, kScaleW = cdiv(BN, 64) * 64;  // whole 64-lane copies
  __shared__ __attribute__((aligned(256))) int32_t scale_x[kScaleX];
  __shared__ __attribute__((aligned(256))) int32_t scale_w[kScaleW];
  int8_t* const ring = lds;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wn = wave % NWN;  // column block of this wave
  const int kg = wave / NWN;  // K group of this wave

  // Logical tile order: M tiles fastest, then N tiles, then K splits; the workgroups that share
  // a weight tile are neighbours and, through the XCD mapping, on one XCD. 32-bit index math
  // (the launcher refuses grids past 2^31 workgroups).
  const uint32_t nbm = (uint32_t)cdiv<int64_t>(p.M, BM);
  const uint32_t nbn = (uint32_t)cdiv<int64_t>(p.N, BN);
  const uint32_t t = (uint32_t)xcd_swizzle((int64_t)blockIdx.y * gridDim.x + blockIdx.x, (int64_t)gridDim.x * gridDim.y);
  const uint32_t bm = t % nbm;
  const uint32_t bnq = t / nbm;
  const uint32_t bn = bnq % nbn;
  const int split = (int)(bnq / nbn);
  const int64_t m0 = (int64_t)bm * BM;
  const int64_t nb0 = (int64_t)bn * BN;  // first column of the workgroup tile
  const int64_t n0 = nb0 + wn * WN;      // first column of this wave
  const int64_t kb = (int64_t)split * p.kch;
  const int64_t ke = min(kb + p.kch, p.kpad);
  const int nk = (int)((ke - kb) >> 6);        // K steps of this split (kch <= 32768: at most 512)
  const int nr = cdiv(nk, KG * kSteps);        // rounds
  const int64_t kt0 = kb >> 6;
  const int64_t last_mt = cdiv<int64_t>(p.M, 16) - 1;
  const int64_t last_nt = cdiv<int64_t>(p.N, 16) - 1;
  const uint32_t voff = lane * 16;  // every load: one contiguous KiB per wave from an SGPR base

  // Row and column scales into LDS (direct-to-LDS dword copies by wave 0, 64 at a time; rows and
  // columns past the matrix and past the tile clamped); they arrive long before the epilogue,
  // behind the loop's waits.
  if (wave == 0) {
    auto copy_scales = [&](const int32_t* src, int64_t first, int64_t last, int32_t* dst) {
      const int32_t* base = src + min(first, last);
      const uint32_t off = (uint32_t)(min(first + lane, last) - min(first, last)) * 4;
      const uint32_t d = (uint32_t)(uintptr_t)(lds_void_t*)dst;
      asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base), "s"(d)
                   : "memory", "m0");
    };
#pragma unroll
    for (int c = 0; c < kScaleX; c += 64) copy_scales(p.sx, m0 + c, p.M - 1, scale_x + c);
#pragma unroll
    for (int c = 0; c < kScaleW; c += 64) copy_scales(p.sw, nb0 + c, p.N - 1, scale_w + c);
  }

  // x fragments this wave copies each round: copy c -> step (c / NFX) of the round (K group
  // c / NFX / 2), fragment c % NFX (plane f / TM, row tile f % TM; tiles past M clamped, their
  // rows are never stored). In LDS the row tiles of group g's steps are rotated by g * TMO, so
  // that group g reads them in its accumulator order at fixed offsets.
  const int8_t* xsrc[LX];
  int xstep[LX], xdst[LX];
#pragma unroll
  for (int i = 0; i < LX; ++i) {
    const int c = (wave + NWAVE * i) % NCOPY;
    const int f = c % NFX, g = c / NFX / kSteps;
    const int64_t tile = min((int64_t)bm * TM + f % TM, last_mt);
    xsrc[i] = p.xh + (tile * p.KT + kt0) * 2048 + (f / TM) * 1024;
    xstep[i] = c / NFX;  // = g * kSteps + s
    xdst[i] = ((c / NFX) * NFX + (f / TM) * TM + ((f % TM - g * TMO) & (TM - 1))) * 1024;
  }
  const int8_t* wsrc[TN];
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) {
    const int64_t tile = min((n0 >> 4) + tn, last_nt);
    wsrc[tn] = p.wh + (tile * p.KT + kt0) * 2048;
  }

  // x copy i of this wave for round `round` into ring slot `slot`
  auto issue_x = [&](int round, int slot, int i) {
    const int step = min(round * KG * kSteps + xstep[i], nk - 1);
    const uint32_t dst = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(lds_void_t*)(ring + slot * kSlot + xdst[i]));
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(xsrc[i] + step * 2048),
                 "s"(dst)
                 : "memory", "m0");
  };
  // Weight fragment f (column tile f / 2, plane f % 2) of step s of round `round` of this wave.
  // Written by the hardware when the load completes: the registers are not read before the
  // explicit wait that covers the load.
  auto issue_w = [&](int round, int s, v4i (&wb)[LW], int f) {
    const int step = min((round * KG + kg) * kSteps + s, nk - 1);
    const int8_t* base = wsrc[f >> 1] + step * 2048 + (f & 1) * 1024;
    if constexpr (NTW)
      asm volatile("global_load_dwordx4 %0, %1, %2 nt" : "=v"(wb[f]) : "v"(voff), "s"(base) : "memory");
    else
      asm volatile("global_load_dwordx4 %0, %1, %2" : "=v"(wb[f]) : "v"(voff), "s"(base) : "memory");
  };

  v4i acc[NACC][TM][TN];
#pragma unroll
  for (int a = 0; a < NACC; ++a)
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) acc[a][tm][tn] = v4i{0, 0, 0, 0};

  // One K step: accumulator row tile t holds the workgroup's row tile (t + kg * TMO) % TM (the
  // ring slot holds them in that order). after_tile(t) issues the loads placed after row tile t.
  auto step_mfmas = [&](const int8_t* stage, const v4i (&wb)[LW], auto&& after_tile) {
#pragma unroll
    for (int t = 0; t < TM; ++t) {
      const int8_t* frag = stage + t * 1024;
      const v4i xh = *reinterpret_cast<const v4i*>(frag);
      const v4i xl = *reinterpret_cast<const v4i*>(frag + TM * 1024);
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) acc[0][t][tn] = mfma_i8(xh, wb[2 * tn], acc[0][t][tn]);
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) acc[1][t][tn] = mfma_i8(xh, wb[2 * tn + 1], acc[1][t][tn]);
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) acc[1][t][tn] = mfma_i8(xl, wb[2 * tn], acc[1][t][tn]);
      if constexpr (!TRUNC) {
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) acc[NACC - 1][t][tn] = mfma_i8(xl, wb[2 * tn + 1], acc[NACC - 1][t][tn]);
      }
      after_tile(t);
    }
  };

  if (nk > 0) {
    constexpr int kPerX = cdiv(LX, TM), kPerW = cdiv(LW, TM);  // loads after each row tile
    v4i w0[LW], w1[LW];
    // queue at the top of round 0 as in every later round: x(0), W0(0), W1(0)
#pragma unroll
    for (int i = 0; i < LX; ++i) issue_x(0, 0, i);
#pragma unroll
    for (int f = 0; f < LW; ++f) issue_w(0, 0, w0, f);
#pragma unroll
    for (int f = 0; f < LW; ++f) issue_w(0, 1, w1, f);
    const int8_t* lds_lane = ring + kg * kSteps * NFX * 1024 + lane * 16;
    for (int r = 0; r < nr; ++r) {
      const int slot = r & 1;
      const int nxt = r + 1 < nr ? r + 1 : nr - 1;
      const int8_t* stage = lds_lane + slot * kSlot;
      // x(r) landed (younger: W0(r), W1(r)); every wave is done with the slot of round r - 1
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(2 * LW) : "memory");
      // W0(r) landed (younger: W1(r))
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(LW) : "memory");
      step_mfmas(stage, w0, [&](int t) {
#pragma unroll
        for (int u = 0; u < kPerX; ++u)
          if (t * kPerX + u < LX) issue_x(nxt, slot ^ 1, t * kPerX + u);
      });
      // W1(r) landed (younger: x(r + 1))
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(LX) : "memory");
      step_mfmas(stage + NFX * 1024, w1, [&](int t) {
#pragma unroll
        for (int u = 0; u < kPerW; ++u)
          if (t * kPerW + u < LW) issue_w(nxt, 0, w0, t * kPerW + u);
      });
#pragma unroll
      for (int f = 0; f < LW; ++f) issue_w(nxt, 1, w1, f);
    }
    // the repeated loads past the last round still target this workgroup's LDS and registers
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  } else {
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  }

  // ---- reduction over the K groups (the ring is free: every wave passed the barrier above).
  // Accumulator row tile t of group g holds the workgroup's row tile (t + g TMO) % TM: tiles
  // t < TMO are the group's own, tile t >= TMO belongs to group (t / TMO + g) % KG.
  if constexpr (KG == 2) {
    // pass q: the group other than q writes its partial sums of group q's rows (its tiles TMO ..
    // TM - 1; block (wn, t, tn, a) of 1 KiB, lane-major), group q adds them to its tiles 0 .. TMO - 1
    auto blk = [&](int t, int tn, int a) { return lds + (((wn * TMO + t) * TN + tn) * NACC + a) * 1024 + lane * 16; };
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      if (kg != q) {
#pragma unroll
        for (int t = 0; t < TMO; ++t)
#pragma unroll
          for (int tn = 0; tn < TN; ++tn)
#pragma unroll
            for (int a = 0; a < NACC; ++a) *reinterpret_cast<v4i*>(blk(t, tn, a)) = acc[a][TMO + t][tn];
      }
      __syncthreads();
      if (kg == q) {
#pragma unroll
        for (int t = 0; t < TMO; ++t)
#pragma unroll
          for (int tn = 0; tn < TN; ++tn)
#pragma unroll
            for (int a = 0; a < NACC; ++a) acc[a][t][tn] += *reinterpret_cast<const v4i*>(blk(t, tn, a));
      }
      __syncthreads();
    }
  } else {
    // every owner at once: each group writes its own tiles' partial sums, the other groups add
    // theirs with LDS atomics (component c of lane l at c * 256 + 4 l: 64 banks per access),
    // each group reads its sums back
    int32_t* red = reinterpret_cast<int32_t*>(lds);
    auto slot = [&](int o, int t, int tn, int a) {
      return red + ((((o * NWN + wn) * TMO + t) * TN + tn) * NACC + a) * 256 + lane;
    };
#pragma unroll
    for (int t = 0; t < TMO; ++t)
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int a = 0; a < NACC; ++a) {
          int32_t* s = slot(kg, t, tn, a);
#pragma unroll
          for (int c = 0; c < 4; ++c) s[c * 64] = acc[a][t][tn][c];
        }
    __syncthreads();
#pragma unroll
    for (int t = TMO; t < TM; ++t) {
      const int o = (t / TMO + kg) % KG;
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int a = 0; a < NACC; ++a) {
          int32_t* s = slot(o, t % TMO, tn, a);
#pragma unroll
          for (int c = 0; c < 4; ++c)
            __hip_atomic_fetch_add(s + c * 64, acc[a][t][tn][c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < TMO; ++t)
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
#pragma unroll
        for (int a = 0; a < NACC; ++a) {
          const int32_t* s = slot(kg, t, tn, a);
#pragma unroll
          for (int c = 0; c < 4; ++c) acc[a][t][tn][c] = s[c * 64];
        }
    __syncthreads();
  }

  // ---- epilogue of the group's own row tiles (accumulator tiles 0 .. TMO - 1)
  const int r16 = lane & 15, kq = lane >> 4;
  const int row0 = kg * TMO * 16 + kq * 4;  // tile row of register 0 of accumulator tile 0
  if constexpr (OUT != kOutWide) {
    constexpr int kRowBytes = staged_row_bytes(BN);
    int32_t swv[TN];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) swv[tn] = scale_w[wn * WN + tn * 16 + r16];
#pragma unroll
    for (int t = 0; t < TMO; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = row0 + t * 16 + r;
        const int32_t sxm = scale_x[row];
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) {
          const float v = exact_epilogue_digits<TRUNC>(acc[0][t][tn][r], acc[1][t][tn][r], acc[NACC - 1][t][tn][r],
                                                       sxm + swv[tn]);
          const uint16_t bits = OUT == kOutBf16 ? f32_to_bf16_rne_finite(v) : __builtin_bit_cast(uint16_t, (_Float16)v);
          *reinterpret_cast<uint16_t*>(lds + row * kRowBytes + (wn * WN + tn * 16 + r16) * 2) = bits;
        }
      }
    __syncthreads();
    constexpr int kPieces = BN / 8;  // 16-byte pieces per row
    const bool whole = reinterpret_cast<uintptr_t>(p.out) % 16 == 0 && p.ldo % 8 == 0;
    for (int i = threadIdx.x; i < BM * kPieces; i += 64 * NWAVE) {
      const int row = i / kPieces, c = i % kPieces;
      const int64_t m = m0 + row, n = nb0 + c * 8;
      if (m >= p.M || n >= p.N) continue;
      const int8_t* src = lds + row * kRowBytes + c * 16;
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
  for (int t = 0; t < TMO; ++t)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = m0 + row0 + t * 16 + r;
        const int64_t n = n0 + tn * 16 + r16;
        if (m < p.M && n < p.N) {
          int64_t tot = ((int64_t)acc[0][t][tn][r] << 16) + ((int64_t)acc[1][t][tn][r] << 8);
          if constexpr (!TRUNC) tot += (int64_t)acc[NACC - 1][t][tn][r];
          if (p.sk > 1) {
            p.ws[((int64_t)split * p.M + m) * p.N + n] = tot;
          } else {
            if (p.offset) tot += offset_terms(p, m, n);
            store_f32_as(p.out, p.out_dtype, m * p.ldo + n,
                         exact_epilogue(tot, scale_x[row0 + t * 16 + r], scale_w[wn * WN + tn * 16 + r16]));
          }
        }
      }
}

template <int BM, int NWN, int WN, int KG, bool TRUNC>
hipError_t launch(const ExactParams& ep, hipStream_t st) {
  constexpr int BN = NWN * WN;
  const int64_t blocks = cdiv<int64_t>(ep.M, BM) * cdiv<int64_t>(ep.N, BN);
  if (blocks * ep.sk > 0x7FFFFFFFLL || ep.sk > 65535) return hipErrorInvalidConfiguration;
  const dim3 grid((unsigned)blocks, (unsigned)ep.sk), block(64 * NWN * KG);
  const bool staged = ep.sk == 1 && ep.out_dtype != VXA_F32 && !ep.offset;
  // One M tile: every weight byte is read by one workgroup, so weights are streamed with
  // nontemporal loads. Several M tiles read the same weight tile close together (XCD swizzle)
  // and should find it in L2.
  const bool ntw = cdiv<int64_t>(ep.M, BM) == 1;
#define VXA_XK_LAUNCH(OUT_)                                                                             \
  if (ntw)                                                                                             \
    hipLaunchKernelGGL((exact_xk_kernel<BM, NWN, WN, KG, TRUNC, OUT_, true>), grid, block, 0, st, ep);  \
  else                                                                                                 \
    hipLaunchKernelGGL((exact_xk_kernel<BM, NWN, WN, KG, TRUNC, OUT_, false>), grid, block, 0, st, ep);
  if (staged && ep.out_dtype == VXA_BF16) {
    VXA_XK_LAUNCH(kOutBf16)
  } else if (staged) {
    VXA_XK_LAUNCH(kOutF16)
  } else {
    VXA_XK_LAUNCH(kOutWide)
  }
#undef VXA_XK_LAUNCH
  return hipGetLastError();
}

// Instantiated (BM, NWN, WN, KG, 4-dot too), 8 waves: cfg (BM, NWN * WN, 64 * KG, 8, 2).
#define VXA_XK_TABLE(X) \
  X(128, 4, 48, 2, 0) X(128, 4, 32, 2, 1) X(64, 2, 48, 4, 1) X(64, 2, 32, 4, 1) X(64, 4, 32, 2, 1) X(64, 4, 48, 2, 1)

template <bool TRUNC>
hipError_t dispatch(const ExactPlan& pl, const ExactParams& ep, hipStream_t st) {
#define VXA_XK(BM_, NWN_, WN_, KG_, FOUR_)                                                               \
  if constexpr (TRUNC || FOUR_) {                                                                       \
    if (pl.bm == BM_ && pl.bn == NWN_ * WN_ && pl.kg == KG_ && pl.stages == 2 && pl.nwk == NWN_ * KG_) \
      return launch<BM_, NWN_, WN_, KG_, TRUNC>(ep, st);                                                \
  }
  VXA_XK_TABLE(VXA_XK)
#undef VXA_XK
  return hipErrorInvalidValue;
}

}  // namespace

bool exact_xk_supported(int bm, int bn, int kg, int r, int waves, bool trunc) {
#define VXA_XK_HAS(BM_, NWN_, WN_, KG_, FOUR_) \
  if (bm == BM_ && bn == NWN_ * WN_ && kg == KG_ && r == 2 && waves == NWN_ * KG_ && (trunc || FOUR_)) return true;
  VXA_XK_TABLE(VXA_XK_HAS)
#undef VXA_XK_HAS
  return false;
}

bool exact_xk_whole_rounds(int kg, int64_t kch, int64_t kpad) {
  const int64_t round = 64 * kSteps * (int64_t)kg;  // K extent of one round
  const int64_t last = kpad - (cdiv<int64_t>(kpad, kch) - 1) * kch;
  return kch % round == 0 && last % round == 0;
}

hipError_t launch_exact_xk(const ExactPlan& pl, const ExactParams& ep, bool trunc, hipStream_t st) {
  return trunc ? dispatch<true>(pl, ep, st) : dispatch<false>(pl, ep, st);
}

