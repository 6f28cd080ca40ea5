// Large-M exact GEMM (MFMA-bound): a multi-stage LDS ring fed by direct-to-LDS loads.
//
// Workgroup tile BM x BN, 4 waves in a 2 x 2 arrangement (wave tile BM/2 x BN/2), one K
// split. The ring holds S stages of one 64-wide K step each; a stage is a set of
// "fragments", 1 KiB each: 16 rows x 64 bytes of one digit plane, stored in MFMA lane order
// (lane l's 16 bytes at offset 16*l: row l & 15, bytes 16*(l >> 4)..+16). Each wave issues
// its share of a stage's fragments as global_load_lds_dwordx4 (gfx950), which land in LDS
// without passing through VGPRs, so S-1 stages stay in flight while one is consumed.
// Fragments are read back with one conflict-free ds_read_b128 each.
//
// Synchronisation per K step: wait until this wave's loads of the step have landed (vmcnt),
// barrier (every wave's loads landed), read + MFMA, then wait for the reads (lgkmcnt) and
// barrier again before the slot is refilled. Both waits sit in the same asm statement as
// their barrier with a memory clobber, so no LDS access moves across a barrier.

#include "exact_gemm_common.h"

namespace {

typedef __attribute__((address_space(3))) void lds_void_t;

template <int BM, int BN, int S, bool TRUNC, bool PACKED>
__global__ __launch_bounds__(256) void exact_lds_kernel(ExactParams p) {
  constexpr int64_t kStep = PACKED ? 2048 : 64;  // bytes between consecutive K steps of one fragment
  constexpr int TM = BM / 32;  // 16x16 MFMA tiles per wave along M
  constexpr int TN = BN / 32;  // ... along N
  constexpr int FX = BM / 16;  // fragments per digit plane of x per stage
  constexpr int FW = BN / 16;  // ... of w
  constexpr int NF = 2 * (FX + FW);
  constexpr int LPW = NF / 4;  // fragments each wave loads per stage
  static_assert(NF % 4 == 0, "fragments split evenly over the 4 waves");
  static_assert((S - 1) * LPW <= 63, "vmcnt limit");
  __shared__ __attribute__((aligned(1024))) int8_t ring[S * NF * 1024];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int wm = wave & 1, wn = wave >> 1;
  const int r16 = lane & 15;
  const int kq = lane >> 4;

  const int64_t nbn = cdiv<int64_t>(p.N, BN);
  const int64_t bn = blockIdx.x % nbn;
  const int64_t bm = blockIdx.x / nbn;
  const int64_t m0 = bm * BM;
  const int64_t n0 = bn * BN;
  const int64_t kb = (int64_t)blockIdx.y * p.kch;
  const int64_t ke = min(kb + p.kch, PACKED ? p.kpad : p.K);
  const int64_t nk = (ke - kb) >> 6;

  // Global source of each fragment this wave loads (rows clamped into the matrices). With a
  // single M tile every weight byte is read by one workgroup only, so weight fragments are
  // streamed with nontemporal loads; x fragments, which every N tile reads, keep the default
  // policy so that they stay in L2.
  const bool stream_w = cdiv<int64_t>(p.M, BM) == 1;
  const int8_t* src[LPW];
  int dst[LPW];
  bool nt[LPW];
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    const int f = wave + 4 * i;
    nt[i] = stream_w && f >= 2 * FX;
    if constexpr (PACKED) {
      // packed: fragment (tile, kt, plane) is 1 KiB of contiguous memory in lane order
      if (f < 2 * FX) {
        const int64_t tile = min(bm * FX + f % FX, cdiv<int64_t>(p.M, 16) - 1);
        src[i] = p.xh + (tile * p.KT + (kb >> 6)) * 2048 + (f < FX ? 0 : 1024) + lane * 16;
      } else {
        const int64_t tile = min(bn * FW + (f - 2 * FX) % FW, cdiv<int64_t>(p.N, 16) - 1);
        src[i] = p.wh + (tile * p.KT + (kb >> 6)) * 2048 + (f < 2 * FX + FW ? 0 : 1024) + lane * 16;
      }
    } else {
      const int8_t* base;
      if (f < 2 * FX) {
        const int mt = f % FX;
        const int64_t m = min(m0 + mt * 16 + r16, p.M - 1);
        base = (f < FX ? p.xh : p.xl) + m * p.ldx;
      } else {
        const int nt = (f - 2 * FX) % FW;
        const int64_t n = min(n0 + nt * 16 + r16, p.N - 1);
        base = (f < 2 * FX + FW ? p.wh : p.wl) + n * p.ldw;
      }
      src[i] = base + kb + kq * 16;
    }
    dst[i] = f * 1024;
  }

  auto issue = [&](int64_t step, int slot) {
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      void* g = (void*)(src[i] + step * kStep);
      lds_void_t* l = (lds_void_t*)(ring + slot * NF * 1024 + dst[i]);
      if (nt[i])
        __builtin_amdgcn_global_load_lds(g, l, 16, 0, 2);  // cache policy: nt
      else
        __builtin_amdgcn_global_load_lds(g, l, 16, 0, 0);
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

#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    if (s < nk) issue(s, s);

  for (int64_t kk = 0; kk < nk; ++kk) {
    if (kk + S - 1 < nk) {
      issue(kk + S - 1, (int)((kk + S - 1) % S));
      asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"((S - 1) * LPW) : "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    }
    const int8_t* slot = ring + (int)(kk % S) * NF * 1024 + lane * 16;
    v4i ah[TM], al[TM], bh[TN], bl[TN];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      ah[tm] = *reinterpret_cast<const v4i*>(slot + (wm * TM + tm) * 1024);
      al[tm] = *reinterpret_cast<const v4i*>(slot + (FX + wm * TM + tm) * 1024);
    }
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      bh[tn] = *reinterpret_cast<const v4i*>(slot + (2 * FX + wn * TN + tn) * 1024);
      bl[tn] = *reinterpret_cast<const v4i*>(slot + (2 * FX + FW + wn * TN + tn) * 1024);
    }
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        hh[tm][tn] = mfma_i8(ah[tm], bh[tn], hh[tm][tn]);
        md[tm][tn] = mfma_i8(ah[tm], bl[tn], md[tm][tn]);
        md[tm][tn] = mfma_i8(al[tm], bh[tn], md[tm][tn]);
        if constexpr (!TRUNC) ll[tm][tn] = mfma_i8(al[tm], bl[tn], ll[tm][tn]);
      }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  }

  // Epilogue from registers: register r of lane holds C[4*(lane>>4) + r][lane & 15].
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = m0 + wm * (BM / 2) + tm * 16 + kq * 4 + r;
        const int64_t n = n0 + wn * (BN / 2) + tn * 16 + r16;
        if (m < p.M && n < p.N) {
          int64_t tot = ((int64_t)hh[tm][tn][r] << 16) + ((int64_t)md[tm][tn][r] << 8);
          if constexpr (!TRUNC) tot += (int64_t)ll[tm][tn][r];
          exact_store(p, blockIdx.y, m, n, tot);
        }
      }
}

template <int BM, int BN, int S, bool TRUNC, bool PACKED>
hipError_t launch(const ExactParams& ep, hipStream_t st) {
  const int64_t blocks = cdiv<int64_t>(ep.M, BM) * cdiv<int64_t>(ep.N, BN);
  if (blocks > 0x7FFFFFFFLL || ep.sk > 65535) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((exact_lds_kernel<BM, BN, S, TRUNC, PACKED>), dim3((unsigned)blocks, (unsigned)ep.sk), dim3(256), 0, st,
                     ep);
  return hipGetLastError();
}

template <bool TRUNC, bool PACKED>
hipError_t dispatch(const ExactPlan& pl, const ExactParams& ep, hipStream_t st) {
#define VXA_LDS(BM_, BN_, S_) \
  if (pl.bm == BM_ && pl.bn == BN_ && pl.stages == S_) return launch<BM_, BN_, S_, TRUNC, PACKED>(ep, st);
  VXA_LDS(64, 64, 2) VXA_LDS(64, 64, 4) VXA_LDS(64, 64, 8)
  VXA_LDS(128, 64, 2) VXA_LDS(128, 64, 4) VXA_LDS(128, 64, 6)
  VXA_LDS(64, 128, 2) VXA_LDS(64, 128, 4) VXA_LDS(64, 128, 6)
  VXA_LDS(128, 128, 2) VXA_LDS(128, 128, 3) VXA_LDS(128, 128, 4)
#undef VXA_LDS
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_exact_lds(const ExactPlan& pl, const ExactParams& ep, bool trunc, bool packed, hipStream_t st) {
  if (packed) return trunc ? dispatch<true, true>(pl, ep, st) : dispatch<false, true>(pl, ep, st);
  return trunc ? dispatch<true, false>(pl, ep, st) : dispatch<false, false>(pl, ep, st);
}
