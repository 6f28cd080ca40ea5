// Small-M exact GEMM (decode batch sizes, HBM-bound): weight digits stream from HBM straight
// into MFMA operand registers.
//
// Workgroup = (16*MT) x (16*NT) output block and one K split; its NWK waves take the
// 64-wide K steps of the split in turn (wave w: steps w, w+NWK, ...), C steps at a time,
// issuing every load of a chunk before its MFMAs so each wave keeps C*(MT+NT)*2 16-byte
// loads in flight. Lane (r16 = lane & 15, kq = lane >> 4) reads bytes [16kq, 16kq+16) of
// row r16 in each step: the four lanes of a row cover 64 contiguous bytes. A (x) and B (w)
// fragments use the same K assignment, so the MFMA's internal K order is irrelevant to the
// integer dot product. Wave partials meet in an LDS int64 tile through ds_add_u64 (exact,
// order-free); the whole workgroup then applies the epilogue with coalesced stores.

#include "exact_gemm_common.h"

namespace {

template <int MT, int NT, int NWK, int C, bool TRUNC, bool PACKED>
__global__ __launch_bounds__(64 * NWK) void exact_sm_kernel(ExactParams p) {
  constexpr int64_t kStep = PACKED ? 2048 : 64;  // bytes between consecutive K steps of one operand
  constexpr int BM = 16 * MT;
  constexpr int BN = 16 * NT;
  __shared__ unsigned long long red[BM * BN];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r16 = lane & 15;
  const int kq = lane >> 4;

  const int64_t nbn = cdiv<int64_t>(p.N, BN);
  const int64_t bn = blockIdx.x % nbn;
  const int64_t bm = blockIdx.x / nbn;
  const int64_t m0 = bm * BM;
  const int64_t n0 = bn * BN;
  const int64_t kb = (int64_t)blockIdx.y * p.kch;
  const int64_t ke = min(kb + p.kch, PACKED ? p.kpad : p.K);

  for (int i = threadIdx.x; i < BM * BN; i += 64 * NWK) red[i] = 0ull;

  // Row pointers clamped into the matrices: out-of-range rows read valid memory and their
  // results are never stored.
  // (packed: row tiles clamped to the last one; fragments of a K step are 1 KiB apart)
  const int8_t* xhp[MT];
  const int8_t* xlp[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    if constexpr (PACKED) {
      // Lanes of rows past M (zero padding of the last tile, or a clamped tile) read the
      // fragment's first 16 bytes instead, which row 0's lanes fetch anyway: at M = 1 that
      // halves the x bytes moved per fragment. Their results are never stored.
      const int64_t tile = min(bm * MT + mt, cdiv<int64_t>(p.M, 16) - 1);
      const bool row_ok = m0 + mt * 16 + r16 < p.M;
      xhp[mt] = p.xh + (tile * p.KT + (kb >> 6)) * 2048 + (row_ok ? lane * 16 : 0);
      xlp[mt] = xhp[mt] + 1024;
    } else {
      const int64_t m = min(m0 + mt * 16 + r16, p.M - 1);
      xhp[mt] = p.xh + m * p.ldx + kb + kq * 16;
      xlp[mt] = p.xl + m * p.ldx + kb + kq * 16;
    }
  }
  const int8_t* whp[NT];
  const int8_t* wlp[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    if constexpr (PACKED) {
      const int64_t tile = min(bn * NT + nt, cdiv<int64_t>(p.N, 16) - 1);
      whp[nt] = p.wh + (tile * p.KT + (kb >> 6)) * 2048 + lane * 16;
      wlp[nt] = whp[nt] + 1024;
    } else {
      const int64_t n = min(n0 + nt * 16 + r16, p.N - 1);
      whp[nt] = p.wh + n * p.ldw + kb + kq * 16;
      wlp[nt] = p.wl + n * p.ldw + kb + kq * 16;
    }
  }

  // With one or two tiles the two cross terms get accumulators of their own (mx for xl*wh),
  // so consecutive MFMAs never depend on each other; with more tiles one accumulator each,
  // updated in passes over all tiles.
  constexpr bool kSplitMd = MT * NT <= 2;
  v4i hh[MT][NT], md[MT][NT], mx[MT][NT], ll[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      hh[mt][nt] = v4i{0, 0, 0, 0};
      md[mt][nt] = v4i{0, 0, 0, 0};
      mx[mt][nt] = v4i{0, 0, 0, 0};
      ll[mt][nt] = v4i{0, 0, 0, 0};
    }

  // One M tile covering all rows reads each weight fragment once: stream it (non-temporal).
  const bool stream_w = cdiv<int64_t>(p.M, BM) == 1;
  const int64_t nsteps = (ke - kb) >> 6;
  for (int64_t s0 = wave; s0 < nsteps; s0 += (int64_t)NWK * C) {
    v4i ah[C][MT], al[C][MT], bh[C][NT], bl[C][NT];
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int64_t s = s0 + (int64_t)c * NWK;
      if (s < nsteps) {
        const int64_t off = s * kStep;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          if (stream_w) {
            bh[c][nt] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(whp[nt] + off));
            bl[c][nt] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wlp[nt] + off));
          } else {
            bh[c][nt] = *reinterpret_cast<const v4i*>(whp[nt] + off);
            bl[c][nt] = *reinterpret_cast<const v4i*>(wlp[nt] + off);
          }
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          ah[c][mt] = *reinterpret_cast<const v4i*>(xhp[mt] + off);
          al[c][mt] = *reinterpret_cast<const v4i*>(xlp[mt] + off);
        }
      }
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
      if (s0 + (int64_t)c * NWK < nsteps) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) hh[mt][nt] = mfma_i8(ah[c][mt], bh[c][nt], hh[mt][nt]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) md[mt][nt] = mfma_i8(ah[c][mt], bl[c][nt], md[mt][nt]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            if constexpr (kSplitMd) mx[mt][nt] = mfma_i8(al[c][mt], bh[c][nt], mx[mt][nt]);
            else md[mt][nt] = mfma_i8(al[c][mt], bh[c][nt], md[mt][nt]);
          }
        if constexpr (!TRUNC) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) ll[mt][nt] = mfma_i8(al[c][mt], bl[c][nt], ll[mt][nt]);
        }
      }
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
        int64_t cross = (int64_t)md[mt][nt][r];
        if constexpr (kSplitMd) cross += (int64_t)mx[mt][nt][r];
        int64_t tot = ((int64_t)hh[mt][nt][r] << 16) + (cross << 8);
        if constexpr (!TRUNC) tot += (int64_t)ll[mt][nt][r];
        if (NWK == 1) {
          red[(mt * 16 + kq * 4 + r) * BN + nt * 16 + r16] = (unsigned long long)tot;
        } else {
          atomicAdd(&red[(mt * 16 + kq * 4 + r) * BN + nt * 16 + r16], (unsigned long long)tot);
        }
      }
  __syncthreads();

  for (int i = threadIdx.x; i < BM * BN; i += 64 * NWK) {
    const int64_t m = m0 + i / BN, n = n0 + i % BN;
    if (m < p.M && n < p.N) exact_store(p, blockIdx.y, m, n, (int64_t)red[i]);
  }
}

template <int MT, int NT, int NWK, int C, bool TRUNC, bool PACKED>
hipError_t launch(const ExactParams& ep, hipStream_t st) {
  const int64_t blocks = cdiv<int64_t>(ep.M, 16 * MT) * cdiv<int64_t>(ep.N, 16 * NT);
  if (blocks > 0x7FFFFFFFLL || ep.sk > 65535) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((exact_sm_kernel<MT, NT, NWK, C, TRUNC, PACKED>), dim3((unsigned)blocks, (unsigned)ep.sk),
                     dim3(64 * NWK), 0, st, ep);
  return hipGetLastError();
}

// (MT, NT, C, NWK) instantiations whose registers fit without spilling: 16 waves cap a
// wave at 128 VGPRs, so only the smallest footprints take 16.
#define VXA_SM_TABLE \
  VXA_SM(1, 1, 1, 4) VXA_SM(1, 1, 1, 8) VXA_SM(1, 1, 1, 16) \
  VXA_SM(1, 1, 2, 4) VXA_SM(1, 1, 2, 8) VXA_SM(1, 1, 2, 16) \
  VXA_SM(1, 1, 4, 4) VXA_SM(1, 1, 4, 8) VXA_SM(1, 1, 4, 16) \
  VXA_SM(1, 2, 1, 4) VXA_SM(1, 2, 1, 8) VXA_SM(1, 2, 1, 16) \
  VXA_SM(1, 2, 2, 4) VXA_SM(1, 2, 2, 8) VXA_SM(1, 2, 2, 16) \
  VXA_SM(1, 2, 4, 4) VXA_SM(1, 2, 4, 8) \
  VXA_SM(1, 4, 1, 4) VXA_SM(1, 4, 1, 8) VXA_SM(1, 4, 1, 16) \
  VXA_SM(1, 4, 2, 4) VXA_SM(1, 4, 2, 8) \
  VXA_SM(2, 1, 1, 4) VXA_SM(2, 1, 1, 8) VXA_SM(2, 1, 1, 16) \
  VXA_SM(2, 1, 2, 4) VXA_SM(2, 1, 2, 8) \
  VXA_SM(2, 2, 1, 4) VXA_SM(2, 2, 1, 8) VXA_SM(2, 2, 1, 16) \
  VXA_SM(2, 2, 2, 4) VXA_SM(2, 2, 2, 8) \
  VXA_SM(2, 4, 1, 4) VXA_SM(2, 4, 1, 8) \
  VXA_SM(4, 1, 1, 4) VXA_SM(4, 1, 1, 8) \
  VXA_SM(4, 1, 2, 4) VXA_SM(4, 1, 2, 8) \
  VXA_SM(4, 2, 1, 4) VXA_SM(4, 2, 1, 8) \
  VXA_SM(4, 4, 1, 4)

template <bool TRUNC, bool PACKED>
hipError_t dispatch(const ExactPlan& pl, const ExactParams& ep, hipStream_t st) {
#define VXA_SM(MT_, NT_, C_, NWK_)                                \
  if (pl.mt == MT_ && pl.nt == NT_ && pl.chunk == C_ && pl.nwk == NWK_) \
    return launch<MT_, NT_, NWK_, C_, TRUNC, PACKED>(ep, st);
  VXA_SM_TABLE
#undef VXA_SM
  return hipErrorInvalidValue;
}

}  // namespace

bool exact_small_supported(int mt, int nt, int chunk, int nwk) {
#define VXA_SM(MT_, NT_, C_, NWK_) \
  if (mt == MT_ && nt == NT_ && chunk == C_ && nwk == NWK_) return true;
  VXA_SM_TABLE
#undef VXA_SM
  return false;
}


hipError_t launch_exact_small(const ExactPlan& pl, const ExactParams& ep, bool trunc, bool packed, hipStream_t st) {
  if (packed) return trunc ? dispatch<true, true>(pl, ep, st) : dispatch<false, true>(pl, ep, st);
  return trunc ? dispatch<true, false>(pl, ep, st) : dispatch<false, false>(pl, ep, st);
}
