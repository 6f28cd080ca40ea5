// Digitize + exact GEMM in one launch: bf16 x, packed weights, F <= 14, the small-M kernel's
// one-row-tile shapes (16 rows of x per workgroup).
//
// The two-launch path runs the digitize kernel (one workgroup per row) and then the GEMM; at
// decode sizes the second launch and the wait between them are a quarter of the op. Here
// every GEMM workgroup digitizes the x it needs itself:
//   1. the absmax of each of its 16 rows over all of K (16 * K * 2 bytes of L2-resident bf16;
//      one wave per row, each lane's loads batched so a row costs one or two L2 round trips)
//      gives each row's scale (digit_scale, the digitize kernels' own helper);
//   2. in the K loop, a lane reads its 16 bf16 columns of its row straight from x and splits
//      them into the two MFMA digit operands (pack_digit_bytes) in registers;
//   3. MFMAs, wave partials and the epilogue are the small-M kernel's (exact_gemm_sm.hip).
// The digits are the ones the digitize kernel writes, so every output bit is the two-launch
// path's. Lanes of rows past M take zero operands; their results are never stored.

#include "exact_gemm_common.h"

namespace {

struct FusedParams {
  const uint16_t* x;  // bf16 [M, K], row stride ldx elements
  int64_t ldx;
  const int8_t* wp;  // packed weight digits
  const int32_t* cw;  // weight digit sums (F = 15)
  const int32_t* sw;
  void* out;
  int64_t ldo;
  int32_t out_dtype;
  int32_t F;
  int64_t M, N, K, KT;
};

// FEW: M <= 4, one tile of at most 4 rows (decode); its row pass is the only one compiled in.
// OFFSET (F = 15, 4 dots): offset digits, each row's digit sum cx added in the epilogue
// (kernels.py:31-34, 96-97), as in the x-in-registers kernel below.
template <int NT, int NWK, int C, bool TRUNC, bool FEW, bool OFFSET>
__global__ __launch_bounds__(64 * NWK) void exact_fused_kernel(FusedParams p) {
  static_assert(!(OFFSET && TRUNC), "offset digits run 4 dots");
  constexpr int BN = 16 * NT;
  constexpr int RPW = (16 + NWK - 1) / NWK;  // tile rows each wave reduces in the row pass
  constexpr int PB = 8;                      // row-pass loads per lane in flight (full tiles)
  __shared__ unsigned long long red[16 * BN];
  __shared__ float s_scale[16];
  __shared__ int32_t s_sh[16];
  __shared__ float s_max[NWK][4];
  __shared__ uint32_t s_cs[OFFSET ? NWK : 1][16];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r16 = lane & 15;
  const int kq = lane >> 4;
  const int nthr = 64 * NWK;
  const int64_t nbn = cdiv<int64_t>(p.N, BN);
  const int64_t bn = blockIdx.x % nbn;
  const int64_t m0 = (int64_t)(blockIdx.x / nbn) * 16;
  const int64_t n0 = bn * BN;
  const int mrows = (int)min<int64_t>(16, p.M - m0);  // rows of this tile below M

  for (int i = threadIdx.x; i < 16 * BN; i += nthr) red[i] = 0ull;

  // Operand addressing.
  const bool row_ok = r16 < mrows;
  float scale = 0.0f;  // this lane's row scale, set after the row-absmax pass
  const uint16_t* xrow = p.x + (m0 + (row_ok ? r16 : 0)) * p.ldx + kq * 16;
  const int8_t* whp[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int64_t tile = min(bn * NT + nt, cdiv<int64_t>(p.N, 16) - 1);
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
  uint32_t cs = 0;  // this lane's part of its row's digit sum (F = 15; wraps like the digitize kernels)
  auto x_digits = [&](int64_t s, const uint4 (&r)[2], v4i& ah, v4i& al) {
    float v[16];
    const int64_t c0 = s * 64 + kq * 16;
    // columns of this lane's 16 inside K (all 16 but in the chunk K ends in; none past it)
    const int lim = (int)max<int64_t>(min<int64_t>(p.K - c0, 16), 0);
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
      int32_t qv[4];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        qv[b] = (int32_t)(v[4 * q + b] * scale);  // truncation toward zero
        if constexpr (OFFSET) {
          // columns past K keep zero digits and stay out of the sum, as in the digitize kernels:
          // q = 128 is zero offset digits, and the sum adds 256 h + l = q - 128
          qv[b] = 4 * q + b < lim ? qv[b] : 128;
          cs += (uint32_t)qv[b] - 128u;
        }
      }
      pack_digit_bytes<OFFSET>(qv, hw[q], lw[q]);
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
  // 1. Row absmax over all of K, in 8-column chunks (one 16-byte load each); the last K % 8
  // columns of a row are read per element. A tile of up to 4 rows (decode) spreads each row
  // over the whole workgroup and meets in LDS; otherwise each wave takes its own rows
  // (w, w + NWK, ...), its items (row j, chunk c) = j * cpr + c going to the lanes in turn
  // with PB loads per lane in flight.
  const int cpr = (int)(p.K / 8);  // whole chunks per row
  if constexpr (FEW) {
    float amax[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) amax[j] = 0.0f;
    const int items = mrows * cpr;
    for (int base = threadIdx.x; base < items; base += nthr * 4) {
      uint4 u[4];
      int jr[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int it = base + nthr * q;
        jr[q] = -1;
        if (it < items) {
          jr[q] = it / cpr;
          u[q] = *reinterpret_cast<const uint4*>(p.x + (m0 + jr[q]) * p.ldx + (int64_t)(it % cpr) * 8);
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (jr[q] < 0) continue;
        const uint32_t w[4] = {u[q].x, u[q].y, u[q].z, u[q].w};
        float m = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          m = fmaxf(m, fabsf(__uint_as_float(w[e] << 16)));
          m = fmaxf(m, fabsf(__uint_as_float(w[e] & 0xFFFF0000u)));
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (j == jr[q]) amax[j] = fmaxf(amax[j], m);
      }
    }
    for (int it = threadIdx.x; it < mrows * (int)(p.K - (int64_t)cpr * 8); it += nthr) {
      const int tail = (int)(p.K - (int64_t)cpr * 8);
      const int j = it / tail;
      const float v = fabsf(bf16_to_f32(p.x[(m0 + j) * p.ldx + (int64_t)cpr * 8 + it % tail]));
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
        if (jj == j) amax[jj] = fmaxf(amax[jj], v);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) amax[j] = fmaxf(amax[j], shfl_xor_f32(amax[j], m));
      if (lane == 0) s_max[wave][j] = amax[j];
    }
    __syncthreads();
    if (threadIdx.x < mrows) {
      float a = 0.0f;
      for (int w = 0; w < NWK; ++w) a = fmaxf(a, s_max[w][threadIdx.x]);
      int sh;
      s_scale[threadIdx.x] = digit_scale(a, p.F, sh);
      s_sh[threadIdx.x] = sh;
    }
  } else {
    int nrw = 0;  // rows this wave reduces
#pragma unroll
    for (int j = 0; j < RPW; ++j)
      if (wave + NWK * j < mrows) nrw = j + 1;
    float amax[RPW];
#pragma unroll
    for (int j = 0; j < RPW; ++j) amax[j] = 0.0f;
    // this lane's items are lane + 64 t; (row jj, chunk cc) advances without a division
    int jj = 0, cc = lane;
    while (jj < nrw && cc >= cpr) {
      cc -= cpr;
      ++jj;
    }
    while (jj < nrw) {
      uint4 u[PB];
      int jr[PB];
#pragma unroll
      for (int q = 0; q < PB; ++q) {
        jr[q] = -1;
        if (jj < nrw) {
          jr[q] = jj;
          u[q] = *reinterpret_cast<const uint4*>(p.x + (m0 + wave + NWK * jj) * p.ldx + (int64_t)cc * 8);
          cc += 64;
          while (jj < nrw && cc >= cpr) {
            cc -= cpr;
            ++jj;
          }
        }
      }
#pragma unroll
      for (int q = 0; q < PB; ++q) {
        if (jr[q] < 0) continue;
        const uint32_t w[4] = {u[q].x, u[q].y, u[q].z, u[q].w};
        float m = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          m = fmaxf(m, fabsf(__uint_as_float(w[e] << 16)));
          m = fmaxf(m, fabsf(__uint_as_float(w[e] & 0xFFFF0000u)));
        }
#pragma unroll
        for (int j = 0; j < RPW; ++j)
          if (j == jr[q]) amax[j] = fmaxf(amax[j], m);
      }
    }
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
      if (j < nrw) {
        const uint16_t* row = p.x + (m0 + wave + NWK * j) * p.ldx;
        for (int64_t k = (int64_t)cpr * 8 + lane; k < p.K; k += 64) amax[j] = fmaxf(amax[j], fabsf(bf16_to_f32(row[k])));
      }
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) amax[j] = fmaxf(amax[j], shfl_xor_f32(amax[j], m));
      if (lane == 0 && j < nrw) {
        int sh;
        s_scale[wave + NWK * j] = digit_scale(amax[j], p.F, sh);
        s_sh[wave + NWK * j] = sh;
      }
    }
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

  // 3. Wave partials meet in LDS (exact int64 adds), then the epilogue; with offset digits the
  // row sums meet too (the row's 4 lanes, then the waves, all mod 2^32).
  if constexpr (OFFSET) {
    cs += __shfl_xor(cs, 16);
    cs += __shfl_xor(cs, 32);
    if (kq == 0) s_cs[wave][r16] = cs;
  }
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      int64_t cross = (int64_t)md[nt][r];
      if constexpr (kSplitMd) cross += (int64_t)mx[nt][r];
      int64_t tot = ((int64_t)hh[nt][r] << 16) + (cross << 8);
      if constexpr (!TRUNC) tot += (int64_t)ll[nt][r];
      const int m = kq * 4 + r;
      if (m < mrows) atomicAdd(&red[m * BN + nt * 16 + r16], (unsigned long long)tot);
    }
  __syncthreads();
  for (int i = threadIdx.x; i < mrows * BN; i += nthr) {
    const int m = i / BN;
    const int64_t n = n0 + i % BN;
    if (n < p.N) {
      int64_t tot = (int64_t)red[i];
      if constexpr (OFFSET) {  // 128 (cx + cw) + 128^2 K (kernels.py:96-97, 148-151)
        uint32_t cx = 0;
#pragma unroll
        for (int w = 0; w < NWK; ++w) cx += s_cs[w][m];
        tot += 128 * ((int64_t)(int32_t)cx + (int64_t)p.cw[n]) + 128 * 128 * p.K;
      }
      store_f32_as(p.out, p.out_dtype, (m0 + m) * p.ldo + n, exact_epilogue(tot, s_sh[m], p.sw[n]));
    }
  }
}

// The same product with x read once, into registers, in the MFMA operand layout: lane
// (r16, kq) of wave w holds its row's 16 columns of every K step w + NWK * i, i < XS (8 VGPRs
// a step). The row absmax comes from those registers (the 4 lanes of a row in a wave, then
// the waves through LDS), and the K loop converts them, so x costs one read and no second
// round trip before the first MFMA. The first round's weights are issued right after x and
// arrive during the absmax; each later round's weights are issued before the MFMAs of the
// round before it. Needs cdiv(KT, NWK) <= XS (the launcher picks XS). OFFSET (F = 15): offset
// digits, with each row's digit sum cx added in the epilogue (kernels.py:31-34, 96-97).
template <int NT, int NWK, int C, bool TRUNC, int XS, bool OFFSET>
__global__ __launch_bounds__(64 * NWK) void exact_fused_xreg_kernel(FusedParams p) {
  static_assert(XS % C == 0, "rounds of C steps");
  constexpr int BN = 16 * NT;
  constexpr int NR = XS / C;  // rounds
  __shared__ unsigned long long red[16 * BN];
  __shared__ float s_max[NWK][16];
  __shared__ uint32_t s_cs[NWK][16];
  __shared__ float s_scale[16];
  __shared__ int32_t s_sh[16];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r16 = lane & 15;
  const int kq = lane >> 4;
  const int nthr = 64 * NWK;
  const int64_t nbn = cdiv<int64_t>(p.N, BN);
  const int64_t bn = blockIdx.x % nbn;
  const int64_t m0 = (int64_t)(blockIdx.x / nbn) * 16;
  const int64_t n0 = bn * BN;
  const int mrows = (int)min<int64_t>(16, p.M - m0);
  const int64_t nsteps = p.KT;

  for (int i = threadIdx.x; i < 16 * BN; i += nthr) red[i] = 0ull;

  const bool row_ok = r16 < mrows;
  const uint16_t* xrow = p.x + (m0 + (row_ok ? r16 : 0)) * p.ldx + kq * 16;
  const int8_t* whp[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int64_t tile = min(bn * NT + nt, cdiv<int64_t>(p.N, 16) - 1);
    whp[nt] = p.wp + tile * p.KT * 2048 + lane * 16;
  }

  // 1. x of this lane's steps, bf16 pairs as loaded (zeros past K and for rows past M).
  uint32_t xw[XS][8];
#pragma unroll
  for (int i = 0; i < XS; ++i) {
    const int64_t s = wave + (int64_t)NWK * i;
    const int64_t c0 = s * 64 + kq * 16;
    if (row_ok && s < nsteps && c0 + 16 <= p.K) {
      const uint4 a = *reinterpret_cast<const uint4*>(xrow + s * 64);
      const uint4 b = *reinterpret_cast<const uint4*>(xrow + s * 64 + 8);
      xw[i][0] = a.x; xw[i][1] = a.y; xw[i][2] = a.z; xw[i][3] = a.w;
      xw[i][4] = b.x; xw[i][5] = b.y; xw[i][6] = b.z; xw[i][7] = b.w;
    } else if (row_ok && s < nsteps && c0 < p.K) {  // the chunk K ends in
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t lo = c0 + 2 * e < p.K ? xrow[s * 64 + 2 * e] : 0u;
        const uint32_t hi = c0 + 2 * e + 1 < p.K ? xrow[s * 64 + 2 * e + 1] : 0u;
        xw[i][e] = lo | (hi << 16);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) xw[i][e] = 0u;
    }
  }

  // 2. Weights, double-buffered by round; round 0 is issued behind x.
  v4i wh[2][C][NT], wl[2][C][NT];
  auto load_round = [&](int r, int buf) {
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int64_t s = wave + (int64_t)NWK * (r * C + c);
      if (s < nsteps) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          wh[buf][c][nt] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(whp[nt] + s * 2048));
          wl[buf][c][nt] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(whp[nt] + s * 2048 + 1024));
        }
      }
    }
  };
  load_round(0, 0);

  // 3. Row absmax over all of K: this lane's values, the row's 4 lanes in the wave, the waves.
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < XS; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      m = fmaxf(m, fabsf(__uint_as_float(xw[i][e] << 16)));
      m = fmaxf(m, fabsf(__uint_as_float(xw[i][e] & 0xFFFF0000u)));
    }
  m = fmaxf(m, shfl_xor_f32(m, 16));
  m = fmaxf(m, shfl_xor_f32(m, 32));
  if (kq == 0) s_max[wave][r16] = m;
  __syncthreads();
  if (threadIdx.x < 16) {
    float a = 0.0f;
#pragma unroll
    for (int w = 0; w < NWK; ++w) a = fmaxf(a, s_max[w][threadIdx.x]);
    int sh;
    s_scale[threadIdx.x] = digit_scale(a, p.F, sh);
    s_sh[threadIdx.x] = sh;
  }
  __syncthreads();
  const float scale = s_scale[r16];  // rows past M: their results are never stored

  // 4. K loop.
  // the cross products in two accumulators, except NT = 2 with 16 waves (128 VGPRs a lane)
  constexpr bool kSplitMd = NT == 1 || (NT == 2 && NWK < 16);
  v4i hh[NT], md[NT], mx[NT], ll[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    hh[nt] = v4i{0, 0, 0, 0};
    md[nt] = v4i{0, 0, 0, 0};
    mx[nt] = v4i{0, 0, 0, 0};
    ll[nt] = v4i{0, 0, 0, 0};
  }
  uint32_t cs = 0;  // this lane's part of its row's digit sum (F = 15; wraps like the digitize kernels)
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    if (wave + (int64_t)NWK * r * C >= nsteps) break;  // this wave has no steps left
    if (r + 1 < NR) load_round(r + 1, (r + 1) & 1);
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int i = r * C + c;
      const int64_t c0 = (wave + (int64_t)NWK * i) * 64 + kq * 16;  // this lane's first column
      if (wave + (int64_t)NWK * i < nsteps) {
        // columns of this lane's 16 inside K (all 16 but in the chunk K ends in)
        const int lim = (int)min<int64_t>(p.K - c0, 16);
        uint32_t hw[4], lw[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          int32_t qv[4];
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            const uint32_t w = xw[i][(4 * q + b) >> 1];
            const float v = __uint_as_float(((4 * q + b) & 1) ? (w & 0xFFFF0000u) : (w << 16));
            qv[b] = (int32_t)(v * scale);  // truncation toward zero
            if constexpr (OFFSET) {
              // columns past K keep zero digits: the weights' padding digits are zero too, and
              // the digitize kernels leave those columns out of the sum (a select, not a branch;
              // q = 128 is zero offset digits, and the sum adds 256 h + l = q - 128)
              qv[b] = 4 * q + b < lim ? qv[b] : 128;
              cs += (uint32_t)qv[b] - 128u;
            }
          }
          pack_digit_bytes<OFFSET>(qv, hw[q], lw[q]);
        }
        const v4i ah = v4i{(int)hw[0], (int)hw[1], (int)hw[2], (int)hw[3]};
        const v4i al = v4i{(int)lw[0], (int)lw[1], (int)lw[2], (int)lw[3]};
        const int buf = r & 1;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) hh[nt] = mfma_i8(ah, wh[buf][c][nt], hh[nt]);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) md[nt] = mfma_i8(ah, wl[buf][c][nt], md[nt]);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          if constexpr (kSplitMd) mx[nt] = mfma_i8(al, wh[buf][c][nt], mx[nt]);
          else md[nt] = mfma_i8(al, wh[buf][c][nt], md[nt]);
        }
        if constexpr (!TRUNC) {
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) ll[nt] = mfma_i8(al, wl[buf][c][nt], ll[nt]);
        }
      }
    }
  }

  // 5. Wave partials meet in LDS (exact int64 adds), then the epilogue; with offset digits the
  // row sums meet too (the row's 4 lanes, then the waves, all mod 2^32).
  if constexpr (OFFSET) {
    cs += __shfl_xor(cs, 16);
    cs += __shfl_xor(cs, 32);
    if (kq == 0) s_cs[wave][r16] = cs;
  }
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      int64_t cross = (int64_t)md[nt][r];
      if constexpr (kSplitMd) cross += (int64_t)mx[nt][r];
      int64_t tot = ((int64_t)hh[nt][r] << 16) + (cross << 8);
      if constexpr (!TRUNC) tot += (int64_t)ll[nt][r];
      const int mr = kq * 4 + r;
      if (mr < mrows) atomicAdd(&red[mr * BN + nt * 16 + r16], (unsigned long long)tot);
    }
  __syncthreads();
  for (int i = threadIdx.x; i < mrows * BN; i += nthr) {
    const int mr = i / BN;
    const int64_t n = n0 + i % BN;
    if (n < p.N) {
      int64_t tot = (int64_t)red[i];
      if constexpr (OFFSET) {  // 128 (cx + cw) + 128^2 K (kernels.py:96-97, 148-151)
        uint32_t cx = 0;
#pragma unroll
        for (int w = 0; w < NWK; ++w) cx += s_cs[w][mr];
        tot += 128 * ((int64_t)(int32_t)cx + (int64_t)p.cw[n]) + 128 * 128 * p.K;
      }
      store_f32_as(p.out, p.out_dtype, (m0 + mr) * p.ldo + n, exact_epilogue(tot, s_sh[mr], p.sw[n]));
    }
  }
}

// Instantiations of the x-in-registers kernel that compile without scratch (gfx950 -O3):
// 4 steps a wave with at most 8 waves (at most 212 VGPRs of their 256), or with 16 waves and
// one column tile, or two with 3 dots (at most 127 of their 128); 8 steps with at most 8
// waves and NT * C <= 2, or four tiles with 3 dots (at most 252). F = 15 (offset digits,
// 4 dots) drops the shapes whose digit sum would spill. Other shapes and longer K take the
// row-pass kernel.
template <int NT, int NWK, int C, int XS, bool TRUNC, bool OFFSET>
constexpr bool xreg_fits() {
  // F = 15 runs 4 dots, and its digit sum needs a few more registers
  if (OFFSET && (TRUNC || (NWK == 16 && C > 1) || NT * C > 4)) return false;
  if (XS == 4) return NWK <= 8 || NT == 1 || (NT == 2 && C == 1 && TRUNC);
  return XS == 8 && NWK <= 8 && (NT * C <= 2 || (NT == 4 && C == 1 && TRUNC && !OFFSET));
}

// Row-pass shapes whose offset-digit (F = 15) instantiation compiles without scratch (gfx950
// -O3): with 16 waves (128 VGPRs a lane) at most two column tiles times steps per round.
template <int NT, int NWK, int C>
constexpr bool rowpass_offset_fits() {
  return NWK < 16 || NT * C < 4;
}

// Compute units of the current device (cached per device; 0 when the query fails).
int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cus[dev] = n;
  }
  return cus[dev];
}

template <int NT, int NWK, int C, bool TRUNC>
hipError_t launch(const FusedParams& fp, hipStream_t st) {
  const int64_t blocks = cdiv<int64_t>(fp.M, 16) * cdiv<int64_t>(fp.N, 16 * NT);
  if (blocks > 0x7FFFFFFFLL) return hipErrorInvalidConfiguration;
  // x in registers when this wave's steps fit an instantiated XS and the grid is at most one
  // workgroup per CU. Its registers (100-250 VGPRs) leave room for one workgroup a CU; with
  // more workgroups than CUs the row-pass kernel (about 75 VGPRs) runs several per CU, which
  // hides more latency than the saved x read gains (measured on gate_up and the lm_head).
  const int64_t per_wave = blocks <= device_cus() ? cdiv<int64_t>(fp.KT, NWK) : INT64_MAX;
#define VXA_XREG(XS_, OFF_)                                                                                      \
  if constexpr (XS_ % C == 0 && xreg_fits<NT, NWK, C, XS_, TRUNC, OFF_>()) {                                \
    if (per_wave <= XS_ && (fp.F == 15) == OFF_) {                                                            \
      hipLaunchKernelGGL((exact_fused_xreg_kernel<NT, NWK, C, TRUNC, XS_, OFF_>), dim3((unsigned)blocks),     \
                         dim3(64 * NWK), 0, st, fp);                                                        \
      return hipGetLastError();                                                                               \
    }                                                                                                       \
  }
  VXA_XREG(4, false) VXA_XREG(8, false) VXA_XREG(4, true) VXA_XREG(8, true)
#undef VXA_XREG
  // the row-pass kernel: balanced digits, or offset digits (F = 15) with 4 dots
#define VXA_ROWPASS(FEW_, OFF_)                                                                                   \
  if ((fp.M <= 4) == FEW_ && (fp.F == 15) == OFF_) {                                                             \
    hipLaunchKernelGGL((exact_fused_kernel<NT, NWK, C, TRUNC, FEW_, OFF_>), dim3((unsigned)blocks), dim3(64 * NWK), \
                       0, st, fp);                                                                               \
    return hipGetLastError();                                                                                    \
  }
  VXA_ROWPASS(true, false) VXA_ROWPASS(false, false)
  if constexpr (!TRUNC && rowpass_offset_fits<NT, NWK, C>()) {
    VXA_ROWPASS(true, true) VXA_ROWPASS(false, true)
  }
#undef VXA_ROWPASS
  return hipErrorInvalidValue;  // offset digits with 3 dots, or a shape whose digit sum would spill
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

hipError_t launch_exact_fused(const ExactPlan& pl, const void* x, int64_t ldx, const int8_t* wp, const int32_t* cw,
                              const int32_t* sw, void* out, int out_dtype, int64_t ldo, int64_t m, int64_t n,
                              int64_t k, int f, bool trunc, hipStream_t st) {
  if (pl.family != kFamilySmall || pl.mt != 1 || pl.sk != 1) return hipErrorInvalidValue;
  FusedParams fp;
  fp.x = reinterpret_cast<const uint16_t*>(x);
  fp.ldx = ldx;
  fp.wp = wp;
  fp.cw = cw;
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
