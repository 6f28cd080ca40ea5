// Paged decode attention with a fixed reduction order (gfx950).
//
// Behaviour follows paged_attn.py:21-114: one query token per request, GQA groups of
// G = H / KV query heads per KV head, keys cut into fixed segments of `split` keys whose
// count NS = cdiv(max_len, split) is fixed by the model length, segment partials
// (m, l, acc) merged in segment order. The floating-point order depends only on the
// request's own length and the constants (split, blk, waves): never on the batch, on the
// other requests, or on where the pages sit in memory.
//
// Kernel shape (MI355X-first, not a translation of the Triton kernel):
//  * workgroup = (request b, KV head g, segment s); NW waves split the segment's 16-key
//    tiles in a fixed interleave and meet in LDS through a fixed-order merge;
//  * S = K q^T on bf16 matrix cores (v_mfma_f32_16x16x32_bf16): rows are 16 keys of a tile,
//    columns the G query heads of the group (bf16 x bf16 products are exact in fp32);
//  * online softmax in base 2 on the hardware v_exp_f32, state per head kept in fp32;
//  * P V on the vector ALU in fp32: each lane owns D/16 output dims for a quarter of the
//    tile's keys, p arrives by ds_bpermute, V is read as 16-byte rows. fp32 p times bf16 v
//    keeps all 24 bits of p, which is what the reference's hi/lo bf16 split of p
//    (paged_attn.py:63-65) approximates with 2 x 8 bits on bf16 tensor cores.
//  * K and V are read with nontemporal loads: every cache byte is read once per step, and on
//    gfx950 a stream of permuted 8 KiB pages reads at ~6.6 TB/s that way against ~5.8 TB/s
//    with the default cache policy (same pages, same lanes; the load policy is all that
//    differs).
// Arithmetic is compiled with -ffp-contract=off; every fused multiply-add is written
// explicitly, so the order is the one in the source.

#include <algorithm>

#include "common.h"

namespace {

struct PagedParams {
  const uint16_t* q;
  int64_t sqt, sqh;
  const uint16_t* kc;
  int64_t skb, skp, skh;
  const uint16_t* vc;
  int64_t svb, svp, svh;
  const int32_t* bt;
  int64_t sbt;
  const int32_t* sl;
  float scale_log2;  // softmax scale * log2(e)
  int32_t split;     // keys per segment (multiple of 16)
  int32_t ns;        // segments per request in the grid (the caller's length bound may trim it)
  int32_t ns_model;  // segments the model's maximum length fixes: NS = cdiv(max_len, split)
  int32_t H, KV;
  int32_t bs;        // page size (tokens per block)
  int32_t bs_shift;  // log2(bs) when bs is a power of two, else -1
  int64_t n;
  const int32_t* n_live;  // device count of requests to compute (<= n), or null for all n
  float* mp;  // [n][H][ns]
  float* lp;  // [n][H][ns]
  float* ap;  // [n][H][ns][D]
  void* out;
  int64_t sot, soh;
  int32_t out_dtype;
};

constexpr float kNegInf = -__builtin_huge_valf();

__device__ inline float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// Fixed-order merge of a softmax state (m, l, a) with another (ms, ls, as_)
// (paged_attn.py:84-93, base-2 logits). A state with m == -inf contributes exactly 0.
__device__ inline void merge_state(float& m, float& l, float& a, float ms, float ls, float as_) {
  const float mn = fmaxf(m, ms);
  const float c_old = (m == kNegInf) ? 0.0f : exp2_hw(m - mn);
  const float c_new = (ms == kNegInf) ? 0.0f : exp2_hw(ms - mn);
  l = fmaf(l, c_old, ls * c_new);
  a = fmaf(a, c_old, as_ * c_new);
  m = mn;
}

// Same merge for the (m, l) pair only.
__device__ inline void merge_ml(float& m, float& l, float ms, float ls) {
  const float mn = fmaxf(m, ms);
  const float c_old = (m == kNegInf) ? 0.0f : exp2_hw(m - mn);
  const float c_new = (ms == kNegInf) ? 0.0f : exp2_hw(ms - mn);
  l = fmaf(l, c_old, ls * c_new);
  m = mn;
}

__device__ inline int32_t page_of(const PagedParams& p, int key) {
  return p.bs_shift >= 0 ? (key >> p.bs_shift) : (int32_t)((uint32_t)key / (uint32_t)p.bs);
}

// Element offset of `key`'s row in a cache with block stride sb and token stride sp. The
// segment's block-table entries sit in LDS (pages[i] = block_table[b][blk0 + i]), so the K/V
// address never waits on a global load of the table.
__device__ inline int64_t page_offset(const PagedParams& p, const int32_t* pages, int blk0, int key, int64_t sb,
                                      int64_t sp) {
  const int32_t blk = page_of(p, key);
  const int32_t off = key - blk * p.bs;
  return (int64_t)pages[blk - blk0] * sb + (int64_t)off * sp;
}

template <int D>
struct DimTraits {
  static constexpr int kQkSteps = D / 32;  // MFMA K steps of 32 over the head dim
  static constexpr int kDpl = D / 16;      // output dims per lane in P V
};

template <int D, int G, int TPG, int NW>
__global__ __launch_bounds__(64 * NW) void paged_partial_kernel(PagedParams p) {
  static_assert(G >= 1 && G <= 16, "GQA group must fit the 16 MFMA columns");
  constexpr int QS = DimTraits<D>::kQkSteps;
  constexpr int DPL = DimTraits<D>::kDpl;
  __shared__ float s_m[NW][G];
  __shared__ float s_l[NW][G];
  __shared__ float s_acc[NW][G][D];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar loop control
  const int col = lane & 15;  // S layout: head column / PV layout: dim chunk
  const int row = lane >> 4;  // S layout: key quad / PV layout: key quarter

  const int64_t per_seg = p.n * p.KV;
  const int s = (int)(blockIdx.x / per_seg);
  const int64_t rem = blockIdx.x % per_seg;
  const int b = (int)(rem / p.KV);
  const int g = (int)(rem % p.KV);
  if (p.n_live != nullptr && b >= *p.n_live) return;  // not a live request: nothing read or written

  const int L = p.sl[b];
  // Segments the request needs, capped at the model's NS as the fixed grid caps them. A grid
  // trimmed by the caller's bound on the batch's lengths covers every request within that
  // bound with the same segments (the same bits); a longer request gets NaN rows, written by
  // its segment-0 workgroups, instead of a sum over fewer keys.
  const int need = min((L + p.split - 1) / p.split, p.ns_model);
  if (need > p.ns) {
    if (s == 0)
      for (int idx = threadIdx.x; idx < G * D; idx += 64 * NW)
        store_f32_as(p.out, p.out_dtype, (int64_t)b * p.sot + (int64_t)(g * G + idx / D) * p.soh + idx % D,
                     __builtin_nanf(""));
    return;
  }
  const int start = s * p.split;
  if (start >= L) return;  // segment past the end: contributes exactly 0, never read
  const int end = min(start + p.split, L);

  // The segment's block-table entries, staged once into LDS (dynamic shared memory sized
  // split / bs + 2 entries by the launcher).
  extern __shared__ int32_t s_pages[];
  const int blk0 = page_of(p, start);
  const int npg = page_of(p, end - 1) - blk0 + 1;
  for (int i = threadIdx.x; i < npg; i += 64 * NW) s_pages[i] = p.bt[(int64_t)b * p.sbt + blk0 + i];
  __syncthreads();
  const int ntile = (end - start + 15) >> 4;
  const int ngroup = (ntile + TPG - 1) / TPG;

  // q as the B operand: column = head (g*G + col), 8 dims per lane per MFMA step.
  v8bf qf[QS];
  {
    const uint16_t* qrow = p.q + (int64_t)b * p.sqt + (int64_t)(g * G + (col < G ? col : 0)) * p.sqh;
#pragma unroll
    for (int i = 0; i < QS; ++i) {
      v8u16 raw = *reinterpret_cast<const v8u16*>(qrow + 32 * i + 8 * row);
      if (col >= G) raw = v8u16{0, 0, 0, 0, 0, 0, 0, 0};
      qf[i] = __builtin_bit_cast(v8bf, raw);
    }
  }

  const int64_t khead = (int64_t)g * p.skh;
  const int64_t vhead = (int64_t)g * p.svh;

  float m_run = kNegInf, l_run = 0.0f;  // per head column (S layout)
  float acc[G][DPL];                     // PV layout: head x owned dims
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int d = 0; d < DPL; ++d) acc[h][d] = 0.0f;

  for (int grp = wave; grp < ngroup; grp += NW) {
    const int kbase = start + grp * 16 * TPG;
    float sc[TPG][4];
#pragma unroll
    for (int t = 0; t < TPG; ++t) {
      // K rows of this tile: lane col -> key, 8 dims per lane per step.
      const int key = min(kbase + 16 * t + col, end - 1);
      const uint16_t* krow = p.kc + page_offset(p, s_pages, blk0, key, p.skb, p.skp) + khead;
      v4f c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int i = 0; i < QS; ++i) {
        const v8bf kf =
            __builtin_bit_cast(v8bf, __builtin_nontemporal_load(reinterpret_cast<const v8u16*>(krow + 32 * i + 8 * row)));
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[i], c, 0, 0, 0);
      }
      // c[r] = S[key kbase + 16t + 4*row + r][head col]
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kk = kbase + 16 * t + 4 * row + r;
        sc[t][r] = (kk < end) ? c[r] * p.scale_log2 : kNegInf;
      }
    }
    // Online softmax update for this group, fixed order.
    float mx = kNegInf;
#pragma unroll
    for (int t = 0; t < TPG; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) mx = fmaxf(mx, sc[t][r]);
    mx = fmaxf(mx, shfl_xor_f32(mx, 16));
    mx = fmaxf(mx, shfl_xor_f32(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = exp2_hw(m_run - m_new);  // m_run == -inf -> 0
    float psum = 0.0f;
#pragma unroll
    for (int t = 0; t < TPG; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sc[t][r] = exp2_hw(sc[t][r] - m_new);
        psum += sc[t][r];
      }
    psum = psum + shfl_xor_f32(psum, 16);
    psum = psum + shfl_xor_f32(psum, 32);
    l_run = fmaf(l_run, alpha, psum);
    m_run = m_new;

    // P V. Rescale the owned accumulators by each head's alpha (held by lane col == h).
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float ah = shfl_f32(alpha, h);
#pragma unroll
      for (int d = 0; d < DPL; ++d) acc[h][d] = acc[h][d] * ah;
    }
#pragma unroll
    for (int t = 0; t < TPG; ++t) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int key = min(kbase + 16 * t + 4 * row + j, end - 1);
        const uint16_t* vrow = p.vc + page_offset(p, s_pages, blk0, key, p.svb, p.svp) + vhead + col * DPL;
        float v[DPL];
        if constexpr (DPL == 4) {
          const v2u32 raw = __builtin_nontemporal_load(reinterpret_cast<const v2u32*>(vrow));
          v[0] = __uint_as_float(raw.x << 16);
          v[1] = __uint_as_float(raw.x & 0xFFFF0000u);
          v[2] = __uint_as_float(raw.y << 16);
          v[3] = __uint_as_float(raw.y & 0xFFFF0000u);
        } else {
#pragma unroll
          for (int c16 = 0; c16 < DPL / 8; ++c16) {
            const v4u32 raw = __builtin_nontemporal_load(reinterpret_cast<const v4u32*>(vrow + 8 * c16));
            const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              v[8 * c16 + 2 * e] = __uint_as_float(w[e] << 16);
              v[8 * c16 + 2 * e + 1] = __uint_as_float(w[e] & 0xFFFF0000u);
            }
          }
        }
#pragma unroll
        for (int h = 0; h < G; ++h) {
          // p for (key kbase+16t+4*row+j, head h) sits in lane (row, h), register j.
          const float ph = shfl_f32(sc[t][j], (row << 4) | h);
#pragma unroll
          for (int d = 0; d < DPL; ++d) acc[h][d] = fmaf(ph, v[d], acc[h][d]);
        }
      }
    }
  }

  // Sum the four key quarters (fixed pairing, identical result in every lane).
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int d = 0; d < DPL; ++d) {
      acc[h][d] = acc[h][d] + shfl_xor_f32(acc[h][d], 16);
      acc[h][d] = acc[h][d] + shfl_xor_f32(acc[h][d], 32);
    }

  if (row == 0 && col < G) {
    s_m[wave][col] = m_run;
    s_l[wave][col] = l_run;
  }
  if (row == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int d = 0; d < DPL; ++d) s_acc[wave][h][col * DPL + d] = acc[h][d];
  }
  __syncthreads();

  // Fixed-order merge of the waves, then either the final output (single-segment request)
  // or the segment partial.
  const int H = p.H;
  const int nsb = need;
  for (int idx = threadIdx.x; idx < G * D; idx += 64 * NW) {
    const int h = idx / D, d = idx % D;
    float m = kNegInf, l = 0.0f, a = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) merge_state(m, l, a, s_m[w][h], s_l[w][h], s_acc[w][h][d]);
    const int head = g * G + h;
    if (nsb == 1) {
      float mm = kNegInf, ll = 0.0f, aa = 0.0f;
      merge_state(mm, ll, aa, m, l, a);
      store_f32_as(p.out, p.out_dtype, (int64_t)b * p.sot + (int64_t)head * p.soh + d, aa / ll);
    } else {
      const int64_t pi = ((int64_t)b * H + head) * p.ns + s;
      if (d == 0) {
        p.mp[pi] = m;
        p.lp[pi] = l;
      }
      p.ap[pi * D + d] = a;
    }
  }
}

// Fixed-order merge over the segments of one (request, head); one wave per (b, head).
template <int D>
__global__ __launch_bounds__(64) void paged_merge_kernel(PagedParams p) {
  static_assert(D % 64 == 0, "a lane owns D / 64 columns");
  constexpr int DPW = D / 64;
  const int64_t bh = blockIdx.x;
  const int b = (int)(bh / p.H);
  const int head = (int)(bh % p.H);
  const int lane = threadIdx.x;
  // Segments are merged in index order, kChunk of them per pass, and a pass issues every load of
  // its segments first, so it waits for one memory latency rather than one per segment. The
  // first pass's loads go out before the request's length is read: they take segments
  // min(c, ns - 1), inside the workspace whatever the length; later passes clamp to the request's
  // last segment. A segment at or past that count is read and never merged.
  constexpr int kChunk = 8;
  const int64_t base = bh * p.ns;
  float ms[kChunk], ls[kChunk], as_[kChunk][DPW];
  auto load_pass = [&](int s0, int last) {
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      const int64_t s = base + min(s0 + c, last);
      ms[c] = p.mp[s];
      ls[c] = p.lp[s];
#pragma unroll
      for (int j = 0; j < DPW; ++j) as_[c][j] = p.ap[s * D + lane + 64 * j];
    }
  };
  load_pass(0, p.ns - 1);
  asm volatile("" ::: "memory");  // the loads above stay above the reads of the length below
  if (p.n_live != nullptr && b >= *p.n_live) return;
  const int L = p.sl[b];
  const int nsb = min((L + p.split - 1) / p.split, p.ns_model);
  if (nsb == 1 || nsb > p.ns) return;  // written by the partial kernel (NaN rows past a trimmed grid)
  float m[DPW], l[DPW], a[DPW];
#pragma unroll
  for (int j = 0; j < DPW; ++j) {
    m[j] = kNegInf;
    l[j] = 0.0f;
    a[j] = 0.0f;
  }
  for (int s0 = 0;;) {
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      if (s0 + c >= nsb) break;
#pragma unroll
      for (int j = 0; j < DPW; ++j) merge_state(m[j], l[j], a[j], ms[c], ls[c], as_[c][j]);
    }
    s0 += kChunk;
    if (s0 >= nsb) break;
    load_pass(s0, nsb - 1);
  }
#pragma unroll
  for (int j = 0; j < DPW; ++j) {
    const int d = lane + 64 * j;
    store_f32_as(p.out, p.out_dtype, (int64_t)b * p.sot + (int64_t)head * p.soh + d, a[j] / l[j]);
  }
}

// LDS bytes of a segment's block-table entries (the pages a `split`-key window can touch).
size_t page_table_bytes(int64_t split, int64_t bs) { return (size_t)(split / bs + 2) * sizeof(int32_t); }

template <int D, int G, int TPG, int NW>
hipError_t launch_partial(const PagedParams& pp, hipStream_t st) {
  const int64_t blocks = pp.n * pp.KV * pp.ns;
  if (blocks > 0x7FFFFFFFLL) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((paged_partial_kernel<D, G, TPG, NW>), dim3((unsigned)blocks), dim3(64 * NW),
                     page_table_bytes(pp.split, pp.bs), st, pp);
  return hipGetLastError();
}

template <int D, int G>
hipError_t dispatch_tpg_nw(int tpg, int nw, const PagedParams& pp, hipStream_t st) {
  if (nw == 4) {
    if (tpg == 1) return launch_partial<D, G, 1, 4>(pp, st);
    if (tpg == 2) return launch_partial<D, G, 2, 4>(pp, st);
    if (tpg == 4) return launch_partial<D, G, 4, 4>(pp, st);
  } else if (nw == 8) {
    if (tpg == 1) return launch_partial<D, G, 1, 8>(pp, st);
    if (tpg == 2) return launch_partial<D, G, 2, 8>(pp, st);
    if (tpg == 4) return launch_partial<D, G, 4, 8>(pp, st);
  }
  return hipErrorInvalidValue;
}

template <int D>
hipError_t dispatch_g(int G, int tpg, int nw, const PagedParams& pp, hipStream_t st) {
  switch (G) {
    case 1: return dispatch_tpg_nw<D, 1>(tpg, nw, pp, st);
    case 2: return dispatch_tpg_nw<D, 2>(tpg, nw, pp, st);
    case 4: return dispatch_tpg_nw<D, 4>(tpg, nw, pp, st);
    case 8: return dispatch_tpg_nw<D, 8>(tpg, nw, pp, st);
    default: return hipErrorInvalidValue;
  }
}

int64_t num_segments(int64_t max_len, int64_t split) {
  const int64_t ns = (max_len + split - 1) / split;
  return ns < 1 ? 1 : ns;
}

}  // namespace

extern "C" int vxa_paged_decode_workspace(int64_t n, int64_t num_heads, int64_t head_dim, int64_t max_len,
                                          int64_t split, size_t* ws_bytes) {
  if (n < 0 || num_heads <= 0 || head_dim <= 0 || split <= 0 || !ws_bytes) return VXA_ERR_ARG;
  const int64_t ns = num_segments(max_len, split);
  *ws_bytes = ns > 1 ? (size_t)n * num_heads * ns * (head_dim + 2) * sizeof(float) : 0;
  return VXA_OK;
}

namespace {

int paged_decode_impl(const void* q, int64_t sqt, int64_t sqh, const void* k_cache, int64_t skb, int64_t skp,
                      int64_t skh, const void* v_cache, int64_t svb, int64_t svp, int64_t svh,
                      const int32_t* block_table, int64_t sbt, const int32_t* seq_lens, float scale, void* out,
                      int out_dtype, int64_t sot, int64_t soh, int64_t n, const int32_t* n_live,
                      int64_t num_heads, int64_t num_kv_heads, int64_t head_dim, int64_t block_size,
                      int64_t max_len, int64_t max_seq_len, int64_t split, int64_t blk, int64_t waves, void* ws,
                      size_t ws_bytes, vxa_stream_t stream) {
  if (n < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 || split <= 0 ||
      max_seq_len < 0)
    return VXA_ERR_ARG;
  if (out_dtype != VXA_F32 && out_dtype != VXA_BF16 && out_dtype != VXA_F16) return VXA_ERR_ARG;
  if (num_heads % num_kv_heads != 0) return VXA_ERR_ARG;
  if (n == 0) return VXA_OK;
  if (!q || !k_cache || !v_cache || !block_table || !seq_lens || !out) return VXA_ERR_ARG;
  const int64_t G = num_heads / num_kv_heads;
  if (split % 16 != 0 || split > (1 << 30)) return VXA_ERR_UNSUPPORTED;
  if (blk != 16 && blk != 32 && blk != 64) return VXA_ERR_UNSUPPORTED;
  if (waves != 4 && waves != 8) return VXA_ERR_UNSUPPORTED;
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) return VXA_ERR_UNSUPPORTED;
  if (G != 1 && G != 2 && G != 4 && G != 8) return VXA_ERR_UNSUPPORTED;
  if (block_size > (1 << 30) || num_heads > (1 << 20)) return VXA_ERR_UNSUPPORTED;
  if (page_table_bytes(split, block_size) > 32768) return VXA_ERR_UNSUPPORTED;  // split / block_size <= 8190
  // 16-byte row loads of q and V and 16/8-byte K fragments need aligned rows.
  if ((uintptr_t)q % 16 || (uintptr_t)k_cache % 16 || (uintptr_t)v_cache % 16 || sqt % 8 || sqh % 8 ||
      skb % 8 || skp % 8 || skh % 8 || svb % 8 || svp % 8 || svh % 8)
    return VXA_ERR_UNSUPPORTED;

  // The grid: the model's NS segments per request, or fewer when the caller bounds the batch's
  // lengths (max_seq_len > 0); the workspace holds the partials of the grid's segments.
  const int64_t ns_model = num_segments(max_len, split);
  const int64_t ns = max_seq_len > 0 ? std::min(ns_model, num_segments(max_seq_len, split)) : ns_model;
  size_t need = 0;
  vxa_paged_decode_workspace(n, num_heads, head_dim, ns * split, split, &need);
  if (need > 0 && (!ws || ws_bytes < need)) return VXA_ERR_WORKSPACE;

  PagedParams pp;
  pp.q = reinterpret_cast<const uint16_t*>(q);
  pp.sqt = sqt; pp.sqh = sqh;
  pp.kc = reinterpret_cast<const uint16_t*>(k_cache);
  pp.skb = skb; pp.skp = skp; pp.skh = skh;
  pp.vc = reinterpret_cast<const uint16_t*>(v_cache);
  pp.svb = svb; pp.svp = svp; pp.svh = svh;
  pp.bt = block_table; pp.sbt = sbt; pp.sl = seq_lens;
  pp.scale_log2 = (float)((double)scale * 1.4426950408889634);
  pp.split = (int32_t)split;
  pp.ns = (int32_t)ns;
  pp.ns_model = (int32_t)ns_model;
  pp.H = (int32_t)num_heads;
  pp.KV = (int32_t)num_kv_heads;
  pp.bs = (int32_t)block_size;
  pp.bs_shift = -1;
  if ((block_size & (block_size - 1)) == 0) {
    int sh = 0;
    while ((1LL << sh) < block_size) ++sh;
    pp.bs_shift = sh;
  }
  pp.n = n;
  pp.n_live = n_live;
  float* wsf = reinterpret_cast<float*>(ws);
  const int64_t nhs = n * num_heads * ns;
  pp.mp = ns > 1 ? wsf : nullptr;
  pp.lp = ns > 1 ? wsf + nhs : nullptr;
  pp.ap = ns > 1 ? wsf + 2 * nhs : nullptr;
  pp.out = out; pp.sot = sot; pp.soh = soh; pp.out_dtype = out_dtype;

  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int tpg = (int)(blk / 16);
  const int nw = (int)waves;
  hipError_t err;
  switch (head_dim) {
    case 64: err = dispatch_g<64>((int)G, tpg, nw, pp, st); break;
    case 128: err = dispatch_g<128>((int)G, tpg, nw, pp, st); break;
    default: err = dispatch_g<256>((int)G, tpg, nw, pp, st); break;
  }
  if (err == hipErrorInvalidValue) return VXA_ERR_UNSUPPORTED;
  if (err != hipSuccess) return VXA_ERR_LAUNCH;
  if (ns > 1) {
    const int64_t blocks = n * num_heads;
    if (blocks > 0x7FFFFFFFLL) return VXA_ERR_UNSUPPORTED;
    switch (head_dim) {
      case 64: hipLaunchKernelGGL(paged_merge_kernel<64>, dim3((unsigned)blocks), dim3(64), 0, st, pp); break;
      case 128: hipLaunchKernelGGL(paged_merge_kernel<128>, dim3((unsigned)blocks), dim3(64), 0, st, pp); break;
      default: hipLaunchKernelGGL(paged_merge_kernel<256>, dim3((unsigned)blocks), dim3(64), 0, st, pp); break;
    }
    if (hipGetLastError() != hipSuccess) return VXA_ERR_LAUNCH;
  }
  return VXA_OK;
}

}  // namespace

extern "C" int vxa_paged_decode(const void* q, int64_t sqt, int64_t sqh, const void* k_cache, int64_t skb,
                                int64_t skp, int64_t skh, const void* v_cache, int64_t svb, int64_t svp,
                                int64_t svh, const int32_t* block_table, int64_t sbt, const int32_t* seq_lens,
                                float scale, void* out, int out_dtype, int64_t sot, int64_t soh, int64_t n,
                                int64_t num_heads, int64_t num_kv_heads, int64_t head_dim, int64_t block_size,
                                int64_t max_len, int64_t max_seq_len, int64_t split, int64_t blk, int64_t waves,
                                void* ws, size_t ws_bytes, vxa_stream_t stream) {
  return paged_decode_impl(q, sqt, sqh, k_cache, skb, skp, skh, v_cache, svb, svp, svh, block_table, sbt, seq_lens,
                           scale, out, out_dtype, sot, soh, n, nullptr, num_heads, num_kv_heads, head_dim,
                           block_size, max_len, max_seq_len, split, blk, waves, ws, ws_bytes, stream);
}

extern "C" int vxa_paged_decode_prefix(const void* q, int64_t sqt, int64_t sqh, const void* k_cache, int64_t skb,
                                       int64_t skp, int64_t skh, const void* v_cache, int64_t svb, int64_t svp,
                                       int64_t svh, const int32_t* block_table, int64_t sbt,
                                       const int32_t* seq_lens, float scale, void* out, int out_dtype,
                                       int64_t sot, int64_t soh, int64_t n, const int32_t* n_live,
                                       int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                                       int64_t block_size, int64_t max_len, int64_t max_seq_len, int64_t split,
                                       int64_t blk, int64_t waves, void* ws, size_t ws_bytes,
                                       vxa_stream_t stream) {
  if (n_live == nullptr) return VXA_ERR_ARG;
  return paged_decode_impl(q, sqt, sqh, k_cache, skb, skp, skh, v_cache, svb, svp, svh, block_table, sbt, seq_lens,
                           scale, out, out_dtype, sot, soh, n, n_live, num_heads, num_kv_heads, head_dim,
                           block_size, max_len, max_seq_len, split, blk, waves, ws, ws_bytes, stream);
}
