/*
 * vllm_exact_amd.h -- C ABI of the MI355X (gfx950) exact linear path.
 *
 * One shared library, libvllm_exact_amd.so, built from the HIP sources in vllm-exact_amd/csrc.
 * Every entry point:
 *   - takes device pointers, 64-bit sizes and element strides (innermost dimension
 *     contiguous), element-type enums and a hipStream_t passed as `vxa_stream_t`;
 *   - never allocates, never synchronises, never reads device memory on the host;
 *   - launches asynchronously on `stream` and returns a VXA_* status code.
 * Workspace (split-K partial sums, attention segment partials) is owned by the caller;
 * its size comes from the matching *_plan / *_workspace query.
 *
 * The Python layer (vllm_exact.kernels / vllm_exact.paged_attn) binds these with ctypes
 * and keeps the reference's Python surface on top of them.
 */
#ifndef VLLM_EXACT_AMD_H
#define VLLM_EXACT_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. The Python binding maps ERR_ARG and ERR_TOO_LARGE to ValueError,
 * ERR_UNSUPPORTED to NotImplementedError (so autotune/tuners can skip a config,
 * kernels.py:313-314), and the rest to RuntimeError. */
enum {
  VXA_OK = 0,
  VXA_ERR_ARG = 1,          /* bad pointer / size / stride / F / dtype */
  VXA_ERR_UNSUPPORTED = 2,  /* shape or config outside what the kernels implement */
  VXA_ERR_WORKSPACE = 3,    /* workspace missing or smaller than the plan requires */
  VXA_ERR_LAUNCH = 4,       /* hipLaunchKernel / hipGetLastError failure */
  VXA_ERR_TOO_LARGE = 5     /* needs more than the fixed scratch of vxa_exact_linear_op_noalloc */
};

/* Element types of floating-point tensors crossing the boundary. */
enum { VXA_F32 = 0, VXA_BF16 = 1, VXA_F16 = 2 };

typedef void* vxa_stream_t; /* a hipStream_t; NULL is the null stream */

/* Library version string and a human-readable status message. */
const char* vxa_version(void);
const char* vxa_status_string(int status);

/*
 * Per-row F-bit fixed-point digitization.
 * Replaces kernels.py:74-85 (`digitize`, device body `_digitize_kernel` kernels.py:47-71;
 * numerical spec kernels.py:3-9, CPU statement `digitize_torch` kernels.py:22-39).
 *   x       [rows, k] with row stride ldx (elements), dtype VXA_F32 / VXA_BF16 / VXA_F16
 *   h, l    int8 [rows, k] digit planes, row stride ldd (bytes == elements)
 *   cs      int32 [rows] row sum of 256*h+l (F == 15), 0 otherwise
 *   sh      int32 [rows] shift: q = trunc(x * 2^sh)
 *   f       fixed-point bits, 1..15; f == 15 uses offset digits, f < 15 balanced digits
 */
int vxa_digitize(const void* x, int x_dtype, int64_t rows, int64_t k, int64_t ldx,
                 int8_t* h, int8_t* l, int64_t ldd, int32_t* cs, int32_t* sh,
                 int f, vxa_stream_t stream);

/*
 * Split-K plan for vxa_exact_linear. Replaces the host arithmetic of kernels.py:268-273:
 * KCH = cdiv(cdiv(K, SK), BK) * BK, SK = cdiv(K, KCH), workspace int64 [SK, M, N] when SK > 1.
 *   cfg, cfg_len  the reference cfg tuple (BM, BN, BK, warps, stages, GM[, SK[, mma]]),
 *                 cfg_len in 6..8 (kernels.py:268-270); mma is accepted and ignored
 *                 (INT8 MFMA gives the same bits).
 *   *sk_out       number of K splits actually used
 *   *kch_out      K extent of one split
 *   *ws_bytes     workspace bytes the caller must pass to vxa_exact_linear (0 if none)
 */
int vxa_exact_linear_plan(int64_t m, int64_t n, int64_t k, const int32_t* cfg, int cfg_len,
                          int32_t* sk_out, int64_t* kch_out, size_t* ws_bytes);

/*
 * Exact two-digit linear layer: out[m, n] = round(2^-(sx[m]+sw[n]) * tot[m, n]) with
 *   tot = 2^16 * sum(xh*wh) + 2^8 * sum(xh*wl + xl*wh) [+ sum(xl*wl) unless trunc]
 *         [+ 128*(cx[m] + cw[n]) + 128*128*K when f == 15]
 * accumulated exactly (int8 MFMA -> int32 -> int64), converted int64 -> fp64 (exact)
 * -> fp32 (RNE) -> out dtype (RNE). Replaces kernels.py:257-289 (`exact_linear`), with the
 * device bodies `_exact_kernel` kernels.py:104-157 and `_exact_fin` kernels.py:159-177.
 *   xh, xl [m, k] int8 row stride ldx; cx, sx int32 [m]      (activation digits)
 *   wh, wl [n, k] int8 row stride ldw; cw, sw int32 [n]      (weight digits, NT layout)
 *   out    [m, n] row stride ldo, dtype VXA_F32 / VXA_BF16 / VXA_F16
 *   ws     int64 workspace of at least the planned ws_bytes (may be NULL if 0)
 * Bits do not depend on cfg: every tiling and split-K partition gives the same output.
 */
int vxa_exact_linear(const int8_t* xh, const int8_t* xl, const int32_t* cx, const int32_t* sx,
                     int64_t ldx,
                     const int8_t* wh, const int8_t* wl, const int32_t* cw, const int32_t* sw,
                     int64_t ldw,
                     void* out, int out_dtype, int64_t ldo,
                     int64_t m, int64_t n, int64_t k, int f, int trunc,
                     const int32_t* cfg, int cfg_len,
                     void* ws, size_t ws_bytes, vxa_stream_t stream);

/*
 * Fragment-major packed digits (the operand order of v_mfma_i32_16x16x64_i8).
 * A [rows, k] pair of digit planes (h, l) packs into cdiv(rows,16) x cdiv(k,64) blocks of
 * 2 KiB: block (rt, kt) = [h fragment | l fragment], fragment byte 16*lane + j holding
 * row 16*rt + (lane & 15), column 64*kt + 16*(lane >> 4) + j; rows >= rows and columns >= k
 * are zero digits. Each MFMA operand is then 1 KiB of contiguous memory. Weights are packed
 * once at load time (the reference digitizes them there, plugin.py:72-79); activations are
 * digitized straight into the packed form. No reference counterpart: the reference keeps
 * row-major digits only. vxa_packed_bytes returns the packed size.
 */
size_t vxa_packed_bytes(int64_t rows, int64_t k);
int vxa_pack_digits(const int8_t* h, const int8_t* l, int64_t rows, int64_t k, int64_t ldd,
                    int8_t* packed, vxa_stream_t stream);
/* digitize (same bits as vxa_digitize) writing the packed layout; cs, sh as vxa_digitize. */
int vxa_digitize_packed(const void* x, int x_dtype, int64_t rows, int64_t k, int64_t ldx,
                        int8_t* packed, int32_t* cs, int32_t* sh, int f, vxa_stream_t stream);
/*
 * vxa_exact_linear on packed operands: same arithmetic, same bits, same cfg and split-K
 * semantics (the plan uses k rounded up to a multiple of 64). xp / wp are packed digits of
 * x [m, k] and w [n, k]. This is the entry point the exactmm::linear op uses for weights
 * packed at load time (plugin.py:51-64 replaces the row-major call there).
 */
int vxa_exact_linear_packed(const int8_t* xp, const int32_t* cx, const int32_t* sx,
                            const int8_t* wp, const int32_t* cw, const int32_t* sw,
                            void* out, int out_dtype, int64_t ldo,
                            int64_t m, int64_t n, int64_t k, int f, int trunc,
                            const int32_t* cfg, int cfg_len,
                            void* ws, size_t ws_bytes, vxa_stream_t stream);

/*
 * Digitize x and run vxa_exact_linear_packed in one launch: the same bits as
 * vxa_digitize_packed followed by vxa_exact_linear_packed.
 *   x    bf16 [m, k], row stride ldx elements
 *   wp, cw, sw  packed weight digits, digit sums and shifts (as vxa_exact_linear_packed); cw
 *           is read for f = 15 only (may be null otherwise)
 *   cfg  a small-M config with one-row tiles (BM <= 16) and SK = 1; k <= 32768, so that the
 *        plan keeps one K split (int32 digit sums stay exact)
 * Each workgroup digitizes its own 16 rows of x (row absmax over k, then the digits in
 * registers). Returns VXA_ERR_UNSUPPORTED for another cfg family, a plan with more than one
 * K split, x rows that are not 16-byte aligned, or f = 15 with 3 dots or on a 16-wave cfg
 * with four column tiles times steps per round (whose digit sum would spill): the caller
 * then takes the two-launch path. No reference counterpart:
 * the reference digitizes x in a launch of its own (plugin.py:62-64); this entry point serves
 * the exactmm::linear op at decode sizes, where that launch is a quarter of the op.
 */
int vxa_exact_linear_bf16x(const void* x, int64_t ldx, const int8_t* wp, const int32_t* cw,
                           const int32_t* sw, void* out, int out_dtype, int64_t ldo,
                           int64_t m, int64_t n, int64_t k, int f, int trunc,
                           const int32_t* cfg, int cfg_len, vxa_stream_t stream);

/*
 * Workspace bytes for vxa_paged_decode: fp32 segment partials m, l [n, H, NS] and
 * acc [n, H, NS, D] with NS = max(1, cdiv(max_len, split)) (paged_attn.py:105-108).
 * Zero when NS == 1 (every request then finishes inside one segment).
 */
int vxa_paged_decode_workspace(int64_t n, int64_t num_heads, int64_t head_dim, int64_t max_len,
                               int64_t split, size_t* ws_bytes);

/*
 * Paged decode attention for one new token per request, with a fixed reduction order.
 * Replaces paged_attn.py:97-114 (`paged_decode`, device bodies `_paged_partial`
 * paged_attn.py:31-72 and `_paged_merge` paged_attn.py:75-94).
 *   q        bf16 [>=n, H, D], strides (sqt, sqh) in elements, innermost contiguous
 *   k_cache, v_cache  bf16 views (num_blocks, block_size, KV, D) with element strides
 *            (skb, skp, skh) and (svb, svp, svh); innermost contiguous
 *            (vLLM FlashAttention layout, paged_attn.py:8-9)
 *   block_table int32 [B, max_blocks] row stride sbt; seq_lens int32 [B]
 *   scale    softmax scale
 *   out      [>=n, H, D] strides (sot, soh), dtype VXA_F32 / VXA_BF16 / VXA_F16
 *   n        number of leading requests to compute (paged_attn.py:99)
 *   max_len  model maximum length: fixes NS = cdiv(max_len, split) (paged_attn.py:105)
 *   max_seq_len  a bound on seq_lens[:n] (the reference's max_seq_len argument,
 *            paged_attn.py:97, which it leaves unused), or 0 for none. The grid then covers
 *            min(NS, cdiv(max_seq_len, split)) segments per request: every request within the
 *            bound gets the bits of the full grid; a request longer than the bound (and within
 *            max_len) gets NaN rows. The workspace needs the partials of that many segments
 *            (vxa_paged_decode_workspace with max_len = min(max_len, max_seq_len)).
 *            VXA_ERR_ARG when negative.
 *   split    keys per segment; blk keys per online-softmax step (16, 32 or 64);
 *            waves per workgroup (4 or 8). split, blk and waves fix the floating-point
 *            order; the result never depends on n or on the other requests.
 */
int vxa_paged_decode(const void* q, int64_t sqt, int64_t sqh,
                     const void* k_cache, int64_t skb, int64_t skp, int64_t skh,
                     const void* v_cache, int64_t svb, int64_t svp, int64_t svh,
                     const int32_t* block_table, int64_t sbt, const int32_t* seq_lens,
                     float scale, void* out, int out_dtype, int64_t sot, int64_t soh,
                     int64_t n, int64_t num_heads, int64_t num_kv_heads, int64_t head_dim,
                     int64_t block_size, int64_t max_len, int64_t max_seq_len, int64_t split,
                     int64_t blk, int64_t waves, void* ws, size_t ws_bytes, vxa_stream_t stream);

/*
 * vxa_paged_decode for the first *n_live requests, with the count read on the device:
 * n (>= *n_live) sizes the grid and the workspace, and the workgroups of requests at or past
 * *n_live return before reading their length, block table, query or cache, and write nothing.
 * Replaces the host round trip of the mixed-step path in paged_attn.py:154-159, where the
 * number of leading decode requests is read back with .item() before the launch; here it
 * stays on the GPU. n_live must be a device pointer (VXA_ERR_ARG when null).
 */
int vxa_paged_decode_prefix(const void* q, int64_t sqt, int64_t sqh,
                            const void* k_cache, int64_t skb, int64_t skp, int64_t skh,
                            const void* v_cache, int64_t svb, int64_t svp, int64_t svh,
                            const int32_t* block_table, int64_t sbt, const int32_t* seq_lens,
                            float scale, void* out, int out_dtype, int64_t sot, int64_t soh,
                            int64_t n, const int32_t* n_live, int64_t num_heads,
                            int64_t num_kv_heads, int64_t head_dim, int64_t block_size,
                            int64_t max_len, int64_t max_seq_len, int64_t split, int64_t blk,
                            int64_t waves, void* ws, size_t ws_bytes, vxa_stream_t stream);

/* Bytes of device memory vxa_exact_linear_op_noalloc holds per GPU (a file-scope array). */
#define VXA_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

/*
 * The exactmm::linear op with no allocation: vxa_digitize_packed of x followed by
 * vxa_exact_linear_packed, the same bits, with the packed activation digits, their row sums
 * and shifts, and the split-K partials kept in a fixed array of VXA_NOALLOC_SCRATCH_BYTES that
 * the library holds on each GPU until the process ends. Calls no hipMalloc or hipFree.
 *   x      [m, k] activations, dtype VXA_F32 / VXA_BF16 / VXA_F16, row stride ldx elements
 *   wp, cw, sw, out, cfg   as vxa_exact_linear_packed
 * Needs vxa_packed_bytes(m, k) + 8 m (each part rounded up to 256 bytes) + the planned split-K
 * workspace to fit the array; larger problems return VXA_ERR_TOO_LARGE before any launch (for
 * example 4096 rows of 4096 columns, or a split-K plan over 256 x 151936 outputs).
 * Every call on one GPU uses that GPU's array: calls that overlap on one GPU (two streams, two
 * threads) race and must be serialised by the caller. The first call on each device looks the
 * array's device address up; make it outside graph capture.
 * No counterpart in the reference (which allocates the digits and the split-K workspace with
 * torch.empty, kernels.py:78-80, 273): for callers that cannot allocate, such as code under
 * HIP graph capture, fixed serving loops and harnesses that forbid allocation.
 */
int vxa_exact_linear_op_noalloc(const void* x, int x_dtype, int64_t ldx, const int8_t* wp,
                                const int32_t* cw, const int32_t* sw, void* out, int out_dtype,
                                int64_t ldo, int64_t m, int64_t n, int64_t k, int f, int trunc,
                                const int32_t* cfg, int cfg_len, vxa_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* VLLM_EXACT_AMD_H */
