/*
 * exact_oracle.c -- CPU oracle for the exact linear path. TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this library,
 * and only to check results (or as the timed CPU baseline). The product path never calls it.
 *
 * It restates, in plain C, the reference's CPU arithmetic:
 *   oracle_digitize_f32      <- kernels.py:22-39 (digitize_torch); exponent via frexp as
 *                               torch.frexp; scale from bits kernels.py:29; truncation
 *                               kernels.py:30 (saturating, NaN -> 0, as the device cast)
 *   oracle_exact_linear      <- kernels.py:89-100 (exact_linear_torch): int64 digit sums,
 *                               2^e from bits (kernels.py:99), fp64 -> fp32 cast (RNE)
 *   oracle_exact_entries     <- same arithmetic for a list of (row, col) entries
 *   oracle_f32_to_bf16       <- fp32 -> bf16 round-to-nearest-even (the bf16 output of
 *                               kernels.py:156-157 / tests/test_gpu.py:30-32)
 *   oracle_paged_decode_f64  <- paged_attn.py:117-132 (paged_decode_torch) in float64
 *
 * Pinned by tests/test_oracle.py (closed forms, hand-computed known answers, exact-integer
 * brute force, torch's independent bf16 conversion, attention special cases).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline double u2d(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }

/* float -> int32 toward zero; out of range saturates, NaN -> 0 (the GPU conversion). */
static inline int32_t trunc_i32(float v) {
  if (v != v) return 0;
  if (v >= 2147483648.0f) return INT32_MAX;
  if (v < -2147483648.0f) return INT32_MIN;
  return (int32_t)v;
}

int oracle_digitize_f32(const float* x, int64_t rows, int64_t k, int f, int8_t* h, int8_t* l, int32_t* cs,
                        int32_t* sh) {
  if (f < 1 || f > 15) return 1;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * k;
    float a = 0.0f;
    for (int64_t i = 0; i < k; ++i) {
      const float v = fabsf(xr[i]);
      if (v > a) a = v;
    }
    int e = 0;
    if (a > 0.0f) (void)frexpf(a, &e);
    const int s = f - e;
    const float scale = u2f((uint32_t)(s + 127) << 23);
    uint32_t csum = 0;
    for (int64_t i = 0; i < k; ++i) {
      const int32_t q = trunc_i32(xr[i] * scale);
      const uint32_t uq = (uint32_t)q;
      int32_t hd, ld;
      if (f == 15) {
        ld = (int32_t)(uq & 255u) - 128;
        hd = (int32_t)(uq - (uint32_t)ld - 128u) >> 8;
        csum += (uint32_t)(256 * hd + ld);
      } else {
        ld = (int32_t)((uq + 128u) & 255u) - 128;
        hd = (int32_t)(uq - (uint32_t)ld) >> 8;
      }
      h[r * k + i] = (int8_t)hd;
      l[r * k + i] = (int8_t)ld;
    }
    cs[r] = f == 15 ? (int32_t)csum : 0;
    sh[r] = s;
  }
  return 0;
}

/* One output element: exact integer sums, then the epilogue. */
static inline float exact_entry(const int8_t* xh, const int8_t* xl, const int8_t* wh, const int8_t* wl, int64_t k,
                                int32_t cx, int32_t cw, int32_t sx, int32_t sw, int f, int trunc) {
  int64_t hh = 0, md = 0, ll = 0;
  /* int32 partial sums over chunks of <= 32768 terms stay exact (|term| <= 2^15). */
  for (int64_t k0 = 0; k0 < k; k0 += 32768) {
    const int64_t k1 = k0 + 32768 < k ? k0 + 32768 : k;
    int32_t a = 0, b = 0, c = 0;
    for (int64_t i = k0; i < k1; ++i) {
      const int32_t p = xh[i], q = xl[i], r = wh[i], s = wl[i];
      a += p * r;
      b += p * s + q * r;
      c += q * s;
    }
    hh += a;
    md += b;
    ll += c;
  }
  int64_t tot = hh * 65536 + md * 256;
  if (!trunc) tot += ll;
  if (f == 15) tot += 128 * ((int64_t)cx + (int64_t)cw) + 128 * 128 * k;
  const int64_t e = -((int64_t)sx + (int64_t)sw);
  const double scale = u2d((uint64_t)(e + 1023) << 52);
  return (float)((double)tot * scale);
}

int oracle_exact_linear(const int8_t* xh, const int8_t* xl, const int32_t* cx, const int32_t* sx, const int8_t* wh,
                        const int8_t* wl, const int32_t* cw, const int32_t* sw, int64_t m, int64_t n, int64_t k,
                        int f, int trunc, float* out) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j)
      out[i * n + j] = exact_entry(xh + i * k, xl + i * k, wh + j * k, wl + j * k, k, cx ? cx[i] : 0,
                                   cw ? cw[j] : 0, sx[i], sw[j], f, trunc);
  return 0;
}

int oracle_exact_entries(const int8_t* xh, const int8_t* xl, const int32_t* cx, const int32_t* sx,
                         const int8_t* wh, const int8_t* wl, const int32_t* cw, const int32_t* sw, int64_t k, int f,
                         int trunc, const int64_t* rows, const int64_t* cols, int64_t count, float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < count; ++t) {
    const int64_t i = rows[t], j = cols[t];
    out[t] = exact_entry(xh + i * k, xl + i * k, wh + j * k, wl + j * k, k, cx ? cx[i] : 0, cw ? cw[j] : 0, sx[i],
                         sw[j], f, trunc);
  }
  return 0;
}

void oracle_f32_to_bf16(const float* in, int64_t count, uint16_t* out) {
  for (int64_t t = 0; t < count; ++t) {
    uint32_t u = f2u(in[t]);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) {
      out[t] = 0x7FC0u;
      continue;
    }
    u += 0x7FFFu + ((u >> 16) & 1u);
    out[t] = (uint16_t)(u >> 16);
  }
}

static inline double bf16d(uint16_t b) { return (double)u2f((uint32_t)b << 16); }

/*
 * Float64 paged decode attention for requests [0, n): per request b and head h,
 * out[b, h, :] = softmax(scale * K_b q_bh) V_b with K_b, V_b gathered through the block
 * table (paged_attn.py:117-132). Element strides as in the kernel's C ABI.
 */
int oracle_paged_decode_f64(const uint16_t* q, int64_t sqt, int64_t sqh, const uint16_t* kc, int64_t skb,
                            int64_t skp, int64_t skh, const uint16_t* vc, int64_t svb, int64_t svp, int64_t svh,
                            const int32_t* bt, int64_t sbt, const int32_t* sl, double scale, int64_t n, int64_t H,
                            int64_t KV, int64_t D, int64_t BS, double* out) {
  const int64_t G = H / KV;
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int64_t b = 0; b < n; ++b)
    for (int64_t h = 0; h < H; ++h) {
      const int64_t L = sl[b];
      const int64_t g = h / G;
      const uint16_t* qr = q + b * sqt + h * sqh;
      double* o = out + (b * H + h) * D;
      for (int64_t d = 0; d < D; ++d) o[d] = 0.0;
      double mx = -INFINITY;
      for (int64_t t = 0; t < L; ++t) {
        const int64_t page = bt[b * sbt + t / BS], off = t % BS;
        const uint16_t* kr = kc + page * skb + off * skp + g * skh;
        double s = 0.0;
        for (int64_t d = 0; d < D; ++d) s += bf16d(qr[d]) * bf16d(kr[d]);
        s *= scale;
        if (s > mx) mx = s;
      }
      double den = 0.0;
      for (int64_t t = 0; t < L; ++t) {
        const int64_t page = bt[b * sbt + t / BS], off = t % BS;
        const uint16_t* kr = kc + page * skb + off * skp + g * skh;
        const uint16_t* vr = vc + page * svb + off * svp + g * svh;
        double s = 0.0;
        for (int64_t d = 0; d < D; ++d) s += bf16d(qr[d]) * bf16d(kr[d]);
        const double p = exp(s * scale - mx);
        den += p;
        for (int64_t d = 0; d < D; ++d) o[d] += p * bf16d(vr[d]);
      }
      for (int64_t d = 0; d < D; ++d) o[d] /= den;
    }
  return 0;
}
