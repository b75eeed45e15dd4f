/*
 * CPU oracle for the fused kernels -- TEST INFRASTRUCTURE ONLY.
 *
 * Plain-C restatement of the reference's fused RMSNorm, SwiGLU and reversible
 * residual arithmetic.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and only as the checker / the timed CPU
 * baseline; the product path never calls it.
 *
 *   oracle_rmsnorm_fwd   src/reversibility/kernels_v3.py:9-16   (_rms_forward)
 *   oracle_rmsnorm_bwd   src/reversibility/kernels_v3.py:19-48  (_rms_dx,
 *                        _rms_dw_partials, _rms_dw_reduce)
 *   oracle_swiglu_fwd    src/reversibility/kernels.py:88-95     (_swiglu_forward)
 *   oracle_swiglu_bwd    src/reversibility/kernels.py:98-110    (_swiglu_backward)
 *   oracle_midpoint      src/reversibility/reversible.py:16-32  (p +/- 2h (A+M))
 *   oracle_midpoint_bwd  autograd of the same eager expression
 *   oracle_euler         src/reversibility/reversible.py:24-25,31-32
 *   oracle_ce_fwd        src/reversibility/kernels.py:14-45,56-67 (_ce_partials,
 *                        _ce_rows, TiledCrossEntropy.forward)
 *   oracle_ce_bwd        src/reversibility/kernels.py:48-60,69-77 (_ce_grad,
 *                        TiledCrossEntropy.backward)
 *   oracle_embed_fwd     src/reversibility/reversible.py:105-106, model.py
 *                        (token_embedding(ids) + position_embedding(arange(T)))
 *   oracle_embed_bwd_pos the position table's gradient through the broadcast
 *                        add: sum over the batch, in batch order
 *   oracle_embed_bwd_tok nn.Embedding's weight gradient, summed per id in the
 *                        fixed order of the device kernel (see below)
 *
 * RMSNorm sums are accumulated in double (a tighter reference than any fp32
 * summation order); outputs are rounded once to float.  SwiGLU uses float
 * arithmetic with the reference's fp16 rounding points, implemented here from
 * the IEEE 754 binary16 format (round to nearest, ties to even).  The
 * residual updates follow the eager expression's rounding points exactly.
 * Loops are OpenMP-parallel; every output element is computed by one thread
 * in a fixed order, so results do not depend on the thread count.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- IEEE 754 binary16 / bfloat16 rounding ------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* float -> binary16 bits, round to nearest even; overflow -> inf; NaN kept. */
uint16_t oracle_f32_to_f16(float f) {
  const uint32_t u = f2u(f);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t exp = (u >> 23) & 0xffu;
  uint32_t man = u & 0x7fffffu;
  if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u));
  const int e = (int)exp - 127;                             /* unbiased */
  if (e > 15) return (uint16_t)(sign | 0x7c00u);           /* overflow */
  if (e >= -14) {                                           /* normal half */
    uint32_t h = ((uint32_t)(e + 15) << 10) | (man >> 13);
    const uint32_t rest = man & 0x1fffu;                    /* 13 dropped bits */
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1u;  /* carry may reach inf */
    return (uint16_t)(sign | h);
  }
  if (e < -25) return (uint16_t)sign;                       /* below half of min subnormal */
  man |= 0x800000u;                                         /* implicit bit */
  const int shift = -e - 1;                                 /* 14..24: value = man * 2^(e-23) */
  uint32_t h = man >> shift;                                /* in units of 2^-24 */
  const uint32_t rest = man & ((1u << shift) - 1u);
  const uint32_t half = 1u << (shift - 1);
  if (rest > half || (rest == half && (h & 1u))) h += 1u;
  return (uint16_t)(sign | h);
}

float oracle_f16_to_f32(uint16_t h) {
  const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  const uint32_t man = h & 0x3ffu;
  if (exp == 0) {
    const float mag = (float)man * 5.9604644775390625e-08f;  /* man * 2^-24, exact */
    return sign ? -mag : mag;
  }
  if (exp == 0x1fu) return u2f(sign | 0x7f800000u | (man << 13));
  return u2f(sign | ((exp - 15 + 127) << 23) | (man << 13));
}

static inline float round_f16(float v) { return oracle_f16_to_f32(oracle_f32_to_f16(v)); }

/* bfloat16: keep the top 16 bits, round to nearest even. */
float oracle_round_bf16(float v) {
  uint32_t u = f2u(v);
  if ((u & 0x7f800000u) == 0x7f800000u) return v;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u2f(u & 0xffff0000u);
}

/* dtype codes shared with include/reversibility_hip.h */
enum { F32 = 0, F16 = 1, BF16 = 2, F64 = 3 };

static inline float round_to(float v, int dtype) {
  if (dtype == F16) return round_f16(v);
  if (dtype == BF16) return oracle_round_bf16(v);
  return v;
}

int oracle_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void oracle_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* ---- RMSNorm ------------------------------------------------------------ */

static double row_rstd(const float* xr, int64_t width, double eps) {
  double ss = 0.0;
  for (int64_t c = 0; c < width; ++c) ss += (double)xr[c] * (double)xr[c];
  return 1.0 / sqrt(ss / (double)width + eps);
}

/* y = (x * r) * w, r = 1/sqrt(mean(x^2) + eps), all in double. */
void oracle_rmsnorm_fwd(const float* x, const float* w, float* y, float* rstd,
                        int64_t rows, int64_t width, double eps) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * width;
    const double rs = row_rstd(xr, width, eps);
    for (int64_t c = 0; c < width; ++c)
      y[r * width + c] = (float)(((double)xr[c] * rs) * (double)w[c]);
    rstd[r] = (float)rs;
  }
}

/* dx = (g - x * (sum(g*x)/width * r^2)) * r with g = dy*w;
 * dw[c] = sum_r dy * (x * r).  r is recomputed in double from x (the value
 * the forward defines), not read back from a rounded float. */
void oracle_rmsnorm_bwd(const float* x, const float* w, const float* dy,
                        float* dx, float* dw, int64_t rows, int64_t width,
                        double eps) {
  double* rs = (double*)malloc((size_t)(rows > 0 ? rows : 1) * sizeof(double));
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * width;
    const float* gr = dy + r * width;
    const double rr = row_rstd(xr, width, eps);
    double dot = 0.0;
    for (int64_t c = 0; c < width; ++c)
      dot += ((double)gr[c] * (double)w[c]) * (double)xr[c];
    const double corr = dot / (double)width * rr * rr;
    for (int64_t c = 0; c < width; ++c) {
      const double g = (double)gr[c] * (double)w[c];
      dx[r * width + c] = (float)((g - (double)xr[c] * corr) * rr);
    }
    rs[r] = rr;
  }
  /* Column blocks of 16: each thread owns whole columns and walks the rows
   * in order, reading each row's block contiguously. */
  const int64_t cb = 16;
  const int64_t nblocks = (width + cb - 1) / cb;
#pragma omp parallel for schedule(static)
  for (int64_t b = 0; b < nblocks; ++b) {
    double acc[16] = {0};
    const int64_t c0 = b * cb;
    const int64_t c1 = c0 + cb < width ? c0 + cb : width;
    for (int64_t r = 0; r < rows; ++r) {
      const float* xr = x + r * width;
      const float* gr = dy + r * width;
      for (int64_t c = c0; c < c1; ++c)
        acc[c - c0] += (double)gr[c] * ((double)xr[c] * rs[r]);
    }
    for (int64_t c = c0; c < c1; ++c) dw[c] = (float)acc[c - c0];
  }
  free(rs);
}

/* ---- SwiGLU (I/O in binary16 bits or float; math in float) -------------- */

static inline float sigmoid_f(float g) { return 1.0f / (1.0f + expf(-g)); }

/* u: [rows, ld_u] with gate cols [0,width), value cols [width,2*width).
 * dtype F16: u/o hold binary16 bits (uint16); F32: floats. */
void oracle_swiglu_fwd(const void* u, int64_t ld_u, void* o, int64_t rows,
                       int64_t width, int dtype) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t c = 0; c < width; ++c) {
      float g, v;
      if (dtype == F16) {
        g = oracle_f16_to_f32(((const uint16_t*)u)[r * ld_u + c]);
        v = oracle_f16_to_f32(((const uint16_t*)u)[r * ld_u + width + c]);
      } else {
        g = ((const float*)u)[r * ld_u + c];
        v = ((const float*)u)[r * ld_u + width + c];
      }
      const float silu = round_to(g / (1.0f + expf(-g)), dtype);
      const float out = silu * v;
      if (dtype == F16) ((uint16_t*)o)[r * width + c] = oracle_f32_to_f16(out);
      else ((float*)o)[r * width + c] = out;
    }
  }
}

void oracle_swiglu_bwd(const void* u, int64_t ld_u, const void* dy, void* du,
                       int64_t rows, int64_t width, int dtype) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t c = 0; c < width; ++c) {
      float g, v, d;
      if (dtype == F16) {
        g = oracle_f16_to_f32(((const uint16_t*)u)[r * ld_u + c]);
        v = oracle_f16_to_f32(((const uint16_t*)u)[r * ld_u + width + c]);
        d = oracle_f16_to_f32(((const uint16_t*)dy)[r * width + c]);
      } else {
        g = ((const float*)u)[r * ld_u + c];
        v = ((const float*)u)[r * ld_u + width + c];
        d = ((const float*)dy)[r * width + c];
      }
      const float s = sigmoid_f(g);
      const float silu = round_to(g * s, dtype);
      const float dgi = round_to(d * v, dtype);
      const float dg = dgi * (s * (1.0f + g * (1.0f - s)));
      const float dv = d * silu;
      if (dtype == F16) {
        ((uint16_t*)du)[r * ld_u + c] = oracle_f32_to_f16(dg);
        ((uint16_t*)du)[r * ld_u + width + c] = oracle_f32_to_f16(dv);
      } else {
        ((float*)du)[r * ld_u + c] = dg;
        ((float*)du)[r * ld_u + width + c] = dv;
      }
    }
  }
}

/* ---- reversible residual updates (state float, force dtype) ------------ */

static inline float load_force(const void* f, int64_t i, int dtype) {
  if (dtype == F16) return oracle_f16_to_f32(((const uint16_t*)f)[i]);
  if (dtype == BF16) return u2f((uint32_t)((const uint16_t*)f)[i] << 16);
  return ((const float*)f)[i];
}

/* out = p + sign * round(round(a + m) * scale)   (fp32 state) */
void oracle_midpoint(const float* p, const void* a, const void* m, float* out,
                     float scale, int sign, int64_t n, int force_dtype) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    const float f = round_to(load_force(a, i, force_dtype) + load_force(m, i, force_dtype), force_dtype);
    const float c = round_to(f * scale, force_dtype);
    out[i] = sign > 0 ? p[i] + c : p[i] - c;
  }
}

/* da = sign * round(round(dout) * scale), returned widened to float. */
void oracle_midpoint_bwd(const float* dout, float* da, float scale, int sign,
                         int64_t n, int force_dtype) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    const float g = round_to(sign > 0 ? dout[i] : -dout[i], force_dtype);
    da[i] = round_to(g * scale, force_dtype);
  }
}

void oracle_midpoint_f64(const double* p, const double* a, const double* m,
                         double* out, double scale, int sign, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    const double c = (a[i] + m[i]) * scale;
    out[i] = sign > 0 ? p[i] + c : p[i] - c;
  }
}

/* out = x + sign * f */
void oracle_euler(const float* x, const void* f, float* out, int sign,
                  int64_t n, int force_dtype) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    const float v = load_force(f, i, force_dtype);
    out[i] = sign > 0 ? x[i] + v : x[i] - v;
  }
}

/* ---- array forms of the conversions (for exhaustive checks) ------------ */

void oracle_f32_to_f16_array(const float* src, uint16_t* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = oracle_f32_to_f16(src[i]);
}

void oracle_f16_to_f32_array(const uint16_t* src, float* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = oracle_f16_to_f32(src[i]);
}

/* ---- tiled cross-entropy (src/reversibility/kernels.py:14-71) ----------
 * Per row of logits x (fp16 bits or float, row stride ld):
 *   maximum     m   = max_j x_j                                  (exact)
 *   denominator lse = log(sum_j exp(x_j - m)), accumulated in double,
 *                     rounded once to float                      (_ce_rows)
 *   logp        = round_T((x_t - m) - lse)     float arithmetic, then the
 *                                              logits dtype T    (_ce_rows)
 *   loss        = -logp, 0 for label == ignore
 *   dx_j        = round_T([j == t] neg - exp(round_T((x_j - m) - lse)) neg),
 *                 neg = round_T(-grad), 0 rows for ignore         (_ce_grad)
 * A label outside [0, cols) other than ignore gives a NaN loss / NaN row. */
static inline float load_logit(const void* x, int64_t i, int dtype) {
  return dtype == F16 ? oracle_f16_to_f32(((const uint16_t*)x)[i]) : ((const float*)x)[i];
}

void oracle_ce_fwd(const void* x, int64_t ld, const int64_t* labels, int64_t rows,
                   int64_t cols, int64_t ignore, int dtype, float* rmax, float* rlse,
                   float* loss) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    float m = -INFINITY;
    for (int64_t j = 0; j < cols; ++j) {
      const float v = load_logit(x, r * ld + j, dtype);
      if (v > m || isnan(v)) m = v;
    }
    double acc = 0.0;
    for (int64_t j = 0; j < cols; ++j) acc += exp((double)load_logit(x, r * ld + j, dtype) - (double)m);
    const float lse = (float)log(acc);
    rmax[r] = m;
    rlse[r] = lse;
    const int64_t t = labels[r];
    if (t == ignore) {
      loss[r] = 0.0f;
    } else if (t < 0 || t >= cols) {
      loss[r] = NAN;
    } else {
      const float xt = load_logit(x, r * ld + t, dtype);
      loss[r] = -round_to((xt - m) - lse, dtype);
    }
  }
}

void oracle_ce_bwd(const void* x, int64_t ld, const int64_t* labels, const float* rmax,
                   const float* rlse, float grad, int64_t rows, int64_t cols, int64_t ignore,
                   int dtype, void* dx) {
  const float neg = round_to(-grad, dtype);
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t t = labels[r];
    const int bad = t != ignore && (t < 0 || t >= cols);
    for (int64_t j = 0; j < cols; ++j) {
      float d;
      if (t == ignore) {
        d = 0.0f;
      } else if (bad) {
        d = NAN;
      } else {
        const float logp = round_to((load_logit(x, r * ld + j, dtype) - rmax[r]) - rlse[r], dtype);
        d = (j == t ? neg : 0.0f) - expf(logp) * neg;
      }
      if (dtype == F16) ((uint16_t*)dx)[r * ld + j] = oracle_f32_to_f16(d);
      else ((float*)dx)[r * ld + j] = d;
    }
  }
}

/* ---- token + position embedding --------------------------------------- */

/* out[i] = tok[ids[i]] + pos[i % seq] (one fp32 add per element); an id
 * outside [0, vocab) gives a NaN row. */
void oracle_embed_fwd(const int64_t* ids, int64_t n, int64_t seq, const float* tok,
                      int64_t vocab, const float* pos, int64_t d, float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    const int64_t id = ids[i];
    const float* pr = pos + (i % seq) * d;
    float* o = out + i * d;
    if (id < 0 || id >= vocab) {
      for (int64_t c = 0; c < d; ++c) o[c] = NAN;
      continue;
    }
    const float* tr = tok + id * d;
    for (int64_t c = 0; c < d; ++c) o[c] = tr[c] + pr[c];
  }
}

/* dpos[t] = (dpos[t] if accumulate else 0) + (((0 + dout[0, t]) + dout[1, t])
 * + ...); rows seq <= t < max_seq are zeroed unless accumulating. */
void oracle_embed_bwd_pos(const float* dout, int64_t batch, int64_t seq, int64_t max_seq,
                          int64_t d, float* dpos, int accumulate) {
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < max_seq; ++t) {
    float* dst = dpos + t * d;
    if (t >= seq) {
      if (!accumulate)
        for (int64_t c = 0; c < d; ++c) dst[c] = 0.0f;
      continue;
    }
    for (int64_t c = 0; c < d; ++c) {
      float acc = 0.0f;
      for (int64_t b = 0; b < batch; ++b) acc = acc + dout[(b * seq + t) * d + c];
      dst[c] = accumulate ? dst[c] + acc : acc;
    }
  }
}

/* dtok[v] = (dtok[v] if accumulate else 0) + S_v, S_v the sum of the dout rows
 * of the occurrences of v in this order: the occurrences, in ascending token
 * index, are the run of v in the id-sorted token list; that list is cut into
 * blocks of `block` entries; each block's part of the run is summed from 0 in
 * order, and the parts are added left to right.  Ids outside [0, vocab)
 * contribute nothing. */
void oracle_embed_bwd_tok(const int64_t* ids, int64_t n, const float* dout, int64_t vocab,
                          int64_t d, int64_t block, float* dtok, int accumulate) {
  if (!accumulate)
    for (int64_t i = 0; i < vocab * d; ++i) dtok[i] = 0.0f;
  /* stable counting sort by id; invalid ids get key vocab (sorted last) */
  int64_t* start = (int64_t*)calloc((size_t)vocab + 2, sizeof(int64_t));
  int64_t* order = (int64_t*)malloc((size_t)(n > 0 ? n : 1) * sizeof(int64_t));
  for (int64_t i = 0; i < n; ++i) {
    const int64_t k = (ids[i] >= 0 && ids[i] < vocab) ? ids[i] : vocab;
    start[k + 1] += 1;
  }
  for (int64_t v = 0; v <= vocab; ++v) start[v + 1] += start[v];
  {
    int64_t* fill = (int64_t*)malloc(((size_t)vocab + 1) * sizeof(int64_t));
    memcpy(fill, start, ((size_t)vocab + 1) * sizeof(int64_t));
    for (int64_t i = 0; i < n; ++i) {
      const int64_t k = (ids[i] >= 0 && ids[i] < vocab) ? ids[i] : vocab;
      order[fill[k]++] = i;
    }
    free(fill);
  }
#pragma omp parallel for schedule(dynamic, 64)
  for (int64_t v = 0; v < vocab; ++v) {
    const int64_t a = start[v], b = start[v + 1];
    if (a == b) continue;
    for (int64_t c = 0; c < d; ++c) {
      float total = 0.0f;
      int first = 1;
      for (int64_t p0 = a; p0 < b;) {
        const int64_t p1 = ((p0 / block) + 1) * block < b ? ((p0 / block) + 1) * block : b;
        float part = 0.0f;
        for (int64_t p = p0; p < p1; ++p) part = part + dout[order[p] * d + c];
        total = first ? part : total + part;
        first = 0;
        p0 = p1;
      }
      dtok[v * d + c] = dtok[v * d + c] + total;
    }
  }
  free(order);
  free(start);
}
