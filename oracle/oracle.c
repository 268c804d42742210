/*
 * CPU oracle for the MI355X matmul / attention dispatch path.
 * TEST INFRASTRUCTURE ONLY: see oracle.h for who may use it and how each
 * routine is pinned. Built with -ffp-contract=off so every f32 multiply and
 * add rounds separately, in the order written.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- f16 ---- */

float oracle_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exponent = (h >> 10) & 0x1fu;
  uint32_t mantissa = h & 0x3ffu;
  uint32_t bits;
  if (exponent == 0) {
    if (mantissa == 0) {
      bits = sign;
    } else {
      /* subnormal: mantissa * 2^-24, exact in f32 */
      float value = ldexpf((float)mantissa, -24);
      memcpy(&bits, &value, 4);
      bits |= sign;
    }
  } else if (exponent == 31) {
    bits = sign | 0x7f800000u | (mantissa << 13);
  } else {
    bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
  }
  float out;
  memcpy(&out, &bits, 4);
  return out;
}

uint16_t oracle_f32_to_f16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t mag = u & 0x7fffffffu;
  if (mag >= 0x7f800000u) { /* inf, or nan keeping the top payload bits */
    uint32_t payload = (mag & 0x7fffffu) >> 13;
    if (mag > 0x7f800000u && payload == 0)
      payload = 0x200u;
    return (uint16_t)(sign | 0x7c00u | payload);
  }
  if (mag >= 0x477ff000u) /* >= 65520 rounds to inf */
    return (uint16_t)(sign | 0x7c00u);
  if (mag < 0x38800000u) { /* below 2^-14: half subnormal or zero */
    float value;
    memcpy(&value, &mag, 4);
    /* value * 2^24 is exact; nearbyintf rounds half to even */
    uint32_t m = (uint32_t)nearbyintf(value * 16777216.0f);
    return (uint16_t)(sign | m);
  }
  uint32_t h = (((mag >> 23) - 112u) << 10) | ((mag >> 13) & 0x3ffu);
  uint32_t rest = mag & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u)))
    ++h;
  return (uint16_t)(sign | h);
}

void oracle_f16_to_f32_array(const uint16_t *src, float *dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    dst[i] = oracle_f16_to_f32(src[i]);
}

void oracle_f32_to_f16_array(const float *src, uint16_t *dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    dst[i] = oracle_f32_to_f16(src[i]);
}

static int bad_dims(int64_t m, int64_t n, int64_t k) {
  return m < 0 || n < 0 || k < 0;
}

/* ------------------------------------------------ blocked k-order core ----
 * Every matmul below computes acc[i][j] = sum_k A[i][k] * B[k][j] with each
 * product rounded to f32 and added to the running sum in ascending k (integer
 * forms: exact products, sums modulo 2^32). Blocking over rows, columns and k
 * changes only which sums are in flight at once, never the operations of one
 * sum: a k block resumes the stored f32 (u32) partial exactly where the
 * previous block left it. B is packed into panels of NR columns, [panel][k][NR]
 * (columns past N zero), A into f32 rows [i][k]. */
#define OR_MR 6    /* rows per register block */
#define OR_NR 16   /* columns per panel (two 8-lane vectors) */
#define OR_KC 256  /* k per block */
#define OR_MC 48   /* rows per task */
#define OR_NC 256  /* columns per task */
typedef float or_v8f __attribute__((vector_size(32)));
typedef uint32_t or_v8u __attribute__((vector_size(32)));

static int64_t or_panels(int64_t n) { return (n + OR_NR - 1) / OR_NR; }

/* One register block: rows [0, rows) of `a` (row pitch lda, rows past `rows`
 * repeat the last, discarded on store) times one panel over k in [k0, k1),
 * resuming and storing the partial sums held in `ct` (row pitch OR_NC). */
static void or_block_f32(const float *a, int64_t lda, int rows,
                         const float *panel, int64_t k0, int64_t k1,
                         float *ct) {
  const float *ar[OR_MR];
  or_v8f c[OR_MR][2];
  for (int r = 0; r < OR_MR; ++r) {
    ar[r] = a + (r < rows ? r : rows - 1) * lda;
    memcpy(&c[r][0], ct + r * OR_NC, 32);
    memcpy(&c[r][1], ct + r * OR_NC + 8, 32);
  }
  for (int64_t kk = k0; kk < k1; ++kk) {
    or_v8f b0, b1;
    memcpy(&b0, panel + kk * OR_NR, 32);
    memcpy(&b1, panel + kk * OR_NR + 8, 32);
    for (int r = 0; r < OR_MR; ++r) {
      const or_v8f av = (or_v8f){0} + ar[r][kk];
      const or_v8f p0 = av * b0, p1 = av * b1;
      c[r][0] = c[r][0] + p0;
      c[r][1] = c[r][1] + p1;
    }
  }
  for (int r = 0; r < rows; ++r) {
    memcpy(ct + r * OR_NC, &c[r][0], 32);
    memcpy(ct + r * OR_NC + 8, &c[r][1], 32);
  }
}

static void or_block_u32(const uint32_t *a, int64_t lda, int rows,
                         const uint32_t *panel, int64_t k0, int64_t k1,
                         uint32_t *ct) {
  const uint32_t *ar[OR_MR];
  or_v8u c[OR_MR][2];
  for (int r = 0; r < OR_MR; ++r) {
    ar[r] = a + (r < rows ? r : rows - 1) * lda;
    memcpy(&c[r][0], ct + r * OR_NC, 32);
    memcpy(&c[r][1], ct + r * OR_NC + 8, 32);
  }
  for (int64_t kk = k0; kk < k1; ++kk) {
    or_v8u b0, b1;
    memcpy(&b0, panel + kk * OR_NR, 32);
    memcpy(&b1, panel + kk * OR_NR + 8, 32);
    for (int r = 0; r < OR_MR; ++r) {
      const or_v8u av = (or_v8u){0} + ar[r][kk];
      c[r][0] = c[r][0] + av * b0;
      c[r][1] = c[r][1] + av * b1;
    }
  }
  for (int r = 0; r < rows; ++r) {
    memcpy(ct + r * OR_NC, &c[r][0], 32);
    memcpy(ct + r * OR_NC + 8, &c[r][1], 32);
  }
}

/* acc [m][n] (pitch n) = A [m][k] . B-panels, 4-byte elements; `u32` picks
 * the integer form. Tasks are (48-row, 256-column) output tiles. */
static void or_gemm(const void *a, const void *bp, void *acc, int64_t m,
                    int64_t n, int64_t k, int u32, int threads) {
  const int64_t tm = (m + OR_MC - 1) / OR_MC, tn = (n + OR_NC - 1) / OR_NC;
  if (threads < 1)
    threads = 1;
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
  for (int64_t task = 0; task < tm * tn; ++task) {
    const int64_t i0 = (task / tn) * OR_MC, j0 = (task % tn) * OR_NC;
    const int64_t rows = m - i0 < OR_MC ? m - i0 : OR_MC;
    const int64_t cols = n - j0 < OR_NC ? n - j0 : OR_NC;
    uint32_t tile[OR_MC * OR_NC];
    memset(tile, 0, sizeof(tile));
    for (int64_t k0 = 0; k0 < k; k0 += OR_KC) {
      const int64_t k1 = k - k0 < OR_KC ? k : k0 + OR_KC;
      for (int64_t jp = 0; jp < cols; jp += OR_NR) {
        const int64_t panel = (j0 + jp) / OR_NR;
        for (int64_t ib = 0; ib < rows; ib += OR_MR) {
          const int r = (int)(rows - ib < OR_MR ? rows - ib : OR_MR);
          if (u32)
            or_block_u32((const uint32_t *)a + (i0 + ib) * k, k, r,
                         (const uint32_t *)bp + panel * k * OR_NR, k0, k1,
                         tile + ib * OR_NC + jp);
          else
            or_block_f32((const float *)a + (i0 + ib) * k, k, r,
                         (const float *)bp + panel * k * OR_NR, k0, k1,
                         (float *)tile + ib * OR_NC + jp);
        }
      }
    }
    for (int64_t i = 0; i < rows; ++i)
      memcpy((uint32_t *)acc + (i0 + i) * n + j0, tile + i * OR_NC,
             (size_t)cols * 4);
  }
}

/* Element (i, j) of a 2-D operand stored row-major with pitch ld, or
 * transposed (element (i, j) at j * ld + i). */
#define OR_AT(p, i, j, ld, t) ((t) ? (p)[(j) * (ld) + (i)] : (p)[(i) * (ld) + (j)])

/* B [K][N] (or [N][K] when transposed) of f16 / int8 as f32 / u32 panels. */
static void *or_pack_b(const void *b, int64_t n, int64_t k, int64_t ldb,
                       int transposed, int kind /* 0 f16, 1 i8->f32, 2 i8->u32 */,
                       int threads) {
  const int64_t np = or_panels(n);
  uint32_t *out = (uint32_t *)calloc((size_t)(np * k * OR_NR + 1), 4);
  if (!out)
    return NULL;
  if (threads < 1)
    threads = 1;
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t p = 0; p < np; ++p)
    for (int64_t kk = 0; kk < k; ++kk)
      for (int64_t c = 0; c < OR_NR && p * OR_NR + c < n; ++c) {
        const int64_t j = p * OR_NR + c;
        uint32_t *dst = out + (p * k + kk) * OR_NR + c;
        if (kind == 0) {
          const float f = oracle_f16_to_f32(
              OR_AT((const uint16_t *)b, kk, j, ldb, transposed));
          memcpy(dst, &f, 4);
        } else {
          const int8_t v = OR_AT((const int8_t *)b, kk, j, ldb, transposed);
          if (kind == 1) {
            const float f = (float)v;
            memcpy(dst, &f, 4);
          } else {
            *dst = (uint32_t)(int32_t)v;
          }
        }
      }
  return out;
}

/* A [M][K] (or [K][M] when transposed) as f32 / u32 rows [i][k]. */
static void *or_pack_a(const void *a, int64_t m, int64_t k, int64_t lda,
                       int transposed, int kind /* 0 f16, 2 i8->u32 */,
                       int threads) {
  uint32_t *out = (uint32_t *)malloc((size_t)(m * k + 1) * 4);
  if (!out)
    return NULL;
  if (threads < 1)
    threads = 1;
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t i = 0; i < m; ++i)
    for (int64_t kk = 0; kk < k; ++kk) {
      uint32_t *dst = out + i * k + kk;
      if (kind == 0) {
        const float f =
            oracle_f16_to_f32(OR_AT((const uint16_t *)a, i, kk, lda, transposed));
        memcpy(dst, &f, 4);
      } else {
        *dst = (uint32_t)(int32_t)OR_AT((const int8_t *)a, i, kk, lda, transposed);
      }
    }
  return out;
}

/* --------------------------------------------------------- matmul f16 ---- */

int oracle_matmul_f16(const uint16_t *a, const uint16_t *b, void *c,
                      int64_t m, int64_t n, int64_t k, int64_t lda,
                      int64_t ldb, int64_t ldc, uint32_t flags, int threads) {
  if (bad_dims(m, n, k))
    return 1;
  const int transposed = (flags & ORACLE_B_TRANSPOSED) != 0;
  const int a_t = (flags & ORACLE_A_TRANSPOSED) != 0;
  const int accumulate = (flags & ORACLE_ACCUMULATE) != 0;
  const int out_f32 = (flags & ORACLE_OUT_F32) != 0;
  float *af = (float *)or_pack_a(a, m, k, lda, a_t, 0, threads);
  float *bf = (float *)or_pack_b(b, n, k, ldb, transposed, 0, threads);
  float *acc = (float *)malloc(sizeof(float) * (size_t)(m * n + 1));
  if (!af || !bf || !acc) {
    free(af);
    free(bf);
    free(acc);
    return 2;
  }
  or_gemm(af, bf, acc, m, n, k, 0, threads);
  for (int64_t mm = 0; mm < m; ++mm)
    for (int64_t nn = 0; nn < n; ++nn) {
      const float s = acc[mm * n + nn];
      if (out_f32) {
        float *cp = (float *)c + mm * ldc + nn;
        *cp = accumulate ? *cp + s : s;
      } else {
        uint16_t *cp = (uint16_t *)c + mm * ldc + nn;
        *cp = oracle_f32_to_f16(accumulate ? oracle_f16_to_f32(*cp) + s : s);
      }
    }
  free(af);
  free(bf);
  free(acc);
  return 0;
}

/* ------------------------------------------- fused epilogue / batches ---- */

/* act(v) in f32 (double for the transcendental). GELU is the tanh form of the
 * reference's epilogue fusion test (LIT/codegen/pipelines/
 * hexagon_hmx_epilogue_keeps_config.mlir); SiLU is v / (1 + e^-v). */
float oracle_activation(float v, uint32_t act) {
  switch (act) {
    case ORACLE_ACT_RELU:
      return v > 0.0f ? v : 0.0f;
    case ORACLE_ACT_GELU_TANH: {
      const double x = v;
      return (float)(0.5 * x *
                     (1.0 + tanh(0.7978845608028654 * (x + 0.044715 * x * x * x))));
    }
    case ORACLE_ACT_SILU:
      return (float)((double)v / (1.0 + exp(-(double)v)));
    default:
      return v;
  }
}

int oracle_batch_matmul_f16(const uint16_t *a, const uint16_t *b, void *c,
                            int64_t batch, int64_t m, int64_t n, int64_t k,
                            int64_t lda, int64_t ldb, int64_t ldc, int64_t sa,
                            int64_t sb, int64_t sc, uint32_t flags,
                            const uint16_t *bias, const uint16_t *mul,
                            int64_t ld_mul, int64_t s_mul, uint32_t act,
                            int threads) {
  if (bad_dims(m, n, k) || batch < 0)
    return 1;
  const int out_f32 = (flags & ORACLE_OUT_F32) != 0;
  const int accumulate = (flags & ORACLE_ACCUMULATE) != 0;
  float *acc = (float *)malloc(sizeof(float) * (size_t)(m * n + 1));
  if (!acc)
    return 2;
  for (int64_t z = 0; z < batch; ++z) {
    /* f32 sums of this batch: the plain matmul into an f32 scratch */
    int rc = oracle_matmul_f16(
        a + z * sa, b + z * sb, acc, m, n, k, lda, ldb, n,
        (flags & (ORACLE_B_TRANSPOSED | ORACLE_A_TRANSPOSED)) | ORACLE_OUT_F32,
        threads);
    if (rc) {
      free(acc);
      return rc;
    }
    for (int64_t i = 0; i < m; ++i)
      for (int64_t j = 0; j < n; ++j) {
        float v = acc[i * n + j];
        if (bias)
          v += oracle_f16_to_f32(bias[j]);
        v = oracle_activation(v, act);
        if (mul)
          v *= oracle_f16_to_f32(mul[z * s_mul + i * ld_mul + j]);
        if (out_f32) {
          float *cp = (float *)c + z * sc + i * ldc + j;
          *cp = accumulate ? *cp + v : v;
        } else {
          uint16_t *cp = (uint16_t *)c + z * sc + i * ldc + j;
          *cp = oracle_f32_to_f16(accumulate ? oracle_f16_to_f32(*cp) + v : v);
        }
      }
  }
  free(acc);
  return 0;
}

/* The reference's GeGLU epilogue exactly as its IR states it
 * (LIT/codegen/pipelines/hexagon_hmx_epilogue_keeps_config.mlir:82-101):
 * h = f16(acc), then every op in f16 (each result rounded to f16):
 * g = h * 0.5 * (1 + tanh(k0 * (h + k1 * h^3))) with the f16 constants
 * k0 = 0.797852, k1 = 0.044708, out = g * up. */
uint16_t oracle_geglu_f16_ops(float acc, uint16_t up) {
#define R16(x) oracle_f16_to_f32(oracle_f32_to_f16((float)(x)))
  const float k0 = R16(7.978520e-01f), k1 = R16(4.470830e-02f);
  const float h = R16(acc);
  const float h3 = R16(R16(h * h) * h);
  const float t0 = R16(h3 * k1);
  const float t1 = R16(h + t0);
  const float t2 = R16(t1 * k0);
  const float t3 = R16(tanh((double)t2));
  const float t4 = R16(t3 + 1.0f);
  const float t5 = R16(t4 * 0.5f);
  const float g = R16(h * t5);
  return oracle_f32_to_f16(g * oracle_f16_to_f32(up));
#undef R16
}

/* ---------------------------------------------------------- matmul i8 ---- */

int oracle_matmul_i8(const int8_t *a, const int8_t *b, int32_t *c, int64_t m,
                     int64_t n, int64_t k, int64_t lda, int64_t ldb,
                     int64_t ldc, uint32_t flags, int threads) {
  if (bad_dims(m, n, k))
    return 1;
  const int transposed = (flags & ORACLE_B_TRANSPOSED) != 0;
  const int accumulate = (flags & ORACLE_ACCUMULATE) != 0;
  uint32_t *ai = (uint32_t *)or_pack_a(a, m, k, lda, 0, 2, threads);
  uint32_t *bi = (uint32_t *)or_pack_b(b, n, k, ldb, transposed, 2, threads);
  uint32_t *acc = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)(m * n + 1));
  if (!ai || !bi || !acc) {
    free(ai);
    free(bi);
    free(acc);
    return 2;
  }
  or_gemm(ai, bi, acc, m, n, k, 1, threads);
  for (int64_t mm = 0; mm < m; ++mm)
    for (int64_t nn = 0; nn < n; ++nn) {
      int32_t *cp = c + mm * ldc + nn;
      /* wrap like two's-complement i32 hardware adds */
      *cp = (int32_t)((accumulate ? (uint32_t)*cp : 0u) + acc[mm * n + nn]);
    }
  free(ai);
  free(bi);
  free(acc);
  return 0;
}

/* -------------------------------------------------------------- w8a16 ---- */

int oracle_w8a16(const uint16_t *x, const int8_t *w, const uint16_t *scale,
                 uint16_t *y, int64_t m, int64_t n, int64_t k, int64_t ldx,
                 int64_t ldw, int64_t ldy, uint32_t flags, int threads) {
  if (bad_dims(m, n, k))
    return 1;
  const int transposed = (flags & ORACLE_B_TRANSPOSED) != 0;
  float *xf = (float *)or_pack_a(x, m, k, ldx, 0, 0, threads);
  float *wf = (float *)or_pack_b(w, n, k, ldw, transposed, 1, threads);
  float *acc = (float *)malloc(sizeof(float) * (size_t)(m * n + 1));
  if (!xf || !wf || !acc) {
    free(xf);
    free(wf);
    free(acc);
    return 2;
  }
  or_gemm(xf, wf, acc, m, n, k, 0, threads);
  for (int64_t mm = 0; mm < m; ++mm)
    for (int64_t nn = 0; nn < n; ++nn)
      y[mm * ldy + nn] =
          oracle_f32_to_f16(acc[mm * n + nn] * oracle_f16_to_f32(scale[nn]));
  free(xf);
  free(wf);
  free(acc);
  return 0;
}

/* ---------------------------------------------------------- attention ---- */

int oracle_attention(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                     void *o, const uint16_t *mask, int64_t batch,
                     int64_t heads, int64_t kv_heads, int64_t seq_q,
                     int64_t seq_kv, int64_t head_dim, int64_t head_dim_v,
                     const int64_t strides[12], const int64_t mask_strides[4],
                     float scale, int causal, int out_f32, int threads) {
  if (batch < 0 || heads < 0 || kv_heads <= 0 || seq_q < 0 || seq_kv < 0 ||
      head_dim < 0 || head_dim_v < 0 || heads % kv_heads != 0)
    return 1;
  const int64_t group = heads / kv_heads;
  const int64_t *qs = strides, *ks = strides + 3, *vs = strides + 6,
                *os = strides + 9;
  if (threads < 1)
    threads = 1;
#pragma omp parallel for num_threads(threads) schedule(dynamic)
  for (int64_t row = 0; row < batch * heads * seq_q; ++row) {
    const int64_t plane = row / seq_q;
    const int64_t i = row % seq_q;
    const int64_t b = plane / heads, h = plane % heads, hk = h / group;
    const uint16_t *qi = q + b * qs[0] + h * qs[1] + i * qs[2];
    const uint16_t *kp = k + b * ks[0] + hk * ks[1];
    const uint16_t *vp = v + b * vs[0] + hk * vs[1];
    const uint16_t *mi =
        mask ? mask + b * mask_strides[0] + h * mask_strides[1] +
                   i * mask_strides[2]
             : NULL;
    float *qf = (float *)malloc(sizeof(float) * (size_t)(head_dim + 1));
    float *s = (float *)malloc(sizeof(float) * (size_t)(seq_kv + 1));
    float *acc = (float *)calloc((size_t)head_dim_v + 1, sizeof(float));
    for (int64_t d = 0; d < head_dim; ++d)
      qf[d] = oracle_f16_to_f32(qi[d]);
    /* top-left causal: key j is seen by query i when j <= i */
    const int64_t last = causal ? (i < seq_kv ? i : seq_kv - 1) : seq_kv - 1;
    float mx = -INFINITY;
    for (int64_t j = 0; j <= last; ++j) {
      float dot = 0.0f;
      for (int64_t d = 0; d < head_dim; ++d) {
        float prod = qf[d] * oracle_f16_to_f32(kp[j * ks[2] + d]);
        dot = dot + prod;
      }
      s[j] = dot * scale;
      if (mi)
        s[j] = s[j] + oracle_f16_to_f32(mi[j * mask_strides[3]]);
      if (s[j] > mx)
        mx = s[j];
    }
    /* keys whose score is -inf (masked) weigh 0; a row with no other key
     * writes 0 (the all-masked guard, attention_layer.mlir:80-102) */
    float sum = 0.0f;
    for (int64_t j = 0; j <= last && mx != -INFINITY; ++j) {
      if (s[j] == -INFINITY)
        continue;
      float p = expf(s[j] - mx);
      sum = sum + p;
      for (int64_t d = 0; d < head_dim_v; ++d) {
        float prod = p * oracle_f16_to_f32(vp[j * vs[2] + d]);
        acc[d] = acc[d] + prod;
      }
    }
    const int64_t at = b * os[0] + h * os[1] + i * os[2];
    for (int64_t d = 0; d < head_dim_v; ++d) {
      const float val = sum > 0.0f ? acc[d] / sum : 0.0f;
      if (out_f32)
        ((float *)o)[at + d] = val;
      else
        ((uint16_t *)o)[at + d] = oracle_f32_to_f16(val);
    }
    free(qf);
    free(s);
    free(acc);
  }
  return 0;
}

int oracle_attention_f16_strided(const uint16_t *q, const uint16_t *k,
                                 const uint16_t *v, uint16_t *o,
                                 int64_t batch, int64_t heads,
                                 int64_t kv_heads, int64_t seq_q,
                                 int64_t seq_kv, int64_t head_dim,
                                 const int64_t strides[12], float scale,
                                 int causal, int threads) {
  const int64_t none[4] = {0, 0, 0, 0};
  return oracle_attention(q, k, v, o, NULL, batch, heads, kv_heads, seq_q,
                          seq_kv, head_dim, head_dim, strides, none, scale,
                          causal, 0, threads);
}

int oracle_attention_f16(const uint16_t *q, const uint16_t *k,
                         const uint16_t *v, uint16_t *o, int64_t batch,
                         int64_t heads, int64_t seq_q, int64_t seq_kv,
                         int64_t head_dim, float scale, int causal,
                         int threads) {
  if (batch < 0 || heads < 0 || seq_q < 0 || seq_kv < 0 || head_dim < 0)
    return 1;
  if (heads == 0)
    return 0;
  const int64_t st[12] = {heads * seq_q * head_dim,  seq_q * head_dim,
                          head_dim,                  heads * seq_kv * head_dim,
                          seq_kv * head_dim,         head_dim,
                          heads * seq_kv * head_dim, seq_kv * head_dim,
                          head_dim,                  heads * seq_q * head_dim,
                          seq_q * head_dim,          head_dim};
  return oracle_attention_f16_strided(q, k, v, o, batch, heads, heads, seq_q,
                                      seq_kv, head_dim, st, scale, causal,
                                      threads);
}

/* ------------------------------------------------------------ planner ---- */

int64_t oracle_choose_static_tiling_factor(int64_t static_bound,
                                           int64_t preferred,
                                           int64_t multiple_of) {
  if (preferred <= 0)
    return 0;
  if (static_bound == INT64_MIN) /* dynamic */
    return preferred;
  int64_t fallback = static_bound < preferred ? static_bound : preferred;
  int64_t step = multiple_of > 1 ? multiple_of : 1;
  if (static_bound <= 0 || static_bound % step != 0 || preferred < step)
    return fallback;
  /* divisors d of bound/step, scanned from the large end: the first large
   * cofactor within the preferred size wins, then the small divisors */
  int64_t bound = static_bound / step;
  int64_t pref = preferred / step;
  int64_t small = 1;
  for (; small <= bound / small; ++small) {
    if (bound % small != 0)
      continue;
    if (bound / small <= pref)
      return (bound / small) * step;
  }
  for (--small; small >= 1; --small)
    if (bound % small == 0 && small <= pref)
      return small * step;
  return fallback;
}

/* Tile candidates of a dimension: HMX-aligned divisors, else the extent. */
static int hmx_candidates(int64_t extent, int64_t hmx_tile, int64_t *out,
                          int cap) {
  int count = 0;
  for (int64_t t = hmx_tile; t <= extent && count < cap; t += hmx_tile)
    if (extent % t == 0)
      out[count++] = t;
  if (count == 0)
    out[count++] = extent;
  return count;
}

int oracle_select_hmx_tile_sizes(const int64_t ranges[3],
                                 const int64_t elem_bytes[3], int b_transposed,
                                 int64_t budget_flag_bytes,
                                 int double_buffering, int64_t hmx_m,
                                 int64_t hmx_n, int64_t tiles[3]) {
  enum { DM = 0, DN = 1, DK = 2 };
  for (int i = 0; i < 3; ++i)
    if (ranges[i] <= 0)
      return 0;
  /* KernelDispatch.cpp:19-23 halves the flag budget when double buffering;
   * VTCMPlanning.cpp:205-208 doubles it back for this search. */
  int64_t options_budget = double_buffering ? budget_flag_bytes / 2
                                            : budget_flag_bytes;
  int64_t budget = options_budget * (double_buffering ? 2 : 1);
  const int64_t max_overrun = 2; /* VTCMPlanning.cpp:212 */
  /* operand indexing maps over (d0=m, d1=n, d2=k) */
  int maps[3][2] = {{DM, DK},
                    {b_transposed ? DN : DK, b_transposed ? DK : DN},
                    {DM, DN}};
  int64_t mc[4096], nc[4096];
  int nm = hmx_candidates(ranges[DM], hmx_m, mc, 4096);
  int nn = hmx_candidates(ranges[DN], hmx_n, nc, 4096);
  int found = 0;
  int64_t best_rank[4] = {0, 0, 0, 0};
  for (int i = 0; i < nm; ++i) {
    for (int j = 0; j < nn; ++j) {
      int64_t t[3] = {mc[i], nc[j], ranges[DK]};
      int64_t num_tiles = 1;
      for (int d = 0; d < 3; ++d)
        num_tiles *= ranges[d] / t[d];
      int64_t vtcm = 0, traffic = 0;
      for (int op = 0; op < 3; ++op) {
        int64_t bytes = elem_bytes[op];
        int invariant = 1;
        for (int r = 0; r < 2; ++r) {
          bytes *= t[maps[op][r]];
          if (t[maps[op][r]] != ranges[maps[op][r]])
            invariant = 0;
        }
        vtcm += (double_buffering && !invariant) ? 2 * bytes : bytes;
        traffic += invariant ? bytes : bytes * num_tiles;
      }
      if (vtcm > max_overrun * budget)
        continue;
      /* rank: (over budget, traffic, number of tiles, -N), lexicographic */
      int64_t rank[4] = {vtcm > budget ? 1 : 0, traffic, num_tiles, -t[DN]};
      int better = !found;
      for (int r = 0; r < 4 && !better; ++r) {
        if (rank[r] < best_rank[r]) {
          better = 1;
          break;
        }
        if (rank[r] > best_rank[r])
          break;
      }
      if (!better)
        continue;
      found = 1;
      memcpy(best_rank, rank, sizeof(rank));
      memcpy(tiles, t, sizeof(t));
    }
  }
  return found;
}

