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

/* B as f32 in [K][N] order (transposing a [N][K] operand), so every matmul
 * below runs the same row-update loop and sums each output in k order. */
static float *widen_b_f16(const uint16_t *b, int64_t n, int64_t k, int64_t ldb,
                          int transposed) {
  float *out = (float *)malloc(sizeof(float) * (size_t)(n * k + 1));
  if (!out)
    return NULL;
  for (int64_t kk = 0; kk < k; ++kk)
    for (int64_t nn = 0; nn < n; ++nn)
      out[kk * n + nn] = oracle_f16_to_f32(transposed ? b[nn * ldb + kk]
                                                      : b[kk * ldb + nn]);
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
  /* A [K,M] (transposed LHS): element (m, k) at k * lda + m. */
  const int64_t a_rs = a_t ? 1 : lda, a_ks = a_t ? lda : 1;
  float *bf = widen_b_f16(b, n, k, ldb, transposed);
  if (!bf)
    return 2;
  if (threads < 1)
    threads = 1;
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t mm = 0; mm < m; ++mm) {
    float *acc = (float *)calloc((size_t)n + 1, sizeof(float));
    for (int64_t kk = 0; kk < k; ++kk) {
      const float av = oracle_f16_to_f32(a[mm * a_rs + kk * a_ks]);
      const float *brow = bf + kk * n;
      for (int64_t nn = 0; nn < n; ++nn) {
        float prod = av * brow[nn];
        acc[nn] = acc[nn] + prod;
      }
    }
    for (int64_t nn = 0; nn < n; ++nn) {
      if (out_f32) {
        float *cp = (float *)c + mm * ldc + nn;
        *cp = accumulate ? *cp + acc[nn] : acc[nn];
      } else {
        uint16_t *cp = (uint16_t *)c + mm * ldc + nn;
        float init = accumulate ? oracle_f16_to_f32(*cp) : 0.0f;
        *cp = oracle_f32_to_f16(accumulate ? init + acc[nn] : acc[nn]);
      }
    }
    free(acc);
  }
  free(bf);
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
  int32_t *bi = (int32_t *)malloc(sizeof(int32_t) * (size_t)(n * k + 1));
  if (!bi)
    return 2;
  for (int64_t kk = 0; kk < k; ++kk)
    for (int64_t nn = 0; nn < n; ++nn)
      bi[kk * n + nn] = transposed ? b[nn * ldb + kk] : b[kk * ldb + nn];
  if (threads < 1)
    threads = 1;
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t mm = 0; mm < m; ++mm) {
    int32_t *acc = (int32_t *)calloc((size_t)n + 1, sizeof(int32_t));
    for (int64_t kk = 0; kk < k; ++kk) {
      const int32_t av = a[mm * lda + kk];
      const int32_t *brow = bi + kk * n;
      for (int64_t nn = 0; nn < n; ++nn)
        acc[nn] += av * brow[nn];
    }
    for (int64_t nn = 0; nn < n; ++nn) {
      int32_t *cp = c + mm * ldc + nn;
      /* wrap like two's-complement i32 hardware adds */
      *cp = accumulate ? (int32_t)((uint32_t)*cp + (uint32_t)acc[nn]) : acc[nn];
    }
    free(acc);
  }
  free(bi);
  return 0;
}

/* -------------------------------------------------------------- w8a16 ---- */

int oracle_w8a16(const uint16_t *x, const int8_t *w, const uint16_t *scale,
                 uint16_t *y, int64_t m, int64_t n, int64_t k, int64_t ldx,
                 int64_t ldw, int64_t ldy, uint32_t flags, int threads) {
  if (bad_dims(m, n, k))
    return 1;
  const int transposed = (flags & ORACLE_B_TRANSPOSED) != 0;
  float *wf = (float *)malloc(sizeof(float) * (size_t)(n * k + 1));
  if (!wf)
    return 2;
  for (int64_t kk = 0; kk < k; ++kk)
    for (int64_t nn = 0; nn < n; ++nn)
      wf[kk * n + nn] = (float)(transposed ? w[nn * ldw + kk] : w[kk * ldw + nn]);
  if (threads < 1)
    threads = 1;
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t mm = 0; mm < m; ++mm) {
    float *acc = (float *)calloc((size_t)n + 1, sizeof(float));
    for (int64_t kk = 0; kk < k; ++kk) {
      const float xv = oracle_f16_to_f32(x[mm * ldx + kk]);
      const float *wrow = wf + kk * n;
      for (int64_t nn = 0; nn < n; ++nn) {
        float prod = xv * wrow[nn];
        acc[nn] = acc[nn] + prod;
      }
    }
    for (int64_t nn = 0; nn < n; ++nn)
      y[mm * ldy + nn] =
          oracle_f32_to_f16(acc[nn] * oracle_f16_to_f32(scale[nn]));
    free(acc);
  }
  free(wf);
  return 0;
}

/* ---------------------------------------------------------- attention ---- */

int oracle_attention_f16(const uint16_t *q, const uint16_t *k,
                         const uint16_t *v, uint16_t *o, int64_t batch,
                         int64_t heads, int64_t seq_q, int64_t seq_kv,
                         int64_t head_dim, float scale, int causal,
                         int threads) {
  if (batch < 0 || heads < 0 || seq_q < 0 || seq_kv < 0 || head_dim < 0)
    return 1;
  const int64_t planes = batch * heads;
  if (threads < 1)
    threads = 1;
#pragma omp parallel for num_threads(threads) schedule(dynamic)
  for (int64_t row = 0; row < planes * seq_q; ++row) {
    const int64_t plane = row / seq_q;
    const int64_t i = row % seq_q;
    const uint16_t *qi = q + (plane * seq_q + i) * head_dim;
    const uint16_t *kp = k + plane * seq_kv * head_dim;
    const uint16_t *vp = v + plane * seq_kv * head_dim;
    float *qf = (float *)malloc(sizeof(float) * (size_t)(head_dim + 1));
    float *s = (float *)malloc(sizeof(float) * (size_t)(seq_kv + 1));
    float *acc = (float *)calloc((size_t)head_dim + 1, sizeof(float));
    for (int64_t d = 0; d < head_dim; ++d)
      qf[d] = oracle_f16_to_f32(qi[d]);
    const int64_t last = causal ? (i < seq_kv ? i : seq_kv - 1) : seq_kv - 1;
    float mx = -INFINITY;
    for (int64_t j = 0; j <= last; ++j) {
      float dot = 0.0f;
      for (int64_t d = 0; d < head_dim; ++d) {
        float prod = qf[d] * oracle_f16_to_f32(kp[j * head_dim + d]);
        dot = dot + prod;
      }
      s[j] = dot * scale;
      if (s[j] > mx)
        mx = s[j];
    }
    float sum = 0.0f;
    for (int64_t j = 0; j <= last; ++j) {
      float p = expf(s[j] - mx);
      sum = sum + p;
      for (int64_t d = 0; d < head_dim; ++d) {
        float prod = p * oracle_f16_to_f32(vp[j * head_dim + d]);
        acc[d] = acc[d] + prod;
      }
    }
    uint16_t *oi = o + (plane * seq_q + i) * head_dim;
    for (int64_t d = 0; d < head_dim; ++d)
      oi[d] = oracle_f32_to_f16(last >= 0 ? acc[d] / sum : 0.0f);
    free(qf);
    free(s);
    free(acc);
  }
  return 0;
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

/* --------------------------------------------------------------- pack ---- */

void oracle_hmx_pack_f16(uint16_t *dest, const uint16_t *src,
                         uint32_t src_stride, uint32_t rows, uint32_t cols,
                         uint32_t row_tiles, uint32_t col_tiles) {
  const uint32_t tile = 32, tile_elems = 1024;
  memset(dest, 0, (size_t)row_tiles * col_tiles * tile_elems * 2);
  for (uint32_t r = 0; r < rows; ++r) {
    for (uint32_t c = 0; c < cols; ++c) {
      uint32_t rt = r / tile, ct = c / tile;
      if (rt >= row_tiles || ct >= col_tiles)
        continue;
      uint32_t tr = r % tile, tc = c % tile;
      dest[(rt * col_tiles + ct) * tile_elems + (tr / 2u) * 64u + 2u * tc +
           (tr & 1u)] = src[(size_t)r * src_stride + c];
    }
  }
}
