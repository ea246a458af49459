/*
 * oracle.c -- CPU restatement of the reference's causal GQA prefill attention path.
 *
 * TEST INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg as the checker, never by the product.  See oracle.h for the function list,
 * the reference lines each one follows and what pins it.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define HQ 16
#define HKV 8
#define HD 128

/* ------------------------------------------------------------------------------------------ */
/* fp16 codec                                                                                  */
/* ------------------------------------------------------------------------------------------ */

uint16_t orc_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
  if (ax >= 0x47800000u) return (uint16_t)(sign | 0x7c00u); /* >= 65536: Inf */
  if (ax < 0x38800000u) {                                    /* below 2^-14: subnormal or 0 */
    float a;
    memcpy(&a, &ax, 4);
    double scaled = (double)a * 16777216.0; /* exact: |a| * 2^24 < 1024 */
    return (uint16_t)(sign | (uint32_t)nearbyint(scaled)); /* RNE; 1024 -> min normal */
  }
  uint32_t e = (ax >> 23) - 127 + 15;
  uint32_t m = ax & 0x7fffffu;
  uint32_t h = (e << 10) | (m >> 13);
  uint32_t rem = m & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1; /* carry may reach Inf: correct */
  return (uint16_t)(sign | h);
}

float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu;
  uint32_t m = h & 0x3ffu;
  uint32_t x;
  if (e == 0) {
    float v = (float)m * 5.9604644775390625e-08f; /* m * 2^-24, exact */
    memcpy(&x, &v, 4);
    x |= sign;
  } else if (e == 31) {
    x = sign | 0x7f800000u | (m << 13);
  } else {
    x = sign | ((e - 15 + 127) << 23) | (m << 13);
  }
  float out;
  memcpy(&out, &x, 4);
  return out;
}

/* src/math/f16.ts:4-25, restated statement by statement. */
uint16_t orc_ref_float_to_half(float value) {
  uint32_t bits;
  memcpy(&bits, &value, 4);
  uint32_t sign = (bits >> 16) & 0x8000u;
  int32_t exponent = (int32_t)((bits >> 23) & 0xffu) - 127 + 15;
  uint32_t mantissa = bits & 0x7fffffu;
  if (exponent <= 0) {
    if (exponent < -10) return (uint16_t)sign;
    mantissa = (mantissa | 0x800000u) >> (uint32_t)(1 - exponent);
    return (uint16_t)(sign | ((mantissa + 0x1000u) >> 13));
  }
  if (exponent >= 31) return (uint16_t)(sign | 0x7c00u);
  if (mantissa & 0x1000u) {
    mantissa += 0x2000u;
    if (mantissa & 0x800000u) {
      mantissa = 0;
      exponent += 1;
      if (exponent >= 31) return (uint16_t)(sign | 0x7c00u);
    }
  }
  return (uint16_t)(sign | ((uint32_t)exponent << 10) | (mantissa >> 13));
}

/* src/gguf/quantization.ts:2-9. */
double orc_ref_half_to_float(uint16_t bits) {
  double sign = (bits & 0x8000u) ? -1.0 : 1.0;
  uint32_t exponent = (bits >> 10) & 0x1fu;
  uint32_t fraction = bits & 0x3ffu;
  if (exponent == 0) return sign * ldexp(1.0, -14) * ((double)fraction / 1024.0);
  if (exponent == 0x1f) return fraction ? NAN : sign * INFINITY;
  return sign * ldexp(1.0, (int)exponent - 15) * (1.0 + (double)fraction / 1024.0);
}

/* f16 rounding of an exactly representable (or f64-rounded) value.  Rounding f64 -> f32 -> f16
 * is a double rounding, so go straight from f64 to f16 here. */
static inline double r16(double x) {
  /* Round x to the nearest binary16 (RNE), return it as a double. */
  double ax = fabs(x);
  if (ax >= 65520.0) return x > 0 ? INFINITY : -INFINITY;
  if (ax < 6.103515625e-05) { /* subnormal spacing 2^-24 */
    return nearbyint(x * 16777216.0) / 16777216.0;
  }
  int e;
  frexp(ax, &e);                   /* ax = f * 2^e, f in [0.5,1) */
  double ulp = ldexp(1.0, e - 11); /* 11 significant bits */
  return nearbyint(x / ulp) * ulp;
}

static inline double h2d(uint16_t h) { return (double)orc_f16_to_f32(h); }

/* ------------------------------------------------------------------------------------------ */
/* generator                                                                                   */
/* ------------------------------------------------------------------------------------------ */

static inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

uint64_t orc_rand_u64(uint64_t seed, uint64_t i) {
  return mix64(seed + (i + 1) * 0x9E3779B97F4A7C15ULL);
}

double orc_normal(uint64_t seed, uint64_t e) {
  uint64_t j = e >> 1;
  double u1 = (double)((orc_rand_u64(seed, 2 * j) >> 11) + 1) * 0x1.0p-53; /* (0, 1] */
  double u2 = (double)(orc_rand_u64(seed, 2 * j + 1) >> 11) * 0x1.0p-53;   /* [0, 1) */
  double r = sqrt(-2.0 * log(u1));
  double th = 6.283185307179586 * u2;
  return (e & 1) ? r * sin(th) : r * cos(th);
}

uint64_t orc_seed(uint32_t config, uint32_t layer, uint32_t tensor) {
  return 0x51574E3300000000ULL | ((uint64_t)(config & 0xff) << 16) |
         ((uint64_t)(layer & 0xff) << 8) | (uint64_t)(tensor & 0xff);
}

void orc_gen_normal_f16(uint64_t seed, int64_t n, uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = orc_f32_to_f16((float)orc_normal(seed, (uint64_t)i));
}

void orc_rope_table(int32_t npos, double theta, float* cos_out, float* sin_out) {
  for (int32_t p = 0; p < npos; ++p)
    for (int32_t i = 0; i < 64; ++i) {
      double angle = (double)p * pow(theta, -(double)i / 64.0);
      cos_out[p * 64 + i] = (float)cos(angle);
      sin_out[p * 64 + i] = (float)sin(angle);
    }
}

void orc_qk_norm_rope(uint16_t* x, int64_t stride, int64_t col0, int32_t heads,
                      const int32_t* cu, int32_t nseq, const float* weight, double eps,
                      double theta) {
  int32_t maxlen = 0;
  for (int32_t s = 0; s < nseq; ++s)
    if (cu[s + 1] - cu[s] > maxlen) maxlen = cu[s + 1] - cu[s];
  float* cs = (float*)malloc(sizeof(float) * (size_t)(maxlen > 0 ? maxlen : 1) * 64);
  float* sn = (float*)malloc(sizeof(float) * (size_t)(maxlen > 0 ? maxlen : 1) * 64);
  orc_rope_table(maxlen, theta, cs, sn);
  for (int32_t s = 0; s < nseq; ++s) {
    int64_t t0 = cu[s], t1 = cu[s + 1];
#pragma omp parallel for schedule(static)
    for (int64_t t = t0; t < t1; ++t) {
      int64_t pos = t - t0;
      for (int32_t h = 0; h < heads; ++h) {
        uint16_t* v = x + t * stride + col0 + (int64_t)h * HD;
        double ss = 0.0;
        for (int d = 0; d < HD; ++d) {
          double xd = h2d(v[d]);
          ss = ss + xd * xd;
        }
        double inv = 1.0 / sqrt(ss / 128.0 + eps);
        float n[HD];
        for (int d = 0; d < HD; ++d) {
          double w = weight ? (double)weight[d] : 1.0;
          n[d] = (float)((h2d(v[d]) * inv) * w);
        }
        for (int d = 0; d < HD; ++d) {
          int i = d & 63;
          float rot = d < 64 ? -n[d + 64] : n[d - 64];
          double r = (double)n[d] * (double)cs[pos * 64 + i] + (double)rot * (double)sn[pos * 64 + i];
          v[d] = orc_f32_to_f16((float)r);
        }
      }
    }
  }
  free(cs);
  free(sn);
}

void orc_gen_lengths(uint64_t seed, int32_t n, int32_t lo, int32_t hi, int32_t* out) {
  uint64_t span = (uint64_t)(hi - lo + 1);
  for (int32_t i = 0; i < n; ++i) out[i] = lo + (int32_t)((orc_rand_u64(seed, (uint64_t)i) >> 33) % span);
}

/* ------------------------------------------------------------------------------------------ */
/* mask                                                                                        */
/* ------------------------------------------------------------------------------------------ */

int orc_retained(int64_t q, int64_t k, int64_t S, int32_t kind, int64_t P, int64_t W) {
  /* ops.ts:206 prefix_size=min(S,176), local_window=min(S,432); ops.ts:220 predicate. */
  if (!(q < S && k <= q && k < S)) return 0;
  if (kind == ORC_MASK_CAUSAL) return 1;
  int64_t prefix_size = S < P ? S : P;
  int64_t local_window = S < W ? S : W;
  return (k < prefix_size) || (k + local_window > q);
}

void orc_mask_bits(int32_t L, int32_t kind, int32_t P, int32_t W, uint32_t* bits) {
  int64_t words = ((int64_t)L + 31) / 32;
  memset(bits, 0, sizeof(uint32_t) * (size_t)(words * L));
  for (int64_t q = 0; q < L; ++q)
    for (int64_t k = 0; k <= q; ++k)
      if (orc_retained(q, k, L, kind, P, W)) bits[q * words + k / 32] |= 1u << (k % 32);
}

int64_t orc_mask_pairs(int32_t L, int32_t kind, int32_t P, int32_t W) {
  int64_t n = 0;
  for (int64_t q = 0; q < L; ++q)
    for (int64_t k = 0; k <= q; ++k) n += orc_retained(q, k, L, kind, P, W);
  return n;
}

int orc_ref_tile_skipped(int64_t S, int64_t q_tile_start, int64_t key_base) {
  /* ops.ts:206-209 with the reference's constants. */
  int64_t prefix_size = S < 176 ? S : 176;
  int64_t local_window = S < 432 ? S : 432;
  int64_t local_start = (q_tile_start + 1 > local_window) ? q_tile_start + 1 - local_window : 0;
  return key_base >= prefix_size && key_base + 15 < local_start;
}

/* ------------------------------------------------------------------------------------------ */
/* attention: exact f64                                                                        */
/* ------------------------------------------------------------------------------------------ */

static int32_t find_seq(const int32_t* cu, int32_t nseq, int64_t t) {
  int32_t lo = 0, hi = nseq - 1;
  while (lo < hi) {
    int32_t mid = (lo + hi + 1) / 2;
    if (cu[mid] <= t) lo = mid; else hi = mid - 1;
  }
  return lo;
}

void orc_attention_exact(const orc_attn_args* a, const int64_t* rows, int64_t nrows, double* out) {
  int64_t T = a->cu_seqlens[a->nseq];
  if (!rows) nrows = T;
  const double scale = 1.0 / sqrt(128.0);
#pragma omp parallel
  {
    int64_t maxlen = 0;
    for (int32_t s = 0; s < a->nseq; ++s)
      if (a->cu_seqlens[s + 1] - a->cu_seqlens[s] > maxlen) maxlen = a->cu_seqlens[s + 1] - a->cu_seqlens[s];
    double* sc = (double*)malloc(sizeof(double) * (size_t)(maxlen + 1));
    double qv[HD];
#pragma omp for schedule(dynamic, 4)
    for (int64_t r = 0; r < nrows; ++r) {
      int64_t t = rows ? rows[r] : r;
      int32_t s = find_seq(a->cu_seqlens, a->nseq, t);
      int64_t t0 = a->cu_seqlens[s], L = a->cu_seqlens[s + 1] - t0, qp = t - t0;
      for (int h = 0; h < HQ; ++h) {
        int kvh = h / (HQ / HKV);
        const uint16_t* qr = a->q + t * a->q_stride + (int64_t)h * HD;
        for (int d = 0; d < HD; ++d) qv[d] = h2d(qr[d]);
        double m = -INFINITY;
        for (int64_t kp = 0; kp <= qp; ++kp) {
          if (!orc_retained(qp, kp, L, a->kind, a->prefix, a->window)) { sc[kp] = -INFINITY; continue; }
          const uint16_t* kr = a->k + (t0 + kp) * a->k_stride + (int64_t)kvh * HD;
          double acc = 0.0;
          for (int d = 0; d < HD; ++d) acc += qv[d] * h2d(kr[d]);
          sc[kp] = acc * scale;
          if (sc[kp] > m) m = sc[kp];
        }
        double den = 0.0;
        double o[HD];
        for (int d = 0; d < HD; ++d) o[d] = 0.0;
        for (int64_t kp = 0; kp <= qp; ++kp) {
          if (sc[kp] == -INFINITY) continue;
          double p = exp(sc[kp] - m);
          den += p;
          const uint16_t* vr = a->v + (t0 + kp) * a->v_stride + a->v_offset + (int64_t)kvh * HD;
          for (int d = 0; d < HD; ++d) o[d] += p * h2d(vr[d]);
        }
        double* dst = out + (r * HQ + h) * HD;
        for (int d = 0; d < HD; ++d) dst[d] = o[d] / den;
      }
    }
    free(sc);
  }
}

/* ------------------------------------------------------------------------------------------ */
/* attention: f16-faithful restatement of the reference's 16x16 tiled kernel                   */
/* ------------------------------------------------------------------------------------------ */

static inline float expf_cr(float x) { return (float)exp((double)x); }

/* One (sequence, q_head, 16-query tile) workgroup of ops.ts:194-240. */
static void tiled16_group(const orc_attn_args* a, int64_t t0, int64_t S, int q_head, int64_t gx,
                          uint16_t* out, int64_t o_stride) {
  const float NEG = -3.402823e38f; /* ops.ts:187, 219 */
  const float SCALE = 0.08838834764831845f; /* ops.ts:223 (as f32) */
  int kv_head = q_head / (HQ / HKV);
  double query_tile[16][HD], key_tile[16][HD], value_tile[16][HD], total_tile[16][HD];
  float scores[16][16];
  double weights[16][16]; /* f16 values */
  float maxima[16];
  double denominators[16], alphas[16], betas[16]; /* f16 values */
  for (int row = 0; row < 16; ++row) {
    int64_t position = gx * 16 + row;
    for (int d = 0; d < HD; ++d) {
      query_tile[row][d] = position < S ? h2d(a->q[(t0 + position) * a->q_stride + (int64_t)q_head * HD + d]) : 0.0;
      total_tile[row][d] = 0.0;
    }
    maxima[row] = NEG;
    denominators[row] = 0.0;
  }
  int64_t key_limit = S < (gx + 1) * 16 ? S : (gx + 1) * 16;
  int64_t prefix_size = S < a->prefix ? S : a->prefix;
  int64_t local_window = S < a->window ? S : a->window;
  int64_t query_tile_start = gx * 16;
  int64_t local_start = query_tile_start + 1 > local_window ? query_tile_start + 1 - local_window : 0;
  int sparse = a->kind == ORC_MASK_PREFIX_LOCAL;
  for (int64_t key_base = 0; key_base < key_limit; key_base += 16) {
    /* ops.ts:209: the reference kernel always applies the sparse skip and predicate; the
     * full-causal variant here reproduces the same kernel with the window/prefix disabled. */
    if (sparse && key_base >= prefix_size && key_base + 15 < local_start) continue;
    for (int row = 0; row < 16; ++row) {
      int64_t k_pos = key_base + row;
      for (int d = 0; d < HD; ++d) {
        if (k_pos < S) {
          key_tile[row][d] = h2d(a->k[(t0 + k_pos) * a->k_stride + (int64_t)kv_head * HD + d]);
          value_tile[row][d] = h2d(a->v[(t0 + k_pos) * a->v_stride + a->v_offset + (int64_t)kv_head * HD + d]);
        } else {
          key_tile[row][d] = 0.0;
          value_tile[row][d] = 0.0;
        }
      }
    }
    /* ops.ts:219-225: score = sum_d4 f32(dot(q4,k4)) * scale; dot4 in strict f16. */
    for (int y = 0; y < 16; ++y) {
      int64_t q_pos = gx * 16 + y;
      for (int x = 0; x < 16; ++x) {
        int64_t k_pos = key_base + x;
        float score = NEG;
        int keep = q_pos < S && k_pos <= q_pos && k_pos < S &&
                   (!sparse || k_pos < prefix_size || k_pos + local_window > q_pos);
        if (keep) {
          score = 0.0f;
          for (int d4 = 0; d4 < 32; ++d4) {
            const double* qq = &query_tile[y][d4 * 4];
            const double* kk = &key_tile[x][d4 * 4];
            double dt = r16(qq[0] * kk[0]);
            dt = r16(dt + r16(qq[1] * kk[1]));
            dt = r16(dt + r16(qq[2] * kk[2]));
            dt = r16(dt + r16(qq[3] * kk[3]));
            score = (float)((double)score + dt); /* f32 add of an f16 value */
          }
          score = score * SCALE;
        }
        scores[y][x] = score;
      }
    }
    /* ops.ts:186-193 update_stats for every row. */
    for (int row = 0; row < 16; ++row) {
      float block_max = NEG;
      for (int c = 0; c < 16; ++c) block_max = fmaxf(block_max, scores[row][c]);
      float block_den = 0.0f;
      for (int c = 0; c < 16; ++c) {
        float weight = expf_cr(scores[row][c] - block_max);
        weights[row][c] = h2d(orc_f32_to_f16(weight));
        block_den = block_den + weight;
      }
      float next_max = fmaxf(maxima[row], block_max);
      float alpha = expf_cr(maxima[row] - next_max);
      float beta = expf_cr(block_max - next_max);
      alphas[row] = h2d(orc_f32_to_f16(alpha));
      betas[row] = h2d(orc_f32_to_f16(beta));
      double bb = h2d(orc_f32_to_f16(beta * block_den)); /* f32 product, then f16 */
      denominators[row] = r16(r16(denominators[row] * alphas[row]) + bb);
      maxima[row] = next_max;
    }
    /* ops.ts:229-233: av = sum_c w*V (f16), total = total*alpha + beta*av (f16). */
    for (int row = 0; row < 16; ++row)
      for (int d = 0; d < HD; ++d) {
        double av = 0.0;
        for (int c = 0; c < 16; ++c) av = r16(av + r16(weights[row][c] * value_tile[c][d]));
        total_tile[row][d] = r16(r16(total_tile[row][d] * alphas[row]) + r16(betas[row] * av));
      }
  }
  /* ops.ts:236-239: O = total / den in f16 for rows inside the sequence. */
  for (int row = 0; row < 16; ++row) {
    int64_t position = gx * 16 + row;
    if (position >= S) continue;
    uint16_t* dst = out + (t0 + position) * o_stride + (int64_t)q_head * HD;
    for (int d = 0; d < HD; ++d) {
      double v = r16(total_tile[row][d] / denominators[row]);
      dst[d] = orc_f32_to_f16((float)v);
    }
  }
}

void orc_attention_tiled16(const orc_attn_args* a, uint16_t* out, int64_t o_stride) {
  int64_t total_groups = 0;
  int64_t* base = (int64_t*)malloc(sizeof(int64_t) * (size_t)(a->nseq + 1));
  for (int32_t s = 0; s < a->nseq; ++s) {
    base[s] = total_groups;
    int64_t L = a->cu_seqlens[s + 1] - a->cu_seqlens[s];
    total_groups += ((L + 15) / 16) * HQ;
  }
  base[a->nseq] = total_groups;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t g = 0; g < total_groups; ++g) {
    int32_t s = 0;
    while (base[s + 1] <= g) ++s;
    int64_t local = g - base[s];
    int64_t t0 = a->cu_seqlens[s], S = a->cu_seqlens[s + 1] - t0;
    tiled16_group(a, t0, S, (int)(local % HQ), local / HQ, out, o_stride);
  }
  free(base);
}

void orc_attention_tiled16_tiles(const orc_attn_args* a, int32_t seq, int64_t tile_begin,
                                 int64_t tile_end, int64_t tile_step, uint16_t* out,
                                 int64_t o_stride) {
  int64_t t0 = a->cu_seqlens[seq], S = a->cu_seqlens[seq + 1] - t0;
  int64_t ntiles = (S + 15) / 16;
  if (tile_end > ntiles) tile_end = ntiles;
  if (tile_step < 1) tile_step = 1;
  int64_t count = tile_begin < tile_end ? (tile_end - tile_begin + tile_step - 1) / tile_step : 0;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t g = 0; g < count * HQ; ++g) {
    int64_t gx = tile_begin + (g / HQ) * tile_step;
    tiled16_group(a, t0, S, (int)(g % HQ), gx, out, o_stride);
  }
}

void orc_set_threads(int32_t n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

int32_t orc_get_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
