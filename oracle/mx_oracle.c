/*
 * mx_oracle.c -- CPU oracle (test infrastructure only; see mx_oracle.h).
 *
 * Every function states the reference lines it restates.  The code is an
 * independent formulation: integer bit manipulation for the element codes,
 * double-precision arithmetic for the attention recurrence.
 */
#include "mx_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ bits */
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------- floorf(log2f(x)) table
 * The reference evaluates floorf(log2f(x)) (mx_fp_math.h:209, :322,
 * mx_golden.cpp:171).  log2f rounds its result to float, so for x just
 * below a power of two 2^(e+1) the rounded logarithm equals e+1 and the floor
 * is one larger than the exponent of x.  Which mantissas are affected depends
 * only on the float spacing around the integer e+1; the table is derived here
 * by rounding a double-precision log2 to float (tests pin it exhaustively
 * against libm's log2f and against the reference's compiled encoder). */
static uint32_t g_thr[256];      /* by biased exponent */
static uint32_t g_sub_thr[23];   /* subnormal, by leading-bit position p */
static pthread_once_t g_once = PTHREAD_ONCE_INIT;

static void build_tables(void) {
  for (int E = 0; E < 256; E++) g_thr[E] = 0x800000u;
  for (int E = 1; E < 255; E++) {
    int e = E - 127;
    uint32_t m = 0x800000u;
    while (m > 0) {
      uint32_t cand = m - 1;
      double x = ldexp(1.0 + (double)cand / 8388608.0, e);
      float r = (float)log2(x);
      if (floorf(r) >= (float)(e + 1)) m = cand; else break;
    }
    g_thr[E] = m;
  }
  for (int p = 0; p < 23; p++) {
    uint32_t lo = 1u << p, hi = 2u << p;   /* mantissa integers in [lo, hi) */
    uint32_t m = hi;
    while (m > lo) {
      uint32_t cand = m - 1;
      double x = ldexp((double)cand, -149);
      float r = (float)log2(x);
      if (floorf(r) >= (float)(p - 149 + 1)) m = cand; else break;
    }
    g_sub_thr[p] = m;   /* == hi means never */
  }
}

void orc_log2_tables(uint32_t thr[256], uint32_t sub_thr[23]) {
  pthread_once(&g_once, build_tables);
  memcpy(thr, g_thr, sizeof g_thr);
  memcpy(sub_thr, g_sub_thr, sizeof g_sub_thr);
}

int orc_floor_log2f(float x) {
  pthread_once(&g_once, build_tables);
  uint32_t b = f2u(x) & 0x7fffffffu;
  uint32_t E = b >> 23, m = b & 0x7fffffu;
  if (E == 0) {
    int p = 31 - __builtin_clz(m);
    return p - 149 + (m >= g_sub_thr[p] ? 1 : 0);
  }
  return (int)E - 127 + (m >= g_thr[E] ? 1 : 0);
}

/* ------------------------------------------------------------ element rules */
/* mx_fp_math.h:11-28: RNE to bf16, +-0 -> +0, tiny results that round to a
 * zero magnitude -> +0, NaN kept quiet. */
uint16_t orc_f32_to_bf16(float x) {
  if (x == 0.0f) return 0;
  uint32_t b = f2u(x);
  if (((b >> 23) & 0xff) == 0xff) {
    uint32_t h = b >> 16;
    if ((b & 0x7fffffu) && !(h & 0x40)) h |= 0x40;
    return (uint16_t)h;
  }
  uint32_t r = (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;
  if ((r & 0x7fffu) == 0) return 0;
  return (uint16_t)r;
}
float orc_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* mx_fp_math.h:205-225 restated on the float bits.  E = floorf(log2f(|v|));
 * E < -6 flushes to 0 (no E4M3 subnormals are produced); E > 8 saturates to
 * 448; otherwise the 23-bit mantissa is rounded to 3 bits, ties to even.
 * When log2f rounded up (|v| just below 2^E) the value rounds to 2^E. */
uint8_t orc_e4m3_encode(float v) {
  if (v == 0.0f || !isfinite(v)) return 0;
  uint32_t b = f2u(v);
  uint8_t s = (uint8_t)((b >> 31) << 7);
  float a = u2f(b & 0x7fffffffu);
  int E = orc_floor_log2f(a);
  if (E < -6) return 0;
  if (E > 8) return s | 0x7e;
  int true_e = (int)((b >> 23) & 0xff) - 127;
  int q;
  if (E != true_e) {
    q = 0;
  } else {
    uint32_t mant = b & 0x7fffffu;
    q = (int)(mant >> 20);
    uint32_t rem = mant & 0xfffffu;
    if (rem > 0x80000u || (rem == 0x80000u && (q & 1))) q++;
    if (q == 8) { q = 0; E++; }
  }
  if (E > 8 || (E == 8 && q == 7)) return s | 0x7e;
  return (uint8_t)(s | ((E + 7) << 3) | q);
}

/* mx_fp_math.h:227-236 */
float orc_e4m3_decode(uint8_t c) {
  int e = (c >> 3) & 15, m = c & 7;
  float v = e ? ldexpf(1.0f + m / 8.0f, e - 7) : ldexpf((float)m, -9);
  return (c & 0x80) ? -v : v;
}

/* mx_fp_math.h:256-264 */
float orc_e3m2_decode(uint8_t c) {
  int e = (c >> 2) & 7, m = c & 3;
  float v = e ? ldexpf(1.0f + m / 4.0f, e - 3) : ldexpf((float)m, -4);
  return (c & 0x20) ? -v : v;
}

/* mx_fp_math.h:249-252 */
double orc_e8m0_decode(uint8_t c) { return c == 0xff ? NAN : ldexp(1.0, (int)c - 127); }

/* mx_fp_math.h:266-335: bf16 -> E4M2 (RNE, subnormal grid 2^-8, overflow ->
 * inf) -> the fixed E4M2->E3M2 value map -> 6-bit code.  Restated as
 * arithmetic on a magnitude counted in units of 2^-8. */
uint8_t orc_e3m2_encode_bf16(uint16_t b) {
  int neg = b >> 15, E = (b >> 7) & 0xff, M = b & 0x7f;
  if (E == 0) return 0;
  double mag;                        /* E4M2 magnitude, +inf on overflow */
  if (E == 255) {
    mag = INFINITY;
  } else {
    int e = E - 127;
    if (e >= -6 && e <= 7) {
      int q = M >> 5, rbit = (M >> 4) & 1, sticky = (M & 15) != 0;
      int sig = q + (rbit & (sticky | (q & 1)));
      if (sig == 4) { sig = 0; e++; }
      mag = e > 7 ? INFINITY : ldexp(1.0 + sig / 4.0, e);
    } else if (e >= -9 && e < -6) {
      /* (128 + M) * 2^(e-7) in units of 2^-8 is (128+M) * 2^(e+1); round half to even */
      double units = (128.0 + M) * ldexp(1.0, e + 1);
      double fl = floor(units), fr = units - fl;
      double k = fr > 0.5 ? fl + 1 : (fr < 0.5 ? fl : (fmod(fl, 2.0) == 0 ? fl : fl + 1));
      mag = k / 256.0;
    } else {
      mag = 0.0;   /* e < -9, and also e > 7: the reference maps these to 0 */
    }
  }
  /* e4m2_to_fp6_float (mx_fp_math.h:295-307) */
  if (!(mag < 32.0)) mag = 28.0;
  else if (mag <= 0.0546875) return 0;
  else if (mag <= 0.21875) mag = mag <= 0.078125 ? 0.0625 : (mag <= 0.15625 ? 0.125 : 0.1875);
  /* fp6_value_to_code (mx_fp_math.h:310-330): every magnitude here is on the
   * E3M2 grid, so the code is its exponent and 2-bit mantissa. */
  int code;
  if (mag < 0.25) {
    code = (int)(mag / 0.0625);
  } else {
    int e = (int)floor(log2(mag));
    int m = (int)((mag / ldexp(1.0, e) - 1.0) * 4.0 + 0.5);
    code = ((e + 3) << 2) | m;
  }
  return (uint8_t)((neg << 5) | code);
}

/* mx_golden.cpp:169-174 (log2_pmax = 8 for E4M3, 4 for E3M2). A non-finite
 * (infinite) block maximum yields code 0, which is what the reference's
 * float->int conversion of floorf(log2f(inf)) produces on x86. */
uint8_t orc_scale_code(float amax, int fmt) {
  if (amax == 0.0f || !(amax == amax)) return 0;
  if (isinf(amax)) return 0;
  int s2 = orc_floor_log2f(amax) - (fmt == ORC_FMT_E4M3 ? 8 : 4) + 127;
  return (uint8_t)(s2 < 0 ? 0 : (s2 > 254 ? 254 : s2));
}

double orc_decode_elem(uint8_t code, int fmt) {
  return fmt == ORC_FMT_E4M3 ? (double)orc_e4m3_decode(code) : (double)orc_e3m2_decode(code & 0x3f);
}

/* mx_golden.cpp:162-190: block amax (NaN ignored by the > compare), scale
 * code, then each element divided by the power-of-two scale and encoded. */
uint8_t orc_quantize_block(const float *v, int64_t stride, int n, int fmt,
                           uint8_t *codes, int64_t code_stride) {
  float amax = 0.0f;
  for (int i = 0; i < n; i++) {
    float a = fabsf(v[i * stride]);
    if (a > amax) amax = a;
  }
  uint8_t sc = orc_scale_code(amax, fmt);
  for (int i = 0; i < n; i++) {
    float y = ldexpf(v[i * stride], 127 - (int)sc);
    codes[i * code_stride] = fmt == ORC_FMT_E4M3 ? orc_e4m3_encode(y)
                                                 : orc_e3m2_encode_bf16(orc_f32_to_bf16(y));
  }
  return sc;
}

void orc_quantize_rows(const float *x, int64_t rows, int64_t cols, int fmt,
                       uint8_t *codes, uint8_t *scales) {
  int64_t nb = cols / 32;
  for (int64_t r = 0; r < rows; r++)
    for (int64_t b = 0; b < nb; b++)
      scales[r * nb + b] = orc_quantize_block(x + r * cols + b * 32, 1, 32, fmt,
                                              codes + r * cols + b * 32, 1);
}

void orc_quantize_cols(const float *x, int64_t rows, int64_t cols, int fmt,
                       uint8_t *codes, uint8_t *scales) {
  int64_t nb = rows / 32;
  for (int64_t b = 0; b < nb; b++)
    for (int64_t c = 0; c < cols; c++)
      scales[b * cols + c] = orc_quantize_block(x + b * 32 * cols + c, cols, 32, fmt,
                                                codes + b * 32 * cols + c, cols);
}

/* ------------------------------------------------------------- attention */
typedef struct {
  const orc_attn_params *p;
  const uint8_t *q, *q_sc, *k, *k_sc, *v, *v_sc;
  float *o;
  int block_n, split_len, n_parts, dense;
  const int32_t *heads;
  int nheads;
  double **kd, **vd;         /* dequantized K/V per flattened kv head (NULL if unused) */
  int64_t nitems, rows_per_item;
  int64_t next;
  pthread_mutex_t mu;
} job_t;

static void dequant_kv(const orc_attn_params *p, const uint8_t *k, const uint8_t *k_sc,
                       const uint8_t *v, const uint8_t *v_sc, int64_t kvh,
                       double *kd, double *vd) {
  int64_t Sk = p->seq_k, D = p->head_dim, nb = D / 32;
  const uint8_t *kc = k + kvh * Sk * D, *ks = k_sc + kvh * Sk * nb;
  const uint8_t *vc = v + kvh * Sk * D, *vs = v_sc + kvh * (Sk / 32) * D;
  for (int64_t t = 0; t < Sk; t++)
    for (int64_t d = 0; d < D; d++) {
      kd[t * D + d] = orc_decode_elem(kc[t * D + d], ORC_FMT_E4M3) * orc_e8m0_decode(ks[t * nb + d / 32]);
      vd[t * D + d] = orc_decode_elem(vc[t * D + d], p->v_fmt) * orc_e8m0_decode(vs[(t / 32) * D + d]);
    }
}

static int key_visible(const orc_attn_params *p, int64_t kpos, int64_t qpos) {
  if (kpos >= p->seq_k) return 0;
  if (p->causal && kpos > qpos) return 0;
  if (p->window > 0 && kpos + p->window <= qpos) return 0;
  return 1;
}

static double score_of(const orc_attn_params *p, const double *qd, const double *kr) {
  double s = 0.0;
  for (int d = 0; d < p->head_dim; d++) s += qd[d] * kr[d];
  s *= (double)p->softmax_scale;
  if (p->softcap > 0.0f) s = (double)p->softcap * tanh(s / (double)p->softcap);
  return s;
}

/* One streaming pass over keys [k0, k1) with blocks aligned to block_n.
 * Outputs unnormalized O, running max m and sum l. */
/* One streaming pass over the key blocks starting at k0, k0 + stride, ... below k1; each
 * block is [b0, min(b0 + block_n, k1)).  stride = block_n: the keys [k0, k1) in order. */
/* Stage record of one row's pass (orc_attention_trace): per key the score S (natural units,
 * -inf where masked) and the P code, per 32-key group the P scale code, per block the running
 * (m, l) after it.  NULL members are not written. */
typedef struct {
  double *S;
  uint8_t *codes, *scales;
  double *ml;
} orc_trace_t;

static void flash_pass_tr(const orc_attn_params *p, const double *qd, const double *kd, const double *vd,
                          int64_t qpos, int64_t k0, int64_t k1, int block_n, int64_t stride,
                          double *O, double *m_out, double *l_out, double *S, float *P, const orc_trace_t *tr);

static void flash_pass(const orc_attn_params *p, const double *qd, const double *kd, const double *vd,
                       int64_t qpos, int64_t k0, int64_t k1, int block_n, int64_t stride,
                       double *O, double *m_out, double *l_out, double *S, float *P) {
  flash_pass_tr(p, qd, kd, vd, qpos, k0, k1, block_n, stride, O, m_out, l_out, S, P, NULL);
}

static void flash_pass_tr(const orc_attn_params *p, const double *qd, const double *kd, const double *vd,
                          int64_t qpos, int64_t k0, int64_t k1, int block_n, int64_t stride,
                          double *O, double *m_out, double *l_out, double *S, float *P, const orc_trace_t *tr) {
  int D = p->head_dim;
  double m = -INFINITY, l = 0.0;
  for (int d = 0; d < D; d++) O[d] = 0.0;
  for (int64_t b0 = k0; b0 < k1; b0 += stride) {
    int64_t b1 = b0 + block_n < k1 ? b0 + block_n : k1;
    int n = (int)(b1 - b0);
    double bmax = -INFINITY;
    for (int t = 0; t < n; t++) {
      int64_t kp = b0 + t;
      S[t] = key_visible(p, kp, qpos) ? score_of(p, qd, kd + kp * D) : -INFINITY;
      if (S[t] > bmax) bmax = S[t];
    }
    double m_new = m > bmax ? m : bmax;
    if (tr && tr->S)
      for (int t = 0; t < n; t++) tr->S[b0 + t] = S[t];
    if (m_new == -INFINITY) {                       /* nothing visible yet */
      if (tr && tr->ml) { tr->ml[2 * (b0 / block_n)] = -INFINITY; tr->ml[2 * (b0 / block_n) + 1] = 0.0; }
      if (tr && tr->codes)
        for (int t = 0; t < n; t++) tr->codes[b0 + t] = 0;
      continue;
    }
    double corr = (m == -INFINITY) ? 0.0 : exp(m - m_new);
    for (int t = 0; t < n; t++) P[t] = S[t] == -INFINITY ? 0.0f : (float)exp(S[t] - m_new);
    /* requant P per 32-key group (global key index): rule R1 E4M3, or rule R2 on the
     * bf16-rounded P (which is then also the P summed into l) */
    uint8_t gcodes[ORC_MAX_BLOCK_N], gsc[ORC_MAX_BLOCK_N / 32];
    for (int t = 0; t < n; t += 32) {
      int g = n - t < 32 ? n - t : 32;
      gsc[t / 32] = p->p_rule == ORC_P_R2 ? orc_r2_quantize_block(P + t, g, P + t, gcodes + t)
                                          : orc_quantize_block(P + t, 1, g, ORC_FMT_E4M3, gcodes + t, 1);
    }
    double lsum = 0.0;
    for (int t = 0; t < n; t++) lsum += (double)P[t];
    l = l * corr + lsum;
    if (tr) {
      if (tr->codes) memcpy(tr->codes + b0, gcodes, (size_t)n);
      if (tr->scales)
        for (int t = 0; t < n; t += 32) tr->scales[(b0 + t) / 32] = gsc[t / 32];
      if (tr->ml) { tr->ml[2 * (b0 / block_n)] = m_new; tr->ml[2 * (b0 / block_n) + 1] = l; }
    }
    for (int d = 0; d < D; d++) O[d] *= corr;
    for (int t = 0; t < n; t += 32) {
      int g = n - t < 32 ? n - t : 32;
      const uint8_t *codes = gcodes + t;
      uint8_t sc = gsc[t / 32];
      double scale = orc_e8m0_decode(sc);
      for (int u = 0; u < g; u++) {
        if (!codes[u]) continue;
        double pq = (double)orc_e4m3_decode(codes[u]) * scale;
        const double *vr = vd + (b0 + t + u) * D;
        for (int d = 0; d < D; d++) O[d] += pq * vr[d];
      }
    }
    m = m_new;
  }
  *m_out = m;
  *l_out = l;
}

static void do_row(job_t *J, int64_t bh, int64_t i, double *qd, double *O, double *Oc, double *S, float *P) {
  const orc_attn_params *p = J->p;
  int64_t D = p->head_dim, nb = D / 32, Sq = p->seq_q;
  int64_t b = bh / p->num_q_heads, h = bh % p->num_q_heads;
  int64_t kvh = b * p->num_kv_heads + h / (p->num_q_heads / p->num_kv_heads);
  const uint8_t *qc = J->q + (bh * Sq + i) * D, *qs = J->q_sc + (bh * Sq + i) * nb;
  for (int64_t d = 0; d < D; d++) qd[d] = orc_decode_elem(qc[d], ORC_FMT_E4M3) * orc_e8m0_decode(qs[d / 32]);
  int64_t qpos = p->q_pos0 + i;
  const double *kd = J->kd[kvh], *vd = J->vd[kvh];
  float *out = J->o + (bh * Sq + i) * D;
  if (J->dense) {
    double m = -INFINITY, l = 0.0;
    for (int64_t t = 0; t < p->seq_k; t++) {
      S[t] = key_visible(p, t, qpos) ? score_of(p, qd, kd + t * D) : -INFINITY;
      if (S[t] > m) m = S[t];
    }
    for (int64_t d = 0; d < D; d++) O[d] = 0.0;
    if (m != -INFINITY)
      for (int64_t t = 0; t < p->seq_k; t++) {
        if (S[t] == -INFINITY) continue;
        double e = exp(S[t] - m);
        l += e;
        for (int64_t d = 0; d < D; d++) O[d] += e * vd[t * D + d];
      }
    for (int64_t d = 0; d < D; d++) out[d] = l > 0.0 ? (float)(O[d] / l) : 0.0f;
    return;
  }
  /* partials: n_parts > 0 -- partial i takes the key blocks i, i + n_parts, i + 2 n_parts,
   * ... (the interleaved decode schedule); else contiguous chunks of split_len keys (one
   * chunk when 0).  Partials are merged in order by log-sum-exp. */
  int64_t Sk = p->seq_k;
  int64_t chunk = J->split_len > 0 ? J->split_len : Sk;
  int64_t nparts = J->n_parts > 0 ? J->n_parts : (Sk + chunk - 1) / chunk;
  double M = -INFINITY, L = 0.0;
  for (int64_t d = 0; d < D; d++) O[d] = 0.0;
  for (int64_t i = 0; i < nparts; i++) {
    double mc, lc;
    if (J->n_parts > 0)
      flash_pass(p, qd, kd, vd, qpos, i * J->block_n, Sk, J->block_n, (int64_t)J->n_parts * J->block_n, Oc, &mc,
                 &lc, S, P);
    else
      flash_pass(p, qd, kd, vd, qpos, i * chunk, (i + 1) * chunk < Sk ? (i + 1) * chunk : Sk, J->block_n,
                 J->block_n, Oc, &mc, &lc, S, P);
    if (mc == -INFINITY || lc <= 0.0) continue;
    if (M == -INFINITY) {
      M = mc; L = lc;
      for (int64_t d = 0; d < D; d++) O[d] = Oc[d];
    } else {
      double Mn = M > mc ? M : mc;
      double a = exp(M - Mn), bb = exp(mc - Mn);
      L = L * a + lc * bb;
      for (int64_t d = 0; d < D; d++) O[d] = O[d] * a + Oc[d] * bb;
      M = Mn;
    }
  }
  for (int64_t d = 0; d < D; d++) out[d] = L > 0.0 ? (float)(O[d] / L) : 0.0f;
}

static void *worker(void *arg) {
  job_t *J = (job_t *)arg;
  const orc_attn_params *p = J->p;
  int64_t D = p->head_dim, Sk = p->seq_k;
  double *qd = malloc(sizeof(double) * D), *O = malloc(sizeof(double) * D), *Oc = malloc(sizeof(double) * D);
  int64_t sl = Sk > J->block_n ? Sk : J->block_n;
  double *S = malloc(sizeof(double) * sl);
  float *P = malloc(sizeof(float) * sl);
  for (;;) {
    pthread_mutex_lock(&J->mu);
    int64_t it = J->next++;
    pthread_mutex_unlock(&J->mu);
    if (it >= J->nitems) break;
    int64_t rows_chunks = (p->seq_q + J->rows_per_item - 1) / J->rows_per_item;
    int64_t hi = it / rows_chunks, rc = it % rows_chunks;
    int64_t bh = J->heads ? J->heads[hi] : hi;
    int64_t r0 = rc * J->rows_per_item, r1 = r0 + J->rows_per_item;
    if (r1 > p->seq_q) r1 = p->seq_q;
    for (int64_t i = r0; i < r1; i++) do_row(J, bh, i, qd, O, Oc, S, P);
  }
  free(qd); free(O); free(Oc); free(S); free(P);
  return NULL;
}

static int run_attention(const orc_attn_params *p, const uint8_t *q, const uint8_t *q_sc,
                         const uint8_t *k, const uint8_t *k_sc, const uint8_t *v, const uint8_t *v_sc,
                         float *o, int block_n, int split_len, int n_parts, int dense,
                         const int32_t *heads, int nheads, int nthreads) {
  if (!p || p->batch <= 0 || p->num_q_heads <= 0 || p->num_kv_heads <= 0 || p->seq_q <= 0 ||
      p->seq_k <= 0 || p->head_dim <= 0 || p->head_dim % 32 || p->seq_k % 32 ||
      p->num_q_heads % p->num_kv_heads)
    return -1;
  if (!dense && (block_n <= 0 || block_n % 32 || block_n > ORC_MAX_BLOCK_N)) return -1;
  if (p->p_rule != ORC_P_R1 && p->p_rule != ORC_P_R2) return -1;
  if (split_len < 0 || (split_len > 0 && split_len % block_n)) return -1;
  if (n_parts < 0 || (n_parts > 0 && split_len > 0)) return -1;
  int64_t nbh = (int64_t)p->batch * p->num_q_heads;
  int64_t nkv = (int64_t)p->batch * p->num_kv_heads;
  int grp = p->num_q_heads / p->num_kv_heads;
  int n_use = heads ? nheads : (int)nbh;
  for (int i = 0; heads && i < nheads; i++)
    if (heads[i] < 0 || heads[i] >= nbh) return -1;
  job_t J;
  memset(&J, 0, sizeof J);
  J.p = p; J.q = q; J.q_sc = q_sc; J.k = k; J.k_sc = k_sc; J.v = v; J.v_sc = v_sc; J.o = o;
  J.block_n = block_n; J.split_len = split_len; J.n_parts = n_parts; J.dense = dense; J.heads = heads; J.nheads = nheads;
  J.kd = calloc((size_t)nkv, sizeof(double *));
  J.vd = calloc((size_t)nkv, sizeof(double *));
  int64_t kvsz = (int64_t)p->seq_k * p->head_dim;
  for (int i = 0; i < n_use; i++) {
    int64_t bh = heads ? heads[i] : i;
    int64_t kvh = (bh / p->num_q_heads) * p->num_kv_heads + (bh % p->num_q_heads) / grp;
    if (!J.kd[kvh]) {
      J.kd[kvh] = malloc(sizeof(double) * kvsz);
      J.vd[kvh] = malloc(sizeof(double) * kvsz);
      dequant_kv(p, k, k_sc, v, v_sc, kvh, J.kd[kvh], J.vd[kvh]);
    }
  }
  J.rows_per_item = 16;
  J.nitems = (int64_t)n_use * ((p->seq_q + J.rows_per_item - 1) / J.rows_per_item);
  pthread_mutex_init(&J.mu, NULL);
  if (nthreads < 1) nthreads = 1;
  pthread_t *th = malloc(sizeof(pthread_t) * nthreads);
  for (int t = 0; t < nthreads; t++) pthread_create(&th[t], NULL, worker, &J);
  for (int t = 0; t < nthreads; t++) pthread_join(th[t], NULL);
  free(th);
  pthread_mutex_destroy(&J.mu);
  for (int64_t i = 0; i < nkv; i++) { free(J.kd[i]); free(J.vd[i]); }
  free(J.kd); free(J.vd);
  return 0;
}

int orc_attention(const orc_attn_params *p, const uint8_t *q, const uint8_t *q_sc,
                  const uint8_t *k, const uint8_t *k_sc, const uint8_t *v, const uint8_t *v_sc,
                  float *o, int block_n, int split_len, int n_parts, const int32_t *heads, int nheads,
                  int nthreads) {
  return run_attention(p, q, q_sc, k, k_sc, v, v_sc, o, block_n, split_len, n_parts, 0, heads, nheads, nthreads);
}

/* The stages of one query row's single streaming pass (the prefill schedule: key blocks of
 * block_n in order): S [seq_k] (natural units after scale, softcap and mask), P codes
 * [seq_k], P scale codes [seq_k / 32], (m, l) after each block [ceil(seq_k / block_n)][2].
 * Returns 0, or -1 on invalid arguments. */
int orc_attention_trace(const orc_attn_params *p, const uint8_t *q, const uint8_t *q_sc,
                        const uint8_t *k, const uint8_t *k_sc, const uint8_t *v, const uint8_t *v_sc,
                        int block_n, int64_t bh, int64_t qi, double *S_out, uint8_t *codes_out,
                        uint8_t *scales_out, double *ml_out) {
  if (!p || p->batch <= 0 || p->num_q_heads <= 0 || p->num_kv_heads <= 0 || p->seq_q <= 0 ||
      p->seq_k <= 0 || p->head_dim <= 0 || p->head_dim % 32 || p->seq_k % 32 ||
      p->num_q_heads % p->num_kv_heads)
    return -1;
  if (block_n <= 0 || block_n % 32 || block_n > ORC_MAX_BLOCK_N) return -1;
  if (p->p_rule != ORC_P_R1 && p->p_rule != ORC_P_R2) return -1;
  if (bh < 0 || bh >= (int64_t)p->batch * p->num_q_heads || qi < 0 || qi >= p->seq_q) return -1;
  int64_t D = p->head_dim, nb = D / 32, Sk = p->seq_k;
  int64_t b = bh / p->num_q_heads, h = bh % p->num_q_heads;
  int64_t kvh = b * p->num_kv_heads + h / (p->num_q_heads / p->num_kv_heads);
  double *kd = malloc(sizeof(double) * Sk * D), *vd = malloc(sizeof(double) * Sk * D);
  double *qd = malloc(sizeof(double) * D), *O = malloc(sizeof(double) * D);
  int64_t sl = Sk > block_n ? Sk : block_n;
  double *S = malloc(sizeof(double) * sl);
  float *P = malloc(sizeof(float) * sl);
  dequant_kv(p, k, k_sc, v, v_sc, kvh, kd, vd);
  const uint8_t *qc = q + (bh * p->seq_q + qi) * D, *qs = q_sc + (bh * p->seq_q + qi) * nb;
  for (int64_t d = 0; d < D; d++) qd[d] = orc_decode_elem(qc[d], ORC_FMT_E4M3) * orc_e8m0_decode(qs[d / 32]);
  orc_trace_t tr = {S_out, codes_out, scales_out, ml_out};
  double m, l;
  flash_pass_tr(p, qd, kd, vd, p->q_pos0 + qi, 0, Sk, block_n, block_n, O, &m, &l, S, P, &tr);
  free(kd); free(vd); free(qd); free(O); free(S); free(P);
  return 0;
}

int orc_attention_dense(const orc_attn_params *p, const uint8_t *q, const uint8_t *q_sc,
                        const uint8_t *k, const uint8_t *k_sc, const uint8_t *v, const uint8_t *v_sc,
                        float *o, const int32_t *heads, int nheads, int nthreads) {
  return run_attention(p, q, q_sc, k, k_sc, v, v_sc, o, 32, 0, 0, 1, heads, nheads, nthreads);
}

/* ------------------------------------------------------------ self-checks */
/* Count float bit patterns b in [lo, hi) (positive, finite) for which the
 * table-based orc_floor_log2f differs from libm's floorf(log2f(x)), the
 * expression the reference evaluates.  Used by the exhaustive tests. */
int64_t orc_check_log2_vs_libm(uint32_t lo, uint32_t hi) {
  int64_t bad = 0;
  for (uint32_t b = lo; b < hi; b++) {
    float x = u2f(b);
    if ((int)floorf(log2f(x)) != orc_floor_log2f(x)) bad++;
  }
  return bad;
}

/* Encode count consecutive float bit patterns from bits_lo (for comparison
 * against the reference's encoder over whole binades). */
void orc_e4m3_encode_range(uint32_t bits_lo, uint32_t count, uint8_t *out) {
  for (uint32_t i = 0; i < count; i++) out[i] = orc_e4m3_encode(u2f(bits_lo + i));
}

void orc_e4m3_encode_array(const float *x, int64_t n, uint8_t *out) {
  for (int64_t i = 0; i < n; i++) out[i] = orc_e4m3_encode(x[i]);
}

/* ------------------------------------------------------------------------------------
 * Rule R4: the reference's SIMT block quantizer (kernels/simt_quant/kernel.cpp:43-117,
 * numpy golden lib/golden/golden.py:129-170).  Block scale e = ceil(log2(amax / 448))
 * from amax's bits: e = (E - 127 - 8) + (mantissa > 0x600000), code clamp(e + 127, 0, 254),
 * amax == 0 -> code 0 and multiplier 1; elements x * 2^-e (fp32 multiply, 2^-e built
 * from bits (127 - e) << 23 as a 32-bit word, as the reference does) encoded with
 * round-half-even, saturation at 448 and E4M3 subnormals kept (grid 2^-9).
 * ------------------------------------------------------------------------------------ */
static uint32_t r4_round_shift(uint32_t v, int sh) {   /* RNE of v / 2^sh, sh > 0 */
  if (sh >= 32) return 0u;
  uint32_t low = v & ((1u << sh) - 1u), half = 1u << (sh - 1), q = v >> sh;
  return q + ((low > half || (low == half && (q & 1u))) ? 1u : 0u);
}

uint8_t orc_r4_encode(float y) {                     /* kernel.cpp:56-81 */
  uint32_t x = f2u(y), s = ((x >> 31) & 1u) << 7, a = x & 0x7fffffffu;
  if (a == 0u) return (uint8_t)s;
  if (u2f(a) >= 448.0f) return (uint8_t)(s | 0x7eu);
  int e = (int)((a >> 23) & 0xffu) - 127;
  uint32_t sig = (1u << 23) | (a & 0x7fffffu);
  if (e < -6) {
    uint32_t q = r4_round_shift(sig, 14 - e);          /* value / 2^-9 */
    return (uint8_t)(s | (q >= 8u ? (8u | (q - 8u)) : q));
  }
  uint32_t r = r4_round_shift(sig, 20);
  int E = e;
  if (r == 16u) { r = 8u; E++; }
  int ef = E + 7;
  uint32_t m = r - 8u;
  if (ef > 15 || (ef == 15 && m == 7u)) return (uint8_t)(s | 0x7eu);
  return (uint8_t)(s | ((uint32_t)ef << 3) | m);
}

uint8_t orc_r4_quantize_block(const float *v, uint8_t *codes) {   /* kernel.cpp:96-117 */
  float amax = 0.0f;
  for (int j = 0; j < 32; j++) {
    float av = u2f(f2u(v[j]) & 0x7fffffffu);
    if (av > amax) amax = av;
  }
  float mul = 1.0f;
  uint8_t sc = 0;
  if (amax != 0.0f) {
    uint32_t ab = f2u(amax);
    int e = ((int)((ab >> 23) & 0xffu) - 127 - 8) + ((ab & 0x7fffffu) > 0x600000u ? 1 : 0);
    int c = e + 127;
    sc = (uint8_t)(c < 0 ? 0 : (c > 254 ? 254 : c));
    mul = u2f((uint32_t)(127 - e) << 23);
  }
  for (int j = 0; j < 32; j++) codes[j] = orc_r4_encode(v[j] * mul);
  return sc;
}

void orc_r4_quantize_rows(const float *x, int64_t rows, int64_t cols, uint8_t *codes, uint8_t *scales) {
  int64_t nb = cols / 32;
  for (int64_t r = 0; r < rows; r++)
    for (int64_t b = 0; b < nb; b++)
      scales[r * nb + b] = orc_r4_quantize_block(x + r * cols + b * 32, codes + r * cols + b * 32);
}

/* Self-checks of the R4 element rule (test infrastructure): over the float bit patterns
 * [lo, hi), count values whose R4 code differs from (mode 0) the R1 code -- the rules
 * coincide from 2^-6 up -- or (mode 1) round-half-even of |y| * 512 on the subnormal grid
 * (exact in double: y * 512 is exact, the rounding is done on the integer and half). */
int64_t orc_r4_check(uint32_t lo, uint32_t hi, int mode) {
  int64_t bad = 0;
  for (uint32_t b = lo; b < hi; b++) {
    float y = u2f(b);
    uint8_t c = orc_r4_encode(y);
    uint8_t want;
    if (mode == 0) {
      want = orc_e4m3_encode(y);
    } else {
      double t = (double)fabsf(y) * 512.0, f = floor(t), d = t - f;
      double q = (d > 0.5 || (d == 0.5 && fmod(f, 2.0) != 0.0)) ? f + 1.0 : f;
      want = (uint8_t)(((b >> 31) << 7) | (q >= 8.0 ? (8u | (uint32_t)(q - 8.0)) : (uint32_t)q));
    }
    bad += c != want;
  }
  return bad;
}

/* ------------------------------------------------------------------------------------
 * Rule R2: the reference device kernels' P requant ("target-0", truncating),
 * kernels/flash_attention_mx_gqa/flash_mx_impl.hpp:53-77 (bf16_floor_log2,
 * bf16_to_e4m3_scaled) and :485-501 / :366-388 (per-block use).  P is bf16; the block
 * exponent se is the unbiased exponent field of the bf16 block maximum, clamped to <= 0,
 * so the maximum maps into [1, 2); scale code se + 127.  An element keeps its bf16
 * exponent minus se and the top 3 bits of its bf16 mantissa (truncation), is flushed
 * when its bf16 exponent field is 0 or the shifted exponent is below -6, and saturates
 * to 448 (E = 8, m = 6) above.
 * ------------------------------------------------------------------------------------ */
uint8_t orc_r2_encode(uint16_t b, int se) {
  int ex = (b >> 7) & 0xff;
  int E = ex - 127 - se;
  if (ex == 0 || E < -6) return 0;
  int m3 = (b >> 4) & 7;
  if (E > 8) {
    E = 8;
    m3 = 6;
  } else if (E == 8 && m3 > 6) {
    m3 = 6;
  }
  return (uint8_t)(((b >> 8) & 0x80) | ((E + 7) << 3) | m3);
}

int orc_r2_scale_exp(float amax) {
  int se = (int)((orc_f32_to_bf16(amax) >> 7) & 0xff) - 127;
  return se > 0 ? 0 : se;
}

/* One block of n <= 32 fp32 probabilities: P rounded to bf16 (written back to pb when
 * non-NULL), scale from the bf16 block maximum, codes.  Returns the E8M0 code. */
uint8_t orc_r2_quantize_block(const float *p, int n, float *pb, uint8_t *codes) {
  uint16_t h[32];
  float amax = 0.0f;
  for (int i = 0; i < n; i++) {
    h[i] = orc_f32_to_bf16(p[i]);
    float v = u2f(((uint32_t)h[i] << 16) & 0x7fffffffu);
    if (v > amax) amax = v;
    if (pb) pb[i] = orc_bf16_to_f32(h[i]);
  }
  int se = orc_r2_scale_exp(amax);
  for (int i = 0; i < n; i++) codes[i] = orc_r2_encode(h[i], se);
  return (uint8_t)(se + 127);
}

void orc_r2_encode_array(const uint16_t *b, const int32_t *se, int64_t n, uint8_t *out) {
  for (int64_t i = 0; i < n; i++) out[i] = orc_r2_encode(b[i], se[i]);
}

void orc_r2_quantize_rows(const float *p, int64_t rows, int64_t cols, float *pb, uint8_t *codes,
                          uint8_t *scales) {
  int64_t nb = cols / 32;
  for (int64_t r = 0; r < rows; r++)
    for (int64_t b = 0; b < nb; b++)
      scales[r * nb + b] = orc_r2_quantize_block(p + r * cols + b * 32, 32, pb ? pb + r * cols + b * 32 : NULL,
                                                 codes + r * cols + b * 32);
}

/* ------------------------------------------------------------------------------------
 * MX GEMM with fp32-style (here: exact, double) accumulation: the tile semantics of the
 * reference's MX-Gemmini GEMM (lib/mxgemm/mxgemm_lib.hpp:11-250; operand layouts of
 * kernels/gemm_mxgemmini/gen_mxgemm_data.py:66-135 and lib/golden/mx_golden.cpp:23-30):
 *   C[m][n] = sum_g 2^(SA[g][m] + SB[g][n] - 254) * sum_{k in g} A[m][k] * B[k][n]
 * with A [M][K] and B [K][N] element codes, SA [K/32][M], SB [K/32][N] E8M0 codes, groups
 * of 32 along K.  Not the Gemmini hardware accumulation (truncated products, narrow
 * per-column accumulators, bf16 group sums) that mx_golden models.  abs_out (optional)
 * receives sum |term| per element, the scale for error bounds.
 * ------------------------------------------------------------------------------------ */
void orc_mx_gemm(const uint8_t *a, const uint8_t *sa, const uint8_t *b, const uint8_t *sb,
                 int64_t M, int64_t N, int64_t K, int a_fmt, int b_fmt, double *c, double *abs_out) {
  int64_t G = K / 32;
  double *bd = malloc(sizeof(double) * K * N);
  for (int64_t k = 0; k < K; k++)
    for (int64_t n = 0; n < N; n++) bd[k * N + n] = orc_decode_elem(b[k * N + n], b_fmt);
  double *ad = malloc(sizeof(double) * K);
  for (int64_t m = 0; m < M; m++) {
    for (int64_t k = 0; k < K; k++) ad[k] = orc_decode_elem(a[m * K + k], a_fmt);
    for (int64_t n = 0; n < N; n++) {
      double acc = 0.0, aacc = 0.0;
      for (int64_t g = 0; g < G; g++) {
        double part = 0.0, apart = 0.0;
        for (int64_t k = 32 * g; k < 32 * g + 32; k++) {
          double t = ad[k] * bd[k * N + n];
          part += t;
          apart += fabs(t);
        }
        double sc = ldexp(1.0, (int)sa[g * M + m] + (int)sb[g * N + n] - 254);
        acc += part * sc;
        aacc += apart * sc;
      }
      c[m * N + n] = acc;
      if (abs_out) abs_out[m * N + n] = aacc;
    }
  }
  free(bd);
  free(ad);
}
