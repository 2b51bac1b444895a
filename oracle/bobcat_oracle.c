/* bobcat_oracle.c — TEST INFRASTRUCTURE ONLY.
 *
 * A CPU restatement, in plain C, of bobcat's scalar reference path: the ops of
 * crates/bobcat/src/scalar.rs and the LFM2 forward pass of
 * crates/bobcat/src/lfm2.rs.  The reference is Rust and cannot be compiled in
 * this image (no cargo/rustc), so this file restates it function by function;
 * each function cites the reference lines it follows.
 *
 * Only the tests, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this library, and only as the checker or the timed CPU baseline.  The
 * product path (bobcat_amd/, libbobcat_hip.so) never links or calls it.
 *
 * Numerics follow the reference exactly where it fixes them: fp16/bf16 decode
 * is bit-exact IEEE, dequantisation rounds each product separately (no FMA
 * contraction: build with -ffp-contract=off), dot products, norms, softmax
 * sums and the convolution accumulate in double and round once to float.
 * Transcendentals (powf, sinf, cosf, expf) come from the host libm, as the
 * reference takes them from the Rust/platform libm.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "../include/bobcat_hip.h"

#define EXPORT __attribute__((visibility("default")))

/* ---------------------------------------------------------------- */
/* Half and bfloat16 (scalar.rs:17-25; the `half` crate 2.7.1 does   */
/* exact IEEE-754 conversion)                                        */
/* ---------------------------------------------------------------- */

static float bits_to_f32(uint32_t bits) {
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

static uint32_t f32_to_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

EXPORT float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exp = (h >> 10) & 0x1f;
  uint32_t man = h & 0x3ff;
  if (exp == 0) {
    if (man == 0) return bits_to_f32(sign);
    /* subnormal: value = man * 2^-24, exact in float */
    float v = (float)man * (1.0f / 16777216.0f);
    return sign ? -v : v;
  }
  if (exp == 31) return bits_to_f32(sign | 0x7f800000u | (man << 13));
  return bits_to_f32(sign | ((exp + 112) << 23) | (man << 13));
}

/* Round-to-nearest-even float -> half, as `half::f16::from_f32` and a GPU's
 * float-to-half conversion do. */
EXPORT uint16_t orc_f32_to_f16(float f) {
  uint32_t x = f32_to_bits(f);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
  uint32_t exp = (x >> 23) & 0xff;
  uint32_t man = x & 0x7fffff;
  if (exp == 0xff) return (uint16_t)(sign | 0x7c00 | (man ? 0x200 | (man >> 13) : 0));
  int e = (int)exp - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7c00);
  if (e <= 0) {
    if (e < -10) return sign;
    man |= 0x800000;
    int shift = 14 - e;
    uint32_t half_man = man >> shift;
    uint32_t rem = man & ((1u << shift) - 1);
    uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (half_man & 1))) half_man++;
    return (uint16_t)(sign | half_man);
  }
  uint32_t half_man = man >> 13;
  uint32_t rem = man & 0x1fff;
  uint16_t out = (uint16_t)(sign | ((uint32_t)e << 10) | half_man);
  if (rem > 0x1000 || (rem == 0x1000 && (half_man & 1))) out++;
  return out;
}

EXPORT float orc_bf16_to_f32(uint16_t b) { return bits_to_f32((uint32_t)b << 16); }

static float f16_at(const uint8_t *p) { return orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* ---------------------------------------------------------------- */
/* Block layouts (crates/bobcat-gguf/src/lib.rs:154-165)             */
/* ---------------------------------------------------------------- */

static int block_shape(uint32_t type, uint32_t *elements, uint32_t *bytes) {
  switch (type) {
    case BCH_F32: *elements = 1; *bytes = 4; return 1;
    case BCH_F16: case BCH_BF16: *elements = 1; *bytes = 2; return 1;
    case BCH_Q4_0: *elements = 32; *bytes = 18; return 1;
    case BCH_Q8_0: *elements = 32; *bytes = 34; return 1;
    case BCH_Q4K: *elements = 256; *bytes = 144; return 1;
    case BCH_Q5K: *elements = 256; *bytes = 176; return 1;
    case BCH_Q6K: *elements = 256; *bytes = 210; return 1;
    default: return 0;
  }
}

/* scalar::row_bytes (scalar.rs:28-31). */
EXPORT uint64_t orc_row_bytes(uint32_t type, uint32_t n_cols) {
  uint32_t e, b;
  if (!block_shape(type, &e, &b) || n_cols % e) return 0;
  return (uint64_t)(n_cols / e) * b;
}

/* ---------------------------------------------------------------- */
/* Dequantisation (scalar.rs:56-202)                                 */
/* ---------------------------------------------------------------- */

/* dequantize_q4_0 (scalar.rs:95-104). */
static void deq_q4_0(const uint8_t *blk, float *out) {
  float d = f16_at(blk);
  for (int i = 0; i < 16; i++) {
    uint8_t q = blk[2 + i];
    out[i] = (float)((int)(q & 0xf) - 8) * d;
    out[i + 16] = (float)((int)(q >> 4) - 8) * d;
  }
}

/* dequantize_q8_0 (scalar.rs:107-112). */
static void deq_q8_0(const uint8_t *blk, float *out) {
  float d = f16_at(blk);
  for (int i = 0; i < 32; i++) out[i] = (float)(int8_t)blk[2 + i] * d;
}

/* q4k_scale_min (scalar.rs:115-125): the 6-bit scale and minimum of
 * 32-element block j from the 12 packed bytes. */
EXPORT void orc_q4k_scale_min(int j, const uint8_t *s, uint8_t *scale, uint8_t *min) {
  if (j < 4) {
    *scale = s[j] & 63;
    *min = s[j + 4] & 63;
  } else {
    *scale = (uint8_t)((s[j + 4] & 0xf) | ((s[j - 4] >> 6) << 4));
    *min = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
  }
}

/* dequantize_q4k (scalar.rs:127-152): element 32j+l of a super-block is
 * (d·sc_j)·q − (dmin·m_j), each product rounded to float on its own. */
static void deq_q4k(const uint8_t *blk, float *out) {
  float d = f16_at(blk), dmin = f16_at(blk + 2);
  const uint8_t *scales = blk + 4, *quants = blk + 16;
  for (int pair = 0; pair < 4; pair++) {
    uint8_t sl, ml, sh, mh;
    orc_q4k_scale_min(2 * pair, scales, &sl, &ml);
    orc_q4k_scale_min(2 * pair + 1, scales, &sh, &mh);
    float d_low = d * (float)sl, m_low = dmin * (float)ml;
    float d_high = d * (float)sh, m_high = dmin * (float)mh;
    const uint8_t *q = quants + 32 * pair;
    float *o = out + 64 * pair;
    for (int l = 0; l < 32; l++) {
      float a = d_low * (float)(q[l] & 0xf);
      float b = d_high * (float)(q[l] >> 4);
      o[l] = a - m_low;
      o[l + 32] = b - m_high;
    }
  }
}

/* dequantize_q5k (scalar.rs:157-176). */
static void deq_q5k(const uint8_t *blk, float *out) {
  float d = f16_at(blk), dmin = f16_at(blk + 2);
  const uint8_t *scales = blk + 4, *high = blk + 16, *quants = blk + 48;
  for (int j = 0; j < 8; j++) {
    uint8_t sc, mn;
    orc_q4k_scale_min(j, scales, &sc, &mn);
    float s = d * (float)sc, m = dmin * (float)mn;
    const uint8_t *q = quants + (j / 2) * 32;
    int shift = 4 * (j % 2);
    for (int l = 0; l < 32; l++) {
      uint8_t v = (uint8_t)(((q[l] >> shift) & 0xf) | (((high[l] >> j) & 1) << 4));
      float p = s * (float)v;
      out[32 * j + l] = p - m;
    }
  }
}

/* dequantize_q6k (scalar.rs:181-202). */
static void deq_q6k(const uint8_t *blk, float *out) {
  float d = f16_at(blk + 208);
  for (int half = 0; half < 2; half++) {
    const uint8_t *low = blk + half * 64, *high = blk + 128 + half * 32;
    const int8_t *sc = (const int8_t *)(blk + 192 + half * 8);
    float *o = out + half * 128;
    for (int l = 0; l < 32; l++) {
      int is = l / 16;
#define Q6(lowv, sh) ((float)((int)((lowv) | (((high[l] >> (sh)) & 3) << 4)) - 32))
#define SC(i) (d * (float)sc[i])
      o[l] = SC(is) * Q6(low[l] & 0xf, 0);
      o[l + 32] = SC(is + 2) * Q6(low[l + 32] & 0xf, 2);
      o[l + 64] = SC(is + 4) * Q6(low[l] >> 4, 4);
      o[l + 96] = SC(is + 6) * Q6(low[l + 32] >> 4, 6);
#undef Q6
#undef SC
    }
  }
}

/* scalar::dequantize (scalar.rs:59-79): n elements of `type` at bytes. */
EXPORT int orc_dequantize(uint32_t type, const void *bytes, uint64_t n, float *out) {
  const uint8_t *p = (const uint8_t *)bytes;
  uint32_t e, b;
  if (!block_shape(type, &e, &b) || n % e) return -1;
  uint64_t nb = n / e;
  for (uint64_t i = 0; i < nb; i++) {
    const uint8_t *blk = p + i * b;
    float *o = out + i * e;
    switch (type) {
      case BCH_F32: memcpy(o, blk, 4); break;
      case BCH_F16: *o = f16_at(blk); break;
      case BCH_BF16: *o = orc_bf16_to_f32((uint16_t)(blk[0] | (blk[1] << 8))); break;
      case BCH_Q4_0: deq_q4_0(blk, o); break;
      case BCH_Q8_0: deq_q8_0(blk, o); break;
      case BCH_Q4K: deq_q4k(blk, o); break;
      case BCH_Q5K: deq_q5k(blk, o); break;
      case BCH_Q6K: deq_q6k(blk, o); break;
    }
  }
  return 0;
}

/* ---------------------------------------------------------------- */
/* Vector ops (scalar.rs:213-304)                                    */
/* ---------------------------------------------------------------- */

/* scalar::dot (scalar.rs:292-304): double sum rounded once. */
EXPORT float orc_dot(const float *a, const float *b, uint64_t n) {
  double s = 0.0;
  for (uint64_t i = 0; i < n; i++) s += (double)a[i] * (double)b[i];
  return (float)s;
}

static int g_threads = 1;
EXPORT void orc_set_threads(int n) { g_threads = n < 1 ? 1 : n; }
EXPORT int orc_get_threads(void) { return g_threads; }

typedef struct {
  uint32_t type;
  const uint8_t *w;
  uint64_t row_bytes;
  const float *x;
  float *y;
  uint32_t cols;
  uint64_t r0, r1;
} mv_job;

static void *mv_run(void *arg) {
  mv_job *j = (mv_job *)arg;
  float *row = (float *)malloc(sizeof(float) * j->cols);
  for (uint64_t r = j->r0; r < j->r1; r++) {
    orc_dequantize(j->type, j->w + r * j->row_bytes, j->cols, row);
    j->y[r] = orc_dot(row, j->x, j->cols);
  }
  free(row);
  return NULL;
}

/* scalar::matvec (scalar.rs:213-220): each row dequantised, then dotted with
 * x in double.  Rows split over orc_set_threads() threads; every row's
 * arithmetic is the same, so the result does not depend on the count. */
EXPORT int orc_matvec(uint32_t type, const void *weights, uint32_t rows, uint32_t cols,
                      const float *x, float *y) {
  uint64_t rb = orc_row_bytes(type, cols);
  if (!rb) return -1;
  int nt = g_threads;
  if ((uint64_t)nt > rows) nt = rows ? (int)rows : 1;
  mv_job jobs[256];
  pthread_t th[256];
  if (nt > 256) nt = 256;
  for (int t = 0; t < nt; t++) {
    jobs[t] = (mv_job){type, (const uint8_t *)weights, rb, x, y, cols,
                       (uint64_t)rows * t / nt, (uint64_t)rows * (t + 1) / nt};
  }
  if (nt == 1) {
    mv_run(&jobs[0]);
    return 0;
  }
  for (int t = 0; t < nt; t++) pthread_create(&th[t], NULL, mv_run, &jobs[t]);
  for (int t = 0; t < nt; t++) pthread_join(th[t], NULL);
  return 0;
}

/* rms_scale (scalar.rs:239-249): 1/sqrt(mean(x²)+eps) in double, rounded. */
static float rms_scale(const float *x, uint64_t n, float eps) {
  double s = 0.0;
  for (uint64_t i = 0; i < n; i++) s += (double)x[i] * (double)x[i];
  double mean = s / (double)n;
  return (float)(1.0 / sqrt(mean + (double)eps));
}

/* scalar::rms_norm (scalar.rs:222-229): out = w·(x·scale). */
EXPORT void orc_rms_norm(const float *x, const float *w, uint64_t n, float eps, float *out) {
  float scale = rms_scale(x, n, eps);
  for (uint64_t i = 0; i < n; i++) out[i] = w[i] * (x[i] * scale);
}

/* scalar::rope_neox (scalar.rs:251-266): element i pairs with i + d/2;
 * frequencies and angles in float, as transformers computes them. */
EXPORT void orc_rope_neox(float *v, uint32_t head_dim, uint32_t pos, float theta) {
  uint32_t half = head_dim / 2;
  for (uint32_t i = 0; i < half; i++) {
    float inv_freq = 1.0f / powf(theta, (float)(2 * i) / (float)head_dim);
    float angle = (float)pos * inv_freq;
    float s = sinf(angle), c = cosf(angle);
    float a = v[i], b = v[i + half];
    v[i] = a * c - b * s;
    v[i + half] = b * c + a * s;
  }
}

/* scalar::silu (scalar.rs:268-271). */
EXPORT float orc_silu(float x) { return x / (1.0f + expf(-x)); }

/* scalar::softmax (scalar.rs:273-289): float exponentials, double sum. */
EXPORT void orc_softmax(float *x, uint64_t n) {
  float max = -INFINITY;
  for (uint64_t i = 0; i < n; i++) max = fmaxf(max, x[i]);
  double sum = 0.0;
  for (uint64_t i = 0; i < n; i++) {
    x[i] = expf(x[i] - max);
    sum += (double)x[i];
  }
  for (uint64_t i = 0; i < n; i++) x[i] = (float)((double)x[i] / sum);
}

/* ---------------------------------------------------------------- */
/* LFM2 forward pass (lfm2.rs:300-560, 677-722)                      */
/* ---------------------------------------------------------------- */

/* lfm2::State (lfm2.rs:565-629). */
typedef struct orc_lfm2_state {
  uint32_t n_ctx, n_past;
  float *k_cache, *v_cache, *conv_history;
  float *hidden, *normed, *block_out, *bcx, *conv_out, *q, *k, *v, *attn, *scores;
  float *gate, *up, *router, *expert_out;
  uint32_t *experts;
} orc_lfm2_state;

static uint32_t count_layers(const bch_lfm2_model *m, int attention) {
  uint32_t n = 0;
  for (uint32_t i = 0; i < m->n_layers; i++) n += (m->layers[i].is_attention != 0) == (attention != 0);
  return n;
}

/* State::new (lfm2.rs:599-628). */
EXPORT orc_lfm2_state *orc_lfm2_state_new(const bch_lfm2_model *m, uint32_t n_ctx) {
  if (n_ctx == 0) return NULL;
  orc_lfm2_state *s = (orc_lfm2_state *)calloc(1, sizeof(*s));
  uint64_t n = m->n_embd, kv = (uint64_t)m->n_kv_heads * m->head_dim, qd = (uint64_t)m->n_heads * m->head_dim;
  uint64_t cache = (uint64_t)count_layers(m, 1) * n_ctx * kv;
  uint64_t conv = (uint64_t)count_layers(m, 0) * (m->conv_kernel - 1) * n;
  uint64_t nff = m->n_ff > m->n_ff_expert ? m->n_ff : m->n_ff_expert;
  s->n_ctx = n_ctx;
  s->k_cache = calloc(cache + 1, 4);
  s->v_cache = calloc(cache + 1, 4);
  s->conv_history = calloc(conv + 1, 4);
  s->hidden = calloc(n, 4);
  s->normed = calloc(n, 4);
  s->block_out = calloc(n, 4);
  s->bcx = calloc(3 * n, 4);
  s->conv_out = calloc(n, 4);
  s->q = calloc(qd, 4);
  s->k = calloc(kv + 1, 4);
  s->v = calloc(kv + 1, 4);
  s->attn = calloc(qd, 4);
  s->scores = calloc(n_ctx, 4);
  s->gate = calloc(nff, 4);
  s->up = calloc(nff, 4);
  s->router = calloc(m->n_experts + 1, 4);
  s->experts = calloc(m->n_experts + 1, 4);
  s->expert_out = calloc(n, 4);
  return s;
}

EXPORT void orc_lfm2_state_free(orc_lfm2_state *s) {
  if (!s) return;
  void *ptrs[] = {s->k_cache, s->v_cache, s->conv_history, s->hidden, s->normed, s->block_out,
                  s->bcx, s->conv_out, s->q, s->k, s->v, s->attn, s->scores, s->gate, s->up,
                  s->router, s->experts, s->expert_out};
  for (size_t i = 0; i < sizeof(ptrs) / sizeof(ptrs[0]); i++) free(ptrs[i]);
  free(s);
}

EXPORT uint32_t orc_lfm2_n_past(const orc_lfm2_state *s) { return s->n_past; }

static void matvec_m(const bch_matrix *mat, const float *x, float *y) {
  orc_matvec(mat->format, mat->data, mat->n_rows, mat->n_cols, x, y);
}

/* Model::matvec_rows (lfm2.rs:397-401): rows first_row.. of a matrix. */
static void matvec_rows(const bch_matrix *mat, uint64_t first_row, uint32_t rows, const float *x,
                        float *y) {
  uint64_t rb = orc_row_bytes(mat->format, mat->n_cols);
  orc_matvec(mat->format, (const uint8_t *)mat->data + first_row * rb, rows, mat->n_cols, x, y);
}

/* swiglu (lfm2.rs:677-682). */
static void swiglu(float *gate, const float *up, uint64_t n) {
  for (uint64_t i = 0; i < n; i++) gate[i] = orc_silu(gate[i]) * up[i];
}

/* route (lfm2.rs:691-709): sigmoid scores, stable descending sort of
 * score + bias (ties to the lower expert), weights = score / (Σpicked + 1e-6). */
EXPORT void orc_lfm2_route(float *scores, const float *bias, uint32_t n_experts, uint32_t n_used,
                           uint32_t *experts) {
  for (uint32_t e = 0; e < n_experts; e++) scores[e] = 1.0f / (1.0f + expf(-scores[e]));
  for (uint32_t e = 0; e < n_experts; e++) experts[e] = e;
  /* insertion sort is stable */
  for (uint32_t i = 1; i < n_experts; i++) {
    uint32_t cur = experts[i];
    float key = scores[cur] + bias[cur];
    int32_t j = (int32_t)i - 1;
    while (j >= 0 && scores[experts[j]] + bias[experts[j]] < key) {
      experts[j + 1] = experts[j];
      j--;
    }
    experts[j + 1] = cur;
  }
  float sum = 0.0f;
  for (uint32_t i = 0; i < n_used; i++) sum += scores[experts[i]];
  float norm = sum + 1e-6f;
  for (uint32_t i = 0; i < n_used; i++) scores[experts[i]] /= norm;
}

/* Model::moe_block (lfm2.rs:413-440). */
static void moe_block(const bch_lfm2_model *m, const bch_lfm2_layer *L, orc_lfm2_state *s) {
  uint32_t n = m->n_embd, nff = m->n_ff_expert, nu = m->n_experts_used;
  matvec_m(&L->router, s->normed, s->router);
  orc_lfm2_route(s->router, L->expert_bias, m->n_experts, nu, s->experts);
  memset(s->block_out, 0, sizeof(float) * n);
  for (uint32_t i = 0; i < nu; i++) {
    uint32_t e = s->experts[i];
    matvec_rows(&L->gate_exps, (uint64_t)e * nff, nff, s->normed, s->gate);
    matvec_rows(&L->up_exps, (uint64_t)e * nff, nff, s->normed, s->up);
    swiglu(s->gate, s->up, nff);
    matvec_rows(&L->down_exps, (uint64_t)e * n, n, s->gate, s->expert_out);
    float w = s->router[e];
    for (uint32_t c = 0; c < n; c++) s->block_out[c] += w * s->expert_out[c];
  }
}

/* Model::dense_block (lfm2.rs:404-409). */
static void dense_block(const bch_lfm2_layer *L, orc_lfm2_state *s) {
  matvec_m(&L->gate, s->normed, s->gate);
  matvec_m(&L->up, s->normed, s->up);
  swiglu(s->gate, s->up, L->gate.n_rows);
  matvec_m(&L->down, s->gate, s->block_out);
}

/* Model::conv_block (lfm2.rs:444-478). */
static void conv_block(const bch_lfm2_model *m, const bch_lfm2_layer *L, uint32_t cache_index,
                       orc_lfm2_state *s) {
  uint32_t n = m->n_embd, k = m->conv_kernel;
  float *hist = s->conv_history + (uint64_t)cache_index * (k - 1) * n;
  matvec_m(&L->in_proj, s->normed, s->bcx);
  const float *b = s->bcx, *c = s->bcx + n, *x = s->bcx + 2 * n;
  for (uint32_t ch = 0; ch < n; ch++) {
    const float *taps = L->conv_taps + (uint64_t)ch * k;
    float bx = b[ch] * x[ch];
    double sum = (double)taps[k - 1] * (double)bx;
    for (uint32_t t = 0; t + 1 < k; t++) sum += (double)taps[t] * (double)hist[t * n + ch];
    for (uint32_t t = 0; t + 2 < k; t++) hist[t * n + ch] = hist[(t + 1) * n + ch];
    hist[(k - 2) * n + ch] = bx;
    s->conv_out[ch] = c[ch] * (float)sum;
  }
  matvec_m(&L->out_proj, s->conv_out, s->block_out);
}

/* scalar::rms_norm_in_place (scalar.rs:232-237). */
static void rms_norm_in_place(float *x, const float *w, uint64_t n, float eps) {
  float scale = rms_scale(x, n, eps);
  for (uint64_t i = 0; i < n; i++) x[i] = w[i] * (x[i] * scale);
}

/* Model::attention_block (lfm2.rs:482-560). */
static void attention_block(const bch_lfm2_model *m, const bch_lfm2_layer *L, uint32_t cache_index,
                            orc_lfm2_state *s, uint32_t pos) {
  uint32_t hd = m->head_dim, kvd = m->n_kv_heads * hd, group = m->n_heads / m->n_kv_heads;
  float scale = 1.0f / sqrtf((float)hd);
  uint64_t layer_len = (uint64_t)s->n_ctx * kvd;
  float *kc = s->k_cache + cache_index * layer_len, *vc = s->v_cache + cache_index * layer_len;
  matvec_m(&L->wq, s->normed, s->q);
  matvec_m(&L->wk, s->normed, s->k);
  matvec_m(&L->wv, s->normed, s->v);
  for (uint32_t h = 0; h < m->n_heads; h++) {
    rms_norm_in_place(s->q + h * hd, L->q_norm, hd, m->norm_eps);
    orc_rope_neox(s->q + h * hd, hd, pos, m->rope_theta);
  }
  for (uint32_t h = 0; h < m->n_kv_heads; h++) {
    rms_norm_in_place(s->k + h * hd, L->k_norm, hd, m->norm_eps);
    orc_rope_neox(s->k + h * hd, hd, pos, m->rope_theta);
  }
  memcpy(kc + (uint64_t)pos * kvd, s->k, sizeof(float) * kvd);
  memcpy(vc + (uint64_t)pos * kvd, s->v, sizeof(float) * kvd);
  uint32_t n_keys = pos + 1;
  for (uint32_t h = 0; h < m->n_heads; h++) {
    uint32_t kv_off = h / group * hd;
    const float *qh = s->q + h * hd;
    for (uint32_t t = 0; t < n_keys; t++) s->scores[t] = scale * orc_dot(qh, kc + (uint64_t)t * kvd + kv_off, hd);
    orc_softmax(s->scores, n_keys);
    for (uint32_t d = 0; d < hd; d++) {
      double sum = 0.0;
      for (uint32_t t = 0; t < n_keys; t++) sum += (double)s->scores[t] * (double)vc[(uint64_t)t * kvd + kv_off + d];
      s->attn[h * hd + d] = (float)sum;
    }
  }
  matvec_m(&L->wo, s->attn, s->block_out);
}

/* Model::step (lfm2.rs:308-394).  Returns 0, or -1 for a full context, -2
 * for a token outside the vocabulary (Error::ContextFull / Error::Token). */
EXPORT int orc_lfm2_step(const bch_lfm2_model *m, orc_lfm2_state *s, uint32_t token, float *logits,
                         float *trace_embedding, float *trace_layers, float *trace_final) {
  uint32_t n = m->n_embd, pos = s->n_past;
  if (pos >= s->n_ctx) return -1;
  if (token >= m->n_vocab) return -2;
  uint64_t rb = orc_row_bytes(m->token_embd.format, n);
  orc_dequantize(m->token_embd.format, (const uint8_t *)m->token_embd.data + (uint64_t)token * rb, n,
                 s->hidden);
  if (trace_embedding) memcpy(trace_embedding, s->hidden, sizeof(float) * n);
  uint32_t attn_index = 0, conv_index = 0;
  for (uint32_t il = 0; il < m->n_layers; il++) {
    const bch_lfm2_layer *L = &m->layers[il];
    orc_rms_norm(s->hidden, L->attn_norm, n, m->norm_eps, s->normed);
    if (L->is_attention)
      attention_block(m, L, attn_index++, s, pos);
    else
      conv_block(m, L, conv_index++, s);
    for (uint32_t i = 0; i < n; i++) s->hidden[i] += s->block_out[i];
    orc_rms_norm(s->hidden, L->ffn_norm, n, m->norm_eps, s->normed);
    if (L->is_moe)
      moe_block(m, L, s);
    else
      dense_block(L, s);
    for (uint32_t i = 0; i < n; i++) s->hidden[i] += s->block_out[i];
    if (trace_layers) memcpy(trace_layers + (uint64_t)il * n, s->hidden, sizeof(float) * n);
  }
  orc_rms_norm(s->hidden, m->output_norm, n, m->norm_eps, s->normed);
  if (trace_final) memcpy(trace_final, s->normed, sizeof(float) * n);
  if (logits) matvec_m(&m->output, s->normed, logits);
  s->n_past++;
  return 0;
}

/* ---------------------------------------------------------------- */
/* Stand-alone pieces of the forward pass, for kernel-level checks   */
/* ---------------------------------------------------------------- */

/* The gated short convolution of conv_block (lfm2.rs:456-475) over
 * n_tokens rows of bcx ([B | C | X] per token), carrying `history`. */
EXPORT void orc_short_conv(const float *bcx, const float *taps, float *hist, float *out, uint32_t n,
                           uint32_t k, uint32_t n_tokens) {
  for (uint32_t t = 0; t < n_tokens; t++) {
    const float *b = bcx + (uint64_t)t * 3 * n, *c = b + n, *x = b + 2 * n;
    for (uint32_t ch = 0; ch < n; ch++) {
      const float *tp = taps + (uint64_t)ch * k;
      float bx = b[ch] * x[ch];
      double sum = (double)tp[k - 1] * (double)bx;
      for (uint32_t j = 0; j + 1 < k; j++) sum += (double)tp[j] * (double)hist[j * n + ch];
      for (uint32_t j = 0; j + 2 < k; j++) hist[j * n + ch] = hist[(j + 1) * n + ch];
      hist[(k - 2) * n + ch] = bx;
      out[(uint64_t)t * n + ch] = c[ch] * (float)sum;
    }
  }
}

/* The causal attention of attention_block (lfm2.rs:520-556) for n_queries
 * queries at positions first_pos.., over f32 caches [pos][n_kv][hd]. */
EXPORT void orc_attention(const float *q, const float *kc, const float *vc, float *out, uint32_t n_heads,
                          uint32_t n_kv, uint32_t hd, uint32_t first_pos, uint32_t n_queries) {
  uint32_t kvd = n_kv * hd, group = n_heads / n_kv;
  float scale = 1.0f / sqrtf((float)hd);
  float *scores = (float *)malloc(sizeof(float) * (first_pos + n_queries));
  for (uint32_t qi = 0; qi < n_queries; qi++) {
    uint32_t n_keys = first_pos + qi + 1;
    for (uint32_t h = 0; h < n_heads; h++) {
      const float *qh = q + ((uint64_t)qi * n_heads + h) * hd;
      uint32_t kv_off = h / group * hd;
      for (uint32_t t = 0; t < n_keys; t++) scores[t] = scale * orc_dot(qh, kc + (uint64_t)t * kvd + kv_off, hd);
      orc_softmax(scores, n_keys);
      for (uint32_t d = 0; d < hd; d++) {
        double sum = 0.0;
        for (uint32_t t = 0; t < n_keys; t++) sum += (double)scores[t] * (double)vc[(uint64_t)t * kvd + kv_off + d];
        out[((uint64_t)qi * n_heads + h) * hd + d] = (float)sum;
      }
    }
  }
  free(scores);
}

/* ---------------------------------------------------------------- */
/* Sampling: Sampler::sample (crates/bobcat-cli/src/sampler.rs:45-129)  */
/* ---------------------------------------------------------------- */

/* wyrand as in fastrand 2.5.0 (Cargo.lock:956-958; not vendored in the
 * reference): state += 0x2d358dccaa6c78a5; the 128-bit product of the state
 * and state ^ 0x8bb84b93962eacc9 folded to 64 bits.  f32: the 23 high bits
 * of the low 32-bit half as the mantissa of [1, 2), minus one.  No golden
 * draws exist in the reference, so the draw stream is parity unpinned. */
EXPORT uint64_t orc_wyrand(uint64_t *state) {
  uint64_t s = *state + 0x2d358dccaa6c78a5ull;
  *state = s;
  unsigned __int128 t = (unsigned __int128)s * (unsigned __int128)(s ^ 0x8bb84b93962eacc9ull);
  return (uint64_t)t ^ (uint64_t)(t >> 64);
}

EXPORT float orc_wyrand_f32(uint64_t *state) {
  uint32_t u = (uint32_t)orc_wyrand(state);
  uint32_t bits = 0x3f800000u | (u >> 9);
  float f;
  memcpy(&f, &bits, 4);
  return f - 1.0f;
}

typedef struct { uint32_t id; float v; } orc_cand;

static int by_logit_desc(const void *a, const void *b) {
  const orc_cand *x = a, *y = b;
  if (x->v > y->v) return -1;
  if (x->v < y->v) return 1;
  return x->id < y->id ? -1 : x->id > y->id;
}

/* softmax (sampler.rs:116-128): sequential f32 sums, as the reference. */
static void cand_softmax(orc_cand *c, uint32_t n, float temperature) {
  float max = -INFINITY;
  for (uint32_t i = 0; i < n; i++) max = c[i].v > max ? c[i].v : max;
  float sum = 0.0f;
  for (uint32_t i = 0; i < n; i++) {
    c[i].v = expf((c[i].v - max) / temperature);
    sum += c[i].v;
  }
  for (uint32_t i = 0; i < n; i++) c[i].v /= sum;
}

/* Sampler::sample (sampler.rs:45-112).  The draw comes from `rng` (fastrand's
 * f32, advancing the state) or, when `rng` is NULL, is `u` itself: the
 * reference's loop over the candidates with `draw` given, so tests can place
 * it on either side of a candidate boundary. */
static uint32_t sample_core(float *logits, uint32_t n, const uint32_t *recent, uint32_t n_recent,
                            const bch_sampling *st, uint64_t *rng, float u) {
  if (fabsf(st->repeat_penalty - 1.0f) > 1.1920929e-7f) {
    uint32_t start = n_recent > 64 ? n_recent - 64 : 0;
    for (uint32_t i = start; i < n_recent; i++) {
      int seen = 0;
      for (uint32_t j = start; j < i; j++) seen |= recent[j] == recent[i];
      if (seen || recent[i] >= n) continue;
      float *l = &logits[recent[i]];
      *l = *l > 0.0f ? *l / st->repeat_penalty : *l * st->repeat_penalty;
    }
  }
  if (st->temperature <= 0.0f) {
    uint32_t best = 0;
    for (uint32_t i = 1; i < n; i++)
      if (logits[i] > logits[best]) best = i;
    return best;
  }
  orc_cand *c = malloc((size_t)n * sizeof(orc_cand));
  for (uint32_t i = 0; i < n; i++) c[i] = (orc_cand){i, logits[i]};
  qsort(c, n, sizeof(orc_cand), by_logit_desc);
  uint32_t m = (st->top_k > 0 && st->top_k < n) ? st->top_k : n;
  cand_softmax(c, m, 1.0f);
  float cum = 0.0f;
  uint32_t keep = m;
  for (uint32_t i = 0; i < m; i++) {
    cum += c[i].v;
    if (cum >= st->top_p) {
      keep = i + 1;
      break;
    }
  }
  float floor_p = c[0].v * st->min_p;
  uint32_t kept = 0;
  for (uint32_t i = 0; i < keep; i++)
    if (c[i].v >= floor_p) c[kept++] = c[i];
  for (uint32_t i = 0; i < kept; i++) c[i].v = logf(c[i].v);
  cand_softmax(c, kept, st->temperature);
  float draw = rng ? orc_wyrand_f32(rng) : u;
  uint32_t token = kept ? c[kept - 1].id : 0;
  for (uint32_t i = 0; i < kept; i++) {
    if (draw < c[i].v) {
      token = c[i].id;
      break;
    }
    draw -= c[i].v;
  }
  free(c);
  return token;
}

EXPORT uint32_t orc_sample(float *logits, uint32_t n, const uint32_t *recent, uint32_t n_recent,
                           const bch_sampling *st, uint64_t *rng) {
  return sample_core(logits, n, recent, n_recent, st, rng, 0.0f);
}

/* orc_sample with the draw given (0 <= u < 1) instead of taken from a generator. */
EXPORT uint32_t orc_sample_u(float *logits, uint32_t n, const uint32_t *recent, uint32_t n_recent,
                             const bch_sampling *st, float u) {
  return sample_core(logits, n, recent, n_recent, st, NULL, u);
}

/* fastrand's f32 of a 32-bit draw: its 23 high bits as the mantissa of a
 * float in [1, 2), minus one (Rng::f32). */
EXPORT float orc_u32_to_f32(uint32_t x) {
  uint32_t bits = 0x3f800000u | (x >> 9);
  float f;
  memcpy(&f, &bits, 4);
  return f - 1.0f;
}

/* ---------------------------------------------------------------- */
/* Qwen3.5 forward pass (qwen35.rs:280-516, 761-778)                 */
/* ---------------------------------------------------------------- */

/* qwen35::State (qwen35.rs:533-640): caches, DeltaNet states, scratch. */
typedef struct orc_qwen35_state {
  uint32_t n_ctx, n_past;
  float *k_cache, *v_cache;         /* [attn layer][pos][kv_dim] */
  float *conv, *state;              /* [delta layer][conv_dim][k-1], [delta layer][n_v][k_dim][v_dim] */
  float *h, *x, *mixer_out, *ffn_gate, *ffn_up, *q_gate, *q, *attn_gate, *k, *v, *attn, *scores;
  float *qkv, *conv_out, *z, *beta, *alpha, *delta, *delta_out;
} orc_qwen35_state;

static uint32_t q35_count(const bch_qwen35_model *m, int attention) {
  uint32_t n = 0;
  for (uint32_t i = 0; i < m->n_layers; i++) n += (m->layers[i].is_attention != 0) == (attention != 0);
  return n;
}

EXPORT orc_qwen35_state *orc_qwen35_state_new(const bch_qwen35_model *m, uint32_t n_ctx) {
  if (n_ctx == 0) return NULL;
  orc_qwen35_state *s = calloc(1, sizeof(*s));
  uint64_t n = m->n_embd, kvd = (uint64_t)m->n_kv_heads * m->head_dim, qd = (uint64_t)m->n_heads * m->head_dim;
  uint64_t key_dim = (uint64_t)m->n_k_heads * m->k_head_dim, value_dim = (uint64_t)m->n_v_heads * m->v_head_dim;
  uint64_t conv_dim = 2 * key_dim + value_dim;
  uint32_t na = q35_count(m, 1), nd = q35_count(m, 0);
  s->n_ctx = n_ctx;
  s->k_cache = calloc((uint64_t)na * n_ctx * kvd + 1, 4);
  s->v_cache = calloc((uint64_t)na * n_ctx * kvd + 1, 4);
  s->conv = calloc((uint64_t)nd * conv_dim * (m->conv_kernel - 1) + 1, 4);
  s->state = calloc((uint64_t)nd * m->n_v_heads * m->k_head_dim * m->v_head_dim + 1, 4);
  s->h = calloc(n, 4);
  s->x = calloc(n, 4);
  s->mixer_out = calloc(n, 4);
  s->ffn_gate = calloc(m->n_ff, 4);
  s->ffn_up = calloc(m->n_ff, 4);
  s->q_gate = calloc(2 * qd + 1, 4);
  s->q = calloc(qd + 1, 4);
  s->attn_gate = calloc(qd + 1, 4);
  s->k = calloc(kvd + 1, 4);
  s->v = calloc(kvd + 1, 4);
  s->attn = calloc(qd + 1, 4);
  s->scores = calloc(n_ctx, 4);
  s->qkv = calloc(conv_dim + 1, 4);
  s->conv_out = calloc(conv_dim + 1, 4);
  s->z = calloc(value_dim + 1, 4);
  s->beta = calloc(m->n_v_heads + 1, 4);
  s->alpha = calloc(m->n_v_heads + 1, 4);
  s->delta = calloc(m->v_head_dim + 1, 4);
  s->delta_out = calloc(value_dim + 1, 4);
  return s;
}

EXPORT void orc_qwen35_state_free(orc_qwen35_state *s) {
  if (!s) return;
  void *p[] = {s->k_cache, s->v_cache, s->conv, s->state, s->h, s->x, s->mixer_out, s->ffn_gate, s->ffn_up,
               s->q_gate, s->q, s->attn_gate, s->k, s->v, s->attn, s->scores, s->qkv, s->conv_out, s->z,
               s->beta, s->alpha, s->delta, s->delta_out};
  for (size_t i = 0; i < sizeof(p) / sizeof(p[0]); i++) free(p[i]);
  free(s);
}

EXPORT uint32_t orc_qwen35_n_past(const orc_qwen35_state *s) { return s->n_past; }

static float q35_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

/* softplus (qwen35.rs:775-778): x above 20, else ln(1 + e^x). */
static float q35_softplus(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

/* l2_normalize (qwen35.rs:761-768): sequential f32 sum, eps 1e-6. */
static void q35_l2(float *x, uint32_t n, float scale) {
  float sum = 0.0f;
  for (uint32_t i = 0; i < n; i++) sum += x[i] * x[i];
  float factor = scale / sqrtf(sum + 1e-6f);
  for (uint32_t i = 0; i < n; i++) x[i] *= factor;
}

/* Model::attention (qwen35.rs:369-426). */
static void q35_attention(const bch_qwen35_model *m, const bch_qwen35_layer *L, uint32_t ci, uint32_t pos,
                          orc_qwen35_state *s) {
  uint32_t hd = m->head_dim, nh = m->n_heads, nkv = m->n_kv_heads, kvd = nkv * hd, group = nh / nkv;
  matvec_m(&L->wq, s->x, s->q_gate);
  matvec_m(&L->wk, s->x, s->k);
  matvec_m(&L->wv, s->x, s->v);
  for (uint32_t h = 0; h < nh; h++) {
    const float *block = s->q_gate + 2ull * h * hd;
    float *q = s->q + (uint64_t)h * hd;
    memcpy(q, block, 4ull * hd);
    rms_norm_in_place(q, L->q_norm, hd, m->norm_eps);
    orc_rope_neox(q, m->n_rot, pos, m->rope_theta);
    memcpy(s->attn_gate + (uint64_t)h * hd, block + hd, 4ull * hd);
  }
  for (uint32_t h = 0; h < nkv; h++) {
    float *k = s->k + (uint64_t)h * hd;
    rms_norm_in_place(k, L->k_norm, hd, m->norm_eps);
    orc_rope_neox(k, m->n_rot, pos, m->rope_theta);
  }
  float *kc = s->k_cache + (uint64_t)ci * s->n_ctx * kvd, *vc = s->v_cache + (uint64_t)ci * s->n_ctx * kvd;
  memcpy(kc + (uint64_t)pos * kvd, s->k, 4ull * kvd);
  memcpy(vc + (uint64_t)pos * kvd, s->v, 4ull * kvd);
  uint32_t n_keys = pos + 1;
  float scale = 1.0f / sqrtf((float)hd);
  for (uint32_t h = 0; h < nh; h++) {
    uint32_t kvh = h / group;
    const float *q = s->q + (uint64_t)h * hd;
    for (uint32_t t = 0; t < n_keys; t++) s->scores[t] = orc_dot(q, kc + (uint64_t)t * kvd + kvh * hd, hd) * scale;
    orc_softmax(s->scores, n_keys);
    float *out = s->attn + (uint64_t)h * hd;
    for (uint32_t d = 0; d < hd; d++) out[d] = 0.0f;
    for (uint32_t t = 0; t < n_keys; t++) {
      const float *v = vc + (uint64_t)t * kvd + kvh * hd;
      for (uint32_t d = 0; d < hd; d++) out[d] += s->scores[t] * v[d];
    }
  }
  for (uint64_t i = 0; i < (uint64_t)nh * hd; i++) s->attn[i] *= q35_sigmoid(s->attn_gate[i]);
  matvec_m(&L->wo, s->attn, s->mixer_out);
}

/* Model::delta_net (qwen35.rs:430-516). */
static void q35_delta(const bch_qwen35_model *m, const bch_qwen35_layer *L, uint32_t ci, orc_qwen35_state *s) {
  uint32_t K = m->conv_kernel, hist = K - 1, nk = m->n_k_heads, nv = m->n_v_heads, dk = m->k_head_dim,
           dv = m->v_head_dim;
  uint64_t key_dim = (uint64_t)nk * dk, conv_dim = 2 * key_dim + (uint64_t)nv * dv;
  float *conv = s->conv + (uint64_t)ci * conv_dim * hist;
  float *state = s->state + (uint64_t)ci * nv * dk * dv;
  matvec_m(&L->qkv, s->x, s->qkv);
  matvec_m(&L->z, s->x, s->z);
  matvec_m(&L->beta, s->x, s->beta);
  matvec_m(&L->alpha, s->x, s->alpha);
  for (uint64_t c = 0; c < conv_dim; c++) {
    const float *taps = L->conv_taps + c * K;
    float *past = conv + c * hist;
    float input = s->qkv[c];
    float sum = taps[hist] * input;
    for (uint32_t j = 0; j < hist; j++) sum += taps[j] * past[j];
    s->conv_out[c] = orc_silu(sum);
    for (uint32_t j = 0; j + 1 < hist; j++) past[j] = past[j + 1];
    if (hist) past[hist - 1] = input;
  }
  float *q = s->conv_out, *k = s->conv_out + key_dim, *v = s->conv_out + 2 * key_dim;
  float q_scale = 1.0f / sqrtf((float)dk);
  for (uint32_t h = 0; h < nk; h++) {
    q35_l2(q + (uint64_t)h * dk, dk, q_scale);
    q35_l2(k + (uint64_t)h * dk, dk, 1.0f);
  }
  for (uint32_t h = 0; h < nv; h++) {
    uint32_t kh = h % nk;
    const float *qh = q + (uint64_t)kh * dk, *kk = k + (uint64_t)kh * dk, *vh = v + (uint64_t)h * dv;
    float beta = q35_sigmoid(s->beta[h]);
    float decay = expf(L->a[h] * q35_softplus(s->alpha[h] + L->dt_bias[h]));
    float *S = state + (uint64_t)h * dk * dv;
    for (uint64_t i = 0; i < (uint64_t)dk * dv; i++) S[i] *= decay;
    for (uint32_t j = 0; j < dv; j++) s->delta[j] = 0.0f;
    for (uint32_t r = 0; r < dk; r++)
      for (uint32_t j = 0; j < dv; j++) s->delta[j] += S[(uint64_t)r * dv + j] * kk[r];
    for (uint32_t j = 0; j < dv; j++) s->delta[j] = (vh[j] - s->delta[j]) * beta;
    float *out = s->delta_out + (uint64_t)h * dv;
    for (uint32_t j = 0; j < dv; j++) out[j] = 0.0f;
    for (uint32_t r = 0; r < dk; r++)
      for (uint32_t j = 0; j < dv; j++) {
        S[(uint64_t)r * dv + j] += kk[r] * s->delta[j];
        out[j] += S[(uint64_t)r * dv + j] * qh[r];
      }
    rms_norm_in_place(out, L->ssm_norm, dv, m->norm_eps);
    const float *g = s->z + (uint64_t)h * dv;
    for (uint32_t j = 0; j < dv; j++) out[j] *= orc_silu(g[j]);
  }
  matvec_m(&L->out, s->delta_out, s->mixer_out);
}

/* One Gated DeltaNet layer of a step (Model::delta_net, qwen35.rs:430-516)
 * on the state's current normalised input: the CPU baseline's "GDN layer
 * step".  Returns -1 when layer il is an attention layer. */
EXPORT int orc_qwen35_delta_step(const bch_qwen35_model *m, orc_qwen35_state *s, uint32_t il) {
  if (il >= m->n_layers || m->layers[il].is_attention) return -1;
  uint32_t di = 0;
  for (uint32_t i = 0; i < il; i++) di += !m->layers[i].is_attention;
  q35_delta(m, &m->layers[il], di, s);
  return 0;
}

/* Model::step (qwen35.rs:280-365); traces as orc_lfm2_step. */
EXPORT int orc_qwen35_step(const bch_qwen35_model *m, orc_qwen35_state *s, uint32_t token, float *logits,
                           float *trace_embedding, float *trace_layers, float *trace_final) {
  uint32_t n = m->n_embd, pos = s->n_past;
  if (pos >= s->n_ctx) return -1;
  if (token >= m->n_vocab) return -2;
  uint64_t rb = orc_row_bytes(m->token_embd.format, n);
  orc_dequantize(m->token_embd.format, (const uint8_t *)m->token_embd.data + (uint64_t)token * rb, n, s->h);
  if (trace_embedding) memcpy(trace_embedding, s->h, 4ull * n);
  uint32_t ai = 0, di = 0;
  for (uint32_t il = 0; il < m->n_layers; il++) {
    const bch_qwen35_layer *L = &m->layers[il];
    orc_rms_norm(s->h, L->attn_norm, n, m->norm_eps, s->x);
    if (L->is_attention)
      q35_attention(m, L, ai++, pos, s);
    else
      q35_delta(m, L, di++, s);
    for (uint32_t i = 0; i < n; i++) s->h[i] += s->mixer_out[i];
    orc_rms_norm(s->h, L->ffn_norm, n, m->norm_eps, s->x);
    matvec_m(&L->gate, s->x, s->ffn_gate);
    matvec_m(&L->up, s->x, s->ffn_up);
    for (uint32_t i = 0; i < m->n_ff; i++) s->ffn_gate[i] = orc_silu(s->ffn_gate[i]) * s->ffn_up[i];
    matvec_m(&L->down, s->ffn_gate, s->mixer_out);
    for (uint32_t i = 0; i < n; i++) s->h[i] += s->mixer_out[i];
    if (trace_layers) memcpy(trace_layers + (uint64_t)il * n, s->h, 4ull * n);
  }
  orc_rms_norm(s->h, m->output_norm, n, m->norm_eps, s->x);
  if (trace_final) memcpy(trace_final, s->x, 4ull * n);
  if (logits) matvec_m(&m->output, s->x, logits);
  s->n_past++;
  return 0;
}
