/*
 * ORACLE — test infrastructure, not part of the product. See oracle.h.
 *
 * CPU restatement of the StrasGPT reference forward pass
 * (source/transformer.c), threaded with OpenMP. Compiled without
 * -ffast-math and with -ffp-contract=off, so the arithmetic is exactly what
 * is written here: fmaf() where the reference's AVX2 dot product issues
 * FMAs, plain sequential fp32 sums elsewhere.
 */
#include "oracle.h"

#include <math.h>
#include <omp.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

struct oracle_model {
  oracle_config_t c;
  size_t per_layer[ORACLE_CLASS_COUNT]; /* elements (bf16) or bytes (u8) */
  void* w[ORACLE_CLASS_COUNT];
  unsigned char* loaded[ORACLE_CLASS_COUNT];
  /* chunk activations */
  float *x, *xn, *q, *att, *g, *u, *tmp;
  /* KV cache [L][kvh][ctx][hd] and RoPE table [ctx][hd] */
  float *kc, *vc, *rope;
  size_t cached;
  int kv_format; /* ORACLE_KV_*: rounding of the values written to kc, vc */
  float *cap, *cap_final;
  /* router tie margins [L][cap_rows] of the capture call (MoE), or NULL */
  float* cap_margin;
  size_t cap_row, cap_rows;
};

/* ------------------------------------------------------------------------ */
/* Primitives                                                                */

/* Reference include/util.h:33-39: the bf16 bits are the top half of the
 * fp32 bits. */
static inline float bf16f(uint16_t w) {
  uint32_t u = (uint32_t)w << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

float oracle_bf16_to_f32(uint16_t w) { return bf16f(w); }

/* Round to the nearest bf16 value, ties to even (the top 16 bits of the
 * fp32 pattern after adding half an ulp of the kept part, plus one when the
 * kept part is odd); infinities stay, NaNs stay NaN. No reference
 * counterpart: the reference cache is fp32. */
float oracle_round_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) {
    u |= 0x00400000u; /* quiet NaN */
  } else {
    u += 0x7fffu + ((u >> 16) & 1u);
  }
  u &= 0xffff0000u;
  memcpy(&x, &u, 4);
  return x;
}

/* Round to the nearest OCP FP8 E4M3 value (bias 7, largest 448, subnormal
 * spacing 2^-9), ties to even, magnitudes past 448 saturating to 448; NaN
 * stays NaN. The spacing of the binade of |x| is a power of two, so the
 * quotient below is exact and rintf (round to nearest even, the default
 * mode) does the rounding. No reference counterpart. */
float oracle_round_fp8_e4m3(float x) {
  if (isnan(x)) return x;
  float a = fabsf(x);
  if (a >= 448.0f) return copysignf(448.0f, x);
  int e;
  frexpf(a, &e);                       /* a = f 2^e, f in [0.5, 1) */
  int q = (a < 0.015625f ? -6 : e - 1) - 3;  /* log2 of the spacing */
  float r = ldexpf(rintf(ldexpf(a, -q)), q);
  if (r > 448.0f) r = 448.0f;
  return copysignf(r, x);
}

void oracle_set_kv_format(oracle_model_t* m, int fmt) { m->kv_format = fmt; }

static float round_kv(int fmt, float v) {
  return fmt == ORACLE_KV_BF16 ? oracle_round_bf16(v) : fmt == ORACLE_KV_FP8_E4M3 ? oracle_round_fp8_e4m3(v) : v;
}
void oracle_bf16_to_f32_array(const uint16_t* w, size_t n, float* out) {
  for (size_t i = 0; i < n; i++) out[i] = bf16f(w[i]);
}

/* OCP Microscaling v1.0: E2M1 element (sign, 2-bit exponent, 1-bit
 * mantissa) times an E8M0 scale 2^(s-127); s = 255 encodes NaN. No
 * reference counterpart. */
float oracle_mxfp4_value(uint8_t code, uint8_t scale) {
  static const float mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  if (scale == 255) return NAN;
  float v = ldexpf(mag[code & 7], (int)scale - 127);
  return (code & 8) ? -v : v;
}

/* The same values as oracle_mxfp4_value element by element: per 32-value
 * block, the 16 codes times the block's power of two (2^(scale - 127),
 * subnormal for scale 0), each product exact. */
void oracle_mxfp4_dequant(const uint8_t* blocks, const uint8_t* scales,
                          size_t value_count, float* out) {
  static const float val[16] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
                                -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};
  for (size_t b = 0; b < value_count / 32; b++) {
    const uint8_t sc = scales[b];
    if (sc == 255) {
      for (int i = 0; i < 32; i++) out[b * 32 + i] = NAN;
      continue;
    }
    const float p2 = ldexpf(1.0f, (int)sc - 127);
    for (int i = 0; i < 16; i++) {
      const uint8_t byte = blocks[b * 16 + i];
      out[b * 32 + 2 * i] = val[byte & 15] * p2;
      out[b * 32 + 2 * i + 1] = val[byte >> 4] * p2;
    }
  }
  for (size_t i = value_count / 32 * 32; i < value_count; i++) {
    uint8_t byte = blocks[i / 2];
    uint8_t code = (i & 1) ? (byte >> 4) : (byte & 15);
    out[i] = oracle_mxfp4_value(code, scales[i / 32]);
  }
}

/* Reference dot() AVX2 variant (source/transformer.c:1095-1167): element i
 * feeds accumulator lane i%8 of accumulator (i/8)%4 with an FMA; the four
 * 8-lane accumulators are summed as (a0+a1)+(a2+a3), then lanes l and l+4,
 * then ((s0+s1)+(s2+s3)). len is a multiple of 32. */
static inline float reduce_4x8(float acc[4][8]) {
  float v[8];
  for (int l = 0; l < 8; l++) v[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
  float s0 = v[0] + v[4], s1 = v[1] + v[5], s2 = v[2] + v[6], s3 = v[3] + v[7];
  return (s0 + s1) + (s2 + s3);
}

float oracle_dot_bf16(size_t len, const float* a, const uint16_t* w) {
  float acc[4][8] = {{0}};
  for (size_t i = 0; i < len; i += 32) {
    for (int j = 0; j < 4; j++) {
      for (int l = 0; l < 8; l++) {
        size_t k = i + 8 * (size_t)j + (size_t)l;
        acc[j][l] = fmaf(a[k], bf16f(w[k]), acc[j][l]);
      }
    }
  }
  return reduce_4x8(acc);
}

/* oracle_dot_bf16 of one weight row with two activation rows at once
 * (independent accumulators, the same roundings as two separate calls). */
static void dot2_bf16(size_t len, const float* a0, const float* a1, const uint16_t* w,
                      float* r0, float* r1) {
  float acc0[4][8] = {{0}}, acc1[4][8] = {{0}};
  for (size_t i = 0; i < len; i += 32) {
    for (int j = 0; j < 4; j++) {
      for (int l = 0; l < 8; l++) {
        size_t k = i + 8 * (size_t)j + (size_t)l;
        float wk = bf16f(w[k]);
        acc0[j][l] = fmaf(a0[k], wk, acc0[j][l]);
        acc1[j][l] = fmaf(a1[k], wk, acc1[j][l]);
      }
    }
  }
  *r0 = reduce_4x8(acc0);
  *r1 = reduce_4x8(acc1);
}

/* Same accumulation order with fp32 weights (dequantised MXFP4 rows). */
static float dot_f32(size_t len, const float* a, const float* w) {
  float acc[4][8] = {{0}};
  for (size_t i = 0; i < len; i += 32) {
    for (int j = 0; j < 4; j++) {
      for (int l = 0; l < 8; l++) {
        size_t k = i + 8 * (size_t)j + (size_t)l;
        acc[j][l] = fmaf(a[k], w[k], acc[j][l]);
      }
    }
  }
  return reduce_4x8(acc);
}

/* Reference rmsnorm (source/transformer.c:978-999): ss = sum x^2 (fp32,
 * in index order), ss /= n, s = (float)(1.0 / sqrtf(ss + eps)),
 * y = (x * s) * w. y may alias x. */
void oracle_rmsnorm(size_t n, float* y, const float* x, const uint16_t* w, float eps) {
  float ss = 0.0f;
  for (size_t j = 0; j < n; j++) ss = fmaf(x[j], x[j], ss);
  ss /= (float)n;
  ss = (float)(1.0 / (double)sqrtf(ss + eps));
  for (size_t j = 0; j < n; j++) y[j] = (x[j] * ss) * bf16f(w[j]);
}

/* Reference state_from_safetensors RoPE table (source/transformer.c:126-146):
 * freq = 1 / theta^((coef*j)/hd), angle = pos * freq, cos at j, sin at
 * j + offset. Half-split: j < hd/2 step 1, offset hd/2, coef 2.
 * Interleaved: j < hd step 2, offset 1, coef 1. */
void oracle_rope_table(size_t ctx, size_t hd, float theta, int interleaved, float* out) {
  size_t bound = interleaved ? hd : hd / 2;
  size_t offset = interleaved ? 1 : hd / 2;
  size_t stride = interleaved ? 2 : 1;
  float coef = interleaved ? 1.0f : 2.0f;
  for (size_t i = 0; i < ctx; i++) {
    for (size_t j = 0; j < bound; j += stride) {
      float freq = 1.0f / powf(theta, (coef * (float)j) / (float)hd);
      float val = (float)i * freq;
      out[i * hd + j] = cosf(val);
      out[i * hd + j + offset] = sinf(val);
    }
  }
}

static void rope_apply(size_t hd, int interleaved, float* v, const float* cs) {
  size_t bound = interleaved ? hd : hd / 2;
  size_t offset = interleaved ? 1 : hd / 2;
  size_t stride = interleaved ? 2 : 1;
  for (size_t h = 0; h < bound; h += stride) {
    float fr = cs[h], fi = cs[h + offset];
    float v0 = v[h], v1 = v[h + offset];
    v[h] = v0 * fr - v1 * fi;
    v[h + offset] = v0 * fi + v1 * fr;
  }
}

/* Reference attention for one (head, token) (source/transformer.c:1383-1419):
 * scores q.k / sqrtf(hd) with the dot summed over h in order, softmax with
 * max subtraction, expf, sequential sum and division, then
 * out[h] = sum over s (in order) of p[s] * v[s][h]. */
void oracle_attention_row(size_t hd, size_t count, const float* q, const float* k,
                          const float* v, float* out) {
  float* p = malloc(count * sizeof(float));
  float scale = sqrtf((float)hd);
  /* 8 keys at a time: independent chains, each still summed over h in
   * order (the same roundings as one key at a time) */
  size_t s = 0;
  for (; s + 8 <= count; s += 8) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (size_t h = 0; h < hd; h++)
      for (int j = 0; j < 8; j++) acc[j] = fmaf(q[h], k[(s + j) * hd + h], acc[j]);
    for (int j = 0; j < 8; j++) p[s + j] = acc[j] / scale;
  }
  for (; s < count; s++) {
    float acc = 0.0f;
    for (size_t h = 0; h < hd; h++) acc = fmaf(q[h], k[s * hd + h], acc);
    p[s] = acc / scale;
  }
  float mx = p[0];
  for (s = 1; s < count; s++) mx = p[s] > mx ? p[s] : mx;
  float sum = 0.0f;
  for (s = 0; s < count; s++) {
    p[s] = expf(p[s] - mx);
    sum += p[s];
  }
  for (s = 0; s < count; s++) p[s] /= sum;
  for (size_t h = 0; h < hd; h++) out[h] = 0.0f;
  for (s = 0; s < count; s++) {
    for (size_t h = 0; h < hd; h++) out[h] = fmaf(p[s], v[s * hd + h], out[h]);
  }
  free(p);
}

/* Reference sample_argmax (source/sampler.c:92-102): first index holding
 * the strict maximum. */
size_t oracle_argmax(const float* x, size_t n) {
  size_t best = 0;
  float bv = x[0];
  for (size_t i = 1; i < n; i++) {
    if (x[i] > bv) {
      best = i;
      bv = x[i];
    }
  }
  return best;
}

/* MoE router (no reference counterpart): the k largest logits in
 * descending order, ties to the lowest index, then softmax over those k
 * with max subtraction, expf and a sequential sum. */
/* ---- Stochastic sampler: reference source/sampler.c:79-337 ---- */

/* Xorshift64* (source/sampler.c:79-85): the state update and the 32-bit
 * output of the published generator. */
static unsigned int sampler_u32(unsigned long long* s) {
  *s ^= *s >> 12;
  *s ^= *s << 25;
  *s ^= *s >> 27;
  return (unsigned int)((*s * 0x2545F4914F6CDD1Dull) >> 32);
}
/* source/sampler.c:87-90: 24 random bits scaled to [0, 1). */
static float sampler_f32(unsigned long long* s) { return (sampler_u32(s) >> 8) / 16777216.0f; }

typedef struct {
  float p;
  size_t i;
} prob_index_t;
/* Descending probability; equal probabilities keep index order (the order
 * a stable sort of the index-ordered array gives, as glibc's merge-sort
 * qsort does for source/sampler.c:159-167). */
static int prob_desc(const void* a_, const void* b_) {
  const prob_index_t *a = a_, *b = b_;
  if (a->p > b->p) return -1;
  if (a->p < b->p) return 1;
  return a->i < b->i ? -1 : a->i > b->i;
}

/* One sampler_sample call (source/sampler.c:234-337) on logits[n] (modified
 * in place like the reference). presence[n] marks tokens seen, prev is the
 * previous token. Reports the coin and the distance from the coin to the
 * nearest boundary of the sampled token's cdf interval (margin), which
 * tells whether a different summation order could pick another token. */
size_t oracle_sample(oracle_sampler_t* s, float* x, size_t n, unsigned char* presence, int prev,
                     float* coin_out, double* margin_out) {
  if (prev >= 0 && (size_t)prev < n) presence[prev] = 1;
  if (s->presence_penalty != 0.0f)
    for (size_t i = 0; i < n; i++)
      if (presence[i]) x[i] -= s->presence_penalty;
  if (coin_out) *coin_out = -1.0f;
  if (margin_out) *margin_out = INFINITY;
  if (s->temperature == 0.0f) return oracle_argmax(x, n);
  for (size_t i = 0; i < n; i++) x[i] /= s->temperature;
  /* softmax (source/sampler.c:104-123) */
  float mx = x[0];
  for (size_t i = 1; i < n; i++)
    if (x[i] > mx) mx = x[i];
  float sum = 0.0f;
  for (size_t i = 0; i < n; i++) {
    x[i] = expf(x[i] - mx);
    sum += x[i];
  }
  for (size_t i = 0; i < n; i++) x[i] /= sum;
  const float coin = sampler_f32(&s->rng_state);
  if (coin_out) *coin_out = coin;
  prob_index_t* pi = malloc(n * sizeof(*pi));
  double cut_margin = INFINITY;
  if (s->top_k > 0) { /* source/sampler.c:170-193 */
    for (size_t i = 0; i < n; i++) pi[i] = (prob_index_t){x[i], i};
    qsort(pi, n, sizeof(*pi), prob_desc);
    for (size_t r = s->top_k < n ? s->top_k : n; r < n; r++) x[pi[r].i] = 0.0f;
  }
  if (s->top_p > 0 && s->top_p <= 1) { /* source/sampler.c:195-229 */
    for (size_t i = 0; i < n; i++) pi[i] = (prob_index_t){x[i], i};
    qsort(pi, n, sizeof(*pi), prob_desc);
    float cum = 0.0f;
    size_t last = n - 1;
    for (size_t r = 0; r < n; r++) {
      const float before = cum;
      cum += pi[r].p;
      if (cum >= s->top_p) {
        last = r;
        cut_margin = fmin((double)cum - s->top_p, (double)s->top_p - before);
        break;
      }
    }
    for (size_t r = last + 1; r < n; r++) x[pi[r].i] = 0.0f;
  }
  free(pi);
  /* renormalize (source/sampler.c:139-157) */
  double dsum = 0.0;
  for (size_t i = 0; i < n; i++) dsum += (double)x[i];
  if (dsum <= 0.0) {
    const float u = 1.0f / (float)n;
    for (size_t i = 0; i < n; i++) x[i] = u;
  } else {
    const float inv = (float)(1.0 / dsum);
    for (size_t i = 0; i < n; i++) x[i] *= inv;
  }
  /* sample_mult (source/sampler.c:125-137) */
  float cdf = 0.0f;
  size_t pick = n - 1;
  for (size_t i = 0; i < n; i++) {
    const float before = cdf;
    cdf += x[i];
    if (coin < cdf) {
      pick = i;
      if (margin_out) *margin_out = fmin(fmin((double)cdf - coin, (double)coin - before), cut_margin);
      break;
    }
  }
  return pick;
}

void oracle_topk_softmax(size_t n, const float* logits, size_t k, int* index, float* weight) {
  unsigned char taken[1024] = {0};
  for (size_t j = 0; j < k; j++) {
    int best = -1;
    for (size_t e = 0; e < n; e++) {
      if (taken[e]) continue;
      if (best < 0 || logits[e] > logits[best]) best = (int)e;
    }
    taken[best] = 1;
    index[j] = best;
  }
  float mx = logits[index[0]], sum = 0.0f;
  for (size_t j = 0; j < k; j++) {
    weight[j] = expf(logits[index[j]] - mx);
    sum += weight[j];
  }
  for (size_t j = 0; j < k; j++) weight[j] /= sum;
}

static inline float silu_mul(float g, float u) {
  /* Reference source/transformer.c:1477-1486. */
  g *= 1.0f / (1.0f + expf(-g));
  return g * u;
}

/* ------------------------------------------------------------------------ */
/* Model                                                                     */

static int is_u8(int cls) {
  return cls >= ORACLE_GATE_BLOCKS && cls <= ORACLE_DOWN_SCALES;
}

oracle_model_t* oracle_create(const oracle_config_t* cfg) {
  oracle_model_t* m = calloc(1, sizeof(*m));
  m->c = *cfg;
  const oracle_config_t* c = &m->c;
  size_t d = c->embedding_dim, hd = c->head_dim, H = c->hidden_dim, E = c->expert_count;
  size_t* p = m->per_layer;
  p[ORACLE_EMBEDDING] = c->vocabulary_len * d;
  p[ORACLE_MHA_NORM] = d;
  p[ORACLE_Q] = c->q_head_count * hd * d;
  p[ORACLE_Q_NORM] = c->qk_norm ? hd : 0;
  p[ORACLE_K] = c->kv_head_count * hd * d;
  p[ORACLE_K_NORM] = c->qk_norm ? hd : 0;
  p[ORACLE_V] = c->kv_head_count * hd * d;
  p[ORACLE_O] = d * c->q_head_count * hd;
  p[ORACLE_FFN_NORM] = d;
  p[ORACLE_GATE] = E ? 0 : H * d;
  p[ORACLE_UP] = E ? 0 : H * d;
  p[ORACLE_DOWN] = E ? 0 : d * H;
  p[ORACLE_OUT_NORM] = d;
  p[ORACLE_OUT] = c->tied ? 0 : c->vocabulary_len * d;
  p[ORACLE_ROUTER] = E * d;
  p[ORACLE_GATE_BLOCKS] = E * H * d / 2;
  p[ORACLE_GATE_SCALES] = E * H * d / 32;
  p[ORACLE_UP_BLOCKS] = E * H * d / 2;
  p[ORACLE_UP_SCALES] = E * H * d / 32;
  p[ORACLE_DOWN_BLOCKS] = E * d * H / 2;
  p[ORACLE_DOWN_SCALES] = E * d * H / 32;
  for (int k = 0; k < ORACLE_CLASS_COUNT; k++) {
    if (!p[k]) continue;
    size_t layers = (k == ORACLE_EMBEDDING || k == ORACLE_OUT_NORM || k == ORACLE_OUT)
                        ? 1 : c->layer_count;
    size_t bytes = p[k] * layers * (is_u8(k) ? 1 : 2);
    m->w[k] = malloc(bytes);
    m->loaded[k] = calloc(layers, 1);
    if (!m->w[k] || !m->loaded[k]) {
      oracle_free(m);
      return NULL;
    }
  }
  size_t T = ORACLE_CHUNK_MAX_LEN, qd = c->q_head_count * hd;
  size_t hid = H > d ? H : d;
  m->x = malloc(T * d * sizeof(float));
  m->xn = malloc(T * d * sizeof(float));
  m->q = malloc(T * qd * sizeof(float));
  m->att = malloc(T * qd * sizeof(float));
  m->g = malloc(T * hid * sizeof(float));
  m->u = malloc(T * hid * sizeof(float));
  m->tmp = malloc(T * d * sizeof(float));
  size_t cache = c->layer_count * c->kv_head_count * c->context_len * hd;
  m->kc = calloc(cache, sizeof(float));
  m->vc = calloc(cache, sizeof(float));
  m->rope = malloc(c->context_len * hd * sizeof(float));
  if (!m->x || !m->xn || !m->q || !m->att || !m->g || !m->u || !m->tmp ||
      !m->kc || !m->vc || !m->rope) {
    oracle_free(m);
    return NULL;
  }
  oracle_rope_table(c->context_len, hd, c->rope_theta, c->rope_interleaved, m->rope);
  return m;
}

int oracle_load_tensor(oracle_model_t* m, int cls, size_t layer, const char* file,
                       size_t offset, size_t size) {
  if (cls < 0 || cls >= ORACLE_CLASS_COUNT || !m->w[cls]) return -1;
  size_t esz = is_u8(cls) ? 1 : 2;
  if (size != m->per_layer[cls] * esz) return -1;
  size_t layers = (cls == ORACLE_EMBEDDING || cls == ORACLE_OUT_NORM || cls == ORACLE_OUT)
                      ? 1 : m->c.layer_count;
  if (layer >= layers) return -1;
  FILE* f = fopen(file, "rb");
  if (!f) return -1;
  int rc = 0;
  if (fseek(f, (long)offset, SEEK_SET) != 0 ||
      fread((char*)m->w[cls] + layer * size, 1, size, f) != size)
    rc = -1;
  fclose(f);
  if (rc == 0) m->loaded[cls][layer] = 1;
  return rc;
}

int oracle_finalize(oracle_model_t* m) {
  int missing = 0;
  for (int k = 0; k < ORACLE_CLASS_COUNT; k++) {
    if (!m->w[k]) continue;
    size_t layers = (k == ORACLE_EMBEDDING || k == ORACLE_OUT_NORM || k == ORACLE_OUT)
                        ? 1 : m->c.layer_count;
    for (size_t l = 0; l < layers; l++) missing += !m->loaded[k][l];
  }
  return missing;
}

void oracle_free(oracle_model_t* m) {
  if (!m) return;
  for (int k = 0; k < ORACLE_CLASS_COUNT; k++) {
    free(m->w[k]);
    free(m->loaded[k]);
  }
  free(m->x); free(m->xn); free(m->q); free(m->att); free(m->g); free(m->u);
  free(m->tmp); free(m->kc); free(m->vc); free(m->rope);
  free(m);
}

void oracle_reset(oracle_model_t* m) { m->cached = 0; }
size_t oracle_cached_count(const oracle_model_t* m) { return m->cached; }
void oracle_set_threads(int n) { if (n > 0) omp_set_num_threads(n); }

void oracle_capture_hidden(oracle_model_t* m, float* out, float* out_final) {
  m->cap = out;
  m->cap_final = out_final;
}

void oracle_capture_router_margin(oracle_model_t* m, float* out) { m->cap_margin = out; }

static const uint16_t* W(const oracle_model_t* m, int cls, size_t layer) {
  return (const uint16_t*)m->w[cls] + layer * m->per_layer[cls];
}

/* Expert FFN of T tokens: per token, the router logits (bf16 dot), top-k
 * with softmax over the selected logits, then the reference SwiGLU FFN
 * (source/transformer.c:1461-1504) with MXFP4 weights per selected expert,
 * accumulated as out = fmaf(weight_j, expert_j(x), out) in top-k order from
 * 0. Work is grouped by expert so that each weight row is dequantised once
 * per chunk; every dot product and the accumulation order per token are
 * those of the per-token formulation. */
static void moe_chunk(const oracle_model_t* m, size_t l, size_t T, const float* xn, float* out) {
  const oracle_config_t* c = &m->c;
  size_t d = c->embedding_dim, H = c->hidden_dim, E = c->expert_count, K = c->expert_used_count;
  int* sel = malloc(T * K * sizeof(int));
  float* wsel = malloc(T * K * sizeof(float));
  float* act = malloc(T * K * H * sizeof(float));
  float* dn = malloc(T * K * d * sizeof(float));
  size_t* pairs = malloc(T * K * sizeof(size_t));
  #pragma omp parallel for schedule(static)
  for (size_t t = 0; t < T; t++) {
    float logits[1024];
    for (size_t e = 0; e < E; e++)
      logits[e] = oracle_dot_bf16(d, xn + t * d, W(m, ORACLE_ROUTER, l) + e * d);
    oracle_topk_softmax(E, logits, K, sel + t * K, wsel + t * K);
    if (m->cap_margin) {
      /* k-th largest logit minus the largest one left out: how far the
       * selected set is from changing */
      float kth = logits[sel[t * K + K - 1]], out_best = -INFINITY;
      for (size_t e = 0; e < E; e++) {
        int chosen = 0;
        for (size_t j = 0; j < K; j++) chosen |= sel[t * K + j] == (int)e;
        if (!chosen && logits[e] > out_best) out_best = logits[e];
      }
      m->cap_margin[l * m->cap_rows + m->cap_row + t] = kth - out_best;
    }
  }
  const uint8_t* gb = (const uint8_t*)m->w[ORACLE_GATE_BLOCKS] + l * m->per_layer[ORACLE_GATE_BLOCKS];
  const uint8_t* gs = (const uint8_t*)m->w[ORACLE_GATE_SCALES] + l * m->per_layer[ORACLE_GATE_SCALES];
  const uint8_t* ub = (const uint8_t*)m->w[ORACLE_UP_BLOCKS] + l * m->per_layer[ORACLE_UP_BLOCKS];
  const uint8_t* us = (const uint8_t*)m->w[ORACLE_UP_SCALES] + l * m->per_layer[ORACLE_UP_SCALES];
  const uint8_t* db = (const uint8_t*)m->w[ORACLE_DOWN_BLOCKS] + l * m->per_layer[ORACLE_DOWN_BLOCKS];
  const uint8_t* ds = (const uint8_t*)m->w[ORACLE_DOWN_SCALES] + l * m->per_layer[ORACLE_DOWN_SCALES];
  for (size_t e = 0; e < E; e++) {
    size_t np = 0;  /* (token, slot) pairs routed to expert e */
    for (size_t p = 0; p < T * K; p++)
      if ((size_t)sel[p] == e) pairs[np++] = p;
    if (!np) continue;
    #pragma omp parallel
    {
      float* rg = malloc(d * sizeof(float));
      float* ru = malloc(d * sizeof(float));
      #pragma omp for schedule(static)
      for (size_t h = 0; h < H; h++) {
        size_t r = e * H + h;
        oracle_mxfp4_dequant(gb + r * d / 2, gs + r * d / 32, d, rg);
        oracle_mxfp4_dequant(ub + r * d / 2, us + r * d / 32, d, ru);
        for (size_t i = 0; i < np; i++) {
          const float* x = xn + (pairs[i] / K) * d;
          act[pairs[i] * H + h] = silu_mul(dot_f32(d, x, rg), dot_f32(d, x, ru));
        }
      }
      free(rg);
      free(ru);
    }
    #pragma omp parallel
    {
      float* rd = malloc(H * sizeof(float));
      #pragma omp for schedule(static)
      for (size_t o = 0; o < d; o++) {
        size_t r = e * d + o;
        oracle_mxfp4_dequant(db + r * H / 2, ds + r * H / 32, H, rd);
        for (size_t i = 0; i < np; i++) dn[pairs[i] * d + o] = dot_f32(H, act + pairs[i] * H, rd);
      }
      free(rd);
    }
  }
  #pragma omp parallel for schedule(static)
  for (size_t t = 0; t < T; t++) {
    for (size_t o = 0; o < d; o++) {
      float acc = 0.0f;
      for (size_t j = 0; j < K; j++) acc = fmaf(wsel[t * K + j], dn[(t * K + j) * d + o], acc);
      out[t * d + o] = acc;
    }
  }
  free(sel);
  free(wsel);
  free(act);
  free(dn);
  free(pairs);
}

/* out(r, t) = dot(K, x[t], w[r]) for r < R, t < T, in blocks of 16 rows x
 * 32 tokens so that both stay in the core's caches (the reference loops
 * over rows then tokens; each dot product is the same either way). */
typedef void (*store_fn)(void* ctx, size_t r, size_t t, float v);
static void project(size_t R, size_t T, size_t K, const uint16_t* w, const float* x, size_t ldx,
                    store_fn st, void* ctx) {
  const size_t RB = 16, TB = 32;
  const size_t nrb = (R + RB - 1) / RB, ntb = (T + TB - 1) / TB;
  #pragma omp parallel for collapse(2) schedule(static)
  for (size_t rb = 0; rb < nrb; rb++) {
    for (size_t tb = 0; tb < ntb; tb++) {
      const size_t r1 = rb * RB + RB < R ? rb * RB + RB : R;
      const size_t t1 = tb * TB + TB < T ? tb * TB + TB : T;
      for (size_t r = rb * RB; r < r1; r++) {
        size_t t = tb * TB;
        for (; t + 2 <= t1; t += 2) {
          float v0, v1;
          dot2_bf16(K, x + t * ldx, x + (t + 1) * ldx, w + r * K, &v0, &v1);
          st(ctx, r, t, v0);
          st(ctx, r, t + 1, v1);
        }
        if (t < t1) st(ctx, r, t, oracle_dot_bf16(K, x + t * ldx, w + r * K));
      }
    }
  }
}

typedef struct {
  float* base;
  size_t ctx, hd, P, ld;
} store_ctx_t;
/* cache row P + t of head r / hd: base[(head ctx + P + t) hd + r % hd] */
static void store_cache(void* c_, size_t r, size_t t, float v) {
  store_ctx_t* c = c_;
  c->base[((r / c->hd) * c->ctx + c->P + t) * c->hd + r % c->hd] = v;
}
/* row-major [t][ld] */
static void store_rows(void* c_, size_t r, size_t t, float v) {
  store_ctx_t* c = c_;
  c->base[t * c->ld + r] = v;
}

/* Reference transformer_predict_chunk (source/transformer.c:1186-1602). */
static void predict_chunk(oracle_model_t* m, size_t T, const int* tok, size_t lc, float* logits,
                          size_t cap_row, size_t cap_rows) {
  m->cap_row = cap_row;
  m->cap_rows = cap_rows;
  const oracle_config_t* c = &m->c;
  size_t d = c->embedding_dim, hd = c->head_dim, H = c->hidden_dim, L = c->layer_count;
  size_t qh = c->q_head_count, kvh = c->kv_head_count, G = qh / kvh, ctx = c->context_len;
  size_t qd = qh * hd, P = m->cached, V = c->vocabulary_len;
  float eps = c->epsilon;
  float *x = m->x, *xn = m->xn, *q = m->q, *att = m->att, *g = m->g, *u = m->u, *tmp = m->tmp;

  for (size_t t = 0; t < T; t++)
    for (size_t e = 0; e < d; e++)
      x[t * d + e] = bf16f(W(m, ORACLE_EMBEDDING, 0)[(size_t)tok[t] * d + e]);

  for (size_t l = 0; l < L; l++) {
    float* kc = m->kc + l * kvh * ctx * hd;
    float* vc = m->vc + l * kvh * ctx * hd;
    #pragma omp parallel for schedule(static)
    for (size_t t = 0; t < T; t++) oracle_rmsnorm(d, xn + t * d, x + t * d, W(m, ORACLE_MHA_NORM, l), eps);

    /* K and V projections into the cache (source/transformer.c:1271-1291) */
    {
      store_ctx_t sk = {kc, ctx, hd, P, 0}, sv = {vc, ctx, hd, P, 0};
      project(kvh * hd, T, d, W(m, ORACLE_K, l), xn, d, store_cache, &sk);
      project(kvh * hd, T, d, W(m, ORACLE_V, l), xn, d, store_cache, &sv);
    }
    /* K-norm and RoPE on the new keys (source/transformer.c:1293-1323) */
    #pragma omp parallel for collapse(2) schedule(static)
    for (size_t head = 0; head < kvh; head++) {
      for (size_t t = 0; t < T; t++) {
        float* kr = kc + (head * ctx + P + t) * hd;
        if (c->qk_norm) oracle_rmsnorm(hd, kr, kr, W(m, ORACLE_K_NORM, l), eps);
        rope_apply(hd, c->rope_interleaved, kr, m->rope + (P + t) * hd);
      }
    }
    /* cache storage format: the new rows as the cache holds them */
    if (m->kv_format != ORACLE_KV_F32) {
      for (size_t head = 0; head < kvh; head++)
        for (size_t i = (head * ctx + P) * hd; i < (head * ctx + P + T) * hd; i++) {
          kc[i] = round_kv(m->kv_format, kc[i]);
          vc[i] = round_kv(m->kv_format, vc[i]);
        }
    }
    /* Q projection, Q-norm, RoPE (source/transformer.c:1327-1373) */
    {
      store_ctx_t sq = {q, 0, 0, 0, qd};
      project(qd, T, d, W(m, ORACLE_Q, l), xn, d, store_rows, &sq);
    }
    #pragma omp parallel for collapse(2) schedule(static)
    for (size_t head = 0; head < qh; head++) {
      for (size_t t = 0; t < T; t++) {
        float* qr = q + t * qd + head * hd;
        if (c->qk_norm) oracle_rmsnorm(hd, qr, qr, W(m, ORACLE_Q_NORM, l), eps);
        rope_apply(hd, c->rope_interleaved, qr, m->rope + (P + t) * hd);
      }
    }
    /* Causal GQA attention (source/transformer.c:1375-1422) */
    #pragma omp parallel for collapse(2) schedule(dynamic, 4)
    for (size_t head = 0; head < qh; head++) {
      for (size_t t = 0; t < T; t++) {
        size_t kvhead = head / G;
        oracle_attention_row(hd, P + t + 1, q + t * qd + head * hd, kc + kvhead * ctx * hd,
                             vc + kvhead * ctx * hd, att + t * qd + head * hd);
      }
    }
    /* Output projection + residual (source/transformer.c:1426-1445) */
    {
      store_ctx_t so = {tmp, 0, 0, 0, d};
      project(d, T, qd, W(m, ORACLE_O, l), att, qd, store_rows, &so);
    }
    for (size_t i = 0; i < T * d; i++) x[i] += tmp[i];

    #pragma omp parallel for schedule(static)
    for (size_t t = 0; t < T; t++) oracle_rmsnorm(d, xn + t * d, x + t * d, W(m, ORACLE_FFN_NORM, l), eps);

    if (c->expert_count == 0) {
      /* Gate, up, SwiGLU, down + residual (source/transformer.c:1461-1504) */
      store_ctx_t sg_ = {g, 0, 0, 0, H}, su = {u, 0, 0, 0, H}, sd = {tmp, 0, 0, 0, d};
      project(H, T, d, W(m, ORACLE_GATE, l), xn, d, store_rows, &sg_);
      project(H, T, d, W(m, ORACLE_UP, l), xn, d, store_rows, &su);
      #pragma omp parallel for schedule(static)
      for (size_t i = 0; i < T * H; i++) g[i] = silu_mul(g[i], u[i]);
      project(d, T, H, W(m, ORACLE_DOWN, l), g, H, store_rows, &sd);
    } else {
      moe_chunk(m, l, T, xn, tmp);
    }
    for (size_t i = 0; i < T * d; i++) x[i] += tmp[i];
    if (m->cap) memcpy(m->cap + (l * cap_rows + cap_row) * d, x, T * d * sizeof(float));
  }

  /* Final RMSNorm in place, classifier for the last lc rows
   * (source/transformer.c:1580-1601) */
  for (size_t t = 0; t < T; t++) oracle_rmsnorm(d, x + t * d, x + t * d, W(m, ORACLE_OUT_NORM, 0), eps);
  if (m->cap_final) memcpy(m->cap_final + cap_row * d, x, T * d * sizeof(float));
  const uint16_t* wout = c->tied ? W(m, ORACLE_EMBEDDING, 0) : W(m, ORACLE_OUT, 0);
  #pragma omp parallel for schedule(static)
  for (size_t v = 0; v < V; v++) {
    for (size_t r = 0; r < lc; r++) {
      logits[r * V + v] = oracle_dot_bf16(d, x + (T - lc + r) * d, wout + v * d);
    }
  }
}

/* Reference transformer_predict (source/transformer.c:1607-1727): chunks
 * of at most 512 tokens, logits for the last min(lc, T) positions. */
int oracle_predict(oracle_model_t* m, size_t T, const int* tok, size_t lc, float* logits) {
  if (!m || !logits || T == 0 || lc == 0) return 0;
  if (T + m->cached > m->c.context_len) return -1;
  if (lc > T) lc = T;
  size_t V = m->c.vocabulary_len, start = T - lc;
  for (size_t t = 0; t < T; t += ORACLE_CHUNK_MAX_LEN) {
    size_t n = T - t < ORACLE_CHUNK_MAX_LEN ? T - t : ORACLE_CHUNK_MAX_LEN;
    size_t lo = t > start ? t : start, hi = t + n;
    size_t clc = lo < hi ? hi - lo : 0;
    float* out = logits + (lo - start) * V;
    if (clc == 0) {
      /* The chunk still runs its classifier loop over zero rows. */
      out = logits;
    }
    predict_chunk(m, n, tok + t, clc, out, t, T);
    m->cached += n;
  }
  m->cap = NULL;
  m->cap_final = NULL;
  m->cap_margin = NULL;
  return 0;
}
