/*
 * oracle.c - TEST INFRASTRUCTURE ONLY. A plain C restatement of tabicl-anywhere's CPU path, written from the
 * reference's Rust source read as text (the reference cannot be built here: it is Rust and there is no Rust
 * toolchain). Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may load it, and only as the
 * checker or the timed CPU baseline; the product (libtah_hip.so) never calls it.
 *
 * Every function follows the reference lines it cites: same loop structure, same online softmax, same
 * quantiser, same elementary functions (the reference's own exp/erf/tanh polynomials). Sums run in plain
 * sequential order where the reference uses SIMD lanes, so results agree to rounding, not bit for bit, except
 * orc_pack, whose integer codes are bit-exact for identical float input.
 *
 * Pinning (what checks each part; see tests/test_oracle.py):
 *   - orc_exp1/erf1/tanh1/gelu: the reference's known answers (src/kern.rs:353-373, 492-499) and libm;
 *   - orc_layer_norm/linear/query/feed_forward/Soft: closed forms in float64 and the committed golden vectors;
 *   - orc_attend_records: float64 plain softmax attention, any chunking, split/merge, integer formats;
 *   - orc_pack: closed form of the quantiser in numpy (round half away from zero, saturating casts);
 *   - orc_fit_columns/rows/icl, orc_embed/represent/in_context: tests/golden/tiny-raw.tirs (numbers dumped from
 *     upstream PyTorch TabICL by the reference's tools/dump_raw.py) at the reference's own tolerance 5e-5.
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;

void orc_set_threads(int n) {
    g_threads = n < 1 ? 1 : n;
#ifdef _OPENMP
    omp_set_num_threads(g_threads);
#endif
}

int orc_threads(void) { return g_threads; }

static void *xcalloc(size_t n, size_t sz) {
    void *p = calloc(n ? n : 1, sz);
    if (!p) abort();
    return p;
}

/* ---------------------------------------------------------------- kern.rs ---------------------------------- */

static float clampf(float x, float lo, float hi) { return x < lo ? lo : (x > hi ? hi : x); }

/* src/kern.rs:185-206: e^x by a degree-7 polynomial after range reduction, clamped to [-87, 88]. */
float orc_exp1(float x) {
    const float LOG2E = 1.44269504088896340736f;
    const float LN2_HI = 0.6933594f;
    const float LN2_LO = -2.1219444e-4f;
    x = clampf(x, -87.0f, 88.0f);
    float n = floorf(x * LOG2E + 0.5f);
    float r = (x - n * LN2_HI) - n * LN2_LO;
    float p = 1.0f / 5040.0f;
    p = p * r + 1.0f / 720.0f;
    p = p * r + 1.0f / 120.0f;
    p = p * r + 1.0f / 24.0f;
    p = p * r + 1.0f / 6.0f;
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    union { uint32_t u; float f; } two;
    two.u = ((uint32_t)((int32_t)n + 127)) << 23;
    return p * two.f;
}

/* src/kern.rs:227-253: Abramowitz and Stegun 7.1.26 away from zero, a power series below 0.5. */
float orc_erf1(float x) {
    float a = fabsf(x);
    float t = 1.0f / (1.0f + 0.3275911f * a);
    float p = 1.0614054f;
    p = p * t - 1.4531521f;
    p = p * t + 1.4214138f;
    p = p * t - 0.28449674f;
    p = p * t + 0.2548296f;
    float far = copysignf(1.0f - p * t * orc_exp1(-a * a), x);
    float x2 = x * x;
    float q = -1.0f / 1320.0f;
    q = q * x2 + 1.0f / 216.0f;
    q = q * x2 - 1.0f / 42.0f;
    q = q * x2 + 0.1f;
    q = q * x2 - 1.0f / 3.0f;
    q = q * x2 + 1.0f;
    float near = q * x * 1.12837916709551257390f; /* 2/sqrt(pi) */
    return a < 0.5f ? near : far;
}

/* src/kern.rs:255-261 */
void orc_gelu(float *x, int n) {
    for (int i = 0; i < n; i++) x[i] = 0.5f * x[i] * (1.0f + orc_erf1(x[i] * 0.70710678118654752440f));
}

/* src/kern.rs:263-268 */
float orc_tanh1(float x) {
    float e = orc_exp1(2.0f * clampf(x, -10.0f, 10.0f));
    return (e - 1.0f) / (e + 1.0f);
}

/* src/kern.rs:326-347: two-pass mean and biased variance, eps 1e-5. */
void orc_layer_norm(const float *x, int n, const float *w, const float *b, float *y) {
    float s = 0.0f;
    for (int i = 0; i < n; i++) s += x[i];
    float mean = s / (float)n;
    float q = 0.0f;
    for (int i = 0; i < n; i++) {
        float d = x[i] - mean;
        q += d * d;
    }
    float var = q / (float)n;
    float inv = 1.0f / sqrtf(var + 1e-5f);
    for (int i = 0; i < n; i++) y[i] = (x[i] - mean) * inv * w[i] + b[i];
}

/* src/kern.rs:64-130: y = w x (+ b). */
void orc_linear(const float *w, const float *b, const float *x, int in, int out, float *y) {
    for (int o = 0; o < out; o++) {
        const float *row = w + (size_t)o * in;
        float s = 0.0f;
        for (int i = 0; i < in; i++) s += row[i] * x[i];
        y[o] = b ? s + b[o] : s;
    }
}

/* src/kern.rs:208-225 */
static float exp_shift_sum(float *x, int n, float shift) {
    float t = 0.0f;
    for (int i = 0; i < n; i++) {
        x[i] = orc_exp1(x[i] - shift);
        t += x[i];
    }
    return t;
}

/* ---------------------------------------------------------------- nn.rs ------------------------------------ */

static int hd_of(const tah_block *b) { return b->d / b->heads; }

/* src/nn.rs:97-107: the scalable softmax's length-dependent factor times 1/sqrt(head width). */
void orc_query_scale(const tah_block *b, int n, float *out) {
    float inv = 1.0f / sqrtf((float)hd_of(b));
    if (b->ss_hidden == 0) {
        for (int i = 0; i < b->d; i++) out[i] = inv;
        return;
    }
    float logn = logf((float)(n > 1 ? n : 1));
    float *hid = xcalloc(b->ss_hidden, sizeof(float));
    for (int j = 0; j < b->ss_hidden; j++) hid[j] = b->b0w[j] * logn + b->b0b[j];
    orc_gelu(hid, b->ss_hidden);
    orc_linear(b->b2w, b->b2b, hid, b->ss_hidden, b->d, out);
    for (int i = 0; i < b->d; i++) out[i] *= inv;
    free(hid);
}

/* src/nn.rs:130-152: q = scale * (Wq norm1(x) + bq), with the query MLP's modulation per head. */
void orc_query(const tah_block *b, const float *scale, const float *x, float *q) {
    int d = b->d, hd = hd_of(b);
    float *t = xcalloc(d, sizeof(float));
    orc_layer_norm(x, d, b->n1w, b->n1b, t);
    orc_linear(b->in_w, b->in_b, t, d, d, q);
    if (b->ss_hidden == 0) {
        for (int i = 0; i < d; i++) q[i] *= scale[i];
    } else {
        float *h64 = xcalloc(b->ss_hidden, sizeof(float));
        float *mm = xcalloc(hd, sizeof(float));
        for (int h = 0; h < b->heads; h++) {
            float *qh = q + h * hd;
            const float *sh = scale + h * hd;
            orc_linear(b->q0w, b->q0b, qh, hd, b->ss_hidden, h64);
            orc_gelu(h64, b->ss_hidden);
            orc_linear(b->q2w, b->q2b, h64, b->ss_hidden, hd, mm);
            for (int i = 0; i < hd; i++) qh[i] *= sh[i] * (1.0f + orc_tanh1(mm[i]));
        }
        free(h64);
        free(mm);
    }
    free(t);
}

/* src/nn.rs:156-164: x += l2(gelu(l1(norm2 x))). */
void orc_feed_forward(const tah_block *b, float *x) {
    int d = b->d;
    float *t = xcalloc(d, sizeof(float));
    float *h = xcalloc(b->ff, sizeof(float));
    orc_layer_norm(x, d, b->n2w, b->n2b, t);
    orc_linear(b->l1w, b->l1b, t, d, b->ff, h);
    orc_gelu(h, b->ff);
    orc_linear(b->l2w, b->l2b, h, b->ff, d, t);
    for (int i = 0; i < d; i++) x[i] += t[i];
    free(t);
    free(h);
}

/* src/nn.rs:166-287: the streaming softmax-weighted average. */
typedef struct {
    int heads, d;
    float *m, *s, *acc;
    float *sc, *tmp; /* scratch: max keys per update, one head */
} Soft;

static Soft soft_new(int heads, int d, int max_keys) {
    Soft s;
    s.heads = heads;
    s.d = d;
    s.m = xcalloc(heads, sizeof(float));
    s.s = xcalloc(heads, sizeof(float));
    s.acc = xcalloc(d, sizeof(float));
    s.sc = xcalloc(max_keys, sizeof(float));
    s.tmp = xcalloc(d / heads, sizeof(float));
    for (int h = 0; h < heads; h++) s.m[h] = -INFINITY;
    return s;
}

static void soft_free(Soft *s) {
    free(s->m);
    free(s->s);
    free(s->acc);
    free(s->sc);
    free(s->tmp);
}

static void soft_reset(Soft *s) {
    for (int h = 0; h < s->heads; h++) {
        s->m[h] = -INFINITY;
        s->s[h] = 0.0f;
    }
    memset(s->acc, 0, sizeof(float) * s->d);
}

/* The part of update_scaled / update_int that follows the scores (src/nn.rs:209-226, 241-257): rescale by the new
 * maximum, add the weights, then the weighted values (given by `vrow(i, j)`, coordinate i of key j in this head). */
static void soft_rescale(Soft *s, int h, int r) {
    int hd = s->d / s->heads;
    float top = -INFINITY;
    for (int j = 0; j < r; j++) top = s->sc[j] > top ? s->sc[j] : top;
    float *acc = s->acc + h * hd;
    if (top > s->m[h]) {
        if (s->s[h] > 0.0f) {
            float f = orc_exp1(s->m[h] - top);
            s->s[h] *= f;
            for (int i = 0; i < hd; i++) acc[i] *= f;
        }
        s->m[h] = top;
    }
    s->s[h] += exp_shift_sum(s->sc, r, s->m[h]);
}

/* src/nn.rs:194-228 (vs NULL: update). q [d]; kt, vt [d][r] floats. */
static void soft_update(Soft *s, const float *q, const float *kt, const float *vt, const float *vs, int r) {
    int hd = s->d / s->heads;
    for (int h = 0; h < s->heads; h++) {
        const float *ks = kt + (size_t)h * hd * r, *vv = vt + (size_t)h * hd * r;
        for (int j = 0; j < r; j++) s->sc[j] = 0.0f;
        for (int i = 0; i < hd; i++) {
            float qi = q[h * hd + i];
            const float *row = ks + (size_t)i * r;
            for (int j = 0; j < r; j++) s->sc[j] += qi * row[j];
        }
        soft_rescale(s, h, r);
        float *acc = s->acc + h * hd;
        for (int i = 0; i < hd; i++) {
            const float *row = vv + (size_t)i * r;
            float t = 0.0f;
            for (int j = 0; j < r; j++) t += row[j] * s->sc[j];
            acc[i] += vs ? t * vs[h * hd + i] : t;
        }
    }
}

/* src/nn.rs:233-258: integer keys and values; q already multiplied by the keys' scales. width 2 (i16) or 1 (i8). */
static void soft_update_int(Soft *s, const float *q, const void *kt, const void *vt, int width, const float *vs, int r) {
    int hd = s->d / s->heads;
    for (int h = 0; h < s->heads; h++) {
        for (int j = 0; j < r; j++) s->sc[j] = 0.0f;
        for (int i = 0; i < hd; i++) {
            float qi = q[h * hd + i];
            size_t base = (size_t)(h * hd + i) * r;
            for (int j = 0; j < r; j++) {
                float v = width == 2 ? (float)((const int16_t *)kt)[base + j] : (float)((const int8_t *)kt)[base + j];
                s->sc[j] += qi * v;
            }
        }
        soft_rescale(s, h, r);
        float *acc = s->acc + h * hd;
        for (int i = 0; i < hd; i++) {
            size_t base = (size_t)(h * hd + i) * r;
            float t = 0.0f;
            for (int j = 0; j < r; j++) {
                float v = width == 2 ? (float)((const int16_t *)vt)[base + j] : (float)((const int8_t *)vt)[base + j];
                t += v * s->sc[j];
            }
            acc[i] += t * vs[h * hd + i];
        }
    }
}

/* src/nn.rs:261-276 */
static void soft_merge(Soft *a, const Soft *o) {
    int hd = a->d / a->heads;
    for (int h = 0; h < a->heads; h++) {
        if (o->s[h] <= 0.0f) continue;
        float top = a->m[h] > o->m[h] ? a->m[h] : o->m[h];
        float fa = a->s[h] > 0.0f ? orc_exp1(a->m[h] - top) : 0.0f;
        float fb = orc_exp1(o->m[h] - top);
        a->s[h] = a->s[h] * fa + o->s[h] * fb;
        for (int i = h * hd; i < (h + 1) * hd; i++) a->acc[i] = a->acc[i] * fa + o->acc[i] * fb;
        a->m[h] = top;
    }
}

/* src/nn.rs:280-286 */
static void soft_finish(Soft *s) {
    int hd = s->d / s->heads;
    for (int h = 0; h < s->heads; h++) {
        float inv = 1.0f / s->s[h];
        for (int i = 0; i < hd; i++) s->acc[h * hd + i] *= inv;
    }
}

/* src/nn.rs:291-301: one whole block for one token against n cached keys and values [d][n]. */
static void cached_block(const tah_block *b, const float *scale, const float *kt, const float *vt, int n, float *x) {
    int d = b->d;
    float *q = xcalloc(d, sizeof(float));
    float *t = xcalloc(d, sizeof(float));
    Soft s = soft_new(b->heads, d, n);
    orc_query(b, scale, x, q);
    soft_update(&s, q, kt, vt, NULL, n);
    soft_finish(&s);
    orc_linear(b->out_w, b->out_b, s.acc, d, d, t);
    for (int i = 0; i < d; i++) x[i] += t[i];
    orc_feed_forward(b, x);
    soft_free(&s);
    free(q);
    free(t);
}

/* src/model.rs:188-200 */
static void add_y(const tah_model_desc *m, const float *table, float y, float *cell, int w) {
    if (m->max_classes > 0) {
        const float *row = table + (size_t)(int)y * w;
        for (int i = 0; i < w; i++) cell[i] += row[i];
    } else {
        for (int i = 0; i < w; i++) cell[i] += table[i] * y + table[w + i];
    }
}

/* src/nn.rs:424-429 */
static void group_values(const float *row, int h, int g, int size, float *out) {
    for (int i = 0; i < size; i++) out[i] = row[(g + (1 << i)) % h];
}

/* The input layer for one cell (src/fit.rs:340-345, src/predict.rs:313-318): all -100 stays -100. */
static void input_cell(const tah_model_desc *m, const float *xrow, int features, int g, float *cell) {
    float vals[8];
    group_values(xrow, features, g, m->group, vals);
    int missing = 1;
    for (int i = 0; i < m->group; i++) missing &= vals[i] == -100.0f;
    if (missing) {
        for (int i = 0; i < m->e; i++) cell[i] = -100.0f;
    } else {
        orc_linear(m->in_w, m->in_b, vals, m->group, m->e, cell);
    }
}

/* src/nn.rs:357-419: the row stage for one row; tok [tokens][e] is scratch, out receives cls * e numbers. */
static void row_forward(const tah_model_desc *m, const float *cosv, const float *sinv, float *tok, int tokens, float *out) {
    int d = m->e, heads = m->row_heads, hd = d / heads, half = hd / 2;
    float inv = 1.0f / sqrtf((float)hd);
    int last = m->row_blocks - 1;
    float *tn = xcalloc(d, sizeof(float));
    float *qkv = xcalloc(3 * d, sizeof(float));
    float *q = xcalloc((size_t)tokens * d, sizeof(float));
    float *kt = xcalloc((size_t)tokens * d, sizeof(float));
    float *vt = xcalloc((size_t)tokens * d, sizeof(float));
    float *nw = xcalloc((size_t)tokens * d, sizeof(float));
    float *sc = xcalloc(tokens, sizeof(float));
    float *att = xcalloc(d, sizeof(float));
    for (int bi = 0; bi < m->row_blocks; bi++) {
        const tah_block *b = &m->row[bi];
        int nq = bi == last ? m->cls : tokens;
        for (int t = 0; t < tokens; t++) {
            orc_layer_norm(tok + (size_t)t * d, d, b->n1w, b->n1b, tn);
            if (t < nq)
                orc_linear(b->in_w, b->in_b, tn, d, 3 * d, qkv);
            else
                orc_linear(b->in_w + (size_t)d * d, b->in_b + d, tn, d, 2 * d, qkv + d);
            const float *cs = cosv + (size_t)t * half, *sn = sinv + (size_t)t * half;
            for (int h = 0; h < heads; h++) {
                if (t < nq) {
                    const float *src = qkv + h * hd;
                    float *dst = q + (size_t)t * d + h * hd;
                    for (int i = 0; i < half; i++) {
                        float a = src[i], c = src[i + half];
                        dst[i] = (a * cs[i] - c * sn[i]) * inv;
                        dst[i + half] = (c * cs[i] + a * sn[i]) * inv;
                    }
                }
                const float *src = qkv + d + h * hd;
                for (int i = 0; i < half; i++) {
                    float a = src[i], c = src[i + half];
                    kt[(size_t)(h * hd + i) * tokens + t] = a * cs[i] - c * sn[i];
                    kt[(size_t)(h * hd + i + half) * tokens + t] = c * cs[i] + a * sn[i];
                }
            }
            for (int j = 0; j < d; j++) vt[(size_t)j * tokens + t] = qkv[2 * d + j];
        }
        for (int t = 0; t < nq; t++) {
            for (int h = 0; h < heads; h++) {
                const float *ks = kt + (size_t)h * hd * tokens, *vv = vt + (size_t)h * hd * tokens;
                for (int j = 0; j < tokens; j++) sc[j] = 0.0f;
                for (int i = 0; i < hd; i++) {
                    float qi = q[(size_t)t * d + h * hd + i];
                    for (int j = 0; j < tokens; j++) sc[j] += qi * ks[(size_t)i * tokens + j];
                }
                float top = -INFINITY;
                for (int j = 0; j < tokens; j++) top = sc[j] > top ? sc[j] : top;
                float s = 1.0f / exp_shift_sum(sc, tokens, top);
                for (int i = 0; i < hd; i++) {
                    float acc = 0.0f;
                    for (int j = 0; j < tokens; j++) acc += vv[(size_t)i * tokens + j] * sc[j];
                    att[h * hd + i] = acc * s;
                }
            }
            float *x = nw + (size_t)t * d;
            orc_linear(b->out_w, b->out_b, att, d, d, x);
            for (int i = 0; i < d; i++) x[i] += tok[(size_t)t * d + i];
            orc_feed_forward(b, x);
        }
        memcpy(tok, nw, sizeof(float) * (size_t)nq * d);
    }
    for (int c = 0; c < m->cls; c++) orc_layer_norm(tok + (size_t)c * d, d, m->out_lnw, m->out_lnb, out + (size_t)c * d);
    free(tn);
    free(qkv);
    free(q);
    free(kt);
    free(vt);
    free(nw);
    free(sc);
    free(att);
}

/* Rope::new, src/nn.rs:304-321: cos and sin of position * frequency, [positions][half]. */
static void rope_tables(const tah_model_desc *m, int positions, float **cosv, float **sinv) {
    int half = m->rope_half;
    *cosv = xcalloc((size_t)positions * half, sizeof(float));
    *sinv = xcalloc((size_t)positions * half, sizeof(float));
    for (int p = 0; p < positions; p++)
        for (int i = 0; i < half; i++) {
            float a = (float)p * m->rope_freqs[i];
            (*cosv)[(size_t)p * half + i] = cosf(a);
            (*sinv)[(size_t)p * half + i] = sinf(a);
        }
}

/* ---------------------------------------------------------------- fit.rs ----------------------------------- */

/* src/fit.rs:549-576: per coordinate row of the chunk, scale = max|v| / top (1 if all zero), code = round(v / s)
 * with Rust's saturating float-to-int cast; the 2d scales are written first. */
void orc_pack(const float *c, int d, int rc, int kv_format, uint8_t *out) {
    if (kv_format == TAH_KV_F32) {
        memcpy(out, c, sizeof(float) * 2 * (size_t)d * rc);
        return;
    }
    float top = kv_format == TAH_KV_I16 ? 32767.0f : 127.0f;
    float *scales = (float *)out;
    uint8_t *body = out + 8 * (size_t)d;
    for (int j = 0; j < 2 * d; j++) {
        const float *row = c + (size_t)j * rc;
        float big = 0.0f;
        for (int r = 0; r < rc; r++) {
            float a = fabsf(row[r]);
            big = a > big ? a : big; /* f32::max: a NaN operand yields the other */
        }
        float s = big > 0.0f ? big / top : 1.0f;
        float inv = 1.0f / s;
        float sv = s;
        memcpy(&scales[j], &sv, 4);
        for (int r = 0; r < rc; r++) {
            float v = roundf(row[r] * inv);
            if (kv_format == TAH_KV_I16) {
                int16_t code = isnan(v) ? 0 : (v >= 32767.0f ? 32767 : (v <= -32768.0f ? -32768 : (int16_t)v));
                memcpy(body + 2 * ((size_t)j * rc + r), &code, 2);
            } else {
                int8_t code = isnan(v) ? 0 : (v >= 127.0f ? 127 : (v <= -128.0f ? -128 : (int8_t)v));
                body[(size_t)j * rc + r] = (uint8_t)code;
            }
        }
    }
}

/* One row's attention over stored records, chunks [c0, c1), into s (src/predict.rs:459-499). */
static void attend_chunks(Soft *s, const float *q, float *qs, const uint8_t *records, int kv_format, int rows, int chunk,
                          int d, int c0, int c1) {
    size_t full = orc_kv_record(kv_format, d, chunk);
    for (int ci = c0; ci < c1; ci++) {
        int rc = rows - ci * chunk < chunk ? rows - ci * chunk : chunk;
        const uint8_t *rec = records + (size_t)ci * full;
        if (kv_format == TAH_KV_F32) {
            const float *all = (const float *)rec;
            soft_update(s, q, all, all + (size_t)d * rc, NULL, rc);
        } else {
            const float *sc = (const float *)rec;
            const uint8_t *body = rec + 8 * (size_t)d;
            int w = kv_format == TAH_KV_I16 ? 2 : 1;
            for (int i = 0; i < d; i++) qs[i] = q[i] * sc[i];
            soft_update_int(s, qs, body, body + (size_t)w * d * rc, w, sc + d, rc);
        }
    }
}

void orc_attend_records(const float *q, int nq, const uint8_t *records, int kv_format, int rows, int chunk, int d,
                        int heads, int key_parts, float *out) {
    int n_chunks = (rows + chunk - 1) / chunk;
    if (key_parts < 1) key_parts = 1;
    if (key_parts > n_chunks) key_parts = n_chunks;
#pragma omp parallel for schedule(dynamic, 1)
    for (int i = 0; i < nq; i++) {
        float *qs = xcalloc(d, sizeof(float));
        Soft first = soft_new(heads, d, chunk);
        int per = (n_chunks + key_parts - 1) / key_parts;
        attend_chunks(&first, q + (size_t)i * d, qs, records, kv_format, rows, chunk, d, 0, per < n_chunks ? per : n_chunks);
        for (int p = 1; p * per < n_chunks; p++) {
            Soft o = soft_new(heads, d, chunk);
            int c1 = (p + 1) * per < n_chunks ? (p + 1) * per : n_chunks;
            attend_chunks(&o, q + (size_t)i * d, qs, records, kv_format, rows, chunk, d, p * per, c1);
            soft_merge(&first, &o);
            soft_free(&o);
        }
        soft_finish(&first);
        memcpy(out + (size_t)i * d, first.acc, sizeof(float) * d);
        soft_free(&first);
        free(qs);
    }
}

void orc_fit_attend(const float *q, const float *kv, int rows, int chunk, int d, int heads, float *out) {
    orc_attend_records(q, rows, (const uint8_t *)kv, TAH_KV_F32, rows, chunk, d, heads, 1, out);
}

/* src/fit.rs:326-423 for one feature group g: src [rows][e] gets the cells after the stage, rec the group's
 * col_kv record [digits][blocks][2][e][inds]. ind_q [blocks][inds][e]. */
static void col_one(const tah_model_desc *m, const float *x, const float *y, int rows, int features, int g,
                    const int *bases, int digits, int chunk, const float *ind_q, const float *a2_scale, float *src,
                    float *rec) {
    int e = m->e, inds = m->inds, nb = m->col_blocks;
    for (int r = 0; r < rows; r++) input_cell(m, x + (size_t)r * features, features, g, src + (size_t)r * e);
    float *plain = NULL, *sum = NULL;
    if (digits > 1) {
        plain = xcalloc((size_t)rows * e, sizeof(float));
        sum = xcalloc((size_t)rows * e, sizeof(float));
        memcpy(plain, src, sizeof(float) * (size_t)rows * e);
    }
    const tah_block *a1_0 = &m->col_a1[0];
    Soft *softs = xcalloc(inds, sizeof(Soft));
    for (int i = 0; i < inds; i++) softs[i] = soft_new(a1_0->heads, e, chunk > inds ? chunk : inds);
    float *kt = xcalloc((size_t)e * chunk, sizeof(float)), *vt = xcalloc((size_t)e * chunk, sizeof(float));
    float *kv = xcalloc(2 * e, sizeof(float)), *t = xcalloc(e, sizeof(float));
    float *hidden = xcalloc((size_t)inds * e, sizeof(float));
    for (int dg = 0; dg < digits; dg++) {
        if (dg > 0) memcpy(src, plain, sizeof(float) * (size_t)rows * e);
        int divisor = 1;
        for (int k = dg + 1; k < digits; k++) divisor *= bases[k];
        for (int r = 0; r < rows; r++) {
            float yv = digits > 1 ? (float)(((int)y[r] / divisor) % bases[dg]) : y[r];
            add_y(m, m->col_y, yv, src + (size_t)r * e, e);
        }
        float *recd = rec + (size_t)dg * nb * 2 * e * inds;
        for (int bi = 0; bi < nb; bi++) {
            const tah_block *a1 = &m->col_a1[bi], *a2 = &m->col_a2[bi];
            for (int i = 0; i < inds; i++) soft_reset(&softs[i]);
            for (int r0 = 0; r0 < rows; r0 += chunk) {
                int rc = rows - r0 < chunk ? rows - r0 : chunk;
                for (int r = 0; r < rc; r++) {
                    orc_layer_norm(src + (size_t)(r0 + r) * e, e, a1->n1w, a1->n1b, t);
                    orc_linear(a1->in_w + (size_t)e * e, a1->in_b + e, t, e, 2 * e, kv);
                    for (int j = 0; j < e; j++) {
                        kt[(size_t)j * rc + r] = kv[j];
                        vt[(size_t)j * rc + r] = kv[e + j];
                    }
                }
                for (int i = 0; i < inds; i++)
                    soft_update(&softs[i], ind_q + ((size_t)bi * inds + i) * e, kt, vt, NULL, rc);
            }
            for (int i = 0; i < inds; i++) {
                soft_finish(&softs[i]);
                float *hid = hidden + (size_t)i * e;
                orc_linear(a1->out_w, a1->out_b, softs[i].acc, e, e, hid);
                for (int j = 0; j < e; j++) hid[j] += m->col_ind[((size_t)bi * inds + i) * e + j];
                orc_feed_forward(a1, hid);
            }
            float *rk = recd + (size_t)bi * 2 * e * inds, *rv = rk + (size_t)e * inds;
            for (int i = 0; i < inds; i++) {
                orc_layer_norm(hidden + (size_t)i * e, e, a2->n1w, a2->n1b, t);
                orc_linear(a2->in_w + (size_t)e * e, a2->in_b + e, t, e, 2 * e, kv);
                for (int j = 0; j < e; j++) {
                    rk[(size_t)j * inds + i] = kv[j];
                    rv[(size_t)j * inds + i] = kv[e + j];
                }
            }
            for (int r = 0; r < rows; r++) cached_block(a2, a2_scale, rk, rv, inds, src + (size_t)r * e);
        }
        if (digits > 1)
            for (size_t k = 0; k < (size_t)rows * e; k++) sum[k] += src[k];
    }
    if (digits > 1) {
        float inv = 1.0f / (float)digits;
        for (size_t k = 0; k < (size_t)rows * e; k++) src[k] = sum[k] * inv;
        free(plain);
        free(sum);
    }
    for (int i = 0; i < inds; i++) soft_free(&softs[i]);
    free(softs);
    free(kt);
    free(vt);
    free(kv);
    free(t);
    free(hidden);
}

/* The column stage of a fit for the feature groups listed in groups [ngroups] (all of them when groups is NULL):
 * col_kv [ngroups][digits][blocks][2][e][inds] and emb [ngroups][rows][e], each group as src/fit.rs:326-423 fits
 * it (groups are independent: a group's cache depends on its own cells over all rows). */
void orc_fit_columns_of(const tah_model_desc *m, const float *x, const float *y, int rows, int features,
                        const int *groups, int ngroups, const int *bases, int digits, int chunk, float *col_kv,
                        float *emb) {
    int e = m->e, inds = m->inds, nb = m->col_blocks;
    /* the inducing points' queries, once per block (src/fit.rs:300-313), scaled for all `rows` */
    float *ind_q = xcalloc((size_t)nb * inds * e, sizeof(float));
    float *scale = xcalloc(e, sizeof(float));
    for (int bi = 0; bi < nb; bi++) {
        orc_query_scale(&m->col_a1[bi], rows, scale);
        for (int i = 0; i < inds; i++)
            orc_query(&m->col_a1[bi], scale, m->col_ind + ((size_t)bi * inds + i) * e, ind_q + ((size_t)bi * inds + i) * e);
    }
    float *a2_scale = xcalloc(e, sizeof(float));
    for (int i = 0; i < e; i++) a2_scale[i] = 1.0f / sqrtf((float)hd_of(&m->col_a2[0]));
    size_t rec_len = (size_t)digits * nb * 2 * e * inds;
    int count = groups ? ngroups : features;
#pragma omp parallel for schedule(dynamic, 1)
    for (int k = 0; k < count; k++)
        col_one(m, x, y, rows, features, groups ? groups[k] : k, bases, digits, chunk, ind_q, a2_scale,
                emb + (size_t)k * rows * e, col_kv + (size_t)k * rec_len);
    free(ind_q);
    free(scale);
    free(a2_scale);
}

void orc_fit_columns(const tah_model_desc *m, const float *x, const float *y, int rows, int features,
                     const int *bases, int digits, int chunk, float *col_kv, float *emb) {
    orc_fit_columns_of(m, x, y, rows, features, NULL, 0, bases, digits, chunk, col_kv, emb);
}

/* The fit's cells of n given training rows (x [n][features], y [n]) after the column stage, from a fitted column
 * cache col_kv [features][digits][blocks][2][e][inds]: each digit's cell (input cell plus that digit's label
 * embedding) through every block against the block's cached inducing keys and values, the digits averaged
 * (src/fit.rs:360-423). emb [features][n][e]. */
void orc_fit_cells_rows(const tah_model_desc *m, const float *col_kv, const int *bases, int digits, const float *x,
                        const float *y, int n, int features, float *emb) {
    int e = m->e, inds = m->inds, nb = m->col_blocks;
    size_t rec_len = (size_t)digits * nb * 2 * e * inds;
    float *a2_scale = xcalloc(e, sizeof(float));
    for (int i = 0; i < e; i++) a2_scale[i] = 1.0f / sqrtf((float)hd_of(&m->col_a2[0]));
#pragma omp parallel for schedule(dynamic, 1)
    for (int g = 0; g < features; g++) {
        float *plain = xcalloc(e, sizeof(float)), *cell = xcalloc(e, sizeof(float)), *sum = xcalloc(e, sizeof(float));
        for (int r = 0; r < n; r++) {
            input_cell(m, x + (size_t)r * features, features, g, plain);
            for (int j = 0; j < e; j++) sum[j] = 0.0f;
            for (int dg = 0; dg < digits; dg++) {
                memcpy(cell, plain, sizeof(float) * e);
                int divisor = 1;
                for (int k = dg + 1; k < digits; k++) divisor *= bases[k];
                float yv = digits > 1 ? (float)(((int)y[r] / divisor) % bases[dg]) : y[r];
                add_y(m, m->col_y, yv, cell, e);
                for (int bi = 0; bi < nb; bi++) {
                    const float *rk = col_kv + (size_t)g * rec_len + ((size_t)dg * nb + bi) * 2 * e * inds;
                    cached_block(&m->col_a2[bi], a2_scale, rk, rk + (size_t)e * inds, inds, cell);
                }
                if (digits > 1)
                    for (int j = 0; j < e; j++) sum[j] += cell[j];
            }
            float *out = emb + ((size_t)g * n + r) * e;
            if (digits > 1) {
                float inv = 1.0f / (float)digits;
                for (int j = 0; j < e; j++) out[j] = sum[j] * inv;
            } else {
                memcpy(out, cell, sizeof(float) * e);
            }
        }
        free(plain);
        free(cell);
        free(sum);
    }
    free(a2_scale);
}

void orc_fit_rows(const tah_model_desc *m, const float *emb, int rows, int features, float *reps) {
    int e = m->e, tokens = m->cls + features;
    float *cosv, *sinv;
    rope_tables(m, tokens, &cosv, &sinv);
#pragma omp parallel for schedule(dynamic, 16)
    for (int r = 0; r < rows; r++) {
        float *tok = xcalloc((size_t)tokens * e, sizeof(float));
        memcpy(tok, m->cls_tokens, sizeof(float) * (size_t)m->cls * e);
        for (int g = 0; g < features; g++)
            memcpy(tok + (size_t)(m->cls + g) * e, emb + ((size_t)g * rows + r) * e, sizeof(float) * e);
        row_forward(m, cosv, sinv, tok, tokens, reps + (size_t)r * m->d);
        free(tok);
    }
    free(cosv);
    free(sinv);
}

/* src/fit.rs:627-663: one layer's keys and values for every row, chunk by chunk, as f32 chunk records. */
static void fill_kv(const tah_block *b, const float *h, int rows, int chunk, float *kv) {
    int d = b->d;
    int n_chunks = (rows + chunk - 1) / chunk;
#pragma omp parallel for schedule(dynamic, 1)
    for (int ci = 0; ci < n_chunks; ci++) {
        int r0 = ci * chunk, rc = rows - r0 < chunk ? rows - r0 : chunk;
        float *kt = kv + 2 * (size_t)d * r0, *vt = kt + (size_t)d * rc;
        float *t = xcalloc(d, sizeof(float)), *two = xcalloc(2 * d, sizeof(float));
        for (int r = 0; r < rc; r++) {
            orc_layer_norm(h + (size_t)(r0 + r) * d, d, b->n1w, b->n1b, t);
            orc_linear(b->in_w + (size_t)d * d, b->in_b + d, t, d, 2 * d, two);
            for (int j = 0; j < d; j++) {
                kt[(size_t)j * rc + r] = two[j];
                vt[(size_t)j * rc + r] = two[d + j];
            }
        }
        free(t);
        free(two);
    }
}

void orc_fit_icl(const tah_model_desc *m, float *h, int rows, int chunk, int kv_format, float *scales,
                 uint8_t *const *records, float *kv_f32) {
    int d = m->d;
    int n_chunks = (rows + chunk - 1) / chunk;
    size_t full = orc_kv_record(kv_format, d, chunk);
    float *kv = xcalloc(2 * (size_t)rows * d, sizeof(float));
    float *q = xcalloc((size_t)rows * d, sizeof(float));
    float *att = xcalloc((size_t)rows * d, sizeof(float));
    for (int l = 0; l < m->icl_layers; l++) {
        const tah_block *b = &m->icl[l];
        float *scale = scales + (size_t)l * d;
        orc_query_scale(b, rows, scale);
        fill_kv(b, h, rows, chunk, kv);
        for (int ci = 0; ci < n_chunks; ci++) {
            int r0 = ci * chunk, rc = rows - r0 < chunk ? rows - r0 : chunk;
            orc_pack(kv + 2 * (size_t)d * r0, d, rc, kv_format, records[l] + (size_t)ci * full);
        }
        if (kv_f32) memcpy(kv_f32 + (size_t)l * 2 * rows * d, kv, sizeof(float) * 2 * (size_t)rows * d);
        if (l + 1 == m->icl_layers) break; /* the last layer's own outputs are never used (src/fit.rs:664-666) */
#pragma omp parallel for schedule(dynamic, 16)
        for (int r = 0; r < rows; r++) orc_query(b, scale, h + (size_t)r * d, q + (size_t)r * d);
        orc_fit_attend(q, kv, rows, chunk, d, b->heads, att);
#pragma omp parallel for schedule(dynamic, 16)
        for (int r = 0; r < rows; r++) {
            float *x = h + (size_t)r * d;
            float *t = xcalloc(d, sizeof(float));
            orc_linear(b->out_w, b->out_b, att + (size_t)r * d, d, d, t);
            for (int j = 0; j < d; j++) x[j] += t[j];
            orc_feed_forward(b, x);
            free(t);
        }
    }
    free(kv);
    free(q);
    free(att);
}

/* One in-context layer's keys and values for n given rows h [n][d] (src/fit.rs:627-663, before the chunk layout):
 * kv [n][2d], keys then values of each row. */
void orc_kv_rows(const tah_model_desc *m, int layer, const float *h, int n, float *kv) {
    const tah_block *b = &m->icl[layer];
    int d = b->d;
#pragma omp parallel for schedule(dynamic, 16)
    for (int r = 0; r < n; r++) {
        float *t = xcalloc(d, sizeof(float));
        orc_layer_norm(h + (size_t)r * d, d, b->n1w, b->n1b, t);
        orc_linear(b->in_w + (size_t)d * d, b->in_b + d, t, d, 2 * d, kv + (size_t)r * 2 * d);
        free(t);
    }
}

/* n rows h [n][d] (in place) through in-context layer `layer`: query (scaled by scale [d]), attention over the
 * layer's stored records, output projection and residual, feed-forward (src/fit.rs:700-744 for training rows over
 * exact f32 records; src/predict.rs:413-568 for test rows). */
void orc_icl_step(const tah_model_desc *m, int layer, const float *scale, const uint8_t *records, int kv_format,
                  int rows, int chunk, float *h, int n) {
    const tah_block *b = &m->icl[layer];
    int d = b->d;
    float *q = xcalloc((size_t)n * d, sizeof(float));
    float *att = xcalloc((size_t)n * d, sizeof(float));
#pragma omp parallel for schedule(dynamic, 16)
    for (int r = 0; r < n; r++) orc_query(b, scale, h + (size_t)r * d, q + (size_t)r * d);
    orc_attend_records(q, n, records, kv_format, rows, chunk, d, b->heads, 1, att);
#pragma omp parallel for schedule(dynamic, 16)
    for (int r = 0; r < n; r++) {
        float *x = h + (size_t)r * d;
        float *t = xcalloc(d, sizeof(float));
        orc_linear(b->out_w, b->out_b, att + (size_t)r * d, d, d, t);
        for (int j = 0; j < d; j++) x[j] += t[j];
        orc_feed_forward(b, x);
        free(t);
    }
    free(q);
    free(att);
}

/* ---------------------------------------------------------------- predict.rs ------------------------------- */

void orc_in_context(const tah_model_desc *m, const float *scales, const uint8_t *const *records, int kv_format,
                    int rows, int chunk, float *h, int n, int out_n, float *out) {
    int d = m->d;
    float *q = xcalloc((size_t)n * d, sizeof(float));
    float *att = xcalloc((size_t)n * d, sizeof(float));
    for (int l = 0; l < m->icl_layers; l++) {
        const tah_block *b = &m->icl[l];
#pragma omp parallel for schedule(dynamic, 16)
        for (int r = 0; r < n; r++) orc_query(b, scales + (size_t)l * d, h + (size_t)r * d, q + (size_t)r * d);
        orc_attend_records(q, n, records[l], kv_format, rows, chunk, d, b->heads, 1, att);
#pragma omp parallel for schedule(dynamic, 16)
        for (int r = 0; r < n; r++) {
            float *x = h + (size_t)r * d;
            float *t = xcalloc(d, sizeof(float));
            orc_linear(b->out_w, b->out_b, att + (size_t)r * d, d, d, t);
            for (int j = 0; j < d; j++) x[j] += t[j];
            orc_feed_forward(b, x);
            free(t);
        }
    }
    /* decoder, src/predict.rs:570-585 */
#pragma omp parallel for schedule(dynamic, 16)
    for (int r = 0; r < n; r++) {
        float *t = xcalloc(d, sizeof(float));
        float *hid = xcalloc(m->dec_hidden, sizeof(float));
        float *all = xcalloc(m->outputs, sizeof(float));
        orc_layer_norm(h + (size_t)r * d, d, m->lnw, m->lnb, t);
        orc_linear(m->dec0w, m->dec0b, t, d, m->dec_hidden, hid);
        orc_gelu(hid, m->dec_hidden);
        orc_linear(m->dec2w, m->dec2b, hid, m->dec_hidden, m->outputs, all);
        memcpy(out + (size_t)r * out_n, all, sizeof(float) * out_n);
        free(t);
        free(hid);
        free(all);
    }
    free(q);
    free(att);
}

void orc_embed(const tah_model_desc *m, const float *col_kv, int digits, const float *x, int n, int features,
               float *tok) {
    int e = m->e, inds = m->inds, nb = m->col_blocks, tokens = m->cls + features;
    size_t per = 2 * (size_t)e * inds, rec_len = (size_t)digits * nb * per;
    float *scale = xcalloc(e, sizeof(float));
    for (int i = 0; i < e; i++) scale[i] = 1.0f / sqrtf((float)hd_of(&m->col_a2[0]));
#pragma omp parallel for schedule(dynamic, 1)
    for (int r = 0; r < n; r++) {
        float *t = tok + (size_t)r * tokens * e;
        const float *xr = x + (size_t)r * features;
        memcpy(t, m->cls_tokens, sizeof(float) * (size_t)m->cls * e);
        float *plain = xcalloc(e, sizeof(float)), *sum = xcalloc(e, sizeof(float)), *one = xcalloc(e, sizeof(float));
        for (int g = 0; g < features; g++) {
            float *cell = t + (size_t)(m->cls + g) * e;
            input_cell(m, xr, features, g, cell);
            const float *recs = col_kv + (size_t)g * rec_len;
            if (digits == 1) {
                for (int bi = 0; bi < nb; bi++)
                    cached_block(&m->col_a2[bi], scale, recs + bi * per, recs + bi * per + (size_t)e * inds, inds, cell);
            } else {
                memcpy(plain, cell, sizeof(float) * e);
                memset(sum, 0, sizeof(float) * e);
                for (int dg = 0; dg < digits; dg++) {
                    memcpy(one, plain, sizeof(float) * e);
                    for (int bi = 0; bi < nb; bi++) {
                        const float *at = recs + ((size_t)dg * nb + bi) * per;
                        cached_block(&m->col_a2[bi], scale, at, at + (size_t)e * inds, inds, one);
                    }
                    for (int i = 0; i < e; i++) sum[i] += one[i];
                }
                for (int i = 0; i < e; i++) cell[i] = sum[i] / (float)digits;
            }
        }
        free(plain);
        free(sum);
        free(one);
    }
    free(scale);
}

void orc_represent(const tah_model_desc *m, float *tok, int n, int tokens, float *rep) {
    float *cosv, *sinv;
    rope_tables(m, tokens, &cosv, &sinv);
#pragma omp parallel for schedule(dynamic, 4)
    for (int r = 0; r < n; r++) row_forward(m, cosv, sinv, tok + (size_t)r * tokens * m->e, tokens, rep + (size_t)r * m->d);
    free(cosv);
    free(sinv);
}

/* Kv::record, src/fit.rs:123-126. */
size_t orc_kv_record(int kv_format, int d, int rc) {
    size_t w = kv_format == TAH_KV_F32 ? 4 : (kv_format == TAH_KV_I16 ? 2 : 1);
    return 2 * (size_t)d * rc * w + (kv_format == TAH_KV_F32 ? 0 : 8 * (size_t)d);
}
