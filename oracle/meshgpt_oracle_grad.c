/*
 * TEST INFRASTRUCTURE ONLY — not part of the product.
 *
 * The reference's training arithmetic restated in C for the checker: the
 * scalar reverse-mode tape of src/gpt/reference.rs:244-390 (every node a value
 * and at most two weighted parent edges), the forward pass recorded on it
 * (reference.rs:104-228,392-603), the next-token loss and its gradient
 * (reference.rs:61-89) with the layout's gradient mask (config.rs:490-500),
 * and the f32 AdamW update of the GPU path (gpu.rs:1366-1391,1971-2003).
 * Pinned by the reference's own finite-difference and answer-only tests
 * (reference.rs:911-989), restated in tests/test_oracle_train.py.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "meshgpt_oracle.h"

#define NONE ((size_t)-1)
#define OG_MAX_ROWS 131072u /* src/gpt/mod.rs:31 */

/* reference.rs:244-259: values plus two (parent, derivative) edges per node;
 * the parameters are the first `count` nodes. */
typedef struct {
    double *val, *d0, *d1;
    size_t *p0, *p1;
    size_t n, cap;
    int failed;
} Tape;

static void tape_reserve(Tape *t, size_t cap) {
    if (cap <= t->cap || t->failed) return;
    double *v = (double *)realloc(t->val, cap * sizeof(double));
    if (v) t->val = v;
    double *a = (double *)realloc(t->d0, cap * sizeof(double));
    if (a) t->d0 = a;
    double *b = (double *)realloc(t->d1, cap * sizeof(double));
    if (b) t->d1 = b;
    size_t *c = (size_t *)realloc(t->p0, cap * sizeof(size_t));
    if (c) t->p0 = c;
    size_t *d = (size_t *)realloc(t->p1, cap * sizeof(size_t));
    if (d) t->p1 = d;
    if (!v || !a || !b || !c || !d) {
        t->failed = 1;
        return;
    }
    t->cap = cap;
}

static size_t node(Tape *t, double value, size_t a, double da, size_t b, double db) {
    if (t->n == t->cap) tape_reserve(t, t->cap ? 2 * t->cap : 1024);
    if (t->failed) return 0;
    size_t id = t->n++;
    t->val[id] = value;
    t->p0[id] = a;
    t->d0[id] = da;
    t->p1[id] = b;
    t->d1[id] = db;
    return id;
}

static void tape_free(Tape *t) {
    free(t->val);
    free(t->d0);
    free(t->d1);
    free(t->p0);
    free(t->p1);
}

/* reference.rs:263-332 */
static size_t t_constant(Tape *t, double v) { return node(t, v, NONE, 0.0, NONE, 0.0); }
static size_t t_add(Tape *t, size_t a, size_t b) { return node(t, t->val[a] + t->val[b], a, 1.0, b, 1.0); }
static size_t t_subtract(Tape *t, size_t a, size_t b) {
    return node(t, t->val[a] - t->val[b], a, 1.0, b, -1.0);
}
static size_t t_multiply(Tape *t, size_t a, size_t b) {
    double va = t->val[a], vb = t->val[b];
    return node(t, va * vb, a, vb, b, va);
}
static size_t t_divide(Tape *t, size_t a, size_t b) {
    double r = 1.0 / t->val[b], va = t->val[a];
    return node(t, va * r, a, r, b, -va * r * r);
}
static size_t t_scale(Tape *t, size_t a, double s) { return node(t, t->val[a] * s, a, s, NONE, 0.0); }
static size_t t_shift(Tape *t, size_t a, double o) { return node(t, t->val[a] + o, a, 1.0, NONE, 0.0); }
static size_t t_exp(Tape *t, size_t a) {
    double v = exp(t->val[a]);
    return node(t, v, a, v, NONE, 0.0);
}
static size_t t_log(Tape *t, size_t a) {
    double x = t->val[a];
    return node(t, log(x), a, 1.0 / x, NONE, 0.0);
}
static size_t t_inverse_sqrt(Tape *t, size_t a) {
    double v = 1.0 / sqrt(t->val[a]);
    return node(t, v, a, -0.5 * v * v * v, NONE, 0.0);
}
static size_t t_clamp_min(Tape *t, size_t a, double m) {
    double x = t->val[a];
    return node(t, x > m ? x : m, a, x >= m ? 1.0 : 0.0, NONE, 0.0);
}
static size_t t_elu(Tape *t, size_t a) {
    double x = t->val[a];
    if (x >= 0.0) return t_scale(t, a, 1.0);
    return node(t, expm1(x), a, exp(x), NONE, 0.0);
}
/* reference.rs:333-347: a left fold; dot multiplies first, then folds */
static size_t t_sum(Tape *t, const size_t *ids, size_t n) {
    size_t total = ids[0];
    for (size_t i = 1; i < n; ++i) total = t_add(t, total, ids[i]);
    return total;
}
static size_t t_dot(Tape *t, const size_t *a, const size_t *b, size_t n, size_t *scratch) {
    for (size_t i = 0; i < n; ++i) scratch[i] = t_multiply(t, a[i], b[i]);
    return t_sum(t, scratch, n);
}
/* reference.rs:348-361: shifts by the f64 maximum, exponentials, their sum */
static size_t t_shifted_exponentials(Tape *t, const size_t *ids, size_t n, double *maximum, size_t *exps) {
    double m = -INFINITY;
    for (size_t i = 0; i < n; ++i)
        if (t->val[ids[i]] > m) m = t->val[ids[i]];
    for (size_t i = 0; i < n; ++i) exps[i] = t_exp(t, t_shift(t, ids[i], -m));
    *maximum = m;
    return t_sum(t, exps, n);
}

/* reference.rs:392-409 on one row of `width` node ids, in place */
static void t_rmsnorm_row(Tape *t, size_t *row, size_t width, size_t heads, size_t *scratch) {
    size_t hw = width / heads;
    for (size_t h = 0; h < heads; ++h) {
        size_t *head = row + h * hw;
        size_t sum = t_dot(t, head, head, hw, scratch);
        size_t ms = t_scale(t, sum, 1.0 / (double)hw);
        size_t st = t_shift(t, ms, (double)1e-5f);
        size_t inv = t_inverse_sqrt(t, st);
        for (size_t i = 0; i < hw; ++i) head[i] = t_multiply(t, head[i], inv);
    }
}

/* reference.rs:422-453 over rows x width ids, in place; tmp holds rows x width */
static void t_mesh(Tape *t, size_t *x, size_t *tmp, size_t rows, size_t width, size_t offset, size_t depth,
                   uint32_t connectivity) {
    og_config shape = {0};
    shape.width = (uint32_t)width;
    shape.connectivity = connectivity;
    for (size_t layer = 0; layer < depth; ++layer) {
        uint32_t stride = og_stride(&shape, (uint32_t)layer);
        for (size_t r = 0; r < rows; ++r) {
            const size_t *row = x + r * width;
            for (size_t ch = 0; ch < width; ++ch) {
                size_t p = offset + layer * 2 * width + 2 * ch;
                size_t left = t_multiply(t, row[ch], p);
                size_t right = t_multiply(t, row[(ch + stride) % width], p + 1);
                size_t sum = t_add(t, left, right);
                tmp[r * width + ch] = layer + 1 == depth ? sum : t_elu(t, sum);
            }
        }
        memcpy(x, tmp, sizeof(size_t) * rows * width);
    }
}

/* reference.rs:462-482 on one row, in place (out holds width ids) */
static void t_rotary_row(Tape *t, size_t *row, size_t width, size_t heads, size_t position, size_t *out) {
    size_t hw = width / heads, half = hw / 2;
    memcpy(out, row, sizeof(size_t) * width);
    for (size_t h = 0; h < heads; ++h)
        for (size_t pair = 0; pair < half; ++pair) {
            double angle = (double)position / pow((double)10000.0f, (double)pair / (double)half);
            double sine = sin(angle), cosine = cos(angle);
            size_t l = h * hw + pair, r = l + half;
            size_t a = t_scale(t, row[l], cosine), b = t_scale(t, row[r], sine);
            out[l] = t_subtract(t, a, b);
            a = t_scale(t, row[r], cosine);
            b = t_scale(t, row[l], sine);
            out[r] = t_add(t, a, b);
        }
    memcpy(row, out, sizeof(size_t) * width);
}

/* reference.rs:510-554: rows x width ids of q, k, v -> out */
static void t_attention(Tape *t, const size_t *q, const size_t *k, const size_t *v, size_t rows, size_t width,
                        size_t heads, size_t sequence, size_t *out, size_t *scratch) {
    size_t hw = width / heads;
    size_t *scores = (size_t *)malloc(sizeof(size_t) * sequence);
    size_t *exps = (size_t *)malloc(sizeof(size_t) * sequence);
    size_t *contrib = (size_t *)malloc(sizeof(size_t) * sequence);
    for (size_t r = 0; r < rows; ++r) {
        size_t position = r % sequence, first = r - position;
        for (size_t h = 0; h < heads; ++h) {
            size_t b = h * hw;
            for (size_t j = 0; j <= position; ++j) {
                size_t s = t_dot(t, q + r * width + b, k + (first + j) * width + b, hw, scratch);
                scores[j] = t_scale(t, s, 1.0 / sqrt((double)hw));
            }
            double maximum;
            size_t sum = t_shifted_exponentials(t, scores, position + 1, &maximum, exps);
            for (size_t j = 0; j <= position; ++j) exps[j] = t_divide(t, exps[j], sum);
            for (size_t ch = b; ch < b + hw; ++ch) {
                for (size_t j = 0; j <= position; ++j) contrib[j] = t_multiply(t, exps[j], v[(first + j) * width + ch]);
                out[r * width + ch] = t_sum(t, contrib, position + 1);
            }
        }
    }
    free(scores);
    free(exps);
    free(contrib);
}

/* reference.rs:577-603 on one row, in place */
static void t_exclusive_row(Tape *t, size_t *y, const size_t *v, size_t width, size_t heads, size_t *scratch,
                            size_t *nv) {
    size_t hw = width / heads;
    double floor = (double)1e-12f * (double)1e-12f;
    for (size_t h = 0; h < heads; ++h) {
        const size_t *vh = v + h * hw;
        size_t *yh = y + h * hw;
        size_t sq = t_dot(t, vh, vh, hw, scratch);
        size_t fl = t_clamp_min(t, sq, floor);
        size_t inv = t_inverse_sqrt(t, fl);
        for (size_t i = 0; i < hw; ++i) nv[i] = t_multiply(t, vh[i], inv);
        size_t proj = t_dot(t, yh, nv, hw, scratch);
        for (size_t i = 0; i < hw; ++i) yh[i] = t_subtract(t, yh[i], t_multiply(t, proj, nv[i]));
    }
}

/* reference.rs:104-152: V x W ids of the effective token vectors */
static void t_embeddings(Tape *t, const og_config *c, size_t offset, size_t *emb, size_t *scratch) {
    size_t V = c->vocab_size, W = c->width;
    float *codes = (float *)malloc(sizeof(float) * V * W);
    og_token_codes(c, codes);
    if (c->embedding == 1) {
        for (size_t i = 0; i < V * W; ++i) emb[i] = offset + i;
    } else {
        size_t *tmp = (size_t *)malloc(sizeof(size_t) * V * W);
        for (size_t i = 0; i < V * W; ++i) emb[i] = t_constant(t, (double)codes[i]);
        t_mesh(t, emb, tmp, V, W, offset, c->attention_mesh_depth, c->connectivity);
        free(tmp);
    }
    if (c->normalization != 0) {
        double scale = c->normalization == 2 ? (double)sqrtf((float)W) : 1.0;
        double floor = (double)1e-12f * (double)1e-12f;
        for (size_t tok = 0; tok < V; ++tok) {
            size_t *row = emb + tok * W;
            size_t sq = t_dot(t, row, row, W, scratch);
            size_t inv = t_scale(t, t_inverse_sqrt(t, t_clamp_min(t, sq, floor)), scale);
            for (size_t i = 0; i < W; ++i) row[i] = t_multiply(t, row[i], inv);
        }
    }
    for (size_t tok = 0; tok < V; ++tok)
        for (size_t i = 0; i < c->preserve_features; ++i)
            emb[tok * W + i] = t_constant(t, (double)codes[tok * W + i]);
    free(codes);
}

int og_loss_and_gradient(const og_config *c, const float *params, const uint32_t *inputs,
                         const uint32_t *targets, size_t n, size_t sequence, double *loss, double *gradient) {
    size_t V = c->vocab_size, W = c->width, H = c->heads, L = c->layers;
    size_t A = c->attention_mesh_depth, F = c->ffn_mesh_depth;
    /* config.rs:210-252 */
    if (sequence == 0 || sequence > c->context || n == 0 || n % sequence != 0 || n > OG_MAX_ROWS) return -1;
    for (size_t i = 0; i < n; ++i)
        if (inputs[i] >= V) return -1;
    size_t supervised = 0;
    for (size_t i = 0; i < n; ++i) {
        if (targets[i] == UINT32_MAX) continue;
        if (targets[i] >= V) return -3;
        ++supervised;
    }
    if (!supervised) return -4;

    size_t count = og_parameter_count(c);
    size_t *offsets = (size_t *)malloc(sizeof(size_t) * (1 + 5 * L));
    og_group_offsets(c, offsets);
    Tape t = {0};
    tape_reserve(&t, count + 4096);
    for (size_t i = 0; i < count; ++i) node(&t, (double)params[i], NONE, 0.0, NONE, 0.0);

    size_t span = W > sequence ? W : sequence;
    size_t *scratch = (size_t *)malloc(sizeof(size_t) * (span > V ? span : V));
    size_t *emb = (size_t *)malloc(sizeof(size_t) * V * W);
    size_t rw = n * W;
    size_t *x = (size_t *)malloc(sizeof(size_t) * rw), *nrm = (size_t *)malloc(sizeof(size_t) * rw);
    size_t *q = (size_t *)malloc(sizeof(size_t) * rw), *k = (size_t *)malloc(sizeof(size_t) * rw);
    size_t *v = (size_t *)malloc(sizeof(size_t) * rw), *y = (size_t *)malloc(sizeof(size_t) * rw);
    size_t *tmp = (size_t *)malloc(sizeof(size_t) * rw), *row = (size_t *)malloc(sizeof(size_t) * W);
    size_t *losses = (size_t *)malloc(sizeof(size_t) * supervised);

    t_embeddings(&t, c, offsets[0], emb, scratch);
    for (size_t r = 0; r < n; ++r) memcpy(x + r * W, emb + (size_t)inputs[r] * W, sizeof(size_t) * W);
    for (size_t b = 0; b < L; ++b) {
        const size_t *g = offsets + 1 + 5 * b;
        memcpy(nrm, x, sizeof(size_t) * rw);
        for (size_t r = 0; r < n; ++r) t_rmsnorm_row(&t, nrm + r * W, W, 1, scratch);
        memcpy(q, nrm, sizeof(size_t) * rw);
        t_mesh(&t, q, tmp, n, W, g[0], A, c->connectivity);
        memcpy(k, nrm, sizeof(size_t) * rw);
        t_mesh(&t, k, tmp, n, W, g[1], A, c->connectivity);
        memcpy(v, nrm, sizeof(size_t) * rw);
        t_mesh(&t, v, tmp, n, W, g[2], A, c->connectivity);
        /* reference.rs:174-193: QK-Norm of all rows, then RoPE of all rows */
        if (c->qk_norm)
            for (size_t r = 0; r < n; ++r) {
                t_rmsnorm_row(&t, q + r * W, W, H, scratch);
                t_rmsnorm_row(&t, k + r * W, W, H, scratch);
            }
        if (c->rope)
            for (size_t r = 0; r < n; ++r) {
                t_rotary_row(&t, q + r * W, W, H, r % sequence, row);
                t_rotary_row(&t, k + r * W, W, H, r % sequence, row);
            }
        t_attention(&t, q, k, v, n, W, H, sequence, y, scratch);
        if (c->xsa)
            for (size_t r = 0; r < n; ++r) t_exclusive_row(&t, y + r * W, v + r * W, W, H, scratch, row);
        t_mesh(&t, y, tmp, n, W, g[3], A, c->connectivity);
        for (size_t i = 0; i < rw; ++i) x[i] = t_add(&t, x[i], y[i]);
        memcpy(nrm, x, sizeof(size_t) * rw);
        for (size_t r = 0; r < n; ++r) t_rmsnorm_row(&t, nrm + r * W, W, 1, scratch);
        t_mesh(&t, nrm, tmp, n, W, g[4], F, c->connectivity);
        for (size_t i = 0; i < rw; ++i) x[i] = t_add(&t, x[i], nrm[i]);
    }
    /* logits and the loss (reference.rs:66-80,218-226) */
    size_t *logit = (size_t *)malloc(sizeof(size_t) * V), *exps = (size_t *)malloc(sizeof(size_t) * V);
    size_t nl = 0;
    for (size_t r = 0; r < n; ++r) {
        memcpy(row, x + r * W, sizeof(size_t) * W);
        t_rmsnorm_row(&t, row, W, 1, scratch);
        if (targets[r] == UINT32_MAX) continue; /* its logits do not reach the loss */
        for (size_t tok = 0; tok < V; ++tok) logit[tok] = t_dot(&t, row, emb + tok * W, W, scratch);
        double maximum;
        size_t sum = t_shifted_exponentials(&t, logit, V, &maximum, exps);
        size_t normalized = t_shift(&t, t_log(&t, sum), maximum);
        losses[nl++] = t_subtract(&t, normalized, logit[targets[r]]);
    }
    size_t total = t_sum(&t, losses, nl);
    size_t loss_id = t_scale(&t, total, 1.0 / (double)supervised);
    int status = t.failed ? -6 : 0;
    if (!status) {
        /* reference.rs:377-390 */
        double *adj = (double *)calloc(t.n, sizeof(double));
        adj[loss_id] = 1.0;
        for (size_t id = t.n; id-- > 0;) {
            double a = adj[id];
            if (a == 0.0) continue;
            if (t.p0[id] != NONE) adj[t.p0[id]] += a * t.d0[id];
            if (t.p1[id] != NONE) adj[t.p1[id]] += a * t.d1[id];
        }
        memcpy(gradient, adj, sizeof(double) * count);
        free(adj);
        /* config.rs:490-500 */
        for (size_t gi = 0; gi < 1 + 5 * L; ++gi) {
            size_t begin, end;
            if (c->frozen && gi == 0) {
                begin = 0;
                end = og_embedding_parameter_count(c);
            } else {
                og_constrained_range(c, gi, &begin, &end);
            }
            for (size_t i = begin; i < end; ++i) gradient[offsets[gi] + i] = 0.0;
        }
        *loss = t.val[loss_id];
        if (!isfinite(*loss)) status = -5;
        for (size_t i = 0; i < count && !status; ++i)
            if (!isfinite(gradient[i])) status = -5;
    }
    tape_free(&t);
    free(offsets);
    free(scratch);
    free(emb);
    free(x);
    free(nrm);
    free(q);
    free(k);
    free(v);
    free(y);
    free(tmp);
    free(row);
    free(losses);
    free(logit);
    free(exps);
    return status;
}

/* gpu.rs:1366-1391 per parameter, all in f32, with the step's bias corrections
 * 1 - beta^t (gpu.rs:1976-1977); the frozen embedding group is skipped by the caller. */
void og_adam(float *value, float *m, float *v, const float *gradient, size_t count, float learning_rate,
             float weight_decay, float beta1, float beta2, float epsilon, float correction1, float correction2) {
    for (size_t i = 0; i < count; ++i) {
        float g = gradient[i];
        m[i] = beta1 * m[i] + (1.0f - beta1) * g;
        v[i] = beta2 * v[i] + (1.0f - beta2) * g * g;
        float mh = m[i] / correction1;
        float vh = v[i] / correction2;
        value[i] -= learning_rate * (mh / (sqrtf(vh) + epsilon) + weight_decay * value[i]);
    }
}
