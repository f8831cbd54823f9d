/*
 * TEST INFRASTRUCTURE ONLY — the CPU baseline of bench.py, not the product.
 *
 * KV-cached f32 decode of a batch of sequences on the host's cores: the same
 * forward as the f64 oracle (reference.rs:104-228, with the KV cache of the
 * device path instead of the reference's full-window recompute), written for
 * speed rather than bit-exactness: f32 throughout, the mesh weights split
 * into self and partner arrays so that each layer is two vectorisable passes
 * over the channels, exp for ELU and softmax from the C library's vector
 * forms (-ffast-math), and one OpenMP thread per sequence (sequences are
 * independent, so the threads never synchronise).  Sampling is the
 * reference's f32 sampler (og_sample, gpu.rs:2028-2049).  It supports the
 * default architecture (mesh or table embedding, parity codes, no embedding
 * normalisation or protected coordinates) with every operator switch.
 *
 * Timing covers the decode steps only: every sequence is prefilled first (one
 * row at a time through the same code, untimed) and samples its first token,
 * then each thread runs its sequences' `steps` steps, each the forward of the
 * last token and the draw of the next (out: B x (P + steps + 1) tokens, as
 * og_generate_cached with count steps + 1).  Its tokens are checked against the oracle's in
 * tests/test_oracle.py.
 */
#include "meshgpt_oracle.h"

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    const og_config *c;
    size_t W, H, hd, half, L, A, F, V;
    float *E;         /* V x W token vectors */
    float **ws, **wp; /* per mesh group: depth x W self / partner weights */
    uint32_t *depth;  /* per mesh group */
    uint32_t *stride; /* per layer index (max depth) */
    float *rope_cos, *rope_sin; /* positions x half */
    size_t positions;
} model_t;

static void mesh(const model_t *m, size_t group, float *x, float *tmp) {
    const size_t W = m->W;
    const uint32_t D = m->depth[group];
    for (uint32_t l = 0; l < D; ++l) {
        const float *ws = m->ws[group] + (size_t)l * W, *wp = m->wp[group] + (size_t)l * W;
        const size_t s = m->stride[l];
#pragma omp simd
        for (size_t ch = 0; ch < W - s; ++ch) tmp[ch] = x[ch] * ws[ch] + x[ch + s] * wp[ch];
        for (size_t ch = W - s; ch < W; ++ch) tmp[ch] = x[ch] * ws[ch] + x[ch + s - W] * wp[ch];
        if (l + 1 < D) {
#pragma omp simd
            for (size_t ch = 0; ch < W; ++ch) x[ch] = tmp[ch] >= 0.0f ? tmp[ch] : expf(tmp[ch]) - 1.0f;
        } else {
            memcpy(x, tmp, W * sizeof(float));
        }
    }
}

static void rmsnorm_groups(float *x, size_t n, size_t groups) {
    const size_t len = n / groups;
    for (size_t g = 0; g < groups; ++g) {
        float *v = x + g * len, sum = 0.0f;
#pragma omp simd reduction(+ : sum)
        for (size_t i = 0; i < len; ++i) sum += v[i] * v[i];
        const float inv = 1.0f / sqrtf(sum / (float)len + 1e-5f);
#pragma omp simd
        for (size_t i = 0; i < len; ++i) v[i] *= inv;
    }
}

static void rope(const model_t *m, float *x, size_t pos) {
    const float *cs = m->rope_cos + pos * m->half, *sn = m->rope_sin + pos * m->half;
    for (size_t h = 0; h < m->H; ++h) {
        float *v = x + h * m->hd;
        for (size_t i = 0; i < m->half; ++i) {
            const float a = v[i], b = v[i + m->half];
            v[i] = a * cs[i] - b * sn[i];
            v[i + m->half] = b * cs[i] + a * sn[i];
        }
    }
}

/* One sequence's forward of the token at `pos`, with K/V rows [0, pos) cached
 * in kc/vc ([L][H][positions][hd]); writes the row's logits. */
static void forward(const model_t *m, uint32_t tok, size_t pos, float *kc, float *vc, float *logits, float *work) {
    const og_config *c = m->c;
    const size_t W = m->W, H = m->H, hd = m->hd, P = m->positions;
    float *x = work, *n = x + W, *q = n + W, *k = q + W, *v = k + W, *y = v + W, *tmp = y + W, *sc = tmp + W;
    memcpy(x, m->E + (size_t)tok * W, W * sizeof(float));
    const float scale = 1.0f / sqrtf((float)hd);
    for (size_t l = 0; l < m->L; ++l) {
        const size_t g = 1 + 5 * l;
        memcpy(n, x, W * sizeof(float));
        rmsnorm_groups(n, W, 1);
        memcpy(q, n, W * sizeof(float));
        memcpy(k, n, W * sizeof(float));
        memcpy(v, n, W * sizeof(float));
        mesh(m, g, q, tmp);
        mesh(m, g + 1, k, tmp);
        mesh(m, g + 2, v, tmp);
        if (c->qk_norm) {
            rmsnorm_groups(q, W, H);
            rmsnorm_groups(k, W, H);
        }
        if (c->rope) {
            rope(m, q, pos);
            rope(m, k, pos);
        }
        float *kl = kc + l * H * P * hd, *vl = vc + l * H * P * hd;
        for (size_t h = 0; h < H; ++h) {
            float *kh = kl + h * P * hd, *vh = vl + h * P * hd;
            memcpy(kh + pos * hd, k + h * hd, hd * sizeof(float));
            memcpy(vh + pos * hd, v + h * hd, hd * sizeof(float));
            const float *qh = q + h * hd;
            float mx = -INFINITY;
            for (size_t t = 0; t <= pos; ++t) {
                const float *kt = kh + t * hd;
                float s = 0.0f;
#pragma omp simd reduction(+ : s)
                for (size_t i = 0; i < hd; ++i) s += qh[i] * kt[i];
                sc[t] = s * scale;
                mx = sc[t] > mx ? sc[t] : mx;
            }
            float sum = 0.0f;
#pragma omp simd reduction(+ : sum)
            for (size_t t = 0; t <= pos; ++t) {
                sc[t] = expf(sc[t] - mx);
                sum += sc[t];
            }
            float *yh = y + h * hd;
            memset(yh, 0, hd * sizeof(float));
            for (size_t t = 0; t <= pos; ++t) {
                const float p = sc[t] / sum, *vt = vh + t * hd;
#pragma omp simd
                for (size_t i = 0; i < hd; ++i) yh[i] += p * vt[i];
            }
            if (c->xsa) {
                const float *vv = v + h * hd;
                float vsq = 0.0f, yv = 0.0f;
                for (size_t i = 0; i < hd; ++i) vsq += vv[i] * vv[i];
                const float norm = sqrtf(vsq) > 1e-12f ? sqrtf(vsq) : 1e-12f;
                for (size_t i = 0; i < hd; ++i) yv += yh[i] * vv[i] / norm;
                for (size_t i = 0; i < hd; ++i) yh[i] -= yv * vv[i] / norm;
            }
        }
        mesh(m, g + 3, y, tmp);
#pragma omp simd
        for (size_t i = 0; i < W; ++i) x[i] += y[i];
        memcpy(n, x, W * sizeof(float));
        rmsnorm_groups(n, W, 1);
        mesh(m, g + 4, n, tmp);
#pragma omp simd
        for (size_t i = 0; i < W; ++i) x[i] += n[i];
    }
    rmsnorm_groups(x, W, 1);
    for (size_t t = 0; t < m->V; ++t) {
        const float *e = m->E + t * W;
        float s = 0.0f;
#pragma omp simd reduction(+ : s)
        for (size_t i = 0; i < W; ++i) s += x[i] * e[i];
        logits[t] = s;
    }
}

int cb_generate_f32(const og_config *c, const float *params, const uint32_t *prompts, size_t B, size_t P,
                    size_t steps, float temperature, uint64_t seed, int threads, uint32_t *out,
                    double *decode_seconds) {
    if (c->form != 0 || c->normalization != 0 || c->preserve_features != 0 || P == 0 || P + steps > c->context)
        return 1;
    model_t m;
    memset(&m, 0, sizeof m);
    m.c = c;
    m.W = c->width;
    m.H = c->heads;
    m.hd = m.W / m.H;
    m.half = m.hd / 2;
    m.L = c->layers;
    m.V = c->vocab_size;
    m.positions = P + steps;
    const size_t W = m.W, ngroups = 1 + 5 * m.L;
    double *E64 = malloc(sizeof(double) * m.V * W);
    if (og_token_embeddings(c, params, E64)) {
        free(E64);
        return 1;
    }
    m.E = malloc(sizeof(float) * m.V * W);
    for (size_t i = 0; i < m.V * W; ++i) m.E[i] = (float)E64[i];
    free(E64);
    size_t *offsets = malloc(sizeof(size_t) * ngroups);
    og_group_offsets(c, offsets);
    m.ws = calloc(ngroups, sizeof(float *));
    m.wp = calloc(ngroups, sizeof(float *));
    m.depth = calloc(ngroups, sizeof(uint32_t));
    uint32_t maxd = 0;
    for (size_t g = 1; g < ngroups; ++g) {
        const uint32_t d = (g - 1) % 5 == 4 ? c->ffn_mesh_depth : c->attention_mesh_depth;
        m.depth[g] = d;
        maxd = d > maxd ? d : maxd;
        m.ws[g] = malloc(sizeof(float) * d * W);
        m.wp[g] = malloc(sizeof(float) * d * W);
        for (size_t i = 0; i < d * W; ++i) {
            m.ws[g][i] = params[offsets[g] + 2 * i];
            m.wp[g][i] = params[offsets[g] + 2 * i + 1];
        }
    }
    m.stride = malloc(sizeof(uint32_t) * maxd);
    for (uint32_t l = 0; l < maxd; ++l) m.stride[l] = og_stride(c, l) % (uint32_t)W;
    m.rope_cos = malloc(sizeof(float) * m.positions * (m.half ? m.half : 1));
    m.rope_sin = malloc(sizeof(float) * m.positions * (m.half ? m.half : 1));
    for (size_t p = 0; p < m.positions; ++p)
        for (size_t i = 0; i < m.half; ++i) {
            const double angle = (double)p * pow(10000.0, -(double)i / (double)m.half);
            m.rope_cos[p * m.half + i] = (float)cos(angle);
            m.rope_sin[p * m.half + i] = (float)sin(angle);
        }
    const size_t kv = m.L * m.H * m.positions * m.hd, T = P + steps + 1;
    float *kc = malloc(sizeof(float) * kv * B), *vc = malloc(sizeof(float) * kv * B);
    float *logits = malloc(sizeof(float) * m.V * B);
    uint64_t *rng = malloc(sizeof(uint64_t) * B);
    const size_t wsize = 8 * W + m.positions;
    if (threads < 1) threads = 1;
    /* Prefill: positions 0 .. P-1 of every sequence, then the first token. */
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
    for (size_t b = 0; b < B; ++b) {
        float *work = malloc(sizeof(float) * wsize);
        memcpy(out + b * T, prompts + b * P, P * sizeof(uint32_t));
        rng[b] = seed + b;
        for (size_t p = 0; p < P; ++p)
            forward(&m, prompts[b * P + p], p, kc + b * kv, vc + b * kv, logits + b * m.V, work);
        out[b * T + P] = og_sample(logits + b * m.V, m.V, temperature, &rng[b]);
        free(work);
    }
    /* Decode step s runs the token at position P + s and samples the next. */
    const double t0 = omp_get_wtime();
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
    for (size_t b = 0; b < B; ++b) {
        float *work = malloc(sizeof(float) * wsize);
        uint32_t *seq = out + b * T;
        for (size_t s = 0; s < steps; ++s) {
            forward(&m, seq[P + s], P + s, kc + b * kv, vc + b * kv, logits + b * m.V, work);
            seq[P + s + 1] = og_sample(logits + b * m.V, m.V, temperature, &rng[b]);
        }
        free(work);
    }
    *decode_seconds = omp_get_wtime() - t0;
    for (size_t g = 1; g < ngroups; ++g) {
        free(m.ws[g]);
        free(m.wp[g]);
    }
    free(m.ws);
    free(m.wp);
    free(m.depth);
    free(m.stride);
    free(m.rope_cos);
    free(m.rope_sin);
    free(m.E);
    free(offsets);
    free(kc);
    free(vc);
    free(logits);
    free(rng);
    return 0;
}
