/*
 * TEST INFRASTRUCTURE ONLY — the CPU checker for the HIP product path.
 *
 * f64 restatement of the reference Mesh GPT forward (/root/reference/src/gpt/
 * reference.rs:104-228, 392-603), its layout/initialisation/token codes
 * (src/gpt/config.rs), SplitMix64 (src/mesh.rs:256-288), the generate loop and
 * sampler (src/gpt/gpu.rs:2006-2053) and the two datasets whose published
 * step-0 losses pin the whole model (src/gpt/text.rs:58-109,
 * src/gpt/grokking.rs:116-271).  Operation order follows the reference's tape
 * (left-fold dot products, reciprocal scaling), so the restatement and the
 * reference round alike.  Build with -ffp-contract=off: the reference's Rust
 * never contracts multiply-add pairs, and its f32 initialisation and sampler
 * are bit-exact only without contraction.
 *
 * Pinning: every function here is checked in tests/test_oracle.py against
 * the reference's KATs (reference.rs:627-998, config.rs:660-807,
 * text.rs:115-155, grokking.rs:391-393), against the two published step-0
 * cross-entropies (docs/mesh-gpt.md:269, docs/cuda-performance.md:238-240), and
 * against closed forms (norm, orthogonality, rotation identities).
 */
#include "meshgpt_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define OG_MAX_ROWS 131072u     /* src/gpt/mod.rs:31 */
#define OG_MAX_CONTEXT 4096u    /* src/gpt/mod.rs:34 */
#define OG_MAX_WIDTH 4096u      /* src/gpt/mod.rs:33 */
#define OG_MAX_HEADS 64u        /* src/gpt/mod.rs:35 */
#define OG_MAX_VOCAB 65536u     /* src/gpt/mod.rs:36 */
static const float OG_ROPE_BASE = 10000.0f;  /* src/gpt/mod.rs:37 */
static const float OG_RMS_EPS = 1e-5f;       /* src/gpt/mod.rs:38 */
static const float OG_XSA_EPS = 1e-12f;      /* src/gpt/mod.rs:40 */

/* ------------------------------------------------------------------ RNG */

/* src/mesh.rs:267-274 */
uint64_t og_rng_next(uint64_t *state) {
    *state += 0x9e3779b97f4a7c15ULL;
    uint64_t bits = *state;
    bits = (bits ^ (bits >> 30)) * 0xbf58476d1ce4e5b9ULL;
    bits = (bits ^ (bits >> 27)) * 0x94d049bb133111ebULL;
    bits ^= bits >> 31;
    return bits;
}

/* src/mesh.rs:263-265: a 24-bit integer scaled by 2^-24, exact in f32 */
float og_rng_unit(uint64_t *state) {
    uint32_t top = (uint32_t)(og_rng_next(state) >> 40);
    return (float)top / 16777216.0f;
}

/* src/mesh.rs:277-288: rejection sampling without modulo bias */
uint64_t og_rng_index(uint64_t *state, uint64_t bound) {
    uint64_t threshold = (0 - bound) % bound;
    for (;;) {
        uint64_t bits = og_rng_next(state);
        if (bits >= threshold) return bits % bound;
    }
}

/* ----------------------------------------------------- config and layout */

static void set_err(char *err, size_t len, const char *msg) {
    if (err && len) {
        strncpy(err, msg, len - 1);
        err[len - 1] = 0;
    }
}

/* ------------------------------------------------------------ geometry */

static uint32_t bit_len(uint64_t x) {
    uint32_t n = 0;
    while (x) {
        x >>= 1;
        ++n;
    }
    return n;
}

static const char *const form_names[10] = {"parity",  "circle",    "fourier",   "orthogonal",
                                           "simplex", "equiangular", "antipodal", "hypercube",
                                           "signed-permutations", "sphere"};

/* src/gpt/geometry.rs:84-151 (the "does not fit" message prints the overlap
 * with Rust's shortest round-trip Display) */
static int validate_geometry(const og_config *c, char *err, size_t err_len) {
    uint32_t v = c->vocab_size, w = c->width;
    if (c->form > 9 || c->order > 2 || c->normalization > 2 || c->frozen > 1 || c->rope > 1 || c->qk_norm > 1 ||
        c->xsa > 1) {
        set_err(err, err_len, "unknown geometry code");
        return -1;
    }
    if (c->frequency == 0 || c->harmonics == 0 || c->harmonics > w / 2) {
        set_err(err, err_len, "embedding frequency must be positive and harmonics in 1..width/2");
        return -1;
    }
    if (!isfinite(c->overlap) || c->preserve_features > w) {
        set_err(err, err_len, "embedding overlap must be finite; preserved features must fit width");
        return -1;
    }
    if (c->preserve_features > 0 && c->normalization != 0) {
        set_err(err, err_len,
                "preserved coordinates require --embedding-norm none; full-vector normalization would rescale "
                "the protected feature");
        return -1;
    }
    int fits = 1;
    if (c->form == 3) fits = w >= v;
    if (c->form == 4) fits = w + 1 >= v;
    if (c->form == 5) {
        float lower = -1.0f / (float)(v - 1);
        fits = c->overlap >= lower && c->overlap <= 1.0f &&
               (c->overlap == 1.0f || w + (c->overlap == lower ? 1u : 0u) >= v);
    }
    if (c->form == 7) fits = w >= bit_len(v - 1);
    if (c->form == 8) fits = w >= 4 && v <= 256;
    if (!fits) {
        char buf[160];
        /* shortest decimal of the f32 overlap that reads back exactly, no exponent */
        char num[64];
        for (int prec = 0; prec < 60; ++prec) {
            snprintf(num, sizeof num, "%.*f", prec, (double)c->overlap);
            if ((float)strtod(num, NULL) == c->overlap) break;
        }
        snprintf(buf, sizeof buf, "%s embedding does not fit vocabulary %u, width %u, overlap %s",
                 form_names[c->form], v, w, num);
        set_err(err, err_len, buf);
        return -1;
    }
    if (c->order != 0) {
        int prime = c->modulus >= 2;
        for (uint32_t d = 2; d < c->modulus; ++d)
            if (c->modulus % d == 0) prime = 0;
        if (c->modulus < 2 || c->modulus > 254 || !prime || v != c->modulus + 2) {
            set_err(err, err_len, "arithmetic embedding order requires a grok prime and vocabulary modulus+2");
            return -1;
        }
        uint32_t special = 2 + (c->order == 2 ? 1 : 0);
        uint32_t pairs = c->form == 2 ? c->harmonics : 1;
        if ((c->form == 1 || c->form == 2) && w < 2 * pairs + special) {
            set_err(err, err_len, "arithmetic circle/Fourier codes need extra coordinates for special symbols");
            return -1;
        }
    }
    return 0;
}

/* src/gpt/grokking.rs:260-271: a Fisher-Yates shuffle of 0..modulus from the
 * tail, with Random::new(seed ^ "symbols\x01") */
void og_residue_permutation(uint32_t modulus, uint64_t seed, uint32_t *out) {
    for (uint32_t i = 0; i < modulus; ++i) out[i] = i;
    uint64_t state = seed ^ 0x73796d626f6c7301ULL;
    for (uint32_t end = modulus; end-- > 1;) {
        uint32_t j = (uint32_t)og_rng_index(&state, (uint64_t)end + 1);
        uint32_t t = out[end];
        out[end] = out[j];
        out[j] = t;
    }
}

/* src/gpt/geometry.rs:166-184 */
uint32_t og_primitive_root(uint32_t prime) {
    if (prime == 2) return 1;
    unsigned char *seen = (unsigned char *)malloc(prime);
    for (uint32_t g = 2; g < prime; ++g) {
        memset(seen, 0, prime);
        uint64_t x = 1;
        int ok = 1;
        for (uint32_t k = 0; k + 1 < prime; ++k) {
            if (seen[x]) {
                ok = 0;
                break;
            }
            seen[x] = 1;
            x = x * g % prime;
        }
        if (ok && x == 1) {
            free(seen);
            return g;
        }
    }
    free(seen);
    return 0;
}

/* src/gpt/geometry.rs:186-211: token at each position and the cycle length */
static size_t ordered_tokens(const og_config *c, uint32_t *order) {
    uint32_t V = c->vocab_size;
    if (c->order == 0) {
        for (uint32_t t = 0; t < V; ++t) order[t] = t;
        return V;
    }
    uint32_t p = c->modulus;
    uint32_t *ids = (uint32_t *)malloc(sizeof(uint32_t) * p);
    og_residue_permutation(p, c->seed, ids);
    size_t n = 0;
    if (c->order == 1) {
        for (uint32_t i = 0; i < p; ++i) order[n++] = ids[i];
    } else {
        uint32_t root = og_primitive_root(p);
        uint64_t residue = 1;
        for (uint32_t k = 0; k + 1 < p; ++k) {
            order[n++] = ids[residue];
            residue = residue * root % p;
        }
    }
    size_t cycle = n;
    if (c->order == 2) order[n++] = ids[0];
    order[n++] = p;
    order[n++] = p + 1;
    free(ids);
    return cycle;
}

static double helmert(size_t row, size_t column, size_t n) {
    double scale = sqrt((double)n / (double)(n - 1));
    double den = sqrt((double)((column + 1) * (column + 2)));
    if (row <= column) return scale / den;
    if (row == column + 1) return -scale * (double)(column + 1) / den;
    return 0.0;
}

/* src/gpt/geometry.rs:238-325 for the non-parity forms */
static void geometric_codes(const og_config *c, float *out) {
    size_t V = c->vocab_size, W = c->width;
    uint32_t *order = (uint32_t *)malloc(sizeof(uint32_t) * V);
    size_t cycle = ordered_tokens(c, order);
    memset(out, 0, sizeof(float) * V * W);
    uint64_t rng = c->seed ^ 0x5350484552453031ULL;
    const double tau = 6.283185307179586;
    for (size_t row = 0; row < V; ++row) {
        float *code = out + (size_t)order[row] * W;
        switch (c->form) {
        case 1:
        case 2: {
            size_t pairs = c->form == 2 ? c->harmonics : 1;
            if (row >= cycle) {
                code[2 * pairs + row - cycle] = 1.0f;
                break;
            }
            double scale = 1.0 / sqrt((double)pairs);
            for (size_t k = 0; k < pairs; ++k) {
                size_t f = ((size_t)c->frequency % cycle + k % cycle) % cycle;
                double angle = tau * (double)f * (double)row / (double)cycle;
                code[2 * k] = (float)(scale * cos(angle));
                code[2 * k + 1] = (float)(scale * sin(angle));
            }
            break;
        }
        case 3: code[row] = 1.0f; break;
        case 4:
        case 5: {
            double rho = c->form == 4 ? -1.0 / (double)(V - 1) : (double)c->overlap;
            if (rho == 1.0) {
                code[0] = 1.0f;
                break;
            }
            double a = sqrt((1.0 - rho) * (double)(V - 1) / (double)V);
            for (size_t col = 0; col + 1 < V; ++col) code[col] = (float)(a * helmert(row, col, V));
            if (W >= V) {
                double t = 1.0 + (double)(V - 1) * rho;
                code[V - 1] = (float)sqrt((t > 0.0 ? t : 0.0) / (double)V);
            }
            break;
        }
        case 6: code[0] = row % 2 == 0 ? 1.0f : -1.0f; break;
        case 7: {
            uint32_t bits = bit_len(V - 1);
            for (uint32_t b = 0; b < bits; ++b)
                code[b] = ((row >> b) & 1 ? 1.0f : -1.0f) / sqrtf((float)bits);
            break;
        }
        case 8: {
            size_t p = row / 16;
            for (size_t col = 0; col < 4; ++col) {
                size_t slot = col < 2 ? (col + (p / 2) % 2) % 2 : 2 + (col - 2 + p % 2) % 2;
                float magnitude = (float)(1 + (slot + p / 4) % 4);
                code[col] = magnitude * ((row >> col) & 1 ? -1.0f : 1.0f);
            }
            break;
        }
        case 9: {
            double squares = 0.0;
            for (size_t col = 0; col < W; ++col) {
                float u = og_rng_unit(&rng);
                if (u < 1.0f / 16777216.0f) u = 1.0f / 16777216.0f;
                double radius = sqrt(-2.0 * log((double)u));
                double angle = tau * (double)og_rng_unit(&rng);
                code[col] = (float)(radius * cos(angle));
                squares += (double)code[col] * (double)code[col];
            }
            for (size_t col = 0; col < W; ++col) code[col] = (float)((double)code[col] / sqrt(squares));
            break;
        }
        default: break;
        }
    }
    free(order);
}

/* src/gpt/config.rs:461-474: the final-layer rows of every projection and FFN
 * mesh that write protected residual coordinates, as [begin, end) offsets */
void og_constrained_range(const og_config *c, size_t group, size_t *begin, size_t *end) {
    *begin = *end = 0;
    if (c->preserve_features == 0 || group == 0) return;
    size_t kind = (group - 1) % 5;
    if (kind != 3 && kind != 4) return;
    size_t depth = kind == 4 ? c->ffn_mesh_depth : c->attention_mesh_depth;
    *begin = (depth - 1) * 2 * (size_t)c->width;
    *end = *begin + 2 * (size_t)c->preserve_features;
}

/* src/gpt/config.rs:144-172 */
int og_validate(const og_config *c, int allow_long_context, char *err, size_t err_len) {
    if (c->vocab_size < 2 || c->vocab_size > OG_MAX_VOCAB) {
        set_err(err, err_len, "vocab_size must be in 2..65536");
        return -1;
    }
    if (c->context < 1 || (!allow_long_context && c->context > OG_MAX_CONTEXT)) {
        set_err(err, err_len, "context must be in 1..4096");
        return -1;
    }
    if (c->width < 2 || c->width > OG_MAX_WIDTH) {
        set_err(err, err_len, "width must be in 2..4096");
        return -1;
    }
    if (c->heads < 1 || c->heads > OG_MAX_HEADS || c->width % c->heads != 0) {
        set_err(err, err_len, "heads must be in 1..64 and divide width");
        return -1;
    }
    if (c->width / c->heads < 2) {
        set_err(err, err_len, "each attention head requires at least two channels");
        return -1;
    }
    if (c->rope && (c->width / c->heads) % 2 != 0) {
        set_err(err, err_len, "slice RoPE requires an even number of channels per head");
        return -1;
    }
    if (c->layers < 1 || c->layers > 64) {
        set_err(err, err_len, "layers must be in 1..64");
        return -1;
    }
    if (c->attention_mesh_depth < 1 || c->attention_mesh_depth > 256 || c->ffn_mesh_depth < 1 ||
        c->ffn_mesh_depth > 256) {
        set_err(err, err_len, "mesh depths must be in 1..256");
        return -1;
    }
    if (c->embedding > 1 || c->connectivity > 1) {
        set_err(err, err_len, "unknown embedding or connectivity code");
        return -1;
    }
    return validate_geometry(c, err, err_len);
}

/* src/gpt/config.rs:179-184 */
size_t og_embedding_parameter_count(const og_config *c) {
    return c->embedding == 0 ? (size_t)2 * c->width * c->attention_mesh_depth
                             : (size_t)c->vocab_size * c->width;
}

/* src/gpt/config.rs:358-398: embedding group, then per block q, k, v, proj, ffn */
void og_group_offsets(const og_config *c, size_t *offsets) {
    size_t at = og_embedding_parameter_count(c);
    size_t mesh = (size_t)2 * c->width * c->attention_mesh_depth;
    size_t ffn = (size_t)2 * c->width * c->ffn_mesh_depth;
    offsets[0] = 0;
    for (uint32_t b = 0; b < c->layers; ++b) {
        for (int g = 0; g < 4; ++g) {
            offsets[1 + 5 * b + g] = at;
            at += mesh;
        }
        offsets[1 + 5 * b + 4] = at;
        at += ffn;
    }
}

size_t og_parameter_count(const og_config *c) {
    return og_embedding_parameter_count(c) +
           (size_t)c->layers * 2 * c->width * (4 * (size_t)c->attention_mesh_depth + c->ffn_mesh_depth);
}

static uint32_t ilog2_u32(uint32_t x) {
    uint32_t r = 0;
    while (x >>= 1) ++r;
    return r;
}

/* src/gpt/config.rs:117-122 */
uint32_t og_stride(const og_config *c, uint32_t layer) {
    if (c->connectivity == 0) return 1;
    return 1u << (layer % ilog2_u32(c->width));
}

static uint32_t popcount_u64(uint64_t x) {
    uint32_t n = 0;
    while (x) {
        x &= x - 1;
        ++n;
    }
    return n;
}

static int is_pow2(uint64_t x) { return x && !(x & (x - 1)); }

/* src/gpt/config.rs:552-591 with the default Parity form and Token order
 * (reorder_parity is the identity then, geometry.rs:213-216) */
void og_token_codes(const og_config *c, float *out) {
    if (c->form != 0) {
        geometric_codes(c, out);
        return;
    }
    uint32_t V = c->vocab_size, W = c->width;
    uint32_t bits = 32 - (uint32_t)__builtin_clz(V - 1);
    uint32_t lanes = W < bits ? W : bits;
    size_t nmasks = 0;
    uint64_t *masks = (uint64_t *)malloc(sizeof(uint64_t) * ((size_t)1 << bits));
    for (uint32_t b = 0; b < bits; ++b) masks[nmasks++] = (uint64_t)1 << b;
    for (uint64_t m = 1; m < ((uint64_t)1 << bits); ++m)
        if (!is_pow2(m)) masks[nmasks++] = m;
    for (uint32_t t = 0; t < V; ++t) {
        for (uint32_t ch = 0; ch < W; ++ch) {
            float value;
            if (W >= bits) {
                value = (popcount_u64((uint64_t)t & masks[ch % nmasks]) % 2 == 0) ? -1.0f : 1.0f;
            } else {
                uint64_t digit = 0, maximum = 0;
                for (uint32_t b = ch % lanes; b < bits; b += lanes) {
                    digit = 2 * digit + ((t >> b) & 1u);
                    maximum = 2 * maximum + 1;
                }
                value = 2.0f * (float)digit / (float)maximum - 1.0f;
            }
            out[(size_t)t * W + ch] = value;
        }
    }
    free(masks);
    if (c->order != 0) {
        /* geometry.rs:213-222: the code of position i belongs to token order[i] */
        uint32_t *order = (uint32_t *)malloc(sizeof(uint32_t) * V);
        ordered_tokens(c, order);
        float *copy = (float *)malloc(sizeof(float) * (size_t)V * W);
        memcpy(copy, out, sizeof(float) * (size_t)V * W);
        for (uint32_t i = 0; i < V; ++i) memcpy(out + (size_t)order[i] * W, copy + (size_t)i * W, sizeof(float) * W);
        free(copy);
        free(order);
    }
}

/* src/gpt/config.rs:436-458: SplitMix64 draws in f32, final layer scaled by 0.3 */
static void initialize_mesh_model(const og_config *c, uint64_t seed, float *out) {
    uint64_t state = seed;
    size_t ngroups = 1 + 5 * (size_t)c->layers;
    size_t *offsets = (size_t *)malloc(sizeof(size_t) * ngroups);
    og_group_offsets(c, offsets);
    for (size_t g = 0; g < ngroups; ++g) {
        uint32_t depth = (g == 0 || (g - 1) % 5 != 4) ? c->attention_mesh_depth : c->ffn_mesh_depth;
        float *values = out + offsets[g];
        for (uint32_t layer = 0; layer < depth; ++layer) {
            for (uint32_t ch = 0; ch < c->width; ++ch) {
                size_t o = (size_t)layer * 2 * c->width + (size_t)ch * 2;
                float u0 = og_rng_unit(&state);
                float a = 0.2f * (u0 - 0.5f);
                values[o] = 0.7f + a;
                float u1 = og_rng_unit(&state);
                values[o + 1] = 0.4f * (u1 - 0.5f);
                if (layer + 1 == depth) {
                    values[o] *= 0.3f;
                    values[o + 1] *= 0.3f;
                }
            }
        }
    }
    for (size_t g = 0; g < ngroups; ++g) {
        size_t begin, end;
        og_constrained_range(c, g, &begin, &end);
        for (size_t i = begin; i < end; ++i) out[offsets[g] + i] = 0.0f;
    }
    free(offsets);
}

static void mesh_rows(double *x, double *tmp, size_t rows, size_t width, const float *params,
                      size_t depth, uint32_t connectivity);

/* table initialisation: tabulate the seeded mesh model (config.rs:416-435,515-547) */
void og_initialize(const og_config *c, uint64_t seed, float *out) {
    if (c->embedding == 0) {
        initialize_mesh_model(c, seed, out);
        return;
    }
    og_config mesh = *c;
    mesh.embedding = 0;
    size_t count = og_parameter_count(&mesh);
    float *init = (float *)malloc(sizeof(float) * count);
    initialize_mesh_model(&mesh, seed, init);
    size_t V = c->vocab_size, W = c->width;
    float *codes = (float *)malloc(sizeof(float) * V * W);
    og_token_codes(c, codes);
    double *vec = (double *)malloc(sizeof(double) * V * W);
    double *tmp = (double *)malloc(sizeof(double) * V * W);
    for (size_t i = 0; i < V * W; ++i) vec[i] = (double)codes[i];
    mesh_rows(vec, tmp, V, W, init, c->attention_mesh_depth, c->connectivity);
    for (size_t i = 0; i < V * W; ++i) out[i] = c->form != 0 ? codes[i] : (float)vec[i];
    size_t emb = og_embedding_parameter_count(&mesh);
    memcpy(out + V * W, init + emb, sizeof(float) * (count - emb));
    free(init);
    free(codes);
    free(vec);
    free(tmp);
}

/* N(0, sigma^2) weights (BASELINE.json's synthetic workloads; config.rs has
 * no such initialiser): parameter i in flat order is sigma times the
 * reference's Box-Muller draw (src/simple/numerical.rs:163-167), u1 and u2
 * two unit() draws of Random::new(seed), sqrt(-2 ln(1 - u1)) cos(tau u2) in
 * f64 rounded to f32, times sigma in f32; protected rows are zeroed as in
 * og_initialize. */
void og_initialize_normal(const og_config *c, uint64_t seed, float sigma, float *out) {
    uint64_t state = seed;
    size_t n = og_parameter_count(c);
    for (size_t i = 0; i < n; ++i) {
        double u1 = (double)og_rng_unit(&state), u2 = (double)og_rng_unit(&state);
        double radius = sqrt(-2.0 * log(1.0 - u1));
        out[i] = (float)(radius * cos(6.283185307179586 * u2)) * sigma;
    }
    size_t ngroups = 1 + 5 * (size_t)c->layers;
    size_t *offsets = (size_t *)malloc(sizeof(size_t) * ngroups);
    og_group_offsets(c, offsets);
    for (size_t g = 0; g < ngroups; ++g) {
        size_t begin, end;
        og_constrained_range(c, g, &begin, &end);
        for (size_t i = begin; i < end; ++i) out[offsets[g] + i] = 0.0f;
    }
    free(offsets);
}

/* ------------------------------------------------------------ operators */

/* Tape::dot: products first, then a left fold starting at the first product
 * (reference.rs:333-347) */
static double dot(const double *a, const double *b, size_t n) {
    double total = a[0] * b[0];
    for (size_t i = 1; i < n; ++i) total = total + a[i] * b[i];
    return total;
}

/* reference.rs:392-409 */
void og_rmsnorm(const double *in, size_t width, size_t heads, double *out) {
    size_t hw = width / heads;
    for (size_t h = 0; h < heads; ++h) {
        const double *x = in + h * hw;
        double sum = dot(x, x, hw);
        double mean_square = sum * (1.0 / (double)hw);
        double stabilized = mean_square + (double)OG_RMS_EPS;
        double inverse = 1.0 / sqrt(stabilized);
        for (size_t i = 0; i < hw; ++i) out[h * hw + i] = x[i] * inverse;
    }
}

static double elu(double x) { return x >= 0.0 ? x * 1.0 : expm1(x); } /* reference.rs:325-332 */

/* reference.rs:422-453 over rows stored contiguously; x is updated in place */
static void mesh_rows(double *x, double *tmp, size_t rows, size_t width, const float *params,
                      size_t depth, uint32_t connectivity) {
    og_config shape = {0};
    shape.width = (uint32_t)width;
    shape.connectivity = connectivity;
    for (size_t layer = 0; layer < depth; ++layer) {
        uint32_t stride = og_stride(&shape, (uint32_t)layer);
        const float *w = params + layer * 2 * width;
        for (size_t r = 0; r < rows; ++r) {
            const double *row = x + r * width;
            double *o = tmp + r * width;
            for (size_t ch = 0; ch < width; ++ch) {
                double left = row[ch] * (double)w[2 * ch];
                double right = row[(ch + stride) % width] * (double)w[2 * ch + 1];
                double sum = left + right;
                o[ch] = (layer + 1 == depth) ? sum : elu(sum);
            }
        }
        memcpy(x, tmp, sizeof(double) * rows * width);
    }
}

void og_mesh(const double *in, size_t rows, size_t width, const float *params, size_t depth,
             uint32_t connectivity, double *out) {
    double *tmp = (double *)malloc(sizeof(double) * rows * width);
    memcpy(out, in, sizeof(double) * rows * width);
    mesh_rows(out, tmp, rows, width, params, depth, connectivity);
    free(tmp);
}

/* reference.rs:462-482 */
static void rotary_row(const double *in, size_t width, size_t heads, size_t position, double *out) {
    size_t hw = width / heads, half = hw / 2;
    memcpy(out, in, sizeof(double) * width);
    for (size_t h = 0; h < heads; ++h) {
        for (size_t pair = 0; pair < half; ++pair) {
            double angle = (double)position / pow((double)OG_ROPE_BASE, (double)pair / (double)half);
            double sine = sin(angle), cosine = cos(angle);
            size_t l = h * hw + pair, r = l + half;
            out[l] = in[l] * cosine - in[r] * sine;
            out[r] = in[r] * cosine + in[l] * sine;
        }
    }
}

void og_rotary(const double *in, size_t width, size_t heads, size_t position, double *out) {
    rotary_row(in, width, heads, position, out);
}

/* reference.rs:510-554 for one query row of a sequence whose rows start at k/v */
static void attention_row(const double *query, const double *k, const double *v, size_t position,
                          size_t width, size_t heads, double *scores, double *out) {
    size_t hw = width / heads;
    double scale = 1.0 / sqrt((double)hw);
    for (size_t h = 0; h < heads; ++h) {
        size_t b = h * hw;
        double maximum = -INFINITY;
        for (size_t j = 0; j <= position; ++j) {
            scores[j] = dot(query + b, k + j * width + b, hw) * scale;
            if (scores[j] > maximum) maximum = scores[j];
        }
        double sum = 0.0;
        for (size_t j = 0; j <= position; ++j) {
            scores[j] = exp(scores[j] + -maximum);
            sum = j == 0 ? scores[0] : sum + scores[j];
        }
        double reciprocal = 1.0 / sum;
        for (size_t j = 0; j <= position; ++j) scores[j] = scores[j] * reciprocal;
        /* Each channel's total is the left fold over j in order; the loops run
         * j outermost so that the value rows are read contiguously (the same
         * operations, in the same order, per channel). */
        for (size_t ch = b; ch < b + hw; ++ch) out[ch] = scores[0] * v[ch];
        for (size_t j = 1; j <= position; ++j) {
            const double s = scores[j], *vj = v + j * width;
            for (size_t ch = b; ch < b + hw; ++ch) out[ch] = out[ch] + s * vj[ch];
        }
    }
}

void og_attention(const double *q, const double *k, const double *v, size_t rows, size_t width,
                  size_t heads, size_t sequence, double *out) {
    double *scores = (double *)malloc(sizeof(double) * sequence);
    for (size_t r = 0; r < rows; ++r) {
        size_t position = r % sequence, first = r - position;
        attention_row(q + r * width, k + first * width, v + first * width, position, width, heads,
                      scores, out + r * width);
    }
    free(scores);
}

/* reference.rs:577-603 */
void og_exclusive(const double *y, const double *v, size_t width, size_t heads, double *out) {
    size_t hw = width / heads;
    double floor2 = (double)OG_XSA_EPS * (double)OG_XSA_EPS;
    double *u = (double *)malloc(sizeof(double) * hw);
    for (size_t h = 0; h < heads; ++h) {
        const double *yh = y + h * hw, *vh = v + h * hw;
        double squared = dot(vh, vh, hw);
        double floored = squared >= floor2 ? squared : floor2;
        double inverse = 1.0 / sqrt(floored);
        for (size_t i = 0; i < hw; ++i) u[i] = vh[i] * inverse;
        double projection = dot(yh, u, hw);
        for (size_t i = 0; i < hw; ++i) out[h * hw + i] = yh[i] - projection * u[i];
    }
    free(u);
}

/* ------------------------------------------------------------ the model */

static int check_tokens(const og_config *c, const uint32_t *tokens, size_t n, size_t sequence) {
    /* src/gpt/config.rs:210-228 */
    if (sequence == 0 || sequence > c->context || n == 0 || n % sequence != 0 || n > OG_MAX_ROWS)
        return -1;
    for (size_t i = 0; i < n; ++i)
        if (tokens[i] >= c->vocab_size) return -2;
    return 0;
}

/* reference.rs:104-152: the mesh of the codes or the table, then the
 * geometry's normalisation (rows scaled to the radius) or protected codes */
int og_token_embeddings(const og_config *c, const float *params, double *out) {
    size_t V = c->vocab_size, W = c->width;
    float *codes = (float *)malloc(sizeof(float) * V * W);
    og_token_codes(c, codes);
    if (c->embedding == 1) {
        for (size_t i = 0; i < V * W; ++i) out[i] = (double)params[i];
    } else {
        double *tmp = (double *)malloc(sizeof(double) * V * W);
        for (size_t i = 0; i < V * W; ++i) out[i] = (double)codes[i];
        mesh_rows(out, tmp, V, W, params, c->attention_mesh_depth, c->connectivity);
        free(tmp);
    }
    if (c->normalization != 0) {
        /* EmbeddingGeometry::radius (geometry.rs:157-162) in f32, then f64 */
        double scale = c->normalization == 2 ? (double)sqrtf((float)W) : 1.0;
        double floor = (double)1e-12f * (double)1e-12f;
        for (size_t t = 0; t < V; ++t) {
            double *row = out + t * W;
            double squares = dot(row, row, W);
            double inverse = 1.0 / sqrt(squares > floor ? squares : floor) * scale;
            for (size_t i = 0; i < W; ++i) row[i] = row[i] * inverse;
        }
    }
    for (size_t t = 0; t < V; ++t)
        for (size_t i = 0; i < c->preserve_features; ++i) out[t * W + i] = (double)codes[t * W + i];
    free(codes);
    return 0;
}

/* One pass of reference.rs:154-228 over n rows.  With cache_k/cache_v set, the
 * rows are positions [first_position, first_position+n) of one sequence whose
 * earlier keys/values are already cached (layer-major, context x W each); the
 * result is identical to recomputing the whole prefix because every row's
 * arithmetic depends only on its own inputs and the cached rows. */
static void forward(const og_config *c, const float *params, const double *E, const uint32_t *tokens,
                    size_t n, size_t sequence, double *logits, double *hidden, double *cache_k,
                    double *cache_v, size_t first_position, size_t logit_rows_from) {
    size_t W = c->width, H = c->heads, V = c->vocab_size, L = c->layers;
    size_t A = c->attention_mesh_depth, F = c->ffn_mesh_depth;
    size_t *offsets = (size_t *)malloc(sizeof(size_t) * (1 + 5 * L));
    og_group_offsets(c, offsets);
    size_t rw = n * W;
    double *x = (double *)malloc(sizeof(double) * rw);
    double *nrm = (double *)malloc(sizeof(double) * rw);
    double *q = (double *)malloc(sizeof(double) * rw);
    double *k = (double *)malloc(sizeof(double) * rw);
    double *v = (double *)malloc(sizeof(double) * rw);
    double *t1 = (double *)malloc(sizeof(double) * rw);
    double *t2 = (double *)malloc(sizeof(double) * rw);
    size_t span = cache_k ? c->context : sequence;
    double *scores = (double *)malloc(sizeof(double) * (span + 1));
    double *row = (double *)malloc(sizeof(double) * W);
    for (size_t r = 0; r < n; ++r) memcpy(x + r * W, E + (size_t)tokens[r] * W, sizeof(double) * W);
    for (size_t b = 0; b < L; ++b) {
        const size_t *g = offsets + 1 + 5 * b;
        for (size_t r = 0; r < n; ++r) og_rmsnorm(x + r * W, W, 1, nrm + r * W);
        memcpy(q, nrm, sizeof(double) * rw);
        mesh_rows(q, t1, n, W, params + g[0], A, c->connectivity);
        memcpy(k, nrm, sizeof(double) * rw);
        mesh_rows(k, t1, n, W, params + g[1], A, c->connectivity);
        memcpy(v, nrm, sizeof(double) * rw);
        mesh_rows(v, t1, n, W, params + g[2], A, c->connectivity);
        for (size_t r = 0; r < n; ++r) {
            /* reference.rs:174-193: QK-Norm, then RoPE, each when switched on */
            size_t position = cache_k ? first_position + r : r % sequence;
            double *qk[2] = {q + r * W, k + r * W};
            for (int m = 0; m < 2; ++m) {
                if (c->qk_norm) {
                    og_rmsnorm(qk[m], W, H, row);
                    memcpy(qk[m], row, sizeof(double) * W);
                }
                if (c->rope) {
                    memcpy(row, qk[m], sizeof(double) * W);
                    rotary_row(row, W, H, position, qk[m]);
                }
            }
        }
        if (cache_k) {
            double *ck = cache_k + b * c->context * W, *cv = cache_v + b * c->context * W;
            memcpy(ck + first_position * W, k, sizeof(double) * rw);
            memcpy(cv + first_position * W, v, sizeof(double) * rw);
            for (size_t r = 0; r < n; ++r)
                attention_row(q + r * W, ck, cv, first_position + r, W, H, scores, t1 + r * W);
        } else {
            og_attention(q, k, v, n, W, H, sequence, t1);
        }
        for (size_t r = 0; r < n; ++r) {
            if (c->xsa)
                og_exclusive(t1 + r * W, v + r * W, W, H, t2 + r * W);
            else
                memcpy(t2 + r * W, t1 + r * W, sizeof(double) * W);
        }
        mesh_rows(t2, t1, n, W, params + g[3], A, c->connectivity);
        for (size_t i = 0; i < rw; ++i) x[i] = x[i] + t2[i];
        for (size_t r = 0; r < n; ++r) og_rmsnorm(x + r * W, W, 1, nrm + r * W);
        mesh_rows(nrm, t1, n, W, params + g[4], F, c->connectivity);
        for (size_t i = 0; i < rw; ++i) x[i] = x[i] + nrm[i];
    }
    if (hidden) memcpy(hidden, x, sizeof(double) * rw);
    if (logits) {
        for (size_t r = logit_rows_from; r < n; ++r) {
            og_rmsnorm(x + r * W, W, 1, row);
            for (size_t t = 0; t < V; ++t)
                logits[(r - logit_rows_from) * V + t] = dot(row, E + t * W, W);
        }
    }
    free(offsets);
    free(x);
    free(nrm);
    free(q);
    free(k);
    free(v);
    free(t1);
    free(t2);
    free(scores);
    free(row);
}

int og_logits(const og_config *c, const float *params, const uint32_t *tokens, size_t n,
              size_t sequence, double *out) {
    if (check_tokens(c, tokens, n, sequence)) return -1;
    double *E = (double *)malloc(sizeof(double) * c->vocab_size * c->width);
    og_token_embeddings(c, params, E);
    forward(c, params, E, tokens, n, sequence, out, NULL, NULL, NULL, 0, 0);
    free(E);
    return 0;
}

int og_hidden_states(const og_config *c, const float *params, const uint32_t *tokens, size_t n,
                     size_t sequence, double *out) {
    if (check_tokens(c, tokens, n, sequence)) return -1;
    double *E = (double *)malloc(sizeof(double) * c->vocab_size * c->width);
    og_token_embeddings(c, params, E);
    forward(c, params, E, tokens, n, sequence, NULL, out, NULL, NULL, 0, 0);
    free(E);
    return 0;
}

/* the f32 loss kernel gpu.rs:949-994 on f32-cast logits, mean in f64 (gpu.rs:2296-2313) */
int og_cross_entropy(const og_config *c, const float *params, const uint32_t *inputs,
                     const uint32_t *targets, size_t n, size_t sequence, double *loss) {
    size_t V = c->vocab_size;
    double *logits = (double *)malloc(sizeof(double) * n * V);
    if (og_logits(c, params, inputs, n, sequence, logits)) {
        free(logits);
        return -1;
    }
    double total = 0.0;
    size_t supervised = 0;
    for (size_t r = 0; r < n; ++r) {
        if (targets[r] == UINT32_MAX) continue;
        const double *row = logits + r * V;
        float maximum = -INFINITY;
        for (size_t t = 0; t < V; ++t)
            if ((float)row[t] > maximum) maximum = (float)row[t];
        float sum = 0.0f;
        for (size_t t = 0; t < V; ++t) sum += expf((float)row[t] - maximum);
        float value = logf(sum) + maximum - (float)row[targets[r]];
        total += (double)value;
        ++supervised;
    }
    free(logits);
    if (!supervised) return -1;
    *loss = total / (double)supervised;
    return 0;
}

/* ------------------------------------------------------------- generate */

/* gpu.rs:2028-2049: f32 maximum, first arg-max when greedy, else f32 exponentials,
 * a sequential f32 sum and a linear scan that defaults to the last token */
uint32_t og_sample(const float *logits, size_t vocab, float temperature, uint64_t *rng) {
    float maximum = -INFINITY;
    for (size_t t = 0; t < vocab; ++t)
        if (logits[t] > maximum) maximum = logits[t];
    if (temperature == 0.0f) {
        for (size_t t = 0; t < vocab; ++t)
            if (logits[t] == maximum) return (uint32_t)t;
        return 0;
    }
    float *p = (float *)malloc(sizeof(float) * vocab);
    float sum = 0.0f;
    for (size_t t = 0; t < vocab; ++t) {
        float shifted = logits[t] - maximum;
        p[t] = expf(shifted / temperature);
    }
    for (size_t t = 0; t < vocab; ++t) sum = sum + p[t];
    float u = og_rng_unit(rng);
    float sample = u * sum;
    uint32_t selected = (uint32_t)(vocab - 1);
    for (size_t t = 0; t < vocab; ++t) {
        sample = sample - p[t];
        if (sample < 0.0f) {
            selected = (uint32_t)t;
            break;
        }
    }
    free(p);
    return selected;
}

static int check_generate(const og_config *c, size_t P, float temperature) {
    if (!isfinite(temperature) || temperature < 0.0f) return -1;
    if (P == 0) return -1;
    return 0;
}

/* gpu.rs:2006-2053: every step recomputes the sliding window */
int og_generate(const og_config *c, const float *params, const uint32_t *prompt, size_t P,
                size_t count, float temperature, uint64_t seed, uint32_t *out) {
    if (check_generate(c, P, temperature)) return -1;
    for (size_t i = 0; i < P; ++i)
        if (prompt[i] >= c->vocab_size) return -1;
    size_t V = c->vocab_size;
    double *E = (double *)malloc(sizeof(double) * V * c->width);
    og_token_embeddings(c, params, E);
    double *logits = (double *)malloc(sizeof(double) * V);
    float *last = (float *)malloc(sizeof(float) * V);
    memcpy(out, prompt, sizeof(uint32_t) * P);
    uint64_t rng = seed;
    size_t len = P;
    for (size_t step = 0; step < count; ++step) {
        size_t start = len > c->context ? len - c->context : 0;
        size_t window = len - start;
        forward(c, params, E, out + start, window, window, logits, NULL, NULL, NULL, 0, window - 1);
        for (size_t t = 0; t < V; ++t) last[t] = (float)logits[t];
        out[len++] = og_sample(last, V, temperature, &rng);
    }
    free(E);
    free(logits);
    free(last);
    return 0;
}

int og_generate_cached(const og_config *c, const float *params, const uint32_t *prompt, size_t P,
                       size_t count, float temperature, uint64_t seed, uint32_t *out,
                       float *last_logits) {
    if (check_generate(c, P, temperature)) return -1;
    if (P + count > c->context) return -1;
    for (size_t i = 0; i < P; ++i)
        if (prompt[i] >= c->vocab_size) return -1;
    size_t V = c->vocab_size, W = c->width;
    double *E = (double *)malloc(sizeof(double) * V * W);
    og_token_embeddings(c, params, E);
    size_t cache = (size_t)c->layers * c->context * W;
    double *ck = (double *)calloc(cache, sizeof(double));
    double *cv = (double *)calloc(cache, sizeof(double));
    double *logits = (double *)malloc(sizeof(double) * V);
    float *last = (float *)malloc(sizeof(float) * V);
    memcpy(out, prompt, sizeof(uint32_t) * P);
    uint64_t rng = seed;
    size_t len = P, done = 0;
    for (size_t step = 0; step < count; ++step) {
        /* feed every token not yet cached (the whole prompt on the first step) */
        forward(c, params, E, out + done, len - done, c->context, logits, NULL, ck, cv, done,
                len - done - 1);
        done = len;
        for (size_t t = 0; t < V; ++t) last[t] = (float)logits[t];
        out[len++] = og_sample(last, V, temperature, &rng);
    }
    if (last_logits && count) memcpy(last_logits, last, sizeof(float) * V);
    free(E);
    free(ck);
    free(cv);
    free(logits);
    free(last);
    return 0;
}

/* ------------------------------------------------------------- datasets */

/* src/gpt/text.rs:63-108 */
int og_text_batch(const uint32_t *tokens, size_t len, int validation, size_t sequence, size_t batch,
                  uint64_t seed, uint32_t *inputs, uint32_t *targets) {
    size_t split = len * 9 / 10;
    const uint32_t *corpus = validation ? tokens + split : tokens;
    size_t clen = validation ? len - split : split;
    if (sequence == 0 || sequence >= clen || batch == 0 || batch > OG_MAX_ROWS / sequence) return -1;
    uint64_t rng = seed;
    for (size_t b = 0; b < batch; ++b) {
        float product = og_rng_unit(&rng) * (float)(clen - sequence);
        size_t start = (size_t)product;
        memcpy(inputs + b * sequence, corpus + start, sizeof(uint32_t) * sequence);
        memcpy(targets + b * sequence, corpus + start + 1, sizeof(uint32_t) * sequence);
    }
    return 0;
}

static uint64_t mod_inverse(uint64_t value, uint64_t modulus) {
    uint64_t result = 1, base = value, exponent = modulus - 2;
    while (exponent) {
        if (exponent % 2 == 1) result = result * base % modulus;
        base = base * base % modulus;
        exponent /= 2;
    }
    return result;
}

/* src/gpt/grokking.rs:52-67 */
static uint64_t apply_op(uint32_t op, uint64_t a, uint64_t b, uint64_t p) {
    switch (op) {
    case 0: return (a + b) % p;
    case 1: return a * b % p;
    case 2: return (a + p - b) % p;
    case 3: return a * mod_inverse(b, p) % p;
    case 4: return (b % 2 == 1) ? a * mod_inverse(b, p) % p : (a + p - b) % p;
    case 5: return (a * a + b * b) % p;
    case 6: return (a * a + a * b + b * b) % p;
    case 7: return (a * a + a * b + b * b + a) % p;
    case 8: return (a * a * a + a * b) % p;
    default: return (a * a * a + a * b * b + b) % p;
    }
}

/* grokking.rs:268-272: Fisher-Yates from the back */
static void shuffle_u32(uint32_t *values, size_t n, size_t item, uint64_t *rng) {
    uint32_t tmp[3];
    for (size_t end = n; end-- > 1;) {
        size_t j = (size_t)og_rng_index(rng, end + 1);
        memcpy(tmp, values + end * item, sizeof(uint32_t) * item);
        memmove(values + end * item, values + j * item, sizeof(uint32_t) * item);
        memcpy(values + j * item, tmp, sizeof(uint32_t) * item);
    }
}

/* grokking.rs:128-186, 260-265 */
int og_equations(uint32_t modulus, uint32_t operation, double train_fraction, uint64_t seed,
                 uint32_t *residue_tokens, uint32_t *train, uint32_t *valid, size_t *n_train,
                 size_t *n_valid) {
    if (modulus < 2 || modulus > 254) return -1;
    for (uint32_t d = 2; d < modulus; ++d)
        if (modulus % d == 0) return -1;
    if (!(train_fraction > 0.0 && train_fraction < 1.0)) return -1;
    for (uint32_t i = 0; i < modulus; ++i) residue_tokens[i] = i;
    uint64_t symbols = seed ^ 0x73796d626f6c7301ULL;
    shuffle_u32(residue_tokens, modulus, 1, &symbols);
    uint32_t first_b = operation == 3 ? 1 : 0;
    size_t total = (size_t)modulus * (modulus - first_b);
    uint32_t *all = (uint32_t *)malloc(sizeof(uint32_t) * 3 * total);
    size_t at = 0;
    for (uint32_t a = 0; a < modulus; ++a)
        for (uint32_t b = first_b; b < modulus; ++b) {
            all[3 * at] = a;
            all[3 * at + 1] = b;
            all[3 * at + 2] = (uint32_t)apply_op(operation, a, b, modulus);
            ++at;
        }
    size_t split = (size_t)floor((double)total * train_fraction);
    if (split < 2 || split >= total) {
        free(all);
        return -1;
    }
    uint64_t splits = seed ^ 0x73706c6974730002ULL;
    shuffle_u32(all, total, 3, &splits);
    memcpy(train, all, sizeof(uint32_t) * 3 * split);
    memcpy(valid, all + 3 * split, sizeof(uint32_t) * 3 * (total - split));
    *n_train = split;
    *n_valid = total - split;
    free(all);
    return 0;
}

/* src/bin/mesh-gpt/grokking.rs:544-557 */
double og_row_metrics(const float *row, size_t vocab, size_t target, size_t *prediction) {
    size_t best = 0;
    for (size_t t = 1; t < vocab; ++t)
        if (row[t] > row[best]) best = t;
    double maximum = (double)row[best];
    double sum = 0.0;
    for (size_t t = 0; t < vocab; ++t) sum = sum + exp((double)row[t] - maximum);
    if (prediction) *prediction = best;
    return log(sum) + maximum - (double)row[target];
}
