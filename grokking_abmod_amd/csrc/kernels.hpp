// Launch wrappers for the gfx950 kernels of the Mesh GPT generate path.
// Host code (model.cpp) calls only these; every kernel lives in kernels.hip.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>

namespace meshgpt::kern {

constexpr int kThreads = 256;

// Model dimensions as the kernels see them.
struct Shape {
    int W;         // width
    int H;         // heads
    int hd;        // head width
    int hdp;       // padded head width: the KV-cache row stride (power of two >= hd)
    int half;      // hd / 2 (RoPE pairs)
    int V;         // vocabulary
    int log2w;     // floor(log2 W): butterfly strides are 1 << (layer % log2w)
    int wshift;    // log2 W when W is a power of two, else -1
    int hdshift;   // log2 hd when hd is a power of two, else -1
    int butterfly; // 1 for butterfly connectivity, 0 for neighbor
    int A;         // attention / embedding mesh depth
    int F;         // feed-forward mesh depth
};

// Which rows a launch covers.  Row r belongs to sequence r / rows_per_seq and
// sits at position base + r % rows_per_seq, where base is len[seq] - 1 during
// decode (len != nullptr) and 0 during prefill.  Its input token is
// tokens[seq * tok_stride + tok_offset + position].
struct Rows {
    int rows;
    int rows_per_seq;
    const int *len;
    const uint32_t *tokens;
    int tok_stride;
    int tok_offset;
};

// One layer of the KV cache: element (seq, head, position, d) lives at
// ((seq * H + head) * cap + position) * hdp + d.
struct KvView {
    float *k;
    float *v;
    int cap;
};

// Rows per workgroup and how many mesh layers of weights are staged in LDS at
// once (0: weights are read straight from global memory).
struct Tiling {
    int rpw;
    int stage_layers;
};

size_t qkv_lds_bytes(const Shape &s, const Tiling &t);
size_t post_lds_bytes(const Shape &s, const Tiling &t);
size_t mesh_lds_bytes(const Shape &s, const Tiling &t);
size_t head_lds_bytes(const Shape &s, int rt);

// Allows dynamic LDS above the 64 KiB default on every kernel that needs it.
void configure_lds(size_t max_bytes);

// out = mesh(in) for rows x W (the embedding table from token codes).
void mesh_rows(const Shape &s, const float *in, float *out, int rows, const float *w, int depth,
               Tiling t, hipStream_t stream);
// Et[c][t] = E[t][c]
void transpose(const float *E, float *Et, int V, int W, hipStream_t stream);
// Pre-attention half of a block for `rows`: (embed), RMSNorm, one of the Q/K/V
// meshes per grid.y, QK-Norm + RoPE, then q rows or the KV-cache append.
void qkv(const Shape &s, const Rows &r, const float *wq, const float *wk, const float *wv,
         const float *E, float *x, float *q, KvView kv, const float2 *rope, int embed, Tiling t,
         hipStream_t stream);
// Split-KV decode attention: one query row per sequence, partial softmax states
// per split of `ks` keys written to part[((b*H+h)*smax+split)*(hdp+2)].
void attn_decode(const Shape &s, const float *q, KvView kv, const int *len, int batch, int ks,
                 int smax, float *part, hipStream_t stream);
// Causal flash attention over whole sequences already appended to the cache.
void attn_prefill(const Shape &s, const float *q, KvView kv, int nseq, int rows_per_seq, float *y,
                  hipStream_t stream);
// Post-attention half of a block: (split combine), XSA, projection mesh +
// residual, RMSNorm, FFN mesh + residual; updates x in place.
void post(const Shape &s, const Rows &r, const float *part, int ks, int smax, const float *y,
          KvView kv, const float *wproj, const float *wffn, float *x, Tiling t, hipStream_t stream);
// logits[i][t] = rmsnorm(x[i*row_mul+row_add]) . E[t]
void head(const Shape &s, const float *x, int nrows, int row_mul, int row_add, const float *Et,
          float *logits, int rt, hipStream_t stream);
// Greedy / temperature sampling per sequence; appends the token and bumps len.
void sample(int V, int batch, const float *logits, float temperature, uint64_t *rng,
            uint32_t *tokens, int tok_stride, int *len, int *flags, hipStream_t stream);

}  // namespace meshgpt::kern
