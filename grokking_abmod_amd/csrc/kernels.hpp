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
    int rope;      // operator switches (config.rs:33-35): 1 on, 0 off
    int qk_norm;
    int xsa;
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
    // Decode attention reads rows past the first `keep` of a slab with the
    // non-temporal cache policy (kv_keep_rows); prefill ignores it.
    int keep = 1 << 30;
};

// One block_kernel launch: the post-attention half of block l-1 (when wproj
// is set) followed by the pre-attention half of block l (when wq is set).
struct BlockArgs {
    Shape s;
    Rows ro;
    float *x;  // residual rows, read (and written when x_out is null)
    // Where the updated residual rows go.  row_block() needs a buffer other
    // than x: its three workgroups of a row read x, and one of them writes the
    // update, which the others could otherwise read when they start later.
    float *x_out;
    // post half: weights, attention output (split partials or rows), block l-1's cache
    const float *wproj, *wffn;
    const float *part;
    int nsplit;
    const float *ybuf;  // attention rows when part is null
    // 1: the post half applies XSA to the attention output (split partials,
    // or rows from attn_prefill); 0: the output already has it (attn_prefill_mfma).
    int xsa_post;
    KvView kv_post;
    // pre half: weights, token vectors when embed, query rows out, block l's cache
    const float *wq, *wk, *wv;
    const float *E;
    int embed;
    float *q;
    KvView kv_pre;
    const float2 *rope;
    float *xn;  // when set: the final RMSNorm of x for the head
    int rpw;    // rows per workgroup
    int teams;  // 3: Q, K, V meshes run concurrently; 1: one after another
};

// Threads per mesh team and channels per thread for width W.
int team_threads(int W);
int channels_per_thread(int W);

// LDS of one block_kernel launch; staged adds the weight stage, which needs
// block_can_stage (the weights fit the per-thread register hold).
size_t block_lds_bytes(const Shape &s, int rpw, int teams, bool staged, bool post, bool pre);
bool block_can_stage(const Shape &s, int teams, bool post, bool pre);
size_t mesh_lds_bytes(const Shape &s, int rpw);
size_t head_lds_bytes(const Shape &s, int rt);
size_t head_sample_lds_bytes(const Shape &s);  // size_t(-1) when V is too large

// Allows dynamic LDS up to max_bytes on every kernel that uses it.
void configure_lds(size_t max_bytes);

// out = mesh(in) for rows x W (the embedding table from token codes).
void mesh_rows(const Shape &s, const float *in, float *out, int rows, const float *w, int depth, int rpw,
               hipStream_t stream);
// The geometry transform of the token vectors (reference.rs:130-149): with
// `normalize`, each row of E scaled to length `radius`; the first `keep`
// channels of each row replaced by the token's code (codes, V x W).
void embedding_geometry(float *E, const float *codes, int V, int W, float radius, int normalize, int keep,
                        hipStream_t stream);
// Et[c][t] = E[t][c], rows of Vp >= V floats with zero padding.
void transpose(const float *E, float *Et, int V, int Vp, int W, hipStream_t stream);
void block(const BlockArgs &a, bool staged, hipStream_t stream);
// Prefill variant of block() for many rows (prefill_rows.hip): tiles of
// 4096 / W rows, channels of those rows in registers, partners through LDS.
// Needs W in {128, 256, 512, 1024}, a power-of-two head width dividing 64, and
// attention rows in a.ybuf (not split partials).
bool rows_block_supported(const Shape &s);
void rows_block(const BlockArgs &a, hipStream_t stream);
// Decode variant of block(): one row per sequence (rows_per_seq == 1), each
// mesh of a row on one wavefront.  Supported for W a power of two in
// [64, 1024] and a power-of-two head width >= 8.
bool block_decode_supported(const Shape &s);
void block_decode(const BlockArgs &a, hipStream_t stream);
// Row-order decode block (three workgroups per row, channels spread over
// row_waves(W) waves: channel c = wave + NW*(lane + 64*j)).  Needs W in
// {128, 256, 512, 1024} and hd / NW in {8, 16, 32}.  Its E, x and mesh weights
// are in row order (row_order()); xn, q and the cache stay in channel order.
// It reads the residual rows from a.x and writes them to a.x_out, which must
// be a different buffer.
int row_waves(int W);
bool row_block_supported(const Shape &s);
void row_block(const BlockArgs &a, hipStream_t stream);
// dst = src with each row of W channels (floats, or float2 weight pairs when
// `pairs`) permuted into row order.
void row_order(const float *src, float *dst, int rows, int W, bool pairs, hipStream_t stream);
// One launch of the persistent decode kernel: `steps` decode steps of `batch`
// sequences (each with its last token not yet run through the blocks), every
// mesh and attention phase inside the launch.  Needs persistent_fits().
struct PersistArgs {
    Shape s;
    int batch, layers, steps;
    const float *E;       // token vectors in row order (V x W)
    const float *w;       // mesh weights in row order, at their parameter offsets
    size_t block0;        // offset of block 0's first mesh
    float *kc, *vc;       // KV cache, layer-major
    size_t layer_elems;   // floats of one layer of the cache
    int cap;              // positions per (sequence, head) slab
    const float *q0;      // layer-0 table (persistent_layer0)
    float *logits;        // [batch][V] logits of the launch's last step
    const float2 *rope;
    uint32_t *tokens;
    int tok_stride;
    int *len;             // each sequence's length, written at the end of the launch
    uint64_t *rng;        // each sequence's sampler state at the start of the launch (read only)
    uint64_t *rng_out;    // ... and at its end, written by the launch
    float temperature;
    int *flags;           // bit 0: non-finite logits
    uint64_t *xch;        // [batch][xstride] tagged exchange words, zero at launch
    size_t xstride;       // persistent_exchange_words(shape)
    int *abort;           // zero at launch; set when a wait times out
    uint64_t wait_ticks;  // a wait's limit in 100 MHz wall-clock ticks (kWaitTicks unless overridden)
    float scale_log2;     // set by persistent_decode
    int xcd_cus;          // CUs per XCD, set by persistent_decode
    // Nonzero: every sequence's hand-offs use the agent-scope atomics, as when
    // its workgroups run on different XCDs, instead of the XCD-local words the
    // launch's handshake otherwise chooses where it can (for testing that
    // protocol; MG_PERSIST_AGENT_SCOPE=1).
    int agent_scope;
    // Cached K/V rows at or past this position load with the non-temporal
    // cache policy (kv_keep_rows).
    int mall_keep;
    // Optional timeline (nullptr: none): for block k, step t and phase l,
    // trace[((k * steps + t) * (layers + 1) + l) * 2 + {0, 1}] receive the
    // wall clock (100 MHz) when the phase's inputs were ready and when its
    // outputs were published.  Mesh teams: l = 0..layers (l = layers: logits
    // ready, token drawn); attention blocks: l = 0..layers-1, and l = layers
    // when the last block's post-attention half is done (slot 0) and their
    // logit slice is published (slot 1).
    uint64_t *trace;
};
bool persistent_fits(const Shape &s, int batch, int device);
// The cached rows of each (sequence, layer, head) that decode attention reads
// with the default cache policy when `batch` sequences decode: the first rows
// of every slab, as many as keep about 80 % of the MI355X's 256 MiB memory-side
// cache (Infinity Cache) for them (MG_MALL_BYTES overrides its size); rows
// past them load with the non-temporal policy.  Read every step and larger
// in total than the cache, the cache rows would otherwise be evicted before
// their reuse by rows read once per step (least recently used replacement
// over a cyclic pass); kept this way, the prefix stays resident across steps
// and only the rest streams from HBM (config 3 at batch 32: 27.4 against
// 30.8 ms per 512-step launch).
int kv_keep_rows(const Shape &s, int batch, int layers);
// Exchange words of one sequence: q/k/v of two layer phases, the attention
// output, the normalised final row, the logits and each workgroup's XCD.
size_t persistent_exchange_words(const Shape &s);
// Builds the layer-0 table q0 (V x 3 x W floats, row order): for each token,
// the Q, K and V meshes of block 0 on its normalised vector, before QK-norm
// and RoPE.  E and w are the row-order token vectors and weights.  False when
// the shape has no persistent kernel.
size_t persistent_layer0_floats(const Shape &s);
bool persistent_layer0(const Shape &s, const float *E, const float *w, size_t block0, float *q0, hipStream_t stream);
hipError_t persistent_decode(const PersistArgs &a, hipStream_t stream);

// Split-KV decode attention: one query row per sequence; the len[b] keys are
// cut into nsplit equal shares whose partial softmax states (acc[hdp], m, l)
// go to part[((b*H+h)*nsplit+split)*(hdp+2)].  When start/stop are given the
// launch goes through hipExtLaunchKernel and the events receive the kernel's
// own begin and end timestamps.
void attn_decode(const Shape &s, const float *q, KvView kv, const int *len, int batch, int nsplit,
                 float *part, hipStream_t stream, hipEvent_t start = nullptr, hipEvent_t stop = nullptr);
// Causal flash attention over whole sequences already appended to the cache.
void attn_prefill(const Shape &s, const float *q, KvView kv, int nseq, int rows_per_seq, float *y,
                  hipStream_t stream);
// The same on the FP32 matrix cores, with XSA applied to each output row when
// xsa != 0 (then the block's post half must not apply it again).  Supported
// when attn_prefill_mfma_supported(); the sequences are at least 64 rows long.
bool attn_prefill_mfma_supported(const Shape &s, int rows_per_seq);
// The same for short sequences (at most 16 rows), one thread per (row, head),
// with XSA applied when xsa != 0.
bool attn_prefill_short_supported(const Shape &s, int rows_per_seq);
void attn_prefill_short(const Shape &s, const float *q, KvView kv, int nseq, int rows_per_seq, float *y, int xsa,
                        hipStream_t stream);
void attn_prefill_mfma(const Shape &s, const float *q, KvView kv, int nseq, int rows_per_seq, float *y, int xsa,
                       hipStream_t stream);
// logits[i][t] = xn[i*row_mul+row_add] . E[t] (xn already RMS-normalised).
void head(const Shape &s, const float *xn, int nrows, int row_mul, int row_add, const float *Et, int Vp,
          float *logits, int rt, hipStream_t stream);
// Decode head fused with sampling: logits of each sequence's row, then the
// next token appended at len[b].
void head_sample(const Shape &s, const float *xn, int batch, const float *Et, int Vp, float *logits,
                 float temperature, uint64_t *rng, uint32_t *tokens, int tok_stride, int *len, int *flags,
                 hipStream_t stream);
// Greedy / temperature sampling from logits rows; appends the token and bumps len.
void sample(int V, int batch, const float *logits, float temperature, uint64_t *rng, uint32_t *tokens,
            int tok_stride, int *len, int *flags, hipStream_t stream);
// Rows the allocation-free sampler accepts: its scratch holds one append
// counter per row (noalloc.hip).
constexpr int kNoAllocRows = 65536;
// The device address of that scratch array on `device` (the current device).
hipError_t noalloc_scratch(int device, int **out);
// p[0..n) = value, by a kernel (no memset node when a caller captures the stream).
void fill_int(int *p, int value, int n, hipStream_t stream);
// y[i] = the sampler's f32 exp of x[i] (for verification).
void device_expf(const float *x, float *y, size_t n, hipStream_t stream);
// dst[i] = src[i] for n float4 elements (bandwidth calibration).
void calibration_copy(const float4 *src, float4 *dst, size_t n, hipStream_t stream);

}  // namespace meshgpt::kern
