// Launch wrappers for the training kernels (train.hip): the forward pass that
// keeps every activation the backward needs, the backward of each operator,
// the next-token loss and AdamW.  Rows are [rows][W] f32 in channel order;
// row r of a batch is position r % sequence of sequence r / sequence.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <vector>

namespace meshgpt::kern::train {

constexpr int kMaxDepth = 16;       // mesh layers per kernel launch (weight gradients stay in registers)
constexpr int kMaxWidth = 1024;     // one thread per channel
constexpr int kMaxHeadWidth = 1024; // wave-per-row kernels keep up to 16 dims a lane
constexpr int kMaxSet = 3;          // stacks (or heads' q and k) sharing one launch

// A mesh stack of `depth` layers; the kernels run it kMaxDepth layers at a
// time, each launch on the layers from layer0 (absolute: the butterfly stride
// of layer l is 1 << (l % log2w)), its top layer linear only when it is the
// stack's last.
struct Mesh {
    int W, depth, butterfly, log2w;
    int layer0 = 0, linear_top = 1;
};

// stack[l] (rows x W, l < depth) = output of mesh layer l on `in`
// (reference.rs:422-453): z = x[c] w_self + x[(c + s) % W] w_partner, ELU on
// all layers but the last.
void mesh_forward(const Mesh &m, const float *in, float *stack, const float *w, int rows, hipStream_t stream);
// Scratch floats mesh_backward needs for `rows` rows: the partial sums, and for
// stacks deeper than kMaxDepth the gradient rows between launches.
size_t mesh_partial_floats(const Mesh &m, int rows);
// Backward of mesh_forward: dout is d loss / d stack[depth - 1]; din (when not
// null) receives d loss / d in (added to what it holds when accumulate); the
// weights' gradient goes to grad[0 .. 2 * W * depth) in the parameter layout.
// Deterministic: per-workgroup partial sums in `partials`, then one reduction.
void mesh_backward(const Mesh &m, const float *in, const float *stack, const float *dout, float *din,
                   bool accumulate, const float *w, float *partials, float *grad, int rows, hipStream_t stream);
// A weight gradient's last step: out[i] = the sum over `groups` partial rows
// of n floats at part, in a fixed order.
struct GradReduce {
    const float *part;
    float *out;
    int groups, n;
};
// Runs reductions, up to sixteen a launch.
void reduce_gradients(const GradReduce *r, size_t count, hipStream_t stream);
// `count` (<= kMaxSet) stacks of the same shape at once, stack i on in[i] with
// weights w[i] (the Q, K and V meshes of a block); the backward needs count x
// mesh_partial_floats of `partials`, and its din[i] must be distinct rows.
// With `deferred`, a stack of at most kMaxDepth layers appends its
// reductions there (its partials must then stay untouched until they run).
void mesh_forward_set(const Mesh &m, int count, const float *const *in, float *const *stack, const float *const *w,
                      int rows, hipStream_t stream);
// The RMSNorm (and residual add) in front of a stack set: x = a (+ b, stored to
// sum), n = x / sqrt(mean(x^2) + 1e-5) stored with its factor inv, and the
// stacks run on n; in the wave kernels all in one launch.
struct NormIn {
    const float *a, *b;
    float *sum, *n, *inv;
};
void norm_mesh_forward_set(const Mesh &m, int count, const NormIn &ni, float *const *stack, const float *const *w,
                           int rows, hipStream_t stream);
// The Q, K and V stacks on RMSNorm(a + b), then QK-Norm (when norm) and slice
// RoPE (when rotate) of Q's and K's last layer into out[0], out[1] with the
// norm factors in inv (as qk_forward); one launch where the wave kernels
// allow it.
struct QkOut {
    float *out[2];
    float *inv[2];
    const float2 *table;
    int sequence, H, norm, rotate;
};
void norm_mesh_forward_qkv(const Mesh &m, const NormIn &ni, float *const *stack, const float *const *w,
                           const QkOut &qk, int rows, hipStream_t stream);
// The backward of one stack whose input is RMSNorm(x): its input gradient goes
// through the norm's backward into dx (added); `scratch` (rows x W) holds it
// in between when the two are separate launches.
struct NormGrad {
    const float *x, *inv;
    float *dx;
};
void mesh_backward_norm(const Mesh &m, const float *in, const float *stack, const float *dout, const NormGrad &ng,
                        float *scratch, const float *w, float *partials, float *grad, int rows, hipStream_t stream,
                        std::vector<GradReduce> *deferred);
void mesh_backward_set(const Mesh &m, int count, const float *const *in, const float *const *stack,
                       const float *const *dout, float *const *din, bool accumulate, const float *const *w,
                       float *partials, float *const *grad, int rows, hipStream_t stream,
                       std::vector<GradReduce> *deferred);

// RMSNorm over `groups` equal groups of each row (reference.rs:392-409):
// y = x / sqrt(mean(x^2) + 1e-5); inv[row * groups + g] keeps the factor.
void rmsnorm_forward(const float *x, float *y, float *inv, int rows, int W, int groups, hipStream_t stream);
// The residual add and the RMSNorm after it (whole rows): sum = a + b, y its norm.
void add_rmsnorm_forward(const float *a, const float *b, float *sum, float *y, float *inv, int rows, int W,
                         hipStream_t stream);
// dx = inv dy - x inv^3 (dy . x) / n per group (dx may alias dy; added to
// dx's contents when accumulate, then it must not alias).
void rmsnorm_backward(const float *x, const float *inv, const float *dy, float *dx, bool accumulate, int rows,
                      int W, int groups, hipStream_t stream);
// The same over whole rows with dy = (dy0 + dy1) + dy2 (the Q, K and V meshes'
// gradients of one input).
void rmsnorm_backward_sum3(const float *x, const float *inv, const float *dy0, const float *dy1, const float *dy2,
                           float *dx, bool accumulate, int rows, int W, hipStream_t stream);

// QK-Norm (when norm) then slice RoPE (when rotate; reference.rs:462-482, at
// position r % sequence from the (cos, sin) table [position][hd / 2]) of the
// rows pre[i] into out[i] for i < count (q and k in one launch;
// reference.rs:174-193); inv[i] (rows x H) keeps the norm's factors.
void qk_forward(int count, const float *const *pre, float *const *out, float *const *inv, const float2 *table,
                int rows, int sequence, int W, int H, bool norm, bool rotate, hipStream_t stream);
// Its backward in place on g[i] (d loss / d out -> d loss / d pre).
void qk_backward(int count, float *const *g, const float *const *pre, const float *const *inv, const float2 *table,
                 int rows, int sequence, int W, int H, bool norm, bool rotate, hipStream_t stream);

// Causal softmax attention per (sequence, head) (reference.rs:510-554) into y,
// then z = XSA(y) (reference.rs:577-603: y - (y.u) u, u = v / max(|v|, 1e-12)
// per head) when xsa, else z = y; lse[r * H + h] = max + ln(sum) of the row's
// scaled scores.
void attention_forward(const float *q, const float *k, const float *v, float *y, float *z, float *lse, int rows,
                       int sequence, int W, int H, bool xsa, hipStream_t stream);
// Its backward from dz = d loss / d z: dq and dk written, dv written (XSA's
// part and attention's); dy (rows x W) and dsum (rows x H) are scratch.
// Sequences of at most 8 rows take one launch for all of it.
void attention_backward(const float *q, const float *k, const float *v, const float *y, const float *lse,
                        const float *dz, float *dy, float *dq, float *dk, float *dv, float *dsum, int rows,
                        int sequence, int W, int H, bool xsa, hipStream_t stream);

// The embedding geometry (reference.rs:130-149) on V raw token rows: scaled to
// `radius` when normalize (rinv[t] keeps 1 / max(|row|, 1e-12)), then the first
// `preserve` coordinates replaced by the codes.
void geometry_forward(const float *raw, const float *codes, float *out, float *rinv, int V, int W, float radius,
                      bool normalize, int preserve, hipStream_t stream);
// Its backward in place on g (d loss / d out -> d loss / d raw).
void geometry_backward(const float *raw, const float *rinv, float *g, int V, int W, float radius, bool normalize,
                       int preserve, hipStream_t stream);

// x[r] = E[tokens[r]]
void gather(const float *E, const uint32_t *tokens, float *x, int rows, int W, hipStream_t stream);
// logits[r][t] = n[r] . E[t] (FP32 matrix cores; each dot product's terms are
// added in another order than the reference's sequential sum, within f32
// rounding of it).
void head_logits(const float *n, const float *E, float *logits, int rows, int W, int V, hipStream_t stream);
// A training step's scalars in device memory, written before each step, so
// that a captured step replays with new values: the AdamW bias corrections
// 1 - beta^t, 1 / (supervised rows), and a flag the loss kernel raises on a
// non-finite loss (the update is then skipped).
struct StepScalars {
    float correction1, correction2, inv_supervised;
    int nonfinite;
};

// The loss kernel of gpu.rs:949-994: per row the f32 cross-entropy and
// d loss / d logits = (softmax - onehot) / supervised; ignored rows give 0.
void cross_entropy(const float *logits, const uint32_t *targets, float *dlogits, float *loss, int rows, int V,
                   StepScalars *scalars, hipStream_t stream);
// p[0 .. n) = v;  b[0 .. n) = a[0 .. n)  (kernels: nothing a graph replays badly)
void fill(float *p, float v, size_t n, hipStream_t stream);
void copy(const float *a, float *b, size_t n, hipStream_t stream);
// dn[r][c] = sum_t dlogits[r][t] E[t][c]
void head_backward(const float *dlogits, const float *E, float *dn, int rows, int W, int V, hipStream_t stream);
// dE[t][c] = sum_r dlogits[r][t] n[r][c] + sum over rows r of token t of dx[r][c],
// by slices of 64 rows into `partials` (embedding_partial_floats), then one
// deterministic reduction.  These products, like head_backward's, run on the
// FP32 matrix cores.
size_t embedding_partial_floats(int rows, int W, int V);
void embedding_gradient(const float *dlogits, const float *n, const uint32_t *tokens, const float *dx, float *dE,
                        float *partials, int rows, int W, int V, hipStream_t stream);

// The forward of short sequences for inference (logits only): one workgroup
// per sequence of at most kShortRows rows, one wave per row, W <= 128 and head
// widths a power of two up to 64 (or 128); E the effective token vectors
// (V x W), Et the same transposed, w the parameters with block 0's query group
// at block0, table the RoPE (cos, sin) pairs [position][hd / 2].  logits: one
// row per sequence (last_only) or per row.
constexpr int kShortRows = 16;
struct ShortForward {
    const float *E, *Et, *w;  // Et: E transposed, [W][vpad]
    const uint32_t *tokens;
    const float2 *table;
    float *logits;
    size_t block0;
    int W, H, L, A, F, V, vpad, sequence, butterfly, log2w, rope, qk_norm, xsa, last_only;
    float scale;  // 1 / sqrt(W / H)
};
bool short_forward_fits(int W, int H, size_t V, int sequence);
void short_forward(const ShortForward &a, int sequences, hipStream_t stream);

struct AdamW {
    float learning_rate, weight_decay, beta1, beta2, epsilon;
};
// gpu.rs:1366-1391 over params[begin, end): f32 moments m, v; the bias
// corrections come from scalars, and nothing changes when its flag is set.
void adam(float *params, float *m, float *v, const float *grad, size_t begin, size_t end, const AdamW &o,
          const StepScalars *scalars, hipStream_t stream);

}  // namespace meshgpt::kern::train
