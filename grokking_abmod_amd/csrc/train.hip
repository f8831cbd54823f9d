// Training kernels for gfx950: the forward pass with its saved activations,
// the backward of every operator of reference.rs:104-228, the next-token loss
// and AdamW (gpu.rs:949-994,1366-1391).  The training rows are few (the
// reference's benchmark: 2048 rows of width 128), so each operator is one
// launch over all rows: a mesh stack runs with the row in LDS, one thread per
// channel; the per-row operators run one wave per (row, group) or one thread
// per (row, head).  Weight gradients are summed deterministically: partial
// sums per workgroup, then one reduction in a fixed order.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <type_traits>

#include "dpp.hpp"
#include "train.hpp"

namespace meshgpt::kern::train {
namespace {

constexpr float kRmsEps = 1e-5f;                                         // src/gpt/mod.rs:38
constexpr float kXsaFloor = float(double(1e-12f) * double(1e-12f));      // XSA_EPSILON^2
constexpr int kThreads = 256;

__device__ __forceinline__ float elu(float z) { return z >= 0.0f ? z : expm1f(z); }

__device__ __forceinline__ int stride_of(const Mesh &m, int l) { return m.butterfly ? 1 << (l % m.log2w) : 1; }

int block_for(int W) { return std::max(64, (W + 63) / 64 * 64); }

unsigned blocks_for(size_t n, int threads = kThreads) { return unsigned((n + threads - 1) / threads); }

// ---- mesh stacks

__global__ void __launch_bounds__(kMaxWidth) mesh_forward_kernel(Mesh m, const float *__restrict__ in,
                                                                 float *__restrict__ stack,
                                                                 const float *__restrict__ w, int rows) {
    extern __shared__ float buf[];  // two rows: the layer's input and output
    const int c = threadIdx.x, W = m.W;
    for (int r = blockIdx.x; r < rows; r += gridDim.x) {
        float *cur = buf, *nxt = buf + W;
        if (c < W) cur[c] = in[size_t(r) * W + c];
        __syncthreads();
        for (int l = 0; l < m.depth; ++l) {
            if (c < W) {
                int p = c + stride_of(m, l);
                if (p >= W) p -= W;
                const float *wl = w + size_t(l) * 2 * W;
                float z = cur[c] * wl[2 * c] + cur[p] * wl[2 * c + 1];
                if (l + 1 < m.depth) z = elu(z);
                nxt[c] = z;
                stack[(size_t(l) * rows + r) * W + c] = z;
            }
            __syncthreads();
            float *t = cur;
            cur = nxt;
            nxt = t;
        }
    }
}

// Each workgroup takes rows blockIdx.x, blockIdx.x + gridDim.x, ...; thread c
// carries d loss / d (channel c) down the layers and adds its two weights'
// gradients over those rows in registers.
__global__ void __launch_bounds__(kMaxWidth) mesh_backward_kernel(Mesh m, const float *__restrict__ in,
                                                                  const float *__restrict__ stack,
                                                                  const float *__restrict__ dout, float *din,
                                                                  int accumulate, const float *__restrict__ w,
                                                                  float *__restrict__ partials, int rows) {
    extern __shared__ float dz_row[];
    const int c = threadIdx.x, W = m.W, depth = m.depth;
    float gs[kMaxDepth], gp[kMaxDepth];
#pragma unroll
    for (int l = 0; l < kMaxDepth; ++l) gs[l] = gp[l] = 0.0f;
    for (int r = blockIdx.x; r < rows; r += gridDim.x) {
        float g = c < W ? dout[size_t(r) * W + c] : 0.0f;
#pragma unroll
        for (int l = kMaxDepth - 1; l >= 0; --l) {
            if (l >= depth) continue;
            const int s = stride_of(m, l);
            if (c < W) {
                float dz = g;
                if (l + 1 < depth) {
                    // ELU'(z) from its output a: 1 for a >= 0, else exp(z) = a + 1.
                    const float a = stack[(size_t(l) * rows + r) * W + c];
                    dz = a >= 0.0f ? g : g * (a + 1.0f);
                }
                const float *x = l == 0 ? in + size_t(r) * W : stack + (size_t(l - 1) * rows + r) * W;
                int p = c + s;
                if (p >= W) p -= W;
                gs[l] = fmaf(dz, x[c], gs[l]);
                gp[l] = fmaf(dz, x[p], gp[l]);
                dz_row[c] = dz;
            }
            __syncthreads();
            if (c < W) {
                // Channel c feeds itself (weight 2c) and channel c - s (weight 2(c - s) + 1).
                int q = c - s;
                if (q < 0) q += W;
                const float *wl = w + size_t(l) * 2 * W;
                g = dz_row[c] * wl[2 * c] + dz_row[q] * wl[2 * q + 1];
            }
            __syncthreads();
        }
        if (c < W && din) {
            const size_t i = size_t(r) * W + c;
            din[i] = accumulate ? din[i] + g : g;
        }
    }
    if (c < W) {
#pragma unroll
        for (int l = 0; l < kMaxDepth; ++l)
            if (l < depth) {
                float *o = partials + ((size_t(blockIdx.x) * depth + l) * W + c) * 2;
                o[0] = gs[l];
                o[1] = gp[l];
            }
    }
}

__global__ void __launch_bounds__(kThreads) mesh_reduce_kernel(const float *__restrict__ partials, int groups,
                                                               int n, float *__restrict__ grad) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    float acc = 0.0f;
    for (int g = 0; g < groups; ++g) acc += partials[size_t(g) * n + i];
    grad[i] = acc;
}

int mesh_groups(const Mesh &m, int rows) { return std::max(1, std::min(rows, 256)); }

// ---- norms (one wave per (row, group))

__global__ void __launch_bounds__(kThreads) rmsnorm_forward_kernel(const float *__restrict__ x, float *y,
                                                                   float *__restrict__ inv, int n_groups, int gw) {
    const int wave = (blockIdx.x * kThreads + threadIdx.x) >> 6, lane = threadIdx.x & 63;
    if (wave >= n_groups) return;
    const float *xs = x + size_t(wave) * gw;
    float acc = 0.0f;
    for (int i = lane; i < gw; i += 64) acc = fmaf(xs[i], xs[i], acc);
    const float iv = rsqrtf(wave_sum(acc) * (1.0f / float(gw)) + kRmsEps);
    for (int i = lane; i < gw; i += 64) y[size_t(wave) * gw + i] = xs[i] * iv;
    if (lane == 0) inv[wave] = iv;
}

__global__ void __launch_bounds__(kThreads) rmsnorm_backward_kernel(const float *__restrict__ x,
                                                                    const float *__restrict__ inv, const float *dy,
                                                                    float *dx, int accumulate, int n_groups, int gw) {
    const int wave = (blockIdx.x * kThreads + threadIdx.x) >> 6, lane = threadIdx.x & 63;
    if (wave >= n_groups) return;
    const size_t o = size_t(wave) * gw;
    float acc = 0.0f;
    for (int i = lane; i < gw; i += 64) acc = fmaf(dy[o + i], x[o + i], acc);
    const float iv = inv[wave];
    const float k = wave_sum(acc) * iv * iv * iv * (1.0f / float(gw));
    for (int i = lane; i < gw; i += 64) {
        const float d = iv * dy[o + i] - x[o + i] * k;
        dx[o + i] = accumulate ? dx[o + i] + d : d;
    }
}

// ---- RoPE (one thread per (row, head, pair))

__global__ void __launch_bounds__(kThreads) rope_kernel(float *x, const float2 *__restrict__ table, int rows,
                                                        int sequence, int W, int H, int inverse) {
    const int hd = W / H, half = hd / 2;
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= rows * H * half) return;
    const int r = i / (H * half), rest = i % (H * half), h = rest / half, pair = rest % half;
    const float2 cs = table[size_t(r % sequence) * half + pair];
    float *row = x + size_t(r) * W + h * hd;
    const float a = row[pair], b = row[pair + half];
    if (inverse) {
        row[pair] = a * cs.x + b * cs.y;
        row[pair + half] = b * cs.x - a * cs.y;
    } else {
        row[pair] = a * cs.x - b * cs.y;
        row[pair + half] = b * cs.x + a * cs.y;
    }
}

// ---- attention (one thread per (row, head); the head row in registers)

template <int HD>
__global__ void __launch_bounds__(kThreads) attention_forward_kernel(const float *__restrict__ q,
                                                                     const float *__restrict__ k,
                                                                     const float *__restrict__ v,
                                                                     float *__restrict__ y,
                                                                     float *__restrict__ lse, int rows,
                                                                     int sequence, int W, int H, float scale) {
    const int t = blockIdx.x * kThreads + threadIdx.x;
    if (t >= rows * H) return;
    const int r = t / H, h = t % H, hd = W / H, pos = r % sequence, first = r - pos;
    float qr[HD], acc[HD];
#pragma unroll
    for (int d = 0; d < HD; ++d) {
        qr[d] = d < hd ? q[size_t(r) * W + h * hd + d] : 0.0f;
        acc[d] = 0.0f;
    }
    float m = -INFINITY, l = 0.0f;
    for (int j = 0; j <= pos; ++j) {
        const float *kr = k + size_t(first + j) * W + h * hd, *vr = v + size_t(first + j) * W + h * hd;
        float s = 0.0f;
#pragma unroll
        for (int d = 0; d < HD; ++d)
            if (d < hd) s = fmaf(qr[d], kr[d], s);
        s *= scale;
        const float mn = fmaxf(m, s), alpha = expf(m - mn), p = expf(s - mn);
        l = l * alpha + p;
#pragma unroll
        for (int d = 0; d < HD; ++d)
            if (d < hd) acc[d] = fmaf(p, vr[d], acc[d] * alpha);
        m = mn;
    }
    const float il = 1.0f / l;
#pragma unroll
    for (int d = 0; d < HD; ++d)
        if (d < hd) y[size_t(r) * W + h * hd + d] = acc[d] * il;
    lse[t] = m + logf(l);
}

// dq_i = scale sum_j P_ij (dy_i . v_j - D_i) k_j with D_i = dy_i . y_i.
template <int HD>
__global__ void __launch_bounds__(kThreads) attention_dq_kernel(const float *__restrict__ q,
                                                                const float *__restrict__ k,
                                                                const float *__restrict__ v,
                                                                const float *__restrict__ y,
                                                                const float *__restrict__ lse,
                                                                const float *__restrict__ dy, float *__restrict__ dq,
                                                                float *__restrict__ dsum, int rows, int sequence,
                                                                int W, int H, float scale) {
    const int t = blockIdx.x * kThreads + threadIdx.x;
    if (t >= rows * H) return;
    const int r = t / H, h = t % H, hd = W / H, pos = r % sequence, first = r - pos;
    const size_t o = size_t(r) * W + h * hd;
    float qr[HD], g[HD], acc[HD];
    float D = 0.0f;
#pragma unroll
    for (int d = 0; d < HD; ++d) {
        qr[d] = d < hd ? q[o + d] : 0.0f;
        g[d] = d < hd ? dy[o + d] : 0.0f;
        if (d < hd) D = fmaf(g[d], y[o + d], D);
        acc[d] = 0.0f;
    }
    const float L = lse[t];
    for (int j = 0; j <= pos; ++j) {
        const float *kr = k + size_t(first + j) * W + h * hd, *vr = v + size_t(first + j) * W + h * hd;
        float s = 0.0f, gv = 0.0f;
#pragma unroll
        for (int d = 0; d < HD; ++d)
            if (d < hd) {
                s = fmaf(qr[d], kr[d], s);
                gv = fmaf(g[d], vr[d], gv);
            }
        const float ds = expf(s * scale - L) * (gv - D);
#pragma unroll
        for (int d = 0; d < HD; ++d)
            if (d < hd) acc[d] = fmaf(ds, kr[d], acc[d]);
    }
#pragma unroll
    for (int d = 0; d < HD; ++d)
        if (d < hd) dq[o + d] = acc[d] * scale;
    dsum[t] = D;
}

// For key row j: dv_j += sum_i P_ij dy_i, dk_j = scale sum_i P_ij (dy_i . v_j - D_i) q_i over the
// queries i >= j of its sequence.
template <int HD>
__global__ void __launch_bounds__(kThreads) attention_dkv_kernel(const float *__restrict__ q,
                                                                 const float *__restrict__ k,
                                                                 const float *__restrict__ v,
                                                                 const float *__restrict__ lse,
                                                                 const float *__restrict__ dy,
                                                                 const float *__restrict__ dsum,
                                                                 float *__restrict__ dk, float *dv, int rows,
                                                                 int sequence, int W, int H, float scale) {
    const int t = blockIdx.x * kThreads + threadIdx.x;
    if (t >= rows * H) return;
    const int j = t / H, h = t % H, hd = W / H, pos = j % sequence, last = j - pos + sequence;
    const size_t o = size_t(j) * W + h * hd;
    float kr[HD], vr[HD], ak[HD], av[HD];
#pragma unroll
    for (int d = 0; d < HD; ++d) {
        kr[d] = d < hd ? k[o + d] : 0.0f;
        vr[d] = d < hd ? v[o + d] : 0.0f;
        ak[d] = av[d] = 0.0f;
    }
    for (int i = j; i < last; ++i) {
        const float *qi = q + size_t(i) * W + h * hd, *gi = dy + size_t(i) * W + h * hd;
        float s = 0.0f, gv = 0.0f;
#pragma unroll
        for (int d = 0; d < HD; ++d)
            if (d < hd) {
                s = fmaf(qi[d], kr[d], s);
                gv = fmaf(gi[d], vr[d], gv);
            }
        const float p = expf(s * scale - lse[size_t(i) * H + h]);
        const float ds = p * (gv - dsum[size_t(i) * H + h]);
#pragma unroll
        for (int d = 0; d < HD; ++d)
            if (d < hd) {
                av[d] = fmaf(p, gi[d], av[d]);
                ak[d] = fmaf(ds, qi[d], ak[d]);
            }
    }
#pragma unroll
    for (int d = 0; d < HD; ++d)
        if (d < hd) {
            dk[o + d] = ak[d] * scale;
            dv[o + d] += av[d];
        }
}

// ---- XSA (one thread per (row, head))

template <int HD>
__global__ void __launch_bounds__(kThreads) xsa_forward_kernel(const float *__restrict__ y,
                                                               const float *__restrict__ v, float *__restrict__ z,
                                                               int rows, int W, int H) {
    const int t = blockIdx.x * kThreads + threadIdx.x;
    if (t >= rows * H) return;
    const int hd = W / H;
    const size_t o = size_t(t / H) * W + (t % H) * hd;
    float yv[HD], u[HD], sq = 0.0f;
#pragma unroll
    for (int d = 0; d < HD; ++d) {
        yv[d] = d < hd ? y[o + d] : 0.0f;
        u[d] = d < hd ? v[o + d] : 0.0f;
        sq = fmaf(u[d], u[d], sq);
    }
    const float inv = rsqrtf(fmaxf(sq, kXsaFloor));
    float s = 0.0f;
#pragma unroll
    for (int d = 0; d < HD; ++d) {
        u[d] *= inv;
        s = fmaf(yv[d], u[d], s);
    }
#pragma unroll
    for (int d = 0; d < HD; ++d)
        if (d < hd) z[o + d] = yv[d] - s * u[d];
}

// dy = dz - (dz.u) u;  du = -((y.u) dz + (dz.u) y);  dv = inv (du - u (u.du))
// above the norm floor, inv du below it.
template <int HD>
__global__ void __launch_bounds__(kThreads) xsa_backward_kernel(const float *__restrict__ y,
                                                                const float *__restrict__ v,
                                                                const float *__restrict__ dz, float *__restrict__ dy,
                                                                float *__restrict__ dv, int rows, int W, int H) {
    const int t = blockIdx.x * kThreads + threadIdx.x;
    if (t >= rows * H) return;
    const int hd = W / H;
    const size_t o = size_t(t / H) * W + (t % H) * hd;
    float yv[HD], u[HD], g[HD], sq = 0.0f;
#pragma unroll
    for (int d = 0; d < HD; ++d) {
        yv[d] = d < hd ? y[o + d] : 0.0f;
        u[d] = d < hd ? v[o + d] : 0.0f;
        g[d] = d < hd ? dz[o + d] : 0.0f;
        sq = fmaf(u[d], u[d], sq);
    }
    const float inv = rsqrtf(fmaxf(sq, kXsaFloor));
    float s = 0.0f, tg = 0.0f;
#pragma unroll
    for (int d = 0; d < HD; ++d) {
        u[d] *= inv;
        s = fmaf(yv[d], u[d], s);
        tg = fmaf(g[d], u[d], tg);
    }
    float udu = 0.0f;
#pragma unroll
    for (int d = 0; d < HD; ++d) udu = fmaf(u[d], -(s * g[d] + tg * yv[d]), udu);
    const float keep = sq >= kXsaFloor ? 1.0f : 0.0f;
#pragma unroll
    for (int d = 0; d < HD; ++d)
        if (d < hd) {
            const float du = -(s * g[d] + tg * yv[d]);
            dy[o + d] = g[d] - tg * u[d];
            dv[o + d] = inv * (du - keep * u[d] * udu);
        }
}

// ---- head, loss and embedding gradient

__global__ void __launch_bounds__(kThreads) gather_kernel(const float *__restrict__ E,
                                                          const uint32_t *__restrict__ tokens, float *__restrict__ x,
                                                          int rows, int W) {
    const size_t i = size_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= size_t(rows) * W) return;
    const size_t r = i / W, c = i % W;
    x[i] = E[size_t(tokens[r]) * W + c];
}

__global__ void __launch_bounds__(kThreads) add_kernel(const float *a, const float *b, float *out, size_t n) {
    const size_t i = size_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i < n) out[i] = a[i] + b[i];
}

__global__ void __launch_bounds__(kThreads) head_logits_kernel(const float *__restrict__ n,
                                                               const float *__restrict__ E,
                                                               float *__restrict__ logits, int rows, int W, int V) {
    const size_t i = size_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= size_t(rows) * V) return;
    const size_t r = i / V, t = i % V;
    const float *a = n + r * W, *b = E + t * W;
    float acc = 0.0f;
    for (int c = 0; c < W; ++c) acc = fmaf(a[c], b[c], acc);
    logits[i] = acc;
}

__global__ void __launch_bounds__(kThreads) cross_entropy_kernel(const float *__restrict__ logits,
                                                                 const uint32_t *__restrict__ targets,
                                                                 float *__restrict__ dlogits, float *__restrict__ loss,
                                                                 int rows, int V, int supervised) {
    const int r = blockIdx.x * kThreads + threadIdx.x;
    if (r >= rows) return;
    const float *row = logits + size_t(r) * V;
    float *out = dlogits + size_t(r) * V;
    const uint32_t target = targets[r];
    if (target == 0xFFFFFFFFu) {
        for (int t = 0; t < V; ++t) out[t] = 0.0f;
        loss[r] = 0.0f;
        return;
    }
    float maximum = -INFINITY;
    for (int t = 0; t < V; ++t) maximum = fmaxf(maximum, row[t]);
    float sum = 0.0f;
    for (int t = 0; t < V; ++t) {
        out[t] = expf(row[t] - maximum);
        sum += out[t];
    }
    loss[r] = logf(sum) + maximum - row[target];
    const float scale = 1.0f / float(supervised);
    for (int t = 0; t < V; ++t) out[t] = (out[t] / sum - (uint32_t(t) == target ? 1.0f : 0.0f)) * scale;
}

__global__ void __launch_bounds__(kThreads) head_backward_kernel(const float *__restrict__ dlogits,
                                                                 const float *__restrict__ E, float *__restrict__ dn,
                                                                 int rows, int W, int V) {
    const size_t i = size_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= size_t(rows) * W) return;
    const size_t r = i / W, c = i % W;
    const float *g = dlogits + r * V;
    float acc = 0.0f;
    for (int t = 0; t < V; ++t) acc = fmaf(g[t], E[size_t(t) * W + c], acc);
    dn[i] = acc;
}

__global__ void __launch_bounds__(kThreads) embedding_gradient_kernel(const float *__restrict__ dlogits,
                                                                      const float *__restrict__ n,
                                                                      const uint32_t *__restrict__ tokens,
                                                                      const float *__restrict__ dx,
                                                                      float *__restrict__ dE, int rows, int W,
                                                                      int V) {
    const size_t i = size_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= size_t(V) * W) return;
    const size_t t = i / W, c = i % W;
    float acc = 0.0f;
    for (int r = 0; r < rows; ++r) {
        acc = fmaf(dlogits[size_t(r) * V + t], n[size_t(r) * W + c], acc);
        if (tokens[r] == t) acc += dx[size_t(r) * W + c];
    }
    dE[i] = acc;
}

__global__ void __launch_bounds__(kThreads) adam_kernel(float *__restrict__ params, float *__restrict__ m,
                                                        float *__restrict__ v, const float *__restrict__ grad,
                                                        size_t begin, size_t end, AdamW o) {
    const size_t i = begin + size_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= end) return;
    // The arithmetic of gpu.rs:1383-1389, unfused.
    const float g = grad[i];
    const float mi = __fadd_rn(__fmul_rn(o.beta1, m[i]), __fmul_rn(1.0f - o.beta1, g));
    const float vi = __fadd_rn(__fmul_rn(o.beta2, v[i]), __fmul_rn(__fmul_rn(1.0f - o.beta2, g), g));
    m[i] = mi;
    v[i] = vi;
    const float mh = mi / o.correction1, vh = vi / o.correction2;
    const float step = __fadd_rn(mh / __fadd_rn(sqrtf(vh), o.epsilon), __fmul_rn(o.weight_decay, params[i]));
    params[i] = __fsub_rn(params[i], __fmul_rn(o.learning_rate, step));
}

template <class F>
void by_head_width(int hd, F &&f) {
    if (hd <= 8)
        f(std::integral_constant<int, 8>{});
    else if (hd <= 16)
        f(std::integral_constant<int, 16>{});
    else if (hd <= 32)
        f(std::integral_constant<int, 32>{});
    else if (hd <= 64)
        f(std::integral_constant<int, 64>{});
    else
        f(std::integral_constant<int, 128>{});
}

}  // namespace

void mesh_forward(const Mesh &m, const float *in, float *stack, const float *w, int rows, hipStream_t stream) {
    const int threads = block_for(m.W);
    const unsigned grid = unsigned(std::min(rows, 2048));
    hipLaunchKernelGGL(mesh_forward_kernel, dim3(grid), dim3(threads), 2 * m.W * sizeof(float), stream, m, in,
                       stack, w, rows);
}

size_t mesh_partial_floats(const Mesh &m, int rows) {
    return size_t(mesh_groups(m, rows)) * m.depth * m.W * 2;
}

void mesh_backward(const Mesh &m, const float *in, const float *stack, const float *dout, float *din,
                   bool accumulate, const float *w, float *partials, float *grad, int rows, hipStream_t stream) {
    const int groups = mesh_groups(m, rows), threads = block_for(m.W);
    hipLaunchKernelGGL(mesh_backward_kernel, dim3(groups), dim3(threads), m.W * sizeof(float), stream, m, in, stack,
                       dout, din, int(accumulate), w, partials, rows);
    const int n = m.depth * m.W * 2;
    hipLaunchKernelGGL(mesh_reduce_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, stream, partials, groups, n, grad);
}

void rmsnorm_forward(const float *x, float *y, float *inv, int rows, int W, int groups, hipStream_t stream) {
    const size_t n = size_t(rows) * groups;
    hipLaunchKernelGGL(rmsnorm_forward_kernel, dim3(blocks_for(n * 64)), dim3(kThreads), 0, stream, x, y, inv,
                       int(n), W / groups);
}

void rmsnorm_backward(const float *x, const float *inv, const float *dy, float *dx, bool accumulate, int rows,
                      int W, int groups, hipStream_t stream) {
    const size_t n = size_t(rows) * groups;
    hipLaunchKernelGGL(rmsnorm_backward_kernel, dim3(blocks_for(n * 64)), dim3(kThreads), 0, stream, x, inv, dy, dx,
                       int(accumulate), int(n), W / groups);
}

void rope(float *x, const float2 *table, int rows, int sequence, int W, int H, bool inverse, hipStream_t stream) {
    const size_t n = size_t(rows) * H * (W / H / 2);
    hipLaunchKernelGGL(rope_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, stream, x, table, rows, sequence, W, H,
                       int(inverse));
}

void attention_forward(const float *q, const float *k, const float *v, float *y, float *lse, int rows,
                       int sequence, int W, int H, hipStream_t stream) {
    const float scale = float(1.0 / std::sqrt(double(W / H)));
    by_head_width(W / H, [&](auto hd) {
        hipLaunchKernelGGL(attention_forward_kernel<decltype(hd)::value>, dim3(blocks_for(size_t(rows) * H)),
                           dim3(kThreads), 0, stream, q, k, v, y, lse, rows, sequence, W, H, scale);
    });
}

void attention_backward(const float *q, const float *k, const float *v, const float *y, const float *lse,
                        const float *dy, float *dq, float *dk, float *dv, float *dsum, int rows, int sequence, int W,
                        int H, hipStream_t stream) {
    const float scale = float(1.0 / std::sqrt(double(W / H)));
    by_head_width(W / H, [&](auto hd) {
        constexpr int HD = decltype(hd)::value;
        hipLaunchKernelGGL(attention_dq_kernel<HD>, dim3(blocks_for(size_t(rows) * H)), dim3(kThreads), 0, stream, q,
                           k, v, y, lse, dy, dq, dsum, rows, sequence, W, H, scale);
        hipLaunchKernelGGL(attention_dkv_kernel<HD>, dim3(blocks_for(size_t(rows) * H)), dim3(kThreads), 0, stream,
                           q, k, v, lse, dy, dsum, dk, dv, rows, sequence, W, H, scale);
    });
}

void xsa_forward(const float *y, const float *v, float *z, int rows, int W, int H, hipStream_t stream) {
    by_head_width(W / H, [&](auto hd) {
        hipLaunchKernelGGL(xsa_forward_kernel<decltype(hd)::value>, dim3(blocks_for(size_t(rows) * H)),
                           dim3(kThreads), 0, stream, y, v, z, rows, W, H);
    });
}

void xsa_backward(const float *y, const float *v, const float *dz, float *dy, float *dv, int rows, int W, int H,
                  hipStream_t stream) {
    by_head_width(W / H, [&](auto hd) {
        hipLaunchKernelGGL(xsa_backward_kernel<decltype(hd)::value>, dim3(blocks_for(size_t(rows) * H)),
                           dim3(kThreads), 0, stream, y, v, dz, dy, dv, rows, W, H);
    });
}

void gather(const float *E, const uint32_t *tokens, float *x, int rows, int W, hipStream_t stream) {
    hipLaunchKernelGGL(gather_kernel, dim3(blocks_for(size_t(rows) * W)), dim3(kThreads), 0, stream, E, tokens, x,
                       rows, W);
}

void add(const float *a, const float *b, float *out, size_t n, hipStream_t stream) {
    hipLaunchKernelGGL(add_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, stream, a, b, out, n);
}

void head_logits(const float *n, const float *E, float *logits, int rows, int W, int V, hipStream_t stream) {
    hipLaunchKernelGGL(head_logits_kernel, dim3(blocks_for(size_t(rows) * V)), dim3(kThreads), 0, stream, n, E,
                       logits, rows, W, V);
}

void cross_entropy(const float *logits, const uint32_t *targets, float *dlogits, float *loss, int rows, int V,
                   int supervised, hipStream_t stream) {
    hipLaunchKernelGGL(cross_entropy_kernel, dim3(blocks_for(rows)), dim3(kThreads), 0, stream, logits, targets,
                       dlogits, loss, rows, V, supervised);
}

void head_backward(const float *dlogits, const float *E, float *dn, int rows, int W, int V, hipStream_t stream) {
    hipLaunchKernelGGL(head_backward_kernel, dim3(blocks_for(size_t(rows) * W)), dim3(kThreads), 0, stream, dlogits,
                       E, dn, rows, W, V);
}

void embedding_gradient(const float *dlogits, const float *n, const uint32_t *tokens, const float *dx, float *dE,
                        int rows, int W, int V, hipStream_t stream) {
    hipLaunchKernelGGL(embedding_gradient_kernel, dim3(blocks_for(size_t(V) * W)), dim3(kThreads), 0, stream,
                       dlogits, n, tokens, dx, dE, rows, W, V);
}

void adam(float *params, float *m, float *v, const float *grad, size_t begin, size_t end, const AdamW &o,
          hipStream_t stream) {
    if (end <= begin) return;
    hipLaunchKernelGGL(adam_kernel, dim3(blocks_for(end - begin)), dim3(kThreads), 0, stream, params, m, v, grad,
                       begin, end, o);
}

}  // namespace meshgpt::kern::train
