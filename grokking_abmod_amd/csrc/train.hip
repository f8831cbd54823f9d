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

// Up to kMaxSet stacks of one shape in one launch, stack blockIdx.y reading
// its own input and weights.
struct MeshSet {
    const float *in[kMaxSet];
    float *stack[kMaxSet];
    const float *w[kMaxSet];
};
struct MeshGradSet {
    const float *in[kMaxSet], *stack[kMaxSet], *dout[kMaxSet], *w[kMaxSet];
    float *din[kMaxSet], *partials[kMaxSet];
};

// Up to kMaxReduce reductions in one launch, reduction blockIdx.y summing
// groups[y] partial rows of n[y] floats.
constexpr int kMaxReduce = 16;
struct ReduceSet {
    const float *part[kMaxReduce];
    float *out[kMaxReduce];
    int groups[kMaxReduce], n[kMaxReduce];
};
// QK-Norm and RoPE of q and k in one launch: out[i] (the gradient rows, in
// place, for the backward) from the pre-norm rows pre[i], factors inv[i].
struct QkSet {
    const float *pre[kMaxSet];
    float *out[kMaxSet];
    float *inv[kMaxSet];
};

constexpr float kRmsEps = 1e-5f;                                         // src/gpt/mod.rs:38
constexpr float kXsaFloor = float(double(1e-12f) * double(1e-12f));      // XSA_EPSILON^2
constexpr int kThreads = 256;
constexpr int kRowThreads = 64;  // per-(row, head) kernels: one wave per workgroup spreads few rows widely

__device__ __forceinline__ float elu(float z) { return z >= 0.0f ? z : expm1f(z); }

__device__ __forceinline__ int stride_of(const Mesh &m, int l) {
    return m.butterfly ? 1 << ((m.layer0 + l) % m.log2w) : 1;
}

// Whether layer l of a launch applies the ELU (every layer but the stack's last).
__device__ __forceinline__ bool elu_layer(const Mesh &m, int l) { return l + 1 < m.depth || !m.linear_top; }

int block_for(int W) { return std::max(64, (W + 63) / 64 * 64); }

unsigned blocks_for(size_t n, int threads = kThreads) { return unsigned((n + threads - 1) / threads); }

// ---- mesh stacks

__global__ void __launch_bounds__(kMaxWidth) mesh_forward_kernel(Mesh m, MeshSet set, int rows) {
    extern __shared__ float buf[];  // two rows: the layer's input and output
    const float *__restrict__ in = set.in[blockIdx.y];
    float *__restrict__ stack = set.stack[blockIdx.y];
    const float *__restrict__ w = set.w[blockIdx.y];
    const int c = threadIdx.x, W = m.W;
    for (int r = blockIdx.x; r < rows; r += gridDim.x) {
        float *cur = buf, *nxt = buf + W;
        if (c < W) cur[c] = in[size_t(r) * W + c];
        __syncthreads();
        for (int l = 0; l < m.depth; ++l) {
            if (c < W) {
                int p = c + stride_of(m, l);
                if (p >= W) p -= W;
                const float2 wl = reinterpret_cast<const float2 *>(w + size_t(l) * 2 * W)[c];
                float z = cur[c] * wl.x + cur[p] * wl.y;
                if (elu_layer(m, l)) z = elu(z);
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

// Rows per workgroup of the mesh backward: sub-blocks of SUB = W rounded up to
// 64 threads, one row each, kMaxWidth threads in all.
__host__ __device__ inline int mesh_sub(int W) { return (W + 63) / 64 * 64; }
__host__ __device__ inline int mesh_rpb(int W) { return kMaxWidth / mesh_sub(W); }

// Sub-block k of workgroup g takes rows (g + j * gridDim.x) * RPB + k; thread
// c of it carries d loss / d (channel c) down the layers and adds its two
// weights' gradients over its rows in registers.  At the end the sub-blocks'
// sums are added in LDS (in sub-block order) into the workgroup's partial.
__global__ void __launch_bounds__(kMaxWidth) mesh_backward_kernel(Mesh m, MeshGradSet set, int accumulate,
                                                                  int rows) {
    extern __shared__ float lds[];  // RPB rows of dz, then RPB x W x 2 sums
    const float *__restrict__ in = set.in[blockIdx.y];
    const float *__restrict__ stack = set.stack[blockIdx.y];
    const float *__restrict__ dout = set.dout[blockIdx.y];
    float *din = set.din[blockIdx.y];
    const float *__restrict__ w = set.w[blockIdx.y];
    float *__restrict__ partials = set.partials[blockIdx.y];
    const int W = m.W, depth = m.depth, SUB = mesh_sub(W), RPB = mesh_rpb(W);
    const int sub = threadIdx.x / SUB, c = threadIdx.x % SUB;
    float *dz_row = lds + sub * W;
    float gs[kMaxDepth], gp[kMaxDepth];
#pragma unroll
    for (int l = 0; l < kMaxDepth; ++l) gs[l] = gp[l] = 0.0f;
    for (int base = blockIdx.x * RPB; base < rows; base += gridDim.x * RPB) {
        const int r = base + sub;
        const bool live = sub < RPB && r < rows && c < W;
        float g = live ? dout[size_t(r) * W + c] : 0.0f;
        // Every layer's input (own channel and partner) and output for this
        // row, loaded at once: the layer chain below waits on none of them.
        float xs[kMaxDepth], xp[kMaxDepth], act[kMaxDepth];
#pragma unroll
        for (int l = 0; l < kMaxDepth; ++l) {
            xs[l] = xp[l] = act[l] = 0.0f;
            if (l >= depth || !live) continue;
            const float *x = l == 0 ? in + size_t(r) * W : stack + (size_t(l - 1) * rows + r) * W;
            int p = c + stride_of(m, l);
            if (p >= W) p -= W;
            xs[l] = x[c];
            xp[l] = x[p];
            if (elu_layer(m, l)) act[l] = stack[(size_t(l) * rows + r) * W + c];
        }
#pragma unroll
        for (int l = kMaxDepth - 1; l >= 0; --l) {
            if (l >= depth) continue;
            const int s = stride_of(m, l);
            if (live) {
                // ELU'(z) from its output a: 1 for a >= 0, else exp(z) = a + 1.
                const float dz = elu_layer(m, l) && act[l] < 0.0f ? g * (act[l] + 1.0f) : g;
                gs[l] = fmaf(dz, xs[l], gs[l]);
                gp[l] = fmaf(dz, xp[l], gp[l]);
                dz_row[c] = dz;
            }
            __syncthreads();
            if (live) {
                // Channel c feeds itself (weight 2c) and channel c - s (weight 2(c - s) + 1).
                int q = c - s;
                if (q < 0) q += W;
                const float *wl = w + size_t(l) * 2 * W;
                g = dz_row[c] * wl[2 * c] + dz_row[q] * wl[2 * q + 1];
            }
            __syncthreads();
        }
        if (live && din) {
            const size_t i = size_t(r) * W + c;
            din[i] = accumulate ? din[i] + g : g;
        }
    }
    float *sums = lds + RPB * W;
#pragma unroll
    for (int l = 0; l < kMaxDepth; ++l) {
        if (l >= depth) continue;
        if (sub < RPB && c < W) {
            sums[(sub * W + c) * 2] = gs[l];
            sums[(sub * W + c) * 2 + 1] = gp[l];
        }
        __syncthreads();
        for (int i = threadIdx.x; i < 2 * W; i += kMaxWidth) {
            float acc = 0.0f;
            for (int k = 0; k < RPB; ++k) acc += sums[k * 2 * W + i];
            partials[(size_t(blockIdx.x) * depth + l) * 2 * W + i] = acc;
        }
        __syncthreads();
    }
}

// out[i] = sum over g < groups of part[g * n + i], in g order per wave and
// the waves' sums in wave order: 64 outputs per workgroup, wave k of its 16
// adding groups k, k + 16, ...
__global__ void __launch_bounds__(1024) reduce_groups_kernel(ReduceSet set) {
    __shared__ float sums[16][64];
    const float *__restrict__ part = set.part[blockIdx.y];
    float *__restrict__ out = set.out[blockIdx.y];
    const int groups = set.groups[blockIdx.y], n = set.n[blockIdx.y];
    if (int(blockIdx.x) * 64 >= n) return;  // the whole workgroup: a shorter reduction of the set
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, i = blockIdx.x * 64 + lane;
    float acc = 0.0f;
    if (i < n)
        for (int g = wave; g < groups; g += 16) acc += part[size_t(g) * n + i];
    sums[wave][lane] = acc;
    __syncthreads();
    if (wave == 0 && i < n) {
        float t = 0.0f;
        for (int k = 0; k < 16; ++k) t += sums[k][lane];
        out[i] = t;
    }
}

int mesh_groups(const Mesh &m, int rows) {
    const int rpb = mesh_rpb(m.W);
    return std::max(1, std::min((rows + rpb - 1) / rpb, 256));
}

// ---- mesh stacks of width <= 64 or 128: one wave per row, channel
// lane + 64 j in register j, partners by lane shuffles (no barriers).

// Lane l gets v of lane (l + 1) mod 64 (DPP wave_rol:1) or of lane (l - 1)
// mod 64 (DPP wave_ror:1): no LDS round trip.
__device__ __forceinline__ float lanes_rol1(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x134, 0xf, 0xf, false));
}
__device__ __forceinline__ float lanes_ror1(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x13C, 0xf, 0xf, false));
}

// out[j] = the value of channel (lane + 64 j + d) mod W, for 0 <= d < W.
// Width 128 (CPL 2): a shift by 64 + d' renames the registers and shifts by
// d'; for d' < 64 every lane reads lane (lane + d') mod 64, whose lanes below
// d' offer their other register (their readers wrapped past lane 63), one lane
// read per register, a DPP rotation for d' = 1 or 63 (the neighbour mesh and
// its backward).
template <int CPL>
__device__ __forceinline__ void channel_shift(const float (&x)[CPL], int d, int W, int lane, float (&out)[CPL]) {
    static_assert(CPL == 1 || CPL == 2, "wave mesh kernels take widths up to 128");
    if constexpr (CPL == 1) {
        if (W == 64 && d == 1) {
            out[0] = lanes_rol1(x[0]);
        } else if (W == 64 && d == 63) {
            out[0] = lanes_ror1(x[0]);
        } else {
            int src = lane + d;
            if (src >= W) src -= W;
            out[0] = __shfl(x[0], src & 63, 64);
        }
    } else {
        const bool swap = d >= 64;
        const float y0 = swap ? x[1] : x[0], y1 = swap ? x[0] : x[1];
        d &= 63;
        if (d == 0) {
            out[0] = y0;
            out[1] = y1;
            return;
        }
        const bool next = lane < d;
        const float o0 = next ? y1 : y0, o1 = next ? y0 : y1;
        if (d == 1) {
            out[0] = lanes_rol1(o0);
            out[1] = lanes_rol1(o1);
        } else if (d == 63) {
            out[0] = lanes_ror1(o0);
            out[1] = lanes_ror1(o1);
        } else {
            const int src = (lane + d) & 63;
            out[0] = __shfl(o0, src, 64);
            out[1] = __shfl(o1, src, 64);
        }
    }
}

constexpr int kMeshWaveRows = 2;  // rows per wave of the wave-per-row mesh backward

// D: the layers a launch may hold (registers are sized for it; the launch's
// own depth is at most D).
// With NORM the stacks' input is RMSNorm(a + b) (b optional) of each row,
// formed here with the arithmetic of rmsnorm_forward_kernel; stack 0 stores the
// sum, the normalised row and its factor.
// With qk.out[0] set, stacks 0 and 1 (Q and K) also get QK-Norm and slice RoPE
// of their last layer, per head of hd = W / H lanes (hd a power of two up to
// 64 within a register, or all 128 channels), stored to qk.out[y] with the
// norm factors in qk.inv[y] (qk_forward_kernel's operations; the head sums
// by lane exchanges).
template <int CPL, int D, bool NORM>
__global__ void __launch_bounds__(kThreads) mesh_forward_wave(Mesh m, MeshSet set, NormIn ni, QkOut qk, int rows) {
    const float *__restrict__ in = set.in[blockIdx.y];
    float *__restrict__ stack = set.stack[blockIdx.y];
    const float *__restrict__ w = set.w[blockIdx.y];
    const int lane = threadIdx.x & 63, W = m.W;
    const int wave = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6), waves = gridDim.x * (kThreads / 64);
    // The stack's weights of this lane's channels, loaded once.
    float2 wt[D][CPL];
#pragma unroll
    for (int l = 0; l < D; ++l)
#pragma unroll
        for (int j = 0; j < CPL; ++j)
            wt[l][j] = l < m.depth && lane + 64 * j < W
                           ? reinterpret_cast<const float2 *>(w + size_t(l) * 2 * W)[lane + 64 * j]
                           : make_float2(0.0f, 0.0f);
    for (int r = wave; r < rows; r += waves) {
        float x[CPL];
        if constexpr (NORM) {
            const bool first = blockIdx.y == 0;
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const int c = lane + 64 * j;
                const size_t i = size_t(r) * W + c;
                x[j] = c < W ? (ni.b ? ni.a[i] + ni.b[i] : ni.a[i]) : 0.0f;
                acc = fmaf(x[j], x[j], acc);
                if (first && ni.b && c < W) ni.sum[i] = x[j];
            }
            const float iv = rsqrtf(wave_sum(acc) * (1.0f / float(W)) + kRmsEps);
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const int c = lane + 64 * j;
                x[j] *= iv;
                if (first && c < W) ni.n[size_t(r) * W + c] = x[j];
            }
            if (first && lane == 0) ni.inv[r] = iv;
        } else {
#pragma unroll
            for (int j = 0; j < CPL; ++j) x[j] = lane + 64 * j < W ? in[size_t(r) * W + lane + 64 * j] : 0.0f;
        }
#pragma unroll
        for (int l = 0; l < D; ++l) {
            if (l >= m.depth) continue;
            float p[CPL];
            channel_shift(x, stride_of(m, l), W, lane, p);
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const int c = lane + 64 * j;
                float z = x[j] * wt[l][j].x + p[j] * wt[l][j].y;
                if (elu_layer(m, l)) z = elu(z);
                x[j] = z;
                if (c < W) stack[(size_t(l) * rows + r) * W + c] = z;
            }
        }
        if (qk.out[0] && blockIdx.y < 2) {
            const int y = blockIdx.y, hd = W / qk.H, half = hd / 2;
            if (qk.norm) {
                float sq[CPL];
#pragma unroll
                for (int j = 0; j < CPL; ++j) sq[j] = x[j] * x[j];
                if (hd <= 64) {
                    for (int off = hd / 2; off >= 1; off >>= 1)
#pragma unroll
                        for (int j = 0; j < CPL; ++j) sq[j] += __shfl_xor(sq[j], off, 64);
                } else {
                    float t = 0.0f;
#pragma unroll
                    for (int j = 0; j < CPL; ++j) t += sq[j];
                    for (int off = 32; off >= 1; off >>= 1) t += __shfl_xor(t, off, 64);
#pragma unroll
                    for (int j = 0; j < CPL; ++j) sq[j] = t;
                }
#pragma unroll
                for (int j = 0; j < CPL; ++j) {
                    const int c = lane + 64 * j;
                    const float iv = rsqrtf(sq[j] * (1.0f / float(hd)) + kRmsEps);
                    x[j] *= iv;
                    if (c < W && c % hd == 0) qk.inv[y][size_t(r) * qk.H + c / hd] = iv;
                }
            }
            if (qk.rotate) {
                float o[CPL];
                if (hd <= 64) {
#pragma unroll
                    for (int j = 0; j < CPL; ++j) o[j] = __shfl_xor(x[j], half, 64);
                } else {
#pragma unroll
                    for (int j = 0; j < CPL; ++j) o[j] = x[(j + 1) % CPL];
                }
                const float2 *row = qk.table + size_t(r % qk.sequence) * half;
#pragma unroll
                for (int j = 0; j < CPL; ++j) {
                    const int d = (lane + 64 * j) % hd;
                    const float2 cs = row[d < half ? d : d - half];
                    x[j] = d < half ? x[j] * cs.x - o[j] * cs.y : x[j] * cs.x + o[j] * cs.y;
                }
            }
#pragma unroll
            for (int j = 0; j < CPL; ++j)
                if (lane + 64 * j < W) qk.out[y][size_t(r) * W + lane + 64 * j] = x[j];
        }
    }
}

// One row's layer inputs and outputs in a wave's registers (the backward's
// operands, loaded at once so that the layer chain waits only on lane shifts).
template <int CPL, int D, bool NORMB>
struct MeshRowSaved {
    float g[CPL], xin[D][CPL], act[D][CPL];
    float xr[NORMB ? CPL : 1], iv = 0.0f;  // the norm's input row and factor (NORMB)
    __device__ __forceinline__ void load(const Mesh &m, const float *__restrict__ in, const float *__restrict__ stack,
                                         const float *dout, const NormGrad &ng, int r, int rows, int lane) {
        const int W = m.W;
#pragma unroll
        for (int j = 0; j < CPL; ++j) g[j] = lane + 64 * j < W ? dout[size_t(r) * W + lane + 64 * j] : 0.0f;
        if constexpr (NORMB) {
#pragma unroll
            for (int j = 0; j < CPL; ++j) xr[j] = lane + 64 * j < W ? ng.x[size_t(r) * W + lane + 64 * j] : 0.0f;
            iv = ng.inv[r];
        }
#pragma unroll
        for (int l = 0; l < D; ++l)
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const int c = lane + 64 * j;
                const bool ok = l < m.depth && c < W;
                const float *x = l == 0 ? in + size_t(r) * W : stack + (size_t(l - 1) * rows + r) * W;
                xin[l][j] = ok ? x[c] : 0.0f;
                act[l][j] = ok && elu_layer(m, l) ? stack[(size_t(l) * rows + r) * W + c] : 0.0f;
            }
    }
};

// Each wave carries d loss / d (its row) down the layers, row after row (the
// next row's operands loading during the current row's chain), and adds the
// weights' gradients in registers; the workgroup's waves add theirs in LDS
// (in wave order) into the workgroup's partial.
// With NORMB the input gradient goes on through the RMSNorm in front of the
// stack (rmsnorm_backward_kernel's arithmetic): dx += iv g - x iv^3 (g . x) / W.
template <int CPL, int D, bool NORMB>
__global__ void __launch_bounds__(kThreads) mesh_backward_wave(Mesh m, MeshGradSet set, NormGrad ng, int accumulate,
                                                               int rows) {
    extern __shared__ float sums[];  // (kThreads / 64) x depth x W x 2
    const float *__restrict__ in = set.in[blockIdx.y];
    const float *__restrict__ stack = set.stack[blockIdx.y];
    // dout may be the rows NORMB adds to (each row is read before it is written).
    const float *dout = set.dout[blockIdx.y];
    float *din = set.din[blockIdx.y];
    const float *__restrict__ w = set.w[blockIdx.y];
    float *__restrict__ partials = set.partials[blockIdx.y];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, W = m.W, depth = m.depth;
    const int wave = blockIdx.x * (kThreads / 64) + wv, waves = gridDim.x * (kThreads / 64);
    // The weights of this lane's channels, loaded once, off the layer chain.
    float2 wt[D][CPL];
#pragma unroll
    for (int l = 0; l < D; ++l)
#pragma unroll
        for (int j = 0; j < CPL; ++j)
            wt[l][j] = l < depth && lane + 64 * j < W
                           ? reinterpret_cast<const float2 *>(w + size_t(l) * 2 * W)[lane + 64 * j]
                           : make_float2(0.0f, 0.0f);
    float gs[D][CPL], gp[D][CPL];
#pragma unroll
    for (int l = 0; l < D; ++l)
#pragma unroll
        for (int j = 0; j < CPL; ++j) gs[l][j] = gp[l][j] = 0.0f;
    MeshRowSaved<CPL, D, NORMB> cur;
    if (wave < rows) cur.load(m, in, stack, dout, ng, wave, rows, lane);
    for (int r = wave; r < rows; r += waves) {
        MeshRowSaved<CPL, D, NORMB> next;
        if (r + waves < rows) next.load(m, in, stack, dout, ng, r + waves, rows, lane);
        float g[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j) g[j] = cur.g[j];
#pragma unroll
        for (int l = D - 1; l >= 0; --l) {
            if (l >= depth) continue;
            const int s = stride_of(m, l);
            float x[CPL], xp[CPL], dz[CPL], t[CPL], back[CPL];
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const int c = lane + 64 * j;
                x[j] = cur.xin[l][j];
                // ELU'(z) from its output a: 1 for a >= 0, else exp(z) = a + 1.
                const float d = cur.act[l][j] < 0.0f ? g[j] * (cur.act[l][j] + 1.0f) : g[j];
                dz[j] = c < W ? d : 0.0f;
                t[j] = dz[j] * wt[l][j].y;
            }
            channel_shift(x, s, W, lane, xp);
            // Channel c feeds itself and channel c - s: its input gradient is
            // dz[c] w_self[c] + dz[c - s] w_partner[c - s].
            channel_shift(t, W - s, W, lane, back);
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const int c = lane + 64 * j;
                gs[l][j] = fmaf(dz[j], x[j], gs[l][j]);
                gp[l][j] = fmaf(dz[j], xp[j], gp[l][j]);
                g[j] = c < W ? dz[j] * wt[l][j].x + back[j] : 0.0f;
            }
        }
        if constexpr (NORMB) {
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < CPL; ++j) acc = fmaf(g[j], cur.xr[j], acc);
            const float iv = cur.iv, k = wave_sum(acc) * iv * iv * iv * (1.0f / float(W));
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const int c = lane + 64 * j;
                if (c >= W) continue;
                const size_t i = size_t(r) * W + c;
                ng.dx[i] += iv * g[j] - cur.xr[j] * k;
            }
        } else if (din) {
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const int c = lane + 64 * j;
                if (c >= W) continue;
                const size_t i = size_t(r) * W + c;
                din[i] = accumulate ? din[i] + g[j] : g[j];
            }
        }
        cur = next;
    }
#pragma unroll
    for (int l = 0; l < D; ++l) {
        if (l >= depth) continue;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = lane + 64 * j;
            if (c >= W) continue;
            float *o = sums + ((size_t(wv) * depth + l) * W + c) * 2;
            o[0] = gs[l][j];
            o[1] = gp[l][j];
        }
    }
    __syncthreads();
    const int n = depth * W * 2;
    for (int i = threadIdx.x; i < n; i += kThreads) {
        float acc = 0.0f;
        for (int k = 0; k < kThreads / 64; ++k) acc += sums[size_t(k) * n + i];
        partials[size_t(blockIdx.x) * n + i] = acc;
    }
}

int mesh_wave_cpl(int W) { return W <= 64 ? 1 : (W == 128 ? 2 : 0); }

int mesh_wave_groups(int rows) {
    const int per = kMeshWaveRows * (kThreads / 64);
    return std::max(1, std::min((rows + per - 1) / per, 256));
}

// ---- norms (one wave per (row, group))

// With RES the normalised row is x + b, which is also stored to `sum` (the
// residual add of the block fused into the norm that follows it).
template <bool RES>
__global__ void __launch_bounds__(kThreads) rmsnorm_forward_kernel(const float *__restrict__ x,
                                                                   const float *__restrict__ b, float *sum, float *y,
                                                                   float *__restrict__ inv, int n_groups, int gw) {
    const int wave = (blockIdx.x * kThreads + threadIdx.x) >> 6, lane = threadIdx.x & 63;
    if (wave >= n_groups) return;
    const size_t o = size_t(wave) * gw;
    auto value = [&](int i) { return RES ? x[o + i] + b[o + i] : x[o + i]; };
    float acc = 0.0f;
    for (int i = lane; i < gw; i += 64) {
        const float v = value(i);
        acc = fmaf(v, v, acc);
    }
    const float iv = rsqrtf(wave_sum(acc) * (1.0f / float(gw)) + kRmsEps);
    for (int i = lane; i < gw; i += 64) {
        const float v = value(i);
        if (RES) sum[o + i] = v;
        y[o + i] = v * iv;
    }
    if (lane == 0) inv[wave] = iv;
}

// dy is the sum of NDY gradients, added in order (dy0 + dy1) + dy2.
template <int NDY>
__global__ void __launch_bounds__(kThreads) rmsnorm_backward_kernel(const float *__restrict__ x,
                                                                    const float *__restrict__ inv, const float *dy0,
                                                                    const float *dy1, const float *dy2, float *dx,
                                                                    int accumulate, int n_groups, int gw) {
    const int wave = (blockIdx.x * kThreads + threadIdx.x) >> 6, lane = threadIdx.x & 63;
    if (wave >= n_groups) return;
    const size_t o = size_t(wave) * gw;
    auto grad = [&](int i) {
        float g = dy0[o + i];
        if (NDY > 1) g += dy1[o + i];
        if (NDY > 2) g += dy2[o + i];
        return g;
    };
    float acc = 0.0f;
    for (int i = lane; i < gw; i += 64) acc = fmaf(grad(i), x[o + i], acc);
    const float iv = inv[wave];
    const float k = wave_sum(acc) * iv * iv * iv * (1.0f / float(gw));
    for (int i = lane; i < gw; i += 64) {
        const float d = iv * grad(i) - x[o + i] * k;
        dx[o + i] = accumulate ? dx[o + i] + d : d;
    }
}

// ---- attention (one thread per (row, head); the head row in registers)

template <int HD>
__global__ void __launch_bounds__(kRowThreads) attention_forward_kernel(const float *__restrict__ q,
                                                                     const float *__restrict__ k,
                                                                     const float *__restrict__ v,
                                                                     float *__restrict__ y,
                                                                     float *__restrict__ lse, int rows,
                                                                     int sequence, int W, int H, float scale) {
    const int t = blockIdx.x * kRowThreads + threadIdx.x;
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
__global__ void __launch_bounds__(kRowThreads) attention_dq_kernel(const float *__restrict__ q,
                                                                const float *__restrict__ k,
                                                                const float *__restrict__ v,
                                                                const float *__restrict__ y,
                                                                const float *__restrict__ lse,
                                                                const float *__restrict__ dy, float *__restrict__ dq,
                                                                float *__restrict__ dsum, int rows, int sequence,
                                                                int W, int H, float scale) {
    const int t = blockIdx.x * kRowThreads + threadIdx.x;
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
__global__ void __launch_bounds__(kRowThreads) attention_dkv_kernel(const float *__restrict__ q,
                                                                 const float *__restrict__ k,
                                                                 const float *__restrict__ v,
                                                                 const float *__restrict__ lse,
                                                                 const float *__restrict__ dy,
                                                                 const float *__restrict__ dsum,
                                                                 float *__restrict__ dk, float *dv, int rows,
                                                                 int sequence, int W, int H, float scale) {
    const int t = blockIdx.x * kRowThreads + threadIdx.x;
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

// ---- one wave per (row, head), lanes over the head's dims (dim lane + 64 e)

template <int EPL>
__device__ __forceinline__ void lanes_load(const float *row, int hd, int lane, float (&v)[EPL]) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) v[e] = lane + 64 * e < hd ? row[lane + 64 * e] : 0.0f;
}

template <int EPL>
__device__ __forceinline__ void lanes_store(float *row, int hd, int lane, const float (&v)[EPL]) {
#pragma unroll
    for (int e = 0; e < EPL; ++e)
        if (lane + 64 * e < hd) row[lane + 64 * e] = v[e];
}

template <int EPL>
__device__ __forceinline__ float lanes_dot(const float (&a)[EPL], const float (&b)[EPL]) {
    float acc = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc = fmaf(a[e], b[e], acc);
    return wave_sum(acc);
}

// The RoPE partner of each lane's dims (d + half or d - half).
template <int EPL>
__device__ __forceinline__ void lanes_partner(const float (&x)[EPL], int hd, int lane, float (&out)[EPL]) {
    const int half = hd / 2;
    if (EPL > 1 && half % 64 == 0) {
        // The partner sits in the same lane, half / 64 registers away.
        const int k = half / 64;
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const int pe = 64 * e < half ? e + k : e - k;
            float v = 0.0f;
#pragma unroll
            for (int f = 0; f < EPL; ++f)
                if (f == pe) v = x[f];
            out[e] = lane + 64 * e < hd ? v : 0.0f;
        }
        return;
    }
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
        const int d = lane + 64 * e, pd = d < half ? d + half : d - half;
        float v = 0.0f;
#pragma unroll
        for (int f = 0; f < EPL; ++f) {
            const float t = __shfl(x[f], pd & 63, 64);
            if ((pd >> 6) == f) v = t;
        }
        out[e] = d < hd ? v : 0.0f;
    }
}

__device__ __forceinline__ int row_wave() { return int((blockIdx.x * kThreads + threadIdx.x) >> 6); }

// QK-Norm (per-head RMSNorm) then RoPE of row r, head h, in place; inv keeps
// the norm's factor (reference.rs:174-193, 392-409, 462-482).
template <int EPL>
__global__ void __launch_bounds__(kThreads) qk_forward_kernel(QkSet set, const float2 *__restrict__ table, int rows,
                                                              int sequence, int W, int H, int norm, int rotate) {
    float *x = set.out[blockIdx.y];
    const float *__restrict__ pre = set.pre[blockIdx.y];
    float *__restrict__ inv = set.inv[blockIdx.y];
    const int t = row_wave(), lane = threadIdx.x & 63;
    if (t >= rows * H) return;
    const int r = t / H, h = t % H, hd = W / H, half = hd / 2;
    float v[EPL];
    lanes_load(pre + size_t(r) * W + h * hd, hd, lane, v);
    if (norm) {
        const float iv = rsqrtf(lanes_dot(v, v) * (1.0f / float(hd)) + kRmsEps);
#pragma unroll
        for (int e = 0; e < EPL; ++e) v[e] *= iv;
        if (lane == 0) inv[t] = iv;
    }
    if (rotate) {
        float o[EPL];
        lanes_partner(v, hd, lane, o);
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const int d = lane + 64 * e;
            const float2 cs = table[size_t(r % sequence) * half + (d < half ? d : d - half) % max(half, 1)];
            v[e] = d < half ? v[e] * cs.x - o[e] * cs.y : v[e] * cs.x + o[e] * cs.y;
        }
    }
    lanes_store(x + size_t(r) * W + h * hd, hd, lane, v);
}

// Its backward in place on g: the transposed rotation, then the norm's
// backward against the pre-norm rows `pre`.
template <int EPL>
__global__ void __launch_bounds__(kThreads) qk_backward_kernel(QkSet set, const float2 *__restrict__ table, int rows,
                                                               int sequence, int W, int H, int norm, int rotate) {
    float *g = set.out[blockIdx.y];
    const float *__restrict__ pre = set.pre[blockIdx.y];
    const float *__restrict__ inv = set.inv[blockIdx.y];
    const int t = row_wave(), lane = threadIdx.x & 63;
    if (t >= rows * H) return;
    const int r = t / H, h = t % H, hd = W / H, half = hd / 2;
    float *row = g + size_t(r) * W + h * hd;
    float v[EPL];
    lanes_load(row, hd, lane, v);
    if (rotate) {
        float o[EPL];
        lanes_partner(v, hd, lane, o);
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const int d = lane + 64 * e;
            const float2 cs = table[size_t(r % sequence) * half + (d < half ? d : d - half) % max(half, 1)];
            v[e] = d < half ? v[e] * cs.x + o[e] * cs.y : v[e] * cs.x - o[e] * cs.y;
        }
    }
    if (norm) {
        float x[EPL];
        lanes_load(pre + size_t(r) * W + h * hd, hd, lane, x);
        const float iv = inv[t], k = lanes_dot(v, x) * iv * iv * iv * (1.0f / float(hd));
#pragma unroll
        for (int e = 0; e < EPL; ++e) v[e] = iv * v[e] - x[e] * k;
    }
    lanes_store(row, hd, lane, v);
}

// Causal attention for short sequences: one wave per query row and head.
// XSA of one (row, head) in a wave's lanes (reference.rs:577-603): y minus
// its component along u = v / max(|v|, 1e-12), in place.
template <int EPL>
__device__ __forceinline__ void lanes_xsa(float (&yv)[EPL], const float (&v)[EPL]) {
    float u[EPL];
    const float inv = rsqrtf(fmaxf(lanes_dot(v, v), kXsaFloor));
#pragma unroll
    for (int e = 0; e < EPL; ++e) u[e] = v[e] * inv;
    const float s = lanes_dot(yv, u);
#pragma unroll
    for (int e = 0; e < EPL; ++e) yv[e] -= s * u[e];
}

// Its backward from g = d loss / d z: g becomes d loss / d y = g - (g.u) u,
// and dv = inv (du - u (u.du)) above the norm floor (inv du below it) with
// du = -((y.u) g + (g.u) y).
template <int EPL>
__device__ __forceinline__ void lanes_xsa_backward(const float (&yv)[EPL], const float (&v)[EPL], float (&g)[EPL],
                                                   float (&dv)[EPL]) {
    float u[EPL];
    const float sq = lanes_dot(v, v), inv = rsqrtf(fmaxf(sq, kXsaFloor));
#pragma unroll
    for (int e = 0; e < EPL; ++e) u[e] = v[e] * inv;
    const float s = lanes_dot(yv, u), tg = lanes_dot(g, u);
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
        dv[e] = -(s * g[e] + tg * yv[e]);
        g[e] = g[e] - tg * u[e];
    }
    const float udu = sq >= kXsaFloor ? lanes_dot(u, dv) : 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) dv[e] = inv * (dv[e] - u[e] * udu);
}

// Causal attention of one (row, head) per wave, then (XSA) the exclusive
// projection against the row's own value: y and z = xsa(y) (or y) stored.
template <int EPL, bool XSA>
__global__ void __launch_bounds__(kThreads) attention_forward_wave(const float *__restrict__ q,
                                                                   const float *__restrict__ k,
                                                                   const float *__restrict__ v, float *__restrict__ y,
                                                                   float *__restrict__ z, float *__restrict__ lse,
                                                                   int rows, int sequence, int W, int H,
                                                                   float scale) {
    const int t = row_wave(), lane = threadIdx.x & 63;
    if (t >= rows * H) return;
    const int r = t / H, h = t % H, hd = W / H, pos = r % sequence, first = r - pos;
    float qr[EPL], acc[EPL] = {};
    lanes_load(q + size_t(r) * W + h * hd, hd, lane, qr);
    float m = -INFINITY, l = 0.0f;
    for (int j = 0; j <= pos; ++j) {
        float kr[EPL], vr[EPL];
        lanes_load(k + size_t(first + j) * W + h * hd, hd, lane, kr);
        lanes_load(v + size_t(first + j) * W + h * hd, hd, lane, vr);
        const float s = lanes_dot(qr, kr) * scale;
        const float mn = fmaxf(m, s), alpha = expf(m - mn), p = expf(s - mn);
        l = l * alpha + p;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[e] = fmaf(p, vr[e], acc[e] * alpha);
        m = mn;
    }
    const float il = 1.0f / l;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] *= il;
    const size_t o = size_t(r) * W + h * hd;
    lanes_store(y + o, hd, lane, acc);
    if (lane == 0) lse[t] = m + logf(l);
    if (XSA) {
        float vs[EPL];
        lanes_load(v + o, hd, lane, vs);
        lanes_xsa(acc, vs);
    }
    lanes_store(z + o, hd, lane, acc);
}

// From dz = d loss / d z: (XSA) its backward first, storing dy and the XSA's
// part of dv; without XSA dy is dz and dv starts at zero.  Then dq and the
// row's dy . y (dsum), which the key-side kernel needs.
template <int EPL, bool XSA>
__global__ void __launch_bounds__(kThreads) attention_dq_wave(const float *__restrict__ q, const float *__restrict__ k,
                                                              const float *__restrict__ v, const float *__restrict__ y,
                                                              const float *__restrict__ lse,
                                                              const float *__restrict__ dz, float *__restrict__ dy,
                                                              float *__restrict__ dv, float *__restrict__ dq,
                                                              float *__restrict__ dsum, int rows, int sequence, int W,
                                                              int H, float scale) {
    const int t = row_wave(), lane = threadIdx.x & 63;
    if (t >= rows * H) return;
    const int r = t / H, h = t % H, hd = W / H, pos = r % sequence, first = r - pos;
    const size_t o = size_t(r) * W + h * hd;
    float qr[EPL], g[EPL], yv[EPL], acc[EPL] = {};
    lanes_load(q + o, hd, lane, qr);
    lanes_load(dz + o, hd, lane, g);
    lanes_load(y + o, hd, lane, yv);
    float dvs[EPL] = {};
    if (XSA) {
        float vs[EPL];
        lanes_load(v + o, hd, lane, vs);
        lanes_xsa_backward(yv, vs, g, dvs);
        lanes_store(dy + o, hd, lane, g);
    }
    lanes_store(dv + o, hd, lane, dvs);
    const float D = lanes_dot(g, yv), L = lse[t];
    for (int j = 0; j <= pos; ++j) {
        float kr[EPL], vr[EPL];
        lanes_load(k + size_t(first + j) * W + h * hd, hd, lane, kr);
        lanes_load(v + size_t(first + j) * W + h * hd, hd, lane, vr);
        const float ds = expf(lanes_dot(qr, kr) * scale - L) * (lanes_dot(g, vr) - D);
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[e] = fmaf(ds, kr[e], acc[e]);
    }
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] *= scale;
    lanes_store(dq + o, hd, lane, acc);
    if (lane == 0) dsum[t] = D;
}

template <int EPL>
__global__ void __launch_bounds__(kThreads) attention_dkv_wave(const float *__restrict__ q,
                                                               const float *__restrict__ k,
                                                               const float *__restrict__ v,
                                                               const float *__restrict__ lse,
                                                               const float *__restrict__ dy,
                                                               const float *__restrict__ dsum, float *__restrict__ dk,
                                                               float *dv, int rows, int sequence, int W, int H,
                                                               float scale) {
    const int t = row_wave(), lane = threadIdx.x & 63;
    if (t >= rows * H) return;
    const int j = t / H, h = t % H, hd = W / H, pos = j % sequence, last = j - pos + sequence;
    const size_t o = size_t(j) * W + h * hd;
    float kr[EPL], vr[EPL], ak[EPL] = {}, av[EPL] = {};
    lanes_load(k + o, hd, lane, kr);
    lanes_load(v + o, hd, lane, vr);
    for (int i = j; i < last; ++i) {
        float qi[EPL], gi[EPL];
        lanes_load(q + size_t(i) * W + h * hd, hd, lane, qi);
        lanes_load(dy + size_t(i) * W + h * hd, hd, lane, gi);
        const float p = expf(lanes_dot(qi, kr) * scale - lse[size_t(i) * H + h]);
        const float ds = p * (lanes_dot(gi, vr) - dsum[size_t(i) * H + h]);
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            av[e] = fmaf(p, gi[e], av[e]);
            ak[e] = fmaf(ds, qi[e], ak[e]);
        }
    }
    float old[EPL];
    lanes_load(dv + o, hd, lane, old);
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
        ak[e] *= scale;
        old[e] += av[e];
    }
    lanes_store(dk + o, hd, lane, ak);
    lanes_store(dv + o, hd, lane, old);
}

// The whole attention backward of short sequences in one launch: waves of
// blockIdx.y = 0 take a query row each (dq, as attention_dq_wave), waves of
// blockIdx.y = 1 a key row each (dk and dv, as attention_dkv_wave), which
// form each later query's XSA backward and dy . y themselves instead of
// waiting for the query waves: the same arithmetic on the same operands.
template <int EPL, bool XSA>
__global__ void __launch_bounds__(kThreads) attention_backward_wave(const float *__restrict__ q,
                                                                    const float *__restrict__ k,
                                                                    const float *__restrict__ v,
                                                                    const float *__restrict__ y,
                                                                    const float *__restrict__ lse,
                                                                    const float *__restrict__ dz,
                                                                    float *__restrict__ dq, float *__restrict__ dk,
                                                                    float *__restrict__ dv, int rows, int sequence,
                                                                    int W, int H, float scale) {
    const int t = row_wave(), lane = threadIdx.x & 63;
    if (t >= rows * H) return;
    const int r = t / H, h = t % H, hd = W / H, pos = r % sequence, first = r - pos;
    // d loss / d y of row i (XSA's backward when on) and its dy . y.
    auto output_grad = [&](int i, float (&g)[EPL], float (&dvs)[EPL]) {
        const size_t oi = size_t(i) * W + h * hd;
        float yv[EPL];
        lanes_load(dz + oi, hd, lane, g);
        lanes_load(y + oi, hd, lane, yv);
#pragma unroll
        for (int e = 0; e < EPL; ++e) dvs[e] = 0.0f;
        if (XSA) {
            float vs[EPL];
            lanes_load(v + oi, hd, lane, vs);
            lanes_xsa_backward(yv, vs, g, dvs);
        }
        return lanes_dot(g, yv);
    };
    const size_t o = size_t(r) * W + h * hd;
    if (blockIdx.y == 0) {
        float qr[EPL], g[EPL], dvs[EPL], acc[EPL] = {};
        lanes_load(q + o, hd, lane, qr);
        const float D = output_grad(r, g, dvs), L = lse[t];
        for (int j = 0; j <= pos; ++j) {
            float kr[EPL], vr[EPL];
            lanes_load(k + size_t(first + j) * W + h * hd, hd, lane, kr);
            lanes_load(v + size_t(first + j) * W + h * hd, hd, lane, vr);
            const float ds = expf(lanes_dot(qr, kr) * scale - L) * (lanes_dot(g, vr) - D);
#pragma unroll
            for (int e = 0; e < EPL; ++e) acc[e] = fmaf(ds, kr[e], acc[e]);
        }
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[e] *= scale;
        lanes_store(dq + o, hd, lane, acc);
        return;
    }
    const int last = first + sequence;
    float kr[EPL], vr[EPL], ak[EPL] = {}, av[EPL] = {}, own[EPL];
    lanes_load(k + o, hd, lane, kr);
    lanes_load(v + o, hd, lane, vr);
    {
        float g[EPL];
        output_grad(r, g, own);  // this row's own XSA part of dv
    }
    for (int i = r; i < last; ++i) {
        float qi[EPL], gi[EPL], unused[EPL];
        lanes_load(q + size_t(i) * W + h * hd, hd, lane, qi);
        const float D = output_grad(i, gi, unused);
        const float p = expf(lanes_dot(qi, kr) * scale - lse[size_t(i) * H + h]);
        const float ds = p * (lanes_dot(gi, vr) - D);
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            av[e] = fmaf(p, gi[e], av[e]);
            ak[e] = fmaf(ds, qi[e], ak[e]);
        }
    }
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
        ak[e] *= scale;
        own[e] += av[e];
    }
    lanes_store(dk + o, hd, lane, ak);
    lanes_store(dv + o, hd, lane, own);
}

template <int EPL>
__global__ void __launch_bounds__(kThreads) xsa_forward_wave(const float *__restrict__ y, const float *__restrict__ v,
                                                             float *__restrict__ z, int rows, int W, int H) {
    const int t = row_wave(), lane = threadIdx.x & 63;
    if (t >= rows * H) return;
    const int hd = W / H;
    const size_t o = size_t(t / H) * W + (t % H) * hd;
    float yv[EPL], vs[EPL];
    lanes_load(y + o, hd, lane, yv);
    lanes_load(v + o, hd, lane, vs);
    lanes_xsa(yv, vs);
    lanes_store(z + o, hd, lane, yv);
}

template <int EPL>
__global__ void __launch_bounds__(kThreads) xsa_backward_wave(const float *__restrict__ y, const float *__restrict__ v,
                                                              const float *__restrict__ dz, float *__restrict__ dy,
                                                              float *__restrict__ dv, int rows, int W, int H) {
    const int t = row_wave(), lane = threadIdx.x & 63;
    if (t >= rows * H) return;
    const int hd = W / H;
    const size_t o = size_t(t / H) * W + (t % H) * hd;
    float yv[EPL], vs[EPL], g[EPL], d[EPL];
    lanes_load(y + o, hd, lane, yv);
    lanes_load(v + o, hd, lane, vs);
    lanes_load(dz + o, hd, lane, g);
    lanes_xsa_backward(yv, vs, g, d);
    lanes_store(dy + o, hd, lane, g);
    lanes_store(dv + o, hd, lane, d);
}

template <class F>
void by_lanes(int hd, F &&f) {
    if (hd <= 64)
        f(std::integral_constant<int, 1>{});
    else if (hd <= 128)
        f(std::integral_constant<int, 2>{});
    else if (hd <= 256)
        f(std::integral_constant<int, 4>{});
    else if (hd <= 512)
        f(std::integral_constant<int, 8>{});
    else
        f(std::integral_constant<int, 16>{});
}

// Sequences up to this length take the wave-per-row attention kernels; longer
// ones the thread-per-row kernels, whose key loops do 64 rows' work per wave
// (head widths up to 128; wider heads always take the wave kernels).
constexpr int kWaveAttentionMax = 64;
// Sequences up to this length run the attention backward as one launch, whose
// key waves redo the later queries' XSA backward (a few rows each).
constexpr int kMergedBackwardMax = 8;

// ---- embedding geometry (reference.rs:130-149): rows scaled to the radius,
// then protected coordinates replaced by their codes.  One wave per token.

__global__ void __launch_bounds__(kThreads) geometry_forward_kernel(const float *__restrict__ raw,
                                                                    const float *__restrict__ codes,
                                                                    float *__restrict__ out, float *__restrict__ rinv,
                                                                    int V, int W, float radius, int normalize,
                                                                    int preserve) {
    const int t = row_wave(), lane = threadIdx.x & 63;
    if (t >= V) return;
    const float *x = raw + size_t(t) * W;
    float scale = 1.0f;
    if (normalize) {
        float sq = 0.0f;
        for (int c = lane; c < W; c += 64) sq = fmaf(x[c], x[c], sq);
        const float r = rsqrtf(fmaxf(wave_sum(sq), kXsaFloor));
        if (lane == 0) rinv[t] = r;
        scale = r * radius;
    }
    for (int c = lane; c < W; c += 64)
        out[size_t(t) * W + c] = c < preserve ? codes[size_t(t) * W + c] : x[c] * scale;
}

// In place on g (d loss / d geometry output -> d loss / d raw rows): protected
// coordinates are constants (gradient 0); the scaling's Jacobian is
// radius r (g - r^2 raw (g . raw)) above the norm floor, radius r g below it.
__global__ void __launch_bounds__(kThreads) geometry_backward_kernel(const float *__restrict__ raw,
                                                                     const float *__restrict__ rinv, float *g, int V,
                                                                     int W, float radius, int normalize,
                                                                     int preserve) {
    const int t = row_wave(), lane = threadIdx.x & 63;
    if (t >= V) return;
    const float *x = raw + size_t(t) * W;
    float *row = g + size_t(t) * W;
    for (int c = lane; c < min(preserve, W); c += 64) row[c] = 0.0f;
    if (!normalize) return;
    float dot = 0.0f, sq = 0.0f;
    for (int c = lane; c < W; c += 64) {
        dot = fmaf(row[c], x[c], dot);
        sq = fmaf(x[c], x[c], sq);
    }
    dot = wave_sum(dot);
    sq = wave_sum(sq);
    const float r = rinv[t], k = sq >= kXsaFloor ? r * r * dot : 0.0f;
    for (int c = lane; c < W; c += 64) row[c] = radius * r * (row[c] - k * x[c]);
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

__global__ void __launch_bounds__(kThreads) fill_kernel(float *p, float v, size_t n) {
    const size_t i = size_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i < n) p[i] = v;
}

__global__ void __launch_bounds__(kThreads) copy_kernel(const float *__restrict__ a, float *__restrict__ b, size_t n) {
    const size_t i = size_t(blockIdx.x) * kThreads + threadIdx.x;
    if (i < n) b[i] = a[i];
}



// One wave per row: the maximum and the sum over the vocabulary by wave
// reductions (the loss kernel of gpu.rs:949-994 sums sequentially; the
// difference is f32 rounding).
__global__ void __launch_bounds__(kThreads) cross_entropy_kernel(const float *__restrict__ logits,
                                                                 const uint32_t *__restrict__ targets,
                                                                 float *__restrict__ dlogits, float *__restrict__ loss,
                                                                 int rows, int V, StepScalars *sc) {
    const int r = (blockIdx.x * kThreads + threadIdx.x) >> 6, lane = threadIdx.x & 63;
    if (r >= rows) return;
    const float *row = logits + size_t(r) * V;
    float *out = dlogits + size_t(r) * V;
    const uint32_t target = targets[r];
    if (target == 0xFFFFFFFFu) {
        for (int t = lane; t < V; t += 64) out[t] = 0.0f;
        if (lane == 0) loss[r] = 0.0f;
        return;
    }
    float maximum = -INFINITY;
    for (int t = lane; t < V; t += 64) maximum = fmaxf(maximum, row[t]);
    for (int k = 32; k >= 1; k >>= 1) maximum = fmaxf(maximum, __shfl_xor(maximum, k, 64));
    float sum = 0.0f;
    for (int t = lane; t < V; t += 64) sum += expf(row[t] - maximum);
    sum = wave_sum(sum);
    const float value = logf(sum) + maximum - row[target];
    if (lane == 0) {
        loss[r] = value;
        if (!isfinite(value)) atomicOr(&sc->nonfinite, 1);
    }
    const float scale = sc->inv_supervised;
    for (int t = lane; t < V; t += 64)
        out[t] = (expf(row[t] - maximum) / sum - (uint32_t(t) == target ? 1.0f : 0.0f)) * scale;
}

typedef float v4f __attribute__((ext_vector_type(4)));

// C = A B, one 16 x 16 tile of C per wave on v_mfma_f32_16x16x4f32 (FP32
// products and sums).  At step s of each 16-wide slice of K, lane l supplies
// A[l % 16][k] and B[k][l % 16] for k = 4 (l / 16) + s, and it holds
// C[4 (l / 16) + j][l % 16] in element j.  A[m][k] is A[m lda + k] (AK) or
// A[k lda + m]; B[k][n] is B[n ldb + k] (BK) or B[k ldb + n].  blockIdx.y
// takes the K slice [y kspan, (y + 1) kspan) and writes C + y cstride.  With
// `tokens` (the embedding gradient: M = vocabulary, K = rows, N = W), each row
// r of the slice also adds dx[r][n] to C[tokens[r]][n].
template <bool AK, bool BK>
__global__ void __launch_bounds__(kThreads) gemm_tile_kernel(const float *__restrict__ A, int lda,
                                                             const float *__restrict__ B, int ldb,
                                                             float *__restrict__ C, int ldc, size_t cstride, int M,
                                                             int N, int K, int kspan, const uint32_t *__restrict__ tokens,
                                                             const float *__restrict__ dx) {
    const int tiles_n = (N + 15) / 16, tiles = (M + 15) / 16 * tiles_n;
    const int wave = int(blockIdx.x) * (kThreads / 64) + int(threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (wave >= tiles) return;
    const int m0 = wave / tiles_n * 16, n0 = wave % tiles_n * 16, i = lane & 15, g = lane >> 4;
    const int m = m0 + i, n = n0 + i, kb = int(blockIdx.y) * kspan, ke = min(K, kb + kspan);
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int k0 = kb; k0 < ke; k0 += 16) {
        float a[4], b[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int k = k0 + 4 * g + s;
            const bool ok = k < ke;
            a[s] = ok && m < M ? (AK ? A[size_t(m) * lda + k] : A[size_t(k) * lda + m]) : 0.0f;
            b[s] = ok && n < N ? (BK ? B[size_t(n) * ldb + k] : B[size_t(k) * ldb + n]) : 0.0f;
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[s], acc, 0, 0, 0);
    }
    if (tokens) {
        for (int r = kb; r < ke; ++r) {
            const int t = int(tokens[r]) - m0;  // the same for every lane
            if (t < 0 || t >= 16 || (t >> 2) != g || n >= N) continue;
            const float d = dx[size_t(r) * N + n];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if ((t & 3) == j) acc[j] += d;
        }
    }
    float *out = C + size_t(blockIdx.y) * cstride;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int row = m0 + 4 * g + j;
        if (row < M && n < N) out[size_t(row) * ldc + n] = acc[j];
    }
}

// Rows of the embedding gradient's K slices (one partial per slice).
constexpr int kEmbeddingSpan = 64;

template <bool AK, bool BK>
void gemm_tiles(const float *A, int lda, const float *B, int ldb, float *C, int ldc, size_t cstride, int M, int N,
                int K, int kspan, const uint32_t *tokens, const float *dx, hipStream_t stream) {
    const int tiles = (M + 15) / 16 * ((N + 15) / 16), splits = (K + kspan - 1) / kspan;
    const dim3 grid(unsigned((tiles + kThreads / 64 - 1) / (kThreads / 64)), unsigned(std::max(splits, 1)));
    hipLaunchKernelGGL((gemm_tile_kernel<AK, BK>), grid, dim3(kThreads), 0, stream, A, lda, B, ldb, C, ldc, cstride,
                       M, N, K, kspan, tokens, dx);
}

__global__ void __launch_bounds__(kThreads) adam_kernel(float *__restrict__ params, float *__restrict__ m,
                                                        float *__restrict__ v, const float *__restrict__ grad,
                                                        size_t begin, size_t end, AdamW o,
                                                        const StepScalars *__restrict__ sc) {
    const size_t i = begin + size_t(blockIdx.x) * kThreads + threadIdx.x;
    // A non-finite loss stops the step before the update (gpu.rs:2296-2313).
    if (i >= end || sc->nonfinite) return;
    // The arithmetic of gpu.rs:1383-1389, unfused.
    const float g = grad[i];
    const float mi = __fadd_rn(__fmul_rn(o.beta1, m[i]), __fmul_rn(1.0f - o.beta1, g));
    const float vi = __fadd_rn(__fmul_rn(o.beta2, v[i]), __fmul_rn(__fmul_rn(1.0f - o.beta2, g), g));
    m[i] = mi;
    v[i] = vi;
    const float mh = mi / sc->correction1, vh = vi / sc->correction2;
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

// ---- the forward of short sequences: a workgroup holds R sequences, one wave
// per position holding that position's row of each (W <= 128, the channel of
// register j given by short_channel); the rows stay in registers through every
// block, the sequences' keys and values meet in LDS, and only the logits leave.

// The short forward carries every mesh value scaled by K = log2(e): a layer
// computes t = K z directly from scaled inputs (the mesh is linear in its
// input up to the ELU), and the ELU in those units is
//   K ELU(t / K) = max(t, K (clamp(exp2(t), 0, 1) - 1))
// (reference.rs:325-332): for t >= 0 the clamped exp2 is 1 and the maximum is
// t; for t < 0, K (2^t - 1) = K (exp(z) - 1) lies above t.  That is one
// multiply fewer per value than exp2(z K) on unscaled values.  The maximum is
// IEEE 754-2019's (v_maximum3_f32), which returns NaN when an operand is NaN,
// so a NaN stays NaN as in the reference (the clamp maps exp2(NaN) to 0, and a
// maxNum or med3 form would return the other operand); t = +inf stays +inf and
// t = -inf gives -K, K ELU(-inf).  The hardware exp2's absolute error (~1e-7)
// is far below the logit tolerance.  The scale enters with the RMSNorm
// factors in front of the meshes, and leaves in the residual adds, the QK-Norm
// epsilon (K^2 eps on K-scaled rows) and the XSA floor.
constexpr float kLog2e = 1.4426950408889634f, kLn2 = 0.6931471805599453f;
__device__ __forceinline__ float elu_log2(float t) {
    const float e = __builtin_amdgcn_fmed3f(__builtin_amdgcn_exp2f(t), 0.0f, 1.0f);
    return __builtin_elementwise_maximum(t, __builtin_fmaf(e, kLog2e, -kLog2e));
}

// The channel of a lane's register j: lane + 64 j, or 2 lane + j when IL (the
// interleaved order of width 128 with neighbour connectivity: channel c + 1 of
// register 0 is register 1 of the same lane, that of register 1 is register 0
// one lane up, wrapping at lane 63 to channel 0, so the mesh shift needs no
// select).
template <bool IL>
__device__ __forceinline__ int short_channel(int lane, int j) { return IL ? 2 * lane + j : lane + 64 * j; }

// Whether channel c holds a value: always at width 128 (two registers a lane),
// below W at the widths of one register.
template <int CPL>
__device__ __forceinline__ bool short_live(int c, int W) { return CPL == 2 || c < W; }

// Sum over the channels of each head of hd channels, left in all of them: the
// aligned groups of hd lanes (hd a power of two up to 64), or both registers
// and the wave when hd = 128; when IL, both registers of hd / 2 lanes (DPP
// moves within 16-lane rows, lane shuffles across them).
template <bool IL, int CPL>
__device__ __forceinline__ void head_sums(float (&v)[CPL], int hd) {
    if constexpr (IL) {
        float t = v[0] + v[1];
        switch (hd) {
            case 2: break;
            case 4: t = group_sum<2>(t); break;
            case 8: t = group_sum<4>(t); break;
            case 16: t = group_sum<8>(t); break;
            case 32: t = group_sum<16>(t); break;
            case 64: t = group_sum<32>(t); break;
            default: t = wave_sum(t); break;
        }
        v[0] = v[1] = t;
        return;
    }
    if (hd > 64) {
        float t = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) t += v[j];
        t = wave_sum(t);
#pragma unroll
        for (int j = 0; j < CPL; ++j) v[j] = t;
        return;
    }
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        switch (hd) {
            case 2: v[j] = group_sum<2>(v[j]); break;
            case 4: v[j] = group_sum<4>(v[j]); break;
            case 8: v[j] = group_sum<8>(v[j]); break;
            case 16: v[j] = group_sum<16>(v[j]); break;
            case 32: v[j] = group_sum<32>(v[j]); break;
            default: v[j] = group_sum<64>(v[j]); break;
        }
    }
}

// One mesh stack (reference.rs:422-453) on the wave's R rows (log2(e)-scaled,
// elu_log2), in place: layer l reads its weights at w + l * 2W, the next
// layer's loading during this one.
// BF: butterfly strides (a lane exchange per distance), else neighbour
// connectivity, whose constant stride keeps the code small enough for the
// instruction cache.
template <int CPL, int R, bool BF, bool IL>
__device__ __forceinline__ void wave_stack(float (&x)[R][CPL], const float *__restrict__ w, int depth,
                                           const Mesh &m, int lane) {
    const int W = m.W;
    float2 cur[CPL], nxt[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = short_channel<IL>(lane, j);
        cur[j] = short_live<CPL>(c, W) ? reinterpret_cast<const float2 *>(w)[c] : make_float2(0.0f, 0.0f);
        nxt[j] = cur[j];
    }
#pragma nounroll
    for (int l = 0; l < depth; ++l) {
        if (l + 1 < depth) {
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const int c = short_channel<IL>(lane, j);
                nxt[j] = short_live<CPL>(c, W) ? reinterpret_cast<const float2 *>(w + size_t(l + 1) * 2 * W)[c] : make_float2(0.0f, 0.0f);
            }
        }
        const int d = BF ? 1 << (l % m.log2w) : 1;
        const bool last = l + 1 == depth;
#pragma unroll
        for (int i = 0; i < R; ++i) {
            float p[CPL];
            if constexpr (IL) {
                p[0] = x[i][1];
                p[1] = lanes_rol1(x[i][0]);
            } else {
                channel_shift(x[i], d, W, lane, p);
            }
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const float z = x[i][j] * cur[j].x + p[j] * cur[j].y;
                x[i][j] = last ? z : elu_log2(z);
            }
        }
#pragma unroll
        for (int j = 0; j < CPL; ++j) cur[j] = nxt[j];
    }
}

// RMSNorm of each of the wave's rows (reference.rs:392-409), times `scale`.
template <int CPL, int R>
__device__ __forceinline__ void wave_rmsnorm(const float (&x)[R][CPL], float (&n)[R][CPL], int W, float scale) {
#pragma unroll
    for (int i = 0; i < R; ++i) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) acc = fmaf(x[i][j], x[i][j], acc);
        const float iv = rsqrtf(wave_sum(acc) * (1.0f / float(W)) + kRmsEps) * scale;
#pragma unroll
        for (int j = 0; j < CPL; ++j) n[i][j] = x[i][j] * iv;
    }
}

template <int CPL, int R, bool BF>
__global__ void __launch_bounds__(1024) short_forward_kernel(ShortForward a, int sequences) {
    // keys, values and final rows, each [R][sequence][W]
    extern __shared__ float lds[];
    const int W = a.W, lane = threadIdx.x & 63, pos = threadIdx.x >> 6, S = a.sequence;
    const int hd = W / a.H, half = hd / 2, slab = R * S * W;
    const float scale2 = a.scale * 1.4426950408889634f;
    constexpr bool IL = CPL == 2 && !BF;
    float *keys = lds, *values = lds + slab, *finals = lds + 2 * slab;
    const Mesh m{W, 0, a.butterfly, a.log2w};
    // Sequence i of the workgroup; past the last one a workgroup recomputes the
    // last and stores nothing for it.
    const int s0 = blockIdx.x * R, valid = min(R, sequences - s0);
    float x[R][CPL];
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const uint32_t tok = a.tokens[size_t(s0 + min(i, valid - 1)) * S + pos];
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = short_channel<IL>(lane, j);
            x[i][j] = short_live<CPL>(c, W) ? a.E[size_t(tok) * W + c] : 0.0f;
        }
    }
    const size_t gA = 2 * size_t(W) * a.A, gF = 2 * size_t(W) * a.F;
    // QK-Norm of K-scaled rows q' = K q: q' / sqrt(mean(q'^2) + K^2 eps) is
    // q / sqrt(mean(q^2) + eps).
    const float qk_eps = kRmsEps * kLog2e * kLog2e;
    for (int b = 0; b < a.L; ++b) {
        const float *wb = a.w + a.block0 + size_t(b) * (4 * gA + gF);
        // With last_only, rows before a sequence's last reach the head only
        // through their keys and values in the last block: those waves run its
        // K and V meshes and skip the rest (wave-uniform; every barrier is
        // still reached).
        const bool tail = a.last_only && b + 1 == a.L && pos + 1 < S;
        float q[R][CPL], k[R][CPL], v[R][CPL];
        wave_rmsnorm(x, q, W, kLog2e);
#pragma unroll
        for (int i = 0; i < R; ++i)
#pragma unroll
            for (int j = 0; j < CPL; ++j) k[i][j] = v[i][j] = q[i][j];
        if (!tail) wave_stack<CPL, R, BF, IL>(q, wb, a.A, m, lane);
        wave_stack<CPL, R, BF, IL>(k, wb + gA, a.A, m, lane);
        wave_stack<CPL, R, BF, IL>(v, wb + 2 * gA, a.A, m, lane);
        // QK-Norm, then slice RoPE at this row's position (reference.rs:174-193).
#pragma unroll
        for (int i = 0; i < R; ++i) {
            if (a.qk_norm) {
                float sq[CPL], sk[CPL];
#pragma unroll
                for (int j = 0; j < CPL; ++j) {
                    sq[j] = q[i][j] * q[i][j];
                    sk[j] = k[i][j] * k[i][j];
                }
                if (!tail) head_sums<IL>(sq, hd);
                head_sums<IL>(sk, hd);
#pragma unroll
                for (int j = 0; j < CPL; ++j) {
                    q[i][j] *= rsqrtf(sq[j] * (1.0f / float(hd)) + qk_eps);
                    k[i][j] *= rsqrtf(sk[j] * (1.0f / float(hd)) + qk_eps);
                }
            } else {
#pragma unroll
                for (int j = 0; j < CPL; ++j) {
                    q[i][j] *= kLn2;
                    k[i][j] *= kLn2;
                }
            }
            if (a.rope) {
                float oq[CPL], ok[CPL];
                if (IL && half == 1) {
#pragma unroll
                    for (int j = 0; j < CPL; ++j) {
                        oq[j] = q[i][(j + 1) % CPL];
                        ok[j] = k[i][(j + 1) % CPL];
                    }
                } else if (IL) {
#pragma unroll
                    for (int j = 0; j < CPL; ++j) {
                        oq[j] = __shfl_xor(q[i][j], half / 2, 64);
                        ok[j] = __shfl_xor(k[i][j], half / 2, 64);
                    }
                } else if (hd <= 64) {
#pragma unroll
                    for (int j = 0; j < CPL; ++j) {
                        oq[j] = __shfl_xor(q[i][j], half, 64);
                        ok[j] = __shfl_xor(k[i][j], half, 64);
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < CPL; ++j) {
                        oq[j] = q[i][(j + 1) % CPL];
                        ok[j] = k[i][(j + 1) % CPL];
                    }
                }
                const float2 *tr = a.table + size_t(pos) * half;
#pragma unroll
                for (int j = 0; j < CPL; ++j) {
                    const int d = short_channel<IL>(lane, j) % hd;
                    const float2 cs = tr[d < half ? d : d - half];
                    q[i][j] = d < half ? q[i][j] * cs.x - oq[j] * cs.y : q[i][j] * cs.x + oq[j] * cs.y;
                    k[i][j] = d < half ? k[i][j] * cs.x - ok[j] * cs.y : k[i][j] * cs.x + ok[j] * cs.y;
                }
            }
        }
        __syncthreads();  // the previous block's readers of keys and values are done
#pragma unroll
        for (int i = 0; i < R; ++i)
#pragma unroll
            for (int j = 0; j < CPL; ++j)
                if (short_live<CPL>(short_channel<IL>(lane, j), W)) {
                    keys[(i * S + pos) * W + short_channel<IL>(lane, j)] = k[i][j];
                    values[(i * S + pos) * W + short_channel<IL>(lane, j)] = v[i][j];
                }
        __syncthreads();
        if (tail) continue;
        // Causal softmax attention over keys 0..pos per head (reference.rs:510-554),
        // the maximum and sum carried along the keys.
        float y[R][CPL], mx[R][CPL], sum[R][CPL];
#pragma unroll
        for (int i = 0; i < R; ++i)
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                y[i][j] = sum[i][j] = 0.0f;
                mx[i][j] = -INFINITY;
            }
        for (int t = 0; t <= pos; ++t) {
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const float *kr = keys + (i * S + t) * W, *vr = values + (i * S + t) * W;
                float sv[CPL];
#pragma unroll
                for (int j = 0; j < CPL; ++j) sv[j] = short_live<CPL>(short_channel<IL>(lane, j), W) ? q[i][j] * kr[short_channel<IL>(lane, j)] : 0.0f;
                head_sums<IL>(sv, hd);
#pragma unroll
                for (int j = 0; j < CPL; ++j) {
                    // Scores in log2 units: exp is the hardware exp2 (relative
                    // error ~1e-7 for the scores' range).
                    const float sc = sv[j] * scale2, top = fmaxf(mx[i][j], sc);
                    const float c = __builtin_amdgcn_exp2f(mx[i][j] - top), e = __builtin_amdgcn_exp2f(sc - top);
                    sum[i][j] = fmaf(sum[i][j], c, e);
                    y[i][j] = fmaf(y[i][j], c, e * (short_live<CPL>(short_channel<IL>(lane, j), W) ? vr[short_channel<IL>(lane, j)] : 0.0f));
                    mx[i][j] = top;
                }
            }
        }
        // The values are K-scaled, so y and the XSA output are too: the
        // projection mesh takes them as they are.
#pragma unroll
        for (int i = 0; i < R; ++i) {
#pragma unroll
            for (int j = 0; j < CPL; ++j) y[i][j] *= __builtin_amdgcn_rcpf(sum[i][j]);
            // XSA against the row's own value (reference.rs:577-603); the norm
            // floor max(|v|, 1e-12) scales with v.
            if (a.xsa) {
                float vv[CPL], yu[CPL];
#pragma unroll
                for (int j = 0; j < CPL; ++j) vv[j] = v[i][j] * v[i][j];
                head_sums<IL>(vv, hd);
#pragma unroll
                for (int j = 0; j < CPL; ++j) {
                    v[i][j] *= rsqrtf(fmaxf(vv[j], kXsaFloor * (kLog2e * kLog2e)));
                    yu[j] = y[i][j] * v[i][j];
                }
                head_sums<IL>(yu, hd);
#pragma unroll
                for (int j = 0; j < CPL; ++j) y[i][j] -= yu[j] * v[i][j];
            }
        }
        wave_stack<CPL, R, BF, IL>(y, wb + 3 * gA, a.A, m, lane);
#pragma unroll
        for (int i = 0; i < R; ++i)
#pragma unroll
            for (int j = 0; j < CPL; ++j) x[i][j] = fmaf(y[i][j], kLn2, x[i][j]);
        wave_rmsnorm(x, y, W, kLog2e);
        wave_stack<CPL, R, BF, IL>(y, wb + 4 * gA, a.F, m, lane);
#pragma unroll
        for (int i = 0; i < R; ++i)
#pragma unroll
            for (int j = 0; j < CPL; ++j) x[i][j] = fmaf(y[i][j], kLn2, x[i][j]);
    }
    // The tied head (reference.rs:218-226) on the final norm of the rows asked for.
    if (!a.last_only || pos == S - 1) {
        float nf[R][CPL];
        wave_rmsnorm(x, nf, W, 1.0f);
#pragma unroll
        for (int i = 0; i < R; ++i)
#pragma unroll
            for (int j = 0; j < CPL; ++j)
                if (short_live<CPL>(short_channel<IL>(lane, j), W)) finals[(i * S + pos) * W + short_channel<IL>(lane, j)] = nf[i][j];
    }
    __syncthreads();
    // The tied head over the rows asked for (at most R * S <= 16): work items
    // pair a run of 64 tokens, one a lane (the reads of Et[c][t] coalesced,
    // each from a uniform column base plus the lane's token), with a group of
    // up to 4 rows, whose channels are LDS broadcasts shared by the lane's
    // tokens; the waves take the items in turn.  Rows go in groups of 4, or of
    // fewer when that would leave waves idle.  Each logit adds its terms in
    // channel order (reference.rs:218-226).
    const int first = a.last_only ? S - 1 : 0, per = S - first, nrow = valid * per;
    const int chunks = (a.V + 63) / 64;
    int G = 4;
    while (G > 1 && chunks * ((nrow + G - 1) / G) < S) G >>= 1;
    const int items = chunks * ((nrow + G - 1) / G);
    float *lo = a.logits + size_t(s0) * per * a.V;
    // One item: rows r0 .. r0 + gn - 1 (gn <= GG; the rows past them repeat
    // the last one and are not stored) for the lane's token.
    auto item = [&](auto GGC, int chunk, int r0, int gn) {
        constexpr int GG = decltype(GGC)::value;
        const int t = chunk * 64 + lane, tt = min(t, a.V - 1);  // lanes past V compute a copy
        const float *fr[GG];
#pragma unroll
        for (int k = 0; k < GG; ++k) {
            const int r = r0 + min(k, gn - 1), i = r / per;
            fr[k] = finals + (i * S + first + r - i * per) * W;
        }
        float acc[GG];
#pragma unroll
        for (int k = 0; k < GG; ++k) acc[k] = 0.0f;
        if constexpr (CPL == 2) {
            // Width 128: channels four at a time (one LDS read per row), 32
            // column loads in flight.
#pragma unroll 8
            for (int c = 0; c < 128; c += 4) {
                float e[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) e[u] = (a.Et + size_t(c + u) * a.vpad)[tt];
#pragma unroll
                for (int k = 0; k < GG; ++k) {
                    const float4 f = *reinterpret_cast<const float4 *>(fr[k] + c);
                    acc[k] = fmaf(f.x, e[0], acc[k]);
                    acc[k] = fmaf(f.y, e[1], acc[k]);
                    acc[k] = fmaf(f.z, e[2], acc[k]);
                    acc[k] = fmaf(f.w, e[3], acc[k]);
                }
            }
        } else {
            for (int c = 0; c < W; ++c) {
                const float e = (a.Et + size_t(c) * a.vpad)[tt];
#pragma unroll
                for (int k = 0; k < GG; ++k) acc[k] = fmaf(fr[k][c], e, acc[k]);
            }
        }
        if (t < a.V) {
#pragma unroll
            for (int k = 0; k < GG; ++k)
                if (k < gn) lo[size_t(r0 + k) * a.V + t] = acc[k];
        }
    };
    for (int it = pos; it < items; it += S) {
        const int chunk = it % chunks, r0 = it / chunks * G, gn = min(G, nrow - r0);
        if (G == 4)
            item(std::integral_constant<int, 4>{}, chunk, r0, gn);
        else if (G == 2)
            item(std::integral_constant<int, 2>{}, chunk, r0, gn);
        else
            item(std::integral_constant<int, 1>{}, chunk, r0, gn);
    }
}

}  // namespace

// f(channels a lane, layers a launch holds) for the wave mesh kernels: 4, 8 or
// 16 layers, the fewest that hold `depth`.
template <class F>
void by_wave_shape(int cpl, int depth, F &&f) {
    auto layers = [&](auto C) {
        if (depth <= 4)
            f(C, std::integral_constant<int, 4>{});
        else if (depth <= 8)
            f(C, std::integral_constant<int, 8>{});
        else
            f(C, std::integral_constant<int, kMaxDepth>{});
    };
    if (cpl == 1)
        layers(std::integral_constant<int, 1>{});
    else
        layers(std::integral_constant<int, 2>{});
}

void reduce_gradients(const GradReduce *r, size_t count, hipStream_t stream) {
    for (size_t b = 0; b < count; b += kMaxReduce) {
        ReduceSet set{};
        int most = 0, k = 0;
        for (; k < kMaxReduce && b + k < count; ++k) {
            set.part[k] = r[b + k].part;
            set.out[k] = r[b + k].out;
            set.groups[k] = r[b + k].groups;
            set.n[k] = r[b + k].n;
            most = std::max(most, r[b + k].n);
        }
        hipLaunchKernelGGL(reduce_groups_kernel, dim3(unsigned((most + 63) / 64), unsigned(k)), dim3(1024), 0, stream,
                           set);
    }
}

// Layers [l0, l0 + kMaxDepth) of m as one launch's stack.
Mesh mesh_chunk(const Mesh &m, int l0) {
    Mesh c = m;
    c.layer0 = m.layer0 + l0;
    c.depth = std::min(kMaxDepth, m.depth - l0);
    c.linear_top = l0 + c.depth == m.depth ? m.linear_top : 0;
    return c;
}

// The wave kernels can put the norm in front of a stack of at most kMaxDepth
// layers in its own launch; every other case takes the norm's own launch.
bool norm_fuses(const Mesh &m) { return mesh_wave_cpl(m.W) != 0 && m.depth <= kMaxDepth; }

void mesh_forward_impl(const Mesh &m, int count, const float *const *in, float *const *stack, const float *const *w,
                       const NormIn *ni, const QkOut *qk, int rows, hipStream_t stream) {
    const size_t plane = size_t(rows) * m.W;
    for (int l0 = 0; l0 < m.depth; l0 += kMaxDepth) {
        const Mesh c = mesh_chunk(m, l0);
        MeshSet set{};
        for (int i = 0; i < count; ++i) {
            set.in[i] = l0 == 0 ? in[i] : stack[i] + (l0 - 1) * plane;
            set.stack[i] = stack[i] + l0 * plane;
            set.w[i] = w[i] + size_t(l0) * 2 * m.W;
        }
        if (const int cpl = mesh_wave_cpl(m.W)) {
            const dim3 grid(unsigned((rows + kThreads / 64 - 1) / (kThreads / 64)), unsigned(count));
            const NormIn none{};
            const QkOut noqk{};
            // Only the launch with the stacks' last layers forms q and k.
            const QkOut &tail = qk && l0 + c.depth == m.depth ? *qk : noqk;
            by_wave_shape(cpl, c.depth, [&](auto C, auto D) {
                constexpr int CC = decltype(C)::value, DD = decltype(D)::value;
                if (ni)
                    hipLaunchKernelGGL((mesh_forward_wave<CC, DD, true>), grid, dim3(kThreads), 0, stream, c, set, *ni,
                                       tail, rows);
                else
                    hipLaunchKernelGGL((mesh_forward_wave<CC, DD, false>), grid, dim3(kThreads), 0, stream, c, set,
                                       none, tail, rows);
            });
        } else {
            const dim3 grid(unsigned(std::min(rows, 2048)), unsigned(count));
            hipLaunchKernelGGL(mesh_forward_kernel, grid, dim3(block_for(m.W)), 2 * m.W * sizeof(float), stream, c,
                               set, rows);
        }
    }
}

void mesh_forward_set(const Mesh &m, int count, const float *const *in, float *const *stack, const float *const *w,
                      int rows, hipStream_t stream) {
    mesh_forward_impl(m, count, in, stack, w, nullptr, nullptr, rows, stream);
}

void norm_mesh_forward_set(const Mesh &m, int count, const NormIn &ni, float *const *stack, const float *const *w,
                           int rows, hipStream_t stream) {
    const float *in[kMaxSet];
    for (int i = 0; i < count; ++i) in[i] = ni.n;
    if (norm_fuses(m)) {
        mesh_forward_impl(m, count, in, stack, w, &ni, nullptr, rows, stream);
        return;
    }
    if (ni.b)
        add_rmsnorm_forward(ni.a, ni.b, ni.sum, ni.n, ni.inv, rows, m.W, stream);
    else
        rmsnorm_forward(ni.a, ni.n, ni.inv, rows, m.W, 1, stream);
    mesh_forward_impl(m, count, in, stack, w, nullptr, nullptr, rows, stream);
}

void norm_mesh_forward_qkv(const Mesh &m, const NormIn &ni, float *const *stack, const float *const *w,
                           const QkOut &qk, int rows, hipStream_t stream) {
    const int hd = m.W / qk.H;
    const bool pow2 = hd >= 2 && (hd & (hd - 1)) == 0;
    if (norm_fuses(m) && pow2 && (hd <= 64 || hd == 128)) {
        const float *in[3] = {ni.n, ni.n, ni.n};
        mesh_forward_impl(m, 3, in, stack, w, &ni, &qk, rows, stream);
        return;
    }
    norm_mesh_forward_set(m, 3, ni, stack, w, rows, stream);
    const size_t last = size_t(m.depth - 1) * rows * m.W;
    const float *pre[2] = {stack[0] + last, stack[1] + last};
    qk_forward(2, pre, qk.out, qk.inv, qk.table, rows, qk.sequence, m.W, qk.H, qk.norm, qk.rotate, stream);
}

void mesh_forward(const Mesh &m, const float *in, float *stack, const float *w, int rows, hipStream_t stream) {
    mesh_forward_set(m, 1, &in, &stack, &w, rows, stream);
}

size_t mesh_partial_floats(const Mesh &m, int rows) {
    const int groups = mesh_wave_cpl(m.W) ? mesh_wave_groups(rows) : mesh_groups(m, rows);
    const size_t partial = size_t(groups) * std::min(m.depth, kMaxDepth) * m.W * 2;
    return m.depth > kMaxDepth ? partial + 2 * size_t(rows) * m.W : partial;
}

// Each stack of the set works in its own mesh_partial_floats of `partials`:
// the partial sums, then (deep stacks) the two planes of gradient rows that
// carry d loss down from one launch of kMaxDepth layers to the next.
void mesh_backward_impl(const Mesh &m, int count, const float *const *in, const float *const *stack,
                        const float *const *dout, float *const *din, bool accumulate, const float *const *w,
                        float *partials, float *const *grad, const NormGrad *ng, int rows, hipStream_t stream,
                        std::vector<GradReduce> *deferred) {
    const size_t plane = size_t(rows) * m.W, per = mesh_partial_floats(m, rows);
    const int top = (m.depth - 1) / kMaxDepth * kMaxDepth;
    const float *g[kMaxSet] = {};
    for (int i = 0; i < count; ++i) g[i] = dout[i];
    for (int l0 = top, k = 0; l0 >= 0; l0 -= kMaxDepth, ++k) {
        const Mesh c = mesh_chunk(m, l0);
        MeshGradSet set{};
        GradReduce red[kMaxSet];
        for (int i = 0; i < count; ++i) {
            float *base = partials + i * per, *between = base + (per - (top > 0 ? 2 * plane : 0));
            float *to = l0 == 0 ? din[i] : between + (k & 1) * plane;
            set.in[i] = l0 == 0 ? in[i] : stack[i] + (l0 - 1) * plane;
            set.stack[i] = stack[i] + l0 * plane;
            set.dout[i] = g[i];
            set.din[i] = to;
            set.w[i] = w[i] + size_t(l0) * 2 * m.W;
            set.partials[i] = base;
            red[i].part = base;
            red[i].out = grad[i] + size_t(l0) * 2 * m.W;
            g[i] = to;
        }
        const int acc = l0 == 0 && accumulate, n = c.depth * m.W * 2;
        int groups;
        if (const int cpl = mesh_wave_cpl(m.W)) {
            groups = mesh_wave_groups(rows);
            const size_t lds = size_t(kThreads / 64) * n * sizeof(float);
            const dim3 grid{unsigned(groups), unsigned(count)};
            const NormGrad none{};
            by_wave_shape(cpl, c.depth, [&](auto C, auto D) {
                constexpr int CC = decltype(C)::value, DD = decltype(D)::value;
                if (ng)
                    hipLaunchKernelGGL((mesh_backward_wave<CC, DD, true>), grid, dim3(kThreads), lds, stream, c, set,
                                       *ng, acc, rows);
                else
                    hipLaunchKernelGGL((mesh_backward_wave<CC, DD, false>), grid, dim3(kThreads), lds, stream, c, set,
                                       none, acc, rows);
            });
        } else {
            groups = mesh_groups(c, rows);
            const int rpb = mesh_rpb(m.W);
            hipLaunchKernelGGL(mesh_backward_kernel, dim3(unsigned(groups), unsigned(count)), dim3(kMaxWidth),
                               size_t(3) * rpb * m.W * sizeof(float), stream, c, set, acc, rows);
        }
        for (int i = 0; i < count; ++i) {
            red[i].groups = groups;
            red[i].n = n;
        }
        // A single launch's sums can wait for the caller's combined reduction;
        // a deep stack's partials are reused by its next launch.
        if (deferred && top == 0)
            deferred->insert(deferred->end(), red, red + count);
        else
            reduce_gradients(red, size_t(count), stream);
    }
}

void mesh_backward_set(const Mesh &m, int count, const float *const *in, const float *const *stack,
                       const float *const *dout, float *const *din, bool accumulate, const float *const *w,
                       float *partials, float *const *grad, int rows, hipStream_t stream,
                       std::vector<GradReduce> *deferred) {
    mesh_backward_impl(m, count, in, stack, dout, din, accumulate, w, partials, grad, nullptr, rows, stream, deferred);
}

void mesh_backward_norm(const Mesh &m, const float *in, const float *stack, const float *dout, const NormGrad &ng,
                        float *scratch, const float *w, float *partials, float *grad, int rows, hipStream_t stream,
                        std::vector<GradReduce> *deferred) {
    if (norm_fuses(m)) {
        float *none = nullptr;
        mesh_backward_impl(m, 1, &in, &stack, &dout, &none, false, &w, partials, &grad, &ng, rows, stream, deferred);
        return;
    }
    mesh_backward_impl(m, 1, &in, &stack, &dout, &scratch, false, &w, partials, &grad, nullptr, rows, stream,
                       deferred);
    rmsnorm_backward(ng.x, ng.inv, scratch, ng.dx, true, rows, m.W, 1, stream);
}

void mesh_backward(const Mesh &m, const float *in, const float *stack, const float *dout, float *din,
                   bool accumulate, const float *w, float *partials, float *grad, int rows, hipStream_t stream) {
    mesh_backward_set(m, 1, &in, &stack, &dout, &din, accumulate, &w, partials, &grad, rows, stream, nullptr);
}

void rmsnorm_forward(const float *x, float *y, float *inv, int rows, int W, int groups, hipStream_t stream) {
    const size_t n = size_t(rows) * groups;
    hipLaunchKernelGGL(rmsnorm_forward_kernel<false>, dim3(blocks_for(n * 64)), dim3(kThreads), 0, stream, x,
                       nullptr, nullptr, y, inv, int(n), W / groups);
}

void add_rmsnorm_forward(const float *a, const float *b, float *sum, float *y, float *inv, int rows, int W,
                         hipStream_t stream) {
    hipLaunchKernelGGL(rmsnorm_forward_kernel<true>, dim3(blocks_for(size_t(rows) * 64)), dim3(kThreads), 0, stream,
                       a, b, sum, y, inv, rows, W);
}

void rmsnorm_backward(const float *x, const float *inv, const float *dy, float *dx, bool accumulate, int rows,
                      int W, int groups, hipStream_t stream) {
    const size_t n = size_t(rows) * groups;
    hipLaunchKernelGGL(rmsnorm_backward_kernel<1>, dim3(blocks_for(n * 64)), dim3(kThreads), 0, stream, x, inv, dy,
                       nullptr, nullptr, dx, int(accumulate), int(n), W / groups);
}

void rmsnorm_backward_sum3(const float *x, const float *inv, const float *dy0, const float *dy1, const float *dy2,
                           float *dx, bool accumulate, int rows, int W, hipStream_t stream) {
    hipLaunchKernelGGL(rmsnorm_backward_kernel<3>, dim3(blocks_for(size_t(rows) * 64)), dim3(kThreads), 0, stream,
                       x, inv, dy0, dy1, dy2, dx, int(accumulate), rows, W);
}

void attention_forward(const float *q, const float *k, const float *v, float *y, float *z, float *lse, int rows,
                       int sequence, int W, int H, bool xsa, hipStream_t stream) {
    const float scale = float(1.0 / std::sqrt(double(W / H)));
    if (sequence <= kWaveAttentionMax || W / H > 128) {
        by_lanes(W / H, [&](auto e) {
            constexpr int EPL = decltype(e)::value;
            const dim3 grid(blocks_for(size_t(rows) * H * 64));
            if (xsa)
                hipLaunchKernelGGL((attention_forward_wave<EPL, true>), grid, dim3(kThreads), 0, stream, q, k, v, y,
                                   z, lse, rows, sequence, W, H, scale);
            else
                hipLaunchKernelGGL((attention_forward_wave<EPL, false>), grid, dim3(kThreads), 0, stream, q, k, v, y,
                                   z, lse, rows, sequence, W, H, scale);
        });
        return;
    }
    by_head_width(W / H, [&](auto hd) {
        hipLaunchKernelGGL(attention_forward_kernel<decltype(hd)::value>, dim3(blocks_for(size_t(rows) * H, kRowThreads)),
                           dim3(kRowThreads), 0, stream, q, k, v, y, lse, rows, sequence, W, H, scale);
    });
    if (xsa) {
        by_lanes(W / H, [&](auto e) {
            hipLaunchKernelGGL(xsa_forward_wave<decltype(e)::value>, dim3(blocks_for(size_t(rows) * H * 64)),
                               dim3(kThreads), 0, stream, y, v, z, rows, W, H);
        });
    } else {
        copy(y, z, size_t(rows) * W, stream);
    }
}

void attention_backward(const float *q, const float *k, const float *v, const float *y, const float *lse,
                        const float *dz, float *dy, float *dq, float *dk, float *dv, float *dsum, int rows,
                        int sequence, int W, int H, bool xsa, hipStream_t stream) {
    const float scale = float(1.0 / std::sqrt(double(W / H)));
    // Without XSA the attention's output gradient is dz itself.
    const float *g = xsa ? dy : dz;
    if (sequence <= kMergedBackwardMax) {
        by_lanes(W / H, [&](auto e) {
            constexpr int EPL = decltype(e)::value;
            const dim3 grid(blocks_for(size_t(rows) * H * 64), 2);
            if (xsa)
                hipLaunchKernelGGL((attention_backward_wave<EPL, true>), grid, dim3(kThreads), 0, stream, q, k, v, y,
                                   lse, dz, dq, dk, dv, rows, sequence, W, H, scale);
            else
                hipLaunchKernelGGL((attention_backward_wave<EPL, false>), grid, dim3(kThreads), 0, stream, q, k, v, y,
                                   lse, dz, dq, dk, dv, rows, sequence, W, H, scale);
        });
        return;
    }
    if (sequence <= kWaveAttentionMax || W / H > 128) {
        by_lanes(W / H, [&](auto e) {
            constexpr int EPL = decltype(e)::value;
            const dim3 grid(blocks_for(size_t(rows) * H * 64));
            if (xsa)
                hipLaunchKernelGGL((attention_dq_wave<EPL, true>), grid, dim3(kThreads), 0, stream, q, k, v, y, lse,
                                   dz, dy, dv, dq, dsum, rows, sequence, W, H, scale);
            else
                hipLaunchKernelGGL((attention_dq_wave<EPL, false>), grid, dim3(kThreads), 0, stream, q, k, v, y, lse,
                                   dz, dy, dv, dq, dsum, rows, sequence, W, H, scale);
            hipLaunchKernelGGL(attention_dkv_wave<EPL>, grid, dim3(kThreads), 0, stream, q, k, v, lse, g, dsum, dk, dv,
                               rows, sequence, W, H, scale);
        });
        return;
    }
    if (xsa) {
        by_lanes(W / H, [&](auto e) {
            hipLaunchKernelGGL(xsa_backward_wave<decltype(e)::value>, dim3(blocks_for(size_t(rows) * H * 64)),
                               dim3(kThreads), 0, stream, y, v, dz, dy, dv, rows, W, H);
        });
    } else {
        fill(dv, 0.0f, size_t(rows) * W, stream);
    }
    by_head_width(W / H, [&](auto hd) {
        constexpr int HD = decltype(hd)::value;
        hipLaunchKernelGGL(attention_dq_kernel<HD>, dim3(blocks_for(size_t(rows) * H, kRowThreads)), dim3(kRowThreads), 0, stream, q,
                           k, v, y, lse, g, dq, dsum, rows, sequence, W, H, scale);
        hipLaunchKernelGGL(attention_dkv_kernel<HD>, dim3(blocks_for(size_t(rows) * H, kRowThreads)), dim3(kRowThreads), 0, stream,
                           q, k, v, lse, g, dsum, dk, dv, rows, sequence, W, H, scale);
    });
}

void qk_forward(int count, const float *const *pre, float *const *out, float *const *inv, const float2 *table,
                int rows, int sequence, int W, int H, bool norm, bool rotate, hipStream_t stream) {
    QkSet set{};
    for (int i = 0; i < count; ++i) {
        set.pre[i] = pre[i];
        set.out[i] = out[i];
        set.inv[i] = inv[i];
    }
    by_lanes(W / H, [&](auto e) {
        hipLaunchKernelGGL(qk_forward_kernel<decltype(e)::value>,
                           dim3(blocks_for(size_t(rows) * H * 64), unsigned(count)), dim3(kThreads), 0, stream, set,
                           table, rows, sequence, W, H, int(norm), int(rotate));
    });
}

void qk_backward(int count, float *const *g, const float *const *pre, const float *const *inv, const float2 *table,
                 int rows, int sequence, int W, int H, bool norm, bool rotate, hipStream_t stream) {
    QkSet set{};
    for (int i = 0; i < count; ++i) {
        set.pre[i] = pre[i];
        set.out[i] = g[i];
        set.inv[i] = const_cast<float *>(inv[i]);  // read only in the backward
    }
    by_lanes(W / H, [&](auto e) {
        hipLaunchKernelGGL(qk_backward_kernel<decltype(e)::value>,
                           dim3(blocks_for(size_t(rows) * H * 64), unsigned(count)), dim3(kThreads), 0, stream, set,
                           table, rows, sequence, W, H, int(norm), int(rotate));
    });
}

void geometry_forward(const float *raw, const float *codes, float *out, float *rinv, int V, int W, float radius,
                      bool normalize, int preserve, hipStream_t stream) {
    hipLaunchKernelGGL(geometry_forward_kernel, dim3(blocks_for(size_t(V) * 64)), dim3(kThreads), 0, stream, raw,
                       codes, out, rinv, V, W, radius, int(normalize), preserve);
}

void geometry_backward(const float *raw, const float *rinv, float *g, int V, int W, float radius, bool normalize,
                       int preserve, hipStream_t stream) {
    hipLaunchKernelGGL(geometry_backward_kernel, dim3(blocks_for(size_t(V) * 64)), dim3(kThreads), 0, stream, raw,
                       rinv, g, V, W, radius, int(normalize), preserve);
}

void gather(const float *E, const uint32_t *tokens, float *x, int rows, int W, hipStream_t stream) {
    hipLaunchKernelGGL(gather_kernel, dim3(blocks_for(size_t(rows) * W)), dim3(kThreads), 0, stream, E, tokens, x,
                       rows, W);
}

void head_logits(const float *n, const float *E, float *logits, int rows, int W, int V, hipStream_t stream) {
    gemm_tiles<true, true>(n, W, E, W, logits, V, 0, rows, V, W, W, nullptr, nullptr, stream);
}

void cross_entropy(const float *logits, const uint32_t *targets, float *dlogits, float *loss, int rows, int V,
                   StepScalars *scalars, hipStream_t stream) {
    hipLaunchKernelGGL(cross_entropy_kernel, dim3(blocks_for(size_t(rows) * 64)), dim3(kThreads), 0, stream, logits,
                       targets, dlogits, loss, rows, V, scalars);
}

void fill(float *p, float v, size_t n, hipStream_t stream) {
    if (n) hipLaunchKernelGGL(fill_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, stream, p, v, n);
}

void copy(const float *a, float *b, size_t n, hipStream_t stream) {
    if (n) hipLaunchKernelGGL(copy_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, stream, a, b, n);
}

void head_backward(const float *dlogits, const float *E, float *dn, int rows, int W, int V, hipStream_t stream) {
    gemm_tiles<true, false>(dlogits, V, E, W, dn, W, 0, rows, W, V, V, nullptr, nullptr, stream);
}

size_t embedding_partial_floats(int rows, int W, int V) {
    return size_t((rows + kEmbeddingSpan - 1) / kEmbeddingSpan) * V * W;
}

void embedding_gradient(const float *dlogits, const float *n, const uint32_t *tokens, const float *dx, float *dE,
                        float *partials, int rows, int W, int V, hipStream_t stream) {
    const int splits = (rows + kEmbeddingSpan - 1) / kEmbeddingSpan, nvw = V * W;
    gemm_tiles<false, false>(dlogits, V, n, W, partials, W, size_t(nvw), V, W, rows, kEmbeddingSpan, tokens, dx,
                             stream);
    const GradReduce red{partials, dE, splits, nvw};
    reduce_gradients(&red, 1, stream);
}

bool short_forward_fits(int W, int H, size_t V, int sequence) {
    const int hd = W / H;
    return mesh_wave_cpl(W) != 0 && sequence >= 1 && sequence <= kShortRows && hd >= 2 && (hd & (hd - 1)) == 0 &&
           (hd <= 64 || hd == 128) && size_t(W) * (V + 3) < (size_t(1) << 31);
}

void short_forward(const ShortForward &a, int sequences, hipStream_t stream) {
    // Sequences a workgroup holds: 4 up to 4 rows, 2 up to 8, else 1 (LDS at
    // most 3 x 16 rows x 128 floats).
    const int R = a.sequence <= 4 ? 4 : (a.sequence <= 8 ? 2 : 1);
    const size_t lds = size_t(3) * R * a.sequence * a.W * sizeof(float);
    const dim3 grid{unsigned((sequences + R - 1) / R)}, block{unsigned(64 * a.sequence)};
    using Kernel = void (*)(ShortForward, int);
    const bool one = mesh_wave_cpl(a.W) == 1;
    Kernel kernel;
    if (a.butterfly)
        kernel = R == 4   ? (one ? short_forward_kernel<1, 4, true> : short_forward_kernel<2, 4, true>)
                 : R == 2 ? (one ? short_forward_kernel<1, 2, true> : short_forward_kernel<2, 2, true>)
                          : (one ? short_forward_kernel<1, 1, true> : short_forward_kernel<2, 1, true>);
    else
        kernel = R == 4   ? (one ? short_forward_kernel<1, 4, false> : short_forward_kernel<2, 4, false>)
                 : R == 2 ? (one ? short_forward_kernel<1, 2, false> : short_forward_kernel<2, 2, false>)
                          : (one ? short_forward_kernel<1, 1, false> : short_forward_kernel<2, 1, false>);
    hipLaunchKernelGGL(kernel, grid, block, lds, stream, a, sequences);
}

void adam(float *params, float *m, float *v, const float *grad, size_t begin, size_t end, const AdamW &o,
          const StepScalars *scalars, hipStream_t stream) {
    if (end <= begin) return;
    hipLaunchKernelGGL(adam_kernel, dim3(blocks_for(end - begin)), dim3(kThreads), 0, stream, params, m, v, grad,
                       begin, end, o, scalars);
}

}  // namespace meshgpt::kern::train
