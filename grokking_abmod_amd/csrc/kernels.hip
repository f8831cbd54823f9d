// gfx950 kernels of the Mesh GPT generate path (prefill and per-token decode).
//
// Everything except attention is row-local, so each decode step is a chain of
//   block_kernel  post-attention half of block l-1 (split combine, XSA,
//                 projection mesh + residual, RMSNorm, FFN mesh + residual)
//                 fused with the pre-attention half of block l (RMSNorm, the
//                 Q/K/V meshes run concurrently by three thread teams, QK-Norm,
//                 RoPE, KV-cache append);
//   attention     attn_decode_kernel (split-KV stream over the cache, the
//                 HBM-bound kernel) or attn_prefill_kernel (causal flash);
// and, after the last block, head_sample_kernel (final RMSNorm, tied head,
// greedy / temperature sampling on device).
// Mesh rows stay in LDS across layers (one barrier per layer); each thread
// streams the [self, partner] weight pairs of its channels from L2 through a
// register ring three layers ahead, and every kernel issues its independent
// global loads before its first wait.  All arithmetic is FP32.
// Reference semantics: src/gpt/reference.rs:104-228, src/gpt/gpu.rs:2006-2053.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdlib>
#include <cmath>
#include <type_traits>
#include <utility>

#include "dpp.hpp"
#include "kernels.hpp"

namespace meshgpt::kern {
namespace {

constexpr float kRmsEps = 1e-5f;  // src/gpt/mod.rs:38
// (f64(1e-12f))^2 rounded to f32: the XSA norm floor of reference.rs:591
// A 64-bit word in global memory: accesses through it are global (not flat)
// loads and stores, which do not count in the LDS wait counter.
typedef __attribute__((address_space(1))) uint64_t global_u64;
constexpr float kXsaFloor = float(double(1e-12f) * double(1e-12f));

#define HIP_LAUNCH_CHECK() (void)hipGetLastError()


__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_move<0xB1>(v, v));
    v = fmaxf(v, dpp_move<0x4E>(v, v));
    v = fmaxf(v, dpp_move<0x141>(v, v));
    v = fmaxf(v, dpp_move<0x140>(v, v));
    v = fmaxf(v, dpp_move<0x142, 0xa>(v, v));
    v = fmaxf(v, dpp_move<0x143, 0xc>(v, v));
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ int dpp_move_int(int old, int v) {
    return __builtin_amdgcn_update_dpp(old, v, CTRL, ROW_MASK, 0xf, false);
}

__device__ __forceinline__ int wave_min_int(int v) {
    v = min(v, dpp_move_int<0xB1>(v, v));
    v = min(v, dpp_move_int<0x4E>(v, v));
    v = min(v, dpp_move_int<0x141>(v, v));
    v = min(v, dpp_move_int<0x140>(v, v));
    v = min(v, dpp_move_int<0x142, 0xa>(v, v));
    v = min(v, dpp_move_int<0x143, 0xc>(v, v));
    return __builtin_amdgcn_readlane(v, 63);
}

__device__ __forceinline__ int wave_or_int(int v) {
    v |= dpp_move_int<0xB1>(v, v);
    v |= dpp_move_int<0x4E>(v, v);
    v |= dpp_move_int<0x141>(v, v);
    v |= dpp_move_int<0x140>(v, v);
    v |= dpp_move_int<0x142, 0xa>(v, v);
    v |= dpp_move_int<0x143, 0xc>(v, v);
    return __builtin_amdgcn_readlane(v, 63);
}

// The lane's value moved by a DPP pattern, 0 where the pattern has no source.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ double dpp_move_f64(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const int lo = __builtin_amdgcn_update_dpp(0, int(uint32_t(b)), CTRL, ROW_MASK, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, int(uint32_t(b >> 32)), CTRL, ROW_MASK, 0xf, false);
    return __builtin_bit_cast(double, (uint64_t(uint32_t(hi)) << 32) | uint32_t(lo));
}

// Inclusive prefix sum over the wave's lanes: row shifts inside each 16-lane
// row, then the row broadcasts carry row totals forward.
__device__ __forceinline__ double wave_inclusive_sum(double x) {
    x += dpp_move_f64<0x111>(x);       // row_shr:1
    x += dpp_move_f64<0x112>(x);       // row_shr:2
    x += dpp_move_f64<0x114>(x);       // row_shr:4
    x += dpp_move_f64<0x118>(x);       // row_shr:8
    x += dpp_move_f64<0x142, 0xa>(x);  // row_bcast:15
    x += dpp_move_f64<0x143, 0xc>(x);  // row_bcast:31
    return x;
}


// Maximum over aligned groups of N lanes, left in every lane of the group
// (the lane pattern of group_sum).
template <int N>
__device__ __forceinline__ float group_max(float v) {
    if constexpr (N >= 2) v = fmaxf(v, dpp_move<0xB1>(v, v));
    if constexpr (N >= 4) v = fmaxf(v, dpp_move<0x4E>(v, v));
    if constexpr (N >= 8) v = fmaxf(v, dpp_move<0x141>(v, v));
    if constexpr (N >= 16) v = fmaxf(v, dpp_move<0x140>(v, v));
    if constexpr (N >= 32) v = fmaxf(v, __shfl_xor(v, 16, 64));
    if constexpr (N >= 64) v = fmaxf(v, __shfl_xor(v, 32, 64));
    return v;
}

// ELU of reference.rs:325-332: max(z, e - 1) with e = exp(z) clamped to
// [0, 1].  For z >= 0, e = 1 and the maximum is z; for z < 0, e - 1 =
// exp(z) - 1 lies above z (exp(z) >= 1 + z), so it is the maximum.  e comes
// from the hardware exp2 with its clamp modifier: the absolute error (~1e-7
// for z near 0) is that of one f32 rounding of the row values, far below the
// logit tolerance, where the library expm1 and a branch select cost several
// instructions more on every mesh layer.  The maximum is IEEE 754-2019's
// (v_maximum3_f32), which returns NaN when an operand is NaN: a NaN z stays NaN
// as in the reference (NaN >= 0 is false and exp_m1(NaN) is NaN), while the
// clamp turns exp2(NaN) into 0 and the older maxNum or med3 forms would have
// returned the other operand.  z = +inf gives e = 1 and +inf; z = -inf gives
// e = 0 and -1, both as the reference.
__device__ __forceinline__ float elu(float z) {
    const float e = __builtin_amdgcn_fmed3f(__builtin_amdgcn_exp2f(z * 1.4426950408889634f), 0.0f, 1.0f);
    return __builtin_elementwise_maximum(z, e - 1.0f);
}

// The row meshes (row_layer and the functions built on it) carry their values
// scaled by log2(e), t = z log2(e): a layer's sum then feeds exp2 directly and
// the ELU in those units, elu(z) log2(e) = max(t, log2(e) (clamp(exp2(t), 0,
// 1) - 1)), takes one instruction fewer than elu() on every value of every
// layer.  NaN and the infinities behave as in elu().  The scale enters with
// the RMSNorm factor (inv_rms_log2) or one multiply in front of a mesh and
// leaves in the residual add (an FMA by ln 2) or one multiply after it.
constexpr float kLog2e = 1.4426950408889634f, kLn2 = 0.6931471805599453f;
__device__ __forceinline__ float elu_log2(float t) {
    const float e = __builtin_amdgcn_fmed3f(__builtin_amdgcn_exp2f(t), 0.0f, 1.0f);
    return __builtin_elementwise_maximum(t, fmaf(e, kLog2e, -kLog2e));
}

// log2(e) / sqrt(sumsq / W + eps): the RMSNorm factor of a row of W values
// with sum of squares sumsq, scaled for a row mesh.
__device__ __forceinline__ float inv_rms_log2(float sumsq, int W) {
    return rsqrtf(sumsq * (1.0f / (float(W) * kLog2e * kLog2e)) + kRmsEps / (kLog2e * kLog2e));
}

// Flat LDS index -> (row, column) for rows of length W.
__device__ __forceinline__ void split_row(int idx, const Shape &s, int &r, int &c) {
    if (s.wshift >= 0) {
        r = idx >> s.wshift;
        c = idx & (s.W - 1);
    } else {
        r = idx / s.W;
        c = idx - r * s.W;
    }
}

// Column -> (head, dim).
__device__ __forceinline__ void split_head(int c, const Shape &s, int &h, int &d) {
    if (s.hdshift >= 0) {
        h = c >> s.hdshift;
        d = c & (s.hd - 1);
    } else {
        h = c / s.hd;
        d = c - h * s.hd;
    }
}

__device__ __forceinline__ void row_position(const Rows &ro, int row, int &seq, int &pos) {
    seq = row / ro.rows_per_seq;
    pos = (ro.len ? ro.len[seq] - 1 : 0) + (row - seq * ro.rows_per_seq);
}

// inv[s] = 1/sqrt(mean(x^2) + eps) for nseg contiguous segments of length len
// (reference.rs:392-409; one wave per segment).
__device__ void segment_inv_rms(const float *buf, int nseg, int len, float *inv) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const float scale = 1.0f / float(len);
    for (int sg = wave; sg < nseg; sg += nw) {
        const float *p = buf + size_t(sg) * len;
        float acc = 0.0f;
        for (int i = lane; i < len; i += 64) acc = fmaf(p[i], p[i], acc);
        acc = wave_sum(acc);
        if (lane == 0) inv[sg] = rsqrtf(acc * scale + kRmsEps);
    }
}

// For XSA: vv[s] = v.v and yv[s] = y.v per segment.
__device__ void segment_dots(const float *y, const float *v, int nseg, int len, float *vv, float *yv) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    for (int sg = wave; sg < nseg; sg += nw) {
        const float *py = y + size_t(sg) * len, *pv = v + size_t(sg) * len;
        float a = 0.0f, b = 0.0f;
        for (int i = lane; i < len; i += 64) {
            a = fmaf(pv[i], pv[i], a);
            b = fmaf(py[i], pv[i], b);
        }
        a = wave_sum(a);
        b = wave_sum(b);
        if (lane == 0) {
            vv[sg] = a;
            yv[sg] = b;
        }
    }
}

// LDS carving shared by host-side sizing and the kernels.
struct LdsCarve {
    char *base;
    size_t at = 0;
    template <typename T>
    __device__ T *take(size_t n) {
        at = (at + 15) & ~size_t(15);
        T *p = reinterpret_cast<T *>(base + at);
        at += n * sizeof(T);
        return p;
    }
};

size_t align16(size_t x) { return (x + 15) & ~size_t(15); }

// ------------------------------------------------------------- mesh stacks

// A mesh stack (reference.rs:422-453) over the nr rows in LDS `in`, computed by
// the team of T threads whose `active` flag is set (thread tt of the team owns
// channels tt + k*T).  `w` holds the [self, partner] pairs of every layer, in
// LDS (staged) or global memory.  Every thread of the block calls it: one
// barrier per layer.  Outputs alternate between a and b; returns the last.
template <int CPT>
__device__ const float *mesh_team(const float *in, float *a, float *b, int nr, const Shape &s,
                                  const float2 *w, int depth, int tt, int T, bool active) {
    const int W = s.W;
    const float *cur = in;
    float *nxt = a;
    for (int l = 0; l < depth; ++l) {
        if (active) {
            const int st = s.butterfly ? (1 << (l % s.log2w)) : 1;
            const bool last = l + 1 == depth;
            const float2 *wl = w + size_t(l) * W;
            if (nr == 1) {
                // One row (decode): the CPT channels' loads, then their
                // arithmetic, interleaved.
                float xs[CPT], xp[CPT];
                float2 ww[CPT];
#pragma unroll
                for (int k = 0; k < CPT; ++k) {
                    const int c = min(tt + k * T, W - 1);
                    int p = c + st;
                    if (p >= W) p -= W;
                    xs[k] = cur[c];
                    xp[k] = cur[p];
                    ww[k] = wl[c];
                }
                // Buffers are padded to CPT*T floats, so lanes past W store
                // (ignored) values without a branch.
#pragma unroll
                for (int k = 0; k < CPT; ++k) {
                    const float z = xs[k] * ww[k].x + xp[k] * ww[k].y;
                    nxt[tt + k * T] = last ? z : elu(z);
                }
            } else {
#pragma unroll
                for (int k = 0; k < CPT; ++k) {
                    const int c = tt + k * T;
                    if (c < W) {
                        int p = c + st;
                        if (p >= W) p -= W;
                        const float2 ww = wl[c];
                        for (int r = 0; r < nr; ++r) {
                            const float z = cur[r * W + c] * ww.x + cur[r * W + p] * ww.y;
                            nxt[r * W + c] = last ? z : elu(z);
                        }
                    }
                }
            }
        }
        __syncthreads();
        cur = nxt;
        nxt = nxt == a ? b : a;
    }
    return cur;
}

// Buffer holding the result of a depth-layer mesh_team run with (a, b).
__device__ __forceinline__ float *mesh_result(float *a, float *b, int depth) { return (depth & 1) ? a : b; }

// Floats of one mesh buffer: rpw rows, at least `sweep` channels, 16-byte rows.
__host__ __device__ inline size_t mesh_buffer_floats(int W, int rpw, int sweep1, int sweep2) {
    const size_t n = std::max<size_t>(size_t(rpw) * W, size_t(std::max(sweep1, sweep2)));
    return (n + 3) / 4 * 4;
}

// Per-thread register capacity (float2) for weights loaded at kernel start:
// the projection + FFN meshes, and the Q/K/V meshes held until LDS frees up.
constexpr int kHoldPF = 16, kHoldQKV = 24;

template <int HOLD>
__device__ __forceinline__ void hold_load(float2 (&h)[HOLD], const float2 *__restrict__ src, int n) {
#pragma unroll
    for (int k = 0; k < HOLD; ++k) h[k] = src[min(k * int(blockDim.x) + int(threadIdx.x), n - 1)];
}

template <int HOLD>
__device__ __forceinline__ void hold_store(const float2 (&h)[HOLD], float2 *dst, int n) {
#pragma unroll
    for (int k = 0; k < HOLD; ++k) {
        const int i = k * int(blockDim.x) + int(threadIdx.x);
        if (i < n) dst[i] = h[k];
    }
}

// ------------------------------------------------------------ block kernel

// Post-attention half of block l-1 (reference.rs:194-216) fused with the
// pre-attention half of block l (reference.rs:164-193) for a tile of rows.
// One workgroup per `rpw` rows, teams x T threads.  STAGED: all mesh weights
// are read from global memory once at kernel start (the projection + FFN pair
// straight into LDS, the Q/K/V triple into registers until the post half has
// released LDS); otherwise the meshes read their weights from global memory.
template <int CPT, bool STAGED, int TEAMS>
__global__ void __launch_bounds__(768)
block_kernel(BlockArgs a) {
    // The projection and FFN meshes run on every thread of the block.
    constexpr int CPTW = TEAMS == 3 ? (CPT + 2) / 3 : CPT;
    extern __shared__ __align__(16) char smem[];
    LdsCarve lds{smem};
    const Shape &s = a.s;
    const int W = s.W, rpw = a.rpw;
    const int T = int(blockDim.x) / TEAMS, team = int(threadIdx.x) / T, tt = int(threadIdx.x) - team * T;
    const bool post = a.wproj != nullptr, pre = a.wq != nullptr;
    const int n_pf = (s.A + s.F) * W, n_qkv = 3 * s.A * W;
    float2 *S = lds.take<float2>(STAGED ? size_t(max(post ? n_pf : 0, pre ? n_qkv : 0)) : 0);
    float *X = lds.take<float>(size_t(rpw) * W);
    // Mesh buffers hold rpw rows, padded to the widest channel sweep so the
    // one-row path stores without bounds checks.  The 2*teams ping-pong buffers
    // are addressed by index (a pointer array would live in scratch memory).
    const size_t bstride = mesh_buffer_floats(W, rpw, CPT * T, CPTW * int(blockDim.x));
    float *N = lds.take<float>(bstride);
    float *bufs = lds.take<float>(bstride * 2 * TEAMS);
    auto buf = [bufs, bstride](int i) { return bufs + size_t(i) * bstride; };
    float *inv1 = lds.take<float>(size_t(rpw) * s.H);
    float *inv2 = lds.take<float>(size_t(rpw) * s.H);
    float *rinv = lds.take<float>(size_t(rpw));
    const int r0 = blockIdx.x * rpw, nr = min(rpw, a.ro.rows - r0);
    float *Y = buf(0), *Vs = buf(1);

    // 1. Every independent global load first: weights, rows, attention output.
    float2 hpf[STAGED ? kHoldPF : 1], hqkv[STAGED ? kHoldQKV : 1];
    if constexpr (STAGED) {
        if (post) hold_load<kHoldPF>(hpf, reinterpret_cast<const float2 *>(a.wproj), n_pf);
        else if (pre) hold_load<kHoldQKV>(hqkv, reinterpret_cast<const float2 *>(a.wq), n_qkv);
    }
    for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) {
        int r, c, h, d, seq, pos;
        split_row(idx, s, r, c);
        const int row = r0 + r;
        row_position(a.ro, row, seq, pos);
        float xv;
        if (a.embed) {
            const uint32_t tok = a.ro.tokens[size_t(seq) * a.ro.tok_stride + a.ro.tok_offset + pos];
            xv = a.E[size_t(tok) * W + c];
            a.x[size_t(row) * W + c] = xv;
        } else {
            xv = a.x[size_t(row) * W + c];
        }
        if (post) {
            split_head(c, s, h, d);
            float yv;
            if (a.part) {
                // Merge the split softmax states (m_s, l_s, acc_s) of this head.
                // Branch-free, so all 24 loads of a group of 8 splits stay in
                // flight together; an empty split (m = -inf) gets weight 0 and
                // the running maximum starts at a finite floor.
                const int stride = s.hdp + 2;
                const float *pp = a.part + (size_t(seq * s.H + h) * a.nsplit) * stride;
                float M = -1e30f, num = 0.0f, den = 0.0f;
                for (int k0 = 0; k0 < a.nsplit; k0 += 8) {
                    float m8[8], l8[8], a8[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const float *q = pp + size_t(min(k0 + u, a.nsplit - 1)) * stride;
                        m8[u] = q[s.hdp];
                        l8[u] = q[s.hdp + 1];
                        a8[u] = q[d];
                    }
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const float mu = k0 + u < a.nsplit ? m8[u] : -INFINITY;
                        const float mn = fmaxf(M, mu);
                        const float sold = exp2f(M - mn), snew = exp2f(mu - mn);
                        num = num * sold + a8[u] * snew;
                        den = den * sold + l8[u] * snew;
                        M = mn;
                    }
                }
                yv = num / den;
            } else {
                yv = a.ybuf[size_t(row) * W + c];
            }
            Y[idx] = yv;
            if (a.xsa_post) Vs[idx] = a.kv_post.v[(size_t(seq * s.H + h) * a.kv_post.cap + pos) * s.hdp + d];
        }
        X[idx] = xv;
    }
    if constexpr (STAGED) {
        if (post) hold_store<kHoldPF>(hpf, S, n_pf);
        else if (pre) hold_store<kHoldQKV>(hqkv, S, n_qkv);
    }
    __syncthreads();

    if (post) {
        // The Q/K/V weights load while the post half computes.
        if constexpr (STAGED) {
            if (pre) hold_load<kHoldQKV>(hqkv, reinterpret_cast<const float2 *>(a.wq), n_qkv);
        }
        const float2 *wp = STAGED ? S : reinterpret_cast<const float2 *>(a.wproj);
        const float2 *wf = wp + size_t(s.A) * W;
        if (a.xsa_post) {
            // XSA (reference.rs:577-603): z = y - (y.u)u with u = v / max(|v|, eps).
            segment_dots(Y, Vs, nr * s.H, s.hd, inv1, inv2);
            __syncthreads();
            for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) {
                int r, c, h, d;
                split_row(idx, s, r, c);
                split_head(c, s, h, d);
                const int sg = r * s.H + h;
                const float iv = rsqrtf(fmaxf(inv1[sg], kXsaFloor));
                Y[idx] = Y[idx] - (inv2[sg] * iv) * (Vs[idx] * iv);
            }
            __syncthreads();
        }
        const float *proj = mesh_team<CPTW>(Y, buf(1), N, nr, s, wp, s.A, threadIdx.x, blockDim.x, true);
        for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) X[idx] += proj[idx];
        __syncthreads();
        segment_inv_rms(X, nr, W, rinv);
        __syncthreads();
        float *Nf = proj == N ? buf(1) : N;  // a buffer the projection result does not occupy
        for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) {
            int r, c;
            split_row(idx, s, r, c);
            Nf[idx] = X[idx] * rinv[r];
        }
        __syncthreads();
        float *fa = Nf == N ? buf(0) : N, *fb = Nf == buf(1) ? buf(0) : buf(1);
        const float *ffn = mesh_team<CPTW>(Nf, fa, fb, nr, s, wf, s.F, threadIdx.x, blockDim.x, true);
        for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) {
            int r, c;
            split_row(idx, s, r, c);
            const float v = X[idx] + ffn[idx];
            X[idx] = v;
            a.x[size_t(r0 + r) * W + c] = v;
        }
        // The Q/K/V weights held since kernel start replace the post weights.
        if constexpr (STAGED) {
            if (pre) hold_store<kHoldQKV>(hqkv, S, n_qkv);
        }
    }
    __syncthreads();

    if (a.xn || pre) {
        // The next RMSNorm: the final one for the head, or the block's pre-norm.
        segment_inv_rms(X, nr, W, rinv);
        __syncthreads();
        for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) {
            int r, c;
            split_row(idx, s, r, c);
            const float v = X[idx] * rinv[r];
            N[idx] = v;
            if (a.xn) a.xn[size_t(r0 + r) * W + c] = v;
        }
        __syncthreads();
    }
    if (!pre) return;

    // Q, K and V meshes: concurrently with three teams, else one after another.
    const float2 *wqkv = STAGED ? S : reinterpret_cast<const float2 *>(a.wq);
    const size_t mesh = size_t(s.A) * W;
    const float *res0, *res1, *res2;
    if constexpr (TEAMS == 3) {
        mesh_team<CPT>(N, buf(2 * team), buf(2 * team + 1), nr, s, wqkv + team * mesh, s.A, tt, T, true);
        res0 = mesh_result(buf(0), buf(1), s.A);
        res1 = mesh_result(buf(2), buf(3), s.A);
        res2 = mesh_result(buf(4), buf(5), s.A);
    } else {
        // One team: Q's result is copied into X (free once x is normalised), K
        // stays in its buffer, and V alternates between the other buffer and N
        // (N is read only by V's first layer).
        const float *q = mesh_team<CPT>(N, buf(0), buf(1), nr, s, wqkv, s.A, tt, T, true);
        for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) X[idx] = q[idx];
        __syncthreads();
        const float *k = mesh_team<CPT>(N, buf(0), buf(1), nr, s, wqkv + mesh, s.A, tt, T, true);
        float *kres = const_cast<float *>(k);
        float *other = kres == buf(0) ? buf(1) : buf(0);
        res2 = mesh_team<CPT>(N, other, N, nr, s, wqkv + 2 * mesh, s.A, tt, T, true);
        res0 = X;
        res1 = kres;
    }
    // QK-Norm per head, split-half RoPE at each row's position, cache append
    // (each skipped when its switch is off, reference.rs:174-193).
    if (s.qk_norm) {
        segment_inv_rms(res0, nr * s.H, s.hd, inv1);
        segment_inv_rms(res1, nr * s.H, s.hd, inv2);
    } else {
        for (int i = threadIdx.x; i < nr * s.H; i += blockDim.x) inv1[i] = inv2[i] = 1.0f;
    }
    __syncthreads();
    if (!s.rope) {
        for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) {
            int r, c, h, d, seq, pos;
            split_row(idx, s, r, c);
            split_head(c, s, h, d);
            row_position(a.ro, r0 + r, seq, pos);
            a.q[size_t(r0 + r) * W + c] = res0[idx] * inv1[r * s.H + h];
            a.kv_pre.k[(size_t(seq * s.H + h) * a.kv_pre.cap + pos) * s.hdp + d] = res1[idx] * inv2[r * s.H + h];
        }
    }
    const int pairs = s.rope ? s.H * s.half : 0;
    for (int idx = threadIdx.x; idx < nr * pairs; idx += blockDim.x) {
        const int r = idx / pairs, rem = idx - r * pairs;
        const int h = rem / s.half, i = rem - h * s.half;
        const int row = r0 + r;
        int seq, pos;
        row_position(a.ro, row, seq, pos);
        const float2 cs = a.rope[size_t(pos) * s.half + i];
        const int lo_i = r * W + h * s.hd + i;
        {
            const float sc = inv1[r * s.H + h];
            const float x0 = res0[lo_i] * sc, x1 = res0[lo_i + s.half] * sc;
            float *dst = a.q + size_t(row) * W + h * s.hd;
            dst[i] = x0 * cs.x - x1 * cs.y;
            dst[i + s.half] = x1 * cs.x + x0 * cs.y;
        }
        {
            const float sc = inv2[r * s.H + h];
            const float x0 = res1[lo_i] * sc, x1 = res1[lo_i + s.half] * sc;
            float *dst = a.kv_pre.k + (size_t(seq * s.H + h) * a.kv_pre.cap + pos) * s.hdp;
            dst[i] = x0 * cs.x - x1 * cs.y;
            dst[i + s.half] = x1 * cs.x + x0 * cs.y;
        }
    }
    for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) {
        int r, c, h, d, seq, pos;
        split_row(idx, s, r, c);
        split_head(c, s, h, d);
        row_position(a.ro, r0 + r, seq, pos);
        a.kv_pre.v[(size_t(seq * s.H + h) * a.kv_pre.cap + pos) * s.hdp + d] = res2[idx];
    }
}

// ------------------------------------------------- decode block kernel
//
// Decode has one row per sequence, and a row's meshes are chains of dependent
// layers: latency, not bandwidth, bounds them.  Here each mesh of a row runs
// on ONE wavefront that keeps the whole row in registers (channel c = j*64 +
// lane sits in register j of lane `lane`, CPL = W/64 registers) and its layer
// weights in registers loaded at kernel start, so a layer is a few lane
// permutes and FMAs with no workgroup barrier.  Four waves per row, one per
// SIMD, so each may use the SIMD's whole register file (arch VGPRs + AGPRs):
//   wave 0    split merge, XSA, projection mesh, residual, RMSNorm, FFN mesh,
//             residual, next RMSNorm -> LDS N
//   wave 1-3  Q, K, V meshes from N; QK-Norm + RoPE; q row and cache append
// with one workgroup barrier between the two stages.

constexpr int kDecodeThreads = 256;

// Mesh layers whose weights one wave holds in registers at a time (2*D*CPL
// registers, sized so the kernel needs no scratch: 9 covers the depth-9
// meshes of width 512).
template <int CPL>
constexpr int wave_mesh_hold() {
    return CPL >= 16 ? 5 : (CPL >= 8 ? 9 : 16);
}

// w[u] = weights of layer l0 + u for the layers below depth.
template <int CPL, int D>
__device__ __forceinline__ void load_mesh_chunk(float2 (&w)[D][CPL], const float2 *__restrict__ wg, int l0,
                                                int depth, int lane) {
#pragma unroll
    for (int u = 0; u < D; ++u) {
        if (l0 + u < depth) {
            const float2 *wl = wg + size_t(l0 + u) * (CPL * 64);
#pragma unroll
            for (int j = 0; j < CPL; ++j) w[u][j] = wl[j * 64 + lane];
        }
    }
}

__device__ __forceinline__ float lane_read(float v, int byte_addr) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(byte_addr, __builtin_bit_cast(int, v)));
}

// Lane l gets v of lane (l + 1) mod 64 (DPP wave_rol:1, no LDS round trip).
// Every lane has a source, so no old value is needed (bound_ctrl), and the
// compiler can fold the move into the instruction that uses it.
__device__ __forceinline__ float wave_rotate1(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x134, 0xf, 0xf, true));
}

// Lanes 0-31 get lanes 32-63 of a, lanes 32-63 get lanes 0-31 of b: one
// v_permlane32_swap, which leaves (a.lo, b.lo) and (a.hi, b.hi).
__device__ __forceinline__ float halves_hi_lo(float a, float b, int lane) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, a), __builtin_bit_cast(int, b), false,
                                                     false);
    return __builtin_bit_cast(float, lane < 32 ? int(sw[1]) : int(sw[0]));
}

// f(integral_constant<int, I>) for I = 0..N-1, expanded by the front end:
// register-array indices built from I are constants before any optimisation
// pass runs, so a select between two elements never becomes a select of the
// index (which would turn the array into dynamically indexed memory).
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F &f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F &&f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// p[j] = value of channel (c + st) mod W for c = j*64 + lane.  For st < 64
// each lane offers register j, or j+1 when it is one of the first st lanes
// (their readers wrapped past lane 63), and the readers take lane (lane+st)
// mod 64; for st = 64k it is register (j + k) mod CPL of the same lane.
template <int CPL>
__device__ __forceinline__ void mesh_partner(const float (&x)[CPL], float (&p)[CPL], int st, int lane) {
    if (st < 64) {
        const int addr = ((lane + st) & 63) << 2;
        const bool next = lane < st;
        static_for<CPL>([&](auto J) {
            constexpr int j = decltype(J)::value;
            const float offer = next ? x[(j + 1) % CPL] : x[j];
            p[j] = lane_read(offer, addr);
        });
        return;
    }
    const int k = st >> 6;
    static_for<CPL>([&](auto K) {
        constexpr int kk = decltype(K)::value;
        if (kk > 0 && (kk & (kk - 1)) == 0 && k == kk) {
            static_for<CPL>([&](auto J) {
                constexpr int j = decltype(J)::value;
                p[j] = x[(j + kk) % CPL];
            });
        }
    });
}

// A mesh stack (reference.rs:422-453) over one row held by one wave.  w holds
// the first D layers' weights (loaded by the caller ahead of time); deeper
// stacks reload it D layers at a time.  With `next`, w is left holding the
// first layers of the next mesh (depth next_depth): when this stack fits in w,
// each slot is refilled right after its layer has run, so those loads overlap
// the rest of this stack.
template <int CPL, int D>
__device__ void wave_mesh(float (&x)[CPL], float2 (&w)[D][CPL], const float2 *__restrict__ wg, int depth,
                          const Shape &s, int lane, const float2 *__restrict__ next = nullptr,
                          int next_depth = 0) {
    const int W = CPL * 64;
    const bool refill = next != nullptr && depth <= D;
    int st = 1;
    for (int l0 = 0;; l0 += D) {
#pragma unroll
        for (int u = 0; u < D; ++u) {
            if (l0 + u < depth) {
                float p[CPL];
                mesh_partner<CPL>(x, p, st, lane);
                const bool last = l0 + u + 1 == depth;
#pragma unroll
                for (int j = 0; j < CPL; ++j) {
                    const float z = x[j] * w[u][j].x + p[j] * w[u][j].y;
                    x[j] = last ? z : elu(z);
                }
                if (s.butterfly) {
                    st <<= 1;
                    if (st >= W) st = 1;
                }
                if (refill && u < next_depth) {
                    const float2 *wl = next + size_t(u) * W;
#pragma unroll
                    for (int j = 0; j < CPL; ++j) w[u][j] = wl[j * 64 + lane];
                }
            }
        }
        if (l0 + D >= depth) break;
        load_mesh_chunk<CPL, D>(w, wg, l0 + D, depth, lane);
    }
    if (next != nullptr) {
        if (refill) {
            // Slots past this stack's depth.
#pragma unroll
            for (int u = 0; u < D; ++u) {
                if (u >= depth && u < next_depth) {
                    const float2 *wl = next + size_t(u) * W;
#pragma unroll
                    for (int j = 0; j < CPL; ++j) w[u][j] = wl[j * 64 + lane];
                }
            }
        } else {
            load_mesh_chunk<CPL, D>(w, next, 0, next_depth, lane);
        }
    }
}

// Fixed-depth form for butterfly meshes: all DEPTH layers unrolled into one
// straight-line block (no per-layer branch, so the scheduler overlaps a
// layer's lane permutes with the previous layer's tail), with each layer's
// stride a constant: strides >= 64 are register renames.
template <int CPL, int ST>
__device__ __forceinline__ void mesh_partner_c(const float (&x)[CPL], float (&p)[CPL], int lane) {
    if constexpr (ST < 64) {
        const int addr = ((lane + ST) & 63) << 2;
        const bool next = lane < ST;
        static_for<CPL>([&](auto J) {
            constexpr int j = decltype(J)::value;
            p[j] = lane_read(next ? x[(j + 1) % CPL] : x[j], addr);
        });
    } else {
        static_for<CPL>([&](auto J) {
            constexpr int j = decltype(J)::value;
            p[j] = x[(j + ST / 64) % CPL];
        });
    }
}

template <int CPL, int DEPTH>
__device__ __forceinline__ void load_mesh_all(float2 (&w)[DEPTH][CPL], const float2 *__restrict__ wg, int lane) {
    static_for<DEPTH>([&](auto U) {
        constexpr int u = decltype(U)::value;
#pragma unroll
        for (int j = 0; j < CPL; ++j) w[u][j] = wg[u * (CPL * 64) + j * 64 + lane];
    });
}

template <int CPL, int DEPTH>
__device__ __forceinline__ void wave_mesh_fixed(float (&x)[CPL], const float2 (&w)[DEPTH][CPL], int lane) {
    constexpr int LOG2W = CPL == 1 ? 6 : CPL == 2 ? 7 : CPL == 4 ? 8 : CPL == 8 ? 9 : 10;
    static_for<DEPTH>([&](auto U) {
        constexpr int u = decltype(U)::value;
        constexpr int ST = 1 << (u % LOG2W);
        float p[CPL];
        mesh_partner_c<CPL, ST>(x, p, lane);
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const float z = x[j] * w[u][j].x + p[j] * w[u][j].y;
            x[j] = u + 1 == DEPTH ? z : elu(z);
        }
    });
}

// out[j] = sum of v over the head holding channel j*64 + lane: HSEG lanes of
// one register (head width <= 64), or `rph` whole registers (64*rph wide).
template <int CPL, int HSEG>
__device__ __forceinline__ void head_sum(const float (&v)[CPL], float (&out)[CPL], int rph) {
    float t[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) t[j] = group_sum<HSEG>(v[j]);
    if (HSEG < 64 || rph == 1) {
#pragma unroll
        for (int j = 0; j < CPL; ++j) out[j] = t[j];
        return;
    }
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int g = j / rph;
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < CPL; ++k)
            if (k / rph == g) acc += t[k];
        out[j] = acc;
    }
}

// Merge of the split softmax states (m_s, l_s, acc_s) of one channel, G splits
// per round with clamped (branch-free) loads; an empty split (m = -inf) gets
// weight 0 and the running maximum starts at a finite floor.
template <int G>
__device__ __forceinline__ float merge_splits(const float *__restrict__ pp, int nsplit, int stride, int hdp,
                                              int d) {
    float M = -1e30f, num = 0.0f, den = 0.0f;
    for (int k0 = 0; k0 < nsplit; k0 += G) {
        float m8[G], l8[G], a8[G];
#pragma unroll
        for (int u = 0; u < G; ++u) {
            const float *q = pp + size_t(min(k0 + u, nsplit - 1)) * stride;
            m8[u] = q[hdp];
            l8[u] = q[hdp + 1];
            a8[u] = q[d];
        }
#pragma unroll
        for (int u = 0; u < G; ++u) {
            const float mu = k0 + u < nsplit ? m8[u] : -INFINITY;
            const float mn = fmaxf(M, mu);
            const float sold = exp2f(M - mn), snew = exp2f(mu - mn);
            num = num * sold + a8[u] * snew;
            den = den * sold + l8[u] * snew;
            M = mn;
        }
    }
    return num / den;
}

// 1/sqrt(mean(x^2) + eps) of the wave's row (reference.rs:392-409).
template <int CPL>
__device__ __forceinline__ float row_inv_rms(const float (&x)[CPL]) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) acc = fmaf(x[j], x[j], acc);
    return rsqrtf(wave_sum(acc) * (1.0f / float(CPL * 64)) + kRmsEps);
}

// One decode row per workgroup (Rows.rows_per_seq == 1); block semantics as
// block_kernel.  Requires W = 64*CPL and head width HSEG (<= 64) or a
// multiple of 64 (HSEG = 64).  DEPTH > 0: butterfly meshes with A = F =
// DEPTH (fixed-depth straight-line meshes, the FFN weights in registers of
// their own); DEPTH = 0: any depth and connectivity.
template <int CPL, int HSEG, int DEPTH>
__global__ void __launch_bounds__(kDecodeThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
block_decode_kernel(BlockArgs a) {
    constexpr int W = CPL * 64;
    constexpr bool FIXED = DEPTH > 0;
    constexpr int D = FIXED ? DEPTH : wave_mesh_hold<CPL>();
    static_assert(!FIXED || 4 * DEPTH * CPL <= 320, "two fixed meshes must fit the register file");
    __shared__ float N[W];
    const Shape &s = a.s;
    const int lane = int(threadIdx.x) & 63, wave = int(threadIdx.x) >> 6;
    const int row = blockIdx.x;
    int seq, pos;
    row_position(a.ro, row, seq, pos);
    const bool post = a.wproj != nullptr, pre = a.wq != nullptr;
    const int rph = HSEG < 64 ? 1 : s.hd >> 6;
    // Head and in-head dim of register j's channel.
    auto head_of = [&](int j) { return HSEG < 64 ? j * (64 / HSEG) + lane / HSEG : j / rph; };
    auto dim_of = [&](int j) { return HSEG < 64 ? lane % HSEG : (j % rph) * 64 + lane; };
    auto load_weights = [&](float2 (&w)[D][CPL], const float *wg, int depth) {
        if constexpr (FIXED) load_mesh_all<CPL, DEPTH>(w, reinterpret_cast<const float2 *>(wg), lane);
        else load_mesh_chunk<CPL, D>(w, reinterpret_cast<const float2 *>(wg), 0, depth, lane);
    };
    float2 w[D][CPL];
    float x[CPL];
    float2 cs[CPL];  // RoPE (cos, sin) of each channel's pair at this position (Q and K waves)

    if (wave == 0) {
        // Every load first: the row, the attention state, the meshes' weights.
        if (a.embed) {
            const uint32_t tok = a.ro.tokens[size_t(seq) * a.ro.tok_stride + a.ro.tok_offset + pos];
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                x[j] = a.E[size_t(tok) * W + j * 64 + lane];
                a.x[size_t(row) * W + j * 64 + lane] = x[j];
            }
        } else {
#pragma unroll
            for (int j = 0; j < CPL; ++j) x[j] = a.x[size_t(row) * W + j * 64 + lane];
        }
        if (post) {
            float y[CPL], v[CPL];
            float2 wf[FIXED ? D : 1][CPL];
            const int stride = s.hdp + 2;
            const float *part0 = a.part + size_t(seq * s.H) * a.nsplit * stride;
#pragma unroll
            for (int j = 0; j < CPL; ++j)
                v[j] = a.kv_post.v[(size_t(seq * s.H + head_of(j)) * a.kv_post.cap + pos) * s.hdp + dim_of(j)];
            if (a.nsplit <= 2) {
                float m2[CPL][2], l2[CPL][2], a2[CPL][2];
#pragma unroll
                for (int j = 0; j < CPL; ++j) {
                    const float *pp = part0 + size_t(head_of(j)) * a.nsplit * stride;
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const float *q = pp + size_t(min(u, a.nsplit - 1)) * stride;
                        m2[j][u] = q[s.hdp];
                        l2[j][u] = q[s.hdp + 1];
                        a2[j][u] = q[dim_of(j)];
                    }
                }
                load_weights(w, a.wproj, s.A);
                if constexpr (FIXED) load_mesh_all<CPL, DEPTH>(wf, reinterpret_cast<const float2 *>(a.wffn), lane);
                // Merge of the two split softmax states (see merge_splits).
#pragma unroll
                for (int j = 0; j < CPL; ++j) {
                    float M = -1e30f, num = 0.0f, den = 0.0f;
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const float mu = u < a.nsplit ? m2[j][u] : -INFINITY;
                        const float mn = fmaxf(M, mu);
                        const float sold = exp2f(M - mn), snew = exp2f(mu - mn);
                        num = num * sold + a2[j][u] * snew;
                        den = den * sold + l2[j][u] * snew;
                        M = mn;
                    }
                    y[j] = num / den;
                }
            } else {
                load_weights(w, a.wproj, s.A);
                if constexpr (FIXED) load_mesh_all<CPL, DEPTH>(wf, reinterpret_cast<const float2 *>(a.wffn), lane);
#pragma unroll
                for (int j = 0; j < CPL; ++j)
                    y[j] = merge_splits<8>(part0 + size_t(head_of(j)) * a.nsplit * stride, a.nsplit, stride,
                                           s.hdp, dim_of(j));
            }
            if (s.xsa) {
                // XSA (reference.rs:577-603): z = y - (y.u)u with u = v / max(|v|, eps).
                float vv[CPL], yv[CPL], t[CPL];
#pragma unroll
                for (int j = 0; j < CPL; ++j) t[j] = v[j] * v[j];
                head_sum<CPL, HSEG>(t, vv, rph);
#pragma unroll
                for (int j = 0; j < CPL; ++j) t[j] = y[j] * v[j];
                head_sum<CPL, HSEG>(t, yv, rph);
#pragma unroll
                for (int j = 0; j < CPL; ++j) {
                    const float iv = rsqrtf(fmaxf(vv[j], kXsaFloor));
                    y[j] = y[j] - (yv[j] * iv) * (v[j] * iv);
                }
            }
            if constexpr (FIXED) wave_mesh_fixed<CPL, DEPTH>(y, w, lane);
            else
                wave_mesh<CPL, D>(y, w, reinterpret_cast<const float2 *>(a.wproj), s.A, s, lane,
                                  reinterpret_cast<const float2 *>(a.wffn), s.F);
#pragma unroll
            for (int j = 0; j < CPL; ++j) x[j] += y[j];
            const float inv = row_inv_rms<CPL>(x);
#pragma unroll
            for (int j = 0; j < CPL; ++j) y[j] = x[j] * inv;
            if constexpr (FIXED) wave_mesh_fixed<CPL, DEPTH>(y, wf, lane);
            else wave_mesh<CPL, D>(y, w, reinterpret_cast<const float2 *>(a.wffn), s.F, s, lane);
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                x[j] += y[j];
                a.x[size_t(row) * W + j * 64 + lane] = x[j];
            }
        }
        if (a.xn || pre) {
            // The next RMSNorm: the final one for the head, or the block's pre-norm.
            const float inv = row_inv_rms<CPL>(x);
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const float v = x[j] * inv;
                N[j * 64 + lane] = v;
                if (a.xn) a.xn[size_t(row) * W + j * 64 + lane] = v;
            }
        }
    } else if (pre) {
        load_weights(w, wave == 1 ? a.wq : (wave == 2 ? a.wk : a.wv), s.A);
        if (wave < 3) {
            const float2 *rope = a.rope + size_t(pos) * s.half;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const int d = dim_of(j);
                cs[j] = rope[d < s.half ? d : d - s.half];
            }
        }
    }
    __syncthreads();
    if (wave == 0 || !pre) return;

#pragma unroll
    for (int j = 0; j < CPL; ++j) x[j] = N[j * 64 + lane];
    if constexpr (FIXED) wave_mesh_fixed<CPL, DEPTH>(x, w, lane);
    else
        wave_mesh<CPL, D>(x, w, reinterpret_cast<const float2 *>(wave == 1 ? a.wq : (wave == 2 ? a.wk : a.wv)), s.A,
                          s, lane);
    const size_t cache_row = size_t(seq * s.H) * a.kv_pre.cap + pos;  // + head * cap, then * hdp
    if (wave == 3) {
#pragma unroll
        for (int j = 0; j < CPL; ++j)
            a.kv_pre.v[(cache_row + size_t(head_of(j)) * a.kv_pre.cap) * s.hdp + dim_of(j)] = x[j];
        return;
    }
    // QK-Norm per head, then split-half RoPE at the row's position.
    float sq[CPL], ss[CPL], other[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) sq[j] = x[j] * x[j];
    head_sum<CPL, HSEG>(sq, ss, rph);
    const int half = s.half;
    if (HSEG < 64 || rph == 1) {
#pragma unroll
        for (int j = 0; j < CPL; ++j) other[j] = __shfl_xor(x[j], half, 64);
    } else {
        const int m = half >> 6;  // partner register offset j ^ m
        static_for<CPL>([&](auto M) {
            constexpr int mm = decltype(M)::value;
            if (mm > 0 && (mm & (mm - 1)) == 0 && m == mm) {
                static_for<CPL>([&](auto J) {
                    constexpr int j = decltype(J)::value;
                    other[j] = x[j ^ mm];
                });
            }
        });
    }
    const float scale = 1.0f / float(s.hd);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int d = dim_of(j);
        const float sc = s.qk_norm ? rsqrtf(ss[j] * scale + kRmsEps) : 1.0f;
        const float self = x[j] * sc, oth = other[j] * sc;
        const float r = !s.rope ? self : (d < half ? self * cs[j].x - oth * cs[j].y : self * cs[j].x + oth * cs[j].y);
        if (wave == 1)
            a.q[size_t(row) * W + j * 64 + lane] = r;
        else
            a.kv_pre.k[(cache_row + size_t(head_of(j)) * a.kv_pre.cap) * s.hdp + d] = r;
    }
}

// --------------------------------------------------- row decode kernel
//
// A faster decode block: the channels of a row are spread over NW waves,
// channel c = wave + NW*(lane + 64*j) for j < CPL (W = 64*NW*CPL).  With this
// map a butterfly stride st < NW crosses waves (one LDS exchange and barrier),
// NW <= st < 64*NW rotates lanes inside every wave (ds_bpermute, no barrier),
// and larger strides only rename registers, so most layers of a width-512
// mesh never wait on a barrier.  Each row runs on three workgroups (teams):
// all three compute the post-attention half of block l-1 (the projection and
// FFN meshes are short, serial and cheap to repeat), then team 0 computes Q
// (and owns the residual row), team 1 K and team 2 V of block l, so the three
// meshes run on three CUs at once.  Mesh weights, token vectors and the
// residual rows are stored pre-permuted into this map ("row order": element
// (j*NW + wave)*64 + lane holds channel c), so every wave's loads are
// contiguous.

// LDS exchange with the channel st < NW further on.  Double-buffered: the
// write of exchange k+2 follows the barrier of exchange k+1, which every wave
// reaches only after its reads of exchange k.
template <int NW, int CPL>
__device__ __forceinline__ void row_partner(const float (&x)[CPL], float (&p)[CPL], int st, int lane, int wave,
                                            float *xch, int &parity) {
    if (st < NW) {
        float *b = xch + (parity & 1) * (NW * CPL * 64);
        ++parity;
#pragma unroll
        for (int j = 0; j < CPL; ++j) b[(j * NW + wave) * 64 + lane] = x[j];
        __syncthreads();
        int w2 = wave + st, l2 = lane, jc = 0;
        if (w2 >= NW) {
            w2 -= NW;
            ++l2;
        }
        if (l2 >= 64) {
            l2 -= 64;
            jc = 1;
        }
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int j2 = j + jc < CPL ? j + jc : 0;
            p[j] = b[(j2 * NW + w2) * 64 + l2];
        }
    } else if (st < 64 * NW) {
        // Reader lane l takes lane (l + k) mod 64; readers that wrap past lane
        // 63 need the next register, and they read exactly the lanes < k.
        // Rotations by 1 and 2 lanes are DPP wave rotations and by 32 a
        // half swap; the others go through the LDS crossbar (ds_bpermute).
        const int k = st / NW;
        const bool next = lane < k;
        if (k == 1 || k == 2) {
            static_for<CPL>([&](auto J) {
                constexpr int j = decltype(J)::value;
                const float r = wave_rotate1(next ? x[(j + 1) % CPL] : x[j]);
                p[j] = k == 1 ? r : wave_rotate1(r);
            });
        } else if (k == 32 && CPL == 2) {
            // Two swaps in place: (x0, x1) -> ([x0.lo, x1.lo], [x0.hi, x1.hi])
            // gives p0, and swapping those back the other way round
            // ([x0.hi, x0.lo], [x1.hi, x1.lo]) gives p1, with no copies.
            const auto s = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, x[0]),
                                                            __builtin_bit_cast(int, x[1 % CPL]), false, false);
            p[0] = __builtin_bit_cast(float, lane < 32 ? int(s[1]) : int(s[0]));
            const auto t = __builtin_amdgcn_permlane32_swap(int(s[1]), int(s[0]), false, false);
            p[1 % CPL] = __builtin_bit_cast(float, lane < 32 ? int(t[1]) : int(t[0]));
        } else if (k == 32) {
            static_for<CPL>([&](auto J) {
                constexpr int j = decltype(J)::value;
                p[j] = halves_hi_lo(x[j], x[(j + 1) % CPL], lane);
            });
        } else {
            const int addr = ((lane + k) & 63) << 2;
            static_for<CPL>([&](auto J) {
                constexpr int j = decltype(J)::value;
                p[j] = lane_read(next ? x[(j + 1) % CPL] : x[j], addr);
            });
        }
    } else {
        const int m = st / (64 * NW);
        static_for<CPL>([&](auto M) {
            constexpr int mm = decltype(M)::value;
            if (mm > 0 && m == mm) {
                static_for<CPL>([&](auto J) {
                    constexpr int j = decltype(J)::value;
                    p[j] = x[(j + mm) % CPL];
                });
            }
        });
    }
}

template <int NW, int CPL>
__device__ __forceinline__ void row_layer(float (&x)[CPL], const float2 (&w)[CPL], int st, bool last, int lane,
                                          int wave, float *xch, int &parity) {
    // The lane's own term first: x is then dead by the time the partner
    // exchange runs, which may consume it (row_partner's in-place swaps).
    float p[CPL], own[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) own[j] = x[j] * w[j].x;
    row_partner<NW, CPL>(x, p, st, lane, wave, xch, parity);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const float z = fmaf(p[j], w[j].y, own[j]);
        x[j] = last ? z : elu_log2(z);
    }
}

// Weights of mesh layer u in row order: float2 (u*CPL + j)*NW*64 + wave*64 + lane.
template <int NW, int CPL, int D>
__device__ __forceinline__ void row_load_weights(float2 (&w)[D][CPL], const float *wg, int lane, int wave) {
    // A uniform base and 32-bit lane offsets: one address register for all
    // the loads instead of a 64-bit address per load.  The weights are in
    // global memory, said so that the loads are global rather than flat ones
    // (which would also count in the LDS wait counter).
    const global_u64 *g = (const global_u64 *)wg;  // a float2 per word
    const uint32_t at = uint32_t(wave * 64 + lane);
#pragma unroll
    for (int u = 0; u < D; ++u)
#pragma unroll
        for (int j = 0; j < CPL; ++j) w[u][j] = __builtin_bit_cast(float2, uint64_t(g[at + uint32_t((u * CPL + j) * NW * 64)]));
}

// A butterfly mesh stack of compile-time depth D (reference.rs:422-453): all
// layers unrolled, each stride a constant.
template <int NW, int CPL, int D>
__device__ __forceinline__ void row_mesh_fixed(float (&x)[CPL], const float2 (&w)[D][CPL], int lane, int wave,
                                               float *xch, int &parity) {
    constexpr int W = 64 * NW * CPL;
    constexpr int LOG2W = W == 128 ? 7 : W == 256 ? 8 : W == 512 ? 9 : 10;
    static_for<D>([&](auto U) {
        constexpr int u = decltype(U)::value;
        row_layer<NW, CPL>(x, w[u], 1 << (u % LOG2W), u + 1 == D, lane, wave, xch, parity);
    });
}

// Any depth and connectivity: weights stream from global memory one layer ahead.
template <int NW, int CPL>
__device__ void row_mesh(float (&x)[CPL], const float *wg, int depth, const Shape &s, int lane, int wave,
                         float *xch, int &parity) {
    const float2 *g = reinterpret_cast<const float2 *>(wg) + wave * 64 + lane;
    float2 wn[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) wn[j] = g[j * NW * 64];
    for (int u = 0; u < depth; ++u) {
        float2 wc[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j) wc[j] = wn[j];
        if (u + 1 < depth) {
#pragma unroll
            for (int j = 0; j < CPL; ++j) wn[j] = g[((u + 1) * CPL + j) * NW * 64];
        }
        const int st = s.butterfly ? (1 << (u % s.log2w)) : 1;
        row_layer<NW, CPL>(x, wc, st, u + 1 == depth, lane, wave, xch, parity);
    }
}

// Sum over the whole row, in every lane (fixed order: waves 0..NW-1).
template <int NW>
__device__ __forceinline__ float row_total(float v, int lane, int wave, float *red) {
    v = wave_sum(v);
    if constexpr (NW == 1) return v;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) t += red[w];
    return t;
}

// Per-head sums: register j of lane `lane` holds head lane/GL + (64/GL)*j at
// dim NW*(lane % GL) + wave, so a head is GL lanes of every wave.
template <int NW, int CPL, int GL>
__device__ __forceinline__ void row_head_sums(const float (&v)[CPL], float (&out)[CPL], int lane, int wave,
                                              float *red) {
    constexpr int G = 64 / GL;
    float t[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) t[j] = group_sum<GL>(v[j]);
    if constexpr (NW == 1) {
#pragma unroll
        for (int j = 0; j < CPL; ++j) out[j] = t[j];
        return;
    }
    if (lane % GL == 0) {
#pragma unroll
        for (int j = 0; j < CPL; ++j) red[(j * NW + wave) * G + lane / GL] = t[j];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        float a = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) a += red[(j * NW + w) * G + lane / GL];
        out[j] = a;
    }
}

// Lane geometry and LDS of one row held by NW waves (see row_partner).
template <int NW, int CPL, int GL>
struct RowCtx {
    static constexpr int W = 64 * NW * CPL, G = 64 / GL, SLOT = CPL * NW * G;
    int lane, wave, parity;
    float *xch;  // 2*W floats: mesh exchange buffers
    float *red;  // reduction slots of SLOT floats each
    __device__ RowCtx(float *x, float *r, int tid = int(threadIdx.x))
        : lane(tid & 63), wave(tid >> 6), parity(0), xch(x), red(r) {}
    // Head and in-head dim of register j: a head is GL lanes of every wave.
    __device__ int head_of(int j) const { return lane / GL + G * j; }
    __device__ int dim() const { return NW * (lane % GL) + wave; }
    __device__ int ridx(int j) const { return (j * NW + wave) * 64 + lane; }  // row-order index
    __device__ int chan(int j) const { return wave + NW * (lane + 64 * j); }   // channel
    __device__ float *slot(int k) const { return red + k * SLOT; }
};

// A mesh stack on the row: fixed depth (weights in registers) or any depth;
// x in and out in the log2(e)-scaled units of row_layer.
template <int NW, int CPL, int GL, int D>
__device__ __forceinline__ void row_run_mesh(RowCtx<NW, CPL, GL> &c, float (&x)[CPL], const float2 (&w)[D][CPL],
                                             const float *wg, int depth, const Shape &s, bool fixed) {
    if (fixed) row_mesh_fixed<NW, CPL, D>(x, w, c.lane, c.wave, c.xch, c.parity);
    else row_mesh<NW, CPL>(x, wg, depth, s, c.lane, c.wave, c.xch, c.parity);
}

// XSA (reference.rs:577-603): y <- y - (y.u)u with u = v / max(|v|, eps) per head.
template <int NW, int CPL, int GL>
__device__ __forceinline__ void row_xsa(RowCtx<NW, CPL, GL> &c, float (&y)[CPL], const float (&v)[CPL]) {
    float vv[CPL], yv[CPL], t[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) t[j] = v[j] * v[j];
    row_head_sums<NW, CPL, GL>(t, vv, c.lane, c.wave, c.slot(0));
#pragma unroll
    for (int j = 0; j < CPL; ++j) t[j] = y[j] * v[j];
    row_head_sums<NW, CPL, GL>(t, yv, c.lane, c.wave, c.slot(1));
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const float iv = rsqrtf(fmaxf(vv[j], kXsaFloor));
        y[j] = y[j] - (yv[j] * iv) * (v[j] * iv);
    }
}

// 1/sqrt(mean(x^2) + eps) over the row (reference.rs:392-409).
template <int NW, int CPL, int GL>
__device__ __forceinline__ float row_inv_rms(RowCtx<NW, CPL, GL> &c, const float (&x)[CPL], int k) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) acc = fmaf(x[j], x[j], acc);
    return rsqrtf(row_total<NW>(acc, c.lane, c.wave, c.slot(k)) * (1.0f / float(c.W)) + kRmsEps);
}

// n = mesh(x * inv_rms(x)), scaled by log2(e) (elu_log2), for a
// compile-time-depth mesh whose first stride
// (1) crosses waves: the row reduction of the RMSNorm and that layer's LDS
// exchange share one barrier (x is exchanged and each lane scales its partner
// itself).  Same arithmetic as row_inv_rms, then row_run_mesh on x * inv.
template <int NW, int CPL, int GL, int D>
__device__ __forceinline__ void row_rms_mesh(RowCtx<NW, CPL, GL> &c, const float (&x)[CPL], float (&n)[CPL],
                                             const float2 (&w)[D][CPL], int k) {
    static_assert(NW > 1 && D >= 1, "the first layer's stride 1 crosses waves");
    constexpr int W = 64 * NW * CPL;
    constexpr int LOG2W = W == 128 ? 7 : W == 256 ? 8 : W == 512 ? 9 : 10;
    const int lane = c.lane, wave = c.wave;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) acc = fmaf(x[j], x[j], acc);
    acc = wave_sum(acc);
    float *red = c.slot(k);
    if (lane == 0) red[wave] = acc;
    float *b = c.xch + (c.parity & 1) * (NW * CPL * 64);
    ++c.parity;
#pragma unroll
    for (int j = 0; j < CPL; ++j) b[(j * NW + wave) * 64 + lane] = x[j];
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int v = 0; v < NW; ++v) t += red[v];
    const float inv = inv_rms_log2(t, W);
    // Partner of channel c is c + 1: the next wave, or wave 0 one lane on.
    int w2 = wave + 1, l2 = lane, jc = 0;
    if (w2 >= NW) {
        w2 -= NW;
        ++l2;
    }
    if (l2 >= 64) {
        l2 -= 64;
        jc = 1;
    }
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int j2 = j + jc < CPL ? j + jc : 0;
        const float nx = x[j] * inv, np = b[(j2 * NW + w2) * 64 + l2] * inv;
        const float z = nx * w[0][j].x + np * w[0][j].y;
        n[j] = D == 1 ? z : elu_log2(z);
    }
    static_for<D>([&](auto U) {
        constexpr int u = decltype(U)::value;
        if constexpr (u > 0) row_layer<NW, CPL>(n, w[u], 1 << (u % LOG2W), u + 1 == D, lane, wave, c.xch, c.parity);
    });
}

// Post-attention half of a block (reference.rs:194-216) on the residual row x,
// given the attention output y and the row's own value vector v.
// With XSA false, y arrives with XSA applied (v unused).
template <int NW, int CPL, int GL, int D, bool XSA = true>
__device__ __forceinline__ void row_post(RowCtx<NW, CPL, GL> &c, float (&x)[CPL], float (&y)[CPL],
                                         const float (&v)[CPL], const float2 (&wp)[D][CPL],
                                         const float2 (&wf)[D][CPL], const float *gp, const float *gf,
                                         const Shape &s, bool fixed) {
    if constexpr (XSA) row_xsa(c, y, v);
#pragma unroll
    for (int j = 0; j < CPL; ++j) y[j] *= kLog2e;
    row_run_mesh(c, y, wp, gp, s.A, s, fixed);
#pragma unroll
    for (int j = 0; j < CPL; ++j) x[j] = fmaf(y[j], kLn2, x[j]);
    if constexpr (NW > 1 && D > 1) {
        if (fixed) {
            row_rms_mesh(c, x, y, wf, 2);
#pragma unroll
            for (int j = 0; j < CPL; ++j) x[j] = fmaf(y[j], kLn2, x[j]);
            return;
        }
    }
    const float inv = row_inv_rms(c, x, 2) * kLog2e;
#pragma unroll
    for (int j = 0; j < CPL; ++j) y[j] = x[j] * inv;
    row_run_mesh(c, y, wf, gf, s.F, s, fixed);
#pragma unroll
    for (int j = 0; j < CPL; ++j) x[j] = fmaf(y[j], kLn2, x[j]);
}

// QK-Norm per head, then split-half RoPE (reference.rs:462-482) at the position
// whose (cos, sin) pair for this lane's dim is cs: the pair partner (dim +-
// hd/2) is GL/2 lanes away in the same wave and register.
template <int NW, int CPL, int GL>
__device__ __forceinline__ void row_qk_rope(RowCtx<NW, CPL, GL> &c, float (&x)[CPL], float2 cs, const Shape &s) {
    float sq[CPL], ss[CPL], other[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) sq[j] = x[j] * x[j];
    row_head_sums<NW, CPL, GL>(sq, ss, c.lane, c.wave, c.slot(4));
#pragma unroll
    for (int j = 0; j < CPL; ++j) other[j] = __shfl_xor(x[j], GL / 2, 64);
    const float scale = 1.0f / float(s.hd);
    const bool low = c.dim() < s.half;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const float sc = rsqrtf(ss[j] * scale + kRmsEps);
        const float self = x[j] * sc, oth = other[j] * sc;
        x[j] = low ? self * cs.x - oth * cs.y : self * cs.x + oth * cs.y;
    }
}

__device__ __forceinline__ float2 rope_pair(const float2 *rope, int pos, int dim, int half) {
    return rope[size_t(pos) * half + (dim < half ? dim : dim - half)];
}

// One decode row (Rows.rows_per_seq == 1) per `teams` workgroups of 64*NW
// threads; block semantics as block_kernel.  DEPTH > 0: butterfly meshes with
// A = F = DEPTH held in registers; DEPTH = 0: any depth and connectivity.
// Requires hd = GL*NW with GL <= 64 (a head is GL lanes of every wave).
template <int NW, int CPL, int GL, int DEPTH>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(1, 1)))
row_block_kernel(BlockArgs a) {
    using Ctx = RowCtx<NW, CPL, GL>;
    constexpr int W = Ctx::W;
    constexpr bool FIXED = DEPTH > 0;
    constexpr int D = FIXED ? DEPTH : 1;
    __shared__ float xch[2 * W];
    __shared__ float red[8 * Ctx::SLOT];
    Ctx c(xch, red);
    const Shape &s = a.s;
    const bool pre = a.wq != nullptr, post = a.wproj != nullptr;
    const int teams = pre ? 3 : 1;
    const int row = int(blockIdx.x) / teams, team = int(blockIdx.x) - row * teams;
    int seq, pos;
    row_position(a.ro, row, seq, pos);
    const int dim = c.dim();

    // Every independent load first: row, attention state, weights.
    float x[CPL];
    if (a.embed) {
        const uint32_t tok = a.ro.tokens[size_t(seq) * a.ro.tok_stride + a.ro.tok_offset + pos];
#pragma unroll
        for (int j = 0; j < CPL; ++j) x[j] = a.E[size_t(tok) * W + c.ridx(j)];
    } else {
#pragma unroll
        for (int j = 0; j < CPL; ++j) x[j] = a.x[size_t(row) * W + c.ridx(j)];
    }
    const float *wmine = pre ? (team == 0 ? a.wq : team == 1 ? a.wk : a.wv) : nullptr;
    float2 wp[D][CPL], wf[D][CPL], wm[D][CPL];
    if constexpr (FIXED) {
        if (post) {
            row_load_weights<NW, CPL, D>(wp, a.wproj, c.lane, c.wave);
            row_load_weights<NW, CPL, D>(wf, a.wffn, c.lane, c.wave);
        }
        if (pre) row_load_weights<NW, CPL, D>(wm, wmine, c.lane, c.wave);
    }

    if (post) {
        float y[CPL], v[CPL];
        const int stride = s.hdp + 2;
        const float *part0 = a.part + size_t(seq * s.H) * a.nsplit * stride;
#pragma unroll
        for (int j = 0; j < CPL; ++j)
            v[j] = a.kv_post.v[(size_t(seq * s.H + c.head_of(j)) * a.kv_post.cap + pos) * s.hdp + dim];
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const float *pp = part0 + size_t(c.head_of(j)) * a.nsplit * stride;
            y[j] = a.nsplit <= 2 ? merge_splits<2>(pp, a.nsplit, stride, s.hdp, dim)
                                 : merge_splits<8>(pp, a.nsplit, stride, s.hdp, dim);
        }
        row_post(c, x, y, v, wp, wf, a.wproj, a.wffn, s, FIXED);
    }
    if (team == 0 && (post || a.embed)) {
        // Into x_out, never x: the row's other workgroups may not have read x yet.
#pragma unroll
        for (int j = 0; j < CPL; ++j) a.x_out[size_t(row) * W + c.ridx(j)] = x[j];
    }
    if (!a.xn && !pre) return;

    // The next RMSNorm: the final one for the head, or the block's pre-norm.
    const float inv = row_inv_rms(c, x, 3);
#pragma unroll
    for (int j = 0; j < CPL; ++j) x[j] *= inv;
    if (a.xn) {
#pragma unroll
        for (int j = 0; j < CPL; ++j) a.xn[size_t(row) * W + c.chan(j)] = x[j];
    }
    if (!pre) return;

#pragma unroll
    for (int j = 0; j < CPL; ++j) x[j] *= kLog2e;
    row_run_mesh(c, x, wm, wmine, s.A, s, FIXED);
#pragma unroll
    for (int j = 0; j < CPL; ++j) x[j] *= kLn2;
    const size_t cache_row = size_t(seq * s.H) * a.kv_pre.cap + pos;  // + head * cap, then * hdp
    if (team == 2) {
#pragma unroll
        for (int j = 0; j < CPL; ++j)
            a.kv_pre.v[(cache_row + size_t(c.head_of(j)) * a.kv_pre.cap) * s.hdp + dim] = x[j];
        return;
    }
    row_qk_rope(c, x, rope_pair(a.rope, pos, dim, s.half), s);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        if (team == 0)
            a.q[size_t(row) * W + c.chan(j)] = x[j];
        else
            a.kv_pre.k[(cache_row + size_t(c.head_of(j)) * a.kv_pre.cap) * s.hdp + dim] = x[j];
    }
}

// ---- Several decode rows per workgroup
//
// row_block_kernel's block for RB rows at once, for batches whose three
// workgroups per row would not fit the GPU in one wave of workgroups: every
// lane holds the same channels of RB rows, so each mesh weight in its
// registers serves RB rows, the rows' independent chains overlap in every
// wave, and a layer whose partner channel is in another wave exchanges all RB
// rows around one barrier.  Fixed-depth butterfly meshes only.

template <int NW, int CPL, int RB>
__device__ __forceinline__ void rows_partner(const float (&x)[RB][CPL], float (&p)[RB][CPL], int st, int lane,
                                             int wave, float *xch, int &parity) {
    constexpr int W = 64 * NW * CPL;
    if (st < NW) {
        float *b = xch + (parity & 1) * (RB * W);
        ++parity;
#pragma unroll
        for (int r = 0; r < RB; ++r)
#pragma unroll
            for (int j = 0; j < CPL; ++j) b[r * W + (j * NW + wave) * 64 + lane] = x[r][j];
        __syncthreads();
        int w2 = wave + st, l2 = lane, jc = 0;
        if (w2 >= NW) {
            w2 -= NW;
            ++l2;
        }
        if (l2 >= 64) {
            l2 -= 64;
            jc = 1;
        }
#pragma unroll
        for (int r = 0; r < RB; ++r)
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const int j2 = j + jc < CPL ? j + jc : 0;
                p[r][j] = b[r * W + (j2 * NW + w2) * 64 + l2];
            }
    } else {
        // In-wave partners (row_partner touches no LDS for these strides).
#pragma unroll
        for (int r = 0; r < RB; ++r) row_partner<NW, CPL>(x[r], p[r], st, lane, wave, xch, parity);
    }
}

// x in and out in the log2(e)-scaled units of row_layer.
template <int NW, int CPL, int D, int RB>
__device__ __forceinline__ void rows_mesh_fixed(float (&x)[RB][CPL], const float2 (&w)[D][CPL], int lane, int wave,
                                                float *xch, int &parity) {
    constexpr int W = 64 * NW * CPL;
    constexpr int LOG2W = W == 128 ? 7 : W == 256 ? 8 : W == 512 ? 9 : 10;
    static_for<D>([&](auto U) {
        constexpr int u = decltype(U)::value;
        float p[RB][CPL];
        rows_partner<NW, CPL, RB>(x, p, 1 << (u % LOG2W), lane, wave, xch, parity);
#pragma unroll
        for (int r = 0; r < RB; ++r)
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const float z = x[r][j] * w[u][j].x + p[r][j] * w[u][j].y;
                x[r][j] = u + 1 == D ? z : elu_log2(z);
            }
    });
}

// LDS of the multi-row block: the exchange buffers of rows_partner and
// reduction slots of RB * SLOT floats.
template <int NW, int CPL, int GL, int RB>
struct RowsCtx {
    static constexpr int W = 64 * NW * CPL, G = 64 / GL, SLOT = CPL * NW * G;
    int lane, wave, parity;
    float *xch, *red;
    __device__ RowsCtx(float *x, float *r) : lane(int(threadIdx.x) & 63), wave(int(threadIdx.x) >> 6), parity(0),
                                             xch(x), red(r) {}
    __device__ int head_of(int j) const { return lane / GL + G * j; }
    __device__ int dim() const { return NW * (lane % GL) + wave; }
    __device__ int ridx(int j) const { return (j * NW + wave) * 64 + lane; }
    __device__ int chan(int j) const { return wave + NW * (lane + 64 * j); }
    __device__ float *slot(int k) const { return red + k * RB * SLOT; }
};

// inv[r] = 1/sqrt(mean(x_r^2) + eps) for every row (row_inv_rms's order).
template <int NW, int CPL, int GL, int RB>
__device__ __forceinline__ void rows_inv_rms(const RowsCtx<NW, CPL, GL, RB> &c, const float (&x)[RB][CPL], int k,
                                             float (&inv)[RB]) {
    float *red = c.slot(k);
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) acc = fmaf(x[r][j], x[r][j], acc);
        acc = wave_sum(acc);
        if (c.lane == 0) red[r * NW + c.wave] = acc;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        float t = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) t += red[r * NW + w];
        inv[r] = rsqrtf(t * (1.0f / float(c.W)) + kRmsEps);
    }
}

// Per-head sums of every row (row_head_sums's order).
template <int NW, int CPL, int GL, int RB>
__device__ __forceinline__ void rows_head_sums(const RowsCtx<NW, CPL, GL, RB> &c, const float (&v)[RB][CPL],
                                               float (&out)[RB][CPL], int k) {
    constexpr int G = 64 / GL, SLOT = RowsCtx<NW, CPL, GL, RB>::SLOT;
    float *red = c.slot(k);
    float t[RB][CPL];
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int j = 0; j < CPL; ++j) t[r][j] = group_sum<GL>(v[r][j]);
    if (c.lane % GL == 0) {
#pragma unroll
        for (int r = 0; r < RB; ++r)
#pragma unroll
            for (int j = 0; j < CPL; ++j) red[r * SLOT + (j * NW + c.wave) * G + c.lane / GL] = t[r][j];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            float a = 0.0f;
#pragma unroll
            for (int w = 0; w < NW; ++w) a += red[r * SLOT + (j * NW + w) * G + c.lane / GL];
            out[r][j] = a;
        }
}

template <int NW, int CPL, int GL, int DEPTH, int RB>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(1, 1)))
row_block_rows_kernel(BlockArgs a) {
    using Ctx = RowsCtx<NW, CPL, GL, RB>;
    constexpr int W = Ctx::W, D = DEPTH;
    static_assert(DEPTH > 0 && NW > 1, "fixed-depth meshes over several waves");
    __shared__ float xch[2 * RB * W];
    __shared__ float red[8 * RB * Ctx::SLOT];
    Ctx c(xch, red);
    const Shape &s = a.s;
    const bool pre = a.wq != nullptr, post = a.wproj != nullptr;
    const int teams = pre ? 3 : 1;
    const int group = int(blockIdx.x) / teams, team = int(blockIdx.x) - group * teams;
    const int dim = c.dim();
    // Rows past the batch repeat its last row and write nothing.
    int row[RB], seq[RB], pos[RB];
    bool valid[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        valid[r] = group * RB + r < a.ro.rows;
        row[r] = min(group * RB + r, a.ro.rows - 1);
        row_position(a.ro, row[r], seq[r], pos[r]);
    }

    float x[RB][CPL];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        if (a.embed) {
            const uint32_t tok = a.ro.tokens[size_t(seq[r]) * a.ro.tok_stride + a.ro.tok_offset + pos[r]];
#pragma unroll
            for (int j = 0; j < CPL; ++j) x[r][j] = a.E[size_t(tok) * W + c.ridx(j)];
        } else {
#pragma unroll
            for (int j = 0; j < CPL; ++j) x[r][j] = a.x[size_t(row[r]) * W + c.ridx(j)];
        }
    }
    const float *wmine = pre ? (team == 0 ? a.wq : team == 1 ? a.wk : a.wv) : nullptr;
    float2 wp[D][CPL], wf[D][CPL], wm[D][CPL];
    if (post) {
        row_load_weights<NW, CPL, D>(wp, a.wproj, c.lane, c.wave);
        row_load_weights<NW, CPL, D>(wf, a.wffn, c.lane, c.wave);
    }
    if (pre) row_load_weights<NW, CPL, D>(wm, wmine, c.lane, c.wave);

    if (post) {
        // Post-attention half of the block (row_post): XSA, projection mesh,
        // residual, RMSNorm, FFN mesh, residual.
        float y[RB][CPL], v[RB][CPL];
        const int stride = s.hdp + 2;
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const float *part0 = a.part + size_t(seq[r] * s.H) * a.nsplit * stride;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                v[r][j] = a.kv_post.v[(size_t(seq[r] * s.H + c.head_of(j)) * a.kv_post.cap + pos[r]) * s.hdp + dim];
                const float *pp = part0 + size_t(c.head_of(j)) * a.nsplit * stride;
                y[r][j] = a.nsplit <= 2 ? merge_splits<2>(pp, a.nsplit, stride, s.hdp, dim)
                                        : merge_splits<8>(pp, a.nsplit, stride, s.hdp, dim);
            }
        }
        {
            float t[RB][CPL], vv[RB][CPL], yv[RB][CPL];
#pragma unroll
            for (int r = 0; r < RB; ++r)
#pragma unroll
                for (int j = 0; j < CPL; ++j) t[r][j] = v[r][j] * v[r][j];
            rows_head_sums(c, t, vv, 0);
#pragma unroll
            for (int r = 0; r < RB; ++r)
#pragma unroll
                for (int j = 0; j < CPL; ++j) t[r][j] = y[r][j] * v[r][j];
            rows_head_sums(c, t, yv, 1);
#pragma unroll
            for (int r = 0; r < RB; ++r)
#pragma unroll
                for (int j = 0; j < CPL; ++j) {
                    const float iv = rsqrtf(fmaxf(vv[r][j], kXsaFloor));
                    y[r][j] = (y[r][j] - (yv[r][j] * iv) * (v[r][j] * iv)) * kLog2e;
                }
        }
        rows_mesh_fixed<NW, CPL, D, RB>(y, wp, c.lane, c.wave, c.xch, c.parity);
        float inv[RB];
#pragma unroll
        for (int r = 0; r < RB; ++r)
#pragma unroll
            for (int j = 0; j < CPL; ++j) x[r][j] = fmaf(y[r][j], kLn2, x[r][j]);
        rows_inv_rms(c, x, 2, inv);
#pragma unroll
        for (int r = 0; r < RB; ++r)
#pragma unroll
            for (int j = 0; j < CPL; ++j) y[r][j] = x[r][j] * (inv[r] * kLog2e);
        rows_mesh_fixed<NW, CPL, D, RB>(y, wf, c.lane, c.wave, c.xch, c.parity);
#pragma unroll
        for (int r = 0; r < RB; ++r)
#pragma unroll
            for (int j = 0; j < CPL; ++j) x[r][j] = fmaf(y[r][j], kLn2, x[r][j]);
    }
    if (team == 0 && (post || a.embed)) {
        // Into x_out, never x: the rows' other workgroups may not have read x yet.
#pragma unroll
        for (int r = 0; r < RB; ++r)
            if (valid[r])
#pragma unroll
                for (int j = 0; j < CPL; ++j) a.x_out[size_t(row[r]) * W + c.ridx(j)] = x[r][j];
    }
    if (!a.xn && !pre) return;

    // The next RMSNorm: the final one for the head, or the block's pre-norm.
    {
        float inv[RB];
        rows_inv_rms(c, x, 3, inv);
#pragma unroll
        for (int r = 0; r < RB; ++r)
#pragma unroll
            for (int j = 0; j < CPL; ++j) x[r][j] *= inv[r];
    }
    if (a.xn) {
#pragma unroll
        for (int r = 0; r < RB; ++r)
            if (valid[r])
#pragma unroll
                for (int j = 0; j < CPL; ++j) a.xn[size_t(row[r]) * W + c.chan(j)] = x[r][j];
    }
    if (!pre) return;

#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int j = 0; j < CPL; ++j) x[r][j] *= kLog2e;
    rows_mesh_fixed<NW, CPL, D, RB>(x, wm, c.lane, c.wave, c.xch, c.parity);
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int j = 0; j < CPL; ++j) x[r][j] *= kLn2;
    if (team == 2) {
#pragma unroll
        for (int r = 0; r < RB; ++r)
            if (valid[r]) {
                const size_t cache_row = size_t(seq[r] * s.H) * a.kv_pre.cap + pos[r];
#pragma unroll
                for (int j = 0; j < CPL; ++j)
                    a.kv_pre.v[(cache_row + size_t(c.head_of(j)) * a.kv_pre.cap) * s.hdp + dim] = x[r][j];
            }
        return;
    }
    // QK-Norm per head, then RoPE at each row's position (row_qk_rope).
    {
        float sq[RB][CPL], ss[RB][CPL];
#pragma unroll
        for (int r = 0; r < RB; ++r)
#pragma unroll
            for (int j = 0; j < CPL; ++j) sq[r][j] = x[r][j] * x[r][j];
        rows_head_sums(c, sq, ss, 4);
        const float scale = 1.0f / float(s.hd);
        const bool low = dim < s.half;
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const float2 cs = rope_pair(a.rope, pos[r], dim, s.half);
            float other[CPL];
#pragma unroll
            for (int j = 0; j < CPL; ++j) other[j] = __shfl_xor(x[r][j], GL / 2, 64);
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const float sc = rsqrtf(ss[r][j] * scale + kRmsEps);
                const float self = x[r][j] * sc, oth = other[j] * sc;
                x[r][j] = low ? self * cs.x - oth * cs.y : self * cs.x + oth * cs.y;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        if (!valid[r]) continue;
        const size_t cache_row = size_t(seq[r] * s.H) * a.kv_pre.cap + pos[r];
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            if (team == 0)
                a.q[size_t(row[r]) * W + c.chan(j)] = x[r][j];
            else
                a.kv_pre.k[(cache_row + size_t(c.head_of(j)) * a.kv_pre.cap) * s.hdp + dim] = x[r][j];
        }
    }
}

// dst[r][(j*NW + wave)*64 + lane] = src[r][wave + NW*(lane + 64*j)] for rows of W
// elements of T (float: token vectors; float2: mesh weight pairs).
template <class T>
__global__ void __launch_bounds__(kThreads)
row_order_kernel(const T *__restrict__ src, T *__restrict__ dst, int rows, int W, int NW) {
    const size_t n = size_t(rows) * W;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += size_t(gridDim.x) * blockDim.x) {
        const int r = int(i / W), k = int(i - size_t(r) * W);
        const int lane = k & 63, jw = k >> 6, wave = jw % NW, j = jw / NW;
        dst[i] = src[size_t(r) * W + wave + NW * (lane + 64 * j)];
    }
}

template <int N>
__device__ __forceinline__ void load_vec(const float *__restrict__ p, float (&o)[N]) {
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int i = 0; i < N / 4; ++i) {
            const float4 t = reinterpret_cast<const float4 *>(p)[i];
            o[4 * i] = t.x;
            o[4 * i + 1] = t.y;
            o[4 * i + 2] = t.z;
            o[4 * i + 3] = t.w;
        }
    } else {
        static_assert(N == 2, "vector width");
        const float2 t = *reinterpret_cast<const float2 *>(p);
        o[0] = t.x;
        o[1] = t.y;
    }
}

// load_vec with the non-temporal cache policy.
template <int N>
__device__ __forceinline__ void load_vec_nt(const float *__restrict__ p, float (&o)[N]) {
    if constexpr (N % 4 == 0) {
        typedef float f4 __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int i = 0; i < N / 4; ++i) {
            const f4 t = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(p) + i);
            o[4 * i] = t.x;
            o[4 * i + 1] = t.y;
            o[4 * i + 2] = t.z;
            o[4 * i + 3] = t.w;
        }
    } else {
        static_assert(N == 2, "vector width");
        typedef float f2 __attribute__((ext_vector_type(2)));
        const f2 t = __builtin_nontemporal_load(reinterpret_cast<const f2 *>(p));
        o[0] = t.x;
        o[1] = t.y;
    }
}

template <int HDP, int TH = 0>
struct DecodeCfg {
    static constexpr int VEC = HDP <= 4 ? HDP : (HDP / 64 > 4 ? HDP / 64 : 4);  // dims per lane
    static constexpr int LPK = HDP / VEC;                                      // lanes per key (<= 64)
    static constexpr int THREADS = TH > 0 ? TH : (HDP >= 4096 ? 128 : 256);
    static constexpr int G = THREADS / LPK;                                    // key groups
    static constexpr int U = VEC >= 32 ? 1 : (VEC >= 16 ? 2 : (VEC >= 8 ? 4 : 8));  // keys per group per step
};

// One round of K/V rows of an attention share: each group of LPK lanes owns
// one key at a time, so every K/V row is one coalesced VEC-wide load per lane,
// and U keys per group load at once.  Rows past `end` are clamped to end - 1
// (in bounds and branch-free) and masked out of the softmax.  UK > 0
// overrides the keys per group.
template <int HDP, int TH, int UK = 0>
struct AttnRound {
    using C = DecodeCfg<HDP, TH>;
    static constexpr int VEC = C::VEC, LPK = C::LPK, G = C::G, U = UK > 0 ? UK : C::U;
    float k[U][VEC], v[U][VEC];
    __device__ __forceinline__ void load(const float *__restrict__ kslab, const float *__restrict__ vslab, int j0,
                                         int end) {
        // 32-bit element offsets from the uniform slab bases (a slab is far
        // below 2^32 elements), so each load needs one address register.
        const uint32_t g = threadIdx.x / LPK, d0 = (threadIdx.x % LPK) * VEC;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t at = uint32_t(min(j0 + u * G + int(g), end - 1)) * HDP + d0;
            load_vec<VEC>(kslab + at, k[u]);
            load_vec<VEC>(vslab + at, v[u]);
        }
    }
    // The same with the non-temporal cache policy.
    __device__ __forceinline__ void load_nt(const float *__restrict__ kslab, const float *__restrict__ vslab, int j0,
                                            int end) {
        const uint32_t g = threadIdx.x / LPK, d0 = (threadIdx.x % LPK) * VEC;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t at = uint32_t(min(j0 + u * G + int(g), end - 1)) * HDP + d0;
            load_vec_nt<VEC>(kslab + at, k[u]);
            load_vec_nt<VEC>(vslab + at, v[u]);
        }
    }
};

// 2^x by the hardware instruction (about 1 ulp).  Results below the normal
// range flush to zero, which the softmax sums absorb: their largest term is 1.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Online-softmax state (reference.rs:510-554) of one key group: scores live in
// the log2 domain, and q stays unscaled (each score is scaled instead) so its
// load does not hold back the first K/V loads.
template <int HDP, int TH, int UK = 0>
struct AttnState {
    using R = AttnRound<HDP, TH, UK>;
    static constexpr int VEC = R::VEC, LPK = R::LPK, G = R::G, U = R::U;
    float m = -INFINITY, l = 0.0f, acc[VEC] = {};
    // Folds in the round loaded at j0 (keys at or past `end` are masked).
    __device__ __forceinline__ void add(const float (&qr)[VEC], const R &cur, int j0, int end, float scale_log2) {
        const int g = threadIdx.x / LPK;
        float sc[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float p = 0.0f;
#pragma unroll
            for (int e = 0; e < VEC; ++e) p = fmaf(qr[e], cur.k[u][e], p);
            p = group_sum<LPK>(p);
            sc[u] = (j0 + u * G + g < end) ? p * scale_log2 : -INFINITY;
        }
        float cm = sc[0];
#pragma unroll
        for (int u = 1; u < U; ++u) cm = fmaxf(cm, sc[u]);
        const float mn = fmaxf(m, cm);
        if (mn != -INFINITY) {
            const float alpha = exp2_fast(m - mn);
            float pu[U], ps = 0.0f;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                pu[u] = exp2_fast(sc[u] - mn);
                ps += pu[u];
            }
            l = l * alpha + ps;
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                float a = acc[e] * alpha;
#pragma unroll
                for (int u = 0; u < U; ++u) a = fmaf(pu[u], cur.v[u][e], a);
                acc[e] = a;
            }
            m = mn;
        }
    }
    // Folds in the rounds loaded at j0 and j1 together: their scores and
    // exponentials are independent, so the two chains overlap.
    __device__ __forceinline__ void add2(const float (&qr)[VEC], const R &c0, int j0, const R &c1, int j1, int end,
                                         float scale_log2) {
        const int g = threadIdx.x / LPK;
        float sc[2 * U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float p0 = 0.0f, p1 = 0.0f;
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                p0 = fmaf(qr[e], c0.k[u][e], p0);
                p1 = fmaf(qr[e], c1.k[u][e], p1);
            }
            p0 = group_sum<LPK>(p0);
            p1 = group_sum<LPK>(p1);
            sc[u] = (j0 + u * G + g < end) ? p0 * scale_log2 : -INFINITY;
            sc[U + u] = (j1 + u * G + g < end) ? p1 * scale_log2 : -INFINITY;
        }
        float cm = sc[0];
#pragma unroll
        for (int u = 1; u < 2 * U; ++u) cm = fmaxf(cm, sc[u]);
        const float mn = fmaxf(m, cm);
        if (mn != -INFINITY) {
            const float alpha = exp2_fast(m - mn);
            float pu[2 * U], ps = 0.0f;
#pragma unroll
            for (int u = 0; u < 2 * U; ++u) {
                pu[u] = exp2_fast(sc[u] - mn);
                ps += pu[u];
            }
            l = l * alpha + ps;
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                float a = acc[e] * alpha, b = 0.0f;
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    a = fmaf(pu[u], c0.v[u][e], a);
                    b = fmaf(pu[U + u], c1.v[u][e], b);
                }
                acc[e] = a + b;
            }
            m = mn;
        }
    }
    // Merges the G groups' states of the block into wave 0: thread d < 64
    // returns the normalised output of dim d (0 for d >= HDP; other waves
    // get 0), with the arithmetic of combine.  sm and sl hold G floats, sacc
    // G * HDP (16-byte aligned), all LDS; the caller's LDS writes before the
    // call are visible to wave 0 after it.
    __device__ __forceinline__ float merge_wave0(float *sm, float *sl, float *sacc) const {
        static_assert(TH >= HDP && HDP <= 64, "one dim per lane of wave 0");
        const int g = threadIdx.x / LPK, li = threadIdx.x % LPK;
#pragma unroll
        for (int e = 0; e < VEC; ++e) sacc[g * HDP + li * VEC + e] = acc[e];
        if (li == 0) {
            sm[g] = m;
            sl[g] = l;
        }
        __syncthreads();
        static_assert(G <= 64, "one lane per group state");
        float y = 0.0f;
        if (threadIdx.x < 64) {
            // Lane k of each G-lane group holds group k's (m, l); the scale
            // factors are computed once there and read from lane k by all.
            const int lane = threadIdx.x, d = min(lane, HDP - 1), k = lane % G;
            const float mk = sm[k], lk = sl[k];
            float ak[G];
#pragma unroll
            for (int kk = 0; kk < G; ++kk) ak[kk] = sacc[kk * HDP + d];
            asm volatile("" ::: "memory");  // every read issued before the first use
            const float M = group_max<G>(mk);
            const float f = exp2_fast(mk - M);
            const float L = group_sum<G>(f * lk);
            // Four partial sums over the groups k = i (mod 4), added
            // pairwise: a chain of G/4 + 2 dependent adds instead of G.
            constexpr int P = G >= 4 ? 4 : G;
            float part[P];
#pragma unroll
            for (int i = 0; i < P; ++i) part[i] = 0.0f;
#pragma unroll
            for (int kk = 0; kk < G; ++kk)
                part[kk % P] = fmaf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, f), kk)),
                                    ak[kk], part[kk % P]);
            float a = part[0];
            if constexpr (P == 4) a = (part[0] + part[1]) + (part[2] + part[3]);
            else if constexpr (P == 2) a = part[0] + part[1];
            y = lane < HDP ? a * __builtin_amdgcn_rcpf(L) : 0.0f;
        }
        return y;
    }
    // Merges the G groups' states of the block: emit(d, a, M, L) for each
    // d < HDP with a = sum of the rescaled accumulators, M the block maximum
    // and L the rescaled denominator.  sm and sl hold G floats, sacc G * HDP
    // (16-byte aligned), all LDS.
    template <class Emit>
    __device__ __forceinline__ void combine(Emit emit, float *sm, float *sl, float *sacc) const {
        const int g = threadIdx.x / LPK, li = threadIdx.x % LPK;
#pragma unroll
        for (int e = 0; e < VEC; ++e) sacc[g * HDP + li * VEC + e] = acc[e];
        if (li == 0) {
            sm[g] = m;
            sl[g] = l;
        }
        __syncthreads();
        if constexpr (TH >= HDP) {
            // One dim per thread, with every LDS read issued before the first
            // is used (the empty asm keeps the scheduler from interleaving
            // each read with its use and waiting out each latency in turn).
            if (int(threadIdx.x) < HDP) {
                const int d = threadIdx.x;
                float mk[G], lk[G], ak[G];
#pragma unroll
                for (int k = 0; k < G; ++k) {
                    mk[k] = sm[k];
                    lk[k] = sl[k];
                    ak[k] = sacc[k * HDP + d];
                }
                asm volatile("" ::: "memory");
                float M = -INFINITY;
#pragma unroll
                for (int k = 0; k < G; ++k) M = fmaxf(M, mk[k]);
                float L = 0.0f, a = 0.0f;
#pragma unroll
                for (int k = 0; k < G; ++k) {
                    const float f = exp2_fast(mk[k] - M);
                    L += f * lk[k];
                    a += f * ak[k];
                }
                emit(d, a, M, L);
            }
        } else {
            float M = -INFINITY;
            for (int k = 0; k < G; ++k) M = fmaxf(M, sm[k]);
            float L = 0.0f;
            for (int k = 0; k < G; ++k) L += exp2_fast(sm[k] - M) * sl[k];
            for (int d = threadIdx.x; d < HDP; d += blockDim.x) {
                float a = 0.0f;
                for (int k = 0; k < G; ++k) a += exp2_fast(sm[k] - M) * sacc[k * HDP + d];
                emit(d, a, M, L);
            }
        }
        __syncthreads();
    }
};

// Online-softmax attention of one query head over keys [start, end) of one
// (sequence, head) cache slab kslab/vslab (position-major rows of HDP floats);
// the block's partial state (acc[HDP], m, l) goes to out[0..HDP+1].  An empty
// share writes the neutral partial (m = -inf, l = 0).
template <int HDP>
__device__ __forceinline__ void attn_share(const float *__restrict__ qh, int hd, const float *__restrict__ kslab,
                                           const float *__restrict__ vslab, int start, int end, float scale_log2,
                                           float *__restrict__ out, int keep = 1 << 30) {
    using S = AttnState<HDP, 0>;
    using R = typename S::R;
    constexpr int VEC = S::VEC, LPK = S::LPK, G = S::G, U = S::U;
    if (start >= end) {
        for (int d = threadIdx.x; d < HDP; d += blockDim.x) out[d] = 0.0f;
        if (threadIdx.x == 0) {
            out[HDP] = -INFINITY;
            out[HDP + 1] = 0.0f;
        }
        return;
    }
    const int d0 = (threadIdx.x % LPK) * VEC;
    float qr[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) qr[e] = d0 + e < hd ? qh[d0 + e] : 0.0f;
    S st;
    for (int j0 = start; j0 < end; j0 += G * U) {
        // Rows past the first `keep` load with the non-temporal policy
        // (kv_keep_rows).
        R cur;
        if (j0 + G * U > keep)
            cur.load_nt(kslab, vslab, j0, end);
        else
            cur.load(kslab, vslab, j0, end);
        st.add(qr, cur, j0, end, scale_log2);
    }
    __shared__ float sm[G], sl[G];
    __shared__ __align__(16) float sacc[G * HDP];
    st.combine(
        [&](int d, float a, float M, float L) {
            out[d] = a;
            if (d == 0) {
                out[HDP] = M;
                out[HDP + 1] = L;
            }
        },
        sm, sl, sacc);
}

// Split-KV decode attention for one query row per sequence.  Block
// (seq * nsplit + split, head) runs attn_share over an equal share of the
// len[seq] keys of the cache.
template <int HDP>
__global__ void __launch_bounds__(DecodeCfg<HDP>::THREADS)
attn_decode_kernel(Shape s, const float *__restrict__ q, KvView kv, const int *__restrict__ len, int nsplit,
                   float *__restrict__ part, float scale_log2) {
    const int b = int(blockIdx.x) / nsplit, split = int(blockIdx.x) - b * nsplit, h = blockIdx.y;
    const int keys = len[b];
    const int chunk = (keys + nsplit - 1) / nsplit;
    const int start = split * chunk;
    const int end = min(start + chunk, keys);
    const size_t slab = size_t(b * s.H + h) * kv.cap * HDP;
    attn_share<HDP>(q + size_t(b) * s.W + h * s.hd, s.hd, kv.k + slab, kv.v + slab, start, end, scale_log2,
                    part + (size_t(b * s.H + h) * nsplit + split) * (HDP + 2), kv.keep);
}

template <int HDP>
struct PrefillCfg {
    static constexpr int DPT = HDP <= 16 ? HDP : (HDP / 64 > 16 ? HDP / 64 : 16);  // dims per thread
    static constexpr int TPQ = HDP / DPT;                                           // threads per query
    static constexpr int QT = kThreads / TPQ;                                       // queries per block
    static constexpr int KT = HDP >= 4096 ? 1 : (4096 / HDP > 64 ? 64 : 4096 / HDP);  // keys per tile
};

// Causal flash attention for whole sequences (reference.rs:510-554).  Block
// (query tile, head, seq); K/V tiles of KT keys are staged in LDS and shared by
// the QT queries of the tile; TPQ threads split each query's head dims.
template <int HDP>
__global__ void __launch_bounds__(kThreads)
attn_prefill_kernel(Shape s, const float *__restrict__ q, KvView kv, int rows_per_seq,
                    float *__restrict__ y, float scale_log2) {
    using C = PrefillCfg<HDP>;
    constexpr int DPT = C::DPT, TPQ = C::TPQ, QT = C::QT, KT = C::KT;
    __shared__ __align__(16) float Ks[KT * HDP];
    __shared__ __align__(16) float Vs[KT * HDP];
    const int ntiles = (rows_per_seq + QT - 1) / QT;
    const int seq = int(blockIdx.x) / ntiles;
    const int qt = ntiles - 1 - (int(blockIdx.x) - seq * ntiles);  // longest rows first
    const int h = blockIdx.y;
    const int qi = threadIdx.x / TPQ, li = threadIdx.x % TPQ, d0 = li * DPT;
    const int qpos = qt * QT + qi;
    const bool qvalid = qpos < rows_per_seq;
    const size_t row = size_t(seq) * rows_per_seq + qpos;
    float qr[DPT], acc[DPT];
#pragma unroll
    for (int e = 0; e < DPT; ++e) {
        const int d = d0 + e;
        qr[e] = (qvalid && d < s.hd) ? q[row * s.W + h * s.hd + d] * scale_log2 : 0.0f;
        acc[e] = 0.0f;
    }
    float m = -INFINITY, l = 0.0f;
    const int last = min((qt + 1) * QT, rows_per_seq) - 1;
    const size_t base = size_t(seq * s.H + h) * kv.cap * HDP;
    for (int k0 = 0; k0 <= last; k0 += KT) {
        const int nk = min(KT, last + 1 - k0);
        __syncthreads();
        const float *ks = kv.k + base + size_t(k0) * HDP;
        const float *vs = kv.v + base + size_t(k0) * HDP;
        if constexpr (HDP % 4 == 0) {
            for (int i = threadIdx.x; i < nk * HDP / 4; i += blockDim.x) {
                reinterpret_cast<float4 *>(Ks)[i] = reinterpret_cast<const float4 *>(ks)[i];
                reinterpret_cast<float4 *>(Vs)[i] = reinterpret_cast<const float4 *>(vs)[i];
            }
        } else {
            for (int i = threadIdx.x; i < nk * HDP; i += blockDim.x) {
                Ks[i] = ks[i];
                Vs[i] = vs[i];
            }
        }
        __syncthreads();
        for (int j0 = 0; j0 < nk; j0 += 8) {
            float sc[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int j = j0 + u;
                float p = 0.0f;
                if (j < nk) {
                    const float *kr = Ks + j * HDP + d0;
#pragma unroll
                    for (int e = 0; e < DPT; ++e) p = fmaf(qr[e], kr[e], p);
                }
                p = group_sum<TPQ>(p);
                sc[u] = (j < nk && k0 + j <= qpos) ? p : -INFINITY;
            }
            float cm = sc[0];
#pragma unroll
            for (int u = 1; u < 8; ++u) cm = fmaxf(cm, sc[u]);
            const float mn = fmaxf(m, cm);
            if (mn != -INFINITY) {
                const float alpha = exp2f(m - mn);
                float pu[8], ps = 0.0f;
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    pu[u] = exp2f(sc[u] - mn);
                    ps += pu[u];
                }
                l = l * alpha + ps;
#pragma unroll
                for (int e = 0; e < DPT; ++e) acc[e] *= alpha;
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    if (j0 + u < nk) {
                        const float *vr = Vs + (j0 + u) * HDP + d0;
#pragma unroll
                        for (int e = 0; e < DPT; ++e) acc[e] = fmaf(pu[u], vr[e], acc[e]);
                    }
                }
                m = mn;
            }
        }
    }
    if (qvalid) {
        const float rl = 1.0f / l;
#pragma unroll
        for (int e = 0; e < DPT; ++e) {
            const int d = d0 + e;
            if (d < s.hd) y[row * s.W + h * s.hd + d] = acc[e] * rl;
        }
    }
}

// ------------------------------------------------------------ head, sampling

// Final RMSNorm rows are produced by block_kernel (xn); the head takes their
// dot products with every token vector (reference.rs:218-226).  Et is [W][Vp]
// with Vp = V rounded up to a multiple of 4 (zero padding).

// Tiled head for many rows (prefill, logits): block = 32 tokens x 8 c-groups,
// rt <= 8 rows; the c-group partials are summed through LDS.
constexpr int kHeadTokens = 32, kHeadGroups = kThreads / kHeadTokens, kHeadMaxRows = 8;

__global__ void __launch_bounds__(kThreads)
head_kernel(Shape s, const float *__restrict__ xn, int nrows, int row_mul, int row_add,
            const float *__restrict__ Et, int Vp, float *__restrict__ logits, int rt) {
    extern __shared__ __align__(16) char smem[];
    LdsCarve lds{smem};
    const int W = s.W, V = s.V;
    float *N = lds.take<float>(size_t(rt) * W);
    float *red = lds.take<float>(size_t(kHeadGroups) * kHeadMaxRows * kHeadTokens);
    const int i0 = blockIdx.y * rt, nr = min(rt, nrows - i0);
    for (int idx = threadIdx.x; idx < rt * W; idx += blockDim.x) {
        int r, c;
        split_row(idx, s, r, c);
        N[idx] = r < nr ? xn[(size_t(i0 + r) * row_mul + row_add) * W + c] : 0.0f;
    }
    __syncthreads();
    const int j = threadIdx.x % kHeadTokens, g = threadIdx.x / kHeadTokens;
    const int t = min(int(blockIdx.x) * kHeadTokens + j, V - 1);
    float acc[kHeadMaxRows];
#pragma unroll
    for (int r = 0; r < kHeadMaxRows; ++r) acc[r] = 0.0f;
    constexpr int kUnroll = 16;
    for (int c0 = g; c0 < W; c0 += kHeadGroups * kUnroll) {
        float e[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) e[u] = Et[size_t(min(c0 + u * kHeadGroups, W - 1)) * Vp + t];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int c = c0 + u * kHeadGroups;
            if (c < W) {
#pragma unroll
                for (int r = 0; r < kHeadMaxRows; ++r)
                    if (r < rt) acc[r] = fmaf(N[r * W + c], e[u], acc[r]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < kHeadMaxRows; ++r) red[(g * kHeadMaxRows + r) * kHeadTokens + j] = acc[r];
    __syncthreads();
    for (int i = threadIdx.x; i < kHeadMaxRows * kHeadTokens; i += blockDim.x) {
        const int r = i / kHeadTokens, jj = i - r * kHeadTokens;
        const int tok = int(blockIdx.x) * kHeadTokens + jj;
        if (r < nr && tok < V) {
            float sum = 0.0f;
            for (int k = 0; k < kHeadGroups; ++k) sum += red[(k * kHeadMaxRows + r) * kHeadTokens + jj];
            logits[size_t(i0 + r) * V + tok] = sum;
        }
    }
}

__device__ __forceinline__ uint64_t splitmix_next(uint64_t &state) {
    state += 0x9e3779b97f4a7c15ULL;
    uint64_t bits = state;
    bits = (bits ^ (bits >> 30)) * 0xbf58476d1ce4e5b9ULL;
    bits = (bits ^ (bits >> 27)) * 0x94d049bb133111ebULL;
    return bits ^ (bits >> 31);
}

// exp(x) rounded once to f32 from an f64 evaluation: the correctly rounded
// value except within about 2^-29 ulp of a rounding midpoint, which is what
// host libm expf returns (the reference's f32::exp).  The device's f32 expf
// can differ by an ulp, and a near-tie draw then picks another token.
// Table of 2^(i/32) in the form the method below uses: the bits of the
// correctly rounded double 2^(i/32) minus i << 47.
__constant__ uint64_t kExp2Tab[32] = {
    0x3ff0000000000000, 0x3fefd9b0d3158574, 0x3fefb5586cf9890f, 0x3fef9301d0125b51, 0x3fef72b83c7d517b,
    0x3fef54873168b9aa, 0x3fef387a6e756238, 0x3fef1e9df51fdee1, 0x3fef06fe0a31b715, 0x3feef1a7373aa9cb,
    0x3feedea64c123422, 0x3feece086061892d, 0x3feebfdad5362a27, 0x3feeb42b569d4f82, 0x3feeab07dd485429,
    0x3feea47eb03a5585, 0x3feea09e667f3bcd, 0x3fee9f75e8ec5f74, 0x3feea11473eb0187, 0x3feea589994cce13,
    0x3feeace5422aa0db, 0x3feeb737b0cdc5e5, 0x3feec49182a3f090, 0x3feed503b23e255d, 0x3feee89f995ad3ad,
    0x3feeff76f2fb5e47, 0x3fef199bdd85529c, 0x3fef3720dcef9069, 0x3fef5818dcfba487, 0x3fef7c97337b9b5f,
    0x3fefa4afa2a490da, 0x3fefd0765b6e4540};

// The reference's f32 exp: Rust's f32::exp is the C library's expf, which in
// glibc >= 2.28 is the exp2f-table method of ARM's optimized-routines
// (published; e_expf.c): x * 32/ln2 = k + r with |r| <= 1/2, exp(x) =
// 2^(k/32) * p(r) with a cubic p, all in double, then one rounding to float.
// This is that method in the operation order of glibc's FMA build (the one
// x86-64 hosts with FMA run): it equals that expf on every one of the 2^32
// float inputs (checked on the host against glibc 2.35); glibc's build for
// hosts without FMA rounds 2 of them differently.
// `tab` is kExp2Tab staged in LDS (a per-lane lookup in constant memory costs
// a memory round trip per call).  Branch-free, so that several calls
// interleave: the cases outside the method's range (x > 0x1.62e42ep6 gives
// +inf, x < -0x1.9fe368p6 and -inf give 0, NaN gives NaN) are selected after
// it runs on x clamped to [-104, 89].
__device__ __forceinline__ float expf_rounded(float x, const uint64_t *tab) {
    constexpr double N = 32.0, InvLn2N = 0x1.71547652b82fep+0 * N, Shift = 0x1.8p+52;
    constexpr double C0 = 0x1.c6af84b912394p-5 / (N * N * N), C1 = 0x1.ebfce50fac4f3p-3 / (N * N),
                     C2 = 0x1.62e42ff0c52d6p-1 / N;
    const double xd = double(fminf(fmaxf(x, -104.0f), 89.0f));
    double kd = InvLn2N * xd + Shift;  // rounds k to the nearest integer
    const uint64_t ki = uint64_t(__double_as_longlong(kd));
    kd -= Shift;
    const double r = fma(InvLn2N, xd, -kd);
    const double sc = __longlong_as_double(int64_t(tab[ki & 31] + (ki << 47)));
    const double z = fma(C0, r, C1), r2 = r * r;
    double y = fma(C2, r, 1.0);
    y = fma(z, r2, y);
    float e = float(y * sc);
    e = x > 0x1.62e42ep6f ? INFINITY : e;
    e = x < -0x1.9fe368p6f ? 0.0f : e;
    return x != x ? x + x : e;
}

// Copies kExp2Tab to `tab` (32 words of LDS); a barrier must follow before use.
__device__ __forceinline__ void stage_exp_table(uint64_t *tab) {
    for (int i = threadIdx.x; i < 32; i += blockDim.x) tab[i] = kExp2Tab[i];
}

// (l - max) / T in f32 (gpu.rs:2037); division by 1 is exact, so T = 1 skips it.
__device__ __forceinline__ float scaled_logit(float l, float mx, float temperature) {
    return temperature == 1.0f ? l - mx : (l - mx) / temperature;
}

// The reference's sequential f32 sampler (gpu.rs:2034-2048) in one lane, for
// a given draw u and p(i) = p_i = exp((l_i - max)/T): a token-order f32 sum of
// the p_i, then a token-order scan of u*sum - p_0 - p_1 - ... that stops at
// the first negative remainder (default: the last token); no multiply-add
// fusion.  The next sixteen values load while the current sixteen are added.
template <class P>
__device__ __forceinline__ int sequential_pick(P p, int V, float u) {
#pragma clang fp contract(off)
    constexpr int kBatch = 16;
    auto fetch = [&](float (&v)[kBatch], int t) {
#pragma unroll
        for (int k = 0; k < kBatch; ++k) v[k] = p(min(t + k, V - 1));
    };
    const int full = V / kBatch * kBatch;
    float sum = 0.0f;
    float cur[kBatch], nxt[kBatch];
    if (full) fetch(nxt, 0);
    for (int t = 0; t < full; t += kBatch) {
#pragma unroll
        for (int k = 0; k < kBatch; ++k) cur[k] = nxt[k];
        if (t + kBatch < full) fetch(nxt, t + kBatch);
#pragma unroll
        for (int k = 0; k < kBatch; ++k) sum = sum + cur[k];
    }
    for (int t = full; t < V; ++t) sum = sum + p(t);
    float sample = u * sum;
    if (full) fetch(nxt, 0);
    for (int t = 0; t < full; t += kBatch) {
#pragma unroll
        for (int k = 0; k < kBatch; ++k) cur[k] = nxt[k];
        if (t + kBatch < full) fetch(nxt, t + kBatch);
        float left[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            sample = sample - cur[k];
            left[k] = sample;
        }
#pragma unroll
        for (int k = 0; k < kBatch; ++k)
            if (left[k] < 0.0f) return t + k;
    }
    for (int t = full; t < V; ++t) {
        sample = sample - p(t);
        if (sample < 0.0f) return t;
    }
    return V - 1;
}

// LDS scratch of choose_token: a float, an int and a double per wave, one
// more double, and the exp table (stage_exp_table, before a barrier).
struct SampleLds {
    float *redf;
    int *redi;
    double *redd;
    const uint64_t *exp_tab;
};

// Block minimum.  The slots it writes are free again only after the caller's
// next barrier.
__device__ __forceinline__ int block_min_int(int v, const SampleLds &m) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    v = wave_min_int(v);
    if (lane == 0) m.redi[wave] = v;
    __syncthreads();
    v = INT_MAX;
    for (int w = 0; w < nw; ++w) v = min(v, m.redi[w]);
    return v;
}

// Block-wide choice of the next token from a logits row (gpu.rs:2028-2049):
// greedy = the first maximal logit; T > 0 = the reference's sampler.  Sets
// bit 0 of *flags when the row holds a non-finite value.
//
// Temperature sampling is decided in parallel with the same result as the
// sequential f32 process: with p_i = exp((l_i - max)/T) in f32, the reference
// sums them in token order in f32 (S32), draws u, and returns the first i
// whose sequential f32 remainder u*S32 - p_0 - ... - p_i is negative.  With
// unit roundoff e = 2^-24 and all p_i >= 0, |S32 - S| <= (V+2) e S for the
// exact sum S, and every remainder is within beta = (V+2) e S32 of the exact
// u*S32 - P_i (P_i the exact prefix sums, here in f64).  So an index is
// surely non-negative when P_i < u*S_lo - beta and surely negative when
// P_i > u*S_hi + beta; the first index that is not surely non-negative is the
// answer when it is surely negative.  Otherwise (a near-tie, or a non-finite
// row) thread 0 runs the sequential f32 process itself with the same u.  The
// SampleLds slots are free again only after the caller's next barrier.
__device__ __forceinline__ int choose_token(const float *row, int V, float temperature, uint64_t *rng, int *flags,
                                            const SampleLds &m, float *pscratch = nullptr) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    // Every wave scans the whole row for the maximum (and for non-finite
    // values) itself: no exchange between waves, so no barrier.
    float mx = -INFINITY;
    int bad = 0;
    for (int t = lane; t < V; t += 64) {
        const float v = row[t];
        bad |= !isfinite(v);
        mx = fmaxf(mx, v);
    }
    mx = wave_max(mx);
    bad = wave_or_int(bad);
    if (bad && threadIdx.x == 0) atomicOr(flags, 1);
    if (temperature == 0.0f) {
        int best = INT_MAX;
        for (int t = lane; t < V; t += 64)
            if (row[t] == mx) best = min(best, t);
        best = wave_min_int(best);
        return best == INT_MAX ? 0 : best;
    }
    // Each thread takes a contiguous run [i0, i1) of the tokens; runs of up to
    // kRunCache tokens keep their p_i in registers between the two passes.
    const int run = (V + int(blockDim.x) - 1) / int(blockDim.x);
    const int i0 = min(int(threadIdx.x) * run, V), i1 = min(i0 + run, V);
    auto pexp = [&](int i) { return expf_rounded(scaled_logit(row[i], mx, temperature), m.exp_tab); };
    constexpr int kRunCache = 4;
    const bool cached = run <= kRunCache;
    float pc[kRunCache];
    double mine = 0.0;
    if (cached) {
#pragma unroll
        for (int k = 0; k < kRunCache; ++k) {
            pc[k] = 0.0f;
            if (k >= run) break;  // uniform: no exp is evaluated past the run
            if (i0 + k < i1) pc[k] = pexp(i0 + k);
            mine += double(pc[k]);
        }
    } else {
        for (int i = i0; i < i1; ++i) mine += double(pexp(i));
    }
    const double incl = wave_inclusive_sum(mine);
    if (lane == 63) m.redd[wave] = incl;
    if (threadIdx.x == 0) {
        // One SplitMix64 draw per sampled token, as Random::unit (src/mesh.rs:263-265).
        uint64_t state = *rng;
        m.redd[nw] = double(float(uint32_t(splitmix_next(state) >> 40)) / 16777216.0f);
        *rng = state;
    }
    __syncthreads();
    // Every read of the row is done: the p_i overwrite it for the fallback.
    if (cached && pscratch) {
#pragma unroll
        for (int k = 0; k < kRunCache; ++k) {
            if (k >= run) break;
            if (i0 + k < i1) pscratch[i0 + k] = pc[k];
        }
    }
    double before = 0.0, S = 0.0;
    for (int w = 0; w < nw; ++w) {
        if (w < wave) before += m.redd[w];
        S += m.redd[w];
    }
    const float u = float(m.redd[nw]);
    const double e = 0x1p-24, slack = 1e-12 * S;
    const double g = double(V + 2) * e * 1.01;
    const double s_lo = S * (1.0 - g) - slack, s_hi = S * (1.0 + g) + slack;
    const double beta = double(V + 2) * e * s_hi * 1.01 + slack;
    const double lo = double(u) * s_lo - beta, hi = double(u) * s_hi + beta;
    double prefix = before + incl - mine;
    // key = 2 * (first index whose prefix reaches lo) + (1 if that index is not
    // decided by the bounds); the block minimum is the earliest such index.
    int key = INT_MAX;
    if (cached) {
#pragma unroll
        for (int k = 0; k < kRunCache; ++k) {
            if (k >= run) break;
            if (key == INT_MAX && i0 + k < i1) {
                prefix += double(pc[k]);
                if (!(prefix < lo)) key = 2 * (i0 + k) + (prefix > hi ? 0 : 1);
            }
        }
    } else {
        for (int i = i0; i < i1; ++i) {
            prefix += double(pexp(i));
            if (!(prefix < lo)) {
                key = 2 * i + (prefix > hi ? 0 : 1);
                break;
            }
        }
    }
    key = block_min_int(key, m);
    if (key == INT_MAX) return V - 1;
    int token = key >> 1;
    if (key & 1) {
        __syncthreads();
        if (threadIdx.x == 0) {
            if (cached && pscratch)
                m.redi[0] = sequential_pick([&](int t) { return pscratch[t]; }, V, u);
            else
                m.redi[0] = sequential_pick(
                    [&](int t) { return expf_rounded(scaled_logit(row[t], mx, temperature), m.exp_tab); }, V, u);
        }
        __syncthreads();
        token = m.redi[0];
    }
    return token;
}

// The lowest lane's value of v among the lanes where `has` holds, else `none`
// (a ballot and a lane read instead of a reduction).
__device__ __forceinline__ int first_lane_value(bool has, int v, int none) {
    const uint64_t mask = __ballot(has);
    return mask ? __builtin_amdgcn_readlane(v, int(__builtin_ctzll(mask))) : none;
}

// The reference's sequential f32 process (sequential_pick) run by a whole
// wave on p_i held in its registers: token t = j*R + k is pc[k] of lane j.
// Each p_i reaches every lane by a lane read (an exact copy), so all lanes
// compute the same sum and remainder; no memory is touched.
template <int RMAX>
__device__ __forceinline__ int wave_sequential_pick(const float (&pc)[RMAX], int R, int V, float u) {
#pragma clang fp contract(off)
    auto at = [&](int k, int j) {
        return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pc[k]), j));
    };
    float sum = 0.0f;
    for (int j = 0; j < 64; ++j) {
#pragma unroll
        for (int k = 0; k < RMAX; ++k)
            if (k < R && j * R + k < V) sum = sum + at(k, j);
    }
    float sample = u * sum;
    for (int j = 0; j < 64; ++j) {
#pragma unroll
        for (int k = 0; k < RMAX; ++k) {
            if (k < R && j * R + k < V) {
                sample = sample - at(k, j);
                if (sample < 0.0f) return j * R + k;
            }
        }
    }
    return V - 1;
}

// choose_token's decision made by one wave on its own: lane l holds the
// logits of the contiguous run [l*R, l*R + R) of tokens in lg[0..R),
// R = ceil(V / 64) <= RMAX, and u is the generator's draw (made by the
// caller, so that it is ready before the logits are).  Every lane returns the
// token.  Nothing touches memory but the non-finite flag: a near-tie runs the
// sequential f32 process on the wave's registers (wave_sequential_pick), so
// waves of one workgroup never share scratch and need no barrier.  VC > 0
// compiles the choice for the vocabulary V = VC: the run length and every
// token mask are then constants, and the uniform branches on them vanish.
template <int RMAX, int VC = 0>
__device__ __forceinline__ int wave_choose_token(const float (&lg)[RMAX], int V, float temperature, float u,
                                                 const uint64_t *exp_tab, int *flags) {
    static_assert(RMAX % 4 == 0, "runs are handled four tokens at a time");
    static_assert(VC >= 0 && (VC + 63) / 64 <= RMAX, "a fixed vocabulary fits the runs");
    if constexpr (VC > 0) {
        V = VC;
    } else {
        // V is hidden from the optimiser so that the f64 constants derived
        // from it are formed here, not hoisted out of a caller's step loop
        // and spilled.
        V = __builtin_amdgcn_readfirstlane(V);
        asm volatile("" : "+s"(V));
    }
    // Every per-token step below is straight-line code in blocks of four
    // tokens (a lane's tokens past V are masked by selects), so the f64
    // evaluations of neighbouring tokens overlap; only `k < R` branches, and
    // it is wave-uniform.  Since the runs ascend with the lane, the first
    // token with a property lies in the lowest lane that has one.
    const int R = (V + 63) / 64, i0 = int(threadIdx.x & 63) * R;
    float mx = -INFINITY;
    bool bad = false;
#pragma unroll
    for (int k = 0; k < RMAX; ++k) {
        if (k < R) {
            const bool v = i0 + k < V;
            bad = bad || (v && !isfinite(lg[k]));
            mx = v ? fmaxf(mx, lg[k]) : mx;
        }
    }
    mx = wave_max(mx);
    if (__ballot(bad) && threadIdx.x == 0) atomicOr(flags, 1);
    if (temperature == 0.0f) {
        int best = INT_MAX;
#pragma unroll
        for (int k = RMAX - 1; k >= 0; --k)
            if (k < R && i0 + k < V && lg[k] == mx) best = i0 + k;
        return first_lane_value(best != INT_MAX, best, 0);
    }
    float pc[RMAX];
    auto exps = [&](auto scaled) {
#pragma unroll
        for (int c = 0; c < RMAX / 4; ++c) {
            if (4 * c < R) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int k = 4 * c + q;
                    const float p = expf_rounded(scaled(lg[k]), exp_tab);
                    pc[k] = k < R && i0 + k < V ? p : 0.0f;
                }
            }
        }
    };
    // (l - max) / T in f32 (gpu.rs:2037); division by 1 is exact, so T = 1
    // skips it.
    if (temperature == 1.0f)
        exps([&](float l) { return l - mx; });
    else
        exps([&](float l) { return (l - mx) / temperature; });
    double mine = 0.0;  // the masked tokens add exact zeros
#pragma unroll
    for (int k = 0; k < RMAX; ++k)
        if (k < R) mine += double(pc[k]);
    const double incl = wave_inclusive_sum(mine);
    const uint64_t sb = __builtin_bit_cast(uint64_t, incl);
    const double S = __builtin_bit_cast(
        double, (uint64_t(uint32_t(__builtin_amdgcn_readlane(int(uint32_t(sb >> 32)), 63))) << 32) |
                    uint32_t(__builtin_amdgcn_readlane(int(uint32_t(sb)), 63)));
    const double e = 0x1p-24, slack = 1e-12 * S;
    const double g = double(V + 2) * e * 1.01;
    const double s_lo = S * (1.0 - g) - slack, s_hi = S * (1.0 + g) + slack;
    const double beta = double(V + 2) * e * s_hi * 1.01 + slack;
    const double lo = double(u) * s_lo - beta, hi = double(u) * s_hi + beta;
    double prefix = incl - mine;
    int key = INT_MAX;
#pragma unroll
    for (int k = 0; k < RMAX; ++k) {
        if (k < R) {
            prefix += double(pc[k]);
            const bool first = key == INT_MAX && i0 + k < V && !(prefix < lo);
            key = first ? 2 * (i0 + k) + (prefix > hi ? 0 : 1) : key;
        }
    }
    key = first_lane_value(key != INT_MAX, key, INT_MAX);
    if (key == INT_MAX) return V - 1;
    if (!(key & 1)) return key >> 1;
    return wave_sequential_pick(pc, R, V, u);
}

// Random::unit (src/mesh.rs:263-265): one SplitMix64 draw per sampled token.
__device__ __forceinline__ float rng_unit(uint64_t &state) {
    return float(uint32_t(splitmix_next(state) >> 40)) / 16777216.0f;
}

__device__ __forceinline__ void append_token(uint32_t *tokens, int tok_stride, int *len, int b, int token) {
    if (threadIdx.x == 0) {
        const int L = len[b];
        tokens[size_t(b) * tok_stride + L] = uint32_t(token);
        len[b] = L + 1;
    }
}

// Sampling from logits already in memory (after a prefill): one block per
// sequence; the row is staged in LDS when it fits.
constexpr int kSampleCap = 4096;

__global__ void __launch_bounds__(kThreads)
sample_kernel(const float *__restrict__ logits, int V, float temperature, uint64_t *rng, uint32_t *tokens,
              int tok_stride, int *len, int *flags) {
    __shared__ __align__(16) float row[kSampleCap];
    __shared__ float redf[kThreads / 64];
    __shared__ int redi[kThreads / 64];
    __shared__ double redd[kThreads / 64 + 1];
    __shared__ uint64_t tab[32];
    const int b = blockIdx.x;
    const float *src = logits + size_t(b) * V;
    const bool staged = V <= kSampleCap;
    if (staged)
        for (int t = threadIdx.x; t < V; t += blockDim.x) row[t] = src[t];
    stage_exp_table(tab);
    __syncthreads();
    const int token = choose_token(staged ? row : src, V, temperature, rng + b, flags,
                                   SampleLds{redf, redi, redd, tab}, staged ? row : nullptr);
    append_token(tokens, tok_stride, len, b, token);
}

// The same choice made by one wave per sequence (wave_choose_token, the
// persistent decode's sampler), for vocabularies of at most kWaveSampleVocab.
// RMAX tokens per lane at most: vocabularies of at most 256 run the
// four-token version the persistent decode uses for them, larger ones the
// sixteen-token version.
constexpr int kWaveSampleVocab = 1024;

template <int RMAX>
__global__ void __launch_bounds__(64)
wave_sample_kernel(const float *__restrict__ logits, int V, float temperature, uint64_t *rng, uint32_t *tokens,
                   int tok_stride, int *len, int *flags) {
    __shared__ uint64_t tab[32];
    const int b = blockIdx.x, R = (V + 63) / 64, i0 = int(threadIdx.x) * R;
    const float *src = logits + size_t(b) * V;
    float lg[RMAX];
#pragma unroll
    for (int k = 0; k < RMAX; ++k) lg[k] = k < R && i0 + k < V ? src[i0 + k] : 0.0f;
    stage_exp_table(tab);
    __syncthreads();
    uint64_t state = rng[b];
    const float u = temperature == 0.0f ? 0.0f : rng_unit(state);  // greedy draws nothing
    const int token = wave_choose_token(lg, V, temperature, u, tab, flags);
    if (threadIdx.x == 0) rng[b] = state;
    append_token(tokens, tok_stride, len, b, token);
}

// Decode head: one block of 1024 threads per sequence.  Thread (token quad q,
// c-group g) accumulates four tokens over channels g, g+16, ... with float4
// loads of Et, sixteen in flight; the groups' partials meet in LDS, then the
// block samples the next token.  Requires V <= kHeadSampleCap.
constexpr int kHsThreads = 1024, kHsGroups = kHsThreads / 64, kHeadSampleCap = 4096;

__global__ void __launch_bounds__(kHsThreads)
head_sample_kernel(Shape s, const float *__restrict__ xn, const float *__restrict__ Et, int Vp,
                   float *__restrict__ logits, float temperature, uint64_t *rng, uint32_t *tokens, int tok_stride,
                   int *len, int *flags) {
    extern __shared__ __align__(16) char smem[];
    LdsCarve lds{smem};
    const int W = s.W, V = s.V, b = blockIdx.x;
    float *N = lds.take<float>(size_t(W));
    float *L = lds.take<float>(size_t(kHeadSampleCap));
    float4 *red = lds.take<float4>(size_t(kHsGroups) * 64);
    float *redf = lds.take<float>(kHsThreads / 64);
    int *redi = lds.take<int>(kHsThreads / 64);
    double *redd = lds.take<double>(kHsThreads / 64 + 1);
    uint64_t *tab = lds.take<uint64_t>(32);
    for (int c = threadIdx.x; c < W; c += blockDim.x) N[c] = xn[size_t(b) * W + c];
    stage_exp_table(tab);
    __syncthreads();
    const int q = threadIdx.x & 63, g = threadIdx.x >> 6, quads = Vp / 4;
    const float4 *E4 = reinterpret_cast<const float4 *>(Et);
    for (int t0 = 0; t0 < V; t0 += 256) {
        const int qi = min(t0 / 4 + q, quads - 1);
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        constexpr int kUnroll = 16;
        for (int c0 = g; c0 < W; c0 += kHsGroups * kUnroll) {
            float4 e[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) e[u] = E4[size_t(min(c0 + u * kHsGroups, W - 1)) * quads + qi];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const int c = c0 + u * kHsGroups;
                if (c < W) {
                    const float n = N[c];
                    acc.x = fmaf(n, e[u].x, acc.x);
                    acc.y = fmaf(n, e[u].y, acc.y);
                    acc.z = fmaf(n, e[u].z, acc.z);
                    acc.w = fmaf(n, e[u].w, acc.w);
                }
            }
        }
        red[g * 64 + q] = acc;
        __syncthreads();
        if (threadIdx.x < 256) {
            const int tq = threadIdx.x >> 2, lane4 = threadIdx.x & 3, t = t0 + threadIdx.x;
            float sum = 0.0f;
            for (int k = 0; k < kHsGroups; ++k) {
                const float4 v = red[k * 64 + tq];
                sum += lane4 == 0 ? v.x : (lane4 == 1 ? v.y : (lane4 == 2 ? v.z : v.w));
            }
            if (t < V) {
                L[t] = sum;
                logits[size_t(b) * V + t] = sum;
            }
        }
        __syncthreads();
    }
    const int token = choose_token(L, V, temperature, rng + b, flags, SampleLds{redf, redi, redd, tab}, L);
    append_token(tokens, tok_stride, len, b, token);
}

// ------------------------------------------------ persistent decode kernel
//
// Every decode step of a batch in one launch, as a dataflow between
// workgroups that stay resident for the whole launch:
//   mesh teams   three per sequence (the row decode kernel's teams): the
//                residual row lives in their registers across layers; each
//                team repeats the post-attention meshes of block l-1, then
//                runs its Q, K or V mesh of block l;
//   attention    one per (sequence, head): appends the head's new K/V row to
//                the cache and attends over the head's keys, each layer.
// After the last block's attention all 3 + H workgroups of a sequence repeat
// its post-attention half and each computes 1/(3 + H) of the logits; the
// three teams then draw the same next token from the same logits and state.
// Sequences advance independently, so one sequence's meshes overlap another's
// KV stream.
//
// Hand-offs are tagged words: every exchanged float travels in a 64-bit word
// whose high half holds the sequence number of the phase that wrote it,
// stored and loaded with single-copy-atomic agent-scope accesses.  A consumer
// polls exactly the words it needs until their tags match, so data and
// readiness arrive together; no flag, fence or store drain sits on the
// chain.  The exchange buffers are zeroed before a launch (tag 0 is never
// waited for), and a word is rewritten only after every reader of its
// previous value has read it (each rewrite depends, through the chain, on
// those reads).  The cache rows of a (sequence, head) are written and later
// read only by that pair's attention workgroup, so its own barriers order
// them.  Every poll is bounded: after the launch's wait limit (kWaitTicks
// unless the host sets another) it raises *abort, a poll that sees *abort
// gives up soon after, and the launch then runs to its end on whatever it
// read (trip counts are fixed and tokens stay in range), so a broken
// hand-off ends the launch with an error, not a hang.
//
// Every block must be resident at once.  The launch is an ordinary one (a
// cooperative launch, which would guarantee it, takes ~12 us longer to start
// and end): the host launches only when every block fits the GPU at once
// (persistent_fits), which an otherwise idle GPU then gives.  Should some
// blocks still have to wait for room (another kernel holding part of the
// GPU), the resident ones time out and the launch ends with *abort set; the
// sampler states go to rng_out, not rng, so the host then has the state
// before the launch and runs the same steps on the per-phase kernels.

constexpr uint64_t kWaitTicks = 20000000;  // 0.2 s of the 100 MHz wall clock
constexpr uint32_t kPollCheck = 16;        // polls between checks of the abort flag and the clock
constexpr int kPersistVocab = 1024;        // largest vocabulary of the persistent path
static_assert(kPersistVocab <= kWaveSampleVocab, "the persistent path draws with the wave sampler");

// Hand-off words of a sequence whose workgroups share one XCD ("local") go
// through that XCD's L2 with non-temporal accesses, which skip the CU's L1
// cache: about 0.45 us a hand-off instead of 0.75 us with agent-scope
// atomics, which reach the memory side.  Sequences spread over XCDs use the
// atomics.  Either way every word is one naturally aligned 64-bit access.
// The exchange words are in global memory: addressed as such (global_u64),
// the accesses are global (not flat) loads and stores.

__device__ __forceinline__ void put_word(uint64_t *p, float v, int tag, bool local) {
    const uint64_t w = (uint64_t(uint32_t(tag)) << 32) | __float_as_uint(v);
    if (local)
        __builtin_nontemporal_store(w, (global_u64 *)p);
    else
        __hip_atomic_store((global_u64 *)p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t get_word(const uint64_t *p, bool local) {
    if (local) return __builtin_nontemporal_load((const global_u64 *)p);
    return __hip_atomic_load((const global_u64 *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// out[i] = the float of the word at addr(i), i < N, once every such word of
// the wave carries `tag`.
template <int N, bool LOCAL, class Addr>
__device__ __forceinline__ void take_words(Addr addr, int tag, float (&out)[N], int *abort, uint64_t wait_ticks) {
    constexpr bool local = LOCAL;
    const uint32_t want = uint32_t(tag);
    uint64_t w[N];
#pragma unroll
    for (int i = 0; i < N; ++i) w[i] = get_word(addr(i), local);
    auto ready = [&] {
        bool r = true;
#pragma unroll
        for (int i = 0; i < N; ++i) r = r && uint32_t(w[i] >> 32) == want;
        return r;
    };
    if (!__all(ready())) {
        const uint64_t t0 = wall_clock64();
        // A limit below the default (a host override, used to force time outs
        // in tests) is checked on every poll.
        static_assert((kPollCheck & (kPollCheck - 1)) == 0, "a power of two");
        const uint32_t check_mask = wait_ticks < kWaitTicks ? 0 : kPollCheck - 1;
        for (uint32_t n = 1;; ++n) {
            __builtin_amdgcn_s_sleep(1);
            asm volatile("" ::: "memory");  // the words change under us: load them again
            // Every word again (no per-word branch, whose evaluation would
            // wait inside the loop): one memory round trip per poll.  The
            // abort flag (an agent-scope load, slower than the words') and
            // the clock are read every kPollCheck polls only, so they do not
            // lengthen the polls that find the words.
#pragma unroll
            for (int i = 0; i < N; ++i) w[i] = get_word(addr(i), local);
            if (__all(ready())) break;
            if ((n & check_mask) == 0) {
                if (__hip_atomic_load(abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) break;
                if (wall_clock64() - t0 > wait_ticks) {
                    if ((threadIdx.x & 63) == 0) __hip_atomic_store(abort, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = __uint_as_float(uint32_t(w[i]));
}

// ---- K/V staging through LDS
//
// The attention workgroups stream their K/V rows into an LDS ring with
// direct-to-LDS loads (global_load_lds_dwordx4: each lane's 16 bytes land at
// a wave-uniform LDS base + 16 * lane), so several rounds are in flight
// without holding registers.  The loads are issued from inline assembly and
// waited for with explicit vmcnt counts: issued through the compiler, every
// LDS read after them would wait for all loads in flight.  Waiting for
// vmcnt <= n, where n counts only this ring's loads issued after the awaited
// round, is always sufficient: other memory operations issued meanwhile only
// make the wait stricter, as loads complete in order.

typedef __attribute__((address_space(3))) float lds_float;

// LDS[l + 16 * lane .. +16) = g[0..4) for every lane; l is wave-uniform.  The
// LDS reads of earlier rounds are complete first (lgkmcnt), so a slot can be
// refilled right after it was read; m0 is preserved.
__device__ __forceinline__ void lds_dma16(const float *g, float *l) {
    const uint32_t m = __builtin_amdgcn_readfirstlane(uint32_t(size_t((lds_float *)l)));
    uint32_t save;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_waitcnt lgkmcnt(0)\n\t"
        "global_load_lds_dwordx4 %2, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(save)
        : "s"(m), "v"(g)
        : "memory");
}

// lds_dma16 with the non-temporal cache policy.
__device__ __forceinline__ void lds_dma16_nt(const float *g, float *l) {
    const uint32_t m = __builtin_amdgcn_readfirstlane(uint32_t(size_t((lds_float *)l)));
    uint32_t save;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_waitcnt lgkmcnt(0)\n\t"
        "global_load_lds_dwordx4 %2, off nt\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(save)
        : "s"(m), "v"(g)
        : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmem() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Ring of NS rounds of an attention share in LDS: round r (keys from r * G *
// UL, laid out as AttnRound) fills slot r % NS; each lane's K and V rows of a
// round are 2 * UL chunks of 16 bytes in its wave's region of the slot.
template <int HDP, int NW, int UL, int NS>
struct KvRing {
    using R = AttnRound<HDP, 64 * NW, UL>;
    static constexpr int VEC = R::VEC, LPK = R::LPK, G = R::G, CH = 2 * UL;
    static constexpr int SLOT = CH * NW * 256;  // floats
    static_assert(VEC == 4, "a lane's part of a row must be one 16-byte load");
    float *buf;  // NS * SLOT floats
    // Rounds that reach past the first `keep` rows load with the
    // non-temporal policy (kv_keep_rows).
    __device__ void issue(const float *kl, const float *vl, int r, int end, int tid, int keep = 1 << 30) const {
        const int g = tid / LPK, d0 = (tid % LPK) * VEC, wave = tid >> 6;
        float *slot = buf + (r % NS) * SLOT + wave * 256;
        if ((r + 1) * G * UL > keep) {
#pragma unroll
            for (int u = 0; u < UL; ++u) {
                const uint32_t at = uint32_t(min(r * G * UL + u * G + g, end - 1)) * HDP + d0;
                lds_dma16_nt(kl + at, slot + (2 * u) * NW * 256);
                lds_dma16_nt(vl + at, slot + (2 * u + 1) * NW * 256);
            }
            return;
        }
#pragma unroll
        for (int u = 0; u < UL; ++u) {
            const uint32_t at = uint32_t(min(r * G * UL + u * G + g, end - 1)) * HDP + d0;
            lds_dma16(kl + at, slot + (2 * u) * NW * 256);
            lds_dma16(vl + at, slot + (2 * u + 1) * NW * 256);
        }
    }
    // Waits until round r has landed, given the rounds issued after it.
    __device__ void wait(int after) const {
        static_assert(NS <= 4, "wait counts");
        switch (after) {
        case 0: wait_vmem<0>(); break;
        case 1: wait_vmem<CH>(); break;
        case 2: wait_vmem<2 * CH>(); break;
        default: wait_vmem<3 * CH>(); break;
        }
    }
    __device__ void read(int r, R &cur, int tid) const {
        const float *slot = buf + (r % NS) * SLOT + (tid >> 6) * 256 + (tid & 63) * 4;
#pragma unroll
        for (int u = 0; u < UL; ++u) {
            const float4 k = *reinterpret_cast<const float4 *>(slot + (2 * u) * NW * 256);
            const float4 v = *reinterpret_cast<const float4 *>(slot + (2 * u + 1) * NW * 256);
            cur.k[u][0] = k.x;
            cur.k[u][1] = k.y;
            cur.k[u][2] = k.z;
            cur.k[u][3] = k.w;
            cur.v[u][0] = v.x;
            cur.v[u][1] = v.y;
            cur.v[u][2] = v.z;
            cur.v[u][3] = v.w;
        }
    }
};

// Geometry of the persistent attention ring: keys per lane group in a round
// (UL) and rounds in flight (NS), chosen to fit beside the kernel's other LDS
// arrays while the registers' limit of two waves per SIMD stays the only
// limit on residency (LDS budget 160 KiB * NW / 8 per workgroup).  Rounds of
// 4 keys per group with two slots are preferred; narrower rounds with more
// slots when those do not fit.
template <int NW, int CPL, int GL, int HDP>
struct PersistRing {
    static constexpr int W = 64 * NW * CPL, gc = 64 / GL;
    static constexpr int budget = 160 * 1024 * NW / 8;
    // persistent_decode_kernel's other LDS: xch, red, xn, row and the exp table
    static constexpr int other = 4 * (2 * W + 8 * CPL * NW * gc + W + kPersistVocab) + 256 + 64;
    static constexpr int fit(int ul) { return (budget - other) / (2 * ul * NW * 1024); }
    static constexpr int UL = fit(4) >= 2 ? 4 : (fit(2) >= 2 ? 2 : 1);
    static constexpr int NS = UL == 4 ? 2 : (fit(UL) >= 4 ? 4 : (fit(UL) >= 3 ? 3 : 2));
    static_assert(fit(UL) >= NS, "the attention ring does not fit in LDS");
};

// Records one trace timestamp (thread 0) when a timeline is requested.
__device__ __forceinline__ void trace_mark(const PersistArgs &a, int row, int step, int l, int which) {
    if (a.trace && threadIdx.x == 0)
        a.trace[((size_t(row) * a.steps + step) * (a.layers + 1) + l) * 2 + which] = wall_clock64();
}

// A trace time taken now and stored later (trace_store): a store in between
// would count in the vector-memory counter that the LDS ring's waits count.
__device__ __forceinline__ uint64_t trace_time(const PersistArgs &a) { return a.trace ? wall_clock64() : 0; }

__device__ __forceinline__ void trace_store(const PersistArgs &a, int row, int step, int l, int which, uint64_t t) {
    if (a.trace && threadIdx.x == 0) a.trace[((size_t(row) * a.steps + step) * (a.layers + 1) + l) * 2 + which] = t;
}

// Row-order index of channel c (the layout RowCtx::ridx enumerates).
template <int NW>
__device__ __forceinline__ int row_of(int c) {
    return ((c / (64 * NW)) * NW + c % NW) * 64 + (c / NW) % 64;
}

// One sequence's exchange words (row order unless noted).  Layer phase
// g = step * layers + l: q/k/v and the attention output of phase g carry tag
// g + 1; the normalised final row and the logits of a step carry tag
// step + 1.
template <bool LOCAL>  // all workgroups of the sequence on one XCD (see put_word)
struct PersistXch {
    static constexpr bool local = LOCAL;
    uint64_t *base;
    int W, V;
    int row;  // this workgroup's row of the trace (3 * batch teams, then batch * H heads)
    uint64_t wait;  // a wait's limit (PersistArgs::wait_ticks)
    __device__ PersistXch(const PersistArgs &a, int b, int row_)
        : base(a.xch + size_t(b) * a.xstride), W(a.s.W), V(a.s.V), row(row_), wait(a.wait_ticks) {}
    // q (t = 0), k (1) or v (2) of phase g, double-buffered by phase parity
    __device__ uint64_t *qkv(int g, int t) const { return base + size_t((g & 1) * 3 + t) * W; }
    __device__ uint64_t *y() const { return base + size_t(6) * W; }     // attention output
    __device__ uint64_t *xrow() const { return base + size_t(7) * W; }  // normalised final row
    __device__ uint64_t *logits() const { return base + size_t(8) * W; }  // token order
    __device__ uint64_t *xcd() const { return base + size_t(8) * W + V; }  // each workgroup's XCD
    __device__ void put(uint64_t *p, float v, int tag) const { put_word(p, v, tag, LOCAL); }
    template <int N, class Addr>
    __device__ void take(Addr addr, int tag, float (&out)[N], int *abort) const {
        take_words<N, LOCAL>(addr, tag, out, abort, wait);
    }
};

// All 3 + H workgroups of a sequence publish their XCD and read everyone's:
// the sequence's hand-offs use the XCD-local protocol when they agree.  This
// first exchange always uses the agent-scope atomics.
__device__ __forceinline__ bool persistent_handshake(const PersistArgs &a, const PersistXch<false> &xc, int role) {
    const int R = 3 + a.s.H;
    uint32_t xcd;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcd));
    xcd &= 0xf;
    if (threadIdx.x == 0) xc.put(xc.xcd() + role, float(xcd), 1);
    float seen[1];
    const int k = int(threadIdx.x) < R ? int(threadIdx.x) : 0;
    xc.take<1>([&](int) { return xc.xcd() + k; }, 1, seen, a.abort);
    return __syncthreads_and(seen[0] == float(xcd)) != 0;
}

// Logits of tokens [t0, t1) for the row-order normalised row xn (in LDS), as
// words tagged `tag`: wave w takes tokens t0 + w, t0 + w + NW, ...; each lane
// a contiguous W/64 channels of the row-order token vectors E.  T tokens'
// loads per wave are in flight before their dot products and wave sums.
// T rows of the tied head at a time: row t = base + u*NW of a wave's rows, from
// E in global memory or from its rows staged in LDS (stage_head_rows: LDS row
// t - t0), dotted with the normalised row and published as logit words.
template <int NW, int W>
struct HeadBatch {
    static constexpr int CW = W / 64, T = 96 / CW < 4 ? 4 : (96 / CW > 8 ? 8 : 96 / CW);
    static_assert(T <= 64, "lane u publishes row u");
    float e[T][CW];
    template <bool STAGED>
    __device__ __forceinline__ void load(const float *__restrict__ rows, int t0, int base, int t1, int lane) {
#pragma unroll
        for (int u = 0; u < T; ++u) {
            // Past t1 a lane reads a row of its own wave (the staged rows a
            // wave may read are the ones it copied) and publishes nothing.
            const int t = base + u * NW;
            const float *row = STAGED ? rows + ((t < t1 ? t : base) - t0) * W + lane * CW
                                      : rows + (uint32_t(min(t, t1 - 1)) * W + uint32_t(lane * CW));
            if constexpr (CW % 4 == 0) {
#pragma unroll
                for (int k = 0; k < CW; k += 4) {
                    const float4 v = *reinterpret_cast<const float4 *>(row + k);
                    e[u][k] = v.x;
                    e[u][k + 1] = v.y;
                    e[u][k + 2] = v.z;
                    e[u][k + 3] = v.w;
                }
            } else {
#pragma unroll
                for (int k = 0; k < CW; ++k) e[u][k] = row[k];
            }
        }
    }
    // Each lane's part of the T dot products, their sums over the wave (for
    // T = 8 all at once, wave_sum8: issued one row after another, eight
    // wave_sum chains cost ~0.4 us), then lane u publishes row u.
    template <class X>
    __device__ __forceinline__ void publish(const float (&xr)[CW], const X &xc, int base, int t1, int tag,
                                            int lane) const {
        float dots[T];
#pragma unroll
        for (int u = 0; u < T; ++u) {
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < CW; ++k) acc = fmaf(xr[k], e[u][k], acc);
            dots[u] = acc;
        }
        float mine = 0.0f;
        if constexpr (T == 8) {
            mine = wave_sum8(dots, lane);
        } else {
#pragma unroll
            for (int u = 0; u < T; ++u) {
                const float s = wave_sum(dots[u]);
                mine = lane == u ? s : mine;
            }
        }
        const int t = base + lane * NW;
        if (lane < T && t < t1) xc.put(xc.logits() + t, mine, tag);
    }
};

// Logits [t0, t1) of the tied head from the normalised row xn (row order, in
// LDS), wave w taking rows t0 + w + u*NW from its first batch at `base` on;
// with STAGED the E rows come from `rows` in LDS (stage_head_rows), else from
// E in global memory.
template <int NW, int W, bool STAGED, class X>
__device__ __forceinline__ void persistent_head_slice(const float *xn, const float *__restrict__ rows, const X &xc,
                                                      int t0, int base, int t1, int tag, int lane) {
    using HB = HeadBatch<NW, W>;
    float xr[HB::CW];
#pragma unroll
    for (int k = 0; k < HB::CW; ++k) xr[k] = xn[lane * HB::CW + k];
    for (; base < t1; base += HB::T * NW) {
        HB hb;
        hb.template load<STAGED>(rows, t0, base, t1, lane);
        hb.publish(xr, xc, base, t1, tag, lane);
    }
}

// Rows [t0, t1) of E copied into LDS at stage + (t - t0) * W by direct loads:
// wave w copies the rows t0 + w + u*NW that it later reads itself, so its own
// wait (wait_vmem) is the only synchronisation needed.
template <int NW, int W>
__device__ __forceinline__ void stage_head_rows(const float *E, float *stage, int t0, int t1, int lane, int wave) {
    static_assert(W % 256 == 0, "a row is whole 1 KiB wave copies");
    for (int t = t0 + wave; t < t1; t += NW) {
        const float *src = E + size_t(t) * W + lane * 4;
        float *dst = stage + (t - t0) * W;
#pragma unroll
        for (int c = 0; c < W / 256; ++c) lds_dma16(src + c * 256, dst + c * 256);
    }
}

// Hides a uniform pointer's value from the optimiser, so the per-load
// addresses derived from it are formed next to their loads instead of being
// hoisted out of the step loop, where they would hold dozens of registers.
template <class T>
__device__ __forceinline__ T *opaque(T *p) {
    // The pointer is wave-uniform; readfirstlane states that, so the operand
    // can live in scalar registers even where p arrives in vector ones.
    const uint64_t u = uint64_t(p);
    uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(u)), hi = __builtin_amdgcn_readfirstlane(uint32_t(u >> 32));
    asm volatile("" : "+s"(lo), "+s"(hi));
    return reinterpret_cast<T *>((uint64_t(hi) << 32) | lo);
}

// Whether row_mesh2 applies: a fixed-depth mesh of depth >= 3 whose first
// two strides (1 and 2) both cross waves.
template <int NW, int D>
constexpr bool kMesh2 = NW >= 4 && D >= 3;

// Layer-0 weights (row order) of channels chan(j) + 2, which row_mesh2 needs
// besides the lane's own.
template <int NW, int CPL, int GL>
__device__ __forceinline__ void load_mesh_far(float2 (&w)[CPL], const float *wg, const RowCtx<NW, CPL, GL> &c) {
    constexpr int W = RowCtx<NW, CPL, GL>::W;
    const global_u64 *g = (const global_u64 *)opaque(wg);
#pragma unroll
    for (int j = 0; j < CPL; ++j) w[j] = __builtin_bit_cast(float2, uint64_t(g[row_of<NW>((c.chan(j) + 2) & (W - 1))]));
}

// n = mesh(x), or mesh(x * inv_rms(x)) with RMS, in the log2(e)-scaled units
// of row_layer (x itself scaled without RMS), for a mesh whose first two
// strides cross waves: one LDS exchange serves both layers (each lane reads
// channels c + 1 .. c + 3 and computes layer 0 of channel c + 2 as well, with
// its weights w0far), and with RMS the row reduction shares its barrier.  The
// arithmetic of row_inv_rms and row_run_mesh, value for value.
template <bool RMS, int NW, int CPL, int GL, int D>
__device__ __forceinline__ void row_mesh2(RowCtx<NW, CPL, GL> &c, const float (&x)[CPL], float (&n)[CPL],
                                          const float2 (&w)[D][CPL], const float2 (&w0far)[CPL], int k) {
    static_assert(kMesh2<NW, D>, "strides 1 and 2 must cross waves");
    constexpr int W = 64 * NW * CPL;
    constexpr int LOG2W = W == 128 ? 7 : W == 256 ? 8 : W == 512 ? 9 : 10;
    const int lane = c.lane, wave = c.wave;
    float *red = c.slot(k);
    if constexpr (RMS) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) acc = fmaf(x[j], x[j], acc);
        acc = wave_sum(acc);
        if (lane == 0) red[wave] = acc;
    }
    float *b = c.xch + (c.parity & 1) * (NW * CPL * 64);
    ++c.parity;
#pragma unroll
    for (int j = 0; j < CPL; ++j) b[(j * NW + wave) * 64 + lane] = x[j];
    __syncthreads();
    float inv = 1.0f;
    if constexpr (RMS) {
        float t = 0.0f;
#pragma unroll
        for (int v = 0; v < NW; ++v) t += red[v];
        inv = inv_rms_log2(t, W);
    }
    auto scaled = [&](float v) { return RMS ? v * inv : v; };
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int ch = c.chan(j);
        const float n0 = scaled(x[j]), n1 = scaled(b[row_of<NW>((ch + 1) & (W - 1))]);
        const float n2 = scaled(b[row_of<NW>((ch + 2) & (W - 1))]), n3 = scaled(b[row_of<NW>((ch + 3) & (W - 1))]);
        const float z0 = elu_log2(n0 * w[0][j].x + n1 * w[0][j].y);
        const float z2 = elu_log2(n2 * w0far[j].x + n3 * w0far[j].y);
        n[j] = elu_log2(z0 * w[1][j].x + z2 * w[1][j].y);
    }
    static_for<D>([&](auto U) {
        constexpr int u = decltype(U)::value;
        if constexpr (u > 1) row_layer<NW, CPL>(n, w[u], 1 << (u % LOG2W), u + 1 == D, lane, wave, c.xch, c.parity);
    });
}

// The post-attention half (row_post without XSA) with row_mesh2 heads: the
// projection mesh on y, the residual, then the FFN mesh on the normalised row
// and its residual.
template <int NW, int CPL, int GL, int D>
__device__ __forceinline__ void team_post_mesh2(RowCtx<NW, CPL, GL> &c, float (&x)[CPL], const float (&y)[CPL],
                                                const float2 (&wp)[D][CPL], const float2 (&wp2)[CPL],
                                                const float2 (&wf)[D][CPL], const float2 (&wf2)[CPL]) {
    float t[CPL], ys[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) ys[j] = y[j] * kLog2e;
    row_mesh2<false>(c, ys, t, wp, wp2, 2);
#pragma unroll
    for (int j = 0; j < CPL; ++j) x[j] = fmaf(t[j], kLn2, x[j]);
    row_mesh2<true>(c, x, t, wf, wf2, 2);
#pragma unroll
    for (int j = 0; j < CPL; ++j) x[j] = fmaf(t[j], kLn2, x[j]);
}

template <int NW, int CPL, int GL, int D>
__device__ __forceinline__ void load_block_weights(float2 (&w)[D][CPL], const float *g, bool fixed, int lane,
                                                   int wave) {
    if (fixed) row_load_weights<NW, CPL, D>(w, opaque(g), lane, wave);
}

struct PersistLds {
    float *xch, *red, *xn, *row, *ring;
    uint64_t *exp_tab;
    int ring_floats;
};

// Whether a workgroup's slice of E rows (at most ceil(V / (3 + H)) rows) fits
// the LDS ring; the teams, which never use the ring otherwise, then keep
// their slices there for the whole launch (stage_head_rows).  (Staging the
// attention workgroups' slices after their last layer costs more in the
// post-attention meshes, which run meanwhile, than the head saves.)
template <int W>
__device__ __forceinline__ bool head_rows_staged(const PersistArgs &a, const PersistLds &m) {
    const int nb = 3 + a.s.H;
    return W % 256 == 0 && (a.s.V + nb - 1) / nb * W <= m.ring_floats;
}

// The attention output of phase g (XSA applied by the attention workgroups),
// the input of the post-attention half.
template <int NW, int CPL, int GL, class X>
__device__ __forceinline__ void take_attention_output(const PersistArgs &a, const RowCtx<NW, CPL, GL> &c, const X &xc,
                                                      int g, float (&y)[CPL]) {
    const uint64_t *yw = xc.y();
    xc.template take<CPL>([&](int j) { return yw + c.ridx(j); }, g + 1, y, a.abort);
}

// The step's token from the published logits, drawn by each wave on its own:
// every wave of every workgroup of the sequence takes the same words and
// keeps the same generator state (`state`, wave-uniform), so all draw the same
// token, with no LDS exchange and no barrier (wave_choose_token).  The logits
// are also copied to `out` when given.
template <bool MARK, class X>
__device__ __forceinline__ uint32_t draw_token(const PersistArgs &a, const X &xc, int step, uint64_t &state,
                                               const PersistLds &m, float *out) {
    constexpr int RMAX = kPersistVocab / 64;
    static_assert(RMAX % 4 == 0, "logit words are taken four at a time");
    // Lane offsets and word addresses are formed here from a thread index and
    // base hidden from the optimiser: hoisted out of the step loop, they would
    // occupy dozens of registers through the layers.
    int tid = int(threadIdx.x);
    asm volatile("" : "+v"(tid));
    const int V = a.s.V, R = (V + 63) / 64, i0 = (tid & 63) * R;
    const uint64_t *lw = opaque(xc.logits());
    const float u = a.temperature == 0.0f ? 0.0f : rng_unit(state);  // greedy draws nothing
    float lg[RMAX];
#pragma unroll
    for (int c = 0; c < RMAX / 4; ++c) {
        if (4 * c < R) {  // uniform: a small vocabulary polls only its words
            float t[4];
            xc.template take<4>([&](int k) { return lw + min(i0 + 4 * c + k, V - 1); }, step + 1, t, a.abort);
#pragma unroll
            for (int k = 0; k < 4; ++k) lg[4 * c + k] = t[k];
        }
    }
    if (MARK) trace_mark(a, xc.row, step, a.layers, 0);
    if (out && tid < 64) {
        float *o = opaque(out) + i0;
#pragma unroll
        for (int k = 0; k < RMAX; ++k)
            if (k < R && i0 + k < V) o[k] = lg[k];
    }
    // A wave issues one instruction per four cycles and this code runs once
    // per step on the critical path: a vocabulary of at most 256 tokens (four
    // per lane) gets the version unrolled for four.
    // The vocabularies of the persistent configurations (256, and 64 for
    // the smallest) get versions compiled for them.
    if (R <= 4) {
        const float l4[4] = {lg[0], lg[1], lg[2], lg[3]};
        if (V == 256) return uint32_t(wave_choose_token<4, 256>(l4, V, a.temperature, u, m.exp_tab, a.flags));
        if (V == 64) return uint32_t(wave_choose_token<4, 64>(l4, V, a.temperature, u, m.exp_tab, a.flags));
        return uint32_t(wave_choose_token(l4, V, a.temperature, u, m.exp_tab, a.flags));
    }
    return uint32_t(wave_choose_token(lg, V, a.temperature, u, m.exp_tab, a.flags));
}

// Post-attention half of the last block on team `slice`'s residual row x and
// the final RMSNorm; team 0 publishes the normalised row for the attention
// workgroups (which would otherwise wait for the weights, loaded only after
// their own last attention); then logit slice `slice` of the 3 + H slices of
// the vocabulary.
template <int NW, int CPL, int GL, int DEPTH, class X>
__device__ __forceinline__ void persistent_last_block(const PersistArgs &a, RowCtx<NW, CPL, GL> &c, float (&x)[CPL],
                                                      const X &xc, int step, int slice, const PersistLds &m) {
    constexpr int W = RowCtx<NW, CPL, GL>::W;
    constexpr bool FIXED = DEPTH > 0;
    constexpr int D = FIXED ? DEPTH : 1;
    const Shape &s = a.s;
    const int L = a.layers, g = step * L + L - 1;
    const size_t gA = 2 * size_t(W) * s.A;
    const float *wlast = a.w + a.block0 + size_t(L - 1) * (4 * gA + 2 * size_t(W) * s.F);
    float2 wp[D][CPL], wf[D][CPL];
    load_block_weights<NW, CPL, GL, D>(wp, wlast + 3 * gA, FIXED, c.lane, c.wave);
    load_block_weights<NW, CPL, GL, D>(wf, wlast + 4 * gA, FIXED, c.lane, c.wave);
    float2 wp2[CPL], wf2[CPL];
    if constexpr (FIXED && kMesh2<NW, D>) {
        load_mesh_far(wp2, wlast + 3 * gA, c);
        load_mesh_far(wf2, wlast + 4 * gA, c);
    }
    float y[CPL];
    take_attention_output(a, c, xc, g, y);
    const int nb = 3 + s.H, V = s.V, t0 = slice * V / nb, t1 = (slice + 1) * V / nb;
    if constexpr (FIXED && kMesh2<NW, D>)
        team_post_mesh2(c, x, y, wp, wp2, wf, wf2);
    else
        row_post<NW, CPL, GL, D, false>(c, x, y, y, wp, wf, wlast + 3 * gA, wlast + 4 * gA, s, FIXED);
    const float inv = row_inv_rms(c, x, 3);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const float n = x[j] * inv;
        m.xn[c.ridx(j)] = n;
        if (slice == 0) xc.put(xc.xrow() + c.ridx(j), n, step + 1);
    }
    __syncthreads();
    if (head_rows_staged<W>(a, m)) {
        wait_vmem<0>();  // this wave's staged rows (staged once)
        persistent_head_slice<NW, W, true>(m.xn, m.ring, xc, t0, t0 + c.wave, t1, step + 1, c.lane);
    } else {
        persistent_head_slice<NW, W, false>(m.xn, a.E, xc, t0, t0 + c.wave, t1, step + 1, c.lane);
    }
}

// An attention workgroup's logit slice `slice`, from the normalised final row
// that team 0 publishes.
template <int NW, int CPL, int GL, class X>
__device__ __forceinline__ void persistent_head_logits(const PersistArgs &a, const RowCtx<NW, CPL, GL> &c,
                                                       const X &xc, int step, int slice, const PersistLds &m) {
    constexpr int W = RowCtx<NW, CPL, GL>::W;
    const int nb = 3 + a.s.H, V = a.s.V, t0 = slice * V / nb, t1 = (slice + 1) * V / nb;
    using HB = HeadBatch<NW, W>;
    // The first batch of E rows loads while the row is awaited.
    const int base = t0 + c.wave;
    HB first;
    if (base < t1) first.template load<false>(a.E, t0, base, t1, c.lane);
    float n[CPL];
    xc.template take<CPL>([&](int j) { return xc.xrow() + c.ridx(j); }, step + 1, n, a.abort);
#pragma unroll
    for (int j = 0; j < CPL; ++j) m.xn[c.ridx(j)] = n[j];
    __syncthreads();
    trace_mark(a, xc.row, step, a.layers, 0);
    if (base < t1) {
        float xr[HB::CW];
#pragma unroll
        for (int k = 0; k < HB::CW; ++k) xr[k] = m.xn[c.lane * HB::CW + k];
        first.publish(xr, xc, base, t1, step + 1, c.lane);
    }
    persistent_head_slice<NW, W, false>(m.xn, a.E, xc, t0, base + HB::T * NW, t1, step + 1, c.lane);
}

// A sequence's decode state at the start of the launch, loaded before the
// XCD handshake so that the loads overlap it.
struct PersistStart {
    int len;       // tokens so far
    uint32_t tok;  // the last of them
    uint64_t rng;  // the sampler's state
};

// Mesh team `team` of sequence b.
template <int NW, int CPL, int GL, int DEPTH, int HDP, class X>
__device__ __forceinline__ void persistent_team(const PersistArgs &a, int b, int team, const PersistLds &m,
                                                const X &xc, const PersistStart &st0) {
    using Ctx = RowCtx<NW, CPL, GL>;
    constexpr int W = Ctx::W;
    constexpr bool FIXED = DEPTH > 0;
    constexpr int D = FIXED ? DEPTH : 1;
    const Shape &s = a.s;
    Ctx c(m.xch, m.red);
    const int L = a.layers, V = s.V;
    int len = st0.len;
    uint32_t tok = st0.tok;
    uint64_t rng = st0.rng;  // the sampler's state, the same in every wave
    if constexpr (W % 256 == 0) {
        // The team's slice of E rows stays in the (otherwise unused) ring.
        const int nb = 3 + s.H;
        if (head_rows_staged<W>(a, m)) stage_head_rows<NW, W>(a.E, m.ring, team * V / nb, (team + 1) * V / nb, c.lane, c.wave);
    }
    const size_t gA = 2 * size_t(W) * s.A;           // floats of one attention-depth mesh
    const size_t blk = 4 * gA + 2 * size_t(W) * s.F;  // floats of one block: q, k, v, proj, ffn
    auto block = [&](int l) { return a.w + a.block0 + size_t(l) * blk; };
    float2 wp[D][CPL], wf[D][CPL], wm[D][CPL];
    for (int step = 0; step < a.steps; ++step) {
        float x[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j) x[j] = a.E[size_t(tok) * W + c.ridx(j)];
        trace_mark(a, xc.row, step, 0, 0);
        // Layer 0's q, k and v are the token's rows of the layer-0 table, which
        // the attention blocks read themselves: the teams start at block 0's
        // post-attention half.
        trace_mark(a, xc.row, step, 0, 1);
        for (int l = 1; l < L; ++l) {
            const int g = step * L + l;
            const float *wb = block(l), *wq = block(l - 1);
            // Post-attention half of block l-1, its weights loading during the wait.
            load_block_weights<NW, CPL, GL, D>(wm, wb + team * gA, FIXED, c.lane, c.wave);
            load_block_weights<NW, CPL, GL, D>(wp, wq + 3 * gA, FIXED, c.lane, c.wave);
            load_block_weights<NW, CPL, GL, D>(wf, wq + 4 * gA, FIXED, c.lane, c.wave);
            float2 wp2[CPL], wf2[CPL], wm2[CPL];  // layer 0 of channels c + 2 (row_mesh2)
            if constexpr (FIXED && kMesh2<NW, D>) {
                load_mesh_far(wp2, wq + 3 * gA, c);
                load_mesh_far(wf2, wq + 4 * gA, c);
                load_mesh_far(wm2, wb + team * gA, c);
            }
            float y[CPL];
            take_attention_output(a, c, xc, g - 1, y);
            trace_mark(a, xc.row, step, l, 0);
            if constexpr (FIXED && kMesh2<NW, D>)
                team_post_mesh2(c, x, y, wp, wp2, wf, wf2);
            else
                row_post<NW, CPL, GL, D, false>(c, x, y, y, wp, wf, wq + 3 * gA, wq + 4 * gA, s, FIXED);
            // q and k go out before QK-norm and RoPE, which the attention
            // workgroups apply per head.
            float n[CPL];
            if constexpr (FIXED && kMesh2<NW, D>) {
                row_mesh2<true>(c, x, n, wm, wm2, 3);
            } else if constexpr (FIXED && NW > 1) {
                row_rms_mesh(c, x, n, wm, 3);
            } else {
                const float inv = row_inv_rms(c, x, 3) * kLog2e;
#pragma unroll
                for (int j = 0; j < CPL; ++j) n[j] = x[j] * inv;
                row_run_mesh(c, n, wm, wb + team * gA, s.A, s, FIXED);
            }
            uint64_t *out = xc.qkv(g, team);
#pragma unroll
            for (int j = 0; j < CPL; ++j) xc.put(out + c.ridx(j), n[j] * kLn2, g + 1);
            trace_mark(a, xc.row, step, l, 1);
        }
        persistent_last_block<NW, CPL, GL, DEPTH>(a, c, x, xc, step, team, m);
        // The launch's last logits are kept for callers that read them.
        tok = draw_token<true>(a, xc, step, rng, m,
                               team == 0 && step + 1 == a.steps ? a.logits + size_t(b) * V : nullptr);
        trace_mark(a, xc.row, step, L, 1);
        if (team == 0 && threadIdx.x == 0) a.tokens[size_t(b) * a.tok_stride + len] = tok;
        ++len;
    }
    if (team == 0 && threadIdx.x == 0) {
        a.len[b] = len;
        a.rng_out[b] = rng;
    }
}

// QK-norm over the head, then RoPE at `pos` (reference.rs:462-482), for an
// attention lane's dims d0 .. d0 + VEC - 1 (each group of LPK lanes holds the
// whole head; the RoPE partner dim, hd/2 away, is LPK/2 lanes away).  The
// head's sum of squares adds each lane's dims first, then the lanes (one
// group reduction instead of one per dim): the same sum as row_qk_rope's in
// another order, within a few f32 roundings of it.
// cs[e] is the (cos, sin) pair of dim d0 + e at the position (rope_pair).
// With qs > 0 the result is scaled by qs (the query's score scale, folded
// into the norm factor as rsqrt((ss / hd + eps) / qs^2)).
template <int LPK, int VEC>
__device__ __forceinline__ void lane_qk_rope(float (&x)[VEC], int d0, const float2 (&cs)[VEC], const Shape &s,
                                             float qs = 0.0f) {
    float other[VEC];
    float sq = 0.0f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) sq = fmaf(x[e], x[e], sq);
    const float ss = group_sum<LPK>(sq);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
        // lane ^ 8 inside a 16-lane row is DPP row_ror:8
        if constexpr (LPK == 16) other[e] = dpp_move<0x128>(0.0f, x[e]);
        else other[e] = __shfl_xor(x[e], LPK / 2, 64);
    }
    const float q2 = qs > 0.0f ? 1.0f / (qs * qs) : 1.0f;  // uniform: off the chain
    const float sc = rsqrtf(ss * ((1.0f / float(s.hd)) * q2) + kRmsEps * q2);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
        const int d = d0 + e;
        const float self = x[e] * sc, oth = other[e] * sc;
        x[e] = d < s.half ? self * cs[e].x - oth * cs[e].y : self * cs[e].x + oth * cs[e].y;
    }
}

// Attention block of (sequence b, head h).  Its query, key and value arrive
// as tagged words, except at layer 0, where they are the token's rows of the
// layer-0 table; QK-norm and RoPE are applied here for every layer.  After
// the last layer it computes its slice of the logits from the final row team
// 0 publishes, and it draws each step's token itself, like the teams.  The
// key/value rows go to the cache for later steps and enter this step's
// attention from registers, so the cached rows read each layer [0, pos) were
// all written before the launch or by this block, and the first rounds of
// them load while the inputs are awaited.
template <int NW, int CPL, int GL, int DEPTH, int HDP, class X>
__device__ __forceinline__ void persistent_attention(const PersistArgs &a, int b, int h, const PersistLds &m,
                                                     const X &xc, int pair, const PersistStart &st0) {
    using Ctx = RowCtx<NW, CPL, GL>;
    using Ring = PersistRing<NW, CPL, GL, HDP>;
    using S = AttnState<HDP, 64 * NW, Ring::UL>;
    using R = typename S::R;
    constexpr int VEC = S::VEC, LPK = S::LPK, G = S::G, U = S::U, NS = Ring::NS;
    const KvRing<HDP, NW, U, NS> ring{m.ring};
    const Shape &s = a.s;
    constexpr int W = Ctx::W;
    const int len0 = st0.len, L = a.layers;

    const size_t slab = size_t(b * s.H + h) * a.cap * HDP;
    static_assert(VEC % NW == 0, "lane dims must cover whole row-order columns");
    uint32_t tok = st0.tok;
    uint64_t rng = st0.rng;
    for (int step = 0; step < a.steps; ++step) {
        const int pos = len0 + step - 1;  // this step's row; rows [0, pos) are cached
        for (int l = 0; l < L; ++l) {
            const int g = step * L + l;
            // Two workgroups sharing a CU (persistent_role's pairs: the same
            // head of two sequences) take turns at the front of the wave
            // arbiter: by layer parity, opposite to each other while their
            // sequences are at the same layer, and by step parity when the
            // layer parities agree (one sequence a layer ahead), where age
            // alone would always favour the first dispatched.  (Measured on
            // config 3: 26.6 ms a 512-step launch by age, 26.1 with the layer
            // parity, 25.9 with both; over the first 20 steps the sequences
            // of the four slots of an XCD averaged 30.1-32.9 us a step by
            // age, 31.0-32.0 and 31.1-31.4.)
            if (pair != 0) {
                const int p = 2 * ((g + pair) & 1) + ((step + pair) & 1);
                if (p == 3) __builtin_amdgcn_s_setprio(3);
                else if (p == 2) __builtin_amdgcn_s_setprio(2);
                else if (p == 1) __builtin_amdgcn_s_setprio(1);
                else __builtin_amdgcn_s_setprio(0);
            }
            // Lane values are formed per layer from a thread index hidden from
            // the optimiser: hoisted out of the loops they would be spilled, and
            // a spill reload waits for the K/V loads in flight.
            int tid = int(threadIdx.x);
            asm volatile("" : "+v"(tid));
            const int grp = tid / LPK, d0 = (tid % LPK) * VEC;
            // Row-order word index of this lane's dims d0 + e: at0 + (e % NW) *
            // 64 + e / NW, as d0 is a multiple of VEC and VEC one of NW.
            const uint32_t at0 = uint32_t(row_of<NW>(h * HDP + d0));
            float *kl = a.kc + size_t(l) * a.layer_elems + slab, *vl = a.vc + size_t(l) * a.layer_elems + slab;
            // RoPE pairs of this lane's dims at pos, loading before anything
            // else of the layer so that they are in by the time q and k are.
            float2 rcs[VEC];
#pragma unroll
            for (int e = 0; e < VEC; ++e) rcs[e] = rope_pair(a.rope, pos, d0 + e, s.half);
            // The first NS rounds load into the ring, and the last two rounds
            // into registers, while the layer's meshes still run (the online
            // softmax takes rounds in any order).
            // Past layer 0, keys that fit two rounds load straight into
            // registers (no LDS ring to fill and read); layer 0's rounds load
            // before the previous step's logits and draw, which need the
            // registers, so they use the ring.  Either way the rounds are
            // folded in in the same order.
            const int nr = (pos + G * U - 1) / (G * U);
            const int ntail = l > 0 && nr <= 2 ? nr : min(max(nr - NS, 0), 2);
            const int nring = nr - ntail;
            // Layer 0's first rounds were issued at the end of the previous
            // step (below), before its logits and draw.
            if (l > 0 || step == 0)
                for (int r = 0; r < min(NS, nring); ++r) ring.issue(kl, vl, r, pos, tid, a.mall_keep);
            R last, last2;
            if ((nring + 1) * G * U > a.mall_keep) {
                if (ntail > 0) last.load_nt(kl, vl, nring * G * U, pos);
                if (ntail > 1) last2.load_nt(kl, vl, (nring + 1) * G * U, pos);
            } else {
                if (ntail > 0) last.load(kl, vl, nring * G * U, pos);
                if (ntail > 1) last2.load(kl, vl, (nring + 1) * G * U, pos);
            }
            float qr[VEC], kn[VEC], vn[VEC];
            if (l == 0) {
                typedef __attribute__((address_space(1))) const float gfloat;
                gfloat *t0 = (gfloat *)opaque(a.q0) + size_t(tok) * 3 * W + at0;
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    const uint32_t o = (e % NW) * 64 + e / NW;
                    qr[e] = t0[o];
                    kn[e] = t0[W + o];
                    vn[e] = t0[2 * W + o];
                }
            } else {
                // Wave 0 takes the head's q, k and v, one dim of each per lane
                // (3 words a lane), and hands them to every lane group in LDS
                // (the mesh exchange buffer, which attention workgroups use
                // otherwise only for a near-tie draw, after the layers).
                static_assert(3 * HDP <= 2 * W && HDP <= 64, "q, k and v of a head in the exchange buffer");
                float *qkvs = m.xch;
                if (tid < 64) {
                    const int d = min(tid, HDP - 1);
                    const uint32_t o = uint32_t(row_of<NW>(h * HDP + d));
                    const uint64_t *qw = opaque(xc.qkv(g, 0)), *kw = opaque(xc.qkv(g, 1)), *vw = opaque(xc.qkv(g, 2));
                    float t[3];
                    xc.template take<3>([&](int i) { return (i == 0 ? qw : (i == 1 ? kw : vw)) + o; }, g + 1, t,
                                        a.abort);
                    if (tid < HDP) {
                        qkvs[d] = t[0];
                        qkvs[HDP + d] = t[1];
                        qkvs[2 * HDP + d] = t[2];
                    }
                }
                __syncthreads();
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    qr[e] = qkvs[d0 + e];
                    kn[e] = qkvs[HDP + d0 + e];
                    vn[e] = qkvs[2 * HDP + d0 + e];
                }
            }
            // QK-norm and RoPE of this head's query and key (the teams and
            // the layer-0 table give them before both).
            // The query carries the score scale (log2(e) / sqrt(hd)), so the
            // scores below need no multiply.
            lane_qk_rope<LPK, VEC>(qr, d0, rcs, s, a.scale_log2);
            lane_qk_rope<LPK, VEC>(kn, d0, rcs, s);
            const uint64_t t_ready = trace_time(a);
            S st;
            {
                // The current token's key first: on the fresh state folding
                // it in is an initialisation (m its score, l = 1, acc its
                // value row), done with selects for lane group 0, which holds
                // it, so no branch splits the rounds that follow.
                float sc = 0.0f;
#pragma unroll
                for (int e = 0; e < VEC; ++e) sc = fmaf(qr[e], kn[e], sc);
                sc = group_sum<LPK>(sc);
                const bool mine = grp == 0;
                st.m = mine ? sc : -INFINITY;
                st.l = mine ? 1.0f : 0.0f;
#pragma unroll
                for (int e = 0; e < VEC; ++e) st.acc[e] = mine ? vn[e] : 0.0f;
            }
            if (ntail > 1)
                st.add2(qr, last, nring * G * U, last2, (nring + 1) * G * U, pos, 1.0f);
            else if (ntail > 0)
                st.add(qr, last, nring * G * U, pos, 1.0f);
            if constexpr (NS == 2) {
                // Two rounds at a time: both slots are read, refilled and
                // folded in together.
                int r = 0;
                for (; r + 1 < nring; r += 2) {
                    ring.wait(0);
                    R c0, c1;
                    ring.read(r, c0, tid);
                    ring.read(r + 1, c1, tid);
                    if (r + 2 < nring) ring.issue(kl, vl, r + 2, pos, tid, a.mall_keep);
                    if (r + 3 < nring) ring.issue(kl, vl, r + 3, pos, tid, a.mall_keep);
                    st.add2(qr, c0, r * G * U, c1, (r + 1) * G * U, pos, 1.0f);
                }
                if (r < nring) {
                    ring.wait(0);
                    R cur;
                    ring.read(r, cur, tid);
                    st.add(qr, cur, r * G * U, pos, 1.0f);
                }
            } else {
                for (int r = 0; r < nring; ++r) {
                    ring.wait(min(NS - 1, nring - 1 - r));
                    R cur;
                    ring.read(r, cur, tid);
                    if (r + NS < nring) ring.issue(kl, vl, r + NS, pos, tid, a.mall_keep);
                    st.add(qr, cur, r * G * U, pos, 1.0f);
                }
            }
            // The merge borrows the LDS of the logits row and of the row
            // reductions, both idle during the layer loop; the value row goes
            // beside the merge scratch for the XSA below.
            static_assert(G * HDP <= kPersistVocab && 2 * G + HDP <= 8 * Ctx::SLOT, "merge scratch");
            float *vrow = m.red + 2 * G;
            if (grp == 0) {
#pragma unroll
                for (int e = 0; e < VEC; ++e) vrow[d0 + e] = vn[e];
            }
            // |v|^2 of the head from each lane group's copy of the value row,
            // ahead of the merge.
            float vsq = 0.0f;
#pragma unroll
            for (int e = 0; e < VEC; ++e) vsq = fmaf(vn[e], vn[e], vsq);
            const float iv = rsqrtf(fmaxf(group_sum<LPK>(vsq), kXsaFloor));
            const float yd = st.merge_wave0(m.red, m.red + G, m.row);
            if (tid < 64) {
                // XSA of the head (reference.rs:577-603): y - (y.u)u with
                // u = v / max(|v|, eps), in wave 0, one dim per lane.
                const int d = tid;
                const float vd = d < HDP ? vrow[d] : 0.0f;
                const float yv = wave_sum(yd * vd);
                if (d < HDP) xc.put(xc.y() + row_of<NW>(h * HDP + d), yd - (yv * iv) * (vd * iv), g + 1);
            }
            // The key and value rows go to the cache for later steps only
            // now: stored before the ring's last wait, which waits for every
            // vector-memory operation, they would hold it up.
            if (grp == 0) {
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    kl[size_t(pos) * HDP + d0 + e] = kn[e];
                    vl[size_t(pos) * HDP + d0 + e] = vn[e];
                }
            }
            __syncthreads();  // the merge scratch is free again
            trace_store(a, xc.row, step, l, 0, t_ready);
            trace_mark(a, xc.row, step, l, 1);
        }
        // This block's logits from the published final row.  The thread
        // index is hidden from the optimiser so the lane arithmetic is formed
        // here, not hoisted out of the step loop to occupy registers through
        // the attention.
        int tid = int(threadIdx.x);
        asm volatile("" : "+v"(tid));
        if (step + 1 < a.steps) {
            // The next step's layer-0 ring rounds depend on no token: they
            // load during the logits and the draw (which wait for them, as
            // loads complete in order, long after they have landed) instead
            // of after the draw.  The ring is idle until then.
            const int p1 = pos + 1, nr1 = (p1 + G * U - 1) / (G * U);
            const int nring1 = nr1 - min(max(nr1 - NS, 0), 2);
            const float *kl0 = a.kc + slab, *vl0 = a.vc + slab;
            for (int r = 0; r < min(NS, nring1); ++r) ring.issue(kl0, vl0, r, p1, tid, a.mall_keep);
        }
        const Ctx c(m.xch, m.red, tid);
        persistent_head_logits<NW, CPL, GL>(a, c, xc, step, 3 + h, m);
        trace_mark(a, xc.row, step, L, 1);
        if (step + 1 < a.steps) tok = draw_token<false>(a, xc, step, rng, m, nullptr);
    }
}

// Role of the k-th of the K = Q * R workgroups of an XCD, as (sequence q of
// the XCD's Q, role r of R = 3 + H).  The dispatcher gives each of the XCD's C
// CUs one workgroup in order, then puts workgroup C + p beside workgroup p
// (two fit per CU): the first P = K - C share a CU with a later one.  Those
// pairs are attention workgroups, a head of one sequence beside the same
// head of another, and the mesh teams, whose phase is the longer one on the
// chain, keep a CU to themselves.  (Measured on config 3 at batch 32: 59.5 us
// per step, against 62.3 with pairs in plain order and 61.7 with each team
// beside a head of its own sequence.)  Of a pair, the workgroup dispatched
// first runs faster (the wave scheduler favours older waves): sequences 0 and
// 2 of an XCD, always first, finish the 512-step launch of config 3 ~11 %
// before sequences 1 and 3.  Mixing the two places within each sequence was
// slower still (518k against 538k tokens/s): a sequence then waits every
// layer for its slowest head.  The paired workgroups instead take turns at the
// front by wave priority (persistent_attention), which narrows the gap.  Any
// other placement only costs speed: every role of a sequence stays on one
// XCD, and the map is a bijection of [0, K).  `pair` is 1 for the first
// workgroup of a pair, 2 for the second and 0 for one that has its CU alone.
__host__ __device__ inline void persistent_role(int k, int K, int C, int R, int &q, int &r, int &pair) {
    const int P = K - C, Q = K / R, H = R - 3;
    pair = 0;
    if (P <= 0 || 2 * P > Q * H || Q < 2 || C < P) {
        q = k / R;
        r = k % R;
        return;
    }
    // Paired slots take heads in head-major order, (q, h) = (i % Q, i / Q):
    // slot p the 2p-th, slot C + p the next, of another sequence.
    auto head_at = [&](int i, int &qq, int &rr) {
        qq = i % Q;
        rr = 3 + i / Q;
    };
    if (k < P) {
        head_at(2 * k, q, r);
        pair = 1;
        return;
    }
    if (k >= C && k < C + P) {
        head_at(2 * (k - C) + 1, q, r);
        pair = 2;
        return;
    }
    // The other roles in (q, r) order over the remaining slots.
    int o = k < C ? k - P : k - 2 * P;
    for (int qq = 0; qq < Q; ++qq)
        for (int rr = 0; rr < R; ++rr) {
            if (rr >= 3 && (rr - 3) * Q + qq < 2 * P) continue;  // a paired head
            if (o-- == 0) {
                q = qq;
                r = rr;
                return;
            }
        }
    q = Q;  // not reached for k < K
    r = 0;
}

// Blocks [0, 3*batch): mesh teams (sequence, team); then (sequence, head)
// attention blocks.  Needs every block resident at once (see above).
template <int NW, int CPL, int GL, int DEPTH, int HDP>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2)))
persistent_decode_kernel(PersistArgs a) {
    constexpr int W = 64 * NW * CPL;
    __shared__ float xch[2 * W];
    __shared__ float red[8 * RowCtx<NW, CPL, GL>::SLOT];
    __shared__ __align__(16) float xn[W];
    __shared__ __align__(16) float row[kPersistVocab];
    using Ring = PersistRing<NW, CPL, GL, HDP>;
    __shared__ __align__(16) float ring[KvRing<HDP, NW, Ring::UL, Ring::NS>::SLOT * Ring::NS];
    __shared__ uint64_t exp_tab[32];
    stage_exp_table(exp_tab);  // the teams' first barrier comes long before their first draw
    const PersistLds m{xch, red, xn, row, ring, exp_tab, KvRing<HDP, NW, Ring::UL, Ring::NS>::SLOT * Ring::NS};
    // Workgroup i runs on XCD i % 8 when the dispatcher deals workgroups out
    // round-robin, as it does on MI355X: the 3 + H workgroups of sequence
    // x + 8q are workgroups x + 8k of XCD x, k given by persistent_role.  (The
    // handshake checks it; any other placement only costs speed.)
    const int R = 3 + a.s.H, x = int(blockIdx.x) % 8, k = int(blockIdx.x) / 8;
    int q, r, pair;
    persistent_role(k, int(gridDim.x) / 8, a.xcd_cus, R, q, r, pair);
    const int b = x + 8 * q;
    if (b >= a.batch) return;
    const int trow = r < 3 ? 3 * b + r : 3 * a.batch + b * a.s.H + (r - 3);
    const PersistXch<false> far(a, b, trow);
    PersistStart st0;
    st0.len = a.len[b];
    st0.tok = a.tokens[size_t(b) * a.tok_stride + st0.len - 1];
    st0.rng = a.rng[b];
    auto run = [&](const auto &xc) {
        if (r < 3)
            persistent_team<NW, CPL, GL, DEPTH, HDP>(a, b, r, m, xc, st0);
        else
            persistent_attention<NW, CPL, GL, DEPTH, HDP>(a, b, r - 3, m, xc, pair, st0);
    };
    if (!a.agent_scope && persistent_handshake(a, far, r))
        run(PersistXch<true>(a, b, trow));
    else
        run(far);
}

// Layer-0 table: row (token v, team t) is team t's mesh of block 0 on the
// RMS-normalised token vector E[v], before QK-norm and RoPE, with the row
// meshes' arithmetic (log2(e)-scaled carry) that a persistent mesh team uses.
template <int NW, int CPL, int GL, int DEPTH>
__global__ void __launch_bounds__(64 * NW)
layer0_kernel(Shape s, const float *__restrict__ E, const float *__restrict__ w, size_t block0, float *q0) {
    using Ctx = RowCtx<NW, CPL, GL>;
    constexpr int W = Ctx::W;
    constexpr bool FIXED = DEPTH > 0;
    constexpr int D = FIXED ? DEPTH : 1;
    __shared__ float xch[2 * W];
    __shared__ float red[8 * Ctx::SLOT];
    Ctx c(xch, red);
    const int v = int(blockIdx.x) / 3, team = int(blockIdx.x) % 3;
    const float *wm = w + block0 + size_t(team) * 2 * W * s.A;
    float2 wr[D][CPL];
    load_block_weights<NW, CPL, GL, D>(wr, wm, FIXED, c.lane, c.wave);
    float x[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) x[j] = E[size_t(v) * W + c.ridx(j)];
    const float inv = row_inv_rms(c, x, 3) * kLog2e;
    float n[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) n[j] = x[j] * inv;
    row_run_mesh(c, n, wr, wm, s.A, s, FIXED);
#pragma unroll
    for (int j = 0; j < CPL; ++j) q0[(size_t(v) * 3 + team) * W + c.ridx(j)] = n[j] * kLn2;
}

// One workgroup per token row (reference.rs:130-149 with gpu.rs:1261-1333's
// arithmetic: scale = radius / max(|row|, 1e-12)).
__global__ void __launch_bounds__(kThreads)
embedding_geometry_kernel(float *__restrict__ E, const float *__restrict__ codes, int W, float radius,
                          int normalize, int keep) {
    __shared__ float red[kThreads / 64];
    float *row = E + size_t(blockIdx.x) * W;
    const float *code = codes + size_t(blockIdx.x) * W;
    float scale = 1.0f;
    if (normalize) {
        float a = 0.0f;
        for (int c = threadIdx.x; c < W; c += blockDim.x) a = fmaf(row[c], row[c], a);
        a = wave_sum(a);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = a;
        __syncthreads();
        float squares = 0.0f;
        for (int w = 0; w < int(blockDim.x) / 64; ++w) squares += red[w];
        scale = radius / fmaxf(sqrtf(squares), 1e-12f);
    }
    for (int c = threadIdx.x; c < W; c += blockDim.x) row[c] = c < keep ? code[c] : row[c] * scale;
}

__global__ void __launch_bounds__(kThreads)
transpose_kernel(const float *__restrict__ E, float *__restrict__ Et, int V, int Vp, int W) {
    __shared__ float tile[32][33];
    const int t0 = blockIdx.x * 32, c0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int k = ty; k < 32; k += 8) {
        const int t = t0 + k, c = c0 + tx;
        if (t < V && c < W) tile[k][tx] = E[size_t(t) * W + c];
    }
    __syncthreads();
    for (int k = ty; k < 32; k += 8) {
        const int c = c0 + k, t = t0 + tx;
        if (c < W && t < Vp) Et[size_t(c) * Vp + t] = t < V ? tile[tx][k] : 0.0f;
    }
}

// out = mesh(in) for rows x W with one team (the embedding table from codes;
// runs once per weight upload, so its weights are read from global memory).
template <int CPT>
__global__ void __launch_bounds__(256)
mesh_rows_kernel(Shape s, const float *__restrict__ in, float *__restrict__ out, int rows,
                 const float *__restrict__ w, int depth, int rpw) {
    extern __shared__ __align__(16) char smem[];
    LdsCarve lds{smem};
    const int W = s.W, T = blockDim.x;
    const size_t n = mesh_buffer_floats(W, rpw, CPT * T, 0);
    float *A = lds.take<float>(n);
    float *B = lds.take<float>(n);
    float *C = lds.take<float>(n);
    const int r0 = blockIdx.x * rpw, nr = min(rpw, rows - r0);
    for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) A[idx] = in[size_t(r0) * W + idx];
    __syncthreads();
    const float *res = mesh_team<CPT>(A, B, C, nr, s, reinterpret_cast<const float2 *>(w), depth, threadIdx.x, T,
                                      true);
    for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) out[size_t(r0) * W + idx] = res[idx];
}

__global__ void __launch_bounds__(kThreads) expf_kernel(const float *__restrict__ x, float *__restrict__ y, size_t n) {
    __shared__ uint64_t tab[32];
    stage_exp_table(tab);
    __syncthreads();
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) y[i] = expf_rounded(x[i], tab);
}

__global__ void __launch_bounds__(kThreads)
calibration_copy_kernel(const float4 *__restrict__ src, float4 *__restrict__ dst, size_t n) {
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

template <int HDP>
void launch_decode_t(const Shape &s, const float *q, KvView kv, const int *len, int batch, int nsplit,
                     float *part, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
    const float scale_log2 = float(1.4426950408889634 / std::sqrt(double(s.hd)));
    dim3 grid(nsplit * batch, s.H);
    if (start || stop) {
        // The events take the dispatch's own begin and end timestamps.
        hipExtLaunchKernelGGL(attn_decode_kernel<HDP>, grid, dim3(DecodeCfg<HDP>::THREADS), 0, stream, start,
                              stop, 0, s, q, kv, len, nsplit, part, scale_log2);
    } else {
        hipLaunchKernelGGL(attn_decode_kernel<HDP>, grid, dim3(DecodeCfg<HDP>::THREADS), 0, stream, s, q, kv,
                           len, nsplit, part, scale_log2);
    }
    HIP_LAUNCH_CHECK();
}

template <int HDP>
void launch_prefill_t(const Shape &s, const float *q, KvView kv, int nseq, int rows_per_seq, float *y,
                      hipStream_t stream) {
    const float scale_log2 = float(1.4426950408889634 / std::sqrt(double(s.hd)));
    const int ntiles = (rows_per_seq + PrefillCfg<HDP>::QT - 1) / PrefillCfg<HDP>::QT;
    dim3 grid(ntiles * nseq, s.H);
    hipLaunchKernelGGL(attn_prefill_kernel<HDP>, grid, dim3(kThreads), 0, stream, s, q, kv, rows_per_seq,
                       y, scale_log2);
    HIP_LAUNCH_CHECK();
}

template <class F>
void with_cpt(int cpt, F &&f) {
    switch (cpt) {
    case 1: return f(std::integral_constant<int, 1>{});
    case 2: return f(std::integral_constant<int, 2>{});
    case 4: return f(std::integral_constant<int, 4>{});
    case 8: return f(std::integral_constant<int, 8>{});
    default: return f(std::integral_constant<int, 16>{});
    }
}

}  // namespace

int team_threads(int W) { return std::min(256, (W + 63) / 64 * 64); }

int channels_per_thread(int W) {
    const int need = (W + team_threads(W) - 1) / team_threads(W);
    int cpt = 1;
    while (cpt < need) cpt <<= 1;
    return cpt;
}

size_t block_stage_bytes(const Shape &s, bool post, bool pre) {
    const size_t pf = post ? size_t(s.A + s.F) * s.W * 8 : 0, qkv = pre ? size_t(3 * s.A) * s.W * 8 : 0;
    return align16(std::max(pf, qkv));
}

size_t block_lds_bytes(const Shape &s, int rpw, int teams, bool staged, bool post, bool pre) {
    const int T = team_threads(s.W), cpt = channels_per_thread(s.W);
    const int cptw = teams == 3 ? (cpt + 2) / 3 : cpt;
    const size_t mesh = mesh_buffer_floats(s.W, rpw, cpt * T, cptw * teams * T) * 4;
    return (staged ? block_stage_bytes(s, post, pre) : 0) + align16(size_t(rpw) * s.W * 4) +
           (1 + 2 * size_t(teams)) * mesh + 2 * align16(size_t(rpw) * s.H * 4) + align16(size_t(rpw) * 4);
}

bool block_can_stage(const Shape &s, int teams, bool post, bool pre) {
    const int threads = teams * team_threads(s.W);
    return (!post || (s.A + s.F) * s.W <= kHoldPF * threads) && (!pre || 3 * s.A * s.W <= kHoldQKV * threads);
}

size_t mesh_lds_bytes(const Shape &s, int rpw) {
    return 3 * align16(mesh_buffer_floats(s.W, rpw, channels_per_thread(s.W) * team_threads(s.W), 0) * 4);
}

size_t head_lds_bytes(const Shape &s, int rt) {
    return align16(size_t(rt) * s.W * 4) + align16(size_t(kHeadGroups) * kHeadMaxRows * kHeadTokens * 4);
}

size_t head_sample_lds_bytes(const Shape &s) {
    if (s.V > kHeadSampleCap) return size_t(-1);
    return align16(size_t(s.W) * 4) + align16(kHeadSampleCap * 4) + align16(size_t(kHsGroups) * 64 * 16) +
           2 * align16(kHsThreads / 64 * 4) + align16((kHsThreads / 64 + 1) * 8) + align16(32 * 8);
}

void configure_lds(size_t max_bytes) {
    const int bytes = int(max_bytes);
    auto allow = [bytes](const void *f) {
        (void)hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    };
    for (int cpt : {1, 2, 4, 8, 16})
        with_cpt(cpt, [&](auto c) {
            allow(reinterpret_cast<const void *>(&block_kernel<decltype(c)::value, true, 3>));
            allow(reinterpret_cast<const void *>(&block_kernel<decltype(c)::value, false, 3>));
            allow(reinterpret_cast<const void *>(&block_kernel<decltype(c)::value, true, 1>));
            allow(reinterpret_cast<const void *>(&block_kernel<decltype(c)::value, false, 1>));
            allow(reinterpret_cast<const void *>(&mesh_rows_kernel<decltype(c)::value>));
        });
    allow(reinterpret_cast<const void *>(&head_kernel));
    allow(reinterpret_cast<const void *>(&head_sample_kernel));
}

void mesh_rows(const Shape &s, const float *in, float *out, int rows, const float *w, int depth, int rpw,
               hipStream_t stream) {
    dim3 grid((rows + rpw - 1) / rpw);
    with_cpt(channels_per_thread(s.W), [&](auto c) {
        hipLaunchKernelGGL(mesh_rows_kernel<decltype(c)::value>, grid, dim3(team_threads(s.W)),
                           mesh_lds_bytes(s, rpw), stream, s, in, out, rows, w, depth, rpw);
    });
    HIP_LAUNCH_CHECK();
}

void embedding_geometry(float *E, const float *codes, int V, int W, float radius, int normalize, int keep,
                        hipStream_t stream) {
    hipLaunchKernelGGL(embedding_geometry_kernel, dim3(V), dim3(kThreads), 0, stream, E, codes, W, radius, normalize,
                       keep);
    HIP_LAUNCH_CHECK();
}

void transpose(const float *E, float *Et, int V, int Vp, int W, hipStream_t stream) {
    dim3 grid((Vp + 31) / 32, (W + 31) / 32);
    hipLaunchKernelGGL(transpose_kernel, grid, dim3(kThreads), 0, stream, E, Et, V, Vp, W);
    HIP_LAUNCH_CHECK();
}

void block(const BlockArgs &a, bool staged, hipStream_t stream) {
    dim3 grid((a.ro.rows + a.rpw - 1) / a.rpw);
    const size_t lds = block_lds_bytes(a.s, a.rpw, a.teams, staged, a.wproj != nullptr, a.wq != nullptr);
    const dim3 threads(a.teams * team_threads(a.s.W));
    with_cpt(channels_per_thread(a.s.W), [&](auto c) {
        constexpr int C = decltype(c)::value;
        if (a.teams == 3) {
            if (staged) hipLaunchKernelGGL((block_kernel<C, true, 3>), grid, threads, lds, stream, a);
            else hipLaunchKernelGGL((block_kernel<C, false, 3>), grid, threads, lds, stream, a);
        } else {
            if (staged) hipLaunchKernelGGL((block_kernel<C, true, 1>), grid, threads, lds, stream, a);
            else hipLaunchKernelGGL((block_kernel<C, false, 1>), grid, threads, lds, stream, a);
        }
    });
    HIP_LAUNCH_CHECK();
}

bool block_decode_supported(const Shape &s) {
    return s.wshift >= 6 && s.W <= 1024 && s.hdshift >= 3;
}

void block_decode(const BlockArgs &a, hipStream_t stream) {
    const Shape &s = a.s;
    const dim3 grid(a.ro.rows), threads(kDecodeThreads);
    // Fixed-depth instantiations for the shipped configurations' shapes.
    const bool fixed = s.butterfly && s.A == s.F;
    if (fixed && s.W == 512 && s.hd == 64 && s.A == 9) {
        hipLaunchKernelGGL((block_decode_kernel<8, 64, 9>), grid, threads, 0, stream, a);
    } else if (fixed && s.W == 128 && s.hd == 32 && s.A == 7) {
        hipLaunchKernelGGL((block_decode_kernel<2, 32, 7>), grid, threads, 0, stream, a);
    } else {
        with_cpt(s.W / 64, [&](auto c) {
            constexpr int C = decltype(c)::value;
            switch (std::min(s.hd, 64)) {
            case 8: hipLaunchKernelGGL((block_decode_kernel<C, 8, 0>), grid, threads, 0, stream, a); break;
            case 16: hipLaunchKernelGGL((block_decode_kernel<C, 16, 0>), grid, threads, 0, stream, a); break;
            case 32: hipLaunchKernelGGL((block_decode_kernel<C, 32, 0>), grid, threads, 0, stream, a); break;
            default: hipLaunchKernelGGL((block_decode_kernel<C, 64, 0>), grid, threads, 0, stream, a); break;
            }
        });
    }
    HIP_LAUNCH_CHECK();
}

int row_waves(int W) { return W >= 256 ? 4 : 2; }

bool row_block_supported(const Shape &s) {
    if (s.wshift < 7 || s.wshift > 10) return false;
    const int nw = row_waves(s.W);
    if (s.hd % nw != 0) return false;
    const int gl = s.hd / nw;
    return gl == 8 || gl == 16 || gl == 32;
}

template <int NW, int CPL>
void launch_row_block(const BlockArgs &a, dim3 grid, hipStream_t stream) {
    const Shape &s = a.s;
    const dim3 threads(64 * NW);
    const bool fixed = s.butterfly && s.A == s.F;
    if constexpr (NW == 4 && CPL == 2) {
        if (fixed && s.A == 9 && s.hd == 64) {
            hipLaunchKernelGGL((row_block_kernel<4, 2, 16, 9>), grid, threads, 0, stream, a);
            return;
        }
    }
    if constexpr (NW == 2 && CPL == 1) {
        if (fixed && s.A == 7 && s.hd == 32) {
            hipLaunchKernelGGL((row_block_kernel<2, 1, 16, 7>), grid, threads, 0, stream, a);
            return;
        }
    }
    if constexpr (NW == 4 && CPL == 4) {
        if (fixed && s.A == 10 && s.hd == 64) {
            hipLaunchKernelGGL((row_block_kernel<4, 4, 16, 10>), grid, threads, 0, stream, a);
            return;
        }
    }
    switch (s.hd / NW) {
    case 8: hipLaunchKernelGGL((row_block_kernel<NW, CPL, 8, 0>), grid, threads, 0, stream, a); break;
    case 16: hipLaunchKernelGGL((row_block_kernel<NW, CPL, 16, 0>), grid, threads, 0, stream, a); break;
    default: hipLaunchKernelGGL((row_block_kernel<NW, CPL, 32, 0>), grid, threads, 0, stream, a); break;
    }
}

// Rows per workgroup of the fixed-depth row blocks: one, or more when the
// batch's workgroups (three per row with the Q/K/V meshes) would take more
// than one wave of one workgroup per CU (the kernels hold every mesh weight
// in registers, so one fits a CU).  MG_ROW_BATCH forces 1, 2 or 4.
int row_batch(int rows, int teams) {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
    }
    const char *e = std::getenv("MG_ROW_BATCH");
    if (e && *e) {
        const int f = std::atoi(e);
        if (f == 1 || f == 2 || f == 4) return f;
    }
    for (int rb : {1, 2})
        if (teams * ((rows + rb - 1) / rb) <= cus) return rb;
    return 4;
}

template <int NW, int CPL, int GL, int DEPTH>
void launch_row_block_rows(const BlockArgs &a, int teams, hipStream_t stream) {
    const int rb = row_batch(a.ro.rows, teams);
    const dim3 threads(64 * NW);
    const unsigned groups = unsigned((a.ro.rows + rb - 1) / rb);
    switch (rb) {
    case 1: hipLaunchKernelGGL((row_block_kernel<NW, CPL, GL, DEPTH>), dim3(a.ro.rows * teams), threads, 0, stream, a); break;
    case 2: hipLaunchKernelGGL((row_block_rows_kernel<NW, CPL, GL, DEPTH, 2>), dim3(groups * teams), threads, 0, stream, a); break;
    default: hipLaunchKernelGGL((row_block_rows_kernel<NW, CPL, GL, DEPTH, 4>), dim3(groups * teams), threads, 0, stream, a); break;
    }
}

void row_block(const BlockArgs &a, hipStream_t stream) {
    const int teams = a.wq != nullptr ? 3 : 1;
    const Shape &s = a.s;
    const bool fixed = s.butterfly && s.A == s.F && s.hd == 64;
    if (fixed && s.W == 512 && s.A == 9) {
        launch_row_block_rows<4, 2, 16, 9>(a, teams, stream);
        HIP_LAUNCH_CHECK();
        return;
    }
    if (fixed && s.W == 1024 && s.A == 10) {
        launch_row_block_rows<4, 4, 16, 10>(a, teams, stream);
        HIP_LAUNCH_CHECK();
        return;
    }
    const dim3 grid(a.ro.rows * teams);
    switch (a.s.W) {
    case 128: launch_row_block<2, 1>(a, grid, stream); break;
    case 256: launch_row_block<4, 1>(a, grid, stream); break;
    case 512: launch_row_block<4, 2>(a, grid, stream); break;
    default: launch_row_block<4, 4>(a, grid, stream); break;
    }
    HIP_LAUNCH_CHECK();
}

void row_order(const float *src, float *dst, int rows, int W, bool pairs, hipStream_t stream) {
    const size_t n = size_t(rows) * W;
    const unsigned blocks = unsigned(std::min<size_t>((n + kThreads - 1) / kThreads, 4096));
    if (pairs)
        hipLaunchKernelGGL(row_order_kernel<float2>, dim3(blocks), dim3(kThreads), 0, stream,
                           reinterpret_cast<const float2 *>(src), reinterpret_cast<float2 *>(dst), rows, W,
                           row_waves(W));
    else
        hipLaunchKernelGGL(row_order_kernel<float>, dim3(blocks), dim3(kThreads), 0, stream, src, dst, rows, W,
                           row_waves(W));
    HIP_LAUNCH_CHECK();
}

// The persistent kernel instantiation for a shape, or nullptr.
// Calls f(NW, CPL, GL, DEPTH, HDP) (integral constants) with the persistent
// kernel variant for the shape; false when the shape has none.
template <int NW, int CPL, int HDP, class F>
void persistent_depth(const Shape &s, F &&f) {
    using std::integral_constant;
    constexpr int GL = HDP / NW;
    const bool fixed = s.butterfly && s.A == s.F;
    if constexpr (NW == 4 && CPL == 2 && HDP == 64) {
        if (fixed && s.A == 9)
            return f(integral_constant<int, 4>{}, integral_constant<int, 2>{}, integral_constant<int, 16>{},
                     integral_constant<int, 9>{}, integral_constant<int, 64>{});
    }
    if constexpr (NW == 2 && CPL == 1 && HDP == 32) {
        if (fixed && s.A == 7)
            return f(integral_constant<int, 2>{}, integral_constant<int, 1>{}, integral_constant<int, 16>{},
                     integral_constant<int, 7>{}, integral_constant<int, 32>{});
    }
    f(integral_constant<int, NW>{}, integral_constant<int, CPL>{}, integral_constant<int, GL>{},
      integral_constant<int, 0>{}, integral_constant<int, HDP>{});
}

template <class F>
bool persistent_visit(const Shape &s, F &&f) {
    if (!row_block_supported(s) || s.hd != s.hdp || s.V > kPersistVocab || s.V > 2 * s.W) return false;
    const int nw = row_waves(s.W);
    if (s.hd / nw != 8 && s.hd / nw != 16) return false;
    switch (s.W * 10000 + s.hd) {
    case 1280032: persistent_depth<2, 1, 32>(s, f); return true;
    case 2560032: persistent_depth<4, 1, 32>(s, f); return true;
    case 2560064: persistent_depth<4, 1, 64>(s, f); return true;
    case 5120032: persistent_depth<4, 2, 32>(s, f); return true;
    case 5120064: persistent_depth<4, 2, 64>(s, f); return true;
    case 10240064: persistent_depth<4, 4, 64>(s, f); return true;
    default: return false;
    }
}

const void *persistent_kernel(const Shape &s) {
    const void *k = nullptr;
    persistent_visit(s, [&](auto nw, auto cpl, auto gl, auto depth, auto hdp) {
        k = reinterpret_cast<const void *>(
            &persistent_decode_kernel<decltype(nw)::value, decltype(cpl)::value, decltype(gl)::value,
                                      decltype(depth)::value, decltype(hdp)::value>);
    });
    return k;
}

int persistent_blocks(const Shape &s, int batch) { return 8 * (3 + s.H) * ((batch + 7) / 8); }

size_t persistent_exchange_words(const Shape &s) { return (size_t(8) * s.W + s.V + 3 + s.H + 31) / 32 * 32; }

bool persistent_fits(const Shape &s, int batch, int device) {
    const void *f = persistent_kernel(s);
    if (!f) return false;
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, 64 * row_waves(s.W), 0) != hipSuccess) return false;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return false;
    return persistent_blocks(s, batch) <= per_cu * cus;
}

int kv_keep_rows(const Shape &s, int batch, int layers) {
    const char *env = std::getenv("MG_MALL_BYTES");
    const double cache = env && *env ? std::atof(env) : 256.0 * 1024 * 1024;
    const double per_row = double(batch) * layers * s.H * 2.0 * s.hdp * 4.0;
    if (per_row <= 0.0) return 1 << 30;
    const double rows = 0.8 * cache / per_row;
    return rows >= double(1 << 30) ? 1 << 30 : int(rows);
}

hipError_t persistent_decode(const PersistArgs &a, hipStream_t stream) {
    const void *f = persistent_kernel(a.s);
    if (!f) return hipErrorInvalidValue;
    PersistArgs args = a;
    args.scale_log2 = float(1.4426950408889634 / std::sqrt(double(a.s.hd)));
    int device = 0, cus = 0;
    if (hipGetDevice(&device) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
        return hipErrorInvalidDevice;
    args.xcd_cus = cus / 8;
    if (args.wait_ticks == 0) args.wait_ticks = kWaitTicks;
    void *params[] = {&args};
    return hipLaunchKernel(f, dim3(persistent_blocks(a.s, a.batch)), dim3(64 * row_waves(a.s.W)), params, 0, stream);
}

size_t persistent_layer0_floats(const Shape &s) { return size_t(s.V) * 3 * s.W; }

bool persistent_layer0(const Shape &s, const float *E, const float *w, size_t block0, float *q0, hipStream_t stream) {
    return persistent_visit(s, [&](auto nw, auto cpl, auto gl, auto depth, auto hdp) {
        constexpr int NW = decltype(nw)::value;
        hipLaunchKernelGGL((layer0_kernel<NW, decltype(cpl)::value, decltype(gl)::value, decltype(depth)::value>),
                           dim3(3 * s.V), dim3(64 * NW), 0, stream, s, E, w, block0, q0);
        HIP_LAUNCH_CHECK();
        (void)hdp;
    });
}

void attn_decode(const Shape &s, const float *q, KvView kv, const int *len, int batch, int nsplit, float *part,
                 hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
    switch (s.hdp) {
    case 2: return launch_decode_t<2>(s, q, kv, len, batch, nsplit, part, stream, start, stop);
    case 4: return launch_decode_t<4>(s, q, kv, len, batch, nsplit, part, stream, start, stop);
    case 8: return launch_decode_t<8>(s, q, kv, len, batch, nsplit, part, stream, start, stop);
    case 16: return launch_decode_t<16>(s, q, kv, len, batch, nsplit, part, stream, start, stop);
    case 32: return launch_decode_t<32>(s, q, kv, len, batch, nsplit, part, stream, start, stop);
    case 64: return launch_decode_t<64>(s, q, kv, len, batch, nsplit, part, stream, start, stop);
    case 128: return launch_decode_t<128>(s, q, kv, len, batch, nsplit, part, stream, start, stop);
    case 256: return launch_decode_t<256>(s, q, kv, len, batch, nsplit, part, stream, start, stop);
    case 512: return launch_decode_t<512>(s, q, kv, len, batch, nsplit, part, stream, start, stop);
    case 1024: return launch_decode_t<1024>(s, q, kv, len, batch, nsplit, part, stream, start, stop);
    case 2048: return launch_decode_t<2048>(s, q, kv, len, batch, nsplit, part, stream, start, stop);
    case 4096: return launch_decode_t<4096>(s, q, kv, len, batch, nsplit, part, stream, start, stop);
    default: break;
    }
}

void attn_prefill(const Shape &s, const float *q, KvView kv, int nseq, int rows_per_seq, float *y,
                  hipStream_t stream) {
    switch (s.hdp) {
    case 2: return launch_prefill_t<2>(s, q, kv, nseq, rows_per_seq, y, stream);
    case 4: return launch_prefill_t<4>(s, q, kv, nseq, rows_per_seq, y, stream);
    case 8: return launch_prefill_t<8>(s, q, kv, nseq, rows_per_seq, y, stream);
    case 16: return launch_prefill_t<16>(s, q, kv, nseq, rows_per_seq, y, stream);
    case 32: return launch_prefill_t<32>(s, q, kv, nseq, rows_per_seq, y, stream);
    case 64: return launch_prefill_t<64>(s, q, kv, nseq, rows_per_seq, y, stream);
    case 128: return launch_prefill_t<128>(s, q, kv, nseq, rows_per_seq, y, stream);
    case 256: return launch_prefill_t<256>(s, q, kv, nseq, rows_per_seq, y, stream);
    case 512: return launch_prefill_t<512>(s, q, kv, nseq, rows_per_seq, y, stream);
    case 1024: return launch_prefill_t<1024>(s, q, kv, nseq, rows_per_seq, y, stream);
    case 2048: return launch_prefill_t<2048>(s, q, kv, nseq, rows_per_seq, y, stream);
    case 4096: return launch_prefill_t<4096>(s, q, kv, nseq, rows_per_seq, y, stream);
    default: break;
    }
}

void head(const Shape &s, const float *xn, int nrows, int row_mul, int row_add, const float *Et, int Vp,
          float *logits, int rt, hipStream_t stream) {
    dim3 grid((s.V + kHeadTokens - 1) / kHeadTokens, (nrows + rt - 1) / rt);
    hipLaunchKernelGGL(head_kernel, grid, dim3(kThreads), head_lds_bytes(s, rt), stream, s, xn, nrows, row_mul,
                       row_add, Et, Vp, logits, rt);
    HIP_LAUNCH_CHECK();
}

void head_sample(const Shape &s, const float *xn, int batch, const float *Et, int Vp, float *logits,
                 float temperature, uint64_t *rng, uint32_t *tokens, int tok_stride, int *len, int *flags,
                 hipStream_t stream) {
    hipLaunchKernelGGL(head_sample_kernel, dim3(batch), dim3(kHsThreads), head_sample_lds_bytes(s), stream, s, xn,
                       Et, Vp, logits, temperature, rng, tokens, tok_stride, len, flags);
    HIP_LAUNCH_CHECK();
}

void device_expf(const float *x, float *y, size_t n, hipStream_t stream) {
    const int blocks = int(std::min<size_t>((n + kThreads - 1) / kThreads, 4096));
    if (blocks > 0) hipLaunchKernelGGL(expf_kernel, dim3(blocks), dim3(kThreads), 0, stream, x, y, n);
    HIP_LAUNCH_CHECK();
}

void calibration_copy(const float4 *src, float4 *dst, size_t n, hipStream_t stream) {
    const size_t blocks = std::min<size_t>((n + kThreads - 1) / kThreads, 256 * 16);
    hipLaunchKernelGGL(calibration_copy_kernel, dim3(unsigned(std::max<size_t>(blocks, 1))), dim3(kThreads), 0,
                       stream, src, dst, n);
    HIP_LAUNCH_CHECK();
}

void sample(int V, int batch, const float *logits, float temperature, uint64_t *rng, uint32_t *tokens,
            int tok_stride, int *len, int *flags, hipStream_t stream) {
    if (V <= 256)
        hipLaunchKernelGGL(wave_sample_kernel<4>, dim3(batch), dim3(64), 0, stream, logits, V, temperature, rng,
                           tokens, tok_stride, len, flags);
    else if (V <= kWaveSampleVocab)
        hipLaunchKernelGGL(wave_sample_kernel<kWaveSampleVocab / 64>, dim3(batch), dim3(64), 0, stream, logits, V,
                           temperature, rng, tokens, tok_stride, len, flags);
    else
        hipLaunchKernelGGL(sample_kernel, dim3(batch), dim3(kThreads), 0, stream, logits, V, temperature, rng, tokens,
                           tok_stride, len, flags);
    HIP_LAUNCH_CHECK();
}

}  // namespace meshgpt::kern
