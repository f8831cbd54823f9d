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
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>

#include "kernels.hpp"

namespace meshgpt::kern {
namespace {

constexpr float kRmsEps = 1e-5f;  // src/gpt/mod.rs:38
// (f64(1e-12f))^2 rounded to f32: the XSA norm floor of reference.rs:591
constexpr float kXsaFloor = float(double(1e-12f) * double(1e-12f));

#define HIP_LAUNCH_CHECK() (void)hipGetLastError()

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ int wave_min_int(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ int wave_or_int(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v |= __shfl_xor(v, o, 64);
    return v;
}

// ELU of reference.rs:325-332 (expm1 for negative inputs).
__device__ __forceinline__ float elu(float z) { return z >= 0.0f ? z : expm1f(z); }

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
        if (lane == 0) inv[sg] = 1.0f / sqrtf(acc * scale + kRmsEps);
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

// The [self, partner] weights of a thread's CPT channels for the next three
// layers of a mesh; a slot is refilled three layers ahead of its use.
template <int CPT>
struct MeshRing {
    float2 w[3][CPT];
};

template <int CPT>
__device__ __forceinline__ void ring_load(float2 (&slot)[CPT], const float2 *__restrict__ wp, int layer, int W,
                                          int tt, int T) {
#pragma unroll
    for (int k = 0; k < CPT; ++k) slot[k] = wp[size_t(layer) * W + min(tt + k * T, W - 1)];
}

template <int CPT>
__device__ __forceinline__ void ring_prime(MeshRing<CPT> &ring, const float *w, int depth, int W, int tt, int T,
                                           bool active) {
    if (!active) return;
    const float2 *wp = reinterpret_cast<const float2 *>(w);
#pragma unroll
    for (int u = 0; u < 3; ++u)
        if (u < depth) ring_load<CPT>(ring.w[u], wp, u, W, tt, T);
}

// A mesh stack (reference.rs:422-453) over the nr rows in LDS `in`, computed by
// the team of T threads whose `active` flag is set (thread tt of the team owns
// channels tt + k*T).  Every thread of the block calls it: one barrier per
// layer.  Layer outputs alternate between a and b; returns the last one.
template <int CPT>
__device__ const float *mesh_team(MeshRing<CPT> &ring, const float *in, float *a, float *b, int nr,
                                  const Shape &s, const float *__restrict__ w, int depth, int tt, int T,
                                  bool active) {
    const int W = s.W;
    const float2 *wp = reinterpret_cast<const float2 *>(w);
    const float *cur = in;
    float *nxt = a;
    for (int l0 = 0; l0 < depth; l0 += 3) {
#pragma unroll
        for (int u = 0; u < 3; ++u) {
            const int l = l0 + u;
            if (l < depth) {
                if (active) {
                    const int st = s.butterfly ? (1 << (l % s.log2w)) : 1;
                    const bool last = l + 1 == depth;
#pragma unroll
                    for (int k = 0; k < CPT; ++k) {
                        const int c = tt + k * T;
                        if (c < W) {
                            int p = c + st;
                            if (p >= W) p -= W;
                            const float2 ww = ring.w[u][k];
                            for (int r = 0; r < nr; ++r) {
                                const float z = cur[r * W + c] * ww.x + cur[r * W + p] * ww.y;
                                nxt[r * W + c] = last ? z : elu(z);
                            }
                        }
                    }
                    if (l + 3 < depth) ring_load<CPT>(ring.w[u], wp, l + 3, W, tt, T);
                }
                __syncthreads();
                cur = nxt;
                nxt = nxt == a ? b : a;
            }
        }
    }
    return cur;
}

// Buffer holding the result of a depth-layer mesh_team run with (a, b).
__device__ __forceinline__ float *mesh_result(float *a, float *b, int depth) { return (depth & 1) ? a : b; }

// ------------------------------------------------------------ block kernel

// Post-attention half of block l-1 (reference.rs:194-216) fused with the
// pre-attention half of block l (reference.rs:164-193) for a tile of rows.
// Launch: one workgroup per `rpw` rows, teams x T threads.
template <int CPT>
__global__ void __launch_bounds__(768)
block_kernel(BlockArgs a) {
    extern __shared__ __align__(16) char smem[];
    LdsCarve lds{smem};
    const Shape &s = a.s;
    const int W = s.W, rpw = a.rpw;
    const int T = int(blockDim.x) / a.teams, team = int(threadIdx.x) / T, tt = int(threadIdx.x) - team * T;
    const bool post = a.wproj != nullptr, pre = a.wq != nullptr;
    float *X = lds.take<float>(size_t(rpw) * W);
    float *N = lds.take<float>(size_t(rpw) * W);
    // 2*teams ping-pong buffers of rpw rows each, addressed by index (no
    // pointer arrays: those would live in scratch memory).
    const size_t bstride = (size_t(rpw) * W * 4 + 15) / 16 * 4;
    float *bufs = lds.take<float>(bstride * 2 * a.teams);
    auto buf = [bufs, bstride](int i) { return bufs + size_t(i) * bstride; };
    float *inv1 = lds.take<float>(size_t(rpw) * s.H);
    float *inv2 = lds.take<float>(size_t(rpw) * s.H);
    float *rinv = lds.take<float>(size_t(rpw));
    float *wsplit = lds.take<float>(a.part ? size_t(rpw) * s.H * a.nsplit : 0);
    const int r0 = blockIdx.x * rpw, nr = min(rpw, a.ro.rows - r0);

    // Weight rings first: their loads overlap the row loads below.
    MeshRing<CPT> rp, rf, rq;
    if (post) {
        ring_prime<CPT>(rp, a.wproj, s.A, W, tt, T, team == 0);
        ring_prime<CPT>(rf, a.wffn, s.F, W, tt, T, team == 0);
    }
    const float *wmine = team == 0 ? a.wq : (team == 1 ? a.wk : a.wv);
    if (pre) ring_prime<CPT>(rq, a.teams == 3 ? wmine : a.wq, s.A, W, tt, T, true);

    // Residual rows: the token vectors (first block) or x.
    for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) {
        int r, c;
        split_row(idx, s, r, c);
        const int row = r0 + r;
        float v;
        if (a.embed) {
            int seq, pos;
            row_position(a.ro, row, seq, pos);
            const uint32_t tok = a.ro.tokens[size_t(seq) * a.ro.tok_stride + a.ro.tok_offset + pos];
            v = a.E[size_t(tok) * W + c];
            a.x[size_t(row) * W + c] = v;
        } else {
            v = a.x[size_t(row) * W + c];
        }
        X[idx] = v;
    }

    if (post) {
        const int stride = s.hdp + 2;
        float *Y = buf(0), *Vs = buf(1);
        if (a.part) {
            // Split combine, step 1: every (row, head, split) softmax maximum in one
            // pass, then per (row, head) the weights exp2(m_s - M) / L.
            const int hs = s.H * a.nsplit;
            for (int i = threadIdx.x; i < nr * hs; i += blockDim.x) {
                const int r = i / hs, rem = i - r * hs;
                int seq, pos;
                row_position(a.ro, r0 + r, seq, pos);
                wsplit[i] = a.part[(size_t(seq) * hs + rem) * stride + s.hdp];
            }
            __syncthreads();
            for (int i = threadIdx.x; i < nr * s.H; i += blockDim.x) {
                const int r = i / s.H, h = i - r * s.H;
                int seq, pos;
                row_position(a.ro, r0 + r, seq, pos);
                const float *pp = a.part + (size_t(seq * s.H + h) * a.nsplit) * stride;
                float *wv = wsplit + size_t(i) * a.nsplit;
                float M = -INFINITY;
                for (int k = 0; k < a.nsplit; ++k) M = fmaxf(M, wv[k]);
                float L = 0.0f;
                for (int k = 0; k < a.nsplit; ++k) {
                    wv[k] = exp2f(wv[k] - M);
                    L = fmaf(wv[k], pp[k * stride + s.hdp + 1], L);
                }
                const float il = 1.0f / L;
                for (int k = 0; k < a.nsplit; ++k) wv[k] *= il;
            }
            __syncthreads();
        }
        // Attention output y and the row's own value v.
        for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) {
            int r, c, h, d, seq, pos;
            split_row(idx, s, r, c);
            split_head(c, s, h, d);
            const int row = r0 + r;
            row_position(a.ro, row, seq, pos);
            float yval;
            if (a.part) {
                // Step 2: y = sum_s w_s acc_s with four splits' loads in flight.
                const float *pp = a.part + (size_t(seq * s.H + h) * a.nsplit) * stride + d;
                const float *wv = wsplit + size_t(r * s.H + h) * a.nsplit;
                float acc = 0.0f;
                int k = 0;
                for (; k + 4 <= a.nsplit; k += 4) {
                    const float a0 = pp[(k + 0) * stride], a1 = pp[(k + 1) * stride];
                    const float a2 = pp[(k + 2) * stride], a3 = pp[(k + 3) * stride];
                    acc = fmaf(wv[k], a0, acc);
                    acc = fmaf(wv[k + 1], a1, acc);
                    acc = fmaf(wv[k + 2], a2, acc);
                    acc = fmaf(wv[k + 3], a3, acc);
                }
                for (; k < a.nsplit; ++k) acc = fmaf(wv[k], pp[k * stride], acc);
                yval = acc;
            } else {
                yval = a.ybuf[size_t(row) * W + c];
            }
            Y[idx] = yval;
            Vs[idx] = a.kv_post.v[(size_t(seq * s.H + h) * a.kv_post.cap + pos) * s.hdp + d];
        }
        __syncthreads();
        // XSA (reference.rs:577-603): z = y - (y.u)u with u = v / max(|v|, eps).
        segment_dots(Y, Vs, nr * s.H, s.hd, inv1, inv2);
        __syncthreads();
        for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) {
            int r, c, h, d;
            split_row(idx, s, r, c);
            split_head(c, s, h, d);
            const int sg = r * s.H + h;
            const float iv = 1.0f / sqrtf(fmaxf(inv1[sg], kXsaFloor));
            Y[idx] = Y[idx] - (inv2[sg] * iv) * (Vs[idx] * iv);
        }
        __syncthreads();
        const float *proj = mesh_team<CPT>(rp, Y, buf(1), N, nr, s, a.wproj, s.A, tt, T, team == 0);
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
        const float *ffn = mesh_team<CPT>(rf, Nf, fa, fb, nr, s, a.wffn, s.F, tt, T, team == 0);
        for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) {
            int r, c;
            split_row(idx, s, r, c);
            const float v = X[idx] + ffn[idx];
            X[idx] = v;
            a.x[size_t(r0 + r) * W + c] = v;
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
    const float *res0, *res1, *res2;
    if (a.teams == 3) {
        mesh_team<CPT>(rq, N, buf(2 * team), buf(2 * team + 1), nr, s, wmine, s.A, tt, T, true);
        res0 = mesh_result(buf(0), buf(1), s.A);
        res1 = mesh_result(buf(2), buf(3), s.A);
        res2 = mesh_result(buf(4), buf(5), s.A);
    } else {
        // One team: Q's result is copied into X (free once x is normalised), K
        // stays in its buffer, and V alternates between the other buffer and N
        // (N is read only by V's first layer).
        const float *q = mesh_team<CPT>(rq, N, buf(0), buf(1), nr, s, a.wq, s.A, tt, T, true);
        for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) X[idx] = q[idx];
        __syncthreads();
        ring_prime<CPT>(rq, a.wk, s.A, W, tt, T, true);
        const float *k = mesh_team<CPT>(rq, N, buf(0), buf(1), nr, s, a.wk, s.A, tt, T, true);
        ring_prime<CPT>(rq, a.wv, s.A, W, tt, T, true);
        float *kres = const_cast<float *>(k);
        float *other = kres == buf(0) ? buf(1) : buf(0);
        const float *v = mesh_team<CPT>(rq, N, other, N, nr, s, a.wv, s.A, tt, T, true);
        res0 = X;
        res1 = kres;
        res2 = v;
    }
    // QK-Norm per head, split-half RoPE at each row's position, cache append.
    segment_inv_rms(res0, nr * s.H, s.hd, inv1);
    segment_inv_rms(res1, nr * s.H, s.hd, inv2);
    __syncthreads();
    const int pairs = s.H * s.half;
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

template <int HDP>
struct DecodeCfg {
    static constexpr int VEC = HDP <= 4 ? HDP : (HDP / 64 > 4 ? HDP / 64 : 4);  // dims per lane
    static constexpr int LPK = HDP / VEC;                                      // lanes per key (<= 64)
    static constexpr int THREADS = HDP >= 4096 ? 128 : 256;
    static constexpr int G = THREADS / LPK;                                    // key groups
    static constexpr int U = VEC >= 32 ? 1 : (VEC >= 16 ? 2 : (VEC >= 8 ? 4 : 8));  // keys per group per step
};

// Split-KV decode attention (reference.rs:510-554 for one query row).  Block
// (seq * nsplit + split, head) streams an equal share of the len[seq] keys of
// the cache; each group of LPK lanes owns one key at a time, so every K/V row
// is one coalesced VEC-wide load per lane, and U keys' loads are issued before
// any is consumed.  Scores live in the log2 domain.  An empty share writes the
// neutral partial (m = -inf, l = 0).
template <int HDP>
__global__ void __launch_bounds__(DecodeCfg<HDP>::THREADS)
attn_decode_kernel(Shape s, const float *__restrict__ q, KvView kv, const int *__restrict__ len, int nsplit,
                   float *__restrict__ part, float scale_log2) {
    using C = DecodeCfg<HDP>;
    constexpr int VEC = C::VEC, LPK = C::LPK, G = C::G, U = C::U;
    __shared__ float sm[G], sl[G];
    __shared__ __align__(16) float sacc[G * HDP];
    const int b = int(blockIdx.x) / nsplit, split = int(blockIdx.x) - b * nsplit, h = blockIdx.y;
    const int keys = len[b];
    const int chunk = (keys + nsplit - 1) / nsplit;
    const int start = split * chunk;
    const int end = min(start + chunk, keys);
    float *out = part + (size_t(b * s.H + h) * nsplit + split) * (HDP + 2);
    if (start >= end) {
        for (int d = threadIdx.x; d < HDP; d += blockDim.x) out[d] = 0.0f;
        if (threadIdx.x == 0) {
            out[HDP] = -INFINITY;
            out[HDP + 1] = 0.0f;
        }
        return;
    }
    const int g = threadIdx.x / LPK, li = threadIdx.x % LPK, d0 = li * VEC;
    // q stays unscaled (the score is scaled instead), so its load does not hold
    // back the first K/V loads.
    float qr[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
        const int d = min(d0 + e, s.hd - 1);
        qr[e] = q[size_t(b) * s.W + h * s.hd + d];
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e)
        if (d0 + e >= s.hd) qr[e] = 0.0f;
    const size_t head = size_t(b * s.H + h) * kv.cap;
    const float *kb = kv.k + head * HDP + d0;
    const float *vb = kv.v + head * HDP + d0;
    float m = -INFINITY, l = 0.0f, acc[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = 0.0f;
    for (int j0 = start; j0 < end; j0 += G * U) {
        float kk[U][VEC], vv[U][VEC];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            // Clamped rows keep every load in bounds and branch-free; keys past
            // `end` are masked out of the softmax below.
            const int j = min(j0 + u * G + g, end - 1);
            load_vec<VEC>(kb + size_t(j) * HDP, kk[u]);
            load_vec<VEC>(vb + size_t(j) * HDP, vv[u]);
        }
        float sc[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float p = 0.0f;
#pragma unroll
            for (int e = 0; e < VEC; ++e) p = fmaf(qr[e], kk[u][e], p);
#pragma unroll
            for (int o = 1; o < LPK; o <<= 1) p += __shfl_xor(p, o, 64);
            sc[u] = (j0 + u * G + g < end) ? p * scale_log2 : -INFINITY;
        }
        float cm = sc[0];
#pragma unroll
        for (int u = 1; u < U; ++u) cm = fmaxf(cm, sc[u]);
        const float mn = fmaxf(m, cm);
        if (mn != -INFINITY) {
            const float alpha = exp2f(m - mn);
            float pu[U], ps = 0.0f;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                pu[u] = exp2f(sc[u] - mn);
                ps += pu[u];
            }
            l = l * alpha + ps;
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                float a = acc[e] * alpha;
#pragma unroll
                for (int u = 0; u < U; ++u) a = fmaf(pu[u], vv[u][e], a);
                acc[e] = a;
            }
            m = mn;
        }
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) sacc[g * HDP + d0 + e] = acc[e];
    if (li == 0) {
        sm[g] = m;
        sl[g] = l;
    }
    __syncthreads();
    float M = -INFINITY;
    for (int k = 0; k < G; ++k) M = fmaxf(M, sm[k]);
    for (int d = threadIdx.x; d < HDP; d += blockDim.x) {
        float a = 0.0f;
        for (int k = 0; k < G; ++k) a += exp2f(sm[k] - M) * sacc[k * HDP + d];
        out[d] = a;
    }
    if (threadIdx.x == 0) {
        float L = 0.0f;
        for (int k = 0; k < G; ++k) L += exp2f(sm[k] - M) * sl[k];
        out[HDP] = M;
        out[HDP + 1] = L;
    }
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
#pragma unroll
                for (int o = 1; o < TPQ; o <<= 1) p += __shfl_xor(p, o, 64);
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

// The reference's sequential f32 sampler (gpu.rs:2034-2048) in one lane: a
// token-order sum, one SplitMix64 draw, and a token-order scan that stops at
// the first negative remainder; no multiply-add fusion.  Values come sixteen at
// a time so only the additions form the serial chain.  CACHED: p holds the
// exponentials; otherwise they are recomputed from the logits row.
template <bool CACHED>
__device__ int sequential_sample(const float *p, const float *row, int V, float mx,
                                              float temperature, uint64_t *rng) {
#pragma clang fp contract(off)
    constexpr int kBatch = 16;
    float sum = 0.0f;
    int t = 0;
    for (; t + kBatch <= V; t += kBatch) {
        float v[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) v[k] = CACHED ? p[t + k] : expf((row[t + k] - mx) / temperature);
#pragma unroll
        for (int k = 0; k < kBatch; ++k) sum = sum + v[k];
    }
    for (; t < V; ++t) sum = sum + (CACHED ? p[t] : expf((row[t] - mx) / temperature));
    uint64_t state = *rng;
    const float u = float(uint32_t(splitmix_next(state) >> 40)) / 16777216.0f;
    *rng = state;
    float sample = u * sum;
    for (t = 0; t + kBatch <= V; t += kBatch) {
        float v[kBatch], left[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) v[k] = CACHED ? p[t + k] : expf((row[t + k] - mx) / temperature);
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            sample = sample - v[k];
            left[k] = sample;
        }
#pragma unroll
        for (int k = 0; k < kBatch; ++k)
            if (left[k] < 0.0f) return t + k;
    }
    for (; t < V; ++t) {
        sample = sample - (CACHED ? p[t] : expf((row[t] - mx) / temperature));
        if (sample < 0.0f) return t;
    }
    return V - 1;
}

// Block-wide choice of the next token from a logits row (gpu.rs:2028-2049):
// greedy = the first maximal logit; T > 0 = the sequential sampler.  `p` is
// LDS scratch of `cap` floats; red holds one float and one int per wave.
__device__ int choose_token(const float *row, int V, float temperature, uint64_t *rng, int *flags, float *p,
                            int cap, float *redf, int *redi) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    float mx = -INFINITY;
    int bad = 0;
    for (int t = threadIdx.x; t < V; t += blockDim.x) {
        const float v = row[t];
        bad |= !isfinite(v);
        mx = fmaxf(mx, v);
    }
    mx = wave_max(mx);
    bad = wave_or_int(bad);
    if (lane == 0) {
        redf[wave] = mx;
        redi[wave] = bad;
    }
    __syncthreads();
    mx = -INFINITY;
    bad = 0;
    for (int w = 0; w < nw; ++w) {
        mx = fmaxf(mx, redf[w]);
        bad |= redi[w];
    }
    __syncthreads();
    if (bad && threadIdx.x == 0) atomicOr(flags, 1);
    if (temperature == 0.0f) {
        int best = INT_MAX;
        for (int t = threadIdx.x; t < V; t += blockDim.x)
            if (row[t] == mx) best = min(best, t);
        best = wave_min_int(best);
        if (lane == 0) redi[wave] = best;
        __syncthreads();
        best = INT_MAX;
        for (int w = 0; w < nw; ++w) best = min(best, redi[w]);
        __syncthreads();
        return best == INT_MAX ? 0 : best;
    }
    const bool cached = V <= cap;
    if (cached)
        for (int t = threadIdx.x; t < V; t += blockDim.x) p[t] = expf((row[t] - mx) / temperature);
    __syncthreads();
    if (threadIdx.x == 0)
        redi[0] = cached ? sequential_sample<true>(p, row, V, mx, temperature, rng)
                         : sequential_sample<false>(p, row, V, mx, temperature, rng);
    __syncthreads();
    const int token = redi[0];
    __syncthreads();
    return token;
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
    __shared__ __align__(16) float p[kSampleCap];
    __shared__ float redf[kThreads / 64];
    __shared__ int redi[kThreads / 64];
    const int b = blockIdx.x;
    const float *src = logits + size_t(b) * V;
    const bool staged = V <= kSampleCap;
    if (staged)
        for (int t = threadIdx.x; t < V; t += blockDim.x) row[t] = src[t];
    __syncthreads();
    const int token = choose_token(staged ? row : src, V, temperature, rng + b, flags, p, kSampleCap, redf, redi);
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
    float *P = lds.take<float>(size_t(kHeadSampleCap));
    float4 *red = lds.take<float4>(size_t(kHsGroups) * 64);
    float *redf = lds.take<float>(kHsThreads / 64);
    int *redi = lds.take<int>(kHsThreads / 64);
    for (int c = threadIdx.x; c < W; c += blockDim.x) N[c] = xn[size_t(b) * W + c];
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
    const int token = choose_token(L, V, temperature, rng + b, flags, P, kHeadSampleCap, redf, redi);
    append_token(tokens, tok_stride, len, b, token);
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

// out = mesh(in) for rows x W with one team (the embedding table from codes).
template <int CPT>
__global__ void __launch_bounds__(256)
mesh_rows_kernel(Shape s, const float *__restrict__ in, float *__restrict__ out, int rows,
                 const float *__restrict__ w, int depth, int rpw) {
    extern __shared__ __align__(16) char smem[];
    LdsCarve lds{smem};
    const int W = s.W, T = blockDim.x;
    float *A = lds.take<float>(size_t(rpw) * W);
    float *B = lds.take<float>(size_t(rpw) * W);
    float *C = lds.take<float>(size_t(rpw) * W);
    const int r0 = blockIdx.x * rpw, nr = min(rpw, rows - r0);
    MeshRing<CPT> ring;
    ring_prime<CPT>(ring, w, depth, W, threadIdx.x, T, true);
    for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) A[idx] = in[size_t(r0) * W + idx];
    __syncthreads();
    const float *res = mesh_team<CPT>(ring, A, B, C, nr, s, w, depth, threadIdx.x, T, true);
    for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) out[size_t(r0) * W + idx] = res[idx];
}

__global__ void __launch_bounds__(kThreads)
calibration_copy_kernel(const float4 *__restrict__ src, float4 *__restrict__ dst, size_t n) {
    const size_t stride = size_t(gridDim.x) * blockDim.x;
    for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

template <int HDP>
void launch_decode_t(const Shape &s, const float *q, KvView kv, const int *len, int batch, int nsplit,
                     float *part, hipStream_t stream) {
    const float scale_log2 = float(1.4426950408889634 / std::sqrt(double(s.hd)));
    dim3 grid(nsplit * batch, s.H);
    hipLaunchKernelGGL(attn_decode_kernel<HDP>, grid, dim3(DecodeCfg<HDP>::THREADS), 0, stream, s, q, kv,
                       len, nsplit, part, scale_log2);
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

size_t block_lds_bytes(const Shape &s, int rpw, int teams, int nsplit) {
    const size_t row = align16(size_t(rpw) * s.W * 4);
    return (2 + 2 * size_t(teams)) * row + 2 * align16(size_t(rpw) * s.H * 4) + align16(size_t(rpw) * 4) +
           align16(size_t(rpw) * s.H * nsplit * 4);
}

size_t mesh_lds_bytes(const Shape &s, int rpw) { return 3 * align16(size_t(rpw) * s.W * 4); }

size_t head_lds_bytes(const Shape &s, int rt) {
    return align16(size_t(rt) * s.W * 4) + align16(size_t(kHeadGroups) * kHeadMaxRows * kHeadTokens * 4);
}

size_t head_sample_lds_bytes(const Shape &s) {
    if (s.V > kHeadSampleCap) return size_t(-1);
    return align16(size_t(s.W) * 4) + 2 * align16(kHeadSampleCap * 4) + align16(size_t(kHsGroups) * 64 * 16) +
           2 * align16(kHsThreads / 64 * 4);
}

void configure_lds(size_t max_bytes) {
    const int bytes = int(max_bytes);
    auto allow = [bytes](const void *f) {
        (void)hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    };
    for (int cpt : {1, 2, 4, 8, 16})
        with_cpt(cpt, [&](auto c) {
            allow(reinterpret_cast<const void *>(&block_kernel<decltype(c)::value>));
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

void transpose(const float *E, float *Et, int V, int Vp, int W, hipStream_t stream) {
    dim3 grid((Vp + 31) / 32, (W + 31) / 32);
    hipLaunchKernelGGL(transpose_kernel, grid, dim3(kThreads), 0, stream, E, Et, V, Vp, W);
    HIP_LAUNCH_CHECK();
}

void block(const BlockArgs &a, hipStream_t stream) {
    dim3 grid((a.ro.rows + a.rpw - 1) / a.rpw);
    const size_t lds = block_lds_bytes(a.s, a.rpw, a.teams, a.part ? a.nsplit : 0);
    with_cpt(channels_per_thread(a.s.W), [&](auto c) {
        hipLaunchKernelGGL(block_kernel<decltype(c)::value>, grid, dim3(a.teams * team_threads(a.s.W)), lds,
                           stream, a);
    });
    HIP_LAUNCH_CHECK();
}

void attn_decode(const Shape &s, const float *q, KvView kv, const int *len, int batch, int nsplit, float *part,
                 hipStream_t stream) {
    switch (s.hdp) {
    case 2: return launch_decode_t<2>(s, q, kv, len, batch, nsplit, part, stream);
    case 4: return launch_decode_t<4>(s, q, kv, len, batch, nsplit, part, stream);
    case 8: return launch_decode_t<8>(s, q, kv, len, batch, nsplit, part, stream);
    case 16: return launch_decode_t<16>(s, q, kv, len, batch, nsplit, part, stream);
    case 32: return launch_decode_t<32>(s, q, kv, len, batch, nsplit, part, stream);
    case 64: return launch_decode_t<64>(s, q, kv, len, batch, nsplit, part, stream);
    case 128: return launch_decode_t<128>(s, q, kv, len, batch, nsplit, part, stream);
    case 256: return launch_decode_t<256>(s, q, kv, len, batch, nsplit, part, stream);
    case 512: return launch_decode_t<512>(s, q, kv, len, batch, nsplit, part, stream);
    case 1024: return launch_decode_t<1024>(s, q, kv, len, batch, nsplit, part, stream);
    case 2048: return launch_decode_t<2048>(s, q, kv, len, batch, nsplit, part, stream);
    case 4096: return launch_decode_t<4096>(s, q, kv, len, batch, nsplit, part, stream);
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

void calibration_copy(const float4 *src, float4 *dst, size_t n, hipStream_t stream) {
    const size_t blocks = std::min<size_t>((n + kThreads - 1) / kThreads, 256 * 16);
    hipLaunchKernelGGL(calibration_copy_kernel, dim3(unsigned(std::max<size_t>(blocks, 1))), dim3(kThreads), 0,
                       stream, src, dst, n);
    HIP_LAUNCH_CHECK();
}

void sample(int V, int batch, const float *logits, float temperature, uint64_t *rng, uint32_t *tokens,
            int tok_stride, int *len, int *flags, hipStream_t stream) {
    hipLaunchKernelGGL(sample_kernel, dim3(batch), dim3(kThreads), 0, stream, logits, V, temperature, rng, tokens,
                       tok_stride, len, flags);
    HIP_LAUNCH_CHECK();
}

}  // namespace meshgpt::kern
