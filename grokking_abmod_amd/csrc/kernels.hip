// gfx950 kernels of the Mesh GPT generate path (prefill and per-token decode).
//
// Everything except attention is row-local, so a block's work is cut into two
// row kernels around the one cross-row operator:
//   qkv_kernel   (embed) + RMSNorm + one Q/K/V mesh stack + QK-Norm + RoPE +
//                KV-cache append, one workgroup per row tile and mesh;
//   attention    attn_decode_kernel (split-KV, HBM-bound stream over the cache)
//                or attn_prefill_kernel (causal flash over LDS K/V tiles);
//   post_kernel  split combine + XSA + projection mesh + residual + RMSNorm +
//                FFN mesh + residual.
// Mesh stacks keep their rows in LDS across all layers (one barrier per layer)
// and stage the layers' [self, partner] weight pairs in LDS in one sweep.
// All arithmetic is FP32.  Reference semantics: src/gpt/reference.rs:104-228.
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>

#include "kernels.hpp"

namespace meshgpt::kern {
namespace {

constexpr float kRmsEps = 1e-5f;  // src/gpt/mod.rs:38
// (f64(1e-12f))^2 rounded to f32: the XSA norm floor of reference.rs:591
constexpr float kXsaFloor = float(double(1e-12f) * double(1e-12f));
constexpr int kSampleLds = 8192;  // logits cached in LDS by the sampler

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

// Runs a two-parent mesh stack (reference.rs:422-453) over nr rows held in LDS.
// `cur` holds the input (visible to all threads); the result pointer is
// returned (cur or nxt).  Weights are [layer][channel][self, partner]; with
// stage_layers > 0 they are copied into LDS `stage` that many layers at a time.
__device__ float *mesh_stack(float *cur, float *nxt, int nr, const Shape &s,
                             const float *__restrict__ w, int depth, float2 *stage, int stage_layers) {
    const int W = s.W, total = nr * W;
    const int chunk = stage_layers > 0 ? stage_layers : depth;
    for (int l0 = 0; l0 < depth; l0 += chunk) {
        const int nl = min(chunk, depth - l0);
        const float2 *src = reinterpret_cast<const float2 *>(w) + size_t(l0) * W;
        if (stage_layers > 0) {
            __syncthreads();
            for (int i = threadIdx.x; i < nl * W; i += blockDim.x) stage[i] = src[i];
            __syncthreads();
        }
        for (int l = l0; l < l0 + nl; ++l) {
            const int st = s.butterfly ? (1 << (l % s.log2w)) : 1;
            const float2 *wl = (stage_layers > 0 ? stage : src) + size_t(l - l0) * W;
            const bool last = l + 1 == depth;
            for (int idx = threadIdx.x; idx < total; idx += blockDim.x) {
                int r, c;
                split_row(idx, s, r, c);
                int p = c + st;
                if (p >= W) p -= W;
                const float2 ww = wl[c];
                const float z = cur[idx] * ww.x + cur[r * W + p] * ww.y;
                nxt[idx] = last ? z : elu(z);
            }
            __syncthreads();
            float *t = cur;
            cur = nxt;
            nxt = t;
        }
    }
    return cur;
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

// ----------------------------------------------------------------- kernels

__global__ void __launch_bounds__(kThreads)
mesh_rows_kernel(Shape s, const float *__restrict__ in, float *__restrict__ out, int rows,
                 const float *__restrict__ w, int depth, Tiling t) {
    extern __shared__ __align__(16) char smem[];
    LdsCarve lds{smem};
    float2 *stage = lds.take<float2>(size_t(t.stage_layers) * s.W);
    float *A = lds.take<float>(size_t(t.rpw) * s.W);
    float *B = lds.take<float>(size_t(t.rpw) * s.W);
    const int r0 = blockIdx.x * t.rpw, nr = min(t.rpw, rows - r0);
    for (int idx = threadIdx.x; idx < nr * s.W; idx += blockDim.x) A[idx] = in[size_t(r0) * s.W + idx];
    __syncthreads();
    const float *res = mesh_stack(A, B, nr, s, w, depth, stage, t.stage_layers);
    for (int idx = threadIdx.x; idx < nr * s.W; idx += blockDim.x) out[size_t(r0) * s.W + idx] = res[idx];
}

__global__ void __launch_bounds__(kThreads)
transpose_kernel(const float *__restrict__ E, float *__restrict__ Et, int V, int W) {
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
        if (c < W && t < V) Et[size_t(c) * V + t] = tile[tx][k];
    }
}

// Pre-attention half of a block (reference.rs:164-193).  grid = (row tiles, 3):
// grid.y selects the query, key or value mesh.
__global__ void __launch_bounds__(kThreads)
qkv_kernel(Shape s, Rows ro, const float *__restrict__ wq, const float *__restrict__ wk,
           const float *__restrict__ wv, const float *__restrict__ E, float *__restrict__ x,
           float *__restrict__ qout, KvView kv, const float2 *__restrict__ rope, int embed, Tiling t) {
    extern __shared__ __align__(16) char smem[];
    LdsCarve lds{smem};
    const int W = s.W;
    float2 *stage = lds.take<float2>(size_t(t.stage_layers) * W);
    float *A = lds.take<float>(size_t(t.rpw) * W);
    float *B = lds.take<float>(size_t(t.rpw) * W);
    float *inv = lds.take<float>(size_t(t.rpw) * s.H);
    const int m = blockIdx.y;
    const int r0 = blockIdx.x * t.rpw, nr = min(t.rpw, ro.rows - r0);

    for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) {
        int r, c;
        split_row(idx, s, r, c);
        const int row = r0 + r;
        float v;
        if (embed) {
            int seq, pos;
            row_position(ro, row, seq, pos);
            const uint32_t tok = ro.tokens[size_t(seq) * ro.tok_stride + ro.tok_offset + pos];
            v = E[size_t(tok) * W + c];
            if (m == 0) x[size_t(row) * W + c] = v;
        } else {
            v = x[size_t(row) * W + c];
        }
        A[idx] = v;
    }
    __syncthreads();
    segment_inv_rms(A, nr, W, inv);
    __syncthreads();
    for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) {
        int r, c;
        split_row(idx, s, r, c);
        A[idx] *= inv[r];
    }
    __syncthreads();
    const float *w = m == 0 ? wq : (m == 1 ? wk : wv);
    float *out = mesh_stack(A, B, nr, s, w, s.A, stage, t.stage_layers);

    if (m < 2) {
        // QK-Norm per head, then split-half RoPE at the row's position.
        segment_inv_rms(out, nr * s.H, s.hd, inv);
        __syncthreads();
        const int pairs = s.H * s.half;
        for (int idx = threadIdx.x; idx < nr * pairs; idx += blockDim.x) {
            const int r = idx / pairs, rem = idx - r * pairs;
            const int h = rem / s.half, i = rem - h * s.half;
            const int row = r0 + r;
            int seq, pos;
            row_position(ro, row, seq, pos);
            const float scale = inv[r * s.H + h];
            const float a = out[r * W + h * s.hd + i] * scale;
            const float b = out[r * W + h * s.hd + i + s.half] * scale;
            const float2 cs = rope[size_t(pos) * s.half + i];
            const float lo = a * cs.x - b * cs.y;
            const float hi = b * cs.x + a * cs.y;
            float *dst = m == 0 ? qout + size_t(row) * W + h * s.hd
                                : kv.k + (size_t(seq * s.H + h) * kv.cap + pos) * s.hdp;
            dst[i] = lo;
            dst[i + s.half] = hi;
        }
    } else {
        for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) {
            int r, c, h, d, seq, pos;
            split_row(idx, s, r, c);
            split_head(c, s, h, d);
            row_position(ro, r0 + r, seq, pos);
            kv.v[(size_t(seq * s.H + h) * kv.cap + pos) * s.hdp + d] = out[idx];
        }
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
    static constexpr int U = VEC >= 32 ? 1 : (VEC >= 16 ? 2 : 4);               // keys per group per step
};

// Split-KV decode attention (reference.rs:510-554 for one query row).  Block
// (split, head, seq) streams keys [split*ks, min(split*ks+ks, pos+1)) of the
// cache; each group of LPK lanes owns one key at a time, so every K/V row is
// one coalesced VEC-wide load per lane.  Scores live in the log2 domain.
template <int HDP>
__global__ void __launch_bounds__(DecodeCfg<HDP>::THREADS)
attn_decode_kernel(Shape s, const float *__restrict__ q, KvView kv, const int *__restrict__ len, int ks,
                   int smax, float *__restrict__ part, float scale_log2) {
    using C = DecodeCfg<HDP>;
    constexpr int VEC = C::VEC, LPK = C::LPK, G = C::G, U = C::U;
    __shared__ float sm[G], sl[G];
    __shared__ __align__(16) float sacc[G * HDP];
    const int b = int(blockIdx.x) / smax, split = int(blockIdx.x) - b * smax, h = blockIdx.y;
    const int pos = len[b] - 1;
    const int start = split * ks;
    if (start > pos) return;
    const int end = min(start + ks, pos + 1);
    const int g = threadIdx.x / LPK, li = threadIdx.x % LPK, d0 = li * VEC;
    float qr[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
        const int d = d0 + e;
        qr[e] = d < s.hd ? q[size_t(b) * s.W + h * s.hd + d] * scale_log2 : 0.0f;
    }
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
            const int j = j0 + u * G + g;
            if (j < end) {
                load_vec<VEC>(kb + size_t(j) * HDP, kk[u]);
                load_vec<VEC>(vb + size_t(j) * HDP, vv[u]);
            } else {
#pragma unroll
                for (int e = 0; e < VEC; ++e) kk[u][e] = vv[u][e] = 0.0f;
            }
        }
        float sc[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float p = 0.0f;
#pragma unroll
            for (int e = 0; e < VEC; ++e) p = fmaf(qr[e], kk[u][e], p);
#pragma unroll
            for (int o = 1; o < LPK; o <<= 1) p += __shfl_xor(p, o, 64);
            sc[u] = (j0 + u * G + g < end) ? p : -INFINITY;
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
    float *out = part + (size_t(b * s.H + h) * smax + split) * (HDP + 2);
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

// Post-attention half of a block (reference.rs:194-216).
__global__ void __launch_bounds__(kThreads)
post_kernel(Shape s, Rows ro, const float *__restrict__ part, int ks, int smax,
            const float *__restrict__ ybuf, KvView kv, const float *__restrict__ wproj,
            const float *__restrict__ wffn, float *__restrict__ x, Tiling t) {
    extern __shared__ __align__(16) char smem[];
    LdsCarve lds{smem};
    const int W = s.W;
    float2 *stage = lds.take<float2>(size_t(t.stage_layers) * W);
    float *X = lds.take<float>(size_t(t.rpw) * W);
    float *A = lds.take<float>(size_t(t.rpw) * W);
    float *B = lds.take<float>(size_t(t.rpw) * W);
    float *vv = lds.take<float>(size_t(t.rpw) * s.H);
    float *yv = lds.take<float>(size_t(t.rpw) * s.H);
    float *rinv = lds.take<float>(size_t(t.rpw));
    const int r0 = blockIdx.x * t.rpw, nr = min(t.rpw, ro.rows - r0);
    const int stride = s.hdp + 2;

    // Attention output y (combining split partials) and the row's own value v.
    for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) {
        int r, c, h, d, seq, pos;
        split_row(idx, s, r, c);
        split_head(c, s, h, d);
        const int row = r0 + r;
        row_position(ro, row, seq, pos);
        float yval;
        if (part) {
            const float *pp = part + size_t(seq * s.H + h) * smax * stride;
            const int nsplit = pos / ks + 1;
            float M = -INFINITY;
            for (int k = 0; k < nsplit; ++k) M = fmaxf(M, pp[k * stride + s.hdp]);
            float num = 0.0f, den = 0.0f;
            for (int k = 0; k < nsplit; ++k) {
                const float wgt = exp2f(pp[k * stride + s.hdp] - M);
                num = fmaf(wgt, pp[k * stride + d], num);
                den = fmaf(wgt, pp[k * stride + s.hdp + 1], den);
            }
            yval = num / den;
        } else {
            yval = ybuf[size_t(row) * W + c];
        }
        A[idx] = yval;
        B[idx] = kv.v[(size_t(seq * s.H + h) * kv.cap + pos) * s.hdp + d];
    }
    __syncthreads();
    // XSA (reference.rs:577-603): z = y - (y.u)u with u = v / max(|v|, eps).
    segment_dots(A, B, nr * s.H, s.hd, vv, yv);
    __syncthreads();
    for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) {
        int r, c, h, d;
        split_row(idx, s, r, c);
        split_head(c, s, h, d);
        const int sg = r * s.H + h;
        const float iv = 1.0f / sqrtf(fmaxf(vv[sg], kXsaFloor));
        const float projection = yv[sg] * iv;
        A[idx] = A[idx] - projection * (B[idx] * iv);
    }
    __syncthreads();
    const float *proj = mesh_stack(A, B, nr, s, wproj, s.A, stage, t.stage_layers);
    for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) {
        int r, c;
        split_row(idx, s, r, c);
        X[idx] = x[size_t(r0 + r) * W + c] + proj[idx];
    }
    __syncthreads();
    segment_inv_rms(X, nr, W, rinv);
    __syncthreads();
    for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) {
        int r, c;
        split_row(idx, s, r, c);
        A[idx] = X[idx] * rinv[r];
    }
    __syncthreads();
    const float *ffn = mesh_stack(A, B, nr, s, wffn, s.F, stage, t.stage_layers);
    for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) {
        int r, c;
        split_row(idx, s, r, c);
        x[size_t(r0 + r) * W + c] = X[idx] + ffn[idx];
    }
}

// Tied vocabulary head (reference.rs:218-226): final RMSNorm, then dot products
// with every token vector.  Block = (64 tokens) x (rt rows); Et is [W][V].
__global__ void __launch_bounds__(kThreads)
head_kernel(Shape s, const float *__restrict__ x, int nrows, int row_mul, int row_add,
            const float *__restrict__ Et, float *__restrict__ logits, int rt) {
    extern __shared__ __align__(16) char smem[];
    LdsCarve lds{smem};
    const int W = s.W, V = s.V;
    float *N = lds.take<float>(size_t(rt) * W);
    float *inv = lds.take<float>(size_t(rt));
    const int i0 = blockIdx.y * rt, nr = min(rt, nrows - i0);
    for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) {
        int r, c;
        split_row(idx, s, r, c);
        N[idx] = x[(size_t(i0 + r) * row_mul + row_add) * W + c];
    }
    __syncthreads();
    segment_inv_rms(N, nr, W, inv);
    __syncthreads();
    for (int idx = threadIdx.x; idx < nr * W; idx += blockDim.x) {
        int r, c;
        split_row(idx, s, r, c);
        N[idx] *= inv[r];
    }
    __syncthreads();
    const int t = blockIdx.x * 64 + (threadIdx.x & 63), rg = threadIdx.x >> 6;
    if (t >= V) return;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int c = 0; c < W; ++c) {
        const float e = Et[size_t(c) * V + t];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int r = rg + 4 * k;
            if (r < nr) acc[k] = fmaf(N[r * W + c], e, acc[k]);
        }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int r = rg + 4 * k;
        if (r < nr) logits[size_t(i0 + r) * V + t] = acc[k];
    }
}

__device__ __forceinline__ uint64_t splitmix_next(uint64_t &state) {
    state += 0x9e3779b97f4a7c15ULL;
    uint64_t bits = state;
    bits = (bits ^ (bits >> 30)) * 0xbf58476d1ce4e5b9ULL;
    bits = (bits ^ (bits >> 27)) * 0x94d049bb133111ebULL;
    return bits ^ (bits >> 31);
}

// The reference's sequential f32 sampler (gpu.rs:2034-2048): the sum and the
// scan run in token order in one lane, without multiply-add fusion.
__device__ __noinline__ int sequential_sample(const float *p, const float *row, int V, float mx,
                                              float temperature, uint64_t *rng, bool cached) {
#pragma clang fp contract(off)
    float sum = 0.0f;
    for (int t = 0; t < V; ++t) sum = sum + (cached ? p[t] : expf((row[t] - mx) / temperature));
    uint64_t state = *rng;
    const float u = float(uint32_t(splitmix_next(state) >> 40)) / 16777216.0f;
    *rng = state;
    float sample = u * sum;
    int selected = V - 1;
    for (int t = 0; t < V; ++t) {
        sample = sample - (cached ? p[t] : expf((row[t] - mx) / temperature));
        if (sample < 0.0f) {
            selected = t;
            break;
        }
    }
    return selected;
}

// One wave per sequence: greedy picks the first maximal logit; T > 0 samples
// with the sequence's SplitMix64 state.  The token is appended at len[b].
__global__ void __launch_bounds__(64)
sample_kernel(const float *__restrict__ logits, int V, float temperature, uint64_t *rng,
              uint32_t *tokens, int tok_stride, int *len, int *flags) {
    __shared__ float p[kSampleLds];
    __shared__ int chosen;
    const int b = blockIdx.x, lane = threadIdx.x;
    const float *row = logits + size_t(b) * V;
    float mx = -INFINITY;
    int bad = 0;
    for (int t = lane; t < V; t += 64) {
        const float v = row[t];
        bad |= !isfinite(v);
        mx = fmaxf(mx, v);
    }
    mx = wave_max(mx);
    bad = wave_or_int(bad);
    if (bad && lane == 0) atomicOr(flags, 1);
    int token;
    if (temperature == 0.0f) {
        int best = INT_MAX;
        for (int t = lane; t < V; t += 64)
            if (row[t] == mx) best = min(best, t);
        best = wave_min_int(best);
        token = best == INT_MAX ? 0 : best;
    } else {
        const bool cached = V <= kSampleLds;
        if (cached)
            for (int t = lane; t < V; t += 64) p[t] = expf((row[t] - mx) / temperature);
        __syncthreads();
        if (lane == 0) chosen = sequential_sample(p, row, V, mx, temperature, rng + b, cached);
        __syncthreads();
        token = chosen;
    }
    if (lane == 0) {
        const int L = len[b];
        tokens[size_t(b) * tok_stride + L] = uint32_t(token);
        len[b] = L + 1;
    }
}

template <int HDP>
void launch_decode_t(const Shape &s, const float *q, KvView kv, const int *len, int batch, int ks,
                     int smax, float *part, hipStream_t stream) {
    const float scale_log2 = float(1.4426950408889634 / std::sqrt(double(s.hd)));
    dim3 grid(smax * batch, s.H);
    hipLaunchKernelGGL(attn_decode_kernel<HDP>, grid, dim3(DecodeCfg<HDP>::THREADS), 0, stream, s, q, kv,
                       len, ks, smax, part, scale_log2);
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

}  // namespace

size_t mesh_lds_bytes(const Shape &s, const Tiling &t) {
    return align16(size_t(t.stage_layers) * s.W * 8) + 2 * align16(size_t(t.rpw) * s.W * 4);
}

size_t qkv_lds_bytes(const Shape &s, const Tiling &t) {
    return mesh_lds_bytes(s, t) + align16(size_t(t.rpw) * s.H * 4);
}

size_t post_lds_bytes(const Shape &s, const Tiling &t) {
    return align16(size_t(t.stage_layers) * s.W * 8) + 3 * align16(size_t(t.rpw) * s.W * 4) +
           2 * align16(size_t(t.rpw) * s.H * 4) + align16(size_t(t.rpw) * 4);
}

size_t head_lds_bytes(const Shape &s, int rt) {
    return align16(size_t(rt) * s.W * 4) + align16(size_t(rt) * 4);
}

void configure_lds(size_t max_bytes) {
    const int bytes = int(max_bytes);
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&mesh_rows_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&qkv_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&post_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    (void)hipFuncSetAttribute(reinterpret_cast<const void *>(&head_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

void mesh_rows(const Shape &s, const float *in, float *out, int rows, const float *w, int depth, Tiling t,
               hipStream_t stream) {
    dim3 grid((rows + t.rpw - 1) / t.rpw);
    hipLaunchKernelGGL(mesh_rows_kernel, grid, dim3(kThreads), mesh_lds_bytes(s, t), stream, s, in, out,
                       rows, w, depth, t);
    HIP_LAUNCH_CHECK();
}

void transpose(const float *E, float *Et, int V, int W, hipStream_t stream) {
    dim3 grid((V + 31) / 32, (W + 31) / 32);
    hipLaunchKernelGGL(transpose_kernel, grid, dim3(kThreads), 0, stream, E, Et, V, W);
    HIP_LAUNCH_CHECK();
}

void qkv(const Shape &s, const Rows &r, const float *wq, const float *wk, const float *wv, const float *E,
         float *x, float *q, KvView kv, const float2 *rope, int embed, Tiling t, hipStream_t stream) {
    dim3 grid((r.rows + t.rpw - 1) / t.rpw, 3);
    hipLaunchKernelGGL(qkv_kernel, grid, dim3(kThreads), qkv_lds_bytes(s, t), stream, s, r, wq, wk, wv, E, x,
                       q, kv, rope, embed, t);
    HIP_LAUNCH_CHECK();
}

void attn_decode(const Shape &s, const float *q, KvView kv, const int *len, int batch, int ks, int smax,
                 float *part, hipStream_t stream) {
    switch (s.hdp) {
    case 2: return launch_decode_t<2>(s, q, kv, len, batch, ks, smax, part, stream);
    case 4: return launch_decode_t<4>(s, q, kv, len, batch, ks, smax, part, stream);
    case 8: return launch_decode_t<8>(s, q, kv, len, batch, ks, smax, part, stream);
    case 16: return launch_decode_t<16>(s, q, kv, len, batch, ks, smax, part, stream);
    case 32: return launch_decode_t<32>(s, q, kv, len, batch, ks, smax, part, stream);
    case 64: return launch_decode_t<64>(s, q, kv, len, batch, ks, smax, part, stream);
    case 128: return launch_decode_t<128>(s, q, kv, len, batch, ks, smax, part, stream);
    case 256: return launch_decode_t<256>(s, q, kv, len, batch, ks, smax, part, stream);
    case 512: return launch_decode_t<512>(s, q, kv, len, batch, ks, smax, part, stream);
    case 1024: return launch_decode_t<1024>(s, q, kv, len, batch, ks, smax, part, stream);
    case 2048: return launch_decode_t<2048>(s, q, kv, len, batch, ks, smax, part, stream);
    case 4096: return launch_decode_t<4096>(s, q, kv, len, batch, ks, smax, part, stream);
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

void post(const Shape &s, const Rows &r, const float *part, int ks, int smax, const float *y, KvView kv,
          const float *wproj, const float *wffn, float *x, Tiling t, hipStream_t stream) {
    dim3 grid((r.rows + t.rpw - 1) / t.rpw);
    hipLaunchKernelGGL(post_kernel, grid, dim3(kThreads), post_lds_bytes(s, t), stream, s, r, part, ks, smax,
                       y, kv, wproj, wffn, x, t);
    HIP_LAUNCH_CHECK();
}

void head(const Shape &s, const float *x, int nrows, int row_mul, int row_add, const float *Et,
          float *logits, int rt, hipStream_t stream) {
    dim3 grid((s.V + 63) / 64, (nrows + rt - 1) / rt);
    hipLaunchKernelGGL(head_kernel, grid, dim3(kThreads), head_lds_bytes(s, rt), stream, s, x, nrows, row_mul,
                       row_add, Et, logits, rt);
    HIP_LAUNCH_CHECK();
}

void sample(int V, int batch, const float *logits, float temperature, uint64_t *rng, uint32_t *tokens,
            int tok_stride, int *len, int *flags, hipStream_t stream) {
    hipLaunchKernelGGL(sample_kernel, dim3(batch), dim3(64), 0, stream, logits, V, temperature, rng, tokens,
                       tok_stride, len, flags);
    HIP_LAUNCH_CHECK();
}

}  // namespace meshgpt::kern
