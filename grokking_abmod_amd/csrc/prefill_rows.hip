// Prefill blocks over many rows: the post-attention half of block l-1
// (reference.rs:194-216: XSA when the attention kernel left it, projection
// mesh and residual, RMSNorm, FFN mesh and residual) fused with the
// pre-attention half of block l (reference.rs:164-193: RMSNorm, Q/K/V meshes,
// QK-Norm, RoPE, K/V cache append), for a tile of R rows per workgroup.
//
// A mesh layer (reference.rs:422-453) is a two-term update of every channel
// from itself and one partner channel, so a tile is kept as R rows x W
// channels where each thread owns CPT channels of RG rows in registers, and
// only the partner values travel: each layer writes the thread's values to
// LDS, one barrier, and reads the partner channel's rows back.  LDS holds the
// tile channel-major (the R rows of a channel contiguous, in 16-byte chunks
// rotated by channel so that neighbouring lanes' 16-byte accesses fall in
// different banks), double-buffered so one barrier per layer suffices.  Each
// thread loads one [self, partner] weight pair per owned channel per layer,
// used for all of its rows.  Row reductions (RMSNorm) go through a small LDS
// scratch; head reductions (QK-Norm, XSA) and the RoPE pair exchange stay
// inside a wave (a head is hd <= 64 consecutive channels = consecutive lanes).
#include <hip/hip_runtime.h>

#include "dpp.hpp"
#include "kernels.hpp"

namespace meshgpt::kern {
namespace {

constexpr float kEps = 1e-5f;  // src/gpt/mod.rs:38
// (f64(1e-12f))^2 rounded to f32: the XSA norm floor of reference.rs:591.
constexpr float kXsaNormFloor = float(double(1e-12f) * double(1e-12f));

__device__ __forceinline__ float elu_f(float z) {
    // max(z, clamp(exp(z), 0, 1) - 1) with the NaN-propagating maximum, which
    // keeps a NaN z NaN (kernels.hip's elu)
    const float e = __builtin_amdgcn_fmed3f(__builtin_amdgcn_exp2f(z * 1.4426950408889634f), 0.0f, 1.0f);
    return __builtin_elementwise_maximum(z, e - 1.0f);
}

template <int W>
struct RowsCfg {
    static constexpr int THREADS = 256;
    static constexpr int T = W < 256 ? W : 256;   // threads per row group (one per channel slot)
    static constexpr int G = THREADS / T;         // row groups
    static constexpr int CPT = W / T;             // channels per thread: slot + T*k
    static constexpr int R = 4096 / W;            // rows per workgroup
    static constexpr int RG = R / G;              // rows per thread
    static constexpr int NCH = R / 4;             // 16-byte chunks of a channel
    static constexpr int ROT = R >= 64 ? 1 : 64 / R;  // channels per chunk rotation step
    static constexpr int TILE = W * R;            // floats of one LDS buffer
    static constexpr int WAVES_G = T / 64 > 0 ? T / 64 : 1;  // waves per row group
    static_assert(RG % 4 == 0 && W % 64 == 0, "tile geometry");
};

// LDS offset of the 16-byte chunk holding rows [4 ch, 4 ch + 4) of channel c.
template <int W>
__device__ __forceinline__ int chunk_at(int c, int ch) {
    using C = RowsCfg<W>;
    return c * C::R + 4 * ((ch + c / C::ROT) & (C::NCH - 1));
}

template <int W>
struct Tile {
    using C = RowsCfg<W>;
    static constexpr int CPT = C::CPT, RG = C::RG;
    float *lds;   // 2 * TILE floats
    float *red;   // row-reduction scratch: [4 waves][RG]
    int parity;
    int slot, rg, lane, wave;  // channel slot, row group
    __device__ int chan(int k) const { return slot + C::T * k; }
    __device__ int row(int i) const { return rg * RG + i; }

    __device__ void put(const float (&v)[CPT][RG]) {
        float *B = lds + parity * C::TILE;
#pragma unroll
        for (int k = 0; k < CPT; ++k)
#pragma unroll
            for (int j = 0; j < RG / 4; ++j)
                *reinterpret_cast<float4 *>(B + chunk_at<W>(chan(k), rg * (RG / 4) + j)) =
                    make_float4(v[k][4 * j], v[k][4 * j + 1], v[k][4 * j + 2], v[k][4 * j + 3]);
    }
    // The values of channel (own channel + st) mod W from the buffer last put.
    __device__ void partner(int st, float (&p)[CPT][RG]) const {
        const float *B = lds + parity * C::TILE;
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            const int c = (chan(k) + st) & (W - 1);
#pragma unroll
            for (int j = 0; j < RG / 4; ++j) {
                const float4 t = *reinterpret_cast<const float4 *>(B + chunk_at<W>(c, rg * (RG / 4) + j));
                p[k][4 * j] = t.x;
                p[k][4 * j + 1] = t.y;
                p[k][4 * j + 2] = t.z;
                p[k][4 * j + 3] = t.w;
            }
        }
    }
    __device__ void flip() { parity ^= 1; }

    // A mesh stack on v in place: layer l maps v[c] to v[c] w0 + v[c + st] w1
    // with ELU on every layer but the last (reference.rs:422-453).
    // Butterfly strides double from 1 and wrap at W (W is a power of two).
    __device__ void mesh(float (&v)[CPT][RG], const float2 *__restrict__ w, int depth, const Shape &s) {
        float2 wc[CPT];
#pragma unroll
        for (int k = 0; k < CPT; ++k) wc[k] = w[chan(k)];
        int st = 1;
        for (int l = 0; l < depth; ++l) {
            put(v);
            __syncthreads();
            float2 wn[CPT];
            if (l + 1 < depth) {
#pragma unroll
                for (int k = 0; k < CPT; ++k) wn[k] = w[size_t(l + 1) * W + chan(k)];
            }
            float p[CPT][RG];
            partner(st, p);
            if (l + 1 < depth) {
#pragma unroll
                for (int k = 0; k < CPT; ++k)
#pragma unroll
                    for (int i = 0; i < RG; ++i) v[k][i] = elu_f(v[k][i] * wc[k].x + p[k][i] * wc[k].y);
#pragma unroll
                for (int k = 0; k < CPT; ++k) wc[k] = wn[k];
            } else {
#pragma unroll
                for (int k = 0; k < CPT; ++k)
#pragma unroll
                    for (int i = 0; i < RG; ++i) v[k][i] = v[k][i] * wc[k].x + p[k][i] * wc[k].y;
            }
            flip();
            st = s.butterfly ? (2 * st == W ? 1 : 2 * st) : 1;
        }
    }

    // inv[i] = 1 / sqrt(mean over the row's W channels of v^2 + eps) for the
    // thread's rows (reference.rs:392-409 with one segment).
    __device__ void row_inv_rms(const float (&v)[CPT][RG], float (&inv)[RG]) {
        float part[RG];
#pragma unroll
        for (int i = 0; i < RG; ++i) {
            float a = 0.0f;
#pragma unroll
            for (int k = 0; k < CPT; ++k) a = fmaf(v[k][i], v[k][i], a);
            part[i] = a;
        }
#pragma unroll
        for (int i = 0; i < RG; ++i) part[i] = wave_sum(part[i]);
        __syncthreads();  // the scratch's previous readers are done
        if (lane == 0) {
#pragma unroll
            for (int i = 0; i < RG; ++i) red[wave * RG + i] = part[i];
        }
        __syncthreads();
        const int w0 = rg * C::WAVES_G;
#pragma unroll
        for (int i = 0; i < RG; ++i) {
            float a = 0.0f;
            for (int q = 0; q < C::WAVES_G; ++q) a += red[(w0 + q) * RG + i];
            inv[i] = rsqrtf(a * (1.0f / float(W)) + kEps);
        }
    }
};

// Sum over the hd lanes of a head (hd a power of two <= 64, heads aligned to
// hd lanes): DPP moves when the head width HD is a compile-time 32 or 64.
template <int HD>
__device__ __forceinline__ float head_sum(float v, int hd) {
    if constexpr (HD > 0) return group_sum<HD>(v);
    for (int m = hd >> 1; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// HD: the head width when it is 32 or 64 (DPP head sums), else 0.  Rows are
// whole prefill sequences (Rows.len is null: a row's position is its index
// within its sequence).
template <int W, int HD>
__global__ void __launch_bounds__(256) rows_block_kernel(BlockArgs a) {
    using C = RowsCfg<W>;
    constexpr int CPT = C::CPT, RG = C::RG;
    __shared__ __align__(16) float lds[2 * C::TILE];
    __shared__ float red[4 * RG];
    const Shape &s = a.s;
    Tile<W> t;
    t.lds = lds;
    t.red = red;
    t.parity = 0;
    t.slot = int(threadIdx.x) % C::T;
    t.rg = int(threadIdx.x) / C::T;
    t.lane = int(threadIdx.x) & 63;
    t.wave = int(threadIdx.x) >> 6;
    const bool post = a.wproj != nullptr, pre = a.wq != nullptr;
    const int r0 = int(blockIdx.x) * C::R;

    // Rows of this thread: rbase + i; rows past the batch repeat its last row
    // and write nothing.  Only the sequences are kept; the row indices and
    // positions are formed where they are used.
    const int rbase = r0 + t.rg * RG, rps = a.ro.rows_per_seq;
    auto rowof = [&](int i) { return min(rbase + i, a.ro.rows - 1); };
    auto live = [&](int i) { return rbase + i < a.ro.rows; };
    int seq[RG];
#pragma unroll
    for (int i = 0; i < RG; ++i) seq[i] = rowof(i) / rps;
    auto grow = [&](int i) { return size_t(rowof(i)); };
    auto posof = [&](int i) { return rowof(i) - seq[i] * rps; };

    float x[CPT][RG];
    if (a.embed) {
#pragma unroll
        for (int i = 0; i < RG; ++i) {
            const uint32_t tok = a.ro.tokens[size_t(seq[i]) * a.ro.tok_stride + a.ro.tok_offset + posof(i)];
#pragma unroll
            for (int k = 0; k < CPT; ++k) x[k][i] = a.E[size_t(tok) * W + t.chan(k)];
        }
    } else {
#pragma unroll
        for (int i = 0; i < RG; ++i)
#pragma unroll
            for (int k = 0; k < CPT; ++k) x[k][i] = a.x[grow(i) * W + t.chan(k)];
    }

    if (post) {
        float y[CPT][RG];
#pragma unroll
        for (int i = 0; i < RG; ++i)
#pragma unroll
            for (int k = 0; k < CPT; ++k) y[k][i] = a.ybuf[grow(i) * W + t.chan(k)];
        if (a.xsa_post) {
            // XSA (reference.rs:577-603): z = y - (y.u)u, u = v / max(|v|, eps).
#pragma unroll
            for (int k = 0; k < CPT; ++k) {
                const int c = t.chan(k), h = c / s.hd, d = c - h * s.hd;
#pragma unroll
                for (int i = 0; i < RG; ++i) {
                    const float v =
                        a.kv_post.v[(size_t(seq[i] * s.H + h) * a.kv_post.cap + posof(i)) * s.hdp + d];
                    const float vv = head_sum<HD>(v * v, s.hd), yv = head_sum<HD>(y[k][i] * v, s.hd);
                    const float iv = rsqrtf(fmaxf(vv, kXsaNormFloor));
                    y[k][i] = y[k][i] - (yv * iv) * (v * iv);
                }
            }
        }
        t.mesh(y, reinterpret_cast<const float2 *>(a.wproj), s.A, s);
#pragma unroll
        for (int k = 0; k < CPT; ++k)
#pragma unroll
            for (int i = 0; i < RG; ++i) x[k][i] += y[k][i];
        float inv[RG];
        t.row_inv_rms(x, inv);
        float n[CPT][RG];
#pragma unroll
        for (int k = 0; k < CPT; ++k)
#pragma unroll
            for (int i = 0; i < RG; ++i) n[k][i] = x[k][i] * inv[i];
        t.mesh(n, reinterpret_cast<const float2 *>(a.wffn), s.F, s);
#pragma unroll
        for (int k = 0; k < CPT; ++k)
#pragma unroll
            for (int i = 0; i < RG; ++i) x[k][i] += n[k][i];
    }
    if (post || a.embed) {
#pragma unroll
        for (int i = 0; i < RG; ++i)
            if (live(i)) {
#pragma unroll
                for (int k = 0; k < CPT; ++k) a.x[grow(i) * W + t.chan(k)] = x[k][i];
            }
    }
    if (!a.xn && !pre) return;

    // The next RMSNorm: the final one for the head, or the block's pre-norm.
    float n[CPT][RG];
    {
        float inv[RG];
        t.row_inv_rms(x, inv);
#pragma unroll
        for (int k = 0; k < CPT; ++k)
#pragma unroll
            for (int i = 0; i < RG; ++i) n[k][i] = x[k][i] * inv[i];
    }
    if (a.xn) {
#pragma unroll
        for (int i = 0; i < RG; ++i)
            if (live(i)) {
#pragma unroll
                for (int k = 0; k < CPT; ++k) a.xn[grow(i) * W + t.chan(k)] = n[k][i];
            }
    }
    if (!pre) return;

    // Q, K and V meshes, one after another, each from the normalised rows.
    const size_t meshw = size_t(s.A) * W;
    for (int m = 0; m < 3; ++m) {
        const float *wm = m == 0 ? a.wq : (m == 1 ? a.wk : a.wv);
        float v[CPT][RG];
#pragma unroll
        for (int k = 0; k < CPT; ++k)
#pragma unroll
            for (int i = 0; i < RG; ++i) v[k][i] = n[k][i];
        t.mesh(v, reinterpret_cast<const float2 *>(wm), s.A, s);
        (void)meshw;
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            const int c = t.chan(k), h = c / s.hd, d = c - h * s.hd;
            if (m < 2) {
                // QK-Norm per head, then RoPE at the row's position, each when
                // its switch is on (reference.rs:174-193); the pair partner
                // d ^ half is the lane half a head away.
#pragma unroll
                for (int i = 0; i < RG; ++i) {
                    float q = v[k][i];
                    if (s.qk_norm) q *= rsqrtf(head_sum<HD>(q * q, s.hd) * (1.0f / float(s.hd)) + kEps);
                    if (s.rope) {
                        const float p = __shfl_xor(q, s.half, 64);
                        const float2 cs = a.rope[size_t(posof(i)) * s.half + (d < s.half ? d : d - s.half)];
                        q = q * cs.x + (d < s.half ? -p : p) * cs.y;
                    }
                    v[k][i] = q;
                }
            }
#pragma unroll
            for (int i = 0; i < RG; ++i) {
                if (!live(i)) continue;
                if (m == 0) {
                    a.q[grow(i) * W + c] = v[k][i];
                } else {
                    float *dst = m == 1 ? a.kv_pre.k : a.kv_pre.v;
                    dst[(size_t(seq[i] * s.H + h) * a.kv_pre.cap + posof(i)) * s.hdp + d] = v[k][i];
                }
            }
        }
    }
}

}  // namespace

bool rows_block_supported(const Shape &s) {
    return (s.W == 128 || s.W == 256 || s.W == 512 || s.W == 1024) && s.hdshift >= 1 && s.hd <= 64 &&
           64 % s.hd == 0;
}

template <int W>
void launch_rows_block(const BlockArgs &a, hipStream_t stream) {
    const dim3 grid((a.ro.rows + RowsCfg<W>::R - 1) / RowsCfg<W>::R);
    if (a.s.hd == 32)
        hipLaunchKernelGGL((rows_block_kernel<W, 32>), grid, dim3(256), 0, stream, a);
    else if (a.s.hd == 64)
        hipLaunchKernelGGL((rows_block_kernel<W, 64>), grid, dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL((rows_block_kernel<W, 0>), grid, dim3(256), 0, stream, a);
}

void rows_block(const BlockArgs &a, hipStream_t stream) {
    switch (a.s.W) {
    case 128: launch_rows_block<128>(a, stream); break;
    case 256: launch_rows_block<256>(a, stream); break;
    case 512: launch_rows_block<512>(a, stream); break;
    default: launch_rows_block<1024>(a, stream); break;
    }
    (void)hipGetLastError();
}

}  // namespace meshgpt::kern
