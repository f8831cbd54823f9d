// Causal flash attention for prefill on the FP32 matrix cores of gfx950, with
// the XSA epilogue (reference.rs:510-554 attention, 577-603 exclusive self
// attention; the reference's GPU kernel is gpt_flash_forward, gpu.rs:381-498).
//
// One workgroup of eight waves (four at head width 32) takes 256 (128)
// queries of one (sequence, head); each wave owns 32 of them (two 16-query
// blocks).  Eight waves share each K/V tile among twice the queries and put
// four waves on every SIMD (two workgroups per CU, by LDS): config 4's
// prefill took 23.69 ms against 23.95 with four waves (and 24.8 with 32-key
// tiles, which let four workgroups share a CU).  Keys stream through LDS in
// tiles of 64 rows of K and V, double-buffered and loaded with direct-to-LDS
// loads (global_load_lds_dwordx4), so a tile lands while the previous one is
// multiplied.  Per tile and 16-query block a wave computes the transposed
// scores S^T = K Q^T with v_mfma_f32_16x16x4f32 (a 16-key x 16-query block per
// 16 instructions at head width 64): in the accumulator layout each lane then
// holds four keys of ONE query, which is exactly the B operand layout of the
// next product O^T = V^T P^T, so the probabilities go from the online softmax
// straight into the second product without leaving registers.  Each lane's
// output accumulators also belong to one query, so the softmax rescale is a
// per-lane multiply, and the softmax needs two cross-lane steps (the four
// lanes of a query) for the maximum, none for the running sum until the end.
//
// LDS rows are XOR-swizzled by 16-byte slot (slot ^ (row mod slots)), which
// keeps the K operand's 16-byte reads and the V operand's 4-byte reads free
// of bank conflicts without padding, so one load instruction fills four
// whole rows.  Scores are in the log2 domain (q pre-scaled by log2(e)/sqrt(hd)).
#include <hip/hip_runtime.h>

#include "kernels.hpp"

namespace meshgpt::kern {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) float lds_f32;

// (f64(1e-12f))^2 rounded to f32: the XSA norm floor of reference.rs:591.
constexpr float kXsaNormFloor = float(double(1e-12f) * double(1e-12f));

// D = A B + C for one 16x16x4 block: lane l supplies A[l % 16][l / 16] and
// B[l / 16][l % 16] and holds D[4 (l / 16) + r][l % 16] in element r.
__device__ __forceinline__ v4f mfma16(float a, float b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// LDS[base + 16 * lane .. +16) = g[0..4) for every lane of the wave; base is
// wave-uniform.  Earlier LDS reads complete first; m0 is preserved.
__device__ __forceinline__ void dma16(const float *g, float *base) {
    const uint32_t m = __builtin_amdgcn_readfirstlane(uint32_t(size_t((lds_f32 *)base)));
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

template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// A workgroup barrier that waits for LDS operations only (in-flight global
// loads, such as the next tile's, keep flying).
__device__ __forceinline__ void barrier_lds() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ float xor_lanes(float v, int mask) {
    return __shfl_xor(v, mask, 64);
}

template <int HD>
struct MfmaCfg {
    static constexpr int BK = 64;                 // keys per tile
    static constexpr int KB = BK / 16;            // 16-key blocks per tile
    static constexpr int NQB = 2;                 // 16-query blocks per wave
    static constexpr int WAVES = HD == 64 ? 8 : 4;
    static constexpr int QT = 16 * NQB * WAVES;   // queries per workgroup
    static constexpr int KS = HD / 4;             // k-steps of Q.K: dim = KS * (lane / 16) + step
    static constexpr int DB = HD / 16;            // 16-dim blocks of the output
    static constexpr int C4 = HD / 4;             // 16-byte slots per row
    static constexpr int TILE = BK * HD;          // floats of one K (or V) tile
    static constexpr int DMA_W = TILE / 256 / WAVES;  // load instructions per wave per tile
    static_assert(HD == 32 || HD == 64, "head widths of the matrix-core path");
};

// LDS float offset of (row, dim) in a swizzled tile of HD-float rows.
template <int HD>
__device__ __forceinline__ int swz(int row, int dim) {
    constexpr int C4 = HD / 4;
    return row * HD + 4 * ((dim >> 2) ^ (row & (C4 - 1))) + (dim & 3);
}

// Issues the loads of keys [t0, t0 + BK) (rows past n - 1 repeat row n - 1)
// of one cache slab into a swizzled LDS tile: wave w's instruction u fills
// floats [256 i, 256 i + 256) of the tile, i = w * DMA_W + u, lane l the 16
// bytes at 256 i + 4 l, which belong to row (256 i + 4 l) / HD.
template <int HD>
__device__ __forceinline__ void issue_tile(const float *slab, int t0, int n, float *tile, int wave, int lane) {
    using C = MfmaCfg<HD>;
#pragma unroll
    for (int u = 0; u < C::DMA_W; ++u) {
        const int i = wave * C::DMA_W + u;
        const int f = 256 * i + 4 * lane;
        const int row = f / HD, slot = (f % HD) / 4;
        const int c4 = slot ^ (row & (C::C4 - 1));
        const int key = min(t0 + row, n - 1);
        dma16(slab + size_t(key) * HD + 4 * c4, tile + 256 * i);
    }
}

// Workgroup i runs on XCD i % 8: the mapping of workgroups to (sequence,
// head) pairs and query tiles keeps every query tile of a pair on one XCD,
// consecutive on it and longest first, so the tiles that stream the same keys
// share that XCD's L2.
template <int HD>
__global__ void __launch_bounds__(64 * MfmaCfg<HD>::WAVES)
attn_prefill_mfma_kernel(Shape s, const float *__restrict__ q, KvView kv, int nseq, int n, float *__restrict__ y,
                         float scale_log2, int xsa) {
    using C = MfmaCfg<HD>;
    constexpr int BK = C::BK, KB = C::KB, NQB = C::NQB, KS = C::KS, DB = C::DB, C4 = C::C4, TILE = C::TILE;
    __shared__ __align__(16) float lds[4 * TILE];  // [stage][K, V]
    const int ntiles = (n + C::QT - 1) / C::QT;
    const int xcd = int(blockIdx.x) % 8, j8 = int(blockIdx.x) / 8;
    const int pair = xcd + 8 * (j8 / ntiles);
    const int qt = ntiles - 1 - j8 % ntiles;
    if (pair >= nseq * s.H) return;
    const int seq = pair / s.H, h = pair - seq * s.H;
    const int lane = int(threadIdx.x) & 63, wave = int(threadIdx.x) >> 6;
    const int jq = lane & 15, g = lane >> 4;
    const int qwave = qt * C::QT + wave * 16 * NQB;  // first query of this wave
    const int qlast_wg = min(qt * C::QT + C::QT, n) - 1;
    const size_t slab = size_t(pair) * kv.cap * HD;
    const float *kslab = kv.k + slab, *vslab = kv.v + slab;

    // B operand of S^T: lane holds q[query jq of block b][KS * g + step], scaled.
    float qop[NQB][KS];
#pragma unroll
    for (int b = 0; b < NQB; ++b) {
        const int qi = min(qwave + 16 * b + jq, n - 1);
        const float4 *src = reinterpret_cast<const float4 *>(q + (size_t(seq) * n + qi) * s.W + h * HD + KS * g);
#pragma unroll
        for (int t = 0; t < KS / 4; ++t) {
            const float4 v = src[t];
            qop[b][4 * t] = v.x * scale_log2;
            qop[b][4 * t + 1] = v.y * scale_log2;
            qop[b][4 * t + 2] = v.z * scale_log2;
            qop[b][4 * t + 3] = v.w * scale_log2;
        }
    }

    v4f oacc[NQB][DB];
    float m[NQB], l[NQB];
#pragma unroll
    for (int b = 0; b < NQB; ++b) {
        m[b] = -INFINITY;
        l[b] = 0.0f;
#pragma unroll
        for (int d = 0; d < DB; ++d) oacc[b][d] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    }

    const int ntile = qlast_wg / BK + 1;
    issue_tile<HD>(kslab, 0, n, lds, wave, lane);
    issue_tile<HD>(vslab, 0, n, lds + TILE, wave, lane);
    for (int t = 0; t < ntile; ++t) {
        if (t + 1 < ntile) {
            float *next = lds + ((t + 1) & 1) * 2 * TILE;
            issue_tile<HD>(kslab, (t + 1) * BK, n, next, wave, lane);
            issue_tile<HD>(vslab, (t + 1) * BK, n, next + TILE, wave, lane);
            wait_vm<2 * C::DMA_W>();
        } else {
            wait_vm<0>();
        }
        barrier_lds();
        const int t0 = t * BK;
        // A wave whose queries all precede the tile has nothing to add.
        if (t0 <= qwave + 16 * NQB - 1) {
            const float *Ks = lds + (t & 1) * 2 * TILE, *Vs = Ks + TILE;
            // S^T blocks: keys kb*16 + 4g + r against this lane's query.
            float kop[KB][KS];
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                const int row = kb * 16 + jq;
#pragma unroll
                for (int tt = 0; tt < KS / 4; ++tt) {
                    const float4 v = *reinterpret_cast<const float4 *>(
                        Ks + row * HD + 4 * (((KS / 4) * g + tt) ^ (row & (C4 - 1))));
                    kop[kb][4 * tt] = v.x;
                    kop[kb][4 * tt + 1] = v.y;
                    kop[kb][4 * tt + 2] = v.z;
                    kop[kb][4 * tt + 3] = v.w;
                }
            }
            v4f sacc[KB][NQB];
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                for (int b = 0; b < NQB; ++b) sacc[kb][b] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int st = 0; st < KS; ++st)
#pragma unroll
                for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                    for (int b = 0; b < NQB; ++b) sacc[kb][b] = mfma16(kop[kb][st], qop[b][st], sacc[kb][b]);
            // Online softmax per query; the causal mask only on tiles that
            // reach past the wave's first query.
            const bool diag = t0 + BK - 1 > qwave;
#pragma unroll
            for (int b = 0; b < NQB; ++b) {
                const int qi = qwave + 16 * b + jq;
                float mx = -INFINITY;
#pragma unroll
                for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float sc = sacc[kb][b][r];
                        if (diag && t0 + kb * 16 + 4 * g + r > qi) sc = -INFINITY;
                        sacc[kb][b][r] = sc;
                        mx = fmaxf(mx, sc);
                    }
                mx = fmaxf(mx, xor_lanes(mx, 16));
                mx = fmaxf(mx, xor_lanes(mx, 32));
                const float mn = fmaxf(m[b], mx);
                const float alpha = __builtin_amdgcn_exp2f(m[b] - mn);
                float ps = 0.0f;
#pragma unroll
                for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float p = __builtin_amdgcn_exp2f(sacc[kb][b][r] - mn);
                        sacc[kb][b][r] = p;
                        ps += p;
                    }
                l[b] = l[b] * alpha + ps;
                m[b] = mn;
#pragma unroll
                for (int d = 0; d < DB; ++d) oacc[b][d] *= alpha;
            }
            // O^T += V^T P^T: k-step (kb, r) pairs lane group g with key
            // kb*16 + 4g + r, the key whose probability the lane holds.
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = kb * 16 + 4 * g + r;
                    float vop[DB];
#pragma unroll
                    for (int d = 0; d < DB; ++d) vop[d] = Vs[swz<HD>(row, d * 16 + jq)];
#pragma unroll
                    for (int b = 0; b < NQB; ++b)
#pragma unroll
                        for (int d = 0; d < DB; ++d) oacc[b][d] = mfma16(vop[d], sacc[kb][b][r], oacc[b][d]);
                }
        }
        barrier_lds();  // the stage is free for the tile after next
    }

    // Epilogue: y = O / l, then XSA against the query's own value row.
#pragma unroll
    for (int b = 0; b < NQB; ++b) {
        const int qi = qwave + 16 * b + jq;
        float L = l[b];
        L += xor_lanes(L, 16);
        L += xor_lanes(L, 32);
        const float inv = 1.0f / L;
        const int qc = min(qi, n - 1);
        float yv[DB][4], vv[DB][4];
        float dot = 0.0f, vsq = 0.0f;
#pragma unroll
        for (int d = 0; d < DB; ++d) {
            const float4 v4 = *reinterpret_cast<const float4 *>(vslab + size_t(qc) * HD + d * 16 + 4 * g);
            const float vr[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                yv[d][r] = oacc[b][d][r] * inv;
                vv[d][r] = vr[r];
                dot = fmaf(yv[d][r], vr[r], dot);
                vsq = fmaf(vr[r], vr[r], vsq);
            }
        }
        dot += xor_lanes(dot, 16);
        dot += xor_lanes(dot, 32);
        vsq += xor_lanes(vsq, 16);
        vsq += xor_lanes(vsq, 32);
        const float iv = rsqrtf(fmaxf(vsq, kXsaNormFloor));
        const float c = xsa ? dot * iv : 0.0f;
        if (qi < n) {
#pragma unroll
            for (int d = 0; d < DB; ++d) {
                float4 o;
                o.x = yv[d][0] - c * (vv[d][0] * iv);
                o.y = yv[d][1] - c * (vv[d][1] * iv);
                o.z = yv[d][2] - c * (vv[d][2] * iv);
                o.w = yv[d][3] - c * (vv[d][3] * iv);
                *reinterpret_cast<float4 *>(y + (size_t(seq) * n + qi) * s.W + h * HD + d * 16 + 4 * g) = o;
            }
        }
    }
}

// Causal attention for short sequences (a few rows each), one thread per
// (row, head): the row's query against the keys at positions 0..pos of its
// (sequence, head) slab with the online softmax of reference.rs:510-554, in
// the log2 domain, then the XSA of reference.rs:577-603 against the value row
// at pos.  Each thread reads whole 128-byte (hd 32) or 256-byte (hd 64) rows.
template <int HD>
__global__ void __launch_bounds__(256)
attn_short_kernel(Shape s, const float *__restrict__ q, KvView kv, int rows, int n, float *__restrict__ y,
                  float scale_log2, int xsa) {
    const int i = int(blockIdx.x) * 256 + int(threadIdx.x);
    if (i >= rows * s.H) return;
    const int h = i % s.H, row = i / s.H, seq = row / n, pos = row - seq * n;
    const size_t slab = size_t(seq * s.H + h) * kv.cap * HD;
    float qv[HD], acc[HD], vrow[HD];
    const float4 *q4 = reinterpret_cast<const float4 *>(q + size_t(row) * s.W + h * HD);
#pragma unroll
    for (int e = 0; e < HD / 4; ++e) {
        const float4 t = q4[e];
        qv[4 * e] = t.x * scale_log2;
        qv[4 * e + 1] = t.y * scale_log2;
        qv[4 * e + 2] = t.z * scale_log2;
        qv[4 * e + 3] = t.w * scale_log2;
    }
#pragma unroll
    for (int e = 0; e < HD; ++e) acc[e] = 0.0f;
    float m = -INFINITY, l = 0.0f;
    for (int j = 0; j <= pos; ++j) {
        const float4 *k4 = reinterpret_cast<const float4 *>(kv.k + slab + size_t(j) * HD);
        const float4 *v4 = reinterpret_cast<const float4 *>(kv.v + slab + size_t(j) * HD);
        float sc = 0.0f;
#pragma unroll
        for (int e = 0; e < HD / 4; ++e) {
            const float4 t = k4[e];
            sc = fmaf(qv[4 * e], t.x, sc);
            sc = fmaf(qv[4 * e + 1], t.y, sc);
            sc = fmaf(qv[4 * e + 2], t.z, sc);
            sc = fmaf(qv[4 * e + 3], t.w, sc);
        }
#pragma unroll
        for (int e = 0; e < HD / 4; ++e) {
            const float4 t = v4[e];
            vrow[4 * e] = t.x;
            vrow[4 * e + 1] = t.y;
            vrow[4 * e + 2] = t.z;
            vrow[4 * e + 3] = t.w;
        }
        const float mn = fmaxf(m, sc);
        const float alpha = __builtin_amdgcn_exp2f(m - mn), p = __builtin_amdgcn_exp2f(sc - mn);
        l = l * alpha + p;
#pragma unroll
        for (int e = 0; e < HD; ++e) acc[e] = fmaf(p, vrow[e], acc[e] * alpha);
        m = mn;
    }
    // vrow now holds the value row at pos, the XSA direction.
    const float inv = 1.0f / l;
    float dot = 0.0f, vsq = 0.0f;
#pragma unroll
    for (int e = 0; e < HD; ++e) {
        acc[e] *= inv;
        dot = fmaf(acc[e], vrow[e], dot);
        vsq = fmaf(vrow[e], vrow[e], vsq);
    }
    const float iv = rsqrtf(fmaxf(vsq, kXsaNormFloor));
    const float c = xsa ? dot * iv : 0.0f;
    float4 *y4 = reinterpret_cast<float4 *>(y + size_t(row) * s.W + h * HD);
#pragma unroll
    for (int e = 0; e < HD / 4; ++e)
        y4[e] = make_float4(acc[4 * e] - c * (vrow[4 * e] * iv), acc[4 * e + 1] - c * (vrow[4 * e + 1] * iv),
                            acc[4 * e + 2] - c * (vrow[4 * e + 2] * iv), acc[4 * e + 3] - c * (vrow[4 * e + 3] * iv));
}

}  // namespace

bool attn_prefill_short_supported(const Shape &s, int rows_per_seq) {
    return s.hd == s.hdp && (s.hd == 32 || s.hd == 64) && s.W % 4 == 0 && rows_per_seq <= 16;
}

void attn_prefill_short(const Shape &s, const float *q, KvView kv, int nseq, int rows_per_seq, float *y, int xsa,
                        hipStream_t stream) {
    const float scale_log2 = float(1.4426950408889634 / std::sqrt(double(s.hd)));
    const int rows = nseq * rows_per_seq, blocks = (rows * s.H + 255) / 256;
    if (s.hd == 32)
        hipLaunchKernelGGL(attn_short_kernel<32>, dim3(blocks), dim3(256), 0, stream, s, q, kv, rows, rows_per_seq,
                           y, scale_log2, xsa);
    else
        hipLaunchKernelGGL(attn_short_kernel<64>, dim3(blocks), dim3(256), 0, stream, s, q, kv, rows, rows_per_seq,
                           y, scale_log2, xsa);
    (void)hipGetLastError();
}

bool attn_prefill_mfma_supported(const Shape &s, int rows_per_seq) {
    return s.hd == s.hdp && (s.hd == 32 || s.hd == 64) && s.W % 4 == 0 && rows_per_seq >= 64;
}

void attn_prefill_mfma(const Shape &s, const float *q, KvView kv, int nseq, int rows_per_seq, float *y, int xsa,
                       hipStream_t stream) {
    const float scale_log2 = float(1.4426950408889634 / std::sqrt(double(s.hd)));
    auto launch = [&](auto kernel, int qt, int waves) {
        const int ntiles = (rows_per_seq + qt - 1) / qt;
        const int px = (nseq * s.H + 7) / 8;
        hipLaunchKernelGGL(kernel, dim3(8 * px * ntiles), dim3(64 * waves), 0, stream, s, q, kv, nseq,
                           rows_per_seq, y, scale_log2, xsa);
    };
    if (s.hd == 32)
        launch(attn_prefill_mfma_kernel<32>, MfmaCfg<32>::QT, MfmaCfg<32>::WAVES);
    else
        launch(attn_prefill_mfma_kernel<64>, MfmaCfg<64>::QT, MfmaCfg<64>::WAVES);
    (void)hipGetLastError();
}

}  // namespace meshgpt::kern
