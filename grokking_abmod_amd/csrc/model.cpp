// Host orchestration of the device-resident Mesh GPT: buffers, the prefill and
// decode sequences of kernel launches, and the HIP graph that replays one
// decode step.
#include "model.hpp"
#include "train.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>

#include "kernels.hpp"

namespace meshgpt {
namespace {

void check(hipError_t e, const char *what) {
    if (e != hipSuccess)
        throw Error(std::string(what) + ": " + hipGetErrorString(e),
                    e == hipErrorOutOfMemory ? kOutOfMemory : kDeviceError);
}

struct DevBuf {
    void *p = nullptr;
    size_t bytes = 0;
    DevBuf() = default;
    DevBuf(const DevBuf &) = delete;
    DevBuf &operator=(const DevBuf &) = delete;
    ~DevBuf() { release(); }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        bytes = 0;
    }
    // Returns true when the buffer was (re)allocated.
    bool ensure(size_t n) {
        if (n <= bytes && p) return false;
        release();
        check(hipMalloc(&p, std::max<size_t>(n, 256)), "hipMalloc");
        bytes = std::max<size_t>(n, 256);
        return true;
    }
    template <class T>
    T *as() const {
        return static_cast<T *>(p);
    }
};

// Page-locked host memory (hipHostMalloc) for the training step's uploads and
// its loss, so that each is one DMA copy.
struct PinnedBuf {
    void *p = nullptr;
    size_t bytes = 0;
    PinnedBuf() = default;
    PinnedBuf(const PinnedBuf &) = delete;
    PinnedBuf &operator=(const PinnedBuf &) = delete;
    ~PinnedBuf() { release(); }
    void release() {
        if (p) (void)hipHostFree(p);
        p = nullptr;
        bytes = 0;
    }
    void ensure(size_t n) {
        if (n <= bytes && p) return;
        release();
        check(hipHostMalloc(&p, std::max<size_t>(n, 256), hipHostMallocDefault), "hipHostMalloc");
        bytes = std::max<size_t>(n, 256);
    }
    template <class T>
    T *as() const {
        return static_cast<T *>(p);
    }
};

int floor_log2(size_t x) {
    int r = 0;
    while (x >>= 1) ++r;
    return r;
}

size_t next_pow2(size_t x) {
    size_t p = 1;
    while (p < x) p <<= 1;
    return p;
}

int env_int(const char *name, int fallback) {
    const char *v = std::getenv(name);
    return v && *v ? std::atoi(v) : fallback;
}

constexpr size_t kNoCache = size_t(-1);

}  // namespace

struct MeshGpt::Impl {
    int device = 0;
    hipStream_t stream = nullptr;
    GptConfig cfg;
    Layout layout;
    kern::Shape shape{};
    int vpad = 0;  // vocabulary rounded up to a multiple of 4: the row stride of Et
    size_t lds_limit = 65536;

    DevBuf params, codes, E, Et, rope;
    // Row-order copies of the block weights and token vectors for the row
    // decode kernel (kern::row_order).
    DevBuf wdec, Edec;
    DevBuf q0;  // persistent decode: layer-0 Q/K/V meshes of every token

    // Decode state: KV cache [L][batch_cap][H][context][hdp], per-sequence
    // tokens [batch_cap][tcap], lengths, SplitMix64 states and logits.
    size_t batch_cap = 0, tcap = 0;
    DevBuf kc, vc, dx, dx2, dxn, dq, part, dtokens, dlen, drng, dlogits, dflags;
    // Sampler states and length right after the last prefill (rewind()).
    DevBuf drng_start;
    // Sampler states a persistent decode launch writes (swapped with drng when
    // the launch completes).
    DevBuf drng_next;
    size_t start_length = 0;
    // Persistent decode kernel state: tagged exchange words of every sequence
    // and the abort flag.
    DevBuf pxch, pabort;
    size_t batch = 0, length = 0, cached = kNoCache;
    float temperature = 0.0f;

    // Prefill / logits workspace, grown on demand.
    DevBuf wx, wxn, wq, wy, wtok, wlogits, wk, wv;

    // Decode graphs replaying 1 and kGraphSteps steps.
    static constexpr size_t kGraphSteps = 8;
    hipGraph_t graph[2] = {nullptr, nullptr};
    hipGraphExec_t exec[2] = {nullptr, nullptr};
    size_t graph_batch = 0;
    float graph_temperature = -1.0f;
    int graph_slices = 0;
    bool use_graph = true;
    // Decode blocks run on the row-order kernel when the shape allows it, else
    // on the one-wave-per-mesh kernel, else on the general block kernel
    // (MG_DISABLE_ROW_DECODE=1 / MG_DISABLE_WAVE_DECODE=1 skip the first two).
    bool row_decode = false;
    bool wave_decode = false;
    // Decode steps run in one persistent launch when the shape and batch allow
    // it (MG_DISABLE_PERSISTENT=1 keeps the per-phase kernels).
    bool persistent_ok = false;
    bool use_mfma_prefill = true;
    bool use_rows_prefill = true;
    bool use_short_prefill = true;

    // Training (gpu.rs:1915-2003): the activations of the last forward, the
    // gradient, AdamW's moments and the running powers of its betas (reset
    // with the weights, gpu.rs:1856-1872).
    // Training: activations, gradient, AdamW moments, reduction scratch, and
    // the step's inputs (StepScalars, then the n tokens, then the n targets)
    // with their pinned host staging (the same layout, then the n row losses).
    DevBuf tact, tgrad, tm, tv, tpart, tin;
    PinnedBuf tstage;
    static constexpr size_t kTrainTokensAt = 256;
    kern::train::StepScalars hyper{};  // host copy uploaded before each step (kept alive for the async copy)
    float beta1_power = 1.0f, beta2_power = 1.0f;
    bool derived_stale = false;  // E and the decode tables lag the weights
    // The captured training step and what it was captured for.
    struct TrainKey {
        size_t n = 0, sequence = 0;
        float lr = 0, wd = 0, b1 = 0, b2 = 0, eps = 0;
        bool operator==(const TrainKey &o) const {
            return n == o.n && sequence == o.sequence && lr == o.lr && wd == o.wd && b1 == o.b1 && b2 == o.b2 &&
                   eps == o.eps;
        }
    } tkey;
    hipGraph_t tgraph = nullptr;
    hipGraphExec_t texec = nullptr;

    // Events around the kernels of the last logits / hidden_states / prefill
    // call (last_call_ms).
    hipEvent_t call_ev[2] = {nullptr, nullptr};
    float call_ms = 0.0f;

    // Per-phase decode of a large batch runs as independent slices of the
    // batch on the model's stream and kMaxSlices - 1 more (default priority),
    // forked from and joined to the model's stream once per graph replay.
    static constexpr int kMaxSlices = 4;
    hipStream_t slice_stream[kMaxSlices - 1] = {};
    hipEvent_t fork_ev = nullptr, join_ev[kMaxSlices - 1] = {};

    ~Impl() {
        drop_graph();
        drop_train_graph();
        for (hipEvent_t e : call_ev)
            if (e) (void)hipEventDestroy(e);
        for (int i = 0; i < kMaxSlices - 1; ++i) {
            if (join_ev[i]) (void)hipEventDestroy(join_ev[i]);
            if (slice_stream[i]) (void)hipStreamDestroy(slice_stream[i]);
        }
        if (fork_ev) (void)hipEventDestroy(fork_ev);
        if (stream) (void)hipStreamDestroy(stream);
    }

    void mark_call(int which) { check(hipEventRecord(call_ev[which], stream), "hipEventRecord"); }

    // After the call's sync: the time between its two marks.
    void close_call() { check(hipEventElapsedTime(&call_ms, call_ev[0], call_ev[1]), "hipEventElapsedTime"); }

    void activate() const { check(hipSetDevice(device), "hipSetDevice"); }

    void drop_graph() {
        for (int i = 0; i < 2; ++i) {
            if (exec[i]) (void)hipGraphExecDestroy(exec[i]);
            if (graph[i]) (void)hipGraphDestroy(graph[i]);
            exec[i] = nullptr;
            graph[i] = nullptr;
        }
        graph_batch = 0;
    }

    size_t layer_cache_elems() const {
        return batch_cap * size_t(shape.H) * cfg.context * size_t(shape.hdp);
    }

    // Splits per (sequence, head) of decode attention: about 512 workgroups
    // for the batch (two per CU).  More, shorter shares measured slower at
    // B=32 H=8: each workgroup's first loads are latency-bound, and the merge
    // in the next block launch grows with the split count.
    int splits_for(size_t b) const {
        const int forced = env_int("MG_DECODE_SPLITS", 0);
        if (forced > 0) return std::min(forced, 256);
        const size_t want = 512 / std::max<size_t>(b * cfg.heads, 1);
        return int(std::max<size_t>(1, std::min<size_t>({want, 64, cfg.context})));
    }

    // Rows per workgroup and team count of block_kernel.  Decode runs one row
    // per workgroup with the Q/K/V meshes in three concurrent teams; prefill
    // packs rows so mesh weights are reused, keeping at least 256 workgroups.
    // Row buffers are sized without the weight stage, which each launch adds
    // when it fits (staged()).
    struct BlockTiling {
        int rpw, teams;
    };
    BlockTiling block_tiling(size_t rows, bool decode) const {
        const size_t budget = decode ? lds_limit : std::min<size_t>(lds_limit, 49152);
        for (int teams : {3, 1}) {
            int rpw = decode ? 1 : 16;
            while (rpw > 1 && ((rows + rpw - 1) / rpw < 256 ||
                               kern::block_lds_bytes(shape, rpw, teams, false, true, true) > budget))
                rpw /= 2;
            if (kern::block_lds_bytes(shape, rpw, teams, false, true, true) <= budget) return {rpw, teams};
        }
        throw Error("model width exceeds the workgroup LDS budget", kUnsupported);
    }

    bool staged(const BlockTiling &t, bool post, bool pre) const {
        return env_int("MG_DISABLE_STAGING", 0) == 0 && kern::block_can_stage(shape, t.teams, post, pre) &&
               kern::block_lds_bytes(shape, t.rpw, t.teams, true, post, pre) <= lds_limit;
    }

    int mesh_rows_per_group(size_t rows) const {
        int rpw = 16;
        while (rpw > 1 && ((rows + rpw - 1) / rpw < 64 || kern::mesh_lds_bytes(shape, rpw) > 49152)) rpw /= 2;
        if (kern::mesh_lds_bytes(shape, rpw) > lds_limit)
            throw Error("model width exceeds the workgroup LDS budget", kUnsupported);
        return rpw;
    }

    int head_rows() const {
        int rt = 8;
        while (rt > 1 && kern::head_lds_bytes(shape, rt) > lds_limit) rt /= 2;
        return rt;
    }

    void init(int dev, const GptConfig &config, uint64_t seed, size_t max_batch) {
        config.validate();
        cfg = config;
        layout = Layout::build(cfg);
        device = dev;
        int count = 0;
        check(hipGetDeviceCount(&count), "hipGetDeviceCount");
        if (dev < 0 || dev >= count) throw Error("invalid device ordinal", kDeviceError);
        activate();
        int lds = 0;
        check(hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev), "LDS query");
        lds_limit = size_t(lds);
        kern::configure_lds(lds_limit);
        check(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreate");
        for (hipEvent_t &e : call_ev) check(hipEventCreate(&e), "hipEventCreate");
        use_graph = env_int("MG_DISABLE_GRAPH", 0) == 0;

        const size_t W = cfg.width, hd = cfg.head_width();
        shape.W = int(W);
        shape.H = int(cfg.heads);
        shape.hd = int(hd);
        shape.hdp = int(next_pow2(hd));
        shape.half = int(hd / 2);
        shape.V = int(cfg.vocab_size);
        shape.log2w = floor_log2(W);
        shape.wshift = (W & (W - 1)) == 0 ? floor_log2(W) : -1;
        shape.hdshift = (hd & (hd - 1)) == 0 ? floor_log2(hd) : -1;
        shape.butterfly = cfg.connectivity == MeshConnectivity::Butterfly ? 1 : 0;
        shape.A = int(cfg.attention_mesh_depth);
        shape.F = int(cfg.ffn_mesh_depth);
        shape.rope = cfg.rope;
        shape.qk_norm = cfg.qk_norm;
        shape.xsa = cfg.xsa;
        const bool all_operators = cfg.rope && cfg.qk_norm && cfg.xsa;
        wave_decode = env_int("MG_DISABLE_WAVE_DECODE", 0) == 0 && kern::block_decode_supported(shape);
        // The row-order and persistent decode kernels run every operator;
        // operator ablations decode on the one-wave or general block kernels.
        row_decode = all_operators && env_int("MG_DISABLE_ROW_DECODE", 0) == 0 && kern::row_block_supported(shape);
        persistent_ok = row_decode && env_int("MG_DISABLE_PERSISTENT", 0) == 0;
        use_mfma_prefill = env_int("MG_DISABLE_MFMA_PREFILL", 0) == 0;
        use_rows_prefill = env_int("MG_DISABLE_ROWS_PREFILL", 0) == 0;
        use_short_prefill = env_int("MG_DISABLE_SHORT_PREFILL", 0) == 0;

        const size_t C = cfg.context;

        // RoPE angles pos / 10000^(i / half) in f64 (reference.rs:468-470), stored as f32.
        std::vector<float> table(C * shape.half * 2);
        for (size_t pos = 0; pos < C; ++pos)
            for (int i = 0; i < shape.half; ++i) {
                const double angle =
                    double(pos) / std::pow(double(kRopeBase), double(i) / double(shape.half));
                table[2 * (pos * shape.half + i)] = float(std::cos(angle));
                table[2 * (pos * shape.half + i) + 1] = float(std::sin(angle));
            }
        rope.ensure(table.size() * 4);
        check(hipMemcpy(rope.p, table.data(), table.size() * 4, hipMemcpyHostToDevice), "upload rope");

        std::vector<float> c = token_codes(cfg);
        codes.ensure(c.size() * 4);
        check(hipMemcpy(codes.p, c.data(), c.size() * 4, hipMemcpyHostToDevice), "upload codes");
        E.ensure(W * cfg.vocab_size * 4);
        vpad = int((cfg.vocab_size + 3) / 4 * 4);
        Et.ensure(W * size_t(vpad) * 4);
        params.ensure(layout.count() * 4);
        std::vector<float> initial = layout.initialize(cfg, seed);
        set_parameters(initial.data(), initial.size());
        ensure_decode(std::max<size_t>(max_batch, 1), 1);
    }

    void set_parameters(const float *values, size_t n) {
        if (n != layout.count()) throw Error("parameter count does not match GPT configuration");
        validate_finite(values, n, "parameters");
        layout.validate_constraints(cfg, values);
        activate();
        check(hipMemcpyAsync(params.p, values, n * 4, hipMemcpyHostToDevice, stream), "upload parameters");
        reset_optimizer();
        refresh_derived();
    }

    // Tables derived from the weights (E, its transpose, the row-order copies
    // and the layer-0 table): rebuilt when the weights change, not per token.
    // After training steps they are rebuilt before the next inference call.
    void ensure_derived() {
        if (!derived_stale) return;
        activate();
        refresh_derived();
    }

    void refresh_derived() {
        const size_t n = layout.count();
        // The token vectors depend only on the weights: computed once here, not per token.
        if (cfg.embedding == TokenEmbedding::Mesh) {
            kern::mesh_rows(shape, codes.as<float>(), E.as<float>(), shape.V, params.as<float>(), shape.A,
                            mesh_rows_per_group(cfg.vocab_size), stream);
        } else {
            check(hipMemcpyAsync(E.p, params.p, cfg.vocab_size * cfg.width * 4, hipMemcpyDeviceToDevice,
                                 stream),
                  "copy table");
        }
        // The geometry's normalisation or protected coordinates (reference.rs:130-149).
        if (cfg.geometry.transformed())
            kern::embedding_geometry(E.as<float>(), codes.as<float>(), shape.V, shape.W,
                                     cfg.geometry.radius(cfg.width),
                                     cfg.geometry.normalization != EmbeddingNorm::None ? 1 : 0,
                                     int(cfg.geometry.preserve_features), stream);
        kern::transpose(E.as<float>(), Et.as<float>(), shape.V, vpad, shape.W, stream);
        if (row_decode) {
            const size_t emb = cfg.embedding_parameter_count();
            const size_t block_rows = cfg.layers * (4 * cfg.attention_mesh_depth + cfg.ffn_mesh_depth);
            wdec.ensure(n * 4);
            Edec.ensure(cfg.vocab_size * cfg.width * 4);
            kern::row_order(E.as<float>(), Edec.as<float>(), shape.V, shape.W, false, stream);
            kern::row_order(params.as<float>() + emb, wdec.as<float>() + emb, int(block_rows), shape.W, true,
                            stream);
            if (persistent_ok) {
                q0.ensure(kern::persistent_layer0_floats(shape) * 4);
                kern::persistent_layer0(shape, Edec.as<float>(), wdec.as<float>(),
                                        layout.groups[layout.blocks[0].query].offset, q0.as<float>(), stream);
            }
        }
        sync();
        derived_stale = false;
    }

    void sync() {
        check(hipGetLastError(), "kernel launch");
        check(hipStreamSynchronize(stream), "hipStreamSynchronize");
    }

    void ensure_decode(size_t b, size_t t) {
        const bool grow_b = b > batch_cap, grow_t = t > tcap;
        if (!grow_b && !grow_t) return;
        sync();
        drop_graph();
        if (grow_b) {
            batch_cap = std::max(b, batch_cap);
            const size_t cache = size_t(cfg.layers) * layer_cache_elems() * 4;
            kc.ensure(cache);
            vc.ensure(cache);
            // Padding lanes (hd < hdp) are read by vector loads and must stay zero.
            check(hipMemsetAsync(kc.p, 0, cache, stream), "zero cache");
            check(hipMemsetAsync(vc.p, 0, cache, stream), "zero cache");
            dx.ensure(batch_cap * cfg.width * 4);
            dx2.ensure(batch_cap * cfg.width * 4);
            dxn.ensure(batch_cap * cfg.width * 4);
            dq.ensure(batch_cap * cfg.width * 4);
            // Partial states of the decode attention: for a batch of k, or k in
            // up to kMaxSlices slices (each at least k / kMaxSlices sequences,
            // and the split count never grows with the batch).
            size_t slots = 0;
            for (size_t k = 1; k <= batch_cap; ++k)
                slots = std::max(slots, k * size_t(splits_for(std::max<size_t>(1, k / kMaxSlices))));
            part.ensure(slots * cfg.heads * (shape.hdp + 2) * 4);
            dlen.ensure(batch_cap * 4);
            drng.ensure(batch_cap * 8);
            drng_start.ensure(batch_cap * 8);
            drng_next.ensure(batch_cap * 8);
            dlogits.ensure(batch_cap * cfg.vocab_size * 4);
            dflags.ensure(4);
            if (persistent_ok) {
                pxch.ensure(batch_cap * kern::persistent_exchange_words(shape) * 8);
                pabort.ensure(8);  // abort flag, then the launch's non-finite flag
            }
        }
        tcap = std::max(t, tcap);
        dtokens.release();
        dtokens.ensure(batch_cap * tcap * 4);
        cached = kNoCache;
        length = 0;
        sync();
    }

    void ensure_workspace(size_t rows, size_t out_rows, bool kv) {
        const size_t W = cfg.width;
        wx.ensure(rows * W * 4);
        wxn.ensure(rows * W * 4);
        wq.ensure(rows * W * 4);
        wy.ensure(rows * W * 4);
        wtok.ensure(rows * 4);
        wlogits.ensure(out_rows * cfg.vocab_size * 4);
        if (kv) {
            const size_t bytes = rows * cfg.heads * size_t(shape.hdp) * 4;
            if (wk.ensure(bytes)) check(hipMemsetAsync(wk.p, 0, wk.bytes, stream), "zero kv");
            if (wv.ensure(bytes)) check(hipMemsetAsync(wv.p, 0, wv.bytes, stream), "zero kv");
        }
    }

    const float *group(size_t id) const { return params.as<float>() + layout.groups[id].offset; }
    const float *group_rows(size_t id) const { return wdec.as<float>() + layout.groups[id].offset; }

    // Every block over `rows`: L+1 block_kernel launches (the first also embeds
    // the tokens, the last writes the final RMSNorm rows to xn) with each
    // block's attention between them.  kv_of(l) is block l's cache view.  With
    // `events`, each decode-attention launch stamps its own begin and end into
    // events[2l] and events[2l+1].
    template <class KvOf>
    // `part_base` is the decode attention's partial-state buffer (default: the
    // start of `part`).
    void run_blocks(const kern::Rows &rows, int nseq, KvOf kv_of, float *x, float *x2, float *q, float *y,
                    float *xn, bool decode, hipEvent_t *events = nullptr, float *part_base = nullptr) {
        if (!part_base) part_base = part.as<float>();
        const int nsplit = decode ? splits_for(size_t(rows.rows)) : 0;
        // Prefill attention on the matrix cores (XSA in its epilogue) where the
        // shape allows it (MG_DISABLE_MFMA_PREFILL=1 keeps the VALU kernel).
        const bool mfma_prefill = !decode && use_mfma_prefill &&
                                  kern::attn_prefill_mfma_supported(shape, rows.rows_per_seq);
        // Short sequences: one thread per (row, head) (MG_DISABLE_SHORT_PREFILL=1
        // keeps the VALU flash kernel).
        const bool short_prefill = !decode && use_short_prefill &&
                                   kern::attn_prefill_short_supported(shape, rows.rows_per_seq);
        // Prefill blocks on the register-tile kernel where the shape allows it
        // (MG_DISABLE_ROWS_PREFILL=1 keeps block_kernel).
        const bool rows_prefill = use_rows_prefill && kern::rows_block_supported(shape) && rows.len == nullptr;
        const BlockTiling t = block_tiling(size_t(rows.rows), decode);
        const size_t L = cfg.layers;
        const bool rows_order = decode && row_decode;
        auto weights = [&](size_t id) { return rows_order ? group_rows(id) : group(id); };
        // The row-order kernel reads the residual rows from one buffer and
        // writes them to the other (kern::BlockArgs::x_out); the rest update in place.
        float *xin = x, *xout = rows_order ? x2 : x;
        for (size_t l = 0; l <= L; ++l) {
            kern::BlockArgs a{};
            a.s = shape;
            a.ro = rows;
            a.x = xin;
            a.x_out = xout;
            a.rpw = t.rpw;
            a.teams = t.teams;
            if (l > 0) {
                const Block &prev = layout.blocks[l - 1];
                a.wproj = weights(prev.projection);
                a.wffn = weights(prev.ffn);
                a.part = decode ? part_base : nullptr;
                a.nsplit = nsplit;
                a.ybuf = decode ? nullptr : y;
                a.xsa_post = cfg.xsa && (decode || !(mfma_prefill || short_prefill)) ? 1 : 0;
                a.kv_post = kv_of(l - 1);
            }
            if (l < L) {
                const Block &blk = layout.blocks[l];
                a.wq = weights(blk.query);
                a.wk = weights(blk.key);
                a.wv = weights(blk.value);
                a.E = rows_order ? Edec.as<float>() : E.as<float>();
                a.embed = l == 0;
                a.q = q;
                a.kv_pre = kv_of(l);
                a.rope = rope.as<float2>();
            } else {
                a.xn = xn;
            }
            if (rows_order) {
                if (xout == xin) throw Error("row-order decode needs two residual buffers", kDeviceError);
                kern::row_block(a, stream);
                std::swap(xin, xout);
            }
            else if (decode && wave_decode)
                kern::block_decode(a, stream);
            else if (!decode && rows_prefill)
                kern::rows_block(a, stream);
            else
                kern::block(a, staged(t, a.wproj != nullptr, a.wq != nullptr), stream);
            if (l == L) break;
            if (decode) {
                kern::attn_decode(shape, q, kv_of(l), rows.len, rows.rows, nsplit, part_base, stream,
                                  events ? events[2 * l] : nullptr, events ? events[2 * l + 1] : nullptr);
            } else if (mfma_prefill) {
                kern::attn_prefill_mfma(shape, q, kv_of(l), nseq, rows.rows_per_seq, y, cfg.xsa, stream);
            } else if (short_prefill) {
                kern::attn_prefill_short(shape, q, kv_of(l), nseq, rows.rows_per_seq, y, cfg.xsa, stream);
            } else {
                kern::attn_prefill(shape, q, kv_of(l), nseq, rows.rows_per_seq, y, stream);
            }
        }
    }

    // Rows of each cached slab that decode attention reads with the default
    // cache policy (kern::kv_keep_rows; MG_KV_KEEP_ROWS overrides it).
    int keep_rows() const {
        return env_int("MG_KV_KEEP_ROWS", kern::kv_keep_rows(shape, int(std::max<size_t>(batch, 1)), int(cfg.layers)));
    }

    kern::KvView cache_layer(size_t l) const {
        const size_t off = l * layer_cache_elems();
        return kern::KvView{kc.as<float>() + off, vc.as<float>() + off, int(cfg.context), keep_rows()};
    }

    // Forward over a flat batch of sequences with a one-layer KV workspace
    // (each block's keys are consumed before the next block overwrites them).
    void forward_rows(const uint32_t *tokens, size_t n, size_t sequence, size_t out_rows) {
        ensure_workspace(n, out_rows, true);
        check(hipMemcpyAsync(wtok.p, tokens, n * 4, hipMemcpyHostToDevice, stream), "upload tokens");
        mark_call(0);
        kern::Rows rows{int(n), int(sequence), nullptr, wtok.as<uint32_t>(), int(sequence), 0};
        const kern::KvView kv{wk.as<float>(), wv.as<float>(), int(sequence)};
        run_blocks(rows, int(n / sequence), [&](size_t) { return kv; }, wx.as<float>(), nullptr, wq.as<float>(),
                   wy.as<float>(), wxn.as<float>(), false);
    }

    std::vector<float> logits(const uint32_t *tokens, size_t n, size_t sequence, bool last_only) {
        cfg.validate_tokens(tokens, n, sequence);
        activate();
        ensure_derived();
        const size_t out_rows = last_only ? n / sequence : n;
        namespace T = kern::train;
        if (T::short_forward_fits(int(cfg.width), int(cfg.heads), cfg.vocab_size, int(sequence))) {
            // Sequences of up to 16 rows: the whole forward and the head in one
            // launch, a workgroup per sequence.
            ensure_workspace(n, out_rows, true);
            check(hipMemcpyAsync(wtok.p, tokens, n * 4, hipMemcpyHostToDevice, stream), "upload tokens");
            mark_call(0);
            T::ShortForward a{};
            a.E = E.as<float>();
            a.Et = Et.as<float>();
            a.vpad = vpad;
            a.w = params.as<float>();
            a.tokens = wtok.as<uint32_t>();
            a.table = rope.as<float2>();
            a.logits = wlogits.as<float>();
            a.block0 = layout.groups[layout.blocks[0].query].offset;
            a.W = int(cfg.width);
            a.H = int(cfg.heads);
            a.L = int(cfg.layers);
            a.A = int(cfg.attention_mesh_depth);
            a.F = int(cfg.ffn_mesh_depth);
            a.V = int(cfg.vocab_size);
            a.sequence = int(sequence);
            a.butterfly = shape.butterfly;
            a.log2w = shape.log2w;
            a.rope = cfg.rope;
            a.qk_norm = cfg.qk_norm;
            a.xsa = cfg.xsa;
            a.last_only = last_only;
            a.scale = float(1.0 / std::sqrt(double(cfg.width / cfg.heads)));
            T::short_forward(a, int(n / sequence), stream);
        } else {
            forward_rows(tokens, n, sequence, out_rows);
            kern::head(shape, wxn.as<float>(), int(out_rows), last_only ? int(sequence) : 1,
                       last_only ? int(sequence) - 1 : 0, Et.as<float>(), vpad, wlogits.as<float>(), head_rows(),
                       stream);
        }
        mark_call(1);
        std::vector<float> out(out_rows * cfg.vocab_size);
        check(hipMemcpyAsync(out.data(), wlogits.p, out.size() * 4, hipMemcpyDeviceToHost, stream),
              "download logits");
        sync();
        close_call();
        validate_finite(out.data(), out.size(), "logits");
        return out;
    }

    std::vector<float> hidden_states(const uint32_t *tokens, size_t n, size_t sequence) {
        cfg.validate_tokens(tokens, n, sequence);
        activate();
        ensure_derived();
        forward_rows(tokens, n, sequence, 1);
        mark_call(1);
        std::vector<float> out(n * cfg.width);
        check(hipMemcpyAsync(out.data(), wx.p, out.size() * 4, hipMemcpyDeviceToHost, stream), "download");
        sync();
        close_call();
        validate_finite(out.data(), out.size(), "features");
        return out;
    }

    // ---- training -------------------------------------------------------------

    void reset_optimizer() {
        beta1_power = beta2_power = 1.0f;
        if (tm.p) {
            check(hipMemsetAsync(tm.p, 0, tm.bytes, stream), "clear moments");
            check(hipMemsetAsync(tv.p, 0, tv.bytes, stream), "clear moments");
        }
    }

    // Offsets (floats) of the training forward's activations and the
    // backward's scratch in tact, for R rows.
    struct TrainBlock {
        size_t n1, inv1, qs, ks, vs, qr, kr, qinv, kinv, y, lse, z, ps, xm, inv2, n2, fs;
    };
    struct TrainPlan {
        size_t es, eg, er, x, invf, nf, logits, dlogits, loss, dx, dn, dnk, dnv, dq, dk, dv, dy, dt, dsum, dE,
            total;
        std::vector<TrainBlock> blocks;
    };

    TrainPlan train_plan(size_t R) const {
        const size_t W = cfg.width, H = cfg.heads, V = cfg.vocab_size, A = cfg.attention_mesh_depth;
        const size_t F = cfg.ffn_mesh_depth, RW = R * W, RH = R * H;
        size_t at = 0;
        auto take = [&](size_t n) {
            const size_t o = at;
            at += (n + 63) / 64 * 64;
            return o;
        };
        TrainPlan p;
        p.es = take(cfg.embedding == TokenEmbedding::Mesh ? A * V * W : 0);
        p.eg = take(cfg.geometry.transformed() ? V * W : 0);
        p.er = take(V);
        p.x = take((cfg.layers + 1) * RW);
        for (size_t b = 0; b < cfg.layers; ++b) {
            TrainBlock k;
            k.n1 = take(RW);
            k.inv1 = take(R);
            k.qs = take(A * RW);
            k.ks = take(A * RW);
            k.vs = take(A * RW);
            k.qr = take(RW);
            k.kr = take(RW);
            k.qinv = take(RH);
            k.kinv = take(RH);
            k.y = take(RW);
            k.lse = take(RH);
            k.z = take(RW);
            k.ps = take(A * RW);
            k.xm = take(RW);
            k.inv2 = take(R);
            k.n2 = take(RW);
            k.fs = take(F * RW);
            p.blocks.push_back(k);
        }
        p.invf = take(R);
        p.nf = take(RW);
        p.logits = take(R * V);
        p.dlogits = take(R * V);
        p.loss = take(R);
        p.dx = take(RW);
        p.dn = take(RW);
        p.dnk = take(RW);
        p.dnv = take(RW);
        p.dq = take(RW);
        p.dk = take(RW);
        p.dv = take(RW);
        p.dy = take(RW);
        p.dt = take(RW);
        p.dsum = take(RH);
        p.dE = take(V * W);
        p.total = at;
        return p;
    }

    void check_trainable() const {
        if (cfg.width > size_t(kern::train::kMaxWidth) || cfg.head_width() > size_t(kern::train::kMaxHeadWidth))
            throw Error("training supports width <= 1024", kUnsupported);
    }

    // config.rs:230-252: inputs as validate_tokens, equal lengths, targets in
    // the vocabulary or IGNORE_TARGET, at least one supervised.
    size_t validate_batch(const uint32_t *inputs, const uint32_t *targets, size_t n, size_t sequence) const {
        cfg.validate_tokens(inputs, n, sequence);
        size_t supervised = 0;
        for (size_t i = 0; i < n; ++i) {
            if (targets[i] == kIgnoreTarget) continue;
            if (targets[i] >= cfg.vocab_size) throw Error("target ID is outside the vocabulary");
            ++supervised;
        }
        if (supervised == 0) throw Error("batch must contain at least one supervised target");
        return supervised;
    }

    // Buffers of a training step over n rows (grown, never shrunk); a
    // reallocation invalidates the captured step.
    void train_prepare(size_t n) {
        namespace T = kern::train;
        const size_t P = layout.count();
        bool grown = tact.ensure(train_plan(n).total * 4);
        grown |= tpart.ensure(train_partial_floats(n) * 4);
        grown |= tgrad.ensure(P * 4);
        static_assert(sizeof(T::StepScalars) <= kTrainTokensAt, "step scalars precede the tokens");
        grown |= tin.ensure(kTrainTokensAt + 8 * n);
        tstage.ensure(kTrainTokensAt + 12 * n);
        if (tm.ensure(P * 4) | tv.ensure(P * 4)) {
            grown = true;
            check(hipMemsetAsync(tm.p, 0, tm.bytes, stream), "clear moments");
            check(hipMemsetAsync(tv.p, 0, tv.bytes, stream), "clear moments");
        }
        if (grown) drop_train_graph();
    }

    // The backward's reduction scratch: a region for each mesh stack's partial
    // sums (their reductions run together at the end), then the embedding
    // gradient's.
    size_t train_partial_floats(size_t n) const {
        namespace T = kern::train;
        const int R = int(n), W = int(cfg.width), V = int(cfg.vocab_size);
        const T::Mesh ma{W, int(cfg.attention_mesh_depth), shape.butterfly, shape.log2w};
        const T::Mesh mf{W, int(cfg.ffn_mesh_depth), shape.butterfly, shape.log2w};
        size_t total = cfg.layers * (4 * T::mesh_partial_floats(ma, R) + T::mesh_partial_floats(mf, R));
        if (cfg.embedding == TokenEmbedding::Mesh) total += T::mesh_partial_floats(ma, V);
        return total + T::embedding_partial_floats(R, W, V);
    }

    void drop_train_graph() {
        if (texec) (void)hipGraphExecDestroy(texec);
        if (tgraph) (void)hipGraphDestroy(tgraph);
        texec = nullptr;
        tgraph = nullptr;
    }

    // Uploads a step's inputs, targets and scalars (outside any graph).
    void train_upload(const uint32_t *inputs, const uint32_t *targets, size_t n, size_t supervised, float c1,
                      float c2) {
        // The previous step's copies are complete: each step ends with a sync.
        hyper = kern::train::StepScalars{c1, c2, 1.0f / float(supervised), 0};
        char *h = tstage.as<char>();
        std::memcpy(h, &hyper, sizeof(hyper));
        std::memcpy(h + kTrainTokensAt, inputs, n * 4);
        std::memcpy(h + kTrainTokensAt + 4 * n, targets, n * 4);
        check(hipMemcpyAsync(tin.p, h, kTrainTokensAt + 8 * n, hipMemcpyHostToDevice, stream), "upload batch");
    }

    // The training forward over n rows (reference.rs:104-228) keeping every
    // activation, the loss kernel, and with `backward` the gradient of the
    // mean loss in tgrad (reference.rs:61-89, masked as config.rs:490-500):
    // kernels only, enqueued on the stream (so a step can be captured).
    void train_enqueue(size_t n, size_t sequence, bool backward) {
        namespace T = kern::train;
        const int R = int(n), W = int(cfg.width), H = int(cfg.heads), V = int(cfg.vocab_size), seq = int(sequence);
        const int A = int(cfg.attention_mesh_depth), F = int(cfg.ffn_mesh_depth), L = int(cfg.layers);
        const size_t RW = n * cfg.width;
        const TrainPlan p = train_plan(n);
        const T::Mesh ma{W, A, shape.butterfly, shape.log2w}, mf{W, F, shape.butterfly, shape.log2w};
        float *act = tact.as<float>(), *part = tpart.as<float>(), *grad = tgrad.as<float>();
        const float *w = params.as<float>();
        const uint32_t *tok = train_tokens(), *tgt = tok + n;
        const float2 *table = rope.as<float2>();
        auto *sc = tin.as<T::StepScalars>();
        auto at = [&](size_t o) { return act + o; };
        auto group = [&](size_t id) { return layout.groups[id].offset; };
        const size_t emb = group(layout.embedding);

        // Token vectors: the embedding mesh of the codes (its layers kept), or the table.
        const float *Eraw = w + emb;
        if (cfg.embedding == TokenEmbedding::Mesh) {
            T::mesh_forward(ma, codes.as<float>(), at(p.es), w + emb, V, stream);
            Eraw = at(p.es) + size_t(A - 1) * V * W;
        }
        // The geometry's normalisation and protected coordinates (reference.rs:130-149).
        const bool geometry = cfg.geometry.transformed(), normalize = cfg.geometry.normalization != EmbeddingNorm::None;
        const float radius = cfg.geometry.radius(cfg.width);
        const int preserve = int(cfg.geometry.preserve_features);
        const float *Ev = Eraw;
        if (geometry) {
            T::geometry_forward(Eraw, codes.as<float>(), at(p.eg), at(p.er), V, W, radius, normalize, preserve, stream);
            Ev = at(p.eg);
        }
        T::gather(Ev, tok, at(p.x), R, W, stream);
        auto X = [&](int b) { return at(p.x) + size_t(b) * RW; };
        auto last = [&](size_t o, int depth) { return at(o) + size_t(depth - 1) * RW; };
        for (int b = 0; b < L; ++b) {
            const TrainBlock &k = p.blocks[b];
            const Block &g = layout.blocks[b];
            // n1 = rmsnorm(x_b), x_b = xm + ffn of the block below (its residual
            // add and this norm are formed in front of the meshes), then Q, K
            // and V of n1 in one launch, then QK-Norm and RoPE of q and k in
            // one (reference.rs:174-193, each when switched on).
            const float *qkv_w[3] = {w + group(g.query), w + group(g.key), w + group(g.value)};
            float *qkv[3] = {at(k.qs), at(k.ks), at(k.vs)};
            const T::NormIn n1 = b == 0 ? T::NormIn{X(0), nullptr, nullptr, at(k.n1), at(k.inv1)}
                                        : T::NormIn{at(p.blocks[b - 1].xm), last(p.blocks[b - 1].fs, F), X(b),
                                                    at(k.n1), at(k.inv1)};
            const T::QkOut qk{{at(k.qr), at(k.kr)}, {at(k.qinv), at(k.kinv)}, table, seq, H, cfg.qk_norm, cfg.rope};
            T::norm_mesh_forward_qkv(ma, n1, qkv, qkv_w, qk, R, stream);
            T::attention_forward(at(k.qr), at(k.kr), last(k.vs, A), at(k.y), at(k.z), at(k.lse), R, seq, W, H,
                                 cfg.xsa, stream);
            T::mesh_forward(ma, at(k.z), at(k.ps), w + group(g.projection), R, stream);
            // xm = x_b + proj and n2 = rmsnorm(xm), formed in front of the FFN mesh.
            float *fs = at(k.fs);
            const float *wf = w + group(g.ffn);
            T::norm_mesh_forward_set(mf, 1, T::NormIn{X(b), last(k.ps, A), at(k.xm), at(k.n2), at(k.inv2)}, &fs, &wf,
                                     R, stream);
        }
        // x_L = xm + ffn of the top block, and the final norm.
        T::add_rmsnorm_forward(at(p.blocks[L - 1].xm), last(p.blocks[L - 1].fs, F), X(L), at(p.nf), at(p.invf), R, W,
                               stream);
        T::head_logits(at(p.nf), Ev, at(p.logits), R, W, V, stream);
        T::cross_entropy(at(p.logits), tgt, at(p.dlogits), at(p.loss), R, V, sc, stream);
        if (!backward) return;

        float *dx = at(p.dx), *dn = at(p.dn), *dq = at(p.dq), *dk = at(p.dk), *dv = at(p.dv);
        float *dy = at(p.dy), *dt = at(p.dt);
        // Each stack's partial sums get their own region of the scratch, and
        // all their reductions run in one launch at the end.
        std::vector<T::GradReduce> reductions;
        float *scratch = part;
        auto region = [&](size_t floats) {
            float *r = scratch;
            scratch += floats;
            return r;
        };
        auto mesh_backward = [&](const T::Mesh &m, const float *in, const float *stack, const float *dout,
                                 float *din, size_t wo, int rows) {
            const float *wp = w + wo;
            float *gp = grad + wo;
            T::mesh_backward_set(m, 1, &in, &stack, &dout, &din, false, &wp, region(T::mesh_partial_floats(m, rows)),
                                 &gp, rows, stream, &reductions);
        };
        T::head_backward(at(p.dlogits), Ev, dn, R, W, V, stream);
        T::rmsnorm_backward(X(L), at(p.invf), dn, dx, false, R, W, 1, stream);
        for (int b = L - 1; b >= 0; --b) {
            const TrainBlock &k = p.blocks[b];
            const Block &g = layout.blocks[b];
            // x_{b+1} = xm + ffn(rmsnorm(xm)); xm = x_b + proj(attention)
            T::mesh_backward_norm(mf, at(k.n2), at(k.fs), dx, T::NormGrad{at(k.xm), at(k.inv2), dx}, dn,
                                  w + group(g.ffn), region(T::mesh_partial_floats(mf, R)), grad + group(g.ffn), R,
                                  stream, &reductions);
            mesh_backward(ma, at(k.z), at(k.ps), dx, dt, group(g.projection), R);
            T::attention_backward(at(k.qr), at(k.kr), last(k.vs, A), at(k.y), at(k.lse), dt, dy, dq, dk, dv,
                                  at(p.dsum), R, seq, W, H, cfg.xsa, stream);
            if (cfg.rope || cfg.qk_norm) {
                float *qk_g[2] = {dq, dk};
                const float *qk_pre[2] = {last(k.qs, A), last(k.ks, A)}, *qk_inv[2] = {at(k.qinv), at(k.kinv)};
                T::qk_backward(2, qk_g, qk_pre, qk_inv, table, R, seq, W, H, cfg.qk_norm, cfg.rope, stream);
            }
            // The Q, K and V meshes' backward in one launch, each into its own
            // rows; the norm's backward adds them (in that order).
            const float *n1 = at(k.n1);
            const float *qkv_in[3] = {n1, n1, n1}, *qkv[3] = {at(k.qs), at(k.ks), at(k.vs)};
            const float *qkv_dout[3] = {dq, dk, dv};
            const float *qkv_w[3] = {w + group(g.query), w + group(g.key), w + group(g.value)};
            float *qkv_din[3] = {dn, at(p.dnk), at(p.dnv)};
            float *qkv_grad[3] = {grad + group(g.query), grad + group(g.key), grad + group(g.value)};
            T::mesh_backward_set(ma, 3, qkv_in, qkv, qkv_dout, qkv_din, false, qkv_w,
                                 region(3 * T::mesh_partial_floats(ma, R)), qkv_grad, R, stream, &reductions);
            T::rmsnorm_backward_sum3(X(b), at(k.inv1), dn, at(p.dnk), at(p.dnv), dx, true, R, W, stream);
        }
        // The tied vectors collect the head's gradient and the gathered rows'.
        T::embedding_gradient(at(p.dlogits), at(p.nf), tok, dx, at(p.dE), region(T::embedding_partial_floats(R, W, V)),
                              R, W, V, stream);
        if (geometry) T::geometry_backward(Eraw, at(p.er), at(p.dE), V, W, radius, normalize, preserve, stream);
        if (cfg.embedding == TokenEmbedding::Mesh)
            mesh_backward(ma, codes.as<float>(), at(p.es), at(p.dE), nullptr, emb, V);
        else
            T::copy(at(p.dE), grad + emb, size_t(V) * W, stream);
        T::reduce_gradients(reductions.data(), reductions.size(), stream);
        // config.rs:490-500: the frozen embedding group, and the final mesh rows
        // that write protected residual coordinates.
        if (cfg.geometry.frozen) T::fill(grad + emb, 0.0f, cfg.embedding_parameter_count(), stream);
        for (size_t id = 0; id < layout.groups.size(); ++id) {
            const auto range = layout.constrained_range(cfg, id);
            if (range.second > range.first)
                T::fill(grad + layout.groups[id].offset + range.first, 0.0f, range.second - range.first, stream);
        }
    }

    // gpu.rs:2296-2313: the per-row f32 losses summed in f64 on the host.
    size_t allocated_device_bytes() const {
        size_t total = 0;
        for (const DevBuf *b : {&params, &codes, &E, &Et, &rope, &wdec, &Edec, &q0, &kc, &vc, &dx, &dx2, &dxn, &dq,
                                &part, &dtokens, &dlen, &drng, &dlogits, &dflags, &drng_start, &drng_next, &pxch, &pabort, &wx,
                                &wxn, &wq, &wy, &wtok, &wlogits, &wk, &wv, &tact, &tgrad, &tm, &tv, &tpart, &tin})
            total += b->bytes;
        return total;
    }

    const uint32_t *train_tokens() const { return reinterpret_cast<const uint32_t *>(tin.as<char>() + kTrainTokensAt); }

    double train_loss(size_t n, size_t supervised) {
        float *rows = reinterpret_cast<float *>(tstage.as<char>() + kTrainTokensAt + 8 * n);
        check(hipMemcpyAsync(rows, tact.as<float>() + train_plan(n).loss, n * 4, hipMemcpyDeviceToHost, stream),
              "download loss");
        sync();
        validate_finite(rows, n, "cross-entropy");
        double total = 0.0;
        for (size_t i = 0; i < n; ++i) total += double(rows[i]);
        return total / double(supervised);
    }

    double train_pass(const uint32_t *inputs, const uint32_t *targets, size_t n, size_t sequence, bool backward) {
        check_trainable();
        const size_t supervised = validate_batch(inputs, targets, n, sequence);
        activate();
        train_prepare(n);
        train_upload(inputs, targets, n, supervised, 1.0f, 1.0f);
        train_enqueue(n, sequence, backward);
        return train_loss(n, supervised);
    }

    std::vector<float> gradient() {
        std::vector<float> out(layout.count());
        check(hipMemcpy(out.data(), tgrad.p, out.size() * 4, hipMemcpyDeviceToHost), "download gradients");
        validate_finite(out.data(), out.size(), "gradients");
        return out;
    }

    // gpu.rs:1971-2003: the gradient, then one AdamW update of every group
    // (the embedding group stays when the geometry is frozen).  The whole
    // step is captured once per (rows, sequence, options) as a HIP graph and
    // replayed; a non-finite loss leaves the weights, moments and step count
    // as they were.
    double train_batch(const uint32_t *inputs, const uint32_t *targets, size_t n, size_t sequence,
                       const AdamWOptions &o) {
        o.validate();
        check_trainable();
        const size_t supervised = validate_batch(inputs, targets, n, sequence);
        activate();
        train_prepare(n);
        const float p1 = beta1_power * o.beta1, p2 = beta2_power * o.beta2;
        train_upload(inputs, targets, n, supervised, 1.0f - p1, 1.0f - p2);
        const TrainKey key{n, sequence, o.learning_rate, o.weight_decay, o.beta1, o.beta2, o.epsilon};
        auto enqueue = [&] {
            train_enqueue(n, sequence, true);
            const size_t begin = cfg.geometry.frozen ? cfg.embedding_parameter_count() : 0;
            kern::train::adam(params.as<float>(), tm.as<float>(), tv.as<float>(), tgrad.as<float>(), begin,
                              layout.count(), {o.learning_rate, o.weight_decay, o.beta1, o.beta2, o.epsilon},
                              tin.as<kern::train::StepScalars>(), stream);
        };
        if (use_graph) {
            if (!texec || !(key == tkey)) {
                drop_train_graph();
                check(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "begin capture");
                enqueue();
                check(hipStreamEndCapture(stream, &tgraph), "end capture");
                check(hipGraphInstantiate(&texec, tgraph, nullptr, nullptr, 0), "instantiate training graph");
                tkey = key;
            }
            check(hipGraphLaunch(texec, stream), "replay training step");
        } else {
            enqueue();
        }
        derived_stale = true;
        const double loss = train_loss(n, supervised);  // throws (weights unchanged) on a non-finite loss
        beta1_power = p1;
        beta2_power = p2;
        return loss;
    }

    // ---- generation -------------------------------------------------------

    void start(const uint32_t *prompts, size_t b, size_t p, float t, uint64_t seed, size_t reserve) {
        if (!std::isfinite(t) || t < 0.0f) throw Error("temperature must be finite and nonnegative (0 is greedy)");
        if (p == 0) throw Error("generation prompt must not be empty");
        if (b == 0) throw Error("generation batch must not be empty");
        for (size_t i = 0; i < b * p; ++i)
            if (prompts[i] >= cfg.vocab_size) throw Error("token ID is outside the vocabulary");
        activate();
        ensure_derived();
        ensure_decode(b, std::max(reserve, p));
        check(hipMemcpy2DAsync(dtokens.p, tcap * 4, prompts, p * 4, p * 4, b, hipMemcpyHostToDevice, stream),
              "upload prompts");
        std::vector<int> lens(b, int(p));
        std::vector<uint64_t> states(b);
        for (size_t i = 0; i < b; ++i) states[i] = seed + i;
        check(hipMemcpyAsync(dlen.p, lens.data(), b * 4, hipMemcpyHostToDevice, stream), "upload lengths");
        check(hipMemcpyAsync(drng.p, states.data(), b * 8, hipMemcpyHostToDevice, stream), "upload rng");
        check(hipMemsetAsync(dflags.p, 0, 4, stream), "clear flags");
        sync();
        batch = b;
        length = p;
        cached = 0;
        temperature = t;
        start_length = 0;
    }

    // The head and sampler for `n` sequence rows of xn (row i at i*row_mul+row_add).
    void head_and_sample(const float *xn, int row_mul, int row_add) {
        if (row_mul == 1 && row_add == 0 && kern::head_sample_lds_bytes(shape) <= lds_limit) {
            kern::head_sample(shape, xn, int(batch), Et.as<float>(), vpad, dlogits.as<float>(), temperature,
                              drng.as<uint64_t>(), dtokens.as<uint32_t>(), int(tcap), dlen.as<int>(),
                              dflags.as<int>(), stream);
            return;
        }
        kern::head(shape, xn, int(batch), row_mul, row_add, Et.as<float>(), vpad, dlogits.as<float>(),
                   head_rows(), stream);
        kern::sample(shape.V, int(batch), dlogits.as<float>(), temperature, drng.as<uint64_t>(),
                     dtokens.as<uint32_t>(), int(tcap), dlen.as<int>(), dflags.as<int>(), stream);
    }

    // Slices of the per-phase decode.  Each sequence's decode is independent
    // of the others' (rows, cache slabs, generator states and tokens are per
    // sequence), so the batch splits into slices that run on their own
    // streams: while one slice's attention streams its keys (memory-bound),
    // another's row blocks run (latency-bound).  Config 5 (batch 256):
    // 1231 us per step in one stream, 1072 in two slices, 1062 in four.
    // Slices need at least 32 sequences each, or 4 once the sequences attend
    // over 2048 keys or more (config 4, batch 8 at 8192 keys: 248 us per step
    // in one stream, 237 in two slices), and the fused head-and-sampler
    // kernel.  MG_DECODE_SLICES overrides the count (1 = one stream),
    // MG_DECODE_SLICE_MIN the sequences a slice needs.
    int decode_slices() const {
        const int want = std::min(env_int("MG_DECODE_SLICES", 2), kMaxSlices);
        if (kern::head_sample_lds_bytes(shape) > lds_limit) return 1;
        const size_t least = size_t(env_int("MG_DECODE_SLICE_MIN", length >= 2048 ? 4 : 32));
        for (int n = want; n > 1; --n)
            if (batch >= least * n) return n;
        return 1;
    }

    // One decode step of sequences [b0, b0 + nb) on `stream`; the slice's
    // attention partial states start at slot `slot0` of `part`.
    void launch_slice_step(size_t b0, size_t nb, size_t slot0) {
        const size_t W = cfg.width;
        const kern::Rows rows{int(nb), 1, dlen.as<int>() + b0, dtokens.as<uint32_t>() + b0 * tcap, int(tcap), 0};
        const size_t kv_off = b0 * size_t(shape.H) * cfg.context * size_t(shape.hdp);
        run_blocks(rows, int(nb),
                   [&](size_t l) {
                       kern::KvView kv = cache_layer(l);
                       kv.k += kv_off;
                       kv.v += kv_off;
                       return kv;
                   },
                   dx.as<float>() + b0 * W, dx2.as<float>() + b0 * W, dq.as<float>() + b0 * W, nullptr,
                   dxn.as<float>() + b0 * W, true, nullptr,
                   part.as<float>() + slot0 * size_t(shape.H) * (shape.hdp + 2));
        kern::head_sample(shape, dxn.as<float>() + b0 * W, int(nb), Et.as<float>(), vpad,
                          dlogits.as<float>() + b0 * shape.V, temperature, drng.as<uint64_t>() + b0,
                          dtokens.as<uint32_t>() + b0 * tcap, int(tcap), dlen.as<int>() + b0, dflags.as<int>(),
                          stream);
    }

    // `n` decode steps of every slice, each slice on its own stream.
    void enqueue_slices(size_t n, int slices) {
        if (!fork_ev) {
            for (int i = 0; i < kMaxSlices - 1; ++i) {
                check(hipStreamCreateWithFlags(&slice_stream[i], hipStreamNonBlocking), "hipStreamCreate");
                check(hipEventCreateWithFlags(&join_ev[i], hipEventDisableTiming), "hipEventCreate");
            }
            check(hipEventCreateWithFlags(&fork_ev, hipEventDisableTiming), "hipEventCreate");
        }
        check(hipEventRecord(fork_ev, stream), "hipEventRecord");
        for (int i = 0; i + 1 < slices; ++i)
            check(hipStreamWaitEvent(slice_stream[i], fork_ev, 0), "hipStreamWaitEvent");
        const hipStream_t own = stream;
        try {
            size_t slot0 = 0;
            for (int p = 0; p < slices; ++p) {
                const size_t b0 = batch * p / slices, nb = batch * (p + 1) / slices - b0;
                stream = p == 0 ? own : slice_stream[p - 1];
                for (size_t i = 0; i < n; ++i) launch_slice_step(b0, nb, slot0);
                slot0 += nb * size_t(splits_for(nb));
                if (p > 0) check(hipEventRecord(join_ev[p - 1], stream), "hipEventRecord");
            }
        } catch (...) {
            stream = own;
            throw;
        }
        stream = own;
        for (int i = 0; i + 1 < slices; ++i) check(hipStreamWaitEvent(stream, join_ev[i], 0), "hipStreamWaitEvent");
    }

    void launch_decode_step(hipEvent_t *events = nullptr) {
        const kern::Rows rows{int(batch), 1, dlen.as<int>(), dtokens.as<uint32_t>(), int(tcap), 0};
        run_blocks(rows, int(batch), [&](size_t l) { return cache_layer(l); }, dx.as<float>(), dx2.as<float>(),
                   dq.as<float>(), nullptr, dxn.as<float>(), true, events);
        head_and_sample(dxn.as<float>(), 1, 0);
    }

    // `n` decode steps (1 or kGraphSteps) as one graph replay; the graphs are
    // captured on first use for the current batch and temperature.
    void decode_steps(size_t n) {
        const int slices = decode_slices();
        auto enqueue = [&] {
            if (slices > 1)
                enqueue_slices(n, slices);
            else
                for (size_t i = 0; i < n; ++i) launch_decode_step();
        };
        if (!use_graph) {
            enqueue();
            return;
        }
        if (graph_batch != batch || graph_temperature != temperature || graph_slices != slices) drop_graph();
        const int g = n == 1 ? 0 : 1;
        if (!exec[g]) {
            check(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "begin capture");
            enqueue();
            check(hipStreamEndCapture(stream, &graph[g]), "end capture");
            check(hipGraphInstantiate(&exec[g], graph[g], nullptr, nullptr, 0), "instantiate graph");
            graph_batch = batch;
            graph_temperature = temperature;
            graph_slices = slices;
        }
        check(hipGraphLaunch(exec[g], stream), "graph launch");
    }

    void decode_step() { decode_steps(1); }

    // Prefill over positions [start, start+n) of every sequence into the cache
    // (positions rebased to 0), then the head on each sequence's last row.
    void prefill_step(size_t start, size_t n) {
        ensure_workspace(batch * n, 1, false);
        const kern::Rows rows{int(batch * n), int(n), nullptr, dtokens.as<uint32_t>(), int(tcap), int(start)};
        run_blocks(rows, int(batch), [&](size_t l) { return cache_layer(l); }, wx.as<float>(), nullptr,
                   wq.as<float>(), wy.as<float>(), wxn.as<float>(), false);
        head_and_sample(wxn.as<float>(), int(n), int(n) - 1);
    }

    // One generated token for every sequence (gpu.rs:2025-2050).
    void step() {
        if (length + 1 > tcap) throw Error("generation exceeds the reserved token capacity");
        if (length <= cfg.context && cached == length - 1) {
            decode_step();
            cached = length;
        } else if (length <= cfg.context) {
            prefill_step(0, length);
            cached = length;
        } else {
            // Beyond the context the window slides and positions restart at 0,
            // so every step recomputes the window exactly like the reference.
            prefill_step(length - cfg.context, cfg.context);
            cached = kNoCache;
        }
        ++length;
    }

    void finish() {
        sync();
        int flags = 0;
        check(hipMemcpy(&flags, dflags.p, 4, hipMemcpyDeviceToHost), "download flags");
        if (flags) throw Error("logits must contain only finite values", kNonfinite);
    }

    void read_tokens(uint32_t *out, size_t b, size_t len) {
        if (b > batch || len > length) throw Error("requested tokens exceed the generated sequences");
        activate();
        check(hipMemcpy2DAsync(out, len * 4, dtokens.p, tcap * 4, len * 4, b, hipMemcpyDeviceToHost, stream),
              "download tokens");
        sync();
    }

    bool decodable(size_t steps) const {
        return batch > 0 && cached == length - 1 && length - 1 + steps <= cfg.context && length + steps <= tcap;
    }

    bool persistent_usable() const {
        return persistent_ok && row_decode && kern::persistent_fits(shape, int(batch), device);
    }

    // Whether `steps` decode steps should run in the persistent kernel (the
    // caller checked persistent_usable()).  It gives each (sequence, head) one
    // workgroup, which streams that head's keys alone; with few sequences and
    // long contexts the per-phase split-KV kernels, which spread the keys over
    // about 512 workgroups, are faster (config 4, batch 8 at 8192..8447 keys:
    // 247 us per step against 355).  MG_FORCE_PERSISTENT=1 always prefers it.
    bool persistent_preferred(size_t steps) const {
        if (env_int("MG_FORCE_PERSISTENT", 0)) return true;
        const size_t keys = length - 1 + steps;  // the launch's last step attends over these
        const size_t slab_bytes = keys * 2 * size_t(shape.hdp) * 4;
        return batch * cfg.heads >= 96 || slab_bytes <= (size_t(128) << 10);
    }

    // `steps` decode steps in one launch of the persistent kernel (the caller
    // checked decodable(steps) and persistent_usable(), which includes that
    // every block fits the GPU at once).  Returns false, with the decode state
    // as before, when the launch does not complete: the runtime refuses it, or
    // a hand-off wait times out, which happens when some blocks could not be
    // resident (another kernel holding part of the GPU).  The caller then runs
    // the same steps on the per-phase kernels.  The sampler states of the
    // launch go to drng_next and its non-finite flag to pabort[1], taken over
    // only when it completes; the token and cache rows past the old length
    // that a timed-out launch wrote are rewritten by the per-phase steps.
    // With MG_PERSIST_STRICT=1 a timed-out launch throws instead, with the
    // decode state as before (tests use it, so that a broken hand-off is not
    // hidden by the fallback).
    // MG_PERSIST_WAIT_TICKS sets the waits' limit in 100 MHz ticks.
    bool persistent(size_t steps, uint64_t *trace = nullptr) {
        const size_t xstride = kern::persistent_exchange_words(shape);
        check(hipMemsetAsync(pxch.p, 0, batch * xstride * 8, stream), "clear exchange words");
        check(hipMemsetAsync(pabort.p, 0, 8, stream), "clear abort and flags");
        kern::PersistArgs a{};
        a.s = shape;
        a.batch = int(batch);
        a.layers = int(cfg.layers);
        a.steps = int(steps);
        a.E = Edec.as<float>();
        a.w = wdec.as<float>();
        a.block0 = layout.groups[layout.blocks[0].query].offset;
        a.kc = kc.as<float>();
        a.vc = vc.as<float>();
        a.layer_elems = layer_cache_elems();
        a.cap = int(cfg.context);
        a.q0 = q0.as<float>();
        a.logits = dlogits.as<float>();
        a.rope = rope.as<float2>();
        a.tokens = dtokens.as<uint32_t>();
        a.tok_stride = int(tcap);
        a.len = dlen.as<int>();
        a.rng = drng.as<uint64_t>();
        a.rng_out = drng_next.as<uint64_t>();
        a.temperature = temperature;
        a.flags = pabort.as<int>() + 1;
        a.xch = pxch.as<uint64_t>();
        a.xstride = xstride;
        a.abort = pabort.as<int>();
        a.wait_ticks = uint64_t(std::max(0, env_int("MG_PERSIST_WAIT_TICKS", 0)));
        a.trace = trace;
        a.agent_scope = env_int("MG_PERSIST_AGENT_SCOPE", 0) != 0;
        a.mall_keep = keep_rows();
        // Events on the stream right around the kernel: last_call_ms() is
        // the launch's own duration.
        mark_call(0);
        const hipError_t launched = kern::persistent_decode(a, stream);
        if (launched == hipErrorOutOfMemory || launched == hipErrorLaunchOutOfResources ||
            launched == hipErrorCooperativeLaunchTooLarge) {
            (void)hipGetLastError();  // the refusal is not a device error
            return false;
        }
        check(launched, "persistent decode launch");
        mark_call(1);
        sync();
        close_call();
        int status[2] = {0, 0};
        check(hipMemcpy(status, pabort.p, 8, hipMemcpyDeviceToHost), "download abort flag");
        if (status[0]) {
            // Every sequence back at the launch's starting length; the sampler
            // states in drng were not touched.
            check(hipMemsetD32Async(hipDeviceptr_t(dlen.p), int(length), batch, stream), "restore lengths");
            if (env_int("MG_PERSIST_STRICT", 0))
                throw Error("persistent decode kernel timed out waiting on a hand-off", kDeviceError);
            return false;
        }
        std::swap(drng.p, drng_next.p);
        std::swap(drng.bytes, drng_next.bytes);
        if (status[1]) check(hipMemsetD32Async(hipDeviceptr_t(dflags.p), 1, 1, stream), "flag non-finite logits");
        cached = length + steps - 1;
        length += steps;
        return true;
    }
};

MeshGpt::MeshGpt(int device, const GptConfig &config, uint64_t seed, size_t max_batch)
    : impl_(std::make_unique<Impl>()) {
    impl_->init(device, config, seed, max_batch);
}

MeshGpt::~MeshGpt() = default;

const GptConfig &MeshGpt::config() const { return impl_->cfg; }

std::vector<float> MeshGpt::parameters() const {
    impl_->activate();
    std::vector<float> out(impl_->layout.count());
    check(hipMemcpy(out.data(), impl_->params.p, out.size() * 4, hipMemcpyDeviceToHost), "download parameters");
    validate_finite(out.data(), out.size(), "parameters");
    return out;
}

void MeshGpt::set_parameters(const float *values, size_t n) { impl_->set_parameters(values, n); }

std::vector<float> MeshGpt::logits(const uint32_t *tokens, size_t n, size_t sequence, bool last_only) {
    return impl_->logits(tokens, n, sequence, last_only);
}

std::vector<float> MeshGpt::token_embeddings() {
    impl_->activate();
    impl_->ensure_derived();
    std::vector<float> out(impl_->cfg.vocab_size * impl_->cfg.width);
    check(hipMemcpy(out.data(), impl_->E.p, out.size() * 4, hipMemcpyDeviceToHost), "download embeddings");
    validate_finite(out.data(), out.size(), "features");
    return out;
}

double MeshGpt::cross_entropy(const uint32_t *inputs, const uint32_t *targets, size_t n, size_t sequence) {
    return impl_->train_pass(inputs, targets, n, sequence, false);
}

double MeshGpt::loss_and_gradient(const uint32_t *inputs, const uint32_t *targets, size_t n, size_t sequence,
                                  std::vector<float> &gradient) {
    const double loss = impl_->train_pass(inputs, targets, n, sequence, true);
    gradient = impl_->gradient();
    return loss;
}

double MeshGpt::train_batch(const uint32_t *inputs, const uint32_t *targets, size_t n, size_t sequence,
                            const AdamWOptions &options) {
    return impl_->train_batch(inputs, targets, n, sequence, options);
}

size_t MeshGpt::allocated_device_bytes() const { return impl_->allocated_device_bytes(); }

std::vector<float> MeshGpt::hidden_states(const uint32_t *tokens, size_t n, size_t sequence) {
    return impl_->hidden_states(tokens, n, sequence);
}

void MeshGpt::generate_tokens(const uint32_t *prompts, size_t batch, size_t prompt_len, size_t count,
                              float temperature, uint64_t seed, uint32_t *out) {
    Impl &m = *impl_;
    m.start(prompts, batch, prompt_len, temperature, seed, prompt_len + count);
    size_t done = 0;
    if (count > 0) {
        m.step();  // the prompt's prefill and the first token
        ++done;
    }
    if (done < count && m.decodable(count - done) && m.persistent_usable() && m.persistent_preferred(count - done) &&
        m.persistent(count - done))
        done = count;
    for (; done < count; ++done) m.step();
    m.finish();
    m.read_tokens(out, batch, prompt_len + count);
}

std::string MeshGpt::generate(const CharacterTokenizer &tokenizer, const std::string &prompt, size_t count,
                              float temperature, uint64_t seed) {
    if (tokenizer.vocab_size() != impl_->cfg.vocab_size)
        throw Error("tokenizer does not match model vocabulary size");
    if (!std::isfinite(temperature) || temperature < 0.0f)
        throw Error("temperature must be finite and nonnegative (0 is greedy)");
    std::vector<uint32_t> tokens = tokenizer.encode(prompt);
    if (tokens.empty()) throw Error("generation prompt must not be empty");
    std::vector<uint32_t> out(tokens.size() + count);
    generate_tokens(tokens.data(), 1, tokens.size(), count, temperature, seed, out.data());
    return tokenizer.decode(out.data(), out.size());
}

void MeshGpt::prefill(const uint32_t *prompts, size_t batch, size_t prompt_len, float temperature, uint64_t seed,
                      size_t reserve) {
    Impl &m = *impl_;
    m.start(prompts, batch, prompt_len, temperature, seed, std::max(reserve, prompt_len + 1));
    m.mark_call(0);
    m.step();
    m.mark_call(1);
    m.finish();
    m.close_call();
    check(hipMemcpyAsync(m.drng_start.p, m.drng.p, m.batch * 8, hipMemcpyDeviceToDevice, m.stream), "save rng");
    m.start_length = m.length;
    m.sync();
}

void MeshGpt::rewind() {
    Impl &m = *impl_;
    if (m.start_length == 0 || m.length < m.start_length || m.start_length > m.cfg.context)
        throw Error("rewind needs a prefilled batch");
    m.activate();
    check(hipMemcpyAsync(m.drng.p, m.drng_start.p, m.batch * 8, hipMemcpyDeviceToDevice, m.stream),
          "restore rng");
    check(hipMemsetD32Async(hipDeviceptr_t(m.dlen.p), int(m.start_length), m.batch, m.stream), "restore lengths");
    m.length = m.start_length;
    m.cached = m.length - 1;
}

void MeshGpt::decode(size_t steps) {
    Impl &m = *impl_;
    if (!m.decodable(steps))
        throw Error("decode steps need a prefilled batch and must stay within the context and reserve");
    m.activate();
    if (m.persistent_usable() && m.persistent_preferred(steps) && m.persistent(steps)) {
        m.finish();
        return;
    }
    size_t done = 0;
    // Whole graphs of kGraphSteps steps, then single steps.
    for (; done + Impl::kGraphSteps <= steps; done += Impl::kGraphSteps) {
        m.decode_steps(Impl::kGraphSteps);
        m.cached = m.length + Impl::kGraphSteps - 1;
        m.length += Impl::kGraphSteps;
    }
    for (; done < steps; ++done) m.step();
    m.finish();
}

std::vector<float> MeshGpt::decode_profiled(size_t steps) {
    Impl &m = *impl_;
    if (!m.decodable(steps))
        throw Error("decode steps need a prefilled batch and must stay within the context and reserve");
    m.activate();
    const size_t L = m.cfg.layers;
    std::vector<hipEvent_t> ev(2 * L * steps);
    for (auto &e : ev) check(hipEventCreate(&e), "hipEventCreate");
    for (size_t s = 0; s < steps; ++s) {
        m.launch_decode_step(ev.data() + 2 * L * s);
        m.cached = m.length;
        ++m.length;
    }
    m.finish();
    std::vector<float> ms(L * steps);
    for (size_t i = 0; i < ms.size(); ++i) check(hipEventElapsedTime(&ms[i], ev[2 * i], ev[2 * i + 1]), "elapsed");
    for (auto &e : ev) (void)hipEventDestroy(e);
    return ms;
}

std::vector<uint64_t> MeshGpt::decode_traced(size_t steps) {
    Impl &m = *impl_;
    if (!m.decodable(steps))
        throw Error("decode steps need a prefilled batch and must stay within the context and reserve");
    m.activate();
    if (!m.persistent_usable()) throw Error("the persistent decode kernel does not support this model and batch",
                                            kUnsupported);
    const size_t blocks = 3 * m.batch + m.batch * m.cfg.heads;
    const size_t n = blocks * steps * (m.cfg.layers + 1) * 2;
    DevBuf trace;
    trace.ensure(n * 8);
    check(hipMemsetAsync(trace.p, 0, n * 8, m.stream), "clear trace");
    if (!m.persistent(steps, trace.as<uint64_t>()))
        throw Error("the persistent decode launch did not complete (the runtime refused it, or a hand-off timed out "
                    "while part of the GPU was busy)",
                    kDeviceError);
    m.finish();
    std::vector<uint64_t> out(n);
    check(hipMemcpy(out.data(), trace.p, n * 8, hipMemcpyDeviceToHost), "download trace");
    return out;
}

size_t MeshGpt::sequence_length() const { return impl_->length; }

float MeshGpt::last_call_ms() const { return impl_->call_ms; }

void MeshGpt::read_tokens(uint32_t *out, size_t batch, size_t length) { impl_->read_tokens(out, batch, length); }

std::vector<float> MeshGpt::last_logits() {
    Impl &m = *impl_;
    m.activate();
    std::vector<float> out(m.batch * m.cfg.vocab_size);
    check(hipMemcpy(out.data(), m.dlogits.p, out.size() * 4, hipMemcpyDeviceToHost), "download logits");
    return out;
}

hipStream_t MeshGpt::stream() const { return impl_->stream; }

bool sample_logits(int device, const float *logits, size_t rows, size_t vocab, float temperature,
                   uint64_t *rng_states, uint32_t *tokens) {
    if (rows == 0) return false;
    if (vocab == 0 || vocab > size_t(1) << 24) throw Error("vocabulary must hold 1..2^24 tokens");
    if (!std::isfinite(temperature) || temperature < 0.0f)
        throw Error("temperature must be finite and nonnegative (0 is greedy)");
    int count = 0;
    check(hipGetDeviceCount(&count), "hipGetDeviceCount");
    if (device < 0 || device >= count) throw Error("invalid device ordinal", kDeviceError);
    check(hipSetDevice(device), "hipSetDevice");
    DevBuf dl, drng, dtok, dlen, dflags;
    dl.ensure(rows * vocab * 4);
    drng.ensure(rows * 8);
    dtok.ensure(rows * 4);
    dlen.ensure(rows * 4);
    dflags.ensure(4);
    check(hipMemcpy(dl.p, logits, rows * vocab * 4, hipMemcpyHostToDevice), "upload logits");
    check(hipMemcpy(drng.p, rng_states, rows * 8, hipMemcpyHostToDevice), "upload rng");
    check(hipMemset(dlen.p, 0, rows * 4), "clear lengths");
    check(hipMemset(dflags.p, 0, 4), "clear flags");
    kern::sample(int(vocab), int(rows), dl.as<float>(), temperature, drng.as<uint64_t>(), dtok.as<uint32_t>(), 1,
                 dlen.as<int>(), dflags.as<int>(), nullptr);
    check(hipGetLastError(), "sample launch");
    check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    check(hipMemcpy(tokens, dtok.p, rows * 4, hipMemcpyDeviceToHost), "download tokens");
    check(hipMemcpy(rng_states, drng.p, rows * 8, hipMemcpyDeviceToHost), "download rng");
    int flags = 0;
    check(hipMemcpy(&flags, dflags.p, 4, hipMemcpyDeviceToHost), "download flags");
    return flags != 0;
}

void sample_logits_noalloc(int device, const float *logits, size_t rows, size_t vocab, float temperature,
                           uint64_t *rng_states, uint32_t *tokens, int *nonfinite, hipStream_t stream) {
    if (rows > size_t(kern::kNoAllocRows))
        throw Error("the allocation-free sampler takes at most " + std::to_string(kern::kNoAllocRows) + " rows");
    if (vocab == 0 || vocab > size_t(1) << 24) throw Error("vocabulary must hold 1..2^24 tokens");
    if (!std::isfinite(temperature) || temperature < 0.0f)
        throw Error("temperature must be finite and nonnegative (0 is greedy)");
    if (nonfinite == nullptr) throw Error("the non-finite flag must not be null");
    int count = 0;
    check(hipGetDeviceCount(&count), "hipGetDeviceCount");
    if (device < 0 || device >= count) throw Error("invalid device ordinal", kDeviceError);
    // The caller's current device is restored on return, also on an error.
    int caller = 0;
    check(hipGetDevice(&caller), "hipGetDevice");
    struct Restore {
        int device;
        ~Restore() { (void)hipSetDevice(device); }
    } restore{caller};
    check(hipSetDevice(device), "hipSetDevice");
    int *counters = nullptr;
    check(kern::noalloc_scratch(device, &counters), "hipGetSymbolAddress(scratch)");
    kern::fill_int(nonfinite, 0, 1, stream);
    check(hipGetLastError(), "flag clear launch");
    if (rows == 0) return;
    kern::fill_int(counters, 0, int(rows), stream);
    check(hipGetLastError(), "counter clear launch");
    kern::sample(int(vocab), int(rows), logits, temperature, rng_states, tokens, 1, counters, nonfinite, stream);
    check(hipGetLastError(), "sample launch");
}

void device_expf(int device, const float *x, size_t n, float *out) {
    if (n == 0) return;
    int count = 0;
    check(hipGetDeviceCount(&count), "hipGetDeviceCount");
    if (device < 0 || device >= count) throw Error("invalid device ordinal", kDeviceError);
    check(hipSetDevice(device), "hipSetDevice");
    DevBuf dx, dy;
    dx.ensure(n * 4);
    dy.ensure(n * 4);
    check(hipMemcpy(dx.p, x, n * 4, hipMemcpyHostToDevice), "upload inputs");
    kern::device_expf(dx.as<float>(), dy.as<float>(), n, nullptr);
    check(hipGetLastError(), "expf launch");
    check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    check(hipMemcpy(out, dy.p, n * 4, hipMemcpyDeviceToHost), "download results");
}

double copy_bandwidth(int device, size_t bytes, int iters) {
    int count = 0;
    check(hipGetDeviceCount(&count), "hipGetDeviceCount");
    if (device < 0 || device >= count) throw Error("invalid device ordinal", kDeviceError);
    check(hipSetDevice(device), "hipSetDevice");
    const size_t n = bytes / 16;
    DevBuf src, dst;
    src.ensure(n * 16);
    dst.ensure(n * 16);
    check(hipMemset(src.p, 0, n * 16), "hipMemset");
    hipEvent_t start, stop;
    check(hipEventCreate(&start), "hipEventCreate");
    check(hipEventCreate(&stop), "hipEventCreate");
    kern::calibration_copy(src.as<float4>(), dst.as<float4>(), n, nullptr);
    check(hipEventRecord(start, nullptr), "event");
    for (int i = 0; i < iters; ++i) kern::calibration_copy(src.as<float4>(), dst.as<float4>(), n, nullptr);
    check(hipEventRecord(stop, nullptr), "event");
    check(hipEventSynchronize(stop), "event sync");
    float ms = 0.0f;
    check(hipEventElapsedTime(&ms, start, stop), "elapsed");
    (void)hipEventDestroy(start);
    (void)hipEventDestroy(stop);
    check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    return 2.0 * double(n * 16) * iters / (double(ms) / 1000.0) / 1e9;
}

void MeshGpt::synchronize() { impl_->sync(); }

}  // namespace meshgpt
