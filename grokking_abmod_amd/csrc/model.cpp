// Host orchestration of the device-resident Mesh GPT: buffers, the prefill and
// decode sequences of kernel launches, and the HIP graph that replays one
// decode step.
#include "model.hpp"

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
    size_t lds_limit = 65536;

    DevBuf params, codes, E, Et, rope;

    // Decode state: KV cache [L][batch_cap][H][context][hdp], per-sequence
    // tokens [batch_cap][tcap], lengths, SplitMix64 states and logits.
    size_t batch_cap = 0, tcap = 0;
    int ks = 64, smax = 1;
    DevBuf kc, vc, dx, dq, part, dtokens, dlen, drng, dlogits, dflags;
    size_t batch = 0, length = 0, cached = kNoCache;
    float temperature = 0.0f;

    // Prefill / logits workspace, grown on demand.
    DevBuf wx, wq, wy, wtok, wlogits, wk, wv;

    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    size_t graph_batch = 0;
    float graph_temperature = -1.0f;
    bool use_graph = true;

    ~Impl() {
        drop_graph();
        if (stream) (void)hipStreamDestroy(stream);
    }

    void activate() const { check(hipSetDevice(device), "hipSetDevice"); }

    void drop_graph() {
        if (exec) (void)hipGraphExecDestroy(exec);
        if (graph) (void)hipGraphDestroy(graph);
        exec = nullptr;
        graph = nullptr;
        graph_batch = 0;
    }

    size_t layer_cache_elems() const {
        return batch_cap * size_t(shape.H) * cfg.context * size_t(shape.hdp);
    }

    // Rows per workgroup and staged mesh layers for a row kernel.
    kern::Tiling tiling(int kind, size_t rows, bool decode) const {
        const int depth = kind == 2 ? int(std::max(cfg.attention_mesh_depth, cfg.ffn_mesh_depth))
                                    : int(cfg.attention_mesh_depth);
        const size_t budget = decode ? lds_limit : std::min<size_t>(lds_limit, 40960);
        auto bytes = [&](kern::Tiling t) {
            return kind == 2 ? kern::post_lds_bytes(shape, t)
                             : (kind == 1 ? kern::qkv_lds_bytes(shape, t) : kern::mesh_lds_bytes(shape, t));
        };
        kern::Tiling t{1, 0};
        if (!decode) {
            t.rpw = std::max(1, std::min(16, 2048 / shape.W));
            while (t.rpw > 1 && (rows + t.rpw - 1) / t.rpw < 512) t.rpw /= 2;
        }
        while (t.rpw > 1 && bytes(t) > budget) t.rpw /= 2;
        const size_t base = bytes(t);
        if (base > lds_limit) throw Error("model width exceeds the workgroup LDS budget", kUnsupported);
        const size_t per_layer = size_t(shape.W) * 8;
        t.stage_layers = base + per_layer + 16 <= budget ? int((budget - base - 16) / per_layer) : 0;
        t.stage_layers = std::min(t.stage_layers, depth);
        return t;
    }

    int head_rows() const {
        size_t rt = 16;
        while (rt > 1 && kern::head_lds_bytes(shape, int(rt)) > lds_limit) rt /= 2;
        return int(rt);
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
        lds_limit = std::min<size_t>(size_t(lds), 65536);
        kern::configure_lds(lds_limit);
        check(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreate");
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

        const size_t C = cfg.context;
        ks = env_int("MG_DECODE_KS", C <= 512 ? 64 : (C <= 2048 ? 128 : 256));
        ks = std::max(1, ks);
        smax = int((C + ks - 1) / ks);

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
        Et.ensure(W * cfg.vocab_size * 4);
        params.ensure(layout.count() * 4);
        std::vector<float> initial = layout.initialize(cfg, seed);
        set_parameters(initial.data(), initial.size());
        ensure_decode(std::max<size_t>(max_batch, 1), 1);
    }

    void set_parameters(const float *values, size_t n) {
        if (n != layout.count()) throw Error("parameter count does not match GPT configuration");
        validate_finite(values, n, "parameters");
        activate();
        check(hipMemcpyAsync(params.p, values, n * 4, hipMemcpyHostToDevice, stream), "upload parameters");
        // The token vectors depend only on the weights: computed once here, not per token.
        if (cfg.embedding == TokenEmbedding::Mesh) {
            kern::mesh_rows(shape, codes.as<float>(), E.as<float>(), shape.V, params.as<float>(), shape.A,
                            tiling(0, cfg.vocab_size, false), stream);
        } else {
            check(hipMemcpyAsync(E.p, params.p, cfg.vocab_size * cfg.width * 4, hipMemcpyDeviceToDevice,
                                 stream),
                  "copy table");
        }
        kern::transpose(E.as<float>(), Et.as<float>(), shape.V, shape.W, stream);
        sync();
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
            dq.ensure(batch_cap * cfg.width * 4);
            part.ensure(batch_cap * cfg.heads * size_t(smax) * (shape.hdp + 2) * 4);
            dlen.ensure(batch_cap * 4);
            drng.ensure(batch_cap * 8);
            dlogits.ensure(batch_cap * cfg.vocab_size * 4);
            dflags.ensure(4);
            cached = kNoCache;
        }
        if (grow_t || grow_b) {
            tcap = std::max(t, tcap);
            std::vector<uint32_t> keep;
            dtokens.release();
            dtokens.ensure(batch_cap * tcap * 4);
            cached = kNoCache;
            length = 0;
        }
        sync();
    }

    void ensure_workspace(size_t rows, size_t out_rows, bool kv) {
        const size_t W = cfg.width;
        wx.ensure(rows * W * 4);
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

    // All blocks over `rows`; kv(l) gives each layer's cache view.
    template <class KvOf>
    void run_blocks(const kern::Rows &rows, int nseq, KvOf kv_of, float *x, float *q, float *y, bool decode) {
        const kern::Tiling tq = tiling(1, size_t(rows.rows), decode);
        const kern::Tiling tp = tiling(2, size_t(rows.rows), decode);
        for (size_t l = 0; l < cfg.layers; ++l) {
            const Block &blk = layout.blocks[l];
            const kern::KvView kv = kv_of(l);
            kern::qkv(shape, rows, group(blk.query), group(blk.key), group(blk.value), E.as<float>(), x, q, kv,
                      rope.as<float2>(), l == 0, tq, stream);
            if (decode) {
                kern::attn_decode(shape, q, kv, rows.len, rows.rows, ks, smax, part.as<float>(), stream);
                kern::post(shape, rows, part.as<float>(), ks, smax, nullptr, kv, group(blk.projection),
                           group(blk.ffn), x, tp, stream);
            } else {
                kern::attn_prefill(shape, q, kv, nseq, rows.rows_per_seq, y, stream);
                kern::post(shape, rows, nullptr, ks, smax, y, kv, group(blk.projection), group(blk.ffn), x, tp,
                           stream);
            }
        }
    }

    kern::KvView cache_layer(size_t l) const {
        const size_t off = l * layer_cache_elems();
        return kern::KvView{kc.as<float>() + off, vc.as<float>() + off, int(cfg.context)};
    }

    // Forward over a flat batch of sequences with a per-call KV workspace.
    void forward_rows(const uint32_t *tokens, size_t n, size_t sequence, size_t out_rows) {
        ensure_workspace(n, out_rows, true);
        check(hipMemcpyAsync(wtok.p, tokens, n * 4, hipMemcpyHostToDevice, stream), "upload tokens");
        kern::Rows rows{int(n), int(sequence), nullptr, wtok.as<uint32_t>(), int(sequence), 0};
        const kern::KvView kv{wk.as<float>(), wv.as<float>(), int(sequence)};
        run_blocks(rows, int(n / sequence), [&](size_t) { return kv; }, wx.as<float>(), wq.as<float>(),
                   wy.as<float>(), false);
    }

    std::vector<float> logits(const uint32_t *tokens, size_t n, size_t sequence, bool last_only) {
        cfg.validate_tokens(tokens, n, sequence);
        activate();
        const size_t out_rows = last_only ? n / sequence : n;
        forward_rows(tokens, n, sequence, out_rows);
        kern::head(shape, wx.as<float>(), int(out_rows), last_only ? int(sequence) : 1,
                   last_only ? int(sequence) - 1 : 0, Et.as<float>(), wlogits.as<float>(), head_rows(), stream);
        std::vector<float> out(out_rows * cfg.vocab_size);
        check(hipMemcpyAsync(out.data(), wlogits.p, out.size() * 4, hipMemcpyDeviceToHost, stream),
              "download logits");
        sync();
        validate_finite(out.data(), out.size(), "logits");
        return out;
    }

    std::vector<float> hidden_states(const uint32_t *tokens, size_t n, size_t sequence) {
        cfg.validate_tokens(tokens, n, sequence);
        activate();
        forward_rows(tokens, n, sequence, 1);
        std::vector<float> out(n * cfg.width);
        check(hipMemcpyAsync(out.data(), wx.p, out.size() * 4, hipMemcpyDeviceToHost, stream), "download");
        sync();
        validate_finite(out.data(), out.size(), "features");
        return out;
    }

    // ---- generation -------------------------------------------------------

    void start(const uint32_t *prompts, size_t b, size_t p, float t, uint64_t seed, size_t reserve) {
        if (!std::isfinite(t) || t < 0.0f) throw Error("temperature must be finite and nonnegative (0 is greedy)");
        if (p == 0) throw Error("generation prompt must not be empty");
        if (b == 0) throw Error("generation batch must not be empty");
        for (size_t i = 0; i < b * p; ++i)
            if (prompts[i] >= cfg.vocab_size) throw Error("token ID is outside the vocabulary");
        activate();
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
    }

    void launch_decode_step() {
        const kern::Rows rows{int(batch), 1, dlen.as<int>(), dtokens.as<uint32_t>(), int(tcap), 0};
        run_blocks(rows, int(batch), [&](size_t l) { return cache_layer(l); }, dx.as<float>(), dq.as<float>(),
                   nullptr, true);
        kern::head(shape, dx.as<float>(), int(batch), 1, 0, Et.as<float>(), dlogits.as<float>(), head_rows(),
                   stream);
        kern::sample(shape.V, int(batch), dlogits.as<float>(), temperature, drng.as<uint64_t>(),
                     dtokens.as<uint32_t>(), int(tcap), dlen.as<int>(), dflags.as<int>(), stream);
    }

    void decode_step() {
        if (!use_graph) {
            launch_decode_step();
            return;
        }
        if (!exec || graph_batch != batch || graph_temperature != temperature) {
            drop_graph();
            check(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "begin capture");
            launch_decode_step();
            check(hipStreamEndCapture(stream, &graph), "end capture");
            check(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "instantiate graph");
            graph_batch = batch;
            graph_temperature = temperature;
        }
        check(hipGraphLaunch(exec, stream), "graph launch");
    }

    // Prefill over positions [start, start+n) of every sequence into the cache
    // (positions rebased to 0), then the head on each sequence's last row.
    void prefill_step(size_t start, size_t n) {
        ensure_workspace(batch * n, 1, false);
        const kern::Rows rows{int(batch * n), int(n), nullptr, dtokens.as<uint32_t>(), int(tcap), int(start)};
        run_blocks(rows, int(batch), [&](size_t l) { return cache_layer(l); }, wx.as<float>(), wq.as<float>(),
                   wy.as<float>(), false);
        kern::head(shape, wx.as<float>(), int(batch), int(n), int(n) - 1, Et.as<float>(), dlogits.as<float>(),
                   head_rows(), stream);
        kern::sample(shape.V, int(batch), dlogits.as<float>(), temperature, drng.as<uint64_t>(),
                     dtokens.as<uint32_t>(), int(tcap), dlen.as<int>(), dflags.as<int>(), stream);
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
    std::vector<float> out(impl_->cfg.vocab_size * impl_->cfg.width);
    check(hipMemcpy(out.data(), impl_->E.p, out.size() * 4, hipMemcpyDeviceToHost), "download embeddings");
    validate_finite(out.data(), out.size(), "features");
    return out;
}

std::vector<float> MeshGpt::hidden_states(const uint32_t *tokens, size_t n, size_t sequence) {
    return impl_->hidden_states(tokens, n, sequence);
}

void MeshGpt::generate_tokens(const uint32_t *prompts, size_t batch, size_t prompt_len, size_t count,
                              float temperature, uint64_t seed, uint32_t *out) {
    Impl &m = *impl_;
    m.start(prompts, batch, prompt_len, temperature, seed, prompt_len + count);
    for (size_t i = 0; i < count; ++i) m.step();
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
    m.step();
    m.finish();
}

void MeshGpt::decode(size_t steps) {
    Impl &m = *impl_;
    if (m.batch == 0 || m.cached != m.length - 1 || m.length - 1 + steps > m.cfg.context ||
        m.length + steps > m.tcap)
        throw Error("decode steps need a prefilled batch and must stay within the context and reserve");
    m.activate();
    for (size_t i = 0; i < steps; ++i) m.step();
    m.finish();
}

std::vector<float> MeshGpt::decode_profiled(size_t steps) {
    Impl &m = *impl_;
    if (m.batch == 0 || m.cached != m.length - 1 || m.length - 1 + steps > m.cfg.context ||
        m.length + steps > m.tcap)
        throw Error("decode steps need a prefilled batch and must stay within the context and reserve");
    m.activate();
    const size_t launches = steps * m.cfg.layers;
    std::vector<hipEvent_t> ev(2 * launches);
    for (auto &e : ev) check(hipEventCreate(&e), "hipEventCreate");
    const kern::Rows rows{int(m.batch), 1, m.dlen.as<int>(), m.dtokens.as<uint32_t>(), int(m.tcap), 0};
    const kern::Tiling tq = m.tiling(1, m.batch, true), tp = m.tiling(2, m.batch, true);
    size_t at = 0;
    for (size_t s = 0; s < steps; ++s) {
        for (size_t l = 0; l < m.cfg.layers; ++l) {
            const Block &blk = m.layout.blocks[l];
            const kern::KvView kv = m.cache_layer(l);
            kern::qkv(m.shape, rows, m.group(blk.query), m.group(blk.key), m.group(blk.value), m.E.as<float>(),
                      m.dx.as<float>(), m.dq.as<float>(), kv, m.rope.as<float2>(), l == 0, tq, m.stream);
            check(hipEventRecord(ev[2 * at], m.stream), "event");
            kern::attn_decode(m.shape, m.dq.as<float>(), kv, rows.len, rows.rows, m.ks, m.smax,
                              m.part.as<float>(), m.stream);
            check(hipEventRecord(ev[2 * at + 1], m.stream), "event");
            ++at;
            kern::post(m.shape, rows, m.part.as<float>(), m.ks, m.smax, nullptr, kv, m.group(blk.projection),
                       m.group(blk.ffn), m.dx.as<float>(), tp, m.stream);
        }
        kern::head(m.shape, m.dx.as<float>(), int(m.batch), 1, 0, m.Et.as<float>(), m.dlogits.as<float>(),
                   m.head_rows(), m.stream);
        kern::sample(m.shape.V, int(m.batch), m.dlogits.as<float>(), m.temperature, m.drng.as<uint64_t>(),
                     m.dtokens.as<uint32_t>(), int(m.tcap), m.dlen.as<int>(), m.dflags.as<int>(), m.stream);
        m.cached = m.length;
        ++m.length;
    }
    m.finish();
    std::vector<float> ms(launches);
    for (size_t i = 0; i < launches; ++i) check(hipEventElapsedTime(&ms[i], ev[2 * i], ev[2 * i + 1]), "elapsed");
    for (auto &e : ev) (void)hipEventDestroy(e);
    return ms;
}

size_t MeshGpt::sequence_length() const { return impl_->length; }

void MeshGpt::read_tokens(uint32_t *out, size_t batch, size_t length) { impl_->read_tokens(out, batch, length); }

std::vector<float> MeshGpt::last_logits() {
    Impl &m = *impl_;
    m.activate();
    std::vector<float> out(m.batch * m.cfg.vocab_size);
    check(hipMemcpy(out.data(), m.dlogits.p, out.size() * 4, hipMemcpyDeviceToHost), "download logits");
    return out;
}

hipStream_t MeshGpt::stream() const { return impl_->stream; }

void MeshGpt::synchronize() { impl_->sync(); }

}  // namespace meshgpt
