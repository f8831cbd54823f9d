// mesh-gpt: the reference's `mesh-gpt generate` and `mesh-gpt train` commands
// (src/bin/mesh-gpt.rs:29-299, the geometry flags of src/bin/mesh-gpt/
// geometry.rs:5-55) on the MI355X library, with the same flags, defaults,
// output, artifacts and error text.  Extensions: --batch N for generate (N
// sequences, seeds seed..seed+N-1, one line each), --config NAME with
// --random-prompt LEN (a seeded synthetic model and prompt, no checkpoint), and
// `init` (write a seeded checkpoint).
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <filesystem>
#include <fstream>
#include <iostream>
#include <string>
#include <vector>

#include "meshgpt_types.hpp"
#include "model.hpp"

using namespace meshgpt;

namespace {

struct Options {
    std::string command = "train";
    GptConfig config;
    GptTrainOptions training;
    size_t device = 0;
    uint64_t seed = 7;
    size_t batch = 1;
    bool batch_set = false;
    std::string dataset = "data/mesh-gpt-demo.txt";
    std::string output = "target/mesh-gpt";
    std::string checkpoint;
    std::string prompt = "the little robot ";
    size_t tokens = 240;
    float temperature = 0.7f;
    std::string synthetic;
    size_t random_prompt = 0;
    bool help = false;
};

// cli::value (src/cli.rs:7-13)
template <class T>
T value(std::vector<std::string>::const_iterator &it, std::vector<std::string>::const_iterator end,
        const std::string &flag) {
    if (++it == end) throw Error("missing value for " + flag);
    const std::string &text = *it;
    try {
        size_t used = 0;
        if constexpr (std::is_same_v<T, float>) {
            float v = std::stof(text, &used);
            if (used != text.size()) throw 0;
            return v;
        } else if constexpr (std::is_same_v<T, std::string>) {
            return text;
        } else {
            if (text.empty() || text[0] == '-' || text[0] == '+') throw 0;
            unsigned long long v = std::stoull(text, &used, 10);
            if (used != text.size()) throw 0;
            return T(v);
        }
    } catch (...) {
        throw Error("invalid value for " + flag + ": " + text);
    }
}

GptConfig named_config(const std::string &name) {
    // Synthetic workloads of the benchmark (vocabulary, width, heads, layers,
    // depths, context); all butterfly meshes except the symbolic one.
    GptConfig c;
    c.connectivity = MeshConnectivity::Butterfly;
    if (name == "tiny") {
        c.vocab_size = 64, c.width = 128, c.heads = 4, c.layers = 2, c.attention_mesh_depth = 7,
        c.ffn_mesh_depth = 7, c.context = 256;
    } else if (name == "mid") {
        c.vocab_size = 256, c.width = 512, c.heads = 8, c.layers = 6, c.attention_mesh_depth = 9,
        c.ffn_mesh_depth = 9, c.context = 1024;
    } else if (name == "long") {
        c.vocab_size = 256, c.width = 512, c.heads = 8, c.layers = 4, c.attention_mesh_depth = 9,
        c.ffn_mesh_depth = 9, c.context = 8448, c.long_context = true;
    } else if (name == "high") {
        c.vocab_size = 256, c.width = 1024, c.heads = 16, c.layers = 12, c.attention_mesh_depth = 10,
        c.ffn_mesh_depth = 10, c.context = 2048;
    } else if (name == "symbolic") {
        c = GptConfig{};
        c.vocab_size = 99, c.width = 128, c.context = 4;
    } else {
        throw Error("unknown config: " + name + "; use tiny, symbolic, mid, long or high");
    }
    return c;
}

// "--rope 0|1" and the like (geometry.rs:50-55).
bool switch_value(std::vector<std::string>::const_iterator &it, std::vector<std::string>::const_iterator end,
                  const std::string &flag) {
    const uint32_t v = value<uint32_t>(it, end, flag);
    if (v > 1) throw Error(flag + " requires 0 or 1");
    return v == 1;
}

// The shared geometry flags (geometry.rs:24-48); false for any other flag.
bool geometry_option(GptConfig &c, const std::string &flag, std::vector<std::string>::const_iterator &it,
                     std::vector<std::string>::const_iterator end) {
    EmbeddingGeometry &g = c.geometry;
    if (flag == "--embedding") c.embedding = parse_embedding(value<std::string>(it, end, flag));
    else if (flag == "--connectivity") c.connectivity = parse_connectivity(value<std::string>(it, end, flag));
    else if (flag == "--embedding-form") g.form = parse_form(value<std::string>(it, end, flag));
    else if (flag == "--embedding-order") g.order = parse_order(value<std::string>(it, end, flag));
    else if (flag == "--embedding-frequency") g.frequency = value<size_t>(it, end, flag);
    else if (flag == "--embedding-harmonics") g.harmonics = value<size_t>(it, end, flag);
    else if (flag == "--equiangular-overlap") g.overlap = value<float>(it, end, flag);
    else if (flag == "--embedding-norm") g.normalization = parse_norm(value<std::string>(it, end, flag));
    else if (flag == "--freeze-embedding") g.frozen = true;
    else if (flag == "--preserve-features") g.preserve_features = value<size_t>(it, end, flag);
    else if (flag == "--geometry-seed") g.seed = value<uint64_t>(it, end, flag);
    else if (flag == "--rope") c.rope = switch_value(it, end, flag);
    else if (flag == "--qk-norm") c.qk_norm = switch_value(it, end, flag);
    else if (flag == "--xsa") c.xsa = switch_value(it, end, flag);
    else return false;
    return true;
}

// geometry::metadata (geometry.rs:56-75): the run's geometry.txt.
std::string geometry_metadata(const GptConfig &c) {
    const EmbeddingGeometry &g = c.geometry;
    auto b = [](bool v) { return v ? "true" : "false"; };
    std::string s;
    s += "embedding_form=" + std::string(name(g.form)) + "\n";
    s += "embedding_order=" + std::string(name(g.order)) + "\n";
    s += "embedding_frequency=" + std::to_string(g.frequency) + "\n";
    s += "embedding_harmonics=" + std::to_string(g.harmonics) + "\n";
    s += "equiangular_overlap=" + display_f32(g.overlap) + "\n";
    s += "embedding_norm=" + std::string(name(g.normalization)) + "\n";
    s += "freeze_embedding=" + std::string(b(g.frozen)) + "\n";
    s += "preserve_features=" + std::to_string(g.preserve_features) + "\n";
    s += "geometry_modulus=" + std::to_string(g.modulus) + "\n";
    s += "geometry_seed=" + std::to_string(g.seed) + "\n";
    s += "rope=" + std::string(b(c.rope)) + "\n";
    s += "qk_norm_enabled=" + std::string(b(c.qk_norm)) + "\n";
    s += "xsa_enabled=" + std::string(b(c.xsa)) + "\n";
    s += "geometry_supplies_arithmetic_order=" + std::string(b(g.order != EmbeddingOrder::Token)) + "\n";
    return s;
}

std::string format(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
std::string format(const char *fmt, ...) {
    char buf[512];
    va_list args;
    va_start(args, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, args);
    va_end(args);
    return buf;
}

std::string read_file(const std::string &path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw Error("cannot open dataset " + path, kIo);
    return std::string(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
}

void write_file(const std::filesystem::path &path, const std::string &text) {
    std::ofstream f(path, std::ios::binary);
    if (!(f << text)) throw Error("cannot write " + path.string(), kIo);
}

Options parse(int argc, char **argv) {
    std::vector<std::string> args(argv + 1, argv + argc);
    Options o;
    auto it = args.cbegin();
    if (it != args.cend() && !it->empty() && (*it)[0] != '-') o.command = *it++;
    for (; it != args.cend(); ++it) {
        const std::string flag = *it;
        auto end = args.cend();
        if (flag == "--width") o.config.width = value<size_t>(it, end, flag);
        else if (flag == "--heads") o.config.heads = value<size_t>(it, end, flag);
        else if (flag == "--layers") o.config.layers = value<size_t>(it, end, flag);
        else if (flag == "--context") o.config.context = value<size_t>(it, end, flag);
        else if (flag == "--attention-depth") o.config.attention_mesh_depth = value<size_t>(it, end, flag);
        else if (flag == "--ffn-depth") o.config.ffn_mesh_depth = value<size_t>(it, end, flag);
        else if (flag == "--steps") o.training.steps = value<size_t>(it, end, flag);
        else if (flag == "--learning-rate") o.training.learning_rate = value<float>(it, end, flag);
        else if (flag == "--weight-decay") o.training.weight_decay = value<float>(it, end, flag);
        else if (flag == "--report-every") o.training.report_every = value<size_t>(it, end, flag);
        else if (geometry_option(o.config, flag, it, end)) continue;
        else if (flag == "--batch") o.batch = value<size_t>(it, end, flag), o.batch_set = true;
        else if (flag == "--seed") o.seed = value<uint64_t>(it, end, flag);
        else if (flag == "--device") o.device = value<size_t>(it, end, flag);
        else if (flag == "--dataset") o.dataset = value<std::string>(it, end, flag);
        else if (flag == "--output") o.output = value<std::string>(it, end, flag);
        else if (flag == "--checkpoint") o.checkpoint = value<std::string>(it, end, flag);
        else if (flag == "--prompt") o.prompt = value<std::string>(it, end, flag);
        else if (flag == "--tokens") o.tokens = value<size_t>(it, end, flag);
        else if (flag == "--temperature") o.temperature = value<float>(it, end, flag);
        else if (flag == "--config") o.synthetic = value<std::string>(it, end, flag);
        else if (flag == "--random-prompt") o.random_prompt = value<size_t>(it, end, flag);
        else if (flag == "--help" || flag == "-h") o.help = true;
        else throw Error("unknown option: " + flag + "; use --help");
    }
    return o;
}

const char *kHelp =
    "Mesh GPT on MI355X: mesh projections, XSA, KV-cached decode, AdamW training\n"
    "Usage: mesh-gpt [train|generate|init] [options]\n\n"
    "--dataset PATH        UTF-8 training corpus (default: data/mesh-gpt-demo.txt)\n"
    "--output PATH         Artifacts (default: target/mesh-gpt)\n"
    "--checkpoint PATH     Load for generate; save for train and init (default: OUTPUT/model.bin)\n"
    "--width N             Channels, 2..1024 for train (default: 32)\n"
    "--heads N             Heads, 1..64, divides width; even channels/head with RoPE (default: 4)\n"
    "--layers N            Transformer blocks, 1..64 (default: 2)\n"
    "--context N           Maximum sequence length, 1..4096 (default: 32)\n"
    "--attention-depth N   Embedding/Q/K/V/output mesh depth, 1..256 (default: 4)\n"
    "--ffn-depth N         Feed-forward mesh depth, 1..256 (default: 6)\n"
    "--steps N             AdamW steps (default: 1000)\n"
    "--batch N             train: sequences per batch (default: 8, at most 131072 token rows);\n"
    "                      generate: sequences, sequence b samples with seed+b (default: 1)\n"
    "--learning-rate X     AdamW learning rate (default: 0.003)\n"
    "--weight-decay X      AdamW decay on all parameters (default: 0.01)\n"
    "--report-every N      Report interval (default: 100)\n"
    "--prompt TEXT         Generation prefix (default: 'the little robot ')\n"
    "--tokens N            New characters (default: 240)\n"
    "--temperature X       Sampling temperature, 0 is greedy (default: 0.7)\n"
    "--seed N              Initialization/data/sampling seed (default: 7)\n"
    "--device N            HIP device ordinal (default: 0)\n"
    "--config NAME         generate: synthetic seeded model: tiny, symbolic, mid, long or high\n"
    "--random-prompt LEN   With --config: LEN seeded uniform token ids as the prompt\n\n"
    "--embedding mesh|table  Tied embedding parameterization (default: mesh)\n"
    "--connectivity neighbor|butterfly  Mesh parents (default: neighbor)\n"
    "--embedding-form NAME  parity (default), circle, fourier, orthogonal, simplex,\n"
    "                       equiangular, antipodal, hypercube, signed-permutations, sphere\n"
    "--embedding-order NAME token (default), residue, discrete-log; arithmetic order is grok-only\n"
    "--embedding-frequency N  First cyclic frequency (default: 1)\n"
    "--embedding-harmonics N  Consecutive Fourier pairs (default: 1)\n"
    "--equiangular-overlap X  Off-diagonal cosine, -1/(V-1)<=X<=1 (default: 0)\n"
    "--embedding-norm NAME  none (default), unit, rms; effective tied vectors\n"
    "--freeze-embedding     Freeze embedding parameters throughout AdamW\n"
    "--preserve-features N  Inject N code coordinates and protect them through residual blocks\n"
    "--geometry-seed N      Sphere-code seed (default: 0)\n"
    "--rope 0|1             Slice RoPE (default: 1)\n"
    "--qk-norm 0|1          Per-head RMS QK normalization (default: 1)\n"
    "--xsa 0|1              Exclusive projection after attention (default: 1)\n";

// report (mesh-gpt.rs:289-299): one stdout line and one loss.csv row.
void report(std::ofstream &history, size_t step, double train, double validation) {
    std::printf("step %6zu: train CE=%.5f, validation CE=%.5f, perplexity=%.3f\n", step, train, validation,
                std::exp(validation));
    std::fflush(stdout);
    history << format("%zu,%.9f,%.9f,%.9f\n", step, train, validation, std::exp(validation));
}

// train (mesh-gpt.rs:173-287): the demo corpus split 90/10, a seeded batch per
// step, a report every `report_every` steps and at the end, then the
// checkpoint, a sample from the trained model and the run's record.
int train(Options &o, const std::string &checkpoint) {
    const std::string text = read_file(o.dataset);
    const CharacterTokenizer tokenizer = CharacterTokenizer::from_text(text);
    GptConfig &config = o.config;
    config.vocab_size = tokenizer.vocab_size();
    config.validate();
    o.training.validate();
    if (o.prompt.empty()) throw Error("generation prompt must not be empty");
    tokenizer.encode(o.prompt);
    const TextDataset dataset(tokenizer.encode(text), config);
    const size_t C = config.context;
    if (o.batch == 0 || o.batch > kMaxRows / C) throw Error("invalid dataset batch dimensions");
    const size_t rows = C * o.batch;
    std::vector<uint32_t> ex(rows), ey(rows), x(rows), y(rows);
    dataset.batch(true, C, o.batch, 101, ex.data(), ey.data());
    MeshGpt model(int(o.device), config, o.seed);
    std::printf("Mesh GPT: blocks=%zu, width=%zu, heads=%zu, context=%zu, vocabulary=%zu, parameters=%zu\n",
                config.layers, config.width, config.heads, C, tokenizer.vocab_size(), config.parameter_count());
    auto b = [](bool v) { return v ? "true" : "false"; };
    std::printf("Meshes: Q/K/V/output depth=%zu, FFN depth=%zu; embeddings=%s, form=%s, norm=%s, protected=%zu; "
                "RoPE=%s, QK-Norm=%s, XSA=%s\n",
                config.attention_mesh_depth, config.ffn_mesh_depth, name(config.embedding),
                name(config.geometry.form), name(config.geometry.normalization), config.geometry.preserve_features,
                b(config.rope), b(config.qk_norm), b(config.xsa));
    const std::filesystem::path output(o.output);
    std::filesystem::create_directories(output);
    write_file(output / "geometry.txt", geometry_metadata(config));
    std::ofstream history(output / "loss.csv", std::ios::binary);
    if (!history) throw Error("cannot write " + (output / "loss.csv").string(), kIo);
    history << "step,train_cross_entropy,validation_cross_entropy,validation_perplexity\n";
    dataset.batch(false, C, o.batch, o.seed, x.data(), y.data());
    const double initial_train = model.cross_entropy(x.data(), y.data(), rows, C);
    const double initial_validation = model.cross_entropy(ex.data(), ey.data(), rows, C);
    report(history, 0, initial_train, initial_validation);
    AdamWOptions adam;
    adam.learning_rate = o.training.learning_rate;
    adam.weight_decay = o.training.weight_decay;
    const auto start = std::chrono::steady_clock::now();
    double sum = 0.0;
    size_t count = 0;
    for (size_t step = 1; step <= o.training.steps; ++step) {
        dataset.batch(false, C, o.batch, o.seed + step, x.data(), y.data());
        sum += model.train_batch(x.data(), y.data(), rows, C, adam);
        ++count;
        if (step % o.training.report_every == 0 || step == o.training.steps) {
            report(history, step, sum / double(count), model.cross_entropy(ex.data(), ey.data(), rows, C));
            sum = 0.0;
            count = 0;
        }
    }
    history.flush();
    const double elapsed = std::chrono::duration<double>(std::chrono::steady_clock::now() - start).count();
    std::printf("Training time: %.3f s\n", elapsed);
    Checkpoint saved;
    saved.config = config;
    saved.tokenizer = tokenizer;
    saved.parameters = model.parameters();
    const std::filesystem::path path(checkpoint);
    if (path.has_parent_path()) std::filesystem::create_directories(path.parent_path());
    saved.save(checkpoint);
    const std::string generated = model.generate(tokenizer, o.prompt, o.tokens, o.temperature, o.seed);
    write_file(output / "sample.txt", generated);
    const double final_validation = model.cross_entropy(ex.data(), ey.data(), rows, C);
    std::string run =
        "attention=xsa\npositions=slice_rope\nrope_base=10000\nnormalization=pre_rmsnorm\nrmsnorm_epsilon=1e-5\n"
        "rmsnorm_affine=false\nqk_norm=per_head_rmsnorm\nbias=false\nembeddings=mesh\n"
        "token_codes=signed_binary_parity_radix\nembedding_depth=attention_mesh_depth\nhead=tied_mesh_embeddings\n"
        "all_parameters=mesh_edges\n";
    run += "dataset=" + o.dataset + "\n";
    run += format("seed=%llu\nsteps=%zu\nbatch=%zu\nwidth=%zu\nheads=%zu\nlayers=%zu\ncontext=%zu\n"
                  "attention_mesh_depth=%zu\nffn_mesh_depth=%zu\nparameters=%zu\n",
                  (unsigned long long)o.seed, o.training.steps, o.batch, config.width, config.heads, config.layers,
                  C, config.attention_mesh_depth, config.ffn_mesh_depth, config.parameter_count());
    run += "learning_rate=" + display_f32(o.training.learning_rate) + "\n";
    run += "weight_decay=" + display_f32(o.training.weight_decay) + "\n";
    run += format("training_seconds=%.6f\ninitial_validation_cross_entropy=%.9f\n"
                  "final_validation_cross_entropy=%.9f\n",
                  elapsed, initial_validation, final_validation);
    write_file(output / "run.txt", run);
    std::printf("Saved checkpoint to %s\n\n%s\n", checkpoint.c_str(), generated.c_str());
    return 0;
}

int run(int argc, char **argv) {
    Options o = parse(argc, argv);
    if (o.help) {
        std::cout << kHelp;
        return 0;
    }
    if (!std::isfinite(o.temperature) || o.temperature < 0.0f)
        throw Error("temperature must be finite and nonnegative");
    const std::string checkpoint = o.checkpoint.empty() ? o.output + "/model.bin" : o.checkpoint;
    if (o.command == "train") {
        if (!o.batch_set) o.batch = 8;  // the training default (mesh-gpt.rs:54)
        return train(o, checkpoint);
    }
    if (o.command == "generate") {
        GptConfig config;
        CharacterTokenizer tokenizer;
        std::vector<float> parameters;
        std::vector<uint32_t> prompt;
        if (!o.synthetic.empty()) {
            config = named_config(o.synthetic);
            std::vector<uint32_t> chars(config.vocab_size);
            for (size_t i = 0; i < chars.size(); ++i) chars[i] = uint32_t(config.vocab_size == 64 ? 0x20 + i : i);
            tokenizer = CharacterTokenizer::from_characters(chars);
            parameters = config.initial_parameters(o.seed);
            if (o.random_prompt) {
                Random r(o.seed);
                for (size_t i = 0; i < o.batch * o.random_prompt; ++i)
                    prompt.push_back(uint32_t(r.index(config.vocab_size)));
            }
        } else {
            Checkpoint saved = Checkpoint::load(checkpoint);
            config = saved.config;
            tokenizer = saved.tokenizer;
            parameters = std::move(saved.parameters);
        }
        MeshGpt model(int(o.device), config, o.seed, o.batch);
        model.set_parameters(parameters.data(), parameters.size());
        if (prompt.empty() && !o.batch_set) {
            std::cout << model.generate(tokenizer, o.prompt, o.tokens, o.temperature, o.seed) << "\n";
            return 0;
        }
        if (prompt.empty()) {
            std::vector<uint32_t> one = tokenizer.encode(o.prompt);
            if (one.empty()) throw Error("generation prompt must not be empty");
            for (size_t b = 0; b < o.batch; ++b) prompt.insert(prompt.end(), one.begin(), one.end());
        }
        const size_t p = prompt.size() / o.batch, n = p + o.tokens;
        std::vector<uint32_t> out(o.batch * n);
        model.generate_tokens(prompt.data(), o.batch, p, o.tokens, o.temperature, o.seed, out.data());
        for (size_t b = 0; b < o.batch; ++b) std::cout << tokenizer.decode(out.data() + b * n, n) << "\n";
        return 0;
    }
    if (o.command == "init") {
        std::FILE *f = std::fopen(o.dataset.c_str(), "rb");
        if (!f) throw Error("cannot open dataset " + o.dataset, kIo);
        std::string text;
        char buf[4096];
        size_t got;
        while ((got = std::fread(buf, 1, sizeof buf, f)) > 0) text.append(buf, got);
        std::fclose(f);
        Checkpoint ck;
        ck.tokenizer = CharacterTokenizer::from_text(text);
        ck.config = o.config;
        ck.config.vocab_size = ck.tokenizer.vocab_size();
        ck.parameters = ck.config.initial_parameters(o.seed);
        ck.save(checkpoint);
        std::cout << "Saved seed-" << o.seed << " checkpoint to " << checkpoint << "\n";
        return 0;
    }
    if (o.command == "grok" || o.command == "grok-simple" || o.command == "verify")
        throw Error("the " + o.command +
                    " command is not part of this build; it provides train and generate (parity checks live in "
                    "tests/)");
    throw Error("unknown command: " + o.command + "; use train, generate or init");
}

}  // namespace

int main(int argc, char **argv) {
    try {
        return run(argc, argv);
    } catch (const std::exception &e) {
        // A Rust main returning Err prints the error's Debug form.
        std::cerr << "Error: \"" << e.what() << "\"\n";
        return 1;
    }
}
