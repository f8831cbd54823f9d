// mesh-gpt-bench: the reference's training benchmark (src/bin/mesh-gpt-bench.rs)
// on the MI355X library, with its flags, defaults, workloads, stdout lines and
// artifacts (timings.csv, run.txt, model.bin).  Each trial restores the seeded
// weights, runs `warmup` untimed AdamW updates, then times `steps` updates by
// the host clock, the final parameter download included.
#include <chrono>
#include <cmath>
#include <cstdio>
#include <filesystem>
#include <fstream>
#include <iostream>
#include <string>
#include <vector>

#include "meshgpt_types.hpp"
#include "model.hpp"

using namespace meshgpt;

namespace {

constexpr size_t kPrime = 97;          // mesh-gpt-bench.rs:18
constexpr size_t kEquationContext = 4;  // EQUATION_CONTEXT (src/gpt/grokking.rs)

struct Options {
    GptConfig config;
    size_t steps = 100, warmup = 10, trials = 3, batch = 512, device = 0;
    std::string directory = "target/mesh-gpt-bench";
};

// cli::value (src/cli.rs:7-13) for the benchmark's unsigned flags.
size_t value(std::vector<std::string>::const_iterator &it, std::vector<std::string>::const_iterator end,
             const std::string &flag) {
    if (++it == end) throw Error("missing value for " + flag);
    const std::string &text = *it;
    try {
        size_t used = 0;
        if (text.empty() || text[0] == '-' || text[0] == '+') throw 0;
        const unsigned long long v = std::stoull(text, &used, 10);
        if (used != text.size()) throw 0;
        return size_t(v);
    } catch (...) {
        throw Error("invalid value for " + flag + ": " + text);
    }
}

const char *kHelp =
    "Usage: mesh-gpt-bench [options]\n"
    "--steps N     Timed updates per trial (default: 100)\n"
    "--warmup N    Untimed updates before each trial (default: 10)\n"
    "--trials N    Repetitions from identical weights (default: 3)\n"
    "--batch N     Fixed sequences (default: 512)\n"
    "--width N     Channels (default: 128)\n"
    "--heads N     Attention heads (default: 4)\n"
    "--context N   Tokens per sequence (default: 4)\n"
    "--layers N    Decoder blocks (default: 2)\n"
    "--attention-depth N  Mesh layers per attention projection (default: 4)\n"
    "--ffn-depth N  Mesh layers per feed-forward projection (default: 6)\n"
    "--device N    HIP device ordinal (default: 0)\n"
    "--output PATH Artifacts (default: target/mesh-gpt-bench)\n";

int run(int argc, char **argv) {
    Options o;
    o.config.width = 128;
    o.config.context = kEquationContext;
    const std::vector<std::string> args(argv + 1, argv + argc);
    for (auto it = args.cbegin(); it != args.cend(); ++it) {
        const std::string flag = *it;
        const auto end = args.cend();
        if (flag == "--steps") o.steps = value(it, end, flag);
        else if (flag == "--warmup") o.warmup = value(it, end, flag);
        else if (flag == "--trials") o.trials = value(it, end, flag);
        else if (flag == "--batch") o.batch = value(it, end, flag);
        else if (flag == "--width") o.config.width = value(it, end, flag);
        else if (flag == "--heads") o.config.heads = value(it, end, flag);
        else if (flag == "--context") o.config.context = value(it, end, flag);
        else if (flag == "--layers") o.config.layers = value(it, end, flag);
        else if (flag == "--attention-depth") o.config.attention_mesh_depth = value(it, end, flag);
        else if (flag == "--ffn-depth") o.config.ffn_mesh_depth = value(it, end, flag);
        else if (flag == "--device") o.device = value(it, end, flag);
        else if (flag == "--output") {
            if (++it == end) throw Error("missing value for " + flag);
            o.directory = *it;
        } else if (flag == "--help" || flag == "-h") {
            std::cout << kHelp;
            return 0;
        } else {
            throw Error("unknown benchmark option: " + flag);
        }
    }
    GptConfig &config = o.config;
    config.validate();
    if (o.steps == 0 || o.trials == 0 || o.batch == 0 || o.batch > kMaxRows / config.context)
        throw Error("steps/trials/batch must be positive, with at most 131072 token rows");
    // The reference's specialisations cap width and heads (mesh-gpt-bench.rs:96-103).
    if (config.width > 1024 || config.heads > 8) throw Error("benchmark requires width <=1024 and <=8 heads");
    if (config.context > 4096 || (config.context > 128 && config.width > 128))
        throw Error("benchmark context must be <=128, or <=4096 with width <=128");

    // mesh-gpt-bench.rs:134-150: the first `batch` training equations of the
    // seeded add-mod-97 split (cycled), or cyclic next-token sequences.
    const EquationDataset dataset = EquationDataset::build(kPrime, 0, 0.5, 7);
    const CharacterTokenizer tokenizer = dataset.tokenizer();
    const size_t V = tokenizer.vocab_size(), rows = o.batch * config.context;
    std::vector<uint32_t> inputs(rows), targets(rows);
    std::string workload;
    if (config.context == kEquationContext) {
        std::vector<size_t> indices(o.batch);
        for (size_t i = 0; i < o.batch; ++i) indices[i] = i % dataset.training.size();
        dataset.batch(false, indices.data(), o.batch, inputs.data(), targets.data());
        workload = "add_mod97";
    } else {
        for (size_t b = 0; b < o.batch; ++b) {
            const size_t start = (7 + b * 37) % V;
            for (size_t p = 0; p < config.context; ++p) {
                inputs[b * config.context + p] = uint32_t((start + p) % V);
                targets[b * config.context + p] = uint32_t((start + p + 1) % V);
            }
        }
        workload = "cyclic_next_token";
    }
    config.vocab_size = V;
    config.validate();
    AdamWOptions adam;
    adam.learning_rate = 0.001f;
    adam.weight_decay = 1.0f;
    adam.beta2 = 0.98f;
    MeshGpt model(int(o.device), config, 7);
    const std::vector<float> initial = model.parameters();
    const std::filesystem::path dir(o.directory);
    std::filesystem::create_directories(dir);
    std::ofstream timings(dir / "timings.csv", std::ios::binary);
    if (!timings) throw Error("cannot write " + (dir / "timings.csv").string(), kIo);
    timings << "trial,steps,total_ms,ms_per_step,first_loss,last_loss,weight_l2\n";
    {
        std::ofstream run_txt(dir / "run.txt", std::ios::binary);
        char buf[1024];
        std::snprintf(buf, sizeof buf,
                      "precision=fp32\nmodel_type=meshgpt::MeshGpt (HIP, gfx950)\nworkload=%s\nseed=7\nwidth=%zu\n"
                      "heads=%zu\nlayers=%zu\nattention_mesh_depth=%zu\nffn_mesh_depth=%zu\nvocabulary=%zu\n"
                      "context=%zu\nbatch=%zu\nsteps=%zu\nwarmup=%zu\ntrials=%zu\nlearning_rate=0.001\n"
                      "weight_decay=1\nbetas=0.9,0.98\ntiming=end_to_end_wall_clock\n"
                      "final_parameter_download=included\nvalidation_and_artifact_io=excluded\n",
                      workload.c_str(), config.width, config.heads, config.layers, config.attention_mesh_depth,
                      config.ffn_mesh_depth, config.vocab_size, config.context, o.batch, o.steps, o.warmup,
                      o.trials);
        if (!(run_txt << buf)) throw Error("cannot write " + (dir / "run.txt").string(), kIo);
    }
    for (size_t trial = 1; trial <= o.trials; ++trial) {
        model.set_parameters(initial.data(), initial.size());
        for (size_t i = 0; i < o.warmup; ++i) model.train_batch(inputs.data(), targets.data(), rows, config.context, adam);
        model.parameters();  // waits for the warm-up's last update
        const auto start = std::chrono::steady_clock::now();
        double first = 0.0, last = 0.0;
        for (size_t step = 0; step < o.steps; ++step) {
            last = model.train_batch(inputs.data(), targets.data(), rows, config.context, adam);
            if (step == 0) first = last;
        }
        const std::vector<float> parameters = model.parameters();
        const double total_ms =
            std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - start).count();
        const double ms_per_step = total_ms / double(o.steps);
        double norm = 0.0;
        for (float x : parameters) norm += double(x) * double(x);
        norm = std::sqrt(norm);
        char line[256];
        std::snprintf(line, sizeof line, "%zu,%zu,%.6f,%.6f,%.9f,%.9f,%.9f\n", trial, o.steps, total_ms, ms_per_step,
                      first, last, norm);
        timings << line;
        std::printf("trial %zu: %.3f ms/update; %.0f tokens/s; CE %.5f -> %.5f\n", trial, ms_per_step,
                    double(rows) * 1000.0 / ms_per_step, first, last);
        if (trial == 1) {
            const size_t bytes = model.allocated_device_bytes();
            std::printf("device buffers: %.1f MiB\n", double(bytes) / 1048576.0);
            std::ofstream(dir / "run.txt", std::ios::binary | std::ios::app)
                << "allocated_device_bytes=" << bytes << "\n";
            Checkpoint saved;
            saved.config = config;
            saved.tokenizer = tokenizer;
            saved.parameters = parameters;
            saved.save((dir / "model.bin").string());
        }
        std::fflush(stdout);
    }
    return 0;
}

}  // namespace

int main(int argc, char **argv) {
    try {
        return run(argc, argv);
    } catch (const std::exception &e) {
        std::cerr << "Error: \"" << e.what() << "\"\n";
        return 1;
    }
}
