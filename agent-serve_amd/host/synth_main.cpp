// tinferno_synth: write a seeded synthetic GGUF for one of the named presets.
//
//   tinferno_synth --preset llama1b_q8 --out /tmp/m.gguf [--seed 42] [--threads N] [--prompt N]
//
// Prints one JSON line: preset, path, weight_bytes, seed and (with --prompt N) the
// N prompt ids drawn from the same seed.
#include <cstdio>
#include <cstdlib>
#include <stdexcept>
#include <string>

#include "synth.hpp"

int main(int argc, char** argv) {
    std::string preset, out;
    long long seed = -1;
    int threads = 0, n_prompt = 0;
    for (int i = 1; i < argc; ++i) {
        std::string a = argv[i];
        auto next = [&]() -> std::string {
            if (i + 1 >= argc) {
                std::fprintf(stderr, "tinferno_synth: missing value for %s\n", a.c_str());
                std::exit(1);
            }
            return argv[++i];
        };
        if (a == "--preset") preset = next();
        else if (a == "--out") out = next();
        else if (a == "--seed") seed = std::stoll(next());
        else if (a == "--threads") threads = std::stoi(next());
        else if (a == "--prompt") n_prompt = std::stoi(next());
        else {
            std::fprintf(stderr, "tinferno_synth: unknown flag %s\n", a.c_str());
            return 1;
        }
    }
    tfh::SynthSpec spec;
    if (preset.empty() || out.empty() || !tfh::synth_preset(preset, &spec)) {
        std::fprintf(stderr, "usage: tinferno_synth --preset NAME --out PATH [--seed N] [--threads N] [--prompt N]\n");
        std::fprintf(stderr, "presets:");
        for (const auto& n : tfh::synth_preset_names()) std::fprintf(stderr, " %s", n.c_str());
        std::fprintf(stderr, "\n");
        return 1;
    }
    if (seed >= 0) spec.seed = (uint64_t)seed;
    try {
        const uint64_t wb = tfh::synth_write(spec, out, threads);
        std::printf("{\"preset\": \"%s\", \"path\": \"%s\", \"weight_bytes\": %llu, \"seed\": %llu, \"prompt\": [",
                    preset.c_str(), out.c_str(), (unsigned long long)wb, (unsigned long long)spec.seed);
        const auto ids = tfh::synth_prompt(spec.seed, n_prompt, spec.n_vocab);
        for (size_t i = 0; i < ids.size(); ++i) std::printf("%s%d", i ? ", " : "", ids[i]);
        std::printf("]}\n");
    } catch (const std::exception& e) {
        std::fprintf(stderr, "tinferno_synth: %s\n", e.what());
        return 1;
    }
    return 0;
}
