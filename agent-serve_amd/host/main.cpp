// tinferno_hip: the reference CLI (main.cpp:40-146) with the token loop on the MI355X.
//
// Same flags and output: prompt ids from --tokens (no BOS added, main.cpp:99) or from
// --prompt through the byte-level BPE tokenizer (BOS unless --no-bos), prefill, then up to
// --n-predict tokens sampled on the GPU (greedy at --temp 0, else temperature / top-p with
// the reference's std::mt19937 draws), stopping when the sampled id is eos after the first
// (main.cpp:112-122); prefill/decode rates on stderr. Adds --device, --decode-path,
// --device-loop and TF_HIP_MAPS_AT_EXIT (below).
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <numeric>
#include <random>
#include <sstream>
#include <string>
#include <thread>
#include <vector>

#include "model.hpp"
#include "tokenizer.hpp"

using namespace tfh;

namespace {

[[noreturn]] void die(const std::string& msg) {
    std::fprintf(stderr, "tinferno: %s\n", msg.c_str());
    std::exit(1);
}

double now_s() {
    using clock = std::chrono::steady_clock;
    return std::chrono::duration<double>(clock::now().time_since_epoch()).count();
}

void usage() {
    std::fprintf(stderr,
                 "tinferno_hip - tinferno's token loop on an MI355X (gfx950)\n"
                 "\n"
                 "usage: tinferno_hip --model PATH [options]\n"
                 "  --model PATH         GGUF file (F32 / F16 / Q8_0 / Q4_0 / Q4_1 / Q6_K)\n"
                 "  --prompt TEXT        prompt string\n"
                 "  --tokens 1,2,3       skip tokenizer; comma-separated ids\n"
                 "  --n-predict N        tokens to generate (default 64)\n"
                 "  --stage v0..v5       stage preset (default v2; selects the KV layout)\n"
                 "  --threads N          accepted for compatibility (the GPU does not use it)\n"
                 "  --temp T             temperature; 0 = greedy (default 0)\n"
                 "  --top-p P            nucleus sampling (default 0.9)\n"
                 "  --seed N             rng seed (default 42)\n"
                 "  --max-seq N          KV cache length (default 4096)\n"
                 "  --kv-layout seq|head override KV layout\n"
                 "  --no-bos             do not prepend BOS\n"
                 "  --device N           HIP device (default 0)\n"
                 "  --decode-path P      step (persistent kernel, the default) | graph; a step kernel the\n"
                 "                       GPU refuses (another process holds it) runs as graph\n"
                 "  --device-loop        greedy tokens from one tf_hip_generate call (one launch of the\n"
                 "                       persistent kernel, as bench.py times it) instead of a decode per token\n"
                 "  --profile            print the per-kernel-class breakdown of one greedy pass\n");
}

std::vector<int> parse_tokens(const std::string& s) {
    std::vector<int> v;
    std::stringstream ss(s);
    std::string item;
    while (std::getline(ss, item, ','))
        if (!item.empty()) v.push_back(std::stoi(item));
    return v;
}

}  // namespace

int main(int argc, char** argv) {
    std::string model_path, prompt, token_str, stage = "v2", kv_layout, decode_path;
    int n_predict = 64, seed = 42, max_seq = 4096, device = 0;
    float temp = 0, topp = 0.9f;
    bool profile = false, add_bos = true, device_loop = false;
    for (int i = 1; i < argc; ++i) {
        std::string a = argv[i];
        auto next = [&]() -> std::string {
            if (i + 1 >= argc) die("missing value for " + a);
            return argv[++i];
        };
        if (a == "--model") model_path = next();
        else if (a == "--prompt") prompt = next();
        else if (a == "--tokens") token_str = next();
        else if (a == "--n-predict") n_predict = std::stoi(next());
        else if (a == "--stage") stage = next();
        else if (a == "--threads") (void)std::stoi(next());
        else if (a == "--temp") temp = std::stof(next());
        else if (a == "--top-p") topp = std::stof(next());
        else if (a == "--seed") seed = std::stoi(next());
        else if (a == "--max-seq") max_seq = std::stoi(next());
        else if (a == "--kv-layout") kv_layout = next();
        else if (a == "--device") device = std::stoi(next());
        else if (a == "--decode-path") decode_path = next();
        else if (a == "--device-loop") device_loop = true;
        else if (a == "--no-bos") add_bos = false;
        else if (a == "--pin") {
        } else if (a == "--profile") profile = true;
        else if (a == "-h" || a == "--help") {
            usage();
            return 0;
        } else {
            die("unknown flag " + a);
        }
    }
    if (model_path.empty()) {
        usage();
        return 1;
    }
    try {
        int hw = (int)std::thread::hardware_concurrency();
        RunConfig cfg = stage_preset(stage, hw > 0 ? hw : 4);
        cfg.n_predict = n_predict;
        cfg.temperature = temp;
        cfg.top_p = topp;
        cfg.seed = seed;
        cfg.max_seq = max_seq;
        cfg.device = device;
        cfg.profile = profile;
        if (kv_layout == "head") cfg.kv_layout = KVLayout::HeadMajor;
        if (kv_layout == "seq") cfg.kv_layout = KVLayout::SeqMajor;
        Model model(model_path, cfg);
        const Tokenizer tok(model.gguf());
        // without the flag the library's choice stands (step, or TF_HIP_DECODE_PATH)
        if (decode_path == "graph" || decode_path == "step") {
            if (tf_hip_set_decode_path(model.ctx(), decode_path == "graph" ? TF_HIP_PATH_GRAPH : TF_HIP_PATH_STEP))
                die("tf_hip_set_decode_path failed");
        } else if (!decode_path.empty()) {
            die("--decode-path takes step or graph");
        }
        std::fprintf(stderr, "%s\n", model.describe().c_str());
        const std::vector<int> ids = !token_str.empty() ? parse_tokens(token_str) : tok.encode(prompt, add_bos);
        if (ids.empty()) die("empty prompt");

        std::vector<float> logits((size_t)model.n_vocab());
        double t0 = now_s();
        model.prefill(ids.data(), (int)ids.size(), logits.data());
        const double t_prefill = now_s() - t0;

        std::mt19937 rng((unsigned)seed);
        std::vector<int> gen;
        t0 = now_s();
        if (device_loop) {
            // the greedy loop as one tf_hip_generate call (one launch of the persistent kernel),
            // the tokens printed up to the first eos after the first token
            if (temp > 0) die("--device-loop needs --temp 0");
            std::vector<int32_t> out((size_t)std::max(n_predict, 0));
            if (n_predict > 0) model.generate(n_predict, out.data());
            for (int i = 0; i < n_predict; ++i) {
                if (out[(size_t)i] == model.eos() && i > 0) break;
                gen.push_back(out[(size_t)i]);
                std::fputs(tok.decode_one(out[(size_t)i]).c_str(), stdout);
            }
            std::fflush(stdout);
        } else {
            for (int i = 0; i < n_predict; ++i) {
                const int id = model.sample(temp, topp, rng);
                if (id == model.eos() && i > 0) break;
                gen.push_back(id);
                std::fputs(tok.decode_one(id).c_str(), stdout);
                std::fflush(stdout);
                model.decode(id, nullptr);
            }
        }
        const double t_decode = now_s() - t0;
        std::fputc('\n', stdout);
        const int n_in = (int)ids.size(), n_out = (int)gen.size();
        std::fprintf(stderr, "\nprefill %d tok in %.3fs  (%.1f tok/s)  TTFT %.3fs\n", n_in, t_prefill,
                     n_in / t_prefill, t_prefill);
        std::fprintf(stderr, "decode  %d tok in %.3fs  (%.1f tok/s)\n", n_out, t_decode,
                     n_out / std::max(t_decode, 1e-9));
        if (profile && model.n_pos() < max_seq) {
            const int n = std::min(8, max_seq - model.n_pos());
            std::vector<int32_t> out((size_t)n);
            float ms[7];
            int32_t launches[7];
            double bytes[7];
            if (tf_hip_profile_generate(model.ctx(), n, out.data(), ms, launches, bytes) == 0) {
                double tot = 0;
                for (float m : ms) tot += m;
                std::fprintf(stderr, "kernels over %d greedy steps:", n);
                for (int k = 0; k < 7; ++k)
                    std::fprintf(stderr, "  %s %.1f%% (%.1f GB/s)", tf_hip_kernel_class_name(k), tot > 0 ? 100.0 * ms[k] / tot : 0.0,
                                 ms[k] > 0 ? bytes[k] / (ms[k] * 1e-3) / 1e9 : 0.0);
                std::fprintf(stderr, "\n");
            }
        }
    } catch (const std::exception& e) {
        die(e.what());
    }
    // TF_HIP_MAPS_AT_EXIT=<file>: the process's memory map once the model is gone, for
    // placing the addresses of a crash in library teardown after main returns
    if (const char* maps_out = std::getenv("TF_HIP_MAPS_AT_EXIT")) {
        FILE* in = std::fopen("/proc/self/maps", "r");
        FILE* out = in ? std::fopen(maps_out, "w") : nullptr;
        char buf[4096];
        size_t n;
        while (out && (n = std::fread(buf, 1, sizeof(buf), in)) > 0) std::fwrite(buf, 1, n, out);
        if (out) std::fclose(out);
        if (in) std::fclose(in);
    }
    return 0;
}
