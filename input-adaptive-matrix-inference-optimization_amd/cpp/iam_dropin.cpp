// iam_dropin - command-line driver over the drop-in C++ classes.
//
//   iam_dropin generate -d DIR -p 1,2,3 -n 16 [-e 0.25] [--eager] [--max-ctx N] [--theta T]
//              [--lm dense|bucket] [--logits FILE]
//       MistralModel greedy generation (test_generation.cpp:125-317 without the
//       tokenizer: the prompt is a list of token ids); prints the new tokens
//       and the prefill / generation rates.  The LM head is the reference's
//       dense product (default) or the bucket layout.  With --eager and
//       --logits, the logits of every step after the prompt are appended to
//       FILE (fp32).
//   iam_dropin layer -d DIR -l L -e E --in h.f32 --out y.f32 [--pos P] [--max-ctx N] [--theta T]
//              [--cache f16|f32]
//       TransformerLayer::forward for positions 0..P with the same input
//       (filling the KV cache), writes the output of the last position.  The
//       caches are fp16 GQA (default) or the reference's fp32 layout.
//   iam_dropin bucketmul -d DIR -w NAME -e E --in x.f32 --out y.f32
//       BucketMul::calcDispatch + mul on one weight; writes y, prints the
//       cutoff and the selected-row count.
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iostream>
#include <sstream>
#include <string>
#include <vector>

#include "model.hpp"
#include "transformer_layer.hpp"

namespace {

struct Args {
    std::string cmd, dir, in, out, weight, prompt = "1", lm = "dense", cache = "f16", logits;
    int n = 8, layer = 0, pos = 0, max_ctx = 2048;
    float effort = 1.0f;
    double theta = 1000000.0;
    bool eager = false;
};

Args parse(int argc, char** argv)
{
    Args a;
    if (argc < 2) throw std::runtime_error("usage: iam_dropin {generate|layer|bucketmul} [options]");
    a.cmd = argv[1];
    for (int i = 2; i < argc; i++) {
        std::string s = argv[i];
        auto next = [&]() -> std::string {
            if (i + 1 >= argc) throw std::runtime_error("missing value for " + s);
            return argv[++i];
        };
        if (s == "-d") a.dir = next();
        else if (s == "-p") a.prompt = next();
        else if (s == "-n") a.n = std::stoi(next());
        else if (s == "-e") a.effort = std::stof(next());
        else if (s == "-l") a.layer = std::stoi(next());
        else if (s == "-w") a.weight = next();
        else if (s == "--pos") a.pos = std::stoi(next());
        else if (s == "--in") a.in = next();
        else if (s == "--out") a.out = next();
        else if (s == "--max-ctx") a.max_ctx = std::stoi(next());
        else if (s == "--theta") a.theta = std::stod(next());
        else if (s == "--eager") a.eager = true;
        else if (s == "--lm") a.lm = next();
        else if (s == "--cache") a.cache = next();
        else if (s == "--logits") a.logits = next();
        else throw std::runtime_error("unknown option " + s);
    }
    return a;
}

std::vector<float> read_f32(const std::string& path)
{
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open " + path);
    f.seekg(0, std::ios::end);
    size_t n = (size_t)f.tellg() / 4;
    f.seekg(0);
    std::vector<float> v(n);
    f.read(reinterpret_cast<char*>(v.data()), (std::streamsize)(n * 4));
    return v;
}

void write_f32(const std::string& path, const std::vector<float>& v)
{
    std::ofstream f(path, std::ios::binary);
    f.write(reinterpret_cast<const char*>(v.data()), (std::streamsize)(v.size() * 4));
}

double now_ms()
{
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

int cmd_generate(const Args& a)
{
    Gpu gpu;
    if (a.lm != "dense" && a.lm != "bucket") throw std::runtime_error("--lm must be dense or bucket");
    MistralModel model(&gpu, a.dir, a.max_ctx, a.theta, -1,
                       a.lm == "dense" ? MistralModel::LmHead::Dense : MistralModel::LmHead::Bucket);
    std::ofstream logf;
    if (!a.logits.empty()) logf.open(a.logits, std::ios::binary);
    std::vector<int> prompt;
    std::stringstream ss(a.prompt);
    std::string tok;
    while (std::getline(ss, tok, ',')) prompt.push_back(std::stoi(tok));
    std::vector<int> out;
    double t0 = now_ms();
    if (a.eager) {
        // test_generation.cpp:197-276: token by token with a host argmax
        const int V = model.config().vocab;
        BufferWrapper<float> logits(&gpu, (size_t)V);
        std::vector<float> host(V);
        for (size_t i = 0; i < prompt.size(); i++) model.forward(prompt[i], (int)i, a.effort, &logits);
        gpu.readBuffer(logits.buffer, (size_t)V * 4, host.data());
        if (logf) logf.write(reinterpret_cast<const char*>(host.data()), (std::streamsize)V * 4);
        int next = (int)(std::max_element(host.begin(), host.end()) - host.begin());
        for (int g = 0; g < a.n; g++) {
            out.push_back(next);
            if (g + 1 == a.n) break;
            model.forward(next, (int)prompt.size() + g, a.effort, &logits);
            gpu.readBuffer(logits.buffer, (size_t)V * 4, host.data());
            if (logf) logf.write(reinterpret_cast<const char*>(host.data()), (std::streamsize)V * 4);
            next = (int)(std::max_element(host.begin(), host.end()) - host.begin());
        }
    } else {
        out = model.generate(prompt, a.n, a.effort, true);
    }
    double t1 = now_ms();
    std::printf("tokens:");
    for (int t : out) std::printf(" %d", t);
    std::printf("\nsteps: %zu in %.2f ms\n", prompt.size() + out.size() - 1, t1 - t0);
    return 0;
}

int cmd_layer(const Args& a)
{
    Gpu gpu;
    TransformerLayer layer(&gpu, a.dir, a.layer, a.max_ctx, a.theta);
    const size_t D = TransformerLayer::HIDDEN_DIM;
    std::vector<float> h = read_f32(a.in);
    if (h.size() != D) throw std::runtime_error("layer: input must hold 4096 floats");
    if (a.cache != "f16" && a.cache != "f32") throw std::runtime_error("--cache must be f16 or f32");
    BufferWrapper<float> in(&gpu, D), hn(&gpu, D), xq(&gpu, D), xk(&gpu, 1024), xv(&gpu, 1024), xkr(&gpu, D),
        xqh(&gpu, D), xkh(&gpu, D), sc(&gpu, (size_t)32 * a.max_ctx), ao(&gpu, D), attn(&gpu, D), fxn(&gpu, D),
        ffn(&gpu, D), out(&gpu, D);
    auto run = [&](auto* kc, auto* vc) {
        kc->zero(&gpu);
        vc->zero(&gpu);
        for (int p = 0; p <= a.pos; p++) {
            in.setData(&gpu, h);
            layer.forward(&in, a.layer, p, a.effort, kc, vc, &hn, &xq, &xk, &xv, &xkr, &xqh, &xkh, &sc, &ao, &attn,
                          &fxn, &ffn, &out);
        }
    };
    if (a.cache == "f16") {
        const size_t kv = (size_t)(a.layer + 1) * a.max_ctx * 8 * 128;
        BufferWrapper<uint16_t> kc(&gpu, kv), vc(&gpu, kv);
        run(&kc, &vc);
    } else {
        // the reference's layout: [layers][max_tokens][32][128] fp32 (model.hpp:97-98)
        const size_t kv = (size_t)(a.layer + 1) * a.max_ctx * D;
        BufferWrapper<float> kc(&gpu, kv), vc(&gpu, kv);
        run(&kc, &vc);
    }
    write_f32(a.out, out.getData(&gpu));
    return 0;
}

int cmd_bucketmul(const Args& a)
{
    Gpu gpu;
    BinaryWeightLoader loader(&gpu, a.dir);
    BucketizedWeight w = loader.load(a.weight);
    const size_t R = w.meta.stats_shape.dim1, C = w.meta.buckets_shape.dim2;
    BufferWrapper<uint16_t> buckets(&gpu, std::vector<size_t>{R, C}), stats(&gpu, std::vector<size_t>{R, 4}),
        probes(&gpu, w.probes_host.size());
    buckets.setData(&gpu, w.buckets_host);
    stats.setData(&gpu, w.stats_host);
    probes.setData(&gpu, w.probes_host);
    std::vector<float> x = read_f32(a.in);
    BufferWrapper<float> in(&gpu, x.size()), y(&gpu, C * 16);
    in.setData(&gpu, x);
    BucketMul* bm = BucketMul::shared(&gpu);
    bm->calcDispatch(&in, &stats, &probes, 0, (int)w.meta.in_dim, (int)C, (int)R, a.effort);
    bm->mul(&buckets, &y);
    uint32_t S = 0;
    float cut = bm->lastCutoff(&S);
    write_f32(a.out, y.getData(&gpu));
    uint32_t bits;
    std::memcpy(&bits, &cut, 4);
    std::printf("cutoff: %.9g bits 0x%08x selected: %u\n", cut, bits, S);
    return 0;
}

}  // namespace

int main(int argc, char** argv)
{
    try {
        Args a = parse(argc, argv);
        if (a.cmd == "generate") return cmd_generate(a);
        if (a.cmd == "layer") return cmd_layer(a);
        if (a.cmd == "bucketmul") return cmd_bucketmul(a);
        throw std::runtime_error("unknown command " + a.cmd);
    } catch (const std::exception& e) {
        std::fprintf(stderr, "error: %s\n", e.what());
        return 1;
    }
}
