// model.hpp - MistralModel of the reference (model.hpp:15-238) over the iam
// C ABI.  The constructor reads the reference's weights directory:
//   layer{L}_{q,k,v,o,gate,up,down}_proj_bucketmul_fp16_{buckets,stats,probes}.bin + _meta.txt
//   layer{L}_input_layernorm.npy, layer{L}_post_attention_layernorm.npy
//   embed_tokens.npy, norm_weight.npy, lm_head.npy (dense fp16 [vocab][dim])
// into one iam_model.  The LM head is the reference's dense fp16 product
// (matmul16x32, model.hpp:207-227) by default; LmHead::Bucket bucketizes
// lm_head.npy on the GPU at load and runs the head through the same
// input-adaptive product at the caller's effort (the decode workload's
// head).  forward() keeps the reference's signature and ends with eval()
// (model.hpp:230).
#ifndef IAM_MODEL_HPP
#define IAM_MODEL_HPP

#include <fstream>
#include <memory>
#include <string>
#include <vector>

#include "binary_loader.hpp"
#include "bucket_mul.hpp"

class MistralModel {
public:
    enum class LmHead { Dense, Bucket };

    MistralModel(Gpu* g, const std::string& weights_dir, int max_tokens = 2048, double rope_theta = 1000000.0,
                 int n_layers = -1, LmHead lm_head = LmHead::Dense)
        : gpu(g), head(lm_head)
    {
        std::vector<size_t> eshape, lshape;
        auto embed = BinaryWeightLoader::loadNpyF16(weights_dir + "/embed_tokens.npy", &eshape);
        auto norm = BinaryWeightLoader::loadNpyF16(weights_dir + "/norm_weight.npy");
        auto lm = BinaryWeightLoader::loadNpyF16(weights_dir + "/lm_head.npy", &lshape);
        if (eshape.size() != 2 || lshape.size() != 2 || eshape[1] != lshape[1] || eshape[0] != lshape[0])
            throw std::runtime_error("MistralModel: embed_tokens and lm_head must both be [vocab][dim]");
        BinaryWeightLoader loader(gpu, weights_dir);
        if (n_layers < 0) {
            n_layers = 0;
            while (std::ifstream(weights_dir + "/layer" + std::to_string(n_layers) +
                                 "_q_proj_bucketmul_fp16_meta.txt"))
                n_layers++;
        }
        if (n_layers < 1) throw std::runtime_error("MistralModel: no layer weights in " + weights_dir);
        const WeightMetadata gate = BinaryWeightLoader::readMetadata(weights_dir + "/layer0_gate_proj_bucketmul_fp16_meta.txt");
        const WeightMetadata kproj = BinaryWeightLoader::readMetadata(weights_dir + "/layer0_k_proj_bucketmul_fp16_meta.txt");
        cfg.n_layers = n_layers;
        cfg.dim = (int)eshape[1];
        cfg.ffn_dim = (int)gate.out_dim;
        cfg.head_dim = 128;
        cfg.n_heads = cfg.dim / cfg.head_dim;
        cfg.n_kv_heads = (int)kproj.out_dim / cfg.head_dim;
        cfg.vocab = (int)eshape[0];
        cfg.max_ctx = max_tokens;
        cfg.rope_theta = rope_theta;
        cfg.norm_eps = 1e-5f;   // aux.cl:190
        iam_cpp::check(iam_model_create(gpu->ctx, &cfg, &m), "MistralModel: create");

        static const char* kNames[7] = {"q", "k", "v", "o", "gate", "up", "down"};
        static const char* kSlots[7] = {"wq", "wk", "wv", "wo", "w1", "w3", "w2"};
        for (int L = 0; L < n_layers; L++) {
            for (int k = 0; k < 7; k++) {
                BucketizedWeight w = loader.loadLayerWeight(L, kNames[k]);
                const std::string base = "layer" + std::to_string(L) + "." + kSlots[k];
                put(base + ".buckets", w.buckets_host);
                put(base + ".stats", w.stats_host);
                put(base + ".probes", w.probes_host);
                compact(base);
            }
            put("layer" + std::to_string(L) + ".attn_gain",
                BinaryWeightLoader::loadNpyF16(weights_dir + "/layer" + std::to_string(L) + "_input_layernorm.npy"));
            put("layer" + std::to_string(L) + ".ffn_gain",
                BinaryWeightLoader::loadNpyF16(weights_dir + "/layer" + std::to_string(L) +
                                               "_post_attention_layernorm.npy"));
        }
        put("embed", embed);
        put("final_gain", norm);
        lm_dense.reset(new BufferWrapper<uint16_t>(gpu, lm.size()));
        lm_dense->setData(gpu, lm);
        if (head == LmHead::Bucket) {
            // dense LM head -> bucket layout on the GPU (preprocess_layer_fixed_gpu.py:110-242)
            iam_cpp::check(iam_bucketize(gpu->ctx, lm_dense->data(), cfg.vocab, cfg.dim, tensor("lm_head.buckets"),
                                         tensor("lm_head.stats"), tensor("lm_head.probes")),
                           "MistralModel: bucketize LM head");
            compact("lm_head");
            gpu->eval();
            lm_dense.reset();
        } else {
            iam_cpp::check(iam_model_set_lm_dense(m, lm_dense->data()), "MistralModel: dense LM head");
        }
        gpu->eval();
    }

    ~MistralModel()
    {
        iam_model_destroy(m);
        lm_dense.reset();
    }

    MistralModel(const MistralModel&) = delete;
    MistralModel& operator=(const MistralModel&) = delete;

    // model.hpp:152-231
    void forward(int token_id, int pos, float effort, BufferWrapper<float>* logits_out)
    {
        iam_cpp::check(iam_model_forward(m, token_id, pos, effort, logits_out->data()), "MistralModel::forward");
        gpu->eval();
    }

    // greedy generation of test_generation.cpp:197-276 with the step
    // replayed as a captured graph
    std::vector<int> generate(const std::vector<int>& prompt, int n_new, float effort, bool use_graph = true)
    {
        std::vector<int> out(n_new);
        iam_cpp::check(iam_model_generate(m, prompt.data(), (int)prompt.size(), n_new, effort, use_graph ? 1 : 0,
                                          out.data()),
                       "MistralModel::generate");
        return out;
    }

    // model.hpp:233-237
    void reset_caches() { iam_cpp::check(iam_model_reset_caches(m), "MistralModel::reset_caches"); }

    const iam_model_config& config() const { return cfg; }
    LmHead lm_head() const { return head; }
    iam_model* handle() const { return m; }

private:
    uint16_t* tensor(const std::string& name)
    {
        void* p = nullptr;
        size_t n = 0;
        iam_cpp::check(iam_model_tensor(m, name.c_str(), &p, &n), "MistralModel: tensor");
        return static_cast<uint16_t*>(p);
    }

    void put(const std::string& name, const std::vector<uint16_t>& host)
    {
        void* p = nullptr;
        size_t n = 0;
        iam_cpp::check(iam_model_tensor(m, name.c_str(), &p, &n), "MistralModel: tensor");
        if (host.size() * 2 > n) throw std::runtime_error("MistralModel: " + name + " larger than the model tensor");
        iam_cpp::check(iam_write(gpu->ctx, p, 0, host.data(), host.size() * 2), "MistralModel: upload");
    }

    void compact(const std::string& base)
    {
        void *s = nullptr, *s3 = nullptr;
        size_t ns = 0, n3 = 0;
        iam_cpp::check(iam_model_tensor(m, (base + ".stats").c_str(), &s, &ns), "MistralModel: tensor");
        iam_cpp::check(iam_model_tensor(m, (base + ".stats3").c_str(), &s3, &n3), "MistralModel: tensor");
        iam_cpp::check(iam_stats_compact(gpu->ctx, (const uint16_t*)s, n3 / 2, 4, 3, (uint16_t*)s3), "stats_compact");
    }

    Gpu* gpu;
    LmHead head;
    iam_model* m = nullptr;
    iam_model_config cfg{};
    std::unique_ptr<BufferWrapper<uint16_t>> lm_dense;   // the dense head's matrix (LmHead::Dense)
};

#endif
