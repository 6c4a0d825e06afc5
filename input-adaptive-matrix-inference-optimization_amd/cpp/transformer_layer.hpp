// transformer_layer.hpp - TransformerLayer of the reference
// (transformer_layer.hpp:14-163) over the iam C ABI: pre-norm attention and
// FFN blocks with residual adds.  Same constructor and forward() arguments;
// forward() takes the reference's fp32 caches or the decode workload's fp16
// GQA caches (see attention.hpp).
#ifndef IAM_TRANSFORMER_LAYER_HPP
#define IAM_TRANSFORMER_LAYER_HPP

#include <memory>
#include <string>
#include <type_traits>

#include "attention.hpp"
#include "feedforward.hpp"

class TransformerLayer {
public:
    static constexpr int HIDDEN_DIM = 4096;   // transformer_layer.hpp:23

    // transformer_layer.hpp:55-68
    TransformerLayer(Gpu* g, const std::string& weights_dir, int layer_idx, int max_tokens = 2048,
                     double rope_theta = 1000000.0)
        : gpu(g)
    {
        attention.reset(new Attention(gpu, weights_dir, layer_idx, max_tokens, rope_theta));
        feedforward.reset(new FeedForward(gpu, weights_dir, layer_idx));
        const std::string base = weights_dir + "/layer" + std::to_string(layer_idx);
        auto a = BinaryWeightLoader::loadNpyF16(base + "_input_layernorm.npy");
        auto f = BinaryWeightLoader::loadNpyF16(base + "_post_attention_layernorm.npy");
        if (a.size() != HIDDEN_DIM || f.size() != HIDDEN_DIM)
            throw std::runtime_error("TransformerLayer: norm weights must have 4096 entries");
        attn_norm_weight.reset(new BufferWrapper<uint16_t>(gpu, HIDDEN_DIM));
        ffn_norm_weight.reset(new BufferWrapper<uint16_t>(gpu, HIDDEN_DIM));
        attn_norm_weight->setData(gpu, a);
        ffn_norm_weight->setData(gpu, f);
    }

    // transformer_layer.hpp:75-122, over fp16 GQA caches or the reference's fp32 ones
    template <typename CacheT>
    void forward(BufferWrapper<float>* input, int layer_idx, int pos, float effort, BufferWrapper<CacheT>* k_cache,
                 BufferWrapper<CacheT>* v_cache, BufferWrapper<float>* h_norm, BufferWrapper<float>* temp_xq,
                 BufferWrapper<float>* temp_xk, BufferWrapper<float>* temp_xv, BufferWrapper<float>* temp_xk_repeated,
                 BufferWrapper<float>* temp_xq_heads, BufferWrapper<float>* temp_xk_heads,
                 BufferWrapper<float>* temp_scores, BufferWrapper<float>* temp_attn_output,
                 BufferWrapper<float>* attn_out, BufferWrapper<float>* fxn, BufferWrapper<float>* ffn_out,
                 BufferWrapper<float>* output)
    {
        static_assert(std::is_same<CacheT, float>::value || std::is_same<CacheT, uint16_t>::value,
                      "caches are fp32 (the reference's layout) or fp16 (GQA)");
        rms_norm(input, attn_norm_weight.get(), h_norm);
        attention->forward(h_norm, layer_idx, pos, effort, k_cache, v_cache, temp_xq, temp_xk, temp_xv,
                           temp_xk_repeated, temp_xq_heads, temp_xk_heads, temp_scores, temp_attn_output, attn_out);
        add_residual(input, attn_out, output);
        rms_norm(output, ffn_norm_weight.get(), fxn);
        feedforward->forward(fxn, ffn_out, effort);
        add_residual(output, ffn_out, output);
    }

private:
    // transformer_layer.hpp:125-151: rmsNorm32fast + mul16x32 in one kernel
    void rms_norm(BufferWrapper<float>* input, BufferWrapper<uint16_t>* weight, BufferWrapper<float>* output)
    {
        iam_cpp::check(iam_rmsnorm_gain(gpu->ctx, input->data(), weight->data(), HIDDEN_DIM, 1e-5f, output->data()),
                       "rms_norm");
    }

    // transformer_layer.hpp:153-162
    void add_residual(BufferWrapper<float>* residual, BufferWrapper<float>* in, BufferWrapper<float>* output)
    {
        iam_cpp::check(iam_add(gpu->ctx, residual->data(), in->data(), HIDDEN_DIM, output->data()), "add_residual");
    }

    Gpu* gpu;
    std::unique_ptr<Attention> attention;
    std::unique_ptr<FeedForward> feedforward;
    std::unique_ptr<BufferWrapper<uint16_t>> attn_norm_weight, ffn_norm_weight;
};

#endif
