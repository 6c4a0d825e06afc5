// attention.hpp - Attention of the reference (attention.hpp:19-405) over the
// iam C ABI.  Same constructor and forward() argument list; the body is
// q/k/v as one cutoff launch and one walk launch, RoPE of q and k fused with
// the KV append, split-context decode attention, then o.
//
// Two cache forms.  With BufferWrapper<float> caches forward() is the
// reference's own: K and V repeated to the 32 query heads, fp32
// [layers][max_tokens][32][128] (model.hpp:97-98), and its fp32 attention
// arithmetic (iam_attention_decode_f32).  With BufferWrapper<uint16_t>
// caches it is the decode workload's: fp16 GQA ([layers][max_tokens][8][128]),
// read in place, evaluated in fp64.  RoPE theta and the KV capacity are
// constructor parameters (attention.hpp:26-27 fixes 1e6 and 2048).  The
// temporaries the reference threads through (temp_xk_repeated,
// temp_xk_heads, temp_scores) are accepted and unused: the heads are
// repeated by the append and the scores never leave the kernels.
#ifndef IAM_ATTENTION_HPP
#define IAM_ATTENTION_HPP

#include <memory>
#include <string>
#include <vector>

#include "bucket_weight.hpp"

class Attention {
public:
    static constexpr int NUM_HEADS = 32;        // attention.hpp:21-24
    static constexpr int NUM_KV_HEADS = 8;
    static constexpr int HEAD_DIM = 128;
    static constexpr int HIDDEN_DIM = NUM_HEADS * HEAD_DIM;

    Attention(Gpu* g, const std::string& weights_dir, int layer_idx, int max_tokens = 2048,
              double rope_theta = 1000000.0)
        : gpu(g), max_tokens_(max_tokens)
    {
        BinaryWeightLoader loader(gpu, weights_dir);
        const std::string prefix = "layer" + std::to_string(layer_idx);
        wq.reset(new BucketWeight(gpu, loader.load(prefix + "_q_proj_bucketmul_fp16")));
        wk.reset(new BucketWeight(gpu, loader.load(prefix + "_k_proj_bucketmul_fp16")));
        wv.reset(new BucketWeight(gpu, loader.load(prefix + "_v_proj_bucketmul_fp16")));
        wo.reset(new BucketWeight(gpu, loader.load(prefix + "_o_proj_bucketmul_fp16")));
        if (wq->out_dim != HIDDEN_DIM || wk->out_dim != NUM_KV_HEADS * HEAD_DIM ||
            wv->out_dim != NUM_KV_HEADS * HEAD_DIM || wo->in_dim != HIDDEN_DIM)
            throw std::runtime_error("Attention: unexpected projection shapes");
        // precompute_rope_cache (attention.hpp:207-235) as one table
        std::vector<float> table((size_t)max_tokens * HEAD_DIM);
        iam_cpp::check(iam_rope_table(rope_theta, HEAD_DIM, max_tokens, table.data()), "rope_table");
        rope.reset(new BufferWrapper<float>(gpu, table.size()));
        rope->setData(gpu, table);
        pos_buf.reset(new BufferWrapper<int>(gpu, 1));
    }

    // attention.hpp:135-202 (asynchronous apart from the 4-byte position write)
    void forward(BufferWrapper<float>* input, int layer_idx, int pos, float effort,
                 BufferWrapper<uint16_t>* k_cache, BufferWrapper<uint16_t>* v_cache,
                 BufferWrapper<float>* temp_xq, BufferWrapper<float>* temp_xk, BufferWrapper<float>* temp_xv,
                 BufferWrapper<float>* /*temp_xk_repeated*/, BufferWrapper<float>* temp_xq_heads,
                 BufferWrapper<float>* /*temp_xk_heads*/, BufferWrapper<float>* /*temp_scores*/,
                 BufferWrapper<float>* temp_attn_output, BufferWrapper<float>* output)
    {
        if (pos < 0 || pos >= max_tokens_) throw std::runtime_error("Attention: position outside the KV capacity");
        project_qkv(input, effort, temp_xq, temp_xk, temp_xv);
        std::vector<int> p = {pos};
        pos_buf->setData(gpu, p);
        const size_t layer_off = (size_t)layer_idx * max_tokens_ * NUM_KV_HEADS * HEAD_DIM;
        uint16_t* kc = k_cache->data() + layer_off;
        uint16_t* vc = v_cache->data() + layer_off;
        iam_cpp::check(iam_rope_kv_append(gpu->ctx, temp_xq->data(), temp_xk->data(), temp_xv->data(), rope->data(),
                                          pos_buf->data(), NUM_HEADS, NUM_KV_HEADS, HEAD_DIM, max_tokens_,
                                          temp_xq_heads->data(), kc, vc),
                       "Attention rope/append");
        iam_cpp::check(iam_attention_decode(gpu->ctx, temp_xq_heads->data(), kc, vc, pos_buf->data(), NUM_HEADS,
                                            NUM_KV_HEADS, HEAD_DIM, max_tokens_, temp_attn_output->data()),
                       "Attention decode");
        project_o(temp_attn_output, effort, output);
    }

    // attention.hpp:135-202 over the reference's fp32 caches (asynchronous
    // apart from the 4-byte position write)
    void forward(BufferWrapper<float>* input, int layer_idx, int pos, float effort, BufferWrapper<float>* k_cache,
                 BufferWrapper<float>* v_cache, BufferWrapper<float>* temp_xq, BufferWrapper<float>* temp_xk,
                 BufferWrapper<float>* temp_xv, BufferWrapper<float>* /*temp_xk_repeated*/,
                 BufferWrapper<float>* temp_xq_heads, BufferWrapper<float>* /*temp_xk_heads*/,
                 BufferWrapper<float>* /*temp_scores*/, BufferWrapper<float>* temp_attn_output,
                 BufferWrapper<float>* output)
    {
        if (pos < 0 || pos >= max_tokens_) throw std::runtime_error("Attention: position outside the KV capacity");
        const size_t per_layer = (size_t)max_tokens_ * HIDDEN_DIM;
        if (k_cache->count < (size_t)(layer_idx + 1) * per_layer || v_cache->count < (size_t)(layer_idx + 1) * per_layer)
            throw std::runtime_error("Attention: the fp32 caches must hold [layers][max_tokens][32][128] floats");
        project_qkv(input, effort, temp_xq, temp_xk, temp_xv);
        std::vector<int> p = {pos};
        pos_buf->setData(gpu, p);
        float* kc = k_cache->data() + (size_t)layer_idx * per_layer;
        float* vc = v_cache->data() + (size_t)layer_idx * per_layer;
        iam_cpp::check(iam_rope_kv_append_f32(gpu->ctx, temp_xq->data(), temp_xk->data(), temp_xv->data(),
                                              rope->data(), pos_buf->data(), NUM_HEADS, NUM_KV_HEADS, HEAD_DIM,
                                              max_tokens_, temp_xq_heads->data(), kc, vc),
                       "Attention rope/append (fp32 caches)");
        iam_cpp::check(iam_attention_decode_f32(gpu->ctx, temp_xq_heads->data(), kc, vc, pos_buf->data(), NUM_HEADS,
                                                HEAD_DIM, max_tokens_, temp_attn_output->data()),
                       "Attention decode (fp32 caches)");
        project_o(temp_attn_output, effort, output);
    }

    int max_tokens() const { return max_tokens_; }

private:
    // attention.hpp:160-170: q, k and v of the input (one cutoff launch and one walk launch)
    void project_qkv(BufferWrapper<float>* input, float effort, BufferWrapper<float>* xq, BufferWrapper<float>* xk,
                     BufferWrapper<float>* xv)
    {
        iam_bucket_matrix qkv[3] = {wq->desc(), wk->desc(), wv->desc()};
        const float* xs[3] = {input->data(), input->data(), input->data()};
        int ins[3] = {HIDDEN_DIM, HIDDEN_DIM, HIDDEN_DIM};
        float* ys[3] = {xq->data(), xk->data(), xv->data()};
        iam_cpp::check(iam_bucketmul_multi(gpu->ctx, 3, qkv, xs, ins, ys, 0, effort), "Attention q/k/v");
    }

    // attention.hpp:198-200: the o projection
    void project_o(BufferWrapper<float>* attn, float effort, BufferWrapper<float>* output)
    {
        iam_bucket_matrix o[1] = {wo->desc()};
        const float* xo[1] = {attn->data()};
        int ino[1] = {HIDDEN_DIM};
        float* yo[1] = {output->data()};
        iam_cpp::check(iam_bucketmul_multi(gpu->ctx, 1, o, xo, ino, yo, 0, effort), "Attention o");
    }

    Gpu* gpu;
    int max_tokens_;
    std::unique_ptr<BucketWeight> wq, wk, wv, wo;
    std::unique_ptr<BufferWrapper<float>> rope;
    std::unique_ptr<BufferWrapper<int>> pos_buf;
};

#endif
