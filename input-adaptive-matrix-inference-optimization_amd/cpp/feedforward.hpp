// feedforward.hpp - FeedForward of the reference (feedforward.hpp:14-183)
// over the iam C ABI: gate and up as one cutoff launch and one walk launch,
// silu32 (matrix.cl:27-32), then down.  Same constructor and forward().
#ifndef IAM_FEEDFORWARD_HPP
#define IAM_FEEDFORWARD_HPP

#include <memory>
#include <string>

#include "bucket_weight.hpp"

class FeedForward {
public:
    // feedforward.hpp:89-170
    FeedForward(Gpu* g, const std::string& weights_dir, int layer_idx, size_t hidden = 4096, size_t ffn = 14336)
        : gpu(g), hidden_dim(hidden), ffn_dim(ffn), layer_idx_(layer_idx)
    {
        BinaryWeightLoader loader(gpu, weights_dir);
        const std::string prefix = "layer" + std::to_string(layer_idx);
        gate.reset(new BucketWeight(gpu, loader.load(prefix + "_gate_proj_bucketmul_fp16")));
        up.reset(new BucketWeight(gpu, loader.load(prefix + "_up_proj_bucketmul_fp16")));
        down.reset(new BucketWeight(gpu, loader.load(prefix + "_down_proj_bucketmul_fp16")));
        if (gate->in_dim) hidden_dim = gate->in_dim;
        if (gate->out_dim) ffn_dim = gate->out_dim;
        if (up->in_dim != (int)hidden_dim || up->out_dim != (int)ffn_dim || down->in_dim != (int)ffn_dim ||
            down->out_dim != (int)hidden_dim)
            throw std::runtime_error("FeedForward: gate/up/down shapes do not chain");
        gate_output.reset(new BufferWrapper<float>(gpu, ffn_dim));
        up_output.reset(new BufferWrapper<float>(gpu, ffn_dim));
        silu_output.reset(new BufferWrapper<float>(gpu, ffn_dim));
    }

    // feedforward.hpp:46-86, 180-182 (asynchronous; output overwritten)
    void forward(BufferWrapper<float>* input, BufferWrapper<float>* output, float effort = 1.0f)
    {
        iam_bucket_matrix gu[2] = {gate->desc(), up->desc()};
        const float* xs[2] = {input->data(), input->data()};
        int ins[2] = {(int)hidden_dim, (int)hidden_dim};
        float* ys[2] = {gate_output->data(), up_output->data()};
        iam_cpp::check(iam_bucketmul_multi(gpu->ctx, 2, gu, xs, ins, ys, 0, effort), "FeedForward gate/up");
        iam_cpp::check(iam_silu_mul(gpu->ctx, gate_output->data(), up_output->data(), (int)ffn_dim,
                                    silu_output->data()),
                       "FeedForward silu");
        iam_bucket_matrix dn[1] = {down->desc()};
        const float* xd[1] = {silu_output->data()};
        int ind[1] = {(int)ffn_dim};
        float* yd[1] = {output->data()};
        iam_cpp::check(iam_bucketmul_multi(gpu->ctx, 1, dn, xd, ind, yd, 0, effort), "FeedForward down");
    }

    size_t hidden() const { return hidden_dim; }
    size_t ffn() const { return ffn_dim; }

private:
    Gpu* gpu;
    std::unique_ptr<BucketWeight> gate, up, down;
    std::unique_ptr<BufferWrapper<float>> gate_output, up_output, silu_output;
    size_t hidden_dim, ffn_dim;
    int layer_idx_;
};

#endif
