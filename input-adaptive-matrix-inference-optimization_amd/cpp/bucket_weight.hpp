// bucket_weight.hpp - one weight matrix in the reference's bucket layout,
// uploaded from a BucketizedWeight (the upload the reference constructors do
// by hand, feedforward.hpp:122-165 and attention.hpp:77-98), plus a compact
// device copy of stats channel 3 so the selection reads 2 bytes per row.
#ifndef IAM_BUCKET_WEIGHT_HPP
#define IAM_BUCKET_WEIGHT_HPP

#include <algorithm>
#include <memory>

#include "binary_loader.hpp"
#include "bucket_mul.hpp"

class BucketWeight {
public:
    std::unique_ptr<BufferWrapper<uint16_t>> buckets, stats, stats3, probes;
    int in_dim = 0, out_dim = 0, expert_count = 1, expert_size = 0, bucket_cols = 0;

    BucketWeight(Gpu* gpu, const BucketizedWeight& w)
    {
        const WeightMetadata& m = w.meta;
        in_dim = (int)m.in_dim;
        out_dim = (int)m.out_dim;
        expert_count = (int)m.stats_shape.dim0;
        expert_size = (int)m.stats_shape.dim1;
        bucket_cols = (int)m.buckets_shape.dim2;
        const size_t rows = (size_t)expert_count * expert_size;
        buckets.reset(new BufferWrapper<uint16_t>(gpu, std::vector<size_t>{rows, (size_t)bucket_cols}));
        stats.reset(new BufferWrapper<uint16_t>(gpu, std::vector<size_t>{rows, (size_t)m.stats_shape.dim2}));
        stats3.reset(new BufferWrapper<uint16_t>(gpu, rows));
        // the cutoff reads 4096 probes per expert even when in_dim is smaller
        const size_t np = std::max(w.probes_host.size(), (size_t)expert_count * IAM_PROBES_COUNT);
        probes.reset(new BufferWrapper<uint16_t>(gpu, np));
        buckets->setData(gpu, w.buckets_host);
        stats->setData(gpu, w.stats_host);
        std::vector<uint16_t> p(np, 0);
        std::copy(w.probes_host.begin(), w.probes_host.end(), p.begin());
        probes->setData(gpu, p);
        iam_cpp::check(iam_stats_compact(gpu->ctx, stats->data(), rows, (int)m.stats_shape.dim2, 3, stats3->data()),
                       "stats_compact");
    }

    iam_bucket_matrix desc() const
    {
        return iam_bucket_matrix{buckets->data(), stats3->data(), probes->data(), expert_size, bucket_cols, 1, 0};
    }
};

#endif
