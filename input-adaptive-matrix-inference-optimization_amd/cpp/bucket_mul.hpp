// bucket_mul.hpp - the reference's operator wrapper (bucket_mul.hpp:13-268)
// over the iam C ABI.  BufferWrapper<T>, ScalarFloat, DynaVectorFloat and
// the BucketMul singleton keep their names, members and call sequence
// (calcDispatch, then mul; or fullMul); the dispatch state lives in the
// context, as the singleton's scratch did.
#ifndef IAM_BUCKET_MUL_HPP
#define IAM_BUCKET_MUL_HPP

#include <cassert>
#include <vector>

#include "gpu.hpp"

template <typename T>
class BufferWrapper : public MTLBufferable {
public:
    size_t count;
    size_t rows;
    size_t cols;
    size_t byte_size;
    Gpu* gpu_ref;

    // bucket_mul.hpp:22-24 (the access flags are ignored)
    BufferWrapper(Gpu* gpu, size_t size, cl_mem_flags /*flags*/ = CL_MEM_READ_WRITE)
        : MTLBufferable(gpu->createBuffer(size * sizeof(T)), 0), count(size), rows(size), cols(1),
          byte_size(size * sizeof(T)), gpu_ref(gpu)
    {
    }

    // bucket_mul.hpp:26-32 (rows = shape[0], cols = shape[1])
    BufferWrapper(Gpu* gpu, const std::vector<size_t>& shape, cl_mem_flags /*flags*/ = CL_MEM_READ_WRITE)
        : MTLBufferable(gpu->createBuffer(calculateSize(shape) * sizeof(T)), 0), count(calculateSize(shape)),
          rows(shape.size() > 0 ? shape[0] : 1), cols(shape.size() > 1 ? shape[1] : 1),
          byte_size(calculateSize(shape) * sizeof(T)), gpu_ref(gpu)
    {
    }

    BufferWrapper(const BufferWrapper&) = delete;
    BufferWrapper& operator=(const BufferWrapper&) = delete;

    // the device memory is released (the reference leaks it, bucket_mul.hpp:59)
    ~BufferWrapper() override
    {
        if (buffer) iam_free(gpu_ref->ctx, buffer);
    }

    T* data() const { return static_cast<T*>(ptr()); }

    // bucket_mul.hpp:34-38 (a fill kernel, asynchronous)
    void zero(Gpu* gpu) { gpu->zeroBuffer(buffer, byte_size, offsetBytes); }

    // bucket_mul.hpp:40-45
    T get(Gpu* gpu, size_t index)
    {
        gpu->eval();
        T v;
        gpu->readBuffer(buffer, sizeof(T), &v, offsetBytes + index * sizeof(T));
        return v;
    }

    // bucket_mul.hpp:47-52
    std::vector<T> getData(Gpu* gpu)
    {
        gpu->eval();
        std::vector<T> out(count);
        gpu->readBuffer(buffer, byte_size, out.data(), offsetBytes);
        return out;
    }

    // bucket_mul.hpp:54-57
    void setData(Gpu* gpu, const std::vector<T>& d)
    {
        if (d.size() != count) throw std::runtime_error("setData: size mismatch");
        gpu->writeBuffer(buffer, byte_size, d.data(), offsetBytes);
    }

    static size_t calculateSize(const std::vector<size_t>& shape)
    {
        size_t size = 1;
        for (auto dim : shape) size *= dim;
        return size;
    }
};

// bucket_mul.hpp:69-84
class ScalarFloat : public BufferWrapper<float> {
public:
    ScalarFloat(Gpu* gpu, float value = 0.0f) : BufferWrapper<float>(gpu, 1)
    {
        gpu->writeBuffer(buffer, sizeof(float), &value);
    }
    float getValue(Gpu* gpu) { return get(gpu, 0); }
};

// bucket_mul.hpp:86-97
class DynaVectorFloat : public BufferWrapper<float> {
public:
    BufferWrapper<uint32_t>* size;
    DynaVectorFloat(Gpu* gpu, const std::vector<size_t>& shape) : BufferWrapper<float>(gpu, shape)
    {
        size = new BufferWrapper<uint32_t>(gpu, 1);
        size->zero(gpu);
    }
    ~DynaVectorFloat() override { delete size; }
};

class BucketMul {
public:
    static constexpr int PROBES_COUNT = IAM_PROBES_COUNT;   // bucket_mul.hpp:101
    Gpu* gpu;

    // bucket_mul.hpp:119-122: one per process; the first Gpu wins
    static BucketMul* shared(Gpu* g)
    {
        static BucketMul instance(g);
        return &instance;
    }

    // bucket_mul.hpp:147-191
    void calcDispatch(BufferWrapper<float>* input, BufferWrapper<uint16_t>* stats,
                      BufferWrapper<uint16_t>* probes, int expertNo, int inSize, int bucketCols,
                      int expertSize, float effort)
    {
        iam_cpp::check(iam_bucketmul_calc_dispatch(gpu->ctx, input->data(), stats->data(), probes->data(),
                                                   expertNo, inSize, bucketCols, expertSize, effort),
                       "calcDispatch");
    }

    // bucket_mul.hpp:193-252: output is overwritten with the product
    void mul(BufferWrapper<uint16_t>* buckets, BufferWrapper<float>* output)
    {
        iam_cpp::check(iam_bucketmul_mul(gpu->ctx, buckets->data(), (int)buckets->cols, output->data()), "mul");
    }

    // bucket_mul.hpp:254-267
    void fullMul(BufferWrapper<float>* input, BufferWrapper<uint16_t>* stats, BufferWrapper<uint16_t>* probes,
                 BufferWrapper<uint16_t>* buckets, int expertNo, int inSize, int bucketCols, int expertSize,
                 float effort, BufferWrapper<float>* output)
    {
        iam_cpp::check(iam_bucketmul_full(gpu->ctx, input->data(), stats->data(), probes->data(), buckets->data(),
                                          expertNo, inSize, bucketCols, expertSize, effort, output->data()),
                       "fullMul");
    }

    // parity outputs of the last calcDispatch: cutoff and selected rows
    float lastCutoff(uint32_t* count = nullptr)
    {
        float c = 0;
        iam_cpp::check(iam_bucketmul_dispatch_info(gpu->ctx, 0, &c, count), "dispatch_info");
        return c;
    }

private:
    explicit BucketMul(Gpu* g) : gpu(g) {}
};

#endif
