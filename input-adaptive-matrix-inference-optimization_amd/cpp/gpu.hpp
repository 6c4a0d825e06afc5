// gpu.hpp - the reference's device runtime class (gpu.hpp:21-588) over the
// iam C ABI: one HIP device, one in-order stream, per-kernel timing.
//
// Same class and method names as the reference; OpenCL handles are replaced
// by plain device pointers (MTLBufferable::buffer is a void*).  Errors are
// thrown as std::runtime_error, as in Gpu::checkError (gpu.hpp:581-587).
#ifndef IAM_GPU_HPP
#define IAM_GPU_HPP

#include <cstdint>
#include <cstdio>
#include <iostream>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/iam.h"

// Memory access flags the reference's call sites pass when they create
// buffers (the OpenCL specification's values).  HIP device memory takes no
// access flags: they are accepted and ignored.
#ifndef CL_MEM_READ_WRITE
typedef uint64_t cl_mem_flags;
#define CL_MEM_READ_WRITE ((cl_mem_flags)1 << 0)
#define CL_MEM_WRITE_ONLY ((cl_mem_flags)1 << 1)
#define CL_MEM_READ_ONLY ((cl_mem_flags)1 << 2)
#define CL_MEM_COPY_HOST_PTR ((cl_mem_flags)1 << 5)
#endif

namespace iam_cpp {

inline void check(int rc, const char* what)
{
    if (rc != IAM_OK)
        throw std::runtime_error(std::string(what) + " failed, iam code " + std::to_string(rc) + ": " +
                                 iam_last_error());
}

}  // namespace iam_cpp

// gpu.hpp:62-71: a device buffer plus a byte offset
class MTLBufferable {
public:
    void* buffer;
    size_t offsetBytes;
    MTLBufferable(void* buf, size_t offset = 0) : buffer(buf), offsetBytes(offset) {}
    virtual ~MTLBufferable() = default;
    void* ptr() const { return static_cast<char*>(buffer) + offsetBytes; }
};

class Gpu {
public:
    iam_ctx* ctx = nullptr;
    bool warnOfEvals = false;
    int evalCount = 0;
    int blockingWriteCount = 0;
    int blockingReadCount = 0;
    bool enableKernelProfiling = false;

    // Gpu::Gpu (gpu.hpp:109-159): picks a device and creates the queue
    explicit Gpu(int device = 0)
    {
        iam_cpp::check(iam_ctx_create(device, &ctx), "context creation");
        char name[256];
        int cus = 0;
        size_t mem = 0;
        iam_cpp::check(iam_device_info(ctx, name, sizeof(name), &cus, &mem), "device query");
        deviceName = name;
        computeUnits = cus;
        globalMem = mem;
    }

    ~Gpu()
    {
        if (enableKernelProfiling) printKernelStats();
        iam_ctx_destroy(ctx);
    }

    Gpu(const Gpu&) = delete;
    Gpu& operator=(const Gpu&) = delete;

    // gpu.hpp:236-248 (the access flags are ignored)
    void* createBuffer(size_t size, cl_mem_flags /*flags*/ = CL_MEM_READ_WRITE)
    {
        void* p = nullptr;
        iam_cpp::check(iam_alloc(ctx, size, &p), "device allocation");
        return p;
    }

    // gpu.hpp:250-262: a buffer initialised from host memory
    void* createBuffer(size_t size, const void* data, cl_mem_flags /*flags*/ = CL_MEM_READ_WRITE)
    {
        void* p = createBuffer(size);
        if (data) iam_cpp::check(iam_write(ctx, p, 0, data, size), "host-to-device write");
        return p;
    }

    // gpu.hpp:264-269
    void releaseBuffer(void* buffer)
    {
        if (buffer) iam_cpp::check(iam_free(ctx, buffer), "device free");
    }

    // gpu.hpp:399-447: wait for the queue; kernel timings are folded in
    void eval(bool noWarn = false)
    {
        evalCount++;
        if (warnOfEvals && !noWarn) std::cout << "note: synchronizing evaluation " << evalCount << std::endl;
        iam_cpp::check(iam_sync(ctx), "stream synchronization");
    }

    // gpu.hpp:449-455
    void copyBuffer(MTLBufferable* src, MTLBufferable* dst, size_t size)
    {
        iam_cpp::check(iam_copy(ctx, dst->buffer, dst->offsetBytes, src->buffer, src->offsetBytes, size),
                       "device copy");
    }

    // gpu.hpp:457-462 (blocking)
    void readBuffer(const void* buffer, size_t size, void* hostPtr, size_t offset = 0)
    {
        blockingReadCount++;
        iam_cpp::check(iam_read(ctx, hostPtr, buffer, offset, size), "device-to-host read");
    }

    // gpu.hpp:464-469 (blocking)
    void writeBuffer(void* buffer, size_t size, const void* hostPtr, size_t offset = 0)
    {
        blockingWriteCount++;
        iam_cpp::check(iam_write(ctx, buffer, offset, hostPtr, size), "host-to-device write");
    }

    void zeroBuffer(void* buffer, size_t size, size_t offset = 0)
    {
        iam_cpp::check(iam_zero(ctx, buffer, offset, size), "device clear");
    }

    void setProfiling(bool on)
    {
        enableKernelProfiling = on;
        iam_cpp::check(iam_profiling(ctx, on ? 1 : 0), "profiling switch");
    }

    // gpu.hpp:190-234
    void printKernelStats()
    {
        std::vector<char> buf(1 << 16);
        if (iam_kernel_stats(ctx, buf.data(), buf.size()) == IAM_OK) {
            std::cout << "\n-- kernel times (HIP events per launch) --\n" << buf.data()
                      << "-- end of kernel times --\n";
        }
    }

    // MemoryTracker::print_status (gpu.hpp:52-56)
    void printMemoryStatus()
    {
        size_t used = 0, usable = 0;
        iam_mem_status(ctx, &used, &usable);
        std::printf("VRAM: %.2f / %.2f GB (%d%%)\n", used / 1073741824.0, usable / 1073741824.0,
                    usable ? (int)(used * 100.0 / usable) : 0);
    }

    std::string deviceName;
    int computeUnits = 0;
    size_t globalMem = 0;
};

#endif
