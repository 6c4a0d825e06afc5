// Context, memory, errors and per-kernel profiling: the HIP replacement of
// the reference's OpenCL runtime class (gpu.hpp:21-588).
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <sstream>
#include <iomanip>

#include "internal.h"

namespace iam {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg)
{
    set_error(msg);
    return code;
}

int ctx_alloc(Ctx* c, size_t bytes, void** out)
{
    if (!out) return fail(IAM_E_INVALID, "alloc: null output pointer");
    *out = nullptr;
    if (bytes == 0) bytes = 1;
    // MemoryTracker::can_allocate (gpu.hpp:40-44)
    if (c->allocated + bytes > c->usable)
        return fail(IAM_E_NOMEM, "alloc: over the context's device memory budget (budget " +
                                     std::to_string(c->usable) + " bytes, in use " +
                                     std::to_string(c->allocated) + ", asked " +
                                     std::to_string(bytes) + ")");
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(IAM_E_NOMEM, std::string("hipMalloc: ") + hipGetErrorString(e));
    }
    c->allocs[(uintptr_t)p] = bytes;
    c->allocated += bytes;
    *out = p;
    return IAM_OK;
}

int ctx_free(Ctx* c, void* p)
{
    if (!p) return IAM_OK;
    auto it = c->allocs.find((uintptr_t)p);
    if (it == c->allocs.end()) return fail(IAM_E_INVALID, "free: pointer not allocated by this context");
    IAM_CHECK_HIP(hipFree(p));
    c->allocated -= it->second;
    c->allocs.erase(it);
    return IAM_OK;
}

int check_dev_range(Ctx* c, const void* p, size_t bytes, const char* what)
{
    // interior pointers of tracked allocations are accepted
    uintptr_t a = (uintptr_t)p;
    auto it = c->allocs.upper_bound(a);
    if (it != c->allocs.begin()) {
        --it;
        if (a >= it->first && a + bytes <= it->first + it->second) return IAM_OK;
    }
    return fail(IAM_E_INVALID, std::string(what) + ": range not inside an allocation of this context");
}

int ensure_slot(Ctx* c, int slot)
{
    DispatchSlot& s = c->slots[slot];
    if (!s.cutoff) {
        if (c->capturing) return fail(IAM_E_STATE, "dispatch buffer allocation during graph capture");
        IAM_TRY(ctx_alloc(c, 16, (void**)&s.cutoff));
        IAM_TRY(zero_async(c, s.cutoff, 16));   // hint 0: none
        c->scratch_gen++;
    }
    return IAM_OK;
}

int ensure_list(Ctx* c, int slot, int chunks)
{
    DispatchSlot& s = c->slots[slot];
    if (!s.counts) IAM_TRY(ctx_alloc(c, sizeof(uint32_t) * kMaxChunks, (void**)&s.counts));
    if ((size_t)chunks > s.cap_chunks) {
        if (s.list) IAM_TRY(ctx_free(c, s.list));
        s.list = nullptr;
        IAM_TRY(ctx_alloc(c, sizeof(uint2) * (size_t)chunks * kChunkRows, (void**)&s.list));
        s.cap_chunks = (size_t)chunks;
    }
    return IAM_OK;
}

// Grow a zero-initialised scratch buffer of `count` elements of `elem` bytes.
static int grow_zeroed(Ctx* c, void** p, size_t* cap, size_t count, size_t elem, const char* what)
{
    if (count <= *cap && *p) return IAM_OK;
    if (c->capturing) return fail(IAM_E_STATE, std::string(what) + " growth during graph capture");
    if (*p) IAM_TRY(ctx_free(c, *p));
    *p = nullptr;
    *cap = 0;
    const size_t n = std::max<size_t>(count, 1);
    IAM_TRY(ctx_alloc(c, n * elem, p));
    IAM_TRY(zero_async(c, *p, n * elem));
    *cap = n;
    c->scratch_gen++;
    return IAM_OK;
}

int ensure_walk_scratch(Ctx* c, int slot, size_t m, size_t T, size_t P)
{
    DispatchSlot& s = c->slots[slot];
    IAM_TRY(grow_zeroed(c, &s.acc, &s.acc_cap, m, 8, "walk accumulator"));
    IAM_TRY(grow_zeroed(c, (void**)&s.tile_ctr, &s.tile_cap, T, sizeof(uint32_t), "walk tile counter"));
    IAM_TRY(grow_zeroed(c, (void**)&s.slice_count, &s.slice_cap, P, sizeof(uint32_t), "walk slice count"));
    return IAM_OK;
}

int ensure_attn_scratch(Ctx* c, size_t acc_words, int n_heads)
{
    IAM_TRY(grow_zeroed(c, &c->attn_acc, &c->attn_acc_cap, acc_words, 8, "attention accumulator"));
    constexpr size_t kCounters = 512;   // one per query head
    size_t cap = c->attn_ctr ? kCounters : 0;
    IAM_REQUIRE(n_heads <= (int)kCounters, "attention: at most 512 query heads");
    return grow_zeroed(c, (void**)&c->attn_ctr, &cap, kCounters, sizeof(uint32_t), "attention counter");
}

int begin_launch(Ctx* c, const char* name, PendingEvent* ev)
{
    for (int i = 0; i < 2; i++) {
        hipEvent_t e;
        if (!c->event_pool.empty()) {
            e = c->event_pool.back();
            c->event_pool.pop_back();
        } else {
            IAM_CHECK_HIP(hipEventCreate(&e));
        }
        (i == 0 ? ev->start : ev->stop) = e;
    }
    ev->name = name;
    return IAM_OK;
}

int end_launch(Ctx* c, PendingEvent* ev, bool have_ev)
{
    if (!have_ev) return IAM_OK;
    c->pending.push_back(*ev);
    return IAM_OK;
}

// fill kernel used instead of hipMemsetAsync so that zeroing is safe inside
// captured graphs
__global__ void k_zero(uint32_t* p, size_t n_words)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < n_words; i += stride) p[i] = 0u;
}

__global__ void k_zero_bytes(uint8_t* p, size_t n)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

int zero_async(Ctx* c, void* p, size_t bytes)
{
    if (bytes == 0) return IAM_OK;
    uintptr_t a = (uintptr_t)p;
    if ((a & 3) == 0 && (bytes & 3) == 0) {
        size_t words = bytes / 4;
        size_t blocks = std::min<size_t>((words + 255) / 256, 4096);
        return launch(c, "zero32", k_zero, dim3((unsigned)blocks), dim3(256), 0, (uint32_t*)p, words);
    }
    return launch(c, "zero8", k_zero_bytes, dim3((unsigned)((bytes + 255) / 256)), dim3(256), 0,
                  (uint8_t*)p, bytes);
}

static int fold_events(Ctx* c)
{
    for (auto& ev : c->pending) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, ev.start, ev.stop) == hipSuccess) {
            KernelStat& s = c->stats[ev.name];
            s.calls++;
            s.total_ms += ms;
            if (ms > s.max_ms) s.max_ms = ms;
        }
        c->event_pool.push_back(ev.start);
        c->event_pool.push_back(ev.stop);
    }
    c->pending.clear();
    return IAM_OK;
}

}  // namespace iam

using namespace iam;

extern "C" {

const char* iam_last_error(void) { return g_last_error.c_str(); }

int iam_ctx_create(int device, iam_ctx** out)
{
    if (!out) return fail(IAM_E_INVALID, "ctx_create: null output");
    *out = nullptr;
    int n = 0;
    IAM_CHECK_HIP(hipGetDeviceCount(&n));
    if (device < 0 || device >= n)
        return fail(IAM_E_INVALID, "ctx_create: device " + std::to_string(device) + " of " +
                                       std::to_string(n));
    IAM_CHECK_HIP(hipSetDevice(device));
    iam_ctx* c = new iam_ctx();
    c->device = device;
    // default priority stream
    hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete c;
        return fail(IAM_E_HIP, std::string("hipStreamCreate: ") + hipGetErrorString(e));
    }
    size_t free_b = 0, total_b = 0;
    IAM_CHECK_HIP(hipMemGetInfo(&free_b, &total_b));
    c->total_mem = total_b;
    const size_t margin = 512ull << 20;   // gpu.hpp:28 safety margin
    c->usable = total_b > margin ? total_b - margin : total_b;
    const size_t cbytes = kCounterWords * sizeof(unsigned long long);
    int rc = ctx_alloc(c, cbytes, (void**)&c->counters);
    if (rc == IAM_OK) rc = zero_async(c, c->counters, cbytes);
    if (rc == IAM_OK && hipStreamSynchronize(c->stream) != hipSuccess) rc = fail(IAM_E_HIP, "ctx_create: sync");
    if (rc != IAM_OK) {
        std::string err = g_last_error;
        iam_ctx_destroy(c);
        return fail(rc, err);
    }
    *out = c;
    return IAM_OK;
}

int iam_ctx_destroy(iam_ctx* c)
{
    if (!c) return IAM_OK;
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    for (auto& kv : c->allocs) (void)hipFree((void*)kv.first);
    c->allocs.clear();
    for (auto& ev : c->pending) {
        (void)hipEventDestroy(ev.start);
        (void)hipEventDestroy(ev.stop);
    }
    for (auto e : c->event_pool) (void)hipEventDestroy(e);
    (void)hipStreamDestroy(c->stream);
    delete c;
    return IAM_OK;
}

int iam_sync(iam_ctx* c)
{
    if (!c) return fail(IAM_E_INVALID, "sync: null context");
    IAM_CHECK_HIP(hipStreamSynchronize(c->stream));
    return fold_events(c);
}

int iam_device_info(iam_ctx* c, char* name, size_t name_len, int* cus, size_t* mem)
{
    if (!c) return fail(IAM_E_INVALID, "device_info: null context");
    hipDeviceProp_t p;
    IAM_CHECK_HIP(hipGetDeviceProperties(&p, c->device));
    if (name && name_len) {
        std::snprintf(name, name_len, "%s (%s)", p.name, p.gcnArchName);
    }
    if (cus) *cus = p.multiProcessorCount;
    if (mem) *mem = p.totalGlobalMem;
    return IAM_OK;
}

int iam_mem_status(iam_ctx* c, size_t* allocated, size_t* usable)
{
    if (!c) return fail(IAM_E_INVALID, "mem_status: null context");
    if (allocated) *allocated = c->allocated;
    if (usable) *usable = c->usable;
    return IAM_OK;
}

int iam_alloc(iam_ctx* c, size_t bytes, void** out)
{
    if (!c) return fail(IAM_E_INVALID, "alloc: null context");
    return ctx_alloc(c, bytes, out);
}

int iam_free(iam_ctx* c, void* p)
{
    if (!c) return fail(IAM_E_INVALID, "free: null context");
    IAM_CHECK_HIP(hipStreamSynchronize(c->stream));
    return ctx_free(c, p);
}

static int check_range(Ctx* c, const void* p, size_t off, size_t bytes, const char* what)
{
    return check_dev_range(c, (const uint8_t*)p + off, bytes, what);
}

int iam_zero(iam_ctx* c, void* p, size_t off, size_t bytes)
{
    if (!c || !p) return fail(IAM_E_INVALID, "zero: null argument");
    IAM_TRY(check_range(c, p, off, bytes, "zero"));
    return zero_async(c, (uint8_t*)p + off, bytes);
}

int iam_write(iam_ctx* c, void* dst, size_t off, const void* src, size_t bytes)
{
    if (!c || !dst || (!src && bytes)) return fail(IAM_E_INVALID, "write: null argument");
    IAM_TRY(check_range(c, dst, off, bytes, "write"));
    IAM_CHECK_HIP(hipMemcpyAsync((uint8_t*)dst + off, src, bytes, hipMemcpyHostToDevice, c->stream));
    IAM_CHECK_HIP(hipStreamSynchronize(c->stream));
    return IAM_OK;
}

int iam_read(iam_ctx* c, void* dst, const void* src, size_t off, size_t bytes)
{
    if (!c || !src || (!dst && bytes)) return fail(IAM_E_INVALID, "read: null argument");
    IAM_TRY(check_range(c, src, off, bytes, "read"));
    IAM_CHECK_HIP(hipMemcpyAsync(dst, (const uint8_t*)src + off, bytes, hipMemcpyDeviceToHost, c->stream));
    IAM_CHECK_HIP(hipStreamSynchronize(c->stream));
    return IAM_OK;
}

int iam_copy(iam_ctx* c, void* dst, size_t doff, const void* src, size_t soff, size_t bytes)
{
    if (!c || !dst || !src) return fail(IAM_E_INVALID, "copy: null argument");
    IAM_TRY(check_range(c, dst, doff, bytes, "copy dst"));
    IAM_TRY(check_range(c, src, soff, bytes, "copy src"));
    IAM_CHECK_HIP(hipMemcpyAsync((uint8_t*)dst + doff, (const uint8_t*)src + soff, bytes,
                                 hipMemcpyDeviceToDevice, c->stream));
    return IAM_OK;
}

// Streaming read of n16 16-byte words: block b reads the b-th contiguous
// chunk, 8 loads in flight per thread (of the shapes measured, the fastest:
// 6.4-6.5 TB/s against 5.5 for a grid-stride loop with 4 loads 8 MB apart).
// The xor of the words is stored only if it equals a value that a
// zero-filled buffer cannot give, so the loads are kept and nothing is
// written.
__global__ __launch_bounds__(256) void k_read_stream(const uint4* __restrict__ p, size_t n16,
                                                    uint32_t* __restrict__ sink)
{
    constexpr int U = 8;
    const size_t chunk = (n16 + gridDim.x - 1) / gridDim.x;
    const size_t b0 = (size_t)blockIdx.x * chunk;
    const size_t b1 = b0 + chunk < n16 ? b0 + chunk : n16;
    uint32_t acc = 0;
    size_t i = b0 + threadIdx.x;
    for (; i + (U - 1) * 256 < b1; i += U * 256) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = p[i + u * 256];
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < b1; i += 256) {
        const uint4 a = p[i];
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    if (acc == 0x9e3779b9u) sink[blockIdx.x] = acc;
}

int iam_read_bandwidth(iam_ctx* c, size_t bytes, int reps, double* gb_per_s)
{
    if (!c || !gb_per_s) return fail(IAM_E_INVALID, "read_bandwidth: null argument");
    IAM_REQUIRE(bytes >= (1u << 20) && bytes % 16 == 0, "read_bandwidth: bytes must be >= 1 MiB and a multiple of 16");
    IAM_REQUIRE(reps >= 1 && reps <= 1000, "read_bandwidth: reps must be in [1, 1000]");
    IAM_REQUIRE(!c->capturing, "read_bandwidth: not allowed during graph capture");
    constexpr unsigned kBlocks = 8192;
    void* buf = nullptr;
    void* sink = nullptr;
    IAM_TRY(ctx_alloc(c, bytes, &buf));
    int rc = ctx_alloc(c, kBlocks * sizeof(uint32_t), &sink);
    if (rc == IAM_OK) rc = zero_async(c, buf, bytes);
    hipEvent_t e0 = nullptr, e1 = nullptr;
    float ms = 0.0f;
    if (rc == IAM_OK && (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess))
        rc = fail(IAM_E_HIP, "read_bandwidth: event creation failed");
    const size_t n16 = bytes / 16;
    // one untimed pass, then reps timed back to back
    if (rc == IAM_OK) {
        hipLaunchKernelGGL(k_read_stream, dim3(kBlocks), dim3(256), 0, c->stream, (const uint4*)buf, n16,
                           (uint32_t*)sink);
        (void)hipEventRecord(e0, c->stream);
        for (int r = 0; r < reps; r++)
            hipLaunchKernelGGL(k_read_stream, dim3(kBlocks), dim3(256), 0, c->stream, (const uint4*)buf, n16,
                               (uint32_t*)sink);
        (void)hipEventRecord(e1, c->stream);
        hipError_t e = hipEventSynchronize(e1);
        if (e == hipSuccess) e = hipGetLastError();
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
        if (e != hipSuccess) rc = fail(IAM_E_HIP, std::string("read_bandwidth: ") + hipGetErrorString(e));
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (sink) (void)ctx_free(c, sink);
    (void)ctx_free(c, buf);
    if (rc != IAM_OK) return rc;
    *gb_per_s = ms > 0.0f ? (double)bytes * reps / (ms * 1e-3) / 1e9 : 0.0;
    return IAM_OK;
}

int iam_profiling(iam_ctx* c, int enable)
{
    if (!c) return fail(IAM_E_INVALID, "profiling: null context");
    c->profiling = enable != 0;
    return IAM_OK;
}

int iam_kernel_stats(iam_ctx* c, char* buf, size_t len)
{
    if (!c || !buf || !len) return fail(IAM_E_INVALID, "kernel_stats: bad argument");
    std::vector<std::pair<std::string, KernelStat>> v(c->stats.begin(), c->stats.end());
    std::sort(v.begin(), v.end(),
              [](const auto& a, const auto& b) { return a.second.total_ms > b.second.total_ms; });
    double total = 0;
    for (auto& kv : v) total += kv.second.total_ms;
    std::ostringstream os;
    os << std::setw(28) << "Kernel" << std::setw(10) << "Calls" << std::setw(14) << "Total (ms)"
       << std::setw(14) << "Avg (ms)" << std::setw(12) << "Max (ms)" << std::setw(12)
       << "% of Total" << "\n";
    for (auto& kv : v) {
        const KernelStat& s = kv.second;
        os << std::setw(28) << kv.first << std::setw(10) << s.calls << std::setw(14)
           << std::fixed << std::setprecision(3) << s.total_ms << std::setw(14)
           << std::setprecision(5) << (s.calls ? s.total_ms / s.calls : 0.0) << std::setw(12)
           << s.max_ms << std::setw(11) << std::setprecision(1)
           << (total > 0 ? 100.0 * s.total_ms / total : 0.0) << "%\n";
    }
    os << std::setw(28) << "TOTAL" << std::setw(10) << "" << std::setw(14) << std::setprecision(3)
       << total << "\n";
    std::string s = os.str();
    std::snprintf(buf, len, "%s", s.c_str());
    return IAM_OK;
}

// sums of the counter rows of labels [g0, g1)
static int read_counters(Ctx* c, int g0, int g1, uint64_t* bytes, uint64_t* rows, uint64_t* mats, int reset)
{
    std::vector<unsigned long long> h(kCounterWords);
    IAM_CHECK_HIP(hipMemcpyAsync(h.data(), c->counters, kCounterWords * sizeof(unsigned long long),
                                 hipMemcpyDeviceToHost, c->stream));
    IAM_CHECK_HIP(hipStreamSynchronize(c->stream));
    unsigned long long t[3] = {0, 0, 0};
    for (int l = g0 * kCounterLanes; l < g1 * kCounterLanes; l++)
        for (int i = 0; i < 3; i++) t[i] += h[(size_t)l * 4 + i];
    if (bytes) *bytes = t[0];
    if (rows) *rows = t[1];
    if (mats) *mats = t[2];
    if (reset) {
        IAM_TRY(zero_async(c, c->counters, kCounterWords * sizeof(unsigned long long)));
        IAM_CHECK_HIP(hipStreamSynchronize(c->stream));
    }
    return IAM_OK;
}

int iam_walk_group_hints(iam_ctx* c, int group, uint64_t* tries, uint64_t* hits)
{
    if (!c) return fail(IAM_E_INVALID, "walk_group_hints: null context");
    if (group < 0 || group >= kWalkLabels)
        return fail(IAM_E_INVALID, "walk_group_hints: group must be one of IAM_WALK_GROUP_*");
    std::vector<unsigned long long> h(kCounterWords);
    IAM_CHECK_HIP(hipMemcpyAsync(h.data(), c->counters, kCounterWords * sizeof(unsigned long long),
                                 hipMemcpyDeviceToHost, c->stream));
    IAM_CHECK_HIP(hipStreamSynchronize(c->stream));
    unsigned long long t = 0, k = 0;
    for (int l = group * kCounterLanes; l < (group + 1) * kCounterLanes; l++) {
        t += h[(size_t)l * 4 + 3] >> 32;
        k += h[(size_t)l * 4 + 3] & 0xffffffffull;
    }
    if (tries) *tries = t;
    if (hits) *hits = k;
    return IAM_OK;
}

int iam_walk_counters(iam_ctx* c, uint64_t* bytes, uint64_t* rows, uint64_t* mats, int reset)
{
    if (!c) return fail(IAM_E_INVALID, "walk_counters: null context");
    return read_counters(c, 0, kWalkLabels, bytes, rows, mats, reset);
}

int iam_walk_group_counters(iam_ctx* c, int group, uint64_t* bytes, uint64_t* rows, uint64_t* mats)
{
    if (!c) return fail(IAM_E_INVALID, "walk_group_counters: null context");
    if (group < 0 || group >= kWalkLabels)
        return fail(IAM_E_INVALID, "walk_group_counters: group must be one of IAM_WALK_GROUP_*");
    return read_counters(c, group, group + 1, bytes, rows, mats, 0);
}

int iam_kernel_stats_reset(iam_ctx* c)
{
    if (!c) return fail(IAM_E_INVALID, "kernel_stats_reset: null context");
    c->stats.clear();
    return IAM_OK;
}

int iam_set_accumulation(iam_ctx* c, int mode)
{
    if (!c) return fail(IAM_E_INVALID, "set_accumulation: null context");
    IAM_REQUIRE(mode == IAM_ACC_FP32 || mode == IAM_ACC_FP64, "set_accumulation: mode must be IAM_ACC_FP32 or IAM_ACC_FP64");
    IAM_REQUIRE(!c->capturing, "set_accumulation: not allowed during graph capture");
    const bool f64 = mode == IAM_ACC_FP64;
    if (f64 != c->acc64) {
        c->acc64 = f64;
        c->scratch_gen++;   // captured graphs hold kernels of the other mode
    }
    return IAM_OK;
}

int iam_set_search_hints(iam_ctx* c, int on)
{
    if (!c) return fail(IAM_E_INVALID, "set_search_hints: null context");
    IAM_REQUIRE(!c->capturing, "set_search_hints: not allowed during graph capture");
    if ((on != 0) != c->hints) {
        c->hints = on != 0;
        c->scratch_gen++;   // captured graphs hold walk launches of the other setting
    }
    return IAM_OK;
}

int iam_set_search_hint(iam_ctx* c, int slot, float value)
{
    if (!c) return fail(IAM_E_INVALID, "set_search_hint: null context");
    IAM_REQUIRE(slot >= 0 && slot < kMaxMulti, "set_search_hint: slot must be 0, 1 or 2");
    IAM_REQUIRE(!c->capturing, "set_search_hint: not allowed during graph capture");
    IAM_TRY(ensure_slot(c, slot));
    IAM_CHECK_HIP(hipMemcpyAsync(c->slots[slot].cutoff + 2, &value, sizeof(float), hipMemcpyHostToDevice, c->stream));
    IAM_CHECK_HIP(hipStreamSynchronize(c->stream));
    return IAM_OK;
}

int iam_set_walk_counting(iam_ctx* c, int on)
{
    if (!c) return fail(IAM_E_INVALID, "set_walk_counting: null context");
    IAM_REQUIRE(!c->capturing, "set_walk_counting: not allowed during graph capture");
    if ((on != 0) != c->counting) {
        c->counting = on != 0;
        c->scratch_gen++;   // captured graphs hold walk launches of the other setting
    }
    return IAM_OK;
}

int iam_set_selection_block(iam_ctx* c, int block_inputs, float below_effort)
{
    if (!c) return fail(IAM_E_INVALID, "set_selection_block: null context");
    IAM_REQUIRE(!c->capturing, "set_selection_block: not allowed during graph capture");
    IAM_REQUIRE(block_inputs == 1 || block_inputs == 2 || block_inputs == 4 || block_inputs == 8 ||
                    block_inputs == 16,
                "set_selection_block: block_inputs must be 1, 2, 4, 8 or 16");
    IAM_REQUIRE(below_effort > 0.0f, "set_selection_block: below_effort must be positive");
    if (block_inputs != c->sel_block || below_effort != c->sel_below) {
        c->sel_block = block_inputs;
        c->sel_below = below_effort;
        c->scratch_gen++;   // captured graphs hold walk launches of the other setting
    }
    return IAM_OK;
}

int iam_get_selection_block(iam_ctx* c, int* block_inputs, float* below_effort)
{
    if (!c || !block_inputs || !below_effort) return fail(IAM_E_INVALID, "get_selection_block: bad argument");
    *block_inputs = c->sel_block;
    *below_effort = c->sel_below;
    return IAM_OK;
}

int iam_get_accumulation(iam_ctx* c, int* mode)
{
    if (!c || !mode) return fail(IAM_E_INVALID, "get_accumulation: bad argument");
    *mode = c->acc64 ? IAM_ACC_FP64 : IAM_ACC_FP32;
    return IAM_OK;
}

int iam_kernel_stat(iam_ctx* c, const char* name, double* total_ms, int* calls)
{
    if (!c || !name) return fail(IAM_E_INVALID, "kernel_stat: bad argument");
    // "bucket_walk" also sums the labelled launches "bucket_walk.<group>";
    // "*" sums every kernel
    const std::string key(name), sub = key + ".";
    const bool all = key == "*";
    double t = 0.0;
    int n = 0;
    for (const auto& kv : c->stats)
        if (all || kv.first == key || (key.find('.') == std::string::npos && kv.first.rfind(sub, 0) == 0)) {
            t += kv.second.total_ms;
            n += kv.second.calls;
        }
    if (total_ms) *total_ms = t;
    if (calls) *calls = n;
    return IAM_OK;
}

}  // extern "C"
