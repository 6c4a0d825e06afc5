// The bucketMul matrix group without any allocation at call time.
//
// iam_bucketmul_fused keeps its scratch (walk accumulators, tile arrival
// counters, per-slice row counts, the cutoffs) in buffers the context grows
// on demand, which can mean a device allocation on a call.  This variant runs
// the same walk kernel with that scratch in one file-scope device array,
// `scratch`, of a fixed size: callers that must not allocate (code under HIP
// graph capture, serving loops, harnesses that forbid hipMalloc) pass only
// their inputs and outputs.
//
// Each device holds its own copy of the array, from the first call on that
// device until the process ends; its address is looked up once per device
// (hipGetSymbolAddress with the device current) and only that address is
// passed to kernels.  Every call on a device uses the same array, so calls
// that overlap on one device -- from two streams, contexts or threads --
// race and give wrong results.  Each call clears what the walk needs zero
// (the accumulators and tile counters it uses) with a fill kernel, so a call
// never depends on what an earlier one left.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <string>

#include "internal.h"

namespace iam {
namespace {

// limits of one call (the group's matrices together)
constexpr size_t kNaOutputs = IAM_NOALLOC_MAX_OUTPUTS;   // outputs (16 * bucket_cols summed)
constexpr int kNaTiles = 256;                              // column tiles per matrix
constexpr int kNaSlices = 1024;                            // input slices per matrix

// layout of the array in 8-byte words: accumulators, then per matrix the
// tile counters, slice counts and the cutoff (each 256-byte aligned)
constexpr size_t kAccWords = kNaOutputs;
constexpr size_t kTileWords = kNaTiles / 2;
constexpr size_t kSliceWords = kNaSlices / 2;
constexpr size_t kCutWords = 32;
constexpr size_t kPerMatWords = kTileWords + kSliceWords + kCutWords;
constexpr size_t kScratchWords = kAccWords + kMaxMulti * kPerMatWords;
static_assert(kTileWords % 32 == 0 && kSliceWords % 32 == 0 && kAccWords % 32 == 0, "256-byte regions");

static __device__ __align__(256) unsigned long long scratch[kScratchWords];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
unsigned long long* g_ptr[kMaxDevices] = {};

// the device address of this device's `scratch` (looked up on first use)
int scratch_address(int device, unsigned long long** out)
{
    if (device < 0 || device >= kMaxDevices) return fail(IAM_E_INVALID, "bucketmul_noalloc: device index out of range");
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_ptr[device]) {
        int cur = -1;
        IAM_CHECK_HIP(hipGetDevice(&cur));
        if (cur != device) IAM_CHECK_HIP(hipSetDevice(device));
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != device) (void)hipSetDevice(cur);
        if (e != hipSuccess)
            return fail(IAM_E_HIP, std::string("bucketmul_noalloc: hipGetSymbolAddress: ") + hipGetErrorString(e));
        if (!p) return fail(IAM_E_HIP, "bucketmul_noalloc: no device address for the scratch array");
        g_ptr[device] = static_cast<unsigned long long*>(p);
    }
    *out = g_ptr[device];
    return IAM_OK;
}

__global__ void k_clear_words(unsigned long long* __restrict__ p, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0ull;
}

int clear_words(Ctx* c, unsigned long long* p, size_t n)
{
    if (n == 0) return IAM_OK;
    const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 1024);
    hipLaunchKernelGGL(k_clear_words, dim3(blocks), dim3(256), 0, c->stream, p, n);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(IAM_E_HIP, std::string("launch clear_words: ") + hipGetErrorString(e));
    return IAM_OK;
}

}  // namespace
}  // namespace iam

using namespace iam;

extern "C" int iam_bucketmul_fused_noalloc(iam_ctx* c, int n, const iam_bucket_matrix* mats, float* x,
                                           int in_size, float* const* ys, int expert_no, float effort,
                                           const float* h, const uint16_t* gain, float eps)
{
    if (!c || !mats || !ys) return fail(IAM_E_INVALID, "bucketmul_noalloc: null argument");
    IAM_REQUIRE(n >= 1 && n <= kMaxMulti, "bucketmul_noalloc: 1..3 matrices per call");
    IAM_REQUIRE(!std::isnan(effort), "bucketmul_noalloc: effort is NaN");
    IAM_REQUIRE(expert_no >= 0, "bucketmul_noalloc: negative expert_no");
    IAM_REQUIRE(in_size > 0, "bucketmul_noalloc: in_size must be positive");
    IAM_REQUIRE(x, "bucketmul_noalloc: null x");
    IAM_REQUIRE(!h == !gain, "bucketmul_noalloc: h and gain go together");
    IAM_REQUIRE(!h || in_size == kProbes, "bucketmul_noalloc: a norm input must be 4096 long");
    // the limits first: shapes beyond them are refused before anything else
    MatOp ops[kMaxMulti];
    size_t outputs = 0;
    WalkGroup tg;                           // the launch's tile width
    const int tc = walk_tile_cols(tg);
    for (int i = 0; i < n; i++) {
        const iam_bucket_matrix& M = mats[i];
        IAM_REQUIRE(M.expert_rows > 0 && M.bucket_cols > 0, "bucketmul_noalloc: empty matrix");
        outputs += (size_t)M.bucket_cols * 16;
        IAM_REQUIRE((M.bucket_cols + tc - 1) / tc <= kNaTiles, "bucketmul_noalloc: more than 256 column tiles");
        ops[i].mat = M;
        ops[i].x = x;
        ops[i].in_size = in_size;
        ops[i].y = ys[i];
    }
    if (outputs > kNaOutputs)
        return fail(IAM_E_INVALID, "bucketmul_noalloc: " + std::to_string(outputs) +
                                       " outputs exceed the scratch limit of " + std::to_string(kNaOutputs));
    // the slices of the plan the launch runs (its selection blocks and tile width)
    const int P = max_slices(n, ops, effort, sel_block_for(c, effort), tc);
    IAM_REQUIRE(P <= kNaSlices, "bucketmul_noalloc: more than 1024 slices");
    // the same argument checks as iam_bucketmul_fused
    for (int i = 0; i < n; i++) {
        const iam_bucket_matrix& M = mats[i];
        IAM_REQUIRE(M.buckets && M.stats && M.probes && ys[i], "bucketmul_noalloc: null buckets/stats/probes/y");
        IAM_REQUIRE(M.stats_stride >= 1 && M.stats_channel >= 0 && M.stats_channel < M.stats_stride,
                    "bucketmul_noalloc: bad stats stride/channel");
        const uint16_t* probes = M.probes + (size_t)expert_no * kProbes;
        IAM_REQUIRE(((uintptr_t)probes & 15) == 0, "bucketmul_noalloc: probes must be 16-byte aligned");
        IAM_REQUIRE(((uintptr_t)M.buckets & 15) == 0, "bucketmul_noalloc: buckets must be 16-byte aligned");
        IAM_REQUIRE(((uintptr_t)ys[i] & 15) == 0, "bucketmul_noalloc: y must be 16-byte aligned");
        const int inputs = (M.expert_rows + 15) / 16;
        IAM_REQUIRE((std::min(inputs, in_size) + kChunkInputs - 1) / kChunkInputs <= kMaxChunks,
                    "bucketmul_noalloc: more than 65536 inputs per expert");
        const size_t xn = std::max<size_t>(kProbes, std::min<size_t>((size_t)in_size, (size_t)inputs));
        IAM_TRY(check_dev_range(c, x, xn * sizeof(float), "bucketmul_noalloc x"));
        IAM_TRY(check_dev_range(c, M.probes, (size_t)(expert_no + 1) * kProbes * 2, "bucketmul_noalloc probes"));
        IAM_TRY(check_dev_range(c, M.stats, (size_t)(expert_no + 1) * M.expert_rows * M.stats_stride * 2,
                                "bucketmul_noalloc stats"));
        IAM_TRY(check_dev_range(c, M.buckets, (size_t)(expert_no + 1) * M.expert_rows * M.bucket_cols * 2,
                                "bucketmul_noalloc buckets"));
        IAM_TRY(check_dev_range(c, ys[i], (size_t)M.bucket_cols * 16 * sizeof(float), "bucketmul_noalloc y"));
    }
    IAM_REQUIRE(((uintptr_t)x & 15) == 0, "bucketmul_noalloc: x must be 16-byte aligned");
    if (h) {
        IAM_TRY(check_dev_range(c, h, (size_t)in_size * sizeof(float), "bucketmul_noalloc h"));
        IAM_TRY(check_dev_range(c, gain, (size_t)in_size * 2, "bucketmul_noalloc gain"));
        IAM_REQUIRE(((uintptr_t)h & 15) == 0 && ((uintptr_t)gain & 15) == 0,
                    "bucketmul_noalloc: h and gain must be 16-byte aligned");
    }

    unsigned long long* base = nullptr;
    IAM_TRY(scratch_address(c->device, &base));
    // accumulators of the group (consecutive), then the per-matrix counters
    unsigned long long* per_mat = base + kAccWords;
    IAM_TRY(clear_words(c, base, outputs));
    IAM_TRY(clear_words(c, per_mat, kMaxMulti * kPerMatWords));

    WalkGroup g;
    g.plain = true;
    g.n = n;
    g.in_mode = h ? kInNorm : kInX;
    g.effort = effort;
    g.expert_no = expert_no;
    g.h = h;
    g.gain = gain;
    g.eps = eps;
    g.fin = kFinStore;
    size_t acc_off = 0;
    for (int i = 0; i < n; i++) {
        unsigned long long* mine = per_mat + (size_t)i * kPerMatWords;
        WalkMat& wm = g.m[i];
        wm.mat = mats[i];
        wm.in_size = in_size;
        wm.x = x;
        wm.acc = base + acc_off;
        wm.tile_ctr = reinterpret_cast<uint32_t*>(mine);
        wm.slice_count = reinterpret_cast<uint32_t*>(mine + kTileWords);
        wm.cutoff = reinterpret_cast<float*>(mine + kTileWords + kSliceWords);
        wm.y = ys[i];
        acc_off += (size_t)mats[i].bucket_cols * 16;
    }
    return walk_group(c, g);
}
