// Internal declarations shared by the HIP translation units of libiam.so.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>

#include <cstdint>
#include <map>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/iam.h"

namespace iam {

// ---------------------------------------------------------------- errors ---
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);

#define IAM_CHECK_HIP(call)                                                         \
    do {                                                                            \
        hipError_t e_ = (call);                                                     \
        if (e_ != hipSuccess)                                                       \
            return ::iam::fail(IAM_E_HIP, std::string(#call) + ": " + hipGetErrorString(e_)); \
    } while (0)

#define IAM_REQUIRE(cond, msg)                                                      \
    do {                                                                            \
        if (!(cond)) return ::iam::fail(IAM_E_INVALID, (msg));                      \
    } while (0)

#define IAM_TRY(expr)                                                               \
    do {                                                                            \
        int rc_ = (expr);                                                           \
        if (rc_ != IAM_OK) return rc_;                                              \
    } while (0)

// ------------------------------------------------------------- constants ---
constexpr int kProbes = IAM_PROBES_COUNT;   // bucketMul.cl:18
constexpr int kChunkInputs = 256;           // inputs per selection chunk (one per thread)
constexpr int kChunkRows = kChunkInputs * 16;
constexpr int kMaxChunks = 256;             // in_dim up to 65536 per expert
constexpr int kMaxMulti = 3;                // matrices per fused launch

// ------------------------------------------------------- dispatch state ---
// One matrix of the last cutoff launch: the selection problem (recorded by
// bucketmul_dispatch, re-evaluated by the walk), the device cutoff and the
// walk's selected-row counter, and the walk partials.  The selected-row
// list (per chunk of 4096 rows, ascending {row id, bits of x[row/16]}) is
// only built for the blocking parity queries.
struct DispatchSlot {
    const float* x = nullptr;
    const uint16_t* stats = nullptr;   // row 0 of the expert
    const uint16_t* probes = nullptr;  // probes of the expert
    int stats_stride = 4;
    int stats_channel = 3;
    int rows = 0;                // expert rows R
    int in_size = 0;
    int bucket_cols = 0;
    int expert_no = 0;
    float effort = 1.0f;
    bool valid = false;
    float* cutoff = nullptr;     // device [2]: k_cutoff's value, the list kernel's value
    uint32_t* count = nullptr;   // device [1]: rows selected by the last walk
    bool counted = false;        // the last walk counted its rows (counting was on)
    uint2* list = nullptr;       // [G][kChunkRows]
    uint32_t* counts = nullptr;  // [kMaxChunks]
    size_t cap_chunks = 0;
    int G = 0;                   // chunks of the last list
    void* part = nullptr;        // walk partial sums [P][m] of the accumulator type
    size_t part_cap = 0;         // bytes
};

struct KernelStat {
    int calls = 0;
    double total_ms = 0.0;
    double max_ms = 0.0;
};

struct PendingEvent {
    const char* name;
    hipEvent_t start, stop;
};

struct Ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    size_t total_mem = 0;
    size_t usable = 0;
    size_t allocated = 0;
    std::map<uintptr_t, size_t> allocs;   // base -> bytes
    bool profiling = false;
    bool capturing = false;
    std::vector<PendingEvent> pending;
    std::vector<hipEvent_t> event_pool;
    std::map<std::string, KernelStat> stats;
    DispatchSlot slots[kMaxMulti];
    float* attn_ws = nullptr;          // split-context attention partials
    size_t attn_ws_floats = 0;
    // bumped whenever a context-owned scratch buffer (dispatch lists, walk
    // partials, attention workspace) is reallocated: captured graphs hold
    // those addresses and must be re-captured when it changes
    uint64_t scratch_gen = 0;
    unsigned long long* counters = nullptr;   // device: walk bytes, rows, matrices
    // the reduce adds up the walk's selected rows into the slot counts and
    // the counters (off: neither is updated, and the reduce is shorter)
    bool counting = true;
    // accumulate the walk in fp64 (sums round once to fp32) instead of fp32
    bool acc64 = true;
};

int ctx_alloc(Ctx* c, size_t bytes, void** out);
// IAM_OK if [p, p+bytes) lies inside one allocation of this context
int check_dev_range(Ctx* c, const void* p, size_t bytes, const char* what);
int ctx_free(Ctx* c, void* p);
int ensure_slot(Ctx* c, int slot);
int ensure_list(Ctx* c, int slot, int chunks);
int ensure_partials(Ctx* c, int slot, size_t bytes);

// Launch bookkeeping: with profiling on (and no graph capture in progress)
// each launch is bracketed by a pair of pooled events.
int begin_launch(Ctx* c, const char* name, PendingEvent* ev);
int end_launch(Ctx* c, PendingEvent* ev, bool have_ev);

template <typename Kernel, typename... Args>
int launch(Ctx* c, const char* name, Kernel k, dim3 grid, dim3 block, size_t shmem,
           Args... args)
{
    if (grid.x == 0 || grid.y == 0 || grid.z == 0) return IAM_OK;
    if (c->profiling && !c->capturing) {
        // the events are stamped by the kernel's own dispatch, so the elapsed
        // time is the kernel's duration, without host-side gaps
        PendingEvent ev{};
        IAM_TRY(begin_launch(c, name, &ev));
        hipExtLaunchKernelGGL(k, grid, block, (uint32_t)shmem, c->stream, ev.start, ev.stop, 0, args...);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess)
            return fail(IAM_E_HIP, std::string("launch ") + name + ": " + hipGetErrorString(e));
        return end_launch(c, &ev, true);
    }
    hipLaunchKernelGGL(k, grid, block, shmem, c->stream, args...);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return fail(IAM_E_HIP, std::string("launch ") + name + ": " + hipGetErrorString(e));
    return IAM_OK;
}

int zero_async(Ctx* c, void* p, size_t bytes);

// ------------------------------------------------------------- bucketMul ---
struct MatOp {
    iam_bucket_matrix mat;
    const float* x;
    int in_size;
    float* y;        // may be null for dispatch-only
};
// record the selection problems of n matrices in slots 0..n-1 and compute
// their cutoffs
int bucketmul_dispatch(Ctx* c, int n, const MatOp* ops, int expert_no, float effort);
// selection + walk of slots 0..n-1 into per-slice partial sums, then the
// fixed-order reduction into each y (overwritten)
int bucketmul_walk(Ctx* c, int n, const MatOp* ops);

// How a fused walk gets its input and cutoff.
enum WalkIn : int {
    kInCutoff = 0,   // x in memory, cutoff from a preceding cutoff launch
    kInX = 1,        // x in memory; every walk workgroup runs the cutoff search itself
    kInNorm = 2,     // x = rmsnorm(h) * gain (4096 inputs) computed by every
                     // walk workgroup (the first one stores it to x), then the search
};

// What the reduce does with y after storing it.
enum Epi : int {
    kEpStore = 0,   // nothing more
    kEpResid = 1,   // out += y (add32, bucketMul.cl:517-520)
    kEpRopeQ = 2,   // out = rope(y) at *pos (rope_mx, aux.cl:227-248)
    kEpRopeK = 3,   // cache row *pos = fp16(rope(y)) (attention.hpp:172-189, 281-309)
    kEpV = 4,       // cache row *pos = fp16(y)
    kEpSilu = 5,    // ops 0 (gate g) and 1 (up u): out = u * g / (1 + exp(-g)) (silu32, matrix.cl:27-32)
};

struct ReduceEp {
    int ep = kEpStore;
    float* out = nullptr;
    const float* table = nullptr;   // RoPE table [max_ctx][64][2]
    const int* pos = nullptr;       // device position
    int max_ctx = 0;
    uint16_t* cache = nullptr;      // fp16 rows [max_ctx][m]
};

// record + (norm, cutoff) + walk + reduce with epilogues of one matrix group;
// ep may be null (store y)
int bucketmul_fused(Ctx* c, int n, const MatOp* ops, int expert_no, float effort, int in_mode, const float* h,
                    const uint16_t* gain, float eps, const ReduceEp* ep);
// size the slots and partial buffers of a group so a later call allocates nothing
int reserve_walk(Ctx* c, int n, const MatOp* ops, float effort);
// grid plan of one matrix in a walk launch
struct WalkPlan {
    int NW;     // waves per workgroup (the same for every matrix of a launch)
    int V;      // columns per lane load
    int T;      // column tiles (128 columns for k_walk64, 64 for k_walk)
    int n_in;   // inputs walked
    int IPS;    // inputs per slice
    int P;      // slices
};
void plan_walk(int n, const MatOp* ops, float effort, bool acc64, WalkPlan* plan);
int ensure_attn_ws(Ctx* c, size_t floats);

int quantile_of(float effort);
double est_rows(int rows, float effort);

}  // namespace iam

struct iam_ctx : iam::Ctx {};
