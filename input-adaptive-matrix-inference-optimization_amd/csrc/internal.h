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
// One matrix of the last cutoff / walk launch: the selection problem
// (recorded by bucketmul_dispatch, re-evaluated by the walk), the device
// cutoff, and the walk's scratch: the output accumulator (zero between
// calls: the walk's last workgroup per column tile reads and clears it),
// the tiles' arrival counters and the per-slice selected-row counts.  The
// selected-row list (per chunk of 4096 rows, ascending {row id, bits of
// x[row/16]}) is only built for the blocking parity queries.
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
    float* cutoff = nullptr;     // device [4]: the search's value, the list kernel's value, the search's hint
    uint2* list = nullptr;       // [G][kChunkRows]
    uint32_t* counts = nullptr;  // [kMaxChunks]
    size_t cap_chunks = 0;
    int G = 0;                   // chunks of the last list
    void* acc = nullptr;         // [acc_cap] accumulators (8 bytes each), zero between calls
    size_t acc_cap = 0;
    uint32_t* tile_ctr = nullptr;     // [tile_cap] arrival counters, zero between calls
    size_t tile_cap = 0;
    uint32_t* slice_count = nullptr;  // [slice_cap] rows selected per slice by the last walk
    size_t slice_cap = 0;
    int walked_P = 0;            // slices of the last walk of this slot (0: none)
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
    // attention, standalone entry point: the splits' partial sums (o and
    // the softmax sum per head and split) and the per-head arrival counters
    // (zero between calls)
    void* attn_acc = nullptr;
    size_t attn_acc_cap = 0;
    uint32_t* attn_ctr = nullptr;
    // the fp32 attention over the reference's cache layout: exp(s) per head
    // and position, the splits' sums and partial outputs
    float* attn32 = nullptr;
    size_t attn32_cap = 0;
    // bumped whenever a context-owned scratch buffer is reallocated:
    // captured graphs hold those addresses and must be re-captured
    uint64_t scratch_gen = 0;
    // device walk counters, one block per walk label (kWalkLabels), each of
    // kCounterLanes rows of {weight bytes, rows, matrices, hinted searches
    // << 32 | their hits}: each walk
    // adds to row (slice % kCounterLanes) of its label's block, so the
    // additions of one launch do not queue on one address
    unsigned long long* counters = nullptr;
    // the walk adds its selected rows and bytes to the counters (off: it
    // does not touch them)
    bool counting = true;
    // accumulate the walk in fp64 (sums round once to fp32) instead of fp32
    bool acc64 = true;
    // block-structured selection: inputs per block (1: the reference's
    // per-row selection), used for efforts below sel_below
    int sel_block = 1;
    float sel_below = 2.0f;
    // fused calls start their cutoff search from the slot's hint, the
    // slot's cutoff of the previous fused call (iam_set_search_hints)
    bool hints = false;
};

int ctx_alloc(Ctx* c, size_t bytes, void** out);
// IAM_OK if [p, p+bytes) lies inside one allocation of this context
int check_dev_range(Ctx* c, const void* p, size_t bytes, const char* what);
int ctx_free(Ctx* c, void* p);
int ensure_slot(Ctx* c, int slot);
int ensure_list(Ctx* c, int slot, int chunks);
// the walk scratch of a slot: accumulators for m outputs, T tile counters,
// P slice counts (grown as needed; new memory is zeroed)
int ensure_walk_scratch(Ctx* c, int slot, size_t m, size_t T, size_t P);
constexpr int kCounterLanes = 64;
constexpr int kWalkLabels = 6;   // standalone, q/k/v, o, w1/w3, w2, LM head
constexpr size_t kCounterWords = (size_t)kWalkLabels * kCounterLanes * 4;

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
// selection + walk of slots 0..n-1 with the cutoffs of the last dispatch,
// y overwritten
int bucketmul_walk(Ctx* c, int n, const MatOp* ops);

// How a walk gets its input (x[0:4096] for the cutoff, and its slice).
enum WalkIn : int {
    kInCutoff = 0,     // x in memory, cutoff from a preceding cutoff launch
    kInX = 1,          // x in memory; every walk workgroup runs the cutoff search
    kInNorm = 2,       // x = rmsnorm(h) * gain (4096 inputs), then the search
    kInResNorm = 3,    // h = h + (float)delta accumulator (add32), stored; x = rmsnorm(h) * gain
    kInEmbedNorm = 4,  // h = embedding row of the device token (optionally scaled), stored; x = rmsnorm(h) * gain
    kInAttn = 5,       // x = o / l from the attention accumulators
};

// What happens to the outputs after the flush into the accumulators.
enum WalkFin : int {
    kFinNone = 0,    // they stay in the accumulators (the consumer reads them)
    kFinStore = 1,   // the last workgroup of each column tile stores them as fp32 and clears them
    kFinSilu = 2,    // matrices 0 (gate) and 1 (up): the last workgroup of each tile stores
                     // up * gate / (1 + exp(-gate)) (silu32, matrix.cl:27-32) and clears both
};

// grid plan of one matrix in a walk launch
struct WalkPlan {
    int NW;     // waves per workgroup (the same for every matrix of a launch)
    int T;      // column tiles of tc columns
    int n_in;   // inputs walked
    int IPS;    // inputs per slice
    int P;      // slices
};
// blk: inputs per selection block (slices start at its multiples); tc:
// columns per tile (the launch's walk_tile_cols)
void plan_walk(int n, const MatOp* ops, float effort, WalkPlan* plan, int blk, int tc);
// the selection block size of a walk at this effort
int sel_block_for(const Ctx* c, float effort);

// A matrix group of the decode step (or of a standalone call): up to 3
// matrices sharing one input mode.  Per matrix: the accumulator (zero on
// entry), and for the finalize modes the tile counters (zero on entry) and
// the fp32 outputs.
struct WalkMat {
    iam_bucket_matrix mat;
    int in_size;
    const float* x;          // kInX / kInCutoff: the input; norm and attention modes: where block 0
                             // stores the computed input (may be null)
    float* cutoff;           // the search's result is stored here (kInCutoff: read from here)
    // or null: the cutoff search's hint, this matrix's cutoff of the
    // previous call (read, then rewritten by the walk); any value is safe
    float* hint = nullptr;
    uint32_t* slice_count;   // [P]
    void* acc;               // [16 * bucket_cols] of the accumulator type
    // a second accumulator of the same size (or null): the slices of odd
    // index add there, halving the chains of adds to one address where one
    // column tile takes every slice (kFinNone only; the consumer adds both)
    void* acc2 = nullptr;
    uint32_t* tile_ctr;      // [T]
    float* y;                // kFinStore: outputs; kFinSilu: the gate / up values (may be null)
};
struct WalkGroup {
    // the model's matrix group of the launch (IAM_WALK_GROUP_*; 0: a
    // standalone call): picks the kernel-statistics name and the counter block
    int label = 0;
    // launch without the profiling events (the no-allocation entry point)
    bool plain = false;
    // columns per tile (64 or 128; 0: the group's default)
    int tile_cols = 0;
    int n = 0;
    WalkMat m[kMaxMulti];
    int in_mode = kInX;
    float effort = 1.0f;
    int expert_no = 0;
    const float* h = nullptr;          // kInNorm / kInResNorm
    const void* res_acc = nullptr;     // kInResNorm (may be null)
    float* h_out = nullptr;            // kInResNorm / kInEmbedNorm (may be null)
    const uint16_t* gain = nullptr;
    float eps = 1e-5f;
    const uint16_t* embed = nullptr;   // kInEmbedNorm
    const int* token = nullptr;
    const float* embed_scale = nullptr;
    int vocab = 0;
    const void* attn_acc = nullptr;    // kInAttn
    int fin = kFinNone;
    float* silu_out = nullptr;         // kFinSilu
    // the last finalizing workgroup (kFinStore with pick_ctr): greedy pick
    // of the stored outputs when token_out is set, then the final clear
    uint32_t* pick_ctr = nullptr;
    void* tile_cand = nullptr;         // [T] (value, index)
    int* token_out = nullptr;
    int* pos = nullptr;
    int* hist = nullptr;
    int hist_len = 0;
    void* final_zero = nullptr;
    int final_zero_n = 0;
    // accumulators cleared by the launch (spread over its workgroups)
    void* zero_p[2] = {nullptr, nullptr};
    int zero_n[2] = {0, 0};
};
// one walk launch of the group (plan from the matrices and effort)
int walk_group(Ctx* c, const WalkGroup& g);
// columns per tile of the group's walk launch (64 or 128)
int walk_tile_cols(const WalkGroup& g);
// column tiles of a matrix at the narrowest tile width (the most any launch
// uses: the size of per-tile counters and candidates)
int walk_tiles(int bucket_cols);
// the largest slice count of the plan a walk of these matrices runs with
// (selection blocks of blk inputs, tiles of tc columns)
int max_slices(int n, const MatOp* ops, float effort, int blk, int tc);

// standalone calls: dispatch + walk with fp32 outputs (y), in_mode kInX or
// kInNorm (the norm of h written to ops[0].x)
int bucketmul_fused(Ctx* c, int n, const MatOp* ops, int expert_no, float effort, int in_mode, const float* h,
                    const uint16_t* gain, float eps);
int ensure_attn_scratch(Ctx* c, size_t acc_words, int n_heads);
int ensure_attn32_scratch(Ctx* c, size_t floats);

int quantile_of(float effort);
double est_rows(int rows, float effort);

}  // namespace iam

struct iam_ctx : iam::Ctx {};
