// Input-adaptive sparse GEMV ("bucketMul") for gfx950.
//
// Reference pipeline (bucket_mul.hpp:147-267, bucketMul.cl):
//   findCutoffBinarySearch -> prepareDispatch -> roundUp/zeroRange32 ->
//   bucketMul -> bucketIntegrate                      (6 launches + 1 fill)
// Here, per group of up to 3 matrices that share an input:
//   k_walk64    one launch (fp64 accumulation): workgroup (input slice p,
//               128-column tile t) computes the RMSNorm of h when the input
//               is a norm of 4096 values (a wider one goes through the
//               RMSNorm kernel first), runs the cutoff search itself (a pure function of
//               x[0:4096] and the probes), selects the rows of its slice and
//               walks them, adding each exact product x*w to its wave's LDS
//               tile with fp64 atomics in a fixed order, and writes one
//               partial row per slice.
//   k_reduce    one launch: sums the slice partials in a fixed order and
//               applies the consumer's epilogue (residual add, RoPE and the
//               fp16 KV append, the SiLU gate, or a store); with walk
//               counting on it also adds up the selected rows.
// k_walk (fp32 accumulation, lane-private accumulators) follows k_cutoff;
// k_cutoff and k_dispatch (one workgroup per matrix / per 256 inputs) serve
// the standalone calls and the parity queries (cutoff, selected rows).
// The cutoff and selection arithmetic is exact IEEE fp32 (no contraction), so
// the cutoff bits and the selected set equal the oracle's.  With fp64
// accumulation (the product of an fp32 input and an fp16 weight is exact in
// fp64) y is the correctly rounded sum up to fp64 rounding, and the fixed
// order makes it the same on every run.
#include <hip/hip_fp16.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "internal.h"
#include "layer_ops.h"
#include "wave.h"

namespace iam {

constexpr float kScale = 100000.0f;   // bucketMul.cl:17
constexpr int kCutThreads = 256;
constexpr int kCutVPT = kProbes / kCutThreads;   // 16 importances per thread

__device__ __forceinline__ float h2f(uint32_t bits16)
{
    return __half2float(__ushort_as_half((unsigned short)(bits16 & 0xffffu)));
}

// --------------------------------------------------------------- cutoff ---
// A wave-uniform float kept in a scalar register.
__device__ __forceinline__ float uniform_f(float v)
{
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}

// The search's bounds are midpoints inside the current bracket (minB,
// maxB], so once the bracket holds few importances, count(imp > b) =
// count(imp > maxB) + #(bracket values > b).  The rounds run on the whole
// workgroup (one count exchange per round) until the bracket holds at most
// kCandCap values by its counts (minCount - maxCount bounds them); those are
// then compacted to LDS, and every wave finishes the rounds on them by itself
// with no barriers.  The tested bounds, counts and stop decisions are the
// reference's exactly.
constexpr int kCandCap = 256;   // 4 per lane of one wave

// The 16 probes of thread tid (probes[16*tid ..]).
__device__ __forceinline__ void load_probes(const uint16_t* __restrict__ probes, uint4 (&pr)[2])
{
    const uint4* pv = reinterpret_cast<const uint4*>(probes + threadIdx.x * kCutVPT);
    pr[0] = pv[0];
    pr[1] = pv[1];
}

// xs holds x[16*tid .. 16*tid + 16) and pr the thread's probes for the
// first kCutThreads threads; a block of NWV > 4 waves runs the same code and
// its other threads hold no importances (NaN: never counted, ignored by the
// min and max).  Scratch: s_red >= 2*NWV floats, s_cnt >= 3*NWV ints,
// s_cand kCandCap floats.  Every thread returns the cutoff; a later writer of
// the scratch must pass a barrier first (the waves read s_cand after the
// last barrier here).
template <int NWV = 4>
__device__ __forceinline__ float block_cutoff_x(const float (&xs)[kCutVPT], const uint4 (&pr)[2], int quantile,
                                                float* s_red, int* s_cnt, float* s_cand)
{
#pragma clang fp contract(off)
    static_assert(NWV % 4 == 0, "4 or 8 waves");
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    float v[kCutVPT];
    {
        const uint4 pa = pr[0], pb = pr[1];
        uint32_t ps[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
#pragma unroll
        for (int k = 0; k < 16; k++) {
            float p = h2f(ps[k >> 1] >> ((k & 1) * 16));
            float prod = __fmul_rn(xs[k], p);
            v[k] = __fmul_rn(kScale, fabsf(prod));   // bucketMul.cl:110
            if (NWV > 4 && tid >= kCutThreads) v[k] = __int_as_float(0x7fc00000);
        }
    }
    float mn = 1e30f, mx = -1e30f;                    // bucketMul.cl:98-99
#pragma unroll
    for (int k = 0; k < 16; k++) {
        mn = fminf(mn, v[k]);
        mx = fmaxf(mx, v[k]);
    }
    mn = wave_min(mn);
    mx = wave_max(mx);
    if (lane == 0) {
        s_red[wave] = mn;
        s_red[NWV + wave] = mx;
    }
    __syncthreads();
    // the search state is uniform: keep it in scalar registers
    float gmin = 1e30f, gmax = -1e30f;
#pragma unroll
    for (int w4 = 0; w4 < NWV; w4 += 4) {
        const float4 mn4 = *reinterpret_cast<const float4*>(s_red + w4);
        const float4 mx4 = *reinterpret_cast<const float4*>(s_red + NWV + w4);
        gmin = fminf(gmin, fminf(fminf(mn4.x, mn4.y), fminf(mn4.z, mn4.w)));
        gmax = fmaxf(gmax, fmaxf(fmaxf(mx4.x, mx4.y), fmaxf(mx4.z, mx4.w)));
    }
    gmin = uniform_f(gmin);
    gmax = uniform_f(gmax);

    const int target = kProbes - quantile;            // bucketMul.cl:81
    float minB = gmin, maxB = gmax;
    float bound = uniform_f(__fmul_rn(__fadd_rn(gmin, gmax), 0.5f));
    int minC = kProbes, maxC = 0;
    // one round of bucketMul.cl:178-200 given the count at bound; true = stop
    auto round = [&](int count) -> bool {
        if (count < target) {                          // bucketMul.cl:178-186
            maxB = bound;
            maxC = count;
        } else {
            minB = bound;
            minC = count;
        }
        const float next = uniform_f(__fmul_rn(__fadd_rn(minB, maxB), 0.5f));
        const int gap = maxC - minC;
        if (count == target || __fsub_rn(maxB, minB) < 0.00001f || (gap < 0 ? -gap : gap) < 3)
            return true;                               // bucketMul.cl:195-200: the tested bound
        bound = next;
        return false;
    };
    int loop = 0;
    for (; loop < 20; loop++) {
        if (minC - maxC <= kCandCap) break;
        int c = 0;
#pragma unroll
        for (int k = 0; k < 16; k++) c += __popcll(__ballot(v[k] > bound));
        if (lane == 0) s_cnt[(loop & 1) * NWV + wave] = c;
        __syncthreads();
        int tot = 0;
#pragma unroll
        for (int w4 = 0; w4 < NWV; w4 += 4) {
            const int4 q4 = *reinterpret_cast<const int4*>(s_cnt + (loop & 1) * NWV + w4);
            tot += q4.x + q4.y + q4.z + q4.w;
        }
        if (round(__builtin_amdgcn_readfirstlane(tot))) return bound;
    }
    if (loop == 20) return bound;                      // bucketMul.cl:211-213: the untested midpoint

    // compact the bracket values (minB, maxB] to s_cand (the count only
    // needs the set, so the order is per wave, then by k, then by lane)
    uint64_t bm[16];
    int wtot = 0;
#pragma unroll
    for (int k = 0; k < 16; k++) {
        bm[k] = __ballot(v[k] > minB && v[k] <= maxB);
        wtot += __popcll(bm[k]);
    }
    if (lane == 0) s_cnt[2 * NWV + wave] = wtot;
    __syncthreads();
    int off = 0, ncand = 0;   // ncand <= minC - maxC <= kCandCap
#pragma unroll
    for (int w2 = 0; w2 < NWV; w2++) {
        const int c2 = s_cnt[2 * NWV + w2];
        if (w2 < wave) off += c2;
        ncand += c2;
    }
#pragma unroll
    for (int k = 0; k < 16; k++) {
        if ((bm[k] >> lane) & 1ull) s_cand[off + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bm[k] >> 32),
                                                  __builtin_amdgcn_mbcnt_lo((uint32_t)bm[k], 0u))] = v[k];
        off += __popcll(bm[k]);
    }
    __syncthreads();
    // every wave finishes the rounds on the compacted values by itself
    float cv[kCandCap / 64];
#pragma unroll
    for (int j = 0; j < kCandCap / 64; j++) cv[j] = lane + 64 * j < ncand ? s_cand[lane + 64 * j] : -INFINITY;
    const int c0 = maxC;                               // count(imp > maxB) at the compaction
    bool done = false;
    for (; loop < 20 && !done; loop++) {
        int c = c0;
#pragma unroll
        for (int j = 0; j < kCandCap / 64; j++) c += __popcll(__ballot(cv[j] > bound));
        done = round(c);
    }
    return bound;
}

__device__ __forceinline__ void load16(const float* __restrict__ x, float (&xs)[kCutVPT])
{
    const float4* xv = reinterpret_cast<const float4*>(x + threadIdx.x * kCutVPT);
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float4 a = xv[k];
        xs[4 * k] = a.x;
        xs[4 * k + 1] = a.y;
        xs[4 * k + 2] = a.z;
        xs[4 * k + 3] = a.w;
    }
}

__device__ float block_cutoff(const float* __restrict__ x, const uint16_t* __restrict__ probes,
                              int quantile, float* s_red, int* s_cnt, float* s_cand)
{
    float xs[kCutVPT];
    uint4 pr[2];
    load_probes(probes, pr);
    load16(x, xs);
    return block_cutoff_x(xs, pr, quantile, s_red, s_cnt, s_cand);
}

// rmsNorm32fast (aux.cl:156-196) of a 4096-vector by one 256-thread
// workgroup, in the reference's fp32 order: 16 consecutive squares per
// thread summed in order, then the 256-way tree (pairs tid, tid + st for st =
// 128 .. 1: the thread sums through LDS, then the tree by every wave on its
// own), scale = 1/sqrt(sum/4096 + eps) rounded from double, then the fp16 gain
// (mul16x32, aux.cl:434-440).  v holds h[16*tid ..] on entry and the
// normalized values on exit; gr the thread's 16 gains (gain[16*tid ..]).
// s_part: kCutThreads floats of scratch that nothing writes again before a
// later barrier (each wave reads it after the one barrier here).
__device__ __forceinline__ void block_rmsnorm4096(float (&v)[kCutVPT], const uint4 (&gr)[2], float eps, float* s_part)
{
#pragma clang fp contract(off)
    const int tid = threadIdx.x;
    const uint4 g0 = gr[0], g1 = gr[1];
    float sq = 0.0f;
#pragma unroll
    for (int k = 0; k < kCutVPT; k++) sq = __fadd_rn(sq, __fmul_rn(v[k], v[k]));
    if (tid < kCutThreads) s_part[tid] = sq;
    __syncthreads();
    // every wave runs the tree itself (no second barrier): lane l takes
    // part[l] + part[l+128] and part[l+64] + part[l+192] (st = 128), their
    // sum (st = 64), then st = 32, 16 as shuffles and st = 8 .. 1 within
    // 16-lane rows by DPP row_shl (lane l takes lane l + st); lane 0 holds
    // the total
    const int lane = tid & 63;
    const float a = __fadd_rn(s_part[lane], s_part[lane + 128]);
    const float b = __fadd_rn(s_part[lane + 64], s_part[lane + 192]);
    sq = __fadd_rn(a, b);
    sq = __fadd_rn(sq, __shfl_down(sq, 32, 64));
    sq = __fadd_rn(sq, __shfl_down(sq, 16, 64));
    sq = __fadd_rn(sq, dpp_f<0x108>(0.0f, sq));
    sq = __fadd_rn(sq, dpp_f<0x104>(0.0f, sq));
    sq = __fadd_rn(sq, dpp_f<0x102>(0.0f, sq));
    sq = __fadd_rn(sq, dpp_f<0x101>(0.0f, sq));
    const float total = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(sq)));
    const float mean = __fdiv_rn(total, 4096.0f);
    const float scale = (float)(1.0 / sqrt((double)__fadd_rn(mean, eps)));
    const uint32_t gw[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
    for (int k = 0; k < kCutVPT; k++)
        v[k] = __fmul_rn(h2f(gw[k >> 1] >> ((k & 1) * 16)), __fmul_rn(v[k], scale));
}

// --------------------------------------------------------------- cutoff ---
// One workgroup per matrix: the cutoff of findCutoffBinarySearch.
struct CutoffDesc {
    const float* x;
    const uint16_t* probes;   // already offset to the expert
    int quantile;
    float* cutoff;
};

struct CutoffArgs {
    CutoffDesc d[kMaxMulti];
    int n;
};

__global__ __launch_bounds__(kCutThreads) void k_cutoff(CutoffArgs a)
{
    __shared__ __align__(16) float s_red[16];
    __shared__ __align__(16) int s_cnt[16];
    __shared__ float s_cand[kCandCap];
    const CutoffDesc& d = a.d[blockIdx.x];
    const float cut = block_cutoff(d.x, d.probes, d.quantile, s_red, s_cnt, s_cand);
    if (threadIdx.x == 0) d.cutoff[0] = cut;
}

// ------------------------------------------------------------- dispatch ---
struct DispatchDesc {
    const float* x;
    const uint16_t* probes;   // already offset to the expert
    const uint16_t* stats;    // row 0 of the expert
    int stats_stride;
    int stats_channel;
    int rows;                 // R
    int in_size;
    int quantile;
    int G;                    // chunks
    uint2* list;
    uint32_t* counts;
    float* cutoff;
    int block_base;
};

struct DispatchArgs {
    DispatchDesc d[kMaxMulti];
    int n;
};

__global__ __launch_bounds__(kCutThreads) void k_dispatch(DispatchArgs a)
{
#pragma clang fp contract(off)
    __shared__ __align__(16) float s_red[16];
    __shared__ __align__(16) int s_cnt[16];
    __shared__ float s_cand[kCandCap];
    __shared__ int s_wsum[4];

    int k = 0;
    for (int i = 1; i < a.n; i++)
        if ((int)blockIdx.x >= a.d[i].block_base) k = i;
    const DispatchDesc& d = a.d[k];
    const int g = (int)blockIdx.x - d.block_base;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    const float cutoff = block_cutoff(d.x, d.probes, d.quantile, s_red, s_cnt, s_cand);
    if (g == 0 && tid == 0) d.cutoff[1] = cutoff;   // cross-checked against k_cutoff's cutoff[0]

    // prepareDispatch (bucketMul.cl:362-385) for the 16 rows of input i
    const int i = g * kChunkInputs + tid;
    const int r0 = i * 16;
    uint32_t mask = 0;
    float xi = 0.0f;
    if (i < d.in_size && r0 < d.rows) {
        xi = d.x[i];
        // the 16 stats of this input, all loads issued before any use
        uint32_t sv[16];
        const uint16_t* st = d.stats + (size_t)r0 * d.stats_stride;
        const bool whole = r0 + 16 <= d.rows;
        if (whole && d.stats_stride == 1 && (((uintptr_t)st) & 15) == 0) {
            const uint4* p4 = reinterpret_cast<const uint4*>(st);
            const uint4 a0 = p4[0], a1 = p4[1];
            const uint32_t w[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
            for (int kk = 0; kk < 16; kk++) sv[kk] = (w[kk >> 1] >> ((kk & 1) * 16)) & 0xffffu;
        } else if (whole && d.stats_stride == 4 && d.stats_channel == 3 && (((uintptr_t)st) & 15) == 0) {
            // reference layout: 4 equal channels per row, channel 3 read
            const uint4* p4 = reinterpret_cast<const uint4*>(st);
            uint4 a[8];
#pragma unroll
            for (int k8 = 0; k8 < 8; k8++) a[k8] = p4[k8];
#pragma unroll
            for (int k8 = 0; k8 < 8; k8++) {
                sv[2 * k8] = a[k8].y >> 16;       // row 2*k8, channel 3
                sv[2 * k8 + 1] = a[k8].w >> 16;   // row 2*k8+1, channel 3
            }
        } else {
#pragma unroll
            for (int kk = 0; kk < 16; kk++) {
                const int rr = min(r0 + kk, d.rows - 1) - r0;
                sv[kk] = st[(size_t)rr * d.stats_stride + d.stats_channel];
            }
        }
#pragma unroll
        for (int kk = 0; kk < 16; kk++) {
            float avg = h2f(sv[kk]);
            float prod = __fmul_rn(xi, avg);
            float imp = __fmul_rn(kScale, fabsf(prod));
            if (imp >= cutoff && r0 + kk < d.rows) mask |= 1u << kk;   // bucketMul.cl:380
        }
    }
    // ordered compaction: block exclusive scan of the per-thread counts
    const int cnt = __popc(mask);
    int incl = cnt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        int t = __shfl_up(incl, o, 64);
        if (lane >= o) incl += t;
    }
    __syncthreads();   // s_cnt/s_red reads of the search are done
    if (lane == 63) s_wsum[wave] = incl;
    __syncthreads();
    int woff = 0;
    for (int w = 0; w < wave; w++) woff += s_wsum[w];
    const int total = s_wsum[0] + s_wsum[1] + s_wsum[2] + s_wsum[3];
    uint2* out = d.list + (size_t)g * kChunkRows + (woff + incl - cnt);
    const uint32_t xb = __float_as_uint(xi);
    while (mask) {
        int kk = __ffs(mask) - 1;
        mask &= mask - 1;
        *out++ = make_uint2((uint32_t)(r0 + kk), xb);
    }
    if (tid == 0) d.counts[g] = (uint32_t)total;
}

// ----------------------------------------------------------------- walk ---
// Blocks are dealt to the 8 XCDs round robin (block b -> XCD b % 8).  Remap
// so that consecutive work items (the column tiles of one row slice, which
// share 128-byte lines at misaligned row starts) land on the same XCD and so
// share its L2.
__device__ __forceinline__ int xcd_remap(int b, int nblocks)
{
    const int q = nblocks >> 3, r = nblocks & 7;
    const int xcd = b & 7, idx = b >> 3;
    return xcd < r ? xcd * (q + 1) + idx : r * (q + 1) + (xcd - r) * q + idx;
}

template <int VEC>
struct VecLoad;
template <>
struct VecLoad<4> {
    using T = uint2;
    __device__ static void split(const T& v, uint32_t* w) { w[0] = v.x; w[1] = v.y; }
};
template <>
struct VecLoad<2> {
    using T = uint32_t;
    __device__ static void split(const T& v, uint32_t* w) { w[0] = v; }
};
template <>
struct VecLoad<1> {
    using T = uint16_t;
    __device__ static void split(const T& v, uint32_t* w) { w[0] = v; }
};

// acc + x * w in the accumulator type: an fp32 product added in fp32
// (bucketMul.cl:430-434), or in fp64, where the product of an fp32 x and an
// fp16 w is exact (24 + 11 significant bits fit in 53).
template <typename Acc>
__device__ __forceinline__ Acc walk_acc(Acc x, Acc w, Acc old);
template <>
__device__ __forceinline__ float walk_acc<float>(float x, float w, float old)
{
    return __fadd_rn(old, __fmul_rn(x, w));   // bucketMul.cl:430-434: fp32 product, then the add
}
template <>
__device__ __forceinline__ double walk_acc<double>(double x, double w, double old)
{
    return fma(x, w, old);   // the product is exact in fp64, so this is one rounded add
}

// Selection + walk.  Workgroup (input slice p, column tile t) owns the
// inputs [p*IPS, (p+1)*IPS) and the 64 columns of tile t.
//
// Selection (prepareDispatch, bucketMul.cl:351-386): thread i takes input
// p*IPS + i, loads its x and the stats of its 16 rows, and marks the rows
// with 1e5 * |x * stat| >= cutoff -- the same fp32 operations as the
// dispatch kernel, so the selected set is the same.  A block scan compacts
// the selected rows in ascending order into LDS.
//
// Walk: lane = q*NJ + j: j picks VEC consecutive columns (NJ = 64/VEC lanes
// cover the 128-byte tile segment of one row), q one of NQ = VEC rows read
// by the same instruction.  Every lane owns private accumulators for its VEC
// columns x 16 output positions at acc[wave][(pos*VEC + e)*64 + lane]: the
// scatter of a packed weight to its position (bucketMul.cl:430-445) is a
// plain LDS read-add-write, with no atomics, and the 64 lanes of one access
// fall in 64 different banks.  Each lane adds its rows in order and the
// flush sums waves and row slots in a fixed order, so the result does not
// depend on scheduling.  The VEC elements of one row go to distinct
// addresses (different e), so their reads are issued together, then their
// writes; the next row's reads follow in the wave's LDS order.  All UNR
// weight loads of a batch are unconditional (past the end a lane re-reads
// the last selected row with x = 0), so they are in flight together.
struct WalkDesc {
    const uint16_t* W;        // rows of the expert: W[row * C + col]
    float* x;
    const uint16_t* stats;    // row 0 of the expert
    float* cutoff;
    uint32_t* slice_count;    // [P]: rows selected per slice (tile-0 workgroups)
    void* part;               // [P][16*C] partial sums (Acc), one row per slice
    const float* h;           // kInNorm: the vector to normalize
    const uint16_t* gain;     // kInNorm: fp16 gain
    const uint16_t* probes;   // kInX / kInNorm: probes of the expert
    float eps;
    int quantile;
    int in_mode;              // WalkIn
    int stats_stride;
    int stats_channel;
    int rows;                 // R
    int n_in;                 // inputs walked: min(ceil(R/16), in_size)
    int C;
    int IPS;                  // inputs per slice (<= threads per workgroup)
    int P;                    // slices
    int T;                    // column tiles
    int block_base;
};

struct WalkArgs {
    WalkDesc d[kMaxMulti];
    int n;
};

// Loads of the selection: the 16 stats (channel stats_channel) of input
// i0 + tid's rows and, unless x_lds, its x.  Issued before the cutoff is
// known so that their latency overlaps the search; the raw words are kept
// (unpacked by select_finish) so that nothing waits for them here.  Layouts:
// compact stats (stride 1, 2 x 16 bytes), the reference's [R][4] with channel
// 3 (8 x 16 bytes), otherwise 16 scalar loads.
struct SelLoads {
    uint4 raw[8];
    uint32_t sv[16];
    float xi;
    int kind;   // 0: stride 1, 1: stride 4 channel 3, 2: scalar
};

__device__ __forceinline__ void select_load(const WalkDesc& d, int i0, int ni, bool x_lds, SelLoads& L)
{
    const int tid = threadIdx.x;
    L.xi = 0.0f;
    const int i = i0 + min(tid, ni - 1);   // threads past the slice re-read its last input
    const int r0 = i * 16;
    const uint16_t* base = d.stats + (size_t)i0 * 16 * d.stats_stride;
    const bool aligned = (((uintptr_t)base) & 15) == 0 && (d.rows & 15) == 0;
    if (!x_lds) L.xi = d.x[i];
    const uint16_t* st = d.stats + (size_t)r0 * d.stats_stride;
    if (aligned && d.stats_stride == 1) {
        L.kind = 0;
        const uint4* p4 = reinterpret_cast<const uint4*>(st);
        L.raw[0] = p4[0];
        L.raw[1] = p4[1];
    } else if (aligned && d.stats_stride == 4 && d.stats_channel == 3) {
        L.kind = 1;
        const uint4* p4 = reinterpret_cast<const uint4*>(st);
#pragma unroll
        for (int k8 = 0; k8 < 8; k8++) L.raw[k8] = p4[k8];
    } else {
        L.kind = 2;
#pragma unroll
        for (int kk = 0; kk < 16; kk++) {
            const int rr = min(r0 + kk, d.rows - 1) - r0;
            L.sv[kk] = st[(size_t)rr * d.stats_stride + d.stats_channel];
        }
    }
}

// The selection of slice p given its loads (prepareDispatch,
// bucketMul.cl:351-386): a row is selected iff 1e5 * |x * stat| >= cutoff,
// the same fp32 operations as the dispatch kernel, so the selected set is
// the same.  A block scan compacts the selected rows in ascending order into
// s_row (slice-local ids input*16 + rank); s_x[i] = x[i0 + i] (with x_lds it
// already holds them, written before a barrier).  Ends with a barrier;
// returns the number of selected rows, which the tile-0 workgroup of the
// slice also stores in slice_count[p].
template <int NT>
__device__ __forceinline__ uint32_t select_finish(const WalkDesc& d, float cutoff, int p, int t, int i0, int ni,
                                                  const SelLoads& L, uint16_t* s_row, float* s_x, uint32_t* s_wsum,
                                                  bool x_lds)
{
#pragma clang fp contract(off)
    constexpr int NW = NT / 64;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    float xi = L.xi;
    uint32_t mask = 0;
    if (tid < ni) {
        if (x_lds) xi = s_x[tid];
        uint32_t sv[16];
        if (L.kind == 0) {
            const uint32_t ww[8] = {L.raw[0].x, L.raw[0].y, L.raw[0].z, L.raw[0].w,
                                    L.raw[1].x, L.raw[1].y, L.raw[1].z, L.raw[1].w};
#pragma unroll
            for (int kk = 0; kk < 16; kk++) sv[kk] = (ww[kk >> 1] >> ((kk & 1) * 16)) & 0xffffu;
        } else if (L.kind == 1) {
#pragma unroll
            for (int k8 = 0; k8 < 8; k8++) {
                sv[2 * k8] = L.raw[k8].y >> 16;       // row 2*k8, channel 3
                sv[2 * k8 + 1] = L.raw[k8].w >> 16;   // row 2*k8+1, channel 3
            }
        } else {
#pragma unroll
            for (int kk = 0; kk < 16; kk++) sv[kk] = L.sv[kk];
        }
        const int r0 = (i0 + tid) * 16;
#pragma unroll
        for (int kk = 0; kk < 16; kk++) {
            const float avg = h2f(sv[kk]);
            const float prod = __fmul_rn(xi, avg);
            const float imp = __fmul_rn(kScale, fabsf(prod));
            if (imp >= cutoff && r0 + kk < d.rows) mask |= 1u << kk;   // bucketMul.cl:380
        }
    }
    const uint32_t cnt = (uint32_t)__popc(mask);
    const uint32_t incl = (uint32_t)wave_incl_sum((int)cnt);
    if (lane == 63) s_wsum[wave] = incl;
    if (!x_lds) s_x[tid] = tid < ni ? xi : 0.0f;
    __syncthreads();
    uint32_t off = incl - cnt;
    uint32_t n_sel = 0;
    for (int i = 0; i < NW; i++) {
        if (i < wave) off += s_wsum[i];
        n_sel += s_wsum[i];
    }
    while (mask) {
        const int kk = __ffs(mask) - 1;
        mask &= mask - 1;
        s_row[off++] = (uint16_t)(tid * 16 + kk);
    }
    __syncthreads();
    if (t == 0 && tid == 0) d.slice_count[p] = n_sel;
    return n_sel;
}

template <int NT>
__device__ uint32_t select_slice(const WalkDesc& d, float cutoff, int p, int t, int i0, int ni, uint16_t* s_row,
                                 float* s_x, uint32_t* s_wsum)
{
    SelLoads L;
    select_load(d, i0, ni, false, L);
    return select_finish<NT>(d, cutoff, p, t, i0, ni, L, s_row, s_x, s_wsum, false);
}

template <int VEC, typename Acc, int NW, int UNR>
__global__ __launch_bounds__(64 * NW) void k_walk(WalkArgs a)
{
#pragma clang fp contract(off)
    constexpr int NT = 64 * NW;
    constexpr int NJ = 64 / VEC, NQ = VEC, TW = 64;
    constexpr int PER = 16 * VEC * 64;         // accumulators per wave
    constexpr int STRIDE = NW * NQ;            // rows per workgroup instruction
    __shared__ Acc acc[NW * PER];
    __shared__ uint16_t s_row[NT * 16];        // selected rows, slice-local (input*16 + rank)
    __shared__ float s_x[NT];
    __shared__ uint32_t s_wsum[NW];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int b = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    int k = 0;
    for (int i = 1; i < a.n; i++)
        if (b >= a.d[i].block_base) k = i;
    const WalkDesc& d = a.d[k];
    const int w = b - d.block_base;
    const int p = w / d.T;
    const int t = w - p * d.T;

    Acc* my = acc + wave * PER + lane;
#pragma unroll
    for (int i = 0; i < 16 * VEC; i++) my[i * 64] = (Acc)0;

    // ---- selection of the slice's rows
    const int i0 = p * d.IPS;
    const int ni = min(d.IPS, d.n_in - i0);
    const uint32_t n_sel = select_slice<NT>(d, *d.cutoff, p, t, i0, ni, s_row, s_x, s_wsum);

    // ---- walk of the selected rows
    const int q = lane / NJ;
    const int j = lane - q * NJ;
    const int col0 = t * TW + j * VEC;
    // Lanes past the last column read column 0 and add zeros.
    const int colc = col0 < d.C ? col0 : 0;
    const float xmask = col0 < d.C ? 1.0f : 0.0f;
    using LT = typename VecLoad<VEC>::T;
    const uint16_t* wb = d.W + (size_t)i0 * 16 * d.C + colc;
    const int ns = (int)n_sel;
    // batch k: the wave's rows base_k + q + u*STRIDE, u < UNR; the loads of
    // batch k+1 are issued before the accumulation of batch k
    int rl[UNR];
    float xl[UNR];
    LT v[UNR];
    auto issue = [&](int base) {
#pragma unroll
        for (int u = 0; u < UNR; u++) rl[u] = s_row[min(base + q + u * STRIDE, ns - 1)];
#pragma unroll
        for (int u = 0; u < UNR; u++) xl[u] = s_x[rl[u] >> 4];
#pragma unroll
        for (int u = 0; u < UNR; u++) v[u] = *reinterpret_cast<const LT*>(wb + (size_t)rl[u] * d.C);
    };
    const int first = wave * NQ;
    if (first < ns) issue(first);
    for (int base = first; base < ns; base += STRIDE * UNR) {
        LT vc[UNR];
        Acc xc[UNR];
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            vc[u] = v[u];
            xc[u] = (Acc)(base + q + u * STRIDE < ns ? xl[u] * xmask : 0.0f);
        }
        if (base + STRIDE * UNR < ns) issue(base + STRIDE * UNR);
        // keep the next batch's loads ahead of this batch's accumulation
        asm volatile("" ::: "memory");
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            uint32_t words[(VEC + 1) / 2];
            VecLoad<VEC>::split(vc[u], words);
            int ad[VEC];
            Acc wv[VEC], old[VEC];
#pragma unroll
            for (int e = 0; e < VEC; e++) {
                const uint32_t h = (words[e >> 1] >> ((e & 1) * 16)) & 0xffffu;
                ad[e] = ((int)(h & 15u) * VEC + e) * 64;
                wv[e] = (Acc)h2f(h);
            }
#pragma unroll
            for (int e = 0; e < VEC; e++) old[e] = my[ad[e]];
#pragma unroll
            for (int e = 0; e < VEC; e++) my[ad[e]] = walk_acc<Acc>(xc[u], wv[e], old[e]);
        }
    }
    __syncthreads();
    // ---- flush.  Thread -> (pos, e, jj) with jj fastest, so the reads of the
    // NW*NQ private copies are lane-contiguous; the sums go through a padded
    // staging copy (one pad per 32 entries) into output order col*16 + pos
    // (bucketMul.cl:442-445), written as one contiguous run of the slice's
    // partial row.
    constexpr int NOUT = TW * 16;
    constexpr int OPT = NOUT / NT;             // outputs per thread
    static_assert(NOUT % NT == 0 && NW * PER >= NOUT + NOUT / 32, "flush staging does not fit");
    Acc sum[OPT];
#pragma unroll
    for (int k2 = 0; k2 < OPT; k2++) {
        const int idx = tid + k2 * NT;
        const int jj = idx % NJ;
        const int pe = idx / NJ;               // pos*VEC + e
        const int ai = pe * 64 + jj;
        Acc s2 = (Acc)0;
        for (int ww = 0; ww < NW; ww++)
#pragma unroll
            for (int qq = 0; qq < NQ; qq++) s2 += acc[ww * PER + ai + qq * NJ];
        sum[k2] = s2;
    }
    __syncthreads();
    Acc* stage = acc;                          // NOUT + NOUT/32 entries, reused
#pragma unroll
    for (int k2 = 0; k2 < OPT; k2++) {
        const int idx = tid + k2 * NT;
        const int jj = idx % NJ;
        const int pe = idx / NJ;
        const int pos = pe / VEC, e = pe - pos * VEC;
        const int o = (jj * VEC + e) * 16 + pos;
        stage[o + (o >> 5)] = sum[k2];
    }
    __syncthreads();
    Acc* prow = reinterpret_cast<Acc*>(d.part) + (size_t)p * d.C * 16 + (size_t)t * NOUT;
    const int nout = min(NOUT, (d.C - t * TW) * 16);
    for (int o = tid; o < nout; o += NT) prow[o] = stage[o + (o >> 5)];
}

// Selection + walk with fp64 accumulation in wave-private LDS tiles.
// Workgroup (input slice p, column tile t) owns the inputs [p*IPS,
// (p+1)*IPS) and the 128 columns [128t, 128t + 128).
//
// Walk: lane = q*16 + j reads 16 bytes (8 columns 8j..8j+7) of row q of a
// group of 4 selected rows, so one load instruction fetches the 256-byte tile
// segments of 4 rows.  Wave w takes the groups w, w + NW, w + 2NW, ...  Each
// packed weight is added, as the exact fp64 product x * w, to the wave's own
// accumulator of its output (column c, position bits & 15) with a
// non-returning LDS fp64 atomic add (bucketMul.cl:430-445 adds the fp32
// product with a plain += per work-item).  Accumulator slot of (8j+e, pos) is
// pos*128 + e*16 + j: for one element e the 16 lanes of a row hit 16
// different bank pairs whatever their positions.  A wave's atomics are
// applied in instruction order and, within an instruction, in lane order, so
// the sums do not depend on scheduling; the flush adds the NW wave tiles in
// wave order.  Rows past the end of the list re-read the last selected row
// with x = 0, so every load of a batch is unconditional.
template <int NW, int UNR>
__global__ __launch_bounds__(64 * NW) void k_walk64(WalkArgs a)
{
#pragma clang fp contract(off)
    constexpr int NT = 64 * NW;
    constexpr int TW = 128;
    constexpr int SLOTS = TW * 16;             // accumulators per wave
    constexpr int GSTRIDE = NW * UNR;          // groups per workgroup batch
    static_assert(NT == kCutThreads || NT == 2 * kCutThreads, "4 or 8 waves");
    // the norm and the search hold x[16*tid ..] in the first kCutThreads threads
    __shared__ double acc[NW * SLOTS];
    __shared__ __align__(16) uint16_t s_row[NT * 16];
    __shared__ float s_x[NT];
    __shared__ uint32_t s_wsum[NW];
    __shared__ __align__(16) float s_red[260];
    __shared__ __align__(16) int s_cnt[32];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int b = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    int k = 0;
    for (int i = 1; i < a.n; i++)
        if (b >= a.d[i].block_base) k = i;
    const WalkDesc& d = a.d[k];
    const int w = b - d.block_base;
    const int p = w / d.T;
    const int t = w - p * d.T;

    // every global load of the prologue is issued before any of it is used
    const int i0 = p * d.IPS;
    const int ni = min(d.IPS, d.n_in - i0);
    const bool x_lds = d.in_mode == kInNorm;
    const bool cut_thread = tid < kCutThreads;
    float xs[kCutVPT];
    uint4 pr[2], gr[2];
#pragma unroll
    for (int k2 = 0; k2 < kCutVPT; k2++) xs[k2] = 0.0f;
    pr[0] = pr[1] = gr[0] = gr[1] = make_uint4(0u, 0u, 0u, 0u);
    float cutoff = 0.0f;
    if (d.in_mode == kInCutoff) {
        cutoff = *d.cutoff;
    } else if (cut_thread) {
        load_probes(d.probes, pr);
        load16(d.in_mode == kInNorm ? d.h : d.x, xs);
        if (d.in_mode == kInNorm) {
            gr[0] = reinterpret_cast<const uint4*>(d.gain + tid * kCutVPT)[0];
            gr[1] = reinterpret_cast<const uint4*>(d.gain + tid * kCutVPT)[1];
        }
    }
    SelLoads L;
    select_load(d, i0, ni, x_lds, L);
    {
        double2* z = reinterpret_cast<double2*>(acc + wave * SLOTS);
#pragma unroll
        for (int i = 0; i < SLOTS / 128; i++) z[i * 64 + lane] = make_double2(0.0, 0.0);
    }
    if (d.in_mode != kInCutoff) {
        if (d.in_mode == kInNorm) {
            block_rmsnorm4096(xs, gr, d.eps, reinterpret_cast<float*>(s_row));
            if (w == 0 && k == 0 && cut_thread) {
                float4* xo = reinterpret_cast<float4*>(d.x + tid * kCutVPT);
#pragma unroll
                for (int k4 = 0; k4 < 4; k4++)
                    xo[k4] = make_float4(xs[4 * k4], xs[4 * k4 + 1], xs[4 * k4 + 2], xs[4 * k4 + 3]);
            }
            // the slice's inputs for the selection (4096 inputs: all in xs)
#pragma unroll
            for (int k2 = 0; k2 < kCutVPT; k2++) {
                const int i = tid * kCutVPT + k2 - i0;
                if (cut_thread && i >= 0 && i < ni) s_x[i] = xs[k2];
            }
        }
        // s_row is free until the selection: it holds the search's bracket values
        static_assert(sizeof(uint16_t) * NT * 16 >= sizeof(float) * kCandCap, "s_row too small");
        cutoff = block_cutoff_x<NW>(xs, pr, d.quantile, s_red, s_cnt, reinterpret_cast<float*>(s_row));
        if (w == 0 && tid == 0) d.cutoff[0] = cutoff;
    }
    const int ns = (int)select_finish<NT>(d, cutoff, p, t, i0, ni, L, s_row, s_x, s_wsum, x_lds);

    const int j = lane & 15;
    const int q = lane >> 4;
    const int col0 = t * TW + j * 8;
    if (col0 < d.C) {   // C % 8 == 0: the lane's 8 columns are all in range
        const uint16_t* wb = d.W + (size_t)i0 * 16 * d.C + col0;
        double* accw = acc + wave * SLOTS + j;
        const int ng = (ns + 3) >> 2;
        int rl[UNR];
        float xl[UNR];
        uint4 v[UNR];
        auto issue = [&](int g0) {
#pragma unroll
            for (int u = 0; u < UNR; u++) {
                const int idx = (g0 + u * NW) * 4 + q;
                rl[u] = s_row[min(idx, ns - 1)];
                xl[u] = idx < ns ? 1.0f : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < UNR; u++) xl[u] *= s_x[rl[u] >> 4];
#pragma unroll
            for (int u = 0; u < UNR; u++)
                v[u] = *reinterpret_cast<const uint4*>(wb + (size_t)rl[u] * d.C);
        };
        if (wave < ng) issue(wave);
        for (int g0 = wave; g0 < ng; g0 += GSTRIDE) {
            uint4 vc[UNR];
            double xc[UNR];
#pragma unroll
            for (int u = 0; u < UNR; u++) {
                vc[u] = v[u];
                xc[u] = (double)xl[u];
            }
            if (g0 + GSTRIDE < ng) issue(g0 + GSTRIDE);
            asm volatile("" ::: "memory");
#pragma unroll
            for (int u = 0; u < UNR; u++) {
                const uint32_t words[4] = {vc[u].x, vc[u].y, vc[u].z, vc[u].w};
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const uint32_t h = (words[e >> 1] >> ((e & 1) * 16)) & 0xffffu;
                    const double wv = (double)h2f(h);
                    // position bits by one bit-field extract (kept as one
                    // instruction), then one shift-add into the address
                    uint32_t pos;
                    asm("v_bfe_u32 %0, %1, %2, 4" : "=v"(pos) : "v"(words[e >> 1]), "i"((e & 1) * 16));
                    atomicAdd(accw + pos * TW + e * 16, xc[u] * wv);
                }
            }
        }
    }
    __syncthreads();
    // ---- flush: thread -> slots tid + k*NT (slot order, conflict-free), sum
    // of the NW wave tiles in wave order, through a padded staging copy (one
    // pad per 128 entries) into output order col*16 + pos (bucketMul.cl:
    // 442-445), written as one contiguous run of the slice's partial row.
    constexpr int OPT = SLOTS / NT;
    static_assert(SLOTS % NT == 0 && NW * SLOTS >= SLOTS + SLOTS / 128, "flush staging does not fit");
    double sum[OPT];
#pragma unroll
    for (int k2 = 0; k2 < OPT; k2++) {
        const int sl = tid + k2 * NT;
        double s2 = acc[sl];
#pragma unroll
        for (int ww = 1; ww < NW; ww++) s2 += acc[ww * SLOTS + sl];
        sum[k2] = s2;
    }
    __syncthreads();
#pragma unroll
    for (int k2 = 0; k2 < OPT; k2++) {
        const int sl = tid + k2 * NT;
        const int pos = sl >> 7, e = (sl >> 4) & 7, jj = sl & 15;
        const int o = (jj * 8 + e) * 16 + pos;
        acc[o + (o >> 7)] = sum[k2];
    }
    __syncthreads();
    double* prow = reinterpret_cast<double*>(d.part) + (size_t)p * d.C * 16 + (size_t)t * SLOTS;
    const int nout = min(SLOTS, (d.C - t * TW) * 16);
    for (int o = tid; o < nout; o += NT) prow[o] = acc[o + (o >> 7)];
}

// y[o] = sum over the P row slices of part[p][o] (bucketIntegrate,
// bucketMul.cl:453-497, sums 64 fixed slices), then the epilogue of the op
// that consumes y.  Workgroup = 128 outputs; thread (ol, pg) sums outputs
// 4ol..4ol+3 over slices pg, pg+8, ...; the 8 group sums are added in group
// order.  The order is fixed, so y is the same on every run.  Block 0 of each
// matrix adds up the per-slice selected-row counts.
struct ReduceDesc {
    const void* part;              // [P][m] of Acc
    float* y;
    const uint32_t* slice_count;   // [P]
    uint32_t* count;               // total selected rows
    const void* part2;             // kEpSilu: the up projection's partials, counts and output
    float* y2;
    const uint32_t* slice_count2;
    uint32_t* count2;
    float* out;
    const float* table;            // RoPE table [max_ctx][hd/2][2]
    const int* pos;
    uint16_t* cache;               // fp16 rows [max_ctx][m]
    int P, P2, m, C;
    int ep;
    int max_ctx;
    int block_base;
};

struct ReduceArgs {
    ReduceDesc d[kMaxMulti];
    int n;
    unsigned long long* counters;  // walk bytes, rows, matrices (null: no counting)
};

constexpr int kRedThreads = 256;
constexpr int kRedHead = 128;    // the RoPE epilogues need a head of 128 outputs in one workgroup

// Workgroup of OUT outputs: thread (ol, pg) sums outputs 4ol..4ol+3 over the
// slices pg, pg + G, ... (G = 256 / (OUT/4) slice groups) in slice order,
// U loads at a time; the G group sums are then added in group order by
// threads 0..OUT-1.
template <typename Acc, int OUT>
struct RedShape {
    static constexpr int QUADS = OUT / 4;
    static constexpr int G = kRedThreads / QUADS;
    static constexpr int U = OUT == kRedHead ? 8 : 4;
};

template <typename Acc, int G, int U>
__device__ __forceinline__ void slice_loads(const Acc* __restrict__ part, int P, int m, int o, int p0, Acc (&r)[U][4])
{
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int p = min(p0 + u * G, P - 1);
#pragma unroll
        for (int i = 0; i < 4; i++) r[u][i] = part[(size_t)p * m + o + i];
    }
}

template <typename Acc, int G, int U>
__device__ __forceinline__ void slice_adds(int P, int p0, const Acc (&r)[U][4], Acc (&s)[4])
{
#pragma unroll
    for (int u = 0; u < U; u++)
        if (p0 + u * G < P)
#pragma unroll
            for (int i = 0; i < 4; i++) s[i] += r[u][i];
}

template <typename Acc, int G, int U>
__device__ __forceinline__ void thread_sums(const Acc* __restrict__ part, int P, int m, int o, int pg, Acc (&s)[4])
{
    for (int p0 = pg; p0 < P; p0 += U * G) {
        Acc r[U][4];
        slice_loads<Acc, G, U>(part, P, m, o, p0, r);
        slice_adds<Acc, G, U>(P, p0, r, s);
    }
}

// the G group sums of output tid (< OUT) in group order
template <typename Acc, int OUT>
__device__ __forceinline__ Acc group_total(const Acc (*red)[OUT])
{
    constexpr int G = RedShape<Acc, OUT>::G;
    const int tid = threadIdx.x;
    Acc t = (Acc)0;
    if (tid < OUT) {
        t = red[0][tid];
#pragma unroll
        for (int g = 1; g < G; g++) t += red[g][tid];
    }
    return t;
}

template <typename Acc, int OUT>
__device__ __forceinline__ Acc group_sums(const Acc* __restrict__ part, int P, int m, int o, int pg,
                                          Acc (*red)[OUT], int ol)
{
    using S = RedShape<Acc, OUT>;
    Acc s[4] = {(Acc)0, (Acc)0, (Acc)0, (Acc)0};
    if (o < m) thread_sums<Acc, S::G, S::U>(part, P, m, o, pg, s);
#pragma unroll
    for (int i = 0; i < 4; i++) red[pg][ol * 4 + i] = s[i];
    __syncthreads();
    return group_total<Acc, OUT>(red);
}

// two matrices of the same output size at once (the gate and up
// projections): when both fit one batch of loads, all loads of both are
// issued together
template <typename Acc, int OUT>
__device__ __forceinline__ void group_sums2(const Acc* __restrict__ part, int P, const Acc* __restrict__ part2,
                                            int P2, int m, int o, int pg, Acc (*red)[OUT], Acc (*red2)[OUT],
                                            int ol, Acc& t1, Acc& t2)
{
    using S = RedShape<Acc, OUT>;
    Acc s[4] = {(Acc)0, (Acc)0, (Acc)0, (Acc)0};
    Acc s2[4] = {(Acc)0, (Acc)0, (Acc)0, (Acc)0};
    if (o < m) {
        if (P <= S::U * S::G && P2 <= S::U * S::G) {
            Acc r[S::U][4], r2[S::U][4];
            slice_loads<Acc, S::G, S::U>(part, P, m, o, pg, r);
            slice_loads<Acc, S::G, S::U>(part2, P2, m, o, pg, r2);
            slice_adds<Acc, S::G, S::U>(P, pg, r, s);
            slice_adds<Acc, S::G, S::U>(P2, pg, r2, s2);
        } else {
            thread_sums<Acc, S::G, S::U>(part, P, m, o, pg, s);
            thread_sums<Acc, S::G, S::U>(part2, P2, m, o, pg, s2);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        red[pg][ol * 4 + i] = s[i];
        red2[pg][ol * 4 + i] = s2[i];
    }
    __syncthreads();
    t1 = group_total<Acc, OUT>(red);
    t2 = group_total<Acc, OUT>(red2);
}

// total selected rows of a matrix (by one wave, no barrier) into count and
// the context's counters
__device__ void sum_counts(const uint32_t* __restrict__ sc, int P, int C, uint32_t* count,
                           unsigned long long* counters)
{
    const int lane = threadIdx.x & 63;
    unsigned long long v = 0;
    for (int p = lane; p < P; p += 64) v += sc[p];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    if (lane == 0) {
        count[0] = (uint32_t)v;
        atomicAdd(counters + 0, v * (unsigned long long)C * 2ull);
        atomicAdd(counters + 1, v);
        atomicAdd(counters + 2, 1ull);
    }
}

template <typename Acc, int OUT>
__global__ __launch_bounds__(kRedThreads) void k_reduce(ReduceArgs a)
{
#pragma clang fp contract(off)
    using S = RedShape<Acc, OUT>;
    __shared__ Acc red[S::G][OUT];
    __shared__ Acc red2[S::G][OUT];
    __shared__ float sy[OUT];
    const int b = (int)blockIdx.x;
    int k = 0;
    for (int i = 1; i < a.n; i++)
        if (b >= a.d[i].block_base) k = i;
    const ReduceDesc& d = a.d[k];
    const int lb = b - d.block_base;
    const int o0 = lb * OUT;
    const int tid = threadIdx.x;
    const int ol = tid % S::QUADS, pg = tid / S::QUADS;
    const int o = o0 + ol * 4;   // m is a multiple of 16: o..o+3 are in range together
    if (a.counters && lb == 0 && tid >= kRedThreads - 64) sum_counts(d.slice_count, d.P, d.C, d.count, a.counters);
    if (a.counters && lb == 0 && d.ep == kEpSilu && tid >= kRedThreads - 128 && tid < kRedThreads - 64)
        sum_counts(d.slice_count2, d.P2, d.C, d.count2, a.counters);
    const int oo = o0 + tid;
    const bool in = tid < OUT && oo < d.m;
    // the epilogue's own loads go out with the partial loads (a RoPE
    // epilogue comes with OUT = kRedHead)
    const bool rope = OUT == kRedHead && (d.ep == kEpRopeQ || d.ep == kEpRopeK);
    const int pos = rope || d.ep == kEpV ? *d.pos : 0;
    const bool pos_ok = pos >= 0 && pos < d.max_ctx;
    float rc = 0.0f, rsn = 0.0f, resid = 0.0f;
    if (rope && in && pos_ok) {
        const int fi = tid < OUT / 2 ? tid : tid - OUT / 2;
        rc = d.table[(size_t)pos * OUT + 2 * fi];
        rsn = d.table[(size_t)pos * OUT + 2 * fi + 1];
    }
    if (d.ep == kEpResid && in) resid = d.out[oo];
    if (d.ep == kEpSilu) {
        Acc t1, t2;
        group_sums2<Acc, OUT>(reinterpret_cast<const Acc*>(d.part), d.P, reinterpret_cast<const Acc*>(d.part2),
                              d.P2, d.m, o, pg, red, red2, ol, t1, t2);
        const float yv = (float)t1, uv = (float)t2;
        if (in) {
            d.y[oo] = yv;
            d.y2[oo] = uv;
            const double x1 = (double)yv;
            d.out[oo] = (float)((double)uv * x1 / (1.0 + exp(-x1)));
        }
        return;
    }
    const float yv = (float)group_sums<Acc, OUT>(reinterpret_cast<const Acc*>(d.part), d.P, d.m, o, pg, red, ol);
    if (in) d.y[oo] = yv;
    if (d.ep == kEpResid) {
        if (in) d.out[oo] = __fadd_rn(resid, yv);
    } else if (d.ep != kEpStore) {
        if (d.ep == kEpV) {
            if (in && pos_ok) d.cache[(size_t)pos * d.m + oo] = __half_as_ushort(__float2half_rn(yv));
        } else if (rope) {
            if (tid < OUT) sy[tid] = yv;
            __syncthreads();
            if (in && pos_ok) {
                const float r = rope_cs(sy, tid, OUT / 2, rc, rsn);
                if (d.ep == kEpRopeQ) d.out[oo] = r;
                else d.cache[(size_t)pos * d.m + oo] = __half_as_ushort(__float2half_rn(r));
            }
        }
    }
}

// ------------------------------------------------------------------ host ---

int quantile_of(float effort) { return (int)((double)(kProbes - 1) * (1.0 - (double)effort)); }

// Expected fraction of selected rows (N(0,1) inputs, N(0, 0.02^2) weights),
// used only to size the walk grid.
static double est_fraction(float effort)
{
    static const double e[] = {0.0, 0.05, 0.125, 0.25, 0.5, 1.0};
    static const double f[] = {0.05, 0.102, 0.158, 0.236, 0.396, 1.0};
    double x = std::min(1.0, std::max(0.0, (double)effort));
    for (int i = 1; i < 6; i++)
        if (x <= e[i]) return f[i - 1] + (f[i] - f[i - 1]) * (x - e[i - 1]) / (e[i] - e[i - 1]);
    return 1.0;
}

double est_rows(int rows, float effort) { return std::max(1.0, rows * est_fraction(effort)); }

// Walk launch shapes: a launch whose expected weight bytes are below
// kWalkWideBytes uses 4 waves per workgroup and 16 rows in flight per lane
// (more waves per slice: these launches are latency bound), a larger one 2
// waves and 8 rows (more workgroups in flight).  Each wave holds 16 KB of
// private accumulators (fp32: 4 columns per lane; fp64: 2); a slice holds at
// most 64 inputs per wave.  A launch gets about one workgroup per
// kWalkWgBytes of expected weight bytes, at least kWalkMinWgs.
#ifndef IAM_WALK_WIDE_BYTES
#define IAM_WALK_WIDE_BYTES 40e6
#endif
#ifndef IAM_WALK_WG_BYTES
#define IAM_WALK_WG_BYTES 98304.0
#endif
#ifndef IAM_WALK_MIN_WGS
#define IAM_WALK_MIN_WGS 256.0
#endif
#ifndef IAM_WALK_SMALL_NW
#define IAM_WALK_SMALL_NW 4
#endif
#ifndef IAM_WALK_SMALL_UNR
#define IAM_WALK_SMALL_UNR 16
#endif
#ifndef IAM_WALK_BIG_NW
#define IAM_WALK_BIG_NW 2
#endif
#ifndef IAM_WALK_BIG_UNR
#define IAM_WALK_BIG_UNR 8
#endif
constexpr double kWalkWideBytes = IAM_WALK_WIDE_BYTES;
constexpr double kWalkWgBytes = IAM_WALK_WG_BYTES;
constexpr double kWalkMinWgs = IAM_WALK_MIN_WGS;
constexpr double kWalkMaxWgs = 3072.0;

// k_walk64 launch shapes: below IAM_W64_WIDE_BYTES of expected weight bytes
// 4 waves per workgroup and about one workgroup per IAM_W64_WG_BYTES (at
// least 256; two fit a CU); above it 8 waves and one workgroup per CU
// (IAM_W64_WIDE_WGS), so that no CU holds more work than another.
#ifndef IAM_W64_UNR
#define IAM_W64_UNR 4
#endif
#ifndef IAM_W64_WG_BYTES
#define IAM_W64_WG_BYTES 131072.0
#endif
#ifndef IAM_W64_WIDE_BYTES
#define IAM_W64_WIDE_BYTES 40e6
#endif
#ifndef IAM_W64_WIDE_WGS
#define IAM_W64_WIDE_WGS 256
#endif

// 8: the fp64 walk with 16-byte loads and 128-column tiles (k_walk64);
// otherwise the columns per lane load of k_walk.
static int vec_of(int C, bool acc64)
{
    if (acc64 && C % 8 == 0) return 8;
    if (C % 4 == 0 && !acc64) return 4;
    if (C % 2 == 0) return 2;
    return 1;
}

// Slices per matrix (only the performance depends on them): the launch's
// workgroups are shared by the matrices in proportion to their bytes.
void plan_walk(int n, const MatOp* ops, float effort, bool acc64, WalkPlan* plan)
{
    double bytes[kMaxMulti], tot = 0;
    bool all64 = true;
    for (int i = 0; i < n; i++) {
        const iam_bucket_matrix& M = ops[i].mat;
        WalkPlan& pl = plan[i];
        pl.V = vec_of(M.bucket_cols, acc64);
        all64 = all64 && pl.V == 8;
        const int tw = pl.V == 8 ? 128 : 64;
        pl.T = (M.bucket_cols + tw - 1) / tw;
        pl.n_in = std::min((M.expert_rows + 15) / 16, ops[i].in_size);
        // the cost of a row is its tiles' width: a k_walk64 workgroup spends
        // the same on a 64-column matrix's half-empty tile as on a full one
        bytes[i] = est_rows(pl.n_in * 16, effort) * (pl.V == 8 ? pl.T * tw : M.bucket_cols) * 2.0;
        tot += bytes[i];
    }
    const bool wide64 = all64 && tot >= IAM_W64_WIDE_BYTES;
    const int nw = all64 ? (wide64 ? 8 : 4) : tot < kWalkWideBytes ? IAM_WALK_SMALL_NW : IAM_WALK_BIG_NW;
    const double wg_bytes = all64 ? IAM_W64_WG_BYTES : kWalkWgBytes;
    double target = std::min(kWalkMaxWgs, std::max(kWalkMinWgs, tot / wg_bytes));
    const bool fit = wide64;   // at most target workgroups
    if (wide64) target = IAM_W64_WIDE_WGS;
    for (int i = 0; i < n; i++) {
        WalkPlan& pl = plan[i];
        pl.NW = nw;
        const double wgs = tot > 0 ? target * bytes[i] / tot : target / n;
        const int slices = std::max(1, fit ? (int)std::floor(wgs / pl.T + 1e-9) : (int)std::lround(wgs / pl.T));
        pl.IPS = std::min(64 * pl.NW, std::max(1, (pl.n_in + slices - 1) / slices));
        pl.P = (pl.n_in + pl.IPS - 1) / pl.IPS;
    }
}

// Validate the n matrix ops and record their selection problems in slots
// 0..n-1; fills the cutoff launch arguments.
static int record_slots(Ctx* c, int n, const MatOp* ops, int expert_no, float effort, CutoffArgs& args)
{
    IAM_REQUIRE(n >= 1 && n <= kMaxMulti, "bucketmul: 1..3 matrices per launch");
    IAM_REQUIRE(!std::isnan(effort), "bucketmul: effort is NaN");
    IAM_REQUIRE(expert_no >= 0, "bucketmul: negative expert_no");
    args.n = n;
    const int qv = quantile_of(effort);
    for (int i = 0; i < n; i++) {
        const iam_bucket_matrix& M = ops[i].mat;
        IAM_REQUIRE(ops[i].x && M.stats && M.probes, "bucketmul: null x/stats/probes");
        IAM_REQUIRE(M.expert_rows > 0 && M.bucket_cols > 0, "bucketmul: empty matrix");
        IAM_REQUIRE(ops[i].in_size > 0, "bucketmul: in_size must be positive");
        IAM_REQUIRE(M.stats_stride >= 1 && M.stats_channel >= 0 && M.stats_channel < M.stats_stride,
                    "bucketmul: bad stats stride/channel");
        IAM_REQUIRE(((uintptr_t)ops[i].x & 15) == 0, "bucketmul: x must be 16-byte aligned");
        const uint16_t* probes = M.probes + (size_t)expert_no * kProbes;
        IAM_REQUIRE(((uintptr_t)probes & 15) == 0, "bucketmul: probes must be 16-byte aligned");
        const int inputs = (M.expert_rows + 15) / 16;
        IAM_REQUIRE((std::min(inputs, ops[i].in_size) + kChunkInputs - 1) / kChunkInputs <= kMaxChunks,
                    "bucketmul: more than 65536 inputs per expert");
        // every device range the kernels read or write must lie inside an
        // allocation of this context (the cutoff always reads x[0:4096])
        const size_t xn = std::max<size_t>(kProbes, std::min<size_t>((size_t)ops[i].in_size, (size_t)inputs));
        IAM_TRY(check_dev_range(c, ops[i].x, xn * sizeof(float), "bucketmul x"));
        IAM_TRY(check_dev_range(c, M.probes, (size_t)(expert_no + 1) * kProbes * 2, "bucketmul probes"));
        IAM_TRY(check_dev_range(c, M.stats, (size_t)(expert_no + 1) * M.expert_rows * M.stats_stride * 2,
                                "bucketmul stats"));
        IAM_TRY(ensure_slot(c, i));
        DispatchSlot& s = c->slots[i];
        s.x = ops[i].x;
        s.stats = M.stats + (size_t)expert_no * (size_t)M.expert_rows * M.stats_stride;
        s.probes = probes;
        s.stats_stride = M.stats_stride;
        s.stats_channel = M.stats_channel;
        s.rows = M.expert_rows;
        s.in_size = ops[i].in_size;
        s.bucket_cols = M.bucket_cols;
        s.expert_no = expert_no;
        s.effort = effort;
        s.valid = true;
        CutoffDesc& d = args.d[i];
        d.x = ops[i].x;
        d.probes = probes;
        d.quantile = qv;
        d.cutoff = s.cutoff;
    }
    return IAM_OK;
}

int bucketmul_dispatch(Ctx* c, int n, const MatOp* ops, int expert_no, float effort)
{
    CutoffArgs args{};
    IAM_TRY(record_slots(c, n, ops, expert_no, effort, args));
    return launch(c, "bucket_cutoff", k_cutoff, dim3(n), dim3(kCutThreads), 0, args);
}

// The selected-row list of slot i (k_dispatch), for the parity queries.
static int bucketmul_list(Ctx* c, int i)
{
    DispatchSlot& s = c->slots[i];
    const int inputs = (s.rows + 15) / 16;
    const int G = std::max(1, (std::min(inputs, s.in_size) + kChunkInputs - 1) / kChunkInputs);
    IAM_TRY(ensure_list(c, i, G));
    DispatchArgs args{};
    args.n = 1;
    DispatchDesc& d = args.d[0];
    d.x = s.x;
    d.probes = s.probes;
    d.stats = s.stats;
    d.stats_stride = s.stats_stride;
    d.stats_channel = s.stats_channel;
    d.rows = s.rows;
    d.in_size = s.in_size;
    d.quantile = quantile_of(s.effort);
    d.G = G;
    d.list = s.list;
    d.counts = s.counts;
    d.cutoff = s.cutoff;
    d.block_base = 0;
    s.G = G;
    return launch(c, "bucket_list", k_dispatch, dim3(G), dim3(kCutThreads), 0, args);
}

template <typename Acc, int NW, int UNR>
static int launch_walk_shape(Ctx* c, int vec, int blocks, const WalkArgs& args)
{
    const dim3 g(blocks), t(64 * NW);
    if constexpr (sizeof(Acc) == 4) {
        if (vec >= 4) return launch(c, "bucket_walk", k_walk<4, Acc, NW, UNR>, g, t, 0, args);
    }
    if (vec >= 2) return launch(c, "bucket_walk", k_walk<2, Acc, NW, UNR>, g, t, 0, args);
    return launch(c, "bucket_walk", k_walk<1, Acc, NW, UNR>, g, t, 0, args);
}

template <typename Acc>
static int launch_walk(Ctx* c, int nw, int vec, int blocks, const WalkArgs& args)
{
    if (nw == IAM_WALK_SMALL_NW) return launch_walk_shape<Acc, IAM_WALK_SMALL_NW, IAM_WALK_SMALL_UNR>(c, vec, blocks, args);
    return launch_walk_shape<Acc, IAM_WALK_BIG_NW, IAM_WALK_BIG_UNR>(c, vec, blocks, args);
}

// Partial sums [P][m] of the accumulator type, then the per-slice selected
// row counts [P].
static size_t partial_bytes(const WalkPlan& pl, int C, bool acc64)
{
    return (size_t)pl.P * C * 16 * (acc64 ? 8 : 4) + (size_t)pl.P * sizeof(uint32_t);
}

static uint32_t* slice_counts(const DispatchSlot& s, const WalkPlan& pl, bool acc64)
{
    return reinterpret_cast<uint32_t*>(static_cast<char*>(s.part) + (size_t)pl.P * s.bucket_cols * 16 * (acc64 ? 8 : 4));
}

int reserve_walk(Ctx* c, int n, const MatOp* ops, float effort)
{
    WalkPlan plan[kMaxMulti];
    plan_walk(n, ops, effort, c->acc64, plan);
    for (int i = 0; i < n; i++) {
        IAM_TRY(ensure_slot(c, i));
        IAM_TRY(ensure_partials(c, i, partial_bytes(plan[i], ops[i].mat.bucket_cols, c->acc64)));
    }
    return IAM_OK;
}

// Walk and reduce of slots 0..n-1 (recorded by record_slots).  in_mode is how
// the k_walk64 launches get x and the cutoff (k_walk always reads the
// cutoff of a preceding k_cutoff launch); ep (null: store y) the epilogue of
// each op, kEpSilu pairing ops 0 (gate) and 1 (up).
static int walk_and_reduce(Ctx* c, int n, const MatOp* ops, int in_mode, const float* h, const uint16_t* gain,
                           float eps, const ReduceEp* ep)
{
    IAM_REQUIRE(n >= 1 && n <= kMaxMulti, "bucketmul: 1..3 matrices per launch");
    for (int i = 0; i < n; i++) {
        const iam_bucket_matrix& M = ops[i].mat;
        const DispatchSlot& s = c->slots[i];
        IAM_REQUIRE(s.valid, "bucketmul: mul without a preceding calc_dispatch");
        IAM_REQUIRE(M.buckets && ops[i].y, "bucketmul: null buckets/y");
        IAM_REQUIRE(s.bucket_cols == M.bucket_cols && s.rows == M.expert_rows,
                    "bucketmul: mul shape differs from calc_dispatch shape");
        IAM_REQUIRE(((uintptr_t)M.buckets & 15) == 0, "bucketmul: buckets must be 16-byte aligned");
        IAM_REQUIRE(((uintptr_t)ops[i].y & 15) == 0, "bucketmul: y must be 16-byte aligned");
        IAM_TRY(check_dev_range(c, M.buckets, (size_t)(s.expert_no + 1) * M.expert_rows * M.bucket_cols * 2,
                                "bucketmul buckets"));
        IAM_TRY(check_dev_range(c, ops[i].y, (size_t)M.bucket_cols * 16 * sizeof(float), "bucketmul y"));
        IAM_REQUIRE(s.effort == c->slots[0].effort, "bucketmul: slots dispatched at different efforts");
    }
    // the walk reads x and in_size from the slots (the dispatch's inputs)
    MatOp wops[kMaxMulti];
    for (int i = 0; i < n; i++) {
        wops[i] = ops[i];
        wops[i].x = c->slots[i].x;
        wops[i].in_size = c->slots[i].in_size;
    }
    WalkPlan plan[kMaxMulti];
    plan_walk(n, wops, c->slots[0].effort, c->acc64, plan);
    for (int i = 0; i < n; i++)
        IAM_TRY(ensure_partials(c, i, partial_bytes(plan[i], ops[i].mat.bucket_cols, c->acc64)));
    const int qv = quantile_of(c->slots[0].effort);

    // walk: one launch per kernel variant (the model's matrices all share one)
    bool used[kMaxMulti] = {false, false, false};
    for (int done = 0; done < n;) {
        int vec = 0, blocks = 0, cnt = 0, nw = 0;
        WalkArgs args{};
        for (int i = 0; i < n; i++) {
            if (used[i] || (vec != 0 && plan[i].V != vec)) continue;
            vec = plan[i].V;
            nw = plan[i].NW;
            const DispatchSlot& s = c->slots[i];
            WalkDesc& d = args.d[cnt++];
            d.W = ops[i].mat.buckets + (size_t)s.expert_no * (size_t)ops[i].mat.expert_rows * ops[i].mat.bucket_cols;
            d.x = const_cast<float*>(s.x);
            d.stats = s.stats;
            d.cutoff = s.cutoff;
            d.slice_count = slice_counts(s, plan[i], c->acc64);
            d.part = s.part;
            d.h = h;
            d.gain = gain;
            d.probes = s.probes;
            d.eps = eps;
            d.quantile = qv;
            d.in_mode = vec == 8 ? in_mode : kInCutoff;
            d.stats_stride = s.stats_stride;
            d.stats_channel = s.stats_channel;
            d.rows = s.rows;
            d.n_in = plan[i].n_in;
            d.C = ops[i].mat.bucket_cols;
            d.IPS = plan[i].IPS;
            d.P = plan[i].P;
            d.T = plan[i].T;
            d.block_base = blocks;
            blocks += plan[i].P * plan[i].T;
            used[i] = true;
            done++;
        }
        args.n = cnt;
        if (vec == 8 && nw == 8)
            IAM_TRY(launch(c, "bucket_walk", k_walk64<8, IAM_W64_UNR>, dim3(blocks), dim3(512), 0, args));
        else if (vec == 8)
            IAM_TRY(launch(c, "bucket_walk", k_walk64<4, IAM_W64_UNR>, dim3(blocks), dim3(256), 0, args));
        else
            IAM_TRY(c->acc64 ? launch_walk<double>(c, nw, vec, blocks, args)
                             : launch_walk<float>(c, nw, vec, blocks, args));
    }
    // fixed-order sum of the slices into y, with the epilogue
    ReduceArgs ra{};
    ra.counters = c->counting ? c->counters : nullptr;   // null: no counting
    for (int i = 0; i < n; i++) c->slots[i].counted = c->counting;
    int rblocks = 0, nd = 0;
    int rout = 32;
    for (int i = 0; ep && i < n; i++)
        if (ep[i].ep == kEpRopeQ || ep[i].ep == kEpRopeK) rout = kRedHead;
    for (int i = 0; i < n; i++) {
        const DispatchSlot& s = c->slots[i];
        ReduceDesc& d = ra.d[nd++];
        d.part = s.part;
        d.y = ops[i].y;
        d.slice_count = slice_counts(s, plan[i], c->acc64);
        d.count = s.count;
        d.P = plan[i].P;
        d.m = ops[i].mat.bucket_cols * 16;
        d.C = ops[i].mat.bucket_cols;
        d.ep = ep ? ep[i].ep : kEpStore;
        if (ep) {
            d.out = ep[i].out;
            d.table = ep[i].table;
            d.pos = ep[i].pos;
            d.max_ctx = ep[i].max_ctx;
            d.cache = ep[i].cache;
        }
        if (d.ep == kEpSilu) {
            IAM_REQUIRE(i == 0 && n == 2 && ops[1].mat.bucket_cols == ops[0].mat.bucket_cols,
                        "bucketmul: the SiLU epilogue pairs two matrices of one shape");
            const DispatchSlot& s2 = c->slots[1];
            d.part2 = s2.part;
            d.y2 = ops[1].y;
            d.slice_count2 = slice_counts(s2, plan[1], c->acc64);
            d.count2 = s2.count;
            d.P2 = plan[1].P;
            i = n;   // the pair is one descriptor
        }
        d.block_base = rblocks;
        rblocks += (d.m + rout - 1) / rout;
    }
    ra.n = nd;
    // a head of 128 outputs per workgroup for RoPE, else 32 outputs (more
    // workgroups, fewer partials per thread)
    if (rout == kRedHead)
        return c->acc64 ? launch(c, "bucket_reduce", k_reduce<double, kRedHead>, dim3(rblocks), dim3(kRedThreads), 0, ra)
                        : launch(c, "bucket_reduce", k_reduce<float, kRedHead>, dim3(rblocks), dim3(kRedThreads), 0, ra);
    return c->acc64 ? launch(c, "bucket_reduce", k_reduce<double, 32>, dim3(rblocks), dim3(kRedThreads), 0, ra)
                    : launch(c, "bucket_reduce", k_reduce<float, 32>, dim3(rblocks), dim3(kRedThreads), 0, ra);
}

int bucketmul_walk(Ctx* c, int n, const MatOp* ops) { return walk_and_reduce(c, n, ops, kInCutoff, nullptr, nullptr, 0.0f, nullptr); }

// One fused matrix group: record the slots, then either (all matrices on
// k_walk64) a walk in which every workgroup computes its input (norm) and
// cutoff itself, or the separate norm / cutoff launches before the walk;
// then the reduce with its epilogue.  in_mode kInNorm: x = rmsnorm(h) *
// gain is written to ops[0].x (every op must name the same x, 4096 inputs).
int bucketmul_fused(Ctx* c, int n, const MatOp* ops, int expert_no, float effort, int in_mode, const float* h,
                    const uint16_t* gain, float eps, const ReduceEp* ep)
{
    CutoffArgs args{};
    IAM_TRY(record_slots(c, n, ops, expert_no, effort, args));
    bool all64 = true;
    for (int i = 0; i < n; i++) all64 = all64 && vec_of(ops[i].mat.bucket_cols, c->acc64) == 8;
    if (in_mode == kInNorm) {
        IAM_REQUIRE(h && gain, "bucketmul: norm input without h/gain");
        const int ni = ops[0].in_size;
        for (int i = 0; i < n; i++)
            IAM_REQUIRE(ops[i].in_size == ni && ops[i].x == ops[0].x,
                        "bucketmul: the norm input is shared by the group");
        IAM_TRY(check_dev_range(c, h, (size_t)ni * sizeof(float), "bucketmul h"));
        IAM_TRY(check_dev_range(c, gain, (size_t)ni * 2, "bucketmul gain"));
        IAM_REQUIRE(((uintptr_t)h & 15) == 0 && ((uintptr_t)gain & 15) == 0, "bucketmul: h and gain must be 16-byte aligned");
        if (ni != kProbes) {
            // the walk's own norm covers 4096 inputs: a wider vector is
            // normalized by the RMSNorm kernel first (same order of sums)
            IAM_REQUIRE(ni % 1024 == 0, "bucketmul: a norm input must be a multiple of 1024 long");
            IAM_TRY(rmsnorm(c, const_cast<float*>(h), nullptr, gain, ni, eps, const_cast<float*>(ops[0].x)));
            in_mode = kInX;
        }
    }
    if (all64) return walk_and_reduce(c, n, ops, in_mode, h, gain, eps, ep);
    if (in_mode == kInNorm)
        IAM_TRY(rmsnorm(c, const_cast<float*>(h), nullptr, gain, ops[0].in_size, eps, const_cast<float*>(ops[0].x)));
    IAM_TRY(launch(c, "bucket_cutoff", k_cutoff, dim3(n), dim3(kCutThreads), 0, args));
    return walk_and_reduce(c, n, ops, kInCutoff, nullptr, nullptr, 0.0f, ep);
}

__global__ void k_stats_compact(const uint16_t* __restrict__ s, size_t rows, int stride, int ch,
                                uint16_t* __restrict__ out)
{
    size_t r = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r < rows) out[r] = s[r * stride + ch];
}

}  // namespace iam

using namespace iam;

extern "C" {

int iam_effort_quantile(float effort) { return quantile_of(effort); }

int iam_bucketmul_calc_dispatch(iam_ctx* c, const float* x, const uint16_t* stats,
                                const uint16_t* probes, int expert_no, int in_size,
                                int bucket_cols, int expert_size, float effort)
{
    if (!c) return fail(IAM_E_INVALID, "calc_dispatch: null context");
    MatOp op{};
    op.mat.stats = stats;
    op.mat.probes = probes;
    op.mat.expert_rows = expert_size;
    op.mat.bucket_cols = bucket_cols;
    op.mat.stats_stride = 4;    // reference file layout (bucketMul.cl:372)
    op.mat.stats_channel = 3;
    op.x = x;
    op.in_size = in_size;
    return bucketmul_dispatch(c, 1, &op, expert_no, effort);
}

int iam_bucketmul_mul(iam_ctx* c, const uint16_t* buckets, int bucket_cols, float* y)
{
    if (!c) return fail(IAM_E_INVALID, "mul: null context");
    const DispatchSlot& s = c->slots[0];
    if (!s.valid) return fail(IAM_E_STATE, "mul: no preceding calc_dispatch");
    IAM_REQUIRE(y, "mul: null y");
    MatOp op{};
    op.mat.buckets = buckets;
    op.mat.expert_rows = s.rows;
    op.mat.bucket_cols = bucket_cols;
    op.y = y;
    return bucketmul_walk(c, 1, &op);
}

int iam_bucketmul_full(iam_ctx* c, const float* x, const uint16_t* stats, const uint16_t* probes,
                       const uint16_t* buckets, int expert_no, int in_size, int bucket_cols,
                       int expert_size, float effort, float* y)
{
    if (!c) return fail(IAM_E_INVALID, "full: null context");
    MatOp op{};
    op.mat.buckets = buckets;
    op.mat.stats = stats;
    op.mat.probes = probes;
    op.mat.expert_rows = expert_size;
    op.mat.bucket_cols = bucket_cols;
    op.mat.stats_stride = 4;
    op.mat.stats_channel = 3;
    op.x = x;
    op.in_size = in_size;
    op.y = y;
    IAM_REQUIRE(y, "full: null y");
    IAM_TRY(bucketmul_dispatch(c, 1, &op, expert_no, effort));
    return bucketmul_walk(c, 1, &op);
}

int iam_bucketmul_multi(iam_ctx* c, int n, const iam_bucket_matrix* mats, const float* const* xs,
                        const int* in_sizes, float* const* ys, int expert_no, float effort)
{
    if (!c || !mats || !xs || !in_sizes || !ys) return fail(IAM_E_INVALID, "multi: null argument");
    if (n < 1 || n > kMaxMulti) return fail(IAM_E_INVALID, "multi: n must be 1..3");
    MatOp ops[kMaxMulti];
    for (int i = 0; i < n; i++) {
        ops[i].mat = mats[i];
        ops[i].x = xs[i];
        ops[i].in_size = in_sizes[i];
        ops[i].y = ys[i];
        IAM_REQUIRE(ys[i] && mats[i].buckets, "multi: null y/buckets");
    }
    IAM_TRY(bucketmul_dispatch(c, n, ops, expert_no, effort));
    return bucketmul_walk(c, n, ops);
}

int iam_bucketmul_fused(iam_ctx* c, int n, const iam_bucket_matrix* mats, float* x, int in_size,
                        float* const* ys, int expert_no, float effort, const float* h, const uint16_t* gain,
                        float eps)
{
    if (!c || !mats || !x || !ys) return fail(IAM_E_INVALID, "fused: null argument");
    if (n < 1 || n > kMaxMulti) return fail(IAM_E_INVALID, "fused: n must be 1..3");
    IAM_REQUIRE((h == nullptr) == (gain == nullptr), "fused: h and gain go together");
    IAM_REQUIRE(!h || (std::isfinite(eps) && eps >= 0.0f), "fused: eps must be finite and >= 0");
    MatOp ops[kMaxMulti];
    for (int i = 0; i < n; i++) {
        ops[i].mat = mats[i];
        ops[i].x = x;
        ops[i].in_size = in_size;
        ops[i].y = ys[i];
        IAM_REQUIRE(ys[i] && mats[i].buckets, "fused: null y/buckets");
    }
    return bucketmul_fused(c, n, ops, expert_no, effort, h ? kInNorm : kInX, h, gain, eps, nullptr);
}

// The cutoff comes from k_cutoff; the selection is re-run by the list kernel
// (which recomputes the cutoff on its own; the two must agree bit for bit).
static int dispatch_query(Ctx* c, int slot, float* cutoff, std::vector<uint32_t>* rows, uint32_t* count)
{
    if (slot < 0 || slot >= kMaxMulti) return fail(IAM_E_INVALID, "dispatch query: bad slot");
    DispatchSlot& s = c->slots[slot];
    if (!s.valid) return fail(IAM_E_STATE, "dispatch query: no dispatch in this slot");
    IAM_REQUIRE(!c->capturing, "dispatch query: not allowed during graph capture");
    IAM_TRY(bucketmul_list(c, slot));
    IAM_CHECK_HIP(hipStreamSynchronize(c->stream));
    float cut[2] = {0, 0};
    std::vector<uint32_t> counts(s.G);
    IAM_CHECK_HIP(hipMemcpy(cut, s.cutoff, sizeof(cut), hipMemcpyDeviceToHost));
    IAM_CHECK_HIP(hipMemcpy(counts.data(), s.counts, sizeof(uint32_t) * s.G, hipMemcpyDeviceToHost));
    uint32_t b0, b1;
    std::memcpy(&b0, &cut[0], 4);
    std::memcpy(&b1, &cut[1], 4);
    if (b0 != b1) return fail(IAM_E_STATE, "dispatch query: cutoff kernels disagree");
    uint64_t S = 0;
    std::vector<uint2> buf;
    for (int g = 0; g < s.G; g++) {
        if (counts[g] > (uint32_t)kChunkRows) return fail(IAM_E_STATE, "dispatch query: corrupt count");
        if (rows && counts[g]) {
            buf.resize(counts[g]);
            IAM_CHECK_HIP(hipMemcpy(buf.data(), s.list + (size_t)g * kChunkRows, sizeof(uint2) * counts[g],
                                    hipMemcpyDeviceToHost));
            for (uint32_t i = 0; i < counts[g]; i++) rows->push_back(buf[i].x);
        }
        S += counts[g];
    }
    if (cutoff) *cutoff = cut[0];
    if (count) *count = (uint32_t)S;
    return IAM_OK;
}

int iam_bucketmul_dispatch_info(iam_ctx* c, int slot, float* cutoff, uint32_t* count)
{
    if (!c) return fail(IAM_E_INVALID, "dispatch_info: null context");
    return dispatch_query(c, slot, cutoff, nullptr, count);
}

int iam_bucketmul_dispatch_rows(iam_ctx* c, int slot, uint32_t* rows, size_t cap, uint32_t* count)
{
    if (!c) return fail(IAM_E_INVALID, "dispatch_rows: null context");
    std::vector<uint32_t> v;
    uint32_t S = 0;
    IAM_TRY(dispatch_query(c, slot, nullptr, &v, &S));
    for (size_t i = 0; i < v.size() && i < cap && rows; i++) rows[i] = v[i];
    if (count) *count = S;
    return IAM_OK;
}

int iam_bucketmul_walk_count(iam_ctx* c, int slot, uint32_t* count)
{
    if (!c || !count || slot < 0 || slot >= kMaxMulti) return fail(IAM_E_INVALID, "walk_count: bad argument");
    const DispatchSlot& s = c->slots[slot];
    if (!s.valid) return fail(IAM_E_STATE, "walk_count: no dispatch in this slot");
    if (!s.counted) return fail(IAM_E_STATE, "walk_count: the last walk of this slot ran with counting off");
    IAM_CHECK_HIP(hipStreamSynchronize(c->stream));
    IAM_CHECK_HIP(hipMemcpy(count, s.count, sizeof(uint32_t), hipMemcpyDeviceToHost));
    return IAM_OK;
}

int iam_stats_compact(iam_ctx* c, const uint16_t* stats, size_t rows, int stride, int channel,
                      uint16_t* out)
{
    if (!c || !stats || !out) return fail(IAM_E_INVALID, "stats_compact: null argument");
    IAM_REQUIRE(stride >= 1 && channel >= 0 && channel < stride, "stats_compact: bad stride/channel");
    if (rows == 0) return IAM_OK;
    IAM_TRY(check_dev_range(c, stats, rows * (size_t)stride * 2, "stats_compact stats"));
    IAM_TRY(check_dev_range(c, out, rows * 2, "stats_compact out"));
    return launch(c, "stats_compact", k_stats_compact, dim3((unsigned)((rows + 255) / 256)), dim3(256),
                  0, stats, rows, stride, channel, out);
}

}  // extern "C"
