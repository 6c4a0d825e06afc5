// Input-adaptive sparse GEMV ("bucketMul") for gfx950.
//
// Reference pipeline (bucket_mul.hpp:147-267, bucketMul.cl):
//   findCutoffBinarySearch -> prepareDispatch -> roundUp/zeroRange32 ->
//   bucketMul -> bucketIntegrate                      (6 launches + 1 fill)
// Here:
//   k_dispatch  one launch: every workgroup recomputes the cutoff (the search
//               is a pure function of x[0:4096] and the probes), then selects
//               the rows of its chunk of 256 inputs and compacts them in
//               ascending order as {row, x[row/16]} (no global atomics, no
//               float-encoded offsets).
//   k_walk      one launch: workgroup (slice p, column tile t) streams its
//               share of the selected rows, scatter-adds x*w into lane-private
//               LDS accumulators (no atomics) and writes one partial row per
//               slice.
//   k_reduce    one launch: sums the slice partials in a fixed order into y.
// The cutoff and selection arithmetic is exact IEEE fp32 (no contraction), so
// the cutoff bits and the selected set equal the oracle's.  The walk
// accumulates in fp32 or, by default, in fp64 (the product of an fp32 input
// and an fp16 weight is exact in fp64), so y is the correctly rounded sum up
// to fp64 rounding and does not depend on the order of the additions.
#include <hip/hip_fp16.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "internal.h"

namespace iam {

constexpr float kScale = 100000.0f;   // bucketMul.cl:17
constexpr int kCutThreads = 256;
constexpr int kCutVPT = kProbes / kCutThreads;   // 16 importances per thread

__device__ __forceinline__ float h2f(uint32_t bits16)
{
    return __half2float(__ushort_as_half((unsigned short)(bits16 & 0xffffu)));
}

// --------------------------------------------------------------- cutoff ---
// findCutoffBinarySearch (bucketMul.cl:68-214) for one 256-thread workgroup.
// Every thread ends with the same cutoff.  s_red needs 8 floats, s_cnt 8 ints.
__device__ float block_cutoff(const float* __restrict__ x, const uint16_t* __restrict__ probes,
                              int quantile, float* s_red, int* s_cnt)
{
#pragma clang fp contract(off)
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    float v[kCutVPT];
    {
        const float4* xv = reinterpret_cast<const float4*>(x + tid * kCutVPT);
        const uint4* pv = reinterpret_cast<const uint4*>(probes + tid * kCutVPT);
        float4 xa = xv[0], xb = xv[1], xc = xv[2], xd = xv[3];
        uint4 pa = pv[0], pb = pv[1];
        float xs[16] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w,
                        xc.x, xc.y, xc.z, xc.w, xd.x, xd.y, xd.z, xd.w};
        uint32_t ps[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
#pragma unroll
        for (int k = 0; k < 16; k++) {
            float p = h2f(ps[k >> 1] >> ((k & 1) * 16));
            float prod = __fmul_rn(xs[k], p);
            v[k] = __fmul_rn(kScale, fabsf(prod));   // bucketMul.cl:110
        }
    }
    float mn = 1e30f, mx = -1e30f;                    // bucketMul.cl:98-99
#pragma unroll
    for (int k = 0; k < 16; k++) {
        mn = fminf(mn, v[k]);
        mx = fmaxf(mx, v[k]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        mn = fminf(mn, __shfl_xor(mn, o, 64));
        mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    }
    if (lane == 0) {
        s_red[wave] = mn;
        s_red[4 + wave] = mx;
    }
    __syncthreads();
    const float gmin = fminf(fminf(s_red[0], s_red[1]), fminf(s_red[2], s_red[3]));
    const float gmax = fmaxf(fmaxf(s_red[4], s_red[5]), fmaxf(s_red[6], s_red[7]));

    const int target = kProbes - quantile;            // bucketMul.cl:81
    float minB = gmin, maxB = gmax;
    float bound = __fmul_rn(__fadd_rn(gmin, gmax), 0.5f);
    int minC = kProbes, maxC = 0;
    for (int loop = 0; loop < 20; loop++) {
        int c = 0;
#pragma unroll
        for (int k = 0; k < 16; k++) c += __popcll(__ballot(v[k] > bound));
        if (lane == 0) s_cnt[(loop & 1) * 4 + wave] = c;
        __syncthreads();
        const int* sc = s_cnt + (loop & 1) * 4;
        const int count = sc[0] + sc[1] + sc[2] + sc[3];
        if (count < target) {                          // bucketMul.cl:178-186
            maxB = bound;
            maxC = count;
        } else {
            minB = bound;
            minC = count;
        }
        const float next = __fmul_rn(__fadd_rn(minB, maxB), 0.5f);
        const int gap = maxC - minC;
        if (count == target || __fsub_rn(maxB, minB) < 0.00001f || (gap < 0 ? -gap : gap) < 3)
            return bound;                              // bucketMul.cl:195-200
        bound = next;
    }
    return bound;                                      // bucketMul.cl:211-213
}

// --------------------------------------------------------------- cutoff ---
// One workgroup per matrix: the cutoff of findCutoffBinarySearch, and the
// selected-row counter of the walk cleared (the walk adds to it).
struct CutoffDesc {
    const float* x;
    const uint16_t* probes;   // already offset to the expert
    int quantile;
    float* cutoff;
    uint32_t* count;
};

struct CutoffArgs {
    CutoffDesc d[kMaxMulti];
    int n;
};

__global__ __launch_bounds__(kCutThreads) void k_cutoff(CutoffArgs a)
{
    __shared__ float s_red[8];
    __shared__ int s_cnt[8];
    const CutoffDesc& d = a.d[blockIdx.x];
    const float cut = block_cutoff(d.x, d.probes, d.quantile, s_red, s_cnt);
    if (threadIdx.x == 0) {
        d.cutoff[0] = cut;
        d.count[0] = 0u;
    }
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
    __shared__ float s_red[8];
    __shared__ int s_cnt[8];
    __shared__ int s_wsum[4];

    int k = 0;
    for (int i = 1; i < a.n; i++)
        if ((int)blockIdx.x >= a.d[i].block_base) k = i;
    const DispatchDesc& d = a.d[k];
    const int g = (int)blockIdx.x - d.block_base;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    const float cutoff = block_cutoff(d.x, d.probes, d.quantile, s_red, s_cnt);
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
    const float* x;
    const uint16_t* stats;    // row 0 of the expert
    const float* cutoff;
    uint32_t* count;          // selected rows, added by the tile-0 workgroups
    void* part;               // [P][16*C] partial sums (Acc), one row per slice
    unsigned long long* counters;   // walk bytes, rows, matrices
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

// Selection of slice p (prepareDispatch, bucketMul.cl:351-386): thread i
// takes input i0 + i, loads its x and the stats of its 16 rows, and marks the
// rows with 1e5 * |x * stat| >= cutoff -- the same fp32 operations as the
// dispatch kernel, so the selected set is the same.  A block scan compacts
// the selected rows in ascending order into s_row (slice-local ids
// input*16 + rank); s_x[i] = x[i0 + i].  Ends with a barrier; returns the
// number of selected rows.  The tile-0 workgroup of the slice adds the count
// to the matrix's counters.
template <int NT>
__device__ uint32_t select_slice(const WalkDesc& d, int p, int t, int i0, int ni, uint16_t* s_row, float* s_x,
                                 uint32_t* s_wsum)
{
#pragma clang fp contract(off)
    constexpr int NW = NT / 64;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const float cutoff = *d.cutoff;
    uint32_t mask = 0;
    float xi = 0.0f;
    if (tid < ni) {
        const int i = i0 + tid;
        const int r0 = i * 16;
        xi = d.x[i];
        uint32_t sv[16];
        const uint16_t* st = d.stats + (size_t)r0 * d.stats_stride;
        const bool whole = r0 + 16 <= d.rows;
        if (whole && d.stats_stride == 1 && (((uintptr_t)st) & 15) == 0) {
            const uint4* p4 = reinterpret_cast<const uint4*>(st);
            const uint4 a0 = p4[0], a1 = p4[1];
            const uint32_t ww[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
            for (int kk = 0; kk < 16; kk++) sv[kk] = (ww[kk >> 1] >> ((kk & 1) * 16)) & 0xffffu;
        } else if (whole && d.stats_stride == 4 && d.stats_channel == 3 && (((uintptr_t)st) & 15) == 0) {
            const uint4* p4 = reinterpret_cast<const uint4*>(st);
            uint4 q8[8];
#pragma unroll
            for (int k8 = 0; k8 < 8; k8++) q8[k8] = p4[k8];
#pragma unroll
            for (int k8 = 0; k8 < 8; k8++) {
                sv[2 * k8] = q8[k8].y >> 16;       // row 2*k8, channel 3
                sv[2 * k8 + 1] = q8[k8].w >> 16;   // row 2*k8+1, channel 3
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
            const float avg = h2f(sv[kk]);
            const float prod = __fmul_rn(xi, avg);
            const float imp = __fmul_rn(kScale, fabsf(prod));
            if (imp >= cutoff && r0 + kk < d.rows) mask |= 1u << kk;   // bucketMul.cl:380
        }
    }
    const uint32_t cnt = (uint32_t)__popc(mask);
    uint32_t incl = cnt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t v = __shfl_up(incl, o, 64);
        if (lane >= o) incl += v;
    }
    if (lane == 63) s_wsum[wave] = incl;
    s_x[tid] = xi;
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
    if (t == 0 && tid == 0) {
        atomicAdd(d.count, n_sel);
        atomicAdd(d.counters + 0, (unsigned long long)n_sel * (unsigned long long)d.C * 2ull);
        atomicAdd(d.counters + 1, (unsigned long long)n_sel);
        if (p == 0) atomicAdd(d.counters + 2, 1ull);
    }
    return n_sel;
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
    const uint32_t n_sel = select_slice<NT>(d, p, t, i0, ni, s_row, s_x, s_wsum);

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
    __shared__ double acc[NW * SLOTS];
    __shared__ uint16_t s_row[NT * 16];
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

    {
        double2* z = reinterpret_cast<double2*>(acc + wave * SLOTS);
#pragma unroll
        for (int i = 0; i < SLOTS / 128; i++) z[i * 64 + lane] = make_double2(0.0, 0.0);
    }

    const int i0 = p * d.IPS;
    const int ni = min(d.IPS, d.n_in - i0);
    const int ns = (int)select_slice<NT>(d, p, t, i0, ni, s_row, s_x, s_wsum);

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
                    atomicAdd(accw + (int)(h & 15u) * TW + e * 16, xc[u] * wv);
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

// y[o] = sum over row slices of part[p][o], in slice order 0..P-1 grouped by
// p mod 16 then combined in group order: a fixed order, so y is the same on
// every run (bucketIntegrate, bucketMul.cl:453-497, sums 64 fixed slices).
struct ReduceDesc {
    const void* part;
    float* y;
    int P;
    int m;
    int block_base;
};

struct ReduceArgs {
    ReduceDesc d[kMaxMulti];
    int n;
};

constexpr int kRedOut = 64;   // outputs per reduce block

template <typename Acc>
__global__ __launch_bounds__(256) void k_reduce(ReduceArgs a)
{
    __shared__ Acc red[16][kRedOut];
    const int b = (int)blockIdx.x;
    int k = 0;
    for (int i = 1; i < a.n; i++)
        if (b >= a.d[i].block_base) k = i;
    const ReduceDesc& d = a.d[k];
    const Acc* part = reinterpret_cast<const Acc*>(d.part);
    const int o0 = (b - d.block_base) * kRedOut;
    const int tid = threadIdx.x;
    const int ol = tid & 15, pg = tid >> 4;
    const int o = o0 + ol * 4;   // m is a multiple of 16, so o..o+3 are in range together
    Acc s[4] = {(Acc)0, (Acc)0, (Acc)0, (Acc)0};
    if (o < d.m) {
        for (int p = pg; p < d.P; p += 16) {
            const Acc* r = part + (size_t)p * d.m + o;
#pragma unroll
            for (int i = 0; i < 4; i++) s[i] += r[i];
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) red[pg][ol * 4 + i] = s[i];
    __syncthreads();
    if (tid < kRedOut && o0 + tid < d.m) {
        Acc t = red[0][tid];
        for (int g = 1; g < 16; g++) t += red[g][tid];
        d.y[o0 + tid] = (float)t;
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

// Walk launch shape: NW waves per workgroup, each with 16 KB of private
// accumulators (fp32: 4 columns per lane; fp64: 2), 16 rows in flight per
// lane; a slice holds at most 64*NW inputs.
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

#ifndef IAM_W64_NW
#define IAM_W64_NW 4
#endif
#ifndef IAM_W64_UNR
#define IAM_W64_UNR 4
#endif
#ifndef IAM_W64_WG_BYTES
#define IAM_W64_WG_BYTES 131072.0
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
        bytes[i] = est_rows(pl.n_in * 16, effort) * M.bucket_cols * 2.0;
        tot += bytes[i];
    }
    const int nw = all64 ? IAM_W64_NW : tot < kWalkWideBytes ? IAM_WALK_SMALL_NW : IAM_WALK_BIG_NW;
    const double wg_bytes = all64 ? IAM_W64_WG_BYTES : kWalkWgBytes;
    const double target = std::min(kWalkMaxWgs, std::max(kWalkMinWgs, tot / wg_bytes));
    for (int i = 0; i < n; i++) {
        WalkPlan& pl = plan[i];
        pl.NW = pl.V == 8 ? IAM_W64_NW : nw;
        const double wgs = tot > 0 ? target * bytes[i] / tot : target / n;
        const int slices = std::max(1, (int)std::lround(wgs / pl.T));
        pl.IPS = std::min(64 * pl.NW, std::max(1, (pl.n_in + slices - 1) / slices));
        pl.P = (pl.n_in + pl.IPS - 1) / pl.IPS;
    }
}

// Record the selection problem of matrix op i in slot i and compute the
// cutoffs (one workgroup per matrix).
int bucketmul_dispatch(Ctx* c, int n, const MatOp* ops, int expert_no, float effort)
{
    IAM_REQUIRE(n >= 1 && n <= kMaxMulti, "bucketmul: 1..3 matrices per launch");
    IAM_REQUIRE(!std::isnan(effort), "bucketmul: effort is NaN");
    IAM_REQUIRE(expert_no >= 0, "bucketmul: negative expert_no");
    CutoffArgs args{};
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
        d.count = s.count;
    }
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

int bucketmul_walk(Ctx* c, int n, const MatOp* ops)
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
    const size_t acc_bytes = c->acc64 ? 8 : 4;
    for (int i = 0; i < n; i++)
        IAM_TRY(ensure_partials(c, i, (size_t)plan[i].P * ops[i].mat.bucket_cols * 16 * acc_bytes));

    // walk: one launch per load width (the model's matrices all share one)
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
            d.x = s.x;
            d.stats = s.stats;
            d.cutoff = s.cutoff;
            d.count = s.count;
            d.part = s.part;
            d.counters = c->counters;
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
        if (vec == 8)
            IAM_TRY(launch(c, "bucket_walk", k_walk64<IAM_W64_NW, IAM_W64_UNR>, dim3(blocks), dim3(64 * IAM_W64_NW),
                           0, args));
        else
            IAM_TRY(c->acc64 ? launch_walk<double>(c, nw, vec, blocks, args)
                             : launch_walk<float>(c, nw, vec, blocks, args));
    }
    // fixed-order sum of the slices into y
    ReduceArgs ra{};
    ra.n = n;
    int rblocks = 0;
    for (int i = 0; i < n; i++) {
        ReduceDesc& d = ra.d[i];
        d.part = c->slots[i].part;
        d.y = ops[i].y;
        d.P = plan[i].P;
        d.m = ops[i].mat.bucket_cols * 16;
        d.block_base = rblocks;
        rblocks += (d.m + kRedOut - 1) / kRedOut;
    }
    if (c->acc64) return launch(c, "bucket_reduce", k_reduce<double>, dim3(rblocks), dim3(256), 0, ra);
    return launch(c, "bucket_reduce", k_reduce<float>, dim3(rblocks), dim3(256), 0, ra);
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
