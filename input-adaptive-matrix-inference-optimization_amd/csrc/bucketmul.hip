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
    if (g == 0 && tid == 0) d.cutoff[0] = cutoff;

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
struct WalkDesc {
    const uint16_t* W;        // rows of the expert: W[row * C + col]
    const uint2* list;
    const uint32_t* counts;
    void* part;               // [P][16*C] partial sums (Acc), one row per row slice
    unsigned long long* counters;   // walk bytes, rows, matrices (block 0 adds)
    int C;
    int G;
    int P;                    // row slices
    int T;                    // column tiles
    int block_base;
};

struct WalkArgs {
    WalkDesc d[kMaxMulti];
    int n;
};

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

// x * w as the accumulator type: an fp32 product (bucketMul.cl:430-434), or
// the exact product in fp64 (24 + 11 significant bits fit in 53).
template <typename Acc>
__device__ __forceinline__ Acc walk_prod(float x, uint32_t h);
template <>
__device__ __forceinline__ float walk_prod<float>(float x, uint32_t h) { return __fmul_rn(x, h2f(h)); }
template <>
__device__ __forceinline__ double walk_prod<double>(float x, uint32_t h)
{
    return (double)x * (double)h2f(h);
}

// Walk of the selected rows.  Workgroup (row slice p, column tile t) takes
// the slice's share of the selected-row list and the 64 columns of tile t.
// Lane = q*NJ + j: j picks VEC consecutive columns (NJ = 64/VEC lanes cover
// the 128-byte tile segment of one row), q picks one of NQ = VEC rows read
// by the same instruction.  Every lane owns private accumulators for its VEC
// columns x 16 output positions at acc[wave][(pos*VEC + e)*64 + lane]: the
// scatter of a packed weight to its position (bucketMul.cl:430-445) is a
// plain LDS read-add-write, with no atomics, and the 64 lanes of one access
// always fall in 64 different banks.  Each lane adds in list order, and the
// flush sums waves and row slots in a fixed order, so the result does not
// depend on scheduling.  The VEC elements of one row go to distinct
// addresses (different e), so their reads are issued together, then their
// writes; the next row's reads follow the writes in the wave's LDS order.
//
// The list is the dispatch output: per chunk of 256 inputs, counts[g]
// entries at list[g * kChunkRows].  All UNR list loads of a batch, then all
// UNR weight loads, are unconditional (past the slice end a lane re-reads
// the slice's last entry with x = 0) so they are in flight together.
template <int VEC, typename Acc, int NW, int UNR>
__global__ __launch_bounds__(64 * NW) void k_walk(WalkArgs a)
{
    constexpr int NJ = 64 / VEC, NQ = VEC, TW = 64;
    constexpr int PER = 16 * VEC * 64;         // accumulators per wave
    constexpr int NT = 64 * NW;
    constexpr int STRIDE = NW * NQ;            // rows per workgroup instruction
    __shared__ Acc acc[NW * PER];
    __shared__ uint32_t s_pre[kMaxChunks + 1];
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

    // exclusive prefix of the chunk counts: thread tid owns chunks
    // [tid*CPT, tid*CPT + CPT)
    constexpr int CPT = (kMaxChunks + NT - 1) / NT;
    uint32_t cl[CPT];
    uint32_t mine = 0;
#pragma unroll
    for (int i = 0; i < CPT; i++) {
        const int g = tid * CPT + i;
        cl[i] = g < d.G ? d.counts[g] : 0u;
        mine += cl[i];
    }
    uint32_t incl = mine;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t v = __shfl_up(incl, o, 64);
        if (lane >= o) incl += v;
    }
    if (lane == 63) s_wsum[wave] = incl;
    __syncthreads();
    uint32_t run = incl - mine;
    for (int i = 0; i < wave; i++) run += s_wsum[i];
#pragma unroll
    for (int i = 0; i < CPT; i++) {
        const int g = tid * CPT + i;
        if (g < d.G) s_pre[g] = run;
        run += cl[i];
    }
    if (tid == NT - 1) s_pre[d.G] = run;   // total (the last thread owns the last chunks)
    __syncthreads();
    const uint32_t S = s_pre[d.G];
    if (w == 0 && tid == 0) {
        atomicAdd(d.counters + 0, (unsigned long long)S * (unsigned long long)d.C * 2ull);
        atomicAdd(d.counters + 1, (unsigned long long)S);
        atomicAdd(d.counters + 2, 1ull);
    }
    const uint32_t lo = (uint32_t)(((uint64_t)S * (uint32_t)p) / (uint32_t)d.P);
    const uint32_t hi = (uint32_t)(((uint64_t)S * (uint32_t)(p + 1)) / (uint32_t)d.P);

    const int q = lane / NJ;
    const int j = lane - q * NJ;
    const int col0 = t * TW + j * VEC;
    // Lanes past the last column read column 0 and add zeros.
    const int colc = col0 < d.C ? col0 : 0;
    const float xmask = col0 < d.C ? 1.0f : 0.0f;
    using LT = typename VecLoad<VEC>::T;

    if (lo < hi) {
        // chunk of the lane's current entry: s_pre[ch] <= idx < chend
        int ch = 0;
        {
            const uint32_t first = lo;
            int l = 0, h = d.G;
            while (h - l > 1) {
                const int m = (l + h) >> 1;
                if (s_pre[m] <= first) l = m;
                else h = m;
            }
            ch = l;
        }
        uint32_t chbeg = s_pre[ch], chend = s_pre[ch + 1];
        for (uint32_t base = lo + (uint32_t)(wave * NQ); base < hi; base += (uint32_t)(STRIDE * UNR)) {
            const uint2* ep[UNR];
            bool ok[UNR];
#pragma unroll
            for (int u = 0; u < UNR; u++) {
                const uint32_t raw = base + (uint32_t)(q + u * STRIDE);
                ok[u] = raw < hi;
                const uint32_t idx = ok[u] ? raw : hi - 1;
                while (idx >= chend) {
                    ch++;
                    chbeg = chend;
                    chend = s_pre[ch + 1];
                }
                ep[u] = d.list + (size_t)ch * kChunkRows + (idx - chbeg);
            }
            uint2 en[UNR];
#pragma unroll
            for (int u = 0; u < UNR; u++) en[u] = *ep[u];
            LT v[UNR];
            float xv[UNR];
#pragma unroll
            for (int u = 0; u < UNR; u++) {
                xv[u] = ok[u] ? __uint_as_float(en[u].y) * xmask : 0.0f;
                v[u] = *reinterpret_cast<const LT*>(d.W + (size_t)en[u].x * d.C + colc);
            }
            // keep all UNR weight loads ahead of the accumulation
            asm volatile("" ::: "memory");
#pragma unroll
            for (int u = 0; u < UNR; u++) {
                uint32_t words[(VEC + 1) / 2];
                VecLoad<VEC>::split(v[u], words);
                int ad[VEC];
                Acc pr[VEC], old[VEC];
#pragma unroll
                for (int e = 0; e < VEC; e++) {
                    const uint32_t h = (words[e >> 1] >> ((e & 1) * 16)) & 0xffffu;
                    ad[e] = ((int)(h & 15u) * VEC + e) * 64;
                    pr[e] = walk_prod<Acc>(xv[u], h);
                }
#pragma unroll
                for (int e = 0; e < VEC; e++) old[e] = my[ad[e]];
#pragma unroll
                for (int e = 0; e < VEC; e++) my[ad[e]] = old[e] + pr[e];
            }
        }
    }
    __syncthreads();
    // flush: output col*16 + pos (bucketMul.cl:442-445) of this tile as one
    // contiguous run of the slice's partial row
    Acc* prow = reinterpret_cast<Acc*>(d.part) + (size_t)p * d.C * 16;
    for (int idx = tid; idx < TW * 16; idx += NT) {
        const int c = idx >> 4;          // column within the tile
        const int pos = idx & 15;
        const int jj = c / VEC, e = c - jj * VEC;
        const int col = t * TW + c;
        if (col >= d.C) continue;
        const int ai = (pos * VEC + e) * 64 + jj;
        Acc s = (Acc)0;
        for (int ww = 0; ww < NW; ww++)
#pragma unroll
            for (int qq = 0; qq < NQ; qq++) s += acc[ww * PER + ai + qq * NJ];
        prow[(size_t)col * 16 + pos] = s;
    }
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

// Row slices per matrix for one walk launch: about kWalkTarget workgroups in
// total, shared by the matrices in proportion to their expected bytes, with
// at least kMinSliceRows rows per slice.  Only the performance depends on it.
constexpr int kWalkTarget = 1024;
constexpr int kMinSliceRows = 64;

static void plan_slices(int n, const double* bytes, const double* rows, const int* T, int* P)
{
    double tot = 0;
    for (int i = 0; i < n; i++) tot += bytes[i];
    for (int i = 0; i < n; i++) {
        double wgs = tot > 0 ? kWalkTarget * bytes[i] / tot : kWalkTarget / n;
        int p = (int)std::lround(wgs / T[i]);
        int pmax = std::max(1, (int)(rows[i] / kMinSliceRows));
        P[i] = std::max(1, std::min(p, std::min(pmax, 4096)));
    }
}

static int vec_of(int C)
{
    if (C % 4 == 0) return 4;
    if (C % 2 == 0) return 2;
    return 1;
}

int bucketmul_dispatch(Ctx* c, int n, const MatOp* ops, int expert_no, float effort)
{
    IAM_REQUIRE(n >= 1 && n <= kMaxMulti, "bucketmul: 1..3 matrices per launch");
    IAM_REQUIRE(!std::isnan(effort), "bucketmul: effort is NaN");
    IAM_REQUIRE(expert_no >= 0, "bucketmul: negative expert_no");
    DispatchArgs args{};
    args.n = n;
    int blocks = 0;
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
        const int G = (std::min(inputs, ops[i].in_size) + kChunkInputs - 1) / kChunkInputs;
        IAM_REQUIRE(G <= kMaxChunks, "bucketmul: more than 65536 inputs per expert");
        // every device range the kernels read or write must lie inside an
        // allocation of this context (the cutoff always reads x[0:4096])
        const size_t xn = std::max<size_t>(kProbes, std::min<size_t>((size_t)ops[i].in_size, (size_t)inputs));
        IAM_TRY(check_dev_range(c, ops[i].x, xn * sizeof(float), "bucketmul x"));
        IAM_TRY(check_dev_range(c, M.probes, (size_t)(expert_no + 1) * kProbes * 2, "bucketmul probes"));
        IAM_TRY(check_dev_range(c, M.stats, (size_t)(expert_no + 1) * M.expert_rows * M.stats_stride * 2,
                                "bucketmul stats"));

        IAM_TRY(ensure_slot(c, i, std::max(G, 1)));
        DispatchSlot& s = c->slots[i];
        DispatchDesc& d = args.d[i];
        d.x = ops[i].x;
        d.probes = probes;
        d.stats = M.stats + (size_t)expert_no * (size_t)M.expert_rows * M.stats_stride;
        d.stats_stride = M.stats_stride;
        d.stats_channel = M.stats_channel;
        d.rows = M.expert_rows;
        d.in_size = ops[i].in_size;
        d.quantile = qv;
        d.G = std::max(G, 1);
        d.list = s.list;
        d.counts = s.counts;
        d.cutoff = s.cutoff;
        d.block_base = blocks;
        blocks += d.G;
        s.G = d.G;
        s.rows = M.expert_rows;
        s.bucket_cols = M.bucket_cols;
        s.expert_no = expert_no;
        s.effort = effort;
        s.valid = true;
    }
    return launch(c, "bucket_dispatch", k_dispatch, dim3(blocks), dim3(kCutThreads), 0, args);
}

void plan_walk(int n, const MatOp* ops, float effort, int* T, int* P, int* V)
{
    double bytes[kMaxMulti], rows[kMaxMulti];
    for (int i = 0; i < n; i++) {
        const iam_bucket_matrix& M = ops[i].mat;
        V[i] = vec_of(M.bucket_cols);
        T[i] = (M.bucket_cols + 63) / 64;   // 64-column tiles
        rows[i] = est_rows(M.expert_rows, effort);
        bytes[i] = rows[i] * M.bucket_cols;
    }
    plan_slices(n, bytes, rows, T, P);
}

// Launch shapes: fp32 accumulators with 4 columns per lane (16 KB of LDS per
// wave), fp64 with 2 (also 16 KB per wave); two waves per workgroup and 16
// rows in flight per lane.  Narrower tiles follow the column count.
constexpr int kWalkWaves = 2;
constexpr int kWalkUnroll = 16;

template <typename Acc>
static int launch_walk(Ctx* c, int vec, int blocks, const WalkArgs& args)
{
    const dim3 g(blocks), t(64 * kWalkWaves);
    constexpr bool f64 = sizeof(Acc) == 8;
    if (vec >= 4 && !f64) return launch(c, "bucket_walk", k_walk<4, Acc, kWalkWaves, kWalkUnroll>, g, t, 0, args);
    if (vec >= 2) return launch(c, "bucket_walk", k_walk<2, Acc, kWalkWaves, kWalkUnroll>, g, t, 0, args);
    return launch(c, "bucket_walk", k_walk<1, Acc, kWalkWaves, kWalkUnroll>, g, t, 0, args);
}

int bucketmul_walk(Ctx* c, int n, const MatOp* ops)
{
    IAM_REQUIRE(n >= 1 && n <= kMaxMulti, "bucketmul: 1..3 matrices per launch");
    int T[kMaxMulti], P[kMaxMulti], V[kMaxMulti];
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
    plan_walk(n, ops, c->slots[0].effort, T, P, V);
    const size_t acc_bytes = c->acc64 ? 8 : 4;
    for (int i = 0; i < n; i++)
        IAM_TRY(ensure_partials(c, i, (size_t)P[i] * ops[i].mat.bucket_cols * 16 * acc_bytes));

    // walk: one launch per load width (the model's matrices all share one)
    bool used[kMaxMulti] = {false, false, false};
    for (int done = 0; done < n;) {
        int vec = 0, blocks = 0, cnt = 0;
        WalkArgs args{};
        for (int i = 0; i < n; i++) {
            if (used[i] || (vec != 0 && V[i] != vec)) continue;
            vec = V[i];
            const DispatchSlot& s = c->slots[i];
            WalkDesc& d = args.d[cnt++];
            d.W = ops[i].mat.buckets + (size_t)s.expert_no * (size_t)ops[i].mat.expert_rows * ops[i].mat.bucket_cols;
            d.list = s.list;
            d.counts = s.counts;
            d.part = s.part;
            d.counters = c->counters;
            d.C = ops[i].mat.bucket_cols;
            d.G = s.G;
            d.P = P[i];
            d.T = T[i];
            d.block_base = blocks;
            blocks += P[i] * T[i];
            used[i] = true;
            done++;
        }
        args.n = cnt;
        IAM_TRY(c->acc64 ? launch_walk<double>(c, vec, blocks, args) : launch_walk<float>(c, vec, blocks, args));
    }
    // fixed-order sum of the slices into y
    ReduceArgs ra{};
    ra.n = n;
    int rblocks = 0;
    for (int i = 0; i < n; i++) {
        ReduceDesc& d = ra.d[i];
        d.part = c->slots[i].part;
        d.y = ops[i].y;
        d.P = P[i];
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

int iam_bucketmul_dispatch_info(iam_ctx* c, int slot, float* cutoff, uint32_t* count)
{
    if (!c || slot < 0 || slot >= kMaxMulti) return fail(IAM_E_INVALID, "dispatch_info: bad argument");
    const DispatchSlot& s = c->slots[slot];
    if (!s.valid) return fail(IAM_E_STATE, "dispatch_info: no dispatch in this slot");
    IAM_CHECK_HIP(hipStreamSynchronize(c->stream));
    float cut = 0;
    std::vector<uint32_t> counts(s.G);
    IAM_CHECK_HIP(hipMemcpy(&cut, s.cutoff, sizeof(float), hipMemcpyDeviceToHost));
    IAM_CHECK_HIP(hipMemcpy(counts.data(), s.counts, sizeof(uint32_t) * s.G, hipMemcpyDeviceToHost));
    uint64_t S = 0;
    for (auto v : counts) S += v;
    if (cutoff) *cutoff = cut;
    if (count) *count = (uint32_t)S;
    return IAM_OK;
}

int iam_bucketmul_dispatch_rows(iam_ctx* c, int slot, uint32_t* rows, size_t cap, uint32_t* count)
{
    if (!c || slot < 0 || slot >= kMaxMulti) return fail(IAM_E_INVALID, "dispatch_rows: bad argument");
    const DispatchSlot& s = c->slots[slot];
    if (!s.valid) return fail(IAM_E_STATE, "dispatch_rows: no dispatch in this slot");
    IAM_CHECK_HIP(hipStreamSynchronize(c->stream));
    std::vector<uint32_t> counts(s.G);
    IAM_CHECK_HIP(hipMemcpy(counts.data(), s.counts, sizeof(uint32_t) * s.G, hipMemcpyDeviceToHost));
    size_t out = 0;
    std::vector<uint2> buf;
    for (int g = 0; g < s.G; g++) {
        if (counts[g] > (uint32_t)kChunkRows) return fail(IAM_E_STATE, "dispatch_rows: corrupt count");
        buf.resize(counts[g]);
        if (counts[g])
            IAM_CHECK_HIP(hipMemcpy(buf.data(), s.list + (size_t)g * kChunkRows,
                                    sizeof(uint2) * counts[g], hipMemcpyDeviceToHost));
        for (uint32_t i = 0; i < counts[g]; i++) {
            if (rows && out < cap) rows[out] = buf[i].x;
            out++;
        }
    }
    if (count) *count = (uint32_t)out;
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
