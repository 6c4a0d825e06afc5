// Input-adaptive sparse GEMV ("bucketMul") for gfx950.
//
// Reference pipeline (bucket_mul.hpp:147-267, bucketMul.cl):
//   findCutoffBinarySearch -> prepareDispatch -> roundUp/zeroRange32 ->
//   bucketMul -> bucketIntegrate                      (6 launches + 1 fill)
// Here one launch per group of up to 3 matrices that share an input
// (k_walk): workgroup (input slice p, 64-column tile t) computes the input
// itself when it is a norm, a residual sum, an embedding row or an attention
// output, runs the cutoff search (a pure function of x[0:4096] and the
// probes, search.h), selects the rows of its slice and walks them, adding
// each product x*w to its wave's LDS tile; the tiles are then added in wave
// order and flushed with one global atomic add per output into an
// accumulator that starts at zero.  The accumulator is read either by the
// next launch of the decode step (which applies the residual add, RoPE or
// the attention normalisation itself) or, in the finalize modes, by the
// last workgroup to flush each column tile: it takes the sums (clearing the
// accumulator for the next call) and stores fp32 outputs, the SiLU gate, or
// the logits and the greedy pick.  k_cutoff serves the split calcDispatch /
// mul calls and k_dispatch the parity queries (cutoff, selected rows).
//
// The cutoff and selection arithmetic is exact IEEE fp32 (no contraction),
// so the cutoff bits and the selected set equal the oracle's.  With fp64
// accumulation the product of an fp32 input and an fp16 weight is exact, so
// each output is the sum of exact products rounded once at the end; only the
// order of the fp64 additions (atomics from the workgroups) varies, far
// below an fp32 ulp.
#include <hip/hip_fp16.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstring>
#include <type_traits>
#include <vector>

#include "accum.h"
#include "internal.h"
#include "layer_ops.h"
#include "search.h"
#include "wave.h"

namespace iam {

constexpr float kScale = 100000.0f;   // bucketMul.cl:17

__device__ __forceinline__ float h2f(uint32_t bits16)
{
    return __half2float(__ushort_as_half((unsigned short)(bits16 & 0xffffu)));
}

// A workgroup of NT threads holds the 4096 inputs the cutoff sees, VPT =
// 4096 / NT consecutive ones per thread (thread tid: [VPT*tid, VPT*tid+VPT)).
template <int VPT>
__device__ __forceinline__ void load_f32(const float* __restrict__ p, float (&v)[VPT])
{
    const float4* q = reinterpret_cast<const float4*>(p + threadIdx.x * VPT);
#pragma unroll
    for (int k = 0; k < VPT / 4; k++) {
        const float4 a = q[k];
        v[4 * k] = a.x;
        v[4 * k + 1] = a.y;
        v[4 * k + 2] = a.z;
        v[4 * k + 3] = a.w;
    }
}

template <int VPT>
__device__ __forceinline__ void load_f64(const double* __restrict__ p, double (&v)[VPT])
{
    const double2* q = reinterpret_cast<const double2*>(p + threadIdx.x * VPT);
#pragma unroll
    for (int k = 0; k < VPT / 2; k++) {
        const double2 a = q[k];
        v[2 * k] = a.x;
        v[2 * k + 1] = a.y;
    }
}

// VPT fp16 values as VPT/2 words (value k in the half k & 1 of word k >> 1)
template <int VPT>
__device__ __forceinline__ void load_h16(const uint16_t* __restrict__ p, uint32_t (&w)[VPT / 2])
{
    const uint4* q = reinterpret_cast<const uint4*>(p + threadIdx.x * VPT);
#pragma unroll
    for (int k = 0; k < VPT / 8; k++) {
        const uint4 a = q[k];
        w[4 * k] = a.x;
        w[4 * k + 1] = a.y;
        w[4 * k + 2] = a.z;
        w[4 * k + 3] = a.w;
    }
}

template <int VPT>
__device__ __forceinline__ float half_at(const uint32_t (&w)[VPT / 2], int k)
{
    return h2f(w[k >> 1] >> ((k & 1) * 16));
}

template <int VPT>
__device__ __forceinline__ void store_f32(float* __restrict__ p, const float (&v)[VPT])
{
    float4* q = reinterpret_cast<float4*>(p + threadIdx.x * VPT);
#pragma unroll
    for (int k = 0; k < VPT / 4; k++) q[k] = make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
}

// imp = 1e5 * |x * probe| (bucketMul.cl:101-117) of the thread's inputs
template <int VPT>
__device__ __forceinline__ void importances(const float (&xs)[VPT], const uint32_t (&pw)[VPT / 2], float (&v)[VPT])
{
#pragma clang fp contract(off)
#pragma unroll
    for (int k = 0; k < VPT; k++) v[k] = __fmul_rn(kScale, fabsf(__fmul_rn(xs[k], half_at<VPT>(pw, k))));
}

// rmsNorm32fast (aux.cl:156-196) of a 4096-vector by one workgroup, in the
// reference's fp32 order: 16 consecutive squares summed in order (with 8
// values per thread, the even lane's running sum continues in the odd
// lane), then the 256-way tree (pairs j, j + st for st = 128 .. 1: the
// partial sums go through LDS, then every wave runs the tree on its own),
// scale = 1/sqrt(sum/4096 + eps) rounded from double, then the fp16 gain
// (mul16x32, aux.cl:434-440).  v holds the thread's inputs on entry and the
// normalized values on exit; gw its gains.  s_part: 256 floats of scratch
// nothing writes again before a later barrier.
template <int VPT>
__device__ __forceinline__ void block_rmsnorm4096(float (&v)[VPT], const uint32_t (&gw)[VPT / 2], float eps,
                                                  float* s_part)
{
#pragma clang fp contract(off)
    static_assert(VPT == 16 || VPT == 8, "16 or 8 values per thread");
    const int tid = threadIdx.x;
    float sq = 0.0f;
    if constexpr (VPT == 8) {
        float lo = 0.0f;
#pragma unroll
        for (int k = 0; k < VPT; k++) lo = __fadd_rn(lo, __fmul_rn(v[k], v[k]));
        sq = dpp_f<0x111>(0.0f, lo);   // the even neighbour's sum (row_shr:1)
#pragma unroll
        for (int k = 0; k < VPT; k++) sq = __fadd_rn(sq, __fmul_rn(v[k], v[k]));
        if (tid & 1) s_part[tid >> 1] = sq;
    } else {
#pragma unroll
        for (int k = 0; k < VPT; k++) sq = __fadd_rn(sq, __fmul_rn(v[k], v[k]));
        s_part[tid] = sq;
    }
    __syncthreads();
    // lane l takes part[l] + part[l+128] and part[l+64] + part[l+192]
    // (st = 128), their sum (st = 64), then st = 32, 16 as shuffles and
    // st = 8 .. 1 within 16-lane rows by DPP row_shl; lane 0 holds the total
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
#pragma unroll
    for (int k = 0; k < VPT; k++) v[k] = __fmul_rn(half_at<VPT>(gw, k), __fmul_rn(v[k], scale));
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

__device__ __forceinline__ float block_cutoff(const float* __restrict__ x, const uint16_t* __restrict__ probes,
                                              int quantile, SearchLds<4>& L)
{
    constexpr int VPT = kCutVPT;
    float xs[VPT], v[VPT];
    uint32_t pw[VPT / 2];
    load_h16<VPT>(probes, pw);
    load_f32<VPT>(x, xs);
    importances<VPT>(xs, pw, v);
    return search_cutoff<4>(v, quantile, L);
}

__global__ __launch_bounds__(kCutThreads) void k_cutoff(CutoffArgs a)
{
    __shared__ SearchLds<4> L;
    const CutoffDesc& d = a.d[blockIdx.x];
    const float cut = block_cutoff(d.x, d.probes, d.quantile, L);
    if (threadIdx.x == 0) d.cutoff[0] = cut;
}

// ------------------------------------------------------------- dispatch ---
// The selected-row list of the parity queries: prepareDispatch
// (bucketMul.cl:351-386) per chunk of 256 inputs, rows in ascending order.
// Block-structured selection (the thesis's future work, p.42-43): rank k
// of every input of a block of blk consecutive inputs is selected when rank
// k of any of them passes the cutoff, i.e. when the block's largest rank-k
// importance does.  The block's inputs sit in consecutive lanes (slices
// start at multiples of blk), so an OR over the lane group does it; lanes
// past the slice contribute nothing.  NaN importances pass for no input.
__device__ __forceinline__ uint32_t block_select(uint32_t mask, int blk, bool valid)
{
    uint32_t m = valid ? mask : 0u;
    for (int o = 1; o < blk; o <<= 1) m |= (uint32_t)__shfl_xor((int)m, o, 64);
    return valid ? m : 0u;
}

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
    int sel_block;            // inputs per selection block (1: per row)
};

__global__ __launch_bounds__(kCutThreads) void k_dispatch(DispatchDesc d)
{
#pragma clang fp contract(off)
    __shared__ SearchLds<4> L;
    __shared__ int s_wsum[4];
    const int g = (int)blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    block_cutoff(d.x, d.probes, d.quantile, L);
    __syncthreads();
    const float cutoff = L.cut;
    if (g == 0 && tid == 0) d.cutoff[1] = cutoff;   // cross-checked against the search launch's cutoff[0]

    const int i = g * kChunkInputs + tid;
    const int r0 = i * 16;
    uint32_t mask = 0;
    float xi = 0.0f;
    if (i < d.in_size && r0 < d.rows) {
        xi = d.x[i];
        uint32_t sv[16];
        const uint16_t* st = d.stats + (size_t)r0 * d.stats_stride;
#pragma unroll
        for (int kk = 0; kk < 16; kk++) {
            const int rr = min(r0 + kk, d.rows - 1) - r0;
            sv[kk] = st[(size_t)rr * d.stats_stride + d.stats_channel];
        }
#pragma unroll
        for (int kk = 0; kk < 16; kk++) {
            const float prod = __fmul_rn(xi, h2f(sv[kk]));
            const float imp = __fmul_rn(kScale, fabsf(prod));
            if (imp >= cutoff && r0 + kk < d.rows) mask |= 1u << kk;   // bucketMul.cl:380
        }
    }
    if (d.sel_block > 1) {
        mask = block_select(mask, d.sel_block, i < d.in_size && r0 < d.rows);
        const int left = d.rows - r0;
        if (left < 16) mask &= left > 0 ? (1u << left) - 1u : 0u;
    }
    const int cnt = __popc(mask);
    const int incl = wave_incl_sum(cnt);
    if (lane == 63) s_wsum[wave] = incl;
    __syncthreads();
    int woff = 0;
    for (int w = 0; w < wave; w++) woff += s_wsum[w];
    const int total = s_wsum[0] + s_wsum[1] + s_wsum[2] + s_wsum[3];
    uint2* out = d.list + (size_t)g * kChunkRows + (woff + incl - cnt);
    const uint32_t xb = __float_as_uint(xi);
    while (mask) {
        const int kk = __ffs(mask) - 1;
        mask &= mask - 1;
        *out++ = make_uint2((uint32_t)(r0 + kk), xb);
    }
    if (tid == 0) d.counts[g] = (uint32_t)total;
}

// ----------------------------------------------------------------- walk ---
// Blocks are dealt to the 8 XCDs round robin (block b -> XCD b % 8).  Remap
// so that consecutive work items (the column tiles of one row slice, which
// read the same stats, inputs and neighbouring lines of the same rows) land
// on the same XCD and share its L2.
__device__ __forceinline__ int xcd_remap(int b, int nblocks)
{
    const int q = nblocks >> 3, r = nblocks & 7;
    const int xcd = b & 7, idx = b >> 3;
    return xcd < r ? xcd * (q + 1) + idx : r * (q + 1) + (xcd - r) * q + idx;
}

// 16 bytes of the weight stream, loaded non-temporally: read once per
// launch, the rows would otherwise evict the small vectors every launch
// reads first (inputs, probes, gains, stats, the KV cache) from L2 and the
// Infinity Cache
__device__ __forceinline__ uint4 load_stream(const uint16_t* p)
{
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 r = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(r.x, r.y, r.z, r.w);
}

// LDS addresses as 32-bit byte offsets (a generic pointer into LDS makes the
// compiler form every slot address with a 64-bit multiply-add)
template <typename T>
using lds_ptr = __attribute__((address_space(3))) T*;
template <typename T>
__device__ __forceinline__ uint32_t lds_offset(T* p)
{
    return (uint32_t)(uintptr_t)(lds_ptr<T>)p;
}
template <typename T>
__device__ __forceinline__ void lds_add(uint32_t byte_offset, int elem, T v)
{
    __hip_atomic_fetch_add((lds_ptr<T>)(uintptr_t)byte_offset + elem, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// column tiles of the walk: 128 columns (256-byte row segments) or 64
// (half the flush's atomic adds per workgroup, for launches whose walk is
// short next to their flush)
constexpr int kTileColsWide = 128;
constexpr int kTileColsNarrow = 64;

struct WalkDesc {
    const uint16_t* W;        // rows of the expert: W[row * C + col]
    float* x;                 // the input (kInX/kInCutoff) or where block 0 stores the computed one
    const uint16_t* stats;    // row 0 of the expert
    const uint16_t* probes;   // probes of the expert
    float* cutoff;
    // or null: the search's hint, the same matrix's cutoff of the previous
    // step (read at the start, written by work item 0 once it has the cutoff)
    float* hint;
    uint32_t* slice_count;    // [P]: rows selected per slice (written by the tile-0 workgroups)
    void* acc;                // [16*C] accumulators
    void* acc2;               // or null: the odd slices' accumulators (kFinNone)
    float* y;                 // kFinStore: outputs; kFinSilu: gate / up values (may be null)
    uint32_t* tile_ctr;       // [T] arrival counters (finalize modes)
    int quantile;
    int stats_stride;
    int stats_channel;
    int rows;                 // R
    int n_in;                 // inputs walked: min(ceil(R/16), in_size)
    int C;
    int IPS;                  // inputs per slice (<= threads per workgroup)
    int P;                    // slices
    int T;                    // column tiles
    int nblocks;              // blocks of this matrix (P * T); the grid's x may be larger
    int expected;             // workgroups that flush into one tile (finalize modes)
};

struct WalkArgs {
    WalkDesc d[kMaxMulti];
    int first[kMaxMulti];     // the first work item of each matrix (the grid's total past the last matrix)
    int n;
    int in_mode;
    const float* h;
    const void* res_acc;
    float* h_out;
    const uint16_t* gain;
    float eps;
    const uint16_t* embed;
    const int* token;
    const float* embed_scale;
    int vocab;
    const void* attn_acc;
    int attn_lofs;            // offset of the softmax denominators in attn_acc
    int fin;
    float* silu_out;
    uint32_t* pick_ctr;
    uint2* tile_cand;
    int* token_out;
    int* pos;
    int* hist;
    int hist_len;
    void* final_zero;
    int final_zero_n;
    void* zero_p[2];
    int zero_n[2];
    unsigned long long* counters;
    int sel_block;            // inputs per selection block (1: the reference's per-row selection)
};

// A pointer the compiler no longer sees as global (after an asm) marked
// global again, so that its loads stay global loads (a flat load also counts
// against the LDS wait counter)
template <typename T>
__device__ __forceinline__ T* as_global(uint64_t u)
{
    return (T*)(__attribute__((address_space(1))) T*)u;
}

// The arguments the first vector loads of a walk block need (the matrices'
// probes and x, the input mode's pointers, the block bases) are read from
// fixed argument offsets and pinned in scalar registers, so they arrive in
// one batch of scalar loads with one wait; the block's matrix then picks
// among them.  A field read through the block's matrix index would cost a
// second round trip before the first vector load; the other fields are read
// that way, and used only once the input and the search are under way.


// Loads of the selection: the 16 stats (channel stats_channel) of the rows
// of the slice input the thread holds (sel_input) and, when the slice's
// inputs are not computed in registers, its x (from memory, or from the
// attention accumulators).  Issued before the cutoff is known so that their
// latency overlaps the search; the raw words are kept.  Layouts: compact
// stats (stride 1, 2 x 16 bytes), the reference's [R][4] with channel 3
// (8 x 16 bytes), otherwise 16 scalar loads.
struct SelLoads {
    uint4 raw[8];
    uint32_t sv[16];
    float xi;
    double an, ad;   // attention input: o and the softmax denominator (divided after the search)
    bool attn;
    int kind;        // 0: stride 1, 1: stride 4 channel 3, 2: scalar
};

// where the selection reads the stats and x of the block's matrix
struct SelSrc {
    const uint16_t* stats;
    const float* x;
    int stride;
    int channel;
    int rows;
};

enum XSrc : int { kXRegs = 0, kXMem = 1, kXAttn = 2 };

// A load issued where the source puts it.  The barriers of the search
// order LDS only, so a plain load whose value is first used after them is
// moved down to that use, and its latency then follows the cutoff instead of
// overlapping the search.  A relaxed atomic load is the same load
// instruction (no cache bypass at workgroup scope), but the compiler keeps
// it in place.
template <typename T>
__device__ __forceinline__ T load_early(const T* p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ uint4 load_early16(const void* p)
{
    const uint64_t* q = reinterpret_cast<const uint64_t*>(p);
    const uint64_t lo = load_early(q), hi = load_early(q + 1);
    return make_uint4((uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32));
}

// The slice input thread tid holds in the selection: waves 1.. take the
// first ones and wave 0 the last, so that for slices of up to 64 * (NW - 1)
// inputs the waves that leave the cutoff search early compute the rows'
// importances, and list the rows certain to be selected, while wave 0
// finishes it.  Consecutive inputs stay in
// consecutive lanes of one wave (blocks of block mode included).
template <int NT>
__device__ __forceinline__ int sel_input(int tid)
{
    return (tid + NT - 64) & (NT - 1);
}

template <int NT>
__device__ __forceinline__ void select_load(const SelSrc& d, const WalkArgs& a, int i0, int ni, int xsrc,
                                            SelLoads& L)
{
    const int li = sel_input<NT>(threadIdx.x);
    L.xi = 0.0f;
    L.an = 0.0;
    L.ad = 1.0;
    L.attn = xsrc == kXAttn;
    const int i = i0 + min(li, ni - 1);   // threads past the slice re-read its last input
    const int r0 = i * 16;
    const uint16_t* base = d.stats + (size_t)i0 * 16 * d.stride;
    const bool aligned = (((uintptr_t)base) & 15) == 0 && (d.rows & 15) == 0;
    if (xsrc == kXMem) {
        L.xi = __uint_as_float(load_early(reinterpret_cast<const uint32_t*>(d.x) + i));
    } else if (xsrc == kXAttn) {
        const uint64_t* A = reinterpret_cast<const uint64_t*>(a.attn_acc);
        L.an = __longlong_as_double((long long)load_early(A + i));
        L.ad = __longlong_as_double((long long)load_early(A + a.attn_lofs + (i >> 7)));
    }
    const uint16_t* st = d.stats + (size_t)r0 * d.stride;
    if (aligned && d.stride == 1) {
        L.kind = 0;
        L.raw[0] = load_early16(st);
        L.raw[1] = load_early16(st + 8);
    } else if (aligned && d.stride == 4 && d.channel == 3) {
        L.kind = 1;
        const uint32_t* p = reinterpret_cast<const uint32_t*>(st);
#pragma unroll
        for (int k8 = 0; k8 < 8; k8++) L.raw[k8] = make_uint4(0u, load_early(p + 4 * k8 + 1), 0u, load_early(p + 4 * k8 + 3));
    } else {
        L.kind = 2;
#pragma unroll
        for (int kk = 0; kk < 16; kk++) {
            const int rr = min(r0 + kk, d.rows - 1) - r0;
            L.sv[kk] = st[(size_t)rr * d.stride + d.channel];
        }
    }
}

// The importances of the 16 rows of the thread's input, 1e5 * |x * stat|
// in the fp32 operations of prepareDispatch (bucketMul.cl:351-386), and the
// bits of its rows inside the expert (none for threads past the slice).
// They need only the loads and x (s_x, published by an earlier barrier, when
// x_lds), so they are computed before the cutoff is known.  Without x_lds
// the thread's x goes to s_x[input] (0 past the slice) for the walk; a
// barrier follows before it is read.
template <int NT>
__device__ __forceinline__ void select_prepare(const SelSrc& d, int i0, int ni, const SelLoads& L, float* s_x,
                                               bool x_lds, float (&imp)[16], uint32_t& vbits)
{
#pragma clang fp contract(off)
    const int li = sel_input<NT>(threadIdx.x);
    float xi = L.xi;
    vbits = 0u;
#pragma unroll
    for (int kk = 0; kk < 16; kk++) imp[kk] = 0.0f;
    if (li < ni) {
        if (x_lds) xi = s_x[li];
        else if (L.attn) xi = (float)(L.an / L.ad);
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
#pragma unroll
        for (int kk = 0; kk < 16; kk++) {
            const float prod = __fmul_rn(xi, h2f(sv[kk]));
            imp[kk] = __fmul_rn(kScale, fabsf(prod));
        }
        const int left = d.rows - (i0 + li) * 16;   // rows of this input inside the expert (>= 1)
        vbits = left >= 16 ? 0xffffu : (1u << left) - 1u;
    }
    if (!x_lds) s_x[li] = li < ni ? xi : 0.0f;
}

// The selection of slice p (prepareDispatch, bucketMul.cl:351-386): a row is
// selected iff its importance >= cutoff (NaN never is), so the selected set
// is the dispatch kernel's.  Block mode (blk > 1): rank k of every input of
// a block is selected when rank k of any of them passes (block_select), rows
// outside the expert excepted.  The rows of the thread's input that are
// selected and were not listed before (importance below `listed`: NaN when
// none were), as a 16-bit mask (bit k: rank k).
__device__ __forceinline__ uint32_t select_mask(float cutoff, float listed, const float (&imp)[16], uint32_t vbits,
                                                int blk)
{
    uint32_t mask = 0;
#pragma unroll
    for (int kk = 0; kk < 16; kk++)
        if (imp[kk] >= cutoff && !(imp[kk] >= listed)) mask |= 1u << kk;   // bucketMul.cl:380
    mask &= vbits;
    if (blk > 1) mask = block_select(mask, blk, vbits != 0u) & vbits;
    return mask;
}

// The wave's rows of `mask` (bit k: row rowb + k of the thread's input)
// appended to the slice's row list: one LDS atomic reserves the wave's
// slots, and each lane writes its rows there, ascending, after those of the
// lanes before it (a DPP prefix sum), so that rows next to each other in the
// weights stay together in the list and a walk load's rows share DRAM pages.
// Where the waves' blocks stand in the list is free (each row's products are
// added wherever it stands); its length is *cnt once every wave has
// appended (after a barrier).
__device__ __forceinline__ void wave_append_rows(uint32_t mask, uint32_t rowb, uint16_t* list, uint32_t* cnt)
{
    const int c = __popc(mask);
    const int incl = wave_incl_sum(c);
    const int total = __builtin_amdgcn_readlane(incl, 63);
    if (total == 0) return;
    uint32_t base = 0;
    if ((threadIdx.x & 63) == 0) base = atomicAdd(cnt, (uint32_t)total);
    uint32_t off = __builtin_amdgcn_readfirstlane(base) + (uint32_t)(incl - c);
    while (mask) {
        const int kk = __ffs(mask) - 1;
        mask &= mask - 1;
        list[off++] = (uint16_t)(rowb | (uint32_t)kk);
    }
}

// first maximum (test_generation.cpp:235, 276) of (value, index) pairs
__device__ __forceinline__ void take_max(float& bv, int& bi, float v, int i)
{
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

// Selection + walk + flush.  Workgroup (input slice p, column tile t) owns
// the inputs [p*IPS, (p+1)*IPS) and the TC columns [TC*t, TC*t + TC)
// (TC = 128 or 64).
//
// Walk: lane = q*LPR + j (LPR = TC/8 lanes per row) reads 16 bytes (columns
// 8j..8j+7) of row q of a group of RPI = 64/LPR selected rows, so one load
// instruction fetches the 2*TC-byte tile segments of RPI rows.  Wave w takes
// the groups w, w + NW, w + 2NW, ...  Each packed weight is added, as the
// product x * w in the accumulator type (exact in fp64), to the workgroup's
// accumulator of its output (column c, position bits & 15) with a
// non-returning LDS atomic add (bucketMul.cl:430-445 adds the product with a
// plain += per work-item); the waves share the tile (LDS atomics of
// different waves on one address cost no more than on different ones).  The
// accumulator of (column 8j+e, position pos) is slot pos*TC + e*LPR + j of
// tile copy q % NCOPY (NCOPY = 128/TC copies, 64 bytes apart in bank
// terms): whatever the positions of
// the 64 lanes' weights (each weight carries its own), an instruction's
// lanes map to bank pairs set by j and the copy alone, so the walk's LDS
// atomics never conflict beyond the 4 rows sharing a bank pair (the fewest
// passes 64 8-byte accumulators need).  Two batches of rows are in flight
// per wave.  Rows past the end of the list re-read the last selected row
// with x = 0, so every load of a batch is unconditional.
//
// Flush: sums of the tile copies, staged in output order (column-major, col*16 + pos, the reference's output index,
// bucketMul.cl:442-445), one atomic add per output and workgroup.
template <typename Acc, int NW, int UNR, int TC>
__global__ __launch_bounds__(64 * NW) void k_walk(WalkArgs a)
{
#pragma clang fp contract(off)
    constexpr int NT = 64 * NW;
    static_assert(TC == 64 || TC == 128, "64- or 128-column tiles");
    constexpr int TOUT = TC * 16;                           // outputs of a column tile
    constexpr int LPR = TC / 8;                             // lanes per row
    constexpr int RPI = 64 / LPR;                           // rows per wave load
    constexpr int NCOPY = 128 / TC;                         // tile copies (rows alternate)
    constexpr int CSLOTS = 16 * TC + (NCOPY > 1 ? 8 : 0);   // one copy (+64 bytes: the next one's banks)
    constexpr int STAGE = TOUT + TOUT / 128;                // the flush's staging copy
    constexpr int TSLOTS = NCOPY * CSLOTS > STAGE ? NCOPY * CSLOTS : STAGE;
    constexpr int GSTRIDE = NW * UNR;                       // groups per workgroup batch
    static_assert(NW == 4 || NW == 8, "4 or 8 waves");
    constexpr int VPT = IAM_PROBES_COUNT / NT;              // inputs of the cutoff per thread
    static_assert(TOUT % NT == 0, "flush mapping");
    // the tile holds fp64 sums in both modes: Acc is the precision of
    // the products (fp32 mode: the reference's fp32 products), and LDS fp64
    // atomic adds run many times faster than fp32 ones on this part
    using Tile = double;
    __shared__ __align__(16) Tile tiles[TSLOTS];   // the tile copies, then the staging copy
    // the search's scratch (the windowed search's, or the radix search's
    // when that one declines)
    constexpr int kSearchBytes = sizeof(SearchLds<NW>) > sizeof(WindowLds<NW>) ? sizeof(SearchLds<NW>) : sizeof(WindowLds<NW>);
    __shared__ __align__(16) uint4 s_search[(kSearchBytes + 15) / 16];
    // the slice's selected rows (slice-local ids input*16 + rank), in the
    // order the waves append them, and their number
    __shared__ __align__(16) uint16_t s_row[NT * 16];
    __shared__ uint32_t s_nrow;
    __shared__ uint32_t s_met;   // waves 1.. that have listed their certain rows
    __shared__ __align__(16) float s_x[NT];
    __shared__ float s_part[256];
    __shared__ int s_last;
    __shared__ float s_bv[NW];
    __shared__ int s_bi[NW];
    SearchLds<NW>& SL = *reinterpret_cast<SearchLds<NW>*>(s_search);
    WindowLds<NW>& WL = *reinterpret_cast<WindowLds<NW>*>(s_search);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    // The grid holds exactly the launch's blocks (no idle ones to take CU
    // slots from real ones): block ids are remapped so that consecutive work
    // items sit on one XCD, and the work items are dealt to the matrices in
    // ranges starting at first[k].  The reads the first vector loads need --
    // the range starts, every matrix's probes and x, the input mode's
    // arguments -- go out as one batch of scalar loads and are pinned there
    // (a later first use would cost another round trip to the arguments,
    // which the weight stream keeps out of the caches); the block's matrix
    // then picks among them.
    int nblk = (int)gridDim.x, f1 = a.first[1], f2 = a.first[2], mode = a.in_mode, attn_lofs = a.attn_lofs;
    uint64_t pr0 = (uint64_t)a.d[0].probes, pr1 = (uint64_t)a.d[1].probes, pr2 = (uint64_t)a.d[2].probes;
    uint64_t x0 = (uint64_t)a.d[0].x, x1 = (uint64_t)a.d[1].x, x2 = (uint64_t)a.d[2].x;
    uint64_t u_h = (uint64_t)a.h, u_res = (uint64_t)a.res_acc, u_gain = (uint64_t)a.gain, u_attn = (uint64_t)a.attn_acc;
    // Fields read only later (the selection mode, the walk's rows, the
    // flush's accumulators, the zeroing and counting pointers) are touched
    // in the same batch: every 64-byte line of the descriptors and of the
    // trailing arguments is then in the scalar cache, and their later reads
    // do not each wait for a round trip to argument memory.
    asm volatile(""
                 : "+s"(nblk), "+s"(f1), "+s"(f2), "+s"(mode), "+s"(attn_lofs), "+s"(pr0), "+s"(pr1), "+s"(pr2), "+s"(x0), "+s"(x1),
                   "+s"(x2), "+s"(u_h), "+s"(u_res), "+s"(u_gain), "+s"(u_attn)
                 : "s"(a.d[0].W), "s"(a.d[0].acc), "s"(a.d[1].W), "s"(a.d[1].acc), "s"(a.d[2].W), "s"(a.d[2].acc),
                   "s"(a.d[2].expected), "s"(a.final_zero), "s"(a.counters), "s"(a.sel_block));
    const int wi = xcd_remap((int)blockIdx.x, nblk);
    const int k = wi >= f2 ? 2 : wi >= f1 ? 1 : 0;
    const int b = wi - (k == 2 ? f2 : k == 1 ? f1 : 0);
    const uint64_t u_pr = k == 2 ? pr2 : k == 1 ? pr1 : pr0, u_x = k == 2 ? x2 : k == 1 ? x1 : x0;
    const uint16_t* probes = as_global<const uint16_t>(u_pr);
    float* dx = as_global<float>(u_x);
    const float* a_h = as_global<const float>(u_h);
    const void* a_res = as_global<const double>(u_res);
    const uint16_t* a_gain = as_global<const uint16_t>(u_gain);
    const void* a_attn = as_global<const double>(u_attn);
    const WalkDesc& d = a.d[k];
    const bool norm = mode == kInNorm || mode == kInResNorm || mode == kInEmbedNorm;
    const bool regs = norm || mode == kInAttn;           // x[0:4096] computed in registers

    // ---- prologue: every global load is issued before any is used.
    // Each array is read only in the modes that load it, and none has a
    // default: the compiler cannot tell the modes apart, and a default it
    // sets on the other modes' path (where that path merges with the
    // loading one) makes those modes wait there for every load in flight.
    float xs[VPT];
    double ra[VPT], rt[VPT];   // the residual delta; the attention sums (apart: see below)
    uint32_t pw[VPT / 2], gw[VPT / 2], ew[VPT / 2];
    float sc[VPT];
    double lsum;
    bool tok_ok = false;
    float cutoff = 0.0f;
    float hint;   // thread 0, with a hint: the search's hint
    if (mode == kInCutoff) {
        cutoff = *d.cutoff;
    } else {
        if (tid == 0 && d.hint) hint = load_early(d.hint);
        load_h16<VPT>(probes, pw);
        if (mode == kInX) load_f32<VPT>(dx, xs);
        if (mode == kInNorm || mode == kInResNorm) load_f32<VPT>(a_h, xs);
        if (mode == kInResNorm && a_res) load_f64<VPT>(reinterpret_cast<const double*>(a_res), ra);
        if (mode == kInEmbedNorm) {
            const int tok = *a.token;
            tok_ok = tok >= 0 && tok < a.vocab;
            if (tok_ok) load_h16<VPT>(a.embed + (size_t)tok * kProbes, ew);
            if (a.embed_scale) load_f32<VPT>(a.embed_scale, sc);
        }
        if (norm) load_h16<VPT>(a_gain, gw);
        if (mode == kInAttn) {
            const double* A = reinterpret_cast<const double*>(a_attn);
            // into registers of their own: loads into ra here would first
            // wait for the residual mode's (the compiler cannot tell the
            // modes apart), and with them for every load in flight
            load_f64<VPT>(A, rt);
            lsum = A[attn_lofs + ((tid * VPT) >> 7)];   // the head of the thread's inputs
        }
    }
    // the tile is cleared while the loads are in flight (the search's
    // barriers order the clearing before the walk's adds)
    {
        uint4* tz = reinterpret_cast<uint4*>(tiles);
        constexpr int kTileVecs = TSLOTS * (int)sizeof(Tile) / 16;
        static_assert(TSLOTS * sizeof(Tile) % 16 == 0, "whole 16-byte stores");
#pragma unroll
        for (int i = 0; i < (kTileVecs + NT - 1) / NT; i++)
            if (i * NT + tid < kTileVecs) tz[i * NT + tid] = make_uint4(0u, 0u, 0u, 0u);
    }
    if (mode != kInCutoff) window_clear<NW>(WL);
    if (tid == 0) {
        s_nrow = 0u;
        s_met = 0u;
    }
    // the block's slice and column tile (from the descriptor read through k)
    const int w = b;
    const int p = w / d.T;
    const int t = w - p * d.T;
    const int i0 = p * d.IPS;
    const int ni = min(d.IPS, d.n_in - i0);
    const SelSrc ss{d.stats, dx, d.stats_stride, d.stats_channel, d.rows};
    const int quantile = d.quantile;
    const bool slice_regs = regs && i0 + ni <= kProbes;  // x of the slice among the computed ones
    const bool first = w == 0 && k == 0;
    SelLoads L;
    select_load<NT>(ss, a, i0, ni, slice_regs ? kXRegs : (mode == kInAttn ? kXAttn : kXMem), L);

    // ---- the input
    if (mode != kInCutoff) {
        if (mode == kInResNorm && a_res) {
#pragma unroll
            for (int k2 = 0; k2 < VPT; k2++) xs[k2] = __fadd_rn(xs[k2], (float)ra[k2]);   // add32
        }
        if (mode == kInEmbedNorm) {   // fetchRow16to32 (aux.cl:442-452), then the optional channel scale
#pragma unroll
            for (int k2 = 0; k2 < VPT; k2++)
                xs[k2] = __fmul_rn(tok_ok ? half_at<VPT>(ew, k2) : 0.0f, a.embed_scale ? sc[k2] : 1.0f);
        }
        if (mode == kInAttn) {
#pragma unroll
            for (int k2 = 0; k2 < VPT; k2++) xs[k2] = (float)(rt[k2] / lsum);
        }
        if ((mode == kInResNorm || mode == kInEmbedNorm) && first && a.h_out) store_f32<VPT>(a.h_out, xs);
    }
    // one value for the whole workgroup (work item 0 of the matrix may
    // rewrite the hint meanwhile), published by the barrier before the search
    if (tid == 0 && d.hint) WL.hint = hint;
    if (norm) block_rmsnorm4096<VPT>(xs, gw, a.eps, s_part);
    if (regs) {
        if (first && dx) store_f32<VPT>(dx, xs);
        if (slice_regs) {
#pragma unroll
            for (int k2 = 0; k2 < VPT; k2++) {
                const int i = tid * VPT + k2 - i0;
                if (i >= 0 && i < ni) s_x[i] = xs[k2];
            }
        }
    }

    // The walk's lane geometry (lane = q*LPR + j reads 16 bytes, columns
    // 8j..8j+7, of row q of each group of RPI rows), and the first batch of
    // a wave, loaded before the cutoff where the rows certain to be selected
    // fill every wave's first batch (below).
    const int j = lane % LPR;
    const int q = lane / LPR;
    const int col0 = t * TC + j * 8;
    const bool whole = (d.C & 7) == 0;
    const uint16_t* wb = d.W + (size_t)i0 * 16 * d.C + col0;
    uint4 pva[UNR];
    Acc pxa[UNR];
    bool pre = false;
    // After waves 1.. have listed their certain rows (they then meet at an
    // LDS counter; a bounded wait), the list's first UNR*NW*RPI entries are
    // final when that many rows are listed: every wave's first batch (rows
    // (wave + u*NW)*RPI + q) is among them, so its loads go out now instead
    // of after the list barrier.  They are the loads the walk issues first,
    // unchanged; x = 1 * s_x of their inputs (written before the listing).
    auto prefetch = [&]() {
        if (!whole || a.sel_block != 1) return;
        bool met = false;
        for (int spin = 0; spin < 4096; spin++) {
            if (__hip_atomic_load(&s_met, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= (uint32_t)(NW - 1)) {
                met = true;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");   // the entries after the count
        const int na = (int)__hip_atomic_load(&s_nrow, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (!met || na < UNR * NW * RPI) return;
        pre = true;
        if (col0 >= d.C) return;
#pragma unroll
        for (int u = 0; u < UNR; u++) {
            const int rl = s_row[(wave + u * NW) * RPI + q];
            pxa[u] = (Acc)s_x[rl >> 4];
            pva[u] = load_stream(wb + __umul24(rl, d.C));
        }
    };

    // ---- cutoff, and the slice's rows.  While wave 0 finishes the windowed
    // search, the other waves compute the importances of their inputs' rows
    // and (per-row selection) append the rows certain to be selected, those
    // whose importance reaches the window's upper bound hi > cutoff
    // (cutoff_upper), to the row list; once the cutoff is known every wave
    // appends its other selected rows, and one barrier publishes the list.
    // When the windowed search declines, the radix search runs.
    float imp[16];
    uint32_t vbits;
    float listed = __int_as_float(0x7fc00000);   // this wave's rows from this importance up are listed
    const uint32_t rowb = (uint32_t)sel_input<NT>(tid) << 4;
    bool hint_hit = false;   // the search's hinted window held the cutoff's ranks
    if (mode != kInCutoff) {
        float v[VPT];
        importances<VPT>(xs, pw, v);
        if (!norm) __syncthreads();   // the window's histograms are clear (the norm's barrier orders them otherwise)
        float cut_w;
        const int found = search_window<NW>(v, quantile, d.hint != nullptr, WL, cut_w, hint_hit, [&](float hi) {
            select_prepare<NT>(ss, i0, ni, L, s_x, slice_regs, imp, vbits);
            // wave 0 comes here at the end of the search: its rows wait for the cutoff
            if (wave != 0 && a.sel_block == 1) {
                uint32_t m = 0;
#pragma unroll
                for (int kk = 0; kk < 16; kk++)
                    if (imp[kk] >= hi) m |= 1u << kk;
                wave_append_rows(m & vbits, rowb, s_row, &s_nrow);
                listed = hi;
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");   // the list entries, then the count
                if (lane == 0) atomicAdd(&s_met, 1u);
            }
            prefetch();
        });
        if (found == 1) {
            cutoff = cut_w;
        } else {
            __syncthreads();   // every wave is done with the window's scratch
            search_cutoff<NW>(v, quantile, SL);
            if (found == 0) select_prepare<NT>(ss, i0, ni, L, s_x, slice_regs, imp, vbits);
            __syncthreads();   // wave 0 has stored the cutoff
            cutoff = SL.cut;
        }
        if (w == 0 && tid == 0) {
            d.cutoff[0] = cutoff;
            if (d.hint) d.hint[0] = cutoff;
        }
    } else {
        select_prepare<NT>(ss, i0, ni, L, s_x, slice_regs, imp, vbits);
        __syncthreads();   // the list's count is clear before any wave appends
    }
    wave_append_rows(select_mask(cutoff, listed, imp, vbits, a.sel_block), rowb, s_row, &s_nrow);
    __syncthreads();
    const int ns = (int)s_nrow;
    if (t == 0 && tid == 0) {
        d.slice_count[p] = (uint32_t)ns;
        if (a.counters) {
            unsigned long long* cr = a.counters + (p % kCounterLanes) * 4;
            atomicAdd(cr + 0, (unsigned long long)ns * (unsigned long long)d.C * 2ull);
            atomicAdd(cr + 1, (unsigned long long)ns);
            if (p == 0) atomicAdd(cr + 2, 1ull);
            // hinted searches (high half) and those whose window held (low half)
            if (p == 0 && d.hint && mode != kInCutoff) atomicAdd(cr + 3, (1ull << 32) | (hint_hit ? 1ull : 0ull));
        }
    }

    // ---- walk of the selected rows
    if (col0 < d.C) {
        // C % 8 == 0 (whole): one 16-byte load per row; otherwise (rows only
        // 2-byte aligned, a lane's last columns may lie past C) eight 2-byte
        // loads, zero past C (they land in slots the flush does not store)
        const int nc = min(8, d.C - col0);
        const uint32_t tbase =
            lds_offset(tiles) + (uint32_t)((q % NCOPY) * CSLOTS + j) * (uint32_t)sizeof(Tile);
        const int ng = (ns + RPI - 1) / RPI;
        // one instance of the loop per row load shape, so that no branch sits
        // in its steady state
        auto walk_rows = [&](auto whole_tag) {
        constexpr bool WHOLE = decltype(whole_tag)::value;
        // batch g0: rows (g0 + u*NW)*RPI + q, u < UNR, into one register set
        auto issue = [&](int g0, uint4 (&v)[UNR], Acc (&xc)[UNR]) {
            int rl[UNR];
            float xl[UNR];
#pragma unroll
            for (int u = 0; u < UNR; u++) {
                const int idx = (g0 + u * NW) * RPI + q;
                rl[u] = s_row[min(idx, ns - 1)];
                xl[u] = idx < ns ? 1.0f : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < UNR; u++) xc[u] = (Acc)(xl[u] * s_x[rl[u] >> 4]);
            if constexpr (WHOLE) {
#pragma unroll
                for (int u = 0; u < UNR; u++) v[u] = load_stream(wb + __umul24(rl[u], d.C));
            } else {
#pragma unroll
                for (int u = 0; u < UNR; u++) {
                    const uint16_t* rp = wb + __umul24(rl[u], d.C);
                    uint32_t e[8];
#pragma unroll
                    for (int c = 0; c < 8; c++) e[c] = c < nc ? (uint32_t)__builtin_nontemporal_load(rp + c) : 0u;
                    v[u] = make_uint4(e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16), e[6] | (e[7] << 16));
                }
            }
        };
        auto consume = [&](const uint4 (&v)[UNR], const Acc (&xc)[UNR]) {
#pragma unroll
            for (int u = 0; u < UNR; u++) {
                const uint32_t words[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const uint32_t hw = words[e >> 1] >> ((e & 1) * 16);
                    // position bits by one bit-field extract, then one
                    // multiply-add into the slot address
                    uint32_t pos;
                    asm("v_bfe_u32 %0, %1, %2, 4" : "=v"(pos) : "v"(words[e >> 1]), "i"((e & 1) * 16));
                    lds_add<Tile>(__umul24(pos, TC * (uint32_t)sizeof(Tile)) + tbase, e * LPR,
                                  (Tile)(xc[u] * (Acc)h2f(hw)));
                }
            }
        };
        // two batches in flight: the steady state issues unconditionally
        // (so the waits before each batch's use count exactly the other
        // batch's loads) and keeps the phases apart; the tail takes the last
        // one to three batches
        uint4 va[UNR], vb[UNR];
        Acc xa[UNR], xb[UNR];
        int g = wave;
        // the first batch: loaded before the cutoff (pre: ng >= UNR*NW > g), or now
        auto first = [&]() {
            if (pre) {
#pragma unroll
                for (int u = 0; u < UNR; u++) {
                    va[u] = pva[u];
                    xa[u] = pxa[u];
                }
            } else {
                issue(g, va, xa);
            }
        };
        if (g + 3 * GSTRIDE < ng) {
            first();
            issue(g + GSTRIDE, vb, xb);
            do {
                consume(va, xa);
                __builtin_amdgcn_sched_barrier(0);
                issue(g + 2 * GSTRIDE, va, xa);
                __builtin_amdgcn_sched_barrier(0);
                consume(vb, xb);
                __builtin_amdgcn_sched_barrier(0);
                issue(g + 3 * GSTRIDE, vb, xb);
                __builtin_amdgcn_sched_barrier(0);
                g += 2 * GSTRIDE;
            } while (g + 3 * GSTRIDE < ng);
        } else {
            if (g < ng) first();
            if (g + GSTRIDE < ng) issue(g + GSTRIDE, vb, xb);
        }
        if (g < ng) consume(va, xa);
        if (g + 2 * GSTRIDE < ng) issue(g + 2 * GSTRIDE, va, xa);
        if (g + GSTRIDE < ng) consume(vb, xb);
        if (g + 2 * GSTRIDE < ng) consume(va, xa);
        };
        if (whole) walk_rows(std::true_type{});
        else walk_rows(std::false_type{});
    }
    __syncthreads();

    // ---- flush: the tile copies summed in copy order, read in slot order
    // (free of bank conflicts), staged in LDS in output order (col*16 + pos,
    // the reference's output index, bucketMul.cl:442-445; one pad per 128
    // entries keeps the staging writes and the reads after them free of
    // conflicts too), then one atomic add per output and workgroup over
    // consecutive outputs.
    constexpr int OPT = TOUT / NT;
    static_assert(TSLOTS >= STAGE, "the staging copy fits the tiles");
    double* out = reinterpret_cast<double*>((p & 1) && d.acc2 ? d.acc2 : d.acc) + (size_t)t * TOUT;
    const int nout = min(TOUT, (d.C - t * TC) * 16);
    {
        Tile sum[OPT];
#pragma unroll
        for (int k2 = 0; k2 < OPT; k2++) {
            const int sl = tid + k2 * NT;
            Tile sv = tiles[sl];
#pragma unroll
            for (int cc = 1; cc < NCOPY; cc++) sv += tiles[cc * CSLOTS + sl];
            sum[k2] = sv;
        }
        __syncthreads();
#pragma unroll
        for (int k2 = 0; k2 < OPT; k2++) {
            const int sl = tid + k2 * NT;
            const int pos = sl / TC, e = (sl / LPR) & 7, jj = sl % LPR;   // slot pos*TC + e*LPR + j
            const int o = (jj * 8 + e) * 16 + pos;
            tiles[o + (o >> 7)] = sum[k2];
        }
        __syncthreads();
    }
    // In the finalize modes the additions return the old values, and the
    // workgroup waits for all of them before it arrives at the tile
    // counter: every addition is then performed, at the one place where all
    // atomics on that address are ordered, before the last workgroup to
    // arrive takes the sums there with atomic exchanges.  The two modes
    // keep loops of their own: within one loop the compiler merges the two
    // additions into a returning one and waits for each return in turn, a
    // round trip per addition in both modes; here the non-returning
    // additions are issued back to back, and the returning ones are all
    // issued before the first wait.
    // The staged sums are all read before the first addition goes out
    // (an LDS read after it may reuse its registers and wait for it).
    Tile sv[OPT];
#pragma unroll
    for (int k2 = 0; k2 < OPT; k2++) {
        const int o = tid + k2 * NT;                          // col_local*16 + pos
        sv[k2] = tiles[o + (o >> 7)];
    }
    double got[OPT];
    if (a.fin != kFinNone) {
#pragma unroll
        for (int k2 = 0; k2 < OPT; k2++) {
            const int o = tid + k2 * NT;
            got[k2] = 0.0;
            if (o < nout && sv[k2] != (Tile)0)
                got[k2] = __hip_atomic_fetch_add(out + o, (double)sv[k2], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    } else {
#pragma unroll
        for (int k2 = 0; k2 < OPT; k2++) {
            const int o = tid + k2 * NT;
            if (o < nout && sv[k2] != (Tile)0) acc_add(out + o, (double)sv[k2]);
        }
    }
    // accumulators of earlier launches that are read no more (after the
    // prologue: their stores would queue ahead of its loads)
    zero_share<double>(a.zero_p[0], a.zero_n[0], NT);
    zero_share<double>(a.zero_p[1], a.zero_n[1], NT);
    if (a.fin == kFinNone) return;

    // ---- finalize: the last workgroup to flush into tile t
#pragma unroll
    for (int k2 = 0; k2 < OPT; k2++) asm volatile("" ::"v"(got[k2]));   // the returned values are in: every addition is performed
    __syncthreads();
    if (tid == 0)
        s_last = __hip_atomic_fetch_add(d.tile_ctr + t, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 (uint32_t)(d.expected - 1);
    __syncthreads();
    if (!s_last) return;
    if (tid == 0) d.tile_ctr[t] = 0u;
    if (a.fin == kFinSilu) {
        double* g_acc = reinterpret_cast<double*>(a.d[0].acc) + (size_t)t * TOUT;
        double* u_acc = reinterpret_cast<double*>(a.d[1].acc) + (size_t)t * TOUT;
        // every exchange goes out before the first value is used
        double gt[OPT], ut[OPT];
#pragma unroll
        for (int k2 = 0; k2 < OPT; k2++) {
            const int o = tid + k2 * NT;
            gt[k2] = ut[k2] = 0.0;
            if (o < nout) {
                gt[k2] = acc_take(g_acc + o);
                ut[k2] = acc_take(u_acc + o);
            }
        }
        // the values' first use, pinned after the last exchange (the
        // compiler would otherwise convert each one inside its branch and
        // wait there)
#pragma unroll
        for (int k2 = 0; k2 < OPT; k2++) asm volatile("" : "+v"(gt[k2]), "+v"(ut[k2]));
#pragma unroll
        for (int k2 = 0; k2 < OPT; k2++) {
            const int o = tid + k2 * NT;
            if (o >= nout) break;
            const float gv = (float)gt[k2], uv = (float)ut[k2];
            const size_t oo = (size_t)t * TOUT + o;
            if (a.d[0].y) a.d[0].y[oo] = gv;
            if (a.d[1].y) a.d[1].y[oo] = uv;
            const double x1 = (double)gv;
            a.silu_out[oo] = (float)((double)uv * x1 / (1.0 + exp(-x1)));   // silu32, matrix.cl:27-32
        }
        return;
    }
    // kFinStore
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    double yt[OPT];
#pragma unroll
    for (int k2 = 0; k2 < OPT; k2++) {
        const int o = tid + k2 * NT;
        yt[k2] = o < nout ? acc_take(out + o) : 0.0;
    }
#pragma unroll
    for (int k2 = 0; k2 < OPT; k2++) asm volatile("" : "+v"(yt[k2]));   // as above: the waits after the last exchange
#pragma unroll
    for (int k2 = 0; k2 < OPT; k2++) {
        const int o = tid + k2 * NT;
        if (o >= nout) break;
        const float yv = (float)yt[k2];
        const int oo = t * TOUT + o;
        d.y[oo] = yv;
        take_max(bv, bi, yv, oo);
    }
    if (!a.pick_ctr) return;
    // the tile's first maximum, then the last tile to finish picks the token
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        take_max(bv, bi, ov, oi);
    }
    if (lane == 0) {
        s_bv[wave] = bv;
        s_bi[wave] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        for (int ww = 1; ww < NW; ww++) take_max(bv, bi, s_bv[ww], s_bi[ww]);
        // the candidate goes to the place the final reader's atomic loads
        // read, and is there before this tile arrives
        const unsigned long long cw = ((unsigned long long)(uint32_t)bi << 32) | __float_as_uint(bv);
        const unsigned long long prev = __hip_atomic_exchange(reinterpret_cast<unsigned long long*>(a.tile_cand + t),
                                                              cw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("" ::"v"(prev));
        s_last = __hip_atomic_fetch_add(a.pick_ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 (uint32_t)(d.T - 1);
    }
    __syncthreads();
    if (!s_last) return;
    if (wave == 0) {
        if (a.token_out) {
            // the tiles' candidates, one per lane (first maximum: a larger
            // value, or an equal one at a smaller index, wins; candidates are
            // never NaN, so the order of the combinations does not matter)
            float v = -INFINITY;
            int idx = 0x7fffffff;
            for (int t0 = 0; t0 < d.T; t0 += 64) {
                const int tt = t0 + lane;
                if (tt < d.T) {
                    const unsigned long long cw = __hip_atomic_load(
                        reinterpret_cast<unsigned long long*>(a.tile_cand + tt), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    take_max(v, idx, __uint_as_float((uint32_t)cw), (int)(cw >> 32));
                }
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const float ov = __shfl_xor(v, o, 64);
                const int oi = __shfl_xor(idx, o, 64);
                take_max(v, idx, ov, oi);
            }
            if (lane == 0) {
                const int tok = idx < d.C * 16 ? idx : 0;
                a.token_out[0] = tok;
                const int ps = a.pos[0];
                if (ps + 1 >= 0 && ps + 1 < a.hist_len) a.hist[ps + 1] = tok;
                a.pos[0] = ps + 1;
            }
        }
        if (lane == 0) a.pick_ctr[0] = 0u;
    }
    if (a.final_zero) {
        double* fz = reinterpret_cast<double*>(a.final_zero);
        for (int i = tid; i < a.final_zero_n; i += NT) fz[i] = 0.0;
    }
}

// ------------------------------------------------------------------ host ---

int quantile_of(float effort) { return (int)((double)(kProbes - 1) * (1.0 - (double)effort)); }

// ranks within this many of either end of the importances take no search hint
constexpr int kHintEdge = 64;

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

// Walk launch shape: 8-wave workgroups (each CU holds one: 128 KB of fp64
// tiles), about IAM_WALK_WGS of them, shared among the matrices in
// proportion to their expected weight bytes (at least one slice each), so
// that no CU holds more work than another.  IAM_WALK_UNR loads of RPI rows
// form a batch, two batches in flight per wave: with 2, each batch's LDS
// adds reach the tile in shorter bursts than with 4 (434.8 against 421.6
// tokens/s in decode), while 1 leaves too little in flight (411).
#ifndef IAM_WALK_UNR
#define IAM_WALK_UNR 2
#endif
#ifndef IAM_WALK_WGS
#define IAM_WALK_WGS 256
#endif
constexpr int kWalkWaves = 8;

int sel_block_for(const Ctx* c, float effort) { return c->sel_block > 1 && effort < c->sel_below ? c->sel_block : 1; }

void plan_walk(int n, const MatOp* ops, float effort, WalkPlan* plan, int blk, int tc)
{
    double bytes[kMaxMulti], tot = 0;
    for (int i = 0; i < n; i++) {
        const iam_bucket_matrix& M = ops[i].mat;
        WalkPlan& pl = plan[i];
        pl.T = (M.bucket_cols + tc - 1) / tc;
        pl.n_in = std::min((M.expert_rows + 15) / 16, ops[i].in_size);
        // the cost of a row is its tiles' width
        bytes[i] = est_rows(pl.n_in * 16, effort) * pl.T * tc * 2.0;
        tot += bytes[i];
    }
    for (int i = 0; i < n; i++) {
        WalkPlan& pl = plan[i];
        pl.NW = kWalkWaves;
        const double wgs = tot > 0 ? IAM_WALK_WGS * bytes[i] / tot : (double)IAM_WALK_WGS / n;
        const int slices = std::max(1, (int)std::floor(wgs / pl.T + 1e-9));
        pl.IPS = std::min(64 * pl.NW, std::max(1, (pl.n_in + slices - 1) / slices));
        if (blk > 1) pl.IPS = std::min(64 * pl.NW, (pl.IPS + blk - 1) / blk * blk);   // blocks within a slice
        pl.P = (pl.n_in + pl.IPS - 1) / pl.IPS;
    }
}

int walk_tiles(int bucket_cols) { return (bucket_cols + kTileColsNarrow - 1) / kTileColsNarrow; }

int max_slices(int n, const MatOp* ops, float effort, int blk, int tc)
{
    WalkPlan plan[kMaxMulti];
    plan_walk(n, ops, effort, plan, blk, tc);
    int P = 1;
    for (int i = 0; i < n; i++) P = std::max(P, plan[i].P);
    return P;
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
    DispatchDesc d{};
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
    d.sel_block = sel_block_for(c, s.effort);
    s.G = G;
    return launch(c, "bucket_list", k_dispatch, dim3(G), dim3(kCutThreads), 0, d);
}

template <typename Acc, int TC>
static int launch_walk(Ctx* c, const char* name, bool plain, dim3 grid, const WalkArgs& args)
{
    auto kern = k_walk<Acc, kWalkWaves, IAM_WALK_UNR, TC>;
    if (plain) {
        hipLaunchKernelGGL(kern, grid, dim3(64 * kWalkWaves), 0, c->stream, args);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return fail(IAM_E_HIP, std::string("launch ") + name + ": " + hipGetErrorString(e));
        return IAM_OK;
    }
    return launch(c, name, kern, grid, dim3(64 * kWalkWaves), 0, args);
}

#ifndef IAM_WALK_TILE_COLS
#define IAM_WALK_TILE_COLS 64
#endif

// The column tile width of a launch.  Narrow tiles halve the flush's atomic
// adds per workgroup (4 per thread on 128-column tiles back up the memory
// pipeline; 2 do not) for a slightly slower walk (twice the rows per load,
// 128-byte segments).
int walk_tile_cols(const WalkGroup& g)
{
    if (g.tile_cols == kTileColsNarrow || g.tile_cols == kTileColsWide) return g.tile_cols;
    return IAM_WALK_TILE_COLS == kTileColsWide ? kTileColsWide : kTileColsNarrow;
}

int walk_group(Ctx* c, const WalkGroup& g)
{
    IAM_REQUIRE(g.n >= 1 && g.n <= kMaxMulti, "walk: 1..3 matrices per launch");
    IAM_REQUIRE(g.label >= 0 && g.label < kWalkLabels, "walk: bad group label");
    IAM_REQUIRE(!std::isnan(g.effort), "walk: effort is NaN");
    MatOp ops[kMaxMulti];
    for (int i = 0; i < g.n; i++) {
        const WalkMat& wm = g.m[i];
        IAM_REQUIRE(((uintptr_t)wm.mat.buckets & 7) == 0, "walk: buckets must be 8-byte aligned");
        // slice-local row offsets (row < 8192) times bucket_cols are formed with 24-bit multiplies
        IAM_REQUIRE(wm.mat.bucket_cols > 0 && wm.mat.bucket_cols < (1 << 18), "walk: bucket_cols out of range");
        IAM_REQUIRE(wm.acc && wm.cutoff && wm.slice_count, "walk: missing scratch");
        IAM_REQUIRE(g.fin == kFinNone || wm.tile_ctr, "walk: missing tile counters");
        IAM_REQUIRE(g.fin != kFinStore || wm.y, "walk: missing outputs");
        IAM_REQUIRE(!wm.acc2 || g.fin == kFinNone, "walk: a second accumulator only without a finalize");
        ops[i].mat = wm.mat;
        ops[i].in_size = wm.in_size;
        ops[i].x = wm.x;
        ops[i].y = wm.y;
    }
    const int blk = sel_block_for(c, g.effort);
    const int tc = walk_tile_cols(g);
    WalkPlan plan[kMaxMulti];
    plan_walk(g.n, ops, g.effort, plan, blk, tc);
    WalkArgs args{};
    args.sel_block = blk;
    args.n = g.n;
    const int qv = quantile_of(g.effort);
    for (int i = 0; i < g.n; i++) {
        const WalkMat& wm = g.m[i];
        const iam_bucket_matrix& M = wm.mat;
        WalkDesc& d = args.d[i];
        d.W = M.buckets + (size_t)g.expert_no * (size_t)M.expert_rows * M.bucket_cols;
        d.x = const_cast<float*>(wm.x);
        d.stats = M.stats + (size_t)g.expert_no * (size_t)M.expert_rows * M.stats_stride;
        d.probes = M.probes + (size_t)g.expert_no * kProbes;
        d.cutoff = wm.cutoff;
        // a hint only for order statistics away from the ends: the few
        // smallest or largest importances (efforts near 1 or 0) move too much
        // between decode steps for a window around the previous one (about
        // half of them missed at effort 1.0, each miss costing the hinted
        // pass on top of the full search)
        const int t_rank = kProbes - qv;
        d.hint = t_rank >= kHintEdge && t_rank <= kProbes - kHintEdge ? wm.hint : nullptr;
        d.slice_count = wm.slice_count;
        d.acc = wm.acc;
        d.acc2 = wm.acc2;
        d.y = wm.y;
        d.tile_ctr = wm.tile_ctr;
        d.quantile = qv;
        d.stats_stride = M.stats_stride;
        d.stats_channel = M.stats_channel;
        d.rows = M.expert_rows;
        d.n_in = plan[i].n_in;
        d.C = M.bucket_cols;
        d.IPS = plan[i].IPS;
        d.P = plan[i].P;
        d.T = plan[i].T;
        d.nblocks = plan[i].P * plan[i].T;
        d.expected = plan[i].P;
    }
    // grid: every matrix's blocks, the matrices' work items in consecutive ranges
    int total = 0;
    for (int i = 0; i < kMaxMulti; i++) {
        args.first[i] = total;
        if (i < g.n) total += args.d[i].nblocks;
    }
    if (g.fin == kFinSilu) {
        IAM_REQUIRE(g.n == 2 && g.m[0].mat.bucket_cols == g.m[1].mat.bucket_cols && g.silu_out,
                    "walk: the SiLU gate pairs two matrices of one shape");
        args.d[0].expected = args.d[1].expected = plan[0].P + plan[1].P;
        args.d[1].tile_ctr = args.d[0].tile_ctr;
    }
    args.in_mode = g.in_mode;
    args.h = g.h;
    args.res_acc = g.res_acc;
    args.h_out = g.h_out;
    args.gain = g.gain;
    args.eps = g.eps;
    args.embed = g.embed;
    args.token = g.token;
    args.embed_scale = g.embed_scale;
    args.vocab = g.vocab;
    args.attn_acc = g.attn_acc;
    args.attn_lofs = g.m[0].in_size;
    args.fin = g.fin;
    args.silu_out = g.silu_out;
    args.pick_ctr = g.pick_ctr;
    args.tile_cand = reinterpret_cast<uint2*>(g.tile_cand);
    args.token_out = g.token_out;
    args.pos = g.pos;
    args.hist = g.hist;
    args.hist_len = g.hist_len;
    args.final_zero = g.final_zero;
    args.final_zero_n = g.final_zero_n;
    for (int z = 0; z < 2; z++) {
        args.zero_p[z] = g.zero_p[z];
        args.zero_n[z] = g.zero_n[z];
    }
    args.counters = c->counting ? c->counters + (size_t)g.label * kCounterLanes * 4 : nullptr;
    // walk_count reads the slice counts of the slots this launch wrote
    for (int i = 0; i < g.n; i++)
        if (g.m[i].slice_count == c->slots[i].slice_count) c->slots[i].walked_P = plan[i].P;
    const dim3 grid((unsigned)total);
    static const char* const names[kWalkLabels] = {"bucket_walk", "bucket_walk.qkv", "bucket_walk.o",
                                                    "bucket_walk.ffn13", "bucket_walk.ffn2", "bucket_walk.lm"};
    const char* name = names[g.label];
    if (tc == kTileColsNarrow)
        return c->acc64 ? launch_walk<double, kTileColsNarrow>(c, name, g.plain, grid, args)
                        : launch_walk<float, kTileColsNarrow>(c, name, g.plain, grid, args);
    return c->acc64 ? launch_walk<double, kTileColsWide>(c, name, g.plain, grid, args)
                    : launch_walk<float, kTileColsWide>(c, name, g.plain, grid, args);
}

// The standalone walk of the n matrices recorded in slots 0..n-1: the
// slots' scratch, fp32 outputs stored by the tiles' last workgroups.
static int walk_slots(Ctx* c, int n, const MatOp* ops, int in_mode, const float* h, const uint16_t* gain, float eps)
{
    WalkGroup g;
    g.n = n;
    g.in_mode = in_mode;
    g.effort = c->slots[0].effort;
    g.expert_no = c->slots[0].expert_no;
    g.h = h;
    g.gain = gain;
    g.eps = eps;
    g.fin = kFinStore;
    MatOp wops[kMaxMulti];
    for (int i = 0; i < n; i++) {
        wops[i] = ops[i];
        wops[i].x = c->slots[i].x;
        wops[i].in_size = c->slots[i].in_size;
    }
    const int P = max_slices(n, wops, g.effort, sel_block_for(c, g.effort), walk_tile_cols(g));
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
        IAM_REQUIRE(s.effort == c->slots[0].effort && s.expert_no == c->slots[0].expert_no,
                    "bucketmul: slots dispatched at different efforts or experts");
        const size_t m = (size_t)M.bucket_cols * 16;
        IAM_TRY(ensure_walk_scratch(c, i, m, walk_tiles((m + 15) / 16), (size_t)P));
        WalkMat& wm = g.m[i];
        wm.mat = M;
        wm.mat.stats = s.stats - (size_t)s.expert_no * (size_t)M.expert_rows * s.stats_stride;
        wm.mat.probes = s.probes - (size_t)s.expert_no * kProbes;
        wm.mat.stats_stride = s.stats_stride;
        wm.mat.stats_channel = s.stats_channel;
        wm.in_size = s.in_size;
        wm.x = s.x;
        wm.cutoff = s.cutoff;
        wm.hint = c->hints && in_mode != kInCutoff ? s.cutoff + 2 : nullptr;
        wm.slice_count = s.slice_count;
        wm.acc = s.acc;
        wm.tile_ctr = s.tile_ctr;
        wm.y = ops[i].y;
    }
    return walk_group(c, g);
}

int bucketmul_walk(Ctx* c, int n, const MatOp* ops) { return walk_slots(c, n, ops, kInCutoff, nullptr, nullptr, 0.0f); }

// One matrix group in one launch: every workgroup computes the input (x, or
// the norm of h written to x) and the cutoff itself.  A norm input of other
// than 4096 values is normalized by the RMSNorm kernel first.
int bucketmul_fused(Ctx* c, int n, const MatOp* ops, int expert_no, float effort, int in_mode, const float* h,
                    const uint16_t* gain, float eps)
{
    CutoffArgs args{};
    IAM_TRY(record_slots(c, n, ops, expert_no, effort, args));
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
            IAM_REQUIRE(ni % 1024 == 0, "bucketmul: a norm input must be a multiple of 1024 long");
            IAM_TRY(rmsnorm(c, const_cast<float*>(h), nullptr, gain, ni, eps, const_cast<float*>(ops[0].x)));
            in_mode = kInX;
        }
    }
    return walk_slots(c, n, ops, in_mode, h, gain, eps);
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
    return bucketmul_fused(c, n, ops, expert_no, effort, h ? kInNorm : kInX, h, gain, eps);
}

// The cutoff comes from the last search of the slot; the selection is re-run
// by the list kernel (which recomputes the cutoff on its own; the two must
// agree bit for bit).
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
    if (s.walked_P <= 0) return fail(IAM_E_STATE, "walk_count: no walk in this slot");
    IAM_CHECK_HIP(hipStreamSynchronize(c->stream));
    std::vector<uint32_t> sc((size_t)s.walked_P);
    IAM_CHECK_HIP(hipMemcpy(sc.data(), s.slice_count, sc.size() * sizeof(uint32_t), hipMemcpyDeviceToHost));
    uint64_t S = 0;
    for (uint32_t v : sc) S += v;
    *count = (uint32_t)S;
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
